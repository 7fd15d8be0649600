// MI355X (gfx950) construction of the resident ternary sketch.
//
// The reader's screen reads a sketch of every expert's gate/up rows: each
// rotated 128-coordinate block of a row is ternarised by the TWN rule and five
// rows' trits at one coordinate share a byte. The reference builds it with a
// torch loop over experts (calibration_free_moe/reader/sketch.py:84-150 of
// AidenGeunGeun/calibration-free-moe); this kernel builds the same format on
// the device in one launch per layer (cfmoe_build_sketch).
//
// Per (expert, row, block), in FP32:
//   v = blockdiag(H128)/sqrt(128) diag(signs) w   (sketch.py:38-50; the seven
//       butterfly stages pair coordinates c, c + w into (l + r, l - r), then
//       one multiply by fp32(1/sqrt(128)): the same operations in the same
//       order as the reference, so the rotated values are bit-identical)
//   keep = |v| > 0.7 * mean|v|, t = keep ? sign(v) : 0
//   scale = sum of kept |v| / max(kept, 1), residual = mean (v - t scale)^2
// Byte j = 2 g + plane of coordinate c packs channels 5 g .. 5 g + 4 of the
// gate (plane 0) or up (plane 1) rows as sum_d (t_d + 1) 3^d (= 121 +
// sum_d t_d 3^d; channels past the width count as zero trits). Bytes [0,
// body) of a coordinate sit at (b 128 + c) body, bytes [body, stride) at
// blocks 128 body + ((b / 2) 128 + c) 32 + (b % 2) 16. The FP16 statistics
// go to the physical [E, blocks, 2, 2 I] layout (scale plane, residual plane).
//
// The sums behind mean|v|, the scale and the residual are wave trees, not
// torch's reduction order: the threshold test can differ from a torch build
// only for |v| within an FP32 rounding of 0.7 mean|v|, and the FP16
// statistics only by a rounding.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cfmoe_reader.h"

namespace cfmoe {

int fail(int code, const char *message);
int check_launch(const char *stage);
int code_stride(int rows);

namespace {

constexpr float kRotationScale = 0.08838834764831845f;  // fp32(1 / sqrt(128))

struct SketchArgs {
  const uint16_t *weights;  // [E, 2 I, H] bf16
  const int8_t *signs;      // [H] +-1, or NULL (unrotated blocks)
  uint8_t *codes;           // [E, storage], padding bytes already 121
  __half *stats;            // physical [E, blocks, 2, 2 I]
  long storage;
  int rows, width, hidden, blocks, groups, stride, body;
};

__device__ __forceinline__ float bf16_value(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Sum over the wave in a fixed xor-butterfly order; every lane gets it.
__device__ __forceinline__ float wave_total(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = v + __shfl_xor(v, m);
  return v;
}

// Workgroup = one wave per (expert e, block b, plane, group g of five
// channels); lane l handles coordinates l and l + 64 of the block.
__global__ __launch_bounds__(64) void build_sketch_kernel(SketchArgs a) {
  const int lane = threadIdx.x;
  long item = blockIdx.x;
  const int g = static_cast<int>(item % a.groups);
  item /= a.groups;
  const int plane = static_cast<int>(item % 2);
  item /= 2;
  const int b = static_cast<int>(item % a.blocks);
  const int e = static_cast<int>(item / a.blocks);
  const int base = b * 128;
  float sign0 = 1.0f, sign1 = 1.0f;
  if (a.signs) {
    sign0 = static_cast<float>(a.signs[base + lane]);
    sign1 = static_cast<float>(a.signs[base + 64 + lane]);
  }
  int code0 = 0, code1 = 0, power = 1;
  for (int d = 0; d < 5; ++d, power *= 3) {
    const int channel = 5 * g + d;
    if (channel >= a.width) {  // past the width: zero trit, digit 1
      code0 += power;
      code1 += power;
      continue;
    }
    const int row = plane * a.width + channel;
    const uint16_t *source = a.weights + (static_cast<long>(e) * a.rows + row) * a.hidden + base;
    float v0 = bf16_value(source[lane]), v1 = bf16_value(source[64 + lane]);
    if (a.signs) {
      v0 = v0 * sign0;
      v1 = v1 * sign1;
#pragma unroll
      for (int stage = 0; stage < 6; ++stage) {
        const int bit = 1 << stage;
        const float p0 = __shfl_xor(v0, bit), p1 = __shfl_xor(v1, bit);
        v0 = (lane & bit) ? p0 - v0 : v0 + p0;
        v1 = (lane & bit) ? p1 - v1 : v1 + p1;
      }
      const float sum = v0 + v1, difference = v0 - v1;
      v0 = sum * kRotationScale;
      v1 = difference * kRotationScale;
    }
    const float m0 = fabsf(v0), m1 = fabsf(v1);
    const float threshold = 0.7f * (wave_total(m0 + m1) / 128.0f);
    const bool keep0 = m0 > threshold, keep1 = m1 > threshold;
    const int kept = __popcll(__ballot(keep0)) + __popcll(__ballot(keep1));
    const float kept_sum = wave_total((keep0 ? m0 : 0.0f) + (keep1 ? m1 : 0.0f));
    const float scale = kept_sum / static_cast<float>(kept > 1 ? kept : 1);
    const float t0 = keep0 ? (v0 > 0.0f ? 1.0f : -1.0f) : 0.0f;
    const float t1 = keep1 ? (v1 > 0.0f ? 1.0f : -1.0f) : 0.0f;
    const float r0 = v0 - t0 * scale, r1 = v1 - t1 * scale;
    const float residual = wave_total(r0 * r0 + r1 * r1) / 128.0f;
    if (lane == 0) {
      __half *stats = a.stats + (static_cast<long>(e) * a.blocks + b) * 2 * a.rows + row;
      stats[0] = __float2half_rn(scale);
      stats[a.rows] = __float2half_rn(residual);
    }
    code0 += (static_cast<int>(t0) + 1) * power;
    code1 += (static_cast<int>(t1) + 1) * power;
  }
  const int j = 2 * g + plane;
  uint8_t *codes = a.codes + static_cast<long>(e) * a.storage;
  auto offset = [&](int c) -> long {
    if (j < a.body) return static_cast<long>(base + c) * a.body + j;
    return static_cast<long>(a.blocks) * 128 * a.body + ((b / 2) * 128 + c) * 32 + (b % 2) * 16 +
           (j - a.body);
  };
  codes[offset(lane)] = static_cast<uint8_t>(code0);
  codes[offset(lane + 64)] = static_cast<uint8_t>(code1);
}

}  // namespace
}  // namespace cfmoe

extern "C" {

using namespace cfmoe;

CFMOE_API int cfmoe_build_sketch(int32_t experts, int32_t width, int32_t hidden,
                                 const void *gate_up, const int8_t *signs, uint8_t *codes,
                                 void *statistics, cfmoe_stream stream) {
  if (experts <= 0 || width <= 0 || hidden <= 0 || hidden % 128)
    return fail(CFMOE_EINVAL, "sketch needs experts, width > 0 and hidden a multiple of 128");
  if (!gate_up || !codes || !statistics) return fail(CFMOE_EINVAL, "NULL argument");
  SketchArgs a;
  a.weights = static_cast<const uint16_t *>(gate_up);
  a.signs = signs;
  a.codes = codes;
  a.stats = static_cast<__half *>(statistics);
  a.rows = 2 * width;
  a.width = width;
  a.hidden = hidden;
  a.blocks = hidden / 128;
  a.groups = (width + 4) / 5;
  a.stride = code_stride(a.rows);
  a.body = a.stride - a.stride % 32;
  const long tail = a.stride % 32 ? static_cast<long>((a.blocks + 1) / 2) * 128 * 32 : 0;
  a.storage = static_cast<long>(a.blocks) * 128 * a.body + tail;
  const long items = static_cast<long>(experts) * a.blocks * 2 * a.groups;
  hipLaunchKernelGGL(build_sketch_kernel, dim3(static_cast<unsigned>(items)), dim3(64), 0, stream,
                     a);
  return check_launch("build_sketch");
}

}  // extern "C"

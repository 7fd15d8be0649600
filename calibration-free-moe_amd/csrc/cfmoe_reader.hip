// MI355X (gfx950) kernels of the sparse expert reader and its C ABI.
//
// One HIP translation unit, no framework types: the Python operator
// (calibration_free_moe/reader/progressive.py) passes device pointers through
// ctypes. The stages follow ProgressiveReader.__call__ of the reference
// (calibration_free_moe/reader/progressive.py:3876-4472):
//
//   prepare_kernel   route + rotate + mask + grid quantisation  (:143-453)
//   screen_kernel    sketch projections per rotation-block split (:478-1108)
//   score_kernel     split sums, BF16 rounding, channel scores   (:1111-1353)
//   select_kernel    per-token top-F (radix select + compaction) (:1584-1775)
//   exact_kernel     native gate/up rows of kept channels         (:1372-1581)
//   encode_kernel    recovery encoder over skipped channels       (:1859-2016)
//   down_kernel      down rows of kept channels, 16-channel tiles (:1778-1856)
//   output_kernel    latent, decoder correction, router mix       (:2019-2111)
//
// Arithmetic contract (shared with the CPU oracle, oracle/cfmoe_oracle.c):
// the screen's per-block dot products are exact integer sums of trits times
// the rotated input on a 21-bit grid relative to the block maximum, so their
// value does not depend on how the sum is split across lanes, waves or
// workgroups; every FP32 chain that follows has one fixed order.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "cfmoe_reader.h"

namespace {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// scalar helpers (identical formulas in oracle/cfmoe_oracle.c)

__device__ __forceinline__ float bf16f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t bits = __float_as_uint(f);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((bits >> 16) | 0x40u);
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return static_cast<uint16_t>(bits >> 16);
}

__device__ __forceinline__ float bfr(float f) { return bf16f(f2bf(f)); }

// exp by Cody-Waite reduction and a degree-7 Taylor polynomial (Horner, fma).
__device__ float cfm_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.972084045410156f) return 0.0f;
  float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.428606765330187045e-06f, r);
  float p = 1.98412698412698413e-04f;
  p = fmaf(p, r, 1.38888888888888889e-03f);
  p = fmaf(p, r, 8.33333333333333333e-03f);
  p = fmaf(p, r, 4.16666666666666667e-02f);
  p = fmaf(p, r, 1.66666666666666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, static_cast<int>(n));
}

__device__ __forceinline__ float cfm_sigmoid(float x) { return 1.0f / (1.0f + cfm_expf(-x)); }

__device__ __forceinline__ float cfm_activate(float g, bool gelu) {
  if (gelu) {
    float cube = ((0.044715f * g) * g) * g;
    float inner = 1.5957691216057308f * (g + cube);
    return g * cfm_sigmoid(inner);
  }
  return g * cfm_sigmoid(g);
}

__device__ float cfm_score(float gate, float up, float gate_variance, float up_variance,
                           float norm, float weight, float alpha, float beta, bool gelu,
                           bool point) {
  const float nodes[5] = {-2.8569700138728056f, -1.355626179974266f, 0.0f,
                          1.355626179974266f, 2.8569700138728056f};
  const float masses[5] = {0.011257411327720693f, 0.2220759220056126f,
                           0.5333333333333333f, 0.2220759220056126f,
                           0.011257411327720693f};
  float g = bfr(gate);
  float u = bfr(up);
  float risk;
  if (point) {
    float value = norm * (cfm_activate(g, gelu) * u);
    risk = value * value;
  } else {
    float sg = sqrtf(gate_variance);
    float su = sqrtf(up_variance);
    float spread = su * su;
    float second = fmaf(u, u, spread);
    float energy = 0.0f, first = 0.0f, paid = 0.0f;
#pragma unroll
    for (int j = 0; j < 5; ++j) {
      float a = cfm_activate(fmaf(nodes[j], sg, g), gelu);
      float weighted = masses[j] * a;
      energy = fmaf(weighted * a, second, energy);
      first = fmaf(weighted, u, first);
      if (j == 2) paid = bfr(a * u);
    }
    float parallel = norm * first - alpha * paid;
    float perpendicular = beta * paid;
    float excess = energy - first * first;
    if (!(excess > 0.0f)) excess = 0.0f;
    risk = ((norm * norm) * excess + parallel * parallel) + perpendicular * perpendicular;
  }
  return (risk * weight) * weight;
}

__device__ __forceinline__ bool is_active(const uint8_t *padding, int t) {
  return padding == nullptr || padding[t] == 0;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (non-temporal: weights are read once per call).
__device__ __forceinline__ uint4 load_stream16(const void *address) {
  const u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4 *>(address));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint64_t lanes_below(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// ---------------------------------------------------------------------------
// prepare: route (progressive.py:349-386) and rotate/mask (:389-453)

struct PrepareArgs {
  const uint16_t *x;
  const int8_t *signs;
  const uint8_t *padding;
  const void *router_ids;
  const void *router_weights;
  int32_t *ids;
  float *weights;
  float *planes;
  int32_t *coords;
  int32_t *qvals;
  int32_t *qexp;
  float *norm2;
  double *read_work;
  double charges[18];
  int H, K, E, keep;
  uint32_t flags;
  int route, rotate;
};

__global__ __launch_bounds__(64) void prepare_kernel(PrepareArgs a) {
  const int t = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const bool active = is_active(a.padding, t);
  if (a.route && b == 0) {
    if (lane == 0) {
      int original[64], ordered[64];
      for (int k = 0; k < a.K; ++k) {
        int id = (a.flags & CFMOE_IDS_INT64)
                     ? static_cast<int>(static_cast<const int64_t *>(a.router_ids)[t * a.K + k])
                     : static_cast<const int32_t *>(a.router_ids)[t * a.K + k];
        // an id outside [0, E) names no local expert: it reads nothing
        if (id < 0 || id >= a.E) id = -1;
        original[k] = ordered[k] = id;
      }
      for (int i = 1; i < a.K; ++i) {
        int v = ordered[i], j = i - 1;
        while (j >= 0 && ordered[j] > v) {
          ordered[j + 1] = ordered[j];
          --j;
        }
        ordered[j + 1] = v;
      }
      for (int k = 0; k < a.K; ++k) {
        float w = 0.0f;
        for (int j = 0; j < a.K; ++j) {
          if (original[j] != ordered[k] || !active) continue;
          float rw = (a.flags & CFMOE_WEIGHTS_BF16)
                         ? bf16f(static_cast<const uint16_t *>(a.router_weights)[t * a.K + j])
                         : static_cast<const float *>(a.router_weights)[t * a.K + j];
          w += rw;
        }
        a.ids[t * a.K + k] = ordered[k];
        a.weights[t * a.K + k] = w;
      }
    }
    if ((a.flags & CFMOE_ACCOUNT) && active && lane < 18 && a.charges[lane] != 0.0)
      atomicAdd(a.read_work + lane, a.charges[lane]);
  }
  if (!a.rotate) return;

  const int H = a.H, keep = a.keep;
  const int base = b * 128;
  float v0 = active ? bf16f(a.x[static_cast<long>(t) * H + base + lane]) : 0.0f;
  float v1 = active ? bf16f(a.x[static_cast<long>(t) * H + base + 64 + lane]) : 0.0f;
  v0 = v0 * static_cast<float>(a.signs[base + lane]);
  v1 = v1 * static_cast<float>(a.signs[base + 64 + lane]);
#pragma unroll
  for (int stage = 0; stage < 6; ++stage) {
    const int bit = 1 << stage;
    float p0 = __shfl_xor(v0, bit);
    float p1 = __shfl_xor(v1, bit);
    v0 = (lane & bit) ? p0 - v0 : v0 + p0;
    v1 = (lane & bit) ? p1 - v1 : v1 + p1;
  }
  {
    float s = v0 + v1, d = v0 - v1;
    v0 = s * 0.08838834764831845f;
    v1 = d * 0.08838834764831845f;
  }
  const uint32_t m0 = __float_as_uint(v0) & 0x7fffffffu;
  const uint32_t m1 = __float_as_uint(v1) & 0x7fffffffu;
  bool kept0 = true, kept1 = true;
  if (keep < 128) {
    uint32_t low = 0, high = 0x7fffffffu;
    while (low < high) {
      uint32_t middle = low + ((high - low + 1u) >> 1);
      int count = __popcll(__ballot(m0 >= middle)) + __popcll(__ballot(m1 >= middle));
      if (count >= keep) low = middle; else high = middle - 1u;
    }
    const uint32_t cutoff = low;
    const int above = __popcll(__ballot(m0 > cutoff)) + __popcll(__ballot(m1 > cutoff));
    const int room = keep - above;
    const uint64_t tied0 = __ballot(m0 == cutoff);
    const uint64_t tied1 = __ballot(m1 == cutoff);
    const int rank0 = __popcll(tied0 & lanes_below(lane));
    const int rank1 = __popcll(tied0) + __popcll(tied1 & lanes_below(lane));
    kept0 = m0 > cutoff || (m0 == cutoff && rank0 < room);
    kept1 = m1 > cutoff || (m1 == cutoff && rank1 < room);
  }
  const uint64_t k0 = __ballot(kept0), k1 = __ballot(kept1);
  const int pos0 = __popcll(k0 & lanes_below(lane));
  const int pos1 = __popcll(k0) + __popcll(k1 & lanes_below(lane));
  __shared__ float compact[128];
  if (kept0) compact[pos0] = v0;
  if (kept1) compact[pos1] = v1;
  __syncthreads();
  const long cell = static_cast<long>(t) * (H / 128) + b;
  float sq = lane < keep ? compact[lane] * compact[lane] : 0.0f;
  if (lane + 64 < keep) sq = fmaf(compact[lane + 64], compact[lane + 64], sq);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) sq = sq + __shfl_xor(sq, m);
  uint32_t peak = (kept0 ? m0 : 0u);
  peak = max(peak, kept1 ? m1 : 0u);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) peak = max(peak, static_cast<uint32_t>(__shfl_xor(static_cast<int>(peak), m)));
  int exponent = 0;
  if (peak) frexpf(__uint_as_float(peak), &exponent);
  const int shift = peak ? 20 - exponent : 0;
  if (lane == 0) {
    a.norm2[cell] = sq;
    a.qexp[cell] = shift;
  }
  if (kept0) {
    a.planes[cell * keep + pos0] = v0;
    a.qvals[cell * keep + pos0] = peak ? static_cast<int32_t>(rintf(ldexpf(v0, shift))) : 0;
    if (keep < 128) a.coords[cell * keep + pos0] = lane;
  }
  if (kept1) {
    a.planes[cell * keep + pos1] = v1;
    a.qvals[cell * keep + pos1] = peak ? static_cast<int32_t>(rintf(ldexpf(v1, shift))) : 0;
    if (keep < 128) a.coords[cell * keep + pos1] = 64 + lane;
  }
}

// ---------------------------------------------------------------------------
// screen (progressive.py:478-1108)
//
// Workgroup (column group g, slot k, token t * S + split s). Lane owns one
// 4-byte code column of every kept coordinate row: two gate and two up code
// bytes, i.e. 10 gate and 10 up channels (20 rows). Waves split the kept
// positions into chunks of 16 (FP32 sums of <= 16 grid values of |q| <= 2^20
// are exact) and `sb` blocks of the split run side by side. Chunk sums are
// combined as integers; wave 0 then applies the per-block grid exponent and
// scale and runs the split's FMA chain in block order.

struct ScreenArgs {
  const uint8_t *codes;
  const uint16_t *stats;
  const int32_t *coords;
  const int32_t *qvals;
  const int32_t *qexp;
  const float *norm2;
  const int32_t *ids;
  const uint8_t *padding;
  float *parts;
  float *vparts;
  long storage;
  int H, I, K, N, keep, stride, splits, span, cn, sb, gh5;
};

constexpr int kRows = 20;

__global__ __launch_bounds__(1024) void screen_kernel(ScreenArgs a) {
  __shared__ _Float16 lut[256 * 6];
  extern __shared__ int reduce[];
  for (int i = threadIdx.x; i < 256; i += blockDim.x) {
    int value = i;
    for (int d = 0; d < 5; ++d) {
      lut[i * 6 + d] = static_cast<_Float16>(static_cast<float>(value % 3 - 1));
      value /= 3;
    }
    lut[i * 6 + 5] = static_cast<_Float16>(0.0f);
  }
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int chunk = wave % a.cn, sub = wave / a.cn;
  const int column = blockIdx.x * kWave + lane;
  const int body = a.stride - a.stride % 32;
  const bool column_ok = column < a.stride / 4;
  const int k = blockIdx.y;
  const int t = blockIdx.z / a.splits, s = blockIdx.z % a.splits;
  const int B = a.H / 128;
  const bool active = is_active(a.padding, t);
  const int e = a.ids[t * a.K + k];
  const bool local = active && e >= 0;
  const int b_begin = s * a.span;
  const int b_end = min(B, (s + 1) * a.span);
  const uint8_t *expert_codes = a.codes + static_cast<long>(local ? e : 0) * a.storage;
  const int rows2 = 2 * a.I;

  float part[kRows], vpart[kRows];
#pragma unroll
  for (int i = 0; i < kRows; ++i) part[i] = vpart[i] = 0.0f;

  for (int group = b_begin; group < b_end; group += a.sb) {
    const int b = group + sub;
    int isum[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) isum[i] = 0;
    if (local && b < b_end && column_ok) {
      const long cell = static_cast<long>(t) * B + b;
      const int p0 = chunk * 16;
      const int p1 = min(a.keep, p0 + 16);
      uint32_t words[16];
      float q[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int p = p0 + j;
        words[j] = 0x79797979u;
        q[j] = 0.0f;
        if (p < p1) {
          const int coord = a.keep < 128 ? a.coords[cell * a.keep + p] : p;
          q[j] = static_cast<float>(a.qvals[cell * a.keep + p]);
          long offset;
          if (4 * column < body)
            offset = (static_cast<long>(b) * 128 + coord) * body + 4 * column;
          else
            offset = static_cast<long>(B) * 128 * body +
                     (static_cast<long>(b / 2) * 128 + coord) * 32 + (b % 2) * 16 +
                     (4 * column - body);
          words[j] = __builtin_nontemporal_load(
              reinterpret_cast<const uint32_t *>(expert_codes + offset));
        }
      }
      float acc[kRows];
#pragma unroll
      for (int i = 0; i < kRows; ++i) acc[i] = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
#pragma unroll
        for (int byte = 0; byte < 4; ++byte) {
          const int code = (words[j] >> (8 * byte)) & 255;
          const _Float16 *entry = lut + code * 6;
#pragma unroll
          for (int d = 0; d < 5; ++d)
            acc[byte * 5 + d] = fmaf(static_cast<float>(entry[d]), q[j], acc[byte * 5 + d]);
        }
      }
#pragma unroll
      for (int i = 0; i < kRows; ++i) isum[i] = static_cast<int>(acc[i]);
    }
#pragma unroll
    for (int i = 0; i < kRows; ++i) reduce[(wave * kRows + i) * kWave + lane] = isum[i];
    __syncthreads();
    if (wave == 0 && column_ok && local) {
      for (int si = 0; si < a.sb; ++si) {
        const int bb = group + si;
        if (bb >= b_end) break;
        const long cell = static_cast<long>(t) * B + bb;
        const int shift = a.qexp[cell];
        const float n2 = a.gh5 ? a.norm2[cell] : 0.0f;
        const uint16_t *plane = a.stats + (static_cast<long>(e) * B + bb) * 2 * rows2;
#pragma unroll
        for (int i = 0; i < kRows; ++i) {
          int total = 0;
          for (int ch = 0; ch < a.cn; ++ch)
            total += reduce[((si * a.cn + ch) * kRows + i) * kWave + lane];
          const int byte = i / 5, d = i % 5;
          const int channel = 5 * (2 * column + byte / 2) + d;
          if (channel < a.I) {
            const int row = (byte % 2) * a.I + channel;
            const float dot = ldexpf(static_cast<float>(total), -shift);
            const float scale = static_cast<float>(__builtin_bit_cast(_Float16, plane[row]));
            part[i] = fmaf(dot, scale, part[i]);
            if (a.gh5) {
              const float resid =
                  static_cast<float>(__builtin_bit_cast(_Float16, plane[rows2 + row]));
              vpart[i] = fmaf(resid, n2, vpart[i]);
            }
          }
        }
      }
    }
    __syncthreads();
  }
  if (wave != 0 || !column_ok) return;
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const int byte = i / 5, d = i % 5;
    const int channel = 5 * (2 * column + byte / 2) + d;
    if (channel >= a.I) continue;
    const long address =
        ((static_cast<long>(t) * a.splits + s) * 2 + byte % 2) * a.N + k * a.I + channel;
    a.parts[address] = part[i];
    if (a.gh5) a.vparts[address] = vpart[i];
  }
}

// ---------------------------------------------------------------------------
// score (progressive.py:1111-1353): split sums in split order, then the score

struct ScoreArgs {
  const float *parts;
  const float *vparts;
  const int32_t *ids;
  const float *weights;
  const uint8_t *padding;
  const float *norms;
  const float *geometry;
  float *partial;
  float *variances;
  float *scores;
  uint8_t *completed;
  uint8_t *selected;
  int I, K, N, splits;
  int gh5, gelu, point;
};

__global__ __launch_bounds__(256) void score_kernel(ScoreArgs a) {
  const int logical = blockIdx.x * 256 + threadIdx.x;
  const int t = blockIdx.y;
  if (logical >= a.N) return;
  const int k = logical / a.I, c = logical % a.I;
  const long stride = 2l * a.N;
  const long base = static_cast<long>(t) * a.splits * stride + logical;
  float g = a.parts[base], u = a.parts[base + a.N];
  float vg = 0.0f, vu = 0.0f;
  if (a.gh5) {
    vg = a.vparts[base];
    vu = a.vparts[base + a.N];
  }
  for (int s = 1; s < a.splits; ++s) {
    g = g + a.parts[base + s * stride];
    u = u + a.parts[base + s * stride + a.N];
    if (a.gh5) {
      vg = vg + a.vparts[base + s * stride];
      vu = vu + a.vparts[base + s * stride + a.N];
    }
  }
  const long address = static_cast<long>(t) * stride + logical;
  a.partial[address] = g;
  a.partial[address + a.N] = u;
  if (a.gh5) {
    a.variances[address] = vg;
    a.variances[address + a.N] = vu;
  }
  const int e = a.ids[t * a.K + k];
  const bool local = is_active(a.padding, t) && e >= 0;
  const float norm = local ? a.norms[static_cast<long>(e) * a.I + c] : 0.0f;
  float alpha = 0.0f, beta = 0.0f;
  if (local && a.geometry) {
    alpha = a.geometry[(static_cast<long>(e) * a.I + c) * 2];
    beta = a.geometry[(static_cast<long>(e) * a.I + c) * 2 + 1];
  }
  const long flat = static_cast<long>(t) * a.N + logical;
  a.scores[flat] = cfm_score(g, u, vg, vu, norm, a.weights[t * a.K + k], alpha, beta,
                             a.gelu != 0, a.point != 0);
  a.completed[flat] = 0;
  a.selected[flat] = 0;
}

// ---------------------------------------------------------------------------
// select (progressive.py:1584-1775): the F best keys of score + 0 per token,
// ties to the lowest candidate id. Three radix passes (11/11/10 bits) find the
// F-th largest key; a block scan compacts the kept ids in candidate order.

struct SelectArgs {
  const float *scores;
  const float *threshold;
  int32_t *next_ids;
  uint8_t *selected;
  int32_t *counts;
  int32_t *starts;
  int32_t *tile_starts;
  int32_t *down_tile_starts;
  int N, F, I, K;
  int thresholded;
};

constexpr int kSelectThreads = 1024;
constexpr int kSelectKeys = 16;  // keys per thread: N <= 16384

__device__ int block_sum(int v, int *scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  int total = 0;
  for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) total += scratch[w];
  return total;
}

// Exclusive prefix over threads in thread order; *total receives the sum.
__device__ int block_exclusive(int v, int *scratch, int *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inclusive = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int n = __shfl_up(inclusive, o);
    if (lane >= o) inclusive += n;
  }
  __syncthreads();
  if (lane == 63) scratch[wave] = inclusive;
  __syncthreads();
  int before = 0, sum = 0;
  for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) {
    if (w < wave) before += scratch[w];
    sum += scratch[w];
  }
  *total = sum;
  return before + inclusive - v;
}

__global__ __launch_bounds__(kSelectThreads) void select_kernel(SelectArgs a) {
  __shared__ int histogram[2048];
  __shared__ int scratch[32];
  __shared__ int slot_counts[64];
  __shared__ uint32_t shared_bin;
  __shared__ int shared_above;
  const int t = blockIdx.x, tid = threadIdx.x;
  const int per = (a.N + kSelectThreads - 1) / kSelectThreads;
  const int first = tid * per;
  uint32_t key[kSelectKeys];
#pragma unroll
  for (int j = 0; j < kSelectKeys; ++j) {
    const int i = first + j;
    key[j] = (j < per && i < a.N)
                 ? __float_as_uint(a.scores[static_cast<long>(t) * a.N + i] + 0.0f)
                 : 0u;
  }
  auto valid = [&](int j) { return j < per && first + j < a.N; };
  int want = a.F;
  if (a.thresholded) {
    const uint32_t bound = __float_as_uint(*a.threshold + 0.0f);
    int passing = 0;
#pragma unroll
    for (int j = 0; j < kSelectKeys; ++j) passing += valid(j) && key[j] >= bound;
    passing = block_sum(passing, scratch);
    want = min(want, passing);
  }
  uint32_t prefix = 0, mask = 0;
  if (want > 0) {
    const int shifts[3] = {21, 10, 0};
    const int widths[3] = {11, 11, 10};
    for (int pass = 0; pass < 3; ++pass) {
      const int shift = shifts[pass];
      const uint32_t bins = 1u << widths[pass];
      for (int i = tid; i < 2048; i += kSelectThreads) histogram[i] = 0;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < kSelectKeys; ++j)
        if (valid(j) && (key[j] & mask) == prefix)
          atomicAdd(&histogram[(key[j] >> shift) & (bins - 1)], 1);
      __syncthreads();
      if (tid < 64) {
        // lane l owns bins [bins - (l + 1) * per_lane, bins - l * per_lane), high first
        const int per_lane = static_cast<int>(bins) / 64;
        const int top = static_cast<int>(bins) - tid * per_lane;
        int mine = 0;
        for (int i = 1; i <= per_lane; ++i) mine += histogram[top - i];
        int inclusive = mine;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          int n = __shfl_up(inclusive, o);
          if (tid >= o) inclusive += n;
        }
        const int before = inclusive - mine;
        const bool crossing = before < want && inclusive >= want;
        if (crossing) {
          int running = before;
          for (int i = 1; i <= per_lane; ++i) {
            const int h = histogram[top - i];
            if (running + h >= want) {
              shared_bin = static_cast<uint32_t>(top - i);
              shared_above = running;
              break;
            }
            running += h;
          }
        }
      }
      __syncthreads();
      prefix |= shared_bin << shift;
      mask |= (bins - 1) << shift;
      want -= shared_above;
      __syncthreads();
    }
  }
  const bool any = a.F > 0 && (a.thresholded ? (want > 0 || mask != 0) : true);
  // After the passes `prefix` is the cutoff key and `want` the ties it keeps.
  const uint32_t cutoff = prefix;
  const int room = want;
  int tied = 0;
#pragma unroll
  for (int j = 0; j < kSelectKeys; ++j) tied += valid(j) && mask != 0 && key[j] == cutoff;
  int tie_total;
  int tie_rank = block_exclusive(tied, scratch, &tie_total);
  bool keep[kSelectKeys];
  int kept = 0;
#pragma unroll
  for (int j = 0; j < kSelectKeys; ++j) {
    keep[j] = false;
    if (!valid(j) || mask == 0 || !any) continue;
    if (key[j] > cutoff) {
      keep[j] = true;
    } else if (key[j] == cutoff) {
      keep[j] = tie_rank < room;
      ++tie_rank;
    }
    kept += keep[j];
  }
  if (tid < 64) slot_counts[tid] = 0;
  int kept_total;
  int position = block_exclusive(kept, scratch, &kept_total);
#pragma unroll
  for (int j = 0; j < kSelectKeys; ++j) {
    if (!valid(j)) continue;
    const int i = first + j;
    a.selected[static_cast<long>(t) * a.N + i] = keep[j];
    if (keep[j] && position < a.F) {
      a.next_ids[static_cast<long>(t) * a.F + position++] = i;
      atomicAdd(&slot_counts[i / a.I], 1);
    }
  }
  for (int p = kept_total + tid; p < a.F; p += kSelectThreads)
    a.next_ids[static_cast<long>(t) * a.F + p] = -1;
  __syncthreads();
  if (tid == 0) {
    int start = 0, tile = 0, tile16 = 0;
    for (int k = 0; k < a.K; ++k) {
      const int count = slot_counts[k];
      a.counts[t * a.K + k] = count;
      a.starts[t * a.K + k] = start;
      a.tile_starts[t * a.K + k] = tile;
      a.down_tile_starts[t * a.K + k] = tile16;
      start += count;
      tile += (count + 127) / 128;
      tile16 += (count + 15) / 16;
    }
  }
}

// Full retention: every candidate is kept (progressive.py:2999-3004).
__global__ void select_all_kernel(SelectArgs a) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < a.N) {
    a.next_ids[static_cast<long>(t) * a.F + i] = i;
    a.selected[static_cast<long>(t) * a.N + i] = 1;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    for (int k = 0; k < a.K; ++k) {
      a.counts[t * a.K + k] = a.I;
      a.starts[t * a.K + k] = k * a.I;
      a.tile_starts[t * a.K + k] = k * ((a.I + 127) / 128);
      a.down_tile_starts[t * a.K + k] = k * ((a.I + 15) / 16);
    }
  }
}

// ---------------------------------------------------------------------------
// exact (progressive.py:1510-1546): one wave per kept channel

struct ExactArgs {
  const uint16_t *gate_up;
  const uint16_t *x;
  const int32_t *ids;
  const uint8_t *padding;
  const int32_t *next_ids;
  float *partial;
  uint16_t *activations;
  uint8_t *completed;
  int H, I, K, N, F, gelu;
};

__global__ __launch_bounds__(256) void exact_kernel(ExactArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int f = blockIdx.x * 4 + wave;
  const int t = blockIdx.y;
  if (f >= a.F) return;
  const int logical = a.next_ids[static_cast<long>(t) * a.F + f];
  if (logical < 0 || logical >= a.N) return;
  const int k = logical / a.I, c = logical % a.I;
  const int e = a.ids[t * a.K + k];
  const bool active = is_active(a.padding, t);
  float g = 0.0f, u = 0.0f;
  if (e >= 0) {
    const uint16_t *grow = a.gate_up + (static_cast<long>(e) * 2 * a.I + c) * a.H;
    const uint16_t *urow = grow + static_cast<long>(a.I) * a.H;
    const uint16_t *xr = a.x + static_cast<long>(t) * a.H;
    for (int j = 0; 512 * j < a.H; ++j) {
      const int h = 512 * j + 8 * lane;
      if (h >= a.H) continue;
      const uint4 gw = load_stream16(grow + h);
      const uint4 uw = load_stream16(urow + h);
      uint4 xw = make_uint4(0, 0, 0, 0);
      if (active) xw = *reinterpret_cast<const uint4 *>(xr + h);
      const uint32_t gv[4] = {gw.x, gw.y, gw.z, gw.w};
      const uint32_t uv[4] = {uw.x, uw.y, uw.z, uw.w};
      const uint32_t xv[4] = {xw.x, xw.y, xw.z, xw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x0 = __uint_as_float(xv[i] << 16), x1 = __uint_as_float(xv[i] & 0xffff0000u);
        g = fmaf(__uint_as_float(gv[i] << 16), x0, g);
        g = fmaf(__uint_as_float(gv[i] & 0xffff0000u), x1, g);
        u = fmaf(__uint_as_float(uv[i] << 16), x0, u);
        u = fmaf(__uint_as_float(uv[i] & 0xffff0000u), x1, u);
      }
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      g = g + __shfl_xor(g, m);
      u = u + __shfl_xor(u, m);
    }
  }
  if (lane == 0) {
    const long address = static_cast<long>(t) * 2 * a.N + logical;
    a.partial[address] = g;
    a.partial[address + a.N] = u;
    const float act = bfr(cfm_activate(bfr(g), a.gelu != 0));
    a.activations[static_cast<long>(t) * a.N + logical] = f2bf(act * bfr(u));
    a.completed[static_cast<long>(t) * a.N + logical] = 1;
  }
}

// ---------------------------------------------------------------------------
// encode (progressive.py:1859-1951): skipped channels of a 64-channel tile

struct EncodeArgs {
  const uint16_t *encoder_t;
  const float *partial;
  const uint16_t *activations;
  const uint8_t *completed;
  const uint8_t *selected;
  const int32_t *ids;
  const uint8_t *padding;
  float *parts;
  int I, K, N, R, tiles, gelu;
};

__global__ __launch_bounds__(64) void encode_kernel(EncodeArgs a) {
  __shared__ float value[64];
  __shared__ int skipped[64];
  const int tile = blockIdx.x, k = blockIdx.y, t = blockIdx.z, lane = threadIdx.x;
  const int c = tile * 64 + lane;
  const long logical = static_cast<long>(t) * a.N + static_cast<long>(k) * a.I + c;
  const int e = a.ids[t * a.K + k];
  const bool local = is_active(a.padding, t) && e >= 0;
  int skip = 0;
  float v = 0.0f;
  if (c < a.I && !a.selected[logical]) {
    skip = 1;
    if (a.completed[logical]) {
      v = bf16f(a.activations[logical]);
    } else {
      const long base = static_cast<long>(t) * 2 * a.N + static_cast<long>(k) * a.I + c;
      const float g = bfr(a.partial[base]);
      const float u = bfr(a.partial[base + a.N]);
      v = bfr(cfm_activate(g, a.gelu != 0) * u);
    }
  }
  value[lane] = v;
  skipped[lane] = skip;
  __syncthreads();
  if (lane >= a.R) return;
  float acc = 0.0f;
  for (int j = 0; j < 64; ++j) {
    if (!skipped[j]) continue;
    const float coefficient =
        local ? bf16f(a.encoder_t[(static_cast<long>(e) * a.I + tile * 64 + j) * a.R + lane])
              : 0.0f;
    acc = fmaf(value[j], coefficient, acc);
  }
  a.parts[((static_cast<long>(t) * a.K + k) * a.tiles + tile) * a.R + lane] = acc;
}

// ---------------------------------------------------------------------------
// down (progressive.py:1778-1856): 16-channel tiles of a slot's kept channels

struct DownArgs {
  const uint16_t *down;
  const uint16_t *activations;
  const int32_t *ids;
  const uint8_t *padding;
  const int32_t *next_ids;
  const int32_t *counts;
  const int32_t *starts;
  const int32_t *down_tile_starts;
  float *parts;
  int H, I, K, N, F, max_tiles;
};

__global__ __launch_bounds__(512) void down_kernel(DownArgs a) {
  const int tile = blockIdx.x, t = blockIdx.y;
  int k = -1, first = 0, count = 0;
  for (int s = 0; s < a.K; ++s) {
    const int c = a.counts[t * a.K + s];
    const int ts = a.down_tile_starts[t * a.K + s];
    if (tile >= ts && tile < ts + (c + 15) / 16) {
      k = s;
      first = (tile - ts) * 16;
      count = c;
    }
  }
  if (k < 0 || tile >= a.max_tiles) return;
  const int o = threadIdx.x * 8;
  if (o >= a.H) return;
  const int e = a.ids[t * a.K + k];
  const bool local = is_active(a.padding, t) && e >= 0;
  const int start = a.starts[t * a.K + k];
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int j = first; j < first + 16 && j < count; ++j) {
    if (start + j >= a.F) break;
    const int logical = a.next_ids[static_cast<long>(t) * a.F + start + j];
    if (logical < 0 || logical >= a.N) break;
    const int c = logical % a.I;
    const float act = bf16f(a.activations[static_cast<long>(t) * a.N + logical]);
    uint4 w = make_uint4(0, 0, 0, 0);
    if (local)
      w = load_stream16(a.down + (static_cast<long>(e) * a.I + c) * a.H + o);
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = fmaf(__uint_as_float(wv[i] << 16), act, acc[2 * i]);
      acc[2 * i + 1] = fmaf(__uint_as_float(wv[i] & 0xffff0000u), act, acc[2 * i + 1]);
    }
  }
  float *out = a.parts + (static_cast<long>(t) * a.max_tiles + tile) * a.H + o;
  *reinterpret_cast<float4 *>(out) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  *reinterpret_cast<float4 *>(out + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

// ---------------------------------------------------------------------------
// output (progressive.py:1954-2111): latent, decoder correction, router mix

struct OutputArgs {
  const float *down_parts;
  const float *encoder_parts;
  const int32_t *counts;
  const int32_t *down_tile_starts;
  const float *weights;
  const uint16_t *decoder;
  const uint8_t *padding;
  float *latent;
  uint16_t *out;
  int H, K, R, max_tiles, encoder_tiles;
};

__global__ __launch_bounds__(256) void output_kernel(OutputArgs a) {
  __shared__ float latent[64];
  const int t = blockIdx.y, tid = threadIdx.x;
  if (tid < a.R) {
    float mixed = 0.0f;
    for (int k = 0; k < a.K; ++k) {
      const float *parts = a.encoder_parts + (static_cast<long>(t) * a.K + k) * a.encoder_tiles * a.R;
      float total = 0.0f;
      for (int j = 0; j < a.encoder_tiles; ++j)
        total = j == 0 ? parts[tid] : total + parts[j * a.R + tid];
      mixed = fmaf(bfr(total), a.weights[t * a.K + k], mixed);
    }
    latent[tid] = mixed;
    if (blockIdx.x == 0) a.latent[static_cast<long>(t) * a.R + tid] = mixed;
  }
  __syncthreads();
  const int o = blockIdx.x * 256 + tid;
  if (o >= a.H) return;
  const bool active = is_active(a.padding, t);
  float routed = 0.0f;
  for (int k = 0; k < a.K; ++k) {
    const int tiles = (a.counts[t * a.K + k] + 15) / 16;
    const int first = a.down_tile_starts[t * a.K + k];
    float total = 0.0f;
    for (int j = 0; j < tiles && first + j < a.max_tiles; ++j) {
      const float p = a.down_parts[(static_cast<long>(t) * a.max_tiles + first + j) * a.H + o];
      total = j == 0 ? p : total + p;
    }
    routed = fmaf(bfr(total), a.weights[t * a.K + k], routed);
  }
  float correction = 0.0f;
  if (a.R > 0 && a.decoder) {
    float acc = 0.0f;
    for (int r = 0; r < a.R; ++r) {
      const float u = active ? bf16f(a.decoder[static_cast<long>(o) * a.R + r]) : 0.0f;
      acc = fmaf(u, bfr(latent[r]), acc);
    }
    correction = bfr(acc);
  }
  a.out[static_cast<long>(t) * a.H + o] = f2bf(routed + correction);
}

// ---------------------------------------------------------------------------
// host side

thread_local char g_error[512] = "";

int fail(int code, const char *message) {
  snprintf(g_error, sizeof(g_error), "%s", message);
  return code;
}

int check_launch(const char *stage) {
  hipError_t status = hipGetLastError();
  if (status != hipSuccess) {
    snprintf(g_error, sizeof(g_error), "%s launch failed: %s", stage, hipGetErrorString(status));
    return CFMOE_EHIP;
  }
  return 0;
}

int code_stride(int rows) {
  const int useful = 2 * ((rows / 2 + 4) / 5);
  return (useful + 15) / 16 * 16;
}

long storage_bytes(int rows, int hidden) {
  const int stride = code_stride(rows);
  const int blocks = hidden / 128;
  const int body = stride - stride % 32, tail = stride % 32;
  return static_cast<long>(blocks) * 128 * body +
         static_cast<long>((blocks + 1) / 2) * 128 * 2 * tail;
}

int validate(const cfmoe_dims *d) {
  if (!d) return fail(CFMOE_EINVAL, "dims is NULL");
  if (d->hidden <= 0 || d->hidden % 128) return fail(CFMOE_EINVAL, "hidden must be a positive multiple of 128");
  if (d->width <= 0 || d->width % 16) return fail(CFMOE_EINVAL, "width must be a positive multiple of 16");
  if (d->top_k < 1 || d->top_k > 64) return fail(CFMOE_EINVAL, "top_k must be in [1, 64]");
  if (d->rank < 0 || d->rank > 64) return fail(CFMOE_EINVAL, "rank must be in [0, 64]");
  if (d->keep < 1 || d->keep > 128) return fail(CFMOE_EINVAL, "keep must be in [1, 128]");
  const int n = d->top_k * d->width;
  if (d->final_count < 1 || d->final_count > n) return fail(CFMOE_EINVAL, "final_count must be in [1, N]");
  if (n > kSelectThreads * kSelectKeys) return fail(CFMOE_EINVAL, "N exceeds 16384 candidates");
  return 0;
}

struct Shape {
  int H, I, K, N, F, R, B, keep, splits, span, max_tiles, encoder_tiles;
  bool screened;
};

Shape shape_of(const cfmoe_dims *d) {
  Shape s;
  s.H = d->hidden;
  s.I = d->width;
  s.K = d->top_k;
  s.N = s.K * s.I;
  s.F = d->final_count;
  s.R = d->rank;
  s.B = s.H / 128;
  s.keep = d->keep;
  s.splits = s.B < 8 ? s.B : 8;
  s.span = (s.B + s.splits - 1) / s.splits;
  s.max_tiles = (s.F + 15) / 16 + s.K - 1;
  s.encoder_tiles = (s.I + 63) / 64;
  s.screened = s.F < s.N;
  return s;
}

int launch_prepare(const Shape &s, const cfmoe_dims *d, const cfmoe_weights *w,
                   const cfmoe_workspace *ws, const void *hidden, const void *router_ids,
                   const void *router_weights, const uint8_t *padding, int tokens,
                   const double *charges, bool route, bool rotate, hipStream_t stream) {
  PrepareArgs a;
  memset(&a, 0, sizeof(a));
  a.x = static_cast<const uint16_t *>(hidden);
  a.signs = w->signs;
  a.padding = padding;
  a.router_ids = router_ids;
  a.router_weights = router_weights;
  a.ids = ws->ids;
  a.weights = ws->weights;
  a.planes = ws->planes;
  a.coords = ws->coordinates;
  a.qvals = ws->qvals;
  a.qexp = ws->qexp;
  a.norm2 = ws->norm2;
  a.read_work = ws->read_work;
  if (charges && (d->flags & CFMOE_ACCOUNT))
    for (int i = 0; i < 18; ++i) a.charges[i] = charges[i];
  a.H = s.H;
  a.K = s.K;
  a.E = d->experts;
  a.keep = s.keep;
  a.flags = d->flags;
  a.route = route;
  a.rotate = rotate;
  dim3 grid(tokens, rotate ? s.B : 1);
  hipLaunchKernelGGL(prepare_kernel, grid, dim3(64), 0, stream, a);
  return check_launch("prepare");
}

}  // namespace

extern "C" {

int cfmoe_abi_version(void) { return CFMOE_ABI_VERSION; }

const char *cfmoe_last_error(void) { return g_error; }

int cfmoe_workspace_sizes(const cfmoe_dims *dims, int32_t capacity, int64_t *sizes,
                          int32_t count) {
  if (int rc = validate(dims)) return -rc;
  const Shape s = shape_of(dims);
  const int64_t cap = capacity;
  const int64_t n = s.N;
  const int64_t table[23] = {
      cap * s.K * 4,                          // ids
      cap * s.K * 4,                          // weights
      cap * s.B * s.keep * 4,                 // planes
      cap * s.B * s.keep * 4,                 // coordinates
      cap * s.B * s.keep * 4,                 // qvals
      cap * s.B * 4,                          // qexp
      cap * s.B * 4,                          // norm2
      cap * 2 * n * 4,                        // partial
      cap * 2 * n * 4,                        // variances
      cap * s.splits * 2 * n * 4,             // screen_parts
      cap * s.splits * 2 * n * 4,             // screen_variance_parts
      cap * n * 4,                            // scores
      cap * s.F * 4,                          // next_ids
      cap * n,                                // selected
      cap * n,                                // completed
      cap * n * 2,                            // activations
      cap * s.K * 4,                          // starts
      cap * s.K * 4,                          // counts
      cap * s.K * 4,                          // tile_starts
      cap * s.K * 4,                          // down_tile_starts
      cap * s.max_tiles * s.H * 4,            // down_parts
      cap * s.K * s.encoder_tiles * s.R * 4,  // encoder_parts
      cap * s.R * 4,                          // latent
  };
  const int written = count < 23 ? count : 23;
  for (int i = 0; i < written; ++i) sizes[i] = table[i];
  return written;
}

int cfmoe_prepare_input(const cfmoe_dims *dims, const cfmoe_weights *weights,
                        const cfmoe_workspace *workspace, const void *hidden,
                        const uint8_t *padding, int32_t tokens, cfmoe_stream stream) {
  if (int rc = validate(dims)) return rc;
  if (!weights || !workspace || !hidden) return fail(CFMOE_EINVAL, "NULL argument");
  if (tokens < 1 || tokens > workspace->capacity) return fail(CFMOE_EINVAL, "tokens out of range");
  const Shape s = shape_of(dims);
  return launch_prepare(s, dims, weights, workspace, hidden, nullptr, nullptr, padding, tokens,
                        nullptr, false, true, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

static int run_stages(uint32_t stages, const cfmoe_dims *dims, const cfmoe_weights *weights,
                      const cfmoe_workspace *workspace, const void *hidden,
                      const void *router_ids, const void *router_weights,
                      const uint8_t *padding, void *out, int32_t tokens,
                      const double *charges, cfmoe_stream stream_handle) {
  if (int rc = validate(dims)) return rc;
  if (!weights || !workspace || !hidden || !router_ids || !router_weights || !out)
    return fail(CFMOE_EINVAL, "NULL argument");
  if (tokens < 1 || tokens > workspace->capacity) return fail(CFMOE_EINVAL, "tokens out of range");
  const Shape s = shape_of(dims);
  if (s.R > 0 && (!weights->encoder_t || !weights->decoder))
    return fail(CFMOE_EINVAL, "rank > 0 needs encoder and decoder");
  if ((dims->flags & CFMOE_THRESHOLD) && !weights->threshold)
    return fail(CFMOE_EINVAL, "threshold flag without threshold");
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_handle);
  const uint32_t flags = dims->flags;
  const bool gh5 = !(flags & CFMOE_POINT);
  const bool gelu = (flags & CFMOE_GELU) != 0;
  const bool rotate = s.screened && !(flags & CFMOE_INPUT_PREPARED);
  int rc = 0;
  if (stages & (1u << CFMOE_STAGE_PREPARE)) {
    rc = launch_prepare(s, dims, weights, workspace, hidden, router_ids, router_weights,
                        padding, tokens, charges, true, rotate, stream);
    if (rc) return rc;
  }

  SelectArgs sel;
  memset(&sel, 0, sizeof(sel));
  sel.scores = workspace->scores;
  sel.threshold = weights->threshold;
  sel.next_ids = workspace->next_ids;
  sel.selected = workspace->selected;
  sel.counts = workspace->counts;
  sel.starts = workspace->starts;
  sel.tile_starts = workspace->tile_starts;
  sel.down_tile_starts = workspace->down_tile_starts;
  sel.N = s.N;
  sel.F = s.F;
  sel.I = s.I;
  sel.K = s.K;
  sel.thresholded = (flags & CFMOE_THRESHOLD) != 0;

  if (s.screened) {
    ScreenArgs sc;
    sc.codes = weights->codes;
    sc.stats = static_cast<const uint16_t *>(weights->statistics);
    sc.coords = workspace->coordinates;
    sc.qvals = workspace->qvals;
    sc.qexp = workspace->qexp;
    sc.norm2 = workspace->norm2;
    sc.ids = workspace->ids;
    sc.padding = padding;
    sc.parts = workspace->screen_parts;
    sc.vparts = workspace->screen_variance_parts;
    sc.storage = storage_bytes(2 * s.I, s.H);
    sc.H = s.H;
    sc.I = s.I;
    sc.K = s.K;
    sc.N = s.N;
    sc.keep = s.keep;
    sc.stride = code_stride(2 * s.I);
    sc.splits = s.splits;
    sc.span = s.span;
    sc.cn = (s.keep + 15) / 16;
    int sb = 11 / sc.cn;
    if (sb < 1) sb = 1;
    if (sb > s.span) sb = s.span;
    sc.sb = sb;
    sc.gh5 = gh5;
    const int groups = (sc.stride / 4 + kWave - 1) / kWave;
    const int threads = kWave * sc.cn * sc.sb;
    const size_t lds = static_cast<size_t>(sc.cn * sc.sb) * kRows * kWave * sizeof(int);
    if (stages & (1u << CFMOE_STAGE_SCREEN)) {
      hipLaunchKernelGGL(screen_kernel, dim3(groups, s.K, tokens * s.splits), dim3(threads),
                         lds, stream, sc);
      if ((rc = check_launch("screen"))) return rc;
    }

    ScoreArgs so;
    so.parts = workspace->screen_parts;
    so.vparts = workspace->screen_variance_parts;
    so.ids = workspace->ids;
    so.weights = workspace->weights;
    so.padding = padding;
    so.norms = weights->norms;
    so.geometry = (flags & CFMOE_GEOMETRY) ? weights->geometry : nullptr;
    so.partial = workspace->partial;
    so.variances = workspace->variances;
    so.scores = workspace->scores;
    so.completed = workspace->completed;
    so.selected = workspace->selected;
    so.I = s.I;
    so.K = s.K;
    so.N = s.N;
    so.splits = s.splits;
    so.gh5 = gh5;
    so.gelu = gelu;
    so.point = !gh5;
    if (stages & (1u << CFMOE_STAGE_SCORE)) {
      hipLaunchKernelGGL(score_kernel, dim3((s.N + 255) / 256, tokens), dim3(256), 0, stream,
                         so);
      if ((rc = check_launch("score"))) return rc;
    }
    if (stages & (1u << CFMOE_STAGE_SELECT)) {
      hipLaunchKernelGGL(select_kernel, dim3(tokens), dim3(kSelectThreads), 0, stream, sel);
      if ((rc = check_launch("select"))) return rc;
    }
  } else if (stages & (1u << CFMOE_STAGE_SELECT)) {
    hipLaunchKernelGGL(select_all_kernel, dim3((s.N + 255) / 256, tokens), dim3(256), 0, stream,
                       sel);
    if ((rc = check_launch("select_all"))) return rc;
  }

  ExactArgs ex;
  ex.gate_up = static_cast<const uint16_t *>(weights->gate_up);
  ex.x = static_cast<const uint16_t *>(hidden);
  ex.ids = workspace->ids;
  ex.padding = padding;
  ex.next_ids = workspace->next_ids;
  ex.partial = workspace->partial;
  ex.activations = static_cast<uint16_t *>(workspace->activations);
  ex.completed = workspace->completed;
  ex.H = s.H;
  ex.I = s.I;
  ex.K = s.K;
  ex.N = s.N;
  ex.F = s.F;
  ex.gelu = gelu;
  if (stages & (1u << CFMOE_STAGE_EXACT)) {
    hipLaunchKernelGGL(exact_kernel, dim3((s.F + 3) / 4, tokens), dim3(256), 0, stream, ex);
    if ((rc = check_launch("exact"))) return rc;
  }

  if (s.R > 0 && (stages & (1u << CFMOE_STAGE_ENCODE))) {
    EncodeArgs en;
    en.encoder_t = static_cast<const uint16_t *>(weights->encoder_t);
    en.partial = workspace->partial;
    en.activations = static_cast<const uint16_t *>(workspace->activations);
    en.completed = workspace->completed;
    en.selected = workspace->selected;
    en.ids = workspace->ids;
    en.padding = padding;
    en.parts = workspace->encoder_parts;
    en.I = s.I;
    en.K = s.K;
    en.N = s.N;
    en.R = s.R;
    en.tiles = s.encoder_tiles;
    en.gelu = gelu;
    hipLaunchKernelGGL(encode_kernel, dim3(s.encoder_tiles, s.K, tokens), dim3(64), 0, stream, en);
    if ((rc = check_launch("encode"))) return rc;
  }

  DownArgs dn;
  dn.down = static_cast<const uint16_t *>(weights->down);
  dn.activations = static_cast<const uint16_t *>(workspace->activations);
  dn.ids = workspace->ids;
  dn.padding = padding;
  dn.next_ids = workspace->next_ids;
  dn.counts = workspace->counts;
  dn.starts = workspace->starts;
  dn.down_tile_starts = workspace->down_tile_starts;
  dn.parts = workspace->down_parts;
  dn.H = s.H;
  dn.I = s.I;
  dn.K = s.K;
  dn.N = s.N;
  dn.F = s.F;
  dn.max_tiles = s.max_tiles;
  const int down_threads = ((s.H / 8 + kWave - 1) / kWave) * kWave;
  if (stages & (1u << CFMOE_STAGE_DOWN)) {
    hipLaunchKernelGGL(down_kernel, dim3(s.max_tiles, tokens), dim3(down_threads), 0, stream,
                       dn);
    if ((rc = check_launch("down"))) return rc;
  }
  if (!(stages & (1u << CFMOE_STAGE_OUTPUT))) return 0;

  OutputArgs op;
  op.down_parts = workspace->down_parts;
  op.encoder_parts = workspace->encoder_parts;
  op.counts = workspace->counts;
  op.down_tile_starts = workspace->down_tile_starts;
  op.weights = workspace->weights;
  op.decoder = static_cast<const uint16_t *>(weights->decoder);
  op.padding = padding;
  op.latent = workspace->latent;
  op.out = static_cast<uint16_t *>(out);
  op.H = s.H;
  op.K = s.K;
  op.R = s.R;
  op.max_tiles = s.max_tiles;
  op.encoder_tiles = s.encoder_tiles;
  hipLaunchKernelGGL(output_kernel, dim3((s.H + 255) / 256, tokens), dim3(256), 0, stream, op);
  return check_launch("output");
}

}  // namespace

extern "C" {

int cfmoe_forward(const cfmoe_dims *dims, const cfmoe_weights *weights,
                  const cfmoe_workspace *workspace, const void *hidden, const void *router_ids,
                  const void *router_weights, const uint8_t *padding, void *out,
                  int32_t tokens, const double *charges, cfmoe_stream stream) {
  return run_stages(~0u, dims, weights, workspace, hidden, router_ids, router_weights, padding,
                    out, tokens, charges, stream);
}

int cfmoe_launch_stage(int32_t stage, const cfmoe_dims *dims, const cfmoe_weights *weights,
                       const cfmoe_workspace *workspace, const void *hidden,
                       const void *router_ids, const void *router_weights,
                       const uint8_t *padding, void *out, int32_t tokens,
                       const double *charges, cfmoe_stream stream) {
  if (stage < 0 || stage >= CFMOE_STAGE_COUNT) return fail(CFMOE_EINVAL, "unknown stage");
  return run_stages(1u << stage, dims, weights, workspace, hidden, router_ids, router_weights,
                    padding, out, tokens, charges, stream);
}

}  // extern "C"

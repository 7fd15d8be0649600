// MI355X (gfx950) kernels of the sparse expert reader and its C ABI.
//
// One HIP translation unit, no framework types: the Python operator
// (calibration_free_moe/reader/progressive.py) passes device pointers through
// ctypes. The stages follow ProgressiveReader.__call__ of the reference
// (calibration_free_moe/reader/progressive.py:3876-4472):
//
//   prepare_kernel   route, expert grouping, rotate + mask + grid (:143-453)
//   small_screen_kernel  sketch projections and scores, batches below the
//                    grouped size: a tile's channel tile per workgroup, its
//                    block splits over the waves (MFMA)   (:478-1108, :1111-1353)
//   fused_screen_kernel  the same for grouped batches: every split of a
//                    channel tile in one wave             (:2428-2606)
//   select_kernel    per-token top-F (radix select + compaction) (:1584-1775)
//   exact_kernel     native gate/up rows of kept channels, batches below
//                    the grouped size: a wave per channel         (:1372-1581)
//   group_exact_kernel  grouped batches: gate/up rows of the channels some
//                    pair of an expert tile kept, read once per tile (:2655-2718)
//   encode_kernel    recovery encoder over skipped channels       (:1859-2016)
//                    (at rank 32 it runs inside the exact launches)
//   down_kernel      down rows of kept channels, 32-channel tiles (:1778-1856)
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
#include <pthread.h>
#include <string.h>

#include <algorithm>
#include <type_traits>

#include "cfmoe_reader.h"

namespace cfmoe {

constexpr int kWave = 64;
constexpr int kMaxSlots = 64;  // top_k limit of the C-ABI
constexpr int kMaxRank = 64;   // recovery rank limit of the C-ABI
constexpr int kDownTile = 32;  // selected channels per down tile (one fp32 partial each)

// ---------------------------------------------------------------------------
// scalar helpers (identical formulas in oracle/cfmoe_oracle.c)

__device__ __forceinline__ float bf16f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// (a select, not a branch: NaN keeps its payload with the quiet bit set)
__device__ __forceinline__ uint16_t f2bf(float f) {
  const uint32_t bits = __float_as_uint(f);
  const uint32_t rounded = bits + 0x7fffu + ((bits >> 16) & 1u);
  const uint32_t quiet = bits | 0x400000u;
  return static_cast<uint16_t>(((bits & 0x7fffffffu) > 0x7f800000u ? quiet : rounded) >> 16);
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

// Loads through the global address space (global_load, counted by vmcnt
// only; a generic pointer would make them flat loads that LDS waits also
// have to drain).
template <typename T>
__device__ __forceinline__ T load_global(const T *p) {
  return *reinterpret_cast<const __attribute__((address_space(1))) T *>(
      reinterpret_cast<uintptr_t>(p));
}

__device__ __forceinline__ uint4 load_global(const uint4 *p) {
  const u32x4 v = *reinterpret_cast<const __attribute__((address_space(1))) u32x4 *>(
      reinterpret_cast<uintptr_t>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint2 load_global(const uint2 *p) {
  const u32x2 v = *reinterpret_cast<const __attribute__((address_space(1))) u32x2 *>(
      reinterpret_cast<uintptr_t>(p));
  return make_uint2(v.x, v.y);
}

// Loads at a 32-bit byte offset from a wave-uniform base: the address stays
// base (scalar registers) + offset (one vector register) instead of a 64-bit
// vector address per lane.
template <typename V>
__device__ __forceinline__ V load_vector_at(const void *base, uint32_t offset) {
  const __attribute__((address_space(1))) char *b =
      reinterpret_cast<const __attribute__((address_space(1))) char *>(reinterpret_cast<uintptr_t>(base));
  return *reinterpret_cast<const __attribute__((address_space(1))) V *>(b + offset);
}

__device__ __forceinline__ uint2 load_uint2_at(const void *base, uint32_t offset) {
  const u32x2 v = load_vector_at<u32x2>(base, offset);
  return make_uint2(v.x, v.y);
}

__device__ __forceinline__ uint4 load_uint4_at(const void *base, uint32_t offset) {
  const u32x4 v = load_vector_at<u32x4>(base, offset);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Load source of dead lanes (no branch around a load, no select after it).
__device__ const uint4 kZeroVector = {0, 0, 0, 0};

// Wave-uniform loads through the scalar data cache (constant address space):
// for values an earlier launch wrote and this one only reads. They bypass the
// vector memory queue, where under load a small read waits behind the
// wave's neighbours' row loads.
template <typename T>
__device__ __forceinline__ T load_uniform(const T *p) {
  return *reinterpret_cast<const __attribute__((address_space(4))) T *>(
      reinterpret_cast<uintptr_t>(p));
}

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

// Raw buffer resource over `bytes` bytes from a wave-uniform base (stride 0,
// the gfx9 default format word): a buffer load past `bytes` reads zeros, and
// every load of the wave shares one 32-bit lane offset (constant parts go into
// the instruction's immediate offset), not a 64-bit address per load.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_resource(const void *base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, int offset) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// non-temporal (weights read once per call)
__device__ __forceinline__ uint4 buffer_stream16(__amdgpu_buffer_rsrc_t r, int offset) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 2);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint64_t lanes_below(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Sum of a wave's 64 values at lane 0 in the xor-butterfly tree (levels m =
// 1, 2, ..., 32: each level adds the neighbouring block of m lanes). After a
// level every lane of a block holds the same bits (a + b == b + a exactly),
// so any lane of the partner block serves: DPP quad permutes for m = 1, 2,
// the half-row and row mirrors for m = 4, 8, and lane reads of the four row
// sums for m = 16, 32. No LDS crossbar traffic.
template <int kControl>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kControl, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_sum_lane0(float v) {
  v = dpp_add<0xb1>(v);   // quad_perm [1, 0, 3, 2]: xor 1
  v = dpp_add<0x4e>(v);   // quad_perm [2, 3, 0, 1]: xor 2
  v = dpp_add<0x141>(v);  // row_half_mirror: the other 4 lanes of the 8
  v = dpp_add<0x140>(v);  // row_mirror: the other 8 lanes of the 16
  const float s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float s1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float s2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float s3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (s0 + s1) + (s2 + s3);
}

// The value of lane (lane ^ kMask), kMask = 1, 2, ..., 32, without the LDS
// crossbar where a DPP move serves: quad permutes for 1 and 2; for 4 a quad
// reversal, then the half-row mirror (lane i reads (i ^ 7) ^ 3 = i ^ 4); for 8
// the row rotation by 8; for 16 a swizzle (xor mask 16 inside each half);
// for 32 a backward permute.
template <int kMask>
__device__ __forceinline__ float lane_xor(float v) {
  const int bits = __float_as_int(v);
  if (kMask == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(bits, 0xb1, 0xf, 0xf, false));
  if (kMask == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(bits, 0x4e, 0xf, 0xf, false));
  if (kMask == 4) {
    const int reversed = __builtin_amdgcn_mov_dpp(bits, 0x1b, 0xf, 0xf, false);
    return __int_as_float(__builtin_amdgcn_mov_dpp(reversed, 0x141, 0xf, 0xf, false));
  }
  if (kMask == 8) return __int_as_float(__builtin_amdgcn_mov_dpp(bits, 0x128, 0xf, 0xf, false));
  if (kMask == 16) return __int_as_float(__builtin_amdgcn_ds_swizzle(bits, 0x401f));
  return __int_as_float(__shfl_xor(bits, 32));
}

// Largest and smallest of a wave's 64 values, every lane gets them (exact in
// any order): the DPP tree of wave_sum_lane0, then lane reads of the rows.
template <bool kMax>
__device__ __forceinline__ uint32_t wave_extreme(uint32_t v) {
  auto pick = [](uint32_t x, uint32_t y) { return kMax ? max(x, y) : min(x, y); };
  v = pick(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0xb1, 0xf, 0xf, false)));
  v = pick(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x4e, 0xf, 0xf, false)));
  v = pick(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x141, 0xf, 0xf, false)));
  v = pick(v, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x140, 0xf, 0xf, false)));
  const uint32_t r0 = __builtin_amdgcn_readlane(static_cast<int>(v), 0);
  const uint32_t r1 = __builtin_amdgcn_readlane(static_cast<int>(v), 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(static_cast<int>(v), 32);
  const uint32_t r3 = __builtin_amdgcn_readlane(static_cast<int>(v), 48);
  return pick(pick(r0, r1), pick(r2, r3));
}

// ---------------------------------------------------------------------------
// block-wide reductions (thread order)

// Integer wave sum, every lane gets the total (exact in any order).
__device__ __forceinline__ int wave_sum_all(int v) {
  v += __builtin_amdgcn_mov_dpp(v, 0xb1, 0xf, 0xf, false);   // xor 1
  v += __builtin_amdgcn_mov_dpp(v, 0x4e, 0xf, 0xf, false);   // xor 2
  v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xf, 0xf, false);  // row_half_mirror
  v += __builtin_amdgcn_mov_dpp(v, 0x140, 0xf, 0xf, false);  // row_mirror
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

// Integer inclusive scan over the wave's lanes: shifts of 1, 2, 4, 8 lanes
// inside each 16-lane row (DPP row_shr, zero from outside the row), then the
// totals of the rows below (lane reads of lanes 15, 31, 47).
__device__ __forceinline__ int wave_inclusive(int v) {
  const int lane = threadIdx.x & 63;
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(v, 15);
  const int r1 = __builtin_amdgcn_readlane(v, 31);
  const int r2 = __builtin_amdgcn_readlane(v, 47);
  return v + (lane >= 16 ? r0 : 0) + (lane >= 32 ? r1 : 0) + (lane >= 48 ? r2 : 0);
}

__device__ int block_sum(int v, int *scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum_all(v);
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
  const int inclusive = wave_inclusive(v);
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

// ---------------------------------------------------------------------------
// prepare: route + expert grouping (progressive.py:349-386, :2329-2373) and
// rotate/mask (:389-453)
//
// 256-thread blocks (1024 from kWidePreparePairs routed pairs). Block 0
// sorts every token's K ids, groups the (token, slot) pairs by expert into
// tiles of at most 16 pairs (touched experts in ascending id order, each with
// its pairs in ascending pair index: deterministic lists, no atomics in the
// order) and adds the fixed read charges. Wave w of cell block i rotates cell
// W i + w = (token, block), W the block's waves.

// Balanced 8-bit digits of a grid value: q = d0 + 2^8 d1 + 2^16 d2 with
// d_i in [-128, 127] (|q| <= 2^20).
__device__ __forceinline__ void grid_digits(int q, int &d0, int &d1, int &d2) {
  d0 = ((q + 128) & 255) - 128;
  const int rest = (q - d0) >> 8;
  d1 = ((rest + 128) & 255) - 128;
  d2 = (rest - d1) >> 8;
}

struct PrepareArgs {
  const uint16_t *x;
  const int8_t *signs;
  const uint8_t *padding;
  // the padding mask as a buffer source: the mask and T bytes, or (no mask)
  // any valid pointer and 0 bytes, whose loads read zero (active)
  const void *padding_source;
  int padding_bytes;
  const void *router_ids;
  const void *router_weights;
  int32_t *ids;
  float *weights;
  float *planes;
  int32_t *coords;
  int32_t *qvals;
  int32_t *qexp;
  int32_t *qsums;
  float *norm2;
  int8_t *digits;  // [T, B, 3, 128] digit planes of the cell's grid values
  int32_t *group_experts;
  int32_t *group_starts;
  int32_t *group_counts;
  int32_t *group_pairs;
  int32_t *group_total;
  int32_t *pair_tiles;
  double *read_work;
  double charges[18];
  // per tile of pairs: sketch bytes the screen streams, its matrix-core
  // MACs, and (grouped dense plans) the gate/up bytes the exact rows read
  double tile_sketch_bytes, tile_screen_macs, tile_row_bytes;
  int T, H, K, E, keep;
  uint32_t flags;
  int route, rotate, cells;
};

constexpr int kMaxPairs = 8192;    // T * K routed pairs grouped per call
constexpr int kWorkspaceBuffers = 31;  // cfmoe_workspace pointers after capacity
constexpr int kGroupPairs = 16;    // pairs per screen tile (one MFMA column block)
constexpr int kMaxExperts = 4096;  // local experts the grouping counts in LDS
// Prepare workgroups: 256 threads, or 1024 from kWidePreparePairs routed
// pairs (the routing workgroup, alone on its CU, is the launch's longest: at
// 2048 pairs 1024 threads take it from 16.8 to 11.7 us, at 512 pairs from
// 8.7 to 8.3 us inside the layer; at 256 pairs the narrower cell workgroups,
// spread over more CUs, win).
constexpr int kPrepareThreads = 256;
constexpr int kWidePrepareThreads = 1024;
constexpr int kWidePreparePairs = 512;

// LDS of the routing block, carved from the launch's dynamic LDS, which the
// host sizes for the call's pairs and experts (route_lds_bytes): the pairs'
// ids in routing order (later each pair's rank among the earlier pairs of
// its expert in its wave's range) and sorted per token, then per-expert
// counters and packed prefixes, then per-wave per-expert pair counts.
struct RouteShared {
  int16_t *sorted, *routed;
  int *counts, *base;
  int16_t *wave_counts;  // [waves][experts]
};

__host__ __device__ inline long route_pairs_padded(int pairs) { return (pairs + 7) / 8 * 8; }

__host__ __device__ inline long route_lds_bytes(int pairs, int experts, int waves) {
  return 2 * 2 * route_pairs_padded(pairs) + 2 * 4 * (experts + 1) + 2L * waves * experts;
}

__device__ inline RouteShared route_layout(char *lds, int pairs, int experts) {
  RouteShared r;
  const long padded = route_pairs_padded(pairs);
  r.sorted = reinterpret_cast<int16_t *>(lds);
  r.routed = r.sorted + padded;
  r.counts = reinterpret_cast<int *>(r.routed + padded);
  r.base = r.counts + experts + 1;
  r.wave_counts = reinterpret_cast<int16_t *>(r.base + experts + 1);
  return r;
}

template <int kPrepareThreads, bool kIds64, bool kWeights16>
__device__ __forceinline__ void route_and_group(const PrepareArgs &a, const RouteShared &shared,
                                                int *scratch) {
  constexpr int kPrepareWaves = kPrepareThreads / 64;
  // (the arguments the routing uses, loaded in one batch at entry)
  asm volatile("" ::"s"(a.router_ids), "s"(a.router_weights), "s"(a.padding_source), "s"(a.padding_bytes),
               "s"(a.ids), "s"(a.weights), "s"(a.pair_tiles), "s"(a.group_pairs), "s"(a.group_experts),
               "s"(a.group_starts), "s"(a.group_counts), "s"(a.group_total), "s"(a.T), "s"(a.K), "s"(a.E),
               "s"(a.flags));
  int16_t *sorted = shared.sorted;
  int16_t *routed = shared.routed;
  int *counts = shared.counts, *base = shared.base;
  const int tid = threadIdx.x;
  const int T = a.T, K = a.K;
  const int pairs = T * K;
  auto weight_of = [&](int q) {
    return kWeights16 ? bf16f(load_global(static_cast<const uint16_t *>(a.router_weights) + q))
                      : load_global(static_cast<const float *>(a.router_weights) + q);
  };
  // Each thread's first kBatch pairs p = tid + kPrepareThreads q (all of
  // them up to 8 pairs per thread: the host runs 1024 threads from 1024
  // pairs unless the experts' LDS lists are too large): the raw ids, the
  // router weights and the pairs' tokens' padding flags in one round trip,
  // every load unconditional (clamped index; the formats are template
  // arguments; a padding source of zero bytes reads zero: active)
  constexpr int kBatch = 8;
  const __amdgpu_buffer_rsrc_t padding = buffer_resource(a.padding_source, a.padding_bytes);
  auto raw_id_of = [&](int p) {
    if (kIds64) {
      const int32_t *words = static_cast<const int32_t *>(a.router_ids) + 2 * p;
      const int low = load_global(words), high = load_global(words + 1);
      return high == (low >> 31) ? low : -1;  // outside the int32 range
    }
    return load_global(static_cast<const int32_t *>(a.router_ids) + p);
  };
  auto store_routed = [&](int p, int raw) {
    routed[p] = static_cast<int16_t>((raw < 0 || raw >= a.E) ? -1 : raw);
    a.pair_tiles[p] = -1;  // pairs in no tile (padded token, no local expert)
  };
  int raw_id[kBatch];
  float own_weight[kBatch];
  uint32_t pad_flags[kBatch];
#pragma unroll
  for (int q = 0; q < kBatch; ++q) {
    const int p = min(tid + kPrepareThreads * q, pairs - 1);
    raw_id[q] = raw_id_of(p);
    own_weight[q] = weight_of(p);
    pad_flags[q] = __builtin_amdgcn_raw_buffer_load_b8(padding, p / K, 0, 0);
  }
  // (every load above is issued before the first is used)
  asm volatile("" ::: "memory");
  int active_tokens = 0;  // tokens counted at their slot 0
#pragma unroll
  for (int q = 0; q < kBatch; ++q) {
    const int p = tid + kPrepareThreads * q;
    if (p < pairs) {
      store_routed(p, raw_id[q]);
      active_tokens += p % K == 0 && pad_flags[q] == 0;
    }
  }
  for (int p = tid + kBatch * kPrepareThreads; p < pairs; p += kPrepareThreads) {
    store_routed(p, raw_id_of(p));
    active_tokens += p % K == 0 && is_active(a.padding, p / K);
  }
  // the fixed read charges go out right after the first barrier, so their
  // atomics travel while the routing runs (the wave sums cross it in scratch)
  const bool account = (a.flags & CFMOE_ACCOUNT) != 0;
  if (account) {
    const int wave_active = wave_sum_all(active_tokens);
    if ((tid & 63) == 0) scratch[tid >> 6] = wave_active;
  }
  __syncthreads();
  if (account && tid < 18) {
    int active = 0;
#pragma unroll
    for (int w = 0; w < kPrepareWaves; ++w) active += scratch[w];
    if (a.charges[tid] != 0.0 && active > 0)
      atomicAdd(a.read_work + tid, a.charges[tid] * static_cast<double>(active));
  }
  // slot k of a token moves to its rank among the token's ids (ties by slot);
  // its weight is the sum of the weights of equal ids (progressive.py:369-375)
  auto place = [&](int p, float own, bool active) {
    const int t = p / K, k = p % K;
    const int id = routed[p];
    int rank = 0, equal = 0;
    for (int j0 = 0; j0 < K; j0 += 8) {
      int other[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) other[j] = routed[t * K + min(j0 + j, K - 1)];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j0 + j >= K) break;
        rank += other[j] < id || (other[j] == id && j0 + j < k);
        equal += other[j] == id;
      }
    }
    float w = 0.0f;
    if (active) {
      if (equal == 1) {
        w = 0.0f + own;
      } else {
        for (int j = 0; j < K; ++j)
          if (routed[t * K + j] == id) w += weight_of(t * K + j);
      }
    }
    a.ids[t * K + rank] = id;
    a.weights[t * K + rank] = w;
    sorted[t * K + rank] = static_cast<int16_t>(active ? id : -1);
  };
#pragma unroll
  for (int q = 0; q < kBatch; ++q) {
    const int p = tid + kPrepareThreads * q;
    if (p >= pairs) break;
    place(p, own_weight[q], pad_flags[q] == 0);
  }
  for (int p = tid + kBatch * kPrepareThreads; p < pairs; p += kPrepareThreads)
    place(p, weight_of(p), is_active(a.padding, p / K));
  const int padded = (pairs + 7) / 8 * 8;
  for (int p = pairs + tid; p < padded; p += kPrepareThreads) sorted[p] = -1;
  __syncthreads();
  // Expert-major grouping as a counting sort by expert, stable in pair order:
  // (1) per-expert counts; (2) one scan of packed (members, tiles) gives each
  // expert its member start and first tile z_e, and its tiles are emitted;
  // (3) wave w ranks the pairs of its contiguous range among the earlier
  // pairs of the same expert (a match of equal experts from one ballot per id
  // bit, 64 pairs at a time, running per-expert counts of the wave); (4) a
  // pair's final slot is 16 z_e + its rank within its wave's range + the
  // counts of the waves before. O(pairs log E), whatever the skew.
  for (int e = tid; e <= a.E; e += kPrepareThreads) counts[e] = 0;
  for (int i = tid; i < kPrepareWaves * a.E; i += kPrepareThreads) shared.wave_counts[i] = 0;
  __syncthreads();
  for (int p = tid; p < pairs; p += kPrepareThreads) {
    const int e = sorted[p];
    if (e >= 0) atomicAdd(&counts[e], 1);
  }
  __syncthreads();
  // thread i owns the experts [i per, (i + 1) per)
  const int per = (a.E + kPrepareThreads - 1) / kPrepareThreads;
  const int first = min(a.E, tid * per), last = min(a.E, first + per);
  int members = 0, tiles = 0;
  for (int e = first; e < last; ++e) {
    members += counts[e];
    tiles += (counts[e] + kGroupPairs - 1) / kGroupPairs;
  }
  int packed_total;  // members and tiles are below 2^16 (pairs <= 8192)
  const int packed = block_exclusive(members | (tiles << 16), scratch, &packed_total);
  const int total_tiles = packed_total >> 16;
  // the per-tile read charges (integers, exact in FP64), issued as soon as
  // the tile count is known
  if (account && total_tiles > 0) {
    const double tile_count = static_cast<double>(total_tiles);
    if (tid == 32 && a.tile_sketch_bytes != 0.0) atomicAdd(a.read_work + 11, tile_count * a.tile_sketch_bytes);
    if (tid == 33 && a.tile_screen_macs != 0.0) atomicAdd(a.read_work + 15, tile_count * a.tile_screen_macs);
    if (tid == 34 && a.tile_row_bytes != 0.0) atomicAdd(a.read_work + 12, tile_count * a.tile_row_bytes);
  }
  {
    int start = packed & 0xffff, z = packed >> 16;
    for (int e = first; e < last; ++e) {
      const int count = counts[e];
      base[e] = start | (z << 16);
      for (int first_pair = 0; first_pair < count; first_pair += kGroupPairs) {
        a.group_experts[z] = e;
        a.group_starts[z] = kGroupPairs * z;
        a.group_counts[z] = min(kGroupPairs, count - first_pair);
        ++z;
      }
      start += count;
    }
    if (tid == kPrepareThreads - 1) base[a.E] = packed_total & 0xffff;
  }
  {
    const int wave = tid >> 6, lane = tid & 63;
    const int chunks = (pairs + 63) / 64;
    const int per_wave = (chunks + kPrepareWaves - 1) / kPrepareWaves;
    const int bits = a.E > 1 ? 32 - __builtin_clz(static_cast<unsigned>(a.E - 1)) : 1;
    int16_t *counted = shared.wave_counts + wave * a.E;
    int16_t *local_rank = routed;
    for (int c = wave * per_wave; c < min(chunks, (wave + 1) * per_wave); ++c) {
      const int p = 64 * c + lane;
      const int e = p < pairs ? sorted[p] : -1;
      // lanes holding the same expert: agree on every id bit
      uint64_t peers = __ballot(e >= 0);
      for (int b = 0; b < bits; ++b) {
        const bool bit = (e >> b) & 1;
        const uint64_t set = __ballot(bit);
        peers &= bit ? set : ~set;
      }
      if (e >= 0) {
        // every lane of the group reads the running count before its lowest
        // lane adds the group (LDS operations of a wave complete in order)
        const int before = counted[e];
        local_rank[p] = static_cast<int16_t>(before + __popcll(peers & lanes_below(lane)));
        if (lane == __builtin_ctzll(peers)) counted[e] = static_cast<int16_t>(before + __popcll(peers));
      }
    }
    __syncthreads();
    for (int p = tid; p < pairs; p += kPrepareThreads) {
      const int e = sorted[p];
      if (e < 0) continue;
      const int owner = (p / 64) / per_wave;
      int rank = local_rank[p];
      for (int v = 0; v < owner; ++v) rank += shared.wave_counts[v * a.E + e];
      const int at = kGroupPairs * (base[e] >> 16) + rank;
      a.group_pairs[at] = p;
      a.pair_tiles[p] = at;
    }
  }
  if (tid == 0) *a.group_total = total_tiles;
}

// One-token routing on one wave, in one round trip and without barriers (the
// same lists as route_and_group). Lane k < K holds slot k's id and weight;
// its rank among the token's ids (ties by slot) and the summed weight of
// equal ids come from lane reads, each lane's sorted id travels to its rank
// by a forward permute, and the runs of equal sorted ids (ascending, absent
// slots first) are the experts' pair lists, cut into tiles of 16.
//
// The slot's id words, weight (both formats) and the token's padding flag:
// buffer loads of every format, none behind a branch (a resource of zero
// bytes reads zero: no padding mask means an active token).
struct RouteLoads {
  int word0, word1;
  uint32_t weight_bits, weight_half, padded;
};

__device__ __forceinline__ RouteLoads route_loads(const PrepareArgs &a) {
  const int lane = threadIdx.x & 63;
  const int K = a.K;
  const int p = lane < K ? lane : K - 1;
  const bool ids64 = (a.flags & CFMOE_IDS_INT64) != 0, weights16 = (a.flags & CFMOE_WEIGHTS_BF16) != 0;
  const __amdgpu_buffer_rsrc_t ids = buffer_resource(a.router_ids, K * (ids64 ? 8 : 4));
  const __amdgpu_buffer_rsrc_t weights = buffer_resource(a.router_weights, K * (weights16 ? 2 : 4));
  const __amdgpu_buffer_rsrc_t padding = buffer_resource(a.padding_source, a.padding_bytes);
  RouteLoads l;
  l.word0 = __builtin_amdgcn_raw_buffer_load_b32(ids, (ids64 ? 8 : 4) * p, 0, 0);
  l.word1 = __builtin_amdgcn_raw_buffer_load_b32(ids, 8 * p + 4, 0, 0);
  l.weight_bits = __builtin_amdgcn_raw_buffer_load_b32(weights, 4 * p, 0, 0);
  l.weight_half = __builtin_amdgcn_raw_buffer_load_b16(weights, 2 * p, 0, 0);
  l.padded = __builtin_amdgcn_raw_buffer_load_b8(padding, 0, 0, 0);
  return l;
}

// The token's routing as lane values: lane k < K holds slot k's id and its
// sorted position (rank); lane q holds the sorted id at position q (-1:
// absent, a padded token, or q >= K), the routed weight there, its run of
// equal ids and its tile slot; `starts` marks the positions that start a tile.
struct TokenRoute {
  int id, rank, sorted, run_end, at;
  float weight;
  bool active, valid, tile_start;
  uint64_t starts;
};

__device__ __forceinline__ TokenRoute route_token(const PrepareArgs &a, const RouteLoads &l) {
  const int lane = threadIdx.x & 63;
  const int K = a.K;
  const bool in = lane < K;
  const bool ids64 = (a.flags & CFMOE_IDS_INT64) != 0, weights16 = (a.flags & CFMOE_WEIGHTS_BF16) != 0;
  // (ids outside the int32 range are absent)
  const int raw = !ids64 ? l.word0 : l.word1 == (l.word0 >> 31) ? l.word0 : -1;
  const float weight = weights16 ? bf16f(static_cast<uint16_t>(l.weight_half)) : __uint_as_float(l.weight_bits);
  TokenRoute r;
  r.active = __builtin_amdgcn_readfirstlane(l.padded) == 0;
  r.id = (raw < 0 || raw >= a.E) ? -1 : raw;
  int rank = 0;
  float w = 0.0f;  // sum of the weights of equal ids in slot order
  for (int j = 0; j < K; ++j) {
    const int other = __builtin_amdgcn_readlane(r.id, j);
    const float other_weight = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(weight), j));
    rank += other < r.id || (other == r.id && j < lane);
    if (other == r.id) w += other_weight;
  }
  if (!r.active) w = 0.0f;
  r.rank = rank;
  // lane q: the sorted id and routed weight at position q
  const int target = 4 * (in ? rank : lane);
  int sorted = __builtin_amdgcn_ds_permute(target, r.active ? r.id : -1);
  r.weight = __int_as_float(__builtin_amdgcn_ds_permute(target, __float_as_int(w)));
  sorted = in ? sorted : -1;
  r.sorted = sorted;
  r.valid = sorted >= 0;
  const int before = __shfl(sorted, max(lane - 1, 0));
  const uint64_t heads = __ballot(r.valid && (lane == 0 || before != sorted));
  const uint64_t upto = lane == 63 ? ~0ull : (2ull << lane) - 1ull;  // lanes 0 .. lane
  const int run_start = r.valid ? 63 - __builtin_clzll(heads & upto) : 0;
  const uint64_t later = heads & ~upto;
  r.run_end = later ? __builtin_ctzll(later) : K;
  const int offset = lane - run_start;
  r.tile_start = r.valid && offset % kGroupPairs == 0;
  r.starts = __ballot(r.tile_start);
  const int z = __popcll(r.starts & upto) - 1;
  r.at = kGroupPairs * z + offset % kGroupPairs;
  return r;
}

// The routing outputs of a one-token call: sorted ids and weights, each
// pair's tile slot, the tile lists (the runs of equal sorted ids, absent
// slots first, cut into tiles of 16), the tile count and the accounting.
__device__ __forceinline__ void store_token_route(const PrepareArgs &a, const TokenRoute &r) {
  const int lane = threadIdx.x & 63;
  const bool in = lane < a.K;
  if (in) {
    a.ids[r.rank] = r.id;
    a.weights[lane] = r.weight;
    a.pair_tiles[lane] = r.valid ? r.at : -1;
  }
  if (r.valid) a.group_pairs[r.at] = lane;
  if (r.tile_start) {
    const int z = r.at / kGroupPairs;
    a.group_experts[z] = r.sorted;
    a.group_starts[z] = kGroupPairs * z;
    a.group_counts[z] = min(kGroupPairs, r.run_end - lane);
  }
  const int total_tiles = __popcll(r.starts);
  if (lane == 0) *a.group_total = total_tiles;
  const bool active = r.active;
  if (a.flags & CFMOE_ACCOUNT) {
    // (uniform indices: the charges stay kernel arguments, not private memory)
#pragma unroll
    for (int i = 0; i < 18; ++i)
      if (lane == i && a.charges[i] != 0.0 && active) atomicAdd(a.read_work + i, a.charges[i]);
    const double tiles = static_cast<double>(total_tiles);
    if (lane == 32 && a.tile_sketch_bytes != 0.0 && total_tiles > 0)
      atomicAdd(a.read_work + 11, tiles * a.tile_sketch_bytes);
    if (lane == 33 && a.tile_screen_macs != 0.0 && total_tiles > 0)
      atomicAdd(a.read_work + 15, tiles * a.tile_screen_macs);
    if (lane == 34 && a.tile_row_bytes != 0.0 && total_tiles > 0)
      atomicAdd(a.read_work + 12, tiles * a.tile_row_bytes);
  }
}

// The routing of a one-token call on one wave, in one round trip and without
// barriers: the same lists as route_and_group.
__device__ __forceinline__ void route_single_token(const PrepareArgs &a) {
  // (the arguments the stores and the accounting use, loaded in one batch)
  asm volatile("" ::"s"(a.ids), "s"(a.weights), "s"(a.pair_tiles), "s"(a.group_pairs),
               "s"(a.group_experts), "s"(a.group_starts), "s"(a.group_counts), "s"(a.group_total),
               "s"(a.read_work), "s"(a.tile_sketch_bytes), "s"(a.tile_screen_macs),
               "s"(a.tile_row_bytes), "s"(a.charges[0]), "s"(a.charges[1]), "s"(a.charges[2]),
               "s"(a.charges[3]), "s"(a.charges[4]), "s"(a.charges[5]), "s"(a.charges[6]),
               "s"(a.charges[7]), "s"(a.charges[8]), "s"(a.charges[9]), "s"(a.charges[10]),
               "s"(a.charges[11]), "s"(a.charges[12]), "s"(a.charges[13]), "s"(a.charges[14]),
               "s"(a.charges[15]), "s"(a.charges[16]), "s"(a.charges[17]));
  const RouteLoads l = route_loads(a);
  asm volatile("" ::"v"(l.word0), "v"(l.word1), "v"(l.weight_bits), "v"(l.weight_half), "v"(l.padded));
  store_token_route(a, route_token(a, l));
}

// One (token, 128-block) cell of the rotation on one wave (progressive.py:
// 389-453): lanes hold coordinates lane and 64 + lane of the signed hidden
// block. Seven butterflies on lane exchanges in xor order (lane_xor: the
// FP32 sums of the xor tree) and the 1/sqrt(128) scale; the keep largest
// magnitudes by bisection on their bits (ties to the lowest coordinate);
// their 21-bit grid values on the kept peak's exponent, the grid sum and
// (kNorm) the kept values' squared norm, summed in compacted order through
// the wave's 128 floats of LDS. `sync` orders the wave's LDS writes before
// its reads (a block barrier where every wave of the block calls it).
struct Cell {
  float v0, v1;
  bool kept0, kept1;
  int pos0, pos1;
  int32_t q0, q1;
  int shift, qsum;
  float sq;
};

template <bool kNorm, class Sync>
__device__ __forceinline__ Cell cell_grid(float v0, float v1, int keep, float *compact, Sync sync) {
  const int lane = threadIdx.x & 63;
  // butterfly stage m: (l + r, l - r) of lanes l and l ^ m
  auto stage = [&](auto mask) {
    constexpr int kMask = decltype(mask)::value;
    const float p0 = lane_xor<kMask>(v0), p1 = lane_xor<kMask>(v1);
    v0 = (lane & kMask) ? p0 - v0 : v0 + p0;
    v1 = (lane & kMask) ? p1 - v1 : v1 + p1;
  };
  stage(std::integral_constant<int, 1>());
  stage(std::integral_constant<int, 2>());
  stage(std::integral_constant<int, 4>());
  stage(std::integral_constant<int, 8>());
  stage(std::integral_constant<int, 16>());
  stage(std::integral_constant<int, 32>());
  {
    float s = v0 + v1, d = v0 - v1;
    v0 = s * 0.08838834764831845f;
    v1 = d * 0.08838834764831845f;
  }
  const uint32_t m0 = __float_as_uint(v0) & 0x7fffffffu;
  const uint32_t m1 = __float_as_uint(v1) & 0x7fffffffu;
  bool kept0 = true, kept1 = true;
  if (keep < 128) {
    // the keep-th largest magnitude by bisection on its bits; when exactly
    // `keep` magnitudes reach the probe, it is the least of them
    uint32_t low = 0, high = 0x7fffffffu;
    while (low < high) {
      uint32_t middle = low + ((high - low + 1u) >> 1);
      int count = __popcll(__ballot(m0 >= middle)) + __popcll(__ballot(m1 >= middle));
      if (count == keep) {
        low = wave_extreme<false>(min(m0 >= middle ? m0 : ~0u, m1 >= middle ? m1 : ~0u));
        break;
      }
      if (count > keep) low = middle; else high = middle - 1u;
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
  Cell c;
  c.v0 = v0;
  c.v1 = v1;
  c.kept0 = kept0;
  c.kept1 = kept1;
  const uint64_t k0 = __ballot(kept0), k1 = __ballot(kept1);
  c.pos0 = __popcll(k0 & lanes_below(lane));
  c.pos1 = __popcll(k0) + __popcll(k1 & lanes_below(lane));
  c.sq = 0.0f;
  if (kNorm) {
    if (kept0) compact[c.pos0] = v0;
    if (kept1) compact[c.pos1] = v1;
    sync();
    float sq = lane < keep ? compact[lane] * compact[lane] : 0.0f;
    if (lane + 64 < keep) sq = fmaf(compact[lane + 64], compact[lane + 64], sq);
    // (the xor-butterfly sum over the lanes, levels m = 1, 2, ..., 32)
    c.sq = wave_sum_lane0(sq);
  }
  const uint32_t peak = wave_extreme<true>(max(kept0 ? m0 : 0u, kept1 ? m1 : 0u));
  int exponent = 0;
  if (peak) frexpf(__uint_as_float(peak), &exponent);
  c.shift = peak ? 20 - exponent : 0;
  c.q0 = kept0 && peak ? static_cast<int32_t>(rintf(ldexpf(v0, c.shift))) : 0;
  c.q1 = kept1 && peak ? static_cast<int32_t>(rintf(ldexpf(v1, c.shift))) : 0;
  // sum of the cell's grid values (exact in any order: |q| <= 2^20, 128 values)
  c.qsum = wave_sum_all(c.q0 + c.q1);
  return c;
}

// A cell's rotated plane, kept coordinates, grid values and digit planes,
// its grid sum, exponent and kept norm (lane 0) into the workspace.
__device__ __forceinline__ void store_cell(const PrepareArgs &a, long cell, const Cell &c) {
  const int lane = threadIdx.x & 63, keep = a.keep;
  if (lane == 0) {
    a.norm2[cell] = c.sq;
    a.qexp[cell] = c.shift;
    a.qsums[cell] = c.qsum;
  }
  if (c.kept0) {
    a.planes[cell * keep + c.pos0] = c.v0;
    a.qvals[cell * keep + c.pos0] = c.q0;
    if (keep < 128) a.coords[cell * keep + c.pos0] = lane;
  }
  if (c.kept1) {
    a.planes[cell * keep + c.pos1] = c.v1;
    a.qvals[cell * keep + c.pos1] = c.q1;
    if (keep < 128) a.coords[cell * keep + c.pos1] = 64 + lane;
  }
  // the dense digit planes the screen stages (zero where not kept: q = 0)
  int8_t *row = a.digits + cell * 3 * 128;
  int d0, d1, d2;
  grid_digits(c.q0, d0, d1, d2);
  row[lane] = static_cast<int8_t>(d0);
  row[128 + lane] = static_cast<int8_t>(d1);
  row[256 + lane] = static_cast<int8_t>(d2);
  grid_digits(c.q1, d0, d1, d2);
  row[64 + lane] = static_cast<int8_t>(d0);
  row[192 + lane] = static_cast<int8_t>(d1);
  row[320 + lane] = static_cast<int8_t>(d2);
}

template <int kPrepareThreads>
__global__ __launch_bounds__(kPrepareThreads) void prepare_kernel(PrepareArgs a) {
  constexpr int kPrepareWaves = kPrepareThreads / 64;
  // block 0 routes and groups (the longest block, dispatched first)
  extern __shared__ __align__(16) char route_lds[];
  __shared__ int route_scratch[32];
  if (a.route && blockIdx.x == 0 && a.T == 1) {
    if (threadIdx.x < 64) route_single_token(a);
    return;
  }
  if (a.route && blockIdx.x == 0) {
    const RouteShared shared = route_layout(route_lds, a.T * a.K, a.E);
    if (a.flags & CFMOE_IDS_INT64) {
      if (a.flags & CFMOE_WEIGHTS_BF16) route_and_group<kPrepareThreads, true, true>(a, shared, route_scratch);
      else route_and_group<kPrepareThreads, true, false>(a, shared, route_scratch);
    } else {
      if (a.flags & CFMOE_WEIGHTS_BF16) route_and_group<kPrepareThreads, false, true>(a, shared, route_scratch);
      else route_and_group<kPrepareThreads, false, false>(a, shared, route_scratch);
    }
    return;
  }
  const int cell_block = static_cast<int>(blockIdx.x) - (a.route ? 1 : 0);
  __shared__ float compact_all[kPrepareWaves][128];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // waves past the last cell still reach the block barrier below
  const int cell_id = min(cell_block * kPrepareWaves + wave, a.cells - 1);
  const bool owner = cell_block * kPrepareWaves + wave < a.cells;
  const int B = a.H / 128;
  const int t = cell_id / B, b = cell_id % B;
  float *compact = compact_all[wave];
  const bool active = is_active(a.padding, t);
  if (!a.rotate) return;

  const int H = a.H, keep = a.keep;
  const int base = b * 128;
  const float v0 = active ? bf16f(a.x[static_cast<long>(t) * H + base + lane]) : 0.0f;
  const float v1 = active ? bf16f(a.x[static_cast<long>(t) * H + base + 64 + lane]) : 0.0f;
  const Cell cell = cell_grid<true>(v0 * static_cast<float>(a.signs[base + lane]),
                                    v1 * static_cast<float>(a.signs[base + 64 + lane]), keep, compact,
                                    [] { __syncthreads(); });
  if (!owner) return;
  store_cell(a, static_cast<long>(t) * B + b, cell);
}

// ---------------------------------------------------------------------------
// screen (progressive.py:478-1108, expert-major as :2428-2606)
//
// Trit planes. The sketch codes hold five trits per byte (byte = sum of
// (t_d + 1) 3^d; byte column j of a coordinate row is plane j % 2, channels
// 5 (j / 2) .. + 4; sketch.py:84-150). The reader repacks them once per layer
// (pack_trit_planes_kernel) into 2-bit digits t + 1 laid out as the screen's
// MFMA A operands: for expert e, block b, row tile rt (gate/up rows
// 16 rt .. 16 rt + 15, rows 0..I-1 gate channels, I..2I-1 up channels) and
// lane l, the uint2 at ((e B + b) RT + rt) 64 + l (RT = 2I / 16) holds in its
// word h the 16 digits of row 16 rt + l % 16 at coordinates
// 64 h + 16 (l / 16) + k, k = 0..15, digit k at bits 8 (k % 4) + 2 (k / 4).
// (word >> 2 s) & 0x03030303 is then operand dword s (k = 4 s .. 4 s + 3):
// one 8-byte coalesced load and eight bit operations give a lane both of its
// operands for a block. 64 I B bytes per expert (2 bits per trit).

constexpr int kRowTile = 16;
constexpr int kPairTile = 16;
static_assert(kPairTile == kGroupPairs, "a screen workgroup holds one grouping tile");
// Rotation blocks per split: the screens are compiled for a span of 2
// (H <= 2048: the common shapes, registers and LDS sized for them) and of
// kMaxSpan (H <= 4096, e.g. Gemma's 2816 = 22 blocks: seven splits of three
// blocks and one of one).
constexpr int kNarrowSpan = 2;
constexpr int kMaxSpan = 4;
constexpr int kDigitStride = 144;  // bytes per pair row of a digit plane (128 + pad)
constexpr int kMaxRows = 4096;     // 2 I gate/up rows of one expert (I <= 2048)

typedef int v4i __attribute__((ext_vector_type(4)));

struct PackArgs {
  const uint8_t *codes;
  uint2 *planes;
  uint8_t *codes_out;  // unpack_trit_planes_kernel's output
  long storage;  // code bytes per expert
  long total;    // uint2 words: E B RT 64
  int I, B, body;
};

__global__ __launch_bounds__(256) void pack_trit_planes_kernel(PackArgs a) {
  const long index = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  if (index >= a.total) return;
  const int lane = static_cast<int>(index % 64);
  const int RT = 2 * a.I / kRowTile;
  const long tile = index / 64;
  const int rt = static_cast<int>(tile % RT);
  const int b = static_cast<int>((tile / RT) % a.B);
  const long e = tile / RT / a.B;
  const int row = kRowTile * rt + lane % 16;
  const int gate_up = row / a.I, channel = row % a.I;
  const int j = 2 * (channel / 5) + gate_up, d = channel % 5;
  const uint32_t power = d == 0 ? 1u : d == 1 ? 3u : d == 2 ? 9u : d == 3 ? 27u : 81u;
  const uint8_t *codes = a.codes + e * a.storage;
  // body: [block][coordinate][body bytes]; the last 16 bytes of a stride that
  // is not a multiple of 32 sit in block-paired tail rows [block / 2][coordinate][32]
  const long column = j < a.body
                          ? static_cast<long>(b) * 128 * a.body + j
                          : static_cast<long>(a.B) * 128 * a.body + (b / 2) * 4096 + (b % 2) * 16 +
                                (j - a.body);
  const int coordinate_bytes = j < a.body ? a.body : 32;
  uint32_t word[2] = {0u, 0u};
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int c = 64 * h + 16 * (lane / 16) + k;
      const uint32_t digit = (codes[column + static_cast<long>(c) * coordinate_bytes] / power) % 3u;
      word[h] |= digit << (8 * (k % 4) + 2 * (k / 4));
    }
  a.planes[index] = make_uint2(word[0], word[1]);
}

// The inverse repacking: thread per code byte of the sketch storage (body,
// then the block-paired tail rows), five channels' digits read back from the
// planes; bytes that carry no channel (a channel past I, the missing half of
// an odd block count's last tail row) hold 121, five zero trits.
__global__ __launch_bounds__(256) void unpack_trit_planes_kernel(PackArgs a) {
  const long index = static_cast<long>(blockIdx.x) * 256 + threadIdx.x;
  const long experts_bytes = a.total;  // E * storage
  if (index >= experts_bytes) return;
  const long e = index / a.storage;
  const long at = index % a.storage;
  const long body_bytes = static_cast<long>(a.B) * 128 * a.body;
  int b, c, j;
  if (at < body_bytes) {
    b = static_cast<int>(at / (128L * a.body));
    const long rest = at % (128L * a.body);
    c = static_cast<int>(rest / a.body);
    j = static_cast<int>(rest % a.body);
  } else {
    const long rest = at - body_bytes;
    const int in_row = static_cast<int>(rest % 4096);
    b = 2 * static_cast<int>(rest / 4096) + (in_row % 32) / 16;
    c = in_row / 32;
    j = a.body + in_row % 16;
  }
  const int RT = 2 * a.I / kRowTile;
  const int gate_up = j % 2;
  uint32_t byte = 0u;
  for (int d = 4; d >= 0; --d) {
    const int channel = 5 * (j / 2) + d;
    uint32_t digit = 1u;  // a zero trit
    if (b < a.B && channel < a.I) {
      const int row = gate_up * a.I + channel;
      const int lane = 16 * ((c % 64) / 16) + row % kRowTile;
      const uint2 w = a.planes[((e * a.B + b) * RT + row / kRowTile) * 64 + lane];
      const int k = c % 16;
      digit = (((c / 64) ? w.y : w.x) >> (8 * (k % 4) + 2 * (k / 4))) & 3u;
    }
    byte = 3u * byte + digit;
  }
  a.codes_out[index] = static_cast<uint8_t>(byte);
}

__device__ __forceinline__ v4i expand_digits(uint32_t x) {
  return v4i{static_cast<int>(x & 0x03030303u), static_cast<int>((x >> 2) & 0x03030303u),
             static_cast<int>((x >> 4) & 0x03030303u), static_cast<int>((x >> 6) & 0x03030303u)};
}

// The gate (up = 0) and up (up = 1) row tiles' integer dots with a pair's
// grid values q = d0 + 2^8 d1 + 2^16 d2 over one 128-coordinate block, minus
// the block's grid sum (`start`): the trits a come as digits 0..2 (a0 and a1:
// coordinates 0-63 and 64-127), so sum (a - 1) q = sum a q - sum q. The digit
// planes go through one accumulator per row tile, high digit first, the
// running sum shifted left by 8 before each lower digit: ((s2 2^8) + s1) 2^8
// + s0 - qsum, the integer sum_a (d0 + 2^8 d1 + 2^16 d2) - qsum exactly (every
// step is a 32-bit integer add or shift; the top digit is below 2^5 in
// magnitude, so no step leaves the int32 range). operand(h, d) is the B
// operand of coordinate half h and digit d.
template <typename Operand>
__device__ __forceinline__ void digit_dots(const v4i (&a0)[2], const v4i (&a1)[2], int start,
                                           Operand operand, v4i (&acc)[2]) {
  const v4i zero = {0, 0, 0, 0};
  // an opaque start: (x << 8) + start is then one v_lshl_add_u32 (a known
  // negation would become a shift and a subtract). The empty asm emits no
  // instruction; an instruction in inline asm reading an MFMA result would
  // get none of the compiler's wait states for that read.
  asm volatile("" : "+v"(start));
#pragma unroll
  for (int d = 2; d >= 0; --d) {
    const v4i b0 = operand(0, d);
#pragma unroll
    for (int up = 0; up < 2; ++up) {
      v4i c = zero;
      if (d == 1) c = acc[up] << 8;
      if (d == 0)
#pragma unroll
        for (int r = 0; r < 4; ++r) c[r] = (acc[up][r] << 8) + start;
      acc[up] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0[up], b0, c, 0, 0, 0);
    }
    const v4i b1 = operand(1, d);
#pragma unroll
    for (int up = 0; up < 2; ++up) acc[up] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[up], b1, acc[up], 0, 0, 0);
  }
}

__device__ __forceinline__ float half_at(uint32_t word, int high) {
  return static_cast<float>(
      __builtin_bit_cast(_Float16, static_cast<uint16_t>(high ? word >> 16 : word & 0xffffu)));
}

// Zero projections and scores of a padded token's slots and of slots with no
// local expert (the screens cover only grouped pairs); `threads` of the
// workgroup share the channels.
template <bool kGh5, class Args>
__device__ void score_absent_slots(const Args &a, int t, int threads) {
  const bool active = is_active(a.padding, t);
  for (int k = 0; k < a.K; ++k) {
    if (active && a.ids[t * a.K + k] >= 0) continue;
    for (int c = threadIdx.x; c < a.I; c += threads) {
      const long flat = static_cast<long>(t) * a.N + static_cast<long>(k) * a.I + c;
      const long base = static_cast<long>(t) * 2 * a.N + static_cast<long>(k) * a.I + c;
      a.partial[base] = 0.0f;
      a.partial[base + a.N] = 0.0f;
      if (kGh5) {
        a.variances[base] = 0.0f;
        a.variances[base + a.N] = 0.0f;
      }
      a.scores[flat] = cfm_score(0.0f, 0.0f, 0.0f, 0.0f, 0.0f, a.weights[t * a.K + k], 0.0f, 0.0f,
                                 a.gelu != 0, a.point != 0);
    }
  }
}

// Score of four channels for one pair from the gate and up estimates (and
// variances); writes the projections, variances and scores
// (progressive.py:1265-1353).
// The score's inputs for one pair and four channels, loaded ahead of the
// screen's arithmetic (so the epilogue waits on no load of its own).
struct ScoreInputs {
  float weight;
  float norm[4], alpha[4], beta[4];
};

template <class Args>
__device__ __forceinline__ ScoreInputs load_score_inputs(const Args &a, int e, int token, int slot,
                                                         int c) {
  ScoreInputs in;
  in.weight = a.weights[token * a.K + slot];
  const float4 norm = *reinterpret_cast<const float4 *>(a.norms + static_cast<long>(e) * a.I + c);
  in.norm[0] = norm.x;
  in.norm[1] = norm.y;
  in.norm[2] = norm.z;
  in.norm[3] = norm.w;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    in.alpha[r] = 0.0f;
    in.beta[r] = 0.0f;
  }
  if (a.geometry) {
    const float4 g01 = *reinterpret_cast<const float4 *>(a.geometry + (static_cast<long>(e) * a.I + c) * 2);
    const float4 g23 = *reinterpret_cast<const float4 *>(a.geometry + (static_cast<long>(e) * a.I + c) * 2 + 4);
    in.alpha[0] = g01.x;
    in.beta[0] = g01.y;
    in.alpha[1] = g01.z;
    in.beta[1] = g01.w;
    in.alpha[2] = g23.x;
    in.beta[2] = g23.y;
    in.alpha[3] = g23.z;
    in.beta[3] = g23.w;
  }
  return in;
}

template <bool kGh5, class Args>
__device__ __forceinline__ void score_four(const Args &a, int token, int slot, int c,
                                           const float gate[4], const float up[4],
                                           const float gate_var[4], const float up_var[4],
                                           const ScoreInputs &in) {
  const long base = static_cast<long>(token) * 2 * a.N + static_cast<long>(slot) * a.I + c;
  *reinterpret_cast<float4 *>(a.partial + base) = make_float4(gate[0], gate[1], gate[2], gate[3]);
  *reinterpret_cast<float4 *>(a.partial + base + a.N) = make_float4(up[0], up[1], up[2], up[3]);
  if (kGh5) {
    *reinterpret_cast<float4 *>(a.variances + base) =
        make_float4(gate_var[0], gate_var[1], gate_var[2], gate_var[3]);
    *reinterpret_cast<float4 *>(a.variances + base + a.N) =
        make_float4(up_var[0], up_var[1], up_var[2], up_var[3]);
  }
  float score[4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
    score[r] = cfm_score(gate[r], up[r], gate_var[r], up_var[r], in.norm[r], in.weight, in.alpha[r],
                         in.beta[r], a.gelu != 0, a.point != 0);
  *reinterpret_cast<float4 *>(a.scores + static_cast<long>(token) * a.N + static_cast<long>(slot) * a.I + c) =
      make_float4(score[0], score[1], score[2], score[3]);
}

// The projections and score of one (pair, channel).
template <bool kGh5, class Args>
__device__ __forceinline__ void score_one(const Args &a, int token, int slot, int c, float gate, float up,
                                          float gate_var, float up_var, float norm, float weight,
                                          float alpha, float beta) {
  const long base = static_cast<long>(token) * 2 * a.N + static_cast<long>(slot) * a.I + c;
  a.partial[base] = gate;
  a.partial[base + a.N] = up;
  if (kGh5) {
    a.variances[base] = gate_var;
    a.variances[base + a.N] = up_var;
  }
  a.scores[static_cast<long>(token) * a.N + static_cast<long>(slot) * a.I + c] =
      cfm_score(gate, up, gate_var, up_var, norm, weight, alpha, beta, a.gelu != 0, a.point != 0);
}

// ---------------------------------------------------------------------------
// Screen and score below the grouped size (progressive.py:478-1108,
// :1111-1353). Workgroup = (16-pair tile z, channel tile ct: gate row tile
// ct and up row tile I/16 + ct); wave w of the eight takes the block splits
// [w P, (w + 1) P), P = ceil(S / 8) (one split each at S <= 8), and stages, for the tile's live pairs only, those
// blocks' digit planes in its own LDS area (no barrier: a wave reads only what
// it wrote, and its LDS operations complete in order). Per split the wave
// forms the partial (fma chain over the split's blocks) of its 2 x 4 rows for
// every pair, and leaves it in LDS; after one barrier wave 0 sums the splits
// in order, ((part_0 + part_1) + part_2) + ..., and scores the 16 channels.
// The MFMA contraction is that of the fused screen (B operands of pairs past
// the count are zero registers, not LDS reads). Workgroups from tile_items
// on (one per token) write the zero results of padded tokens and absent slots.

constexpr int kSmallWaves = 8;
constexpr int kMaxSplits = 8;

struct SmallScreenArgs {
  const uint2 *planes;
  const uint16_t *stats;
  const int8_t *digits;
  const int32_t *qexp;
  const int32_t *qsums;
  const float *norm2;
  const int32_t *group_experts;
  const int32_t *group_counts;
  const int32_t *group_pairs;
  const int32_t *group_total;
  const int32_t *ids;
  const float *weights;
  const uint8_t *padding;
  const float *norms;
  const float *geometry;
  float *partial;
  float *variances;
  float *scores;
  int H, I, K, N, T, splits, span, tile_items, max_pairs;
  int gelu, point;
};

// One (block, row tile) step's loads: operand words, FP16 scale (and
// residual) words of the lane's four rows.
struct StepLoads {
  uint2 words, scale, residual;
};

// An empty use of a step's registers: the wait for its loads happens here,
// on every path, and not where the compiler would merge paths (a loop head).
__device__ __forceinline__ void consume(const StepLoads &l) {
  asm volatile("" ::"v"(l.words.x), "v"(l.words.y), "v"(l.scale.x), "v"(l.scale.y));
}


constexpr int kWaveSplits = (kMaxSplits + kSmallWaves - 1) / kSmallWaves;

// Dynamic LDS bytes of small_screen_kernel<.., span> for tiles of at most
// `max_pairs`.
__host__ __device__ inline long small_screen_lds(int max_pairs, int span) {
  return static_cast<long>(kSmallWaves) * kWaveSplits * span * 3 * max_pairs * kDigitStride;
}

template <bool kGh5, int kSpan>
__global__ __launch_bounds__(64 * kSmallWaves) void small_screen_kernel(SmallScreenArgs a) {
  constexpr int kWaveBlocks = kWaveSplits * kSpan;
  // per wave: its blocks' digit rows [block][digit][pair < max_pairs][kDigitStride]
  extern __shared__ __align__(16) int8_t small_digits[];
  __shared__ float parts[kMaxSplits][2][64][4];
  __shared__ float vparts[kGh5 ? kMaxSplits : 1][2][64][4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (static_cast<int>(blockIdx.x) >= a.tile_items) {
    const int t = blockIdx.x - a.tile_items;
    if (t < a.T) score_absent_slots<kGh5>(a, t, 64 * kSmallWaves);
    return;
  }
  const int CT = a.I / kRowTile, RT = 2 * CT;
  const int z = blockIdx.x / CT, ct = blockIdx.x % CT;
  // the tile count, the tile's expert, pair count and 16 pair slots through
  // the scalar cache in one round trip (z < tile bound <= T * K keeps every
  // address in bounds whatever the count; slots past the count are unused)
  const int total = load_uniform(a.group_total);
  const int e = load_uniform(a.group_experts + z);
  const int count = load_uniform(a.group_counts + z);
  const i32x16 slots = load_uniform(reinterpret_cast<const i32x16 *>(a.group_pairs + kGroupPairs * z));
  asm volatile("" ::"s"(total), "s"(e), "s"(count), "s"(slots));
  if (z >= total) return;
  const int B = a.H / 128;
  const int pp = lane % 16, k0 = 16 * (lane / 16), row_in_tile = 4 * (lane / 16);
  // lane pp's pair (pairs past the count repeat the last one); lane p < 16
  // holds pair p's token for the staging below
  const int my_row = min(pp, count - 1);
  int my_pair = slots[0];
#pragma unroll
  for (int p = 1; p < kPairTile; ++p) my_pair = my_row == p ? slots[p] : my_pair;
  const int my_token = my_pair / a.K;
  const int span = a.span, splits = a.splits;
  const int per_wave = (splits + kSmallWaves - 1) / kSmallWaves;
  const int s_begin = wave * per_wave, s_end = min(splits, s_begin + per_wave);
  const int b_begin = s_begin * span;
  // the wave's steps (split si, block j, gate/up) are loaded first
  const uint2 *planes = a.planes + static_cast<long>(e) * B * RT * 64 + lane;
  const uint16_t *stats = a.stats + static_cast<long>(e) * B * 4 * a.I + row_in_tile;
  StepLoads step[kWaveSplits][kSpan][2];
#pragma unroll
  for (int si = 0; si < kWaveSplits; ++si)
#pragma unroll
    for (int j = 0; j < kSpan; ++j)
#pragma unroll
      for (int up = 0; up < 2; ++up) {
        const int b = min((s_begin + si) * span + j, B - 1);  // past the range: unused
        const int rt = up ? CT + ct : ct;
        step[si][j][up].words = load_global(planes + (static_cast<long>(b) * RT + rt) * 64);
        const uint16_t *plane = stats + static_cast<long>(b) * 4 * a.I + kRowTile * rt;
        step[si][j][up].scale = load_global(reinterpret_cast<const uint2 *>(plane));
        if (kGh5)
          step[si][j][up].residual = load_global(reinterpret_cast<const uint2 *>(plane + 2 * a.I));
      }
  const bool live_pair = pp < count;
  const long pair_cell = static_cast<long>(my_token) * B;
  // the score's inputs of lane l's first epilogue item (wave 0: pair l / 16,
  // the tile's channel l % 16) in this round trip
  const int item_row = min(lane / kRowTile, count - 1);
  int item_pair = slots[0];
#pragma unroll
  for (int p = 1; p < kPairTile; ++p) item_pair = item_row == p ? slots[p] : item_pair;
  const int item_c = kRowTile * ct + lane % kRowTile;
  const float item_weight = load_global(a.weights + item_pair);
  const float item_norm = load_global(a.norms + static_cast<long>(e) * a.I + item_c);
  const float item_alpha = a.geometry ? load_global(a.geometry + (static_cast<long>(e) * a.I + item_c) * 2) : 0.0f;
  const float item_beta = a.geometry ? load_global(a.geometry + (static_cast<long>(e) * a.I + item_c) * 2 + 1) : 0.0f;
  // the lane's pair's grid sums, exponents (and kept norms) of the wave's blocks
  int qsum[kWaveSplits][kSpan], shift[kWaveSplits][kSpan];
  float n2[kWaveSplits][kSpan];
#pragma unroll
  for (int si = 0; si < kWaveSplits; ++si)
#pragma unroll
    for (int j = 0; j < kSpan; ++j) {
      const long cell = pair_cell + min((s_begin + si) * span + j, B - 1);
      qsum[si][j] = live_pair ? load_global(a.qsums + cell) : 0;
      shift[si][j] = live_pair ? load_global(a.qexp + cell) : 0;
      n2[si][j] = kGh5 && live_pair ? load_global(a.norm2 + cell) : 0.0f;
    }
  // stage the wave's blocks for the live pairs: rows (block, digit, pair) of
  // 128 bytes, eight lanes per row
  int8_t *mine = small_digits + static_cast<long>(wave) * kWaveBlocks * 3 * a.max_pairs * kDigitStride;
  const int wave_rows = max(0, min(B, s_end * span) - min(B, b_begin)) * 3 * count;
  // (the lane read of pair p's token runs with every lane active: a lane
  // read from an inactive lane returns zero)
  for (int base = 0; base < wave_rows * 8; base += 64) {
    const int item = base + lane;
    const int row = item / 8, piece = item % 8;
    const int bl = row / (3 * count), d = (row / count) % 3, p = row % count;
    const long cell = static_cast<long>(__shfl(my_token, p)) * B + b_begin + bl;
    if (item < wave_rows * 8) {
      const uint4 v = load_global(reinterpret_cast<const uint4 *>(a.digits + (cell * 3 + d) * 128) + piece);
      *reinterpret_cast<uint4 *>(mine + ((bl * 3 + d) * a.max_pairs + p) * kDigitStride + 16 * piece) = v;
    }
  }
#pragma unroll
  for (int si = 0; si < kWaveSplits; ++si) {
    const int s = s_begin + si;
    if (s >= s_end) break;
    float part[2][4] = {}, vpart[2][4] = {};
#pragma unroll
    for (int j = 0; j < kSpan; ++j) {
      const int b = s * span + j;
      if (j >= span || b >= B) break;
      const int bl = b - b_begin;
      const int start = -qsum[si][j];
      auto operand = [&](int h, int d) {
        const v4i v = *reinterpret_cast<const v4i *>(
            mine + ((bl * 3 + d) * a.max_pairs + my_row) * kDigitStride + 64 * h + k0);
        return live_pair ? v : v4i{0, 0, 0, 0};
      };
      v4i a0[2], a1[2];
#pragma unroll
      for (int up = 0; up < 2; ++up) {
        a0[up] = expand_digits(step[si][j][up].words.x);
        a1[up] = expand_digits(step[si][j][up].words.y);
      }
      v4i acc[2];
      digit_dots(a0, a1, start, operand, acc);
#pragma unroll
      for (int up = 0; up < 2; ++up)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int sum = acc[up][r];
          const float dot = ldexpf(static_cast<float>(sum), -shift[si][j]);
          const uint32_t sw = r < 2 ? step[si][j][up].scale.x : step[si][j][up].scale.y;
          part[up][r] = fmaf(dot, half_at(sw, r & 1), part[up][r]);
          if (kGh5) {
            const uint32_t rw = r < 2 ? step[si][j][up].residual.x : step[si][j][up].residual.y;
            vpart[up][r] = fmaf(half_at(rw, r & 1), n2[si][j], vpart[up][r]);
          }
        }
    }
#pragma unroll
    for (int up = 0; up < 2; ++up) {
      *reinterpret_cast<float4 *>(&parts[s][up][lane][0]) =
          make_float4(part[up][0], part[up][1], part[up][2], part[up][3]);
      if (kGh5)
        *reinterpret_cast<float4 *>(&vparts[s][up][lane][0]) =
            make_float4(vpart[up][0], vpart[up][1], vpart[up][2], vpart[up][3]);
    }
  }
  __syncthreads();
  if (wave != 0) return;
  // wave 0 sums the splits in order and scores, one (pair p, channel row)
  // item per lane: lane p + 16 (row / 4) holds the item's partials in its
  // register row % 4 (the MFMA result layout)
  for (int i = lane; i < count * kRowTile; i += kWave) {
    const int p = i / kRowTile, row = i % kRowTile;
    const int src = p + kRowTile * (row / 4), r = row % 4;
    float gate = parts[0][0][src][r], up = parts[0][1][src][r];
    float gate_var = kGh5 ? vparts[0][0][src][r] : 0.0f, up_var = kGh5 ? vparts[0][1][src][r] : 0.0f;
    for (int s = 1; s < splits; ++s) {
      gate = gate + parts[s][0][src][r];
      up = up + parts[s][1][src][r];
      if (kGh5) {
        gate_var = gate_var + vparts[s][0][src][r];
        up_var = up_var + vparts[s][1][src][r];
      }
    }
    int pair = item_pair;
    float weight = item_weight, norm = item_norm, alpha = item_alpha, beta = item_beta;
    if (i >= kWave) {  // more than four pairs: this item's inputs
      pair = slots[0];
#pragma unroll
      for (int q = 1; q < kPairTile; ++q) pair = p == q ? slots[q] : pair;
      weight = a.weights[pair];
      norm = a.norms[static_cast<long>(e) * a.I + item_c];
      alpha = a.geometry ? a.geometry[(static_cast<long>(e) * a.I + item_c) * 2] : 0.0f;
      beta = a.geometry ? a.geometry[(static_cast<long>(e) * a.I + item_c) * 2 + 1] : 0.0f;
    }
    score_one<kGh5>(a, pair / a.K, pair % a.K, item_c, gate, up, gate_var, up_var, norm, weight, alpha,
                    beta);
  }
}

// ---------------------------------------------------------------------------
// Fused screen and score for grouped batches (progressive.py:2428-2606 and
// :1111-1353). Wave = (16-pair tile z, channel tile ct): the gate row tile ct
// and the up row tile I/16 + ct, over every rotation block. The blocks run in
// split order; split s's partial is the fma chain over its blocks and the
// estimate is ((part_0 + part_1) + part_2) + ... -- the arithmetic of
// small_screen_kernel, with the partials kept in registers. The workgroup's waves share the tile's digit planes in LDS,
// staged kStageAhead splits ahead (ring of kStageAhead + 1 buffers, one
// barrier per split); a wave's block steps are loaded one split ahead, each
// step's successor issued as soon as the step is used. The score epilogue
// writes the projections and scores of the wave's 16 channels for the tile's
// pairs. Workgroups past the tiles (one per token) write the zero projections
// and scores of padded tokens and absent slots.

constexpr int kFusedWaves = 4;
constexpr int kFusedThreads = 64 * kFusedWaves;
// FP16 scale entries of a block: gate and up, each wave's row tile, four
// entries of four rows each
constexpr int kScaleQuads = kRowTile / 4;
constexpr int kScaleBlock = 2 * kFusedWaves * kScaleQuads;
// Tokens from which the fused screen runs: the per-channel-tile workgroups of
// small_screen_kernel do a whole tile's work for each one-pair tile, so from
// two tokens the fused screen is faster (Qwen3 layer: 13.0 against 17.2 us at
// 2 tokens, 20.8 against 54.0 at 8; at one token 12.8 against 8.5).
constexpr int kFusedScreenTokens = 2;
constexpr int kStageAhead = 1;
constexpr int kStageBuffers = kStageAhead + 1;

struct FusedScreenArgs {
  const uint2 *planes;
  const uint16_t *stats;
  const int8_t *digits;
  const int32_t *qexp;
  const int32_t *qsums;
  const float *norm2;
  const int32_t *ids;
  const float *weights;
  const uint8_t *padding;
  const float *norms;
  const float *geometry;
  const int32_t *group_experts;
  const int32_t *group_counts;
  const int32_t *group_pairs;
  const int32_t *group_total;
  float *partial;
  float *variances;
  float *scores;
  uint32_t *tile_masks;  // cleared for the wave's channels (or NULL)
  int H, I, K, N, T, splits, span, channel_groups, tile_items;
  int gelu, point;
};

template <bool kGh5, int kSpan>
struct FusedShared {
  alignas(16) int8_t digits[kStageBuffers][kSpan][3][kPairTile][kDigitStride];
  // the split's FP16 scales (and residual scales) of the workgroup's gate and
  // up row tiles (one of each per wave): entry kScaleBlock (kSpan kind + bl)
  // + 4 kFusedWaves up + 4 w + q holds rows 4q .. 4q + 3 of wave w's row tile
  uint2 scales[kStageBuffers][(kGh5 ? 2 : 1) * kSpan * kScaleBlock];
  int qsum[kSpan * kMaxSplits][kPairTile];  // blocks x pairs
  int shift[kSpan * kMaxSplits][kPairTile];
  float norm2[kGh5 ? kSpan * kMaxSplits : 1][kPairTile];
  int pair_token[kPairTile], pair_slot[kPairTile];
};

template <bool kGh5, int kSpan>
__global__ __launch_bounds__(kFusedThreads) __attribute__((amdgpu_waves_per_eu(kSpan == kNarrowSpan ? (kGh5 ? 3 : 5) : 2))) void fused_screen_kernel(FusedScreenArgs a) {
  __shared__ FusedShared<kGh5, kSpan> sh;
  // (the wave index through a scalar register: every wave-uniform address
  // term below is then scalar arithmetic, not a vector instruction per lane)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int B = a.H / 128;
  if (static_cast<int>(blockIdx.x) >= a.tile_items) {
    const int t = blockIdx.x - a.tile_items;
    if (t < a.T) score_absent_slots<kGh5>(a, t, kFusedThreads);
    return;
  }
  const int z = blockIdx.x / a.channel_groups;
  if (z >= load_uniform(a.group_total)) return;
  const int CT = a.I / kRowTile, RT = 2 * CT;
  const int group = blockIdx.x % a.channel_groups;
  const int ct = group * kFusedWaves + wave;
  const bool working = ct < CT;  // a wave past the channels still stages and waits
  const int cc = min(ct, CT - 1);
  const int e = load_uniform(a.group_experts + z);
  const int count = load_uniform(a.group_counts + z);
  const int pp = lane % 16, k0 = 16 * (lane / 16), row_in_tile = 4 * (lane / 16);
  const int span = a.span, splits = a.splits;
  // the wave's trit planes: gate row tile cc, up row tile CT + cc (a
  // wave-uniform row-tile base, lane l's 8 bytes at 8 l); the scales come
  // with the staging
  const uint2 *planes = a.planes + static_cast<long>(e) * B * RT * 64;
  const uint16_t *stats = a.stats + static_cast<long>(e) * B * 4 * a.I;
  auto load_step = [&](int s, int bl, int up) {
    const int b = min(s * span + min(bl, span - 1), B - 1);  // past H: a repeat, unused
    const int rt = up ? CT + cc : cc;
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(
        buffer_resource(planes + (b * RT + rt) * 64, 64 * 8), lane * 8, 0, 0);
    return make_uint2(v.x, v.y);
  };
  // split 0's steps in flight while the tile is staged; each step's
  // successor (the next split's) is loaded into its registers as soon as the
  // step is expanded
  uint2 step[kSpan][2];
#pragma unroll
  for (int bl = 0; bl < kSpan; ++bl)
#pragma unroll
    for (int up = 0; up < 2; ++up) step[bl][up] = load_step(0, bl, up);

  // ---- the tile's pairs (through the scalar cache: the tile list is an
  // earlier launch's output) and per-(block, pair) constants
  if (tid < kPairTile) {
    const i32x8 lo = load_uniform(reinterpret_cast<const i32x8 *>(a.group_pairs + kGroupPairs * z));
    const i32x8 hi = load_uniform(reinterpret_cast<const i32x8 *>(a.group_pairs + kGroupPairs * z + 8));
    int pair = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      pair = tid == q ? lo[q] : pair;
      pair = tid == q + 8 ? hi[q] : pair;
    }
    pair = tid < count ? pair : 0;
    sh.pair_token[tid] = pair / a.K;
    sh.pair_slot[tid] = pair % a.K;
  }
  __syncthreads();
  // thread tid's (block, pair) entries: tid = 16 b + p, then 16 (b + 16) + p
  // at span 4 (up to 32 blocks); loaded with the first split's staging,
  // stored after it
  constexpr int kTableBlocks = kSpan * kMaxSplits;
  constexpr int kTableRounds = (kTableBlocks * kPairTile + kFusedThreads - 1) / kFusedThreads;
  const int tp = tid % kPairTile;
  int qsum_value[kTableRounds], shift_value[kTableRounds];
  float norm2_value[kTableRounds];
  bool table_live[kTableRounds];
#pragma unroll
  for (int r = 0; r < kTableRounds; ++r) {
    const int tb = tid / kPairTile + r * (kFusedThreads / kPairTile);
    table_live[r] = tb < B && tp < count;
    const int table_cell = table_live[r] ? sh.pair_token[tp] * B + tb : 0;
    qsum_value[r] = load_global(a.qsums + table_cell);
    shift_value[r] = load_global(a.qexp + table_cell);
    norm2_value[r] = kGh5 ? load_global(a.norm2 + table_cell) : 0.0f;
  }
  // staging of split s: rows (block, digit, pair) of 128 bytes, 16 bytes per
  // thread and item. Every load is unconditional and in bounds: a pair past
  // the count reads the tile's first pair (its MFMA B column feeds only that
  // pair's unused results) and a block past H or the split reads block B - 1
  // (never used)
  constexpr int kStageRows = kSpan * 3 * kPairTile;
  constexpr int kStageItems = kStageRows * 8;  // uint4 per split
  constexpr int kStagePerThread = kStageItems / kFusedThreads;
  static_assert(kStageItems % kFusedThreads == 0, "staging items per thread");
  // an item's block (item / 384) is wave-uniform: 384 items are six waves
  static_assert((8 * 3 * kPairTile) % kWave == 0, "staging blocks change at wave boundaries");
  // Thread i also loads scale entry i (see FusedShared; threads past the
  // entries repeat entry i % entries, and a row tile past the channels reads
  // the last one). Lane offsets are fixed; per split the entries come through
  // a buffer resource over the split's blocks to the expert's last, so an
  // entry of a block past the expert (never used) reads zeros
  constexpr int kScaleEntries = (kGh5 ? 2 : 1) * kSpan * kScaleBlock;
  static_assert(kScaleEntries <= kFusedThreads, "one scale entry per thread at most");
  const int sentry = tid % kScaleEntries;
  const int sk = kGh5 ? sentry / (kScaleBlock * kSpan) : 0, sbl = (sentry / kScaleBlock) % kSpan;
  const int within = sentry % kScaleBlock;
  const int sup = within / (kFusedWaves * kScaleQuads), sw = (within / kScaleQuads) % kFusedWaves;
  const int stile = (sup ? CT : 0) + min(group * kFusedWaves + sw, CT - 1);
  const int srow = (sk ? 2 * a.I : 0) + kRowTile * stile + 4 * (within % kScaleQuads);
  const int scale_offset = (sbl * 4 * a.I + srow) * 2;
  // each staging item's byte offset without its block term (fixed per thread)
  int stage_offset[kStagePerThread];
#pragma unroll
  for (int j = 0; j < kStagePerThread; ++j) {
    const int item = tid + j * kFusedThreads;
    const int row = item / 8, piece = item % 8;
    const int d = (row / kPairTile) % 3, p = row % kPairTile;
    stage_offset[j] = sh.pair_token[min(p, max(count, 1) - 1)] * B * 384 + d * 128 + 16 * piece;
  }
  auto stage_load = [&](int s, uint4 *held, uint2 &scale) {
#pragma unroll
    for (int j = 0; j < kStagePerThread; ++j) {
      const int bl = (kWave * wave + j * kFusedThreads) / (8 * 3 * kPairTile);
      const int b = min(s * span + bl, B - 1);
      held[j] = buffer_load16(buffer_resource(a.digits + b * 384, (a.T * B - b) * 384), stage_offset[j]);
    }
    const int first = min(s * span, B);  // B for the prefetch past the last split: no records
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(
        buffer_resource(stats + first * 4 * a.I, (B - first) * 8 * a.I), scale_offset, 0, 0);
    scale = make_uint2(v.x, v.y);
  };
  // (row (bl 3 + d) 16 + p of a buffer is item / 8: one base offset per
  // thread, item j a constant past it)
  auto stage_store = [&](int buffer, const uint4 *held, uint2 scale) {
    int8_t *rows = &sh.digits[buffer][0][0][0][0] + (tid / 8) * kDigitStride + 16 * (tid % 8);
#pragma unroll
    for (int j = 0; j < kStagePerThread; ++j)
      *reinterpret_cast<uint4 *>(rows + j * (kFusedThreads / 8) * kDigitStride) = held[j];
    sh.scales[buffer][tid % kScaleEntries] = scale;
  };
  uint4 held[kStagePerThread];
  uint2 held_scale;
  static_assert(kStageAhead == 1, "one split staged ahead");
  stage_load(0, held, held_scale);
  // (no store moves above this point: the table and staging loads are all
  // issued before the first wait)
  asm volatile("" ::: "memory");
#pragma unroll
  for (int r = 0; r < kTableRounds; ++r) {
    const int tb = tid / kPairTile + r * (kFusedThreads / kPairTile);
    // (stored negated: the block's chain starts from -qsum and scales by
    // 2^-shift)
    if (kTableRounds * (kFusedThreads / kPairTile) > kTableBlocks && tb >= kTableBlocks) continue;
    sh.qsum[tb][tp] = table_live[r] ? -qsum_value[r] : 0;
    sh.shift[tb][tp] = table_live[r] ? -shift_value[r] : 0;
    if (kGh5) sh.norm2[kGh5 ? tb : 0][tp] = table_live[r] ? norm2_value[r] : 0.0f;
  }
  stage_store(0, held, held_scale);
  __syncthreads();

  float est[2][4] = {}, var[2][4] = {};
  // splits from ceil(B / span) on hold no block (B = 9: splits 5-7 of span
  // 2): their zero partials are added after the loop, so every split in it
  // has a first block below B
  const int live_splits = (B + span - 1) / span;
  for (int s = 0; s < live_splits; ++s) {
    const int buffer = s % kStageBuffers;
    // split s + kStageAhead's digits go to the buffer split s - 1 used, which
    // every wave finished before the last barrier
    stage_load(s + kStageAhead, held, held_scale);
    // (a split's first block, always below B, starts the chains from zero
    // as an fma operand; a later block past the split or H leaves them)
    float part[2][4], vpart[2][4];
#pragma unroll
    for (int bl = 0; bl < kSpan; ++bl) {
      const int b = s * span + bl;
      const bool live_block = bl == 0 || (bl < span && b < B);
      const int start = sh.qsum[min(b, B - 1)][pp], shift = sh.shift[min(b, B - 1)][pp];
      const float n2 = kGh5 ? sh.norm2[kGh5 ? min(b, B - 1) : 0][pp] : 0.0f;
      auto operand = [&](int h, int d) {
        return *reinterpret_cast<const v4i *>(&sh.digits[buffer][bl][d][pp][64 * h + k0]);
      };
      // gate and up row tiles share each B operand read; the expanded step's
      // registers take its successor (a repeat past the last split)
      v4i a0[2], a1[2];
#pragma unroll
      for (int up = 0; up < 2; ++up) {
        a0[up] = expand_digits(step[bl][up].x);
        a1[up] = expand_digits(step[bl][up].y);
        // (the successor load stays below the expansion, so it can take the
        // step's own registers: no copy round the loop waits for it)
        asm volatile("" ::"v"(a0[up]), "v"(a1[up]) : "memory");
        step[bl][up] = load_step(s + 1 < live_splits ? s + 1 : s, bl, up);
      }
      if (!live_block) continue;
      v4i acc[2];
      digit_dots(a0, a1, start, operand, acc);
#pragma unroll
      for (int up = 0; up < 2; ++up) {
        const int entry = kScaleBlock * bl + kFusedWaves * kScaleQuads * up + kScaleQuads * wave + (lane >> 4);
        const uint2 scale = sh.scales[buffer][entry];
        const uint2 residual = kGh5 ? sh.scales[buffer][kScaleBlock * kSpan + entry] : make_uint2(0u, 0u);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int sum = acc[up][r];
          const float dot = ldexpf(static_cast<float>(sum), shift);
          const uint32_t sw = r < 2 ? scale.x : scale.y;
          part[up][r] = fmaf(dot, half_at(sw, r & 1), bl == 0 ? 0.0f : part[up][r]);
          if (kGh5) {
            const uint32_t rw = r < 2 ? residual.x : residual.y;
            vpart[up][r] = fmaf(half_at(rw, r & 1), n2, bl == 0 ? 0.0f : vpart[up][r]);
          }
        }
      }
    }
#pragma unroll
    for (int up = 0; up < 2; ++up)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        est[up][r] = s == 0 ? part[up][r] : est[up][r] + part[up][r];
        if (kGh5) var[up][r] = s == 0 ? vpart[up][r] : var[up][r] + vpart[up][r];
      }
    if (s + 1 < live_splits) {
      stage_store((s + kStageAhead) % kStageBuffers, held, held_scale);
      __syncthreads();
    }
  }
  for (int s = live_splits; s < splits; ++s)
#pragma unroll
    for (int up = 0; up < 2; ++up)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        est[up][r] = est[up][r] + 0.0f;
        if (kGh5) var[up][r] = var[up][r] + 0.0f;
      }
  // ---- score epilogue: lane (pair pp, channels c .. c + 3)
  if (!working) return;
  if (a.tile_masks && lane < kRowTile)
    a.tile_masks[static_cast<long>(z) * a.I + kRowTile * ct + lane] = 0u;
  if (pp >= count) return;
  // (the score's inputs here: held across the splits they would cost a wave per SIMD)
  const int c = kRowTile * ct + row_in_tile;
  const ScoreInputs inputs = load_score_inputs(a, e, sh.pair_token[pp], sh.pair_slot[pp], c);
  score_four<kGh5>(a, sh.pair_token[pp], sh.pair_slot[pp], c, est[0], est[1], var[0], var[1],
                   inputs);
}

// ---------------------------------------------------------------------------
// select (progressive.py:1584-1775): the F best keys of score + 0 per token,
// ties to the lowest candidate id. Two 12-bit radix passes (and an 8-bit one
// when the cutoff's 24-bit bin holds more keys than remain) find the F-th
// largest key; a block scan compacts the kept ids in candidate order.

struct SelectArgs {
  const float *scores;
  const float *threshold;
  const int32_t *pair_tiles;  // tile slot 16 z + p of each pair, -1 if none
  uint32_t *tile_masks;       // [tile][channel] bit p: tile pair p kept it (or NULL)
  int32_t *next_ids;
  uint8_t *selected;
  uint8_t *completed;  // cleared here; the exact rows set their channels' flags
  int32_t *counts;
  int32_t *starts;
  int32_t *tile_starts;
  int32_t *down_tile_starts;
  int N, F, I, K;
  int thresholded;
};

constexpr int kSelectThreads = 1024;
constexpr int kSelectKeys = 16;  // keys per thread: N <= 16384
constexpr int kSelectExactTokens = 4;  // select and exact in one launch up to this batch

// Histogram slot of a radix bin: one pad word per 32 bins, so that lanes
// reading bins 32 apart use different LDS banks.
__device__ __forceinline__ int select_slot(int bin) { return bin + (bin >> 5); }

// Radix digits of the select passes: 12 and 12 bits, then the last 8 only
// when the cutoff's 24-bit bin holds more keys than remain to be kept (else
// every key of that bin is kept, whatever its low bits).
constexpr int kSelectWideBins = 4096;
constexpr int kSelectWideSlots = kSelectWideBins + kSelectWideBins / 32;
constexpr int kSelectLastBins = 256;
constexpr int kSelectLastSlots = kSelectLastBins + kSelectLastBins / 32;
constexpr int kSelectWaves = kSelectThreads / kWave;
constexpr int kSelectChunk = kSelectWideBins / kSelectWaves;  // bins per wave, 4 per lane

// A pass's cutoff bin as every wave finds it, within the 64 kPer-bin lane
// ranges below bin `top` (highest first): the first bin where `before` plus
// the keys counted from `top` down reaches `want`, which the range holds.
// Returns the bin; *above receives the keys in higher bins, *count the bin's.
template <int kPer>
__device__ __forceinline__ int select_scan(const int *histogram, int top, int want, int before,
                                           int *above, int *count) {
  const int lane = threadIdx.x & 63;
  const int lane_top = top - lane * kPer;
  int c[kPer], mine = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    c[i] = histogram[select_slot(lane_top - 1 - i)];
    mine += c[i];
  }
  const int inclusive = before + wave_inclusive(mine);
  const uint64_t reached = __ballot(inclusive >= want);
  const int owner = reached ? __builtin_ctzll(reached) : kWave - 1;
  int running = __builtin_amdgcn_readlane(inclusive - mine, owner);
  int bin = top - owner * kPer - kPer, at_above = running, at_count = 0;
  bool found = false;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int ci = __builtin_amdgcn_readlane(c[i], owner);
    if (!found && running + ci >= want) {
      found = true;
      bin = top - owner * kPer - 1 - i;
      at_above = running;
      at_count = ci;
    }
    running += ci;
  }
  *above = at_above;
  *count = at_count;
  return bin;
}

// The cutoff bin of a 4096-bin pass: wave w first sums its chunk of 256
// bins (the w-th from the top) into totals[w]; after the barrier every wave
// finds the chunk where the count reaches `want` from the 16 totals, then the
// bin inside it (select_scan). No wave waits for another's result.
__device__ __forceinline__ int select_wide(const int *histogram, int *totals, int want, int *above,
                                           int *count) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int chunk_top = kSelectWideBins - kSelectChunk * wave - 4 * lane;
  int sum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) sum += histogram[select_slot(chunk_top - 1 - i)];
  sum = wave_sum_all(sum);
  if (lane == 0) totals[wave] = sum;
  __syncthreads();
  const int mine = lane < kSelectWaves ? totals[lane] : 0;
  const int inclusive = wave_inclusive(mine);
  const uint64_t reached = __ballot(lane < kSelectWaves && inclusive >= want);
  const int owner = reached ? __builtin_ctzll(reached) : kSelectWaves - 1;
  const int before = __builtin_amdgcn_readlane(inclusive - mine, owner);
  return select_scan<4>(histogram, kSelectWideBins - kSelectChunk * owner, want, before, above,
                        count);
}

// The selection of token t by one workgroup of kSelectThreads threads (every
// thread calls it; `write` is the same for the whole workgroup). Leaves the
// thread's kept bits (bit j: candidate tid * per + j) in *kept_out and the
// kept count before the thread in *base_out. With `write` it also stores the
// outputs: kept ids, selected flags, completed flags (zeros, or with
// `completed_kept` the selected flags, which the exact rows of a launch that
// also runs them set anyway), slot records and tile mask bits.
template <int kKeys>  // keys per thread: N <= kKeys * kSelectThreads
__device__ __forceinline__ void select_token(const SelectArgs &a, int t, bool write, bool completed_kept,
                                             uint32_t *kept_out, int *base_out) {
  __shared__ int wide[2][kSelectWideSlots];
  __shared__ int last[kSelectLastSlots];
  __shared__ int scratch[32];
  __shared__ int totals[kSelectWaves];
  __shared__ int wave_totals[kSelectWaves];
  __shared__ int slot_start[65];
  __shared__ int slot_tiles[64];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  if (a.tile_masks && tid < a.K) slot_tiles[tid] = a.pair_tiles[t * a.K + tid];
  for (int i = tid; i < 2 * kSelectWideSlots; i += kSelectThreads) (&wide[0][0])[i] = 0;
  if (tid < kSelectLastSlots) last[tid] = 0;
  const int per = (a.N + kSelectThreads - 1) / kSelectThreads;
  const int first = tid * per;
  // keys: every load issued unconditionally (absent keys read a zero), four
  // or two at a time when the thread's run allows (N is a multiple of 16, so
  // a run of 4 or 2 keys is inside the row or wholly past it)
  uint32_t key[kKeys];
  const float *row = a.scores + static_cast<long>(t) * a.N;
  auto normal = [](uint32_t bits) { return __float_as_uint(__uint_as_float(bits) + 0.0f); };
  if (per % 4 == 0) {
#pragma unroll
    for (int j = 0; j < kKeys; j += 4) {
      const bool present = j < per && first + j < a.N;
      const uint4 v =
          load_global(present ? reinterpret_cast<const uint4 *>(row + first + j) : &kZeroVector);
      key[j] = normal(v.x);
      key[j + 1] = normal(v.y);
      key[j + 2] = normal(v.z);
      key[j + 3] = normal(v.w);
    }
  } else if (per % 2 == 0) {
#pragma unroll
    for (int j = 0; j < kKeys; j += 2) {
      const bool present = j < per && first + j < a.N;
      const uint2 v = load_global(present ? reinterpret_cast<const uint2 *>(row + first + j)
                                          : reinterpret_cast<const uint2 *>(&kZeroVector));
      key[j] = normal(v.x);
      key[j + 1] = normal(v.y);
    }
  } else {
#pragma unroll
    for (int j = 0; j < kKeys; ++j) {
      const bool present = j < per && first + j < a.N;
      const float *source =
          present ? row + first + j : reinterpret_cast<const float *>(&kZeroVector);
      key[j] = normal(__float_as_uint(load_global(source)));
    }
  }
  auto valid = [&](int j) { return j < per && first + j < a.N; };
  int want = a.F;
  if (a.thresholded) {
    const uint32_t bound = __float_as_uint(*a.threshold + 0.0f);
    int passing = 0;
#pragma unroll
    for (int j = 0; j < kKeys; ++j) passing += valid(j) && key[j] >= bound;
    passing = block_sum(passing, scratch);
    want = min(want, passing);
  } else {
    __syncthreads();  // the histograms are zero
  }
  // radix passes find the want-th largest key: `prefix` holds its known
  // bits, `mask` which bits those are
  uint32_t prefix = 0, mask = 0;
  if (want > 0) {
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int shift = pass == 0 ? 20 : 8;
#pragma unroll
      for (int j = 0; j < kKeys; ++j)
        if (valid(j) && (key[j] & mask) == prefix)
          atomicAdd(&wide[pass][select_slot((key[j] >> shift) & (kSelectWideBins - 1))], 1);
      __syncthreads();
      int above, count;
      const int bin = select_wide(wide[pass], totals, want, &above, &count);
      prefix |= static_cast<uint32_t>(bin) << shift;
      mask |= static_cast<uint32_t>(kSelectWideBins - 1) << shift;
      want -= above;
      if (pass == 1 && count > want) {
#pragma unroll
        for (int j = 0; j < kKeys; ++j)
          if (valid(j) && (key[j] & mask) == prefix)
            atomicAdd(&last[select_slot(key[j] & (kSelectLastBins - 1))], 1);
        __syncthreads();
        const int low = select_scan<kSelectLastBins / kWave>(last, kSelectLastBins, want, 0,
                                                              &above, &count);
        prefix |= static_cast<uint32_t>(low);
        mask = 0xffffffffu;
        want -= above;
      }
    }
  }
  const bool any = a.F > 0 && mask != 0;
  // After the passes `prefix` is the cutoff key on the bits of `mask` and
  // `want` the ties it keeps (all keys of the cutoff's bin when the last pass
  // was skipped). One scan of packed (above, tied) counts gives every thread
  // the kept keys before it: all keys above the cutoff, ties in ascending
  // candidate order.
  const uint32_t cutoff = prefix;
  const int room = want;
  // bit j of the thread's masks: candidate first + j is above / at the cutoff
  uint32_t above_bits = 0, tied_bits = 0;
#pragma unroll
  for (int j = 0; j < kKeys; ++j) {
    const uint32_t k = key[j] & mask;
    above_bits |= static_cast<uint32_t>(any && valid(j) && k > cutoff) << j;
    tied_bits |= static_cast<uint32_t>(any && valid(j) && k == cutoff) << j;
  }
  const int above_here = __builtin_popcount(above_bits), tied_here = __builtin_popcount(tied_bits);
  // exclusive prefix over threads (16-bit fields: at most N keys each), one
  // barrier: the wave totals have an array of their own
  const int packed_here = above_here | (tied_here << 16);
  const int inclusive = wave_inclusive(packed_here);
  if (lane == kWave - 1) wave_totals[wave] = inclusive;
  __syncthreads();
  int packed = inclusive - packed_here, packed_total = 0;
#pragma unroll
  for (int w = 0; w < kSelectWaves; ++w) {
    const int v = wave_totals[w];
    packed_total += v;
    packed += w < wave ? v : 0;
  }
  const int kept_total = (packed_total & 0xffff) + min(packed_total >> 16, room);
  const int above_before = packed & 0xffff, tied_before = packed >> 16;
  // the thread's kept keys: every key above the cutoff and its first ties
  // while the ties before them leave room; kept keys take consecutive
  // positions from `base`, the kept count before the thread
  const int tied_keep = max(0, min(room - tied_before, tied_here));
  uint32_t kept_tied = 0, rest = tied_bits;
  for (int n = 0; n < tied_keep; ++n) {
    kept_tied |= rest & (0u - rest);
    rest &= rest - 1;
  }
  const uint32_t kept_bits = above_bits | kept_tied;  // bit j: candidate first + j kept
  const int base = above_before + min(tied_before, room);
  *kept_out = kept_bits;
  *base_out = base;
  if (!write) return;
  auto kept_below = [&](int j) { return __builtin_popcount(kept_bits & ((1u << j) - 1u)); };
  // a slot's first candidate in the thread's run (at most one: I >= the run):
  // the kept ids before it start the slot
  const int slot0 = first / a.I, jb = (slot0 + 1) * a.I - first;
  if (first % a.I == 0 && valid(0)) slot_start[slot0] = any ? min(base, a.F) : 0;
  if (jb < per && first + jb < a.N) slot_start[slot0 + 1] = any ? min(base + kept_below(jb), a.F) : 0;
  for (uint32_t m = kept_bits; m; m &= m - 1) {
    const int j = __builtin_ctz(m);
    const int i = first + j, position = base + kept_below(j);
    if (position < a.F) {
      a.next_ids[static_cast<long>(t) * a.F + position] = i;
      // the channel's bit for this pair in its tile's mask (OR: any order)
      const int slot = j < jb ? slot0 : slot0 + 1;
      const int slot_tile = a.tile_masks ? slot_tiles[slot] : -1;
      if (slot_tile >= 0)
        atomicOr(&a.tile_masks[static_cast<long>(slot_tile / kGroupPairs) * a.I + (i - slot * a.I)],
                 1u << (slot_tile % kGroupPairs));
    }
  }
  // the run's selected flags (and completed flags: cleared, or the selected
  // ones) as one store per 4 or 2 candidates where the run allows
  {
    uint8_t *selected = a.selected + static_cast<long>(t) * a.N + first;
    uint8_t *completed = a.completed + static_cast<long>(t) * a.N + first;
    auto flag = [&](int j) { return (kept_bits >> j) & 1u; };
    if (per % 4 == 0) {
#pragma unroll
      for (int j = 0; j < kKeys; j += 4)
        if (j < per && first + j < a.N) {
          const uint32_t flags = flag(j) | flag(j + 1) << 8 | flag(j + 2) << 16 | flag(j + 3) << 24;
          *reinterpret_cast<uint32_t *>(selected + j) = flags;
          *reinterpret_cast<uint32_t *>(completed + j) = completed_kept ? flags : 0u;
        }
    } else if (per % 2 == 0) {
#pragma unroll
      for (int j = 0; j < kKeys; j += 2)
        if (j < per && first + j < a.N) {
          const uint16_t flags = static_cast<uint16_t>(flag(j) | flag(j + 1) << 8);
          *reinterpret_cast<uint16_t *>(selected + j) = flags;
          *reinterpret_cast<uint16_t *>(completed + j) = completed_kept ? flags : 0;
        }
    } else {
#pragma unroll
      for (int j = 0; j < kKeys; ++j)
        if (j < per && first + j < a.N) {
          selected[j] = static_cast<uint8_t>(flag(j));
          completed[j] = completed_kept ? static_cast<uint8_t>(flag(j)) : 0;
        }
    }
  }
  for (int p = kept_total + tid; p < a.F; p += kSelectThreads)
    a.next_ids[static_cast<long>(t) * a.F + p] = -1;
  if (tid == 0) slot_start[a.K] = min(kept_total, a.F);
  __syncthreads();
  // wave 0: lane k writes slot k's count, start and tile starts (K <= 64)
  if (tid < kWave) {
    const bool slot = tid < a.K;
    const int start = slot ? slot_start[tid] : 0;
    const int count = slot ? slot_start[tid + 1] - start : 0;
    const int tiles = (count + 127) / 128, tiles16 = (count + kDownTile - 1) / kDownTile;
    const int tile = wave_inclusive(tiles) - tiles, tile16 = wave_inclusive(tiles16) - tiles16;
    if (slot) {
      a.counts[t * a.K + tid] = count;
      a.starts[t * a.K + tid] = start;
      a.tile_starts[t * a.K + tid] = tile;
      a.down_tile_starts[t * a.K + tid] = tile16;
    }
  }
}

template <int kKeys>
__global__ __launch_bounds__(kSelectThreads) void select_kernel(SelectArgs a) {
  uint32_t kept;
  int base;
  select_token<kKeys>(a, blockIdx.x, true, false, &kept, &base);
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
      a.down_tile_starts[t * a.K + k] = k * ((a.I + kDownTile - 1) / kDownTile);
    }
  }
}

// ---------------------------------------------------------------------------
// encode (progressive.py:1859-1951): skipped channels of a 64-channel tile

struct EncodeArgs {
  const uint16_t *encoder_t;
  const uint16_t *encoder_tiles;  // [E, tiles, R, 64] (R = kDirectRank) or NULL
  const float *partial;
  const uint16_t *activations;
  const uint8_t *completed;
  const uint8_t *selected;
  const int32_t *ids;
  const uint8_t *padding;
  float *parts;
  int I, K, N, R, tiles, gelu, E;
};

constexpr int kEncodeStride = 72;  // LDS row stride (bf16) of a staged encoder row

// One (64-channel tile, slot, token) item on one wave; `coefficients` is the
// wave's own LDS slice of 64 rows of `stride` bf16. Every wave of the
// workgroup calls it (its barrier is the workgroup's); `store` is false for a
// wave whose item is past the work (it runs on a clamped item, stores nothing).
__device__ __forceinline__ void encode_tile(const EncodeArgs &a, int tile, int k, int t,
                                            bool store, uint16_t *coefficients, int stride) {
  const int lane = threadIdx.x & 63;
  const int c = tile * 64 + lane;
  const int e = a.ids[t * a.K + k];
  const bool local = is_active(a.padding, t) && e >= 0;
  // every load issued unconditionally (clamped channel, zero row source)
  const int cc = min(c, a.I - 1);
  const long flat = static_cast<long>(t) * a.N + static_cast<long>(k) * a.I + cc;
  const long base = static_cast<long>(t) * 2 * a.N + static_cast<long>(k) * a.I + cc;
  const uint8_t is_selected = load_global(a.selected + flat);
  const uint8_t is_completed = load_global(a.completed + flat);
  const uint16_t exact = load_global(a.activations + flat);
  const float gate = load_global(a.partial + base);
  const float up = load_global(a.partial + base + a.N);
  const bool rows16 = (a.R & 7) == 0;
  uint4 coefficient_rows[kMaxRank / 8];
  const uint16_t *row = a.encoder_t + (static_cast<long>(local ? e : 0) * a.I + cc) * a.R;
  if (rows16) {
#pragma unroll
    for (int q = 0; q < kMaxRank / 8; ++q) {
      const uint4 *source = (local && 8 * q < a.R) ? reinterpret_cast<const uint4 *>(row + 8 * q)
                                                   : &kZeroVector;
      coefficient_rows[q] = load_global(source);
    }
  }
  const int skip = c < a.I && !is_selected;
  float v = 0.0f;
  if (skip)
    v = is_completed ? bf16f(exact) : bfr(cfm_activate(bfr(gate), a.gelu != 0) * bfr(up));
  uint16_t *staged = &coefficients[lane * stride];
  if (rows16) {
#pragma unroll
    for (int q = 0; q < kMaxRank / 8; ++q)
      if (8 * q < a.R) *reinterpret_cast<uint4 *>(staged + 8 * q) = coefficient_rows[q];
  } else if (skip && local) {
    for (int q = 0; q < a.R; ++q) staged[q] = row[q];
  }
  const uint64_t skipped = __ballot(skip);
  __syncthreads();
  // lane r < R: chain over the tile's skipped channels in order; a kept
  // channel leaves the sum untouched (a select, not an added zero), so the
  // loop has no branch and its LDS reads issue together (lanes >= R read
  // in-bounds staged columns and store nothing)
  float acc = 0.0f;
  const int column = min(lane, stride - 1);
#pragma unroll
  for (int j = 0; j < 64; ++j) {
    const float value = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
    const float coefficient = local ? bf16f(coefficients[j * stride + column]) : 0.0f;
    const float next = fmaf(value, coefficient, acc);
    acc = (skipped >> j) & 1ull ? next : acc;
  }
  if (store && lane < a.R)
    a.parts[((static_cast<long>(t) * a.K + k) * a.tiles + tile) * a.R + lane] = acc;
}

__global__ __launch_bounds__(64) void encode_kernel(EncodeArgs a) {
  __shared__ __align__(16) uint16_t coefficients[64 * kEncodeStride];
  encode_tile(a, blockIdx.x, blockIdx.y, blockIdx.z, true, coefficients, kEncodeStride);
}

// Two (64-channel tile, slot, token) items on one wave at R = kDirectRank:
// item q = tile + tiles (k + K t) of the flat item order, the wave's pair
// 2 p and 2 p + 1 (the second may be past `items`: its half stores nothing).
// Lane 32 h + r takes rank r of item 2 p + h and runs its whole chain over
// the tile's 64 channels in order. Lanes 32 h + j and 32 h + 32 + j first
// form item h's values of channels j and 32 + j (zero for a kept channel, a
// channel past I or a slot with no local expert: fma(0, b, acc) == acc
// exactly for finite b, since the chain starts at +0 and never holds -0, so
// a zero value leaves the chain as skipping it would) and put them in LDS,
// from where every step reads four values of its half's item at once
// (broadcast reads). The coefficients E[c][r] arrive packed two to a word.
// Same order and roundings as encode_tile.
//
// The selected and completed flags come from the workspace (one-wave
// workgroups, whose LDS values array is the function's own), or, in a
// workgroup of several waves that ran the token's selection itself
// (KeptBits), the selected flags from that selection's kept bits and no
// completed flag (a skipped channel is never completed), the values through
// the wave's own LDS rows `staged`.
constexpr int kDirectRank = 32;

struct WorkspaceFlags {};
struct KeptBits {
  const uint32_t *bits;  // thread j's kept bits: bit i is candidate j per + i of the token
  int per;
};

template <class Args, class Flags = WorkspaceFlags>  // Args: EncodeArgs or the grouped exact launch's
__device__ __forceinline__ void encode_pair_direct(const Args &a, int p, int items, int t_base,
                                                   Flags flags = Flags(), float (*staged)[64] = nullptr) {
  constexpr int R = kDirectRank;
  constexpr bool kFromBits = std::is_same<Flags, KeptBits>::value;
  __shared__ __align__(16) float own_values[kFromBits ? 1 : 2][64];
  float (*channel_values)[64] = kFromBits ? staged : own_values;
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, r = lane & 31;
  const int q = min(2 * p + h, items - 1);
  const bool store = 2 * p + h < items;
  const int tile = q % a.tiles, rest = q / a.tiles;
  const int k = rest % a.K, t = t_base + rest / a.K;
  // the item's expert (lanes of a half agree); the flag and value loads
  // below do not wait for it
  const int e = load_global(a.ids + t * a.K + k);
  const bool active = is_active(a.padding, t);
  // the item's flags and values of channels r and 32 + r
  const long flat = static_cast<long>(t) * a.N + static_cast<long>(k) * a.I + tile * 64;
  const long base = static_cast<long>(t) * 2 * a.N + static_cast<long>(k) * a.I + tile * 64;
  uint8_t is_selected[2], is_completed[2];
  uint16_t exact[2];
  float gate[2], up[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int j = 32 * s + r;
    const bool inside = tile * 64 + j < a.I;
    const long at = inside ? j : 0;
    if constexpr (kFromBits) {
      const int i = k * a.I + tile * 64 + static_cast<int>(at);
      is_selected[s] = inside ? (flags.bits[i / flags.per] >> (i % flags.per)) & 1u : 1;
      is_completed[s] = 0;
    } else {
      is_selected[s] = inside ? a.selected[flat + at] : 1;
      is_completed[s] = a.completed[flat + at];
    }
    exact[s] = a.activations[flat + at];
    gate[s] = a.partial[base + at];
    up[s] = a.partial[base + a.N + at];
  }
  const bool local = active && e >= 0;
  // coefficients E[tile 64 + c][r], c < 64: rank r's contiguous 128-byte row
  // of the tile-major copy, two channels to a word (channels past I are zero;
  // an absent slot reads expert 0's, which meet only zero values)
  const __amdgpu_buffer_rsrc_t coefficients = buffer_resource(
      a.encoder_tiles, static_cast<int>(static_cast<long>(a.E) * a.tiles * R * 64 * 2));
  const int row = ((max(e, 0) * a.tiles + tile) * R + r) * 128;
  uint32_t coefficient[32];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const uint4 w = buffer_load16(coefficients, row + 16 * m);
    coefficient[4 * m] = w.x;
    coefficient[4 * m + 1] = w.y;
    coefficient[4 * m + 2] = w.z;
    coefficient[4 * m + 3] = w.w;
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const bool skip = local && !is_selected[s];
    float value = 0.0f;
    if (skip)
      value = is_completed[s] ? bf16f(exact[s]) : bfr(cfm_activate(bfr(gate[s]), a.gelu != 0) * bfr(up[s]));
    channel_values[h][32 * s + r] = value;
  }
  if constexpr (kFromBits) {
    // the wave's own rows: its LDS writes before its reads (in order within
    // a wave; the fences keep the compiler from moving them)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  } else {
    __syncthreads();  // one-wave workgroups: orders the LDS writes before the reads
  }
  const float4 *values = reinterpret_cast<const float4 *>(channel_values[h]);
  float acc = 0.0f;
#pragma unroll
  for (int g = 0; g < 16; ++g) {
    const float4 v = values[g];
    acc = fmaf(v.x, __uint_as_float(coefficient[2 * g] << 16), acc);
    acc = fmaf(v.y, __uint_as_float(coefficient[2 * g] & 0xffff0000u), acc);
    acc = fmaf(v.z, __uint_as_float(coefficient[2 * g + 1] << 16), acc);
    acc = fmaf(v.w, __uint_as_float(coefficient[2 * g + 1] & 0xffff0000u), acc);
  }
  if (store) a.parts[(static_cast<long>(t_base) * a.K * a.tiles + q) * R + r] = acc;
}

// Grouped exact rows (batches of grouped_tokens or more, as
// progressive.py:2655-2718): wave = (16-pair expert tile, kExactChannels
// channels). The select kernel's tile masks name the tile's pairs that kept
// each channel; they and the tile's pairs (16 slots per tile) are read
// together. For each channel some pair kept, in turn, its gate and up rows
// are read once and dotted with each such pair's hidden row in the lane
// order of row_dots (identical results).
// Workgroups past the tiles (one per token) write the zero results of padded
// tokens and non-local slots, which the grouping leaves out.
struct GroupExactArgs {
  const uint16_t *gate_up;
  const uint16_t *x;
  const uint8_t *padding;
  const int32_t *ids;
  const int32_t *next_ids;
  const int32_t *counts;
  const int32_t *starts;
  const uint8_t *selected;
  const int32_t *group_experts;
  const int32_t *group_starts;
  const int32_t *group_counts;
  const int32_t *group_pairs;
  const int32_t *group_total;
  const uint32_t *tile_masks;
  float *partial;
  uint16_t *activations;
  uint8_t *completed;
  int H, I, K, N, F, T, gelu, channel_groups, tile_items;
  int dense;  // every channel kept by every pair (no tile masks)
  // recovery encoder items (R = kDirectRank) run past the exact tiles
  const uint16_t *encoder_t;
  const uint16_t *encoder_tiles;
  float *parts;  // encoder partials
  int tiles, encode_items, E;
  // the down kernel's workgroup order, built by the first kDownBuilders
  // workgroups (or NULL): list of down_blocks items, then per-builder slot
  // records (two words each) from word order_words, slot_capacity per builder
  int32_t *down_order;
  const int32_t *pair_tiles;
  const int32_t *down_tile_starts;
  int max_tiles, down_blocks, order_words, slot_capacity;
  // union-row accounting (or NULL): kUnionCounters workgroups after the
  // builders add union_row_bytes to slot 12 per nonzero tile mask word
  double *read_work;
  double union_row_bytes;
};

constexpr int kMaxHidden = 4096;
constexpr int kDownBuilders = 8;     // one per XCD
constexpr int kUnionCounters = 64;  // workgroups counting the tile masks' nonzero words
// 16-byte parts per lane of a hidden-size row: 4 up to H = 2048 (the common
// shapes, 72 VGPRs in the grouped kernel), 8 up to kMaxHidden
constexpr int kNarrowParts = 4;
constexpr int kWideParts = kMaxHidden / 512;
__host__ __device__ inline int hidden_parts(int H) { return H <= 512 * kNarrowParts ? kNarrowParts : kWideParts; }

// Lane-ordered gate and up dots with a hidden row, each row held as kParts
// 16-byte parts per lane (part j of lane l: h = 512 j + 8 l + i, i < 8): the
// lane's partial sums in h order; parts past H leave them untouched. Every
// exact row of the reader is this chain, then wave_sum_lane0.
template <int kParts>
__device__ __forceinline__ void row_dots(const uint4 (&gw)[kParts], const uint4 (&uw)[kParts],
                                         const uint4 (&xw)[kParts], int H, int lane,
                                         float &g, float &u) {
#pragma unroll
  for (int j = 0; j < kParts; ++j) {
    const bool inside = 512 * j + 8 * lane < H;
    const uint32_t gv[4] = {gw[j].x, gw[j].y, gw[j].z, gw[j].w};
    const uint32_t uv[4] = {uw[j].x, uw[j].y, uw[j].z, uw[j].w};
    const uint32_t xv[4] = {xw[j].x, xw[j].y, xw[j].z, xw[j].w};
    float gj = g, uj = u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x0 = __uint_as_float(xv[i] << 16), x1 = __uint_as_float(xv[i] & 0xffff0000u);
      gj = fmaf(__uint_as_float(gv[i] << 16), x0, gj);
      gj = fmaf(__uint_as_float(gv[i] & 0xffff0000u), x1, gj);
      uj = fmaf(__uint_as_float(uv[i] << 16), x0, uj);
      uj = fmaf(__uint_as_float(uv[i] & 0xffff0000u), x1, uj);
    }
    g = inside ? gj : g;
    u = inside ? uj : u;
  }
}

// Builder x of the down kernel's workgroup order. Workgroup b of the down
// launch runs on XCD b % 8, in the order b / 8 there; entry 8 r + x of the
// list gives XCD x the r-th item of its run, and the runs split the items,
// in expert order (the routing's tiles of pairs, each pair's tiles in turn,
// then the pairs outside the tiles), into eight contiguous parts: a tile's
// pairs then read their expert's down rows close together on one XCD, whose
// L2 serves the rows they share. Entries past a run hold -1. Every builder
// derives the whole order from the workspace (no communication between
// workgroups); loads are issued four chunks at a time.
__device__ void build_down_order(const GroupExactArgs &a, int x) {
  const int lane = threadIdx.x & 63;
  const int pairs = a.T * a.K;
  const int slots = kGroupPairs * load_global(a.group_total);
  uint2 *records = reinterpret_cast<uint2 *>(a.down_order + a.order_words) +
                   static_cast<long>(x) * a.slot_capacity;
  // every pair's tile count; grouped pairs leave (tiles, first item) at their slot
  int total = 0;
  for (int i0 = 0; i0 < pairs; i0 += 4 * kWave) {
    int slot[4], count[4], first[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = min(i0 + kWave * u + lane, pairs - 1);
      slot[u] = load_global(a.pair_tiles + i);
      count[u] = load_global(a.counts + i);
      first[u] = load_global(a.down_tile_starts + i);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + kWave * u + lane;
      if (i >= pairs) continue;
      const int tiles = (count[u] + kDownTile - 1) / kDownTile;
      total += tiles;
      if (slot[u] >= 0)
        records[slot[u]] = make_uint2(tiles, static_cast<uint32_t>((i / a.K) * a.max_tiles + first[u]));
    }
  }
  total = wave_sum_all(total);
  __syncthreads();  // the slot records are visible to every lane
  const int run = (total + 7) / 8, lo = x * run, hi = min(total, lo + run);
  int placed = 0;
  // the lane's n items item0 + j follow the lower lanes' and those placed
  auto place = [&](int n, int item0) {
    const int inclusive = wave_inclusive(n);
    int m = placed + inclusive - n;
    for (int j = 0; j < n; ++j, ++m)
      if (m >= lo && m < hi) a.down_order[8 * (m - lo) + x] = item0 + j;
    placed += __builtin_amdgcn_readlane(inclusive, 63);
  };
  for (int s0 = 0; s0 < slots; s0 += 4 * kWave) {
    uint2 record[4];
    int members[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int s = min(s0 + kWave * u + lane, slots - 1);
      record[u] = load_global(records + s);
      members[u] = load_global(a.group_counts + s / kGroupPairs);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int s = s0 + kWave * u + lane;
      const bool valid = s < slots && s % kGroupPairs < members[u];
      place(valid ? static_cast<int>(record[u].x) : 0, static_cast<int>(record[u].y));
    }
  }
  for (int i0 = 0; i0 < pairs; i0 += 4 * kWave) {
    int slot[4], count[4], first[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = min(i0 + kWave * u + lane, pairs - 1);
      slot[u] = load_global(a.pair_tiles + i);
      count[u] = load_global(a.counts + i);
      first[u] = load_global(a.down_tile_starts + i);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + kWave * u + lane;
      const bool outside = i < pairs && slot[u] < 0;
      place(outside ? (count[u] + kDownTile - 1) / kDownTile : 0,
            (min(i, pairs - 1) / a.K) * a.max_tiles + first[u]);
    }
  }
  // the rest of this XCD's run is empty
  for (int r = max(hi - lo, 0) + lane; r < a.down_blocks / 8; r += kWave) a.down_order[8 * r + x] = -1;
}

// Counter x of the union rows: the nonzero (tile, channel) mask words of
// the routing's tiles, four loads per lane in flight, one FP64 add per
// workgroup. Each word is counted once, whichever pairs set it.
__device__ void count_union_rows(const GroupExactArgs &a, int x) {
  const int lane = threadIdx.x & 63;
  const long words = static_cast<long>(load_global(a.group_total)) * a.I;
  int rows = 0;
  for (long w0 = static_cast<long>(x) * 4 * kWave; w0 < words;
       w0 += static_cast<long>(kUnionCounters) * 4 * kWave) {
    uint32_t m[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long w = w0 + u * kWave + lane;
      m[u] = load_global(a.tile_masks + min(w, words - 1));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) rows += w0 + u * kWave + lane < words && m[u] != 0u;
  }
  rows = wave_sum_all(rows);
  if (lane == 0 && rows > 0) atomicAdd(a.read_work + 12, rows * a.union_row_bytes);
}

__device__ __forceinline__ void exact_results(const GroupExactArgs &a, int t, int logical,
                                              float g, float u) {
  const long address = static_cast<long>(t) * 2 * a.N + logical;
  a.partial[address] = g;
  a.partial[address + a.N] = u;
  const float act = bfr(cfm_activate(bfr(g), a.gelu != 0));
  a.activations[static_cast<long>(t) * a.N + logical] = f2bf(act * bfr(u));
  a.completed[static_cast<long>(t) * a.N + logical] = 1;
}

// Waves per workgroup. One: a workgroup's waves are placed one per SIMD, so
// a workgroup of several waves, whose lifetimes differ (channels that no pair
// kept end at once), can start only when every SIMD of a CU has a free slot.
constexpr int kGroupExactWaves = 1;
constexpr int kExactChannels = 2;  // channels of one tile per grouped exact wave, in turn

// The grouped exact launch's workgroups that are not (tile, channel) work:
// the first kDownBuilders build the down order, those past the routing's
// tile items run recovery encoder items, then one per token writes the zero
// results of a padded token or of slots with no local expert, and the rest
// (the grid's tile items past the tile count) have nothing to do. Returns
// the tile item index of a work workgroup, or -1 when its part is done.
__device__ __forceinline__ int group_exact_side_items(const GroupExactArgs &a, int threads) {
  int block = blockIdx.x;
  if (a.down_order) {
    if (block < kDownBuilders) {
      build_down_order(a, block);
      return -1;
    }
    block -= kDownBuilders;
  }
  if (a.read_work) {
    if (block < kUnionCounters) {
      count_union_rows(a, block);
      return -1;
    }
    block -= kUnionCounters;
  }
  // the items of the routing's tiles come first, then the encoder and token
  // items, then the tile items past the tile count (nothing to do): the
  // encoder items are not dispatched behind the empty ones
  const int live_items = min(load_uniform(a.group_total) * a.channel_groups, a.tile_items);
  if (block < live_items) return block;
  const int item = block - live_items;
  const int encode_blocks = (a.encode_items + 1) / 2;
  if (item < encode_blocks) {
    // two recovery encoder items (tile, slot, token), tile fastest; they read
    // no exact result (a skipped channel is never completed)
    encode_pair_direct(a, item, a.encode_items, 0);
    return -1;
  }
  const int t = item - encode_blocks;
  if (t >= a.T) return -1;  // (and the tile items past the tile count)
  const bool active = is_active(a.padding, t);
  for (int k = 0; k < a.K; ++k) {
    if (active && a.ids[t * a.K + k] >= 0) continue;
    const int start = a.starts[t * a.K + k], count = a.counts[t * a.K + k];
    for (int j = static_cast<int>(threadIdx.x); j < count && start + j < a.F; j += threads) {
      const int logical = a.next_ids[static_cast<long>(t) * a.F + start + j];
      if (logical >= 0 && logical < a.N) exact_results(a, t, logical, 0.0f, 0.0f);
    }
  }
  return -1;
}

template <int kParts>
__global__ __launch_bounds__(64 * kGroupExactWaves) __attribute__((amdgpu_waves_per_eu(kParts == kNarrowParts ? 7 : 4))) void
group_exact_kernel(GroupExactArgs a) {
  const int lane = threadIdx.x & 63;
  const int block = group_exact_side_items(a, 64 * kGroupExactWaves);
  if (block < 0) return;
  const int z = block / a.channel_groups;
  const int c0 = (block % a.channel_groups) * kExactChannels;
  // An expert's tiles are consecutive. An even tile whose successor has the
  // same expert takes both tiles' pairs (32 pair slots, contiguous), so the
  // expert's rows are read once per two tiles; the odd tile's item then has
  // nothing to do. The tile count, both tiles' experts, pair counts and pair
  // slots through the scalar cache, and lane l < 4 the mask of channel
  // c0 + l % 2 in tile z + l / 2, in one round trip: z + 1 < tile bound <=
  // T * K keeps every address in bounds whatever the tile count, and only
  // slots named by mask bits (< count) are used.
  const int bound = a.tile_items / a.channel_groups;
  const int next_z = min(z + 1, bound - 1);
  const int total = load_uniform(a.group_total);
  const int e = load_uniform(a.group_experts + z);
  const int count = load_uniform(a.group_counts + z);
  const int next_count = load_uniform(a.group_counts + next_z);
  const i32x16 slots = load_uniform(reinterpret_cast<const i32x16 *>(a.group_pairs + kGroupPairs * z));
  const i32x16 next_slots =
      load_uniform(reinterpret_cast<const i32x16 *>(a.group_pairs + kGroupPairs * next_z));
  const int lane_channel = c0 + (lane & (kExactChannels - 1));
  const int lane_tile = lane < kExactChannels ? z : next_z;
  const bool lane_in = lane < 2 * kExactChannels && lane_channel < a.I;
  const uint32_t mask_word =
      lane_in ? load_global(a.tile_masks + static_cast<long>(lane_tile) * a.I + lane_channel) : 0u;
  // the neighbouring tiles' experts: an expert split into several tiles has
  // its rows read by each of them (entries past the count are never used)
  const int before = load_uniform(a.group_experts + max(z - 1, 0));
  const int after = load_uniform(a.group_experts + next_z);
  // all issued before any is tested (else each waits under its branch)
  asm volatile("" ::"s"(total), "s"(e), "s"(count), "s"(next_count), "s"(slots), "s"(next_slots),
               "s"(before), "s"(after));
  if (z >= total) return;
  if ((z & 1) && before == e) return;  // the previous (even) tile's item holds this tile
  const bool with_next = !(z & 1) && z + 1 < total && after == e;
  const bool shared_rows = (z > 0 && before == e) || (z + 1 < total && after == e);
  // lane p < 32: pair p of the two tiles (p >= 16: the next tile's p - 16)
  int pair = slots[0];
#pragma unroll
  for (int p = 1; p < kGroupPairs; ++p) pair = (lane & (kGroupPairs - 1)) == p ? slots[p] : pair;
  int next_pair = next_slots[0];
#pragma unroll
  for (int p = 1; p < kGroupPairs; ++p) next_pair = (lane & (kGroupPairs - 1)) == p ? next_slots[p] : next_pair;
  pair = (lane & kGroupPairs) ? next_pair : pair;
  const int token = pair / a.K, pair_slot = pair % a.K;
  // counts <= 16; lane l < kExactChannels: channel c0 + l's mask over both tiles
  const uint32_t next_word = static_cast<uint32_t>(__shfl(static_cast<int>(mask_word), lane + kExactChannels));
  const uint32_t own = a.dense ? (1u << count) - 1u : mask_word;
  const uint32_t next_own = a.dense ? (1u << next_count) - 1u : next_word;
  const bool lane_own = lane < kExactChannels && lane_channel < a.I;
  const uint32_t lane_mask = !lane_own ? 0u : own | (with_next ? next_own << kGroupPairs : 0u);
  // the wave's channels that some pair kept, in order
  for (uint64_t kept = __ballot(lane_mask != 0u); kept; kept &= kept - 1) {
    const int at = __builtin_ctzll(kept);
    const int c = c0 + at;
    const uint32_t mask = __builtin_amdgcn_readlane(lane_mask, at);
    const int logical = pair_slot * a.I + c;
    // rows and hidden rows through buffer resources: lane offset 16 lane, part j
    // at 1024 j bytes; parts past H read zeros and their chains are discarded
    const int row_bytes = 2 * a.H, offset = 16 * lane;
    const long grow = (static_cast<long>(e) * 2 * a.I + c) * a.H;
    const __amdgpu_buffer_rsrc_t gate_rows = buffer_resource(a.gate_up + grow, row_bytes);
    const __amdgpu_buffer_rsrc_t up_rows =
        buffer_resource(a.gate_up + grow + static_cast<long>(a.I) * a.H, row_bytes);
    uint4 xw[kParts];
    auto load_hidden = [&](int pp) {
      const int t = __builtin_amdgcn_readlane(token, pp);
      const __amdgpu_buffer_rsrc_t hidden =
          buffer_resource(a.x + static_cast<long>(t) * a.H, row_bytes);
#pragma unroll
      for (int j = 0; j < kParts; ++j) xw[j] = buffer_load16(hidden, offset + 1024 * j);
    };
    // the first keeping pair's hidden row travels with the gate/up rows
    load_hidden(__builtin_ctz(mask));
    // rows read once stream past the caches; rows the expert's other tiles read
    // again stay cached for them
    uint4 gw[kParts], uw[kParts];
    if (shared_rows) {
#pragma unroll
      for (int j = 0; j < kParts; ++j) {
        gw[j] = buffer_load16(gate_rows, offset + 1024 * j);
        uw[j] = buffer_load16(up_rows, offset + 1024 * j);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kParts; ++j) {
        gw[j] = buffer_stream16(gate_rows, offset + 1024 * j);
        uw[j] = buffer_stream16(up_rows, offset + 1024 * j);
      }
    }
    // lane p holds pair p's sums; the results are stored after the loop (a
    // store inside it would delay the next pair's loads, which wait in order)
    float kept_g = 0.0f, kept_u = 0.0f;
    for (uint32_t rest = mask; rest; rest &= rest - 1) {
      const int pp = __builtin_ctz(rest);
      if (rest != mask) load_hidden(pp);
      float g = 0.0f, uu = 0.0f;
      // keep the rows packed across pairs (unpacking them once ahead of the
      // loop would hold 64 more registers and halve the waves per SIMD)
#pragma unroll
      for (int j = 0; j < kParts; ++j)
        asm volatile("" : "+v"(gw[j].x), "+v"(gw[j].y), "+v"(gw[j].z), "+v"(gw[j].w),
                     "+v"(uw[j].x), "+v"(uw[j].y), "+v"(uw[j].z), "+v"(uw[j].w));
      row_dots(gw, uw, xw, a.H, lane, g, uu);
      g = wave_sum_lane0(g);
      uu = wave_sum_lane0(uu);
      kept_g = lane == pp ? g : kept_g;
      kept_u = lane == pp ? uu : kept_u;
    }
    if (lane < 2 * kGroupPairs && ((mask >> lane) & 1u)) exact_results(a, token, logical, kept_g, kept_u);
  }
}

// ---------------------------------------------------------------------------
// down (progressive.py:1778-1856): 32-channel tiles of a slot's kept channels

struct DownArgs {
  const uint16_t *down;
  const uint16_t *activations;
  const int32_t *ids;
  const uint8_t *padding;
  const int32_t *next_ids;
  const int32_t *counts;
  const int32_t *starts;
  const int32_t *down_tile_starts;
  const int32_t *order;  // workgroup b's item t * max_tiles + tile (-1: none), or NULL
  float *parts;
  int H, I, K, N, F, max_tiles;
  const void *padding_source;  // the padding mask and T bytes, or any pointer and 0 bytes
  int padding_bytes;
};

constexpr int kDownOutputs = 8;  // outputs per down thread (H / 8 threads)

// The slot of a token's down tile: the slot whose tiles hold it, the tile's
// first position in the slot's kept list, and the slot's count, expert and
// start in next_ids (k = -1: the tile is past the token's tiles).
struct DownTile {
  int k, first, count, e, start;
};

// At K = 8 the token's four records arrive through the scalar cache in one
// round trip.
__device__ __forceinline__ DownTile down_tile_slot(const int32_t *counts, const int32_t *tile_starts,
                                                   const int32_t *ids, const int32_t *starts,
                                                   int K, int t, int tile) {
  DownTile d = {-1, 0, 0, -1, 0};
  if (K == 8) {
    const long row = static_cast<long>(t) * 8;
    const i32x8 c8 = load_uniform(reinterpret_cast<const i32x8 *>(counts + row));
    const i32x8 t8 = load_uniform(reinterpret_cast<const i32x8 *>(tile_starts + row));
    const i32x8 e8 = load_uniform(reinterpret_cast<const i32x8 *>(ids + row));
    const i32x8 s8 = load_uniform(reinterpret_cast<const i32x8 *>(starts + row));
    asm volatile("" ::"s"(c8), "s"(t8), "s"(e8), "s"(s8));
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (tile >= t8[s] && tile < t8[s] + (c8[s] + kDownTile - 1) / kDownTile) {
        d.k = s;
        d.first = (tile - t8[s]) * kDownTile;
        d.count = c8[s];
        d.e = e8[s];
        d.start = s8[s];
      }
    }
  } else {
    for (int s = 0; s < K; ++s) {
      const int c = counts[t * K + s];
      const int ts = tile_starts[t * K + s];
      if (tile >= ts && tile < ts + (c + kDownTile - 1) / kDownTile) {
        d.k = s;
        d.first = (tile - ts) * kDownTile;
        d.count = c;
      }
    }
    if (d.k >= 0) {
      d.e = ids[t * K + d.k];
      d.start = starts[t * K + d.k];
    }
  }
  return d;
}

// Workgroup per (32-channel tile, token) with H / 8 threads of eight outputs
// each (grouped batches), or per (tile, token, 512 outputs) with one wave
// (smaller batches: more CUs share a batch-1 call). Every wave works alone (no LDS, no barrier): the token's slot records
// (counts, tile starts, ids, starts) come through the scalar cache in one
// round trip, lanes l < 32 of the wave load the tile's channel id l (the tile
// stops at the count or at the first invalid id, found by a ballot), the ids
// are broadcast by lane reads and every thread issues the tile's 32 row loads
// together, then the 32 activations (one per lane, broadcast the same way).
__global__ __launch_bounds__(512) void down_kernel(DownArgs a) {
  asm volatile("" ::"s"(a.parts), "s"(a.down), "s"(a.activations), "s"(a.next_ids), "s"(a.padding_source),
               "s"(a.padding_bytes), "s"(a.max_tiles), "s"(a.H), "s"(a.I), "s"(a.N), "s"(a.F));
  int tile = blockIdx.x, t = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  if (a.order) {
    const int item = load_uniform(a.order + blockIdx.x);
    if (item < 0) return;
    tile = item % a.max_tiles;
    t = item / a.max_tiles;
  }
  const DownTile d = down_tile_slot(a.counts, a.down_tile_starts, a.ids, a.starts, a.K, t, tile);
  const int k = d.k, first = d.first, count = d.count, e = d.e, start = d.start;
  if (k < 0 || tile >= a.max_tiles) return;
  // the tile's channel ids and the token's padding flag in one round trip
  const int j = first + (lane & (kDownTile - 1));
  const int logical = load_global(a.next_ids + static_cast<long>(t) * a.F + min(start + j, a.F - 1));
  const uint32_t padded =
      __builtin_amdgcn_raw_buffer_load_b8(buffer_resource(a.padding_source, a.padding_bytes), t, 0, 0);
  asm volatile("" ::"v"(logical), "v"(padded));
  const bool local = __builtin_amdgcn_readfirstlane(padded) == 0 && e >= 0;
  const bool valid = j < count && start + j < a.F && logical >= 0 && logical < a.N;
  // the tile's valid ids: the prefix before the first invalid one
  const uint32_t invalid = static_cast<uint32_t>(__ballot(!valid));
  const uint32_t live = invalid ? (1u << __builtin_ctz(invalid)) - 1u : 0xffffffffu;
  const int channel = valid ? logical % a.I : 0;
  // z: 512-output chunk of the per-token launch's one-wave workgroups (the
  // grouped launch has one chunk)
  const int o = (blockIdx.z * kWave + tid) * kDownOutputs;
  const bool outputs = o < a.H;
  // the expert's rows through one buffer resource (none without a local
  // expert: every row then reads zeros), row c at scalar offset 2 H c; rows
  // past the live prefix read channel 0's row, which the chain never uses
  const __amdgpu_buffer_rsrc_t rows =
      buffer_resource(a.down + (local ? static_cast<long>(e) * a.I * a.H : 0), local ? 2 * a.I * a.H : 0);
  const int column = 2 * min(o, a.H - kDownOutputs);
  uint4 w[kDownTile];
#pragma unroll
  for (int jj = 0; jj < kDownTile; ++jj) {
    const int c = __builtin_amdgcn_readlane(channel, jj);
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rows, column, 2 * a.H * c, 0);
    w[jj] = make_uint4(v.x, v.y, v.z, v.w);
  }
  const bool mine = (live >> (lane & (kDownTile - 1))) & 1u;
  const uint16_t act_bits =
      load_global(mine ? a.activations + static_cast<long>(t) * a.N + logical
                       : reinterpret_cast<const uint16_t *>(&kZeroVector));
  // (every row load is issued before the first is used)
  asm volatile("" ::: "memory");
  const int act_lane = static_cast<int>(__float_as_uint(bf16f(act_bits)));
  // (every lane stays active through the chain: its lane reads fetch
  // activations from lanes whose outputs may lie past H)
  float acc[kDownOutputs];
#pragma unroll
  for (int i = 0; i < kDownOutputs; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int jj = 0; jj < kDownTile; ++jj) {
    if (!((live >> jj) & 1u)) break;
    const float act = __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(act_lane, jj)));
    const uint32_t wv[4] = {w[jj].x, w[jj].y, w[jj].z, w[jj].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = fmaf(__uint_as_float(wv[i] << 16), act, acc[2 * i]);
      acc[2 * i + 1] = fmaf(__uint_as_float(wv[i] & 0xffff0000u), act, acc[2 * i + 1]);
    }
  }
  if (!outputs) return;
  float *out = a.parts + (static_cast<long>(t) * a.max_tiles + tile) * a.H + o;
  *reinterpret_cast<float4 *>(out) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  *reinterpret_cast<float4 *>(out + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
}

// ---------------------------------------------------------------------------
// exact below the grouped size (progressive.py:1510-1546): one wave per kept
// channel

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
  // recovery encoder items (R = kDirectRank) of the token, one per workgroup
  // past exact_blocks (0: none); encode reads no exact result (a skipped
  // channel is never completed)
  EncodeArgs encode;
  int exact_blocks, encode_items;
  const void *padding_source;  // the padding mask and T bytes, or any pointer and 0 bytes
  int padding_bytes;
};

// Kept channel `logical` of token t on one wave (lane k < K holds slot k's
// expert in slot_id, `padded` the token's padding flag): the gate, up and
// hidden rows with every part in flight (buffer resources: parts past H, and
// a padded token's hidden row, read zeros), the chain row_dots as in
// group_exact_kernel, then lane 0 stores the results.
template <int kParts>
__device__ __forceinline__ void exact_channel(const ExactArgs &a, int t, int logical, int slot_id,
                                              uint32_t padded) {
  const int lane = threadIdx.x & 63;
  const int k = logical / a.I, c = logical % a.I;
  const int e = __builtin_amdgcn_readlane(slot_id, k);
  float g = 0.0f, u = 0.0f;
  if (e >= 0) {
    const bool active = __builtin_amdgcn_readfirstlane(padded) == 0;
    const int row_bytes = 2 * a.H, offset = 16 * lane;
    const long grow = (static_cast<long>(e) * 2 * a.I + c) * a.H;
    const __amdgpu_buffer_rsrc_t gate_row = buffer_resource(a.gate_up + grow, row_bytes);
    const __amdgpu_buffer_rsrc_t up_row =
        buffer_resource(a.gate_up + grow + static_cast<long>(a.I) * a.H, row_bytes);
    const __amdgpu_buffer_rsrc_t hidden =
        buffer_resource(a.x + static_cast<long>(t) * a.H, active ? row_bytes : 0);
    uint4 gw[kParts], uw[kParts], xw[kParts];
#pragma unroll
    for (int p = 0; p < kParts; ++p) {
      xw[p] = buffer_load16(hidden, offset + 1024 * p);
      gw[p] = buffer_stream16(gate_row, offset + 1024 * p);
      uw[p] = buffer_stream16(up_row, offset + 1024 * p);
    }
    // (every row part is issued before the first is used)
#pragma unroll
    for (int p = 0; p < kParts; ++p)
      asm volatile("" ::"v"(gw[p].x), "v"(gw[p].y), "v"(gw[p].z), "v"(gw[p].w), "v"(uw[p].x), "v"(uw[p].y),
                   "v"(uw[p].z), "v"(uw[p].w), "v"(xw[p].x), "v"(xw[p].y), "v"(xw[p].z), "v"(xw[p].w));
    row_dots(gw, uw, xw, a.H, lane, g, u);
    g = wave_sum_lane0(g);
    u = wave_sum_lane0(u);
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

// Workgroup = one wave = kept channel f of token t: single-wave workgroups
// spread a batch-1 call's rows over every CU. The kept id, the token's expert
// ids and its padding flag arrive in one round trip, then the gate, up and
// hidden rows with every part in flight (buffer resources: parts past H, and
// a padded token's hidden row, read zeros); the chain is row_dots, as in
// group_exact_kernel.
template <int kParts>
__global__ __launch_bounds__(64) void exact_kernel(ExactArgs a) {
  const int lane = threadIdx.x;
  const int t = blockIdx.y;
  if (static_cast<int>(blockIdx.x) >= a.exact_blocks) {
    const int item = blockIdx.x - a.exact_blocks;  // (tile, slot), tile fastest
    if (2 * item < a.encode_items) encode_pair_direct(a.encode, item, a.encode_items, t);
    return;
  }
  const int f = blockIdx.x;
  asm volatile("" ::"s"(a.partial), "s"(a.activations), "s"(a.completed), "s"(a.gate_up), "s"(a.x),
               "s"(a.H), "s"(a.I), "s"(a.N), "s"(a.gelu), "s"(a.ids), "s"(a.next_ids), "s"(a.K),
               "s"(a.F), "s"(a.padding_source), "s"(a.padding_bytes));
  const int slot_id = lane < a.K ? load_global(a.ids + t * a.K + lane) : -1;
  const uint32_t padded =
      __builtin_amdgcn_raw_buffer_load_b8(buffer_resource(a.padding_source, a.padding_bytes), t, 0, 0);
  const int logical =
      __builtin_amdgcn_readfirstlane(load_global(a.next_ids + static_cast<long>(t) * a.F + f));
  asm volatile("" ::"v"(padded));  // the flag's load stays in this round trip
  if (logical < 0 || logical >= a.N) return;
  exact_channel<kParts>(a, t, logical, slot_id, padded);
}

// Select and exact in one launch for the smallest batches (no kernel boundary
// and no kept-id round trip between them). Workgroup (g, token t) of
// kSelectThreads threads runs the token's selection (select_token: the same
// keys, passes and scans in every workgroup, so all find the same kept
// ids); workgroup 0 stores the select outputs, and wave w < item_waves of
// workgroup g > 0 takes item q = item_waves (g - 1) + w: the q-th kept
// channel (q < F), found from the threads' kept bits and inclusive kept counts
// in LDS, or past F the recovery encoder pair item q - F, whose selected
// flags come from the same bits. The slot experts and padding flag are loaded
// before the selection. The host sizes item_waves so that the workgroups
// (one per compute unit at 16 waves of this kernel's registers) run in one
// round: the rows then come through as many compute units as that allows.
template <int kKeys, int kParts>
__global__ __launch_bounds__(kSelectThreads) void select_exact_kernel(SelectArgs s, ExactArgs a,
                                                                      int item_waves) {
  __shared__ int kept_end[kSelectThreads];
  __shared__ uint32_t kept_bits[kSelectThreads];
  __shared__ __align__(16) float values[kSelectWaves][2][64];
  const int t = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool writer = blockIdx.x == 0;
  const int slot_id = lane < a.K ? load_global(a.ids + t * a.K + lane) : -1;
  const uint32_t padded =
      __builtin_amdgcn_raw_buffer_load_b8(buffer_resource(a.padding_source, a.padding_bytes), t, 0, 0);
  uint32_t kept;
  int base;
  select_token<kKeys>(s, t, writer, true, &kept, &base);
  if (writer) return;
  kept_end[tid] = base + __builtin_popcount(kept);
  kept_bits[tid] = kept;
  __syncthreads();
  if (wave >= item_waves) return;
  const int per = (s.N + kSelectThreads - 1) / kSelectThreads;
  const int q = (static_cast<int>(blockIdx.x) - 1) * item_waves + wave;
  if (q < a.F) {
    // the thread j whose kept run holds position q: lane l reads the end of
    // threads 16 l .. 16 l + 15, then lane l < 16 thread 16 c + l's
    const int chunk_end = kept_end[16 * lane + 15];
    const uint64_t past = __ballot(chunk_end > q);
    if (!past) return;  // q is at or past the kept count: no channel
    const int c = __builtin_ctzll(past);
    const int end = lane < 16 ? kept_end[16 * c + lane] : 0;
    const int j = 16 * c + __builtin_ctzll(__ballot(lane < 16 && end > q));
    const int before = j > 0 ? kept_end[j - 1] : 0;
    uint32_t bits = kept_bits[j];
    for (int n = q - before; n > 0; --n) bits &= bits - 1;
    const int logical = __builtin_amdgcn_readfirstlane(j * per + __builtin_ctz(bits));
    exact_channel<kParts>(a, t, logical, slot_id, padded);
  } else if (2 * (q - a.F) < a.encode_items) {
    encode_pair_direct(a.encode, q - a.F, a.encode_items, t, KeptBits{kept_bits, per}, values[wave]);
  }
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
  const void *padding_source;  // the padding mask and T bytes, or any pointer and 0 bytes
  int padding_bytes;
  float *latent;
  uint16_t *out;
  int H, K, R, max_tiles, encoder_tiles;
  int columns;  // outputs per workgroup (64 or 256, at most kOutputThreads)
};

constexpr int kOutputThreads = 512;
constexpr int kMaxEncoderTiles = 16; // encoder tiles folded per batch: ceil(I / 64) at I <= 1024
constexpr int kTileBatch = 8;        // tile partials loaded together per thread

// Workgroup = `columns` outputs of one token, 512 threads (64 outputs below
// 16 tokens for latency, 256 from there: every workgroup folds its token's
// encoder tiles, so fewer, wider workgroups read them fewer times). Thread
// item (slot k, output) sums the slot's 32-channel tile partials in tile order
// (all loads of a batch issued together) and rounds to BF16; one thread per
// output then mixes the slots in order with the router weights and adds the
// decoder correction. The per-(slot, output) values live in dynamic LDS.
// The decoder correction of one output: an fma chain over r of U[o, r] and
// bf16(latent_r) (`rounded` holds them, 16-byte aligned; a padded token's row
// is zero), rounded to BF16. `row_words` holds U[o, :] when R is a multiple of
// 8 and at most 32, else the row is read here.
__device__ __forceinline__ float decoder_correction(const OutputArgs &a, const uint4 (&row_words)[4],
                                                    bool row_ahead, bool active, int o,
                                                    const float *rounded) {
  const int R = a.R;
  float acc = 0.0f;
  if (row_ahead) {
    float4 l[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) l[i] = reinterpret_cast<const float4 *>(rounded)[min(i, R / 4 - 1)];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (8 * q >= R) break;
      const uint32_t wv[4] = {active ? row_words[q].x : 0u, active ? row_words[q].y : 0u,
                              active ? row_words[q].z : 0u, active ? row_words[q].w : 0u};
      const float lv[8] = {l[2 * q].x, l[2 * q].y, l[2 * q].z, l[2 * q].w,
                           l[2 * q + 1].x, l[2 * q + 1].y, l[2 * q + 1].z, l[2 * q + 1].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc = fmaf(__uint_as_float(wv[i] << 16), lv[2 * i], acc);
        acc = fmaf(__uint_as_float(wv[i] & 0xffff0000u), lv[2 * i + 1], acc);
      }
    }
  } else {
    const uint16_t *row = a.decoder + static_cast<long>(o) * R;
    if ((R & 7) == 0) {
      for (int q = 0; q < R; q += 8) {
        const uint4 w = active ? *reinterpret_cast<const uint4 *>(row + q) : make_uint4(0, 0, 0, 0);
        const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc = fmaf(__uint_as_float(wv[i] << 16), rounded[q + 2 * i], acc);
          acc = fmaf(__uint_as_float(wv[i] & 0xffff0000u), rounded[q + 2 * i + 1], acc);
        }
      }
    } else {
      for (int r = 0; r < R; ++r) {
        const float u = active ? bf16f(row[r]) : 0.0f;
        acc = fmaf(u, rounded[r], acc);
      }
    }
  }
  return bfr(acc);
}

// The decoder row of output o0 + min(tid, columns - 1), issued before any
// other load of the launch (R a multiple of 8, at most 32).
__device__ __forceinline__ void load_decoder_row(const OutputArgs &a, int o0, int columns,
                                                 uint4 (&row_words)[4]) {
  const uint16_t *row = a.decoder + static_cast<long>(min(o0 + min(static_cast<int>(threadIdx.x), columns - 1), a.H - 1)) * a.R;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    row_words[q] = 8 * q < a.R ? *reinterpret_cast<const uint4 *>(row + 8 * q) : make_uint4(0, 0, 0, 0);
}

__global__ __launch_bounds__(kOutputThreads) void output_kernel(OutputArgs a) {
  __shared__ float slot_latent[kMaxSlots * kMaxRank];
  __shared__ __align__(16) float latent[kMaxRank];  // bf16(latent_r) of the token
  __shared__ float slot_weight[kMaxSlots];
  extern __shared__ float slot_value[];  // [K][columns]
  const int t = blockIdx.y, tid = threadIdx.x;
  const int columns = a.columns;
  const int o0 = blockIdx.x * columns;
  const int K = a.K, R = a.R;
  const bool row_ahead = R > 0 && a.decoder && (R & 7) == 0 && R <= 32;
  uint4 row_words[4] = {};
  if (row_ahead) load_decoder_row(a, o0, columns, row_words);
  for (int k = tid; k < K; k += kOutputThreads) slot_weight[k] = a.weights[t * K + k];
  // each slot's encoder tiles summed in tile order, rounded to BF16
  for (int item = tid; item < K * R; item += kOutputThreads) {
    const int k = item / R, r = item % R;
    const float *parts = a.encoder_parts + (static_cast<long>(t) * K + k) * a.encoder_tiles * R + r;
    // batches of kMaxEncoderTiles tiles, each batch's loads issued together
    // (one batch up to I = 1024)
    float total = 0.0f;
    for (int j0 = 0; j0 < a.encoder_tiles; j0 += kMaxEncoderTiles) {
      float v[kMaxEncoderTiles];
#pragma unroll
      for (int j = 0; j < kMaxEncoderTiles; ++j)
        v[j] = j0 + j < a.encoder_tiles ? parts[(j0 + j) * R] : 0.0f;
#pragma unroll
      for (int j = 0; j < kMaxEncoderTiles; ++j)
        if (j0 + j < a.encoder_tiles) total = j0 + j == 0 ? v[j] : total + v[j];
    }
    slot_latent[k * R + r] = bfr(total);
  }
  // each slot's down tiles summed in tile order, rounded to BF16
  for (int item = tid; item < K * columns; item += kOutputThreads) {
    const int k = item / columns, column = item % columns;
    const int o = o0 + column;
    const int first = a.down_tile_starts[t * K + k];
    const int tiles = min((a.counts[t * K + k] + kDownTile - 1) / kDownTile, a.max_tiles - first);
    const float *parts = a.down_parts + (static_cast<long>(t) * a.max_tiles + first) * a.H +
                         min(o, a.H - 1);
    float total = 0.0f;
    for (int j0 = 0; j0 < tiles; j0 += kTileBatch) {
      float v[kTileBatch];
#pragma unroll
      for (int j = 0; j < kTileBatch; ++j)
        v[j] = parts[static_cast<long>(min(j0 + j, tiles - 1)) * a.H];
#pragma unroll
      for (int j = 0; j < kTileBatch; ++j)
        if (j0 + j < tiles) total = j0 + j == 0 ? v[j] : total + v[j];
    }
    slot_value[k * columns + column] = bfr(total);
  }
  __syncthreads();
  if (tid < R) {
    float mixed = 0.0f;
    for (int k = 0; k < K; ++k) mixed = fmaf(slot_latent[k * R + tid], slot_weight[k], mixed);
    latent[tid] = bfr(mixed);
    if (blockIdx.x == 0) a.latent[static_cast<long>(t) * R + tid] = mixed;
  }
  __syncthreads();
  const int o = o0 + tid;
  if (tid >= columns || o >= a.H) return;
  float routed = 0.0f;
  for (int k = 0; k < K; ++k) routed = fmaf(slot_value[k * columns + tid], slot_weight[k], routed);
  const float correction =
      R > 0 && a.decoder ? decoder_correction(a, row_words, row_ahead, is_active(a.padding, t), o, latent) : 0.0f;
  a.out[static_cast<long>(t) * a.H + o] = f2bf(routed + correction);
}

// Output below the grouped size in one round trip: every load of the launch
// is issued before any is used, as buffer loads over the token's ranges (a
// read past a range returns zero, so none sits behind a branch): the decoder
// row, the padding flag, the thread's encoder tiles (item tid = k R + r), all
// max_tiles tile partials of the workgroup's columns (kRounds per thread, into
// LDS) and the slot records. Each item then sums its slot's tiles from LDS in
// the order of output_kernel, with the same roundings. The host launches it
// for K R <= 512 threads, at most kMaxEncoderTiles encoder tiles and
// max_tiles x columns <= kRounds x 512 partials.
constexpr int kStagedRoundsMax = 16;  // 32 KB of staged partials

template <int kRounds>
__global__ __launch_bounds__(kOutputThreads) void output_staged_kernel(OutputArgs a) {
  __shared__ float slot_latent[kMaxSlots * kMaxRank];
  __shared__ __align__(16) float latent[kMaxRank];  // bf16(latent_r) of the token
  __shared__ float slot_weight[kMaxSlots];
  __shared__ int slot_first[kMaxSlots], slot_tiles[kMaxSlots];
  extern __shared__ float slot_value[];  // [K][columns], then the partials [max_tiles][columns]
  const int t = blockIdx.y, tid = threadIdx.x;
  const int columns = a.columns;
  const int o0 = blockIdx.x * columns;
  const int K = a.K, R = a.R;
  const bool row_ahead = R > 0 && a.decoder && (R & 7) == 0 && R <= 32;
  uint4 row_words[4] = {};
  if (row_ahead) load_decoder_row(a, o0, columns, row_words);
  const uint32_t padded =
      __builtin_amdgcn_raw_buffer_load_b8(buffer_resource(a.padding_source, a.padding_bytes), t, 0, 0);
  // encoder tiles of item tid (tiles past the item's read another item's or zero)
  const int item_tiles = K * a.encoder_tiles * R;
  const __amdgpu_buffer_rsrc_t encoder =
      buffer_resource(a.encoder_parts + static_cast<long>(t) * item_tiles, 4 * item_tiles);
  const int encoder_item = min(tid, max(K * R - 1, 0));
  const int encoder_base = ((encoder_item / max(R, 1)) * a.encoder_tiles * R + encoder_item % max(R, 1)) * 4;
  float encoder_v[kMaxEncoderTiles];
#pragma unroll
  for (int j = 0; j < kMaxEncoderTiles; ++j)
    encoder_v[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(encoder, encoder_base + 4 * j * R, 0, 0));
  // the staged partials: item i = tid + 512 j is (tile i / columns, column i % columns)
  const __amdgpu_buffer_rsrc_t parts =
      buffer_resource(a.down_parts + static_cast<long>(t) * a.max_tiles * a.H, 4 * a.max_tiles * a.H);
  float v[kRounds];
#pragma unroll
  for (int j = 0; j < kRounds; ++j) {
    const int item = tid + j * kOutputThreads;
    v[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        parts, ((item / columns) * a.H + o0 + item % columns) * 4, 0, 0));
  }
  // slot records of slot tid < K
  const __amdgpu_buffer_rsrc_t weights = buffer_resource(a.weights + t * K, 4 * K);
  const __amdgpu_buffer_rsrc_t firsts = buffer_resource(a.down_tile_starts + t * K, 4 * K);
  const __amdgpu_buffer_rsrc_t counts = buffer_resource(a.counts + t * K, 4 * K);
  const uint32_t record_weight = __builtin_amdgcn_raw_buffer_load_b32(weights, 4 * tid, 0, 0);
  const int record_first = __builtin_amdgcn_raw_buffer_load_b32(firsts, 4 * tid, 0, 0);
  const int record_count = __builtin_amdgcn_raw_buffer_load_b32(counts, 4 * tid, 0, 0);
  static_assert(kMaxEncoderTiles == 16, "the operand list below");
  asm volatile("" ::"v"(encoder_v[0]), "v"(encoder_v[1]), "v"(encoder_v[2]), "v"(encoder_v[3]),
               "v"(encoder_v[4]), "v"(encoder_v[5]), "v"(encoder_v[6]), "v"(encoder_v[7]),
               "v"(encoder_v[8]), "v"(encoder_v[9]), "v"(encoder_v[10]), "v"(encoder_v[11]),
               "v"(encoder_v[12]), "v"(encoder_v[13]), "v"(encoder_v[14]), "v"(encoder_v[15]),
               "v"(record_weight), "v"(record_first), "v"(record_count), "v"(padded));
#pragma unroll
  for (int j = 0; j < kRounds; ++j) asm volatile("" ::"v"(v[j]));
  float *staged = slot_value + K * columns;
  const int entries = a.max_tiles * columns;
#pragma unroll
  for (int j = 0; j < kRounds; ++j)
    if (tid + j * kOutputThreads < entries) staged[tid + j * kOutputThreads] = v[j];
  if (tid < K) {
    slot_weight[tid] = __uint_as_float(record_weight);
    slot_first[tid] = record_first;
    slot_tiles[tid] = min((record_count + kDownTile - 1) / kDownTile, a.max_tiles - record_first);
  }
  // each slot's encoder tiles summed in tile order, rounded to BF16
  if (tid < K * R) {
    float total = encoder_v[0];
#pragma unroll
    for (int j = 1; j < kMaxEncoderTiles; ++j)
      if (j < a.encoder_tiles) total = total + encoder_v[j];
    slot_latent[tid] = bfr(total);
  }
  __syncthreads();
  // each slot's down tiles summed in tile order, rounded to BF16
  for (int item = tid; item < K * columns; item += kOutputThreads) {
    const int k = item / columns, column = item % columns;
    const int first = slot_first[k], tiles = slot_tiles[k];
    float total = 0.0f;
    for (int j = 0; j < tiles; ++j) {
      const float value = staged[(first + j) * columns + column];
      total = j == 0 ? value : total + value;
    }
    slot_value[item] = bfr(total);
  }
  __syncthreads();
  if (tid < R) {
    float mixed = 0.0f;
    for (int k = 0; k < K; ++k) mixed = fmaf(slot_latent[k * R + tid], slot_weight[k], mixed);
    latent[tid] = bfr(mixed);
    if (blockIdx.x == 0) a.latent[static_cast<long>(t) * R + tid] = mixed;
  }
  __syncthreads();
  const int o = o0 + tid;
  if (tid >= columns || o >= a.H) return;
  float routed = 0.0f;
  for (int k = 0; k < K; ++k) routed = fmaf(slot_value[k * columns + tid], slot_weight[k], routed);
  const float correction =
      R > 0 && a.decoder ? decoder_correction(a, row_words, row_ahead, padded == 0, o, latent) : 0.0f;
  a.out[static_cast<long>(t) * a.H + o] = f2bf(routed + correction);
}

constexpr int kOutputItems = 8;      // (slot, output) items per thread: K x columns <= 8 x 512
constexpr int kWideTileBatch = 4;        // tile partials of an item loaded with the other items'

// The output launch from 128 tokens (512 outputs per workgroup): the same
// arithmetic as output_kernel in two round trips, first the token's slot
// records (into LDS), each thread's encoder tiles and its output's decoder
// row, then the tile partials of all of the thread's (slot k, output) items
// at once (c4: 26.7 -> 23.4 us; below 128 tokens, where a workgroup holds
// fewer items, output_kernel's order is faster). Each
// item sums its slot's 32-channel tile partials in tile order and rounds to
// BF16; one thread per output then mixes the slots in order with the router
// weights and adds the decoder correction. The per-(slot, output) values
// live in dynamic LDS.
__global__ __launch_bounds__(kOutputThreads) void output_wide_kernel(OutputArgs a) {
  __shared__ float slot_latent[kMaxSlots * kMaxRank];
  __shared__ __align__(16) float latent[kMaxRank];  // bf16(latent_r) of the token
  __shared__ float slot_weight[kMaxSlots];
  __shared__ int slot_first[kMaxSlots], slot_tiles[kMaxSlots];
  extern __shared__ float slot_value[];  // [K][columns]
  const int t = blockIdx.y, tid = threadIdx.x;
  const int columns = a.columns;
  const int o0 = blockIdx.x * columns;
  const int K = a.K, R = a.R;
  const int o = o0 + tid;
  const bool mine = tid < columns && o < a.H;
  // round trip 1: slot records, encoder tiles, decoder row
  for (int k = tid; k < K; k += kOutputThreads) {
    slot_weight[k] = a.weights[t * K + k];
    const int first = a.down_tile_starts[t * K + k];
    slot_first[k] = first;
    slot_tiles[k] = min((a.counts[t * K + k] + kDownTile - 1) / kDownTile, a.max_tiles - first);
  }
  const bool direct_encoder = K * R <= kOutputThreads && a.encoder_tiles <= kMaxEncoderTiles;
  float encoder_v[kMaxEncoderTiles];
  if (direct_encoder && tid < K * R) {
    const float *parts = a.encoder_parts + (static_cast<long>(t) * K + tid / R) * a.encoder_tiles * R + tid % R;
#pragma unroll
    for (int j = 0; j < kMaxEncoderTiles; ++j) encoder_v[j] = j < a.encoder_tiles ? parts[j * R] : 0.0f;
  }
  const bool active = is_active(a.padding, t);
  const bool row_ahead = R > 0 && a.decoder && (R & 7) == 0 && R <= 32;
  uint4 decoder_row[4];
  if (row_ahead) {
    const uint16_t *row = a.decoder + static_cast<long>(min(o, a.H - 1)) * R;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      decoder_row[q] = 8 * q < R && active ? *reinterpret_cast<const uint4 *>(row + 8 * q) : make_uint4(0, 0, 0, 0);
  }
  __syncthreads();
  // round trip 2: the tile partials of the thread's items (the first
  // kWideTileBatch tiles of each together; longer slots continue in batches)
  const int items = K * columns;
  float v[kOutputItems][kWideTileBatch];
  const float *item_parts[kOutputItems];
  int item_tiles[kOutputItems];
#pragma unroll
  for (int i = 0; i < kOutputItems; ++i) {
    const int item = tid + i * kOutputThreads;
    const int k = item < items ? item / columns : 0;
    const int column = item < items ? item % columns : 0;
    const int first = slot_first[k];
    item_tiles[i] = item < items ? slot_tiles[k] : 0;
    item_parts[i] = a.down_parts + (static_cast<long>(t) * a.max_tiles + first) * a.H + min(o0 + column, a.H - 1);
#pragma unroll
    for (int j = 0; j < kWideTileBatch; ++j)
      v[i][j] = j < item_tiles[i] ? item_parts[i][static_cast<long>(j) * a.H] : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < kOutputItems; ++i) {
    const int item = tid + i * kOutputThreads;
    if (item >= items) continue;
    float total = 0.0f;
#pragma unroll
    for (int j = 0; j < kWideTileBatch; ++j)
      if (j < item_tiles[i]) total = j == 0 ? v[i][j] : total + v[i][j];
    for (int j0 = kWideTileBatch; j0 < item_tiles[i]; j0 += kWideTileBatch) {
      float w[kWideTileBatch];
#pragma unroll
      for (int j = 0; j < kWideTileBatch; ++j)
        w[j] = item_parts[i][static_cast<long>(min(j0 + j, item_tiles[i] - 1)) * a.H];
#pragma unroll
      for (int j = 0; j < kWideTileBatch; ++j)
        if (j0 + j < item_tiles[i]) total = total + w[j];
    }
    slot_value[item] = bfr(total);  // item = k * columns + column
  }
  // each slot's encoder tiles summed in tile order, rounded to BF16
  if (direct_encoder) {
    if (tid < K * R) {
      float total = encoder_v[0];
#pragma unroll
      for (int j = 1; j < kMaxEncoderTiles; ++j)
        if (j < a.encoder_tiles) total = total + encoder_v[j];
      slot_latent[tid] = bfr(total);  // tid = k * R + r
    }
  } else {
    for (int item = tid; item < K * R; item += kOutputThreads) {
      const int k = item / R, r = item % R;
      const float *parts = a.encoder_parts + (static_cast<long>(t) * K + k) * a.encoder_tiles * R + r;
      float total = parts[0];
      for (int j = 1; j < a.encoder_tiles; ++j) total = total + parts[j * R];
      slot_latent[k * R + r] = bfr(total);
    }
  }
  __syncthreads();
  if (tid < R) {
    float mixed = 0.0f;
    for (int k = 0; k < K; ++k) mixed = fmaf(slot_latent[k * R + tid], slot_weight[k], mixed);
    latent[tid] = bfr(mixed);
    if (blockIdx.x == 0) a.latent[static_cast<long>(t) * R + tid] = mixed;
  }
  __syncthreads();
  if (!mine) return;
  float routed = 0.0f;
  for (int k = 0; k < K; ++k) routed = fmaf(slot_value[k * columns + tid], slot_weight[k], routed);
  const float correction =
      R > 0 && a.decoder ? decoder_correction(a, decoder_row, row_ahead, active, o, latent) : 0.0f;
  a.out[static_cast<long>(t) * a.H + o] = f2bf(routed + correction);
}

// ---------------------------------------------------------------------------
// host side

thread_local char g_error[512] = "";

// Upper bound of the grouping's tile count: every touched expert contributes
// one tile plus one per 16 further pairs.
long tile_bound(int tokens, int top_k, int experts) {
  const long pairs = static_cast<long>(tokens) * top_k;
  const long touched = pairs < experts ? pairs : experts;
  const long bound = touched + pairs / kGroupPairs;
  return pairs < bound ? pairs : bound;
}

// Compute units of the current device (cached per device).
long compute_units() {
  static int cached[64] = {};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 256;
  if (cached[device] == 0) {
    int units = 0;
    if (hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device) !=
            hipSuccess ||
        units <= 0)
      units = 256;
    cached[device] = units;
  }
  return cached[device];
}

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
  if (d->top_k < 1 || d->top_k > kMaxSlots) return fail(CFMOE_EINVAL, "top_k must be in [1, 64]");
  if (d->rank < 0 || d->rank > kMaxRank) return fail(CFMOE_EINVAL, "rank must be in [0, 64]");
  if (d->keep < 1 || d->keep > 128) return fail(CFMOE_EINVAL, "keep must be in [1, 128]");
  const int n = d->top_k * d->width;
  if (d->final_count < 1 || d->final_count > n) return fail(CFMOE_EINVAL, "final_count must be in [1, N]");
  if (n > kSelectThreads * kSelectKeys) return fail(CFMOE_EINVAL, "N exceeds 16384 candidates");
  if (d->experts < 1 || d->experts > kMaxExperts) return fail(CFMOE_EINVAL, "experts must be in [1, 4096]");
  if (d->hidden > 128 * 8 * kMaxSpan || d->hidden > kMaxHidden)
    return fail(CFMOE_EINVAL, "hidden must be at most 4096");
  if (2 * d->width > kMaxRows) return fail(CFMOE_EINVAL, "width must be at most 2048");
  // a grouped call needs the fused screen, which clears the tile masks that
  // select and the grouped exact rows share: two tokens at least
  if (d->grouped_tokens < 0 || d->grouped_tokens == 1)
    return fail(CFMOE_EINVAL, "grouped_tokens must be 0 (the default) or at least 2");
  return 0;
}

constexpr int kDefaultGroupedTokens = 16;  // cfmoe_dims.grouped_tokens = 0

struct Shape {
  int H, I, K, N, F, R, B, keep, splits, span, max_tiles, encoder_tiles, grouped_tokens;
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
  s.max_tiles = (s.F + kDownTile - 1) / kDownTile + s.K - 1;
  s.encoder_tiles = (s.I + 63) / 64;
  s.screened = s.F < s.N;
  s.grouped_tokens = d->grouped_tokens > 0 ? d->grouped_tokens : kDefaultGroupedTokens;
  return s;
}

// down_order layout: the down kernel's workgroup list (capacity * max_tiles + 8
// entries, rounded up to even), then kDownBuilders areas of slot records,
// 16 * capacity * K records of two words each (a slot per routing-tile pair:
// tiles <= T * K).
long down_list_words(long capacity, const Shape &s) {
  return (capacity * s.max_tiles + 8 + 1) / 2 * 2;
}
long down_slot_capacity(long capacity, const Shape &s) { return kGroupPairs * capacity * s.K; }
long down_order_words(long capacity, const Shape &s) {
  return down_list_words(capacity, s) + 2L * kDownBuilders * down_slot_capacity(capacity, s);
}


PrepareArgs prepare_args(const Shape &s, const cfmoe_dims *d, const cfmoe_weights *w,
                         const cfmoe_workspace *ws, const void *hidden, const void *router_ids,
                         const void *router_weights, const uint8_t *padding, int tokens,
                         const double *charges, bool route, bool rotate) {
  PrepareArgs a;
  memset(&a, 0, sizeof(a));
  a.x = static_cast<const uint16_t *>(hidden);
  a.signs = w->signs;
  a.padding = padding;
  a.padding_source = padding ? static_cast<const void *>(padding) : static_cast<const void *>(w->signs);
  a.padding_bytes = padding ? tokens : 0;
  a.router_ids = router_ids;
  a.router_weights = router_weights;
  a.ids = ws->ids;
  a.weights = ws->weights;
  a.planes = ws->planes;
  a.coords = ws->coordinates;
  a.qvals = ws->qvals;
  a.qexp = ws->qexp;
  a.qsums = ws->qsums;
  a.norm2 = ws->norm2;
  a.digits = ws->digits;
  a.group_experts = ws->group_experts;
  a.group_starts = ws->group_starts;
  a.group_counts = ws->group_counts;
  a.group_pairs = ws->group_pairs;
  a.pair_tiles = ws->pair_tiles;
  a.group_total = ws->group_total;
  a.read_work = ws->read_work;
  if (charges && (d->flags & CFMOE_ACCOUNT))
    for (int i = 0; i < 18; ++i) a.charges[i] = charges[i];
  if (route && (d->flags & CFMOE_ACCOUNT)) {
    // per tile: the screen streams the expert's trit planes (64 I B bytes)
    // and its FP16 scale (and residual) planes, and issues 2 I x 16 pairs x
    // 128 coordinates x 3 grid digits int8 MACs per block; a grouped call of
    // a dense plan reads every gate/up row of the tile's expert once
    const bool gh5 = !(d->flags & CFMOE_POINT);
    if (s.screened) {
      a.tile_sketch_bytes = 64.0 * s.I * s.B + 2.0 * 2 * s.I * s.B * (gh5 ? 2 : 1);
      a.tile_screen_macs = 2.0 * s.I * kGroupPairs * 128.0 * 3 * s.B;
    } else if (tokens >= s.grouped_tokens) {
      a.tile_row_bytes = 4.0 * s.H * s.I;
    }
  }
  a.T = tokens;
  a.H = s.H;
  a.K = s.K;
  a.E = d->experts;
  a.keep = s.keep;
  a.flags = d->flags;
  a.route = route;
  a.rotate = rotate;
  a.cells = tokens * (rotate ? s.B : 1);
  return a;
}

int launch_prepare(const Shape &s, const cfmoe_dims *d, const cfmoe_weights *w,
                   const cfmoe_workspace *ws, const void *hidden, const void *router_ids,
                   const void *router_weights, const uint8_t *padding, int tokens,
                   const double *charges, bool route, bool rotate, hipStream_t stream) {
  const PrepareArgs a =
      prepare_args(s, d, w, ws, hidden, router_ids, router_weights, padding, tokens, charges, route, rotate);
  const int pairs = tokens * s.K;
  const bool wide = route && pairs >= kWidePreparePairs &&
                    route_lds_bytes(pairs, d->experts, kWidePrepareThreads / 64) <= 96 * 1024;
  const int threads = wide ? kWidePrepareThreads : kPrepareThreads;
  const int cell_blocks = (a.cells + threads / 64 - 1) / (threads / 64);
  // (a one-token call routes on one wave, without the LDS lists)
  const long lds = route && tokens > 1 ? route_lds_bytes(pairs, d->experts, threads / 64) : 0;
  if (wide)
    hipLaunchKernelGGL(prepare_kernel<kWidePrepareThreads>, dim3(cell_blocks + 1), dim3(threads),
                       static_cast<unsigned>(lds), stream, a);
  else
    hipLaunchKernelGGL(prepare_kernel<kPrepareThreads>, dim3(cell_blocks + (route ? 1 : 0)), dim3(threads),
                       static_cast<unsigned>(lds), stream, a);
  return check_launch("prepare");
}

}  // namespace cfmoe

extern "C" {

using namespace cfmoe;


int cfmoe_abi_version(void) { return CFMOE_ABI_VERSION; }

const char *cfmoe_last_error(void) { return g_error; }

int cfmoe_workspace_sizes(const cfmoe_dims *dims, int32_t capacity, int64_t *sizes,
                          int32_t count) {
  if (int rc = validate(dims)) return -rc;
  const Shape s = shape_of(dims);
  const int64_t cap = capacity;
  const int64_t n = s.N;
  const int64_t table[kWorkspaceBuffers] = {
      cap * s.K * 4,                          // ids
      cap * s.K * 4,                          // weights
      cap * s.B * s.keep * 4,                 // planes
      cap * s.B * s.keep * 4,                 // coordinates
      cap * s.B * s.keep * 4,                 // qvals
      cap * s.B * 4,                          // qexp
      cap * s.B * 4,                          // qsums
      cap * s.B * 4,                          // norm2
      cap * 2 * n * 4,                        // partial
      cap * 2 * n * 4,                        // variances
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
      cap * s.K * 4,                          // group_experts
      cap * s.K * 4,                          // group_starts
      cap * s.K * 4,                          // group_counts
      cap * s.K * kGroupPairs * 4,            // group_pairs (16 slots per tile)
      4,                                      // group_total
      cap * s.K * 4,                          // pair_tiles
      cap * n * 4,                            // tile_masks (tiles * I <= cap * N)
      down_order_words(cap, s) * 4,           // down_order (list + builders' slot records)
      cap * s.B * 3 * 128,                    // digits
  };
  const int written = count < kWorkspaceBuffers ? count : kWorkspaceBuffers;
  for (int i = 0; i < written; ++i) sizes[i] = table[i];
  return written;
}

int64_t cfmoe_trit_plane_bytes(const cfmoe_dims *dims) {
  if (int rc = validate(dims)) return -rc;
  return static_cast<int64_t>(dims->experts) * (dims->hidden / 128) * dims->width * 64;
}

int cfmoe_pack_trit_planes(const cfmoe_dims *dims, const uint8_t *codes, uint32_t *planes,
                           cfmoe_stream stream) {
  if (int rc = validate(dims)) return rc;
  if (!codes || !planes) return fail(CFMOE_EINVAL, "NULL argument");
  if (reinterpret_cast<uintptr_t>(planes) % 8)
    return fail(CFMOE_EINVAL, "trit_planes must be 8-byte aligned");
  PackArgs a;
  a.codes = codes;
  a.planes = reinterpret_cast<uint2 *>(planes);
  a.I = dims->width;
  a.B = dims->hidden / 128;
  a.storage = storage_bytes(2 * a.I, dims->hidden);
  const int stride = code_stride(2 * a.I);
  a.body = stride - stride % 32;
  a.total = static_cast<long>(dims->experts) * a.B * (2 * a.I / kRowTile) * 64;
  const long blocks = (a.total + 255) / 256;
  hipLaunchKernelGGL(pack_trit_planes_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return check_launch("pack_trit_planes");
}

int cfmoe_unpack_trit_planes(const cfmoe_dims *dims, const uint32_t *planes, uint8_t *codes,
                             cfmoe_stream stream) {
  if (int rc = validate(dims)) return rc;
  if (!codes || !planes) return fail(CFMOE_EINVAL, "NULL argument");
  if (reinterpret_cast<uintptr_t>(planes) % 8)
    return fail(CFMOE_EINVAL, "trit_planes must be 8-byte aligned");
  PackArgs a;
  a.codes = nullptr;
  a.planes = reinterpret_cast<uint2 *>(const_cast<uint32_t *>(planes));
  a.codes_out = codes;
  a.I = dims->width;
  a.B = dims->hidden / 128;
  a.storage = storage_bytes(2 * a.I, dims->hidden);
  const int stride = code_stride(2 * a.I);
  a.body = stride - stride % 32;
  a.total = static_cast<long>(dims->experts) * a.storage;
  const long blocks = (a.total + 255) / 256;
  hipLaunchKernelGGL(unpack_trit_planes_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return check_launch("unpack_trit_planes");
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

namespace cfmoe {

static SmallScreenArgs small_screen_args(const Shape &s, const cfmoe_dims *dims, const cfmoe_weights *weights,
                                         const cfmoe_workspace *workspace, const uint8_t *padding,
                                         int32_t tokens) {
  const uint32_t flags = dims->flags;
  SmallScreenArgs ss;
  ss.planes = reinterpret_cast<const uint2 *>(weights->trit_planes);
  ss.stats = static_cast<const uint16_t *>(weights->statistics);
  ss.digits = workspace->digits;
  ss.qexp = workspace->qexp;
  ss.qsums = workspace->qsums;
  ss.norm2 = workspace->norm2;
  ss.group_experts = workspace->group_experts;
  ss.group_counts = workspace->group_counts;
  ss.group_pairs = workspace->group_pairs;
  ss.group_total = workspace->group_total;
  ss.ids = workspace->ids;
  ss.weights = workspace->weights;
  ss.padding = padding;
  ss.norms = weights->norms;
  ss.geometry = (flags & CFMOE_GEOMETRY) ? weights->geometry : nullptr;
  ss.partial = workspace->partial;
  ss.variances = workspace->variances;
  ss.scores = workspace->scores;
  ss.H = s.H;
  ss.I = s.I;
  ss.K = s.K;
  ss.N = s.N;
  ss.T = tokens;
  ss.splits = s.splits;
  ss.span = s.span;
  ss.tile_items = static_cast<int>(tile_bound(tokens, s.K, dims->experts)) * (s.I / kRowTile);
  // a tile holds at most 16 pairs, and at most tokens * K
  ss.max_pairs = static_cast<int>(std::min<long>(kPairTile, static_cast<long>(tokens) * s.K));
  ss.gelu = (flags & CFMOE_GELU) != 0;
  ss.point = (flags & CFMOE_POINT) != 0;
  return ss;
}

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
  if (tokens * s.K > kMaxPairs) return fail(CFMOE_EINVAL, "tokens * top_k exceeds 8192 pairs");
  if (s.R > 0 && (!weights->encoder_t || !weights->decoder))
    return fail(CFMOE_EINVAL, "rank > 0 needs encoder and decoder");
  if (s.R == kDirectRank && (!weights->encoder_tiles || reinterpret_cast<uintptr_t>(weights->encoder_tiles) % 16))
    return fail(CFMOE_EINVAL, "encoder_tiles (16-byte aligned) is required at rank 32");
  if ((dims->flags & CFMOE_THRESHOLD) && !weights->threshold)
    return fail(CFMOE_EINVAL, "threshold flag without threshold");
  if (s.screened && (!weights->trit_planes || reinterpret_cast<uintptr_t>(weights->trit_planes) % 8))
    return fail(CFMOE_EINVAL, "trit_planes must be an 8-byte aligned cfmoe_pack_trit_planes output");
  if (s.screened && (!weights->statistics || reinterpret_cast<uintptr_t>(weights->statistics) % 8))
    return fail(CFMOE_EINVAL, "statistics must be 8-byte aligned (the screen loads four at a time)");
  // the fused screen stores four projections or scores at a time, reads four norms
  if (s.screened && ((reinterpret_cast<uintptr_t>(workspace->partial) |
                      reinterpret_cast<uintptr_t>(workspace->variances) |
                      reinterpret_cast<uintptr_t>(workspace->scores) |
                      reinterpret_cast<uintptr_t>(workspace->digits) |
                      reinterpret_cast<uintptr_t>(weights->norms) |
                      reinterpret_cast<uintptr_t>((dims->flags & CFMOE_GEOMETRY) ? weights->geometry
                                                                           : nullptr)) % 16))
    return fail(CFMOE_EINVAL,
                "partial, variances, scores, digits, norms and geometry must be 16-byte aligned");
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
  sel.completed = workspace->completed;
  sel.counts = workspace->counts;
  sel.starts = workspace->starts;
  sel.tile_starts = workspace->tile_starts;
  sel.down_tile_starts = workspace->down_tile_starts;
  sel.N = s.N;
  sel.F = s.F;
  sel.I = s.I;
  sel.K = s.K;
  sel.thresholded = (flags & CFMOE_THRESHOLD) != 0;
  // per-(tile, channel) pair masks for the grouped exact kernel; that launch
  // counts their nonzero words as the union rows it reads (4 H bytes each)
  const bool grouped = tokens >= s.grouped_tokens;
  const bool masked = s.screened && grouped;
  sel.pair_tiles = workspace->pair_tiles;
  sel.tile_masks = masked ? workspace->tile_masks : nullptr;
  // Up to kSelectExactTokens tokens a call that runs both stages runs select
  // and exact as one launch (select_exact_kernel, in the exact launch's place)
  // when its workgroups at 16 item waves each fit on the compute units at
  // once (a second round would cost more than the launch saves)
  const int fused_items = s.F + (s.R == kDirectRank ? (s.encoder_tiles * s.K + 1) / 2 : 0);
  const bool fuse_select = s.screened && !grouped && tokens <= kSelectExactTokens &&
                           (stages & (1u << CFMOE_STAGE_SELECT)) && (stages & (1u << CFMOE_STAGE_EXACT)) &&
                           hidden_parts(s.H) == kNarrowParts &&
                           tokens * (1L + (fused_items + kSelectWaves - 1) / kSelectWaves) <= compute_units();

  if (s.screened) {
    const uint2 *trit_planes = reinterpret_cast<const uint2 *>(weights->trit_planes);
    const uint16_t *statistics = static_cast<const uint16_t *>(weights->statistics);
    const long tiles = tile_bound(tokens, s.K, dims->experts);
    // From kFusedScreenTokens tokens the fused screen (every split of a
    // channel tile in one wave, four channel tiles per workgroup); a batch-1
    // call: a workgroup per channel tile whose waves share the splits (lower
    // latency for one pair per tile). Both score in place and give the same
    // bits; workgroups of tiles past the device's tile count exit at once, and
    // one workgroup per token writes absent slots.
    if ((stages & (1u << CFMOE_STAGE_SCREEN)) && tokens >= kFusedScreenTokens) {
      FusedScreenArgs fs;
      fs.planes = trit_planes;
      fs.stats = statistics;
      fs.digits = workspace->digits;
      fs.qexp = workspace->qexp;
      fs.qsums = workspace->qsums;
      fs.norm2 = workspace->norm2;
      fs.ids = workspace->ids;
      fs.weights = workspace->weights;
      fs.padding = padding;
      fs.norms = weights->norms;
      fs.geometry = (flags & CFMOE_GEOMETRY) ? weights->geometry : nullptr;
      fs.group_experts = workspace->group_experts;
      fs.group_counts = workspace->group_counts;
      fs.group_pairs = workspace->group_pairs;
      fs.group_total = workspace->group_total;
      fs.partial = workspace->partial;
      fs.variances = workspace->variances;
      fs.scores = workspace->scores;
      fs.tile_masks = sel.tile_masks;
      fs.H = s.H;
      fs.I = s.I;
      fs.K = s.K;
      fs.N = s.N;
      fs.T = tokens;
      fs.splits = s.splits;
      fs.span = s.span;
      fs.channel_groups = (s.I / kRowTile + kFusedWaves - 1) / kFusedWaves;
      fs.tile_items = static_cast<int>(tiles) * fs.channel_groups;
      fs.gelu = gelu;
      fs.point = !gh5;
      const unsigned blocks = static_cast<unsigned>(fs.tile_items + tokens);
      const bool narrow = s.span <= kNarrowSpan;
      if (gh5 && narrow)
        hipLaunchKernelGGL((fused_screen_kernel<true, kNarrowSpan>), dim3(blocks), dim3(kFusedThreads), 0, stream, fs);
      else if (gh5)
        hipLaunchKernelGGL((fused_screen_kernel<true, kMaxSpan>), dim3(blocks), dim3(kFusedThreads), 0, stream, fs);
      else if (narrow)
        hipLaunchKernelGGL((fused_screen_kernel<false, kNarrowSpan>), dim3(blocks), dim3(kFusedThreads), 0, stream, fs);
      else
        hipLaunchKernelGGL((fused_screen_kernel<false, kMaxSpan>), dim3(blocks), dim3(kFusedThreads), 0, stream, fs);
      if ((rc = check_launch("screen"))) return rc;
    } else if (stages & (1u << CFMOE_STAGE_SCREEN)) {
      const SmallScreenArgs ss = small_screen_args(s, dims, weights, workspace, padding, tokens);
      const unsigned blocks = static_cast<unsigned>(ss.tile_items + tokens);
      const bool narrow = s.span <= kNarrowSpan;
      const unsigned lds = static_cast<unsigned>(small_screen_lds(ss.max_pairs, narrow ? kNarrowSpan : kMaxSpan));
      if (gh5 && narrow)
        hipLaunchKernelGGL((small_screen_kernel<true, kNarrowSpan>), dim3(blocks), dim3(64 * kSmallWaves), lds,
                           stream, ss);
      else if (gh5)
        hipLaunchKernelGGL((small_screen_kernel<true, kMaxSpan>), dim3(blocks), dim3(64 * kSmallWaves), lds,
                           stream, ss);
      else if (narrow)
        hipLaunchKernelGGL((small_screen_kernel<false, kNarrowSpan>), dim3(blocks), dim3(64 * kSmallWaves), lds,
                           stream, ss);
      else
        hipLaunchKernelGGL((small_screen_kernel<false, kMaxSpan>), dim3(blocks), dim3(64 * kSmallWaves), lds,
                           stream, ss);
      if ((rc = check_launch("screen"))) return rc;
    }

    if ((stages & (1u << CFMOE_STAGE_SELECT)) && !fuse_select) {
      if (s.N <= 8 * kSelectThreads)
        hipLaunchKernelGGL(select_kernel<8>, dim3(tokens), dim3(kSelectThreads), 0, stream, sel);
      else
        hipLaunchKernelGGL(select_kernel<kSelectKeys>, dim3(tokens), dim3(kSelectThreads), 0,
                           stream, sel);
      if ((rc = check_launch("select"))) return rc;
    }
  } else if (stages & (1u << CFMOE_STAGE_SELECT)) {
    hipLaunchKernelGGL(select_all_kernel, dim3((s.N + 255) / 256, tokens), dim3(256), 0, stream,
                       sel);
    if ((rc = check_launch("select_all"))) return rc;
  }

  EncodeArgs en;
  memset(&en, 0, sizeof(en));
  en.encoder_t = static_cast<const uint16_t *>(weights->encoder_t);
  en.encoder_tiles = static_cast<const uint16_t *>(weights->encoder_tiles);
  en.E = dims->experts;
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
  // At R = kDirectRank the encoder runs inside the exact launch (it needs no
  // LDS there), which the exact stage launches (also alone, through
  // cfmoe_launch_stage); the encode stage then has no launch of its own.
  // Grouped batches build the down kernel's workgroup order (expert-grouped
  // per XCD) in the exact launch and read it in the down launch.
  const bool encode_in_exact = s.R == kDirectRank;
  const bool fuse_encode = encode_in_exact && (stages & (1u << CFMOE_STAGE_EXACT));
  const int encode_items = fuse_encode ? s.encoder_tiles * s.K : 0;  // per token
  const int down_blocks = (tokens * s.max_tiles + 7) / 8 * 8;
  const uint16_t *gate_up = static_cast<const uint16_t *>(weights->gate_up);
  const uint16_t *down = static_cast<const uint16_t *>(weights->down);
  uint16_t *activations = static_cast<uint16_t *>(workspace->activations);
  if ((stages & (1u << CFMOE_STAGE_EXACT)) && grouped) {
    GroupExactArgs gx;
    gx.gate_up = gate_up;
    gx.x = static_cast<const uint16_t *>(hidden);
    gx.padding = padding;
    gx.ids = workspace->ids;
    gx.next_ids = workspace->next_ids;
    gx.counts = workspace->counts;
    gx.starts = workspace->starts;
    gx.selected = workspace->selected;
    gx.group_experts = workspace->group_experts;
    gx.group_starts = workspace->group_starts;
    gx.group_counts = workspace->group_counts;
    gx.group_pairs = workspace->group_pairs;
    gx.group_total = workspace->group_total;
    gx.tile_masks = workspace->tile_masks;
    gx.dense = s.screened ? 0 : 1;
    gx.partial = workspace->partial;
    gx.activations = activations;
    gx.completed = workspace->completed;
    gx.H = s.H;
    gx.I = s.I;
    gx.K = s.K;
    gx.N = s.N;
    gx.F = s.F;
    gx.T = tokens;
    gx.gelu = gelu;
    gx.channel_groups = (s.I + kExactChannels - 1) / kExactChannels;
    gx.tile_items = static_cast<int>(tile_bound(tokens, s.K, dims->experts)) * gx.channel_groups;
    gx.encoder_t = en.encoder_t;
    gx.encoder_tiles = en.encoder_tiles;
    gx.E = en.E;
    gx.parts = en.parts;
    gx.tiles = en.tiles;
    gx.encode_items = encode_items * tokens;
    gx.down_order = workspace->down_order;
    gx.pair_tiles = workspace->pair_tiles;
    gx.down_tile_starts = workspace->down_tile_starts;
    gx.max_tiles = s.max_tiles;
    gx.down_blocks = down_blocks;
    gx.order_words = static_cast<int>(down_list_words(workspace->capacity, s));
    gx.slot_capacity = static_cast<int>(down_slot_capacity(workspace->capacity, s));
    gx.read_work = masked && (flags & CFMOE_ACCOUNT) ? workspace->read_work : nullptr;
    gx.union_row_bytes = 4.0 * s.H;
    const int counters = gx.read_work ? kUnionCounters : 0;
    if (hidden_parts(s.H) == kNarrowParts)
      hipLaunchKernelGGL(group_exact_kernel<kNarrowParts>,
                       dim3(kDownBuilders + counters + gx.tile_items + (gx.encode_items + 1) / 2 + tokens),
                       dim3(64 * kGroupExactWaves), 0, stream, gx);
    else
      hipLaunchKernelGGL(group_exact_kernel<kWideParts>,
                       dim3(kDownBuilders + counters + gx.tile_items + (gx.encode_items + 1) / 2 + tokens),
                       dim3(64 * kGroupExactWaves), 0, stream, gx);
    if ((rc = check_launch("exact"))) return rc;
  } else if (stages & (1u << CFMOE_STAGE_EXACT)) {
    ExactArgs ex;
    ex.gate_up = gate_up;
    ex.x = static_cast<const uint16_t *>(hidden);
    ex.ids = workspace->ids;
    ex.padding = padding;
    ex.next_ids = workspace->next_ids;
    ex.partial = workspace->partial;
    ex.activations = activations;
    ex.completed = workspace->completed;
    ex.H = s.H;
    ex.I = s.I;
    ex.K = s.K;
    ex.N = s.N;
    ex.F = s.F;
    ex.gelu = gelu;
    ex.encode = en;
    ex.exact_blocks = s.F;
    ex.encode_items = encode_items;
    ex.padding_source = padding ? static_cast<const void *>(padding) : static_cast<const void *>(weights->signs);
    ex.padding_bytes = padding ? tokens : 0;
    if (fuse_select) {
      // the fewest item waves per workgroup that fit the launch's workgroups
      // (one per token writing, the rest taking items) on the compute units
      const int items = s.F + (encode_items + 1) / 2;  // fused_items
      const long groups = std::max(1L, compute_units() / tokens - 1);
      const int item_waves =
          static_cast<int>(std::min<long>(kSelectWaves, std::max<long>(1, (items + groups - 1) / groups)));
      const dim3 grid(1 + (items + item_waves - 1) / item_waves, tokens);
      if (s.N <= 8 * kSelectThreads)
        hipLaunchKernelGGL((select_exact_kernel<8, kNarrowParts>), grid, dim3(kSelectThreads), 0, stream, sel, ex,
                           item_waves);
      else
        hipLaunchKernelGGL((select_exact_kernel<kSelectKeys, kNarrowParts>), grid, dim3(kSelectThreads), 0, stream,
                           sel, ex, item_waves);
    } else if (hidden_parts(s.H) == kNarrowParts)
      hipLaunchKernelGGL(exact_kernel<kNarrowParts>, dim3(s.F + (encode_items + 1) / 2, tokens), dim3(kWave), 0,
                         stream, ex);
    else
      hipLaunchKernelGGL(exact_kernel<kWideParts>, dim3(s.F + (encode_items + 1) / 2, tokens), dim3(kWave), 0,
                         stream, ex);
    if ((rc = check_launch("exact"))) return rc;
  }

  if (s.R > 0 && (stages & (1u << CFMOE_STAGE_ENCODE)) && !encode_in_exact) {
    hipLaunchKernelGGL(encode_kernel, dim3(s.encoder_tiles, s.K, tokens), dim3(64), 0, stream, en);
    if ((rc = check_launch("encode"))) return rc;
  }

  if (stages & (1u << CFMOE_STAGE_DOWN)) {
    DownArgs dn;
    dn.down = down;
    dn.activations = activations;
    dn.ids = workspace->ids;
    dn.padding = padding;
    dn.next_ids = workspace->next_ids;
    dn.counts = workspace->counts;
    dn.starts = workspace->starts;
    dn.down_tile_starts = workspace->down_tile_starts;
    dn.order = grouped ? workspace->down_order : nullptr;
    dn.parts = workspace->down_parts;
    dn.H = s.H;
    dn.I = s.I;
    dn.K = s.K;
    dn.N = s.N;
    dn.F = s.F;
    dn.max_tiles = s.max_tiles;
    dn.padding_source = padding ? static_cast<const void *>(padding) : static_cast<const void *>(weights->signs);
    dn.padding_bytes = padding ? tokens : 0;
    const int down_threads = ((s.H / kDownOutputs + kWave - 1) / kWave) * kWave;
    if (grouped) {
      hipLaunchKernelGGL(down_kernel, dim3(down_blocks), dim3(down_threads), 0, stream, dn);
    } else {
      // one wave per workgroup and 512 outputs each: a batch-1 call's tiles
      // spread over H / 512 times as many CUs
      hipLaunchKernelGGL(down_kernel, dim3(s.max_tiles, tokens, down_threads / kWave), dim3(kWave),
                         0, stream, dn);
    }
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
  op.padding_source = padding ? static_cast<const void *>(padding) : static_cast<const void *>(weights->signs);
  op.padding_bytes = padding ? tokens : 0;
  op.latent = workspace->latent;
  op.out = static_cast<uint16_t *>(out);
  op.H = s.H;
  op.K = s.K;
  op.R = s.R;
  op.max_tiles = s.max_tiles;
  op.encoder_tiles = s.encoder_tiles;
  // wider workgroups fold each token's encoder tiles fewer times: 512 outputs
  // from 64 tokens (c3 at 128 tokens: 18.4 -> 14.6 us; at 100 tokens 13.7 ->
  // 10.0, the launch's workgroups then fit at two per CU), 256 from the
  // grouped size, 64 below it; LDS K x columns x 4 <= 16 KB
  op.columns = !grouped ? 64 : s.K <= 8 && tokens >= 64 ? 512 : s.K <= 16 ? 256 : 64;
  const unsigned value_lds = static_cast<unsigned>(s.K * op.columns * sizeof(float));
  const long staged = static_cast<long>(s.max_tiles) * op.columns;  // partials per workgroup
  const long rounds = (staged + kOutputThreads - 1) / kOutputThreads;
  const unsigned staged_lds = value_lds + static_cast<unsigned>(staged * sizeof(float));
  const dim3 grid((s.H + op.columns - 1) / op.columns, tokens);
  const bool stageable = s.H % op.columns == 0 && s.K * s.R <= kOutputThreads &&
                         s.encoder_tiles <= kMaxEncoderTiles && rounds <= kStagedRoundsMax;
  // the two-round-trip kernel (slot records, encoder tiles and decoder row;
  // then every item's tile partials at once) from 64 tokens, at 512 columns
  // or, above top-8, 256 (c2's layer 160.9 -> 159.3 us; at 16 and 32 tokens
  // it measured 0.4-0.6 us slower than the one-pass kernel)
  if (tokens >= 64 && op.columns >= 256)
    hipLaunchKernelGGL(output_wide_kernel, grid, dim3(kOutputThreads), value_lds, stream, op);
  else if (stageable && rounds <= 4)
    hipLaunchKernelGGL(output_staged_kernel<4>, grid, dim3(kOutputThreads), staged_lds, stream, op);
  else if (stageable && rounds <= 8)
    hipLaunchKernelGGL(output_staged_kernel<8>, grid, dim3(kOutputThreads), staged_lds, stream, op);
  else if (stageable)
    hipLaunchKernelGGL(output_staged_kernel<16>, grid, dim3(kOutputThreads), staged_lds, stream, op);
  else
    hipLaunchKernelGGL(output_kernel, grid, dim3(kOutputThreads), value_lds, stream, op);
  return check_launch("output");
}

}  // namespace cfmoe

extern "C" {

using namespace cfmoe;


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

// ---------------------------------------------------------------------------
// Allocation-free forward: the workspace lives in one file-scope device array.
//
// For callers that cannot allocate device memory (code under graph capture,
// tight serving loops, hosts that forbid hipMalloc). Every GPU the library
// runs on holds its own copy of `scratch` until the process ends. In host code
// the array's name is only a stand-in for the symbol: its device address on
// the current GPU comes from hipGetSymbolAddress, looked up once per device
// and kept in g_scratch_address; only that address is handed to kernels.

namespace cfmoe {

constexpr long kScratchBytes = 64L << 20;  // the largest workspace it carves
constexpr long kScratchAlign = 256;        // every carved buffer starts on 256 B
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

pthread_mutex_t g_scratch_mutex = PTHREAD_MUTEX_INITIALIZER;
void *g_scratch_address[kMaxDevices] = {};

// Bytes of the workspace for `tokens` tokens, each buffer rounded up to
// kScratchAlign; sizes[] receives the unrounded sizes.
long carved_bytes(const cfmoe_dims *dims, int tokens, int64_t *sizes) {
  cfmoe_workspace_sizes(dims, tokens, sizes, kWorkspaceBuffers);
  long total = 0;
  for (int i = 0; i < kWorkspaceBuffers; ++i)
    total += (sizes[i] + kScratchAlign - 1) / kScratchAlign * kScratchAlign;
  return total;
}

// The device address of `scratch` on `device` (the current device).
int scratch_address(int device, unsigned char **address) {
  if (device < 0 || device >= kMaxDevices) return fail(CFMOE_EINVAL, "device index out of range");
  pthread_mutex_lock(&g_scratch_mutex);
  int rc = 0;
  if (!g_scratch_address[device]) {
    void *found = nullptr;
    const hipError_t status = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
    if (status != hipSuccess || !found) {
      snprintf(g_error, sizeof(g_error), "hipGetSymbolAddress(scratch) failed: %s",
               hipGetErrorString(status));
      rc = CFMOE_EHIP;
    } else {
      g_scratch_address[device] = found;
    }
  }
  if (!rc) *address = static_cast<unsigned char *>(g_scratch_address[device]);
  pthread_mutex_unlock(&g_scratch_mutex);
  return rc;
}

}  // namespace cfmoe

extern "C" {

using namespace cfmoe;

int64_t cfmoe_noalloc_scratch_bytes(void) { return kScratchBytes; }

int cfmoe_forward_noalloc(const cfmoe_dims *dims, const cfmoe_weights *weights,
                          const void *hidden, const void *router_ids,
                          const void *router_weights, const uint8_t *padding, void *out,
                          int32_t tokens, double *read_work, const double *charges,
                          cfmoe_stream stream) {
  if (int rc = validate(dims)) return rc;
  if (tokens < 1) return fail(CFMOE_EINVAL, "tokens out of range");
  if ((dims->flags & CFMOE_ACCOUNT) && !read_work)
    return fail(CFMOE_EINVAL, "CFMOE_ACCOUNT needs read_work");
  // the size check is host arithmetic only: nothing is touched on a device
  int64_t sizes[kWorkspaceBuffers];
  const long need = carved_bytes(dims, tokens, sizes);
  if (need > kScratchBytes) {
    snprintf(g_error, sizeof(g_error),
             "the call needs %ld workspace bytes; the allocation-free entry point holds %ld "
             "(use cfmoe_forward with a caller workspace)",
             need, kScratchBytes);
    return CFMOE_EINVAL;
  }
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return fail(CFMOE_EHIP, "hipGetDevice failed");
  if (stream) {
    hipDevice_t stream_device = 0;
    if (hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &stream_device) != hipSuccess)
      return fail(CFMOE_EHIP, "hipStreamGetDevice failed");
    if (stream_device != device)
      return fail(CFMOE_EINVAL, "the stream is not on the current device");
  }
  unsigned char *base = nullptr;
  if (int rc = scratch_address(device, &base)) return rc;
  // carve the buffers in struct order
  cfmoe_workspace ws;
  memset(&ws, 0, sizeof(ws));
  ws.capacity = tokens;
  void **slots[kWorkspaceBuffers] = {
      reinterpret_cast<void **>(&ws.ids), reinterpret_cast<void **>(&ws.weights),
      reinterpret_cast<void **>(&ws.planes), reinterpret_cast<void **>(&ws.coordinates),
      reinterpret_cast<void **>(&ws.qvals), reinterpret_cast<void **>(&ws.qexp),
      reinterpret_cast<void **>(&ws.qsums), reinterpret_cast<void **>(&ws.norm2),
      reinterpret_cast<void **>(&ws.partial), reinterpret_cast<void **>(&ws.variances),
      reinterpret_cast<void **>(&ws.scores), reinterpret_cast<void **>(&ws.next_ids),
      reinterpret_cast<void **>(&ws.selected), reinterpret_cast<void **>(&ws.completed),
      reinterpret_cast<void **>(&ws.activations), reinterpret_cast<void **>(&ws.starts),
      reinterpret_cast<void **>(&ws.counts), reinterpret_cast<void **>(&ws.tile_starts),
      reinterpret_cast<void **>(&ws.down_tile_starts),
      reinterpret_cast<void **>(&ws.down_parts), reinterpret_cast<void **>(&ws.encoder_parts),
      reinterpret_cast<void **>(&ws.latent), reinterpret_cast<void **>(&ws.group_experts),
      reinterpret_cast<void **>(&ws.group_starts), reinterpret_cast<void **>(&ws.group_counts),
      reinterpret_cast<void **>(&ws.group_pairs), reinterpret_cast<void **>(&ws.group_total),
      reinterpret_cast<void **>(&ws.pair_tiles), reinterpret_cast<void **>(&ws.tile_masks),
      reinterpret_cast<void **>(&ws.down_order), reinterpret_cast<void **>(&ws.digits),
  };
  long offset = 0;
  for (int i = 0; i < kWorkspaceBuffers; ++i) {
    *slots[i] = sizes[i] > 0 ? static_cast<void *>(base + offset) : nullptr;
    offset += (sizes[i] + kScratchAlign - 1) / kScratchAlign * kScratchAlign;
  }
  ws.read_work = read_work;
  return run_stages(~0u, dims, weights, &ws, hidden, router_ids, router_weights, padding, out,
                    tokens, charges, stream);
}

}  // extern "C"

/*
 * CPU oracle of the sparse expert reader -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker for the HIP reader: only tests/, the smoke entry
 * and the bench's CPU-baseline leg load it. The product path never calls it.
 *
 * It restates the reference reader (calibration_free_moe/reader/progressive.py
 * of AidenGeunGeun/calibration-free-moe) stage by stage, with every FP32
 * rounding point fixed, so the HIP kernels can be held to it bit for bit:
 *
 *   route      progressive.py:349-386   sort K ids ascending, carry weights
 *   rotate     progressive.py:389-453   signs, 7 butterflies, x 1/sqrt(128),
 *              sketch.py:38-68          top-KEEP |v| mask, ties to lower coords
 *   screen     progressive.py:478-1108  per block: sum over kept coordinates of
 *                                       trit * x; per row: sum over blocks of
 *                                       scale * dot (FP32, fixed split order)
 *   score      progressive.py:1274-1353 point score / five-node Gauss-Hermite
 *   select     progressive.py:1584-1775 top-F by uint32 key of score + 0, ties
 *                                       by ascending candidate id
 *   exact      progressive.py:1510-1546 native gate/up dots, BF16 activation
 *   down       progressive.py:1778-1856 selected channels' down rows
 *   encode     progressive.py:1859-2016 skipped channels into the latent
 *   output     progressive.py:2019-2111 router mix + decoder correction
 *
 * Arithmetic contract shared with the HIP kernels (both sides follow it):
 *  - Screen dot of block b: the kept values v_p are put on a 21-bit grid
 *    relative to the block maximum m (frexp(m) = (f, e), q_p = rint(v_p *
 *    2^(20 - e)), |q_p| <= 2^20) and sum_p trit_p * q_p is formed EXACTLY in
 *    integers, then dot = ldexp((float)sum, e - 20). Any order or grouping of
 *    the integer sum gives the same dot.
 *  - Row estimate: SPLITS = min(8, B) block ranges of ceil(B / SPLITS)
 *    blocks; part_s = fma chain of (dot_b, scale_b) over its blocks from 0;
 *    estimate = ((part_0 + part_1) + part_2) + ...
 *  - exp(x): Cody-Waite reduction with a two-part ln 2 and a degree-7 Taylor
 *    polynomial in Horner form (fmaf), scaled by ldexpf; sigmoid(x) =
 *    1 / (1 + exp(-x)) with IEEE division.
 *  - Exact dot of a native row: 64 lane partials (lane l takes coordinates
 *    512 j + 8 l + i in (j, i) order) then a pairwise tree over lane ids.
 *  - Down: each slot's selected channels in ascending order, in tiles of 32;
 *    fma chain per tile, tiles summed in order, BF16 per slot.
 *  - Encode: skipped channels in 64-channel tiles; fma chain per tile; tiles
 *    summed in order; BF16 per slot; latent = fma chain over slots.
 *  - Output: routed = fma chain over slots of (bf16 slot sum, weight);
 *    correction = bf16(fma chain over r of U[o, r] * bf16(latent_r));
 *    out = bf16(routed + correction).
 *
 * Build: see oracle/Makefile (-O2 -ffp-contract=off, no fast-math, OpenMP).
 *
 * Threads: the `threads` argument of the heavy stages splits independent
 * outputs (rows, kept channels, output columns, candidates) over OpenMP
 * threads; every output is still computed by one thread in the order above,
 * so the results do not depend on the thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* scalar helpers                                                      */

static float bf16_to_float(uint16_t h) {
  uint32_t bits = (uint32_t)h << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static uint16_t float_to_bf16(float f) {
  uint32_t bits;
  memcpy(&bits, &f, 4);
  if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x40u);
  bits += 0x7fffu + ((bits >> 16) & 1u);
  return (uint16_t)(bits >> 16);
}

static float bf16_round(float f) { return bf16_to_float(float_to_bf16(f)); }

static float half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exponent = (h >> 10) & 0x1fu;
  uint32_t mantissa = h & 0x3ffu;
  uint32_t bits;
  if (exponent == 0) {
    if (mantissa == 0) {
      bits = sign;
    } else {
      /* subnormal half: value = mantissa * 2^-24, exact in float */
      float value = ldexpf((float)mantissa, -24);
      memcpy(&bits, &value, 4);
      bits |= sign;
    }
  } else if (exponent == 31) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else {
    bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static uint32_t float_bits(float f) {
  uint32_t bits;
  memcpy(&bits, &f, 4);
  return bits;
}

/* exp(x) by Cody-Waite reduction x = n ln2 + r, |r| <= ln2 / 2, and the
 * degree-7 Taylor polynomial of e^r (truncation < 6e-9 relative). */
float orc_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.972084045410156f) return 0.0f;
  float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.428606765330187045e-06f, r);
  float p = 1.98412698412698413e-04f;     /* 1/5040 */
  p = fmaf(p, r, 1.38888888888888889e-03f); /* 1/720 */
  p = fmaf(p, r, 8.33333333333333333e-03f); /* 1/120 */
  p = fmaf(p, r, 4.16666666666666667e-02f); /* 1/24 */
  p = fmaf(p, r, 1.66666666666666667e-01f); /* 1/6 */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

float orc_sigmoid(float x) { return 1.0f / (1.0f + orc_expf(-x)); }

/* phi(g): SiLU g * sigmoid(g), or tanh-GELU g * sigmoid(1.59577 (g + 0.044715 g^3))
 * (progressive.py:1265-1271). */
float orc_activate(float g, int gelu) {
  if (gelu) {
    float cube = ((0.044715f * g) * g) * g;
    float inner = 1.5957691216057308f * (g + cube);
    return g * orc_sigmoid(inner);
  }
  return g * orc_sigmoid(g);
}

/* ------------------------------------------------------------------ */
/* layout helpers                                                       */

int orc_code_stride(int rows) {
  int useful = 2 * ((rows / 2 + 4) / 5);
  return (useful + 15) / 16 * 16;
}

long orc_storage_bytes(int rows, int hidden) {
  int stride = orc_code_stride(rows);
  int blocks = hidden / 128;
  int body = stride - stride % 32, tail = stride % 32;
  return (long)blocks * 128 * body + (long)((blocks + 1) / 2) * 128 * 2 * tail;
}

/* Byte offset (within one expert) of code byte `byte` of coordinate `coord`
 * (0..127) of rotation block `block` (sketch.py:84-150 layout). */
static long code_offset(int blocks, int stride, int block, int coord, int byte) {
  int body = stride - stride % 32;
  if (byte < body) return ((long)block * 128 + coord) * body + byte;
  return (long)blocks * 128 * body + ((long)(block / 2) * 128 + coord) * 32 +
         (block % 2) * 16 + (byte - body);
}

/* Trit of row `row` (gate rows [0, I), up rows [I, 2I)) at one coordinate. */
static int decode_trit(const uint8_t *codes, int I, int blocks, int stride, int row,
                       int block, int coord) {
  int channel = row % I;
  int byte = 2 * (channel / 5) + row / I;
  int value = codes[code_offset(blocks, stride, block, coord, byte)];
  static const int power[5] = {1, 3, 9, 27, 81};
  return (value / power[channel % 5]) % 3 - 1;
}

/* ------------------------------------------------------------------ */
/* route: progressive.py:349-386                                        */

void orc_route(int T, int K, int E, const int64_t *router_ids, const float *router_weights,
               const uint8_t *padding, int32_t *ids, float *weights) {
  for (int t = 0; t < T; ++t) {
    int active = padding ? !padding[t] : 1;
    int32_t original[64];
    int32_t ordered[64];
    for (int k = 0; k < K; ++k) {
      int64_t id = router_ids[t * K + k];
      /* an id outside [0, E) names no local expert */
      original[k] = ordered[k] = (id < 0 || id >= E) ? -1 : (int32_t)id;
    }
    /* insertion sort, ascending */
    for (int a = 1; a < K; ++a) {
      int32_t v = ordered[a];
      int b = a - 1;
      while (b >= 0 && ordered[b] > v) { ordered[b + 1] = ordered[b]; --b; }
      ordered[b + 1] = v;
    }
    for (int k = 0; k < K; ++k) {
      float w = 0.0f;
      for (int j = 0; j < K; ++j)
        if (original[j] == ordered[k]) w += active ? router_weights[t * K + j] : 0.0f;
      ids[t * K + k] = ordered[k];
      weights[t * K + k] = w;
    }
  }
}

/* ------------------------------------------------------------------ */
/* rotate + mask + quantise: progressive.py:389-453, sketch.py:38-68     */

/* planes/coords: [T, B, keep]; qvals: [T, B, keep]; qexp, norm2: [T, B] */
void orc_rotate(int T, int H, int keep, const uint16_t *x, const int8_t *signs,
                const uint8_t *padding, float *planes, int32_t *coords, int32_t *qvals,
                int32_t *qexp, float *norm2) {
  int B = H / 128;
  for (int t = 0; t < T; ++t) {
    int active = padding ? !padding[t] : 1;
    for (int b = 0; b < B; ++b) {
      float v[128];
      for (int c = 0; c < 128; ++c) {
        float xv = active ? bf16_to_float(x[(long)t * H + b * 128 + c]) : 0.0f;
        v[c] = xv * (float)signs[b * 128 + c];
      }
      for (int stage = 0; stage < 7; ++stage) {
        int bit = 1 << stage;
        for (int c = 0; c < 128; ++c) {
          if (c & bit) continue;
          float left = v[c], right = v[c | bit];
          v[c] = left + right;
          v[c | bit] = left - right;
        }
      }
      for (int c = 0; c < 128; ++c) v[c] = v[c] * 0.08838834764831845f;
      /* top-keep magnitudes, ties to lower coordinates */
      int kept[128];
      if (keep >= 128) {
        for (int c = 0; c < 128; ++c) kept[c] = 1;
      } else {
        for (int c = 0; c < 128; ++c) {
          uint32_t mc = float_bits(v[c]) & 0x7fffffffu;
          int rank = 0;
          for (int d = 0; d < 128; ++d) {
            uint32_t md = float_bits(v[d]) & 0x7fffffffu;
            if (md > mc || (md == mc && d < c)) ++rank;
          }
          kept[c] = rank < keep;
        }
      }
      long cell = (long)t * B + b;
      int p = 0;
      float compact[128];
      for (int c = 0; c < 128; ++c) {
        if (!kept[c]) continue;
        compact[p] = v[c];
        planes[cell * keep + p] = v[c];
        if (coords) coords[cell * keep + p] = c;
        ++p;
      }
      /* squared norm: lane l of 64 holds positions l and l + 64, then a
       * pairwise tree over lanes */
      float lane[64];
      for (int l = 0; l < 64; ++l) {
        float a = l < keep ? compact[l] * compact[l] : 0.0f;
        if (l + 64 < keep) a = fmaf(compact[l + 64], compact[l + 64], a);
        lane[l] = a;
      }
      for (int m = 1; m < 64; m <<= 1)
        for (int l = 0; l < 64; ++l)
          if (!(l & m)) {
            float s = lane[l] + lane[l | m];
            lane[l] = s;
            lane[l | m] = s;
          }
      norm2[cell] = lane[0];
      /* 21-bit grid relative to the block maximum */
      uint32_t peak = 0;
      for (int q = 0; q < keep; ++q) {
        uint32_t mag = float_bits(compact[q]) & 0x7fffffffu;
        if (mag > peak) peak = mag;
      }
      int exponent = 0;
      if (peak != 0) {
        float m;
        uint32_t bits = peak;
        memcpy(&m, &bits, 4);
        frexpf(m, &exponent);
      }
      int shift = peak ? 20 - exponent : 0;
      qexp[cell] = shift;
      for (int q = 0; q < keep; ++q)
        qvals[cell * keep + q] = peak ? (int32_t)rintf(ldexpf(compact[q], shift)) : 0;
    }
  }
}

/* ------------------------------------------------------------------ */
/* screen: progressive.py:478-1108 (per-token) and :2428-2606 (grouped)  */

/* partial, variances: [T, 2, N]; ids [T, K] (local, -1 = absent);
 * stats: [E][B][2][2I] fp16 bits (physical). variances may be NULL. */
void orc_screen(int T, int H, int I, int K, int keep, const uint8_t *codes,
                const uint16_t *stats, const int32_t *coords, const int32_t *qvals,
                const int32_t *qexp, const float *norm2, const int32_t *ids,
                const uint8_t *padding, float *partial, float *variances, int threads) {
  int B = H / 128, N = K * I, rows = 2 * I;
  int stride = orc_code_stride(rows);
  long storage = orc_storage_bytes(rows, H);
  int splits = B < 8 ? B : 8;
  int span = (B + splits - 1) / splits;
  for (int t = 0; t < T; ++t) {
    int active = padding ? !padding[t] : 1;
    for (int k = 0; k < K; ++k) {
      int e = ids[t * K + k];
      int local = active && e >= 0;
      const uint8_t *ec = local ? codes + (long)e * storage : NULL;
#pragma omp parallel for schedule(static) num_threads(threads)
      for (int r = 0; r < rows; ++r) {
        float estimate = 0.0f, variance = 0.0f;
        for (int s = 0; s < splits; ++s) {
          float part = 0.0f, vpart = 0.0f;
          for (int b = s * span; b < (s + 1) * span && b < B; ++b) {
            long cell = (long)t * B + b;
            /* exact integer block dot on the grid, then one rounding */
            int64_t sum = 0;
            if (local)
              for (int p = 0; p < keep; ++p) {
                int coord = keep >= 128 ? p : coords[cell * keep + p];
                sum += (int64_t)decode_trit(ec, I, B, stride, r, b, coord) * qvals[cell * keep + p];
              }
            float dot = ldexpf((float)(int32_t)sum, -qexp[cell]);
            if (local) {
              const uint16_t *plane = stats + (((long)e * B + b) * 2) * rows;
              part = fmaf(dot, half_to_float(plane[r]), part);
              vpart = fmaf(half_to_float(plane[rows + r]), norm2[cell], vpart);
            }
          }
          estimate = s == 0 ? part : estimate + part;
          variance = s == 0 ? vpart : variance + vpart;
        }
        int half = r / I, channel = r % I;
        long address = ((long)t * 2 + half) * N + (long)k * I + channel;
        partial[address] = estimate;
        if (variances) variances[address] = variance;
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* score: progressive.py:1274-1353                                      */

static const float GH_NODES[5] = {-2.8569700138728056f, -1.355626179974266f, 0.0f,
                                  1.355626179974266f, 2.8569700138728056f};
static const float GH_WEIGHTS[5] = {0.011257411327720693f, 0.2220759220056126f,
                                    0.5333333333333333f, 0.2220759220056126f,
                                    0.011257411327720693f};

float orc_score_one(float gate, float up, float gate_variance, float up_variance,
                    float norm, float weight, float alpha, float beta, int gelu,
                    int point) {
  float g = bf16_round(gate);
  float u = bf16_round(up);
  float risk;
  if (point) {
    float value = norm * (orc_activate(g, gelu) * u);
    risk = value * value;
  } else {
    float sg = sqrtf(gate_variance);
    float su = sqrtf(up_variance);
    float spread = su * su;
    float second = fmaf(u, u, spread);
    float energy = 0.0f, first = 0.0f, paid = 0.0f;
    for (int j = 0; j < 5; ++j) {
      float a = orc_activate(fmaf(GH_NODES[j], sg, g), gelu);
      float weighted = GH_WEIGHTS[j] * a;
      energy = fmaf(weighted * a, second, energy);
      first = fmaf(weighted, u, first);
      if (j == 2) paid = bf16_round(a * u);
    }
    float parallel = norm * first - alpha * paid;
    float perpendicular = beta * paid;
    float excess = energy - first * first;
    if (!(excess > 0.0f)) excess = 0.0f;
    risk = ((norm * norm) * excess + parallel * parallel) + perpendicular * perpendicular;
  }
  return (risk * weight) * weight;
}

/* scores [T, N]; norms [E, I]; geometry [E, I, 2] or NULL */
void orc_score(int T, int I, int K, const float *partial, const float *variances,
               const int32_t *ids, const float *weights, const uint8_t *padding,
               const float *norms, const float *geometry, int gelu, int point,
               float *scores) {
  int N = K * I;
  for (int t = 0; t < T; ++t) {
    int active = padding ? !padding[t] : 1;
    for (int k = 0; k < K; ++k) {
      int e = ids[t * K + k];
      int local = active && e >= 0;
      float w = weights[t * K + k];
      for (int c = 0; c < I; ++c) {
        long logical = (long)k * I + c;
        float g = partial[((long)t * 2) * N + logical];
        float u = partial[((long)t * 2 + 1) * N + logical];
        float vg = variances ? variances[((long)t * 2) * N + logical] : 0.0f;
        float vu = variances ? variances[((long)t * 2 + 1) * N + logical] : 0.0f;
        float n = local ? norms[(long)e * I + c] : 0.0f;
        float alpha = (local && geometry) ? geometry[((long)e * I + c) * 2] : 0.0f;
        float beta = (local && geometry) ? geometry[((long)e * I + c) * 2 + 1] : 0.0f;
        scores[(long)t * N + logical] =
            orc_score_one(g, u, vg, vu, n, w, alpha, beta, gelu, point);
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* select: progressive.py:1584-1775                                     */

/* next_ids [T, F] (padded with -1 under a threshold); selected [T, N];
 * counts/starts/tile_starts [T, K]; tile = 128 channels for tile_starts. */
void orc_select(int T, int N, int F, int I, int K, const float *scores, int thresholded,
                float threshold, int32_t *next_ids, uint8_t *selected, int32_t *counts,
                int32_t *starts, int32_t *tile_starts) {
  uint32_t *keys = malloc(sizeof(uint32_t) * N);
  for (int t = 0; t < T; ++t) {
    for (int i = 0; i < N; ++i) keys[i] = float_bits(scores[(long)t * N + i] + 0.0f);
    int want = F;
    uint32_t cutoff;
    long above = 0, tied = 0;
    if (thresholded) {
      uint32_t bound = float_bits(threshold + 0.0f);
      long passing = 0;
      for (int i = 0; i < N; ++i) passing += keys[i] >= bound;
      if (passing < want) want = (int)passing;
    }
    /* the want-th largest key (binary search over the 32-bit keys) */
    if (want == 0) {
      cutoff = 0xffffffffu;
    } else {
      uint32_t low = 0, high = 0xffffffffu;
      while (low < high) {
        uint32_t middle = low + (uint32_t)(((uint64_t)high - low + 1) / 2);
        long count = 0;
        for (int i = 0; i < N; ++i) count += keys[i] >= middle;
        if (count >= want) low = middle; else high = middle - 1;
      }
      cutoff = low;
    }
    for (int i = 0; i < N; ++i) above += keys[i] > cutoff;
    long room = want - above;
    int position = 0;
    for (int k = 0; k < K; ++k) counts[t * K + k] = 0;
    for (int i = 0; i < N; ++i) {
      int keep = 0;
      if (want > 0) {
        if (keys[i] > cutoff) keep = 1;
        else if (keys[i] == cutoff && tied < room) { keep = 1; ++tied; }
      }
      selected[(long)t * N + i] = (uint8_t)keep;
      if (keep) {
        next_ids[(long)t * F + position++] = i;
        counts[t * K + i / I] += 1;
      }
    }
    for (; position < F; ++position) next_ids[(long)t * F + position] = -1;
    int start = 0, tile = 0;
    for (int k = 0; k < K; ++k) {
      starts[t * K + k] = start;
      tile_starts[t * K + k] = tile;
      start += counts[t * K + k];
      tile += (counts[t * K + k] + 127) / 128;
    }
  }
  free(keys);
}

/* ------------------------------------------------------------------ */
/* exact computation: progressive.py:1510-1546                          */

float orc_row_dot(int H, const uint16_t *row, const uint16_t *x) {
  float lane[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int j = 0; j * 512 < H; ++j)
      for (int i = 0; i < 8; ++i) {
        int h = 512 * j + 8 * l + i;
        if (h < H) acc = fmaf(bf16_to_float(row[h]), bf16_to_float(x[h]), acc);
      }
    lane[l] = acc;
  }
  for (int m = 1; m < 64; m <<= 1)
    for (int l = 0; l < 64; ++l)
      if (!(l & m)) {
        float s = lane[l] + lane[l | m];
        lane[l] = s;
        lane[l | m] = s;
      }
  return lane[0];
}

/* gate_up [E, 2I, H] bf16; x [T, H] bf16; partial [T, 2, N] (selected rows are
 * overwritten with exact projections); activations [T, N] bf16 bits;
 * completed [T, N]. */
void orc_exact(int T, int H, int I, int K, int F, const uint16_t *gate_up,
               const uint16_t *x, const int32_t *ids, const uint8_t *padding,
               const int32_t *next_ids, int gelu, float *partial,
               uint16_t *activations, uint8_t *completed, int threads) {
  int N = K * I;
  uint16_t *zero = calloc((size_t)H, sizeof(uint16_t));
  for (int t = 0; t < T; ++t) {
    int active = padding ? !padding[t] : 1;
    memset(completed + (long)t * N, 0, N);
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads)
    for (int f = 0; f < F; ++f) {
      int logical = next_ids[(long)t * F + f];
      if (logical < 0) continue; /* the -1 padding of a thresholded list */
      int k = logical / I, c = logical % I;
      int e = ids[t * K + k];
      float g = 0.0f, u = 0.0f;
      if (e >= 0) {
        const uint16_t *xr = active ? x + (long)t * H : zero;
        g = orc_row_dot(H, gate_up + ((long)e * 2 * I + c) * H, xr);
        u = orc_row_dot(H, gate_up + ((long)e * 2 * I + I + c) * H, xr);
      }
      partial[((long)t * 2) * N + logical] = g;
      partial[((long)t * 2 + 1) * N + logical] = u;
      float act = bf16_round(orc_activate(bf16_round(g), gelu));
      activations[(long)t * N + logical] = float_to_bf16(act * bf16_round(u));
      completed[(long)t * N + logical] = 1;
    }
  }
  free(zero);
}

/* ------------------------------------------------------------------ */
/* down: progressive.py:1778-1856; values [T, K, H] (BF16-rounded sums)  */

#define DOWN_TILE 32 /* selected channels per tile (the reference tiles 128) */

void orc_down(int T, int H, int I, int K, int F, const uint16_t *down,
              const uint16_t *activations, const int32_t *ids, const uint8_t *padding,
              const int32_t *next_ids, const int32_t *counts, const int32_t *starts,
              float *values, int threads) {
  int N = K * I;
  for (int t = 0; t < T; ++t) {
    int active = padding ? !padding[t] : 1;
    for (int k = 0; k < K; ++k) {
      int e = ids[t * K + k];
      int count = counts[t * K + k], start = starts[t * K + k];
      /* output columns in chunks of 64, one thread each */
#pragma omp parallel for schedule(static) num_threads(threads)
      for (int o0 = 0; o0 < H; o0 += 64) {
        int o1 = o0 + 64 < H ? o0 + 64 : H;
        float total[64], tile[64];
        for (int o = o0; o < o1; ++o) total[o - o0] = 0.0f;
        for (int begin = 0; begin < count; begin += DOWN_TILE) {
          for (int o = o0; o < o1; ++o) tile[o - o0] = 0.0f;
          for (int j = begin; j < begin + DOWN_TILE && j < count; ++j) {
            int logical = next_ids[(long)t * F + start + j];
            int c = logical % I;
            float a = bf16_to_float(activations[(long)t * N + logical]);
            const uint16_t *row = down + ((long)e * I + c) * H;
            for (int o = o0; o < o1; ++o) {
              float d = (active && e >= 0) ? bf16_to_float(row[o]) : 0.0f;
              tile[o - o0] = fmaf(d, a, tile[o - o0]);
            }
          }
          for (int o = o0; o < o1; ++o)
            total[o - o0] = begin == 0 ? tile[o - o0] : total[o - o0] + tile[o - o0];
        }
        for (int o = o0; o < o1; ++o) values[((long)t * K + k) * H + o] = bf16_round(total[o - o0]);
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* encode + latent: progressive.py:1859-2016; encoder_t [E, I, R] bf16   */

void orc_encode(int T, int I, int K, int R, const uint16_t *encoder_t,
                const float *partial, const uint16_t *activations,
                const uint8_t *completed, const uint8_t *selected, const int32_t *ids,
                const float *weights, const uint8_t *padding, int gelu, float *latent) {
  int N = K * I;
  float total[256], tile[256];
  for (int t = 0; t < T; ++t) {
    int active = padding ? !padding[t] : 1;
    for (int r = 0; r < R; ++r) latent[(long)t * R + r] = 0.0f;
    for (int k = 0; k < K; ++k) {
      int e = ids[t * K + k];
      int local = active && e >= 0;
      for (int r = 0; r < R; ++r) total[r] = 0.0f;
      for (int begin = 0; begin < I; begin += 64) {
        for (int r = 0; r < R; ++r) tile[r] = 0.0f;
        for (int c = begin; c < begin + 64 && c < I; ++c) {
          long logical = (long)t * N + (long)k * I + c;
          if (selected[logical]) continue;
          float value;
          if (completed[logical]) {
            value = bf16_to_float(activations[logical]);
          } else {
            float g = bf16_round(partial[(long)t * 2 * N + (long)k * I + c]);
            float u = bf16_round(partial[(long)t * 2 * N + N + (long)k * I + c]);
            value = bf16_round(orc_activate(g, gelu) * u);
          }
          const uint16_t *row = encoder_t + ((long)(local ? e : 0) * I + c) * R;
          for (int r = 0; r < R; ++r) {
            float coefficient = local ? bf16_to_float(row[r]) : 0.0f;
            tile[r] = fmaf(value, coefficient, tile[r]);
          }
        }
        for (int r = 0; r < R; ++r) total[r] = begin == 0 ? tile[r] : total[r] + tile[r];
      }
      float w = weights[t * K + k];
      for (int r = 0; r < R; ++r)
        latent[(long)t * R + r] = fmaf(bf16_round(total[r]), w, latent[(long)t * R + r]);
    }
  }
}

/* ------------------------------------------------------------------ */
/* output: progressive.py:2019-2111; decoder [H, R] bf16 or NULL         */

void orc_output(int T, int H, int K, int R, const float *values, const float *weights,
                const float *latent, const uint16_t *decoder, const uint8_t *padding,
                uint16_t *out) {
  for (int t = 0; t < T; ++t) {
    int active = padding ? !padding[t] : 1;
    for (int o = 0; o < H; ++o) {
      float routed = 0.0f;
      for (int k = 0; k < K; ++k)
        routed = fmaf(values[((long)t * K + k) * H + o], weights[t * K + k], routed);
      float correction = 0.0f;
      if (decoder && R > 0) {
        float acc = 0.0f;
        for (int r = 0; r < R; ++r) {
          float u = active ? bf16_to_float(decoder[(long)o * R + r]) : 0.0f;
          acc = fmaf(u, bf16_round(latent[(long)t * R + r]), acc);
        }
        correction = bf16_round(acc);
      }
      out[(long)t * H + o] = float_to_bf16(routed + correction);
    }
  }
}

/*
 * C ABI of the MI355X sparse expert reader (libcfmoe_reader.so).
 *
 * Plain C: device pointers and sizes only, no framework types. Every call is
 * stream-ordered on the given HIP stream, never synchronises the host, never
 * allocates and never frees, so a caller may capture it in a HIP graph. The
 * caller owns every buffer (weights, workspace, inputs, outputs).
 *
 * It replaces the Triton launches of the reference operator
 * calibration_free_moe/reader/progressive.py (AidenGeunGeun/
 * calibration-free-moe): ProgressiveReader.__call__ (progressive.py:3876-4472)
 * maps to cfmoe_forward and ProgressiveReader.prepare_input
 * (progressive.py:3829-3873) to cfmoe_prepare_input. The Python operator
 * (calibration_free_moe/reader/progressive.py in this package) keeps the
 * reference's constructor, call signature, attributes and report() and calls
 * these entry points through ctypes.
 *
 * Return value: 0 on success; otherwise a nonzero code and a message readable
 * through cfmoe_last_error() (thread-local). Contract violations that the
 * Python layer already rejects with ValueError return CFMOE_EINVAL here.
 */
#ifndef CFMOE_READER_H
#define CFMOE_READER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define CFMOE_API __attribute__((visibility("default")))
#else
#define CFMOE_API
#endif

typedef struct ihipStream_t *cfmoe_stream;

#define CFMOE_ABI_VERSION 10

/* cfmoe_dims.flags */
#define CFMOE_POINT 1u          /* point score (else five-node Gauss-Hermite) */
#define CFMOE_GELU 2u           /* tanh-GELU gate activation (else SiLU) */
#define CFMOE_GEOMETRY 4u       /* recovery geometry (alpha, beta) is read */
#define CFMOE_THRESHOLD 8u      /* keep scores >= *threshold, at most F */
#define CFMOE_ACCOUNT 16u       /* add the call's read statistics to read_work */
#define CFMOE_IDS_INT64 32u     /* router ids are int64 (else int32) */
#define CFMOE_WEIGHTS_BF16 64u  /* router weights are bf16 (else fp32) */
#define CFMOE_INPUT_PREPARED 128u /* cfmoe_prepare_input already rotated */

/* Stages of one call, in launch order (cfmoe_launch_stage). */
#define CFMOE_STAGE_PREPARE 0 /* route, rotate, mask, grid quantisation */
#define CFMOE_STAGE_SCREEN 1  /* sketch projections and the channel scores */
#define CFMOE_STAGE_SCORE 2   /* split sums and channel scores (launches nothing: the
                                 screen launch scores) */
#define CFMOE_STAGE_SELECT 3  /* per-token top-F */
#define CFMOE_STAGE_EXACT 4   /* native gate/up rows of kept channels (and at rank 32 the
                                 encoder) */
#define CFMOE_STAGE_ENCODE 5  /* recovery encoder over skipped channels; at rank 32 it
                                 runs inside the exact launch, and this stage launches
                                 nothing */
#define CFMOE_STAGE_DOWN 6    /* down rows of kept channels */
#define CFMOE_STAGE_OUTPUT 7  /* latent, decoder correction, router mix */
#define CFMOE_STAGE_COUNT 8

#define CFMOE_EINVAL 1
#define CFMOE_EHIP 2

/* Layer and plan dimensions (progressive.py:3133-3515 validates the same). */
typedef struct cfmoe_dims {
  int32_t hidden;      /* H, multiple of 128 */
  int32_t width;       /* I, multiple of 16 */
  int32_t top_k;       /* K <= 64; tokens * K <= 8192 per call */
  int32_t experts;     /* E local experts */
  int32_t rank;        /* R recovery rank, 0 = no recovery map, <= 64 */
  int32_t final_count; /* F, channels kept per token */
  int32_t keep;        /* rotated coordinates kept per 128-block (1..128) */
  uint32_t flags;
  int32_t grouped_tokens; /* calls of at least this many tokens compute the kept
                             channels expert-major (one read of each union row
                             per tile of <= 16 pairs); 0 = the default, 16;
                             otherwise at least 2 (1 is refused: EINVAL) */
} cfmoe_dims;

/* Resident per-layer tensors. The reader borrows them; none is written. */
typedef struct cfmoe_weights {
  const void *gate_up;     /* bf16 [E, 2I, H] */
  const void *down;        /* bf16, physical [E, I, H] (channel-major) */
  const uint8_t *codes;    /* unused by the forward calls (may be NULL): the screen reads
                              trit_planes, which cfmoe_pack_trit_planes builds from the codes */
  const void *statistics;  /* fp16, physical [E, H/128, 2, 2I] */
  const float *norms;      /* [E, I] down-column L2 norms */
  const float *geometry;   /* [E, I, 2] (alpha, beta) or NULL */
  const void *encoder_t;   /* bf16 [E, I, R] or NULL */
  const void *decoder;     /* bf16 [H, R] or NULL */
  const int8_t *signs;     /* [H] rotation signs */
  const float *threshold;  /* [1] selection threshold or NULL */
  const uint32_t *trit_planes; /* screen layout of `codes` (cfmoe_pack_trit_planes) */
  const void *encoder_tiles;   /* bf16 [E, ceil(I/64), R, 64]: encoder_t tile-major, channels past
                                  I zero; required at R == 32 (the exact launch's encoder), else
                                  unused */
} cfmoe_weights;

/* Caller-allocated scratch, sized for `capacity` tokens (sizes in bytes from
 * cfmoe_workspace_sizes). Layouts match the reference workspace
 * (progressive.py:2868-3121) where the Python operator exposes them. Every
 * buffer is 16-byte aligned (checked for the projections, variances, scores,
 * digits and norms, which take 16-byte accesses). */
typedef struct cfmoe_workspace {
  int32_t capacity;
  int32_t *ids;               /* [cap, K] sorted local expert ids */
  float *weights;             /* [cap, K] router weights in id order */
  float *planes;              /* [cap, B, keep] kept rotated values */
  int32_t *coordinates;       /* [cap, B, keep] their coordinates */
  int32_t *qvals;             /* [cap, B, keep] values on the 21-bit grid */
  int32_t *qexp;              /* [cap, B] grid exponents */
  int32_t *qsums;             /* [cap, B] sums of the kept grid values */
  float *norm2;               /* [cap, B] squared norm of kept values */
  float *partial;             /* [cap, 2, N] gate/up projections */
  float *variances;           /* [cap, 2, N] */
  float *scores;              /* [cap, N] */
  int32_t *next_ids;          /* [cap, F] kept candidate ids, ascending */
  uint8_t *selected;          /* [cap, N] */
  uint8_t *completed;         /* [cap, N] */
  void *activations;          /* bf16 [cap, N] */
  int32_t *starts;            /* [cap, K] */
  int32_t *counts;            /* [cap, K] */
  int32_t *tile_starts;       /* [cap, K] 128-channel tiles */
  int32_t *down_tile_starts;  /* [cap, K] 32-channel tiles */
  float *down_parts;          /* [cap, ceil(F/32) + K - 1, H] */
  float *encoder_parts;       /* [cap, K, ceil(I/64), R] */
  float *latent;              /* [cap, R] */
  int32_t *group_experts;     /* [cap * K] expert of each tile of <= 16 pairs, ascending */
  int32_t *group_starts;      /* [cap * K] first slot of each tile in group_pairs (16 z) */
  int32_t *group_counts;      /* [cap * K] pairs of each tile (1..16) */
  int32_t *group_pairs;       /* [cap * K * 16] token * K + slot; tile z at 16 z .. */
  int32_t *group_total;       /* [1] number of tiles */
  int32_t *pair_tiles;        /* [cap * K] slot 16 z + p of each pair in group_pairs, or -1 */
  uint32_t *tile_masks;       /* [cap * N] per (tile, channel): bit p set if pair p kept it */
  int32_t *down_order;        /* down workgroups' items grouped by expert per XCD, then the
                                 builders' slot records (size from cfmoe_workspace_sizes) */
  int8_t *digits;             /* [cap, B, 3, 128] the kept grid values' three balanced
                                 8-bit digits per rotated coordinate (0 where not kept) */
  double *read_work;          /* [20] read statistics (progressive.py:3507-3515) */
} cfmoe_workspace;

/* Byte sizes of every workspace buffer, in struct order after `capacity`
 * (31 entries, read_work excluded). Returns the number written. */
CFMOE_API int cfmoe_workspace_sizes(const cfmoe_dims *dims, int32_t capacity, int64_t *sizes,
                          int32_t count);

/* One reader call: routed-expert output of `tokens` rows (progressive.py:
 * 3876-4472). hidden bf16 [T, H]; router_ids [T, K] int32/int64; router
 * weights [T, K] fp32/bf16; padding uint8 [T] or NULL; out bf16 [T, H].
 * With CFMOE_ACCOUNT set the call adds its read statistics to read_work
 * (progressive.py:3507-3515, :4492-4524, :2114-2317): charges[0..17] times
 * the active tokens, plus what the device counts itself -- the sketch bytes
 * the screen streams and its matrix-core MACs per tile of pairs (slots 11,
 * 15) and, for grouped calls, the gate/up rows of each tile's union of kept
 * channels (slot 12). charges may be NULL (no per-token terms). */
CFMOE_API int cfmoe_forward(const cfmoe_dims *dims, const cfmoe_weights *weights,
                  const cfmoe_workspace *workspace, const void *hidden,
                  const void *router_ids, const void *router_weights,
                  const uint8_t *padding, void *out, int32_t tokens,
                  const double *charges, cfmoe_stream stream);

/* Launch one stage of cfmoe_forward with the same arguments, reading the
 * workspace state that earlier stages left. For per-kernel timing and tests;
 * no reference counterpart (the reference launches its Triton kernels
 * individually from Python, progressive.py:3955-4471). A stage launched alone
 * runs its own kernel even where cfmoe_forward runs it in one launch with the
 * next (select and exact up to four tokens); the results are the same. */
CFMOE_API int cfmoe_launch_stage(int32_t stage, const cfmoe_dims *dims, const cfmoe_weights *weights,
                       const cfmoe_workspace *workspace, const void *hidden,
                       const void *router_ids, const void *router_weights,
                       const uint8_t *padding, void *out, int32_t tokens,
                       const double *charges, cfmoe_stream stream);

/* Bytes of the screen's trit planes for all `experts` (64 * width * hidden /
 * 128 per expert), or minus an error code. */
CFMOE_API int64_t cfmoe_trit_plane_bytes(const cfmoe_dims *dims);

/* Repack the sketch codes (the reference's five-trits-per-byte layout,
 * sketch.py:84-150, validated at progressive.py:3318-3328) into the screen's
 * resident 2-bit layout `trit_planes` (cfmoe_trit_plane_bytes bytes, 8-byte
 * aligned): digit t + 1 of every gate/up row and rotated coordinate, in the
 * order the screen's matrix-core operands are loaded. Run once per layer when
 * the reader is built (the reference reads the codes directly); no
 * counterpart call in the reference. */
CFMOE_API int cfmoe_pack_trit_planes(const cfmoe_dims *dims, const uint8_t *codes,
                                     uint32_t *trit_planes, cfmoe_stream stream);

/* The inverse of cfmoe_pack_trit_planes: write the sketch codes of all
 * `experts` ([E, sketch_storage_bytes(2I, H)], the reference's layout,
 * sketch.py:84-150) from the trit planes, 121 (five zero trits) in every byte
 * that carries no channel. The reader keeps only the planes resident and
 * rebuilds the codes when its `sketch_codes` attribute is read (the reference
 * keeps the codes themselves, progressive.py:3317); no counterpart call. */
CFMOE_API int cfmoe_unpack_trit_planes(const cfmoe_dims *dims, const uint32_t *trit_planes,
                                       uint8_t *codes, cfmoe_stream stream);

/* Build the resident ternary sketch of `experts` experts' gate/up rows
 * (bf16 [experts, 2 width, hidden], hidden a multiple of 128) on the device:
 * the reference's construction (build_sketch, sketch.py:84-150: rotation by
 * `signs` [hidden] +-1 int8 or none when NULL, TWN ternarisation per
 * 128-coordinate block, five trits per byte, body/tail byte layout) in one
 * launch instead of its per-expert torch loop. `codes` [experts,
 * sketch_storage_bytes] must hold 121 (five zero trits) in every byte before
 * the call (the kernel writes only the bytes that carry channels);
 * `statistics` is fp16 in the physical [experts, hidden / 128, 2, 2 width]
 * layout (scale plane, residual plane). */
CFMOE_API int cfmoe_build_sketch(int32_t experts, int32_t width, int32_t hidden,
                                 const void *gate_up, const int8_t *signs, uint8_t *codes,
                                 void *statistics, cfmoe_stream stream);

/* Routing-independent input rotation ahead of the router
 * (progressive.py:3829-3873). A following cfmoe_forward with
 * CFMOE_INPUT_PREPARED set skips its own rotation. */
CFMOE_API int cfmoe_prepare_input(const cfmoe_dims *dims, const cfmoe_weights *weights,
                        const cfmoe_workspace *workspace, const void *hidden,
                        const uint8_t *padding, int32_t tokens, cfmoe_stream stream);

/* Allocation-free variant of cfmoe_forward. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP-graph
 * capture, tight serving loops, hosts that forbid hipMalloc). Same arguments
 * as cfmoe_forward minus the workspace, plus the caller's read_work [20]
 * (needed only with CFMOE_ACCOUNT). The workspace is carved from one static
 * device array of cfmoe_noalloc_scratch_bytes() bytes (64 MiB) that each GPU
 * holds until the process ends; a call needing more returns CFMOE_EINVAL
 * without touching the device. It calls no allocating routine. Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (several
 * streams or threads) race. The stream must belong to the current device. */
CFMOE_API int cfmoe_forward_noalloc(const cfmoe_dims *dims, const cfmoe_weights *weights,
                                    const void *hidden, const void *router_ids,
                                    const void *router_weights, const uint8_t *padding,
                                    void *out, int32_t tokens, double *read_work,
                                    const double *charges, cfmoe_stream stream);

/* Bytes of the static device array behind cfmoe_forward_noalloc. */
CFMOE_API int64_t cfmoe_noalloc_scratch_bytes(void);

/* Thread-local message of the last failing call. */
CFMOE_API const char *cfmoe_last_error(void);

CFMOE_API int cfmoe_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif

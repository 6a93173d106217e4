/*
 * pk_palette.h - C ABI of the MI355X (gfx950) palette-weight GEMM library.
 *
 * This is the drop-in boundary for parakeet.wgsl's palette GEMM path. Every
 * entry point takes plain pointers and sizes; device pointers are HIP device
 * allocations (from pk_alloc or any other allocator on the same device) and
 * streams are hipStream_t values passed as void* (NULL = the context stream).
 *
 * Status codes follow the int-enum style of the reference's only native ABI
 * (model/native/kmeans1d_sorted_unique.h:21-47): every call returns a
 * pk_status and pk_last_error() holds the calling thread's last message.
 * PK_RANGE_ERROR marks the failures the reference raises as RangeError
 * (src/webgpu/kernels/gemm.ts:431-438, :982); PK_INVALID_ARGUMENT marks the
 * ones it raises as Error.
 *
 * Reference interfaces replaced (parakeet.wgsl, TypeScript over WebGPU):
 *   pk_context_*            F16GemmKernel.create / F32GemmKernel.create and
 *                           destroy (src/webgpu/kernels/gemm.ts:519-619,
 *                           :849-855, :3009-3095)
 *   pk_gemm_create          F16GemmKernel.createDispatch (gemm.ts:621-704),
 *                           F32GemmKernel.createDispatch (gemm.ts:3097-3182)
 *                           with the contract checks requireGemmShape
 *                           (:971-1011), requireProductionSpecialization
 *                           (:1031-1067), requireRuntimeWeight (:1069-1161)
 *   pk_gemm_validate        the same contract checks without a device
 *   pk_gemm_enqueue(_timed) GemmDispatch.encode(encoder, timestampWrites,
 *                           shape) (gemm.ts:419-463; F32 twin :2912-2960)
 *   pk_gemm_destroy         GemmDispatch.destroy (gemm.ts:465-469)
 *   pk_prepared_weight_*    F16GemmKernel.createPreparedPaletteWeight
 *                           (gemm.ts:706-748), PreparedPaletteWeight (:375-385)
 *   pk_palette_expand       PaletteWeightExpander.createPooledDispatch +
 *                           encode (src/model/palette-expander.ts:234-303),
 *                           shader paletteDequantWgslForScalar (:478-587)
 *   pk_unpack_codes         the code extraction of palette-expander.ts:500-511
 *                           exposed on its own for bit-exact checks
 *   pk_gemm_plan            planF16SubgroupGemm / planF32SubgroupGemm
 *                           (gemm.ts:941-969, :2317-2345): the launch grid
 *   pk_stream_*, pk_event_* GPUQueue.onSubmittedWorkDone / GpuTimestampRecorder
 *                           (src/webgpu/timestamp.ts:44-80) equivalents
 *   pk_alloc / pk_upload /  GPUDevice.createBuffer / queue.writeBuffer /
 *   pk_download / pk_free   mapAsync readback (src/webgpu/arena.ts:141-157)
 */
#ifndef PK_PALETTE_H
#define PK_PALETTE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PK_ABI_VERSION 1

typedef enum pk_status {
  PK_OK = 0,
  PK_INVALID_ARGUMENT = 1,
  PK_ALLOCATION_FAILURE = 2,
  PK_INTERNAL_ERROR = 3,
  PK_DEVICE_ERROR = 4,
  PK_DESTROYED = 5,
  PK_RANGE_ERROR = 6,
} pk_status;

typedef enum pk_precision {
  PK_PRECISION_F16 = 0, /* f16 activations/LUT/output, f32 MFMA accumulate */
  PK_PRECISION_F32 = 1, /* f32 activations/LUT/output, f32 MFMA accumulate */
} pk_precision;

typedef enum pk_activation {
  PK_ACTIVATION_NONE = 0,
  PK_ACTIVATION_SILU = 1,
  PK_ACTIVATION_RELU = 2,
} pk_activation;

/* pk_gemm_desc.flags */
#define PK_GEMM_REQUIRE_PRODUCTION_SIGNATURE 0x1u /* gemm.ts:204-356, :2154-2306 */
/* GLU epilogue, fused from the Conformer convolution that consumes the
   pointwise-1 output (src/webgpu/kernels/conformer-conv.ts:520-535): of the
   N columns, [0, N/2) are GLU values and [N/2, N) their gates, and the
   output is [rows, N/2] = f16(value) * sigmoid(f16(gate)) (each half
   rounded to f16 as the reference's pointwise buffer holds it; sigmoid with
   the reference's clamp at +-20), rounded to f16. f16 precision only; needs
   one palette group, N % 64 == 0, no bias, activation or residual, and no
   shared prepared weight (the op lays out its own codes with value and gate
   blocks interleaved). No counterpart in the reference's GEMM: there the
   GLU runs in the convolution kernel. */
#define PK_GEMM_GLU 0x2u
/* Row LayerNorm fused into the GEMM's input. No counterpart in the
   reference's GEMM: there a LayerNorm dispatch writes the normalised rows
   and the GEMM reads them (layernorm.ts:29-281 before the projections of
   encoder.ts:1897-2116). With this flag the op multiplies LN(A) instead of
   A: LN(a)_k = (a_k - mean) * rstd * gamma_k + beta_k, mean and variance
   max(E[a^2] - mean^2, 0) over the K channels of the row, rstd =
   1 / sqrt(variance + epsilon) (layernorm.ts:309-390), with no pass that
   writes the normalised rows. The kernel multiplies f16(a_k *
   f16(gamma_k)) and finishes each output as rstd * (acc - mean * G_n) +
   B_n with G = f16(gamma) . W and B = beta . W, computed once at create;
   the normalised row is thus not rounded to f16 as the reference's
   LayerNorm output is. f16 only; needs K % 64 == 0, K <= 2048, the packed
   codes (no shared prepared weight), no GLU epilogue, and one palette group
   or groups whose width is a multiple of 256 columns. Runs on the pair-code
   kernels. */
#define PK_GEMM_ROW_NORM 0x4u
/* A store hint with no counterpart in the reference. The f16 pair-code
   kernels store their output non-temporally unless this flag is set: the
   output is mostly read by workgroups on other XCDs than the one that
   wrote each line, and streamed lines need no write-back from L2 when the
   kernel ends. With the flag the stores stay ordinary: for an output that
   a bandwidth-bound launch reads next and finds in the memory-side cache
   (the encoder's first subsampling pointwise GEMM, read by the depthwise
   convolution). Results are the same either way;
   pk_gemm_plan_info.stream_stores tells which a launch uses. */
#define PK_GEMM_CACHED_OUTPUT 0x8u

typedef struct pk_context pk_context;
typedef struct pk_gemm_op pk_gemm_op;
typedef struct pk_prepared_weight pk_prepared_weight;
typedef struct pk_gemm_group pk_gemm_group;

/* ---- library / context --------------------------------------------------- */

int pk_abi_version(void);
const char *pk_last_error(void);
const char *pk_status_name(int status);

/* Create a context on HIP device `device` (it owns one default stream). */
int pk_context_create(int device, pk_context **out);
/* Drops the owner's handle of the context (the reference's device destroy).
   Calls that take the context fail with PK_DESTROYED from then on. Ops,
   prepared weights, graphs and encoders made on it keep its stream and
   device alive until they are released, so they may be released in any
   order afterwards. Call it once per context; NULL is accepted. */
int pk_context_destroy(pk_context *ctx);
int pk_context_device(const pk_context *ctx, int *device);
/* The context's default stream as a hipStream_t. */
int pk_context_stream(const pk_context *ctx, void **stream);

typedef struct pk_device_info {
  char name[64];
  char arch[32];           /* e.g. "gfx950" */
  int32_t compute_units;
  int32_t wavefront_size;
  int64_t global_memory_bytes;
  int32_t lds_bytes_per_block;
  int32_t clock_khz;
} pk_device_info;
int pk_device_query(const pk_context *ctx, pk_device_info *info);

/* ---- memory and streams --------------------------------------------------- */

int pk_alloc(pk_context *ctx, uint64_t bytes, void **device_ptr);
int pk_free(pk_context *ctx, void *device_ptr);
/* Host<->device copies, ordered on `stream` and complete on return. */
int pk_upload(pk_context *ctx, void *device_dst, const void *host_src,
              uint64_t bytes, void *stream);
int pk_download(pk_context *ctx, void *host_dst, const void *device_src,
                uint64_t bytes, void *stream);
int pk_copy_device(pk_context *ctx, void *device_dst, const void *device_src,
                   uint64_t bytes, void *stream);
int pk_stream_create(pk_context *ctx, void **stream);
int pk_stream_destroy(pk_context *ctx, void *stream);
int pk_stream_synchronize(pk_context *ctx, void *stream);

/* No reference counterpart (a WebGPU command buffer is re-encoded per
   submit): records the enqueues a caller makes on `stream` between begin
   and end (this thread only) into a HIP graph of kernel nodes, which
   pk_graph_launch replays on any stream of the context. For callers whose
   step is a few launches, as a serving loop: replays skip the per-launch
   host cost. A graph replays the ops as they were when captured (their
   buffers and active sizes); timed enqueues cannot be captured. */
typedef struct pk_graph pk_graph;
int pk_graph_begin_capture(pk_context *ctx, void *stream);
int pk_graph_end_capture(pk_context *ctx, void *stream, pk_graph **out);
int pk_graph_launch(pk_graph *graph, void *stream);
int pk_graph_destroy(pk_graph *graph);
int pk_event_create(pk_context *ctx, void **event);
int pk_event_destroy(pk_context *ctx, void *event);
int pk_event_record(pk_context *ctx, void *event, void *stream);
int pk_event_synchronize(pk_context *ctx, void *event);
int pk_event_elapsed_ms(pk_context *ctx, void *start, void *end, float *ms);

/* ---- palette weights ------------------------------------------------------ */

/* Packed weight in the reference package format (model/convert.py:2119-2203,
   src/model/runtime-plan.ts:529-588): a logical [inner=K, columns=N] matrix
   of `bits`-bit codes, K-major, cut into groups of 32 codes in 5 words
   (5-bit) or 16 codes in 3 words (6-bit), code i of a group at bit i*bits,
   LSB first. packed_bytes must equal K*N/codes_per_group*words*4. */
typedef struct pk_weight_desc {
  uint32_t struct_size;    /* sizeof(pk_weight_desc) */
  const char *label;
  int32_t palette_bits;    /* 5 or 6 */
  uint32_t inner;          /* K */
  uint32_t columns;        /* N */
  const uint32_t *packed;  /* device */
  uint64_t packed_bytes;
} pk_weight_desc;

/* One-time preparation of a packed weight for the fused GEMM: the codes are
   re-ordered on the device into the MFMA operand order (same bits per code,
   no dense expansion). Several GEMM ops may share one prepared weight. */
int pk_prepared_weight_create(pk_context *ctx, const pk_weight_desc *desc,
                              void *stream, pk_prepared_weight **out);
int pk_prepared_weight_destroy(pk_prepared_weight *weight);
/* Device bytes held by the prepared weight: its codes in MFMA operand order,
 * the one layout every kernel reads, as many bits per code as the packed
 * format (K and N padded to 64 and 32): K * N * bits / 8 at the encoder's
 * shapes. */
int pk_prepared_weight_bytes(const pk_prepared_weight *weight, uint64_t *bytes);

/* ---- GEMM ----------------------------------------------------------------- */

/* C[m, n] = epilogue(sum_k A[m, k] * LUT[g(n)][code(k, n)]) with the
   reference epilogue order bias -> activation -> residual + scale * value
   (gemm.ts:2006-2044). g(n) = min(n / palette_group_columns, groups - 1)
   (palette-expander.ts:543-549). */
typedef struct pk_gemm_desc {
  uint32_t struct_size;          /* sizeof(pk_gemm_desc) */
  uint32_t flags;                /* PK_GEMM_* */
  const char *label;
  int32_t precision;             /* pk_precision */
  int32_t palette_bits;          /* 5 or 6 */
  uint32_t rows;                 /* M capacity */
  uint32_t inner;                /* K */
  uint32_t columns;              /* N */
  uint32_t palette_groups;       /* G */
  uint32_t palette_group_columns;/* N / G */
  const void *a;                 /* [rows, inner] f16|f32, row-major */
  uint64_t a_bytes;
  const uint32_t *packed;        /* reference-format codes (or NULL when prepared) */
  uint64_t packed_bytes;
  const void *palette;           /* [G, 2^bits] f16|f32 */
  uint64_t palette_bytes;
  void *output;                  /* [rows, columns] f16|f32, row-major */
  uint64_t output_bytes;
  const float *bias;             /* [columns] f32, or NULL */
  uint64_t bias_bytes;
  const void *residual;          /* [rows, columns] like output, or NULL */
  uint64_t residual_bytes;
  int32_t has_residual_scale;    /* 0: scale 1 when a residual is given */
  float residual_scale;
  int32_t activation;            /* pk_activation */
  const pk_prepared_weight *prepared; /* optional shared prepared weight */
  /* PK_GEMM_ROW_NORM only: the LayerNorm's parameters. */
  const float *norm_gamma;       /* [inner] f32 */
  uint64_t norm_gamma_bytes;
  const float *norm_beta;        /* [inner] f32 */
  uint64_t norm_beta_bytes;
  float norm_epsilon;            /* 0 selects 1e-5 */
} pk_gemm_desc;

int pk_gemm_create(pk_context *ctx, const pk_gemm_desc *desc, void *stream,
                   pk_gemm_op **out);
/* The descriptor checks of pk_gemm_create alone, with no device and no
   allocation (the reference's createDispatch validation is host-side too,
   gemm.ts:971-1161). A prepared weight is checked against its own geometry
   only. */
int pk_gemm_validate(const pk_gemm_desc *desc);
/* Launch on `stream` for the first `active_rows` rows (0 = all rows). An f16
   prefix is planned for its own row count (the reference re-plans the grid
   per active batch, gemm.ts:427-451): the tile shape may change, but not the
   kernel family or K split, so the codes the op holds serve it and a
   prefix's outputs are bit-identical to the same rows of a full launch; the
   choice is cached per op. A row count given to pk_gemm_prepare_rows runs
   its prepared plan instead. */
int pk_gemm_enqueue(pk_gemm_op *op, uint32_t active_rows, void *stream);
/* No reference counterpart (there one pipeline serves every active batch,
   gemm.ts:427-451): prepares each of `count` active row counts to run the
   plan that pk_gemm_create makes for a descriptor of that many rows - its
   tile, kernel family and K split - so such a prefix is as fast as a
   dedicated op and its outputs are bit-identical to that op's (and within
   the GEMM's tolerance of the same rows of a full launch). A plan that
   reads the codes split into other K parts gets a copy of the codes in
   that layout, derived on the device from the op's own and kept by the op
   (up to two copies). Call before launches that use those row counts (not
   while a launch of the op is in flight); pk_gemm_set_variant and
   pk_gemm_set_splits drop the prepared plans. Row counts must be in
   [1, rows] (PK_RANGE_ERROR); repeated counts are prepared once. */
int pk_gemm_prepare_rows(pk_gemm_op *op, const uint32_t *active_rows, uint32_t count);
/* pk_gemm_enqueue with the timestampWrites of GemmDispatch.encode
   (gemm.ts:419-463): the kernel's own dispatch stamps `start_event` when it
   begins and `end_event` when it ends (either may be NULL; both from
   pk_event_create), so timing adds nothing to the stream. */
int pk_gemm_enqueue_timed(pk_gemm_op *op, uint32_t active_rows, void *stream,
                          void *start_event, void *end_event);
/* Releases the op's device resources. Idempotent: a second call is a no-op
   returning PK_OK; enqueue after destroy returns PK_DESTROYED. The handle
   itself stays valid until pk_gemm_release. */
int pk_gemm_destroy(pk_gemm_op *op);
/* Destroys (if needed) and frees the handle; it must not be used again. */
int pk_gemm_release(pk_gemm_op *op);

/* Tuning hooks: the planner picks a compiled tile shape and a split-K
   factor at create time; these list and force the choice (used by the
   benchmark's sweeps) for every active row count. Both resize the op's
   split-K workspace, and a variant that reads another split of the codes
   re-lays the op's own weight out on the device (PK_RANGE_ERROR for a
   weight shared with other ops); neither may be called while a launch of
   the op is in flight. */
int pk_gemm_variant_count(int precision);
typedef struct pk_gemm_variant_desc {
  uint32_t tile_rows;
  uint32_t tile_columns;
  uint32_t block_threads;
  uint32_t k_split;     /* wavefronts that share each output tile over K */
  uint32_t code_parts;  /* K parts of the prepared code layout it reads */
  int32_t groupable;    /* 1: a pk_gemm_group can run it */
  char kernel5[64];     /* kernel name for 5-bit and 6-bit weights */
  char kernel6[64];
} pk_gemm_variant_desc;
int pk_gemm_variant_describe(int precision, int variant, pk_gemm_variant_desc *desc);
/* Selecting a variant without a split-K path (the f16 pair-code K-split
   variants, every f32 variant) also resets the split count to 1. */
int pk_gemm_set_variant(pk_gemm_op *op, int variant);
/* 1 <= splits <= ceil(inner / 64) for the f16 operand-order variants;
   other variants take 1 only (PK_RANGE_ERROR otherwise). */
int pk_gemm_set_splits(pk_gemm_op *op, uint32_t splits);

typedef struct pk_gemm_plan_info {
  uint32_t grid[3];
  uint32_t block_threads;
  uint32_t tile_rows;
  uint32_t tile_columns;
  uint32_t split_inner;          /* K slices reduced in-kernel (1 = none) */
  uint32_t lds_bytes;
  uint64_t workspace_bytes;      /* split-K partial tiles + tile counters */
  uint64_t flops;                /* 2*M*K*N for active rows */
  uint64_t algorithmic_bytes;    /* compulsory HBM bytes per launch */
  char kernel[64];
  uint32_t stream_stores;        /* 1: non-temporal output stores (PK_GEMM_CACHED_OUTPUT) */
  uint32_t reserved;
} pk_gemm_plan_info;

/* Plan of the launch pk_gemm_enqueue would make for `active_rows`. */
int pk_gemm_plan(const pk_gemm_op *op, uint32_t active_rows,
                 pk_gemm_plan_info *info);

/* ---- GEMM groups ----------------------------------------------------------

   No counterpart in the reference, which dispatches one GEMM at a time. For
   callers with many independent GEMMs of few rows (a batch-1 stream's
   projections that do not feed each other, every layer's rel-pos linear of
   one window length, weight-streaming servers): one launch of the small-M
   kernel runs them all, so the per-launch latency is paid once and the
   weight streams of all members overlap on the device.

   A group holds a snapshot of its members' bindings (input, output, bias,
   residual, palette, epilogue) taken at create; members run concurrently,
   so no member may read a buffer another member writes. Members must be
   f16 ops without the GLU epilogue whose prepared weights hold the codes in
   one K part (the layout of the small-M kernels: an op planned on them, or
   switched to one with pk_gemm_set_variant); PK_RANGE_ERROR names the first
   member that is not. The group keeps each member's prepared weight alive;
   the ops themselves may be released, and a member op's weight can no
   longer be re-laid out by pk_gemm_set_variant while the group lives. At
   most 65535 members of at most 2,097,152 columns each. */
int pk_gemm_group_create(pk_context *ctx, pk_gemm_op *const *ops, uint32_t count,
                         const char *label, pk_gemm_group **out);
/* Launches every member on its first `active_rows` rows (0 = the smallest
   row capacity among the members; PK_RANGE_ERROR above it). */
int pk_gemm_group_enqueue(pk_gemm_group *group, uint32_t active_rows, void *stream);
int pk_gemm_group_enqueue_timed(pk_gemm_group *group, uint32_t active_rows, void *stream,
                                void *start_event, void *end_event);
/* Forces one small-M variant (an index of pk_gemm_variant_count(F16)) for
   every row count, or -1 to return to the planned one; PK_RANGE_ERROR for a
   variant of another kernel family. */
int pk_gemm_group_set_variant(pk_gemm_group *group, int variant);
/* The launch pk_gemm_group_enqueue would make: grid, tile, LDS, the
   members' summed flops and algorithmic bytes, and the kernel name. */
int pk_gemm_group_plan(const pk_gemm_group *group, uint32_t active_rows,
                       pk_gemm_plan_info *info);
/* Waits for the context's stream, frees the group's tables, drops its
   weight references and frees the handle, which must not be used again. */
int pk_gemm_group_destroy(pk_gemm_group *group);

/* ---- expansion and unpack (bit-exact reference semantics) ---------------- */

typedef enum pk_expand_layout {
  PK_EXPAND_ROW_MAJOR = 0,  /* "k-by-output-row-major-f16|f32" */
  PK_EXPAND_TILE_MAJOR = 1, /* "n256-k32-tile-major-f16", "n128-k32-tile-major-f32" */
} pk_expand_layout;

typedef struct pk_expand_desc {
  uint32_t struct_size;          /* sizeof(pk_expand_desc) */
  const char *label;
  int32_t precision;             /* element type of palette and target */
  int32_t palette_bits;
  int32_t layout;                /* pk_expand_layout */
  uint32_t inner;
  uint32_t columns;
  uint32_t palette_groups;
  uint32_t palette_group_columns;
  const uint32_t *packed;
  uint64_t packed_bytes;
  const void *palette;
  uint64_t palette_bytes;
  void *target;                  /* inner*columns elements */
  uint64_t target_bytes;
} pk_expand_desc;

int pk_palette_expand(pk_context *ctx, const pk_expand_desc *desc, void *stream);

/* codes[g*cpg + i] = code i of group g, one byte per code. */
int pk_unpack_codes(pk_context *ctx, int palette_bits, const uint32_t *words,
                    uint64_t group_count, uint8_t *codes, void *stream);

#ifdef __cplusplus
}
#endif

#endif

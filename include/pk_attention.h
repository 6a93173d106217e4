/*
 * pk_attention.h - C ABI of the Transformer-XL relative-position attention
 * on gfx950 (8 heads x 128 channels). Same library, contexts, streams,
 * events and status codes as pk_palette.h.
 *
 * Reference interfaces replaced (src/webgpu/kernels/attention.ts):
 *   pk_attention_validate / pk_attention_create
 *                            RelativeAttentionKernel.createDispatch (:219-314)
 *                            with the shape check (:222-229, RangeError
 *                            "Unsupported attention shape for <label>"),
 *                            requireArenaCapacity (:378-390), requireProjected-
 *                            Positions (:323-353) and requireAttentionBias
 *                            (:355-370), same messages
 *   pk_attention_enqueue(_timed)
 *                            RelativeAttentionDispatch.encode (:62-91), active
 *                            windows as EncoderDispatchShape.batchSize
 *   pk_attention_destroy     RelativeAttentionDispatch.destroy (:93-96)
 *   pk_attention_plan        the dispatch grid of createDispatch (:305-313)
 * RelativeAttentionKernel.create / destroy (:130-217, :316-320) compile the
 * pipeline and own a uniform pool; here the kernels are compiled into the
 * library and the pk_context stands for the kernel object.
 *
 * Frames: the reference accepts 1..192 (one workgroup lane per key); this
 * library takes 1..4096 (flash-style key tiles), so 750-frame windows run.
 */
#ifndef PK_ATTENTION_H
#define PK_ATTENTION_H

#include "pk_palette.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PK_ATTENTION_HEADS 8
#define PK_ATTENTION_HEAD_SIZE 128
#define PK_ATTENTION_MAX_FRAMES 4096

/* pk_attention_desc.flags */
/* projected_positions is [2T-1, 1024] row-major (e.g. straight from a
   palette GEMM of the sinusoid table) instead of the reference's
   "head-vector-position-vec4" order [8][32][2T-1][4]. No counterpart in the
   reference, whose converter packs the table offline. */
#define PK_ATTENTION_POSITIONS_ROW_MAJOR 0x1u
/* An active batch below batch_size runs the variant that pk_attention_create
   plans for a descriptor of that many windows (as a dedicated op would;
   outputs bit-identical to such an op), not the op's own. No counterpart
   in the reference, whose one pipeline serves every active batch
   (attention.ts:62-91). pk_attention_set_variant overrides it. */
#define PK_ATTENTION_PLAN_ACTIVE 0x2u

typedef struct pk_attention_op pk_attention_op;

typedef struct pk_attention_desc {
  uint32_t struct_size;              /* sizeof(pk_attention_desc) */
  uint32_t flags;                    /* PK_ATTENTION_* */
  const char *label;
  int32_t precision;                 /* pk_precision of qkv, positions, output */
  uint32_t batch_size;               /* windows */
  uint32_t frames;                   /* T */
  const void *qkv;                   /* [B*T, 3072]: Q, K, V blocks of 1024, head h at 128h */
  uint64_t qkv_bytes;                /* capacity, >= B*T*3072*elem */
  const void *projected_positions;   /* 2T-1 relative positions x 1024 (layout per flags) */
  uint64_t projected_positions_bytes;/* exactly (2T-1)*1024*elem */
  const float *bias_u;               /* [8, 128] f32 */
  uint64_t bias_u_bytes;             /* exactly 4096 */
  const float *bias_v;               /* [8, 128] f32 */
  uint64_t bias_v_bytes;             /* exactly 4096 */
  const uint32_t *valid_lengths;     /* [B] */
  uint64_t valid_lengths_bytes;      /* capacity, >= 4*B */
  void *output;                      /* [B*T, 1024]; must not overlap qkv */
  uint64_t output_bytes;             /* capacity, >= B*T*1024*elem */
} pk_attention_desc;

typedef struct pk_attention_plan_info {
  uint32_t grid[3];
  uint32_t block_threads;
  uint32_t lds_bytes;
  uint32_t query_tiles;
  uint64_t algorithmic_bytes;        /* qkv + positions + biases + lengths + output of the active windows */
  char kernel[64];
} pk_attention_plan_info;

int pk_attention_validate(const pk_attention_desc *desc);
int pk_attention_create(pk_context *ctx, const pk_attention_desc *desc, pk_attention_op **out);
/* Launch for the first `active_batch` windows (0 = batch_size). */
int pk_attention_enqueue(pk_attention_op *op, uint32_t active_batch, void *stream);
int pk_attention_enqueue_timed(pk_attention_op *op, uint32_t active_batch, void *stream,
                               void *start_event, void *end_event);
int pk_attention_plan(const pk_attention_op *op, uint32_t active_batch, pk_attention_plan_info *info);
int pk_attention_destroy(pk_attention_op *op);
int pk_attention_release(pk_attention_op *op);
/* Tuning hooks: f16 launch shapes - 0..2: one 32-query tile per workgroup
   with 4, 2 or 1 wavefronts splitting the key tiles (planned up to 256
   frames); 3, 4: 2 or 4 wavefronts of 32 queries sharing each staged K, V
   and position tile (4 planned beyond 256 frames). f32 - 0: the flash
   kernel on f32 MFMAs, a wavefront per 32-query tile (planned); 1: one
   workgroup per query in the reference's own operation order. */
int pk_attention_variant_count(int precision);
int pk_attention_set_variant(pk_attention_op *op, int variant);

#ifdef __cplusplus
}
#endif

#endif

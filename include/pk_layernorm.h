/*
 * pk_layernorm.h - C ABI of the row LayerNorm on gfx950. Same library,
 * contexts, streams, events and status codes as pk_palette.h.
 *
 * Reference interfaces replaced (src/webgpu/kernels/layernorm.ts):
 *   pk_layernorm_validate / pk_layernorm_create
 *                             LayerNormKernel.createDispatch (:165-240): the
 *                             shape check (RangeError "Invalid LayerNorm shape
 *                             for <label>"), requireArenaCapacity (:248-260)
 *                             and requirePackedTensor (:262-281), same messages
 *   pk_layernorm_enqueue(_timed)
 *                             LayerNormDispatch.encode (:40-65): active rows as
 *                             EncoderDispatchShape.rows
 *   pk_layernorm_destroy      LayerNormDispatch.destroy (:67-70)
 * LayerNormKernel.create / destroy compile a pipeline and own a uniform pool;
 * the pk_context stands for that kernel object here.
 */
#ifndef PK_LAYERNORM_H
#define PK_LAYERNORM_H

#include "pk_palette.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct pk_layernorm_op pk_layernorm_op;

typedef struct pk_layernorm_desc {
  uint32_t struct_size;        /* sizeof(pk_layernorm_desc) */
  const char *label;
  int32_t precision;           /* pk_precision of input and output */
  uint32_t rows;
  uint32_t channels;           /* multiple of 4 */
  const void *input;           /* [rows, channels] */
  uint64_t input_bytes;        /* capacity */
  const float *gamma;          /* [channels] f32, "channel" layout */
  uint64_t gamma_bytes;        /* exactly 4 * channels */
  const float *beta;           /* [channels] f32 */
  uint64_t beta_bytes;         /* exactly 4 * channels */
  void *output;                /* [rows, channels]; may equal input */
  uint64_t output_bytes;       /* capacity */
  int32_t has_epsilon;         /* 0: epsilon 1e-5 (the reference default) */
  float epsilon;
  /* Optional chained LayerNorm, no reference counterpart (the reference
     runs two dispatches): with next_output set, the same launch also
     writes next_output = LayerNorm(output as stored) with next_gamma /
     next_beta ([channels] f32) and the same epsilon, bit-identical to a
     second LayerNorm over the output. Rows of at most 4096 bytes (2048 f16
     or 1024 f32 channels); next_output must not overlap output and must be
     the input or not overlap it. NULL next_output: none. */
  const float *next_gamma;
  uint64_t next_gamma_bytes;   /* exactly 4 * channels */
  const float *next_beta;
  uint64_t next_beta_bytes;    /* exactly 4 * channels */
  void *next_output;           /* [rows, channels] */
  uint64_t next_output_bytes;  /* capacity */
} pk_layernorm_desc;

int pk_layernorm_validate(const pk_layernorm_desc *desc);
int pk_layernorm_create(pk_context *ctx, const pk_layernorm_desc *desc, pk_layernorm_op **out);
/* Normalise the first `active_rows` rows (0 = all). */
int pk_layernorm_enqueue(pk_layernorm_op *op, uint32_t active_rows, void *stream);
int pk_layernorm_enqueue_timed(pk_layernorm_op *op, uint32_t active_rows, void *stream,
                               void *start_event, void *end_event);
int pk_layernorm_destroy(pk_layernorm_op *op);
int pk_layernorm_release(pk_layernorm_op *op);

#ifdef __cplusplus
}
#endif

#endif

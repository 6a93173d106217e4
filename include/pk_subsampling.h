/*
 * pk_subsampling.h - the convolution stages of the encoder's subsampling
 * front end on gfx950 (8x in time and frequency, NeMo's "dw_striding":
 * conv0 1->256 3x3/2 + ReLU, depthwise 3x3/2, pointwise 256->256 + ReLU,
 * depthwise 3x3/2, pointwise + ReLU, flatten, linear 4096->1024). The
 * pointwise and linear stages are palette GEMMs (pk_palette.h); this header
 * covers the three non-GEMM kernels. Same library, contexts, streams, events
 * and status codes as pk_palette.h.
 *
 * Reference interfaces replaced (src/webgpu/kernels/subsampling.ts):
 *   pk_subsampling_output_dimension  subsamplingOutputDimension (:119-122)
 *   pk_subsampling_valid_length      subsamplingValidLength (:124-135)
 *   pk_subsampling_fused_create      FusedSubsamplingConv0Depthwise2Kernel
 *                                    .createDispatch (:334-425), planFused...
 *                                    (:145-206), shader :1092-1239
 *   pk_subsampling_depthwise_create  DepthwiseSubsamplingKernel.createDispatch
 *                                    (:495-560), planDepthwise (:795-853),
 *                                    shader :1241-1330
 *   pk_subsampling_mask_create       SubsamplingTimeMaskKernel.createDispatch
 *                                    (:698-790), shader :1332-1430
 *   pk_subsampling_enqueue(_timed)   SubsamplingDispatch.encode (:221-240) and
 *                                    SubsamplingTimeMaskDispatch.encode
 *   pk_subsampling_destroy           the dispatches' destroy()
 * The *_validate functions run the createDispatch checks on the host alone.
 *
 * Error behaviour follows the reference: a shape, capacity, length offset or
 * step count it rejects with RangeError returns PK_RANGE_ERROR; a tensor of
 * the wrong type, layout or size returns PK_INVALID_ARGUMENT; the message
 * (pk_last_error) has the reference's wording with the descriptor's label.
 * The fused stage takes any number of input frames (the reference fixes
 * 1501); bins and channels are fixed at 128 and 256 as there.
 */
#ifndef PK_SUBSAMPLING_H
#define PK_SUBSAMPLING_H

#include "pk_palette.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PK_SUBSAMPLING_BINS 128
#define PK_SUBSAMPLING_CHANNELS 256

typedef struct pk_subsampling_op pk_subsampling_op;

/* floor((input + 2 - 3) / 2) + 1 for input >= 1; 0 for 0. */
uint32_t pk_subsampling_output_dimension(uint32_t input);
/* `steps` applications of pk_subsampling_output_dimension to a frame count. */
uint32_t pk_subsampling_valid_length(uint32_t feature_length, uint32_t steps);

typedef struct pk_subsampling_fused_desc {
  uint32_t struct_size;          /* sizeof(pk_subsampling_fused_desc) */
  const char *label;
  int32_t precision;             /* PK_PRECISION_F16 | PK_PRECISION_F32 */
  uint32_t batch_size;
  uint32_t input_height;         /* feature frames (1501 for 15 s) */
  uint32_t input_width;          /* mel bins, 128 */
  uint32_t channels;             /* 256 */
  const float *input;            /* f32 feature-major [batch, width, height] */
  uint64_t input_bytes;
  const void *conv0_weights;     /* [3,3,C] kh-kw-output-channel-vec4 (precision) */
  uint64_t conv0_weights_bytes;
  const float *conv0_bias;       /* [C] f32 */
  uint64_t conv0_bias_bytes;
  const void *depthwise_weights; /* [3,3,C] kh-kw-channel-vec4 (precision) */
  uint64_t depthwise_weights_bytes;
  const float *depthwise_bias;   /* [C] f32 */
  uint64_t depthwise_bias_bytes;
  void *output;                  /* channel-last [batch, Ho, Wo, C] (precision) */
  uint64_t output_bytes;
  const uint32_t *valid_lengths; /* raw feature frames per window */
  uint64_t valid_lengths_bytes;
  uint32_t valid_length_batch_offset; /* first entry of valid_lengths used */
} pk_subsampling_fused_desc;

typedef struct pk_subsampling_depthwise_desc {
  uint32_t struct_size;          /* sizeof(pk_subsampling_depthwise_desc) */
  const char *label;
  int32_t precision;
  uint32_t batch_size;
  uint32_t input_height;
  uint32_t input_width;
  uint32_t channels;             /* multiple of 4 */
  const void *input;             /* channel-last [batch, H, W, C] */
  uint64_t input_bytes;
  const void *weights;           /* [3,3,C] kh-kw-channel-vec4 */
  uint64_t weights_bytes;
  const float *bias;             /* [C] f32 */
  uint64_t bias_bytes;
  void *output;                  /* [batch, sub(H), sub(W), C] */
  uint64_t output_bytes;
  const uint32_t *valid_lengths; /* raw feature frames per window */
  uint64_t valid_lengths_bytes;
  uint32_t valid_length_batch_offset;
  uint32_t valid_length_subsampling_steps; /* stride-2 stages through this output */
} pk_subsampling_depthwise_desc;

typedef struct pk_subsampling_mask_desc {
  uint32_t struct_size;          /* sizeof(pk_subsampling_mask_desc) */
  const char *label;
  int32_t precision;
  uint32_t batch_size;
  uint32_t height;
  uint32_t width;
  uint32_t channels;             /* multiple of 4 */
  void *values;                  /* in place, [batch, height, width, channels] */
  uint64_t values_bytes;
  const uint32_t *valid_lengths; /* raw feature frames per window */
  uint64_t valid_lengths_bytes;
  uint32_t valid_length_batch_offset;
  uint32_t valid_length_subsampling_steps;
} pk_subsampling_mask_desc;

int pk_subsampling_fused_validate(const pk_subsampling_fused_desc *desc);
int pk_subsampling_fused_create(pk_context *ctx, const pk_subsampling_fused_desc *desc, pk_subsampling_op **out);
int pk_subsampling_depthwise_validate(const pk_subsampling_depthwise_desc *desc);
int pk_subsampling_depthwise_create(pk_context *ctx, const pk_subsampling_depthwise_desc *desc,
                                    pk_subsampling_op **out);
int pk_subsampling_mask_validate(const pk_subsampling_mask_desc *desc);
int pk_subsampling_mask_create(pk_context *ctx, const pk_subsampling_mask_desc *desc, pk_subsampling_op **out);

/* Launch over the first `active_batch` windows (0 = all) on `stream`. */
int pk_subsampling_enqueue(pk_subsampling_op *op, uint32_t active_batch, void *stream);
int pk_subsampling_enqueue_timed(pk_subsampling_op *op, uint32_t active_batch, void *stream, void *start_event,
                                 void *end_event);

typedef struct pk_subsampling_plan_info {
  uint32_t output_height;
  uint32_t output_width;
  uint32_t grid[3];
  uint32_t block_threads;
  uint32_t lds_bytes;
  uint64_t algorithmic_bytes;    /* compulsory HBM bytes per launch */
  uint64_t flops;                /* multiply-adds x 2 */
  char kernel[64];
} pk_subsampling_plan_info;

int pk_subsampling_plan(const pk_subsampling_op *op, uint32_t active_batch, pk_subsampling_plan_info *info);
/* Idempotent; enqueue after destroy returns PK_DESTROYED. */
int pk_subsampling_destroy(pk_subsampling_op *op);
int pk_subsampling_release(pk_subsampling_op *op);

#ifdef __cplusplus
}
#endif

#endif

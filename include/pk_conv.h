/*
 * pk_conv.h - C ABI of the fused Conformer convolution tail on gfx950: GLU of
 * the pointwise-1 output, same-padded depthwise convolution with kernel 9
 * over frames, folded batch norm and SiLU, in one kernel. Lives in the same
 * library as pk_palette.h and shares its contexts, memory, streams, events and
 * status codes (pk_status, pk_last_error).
 *
 * Reference interfaces replaced (src/webgpu/kernels/conformer-conv.ts):
 *   pk_conv_plan_shape       planFusedConformerConv (:72-115)
 *   pk_conv_validate         the createDispatch checks (:255-300) without a
 *                            device: requirePositiveInteger (:454-458),
 *                            requireArenaCapacity (:390-401) and
 *                            requirePackedTensor (:403-432)
 *   pk_conv_create           FusedConformerConvKernel.createDispatch (:255-344)
 *   pk_conv_enqueue(_timed)  FusedConformerConvDispatch.encode (:128-157),
 *                            active batch as EncoderDispatchShape.batchSize
 *   pk_conv_destroy          FusedConformerConvDispatch.destroy (:159-162)
 * FusedConformerConvKernel.create / destroy (:194-253, :346-350) compile a
 * pipeline and own a uniform pool; here the kernels are compiled into the
 * library and the pk_context stands for the device, so there is no separate
 * kernel object.
 *
 * Shapes. channels = 0 means 1024 (CONFORMER_CONV_CHANNELS, :13); any
 * multiple of 8 is accepted. Element type (pk_precision) applies to the
 * pointwise input, the depthwise weights and the output; the folded batch
 * norm is f32 in both precisions, like the reference's "channel" tensors.
 */
#ifndef PK_CONV_H
#define PK_CONV_H

#include "pk_palette.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PK_CONV_KERNEL_SIZE 9
#define PK_CONV_DEFAULT_CHANNELS 1024

typedef struct pk_conv_op pk_conv_op;

/* pk_conv_desc.flags */
/* The pointwise input already holds the GLU, [batch*frames, C] (e.g. the
   output of a pk_gemm op with PK_GEMM_GLU), instead of [.., 2C] values and
   gates; the convolution applies only the frame mask to it. No counterpart
   in the reference, whose convolution kernel always forms the GLU. */
#define PK_CONV_INPUT_GLU 0x1u

typedef struct pk_conv_desc {
  uint32_t struct_size;            /* sizeof(pk_conv_desc) */
  uint32_t flags;                  /* PK_CONV_* */
  const char *label;
  int32_t precision;               /* pk_precision */
  uint32_t batch_size;             /* windows (batch items) */
  uint32_t frames;                 /* frames per window */
  uint32_t channels;               /* C; 0 = 1024 */
  const void *pointwise_input;     /* [batch*frames, 2C]: GLU values [0, C), gates [C, 2C)
                                      ([batch*frames, C] GLU with PK_CONV_INPUT_GLU) */
  uint64_t pointwise_input_bytes;  /* capacity, >= rows*2C*elem (rows*C*elem) */
  const void *depthwise_weights;   /* [9, C] channel-last ("kernel-channel-vec4") */
  uint64_t depthwise_weights_bytes;/* exactly 9*C*elem */
  const float *batch_norm_scale;   /* [C] gamma / sqrt(var + eps) */
  uint64_t batch_norm_scale_bytes; /* exactly 4*C */
  const float *batch_norm_shift;   /* [C] beta - mean * scale (+ folded conv bias) */
  uint64_t batch_norm_shift_bytes; /* exactly 4*C */
  const uint32_t *valid_lengths;   /* [batch] valid frames per window */
  uint64_t valid_lengths_bytes;    /* capacity, >= 4*batch */
  void *output;                    /* [batch*frames, C]; must not overlap the input */
  uint64_t output_bytes;           /* capacity, >= rows*C*elem */
} pk_conv_desc;

typedef struct pk_conv_plan_info {
  uint32_t rows;                   /* batch * frames */
  uint64_t input_bytes;            /* inputByteLength (of a [rows, 2C] input) */
  uint64_t output_bytes;           /* outputByteLength */
  uint64_t valid_lengths_bytes;    /* validLengthsByteLength */
  uint64_t depthwise_weight_bytes; /* depthwiseWeightByteLength */
  uint64_t affine_bytes;           /* affineByteLength */
  uint32_t grid[3];                /* launch grid (one dimension used) */
  uint32_t block_threads;
  uint32_t lds_bytes;              /* 0: the GLU window lives in registers */
  uint64_t algorithmic_bytes;      /* compulsory HBM bytes for the active batch */
  char kernel[64];
} pk_conv_plan_info;

/* planFusedConformerConv for a shape, without a device: the byte lengths and
   this library's launch for `batch_size` windows of `frames` frames. */
int pk_conv_plan_shape(int precision, uint32_t batch_size, uint32_t frames,
                       uint32_t channels, pk_conv_plan_info *info);
/* The descriptor checks of pk_conv_create, host-only. */
int pk_conv_validate(const pk_conv_desc *desc);
int pk_conv_create(pk_context *ctx, const pk_conv_desc *desc, pk_conv_op **out);
/* Launch for the first `active_batch` windows (0 = batch_size); outside
   [1, batch_size] is PK_RANGE_ERROR ("active batch must be in [1, B]"). */
int pk_conv_enqueue(pk_conv_op *op, uint32_t active_batch, void *stream);
/* pk_conv_enqueue whose dispatch stamps `start_event` / `end_event` (either
   may be NULL), the timestampWrites of encode (:128-157). */
int pk_conv_enqueue_timed(pk_conv_op *op, uint32_t active_batch, void *stream,
                          void *start_event, void *end_event);
/* Plan of the launch pk_conv_enqueue would make. */
int pk_conv_plan(const pk_conv_op *op, uint32_t active_batch, pk_conv_plan_info *info);
/* Idempotent; enqueue afterwards returns PK_DESTROYED. */
int pk_conv_destroy(pk_conv_op *op);
/* Destroys (if needed) and frees the handle. */
int pk_conv_release(pk_conv_op *op);
/* Tuning hooks: compiled launch shapes (channels per thread x frames per
   thread) for a precision, and forcing one on an op. */
int pk_conv_variant_count(int precision);
int pk_conv_set_variant(pk_conv_op *op, int variant);

#ifdef __cplusplus
}
#endif

#endif

/*
 * pk_encoder.h - the FastConformer encoder layer stack on gfx950, composed
 * natively from this library's ops (palette GEMMs, LayerNorm, relative
 * attention, fused convolution tail). Same library, contexts, streams,
 * events and status codes as pk_palette.h.
 *
 * Reference interfaces replaced: the encoder graph of src/webgpu/encoder.ts -
 * createEncoderLayerDispatches (:1868-2135), fifteen dispatches per layer in
 * this order:
 *   LN ff1 -> FF1 W1 + SiLU -> FF1 W2 + 0.5 x         (x1)
 *   LN att -> QKV -> relative attention -> Wo + x1    (x2)
 *   LN conv -> PW1 -> GLU/DW9/BN/SiLU -> PW2 + x2     (x3)
 *   LN ff2 -> FF2 W1 + SiLU -> FF2 W2 + 0.5 x3        (x4)
 *   LN out -> next layer
 * and the encode loop that records them for the active windows. The
 * subsampling front end (src/webgpu/kernels/subsampling.ts) and the TDT
 * decoder are not part of this object: its input is the subsampled
 * [windows * frames, 1024] feature block.
 */
#ifndef PK_ENCODER_H
#define PK_ENCODER_H

#include "pk_palette.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PK_ENCODER_CHANNELS 1024
#define PK_ENCODER_INTERMEDIATE 4096

/* pk_encoder_desc.flags */
#define PK_ENCODER_FUSED_GLU 0x1u  /* PW1 carries the GLU epilogue (PK_GEMM_GLU) */

typedef struct pk_encoder pk_encoder;

/* One palette matrix in the reference package format: packed codes
   (K*N*bits/8 bytes) and its palette ([groups, 2^bits] f16). */
typedef struct pk_encoder_matrix {
  const uint32_t *packed;
  const void *palette;
} pk_encoder_matrix;

/* Device pointers of one layer's package tensors (encoder.ts names).
   Bit widths are the reference package's (model/convert.py:1360-1475):
   feed-forward and pointwise 5-bit, QKV 5-bit with 3 palette groups, Wo
   6-bit. Sizes follow from the shapes; every pointer is 16-byte aligned. */
typedef struct pk_encoder_layer {
  const float *norm_gamma[5];    /* norm_feed_forward1, norm_self_att, norm_conv, norm_feed_forward2, norm_out [1024] */
  const float *norm_beta[5];
  pk_encoder_matrix ff1_linear1; /* 1024 -> 4096 */
  pk_encoder_matrix ff1_linear2; /* 4096 -> 1024 */
  pk_encoder_matrix qkv;         /* 1024 -> 3072, 3 palette groups */
  const void *projected_positions; /* [8][32][2T-1][4] head-vector-position-vec4 */
  const float *bias_u;           /* [8, 128] */
  const float *bias_v;           /* [8, 128] */
  pk_encoder_matrix o_proj;      /* 1024 -> 1024, 6-bit */
  pk_encoder_matrix pointwise1;  /* 1024 -> 2048 */
  const void *depthwise;         /* [9, 1024] kernel-channel-vec4 */
  const float *bn_scale;         /* [1024] folded batch norm */
  const float *bn_shift;         /* [1024] */
  pk_encoder_matrix pointwise2;  /* 1024 -> 1024 */
  pk_encoder_matrix ff2_linear1;
  pk_encoder_matrix ff2_linear2;
} pk_encoder_layer;

typedef struct pk_encoder_desc {
  uint32_t struct_size;          /* sizeof(pk_encoder_desc) */
  uint32_t flags;                /* PK_ENCODER_* */
  const char *label;
  int32_t precision;             /* PK_PRECISION_F16 */
  uint32_t batch_size;           /* windows */
  uint32_t frames;               /* encoder frames per window (188) */
  uint32_t layers;               /* 1..64 */
  const pk_encoder_layer *layer; /* host array of `layers` entries */
  const uint32_t *valid_lengths; /* device [batch] encoder frames per window */
  const void *input;             /* device [batch*frames, 1024] f16: subsampled features (not modified) */
  void *output;                  /* device [batch*frames, 1024] f16: encoder output, not overlapping input */
} pk_encoder_desc;

/* The descriptor checks of pk_encoder_create, host-only: the stack's own
   fields, then every op's descriptor (pk_gemm_validate, pk_layernorm_validate,
   pk_attention_validate, pk_conv_validate) as the stack would build it, with
   the failing op's label (e.g. "encoder.layers.3-self-attention-qkv") in the
   message. */
int pk_encoder_validate(const pk_encoder_desc *desc);
/* Prepares every layer's codes, allocates the activation arena and creates
   the fifteen ops per layer. */
int pk_encoder_create(pk_context *ctx, const pk_encoder_desc *desc, void *stream, pk_encoder **out);
/* One encoder pass over the first `active_batch` windows (0 = all). With
   `use_graph` the pass is captured once per active batch into a HIP graph
   and replayed (no per-launch host work). */
int pk_encoder_enqueue(pk_encoder *enc, uint32_t active_batch, void *stream, int use_graph);
/* One eager pass whose dispatches stamp timestamps, as the reference's
   profiled encode does (encoder.ts:1641-1674 with timestampWrites per
   dispatch, test/webgpu/encoder-profile.test.ts): `start_events[i]` /
   `end_events[i]` (from pk_event_create) belong to launch i of the pass,
   15 per layer in the order above; either array, or any entry, may be NULL. */
int pk_encoder_enqueue_profiled(pk_encoder *enc, uint32_t active_batch, void *stream,
                                void *const *start_events, void *const *end_events);
/* Launches in one pass and device bytes held (prepared codes + arena). */
int pk_encoder_info(const pk_encoder *enc, uint32_t *launches, uint64_t *device_bytes);
int pk_encoder_destroy(pk_encoder *enc);

#ifdef __cplusplus
}
#endif

#endif

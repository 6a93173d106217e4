/*
 * pk_encoder.h - the FastConformer encoder layer stack on gfx950, composed
 * natively from this library's ops (palette GEMMs, LayerNorm, relative
 * attention, fused convolution tail). Same library, contexts, streams,
 * events and status codes as pk_palette.h.
 *
 * Reference interfaces replaced: the encoder graph of src/webgpu/encoder.ts -
 * createEncoderLayerDispatches (:1868-2135), fifteen dispatch slots per
 * layer in this order (after the first layer the LN ff1 slot launches
 * nothing: the LN out before it wrote that LayerNorm too, unless
 * PK_ENCODER_UNCHAINED_NORMS; with
 * PK_ENCODER_FUSED_NORMS the four LayerNorms that feed a GEMM run inside
 * that GEMM and their slots launch nothing):
 *   LN ff1 -> FF1 W1 + SiLU -> FF1 W2 + 0.5 x         (x1)
 *   LN att -> QKV -> relative attention -> Wo + x1    (x2)
 *   LN conv -> PW1 -> GLU/DW9/BN/SiLU -> PW2 + x2     (x3)
 *   LN ff2 -> FF2 W1 + SiLU -> FF2 W2 + 0.5 x3        (x4)
 *   LN out -> next layer
 * and the encode loop that records them for the active windows
 * (ParakeetEncoderGraph.encode, encoder.ts:1690-1706): optionally the
 * subsampling front end first (createSubsamplingCommands, encoder.ts:
 * 2140-2400: fused conv0+depthwise2, pointwise3 + ReLU, depthwise5,
 * pointwise6 + ReLU, the time mask, the flatten linear), then the layers,
 * then optionally the projector (encoder.ts:1489-1509). Without the front
 * end the input is the subsampled [windows * frames, 1024] feature block.
 * The TDT decoder is not part of this object.
 */
#ifndef PK_ENCODER_H
#define PK_ENCODER_H

#include "pk_palette.h"
#include "pk_subsampling.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PK_ENCODER_CHANNELS 1024
#define PK_ENCODER_INTERMEDIATE 4096

/* pk_encoder_desc.flags */
/* PW1 carries the GLU epilogue (PK_GEMM_GLU) and the convolution reads the
   [rows, 1024] GLU (PK_CONV_INPUT_GLU). This is the default; the flag is
   still accepted. */
#define PK_ENCODER_FUSED_GLU 0x1u
/* Keep the reference's order instead: PW1 writes values and gates
   ([rows, 2048]) and the convolution forms the GLU in f32. The default
   rounds the GLU to f16 once more and was measured 80 us faster per
   16-window pass (PW1 and the convolution tail both move less). Not with
   PK_ENCODER_FUSED_GLU. */
#define PK_ENCODER_SEPARATE_GLU 0x8u
/* Run the LayerNorms before FF1 W1, QKV, PW1 and FF2 W1 inside the GEMMs
   that read them (PK_GEMM_ROW_NORM; PW1 only with PK_ENCODER_SEPARATE_GLU):
   96 fewer launches per 24-layer pass, but each of those GEMMs does the
   row statistics of every column tile again; on 16 windows the pass is
   about 5% slower than with the separate LayerNorm launches, which stay
   the default. */
#define PK_ENCODER_FUSED_NORMS 0x2u
/* Without this flag (and without PK_ENCODER_FUSED_NORMS), the last
   LayerNorm of each layer also writes the next layer's first LayerNorm
   (LN ff1 of its own output) in the same launch, so layers after the
   first launch nothing in their LN ff1 slot: 23 fewer launches per 24-layer
   pass, bit-identical outputs. This flag keeps one launch per LayerNorm. */
#define PK_ENCODER_UNCHAINED_NORMS 0x4u
/* By default an active batch a below batch_size runs every GEMM and the
   attention with the plan a graph built for a windows would use
   (pk_gemm_prepare_rows for every a at create, PK_ATTENTION_PLAN_ACTIVE):
   a prefix runs as fast as a dedicated graph and its outputs are
   bit-identical to that graph's, within tolerance of the same windows of a
   full pass; the GEMMs whose prefix plans read codes in other K parts keep
   copies of their codes (device_bytes counts them). With this flag a
   prefix keeps each op's kernel family and K split, as the reference's
   single pipeline per dispatch does (encoder.ts:197-200, gemm.ts:427-451):
   outputs bit-identical to the same windows of a full pass, at up to
   1.7x the time of a dedicated graph for small prefixes. */
#define PK_ENCODER_PREFIX_SAME_PLAN 0x10u

typedef struct pk_encoder pk_encoder;

/* One palette matrix in the reference package format: packed codes
   (K*N*bits/8 bytes) and its palette ([groups, 2^bits] in the encoder's
   precision). Below, "f16" tensors (palettes, projected positions,
   depthwise and front-end convolution weights, activations) are f32 with
   PK_PRECISION_F32, the reference's fp32 profile (encoder.ts:947-1165). */
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

/* The subsampling front end's package tensors (encoder.subsampling.*,
   model/convert.py:1264-1340): conv0 and both depthwise kernels [3,3,256]
   f16 (kh-kw-output-channel-vec4 / kh-kw-channel-vec4) with f32 biases
   [256]; the 5-bit pointwise matrices 256->256 with f32 biases; the 5-bit
   flatten linear 4096->1024 (columns in frequency-major order) with its f32
   bias [1024]. */
typedef struct pk_encoder_subsampling {
  const void *conv0_weights;
  const float *conv0_bias;
  const void *depthwise2_weights;
  const float *depthwise2_bias;
  pk_encoder_matrix pointwise3;
  const float *pointwise3_bias;
  const void *depthwise5_weights;
  const float *depthwise5_bias;
  pk_encoder_matrix pointwise6;
  const float *pointwise6_bias;
  pk_encoder_matrix linear;
  const float *linear_bias;
} pk_encoder_subsampling;

typedef struct pk_encoder_desc {
  uint32_t struct_size;          /* sizeof(pk_encoder_desc) */
  uint32_t flags;                /* PK_ENCODER_* */
  const char *label;
  int32_t precision;             /* PK_PRECISION_F16, or PK_PRECISION_F32 (the fp32 profile: f32 GEMMs,
                                    LayerNorm, attention, convolution and front end; the GLU stays in the
                                    convolution; not with PK_ENCODER_FUSED_GLU or PK_ENCODER_FUSED_NORMS) */
  uint32_t batch_size;           /* windows */
  uint32_t frames;               /* encoder frames per window (188) */
  uint32_t layers;               /* 1..64 */
  const pk_encoder_layer *layer; /* host array of `layers` entries */
  const uint32_t *valid_lengths; /* device [batch] encoder frames per window */
  const void *input;             /* device, not modified: [batch*frames, 1024] f16 subsampled features, or
                                    with `subsampling` the f32 feature-major fbank [batch, 128, feature_frames] */
  void *output;                  /* device [batch*frames, 1024] f16: encoder output, not overlapping input */
  /* Front end (NULL: none). frames must be pk_subsampling_valid_length(
     feature_frames, 3) and valid_lengths hold pk_subsampling_valid_length(
     feature_lengths[i], 3), as uploadValidFeatureLengths derives them
     (encoder.ts:1555-1582). */
  const pk_encoder_subsampling *subsampling;
  uint32_t feature_frames;       /* fbank frames per window (1501 for 15 s) */
  const uint32_t *feature_lengths; /* device [batch] raw fbank frames per window */
  /* Projector (projected_channels 0: none): 5-bit palette GEMM
     1024 -> projected_channels + f32 bias, reading `output`. */
  pk_encoder_matrix projector;
  const float *projector_bias;
  uint32_t projected_channels;   /* reference 640 */
  void *projected_output;        /* device [batch*frames, projected_channels] f16 */
} pk_encoder_desc;

/* The descriptor checks of pk_encoder_create, host-only: the stack's own
   fields, then every op's descriptor (pk_gemm_validate, pk_layernorm_validate,
   pk_attention_validate, pk_conv_validate) as the stack would build it, with
   the failing op's label (e.g. "encoder.layers.3-self-attention-qkv") in the
   message. */
int pk_encoder_validate(const pk_encoder_desc *desc);
/* Prepares every layer's codes, allocates the activation arena and creates
   the ops of every layer (fifteen, or eleven with fused norms). */
int pk_encoder_create(pk_context *ctx, const pk_encoder_desc *desc, void *stream, pk_encoder **out);
/* One encoder pass over the first `active_batch` windows (0 = all). With
   `use_graph` the pass is captured once per active batch into a HIP graph
   and replayed (no per-launch host work). */
int pk_encoder_enqueue(pk_encoder *enc, uint32_t active_batch, void *stream, int use_graph);
/* One eager pass whose dispatches stamp timestamps, as the reference's
   profiled encode does (encoder.ts:1641-1674 with timestampWrites per
   dispatch, test/webgpu/encoder-profile.test.ts): `start_events[i]` /
   `end_events[i]` (from pk_event_create) belong to dispatch slot i of the
   pass (pk_encoder_info's count, in order: the six front-end launches,
   fifteen per layer, the projector); a LayerNorm slot fused into the GEMM
   after it records both of its events back to back on the stream. Either
   array, or any entry, may be NULL. */
int pk_encoder_enqueue_profiled(pk_encoder *enc, uint32_t active_batch, void *stream,
                                void *const *start_events, void *const *end_events);
/* Dispatch slots of one pass (the profiled pass's event count) and device
   bytes held (prepared codes, the fused norms' column sums, the arena). */
int pk_encoder_info(const pk_encoder *enc, uint32_t *launches, uint64_t *device_bytes);
int pk_encoder_destroy(pk_encoder *enc);

#ifdef __cplusplus
}
#endif

#endif

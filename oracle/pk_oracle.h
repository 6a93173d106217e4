/*
 * pk_oracle.h - CPU restatement of parakeet.wgsl's palette-weight GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP product
 * is compared against; it is never linked into, loaded by or called from the
 * product library (parakeet.wgsl_amd/csrc). Only tests/, the smoke check and
 * the CPU-baseline leg of bench.py may load it.
 *
 * Every function restates one piece of the reference and cites it. The
 * reference runs only as WGSL inside a WebGPU browser, so it cannot execute in
 * this environment; each function's pin is listed beside it:
 *
 *   pko_pack_codes        model/convert.py:2130-2156 (pack_palette_codes_lsb)
 *                         pinned: model/tests/test_convert.py:447-479 KATs,
 *                         pack/unpack round trip, brute-force bit positions.
 *   pko_unpack_codes      src/model/palette-expander.ts:500-511 (codeExpression)
 *                         and model/tests/test_convert.py:90-115
 *                         pinned: the same KATs, exhaustive 5/6-bit patterns.
 *   pko_palette_group     src/model/palette-expander.ts:543-549
 *                         pinned: closed form, test_convert.py:481-511 fixture.
 *   pko_tile_major_index  src/model/runtime-plan.ts:454-490
 *                         pinned: bijection + tile contiguity invariants of
 *                         test/model/palette-expander.test.ts:147-247.
 *   pko_expand            src/model/palette-expander.ts:478-587
 *                         pinned: one-hot LUTs recover the codes exactly.
 *   pko_gemm (F32_CHAIN)  src/webgpu/kernels/gemm.ts:2356-2599, epilogue
 *                         :2847-2869 - pinned: exact integer-valued inputs vs
 *                         the textbook product, constant-LUT closed form,
 *                         brute force on tiny shapes.
 *   pko_gemm (F16_CHAIN)  src/webgpu/kernels/gemm.ts:1362-1716 (f16
 *                         accumulator, increasing k), epilogue :2006-2044
 *                         pinned: exact small-integer cases, the f16 rounding
 *                         function against every f16 value and its midpoints.
 *   pko_gemm (F64)        reference-independent truth of the same expression.
 *   pko_relative_attention  src/webgpu/kernels/attention.ts:418-727 (Transformer-XL
 *                         relative-position attention, 8 heads x 128); pinned by
 *                         a float64 torch restatement, plain attention when the
 *                         positions and biases are zero, the direction of the
 *                         relative shift, one valid key and empty windows.
 *   pko_layernorm         src/webgpu/kernels/layernorm.ts:309-390 (row mean, biased
 *                         variance as E[x^2] - mean^2 clamped at 0, rsqrt of
 *                         variance + epsilon, gamma and beta); pinned by torch's
 *                         layer_norm, constant rows and the unit-affine moments.
 *   pko_glu               the GLU step of conformer-conv.ts:520-535 on its own
 *                         (value * sigmoid(gate) of a [rows, 2C] input);
 *                         pinned by torch's glu and the gate clamp in
 *                         tests/test_oracle.py.
 *   pko_conformer_conv    src/webgpu/kernels/conformer-conv.ts:495-573 (GLU of
 *                         the pointwise-1 output, same-padded depthwise k9 over
 *                         frames, folded batch norm, SiLU); pinned by closed
 *                         forms in tests/test_oracle.py (one-hot taps, zero
 *                         gates, frames past the valid length, the f64 twin).
 *   pko_subsampled_length src/webgpu/kernels/subsampling.ts:119-135 and the
 *                         shaders' (length + 1) / 2 per stride-2 step; pinned by
 *                         test/webgpu/subsampling-kernel-shapes.test.ts:27-50.
 *   pko_subsampling_fused src/webgpu/kernels/subsampling.ts:1092-1239 (conv0
 *                         1->C 3x3 stride 2 pad 1 + ReLU, rounded to the
 *                         storage type, then depthwise 3x3 stride 2 + bias);
 *   pko_subsampling_depthwise  subsampling.ts:1241-1330 (channel-last depthwise
 *                         3x3 stride 2 + bias, no activation);
 *   pko_subsampling_mask  subsampling.ts:1332-1430 (zero the frames at or past
 *                         the subsampled valid length); the three are pinned by
 *                         torch's conv2d in float64, one-hot kernels and the
 *                         length edges in tests/test_oracle.py.
 *   pko_tdt_decode        src/webgpu/kernels/tdt-decoder.ts:1133-2010 (greedy TDT
 *                         decode: two-layer LSTM predictor with gate chains in
 *                         the profile's format (f16 or f32), f32 cell update,
 *                         f32 decoder projector, ReLU joint, vocabulary head in
 *                         the profile's format, lowest-id argmax, durations, the
 *                         10-symbol cap and the bounded end-of-stream flush);
 *                         pinned by closed forms (zero-weight heads that fix the
 *                         token and duration), torch.nn.LSTM / matmul restatements
 *                         of one predictor step and one joint, and its exp and
 *                         tanh against the math library.
 *   pko_exp_f32, pko_tanh_f32  the decoder's transcendental functions, written
 *                         from range reduction and a Taylor polynomial (the
 *                         reference uses WGSL's exp / tanh, whose last bits are
 *                         implementation-defined); pinned against numpy.
 *
 * Status codes: 0 ok, 1 invalid argument.
 */
#ifndef PK_ORACLE_H
#define PK_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  PKO_ACT_NONE = 0,
  PKO_ACT_SILU = 1,
  PKO_ACT_RELU = 2,
};

enum {
  PKO_MODE_F32_CHAIN = 0, /* f32 accumulator, fmaf in increasing k */
  PKO_MODE_F16_CHAIN = 1, /* f16 accumulator, one rounding per fused fma */
  PKO_MODE_F64 = 2,       /* double accumulation, double epilogue */
};

enum {
  PKO_DTYPE_F16 = 0,
  PKO_DTYPE_F32 = 1,
  PKO_DTYPE_F64 = 2, /* pko_conformer_conv only: double input and output */
};

typedef struct pko_gemm_args {
  uint32_t rows;              /* M */
  uint32_t inner;             /* K */
  uint32_t columns;           /* N */
  int32_t bits;               /* 5 or 6 */
  uint32_t palette_groups;    /* G */
  uint32_t palette_group_columns;
  int32_t dtype;              /* PKO_DTYPE_F16: A, LUT, residual, output f16 */
  const uint32_t *packed;     /* reference layout words */
  const void *palette;        /* [G, 2^bits] */
  const void *a;              /* [M, K] */
  const float *bias;          /* [N] or NULL */
  const void *residual;       /* [M, N] or NULL */
  float residual_scale;
  int32_t activation;
  void *out;                  /* [M, N]: f16 / f32 per dtype, double for F64 */
} pko_gemm_args;

uint16_t pko_f64_to_f16(double value);
double pko_f16_to_f64(uint16_t bits);
/* The nearest binary16 value of `value` (ties to even) as a double; equal to
   pko_f16_to_f64(pko_f64_to_f16(value)), without the bit assembly. */
double pko_round_f16(double value);
void pko_f32_to_f16_array(const float *src, uint16_t *dst, uint64_t count);
void pko_f16_to_f32_array(const uint16_t *src, float *dst, uint64_t count);

int pko_pack_codes(int bits, const uint8_t *codes, uint64_t code_count,
                   uint32_t *words);
int pko_unpack_codes(int bits, const uint32_t *words, uint64_t group_count,
                     uint8_t *codes);
uint32_t pko_palette_group(uint32_t column, uint32_t palette_group_columns,
                           uint32_t palette_groups);
uint64_t pko_tile_major_index(uint64_t scalar_index, uint32_t inner,
                              uint32_t columns, uint32_t tile_columns);
int pko_expand(int bits, int dtype, int tile_major, const uint32_t *packed,
               uint32_t inner, uint32_t columns,
               uint32_t palette_group_columns, uint32_t palette_groups,
               const void *palette, void *out);
int pko_gemm(const pko_gemm_args *args, int mode, int threads);

/* Conformer convolution tail. input [batch*frames, 2*channels] (dtype):
   channels [0, C) are GLU values, [C, 2C) gates; weights [9, channels]
   (dtype); scale, shift [channels] f32; valid [batch] frame counts;
   output [batch*frames, channels] (dtype). mode PKO_MODE_F32_CHAIN: the
   reference's f32 arithmetic (fma over taps 0..8); PKO_MODE_F64: the same
   expression in double (output still rounded to dtype). dtype PKO_DTYPE_F64
   takes double input and weights and writes double output (truth chains). */
/* Relative-position self-attention of attention.ts:418-727 over 8 heads of
   128 channels. qkv [batch*frames, 3072] (dtype; Q, K, V column blocks of
   1024, head h at columns 128h..); positions: projected relative positions in
   the reference's "head-vector-position-vec4" order [8][32][2T-1][4] (dtype),
   position p holds relative distance T-1-p; bias_u, bias_v [8, 128] f32;
   valid [batch]; out [batch*frames, 1024] (dtype). For a query q below
   valid = min(valid[b], T):
     score(q, k) = sum_d (q_d + u_d) k_d + (q_d + v_d) R[T-1-q+k]_d, d in
                   order, both products per d by fma, times 1/sqrt(128),
     p(q, k)     = exp(score - max_k score) / sum_k exp(...) over k < valid,
     out(q)      = sum_k p(q, k) v_k (fma in key order);
   rows q >= valid are zero. mode PKO_MODE_F32_CHAIN: the reference's f32
   arithmetic; PKO_MODE_F64: the same in double, rounded to dtype at the
   end (PKO_DTYPE_F64: double in and out). */
int pko_relative_attention(int dtype, int mode, uint32_t batch, uint32_t frames, const void *qkv,
                           const void *positions, const float *bias_u, const float *bias_v,
                           const uint32_t *valid, void *out);

/* LayerNorm of [rows, channels] (dtype) with gamma, beta [channels] f32:
   mean = sum / C, variance = max(sum of squares / C - mean^2, 0),
   out = (x - mean) * rsqrt(variance + epsilon) * gamma + beta; f32 sums in
   PKO_MODE_F32_CHAIN, double in PKO_MODE_F64; output rounded to dtype. */
int pko_layernorm(int dtype, int mode, uint64_t rows, uint32_t channels, const void *input, const float *gamma,
                  const float *beta, float epsilon, void *output);

/* GLU of a [rows, 2*channels] input (values, then gates) into [rows,
   channels]: value * sigmoid(gate) with the reference's clamp, in f32
   (PKO_MODE_F32_CHAIN) or double (PKO_MODE_F64), rounded to dtype
   (PKO_DTYPE_F64: double input and output). */
int pko_glu(int dtype, int mode, uint64_t rows, uint32_t channels, const void *input, void *output);

int pko_conformer_conv(int dtype, int mode, uint32_t batch, uint32_t frames, uint32_t channels,
                       const void *input, const void *weights, const float *scale,
                       const float *shift, const uint32_t *valid, void *output);

/* Length after `steps` same-padded stride-2 3x3 convolutions:
   length = (length + 1) / 2 per step (floor((n + 2 - 3) / 2) + 1). */
uint32_t pko_subsampled_length(uint32_t length, uint32_t steps);

/* Fused conv0 + depthwise2 of the subsampling front end. input: f32
   feature-major [batch, width, height] (width = mel bins, height = frames);
   conv0_weights, depthwise_weights: [3, 3, channels] (dtype); biases f32
   [channels]; valid: raw frame lengths [batch]; output (dtype) channel-last
   [batch, Ho, Wo, channels] with H1 = sub(height), W1 = sub(width), Ho =
   sub(H1), Wo = sub(W1). conv0 at (y, x) for y < min(H1, sub(L, 1)):
   bias + fma over taps (ky, kx) in order, skipping taps outside the input,
   then ReLU, rounded to dtype (f16 storage) or kept (f32, f64); zero
   elsewhere. Output rows y >= sub(L, 2) are zero; the others are bias + fma
   over the in-range conv0 taps (rows below sub(L, 1)), rounded to dtype.
   dtype PKO_DTYPE_F64 computes in double throughout. */
int pko_subsampling_fused(int dtype, uint32_t batch, uint32_t height, uint32_t width, uint32_t channels,
                          const float *input, const void *conv0_weights, const float *conv0_bias,
                          const void *depthwise_weights, const float *depthwise_bias, const uint32_t *valid,
                          void *output);

/* Channel-last depthwise 3x3 stride-2 pad-1 convolution [batch, height,
   width, channels] -> [batch, sub(height), sub(width), channels] (dtype):
   output rows y >= sub(L, steps) are zero; the others are bias + fma over
   the taps in order, skipping input rows outside [0, min(height,
   sub(L, steps - 1))) and columns outside [0, width). */
int pko_subsampling_depthwise(int dtype, uint32_t batch, uint32_t height, uint32_t width, uint32_t channels,
                              const void *input, const void *weights, const float *bias, const uint32_t *valid,
                              uint32_t steps, void *output);

/* Zero, in place, the rows y >= sub(L, steps) of [batch, height, width,
   channels] values (dtype). */
int pko_subsampling_mask(int dtype, uint32_t batch, uint32_t height, uint32_t width, uint32_t channels,
                         void *values, const uint32_t *valid, uint32_t steps);

/* ---- greedy TDT decoder ---------------------------------------------- */

#define PKO_TDT_HIDDEN 640
#define PKO_TDT_GATES 2560
#define PKO_TDT_TOKENS 1025     /* 1024 tokens + blank (1024) */
#define PKO_TDT_HEAD 1032       /* tokens, blank, 5 durations, 2 padding */
#define PKO_TDT_BLANK 1024
#define PKO_TDT_DURATIONS 5
#define PKO_TDT_OVERFLOW 1u

/* exp(x) for |x| <= 87 (normal results) in f32: n = rint(x log2 e), r = x - n ln2 (two-part
   ln2, fmaf), e^r by a degree-7 Taylor polynomial (Horner, fmaf), times 2^n;
   within 2 ulp of the exact value. */
float pko_exp_f32(float x);
/* tanh(x) = sign(x) (1 - 2 / (exp(2|x|) + 1)) in f32 (absolute error below
   2^-23); callers clamp to [-10, 10] as the reference does. */
float pko_tanh_f32(float x);

typedef struct pko_tdt_weights {
  /* weights: f16 (uint16_t bits) in the f16 profile, f32 when f32 != 0 */
  const void *embedding;           /* [1025, 640] token-by-channel */
  const void *lstm_weight[2];      /* [1280, 2560] k-by-ifgo (k < 640: input, k >= 640: recurrent h) */
  const float *lstm_bias[2];       /* f32 [2560] (bias_ih + bias_hh) */
  const void *projector_weight;    /* [640, 640] k-by-output */
  const float *projector_bias;     /* f32 [640] */
  const void *head_weight;         /* [640, 1032] k-by-output (1030 used) */
  const float *head_bias;          /* f32 [1032] */
  int32_t f32;                     /* 0: f16 profile, 1: f32 profile (tdt-decoder.ts:196-218) */
} pko_tdt_weights;

/* Greedy TDT decode of `batch` windows (tdt-decoder.ts:1664-2010):
   encoder_projected [batch, frames, 640] in the profile's element (f16 bits
   or f32); lengths, starts, ends, flush [batch]; outputs tokens /
   token_frames / token_durations [batch, max_tokens], counts and status
   [batch]. state f32 [batch, 4, 640] and scratch f32 [batch, 5, 640] are
   working memory (written). The f16 profile runs every chain in binary16
   (inputs and biases rounded to f16), the f32 profile in binary32 with
   nothing rounded (the f32 readers and chains, :595-614, :700-716,
   :1033-1058, :1092-1104). */
int pko_tdt_decode(const pko_tdt_weights *w, uint32_t batch, uint32_t frames, uint32_t max_tokens,
                   const void *encoder_projected, const uint32_t *lengths, const uint32_t *starts,
                   const uint32_t *ends, const uint32_t *flush, float *state, float *scratch, uint32_t *tokens,
                   uint32_t *token_frames, uint32_t *token_durations, uint32_t *counts, uint32_t *status);

/* One predictor step of window-independent pieces, for pins: from token
   (ignored when initial) and the committed state [4, 640] (h0, c0, h1, c1)
   to the candidates [5, 640] (h0, c0, h1, c1, projection). */
void pko_tdt_predictor(const pko_tdt_weights *w, uint32_t token, int initial, const float *state, float *candidate);
/* One joint: scores [1032] (f32 values of the head accumulators) of
   relu(encoder_row + projection) through the head (encoder_row in the
   profile's element); returns the chosen token and duration through
   `token` / `duration`. */
void pko_tdt_joint(const pko_tdt_weights *w, const void *encoder_row, const float *projection, float *scores,
                   uint32_t *token, uint32_t *duration);

#ifdef __cplusplus
}
#endif

#endif

/*
 * pk_oracle.c - CPU restatement of parakeet.wgsl's palette-weight GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP product, never part of
 * it. Built with -ffp-contract=off so every rounding written here is the
 * rounding performed. See pk_oracle.h for the per-function reference
 * citations and the checks that pin each function.
 */
#include "pk_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* binary16 conversion (IEEE 754 round-to-nearest-even, written from the    */
/* format definition: 1 sign, 5 exponent (bias 15), 10 fraction bits).       */
/* ------------------------------------------------------------------------ */

uint16_t pko_f64_to_f16(double value) {
  uint64_t bits;
  memcpy(&bits, &value, sizeof bits);
  const uint16_t sign = (uint16_t)((bits >> 48) & 0x8000u);
  const uint64_t magnitude = bits & 0x7fffffffffffffffull;
  const int biased = (int)(magnitude >> 52);
  const uint64_t fraction = magnitude & ((1ull << 52) - 1);
  if (biased == 0x7ff) {
    return (uint16_t)(sign | (fraction ? 0x7e00u : 0x7c00u));
  }
  const int exponent = biased - 1023;
  if (exponent > 15) return (uint16_t)(sign | 0x7c00u);
  if (exponent >= -14) {
    /* normal binary16: keep 10 fraction bits, round on the other 42 */
    const uint64_t keep = fraction >> 42;
    const uint64_t rest = fraction & ((1ull << 42) - 1);
    const uint64_t half = 1ull << 41;
    uint32_t h = ((uint32_t)(exponent + 15) << 10) | (uint32_t)keep;
    if (rest > half || (rest == half && (keep & 1u))) h += 1u; /* may carry to inf */
    return (uint16_t)(sign | h);
  }
  if (exponent < -25) return sign; /* below half the smallest subnormal */
  /* subnormal binary16: integer multiple of 2^-24 */
  const uint64_t significand = (1ull << 52) | fraction;
  const int shift = 28 - exponent; /* 43..53 */
  uint64_t q = significand >> shift;
  const uint64_t rest = significand & ((1ull << shift) - 1);
  const uint64_t half = 1ull << (shift - 1);
  if (rest > half || (rest == half && (q & 1u))) q += 1u; /* 1024 = min normal */
  return (uint16_t)(sign | (uint16_t)q);
}

double pko_f16_to_f64(uint16_t h) {
  const double sign = (h & 0x8000u) ? -1.0 : 1.0;
  const int biased = (h >> 10) & 0x1f;
  const int fraction = h & 0x3ff;
  if (biased == 0x1f) return fraction ? NAN : sign * INFINITY;
  if (biased == 0) return sign * (double)fraction * 0x1p-24; /* exact */
  /* normal: the same sign, exponent and fraction in binary64 fields */
  const uint64_t bits = ((uint64_t)(h & 0x8000u) << 48) | ((uint64_t)(biased - 15 + 1023) << 52) |
                        ((uint64_t)fraction << 42);
  double value;
  memcpy(&value, &bits, sizeof value);
  return value;
}

void pko_f32_to_f16_array(const float *src, uint16_t *dst, uint64_t count) {
  for (uint64_t i = 0; i < count; ++i) dst[i] = pko_f64_to_f16((double)src[i]);
}

void pko_f16_to_f32_array(const uint16_t *src, float *dst, uint64_t count) {
  for (uint64_t i = 0; i < count; ++i) dst[i] = (float)pko_f16_to_f64(src[i]);
}

/* Round a double to the nearest binary16 value (ties to even), returned as
   a double. Adding and subtracting C = 1.5 * 2^52 * ulp rounds to a multiple
   of ulp in the current (round-to-nearest-even) mode; ulp is 2^(e-10) for
   binary16 normals (2^e <= |v| < 2^(e+1), e >= -14) and 2^-24 below. */
double pko_round_f16(double value) {
  uint64_t bits;
  memcpy(&bits, &value, sizeof bits);
  const int biased = (int)((bits >> 52) & 0x7ff);
  if (biased == 0x7ff) return value; /* inf, nan */
  int ulp_exponent = biased - 1023 - 10;
  if (ulp_exponent < -24) ulp_exponent = -24;
  if (ulp_exponent > 5) return (bits >> 63) ? -INFINITY : INFINITY; /* |v| >= 2^16 */
  const uint64_t c_bits = ((uint64_t)(ulp_exponent + 52 + 1023) << 52) | (1ull << 51);
  double c;
  memcpy(&c, &c_bits, sizeof c);
  const volatile double sum = value + c; /* keep the two roundings apart */
  const double rounded = sum - c;
  if (rounded >= 65536.0) return INFINITY;
  if (rounded <= -65536.0) return -INFINITY;
  return rounded == 0.0 ? copysign(0.0, value) : rounded;
}

static inline double round_to_f16(double value) { return pko_round_f16(value); }

/* ------------------------------------------------------------------------ */
/* Packed code format                                                        */
/* ------------------------------------------------------------------------ */

static int group_spec(int bits, uint32_t *codes_per_group,
                      uint32_t *words_per_group) {
  /* model/convert.py:2119-2127 palette_code_group_spec */
  if (bits == 5) {
    *codes_per_group = 32;
    *words_per_group = 5;
    return 0;
  }
  if (bits == 6) {
    *codes_per_group = 16;
    *words_per_group = 3;
    return 0;
  }
  return 1;
}

int pko_pack_codes(int bits, const uint8_t *codes, uint64_t code_count,
                   uint32_t *words) {
  /* model/convert.py:2130-2156: code i of a group at bit i*bits, LSB first;
     a code crossing a word boundary puts its high bits in the next word. */
  uint32_t cpg = 0, wpg = 0;
  if (group_spec(bits, &cpg, &wpg) || code_count % cpg) return 1;
  const uint64_t groups = code_count / cpg;
  const uint32_t limit = 1u << bits;
  for (uint64_t g = 0; g < groups; ++g) {
    uint32_t *w = words + g * wpg;
    for (uint32_t i = 0; i < wpg; ++i) w[i] = 0;
    for (uint32_t i = 0; i < cpg; ++i) {
      const uint32_t code = codes[g * cpg + i];
      if (code >= limit) return 1;
      const uint32_t bit = i * (uint32_t)bits;
      const uint32_t word = bit / 32, shift = bit % 32;
      w[word] |= code << shift;
      const int overflow = (int)(shift + (uint32_t)bits) - 32;
      if (overflow > 0) w[word + 1] |= code >> ((uint32_t)bits - (uint32_t)overflow);
    }
  }
  return 0;
}

int pko_unpack_codes(int bits, const uint32_t *words, uint64_t group_count,
                     uint8_t *codes) {
  /* src/model/palette-expander.ts:500-511 codeExpression, u32 arithmetic:
     ((w[b/32] >> b%32) | (w[b/32+1] << (32 - b%32))) & mask */
  uint32_t cpg = 0, wpg = 0;
  if (group_spec(bits, &cpg, &wpg)) return 1;
  const uint32_t mask = (1u << bits) - 1u;
  for (uint64_t g = 0; g < group_count; ++g) {
    const uint32_t *w = words + g * wpg;
    for (uint32_t i = 0; i < cpg; ++i) {
      const uint32_t bit = i * (uint32_t)bits;
      const uint32_t word = bit / 32, shift = bit % 32;
      uint32_t value = w[word] >> shift;
      if (shift + (uint32_t)bits > 32) value |= w[word + 1] << (32 - shift);
      codes[g * cpg + i] = (uint8_t)(value & mask);
    }
  }
  return 0;
}

uint32_t pko_palette_group(uint32_t column, uint32_t palette_group_columns,
                           uint32_t palette_groups) {
  /* src/model/palette-expander.ts:543-549 */
  const uint32_t g = column / palette_group_columns;
  return g < palette_groups - 1u ? g : palette_groups - 1u;
}

uint64_t pko_tile_major_index(uint64_t scalar_index, uint32_t inner,
                              uint32_t columns, uint32_t tile_columns) {
  /* src/model/runtime-plan.ts:454-490 (k tiles of 32, n tiles of
     tile_columns, tile-major then k-in-tile then n-in-tile) */
  const uint64_t k = scalar_index / columns;
  const uint64_t n = scalar_index % columns;
  const uint64_t n_tile = n / tile_columns;
  const uint64_t k_tile = k / 32u;
  const uint64_t k_tiles = inner / 32u;
  const uint64_t k_in_tile = k % 32u;
  const uint64_t n_in_tile = n % tile_columns;
  return ((n_tile * k_tiles + k_tile) * 32u + k_in_tile) * tile_columns +
         n_in_tile;
}

static int check_palette_geometry(int bits, uint32_t inner, uint32_t columns,
                                  uint32_t group_columns, uint32_t groups) {
  uint32_t cpg = 0, wpg = 0;
  if (group_spec(bits, &cpg, &wpg)) return 1;
  if (!inner || !columns || !groups || !group_columns) return 1;
  if (columns % cpg) return 1;                         /* runtime-plan.ts:550 */
  if ((uint64_t)group_columns * groups != columns) return 1; /* :576-585 */
  return 0;
}

int pko_expand(int bits, int dtype, int tile_major, const uint32_t *packed,
               uint32_t inner, uint32_t columns,
               uint32_t palette_group_columns, uint32_t palette_groups,
               const void *palette, void *out) {
  /* src/model/palette-expander.ts:573-585: one group of codes at a time,
     palette group taken from the group's first scalar, dense value
     LUT[group * 2^bits + code] written row-major or tile-major
     (n256-k32 for f16, n128-k32 for f32; runtime-plan.ts:26-37). */
  if (check_palette_geometry(bits, inner, columns, palette_group_columns,
                             palette_groups))
    return 1;
  if (dtype != PKO_DTYPE_F16 && dtype != PKO_DTYPE_F32) return 1;
  const uint32_t tile_columns = dtype == PKO_DTYPE_F16 ? 256u : 128u;
  if (tile_major && (inner % 32u || columns % tile_columns)) return 1;
  uint32_t cpg = 0, wpg = 0;
  group_spec(bits, &cpg, &wpg);
  const uint64_t scalars = (uint64_t)inner * columns;
  const uint64_t groups = scalars / cpg;
  const uint32_t entries = 1u << bits;
  uint8_t codes[32];
  for (uint64_t g = 0; g < groups; ++g) {
    pko_unpack_codes(bits, packed + g * wpg, 1, codes);
    const uint64_t base = g * cpg;
    const uint32_t pg = pko_palette_group((uint32_t)(base % columns),
                                          palette_group_columns,
                                          palette_groups);
    for (uint32_t i = 0; i < cpg; ++i) {
      const uint64_t scalar = base + i;
      const uint64_t dst =
          tile_major ? pko_tile_major_index(scalar, inner, columns, tile_columns)
                     : scalar;
      const uint32_t entry = pg * entries + codes[i];
      if (dtype == PKO_DTYPE_F16)
        ((uint16_t *)out)[dst] = ((const uint16_t *)palette)[entry];
      else
        ((float *)out)[dst] = ((const float *)palette)[entry];
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* GEMM + epilogue                                                           */
/* ------------------------------------------------------------------------ */

typedef struct gemm_job {
  const pko_gemm_args *args;
  int mode;
  const void *dense;   /* expanded W: float (F32 chain) or double */
  uint32_t row_begin, row_end;
} gemm_job;

/* Epilogue in f32 (gemm.ts:2006-2044 and :2847-2869): bias, then activation,
   then residual + scale * value. */
static inline float epilogue_f32(const pko_gemm_args *p, float value,
                                 uint32_t m, uint32_t n) {
  if (p->bias) value += p->bias[n];
  if (p->activation == PKO_ACT_SILU) {
    const float bounded = fminf(fmaxf(value, -20.0f), 20.0f);
    value = value / (1.0f + expf(-bounded));
  } else if (p->activation == PKO_ACT_RELU) {
    value = fmaxf(value, 0.0f);
  }
  if (p->residual) {
    const uint64_t idx = (uint64_t)m * p->columns + n;
    const float r = p->dtype == PKO_DTYPE_F16
                        ? (float)pko_f16_to_f64(((const uint16_t *)p->residual)[idx])
                        : ((const float *)p->residual)[idx];
    value = r + p->residual_scale * value;
  }
  return value;
}

static inline double epilogue_f64(const pko_gemm_args *p, double value,
                                  uint32_t m, uint32_t n) {
  if (p->bias) value += (double)p->bias[n];
  if (p->activation == PKO_ACT_SILU) {
    const double bounded = fmin(fmax(value, -20.0), 20.0);
    value = value / (1.0 + exp(-bounded));
  } else if (p->activation == PKO_ACT_RELU) {
    value = fmax(value, 0.0);
  }
  if (p->residual) {
    const uint64_t idx = (uint64_t)m * p->columns + n;
    const double r = p->dtype == PKO_DTYPE_F16
                         ? pko_f16_to_f64(((const uint16_t *)p->residual)[idx])
                         : (double)((const float *)p->residual)[idx];
    value = r + (double)p->residual_scale * value;
  }
  return value;
}

static inline double a_value(const pko_gemm_args *p, uint64_t idx) {
  return p->dtype == PKO_DTYPE_F16
             ? pko_f16_to_f64(((const uint16_t *)p->a)[idx])
             : (double)((const float *)p->a)[idx];
}

/* Rows are processed in blocks of ROW_BLOCK so each expanded weight row is
   read once per block rather than once per output row; every output element
   still accumulates its own products in increasing k, so the arithmetic of
   each element is that of the one-row loop. */
#define ROW_BLOCK 8

/* f32 accumulator chain, increasing k, one fused multiply-add per step
   (gemm.ts:2398-2420 acc = fma(vec4<f32>(a), b, acc)). */
#define F32_CHAIN_BODY                                                       \
  for (uint32_t k = 0; k < K; ++k) {                                         \
    const float *wrow = w + (uint64_t)k * N;                                 \
    for (uint32_t r = 0; r < rows; ++r) {                                    \
      const float a = (float)a_value(p, (uint64_t)(m0 + r) * K + k);         \
      float *accr = acc + (uint64_t)r * N;                                   \
      for (uint32_t n = 0; n < N; ++n) accr[n] = fmaf(a, wrow[n], accr[n]);  \
    }                                                                        \
  }

__attribute__((target("fma"))) static void f32_rows_fma(const pko_gemm_args *p, const float *w, float *acc,
                                                        uint32_t m0, uint32_t rows) {
  const uint32_t K = p->inner, N = p->columns;
  F32_CHAIN_BODY
}

static void f32_rows_generic(const pko_gemm_args *p, const float *w, float *acc, uint32_t m0, uint32_t rows) {
  const uint32_t K = p->inner, N = p->columns;
  F32_CHAIN_BODY
}

static void *gemm_worker(void *opaque) {
  gemm_job *job = (gemm_job *)opaque;
  const pko_gemm_args *p = job->args;
  const uint32_t K = p->inner, N = p->columns;
  if (job->mode == PKO_MODE_F32_CHAIN) {
    const float *w = (const float *)job->dense;
    float *acc = (float *)malloc(sizeof(float) * N * ROW_BLOCK);
    const int use_fma = __builtin_cpu_supports("fma");
    for (uint32_t m0 = job->row_begin; m0 < job->row_end; m0 += ROW_BLOCK) {
      const uint32_t rows = job->row_end - m0 < ROW_BLOCK ? job->row_end - m0 : ROW_BLOCK;
      for (uint64_t i = 0; i < (uint64_t)rows * N; ++i) acc[i] = 0.0f;
      if (use_fma)
        f32_rows_fma(p, w, acc, m0, rows);
      else
        f32_rows_generic(p, w, acc, m0, rows);
      for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t n = 0; n < N; ++n) {
          const float v = epilogue_f32(p, acc[(uint64_t)r * N + n], m0 + r, n);
          const uint64_t idx = (uint64_t)(m0 + r) * N + n;
          if (p->dtype == PKO_DTYPE_F16)
            ((uint16_t *)p->out)[idx] = pko_f64_to_f16((double)v);
          else
            ((float *)p->out)[idx] = v;
        }
    }
    free(acc);
  } else if (job->mode == PKO_MODE_F16_CHAIN) {
    /* gemm.ts:1445-1453, :1476-1481: vec4<f16> accumulators, fma in
       increasing k. The product of two binary16 values is exact in double
       and, below binary16 overflow, so is its sum with a binary16
       accumulator; one round_to_f16 per step is therefore a fused fma. */
    const double *w = (const double *)job->dense;
    double *acc = (double *)malloc(sizeof(double) * N * ROW_BLOCK);
    for (uint32_t m0 = job->row_begin; m0 < job->row_end; m0 += ROW_BLOCK) {
      const uint32_t rows = job->row_end - m0 < ROW_BLOCK ? job->row_end - m0 : ROW_BLOCK;
      for (uint64_t i = 0; i < (uint64_t)rows * N; ++i) acc[i] = 0.0;
      for (uint32_t k = 0; k < K; ++k) {
        const double *wrow = w + (uint64_t)k * N;
        for (uint32_t r = 0; r < rows; ++r) {
          const double a = a_value(p, (uint64_t)(m0 + r) * K + k);
          double *accr = acc + (uint64_t)r * N;
          for (uint32_t n = 0; n < N; ++n) accr[n] = round_to_f16(a * wrow[n] + accr[n]);
        }
      }
      for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t n = 0; n < N; ++n) {
          const float v = epilogue_f32(p, (float)acc[(uint64_t)r * N + n], m0 + r, n);
          ((uint16_t *)p->out)[(uint64_t)(m0 + r) * N + n] = pko_f64_to_f16((double)v);
        }
    }
    free(acc);
  } else {
    const double *w = (const double *)job->dense;
    double *acc = (double *)malloc(sizeof(double) * N * ROW_BLOCK);
    for (uint32_t m0 = job->row_begin; m0 < job->row_end; m0 += ROW_BLOCK) {
      const uint32_t rows = job->row_end - m0 < ROW_BLOCK ? job->row_end - m0 : ROW_BLOCK;
      for (uint64_t i = 0; i < (uint64_t)rows * N; ++i) acc[i] = 0.0;
      for (uint32_t k = 0; k < K; ++k) {
        const double *wrow = w + (uint64_t)k * N;
        for (uint32_t r = 0; r < rows; ++r) {
          const double a = a_value(p, (uint64_t)(m0 + r) * K + k);
          double *accr = acc + (uint64_t)r * N;
          for (uint32_t n = 0; n < N; ++n) accr[n] += a * wrow[n];
        }
      }
      for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t n = 0; n < N; ++n)
          ((double *)p->out)[(uint64_t)(m0 + r) * N + n] = epilogue_f64(p, acc[(uint64_t)r * N + n], m0 + r, n);
    }
    free(acc);
  }
  return NULL;
}

int pko_gemm(const pko_gemm_args *p, int mode, int threads) {
  if (!p || !p->packed || !p->palette || !p->a || !p->out) return 1;
  if (check_palette_geometry(p->bits, p->inner, p->columns,
                             p->palette_group_columns, p->palette_groups))
    return 1;
  if (p->dtype != PKO_DTYPE_F16 && p->dtype != PKO_DTYPE_F32) return 1;
  if (mode == PKO_MODE_F16_CHAIN && p->dtype != PKO_DTYPE_F16) return 1;
  if (mode < PKO_MODE_F32_CHAIN || mode > PKO_MODE_F64) return 1;
  if (!p->rows) return 0;
  if (threads < 1) threads = 1;
  const uint64_t scalars = (uint64_t)p->inner * p->columns;

  /* Expand the palette weight once (palette-expander.ts:573-585), widened to
     the working precision of the chain. */
  void *dense = NULL;
  {
    const size_t elem = p->dtype == PKO_DTYPE_F16 ? 2 : 4;
    void *narrow = malloc(scalars * elem);
    if (!narrow) return 1;
    pko_expand(p->bits, p->dtype, 0, p->packed, p->inner, p->columns,
               p->palette_group_columns, p->palette_groups, p->palette, narrow);
    if (mode == PKO_MODE_F32_CHAIN) {
      float *w = (float *)malloc(scalars * sizeof(float));
      for (uint64_t i = 0; i < scalars; ++i)
        w[i] = p->dtype == PKO_DTYPE_F16
                   ? (float)pko_f16_to_f64(((uint16_t *)narrow)[i])
                   : ((float *)narrow)[i];
      dense = w;
    } else {
      double *w = (double *)malloc(scalars * sizeof(double));
      for (uint64_t i = 0; i < scalars; ++i)
        w[i] = p->dtype == PKO_DTYPE_F16
                   ? pko_f16_to_f64(((uint16_t *)narrow)[i])
                   : (double)((float *)narrow)[i];
      dense = w;
    }
    free(narrow);
  }

  if ((uint32_t)threads > p->rows) threads = (int)p->rows;
  pthread_t *tids = (pthread_t *)calloc((size_t)threads, sizeof(pthread_t));
  char *running = (char *)calloc((size_t)threads, 1);
  gemm_job *jobs = (gemm_job *)calloc((size_t)threads, sizeof(gemm_job));
  const uint32_t per = (p->rows + (uint32_t)threads - 1) / (uint32_t)threads;
  for (int t = 0; t < threads; ++t) {
    jobs[t].args = p;
    jobs[t].mode = mode;
    jobs[t].dense = dense;
    jobs[t].row_begin = (uint32_t)t * per;
    jobs[t].row_end = jobs[t].row_begin + per > p->rows ? p->rows
                                                        : jobs[t].row_begin + per;
    if (jobs[t].row_begin >= jobs[t].row_end) continue;
    if (threads > 1 && pthread_create(&tids[t], NULL, gemm_worker, &jobs[t]) == 0)
      running[t] = 1;
    else
      gemm_worker(&jobs[t]); /* single thread, or thread creation failed */
  }
  for (int t = 0; t < threads; ++t)
    if (running[t]) pthread_join(tids[t], NULL);
  free(running);
  free(tids);
  free(jobs);
  free(dense);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Conformer convolution tail (src/webgpu/kernels/conformer-conv.ts:495-573) */
/* ------------------------------------------------------------------------ */

static inline double conv_in(int dtype, const void *p, uint64_t idx) {
  if (dtype == PKO_DTYPE_F16) return pko_f16_to_f64(((const uint16_t *)p)[idx]);
  if (dtype == PKO_DTYPE_F64) return ((const double *)p)[idx];
  return (double)((const float *)p)[idx];
}

/* sigmoid with the reference's clamp: 1 / (1 + exp(-clamp(v, -20, 20))). */
static inline float sigmoid_f32(float v) {
  const float bounded = fminf(fmaxf(v, -20.0f), 20.0f);
  return 1.0f / (1.0f + expf(-bounded));
}
static inline double sigmoid_f64(double v) {
  const double bounded = fmin(fmax(v, -20.0), 20.0);
  return 1.0 / (1.0 + exp(-bounded));
}

int pko_conformer_conv(int dtype, int mode, uint32_t batch, uint32_t frames, uint32_t channels,
                       const void *input, const void *weights, const float *scale,
                       const float *shift, const uint32_t *valid, void *output) {
  enum { TAPS = 9, RADIUS = 4 };
  if (!input || !weights || !scale || !shift || !valid || !output || batch == 0 || frames == 0 ||
      channels == 0 || (dtype != PKO_DTYPE_F16 && dtype != PKO_DTYPE_F32 && dtype != PKO_DTYPE_F64) ||
      (mode != PKO_MODE_F32_CHAIN && mode != PKO_MODE_F64))
    return 1;
  const uint64_t in_row = 2ull * channels;
  for (uint32_t b = 0; b < batch; ++b) {
    for (uint32_t f = 0; f < frames; ++f) {
      for (uint32_t c = 0; c < channels; ++c) {
        float sum32 = 0.0f;
        double sum64 = 0.0;
        for (int k = 0; k < TAPS; ++k) {
          /* GLU of frame f - 4 + k, zero outside [0, frames) and past the
             batch item's valid length (conformer-conv.ts:520-540). */
          const int64_t t = (int64_t)f - RADIUS + k;
          double value = 0.0, gate = 0.0;
          const int live = t >= 0 && t < (int64_t)frames && t < (int64_t)valid[b];
          if (live) {
            const uint64_t row = (uint64_t)b * frames + (uint64_t)t;
            value = conv_in(dtype, input, row * in_row + c);
            gate = conv_in(dtype, input, row * in_row + channels + c);
          }
          const double w = conv_in(dtype, weights, (uint64_t)k * channels + c);
          if (mode == PKO_MODE_F32_CHAIN) {
            const float glu = live ? (float)value * sigmoid_f32((float)gate) : 0.0f;
            sum32 = fmaf(glu, (float)w, sum32);
          } else {
            const double glu = live ? value * sigmoid_f64(gate) : 0.0;
            sum64 += glu * w;
          }
        }
        double activated;
        if (mode == PKO_MODE_F32_CHAIN) {
          const float affine = sum32 * scale[c] + shift[c];
          activated = (double)(affine * sigmoid_f32(affine));
        } else {
          const double affine = sum64 * (double)scale[c] + (double)shift[c];
          activated = affine * sigmoid_f64(affine);
        }
        const uint64_t out_idx = ((uint64_t)b * frames + f) * channels + c;
        if (dtype == PKO_DTYPE_F16)
          ((uint16_t *)output)[out_idx] = pko_f64_to_f16(activated);
        else if (dtype == PKO_DTYPE_F64)
          ((double *)output)[out_idx] = activated;
        else
          ((float *)output)[out_idx] = (float)activated;
      }
    }
  }
  return 0;
}

/* GLU alone: the step conformer-conv.ts:520-535 applies to each input row. */
int pko_glu(int dtype, int mode, uint64_t rows, uint32_t channels, const void *input, void *output) {
  if (!input || !output || channels == 0 ||
      (dtype != PKO_DTYPE_F16 && dtype != PKO_DTYPE_F32 && dtype != PKO_DTYPE_F64) ||
      (mode != PKO_MODE_F32_CHAIN && mode != PKO_MODE_F64))
    return 1;
  for (uint64_t r = 0; r < rows; ++r) {
    for (uint32_t c = 0; c < channels; ++c) {
      const double value = conv_in(dtype, input, r * 2u * channels + c);
      const double gate = conv_in(dtype, input, r * 2u * channels + channels + c);
      const double glu = mode == PKO_MODE_F32_CHAIN ? (double)((float)value * sigmoid_f32((float)gate))
                                                    : value * sigmoid_f64(gate);
      const uint64_t at = r * channels + c;
      if (dtype == PKO_DTYPE_F16)
        ((uint16_t *)output)[at] = pko_f64_to_f16(glu);
      else if (dtype == PKO_DTYPE_F64)
        ((double *)output)[at] = glu;
      else
        ((float *)output)[at] = (float)glu;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Relative-position attention (src/webgpu/kernels/attention.ts:418-727)     */
/* ------------------------------------------------------------------------ */

static inline void store_out(int dtype, void *p, uint64_t idx, double v) {
  if (dtype == PKO_DTYPE_F16)
    ((uint16_t *)p)[idx] = pko_f64_to_f16(v);
  else if (dtype == PKO_DTYPE_F64)
    ((double *)p)[idx] = v;
  else
    ((float *)p)[idx] = (float)v;
}

int pko_relative_attention(int dtype, int mode, uint32_t batch, uint32_t frames, const void *qkv,
                           const void *positions, const float *bias_u, const float *bias_v,
                           const uint32_t *valid, void *out) {
  enum { HEADS = 8, HEAD = 128, HIDDEN = 1024 };
  if (!qkv || !positions || !bias_u || !bias_v || !valid || !out || batch == 0 || frames == 0 ||
      (dtype != PKO_DTYPE_F16 && dtype != PKO_DTYPE_F32 && dtype != PKO_DTYPE_F64) ||
      (mode != PKO_MODE_F32_CHAIN && mode != PKO_MODE_F64))
    return 1;
  const uint64_t T = frames, P = 2ull * frames - 1u;
  const int f32 = mode == PKO_MODE_F32_CHAIN;
  const float scale32 = (float)(1.0 / sqrt(128.0));
  const double scale64 = 1.0 / sqrt(128.0);
  /* one (window, head) at a time, its operands decoded once */
  double *q = (double *)malloc(sizeof(double) * T * HEAD), *k = (double *)malloc(sizeof(double) * T * HEAD);
  double *v = (double *)malloc(sizeof(double) * T * HEAD), *r = (double *)malloc(sizeof(double) * P * HEAD);
  double *s = (double *)malloc(sizeof(double) * T);
  if (!q || !k || !v || !r || !s) {
    free(q), free(k), free(v), free(r), free(s);
    return 1;
  }
  for (uint32_t b = 0; b < batch; ++b) {
    const uint64_t live = valid[b] < frames ? valid[b] : frames;
    for (uint32_t h = 0; h < HEADS; ++h) {
      for (uint64_t t = 0; t < T; ++t)
        for (uint32_t d = 0; d < HEAD; ++d) {
          const uint64_t row = ((uint64_t)b * T + t) * 3u * HIDDEN + h * HEAD + d;
          q[t * HEAD + d] = conv_in(dtype, qkv, row);
          k[t * HEAD + d] = conv_in(dtype, qkv, row + HIDDEN);
          v[t * HEAD + d] = conv_in(dtype, qkv, row + 2u * HIDDEN);
        }
      /* head-vector-position-vec4: [h][d / 4][p][d % 4] */
      for (uint64_t p = 0; p < P; ++p)
        for (uint32_t d = 0; d < HEAD; ++d)
          r[p * HEAD + d] = conv_in(dtype, positions, (((uint64_t)h * 32u + d / 4u) * P + p) * 4u + d % 4u);
      const float *u = bias_u + h * HEAD, *w = bias_v + h * HEAD;
      for (uint64_t i = 0; i < T; ++i) {
        const uint64_t qrow = (uint64_t)b * T + i;
        if (i >= live) {
          for (uint32_t d = 0; d < HEAD; ++d) store_out(dtype, out, qrow * HIDDEN + h * HEAD + d, 0.0);
          continue;
        }
        const double *qi = q + i * HEAD;
        /* scores of the live keys */
        double maximum = -HUGE_VAL;
        for (uint64_t j = 0; j < live; ++j) {
          const double *kj = k + j * HEAD, *rj = r + (T - 1u - i + j) * HEAD;
          if (f32) {
            float acc = 0.0f;
            for (uint32_t d = 0; d < HEAD; ++d) {
              acc = fmaf((float)qi[d] + u[d], (float)kj[d], acc);
              acc = fmaf((float)qi[d] + w[d], (float)rj[d], acc);
            }
            s[j] = (double)(acc * scale32);
          } else {
            double acc = 0.0;
            for (uint32_t d = 0; d < HEAD; ++d) acc += (qi[d] + u[d]) * kj[d] + (qi[d] + w[d]) * rj[d];
            s[j] = acc * scale64;
          }
          if (s[j] > maximum) maximum = s[j];
        }
        /* softmax */
        if (f32) {
          float sum = 0.0f;
          for (uint64_t j = 0; j < live; ++j) {
            const float e = expf((float)s[j] - (float)maximum);
            s[j] = e;
            sum += e;
          }
          const float inverse = 1.0f / sum;
          for (uint64_t j = 0; j < live; ++j) s[j] = (double)((float)s[j] * inverse);
        } else {
          double sum = 0.0;
          for (uint64_t j = 0; j < live; ++j) sum += (s[j] = exp(s[j] - maximum));
          for (uint64_t j = 0; j < live; ++j) s[j] /= sum;
        }
        /* context */
        for (uint32_t d = 0; d < HEAD; ++d) {
          double o;
          if (f32) {
            float acc = 0.0f;
            for (uint64_t j = 0; j < live; ++j) acc = fmaf((float)s[j], (float)v[j * HEAD + d], acc);
            o = acc;
          } else {
            o = 0.0;
            for (uint64_t j = 0; j < live; ++j) o += s[j] * v[j * HEAD + d];
          }
          store_out(dtype, out, qrow * HIDDEN + h * HEAD + d, o);
        }
      }
    }
  }
  free(q), free(k), free(v), free(r), free(s);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* LayerNorm (src/webgpu/kernels/layernorm.ts:309-390)                        */
/* ------------------------------------------------------------------------ */

int pko_layernorm(int dtype, int mode, uint64_t rows, uint32_t channels, const void *input, const float *gamma,
                  const float *beta, float epsilon, void *output) {
  if (!input || !gamma || !beta || !output || channels == 0 ||
      (dtype != PKO_DTYPE_F16 && dtype != PKO_DTYPE_F32 && dtype != PKO_DTYPE_F64) ||
      (mode != PKO_MODE_F32_CHAIN && mode != PKO_MODE_F64))
    return 1;
  for (uint64_t r = 0; r < rows; ++r) {
    const uint64_t base = r * channels;
    if (mode == PKO_MODE_F32_CHAIN) {
      float sum = 0.0f, square = 0.0f;
      for (uint32_t c = 0; c < channels; ++c) {
        const float x = (float)conv_in(dtype, input, base + c);
        sum += x;
        square = fmaf(x, x, square);
      }
      const float inverse_channels = 1.0f / (float)channels;
      const float mean = sum * inverse_channels;
      const float variance = fmaxf(square * inverse_channels - mean * mean, 0.0f);
      const float inverse_std = 1.0f / sqrtf(variance + epsilon);
      for (uint32_t c = 0; c < channels; ++c) {
        const float x = (float)conv_in(dtype, input, base + c);
        store_out(dtype, output, base + c, (double)((x - mean) * inverse_std * gamma[c] + beta[c]));
      }
    } else {
      double sum = 0.0, square = 0.0;
      for (uint32_t c = 0; c < channels; ++c) {
        const double x = conv_in(dtype, input, base + c);
        sum += x;
        square += x * x;
      }
      const double mean = sum / channels;
      const double variance = fmax(square / channels - mean * mean, 0.0);
      const double inverse_std = 1.0 / sqrt(variance + (double)epsilon);
      for (uint32_t c = 0; c < channels; ++c)
        store_out(dtype, output, base + c,
                  (conv_in(dtype, input, base + c) - mean) * inverse_std * gamma[c] + beta[c]);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Subsampling front end (src/webgpu/kernels/subsampling.ts)                 */
/* ------------------------------------------------------------------------ */

/* fused_subsampled_length / subsampled_length (subsampling.ts:1115-1121,
   :1283-1289). */
uint32_t pko_subsampled_length(uint32_t length, uint32_t steps) {
  for (uint32_t s = 0; s < steps; ++s) length = (uint32_t)(((uint64_t)length + 1u) / 2u);
  return length;
}

/* One accumulation step in the storage type's arithmetic: fmaf for the f16
   and f32 profiles (WGSL fma on vec4<f32>), fma in double for the f64 twin. */
static inline double acc_step(int dtype, double a, double b, double sum) {
  if (dtype == PKO_DTYPE_F64) return fma(a, b, sum);
  return (double)fmaf((float)a, (float)b, (float)sum);
}

/* Round an intermediate to the storage type (f16 tile, f32 tile, double). */
static inline double to_storage(int dtype, double v) {
  if (dtype == PKO_DTYPE_F16) return pko_round_f16(v);
  if (dtype == PKO_DTYPE_F32) return (double)(float)v;
  return v;
}

int pko_subsampling_fused(int dtype, uint32_t batch, uint32_t height, uint32_t width, uint32_t channels,
                          const float *input, const void *conv0_weights, const float *conv0_bias,
                          const void *depthwise_weights, const float *depthwise_bias, const uint32_t *valid,
                          void *output) {
  if (!input || !conv0_weights || !conv0_bias || !depthwise_weights || !depthwise_bias || !valid || !output ||
      height == 0 || width == 0 || channels == 0 ||
      (dtype != PKO_DTYPE_F16 && dtype != PKO_DTYPE_F32 && dtype != PKO_DTYPE_F64))
    return 1;
  const uint32_t h1 = pko_subsampled_length(height, 1), w1 = pko_subsampled_length(width, 1);
  const uint32_t ho = pko_subsampled_length(h1, 1), wo = pko_subsampled_length(w1, 1);
  double *conv0 = (double *)malloc(sizeof(double) * (uint64_t)h1 * w1 * channels);
  if (!conv0) return 1;
  for (uint32_t b = 0; b < batch; ++b) {
    const uint32_t valid1 = pko_subsampled_length(valid[b], 1), valid2 = pko_subsampled_length(valid[b], 2);
    /* conv0 + ReLU, stored in the tile's type (subsampling.ts:1152-1201) */
    for (uint32_t y = 0; y < h1; ++y)
      for (uint32_t x = 0; x < w1; ++x)
        for (uint32_t c = 0; c < channels; ++c) {
          double v = 0.0;
          if (y < valid1) {
            double sum = conv0_bias[c];
            for (int ky = 0; ky < 3; ++ky) {
              const int iy = (int)y * 2 + ky - 1;
              if (iy < 0 || iy >= (int)height) continue;
              for (int kx = 0; kx < 3; ++kx) {
                const int ix = (int)x * 2 + kx - 1;
                if (ix < 0 || ix >= (int)width) continue;
                const double w = conv_in(dtype, conv0_weights, ((uint64_t)ky * 3 + kx) * channels + c);
                const double f = input[((uint64_t)b * width + (uint32_t)ix) * height + (uint32_t)iy];
                sum = acc_step(dtype, w, f, sum);
              }
            }
            v = to_storage(dtype, sum > 0.0 ? sum : 0.0);
          }
          conv0[((uint64_t)y * w1 + x) * channels + c] = v;
        }
    /* depthwise2 (subsampling.ts:1205-1238) */
    for (uint32_t y = 0; y < ho; ++y)
      for (uint32_t x = 0; x < wo; ++x)
        for (uint32_t c = 0; c < channels; ++c) {
          const uint64_t out_idx = (((uint64_t)b * ho + y) * wo + x) * channels + c;
          if (y >= valid2) {
            store_out(dtype, output, out_idx, 0.0);
            continue;
          }
          double sum = depthwise_bias[c];
          for (int ky = 0; ky < 3; ++ky) {
            const int iy = (int)y * 2 + ky - 1;
            if (iy < 0 || iy >= (int)h1 || iy >= (int)valid1) continue;
            for (int kx = 0; kx < 3; ++kx) {
              const int ix = (int)x * 2 + kx - 1;
              if (ix < 0 || ix >= (int)w1) continue;
              const double w = conv_in(dtype, depthwise_weights, ((uint64_t)ky * 3 + kx) * channels + c);
              sum = acc_step(dtype, conv0[((uint64_t)iy * w1 + (uint32_t)ix) * channels + c], w, sum);
            }
          }
          store_out(dtype, output, out_idx, sum);
        }
  }
  free(conv0);
  return 0;
}

int pko_subsampling_depthwise(int dtype, uint32_t batch, uint32_t height, uint32_t width, uint32_t channels,
                              const void *input, const void *weights, const float *bias, const uint32_t *valid,
                              uint32_t steps, void *output) {
  if (!input || !weights || !bias || !valid || !output || height == 0 || width == 0 || channels == 0 ||
      steps == 0 || (dtype != PKO_DTYPE_F16 && dtype != PKO_DTYPE_F32 && dtype != PKO_DTYPE_F64))
    return 1;
  const uint32_t ho = pko_subsampled_length(height, 1), wo = pko_subsampled_length(width, 1);
  for (uint32_t b = 0; b < batch; ++b) {
    const uint32_t valid_in = pko_subsampled_length(valid[b], steps - 1);
    const uint32_t valid_out = pko_subsampled_length(valid[b], steps);
    for (uint32_t y = 0; y < ho; ++y)
      for (uint32_t x = 0; x < wo; ++x)
        for (uint32_t c = 0; c < channels; ++c) {
          const uint64_t out_idx = (((uint64_t)b * ho + y) * wo + x) * channels + c;
          if (y >= valid_out) {
            store_out(dtype, output, out_idx, 0.0);
            continue;
          }
          double sum = bias[c];
          for (int ky = 0; ky < 3; ++ky) {
            const int iy = (int)y * 2 + ky - 1;
            if (iy < 0 || iy >= (int)height || iy >= (int)valid_in) continue;
            for (int kx = 0; kx < 3; ++kx) {
              const int ix = (int)x * 2 + kx - 1;
              if (ix < 0 || ix >= (int)width) continue;
              const double v =
                  conv_in(dtype, input, (((uint64_t)b * height + (uint32_t)iy) * width + (uint32_t)ix) * channels + c);
              sum = acc_step(dtype, v, conv_in(dtype, weights, ((uint64_t)ky * 3 + kx) * channels + c), sum);
            }
          }
          store_out(dtype, output, out_idx, sum);
        }
  }
  return 0;
}

int pko_subsampling_mask(int dtype, uint32_t batch, uint32_t height, uint32_t width, uint32_t channels,
                         void *values, const uint32_t *valid, uint32_t steps) {
  if (!values || !valid || (dtype != PKO_DTYPE_F16 && dtype != PKO_DTYPE_F32 && dtype != PKO_DTYPE_F64)) return 1;
  const uint64_t frame = (uint64_t)width * channels;
  for (uint32_t b = 0; b < batch; ++b) {
    const uint32_t keep = pko_subsampled_length(valid[b], steps);
    for (uint32_t y = keep; y < height; ++y)
      for (uint64_t i = 0; i < frame; ++i) store_out(dtype, values, ((uint64_t)b * height + y) * frame + i, 0.0);
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Greedy TDT decoder (src/webgpu/kernels/tdt-decoder.ts:1133-2010)          */
/* ------------------------------------------------------------------------ */

/* binary16 neighbours of v: *lo <= v <= *hi (equal when v is one). */
static void f16_bracket(double v, double *lo, double *hi) {
  const uint16_t bits = pko_f64_to_f16(v);
  const double r = pko_f16_to_f64(bits);
  if (r == v || isinf(r) || isnan(r)) {
    *lo = *hi = r;
    return;
  }
  /* the neighbour on the other side of v: one step in magnitude */
  uint16_t other_bits;
  if ((r > v) == !(bits & 0x8000u)) /* r above v in magnitude: step toward zero */
    other_bits = (bits & 0x7fffu) ? (uint16_t)(bits - 1u) : (uint16_t)(bits ^ 0x8000u);
  else
    other_bits = (uint16_t)(bits + 1u);
  const double o = pko_f16_to_f64(other_bits);
  *lo = r < o ? r : o;
  *hi = r < o ? o : r;
}

/* fma in binary16 with one rounding: round16(a * b + c) for binary16 a, b,
   c. a * b is exact in double; the double sum s plus its error e (TwoSum)
   is the exact value, and e only decides the rounding when s sits exactly
   on a binary16 midpoint. */
static double fma16(double a, double b, double c) {
  const double p = a * b;
  const double s = p + c;
  const double t = s - p;
  const double e = (p - (s - t)) + (c - t);
  if (e == 0.0 || isinf(s)) return pko_round_f16(s);
  double lo, hi;
  f16_bracket(s, &lo, &hi);
  if (lo != hi && s == lo + (hi - lo) / 2.0) return e > 0.0 ? hi : lo;
  return pko_round_f16(s);
}

float pko_exp_f32(float x) {
  /* n = rint(x / ln2); r = x - n ln2 with ln2 = 0.693145751953125 (exact in
     f32, 12 bits) + 1.42860682030941723212e-6; e^r = sum r^i / i!, i <= 7
     (|r| <= 0.347: truncation below 2^-27 relative). */
  const float log2e = 1.44269502f;
  const float ln2_hi = 0.693145751953125f;
  const float ln2_lo = 1.42860682030941723212e-6f;
  const float n = rintf(x * log2e);
  float r = fmaf(-n, ln2_hi, x);
  r = fmaf(-n, ln2_lo, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int32_t ni = (int32_t)n;
  uint32_t scale_bits = (uint32_t)(ni + 127) << 23;
  float scale;
  memcpy(&scale, &scale_bits, sizeof scale);
  return p * scale;
}

float pko_tanh_f32(float x) {
  const float a = fabsf(x);
  const float t = 1.0f - 2.0f / (pko_exp_f32(2.0f * a) + 1.0f);
  return x < 0.0f ? -t : t;
}

/* 1 / (1 + exp(-clamp(v, -20, 20))) (tdt-decoder.ts:1309-1311). */
static float tdt_sigmoid(float v) {
  const float bounded = fminf(fmaxf(v, -20.0f), 20.0f);
  return 1.0f / (1.0f + pko_exp_f32(-bounded));
}

/* tanh(clamp(v, -10, 10)) (tdt-decoder.ts:1318-1322). */
static float tdt_tanh(float v) { return pko_tanh_f32(fminf(fmaxf(v, -10.0f), 10.0f)); }

/* The decoder's weights widened to double once per call (exact for f16 and
   f32 values); f32 selects the f32 profile's chains. */
typedef struct tdt_dense {
  double *embedding, *lstm[2], *projector, *head;
  const float *lstm_bias[2], *projector_bias, *head_bias;
  int f32;
} tdt_dense;

static double *widen(const void *src, uint64_t count, int f32) {
  double *out = (double *)malloc(sizeof(double) * count);
  if (out)
    for (uint64_t i = 0; i < count; ++i)
      out[i] = f32 ? (double)((const float *)src)[i] : pko_f16_to_f64(((const uint16_t *)src)[i]);
  return out;
}

/* Element i of a row in the profile's element, as a double. */
static double tdt_element(const void *row, uint64_t i, int f32) {
  return f32 ? (double)((const float *)row)[i] : pko_f16_to_f64(((const uint16_t *)row)[i]);
}

/* One step of a chain: fma with one rounding in the profile's format. */
static double tdt_fma(double a, double b, double c, int f32) {
  return f32 ? (double)fmaf((float)a, (float)b, (float)c) : fma16(a, b, c);
}

/* A chain input or a bias as the chain sees it (rounded to f16 in the f16
   profile, the f32 value in the f32 profile). */
static double tdt_input(float v, int f32) { return f32 ? (double)v : pko_round_f16((double)v); }

static void tdt_dense_free(tdt_dense *d) {
  free(d->embedding);
  free(d->lstm[0]);
  free(d->lstm[1]);
  free(d->projector);
  free(d->head);
}

static int tdt_dense_make(const pko_tdt_weights *w, tdt_dense *d) {
  const uint64_t H = PKO_TDT_HIDDEN;
  memset(d, 0, sizeof *d);
  const int f32 = w->f32 != 0;
  d->f32 = f32;
  d->embedding = widen(w->embedding, (uint64_t)PKO_TDT_TOKENS * H, f32);
  d->lstm[0] = widen(w->lstm_weight[0], 2 * H * PKO_TDT_GATES, f32);
  d->lstm[1] = widen(w->lstm_weight[1], 2 * H * PKO_TDT_GATES, f32);
  d->projector = widen(w->projector_weight, H * H, f32);
  d->head = widen(w->head_weight, H * PKO_TDT_HEAD, f32);
  d->lstm_bias[0] = w->lstm_bias[0];
  d->lstm_bias[1] = w->lstm_bias[1];
  d->projector_bias = w->projector_bias;
  d->head_bias = w->head_bias;
  if (!d->embedding || !d->lstm[0] || !d->lstm[1] || !d->projector || !d->head) {
    tdt_dense_free(d);
    return 1;
  }
  return 0;
}

/* One LSTM layer's gates (tdt-decoder.ts:1341-1382, accumulators :572-686
   in f16, :595-614 and :642-666 in f32): per gate a chain over even k
   starting at the bias and one over odd k starting at 0, fma in increasing
   k, the two added at the end, all in the profile's format (the bias
   rounded to f16 in the f16 profile). x[k] is the chain input of row k;
   `limit` rows are used (0: none). */
static void tdt_gates(const double *weight, const float *bias, const double *x, uint32_t limit, float *gates,
                      int f32) {
  double even[PKO_TDT_GATES], odd[PKO_TDT_GATES];
  for (uint32_t j = 0; j < PKO_TDT_GATES; ++j) {
    even[j] = tdt_input(bias[j], f32);
    odd[j] = 0.0;
  }
  for (uint32_t k = 0; k < limit; k += 2) {
    const double *we = weight + (uint64_t)k * PKO_TDT_GATES, *wo = we + PKO_TDT_GATES;
    const double xe = x[k], xo = x[k + 1];
    for (uint32_t j = 0; j < PKO_TDT_GATES; ++j) {
      even[j] = tdt_fma(xe, we[j], even[j], f32);
      odd[j] = tdt_fma(xo, wo[j], odd[j], f32);
    }
  }
  for (uint32_t j = 0; j < PKO_TDT_GATES; ++j)
    gates[j] = f32 ? (float)even[j] + (float)odd[j] : (float)pko_round_f16(even[j] + odd[j]);
}

/* Cell update (tdt-decoder.ts:1384-1410) into h, c. */
static void tdt_cell(const float *gates, const float *c_prev, float *h, float *c) {
  for (uint32_t ch = 0; ch < PKO_TDT_HIDDEN; ++ch) {
    const float ig = tdt_sigmoid(gates[ch]);
    const float fg = tdt_sigmoid(gates[PKO_TDT_HIDDEN + ch]);
    const float gg = tdt_tanh(gates[2 * PKO_TDT_HIDDEN + ch]);
    const float og = tdt_sigmoid(gates[3 * PKO_TDT_HIDDEN + ch]);
    const float cell = fmaf(fg, c_prev[ch], ig * gg);
    c[ch] = cell;
    h[ch] = og * tdt_tanh(cell);
  }
}

static void tdt_predictor(const tdt_dense *w, uint32_t token, int initial, const float *state, float *cand) {
  const uint32_t H = PKO_TDT_HIDDEN;
  double x[2 * PKO_TDT_HIDDEN];
  float gates[PKO_TDT_GATES];
  const int f32 = w->f32;
  /* layer 0: [embedding(token); h0], skipped for the start token (zero x, h) */
  for (uint32_t k = 0; k < H; ++k) {
    x[k] = initial ? 0.0 : w->embedding[(uint64_t)token * H + k];
    x[H + k] = tdt_input(state[k], f32);
  }
  tdt_gates(w->lstm[0], w->lstm_bias[0], x, initial ? 0 : 2 * H, gates, f32);
  tdt_cell(gates, state + H, cand, cand + H);
  /* layer 1: [candidate h0; h1]; the start token uses candidate h0 only */
  for (uint32_t k = 0; k < H; ++k) {
    x[k] = tdt_input(cand[k], f32);
    x[H + k] = tdt_input(state[2 * H + k], f32);
  }
  tdt_gates(w->lstm[1], w->lstm_bias[1], x, initial ? H : 2 * H, gates, f32);
  tdt_cell(gates, state + 3 * H, cand + 2 * H, cand + 3 * H);
  /* decoder projector in f32 (tdt-decoder.ts:1462-1491) */
  for (uint32_t o = 0; o < H; ++o) {
    float acc = w->projector_bias[o];
    for (uint32_t k = 0; k < H; ++k) acc = fmaf(cand[2 * H + k], (float)w->projector[(uint64_t)k * H + o], acc);
    cand[4 * H + o] = acc;
  }
}

static float sanitize_score(float v) { return v != v ? -3.402823466e+38f : v; }

static void tdt_joint(const tdt_dense *w, const void *encoder_row, const float *projection, float *scores,
                      uint32_t *token, uint32_t *duration) {
  const uint32_t H = PKO_TDT_HIDDEN;
  const int f32 = w->f32;
  double acc[PKO_TDT_HEAD];
  float joint[PKO_TDT_HIDDEN];
  for (uint32_t c = 0; c < H; ++c) {
    const float v = (float)tdt_element(encoder_row, c, f32) + projection[c];
    joint[c] = v > 0.0f ? v : 0.0f; /* max(v, 0) */
  }
  for (uint32_t o = 0; o < PKO_TDT_HEAD; ++o) acc[o] = tdt_input(w->head_bias[o], f32);
  /* chains in increasing k in the profile's format; exact +0 inputs skipped
     until a -0 or NaN input has been seen (tdt-decoder.ts:977-1031 in f16,
     :877-919 and :1033-1058 in f32) */
  int zero_skip_safe = 1;
  for (uint32_t k = 0; k < H; ++k) {
    uint32_t bits;
    memcpy(&bits, &joint[k], sizeof bits);
    const int is_nan = (bits & 0x7fffffffu) > 0x7f800000u;
    const int exceptional = bits == 0x80000000u || is_nan;
    zero_skip_safe = zero_skip_safe && !exceptional;
    if (zero_skip_safe && bits == 0u) continue;
    const double x = tdt_input(joint[k], f32);
    const double *row = w->head + (uint64_t)k * PKO_TDT_HEAD;
    for (uint32_t o = 0; o < PKO_TDT_HEAD; ++o) acc[o] = tdt_fma(x, row[o], acc[o], f32);
  }
  /* argmax over tokens and blank, then over durations: the largest value,
     the lowest id among equal values (choose_better, :1517-1525) */
  uint32_t best = 0xffffffffu, best_d = 0xffffffffu;
  float best_v = -3.402823466e+38f, best_dv = -3.402823466e+38f;
  for (uint32_t o = 0; o < PKO_TDT_HEAD; ++o) {
    const float v = sanitize_score((float)acc[o]);
    if (scores) scores[o] = (float)acc[o];
    if (o <= PKO_TDT_BLANK) {
      if (v > best_v || (v == best_v && o < best)) {
        best_v = v;
        best = o;
      }
    } else if (o < PKO_TDT_BLANK + 1 + PKO_TDT_DURATIONS) {
      const uint32_t d = o - PKO_TDT_BLANK - 1;
      if (v > best_dv || (v == best_dv && d < best_d)) {
        best_dv = v;
        best_d = d;
      }
    }
  }
  *token = best;
  *duration = best_d;
}

void pko_tdt_predictor(const pko_tdt_weights *w, uint32_t token, int initial, const float *state, float *cand) {
  tdt_dense d;
  if (tdt_dense_make(w, &d)) return;
  tdt_predictor(&d, token, initial, state, cand);
  tdt_dense_free(&d);
}

void pko_tdt_joint(const pko_tdt_weights *w, const void *encoder_row, const float *projection, float *scores,
                   uint32_t *token, uint32_t *duration) {
  tdt_dense d;
  if (tdt_dense_make(w, &d)) return;
  tdt_joint(&d, encoder_row, projection, scores, token, duration);
  tdt_dense_free(&d);
}

typedef struct tdt_job {
  const tdt_dense *w;
  uint32_t b, frames, max_tokens;
  const void *encoder_projected;
  const uint32_t *lengths, *starts, *ends, *flush;
  float *state_all, *scratch_all;
  uint32_t *tokens, *token_frames, *token_durations, *counts, *status;
} tdt_job;

/* The decode of one window (tdt-decoder.ts:1664-2010). */
static void tdt_decode_window(const tdt_job *j) {
  const uint32_t H = PKO_TDT_HIDDEN, b = j->b, frames = j->frames, max_tokens = j->max_tokens;
  const tdt_dense *w = j->w;
  float *state = j->state_all + (uint64_t)b * 4 * H;
  float *cand = j->scratch_all + (uint64_t)b * 5 * H;
  const size_t element = w->f32 ? 4 : 2;
  const unsigned char *enc = (const unsigned char *)j->encoder_projected + (uint64_t)b * frames * H * element;
  memset(state, 0, sizeof(float) * 4 * H);
  uint32_t count = 0, st = 0, symbols = 0;
  const uint32_t limit = j->lengths[b] < frames ? j->lengths[b] : frames;
  const uint32_t encoded = limit < j->ends[b] ? limit : j->ends[b];
  uint32_t time = j->starts[b] < encoded ? j->starts[b] : encoded;
  uint32_t token = 0, duration = 0;
  if (time < encoded) tdt_predictor(w, 0, 1, state, cand);
  /* emission and the predictor update after a non-blank (:1740-1810) */
#define TDT_EMIT(frame_value)                                                          \
  do {                                                                                 \
    if (count < max_tokens) {                                                          \
      const uint64_t at = (uint64_t)b * max_tokens + count;                            \
      j->tokens[at] = token;                                                           \
      j->token_frames[at] = (frame_value);                                             \
      j->token_durations[at] = duration;                                               \
      ++count;                                                                         \
    } else {                                                                           \
      st |= PKO_TDT_OVERFLOW;                                                          \
    }                                                                                  \
  } while (0)
#define TDT_ADVANCE_PREDICTOR()                    \
  do {                                             \
    memcpy(state, cand, sizeof(float) * 4 * H);    \
    tdt_predictor(w, token, 0, state, cand);       \
  } while (0)
  while (time < encoded) {
    tdt_joint(w, enc + (uint64_t)time * H * element, cand + 4 * H, NULL, &token, &duration);
    const int emitted = token != PKO_TDT_BLANK;
    if (emitted) TDT_EMIT(time);
    symbols += 1;
    if (duration != 0) {
      time += duration;
      symbols = 0;
    } else if (!emitted || symbols >= 10) {
      time += 1;
      symbols = 0;
    }
    if (emitted) TDT_ADVANCE_PREDICTOR();
  }
  /* bounded end-of-stream flush (:1812-1998) */
  if (j->flush[b] != 0 && j->starts[b] < encoded) {
    uint32_t flush_blanks = 0, flush_time = time;
    symbols = 0;
    while (symbols < 10 && flush_blanks < 5) {
      const uint32_t variation = symbols % 3;
      if (variation == 0) {
        const uint32_t last = limit - 1u;
        time = flush_time < last ? flush_time : last;
      } else if (variation == 1) {
        time = encoded - 1u < frames - 1u ? encoded - 1u : frames - 1u;
      } else {
        const uint32_t m = (encoded > 2u ? encoded : 2u) - 2u;
        time = m < frames - 1u ? m : frames - 1u;
      }
      tdt_joint(w, enc + (uint64_t)time * H * element, cand + 4 * H, NULL, &token, &duration);
      const int emitted = token != PKO_TDT_BLANK;
      if (!emitted) {
        flush_blanks += 1;
      } else {
        flush_blanks = 0;
        TDT_EMIT(flush_time < encoded - 1u ? flush_time : encoded - 1u);
      }
      const uint32_t step = duration > 1u ? duration : 1u;
      flush_time = flush_time + step < encoded ? flush_time + step : encoded;
      symbols += 1;
      if (emitted) TDT_ADVANCE_PREDICTOR();
    }
  }
#undef TDT_EMIT
#undef TDT_ADVANCE_PREDICTOR
  j->counts[b] = count;
  j->status[b] = st;
}

static void *tdt_worker(void *opaque) {
  tdt_decode_window((const tdt_job *)opaque);
  return NULL;
}

int pko_tdt_decode(const pko_tdt_weights *w, uint32_t batch, uint32_t frames, uint32_t max_tokens,
                   const void *encoder_projected, const uint32_t *lengths, const uint32_t *starts,
                   const uint32_t *ends, const uint32_t *flush, float *state_all, float *scratch_all,
                   uint32_t *tokens, uint32_t *token_frames, uint32_t *token_durations, uint32_t *counts,
                   uint32_t *status) {
  if (!w || !encoder_projected || !lengths || !starts || !ends || !flush || !state_all || !scratch_all || !tokens ||
      !token_frames || !token_durations || !counts || !status || frames == 0 || max_tokens == 0)
    return 1;
  tdt_dense d;
  if (tdt_dense_make(w, &d)) return 1;
  /* windows are independent: one thread each */
  tdt_job *jobs = (tdt_job *)calloc(batch ? batch : 1, sizeof(tdt_job));
  pthread_t *tids = (pthread_t *)calloc(batch ? batch : 1, sizeof(pthread_t));
  char *running = (char *)calloc(batch ? batch : 1, 1);
  for (uint32_t b = 0; b < batch; ++b) {
    tdt_job j = {&d, b, frames, max_tokens, encoder_projected, lengths, starts, ends, flush, state_all,
                 scratch_all, tokens, token_frames, token_durations, counts, status};
    jobs[b] = j;
    if (pthread_create(&tids[b], NULL, tdt_worker, &jobs[b]) == 0)
      running[b] = 1;
    else
      tdt_decode_window(&jobs[b]);
  }
  for (uint32_t b = 0; b < batch; ++b)
    if (running[b]) pthread_join(tids[b], NULL);
  free(running);
  free(tids);
  free(jobs);
  tdt_dense_free(&d);
  return 0;
}

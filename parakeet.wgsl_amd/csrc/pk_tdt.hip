// pk_tdt.hip - greedy TDT decoding for gfx950 (reference:
// src/webgpu/kernels/tdt-decoder.ts, shader :1133-2010).
//
// One workgroup of 640 threads decodes one window: the two-layer LSTM
// predictor (one thread per four gates, the 1280 inputs staged in LDS as
// f16), the f32 cell update, the f32 decoder projector, the ReLU joint and
// the f16 vocabulary head (one thread per four outputs), the lowest-id
// argmax, and the duration / 10-symbol / flush control in thread 0, all
// without leaving the kernel. The predictor runs only after a non-blank
// emission, as in the reference.
//
// Arithmetic is the shader's, term for term: every gate is an f16 chain
// over even rows starting at f16(bias) plus one over odd rows starting at
// zero, fma in increasing k (v_pk_fma_f16, one rounding), added in f16; the
// head is an f16 chain over k skipping exact +0 joint inputs until a -0 or
// NaN input is seen; the projector is an f32 fma chain; the cell update and
// the activations are f32 with exp written out (range reduction and a
// degree-7 Taylor polynomial) rather than taken from a library, so the
// decode is reproducible to the bit. Contraction is off in this file: every
// fused multiply-add is written as one.
#include "pk_internal.h"

#pragma clang fp contract(off)

namespace pk {
namespace {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));

constexpr uint32_t H = kTdtHidden;
constexpr uint32_t kThreads = kTdtThreads;

__device__ __forceinline__ float exp_f32(float x) {
  const float log2e = 1.44269502f;
  const float ln2_hi = 0.693145751953125f;
  const float ln2_lo = 1.42860682030941723212e-6f;
  const float n = __builtin_rintf(x * log2e);
  float r = __builtin_fmaf(-n, ln2_hi, x);
  r = __builtin_fmaf(-n, ln2_lo, r);
  float p = 1.0f / 5040.0f;
  p = __builtin_fmaf(p, r, 1.0f / 720.0f);
  p = __builtin_fmaf(p, r, 1.0f / 120.0f);
  p = __builtin_fmaf(p, r, 1.0f / 24.0f);
  p = __builtin_fmaf(p, r, 1.0f / 6.0f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const float scale = __uint_as_float((uint32_t)(ni + 127) << 23);
  return p * scale;
}

__device__ __forceinline__ float tanh_f32(float x) {
  const float a = fabsf(x);
  const float t = 1.0f - 2.0f / (exp_f32(2.0f * a) + 1.0f);
  return x < 0.0f ? -t : t;
}

__device__ __forceinline__ float sigmoid_f32(float v) {
  const float bounded = fminf(fmaxf(v, -20.0f), 20.0f);
  return 1.0f / (1.0f + exp_f32(-bounded));
}

__device__ __forceinline__ float clamped_tanh(float v) { return tanh_f32(fminf(fmaxf(v, -10.0f), 10.0f)); }

__device__ __forceinline__ half4 splat(_Float16 x) { return half4{x, x, x, x}; }

__device__ __forceinline__ half4 load_half4(const _Float16* p) { return *reinterpret_cast<const half4*>(p); }

struct Shared {
  _Float16 x[2 * H];      // LSTM layer inputs (f16)
  float gates[kTdtGates]; // f32 values of the f16 gate sums
  float joint[H];         // relu(encoder + projection)
  float scores[kTdtHead]; // f32 values of the f16 head accumulators
  // control, written by thread 0
  uint32_t go, emitted, token, duration, joint_time;
};

// Rows of weights loaded before any is used: the k loops are latency
// bound, so each thread keeps this many 8-byte loads in flight.
constexpr uint32_t kBatchRows = 16;

// Gates of one LSTM layer: thread t owns gates 4t..4t+3 over `limit` rows
// (a multiple of kBatchRows).
__device__ void lstm_gates(Shared& s, const _Float16* weight, const float* bias, uint32_t limit) {
  const uint32_t t = threadIdx.x;
  const float4 b = *reinterpret_cast<const float4*>(bias + 4 * t);
  half4 even = half4{(_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
  half4 odd = half4{0, 0, 0, 0};
  const _Float16* column = weight + 4 * t;
  for (uint32_t k0 = 0; k0 < limit; k0 += kBatchRows) {
    half4 w[kBatchRows];
#pragma unroll
    for (uint32_t r = 0; r < kBatchRows; ++r) w[r] = load_half4(column + (uint64_t)(k0 + r) * kTdtGates);
#pragma unroll
    for (uint32_t r = 0; r < kBatchRows; r += 2) {
      even = __builtin_elementwise_fma(splat(s.x[k0 + r]), w[r], even);
      odd = __builtin_elementwise_fma(splat(s.x[k0 + r + 1]), w[r + 1], odd);
    }
  }
  const half4 sum = even + odd;
  for (int i = 0; i < 4; ++i) s.gates[4 * t + i] = (float)sum[i];
}

// Cell update of one layer (threads 0..159, four channels each): h and c to
// the candidate slots of `cand`.
__device__ void lstm_cell(Shared& s, const float* c_prev, float* h_out, float* c_out) {
  const uint32_t t = threadIdx.x;
  if (t < H / 4) {
    for (int i = 0; i < 4; ++i) {
      const uint32_t ch = 4 * t + i;
      const float ig = sigmoid_f32(s.gates[ch]);
      const float fg = sigmoid_f32(s.gates[H + ch]);
      const float gg = clamped_tanh(s.gates[2 * H + ch]);
      const float og = sigmoid_f32(s.gates[3 * H + ch]);
      const float cell = __builtin_fmaf(fg, c_prev[ch], ig * gg);
      c_out[ch] = cell;
      h_out[ch] = og * clamped_tanh(cell);
    }
  }
}

// prepare_predictor (tdt-decoder.ts:1341-1500): candidates from `token`
// and the committed state.
__device__ void predictor(Shared& s, const TdtArgs& a, const float* state, float* cand, uint32_t token,
                          bool initial) {
  const uint32_t t = threadIdx.x;
  for (uint32_t k = t; k < H; k += kThreads) {
    s.x[k] = initial ? (_Float16)0.0f : a.embedding[(uint64_t)token * H + k];
    s.x[H + k] = (_Float16)state[k];
  }
  __syncthreads();
  lstm_gates(s, a.lstm[0], a.lstm_bias[0], initial ? 0u : 2 * H);
  __syncthreads();
  lstm_cell(s, state + H, cand, cand + H);
  __syncthreads();
  for (uint32_t k = t; k < H; k += kThreads) {
    s.x[k] = (_Float16)cand[k];
    s.x[H + k] = (_Float16)state[2 * H + k];
  }
  __syncthreads();
  lstm_gates(s, a.lstm[1], a.lstm_bias[1], initial ? H : 2 * H);
  __syncthreads();
  lstm_cell(s, state + 3 * H, cand + 2 * H, cand + 3 * H);
  __syncthreads();
  if (t < H / 4) {
    // decoder projector, f32 fma chain over k (tdt-decoder.ts:1462-1491)
    const float4 b = *reinterpret_cast<const float4*>(a.projector_bias + 4 * t);
    float acc[4] = {b.x, b.y, b.z, b.w};
    const float* h1 = cand + 2 * H;
    for (uint32_t k0 = 0; k0 < H; k0 += kBatchRows) {
      half4 w[kBatchRows];
#pragma unroll
      for (uint32_t r = 0; r < kBatchRows; ++r) w[r] = load_half4(a.projector + (uint64_t)(k0 + r) * H + 4 * t);
#pragma unroll
      for (uint32_t r = 0; r < kBatchRows; ++r) {
        const float h = h1[k0 + r];
        for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(h, (float)w[r][i], acc[i]);
      }
    }
    for (int i = 0; i < 4; ++i) cand[4 * H + 4 * t + i] = acc[i];
  }
  __syncthreads();
}

// run_joint_pair for one window (tdt-decoder.ts:1605-1662, head :977-1031)
// and the argmax (:773-853, :1517-1603): s.token, s.duration.
__device__ void joint(Shared& s, const TdtArgs& a, const _Float16* encoder_row, const float* projection) {
  const uint32_t t = threadIdx.x;
  for (uint32_t c = t; c < H; c += kThreads) {
    // max(v, 0) as a comparison: -0 and NaN give +0 (the oracle's rule)
    const float v = (float)encoder_row[c] + projection[c];
    s.joint[c] = v > 0.0f ? v : 0.0f;
  }
  __syncthreads();
  if (t < kTdtHead / 4) {
    const float4 b = *reinterpret_cast<const float4*>(a.head_bias + 4 * t);
    half4 acc = half4{(_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
    bool zero_skip_safe = true;
    const _Float16* column = a.head + 4 * t;
    for (uint32_t k0 = 0; k0 < H; k0 += kBatchRows) {
      half4 w[kBatchRows];
#pragma unroll
      for (uint32_t r = 0; r < kBatchRows; ++r) w[r] = load_half4(column + (uint64_t)(k0 + r) * kTdtHead);
#pragma unroll
      for (uint32_t r = 0; r < kBatchRows; ++r) {
        const float x = s.joint[k0 + r];
        const uint32_t bits = __float_as_uint(x);
        const bool is_nan = (bits & 0x7fffffffu) > 0x7f800000u;
        zero_skip_safe = zero_skip_safe && !(bits == 0x80000000u || is_nan);
        if (!(zero_skip_safe && bits == 0u)) acc = __builtin_elementwise_fma(splat((_Float16)x), w[r], acc);
      }
    }
    for (int i = 0; i < 4; ++i) s.scores[4 * t + i] = (float)acc[i];
  }
  __syncthreads();
  if (t < 64) {
    // the largest score, the lowest id among equal scores; NaN never wins
    float best = -3.402823466e+38f;
    uint32_t id = 0xffffffffu;
    for (uint32_t o = t; o <= kTdtBlank; o += 64) {
      float v = s.scores[o];
      v = v != v ? -3.402823466e+38f : v;
      if (v > best || (v == best && o < id)) {
        best = v;
        id = o;
      }
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(best, off, 64);
      const uint32_t oid = __shfl_xor(id, off, 64);
      if (ov > best || (ov == best && oid < id)) {
        best = ov;
        id = oid;
      }
    }
    if (t == 0) {
      float dbest = -3.402823466e+38f;
      uint32_t d = 0xffffffffu;
      for (uint32_t j = 0; j < 5; ++j) {
        float v = s.scores[kTdtBlank + 1 + j];
        v = v != v ? -3.402823466e+38f : v;
        if (v > dbest || (v == dbest && j < d)) {
          dbest = v;
          d = j;
        }
      }
      s.token = id;
      s.duration = d;
    }
  }
  __syncthreads();
}

__global__ __launch_bounds__(kTdtThreads) void tdt_decode_kernel(TdtArgs a) {
  __shared__ Shared s;
  const uint32_t b = blockIdx.x, t = threadIdx.x;
  float* state = a.state + (uint64_t)b * 4 * H;
  float* cand = a.scratch + (uint64_t)b * 5 * H;
  const _Float16* encoder = a.encoder + (uint64_t)b * a.frames * H;
  for (uint32_t i = t; i < 4 * H; i += kThreads) state[i] = 0.0f;

  // control state, thread 0 only
  const uint32_t limit = min(a.lengths[b], a.frames);
  const uint32_t encoded = min(limit, a.ends[b]);
  uint32_t time = min(a.starts[b], encoded), count = 0, st = 0, symbols = 0;
  bool flushing = false;
  uint32_t flush_blanks = 0, flush_time = 0;
  const bool flush_requested = a.flush[b] != 0 && a.starts[b] < encoded;
  __syncthreads();
  if (time < encoded) predictor(s, a, state, cand, 0, true);

  // Every iteration advances the time or the symbol count (at most 10 per
  // frame) or the flush (at most 10 steps): the bound is never reached.
  const uint32_t max_steps = 11 * a.frames + 32;
  for (uint32_t step = 0; step < max_steps; ++step) {
    if (t == 0) {
      // choose the frame of this step's joint, or stop (:1722-1735, :1812-1880)
      s.go = 0;
      if (!flushing && time < encoded) {
        s.go = 1;
        s.joint_time = time;
      } else {
        if (!flushing && flush_requested) {
          flushing = true;
          symbols = 0;
          flush_blanks = 0;
          flush_time = time;
        }
        if (flushing && symbols < 10 && flush_blanks < 5) {
          const uint32_t variation = symbols % 3;
          if (variation == 0)
            time = min(flush_time, limit - 1u);
          else if (variation == 1)
            time = min(encoded - 1u, a.frames - 1u);
          else
            time = min(max(encoded, 2u) - 2u, a.frames - 1u);
          s.go = 1;
          s.joint_time = time;
        }
      }
    }
    __syncthreads();
    if (!s.go) break;
    joint(s, a, encoder + (uint64_t)s.joint_time * H, cand + 4 * H);
    if (t == 0) {
      const uint32_t token = s.token, duration = s.duration;
      const bool emitted = token != kTdtBlank;
      const uint32_t frame = flushing ? min(flush_time, encoded - 1u) : time;
      if (emitted) {
        if (count < a.max_tokens) {
          const uint64_t at = (uint64_t)b * a.max_tokens + count;
          a.tokens[at] = token;
          a.token_frames[at] = frame;
          a.token_durations[at] = duration;
          ++count;
        } else {
          st |= 1u;
        }
      }
      if (!flushing) {
        symbols += 1;
        if (duration != 0) {
          time += duration;
          symbols = 0;
        } else if (!emitted || symbols >= 10) {
          time += 1;
          symbols = 0;
        }
      } else {
        flush_blanks = emitted ? 0u : flush_blanks + 1u;
        flush_time = min(flush_time + max(1u, duration), encoded);
        symbols += 1;
      }
      s.emitted = emitted;
    }
    __syncthreads();
    if (s.emitted) {
      // commit_predictor (:1502-1515), then the next token's candidates
      for (uint32_t i = t; i < 4 * H; i += kThreads) state[i] = cand[i];
      __syncthreads();
      predictor(s, a, state, cand, s.token, false);
    }
  }
  if (t == 0) {
    a.counts[b] = count;
    a.status[b] = st;
  }
}

}  // namespace

hipError_t launch_tdt_decode(const TdtArgs& args, uint32_t batch, hipStream_t stream, hipEvent_t start,
                             hipEvent_t stop) {
  if (batch == 0) return hipSuccess;
  if (start || stop)
    hipExtLaunchKernelGGL(tdt_decode_kernel, dim3(batch), dim3(kTdtThreads), 0, stream, start, stop, 0, args);
  else
    hipLaunchKernelGGL(tdt_decode_kernel, dim3(batch), dim3(kTdtThreads), 0, stream, args);
  return hipGetLastError();
}

}  // namespace pk

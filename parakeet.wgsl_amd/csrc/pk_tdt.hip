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
// Arithmetic is the shader's, term for term, in both execution profiles
// (tdt-decoder.ts:1155-1190 picks the readers and chains by precision):
// every gate is a chain over even rows starting at the bias plus one over
// odd rows starting at zero, fma in increasing k (one rounding each), the
// two added at the end; the head is a chain over k skipping exact +0 joint
// inputs until a -0 or NaN input is seen; the projector is an f32 fma chain;
// the cell update and the activations are f32 with exp written out (range
// reduction and a degree-7 Taylor polynomial) rather than taken from a
// library, so the decode is reproducible to the bit. In the f16 profile
// (weights, encoder rows and chains in f16: v_pk_fma_f16) the chain inputs
// and the biases are rounded to f16 (:572-666, :687-742, :977-1031); in the
// f32 profile (f32 weights and encoder rows, :595-614, :642-666, :700-716,
// :743-771, :1033-1058) every chain is f32 and nothing is rounded. The
// kernels are templates over the profile (`ProfileF16`, `ProfileF32`).
// Contraction is off in this file: every fused multiply-add is written as
// one.
#include "pk_internal.h"

#pragma clang fp contract(off)

namespace pk {
namespace {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

// W: weight and encoder-row element; W4: four weights (one 8- or 16-byte
// load); X: a chain input as staged in LDS; A4: four chain accumulators.
struct ProfileF16 {
  typedef _Float16 W;
  typedef half4 W4;
  typedef _Float16 X;
  typedef half4 A4;
};
struct ProfileF32 {
  typedef float W;
  typedef float4v W4;
  typedef float X;
  typedef float4v A4;
};

template <class P>
__device__ __forceinline__ const typename P::W* wptr(const void* p) {
  return static_cast<const typename P::W*>(p);
}

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

template <class V, class S>
__device__ __forceinline__ V splat(S x) {
  return V{x, x, x, x};
}

template <class V, class S>
__device__ __forceinline__ V load4(const S* p) {
  return *reinterpret_cast<const V*>(p);
}

// Four f32 biases as chain accumulators (rounded to f16 in that profile).
template <class A4>
__device__ __forceinline__ A4 bias4(const float* p) {
  const float4 b = *reinterpret_cast<const float4*>(p);
  typedef decltype(A4{}[0]) E;
  return A4{(E)b.x, (E)b.y, (E)b.z, (E)b.w};
}

template <class P>
struct Shared {
  typename P::X x[2 * H]; // LSTM layer inputs
  float gates[kTdtGates]; // f32 values of the gate sums
  float joint[H];         // relu(encoder + projection)
  float scores[kTdtHead]; // f32 values of the head accumulators
  bool use[H];            // head row k enters the chain (the +0-skip rule)
  // control, written by thread 0
  uint32_t go, emitted, token, duration, joint_time, first_bad;
};

// Rows of weights loaded before any is used: the k loops are latency
// bound, so each thread keeps this many 8-byte loads in flight.
constexpr uint32_t kBatchRows = 16;

// Gates of one LSTM layer: thread t owns gates 4t..4t+3 over `limit` rows
// (a multiple of kBatchRows).
template <class P>
__device__ void lstm_gates(Shared<P>& s, const void* weight, const float* bias, uint32_t limit) {
  typedef typename P::A4 A4;
  typedef typename P::W4 W4;
  const uint32_t t = threadIdx.x;
  A4 even = bias4<A4>(bias + 4 * t);
  A4 odd = A4{0, 0, 0, 0};
  const typename P::W* column = wptr<P>(weight) + 4 * t;
  for (uint32_t k0 = 0; k0 < limit; k0 += kBatchRows) {
    W4 w[kBatchRows];
#pragma unroll
    for (uint32_t r = 0; r < kBatchRows; ++r) w[r] = load4<W4>(column + (uint64_t)(k0 + r) * kTdtGates);
#pragma unroll
    for (uint32_t r = 0; r < kBatchRows; r += 2) {
      even = __builtin_elementwise_fma(splat<A4>(s.x[k0 + r]), w[r], even);
      odd = __builtin_elementwise_fma(splat<A4>(s.x[k0 + r + 1]), w[r + 1], odd);
    }
  }
  const A4 sum = even + odd;
  for (int i = 0; i < 4; ++i) s.gates[4 * t + i] = (float)sum[i];
}

// Cell update of one layer (threads 0..159, four channels each): h and c to
// the candidate slots of `cand`.
template <class P>
__device__ void lstm_cell(Shared<P>& s, const float* c_prev, float* h_out, float* c_out) {
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
template <class P>
__device__ void predictor(Shared<P>& s, const TdtArgs& a, const float* state, float* cand, uint32_t token,
                          bool initial) {
  typedef typename P::X X;
  const uint32_t t = threadIdx.x;
  const typename P::W* embedding = wptr<P>(a.embedding);
  for (uint32_t k = t; k < H; k += kThreads) {
    s.x[k] = initial ? (X)0.0f : (X)embedding[(uint64_t)token * H + k];
    s.x[H + k] = (X)state[k];
  }
  __syncthreads();
  lstm_gates(s, a.lstm[0], a.lstm_bias[0], initial ? 0u : 2 * H);
  __syncthreads();
  lstm_cell(s, state + H, cand, cand + H);
  __syncthreads();
  for (uint32_t k = t; k < H; k += kThreads) {
    s.x[k] = (X)cand[k];
    s.x[H + k] = (X)state[2 * H + k];
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
    const typename P::W* projector = wptr<P>(a.projector);
    for (uint32_t k0 = 0; k0 < H; k0 += kBatchRows) {
      typename P::W4 w[kBatchRows];
#pragma unroll
      for (uint32_t r = 0; r < kBatchRows; ++r)
        w[r] = load4<typename P::W4>(projector + (uint64_t)(k0 + r) * H + 4 * t);
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
template <class P>
__device__ void joint(Shared<P>& s, const TdtArgs& a, const typename P::W* encoder_row, const float* projection) {
  typedef typename P::A4 A4;
  typedef typename P::W4 W4;
  const uint32_t t = threadIdx.x;
  for (uint32_t c = t; c < H; c += kThreads) {
    // max(v, 0) as a comparison: -0 and NaN give +0 (the oracle's rule)
    const float v = (float)encoder_row[c] + projection[c];
    s.joint[c] = v > 0.0f ? v : 0.0f;
  }
  if (t == 0) s.first_bad = H;
  __syncthreads();
  // An exact +0 input is skipped while no -0 or NaN has appeared at or
  // before it: find the first such row, then flag every row and keep the
  // chain inputs, so the chain below selects instead of branching.
  for (uint32_t c = t; c < H; c += kThreads) {
    const uint32_t bits = __float_as_uint(s.joint[c]);
    if (bits == 0x80000000u || (bits & 0x7fffffffu) > 0x7f800000u) atomicMin(&s.first_bad, c);
  }
  __syncthreads();
  for (uint32_t c = t; c < H; c += kThreads) {
    s.x[c] = (typename P::X)s.joint[c];
    s.use[c] = __float_as_uint(s.joint[c]) != 0u || c >= s.first_bad;
  }
  __syncthreads();
  if (t < kTdtHead / 4) {
    A4 acc = bias4<A4>(a.head_bias + 4 * t);
    const typename P::W* column = wptr<P>(a.head) + 4 * t;
    for (uint32_t k0 = 0; k0 < H; k0 += kBatchRows) {
      W4 w[kBatchRows];
#pragma unroll
      for (uint32_t r = 0; r < kBatchRows; ++r) w[r] = load4<W4>(column + (uint64_t)(k0 + r) * kTdtHead);
#pragma unroll
      for (uint32_t r = 0; r < kBatchRows; ++r) {
        const A4 next = __builtin_elementwise_fma(splat<A4>(s.x[k0 + r]), w[r], acc);
        acc = s.use[k0 + r] ? next : acc;
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

template <class P>
__global__ __launch_bounds__(kTdtThreads) void tdt_decode_kernel(TdtArgs a) {
  __shared__ Shared<P> s;
  const uint32_t b = blockIdx.x, t = threadIdx.x;
  float* state = a.state + (uint64_t)b * 4 * H;
  float* cand = a.scratch + (uint64_t)b * 5 * H;
  const typename P::W* encoder = wptr<P>(a.encoder) + (uint64_t)b * a.frames * H;
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


// ---------------------------------------------------------------- teams
//
// Team decoding spreads one window over P workgroups ("members") of 256
// threads. Member p owns hidden units [pU, pU + U) (U = 640 / P): the four
// gate columns of those units in both LSTM layers, the same projector
// columns, and a range of head quads. Every matrix slice streams through
// two LDS stages (one chunk of rows in registers while the previous chunk
// is multiplied), so a member reads 1/P of the weights per step; with the
// workgroup ids laid out window-major, member p of every window lands on
// the same XCD (dispatch is round robin over the eight XCDs), whose L2 then
// holds the slices of its two member indices.
//
// The arithmetic is the single-workgroup kernel's, chain for chain: a gate
// column is still one f16 chain over even rows from f16(bias) and one over
// odd rows from zero, in increasing k; the projector and head columns are
// the same f32 and f16 chains; the argmax combines per-member (best value,
// lowest id) pairs, which selects the same id as one scan. Control state is
// kept by thread 0 of every member and evolves identically; member 0
// writes the outputs.
//
// Exchange between members goes through the window's state and scratch
// slices in global memory with relaxed agent-scope atomic loads and stores
// (coherent across the XCDs' L2s without cache maintenance), ordered by team
// barriers: every wave's stores complete (workgroup release), then an
// atomic arrival count and a bounded poll (team_barrier states what of the
// code generation this ordering rests on). Agent-scope fences would write
// back and invalidate the XCD's whole L2 at every barrier, which measured
// slower than one workgroup per window; the weights, read with ordinary
// loads, stay cached. A barrier that waits
// longer than `spin_limit` polls raises the window's abort flag and every
// member leaves its loop at its next barrier (status kTdtSyncTimeout), so
// every wave reaches the end. The launch is an ordinary one whose grid
// never exceeds the workgroups the device holds at once (the occupancy
// bound checked at launch), so on an otherwise idle device every member is
// resident; a member that is not (another kernel holds its compute unit)
// only delays the barrier until it is scheduled, and the bounded poll turns
// a wait that never ends into the timeout status.

constexpr uint32_t TT = kTdtTeamThreads;

// Exchanged values: relaxed agent-scope atomics, coherent between XCDs.
__device__ __forceinline__ float xload(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void xstore(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t xload(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void xstore(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr uint32_t kStageUnits = 6400;  // half4 units per staged chunk (51,200 bytes)

struct TeamShared {
  half4 stage[2][kStageUnits];
  _Float16 x[2 * H];
  float vec[H];
  float gates[4 * 80];
  half4 odd[80];
  float scores[33 * 4];
  uint32_t part[16 * 4];
  bool use[H];
  uint32_t go, emitted, token, duration, joint_time, failed, first_bad;
};

struct Slice {
  const _Float16* base;  // matrix
  uint32_t stride;       // halves per row
  uint32_t quads;        // half4 units per row of the slice
  uint32_t seg_quads;    // quads per segment (segments are `seg_stride` columns apart)
  uint32_t seg_stride;
  uint32_t col0;         // first column of segment 0
  uint32_t rows;         // rows per chunk
};

constexpr uint32_t kUnitsPerThread = kStageUnits / TT;  // 25

// Element offsets (relative to row 0) of this thread's units of a chunk,
// the same for every chunk of the slice; ~0u past the chunk's units.
__device__ __forceinline__ void slice_offsets(const Slice& sl, uint32_t (&off)[kUnitsPerThread]) {
  const uint32_t units = sl.rows * sl.quads;
  uint32_t r = threadIdx.x / sl.quads, q = threadIdx.x % sl.quads;
  const uint32_t dr = TT / sl.quads, dq = TT % sl.quads;
#pragma unroll
  for (uint32_t i = 0; i < kUnitsPerThread; ++i) {
    const uint32_t u = threadIdx.x + i * TT;
    off[i] = u < units ? r * sl.stride + sl.col0 + (q / sl.seg_quads) * sl.seg_stride + (q % sl.seg_quads) * 4u
                       : ~0u;  // past the chunk: loads row 0's first quad, never stored
    q += dq;
    r += dr;
    if (q >= sl.quads) {
      q -= sl.quads;
      r += 1;
    }
  }
}

__device__ __forceinline__ void stage_load(const Slice& sl, uint32_t k0, const uint32_t (&off)[kUnitsPerThread],
                                           half4 (&reg)[kUnitsPerThread]) {
  const _Float16* base = sl.base + (uint64_t)k0 * sl.stride;
  // unconditional, so all of a thread's loads issue back to back
#pragma unroll
  for (uint32_t i = 0; i < kUnitsPerThread; ++i) reg[i] = load4<half4>(base + (off[i] == ~0u ? 0u : off[i]));
}

__device__ __forceinline__ void stage_store(half4* dst, const uint32_t (&off)[kUnitsPerThread],
                                            const half4 (&reg)[kUnitsPerThread]) {
#pragma unroll
  for (uint32_t i = 0; i < kUnitsPerThread; ++i)
    if (off[i] != ~0u) dst[threadIdx.x + i * TT] = reg[i];
}

// Streams rows [0, limit) of the slice through the two stages and calls
// body(stage, k0) for every chunk (all threads, after a barrier).
template <class Body>
__device__ void stream_slice(TeamShared& s, const Slice& sl, uint32_t limit, Body body) {
  const uint32_t chunks = limit / sl.rows;
  if (chunks == 0) return;
  uint32_t off[kUnitsPerThread];
  slice_offsets(sl, off);
  half4 reg[kUnitsPerThread];
  stage_load(sl, 0, off, reg);
  for (uint32_t c = 0; c < chunks; ++c) {
    half4* cur = s.stage[c & 1u];
    stage_store(cur, off, reg);
    __syncthreads();
    if (c + 1 < chunks) stage_load(sl, (c + 1) * sl.rows, off, reg);
    body(cur, c * sl.rows);
  }
  __syncthreads();
}

// dst[k] = src[k] for k < H (exchanged values): a thread's three loads are
// issued before any is used.
__device__ __forceinline__ void load_exchanged(float* dst, const float* src) {
  const uint32_t t = threadIdx.x;
  float v[3];
#pragma unroll
  for (uint32_t i = 0; i < 3; ++i)
    if (t + i * TT < H) v[i] = xload(src + t + i * TT);
#pragma unroll
  for (uint32_t i = 0; i < 3; ++i)
    if (t + i * TT < H) dst[t + i * TT] = v[i];
}

__device__ __forceinline__ void load_exchanged_f16(_Float16* dst, const float* src) {
  const uint32_t t = threadIdx.x;
  float v[3];
#pragma unroll
  for (uint32_t i = 0; i < 3; ++i)
    if (t + i * TT < H) v[i] = xload(src + t + i * TT);
#pragma unroll
  for (uint32_t i = 0; i < 3; ++i)
    if (t + i * TT < H) dst[t + i * TT] = (_Float16)v[i];
}

// One team barrier: the n-th barrier of a window waits for count >= P * n.
//
// Ordering. The exchanged values and the counter are relaxed agent-scope
// atomics, which order nothing among themselves in the C++ / HIP model;
// what orders them here is gfx950's code generation, on which this relies:
// (1) a relaxed agent-scope store or load is a global store / load with the
// sc1 bit, performed at the agent's coherence point rather than in an
// XCD's L2; (2) vmcnt counts stores as well as loads (gfx9), so
// s_waitcnt(0) returns only once every earlier store of the wave has been
// acknowledged there; (3) a member polls the counter until it reaches the
// target before any load that follows the barrier issues. The signal
// fences keep the compiler from moving exchanged accesses across the
// arrival or above the end of the poll. Formal release / acquire at agent
// scope would add an L2 write-back and invalidate to every barrier, and the
// invalidate evicts the weight slices the members re-read from their XCD's
// L2 at every step (measured slower than one workgroup per window).
__device__ bool team_barrier(TeamShared& s, const TdtTeam& tm, uint32_t b, uint32_t& n) {
  ++n;
  // every wave waits for its exchanged (coherent) stores to complete before
  // the arrival; a workgroup barrier alone does not wait for them
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    // one 256-byte line per counter and per flag: the windows' teams poll
    // their own lines, never a shared one
    uint32_t* counter = tm.sync + (uint64_t)b * kTdtSyncStride;
    uint32_t* abort = tm.sync + ((uint64_t)tm.capacity + b) * kTdtSyncStride;
    uint32_t failed = 0;
    __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t target = tm.members * n;
    uint32_t polls = 0;
    while (xload(counter) < target) {
      if ((polls & 31u) == 31u && xload(abort) != 0u) {
        failed = 1;
        break;
      }
      if (++polls > tm.spin_limit) {
        __hip_atomic_fetch_or(abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        failed = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    s.failed = failed;
  }
  __syncthreads();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  return s.failed == 0;
}

// Gates of this member's units in one LSTM layer, then their cell update:
// h and c of units [u0, u0 + U) to h_out / c_out.
__device__ void team_lstm(TeamShared& s, const _Float16* weight, const float* bias, uint32_t limit, uint32_t u0,
                          uint32_t U, const float* c_prev, float* h_out, float* c_out) {
  const uint32_t t = threadIdx.x;
  const uint32_t Q = U;  // U / 4 quads in each of the four gate segments
  const Slice sl{weight, kTdtGates, Q, U / 4, H, u0, kStageUnits / Q};
  const uint32_t parity = t / Q, q = t % Q;
  const bool chain = t < 2 * Q;
  const uint32_t col = (q / (U / 4)) * H + u0 + (q % (U / 4)) * 4;
  half4 acc = half4{0, 0, 0, 0};
  if (chain && parity == 0) {
    const float4 bb = *reinterpret_cast<const float4*>(bias + col);
    acc = half4{(_Float16)bb.x, (_Float16)bb.y, (_Float16)bb.z, (_Float16)bb.w};
  }
  stream_slice(s, sl, limit, [&](const half4* st, uint32_t k0) {
    if (chain) {
      // rows come in batches of 16 (chunks hold 80 or 160 rows): the 8 rows
      // of this parity are read from LDS before the dependent chain runs
      for (uint32_t r0 = 0; r0 < sl.rows; r0 += 16) {
        half4 w[8];
        _Float16 x[8];
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
          const uint32_t r = r0 + 2 * i + parity;
          w[i] = st[r * Q + q];
          x[i] = s.x[k0 + r];
        }
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) acc = __builtin_elementwise_fma(splat<half4>(x[i]), w[i], acc);
      }
    }
  });
  if (chain && parity == 1) s.odd[q] = acc;
  __syncthreads();
  if (chain && parity == 0) {
    const half4 sum = acc + s.odd[q];
    for (int i = 0; i < 4; ++i) s.gates[4 * q + i] = (float)sum[i];
  }
  __syncthreads();
  if (t < U) {
    // unit j's gate g sits at quad g * U / 4 + j / 4, lane j % 4: index g * U + j
    const uint32_t ch = u0 + t;
    const float ig = sigmoid_f32(s.gates[t]);
    const float fg = sigmoid_f32(s.gates[U + t]);
    const float gg = clamped_tanh(s.gates[2 * U + t]);
    const float og = sigmoid_f32(s.gates[3 * U + t]);
    const float cell = __builtin_fmaf(fg, xload(c_prev + ch), ig * gg);
    xstore(c_out + ch, cell);
    xstore(h_out + ch, og * clamped_tanh(cell));
  }
}

// prepare_predictor with this member's slices; three team barriers.
__device__ bool team_predictor(TeamShared& s, const TdtArgs& a, const TdtTeam& tm, uint32_t b, uint32_t& n,
                               const float* state, float* cand, uint32_t token, bool initial, uint32_t u0,
                               uint32_t U) {
  const uint32_t t = threadIdx.x;
  const _Float16* embedding = static_cast<const _Float16*>(a.embedding);
  for (uint32_t k = t; k < H; k += TT) s.x[k] = initial ? (_Float16)0.0f : embedding[(uint64_t)token * H + k];
  load_exchanged_f16(s.x + H, state);
  __syncthreads();
  team_lstm(s, static_cast<const _Float16*>(a.lstm[0]), a.lstm_bias[0], initial ? 0u : 2 * H, u0, U, state + H, cand,
            cand + H);
  if (!team_barrier(s, tm, b, n)) return false;
  load_exchanged_f16(s.x, cand);
  load_exchanged_f16(s.x + H, state + 2 * H);
  __syncthreads();
  team_lstm(s, static_cast<const _Float16*>(a.lstm[1]), a.lstm_bias[1], initial ? H : 2 * H, u0, U, state + 3 * H,
            cand + 2 * H, cand + 3 * H);
  if (!team_barrier(s, tm, b, n)) return false;
  // decoder projector columns [u0, u0 + U): f32 fma chain over k
  load_exchanged(s.vec, cand + 2 * H);
  const Slice sl{static_cast<const _Float16*>(a.projector), H, U / 4, U / 4, 0, u0, kStageUnits / (U / 4)};
  float acc = 0.0f;
  if (t < U) acc = a.projector_bias[u0 + t];
  stream_slice(s, sl, H, [&](const half4* st, uint32_t k0) {
    if (t < U) {
      for (uint32_t r0 = 0; r0 < sl.rows; r0 += 16) {
        float w[16], h[16];
#pragma unroll
        for (uint32_t i = 0; i < 16; ++i) {
          w[i] = (float)st[(r0 + i) * (U / 4) + t / 4][t % 4];
          h[i] = s.vec[k0 + r0 + i];
        }
#pragma unroll
        for (uint32_t i = 0; i < 16; ++i) acc = __builtin_fmaf(h[i], w[i], acc);
      }
    }
  });
  if (t < U) xstore(cand + 4 * H + u0 + t, acc);
  return team_barrier(s, tm, b, n);
}

// The joint over this member's head quads [hq0, hq1) and the team argmax:
// s.token, s.duration.
__device__ bool team_joint(TeamShared& s, const TdtArgs& a, const TdtTeam& tm, uint32_t b, uint32_t& n,
                           uint32_t p, uint32_t buf, const _Float16* encoder_row, const float* projection,
                           uint32_t hq0, uint32_t hq1) {
  const uint32_t t = threadIdx.x;
  load_exchanged(s.vec, projection);
  __syncthreads();
  for (uint32_t c = t; c < H; c += TT) {
    const float v = (float)encoder_row[c] + s.vec[c];
    s.vec[c] = v > 0.0f ? v : 0.0f;
  }
  __syncthreads();
  // The head chain skips an exact +0 input while no -0 or NaN has appeared
  // at or before it: s.x holds the f16 inputs, s.use whether row k enters
  // the chain (the first -0 / NaN row found by a min-reduction).
  if (t == 0) s.first_bad = H;
  __syncthreads();
  for (uint32_t c = t; c < H; c += TT) {
    const uint32_t bits = __float_as_uint(s.vec[c]);
    if (bits == 0x80000000u || (bits & 0x7fffffffu) > 0x7f800000u) atomicMin(&s.first_bad, c);
  }
  __syncthreads();
  for (uint32_t c = t; c < H; c += TT) {
    s.x[c] = (_Float16)s.vec[c];
    s.use[c] = __float_as_uint(s.vec[c]) != 0u || c >= s.first_bad;
  }
  const uint32_t HQ = hq1 - hq0;  // at most 17 (16 members) or 33 (8 members)
  const Slice sl{static_cast<const _Float16*>(a.head), kTdtHead, HQ, HQ, 0, hq0 * 4, HQ * 320 <= kStageUnits ? 320u : 160u};
  half4 acc = half4{0, 0, 0, 0};
  if (t < HQ) {
    const float4 bb = *reinterpret_cast<const float4*>(a.head_bias + 4 * (hq0 + t));
    acc = half4{(_Float16)bb.x, (_Float16)bb.y, (_Float16)bb.z, (_Float16)bb.w};
  }
  __syncthreads();
  stream_slice(s, sl, H, [&](const half4* st, uint32_t k0) {
    if (t < HQ) {
      for (uint32_t r0 = 0; r0 < sl.rows; r0 += 16) {
        half4 w[16];
        _Float16 xs[16];
        bool use[16];
#pragma unroll
        for (uint32_t i = 0; i < 16; ++i) {
          w[i] = st[(r0 + i) * HQ + t];
          xs[i] = s.x[k0 + r0 + i];
          use[i] = s.use[k0 + r0 + i];
        }
        // the flag is the same for every lane: a scalar branch skips the
        // row without touching the dependent chain
#pragma unroll
        for (uint32_t i = 0; i < 16; ++i)
          if (__builtin_amdgcn_readfirstlane((int)use[i])) acc = __builtin_elementwise_fma(splat<half4>(xs[i]), w[i], acc);
      }
    }
  });
  if (t < HQ)
    for (int i = 0; i < 4; ++i) s.scores[4 * t + i] = (float)acc[i];
  __syncthreads();
  uint32_t* part = tm.partials + (((uint64_t)b * 2 + buf) * tm.members) * 4;
  if (t < 64) {
    // this member's best token (value, lowest id) and best duration: each
    // lane scans scores t, t + 64, t + 128, then a shuffle reduction
    float best = -3.402823466e+38f, dbest = -3.402823466e+38f;
    uint32_t id = 0xffffffffu, d = 0xffffffffu;
    for (uint32_t i = t; i < 4 * HQ; i += 64) {
      const uint32_t o = 4 * hq0 + i;
      float v = s.scores[i];
      v = v != v ? -3.402823466e+38f : v;
      if (o <= kTdtBlank) {
        if (v > best || (v == best && o < id)) {
          best = v;
          id = o;
        }
      } else if (o <= kTdtBlank + 5) {
        const uint32_t j = o - kTdtBlank - 1;
        if (v > dbest || (v == dbest && j < d)) {
          dbest = v;
          d = j;
        }
      }
    }
    for (int offset = 32; offset > 0; offset >>= 1) {
      const float ov = __shfl_xor(best, offset, 64);
      const uint32_t oid = __shfl_xor(id, offset, 64);
      if (ov > best || (ov == best && oid < id)) {
        best = ov;
        id = oid;
      }
      const float odv = __shfl_xor(dbest, offset, 64);
      const uint32_t od = __shfl_xor(d, offset, 64);
      if (odv > dbest || (odv == dbest && od < d)) {
        dbest = odv;
        d = od;
      }
    }
    if (t == 0) {
      xstore(part + 4 * p + 0, __float_as_uint(best));
      xstore(part + 4 * p + 1, id);
      xstore(part + 4 * p + 2, __float_as_uint(dbest));
      xstore(part + 4 * p + 3, d);
    }
  }
  if (!team_barrier(s, tm, b, n)) return false;
  if (t < 4 * tm.members) s.part[t] = xload(part + t);  // every partial in one round trip
  __syncthreads();
  if (t == 0) {
    float best = -3.402823466e+38f, dbest = -3.402823466e+38f;
    uint32_t id = 0xffffffffu, d = 0xffffffffu;
    for (uint32_t m = 0; m < tm.members; ++m) {
      const float v = __uint_as_float(s.part[4 * m + 0]);
      const uint32_t o = s.part[4 * m + 1];
      if (o != 0xffffffffu && (v > best || (v == best && o < id))) {
        best = v;
        id = o;
      }
      const float dv = __uint_as_float(s.part[4 * m + 2]);
      const uint32_t j = s.part[4 * m + 3];
      if (j != 0xffffffffu && (dv > dbest || (dv == dbest && j < d))) {
        dbest = dv;
        d = j;
      }
    }
    s.token = id;
    s.duration = d;
  }
  __syncthreads();
  return true;
}

__global__ __launch_bounds__(kTdtTeamThreads) void tdt_team_kernel(TdtArgs a, TdtTeam tm) {
  __shared__ TeamShared s;
  const uint32_t P = tm.members;
  const uint32_t b = blockIdx.x / P, p = blockIdx.x % P, t = threadIdx.x;
  const uint32_t U = H / P, u0 = p * U;
  const uint32_t hq0 = p * (kTdtHead / 4) / P, hq1 = (p + 1) * (kTdtHead / 4) / P;
  float* state = a.state + (uint64_t)b * 4 * H;
  float* cand = a.scratch + (uint64_t)b * 5 * H;
  const _Float16* encoder = static_cast<const _Float16*>(a.encoder) + (uint64_t)b * a.frames * H;
  uint32_t n = 0;  // team barriers passed
  for (uint32_t i = t; i < U; i += TT)
    for (uint32_t j = 0; j < 4; ++j) xstore(state + j * H + u0 + i, 0.0f);

  const uint32_t limit = min(a.lengths[b], a.frames);
  const uint32_t encoded = min(limit, a.ends[b]);
  uint32_t time = min(a.starts[b], encoded), count = 0, st = 0, symbols = 0;
  bool flushing = false;
  uint32_t flush_blanks = 0, flush_time = 0, joints = 0;
  const bool flush_requested = a.flush[b] != 0 && a.starts[b] < encoded;
  bool alive = team_barrier(s, tm, b, n);
  if (alive && time < encoded) alive = team_predictor(s, a, tm, b, n, state, cand, 0, true, u0, U);

  const uint32_t max_steps = 11 * a.frames + 32;
  for (uint32_t step = 0; alive && step < max_steps; ++step) {
    if (t == 0) {
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
    alive = team_joint(s, a, tm, b, n, p, joints & 1u, encoder + (uint64_t)s.joint_time * H, cand + 4 * H, hq0,
                       hq1);
    ++joints;
    if (!alive) break;
    if (t == 0) {
      const uint32_t token = s.token, duration = s.duration;
      const bool emitted = token != kTdtBlank;
      const uint32_t frame = flushing ? min(flush_time, encoded - 1u) : time;
      if (emitted) {
        if (count < a.max_tokens) {
          if (p == 0) {
            const uint64_t at = (uint64_t)b * a.max_tokens + count;
            a.tokens[at] = token;
            a.token_frames[at] = frame;
            a.token_durations[at] = duration;
          }
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
      // commit_predictor: this member's units
      for (uint32_t i = t; i < U; i += TT)
        for (uint32_t j = 0; j < 4; ++j) xstore(state + j * H + u0 + i, xload(cand + j * H + u0 + i));
      alive = team_barrier(s, tm, b, n);
      if (alive) alive = team_predictor(s, a, tm, b, n, state, cand, s.token, false, u0, U);
    }
  }
  if (t == 0 && p == 0) {
    a.counts[b] = count;
    a.status[b] = st | (alive ? 0u : kTdtSyncTimeout);
  }
}

__global__ void tdt_team_clear(uint32_t* sync, uint32_t words) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < words) sync[i] = 0u;
}

}  // namespace

hipError_t launch_tdt_decode(const TdtArgs& args, uint32_t batch, bool f32, hipStream_t stream, hipEvent_t start,
                             hipEvent_t stop) {
  if (batch == 0) return hipSuccess;
  const dim3 grid(batch), block(kTdtThreads);
  if (f32) {
    if (start || stop)
      hipExtLaunchKernelGGL(tdt_decode_kernel<ProfileF32>, grid, block, 0, stream, start, stop, 0, args);
    else
      hipLaunchKernelGGL(tdt_decode_kernel<ProfileF32>, grid, block, 0, stream, args);
  } else {
    if (start || stop)
      hipExtLaunchKernelGGL(tdt_decode_kernel<ProfileF16>, grid, block, 0, stream, start, stop, 0, args);
    else
      hipLaunchKernelGGL(tdt_decode_kernel<ProfileF16>, grid, block, 0, stream, args);
  }
  return hipGetLastError();
}

bool tdt_team_members_supported(uint32_t members) { return members == 8 || members == 16; }

uint32_t tdt_team_capacity(int device) {
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(tdt_team_kernel),
                                                   kTdtTeamThreads, 0) != hipSuccess)
    return 0;
  return (uint32_t)(cus * per_cu);
}

hipError_t launch_tdt_team(const TdtArgs& args, const TdtTeam& team, uint32_t batch, hipStream_t stream,
                           hipEvent_t start, hipEvent_t stop) {
  if (batch == 0) return hipSuccess;
  if (!tdt_team_members_supported(team.members) || batch > team.capacity) return hipErrorInvalidValue;
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return e;
  if ((uint64_t)batch * team.members > tdt_team_capacity(device)) return hipErrorInvalidConfiguration;
  const uint32_t words = 2 * team.capacity * kTdtSyncStride;
  hipLaunchKernelGGL(tdt_team_clear, dim3((words + 255) / 256), dim3(256), 0, stream, team.sync, words);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const dim3 grid(batch * team.members), block(kTdtTeamThreads);
  if (start || stop)
    hipExtLaunchKernelGGL(tdt_team_kernel, grid, block, 0, stream, start, stop, 0, args, team);
  else
    hipLaunchKernelGGL(tdt_team_kernel, grid, block, 0, stream, args, team);
  return hipGetLastError();
}

}  // namespace pk

// pk_layernorm.hip - row LayerNorm for gfx950 (reference:
// src/webgpu/kernels/layernorm.ts, shader :309-390, dispatch :29-240).
//
// mean = sum(x) / C, variance = max(sum(x^2) / C - mean^2, 0),
// out = (x - mean) * rsqrt(variance + epsilon) * gamma + beta, statistics in
// f32, output rounded to the storage type (the arithmetic of pk_rownorm.h).
// One wavefront per row: each lane
// loads 16-byte vectors (8 f16 or 4 f32 channels; 4 f16 channels when the
// row length is not a multiple of 8) at a stride of 64 vectors, together
// with the gamma and beta of those channels, so a row costs one memory round
// trip before its two sums are reduced across the wavefront with cross-lane
// exchanges (no LDS, no barrier). The lane then normalises the vectors it
// still holds in registers (the first 4 KB of a row: 2048 f16 or 1024 f32
// channels) or re-reads from L2 beyond that. A chained launch (rows of at
// most 4 KB) then normalises the rounded output it still holds with a
// second gamma and beta, loaded in the first burst too: the sums run over
// the same values in the same lane order as a separate launch over the
// stored output, so both outputs are bit-identical to two launches.
#include "pk_internal.h"
#include "pk_rownorm.h"

namespace pk {
namespace {

constexpr int kRowsPerBlock = 4;
// HELD_BYTES: bytes of a row kept in registers, 2 KB for rows that fit
// (fewer registers, more waves per SIMD) or kLayerNormChainBytes.
template <typename T, int VEC, uint32_t HELD_BYTES, bool CHAIN>
__global__ __launch_bounds__(64 * kRowsPerBlock) void layernorm_kernel(LayerNormArgs args) {
  typedef T V __attribute__((ext_vector_type(VEC)));
  constexpr int kHeld = (int)(HELD_BYTES / (64u * VEC * sizeof(T)));  // vectors a lane keeps
  constexpr int F4 = VEC / 4;                                 // float4s of gamma per vector
  constexpr int kNext = CHAIN ? kHeld : 1;
  const int lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= args.rows) return;
  const uint32_t vectors = args.channels / (uint32_t)VEC;
  const V* in = static_cast<const V*>(args.input) + (uint64_t)row * vectors;
  V* out = static_cast<V*>(args.output) + (uint64_t)row * vectors;
  const float4* gamma = reinterpret_cast<const float4*>(args.gamma);
  const float4* beta = reinterpret_cast<const float4*>(args.beta);

  V held[kHeld];
  float4 g_held[kHeld][F4], b_held[kHeld][F4];
  float4 g_next[kNext][F4], b_next[kNext][F4];
#pragma unroll
  for (int i = 0; i < kHeld; ++i) {
    const uint32_t v = lane + 64u * i;
    if (v < vectors) held[i] = in[v];
  }
  auto load_affine = [&](const float* g, const float* b, int count, float4 (*gd)[F4], float4 (*bd)[F4]) {
    const float4* g4 = reinterpret_cast<const float4*>(g);
    const float4* b4 = reinterpret_cast<const float4*>(b);
#pragma unroll
    for (int i = 0; i < count; ++i) {
      const uint32_t v = lane + 64u * i;
      if (v < vectors)
#pragma unroll
        for (int f = 0; f < F4; ++f) {
          gd[i][f] = g4[v * F4 + f];
          bd[i][f] = b4[v * F4 + f];
        }
    }
  };
  load_affine(args.gamma, args.beta, kHeld, g_held, b_held);
  if constexpr (CHAIN) load_affine(args.next_gamma, args.next_beta, kNext, g_next, b_next);

  // Mean and 1 / sqrt(variance + epsilon) of the row whose held vectors are
  // `x` (and, past those, re-read from `rest`).
  auto statistics = [&](const V (&x)[kHeld], const V* rest) {
    float sum = 0.0f, square = 0.0f;
#pragma unroll
    for (int i = 0; i < kHeld; ++i)
      if (lane + 64u * i < vectors) rownorm_accumulate<VEC>(x[i], sum, square);
    for (uint32_t v = lane + 64u * kHeld; v < vectors; v += 64u) rownorm_accumulate<VEC>(rest[v], sum, square);
    return rownorm_finish(sum, square, args.channels, args.epsilon);
  };
  auto normalize = [&](const V& x, float2 st, const float4 (&g4)[F4], const float4 (&b4)[F4]) {
    return rownorm_apply<T, VEC>(x, st, g4, b4);
  };

  const float2 st = statistics(held, in);
#pragma unroll
  for (int i = 0; i < kHeld; ++i) {
    const uint32_t v = lane + 64u * i;
    if (v < vectors) {
      held[i] = normalize(held[i], st, g_held[i], b_held[i]);
      out[v] = held[i];
    }
  }
  if constexpr (CHAIN) {
    // The whole row is held (the host checks its size): normalise it again.
    V* next = static_cast<V*>(args.next_output) + (uint64_t)row * vectors;
    const float2 st2 = statistics(held, nullptr);
#pragma unroll
    for (int i = 0; i < kHeld; ++i) {
      const uint32_t v = lane + 64u * i;
      if (v < vectors) next[v] = normalize(held[i], st2, g_next[i], b_next[i]);
    }
  } else {
    for (uint32_t v = lane + 64u * kHeld; v < vectors; v += 64u) {
      float4 g4[F4], b4[F4];
#pragma unroll
      for (int f = 0; f < F4; ++f) {
        g4[f] = gamma[v * F4 + f];
        b4[f] = beta[v * F4 + f];
      }
      out[v] = normalize(in[v], st, g4, b4);
    }
  }
}

}  // namespace

uint32_t layernorm_grid(uint32_t rows) { return (rows + kRowsPerBlock - 1) / kRowsPerBlock; }

hipError_t launch_layernorm(bool f16, const LayerNormArgs& args, hipStream_t stream, hipEvent_t start,
                            hipEvent_t stop) {
  const uint32_t grid = layernorm_grid(args.rows);
  if (grid == 0) return hipSuccess;
  // 16-byte f16 vectors need rows of whole vectors (the bindings are
  // 16-byte aligned).
  const bool chain = args.next_output != nullptr;
  const uint64_t row_bytes = (uint64_t)args.channels * (f16 ? 2u : 4u);
  if (chain && row_bytes > kLayerNormChainBytes) return hipErrorInvalidValue;
  const bool small = row_bytes <= 2048u;
  const int shape = !f16 ? 0 : args.channels % 8u == 0u ? 1 : 2;  // f32 x4, f16 x8, f16 x4
  typedef void (*Kernel)(LayerNormArgs);
  static const Kernel kernels[3][2][2] = {
      {{layernorm_kernel<float, 4, kLayerNormChainBytes, false>, layernorm_kernel<float, 4, kLayerNormChainBytes, true>},
       {layernorm_kernel<float, 4, 2048, false>, layernorm_kernel<float, 4, 2048, true>}},
      {{layernorm_kernel<_Float16, 8, kLayerNormChainBytes, false>,
        layernorm_kernel<_Float16, 8, kLayerNormChainBytes, true>},
       {layernorm_kernel<_Float16, 8, 2048, false>, layernorm_kernel<_Float16, 8, 2048, true>}},
      {{layernorm_kernel<_Float16, 4, kLayerNormChainBytes, false>,
        layernorm_kernel<_Float16, 4, kLayerNormChainBytes, true>},
       {layernorm_kernel<_Float16, 4, 2048, false>, layernorm_kernel<_Float16, 4, 2048, true>}},
  };
  const Kernel kernel = kernels[shape][small][chain];
  if (start || stop)
    hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kRowsPerBlock), 0, stream, start, stop, 0, args);
  else
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kRowsPerBlock), 0, stream, args);
  return hipGetLastError();
}

}  // namespace pk

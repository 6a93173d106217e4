// pk_layernorm.hip - row LayerNorm for gfx950 (reference:
// src/webgpu/kernels/layernorm.ts, shader :309-390, dispatch :29-240).
//
// mean = sum(x) / C, variance = max(sum(x^2) / C - mean^2, 0),
// out = (x - mean) * rsqrt(variance + epsilon) * gamma + beta, statistics in
// f32, output rounded to the storage type. One wavefront per row: each lane
// loads 16-byte vectors (8 f16 or 4 f32 channels; 4 f16 channels when the
// row length is not a multiple of 8) at a stride of 64 vectors, together
// with the gamma and beta of those channels, so a row costs one memory round
// trip before its two sums are reduced across the wavefront with cross-lane
// exchanges (no LDS, no barrier). The lane then normalises the vectors it
// still holds in registers (the first 4 KB of a row: 2048 f16 or 1024 f32
// channels) or re-reads from L2 beyond that.
#include "pk_internal.h"

namespace pk {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr uint32_t kHeldBytes = 4096;  // bytes of a row kept in registers

template <typename T, int VEC>
__global__ __launch_bounds__(64 * kRowsPerBlock) void layernorm_kernel(LayerNormArgs args) {
  typedef T V __attribute__((ext_vector_type(VEC)));
  constexpr int kHeld = (int)(kHeldBytes / (64u * VEC * sizeof(T)));  // vectors a lane keeps
  constexpr int F4 = VEC / 4;                                 // float4s of gamma per vector
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
#pragma unroll
  for (int i = 0; i < kHeld; ++i) {
    const uint32_t v = lane + 64u * i;
    if (v < vectors) held[i] = in[v];
  }
#pragma unroll
  for (int i = 0; i < kHeld; ++i) {
    const uint32_t v = lane + 64u * i;
    if (v < vectors)
#pragma unroll
      for (int f = 0; f < F4; ++f) {
        g_held[i][f] = gamma[v * F4 + f];
        b_held[i][f] = beta[v * F4 + f];
      }
  }
  float sum = 0.0f, square = 0.0f;
  auto accumulate = [&](const V& x) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const float xc = (float)x[c];
      sum += xc;
      square = __builtin_fmaf(xc, xc, square);
    }
  };
#pragma unroll
  for (int i = 0; i < kHeld; ++i)
    if (lane + 64u * i < vectors) accumulate(held[i]);
  for (uint32_t v = lane + 64u * kHeld; v < vectors; v += 64u) accumulate(in[v]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    sum += __shfl_xor(sum, off, 64);
    square += __shfl_xor(square, off, 64);
  }
  const float inverse_channels = 1.0f / (float)args.channels;
  const float mean = sum * inverse_channels;
  const float variance = fmaxf(square * inverse_channels - mean * mean, 0.0f);
  const float inverse_std = 1.0f / __builtin_sqrtf(variance + args.epsilon);

  auto normalize = [&](uint32_t v, const V& x, const float4 (&g4)[F4], const float4 (&b4)[F4]) {
    V y;
#pragma unroll
    for (int f = 0; f < F4; ++f) {
      const float gg[4] = {g4[f].x, g4[f].y, g4[f].z, g4[f].w}, bb[4] = {b4[f].x, b4[f].y, b4[f].z, b4[f].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) y[4 * f + c] = (T)(((float)x[4 * f + c] - mean) * inverse_std * gg[c] + bb[c]);
    }
    out[v] = y;
  };
#pragma unroll
  for (int i = 0; i < kHeld; ++i) {
    const uint32_t v = lane + 64u * i;
    if (v < vectors) normalize(v, held[i], g_held[i], b_held[i]);
  }
  for (uint32_t v = lane + 64u * kHeld; v < vectors; v += 64u) {
    float4 g4[F4], b4[F4];
#pragma unroll
    for (int f = 0; f < F4; ++f) {
      g4[f] = gamma[v * F4 + f];
      b4[f] = beta[v * F4 + f];
    }
    normalize(v, in[v], g4, b4);
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
  void (*kernel)(LayerNormArgs) = !f16                     ? layernorm_kernel<float, 4>
                                  : args.channels % 8u == 0u ? layernorm_kernel<_Float16, 8>
                                                             : layernorm_kernel<_Float16, 4>;
  if (start || stop)
    hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kRowsPerBlock), 0, stream, start, stop, 0, args);
  else
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kRowsPerBlock), 0, stream, args);
  return hipGetLastError();
}

}  // namespace pk

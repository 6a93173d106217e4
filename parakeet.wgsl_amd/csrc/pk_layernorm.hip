// pk_layernorm.hip - row LayerNorm for gfx950 (reference:
// src/webgpu/kernels/layernorm.ts, shader :309-390, dispatch :29-240).
//
// mean = sum(x) / C, variance = max(sum(x^2) / C - mean^2, 0),
// out = (x - mean) * rsqrt(variance + epsilon) * gamma + beta, statistics in
// f32, output rounded to the storage type. One wavefront per row: each lane
// loads 4-channel vectors at a stride of 256 channels, the two sums are
// reduced across the wavefront with cross-lane exchanges (no LDS, no
// barrier), then the lane normalises the vectors it still holds in
// registers (rows up to 2048 channels) or re-reads from L2 beyond that.
#include "pk_internal.h"

namespace pk {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr int kHeld = 8;  // vectors a lane keeps in registers (2048 channels)

template <typename T>
struct Vec4 {
  typedef T type __attribute__((ext_vector_type(4)));
};

template <typename T>
__global__ __launch_bounds__(64 * kRowsPerBlock) void layernorm_kernel(LayerNormArgs args) {
  typedef typename Vec4<T>::type V;
  const int lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= args.rows) return;
  const uint32_t vectors = args.channels / 4u;
  const V* in = static_cast<const V*>(args.input) + (uint64_t)row * vectors;
  V* out = static_cast<V*>(args.output) + (uint64_t)row * vectors;
  const float4* gamma = reinterpret_cast<const float4*>(args.gamma);
  const float4* beta = reinterpret_cast<const float4*>(args.beta);

  V held[kHeld];
  float sum = 0.0f, square = 0.0f;
#pragma unroll
  for (int i = 0; i < kHeld; ++i) {
    const uint32_t v = lane + 64u * i;
    if (v < vectors) {
      held[i] = in[v];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float x = (float)held[i][c];
        sum += x;
        square = __builtin_fmaf(x, x, square);
      }
    }
  }
  for (uint32_t v = lane + 64u * kHeld; v < vectors; v += 64u) {
    const V x4 = in[v];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float x = (float)x4[c];
      sum += x;
      square = __builtin_fmaf(x, x, square);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    sum += __shfl_xor(sum, off, 64);
    square += __shfl_xor(square, off, 64);
  }
  const float inverse_channels = 1.0f / (float)args.channels;
  const float mean = sum * inverse_channels;
  const float variance = fmaxf(square * inverse_channels - mean * mean, 0.0f);
  const float inverse_std = 1.0f / __builtin_sqrtf(variance + args.epsilon);

  auto normalize = [&](uint32_t v, const V& x4) {
    const float4 g = gamma[v], b = beta[v];
    const float gg[4] = {g.x, g.y, g.z, g.w}, bb[4] = {b.x, b.y, b.z, b.w};
    V y;
#pragma unroll
    for (int c = 0; c < 4; ++c) y[c] = (T)(((float)x4[c] - mean) * inverse_std * gg[c] + bb[c]);
    out[v] = y;
  };
#pragma unroll
  for (int i = 0; i < kHeld; ++i) {
    const uint32_t v = lane + 64u * i;
    if (v < vectors) normalize(v, held[i]);
  }
  for (uint32_t v = lane + 64u * kHeld; v < vectors; v += 64u) normalize(v, in[v]);
}

}  // namespace

uint32_t layernorm_grid(uint32_t rows) { return (rows + kRowsPerBlock - 1) / kRowsPerBlock; }

hipError_t launch_layernorm(bool f16, const LayerNormArgs& args, hipStream_t stream, hipEvent_t start,
                            hipEvent_t stop) {
  const uint32_t grid = layernorm_grid(args.rows);
  if (grid == 0) return hipSuccess;
  void (*kernel)(LayerNormArgs) = f16 ? layernorm_kernel<_Float16> : layernorm_kernel<float>;
  if (start || stop)
    hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kRowsPerBlock), 0, stream, start, stop, 0, args);
  else
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * kRowsPerBlock), 0, stream, args);
  return hipGetLastError();
}

}  // namespace pk

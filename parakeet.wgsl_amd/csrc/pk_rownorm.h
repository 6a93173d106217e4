// pk_rownorm.h - the per-row LayerNorm arithmetic of the LayerNorm kernel
// (reference: src/webgpu/kernels/layernorm.ts, shader :309-390):
//   mean = sum(x) / C, variance = max(sum(x^2) / C - mean^2, 0),
//   out = (x - mean) * rsqrt(variance + epsilon) * gamma + beta,
// statistics in f32, one wavefront per row, a lane summing its vectors in
// order and the lanes' sums meeting by cross-lane exchanges. Every fused
// multiply-add is written out and each output is rounded from its f32
// value on its own, so no kernel's instruction selection (fp contraction,
// a mixed-precision fma that rounds straight to f16) changes the bits.
#pragma once
#include <hip/hip_runtime.h>

namespace pk {

// Adds the VEC channels of one vector to a lane's sum and sum of squares.
template <int VEC, typename V>
__device__ __forceinline__ void rownorm_accumulate(const V& xv, float& sum, float& square) {
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    const float xc = (float)xv[c];
    sum += xc;
    square = __builtin_fmaf(xc, xc, square);
  }
}

// (mean, 1 / sqrt(variance + epsilon)) of a row from its lanes' sums once
// they are reduced over the wavefront (rownorm_reduce).
__device__ __forceinline__ float2 rownorm_stats(float sum, float square, uint32_t channels, float epsilon) {
  const float inverse_channels = 1.0f / (float)channels;
  const float mean = sum * inverse_channels;
  const float variance = fmaxf(__builtin_fmaf(-mean, mean, square * inverse_channels), 0.0f);
  return make_float2(mean, 1.0f / __builtin_sqrtf(variance + epsilon));
}

// The butterfly over the 64 lanes: partners 32, 16, ..., 1 apart, each
// lane adding its partner's value (the same sums in every lane).
template <int ROWS>
__device__ __forceinline__ void rownorm_reduce(float (&sum)[ROWS], float (&square)[ROWS]) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      sum[r] += __shfl_xor(sum[r], off, 64);
      square[r] += __shfl_xor(square[r], off, 64);
    }
}

// (mean, 1 / sqrt(variance + epsilon)) of a row from its 64 lanes' sums.
__device__ __forceinline__ float2 rownorm_finish(float sum, float square, uint32_t channels, float epsilon) {
  float s[1] = {sum}, q[1] = {square};
  rownorm_reduce<1>(s, q);
  return rownorm_stats(s[0], q[0], channels, epsilon);
}

// One normalised vector, rounded to the storage type T.
template <typename T, int VEC, typename V>
__device__ __forceinline__ V rownorm_apply(const V& x, float2 st, const float4 (&g4)[VEC / 4],
                                           const float4 (&b4)[VEC / 4]) {
  V y;
#pragma unroll
  for (int f = 0; f < VEC / 4; ++f) {
    const float gg[4] = {g4[f].x, g4[f].y, g4[f].z, g4[f].w}, bb[4] = {b4[f].x, b4[f].y, b4[f].z, b4[f].w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float t = __builtin_fmaf(((float)x[4 * f + c] - st.x) * st.y, gg[c], bb[c]);
      __asm__("" : "+v"(t));  // t itself is rounded to T
      y[4 * f + c] = (T)t;
    }
  }
  return y;
}

}  // namespace pk

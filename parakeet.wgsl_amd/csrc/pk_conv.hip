// pk_conv.hip - the fused Conformer convolution tail for gfx950: GLU of the
// pointwise-1 output, same-padded depthwise k9 over frames, folded batch norm
// and SiLU in one HBM pass (reference: src/webgpu/kernels/conformer-conv.ts,
// shader :470-575, dispatch :117-162).
//
// Work split. A thread owns CPT adjacent channels of one batch item over a
// run of F output frames. It issues the F + 8 row loads its window needs
// (frames f0-4 .. f0+F+3, one vector load per half: value and gate) back to
// back, forms each row's GLU once in registers and slides the nine-tap window
// over them, so sigmoid runs (F + 8) / F times per GLU value instead of
// nine. Lanes run along channels: one wave load covers 64*CPT contiguous
// channels of a row, fully coalesced, and the neighbouring runs that re-read
// a run's eight halo rows sit in blocks placed on the same XCD (one L2).
// Measured on gfx950 the kernel is bound by its exp/rcp count, not by HBM:
// short runs keep every SIMD busy, longer runs (fewer halo sigmoids) pay
// back only once there are several waves per SIMD.
//
// Arithmetic follows the reference shader: glu = value * sigmoid(gate) in f32,
// zero for frames outside [0, frames) or past the item's valid length;
// sum = fma(glu, w[k], sum) over taps k = 0..8 in order; affine = sum * scale
// + shift; out = affine * sigmoid(affine), rounded to the storage type.
// sigmoid(x) = 1 / (1 + exp(-clamp(x, -20, 20))) with v_exp_f32 / v_rcp_f32.
#include <type_traits>

#include "pk_internal.h"

namespace pk {
namespace {

constexpr int kTaps = 9;
constexpr int kRadius = 4;
constexpr int kConvThreads = 256;

__device__ __forceinline__ float sigmoid(float v) {
  const float bounded = __builtin_amdgcn_fmed3f(v, -20.0f, 20.0f);
  const float e = __builtin_amdgcn_exp2f(bounded * -1.4426950408889634f);
  return __builtin_amdgcn_rcpf(1.0f + e);
}

template <typename T, int CPT>
struct Lanes {
  typedef T vec __attribute__((ext_vector_type(CPT)));
};

template <typename T, int CPT>
__device__ __forceinline__ void load_row(const T* p, float (&out)[CPT]) {
  typedef typename Lanes<T, CPT>::vec V;
  const V v = *reinterpret_cast<const V*>(p);
#pragma unroll
  for (int c = 0; c < CPT; ++c) out[c] = static_cast<float>(v[c]);
}

template <typename T, int CPT>
__device__ __forceinline__ void store_row(T* p, const float (&in)[CPT]) {
  typedef typename Lanes<T, CPT>::vec V;
  V v;
#pragma unroll
  for (int c = 0; c < CPT; ++c) v[c] = static_cast<T>(in[c]);
  *reinterpret_cast<V*>(p) = v;
}

// GLU_IN: the input rows already hold the GLU ([rows, C]); only the frame
// mask is applied to them.
template <typename T, int CPT, int F, bool GLU_IN>
__global__ __launch_bounds__(kConvThreads) void conformer_conv_kernel(ConvArgs args) {
  const uint32_t logical = xcd_local_order(blockIdx.x, gridDim.x);
  const uint32_t item = logical / args.blocks_per_item;
  const uint32_t slot = (logical % args.blocks_per_item) * kConvThreads + threadIdx.x;
  const uint32_t C = args.channels;
  const uint32_t groups = C / CPT;
  const uint32_t run = slot / groups;
  if (run >= args.runs) return;
  const uint32_t c0 = (slot % groups) * CPT;
  const int frames = (int)args.frames;
  const int live_end = (int)min(args.frames, args.valid_lengths[item]);
  const int f0 = (int)run * F;

  constexpr uint32_t kInRows = GLU_IN ? 1u : 2u;  // input row length in channels
  const T* in = static_cast<const T*>(args.input) + (uint64_t)item * args.frames * (kInRows * C) + c0;
  const T* weights = static_cast<const T*>(args.weights) + c0;
  T* out = static_cast<T*>(args.output) + (uint64_t)item * args.frames * C + c0;

  // Every row load is issued unconditionally from a clamped frame, so the
  // F + 8 loads go out back to back; rows outside the live range are zeroed
  // after the load.
  typedef typename Lanes<T, CPT>::vec V;
  V value[F + kTaps - 1], gate[F + kTaps - 1];
#pragma unroll
  for (int i = 0; i < F + kTaps - 1; ++i) {
    const T* row = in + (uint64_t)min(max(f0 - kRadius + i, 0), frames - 1) * (kInRows * C);
    value[i] = *reinterpret_cast<const V*>(row);
    if constexpr (!GLU_IN) gate[i] = *reinterpret_cast<const V*>(row + C);
  }
  float w[kTaps][CPT], scale[CPT], shift[CPT];
#pragma unroll
  for (int k = 0; k < kTaps; ++k) load_row<T, CPT>(weights + (uint64_t)k * C, w[k]);
  load_row<float, CPT>(args.scale + c0, scale);
  load_row<float, CPT>(args.shift + c0, shift);

  float glu[F + kTaps - 1][CPT];
#pragma unroll
  for (int i = 0; i < F + kTaps - 1; ++i) {
    const int r = f0 - kRadius + i;
    const bool live = r >= 0 && r < live_end;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      if constexpr (GLU_IN)
        glu[i][c] = live ? static_cast<float>(value[i][c]) : 0.0f;
      else
        glu[i][c] = live ? static_cast<float>(value[i][c]) * sigmoid(static_cast<float>(gate[i][c])) : 0.0f;
    }
  }

#pragma unroll
  for (int o = 0; o < F; ++o) {
    const int f = f0 + o;
    if (f >= frames) break;
    float result[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      float sum = 0.0f;
#pragma unroll
      for (int k = 0; k < kTaps; ++k) sum = __builtin_fmaf(glu[o + k][c], w[k][c], sum);
      const float affine = sum * scale[c] + shift[c];
      result[c] = affine * sigmoid(affine);
    }
    store_row<T, CPT>(out + (uint64_t)f * C, result);
  }
}

struct ConvVariant {
  const char* name;
  const char* glu_name;
  int channels_per_thread;
  int frames_per_thread;
  void (*kernel)(ConvArgs);
  void (*glu_kernel)(ConvArgs);  // GLU_IN
};

#define PK_CONV_VARIANT(T, TN, CPT, F)                                                                     \
  ConvVariant {                                                                                            \
    "pk_conformer_conv_" TN "_c" #CPT "_f" #F, "pk_conformer_conv_glu_" TN "_c" #CPT "_f" #F, CPT, F,      \
        conformer_conv_kernel<T, CPT, F, false>, conformer_conv_kernel<T, CPT, F, true>                    \
  }

// First entry of each list is the default launch shape (fastest measured on
// 16 x 188 x 1024 and 64 x 188 x 1024).
const ConvVariant kF16Variants[] = {
    PK_CONV_VARIANT(_Float16, "f16", 2, 8),
    PK_CONV_VARIANT(_Float16, "f16", 2, 16),
    PK_CONV_VARIANT(_Float16, "f16", 2, 4),
    PK_CONV_VARIANT(_Float16, "f16", 4, 4),
    PK_CONV_VARIANT(_Float16, "f16", 4, 8),
};
const ConvVariant kF32Variants[] = {
    PK_CONV_VARIANT(float, "f32", 2, 8),
    PK_CONV_VARIANT(float, "f32", 2, 16),
    PK_CONV_VARIANT(float, "f32", 4, 4),
    PK_CONV_VARIANT(float, "f32", 4, 8),
};

const ConvVariant& conv_variant_at(bool f16, int index) { return f16 ? kF16Variants[index] : kF32Variants[index]; }

}  // namespace

int conv_variant_count(bool f16) {
  return f16 ? (int)(sizeof(kF16Variants) / sizeof(kF16Variants[0]))
             : (int)(sizeof(kF32Variants) / sizeof(kF32Variants[0]));
}

ConvGeometry conv_geometry(bool f16, int variant, uint32_t frames, uint32_t channels, uint32_t batch,
                           bool input_glu) {
  const ConvVariant& v = conv_variant_at(f16, variant);
  ConvGeometry g;
  g.name = input_glu ? v.glu_name : v.name;
  g.channels_per_thread = v.channels_per_thread;
  g.runs = (frames + v.frames_per_thread - 1) / v.frames_per_thread;
  const uint64_t threads = (uint64_t)g.runs * (channels / v.channels_per_thread);
  g.blocks_per_item = (uint32_t)((threads + kConvThreads - 1) / kConvThreads);
  g.grid = g.blocks_per_item * batch;
  g.block_threads = kConvThreads;
  return g;
}

hipError_t launch_conformer_conv(bool f16, int variant, const ConvArgs& base, uint32_t batch, hipStream_t stream,
                                 hipEvent_t start, hipEvent_t stop) {
  const ConvVariant& v = conv_variant_at(f16, variant);
  const ConvGeometry g = conv_geometry(f16, variant, base.frames, base.channels, batch, base.input_glu != 0);
  if (g.grid == 0) return hipSuccess;
  ConvArgs args = base;
  args.runs = g.runs;
  args.blocks_per_item = g.blocks_per_item;
  void (*kernel)(ConvArgs) = base.input_glu ? v.glu_kernel : v.kernel;
  if (start || stop)
    hipExtLaunchKernelGGL(kernel, dim3(g.grid), dim3(g.block_threads), 0, stream, start, stop, 0, args);
  else
    hipLaunchKernelGGL(kernel, dim3(g.grid), dim3(g.block_threads), 0, stream, args);
  return hipGetLastError();
}

}  // namespace pk

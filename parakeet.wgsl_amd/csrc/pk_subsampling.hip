// pk_subsampling.hip - the convolution stages of the subsampling front end
// for gfx950 (reference: src/webgpu/kernels/subsampling.ts, shaders
// :1092-1430).
//
// Fused conv0 + depthwise2. A block owns a 4 x 8 tile of output positions
// for 64 channels of one window. It stages the 19 x 35 feature patch the
// tile needs in LDS (time-contiguous loads from the feature-major input),
// evaluates the 9 x 17 conv0 positions under the tile once per channel
// (bias + nine fma in tap order, ReLU, rounded to the storage type into an
// LDS tile) and then the 32 depthwise outputs from that tile. Each thread
// keeps one channel group's weights of each stage in registers (8 channels
// for f32, so one LDS feature read feeds eight fma; 4 for f16), and a tile
// whose every tap is in range (most of them) runs without the per-tap
// checks. conv0 never reaches HBM:
// the kernel reads the features once and writes the [Ho, Wo, C] output
// once.
//
// Depthwise (stage 5) and the time mask are bandwidth kernels: one thread
// per output position and 4-channel group, lanes along channels, so a
// wavefront reads and writes contiguous 512-byte runs of a row.
//
// Arithmetic follows the shaders exactly: every sum starts from the bias
// and adds one fmaf per in-range tap in (ky, kx) order, skipping taps outside
// the input or past the valid rows; outputs are rounded to the storage type
// once. Valid rows after s stride-2 stages are (L + 1) / 2 applied s times.
#include <type_traits>

#include "pk_internal.h"

namespace pk {
namespace {

constexpr int kTileRows = 4;
constexpr int kTileCols = 8;
constexpr int kBlockChannels = 64;

constexpr int kConvRows = 2 * kTileRows + 1;         // 9
constexpr int kConvCols = 2 * kTileCols + 1;         // 17
constexpr int kConvPositions = kConvRows * kConvCols;  // 153
constexpr int kFeatureRows = 2 * kConvRows + 1;       // 19 frames
constexpr int kFeatureCols = 2 * kConvCols + 1;       // 35 bins
constexpr int kFusedThreads = 256;
constexpr int kStreamThreads = 256;

__device__ __forceinline__ uint32_t subsampled(uint32_t length, uint32_t steps) {
  for (uint32_t s = 0; s < steps; ++s) length = (length + 1u) / 2u;
  return length;
}

template <typename T>
struct Vec4 {
  typedef T type __attribute__((ext_vector_type(4)));
};

template <typename T>
__device__ __forceinline__ void load4(const T* p, float (&out)[4]) {
  const typename Vec4<T>::type v = *reinterpret_cast<const typename Vec4<T>::type*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = (float)v[i];
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const float (&in)[4]) {
  typename Vec4<T>::type v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = (T)in[i];
  *reinterpret_cast<typename Vec4<T>::type*>(p) = v;
}

template <typename T, int N>
struct VecN {
  typedef T type __attribute__((ext_vector_type(N)));
};

// N (4 or 8) channels from / to memory, as f32.
template <int N, typename T>
__device__ __forceinline__ void load_n(const T* p, float (&out)[N]) {
#pragma unroll
  for (int h = 0; h < N / 4; ++h) {
    float part[4];
    load4(p + 4 * h, part);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[4 * h + i] = part[i];
  }
}

template <int N, typename T>
__device__ __forceinline__ void store_n(T* p, const float (&in)[N]) {
  typename VecN<T, N>::type v;
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = (T)in[i];
  *reinterpret_cast<typename VecN<T, N>::type*>(p) = v;
}

// grid: (ceil(Wo / 8), ceil(Ho / 4), batch * C / 64); CPT channels per
// thread (8 for f32: one LDS feature read feeds eight fma; 4 for f16, whose
// lighter threads keep more workgroups resident, which measured faster).
template <typename T, int CPT>
__global__ __launch_bounds__(kFusedThreads) void subsampling_fused_kernel(SubsamplingArgs a) {
  typedef typename VecN<T, CPT>::type V;
  constexpr int kGroups = kBlockChannels / CPT;
  constexpr int kPositionLanes = kFusedThreads / kGroups;
  __shared__ float features[kFeatureCols][kFeatureRows];
  __shared__ V conv0[kConvPositions][kGroups];

  const uint32_t blocks_per_window = a.channels / kBlockChannels;
  const uint32_t window = blockIdx.z / blocks_per_window;
  const uint32_t c0 = (blockIdx.z % blocks_per_window) * kBlockChannels + (threadIdx.x % kGroups) * CPT;
  const int group = threadIdx.x % kGroups;
  const int lane = threadIdx.x / kGroups;
  const int oy0 = blockIdx.y * kTileRows, ox0 = blockIdx.x * kTileCols;
  const int cy0 = 2 * oy0 - 1, cx0 = 2 * ox0 - 1;  // conv0 origin of the tile
  const int fy0 = 2 * cy0 - 1, fx0 = 2 * cx0 - 1;  // feature origin
  const int height = (int)a.height, width = (int)a.width;
  const int mid_height = (int)a.mid_height, mid_width = (int)a.mid_width;
  const uint32_t length = a.valid_lengths[window];
  const int valid1 = (int)subsampled(length, 1), valid2 = (int)subsampled(length, 2);
  // Every conv0 position under the tile and every tap of both stages in
  // range: no tap is skipped, so the sums need no per-tap checks (the
  // same terms in the same order as the checked path).
  const bool interior = fy0 >= 0 && fy0 + kFeatureRows <= height && fx0 >= 0 && fx0 + kFeatureCols <= width &&
                        cy0 >= 0 && cy0 + kConvRows <= min(mid_height, valid1) && cx0 >= 0 &&
                        cx0 + kConvCols <= mid_width && oy0 + kTileRows <= min((int)a.out_height, valid2) &&
                        ox0 + kTileCols <= (int)a.out_width;

  const float* input = static_cast<const float*>(a.input) + (uint64_t)window * a.width * a.height;
  for (int e = threadIdx.x; e < kFeatureCols * kFeatureRows; e += kFusedThreads) {
    const int col = e / kFeatureRows, row = e % kFeatureRows;
    const int bin = fx0 + col, frame = fy0 + row;
    features[col][row] = (bin >= 0 && bin < width && frame >= 0 && frame < height)
                             ? input[(uint64_t)bin * a.height + frame]
                             : 0.0f;
  }
  float w[9][CPT], bias[CPT];
  const T* conv0_weights = static_cast<const T*>(a.weights) + c0;
#pragma unroll
  for (int t = 0; t < 9; ++t) load_n<CPT>(conv0_weights + (uint64_t)t * a.channels, w[t]);
  load_n<CPT>(a.bias + c0, bias);
  __syncthreads();

  // conv0: bias + nine fma in (ky, kx) order, ReLU, rounded to T.
  auto conv0_at = [&](int p, auto checked) {
    constexpr bool CHECK = decltype(checked)::value;
    const int r = p / kConvCols, q = p % kConvCols;
    const int cy = cy0 + r, cx = cx0 + q;
    float v[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) v[i] = 0.0f;
    if (!CHECK || (cy >= 0 && cy < mid_height && cy < valid1 && cx >= 0 && cx < mid_width)) {
      float sum[CPT];
#pragma unroll
      for (int i = 0; i < CPT; ++i) sum[i] = bias[i];
#pragma unroll
      for (int ky = 0; ky < 3; ++ky) {
        const int iy = 2 * cy + ky - 1;
        if (CHECK && (iy < 0 || iy >= height)) continue;
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
          const int ix = 2 * cx + kx - 1;
          if (CHECK && (ix < 0 || ix >= width)) continue;
          const float f = features[2 * q + kx][2 * r + ky];
#pragma unroll
          for (int i = 0; i < CPT; ++i) sum[i] = __builtin_fmaf(w[ky * 3 + kx][i], f, sum[i]);
        }
      }
#pragma unroll
      for (int i = 0; i < CPT; ++i) v[i] = fmaxf(sum[i], 0.0f);
    }
    V stored;
#pragma unroll
    for (int i = 0; i < CPT; ++i) stored[i] = (T)v[i];
    conv0[p][group] = stored;
  };
  if (interior) {
    for (int p = lane; p < kConvPositions; p += kPositionLanes) conv0_at(p, std::false_type{});
  } else {
    for (int p = lane; p < kConvPositions; p += kPositionLanes) conv0_at(p, std::true_type{});
  }
  const T* depthwise_weights = static_cast<const T*>(a.weights2) + c0;
#pragma unroll
  for (int t = 0; t < 9; ++t) load_n<CPT>(depthwise_weights + (uint64_t)t * a.channels, w[t]);
  load_n<CPT>(a.bias2 + c0, bias);
  __syncthreads();

  // depthwise2: bias + nine fma in (ky, kx) order, rounded to T.
  T* out = static_cast<T*>(a.output);
  auto depthwise_at = [&](int q, auto checked) {
    constexpr bool CHECK = decltype(checked)::value;
    const int orow = q / kTileCols, ocol = q % kTileCols;
    const int oy = oy0 + orow, ox = ox0 + ocol;
    if (CHECK && (oy >= (int)a.out_height || ox >= (int)a.out_width)) return;
    T* dst = out + (((uint64_t)window * a.out_height + oy) * a.out_width + ox) * a.channels + c0;
    float sum[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) sum[i] = 0.0f;
    if (!CHECK || oy < valid2) {
#pragma unroll
      for (int i = 0; i < CPT; ++i) sum[i] = bias[i];
#pragma unroll
      for (int ky = 0; ky < 3; ++ky) {
        const int iy = 2 * oy + ky - 1;
        if (CHECK && (iy < 0 || iy >= mid_height || iy >= valid1)) continue;
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
          const int ix = 2 * ox + kx - 1;
          if (CHECK && (ix < 0 || ix >= mid_width)) continue;
          const V c = conv0[(2 * orow + ky) * kConvCols + 2 * ocol + kx][group];
#pragma unroll
          for (int i = 0; i < CPT; ++i) sum[i] = __builtin_fmaf((float)c[i], w[ky * 3 + kx][i], sum[i]);
        }
      }
    }
    store_n<CPT>(dst, sum);
  };
  if (interior) {
    for (int q = lane; q < kTileRows * kTileCols; q += kPositionLanes) depthwise_at(q, std::false_type{});
  } else {
    for (int q = lane; q < kTileRows * kTileCols; q += kPositionLanes) depthwise_at(q, std::true_type{});
  }
}

// One thread per (window, output row, output column, 4-channel group).
template <typename T>
__global__ __launch_bounds__(kStreamThreads) void subsampling_depthwise_kernel(SubsamplingArgs a, uint64_t total) {
  const uint64_t idx = (uint64_t)blockIdx.x * kStreamThreads + threadIdx.x;
  if (idx >= total) return;
  const uint32_t groups = a.channels / 4u;
  const uint32_t c0 = (uint32_t)(idx % groups) * 4u;
  uint64_t pos = idx / groups;
  const int ox = (int)(pos % a.out_width);
  pos /= a.out_width;
  const int oy = (int)(pos % a.out_height);
  const uint32_t window = (uint32_t)(pos / a.out_height);
  const uint32_t length = a.valid_lengths[window];
  T* dst = static_cast<T*>(a.output) + (((uint64_t)window * a.out_height + oy) * a.out_width + ox) * a.channels + c0;
  float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (oy < (int)subsampled(length, a.steps)) {
    const int valid_in = (int)subsampled(length, a.steps - 1u);
    load4(a.bias + c0, sum);
    const T* in = static_cast<const T*>(a.input) + (uint64_t)window * a.height * a.width * a.channels + c0;
    const T* weights = static_cast<const T*>(a.weights) + c0;
#pragma unroll
    for (int ky = 0; ky < 3; ++ky) {
      const int iy = 2 * oy + ky - 1;
      if (iy < 0 || iy >= (int)a.height || iy >= valid_in) continue;
#pragma unroll
      for (int kx = 0; kx < 3; ++kx) {
        const int ix = 2 * ox + kx - 1;
        if (ix < 0 || ix >= (int)a.width) continue;
        float x[4], w[4];
        load4(in + ((uint64_t)iy * a.width + ix) * a.channels, x);
        load4(weights + (uint64_t)(ky * 3 + kx) * a.channels, w);
#pragma unroll
        for (int i = 0; i < 4; ++i) sum[i] = __builtin_fmaf(x[i], w[i], sum[i]);
      }
    }
  }
  store4(dst, sum);
}

// grid: (height, batch); frames at or past the valid rows are zeroed.
template <typename T>
__global__ __launch_bounds__(kStreamThreads) void subsampling_mask_kernel(SubsamplingArgs a) {
  const uint32_t frame = blockIdx.x, window = blockIdx.y;
  if (frame < subsampled(a.valid_lengths[window], a.steps)) return;
  const uint32_t vectors = a.width * (a.channels / 4u);
  T* row = static_cast<T*>(a.output) + ((uint64_t)window * a.height + frame) * a.width * a.channels;
  const float zero[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t v = threadIdx.x; v < vectors; v += kStreamThreads) store4(row + (uint64_t)v * 4u, zero);
}

}  // namespace

SubsamplingGeometry subsampling_geometry(int kind, bool f16, const SubsamplingArgs& a, uint32_t batch) {
  SubsamplingGeometry g{};
  g.grid[1] = g.grid[2] = 1;
  if (kind == kSubsamplingFused) {
    g.name = f16 ? "pk_subsampling_conv0_depthwise2_f16" : "pk_subsampling_conv0_depthwise2_f32";
    g.grid[0] = (a.out_width + kTileCols - 1) / kTileCols;
    g.grid[1] = (a.out_height + kTileRows - 1) / kTileRows;
    g.grid[2] = batch * (a.channels / kBlockChannels);
    g.block_threads = kFusedThreads;
    g.lds_bytes = kFeatureCols * kFeatureRows * 4 + kConvPositions * kBlockChannels * (f16 ? 2 : 4);
  } else if (kind == kSubsamplingDepthwise) {
    g.name = f16 ? "pk_subsampling_depthwise_f16" : "pk_subsampling_depthwise_f32";
    const uint64_t total = (uint64_t)batch * a.out_height * a.out_width * (a.channels / 4u);
    g.grid[0] = (uint32_t)((total + kStreamThreads - 1) / kStreamThreads);
    g.block_threads = kStreamThreads;
  } else {
    g.name = f16 ? "pk_subsampling_time_mask_f16" : "pk_subsampling_time_mask_f32";
    g.grid[0] = a.height;
    g.grid[1] = batch;
    g.block_threads = kStreamThreads;
  }
  return g;
}

hipError_t launch_subsampling(int kind, bool f16, const SubsamplingArgs& args, uint32_t batch, hipStream_t stream,
                              hipEvent_t start, hipEvent_t stop) {
  const SubsamplingGeometry g = subsampling_geometry(kind, f16, args, batch);
  if (batch == 0 || g.grid[0] == 0 || g.grid[1] == 0 || g.grid[2] == 0) return hipSuccess;
  const dim3 grid(g.grid[0], g.grid[1], g.grid[2]), block(g.block_threads);
  const uint64_t total = (uint64_t)batch * args.out_height * args.out_width * (args.channels / 4u);
  const bool timed = start || stop;
  if (kind == kSubsamplingFused) {
    void (*k)(SubsamplingArgs) = f16 ? subsampling_fused_kernel<_Float16, 4> : subsampling_fused_kernel<float, 8>;
    if (timed)
      hipExtLaunchKernelGGL(k, grid, block, 0, stream, start, stop, 0, args);
    else
      hipLaunchKernelGGL(k, grid, block, 0, stream, args);
  } else if (kind == kSubsamplingDepthwise) {
    void (*k)(SubsamplingArgs, uint64_t) =
        f16 ? subsampling_depthwise_kernel<_Float16> : subsampling_depthwise_kernel<float>;
    if (timed)
      hipExtLaunchKernelGGL(k, grid, block, 0, stream, start, stop, 0, args, total);
    else
      hipLaunchKernelGGL(k, grid, block, 0, stream, args, total);
  } else {
    void (*k)(SubsamplingArgs) = f16 ? subsampling_mask_kernel<_Float16> : subsampling_mask_kernel<float>;
    if (timed)
      hipExtLaunchKernelGGL(k, grid, block, 0, stream, start, stop, 0, args);
    else
      hipLaunchKernelGGL(k, grid, block, 0, stream, args);
  }
  return hipGetLastError();
}

}  // namespace pk

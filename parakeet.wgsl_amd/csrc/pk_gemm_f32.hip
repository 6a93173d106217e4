// pk_gemm_f32.hip - fused palette-weight GEMM, f32 operands and f32 MFMA
// (v_mfma_f32_32x32x2_f32) for gfx950: the FP32 twin of pk_gemm_f16.hip
// (reference: src/webgpu/kernels/gemm.ts:2356-2599, epilogue :2847-2869).
//
// Same operand-order codes as the f16 kernel: in MFMA step s (0..31) of a
// 64-deep K block, lane half h stands for k = 64*kb + 32*h + s in both
// operands, which is code u = s of the lane's 32-code stream. One decoded
// code per lane feeds one MFMA per row block, so decode work is small next
// to the 64-cycle f32 MFMA.
#include "pk_internal.h"

namespace pk {
namespace {

typedef float float16v __attribute__((ext_vector_type(16)));

template <int BITS>
__device__ __forceinline__ uint32_t lane_code(const uint32_t* w, int u) {
  constexpr uint32_t mask = (1u << BITS) - 1u;
  const int bit = u * BITS;
  const int word = bit >> 5;
  const int shift = bit & 31;
  if (shift + BITS <= 32) return (w[word] >> shift) & mask;
  return __builtin_amdgcn_alignbit(w[word + 1], w[word], shift) & mask;
}

// SiLU of the reference epilogue, v / (1 + exp(-clamp(v, -20, 20)))
// (gemm.ts:2847-2869 with the activation of :2006-2044): clamp, exp as
// v_exp_f32 of the base-2 argument and v_rcp_f32, each within ~1 ulp.
__device__ __forceinline__ float silu(float v) {
  const float bounded = __builtin_amdgcn_fmed3f(v, -20.0f, 20.0f);
  const float e = __builtin_amdgcn_exp2f(bounded * -1.4426950408889634f);
  return v * __builtin_amdgcn_rcpf(1.0f + e);
}

template <int BITS, int WM, int WN, int MB, int NB>
__global__ __launch_bounds__(64 * WM * WN) void gemm_f32_kernel(GemmArgs args) {
  constexpr int T = 64 * WM * WN;
  constexpr int BM = 32 * WM * MB;
  constexpr int BN = 32 * WN * NB;
  constexpr int E = 1 << BITS;
  constexpr int LUT_CAP = (BN / 16 + 2) * E;
  constexpr int ROW_BYTES = 256;  // 64 floats of one row per K step
  constexpr int CH = BM * 16 / T;
  static_assert(BM * 16 % T == 0, "A tile chunks must divide evenly");

  __shared__ __attribute__((aligned(16))) uint8_t a_lds[2][BM * ROW_BYTES];
  __shared__ float lut_lds[LUT_CAP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_m = wave / WN;
  const int wave_n = wave % WN;
  const int j = lane & 31;
  const int h = lane >> 5;

  const uint32_t M = args.rows;
  const uint32_t K = args.inner;
  const uint32_t N = args.columns;
  const uint32_t k_blocks = (K + 63u) / 64u;
  const uint32_t n_blocks_total = (N + 31u) / 32u;
  const uint32_t n0 = blockIdx.x * BN;
  const uint32_t m0 = blockIdx.y * BM;

  const uint32_t gc = args.palette_group_columns;
  const uint32_t G = args.palette_groups;
  const uint32_t g_lo = min(n0 / gc, G - 1u);
  const uint32_t g_hi = min((min(n0 + BN, N) - 1u) / gc, G - 1u);
  {
    const uint32_t entries = (g_hi - g_lo + 1u) * E;
    const float* src = static_cast<const float*>(args.palette) + (uint64_t)g_lo * E;
    for (uint32_t i = tid; i < entries; i += T) lut_lds[i] = src[i];
  }
  const float* lut_col[NB];
#pragma unroll
  for (int ni = 0; ni < NB; ++ni) {
    const uint32_t n = n0 + (wave_n * NB + ni) * 32 + j;
    const uint32_t g = min(n / gc, G - 1u) - g_lo;
    lut_col[ni] = lut_lds + g * E;
  }

  const uint32_t nb0 = n0 / 32u + wave_n * NB;
  uint32_t cw[NB][BITS];
  auto load_codes = [&](uint32_t kb, uint32_t (&dst)[NB][BITS]) {
#pragma unroll
    for (int ni = 0; ni < NB; ++ni) {
      const uint32_t nb = nb0 + ni;
      if (nb < n_blocks_total) {
        const uint32_t* blk = args.codes + ((uint64_t)nb * k_blocks + kb) * block_words(BITS);
        const uint4 p0 = reinterpret_cast<const uint4*>(blk)[lane];
        dst[ni][0] = p0.x;
        dst[ni][1] = p0.y;
        dst[ni][2] = p0.z;
        dst[ni][3] = p0.w;
        if constexpr (BITS == 5) {
          dst[ni][4] = blk[256 + lane];
        } else {
          const uint2 p1 = reinterpret_cast<const uint2*>(blk + 256)[lane];
          dst[ni][4] = p1.x;
          dst[ni][5] = p1.y;
        }
      } else {
#pragma unroll
        for (int q = 0; q < BITS; ++q) dst[ni][q] = 0u;
      }
    }
  };

  const float* a_ptr = static_cast<const float*>(args.a);
  uint4 a_stage[CH];
  auto load_a = [&](uint32_t kb) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int idx = tid + c * T;
      const int r = idx >> 4;
      const int ch = idx & 15;
      const uint32_t m = m0 + r;
      const uint32_t k = kb * 64u + ch * 4u;
      if (m < M && k < K)
        a_stage[c] = *reinterpret_cast<const uint4*>(a_ptr + (uint64_t)m * K + k);
      else
        a_stage[c] = make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int idx = tid + c * T;
      const int r = idx >> 4;
      const int ch = idx & 15;
      *reinterpret_cast<uint4*>(&a_lds[buf][r * ROW_BYTES + ((ch ^ (r & 7)) << 4)]) = a_stage[c];
    }
  };

  float16v acc[MB][NB];
#pragma unroll
  for (int mi = 0; mi < MB; ++mi)
#pragma unroll
    for (int ni = 0; ni < NB; ++ni)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ni][v] = 0.0f;

  load_codes(0, cw);
  load_a(0);
  store_a(0);
  __syncthreads();

  for (uint32_t kb = 0; kb < k_blocks; ++kb) {
    const int buf = kb & 1;
    const bool more = kb + 1 < k_blocks;
    uint32_t cn[NB][BITS];
    if (more) {
      load_codes(kb + 1, cn);
      load_a(kb + 1);
    }
    const uint8_t* tile = a_lds[buf];
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {
      float4 af[MB];
#pragma unroll
      for (int mi = 0; mi < MB; ++mi) {
        const int r = (wave_m * MB + mi) * 32 + j;
        const int ch = h * 8 + s4;
        af[mi] = *reinterpret_cast<const float4*>(&tile[r * ROW_BYTES + ((ch ^ (r & 7)) << 4)]);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float bw[NB];
#pragma unroll
        for (int ni = 0; ni < NB; ++ni) bw[ni] = lut_col[ni][lane_code<BITS>(cw[ni], s4 * 4 + t)];
#pragma unroll
        for (int mi = 0; mi < MB; ++mi) {
          const float a = t == 0 ? af[mi].x : t == 1 ? af[mi].y : t == 2 ? af[mi].z : af[mi].w;
#pragma unroll
          for (int ni = 0; ni < NB; ++ni)
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(bw[ni], a, acc[mi][ni], 0, 0, 0);
        }
      }
    }
    if (more) {
      store_a(buf ^ 1);
#pragma unroll
      for (int ni = 0; ni < NB; ++ni)
#pragma unroll
        for (int q = 0; q < BITS; ++q) cw[ni][q] = cn[ni][q];
    }
    __syncthreads();
  }

  float* out = static_cast<float*>(args.out);
  const float* residual = static_cast<const float*>(args.residual);
#pragma unroll
  for (int mi = 0; mi < MB; ++mi) {
    const uint32_t m = m0 + (wave_m * MB + mi) * 32 + j;
    if (m >= M) continue;
#pragma unroll
    for (int ni = 0; ni < NB; ++ni) {
      const uint32_t nbase = n0 + (wave_n * NB + ni) * 32 + h * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t n = nbase + q * 8;
        if (n >= N) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[mi][ni][q * 4 + e];
        if (args.bias) {
          const float4 b = *reinterpret_cast<const float4*>(args.bias + n);
          v[0] += b.x;
          v[1] += b.y;
          v[2] += b.z;
          v[3] += b.w;
        }
        if (args.activation == kActSilu) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = silu(v[e]);
        } else if (args.activation == kActRelu) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = fmaxf(v[e], 0.0f);
        }
        const uint64_t at = (uint64_t)m * N + n;
        if (residual) {
          const float4 r = *reinterpret_cast<const float4*>(residual + at);
          v[0] = r.x + args.residual_scale * v[0];
          v[1] = r.y + args.residual_scale * v[1];
          v[2] = r.z + args.residual_scale * v[2];
          v[3] = r.w + args.residual_scale * v[3];
        }
        *reinterpret_cast<float4*>(out + at) = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  }
}

struct Variant {
  TileShape shape;
  const char* name5;
  const char* name6;
  void (*kernel5)(GemmArgs);
  void (*kernel6)(GemmArgs);
};

#define PK_F32_VARIANT(WM, WN, MB, NB)                                             \
  Variant {                                                                        \
    TileShape{WM, WN, MB, NB}, "pk_gemm_f32_b5_w" #WM "x" #WN "_m" #MB "n" #NB,    \
        "pk_gemm_f32_b6_w" #WM "x" #WN "_m" #MB "n" #NB,                           \
        gemm_f32_kernel<5, WM, WN, MB, NB>, gemm_f32_kernel<6, WM, WN, MB, NB>     \
  }

const Variant kVariants[] = {
    PK_F32_VARIANT(1, 4, 1, 1),  // 32 x 128
    PK_F32_VARIANT(1, 4, 2, 1),  // 64 x 128
    PK_F32_VARIANT(1, 4, 2, 2),  // 64 x 256
    PK_F32_VARIANT(2, 2, 2, 2),  // 128 x 128
    PK_F32_VARIANT(1, 2, 1, 1),  // 32 x 64
};

}  // namespace

int f32_variant_count() { return (int)(sizeof(kVariants) / sizeof(kVariants[0])); }
TileShape f32_variant(int index) { return kVariants[index].shape; }
const char* f32_variant_name(int bits, int index) {
  return bits == 5 ? kVariants[index].name5 : kVariants[index].name6;
}

hipError_t launch_gemm_f32(int bits, int variant, const GemmArgs& args, hipStream_t stream, hipEvent_t start,
                           hipEvent_t stop) {
  const Variant& v = kVariants[variant];
  const uint32_t n_pad = padded_columns(args.columns);
  const dim3 grid((n_pad + v.shape.tile_columns() - 1) / v.shape.tile_columns(),
                  (args.rows + v.shape.tile_rows() - 1) / v.shape.tile_rows());
  if (grid.y == 0) return hipSuccess;
  return launch_timed(bits == 5 ? v.kernel5 : v.kernel6, grid, dim3(v.shape.threads()), stream, start, stop, args);
}

}  // namespace pk

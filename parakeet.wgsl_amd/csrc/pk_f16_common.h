// pk_f16_common.h - device helpers shared by the f16 palette GEMM kernels
// (pk_gemm_f16.hip, pk_gemm_f16k.hip): code extraction and palette gathers,
// the split-K reduction and the LDS-staged epilogue.
#pragma once

#include "pk_internal.h"

namespace pk {
namespace f16 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kRowBytes = 128;  // 64 halves of one row (or column) per K block

// Code u (0..31) of a lane's 32-code stream, LSB first at bit u*BITS.
template <int BITS>
__device__ __forceinline__ uint32_t lane_code(const uint32_t (&w)[BITS], int u) {
  constexpr uint32_t mask = (1u << BITS) - 1u;
  const int bit = u * BITS;
  const int word = bit >> 5;
  const int shift = bit & 31;
  if (shift + BITS <= 32) return (w[word] >> shift) & mask;
  return __builtin_amdgcn_alignbit(w[word + 1], w[word], shift) & mask;
}

// The 8 weights of codes 8s..8s+7: palette entries gathered from LDS.
template <int BITS>
__device__ __forceinline__ half8 decode_fragment(const uint32_t (&w)[BITS], int s, const _Float16* lut) {
  half8 f;
#pragma unroll
  for (int t = 0; t < 8; ++t) f[t] = lut[lane_code<BITS>(w, s * 8 + t)];
  return f;
}

// 16-byte chunk c of row (or column) r of a 64-deep K block in LDS: chunks
// are XOR-swizzled with (r >> 1) & 7, which keeps the 16 lanes of every
// ds_read_b128 / ds_write_b128 phase on distinct bank groups (64 banks of
// 4 bytes) when lanes walk consecutive rows.
__device__ __forceinline__ int swizzled(int r, int c) { return r * kRowBytes + ((c ^ ((r >> 1) & 7)) << 4); }

// SiLU of the reference epilogue, v / (1 + exp(-clamp(v, -20, 20)))
// (src/webgpu/kernels/gemm.ts:2006-2044), on the hardware transcendental
// units: v_med3_f32 clamp, v_exp_f32 of the base-2 argument and v_rcp_f32
// (each within about 1 ulp of f32), six VALU operations instead of a full
// libm expf and a division; the relative error (~1e-6) is far below the f16
// rounding of the result.
__device__ __forceinline__ float silu(float v) {
  const float bounded = __builtin_amdgcn_fmed3f(v, -20.0f, 20.0f);
  const float e = __builtin_amdgcn_exp2f(bounded * -1.4426950408889634f);
  return v * __builtin_amdgcn_rcpf(1.0f + e);
}

// sigmoid(v) = 1 / (1 + exp(-clamp(v, -20, 20))), the GLU gate of the
// reference (src/webgpu/kernels/conformer-conv.ts:489-492).
__device__ __forceinline__ float sigmoid(float v) {
  const float bounded = __builtin_amdgcn_fmed3f(v, -20.0f, 20.0f);
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(bounded * -1.4426950408889634f));
}

// v rounded to f16 and back: the value a reference f16 buffer would hold.
__device__ __forceinline__ float through_f16(float v) { return (float)(_Float16)v; }

__device__ __forceinline__ uint32_t pack_half2(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
         ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}

// Split-K: publish this workgroup's partial tile; returns false when another
// workgroup of the tile finishes it. The last one to arrive (by the tile's
// arrival counter) sums all partials in split order into `acc` - the result
// does not depend on arrival order - and resets the counter for the next
// launch.
template <int R, int C, int T>
__device__ bool split_k_reduce(const GemmArgs& args, floatx16 (&acc)[R][C], uint32_t tile, uint32_t split,
                               int tid, uint32_t* last_flag) {
  const uint32_t S = args.splits;
  constexpr int EPT = R * C * 16;  // f32 accumulator values per thread
  float* mine = args.partials + ((uint64_t)tile * S + split) * (uint64_t)(EPT * T);
#pragma unroll
  for (int mi = 0; mi < R; ++mi)
#pragma unroll
    for (int ci = 0; ci < C; ++ci)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e4 = (mi * C + ci) * 4 + q;
        *reinterpret_cast<float4*>(mine + ((uint64_t)e4 * T + tid) * 4) =
            make_float4(acc[mi][ci][4 * q], acc[mi][ci][4 * q + 1], acc[mi][ci][4 * q + 2], acc[mi][ci][4 * q + 3]);
      }
  __threadfence();
  __syncthreads();
  if (tid == 0) *last_flag = atomicAdd(args.counters + tile, 1u) == S - 1u;
  __syncthreads();
  if (!*last_flag) return false;
  __threadfence();
  if (tid == 0) args.counters[tile] = 0u;
  const float* base = args.partials + (uint64_t)tile * S * (uint64_t)(EPT * T);
#pragma unroll
  for (int mi = 0; mi < R; ++mi)
#pragma unroll
    for (int ci = 0; ci < C; ++ci)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int e4 = (mi * C + ci) * 4 + q;
        float4 sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (uint32_t p = 0; p < S; ++p) {
          float4 v;
          if (p == split)
            v = make_float4(acc[mi][ci][4 * q], acc[mi][ci][4 * q + 1], acc[mi][ci][4 * q + 2], acc[mi][ci][4 * q + 3]);
          else
            v = *reinterpret_cast<const float4*>(base + (uint64_t)p * (EPT * T) + ((uint64_t)e4 * T + tid) * 4);
          sum.x += v.x;
          sum.y += v.y;
          sum.z += v.z;
          sum.w += v.w;
        }
        acc[mi][ci][4 * q] = sum.x;
        acc[mi][ci][4 * q + 1] = sum.y;
        acc[mi][ci][4 * q + 2] = sum.z;
        acc[mi][ci][4 * q + 3] = sum.w;
      }
  return true;
}

// Epilogue of a BM x BN tile held by WM x WN wavefronts of R x C MFMA
// blocks. In registers a lane holds row m = m0 + (wave_m*R + mi)*32 + j and,
// for q = 0..3, the 4 columns n = n0 + (wave_n*C + ci)*32 + 8q + 4h + {0..3}.
// The tile goes out through an LDS staging area of `stage_bytes` so global
// traffic is 16-byte chunks along rows: a pass stages MPP m-blocks of every
// wavefront as row-major f16 rows of BN columns, 8-byte units XOR-swizzled
// by row. With a residual, its tile is first loaded the same way so that
// residual + scale * value is formed in f32 and rounded once. The order
// bias -> SiLU/ReLU -> residual follows src/webgpu/kernels/gemm.ts:2006-2044.
template <int WM, int WN, int R, int C, int STAGE_BYTES>
__device__ void store_tile(const GemmArgs& args, const floatx16 (&acc)[R][C], uint8_t* stage, uint32_t m0,
                           uint32_t n0, int wave_m, int wave_n, int j, int h, int tid) {
  constexpr int T = 64 * WM * WN;
  constexpr int BN = 32 * C * WN;
  constexpr int ROWB = BN * 2;  // bytes per staged row
  constexpr int MPP_FIT = STAGE_BYTES / (WM * 32 * ROWB);
  constexpr int MPP = MPP_FIT >= R ? R : (MPP_FIT >= 1 ? MPP_FIT : 1);
  constexpr int SR = WM * MPP * 32;  // staged rows per pass
  constexpr int CPR = BN / 8;        // 16-byte chunks per staged row
  static_assert(SR * ROWB <= STAGE_BYTES, "epilogue staging exceeds its LDS area");
  static_assert(R % MPP == 0, "epilogue passes must cover whole m-blocks");
  static_assert(BN >= 128, "the staging swizzle needs rows of at least 32 8-byte units");
  const uint32_t M = args.rows, N = args.columns;
  auto stage_at = [&](int sr, int unit) { return sr * ROWB + ((unit ^ ((sr & 15) << 1)) << 3); };
  auto chunk_row = [&](int sr, int mi0) {
    return m0 + (uint32_t)(((sr / 32) / MPP * R + mi0 + (sr / 32) % MPP) * 32 + (sr & 31));
  };
  const _Float16* residual = static_cast<const _Float16*>(args.residual);
  _Float16* out = static_cast<_Float16*>(args.out);
  __syncthreads();
#pragma unroll
  for (int mi0 = 0; mi0 < R; mi0 += MPP) {
    if (residual) {
      for (int chunk = tid; chunk < SR * CPR; chunk += T) {
        const int sr = chunk / CPR, c16 = chunk % CPR;
        const uint32_t m = chunk_row(sr, mi0);
        const uint32_t n = n0 + (uint32_t)c16 * 8u;
        if (m < M && n < N)
          *reinterpret_cast<uint4*>(stage + stage_at(sr, 2 * c16)) =
              *reinterpret_cast<const uint4*>(residual + (uint64_t)m * N + n);
      }
      __syncthreads();
    }
#pragma unroll
    for (int ml = 0; ml < MPP; ++ml) {
      const int mi = mi0 + ml;
      const int sr = (wave_m * MPP + ml) * 32 + j;
#pragma unroll
      for (int ci = 0; ci < C; ++ci) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int unit = (wave_n * C + ci) * 8 + 2 * q + h;
          const uint32_t n = n0 + (uint32_t)unit * 4u;
          float v0 = acc[mi][ci][4 * q], v1 = acc[mi][ci][4 * q + 1];
          float v2 = acc[mi][ci][4 * q + 2], v3 = acc[mi][ci][4 * q + 3];
          if (args.bias && n < N) {
            const float4 b = *reinterpret_cast<const float4*>(args.bias + n);
            v0 += b.x;
            v1 += b.y;
            v2 += b.z;
            v3 += b.w;
          }
          if (args.activation == kActSilu) {
            v0 = silu(v0);
            v1 = silu(v1);
            v2 = silu(v2);
            v3 = silu(v3);
          } else if (args.activation == kActRelu) {
            v0 = fmaxf(v0, 0.0f);
            v1 = fmaxf(v1, 0.0f);
            v2 = fmaxf(v2, 0.0f);
            v3 = fmaxf(v3, 0.0f);
          }
          uint2* slot = reinterpret_cast<uint2*>(stage + stage_at(sr, unit));
          if (residual) {
            const uint2 rb = *slot;
            const float sc = args.residual_scale;
            v0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.x & 0xffffu)) + sc * v0;
            v1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.x >> 16)) + sc * v1;
            v2 = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.y & 0xffffu)) + sc * v2;
            v3 = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.y >> 16)) + sc * v3;
          }
          *slot = make_uint2(pack_half2(v0, v1), pack_half2(v2, v3));
        }
      }
    }
    __syncthreads();
    for (int chunk = tid; chunk < SR * CPR; chunk += T) {
      const int sr = chunk / CPR, c16 = chunk % CPR;
      const uint32_t m = chunk_row(sr, mi0);
      const uint32_t n = n0 + (uint32_t)c16 * 8u;
      if (m < M && n < N)
        *reinterpret_cast<uint4*>(out + (uint64_t)m * N + n) =
            *reinterpret_cast<const uint4*>(stage + stage_at(sr, 2 * c16));
    }
    __syncthreads();
  }
}

// Registry entry of one compiled f16 tile shape: `single` kernels require
// K % 64 == 0 and one palette group per tile, `general` kernels take any
// shape the ABI accepts.
struct F16Variant {
  TileShape shape;
  const char* name5;
  const char* name6;
  void (*single[2])(GemmArgs);  // [bits == 6]
  void (*general[2])(GemmArgs);
  uint32_t lds_bytes;           // static LDS of the kernel
  void (*normed[2])(GemmArgs);  // fused row LayerNorm (single path), or null
  void (*streamed[2])(GemmArgs);  // single path with non-temporal output stores, or null
};

// The `single` kernels need K % 64 == 0 and every tile inside one palette
// group (its palette staged at a fixed LDS address); tiles start at
// multiples of the tile width, so the latter holds with one group or when
// the group width is a multiple of the tile width.
inline bool single_path(const TileShape& s, const GemmArgs& a) {
  return (a.inner & 63u) == 0u &&
         (a.palette_groups == 1 || a.palette_group_columns % (uint32_t)s.tile_columns() == 0);
}

// Whether a launch of `v` with `a` runs its non-temporal-store kernel.
inline bool streams(const F16Variant& v, int bits, const GemmArgs& a) {
  return a.stream_out && !a.norm_columns && v.streamed[bits == 6] && single_path(v.shape, a);
}

}  // namespace f16

// Pair-code K-split tile shapes (pk_gemm_f16k.hip).
int f16k_variant_count();
const f16::F16Variant& f16k_variant(int index);
hipError_t launch_gemm_f16k(int bits, const f16::F16Variant& v, const GemmArgs& args, hipStream_t stream,
                            hipEvent_t start, hipEvent_t stop);

// Small-M shapes (pk_gemm_f16s.hip).
int f16s_variant_count();
const f16::F16Variant& f16s_variant(int index);
hipError_t launch_gemm_f16s(int bits, const f16::F16Variant& v, const GemmArgs& args, hipStream_t stream,
                            hipEvent_t start, hipEvent_t stop);
const char* f16s_group_name(int index);
bool f16s_group_persistent(int index);
bool f16s_group_streams(int index, uint32_t inner, uint32_t palette_groups, uint32_t palette_group_columns);
uint32_t f16s_group_launch(int index, const SmallMGroupArgs& g, void (**kernel)(SmallMGroupArgs), const char** name);
hipError_t launch_gemm_f16s_group(int index, const SmallMGroupArgs& group, hipStream_t stream, hipEvent_t start,
                                  hipEvent_t stop);

}  // namespace pk

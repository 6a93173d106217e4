// pk_gemm_f16s.hip - fused palette-weight GEMM for small M (M <= 256, the
// weight-bandwidth-bound shapes): f16 operands, f32 MFMA accumulation,
// operand-order codes, K split over the eight wavefronts of a workgroup
// (gfx950, wave64).
//
// C[m, n] = epilogue(sum_k A[m, k] * LUT[g(n)][code(k, n)])
// (reference: src/webgpu/kernels/gemm.ts:1362-1716, epilogue :2006-2044).
//
// With few rows the work is the weight stream itself: ceil(K*N*bits/8)
// bytes, read once. A workgroup owns one 32-column block and RW 32-row
// blocks; its eight wavefronts take the K blocks round robin (wavefront w:
// blocks w, w+8, ...), so every weight byte is fetched by exactly one
// wavefront, as one coalesced 16-byte + one 4/8-byte load per lane of the
// operand-order stream (the package's own bits per code, no larger
// layout). Activation fragments come straight from global memory (the
// activations are a few hundred KB, L2-resident), so the K loop has no LDS
// tile and no barrier: a wavefront issues the loads of its next K block,
// decodes the current one (shift/mask/v_alignbit per code, palette gather
// from LDS) into MFMA operands and runs the MFMAs. The eight partial tiles
// are summed through LDS in wavefront order (deterministic), then bias,
// SiLU/ReLU and residual + scale * value in f32, rounded once, 8-byte row
// stores. v_mfma_f32_32x32x16_f16 computes W^T * A^T with lane half h,
// element t of sub-step s standing for k = 64*kb + 32*h + 8*s + t in both
// operands.
#include "pk_f16_common.h"

namespace pk {
namespace {

using namespace f16;

constexpr int kSkinnyWaves = 8;

// GENERAL: the 32 columns may span two palette groups (per-lane palette
// base) or K may be 32 (mod 64) (the upper half of the last K block is
// padding: its activation fragments are zeroed).
template <int BITS, int RW, bool GENERAL>
__global__ __launch_bounds__(64 * kSkinnyWaves) void gemm_f16s_kernel(GemmArgs args) {
  constexpr int W = kSkinnyWaves;
  constexpr int T = 64 * W;
  constexpr int E = 1 << BITS;
  constexpr uint32_t BW = block_words(BITS);
  // Partials: [wave][m-block][quad q][slot] float4, slot = lane ^ 2(2q + h),
  // which keeps both the per-lane writes and the row-wise reads on distinct
  // bank groups.
  __shared__ float4 red[W * RW * 4 * 64];
  __shared__ _Float16 lut_lds[2 * E];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31;
  const int h = lane >> 5;

  const uint32_t M = args.rows;
  const uint32_t K = args.inner;
  const uint32_t N = args.columns;
  const uint32_t KB = (K + 63u) / 64u;
  const uint32_t NBT = (N + 31u) / 32u;
  const uint32_t nb = blockIdx.x % NBT;
  const uint32_t mg = blockIdx.x / NBT;
  const uint32_t n0 = nb * 32u;
  const uint32_t m0 = mg * (uint32_t)(RW * 32);

  // Palettes of the block's columns (palette-expander.ts:543-549): a
  // 32-column block spans at most two groups (groups are >= 16 columns).
  const uint32_t gc = args.palette_group_columns;
  const uint32_t G = args.palette_groups;
  const uint32_t g_lo = min(n0 / gc, G - 1u);
  {
    const uint32_t g_hi = GENERAL ? min((min(n0 + 32u, N) - 1u) / gc, G - 1u) : g_lo;
    const uint32_t entries = (g_hi - g_lo + 1u) * E;
    const _Float16* src = static_cast<const _Float16*>(args.palette) + (uint64_t)g_lo * E;
    for (uint32_t i = tid; i < entries; i += T) lut_lds[i] = src[i];
  }
  const _Float16* lut = lut_lds;
  if constexpr (GENERAL) lut = lut_lds + (min(min(n0 + (uint32_t)j, N - 1u) / gc, G - 1u) - g_lo) * E;

  // This wavefront's K blocks: wave, wave + W, ...
  const uint32_t nblocks = (uint32_t)wave < KB ? (KB - (uint32_t)wave + W - 1u) / W : 0u;
  const uint32_t* code_base = args.codes + (uint64_t)nb * KB * BW;
  auto load_codes = [&](uint32_t kb, uint32_t (&dst)[BITS]) {
    const uint32_t* blk = code_base + (uint64_t)kb * BW;
    const uint4 p0 = reinterpret_cast<const uint4*>(blk)[lane];
    dst[0] = p0.x;
    dst[1] = p0.y;
    dst[2] = p0.z;
    dst[3] = p0.w;
    if constexpr (BITS == 5) {
      dst[4] = blk[256 + lane];
    } else {
      const uint2 p1 = reinterpret_cast<const uint2*>(blk + 256)[lane];
      dst[4] = p1.x;
      dst[5] = p1.y;
    }
  };
  // Activation fragment (m-block mi, sub-step s): row m0 + 32mi + j (rows
  // past M re-read row M-1, never stored), k = 64kb + 32h + 8s. In a
  // K = 32 (mod 64) tail block the upper lane half re-reads k - 32 and is
  // zeroed.
  const _Float16* a_row[RW];
#pragma unroll
  for (int mi = 0; mi < RW; ++mi)
    a_row[mi] = static_cast<const _Float16*>(args.a) + (uint64_t)min(m0 + (uint32_t)(mi * 32 + j), M - 1u) * K;
  auto load_a = [&](uint32_t kb, half8 (&dst)[RW][4]) {
    const bool pad = GENERAL && (K & 63u) != 0u && kb + 1u == KB && h;
    const uint32_t k0 = kb * 64u + (uint32_t)(32 * h) - (pad ? 32u : 0u);
#pragma unroll
    for (int mi = 0; mi < RW; ++mi)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        half8 v = *reinterpret_cast<const half8*>(a_row[mi] + k0 + 8u * s);
        if (pad) v = half8{};
        dst[mi][s] = v;
      }
  };

  floatx16 acc[RW];
#pragma unroll
  for (int mi = 0; mi < RW; ++mi)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[mi][v] = 0.0f;

  auto multiply = [&](const uint32_t (&cw)[BITS], const half8 (&af)[RW][4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const half8 wf = decode_fragment<BITS>(cw, s, lut);
#pragma unroll
      for (int mi = 0; mi < RW; ++mi) acc[mi] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf, af[mi][s], acc[mi], 0, 0, 0);
    }
  };

  __syncthreads();  // palettes staged
  if (nblocks > 0) {
    // Two register sets, the next K block's loads issued before the current
    // block is decoded; loads past this wavefront's last block re-read it.
    const uint32_t last = (uint32_t)wave + (nblocks - 1u) * W;
    uint32_t c0[BITS], c1[BITS];
    half8 a0[RW][4], a1[RW][4];
    load_codes((uint32_t)wave, c0);
    load_a((uint32_t)wave, a0);
    uint32_t t = 0;
    for (; t + 2u <= nblocks; t += 2u) {
      const uint32_t kb = (uint32_t)wave + t * W;
      load_codes(min(kb + W, last), c1);
      load_a(min(kb + W, last), a1);
      multiply(c0, a0);
      load_codes(min(kb + 2u * W, last), c0);
      load_a(min(kb + 2u * W, last), a0);
      multiply(c1, a1);
    }
    if (t < nblocks) multiply(c0, a0);
  }

#pragma unroll
  for (int ml = 0; ml < RW; ++ml)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      red[((wave * RW + ml) * 4 + q) * 64 + (lane ^ (2 * (2 * q + h)))] =
          make_float4(acc[ml][4 * q], acc[ml][4 * q + 1], acc[ml][4 * q + 2], acc[ml][4 * q + 3]);
  __syncthreads();

  // Unit u: row r = u / 8 of the block, 4 columns 4 * (u % 8); the lane of
  // the MFMA layout holding them is 32 * (cg & 1) + (r & 31), quad cg / 2.
  const _Float16* residual = static_cast<const _Float16*>(args.residual);
  _Float16* out = static_cast<_Float16*>(args.out);
  for (int u = tid; u < RW * 32 * 8; u += T) {
    const int r = u >> 3, cg = u & 7;
    const int ml = r >> 5, q = cg >> 1, hh = cg & 1;
    const uint32_t m = m0 + (uint32_t)r;
    const uint32_t n = n0 + (uint32_t)(4 * cg);
    if (m >= M || n >= N) continue;
    const int slot = (32 * hh + (r & 31)) ^ (2 * (2 * q + hh));
    float4 sum = red[(ml * 4 + q) * 64 + slot];
#pragma unroll
    for (int w = 1; w < W; ++w) {
      const float4 x = red[((w * RW + ml) * 4 + q) * 64 + slot];
      sum.x += x.x;
      sum.y += x.y;
      sum.z += x.z;
      sum.w += x.w;
    }
    float v[4] = {sum.x, sum.y, sum.z, sum.w};
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
      const uint2 rb = *reinterpret_cast<const uint2*>(residual + at);
      const float sc = args.residual_scale;
      v[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.x & 0xffffu)) + sc * v[0];
      v[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.x >> 16)) + sc * v[1];
      v[2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.y & 0xffffu)) + sc * v[2];
      v[3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.y >> 16)) + sc * v[3];
    }
    *reinterpret_cast<uint2*>(out + at) = make_uint2(pack_half2(v[0], v[1]), pack_half2(v[2], v[3]));
  }
}

#define PK_F16S_VARIANT(RW)                                                                               \
  F16Variant {                                                                                            \
    TileShape{1, 1, RW, 1, kSkinnyWaves}, "pk_gemm_f16s_b5_k8_m" #RW, "pk_gemm_f16s_b6_k8_m" #RW,         \
        {gemm_f16s_kernel<5, RW, false>, gemm_f16s_kernel<6, RW, false>},                                 \
        {gemm_f16s_kernel<5, RW, true>, gemm_f16s_kernel<6, RW, true>},                                   \
        (uint32_t)(kSkinnyWaves * RW * 4 * 64 * 16 + 2 * 64 * 2)                                          \
  }

const F16Variant kVariants[] = {
    PK_F16S_VARIANT(1),  // 32 rows x 32 columns per workgroup
    PK_F16S_VARIANT(2),  // 64 x 32
    PK_F16S_VARIANT(4),  // 128 x 32
};

}  // namespace

int f16s_variant_count() { return (int)(sizeof(kVariants) / sizeof(kVariants[0])); }
const f16::F16Variant& f16s_variant(int index) { return kVariants[index]; }

// One workgroup per (32-column block, RW 32-row blocks). The `single`
// kernel needs K % 64 == 0 and the block inside one palette group.
hipError_t launch_gemm_f16s(int bits, const f16::F16Variant& v, const GemmArgs& args, hipStream_t stream,
                            hipEvent_t start, hipEvent_t stop) {
  const uint32_t groups = tiles_m(v.shape, args.rows) * tiles_n(v.shape, args.columns);
  if (groups == 0) return hipSuccess;
  const bool single =
      (args.inner & 63u) == 0u && (args.palette_groups == 1 || args.palette_group_columns % 32u == 0);
  return launch_timed(single ? v.single[bits == 6] : v.general[bits == 6], dim3(groups), dim3(v.shape.threads()),
                      stream, start, stop, args);
}

}  // namespace pk

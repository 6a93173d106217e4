// pk_gemm_f16.hip - fused palette-weight GEMM, f16 operands, f32 MFMA
// accumulation, for gfx950 (CDNA4, wave64).
//
// C[m, n] = epilogue(sum_k A[m, k] * LUT[g(n)][code(k, n)])
//
// The dense weight is never materialised. A workgroup of WM x WN wavefronts
// owns a BM x BN output tile (BM = 32*R*WM, BN = 32*C*WN); each wavefront owns
// R x C MFMA blocks of 32 x 32 and walks K in 64-deep blocks:
//   * codes: per 32-column block one coalesced 16-byte + one 4/8-byte load
//     per lane of the operand-order stream (pk_internal.h), two K blocks
//     ahead;
//   * activations: the BM x 64 f16 tile of K block i+3 is loaded into
//     registers while block i is multiplied, and written to a double
//     buffered LDS tile at the end of block i+2. Its 16-byte chunks are
//     XOR-swizzled with (row >> 1) & 7, which keeps the 16 lanes of each
//     ds_read_b128 phase on distinct LDS banks (64 banks of 4 bytes);
//   * decode: each lane cuts the 8 codes of a 16-deep sub-step out of its
//     code words (shift/mask, v_alignbit_b32 across words) and gathers them
//     from the palette staged in LDS straight into the 8 halves of the MFMA
//     operand. When a tile lies inside one palette group the palette sits at
//     a fixed LDS address, so the gather address is the code alone. The
//     fragment of sub-step s+1 is gathered while the MFMAs of s run;
//   * v_mfma_f32_32x32x16_f16 computes D = W^T * A^T (weights as the 32 x 16
//     "A" operand, activations as "B"), so a lane ends with 4 runs of 4
//     consecutive output columns of one row; the epilogue regroups the tile
//     through LDS into 16-byte row chunks for the global stores.
// K-slot pairing: in sub-step s, lane half h, operand element t stands for
// k = 64*kb + 32*h + 8*s + t in BOTH operands, so the hardware's own pairing
// of A and B slots always multiplies matching k. The main loop is unrolled
// by three so the rotating register sets are fixed registers: no copy ever
// waits on a load that is still in flight.
//
// Epilogue (src/webgpu/kernels/gemm.ts:2006-2044): f32 value, + bias[n],
// SiLU v/(1+exp(-clamp(v,-20,20))) or ReLU, then residual + scale * value,
// rounded to f16.
#include "pk_f16_common.h"

namespace pk {
namespace {

using namespace f16;

// GENERAL: the tile's columns may span several palette groups (per-lane
// palette base) and K may be 32 (mod 64). Otherwise (the common case) the
// tile's one palette sits at a fixed LDS address and K is a multiple of 64.
template <int BITS, int WM, int WN, int R, int C, bool GENERAL>
__global__ __launch_bounds__(64 * WM * WN) void gemm_f16_kernel(GemmArgs args) {
  constexpr int T = 64 * WM * WN;
  constexpr int BM = 32 * R * WM;
  constexpr int BN = 32 * C * WN;
  constexpr int E = 1 << BITS;
  constexpr int CPG = (int)codes_per_group(BITS);
  constexpr int LUT_CAP = GENERAL ? (BN / CPG + 2) * E : E;
  constexpr int ROW_BYTES = 128;  // 64 halves of one row per K block
  constexpr int CH = BM * 8 / T;  // 16-byte activation chunks per thread per K block
  constexpr uint32_t BW = block_words(BITS);
  static_assert(BM * 8 % T == 0, "activation tile chunks must divide evenly");

  __shared__ __attribute__((aligned(16))) uint8_t a_lds[2 * BM * ROW_BYTES];
  __shared__ _Float16 lut_lds[LUT_CAP];
  __shared__ uint32_t last_flag;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wave_m = wave / WN;
  const int wave_n = wave % WN;
  const int j = lane & 31;
  const int h = lane >> 5;

  const uint32_t M = args.rows;
  const uint32_t K = args.inner;
  const uint32_t N = args.columns;
  const uint32_t KB = (K + 63u) / 64u;
  const uint32_t NBT = (N + 31u) / 32u;
  const uint32_t S = args.splits;
  const uint32_t TN = (NBT * 32u + BN - 1u) / BN;

  // Work item: split fastest, then column tile, then row tile, laid out so
  // that the workgroups of one XCD take consecutive items.
  uint32_t item = xcd_local_order(blockIdx.x, gridDim.x);
  const uint32_t split = item % S;
  item /= S;
  const uint32_t tile = item;
  const uint32_t tn = item % TN;
  const uint32_t tm = item / TN;
  const uint32_t m0 = tm * BM;
  const uint32_t n0 = tn * BN;
  const uint32_t kb_begin = split * KB / S;
  const uint32_t kb_end = (split + 1u) * KB / S;
  const uint32_t steps = kb_end - kb_begin;
  // K = 32 (mod 64): the last K block is half padding.
  const bool tail_block = (K & 63u) != 0u && kb_end == KB;

  // Palette window of this tile's columns (palette-expander.ts:543-549).
  // GENERAL kernels also keep E zero entries after the staged palettes:
  // lanes gathering padded k of a K = 32 (mod 64) tail read weights from
  // there.
  const uint32_t gc = args.palette_group_columns;
  const uint32_t G = args.palette_groups;
  const uint32_t g_lo = min(n0 / gc, G - 1u);
  {
    const uint32_t g_hi = GENERAL ? min((min(n0 + BN, N) - 1u) / gc, G - 1u) : g_lo;
    const uint32_t entries = (g_hi - g_lo + 1u) * E;
    const _Float16* src = static_cast<const _Float16*>(args.palette) + (uint64_t)g_lo * E;
    for (uint32_t i = tid; i < entries; i += T) lut_lds[i] = src[i];
    if constexpr (GENERAL)
      for (uint32_t i = tid; i < (uint32_t)E; i += T) lut_lds[LUT_CAP - E + i] = (_Float16)0.0f;
  }
  const _Float16* lut_col[C];
#pragma unroll
  for (int ci = 0; ci < C; ++ci) {
    if constexpr (GENERAL) {
      const uint32_t n = min(n0 + (wave_n * C + ci) * 32 + j, N - 1u);
      lut_col[ci] = lut_lds + (min(n / gc, G - 1u) - g_lo) * E;
    } else {
      lut_col[ci] = lut_lds;
    }
  }
  const _Float16* const lut_zero = lut_lds + (LUT_CAP - E);

  // Code streams of this wavefront's column blocks: a wave-uniform block
  // base plus this lane's fixed offset. Blocks past the last column block
  // re-read the last one (their columns are never stored), so every load is
  // unconditional.
  const uint32_t nb0 = n0 / 32u + wave_n * C;
  const uint32_t* code_base[C];
#pragma unroll
  for (int ci = 0; ci < C; ++ci)
    code_base[ci] = args.codes + (uint64_t)min(nb0 + ci, NBT - 1u) * KB * BW;
  auto load_codes = [&](uint32_t kb, uint32_t (&dst)[C][BITS]) {
#pragma unroll
    for (int ci = 0; ci < C; ++ci) {
      const uint32_t* blk = code_base[ci] + kb * BW;
      const uint4 p0 = reinterpret_cast<const uint4*>(blk)[lane];
      dst[ci][0] = p0.x;
      dst[ci][1] = p0.y;
      dst[ci][2] = p0.z;
      dst[ci][3] = p0.w;
      if constexpr (BITS == 5) {
        dst[ci][4] = blk[256 + lane];
      } else {
        const uint2 p1 = reinterpret_cast<const uint2*>(blk + 256)[lane];
        dst[ci][4] = p1.x;
        dst[ci][5] = p1.y;
      }
    }
  };

  // Activation tile: chunk c of this thread is row r = (tid + c*T) / 8,
  // 16-byte column chunk ch = (tid + c*T) % 8, at a fixed byte offset from
  // the wave-uniform address of (m0, 64*kb). Rows past M re-read row M-1
  // (their results are never stored). In a K = 32 (mod 64) tail, chunks
  // past K re-read the row's chunk ch - 4 and are stored as zeros.
  const char* a_tile = reinterpret_cast<const char*>(static_cast<const _Float16*>(args.a) + (uint64_t)m0 * K);
  uint32_t a_off[CH], a_st[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int idx = tid + c * T;
    const int r = idx >> 3, ch = idx & 7;
    a_off[c] = ((min(m0 + (uint32_t)r, M - 1u) - m0) * K + (uint32_t)ch * 8u) * 2u;
    a_st[c] = (uint32_t)(r * ROW_BYTES + ((ch ^ ((r >> 1) & 7)) << 4));
  }
  auto load_a = [&](uint32_t kb, uint4 (&dst)[CH]) {
    const char* base = a_tile + (uint64_t)kb * 128u;
    const bool partial = GENERAL && (K & 63u) != 0u && kb + 1u == KB;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const bool pad = partial && ((tid + c * T) & 7) >= 4;
      dst[c] = *reinterpret_cast<const uint4*>(base + (pad ? a_off[c] - 64u : a_off[c]));
    }
  };
  auto store_a = [&](uint32_t kb, uint32_t buf, const uint4 (&src)[CH]) {
    const bool partial = GENERAL && (K & 63u) != 0u && kb + 1u == KB;
    uint8_t* dst = a_lds + buf * (BM * ROW_BYTES);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      uint4 v = src[c];
      if (partial && ((tid + c * T) & 7) >= 4) v = make_uint4(0u, 0u, 0u, 0u);
      *reinterpret_cast<uint4*>(dst + a_st[c]) = v;
    }
  };
  // LDS byte offset of this lane's activation fragment for sub-step s of
  // m-block 0: row wave_m*R*32 + j, chunk 4h + s (swizzled; the swizzle of
  // rows 32*mi + j equals that of row j).
  uint32_t a_frag_off[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    a_frag_off[s] = (uint32_t)((wave_m * R * 32 + j) * ROW_BYTES + (((4 * h + s) ^ ((j >> 1) & 7)) << 4));

  floatx16 acc[R][C];
#pragma unroll
  for (int mi = 0; mi < R; ++mi)
#pragma unroll
    for (int ci = 0; ci < C; ++ci)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ci][v] = 0.0f;

  // One K block per step. Codes run two blocks ahead and activations three,
  // in three register sets each that rotate with the step index, so the
  // loop is unrolled by three and every set is a fixed register range.
  // Loads past the split's last block re-read that block: every step issues
  // the same loads, which keeps the in-order load counter waits exact.
  //   cur: codes of block i, nx1: block i+1 (loaded a step ago), nx2:
  //   receives block i+2; a_load receives block i+3's activations, a_store
  //   holds block i+1's and is written to LDS at the end of the step.
  // Weight fragments alternate between frag[0] and frag[1]: sub-step s
  // multiplies frag[s & 1] while gathering sub-step s+1 into the other, and
  // a step ends with the next block's first fragment in frag[0].
  const uint32_t last_kb = kb_end - 1u;
  half8 frag[2][C];
  auto step = [&](uint32_t i, const uint32_t (&cur)[C][BITS], const uint32_t (&nx1)[C][BITS],
                  uint32_t (&nx2)[C][BITS], uint4 (&a_load)[CH], const uint4 (&a_store)[CH]) {
    load_codes(min(kb_begin + i + 2u, last_kb), nx2);
    __builtin_amdgcn_sched_barrier(0);
    load_a(min(kb_begin + i + 3u, last_kb), a_load);
    __builtin_amdgcn_sched_barrier(0);
    // Palettes for the gathers of this block and of the next block's first
    // sub-step: the zero palette for lane half 1 (k >= 32) of a tail block.
    const _Float16* lut_this[C];
    const _Float16* lut_next[C];
#pragma unroll
    for (int ci = 0; ci < C; ++ci) {
      lut_this[ci] = lut_col[ci];
      lut_next[ci] = lut_col[ci];
      if constexpr (GENERAL) {
        if (tail_block && h) {
          if (i + 1u == steps) lut_this[ci] = lut_zero;
          if (i + 2u == steps) lut_next[ci] = lut_zero;
        }
      }
    }
    const uint8_t* tile_a = a_lds + (i & 1u) * (BM * ROW_BYTES);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      half8 af[R];
#pragma unroll
      for (int mi = 0; mi < R; ++mi)
        af[mi] = *reinterpret_cast<const half8*>(tile_a + a_frag_off[s] + mi * 32 * ROW_BYTES);
#pragma unroll
      for (int ci = 0; ci < C; ++ci)
        frag[(s + 1) & 1][ci] = s < 3 ? decode_fragment<BITS>(cur[ci], s + 1, lut_this[ci])
                                      : decode_fragment<BITS>(nx1[ci], 0, lut_next[ci]);
#pragma unroll
      for (int ci = 0; ci < C; ++ci)
#pragma unroll
        for (int mi = 0; mi < R; ++mi)
          acc[mi][ci] = __builtin_amdgcn_mfma_f32_32x32x16_f16(frag[s & 1][ci], af[mi], acc[mi][ci], 0, 0, 0);
    }
    store_a(min(kb_begin + i + 1u, last_kb), (i + 1u) & 1u, a_store);
    __syncthreads();
  };

  if (steps > 0) {
    uint32_t c0[C][BITS], c1[C][BITS], c2[C][BITS];
    uint4 s0[CH], s1[CH], s2[CH];
    load_codes(kb_begin, c0);
    load_codes(min(kb_begin + 1u, last_kb), c1);
    load_a(kb_begin, s0);
    load_a(min(kb_begin + 1u, last_kb), s1);
    load_a(min(kb_begin + 2u, last_kb), s2);
    store_a(kb_begin, 0u, s0);
    __syncthreads();
#pragma unroll
    for (int ci = 0; ci < C; ++ci)
      frag[0][ci] = decode_fragment<BITS>(c0[ci], 0, (GENERAL && tail_block && h && steps == 1u) ? lut_zero
                                                                                                  : lut_col[ci]);

    uint32_t i = 0;
    for (; i + 3u <= steps; i += 3u) {
      step(i, c0, c1, c2, s0, s1);
      step(i + 1u, c1, c2, c0, s1, s2);
      step(i + 2u, c2, c0, c1, s2, s0);
    }
    if (i < steps) step(i, c0, c1, c2, s0, s1);
    if (i + 1u < steps) step(i + 1u, c1, c2, c0, s1, s2);
  }

  // Split-K: only the last workgroup of the tile continues, with the sum of
  // all partials in split order.
  if (S > 1 && !split_k_reduce<R, C, T>(args, acc, tile, split, tid, &last_flag)) return;

  store_tile<WM, WN, R, C, 2 * BM * ROW_BYTES>(args, acc, a_lds, m0, n0, wave_m, wave_n, j, h, tid);
}

template <int WM, int WN, int R, int C>
constexpr uint32_t kernel_lds_bytes(int bits) {
  const int e = 1 << bits;
  const int lut = (32 * C * WN / (int)codes_per_group(bits) + 2) * e;
  return (uint32_t)(2 * 32 * R * WM * 128 + lut * 2 + 4);
}

#define PK_F16_VARIANT(WM, WN, R, C)                                                              \
  F16Variant {                                                                                    \
    TileShape{WM, WN, R, C}, "pk_gemm_f16_b5_w" #WM "x" #WN "_m" #R "n" #C,                       \
        "pk_gemm_f16_b6_w" #WM "x" #WN "_m" #R "n" #C,                                            \
        {gemm_f16_kernel<5, WM, WN, R, C, false>, gemm_f16_kernel<6, WM, WN, R, C, false>},       \
        {gemm_f16_kernel<5, WM, WN, R, C, true>, gemm_f16_kernel<6, WM, WN, R, C, true>},         \
        kernel_lds_bytes<WM, WN, R, C>(6)                                                         \
  }

const F16Variant kVariants[] = {
    PK_F16_VARIANT(1, 4, 1, 1),  // 32 x 128
    PK_F16_VARIANT(1, 4, 2, 1),  // 64 x 128
    PK_F16_VARIANT(1, 4, 4, 1),  // 128 x 128
    PK_F16_VARIANT(1, 4, 6, 1),  // 192 x 128
    PK_F16_VARIANT(1, 4, 2, 2),  // 64 x 256
    PK_F16_VARIANT(1, 4, 3, 2),  // 96 x 256
};

constexpr int kLocal = (int)(sizeof(kVariants) / sizeof(kVariants[0]));

const F16Variant& variant_at(int index) {
  if (index < kLocal) return kVariants[index];
  index -= kLocal;
  if (index < f16k_variant_count()) return f16k_variant(index);
  return f16s_variant(index - f16k_variant_count());
}

}  // namespace

// f16 tile shapes: the operand-order kernels of this file, then the
// pair-code K-split kernels of pk_gemm_f16k.hip, then the small-M kernels
// of pk_gemm_f16s.hip.
int f16_variant_count() { return kLocal + f16k_variant_count() + f16s_variant_count(); }
TileShape f16_variant(int index) { return variant_at(index).shape; }
const char* f16_variant_name(int bits, int index) {
  return bits == 5 ? variant_at(index).name5 : variant_at(index).name6;
}
uint32_t f16_variant_lds_bytes(int index) { return variant_at(index).lds_bytes; }
int f16_variant_family(int index) {
  if (index < kLocal) return kFamilyOperandOrder;
  return index < kLocal + f16k_variant_count() ? kFamilyPairCode : kFamilySmallM;
}

uint32_t f16_variant_grid(int index, uint32_t rows, uint32_t columns, uint32_t splits) {
  const TileShape s = f16_variant(index);
  if (f16_variant_family(index) == kFamilySmallM) return small_m_grid(s, tiles_n(s, columns), rows);
  return tiles_m(s, rows) * tiles_n(s, columns) * splits;
}

const char* f16_group_kernel_name(int index) {
  return f16_variant_family(index) == kFamilySmallM ? f16s_group_name(index - kLocal - f16k_variant_count())
                                                     : nullptr;
}

bool f16_group_persistent(int index) {
  return f16_variant_family(index) == kFamilySmallM && f16s_group_persistent(index - kLocal - f16k_variant_count());
}

bool f16_group_streams(int index, uint32_t inner, uint32_t palette_groups, uint32_t palette_group_columns) {
  return f16_variant_family(index) == kFamilySmallM &&
         f16s_group_streams(index - kLocal - f16k_variant_count(), inner, palette_groups, palette_group_columns);
}

uint32_t f16_group_launch_plan(int index, const SmallMGroupArgs& group, const char** kernel) {
  void (*fn)(SmallMGroupArgs) = nullptr;
  *kernel = nullptr;
  if (f16_variant_family(index) != kFamilySmallM) return 0;
  return f16s_group_launch(index - kLocal - f16k_variant_count(), group, &fn, kernel);
}

hipError_t launch_gemm_f16_group(int index, const SmallMGroupArgs& group, hipStream_t stream, hipEvent_t start,
                                 hipEvent_t stop) {
  if (f16_variant_family(index) != kFamilySmallM) return hipErrorInvalidValue;
  return launch_gemm_f16s_group(index - kLocal - f16k_variant_count(), group, stream, start, stop);
}

bool f16_variant_streams(int bits, int variant, const GemmArgs& args) {
  return variant >= kLocal && variant < kLocal + f16k_variant_count() &&
         f16::streams(variant_at(variant), bits, args);
}

hipError_t launch_gemm_f16(int bits, int variant, const GemmArgs& args, hipStream_t stream, hipEvent_t start,
                           hipEvent_t stop) {
  if (variant >= kLocal + f16k_variant_count())
    return launch_gemm_f16s(bits, variant_at(variant), args, stream, start, stop);
  if (variant >= kLocal) return launch_gemm_f16k(bits, variant_at(variant), args, stream, start, stop);
  const F16Variant& v = variant_at(variant);
  const uint32_t groups = tiles_m(v.shape, args.rows) * tiles_n(v.shape, args.columns) * args.splits;
  if (groups == 0) return hipSuccess;
  void (*kernel)(GemmArgs) = f16::single_path(v.shape, args) ? v.single[bits == 6] : v.general[bits == 6];
  return launch_timed(kernel, dim3(groups), dim3(v.shape.threads()), stream, start, stop, args);
}

}  // namespace pk

// pk_gemm_f16_shared.hip - fused palette-weight GEMM for tall tiles on
// gfx950: the workgroup decodes each weight code once into an f16 weight
// tile in LDS, and every wavefront reads MFMA operand fragments from LDS.
//
// C[m, n] = epilogue(sum_k A[m, k] * LUT[g(n)][code(k, n)])
//
// The VALU cost of decoding (a shift, a mask and an LDS palette gather per
// code, 8 codes per 32 x 32 x 16 MFMA fragment) is paid once per code per
// workgroup, i.e. once per BM rows of A. WM wavefronts stacked along M (each
// R x C MFMA blocks of 32 x 32) give BM = 32*R*WM rows per decoded weight, so
// tall tiles keep the decode well below the MFMA rate. Per 64-deep K block:
//   * each thread loads its operand-order code lane(s) (a 16-byte + a
//     4/8-byte coalesced load per lane, pk_internal.h) three K blocks ahead;
//   * while the MFMAs of block i run, the threads decode block i+1: a lane's
//     32 codes are one column's 32 consecutive k, written as four 16-byte
//     chunks into the column-major weight tile [BN columns][64 k]
//     (double-buffered, chunks swizzled like the activation tile);
//   * the BM x 64 activation tile is loaded three K blocks ahead through
//     registers into a double-buffered LDS tile;
//   * sub-step s reads R activation and C weight fragments (ds_read_b128,
//     conflict-free) and issues R x C v_mfma_f32_32x32x16_f16 computing
//     W^T * A^T; fragments of sub-step s+1 are read while s multiplies.
// In sub-step s, lane half h, operand element t stands for k = 64*kb + 32*h
// + 8*s + t in both operands. The loop is unrolled by three so the rotating
// register sets are fixed registers, and every prefetch is unconditional
// (clamped to the split's last block).
#include "pk_f16_common.h"

namespace pk {
namespace {

using namespace f16;

template <int BITS, int WM, int R, int C, bool GENERAL>
__global__ __launch_bounds__(64 * WM) void gemm_f16_shared_kernel(GemmArgs args) {
  constexpr int T = 64 * WM;
  constexpr int BM = 32 * R * WM;
  constexpr int BN = 32 * C;
  constexpr int E = 1 << BITS;
  constexpr int CPG = (int)codes_per_group(BITS);
  constexpr int LUT_CAP = GENERAL ? (BN / CPG + 2) * E : E;
  constexpr int CH = BM * 8 / T;   // 16-byte activation chunks per thread per K block
  constexpr int U = 2 * BN / T;    // code lanes decoded per thread per K block
  constexpr uint32_t BW = block_words(BITS);
  static_assert(BM * 8 % T == 0, "activation tile chunks must divide evenly");
  static_assert(2 * BN % T == 0 && U >= 1, "weight tile lanes must divide evenly");

  __shared__ __attribute__((aligned(16))) uint8_t a_lds[2 * BM * kRowBytes];
  __shared__ __attribute__((aligned(16))) uint8_t b_lds[2 * BN * kRowBytes];
  __shared__ _Float16 lut_lds[LUT_CAP];
  __shared__ uint32_t last_flag;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave_m = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31;
  const int h = lane >> 5;

  const uint32_t M = args.rows;
  const uint32_t K = args.inner;
  const uint32_t N = args.columns;
  const uint32_t KB = (K + 63u) / 64u;
  const uint32_t NBT = (N + 31u) / 32u;
  const uint32_t S = args.splits;
  const uint32_t TN = (NBT * 32u + BN - 1u) / BN;

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
  const uint32_t last_kb = kb_end - 1u;
  const bool tail_block = (K & 63u) != 0u && kb_end == KB;

  // Palettes of the tile's columns (palette-expander.ts:543-549); GENERAL
  // kernels keep E zeros after them for the padded k of a K = 32 (mod 64)
  // tail.
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
  const _Float16* const lut_zero = lut_lds + (LUT_CAP - E);

  // The code lanes this thread decodes: unit u is tile lane g = tid + u*T,
  // i.e. 32-column block g / 64 of the tile, lane g % 64 of that block
  // (column (g/64)*32 + g%32, k half (g % 64) / 32).
  const uint32_t* code_base[U];
  const _Float16* lut_unit[U];
  int b_col[U], b_half[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int g = tid + u * T;
    const int nb = g >> 6, gl = g & 63;
    code_base[u] = args.codes + (uint64_t)min(n0 / 32u + (uint32_t)nb, NBT - 1u) * KB * BW;
    b_col[u] = nb * 32 + (gl & 31);
    b_half[u] = gl >> 5;
    if constexpr (GENERAL) {
      const uint32_t n = min(n0 + (uint32_t)b_col[u], N - 1u);
      lut_unit[u] = lut_lds + (min(n / gc, G - 1u) - g_lo) * E;
    } else {
      lut_unit[u] = lut_lds;
    }
  }
  auto load_codes = [&](uint32_t kb, uint32_t (&dst)[U][BITS]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t* blk = code_base[u] + kb * BW;
      const int gl = (tid + u * T) & 63;
      const uint4 p0 = reinterpret_cast<const uint4*>(blk)[gl];
      dst[u][0] = p0.x;
      dst[u][1] = p0.y;
      dst[u][2] = p0.z;
      dst[u][3] = p0.w;
      if constexpr (BITS == 5) {
        dst[u][4] = blk[256 + gl];
      } else {
        const uint2 p1 = reinterpret_cast<const uint2*>(blk + 256)[gl];
        dst[u][4] = p1.x;
        dst[u][5] = p1.y;
      }
    }
  };
  // Chunk q (codes 8q..8q+7) of every unit of block `step`, into weight
  // tile buffer `buf`: column b_col, k chunk 4*b_half + q.
  auto decode_chunk = [&](const uint32_t (&w)[U][BITS], int q, uint32_t buf, uint32_t step) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const _Float16* lut = lut_unit[u];
      if constexpr (GENERAL) {
        if (tail_block && step + 1u == steps && b_half[u]) lut = lut_zero;
      }
      const half8 f = decode_fragment<BITS>(w[u], q, lut);
      *reinterpret_cast<half8*>(b_lds + buf * (BN * kRowBytes) + swizzled(b_col[u], 4 * b_half[u] + q)) = f;
    }
  };

  // Activation tile: chunk c of this thread is row r = (tid + c*T) / 8,
  // 16-byte chunk ch = (tid + c*T) % 8. Rows past M re-read row M-1; in a
  // K = 32 (mod 64) tail, chunks past K re-read chunk ch - 4 and are stored
  // as zeros.
  const char* a_tile = reinterpret_cast<const char*>(static_cast<const _Float16*>(args.a) + (uint64_t)m0 * K);
  uint32_t a_off[CH], a_st[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int idx = tid + c * T;
    const int r = idx >> 3, ch = idx & 7;
    a_off[c] = ((min(m0 + (uint32_t)r, M - 1u) - m0) * K + (uint32_t)ch * 8u) * 2u;
    a_st[c] = (uint32_t)swizzled(r, ch);
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
    uint8_t* dst = a_lds + buf * (BM * kRowBytes);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      uint4 v = src[c];
      if (partial && ((tid + c * T) & 7) >= 4) v = make_uint4(0u, 0u, 0u, 0u);
      *reinterpret_cast<uint4*>(dst + a_st[c]) = v;
    }
  };

  // This lane's fragment offsets for sub-step s: activation row
  // wave_m*R*32 + 32*mi + j, weight column 32*ci + j, chunk 4h + s (the
  // swizzle of row 32*i + j equals that of row j).
  uint32_t a_frag[4], b_frag[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    a_frag[s] = (uint32_t)swizzled(wave_m * R * 32 + j, 4 * h + s);
    b_frag[s] = (uint32_t)swizzled(j, 4 * h + s);
  }

  floatx16 acc[R][C];
#pragma unroll
  for (int mi = 0; mi < R; ++mi)
#pragma unroll
    for (int ci = 0; ci < C; ++ci)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ci][v] = 0.0f;

  // Step i multiplies block i from buffers i & 1 while decoding block i+1
  // (codes `dec`, loaded two steps ago) into the other weight buffer, loads
  // block i+3's codes into `ld_codes` and activations into `a_load`, and at
  // the end stores block i+1's activations (`a_store`, loaded two steps
  // ago) into the other activation buffer.
  auto step = [&](uint32_t i, const uint32_t (&dec)[U][BITS], uint32_t (&ld_codes)[U][BITS],
                  uint4 (&a_load)[CH], const uint4 (&a_store)[CH]) {
    load_codes(min(kb_begin + i + 3u, last_kb), ld_codes);
    __builtin_amdgcn_sched_barrier(0);
    load_a(min(kb_begin + i + 3u, last_kb), a_load);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t cur = i & 1u, nxt = cur ^ 1u;
    const uint8_t* ta = a_lds + cur * (BM * kRowBytes);
    const uint8_t* tb = b_lds + cur * (BN * kRowBytes);
    half8 af[2][R], bf[2][C];
#pragma unroll
    for (int mi = 0; mi < R; ++mi) af[0][mi] = *reinterpret_cast<const half8*>(ta + a_frag[0] + mi * 32 * kRowBytes);
#pragma unroll
    for (int ci = 0; ci < C; ++ci) bf[0][ci] = *reinterpret_cast<const half8*>(tb + b_frag[0] + ci * 32 * kRowBytes);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s < 3) {
#pragma unroll
        for (int mi = 0; mi < R; ++mi)
          af[(s + 1) & 1][mi] = *reinterpret_cast<const half8*>(ta + a_frag[s + 1] + mi * 32 * kRowBytes);
#pragma unroll
        for (int ci = 0; ci < C; ++ci)
          bf[(s + 1) & 1][ci] = *reinterpret_cast<const half8*>(tb + b_frag[s + 1] + ci * 32 * kRowBytes);
      }
      if (i + 1u < steps) decode_chunk(dec, s, nxt, i + 1u);
#pragma unroll
      for (int ci = 0; ci < C; ++ci)
#pragma unroll
        for (int mi = 0; mi < R; ++mi)
          acc[mi][ci] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[s & 1][ci], af[s & 1][mi], acc[mi][ci], 0, 0, 0);
    }
    store_a(min(kb_begin + i + 1u, last_kb), nxt, a_store);
    __syncthreads();
  };

  if (steps > 0) {
    uint32_t c0[U][BITS], c1[U][BITS], c2[U][BITS];
    uint4 s0[CH], s1[CH], s2[CH];
    load_codes(kb_begin, c0);
    load_codes(min(kb_begin + 1u, last_kb), c1);
    load_codes(min(kb_begin + 2u, last_kb), c2);
    load_a(kb_begin, s0);
    load_a(min(kb_begin + 1u, last_kb), s1);
    load_a(min(kb_begin + 2u, last_kb), s2);
    __syncthreads();  // palettes staged
#pragma unroll
    for (int q = 0; q < 4; ++q) decode_chunk(c0, q, 0u, 0u);
    store_a(kb_begin, 0u, s0);
    __syncthreads();

    // Code sets: block b lives in set b % 3; activation sets likewise.
    uint32_t i = 0;
    for (; i + 3u <= steps; i += 3u) {
      step(i, c1, c0, s0, s1);
      step(i + 1u, c2, c1, s1, s2);
      step(i + 2u, c0, c2, s2, s0);
    }
    if (i < steps) step(i, c1, c0, s0, s1);
    if (i + 1u < steps) step(i + 1u, c2, c1, s1, s2);
  }

  if (S > 1 && !split_k_reduce<R, C, T>(args, acc, tile, split, tid, &last_flag)) return;
  store_tile<WM, 1, R, C, 2 * BM * kRowBytes>(args, acc, a_lds, m0, n0, wave_m, 0, j, h, tid);
}

#define PK_F16S_VARIANT(WM, R, C)                                                                         \
  F16Variant {                                                                                            \
    TileShape{WM, 1, R, C}, "pk_gemm_f16s_b5_w" #WM "x1_m" #R "n" #C, "pk_gemm_f16s_b6_w" #WM "x1_m" #R "n" #C, \
        {gemm_f16_shared_kernel<5, WM, R, C, false>, gemm_f16_shared_kernel<6, WM, R, C, false>},         \
        {gemm_f16_shared_kernel<5, WM, R, C, true>, gemm_f16_shared_kernel<6, WM, R, C, true>}            \
  }

const F16Variant kShared[] = {
    PK_F16S_VARIANT(4, 2, 4),  // 256 x 128
    PK_F16S_VARIANT(4, 1, 4),  // 128 x 128
};

}  // namespace

int f16_shared_variant_count() { return (int)(sizeof(kShared) / sizeof(kShared[0])); }
const f16::F16Variant& f16_shared_variant(int index) { return kShared[index]; }

}  // namespace pk

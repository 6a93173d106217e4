// pk_gemm_f16k.hip - fused palette-weight GEMM for the large-M shapes: f16
// operands, f32 MFMA accumulation, pair codes, K split across the
// wavefronts of a workgroup (gfx950, wave64).
//
// C[m, n] = epilogue(sum_k A[m, k] * LUT[g(n)][code(k, n)])
// (reference: src/webgpu/kernels/gemm.ts:1362-1716, epilogue :2006-2044).
//
// What bounds these shapes is LDS traffic, not MFMA issue: every weight
// comes out of a palette gather and every activation fragment is a
// ds_read_b128. A workgroup of four wavefronts owns a BM x BN tile
// (BM = 32*R, BN = 32*C*WN) as WN column groups x KS K parts: wavefront
// (wn, kp) multiplies R x C MFMA blocks but only over the 4/KS sub-steps of
// each 64-deep K block that belong to part kp. So every code of the tile is
// gathered once per workgroup and every activation fragment is read by WN
// wavefronts, not by all four; the KS partial tiles are added through LDS
// at the end.
//
//   * codes: the operand-order layout split into KS parts (pk_internal.h):
//     a wavefront of K part kp loads only its own part, one coalesced run
//     per lane and column block (16 + 4/8 bytes with one part, 16 bytes with
//     two, 8 with four), CLA K blocks ahead. With one part (the packed
//     density) two K-adjacent codes are next to each other, so their
//     2*bits-bit field c0 | c1 << bits, at a fixed bit, indexes a packed
//     pair of palette entries: one extract (plus a funnel shift where the
//     field crosses a word) and one ds_read_b32 yield a whole operand
//     register (two halves); with two or four parts each pair is a 16-bit
//     slot that already holds the entry's byte offset. The 2^bits x 2^bits
//     pair table is built in LDS by each workgroup from the tile's palette.
//   * activations: the BM x 64 tile of K block i+4 is loaded into registers
//     while block i is multiplied and written to a ring of three LDS tiles
//     at the end of block i+2; 16-byte chunks are XOR-swizzled with
//     (row >> 1) & 7 so the 16 lanes of every ds_read_b128 phase hit
//     distinct bank groups. With three tiles the fragments of block i+1 can
//     be read during block i.
//   * sub-step s+1's weight and activation fragments are fetched while the
//     MFMAs of sub-step s run (ping-pong register sets), and the fetches
//     are spread between the MFMAs (sched_group_barrier).
//   * v_mfma_f32_32x32x16_f16 computes D = W^T * A^T; in sub-step s, lane
//     half h, element t stands for k = 64*kb + 32*h + 8*s + t in both
//     operands.
//   * epilogue: the partial tiles of a few m-blocks at a time go to LDS as
//     float4 runs (lane index XOR 4q so both the writes and the row-wise
//     reads are conflict-free); each thread then sums the KS partials of
//     8 consecutive columns of one row in K-part order, applies bias,
//     SiLU/ReLU and residual + scale * value in f32, and stores 16 bytes.
//   * GLU epilogue (args.glu): the weight's column blocks were interleaved
//     at preparation (block 2i = values of channels 32i.., block 2i+1 =
//     their gates), so a tile holds both halves of its channels; a thread
//     sums the value and gate partials of 8 channels, rounds each to f16
//     (the reference stores the pointwise output in f16 before its GLU,
//     conformer-conv.ts:520-535) and writes value * sigmoid(gate) to a
//     [M, N/2] output.
//   * fused row LayerNorm (NORM, args.norm_columns; see GemmArgs): the
//     activation staging multiplies each chunk by gamma (packed f16, gamma
//     staged in LDS) and adds the chunk's sum and sum of squares to the
//     staging thread's row accumulators (v_dot2_f32_f16); the eight threads
//     of a row combine them after the K loop into mean and rstd, and the
//     epilogue finishes rstd * (acc - mean * G_n) + B_n before bias and
//     activation.
#include <utility>

#include "pk_f16_common.h"

namespace pk {
namespace {

using namespace f16;

// Each staged palette group occupies 65 LDS entries: its 2^bits centroids
// and zeros up to entry 64.
constexpr int kLutStride = 65;
constexpr uint32_t kLutStrideBytes = 2u * kLutStride;
// LDS budget of the partial-tile exchange. The 96 x 128 tile (WN = KS = 2,
// R = 3) keeps one m-block per pass: its registers allow two wavefronts per
// SIMD, and with a 32 KB exchange two of its workgroups fit one compute
// unit's LDS, so one workgroup's prologue and epilogue overlap the other's
// K loop. The planner gives it the shapes with more tiles than compute
// units. Every other tile runs one workgroup per compute unit and takes
// the exchange in as few passes as 96 KB allow.
constexpr int exchange_cap(int wn, int ks, int r) { return wn == 2 && ks == 2 && r == 3 ? 32 * 1024 : 96 * 1024; }

// m-blocks per epilogue pass: the largest divisor of R whose partial tiles
// fit the exchange budget.
constexpr int pass_blocks(int wn, int ks, int r, int block_bytes) {
  int best = 1;
  for (int p = 1; p <= r; ++p)
    if (r % p == 0 && p * block_bytes <= exchange_cap(wn, ks, r)) best = p;
  return best;
}

template <int I>
struct Step {
  static constexpr int value = I;
};

template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>), in order.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Instruction interleave of one sub-step (one scheduling region, fenced by
// sched_barrier): the R*C MFMAs are spread over the region. The first two
// thirds of the MFMA slots each carry an even share of the next sub-step's
// LDS work - pair-offset extracts (VPP VALU per pair), palette-pair gathers
// and activation fragment reads - so it issues in the shadow of the MFMA
// pipe and has the last third of the region to land; the last third
// carries the VMEM loads (sub-step 0) and the activation tile's LDS stores
// (last sub-step).
template <int R, int C, int VMEM, int DSW, int VPP, int XV = 0>
__device__ __forceinline__ void interleave_sub_step() {
  constexpr int NM = R * C;
  constexpr int NL = (2 * NM) / 3 > 0 ? (2 * NM) / 3 : 1;
  constexpr int NT = NM - NL > 0 ? NM - NL : 1;
  constexpr int V_PER = (4 * VPP * C + NL - 1) / NL;
  constexpr int D_PER = (4 * C + R + NL - 1) / NL;
  constexpr int M_PER = (VMEM + NT - 1) / NT;
  constexpr int W_PER = (DSW + NT - 1) / NT;
  constexpr int X_PER = (XV + NT - 1) / NT;  // staging VALU (fused row norm) beside the stores
  constexpr int kMfma = 0x008, kValu = 0x002, kVmemRead = 0x020, kDsRead = 0x100, kDsWrite = 0x200;
  for (int x = 0; x < NL; ++x) {
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kValu, V_PER, 0);
    __builtin_amdgcn_sched_group_barrier(kDsRead, D_PER, 0);
  }
  for (int x = NL; x < NM; ++x) {
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    if constexpr (M_PER > 0) __builtin_amdgcn_sched_group_barrier(kVmemRead, M_PER, 0);
    if constexpr (X_PER > 0) __builtin_amdgcn_sched_group_barrier(kValu, X_PER, 0);
    if constexpr (W_PER > 0) __builtin_amdgcn_sched_group_barrier(kDsWrite, W_PER, 0);
  }
}


// GENERAL: the tile's columns may span palette groups (per-lane palette
// base) or K may be 32 (mod 64) (the last K block's upper half is zeroed,
// so the code-0 padding of the operand order multiplies zeros).
template <int BITS, int WN, int KS, int R, int C, bool GENERAL, bool SCHED, int CLA, bool NORM = false,
          bool STREAM = false>
__global__ __launch_bounds__(256) void gemm_f16k_kernel(GemmArgs args) {
  constexpr int T = 256;
  constexpr int BM = 32 * R;
  constexpr int BN = 32 * C * WN;
  constexpr int NCB = BN / 32;    // 32-column blocks of the tile
  constexpr int SPW = 4 / KS;     // sub-steps per wavefront per K block
  constexpr int A_BYTES = BM * kRowBytes;
  constexpr int CH = BM * 8 / T;  // 16-byte activation chunks per thread per K block
  constexpr int BLOCK_EX = KS * WN * C * 4 * 64 * 16;  // exchange bytes of one m-block
  constexpr int PM = pass_blocks(WN, KS, R, BLOCK_EX);
  constexpr int EX_BYTES = PM * BLOCK_EX;
  constexpr int SMEM = EX_BYTES > 3 * A_BYTES ? EX_BYTES : 3 * A_BYTES;
  constexpr int GROUPS = GENERAL ? BN / 16 + 2 : 1;
  constexpr uint32_t E = 1u << BITS;               // palette entries
  constexpr int PAIRS = GENERAL ? 1 : (int)(E * E);  // pair table of the tile's palette
  constexpr uint32_t BLOCK_WORDS = block_words(BITS, KS);
  // 32-bit words of this wavefront's K part of one block.
  constexpr int LW = (int)parts_words(BITS, KS);
  constexpr uint32_t FIELD_MASK = (1u << (2 * BITS)) - 1u;
  static_assert(WN * KS == 4, "a workgroup is four wavefronts");
  static_assert(KS == 1 || KS == 2 || KS == 4, "K parts split the four sub-steps evenly");
  static_assert(BM * 8 % T == 0, "activation tile chunks must divide evenly");
  static_assert(!(NORM && GENERAL), "the fused row norm runs on the fixed-palette path");

  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];
  __shared__ __attribute__((aligned(16))) _Float16 lut_lds[GROUPS * kLutStride];
  __shared__ __attribute__((aligned(16))) uint32_t pair_lds[PAIRS];
  // Fused row norm: gamma of every K channel (f16) and (mean, rstd) of
  // every tile row.
  __shared__ __attribute__((aligned(16))) _Float16 gamma_lds[NORM ? kNormMaxInner : 1];
  __shared__ float2 row_stats[NORM ? BM : 1];
  __shared__ float2 column_gb[NORM ? BN : 1];  // (G_n, B_n) of the tile's columns

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % WN;
  const int kp = wave / WN;
  const int j = lane & 31;
  const int h = lane >> 5;

  const uint32_t M = args.rows;
  const uint32_t K = args.inner;
  const uint32_t N = args.columns;
  const uint32_t KB = (K + 63u) / 64u;
  const uint32_t NBT = (N + 31u) / 32u;
  const uint32_t TN = (NBT + NCB - 1u) / NCB;

  // Work items come in bands of GM row tiles with the row tile fastest
  // inside a band, and xcd_local_order gives each XCD a contiguous range of
  // items: an XCD works on a block of about GM row tiles x (its share / GM)
  // column tiles, so its L2 holds a few activation row bands and a slice
  // of the weights instead of all of either.
  constexpr uint32_t GM = 4;
  const uint32_t TM = (M + BM - 1u) / BM;
  const uint32_t item = xcd_local_order(blockIdx.x, gridDim.x);
  const uint32_t band = item / (GM * TN);
  const uint32_t band_rows = min(GM, TM - band * GM);
  const uint32_t in_band = item - band * GM * TN;
  const uint32_t tm = band * GM + in_band % band_rows;
  const uint32_t tn = in_band / band_rows;
  const uint32_t m0 = tm * BM;
  const uint32_t n0 = tn * BN;

  // Palettes of the tile's columns (palette-expander.ts:543-549).
  const uint32_t gc = args.palette_group_columns;
  const uint32_t G = args.palette_groups;
  const uint32_t g_lo = min(n0 / gc, G - 1u);
  // Staged in the prologue, while the first global loads are in flight:
  // the palettes of the tile's groups and, for single-group tiles, the
  // table of packed palette pairs, entry c0 | c1 << bits = LUT[c0] |
  // LUT[c1] << 16.
  auto stage_palettes = [&]() {
    if constexpr (NORM) {
      for (uint32_t i = tid; i < K; i += T) gamma_lds[i] = args.norm_gamma[i];
      for (uint32_t i = tid; i < (uint32_t)BN; i += T) {
        const uint32_t n = min(n0 + i, N - 1u);
        column_gb[i] = make_float2(args.norm_columns[n], args.norm_columns[N + n]);
      }
    }
    const uint32_t g_hi = GENERAL ? min((min(n0 + BN, N) - 1u) / gc, G - 1u) : g_lo;
    const uint32_t entries = (g_hi - g_lo + 1u) * kLutStride;
    const _Float16* src = static_cast<const _Float16*>(args.palette);
    for (uint32_t i = tid; i < entries; i += T) {
      const uint32_t g = i / kLutStride, e = i % kLutStride;
      lut_lds[i] = e < E ? src[(uint64_t)(g_lo + g) * E + e] : (_Float16)0.0f;
    }
    if constexpr (!GENERAL) {
      __syncthreads();
      const uint16_t* lut16 = reinterpret_cast<const uint16_t*>(lut_lds);
#pragma unroll 4
      for (uint32_t p = tid; p < E * E; p += T)
        pair_lds[p] = (uint32_t)lut16[p & (E - 1u)] | ((uint32_t)lut16[p >> BITS] << 16);
    }
  };
  const uint8_t* lut_bytes = reinterpret_cast<const uint8_t*>(lut_lds);
  const uint8_t* pair_bytes = reinterpret_cast<const uint8_t*>(pair_lds);
  uint32_t lut_base[C];
#pragma unroll
  for (int ci = 0; ci < C; ++ci) {
    if constexpr (GENERAL) {
      const uint32_t n = min(n0 + (uint32_t)((wn * C + ci) * 32 + j), N - 1u);
      lut_base[ci] = (min(n / gc, G - 1u) - g_lo) * kLutStrideBytes;
    } else {
      lut_base[ci] = 0u;
    }
  }

  // Codes of this wavefront's column blocks and K part. Blocks past the
  // last column block re-read the last one (never stored).
  typedef uint32_t Codes[C][LW];
  const uint32_t nb0 = n0 / 32u + (uint32_t)(wn * C);
  const uint32_t* code_base[C];
#pragma unroll
  for (int ci = 0; ci < C; ++ci)
    code_base[ci] = args.codes + (uint64_t)min(nb0 + ci, NBT - 1u) * KB * BLOCK_WORDS;
  auto load_codes = [&](uint32_t kb, Codes& dst) {
#pragma unroll
    for (int ci = 0; ci < C; ++ci) {
      const uint32_t* blk = code_base[ci] + (uint64_t)kb * BLOCK_WORDS;
      if constexpr (KS == 1) {
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
      } else if constexpr (LW == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(blk + ((uint32_t)kp * 64u + (uint32_t)lane) * 4u);
        dst[ci][0] = v.x;
        dst[ci][1] = v.y;
        dst[ci][2] = v.z;
        dst[ci][3] = v.w;
      } else {
        const uint2 v = *reinterpret_cast<const uint2*>(blk + ((uint32_t)kp * 64u + (uint32_t)lane) * 2u);
        dst[ci][0] = v.x;
        dst[ci][1] = v.y;
      }
    }
  };

  // Activation tile: chunk c of this thread is row r = (tid + c*T) / 8,
  // 16-byte column chunk ch = (tid + c*T) % 8. Rows past M re-read row M-1
  // (never stored). In a K = 32 (mod 64) tail block, chunks past K re-read
  // chunk ch - 4 of the row and are stored as zeros.
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
  // Fused row norm: this thread's share of the sum and the sum of squares
  // of rows (tid >> 3) + 32c, over the K blocks it stages.
  float row_sum[NORM ? CH : 1], row_sq[NORM ? CH : 1];
#pragma unroll
  for (int c = 0; c < (NORM ? CH : 1); ++c) row_sum[c] = row_sq[c] = 0.0f;
  // Stores K block `want` (clamped to the last block).
  auto store_a = [&](uint32_t want, int buf, const uint4 (&src)[CH]) {
    const uint32_t kb = min(want, KB - 1u);
    const bool partial = GENERAL && (K & 63u) != 0u && kb + 1u == KB;
    uint8_t* dst = smem + buf * A_BYTES;
    if constexpr (NORM) {
      typedef _Float16 half2v __attribute__((ext_vector_type(2)));
      const uint4 g4 = *reinterpret_cast<const uint4*>(gamma_lds + kb * 64u + (uint32_t)(tid & 7) * 8u);
      const half2v g[4] = {__builtin_bit_cast(half2v, g4.x), __builtin_bit_cast(half2v, g4.y),
                           __builtin_bit_cast(half2v, g4.z), __builtin_bit_cast(half2v, g4.w)};
      const half2v one = {(_Float16)1.0f, (_Float16)1.0f};
      // Clamped repeats of the last block enter the statistics too; they are
      // taken out once after the K loop.
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const uint32_t w[4] = {src[c].x, src[c].y, src[c].z, src[c].w};
        uint32_t y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const half2v x = __builtin_bit_cast(half2v, w[e]);
          row_sum[c] = __builtin_amdgcn_fdot2(x, one, row_sum[c], false);
          row_sq[c] = __builtin_amdgcn_fdot2(x, x, row_sq[c], false);
          y[e] = __builtin_bit_cast(uint32_t, x * g[e]);
        }
        *reinterpret_cast<uint4*>(dst + a_st[c]) = make_uint4(y[0], y[1], y[2], y[3]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        uint4 v = src[c];
        if (partial && ((tid + c * T) & 7) >= 4) v = make_uint4(0u, 0u, 0u, 0u);
        *reinterpret_cast<uint4*>(dst + a_st[c]) = v;
      }
    }
  };
  // LDS offset of this lane's activation fragment in local sub-step ls of
  // m-block 0 (sub-step s = kp*SPW + ls: row j, chunk 4h + s, swizzled;
  // rows 32*mi + j share the swizzle of row j).
  uint32_t a_frag_off[SPW];
#pragma unroll
  for (int ls = 0; ls < SPW; ++ls)
    a_frag_off[ls] = (uint32_t)(j * kRowBytes + (((4 * h + kp * SPW + ls) ^ ((j >> 1) & 7)) << 4));

  auto read_a = [&](int buf, int ls, half8 (&dst)[R]) {
    const uint8_t* t = smem + buf * A_BYTES + a_frag_off[ls];
#pragma unroll
    for (int mi = 0; mi < R; ++mi) dst[mi] = *reinterpret_cast<const half8*>(t + mi * 32 * kRowBytes);
  };
  // Weight fragment of local sub-step ls: register e of column block ci is
  // the packed pair (halves 2e, 2e+1) of codes 8 ls + 2e, + 1 of the
  // wavefront's part, i.e. the 2*bits-bit field at bit 2 bits (4 ls + e)
  // of its words (with one part: words 0-3 and 4(-5), contiguous), or with
  // two or four parts the 16-bit slot 4 ls + e holding four times that
  // field. Single-group
  // tiles gather it whole from the pair table; GENERAL tiles split the
  // field into its two codes and gather each from the lane's own group
  // palette.
  auto gather = [&](const Codes& cw, auto lsc, half8 (&dst)[C]) {
    constexpr int ls = decltype(lsc)::value;
#pragma unroll
    for (int ci = 0; ci < C; ++ci) {
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      u32x4 w;
      static_for<4>([&](auto ec) {
        constexpr int e = decltype(ec)::value;
        uint32_t offset;  // 4 * field: the byte offset of the pair's table entry
        if constexpr (KS > 1) {
          // 16-bit pair slots that already hold the offset: slot 4 ls + e
          constexpr int slot = 4 * ls + e;
          offset = (cw[ci][slot >> 1] >> (16 * (slot & 1))) & 0xffffu;
        } else {
          constexpr int bit = 2 * BITS * (4 * ls + e);
          constexpr int wi = bit >> 5, sh = bit & 31;
          uint32_t field;
          if constexpr (sh + 2 * BITS <= 32)
            field = (cw[ci][wi] >> sh) & FIELD_MASK;
          else
            field = __builtin_amdgcn_alignbit(cw[ci][wi + 1], cw[ci][wi], (uint32_t)sh) & FIELD_MASK;
          offset = 4u * field;
        }
        if constexpr (GENERAL) {
          const uint32_t field = offset >> 2;
          const uint8_t* lut = lut_bytes + lut_base[ci];
          w[e] = (uint32_t)*reinterpret_cast<const uint16_t*>(lut + 2u * (field & (E - 1u))) |
                 ((uint32_t)*reinterpret_cast<const uint16_t*>(lut + 2u * (field >> BITS)) << 16);
        } else {
          w[e] = *reinterpret_cast<const uint32_t*>(pair_bytes + offset);
        }
      });
      dst[ci] = __builtin_bit_cast(half8, w);
    }
  };

  floatx16 acc[R][C];
#pragma unroll
  for (int mi = 0; mi < R; ++mi)
#pragma unroll
    for (int ci = 0; ci < C; ++ci)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ci][v] = 0.0f;

  // Register sets rotate with the K block index i. Codes run CLA blocks
  // ahead in CLA + 1 sets: step i loads block i+CLA into cs[(i+CLA) % NCS]
  // and gathers from cs[i % NCS] (this block) and cs[(i+1) % NCS] (the
  // next block's first sub-step). Activations run four blocks ahead in
  // three sets: step i loads block i+4 into sa[(i+1) % 3] and stores block
  // i+2 (loaded at step i-2) from sa[(i+2) % 3] to LDS tile (i+2) % 3.
  // Activation fragments alternate between two sets by the parity of the
  // global sub-step index, so the loop is unrolled by six (NCS divides 6).
  // Loads past the last block re-read it, which keeps every step's loads
  // identical.
  constexpr int NCS = CLA + 1;
  static_assert(6 % NCS == 0, "code register sets must divide the unroll");
  Codes cs[NCS];
  uint4 sa[3][CH];
  half8 af[2][R];
  half8 bf[2][C];
  const uint32_t last = KB - 1u;

  auto step = [&](auto idx, uint32_t i) {
    constexpr int I = decltype(idx)::value;
    constexpr int BUF = I % 3;
    static_for<SPW>([&](auto lsc) {
      constexpr int ls = decltype(lsc)::value;
      constexpr int g = (I * SPW + ls) & 1;
      if constexpr (ls == 0) {
        load_codes(min(i + (uint32_t)CLA, last), cs[(I + CLA) % NCS]);
        load_a(min(i + 4u, last), sa[(I + 1) % 3]);
      }
      if constexpr (ls + 1 < SPW) {
        read_a(BUF, ls + 1, af[g ^ 1]);
        gather(cs[I % NCS], std::integral_constant<int, ls + 1>{}, bf[g ^ 1]);
      } else {
        read_a((BUF + 1) % 3, 0, af[g ^ 1]);
        gather(cs[(I + 1) % NCS], std::integral_constant<int, 0>{}, bf[g ^ 1]);
      }
#pragma unroll
      for (int ci = 0; ci < C; ++ci)
#pragma unroll
        for (int mi = 0; mi < R; ++mi)
          acc[mi][ci] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[g][ci], af[g][mi], acc[mi][ci], 0, 0, 0);
      if constexpr (ls + 1 == SPW) store_a(i + 2u, (BUF + 2) % 3, sa[(I + 2) % 3]);
      if constexpr (SCHED) {
        interleave_sub_step<R, C, ls == 0 ? CH + C * (KS == 1 ? 2 : 1) : 0, ls + 1 == SPW ? CH : 0, KS == 1 ? 2 : 1,
                            NORM && ls + 1 == SPW ? 12 * CH : 0>();
        if constexpr (ls + 1 < SPW) __builtin_amdgcn_sched_barrier(0);
      }
    });
    __syncthreads();
  };

#pragma unroll
  for (int b = 0; b < CLA; ++b) load_codes(min((uint32_t)b, last), cs[b]);
  load_a(0u, sa[0]);
  load_a(min(1u, last), sa[1]);
  load_a(min(2u, last), sa[2]);
  stage_palettes();
  store_a(0u, 0, sa[0]);
  store_a(1u, 1, sa[1]);
  load_a(min(3u, last), sa[0]);
  __syncthreads();
  read_a(0, 0, af[0]);
  gather(cs[0], std::integral_constant<int, 0>{}, bf[0]);

  uint32_t i = 0;
  for (; i + 6u <= KB; i += 6u) {
    step(Step<0>{}, i);
    step(Step<1>{}, i + 1u);
    step(Step<2>{}, i + 2u);
    step(Step<3>{}, i + 3u);
    step(Step<4>{}, i + 4u);
    step(Step<5>{}, i + 5u);
  }
  if (i < KB) step(Step<0>{}, i);
  if (i + 1u < KB) step(Step<1>{}, i + 1u);
  if (i + 2u < KB) step(Step<2>{}, i + 2u);
  if (i + 3u < KB) step(Step<3>{}, i + 3u);
  if (i + 4u < KB) step(Step<4>{}, i + 4u);

  if constexpr (NORM) {
    // Every K-block index from 0 to KB + 1 is staged once, the two past the
    // end as repeats of the last block, which every activation register set
    // holds when the loop ends (loads past the end are clamped to it): the
    // repeats' share is taken out of the sums here.
    {
      typedef _Float16 half2v __attribute__((ext_vector_type(2)));
      const half2v one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const uint32_t w[4] = {sa[0][c].x, sa[0][c].y, sa[0][c].z, sa[0][c].w};
        float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const half2v x = __builtin_bit_cast(half2v, w[e]);
          s1 = __builtin_amdgcn_fdot2(x, one, s1, false);
          s2 = __builtin_amdgcn_fdot2(x, x, s2, false);
        }
        row_sum[c] -= 2.0f * s1;
        row_sq[c] -= 2.0f * s2;
      }
    }
    // The eight threads of a row (consecutive lanes) combine their shares;
    // mean, variance max(E[x^2] - mean^2, 0) and 1 / sqrt(variance + eps)
    // as the reference LayerNorm (layernorm.ts:309-390). The first barrier
    // of the epilogue orders these stores before the reads.
    const float inverse_k = 1.0f / (float)K;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float sm = row_sum[c], sq = row_sq[c];
#pragma unroll
      for (int off = 1; off < 8; off <<= 1) {
        sm += __shfl_xor(sm, off, 64);
        sq += __shfl_xor(sq, off, 64);
      }
      if ((tid & 7) == 0) {
        const float mean = sm * inverse_k;
        const float variance = fmaxf(sq * inverse_k - mean * mean, 0.0f);
        row_stats[(tid >> 3) + 32 * c] = make_float2(mean, 1.0f / __builtin_sqrtf(variance + args.norm_epsilon));
      }
    }
  }

  // Fused row norm: every epilogue unit of this thread covers the same 8
  // columns (quad tid & 3 of column block (tid >> 4) % NCB; NCB divides 16),
  // so their G and B are read once.
  float norm_g[NORM ? 8 : 1], norm_b[NORM ? 8 : 1];
  if constexpr (NORM) {
    static_assert(16 % NCB == 0, "a thread's epilogue units share their columns");
    const int c0 = ((tid >> 4) % NCB) * 32 + (tid & 3) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float2 gb = column_gb[c0 + e];
      norm_g[e] = gb.x;
      norm_b[e] = gb.y;
    }
  }

  const _Float16* residual = static_cast<const _Float16*>(args.residual);
  _Float16* out = static_cast<_Float16*>(args.out);
  // Epilogue, PM m-blocks per pass. Exchange slot of (kp, wn, m-block,
  // column block ci, quad q, lane): float4 of acc[..][4q..4q+3], i.e. row
  // 32*mi + j, columns 32*ci + 8q + 4h + {0..3} of the wavefront's blocks.
  float4* ex = reinterpret_cast<float4*>(smem);
  constexpr int UNITS = PM * 32 * NCB * 4;  // 8-column row units per pass
  constexpr int UPT = UNITS / T;            // units per thread
  static_assert(UNITS % T == 0, "epilogue units must divide evenly");
#pragma unroll
  for (int p0 = 0; p0 < R; p0 += PM) {
    __syncthreads();
#pragma unroll
    for (int ml = 0; ml < PM; ++ml)
#pragma unroll
      for (int ci = 0; ci < C; ++ci)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int slot = (((kp * WN + wn) * PM + ml) * C + ci) * 4 + q;
          ex[slot * 64 + (lane ^ (q << 2))] = make_float4(acc[p0 + ml][ci][4 * q], acc[p0 + ml][ci][4 * q + 1],
                                                          acc[p0 + ml][ci][4 * q + 2], acc[p0 + ml][ci][4 * q + 3]);
        }
    __syncthreads();
    // Sum of the KS partials of 8 columns (column block cb, quad q) of tile
    // row 32*ml + jj.
    auto unit_sum = [&](int cb, int ml, int jj, int q, float (&v)[8]) {
      const int wn_u = cb / C, ci_u = cb % C;
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const int slot = (((k * WN + wn_u) * PM + ml) * C + ci_u) * 4 + q;
        const float4 x0 = ex[slot * 64 + (jj ^ (q << 2))];
        const float4 x1 = ex[slot * 64 + 32 + (jj ^ (q << 2))];
        const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = k == 0 ? x[e] : v[e] + x[e];
      }
    };
    if constexpr (NCB % 2 == 0) {
      if (args.glu) {
        // Unit u covers 8 channels of one row: the value block 2*cp and the
        // gate block 2*cp + 1 of column-block pair cp.
        constexpr int GUNITS = PM * 32 * (NCB / 2) * 4;
        constexpr int GUPT = (GUNITS + T - 1) / T;
        const uint32_t NC = N / 2u;
#pragma unroll
        for (int it = 0; it < GUPT; ++it) {
          const int u = tid + it * T;
          if (GUNITS % T != 0 && u >= GUNITS) break;
          const int q = u & 3;
          const int rest = u >> 4;
          const int cp = rest % (NCB / 2);
          const int rl = (rest / (NCB / 2)) * 4 + ((u >> 2) & 3);
          const uint32_t m = m0 + (uint32_t)(p0 * 32 + rl);
          const uint32_t c = n0 / 2u + (uint32_t)(cp * 32 + q * 8);
          float value[8], gate[8];
          unit_sum(2 * cp, rl >> 5, rl & 31, q, value);
          unit_sum(2 * cp + 1, rl >> 5, rl & 31, q, gate);
          float g[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) g[e] = through_f16(value[e]) * sigmoid(through_f16(gate[e]));
          if (m < M && c < NC) {
            const uint4 y = make_uint4(pack_half2(g[0], g[1]), pack_half2(g[2], g[3]), pack_half2(g[4], g[5]),
                                       pack_half2(g[6], g[7]));
            if constexpr (STREAM)
              stream_store(reinterpret_cast<uint4*>(out + (uint64_t)m * NC + c), y);
            else
              *reinterpret_cast<uint4*>(out + (uint64_t)m * NC + c) = y;
          }
        }
        continue;
      }
    }
    // Unit u: quad q = u & 3 and row low bits u >> 2 & 3 vary fastest, so a
    // 16-lane phase reads 16 distinct bank groups and a wavefront stores
    // 4 rows x 64 contiguous bytes per column block. A thread's UPT units
    // go through each stage together (all partial reads, then bias, the
    // activation, the residual loads and the stores), which keeps many
    // independent VALU chains and memory operations in flight. Units past M
    // or N read clamped, in-bounds addresses and store nothing.
    float v[UPT][8];
    uint64_t at[UPT];
    uint32_t n_of[UPT];
    bool keep[UPT];
#pragma unroll
    for (int it = 0; it < UPT; ++it) {
      const int u = tid + it * T;
      const int q = u & 3;
      const int rest = u >> 4;
      const int cb = rest % NCB;
      const int rl = (rest / NCB) * 4 + ((u >> 2) & 3);
      const int ml = rl >> 5, jj = rl & 31;
      const uint32_t m = m0 + (uint32_t)(p0 * 32 + rl);
      const uint32_t n = n0 + (uint32_t)(cb * 32 + q * 8);
      keep[it] = m < M && n < N;
      n_of[it] = min(n, N - 8u);
      at[it] = (uint64_t)min(m, M - 1u) * N + n_of[it];
      unit_sum(cb, ml, jj, q, v[it]);
      if constexpr (NORM) {
        // rstd * (acc - mean * G_n) + B_n: the GEMM of the normalised row.
        const float2 st = row_stats[p0 * 32 + rl];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[it][e] = st.y * (v[it][e] - st.x * norm_g[e]) + norm_b[e];
      }
    }
    if (args.bias) {
#pragma unroll
      for (int it = 0; it < UPT; ++it) {
        const float4 b0 = *reinterpret_cast<const float4*>(args.bias + n_of[it]);
        const float4 b1 = *reinterpret_cast<const float4*>(args.bias + n_of[it] + 4);
        v[it][0] += b0.x;
        v[it][1] += b0.y;
        v[it][2] += b0.z;
        v[it][3] += b0.w;
        v[it][4] += b1.x;
        v[it][5] += b1.y;
        v[it][6] += b1.z;
        v[it][7] += b1.w;
      }
    }
    if (args.activation == kActSilu) {
#pragma unroll
      for (int it = 0; it < UPT; ++it)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[it][e] = silu(v[it][e]);
    } else if (args.activation == kActRelu) {
#pragma unroll
      for (int it = 0; it < UPT; ++it)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[it][e] = fmaxf(v[it][e], 0.0f);
    }
    if (residual) {
      const float sc = args.residual_scale;
#pragma unroll
      for (int it = 0; it < UPT; ++it) {
        const uint4 rb = *reinterpret_cast<const uint4*>(residual + at[it]);
        const uint32_t rw[4] = {rb.x, rb.y, rb.z, rb.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[it][2 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(rw[e] & 0xffffu)) + sc * v[it][2 * e];
          v[it][2 * e + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(rw[e] >> 16)) + sc * v[it][2 * e + 1];
        }
      }
    }
#pragma unroll
    for (int it = 0; it < UPT; ++it)
      if (keep[it]) {
        const uint4 y = make_uint4(pack_half2(v[it][0], v[it][1]), pack_half2(v[it][2], v[it][3]),
                                   pack_half2(v[it][4], v[it][5]), pack_half2(v[it][6], v[it][7]));
        if constexpr (STREAM)
          stream_store(reinterpret_cast<uint4*>(out + at[it]), y);
        else
          *reinterpret_cast<uint4*>(out + at[it]) = y;
      }
  }
}

template <int WN, int KS, int R, int C>
constexpr uint32_t kernel_lds_bytes() {
  constexpr int A_BYTES = 32 * R * kRowBytes;
  constexpr int BLOCK_EX = KS * WN * C * 4 * 64 * 16;
  constexpr int EX = pass_blocks(WN, KS, R, BLOCK_EX) * BLOCK_EX;
  return (uint32_t)((EX > 3 * A_BYTES ? EX : 3 * A_BYTES) + kLutStride * 2 + 64 * 64 * 4);
}

#define PK_F16K_VARIANT(WN, KS, R, C, S, CLA, TAG)                                                              \
  F16Variant {                                                                                              \
    TileShape{1, WN, R, C, KS}, "pk_gemm_f16p_b5_n" #WN "k" #KS "_m" #R "n" #C TAG,                         \
        "pk_gemm_f16p_b6_n" #WN "k" #KS "_m" #R "n" #C TAG,                                                 \
        {gemm_f16k_kernel<5, WN, KS, R, C, false, S, CLA>, gemm_f16k_kernel<6, WN, KS, R, C, false, S, CLA>}, \
        {gemm_f16k_kernel<5, WN, KS, R, C, true, S, CLA>, gemm_f16k_kernel<6, WN, KS, R, C, true, S, CLA>},   \
        kernel_lds_bytes<WN, KS, R, C>(),                                                                   \
        {gemm_f16k_kernel<5, WN, KS, R, C, false, S, CLA, true>,                                            \
         gemm_f16k_kernel<6, WN, KS, R, C, false, S, CLA, true>},                                           \
        {gemm_f16k_kernel<5, WN, KS, R, C, false, S, CLA, false, true>,                                     \
         gemm_f16k_kernel<6, WN, KS, R, C, false, S, CLA, false, true>},                                    \
  }

const F16Variant kVariants[] = {
    PK_F16K_VARIANT(2, 2, 6, 2, true, 2, ""),  // 192 x 128
    PK_F16K_VARIANT(4, 1, 6, 1, true, 5, ""),  // 192 x 128, no K split
    PK_F16K_VARIANT(2, 2, 4, 2, true, 5, ""),  // 128 x 128
    PK_F16K_VARIANT(2, 2, 3, 2, true, 5, ""),  // 96 x 128
    PK_F16K_VARIANT(2, 2, 6, 1, true, 5, ""),  // 192 x 64
    PK_F16K_VARIANT(1, 4, 4, 2, true, 5, ""),  // 128 x 64
    PK_F16K_VARIANT(1, 4, 3, 2, true, 5, ""),  // 96 x 64
    PK_F16K_VARIANT(1, 4, 2, 2, true, 5, ""),  // 64 x 64
    PK_F16K_VARIANT(4, 1, 6, 2, true, 2, ""),  // 192 x 256, no K split
    PK_F16K_VARIANT(4, 1, 4, 2, true, 2, ""),  // 128 x 256, no K split
    PK_F16K_VARIANT(4, 1, 3, 2, true, 5, ""),  // 96 x 256, no K split
    PK_F16K_VARIANT(4, 1, 5, 2, true, 2, ""),  // 160 x 256, no K split
};

}  // namespace

int f16k_variant_count() { return (int)(sizeof(kVariants) / sizeof(kVariants[0])); }
const f16::F16Variant& f16k_variant(int index) { return kVariants[index]; }

// Launch of a byte-code tile variant: a 1-D grid of row tiles x column
// tiles; the `single` kernel needs K % 64 == 0 and every tile inside one
// palette group.
hipError_t launch_gemm_f16k(int bits, const f16::F16Variant& v, const GemmArgs& args, hipStream_t stream,
                            hipEvent_t start, hipEvent_t stop) {
  const uint32_t groups = tiles_m(v.shape, args.rows) * tiles_n(v.shape, args.columns);
  if (groups == 0) return hipSuccess;
  const bool single = f16::single_path(v.shape, args);
  if (args.norm_columns) {
    // The fused row norm needs the fixed-palette path and K staged in LDS.
    if (!single || args.inner > kNormMaxInner || !v.normed[bits == 6]) return hipErrorInvalidValue;
    return launch_timed(v.normed[bits == 6], dim3(groups), dim3(v.shape.threads()), stream, start, stop, args);
  }
  void (*kernel)(GemmArgs) = single ? v.single[bits == 6] : v.general[bits == 6];
  if (f16::streams(v, bits, args)) kernel = v.streamed[bits == 6];
  return launch_timed(kernel, dim3(groups), dim3(v.shape.threads()), stream, start, stop, args);
}

}  // namespace pk

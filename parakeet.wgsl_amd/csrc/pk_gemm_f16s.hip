// pk_gemm_f16s.hip - fused palette-weight GEMM for small M (M <= 256, the
// weight-bandwidth-bound shapes): f16 operands, f32 MFMA accumulation,
// operand-order codes, K split over the wavefronts of a workgroup (gfx950,
// wave64). One launch runs one GEMM, or a group of independent GEMMs.
//
// C[m, n] = epilogue(sum_k A[m, k] * LUT[g(n)][code(k, n)])
// (reference: src/webgpu/kernels/gemm.ts:1362-1716, epilogue :2006-2044).
//
// With few rows the work is the weight stream itself: ceil(K*N*bits/8)
// bytes, read once. A workgroup owns CB 32-column blocks and RW 32-row
// blocks; its W wavefronts take the K blocks round robin (wavefront w:
// blocks w, w+W, ...), so every weight byte is fetched by exactly one
// wavefront, as one coalesced 16-byte + one 4/8-byte load per lane and
// column block of the operand-order stream (the package's own bits per
// code, no larger layout). Activation fragments come straight from global
// memory (a few hundred KB, L2-resident); a wavefront reuses each fragment
// for its CB column blocks, so the activation bytes a workgroup pulls from
// L2 are 3.2 * RW / CB times its weight bytes (5-bit). The K loop has no
// LDS tile and no barrier: a wavefront issues the loads of its next K
// block, decodes the current one (shift/mask/v_alignbit per code, palette
// gather from LDS) into MFMA operands and runs the MFMAs. The W partial
// tiles are summed through LDS in wavefront order (deterministic), then
// bias, SiLU/ReLU and residual + scale * value in f32, rounded once, 8-byte
// row stores. v_mfma_f32_32x32x16_f16 computes W^T * A^T with lane half h,
// element t of sub-step s standing for k = 64*kb + 32*h + 8*s + t in both
// operands.
//
// Work order: workgroup b runs on XCD b % 8 (round robin); its work item
// is column group 8 * ((b / 8) / TM) + b % 8 and row group (b / 8) % TM, so
// the TM row groups of one column group run back to back on one XCD and
// read its codes through that XCD's L2.
#include "pk_f16_common.h"

namespace pk {
namespace {

using namespace f16;

// LDS of a variant: the W partial tiles, which during the K loop hold the
// pair table of a one-palette item instead, and the palettes of up to
// CB * 32 / 16 + 2 groups of 64 entries.
template <int W, int RW, int CB>
struct SmallMShared {
  union {
    float4 red[W * CB * RW * 4 * 64];
    uint32_t pairs[64 * 64];
  };
  _Float16 lut[(CB * 2 + 2) * 64];
};

// Byte offset into the pair table of codes u and u + 1 of a lane's 32-code
// stream: 4 * (code(u) | code(u + 1) << BITS), the 2*BITS-bit field at bit
// u*BITS cut out and scaled in two operations.
template <int BITS>
__device__ __forceinline__ uint32_t pair_offset(const uint32_t (&w)[BITS], int u) {
  constexpr uint32_t mask = ((1u << (2 * BITS)) - 1u) << 2;
  const int bit = u * BITS;
  const int word = bit >> 5;
  const int shift = bit & 31;
  if (shift + 2 * BITS <= 32) {
    if (shift >= 2) return (w[word] >> (shift - 2)) & mask;
    return (w[word] << (2 - shift)) & mask;
  }
  return __builtin_amdgcn_alignbit(w[word + 1], w[word], shift - 2) & mask;
}

// The 8 weights of codes 8s..8s+7 as four pair-table gathers: entry
// c0 | c1 << BITS holds LUT[c0] in its low half and LUT[c1] in its high
// half, the layout of two consecutive k of an MFMA operand register.
template <int BITS>
__device__ __forceinline__ half8 decode_pairs(const uint32_t (&w)[BITS], int s, const uint32_t* pairs) {
  uint4 v;
  v.x = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(pairs) + pair_offset<BITS>(w, 8 * s));
  v.y = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(pairs) + pair_offset<BITS>(w, 8 * s + 2));
  v.z = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(pairs) + pair_offset<BITS>(w, 8 * s + 4));
  v.w = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(pairs) + pair_offset<BITS>(w, 8 * s + 6));
  return __builtin_bit_cast(half8, v);
}

// One work item: column group `cg` (CB blocks of 32 columns) and row group
// `mg` (RW blocks of 32 rows) of the GEMM in `args`.
// GENERAL: the columns may span several palette groups (per-lane palette
// base) or K may be 32 (mod 64) (the upper half of the last K block is
// padding: its activation fragments are zeroed).
template <int BITS, int W, int RW, int CB, int D, bool GENERAL>
__device__ __forceinline__ void small_m_item(const GemmArgs& args, uint32_t cg, uint32_t mg,
                                             SmallMShared<W, RW, CB>& sh) {
  constexpr int T = 64 * W;
  constexpr int E = 1 << BITS;
  constexpr uint32_t BW = block_words(BITS);
  constexpr int TILES = CB * RW;

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
  const uint32_t n0 = cg * (uint32_t)(CB * 32);
  const uint32_t m0 = mg * (uint32_t)(RW * 32);

  // Palettes of the item's columns (palette-expander.ts:543-549): groups
  // g_lo..g_hi, at most CB * 32 / CPG + 2 of them (a group is at least one
  // packed group of CPG codes wide). Each thread loads its entries into
  // registers first (clamped, unconditional), so that its later LDS store
  // waits for these loads only and not for the code loads issued after.
  constexpr int CPG = (int)codes_per_group(BITS);
  constexpr int LUT_CAP = GENERAL ? (CB * 32 / CPG + 2) * E : E;
  constexpr int PPT = (LUT_CAP + T - 1) / T;
  static_assert(LUT_CAP <= (CB * 2 + 2) * 64, "palette window exceeds its LDS area");
  const uint32_t gc = args.palette_group_columns;
  const uint32_t G = args.palette_groups;
  const uint32_t g_lo = min(n0 / gc, G - 1u);
  const uint32_t g_hi = GENERAL ? min((min(n0 + (uint32_t)(CB * 32), N) - 1u) / gc, G - 1u) : g_lo;
  const uint32_t entries = (g_hi - g_lo + 1u) * E;
  _Float16 pv[PPT];
  {
    const _Float16* src = static_cast<const _Float16*>(args.palette) + (uint64_t)g_lo * E;
#pragma unroll
    for (int p = 0; p < PPT; ++p) pv[p] = src[min((uint32_t)(tid + p * T), entries - 1u)];
  }
  // Keeps these loads ahead of the code loads (the compiler would otherwise
  // sink them to their LDS store, after every code load).
  asm volatile("" ::: "memory");

  // This wavefront's K blocks: wave, wave + W, ..., `nblocks` of them. Code
  // loads run D blocks ahead of the block being multiplied (D register
  // sets, fixed by unrolling the main loop D times), activation loads one
  // block ahead (two sets): with a few blocks per wavefront most of its
  // code stream is in flight at once. Every load is unconditional, clamped
  // to the wavefront's last block (a wavefront without blocks reads block
  // KB - 1 and never uses it), so the wait counts stay exact.
  const uint32_t nblocks = (uint32_t)wave < KB ? (KB - (uint32_t)wave + W - 1u) / W : 0u;
  const uint32_t last = nblocks ? (uint32_t)wave + (nblocks - 1u) * W : KB - 1u;
  auto block = [&](uint32_t i) { return min((uint32_t)wave + i * W, last); };
  const uint32_t* code_base[CB];
#pragma unroll
  for (int c = 0; c < CB; ++c)
    code_base[c] = args.codes + (uint64_t)min(n0 / 32u + (uint32_t)c, NBT - 1u) * KB * BW;
  auto load_codes = [&](uint32_t kb, uint32_t (&dst)[CB][BITS]) {
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      const uint32_t* blk = code_base[c] + (uint64_t)kb * BW;
      const uint4 p0 = reinterpret_cast<const uint4*>(blk)[lane];
      dst[c][0] = p0.x;
      dst[c][1] = p0.y;
      dst[c][2] = p0.z;
      dst[c][3] = p0.w;
      if constexpr (BITS == 5) {
        dst[c][4] = blk[256 + lane];
      } else {
        const uint2 p1 = reinterpret_cast<const uint2*>(blk + 256)[lane];
        dst[c][4] = p1.x;
        dst[c][5] = p1.y;
      }
    }
  };
  // Activation fragment (m-block mi, sub-step s): row m0 + 32mi + j (rows
  // past M re-read row M-1, never stored), k = 64kb + 32h + 8s. In a
  // K = 32 (mod 64) tail block the upper lane half re-reads k - 32, and
  // the multiply zeroes those fragments (at use, not at load, so no wait).
  const _Float16* a_row[RW];
#pragma unroll
  for (int mi = 0; mi < RW; ++mi)
    a_row[mi] = static_cast<const _Float16*>(args.a) + (uint64_t)min(m0 + (uint32_t)(mi * 32 + j), M - 1u) * K;
  auto padded = [&](uint32_t kb) { return GENERAL && (K & 63u) != 0u && kb + 1u == KB && h; };
  auto load_a = [&](uint32_t kb, half8 (&dst)[RW][4]) {
    const uint32_t k0 = kb * 64u + (uint32_t)(32 * h) - (padded(kb) ? 32u : 0u);
#pragma unroll
    for (int mi = 0; mi < RW; ++mi)
#pragma unroll
      for (int s = 0; s < 4; ++s) dst[mi][s] = *reinterpret_cast<const half8*>(a_row[mi] + k0 + 8u * s);
  };
  uint32_t cr[D][CB][BITS];
  half8 ar[2][RW][4];
#pragma unroll
  for (int d = 0; d < D; ++d) load_codes(block(d), cr[d]);
  load_a(block(0), ar[0]);

#pragma unroll
  for (int p = 0; p < PPT; ++p)
    if ((uint32_t)(tid + p * T) < entries) sh.lut[tid + p * T] = pv[p];
  // One palette (the fixed-palette body): its 2^BITS x 2^BITS pair table.
  if constexpr (!GENERAL) {
    __syncthreads();
    const uint16_t* lut16 = reinterpret_cast<const uint16_t*>(sh.lut);
    for (int p = tid; p < E * E; p += T) sh.pairs[p] = (uint32_t)lut16[p & (E - 1)] | (uint32_t)lut16[p >> BITS] << 16;
  }
  const _Float16* lut[CB];
#pragma unroll
  for (int c = 0; c < CB; ++c) {
    lut[c] = sh.lut;
    if constexpr (GENERAL)
      lut[c] = sh.lut + (min(min(n0 + (uint32_t)(c * 32 + j), N - 1u) / gc, G - 1u) - g_lo) * E;
  }

  floatx16 acc[CB][RW];
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int mi = 0; mi < RW; ++mi)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[c][mi][v] = 0.0f;

  auto multiply = [&](const uint32_t (&cw)[CB][BITS], const half8 (&af)[RW][4], uint32_t kb) {
    const bool pad = padded(kb);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        half8 wf;
        if constexpr (GENERAL)
          wf = decode_fragment<BITS>(cw[c], s, lut[c]);
        else
          wf = decode_pairs<BITS>(cw[c], s, sh.pairs);
#pragma unroll
        for (int mi = 0; mi < RW; ++mi)
          acc[c][mi] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf, pad ? half8{} : af[mi][s], acc[c][mi], 0, 0, 0);
      }
  };

  __syncthreads();  // palettes (and pair table) staged
  // Whole groups of D blocks, then the last nblocks % D (their codes are
  // already loaded).
  uint32_t t = 0;
  for (; t + (uint32_t)D <= nblocks; t += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const uint32_t i = t + (uint32_t)u;
      load_a(block(i + 1u), ar[(u + 1) & 1]);
      multiply(cr[u], ar[u & 1], block(i));
      load_codes(block(i + (uint32_t)D), cr[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < D - 1; ++u) {
    if (t + (uint32_t)u < nblocks) {
      load_a(block(t + (uint32_t)u + 1u), ar[(u + 1) & 1]);
      multiply(cr[u], ar[u & 1], block(t + (uint32_t)u));
    }
  }

  if constexpr (!GENERAL) __syncthreads();  // the partials overwrite the pair table
  // Partials: [wave][tile][quad q][slot] float4, tile = c * RW + mi,
  // slot = lane ^ 2(2q + h), which keeps both the per-lane writes and the
  // row-wise reads on distinct bank groups.
#pragma unroll
  for (int c = 0; c < CB; ++c)
#pragma unroll
    for (int mi = 0; mi < RW; ++mi)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        sh.red[((wave * TILES + c * RW + mi) * 4 + q) * 64 + (lane ^ (2 * (2 * q + h)))] =
            make_float4(acc[c][mi][4 * q], acc[c][mi][4 * q + 1], acc[c][mi][4 * q + 2], acc[c][mi][4 * q + 3]);
  __syncthreads();

  // Unit u: tile u / 256 (column block c, m-block mi), row r = (u / 8) % 32
  // of it, 4 columns 4 * (u % 8); the lane of the MFMA layout holding them
  // is 32 * (cg8 & 1) + r, quad cg8 / 2.
  const _Float16* residual = static_cast<const _Float16*>(args.residual);
  _Float16* out = static_cast<_Float16*>(args.out);
  for (int u = tid; u < TILES * 256; u += T) {
    const int tile = u >> 8, r = (u >> 3) & 31, cg8 = u & 7;
    const int c = tile / RW, mi = tile % RW;
    const int q = cg8 >> 1, hh = cg8 & 1;
    const uint32_t m = m0 + (uint32_t)(mi * 32 + r);
    const uint32_t n = n0 + (uint32_t)(c * 32 + 4 * cg8);
    if (m >= M || n >= N) continue;
    const int slot = (32 * hh + r) ^ (2 * (2 * q + hh));
    float4 sum = sh.red[(tile * 4 + q) * 64 + slot];
#pragma unroll
    for (int w = 1; w < W; ++w) {
      const float4 x = sh.red[((w * TILES + tile) * 4 + q) * 64 + slot];
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

// Work item of workgroup b (see the file comment): false for the padding
// workgroups of the last column groups.
__device__ __forceinline__ bool small_m_work(uint32_t column_groups, uint32_t row_groups, uint32_t& cg,
                                             uint32_t& mg) {
  const uint32_t b = blockIdx.x;
  const uint32_t slot = b / 8u;
  cg = slot / row_groups * 8u + b % 8u;
  mg = slot % row_groups;
  return cg < column_groups;
}

template <int BITS, int W, int RW, int CB, int D, bool GENERAL>
__global__ __launch_bounds__(64 * W) void gemm_f16s_kernel(GemmArgs args) {
  __shared__ SmallMShared<W, RW, CB> sh;
  const uint32_t ncg = ((args.columns + 31u) / 32u + CB - 1u) / CB;
  const uint32_t tm = (args.rows + RW * 32u - 1u) / (RW * 32u);
  uint32_t cg, mg;
  if (!small_m_work(ncg, tm, cg, mg)) return;
  small_m_item<BITS, W, RW, CB, D, GENERAL>(args, cg, mg, sh);
}

// A group: item i of the column-group table names member items[i] >> 16 and
// its column group items[i] & 0xffff. Every member takes the group's rows.
template <int W, int RW, int CB, int D>
__global__ __launch_bounds__(64 * W) void gemm_f16s_group_kernel(SmallMGroupArgs g) {
  __shared__ SmallMShared<W, RW, CB> sh;
  uint32_t i, mg;
  if (!small_m_work(g.items_count, g.row_groups, i, mg)) return;
  const uint32_t item = g.items[i];
  const SmallMMember& member = g.members[item >> 16];
  GemmArgs args = member.args;
  args.rows = g.rows;
  const uint32_t cg = item & 0xffffu;
  // The fixed-palette body needs K % 64 == 0 and the item's columns inside
  // one palette group.
  const bool general = (args.inner & 63u) != 0u ||
                       (args.palette_groups > 1u && args.palette_group_columns % (uint32_t)(CB * 32) != 0u);
  if (member.bits == 5) {
    if (general)
      small_m_item<5, W, RW, CB, D, true>(args, cg, mg, sh);
    else
      small_m_item<5, W, RW, CB, D, false>(args, cg, mg, sh);
  } else {
    if (general)
      small_m_item<6, W, RW, CB, D, true>(args, cg, mg, sh);
    else
      small_m_item<6, W, RW, CB, D, false>(args, cg, mg, sh);
  }
}

struct SmallMVariant {
  F16Variant v;
  void (*group)(SmallMGroupArgs);
  const char* group_name;
};

#define PK_F16S_VARIANT(W, RW, CB, D)                                                                      \
  SmallMVariant {                                                                                          \
    F16Variant{TileShape{1, 1, RW, CB, W}, "pk_gemm_f16s_b5_k" #W "_m" #RW "n" #CB "d" #D,                \
               "pk_gemm_f16s_b6_k" #W "_m" #RW "n" #CB "d" #D,                                             \
               {gemm_f16s_kernel<5, W, RW, CB, D, false>, gemm_f16s_kernel<6, W, RW, CB, D, false>},       \
               {gemm_f16s_kernel<5, W, RW, CB, D, true>, gemm_f16s_kernel<6, W, RW, CB, D, true>},         \
               (uint32_t)sizeof(SmallMShared<W, RW, CB>)},                                                 \
        gemm_f16s_group_kernel<W, RW, CB, D>, "pk_gemm_f16s_group_k" #W "_m" #RW "n" #CB "d" #D            \
  }

// (W, RW, CB, D): K over W wavefronts, RW x CB MFMA blocks per wavefront,
// code loads D K blocks ahead.
const SmallMVariant kVariants[] = {
    PK_F16S_VARIANT(8, 1, 1, 2),  // 32 rows x 32 columns per workgroup
    PK_F16S_VARIANT(8, 2, 1, 2),  // 64 x 32
    PK_F16S_VARIANT(8, 4, 1, 2),  // 128 x 32
    PK_F16S_VARIANT(4, 1, 4, 4),  // 32 x 128
    PK_F16S_VARIANT(4, 2, 2, 4),  // 64 x 64
    PK_F16S_VARIANT(4, 1, 2, 4),  // 32 x 64
};

}  // namespace

int f16s_variant_count() { return (int)(sizeof(kVariants) / sizeof(kVariants[0])); }
const f16::F16Variant& f16s_variant(int index) { return kVariants[index].v; }
const char* f16s_group_name(int index) { return kVariants[index].group_name; }

// One workgroup per (column group, row group), padded to whole rounds of the
// eight XCDs. The `single` kernel needs K % 64 == 0 and the CB * 32
// columns of an item inside one palette group.
hipError_t launch_gemm_f16s(int bits, const f16::F16Variant& v, const GemmArgs& args, hipStream_t stream,
                            hipEvent_t start, hipEvent_t stop) {
  const uint32_t cgs = tiles_n(v.shape, args.columns);
  if (cgs == 0 || args.rows == 0) return hipSuccess;
  const bool single = (args.inner & 63u) == 0u &&
                      (args.palette_groups == 1 || args.palette_group_columns % (uint32_t)v.shape.tile_columns() == 0);
  return launch_timed(single ? v.single[bits == 6] : v.general[bits == 6],
                      dim3(small_m_grid(v.shape, cgs, args.rows)), dim3(v.shape.threads()), stream, start, stop, args);
}

hipError_t launch_gemm_f16s_group(int index, const SmallMGroupArgs& g, hipStream_t stream, hipEvent_t start,
                                  hipEvent_t stop) {
  const SmallMVariant& sv = kVariants[index];
  if (g.items_count == 0 || g.rows == 0) return hipSuccess;
  const dim3 grid(small_m_grid(sv.v.shape, g.items_count, g.rows)), block(sv.v.shape.threads());
  if (start || stop)
    hipExtLaunchKernelGGL(sv.group, grid, block, 0, stream, start, stop, 0, g);
  else
    hipLaunchKernelGGL(sv.group, grid, block, 0, stream, g);
  return hipGetLastError();
}

}  // namespace pk

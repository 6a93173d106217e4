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
#include <atomic>
#include <type_traits>

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

// Work item b (see the file comment): false for the padding items of the
// last column groups. For a fixed b % 8, cg grows with b, so along b, b + G,
// b + 2G, ... (G % 8 == 0) the valid items form a prefix.
__device__ __forceinline__ bool small_m_work_of(uint32_t b, uint32_t column_groups, uint32_t row_groups,
                                                uint32_t& cg, uint32_t& mg) {
  const uint32_t slot = b / 8u;
  cg = slot / row_groups * 8u + b % 8u;
  mg = slot % row_groups;
  return cg < column_groups;
}

__device__ __forceinline__ bool small_m_work(uint32_t column_groups, uint32_t row_groups, uint32_t& cg,
                                             uint32_t& mg) {
  return small_m_work_of(blockIdx.x, column_groups, row_groups, cg, mg);
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

// ---- Persistent group launch ------------------------------------------------
//
// One launch of the group kernel above runs one work item per workgroup:
// each item opens with a full memory round trip (palette, first code
// blocks) and closes with a reduction and epilogue during which its compute
// unit issues no weight loads, and only two workgroups share a compute unit
// (registers and LDS). The persistent form keeps one round of workgroups
// resident and walks the same items: workgroup b runs items b, b + G,
// b + 2G, ... (G, the grid, a multiple of 8, so each item stays on the XCD
// of the one-shot order). While it multiplies an item's last D K blocks it
// issues the next item's palette entry, first D code blocks and first
// activation fragments into the registers those blocks free; each item's
// bias and residual are staged in LDS before its K loop, so that the
// epilogue issues no load (its waits would reach the prefetched ones).
// Same K blocks per wavefront, same MFMA and reduction order: every output
// equals the one-shot kernel's.
//
// Fixed-palette body only; the host runs it when every member has
// K % (64 * W * D) == 0 (each wavefront takes a whole number of groups of
// D blocks) and an item's columns inside one palette group.

// The uniform values of one work item. Its pointers are read from the
// member table after the kernel's own stores, where the compiler can no
// longer infer that they address global memory: they are declared so
// (global loads and stores, not flat ones, which would also count against
// the LDS wait counter).
template <typename T>
using global_ptr = __attribute__((address_space(1))) T*;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct StreamItem {
  global_ptr<const uint32_t> codes;
  global_ptr<const _Float16> palette;  // the item's palette group
  global_ptr<const _Float16> a;
  global_ptr<const float> bias;
  global_ptr<const _Float16> residual;
  global_ptr<_Float16> out;
  float residual_scale;
  int activation;
  int bits;
  uint32_t K, N, KB, NBT, n0, m0;
};

// Uniform values read after the kernel's own stores come back in vector
// registers (the loads cannot be proven free of them); these move them to
// scalar registers.
__device__ __forceinline__ uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float uniform(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(uint32_t, v)));
}
template <typename T>
__device__ __forceinline__ global_ptr<T> uniform_global(const void* p) {
  const uint64_t v = (uint64_t)p;
  return (global_ptr<T>)((uint64_t)uniform((uint32_t)(v >> 32)) << 32 | uniform((uint32_t)v));
}

template <int RW, int CB>
__device__ __forceinline__ StreamItem stream_item(const SmallMGroupArgs& g, uint32_t i, uint32_t mg) {
  const uint32_t item = uniform(g.items[i]);
  const SmallMMember& member = g.members[item >> 16];
  const GemmArgs& m = member.args;
  StreamItem s;
  s.bits = (int)uniform((uint32_t)member.bits);
  s.K = uniform(m.inner);
  s.N = uniform(m.columns);
  s.KB = s.K / 64u;
  s.NBT = (s.N + 31u) / 32u;
  s.n0 = (item & 0xffffu) * (uint32_t)(CB * 32);
  s.m0 = mg * (uint32_t)(RW * 32);
  s.codes = uniform_global<const uint32_t>(m.codes);
  const uint32_t group = min(s.n0 / uniform(m.palette_group_columns), uniform(m.palette_groups) - 1u);
  s.palette = uniform_global<const _Float16>(m.palette) + (uint64_t)group * (1u << s.bits);
  s.a = uniform_global<const _Float16>(m.a);
  s.bias = uniform_global<const float>(m.bias);
  s.residual = uniform_global<const _Float16>(m.residual);
  s.out = uniform_global<_Float16>(m.out);
  s.residual_scale = uniform(m.residual_scale);
  s.activation = (int)uniform((uint32_t)m.activation);
  return s;
}

// LDS of the persistent kernel: the one-shot kernel's, plus the item's
// residual (one 8-byte slot per epilogue unit, written and read by the same
// thread) and bias (its CB * 32 columns).
template <int W, int RW, int CB>
struct StreamShared : SmallMShared<W, RW, CB> {
  u32x2 residual[CB * RW * 256];
  f32x4 bias[CB * 8];
};

// OCC: the waves per SIMD its registers must allow (compiler target).
template <int W, int RW, int CB, int D, int OCC>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void gemm_f16s_stream_kernel(
    SmallMGroupArgs g) {
  __shared__ StreamShared<W, RW, CB> sh;
  constexpr int T = 64 * W;
  constexpr int TILES = CB * RW;
  constexpr int U = TILES * 256 / T;  // epilogue units per thread
  static_assert(TILES * 256 % T == 0, "epilogue units per thread");
  static_assert(CB * 8 <= T, "one thread per bias vector");
  static_assert(D % 2 == 0, "block i multiplies activation set i % 2 across items");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31;
  const int h = lane >> 5;
  const uint32_t M = g.rows;

  uint32_t b = blockIdx.x, i, mg;
  if (!small_m_work_of(b, g.items_count, g.row_groups, i, mg)) return;
  StreamItem cur = stream_item<RW, CB>(g, i, mg);

  // Loads of item s, wavefront block q (K block wave + q * W). Both code
  // widths issue the same three loads per column block (a 6-bit block's
  // last two words per lane, a 5-bit block's last word twice), so the
  // count of loads in flight does not depend on the items' widths.
  auto load_codes = [&](const StreamItem& s, uint32_t q, uint32_t (&dst)[CB][6]) {
    const uint32_t kb = (uint32_t)wave + q * (uint32_t)W;
    const uint32_t bw = s.bits == 5 ? block_words(5) : block_words(6);
    const uint32_t x = s.bits == 5 ? 256u + (uint32_t)lane : 256u + 2u * (uint32_t)lane;
    const uint32_t y = s.bits == 5 ? x : x + 1u;
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      const global_ptr<const uint32_t> blk = s.codes + ((uint64_t)min(s.n0 / 32u + (uint32_t)c, s.NBT - 1u) * s.KB + kb) * bw;
      const u32x4 p0 = ((global_ptr<const u32x4>)blk)[lane];
      dst[c][0] = p0.x;
      dst[c][1] = p0.y;
      dst[c][2] = p0.z;
      dst[c][3] = p0.w;
      dst[c][4] = blk[x];
      dst[c][5] = blk[y];
    }
  };
  auto load_a = [&](const StreamItem& s, uint32_t q, half8 (&dst)[RW][4]) {
    const uint32_t k0 = ((uint32_t)wave + q * (uint32_t)W) * 64u + (uint32_t)(32 * h);
#pragma unroll
    for (int mi = 0; mi < RW; ++mi) {
      const global_ptr<const _Float16> row = s.a + (uint64_t)min(s.m0 + (uint32_t)(mi * 32 + j), M - 1u) * s.K + k0;
#pragma unroll
      for (int t = 0; t < 4; ++t) dst[mi][t] = *(global_ptr<const half8>)(row + 8 * t);
    }
  };
  auto load_palette = [&](const StreamItem& s) { return s.palette[min((uint32_t)tid, (1u << s.bits) - 1u)]; };
  auto stage_palette = [&](const StreamItem& s, _Float16 v) {
    if ((uint32_t)tid < (1u << s.bits)) sh.lut[tid] = v;
  };

  uint32_t cr[D][CB][6];
  half8 ar[2][RW][4];
  floatx16 acc[CB][RW];

  _Float16 pv = load_palette(cur);
  asm volatile("" ::: "memory");
#pragma unroll
  for (int d = 0; d < D; ++d) load_codes(cur, (uint32_t)d, cr[d]);
  load_a(cur, 0, ar[0]);
  stage_palette(cur, pv);

  for (;;) {
    // The thread index as a value of this item only: addresses derived from
    // it for the pair table, staging, partials and epilogue are recomputed
    // per item instead of being held in registers across the K loop.
    int it = tid;
    asm volatile("" : "+v"(it));
    const int ilane = it & 63;
    const int ih = ilane >> 5;
    const uint32_t nb = b + gridDim.x;
    uint32_t ni, nmg;
    const bool more = small_m_work_of(nb, g.items_count, g.row_groups, ni, nmg);
    const StreamItem nxt = more ? stream_item<RW, CB>(g, ni, nmg) : cur;

    __syncthreads();  // the item's palette staged; the last item's partials read
    {
      const uint16_t* lut16 = reinterpret_cast<const uint16_t*>(sh.lut);
      if (cur.bits == 5) {
        for (int p = it; p < 32 * 32; p += T) sh.pairs[p] = (uint32_t)lut16[p & 31] | (uint32_t)lut16[p >> 5] << 16;
      } else {
        for (int p = it; p < 64 * 64; p += T) sh.pairs[p] = (uint32_t)lut16[p & 63] | (uint32_t)lut16[p >> 6] << 16;
      }
    }
    // The item's epilogue operands, staged while its first code blocks are
    // still arriving (these loads wait for them, which its first multiply
    // does anyway).
    // (Clamped loads, all issued before the first store.)
    if (cur.residual) {
      u32x2 rv[U];
#pragma unroll
      for (int q = 0; q < U; ++q) {
        const int u = it + q * T;
        const int tile = u >> 8, r = (u >> 3) & 31, cg8 = u & 7;
        const uint32_t m = min(cur.m0 + (uint32_t)((tile % RW) * 32 + r), M - 1u);
        const uint32_t n = min(cur.n0 + (uint32_t)((tile / RW) * 32 + 4 * cg8), cur.N - 4u);
        rv[q] = *(global_ptr<const u32x2>)(cur.residual + (uint64_t)m * cur.N + n);
      }
#pragma unroll
      for (int q = 0; q < U; ++q) sh.residual[it + q * T] = rv[q];
    }
    if (cur.bias && it < CB * 8)
      sh.bias[it] = *(global_ptr<const f32x4>)(cur.bias + min(cur.n0 + 4u * (uint32_t)it, cur.N - 4u));
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int mi = 0; mi < RW; ++mi)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[c][mi][v] = 0.0f;
    __syncthreads();  // pair table built

    // The code width only changes the decode: one K loop (its loads, and
    // the registers the next item's loads land in, are the same for both),
    // a uniform branch around each block's decode and MFMAs.
    auto multiply_bits = [&](auto width, const uint32_t (&cw)[CB][6], const half8 (&af)[RW][4]) {
      constexpr int BITS = decltype(width)::value;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int c = 0; c < CB; ++c) {
          const half8 wf = decode_pairs<BITS>(*reinterpret_cast<const uint32_t(*)[BITS]>(cw[c]), s, sh.pairs);
#pragma unroll
          for (int mi = 0; mi < RW; ++mi)
            acc[c][mi] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf, af[mi][s], acc[c][mi], 0, 0, 0);
        }
    };
    auto multiply = [&](const uint32_t (&cw)[CB][6], const half8 (&af)[RW][4]) {
      if (cur.bits == 5)
        multiply_bits(std::integral_constant<int, 5>{}, cw, af);
      else
        multiply_bits(std::integral_constant<int, 6>{}, cw, af);
    };
    // Groups of D blocks. Each issues the same loads: the next block's
    // activation fragments and the codes D blocks ahead, which in the
    // item's last group are the next item's first block and first D
    // blocks (and the palette entry, loaded by every group, is the next
    // item's); the item of each load is a uniform select.
    const uint32_t nblocks = cur.KB / (uint32_t)W;
    for (uint32_t t = 0; t < nblocks; t += (uint32_t)D) {
      const bool last = t + (uint32_t)D >= nblocks;
      const StreamItem& ahead = last ? nxt : cur;
      const uint32_t ahead_block = last ? 0u : t + (uint32_t)D;
      pv = load_palette(ahead);
#pragma unroll
      for (int u = 0; u < D; ++u) {
        if (u + 1 < D)
          load_a(cur, t + (uint32_t)u + 1u, ar[(u + 1) & 1]);
        else
          load_a(ahead, ahead_block, ar[0]);
        multiply(cr[u], ar[u & 1]);
        load_codes(ahead, ahead_block + (uint32_t)u, cr[u]);
      }
    }
    // The palette area was last read by this item's pair table build (before
    // the barrier ahead of the K loop): the next item's entries go in now.
    if ((uint32_t)it < (1u << nxt.bits)) sh.lut[it] = pv;

    __syncthreads();  // the partials overwrite the pair table
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
      for (int mi = 0; mi < RW; ++mi)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          sh.red[((wave * TILES + c * RW + mi) * 4 + q) * 64 + (ilane ^ (2 * (2 * q + ih)))] =
              make_float4(acc[c][mi][4 * q], acc[c][mi][4 * q + 1], acc[c][mi][4 * q + 2], acc[c][mi][4 * q + 3]);
    __syncthreads();

#pragma unroll
    for (int q = 0; q < U; ++q) {
      const int u = it + q * T;
      const int tile = u >> 8, r = (u >> 3) & 31, cg8 = u & 7;
      const int qq = cg8 >> 1, hh = cg8 & 1;
      const uint32_t m = cur.m0 + (uint32_t)((tile % RW) * 32 + r);
      const uint32_t n = cur.n0 + (uint32_t)((tile / RW) * 32 + 4 * cg8);
      if (m >= M || n >= cur.N) continue;
      const int slot = (32 * hh + r) ^ (2 * (2 * qq + hh));
      float4 sum = sh.red[(tile * 4 + qq) * 64 + slot];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        const float4 x = sh.red[((w * TILES + tile) * 4 + qq) * 64 + slot];
        sum.x += x.x;
        sum.y += x.y;
        sum.z += x.z;
        sum.w += x.w;
      }
      float v[4] = {sum.x, sum.y, sum.z, sum.w};
      if (cur.bias) {
        const f32x4 bv = sh.bias[(tile / RW) * 8 + cg8];
        v[0] += bv.x;
        v[1] += bv.y;
        v[2] += bv.z;
        v[3] += bv.w;
      }
      if (cur.activation == kActSilu) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = silu(v[e]);
      } else if (cur.activation == kActRelu) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = fmaxf(v[e], 0.0f);
      }
      if (cur.residual) {
        const u32x2 rb = sh.residual[u];
        const float sc = cur.residual_scale;
        v[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.x & 0xffffu)) + sc * v[0];
        v[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.x >> 16)) + sc * v[1];
        v[2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.y & 0xffffu)) + sc * v[2];
        v[3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(rb.y >> 16)) + sc * v[3];
      }
      *(global_ptr<u32x2>)(cur.out + (uint64_t)m * cur.N + n) = u32x2{pack_half2(v[0], v[1]), pack_half2(v[2], v[3])};
    }
    if (!more) break;
    cur = nxt;
    b = nb;
  }
}

struct SmallMVariant {
  F16Variant v;
  void (*group)(SmallMGroupArgs);
  const char* group_name;
  // The persistent form of the group launch (null: one-shot only).
  void (*stream)(SmallMGroupArgs);
  const char* stream_name;
  int k_waves, blocks_ahead;
};

#define PK_F16S_SHAPE(W, RW, CB, D)                                                                          \
  F16Variant {                                                                                             \
    TileShape{1, 1, RW, CB, W}, "pk_gemm_f16s_b5_k" #W "_m" #RW "n" #CB "d" #D,                           \
        "pk_gemm_f16s_b6_k" #W "_m" #RW "n" #CB "d" #D,                                                    \
        {gemm_f16s_kernel<5, W, RW, CB, D, false>, gemm_f16s_kernel<6, W, RW, CB, D, false>},               \
        {gemm_f16s_kernel<5, W, RW, CB, D, true>, gemm_f16s_kernel<6, W, RW, CB, D, true>},                 \
        (uint32_t)sizeof(SmallMShared<W, RW, CB>)                                                          \
  }
#define PK_F16S_VARIANT(W, RW, CB, D)                                                                      \
  SmallMVariant {                                                                                          \
    PK_F16S_SHAPE(W, RW, CB, D), gemm_f16s_group_kernel<W, RW, CB, D>,                                    \
        "pk_gemm_f16s_group_k" #W "_m" #RW "n" #CB "d" #D, nullptr, nullptr, W, D                          \
  }
// A persistent group variant: the single launches and the fallback group
// launch are those of the one-shot variant of the same shape.
#define PK_F16S_STREAM_VARIANT(W, RW, CB, D, OCC)                                                          \
  SmallMVariant {                                                                                          \
    PK_F16S_SHAPE(W, RW, CB, D), gemm_f16s_group_kernel<W, RW, CB, D>,                                    \
        "pk_gemm_f16s_group_k" #W "_m" #RW "n" #CB "d" #D, gemm_f16s_stream_kernel<W, RW, CB, D, OCC>,    \
        "pk_gemm_f16s_stream_k" #W "_m" #RW "n" #CB "d" #D "o" #OCC, W, D                                 \
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
    // Persistent forms (W, RW, CB, D, waves per SIMD). 32 x 128 loads codes
    // two blocks ahead: at four a wavefront needs more than the 256
    // registers of two waves per SIMD.
    PK_F16S_STREAM_VARIANT(4, 1, 4, 2, 2),  // 32 x 128
    PK_F16S_STREAM_VARIANT(4, 2, 2, 2, 2),  // 64 x 64
    PK_F16S_STREAM_VARIANT(4, 1, 2, 2, 3),  // 32 x 64
    PK_F16S_STREAM_VARIANT(4, 1, 2, 4, 2),  // 32 x 64
};
constexpr int kVariantCount = (int)(sizeof(kVariants) / sizeof(kVariants[0]));

// Workgroups of the persistent kernel of variant `index` that fit on the
// current device at once, rounded down to whole rounds of the eight XCDs
// (0 if the runtime cannot say); asked once per device and variant.
uint32_t stream_capacity(int index) {
  constexpr int kDevices = 64;
  static std::atomic<uint32_t> cache[kDevices][kVariantCount];
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kDevices) return 0;
  uint32_t cap = cache[device][index].load(std::memory_order_relaxed);
  if (cap) return cap;
  int blocks = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kVariants[index].stream,
                                                   (int)kVariants[index].v.shape.threads(), 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return 0;
  cap = (uint32_t)(blocks * cus) / 8u * 8u;
  cache[device][index].store(cap, std::memory_order_relaxed);
  return cap;
}

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

bool f16s_group_persistent(int index) { return kVariants[index].stream != nullptr; }

bool f16s_group_streams(int index, uint32_t inner, uint32_t palette_groups, uint32_t palette_group_columns) {
  const SmallMVariant& sv = kVariants[index];
  if (!sv.stream) return false;
  const uint32_t span = 64u * (uint32_t)(sv.k_waves * sv.blocks_ahead);
  return inner % span == 0u && (palette_groups == 1u || palette_group_columns % sv.v.shape.tile_columns() == 0u);
}

// The kernel and grid a group launch runs: the persistent kernel on at most
// one round of resident workgroups when the variant has one and the host
// set g.persistent (every member eligible), else one workgroup per item.
uint32_t f16s_group_launch(int index, const SmallMGroupArgs& g, void (**kernel)(SmallMGroupArgs), const char** name) {
  const SmallMVariant& sv = kVariants[index];
  const uint32_t items = small_m_grid(sv.v.shape, g.items_count, g.rows);
  if (sv.stream && g.persistent) {
    const uint32_t resident = stream_capacity(index);
    if (resident) {
      *kernel = sv.stream;
      *name = sv.stream_name;
      return min(items, resident);
    }
  }
  *kernel = sv.group;
  *name = sv.group_name;
  return items;
}

hipError_t launch_gemm_f16s_group(int index, const SmallMGroupArgs& g, hipStream_t stream, hipEvent_t start,
                                  hipEvent_t stop) {
  if (g.items_count == 0 || g.rows == 0) return hipSuccess;
  void (*kernel)(SmallMGroupArgs) = nullptr;
  const char* name = nullptr;
  const dim3 grid(f16s_group_launch(index, g, &kernel, &name)), block(kVariants[index].v.shape.threads());
  if (start || stop)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0, g);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, g);
  return hipGetLastError();
}

}  // namespace pk

// pk_codes.hip - packed palette code kernels for gfx950: bit-exact unpack,
// the reference-compatible dense expander and the one-time conversion of a
// reference-format weight into the MFMA operand order read by the fused GEMM.
#include "pk_internal.h"

namespace pk {
namespace {

constexpr int kThreads = 256;

// Code i of a reference group: ((w[b/32] >> b%32) | (w[b/32+1] << (32-b%32)))
// & mask with b = i*bits, computed on u32 (src/model/palette-expander.ts:500-511).
template <int BITS>
__device__ __forceinline__ uint32_t group_code(const uint32_t* w, int i) {
  const int bit = i * BITS;
  const int word = bit >> 5;
  const int shift = bit & 31;
  uint32_t value = w[word] >> shift;
  if (shift + BITS > 32) value |= w[word + 1] << (32 - shift);
  return value & ((1u << BITS) - 1u);
}

template <int BITS>
__global__ __launch_bounds__(kThreads) void unpack_kernel(const uint32_t* __restrict__ words,
                                                          uint64_t groups,
                                                          uint8_t* __restrict__ codes) {
  constexpr int CPG = (int)codes_per_group(BITS);
  constexpr int WPG = (int)words_per_group(BITS);
  const uint64_t g = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (g >= groups) return;
  uint32_t w[WPG + 1];
#pragma unroll
  for (int i = 0; i < WPG; ++i) w[i] = words[g * WPG + i];
  w[WPG] = 0;
  uint32_t packed[CPG / 4];
#pragma unroll
  for (int i = 0; i < CPG / 4; ++i) packed[i] = 0;
#pragma unroll
  for (int i = 0; i < CPG; ++i) packed[i / 4] |= group_code<BITS>(w, i) << (8 * (i % 4));
  uint4* dst = reinterpret_cast<uint4*>(codes + g * CPG);
#pragma unroll
  for (int v = 0; v < CPG / 16; ++v)
    dst[v] = make_uint4(packed[4 * v], packed[4 * v + 1], packed[4 * v + 2], packed[4 * v + 3]);
}

// Tile-major scratch index (src/model/runtime-plan.ts:454-490).
__device__ __forceinline__ uint64_t tile_major_index(uint64_t scalar, uint32_t inner,
                                                     uint32_t columns, uint32_t tile_columns) {
  const uint64_t k = scalar / columns;
  const uint64_t n = scalar % columns;
  const uint64_t k_tiles = inner / 32u;
  return (((n / tile_columns) * k_tiles + k / 32u) * 32u + k % 32u) * tile_columns +
         n % tile_columns;
}

// One thread per code group, like paletteDequantWgslForScalar
// (palette-expander.ts:573-585): palette group from the group's first
// scalar, one LUT gather per code, dense row-major or tile-major stores.
template <int BITS, typename T, bool TILE>
__global__ __launch_bounds__(kThreads) void expand_kernel(
    const uint32_t* __restrict__ packed, uint64_t scalar_count, uint32_t inner,
    uint32_t columns, uint32_t group_columns, uint32_t groups,
    const T* __restrict__ palette, T* __restrict__ target) {
  constexpr int CPG = (int)codes_per_group(BITS);
  constexpr int WPG = (int)words_per_group(BITS);
  constexpr uint32_t kEntries = 1u << BITS;
  constexpr uint32_t kTileColumns = sizeof(T) == 2 ? 256u : 128u;
  const uint64_t g = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  const uint64_t scalar_base = g * CPG;
  if (scalar_base >= scalar_count) return;
  uint32_t w[WPG + 1];
#pragma unroll
  for (int i = 0; i < WPG; ++i) w[i] = packed[g * WPG + i];
  w[WPG] = 0;
  const uint32_t column = (uint32_t)(scalar_base % columns);
  const uint32_t pg = min(column / group_columns, groups - 1u);
  const T* lut = palette + (uint64_t)pg * kEntries;
#pragma unroll
  for (int v = 0; v < CPG / 4; ++v) {
    T values[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) values[c] = lut[group_code<BITS>(w, 4 * v + c)];
    const uint64_t first = scalar_base + 4u * v;
    const uint64_t dst = TILE ? tile_major_index(first, inner, columns, kTileColumns) : first;
    if constexpr (sizeof(T) == 2) {
      uint2 bits;
      bits.x = (uint32_t)__builtin_bit_cast(uint16_t, values[0]) |
               ((uint32_t)__builtin_bit_cast(uint16_t, values[1]) << 16);
      bits.y = (uint32_t)__builtin_bit_cast(uint16_t, values[2]) |
               ((uint32_t)__builtin_bit_cast(uint16_t, values[3]) << 16);
      *reinterpret_cast<uint2*>(target + dst) = bits;
    } else {
      *reinterpret_cast<float4*>(target + dst) = make_float4(values[0], values[1], values[2], values[3]);
    }
  }
}

// A lane's 32 codes into its words of a block in the P-part layout
// (pk_internal.h): P = 1 packs them LSB-first into BITS words (words 0-3
// lane-interleaved as plane 0, the rest as plane 1); P = 2 or 4 stores the
// 16-bit pair slots 4 * (c0 | c1 << BITS) of part p at [p][lane].
template <int BITS, int P>
__device__ __forceinline__ void store_lane_codes(const uint32_t (&code)[32], uint32_t* base, uint32_t lane) {
  constexpr uint32_t PW = parts_words(BITS, P);
  constexpr int PER = 32 / P;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    uint32_t w[PW + 1];
#pragma unroll
    for (uint32_t q = 0; q <= PW; ++q) w[q] = 0;
    if constexpr (P > 1) {
#pragma unroll
      for (int e = 0; e < PER / 2; ++e)
        w[e >> 1] |= (4u * (code[p * PER + 2 * e] | (code[p * PER + 2 * e + 1] << BITS))) << (16 * (e & 1));
    } else {
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const uint32_t b = (uint32_t)u * BITS;
        w[b >> 5] |= code[p * PER + u] << (b & 31u);
        if ((b & 31u) + BITS > 32u) w[(b >> 5) + 1] |= code[p * PER + u] >> (32u - (b & 31u));
      }
    }
    if constexpr (P == 1) {
      reinterpret_cast<uint4*>(base)[lane] = make_uint4(w[0], w[1], w[2], w[3]);
      if constexpr (BITS == 5)
        base[256 + lane] = w[4];
      else
        reinterpret_cast<uint2*>(base + 256)[lane] = make_uint2(w[4], w[5]);
    } else {
      uint32_t* dst = base + ((uint64_t)p * 64u + lane) * PW;
#pragma unroll
      for (uint32_t q = 0; q < PW; ++q) dst[q] = w[q];
    }
  }
}

// The inverse: a lane's 32 codes from its words of a block.
template <int BITS, int P>
__device__ __forceinline__ void load_lane_codes(const uint32_t* base, uint32_t lane, uint32_t (&code)[32]) {
  constexpr uint32_t PW = parts_words(BITS, P);
  constexpr int PER = 32 / P;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    uint32_t w[PW + 1];
    if constexpr (P == 1) {
      const uint4 v = reinterpret_cast<const uint4*>(base)[lane];
      w[0] = v.x;
      w[1] = v.y;
      w[2] = v.z;
      w[3] = v.w;
      if constexpr (BITS == 5) {
        w[4] = base[256 + lane];
      } else {
        const uint2 x = reinterpret_cast<const uint2*>(base + 256)[lane];
        w[4] = x.x;
        w[5] = x.y;
      }
    } else {
      const uint32_t* src = base + ((uint64_t)p * 64u + lane) * PW;
#pragma unroll
      for (uint32_t q = 0; q < PW; ++q) w[q] = src[q];
    }
    w[PW] = 0;
    if constexpr (P > 1) {
#pragma unroll
      for (int e = 0; e < PER / 2; ++e) {
        const uint32_t field = ((w[e >> 1] >> (16 * (e & 1))) & 0xffffu) >> 2;
        code[p * PER + 2 * e] = field & ((1u << BITS) - 1u);
        code[p * PER + 2 * e + 1] = field >> BITS;
      }
    } else {
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const uint32_t b = (uint32_t)u * BITS;
        uint32_t v = w[b >> 5] >> (b & 31u);
        if ((b & 31u) + BITS > 32u) v |= w[(b >> 5) + 1] << (32u - (b & 31u));
        code[p * PER + u] = v & ((1u << BITS) - 1u);
      }
    }
  }
}

// Reference format -> MFMA operand order with P parts (layout in
// pk_internal.h). One thread per (block, lane); runs once per weight. With
// glu_interleave the physical column blocks alternate the two halves of the
// logical columns (GLU values, then their gates).
template <int BITS, int P>
__global__ __launch_bounds__(kThreads) void operand_order_kernel(
    const uint32_t* __restrict__ packed, uint32_t inner, uint32_t columns,
    uint32_t k_blocks, uint64_t total_lanes, uint32_t* __restrict__ out, bool glu_interleave) {
  constexpr uint32_t CPG = codes_per_group(BITS);
  constexpr uint32_t WPG = words_per_group(BITS);
  const uint64_t t = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= total_lanes) return;
  const uint32_t lane = (uint32_t)(t & 63u);
  const uint64_t block = t >> 6;
  const uint32_t nb = (uint32_t)(block / k_blocks);
  const uint32_t kb = (uint32_t)(block % k_blocks);
  const uint32_t logical_nb = glu_interleave ? (nb & 1u) * (columns / 64u) + (nb >> 1) : nb;
  const uint32_t n = logical_nb * 32u + (lane & 31u);
  const uint32_t k0 = kb * 64u + (lane >> 5) * 32u;
  uint32_t code[32];
#pragma unroll
  for (uint32_t u = 0; u < 32u; ++u) {
    const uint32_t k = k0 + u;
    code[u] = 0;
    if (k < inner && n < columns) {
      const uint64_t scalar = (uint64_t)k * columns + n;
      const uint64_t g = scalar / CPG;
      const uint32_t bit = (uint32_t)(scalar % CPG) * BITS;
      const uint32_t word = bit >> 5, shift = bit & 31u;
      uint32_t value = packed[g * WPG + word] >> shift;
      if (shift + BITS > 32u) value |= packed[g * WPG + word + 1] << (32u - shift);
      code[u] = value & ((1u << BITS) - 1u);
    }
  }
  store_lane_codes<BITS, P>(code, out + block * block_words(BITS, P), lane);
}

// One P-part layout -> another, one thread per (block, lane).
template <int BITS, int PS, int PD>
__global__ __launch_bounds__(kThreads) void relayout_kernel(const uint32_t* __restrict__ src,
                                                            uint32_t* __restrict__ dst, uint64_t total_lanes) {
  const uint64_t t = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= total_lanes) return;
  const uint32_t lane = (uint32_t)(t & 63u);
  const uint64_t block = t >> 6;
  uint32_t code[32];
  load_lane_codes<BITS, PS>(src + block * block_words(BITS, PS), lane, code);
  store_lane_codes<BITS, PD>(code, dst + block * block_words(BITS, PD), lane);
}

inline dim3 grid_for(uint64_t items) {
  return dim3((unsigned)((items + kThreads - 1) / kThreads));
}

}  // namespace

hipError_t launch_unpack(int bits, const uint32_t* words, uint64_t groups,
                         uint8_t* codes, hipStream_t stream) {
  if (groups == 0) return hipSuccess;
  if (bits == 5)
    hipLaunchKernelGGL(unpack_kernel<5>, grid_for(groups), dim3(kThreads), 0, stream, words, groups, codes);
  else
    hipLaunchKernelGGL(unpack_kernel<6>, grid_for(groups), dim3(kThreads), 0, stream, words, groups, codes);
  return hipGetLastError();
}

template <int BITS, typename T>
static void launch_expand_typed(bool tile_major, const uint32_t* packed, uint32_t inner,
                                uint32_t columns, uint32_t group_columns, uint32_t groups,
                                const void* palette, void* target, hipStream_t stream) {
  const uint64_t scalars = (uint64_t)inner * columns;
  const uint64_t code_groups = scalars / codes_per_group(BITS);
  const dim3 grid = grid_for(code_groups);
  if (tile_major)
    hipLaunchKernelGGL((expand_kernel<BITS, T, true>), grid, dim3(kThreads), 0, stream, packed,
                       scalars, inner, columns, group_columns, groups,
                       static_cast<const T*>(palette), static_cast<T*>(target));
  else
    hipLaunchKernelGGL((expand_kernel<BITS, T, false>), grid, dim3(kThreads), 0, stream, packed,
                       scalars, inner, columns, group_columns, groups,
                       static_cast<const T*>(palette), static_cast<T*>(target));
}

hipError_t launch_expand(int bits, bool f16, bool tile_major, const uint32_t* packed,
                         uint32_t inner, uint32_t columns, uint32_t group_columns,
                         uint32_t groups, const void* palette, void* target,
                         hipStream_t stream) {
  if (bits == 5) {
    if (f16)
      launch_expand_typed<5, _Float16>(tile_major, packed, inner, columns, group_columns, groups, palette, target, stream);
    else
      launch_expand_typed<5, float>(tile_major, packed, inner, columns, group_columns, groups, palette, target, stream);
  } else {
    if (f16)
      launch_expand_typed<6, _Float16>(tile_major, packed, inner, columns, group_columns, groups, palette, target, stream);
    else
      launch_expand_typed<6, float>(tile_major, packed, inner, columns, group_columns, groups, palette, target, stream);
  }
  return hipGetLastError();
}

hipError_t launch_to_operand_order(int bits, const uint32_t* packed, uint32_t inner,
                                   uint32_t columns, uint32_t* codes, hipStream_t stream, bool glu_interleave,
                                   int parts) {
  if (glu_interleave && columns % 64u != 0) return hipErrorInvalidValue;
  if (bits != 5 && bits != 6) return hipErrorInvalidValue;
  const uint32_t k_blocks = padded_inner(inner) / 64u;
  const uint64_t blocks = (uint64_t)(padded_columns(columns) / 32u) * k_blocks;
  const uint64_t lanes = blocks * 64u;
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid_for(lanes), dim3(kThreads), 0, stream, packed, inner, columns, k_blocks, lanes,
                       codes, glu_interleave);
  };
  switch (parts * 10 + bits) {
    case 15: go(operand_order_kernel<5, 1>); break;
    case 16: go(operand_order_kernel<6, 1>); break;
    case 25: go(operand_order_kernel<5, 2>); break;
    case 26: go(operand_order_kernel<6, 2>); break;
    case 45: go(operand_order_kernel<5, 4>); break;
    case 46: go(operand_order_kernel<6, 4>); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

namespace {
template <int BITS, int PS>
hipError_t relayout_from(const uint32_t* src, uint32_t* dst, int dst_parts, uint64_t lanes, hipStream_t stream) {
  switch (dst_parts) {
    case 1: hipLaunchKernelGGL((relayout_kernel<BITS, PS, 1>), grid_for(lanes), dim3(kThreads), 0, stream, src, dst, lanes); break;
    case 2: hipLaunchKernelGGL((relayout_kernel<BITS, PS, 2>), grid_for(lanes), dim3(kThreads), 0, stream, src, dst, lanes); break;
    case 4: hipLaunchKernelGGL((relayout_kernel<BITS, PS, 4>), grid_for(lanes), dim3(kThreads), 0, stream, src, dst, lanes); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
template <int BITS>
hipError_t relayout_bits(const uint32_t* src, int src_parts, uint32_t* dst, int dst_parts, uint64_t lanes,
                         hipStream_t stream) {
  switch (src_parts) {
    case 1: return relayout_from<BITS, 1>(src, dst, dst_parts, lanes, stream);
    case 2: return relayout_from<BITS, 2>(src, dst, dst_parts, lanes, stream);
    case 4: return relayout_from<BITS, 4>(src, dst, dst_parts, lanes, stream);
    default: return hipErrorInvalidValue;
  }
}
}  // namespace

hipError_t launch_relayout(int bits, const uint32_t* src, int src_parts, uint32_t* dst, int dst_parts,
                           uint64_t blocks, hipStream_t stream) {
  const uint64_t lanes = blocks * 64u;
  if (lanes == 0) return hipSuccess;
  if (bits == 5) return relayout_bits<5>(src, src_parts, dst, dst_parts, lanes, stream);
  if (bits == 6) return relayout_bits<6>(src, src_parts, dst, dst_parts, lanes, stream);
  return hipErrorInvalidValue;
}

namespace {

// Fused row LayerNorm preparation of one weight: gamma16[k] = f16(gamma[k])
// and, per column n, G_n = sum_k f16(gamma_k) W_kn and B_n = sum_k beta_k W_kn
// in k order (f32), W_kn = LUT[g(n)][code(k, n)] from the reference-format
// codes (flat index k * N + n).
template <int BITS>
__global__ __launch_bounds__(kThreads) void norm_prepare_kernel(const uint32_t* __restrict__ packed, uint32_t inner,
                                                               uint32_t columns, uint32_t group_columns,
                                                               uint32_t groups, const _Float16* __restrict__ palette,
                                                               const float* __restrict__ gamma,
                                                               const float* __restrict__ beta,
                                                               _Float16* __restrict__ gamma16, float* __restrict__ sums) {
  constexpr uint32_t CPG = codes_per_group(BITS);
  constexpr uint32_t WPG = words_per_group(BITS);
  constexpr uint32_t E = 1u << BITS;
  const uint32_t n = blockIdx.x * kThreads + threadIdx.x;
  for (uint32_t k = n; k < inner; k += gridDim.x * kThreads) gamma16[k] = (_Float16)gamma[k];
  if (n >= columns) return;
  const _Float16* lut = palette + (uint64_t)min(n / group_columns, groups - 1u) * E;
  float g = 0.0f, b = 0.0f;
  for (uint32_t k = 0; k < inner; ++k) {
    const uint64_t i = (uint64_t)k * columns + n;
    const uint32_t* w = packed + (i / CPG) * WPG;
    const float wv = (float)lut[group_code<BITS>(w, (int)(i % CPG))];
    g = __builtin_fmaf((float)(_Float16)gamma[k], wv, g);
    b = __builtin_fmaf(beta[k], wv, b);
  }
  sums[n] = g;
  sums[columns + n] = b;
}

}  // namespace

hipError_t launch_norm_prepare(int bits, const uint32_t* packed, uint32_t inner, uint32_t columns,
                               uint32_t group_columns, uint32_t groups, const void* palette, const float* gamma,
                               const float* beta, void* gamma16, float* sums, hipStream_t stream) {
  const dim3 grid((max(columns, inner) + kThreads - 1) / kThreads);
  const _Float16* lut = static_cast<const _Float16*>(palette);
  _Float16* g16 = static_cast<_Float16*>(gamma16);
  if (bits == 5)
    hipLaunchKernelGGL(norm_prepare_kernel<5>, grid, dim3(kThreads), 0, stream, packed, inner, columns,
                       group_columns, groups, lut, gamma, beta, g16, sums);
  else if (bits == 6)
    hipLaunchKernelGGL(norm_prepare_kernel<6>, grid, dim3(kThreads), 0, stream, packed, inner, columns,
                       group_columns, groups, lut, gamma, beta, g16, sums);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace pk

// pk_attention.hip - Transformer-XL relative-position self-attention for
// gfx950 (reference: src/webgpu/kernels/attention.ts, shader :418-727,
// dispatch :51-316), 8 heads of 128 channels.
//
// For window b, head h and a query q below valid = min(valid[b], T):
//   score(q, k) = ((q + u)·k + (q + v)·R[T-1-q+k]) / sqrt(128),
//   out(q)      = softmax_k(score) · V over the keys k < valid,
// rows valid <= q < T are zero. R is the projected relative-position table
// (row p = relative distance T-1-p), in the reference's
// "head-vector-position-vec4" order [8][32][2T-1][4] or, with the row-major
// flag, as [2T-1, 1024] straight from a palette GEMM.
//
// f16 kernel (flash style, MFMA): a workgroup owns one (window, head,
// 32-query tile) and KSPLIT wavefronts, which take the 32-key tiles
// round robin and keep their own online-softmax state; the states meet in
// LDS at the end. Per key tile a wavefront computes, with
// v_mfma_f32_32x32x16_f16 (f32 accumulation):
//   * S^T = K · (Q+u)^T: keys are rows, so a lane holds 16 keys of one
//     query and a query's softmax needs one cross-half exchange only;
//   * the relative term over the 64-position window the tile needs,
//     W^T = R[p_lo .. p_lo+63] · (Q+v)^T with p_lo = T-1-q0-31+k0, written
//     to LDS and read back along the diagonal, score(q0+j, k0+i) taking
//     W^T[31 - j + i][j];
//   * O^T += V^T · P^T: the V tile goes to LDS transposed with key index
//     bits 2 and 3 swapped, which makes the probabilities a lane already
//     holds (keys 8a + 4h + b) exactly its MFMA operand, and the V^T rows one
//     ds_read_b128 each.
// (Q+u) and (Q+v) are formed in f32 and rounded to f16 once per workgroup;
// probabilities go to f16 for the PV product; everything else stays in f32.
//
// f32 kernels: a flash kernel on f32 MFMAs (planned), and a workgroup per
// (window, head, query) in the reference's own arithmetic (fma chains in
// channel order, max / exp / sum, fma over keys).
#include "pk_internal.h"

namespace pk {
namespace {

constexpr int kHeads = 8;
constexpr int kHead = 128;
constexpr int kHidden = kHeads * kHead;
constexpr int kQkvRow = 3 * kHidden;
constexpr int kTile = 32;          // queries per workgroup and keys per tile
constexpr int kVtStride = 40;      // halves per transposed V row (80 bytes: conflict-free b128 reads)
constexpr int kOtStride = 129;     // floats per merged output row
constexpr int kWaveLds = 64 * kTile * 4 + kHead * kVtStride * 2;  // diagonal window + V^T
static_assert(kTile * kOtStride * 4 + 2 * kTile * 4 <= kWaveLds, "merge state fits a wavefront's region");

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ half8 load8(const _Float16* p) { return *reinterpret_cast<const half8*>(p); }

// 8 channels d0 .. d0+7 (d0 % 8 == 0) of relative position p of one head.
template <bool ROW_MAJOR>
__device__ __forceinline__ half8 load_position(const _Float16* positions, uint32_t rows, int head, int p, int d0) {
  if constexpr (ROW_MAJOR) {
    return load8(positions + (uint64_t)p * kHidden + head * kHead + d0);
  } else {
    const int v = d0 / 4;  // two vec4 planes of [8][32][rows][4]
    const half4 lo = *reinterpret_cast<const half4*>(positions + (((uint64_t)head * 32 + v) * rows + p) * 4);
    const half4 hi = *reinterpret_cast<const half4*>(positions + (((uint64_t)head * 32 + v + 1) * rows + p) * 4);
    return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
}

__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// Headroom of the lazily moved softmax maximum (natural-log units).
constexpr float kRescaleMargin = 8.0f;

template <int KSPLIT, bool ROW_MAJOR>
__global__ __launch_bounds__(64 * KSPLIT) void rel_attention_f16_kernel(AttnArgs args) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[KSPLIT * kWaveLds];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j = lane & 31;
  const int hh = lane >> 5;

  const uint32_t qt = blockIdx.x % args.query_tiles;
  const uint32_t bh = blockIdx.x / args.query_tiles;
  const int head = (int)(bh % kHeads);
  const uint32_t b = bh / kHeads;
  const int T = (int)args.frames;
  const int live = (int)min(args.frames, args.valid_lengths[b]);
  const int q0 = (int)qt * kTile;
  const _Float16* qkv = static_cast<const _Float16*>(args.qkv) + (uint64_t)b * T * kQkvRow + head * kHead;
  _Float16* out = static_cast<_Float16*>(args.output) + (uint64_t)b * T * kHidden + head * kHead;

  if (q0 >= live) {
    // Every query of the tile is past the valid length: zero rows.
    for (int c = threadIdx.x; c < kTile * (kHead / 8); c += 64 * KSPLIT) {
      const int q = q0 + c / (kHead / 8);
      if (q < T) *reinterpret_cast<half8*>(out + (uint64_t)q * kHidden + (c % (kHead / 8)) * 8) = half8{};
    }
    return;
  }

  // (Q+u)^T and (Q+v)^T operands of query q0 + j: channels 16s + 8hh + 0..7.
  half8 qu[8], qv[8];
  {
    const _Float16* qrow = qkv + (uint64_t)min(q0 + j, T - 1) * kQkvRow;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int d0 = 16 * s + 8 * hh;
      const half8 x = load8(qrow + d0);
      const float4 u0 = *reinterpret_cast<const float4*>(args.bias_u + head * kHead + d0);
      const float4 u1 = *reinterpret_cast<const float4*>(args.bias_u + head * kHead + d0 + 4);
      const float4 v0 = *reinterpret_cast<const float4*>(args.bias_v + head * kHead + d0);
      const float4 v1 = *reinterpret_cast<const float4*>(args.bias_v + head * kHead + d0 + 4);
      const float uu[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
      const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        qu[s][t] = (_Float16)((float)x[t] + uu[t]);
        qv[s][t] = (_Float16)((float)x[t] + vv[t]);
      }
    }
  }

  float* window = reinterpret_cast<float*>(smem + wave * kWaveLds);                        // [64][32]
  _Float16* vt = reinterpret_cast<_Float16*>(smem + wave * kWaveLds + 64 * kTile * 4);     // [128][40]
  const float scale = 0.08838834764831845f;  // 1 / sqrt(128)

  float m = -INFINITY, l = 0.0f;
  floatx16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;

  const int tiles = (live + kTile - 1) / kTile;
  for (int kt = wave; kt < tiles; kt += KSPLIT) {
    const int k0 = kt * kTile;
    const int p_lo = T - 1 - q0 - (kTile - 1) + k0;
    const int pmax = (int)args.position_rows - 1;
    // S^T = K (Q+u)^T and W^T = R[p_lo ..] (Q+v)^T.
    floatx16 ac, w0, w1;
#pragma unroll
    for (int r = 0; r < 16; ++r) ac[r] = w0[r] = w1[r] = 0.0f;
    const _Float16* krow = qkv + (uint64_t)min(k0 + j, T - 1) * kQkvRow + kHidden;
    const int pa = min(max(p_lo + j, 0), pmax), pb = min(max(p_lo + kTile + j, 0), pmax);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int d0 = 16 * s + 8 * hh;
      const half8 kv = load8(krow + d0);
      const half8 ra = load_position<ROW_MAJOR>(static_cast<const _Float16*>(args.positions), args.position_rows,
                                                head, pa, d0);
      const half8 rb = load_position<ROW_MAJOR>(static_cast<const _Float16*>(args.positions), args.position_rows,
                                                head, pb, d0);
      ac = __builtin_amdgcn_mfma_f32_32x32x16_f16(kv, qu[s], ac, 0, 0, 0);
      w0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ra, qv[s], w0, 0, 0, 0);
      w1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(rb, qv[s], w1, 0, 0, 0);
    }
    // V tile -> LDS, transposed: vt[d][swap23(key)].
    {
      const _Float16* vrow = qkv + (uint64_t)min(k0 + j, T - 1) * kQkvRow + 2 * kHidden;
      const int slot = (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int d0 = 16 * c + 8 * hh;
        const half8 x = load8(vrow + d0);
#pragma unroll
        for (int t = 0; t < 8; ++t) vt[(d0 + t) * kVtStride + slot] = x[t];
      }
    }
    // Window rows c = 32 blk + 8 (r/4) + 4 hh + r%4, column j.
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int c = 8 * (r / 4) + 4 * hh + (r % 4);
      window[c * kTile + j] = w0[r];
      window[(kTile + c) * kTile + j] = w1[r];
    }
    // LDS operations of one wavefront complete in order; the fence keeps the
    // compiler from moving the reads above the writes.
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // Scores of keys k0 + i, i = 8 (r/4) + 4 hh + r%4, for query q0 + j.
    // All sixteen reads go out before the first use: left to itself the
    // compiler waits on each read in turn (a full LDS round trip apiece).
    float rel[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 8 * (r / 4) + 4 * hh + (r % 4);
      rel[r] = window[(kTile - 1 - j + i) * kTile + j];
    }
    __builtin_amdgcn_sched_barrier(0);
    float sc[16];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 8 * (r / 4) + 4 * hh + (r % 4);
      sc[r] = k0 + i < live ? (ac[r] + rel[r]) * scale : -INFINITY;
      mx = fmaxf(mx, sc[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // The running maximum (and with it O and l) moves only when some query's
    // scores exceed it by more than kRescaleMargin; below that the
    // probabilities stay under e^8, well inside f16, and O / l is unchanged.
    const bool moved = __builtin_amdgcn_ballot_w64(mx > m + kRescaleMargin) != 0;
    const float m_new = moved ? fmaxf(m, mx) : m;
    const float alpha = fast_exp(m - m_new);
    float rs = 0.0f;
    half8 pb8[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp(sc[r] - m_new);
      rs += p;
      pb8[r / 8][r % 8] = (_Float16)p;
    }
    rs += __shfl_xor(rs, 32, 64);
    l = l * alpha + rs;
    m = m_new;
    if (moved) {
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
    }
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const half8 va = load8(vt + (32 * db + j) * kVtStride + 16 * s + 8 * hh);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb8[s], o[db], 0, 0, 0);
      }
    }
    // The next tile rewrites this wavefront's window and V^T after these reads.
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  }

  // Merge the KSPLIT states; wavefront w then finishes channel blocks
  // [4w/KSPLIT, 4(w+1)/KSPLIT).
  constexpr int DB_PER = 4 / KSPLIT;
  float res[DB_PER][16];
  float* ot = reinterpret_cast<float*>(smem + wave * kWaveLds);       // [32][129]
  float* ml = ot + kTile * kOtStride;                                  // m[32], l[32]
  if constexpr (KSPLIT == 1) {
    const float inv = 1.0f / l;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) res[db][r] = o[db][r] * inv;
  } else {
    __syncthreads();
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) ot[j * kOtStride + 32 * db + 8 * (r / 4) + 4 * hh + (r % 4)] = o[db][r];
    if (hh == 0) {
      ml[j] = m;
      ml[kTile + j] = l;
    }
    __syncthreads();
    float mw[KSPLIT], big = -INFINITY;
#pragma unroll
    for (int w = 0; w < KSPLIT; ++w) {
      mw[w] = reinterpret_cast<const float*>(smem + w * kWaveLds)[kTile * kOtStride + j];
      big = fmaxf(big, mw[w]);
    }
    float f[KSPLIT], total = 0.0f;
#pragma unroll
    for (int w = 0; w < KSPLIT; ++w) {
      f[w] = fast_exp(mw[w] - big);
      total += f[w] * reinterpret_cast<const float*>(smem + w * kWaveLds)[kTile * kOtStride + kTile + j];
    }
    const float inv = 1.0f / total;
#pragma unroll
    for (int dl = 0; dl < DB_PER; ++dl) {
      const int db = wave * DB_PER + dl;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = 32 * db + 8 * (r / 4) + 4 * hh + (r % 4);
        float acc = 0.0f;
#pragma unroll
        for (int w = 0; w < KSPLIT; ++w)
          acc += f[w] * reinterpret_cast<const float*>(smem + w * kWaveLds)[j * kOtStride + d];
        res[dl][r] = acc * inv;
      }
    }
  }
  const int q = q0 + j;
  if (q < T) {
    const bool keep = q < live;
#pragma unroll
    for (int dl = 0; dl < DB_PER; ++dl) {
      const int db = (KSPLIT == 1 ? 0 : wave * DB_PER) + dl;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * db + 8 * g + 4 * hh;
        half4 h;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = keep ? (_Float16)res[dl][4 * g + e] : (_Float16)0.0f;
        *reinterpret_cast<half4*>(out + (uint64_t)q * kHidden + d) = h;
      }
    }
  }
}

// Shared-tile variant for long windows: NQ wavefronts own 32 queries each
// (32 NQ per workgroup) and walk every key tile together, so per tile all
// threads stage the K rows and the V^T tile once for the workgroup. The
// relative positions need even less: wavefront w's window for key tile kt
// is position blocks kt + NQ - 1 - w and kt + NQ - w (32 rows each, block 0
// starting at row T - q0 - 32 NQ), so the first half is the second half it
// used at tile kt - 1 and the second half is what wavefront w - 1 used
// then. The workgroup keeps the blocks in a ring of NQ + 1 and stages one
// new block per tile; each wavefront carries its second-half product over
// as the next tile's first half (16 instead of 24 score MFMAs per tile) and
// writes only that half of its diagonal window. The next two tiles' rows are
// on their way into registers while the current one is computed, and the
// output rescale is skipped when no query's running maximum moved.
template <int NQ, bool ROW_MAJOR>
__global__ __launch_bounds__(64 * NQ) void rel_attention_f16_shared_kernel(AttnArgs args) {
  constexpr int THREADS = 64 * NQ;
  constexpr int KSTRIDE = kHead + 8;     // halves per staged K / R row (272 bytes)
  constexpr int RING = NQ + 1;           // position blocks of 32 rows held at once
  constexpr int BCH = kTile * kHead / 8; // 16-byte chunks of one 32-row block
  constexpr int PER = BCH / THREADS;     // chunks per thread of each of K, V, positions
  static_assert(BCH % THREADS == 0, "a 32-row block splits evenly over the workgroup");
  __shared__ __attribute__((aligned(16))) _Float16 ks[kTile * KSTRIDE];
  __shared__ __attribute__((aligned(16))) _Float16 vts[kHead * kVtStride];
  __shared__ __attribute__((aligned(16))) _Float16 rs[RING * kTile * KSTRIDE];
  __shared__ __attribute__((aligned(16))) float windows[NQ * 64 * kTile];
  __shared__ __attribute__((aligned(16))) float uv[2 * kHead];  // u, then v, of this head

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int j = lane & 31;
  const int hh = lane >> 5;
  const uint32_t qt = blockIdx.x % args.query_tiles;
  const uint32_t bh = blockIdx.x / args.query_tiles;
  const int head = (int)(bh % kHeads);
  const uint32_t b = bh / kHeads;
  const int T = (int)args.frames;
  const int live = (int)min(args.frames, args.valid_lengths[b]);
  const int q0 = (int)qt * kTile * NQ;
  const _Float16* qkv = static_cast<const _Float16*>(args.qkv) + (uint64_t)b * T * kQkvRow + head * kHead;
  const _Float16* positions = static_cast<const _Float16*>(args.positions);
  _Float16* out = static_cast<_Float16*>(args.output) + (uint64_t)b * T * kHidden + head * kHead;

  if (q0 >= live) {
    for (int c = tid; c < kTile * NQ * (kHead / 8); c += THREADS) {
      const int q = q0 + c / (kHead / 8);
      if (q < T) *reinterpret_cast<half8*>(out + (uint64_t)q * kHidden + (c % (kHead / 8)) * 8) = half8{};
    }
    return;
  }

  const int qw = q0 + kTile * wave;  // this wavefront's first query
  const int pmax = (int)args.position_rows - 1;
  const int pbase = T - q0 - kTile * NQ;  // first row of position block 0
  auto position_chunk = [&](int block, int c) {
    const int row = c / (kHead / 8), part = c % (kHead / 8);
    return load_position<ROW_MAJOR>(positions, args.position_rows, head,
                                    min(max(pbase + kTile * block + row, 0), pmax), part * 8);
  };
  auto store_position = [&](int block, int c, const half8& x) {
    const int row = c / (kHead / 8), part = c % (kHead / 8);
    *reinterpret_cast<half8*>(rs + ((block % RING) * kTile + row) * KSTRIDE + part * 8) = x;
  };
  // Per key tile kt each thread moves PER chunks of the K rows, of the V
  // rows and of position block kt + NQ. K and position chunk c is row c / 16,
  // part c % 16; V chunk c is row c % 32, part c / 32, so that the 64 lanes
  // of one transposed 2-byte store write 32 banks, lane pairs sharing a
  // dword (part-major lanes put a whole wavefront on four banks).
  struct Staged {
    half8 k[PER], v[PER], r[PER];
  };
  auto fetch = [&](int kt, Staged& st) {
    const int k0 = kt * kTile;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * THREADS;
      const _Float16* row = qkv + (uint64_t)min(k0 + c / (kHead / 8), T - 1) * kQkvRow + (c % (kHead / 8)) * 8;
      st.k[i] = load8(row + kHidden);
      st.v[i] = load8(qkv + (uint64_t)min(k0 + c % kTile, T - 1) * kQkvRow + 2 * kHidden + (c / kTile) * 8);
      st.r[i] = position_chunk(kt + NQ, c);
    }
  };
  auto stage = [&](int kt, const Staged& st) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = tid + i * THREADS;
      const int kk = c / (kHead / 8), part = c % (kHead / 8);
      *reinterpret_cast<half8*>(ks + kk * KSTRIDE + part * 8) = st.k[i];
      const int vk = c % kTile, vpart = c / kTile;
      const int slot = (vk & ~12) | ((vk & 4) << 1) | ((vk & 8) >> 1);
#pragma unroll
      for (int t = 0; t < 8; ++t) vts[(vpart * 8 + t) * kVtStride + slot] = st.v[i][t];
      store_position(kt + NQ, c, st.r[i]);
    }
  };

  // Prologue loads, issued together so that one memory latency covers them:
  // position blocks 0 .. NQ-1 (block NQ comes with the first tile), this
  // wavefront's query rows with u and v, then the first two tiles' rows
  // (tile kt's registers are set kt % 2, refilled with tile kt + 2 as soon
  // as they are staged; fetches are unconditional, past the last tile they
  // re-read it and are never staged, so each wait counts only older loads).
  const int tiles = (live + kTile - 1) / kTile;
  constexpr int PRE = NQ * BCH / THREADS;
  static_assert((NQ * BCH) % THREADS == 0, "the prologue's position blocks split evenly");
  half8 pre[PRE];
#pragma unroll
  for (int i = 0; i < PRE; ++i) {
    const int c = tid + i * THREADS;
    pre[i] = position_chunk(c / BCH, c % BCH);
  }
  half8 qx[8];
  const _Float16* qrow = qkv + (uint64_t)min(qw + j, T - 1) * kQkvRow;
#pragma unroll
  for (int s = 0; s < 8; ++s) qx[s] = load8(qrow + 16 * s + 8 * hh);
  // u and v of the head: one value per thread into LDS (every wavefront
  // needs all 256; loading them per lane cost more than the query rows).
  constexpr int UVN = 2 * kHead / THREADS;
  static_assert((2 * kHead) % THREADS == 0, "u and v split evenly over the workgroup");
  float uv_value[UVN];
#pragma unroll
  for (int i = 0; i < UVN; ++i) {
    const int c = tid + i * THREADS;
    uv_value[i] = c < kHead ? args.bias_u[head * kHead + c] : args.bias_v[head * kHead + c - kHead];
  }
  Staged staged[2];
  fetch(0, staged[0]);
  fetch(min(1, tiles - 1), staged[1]);
#pragma unroll
  for (int i = 0; i < PRE; ++i) {
    const int c = tid + i * THREADS;
    store_position(c / BCH, c % BCH, pre[i]);
  }
#pragma unroll
  for (int i = 0; i < UVN; ++i) uv[tid + i * THREADS] = uv_value[i];
  __syncthreads();
  half8 qu[8], qv[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int d0 = 16 * s + 8 * hh;
    const float4 u0 = *reinterpret_cast<const float4*>(uv + d0), u1 = *reinterpret_cast<const float4*>(uv + d0 + 4);
    const float4 v0 = *reinterpret_cast<const float4*>(uv + kHead + d0);
    const float4 v1 = *reinterpret_cast<const float4*>(uv + kHead + d0 + 4);
    const float uu[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
    const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      qu[s][t] = (_Float16)((float)qx[s][t] + uu[t]);
      qv[s][t] = (_Float16)((float)qx[s][t] + vv[t]);
    }
  }

  float* window = windows + wave * 64 * kTile;
  const float scale = 0.08838834764831845f;
  float m = -INFINITY, l = 0.0f;
  floatx16 o[4], w_prev;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;

  auto tile = [&](auto slot, int kt) {
    constexpr int SL = decltype(slot)::value;
    const int k0 = kt * kTile;
    __syncthreads();  // every wavefront is done with the previous tile
    stage(kt, staged[SL]);
    __syncthreads();
    fetch(min(kt + 2, tiles - 1), staged[SL]);

    // S^T = K (Q+u)^T; second window half from block kt + NQ - wave.
    const _Float16* r_new = rs + (((kt + NQ - wave) % RING) * kTile + j) * KSTRIDE;
    floatx16 ac, w1;
#pragma unroll
    for (int r = 0; r < 16; ++r) ac[r] = w1[r] = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int d0 = 16 * s + 8 * hh;
      const half8 kv = *reinterpret_cast<const half8*>(ks + j * KSTRIDE + d0);
      const half8 rb = *reinterpret_cast<const half8*>(r_new + d0);
      ac = __builtin_amdgcn_mfma_f32_32x32x16_f16(kv, qu[s], ac, 0, 0, 0);
      w1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(rb, qv[s], w1, 0, 0, 0);
    }
    // Window half L of tile kt sits in physical half (L + kt) & 1.
    const int new_half = (1 + kt) & 1;
    if (kt == 0) {
      const _Float16* r_old = rs + (((NQ - 1 - wave) % RING) * kTile + j) * KSTRIDE;
#pragma unroll
      for (int r = 0; r < 16; ++r) w_prev[r] = 0.0f;
#pragma unroll
      for (int s = 0; s < 8; ++s)
        w_prev = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8*>(r_old + 16 * s + 8 * hh),
                                                        qv[s], w_prev, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 16; ++r) window[(8 * (r / 4) + 4 * hh + (r % 4)) * kTile + j] = w_prev[r];
    }
#pragma unroll
    for (int r = 0; r < 16; ++r)
      window[(new_half * kTile + 8 * (r / 4) + 4 * hh + (r % 4)) * kTile + j] = w1[r];
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // All sixteen reads go out before the first use (see the kernel above),
    // and with them the V^T operands of the PV product, which do not wait
    // for the softmax.
    float rel[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int c = kTile - 1 - j + 8 * (r / 4) + 4 * hh + (r % 4);
      rel[r] = window[((((c >> 5) + kt) & 1) * kTile + (c & 31)) * kTile + j];
    }
    half8 va[4][2];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        va[db][s] = *reinterpret_cast<const half8*>(vts + (32 * db + j) * kVtStride + 16 * s + 8 * hh);
    __builtin_amdgcn_sched_barrier(0);
    float sc[16];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 8 * (r / 4) + 4 * hh + (r % 4);
      sc[r] = k0 + i < live ? (ac[r] + rel[r]) * scale : -INFINITY;
      mx = fmaxf(mx, sc[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // The running maximum (and with it O and l) moves only when some query's
    // scores exceed it by more than kRescaleMargin; below that the
    // probabilities stay under e^8, well inside f16, and O / l is unchanged.
    const bool moved = __builtin_amdgcn_ballot_w64(mx > m + kRescaleMargin) != 0;
    const float m_new = moved ? fmaxf(m, mx) : m;
    const float alpha = fast_exp(m - m_new);
    float rsum = 0.0f;
    half8 pb8[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = fast_exp(sc[r] - m_new);
      rsum += p;
      pb8[r / 8][r % 8] = (_Float16)p;
    }
    rsum += __shfl_xor(rsum, 32, 64);
    l = l * alpha + rsum;
    m = m_new;
    if (moved) {
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
    }
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int s = 0; s < 2; ++s) o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[db][s], pb8[s], o[db], 0, 0, 0);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  };
  for (int kt = 0; kt < tiles; kt += 2) {
    tile(std::integral_constant<int, 0>{}, kt);
    if (kt + 1 < tiles) tile(std::integral_constant<int, 1>{}, kt + 1);
  }

  const int q = qw + j;
  if (q < T) {
    const bool keep = q < live;
    const float inv = 1.0f / l;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * db + 8 * g + 4 * hh;
        half4 h;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = keep ? (_Float16)(o[db][4 * g + e] * inv) : (_Float16)0.0f;
        *reinterpret_cast<half4*>(out + (uint64_t)q * kHidden + d) = h;
      }
  }
}

// The reference's arithmetic in f32: one workgroup of 256 threads per
// (window, head, query); scores of all keys live in LDS (T <= kMaxFrames).
template <bool ROW_MAJOR>
__global__ __launch_bounds__(256) void rel_attention_f32_kernel(AttnArgs args) {
  __shared__ float qu[kHead], qv[kHead];
  __shared__ float scores[kAttentionMaxFrames];
  __shared__ float red[8];
  const int tid = threadIdx.x;
  const int T = (int)args.frames;
  const int q = (int)(blockIdx.x % args.frames);
  const uint32_t bh = blockIdx.x / args.frames;
  const int head = (int)(bh % kHeads);
  const uint32_t b = bh / kHeads;
  const int live = (int)min(args.frames, args.valid_lengths[b]);
  const float* qkv = static_cast<const float*>(args.qkv) + (uint64_t)b * T * kQkvRow + head * kHead;
  float* out = static_cast<float*>(args.output) + ((uint64_t)b * T + q) * kHidden + head * kHead;
  const float* positions = static_cast<const float*>(args.positions);
  if (q >= live) {
    if (tid < kHead) out[tid] = 0.0f;
    return;
  }
  if (tid < kHead) {
    const float x = qkv[(uint64_t)q * kQkvRow + tid];
    qu[tid] = x + args.bias_u[head * kHead + tid];
    qv[tid] = x + args.bias_v[head * kHead + tid];
  }
  __syncthreads();
  float local_max = -3.402823466e+38f;
  for (int k = tid; k < live; k += 256) {
    const float* key = qkv + (uint64_t)k * kQkvRow + kHidden;
    const int rel = T - 1 - q + k;
    float acc = 0.0f;
    for (int d = 0; d < kHead; ++d) {
      const float r = ROW_MAJOR ? positions[(uint64_t)rel * kHidden + head * kHead + d]
                                : positions[(((uint64_t)head * 32 + d / 4) * args.position_rows + rel) * 4 + d % 4];
      acc = __builtin_fmaf(qu[d], key[d], acc);
      acc = __builtin_fmaf(qv[d], r, acc);
    }
    acc *= 0.08838834764831845f;
    scores[k] = acc;
    local_max = fmaxf(local_max, acc);
  }
  // workgroup max, then sum of exp
  for (int off = 32; off > 0; off >>= 1) local_max = fmaxf(local_max, __shfl_xor(local_max, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = local_max;
  __syncthreads();
  const float maximum = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float local_sum = 0.0f;
  for (int k = tid; k < live; k += 256) {
    const float e = expf(scores[k] - maximum);
    scores[k] = e;
    local_sum += e;
  }
  for (int off = 32; off > 0; off >>= 1) local_sum += __shfl_xor(local_sum, off, 64);
  __syncthreads();
  if ((tid & 63) == 0) red[4 + (tid >> 6)] = local_sum;
  __syncthreads();
  const float inverse = 1.0f / (red[4] + red[5] + red[6] + red[7]);
  if (tid < kHead) {
    float acc = 0.0f;
    for (int k = 0; k < live; ++k)
      acc = __builtin_fmaf(scores[k] * inverse, qkv[(uint64_t)k * kQkvRow + 2 * kHidden + tid], acc);
    out[tid] = acc;
  }
}

// f32 flash kernel on v_mfma_f32_32x32x2_f32: a wavefront owns one
// (window, head, 32-query tile) and walks the key tiles in order, four
// independent wavefronts per workgroup. The products are the f16 kernel's
// (S^T = K (Q+u)^T, the 64-position window W^T = R (Q+v)^T read back along
// the diagonal, O^T += V^T P^T), with three changes for single-K f32 MFMAs:
//   * lane half h supplies channel 64h + s to product s of the 64 that make
//     up a 128-channel dot product, so each lane reads 64 contiguous
//     channels of its key, position and query rows;
//   * the window's lower 32 rows are the previous tile's upper 32 (p_lo
//     moves by 32 per key tile), so only 32 new positions are multiplied per
//     tile;
//   * PV product t takes keys 8(t/4) + 4h + t%4 in slot h, the keys whose
//     probabilities lane half h already holds in register t, and output
//     block e takes channel 4c + e in row c, so each lane reads V as one
//     float4 of 4 consecutive channels per key and writes O as float4s.
// All arithmetic is f32 (MFMA products accumulate in f32 in hardware
// order); results stay within a few 1e-6 of the reference order.
constexpr int kF32Waves = 4;

template <bool ROW_MAJOR>
__device__ __forceinline__ float4 load_position_f32(const float* positions, uint32_t rows, int head, int p, int d0) {
  if constexpr (ROW_MAJOR)
    return *reinterpret_cast<const float4*>(positions + (uint64_t)p * kHidden + head * kHead + d0);
  else
    return *reinterpret_cast<const float4*>(positions + (((uint64_t)head * 32 + d0 / 4) * rows + p) * 4);
}

template <bool ROW_MAJOR>
__global__ __launch_bounds__(64 * kF32Waves) void rel_attention_f32_mfma_kernel(AttnArgs args) {
  __shared__ __attribute__((aligned(16))) float windows[kF32Waves * 64 * kTile];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j = lane & 31;
  const int hh = lane >> 5;
  // No workgroup barrier below: a wavefront past the last item just ends.
  const uint32_t item = blockIdx.x * kF32Waves + (uint32_t)wave;
  if (item >= args.work_items) return;
  const uint32_t qt = item % args.query_tiles;
  const uint32_t bh = item / args.query_tiles;
  const int head = (int)(bh % kHeads);
  const uint32_t b = bh / kHeads;
  const int T = (int)args.frames;
  const int live = (int)min(args.frames, args.valid_lengths[b]);
  const int q0 = (int)qt * kTile;
  const float* qkv = static_cast<const float*>(args.qkv) + (uint64_t)b * T * kQkvRow + head * kHead;
  float* out = static_cast<float*>(args.output) + (uint64_t)b * T * kHidden + head * kHead;

  if (q0 >= live) {
    for (int c = lane; c < kTile * (kHead / 4); c += 64) {
      const int q = q0 + c / (kHead / 4);
      if (q < T) *reinterpret_cast<float4*>(out + (uint64_t)q * kHidden + (c % (kHead / 4)) * 4) = float4{};
    }
    return;
  }

  const int d_half = 64 * hh;  // channels d_half + s of product s
  float qu[64], qv[64];
  {
    const float* qrow = qkv + (uint64_t)min(q0 + j, T - 1) * kQkvRow + d_half;
    const float* bu = args.bias_u + head * kHead + d_half;
    const float* bv = args.bias_v + head * kHead + d_half;
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      const float4 x = *reinterpret_cast<const float4*>(qrow + 4 * g);
      const float4 u = *reinterpret_cast<const float4*>(bu + 4 * g);
      const float4 v = *reinterpret_cast<const float4*>(bv + 4 * g);
      qu[4 * g] = x.x + u.x;
      qu[4 * g + 1] = x.y + u.y;
      qu[4 * g + 2] = x.z + u.z;
      qu[4 * g + 3] = x.w + u.w;
      qv[4 * g] = x.x + v.x;
      qv[4 * g + 1] = x.y + v.y;
      qv[4 * g + 2] = x.z + v.z;
      qv[4 * g + 3] = x.w + v.w;
    }
  }

  const float* positions = static_cast<const float*>(args.positions);
  const int pmax = (int)args.position_rows - 1;
  // 32 window rows p_first .. p_first + 31 for the 32 queries: R (Q+v)^T.
  // Rows outside [0, 2T-2] are clamped; they only meet masked keys or
  // queries past the valid length.
  auto window_rows = [&](int p_first) {
    floatx16 w;
#pragma unroll
    for (int r = 0; r < 16; ++r) w[r] = 0.0f;
    const int p = min(max(p_first + j, 0), pmax);
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      const float4 x = load_position_f32<ROW_MAJOR>(positions, args.position_rows, head, p, d_half + 4 * g);
      w = __builtin_amdgcn_mfma_f32_32x32x2f32(x.x, qv[4 * g], w, 0, 0, 0);
      w = __builtin_amdgcn_mfma_f32_32x32x2f32(x.y, qv[4 * g + 1], w, 0, 0, 0);
      w = __builtin_amdgcn_mfma_f32_32x32x2f32(x.z, qv[4 * g + 2], w, 0, 0, 0);
      w = __builtin_amdgcn_mfma_f32_32x32x2f32(x.w, qv[4 * g + 3], w, 0, 0, 0);
    }
    return w;
  };

  float* window = windows + wave * 64 * kTile;  // [64][32]
  const float scale = 0.08838834764831845f;      // 1 / sqrt(128)
  float m = -INFINITY, l = 0.0f;
  floatx16 o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[e][r] = 0.0f;

  const int tiles = (live + kTile - 1) / kTile;
  floatx16 w_low = window_rows(T - 1 - q0 - (kTile - 1));
  for (int kt = 0; kt < tiles; ++kt) {
    const int k0 = kt * kTile;
    const int p_lo = T - 1 - q0 - (kTile - 1) + k0;
    floatx16 ac;
#pragma unroll
    for (int r = 0; r < 16; ++r) ac[r] = 0.0f;
    const float* krow = qkv + (uint64_t)min(k0 + j, T - 1) * kQkvRow + kHidden + d_half;
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      const float4 x = *reinterpret_cast<const float4*>(krow + 4 * g);
      ac = __builtin_amdgcn_mfma_f32_32x32x2f32(x.x, qu[4 * g], ac, 0, 0, 0);
      ac = __builtin_amdgcn_mfma_f32_32x32x2f32(x.y, qu[4 * g + 1], ac, 0, 0, 0);
      ac = __builtin_amdgcn_mfma_f32_32x32x2f32(x.z, qu[4 * g + 2], ac, 0, 0, 0);
      ac = __builtin_amdgcn_mfma_f32_32x32x2f32(x.w, qu[4 * g + 3], ac, 0, 0, 0);
    }
    const floatx16 w_high = window_rows(p_lo + kTile);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int c = 8 * (r / 4) + 4 * hh + (r % 4);
      window[c * kTile + j] = w_low[r];
      window[(kTile + c) * kTile + j] = w_high[r];
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    float rel[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 8 * (r / 4) + 4 * hh + (r % 4);
      rel[r] = window[(kTile - 1 - j + i) * kTile + j];
    }
    __builtin_amdgcn_sched_barrier(0);
    float sc[16];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 8 * (r / 4) + 4 * hh + (r % 4);
      sc[r] = k0 + i < live ? (ac[r] + rel[r]) * scale : -INFINITY;
      mx = fmaxf(mx, sc[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const bool moved = __builtin_amdgcn_ballot_w64(mx > m + kRescaleMargin) != 0;
    const float m_new = moved ? fmaxf(m, mx) : m;
    const float alpha = fast_exp(m - m_new);
    float rs = 0.0f;
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      p[r] = fast_exp(sc[r] - m_new);
      rs += p[r];
    }
    rs += __shfl_xor(rs, 32, 64);
    l = l * alpha + rs;
    m = m_new;
    if (moved) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[e][r] *= alpha;
    }
    // O^T += V^T P^T: product t pairs key 8(t/4) + 4 hh + t%4 (slot hh) with
    // channels 4j .. 4j+3 of that key, one per output block.
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int key = min(k0 + 8 * (t / 4) + 4 * hh + (t % 4), T - 1);
      const float4 v = *reinterpret_cast<const float4*>(qkv + (uint64_t)key * kQkvRow + 2 * kHidden + 4 * j);
      o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(v.x, p[t], o[0], 0, 0, 0);
      o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(v.y, p[t], o[1], 0, 0, 0);
      o[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(v.z, p[t], o[2], 0, 0, 0);
      o[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(v.w, p[t], o[3], 0, 0, 0);
    }
    // The next tile rewrites the window after these reads.
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    w_low = w_high;
  }

  // Block e, register r of lane (j, hh): channel 4 (8(r/4) + 4hh + r%4) + e
  // of query q0 + j.
  const int q = q0 + j;
  if (q < T) {
    const bool keep = q < live;
    const float inv = 1.0f / l;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int c = 8 * (r / 4) + 4 * hh + (r % 4);
      const float4 y = keep ? float4{o[0][r] * inv, o[1][r] * inv, o[2][r] * inv, o[3][r] * inv} : float4{};
      *reinterpret_cast<float4*>(out + (uint64_t)q * kHidden + 4 * c) = y;
    }
  }
}

struct AttnVariant {
  const char* name;
  int waves;
  int queries;  // per workgroup
  uint32_t lds_bytes;
  void (*packed)(AttnArgs);
  void (*row_major)(AttnArgs);
};

#define PK_ATTN_VARIANT(K)                                                                                 \
  AttnVariant {                                                                                            \
    "pk_rel_attention_f16_q32_w" #K, K, kTile, (uint32_t)(K * kWaveLds), rel_attention_f16_kernel<K, false>, \
        rel_attention_f16_kernel<K, true>                                                                  \
  }
#define PK_ATTN_SHARED_VARIANT(NQ)                                                                         \
  AttnVariant {                                                                                            \
    "pk_rel_attention_f16_q" #NQ "x32_shared", NQ, NQ * kTile,                                             \
        (uint32_t)((kTile + (NQ + 1) * kTile) * (kHead + 8) * 2 + kHead * kVtStride * 2 + NQ * 64 * kTile * 4 + \
                   2 * kHead * 4),                                                                         \
        rel_attention_f16_shared_kernel<NQ, false>, rel_attention_f16_shared_kernel<NQ, true>              \
  }

// Planned (32-query tiles = windows x 8 heads x ceil(T / 32), measured at
// T = 188 on one MI355X): index 0 while one round of its workgroups fills
// the device (4 windows: 12.3 us against 15.9 us for index 3); index 3 up to
// 384 tiles (8 windows: 16.0 us against 18.3 us for index 4 and 19.9 us for
// index 1); index 4 below 1152 (12 / 16 windows: 19.1 / 19.6 us); index 3
// from 1152 (24 windows: 32.4 against 33.5 us; 40 windows: 39.5 against
// 51.3 us, where index 4's half-empty second query block per window and
// head costs more than its shared staging saves); index 4 for windows
// longer than 256 frames (4 x 750: 46.2 us against 50.6 us for index 3 and
// 86.9 us for index 0).
const AttnVariant kF16Variants[] = {PK_ATTN_VARIANT(4), PK_ATTN_VARIANT(2), PK_ATTN_VARIANT(1),
                                    PK_ATTN_SHARED_VARIANT(2), PK_ATTN_SHARED_VARIANT(4)};
// f32: index 0 the MFMA kernel (planned), index 1 one workgroup per query in
// the reference's own operation order.
const AttnVariant kF32Variants[] = {
    {"pk_rel_attention_f32_mfma", kF32Waves, kTile, (uint32_t)(kF32Waves * 64 * kTile * 4),
     rel_attention_f32_mfma_kernel<false>, rel_attention_f32_mfma_kernel<true>},
    {"pk_rel_attention_f32", 4, 1, (uint32_t)((2 * kHead + kAttentionMaxFrames + 8) * 4), rel_attention_f32_kernel<false>,
     rel_attention_f32_kernel<true>}};

}  // namespace

int attention_default_variant(bool f16, uint32_t frames, uint32_t batch) {
  if (!f16) return 0;
  if (frames > 256u) return 4;
  const uint64_t tiles = (uint64_t)batch * kHeads * ((frames + kTile - 1) / kTile);
  return tiles <= 256u ? 0 : tiles <= 384u ? 3 : tiles < 1152u ? 4 : 3;
}

int attention_variant_count(bool f16) {
  return f16 ? (int)(sizeof(kF16Variants) / sizeof(kF16Variants[0]))
             : (int)(sizeof(kF32Variants) / sizeof(kF32Variants[0]));
}

AttnGeometry attention_geometry(bool f16, int variant, uint32_t frames, uint32_t batch) {
  AttnGeometry g;
  if (f16) {
    const AttnVariant& v = kF16Variants[variant];
    g.name = v.name;
    g.query_tiles = (frames + v.queries - 1) / v.queries;
    g.grid = batch * kHeads * g.query_tiles;
    g.block_threads = 64 * v.waves;
    g.lds_bytes = v.lds_bytes;
  } else if (variant == 0) {
    const AttnVariant& v = kF32Variants[0];
    g.name = v.name;
    g.query_tiles = (frames + kTile - 1) / kTile;
    g.grid = (batch * kHeads * g.query_tiles + kF32Waves - 1) / kF32Waves;
    g.block_threads = 64 * kF32Waves;
    g.lds_bytes = v.lds_bytes;
  } else {
    const AttnVariant& v = kF32Variants[1];
    g.name = v.name;
    g.query_tiles = frames;
    g.grid = batch * kHeads * frames;
    g.block_threads = 256;
    g.lds_bytes = v.lds_bytes;
  }
  return g;
}

hipError_t launch_attention(bool f16, int variant, const AttnArgs& base, uint32_t batch, hipStream_t stream,
                            hipEvent_t start, hipEvent_t stop) {
  const AttnGeometry g = attention_geometry(f16, variant, base.frames, batch);
  if (g.grid == 0) return hipSuccess;
  AttnArgs args = base;
  args.query_tiles = g.query_tiles;
  args.work_items = batch * kHeads * g.query_tiles;
  const AttnVariant& v = f16 ? kF16Variants[variant] : kF32Variants[variant];
  void (*kernel)(AttnArgs) = base.positions_row_major ? v.row_major : v.packed;
  if (start || stop)
    hipExtLaunchKernelGGL(kernel, dim3(g.grid), dim3(g.block_threads), 0, stream, start, stop, 0, args);
  else
    hipLaunchKernelGGL(kernel, dim3(g.grid), dim3(g.block_threads), 0, stream, args);
  return hipGetLastError();
}

}  // namespace pk

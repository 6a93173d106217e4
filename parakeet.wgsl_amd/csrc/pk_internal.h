// pk_internal.h - shared declarations of the palette GEMM library (gfx950).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pk {

// Reference packed-format group geometry (model/convert.py:2119-2127).
__host__ __device__ constexpr uint32_t codes_per_group(int bits) { return bits == 5 ? 32u : 16u; }
__host__ __device__ constexpr uint32_t words_per_group(int bits) { return bits == 5 ? 5u : 3u; }

// ---------------------------------------------------------------------------
// MFMA-native packed layout ("operand order"), built once per weight.
//
// The logical [K, N] code matrix is cut into blocks of 64 k x 32 n. Inside a
// block, lane l = 32*h + j (h in {0,1}, j in [0,32)) of a wavefront owns the
// 32 codes of column n = 32*nb + j at k = 64*kb + 32*h + u, u = 0..31, packed
// LSB-first at bit u*bits of a `bits`-word stream (the same bits per code as
// the reference format, so the same number of bytes). Words 0..3 of every
// lane are stored lane-interleaved as one 16-byte vector per lane (plane 0),
// the remaining bits-4 words as one 4- or 8-byte vector per lane (plane 1),
// so a wavefront fetches a block with one coalesced 128-bit load plus one
// 32/64-bit load per lane. Blocks are ordered [nb][kb], making the stream a
// wavefront reads along K contiguous. K pads to 64 and N to 32 with code 0.
//
// Split into P parts (P = 2 or 4, for kernels whose workgroup splits each
// K block over P wavefronts): a lane's 32 codes form P parts of 32 / P
// K-consecutive codes, part p holding k = 64*kb + 32*h + 32p/P + u', in its
// own parts_words(bits, P) words: each pair of codes (k even, k + 1) is a
// 16-bit slot holding 4 * (c0 | c1 << bits), the byte offset of the pair's
// entry in a 2^bits x 2^bits LDS table (one byte per weight). A block is
// [part][lane][words], so the wavefront of part p reads one contiguous 16-
// or 8-byte run per lane and nothing else, and decodes a pair with one
// extract.
//
// A weight is prepared once in the one layout (P) its GEMM's kernel reads:
// P = 1 at the packed format's density (5/8 or 6/8 byte per weight), P = 2
// or 4 at one byte.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr uint32_t parts_words(int bits, int parts) {
  return parts == 1 ? (uint32_t)bits : parts == 2 ? 4u : 2u;
}
__host__ __device__ constexpr uint32_t block_words(int bits, int parts = 1) {
  return 64u * (uint32_t)parts * parts_words(bits, parts);
}
__host__ __device__ constexpr uint32_t padded_inner(uint32_t inner) { return (inner + 63u) / 64u * 64u; }
__host__ __device__ constexpr uint32_t padded_columns(uint32_t columns) { return (columns + 31u) / 32u * 32u; }
__host__ __device__ constexpr uint64_t operand_order_words(int bits, uint32_t inner, uint32_t columns,
                                                           int parts = 1) {
  return (uint64_t)(padded_columns(columns) / 32u) * (padded_inner(inner) / 64u) * block_words(bits, parts);
}

enum Activation : int { kActNone = 0, kActSilu = 1, kActRelu = 2 };

// Largest K of a GEMM with the fused row LayerNorm (its gamma is staged in
// LDS as f16).
constexpr uint32_t kNormMaxInner = 2048;

struct GemmArgs {
  const void* a;             // [M, K]
  const uint32_t* codes;     // operand-order codes
  const void* palette;       // [G, 2^bits]
  void* out;                 // [M, N]
  const float* bias;         // [N] or null
  const void* residual;      // [M, N] or null
  float residual_scale;
  int activation;
  // GLU epilogue (pair-code kernels only): the weight's 32-column blocks
  // alternate values and gates (launch_to_operand_order with glu_interleave),
  // and out is [M, N/2] = value * sigmoid(gate).
  int glu;
  uint32_t rows;             // active M
  uint32_t inner;            // K
  uint32_t columns;          // N
  uint32_t palette_groups;
  uint32_t palette_group_columns;
  uint32_t palette_entries;  // 2^bits
  // Split-K: `splits` workgroups share one output tile, each over a
  // contiguous range of 64-deep K blocks. With splits > 1 every workgroup
  // writes its f32 partial tile to `partials` and bumps the tile's counter;
  // the last one to arrive sums the partials in split order (so the result
  // does not depend on arrival order), applies the epilogue, stores the
  // tile and resets the counter to zero for the next launch.
  uint32_t splits;
  float* partials;           // [tiles][splits][tile elements] or null
  uint32_t* counters;        // [tiles], zero between launches, or null
  // Row LayerNorm fused into the input (pair-code kernels; K % 64 == 0,
  // one palette group per tile). With norm_columns set the GEMM multiplies
  // LN(A), LN(a)_k = (a_k - mean) * rstd * gamma_k + beta_k with mean and
  // variance over the K channels of the row, without a separate pass: the
  // kernel stages a_k * gamma_k (gamma as f16) and the row's sum and sum
  // of squares, and finishes each output as rstd * (acc - mean * G_n) + B_n
  // with G = gamma . W and B = beta . W (norm_columns = G then B, 2N f32).
  const _Float16* norm_gamma;  // [K] or null
  const float* norm_columns;   // [2N] or null
  float norm_epsilon;
  // Set by the host for f16 ops unless they keep their output cached
  // (PK_GEMM_CACHED_OUTPUT): the launch then runs a kernel instantiation
  // whose output stores are non-temporal (stream_store), where one is
  // compiled. The next launch mostly reads an output from other XCDs than
  // the one that wrote each line, and streamed lines need no write-back
  // from L2 when the kernel ends: on the 16-window encoder pass this takes
  // 0.3-1.4 us off each layer GEMM (1.6% off the pass); at 1 and 4 windows
  // the pass time is unchanged within 0.3%. A runtime branch between the
  // two store kinds would not do: the compiler merges the two stores into
  // one and drops the non-temporal hint.
  int stream_out;
};

// A store of an output that no later instruction of this kernel reads,
// marked non-temporal (global_store ... nt).
template <class T>
__device__ __forceinline__ void stream_store(T* p, const T& v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8 || sizeof(T) == 16, "dword, dwordx2 or dwordx4 stores");
  if constexpr (sizeof(T) == 4) {
    __builtin_nontemporal_store(__builtin_bit_cast(uint32_t, v), reinterpret_cast<uint32_t*>(p));
  } else {
    typedef uint32_t words __attribute__((ext_vector_type(sizeof(T) / 4)));
    __builtin_nontemporal_store(__builtin_bit_cast(words, v), reinterpret_cast<words*>(p));
  }
}


// Tile shapes compiled for the fused GEMM. Every variant is one workgroup of
// waves_m x waves_n x k_split wavefronts; a wavefront owns m_blocks x
// n_blocks MFMA output blocks of 32 x 32, and with k_split > 1 the
// k_split wavefronts of one (m, n) position each multiply their own part
// of every K block and add their partial tiles at the end.
struct TileShape {
  int waves_m, waves_n, m_blocks, n_blocks;
  int k_split = 1;
  __host__ __device__ constexpr int threads() const { return 64 * waves_m * waves_n * k_split; }
  __host__ __device__ constexpr int tile_rows() const { return 32 * waves_m * m_blocks; }
  __host__ __device__ constexpr int tile_columns() const { return 32 * waves_n * n_blocks; }
  // f32 elements of one workgroup's split-K partial tile.
  __host__ __device__ constexpr uint32_t tile_elements() const {
    return (uint32_t)(tile_rows() * tile_columns());
  }
};

// Output tiles of a launch over `rows` x `columns` (columns padded to 32).
inline uint32_t tiles_m(const TileShape& s, uint32_t rows) {
  return (rows + s.tile_rows() - 1) / s.tile_rows();
}
inline uint32_t tiles_n(const TileShape& s, uint32_t columns) {
  return (padded_columns(columns) + s.tile_columns() - 1) / s.tile_columns();
}

// Workgroups of a small-M launch over `column_groups` column groups of
// `s`: whole rounds of the eight XCDs per row group (pk_gemm_f16s.hip).
inline uint32_t small_m_grid(const TileShape& s, uint32_t column_groups, uint32_t rows) {
  return (column_groups + 7u) / 8u * 8u * tiles_m(s, rows);
}

// Workgroup i is dispatched to XCD i % 8 (round robin). This bijection on
// [0, count) gives the workgroups of one XCD a contiguous range of work
// items, so tiles that share activation rows share that XCD's L2.
__host__ __device__ inline uint32_t xcd_local_order(uint32_t i, uint32_t count) {
  constexpr uint32_t kXcds = 8;
  const uint32_t xcd = i % kXcds, slot = i / kXcds;
  const uint32_t per = count / kXcds, rem = count % kXcds;
  return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

// One launch of a GEMM kernel on `stream`. With a start and/or stop event
// the dispatch itself stamps them (hipExtLaunchKernel), so timing a kernel
// adds no packets to the stream.
inline hipError_t launch_timed(void (*kernel)(GemmArgs), dim3 grid, dim3 block, hipStream_t stream,
                               hipEvent_t start, hipEvent_t stop, const GemmArgs& args) {
  if (start || stop)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0, args);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, args);
  return hipGetLastError();
}

// Launchers. Each returns the hipError_t of the launch.
hipError_t launch_unpack(int bits, const uint32_t* words, uint64_t groups,
                         uint8_t* codes, hipStream_t stream);
hipError_t launch_expand(int bits, bool f16, bool tile_major, const uint32_t* packed,
                         uint32_t inner, uint32_t columns, uint32_t group_columns,
                         uint32_t groups, const void* palette, void* target,
                         hipStream_t stream);
// glu_interleave: physical column block 2i takes logical block i (a GLU
// value block) and block 2i+1 takes logical block N/64 + i (its gates);
// needs N % 64 == 0. `parts` selects the P-part split (1, 2 or 4).
hipError_t launch_to_operand_order(int bits, const uint32_t* packed, uint32_t inner,
                                   uint32_t columns, uint32_t* codes, hipStream_t stream,
                                   bool glu_interleave = false, int parts = 1);
// Fused row LayerNorm of a GEMM's input (GemmArgs::norm_columns): writes
// gamma16 = f16(gamma) [K] and sums = G then B [2N] from the reference-format
// codes and the f16 palette.
hipError_t launch_norm_prepare(int bits, const uint32_t* packed, uint32_t inner, uint32_t columns,
                               uint32_t group_columns, uint32_t groups, const void* palette, const float* gamma,
                               const float* beta, void* gamma16, float* sums, hipStream_t stream);
// The same codes moved from one P-part split to another (no packed source
// needed); `blocks` = operand-order blocks of the weight.
hipError_t launch_relayout(int bits, const uint32_t* src, int src_parts, uint32_t* dst, int dst_parts,
                           uint64_t blocks, hipStream_t stream);

// Fused palette GEMM. `variant` indexes f16_variants() / f32_variants().
int f16_variant_count();
TileShape f16_variant(int index);
const char* f16_variant_name(int bits, int index);
uint32_t f16_variant_lds_bytes(int index);
// Kernel family of an f16 variant. Only the operand-order family also runs
// split-K across workgroups; the others split K inside the workgroup.
enum F16Family : int { kFamilyOperandOrder = 0, kFamilyPairCode = 1, kFamilySmallM = 2 };
int f16_variant_family(int index);
inline bool f16_variant_splits(int index) { return f16_variant_family(index) == kFamilyOperandOrder; }
// Parts of the code layout an f16 variant reads (pk_internal.h layout): its
// K split for the pair-code family, 1 for every other kernel.
inline int f16_variant_parts(int index) {
  return f16_variant_family(index) == kFamilyPairCode ? f16_variant(index).k_split : 1;
}
hipError_t launch_gemm_f16(int bits, int variant, const GemmArgs& args, hipStream_t stream,
                           hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// Whether launch_gemm_f16 runs `variant` with non-temporal output stores
// for `args` (stream_out set and a streamed kernel compiled for it: the
// pair-code family's single-path kernels).
bool f16_variant_streams(int bits, int variant, const GemmArgs& args);
// Workgroups of one launch of an f16 variant.
uint32_t f16_variant_grid(int index, uint32_t rows, uint32_t columns, uint32_t splits);

// A group of independent f16 GEMMs run by one launch of a small-M variant:
// `items` lists (member << 16 | column group) over the members' column
// groups of that variant's width; every member takes `rows` rows and
// reads operand-order codes of one part.
struct SmallMMember {
  GemmArgs args;
  int bits;
  int reserved;
};
struct SmallMGroupArgs {
  const SmallMMember* members;
  const uint32_t* items;
  uint32_t items_count;
  uint32_t rows;
  uint32_t row_groups;  // tiles_m of the variant at `rows`
  uint32_t persistent;  // 1: every member fits the variant's persistent kernel
};
const char* f16_group_kernel_name(int index);
// Whether small-M variant `index` has a persistent group kernel.
bool f16_group_persistent(int index);
// Whether a member of K `inner` and the given palette grouping fits the
// persistent group kernel of small-M variant `index` (false for a variant
// without one).
bool f16_group_streams(int index, uint32_t inner, uint32_t palette_groups, uint32_t palette_group_columns);
// Grid (x) and kernel name of the launch launch_gemm_f16_group makes.
uint32_t f16_group_launch_plan(int index, const SmallMGroupArgs& group, const char** kernel);
hipError_t launch_gemm_f16_group(int index, const SmallMGroupArgs& group, hipStream_t stream,
                                 hipEvent_t start = nullptr, hipEvent_t stop = nullptr);

int f32_variant_count();
TileShape f32_variant(int index);
const char* f32_variant_name(int bits, int index);
hipError_t launch_gemm_f32(int bits, int variant, const GemmArgs& args, hipStream_t stream,
                           hipEvent_t start = nullptr, hipEvent_t stop = nullptr);

// Fused Conformer convolution tail (pk_conv.hip). Element type of input,
// weights and output is f16 or f32; scale/shift are f32.
struct ConvArgs {
  const void* input;              // [batch * frames, 2 * channels]: values, then gates
  const void* weights;            // [9, channels]
  const float* scale;             // [channels] folded batch-norm scale
  const float* shift;             // [channels] folded batch-norm shift
  const uint32_t* valid_lengths;  // [batch]
  void* output;                   // [batch * frames, channels]
  uint32_t frames;
  uint32_t channels;              // multiple of 8
  int input_glu;                  // input is [batch * frames, channels] GLU
  uint32_t runs;                  // frame runs per item (set by the launcher)
  uint32_t blocks_per_item;       // set by the launcher
};

struct ConvGeometry {
  const char* name;
  int channels_per_thread;
  uint32_t runs;
  uint32_t blocks_per_item;
  uint32_t grid;
  uint32_t block_threads;
};

// Relative-position attention (pk_attention.hip), 8 heads x 128 channels.
constexpr uint32_t kAttentionMaxFrames = 4096;
struct AttnArgs {
  const void* qkv;                // [batch * frames, 3072]: Q, K, V blocks of 1024
  const void* positions;          // [8][32][2T-1][4], or [2T-1, 1024] with positions_row_major
  const float* bias_u;            // [8, 128]
  const float* bias_v;            // [8, 128]
  const uint32_t* valid_lengths;  // [batch]
  void* output;                   // [batch * frames, 1024]
  uint32_t frames;
  uint32_t position_rows;         // 2 * frames - 1
  int positions_row_major;
  uint32_t query_tiles;           // set by the launcher
  uint32_t work_items;            // (window, head, query tile) items, set by the launcher
};

struct AttnGeometry {
  const char* name;
  uint32_t query_tiles;
  uint32_t grid;
  uint32_t block_threads;
  uint32_t lds_bytes;
};

int attention_variant_count(bool f16);
// Planned launch shape: key-split 32-query tiles for windows up to 256
// frames while their workgroups fill about one round of the device, shared
// K/V/position tiles beyond (longer windows or more windows).
int attention_default_variant(bool f16, uint32_t frames, uint32_t batch);
AttnGeometry attention_geometry(bool f16, int variant, uint32_t frames, uint32_t batch);
hipError_t launch_attention(bool f16, int variant, const AttnArgs& args, uint32_t batch, hipStream_t stream,
                            hipEvent_t start = nullptr, hipEvent_t stop = nullptr);

// Row LayerNorm (pk_layernorm.hip).
struct LayerNormArgs {
  const void* input;   // [rows, channels]
  const float* gamma;  // [channels]
  const float* beta;   // [channels]
  void* output;        // [rows, channels]; may be the input
  uint32_t rows;       // active rows
  uint32_t channels;   // multiple of 4
  float epsilon;
  // Chained LayerNorm (null next_output: none): next_output =
  // LayerNorm(output as stored) with next_gamma / next_beta and the same
  // epsilon; rows of at most kLayerNormChainBytes.
  const float* next_gamma;
  const float* next_beta;
  void* next_output;
};
constexpr uint32_t kLayerNormChainBytes = 4096;
uint32_t layernorm_grid(uint32_t rows);
hipError_t launch_layernorm(bool f16, const LayerNormArgs& args, hipStream_t stream, hipEvent_t start = nullptr,
                            hipEvent_t stop = nullptr);

// Subsampling front end convolutions (pk_subsampling.hip).
enum SubsamplingKind { kSubsamplingFused = 0, kSubsamplingDepthwise = 1, kSubsamplingMask = 2 };
struct SubsamplingArgs {
  const void* input;             // fused: f32 [batch, width, height]; depthwise: [batch, H, W, C]
  const void* weights;           // conv0 (fused) or depthwise [3, 3, C]
  const float* bias;             // [C]
  const void* weights2;          // fused: depthwise2 [3, 3, C]
  const float* bias2;            // fused: [C]
  void* output;                  // [batch, out_height, out_width, C]; mask: values in place
  const uint32_t* valid_lengths; // raw feature frames, from valid_offset
  uint32_t height, width;        // input (mask: values) spatial shape
  uint32_t mid_height, mid_width;  // fused: conv0 shape
  uint32_t out_height, out_width;
  uint32_t channels;
  uint32_t valid_offset;
  uint32_t steps;                // depthwise and mask
};
struct SubsamplingGeometry {
  const char* name;
  uint32_t grid[3];
  uint32_t block_threads;
  uint32_t lds_bytes;
};
SubsamplingGeometry subsampling_geometry(int kind, bool f16, const SubsamplingArgs& args, uint32_t batch);
hipError_t launch_subsampling(int kind, bool f16, const SubsamplingArgs& args, uint32_t batch, hipStream_t stream,
                              hipEvent_t start = nullptr, hipEvent_t stop = nullptr);

// Greedy TDT decoder (pk_tdt.hip).
constexpr uint32_t kTdtHidden = 640;
constexpr uint32_t kTdtGates = 2560;
constexpr uint32_t kTdtHead = 1032;
constexpr uint32_t kTdtBlank = 1024;
constexpr uint32_t kTdtThreads = 640;
struct TdtArgs {
  // Weights and encoder rows are f16 in the f16 profile and f32 in the f32
  // profile (launch_tdt_decode's `f32`); biases, state and scratch are f32.
  const void* embedding;         // [1025, 640]
  const void* lstm[2];           // [1280, 2560] k by ifgo
  const float* lstm_bias[2];     // [2560]
  const void* projector;         // [640, 640] k by output
  const float* projector_bias;   // [640]
  const void* head;              // [640, 1032] k by output
  const float* head_bias;        // [1032]
  const void* encoder;           // [batch, frames, 640]
  const uint32_t *lengths, *starts, *ends, *flush;  // [batch]
  float* state;                  // [batch, 4, 640]: h0, c0, h1, c1
  float* scratch;                // [batch, 5, 640]: candidates and projection
  uint32_t *tokens, *token_frames, *token_durations;  // [batch, max_tokens]
  uint32_t *counts, *status;     // [batch]
  uint32_t frames, max_tokens;
};
// One workgroup per window; `f32` selects the f32 profile's kernel.
hipError_t launch_tdt_decode(const TdtArgs& args, uint32_t batch, bool f32, hipStream_t stream,
                             hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// Team decoding (f16 profile): `members` workgroups of kTdtTeamThreads per
// window, each streaming one slice of every weight matrix, meeting at
// bounded barriers in global memory; an ordinary launch whose grid fits the
// workgroups the device holds at once.
constexpr uint32_t kTdtTeamThreads = 256;
constexpr uint32_t kTdtSyncTimeout = 2u;  // status bit: a team barrier gave up waiting
constexpr uint32_t kTdtSyncStride = 64;   // u32 words between barrier counters (256 bytes)
struct TdtTeam {
  uint32_t members;     // 8 or 16
  uint32_t* sync;       // [2 * capacity * kTdtSyncStride]: counters, then abort flags; zeroed per launch
  uint32_t* partials;   // [capacity, 2, members, 4]: per-member argmax partials, two buffers
  uint32_t capacity;    // windows the buffers hold
  uint32_t spin_limit;  // polls before a barrier gives up
};
bool tdt_team_members_supported(uint32_t members);
// Team workgroups that can be resident at once on `device` (0 if unknown).
uint32_t tdt_team_capacity(int device);
hipError_t launch_tdt_team(const TdtArgs& args, const TdtTeam& team, uint32_t batch, hipStream_t stream,
                           hipEvent_t start = nullptr, hipEvent_t stop = nullptr);

int conv_variant_count(bool f16);
ConvGeometry conv_geometry(bool f16, int variant, uint32_t frames, uint32_t channels, uint32_t batch,
                           bool input_glu = false);
hipError_t launch_conformer_conv(bool f16, int variant, const ConvArgs& args, uint32_t batch,
                                 hipStream_t stream, hipEvent_t start = nullptr, hipEvent_t stop = nullptr);

}  // namespace pk

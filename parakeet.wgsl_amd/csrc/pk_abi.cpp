// pk_abi.cpp - C ABI of the palette GEMM library: contexts, memory, streams,
// the reference's descriptor contract checks and launch planning.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "pk_abi_internal.h"
#include "pk_internal.h"
#include "pk_palette.h"

namespace pk_abi {

thread_local std::string g_error;

int fail(int status, const char* fmt, ...) {
  char buffer[512];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buffer, sizeof buffer, fmt, args);
  va_end(args);
  g_error = buffer;
  return status;
}

int check_ctx(const pk_context* ctx) {
  if (!ctx) return fail(PK_INVALID_ARGUMENT, "context is null");
  if (ctx->destroyed.load()) return fail(PK_DESTROYED, "context was destroyed");
  return PK_OK;
}

pk_context* ctx_retain(pk_context* ctx) {
  if (ctx) ctx->refs.fetch_add(1);
  return ctx;
}

void ctx_release(pk_context* ctx) {
  if (!ctx || ctx->refs.fetch_sub(1) != 1) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

}  // namespace pk_abi

using namespace pk_abi;

namespace {

const char* safe_label(const char* label) { return label ? label : "palette-gemm"; }

// The 14 fixed production signatures (src/webgpu/kernels/gemm.ts:204-356;
// the FP32 registry :2154-2306 has the same signatures). residual_scale < 0
// means "no residual".
struct Signature {
  const char* label;
  uint32_t rows, inner, columns;
  int activation;
  bool bias;
  float residual_scale;
};
constexpr Signature kProductionSignatures[] = {
    {"encoder-layer-ff-expand", 7520, 1024, 4096, PK_ACTIVATION_SILU, false, -1.0f},
    {"encoder-layer-ff-contract", 7520, 4096, 1024, PK_ACTIVATION_NONE, false, 0.5f},
    {"encoder-layer-attention-qkv", 7520, 1024, 3072, PK_ACTIVATION_NONE, false, -1.0f},
    {"encoder-layer-residual-1024", 7520, 1024, 1024, PK_ACTIVATION_NONE, false, 1.0f},
    {"encoder-layer-convolution-expand", 7520, 1024, 2048, PK_ACTIVATION_NONE, false, -1.0f},
    {"encoder-projector", 7520, 1024, 640, PK_ACTIVATION_NONE, true, -1.0f},
    {"subsampling-pointwise3", 12032, 256, 256, PK_ACTIVATION_RELU, true, -1.0f},
    {"subsampling-pointwise3-b2", 24064, 256, 256, PK_ACTIVATION_RELU, true, -1.0f},
    {"subsampling-pointwise3-b3", 36096, 256, 256, PK_ACTIVATION_RELU, true, -1.0f},
    {"subsampling-pointwise6", 3008, 256, 256, PK_ACTIVATION_RELU, true, -1.0f},
    {"subsampling-pointwise6-b2", 6016, 256, 256, PK_ACTIVATION_RELU, true, -1.0f},
    {"subsampling-pointwise6-b3", 9024, 256, 256, PK_ACTIVATION_RELU, true, -1.0f},
    {"subsampling-flatten-project", 188, 4096, 1024, PK_ACTIVATION_NONE, true, -1.0f},
    {"subsampling-flatten-project-b2", 376, 4096, 1024, PK_ACTIVATION_NONE, true, -1.0f},
    {"subsampling-flatten-project-b3", 564, 4096, 1024, PK_ACTIVATION_NONE, true, -1.0f},
};

const char* activation_name(int a) {
  return a == PK_ACTIVATION_SILU ? "silu" : a == PK_ACTIVATION_RELU ? "relu" : "none";
}

}  // namespace

struct pk_prepared_weight {
  pk_abi::CtxRef ctx;
  std::string label;
  int bits = 5;
  uint32_t inner = 0, columns = 0;
  uint32_t* codes = nullptr;      // operand-order codes (device), split into `parts` K parts
  int parts = 1;                  // the one layout held: what the planned kernel reads
  uint64_t bytes = 0;
  bool glu = false;               // column blocks interleaved for the GLU epilogue
  std::atomic<int> refs{1};
  bool owner_released = false;
};

struct pk_gemm_op {
  pk_abi::CtxRef ctx;
  std::string label;
  int precision = PK_PRECISION_F16;
  int bits = 5;
  uint32_t rows = 0;
  pk::GemmArgs args{};
  pk_prepared_weight* weight = nullptr;
  int variant = 0;
  uint32_t splits = 1;
  int cus = 256;
  bool cached_output = false;  // PK_GEMM_CACHED_OUTPUT
  // A variant chosen by pk_gemm_set_variant / pk_gemm_set_splits runs at
  // every active row count; otherwise an active prefix is re-planned among
  // the kernels that read the weight's layout (the last choice cached).
  bool forced = false;
  uint32_t active_rows_planned = 0;
  int active_variant = 0;
  // Split-K workspace: f32 partial tiles, then one counter per tile.
  void* workspace = nullptr;
  uint64_t workspace_bytes = 0;
  // Fused row LayerNorm (PK_GEMM_ROW_NORM): G and B [2N] f32, then f16 gamma [K].
  void* norm_buffer = nullptr;
  // Active row counts given to pk_gemm_prepare_rows: the variant a
  // dedicated op of that many rows plans and the codes it reads (the
  // weight's own layout, or one of `layouts`: the same codes split into 1,
  // 2 or 4 K parts, owned by the op).
  struct RowPlan {
    int variant;
    const uint32_t* codes;
  };
  std::map<uint32_t, RowPlan> row_plans;
  uint32_t* layouts[3] = {};
  uint64_t layout_bytes = 0;
  bool shared_weight = false;  // created over a pk_prepared_weight of the caller
  bool destroyed = false;
};

uint64_t pk_abi::gemm_weight_bytes(const pk_gemm_op* op) {
  return op && op->weight ? op->weight->bytes + op->layout_bytes : 0;
}

namespace {

void weight_unref(pk_prepared_weight* w) {
  if (!w) return;
  if (w->refs.fetch_sub(1) == 1) {
    free_after_drain(w->ctx->device, w->codes);
    delete w;
  }
}

// Prepares a packed weight in the one layout its kernel reads: the codes in
// operand order split into `parts` K parts (pk_internal.h), with `glu` the
// value and gate column blocks interleaved (the GLU epilogue runs in the
// pair-code kernels alone).
int make_weight(pk_context* ctx, const char* label, int bits, uint32_t inner, uint32_t columns,
                const uint32_t* packed, hipStream_t stream, pk_prepared_weight** out, bool glu = false,
                int parts = 1) {
  auto* w = new pk_prepared_weight();
  w->ctx = ctx;
  w->label = safe_label(label);
  w->bits = bits;
  w->inner = inner;
  w->columns = columns;
  w->glu = glu;
  w->parts = parts;
  w->bytes = pk::operand_order_words(bits, inner, columns, parts) * 4u;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&w->codes), w->bytes);
  if (e != hipSuccess) {
    const unsigned long long want = (unsigned long long)w->bytes;
    delete w;
    return fail(PK_ALLOCATION_FAILURE, "%s: cannot allocate %llu bytes of prepared palette codes: %s",
                safe_label(label), want, hipGetErrorString(e));
  }
  e = pk::launch_to_operand_order(bits, packed, inner, columns, w->codes, stream, glu, parts);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) {
    (void)hipFree(w->codes);
    delete w;
    return fail(PK_DEVICE_ERROR, "%s: palette code preparation failed: %s", safe_label(label),
                hipGetErrorString(e));
  }
  *out = w;
  return PK_OK;
}

// Moves an op's own weight to the layout of `parts` (a variant switch to a
// kernel that reads another split): the new layout is derived on the device
// from the old one, which is then freed, so the weight still holds one.
int relayout_weight(pk_prepared_weight* w, int parts, hipStream_t stream) {
  if (w->parts == parts) return PK_OK;
  const uint64_t bytes = pk::operand_order_words(w->bits, w->inner, w->columns, parts) * 4u;
  uint32_t* codes = nullptr;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&codes), bytes);
  if (e != hipSuccess)
    return fail(PK_ALLOCATION_FAILURE, "%s: cannot allocate %llu bytes of prepared palette codes: %s",
                w->label.c_str(), (unsigned long long)bytes, hipGetErrorString(e));
  const uint64_t blocks = (uint64_t)(pk::padded_columns(w->columns) / 32u) * (pk::padded_inner(w->inner) / 64u);
  e = pk::launch_relayout(w->bits, w->codes, w->parts, codes, parts, blocks, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) {
    (void)hipFree(codes);
    return fail(PK_DEVICE_ERROR, "%s: palette code relayout failed: %s", w->label.c_str(), hipGetErrorString(e));
  }
  free_after_drain(w->ctx->device, w->codes);
  w->codes = codes;
  w->parts = parts;
  w->bytes = bytes;
  return PK_OK;
}

int variant_parts(int precision, int variant) {
  return precision == PK_PRECISION_F16 ? pk::f16_variant_parts(variant) : 1;
}

// Packed-code contract of requireGemmShape (gemm.ts:997-1010) and
// validatePalettePair (runtime-plan.ts:529-588).
int check_packed(const char* label, int bits, uint32_t inner, uint32_t columns, uint64_t packed_bytes) {
  const uint64_t scalars = (uint64_t)inner * columns;
  const uint32_t cpg = pk::codes_per_group(bits);
  if (scalars % cpg != 0 || columns % cpg != 0)
    return fail(PK_INVALID_ARGUMENT, "%s palette codes are not group aligned", label);
  const uint64_t expected = scalars / cpg * pk::words_per_group(bits) * 4u;
  if (packed_bytes != expected)
    return fail(PK_INVALID_ARGUMENT, "%s has invalid packed palette indices", label);
  return PK_OK;
}

pk::TileShape shape_of(int precision, int variant) {
  return precision == PK_PRECISION_F16 ? pk::f16_variant(variant) : pk::f32_variant(variant);
}

uint32_t k_blocks(uint32_t inner) { return (inner + 63u) / 64u; }

// f16 outputs are stored non-temporally unless the op keeps them cached
// (GemmArgs::stream_out).
bool stream_outputs(const pk_gemm_op* op) { return op->precision == PK_PRECISION_F16 && !op->cached_output; }

// Column-group widths (blocks of 32 columns) a GEMM group keeps item lists
// for: those of the small-M variants.
constexpr uint32_t kGroupWidths[3] = {1u, 2u, 4u};

int group_width_index(uint32_t column_blocks) {
  for (int i = 0; i < 3; ++i)
    if (kGroupWidths[i] == column_blocks) return i;
  return -1;
}

// Compulsory HBM bytes of one launch over `rows` rows: the packed codes at
// the format's density, the palettes, A, the output (+ bias, residual).
uint64_t algorithmic_bytes(const pk::GemmArgs& a, int bits, uint64_t rows, uint32_t elem) {
  const uint64_t K = a.inner, N = a.columns;
  uint64_t bytes = (K * N * (uint64_t)bits + 7u) / 8u;
  bytes += (uint64_t)a.palette_groups * (1u << bits) * elem;
  bytes += rows * K * elem + rows * (a.glu ? N / 2u : N) * elem;
  if (a.bias) bytes += 4u * N;
  if (a.residual) bytes += rows * N * elem;
  return bytes;
}

// Split-K workspace: `splits` f32 partial tiles per output tile, then one
// u32 arrival counter per output tile (256-byte aligned).
uint64_t workspace_bytes_for(const pk::TileShape& s, uint32_t rows, uint32_t columns, uint32_t splits) {
  if (splits <= 1) return 0;
  const uint64_t tiles = (uint64_t)pk::tiles_m(s, rows) * pk::tiles_n(s, columns);
  const uint64_t partial = tiles * splits * s.tile_elements() * 4u;
  return (partial + 255u) / 256u * 256u + tiles * 4u;
}

struct Plan {
  int variant;
  uint32_t splits;
};

// The compiled variant of a family with a given tile shape (-1 if none).
int find_variant(int precision, int family, int waves_m, int waves_n, int m_blocks, int n_blocks,
                 int k_split = 1) {
  const int count = precision == PK_PRECISION_F16 ? pk::f16_variant_count() : pk::f32_variant_count();
  for (int i = 0; i < count; ++i) {
    const pk::TileShape s = shape_of(precision, i);
    const int f = precision == PK_PRECISION_F16 ? pk::f16_variant_family(i) : 0;
    if (f == family && s.waves_m == waves_m && s.waves_n == waves_n && s.m_blocks == m_blocks &&
        s.n_blocks == n_blocks && s.k_split == k_split)
      return i;
  }
  return -1;
}

// Launch planner. The f16 choice follows MI355X measurements of every
// compiled tile shape over the encoder's GEMM shapes (M 1..3008, K
// 1024/4096, N 1024..4096, the rel-pos linear's 2T-1 rows). Up to 64 rows,
// and up to 256 rows of a deep-K (K >= 2048) or at most 1024 columns wide
// GEMM, the small-M kernel (32-row blocks, K round robin over eight
// wavefronts) wins (output projection at 188 rows: 5.96 us against 7.88 us
// for the 64 x 64 pair-code tile); up to 256 rows otherwise the 64 x 64
// pair-code tile (FF expand at 188 rows: 8.30 us against 8.84 us for the
// best small-M shape); deep-K shapes take 96 x 64 while
// those fill the chip and 96 x 128 beyond. Every other shape takes the
// candidate with the least (rounds of workgroups) x (measured time of one
// workgroup), which puts 192 x 128 on the FF expand and convolution PW1,
// 96 x 128 on 3000-row 1024-wide GEMMs, 64 x 64 on 752 x 1024 and the
// small-M kernel on the 375-row rel-pos linear; 96 x 128 also takes shapes
// whose larger tiles would leave a costly partial round (3000-row QKV).
// f32 keeps its own smallest-cost shape.
Plan plan_launch(int precision, uint32_t rows, uint32_t inner, uint32_t columns, int cus) {
  if (precision == PK_PRECISION_F16) {
    auto pair_variant = [](int wn, int r, int c, int ks) {
      const int v = find_variant(PK_PRECISION_F16, pk::kFamilyPairCode, 1, wn, r, c, ks);
      return v < 0 ? 0 : v;
    };
    auto tiles = [&](int tile_rows, int tile_columns) {
      return (uint64_t)((rows + tile_rows - 1) / tile_rows) * ((columns + tile_columns - 1) / tile_columns);
    };
    const uint64_t wave = (uint64_t)cus;
    if (rows <= 64u || (rows <= 256u && inner >= 2048u)) {
      const int v = find_variant(PK_PRECISION_F16, pk::kFamilySmallM, 1, 1, 1, 1, 8);
      return {v < 0 ? 0 : v, 1u};
    }
    if (rows <= 256u) {
      if (columns <= 1024u) {
        const int v = find_variant(PK_PRECISION_F16, pk::kFamilySmallM, 1, 1, 1, 1, 8);
        if (v >= 0) return {v, 1u};
      }
      return {pair_variant(1, 2, 2, 4), 1u};
    }
    if (inner >= 2048u) return {tiles(96, 64) <= wave ? pair_variant(1, 3, 2, 4) : pair_variant(2, 3, 2, 2), 1u};
    // K <= 256 (the subsampling pointwise convolutions, K = N = 256 over
    // tens of thousands of rows): a workgroup's fixed costs outweigh its K
    // loop, so the K = 1024 figures below mislead. Measured on one MI355X:
    // 48,128 rows 17.8 us on one round of 192 x 256 against 20.0 us for
    // 96 x 128 and 23.7 us for 192 x 128; 192,512 rows 64.0 us for the
    // 96 x 128 queue against 65.2 us for 192 x 256 and 83.2 us for 192 x 128.
    if (inner <= 256u) {
      const uint64_t wide = tiles(192, 256);
      if (columns >= 256u && 2u * wide > wave && wide <= wave) {
        const int v = find_variant(PK_PRECISION_F16, pk::kFamilyPairCode, 1, 4, 6, 2, 1);
        if (v >= 0) return {v, 1u};
      }
      if (tiles(96, 128) > wave) return {pair_variant(2, 3, 2, 2), 1u};
    }
    // K < 2048: the fewest rounds of workgroups times the measured time of one
    // workgroup of each tile at K = 1024 with one workgroup per compute unit.
    struct Candidate {
      int wn, r, c, ks;  // pair-code shape; wn = 0 marks the small-M RW = 2 kernel
      int tile_rows, tile_columns;
      double us;
    };
    // The 192 x 256 and 160 x 256 tiles without a K split (four wavefronts of
    // 192 or 160 x 64) measured 28.5 and 26.8 us per workgroup; they are
    // candidates for the wide GEMMs at K = 1024 only (N >= 3072, and N >= 4096
    // for 160 x 256), where they were measured against the others: FF expand
    // 3008 x 1024 x 4096 34.7 us against 42.1 us for two rounds of 192 x 128
    // and 50.8 us for two rounds of 160 x 256; at 7520 rows 81.4 us on three
    // rounds of 160 x 256 against 88.4 us on three of 192 x 256 (inside the
    // encoder pass, same box); QKV 3008 x 1024 x 3072 29.2 us on 192
    // workgroups of 192 x 256 against 30.3 us for 96 x 128, and with the
    // non-temporal output stores 27.1 us on 228 workgroups of 160 x 256
    // against 27.6 us on 192 x 256 inside the encoder pass (three runs each,
    // interleaved on one box; pass 7.13 against 7.16 ms).
    constexpr Candidate kCandidates[] = {
        {2, 6, 2, 2, 192, 128, 22.3}, {2, 4, 2, 2, 128, 128, 17.2}, {2, 3, 2, 2, 96, 128, 14.8},
        {1, 3, 2, 4, 96, 64, 11.0},   {1, 2, 2, 4, 64, 64, 9.3},    {0, 2, 1, 8, 64, 32, 8.2},
        {4, 6, 2, 1, 192, 256, 28.5}, {4, 5, 2, 1, 160, 256, 26.8},
    };
    int best = -1;
    double best_us = 1e300;
    for (const Candidate& c : kCandidates) {
      if (c.tile_columns == 256 && (columns < 3072u || inner < 1024u)) continue;
      if (c.tile_columns == 256 && c.tile_rows == 160 && columns < 3072u) continue;
      const int v = c.wn ? find_variant(PK_PRECISION_F16, pk::kFamilyPairCode, 1, c.wn, c.r, c.c, c.ks)
                         : find_variant(PK_PRECISION_F16, pk::kFamilySmallM, 1, 1, c.r, 1, 8);
      if (v < 0) continue;
      const double rounds = (double)((tiles(c.tile_rows, c.tile_columns) + wave - 1) / wave);
      if (rounds * c.us < best_us * 0.98) {
        best_us = rounds * c.us;
        best = v;
      }
    }
    // Two 96 x 128 workgroups share a compute unit (their registers and
    // 54 KB of LDS allow it), so beyond one round that tile runs as a fluid
    // queue: measured 10.2 us per workgroup per compute unit at K = 1024
    // (QKV 3008 x 1024 x 3072: 768 tiles in 30.5 us against 36.6 us for
    // 2 rounds of 192 x 128). It replaces a choice that leaves a partial
    // round when it is predicted at least 15% faster.
    const uint64_t t96 = tiles(96, 128);
    if (t96 > wave) {
      const double fluid_us = 10.2 * (double)t96 / (double)wave;
      const int v = pair_variant(2, 3, 2, 2);
      if (fluid_us < 0.85 * best_us) best = v;
    }
    return {best < 0 ? pair_variant(2, 6, 2, 2) : best, 1u};
  }
  // f32: the largest tile that still fills the compute units.
  const int count = pk::f32_variant_count();
  int best = 0;
  double best_cost = 1e300;
  for (int i = 0; i < count; ++i) {
    const pk::TileShape s = shape_of(precision, i);
    const double tiles = (double)pk::tiles_m(s, rows) * pk::tiles_n(s, columns);
    const double rounds = std::ceil(tiles / cus);
    const double cost = rounds * s.tile_rows() * s.tile_columns() * (1.0 + 0.25 / s.m_blocks);
    if (cost < best_cost * 0.999) {
      best_cost = cost;
      best = i;
    }
  }
  return {best, 1u};
}

// The pair-code tile with K split `ks` (the layout of that many parts) that
// takes `rows` x `columns` in the least (rounds of workgroups) x (time of one
// workgroup at K = 1024: measured for the tiles the unrestricted plan uses,
// scaled by tile area for the others); -1 if none.
int best_pair_tile(uint32_t rows, uint32_t columns, int cus, bool glu, int ks) {
  struct Tile {
    int wn, ks, r, c;
    double us;
  };
  constexpr Tile kTiles[] = {
      {4, 1, 6, 2, 28.5}, {4, 1, 4, 2, 20.0}, {4, 1, 3, 2, 16.0}, {4, 1, 6, 1, 20.0},  // one part
      {2, 2, 6, 2, 22.3}, {2, 2, 4, 2, 17.2}, {2, 2, 3, 2, 14.8}, {2, 2, 6, 1, 14.0},  // two parts
      {1, 4, 4, 2, 13.0}, {1, 4, 3, 2, 11.0}, {1, 4, 2, 2, 9.3},                       // four parts
  };
  int best = -1;
  double best_us = 1e300;
  for (const Tile& t : kTiles) {
    if (t.ks != ks) continue;
    const int v = find_variant(PK_PRECISION_F16, pk::kFamilyPairCode, 1, t.wn, t.r, t.c, t.ks);
    if (v < 0) continue;
    const pk::TileShape s = pk::f16_variant(v);
    if (glu && (s.tile_columns() / 32) % 2 != 0) continue;
    const uint64_t tiles = (uint64_t)pk::tiles_m(s, rows) * pk::tiles_n(s, columns);
    const double us = (double)((tiles + cus - 1) / cus) * t.us;
    if (us < best_us * 0.98) {
      best_us = us;
      best = v;
    }
  }
  return best;
}

// The plan of one op: plan_launch, with a GLU epilogue or a fused row norm
// moved to the pair-code kernels (small-M plans take their 64 x 64 tile), and with a
// shared prepared weight restricted to the tiles that read the layout it
// holds (`required_parts`, 0 = any).
Plan plan_op(int precision, uint32_t rows, uint32_t inner, uint32_t columns, int cus, bool glu,
             int required_parts, bool pair_only = false) {
  Plan plan = plan_launch(precision, rows, inner, columns, cus);
  if ((glu || pair_only) && pk::f16_variant_family(plan.variant) != pk::kFamilyPairCode)
    plan = {find_variant(PK_PRECISION_F16, pk::kFamilyPairCode, 1, 1, 2, 2, 4), 1u};
  if (required_parts && variant_parts(precision, plan.variant) != required_parts) {
    if (required_parts == 1 && !glu && (rows <= 64u || (rows <= 256u && inner >= 2048u))) {
      const int v = find_variant(PK_PRECISION_F16, pk::kFamilySmallM, 1, 1, 2, 1, 8);  // small-M 64 x 32
      if (v >= 0) return {v, 1u};
    }
    const int v = best_pair_tile(rows, columns, cus, glu, required_parts);
    if (v >= 0) plan = {v, 1u};
  }
  return plan;
}

// Applies a (variant, splits) choice: resizes the split-K workspace for the
// op's row capacity and zeroes its counters.
int configure_launch(pk_gemm_op* op, int variant, uint32_t splits) {
  const pk::TileShape s = shape_of(op->precision, variant);
  if (splits > 1 && !(op->precision == PK_PRECISION_F16 && pk::f16_variant_splits(variant)))
    return fail(PK_RANGE_ERROR, "%s tile variant %d has no split-K path", op->label.c_str(), variant);
  const uint64_t need = workspace_bytes_for(s, op->rows, op->args.columns, splits);
  PK_HIP(hipSetDevice(op->ctx->device), "hipSetDevice");
  if (need != op->workspace_bytes) {
    if (op->workspace) {
      PK_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
      PK_HIP(hipFree(op->workspace), "hipFree");
      op->workspace = nullptr;
      op->workspace_bytes = 0;
    }
    if (need) {
      const hipError_t e = hipMalloc(&op->workspace, need);
      if (e != hipSuccess)
        return fail(PK_ALLOCATION_FAILURE, "%s: cannot allocate %llu bytes of split-K workspace: %s",
                    op->label.c_str(), (unsigned long long)need, hipGetErrorString(e));
      op->workspace_bytes = need;
    }
  }
  if (op->workspace) {
    const uint64_t tiles = (uint64_t)pk::tiles_m(s, op->rows) * pk::tiles_n(s, op->args.columns);
    const uint64_t counters_at = need - tiles * 4u;
    PK_HIP(hipMemset(static_cast<uint8_t*>(op->workspace) + counters_at, 0, tiles * 4u), "hipMemset");
    op->args.partials = static_cast<float*>(op->workspace);
    op->args.counters = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(op->workspace) + counters_at);
  } else {
    op->args.partials = nullptr;
    op->args.counters = nullptr;
  }
  op->variant = variant;
  op->splits = splits;
  op->args.splits = splits;
  return PK_OK;
}

// The descriptor contract of createDispatch: requireGemmShape,
// requireProductionSpecialization and requireRuntimeWeight
// (src/webgpu/kernels/gemm.ts:971-1161; FP32 twins :3342-3557) plus the
// binding sizes and vector alignment the kernels rely on. Host-only: ctx
// may be null (pk_gemm_validate), then the prepared weight's context is not
// compared.
int validate_gemm_desc(const pk_context* ctx, const pk_gemm_desc* d) {
  if (!d) return fail(PK_INVALID_ARGUMENT, "GEMM descriptor is null");
  if (d->struct_size != sizeof(pk_gemm_desc))
    return fail(PK_INVALID_ARGUMENT, "pk_gemm_desc.struct_size mismatch");
  const char* label = safe_label(d->label);
  const bool f16 = d->precision == PK_PRECISION_F16;
  if (!f16 && d->precision != PK_PRECISION_F32)
    return fail(PK_INVALID_ARGUMENT, "%s has an unsupported precision %d", label, d->precision);
  const uint32_t elem = f16 ? 2u : 4u;
  // requireGemmShape (gemm.ts:971-983; FP32 twin N%4)
  if (d->rows == 0 || d->inner == 0 || d->inner % 32u != 0 || d->columns == 0 ||
      d->columns % (f16 ? 8u : 4u) != 0)
    return fail(PK_RANGE_ERROR, "Unsupported %sGEMM shape for %s", f16 ? "" : "FP32 ", label);
  if (d->palette_bits != 5 && d->palette_bits != 6)
    return fail(PK_INVALID_ARGUMENT, "%s has an unsupported weight format", label);
  const int bits = d->palette_bits;
  // requireProductionSpecialization (gemm.ts:1031-1067)
  if (!d->residual && d->has_residual_scale)
    return fail(PK_INVALID_ARGUMENT, "%s supplies a residual scale without a residual", label);
  if (d->activation < PK_ACTIVATION_NONE || d->activation > PK_ACTIVATION_RELU)
    return fail(PK_INVALID_ARGUMENT, "%s has an unsupported activation %d", label, d->activation);
  const float residual_scale = d->residual ? (d->has_residual_scale ? d->residual_scale : 1.0f) : -1.0f;
  if (d->flags & ~(PK_GEMM_REQUIRE_PRODUCTION_SIGNATURE | PK_GEMM_GLU | PK_GEMM_ROW_NORM | PK_GEMM_CACHED_OUTPUT))
    return fail(PK_INVALID_ARGUMENT, "%s has unknown flags 0x%x", label, d->flags);
  if (d->flags & PK_GEMM_REQUIRE_PRODUCTION_SIGNATURE) {
    bool found = false;
    for (const Signature& s : kProductionSignatures)
      if (s.rows == d->rows && s.inner == d->inner && s.columns == d->columns &&
          s.activation == d->activation && s.bias == (d->bias != nullptr) &&
          s.residual_scale == residual_scale)
        found = true;
    if (!found) {
      char scale[32];
      if (d->residual)
        std::snprintf(scale, sizeof scale, "%g", residual_scale);
      else
        std::snprintf(scale, sizeof scale, "none");
      return fail(PK_INVALID_ARGUMENT,
                  "%s is not a fixed production GEMM signature: M=%u, K=%u, N=%u, "
                  "activation=%s, bias=%s, residualScale=%s",
                  label, d->rows, d->inner, d->columns, activation_name(d->activation),
                  d->bias ? "true" : "false", scale);
    }
  }
  // f16SubgroupGemmWgsl (gemm.ts:1372-1378)
  if (d->bias && d->residual)
    return fail(PK_INVALID_ARGUMENT, "%s cannot fuse bias and residual together", label);
  const bool glu = (d->flags & PK_GEMM_GLU) != 0;
  if (glu && (!f16 || d->palette_groups != 1 || d->columns % 64u != 0 || d->bias || d->residual ||
              d->activation != PK_ACTIVATION_NONE || d->prepared))
    return fail(PK_INVALID_ARGUMENT,
                "%s GLU epilogue needs f16, one palette group, N %% 64 == 0, no bias, activation, residual "
                "or shared prepared weight",
                label);
  const bool norm = (d->flags & PK_GEMM_ROW_NORM) != 0;
  if (norm) {
    if (!f16 || glu || d->prepared || d->inner % 64u != 0 || d->inner > pk::kNormMaxInner ||
        (d->palette_groups != 1 && d->palette_group_columns % 256u != 0))
      return fail(PK_INVALID_ARGUMENT,
                  "%s row norm needs f16, K %% 64 == 0, K <= %u, packed codes, no GLU epilogue and one palette "
                  "group or groups of a multiple of 256 columns",
                  label, pk::kNormMaxInner);
    const uint64_t need = (uint64_t)d->inner * 4u;
    if (!d->norm_gamma || !d->norm_beta || d->norm_gamma_bytes < need || d->norm_beta_bytes < need ||
        !aligned(d->norm_gamma, 4) || !aligned(d->norm_beta, 4) || !(d->norm_epsilon >= 0.0f))
      return fail(PK_INVALID_ARGUMENT, "%s row norm needs gamma and beta of %llu bytes and epsilon >= 0", label,
                  (unsigned long long)need);
  }
  // requireRuntimeWeight (gemm.ts:1069-1161): palette geometry and storage
  const uint32_t entries = 1u << bits;
  const uint32_t cpg = pk::codes_per_group(bits);
  if (d->palette_groups == 0 || d->palette_group_columns == 0 ||
      (uint64_t)d->palette_group_columns * d->palette_groups != d->columns ||
      d->palette_group_columns % cpg != 0 || !d->palette ||
      d->palette_bytes != (uint64_t)d->palette_groups * entries * elem || !aligned(d->palette, elem))
    return fail(PK_INVALID_ARGUMENT, "%s has invalid transient palette weights", label);
  if (d->prepared) {
    const pk_prepared_weight* w = d->prepared;
    if (w->owner_released || w->bits != bits || w->inner != d->inner || w->columns != d->columns ||
        (ctx && w->ctx != ctx))
      return fail(PK_INVALID_ARGUMENT, "%s has a mismatched prepared palette weight", label);
  } else {
    if (int s = check_packed(label, bits, d->inner, d->columns, d->packed_bytes)) return s;
    if (!d->packed || !aligned(d->packed, 4))
      return fail(PK_INVALID_ARGUMENT, "%s has invalid packed palette indices", label);
  }
  // Bindings: sizes (gemm.ts:1302-1333 minBindingSize) and vector alignment.
  const uint64_t a_need = (uint64_t)d->rows * d->inner * elem;
  const uint64_t c_need = (uint64_t)d->rows * (glu ? d->columns / 2u : d->columns) * elem;
  if (!d->a || d->a_bytes < a_need || !aligned(d->a, 16))
    return fail(PK_INVALID_ARGUMENT, "%s input binding must hold %llu bytes at 16-byte alignment",
                label, (unsigned long long)a_need);
  if (!d->output || d->output_bytes < c_need || !aligned(d->output, 16))
    return fail(PK_INVALID_ARGUMENT, "%s output binding must hold %llu bytes at 16-byte alignment",
                label, (unsigned long long)c_need);
  if (d->bias && (d->bias_bytes < (uint64_t)d->columns * 4u || !aligned(d->bias, 16)))
    return fail(PK_INVALID_ARGUMENT, "%s bias binding must hold %llu bytes at 16-byte alignment",
                label, (unsigned long long)d->columns * 4u);
  if (d->residual && (d->residual_bytes < c_need || !aligned(d->residual, 16)))
    return fail(PK_INVALID_ARGUMENT, "%s residual binding must hold %llu bytes at 16-byte alignment",
                label, (unsigned long long)c_need);

  return PK_OK;
}

}  // namespace

extern "C" {

int pk_abi_version(void) { return PK_ABI_VERSION; }

const char* pk_last_error(void) { return g_error.c_str(); }

const char* pk_status_name(int status) {
  switch (status) {
    case PK_OK: return "PK_OK";
    case PK_INVALID_ARGUMENT: return "PK_INVALID_ARGUMENT";
    case PK_ALLOCATION_FAILURE: return "PK_ALLOCATION_FAILURE";
    case PK_INTERNAL_ERROR: return "PK_INTERNAL_ERROR";
    case PK_DEVICE_ERROR: return "PK_DEVICE_ERROR";
    case PK_DESTROYED: return "PK_DESTROYED";
    case PK_RANGE_ERROR: return "PK_RANGE_ERROR";
    default: return "PK_UNKNOWN";
  }
}

int pk_context_create(int device, pk_context** out) {
  if (!out) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  *out = nullptr;
  int count = 0;
  PK_HIP(hipGetDeviceCount(&count), "hipGetDeviceCount");
  if (device < 0 || device >= count)
    return fail(PK_INVALID_ARGUMENT, "HIP device %d does not exist (%d visible)", device, count);
  PK_HIP(hipSetDevice(device), "hipSetDevice");
  auto* ctx = new pk_context();
  ctx->device = device;
  const hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return fail(PK_DEVICE_ERROR, "hipStreamCreate failed: %s", hipGetErrorString(e));
  }
  *out = ctx;
  return ok();
}

int pk_context_destroy(pk_context* ctx) {
  if (!ctx) return ok();
  if (ctx->destroyed.exchange(true)) return ok();
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  ctx_release(ctx);
  return ok();
}

int pk_context_device(const pk_context* ctx, int* device) {
  if (int s = check_ctx(ctx)) return s;
  if (!device) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  *device = ctx->device;
  return ok();
}

int pk_context_stream(const pk_context* ctx, void** stream) {
  if (int s = check_ctx(ctx)) return s;
  if (!stream) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  *stream = ctx->stream;
  return ok();
}

int pk_device_query(const pk_context* ctx, pk_device_info* info) {
  if (int s = check_ctx(ctx)) return s;
  if (!info) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  hipDeviceProp_t prop;
  PK_HIP(hipGetDeviceProperties(&prop, ctx->device), "hipGetDeviceProperties");
  std::memset(info, 0, sizeof *info);
  std::snprintf(info->name, sizeof info->name, "%s", prop.name);
  std::snprintf(info->arch, sizeof info->arch, "%s", prop.gcnArchName);
  info->compute_units = prop.multiProcessorCount;
  info->wavefront_size = prop.warpSize;
  info->global_memory_bytes = (int64_t)prop.totalGlobalMem;
  info->lds_bytes_per_block = (int32_t)prop.sharedMemPerBlock;
  info->clock_khz = prop.clockRate;
  return ok();
}

int pk_alloc(pk_context* ctx, uint64_t bytes, void** device_ptr) {
  if (int s = check_ctx(ctx)) return s;
  if (!device_ptr) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  *device_ptr = nullptr;
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  const hipError_t e = hipMalloc(device_ptr, bytes ? bytes : 1);
  if (e != hipSuccess)
    return fail(PK_ALLOCATION_FAILURE, "cannot allocate %llu device bytes: %s",
                (unsigned long long)bytes, hipGetErrorString(e));
  return ok();
}

int pk_free(pk_context* ctx, void* device_ptr) {
  if (int s = check_ctx(ctx)) return s;
  if (!device_ptr) return ok();
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  PK_HIP(hipFree(device_ptr), "hipFree");
  return ok();
}

int pk_upload(pk_context* ctx, void* device_dst, const void* host_src, uint64_t bytes, void* stream) {
  if (int s = check_ctx(ctx)) return s;
  if (!bytes) return ok();
  if (!device_dst || !host_src) return fail(PK_INVALID_ARGUMENT, "upload pointer is null");
  hipStream_t st = stream_or_default(ctx, stream);
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  PK_HIP(hipMemcpyAsync(device_dst, host_src, bytes, hipMemcpyHostToDevice, st), "hipMemcpyAsync(upload)");
  PK_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
  return ok();
}

int pk_download(pk_context* ctx, void* host_dst, const void* device_src, uint64_t bytes, void* stream) {
  if (int s = check_ctx(ctx)) return s;
  if (!bytes) return ok();
  if (!device_src || !host_dst) return fail(PK_INVALID_ARGUMENT, "download pointer is null");
  hipStream_t st = stream_or_default(ctx, stream);
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  PK_HIP(hipMemcpyAsync(host_dst, device_src, bytes, hipMemcpyDeviceToHost, st), "hipMemcpyAsync(download)");
  PK_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
  return ok();
}

int pk_copy_device(pk_context* ctx, void* device_dst, const void* device_src, uint64_t bytes, void* stream) {
  if (int s = check_ctx(ctx)) return s;
  if (!bytes) return ok();
  if (!device_src || !device_dst) return fail(PK_INVALID_ARGUMENT, "copy pointer is null");
  hipStream_t st = stream_or_default(ctx, stream);
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  PK_HIP(hipMemcpyAsync(device_dst, device_src, bytes, hipMemcpyDeviceToDevice, st), "hipMemcpyAsync(copy)");
  return ok();
}

int pk_stream_create(pk_context* ctx, void** stream) {
  if (int s = check_ctx(ctx)) return s;
  if (!stream) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  hipStream_t st = nullptr;
  PK_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate");
  *stream = st;
  return ok();
}

int pk_stream_destroy(pk_context* ctx, void* stream) {
  if (int s = check_ctx(ctx)) return s;
  if (!stream || stream == ctx->stream) return ok();
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  PK_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)), "hipStreamDestroy");
  return ok();
}

int pk_stream_synchronize(pk_context* ctx, void* stream) {
  if (int s = check_ctx(ctx)) return s;
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  PK_HIP(hipStreamSynchronize(stream_or_default(ctx, stream)), "hipStreamSynchronize");
  return ok();
}

struct pk_graph {
  pk_abi::CtxRef ctx;
  hipGraphExec_t exec = nullptr;
};

int pk_graph_begin_capture(pk_context* ctx, void* stream) {
  if (int s = check_ctx(ctx)) return s;
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  PK_HIP(hipStreamBeginCapture(stream_or_default(ctx, stream), hipStreamCaptureModeThreadLocal),
         "hipStreamBeginCapture");
  return ok();
}

int pk_graph_end_capture(pk_context* ctx, void* stream, pk_graph** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!out) return fail(PK_INVALID_ARGUMENT, "graph output is null");
  *out = nullptr;
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  hipGraph_t graph = nullptr;
  PK_HIP(hipStreamEndCapture(stream_or_default(ctx, stream), &graph), "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  PK_HIP(inst, "hipGraphInstantiate");
  auto* g = new pk_graph();
  g->ctx = ctx;
  g->exec = exec;
  *out = g;
  return ok();
}

int pk_graph_launch(pk_graph* graph, void* stream) {
  if (!graph) return fail(PK_INVALID_ARGUMENT, "graph is null");
  PK_HIP(hipSetDevice(graph->ctx->device), "hipSetDevice");
  PK_HIP(hipGraphLaunch(graph->exec, stream_or_default(graph->ctx, stream)), "hipGraphLaunch");
  return ok();
}

int pk_graph_destroy(pk_graph* graph) {
  if (!graph) return ok();
  (void)hipSetDevice(graph->ctx->device);
  (void)hipGraphExecDestroy(graph->exec);
  delete graph;
  return ok();
}

int pk_event_create(pk_context* ctx, void** event) {
  if (int s = check_ctx(ctx)) return s;
  if (!event) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  hipEvent_t e = nullptr;
  PK_HIP(hipEventCreate(&e), "hipEventCreate");
  *event = e;
  return ok();
}

int pk_event_destroy(pk_context* ctx, void* event) {
  if (int s = check_ctx(ctx)) return s;
  if (!event) return ok();
  PK_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
  return ok();
}

int pk_event_record(pk_context* ctx, void* event, void* stream) {
  if (int s = check_ctx(ctx)) return s;
  if (!event) return fail(PK_INVALID_ARGUMENT, "event is null");
  PK_HIP(hipEventRecord(static_cast<hipEvent_t>(event), stream_or_default(ctx, stream)), "hipEventRecord");
  return ok();
}

int pk_event_synchronize(pk_context* ctx, void* event) {
  if (int s = check_ctx(ctx)) return s;
  if (!event) return fail(PK_INVALID_ARGUMENT, "event is null");
  PK_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
  return ok();
}

int pk_event_elapsed_ms(pk_context* ctx, void* start, void* end, float* ms) {
  if (int s = check_ctx(ctx)) return s;
  if (!start || !end || !ms) return fail(PK_INVALID_ARGUMENT, "event pointer is null");
  PK_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)),
         "hipEventElapsedTime");
  return ok();
}

int pk_prepared_weight_create(pk_context* ctx, const pk_weight_desc* d, void* stream,
                              pk_prepared_weight** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!d || !out) return fail(PK_INVALID_ARGUMENT, "weight descriptor or output is null");
  *out = nullptr;
  if (d->struct_size != sizeof(pk_weight_desc))
    return fail(PK_INVALID_ARGUMENT, "pk_weight_desc.struct_size mismatch");
  const char* label = safe_label(d->label);
  if (d->palette_bits != 5 && d->palette_bits != 6)
    return fail(PK_INVALID_ARGUMENT, "%s is not a palette-compressed weight", label);
  if (d->inner == 0 || d->columns == 0 || d->inner % 32u != 0)
    return fail(PK_RANGE_ERROR, "Unsupported GEMM shape for %s", label);
  if (int s = check_packed(label, d->palette_bits, d->inner, d->columns, d->packed_bytes)) return s;
  if (!d->packed || !aligned(d->packed, 4))
    return fail(PK_INVALID_ARGUMENT, "%s has invalid packed palette indices", label);
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  return make_weight(ctx, label, d->palette_bits, d->inner, d->columns, d->packed,
                     stream_or_default(ctx, stream), out);
}

int pk_prepared_weight_destroy(pk_prepared_weight* weight) {
  if (!weight) return ok();
  if (weight->owner_released) return ok();
  weight->owner_released = true;
  weight_unref(weight);
  return ok();
}

int pk_prepared_weight_bytes(const pk_prepared_weight* weight, uint64_t* bytes) {
  if (!weight || !bytes) return fail(PK_INVALID_ARGUMENT, "argument is null");
  *bytes = weight->bytes;
  return ok();
}

int pk_gemm_validate(const pk_gemm_desc* d) { return validate_gemm_desc(nullptr, d); }

int pk_gemm_create(pk_context* ctx, const pk_gemm_desc* d, void* stream, pk_gemm_op** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!d || !out) return fail(PK_INVALID_ARGUMENT, "GEMM descriptor or output is null");
  *out = nullptr;
  if (int s = validate_gemm_desc(ctx, d)) return s;
  const char* label = safe_label(d->label);
  const int bits = d->palette_bits;
  const float residual_scale = d->residual ? (d->has_residual_scale ? d->residual_scale : 1.0f) : -1.0f;
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  auto* op = new pk_gemm_op();
  op->ctx = ctx;
  op->label = label;
  op->precision = d->precision;
  op->bits = bits;
  op->rows = d->rows;
  hipDeviceProp_t prop;
  int cus = 256;
  if (hipGetDeviceProperties(&prop, ctx->device) == hipSuccess && prop.multiProcessorCount > 0)
    cus = prop.multiProcessorCount;
  const bool glu = (d->flags & PK_GEMM_GLU) != 0;
  const bool norm = (d->flags & PK_GEMM_ROW_NORM) != 0;
  op->cus = cus;
  op->cached_output = (d->flags & PK_GEMM_CACHED_OUTPUT) != 0;
  // The plan comes first: the weight is prepared in the one layout the
  // planned kernel reads (a shared prepared weight fixes it instead).
  Plan plan = plan_op(d->precision, d->rows, d->inner, d->columns, cus, glu,
                      d->prepared ? d->prepared->parts : 0, norm);
  if (d->prepared) {
    op->weight = const_cast<pk_prepared_weight*>(d->prepared);
    op->weight->refs.fetch_add(1);
    op->shared_weight = true;
  } else {
    pk_prepared_weight* w = nullptr;
    if (int s = make_weight(ctx, label, bits, d->inner, d->columns, d->packed, stream_or_default(ctx, stream), &w,
                            glu, variant_parts(d->precision, plan.variant))) {
      delete op;
      return s;
    }
    w->owner_released = true;  // owned by the op alone
    op->weight = w;
  }
  pk::GemmArgs& a = op->args;
  a.a = d->a;
  a.codes = op->weight->codes;
  a.palette = d->palette;
  a.out = d->output;
  a.bias = d->bias;
  a.residual = d->residual;
  a.residual_scale = d->residual ? residual_scale : 0.0f;
  a.activation = d->activation;
  a.rows = d->rows;
  a.inner = d->inner;
  a.columns = d->columns;
  a.palette_groups = d->palette_groups;
  a.palette_group_columns = d->palette_group_columns;
  a.palette_entries = 1u << bits;
  a.glu = glu ? 1 : 0;
  a.splits = 1;
  if (norm) {
    // G and B (2N f32), then gamma as f16 (K halves), from the packed codes.
    const uint64_t sums = (uint64_t)d->columns * 8u;
    hipError_t e = hipMalloc(&op->norm_buffer, sums + (uint64_t)d->inner * 2u);
    if (e != hipSuccess) {
      op->norm_buffer = nullptr;
      weight_unref(op->weight);
      delete op;
      return fail(PK_ALLOCATION_FAILURE, "%s: cannot allocate the row norm's column sums: %s", label,
                  hipGetErrorString(e));
    }
    float* column_sums = static_cast<float*>(op->norm_buffer);
    void* gamma16 = static_cast<uint8_t*>(op->norm_buffer) + sums;
    const hipStream_t st = stream_or_default(ctx, stream);
    e = pk::launch_norm_prepare(bits, d->packed, d->inner, d->columns, d->palette_group_columns, d->palette_groups,
                                d->palette, d->norm_gamma, d->norm_beta, gamma16, column_sums, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
      (void)hipFree(op->norm_buffer);
      weight_unref(op->weight);
      delete op;
      return fail(PK_DEVICE_ERROR, "%s: row norm preparation failed: %s", label, hipGetErrorString(e));
    }
    a.norm_columns = column_sums;
    a.norm_gamma = static_cast<const _Float16*>(gamma16);
    a.norm_epsilon = d->norm_epsilon > 0.0f ? d->norm_epsilon : 1e-5f;
  }
  if (int st = configure_launch(op, plan.variant, plan.splits)) {
    if (op->norm_buffer) (void)hipFree(op->norm_buffer);
    weight_unref(op->weight);
    delete op;
    return st;
  }
  *out = op;
  return ok();
}

int pk_gemm_enqueue(pk_gemm_op* op, uint32_t active_rows, void* stream) {
  return pk_gemm_enqueue_timed(op, active_rows, stream, nullptr, nullptr);
}

// The variant that runs `rows` active rows: the op's own (planned at its
// row capacity, or forced), or for an f16 prefix the plan of that row count
// among the kernels that read the weight's layout (the reference re-plans
// the grid of one pipeline, gemm.ts:427-451; here the tile may change too).
// A prefix keeps the op's kernel family and K split, so every row is summed
// over K in the same order as in a full-rows launch and the prefix's outputs
// are bit-identical to the same rows of the full launch: only a pair-code
// tile shape changes (the small-M and operand-order kernels take any row
// count as they are).
int planned_variant(const pk_gemm_op* op, uint32_t rows) {
  if (op->forced || rows == op->rows || op->precision != PK_PRECISION_F16 ||
      pk::f16_variant_family(op->variant) != pk::kFamilyPairCode)
    return op->variant;
  const int v = best_pair_tile(rows, op->args.columns, op->cus, op->args.glu != 0, pk::f16_variant(op->variant).k_split);
  return v >= 0 ? v : op->variant;
}

int variant_for_rows(pk_gemm_op* op, uint32_t rows) {
  if (op->forced || rows == op->rows || op->precision != PK_PRECISION_F16) return op->variant;
  if (rows != op->active_rows_planned) {
    op->active_variant = planned_variant(op, rows);
    op->active_rows_planned = rows;
  }
  return op->active_variant;
}

// The prepared plan of `rows` active rows (pk_gemm_prepare_rows), or null.
const pk_gemm_op::RowPlan* row_plan(const pk_gemm_op* op, uint32_t rows) {
  if (op->forced || rows == op->rows) return nullptr;
  const auto it = op->row_plans.find(rows);
  return it == op->row_plans.end() ? nullptr : &it->second;
}

int layout_index(int parts) { return parts == 1 ? 0 : parts == 2 ? 1 : 2; }

// The op's codes split into `parts` K parts: the weight's own layout, or a
// copy the op derives from it on the device once and keeps.
int codes_in_layout(pk_gemm_op* op, int parts, const uint32_t** out) {
  pk_prepared_weight* w = op->weight;
  if (parts == w->parts) {
    *out = w->codes;
    return PK_OK;
  }
  uint32_t*& dst = op->layouts[layout_index(parts)];
  if (!dst) {
    const uint64_t bytes = pk::operand_order_words(w->bits, w->inner, w->columns, parts) * 4u;
    hipError_t e = hipMalloc(reinterpret_cast<void**>(&dst), bytes);
    if (e != hipSuccess) {
      dst = nullptr;
      return fail(PK_ALLOCATION_FAILURE, "%s: cannot allocate %llu bytes of codes in %d K parts: %s",
                  op->label.c_str(), (unsigned long long)bytes, parts, hipGetErrorString(e));
    }
    const uint64_t blocks = (uint64_t)(pk::padded_columns(w->columns) / 32u) * (pk::padded_inner(w->inner) / 64u);
    e = pk::launch_relayout(w->bits, w->codes, w->parts, dst, parts, blocks, op->ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(op->ctx->stream);
    if (e != hipSuccess) {
      (void)hipFree(dst);
      dst = nullptr;
      return fail(PK_DEVICE_ERROR, "%s: palette code relayout failed: %s", op->label.c_str(), hipGetErrorString(e));
    }
    op->layout_bytes += bytes;
  }
  *out = dst;
  return PK_OK;
}

void drop_row_plans(pk_gemm_op* op) {
  op->row_plans.clear();
  for (uint32_t*& l : op->layouts) {
    free_after_drain(op->ctx->device, l);
    l = nullptr;
  }
  op->layout_bytes = 0;
}

int pk_gemm_enqueue_timed(pk_gemm_op* op, uint32_t active_rows, void* stream, void* start_event, void* end_event) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "GEMM op is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const uint32_t rows = active_rows ? active_rows : op->rows;
  // GemmDispatch.encode (gemm.ts:427-438)
  if (rows > op->rows)
    return fail(PK_RANGE_ERROR, "%s active rows must be in [1, %u]", op->label.c_str(), op->rows);
  const pk_gemm_op::RowPlan* prepared = row_plan(op, rows);
  const int variant = prepared ? prepared->variant : variant_for_rows(op, rows);
  pk::GemmArgs args = op->args;
  args.rows = rows;
  if (prepared) args.codes = prepared->codes;
  args.stream_out = stream_outputs(op);
  // A split never gets an empty K range.
  args.splits = std::min(op->splits, k_blocks(op->args.inner));
  hipStream_t st = stream_or_default(op->ctx, stream);
  PK_HIP(hipSetDevice(op->ctx->device), "hipSetDevice");
  hipEvent_t start = static_cast<hipEvent_t>(start_event), stop = static_cast<hipEvent_t>(end_event);
  const hipError_t e = op->precision == PK_PRECISION_F16
                           ? pk::launch_gemm_f16(op->bits, variant, args, st, start, stop)
                           : pk::launch_gemm_f32(op->bits, variant, args, st, start, stop);
  PK_HIP(e, "palette GEMM launch");
  return ok();
}

int pk_gemm_destroy(pk_gemm_op* op) {
  if (!op || op->destroyed) return ok();
  op->destroyed = true;
  weight_unref(op->weight);
  op->weight = nullptr;
  // the op may have been enqueued on a caller's stream: every free waits
  // for the device to drain
  free_after_drain(op->ctx->device, op->norm_buffer);
  op->norm_buffer = nullptr;
  free_after_drain(op->ctx->device, op->workspace);
  op->workspace = nullptr;
  op->workspace_bytes = 0;
  drop_row_plans(op);
  return ok();
}

int pk_gemm_release(pk_gemm_op* op) {
  if (!op) return ok();
  pk_gemm_destroy(op);
  delete op;
  return ok();
}

int pk_gemm_set_variant(pk_gemm_op* op, int variant) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "GEMM op is null");
  const int count = op->precision == PK_PRECISION_F16 ? pk::f16_variant_count() : pk::f32_variant_count();
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  if (variant < 0 || variant >= count)
    return fail(PK_RANGE_ERROR, "tile variant %d outside [0, %d)", variant, count);
  if (op->args.glu && pk::f16_variant_family(variant) != pk::kFamilyPairCode)
    return fail(PK_RANGE_ERROR, "%s tile variant %d has no GLU epilogue", op->label.c_str(), variant);
  if (op->args.norm_columns && pk::f16_variant_family(variant) != pk::kFamilyPairCode)
    return fail(PK_RANGE_ERROR, "%s tile variant %d has no fused row norm", op->label.c_str(), variant);
  // A forced variant runs at every row count: prepared row plans go (the
  // relayout below may free the codes they read).
  drop_row_plans(op);
  // A variant that reads another split of the codes: an op alone on its
  // weight moves it to that layout; a weight shared with other ops stays.
  const int parts = variant_parts(op->precision, variant);
  if (parts != op->weight->parts) {
    if (!(op->weight->owner_released && op->weight->refs.load() == 1))
      return fail(PK_RANGE_ERROR, "%s tile variant %d reads codes split into %d K parts; the shared prepared weight "
                  "holds %d", op->label.c_str(), variant, parts, op->weight->parts);
    PK_HIP(hipSetDevice(op->ctx->device), "hipSetDevice");
    if (int s = relayout_weight(op->weight, parts, op->ctx->stream)) return s;
    op->args.codes = op->weight->codes;
  }
  // Variants without a split-K path run unsplit.
  const bool splittable = op->precision == PK_PRECISION_F16 && pk::f16_variant_splits(variant);
  if (int s = configure_launch(op, variant, splittable ? op->splits : 1u)) return s;
  op->forced = true;
  return ok();
}

int pk_gemm_prepare_rows(pk_gemm_op* op, const uint32_t* active_rows, uint32_t count) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "GEMM op is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  if (count && !active_rows) return fail(PK_INVALID_ARGUMENT, "%s: active row list is null", op->label.c_str());
  for (uint32_t i = 0; i < count; ++i)
    if (active_rows[i] == 0 || active_rows[i] > op->rows)
      return fail(PK_RANGE_ERROR, "%s active rows must be in [1, %u]", op->label.c_str(), op->rows);
  PK_HIP(hipSetDevice(op->ctx->device), "hipSetDevice");
  for (uint32_t i = 0; i < count; ++i) {
    const uint32_t rows = active_rows[i];
    if (rows == op->rows || op->row_plans.count(rows)) continue;
    // The plan of pk_gemm_create for a descriptor of `rows` rows (a shared
    // prepared weight keeps its layout there too).
    const Plan plan = plan_op(op->precision, rows, op->args.inner, op->args.columns, op->cus, op->args.glu != 0,
                              op->shared_weight ? op->weight->parts : 0, op->args.norm_columns != nullptr);
    if (plan.splits != 1) continue;  // a split-K plan would need its own workspace: keep the prefix plan
    const uint32_t* codes = nullptr;
    if (int s = codes_in_layout(op, variant_parts(op->precision, plan.variant), &codes)) return s;
    op->row_plans[rows] = pk_gemm_op::RowPlan{plan.variant, codes};
  }
  return ok();
}

int pk_gemm_set_splits(pk_gemm_op* op, uint32_t splits) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "GEMM op is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const uint32_t limit = op->precision == PK_PRECISION_F16 ? k_blocks(op->args.inner) : 1u;
  if (splits < 1 || splits > limit)
    return fail(PK_RANGE_ERROR, "%s split count %u outside [1, %u]", op->label.c_str(), splits, limit);
  if (int s = configure_launch(op, op->variant, splits)) return s;
  drop_row_plans(op);
  op->forced = true;
  return ok();
}

int pk_gemm_variant_count(int precision) {
  return precision == PK_PRECISION_F16 ? pk::f16_variant_count() : pk::f32_variant_count();
}

int pk_gemm_variant_describe(int precision, int variant, pk_gemm_variant_desc* desc) {
  if (!desc) return fail(PK_INVALID_ARGUMENT, "argument is null");
  if (precision != PK_PRECISION_F16 && precision != PK_PRECISION_F32)
    return fail(PK_INVALID_ARGUMENT, "unsupported precision %d", precision);
  const bool f16 = precision == PK_PRECISION_F16;
  const int count = f16 ? pk::f16_variant_count() : pk::f32_variant_count();
  if (variant < 0 || variant >= count)
    return fail(PK_RANGE_ERROR, "tile variant %d outside [0, %d)", variant, count);
  const pk::TileShape s = shape_of(precision, variant);
  std::memset(desc, 0, sizeof *desc);
  desc->tile_rows = s.tile_rows();
  desc->tile_columns = s.tile_columns();
  desc->block_threads = s.threads();
  desc->k_split = s.k_split;
  desc->code_parts = variant_parts(precision, variant);
  desc->groupable = f16 && pk::f16_variant_family(variant) == pk::kFamilySmallM &&
                    group_width_index((uint32_t)s.n_blocks) >= 0;
  std::snprintf(desc->kernel5, sizeof desc->kernel5, "%s",
                f16 ? pk::f16_variant_name(5, variant) : pk::f32_variant_name(5, variant));
  std::snprintf(desc->kernel6, sizeof desc->kernel6, "%s",
                f16 ? pk::f16_variant_name(6, variant) : pk::f32_variant_name(6, variant));
  return ok();
}

int pk_gemm_plan(const pk_gemm_op* op, uint32_t active_rows, pk_gemm_plan_info* info) {
  if (!op || !info) return fail(PK_INVALID_ARGUMENT, "argument is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const uint32_t rows = active_rows ? active_rows : op->rows;
  if (rows > op->rows)
    return fail(PK_RANGE_ERROR, "%s active rows must be in [1, %u]", op->label.c_str(), op->rows);
  const bool f16 = op->precision == PK_PRECISION_F16;
  const pk_gemm_op::RowPlan* prepared = row_plan(op, rows);
  const int variant = prepared ? prepared->variant : planned_variant(op, rows);
  const pk::TileShape s = f16 ? pk::f16_variant(variant) : pk::f32_variant(variant);
  std::memset(info, 0, sizeof *info);
  const uint32_t splits = std::min(op->splits, k_blocks(op->args.inner));
  if (f16) {
    info->grid[0] = pk::f16_variant_grid(variant, rows, op->args.columns, splits);
    info->grid[1] = 1;
  } else {
    info->grid[0] = pk::tiles_n(s, op->args.columns);
    info->grid[1] = pk::tiles_m(s, rows);
  }
  info->grid[2] = 1;
  info->block_threads = s.threads();
  info->tile_rows = s.tile_rows();
  info->tile_columns = s.tile_columns();
  info->split_inner = splits;
  info->workspace_bytes = op->workspace_bytes;
  const uint32_t elem = f16 ? 2u : 4u;
  if (f16) {
    info->lds_bytes = pk::f16_variant_lds_bytes(variant);
  } else {
    const uint32_t lut_cap = (s.tile_columns() / 16u + 2u) * (1u << op->bits);
    info->lds_bytes = 2u * s.tile_rows() * 256u + lut_cap * elem;
  }
  info->flops = 2ull * rows * op->args.inner * op->args.columns;
  info->algorithmic_bytes = algorithmic_bytes(op->args, op->bits, rows, elem);
  std::snprintf(info->kernel, sizeof info->kernel, "%s",
                f16 ? pk::f16_variant_name(op->bits, variant) : pk::f32_variant_name(op->bits, variant));
  pk::GemmArgs launched = op->args;
  launched.rows = rows;
  launched.stream_out = stream_outputs(op);
  info->stream_stores = f16 && pk::f16_variant_streams(op->bits, variant, launched);
  return ok();
}

}  // extern "C"

// A group of independent f16 GEMMs run by one small-M launch. Device table:
// the members' launch arguments, then one item list per column-group width
// of the small-M variants (1, 2 and 4 blocks of 32 columns).
struct pk_gemm_group {
  pk_abi::CtxRef ctx;
  std::string label;
  std::vector<pk_prepared_weight*> weights;  // one reference each
  std::vector<pk::SmallMMember> members;
  uint32_t capacity = 0;
  int forced = -1;
  void* table = nullptr;
  uint32_t* items[3] = {};
  uint32_t items_count[3] = {};
};

namespace {

// The launch arguments of `g` on `variant` at `rows`.
pk::SmallMGroupArgs group_args(const pk_gemm_group* g, int variant, uint32_t rows) {
  const pk::TileShape s = pk::f16_variant(variant);
  const int w = group_width_index((uint32_t)s.n_blocks);
  pk::SmallMGroupArgs args{};
  args.members = static_cast<const pk::SmallMMember*>(g->table);
  args.items = w < 0 ? nullptr : g->items[w];
  args.items_count = w < 0 ? 0u : g->items_count[w];
  args.rows = rows;
  args.row_groups = pk::tiles_m(s, rows);
  args.persistent = 1u;
  for (const pk::SmallMMember& m : g->members)
    if (!pk::f16_group_streams(variant, m.args.inner, m.args.palette_groups, m.args.palette_group_columns))
      args.persistent = 0u;
  return args;
}

// The small-M variant a group runs: K over four wavefronts, each reusing
// its activation fragments over four column blocks (32 x 128). Measured on
// MI355X over the encoder's 192 weights (365 MB), kernel-stamped: the
// persistent form (one round of resident workgroups, the next item's loads
// under the current item's last blocks; code loads two blocks ahead) ran
// 100.4 us at 16 rows and 192.7 us at 64, against 115.6 and 228.3 us for
// the one-shot launch with code loads four blocks ahead, the fastest
// one-shot shape at 16, 64 and 188 rows. Groups with a member the
// persistent kernel cannot run (K not a multiple of 512, an item across
// palette groups) take that one-shot variant.
int plan_group(const pk_gemm_group* g, uint32_t rows) {
  const int count = pk::f16_variant_count();
  for (int i = 0; i < count; ++i) {
    const pk::TileShape s = pk::f16_variant(i);
    if (pk::f16_group_persistent(i) && s.m_blocks == 1 && s.n_blocks == 4 && s.k_split == 4 &&
        group_args(g, i, rows).persistent)
      return i;
  }
  const int v = find_variant(PK_PRECISION_F16, pk::kFamilySmallM, 1, 1, 1, 4, 4);
  return v < 0 ? find_variant(PK_PRECISION_F16, pk::kFamilySmallM, 1, 1, 1, 1, 8) : v;
}

int group_variant(const pk_gemm_group* g, uint32_t rows) { return g->forced >= 0 ? g->forced : plan_group(g, rows); }

}  // namespace

extern "C" {

int pk_gemm_group_create(pk_context* ctx, pk_gemm_op* const* ops, uint32_t count, const char* label,
                         pk_gemm_group** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!out || !ops) return fail(PK_INVALID_ARGUMENT, "argument is null");
  *out = nullptr;
  const char* name = label ? label : "palette-gemm-group";
  if (count == 0 || count > 65535u)
    return fail(PK_RANGE_ERROR, "%s member count %u outside [1, 65535]", name, count);
  uint32_t capacity = UINT32_MAX;
  for (uint32_t i = 0; i < count; ++i) {
    const pk_gemm_op* op = ops[i];
    if (!op) return fail(PK_INVALID_ARGUMENT, "%s member %u is null", name, i);
    if (op->destroyed) return fail(PK_DESTROYED, "%s member %u (%s) was destroyed", name, i, op->label.c_str());
    if (op->ctx != ctx)
      return fail(PK_INVALID_ARGUMENT, "%s member %u (%s) belongs to another context", name, i, op->label.c_str());
    if (op->precision != PK_PRECISION_F16 || op->args.glu || op->args.norm_columns)
      return fail(PK_RANGE_ERROR, "%s member %u (%s) is not an f16 GEMM without GLU epilogue or row norm",
                  name, i, op->label.c_str());
    if (op->weight->parts != 1)
      return fail(PK_RANGE_ERROR,
                  "%s member %u (%s) holds codes split into %d K parts; group members need the small-M "
                  "layout (one part)",
                  name, i, op->label.c_str(), op->weight->parts);
    if (pk::padded_columns(op->args.columns) / 32u > 65536u)
      return fail(PK_RANGE_ERROR, "%s member %u (%s) has more than 65536 column blocks", name, i,
                  op->label.c_str());
    capacity = std::min(capacity, op->rows);
  }
  auto* g = new pk_gemm_group();
  g->ctx = ctx;
  g->label = name;
  g->capacity = capacity;
  for (uint32_t i = 0; i < count; ++i) {
    pk::SmallMMember m{};
    m.args = ops[i]->args;
    m.args.splits = 1;
    m.args.partials = nullptr;
    m.args.counters = nullptr;
    m.bits = ops[i]->bits;
    g->members.push_back(m);
    ops[i]->weight->refs.fetch_add(1);
    g->weights.push_back(ops[i]->weight);
  }
  // Items: deepest K first (their workgroups run longest), then member and
  // column group order.
  std::vector<uint32_t> order(count);
  for (uint32_t i = 0; i < count; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) {
    return g->members[x].args.inner > g->members[y].args.inner;
  });
  std::vector<uint32_t> lists[3];
  for (int w = 0; w < 3; ++w) {
    for (uint32_t i : order) {
      const uint32_t groups = (pk::padded_columns(g->members[i].args.columns) / 32u + kGroupWidths[w] - 1u) /
                              kGroupWidths[w];
      for (uint32_t cg = 0; cg < groups; ++cg) lists[w].push_back(i << 16 | cg);
    }
    g->items_count[w] = (uint32_t)lists[w].size();
  }
  const uint64_t member_bytes = (uint64_t)count * sizeof(pk::SmallMMember);
  uint64_t bytes = (member_bytes + 255u) / 256u * 256u;
  uint64_t at[3];
  for (int w = 0; w < 3; ++w) {
    at[w] = bytes;
    bytes += ((uint64_t)g->items_count[w] * 4u + 255u) / 256u * 256u;
  }
  auto release = [&](int status) {
    for (pk_prepared_weight* w : g->weights) weight_unref(w);
    if (g->table) (void)hipFree(g->table);
    delete g;
    return status;
  };
  if (hipSetDevice(ctx->device) != hipSuccess) return release(fail(PK_DEVICE_ERROR, "hipSetDevice failed"));
  hipError_t e = hipMalloc(&g->table, bytes);
  if (e != hipSuccess) {
    g->table = nullptr;
    return release(fail(PK_ALLOCATION_FAILURE, "%s: cannot allocate %llu bytes of group tables: %s", name,
                        (unsigned long long)bytes, hipGetErrorString(e)));
  }
  auto* base = static_cast<uint8_t*>(g->table);
  e = hipMemcpy(base, g->members.data(), member_bytes, hipMemcpyHostToDevice);
  for (int w = 0; w < 3 && e == hipSuccess; ++w) {
    g->items[w] = reinterpret_cast<uint32_t*>(base + at[w]);
    e = hipMemcpy(g->items[w], lists[w].data(), (uint64_t)g->items_count[w] * 4u, hipMemcpyHostToDevice);
  }
  if (e != hipSuccess)
    return release(fail(PK_DEVICE_ERROR, "%s: group table upload failed: %s", name, hipGetErrorString(e)));
  *out = g;
  return ok();
}

int pk_gemm_group_enqueue(pk_gemm_group* group, uint32_t active_rows, void* stream) {
  return pk_gemm_group_enqueue_timed(group, active_rows, stream, nullptr, nullptr);
}

int pk_gemm_group_enqueue_timed(pk_gemm_group* g, uint32_t active_rows, void* stream, void* start_event,
                                void* end_event) {
  if (!g) return fail(PK_INVALID_ARGUMENT, "GEMM group is null");
  if (int s = check_ctx(g->ctx)) return s;
  const uint32_t rows = active_rows ? active_rows : g->capacity;
  if (rows > g->capacity)
    return fail(PK_RANGE_ERROR, "%s active rows must be in [1, %u]", g->label.c_str(), g->capacity);
  const int variant = group_variant(g, rows);
  const pk::TileShape s = pk::f16_variant(variant);
  const int w = group_width_index((uint32_t)s.n_blocks);
  if (w < 0) return fail(PK_INTERNAL_ERROR, "%s: variant %d has no group item list", g->label.c_str(), variant);
  const pk::SmallMGroupArgs args = group_args(g, variant, rows);
  PK_HIP(hipSetDevice(g->ctx->device), "hipSetDevice");
  PK_HIP(pk::launch_gemm_f16_group(variant, args, stream_or_default(g->ctx, stream),
                                   static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(end_event)),
         "palette GEMM group launch");
  return ok();
}

int pk_gemm_group_set_variant(pk_gemm_group* g, int variant) {
  if (!g) return fail(PK_INVALID_ARGUMENT, "GEMM group is null");
  if (variant == -1) {
    g->forced = -1;
    return ok();
  }
  if (variant < 0 || variant >= pk::f16_variant_count() || pk::f16_variant_family(variant) != pk::kFamilySmallM ||
      group_width_index((uint32_t)pk::f16_variant(variant).n_blocks) < 0)
    return fail(PK_RANGE_ERROR, "%s: variant %d is not a small-M variant", g->label.c_str(), variant);
  g->forced = variant;
  return ok();
}

int pk_gemm_group_plan(const pk_gemm_group* g, uint32_t active_rows, pk_gemm_plan_info* info) {
  if (!g || !info) return fail(PK_INVALID_ARGUMENT, "argument is null");
  const uint32_t rows = active_rows ? active_rows : g->capacity;
  if (rows > g->capacity)
    return fail(PK_RANGE_ERROR, "%s active rows must be in [1, %u]", g->label.c_str(), g->capacity);
  const int variant = group_variant(g, rows);
  const pk::TileShape s = pk::f16_variant(variant);
  const int w = group_width_index((uint32_t)s.n_blocks);
  std::memset(info, 0, sizeof *info);
  const char* kernel = nullptr;
  info->grid[0] = w < 0 ? 0u : pk::f16_group_launch_plan(variant, group_args(g, variant, rows), &kernel);
  info->grid[1] = info->grid[2] = 1;
  info->block_threads = s.threads();
  info->tile_rows = s.tile_rows();
  info->tile_columns = s.tile_columns();
  info->split_inner = 1;
  info->lds_bytes = pk::f16_variant_lds_bytes(variant);
  for (const pk::SmallMMember& m : g->members) {
    info->flops += 2ull * rows * m.args.inner * m.args.columns;
    info->algorithmic_bytes += algorithmic_bytes(m.args, m.bits, rows, 2u);
  }
  std::snprintf(info->kernel, sizeof info->kernel, "%s", kernel ? kernel : pk::f16_group_kernel_name(variant));
  return ok();
}

int pk_gemm_group_destroy(pk_gemm_group* g) {
  if (!g) return ok();
  free_after_drain(g->ctx->device, g->table);
  for (pk_prepared_weight* w : g->weights) weight_unref(w);
  delete g;
  return ok();
}

int pk_palette_expand(pk_context* ctx, const pk_expand_desc* d, void* stream) {
  if (int s = check_ctx(ctx)) return s;
  if (!d) return fail(PK_INVALID_ARGUMENT, "expansion descriptor is null");
  if (d->struct_size != sizeof(pk_expand_desc))
    return fail(PK_INVALID_ARGUMENT, "pk_expand_desc.struct_size mismatch");
  const char* label = safe_label(d->label);
  const bool f16 = d->precision == PK_PRECISION_F16;
  if ((!f16 && d->precision != PK_PRECISION_F32) || (d->palette_bits != 5 && d->palette_bits != 6))
    return fail(PK_INVALID_ARGUMENT, "%s has a mismatched palette execution layout", label);
  const uint32_t elem = f16 ? 2u : 4u;
  const uint32_t cpg = pk::codes_per_group(d->palette_bits);
  const uint64_t scalars = (uint64_t)d->inner * d->columns;
  // requireTransientDescriptor (palette-expander.ts:361-420)
  if (scalars == 0 || scalars % cpg != 0 || d->columns % cpg != 0 || d->palette_group_columns == 0 ||
      d->columns % d->palette_group_columns != 0 || d->palette_groups == 0 ||
      (uint64_t)d->palette_group_columns * d->palette_groups != d->columns ||
      d->packed_bytes != scalars / cpg * pk::words_per_group(d->palette_bits) * 4u ||
      d->palette_bytes != (uint64_t)d->palette_groups * (1u << d->palette_bits) * elem ||
      d->target_bytes != scalars * elem || !d->packed || !d->palette || !d->target ||
      !aligned(d->packed, 4) || !aligned(d->palette, elem) || !aligned(d->target, 16))
    return fail(PK_INVALID_ARGUMENT, "%s has invalid transient palette geometry", label);
  const bool tile = d->layout == PK_EXPAND_TILE_MAJOR;
  if (!tile && d->layout != PK_EXPAND_ROW_MAJOR)
    return fail(PK_INVALID_ARGUMENT, "%s has unsupported expanded layout %d", label, d->layout);
  if (tile && (d->inner % 32u != 0 || d->columns % (f16 ? 256u : 128u) != 0))
    return fail(PK_INVALID_ARGUMENT, "%s has invalid tile-major geometry", label);
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  PK_HIP(pk::launch_expand(d->palette_bits, f16, tile, d->packed, d->inner, d->columns,
                           d->palette_group_columns, d->palette_groups, d->palette, d->target,
                           stream_or_default(ctx, stream)),
         "palette expansion launch");
  return ok();
}

int pk_unpack_codes(pk_context* ctx, int palette_bits, const uint32_t* words, uint64_t group_count,
                    uint8_t* codes, void* stream) {
  if (int s = check_ctx(ctx)) return s;
  if (palette_bits != 5 && palette_bits != 6)
    return fail(PK_INVALID_ARGUMENT, "Unsupported palette code width %d", palette_bits);
  if (group_count == 0) return ok();
  if (!words || !codes || !aligned(words, 4) || !aligned(codes, 16))
    return fail(PK_INVALID_ARGUMENT, "unpack needs 4-byte aligned words and 16-byte aligned codes");
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  PK_HIP(pk::launch_unpack(palette_bits, words, group_count, codes, stream_or_default(ctx, stream)),
         "unpack launch");
  return ok();
}

}  // extern "C"

// pk_attention_abi.cpp - C ABI of the relative-position attention: the
// createDispatch contract checks and the encode launch
// (src/webgpu/kernels/attention.ts:51-96, :219-390).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "pk_abi_internal.h"
#include "pk_attention.h"
#include "pk_internal.h"

using namespace pk_abi;

struct pk_attention_op {
  pk_abi::CtxRef ctx;
  std::string label;
  int precision = PK_PRECISION_F16;
  uint32_t batch = 0;
  pk::AttnArgs args{};
  int variant = 0;
  bool plan_active = false;  // PK_ATTENTION_PLAN_ACTIVE (until a variant is forced)
  bool destroyed = false;
};

namespace {

const char* attention_label(const char* label) { return label ? label : "relative-attention"; }

bool overlaps(const void* a, uint64_t a_bytes, const void* b, uint64_t b_bytes) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + b_bytes && y < x + a_bytes;
}

int validate_attention_desc(const pk_attention_desc* d) {
  if (!d) return fail(PK_INVALID_ARGUMENT, "attention descriptor is null");
  if (d->struct_size != sizeof(pk_attention_desc))
    return fail(PK_INVALID_ARGUMENT, "pk_attention_desc.struct_size mismatch");
  const char* label = attention_label(d->label);
  if (d->flags & ~(PK_ATTENTION_POSITIONS_ROW_MAJOR | PK_ATTENTION_PLAN_ACTIVE))
    return fail(PK_INVALID_ARGUMENT, "%s has unknown flags 0x%x", label, d->flags);
  if (d->precision != PK_PRECISION_F16 && d->precision != PK_PRECISION_F32)
    return fail(PK_INVALID_ARGUMENT, "%s has an unsupported precision %d", label, d->precision);
  // createDispatch shape check (attention.ts:222-229), frames up to this
  // library's bound instead of one workgroup's lanes.
  if (d->batch_size == 0 || d->frames == 0 || d->frames > PK_ATTENTION_MAX_FRAMES)
    return fail(PK_RANGE_ERROR, "Unsupported attention shape for %s", label);
  const uint64_t elem = d->precision == PK_PRECISION_F16 ? 2u : 4u;
  const uint64_t rows = (uint64_t)d->batch_size * d->frames;
  const uint64_t position_rows = 2ull * d->frames - 1u;
  struct Slice {
    const char* role;
    const void* ptr;
    uint64_t bytes, need;
  };
  const Slice slices[] = {
      {"QKV", d->qkv, d->qkv_bytes, rows * 3072u * elem},
      {"output", d->output, d->output_bytes, rows * 1024u * elem},
      {"valid lengths", d->valid_lengths, d->valid_lengths_bytes, (uint64_t)d->batch_size * 4u},
  };
  for (const Slice& s : slices) {
    const uint64_t have = s.ptr ? s.bytes : 0;
    if (have < s.need)
      return fail(PK_RANGE_ERROR, "%s %s needs %llu bytes; arena slice has %llu", label, s.role,
                  (unsigned long long)s.need, (unsigned long long)have);
  }
  const char* dtype = d->precision == PK_PRECISION_F16 ? "float16" : "float32";
  if (!d->projected_positions || d->projected_positions_bytes != position_rows * 1024u * elem) {
    if (d->flags & PK_ATTENTION_POSITIONS_ROW_MAJOR)
      return fail(PK_INVALID_ARGUMENT, "Projected positions must be %s row-major, logical [%llu,1024]", dtype,
                  (unsigned long long)position_rows);
    return fail(PK_INVALID_ARGUMENT,
                "Projected positions must be %s head-vector-position-vec4, logical [%llu,1024], storage "
                "[8,32,%llu,4]",
                dtype, (unsigned long long)position_rows, (unsigned long long)position_rows);
  }
  const char* bias_role[2] = {"U", "V"};
  const float* bias_ptr[2] = {d->bias_u, d->bias_v};
  const uint64_t bias_bytes[2] = {d->bias_u_bytes, d->bias_v_bytes};
  for (int i = 0; i < 2; ++i)
    if (!bias_ptr[i] || bias_bytes[i] != 4096u)
      return fail(PK_INVALID_ARGUMENT, "%s bias %s must be float32 head-by-channel logical/storage [8,128]", label,
                  bias_role[i]);
  if (!aligned(d->qkv, 16) || !aligned(d->output, 16) || !aligned(d->projected_positions, 16) ||
      !aligned(d->bias_u, 16) || !aligned(d->bias_v, 16) || !aligned(d->valid_lengths, 4))
    return fail(PK_INVALID_ARGUMENT, "%s bindings must be 16-byte aligned (valid lengths 4-byte)", label);
  if (overlaps(d->output, rows * 1024u * elem, d->qkv, rows * 3072u * elem))
    return fail(PK_INVALID_ARGUMENT, "%s output must not overlap the QKV input", label);
  return PK_OK;
}

// The variant that runs `batch` windows: the op's own, or with
// PK_ATTENTION_PLAN_ACTIVE the one created for that many windows.
int variant_for(const pk_attention_op* op, uint32_t batch) {
  if (!op->plan_active || batch == op->batch) return op->variant;
  return pk::attention_default_variant(op->precision == PK_PRECISION_F16, op->args.frames, batch);
}

void fill_plan(const pk_attention_op* op, uint32_t batch, pk_attention_plan_info* info) {
  std::memset(info, 0, sizeof *info);
  const bool f16 = op->precision == PK_PRECISION_F16;
  const pk::AttnGeometry g = pk::attention_geometry(f16, variant_for(op, batch), op->args.frames, batch);
  info->grid[0] = g.grid;
  info->grid[1] = 1;
  info->grid[2] = 1;
  info->block_threads = g.block_threads;
  info->lds_bytes = g.lds_bytes;
  info->query_tiles = g.query_tiles;
  const uint64_t elem = f16 ? 2u : 4u;
  const uint64_t rows = (uint64_t)batch * op->args.frames;
  info->algorithmic_bytes = rows * (3072u + 1024u) * elem + (uint64_t)op->args.position_rows * 1024u * elem +
                            2u * 4096u + 4u * batch;
  std::snprintf(info->kernel, sizeof info->kernel, "%s", g.name);
}

}  // namespace

extern "C" {

int pk_attention_validate(const pk_attention_desc* d) { return validate_attention_desc(d); }

int pk_attention_create(pk_context* ctx, const pk_attention_desc* d, pk_attention_op** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!d || !out) return fail(PK_INVALID_ARGUMENT, "attention descriptor or output is null");
  *out = nullptr;
  if (int s = validate_attention_desc(d)) return s;
  auto* op = new pk_attention_op();
  op->ctx = ctx;
  op->label = attention_label(d->label);
  op->precision = d->precision;
  op->batch = d->batch_size;
  op->variant = pk::attention_default_variant(d->precision == PK_PRECISION_F16, d->frames, d->batch_size);
  op->plan_active = (d->flags & PK_ATTENTION_PLAN_ACTIVE) != 0;
  pk::AttnArgs& a = op->args;
  a.qkv = d->qkv;
  a.positions = d->projected_positions;
  a.bias_u = d->bias_u;
  a.bias_v = d->bias_v;
  a.valid_lengths = d->valid_lengths;
  a.output = d->output;
  a.frames = d->frames;
  a.position_rows = 2u * d->frames - 1u;
  a.positions_row_major = (d->flags & PK_ATTENTION_POSITIONS_ROW_MAJOR) ? 1 : 0;
  *out = op;
  return ok();
}

int pk_attention_enqueue(pk_attention_op* op, uint32_t active_batch, void* stream) {
  return pk_attention_enqueue_timed(op, active_batch, stream, nullptr, nullptr);
}

int pk_attention_enqueue_timed(pk_attention_op* op, uint32_t active_batch, void* stream, void* start_event,
                               void* end_event) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "attention op is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const uint32_t batch = active_batch ? active_batch : op->batch;
  // RelativeAttentionDispatch.encode (attention.ts:67-77)
  if (batch > op->batch)
    return fail(PK_RANGE_ERROR, "%s active batch must be in [1, %u]", op->label.c_str(), op->batch);
  PK_HIP(hipSetDevice(op->ctx->device), "hipSetDevice");
  const hipError_t e =
      pk::launch_attention(op->precision == PK_PRECISION_F16, variant_for(op, batch), op->args, batch,
                           stream_or_default(op->ctx, stream), static_cast<hipEvent_t>(start_event),
                           static_cast<hipEvent_t>(end_event));
  PK_HIP(e, "relative attention launch");
  return ok();
}

int pk_attention_plan(const pk_attention_op* op, uint32_t active_batch, pk_attention_plan_info* info) {
  if (!op || !info) return fail(PK_INVALID_ARGUMENT, "argument is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const uint32_t batch = active_batch ? active_batch : op->batch;
  if (batch > op->batch)
    return fail(PK_RANGE_ERROR, "%s active batch must be in [1, %u]", op->label.c_str(), op->batch);
  fill_plan(op, batch, info);
  return ok();
}

int pk_attention_destroy(pk_attention_op* op) {
  if (!op || op->destroyed) return ok();
  op->destroyed = true;
  return ok();
}

int pk_attention_release(pk_attention_op* op) {
  if (!op) return ok();
  pk_attention_destroy(op);
  delete op;
  return ok();
}

int pk_attention_variant_count(int precision) {
  return pk::attention_variant_count(precision == PK_PRECISION_F16);
}

int pk_attention_set_variant(pk_attention_op* op, int variant) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "attention op is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const int count = pk::attention_variant_count(op->precision == PK_PRECISION_F16);
  if (variant < 0 || variant >= count)
    return fail(PK_RANGE_ERROR, "attention variant %d outside [0, %d)", variant, count);
  op->variant = variant;
  op->plan_active = false;
  return ok();
}

}  // extern "C"

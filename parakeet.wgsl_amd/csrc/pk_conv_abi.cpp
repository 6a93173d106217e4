// pk_conv_abi.cpp - C ABI of the fused Conformer convolution tail: the
// planFusedConformerConv arithmetic, the createDispatch contract checks and
// the encode launch (src/webgpu/kernels/conformer-conv.ts:72-162, :255-458).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "pk_abi_internal.h"
#include "pk_conv.h"
#include "pk_internal.h"

using namespace pk_abi;

struct pk_conv_op {
  pk_abi::CtxRef ctx;
  std::string label;
  int precision = PK_PRECISION_F16;
  uint32_t batch = 0;
  pk::ConvArgs args{};
  int variant = 0;
  bool destroyed = false;
};

namespace {

const char* conv_label(const char* label) { return label ? label : "conformer-conv"; }

uint32_t channels_of(uint32_t channels) { return channels ? channels : PK_CONV_DEFAULT_CHANNELS; }

// Default launch shape per precision: the first compiled variant (2
// channels per thread over runs of 8 frames).
int default_variant(int /*precision*/) { return 0; }

struct Sizes {
  uint64_t rows, input, output, valid, weights, affine;
};

// planFusedConformerConv (conformer-conv.ts:72-115): requirePositiveInteger
// on both dimensions, then the byte lengths.
int plan_sizes(const char* label, int precision, uint32_t batch, uint32_t frames, uint32_t channels, Sizes* s) {
  if (precision != PK_PRECISION_F16 && precision != PK_PRECISION_F32)
    return fail(PK_INVALID_ARGUMENT, "%s has an unsupported precision %d", label, precision);
  if (batch == 0) return fail(PK_RANGE_ERROR, "batchSize must be a positive integer");
  if (frames == 0) return fail(PK_RANGE_ERROR, "frames must be a positive integer");
  if (channels % 8u != 0)
    return fail(PK_RANGE_ERROR, "%s channels must be a positive multiple of 8 (got %u)", label, channels);
  const uint64_t rows = (uint64_t)batch * frames;
  if (rows > 0xffffffffull) return fail(PK_RANGE_ERROR, "Conformer rows exceeds the safe integer range");
  const uint64_t elem = precision == PK_PRECISION_F16 ? 2u : 4u;
  s->rows = rows;
  s->input = rows * 2u * channels * elem;
  s->output = rows * channels * elem;
  s->valid = (uint64_t)batch * 4u;
  s->weights = (uint64_t)PK_CONV_KERNEL_SIZE * channels * elem;
  s->affine = (uint64_t)channels * 4u;
  return PK_OK;
}

// The input bytes a launch reads per window: [frames, 2C], or [frames, C]
// of ready GLU.
uint64_t input_bytes_of(const Sizes& s, bool input_glu) { return input_glu ? s.input / 2u : s.input; }

void fill_plan(int precision, int variant, uint32_t batch, uint32_t frames, uint32_t channels, uint32_t active,
               const Sizes& s, bool input_glu, pk_conv_plan_info* info) {
  std::memset(info, 0, sizeof *info);
  info->rows = (uint32_t)s.rows;
  info->input_bytes = s.input;
  info->output_bytes = s.output;
  info->valid_lengths_bytes = s.valid;
  info->depthwise_weight_bytes = s.weights;
  info->affine_bytes = s.affine;
  const bool f16 = precision == PK_PRECISION_F16;
  const pk::ConvGeometry g = pk::conv_geometry(f16, variant, frames, channels, active, input_glu);
  info->grid[0] = g.grid;
  info->grid[1] = 1;
  info->grid[2] = 1;
  info->block_threads = g.block_threads;
  info->lds_bytes = 0;
  const uint64_t per_item = (input_bytes_of(s, input_glu) + s.output) / batch;
  info->algorithmic_bytes = per_item * active + s.weights + 2u * s.affine + 4ull * active;
  std::snprintf(info->kernel, sizeof info->kernel, "%s", g.name);
}

bool overlaps(const void* a, uint64_t a_bytes, const void* b, uint64_t b_bytes) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + b_bytes && y < x + a_bytes;
}

// createDispatch (conformer-conv.ts:255-300): requireArenaCapacity for the
// arena slices (:390-401), requirePackedTensor for the weights and folded
// batch norm (:403-432), plus the alignment the vector loads rely on.
int validate_conv_desc(const pk_conv_desc* d) {
  if (!d) return fail(PK_INVALID_ARGUMENT, "convolution descriptor is null");
  if (d->struct_size != sizeof(pk_conv_desc))
    return fail(PK_INVALID_ARGUMENT, "pk_conv_desc.struct_size mismatch");
  const char* label = conv_label(d->label);
  const uint32_t C = channels_of(d->channels);
  if (d->flags & ~PK_CONV_INPUT_GLU) return fail(PK_INVALID_ARGUMENT, "%s has unknown flags 0x%x", label, d->flags);
  const bool input_glu = (d->flags & PK_CONV_INPUT_GLU) != 0;
  Sizes s;
  if (int st = plan_sizes(label, d->precision, d->batch_size, d->frames, C, &s)) return st;
  const uint64_t input_need = input_bytes_of(s, input_glu);
  struct Slice {
    const char* role;
    const void* ptr;
    uint64_t bytes, need;
  };
  const Slice slices[] = {
      {"pointwise input", d->pointwise_input, d->pointwise_input_bytes, input_need},
      {"output", d->output, d->output_bytes, s.output},
      {"valid lengths", d->valid_lengths, d->valid_lengths_bytes, s.valid},
  };
  for (const Slice& sl : slices) {
    const uint64_t have = sl.ptr ? sl.bytes : 0;
    if (have < sl.need)
      return fail(PK_RANGE_ERROR, "%s %s needs %llu bytes; arena slice has %llu", label, sl.role,
                  (unsigned long long)sl.need, (unsigned long long)have);
  }
  const bool f16 = d->precision == PK_PRECISION_F16;
  const char* dtype = f16 ? "float16" : "float32";
  if (!d->depthwise_weights || d->depthwise_weights_bytes != s.weights)
    return fail(PK_INVALID_ARGUMENT,
                "%s depthwise weights must be %s kernel-channel-vec4 logical [%d,%u], storage [%d,%u,4], %llu bytes",
                label, dtype, PK_CONV_KERNEL_SIZE, C, PK_CONV_KERNEL_SIZE, C / 4u, (unsigned long long)s.weights);
  const char* affine_role[2] = {"scale", "shift"};
  const float* affine_ptr[2] = {d->batch_norm_scale, d->batch_norm_shift};
  const uint64_t affine_bytes[2] = {d->batch_norm_scale_bytes, d->batch_norm_shift_bytes};
  for (int i = 0; i < 2; ++i)
    if (!affine_ptr[i] || affine_bytes[i] != s.affine)
      return fail(PK_INVALID_ARGUMENT,
                  "%s folded batch norm %s must be float32 channel logical [%u], storage [%u], %llu bytes", label,
                  affine_role[i], C, C, (unsigned long long)s.affine);
  if (!aligned(d->pointwise_input, 16) || !aligned(d->output, 16) || !aligned(d->depthwise_weights, 16) ||
      !aligned(d->batch_norm_scale, 16) || !aligned(d->batch_norm_shift, 16) || !aligned(d->valid_lengths, 4))
    return fail(PK_INVALID_ARGUMENT, "%s bindings must be 16-byte aligned (valid lengths 4-byte)", label);
  // Frames read other frames' GLU inputs, so the output may not alias them.
  if (overlaps(d->output, s.output, d->pointwise_input, input_need))
    return fail(PK_INVALID_ARGUMENT, "%s output must not overlap the pointwise input", label);
  return PK_OK;
}

}  // namespace

extern "C" {

int pk_conv_plan_shape(int precision, uint32_t batch_size, uint32_t frames, uint32_t channels,
                       pk_conv_plan_info* info) {
  if (!info) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  const uint32_t C = channels_of(channels);
  Sizes s;
  if (int st = plan_sizes(conv_label(nullptr), precision, batch_size, frames, C, &s)) return st;
  fill_plan(precision, default_variant(precision), batch_size, frames, C, batch_size, s, false, info);
  return ok();
}

int pk_conv_validate(const pk_conv_desc* d) { return validate_conv_desc(d); }

int pk_conv_create(pk_context* ctx, const pk_conv_desc* d, pk_conv_op** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!d || !out) return fail(PK_INVALID_ARGUMENT, "convolution descriptor or output is null");
  *out = nullptr;
  if (int s = validate_conv_desc(d)) return s;
  auto* op = new pk_conv_op();
  op->ctx = ctx;
  op->label = conv_label(d->label);
  op->precision = d->precision;
  op->batch = d->batch_size;
  op->variant = default_variant(d->precision);
  pk::ConvArgs& a = op->args;
  a.input = d->pointwise_input;
  a.weights = d->depthwise_weights;
  a.scale = d->batch_norm_scale;
  a.shift = d->batch_norm_shift;
  a.valid_lengths = d->valid_lengths;
  a.output = d->output;
  a.frames = d->frames;
  a.channels = channels_of(d->channels);
  a.input_glu = (d->flags & PK_CONV_INPUT_GLU) ? 1 : 0;
  *out = op;
  return ok();
}

int pk_conv_enqueue(pk_conv_op* op, uint32_t active_batch, void* stream) {
  return pk_conv_enqueue_timed(op, active_batch, stream, nullptr, nullptr);
}

int pk_conv_enqueue_timed(pk_conv_op* op, uint32_t active_batch, void* stream, void* start_event,
                          void* end_event) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "convolution op is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const uint32_t batch = active_batch ? active_batch : op->batch;
  // FusedConformerConvDispatch.encode (conformer-conv.ts:133-143)
  if (batch > op->batch)
    return fail(PK_RANGE_ERROR, "%s active batch must be in [1, %u]", op->label.c_str(), op->batch);
  PK_HIP(hipSetDevice(op->ctx->device), "hipSetDevice");
  const hipError_t e = pk::launch_conformer_conv(
      op->precision == PK_PRECISION_F16, op->variant, op->args, batch, stream_or_default(op->ctx, stream),
      static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(end_event));
  PK_HIP(e, "conformer convolution launch");
  return ok();
}

int pk_conv_plan(const pk_conv_op* op, uint32_t active_batch, pk_conv_plan_info* info) {
  if (!op || !info) return fail(PK_INVALID_ARGUMENT, "argument is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const uint32_t batch = active_batch ? active_batch : op->batch;
  if (batch > op->batch)
    return fail(PK_RANGE_ERROR, "%s active batch must be in [1, %u]", op->label.c_str(), op->batch);
  Sizes s;
  if (int st = plan_sizes(op->label.c_str(), op->precision, op->batch, op->args.frames, op->args.channels, &s))
    return st;
  fill_plan(op->precision, op->variant, op->batch, op->args.frames, op->args.channels, batch, s,
            op->args.input_glu != 0, info);
  return ok();
}

int pk_conv_destroy(pk_conv_op* op) {
  if (!op || op->destroyed) return ok();
  op->destroyed = true;
  return ok();
}

int pk_conv_release(pk_conv_op* op) {
  if (!op) return ok();
  pk_conv_destroy(op);
  delete op;
  return ok();
}

int pk_conv_variant_count(int precision) { return pk::conv_variant_count(precision == PK_PRECISION_F16); }

int pk_conv_set_variant(pk_conv_op* op, int variant) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "convolution op is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const int count = pk::conv_variant_count(op->precision == PK_PRECISION_F16);
  if (variant < 0 || variant >= count)
    return fail(PK_RANGE_ERROR, "convolution variant %d outside [0, %d)", variant, count);
  op->variant = variant;
  return ok();
}

}  // extern "C"

// pk_subsampling_abi.cpp - C ABI of the subsampling front end's convolution
// stages: the createDispatch checks and the encode launches of
// src/webgpu/kernels/subsampling.ts (:119-790).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "pk_abi_internal.h"
#include "pk_internal.h"
#include "pk_subsampling.h"

using namespace pk_abi;

struct pk_subsampling_op {
  pk_abi::CtxRef ctx;
  std::string label;
  int kind = pk::kSubsamplingFused;
  int precision = PK_PRECISION_F16;
  uint32_t batch = 0;
  pk::SubsamplingArgs args{};
  bool destroyed = false;
};

namespace {

uint32_t output_dimension(uint32_t n) { return n == 0 ? 0u : (uint32_t)(((uint64_t)n + 1u) / 2u); }

uint32_t valid_length(uint32_t n, uint32_t steps) {
  for (uint32_t s = 0; s < steps; ++s) n = output_dimension(n);
  return n;
}

const char* label_of(const char* label, const char* fallback) { return label ? label : fallback; }

int check_precision(int32_t precision, const char* label) {
  if (precision != PK_PRECISION_F16 && precision != PK_PRECISION_F32)
    return fail(PK_INVALID_ARGUMENT, "%s has an unsupported precision %d", label, precision);
  return PK_OK;
}

// requirePositiveInteger (subsampling.ts:1075-1079)
int positive(uint32_t value, const char* name) {
  if (value == 0) return fail(PK_RANGE_ERROR, "%s must be a positive integer", name);
  return PK_OK;
}

// requireArenaCapacity (subsampling.ts:951-962)
int capacity(const void* p, uint64_t have, uint64_t need, const char* role, const char* label) {
  const uint64_t got = p ? have : 0;
  if (got < need)
    return fail(PK_RANGE_ERROR, "%s %s needs %llu bytes; arena slice has %llu", label, role,
                (unsigned long long)need, (unsigned long long)got);
  return PK_OK;
}

// requirePackedTensor (subsampling.ts:1009-1034) for a [3,3,C] kernel.
int kernel_tensor(const void* p, uint64_t bytes, int precision, uint32_t channels, const char* layout,
                  const char* label, const char* what) {
  const uint64_t need = 9ull * channels * (precision == PK_PRECISION_F16 ? 2u : 4u);
  if (!p || bytes != need || !aligned(p, 16))
    return fail(PK_INVALID_ARGUMENT, "%s %s must be %s %s logical [3,3,%u], storage [3,3,%u,4], %llu bytes", label,
                what, precision == PK_PRECISION_F16 ? "float16" : "float32", layout, channels, channels / 4,
                (unsigned long long)need);
  return PK_OK;
}

int bias_tensor(const void* p, uint64_t bytes, uint32_t channels, const char* label, const char* what) {
  const uint64_t need = 4ull * channels;
  if (!p || bytes != need || !aligned(p, 16))
    return fail(PK_INVALID_ARGUMENT,
                "%s %s must be float32 output-channel logical [%u], storage [%u], %llu bytes", label, what, channels,
                channels, (unsigned long long)need);
  return PK_OK;
}

int lengths(const uint32_t* p, uint64_t bytes, uint32_t offset, uint32_t batch, const char* label) {
  return capacity(p, bytes, ((uint64_t)offset + batch) * 4u, "valid lengths", label);
}

int validate_fused(const pk_subsampling_fused_desc* d) {
  if (!d) return fail(PK_INVALID_ARGUMENT, "subsampling descriptor is null");
  if (d->struct_size != sizeof(pk_subsampling_fused_desc))
    return fail(PK_INVALID_ARGUMENT, "pk_subsampling_fused_desc.struct_size mismatch");
  const char* label = label_of(d->label, "subsampling-fused-conv0-depthwise2");
  if (int s = check_precision(d->precision, label)) return s;
  // planFusedSubsamplingConv0Depthwise2 (subsampling.ts:145-206)
  if (int s = positive(d->batch_size, "batchSize")) return s;
  if (int s = positive(d->input_height, "inputHeight")) return s;
  if (d->input_width != PK_SUBSAMPLING_BINS || d->channels != PK_SUBSAMPLING_CHANNELS)
    return fail(PK_RANGE_ERROR, "Fused conv0+depthwise2 requires fixed [batch,frames,128,256]");
  const uint64_t e = d->precision == PK_PRECISION_F16 ? 2u : 4u;
  const uint32_t ho = valid_length(d->input_height, 2), wo = valid_length(d->input_width, 2);
  const uint64_t in_bytes = (uint64_t)d->batch_size * d->input_height * d->input_width * 4u;
  const uint64_t out_bytes = (uint64_t)d->batch_size * ho * wo * d->channels * e;
  if (int s = capacity(d->input, d->input_bytes, in_bytes, "input", label)) return s;
  if (int s = capacity(d->output, d->output_bytes, out_bytes, "output", label)) return s;
  if (int s = lengths(d->valid_lengths, d->valid_lengths_bytes, d->valid_length_batch_offset, d->batch_size, label))
    return s;
  if (int s = kernel_tensor(d->conv0_weights, d->conv0_weights_bytes, d->precision, d->channels,
                            "kh-kw-output-channel-vec4", label, "conv0 weights"))
    return s;
  if (int s = bias_tensor(d->conv0_bias, d->conv0_bias_bytes, d->channels, label, "conv0 bias")) return s;
  if (int s = kernel_tensor(d->depthwise_weights, d->depthwise_weights_bytes, d->precision, d->channels,
                            "kh-kw-channel-vec4", label, "depthwise2 weights"))
    return s;
  if (int s = bias_tensor(d->depthwise_bias, d->depthwise_bias_bytes, d->channels, label, "depthwise2 bias"))
    return s;
  if (!aligned(d->input, 16) || !aligned(d->output, 16) || !aligned(d->valid_lengths, 4))
    return fail(PK_INVALID_ARGUMENT, "%s bindings must be 16-byte aligned", label);
  return PK_OK;
}

int validate_depthwise(const pk_subsampling_depthwise_desc* d) {
  if (!d) return fail(PK_INVALID_ARGUMENT, "subsampling descriptor is null");
  if (d->struct_size != sizeof(pk_subsampling_depthwise_desc))
    return fail(PK_INVALID_ARGUMENT, "pk_subsampling_depthwise_desc.struct_size mismatch");
  const char* label = label_of(d->label, "subsampling-depthwise");
  if (int s = check_precision(d->precision, label)) return s;
  // planDepthwise (subsampling.ts:795-853)
  if (int s = positive(d->batch_size, "batchSize")) return s;
  if (int s = positive(d->input_height, "inputHeight")) return s;
  if (int s = positive(d->input_width, "inputWidth")) return s;
  if (int s = positive(d->channels, "channels")) return s;
  if (d->channels % 4u) return fail(PK_RANGE_ERROR, "Subsampling channels must be divisible by four");
  const uint64_t e = d->precision == PK_PRECISION_F16 ? 2u : 4u;
  const uint64_t in_bytes = (uint64_t)d->batch_size * d->input_height * d->input_width * d->channels * e;
  const uint64_t out_bytes = (uint64_t)d->batch_size * output_dimension(d->input_height) *
                             output_dimension(d->input_width) * d->channels * e;
  // createDispatch (subsampling.ts:495-531)
  if (int s = capacity(d->input, d->input_bytes, in_bytes, "input", label)) return s;
  if (d->valid_length_subsampling_steps == 0)
    return fail(PK_RANGE_ERROR, "%s valid-length subsampling steps must be a positive integer", label);
  if (int s = lengths(d->valid_lengths, d->valid_lengths_bytes, d->valid_length_batch_offset, d->batch_size, label))
    return s;
  if (int s = capacity(d->output, d->output_bytes, out_bytes, "output", label)) return s;
  if (int s = kernel_tensor(d->weights, d->weights_bytes, d->precision, d->channels, "kh-kw-channel-vec4", label,
                            "weights"))
    return s;
  if (int s = bias_tensor(d->bias, d->bias_bytes, d->channels, label, "bias")) return s;
  if (!aligned(d->input, 16) || !aligned(d->output, 16) || !aligned(d->valid_lengths, 4))
    return fail(PK_INVALID_ARGUMENT, "%s bindings must be 16-byte aligned", label);
  return PK_OK;
}

int validate_mask(const pk_subsampling_mask_desc* d) {
  if (!d) return fail(PK_INVALID_ARGUMENT, "subsampling descriptor is null");
  if (d->struct_size != sizeof(pk_subsampling_mask_desc))
    return fail(PK_INVALID_ARGUMENT, "pk_subsampling_mask_desc.struct_size mismatch");
  const char* label = label_of(d->label, "subsampling-time-mask");
  if (int s = check_precision(d->precision, label)) return s;
  // createDispatch (subsampling.ts:698-748)
  if (int s = positive(d->batch_size, "batchSize")) return s;
  if (int s = positive(d->height, "height")) return s;
  if (int s = positive(d->width, "width")) return s;
  if (int s = positive(d->channels, "channels")) return s;
  if (d->channels % 4u) return fail(PK_RANGE_ERROR, "Subsampling mask channels must be divisible by four");
  if (d->valid_length_subsampling_steps == 0)
    return fail(PK_RANGE_ERROR, "%s valid-length subsampling steps must be a positive integer", label);
  const uint64_t e = d->precision == PK_PRECISION_F16 ? 2u : 4u;
  const uint64_t bytes = (uint64_t)d->batch_size * d->height * d->width * d->channels * e;
  if (int s = capacity(d->values, d->values_bytes, bytes, "values", label)) return s;
  if (int s = lengths(d->valid_lengths, d->valid_lengths_bytes, d->valid_length_batch_offset, d->batch_size, label))
    return s;
  if (!aligned(d->values, 16) || !aligned(d->valid_lengths, 4))
    return fail(PK_INVALID_ARGUMENT, "%s bindings must be 16-byte aligned", label);
  return PK_OK;
}

pk_subsampling_op* new_op(pk_context* ctx, const char* label, int kind, int precision, uint32_t batch) {
  auto* op = new pk_subsampling_op();
  op->ctx = ctx;
  op->label = label;
  op->kind = kind;
  op->precision = precision;
  op->batch = batch;
  return op;
}

}  // namespace

extern "C" {

uint32_t pk_subsampling_output_dimension(uint32_t input) { return output_dimension(input); }

uint32_t pk_subsampling_valid_length(uint32_t feature_length, uint32_t steps) {
  return valid_length(feature_length, steps);
}

int pk_subsampling_fused_validate(const pk_subsampling_fused_desc* d) { return validate_fused(d); }
int pk_subsampling_depthwise_validate(const pk_subsampling_depthwise_desc* d) { return validate_depthwise(d); }
int pk_subsampling_mask_validate(const pk_subsampling_mask_desc* d) { return validate_mask(d); }

int pk_subsampling_fused_create(pk_context* ctx, const pk_subsampling_fused_desc* d, pk_subsampling_op** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!out) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  *out = nullptr;
  if (int s = validate_fused(d)) return s;
  auto* op = new_op(ctx, label_of(d->label, "subsampling-fused-conv0-depthwise2"), pk::kSubsamplingFused,
                    d->precision, d->batch_size);
  pk::SubsamplingArgs& a = op->args;
  a.input = d->input;
  a.weights = d->conv0_weights;
  a.bias = d->conv0_bias;
  a.weights2 = d->depthwise_weights;
  a.bias2 = d->depthwise_bias;
  a.output = d->output;
  a.valid_lengths = d->valid_lengths + d->valid_length_batch_offset;
  a.height = d->input_height;
  a.width = d->input_width;
  a.mid_height = output_dimension(d->input_height);
  a.mid_width = output_dimension(d->input_width);
  a.out_height = output_dimension(a.mid_height);
  a.out_width = output_dimension(a.mid_width);
  a.channels = d->channels;
  a.valid_offset = d->valid_length_batch_offset;
  a.steps = 2;
  *out = op;
  return ok();
}

int pk_subsampling_depthwise_create(pk_context* ctx, const pk_subsampling_depthwise_desc* d,
                                    pk_subsampling_op** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!out) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  *out = nullptr;
  if (int s = validate_depthwise(d)) return s;
  auto* op = new_op(ctx, label_of(d->label, "subsampling-depthwise"), pk::kSubsamplingDepthwise, d->precision,
                    d->batch_size);
  pk::SubsamplingArgs& a = op->args;
  a.input = d->input;
  a.weights = d->weights;
  a.bias = d->bias;
  a.output = d->output;
  a.valid_lengths = d->valid_lengths + d->valid_length_batch_offset;
  a.height = d->input_height;
  a.width = d->input_width;
  a.out_height = output_dimension(d->input_height);
  a.out_width = output_dimension(d->input_width);
  a.channels = d->channels;
  a.valid_offset = d->valid_length_batch_offset;
  a.steps = d->valid_length_subsampling_steps;
  *out = op;
  return ok();
}

int pk_subsampling_mask_create(pk_context* ctx, const pk_subsampling_mask_desc* d, pk_subsampling_op** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!out) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  *out = nullptr;
  if (int s = validate_mask(d)) return s;
  auto* op = new_op(ctx, label_of(d->label, "subsampling-time-mask"), pk::kSubsamplingMask, d->precision,
                    d->batch_size);
  pk::SubsamplingArgs& a = op->args;
  a.output = d->values;
  a.valid_lengths = d->valid_lengths + d->valid_length_batch_offset;
  a.height = a.out_height = d->height;
  a.width = a.out_width = d->width;
  a.channels = d->channels;
  a.valid_offset = d->valid_length_batch_offset;
  a.steps = d->valid_length_subsampling_steps;
  *out = op;
  return ok();
}

int pk_subsampling_enqueue(pk_subsampling_op* op, uint32_t active_batch, void* stream) {
  return pk_subsampling_enqueue_timed(op, active_batch, stream, nullptr, nullptr);
}

int pk_subsampling_enqueue_timed(pk_subsampling_op* op, uint32_t active_batch, void* stream, void* start_event,
                                 void* end_event) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "subsampling op is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const uint32_t batch = active_batch ? active_batch : op->batch;
  if (batch > op->batch)
    return fail(PK_RANGE_ERROR, "%s active batch must be in [1, %u]", op->label.c_str(), op->batch);
  PK_HIP(hipSetDevice(op->ctx->device), "hipSetDevice");
  PK_HIP(pk::launch_subsampling(op->kind, op->precision == PK_PRECISION_F16, op->args, batch,
                                stream_or_default(op->ctx, stream), static_cast<hipEvent_t>(start_event),
                                static_cast<hipEvent_t>(end_event)),
         "subsampling launch");
  return ok();
}

int pk_subsampling_plan(const pk_subsampling_op* op, uint32_t active_batch, pk_subsampling_plan_info* info) {
  if (!op || !info) return fail(PK_INVALID_ARGUMENT, "subsampling op or plan output is null");
  const uint32_t batch = active_batch ? active_batch : op->batch;
  if (batch > op->batch)
    return fail(PK_RANGE_ERROR, "%s active batch must be in [1, %u]", op->label.c_str(), op->batch);
  const bool f16 = op->precision == PK_PRECISION_F16;
  const pk::SubsamplingArgs& a = op->args;
  const pk::SubsamplingGeometry g = pk::subsampling_geometry(op->kind, f16, a, batch);
  std::memset(info, 0, sizeof *info);
  info->output_height = a.out_height;
  info->output_width = a.out_width;
  for (int i = 0; i < 3; ++i) info->grid[i] = g.grid[i];
  info->block_threads = g.block_threads;
  info->lds_bytes = g.lds_bytes;
  const uint64_t e = f16 ? 2u : 4u;
  const uint64_t out_elems = (uint64_t)batch * a.out_height * a.out_width * a.channels;
  const uint64_t kernel = 9ull * a.channels * e + 4ull * a.channels;
  if (op->kind == pk::kSubsamplingFused) {
    info->algorithmic_bytes = (uint64_t)batch * a.height * a.width * 4u + out_elems * e + 2 * kernel + 4ull * batch;
    info->flops = 2ull * 9u * ((uint64_t)batch * a.mid_height * a.mid_width * a.channels + out_elems);
  } else if (op->kind == pk::kSubsamplingDepthwise) {
    info->algorithmic_bytes =
        (uint64_t)batch * a.height * a.width * a.channels * e + out_elems * e + kernel + 4ull * batch;
    info->flops = 2ull * 9u * out_elems;
  } else {
    // upper bound: every frame past its window's length is rewritten
    info->algorithmic_bytes = out_elems * e + 4ull * batch;
  }
  std::snprintf(info->kernel, sizeof info->kernel, "%s", g.name);
  return ok();
}

int pk_subsampling_destroy(pk_subsampling_op* op) {
  if (!op || op->destroyed) return ok();
  op->destroyed = true;
  return ok();
}

int pk_subsampling_release(pk_subsampling_op* op) {
  if (!op) return ok();
  pk_subsampling_destroy(op);
  delete op;
  return ok();
}

}  // extern "C"

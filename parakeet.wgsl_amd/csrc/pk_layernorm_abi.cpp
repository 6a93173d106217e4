// pk_layernorm_abi.cpp - C ABI of the row LayerNorm: the createDispatch
// checks and the encode launch (src/webgpu/kernels/layernorm.ts:29-281).
#include <hip/hip_runtime.h>

#include <string>

#include "pk_abi_internal.h"
#include "pk_internal.h"
#include "pk_layernorm.h"

using namespace pk_abi;

struct pk_layernorm_op {
  pk_abi::CtxRef ctx;
  std::string label;
  int precision = PK_PRECISION_F16;
  uint32_t rows = 0;
  pk::LayerNormArgs args{};
  bool destroyed = false;
};

namespace {

const char* ln_label(const char* label) { return label ? label : "layernorm"; }

int validate_layernorm_desc(const pk_layernorm_desc* d) {
  if (!d) return fail(PK_INVALID_ARGUMENT, "LayerNorm descriptor is null");
  if (d->struct_size != sizeof(pk_layernorm_desc))
    return fail(PK_INVALID_ARGUMENT, "pk_layernorm_desc.struct_size mismatch");
  const char* label = ln_label(d->label);
  if (d->precision != PK_PRECISION_F16 && d->precision != PK_PRECISION_F32)
    return fail(PK_INVALID_ARGUMENT, "%s has an unsupported precision %d", label, d->precision);
  // createDispatch (layernorm.ts:166-175)
  if (d->rows == 0 || d->channels == 0 || d->channels % 4u != 0)
    return fail(PK_RANGE_ERROR, "Invalid LayerNorm shape for %s", label);
  const uint64_t elem = d->precision == PK_PRECISION_F16 ? 2u : 4u;
  const uint64_t bytes = (uint64_t)d->rows * d->channels * elem;
  const uint64_t in_have = d->input ? d->input_bytes : 0, out_have = d->output ? d->output_bytes : 0;
  if (in_have < bytes)
    return fail(PK_RANGE_ERROR, "%s input needs %llu bytes; arena slice has %llu", label, (unsigned long long)bytes,
                (unsigned long long)in_have);
  if (out_have < bytes)
    return fail(PK_RANGE_ERROR, "%s output needs %llu bytes; arena slice has %llu", label, (unsigned long long)bytes,
                (unsigned long long)out_have);
  const uint64_t affine = (uint64_t)d->channels * 4u;
  if (!d->gamma || d->gamma_bytes != affine)
    return fail(PK_INVALID_ARGUMENT, "%s gamma must be float32 channel logical/storage [%u], %llu bytes", label,
                d->channels, (unsigned long long)affine);
  if (!d->beta || d->beta_bytes != affine)
    return fail(PK_INVALID_ARGUMENT, "%s beta must be float32 channel logical/storage [%u], %llu bytes", label,
                d->channels, (unsigned long long)affine);
  if (!aligned(d->input, 16) || !aligned(d->output, 16) || !aligned(d->gamma, 16) || !aligned(d->beta, 16))
    return fail(PK_INVALID_ARGUMENT, "%s bindings must be 16-byte aligned", label);
  if (d->has_epsilon && !(d->epsilon >= 0.0f))
    return fail(PK_INVALID_ARGUMENT, "%s epsilon must be a non-negative number", label);
  if (d->next_output) {
    // The chained LayerNorm holds the whole row in registers.
    if ((uint64_t)d->channels * elem > pk::kLayerNormChainBytes)
      return fail(PK_RANGE_ERROR, "%s chained LayerNorm needs rows of at most %u bytes", label,
                  pk::kLayerNormChainBytes);
    if (d->next_output_bytes < bytes)
      return fail(PK_RANGE_ERROR, "%s next output needs %llu bytes; arena slice has %llu", label,
                  (unsigned long long)bytes, (unsigned long long)d->next_output_bytes);
    if (!d->next_gamma || d->next_gamma_bytes != affine || !d->next_beta || d->next_beta_bytes != affine)
      return fail(PK_INVALID_ARGUMENT, "%s next gamma and beta must be float32 [%u], %llu bytes", label, d->channels,
                  (unsigned long long)affine);
    if (!aligned(d->next_output, 16) || !aligned(d->next_gamma, 16) || !aligned(d->next_beta, 16))
      return fail(PK_INVALID_ARGUMENT, "%s bindings must be 16-byte aligned", label);
    const auto at = [](const void* p) { return reinterpret_cast<uintptr_t>(p); };
    const auto overlap = [&](const void* p, const void* q) { return at(p) < at(q) + bytes && at(q) < at(p) + bytes; };
    if (overlap(d->next_output, d->output) || (d->next_output != d->input && overlap(d->next_output, d->input)))
      return fail(PK_INVALID_ARGUMENT, "%s next output must not overlap the output, and be the input or not overlap it",
                  label);
  }
  return PK_OK;
}

}  // namespace

extern "C" {

int pk_layernorm_validate(const pk_layernorm_desc* d) { return validate_layernorm_desc(d); }

int pk_layernorm_create(pk_context* ctx, const pk_layernorm_desc* d, pk_layernorm_op** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!d || !out) return fail(PK_INVALID_ARGUMENT, "LayerNorm descriptor or output is null");
  *out = nullptr;
  if (int s = validate_layernorm_desc(d)) return s;
  auto* op = new pk_layernorm_op();
  op->ctx = ctx;
  op->label = ln_label(d->label);
  op->precision = d->precision;
  op->rows = d->rows;
  op->args.input = d->input;
  op->args.gamma = d->gamma;
  op->args.beta = d->beta;
  op->args.output = d->output;
  op->args.rows = d->rows;
  op->args.channels = d->channels;
  op->args.epsilon = d->has_epsilon ? d->epsilon : 1e-5f;
  op->args.next_gamma = d->next_output ? d->next_gamma : nullptr;
  op->args.next_beta = d->next_output ? d->next_beta : nullptr;
  op->args.next_output = d->next_output;
  *out = op;
  return ok();
}

int pk_layernorm_enqueue(pk_layernorm_op* op, uint32_t active_rows, void* stream) {
  return pk_layernorm_enqueue_timed(op, active_rows, stream, nullptr, nullptr);
}

int pk_layernorm_enqueue_timed(pk_layernorm_op* op, uint32_t active_rows, void* stream, void* start_event,
                               void* end_event) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "LayerNorm op is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const uint32_t rows = active_rows ? active_rows : op->rows;
  // LayerNormDispatch.encode (layernorm.ts:45-55)
  if (rows > op->rows)
    return fail(PK_RANGE_ERROR, "%s active rows must be in [1, %u]", op->label.c_str(), op->rows);
  pk::LayerNormArgs args = op->args;
  args.rows = rows;
  PK_HIP(hipSetDevice(op->ctx->device), "hipSetDevice");
  PK_HIP(pk::launch_layernorm(op->precision == PK_PRECISION_F16, args, stream_or_default(op->ctx, stream),
                              static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(end_event)),
         "LayerNorm launch");
  return ok();
}

int pk_layernorm_destroy(pk_layernorm_op* op) {
  if (!op || op->destroyed) return ok();
  op->destroyed = true;
  return ok();
}

int pk_layernorm_release(pk_layernorm_op* op) {
  if (!op) return ok();
  pk_layernorm_destroy(op);
  delete op;
  return ok();
}

}  // extern "C"

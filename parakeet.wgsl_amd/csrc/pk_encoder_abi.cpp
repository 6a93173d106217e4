// pk_encoder_abi.cpp - the encoder layer stack composed from this library's
// ops, in the order of createEncoderLayerDispatches
// (src/webgpu/encoder.ts:1868-2135), with an optional HIP graph of a whole
// pass.
#include <hip/hip_runtime.h>

#include <map>
#include <string>
#include <vector>

#include "pk_abi_internal.h"
#include "pk_attention.h"
#include "pk_conv.h"
#include "pk_encoder.h"
#include "pk_internal.h"
#include "pk_layernorm.h"

using namespace pk_abi;

namespace {

constexpr uint32_t kC = PK_ENCODER_CHANNELS;
constexpr uint32_t kHidden = PK_ENCODER_INTERMEDIATE;
constexpr uint32_t kMaxLayers = 64;

struct LayerOps {
  pk_layernorm_op* norm[5] = {};
  pk_gemm_op* ff1a = nullptr;
  pk_gemm_op* ff1b = nullptr;
  pk_gemm_op* qkv = nullptr;
  pk_attention_op* attention = nullptr;
  pk_gemm_op* o = nullptr;
  pk_gemm_op* pw1 = nullptr;
  pk_conv_op* conv = nullptr;
  pk_gemm_op* pw2 = nullptr;
  pk_gemm_op* ff2a = nullptr;
  pk_gemm_op* ff2b = nullptr;
};

uint64_t packed_bytes(int bits, uint32_t inner, uint32_t columns) {
  return (uint64_t)inner * columns / pk::codes_per_group(bits) * pk::words_per_group(bits) * 4u;
}

}  // namespace

struct pk_encoder {
  pk_context* ctx = nullptr;
  std::string label;
  uint32_t batch = 0, frames = 0, layers = 0, rows = 0;
  bool fused_glu = false;
  const uint32_t* valid_lengths = nullptr;
  const void* input = nullptr;
  void* output = nullptr;
  void* arena = nullptr;
  uint64_t arena_bytes = 0, weight_bytes = 0;
  // Arena slices: four [rows, 1024] activation buffers, the FF hidden block,
  // QKV, the attention context, the pointwise-1 output and the conv output.
  _Float16 *a = nullptr, *b = nullptr, *c = nullptr, *d = nullptr, *h = nullptr, *qkv = nullptr, *ctxt = nullptr,
           *pw = nullptr, *cout = nullptr;
  std::vector<LayerOps> ops;
  std::map<uint32_t, hipGraphExec_t> graphs;  // per active batch
};

namespace {

void release_layer(LayerOps& l) {
  for (auto* n : l.norm) pk_layernorm_release(n);
  for (pk_gemm_op* g : {l.ff1a, l.ff1b, l.qkv, l.o, l.pw1, l.pw2, l.ff2a, l.ff2b}) pk_gemm_release(g);
  pk_attention_release(l.attention);
  pk_conv_release(l.conv);
  l = LayerOps{};
}

void release_encoder(pk_encoder* e) {
  for (auto& kv : e->graphs) (void)hipGraphExecDestroy(kv.second);
  e->graphs.clear();
  for (auto& l : e->ops) release_layer(l);
  e->ops.clear();
  if (e->arena) {
    (void)hipSetDevice(e->ctx->device);
    (void)hipFree(e->arena);
    e->arena = nullptr;
  }
}

// The fifteen ops of layer `li` over the arena (encoder.ts:1868-2135):
//   A (the input for layer 0) -LN-> B -W1-> H -W2(+0.5 A)-> B -LN-> C -QKV-> Q -att-> X -Wo(+B)-> C
//   -LN-> D -PW1-> P -conv-> O -PW2(+C)-> D -LN-> B -W1-> H -W2(+0.5 D)-> B
//   -LN-> A (the last layer writes the output instead).
// With `validate_only` the ops' descriptors are checked on the host
// (pk_*_validate) and nothing is created.
int build_layer(pk_encoder* e, const pk_encoder_layer& w, uint32_t li, hipStream_t stream, LayerOps& l,
                bool validate_only) {
  const uint64_t R = e->rows;
  const std::string prefix = e->label + ".layers." + std::to_string(li);
  std::string label;
  auto name = [&](const char* suffix) {
    label = prefix + suffix;
    return label.c_str();
  };
  auto norm = [&](int i, const char* suffix, const void* in, void* out) {
    pk_layernorm_desc d{};
    d.struct_size = sizeof d;
    d.label = name(suffix);
    d.precision = PK_PRECISION_F16;
    d.rows = e->rows;
    d.channels = kC;
    d.input = in;
    d.input_bytes = R * kC * 2;
    d.gamma = w.norm_gamma[i];
    d.gamma_bytes = kC * 4;
    d.beta = w.norm_beta[i];
    d.beta_bytes = kC * 4;
    d.output = out;
    d.output_bytes = R * kC * 2;
    return validate_only ? pk_layernorm_validate(&d) : pk_layernorm_create(e->ctx, &d, &l.norm[i]);
  };
  auto gemm = [&](pk_gemm_op** op, const char* suffix, const pk_encoder_matrix& m, int bits, uint32_t inner,
                  uint32_t columns, uint32_t groups, const void* a, void* out, const void* residual, float scale,
                  int activation, uint32_t flags) {
    pk_gemm_desc d{};
    d.struct_size = sizeof d;
    d.flags = flags;
    d.label = name(suffix);
    d.precision = PK_PRECISION_F16;
    d.palette_bits = bits;
    d.rows = e->rows;
    d.inner = inner;
    d.columns = columns;
    d.palette_groups = groups;
    d.palette_group_columns = columns / groups;
    d.a = a;
    d.a_bytes = R * inner * 2;
    d.packed = m.packed;
    d.packed_bytes = packed_bytes(bits, inner, columns);
    d.palette = m.palette;
    d.palette_bytes = (uint64_t)groups * (1u << bits) * 2;
    d.output = out;
    d.output_bytes = R * ((flags & PK_GEMM_GLU) ? columns / 2 : columns) * 2;
    d.residual = residual;
    d.residual_bytes = residual ? R * columns * 2 : 0;
    d.has_residual_scale = residual ? 1 : 0;
    d.residual_scale = scale;
    d.activation = activation;
    if (validate_only) return pk_gemm_validate(&d);
    const int s = pk_gemm_create(e->ctx, &d, stream, op);
    if (s == PK_OK) {
      e->weight_bytes += pk::pair_code_bytes(inner, columns);
      if (!(flags & PK_GEMM_GLU)) e->weight_bytes += pk::operand_order_words(bits, inner, columns) * 4u;
    }
    return s;
  };
  // Layer 0 reads the caller's input in place of A.
  const void* x = li == 0 ? e->input : e->a;
  int s;
  if ((s = norm(0, ".norm_feed_forward1", x, e->b))) return s;
  if ((s = gemm(&l.ff1a, "-feed-forward1-linear1", w.ff1_linear1, 5, kC, kHidden, 1, e->b, e->h, nullptr, 0.0f,
                PK_ACTIVATION_SILU, 0)))
    return s;
  if ((s = gemm(&l.ff1b, "-feed-forward1-linear2-residual", w.ff1_linear2, 5, kHidden, kC, 1, e->h, e->b, x, 0.5f,
                PK_ACTIVATION_NONE, 0)))
    return s;
  if ((s = norm(1, ".norm_self_att", e->b, e->c))) return s;
  if ((s = gemm(&l.qkv, "-self-attention-qkv", w.qkv, 5, kC, 3 * kC, 3, e->c, e->qkv, nullptr, 0.0f,
                PK_ACTIVATION_NONE, 0)))
    return s;
  {
    pk_attention_desc d{};
    d.struct_size = sizeof d;
    d.label = name("-relative-attention");
    d.precision = PK_PRECISION_F16;
    d.batch_size = e->batch;
    d.frames = e->frames;
    d.qkv = e->qkv;
    d.qkv_bytes = R * 3 * kC * 2;
    d.projected_positions = w.projected_positions;
    d.projected_positions_bytes = (2ull * e->frames - 1u) * kC * 2;
    d.bias_u = w.bias_u;
    d.bias_u_bytes = 4096;
    d.bias_v = w.bias_v;
    d.bias_v_bytes = 4096;
    d.valid_lengths = e->valid_lengths;
    d.valid_lengths_bytes = (uint64_t)e->batch * 4u;
    d.output = e->ctxt;
    d.output_bytes = R * kC * 2;
    if ((s = validate_only ? pk_attention_validate(&d) : pk_attention_create(e->ctx, &d, &l.attention))) return s;
  }
  if ((s = gemm(&l.o, "-self-attention-output-residual", w.o_proj, 6, kC, kC, 1, e->ctxt, e->c, e->b, 1.0f,
                PK_ACTIVATION_NONE, 0)))
    return s;
  if ((s = norm(2, ".norm_conv", e->c, e->d))) return s;
  if ((s = gemm(&l.pw1, "-convolution-pointwise1", w.pointwise1, 5, kC, 2 * kC, 1, e->d, e->pw, nullptr, 0.0f,
                PK_ACTIVATION_NONE, e->fused_glu ? PK_GEMM_GLU : 0u)))
    return s;
  {
    pk_conv_desc d{};
    d.struct_size = sizeof d;
    d.flags = e->fused_glu ? PK_CONV_INPUT_GLU : 0u;
    d.label = name("-convolution-glu-depthwise-bn-silu");
    d.precision = PK_PRECISION_F16;
    d.batch_size = e->batch;
    d.frames = e->frames;
    d.channels = kC;
    d.pointwise_input = e->pw;
    d.pointwise_input_bytes = R * (e->fused_glu ? kC : 2 * kC) * 2;
    d.depthwise_weights = w.depthwise;
    d.depthwise_weights_bytes = 9ull * kC * 2;
    d.batch_norm_scale = w.bn_scale;
    d.batch_norm_scale_bytes = kC * 4;
    d.batch_norm_shift = w.bn_shift;
    d.batch_norm_shift_bytes = kC * 4;
    d.valid_lengths = e->valid_lengths;
    d.valid_lengths_bytes = (uint64_t)e->batch * 4u;
    d.output = e->cout;
    d.output_bytes = R * kC * 2;
    if ((s = validate_only ? pk_conv_validate(&d) : pk_conv_create(e->ctx, &d, &l.conv))) return s;
  }
  if ((s = gemm(&l.pw2, "-convolution-pointwise2-residual", w.pointwise2, 5, kC, kC, 1, e->cout, e->d, e->c, 1.0f,
                PK_ACTIVATION_NONE, 0)))
    return s;
  if ((s = norm(3, ".norm_feed_forward2", e->d, e->b))) return s;
  if ((s = gemm(&l.ff2a, "-feed-forward2-linear1", w.ff2_linear1, 5, kC, kHidden, 1, e->b, e->h, nullptr, 0.0f,
                PK_ACTIVATION_SILU, 0)))
    return s;
  if ((s = gemm(&l.ff2b, "-feed-forward2-linear2-residual", w.ff2_linear2, 5, kHidden, kC, 1, e->h, e->b, e->d,
                0.5f, PK_ACTIVATION_NONE, 0)))
    return s;
  const bool last = li + 1 == e->layers;
  return norm(4, ".norm_out", e->b, last ? e->output : e->a);
}

// One pass over the first `batch` windows on `stream`. With `starts` /
// `ends` (15 per layer, in dispatch order; NULL entries skip), each launch's
// own dispatch stamps its pair of events.
int enqueue_pass(pk_encoder* e, uint32_t batch, hipStream_t stream, void* const* starts = nullptr,
                 void* const* ends = nullptr) {
  const uint32_t rows = batch * e->frames;
  uint32_t slot = 0;
  auto ev = [&](void* const* list) { return list ? list[slot] : nullptr; };
  auto norm = [&](pk_layernorm_op* op) {
    const int s = pk_layernorm_enqueue_timed(op, rows, stream, ev(starts), ev(ends));
    ++slot;
    return s;
  };
  auto gemm = [&](pk_gemm_op* op) {
    const int s = pk_gemm_enqueue_timed(op, rows, stream, ev(starts), ev(ends));
    ++slot;
    return s;
  };
  for (LayerOps& l : e->ops) {
    int s;
    if ((s = norm(l.norm[0])) || (s = gemm(l.ff1a)) || (s = gemm(l.ff1b)) || (s = norm(l.norm[1])) ||
        (s = gemm(l.qkv)))
      return s;
    if ((s = pk_attention_enqueue_timed(l.attention, batch, stream, ev(starts), ev(ends)))) return s;
    ++slot;
    if ((s = gemm(l.o)) || (s = norm(l.norm[2])) || (s = gemm(l.pw1))) return s;
    if ((s = pk_conv_enqueue_timed(l.conv, batch, stream, ev(starts), ev(ends)))) return s;
    ++slot;
    if ((s = gemm(l.pw2)) || (s = norm(l.norm[3])) || (s = gemm(l.ff2a)) || (s = gemm(l.ff2b)) ||
        (s = norm(l.norm[4])))
      return s;
  }
  return PK_OK;
}

// Arena slices: A, B, C, D [rows, 1024], H [rows, 4096], QKV [rows, 3072],
// the attention context [rows, 1024], the pointwise-1 output ([rows, 2048],
// or [rows, 1024] with the GLU epilogue) and the conv output [rows, 1024],
// each 256-byte aligned. Returns the bytes used from `base`.
uint64_t place_arena(pk_encoder* e, uint8_t* base) {
  const uint64_t R = e->rows;
  const uint64_t elems[9] = {R * kC, R * kC, R * kC, R * kC, R * kHidden, R * 3 * kC, R * kC,
                             R * (e->fused_glu ? kC : 2 * kC), R * kC};
  _Float16** slots[9] = {&e->a, &e->b, &e->c, &e->d, &e->h, &e->qkv, &e->ctxt, &e->pw, &e->cout};
  uint64_t at = 0;
  for (int i = 0; i < 9; ++i) {
    if (base) *slots[i] = reinterpret_cast<_Float16*>(base + at);
    at += (elems[i] * 2 + 255u) / 256u * 256u;
  }
  return at;
}

uint64_t arena_bytes(pk_encoder* e) { return place_arena(e, nullptr); }

void describe(pk_encoder* e, const pk_encoder_desc* d) {
  e->label = d->label ? d->label : "encoder";
  e->batch = d->batch_size;
  e->frames = d->frames;
  e->layers = d->layers;
  e->rows = d->batch_size * d->frames;
  e->fused_glu = (d->flags & PK_ENCODER_FUSED_GLU) != 0;
  e->valid_lengths = d->valid_lengths;
  e->input = d->input;
  e->output = d->output;
}

int validate_encoder_desc(const pk_encoder_desc* d) {
  if (!d) return fail(PK_INVALID_ARGUMENT, "encoder descriptor is null");
  if (d->struct_size != sizeof(pk_encoder_desc))
    return fail(PK_INVALID_ARGUMENT, "pk_encoder_desc.struct_size mismatch");
  const char* label = d->label ? d->label : "encoder";
  if (d->flags & ~PK_ENCODER_FUSED_GLU) return fail(PK_INVALID_ARGUMENT, "%s has unknown flags 0x%x", label, d->flags);
  if (d->precision != PK_PRECISION_F16)
    return fail(PK_INVALID_ARGUMENT, "%s: the encoder stack runs in f16", label);
  if (d->batch_size == 0 || d->frames == 0 || d->layers == 0 || d->layers > kMaxLayers)
    return fail(PK_RANGE_ERROR, "Unsupported encoder shape for %s: %u windows x %u frames x %u layers", label,
                d->batch_size, d->frames, d->layers);
  if (!d->layer || !d->valid_lengths || !d->input || !d->output)
    return fail(PK_INVALID_ARGUMENT, "%s needs layer weights, valid lengths, input and output", label);
  if (!aligned(d->input, 16) || !aligned(d->output, 16))
    return fail(PK_INVALID_ARGUMENT, "%s input and output must be 16-byte aligned", label);
  const uintptr_t bytes = (uintptr_t)d->batch_size * d->frames * kC * 2;
  const uintptr_t in = reinterpret_cast<uintptr_t>(d->input), out = reinterpret_cast<uintptr_t>(d->output);
  if (in < out + bytes && out < in + bytes)
    return fail(PK_INVALID_ARGUMENT, "%s output must not overlap its input", label);
  return PK_OK;
}

}  // namespace

extern "C" {

int pk_encoder_create(pk_context* ctx, const pk_encoder_desc* d, void* stream, pk_encoder** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!out) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  *out = nullptr;
  if (int s = validate_encoder_desc(d)) return s;
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  auto* e = new pk_encoder();
  e->ctx = ctx;
  describe(e, d);
  hipError_t err = hipMalloc(&e->arena, arena_bytes(e));
  if (err != hipSuccess) {
    const uint64_t total = arena_bytes(e);
    delete e;
    return fail(PK_ALLOCATION_FAILURE, "cannot allocate the %llu-byte encoder arena: %s", (unsigned long long)total,
                hipGetErrorString(err));
  }
  e->arena_bytes = place_arena(e, static_cast<uint8_t*>(e->arena));
  e->ops.resize(e->layers);
  for (uint32_t li = 0; li < e->layers; ++li) {
    if (int s = build_layer(e, d->layer[li], li, stream_or_default(ctx, stream), e->ops[li], false)) {
      const std::string message = g_error;
      release_encoder(e);
      delete e;
      return fail(s, "%s", message.c_str());
    }
  }
  *out = e;
  return ok();
}

int pk_encoder_validate(const pk_encoder_desc* d) {
  if (int s = validate_encoder_desc(d)) return s;
  // Check every op's descriptor over an arena placed at a nominal,
  // suitably aligned address; nothing is dereferenced.
  pk_encoder e;
  describe(&e, d);
  place_arena(&e, reinterpret_cast<uint8_t*>(uintptr_t(1) << 40));
  LayerOps unused;
  for (uint32_t li = 0; li < e.layers; ++li)
    if (int s = build_layer(&e, d->layer[li], li, nullptr, unused, true)) return s;
  return ok();
}

int pk_encoder_enqueue(pk_encoder* e, uint32_t active_batch, void* stream, int use_graph) {
  if (!e) return fail(PK_INVALID_ARGUMENT, "encoder is null");
  const uint32_t batch = active_batch ? active_batch : e->batch;
  if (batch > e->batch)
    return fail(PK_RANGE_ERROR, "%s active batch must be in [1, %u]", e->label.c_str(), e->batch);
  hipStream_t st = stream_or_default(e->ctx, stream);
  PK_HIP(hipSetDevice(e->ctx->device), "hipSetDevice");
  if (!use_graph) return enqueue_pass(e, batch, st);
  auto it = e->graphs.find(batch);
  if (it == e->graphs.end()) {
    // Capture one pass on this stream: kernel nodes only.
    PK_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    const int s = enqueue_pass(e, batch, st);
    hipGraph_t graph = nullptr;
    const hipError_t end = hipStreamEndCapture(st, &graph);
    if (s != PK_OK) {
      if (graph) (void)hipGraphDestroy(graph);
      return s;
    }
    PK_HIP(end, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    PK_HIP(inst, "hipGraphInstantiate");
    it = e->graphs.emplace(batch, exec).first;
  }
  PK_HIP(hipGraphLaunch(it->second, st), "hipGraphLaunch");
  return ok();
}

int pk_encoder_enqueue_profiled(pk_encoder* e, uint32_t active_batch, void* stream, void* const* start_events,
                                void* const* end_events) {
  if (!e) return fail(PK_INVALID_ARGUMENT, "encoder is null");
  const uint32_t batch = active_batch ? active_batch : e->batch;
  if (batch > e->batch)
    return fail(PK_RANGE_ERROR, "%s active batch must be in [1, %u]", e->label.c_str(), e->batch);
  PK_HIP(hipSetDevice(e->ctx->device), "hipSetDevice");
  return enqueue_pass(e, batch, stream_or_default(e->ctx, stream), start_events, end_events);
}

int pk_encoder_info(const pk_encoder* e, uint32_t* launches, uint64_t* device_bytes) {
  if (!e) return fail(PK_INVALID_ARGUMENT, "encoder is null");
  if (launches) *launches = 15u * e->layers;
  if (device_bytes) *device_bytes = e->arena_bytes + e->weight_bytes;
  return ok();
}

int pk_encoder_destroy(pk_encoder* e) {
  if (!e) return ok();
  (void)hipSetDevice(e->ctx->device);
  (void)hipStreamSynchronize(e->ctx->stream);
  release_encoder(e);
  delete e;
  return ok();
}

}  // extern "C"

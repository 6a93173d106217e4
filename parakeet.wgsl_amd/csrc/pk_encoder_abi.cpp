// pk_encoder_abi.cpp - the encoder graph composed from this library's ops:
// the optional subsampling front end (createSubsamplingCommands,
// src/webgpu/encoder.ts:2140-2400), the layer stack in the order of
// createEncoderLayerDispatches (:1868-2135) and the optional projector
// (:1489-1509), with an optional HIP graph of a whole pass.
//
// Windows are never split into microbatches: the reference runs the front
// end three windows at a time to bound its WebGPU arena (encoder.ts:80,
// :1599-1624); with HBM to spare here, every stage runs once over all
// active windows, which keeps each GEMM's M large.
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
#include "pk_subsampling.h"

using namespace pk_abi;

namespace {

constexpr uint32_t kC = PK_ENCODER_CHANNELS;
constexpr uint32_t kHidden = PK_ENCODER_INTERMEDIATE;
constexpr uint32_t kMaxLayers = 64;
constexpr uint32_t kSubC = PK_SUBSAMPLING_CHANNELS;
constexpr uint32_t kBins = PK_SUBSAMPLING_BINS;
constexpr uint32_t kFrontLaunches = 6;

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

struct FrontOps {
  pk_subsampling_op* fused = nullptr;
  pk_gemm_op* pointwise3 = nullptr;
  pk_subsampling_op* depthwise5 = nullptr;
  pk_gemm_op* pointwise6 = nullptr;
  pk_subsampling_op* mask = nullptr;
  pk_gemm_op* linear = nullptr;
};

uint64_t packed_bytes(int bits, uint32_t inner, uint32_t columns) {
  return (uint64_t)inner * columns / pk::codes_per_group(bits) * pk::words_per_group(bits) * 4u;
}

uint32_t halve(uint32_t n, uint32_t steps) { return pk_subsampling_valid_length(n, steps); }

}  // namespace

struct pk_encoder {
  pk_abi::CtxRef ctx;
  std::string label;
  uint32_t batch = 0, frames = 0, layers = 0, rows = 0;
  int precision = PK_PRECISION_F16;  // of the activations, palettes and per-channel tensors
  uint64_t elem = 2;                 // bytes per element in that precision
  bool fused_glu = true;
  bool fused_norms = false;
  bool chained_norms = true;  // norm_out also writes the next layer's norm_feed_forward1
  bool prefix_same_plan = false;  // prefixes keep the capacity's kernel families (PK_ENCODER_PREFIX_SAME_PLAN)
  const uint32_t* valid_lengths = nullptr;
  const void* input = nullptr;
  void* output = nullptr;
  // front end
  bool front = false;
  uint32_t feature_frames = 0, front_height = 0;  // fbank frames, rows after two stride-2 stages
  const uint32_t* feature_lengths = nullptr;
  // projector
  uint32_t projected_channels = 0;
  void* projected_output = nullptr;

  void* arena = nullptr;
  uint64_t arena_bytes = 0, weight_bytes = 0;
  // Arena slices: four [rows, 1024] activation buffers, the FF hidden block,
  // QKV, the attention context, the pointwise-1 output, the conv output and,
  // with the front end, two [windows, H2, 32, 256] stage buffers.
  void *a = nullptr, *b = nullptr, *c = nullptr, *d = nullptr, *h = nullptr, *qkv = nullptr, *ctxt = nullptr,
           *pw = nullptr, *cout = nullptr, *s1 = nullptr, *s2 = nullptr;
  FrontOps front_ops;
  std::vector<LayerOps> ops;
  pk_gemm_op* projector = nullptr;
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
  FrontOps& f = e->front_ops;
  for (pk_subsampling_op* op : {f.fused, f.depthwise5, f.mask}) pk_subsampling_release(op);
  for (pk_gemm_op* op : {f.pointwise3, f.pointwise6, f.linear}) pk_gemm_release(op);
  f = FrontOps{};
  for (auto& l : e->ops) release_layer(l);
  e->ops.clear();
  pk_gemm_release(e->projector);
  e->projector = nullptr;
  free_after_drain(e->ctx->device, e->arena);
  e->arena = nullptr;
}

// One palette GEMM of the graph, in the encoder's precision, over `rows` rows.
struct GemmSpec {
  pk_encoder_matrix matrix;
  int bits = 5;
  uint32_t rows = 0, inner = 0, columns = 0, groups = 1;
  const void* a = nullptr;
  void* out = nullptr;
  const float* bias = nullptr;
  const void* residual = nullptr;
  float scale = 0.0f;
  int activation = PK_ACTIVATION_NONE;
  uint32_t flags = 0;
  const float* norm_gamma = nullptr;  // with PK_GEMM_ROW_NORM
  const float* norm_beta = nullptr;
};

// With `validate_only` the descriptor is checked on the host
// (pk_gemm_validate) and nothing is created.
int make_gemm(pk_encoder* e, const std::string& label, const GemmSpec& g, hipStream_t stream, pk_gemm_op** op,
              bool validate_only) {
  const uint64_t R = g.rows;
  pk_gemm_desc d{};
  d.struct_size = sizeof d;
  d.flags = g.flags;
  d.label = label.c_str();
  d.precision = e->precision;
  d.palette_bits = g.bits;
  d.rows = g.rows;
  d.inner = g.inner;
  d.columns = g.columns;
  d.palette_groups = g.groups;
  d.palette_group_columns = g.columns / g.groups;
  d.a = g.a;
  d.a_bytes = R * g.inner * e->elem;
  d.packed = g.matrix.packed;
  d.packed_bytes = packed_bytes(g.bits, g.inner, g.columns);
  d.palette = g.matrix.palette;
  d.palette_bytes = (uint64_t)g.groups * (1u << g.bits) * e->elem;
  d.output = g.out;
  d.output_bytes = R * ((g.flags & PK_GEMM_GLU) ? g.columns / 2 : g.columns) * e->elem;
  d.bias = g.bias;
  d.bias_bytes = g.bias ? (uint64_t)g.columns * 4u : 0;
  d.residual = g.residual;
  d.residual_bytes = g.residual ? R * g.columns * e->elem : 0;
  d.has_residual_scale = g.residual ? 1 : 0;
  d.residual_scale = g.scale;
  d.activation = g.activation;
  if (g.flags & PK_GEMM_ROW_NORM) {
    d.norm_gamma = g.norm_gamma;
    d.norm_gamma_bytes = (uint64_t)g.inner * 4u;
    d.norm_beta = g.norm_beta;
    d.norm_beta_bytes = (uint64_t)g.inner * 4u;
    d.norm_epsilon = 1e-5f;
  }
  if (validate_only) return pk_gemm_validate(&d);
  const int s = pk_gemm_create(e->ctx, &d, stream, op);
  if (s == PK_OK) e->weight_bytes += gemm_weight_bytes(*op);
  return s;
}

// The front end over the fbank (createSubsamplingCommands, encoder.ts:
// 2140-2400; labels follow its dispatch labels):
//   fbank -conv0+dw2-> S1 [W, H2, 32, 256] -PW3+ReLU-> S2 -DW5-> S1
//   [W, H3, 16, 256] -PW6+ReLU-> S2 -mask-> S2 -linear-> A [W*H3, 1024]
int build_front(pk_encoder* e, const pk_encoder_subsampling& w, hipStream_t stream, FrontOps& f,
                bool validate_only) {
  const std::string prefix = e->label + ".subsampling-";
  const uint32_t h2 = e->front_height, h3 = e->frames, w2 = halve(kBins, 2), w3 = halve(kBins, 3);
  const uint64_t stage2 = (uint64_t)e->batch * h2 * w2 * kSubC * e->elem;
  const uint64_t stage3 = (uint64_t)e->batch * h3 * w3 * kSubC * e->elem;
  std::string label;
  int s;
  {
    label = prefix + "fused-conv0-depthwise2";
    pk_subsampling_fused_desc d{};
    d.struct_size = sizeof d;
    d.label = label.c_str();
    d.precision = e->precision;
    d.batch_size = e->batch;
    d.input_height = e->feature_frames;
    d.input_width = kBins;
    d.channels = kSubC;
    d.input = static_cast<const float*>(e->input);
    d.input_bytes = (uint64_t)e->batch * kBins * e->feature_frames * 4u;
    d.conv0_weights = w.conv0_weights;
    d.conv0_weights_bytes = 9ull * kSubC * e->elem;
    d.conv0_bias = w.conv0_bias;
    d.conv0_bias_bytes = kSubC * 4u;
    d.depthwise_weights = w.depthwise2_weights;
    d.depthwise_weights_bytes = 9ull * kSubC * e->elem;
    d.depthwise_bias = w.depthwise2_bias;
    d.depthwise_bias_bytes = kSubC * 4u;
    d.output = e->s1;
    d.output_bytes = stage2;
    d.valid_lengths = e->feature_lengths;
    d.valid_lengths_bytes = (uint64_t)e->batch * 4u;
    if ((s = validate_only ? pk_subsampling_fused_validate(&d) : pk_subsampling_fused_create(e->ctx, &d, &f.fused)))
      return s;
  }
  GemmSpec g;
  g.matrix = w.pointwise3;
  g.rows = e->batch * h2 * w2;
  g.inner = g.columns = kSubC;
  g.a = e->s1;
  g.out = e->s2;
  g.bias = w.pointwise3_bias;
  g.activation = PK_ACTIVATION_RELU;
  // The depthwise convolution reads it next, bandwidth-bound: at 16
  // windows streamed stores would take 5 us off this GEMM and add 8.5 us
  // to the convolution.
  g.flags = PK_GEMM_CACHED_OUTPUT;
  if ((s = make_gemm(e, prefix + "pointwise3", g, stream, &f.pointwise3, validate_only))) return s;
  {
    label = prefix + "depthwise5";
    pk_subsampling_depthwise_desc d{};
    d.struct_size = sizeof d;
    d.label = label.c_str();
    d.precision = e->precision;
    d.batch_size = e->batch;
    d.input_height = h2;
    d.input_width = w2;
    d.channels = kSubC;
    d.input = e->s2;
    d.input_bytes = stage2;
    d.weights = w.depthwise5_weights;
    d.weights_bytes = 9ull * kSubC * e->elem;
    d.bias = w.depthwise5_bias;
    d.bias_bytes = kSubC * 4u;
    d.output = e->s1;
    d.output_bytes = stage3;
    d.valid_lengths = e->feature_lengths;
    d.valid_lengths_bytes = (uint64_t)e->batch * 4u;
    d.valid_length_subsampling_steps = 3;
    if ((s = validate_only ? pk_subsampling_depthwise_validate(&d)
                           : pk_subsampling_depthwise_create(e->ctx, &d, &f.depthwise5)))
      return s;
  }
  g = GemmSpec{};
  g.matrix = w.pointwise6;
  g.rows = e->batch * h3 * w3;
  g.inner = g.columns = kSubC;
  g.a = e->s1;
  g.out = e->s2;
  g.bias = w.pointwise6_bias;
  g.activation = PK_ACTIVATION_RELU;
  if ((s = make_gemm(e, prefix + "pointwise6", g, stream, &f.pointwise6, validate_only))) return s;
  {
    // Pointwise 6 can turn zero rows past the length into its ReLU'd bias,
    // so its rows there are cleared before the flatten (encoder.ts:2361-2391).
    label = prefix + "pointwise6-mask";
    pk_subsampling_mask_desc d{};
    d.struct_size = sizeof d;
    d.label = label.c_str();
    d.precision = e->precision;
    d.batch_size = e->batch;
    d.height = h3;
    d.width = w3;
    d.channels = kSubC;
    d.values = e->s2;
    d.values_bytes = stage3;
    d.valid_lengths = e->feature_lengths;
    d.valid_lengths_bytes = (uint64_t)e->batch * 4u;
    d.valid_length_subsampling_steps = 3;
    if ((s = validate_only ? pk_subsampling_mask_validate(&d) : pk_subsampling_mask_create(e->ctx, &d, &f.mask)))
      return s;
  }
  g = GemmSpec{};
  g.matrix = w.linear;
  g.rows = e->rows;
  g.inner = w3 * kSubC;
  g.columns = kC;
  g.a = e->s2;
  g.out = e->a;
  g.bias = w.linear_bias;
  return make_gemm(e, prefix + "flatten-project", g, stream, &f.linear, validate_only);
}

// The fifteen ops of layer `li` over the arena (encoder.ts:1868-2135):
//   A (the caller's input for layer 0 without the front end) -LN-> B -W1->
//   H -W2(+0.5 A)-> B -LN-> C -QKV-> Q -att-> X -Wo(+B)-> C -LN-> D -PW1->
//   P -conv-> O -PW2(+C)-> D -LN-> B -W1-> H -W2(+0.5 D)-> B -LN-> A (the
//   last layer writes the output instead). With PK_ENCODER_FUSED_NORMS the
//   four LayerNorms before W1, QKV, PW1 and W1 are not created: those GEMMs
//   read the LayerNorm's input (A, B, C, D) with PK_GEMM_ROW_NORM. Otherwise,
//   unless PK_ENCODER_UNCHAINED_NORMS, the last LayerNorm of a layer also
//   writes B = LN ff1(A) of the layer `next` (a chained LayerNorm) and that
//   layer creates no LayerNorm of its own there.
int build_layer(pk_encoder* e, const pk_encoder_layer& w, const pk_encoder_layer* next, uint32_t li,
                hipStream_t stream, LayerOps& l, bool validate_only) {
  const uint64_t R = e->rows;
  const std::string prefix = e->label + ".layers." + std::to_string(li);
  std::string label;
  auto name = [&](const char* suffix) {
    label = prefix + suffix;
    return label.c_str();
  };
  auto norm = [&](int i, const char* suffix, const void* in, void* out, void* chained_out = nullptr) {
    pk_layernorm_desc d{};
    d.struct_size = sizeof d;
    d.label = name(suffix);
    d.precision = e->precision;
    d.rows = e->rows;
    d.channels = kC;
    d.input = in;
    d.input_bytes = R * kC * e->elem;
    d.gamma = w.norm_gamma[i];
    d.gamma_bytes = kC * 4;
    d.beta = w.norm_beta[i];
    d.beta_bytes = kC * 4;
    d.output = out;
    d.output_bytes = R * kC * e->elem;
    if (chained_out) {
      d.next_gamma = next->norm_gamma[0];
      d.next_gamma_bytes = kC * 4;
      d.next_beta = next->norm_beta[0];
      d.next_beta_bytes = kC * 4;
      d.next_output = chained_out;
      d.next_output_bytes = R * kC * e->elem;
    }
    return validate_only ? pk_layernorm_validate(&d) : pk_layernorm_create(e->ctx, &d, &l.norm[i]);
  };
  // LayerNorm i runs inside the GEMM it feeds (not with the GLU epilogue).
  auto fused = [&](int i) { return e->fused_norms && !(i == 2 && e->fused_glu); };
  int norm_of = -1;  // the LayerNorm the next gemm() call fuses
  auto gemm = [&](pk_gemm_op** op, const char* suffix, const pk_encoder_matrix& m, int bits, uint32_t inner,
                  uint32_t columns, uint32_t groups, const void* a, void* out, const void* residual, float scale,
                  int activation, uint32_t flags) {
    GemmSpec g;
    if (norm_of >= 0) {
      flags |= PK_GEMM_ROW_NORM;
      g.norm_gamma = w.norm_gamma[norm_of];
      g.norm_beta = w.norm_beta[norm_of];
      norm_of = -1;
    }
    g.matrix = m;
    g.bits = bits;
    g.rows = e->rows;
    g.inner = inner;
    g.columns = columns;
    g.groups = groups;
    g.a = a;
    g.out = out;
    g.residual = residual;
    g.scale = scale;
    g.activation = activation;
    g.flags = flags;
    return make_gemm(e, prefix + suffix, g, stream, op, validate_only);
  };
  const void* x = (li == 0 && !e->front) ? e->input : e->a;
  int s;
  // The input of a fused LayerNorm's GEMM, or the separate LayerNorm.
  auto norm_into = [&](int i, const char* suffix, const void* in, void* out) -> const void* {
    if (fused(i)) {
      norm_of = i;
      return in;
    }
    s = norm(i, suffix, in, out);
    return out;
  };
  s = PK_OK;
  // A chained LayerNorm of the layer before wrote B = LN ff1(A) already.
  const bool chained_in = e->chained_norms && li > 0;
  const void* in = chained_in ? e->b : norm_into(0, ".norm_feed_forward1", x, e->b);
  if (s || (s = gemm(&l.ff1a, "-feed-forward1-linear1", w.ff1_linear1, 5, kC, kHidden, 1, in, e->h, nullptr, 0.0f,
                     PK_ACTIVATION_SILU, 0)))
    return s;
  if ((s = gemm(&l.ff1b, "-feed-forward1-linear2-residual", w.ff1_linear2, 5, kHidden, kC, 1, e->h, e->b, x, 0.5f,
                PK_ACTIVATION_NONE, 0)))
    return s;
  in = norm_into(1, ".norm_self_att", e->b, e->c);
  if (s || (s = gemm(&l.qkv, "-self-attention-qkv", w.qkv, 5, kC, 3 * kC, 3, in, e->qkv, nullptr, 0.0f,
                     PK_ACTIVATION_NONE, 0)))
    return s;
  {
    pk_attention_desc d{};
    d.struct_size = sizeof d;
    d.label = name("-relative-attention");
    d.flags = e->prefix_same_plan ? 0u : PK_ATTENTION_PLAN_ACTIVE;
    d.precision = e->precision;
    d.batch_size = e->batch;
    d.frames = e->frames;
    d.qkv = e->qkv;
    d.qkv_bytes = R * 3 * kC * e->elem;
    d.projected_positions = w.projected_positions;
    d.projected_positions_bytes = (2ull * e->frames - 1u) * kC * e->elem;
    d.bias_u = w.bias_u;
    d.bias_u_bytes = 4096;
    d.bias_v = w.bias_v;
    d.bias_v_bytes = 4096;
    d.valid_lengths = e->valid_lengths;
    d.valid_lengths_bytes = (uint64_t)e->batch * 4u;
    d.output = e->ctxt;
    d.output_bytes = R * kC * e->elem;
    if ((s = validate_only ? pk_attention_validate(&d) : pk_attention_create(e->ctx, &d, &l.attention))) return s;
  }
  if ((s = gemm(&l.o, "-self-attention-output-residual", w.o_proj, 6, kC, kC, 1, e->ctxt, e->c, e->b, 1.0f,
                PK_ACTIVATION_NONE, 0)))
    return s;
  in = norm_into(2, ".norm_conv", e->c, e->d);
  if (s || (s = gemm(&l.pw1, "-convolution-pointwise1", w.pointwise1, 5, kC, 2 * kC, 1, in, e->pw, nullptr, 0.0f,
                     PK_ACTIVATION_NONE, e->fused_glu ? PK_GEMM_GLU : 0u)))
    return s;
  {
    pk_conv_desc d{};
    d.struct_size = sizeof d;
    d.flags = e->fused_glu ? PK_CONV_INPUT_GLU : 0u;
    d.label = name("-convolution-glu-depthwise-bn-silu");
    d.precision = e->precision;
    d.batch_size = e->batch;
    d.frames = e->frames;
    d.channels = kC;
    d.pointwise_input = e->pw;
    d.pointwise_input_bytes = R * (e->fused_glu ? kC : 2 * kC) * e->elem;
    d.depthwise_weights = w.depthwise;
    d.depthwise_weights_bytes = 9ull * kC * e->elem;
    d.batch_norm_scale = w.bn_scale;
    d.batch_norm_scale_bytes = kC * 4;
    d.batch_norm_shift = w.bn_shift;
    d.batch_norm_shift_bytes = kC * 4;
    d.valid_lengths = e->valid_lengths;
    d.valid_lengths_bytes = (uint64_t)e->batch * 4u;
    d.output = e->cout;
    d.output_bytes = R * kC * e->elem;
    if ((s = validate_only ? pk_conv_validate(&d) : pk_conv_create(e->ctx, &d, &l.conv))) return s;
  }
  if ((s = gemm(&l.pw2, "-convolution-pointwise2-residual", w.pointwise2, 5, kC, kC, 1, e->cout, e->d, e->c, 1.0f,
                PK_ACTIVATION_NONE, 0)))
    return s;
  in = norm_into(3, ".norm_feed_forward2", e->d, e->b);
  if (s || (s = gemm(&l.ff2a, "-feed-forward2-linear1", w.ff2_linear1, 5, kC, kHidden, 1, in, e->h, nullptr, 0.0f,
                     PK_ACTIVATION_SILU, 0)))
    return s;
  const bool last = li + 1 == e->layers;
  void* out_norm = last ? e->output : e->a;
  void* chained_ff1 = e->chained_norms && next ? e->b : nullptr;
  if ((s = gemm(&l.ff2b, "-feed-forward2-linear2-residual", w.ff2_linear2, 5, kHidden, kC, 1, e->h, e->b, e->d,
                0.5f, PK_ACTIVATION_NONE, 0)))
    return s;
  return norm(4, ".norm_out", e->b, out_norm, chained_ff1);
}

int build_projector(pk_encoder* e, const pk_encoder_desc* d, hipStream_t stream, pk_gemm_op** op,
                    bool validate_only) {
  GemmSpec g;
  g.matrix = d->projector;
  g.rows = e->rows;
  g.inner = kC;
  g.columns = e->projected_channels;
  g.a = e->output;
  g.out = e->projected_output;
  g.bias = d->projector_bias;
  return make_gemm(e, e->label + "-projector", g, stream, op, validate_only);
}

uint32_t launch_count(const pk_encoder* e) {
  return (e->front ? kFrontLaunches : 0u) + 15u * e->layers + (e->projected_channels ? 1u : 0u);
}

// One pass over the first `batch` windows on `stream`: the front end, the
// layers, the projector. With `starts` / `ends` (one entry per launch, in
// order; NULL entries skip), each launch's own dispatch stamps its events.
int enqueue_pass(pk_encoder* e, uint32_t batch, hipStream_t stream, void* const* starts = nullptr,
                 void* const* ends = nullptr) {
  const uint32_t rows = batch * e->frames;
  uint32_t slot = 0;
  auto ev = [&](void* const* list) { return list ? list[slot] : nullptr; };
  // A LayerNorm slot: its launch, or for a LayerNorm fused into the next
  // GEMM its two events back to back.
  auto norm = [&](pk_layernorm_op* op) {
    int s = PK_OK;
    if (op) {
      s = pk_layernorm_enqueue_timed(op, rows, stream, ev(starts), ev(ends));
    } else {
      hipError_t err = hipSuccess;
      if (ev(starts)) err = hipEventRecord(static_cast<hipEvent_t>(ev(starts)), stream);
      if (err == hipSuccess && ev(ends)) err = hipEventRecord(static_cast<hipEvent_t>(ev(ends)), stream);
      if (err != hipSuccess) s = fail(PK_DEVICE_ERROR, "event record failed: %s", hipGetErrorString(err));
    }
    ++slot;
    return s;
  };
  auto gemm = [&](pk_gemm_op* op, uint32_t active_rows) {
    const int s = pk_gemm_enqueue_timed(op, active_rows, stream, ev(starts), ev(ends));
    ++slot;
    return s;
  };
  auto sub = [&](pk_subsampling_op* op) {
    const int s = pk_subsampling_enqueue_timed(op, batch, stream, ev(starts), ev(ends));
    ++slot;
    return s;
  };
  int s;
  if (e->front) {
    const FrontOps& f = e->front_ops;
    const uint32_t w2 = halve(kBins, 2), w3 = halve(kBins, 3);
    if ((s = sub(f.fused)) || (s = gemm(f.pointwise3, batch * e->front_height * w2)) || (s = sub(f.depthwise5)) ||
        (s = gemm(f.pointwise6, batch * e->frames * w3)) || (s = sub(f.mask)) || (s = gemm(f.linear, rows)))
      return s;
  }
  for (LayerOps& l : e->ops) {
    if ((s = norm(l.norm[0])) || (s = gemm(l.ff1a, rows)) || (s = gemm(l.ff1b, rows)) || (s = norm(l.norm[1])) ||
        (s = gemm(l.qkv, rows)))
      return s;
    if ((s = pk_attention_enqueue_timed(l.attention, batch, stream, ev(starts), ev(ends)))) return s;
    ++slot;
    if ((s = gemm(l.o, rows)) || (s = norm(l.norm[2])) || (s = gemm(l.pw1, rows))) return s;
    if ((s = pk_conv_enqueue_timed(l.conv, batch, stream, ev(starts), ev(ends)))) return s;
    ++slot;
    if ((s = gemm(l.pw2, rows)) || (s = norm(l.norm[3])) || (s = gemm(l.ff2a, rows)) || (s = gemm(l.ff2b, rows)) ||
        (s = norm(l.norm[4])))
      return s;
  }
  if (e->projector && (s = gemm(e->projector, rows))) return s;
  return PK_OK;
}

// Arena slices (256-byte aligned): A, B, C, D [rows, 1024], H [rows, 4096],
// QKV [rows, 3072], the attention context [rows, 1024], the pointwise-1
// output ([rows, 2048], or [rows, 1024] with the GLU epilogue), the conv
// output [rows, 1024] and, with the front end, S1 and S2 [windows, H2, 32,
// 256] (each later holds the [windows, H3, 16, 256] stage). Returns the
// bytes used from `base`.
uint64_t place_arena(pk_encoder* e, uint8_t* base) {
  const uint64_t R = e->rows;
  const uint64_t stage = e->front ? (uint64_t)e->batch * e->front_height * halve(kBins, 2) * kSubC : 0;
  const uint64_t elems[11] = {R * kC,     R * kC, R * kC, R * kC, R * kHidden, R * 3 * kC, R * kC,
                              R * (e->fused_glu ? kC : 2 * kC), R * kC, stage, stage};
  void** slots[11] = {&e->a, &e->b, &e->c, &e->d, &e->h, &e->qkv, &e->ctxt, &e->pw, &e->cout, &e->s1, &e->s2};
  uint64_t at = 0;
  for (int i = 0; i < 11; ++i) {
    if (base) *slots[i] = elems[i] ? static_cast<void*>(base + at) : nullptr;
    at += (elems[i] * e->elem + 255u) / 256u * 256u;
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
  e->precision = d->precision;
  e->elem = d->precision == PK_PRECISION_F32 ? 4u : 2u;
  // The GLU epilogue and the fused row norm are f16 kernels.
  e->fused_glu = (d->flags & PK_ENCODER_SEPARATE_GLU) == 0 && d->precision == PK_PRECISION_F16;
  e->fused_norms = (d->flags & PK_ENCODER_FUSED_NORMS) != 0;
  e->chained_norms = (d->flags & (PK_ENCODER_FUSED_NORMS | PK_ENCODER_UNCHAINED_NORMS)) == 0;
  e->prefix_same_plan = (d->flags & PK_ENCODER_PREFIX_SAME_PLAN) != 0;
  e->valid_lengths = d->valid_lengths;
  e->input = d->input;
  e->output = d->output;
  e->front = d->subsampling != nullptr;
  e->feature_frames = e->front ? d->feature_frames : 0;
  e->front_height = e->front ? halve(d->feature_frames, 2) : 0;
  e->feature_lengths = e->front ? d->feature_lengths : nullptr;
  e->projected_channels = d->projected_channels;
  e->projected_output = d->projected_channels ? d->projected_output : nullptr;
}

bool overlap(const void* p, uint64_t pn, const void* q, uint64_t qn) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p), b = reinterpret_cast<uintptr_t>(q);
  return a < b + qn && b < a + pn;
}

int validate_encoder_desc(const pk_encoder_desc* d) {
  if (!d) return fail(PK_INVALID_ARGUMENT, "encoder descriptor is null");
  if (d->struct_size != sizeof(pk_encoder_desc))
    return fail(PK_INVALID_ARGUMENT, "pk_encoder_desc.struct_size mismatch");
  const char* label = d->label ? d->label : "encoder";
  if (d->flags & ~(PK_ENCODER_FUSED_GLU | PK_ENCODER_SEPARATE_GLU | PK_ENCODER_FUSED_NORMS |
                   PK_ENCODER_UNCHAINED_NORMS | PK_ENCODER_PREFIX_SAME_PLAN))
    return fail(PK_INVALID_ARGUMENT, "%s has unknown flags 0x%x", label, d->flags);
  if ((d->flags & PK_ENCODER_FUSED_GLU) && (d->flags & PK_ENCODER_SEPARATE_GLU))
    return fail(PK_INVALID_ARGUMENT, "%s: PK_ENCODER_FUSED_GLU and PK_ENCODER_SEPARATE_GLU exclude each other", label);
  if (d->precision != PK_PRECISION_F16 && d->precision != PK_PRECISION_F32)
    return fail(PK_INVALID_ARGUMENT, "%s has an unsupported precision %d", label, d->precision);
  if (d->precision == PK_PRECISION_F32 &&
      (d->flags & (PK_ENCODER_FUSED_GLU | PK_ENCODER_FUSED_NORMS)))
    return fail(PK_INVALID_ARGUMENT, "%s: the GLU epilogue and the fused LayerNorms need f16", label);
  const uint64_t elem = d->precision == PK_PRECISION_F32 ? 4u : 2u;
  if (d->batch_size == 0 || d->frames == 0 || d->layers == 0 || d->layers > kMaxLayers)
    return fail(PK_RANGE_ERROR, "Unsupported encoder shape for %s: %u windows x %u frames x %u layers", label,
                d->batch_size, d->frames, d->layers);
  if (!d->layer || !d->valid_lengths || !d->input || !d->output)
    return fail(PK_INVALID_ARGUMENT, "%s needs layer weights, valid lengths, input and output", label);
  if (!aligned(d->input, 16) || !aligned(d->output, 16))
    return fail(PK_INVALID_ARGUMENT, "%s input and output must be 16-byte aligned", label);
  uint64_t in_bytes = (uint64_t)d->batch_size * d->frames * kC * elem;
  if (d->subsampling) {
    if (d->feature_frames == 0 || halve(d->feature_frames, 3) != d->frames)
      return fail(PK_RANGE_ERROR, "%s: %u encoder frames do not follow from %u feature frames (expected %u)", label,
                  d->frames, d->feature_frames, halve(d->feature_frames, 3));
    if (!d->feature_lengths || !aligned(d->feature_lengths, 4))
      return fail(PK_INVALID_ARGUMENT, "%s: the front end needs per-window feature lengths", label);
    in_bytes = (uint64_t)d->batch_size * kBins * d->feature_frames * 4u;
  }
  const uint64_t out_bytes = (uint64_t)d->batch_size * d->frames * kC * elem;
  if (overlap(d->input, in_bytes, d->output, out_bytes))
    return fail(PK_INVALID_ARGUMENT, "%s output must not overlap its input", label);
  if (d->projected_channels) {
    const uint64_t proj_bytes = (uint64_t)d->batch_size * d->frames * d->projected_channels * elem;
    if (!d->projected_output || !aligned(d->projected_output, 16))
      return fail(PK_INVALID_ARGUMENT, "%s: the projector needs a 16-byte aligned projected output", label);
    if (overlap(d->projected_output, proj_bytes, d->output, out_bytes) ||
        overlap(d->projected_output, proj_bytes, d->input, in_bytes))
      return fail(PK_INVALID_ARGUMENT, "%s projected output must not overlap the input or output", label);
  }
  return PK_OK;
}

// Builds (or, with `validate_only`, checks) every op of the graph.
int build_all(pk_encoder* e, const pk_encoder_desc* d, hipStream_t stream, bool validate_only) {
  if (e->front)
    if (int s = build_front(e, *d->subsampling, stream, e->front_ops, validate_only)) return s;
  e->ops.resize(e->layers);
  for (uint32_t li = 0; li < e->layers; ++li)
    if (int s = build_layer(e, d->layer[li], li + 1 < e->layers ? &d->layer[li + 1] : nullptr, li, stream, e->ops[li],
                            validate_only))
      return s;
  if (e->projected_channels)
    if (int s = build_projector(e, d, stream, &e->projector, validate_only)) return s;
  if (validate_only || e->prefix_same_plan || e->batch == 1) return PK_OK;
  // Every active batch below the capacity runs the GEMM plans of a graph
  // built for that many windows.
  auto prepare = [&](pk_gemm_op* op, uint32_t rows_per_window) -> int {
    if (!op) return PK_OK;
    std::vector<uint32_t> rows;
    for (uint32_t a = 1; a < e->batch; ++a) rows.push_back(a * rows_per_window);
    const uint64_t before = gemm_weight_bytes(op);
    const int s = pk_gemm_prepare_rows(op, rows.data(), (uint32_t)rows.size());
    e->weight_bytes += gemm_weight_bytes(op) - before;
    return s;
  };
  int s = PK_OK;
  if (e->front) {
    const FrontOps& f = e->front_ops;
    if ((s = prepare(f.pointwise3, e->front_height * halve(kBins, 2))) ||
        (s = prepare(f.pointwise6, e->frames * halve(kBins, 3))) || (s = prepare(f.linear, e->frames)))
      return s;
  }
  for (LayerOps& l : e->ops)
    for (pk_gemm_op* op : {l.ff1a, l.ff1b, l.qkv, l.o, l.pw1, l.pw2, l.ff2a, l.ff2b})
      if ((s = prepare(op, e->frames))) return s;
  return prepare(e->projector, e->frames);
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
  const uint64_t total = arena_bytes(e);
  hipError_t err = hipMalloc(&e->arena, total);
  if (err != hipSuccess) {
    delete e;
    return fail(PK_ALLOCATION_FAILURE, "cannot allocate the %llu-byte encoder arena: %s", (unsigned long long)total,
                hipGetErrorString(err));
  }
  e->arena_bytes = place_arena(e, static_cast<uint8_t*>(e->arena));
  if (int s = build_all(e, d, stream_or_default(ctx, stream), false)) {
    const std::string message = g_error;
    release_encoder(e);
    delete e;
    return fail(s, "%s", message.c_str());
  }
  *out = e;
  return ok();
}

int pk_encoder_validate(const pk_encoder_desc* d) {
  if (int s = validate_encoder_desc(d)) return s;
  // Check every op's descriptor over an arena placed at a nominal,
  // suitably aligned address; nothing is dereferenced or created.
  pk_encoder e;
  describe(&e, d);
  place_arena(&e, reinterpret_cast<uint8_t*>(uintptr_t(1) << 40));
  if (int s = build_all(&e, d, nullptr, true)) return s;
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
  if (launches) *launches = launch_count(e);
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

// pk_tdt_abi.cpp - C ABI of the greedy TDT decoder: the create and
// createDispatch checks and the encode launch of
// src/webgpu/kernels/tdt-decoder.ts (:39-547).
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "pk_abi_internal.h"
#include "pk_internal.h"
#include "pk_tdt.h"

using namespace pk_abi;

struct pk_tdt_op {
  pk_abi::CtxRef ctx;
  std::string label;
  uint32_t batch = 0;
  pk::TdtArgs args{};
  bool f32 = false;     // the f32 profile (one workgroup per window)
  pk::TdtTeam team{};   // members == 0: one workgroup per window
  uint32_t* team_memory = nullptr;
  bool destroyed = false;
};

namespace {

constexpr uint64_t H = PK_TDT_HIDDEN;

// requireTensor (tdt-decoder.ts:458-478): the decoder tensor's size.
int tensor(const void* p, uint64_t bytes, uint64_t need, const char* layout, const char* shape) {
  if (!p || bytes != need || !aligned(p, 16))
    return fail(PK_INVALID_ARGUMENT, "Unexpected decoder tensor %s [%s]", layout, shape);
  return PK_OK;
}

// requireSliceBytes (tdt-decoder.ts:549-553).
int slice(const void* p, uint64_t bytes, uint64_t need, const char* name) {
  if (!p || bytes < need) return fail(PK_RANGE_ERROR, "%s is too small for TDT decoding", name);
  if (!aligned(p, 4)) return fail(PK_RANGE_ERROR, "%s is not word aligned", name);
  return PK_OK;
}

int validate(const pk_tdt_desc* d) {
  if (!d) return fail(PK_INVALID_ARGUMENT, "TDT decoder descriptor is null");
  if (d->struct_size != sizeof(pk_tdt_desc)) return fail(PK_INVALID_ARGUMENT, "pk_tdt_desc.struct_size mismatch");
  // the profile's weight and encoder-row element (tdt-decoder.ts:196-218,
  // requireDecoderWeights :378-405)
  if (d->precision != PK_PRECISION_F16 && d->precision != PK_PRECISION_F32)
    return fail(PK_INVALID_ARGUMENT, "TDT decoder precision must be f16 or f32 (precision %d)", d->precision);
  const uint64_t e = d->precision == PK_PRECISION_F32 ? 4 : 2;
  // validateDescriptor (:507-547)
  if (d->batch_size == 0) return fail(PK_RANGE_ERROR, "Invalid TDT decoder batchSize");
  if (d->frames == 0) return fail(PK_RANGE_ERROR, "Invalid TDT decoder frames");
  if (d->max_tokens == 0) return fail(PK_RANGE_ERROR, "Invalid TDT decoder maxTokens");
  const uint64_t B = d->batch_size;
  int s;
  if ((s = slice(d->encoder_projected, d->encoder_projected_bytes, B * d->frames * H * e, "encoderProjected")) ||
      (s = slice(d->encoded_lengths, d->encoded_lengths_bytes, B * 4, "encodedLengths")) ||
      (s = slice(d->decode_starts, d->decode_starts_bytes, B * 4, "decodeStarts")) ||
      (s = slice(d->decode_ends, d->decode_ends_bytes, B * 4, "decodeEnds")) ||
      (s = slice(d->flush_finals, d->flush_finals_bytes, B * 4, "flushFinals")) ||
      (s = slice(d->state, d->state_bytes, B * 4 * H * 4, "state")) ||
      (s = slice(d->predictor_scratch, d->predictor_scratch_bytes, B * 5 * H * 4, "predictorScratch")) ||
      (s = slice(d->tokens, d->tokens_bytes, B * d->max_tokens * 4, "tokens")) ||
      (s = slice(d->token_frames, d->token_frames_bytes, B * d->max_tokens * 4, "tokenFrames")) ||
      (s = slice(d->token_durations, d->token_durations_bytes, B * d->max_tokens * 4, "tokenDurations")) ||
      (s = slice(d->metadata, d->metadata_bytes, B * 2 * 4, "metadata")))
    return s;
  // requireDecoderWeights (:378-456)
  const pk_tdt_weights& w = d->weights;
  if ((s = tensor(w.embedding, w.embedding_bytes, PK_TDT_TOKEN_OUTPUTS * H * e, "token-by-channel-row-major",
                  "1025,640")) ||
      (s = tensor(w.lstm_weight[0], w.lstm_weight_bytes[0], 2 * H * 4 * H * e,
                  "input-hidden-k-by-ifgo-row-major-vec4", "1280,2560")) ||
      (s = tensor(w.lstm_weight[1], w.lstm_weight_bytes[1], 2 * H * 4 * H * e,
                  "input-hidden-k-by-ifgo-row-major-vec4", "1280,2560")) ||
      (s = tensor(w.lstm_bias[0], w.lstm_bias_bytes[0], 4 * H * 4, "ifgo-gates", "2560")) ||
      (s = tensor(w.lstm_bias[1], w.lstm_bias_bytes[1], 4 * H * 4, "ifgo-gates", "2560")) ||
      (s = tensor(w.projector_weight, w.projector_weight_bytes, H * H * e, "k-by-output-row-major-vec4",
                  "640,640")) ||
      (s = tensor(w.projector_bias, w.projector_bias_bytes, H * 4, "output-channel", "640")) ||
      (s = tensor(w.head_weight, w.head_weight_bytes, H * PK_TDT_HEAD_OUTPUTS * e, "k-by-output-row-major-vec4",
                  "640,1032")) ||
      (s = tensor(w.head_bias, w.head_bias_bytes, PK_TDT_HEAD_OUTPUTS * 4, "output-channel-padded-vec4", "1032")))
    return s;
  if (!aligned(d->encoder_projected, 16) || !aligned(d->state, 16) || !aligned(d->predictor_scratch, 16))
    return fail(PK_INVALID_ARGUMENT, "%s bindings must be 16-byte aligned", d->label ? d->label : "tdt-decoder");
  return PK_OK;
}

// Team size of a batch: the largest supported size whose workgroups can all
// be resident at once (0: one workgroup per window, always for the f32
// profile, whose kernel has no team form).
uint32_t choose_members(int device, uint32_t batch, bool f32) {
  if (f32) return 0;
  const uint32_t capacity = pk::tdt_team_capacity(device);
  for (uint32_t m : {16u, 8u})
    if ((uint64_t)batch * m <= capacity) return m;
  return 0;
}

// Frees the team buffers once no launch can still use them (hipFree alone
// would not order the free after work enqueued on another stream).
void free_team(pk_tdt_op* op) {
  if (op->team_memory) {
    (void)hipSetDevice(op->ctx->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(op->team_memory);
  }
  op->team_memory = nullptr;
  op->team = pk::TdtTeam{};
}

int set_team(pk_tdt_op* op, uint32_t members) {
  free_team(op);
  if (members == 0) return PK_OK;
  const uint64_t sync_words = 2ull * op->batch * pk::kTdtSyncStride;
  const uint64_t words = sync_words + (uint64_t)op->batch * 2 * members * 4;
  PK_HIP(hipSetDevice(op->ctx->device), "hipSetDevice");
  const hipError_t e = hipMalloc(reinterpret_cast<void**>(&op->team_memory), words * 4);
  if (e != hipSuccess)
    return fail(PK_ALLOCATION_FAILURE, "%s: cannot allocate the decoder's team buffers: %s", op->label.c_str(),
                hipGetErrorString(e));
  op->team.members = members;
  op->team.sync = op->team_memory;
  op->team.partials = op->team_memory + sync_words;
  op->team.capacity = op->batch;
  op->team.spin_limit = 1u << 24;
  return PK_OK;
}

// Kernel arguments of a validated descriptor.
pk::TdtArgs args_of(const pk_tdt_desc* d) {
  pk::TdtArgs a{};
  const pk_tdt_weights& w = d->weights;
  a.embedding = w.embedding;
  a.lstm[0] = w.lstm_weight[0];
  a.lstm[1] = w.lstm_weight[1];
  a.lstm_bias[0] = w.lstm_bias[0];
  a.lstm_bias[1] = w.lstm_bias[1];
  a.projector = w.projector_weight;
  a.projector_bias = w.projector_bias;
  a.head = w.head_weight;
  a.head_bias = w.head_bias;
  a.encoder = d->encoder_projected;
  a.lengths = d->encoded_lengths;
  a.starts = d->decode_starts;
  a.ends = d->decode_ends;
  a.flush = d->flush_finals;
  a.state = d->state;
  a.scratch = d->predictor_scratch;
  a.tokens = d->tokens;
  a.token_frames = d->token_frames;
  a.token_durations = d->token_durations;
  a.counts = d->metadata;
  a.status = d->metadata + d->batch_size;
  a.frames = d->frames;
  a.max_tokens = d->max_tokens;
  return a;
}

// Team buffers of pk_tdt_decode_static: the barrier counters and abort
// flags of up to kStaticWindows windows (two 256-byte lines each), then the
// argmax partials of teams of up to 16 members (two buffers of four words
// per member). One copy per GPU, held until the process ends; the launch
// clears the counters and flags with a kernel, the partials are written
// before they are read.
constexpr uint32_t kStaticWindows = PK_TDT_STATIC_MAX_WINDOWS;
constexpr uint32_t kStaticSyncWords = 2 * kStaticWindows * pk::kTdtSyncStride;
constexpr uint32_t kStaticPartialWords = kStaticWindows * 2 * 16 * 4;

}  // namespace

static __device__ __align__(256) uint32_t scratch[kStaticSyncWords + kStaticPartialWords];

namespace {

// The device address of `scratch` on each GPU, looked up once per device
// with that device current (the host symbol is not a device address).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
uint32_t* g_scratch[kMaxDevices] = {};

int scratch_address(int device, uint32_t** out) {
  if (device < 0 || device >= kMaxDevices)
    return fail(PK_INVALID_ARGUMENT, "device %d is outside the static decoder buffers' table", device);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[device]) {
    void* p = nullptr;
    PK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    g_scratch[device] = static_cast<uint32_t*>(p);
  }
  *out = g_scratch[device];
  return PK_OK;
}

}  // namespace

extern "C" {

int pk_tdt_plan_execution(uint32_t batch_size, pk_tdt_execution_plan* plan) {
  if (!plan) return fail(PK_INVALID_ARGUMENT, "plan output is null");
  if (batch_size == 0) return fail(PK_RANGE_ERROR, "TDT decoder batchSize must be a positive integer");
  plan->workgroup_count = batch_size;
  plan->block_threads = pk::kTdtThreads;
  plan->predictor_scratch_bytes = (uint64_t)batch_size * 5 * H * 4;
  return ok();
}

int pk_tdt_validate(const pk_tdt_desc* d) { return validate(d); }

int pk_tdt_create(pk_context* ctx, const pk_tdt_desc* d, pk_tdt_op** out) {
  if (int s = check_ctx(ctx)) return s;
  if (!out) return fail(PK_INVALID_ARGUMENT, "output pointer is null");
  *out = nullptr;
  if (int s = validate(d)) return s;
  auto* op = new pk_tdt_op();
  op->ctx = ctx;
  op->label = d->label ? d->label : "parakeet-persistent-tdt-decode";
  op->batch = d->batch_size;
  op->args = args_of(d);
  op->f32 = d->precision == PK_PRECISION_F32;
  if (int st = set_team(op, choose_members(ctx->device, op->batch, op->f32))) {
    delete op;
    return st;
  }
  *out = op;
  return ok();
}

int pk_tdt_set_team_size(pk_tdt_op* op, uint32_t members) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "TDT decoder op is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  if (members == 0) members = choose_members(op->ctx->device, op->batch, op->f32);
  else if (members == 1) members = 0;
  else if (!pk::tdt_team_members_supported(members))
    return fail(PK_RANGE_ERROR, "%s team size must be 0, 1, 8 or 16", op->label.c_str());
  else if (op->f32)
    return fail(PK_RANGE_ERROR, "%s: team decoding is built for the f16 profile (f32 team size 1)",
                op->label.c_str());
  else if ((uint64_t)op->batch * members > pk::tdt_team_capacity(op->ctx->device))
    return fail(PK_RANGE_ERROR, "%s: %u windows x %u workgroups cannot be resident together", op->label.c_str(),
                op->batch, members);
  PK_HIP(hipSetDevice(op->ctx->device), "hipSetDevice");
  return set_team(op, members);
}

int pk_tdt_team_size(const pk_tdt_op* op, uint32_t* members) {
  if (!op || !members) return fail(PK_INVALID_ARGUMENT, "TDT decoder op or output is null");
  *members = op->team.members ? op->team.members : 1u;
  return ok();
}

int pk_tdt_enqueue(pk_tdt_op* op, uint32_t active_batch, void* stream) {
  return pk_tdt_enqueue_timed(op, active_batch, stream, nullptr, nullptr);
}

int pk_tdt_enqueue_timed(pk_tdt_op* op, uint32_t active_batch, void* stream, void* start_event, void* end_event) {
  if (!op) return fail(PK_INVALID_ARGUMENT, "TDT decoder op is null");
  if (op->destroyed) return fail(PK_DESTROYED, "%s was destroyed", op->label.c_str());
  const uint32_t batch = active_batch ? active_batch : op->batch;
  // TdtDecoderDispatch.encode (:84-130)
  if (batch > op->batch)
    return fail(PK_RANGE_ERROR, "%s active batch must be in [1, %u]", op->label.c_str(), op->batch);
  PK_HIP(hipSetDevice(op->ctx->device), "hipSetDevice");
  const hipStream_t s = stream_or_default(op->ctx, stream);
  // The decode is data dependent and its team buffers can be replaced by
  // pk_tdt_set_team_size, so it is never recorded into a graph.
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  PK_HIP(hipStreamIsCapturing(s, &capture), "hipStreamIsCapturing");
  if (capture != hipStreamCaptureStatusNone)
    return fail(PK_INVALID_ARGUMENT, "%s cannot be enqueued on a capturing stream", op->label.c_str());
  if (op->team.members) {
    // A refused team launch is an error: the op keeps its team size, and a
    // caller that wants one workgroup per window sets team size 1.
    const hipError_t e = pk::launch_tdt_team(op->args, op->team, batch, s, static_cast<hipEvent_t>(start_event),
                                             static_cast<hipEvent_t>(end_event));
    if (e != hipSuccess)
      return fail(PK_DEVICE_ERROR, "%s: team launch (%u x %u workgroups) failed: %s", op->label.c_str(), batch,
                  op->team.members, hipGetErrorString(e));
    return ok();
  }
  PK_HIP(pk::launch_tdt_decode(op->args, batch, op->f32, s, static_cast<hipEvent_t>(start_event),
                               static_cast<hipEvent_t>(end_event)),
         "TDT decoder launch");
  return ok();
}

int pk_tdt_destroy(pk_tdt_op* op) {
  if (!op || op->destroyed) return ok();
  op->destroyed = true;
  free_team(op);
  return ok();
}

int pk_tdt_release(pk_tdt_op* op) {
  if (!op) return ok();
  pk_tdt_destroy(op);
  delete op;
  return ok();
}

int pk_tdt_decode_static(pk_context* ctx, const pk_tdt_desc* d, uint32_t members, void* stream) {
  if (int s = check_ctx(ctx)) return s;
  if (int s = validate(d)) return s;
  const char* label = d->label ? d->label : "parakeet-persistent-tdt-decode";
  const uint32_t batch = d->batch_size;
  if (batch > kStaticWindows)
    return fail(PK_RANGE_ERROR, "%s: %u windows exceed the %u of the static decoder buffers", label, batch,
                kStaticWindows);
  const bool f32 = d->precision == PK_PRECISION_F32;
  if (members == 0) members = choose_members(ctx->device, batch, f32);
  else if (members == 1) members = 0;
  else if (!pk::tdt_team_members_supported(members))
    return fail(PK_RANGE_ERROR, "%s team size must be 0, 1, 8 or 16", label);
  else if (f32)
    return fail(PK_RANGE_ERROR, "%s: team decoding is built for the f16 profile (f32 team size 1)", label);
  else if ((uint64_t)batch * members > pk::tdt_team_capacity(ctx->device))
    return fail(PK_RANGE_ERROR, "%s: %u windows x %u workgroups cannot be resident together", label, batch, members);
  PK_HIP(hipSetDevice(ctx->device), "hipSetDevice");
  const hipStream_t st = stream_or_default(ctx, stream);
  const pk::TdtArgs args = args_of(d);
  if (members == 0) {
    PK_HIP(pk::launch_tdt_decode(args, batch, f32, st), "TDT decoder launch");
    return ok();
  }
  uint32_t* buffers = nullptr;
  if (int s = scratch_address(ctx->device, &buffers)) return s;
  pk::TdtTeam team{};
  team.members = members;
  team.sync = buffers;
  team.partials = buffers + kStaticSyncWords;
  team.capacity = batch;
  team.spin_limit = 1u << 24;
  const hipError_t e = pk::launch_tdt_team(args, team, batch, st);
  if (e != hipSuccess)
    return fail(PK_DEVICE_ERROR, "%s: team launch (%u x %u workgroups) failed: %s", label, batch, members,
                hipGetErrorString(e));
  return ok();
}

}  // extern "C"

/*
 * pk_tdt.h - greedy TDT decoding on gfx950: the two-layer LSTM predictor,
 * the joint network over the encoder projector's output and the
 * token-and-duration argmax, with the whole autoregressive loop inside one
 * launch. Same library, contexts, streams, events and status codes as
 * pk_palette.h.
 *
 * Reference interfaces replaced (src/webgpu/kernels/tdt-decoder.ts):
 *   pk_tdt_plan_execution      planTdtDecoderExecution (:39-52)
 *   pk_tdt_validate / create   PersistentTdtDecoderKernel.create (:164-292)
 *                              with requireDecoderWeights / requireTensor
 *                              (:378-478) and createDispatch
 *                              (:294-366) with validateDescriptor (:507-547)
 *   pk_tdt_enqueue(_timed)     TdtDecoderDispatch.encode (:84-130): the
 *                              active batch selects a prefix of the windows
 *   pk_tdt_destroy             TdtDecoderDispatch.destroy (:132-136)
 * Outputs and working slices are the reference's: tokens, token frames and
 * durations [batch, max_tokens]; metadata [2 * batch] (counts, then status
 * flags, PK_TDT_OVERFLOW when a window had more tokens than max_tokens);
 * state [batch, 4, 640] (committed h0, c0, h1, c1) and predictor scratch
 * [batch, 5, 640] (candidates and the projection), both f32. Both
 * execution profiles (tdt-decoder.ts:196-218): PK_PRECISION_F16 takes f16
 * weights and encoder rows with f16 chains, PK_PRECISION_F32 f32 weights and
 * encoder rows with f32 chains; biases are f32 in both.
 */
#ifndef PK_TDT_H
#define PK_TDT_H

#include "pk_palette.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PK_TDT_HIDDEN 640
#define PK_TDT_TOKEN_OUTPUTS 1025   /* 1024 tokens + blank */
#define PK_TDT_BLANK_TOKEN 1024
#define PK_TDT_HEAD_OUTPUTS 1032    /* tokens, blank, 5 durations, 2 padding */
#define PK_TDT_OVERFLOW 1u
#define PK_TDT_SYNC_TIMEOUT 2u      /* a team barrier gave up waiting (no reference counterpart) */

typedef struct pk_tdt_op pk_tdt_op;

/* The decoder package tensors (model/convert.py:1608-1702), device
   pointers: */
typedef struct pk_tdt_weights {
  /* weights: f16 in the f16 profile, f32 in the f32 profile */
  const void *embedding;         /* [1025, 640] token-by-channel-row-major */
  uint64_t embedding_bytes;
  const void *lstm_weight[2];    /* [1280, 2560] input-hidden-k-by-ifgo-row-major-vec4 */
  uint64_t lstm_weight_bytes[2];
  const float *lstm_bias[2];     /* f32 [2560] ifgo-gates (input + recurrent bias) */
  uint64_t lstm_bias_bytes[2];
  const void *projector_weight;  /* [640, 640] k-by-output-row-major-vec4 */
  uint64_t projector_weight_bytes;
  const float *projector_bias;   /* f32 [640] output-channel */
  uint64_t projector_bias_bytes;
  const void *head_weight;       /* [640, 1032] k-by-output-row-major-vec4 */
  uint64_t head_weight_bytes;
  const float *head_bias;        /* f32 [1032] output-channel-padded-vec4 */
  uint64_t head_bias_bytes;
} pk_tdt_weights;

typedef struct pk_tdt_desc {
  uint32_t struct_size;          /* sizeof(pk_tdt_desc) */
  const char *label;
  int32_t precision;             /* PK_PRECISION_F16 or PK_PRECISION_F32 */
  uint32_t batch_size;
  uint32_t frames;
  uint32_t max_tokens;
  pk_tdt_weights weights;
  const void *encoder_projected; /* [batch, frames, 640], the profile's element */
  uint64_t encoder_projected_bytes;
  const uint32_t *encoded_lengths; /* [batch] */
  uint64_t encoded_lengths_bytes;
  const uint32_t *decode_starts; /* [batch]: first frame decoded */
  uint64_t decode_starts_bytes;
  const uint32_t *decode_ends;   /* [batch]: exclusive last frame */
  uint64_t decode_ends_bytes;
  const uint32_t *flush_finals;  /* [batch]: nonzero runs the end-of-stream flush */
  uint64_t flush_finals_bytes;
  float *state;                  /* [batch, 4, 640] */
  uint64_t state_bytes;
  float *predictor_scratch;      /* [batch, 5, 640] */
  uint64_t predictor_scratch_bytes;
  uint32_t *tokens;              /* [batch, max_tokens] */
  uint64_t tokens_bytes;
  uint32_t *token_frames;        /* [batch, max_tokens] */
  uint64_t token_frames_bytes;
  uint32_t *token_durations;     /* [batch, max_tokens] */
  uint64_t token_durations_bytes;
  uint32_t *metadata;            /* [2 * batch]: counts, then status */
  uint64_t metadata_bytes;
} pk_tdt_desc;

typedef struct pk_tdt_execution_plan {
  uint32_t workgroup_count;      /* one workgroup per window; an op in team mode
                                    launches pk_tdt_team_size() per window */
  uint32_t block_threads;
  uint64_t predictor_scratch_bytes;
} pk_tdt_execution_plan;

int pk_tdt_plan_execution(uint32_t batch_size, pk_tdt_execution_plan *plan);
int pk_tdt_validate(const pk_tdt_desc *desc);
int pk_tdt_create(pk_context *ctx, const pk_tdt_desc *desc, pk_tdt_op **out);
int pk_tdt_enqueue(pk_tdt_op *op, uint32_t active_batch, void *stream);
int pk_tdt_enqueue_timed(pk_tdt_op *op, uint32_t active_batch, void *stream, void *start_event,
                         void *end_event);
/* No reference counterpart: how many workgroups decode one window. 0
   chooses (16 or 8 when every workgroup of the batch can be resident
   together, else 1), 1 runs one workgroup per window, 8 and 16 split
   every weight matrix over a team that meets at barriers in global memory
   (bounded waits: a barrier that never completes sets the window's
   PK_TDT_SYNC_TIMEOUT status). Results are bit-identical for every size.
   Teams are built for the f16 profile: an f32 op always runs one
   workgroup per window (0 chooses 1; 8 and 16 return PK_RANGE_ERROR).
   A team launch is an ordinary launch whose grid fits the workgroups an
   idle device holds at once: kernels running on other streams at the same
   time can keep members from being resident, and a barrier that then
   waits 2^24 polls gives up, so a team decode that overlaps other work can
   end with PK_TDT_SYNC_TIMEOUT in its windows' status words. Callers check
   the status words (overflow and sync timeout are separate bits) and
   decode such windows again, or use team size 1, which never waits.
   The create call chooses automatically; the setter synchronizes the
   device. A team launch that the runtime refuses returns PK_DEVICE_ERROR
   and leaves the team size as it was. */
int pk_tdt_set_team_size(pk_tdt_op *op, uint32_t members);
int pk_tdt_team_size(const pk_tdt_op *op, uint32_t *members);
/* Idempotent; frees the team buffers (after the device has drained), and
   enqueue after destroy returns PK_DESTROYED. Enqueue on a stream that is
   capturing a graph returns PK_INVALID_ARGUMENT. */
int pk_tdt_destroy(pk_tdt_op *op);
int pk_tdt_release(pk_tdt_op *op);

/* No counterpart in the reference: the whole decode of `desc` as one call
   that allocates nothing, for callers that cannot allocate device memory
   (code under HIP graph capture, tight serving loops, harnesses that forbid
   hipMalloc). It validates like pk_tdt_create, then launches like
   pk_tdt_enqueue of every window with team size `members` (0 chooses, 1,
   8 or 16; bit-identical results for each), taking the team's barrier
   counters and argmax partials from a static device array of the library
   (64 KB per GPU, held until the process ends) instead of buffers of an
   op. At most PK_TDT_STATIC_MAX_WINDOWS windows (PK_RANGE_ERROR beyond).
   Every call on one GPU shares that array: calls whose decodes overlap on
   the same GPU (other streams, other threads) race and must be ordered by
   the caller. The call may be recorded into a HIP graph (the counters are
   cleared by a kernel, not a memset); a team replayed beside other work
   can end with PK_TDT_SYNC_TIMEOUT as described at pk_tdt_set_team_size. */
#define PK_TDT_STATIC_MAX_WINDOWS 64u
int pk_tdt_decode_static(pk_context *ctx, const pk_tdt_desc *desc, uint32_t members, void *stream);

#ifdef __cplusplus
}
#endif

#endif

/*
 * pk_napi.c - Node-API (N-API 8) addon over the palette GEMM C ABI
 * (include/pk_palette.h), the fused Conformer convolution tail
 * (include/pk_conv.h), the relative-position attention
 * (include/pk_attention.h), the row LayerNorm (include/pk_layernorm.h), the
 * subsampling convolutions (include/pk_subsampling.h) and the encoder graph
 * (include/pk_encoder.h). It is the thin native layer under the JavaScript
 * host in ../host: every function forwards to one pk_* call, converts device
 * pointers to BigInt, and turns a failing pk_status into a thrown Error
 * (RangeError for PK_RANGE_ERROR, as the reference throws RangeError for
 * those cases, src/webgpu/kernels/gemm.ts:431-438, :982) whose message is
 * pk_last_error() and whose `code` is the status name.
 *
 * Handles (context, op, prepared weight, event, stream) are N-API externals;
 * ops and weights are released by their finalizer if JavaScript never
 * releases them explicitly.
 */
#define NAPI_VERSION 8
#include <node_api.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pk_attention.h"
#include "pk_conv.h"
#include "pk_encoder.h"
#include "pk_layernorm.h"
#include "pk_palette.h"
#include "pk_subsampling.h"
#include "pk_tdt.h"

#define NAPI_CALL(env, call)                                              \
  do {                                                                    \
    if ((call) != napi_ok) {                                              \
      napi_throw_error((env), "PK_NAPI", "N-API call failed: " #call);    \
      return NULL;                                                        \
    }                                                                     \
  } while (0)

static napi_value throw_status(napi_env env, int status) {
  const char *message = pk_last_error();
  if (status == PK_RANGE_ERROR)
    napi_throw_range_error(env, pk_status_name(status), message);
  else
    napi_throw_error(env, pk_status_name(status), message);
  return NULL;
}

#define PK_CALL(env, call)                 \
  do {                                     \
    int pk_s_ = (call);                    \
    if (pk_s_ != PK_OK) return throw_status((env), pk_s_); \
  } while (0)

/* ---- argument helpers ---------------------------------------------------- */

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value *argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok) return 0;
  for (size_t i = argc; i < want; ++i) napi_get_undefined(env, &argv[i]);
  return 1;
}

static int is_nullish(napi_env env, napi_value v) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  return t == napi_undefined || t == napi_null;
}

static void *get_external(napi_env env, napi_value v) {
  void *p = NULL;
  if (is_nullish(env, v)) return NULL;
  if (napi_get_value_external(env, v, &p) != napi_ok) return NULL;
  return p;
}

/* uint64 from a BigInt or a (safe-integer) Number. */
static int get_u64(napi_env env, napi_value v, uint64_t *out) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_bigint) {
    bool lossless = true;
    return napi_get_value_bigint_uint64(env, v, out, &lossless) == napi_ok && lossless;
  }
  if (t == napi_number) {
    double d;
    if (napi_get_value_double(env, v, &d) != napi_ok || d < 0 || d > 9007199254740991.0 || d != (double)(uint64_t)d)
      return 0;
    *out = (uint64_t)d;
    return 1;
  }
  return 0;
}

static int get_u32(napi_env env, napi_value v, uint32_t *out) {
  uint64_t x;
  if (!get_u64(env, v, &x) || x > 0xffffffffull) return 0;
  *out = (uint32_t)x;
  return 1;
}

static int prop(napi_env env, napi_value obj, const char *name, napi_value *out) {
  bool has = false;
  if (napi_has_named_property(env, obj, name, &has) != napi_ok || !has) return 0;
  if (napi_get_named_property(env, obj, name, out) != napi_ok) return 0;
  return !is_nullish(env, *out);
}

static int prop_u64(napi_env env, napi_value obj, const char *name, uint64_t *out) {
  napi_value v;
  return prop(env, obj, name, &v) && get_u64(env, v, out);
}

static int prop_u32(napi_env env, napi_value obj, const char *name, uint32_t *out) {
  napi_value v;
  return prop(env, obj, name, &v) && get_u32(env, v, out);
}

static int prop_i32(napi_env env, napi_value obj, const char *name, int32_t *out) {
  napi_value v;
  return prop(env, obj, name, &v) && napi_get_value_int32(env, v, out) == napi_ok;
}

/* A heap copy of a string property (caller frees), or NULL. */
static char *prop_string(napi_env env, napi_value obj, const char *name) {
  napi_value v;
  size_t len = 0;
  if (!prop(env, obj, name, &v)) return NULL;
  if (napi_get_value_string_utf8(env, v, NULL, 0, &len) != napi_ok) return NULL;
  char *s = (char *)malloc(len + 1);
  if (!s) return NULL;
  napi_get_value_string_utf8(env, v, s, len + 1, &len);
  return s;
}

static napi_value make_u64(napi_env env, uint64_t x) {
  napi_value v;
  napi_create_bigint_uint64(env, x, &v);
  return v;
}

static napi_value make_number(napi_env env, double x) {
  napi_value v;
  napi_create_double(env, x, &v);
  return v;
}

static napi_value undefined(napi_env env) {
  napi_value v;
  napi_get_undefined(env, &v);
  return v;
}

static napi_value bad_argument(napi_env env, const char *what) {
  napi_throw_type_error(env, "PK_INVALID_ARGUMENT", what);
  return NULL;
}

/* ---- context -------------------------------------------------------------- */

static napi_value js_abi_version(napi_env env, napi_callback_info info) {
  (void)info;
  return make_number(env, pk_abi_version());
}

static napi_value js_context_create(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  int32_t device = 0;
  if (!get_args(env, info, 1, argv)) return NULL;
  if (!is_nullish(env, argv[0]) && napi_get_value_int32(env, argv[0], &device) != napi_ok)
    return bad_argument(env, "device index must be a number");
  pk_context *ctx = NULL;
  PK_CALL(env, pk_context_create(device, &ctx));
  napi_value ext;
  NAPI_CALL(env, napi_create_external(env, ctx, NULL, NULL, &ext));
  return ext;
}

static napi_value js_context_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  PK_CALL(env, pk_context_destroy((pk_context *)get_external(env, argv[0])));
  return undefined(env);
}

static napi_value js_device_info(napi_env env, napi_callback_info info) {
  napi_value argv[1], obj, v;
  if (!get_args(env, info, 1, argv)) return NULL;
  pk_device_info di;
  PK_CALL(env, pk_device_query((pk_context *)get_external(env, argv[0]), &di));
  NAPI_CALL(env, napi_create_object(env, &obj));
  napi_create_string_utf8(env, di.name, NAPI_AUTO_LENGTH, &v);
  napi_set_named_property(env, obj, "name", v);
  napi_create_string_utf8(env, di.arch, NAPI_AUTO_LENGTH, &v);
  napi_set_named_property(env, obj, "arch", v);
  napi_set_named_property(env, obj, "computeUnits", make_number(env, di.compute_units));
  napi_set_named_property(env, obj, "wavefrontSize", make_number(env, di.wavefront_size));
  napi_set_named_property(env, obj, "globalMemoryBytes", make_number(env, (double)di.global_memory_bytes));
  napi_set_named_property(env, obj, "ldsBytesPerBlock", make_number(env, di.lds_bytes_per_block));
  napi_set_named_property(env, obj, "clockKhz", make_number(env, di.clock_khz));
  return obj;
}

/* ---- memory --------------------------------------------------------------- */

static napi_value js_alloc(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  uint64_t bytes;
  if (!get_args(env, info, 2, argv)) return NULL;
  if (!get_u64(env, argv[1], &bytes)) return bad_argument(env, "byte count must be a non-negative integer");
  void *p = NULL;
  PK_CALL(env, pk_alloc((pk_context *)get_external(env, argv[0]), bytes, &p));
  return make_u64(env, (uint64_t)(uintptr_t)p);
}

static napi_value js_free(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  uint64_t ptr;
  if (!get_args(env, info, 2, argv)) return NULL;
  if (!get_u64(env, argv[1], &ptr)) return bad_argument(env, "device pointer must be a BigInt");
  PK_CALL(env, pk_free((pk_context *)get_external(env, argv[0]), (void *)(uintptr_t)ptr));
  return undefined(env);
}

/* Host view (TypedArray, DataView or ArrayBuffer) -> data pointer and length. */
static int host_bytes(napi_env env, napi_value v, void **data, size_t *length) {
  bool is;
  if (napi_is_typedarray(env, v, &is) == napi_ok && is) {
    napi_typedarray_type type;
    size_t count, offset;
    napi_value ab;
    if (napi_get_typedarray_info(env, v, &type, &count, data, &ab, &offset) != napi_ok) return 0;
    size_t elem = 1;
    switch (type) {
      case napi_int16_array: case napi_uint16_array: elem = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: elem = 4; break;
      case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: elem = 8; break;
      default: elem = 1;
    }
    *length = count * elem;
    return 1;
  }
  if (napi_is_dataview(env, v, &is) == napi_ok && is) {
    napi_value ab;
    size_t offset;
    return napi_get_dataview_info(env, v, length, data, &ab, &offset) == napi_ok;
  }
  if (napi_is_arraybuffer(env, v, &is) == napi_ok && is)
    return napi_get_arraybuffer_info(env, v, data, length) == napi_ok;
  return 0;
}

/* upload(ctx, devicePtr, byteOffset, hostView, stream?) - complete on return */
static napi_value js_upload(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  uint64_t ptr, offset;
  void *data;
  size_t len;
  if (!get_args(env, info, 5, argv)) return NULL;
  if (!get_u64(env, argv[1], &ptr) || !get_u64(env, argv[2], &offset) || !host_bytes(env, argv[3], &data, &len))
    return bad_argument(env, "upload(ctx, devicePtr, byteOffset, hostView)");
  PK_CALL(env, pk_upload((pk_context *)get_external(env, argv[0]), (void *)(uintptr_t)(ptr + offset), data, len,
                         get_external(env, argv[4])));
  return undefined(env);
}

/* download(ctx, devicePtr, byteOffset, hostView, stream?) - complete on return */
static napi_value js_download(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  uint64_t ptr, offset;
  void *data;
  size_t len;
  if (!get_args(env, info, 5, argv)) return NULL;
  if (!get_u64(env, argv[1], &ptr) || !get_u64(env, argv[2], &offset) || !host_bytes(env, argv[3], &data, &len))
    return bad_argument(env, "download(ctx, devicePtr, byteOffset, hostView)");
  PK_CALL(env, pk_download((pk_context *)get_external(env, argv[0]), data, (const void *)(uintptr_t)(ptr + offset),
                           len, get_external(env, argv[4])));
  return undefined(env);
}

static napi_value js_synchronize(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  PK_CALL(env, pk_stream_synchronize((pk_context *)get_external(env, argv[0]), get_external(env, argv[1])));
  return undefined(env);
}

/* synchronizeAsync(ctx, stream?) -> Promise resolved when the stream drains
   (the GPUQueue.onSubmittedWorkDone of the reference, webgpu-engine.ts:993).
   The wait runs on a libuv worker thread. */
typedef struct {
  napi_async_work work;
  napi_deferred deferred;
  pk_context *ctx;
  void *stream;
  int status;
  char message[512];
} sync_job;

static void sync_execute(napi_env env, void *data) {
  (void)env;
  sync_job *job = (sync_job *)data;
  job->status = pk_stream_synchronize(job->ctx, job->stream);
  if (job->status != PK_OK) snprintf(job->message, sizeof job->message, "%s", pk_last_error());
}

static void sync_complete(napi_env env, napi_status status, void *data) {
  sync_job *job = (sync_job *)data;
  if (status == napi_ok && job->status == PK_OK) {
    napi_resolve_deferred(env, job->deferred, undefined(env));
  } else {
    napi_value msg, code, err;
    napi_create_string_utf8(env, job->status == PK_OK ? "synchronization was cancelled" : job->message,
                            NAPI_AUTO_LENGTH, &msg);
    napi_create_string_utf8(env, pk_status_name(job->status), NAPI_AUTO_LENGTH, &code);
    napi_create_error(env, code, msg, &err);
    napi_reject_deferred(env, job->deferred, err);
  }
  napi_delete_async_work(env, job->work);
  free(job);
}

static napi_value js_synchronize_async(napi_env env, napi_callback_info info) {
  napi_value argv[2], promise, name;
  if (!get_args(env, info, 2, argv)) return NULL;
  sync_job *job = (sync_job *)calloc(1, sizeof *job);
  if (!job) return bad_argument(env, "out of host memory");
  job->ctx = (pk_context *)get_external(env, argv[0]);
  job->stream = get_external(env, argv[1]);
  NAPI_CALL(env, napi_create_promise(env, &job->deferred, &promise));
  napi_create_string_utf8(env, "pk_stream_synchronize", NAPI_AUTO_LENGTH, &name);
  NAPI_CALL(env, napi_create_async_work(env, NULL, name, sync_execute, sync_complete, job, &job->work));
  NAPI_CALL(env, napi_queue_async_work(env, job->work));
  return promise;
}

/* ---- events (timestamps) -------------------------------------------------- */

static napi_value js_event_create(napi_env env, napi_callback_info info) {
  napi_value argv[1], ext;
  if (!get_args(env, info, 1, argv)) return NULL;
  void *ev = NULL;
  PK_CALL(env, pk_event_create((pk_context *)get_external(env, argv[0]), &ev));
  NAPI_CALL(env, napi_create_external(env, ev, NULL, NULL, &ext));
  return ext;
}

static napi_value js_event_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  PK_CALL(env, pk_event_destroy((pk_context *)get_external(env, argv[0]), get_external(env, argv[1])));
  return undefined(env);
}

static napi_value js_event_record(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return NULL;
  PK_CALL(env, pk_event_record((pk_context *)get_external(env, argv[0]), get_external(env, argv[1]),
                               get_external(env, argv[2])));
  return undefined(env);
}

static napi_value js_event_elapsed_ms(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  float ms = 0.0f;
  if (!get_args(env, info, 3, argv)) return NULL;
  PK_CALL(env, pk_event_elapsed_ms((pk_context *)get_external(env, argv[0]), get_external(env, argv[1]),
                                   get_external(env, argv[2]), &ms));
  return make_number(env, ms);
}

/* ---- prepared weights ----------------------------------------------------- */

/* The JavaScript handle holds the weight through a box: the explicit destroy
   releases the owner's reference and empties the box, the finalizer
   releases only a weight still in the box. An op created from the weight
   keeps its own reference, so the weight may outlive the handle. */
typedef struct weight_box {
  pk_prepared_weight *w;
} weight_box;

static void weight_finalize(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  weight_box *box = (weight_box *)data;
  if (box->w) pk_prepared_weight_destroy(box->w);
  free(box);
}

/* preparedWeightCreate(ctx, {label, paletteBits, inner, columns, packed, packedBytes}) */
static napi_value js_prepared_weight_create(napi_env env, napi_callback_info info) {
  napi_value argv[2], ext;
  if (!get_args(env, info, 2, argv)) return NULL;
  pk_weight_desc d;
  memset(&d, 0, sizeof d);
  d.struct_size = sizeof d;
  uint64_t packed = 0;
  if (!prop_i32(env, argv[1], "paletteBits", &d.palette_bits) || !prop_u32(env, argv[1], "inner", &d.inner) ||
      !prop_u32(env, argv[1], "columns", &d.columns) || !prop_u64(env, argv[1], "packed", &packed) ||
      !prop_u64(env, argv[1], "packedBytes", &d.packed_bytes))
    return bad_argument(env, "weight descriptor needs paletteBits, inner, columns, packed, packedBytes");
  char *label = prop_string(env, argv[1], "label");
  d.label = label;
  d.packed = (const uint32_t *)(uintptr_t)packed;
  pk_prepared_weight *w = NULL;
  const int status = pk_prepared_weight_create((pk_context *)get_external(env, argv[0]), &d, NULL, &w);
  free(label);
  if (status != PK_OK) return throw_status(env, status);
  weight_box *box = (weight_box *)malloc(sizeof *box);
  if (!box) {
    pk_prepared_weight_destroy(w);
    napi_throw_error(env, "PK_ALLOCATION_FAILURE", "cannot allocate the weight handle");
    return NULL;
  }
  box->w = w;
  NAPI_CALL(env, napi_create_external(env, box, weight_finalize, NULL, &ext));
  return ext;
}

static napi_value js_prepared_weight_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  weight_box *box = (weight_box *)get_external(env, argv[0]);
  if (box && box->w) {
    pk_prepared_weight *w = box->w;
    box->w = NULL;
    PK_CALL(env, pk_prepared_weight_destroy(w));
  }
  return undefined(env);
}

/* ---- GEMM ----------------------------------------------------------------- */

static void op_finalize(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  pk_gemm_release((pk_gemm_op *)data);
}

/* A JavaScript GEMM descriptor: {label, flags, precision ("f16"|"f32"),
   paletteBits, rows, inner, columns, paletteGroups, paletteGroupColumns,
   a, aBytes, packed, packedBytes, palette, paletteBytes, output,
   outputBytes, bias?, biasBytes?, residual?, residualBytes?,
   residualScale?, activation ("none"|"silu"|"relu"), prepared?}; device
   pointers are BigInt. Returns 0 after throwing; *label is heap-owned. */
static int parse_gemm_desc(napi_env env, napi_value o, pk_gemm_desc *d, char **label) {
  napi_value v;
  memset(d, 0, sizeof *d);
  d->struct_size = sizeof *d;
  *label = NULL;
  uint64_t a = 0, packed = 0, palette = 0, output = 0, bias = 0, residual = 0, norm_gamma = 0, norm_beta = 0;
  char *precision = prop_string(env, o, "precision");
  char *activation = prop_string(env, o, "activation");
  d->precision = !precision || strcmp(precision, "f16") == 0 ? PK_PRECISION_F16
                 : strcmp(precision, "f32") == 0            ? PK_PRECISION_F32
                                                            : -1;
  d->activation = !activation || strcmp(activation, "none") == 0 ? PK_ACTIVATION_NONE
                  : strcmp(activation, "silu") == 0             ? PK_ACTIVATION_SILU
                  : strcmp(activation, "relu") == 0             ? PK_ACTIVATION_RELU
                                                                : -1;
  free(precision);
  free(activation);
  if (!prop_i32(env, o, "paletteBits", &d->palette_bits) || !prop_u32(env, o, "rows", &d->rows) ||
      !prop_u32(env, o, "inner", &d->inner) || !prop_u32(env, o, "columns", &d->columns) ||
      !prop_u32(env, o, "paletteGroups", &d->palette_groups) ||
      !prop_u32(env, o, "paletteGroupColumns", &d->palette_group_columns) || !prop_u64(env, o, "a", &a) ||
      !prop_u64(env, o, "aBytes", &d->a_bytes) || !prop_u64(env, o, "palette", &palette) ||
      !prop_u64(env, o, "paletteBytes", &d->palette_bytes) || !prop_u64(env, o, "output", &output) ||
      !prop_u64(env, o, "outputBytes", &d->output_bytes)) {
    bad_argument(env, "GEMM descriptor is missing a required field");
    return 0;
  }
  prop_u32(env, o, "flags", &d->flags);
  if (prop_u64(env, o, "packed", &packed)) prop_u64(env, o, "packedBytes", &d->packed_bytes);
  if (prop_u64(env, o, "bias", &bias)) prop_u64(env, o, "biasBytes", &d->bias_bytes);
  if (prop_u64(env, o, "residual", &residual)) prop_u64(env, o, "residualBytes", &d->residual_bytes);
  if (prop(env, o, "residualScale", &v)) {
    double scale;
    if (napi_get_value_double(env, v, &scale) != napi_ok) {
      bad_argument(env, "residualScale must be a number");
      return 0;
    }
    d->has_residual_scale = 1;
    d->residual_scale = (float)scale;
  }
  if (prop_u64(env, o, "normGamma", &norm_gamma)) prop_u64(env, o, "normGammaBytes", &d->norm_gamma_bytes);
  if (prop_u64(env, o, "normBeta", &norm_beta)) prop_u64(env, o, "normBetaBytes", &d->norm_beta_bytes);
  if (prop(env, o, "normEpsilon", &v)) {
    double epsilon;
    if (napi_get_value_double(env, v, &epsilon) != napi_ok) {
      bad_argument(env, "normEpsilon must be a number");
      return 0;
    }
    d->norm_epsilon = (float)epsilon;
  }
  if (prop(env, o, "prepared", &v)) {
    const weight_box *box = (const weight_box *)get_external(env, v);
    if (!box || !box->w) {
      napi_throw_error(env, "PK_DESTROYED", "prepared palette weight was destroyed");
      return 0;
    }
    d->prepared = box->w;
  }
  d->a = (const void *)(uintptr_t)a;
  d->packed = (const uint32_t *)(uintptr_t)packed;
  d->palette = (const void *)(uintptr_t)palette;
  d->output = (void *)(uintptr_t)output;
  d->bias = (const float *)(uintptr_t)bias;
  d->norm_gamma = (const float *)(uintptr_t)norm_gamma;
  d->norm_beta = (const float *)(uintptr_t)norm_beta;
  d->residual = (const void *)(uintptr_t)residual;
  *label = prop_string(env, o, "label");
  d->label = *label;
  return 1;
}

/* gemmValidate(desc): the descriptor contract without a device. */
static napi_value js_gemm_validate(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  pk_gemm_desc d;
  char *label;
  if (!parse_gemm_desc(env, argv[0], &d, &label)) return NULL;
  const int status = pk_gemm_validate(&d);
  free(label);
  if (status != PK_OK) return throw_status(env, status);
  return undefined(env);
}

/* gemmCreate(ctx, desc) -> op */
static napi_value js_gemm_create(napi_env env, napi_callback_info info) {
  napi_value argv[2], ext;
  if (!get_args(env, info, 2, argv)) return NULL;
  pk_gemm_desc d;
  char *label;
  if (!parse_gemm_desc(env, argv[1], &d, &label)) return NULL;
  pk_gemm_op *op = NULL;
  const int status = pk_gemm_create((pk_context *)get_external(env, argv[0]), &d, NULL, &op);
  free(label);
  if (status != PK_OK) return throw_status(env, status);
  NAPI_CALL(env, napi_create_external(env, op, op_finalize, NULL, &ext));
  return ext;
}

/* gemmEnqueue(op, activeRows, stream?, startEvent?, endEvent?) */
static napi_value js_gemm_enqueue(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  uint32_t rows = 0;
  if (!get_args(env, info, 5, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &rows))
    return bad_argument(env, "active rows must be a non-negative integer");
  PK_CALL(env, pk_gemm_enqueue_timed((pk_gemm_op *)get_external(env, argv[0]), rows, get_external(env, argv[2]),
                                     get_external(env, argv[3]), get_external(env, argv[4])));
  return undefined(env);
}

static napi_value js_gemm_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  PK_CALL(env, pk_gemm_destroy((pk_gemm_op *)get_external(env, argv[0])));
  return undefined(env);
}

static napi_value js_gemm_plan(napi_env env, napi_callback_info info) {
  napi_value argv[2], obj, grid, v;
  uint32_t rows = 0;
  if (!get_args(env, info, 2, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &rows))
    return bad_argument(env, "active rows must be a non-negative integer");
  pk_gemm_plan_info p;
  PK_CALL(env, pk_gemm_plan((pk_gemm_op *)get_external(env, argv[0]), rows, &p));
  NAPI_CALL(env, napi_create_object(env, &obj));
  NAPI_CALL(env, napi_create_array_with_length(env, 3, &grid));
  for (uint32_t i = 0; i < 3; ++i) napi_set_element(env, grid, i, make_number(env, p.grid[i]));
  napi_set_named_property(env, obj, "workgroups", grid);
  napi_set_named_property(env, obj, "blockThreads", make_number(env, p.block_threads));
  napi_set_named_property(env, obj, "tileRows", make_number(env, p.tile_rows));
  napi_set_named_property(env, obj, "tileColumns", make_number(env, p.tile_columns));
  napi_set_named_property(env, obj, "splitInner", make_number(env, p.split_inner));
  napi_set_named_property(env, obj, "ldsBytes", make_number(env, p.lds_bytes));
  napi_set_named_property(env, obj, "workspaceBytes", make_number(env, (double)p.workspace_bytes));
  napi_set_named_property(env, obj, "flops", make_number(env, (double)p.flops));
  napi_set_named_property(env, obj, "algorithmicBytes", make_number(env, (double)p.algorithmic_bytes));
  napi_create_string_utf8(env, p.kernel, NAPI_AUTO_LENGTH, &v);
  napi_set_named_property(env, obj, "kernel", v);
  napi_get_boolean(env, p.stream_stores != 0, &v);
  napi_set_named_property(env, obj, "streamStores", v);
  return obj;
}

/* ---- Conformer convolution tail ------------------------------------------ */

static void conv_finalize(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  pk_conv_release((pk_conv_op *)data);
}

static int parse_precision(napi_env env, napi_value o, int32_t *precision) {
  char *p = prop_string(env, o, "precision");
  *precision = !p || strcmp(p, "f16") == 0 ? PK_PRECISION_F16 : strcmp(p, "f32") == 0 ? PK_PRECISION_F32 : -1;
  free(p);
  return 1;
}

/* A JavaScript conv descriptor: {label, flags?, precision, batchSize, frames,
   channels?, pointwiseInput, pointwiseInputBytes, depthwiseWeights,
   depthwiseWeightsBytes, batchNormScale, batchNormScaleBytes,
   batchNormShift, batchNormShiftBytes, validLengths, validLengthsBytes,
   output, outputBytes}; device pointers are BigInt. */
static int parse_conv_desc(napi_env env, napi_value o, pk_conv_desc *d, char **label) {
  memset(d, 0, sizeof *d);
  d->struct_size = sizeof *d;
  *label = NULL;
  uint64_t input = 0, weights = 0, scale = 0, shift = 0, valid = 0, output = 0;
  parse_precision(env, o, &d->precision);
  if (!prop_u32(env, o, "batchSize", &d->batch_size) || !prop_u32(env, o, "frames", &d->frames) ||
      !prop_u64(env, o, "pointwiseInput", &input) ||
      !prop_u64(env, o, "pointwiseInputBytes", &d->pointwise_input_bytes) ||
      !prop_u64(env, o, "depthwiseWeights", &weights) ||
      !prop_u64(env, o, "depthwiseWeightsBytes", &d->depthwise_weights_bytes) ||
      !prop_u64(env, o, "batchNormScale", &scale) ||
      !prop_u64(env, o, "batchNormScaleBytes", &d->batch_norm_scale_bytes) ||
      !prop_u64(env, o, "batchNormShift", &shift) ||
      !prop_u64(env, o, "batchNormShiftBytes", &d->batch_norm_shift_bytes) ||
      !prop_u64(env, o, "validLengths", &valid) || !prop_u64(env, o, "validLengthsBytes", &d->valid_lengths_bytes) ||
      !prop_u64(env, o, "output", &output) || !prop_u64(env, o, "outputBytes", &d->output_bytes)) {
    bad_argument(env, "convolution descriptor is missing a required field");
    return 0;
  }
  prop_u32(env, o, "channels", &d->channels);
  prop_u32(env, o, "flags", &d->flags);
  d->pointwise_input = (const void *)(uintptr_t)input;
  d->depthwise_weights = (const void *)(uintptr_t)weights;
  d->batch_norm_scale = (const float *)(uintptr_t)scale;
  d->batch_norm_shift = (const float *)(uintptr_t)shift;
  d->valid_lengths = (const uint32_t *)(uintptr_t)valid;
  d->output = (void *)(uintptr_t)output;
  *label = prop_string(env, o, "label");
  d->label = *label;
  return 1;
}

static napi_value conv_plan_object(napi_env env, const pk_conv_plan_info *p) {
  napi_value obj, grid, v;
  NAPI_CALL(env, napi_create_object(env, &obj));
  NAPI_CALL(env, napi_create_array_with_length(env, 3, &grid));
  for (uint32_t i = 0; i < 3; ++i) napi_set_element(env, grid, i, make_number(env, p->grid[i]));
  napi_set_named_property(env, obj, "rows", make_number(env, p->rows));
  napi_set_named_property(env, obj, "inputByteLength", make_number(env, (double)p->input_bytes));
  napi_set_named_property(env, obj, "outputByteLength", make_number(env, (double)p->output_bytes));
  napi_set_named_property(env, obj, "validLengthsByteLength", make_number(env, (double)p->valid_lengths_bytes));
  napi_set_named_property(env, obj, "depthwiseWeightByteLength", make_number(env, (double)p->depthwise_weight_bytes));
  napi_set_named_property(env, obj, "affineByteLength", make_number(env, (double)p->affine_bytes));
  napi_set_named_property(env, obj, "workgroups", grid);
  napi_set_named_property(env, obj, "blockThreads", make_number(env, p->block_threads));
  napi_set_named_property(env, obj, "workgroupStorageBytes", make_number(env, p->lds_bytes));
  napi_set_named_property(env, obj, "algorithmicBytes", make_number(env, (double)p->algorithmic_bytes));
  napi_create_string_utf8(env, p->kernel, NAPI_AUTO_LENGTH, &v);
  napi_set_named_property(env, obj, "kernel", v);
  return obj;
}

/* convPlanShape(precision, batchSize, frames, channels?) */
static napi_value js_conv_plan_shape(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return NULL;
  char buf[8] = {0};
  size_t n = 0;
  napi_get_value_string_utf8(env, argv[0], buf, sizeof buf, &n);
  const int precision = strcmp(buf, "f32") == 0 ? PK_PRECISION_F32 : strcmp(buf, "f16") == 0 ? PK_PRECISION_F16 : -1;
  uint32_t batch = 0, frames = 0, channels = 0;
  if (!get_u32(env, argv[1], &batch) || !get_u32(env, argv[2], &frames))
    return bad_argument(env, "batchSize and frames must be non-negative integers");
  if (!is_nullish(env, argv[3]) && !get_u32(env, argv[3], &channels))
    return bad_argument(env, "channels must be a non-negative integer");
  pk_conv_plan_info p;
  PK_CALL(env, pk_conv_plan_shape(precision, batch, frames, channels, &p));
  return conv_plan_object(env, &p);
}

/* convValidate(desc) */
static napi_value js_conv_validate(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  pk_conv_desc d;
  char *label;
  if (!parse_conv_desc(env, argv[0], &d, &label)) return NULL;
  const int status = pk_conv_validate(&d);
  free(label);
  if (status != PK_OK) return throw_status(env, status);
  return undefined(env);
}

/* convCreate(ctx, desc) -> op */
static napi_value js_conv_create(napi_env env, napi_callback_info info) {
  napi_value argv[2], ext;
  if (!get_args(env, info, 2, argv)) return NULL;
  pk_conv_desc d;
  char *label;
  if (!parse_conv_desc(env, argv[1], &d, &label)) return NULL;
  pk_conv_op *op = NULL;
  const int status = pk_conv_create((pk_context *)get_external(env, argv[0]), &d, &op);
  free(label);
  if (status != PK_OK) return throw_status(env, status);
  NAPI_CALL(env, napi_create_external(env, op, conv_finalize, NULL, &ext));
  return ext;
}

/* convEnqueue(op, activeBatch, stream?, startEvent?, endEvent?) */
static napi_value js_conv_enqueue(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  uint32_t batch = 0;
  if (!get_args(env, info, 5, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &batch))
    return bad_argument(env, "active batch must be a non-negative integer");
  PK_CALL(env, pk_conv_enqueue_timed((pk_conv_op *)get_external(env, argv[0]), batch, get_external(env, argv[2]),
                                     get_external(env, argv[3]), get_external(env, argv[4])));
  return undefined(env);
}

static napi_value js_conv_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  PK_CALL(env, pk_conv_destroy((pk_conv_op *)get_external(env, argv[0])));
  return undefined(env);
}

/* convPlan(op, activeBatch?) */
static napi_value js_conv_plan(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  uint32_t batch = 0;
  if (!get_args(env, info, 2, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &batch))
    return bad_argument(env, "active batch must be a non-negative integer");
  pk_conv_plan_info p;
  PK_CALL(env, pk_conv_plan((pk_conv_op *)get_external(env, argv[0]), batch, &p));
  return conv_plan_object(env, &p);
}

/* ---- relative-position attention ------------------------------------------ */

static void attention_finalize(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  pk_attention_release((pk_attention_op *)data);
}

/* A JavaScript attention descriptor: {label, flags?, precision, batchSize,
   frames, qkv, qkvBytes, projectedPositions, projectedPositionsBytes, biasU,
   biasUBytes, biasV, biasVBytes, validLengths, validLengthsBytes, output,
   outputBytes}; device pointers are BigInt. */
static int parse_attention_desc(napi_env env, napi_value o, pk_attention_desc *d, char **label) {
  memset(d, 0, sizeof *d);
  d->struct_size = sizeof *d;
  *label = NULL;
  uint64_t qkv = 0, positions = 0, bu = 0, bv = 0, valid = 0, output = 0;
  parse_precision(env, o, &d->precision);
  if (!prop_u32(env, o, "batchSize", &d->batch_size) || !prop_u32(env, o, "frames", &d->frames) ||
      !prop_u64(env, o, "qkv", &qkv) || !prop_u64(env, o, "qkvBytes", &d->qkv_bytes) ||
      !prop_u64(env, o, "projectedPositions", &positions) ||
      !prop_u64(env, o, "projectedPositionsBytes", &d->projected_positions_bytes) ||
      !prop_u64(env, o, "biasU", &bu) || !prop_u64(env, o, "biasUBytes", &d->bias_u_bytes) ||
      !prop_u64(env, o, "biasV", &bv) || !prop_u64(env, o, "biasVBytes", &d->bias_v_bytes) ||
      !prop_u64(env, o, "validLengths", &valid) || !prop_u64(env, o, "validLengthsBytes", &d->valid_lengths_bytes) ||
      !prop_u64(env, o, "output", &output) || !prop_u64(env, o, "outputBytes", &d->output_bytes)) {
    bad_argument(env, "attention descriptor is missing a required field");
    return 0;
  }
  prop_u32(env, o, "flags", &d->flags);
  d->qkv = (const void *)(uintptr_t)qkv;
  d->projected_positions = (const void *)(uintptr_t)positions;
  d->bias_u = (const float *)(uintptr_t)bu;
  d->bias_v = (const float *)(uintptr_t)bv;
  d->valid_lengths = (const uint32_t *)(uintptr_t)valid;
  d->output = (void *)(uintptr_t)output;
  *label = prop_string(env, o, "label");
  d->label = *label;
  return 1;
}

/* attentionValidate(desc) */
static napi_value js_attention_validate(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  pk_attention_desc d;
  char *label;
  if (!parse_attention_desc(env, argv[0], &d, &label)) return NULL;
  const int status = pk_attention_validate(&d);
  free(label);
  if (status != PK_OK) return throw_status(env, status);
  return undefined(env);
}

/* attentionCreate(ctx, desc) -> op */
static napi_value js_attention_create(napi_env env, napi_callback_info info) {
  napi_value argv[2], ext;
  if (!get_args(env, info, 2, argv)) return NULL;
  pk_attention_desc d;
  char *label;
  if (!parse_attention_desc(env, argv[1], &d, &label)) return NULL;
  pk_attention_op *op = NULL;
  const int status = pk_attention_create((pk_context *)get_external(env, argv[0]), &d, &op);
  free(label);
  if (status != PK_OK) return throw_status(env, status);
  NAPI_CALL(env, napi_create_external(env, op, attention_finalize, NULL, &ext));
  return ext;
}

/* attentionEnqueue(op, activeBatch, stream?, startEvent?, endEvent?) */
static napi_value js_attention_enqueue(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  uint32_t batch = 0;
  if (!get_args(env, info, 5, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &batch))
    return bad_argument(env, "active batch must be a non-negative integer");
  PK_CALL(env, pk_attention_enqueue_timed((pk_attention_op *)get_external(env, argv[0]), batch,
                                          get_external(env, argv[2]), get_external(env, argv[3]),
                                          get_external(env, argv[4])));
  return undefined(env);
}

static napi_value js_attention_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  PK_CALL(env, pk_attention_destroy((pk_attention_op *)get_external(env, argv[0])));
  return undefined(env);
}

/* attentionPlan(op, activeBatch?) */
static napi_value js_attention_plan(napi_env env, napi_callback_info info) {
  napi_value argv[2], obj, grid, v;
  uint32_t batch = 0;
  if (!get_args(env, info, 2, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &batch))
    return bad_argument(env, "active batch must be a non-negative integer");
  pk_attention_plan_info p;
  PK_CALL(env, pk_attention_plan((pk_attention_op *)get_external(env, argv[0]), batch, &p));
  NAPI_CALL(env, napi_create_object(env, &obj));
  NAPI_CALL(env, napi_create_array_with_length(env, 3, &grid));
  for (uint32_t i = 0; i < 3; ++i) napi_set_element(env, grid, i, make_number(env, p.grid[i]));
  napi_set_named_property(env, obj, "workgroups", grid);
  napi_set_named_property(env, obj, "blockThreads", make_number(env, p.block_threads));
  napi_set_named_property(env, obj, "workgroupStorageBytes", make_number(env, p.lds_bytes));
  napi_set_named_property(env, obj, "queryTiles", make_number(env, p.query_tiles));
  napi_set_named_property(env, obj, "algorithmicBytes", make_number(env, (double)p.algorithmic_bytes));
  napi_create_string_utf8(env, p.kernel, NAPI_AUTO_LENGTH, &v);
  napi_set_named_property(env, obj, "kernel", v);
  return obj;
}

/* ---- row LayerNorm ------------------------------------------------------- */

static void layernorm_finalize(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  pk_layernorm_release((pk_layernorm_op *)data);
}

/* {label, precision, rows, channels, input, inputBytes, gamma, gammaBytes,
   beta, betaBytes, output, outputBytes, epsilon?, nextGamma?,
   nextGammaBytes?, nextBeta?, nextBetaBytes?, nextOutput?,
   nextOutputBytes?} (the next* fields: a chained LayerNorm) */
static int parse_layernorm_desc(napi_env env, napi_value o, pk_layernorm_desc *d, char **label) {
  memset(d, 0, sizeof *d);
  d->struct_size = sizeof *d;
  *label = NULL;
  uint64_t input = 0, gamma = 0, beta = 0, output = 0, next_gamma = 0, next_beta = 0, next_output = 0;
  parse_precision(env, o, &d->precision);
  if (!prop_u32(env, o, "rows", &d->rows) || !prop_u32(env, o, "channels", &d->channels) ||
      !prop_u64(env, o, "input", &input) || !prop_u64(env, o, "inputBytes", &d->input_bytes) ||
      !prop_u64(env, o, "gamma", &gamma) || !prop_u64(env, o, "gammaBytes", &d->gamma_bytes) ||
      !prop_u64(env, o, "beta", &beta) || !prop_u64(env, o, "betaBytes", &d->beta_bytes) ||
      !prop_u64(env, o, "output", &output) || !prop_u64(env, o, "outputBytes", &d->output_bytes)) {
    bad_argument(env, "LayerNorm descriptor is missing a required field");
    return 0;
  }
  napi_value eps;
  if (prop(env, o, "epsilon", &eps)) {
    double e = 0;
    napi_get_value_double(env, eps, &e);
    d->has_epsilon = 1;
    d->epsilon = (float)e;
  }
  if (prop_u64(env, o, "nextGamma", &next_gamma)) prop_u64(env, o, "nextGammaBytes", &d->next_gamma_bytes);
  if (prop_u64(env, o, "nextBeta", &next_beta)) prop_u64(env, o, "nextBetaBytes", &d->next_beta_bytes);
  if (prop_u64(env, o, "nextOutput", &next_output)) prop_u64(env, o, "nextOutputBytes", &d->next_output_bytes);
  d->input = (const void *)(uintptr_t)input;
  d->gamma = (const float *)(uintptr_t)gamma;
  d->beta = (const float *)(uintptr_t)beta;
  d->output = (void *)(uintptr_t)output;
  d->next_gamma = (const float *)(uintptr_t)next_gamma;
  d->next_beta = (const float *)(uintptr_t)next_beta;
  d->next_output = (void *)(uintptr_t)next_output;
  *label = prop_string(env, o, "label");
  d->label = *label;
  return 1;
}

static napi_value js_layernorm_validate(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  pk_layernorm_desc d;
  char *label;
  if (!parse_layernorm_desc(env, argv[0], &d, &label)) return NULL;
  const int status = pk_layernorm_validate(&d);
  free(label);
  if (status != PK_OK) return throw_status(env, status);
  return undefined(env);
}

static napi_value js_layernorm_create(napi_env env, napi_callback_info info) {
  napi_value argv[2], ext;
  if (!get_args(env, info, 2, argv)) return NULL;
  pk_layernorm_desc d;
  char *label;
  if (!parse_layernorm_desc(env, argv[1], &d, &label)) return NULL;
  pk_layernorm_op *op = NULL;
  const int status = pk_layernorm_create((pk_context *)get_external(env, argv[0]), &d, &op);
  free(label);
  if (status != PK_OK) return throw_status(env, status);
  NAPI_CALL(env, napi_create_external(env, op, layernorm_finalize, NULL, &ext));
  return ext;
}

/* layernormEnqueue(op, activeRows, stream?, startEvent?, endEvent?) */
static napi_value js_layernorm_enqueue(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  uint32_t rows = 0;
  if (!get_args(env, info, 5, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &rows))
    return bad_argument(env, "active rows must be a non-negative integer");
  PK_CALL(env, pk_layernorm_enqueue_timed((pk_layernorm_op *)get_external(env, argv[0]), rows,
                                          get_external(env, argv[2]), get_external(env, argv[3]),
                                          get_external(env, argv[4])));
  return undefined(env);
}

static napi_value js_layernorm_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  PK_CALL(env, pk_layernorm_destroy((pk_layernorm_op *)get_external(env, argv[0])));
  return undefined(env);
}

/* ---- subsampling ---------------------------------------------------------- */

static void subsampling_finalize(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  pk_subsampling_release((pk_subsampling_op *)data);
}

static napi_value js_subsampling_output_dimension(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  uint32_t n = 0;
  if (!get_args(env, info, 1, argv) || !get_u32(env, argv[0], &n)) return bad_argument(env, "dimension");
  return make_number(env, pk_subsampling_output_dimension(n));
}

static napi_value js_subsampling_valid_length(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  uint32_t n = 0, steps = 0;
  if (!get_args(env, info, 2, argv) || !get_u32(env, argv[0], &n) || !get_u32(env, argv[1], &steps))
    return bad_argument(env, "length and steps");
  return make_number(env, pk_subsampling_valid_length(n, steps));
}

/* Address and byte size fields "<name>" and "<name>Bytes". */
static int ptr_field(napi_env env, napi_value o, const char *name, const void **p, uint64_t *bytes) {
  char key[96];
  uint64_t a = 0;
  snprintf(key, sizeof key, "%sBytes", name);
  if (!prop_u64(env, o, name, &a) || !prop_u64(env, o, key, bytes)) return 0;
  *p = (const void *)(uintptr_t)a;
  return 1;
}

/* kind "fused": {label, precision, batchSize, inputHeight, inputWidth?,
   channels?, input, conv0Weights, conv0Bias, depthwiseWeights,
   depthwiseBias, output, validLengths (each with <name>Bytes),
   validLengthBatchOffset?}; kind "depthwise": {label, precision, batchSize,
   inputHeight, inputWidth, channels, input, weights, bias, output,
   validLengths, validLengthBatchOffset?, validLengthSubsamplingSteps};
   kind "mask": {label, precision, batchSize, height, width, channels,
   values, validLengths, validLengthBatchOffset?, validLengthSubsamplingSteps}. */
static int subsampling_call(napi_env env, napi_value kind_value, napi_value o, pk_context *ctx, int create,
                            pk_subsampling_op **out) {
  char kind[16] = {0};
  size_t len = 0;
  if (napi_get_value_string_utf8(env, kind_value, kind, sizeof kind, &len) != napi_ok) {
    bad_argument(env, "subsampling kind must be \"fused\", \"depthwise\" or \"mask\"");
    return -1;
  }
  char *label = prop_string(env, o, "label");
  int32_t precision = PK_PRECISION_F16;
  parse_precision(env, o, &precision);
  int status = PK_OK, ok = 1;
  const void *p = NULL;
  if (strcmp(kind, "fused") == 0) {
    pk_subsampling_fused_desc d;
    memset(&d, 0, sizeof d);
    d.struct_size = sizeof d;
    d.label = label;
    d.precision = precision;
    d.input_width = PK_SUBSAMPLING_BINS;
    d.channels = PK_SUBSAMPLING_CHANNELS;
    prop_u32(env, o, "inputWidth", &d.input_width);
    prop_u32(env, o, "channels", &d.channels);
    prop_u32(env, o, "validLengthBatchOffset", &d.valid_length_batch_offset);
    ok = prop_u32(env, o, "batchSize", &d.batch_size) && prop_u32(env, o, "inputHeight", &d.input_height);
    ok = ok && ptr_field(env, o, "input", &p, &d.input_bytes);
    d.input = (const float *)p;
    ok = ok && ptr_field(env, o, "conv0Weights", &d.conv0_weights, &d.conv0_weights_bytes);
    ok = ok && ptr_field(env, o, "conv0Bias", &p, &d.conv0_bias_bytes);
    d.conv0_bias = (const float *)p;
    ok = ok && ptr_field(env, o, "depthwiseWeights", &d.depthwise_weights, &d.depthwise_weights_bytes);
    ok = ok && ptr_field(env, o, "depthwiseBias", &p, &d.depthwise_bias_bytes);
    d.depthwise_bias = (const float *)p;
    ok = ok && ptr_field(env, o, "output", &p, &d.output_bytes);
    d.output = (void *)p;
    ok = ok && ptr_field(env, o, "validLengths", &p, &d.valid_lengths_bytes);
    d.valid_lengths = (const uint32_t *)p;
    if (ok) status = create ? pk_subsampling_fused_create(ctx, &d, out) : pk_subsampling_fused_validate(&d);
  } else if (strcmp(kind, "depthwise") == 0) {
    pk_subsampling_depthwise_desc d;
    memset(&d, 0, sizeof d);
    d.struct_size = sizeof d;
    d.label = label;
    d.precision = precision;
    prop_u32(env, o, "validLengthBatchOffset", &d.valid_length_batch_offset);
    ok = prop_u32(env, o, "batchSize", &d.batch_size) && prop_u32(env, o, "inputHeight", &d.input_height) &&
         prop_u32(env, o, "inputWidth", &d.input_width) && prop_u32(env, o, "channels", &d.channels) &&
         prop_u32(env, o, "validLengthSubsamplingSteps", &d.valid_length_subsampling_steps);
    ok = ok && ptr_field(env, o, "input", &d.input, &d.input_bytes);
    ok = ok && ptr_field(env, o, "weights", &d.weights, &d.weights_bytes);
    ok = ok && ptr_field(env, o, "bias", &p, &d.bias_bytes);
    d.bias = (const float *)p;
    ok = ok && ptr_field(env, o, "output", &p, &d.output_bytes);
    d.output = (void *)p;
    ok = ok && ptr_field(env, o, "validLengths", &p, &d.valid_lengths_bytes);
    d.valid_lengths = (const uint32_t *)p;
    if (ok)
      status = create ? pk_subsampling_depthwise_create(ctx, &d, out) : pk_subsampling_depthwise_validate(&d);
  } else if (strcmp(kind, "mask") == 0) {
    pk_subsampling_mask_desc d;
    memset(&d, 0, sizeof d);
    d.struct_size = sizeof d;
    d.label = label;
    d.precision = precision;
    prop_u32(env, o, "validLengthBatchOffset", &d.valid_length_batch_offset);
    ok = prop_u32(env, o, "batchSize", &d.batch_size) && prop_u32(env, o, "height", &d.height) &&
         prop_u32(env, o, "width", &d.width) && prop_u32(env, o, "channels", &d.channels) &&
         prop_u32(env, o, "validLengthSubsamplingSteps", &d.valid_length_subsampling_steps);
    ok = ok && ptr_field(env, o, "values", &p, &d.values_bytes);
    d.values = (void *)p;
    ok = ok && ptr_field(env, o, "validLengths", &p, &d.valid_lengths_bytes);
    d.valid_lengths = (const uint32_t *)p;
    if (ok) status = create ? pk_subsampling_mask_create(ctx, &d, out) : pk_subsampling_mask_validate(&d);
  } else {
    free(label);
    bad_argument(env, "subsampling kind must be \"fused\", \"depthwise\" or \"mask\"");
    return -1;
  }
  free(label);
  if (!ok) {
    bad_argument(env, "subsampling descriptor is missing a required field");
    return -1;
  }
  return status;
}

/* subsamplingValidate(kind, desc) */
static napi_value js_subsampling_validate(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  const int status = subsampling_call(env, argv[0], argv[1], NULL, 0, NULL);
  if (status < 0) return NULL;
  if (status != PK_OK) return throw_status(env, status);
  return undefined(env);
}

/* subsamplingCreate(ctx, kind, desc) -> op */
static napi_value js_subsampling_create(napi_env env, napi_callback_info info) {
  napi_value argv[3], ext;
  if (!get_args(env, info, 3, argv)) return NULL;
  pk_subsampling_op *op = NULL;
  const int status = subsampling_call(env, argv[1], argv[2], (pk_context *)get_external(env, argv[0]), 1, &op);
  if (status < 0) return NULL;
  if (status != PK_OK) return throw_status(env, status);
  NAPI_CALL(env, napi_create_external(env, op, subsampling_finalize, NULL, &ext));
  return ext;
}

/* subsamplingEnqueue(op, activeBatch, stream?, startEvent?, endEvent?) */
static napi_value js_subsampling_enqueue(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  uint32_t batch = 0;
  if (!get_args(env, info, 5, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &batch))
    return bad_argument(env, "active batch must be a non-negative integer");
  PK_CALL(env, pk_subsampling_enqueue_timed((pk_subsampling_op *)get_external(env, argv[0]), batch,
                                            get_external(env, argv[2]), get_external(env, argv[3]),
                                            get_external(env, argv[4])));
  return undefined(env);
}

static napi_value js_subsampling_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  PK_CALL(env, pk_subsampling_destroy((pk_subsampling_op *)get_external(env, argv[0])));
  return undefined(env);
}

/* subsamplingPlan(op, activeBatch?) */
static napi_value js_subsampling_plan(napi_env env, napi_callback_info info) {
  napi_value argv[2], obj, grid, v;
  uint32_t batch = 0;
  if (!get_args(env, info, 2, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &batch))
    return bad_argument(env, "active batch must be a non-negative integer");
  pk_subsampling_plan_info p;
  PK_CALL(env, pk_subsampling_plan((pk_subsampling_op *)get_external(env, argv[0]), batch, &p));
  NAPI_CALL(env, napi_create_object(env, &obj));
  NAPI_CALL(env, napi_create_array_with_length(env, 3, &grid));
  for (uint32_t i = 0; i < 3; ++i) napi_set_element(env, grid, i, make_number(env, p.grid[i]));
  napi_set_named_property(env, obj, "workgroups", grid);
  napi_set_named_property(env, obj, "outputHeight", make_number(env, p.output_height));
  napi_set_named_property(env, obj, "outputWidth", make_number(env, p.output_width));
  napi_set_named_property(env, obj, "blockThreads", make_number(env, p.block_threads));
  napi_set_named_property(env, obj, "workgroupStorageBytes", make_number(env, p.lds_bytes));
  napi_set_named_property(env, obj, "algorithmicBytes", make_number(env, (double)p.algorithmic_bytes));
  napi_set_named_property(env, obj, "flops", make_number(env, (double)p.flops));
  napi_create_string_utf8(env, p.kernel, NAPI_AUTO_LENGTH, &v);
  napi_set_named_property(env, obj, "kernel", v);
  return obj;
}

/* ---- encoder graph -------------------------------------------------------- */

/* The JavaScript handle owns the encoder through a box so an explicit
   destroy and the finalizer never free it twice. */
typedef struct encoder_box {
  pk_encoder *enc;
} encoder_box;

static void encoder_finalize(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  encoder_box *box = (encoder_box *)data;
  if (box->enc) pk_encoder_destroy(box->enc);
  free(box);
}

static int matrix_field(napi_env env, napi_value o, const char *name, pk_encoder_matrix *m) {
  napi_value v;
  uint64_t packed = 0, palette = 0;
  if (!prop(env, o, name, &v) || !prop_u64(env, v, "packed", &packed) || !prop_u64(env, v, "palette", &palette))
    return 0;
  m->packed = (const uint32_t *)(uintptr_t)packed;
  m->palette = (const void *)(uintptr_t)palette;
  return 1;
}

static int address_field(napi_env env, napi_value o, const char *name, const void **p) {
  uint64_t a = 0;
  if (!prop_u64(env, o, name, &a)) return 0;
  *p = (const void *)(uintptr_t)a;
  return 1;
}

static int address_list(napi_env env, napi_value o, const char *name, const float **out, uint32_t count) {
  napi_value list, item;
  uint32_t n = 0;
  if (!prop(env, o, name, &list) || napi_get_array_length(env, list, &n) != napi_ok || n != count) return 0;
  for (uint32_t i = 0; i < count; ++i) {
    uint64_t a = 0;
    if (napi_get_element(env, list, i, &item) != napi_ok || !get_u64(env, item, &a)) return 0;
    out[i] = (const float *)(uintptr_t)a;
  }
  return 1;
}

static int parse_encoder_layer(napi_env env, napi_value o, pk_encoder_layer *l) {
  const void *p = NULL;
  int ok = address_list(env, o, "normGamma", l->norm_gamma, 5) && address_list(env, o, "normBeta", l->norm_beta, 5);
  ok = ok && matrix_field(env, o, "ff1Linear1", &l->ff1_linear1) && matrix_field(env, o, "ff1Linear2", &l->ff1_linear2);
  ok = ok && matrix_field(env, o, "qkv", &l->qkv) && address_field(env, o, "projectedPositions", &l->projected_positions);
  ok = ok && address_field(env, o, "biasU", &p);
  l->bias_u = (const float *)p;
  ok = ok && address_field(env, o, "biasV", &p);
  l->bias_v = (const float *)p;
  ok = ok && matrix_field(env, o, "oProj", &l->o_proj) && matrix_field(env, o, "pointwise1", &l->pointwise1);
  ok = ok && address_field(env, o, "depthwise", &l->depthwise) && address_field(env, o, "bnScale", &p);
  l->bn_scale = (const float *)p;
  ok = ok && address_field(env, o, "bnShift", &p);
  l->bn_shift = (const float *)p;
  ok = ok && matrix_field(env, o, "pointwise2", &l->pointwise2) && matrix_field(env, o, "ff2Linear1", &l->ff2_linear1) &&
       matrix_field(env, o, "ff2Linear2", &l->ff2_linear2);
  return ok;
}

static int parse_encoder_subsampling(napi_env env, napi_value o, pk_encoder_subsampling *f) {
  const void *p = NULL;
  int ok = address_field(env, o, "conv0Weights", &f->conv0_weights) && address_field(env, o, "conv0Bias", &p);
  f->conv0_bias = (const float *)p;
  ok = ok && address_field(env, o, "depthwise2Weights", &f->depthwise2_weights) &&
       address_field(env, o, "depthwise2Bias", &p);
  f->depthwise2_bias = (const float *)p;
  ok = ok && matrix_field(env, o, "pointwise3", &f->pointwise3) && address_field(env, o, "pointwise3Bias", &p);
  f->pointwise3_bias = (const float *)p;
  ok = ok && address_field(env, o, "depthwise5Weights", &f->depthwise5_weights) &&
       address_field(env, o, "depthwise5Bias", &p);
  f->depthwise5_bias = (const float *)p;
  ok = ok && matrix_field(env, o, "pointwise6", &f->pointwise6) && address_field(env, o, "pointwise6Bias", &p);
  f->pointwise6_bias = (const float *)p;
  ok = ok && matrix_field(env, o, "linear", &f->linear) && address_field(env, o, "linearBias", &p);
  f->linear_bias = (const float *)p;
  return ok;
}

/* Parses an encoder descriptor: {label, precision?, fusedGlu?, fusedNorms?, unchainedNorms?, prefixSamePlan?,
   batchSize, frames,
   layers: [layer...], validLengths, input, output, subsampling?,
   featureFrames?, featureLengths?, projector?, projectorBias?,
   projectedChannels?, projectedOutput?}. The layer array, front end and
   label are heap copies the caller frees with free_encoder_desc. */
static int parse_encoder_desc(napi_env env, napi_value o, pk_encoder_desc *d) {
  memset(d, 0, sizeof *d);
  d->struct_size = sizeof *d;
  parse_precision(env, o, &d->precision); /* "f16" (default) or "f32", the fp32 profile */
  napi_value layers, item, v;
  uint32_t n = 0;
  bool glu = true;
  if (prop(env, o, "fusedGlu", &v) && napi_get_value_bool(env, v, &glu) == napi_ok && !glu)
    d->flags |= PK_ENCODER_SEPARATE_GLU;
  bool fused_norms = false, unchained_norms = false;
  if (prop(env, o, "fusedNorms", &v) && napi_get_value_bool(env, v, &fused_norms) == napi_ok && fused_norms)
    d->flags |= PK_ENCODER_FUSED_NORMS;
  if (prop(env, o, "unchainedNorms", &v) && napi_get_value_bool(env, v, &unchained_norms) == napi_ok &&
      unchained_norms)
    d->flags |= PK_ENCODER_UNCHAINED_NORMS;
  bool same_plan = false;
  if (prop(env, o, "prefixSamePlan", &v) && napi_get_value_bool(env, v, &same_plan) == napi_ok && same_plan)
    d->flags |= PK_ENCODER_PREFIX_SAME_PLAN;
  if (!prop_u32(env, o, "batchSize", &d->batch_size) || !prop_u32(env, o, "frames", &d->frames) ||
      !prop(env, o, "layers", &layers) || napi_get_array_length(env, layers, &n) != napi_ok || n == 0) {
    bad_argument(env, "encoder descriptor is missing a required field");
    return 0;
  }
  pk_encoder_layer *array = (pk_encoder_layer *)calloc(n, sizeof *array);
  d->layer = array;
  d->layers = n;
  d->label = prop_string(env, o, "label");
  for (uint32_t i = 0; i < n; ++i) {
    if (napi_get_element(env, layers, i, &item) != napi_ok || !parse_encoder_layer(env, item, &array[i])) {
      bad_argument(env, "encoder layer descriptor is missing a required field");
      return 0;
    }
  }
  const void *p = NULL;
  if (!address_field(env, o, "validLengths", &p)) {
    bad_argument(env, "encoder descriptor is missing validLengths");
    return 0;
  }
  d->valid_lengths = (const uint32_t *)p;
  if (!address_field(env, o, "input", &d->input) || !address_field(env, o, "output", &p)) {
    bad_argument(env, "encoder descriptor is missing input or output");
    return 0;
  }
  d->output = (void *)p;
  if (prop(env, o, "subsampling", &v)) {
    pk_encoder_subsampling *front = (pk_encoder_subsampling *)calloc(1, sizeof *front);
    d->subsampling = front;
    if (!parse_encoder_subsampling(env, v, front) || !prop_u32(env, o, "featureFrames", &d->feature_frames) ||
        !address_field(env, o, "featureLengths", &p)) {
      bad_argument(env, "encoder front end is missing a required field");
      return 0;
    }
    d->feature_lengths = (const uint32_t *)p;
  }
  if (prop(env, o, "projector", &v)) {
    if (!matrix_field(env, o, "projector", &d->projector) || !address_field(env, o, "projectorBias", &p) ||
        !prop_u32(env, o, "projectedChannels", &d->projected_channels)) {
      bad_argument(env, "encoder projector is missing a required field");
      return 0;
    }
    d->projector_bias = (const float *)p;
    if (!address_field(env, o, "projectedOutput", &p)) {
      bad_argument(env, "encoder projector is missing projectedOutput");
      return 0;
    }
    d->projected_output = (void *)p;
  }
  return 1;
}

static void free_encoder_desc(pk_encoder_desc *d) {
  free((void *)d->layer);
  free((void *)d->subsampling);
  free((void *)d->label);
}

static napi_value js_encoder_validate(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  pk_encoder_desc d;
  const int parsed = parse_encoder_desc(env, argv[0], &d);
  const int status = parsed ? pk_encoder_validate(&d) : PK_OK;
  free_encoder_desc(&d);
  if (!parsed) return NULL;
  if (status != PK_OK) return throw_status(env, status);
  return undefined(env);
}

/* encoderCreate(ctx, desc) -> encoder */
static napi_value js_encoder_create(napi_env env, napi_callback_info info) {
  napi_value argv[2], ext;
  if (!get_args(env, info, 2, argv)) return NULL;
  pk_encoder_desc d;
  if (!parse_encoder_desc(env, argv[1], &d)) {
    free_encoder_desc(&d);
    return NULL;
  }
  pk_encoder *enc = NULL;
  const int status = pk_encoder_create((pk_context *)get_external(env, argv[0]), &d, NULL, &enc);
  free_encoder_desc(&d);
  if (status != PK_OK) return throw_status(env, status);
  encoder_box *box = (encoder_box *)malloc(sizeof *box);
  box->enc = enc;
  NAPI_CALL(env, napi_create_external(env, box, encoder_finalize, NULL, &ext));
  return ext;
}

static pk_encoder *encoder_of(napi_env env, napi_value v) {
  encoder_box *box = (encoder_box *)get_external(env, v);
  return box ? box->enc : NULL;
}

/* encoderEnqueue(encoder, activeBatch, stream?, useGraph?) */
static napi_value js_encoder_enqueue(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  uint32_t batch = 0;
  bool graph = false;
  if (!get_args(env, info, 4, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &batch))
    return bad_argument(env, "active batch must be a non-negative integer");
  if (!is_nullish(env, argv[3])) napi_get_value_bool(env, argv[3], &graph);
  PK_CALL(env, pk_encoder_enqueue(encoder_of(env, argv[0]), batch, get_external(env, argv[2]), graph ? 1 : 0));
  return undefined(env);
}

/* encoderEnqueueProfiled(encoder, activeBatch, stream?, startEvents[], endEvents[]) */
static napi_value js_encoder_enqueue_profiled(napi_env env, napi_callback_info info) {
  napi_value argv[5], item;
  uint32_t batch = 0, launches = 0, n0 = 0, n1 = 0;
  if (!get_args(env, info, 5, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &batch))
    return bad_argument(env, "active batch must be a non-negative integer");
  pk_encoder *enc = encoder_of(env, argv[0]);
  PK_CALL(env, pk_encoder_info(enc, &launches, NULL));
  if (napi_get_array_length(env, argv[3], &n0) != napi_ok || napi_get_array_length(env, argv[4], &n1) != napi_ok ||
      n0 != launches || n1 != launches)
    return bad_argument(env, "a profiled pass takes one start and one end event per launch");
  void **events = (void **)calloc(2u * launches, sizeof(void *));
  for (uint32_t i = 0; i < launches; ++i) {
    napi_get_element(env, argv[3], i, &item);
    events[i] = get_external(env, item);
    napi_get_element(env, argv[4], i, &item);
    events[launches + i] = get_external(env, item);
  }
  const int status = pk_encoder_enqueue_profiled(enc, batch, get_external(env, argv[2]), events, events + launches);
  free(events);
  if (status != PK_OK) return throw_status(env, status);
  return undefined(env);
}

/* encoderInfo(encoder) -> {launches, deviceBytes} */
static napi_value js_encoder_info(napi_env env, napi_callback_info info) {
  napi_value argv[1], obj;
  uint32_t launches = 0;
  uint64_t bytes = 0;
  if (!get_args(env, info, 1, argv)) return NULL;
  PK_CALL(env, pk_encoder_info(encoder_of(env, argv[0]), &launches, &bytes));
  NAPI_CALL(env, napi_create_object(env, &obj));
  napi_set_named_property(env, obj, "launches", make_number(env, launches));
  napi_set_named_property(env, obj, "deviceBytes", make_number(env, (double)bytes));
  return obj;
}

/* encoderDestroy(encoder): idempotent. */
static napi_value js_encoder_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  encoder_box *box = (encoder_box *)get_external(env, argv[0]);
  if (box && box->enc) {
    pk_encoder *enc = box->enc;
    box->enc = NULL;
    PK_CALL(env, pk_encoder_destroy(enc));
  }
  return undefined(env);
}

/* ---- greedy TDT decoder --------------------------------------------------- */

static void tdt_finalize(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  pk_tdt_release((pk_tdt_op *)data);
}

/* {label, precision? ("f16" default, or "f32": the fp32 profile), batchSize,
   frames, maxTokens, weights: {embedding, lstmWeight0,
   lstmWeight1, lstmBias0, lstmBias1, projectorWeight, projectorBias,
   headWeight, headBias}, encoderProjected, encodedLengths, decodeStarts,
   decodeEnds, flushFinals, state, predictorScratch, tokens, tokenFrames,
   tokenDurations, metadata}, every address with its "<name>Bytes". */
static int parse_tdt_desc(napi_env env, napi_value o, pk_tdt_desc *d, char **label) {
  memset(d, 0, sizeof *d);
  d->struct_size = sizeof *d;
  d->precision = PK_PRECISION_F16;
  parse_precision(env, o, &d->precision);
  *label = NULL;
  napi_value w;
  const void *p = NULL;
  int ok = prop_u32(env, o, "batchSize", &d->batch_size) && prop_u32(env, o, "frames", &d->frames) &&
           prop_u32(env, o, "maxTokens", &d->max_tokens) && prop(env, o, "weights", &w);
  pk_tdt_weights *t = &d->weights;
  ok = ok && ptr_field(env, w, "embedding", &t->embedding, &t->embedding_bytes);
  ok = ok && ptr_field(env, w, "lstmWeight0", &t->lstm_weight[0], &t->lstm_weight_bytes[0]);
  ok = ok && ptr_field(env, w, "lstmWeight1", &t->lstm_weight[1], &t->lstm_weight_bytes[1]);
  ok = ok && ptr_field(env, w, "lstmBias0", &p, &t->lstm_bias_bytes[0]);
  t->lstm_bias[0] = (const float *)p;
  ok = ok && ptr_field(env, w, "lstmBias1", &p, &t->lstm_bias_bytes[1]);
  t->lstm_bias[1] = (const float *)p;
  ok = ok && ptr_field(env, w, "projectorWeight", &t->projector_weight, &t->projector_weight_bytes);
  ok = ok && ptr_field(env, w, "projectorBias", &p, &t->projector_bias_bytes);
  t->projector_bias = (const float *)p;
  ok = ok && ptr_field(env, w, "headWeight", &t->head_weight, &t->head_weight_bytes);
  ok = ok && ptr_field(env, w, "headBias", &p, &t->head_bias_bytes);
  t->head_bias = (const float *)p;
  ok = ok && ptr_field(env, o, "encoderProjected", &d->encoder_projected, &d->encoder_projected_bytes);
  ok = ok && ptr_field(env, o, "encodedLengths", &p, &d->encoded_lengths_bytes);
  d->encoded_lengths = (const uint32_t *)p;
  ok = ok && ptr_field(env, o, "decodeStarts", &p, &d->decode_starts_bytes);
  d->decode_starts = (const uint32_t *)p;
  ok = ok && ptr_field(env, o, "decodeEnds", &p, &d->decode_ends_bytes);
  d->decode_ends = (const uint32_t *)p;
  ok = ok && ptr_field(env, o, "flushFinals", &p, &d->flush_finals_bytes);
  d->flush_finals = (const uint32_t *)p;
  ok = ok && ptr_field(env, o, "state", &p, &d->state_bytes);
  d->state = (float *)p;
  ok = ok && ptr_field(env, o, "predictorScratch", &p, &d->predictor_scratch_bytes);
  d->predictor_scratch = (float *)p;
  ok = ok && ptr_field(env, o, "tokens", &p, &d->tokens_bytes);
  d->tokens = (uint32_t *)p;
  ok = ok && ptr_field(env, o, "tokenFrames", &p, &d->token_frames_bytes);
  d->token_frames = (uint32_t *)p;
  ok = ok && ptr_field(env, o, "tokenDurations", &p, &d->token_durations_bytes);
  d->token_durations = (uint32_t *)p;
  ok = ok && ptr_field(env, o, "metadata", &p, &d->metadata_bytes);
  d->metadata = (uint32_t *)p;
  if (!ok) {
    bad_argument(env, "TDT decoder descriptor is missing a required field");
    return 0;
  }
  *label = prop_string(env, o, "label");
  d->label = *label;
  return 1;
}

static napi_value js_tdt_plan_execution(napi_env env, napi_callback_info info) {
  napi_value argv[1], obj;
  uint32_t batch = 0;
  if (!get_args(env, info, 1, argv)) return NULL;
  if (!get_u32(env, argv[0], &batch)) batch = 0;
  pk_tdt_execution_plan plan;
  PK_CALL(env, pk_tdt_plan_execution(batch, &plan));
  NAPI_CALL(env, napi_create_object(env, &obj));
  napi_set_named_property(env, obj, "workgroupCount", make_number(env, plan.workgroup_count));
  napi_set_named_property(env, obj, "blockThreads", make_number(env, plan.block_threads));
  napi_set_named_property(env, obj, "predictorScratchByteLength", make_number(env, (double)plan.predictor_scratch_bytes));
  return obj;
}

static napi_value js_tdt_validate(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  pk_tdt_desc d;
  char *label;
  if (!parse_tdt_desc(env, argv[0], &d, &label)) return NULL;
  const int status = pk_tdt_validate(&d);
  free(label);
  if (status != PK_OK) return throw_status(env, status);
  return undefined(env);
}

static napi_value js_tdt_create(napi_env env, napi_callback_info info) {
  napi_value argv[2], ext;
  if (!get_args(env, info, 2, argv)) return NULL;
  pk_tdt_desc d;
  char *label;
  if (!parse_tdt_desc(env, argv[1], &d, &label)) return NULL;
  pk_tdt_op *op = NULL;
  const int status = pk_tdt_create((pk_context *)get_external(env, argv[0]), &d, &op);
  free(label);
  if (status != PK_OK) return throw_status(env, status);
  NAPI_CALL(env, napi_create_external(env, op, tdt_finalize, NULL, &ext));
  return ext;
}

/* tdtEnqueue(op, activeBatch, stream?, startEvent?, endEvent?) */
static napi_value js_tdt_enqueue(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  uint32_t batch = 0;
  if (!get_args(env, info, 5, argv)) return NULL;
  if (!is_nullish(env, argv[1]) && !get_u32(env, argv[1], &batch))
    return bad_argument(env, "active batch must be a non-negative integer");
  PK_CALL(env, pk_tdt_enqueue_timed((pk_tdt_op *)get_external(env, argv[0]), batch, get_external(env, argv[2]),
                                    get_external(env, argv[3]), get_external(env, argv[4])));
  return undefined(env);
}

/* tdtSetTeamSize(op, members): 0 chooses, 1 one workgroup per window, 8 or 16 */
static napi_value js_tdt_set_team_size(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  uint32_t members = 0;
  if (!get_args(env, info, 2, argv) || !get_u32(env, argv[1], &members))
    return bad_argument(env, "team size must be a non-negative integer");
  PK_CALL(env, pk_tdt_set_team_size((pk_tdt_op *)get_external(env, argv[0]), members));
  return undefined(env);
}

/* tdtTeamSize(op) -> workgroups per window of the next launch */
static napi_value js_tdt_team_size(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  uint32_t members = 0;
  if (!get_args(env, info, 1, argv)) return NULL;
  PK_CALL(env, pk_tdt_team_size((const pk_tdt_op *)get_external(env, argv[0]), &members));
  return make_number(env, members);
}

static napi_value js_tdt_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  PK_CALL(env, pk_tdt_destroy((pk_tdt_op *)get_external(env, argv[0])));
  return undefined(env);
}

/* ---- module --------------------------------------------------------------- */

static napi_value init(napi_env env, napi_value exports) {
  const struct {
    const char *name;
    napi_callback fn;
  } fns[] = {
      {"abiVersion", js_abi_version},
      {"contextCreate", js_context_create},
      {"contextDestroy", js_context_destroy},
      {"deviceInfo", js_device_info},
      {"alloc", js_alloc},
      {"free", js_free},
      {"upload", js_upload},
      {"download", js_download},
      {"synchronize", js_synchronize},
      {"synchronizeAsync", js_synchronize_async},
      {"eventCreate", js_event_create},
      {"eventDestroy", js_event_destroy},
      {"eventRecord", js_event_record},
      {"eventElapsedMs", js_event_elapsed_ms},
      {"preparedWeightCreate", js_prepared_weight_create},
      {"preparedWeightDestroy", js_prepared_weight_destroy},
      {"gemmValidate", js_gemm_validate},
      {"gemmCreate", js_gemm_create},
      {"gemmEnqueue", js_gemm_enqueue},
      {"gemmDestroy", js_gemm_destroy},
      {"gemmPlan", js_gemm_plan},
      {"convPlanShape", js_conv_plan_shape},
      {"convValidate", js_conv_validate},
      {"convCreate", js_conv_create},
      {"convEnqueue", js_conv_enqueue},
      {"convDestroy", js_conv_destroy},
      {"convPlan", js_conv_plan},
      {"attentionValidate", js_attention_validate},
      {"attentionCreate", js_attention_create},
      {"attentionEnqueue", js_attention_enqueue},
      {"attentionDestroy", js_attention_destroy},
      {"attentionPlan", js_attention_plan},
      {"layernormValidate", js_layernorm_validate},
      {"layernormCreate", js_layernorm_create},
      {"layernormEnqueue", js_layernorm_enqueue},
      {"layernormDestroy", js_layernorm_destroy},
      {"subsamplingOutputDimension", js_subsampling_output_dimension},
      {"subsamplingValidLength", js_subsampling_valid_length},
      {"subsamplingValidate", js_subsampling_validate},
      {"subsamplingCreate", js_subsampling_create},
      {"subsamplingEnqueue", js_subsampling_enqueue},
      {"subsamplingDestroy", js_subsampling_destroy},
      {"subsamplingPlan", js_subsampling_plan},
      {"encoderValidate", js_encoder_validate},
      {"encoderCreate", js_encoder_create},
      {"encoderEnqueue", js_encoder_enqueue},
      {"encoderEnqueueProfiled", js_encoder_enqueue_profiled},
      {"encoderInfo", js_encoder_info},
      {"encoderDestroy", js_encoder_destroy},
      {"tdtPlanExecution", js_tdt_plan_execution},
      {"tdtValidate", js_tdt_validate},
      {"tdtCreate", js_tdt_create},
      {"tdtEnqueue", js_tdt_enqueue},
      {"tdtDestroy", js_tdt_destroy},
      {"tdtSetTeamSize", js_tdt_set_team_size},
      {"tdtTeamSize", js_tdt_team_size},
  };
  for (size_t i = 0; i < sizeof fns / sizeof fns[0]; ++i) {
    napi_value f;
    NAPI_CALL(env, napi_create_function(env, fns[i].name, NAPI_AUTO_LENGTH, fns[i].fn, NULL, &f));
    NAPI_CALL(env, napi_set_named_property(env, exports, fns[i].name, f));
  }
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)

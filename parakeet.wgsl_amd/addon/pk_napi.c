/*
 * pk_napi.c - Node-API (N-API 8) addon over the palette GEMM C ABI
 * (include/pk_palette.h), the fused Conformer convolution tail
 * (include/pk_conv.h) and the relative-position attention
 * (include/pk_attention.h). It is the thin native layer under the JavaScript
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
#include "pk_palette.h"

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

static void weight_finalize(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  pk_prepared_weight_destroy((pk_prepared_weight *)data);
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
  NAPI_CALL(env, napi_create_external(env, w, weight_finalize, NULL, &ext));
  return ext;
}

static napi_value js_prepared_weight_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  PK_CALL(env, pk_prepared_weight_destroy((pk_prepared_weight *)get_external(env, argv[0])));
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
  uint64_t a = 0, packed = 0, palette = 0, output = 0, bias = 0, residual = 0;
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
  if (prop(env, o, "prepared", &v)) d->prepared = (const pk_prepared_weight *)get_external(env, v);
  d->a = (const void *)(uintptr_t)a;
  d->packed = (const uint32_t *)(uintptr_t)packed;
  d->palette = (const void *)(uintptr_t)palette;
  d->output = (void *)(uintptr_t)output;
  d->bias = (const float *)(uintptr_t)bias;
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
  };
  for (size_t i = 0; i < sizeof fns / sizeof fns[0]; ++i) {
    napi_value f;
    NAPI_CALL(env, napi_create_function(env, fns[i].name, NAPI_AUTO_LENGTH, fns[i].fn, NULL, &f));
    NAPI_CALL(env, napi_set_named_property(env, exports, fns[i].name, f));
  }
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)

"""ctypes binding of libpk_palette.so (include/pk_palette.h, pk_conv.h, pk_attention.h,
pk_layernorm.h, pk_subsampling.h, pk_encoder.h, pk_tdt.h).

A thin Python view of the C ABI, used by the tests and the benchmark. It
raises PaletteError (or PaletteRangeError, mirroring the reference's
RangeError cases) carrying pk_last_error() when a call fails, and it never
falls back to anything: if the library is missing, load() raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "lib", "libpk_palette.so")

OK, INVALID_ARGUMENT, ALLOCATION_FAILURE, INTERNAL_ERROR, DEVICE_ERROR, DESTROYED, RANGE_ERROR = range(7)
PRECISION = {"f16": 0, "f32": 1}
ACTIVATION = {"none": 0, "silu": 1, "relu": 2}
REQUIRE_PRODUCTION_SIGNATURE = 0x1
GEMM_GLU = 0x2
GEMM_ROW_NORM = 0x4
GEMM_CACHED_OUTPUT = 0x8
CONV_INPUT_GLU = 0x1
ATTENTION_POSITIONS_ROW_MAJOR = 0x1
ATTENTION_PLAN_ACTIVE = 0x2
ENCODER_FUSED_GLU = 0x1
ENCODER_FUSED_NORMS = 0x2
ENCODER_SEPARATE_GLU = 0x8
ENCODER_UNCHAINED_NORMS = 0x4
ENCODER_PREFIX_SAME_PLAN = 0x10
ENCODER_CHANNELS = 1024
ENCODER_INTERMEDIATE = 4096
# The fifteen dispatches of one encoder layer, in launch order
# (createEncoderLayerDispatches, encoder.ts:1868-2135).
ENCODER_DISPATCHES = ("norm_feed_forward1", "feed-forward1-linear1", "feed-forward1-linear2-residual",
                      "norm_self_att", "self-attention-qkv", "relative-attention",
                      "self-attention-output-residual", "norm_conv", "convolution-pointwise1",
                      "convolution-glu-depthwise-bn-silu", "convolution-pointwise2-residual", "norm_feed_forward2",
                      "feed-forward2-linear1", "feed-forward2-linear2-residual", "norm_out")
EXPAND_LAYOUT = {"row-major": 0, "tile-major": 1}


class PaletteError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class PaletteRangeError(PaletteError):
    pass


class PaletteDestroyedError(PaletteError):
    pass


class WeightDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("label", ctypes.c_char_p),
        ("palette_bits", ctypes.c_int32),
        ("inner", ctypes.c_uint32),
        ("columns", ctypes.c_uint32),
        ("packed", ctypes.c_void_p),
        ("packed_bytes", ctypes.c_uint64),
    ]


class GemmDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("label", ctypes.c_char_p),
        ("precision", ctypes.c_int32),
        ("palette_bits", ctypes.c_int32),
        ("rows", ctypes.c_uint32),
        ("inner", ctypes.c_uint32),
        ("columns", ctypes.c_uint32),
        ("palette_groups", ctypes.c_uint32),
        ("palette_group_columns", ctypes.c_uint32),
        ("a", ctypes.c_void_p),
        ("a_bytes", ctypes.c_uint64),
        ("packed", ctypes.c_void_p),
        ("packed_bytes", ctypes.c_uint64),
        ("palette", ctypes.c_void_p),
        ("palette_bytes", ctypes.c_uint64),
        ("output", ctypes.c_void_p),
        ("output_bytes", ctypes.c_uint64),
        ("bias", ctypes.c_void_p),
        ("bias_bytes", ctypes.c_uint64),
        ("residual", ctypes.c_void_p),
        ("residual_bytes", ctypes.c_uint64),
        ("has_residual_scale", ctypes.c_int32),
        ("residual_scale", ctypes.c_float),
        ("activation", ctypes.c_int32),
        ("prepared", ctypes.c_void_p),
        ("norm_gamma", ctypes.c_void_p),
        ("norm_gamma_bytes", ctypes.c_uint64),
        ("norm_beta", ctypes.c_void_p),
        ("norm_beta_bytes", ctypes.c_uint64),
        ("norm_epsilon", ctypes.c_float),
    ]


class PlanInfo(ctypes.Structure):
    _fields_ = [
        ("grid", ctypes.c_uint32 * 3),
        ("block_threads", ctypes.c_uint32),
        ("tile_rows", ctypes.c_uint32),
        ("tile_columns", ctypes.c_uint32),
        ("split_inner", ctypes.c_uint32),
        ("lds_bytes", ctypes.c_uint32),
        ("workspace_bytes", ctypes.c_uint64),
        ("flops", ctypes.c_uint64),
        ("algorithmic_bytes", ctypes.c_uint64),
        ("kernel", ctypes.c_char * 64),
        ("stream_stores", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


class VariantDesc(ctypes.Structure):
    _fields_ = [
        ("tile_rows", ctypes.c_uint32),
        ("tile_columns", ctypes.c_uint32),
        ("block_threads", ctypes.c_uint32),
        ("k_split", ctypes.c_uint32),
        ("code_parts", ctypes.c_uint32),
        ("groupable", ctypes.c_int32),
        ("kernel5", ctypes.c_char * 64),
        ("kernel6", ctypes.c_char * 64),
    ]


class ExpandDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("label", ctypes.c_char_p),
        ("precision", ctypes.c_int32),
        ("palette_bits", ctypes.c_int32),
        ("layout", ctypes.c_int32),
        ("inner", ctypes.c_uint32),
        ("columns", ctypes.c_uint32),
        ("palette_groups", ctypes.c_uint32),
        ("palette_group_columns", ctypes.c_uint32),
        ("packed", ctypes.c_void_p),
        ("packed_bytes", ctypes.c_uint64),
        ("palette", ctypes.c_void_p),
        ("palette_bytes", ctypes.c_uint64),
        ("target", ctypes.c_void_p),
        ("target_bytes", ctypes.c_uint64),
    ]


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 64),
        ("arch", ctypes.c_char * 32),
        ("compute_units", ctypes.c_int32),
        ("wavefront_size", ctypes.c_int32),
        ("global_memory_bytes", ctypes.c_int64),
        ("lds_bytes_per_block", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
    ]


class ConvDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("label", ctypes.c_char_p),
        ("precision", ctypes.c_int32),
        ("batch_size", ctypes.c_uint32),
        ("frames", ctypes.c_uint32),
        ("channels", ctypes.c_uint32),
        ("pointwise_input", ctypes.c_void_p),
        ("pointwise_input_bytes", ctypes.c_uint64),
        ("depthwise_weights", ctypes.c_void_p),
        ("depthwise_weights_bytes", ctypes.c_uint64),
        ("batch_norm_scale", ctypes.c_void_p),
        ("batch_norm_scale_bytes", ctypes.c_uint64),
        ("batch_norm_shift", ctypes.c_void_p),
        ("batch_norm_shift_bytes", ctypes.c_uint64),
        ("valid_lengths", ctypes.c_void_p),
        ("valid_lengths_bytes", ctypes.c_uint64),
        ("output", ctypes.c_void_p),
        ("output_bytes", ctypes.c_uint64),
    ]


class ConvPlanInfo(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_uint32),
        ("input_bytes", ctypes.c_uint64),
        ("output_bytes", ctypes.c_uint64),
        ("valid_lengths_bytes", ctypes.c_uint64),
        ("depthwise_weight_bytes", ctypes.c_uint64),
        ("affine_bytes", ctypes.c_uint64),
        ("grid", ctypes.c_uint32 * 3),
        ("block_threads", ctypes.c_uint32),
        ("lds_bytes", ctypes.c_uint32),
        ("algorithmic_bytes", ctypes.c_uint64),
        ("kernel", ctypes.c_char * 64),
    ]


class AttentionDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("label", ctypes.c_char_p),
        ("precision", ctypes.c_int32),
        ("batch_size", ctypes.c_uint32),
        ("frames", ctypes.c_uint32),
        ("qkv", ctypes.c_void_p),
        ("qkv_bytes", ctypes.c_uint64),
        ("projected_positions", ctypes.c_void_p),
        ("projected_positions_bytes", ctypes.c_uint64),
        ("bias_u", ctypes.c_void_p),
        ("bias_u_bytes", ctypes.c_uint64),
        ("bias_v", ctypes.c_void_p),
        ("bias_v_bytes", ctypes.c_uint64),
        ("valid_lengths", ctypes.c_void_p),
        ("valid_lengths_bytes", ctypes.c_uint64),
        ("output", ctypes.c_void_p),
        ("output_bytes", ctypes.c_uint64),
    ]


class AttentionPlanInfo(ctypes.Structure):
    _fields_ = [
        ("grid", ctypes.c_uint32 * 3),
        ("block_threads", ctypes.c_uint32),
        ("lds_bytes", ctypes.c_uint32),
        ("query_tiles", ctypes.c_uint32),
        ("algorithmic_bytes", ctypes.c_uint64),
        ("kernel", ctypes.c_char * 64),
    ]


class LayerNormDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("label", ctypes.c_char_p),
        ("precision", ctypes.c_int32),
        ("rows", ctypes.c_uint32),
        ("channels", ctypes.c_uint32),
        ("input", ctypes.c_void_p),
        ("input_bytes", ctypes.c_uint64),
        ("gamma", ctypes.c_void_p),
        ("gamma_bytes", ctypes.c_uint64),
        ("beta", ctypes.c_void_p),
        ("beta_bytes", ctypes.c_uint64),
        ("output", ctypes.c_void_p),
        ("output_bytes", ctypes.c_uint64),
        ("has_epsilon", ctypes.c_int32),
        ("epsilon", ctypes.c_float),
        ("next_gamma", ctypes.c_void_p),
        ("next_gamma_bytes", ctypes.c_uint64),
        ("next_beta", ctypes.c_void_p),
        ("next_beta_bytes", ctypes.c_uint64),
        ("next_output", ctypes.c_void_p),
        ("next_output_bytes", ctypes.c_uint64),
    ]


class SubsamplingFusedDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("label", ctypes.c_char_p),
        ("precision", ctypes.c_int32),
        ("batch_size", ctypes.c_uint32),
        ("input_height", ctypes.c_uint32),
        ("input_width", ctypes.c_uint32),
        ("channels", ctypes.c_uint32),
        ("input", ctypes.c_void_p),
        ("input_bytes", ctypes.c_uint64),
        ("conv0_weights", ctypes.c_void_p),
        ("conv0_weights_bytes", ctypes.c_uint64),
        ("conv0_bias", ctypes.c_void_p),
        ("conv0_bias_bytes", ctypes.c_uint64),
        ("depthwise_weights", ctypes.c_void_p),
        ("depthwise_weights_bytes", ctypes.c_uint64),
        ("depthwise_bias", ctypes.c_void_p),
        ("depthwise_bias_bytes", ctypes.c_uint64),
        ("output", ctypes.c_void_p),
        ("output_bytes", ctypes.c_uint64),
        ("valid_lengths", ctypes.c_void_p),
        ("valid_lengths_bytes", ctypes.c_uint64),
        ("valid_length_batch_offset", ctypes.c_uint32),
    ]


class SubsamplingDepthwiseDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("label", ctypes.c_char_p),
        ("precision", ctypes.c_int32),
        ("batch_size", ctypes.c_uint32),
        ("input_height", ctypes.c_uint32),
        ("input_width", ctypes.c_uint32),
        ("channels", ctypes.c_uint32),
        ("input", ctypes.c_void_p),
        ("input_bytes", ctypes.c_uint64),
        ("weights", ctypes.c_void_p),
        ("weights_bytes", ctypes.c_uint64),
        ("bias", ctypes.c_void_p),
        ("bias_bytes", ctypes.c_uint64),
        ("output", ctypes.c_void_p),
        ("output_bytes", ctypes.c_uint64),
        ("valid_lengths", ctypes.c_void_p),
        ("valid_lengths_bytes", ctypes.c_uint64),
        ("valid_length_batch_offset", ctypes.c_uint32),
        ("valid_length_subsampling_steps", ctypes.c_uint32),
    ]


class SubsamplingMaskDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("label", ctypes.c_char_p),
        ("precision", ctypes.c_int32),
        ("batch_size", ctypes.c_uint32),
        ("height", ctypes.c_uint32),
        ("width", ctypes.c_uint32),
        ("channels", ctypes.c_uint32),
        ("values", ctypes.c_void_p),
        ("values_bytes", ctypes.c_uint64),
        ("valid_lengths", ctypes.c_void_p),
        ("valid_lengths_bytes", ctypes.c_uint64),
        ("valid_length_batch_offset", ctypes.c_uint32),
        ("valid_length_subsampling_steps", ctypes.c_uint32),
    ]


class SubsamplingPlanInfo(ctypes.Structure):
    _fields_ = [
        ("output_height", ctypes.c_uint32),
        ("output_width", ctypes.c_uint32),
        ("grid", ctypes.c_uint32 * 3),
        ("block_threads", ctypes.c_uint32),
        ("lds_bytes", ctypes.c_uint32),
        ("algorithmic_bytes", ctypes.c_uint64),
        ("flops", ctypes.c_uint64),
        ("kernel", ctypes.c_char * 64),
    ]


class TdtWeights(ctypes.Structure):
    _fields_ = [
        ("embedding", ctypes.c_void_p),
        ("embedding_bytes", ctypes.c_uint64),
        ("lstm_weight", ctypes.c_void_p * 2),
        ("lstm_weight_bytes", ctypes.c_uint64 * 2),
        ("lstm_bias", ctypes.c_void_p * 2),
        ("lstm_bias_bytes", ctypes.c_uint64 * 2),
        ("projector_weight", ctypes.c_void_p),
        ("projector_weight_bytes", ctypes.c_uint64),
        ("projector_bias", ctypes.c_void_p),
        ("projector_bias_bytes", ctypes.c_uint64),
        ("head_weight", ctypes.c_void_p),
        ("head_weight_bytes", ctypes.c_uint64),
        ("head_bias", ctypes.c_void_p),
        ("head_bias_bytes", ctypes.c_uint64),
    ]


class TdtDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("label", ctypes.c_char_p),
        ("precision", ctypes.c_int32),
        ("batch_size", ctypes.c_uint32),
        ("frames", ctypes.c_uint32),
        ("max_tokens", ctypes.c_uint32),
        ("weights", TdtWeights),
    ] + [(name, t) for field in ("encoder_projected", "encoded_lengths", "decode_starts", "decode_ends",
                                 "flush_finals", "state", "predictor_scratch", "tokens", "token_frames",
                                 "token_durations", "metadata")
         for name, t in ((field, ctypes.c_void_p), (field + "_bytes", ctypes.c_uint64))]


class TdtExecutionPlan(ctypes.Structure):
    _fields_ = [("workgroup_count", ctypes.c_uint32), ("block_threads", ctypes.c_uint32),
                ("predictor_scratch_bytes", ctypes.c_uint64)]


class EncoderMatrix(ctypes.Structure):
    _fields_ = [("packed", ctypes.c_void_p), ("palette", ctypes.c_void_p)]


class EncoderLayer(ctypes.Structure):
    _fields_ = [
        ("norm_gamma", ctypes.c_void_p * 5),
        ("norm_beta", ctypes.c_void_p * 5),
        ("ff1_linear1", EncoderMatrix),
        ("ff1_linear2", EncoderMatrix),
        ("qkv", EncoderMatrix),
        ("projected_positions", ctypes.c_void_p),
        ("bias_u", ctypes.c_void_p),
        ("bias_v", ctypes.c_void_p),
        ("o_proj", EncoderMatrix),
        ("pointwise1", EncoderMatrix),
        ("depthwise", ctypes.c_void_p),
        ("bn_scale", ctypes.c_void_p),
        ("bn_shift", ctypes.c_void_p),
        ("pointwise2", EncoderMatrix),
        ("ff2_linear1", EncoderMatrix),
        ("ff2_linear2", EncoderMatrix),
    ]


class EncoderSubsampling(ctypes.Structure):
    _fields_ = [
        ("conv0_weights", ctypes.c_void_p),
        ("conv0_bias", ctypes.c_void_p),
        ("depthwise2_weights", ctypes.c_void_p),
        ("depthwise2_bias", ctypes.c_void_p),
        ("pointwise3", EncoderMatrix),
        ("pointwise3_bias", ctypes.c_void_p),
        ("depthwise5_weights", ctypes.c_void_p),
        ("depthwise5_bias", ctypes.c_void_p),
        ("pointwise6", EncoderMatrix),
        ("pointwise6_bias", ctypes.c_void_p),
        ("linear", EncoderMatrix),
        ("linear_bias", ctypes.c_void_p),
    ]


class EncoderDesc(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("label", ctypes.c_char_p),
        ("precision", ctypes.c_int32),
        ("batch_size", ctypes.c_uint32),
        ("frames", ctypes.c_uint32),
        ("layers", ctypes.c_uint32),
        ("layer", ctypes.POINTER(EncoderLayer)),
        ("valid_lengths", ctypes.c_void_p),
        ("input", ctypes.c_void_p),
        ("output", ctypes.c_void_p),
        ("subsampling", ctypes.POINTER(EncoderSubsampling)),
        ("feature_frames", ctypes.c_uint32),
        ("feature_lengths", ctypes.c_void_p),
        ("projector", EncoderMatrix),
        ("projector_bias", ctypes.c_void_p),
        ("projected_channels", ctypes.c_uint32),
        ("projected_output", ctypes.c_void_p),
    ]


# Every function the headers declare: name -> (restype, argtypes).
_VP = ctypes.c_void_p
_PPV = ctypes.POINTER(ctypes.c_void_p)
SIGNATURES = {
    "pk_abi_version": (ctypes.c_int, []),
    "pk_last_error": (ctypes.c_char_p, []),
    "pk_status_name": (ctypes.c_char_p, [ctypes.c_int]),
    "pk_context_create": (ctypes.c_int, [ctypes.c_int, _PPV]),
    "pk_context_destroy": (ctypes.c_int, [_VP]),
    "pk_context_device": (ctypes.c_int, [_VP, ctypes.POINTER(ctypes.c_int)]),
    "pk_context_stream": (ctypes.c_int, [_VP, _PPV]),
    "pk_device_query": (ctypes.c_int, [_VP, ctypes.POINTER(DeviceInfo)]),
    "pk_alloc": (ctypes.c_int, [_VP, ctypes.c_uint64, _PPV]),
    "pk_free": (ctypes.c_int, [_VP, _VP]),
    "pk_upload": (ctypes.c_int, [_VP, _VP, _VP, ctypes.c_uint64, _VP]),
    "pk_download": (ctypes.c_int, [_VP, _VP, _VP, ctypes.c_uint64, _VP]),
    "pk_copy_device": (ctypes.c_int, [_VP, _VP, _VP, ctypes.c_uint64, _VP]),
    "pk_stream_create": (ctypes.c_int, [_VP, _PPV]),
    "pk_stream_destroy": (ctypes.c_int, [_VP, _VP]),
    "pk_stream_synchronize": (ctypes.c_int, [_VP, _VP]),
    "pk_event_create": (ctypes.c_int, [_VP, _PPV]),
    "pk_event_destroy": (ctypes.c_int, [_VP, _VP]),
    "pk_event_record": (ctypes.c_int, [_VP, _VP, _VP]),
    "pk_event_synchronize": (ctypes.c_int, [_VP, _VP]),
    "pk_event_elapsed_ms": (ctypes.c_int, [_VP, _VP, _VP, ctypes.POINTER(ctypes.c_float)]),
    "pk_prepared_weight_create": (ctypes.c_int, [_VP, ctypes.POINTER(WeightDesc), _VP, _PPV]),
    "pk_prepared_weight_destroy": (ctypes.c_int, [_VP]),
    "pk_prepared_weight_bytes": (ctypes.c_int, [_VP, ctypes.POINTER(ctypes.c_uint64)]),
    "pk_gemm_create": (ctypes.c_int, [_VP, ctypes.POINTER(GemmDesc), _VP, _PPV]),
    "pk_gemm_validate": (ctypes.c_int, [ctypes.POINTER(GemmDesc)]),
    "pk_gemm_enqueue": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP]),
    "pk_gemm_enqueue_timed": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP, _VP, _VP]),
    "pk_gemm_destroy": (ctypes.c_int, [_VP]),
    "pk_gemm_release": (ctypes.c_int, [_VP]),
    "pk_gemm_variant_count": (ctypes.c_int, [ctypes.c_int]),
    "pk_gemm_variant_describe": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.POINTER(VariantDesc)]),
    "pk_gemm_set_variant": (ctypes.c_int, [_VP, ctypes.c_int]),
    "pk_gemm_set_splits": (ctypes.c_int, [_VP, ctypes.c_uint32]),
    "pk_gemm_prepare_rows": (ctypes.c_int, [_VP, ctypes.POINTER(ctypes.c_uint32), ctypes.c_uint32]),
    "pk_gemm_plan": (ctypes.c_int, [_VP, ctypes.c_uint32, ctypes.POINTER(PlanInfo)]),
    "pk_gemm_group_create": (ctypes.c_int, [_VP, ctypes.POINTER(_VP), ctypes.c_uint32, ctypes.c_char_p, _PPV]),
    "pk_gemm_group_enqueue": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP]),
    "pk_gemm_group_enqueue_timed": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP, _VP, _VP]),
    "pk_gemm_group_set_variant": (ctypes.c_int, [_VP, ctypes.c_int]),
    "pk_gemm_group_plan": (ctypes.c_int, [_VP, ctypes.c_uint32, ctypes.POINTER(PlanInfo)]),
    "pk_gemm_group_destroy": (ctypes.c_int, [_VP]),
    "pk_palette_expand": (ctypes.c_int, [_VP, ctypes.POINTER(ExpandDesc), _VP]),
    "pk_unpack_codes": (ctypes.c_int, [_VP, ctypes.c_int, _VP, ctypes.c_uint64, _VP, _VP]),
    "pk_conv_plan_shape": (ctypes.c_int, [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                          ctypes.POINTER(ConvPlanInfo)]),
    "pk_conv_validate": (ctypes.c_int, [ctypes.POINTER(ConvDesc)]),
    "pk_conv_create": (ctypes.c_int, [_VP, ctypes.POINTER(ConvDesc), _PPV]),
    "pk_conv_enqueue": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP]),
    "pk_conv_enqueue_timed": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP, _VP, _VP]),
    "pk_conv_plan": (ctypes.c_int, [_VP, ctypes.c_uint32, ctypes.POINTER(ConvPlanInfo)]),
    "pk_conv_destroy": (ctypes.c_int, [_VP]),
    "pk_conv_release": (ctypes.c_int, [_VP]),
    "pk_conv_variant_count": (ctypes.c_int, [ctypes.c_int]),
    "pk_conv_set_variant": (ctypes.c_int, [_VP, ctypes.c_int]),
    "pk_attention_validate": (ctypes.c_int, [ctypes.POINTER(AttentionDesc)]),
    "pk_attention_create": (ctypes.c_int, [_VP, ctypes.POINTER(AttentionDesc), _PPV]),
    "pk_attention_enqueue": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP]),
    "pk_attention_enqueue_timed": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP, _VP, _VP]),
    "pk_attention_plan": (ctypes.c_int, [_VP, ctypes.c_uint32, ctypes.POINTER(AttentionPlanInfo)]),
    "pk_attention_destroy": (ctypes.c_int, [_VP]),
    "pk_attention_release": (ctypes.c_int, [_VP]),
    "pk_attention_variant_count": (ctypes.c_int, [ctypes.c_int]),
    "pk_attention_set_variant": (ctypes.c_int, [_VP, ctypes.c_int]),
    "pk_layernorm_validate": (ctypes.c_int, [ctypes.POINTER(LayerNormDesc)]),
    "pk_layernorm_create": (ctypes.c_int, [_VP, ctypes.POINTER(LayerNormDesc), _PPV]),
    "pk_layernorm_enqueue": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP]),
    "pk_layernorm_enqueue_timed": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP, _VP, _VP]),
    "pk_layernorm_destroy": (ctypes.c_int, [_VP]),
    "pk_layernorm_release": (ctypes.c_int, [_VP]),
    "pk_subsampling_output_dimension": (ctypes.c_uint32, [ctypes.c_uint32]),
    "pk_subsampling_valid_length": (ctypes.c_uint32, [ctypes.c_uint32, ctypes.c_uint32]),
    "pk_subsampling_fused_validate": (ctypes.c_int, [ctypes.POINTER(SubsamplingFusedDesc)]),
    "pk_subsampling_fused_create": (ctypes.c_int, [_VP, ctypes.POINTER(SubsamplingFusedDesc), _PPV]),
    "pk_subsampling_depthwise_validate": (ctypes.c_int, [ctypes.POINTER(SubsamplingDepthwiseDesc)]),
    "pk_subsampling_depthwise_create": (ctypes.c_int, [_VP, ctypes.POINTER(SubsamplingDepthwiseDesc), _PPV]),
    "pk_subsampling_mask_validate": (ctypes.c_int, [ctypes.POINTER(SubsamplingMaskDesc)]),
    "pk_subsampling_mask_create": (ctypes.c_int, [_VP, ctypes.POINTER(SubsamplingMaskDesc), _PPV]),
    "pk_subsampling_enqueue": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP]),
    "pk_subsampling_enqueue_timed": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP, _VP, _VP]),
    "pk_subsampling_plan": (ctypes.c_int, [_VP, ctypes.c_uint32, ctypes.POINTER(SubsamplingPlanInfo)]),
    "pk_subsampling_destroy": (ctypes.c_int, [_VP]),
    "pk_subsampling_release": (ctypes.c_int, [_VP]),
    "pk_tdt_plan_execution": (ctypes.c_int, [ctypes.c_uint32, ctypes.POINTER(TdtExecutionPlan)]),
    "pk_tdt_validate": (ctypes.c_int, [ctypes.POINTER(TdtDesc)]),
    "pk_tdt_create": (ctypes.c_int, [_VP, ctypes.POINTER(TdtDesc), _PPV]),
    "pk_tdt_enqueue": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP]),
    "pk_tdt_enqueue_timed": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP, _VP, _VP]),
    "pk_tdt_destroy": (ctypes.c_int, [_VP]),
    "pk_tdt_release": (ctypes.c_int, [_VP]),
    "pk_tdt_set_team_size": (ctypes.c_int, [_VP, ctypes.c_uint32]),
    "pk_graph_begin_capture": (ctypes.c_int, [_VP, _VP]),
    "pk_graph_end_capture": (ctypes.c_int, [_VP, _VP, _PPV]),
    "pk_graph_launch": (ctypes.c_int, [_VP, _VP]),
    "pk_graph_destroy": (ctypes.c_int, [_VP]),
    "pk_tdt_team_size": (ctypes.c_int, [_VP, ctypes.POINTER(ctypes.c_uint32)]),
    "pk_tdt_decode_static": (ctypes.c_int, [_VP, ctypes.POINTER(TdtDesc), ctypes.c_uint32, _VP]),
    "pk_encoder_validate": (ctypes.c_int, [ctypes.POINTER(EncoderDesc)]),
    "pk_encoder_create": (ctypes.c_int, [_VP, ctypes.POINTER(EncoderDesc), _VP, _PPV]),
    "pk_encoder_enqueue": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP, ctypes.c_int]),
    "pk_encoder_enqueue_profiled": (ctypes.c_int, [_VP, ctypes.c_uint32, _VP, _PPV, _PPV]),
    "pk_encoder_info": (ctypes.c_int, [_VP, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint64)]),
    "pk_encoder_destroy": (ctypes.c_int, [_VP]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load the in-tree libpk_palette.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `python parakeet.wgsl_amd/build.py`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status == OK:
        return
    message = load().pk_last_error().decode(errors="replace")
    if status == RANGE_ERROR:
        raise PaletteRangeError(status, message)
    if status == DESTROYED:
        raise PaletteDestroyedError(status, message)
    raise PaletteError(status, message)


def codes_per_group(bits: int) -> int:
    return {5: 32, 6: 16}[bits]


def words_per_group(bits: int) -> int:
    return {5: 5, 6: 3}[bits]


class DeviceArray:
    """A device allocation with a numpy dtype and shape."""

    def __init__(self, ctx: "Context", shape, dtype):
        self.ctx = ctx
        if isinstance(shape, (int, np.integer)):
            shape = (int(shape),)
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        ptr = ctypes.c_void_p()
        check(load().pk_alloc(ctx.handle, self.nbytes, ctypes.byref(ptr)))
        self.ptr = ptr.value

    def upload(self, array: np.ndarray, stream=None) -> "DeviceArray":
        array = np.ascontiguousarray(array, dtype=self.dtype)
        if array.nbytes != self.nbytes:
            raise ValueError(f"upload of {array.nbytes} bytes into {self.nbytes}")
        check(load().pk_upload(self.ctx.handle, self.ptr, array.ctypes.data, self.nbytes, stream))
        return self

    def download(self, stream=None) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        check(load().pk_download(self.ctx.handle, out.ctypes.data, self.ptr, self.nbytes, stream))
        return out

    def free(self) -> None:
        if self.ptr:
            check(load().pk_free(self.ctx.handle, self.ptr))
            self.ptr = None


class Context:
    def __init__(self, device: int = 0):
        handle = ctypes.c_void_p()
        check(load().pk_context_create(device, ctypes.byref(handle)))
        self.handle = handle.value
        stream = ctypes.c_void_p()
        check(load().pk_context_stream(self.handle, ctypes.byref(stream)))
        self.stream = stream.value

    def close(self) -> None:
        if self.handle:
            check(load().pk_context_destroy(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> DeviceInfo:
        info = DeviceInfo()
        check(load().pk_device_query(self.handle, ctypes.byref(info)))
        return info

    def array(self, host: np.ndarray) -> DeviceArray:
        host = np.ascontiguousarray(host)
        return DeviceArray(self, host.shape, host.dtype).upload(host)

    def empty(self, shape, dtype) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def synchronize(self, stream=None) -> None:
        check(load().pk_stream_synchronize(self.handle, stream))

    def copy(self, dst: DeviceArray, src: DeviceArray, stream=None) -> None:
        check(load().pk_copy_device(self.handle, dst.ptr, src.ptr, min(dst.nbytes, src.nbytes), stream))

    def event(self) -> "Event":
        return Event(self)

    def unpack_codes(self, bits: int, words: DeviceArray, codes: DeviceArray, stream=None) -> None:
        groups = words.nbytes // (4 * words_per_group(bits))
        check(load().pk_unpack_codes(self.handle, bits, words.ptr, groups, codes.ptr, stream))

    def expand(self, bits: int, packed: DeviceArray, palette: DeviceArray, target: DeviceArray,
               inner: int, columns: int, *, layout: str = "row-major", label: str = "expand",
               stream=None) -> None:
        precision = "f16" if palette.dtype == np.float16 else "f32"
        groups = palette.shape[0]
        desc = ExpandDesc(
            ctypes.sizeof(ExpandDesc), label.encode(), PRECISION[precision], bits,
            EXPAND_LAYOUT[layout], inner, columns, groups, columns // groups,
            packed.ptr, packed.nbytes, palette.ptr, palette.nbytes, target.ptr, target.nbytes)
        check(load().pk_palette_expand(self.handle, ctypes.byref(desc), stream))


class Event:
    def __init__(self, ctx: Context):
        self.ctx = ctx
        handle = ctypes.c_void_p()
        check(load().pk_event_create(ctx.handle, ctypes.byref(handle)))
        self.handle = handle.value

    def record(self, stream=None) -> None:
        check(load().pk_event_record(self.ctx.handle, self.handle, stream))

    def synchronize(self) -> None:
        check(load().pk_event_synchronize(self.ctx.handle, self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(load().pk_event_elapsed_ms(self.ctx.handle, self.handle, end.handle, ctypes.byref(ms)))
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            check(load().pk_event_destroy(self.ctx.handle, self.handle))
            self.handle = None


class PreparedWeight:
    def __init__(self, ctx: Context, bits: int, inner: int, columns: int, packed: DeviceArray,
                 label: str = "prepared-weight", stream=None):
        desc = WeightDesc(ctypes.sizeof(WeightDesc), label.encode(), bits, inner, columns,
                          packed.ptr, packed.nbytes)
        handle = ctypes.c_void_p()
        check(load().pk_prepared_weight_create(ctx.handle, ctypes.byref(desc), stream, ctypes.byref(handle)))
        self.handle = handle.value

    def nbytes(self) -> int:
        value = ctypes.c_uint64()
        check(load().pk_prepared_weight_bytes(self.handle, ctypes.byref(value)))
        return int(value.value)

    def destroy(self) -> None:
        if self.handle:
            check(load().pk_prepared_weight_destroy(self.handle))
            self.handle = None


class GemmOp:
    """One fused palette GEMM dispatch (pk_gemm_create ... pk_gemm_release)."""

    def __init__(self, ctx: Context, *, a: DeviceArray, packed: DeviceArray | None, palette: DeviceArray,
                 output: DeviceArray, bits: int, rows: int, inner: int, columns: int,
                 bias: DeviceArray | None = None, residual: DeviceArray | None = None,
                 residual_scale: float | None = None, activation: str = "none",
                 prepared: PreparedWeight | None = None, label: str = "palette-gemm",
                 production_only: bool = False, glu: bool = False, stream=None,
                 norm_gamma: DeviceArray | None = None, norm_beta: DeviceArray | None = None,
                 norm_epsilon: float = 0.0, cached_output: bool = False):
        """With norm_gamma / norm_beta (f32 [inner]) the op multiplies the
        row LayerNorm of `a` (PK_GEMM_ROW_NORM); cached_output keeps the
        output stores ordinary (PK_GEMM_CACHED_OUTPUT), which are otherwise
        non-temporal on the f16 pair-code kernels."""
        precision = "f16" if palette.dtype == np.float16 else "f32"
        groups = palette.shape[0]
        flags = ((REQUIRE_PRODUCTION_SIGNATURE if production_only else 0) | (GEMM_GLU if glu else 0) |
                 (GEMM_ROW_NORM if norm_gamma is not None else 0) | (GEMM_CACHED_OUTPUT if cached_output else 0))

        self.desc = GemmDesc(
            ctypes.sizeof(GemmDesc), flags,
            label.encode(), PRECISION[precision], bits, rows, inner, columns, groups,
            columns // groups if groups else 0,
            a.ptr, a.nbytes,
            packed.ptr if packed is not None else None, packed.nbytes if packed is not None else 0,
            palette.ptr, palette.nbytes, output.ptr, output.nbytes,
            bias.ptr if bias is not None else None, bias.nbytes if bias is not None else 0,
            residual.ptr if residual is not None else None, residual.nbytes if residual is not None else 0,
            int(residual_scale is not None), float(residual_scale or 0.0), ACTIVATION[activation],
            prepared.handle if prepared is not None else None,
            norm_gamma.ptr if norm_gamma is not None else None, norm_gamma.nbytes if norm_gamma is not None else 0,
            norm_beta.ptr if norm_beta is not None else None, norm_beta.nbytes if norm_beta is not None else 0,
            float(norm_epsilon))
        handle = ctypes.c_void_p()
        check(load().pk_gemm_create(ctx.handle, ctypes.byref(self.desc), stream, ctypes.byref(handle)))
        self.handle = handle.value
        self.ctx = ctx

    def enqueue(self, active_rows: int = 0, stream=None, start: "Event" = None, end: "Event" = None) -> None:
        """Launch; `start`/`end` events, when given, are stamped by the
        kernel's own dispatch (pk_gemm_enqueue_timed)."""
        if start is None and end is None:
            check(load().pk_gemm_enqueue(self.handle, active_rows, stream))
        else:
            check(load().pk_gemm_enqueue_timed(self.handle, active_rows, stream,
                                               start.handle if start else None, end.handle if end else None))

    def plan(self, active_rows: int = 0) -> PlanInfo:
        info = PlanInfo()
        check(load().pk_gemm_plan(self.handle, active_rows, ctypes.byref(info)))
        return info

    def set_variant(self, variant: int) -> None:
        check(load().pk_gemm_set_variant(self.handle, variant))

    def set_splits(self, splits: int) -> None:
        check(load().pk_gemm_set_splits(self.handle, splits))

    def prepare_rows(self, rows) -> None:
        """pk_gemm_prepare_rows: these active row counts run the plan of an op
        created for that many rows."""
        array = (ctypes.c_uint32 * len(rows))(*[int(r) for r in rows])
        check(load().pk_gemm_prepare_rows(self.handle, array, len(rows)))

    def destroy(self) -> None:
        check(load().pk_gemm_destroy(self.handle))

    def release(self) -> None:
        if self.handle:
            check(load().pk_gemm_release(self.handle))
            self.handle = None


class GemmGroup:
    """Independent f16 GEMM ops launched as one small-M kernel
    (pk_gemm_group_create ... pk_gemm_group_destroy). The group snapshots
    the ops' bindings and keeps their prepared weights alive."""

    def __init__(self, ctx: Context, ops, label: str = "palette-gemm-group"):
        self.ctx = ctx
        handles = (_VP * len(ops))(*[op.handle for op in ops])
        handle = ctypes.c_void_p()
        check(load().pk_gemm_group_create(ctx.handle, handles, len(ops), label.encode(), ctypes.byref(handle)))
        self.handle = handle.value

    def enqueue(self, active_rows: int = 0, stream=None, start: "Event" = None, end: "Event" = None) -> None:
        if start is None and end is None:
            check(load().pk_gemm_group_enqueue(self.handle, active_rows, stream))
        else:
            check(load().pk_gemm_group_enqueue_timed(self.handle, active_rows, stream,
                                                     start.handle if start else None, end.handle if end else None))

    def plan(self, active_rows: int = 0) -> PlanInfo:
        info = PlanInfo()
        check(load().pk_gemm_group_plan(self.handle, active_rows, ctypes.byref(info)))
        return info

    def set_variant(self, variant: int) -> None:
        """A small-M variant index, or -1 for the planned one."""
        check(load().pk_gemm_group_set_variant(self.handle, variant))

    def release(self) -> None:
        if self.handle:
            check(load().pk_gemm_group_destroy(self.handle))
            self.handle = None


def variant_count(precision: str) -> int:
    return int(load().pk_gemm_variant_count(PRECISION[precision]))


def describe_variant(precision: str, variant: int) -> VariantDesc:
    desc = VariantDesc()
    check(load().pk_gemm_variant_describe(PRECISION[precision], variant, ctypes.byref(desc)))
    return desc


def small_m_variants() -> list:
    """f16 variants a GemmGroup can run (the small-M kernels), by index."""
    return [v for v in range(variant_count("f16")) if describe_variant("f16", v).groupable]


def _slice(array):
    """(pointer, bytes) of a DeviceArray, or (None, 0)."""
    return (array.ptr, array.nbytes) if array is not None else (None, 0)


def conv_desc(*, pointwise_input, depthwise_weights, batch_norm_scale, batch_norm_shift, valid_lengths, output,
              batch_size: int, frames: int, channels: int = 0, precision: str | None = None,
              label: str = "conformer-conv", input_glu: bool = False) -> ConvDesc:
    """A pk_conv_desc over DeviceArrays (or any objects with ptr/nbytes);
    input_glu: the pointwise input is the [rows, C] GLU (PK_CONV_INPUT_GLU)."""
    if precision is None:
        precision = "f16" if pointwise_input.dtype == np.float16 else "f32"
    return ConvDesc(ctypes.sizeof(ConvDesc), CONV_INPUT_GLU if input_glu else 0, label.encode(),
                    PRECISION[precision], batch_size, frames, channels,
                    *_slice(pointwise_input), *_slice(depthwise_weights), *_slice(batch_norm_scale),
                    *_slice(batch_norm_shift), *_slice(valid_lengths), *_slice(output))


def plan_conformer_conv(batch_size: int, frames: int, precision: str = "f16", channels: int = 0) -> ConvPlanInfo:
    """planFusedConformerConv (conformer-conv.ts:72-115) through pk_conv_plan_shape."""
    info = ConvPlanInfo()
    check(load().pk_conv_plan_shape(PRECISION[precision], batch_size, frames, channels, ctypes.byref(info)))
    return info


class ConformerConvOp:
    """One fused GLU / depthwise k9 / folded BN / SiLU dispatch
    (FusedConformerConvKernel.createDispatch, conformer-conv.ts:255-344)."""

    def __init__(self, ctx: Context, **descriptor):
        self.desc = conv_desc(**descriptor)
        handle = ctypes.c_void_p()
        check(load().pk_conv_create(ctx.handle, ctypes.byref(self.desc), ctypes.byref(handle)))
        self.handle = handle.value
        self.ctx = ctx

    def enqueue(self, active_batch: int = 0, stream=None, start: "Event" = None, end: "Event" = None) -> None:
        if start is None and end is None:
            check(load().pk_conv_enqueue(self.handle, active_batch, stream))
        else:
            check(load().pk_conv_enqueue_timed(self.handle, active_batch, stream,
                                               start.handle if start else None, end.handle if end else None))

    def plan(self, active_batch: int = 0) -> ConvPlanInfo:
        info = ConvPlanInfo()
        check(load().pk_conv_plan(self.handle, active_batch, ctypes.byref(info)))
        return info

    def set_variant(self, variant: int) -> None:
        check(load().pk_conv_set_variant(self.handle, variant))

    def destroy(self) -> None:
        check(load().pk_conv_destroy(self.handle))

    def release(self) -> None:
        if self.handle:
            check(load().pk_conv_release(self.handle))
            self.handle = None


def conv_variant_count(precision: str) -> int:
    return int(load().pk_conv_variant_count(PRECISION[precision]))


def attention_desc(*, qkv, projected_positions, bias_u, bias_v, valid_lengths, output, batch_size: int, frames: int,
                   precision: str | None = None, label: str = "relative-attention",
                   positions_row_major: bool = False, plan_active: bool = False) -> AttentionDesc:
    """A pk_attention_desc over DeviceArrays (or any objects with ptr/nbytes)."""
    if precision is None:
        precision = "f16" if qkv.dtype == np.float16 else "f32"
    flags = (ATTENTION_POSITIONS_ROW_MAJOR if positions_row_major else 0) | (ATTENTION_PLAN_ACTIVE if plan_active else 0)
    return AttentionDesc(ctypes.sizeof(AttentionDesc), flags,
                         label.encode(), PRECISION[precision], batch_size, frames, *_slice(qkv),
                         *_slice(projected_positions), *_slice(bias_u), *_slice(bias_v), *_slice(valid_lengths),
                         *_slice(output))


class RelativeAttentionOp:
    """One relative-position attention dispatch
    (RelativeAttentionKernel.createDispatch, attention.ts:219-314)."""

    def __init__(self, ctx: Context, **descriptor):
        self.desc = attention_desc(**descriptor)
        handle = ctypes.c_void_p()
        check(load().pk_attention_create(ctx.handle, ctypes.byref(self.desc), ctypes.byref(handle)))
        self.handle = handle.value
        self.ctx = ctx

    def enqueue(self, active_batch: int = 0, stream=None, start: "Event" = None, end: "Event" = None) -> None:
        if start is None and end is None:
            check(load().pk_attention_enqueue(self.handle, active_batch, stream))
        else:
            check(load().pk_attention_enqueue_timed(self.handle, active_batch, stream,
                                                    start.handle if start else None, end.handle if end else None))

    def plan(self, active_batch: int = 0) -> AttentionPlanInfo:
        info = AttentionPlanInfo()
        check(load().pk_attention_plan(self.handle, active_batch, ctypes.byref(info)))
        return info

    def set_variant(self, variant: int) -> None:
        check(load().pk_attention_set_variant(self.handle, variant))

    def destroy(self) -> None:
        check(load().pk_attention_destroy(self.handle))

    def release(self) -> None:
        if self.handle:
            check(load().pk_attention_release(self.handle))
            self.handle = None


def attention_variant_count(precision: str) -> int:
    return int(load().pk_attention_variant_count(PRECISION[precision]))


def layernorm_desc(*, input, gamma, beta, output, rows: int, channels: int, epsilon: float | None = None,
                   precision: str | None = None, label: str = "layernorm", next_gamma=None, next_beta=None,
                   next_output=None) -> LayerNormDesc:
    """A pk_layernorm_desc; with next_gamma / next_beta / next_output the
    launch also writes the LayerNorm of its output (a chained LayerNorm)."""
    if precision is None:
        precision = "f16" if input.dtype == np.float16 else "f32"
    return LayerNormDesc(ctypes.sizeof(LayerNormDesc), label.encode(), PRECISION[precision], rows, channels,
                         *_slice(input), *_slice(gamma), *_slice(beta), *_slice(output), int(epsilon is not None),
                         float(epsilon or 0.0), *_slice(next_gamma), *_slice(next_beta), *_slice(next_output))


class LayerNormOp:
    """One LayerNorm dispatch (LayerNormKernel.createDispatch, layernorm.ts:165-240)."""

    def __init__(self, ctx: Context, **descriptor):
        self.desc = layernorm_desc(**descriptor)
        handle = ctypes.c_void_p()
        check(load().pk_layernorm_create(ctx.handle, ctypes.byref(self.desc), ctypes.byref(handle)))
        self.handle = handle.value

    def enqueue(self, active_rows: int = 0, stream=None, start: "Event" = None, end: "Event" = None) -> None:
        if start is None and end is None:
            check(load().pk_layernorm_enqueue(self.handle, active_rows, stream))
        else:
            check(load().pk_layernorm_enqueue_timed(self.handle, active_rows, stream,
                                                    start.handle if start else None, end.handle if end else None))

    def destroy(self) -> None:
        check(load().pk_layernorm_destroy(self.handle))

    def release(self) -> None:
        if self.handle:
            check(load().pk_layernorm_release(self.handle))
            self.handle = None


def subsampling_fused_desc(*, input, conv0_weights, conv0_bias, depthwise_weights, depthwise_bias, output,
                           valid_lengths, batch_size: int, input_height: int = 1501, input_width: int = 128,
                           channels: int = 256, valid_length_batch_offset: int = 0, precision: str | None = None,
                           label: str = "subsampling-fused-conv0-depthwise2") -> SubsamplingFusedDesc:
    if precision is None:
        precision = "f16" if conv0_weights.dtype == np.float16 else "f32"
    return SubsamplingFusedDesc(ctypes.sizeof(SubsamplingFusedDesc), label.encode(), PRECISION[precision], batch_size,
                                input_height, input_width, channels, *_slice(input), *_slice(conv0_weights),
                                *_slice(conv0_bias), *_slice(depthwise_weights), *_slice(depthwise_bias),
                                *_slice(output), *_slice(valid_lengths), valid_length_batch_offset)


def subsampling_depthwise_desc(*, input, weights, bias, output, valid_lengths, batch_size: int, input_height: int,
                               input_width: int, channels: int, steps: int, valid_length_batch_offset: int = 0,
                               precision: str | None = None,
                               label: str = "subsampling-depthwise") -> SubsamplingDepthwiseDesc:
    if precision is None:
        precision = "f16" if weights.dtype == np.float16 else "f32"
    return SubsamplingDepthwiseDesc(ctypes.sizeof(SubsamplingDepthwiseDesc), label.encode(), PRECISION[precision],
                                    batch_size, input_height, input_width, channels, *_slice(input),
                                    *_slice(weights), *_slice(bias), *_slice(output), *_slice(valid_lengths),
                                    valid_length_batch_offset, steps)


def subsampling_mask_desc(*, values, valid_lengths, batch_size: int, height: int, width: int, channels: int,
                          steps: int, valid_length_batch_offset: int = 0, precision: str | None = None,
                          label: str = "subsampling-time-mask") -> SubsamplingMaskDesc:
    if precision is None:
        precision = "f16" if values.dtype == np.float16 else "f32"
    return SubsamplingMaskDesc(ctypes.sizeof(SubsamplingMaskDesc), label.encode(), PRECISION[precision], batch_size,
                               height, width, channels, *_slice(values), *_slice(valid_lengths),
                               valid_length_batch_offset, steps)


class SubsamplingOp:
    """One subsampling convolution dispatch: kind "fused" (conv0 + ReLU +
    depthwise2), "depthwise" or "mask" (subsampling.ts createDispatch)."""

    _DESC = {"fused": (subsampling_fused_desc, "pk_subsampling_fused_create"),
             "depthwise": (subsampling_depthwise_desc, "pk_subsampling_depthwise_create"),
             "mask": (subsampling_mask_desc, "pk_subsampling_mask_create")}

    def __init__(self, ctx: Context, kind: str, **descriptor):
        make, create = self._DESC[kind]
        self.desc = make(**descriptor)
        handle = ctypes.c_void_p()
        check(getattr(load(), create)(ctx.handle, ctypes.byref(self.desc), ctypes.byref(handle)))
        self.handle = handle.value

    def enqueue(self, active_batch: int = 0, stream=None, start: "Event" = None, end: "Event" = None) -> None:
        if start is None and end is None:
            check(load().pk_subsampling_enqueue(self.handle, active_batch, stream))
        else:
            check(load().pk_subsampling_enqueue_timed(self.handle, active_batch, stream,
                                                      start.handle if start else None, end.handle if end else None))

    def plan(self, active_batch: int = 0) -> SubsamplingPlanInfo:
        info = SubsamplingPlanInfo()
        check(load().pk_subsampling_plan(self.handle, active_batch, ctypes.byref(info)))
        return info

    def destroy(self) -> None:
        check(load().pk_subsampling_destroy(self.handle))

    def release(self) -> None:
        if self.handle:
            check(load().pk_subsampling_release(self.handle))
            self.handle = None


_ENCODER_MATRICES = ("ff1_linear1", "ff1_linear2", "qkv", "o_proj", "pointwise1", "pointwise2", "ff2_linear1",
                     "ff2_linear2")
_ENCODER_VECTORS = ("projected_positions", "bias_u", "bias_v", "depthwise", "bn_scale", "bn_shift")


def _addr(x) -> int | None:
    """Device address of a DeviceArray, or an integer address as given."""
    return x.ptr if hasattr(x, "ptr") else x


def encoder_layer(weights: dict) -> EncoderLayer:
    """An EncoderLayer of device pointers from a dict keyed by the
    pk_encoder_layer field names (`norm_gamma` / `norm_beta` are lists of
    five; each matrix is a (packed, palette) pair), holding DeviceArrays or
    integer addresses."""
    layer = EncoderLayer()
    for i in range(5):
        layer.norm_gamma[i] = _addr(weights["norm_gamma"][i])
        layer.norm_beta[i] = _addr(weights["norm_beta"][i])
    for name in _ENCODER_MATRICES:
        packed, palette = weights[name]
        setattr(layer, name, EncoderMatrix(_addr(packed), _addr(palette)))
    for name in _ENCODER_VECTORS:
        setattr(layer, name, _addr(weights[name]))
    return layer


_SUBSAMPLING_MATRICES = ("pointwise3", "pointwise6", "linear")


def encoder_subsampling(weights: dict) -> EncoderSubsampling:
    """An EncoderSubsampling from a dict keyed by its field names (each
    matrix a (packed, palette) pair), holding DeviceArrays or addresses."""
    front = EncoderSubsampling()
    for name, _ in EncoderSubsampling._fields_:
        if name in _SUBSAMPLING_MATRICES:
            packed, palette = weights[name]
            setattr(front, name, EncoderMatrix(_addr(packed), _addr(palette)))
        else:
            setattr(front, name, _addr(weights[name]))
    return front


def encoder_desc(*, layers, valid_lengths, input, output, batch_size: int, frames: int, fused_glu: bool = True,
                 fused_norms: bool = False, unchained_norms: bool = False, prefix_same_plan: bool = False,
                 subsampling: dict | None = None,
                 feature_frames: int = 0, feature_lengths=None, projector=None, projector_bias=None,
                 projected_output=None, projected_channels: int = 0, label: str = "encoder",
                 precision: str = "f16") -> EncoderDesc:
    """An EncoderDesc over `layers` (dicts as encoder_layer takes), with the
    optional front end (`subsampling` dict, feature frames and lengths) and
    projector ((packed, palette) pair, bias, output); the returned structure
    keeps what it points to alive. `precision` "f32" is the reference's fp32
    profile: activations, palettes, positions and depthwise weights in f32
    (the GLU then stays in the convolution)."""
    array = (EncoderLayer * len(layers))(*[encoder_layer(w) for w in layers])
    front = encoder_subsampling(subsampling) if subsampling is not None else None
    flags = ((0 if fused_glu else ENCODER_SEPARATE_GLU) | (ENCODER_FUSED_NORMS if fused_norms else 0) |
             (ENCODER_UNCHAINED_NORMS if unchained_norms else 0) |
             (ENCODER_PREFIX_SAME_PLAN if prefix_same_plan else 0))
    desc = EncoderDesc(ctypes.sizeof(EncoderDesc), flags, label.encode(),
                       PRECISION[precision], batch_size, frames, len(layers),
                       ctypes.cast(array, ctypes.POINTER(EncoderLayer)), _addr(valid_lengths), _addr(input),
                       _addr(output), ctypes.pointer(front) if front is not None else None, feature_frames,
                       _addr(feature_lengths) if feature_lengths is not None else None,
                       EncoderMatrix(*(_addr(x) for x in projector)) if projector is not None else EncoderMatrix(),
                       _addr(projector_bias) if projector_bias is not None else None, projected_channels,
                       _addr(projected_output) if projected_output is not None else None)
    desc._keep = (array, front)
    return desc


class EncoderOp:
    """The encoder layer stack (createEncoderLayerDispatches, encoder.ts:1868-2135)
    over device tensors."""

    def __init__(self, ctx: Context, stream=None, **descriptor):
        self.desc = encoder_desc(**descriptor)
        handle = ctypes.c_void_p()
        check(load().pk_encoder_create(ctx.handle, ctypes.byref(self.desc), stream, ctypes.byref(handle)))
        self.handle = handle.value

    def enqueue(self, active_batch: int = 0, stream=None, graph: bool = False) -> None:
        check(load().pk_encoder_enqueue(self.handle, active_batch, stream, int(graph)))

    def enqueue_profiled(self, starts, ends, active_batch: int = 0, stream=None) -> None:
        """One eager pass whose launch i stamps starts[i] / ends[i] (Events,
        or None for a launch that stamps nothing); both lists hold one entry
        per launch of the pass."""
        launches = self.info()[0]
        if len(starts) != launches or len(ends) != launches:
            raise ValueError(f"a profiled pass takes {launches} start and end events")
        start_array = (ctypes.c_void_p * len(starts))(*[ev.handle if ev is not None else None for ev in starts])
        end_array = (ctypes.c_void_p * len(ends))(*[ev.handle if ev is not None else None for ev in ends])
        check(load().pk_encoder_enqueue_profiled(self.handle, active_batch, stream, start_array, end_array))

    def info(self) -> tuple[int, int]:
        launches, device_bytes = ctypes.c_uint32(), ctypes.c_uint64()
        check(load().pk_encoder_info(self.handle, ctypes.byref(launches), ctypes.byref(device_bytes)))
        return launches.value, device_bytes.value

    def release(self) -> None:
        if self.handle:
            check(load().pk_encoder_destroy(self.handle))
            self.handle = None


TDT_WEIGHT_NAMES = ("embedding", "lstm_weight_l0", "lstm_weight_l1", "lstm_bias_l0", "lstm_bias_l1",
                    "projector_weight", "projector_bias", "head_weight", "head_bias")


def tdt_desc(*, weights: dict, encoder_projected, encoded_lengths, decode_starts, decode_ends, flush_finals, state,
             predictor_scratch, tokens, token_frames, token_durations, metadata, batch_size: int, frames: int,
             max_tokens: int, label: str = "parakeet-persistent-tdt-decode", precision: str = "f16") -> TdtDesc:
    """A TdtDesc from device slices (DeviceArrays, or (address, bytes) pairs);
    `weights` is keyed by TDT_WEIGHT_NAMES; `precision` "f16" or "f32" is the
    execution profile (weights and encoder rows in that element)."""
    def sl(x):
        return tuple(x) if isinstance(x, tuple) else _slice(x)
    w = {k: sl(weights[k]) for k in TDT_WEIGHT_NAMES}
    tw = TdtWeights(*w["embedding"], (ctypes.c_void_p * 2)(w["lstm_weight_l0"][0], w["lstm_weight_l1"][0]),
                    (ctypes.c_uint64 * 2)(w["lstm_weight_l0"][1], w["lstm_weight_l1"][1]),
                    (ctypes.c_void_p * 2)(w["lstm_bias_l0"][0], w["lstm_bias_l1"][0]),
                    (ctypes.c_uint64 * 2)(w["lstm_bias_l0"][1], w["lstm_bias_l1"][1]),
                    *w["projector_weight"], *w["projector_bias"], *w["head_weight"], *w["head_bias"])
    fields = []
    for x in (encoder_projected, encoded_lengths, decode_starts, decode_ends, flush_finals, state, predictor_scratch,
              tokens, token_frames, token_durations, metadata):
        fields += list(sl(x))
    return TdtDesc(ctypes.sizeof(TdtDesc), label.encode(), PRECISION[precision], batch_size, frames, max_tokens, tw,
                   *fields)


TDT_STATIC_MAX_WINDOWS = 64  # PK_TDT_STATIC_MAX_WINDOWS
TDT_OVERFLOW = 1       # PK_TDT_OVERFLOW: more tokens than max_tokens (tdt-decoder.ts:1756-1775)
TDT_SYNC_TIMEOUT = 2   # PK_TDT_SYNC_TIMEOUT: a team barrier gave up waiting (no reference counterpart)


def decode_tdt_status(status) -> dict:
    """Counts of the decoder's per-window status words by cause: windows
    whose tokens overflowed max_tokens, windows whose team barrier timed out
    (their outputs are incomplete and must be decoded again), and windows
    with bits this library does not define."""
    words = np.asarray(status, dtype=np.uint32).reshape(-1)
    known = TDT_OVERFLOW | TDT_SYNC_TIMEOUT
    return {"overflow_windows": int(((words & TDT_OVERFLOW) != 0).sum()),
            "sync_timeout_windows": int(((words & TDT_SYNC_TIMEOUT) != 0).sum()),
            "unknown_status_windows": int(((words & ~np.uint32(known)) != 0).sum())}


def tdt_decode_static(ctx: Context, members: int = 0, stream=None, **descriptor) -> None:
    """pk_tdt_decode_static: the whole decode of a descriptor with no op and
    no allocation (the team buffers are the library's static array)."""
    desc = tdt_desc(**descriptor)
    check(load().pk_tdt_decode_static(ctx.handle, ctypes.byref(desc), members, stream))


class TdtDecoderOp:
    """The greedy TDT decoder (PersistentTdtDecoderKernel.createDispatch,
    tdt-decoder.ts:294-366)."""

    def __init__(self, ctx: Context, **descriptor):
        self.desc = tdt_desc(**descriptor)
        handle = ctypes.c_void_p()
        check(load().pk_tdt_create(ctx.handle, ctypes.byref(self.desc), ctypes.byref(handle)))
        self.handle = handle.value

    def enqueue(self, active_batch: int = 0, stream=None, start: "Event" = None, end: "Event" = None) -> None:
        if start is None and end is None:
            check(load().pk_tdt_enqueue(self.handle, active_batch, stream))
        else:
            check(load().pk_tdt_enqueue_timed(self.handle, active_batch, stream,
                                              start.handle if start else None, end.handle if end else None))

    def set_team_size(self, members: int) -> None:
        """0 chooses, 1 runs one workgroup per window, 8 / 16 split each window over a team."""
        check(load().pk_tdt_set_team_size(self.handle, members))

    def team_size(self) -> int:
        out = ctypes.c_uint32()
        check(load().pk_tdt_team_size(self.handle, ctypes.byref(out)))
        return out.value

    def destroy(self) -> None:
        check(load().pk_tdt_destroy(self.handle))

    def release(self) -> None:
        if self.handle:
            check(load().pk_tdt_release(self.handle))
            self.handle = None


class Graph:
    """pk_graph: the enqueues made on `stream` inside `with Graph.capture(ctx, stream) as g:`,
    replayed by g.launch()."""

    def __init__(self, ctx: "Context", stream=None):
        self.ctx, self.stream, self.handle = ctx, stream, None

    @classmethod
    def capture(cls, ctx: "Context", stream=None) -> "Graph":
        return cls(ctx, stream)

    def __enter__(self) -> "Graph":
        check(load().pk_graph_begin_capture(self.ctx.handle, self.stream))
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        handle = ctypes.c_void_p()
        status = load().pk_graph_end_capture(self.ctx.handle, self.stream, ctypes.byref(handle))
        if exc_type is None:
            check(status)
            self.handle = handle.value

    def launch(self, stream=None) -> None:
        check(load().pk_graph_launch(self.handle, self.stream if stream is None else stream))

    def release(self) -> None:
        if self.handle:
            load().pk_graph_destroy(self.handle)
            self.handle = None


def plan_tdt_execution(batch_size: int) -> TdtExecutionPlan:
    plan = TdtExecutionPlan()
    check(load().pk_tdt_plan_execution(batch_size, ctypes.byref(plan)))
    return plan

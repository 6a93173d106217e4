"""ctypes wrapper around liboracle.so, the CPU restatement of parakeet.wgsl's
palette-weight GEMM path.

TEST INFRASTRUCTURE ONLY. Imported by tests/, by the smoke check in
__graft_entry__.py and by the CPU-baseline leg of bench.py, as the checker.
The product library never loads it.

Reference functions restated (see pk_oracle.h for the pins):
  pack_codes      model/convert.py:2130-2156
  unpack_codes    src/model/palette-expander.ts:500-511, model/tests/test_convert.py:90-115
  palette_group   src/model/palette-expander.ts:543-549
  tile_major_index src/model/runtime-plan.ts:454-490
  expand          src/model/palette-expander.ts:478-587
  gemm            src/webgpu/kernels/gemm.ts:1362-1716, :2006-2044 (f16),
                  :2356-2599, :2847-2869 (f32)
  conformer_conv  src/webgpu/kernels/conformer-conv.ts:495-573
  glu             the GLU step of conformer-conv.ts:520-535
  layernorm       src/webgpu/kernels/layernorm.ts:309-390
  relative_attention  src/webgpu/kernels/attention.ts:418-727
  subsampled_length       src/webgpu/kernels/subsampling.ts:119-135
  subsampling_fused       subsampling.ts:1092-1239 (conv0 + ReLU + depthwise2)
  subsampling_depthwise   subsampling.ts:1241-1330
  subsampling_mask        subsampling.ts:1332-1430
  encoder_layer   the dispatch order of src/webgpu/encoder.ts:1868-2135,
                  composed from the functions above
  tdt_decode / tdt_predictor / tdt_joint  src/webgpu/kernels/tdt-decoder.ts:1133-2010
  exp_f32 / tanh_f32   the decoder's transcendental functions
  encoder_front_end  createSubsamplingCommands, encoder.ts:2140-2400
  encoder_graph   ParakeetEncoderGraph.encode, encoder.ts:1690-1706 (front
                  end, layers, projector)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

ACT = {"none": 0, "silu": 1, "relu": 2}
MODE = {"f32-chain": 0, "f16-chain": 1, "f64": 2}
DTYPE = {"f16": 0, "f32": 1, "f64": 2}


def build() -> None:
    """Compile liboracle.so from pk_oracle.c with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liboracle.so"], check=True)


class _GemmArgs(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_uint32),
        ("inner", ctypes.c_uint32),
        ("columns", ctypes.c_uint32),
        ("bits", ctypes.c_int32),
        ("palette_groups", ctypes.c_uint32),
        ("palette_group_columns", ctypes.c_uint32),
        ("dtype", ctypes.c_int32),
        ("packed", ctypes.c_void_p),
        ("palette", ctypes.c_void_p),
        ("a", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("residual", ctypes.c_void_p),
        ("residual_scale", ctypes.c_float),
        ("activation", ctypes.c_int32),
        ("out", ctypes.c_void_p),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.pko_f64_to_f16.restype = ctypes.c_uint16
        _lib.pko_f64_to_f16.argtypes = [ctypes.c_double]
        _lib.pko_f16_to_f64.restype = ctypes.c_double
        _lib.pko_f16_to_f64.argtypes = [ctypes.c_uint16]
        _lib.pko_subsampled_length.restype = ctypes.c_uint32
        _lib.pko_subsampled_length.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        _lib.pko_round_f16.restype = ctypes.c_double
        _lib.pko_round_f16.argtypes = [ctypes.c_double]
        _lib.pko_pack_codes.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
        _lib.pko_unpack_codes.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
        _lib.pko_palette_group.restype = ctypes.c_uint32
        _lib.pko_palette_group.argtypes = [ctypes.c_uint32] * 3
        _lib.pko_tile_major_index.restype = ctypes.c_uint64
        _lib.pko_tile_major_index.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        _lib.pko_expand.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
            ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
            ctypes.c_void_p, ctypes.c_void_p,
        ]
        _lib.pko_gemm.argtypes = [ctypes.POINTER(_GemmArgs), ctypes.c_int, ctypes.c_int]
        _lib.pko_conformer_conv.argtypes = [ctypes.c_int, ctypes.c_int] + [ctypes.c_uint32] * 3 + [ctypes.c_void_p] * 6
        _lib.pko_relative_attention.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32] + \
            [ctypes.c_void_p] * 6
        _lib.pko_layernorm.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint32] + \
            [ctypes.c_void_p] * 3 + [ctypes.c_float, ctypes.c_void_p]
        _lib.pko_glu.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_void_p,
                                 ctypes.c_void_p]
        _lib.pko_exp_f32.restype = ctypes.c_float
        _lib.pko_exp_f32.argtypes = [ctypes.c_float]
        _lib.pko_tanh_f32.restype = ctypes.c_float
        _lib.pko_tanh_f32.argtypes = [ctypes.c_float]
        _lib.pko_tdt_decode.argtypes = [ctypes.POINTER(_TdtWeights)] + [ctypes.c_uint32] * 3 + [ctypes.c_void_p] * 12
        _lib.pko_tdt_predictor.argtypes = [ctypes.POINTER(_TdtWeights), ctypes.c_uint32, ctypes.c_int,
                                           ctypes.c_void_p, ctypes.c_void_p]
        _lib.pko_tdt_joint.argtypes = [ctypes.POINTER(_TdtWeights)] + [ctypes.c_void_p] * 5
        _lib.pko_subsampling_fused.argtypes = [ctypes.c_int] + [ctypes.c_uint32] * 4 + [ctypes.c_void_p] * 7
        _lib.pko_subsampling_depthwise.argtypes = [ctypes.c_int] + [ctypes.c_uint32] * 4 + [ctypes.c_void_p] * 4 + \
            [ctypes.c_uint32, ctypes.c_void_p]
        _lib.pko_subsampling_mask.argtypes = [ctypes.c_int] + [ctypes.c_uint32] * 4 + [ctypes.c_void_p] * 2 + \
            [ctypes.c_uint32]
    return _lib


def _ptr(array: np.ndarray | None) -> int | None:
    if array is None:
        return None
    assert array.flags["C_CONTIGUOUS"]
    return array.ctypes.data


def codes_per_group(bits: int) -> int:
    return {5: 32, 6: 16}[bits]


def words_per_group(bits: int) -> int:
    return {5: 5, 6: 3}[bits]


def f64_to_f16_bits(value: float) -> int:
    return int(lib().pko_f64_to_f16(float(value)))


def round_f16(value: float) -> float:
    return float(lib().pko_round_f16(float(value)))


def f16_bits_to_f64(bits: int) -> float:
    return float(lib().pko_f16_to_f64(int(bits)))


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1)
    cpg = codes_per_group(bits)
    if codes.size % cpg:
        raise ValueError("code count is not group aligned")
    words = np.zeros((codes.size // cpg, words_per_group(bits)), dtype="<u4")
    if lib().pko_pack_codes(bits, _ptr(codes), codes.size, _ptr(words)):
        raise ValueError("pack_codes rejected its input")
    return words


def unpack_codes(words: np.ndarray, bits: int) -> np.ndarray:
    words = np.ascontiguousarray(words, dtype="<u4").reshape(-1)
    wpg = words_per_group(bits)
    groups = words.size // wpg
    codes = np.empty(groups * codes_per_group(bits), dtype=np.uint8)
    if lib().pko_unpack_codes(bits, _ptr(words), groups, _ptr(codes)):
        raise ValueError("unpack_codes rejected its input")
    return codes


def palette_group(column: int, group_columns: int, groups: int) -> int:
    return int(lib().pko_palette_group(column, group_columns, groups))


def tile_major_index(scalar: int, inner: int, columns: int, tile_columns: int) -> int:
    return int(lib().pko_tile_major_index(scalar, inner, columns, tile_columns))


def expand(words, bits, inner, columns, palette, *, tile_major=False) -> np.ndarray:
    """Dense [K, N] weights (or the tile-major scratch) from packed codes."""
    palette = np.ascontiguousarray(palette)
    dtype = "f16" if palette.dtype == np.float16 else "f32"
    groups = palette.shape[0]
    out = np.empty(inner * columns, dtype=palette.dtype)
    words = np.ascontiguousarray(words, dtype="<u4")
    rc = lib().pko_expand(bits, DTYPE[dtype], int(tile_major), _ptr(words), inner, columns,
                          columns // groups, groups, _ptr(palette), _ptr(out))
    if rc:
        raise ValueError("expand rejected its geometry")
    return out if tile_major else out.reshape(inner, columns)


def gemm(a, words, bits, palette, columns, *, bias=None, residual=None,
         residual_scale=None, activation="none", mode=None, threads=1) -> np.ndarray:
    """Palette GEMM with the reference epilogue.

    a: [M, K] float16 or float32; palette: [G, 2^bits] of the same dtype.
    mode: "f16-chain" (reference fp16 semantics), "f32-chain" (reference fp32
    semantics) or "f64" (double truth). Returns float16/float32 for the chain
    modes and float64 for "f64".
    """
    a = np.ascontiguousarray(a)
    palette = np.ascontiguousarray(palette)
    dtype = "f16" if a.dtype == np.float16 else "f32"
    if palette.dtype != a.dtype:
        raise ValueError("palette dtype must match the activation dtype")
    if mode is None:
        mode = "f16-chain" if dtype == "f16" else "f32-chain"
    rows, inner = a.shape
    groups = palette.shape[0]
    if mode == "f64":
        out = np.empty((rows, columns), dtype=np.float64)
    else:
        out = np.empty((rows, columns), dtype=a.dtype)
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float32)
    if residual is not None:
        residual = np.ascontiguousarray(residual, dtype=a.dtype)
        if residual_scale is None:
            residual_scale = 1.0
    words = np.ascontiguousarray(words, dtype="<u4")
    args = _GemmArgs(
        rows, inner, columns, bits, groups, columns // groups, DTYPE[dtype],
        _ptr(words), _ptr(palette), _ptr(a), _ptr(bias), _ptr(residual),
        float(residual_scale if residual_scale is not None else 0.0), ACT[activation], _ptr(out),
    )
    if lib().pko_gemm(ctypes.byref(args), MODE[mode], int(threads)):
        raise ValueError("gemm rejected its arguments")
    return out


def conformer_conv(pointwise, weights, scale, shift, valid, *, batch, frames, mode="f32-chain") -> np.ndarray:
    """Conformer convolution tail (conformer-conv.ts:495-573): GLU of the
    pointwise-1 output [batch*frames, 2C], depthwise k9 over frames (zero
    outside [0, frames) and past each valid length), folded batch norm, SiLU.
    mode "f32-chain" (reference arithmetic) or "f64"; the output has the
    input's dtype (float16, float32, or float64 for truth chains)."""
    pointwise = np.ascontiguousarray(pointwise)
    weights = np.ascontiguousarray(weights, dtype=pointwise.dtype)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    shift = np.ascontiguousarray(shift, dtype=np.float32)
    valid = np.ascontiguousarray(valid, dtype=np.uint32)
    channels = pointwise.shape[1] // 2
    if pointwise.shape != (batch * frames, 2 * channels) or weights.shape != (9, channels):
        raise ValueError("conformer_conv shape mismatch")
    out = np.empty((batch * frames, channels), dtype=pointwise.dtype)
    names = {np.dtype(np.float16): "f16", np.dtype(np.float32): "f32", np.dtype(np.float64): "f64"}
    if pointwise.dtype not in names:
        raise ValueError(f"conformer_conv takes float16/32/64 input, not {pointwise.dtype}")
    dtype = DTYPE[names[pointwise.dtype]]
    if lib().pko_conformer_conv(dtype, MODE[mode], batch, frames, channels, _ptr(pointwise), _ptr(weights),
                                _ptr(scale), _ptr(shift), _ptr(valid), _ptr(out)):
        raise ValueError("conformer_conv rejected its arguments")
    return out


def relative_attention(qkv, positions, bias_u, bias_v, valid, *, batch, frames, mode="f32-chain") -> np.ndarray:
    """Relative-position attention (attention.ts:418-727): qkv [B*T, 3072],
    positions in head-vector-position-vec4 order [8, 32, 2T-1, 4], biases
    [8, 128] f32, valid [B]; returns [B*T, 1024] in the input's dtype."""
    qkv = np.ascontiguousarray(qkv)
    names = {np.dtype(np.float16): "f16", np.dtype(np.float32): "f32", np.dtype(np.float64): "f64"}
    if qkv.dtype not in names:
        raise ValueError(f"relative_attention takes float16/32/64, not {qkv.dtype}")
    positions = np.ascontiguousarray(positions, dtype=qkv.dtype)
    bias_u = np.ascontiguousarray(bias_u, dtype=np.float32)
    bias_v = np.ascontiguousarray(bias_v, dtype=np.float32)
    valid = np.ascontiguousarray(valid, dtype=np.uint32)
    if qkv.shape != (batch * frames, 3072) or positions.size != 8 * 128 * (2 * frames - 1) or \
            bias_u.size != 1024 or bias_v.size != 1024 or valid.size != batch:
        raise ValueError("relative_attention shape mismatch")
    out = np.empty((batch * frames, 1024), dtype=qkv.dtype)
    if lib().pko_relative_attention(DTYPE[names[qkv.dtype]], MODE[mode], batch, frames, _ptr(qkv), _ptr(positions),
                                    _ptr(bias_u), _ptr(bias_v), _ptr(valid), _ptr(out)):
        raise ValueError("relative_attention rejected its arguments")
    return out


def layernorm(x, gamma, beta, *, epsilon=1e-5, mode="f32-chain") -> np.ndarray:
    """LayerNorm over the last axis of a [rows, C] array (layernorm.ts:309-390)."""
    x = np.ascontiguousarray(x)
    names = {np.dtype(np.float16): "f16", np.dtype(np.float32): "f32", np.dtype(np.float64): "f64"}
    if x.dtype not in names or x.ndim != 2:
        raise ValueError("layernorm takes a [rows, C] float16/32/64 array")
    gamma = np.ascontiguousarray(gamma, dtype=np.float32)
    beta = np.ascontiguousarray(beta, dtype=np.float32)
    out = np.empty_like(x)
    if lib().pko_layernorm(DTYPE[names[x.dtype]], MODE[mode], x.shape[0], x.shape[1], _ptr(x), _ptr(gamma),
                           _ptr(beta), float(epsilon), _ptr(out)):
        raise ValueError("layernorm rejected its arguments")
    return out


def glu(pointwise, mode="f32-chain") -> np.ndarray:
    """value * sigmoid(gate) of a [rows, 2C] input (values, then gates), with
    the reference's gate clamp; output [rows, C] in the input's dtype."""
    pointwise = np.ascontiguousarray(pointwise)
    names = {np.dtype(np.float16): "f16", np.dtype(np.float32): "f32", np.dtype(np.float64): "f64"}
    if pointwise.dtype not in names or pointwise.ndim != 2 or pointwise.shape[1] % 2:
        raise ValueError("glu takes a [rows, 2C] float16/32/64 array")
    rows, channels = pointwise.shape[0], pointwise.shape[1] // 2
    out = np.empty((rows, channels), dtype=pointwise.dtype)
    if lib().pko_glu(DTYPE[names[pointwise.dtype]], MODE[mode], rows, channels, _ptr(pointwise), _ptr(out)):
        raise ValueError("glu rejected its arguments")
    return out


_NAMES = {np.dtype(np.float16): "f16", np.dtype(np.float32): "f32", np.dtype(np.float64): "f64"}


def subsampled_length(length: int, steps: int) -> int:
    """Frames left after `steps` same-padded stride-2 convolutions."""
    return int(lib().pko_subsampled_length(int(length), int(steps)))


def subsampling_fused(features, conv0_weights, conv0_bias, depthwise_weights, depthwise_bias, valid,
                      *, dtype=np.float16) -> np.ndarray:
    """conv0 (1 -> C, 3x3, stride 2, ReLU) then depthwise2 (3x3, stride 2)
    of f32 feature-major features [batch, width(bins), height(frames)];
    weights [3, 3, C] and the output [batch, Ho, Wo, C] in `dtype` (float16
    and float32 follow the reference profiles, float64 is the double twin)."""
    features = np.ascontiguousarray(features, dtype=np.float32)
    batch, width, height = features.shape
    channels = conv0_weights.shape[-1]
    dtype = np.dtype(dtype)
    conv0_weights = np.ascontiguousarray(conv0_weights, dtype=dtype).reshape(3, 3, channels)
    depthwise_weights = np.ascontiguousarray(depthwise_weights, dtype=dtype).reshape(3, 3, channels)
    conv0_bias = np.ascontiguousarray(conv0_bias, dtype=np.float32)
    depthwise_bias = np.ascontiguousarray(depthwise_bias, dtype=np.float32)
    valid = np.ascontiguousarray(valid, dtype=np.uint32)
    h1, w1 = subsampled_length(height, 1), subsampled_length(width, 1)
    out = np.empty((batch, subsampled_length(h1, 1), subsampled_length(w1, 1), channels), dtype=dtype)
    if valid.size != batch or conv0_bias.size != channels or depthwise_bias.size != channels:
        raise ValueError("subsampling_fused shape mismatch")
    if lib().pko_subsampling_fused(DTYPE[_NAMES[dtype]], batch, height, width, channels, _ptr(features),
                                   _ptr(conv0_weights), _ptr(conv0_bias), _ptr(depthwise_weights),
                                   _ptr(depthwise_bias), _ptr(valid), _ptr(out)):
        raise ValueError("subsampling_fused rejected its arguments")
    return out


def subsampling_depthwise(x, weights, bias, valid, steps) -> np.ndarray:
    """Channel-last depthwise 3x3 stride-2 convolution of x [batch, H, W, C]
    (float16/32/64) with the valid-length masking of stage `steps`."""
    x = np.ascontiguousarray(x)
    batch, height, width, channels = x.shape
    weights = np.ascontiguousarray(weights, dtype=x.dtype).reshape(3, 3, channels)
    bias = np.ascontiguousarray(bias, dtype=np.float32)
    valid = np.ascontiguousarray(valid, dtype=np.uint32)
    out = np.empty((batch, subsampled_length(height, 1), subsampled_length(width, 1), channels), dtype=x.dtype)
    if lib().pko_subsampling_depthwise(DTYPE[_NAMES[x.dtype]], batch, height, width, channels, _ptr(x),
                                       _ptr(weights), _ptr(bias), _ptr(valid), int(steps), _ptr(out)):
        raise ValueError("subsampling_depthwise rejected its arguments")
    return out


def subsampling_mask(x, valid, steps) -> np.ndarray:
    """A copy of x [batch, H, W, C] with rows at or past sub(L, steps) zeroed."""
    out = np.array(x, copy=True, order="C")
    batch, height, width, channels = out.shape
    valid = np.ascontiguousarray(valid, dtype=np.uint32)
    if lib().pko_subsampling_mask(DTYPE[_NAMES[out.dtype]], batch, height, width, channels, _ptr(out), _ptr(valid),
                                  int(steps)):
        raise ValueError("subsampling_mask rejected its arguments")
    return out


# name -> (bits, palette groups) of an encoder layer's matrices
# (model/convert.py:1360-1475, encoder.ts:2458-2512).
ENCODER_BITS = {"ff1_linear1": 5, "ff1_linear2": 5, "qkv": 5, "o_proj": 6, "pointwise1": 5, "pointwise2": 5,
                "ff2_linear1": 5, "ff2_linear2": 5}


def _chain(dtype, gemm_mode):
    """The storage dtype and GEMM mode of an encoder chain: f16 storage with
    the reference's f16 GEMM arithmetic by default, f32 storage (the
    reference's fp32 profile, encoder.ts:947-1165) with its f32 chain."""
    dtype = np.dtype(dtype)
    if dtype not in (np.dtype(np.float16), np.dtype(np.float32)):
        raise ValueError("the encoder chain stores float16 or float32")
    if gemm_mode is None:
        gemm_mode = "f16-chain" if dtype == np.float16 else "f32-chain"
    return dtype, gemm_mode


def encoder_layer(x, layer, valid, *, batch, frames, gemm_mode=None, threads=8, dtype=np.float16) -> np.ndarray:
    """One FastConformer layer over f16 features x [batch*frames, 1024], in
    the order of createEncoderLayerDispatches (encoder.ts:1868-2135):
      x1 = x + 0.5 FF1(LN(x)),  FF(h) = SiLU(h W1) W2
      x2 = x1 + attention(LN(x1) Wqkv) Wo
      x3 = x2 + SiLU(BN(DW9(GLU(LN(x2) PW1)))) PW2
      x4 = x3 + 0.5 FF2(LN(x3));  out = LN(x4)
    Every intermediate is stored in `dtype` (f16 by default, f32 for the
    reference's fp32 profile) like the reference's arena. `layer` is keyed
    like pk_encoder_layer (norm_gamma / norm_beta [5, 1024], each matrix a
    (packed words, palette) pair; palettes, positions and depthwise weights
    are taken in `dtype`). gemm_mode "f16-chain" is the reference's fp16 GEMM
    arithmetic, "f32-chain" its fp32 one (the defaults), "f64" the exact sum
    rounded once."""
    dtype, gemm_mode = _chain(dtype, gemm_mode)
    x = np.ascontiguousarray(x, dtype=dtype)

    def norm(i, h):
        return layernorm(h, layer["norm_gamma"][i], layer["norm_beta"][i])

    def mm(name, a, columns, **epilogue):
        words, palette = layer[name]
        out = gemm(a, words, ENCODER_BITS[name], np.asarray(palette, dtype=dtype), columns, mode=gemm_mode,
                   threads=threads, **epilogue)
        return out.astype(dtype)

    hidden = mm("ff1_linear1", norm(0, x), 4096, activation="silu")
    x1 = mm("ff1_linear2", hidden, 1024, residual=x, residual_scale=0.5)
    qkv = mm("qkv", norm(1, x1), 3072)
    context = relative_attention(qkv, layer["projected_positions"], layer["bias_u"], layer["bias_v"], valid,
                                 batch=batch, frames=frames)
    x2 = mm("o_proj", context, 1024, residual=x1, residual_scale=1.0)
    pointwise = mm("pointwise1", norm(2, x2), 2048)
    conv = conformer_conv(pointwise, layer["depthwise"], layer["bn_scale"], layer["bn_shift"], valid,
                          batch=batch, frames=frames)
    x3 = mm("pointwise2", conv, 1024, residual=x2, residual_scale=1.0)
    hidden = mm("ff2_linear1", norm(3, x3), 4096, activation="silu")
    x4 = mm("ff2_linear2", hidden, 1024, residual=x3, residual_scale=0.5)
    return norm(4, x4)


def encoder(x, layers, valid, *, batch, frames, gemm_mode=None, threads=8, dtype=np.float16) -> np.ndarray:
    """The layer stack: encoder_layer applied for each entry of `layers`."""
    for layer in layers:
        x = encoder_layer(x, layer, valid, batch=batch, frames=frames, gemm_mode=gemm_mode, threads=threads,
                          dtype=dtype)
    return x


TDT_HIDDEN, TDT_GATES, TDT_HEAD, TDT_BLANK = 640, 2560, 1032, 1024


class _TdtWeights(ctypes.Structure):
    _fields_ = [("embedding", ctypes.c_void_p), ("lstm_weight", ctypes.c_void_p * 2),
                ("lstm_bias", ctypes.c_void_p * 2), ("projector_weight", ctypes.c_void_p),
                ("projector_bias", ctypes.c_void_p), ("head_weight", ctypes.c_void_p), ("head_bias", ctypes.c_void_p),
                ("f32", ctypes.c_int32)]


def _tdt_weights(weights: dict):
    """(struct, keep-alive list, element dtype) from a dict keyed like the
    decoder package: embedding [1025, 640], lstm_weight_l0/_l1 [1280, 2560],
    lstm_bias_l0/_l1 f32 [2560], projector_weight [640, 640], projector_bias
    f32 [640], head_weight [640, 1032], head_bias f32 [1032]. The weights are
    all f16 (the f16 profile) or all f32 (the f32 profile), which the
    embedding's dtype selects (tdt-decoder.ts:196-218, :378-405)."""
    keep = {k: np.ascontiguousarray(v) for k, v in weights.items()}
    wt = np.float32 if keep["embedding"].dtype == np.float32 else np.float16
    expect = {"embedding": (wt, (1025, 640)), "lstm_weight_l0": (wt, (1280, 2560)),
              "lstm_weight_l1": (wt, (1280, 2560)), "lstm_bias_l0": (np.float32, (2560,)),
              "lstm_bias_l1": (np.float32, (2560,)), "projector_weight": (wt, (640, 640)),
              "projector_bias": (np.float32, (640,)), "head_weight": (wt, (640, 1032)),
              "head_bias": (np.float32, (1032,))}
    for name, (dtype, shape) in expect.items():
        if keep[name].dtype != dtype or keep[name].shape != shape:
            raise ValueError(f"decoder tensor {name} must be {np.dtype(dtype).name} {shape}")
    w = _TdtWeights(_ptr(keep["embedding"]), (ctypes.c_void_p * 2)(_ptr(keep["lstm_weight_l0"]),
                                                                    _ptr(keep["lstm_weight_l1"])),
                    (ctypes.c_void_p * 2)(_ptr(keep["lstm_bias_l0"]), _ptr(keep["lstm_bias_l1"])),
                    _ptr(keep["projector_weight"]), _ptr(keep["projector_bias"]), _ptr(keep["head_weight"]),
                    _ptr(keep["head_bias"]), int(wt == np.float32))
    return w, keep, wt


def exp_f32(x: float) -> float:
    return float(lib().pko_exp_f32(float(x)))


def tanh_f32(x: float) -> float:
    return float(lib().pko_tanh_f32(float(x)))


def tdt_predictor(weights: dict, token: int, state, initial: bool = False) -> np.ndarray:
    """Candidates [5, 640] (h0, c0, h1, c1, projection) of one predictor step
    from the committed state [4, 640] (tdt-decoder.ts:1341-1500)."""
    w, keep, _ = _tdt_weights(weights)
    state = np.ascontiguousarray(state, dtype=np.float32).reshape(4, TDT_HIDDEN)
    cand = np.empty((5, TDT_HIDDEN), dtype=np.float32)
    lib().pko_tdt_predictor(ctypes.byref(w), int(token), int(initial), _ptr(state), _ptr(cand))
    return cand


def tdt_joint(weights: dict, encoder_row, projection):
    """(scores [1032], token, duration) of one joint (tdt-decoder.ts:1605-1662);
    encoder_row in the weights' element type."""
    w, keep, wt = _tdt_weights(weights)
    encoder_row = np.ascontiguousarray(encoder_row, dtype=wt)
    projection = np.ascontiguousarray(projection, dtype=np.float32)
    scores = np.empty(TDT_HEAD, dtype=np.float32)
    token, duration = ctypes.c_uint32(), ctypes.c_uint32()
    lib().pko_tdt_joint(ctypes.byref(w), _ptr(encoder_row), _ptr(projection), _ptr(scores), ctypes.byref(token),
                        ctypes.byref(duration))
    return scores, token.value, duration.value


def tdt_decode(weights: dict, encoder_projected, lengths, *, max_tokens: int, starts=None, ends=None, flush=None):
    """Greedy TDT decode (tdt-decoder.ts:1664-2010) of encoder_projected
    [batch, frames, 640] in the weights' element type (f16 or f32 profile);
    returns dict(tokens, frames, durations [batch,
    max_tokens] u32, counts, status [batch], and the final state [batch, 4,
    640] and predictor scratch [batch, 5, 640])."""
    w, keep, wt = _tdt_weights(weights)
    enc = np.ascontiguousarray(encoder_projected, dtype=wt)
    batch, frames, hidden = enc.shape
    if hidden != TDT_HIDDEN:
        raise ValueError("encoder_projected must be [batch, frames, 640]")

    def vec(v, default):
        return np.ascontiguousarray(np.full(batch, default) if v is None else v, dtype=np.uint32)
    lengths = vec(lengths, frames)
    starts, ends, flush = vec(starts, 0), vec(ends, 0xFFFFFFFF), vec(flush, 0)
    state = np.zeros((batch, 4, TDT_HIDDEN), np.float32)
    scratch = np.zeros((batch, 5, TDT_HIDDEN), np.float32)
    out = {k: np.zeros((batch, max_tokens), np.uint32) for k in ("tokens", "frames", "durations")}
    counts, status = np.zeros(batch, np.uint32), np.zeros(batch, np.uint32)
    if lib().pko_tdt_decode(ctypes.byref(w), batch, frames, max_tokens, _ptr(enc), _ptr(lengths), _ptr(starts),
                            _ptr(ends), _ptr(flush), _ptr(state), _ptr(scratch), _ptr(out["tokens"]),
                            _ptr(out["frames"]), _ptr(out["durations"]), _ptr(counts), _ptr(status)):
        raise ValueError("tdt_decode rejected its arguments")
    out.update(counts=counts, status=status, state=state, scratch=scratch)
    return out


def encoder_front_end(features, front, feature_lengths, *, gemm_mode=None, threads=8,
                      dtype=np.float16) -> np.ndarray:
    """The subsampling front end (encoder.ts:2140-2400) over f32
    feature-major fbank [batch, 128, F] into [batch * sub(F, 3), 1024] f16:
    conv0 + ReLU + depthwise2, pointwise3 + bias + ReLU, depthwise5,
    pointwise6 + bias + ReLU, rows past sub(L, 3) zeroed, flatten (frequency
    major) and the linear 4096 -> 1024 + bias. `front` is keyed like
    pk_encoder_subsampling; stages stored in `dtype` (as encoder_layer)."""
    dtype, gemm_mode = _chain(dtype, gemm_mode)
    batch = features.shape[0]
    stage = subsampling_fused(features, front["conv0_weights"], front["conv0_bias"], front["depthwise2_weights"],
                              front["depthwise2_bias"], feature_lengths, dtype=dtype)
    _, h2, w2, channels = stage.shape

    def mm(name, a, columns, **epilogue):
        words, palette = front[name]
        out = gemm(a, words, 5, np.asarray(palette, dtype=dtype), columns, mode=gemm_mode, threads=threads,
                   **epilogue)
        return out.astype(dtype)
    projected = mm("pointwise3", stage.reshape(-1, channels), channels, bias=front["pointwise3_bias"],
                   activation="relu").reshape(batch, h2, w2, channels)
    stage = subsampling_depthwise(projected, front["depthwise5_weights"], front["depthwise5_bias"], feature_lengths, 3)
    _, h3, w3, _ = stage.shape
    projected = mm("pointwise6", stage.reshape(-1, channels), channels, bias=front["pointwise6_bias"],
                   activation="relu").reshape(batch, h3, w3, channels)
    projected = subsampling_mask(projected, feature_lengths, 3)
    return mm("linear", projected.reshape(batch * h3, w3 * channels), 1024, bias=front["linear_bias"])


def encoder_graph(x, layers, valid, *, batch, frames, front=None, features=None, feature_lengths=None,
                  projector=None, projector_bias=None, gemm_mode=None, threads=8, dtype=np.float16):
    """ParakeetEncoderGraph.encode (encoder.ts:1690-1706): the front end when
    `front` is given (from `features`; `x` is then unused), the layers, and
    the projector when given, every stage stored in `dtype`. Returns
    (output, projected or None)."""
    dtype, gemm_mode = _chain(dtype, gemm_mode)
    if front is not None:
        x = encoder_front_end(features, front, feature_lengths, gemm_mode=gemm_mode, threads=threads, dtype=dtype)
    out = encoder(x, layers, valid, batch=batch, frames=frames, gemm_mode=gemm_mode, threads=threads, dtype=dtype)
    projected = None
    if projector is not None:
        words, palette = projector
        projected = gemm(out, words, 5, np.asarray(palette, dtype=dtype), projector_bias.size, bias=projector_bias,
                         mode=gemm_mode, threads=threads).astype(dtype)
    return out, projected


def relative_errors(got: np.ndarray, want: np.ndarray) -> tuple[float, float]:
    """(norm-wise, max-wise) relative error of got against want, in double."""
    g = np.asarray(got, dtype=np.float64)
    w = np.asarray(want, dtype=np.float64)
    diff = g - w
    norm = float(np.linalg.norm(diff) / max(np.linalg.norm(w), 1e-300))
    peak = float(np.max(np.abs(diff)) / max(np.max(np.abs(w)), 1e-300)) if w.size else 0.0
    return norm, peak

"""Seeded synthetic inputs for the palette GEMM workloads.

The weights are random palette codes packed in the reference package format
(model/convert.py:2130-2156: groups of 32 codes in 5 little-endian u32 words
for 5-bit, 16 codes in 3 words for 6-bit, code i of a group at bit i*bits,
LSB first) with random LUTs, as the benchmark configurations prescribe; no
checkpoint is involved. Everything derives from numpy's PCG64 generator so a
seed fixes every array.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


def codes_per_group(bits: int) -> int:
    return {5: 32, 6: 16}[bits]


def words_per_group(bits: int) -> int:
    return {5: 5, 6: 3}[bits]


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Bit-pack codes ([K, N] K-major or flat) into [groups, words] u32 words."""
    cpg, wpg = codes_per_group(bits), words_per_group(bits)
    flat = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1)
    if flat.size % cpg:
        raise ValueError(f"{flat.size} codes are not a multiple of {cpg}")
    if flat.size and int(flat.max()) >= 1 << bits:
        raise ValueError(f"{bits}-bit codes must be below {1 << bits}")
    grouped = flat.reshape(-1, cpg).astype(np.uint64)
    # one 160- or 96-bit integer per group, then split into u32 words
    shifts = (np.arange(cpg, dtype=np.uint64) * np.uint64(bits))
    words = np.zeros((grouped.shape[0], wpg), dtype=np.uint64)
    for i in range(cpg):
        bit = int(shifts[i])
        word, shift = divmod(bit, 32)
        words[:, word] |= (grouped[:, i] << np.uint64(shift)) & np.uint64(0xFFFFFFFF)
        if shift + bits > 32:
            words[:, word + 1] |= grouped[:, i] >> np.uint64(32 - shift)
    return words.astype("<u4")


@dataclass
class PaletteMatrix:
    """A random palette weight: codes [K, N], packed words, LUT [G, 2^bits]."""
    bits: int
    inner: int
    columns: int
    codes: np.ndarray
    packed: np.ndarray
    palette: np.ndarray

    @property
    def groups(self) -> int:
        return self.palette.shape[0]


def palette_matrix(rng: np.random.Generator, bits: int, inner: int, columns: int, *,
                   dtype=np.float16, groups: int = 1, lut_std: float = 0.02) -> PaletteMatrix:
    codes = rng.integers(0, 1 << bits, size=(inner, columns), dtype=np.uint8)
    palette = (rng.standard_normal((groups, 1 << bits)) * lut_std).astype(dtype)
    return PaletteMatrix(bits, inner, columns, codes, pack_codes(codes, bits), palette)


def normal(rng: np.random.Generator, shape, std: float = 1.0, dtype=np.float16) -> np.ndarray:
    return (rng.standard_normal(shape) * std).astype(dtype)


@dataclass
class GemmCase:
    """One palette GEMM with its epilogue operands."""
    name: str
    a: np.ndarray
    weight: PaletteMatrix
    bias: np.ndarray | None = None
    residual: np.ndarray | None = None
    residual_scale: float | None = None
    activation: str = "none"
    extra: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return self.a.shape[0]

    @property
    def flops(self) -> int:
        return 2 * self.rows * self.weight.inner * self.weight.columns

    def algorithmic_bytes(self) -> int:
        """Compulsory HBM bytes: each tensor once, the dense weight never."""
        e = self.a.dtype.itemsize
        w = self.weight
        total = (w.inner * w.columns * w.bits + 7) // 8
        total += w.palette.size * w.palette.dtype.itemsize
        total += self.a.size * e + self.rows * w.columns * e
        if self.bias is not None:
            total += 4 * w.columns
        if self.residual is not None:
            total += self.rows * w.columns * e
        return total


def single_gemm_fp32(seed: int = 0, rows: int = 256) -> GemmCase:
    """X[256x1024] ~ N(0,1) f32, 6-bit W 1024->4096, one 64-entry f32 LUT
    ~ N(0, 0.02), bias ~ N(0, 0.01): Y = X W + b."""
    rng = np.random.default_rng(seed)
    x = normal(rng, (rows, 1024), 1.0, np.float32)
    w = palette_matrix(rng, 6, 1024, 4096, dtype=np.float32)
    bias = normal(rng, (4096,), 0.01, np.float32)
    return GemmCase("single-gemm-fp32", x, w, bias=bias)


@dataclass
class FeedForwardBlock:
    """Conformer feed-forward block: H = SiLU(X W1), Y = X + 0.5 (H W2)."""
    x: np.ndarray
    w1: PaletteMatrix
    w2: PaletteMatrix

    def expand_case(self) -> GemmCase:
        return GemmCase("ff-expand", self.x, self.w1, activation="silu")

    def contract_case(self, hidden: np.ndarray) -> GemmCase:
        return GemmCase("ff-contract", hidden, self.w2, residual=self.x, residual_scale=0.5)

    @property
    def flops(self) -> int:
        m = self.x.shape[0]
        return 2 * m * self.w1.inner * self.w1.columns + 2 * m * self.w2.inner * self.w2.columns


def feed_forward_block(seed: int = 0, windows: int = 8, frames: int = 188, d_model: int = 1024,
                       hidden: int = 4096, bits: int = 5) -> FeedForwardBlock:
    """Input [windows x frames x d_model] f16 ~ N(0,1); 5-bit W1 d->4d and W2
    4d->d, one 32-entry f16 LUT each ~ N(0, 0.02)."""
    rng = np.random.default_rng(seed)
    x = normal(rng, (windows * frames, d_model), 1.0, np.float16)
    w1 = palette_matrix(rng, bits, d_model, hidden, dtype=np.float16)
    w2 = palette_matrix(rng, bits, hidden, d_model, dtype=np.float16)
    return FeedForwardBlock(x, w1, w2)


def gemm_case(seed: int, rows: int, inner: int, columns: int, bits: int, *, dtype=np.float16,
              groups: int = 1, activation: str = "none", bias: bool = False,
              residual_scale: float | None = None, a_std: float = 1.0) -> GemmCase:
    """A generic seeded palette GEMM for parity sweeps."""
    rng = np.random.default_rng(seed)
    a = normal(rng, (rows, inner), a_std, dtype)
    w = palette_matrix(rng, bits, inner, columns, dtype=dtype, groups=groups)
    b = normal(rng, (columns,), 0.01, np.float32) if bias else None
    r = normal(rng, (rows, columns), 1.0, dtype) if residual_scale is not None else None
    return GemmCase(f"gemm-{rows}x{inner}x{columns}-b{bits}", a, w, bias=b, residual=r,
                    residual_scale=residual_scale, activation=activation)


@dataclass
class ConvCase:
    """Operands of the fused Conformer convolution tail: the pointwise-1 output
    [batch*frames, 2C] (GLU values, then gates), depthwise weights [9, C],
    folded batch-norm scale and shift [C] (f32) and valid lengths [batch]."""
    pointwise: np.ndarray | None
    weights: np.ndarray
    scale: np.ndarray
    shift: np.ndarray
    valid: np.ndarray
    batch: int
    frames: int

    @property
    def channels(self) -> int:
        return self.weights.shape[1]

    def algorithmic_bytes(self, batch: int | None = None) -> int:
        """Compulsory HBM bytes of one launch over `batch` windows: the
        pointwise input and the output once, weights, affine, lengths."""
        batch = self.batch if batch is None else batch
        e = self.weights.dtype.itemsize
        rows = batch * self.frames
        return rows * 3 * self.channels * e + self.weights.nbytes + 8 * self.channels + 4 * batch


def conv_case(seed: int, batch: int, frames: int, channels: int = 1024, *, dtype=np.float16,
              valid=None, weight_std: float = 0.05, with_input: bool = True) -> ConvCase:
    """Seeded conv-tail operands: pointwise input ~ N(0,1), depthwise weights
    ~ N(0, weight_std), scale ~ 1 + N(0, 0.1), shift ~ N(0, 0.1); valid lengths
    uniform integers in [ceil(frames/2), frames] unless given."""
    rng = np.random.default_rng(seed)
    pointwise = normal(rng, (batch * frames, 2 * channels), 1.0, dtype) if with_input else None
    weights = normal(rng, (9, channels), weight_std, dtype)
    scale = (1.0 + 0.1 * rng.standard_normal(channels)).astype(np.float32)
    shift = (0.1 * rng.standard_normal(channels)).astype(np.float32)
    if valid is None:
        valid = rng.integers((frames + 1) // 2, frames + 1, size=batch)
    return ConvCase(pointwise, weights, scale, shift, np.asarray(valid, dtype=np.uint32), batch, frames)


@dataclass
class ConvModule:
    """Conformer convolution module after its layer norm: P = X PW1, Z =
    SiLU(BN(DW9(GLU(P)))), Y = X + Z PW2 (src/webgpu/encoder.ts:2011-2075)."""
    x: np.ndarray
    pw1: PaletteMatrix
    pw2: PaletteMatrix
    conv: ConvCase

    def pw1_case(self) -> GemmCase:
        return GemmCase("conv-pointwise1", self.x, self.pw1)

    def pw2_case(self, z: np.ndarray) -> GemmCase:
        return GemmCase("conv-pointwise2-residual", z, self.pw2, residual=self.x, residual_scale=1.0)

    @property
    def flops(self) -> int:
        m = self.x.shape[0]
        return 2 * m * self.pw1.inner * self.pw1.columns + 2 * m * self.pw2.inner * self.pw2.columns


def conv_module(seed: int = 0, windows: int = 16, frames: int = 188, d_model: int = 1024,
                bits: int = 6) -> ConvModule:
    """Input [windows x frames x d_model] f16 ~ N(0,1); 6-bit PW1 d->2d and
    PW2 d->d with one 64-entry f16 LUT each ~ N(0, 0.02); depthwise k9 f16
    weights ~ N(0, 0.05); folded BN scale ~ 1 + N(0, 0.1), shift ~ N(0, 0.1);
    valid lengths uniform in [frames/2, frames]."""
    rng = np.random.default_rng(seed)
    x = normal(rng, (windows * frames, d_model), 1.0, np.float16)
    pw1 = palette_matrix(rng, bits, d_model, 2 * d_model, dtype=np.float16)
    pw2 = palette_matrix(rng, bits, d_model, d_model, dtype=np.float16)
    conv = conv_case(int(rng.integers(1 << 31)), windows, frames, d_model, with_input=False)
    return ConvModule(x, pw1, pw2, conv)


def relative_position_table(frames: int, channels: int = 1024) -> np.ndarray:
    """The descending Transformer-XL sinusoid table [2T-1, channels] f32 the
    reference converter builds (model/convert.py:1143-1165): row p is relative
    distance T-1-p, even channels sin(pos * 10000^(-c/C)), odd channels cos."""
    if frames < 1 or channels < 2 or channels % 2:
        raise ValueError("frames must be positive and channels a positive even number")
    positions = np.arange(frames - 1, -frames, -1, dtype=np.float32).reshape(-1, 1)
    exponent = np.float32(-(np.log(10_000.0) / channels))
    div_term = np.exp(np.arange(0, channels, 2, dtype=np.float32) * exponent)
    angles = positions * div_term.reshape(1, -1)
    table = np.empty((2 * frames - 1, channels), dtype=np.float32)
    table[:, 0::2] = np.sin(angles)
    table[:, 1::2] = np.cos(angles)
    return table


def pack_projected_positions(projected: np.ndarray, heads: int = 8, vector_width: int = 4) -> np.ndarray:
    """[positions, channels] -> the reference's "head-vector-position-vec4"
    order [heads, head_size / 4, positions, 4] (model/convert.py:1196-1225)."""
    rows, channels = projected.shape
    head = channels // heads
    return np.ascontiguousarray(projected.reshape(rows, heads, head // vector_width, vector_width)
                                .transpose(1, 2, 0, 3))


@dataclass
class AttentionCase:
    """Operands of the relative-position attention: qkv [B*T, 3072], projected
    positions [2T-1, 1024] (row-major; pack_projected_positions gives the
    reference's order), biases u, v [8, 128] f32, valid lengths [B]."""
    qkv: np.ndarray
    positions: np.ndarray
    bias_u: np.ndarray
    bias_v: np.ndarray
    valid: np.ndarray
    batch: int
    frames: int

    @property
    def packed_positions(self) -> np.ndarray:
        return pack_projected_positions(self.positions)

    def flops(self, batch: int | None = None) -> int:
        """Score (two products per key) and context FLOP of the live keys."""
        batch = self.batch if batch is None else batch
        live = np.minimum(self.valid[:batch].astype(np.int64), self.frames)
        return int((live * live).sum()) * 8 * 128 * 2 * 3

    def algorithmic_bytes(self, batch: int | None = None) -> int:
        batch = self.batch if batch is None else batch
        e = self.qkv.dtype.itemsize
        rows = batch * self.frames
        return rows * 3072 * e + self.positions.size * e + 2 * 4096 + 4 * batch + rows * 1024 * e


def attention_case(seed: int, batch: int, frames: int, *, dtype=np.float16, valid=None, qkv_std: float = 0.6,
                   position_std: float = 0.6) -> AttentionCase:
    """Seeded attention operands: qkv ~ N(0, qkv_std) (about what a 1024-wide
    palette projection with N(0, 0.02) centroids makes of unit inputs),
    positions ~ N(0, position_std), u, v ~ N(0, 0.02); valid lengths uniform
    integers in [ceil(T/2), T] unless given."""
    rng = np.random.default_rng(seed)
    qkv = normal(rng, (batch * frames, 3072), qkv_std, dtype)
    positions = normal(rng, (2 * frames - 1, 1024), position_std, dtype)
    bias_u = normal(rng, (8, 128), 0.02, np.float32)
    bias_v = normal(rng, (8, 128), 0.02, np.float32)
    if valid is None:
        valid = rng.integers((frames + 1) // 2, frames + 1, size=batch)
    return AttentionCase(qkv, positions, bias_u, bias_v, np.asarray(valid, dtype=np.uint32), batch, frames)


@dataclass
class MhaModule:
    """Relative-position multi-head attention block after its layer norm
    (src/webgpu/encoder.ts:1930-2010): QKV = X Wqkv (3 palette groups, Q|K|V),
    P = table(T) Wpos (the rel-pos linear over the 2T-1 sinusoid rows),
    C = attention(QKV, P, u, v, valid), Y = X + C Wo."""
    x: np.ndarray
    wqkv: PaletteMatrix
    wpos: PaletteMatrix
    wo: PaletteMatrix
    table: np.ndarray          # [2T-1, 1024] f16 sinusoid rows
    bias_u: np.ndarray
    bias_v: np.ndarray
    valid: np.ndarray
    batch: int
    frames: int

    def gemm_flops(self) -> int:
        m, p = self.x.shape[0], self.table.shape[0]
        return 2 * m * 1024 * 3072 + 2 * p * 1024 * 1024 + 2 * m * 1024 * 1024

    def attention_flops(self) -> int:
        live = np.minimum(self.valid.astype(np.int64), self.frames)
        return int((live * live).sum()) * 8 * 128 * 2 * 3


def mha_module(seed: int = 0, windows: int = 4, frames: int = 188, d_model: int = 1024, bits: int = 6) -> MhaModule:
    """Input [windows x frames x 1024] f16 ~ N(0,1); 6-bit Wqkv 1024->3072
    with three 64-entry f16 LUTs (one per Q/K/V block, the reference's QKV
    layout), 6-bit Wpos and Wo 1024->1024, LUTs ~ N(0, 0.02); u, v ~
    N(0, 0.02); valid lengths uniform integers in [ceil(T/2), T]."""
    rng = np.random.default_rng(seed)
    x = normal(rng, (windows * frames, d_model), 1.0, np.float16)
    wqkv = palette_matrix(rng, bits, d_model, 3 * d_model, dtype=np.float16, groups=3)
    wpos = palette_matrix(rng, bits, d_model, d_model, dtype=np.float16)
    wo = palette_matrix(rng, bits, d_model, d_model, dtype=np.float16)
    bias_u = normal(rng, (8, 128), 0.02, np.float32)
    bias_v = normal(rng, (8, 128), 0.02, np.float32)
    valid = rng.integers((frames + 1) // 2, frames + 1, size=windows).astype(np.uint32)
    table = relative_position_table(frames, d_model).astype(np.float16)
    return MhaModule(x, wqkv, wpos, wo, table, bias_u, bias_v, valid, windows, frames)


# Encoder layer matrices: name -> (bits, inner, columns, palette groups), the
# reference package's widths (model/convert.py:1360-1475, encoder.ts:2458-2512).
ENCODER_MATRICES = {
    "ff1_linear1": (5, 1024, 4096, 1),
    "ff1_linear2": (5, 4096, 1024, 1),
    "qkv": (5, 1024, 3072, 3),
    "o_proj": (6, 1024, 1024, 1),
    "pointwise1": (5, 1024, 2048, 1),
    "pointwise2": (5, 1024, 1024, 1),
    "ff2_linear1": (5, 1024, 4096, 1),
    "ff2_linear2": (5, 4096, 1024, 1),
}


def random_packed_words(rng: np.random.Generator, bits: int, inner: int, columns: int) -> np.ndarray:
    """Packed words of uniformly random codes: every bit of a packed group is
    a code bit, so uniform words are uniform codes."""
    count = inner * columns // codes_per_group(bits) * words_per_group(bits)
    return rng.integers(0, 1 << 32, size=count, dtype=np.uint32)


@dataclass
class EncoderStack:
    """Random-init FastConformer encoder layers over subsampled features
    x [windows*frames, 1024] f16. Each layer is a dict keyed like
    pk_encoder_layer: norm_gamma / norm_beta [5, 1024] f32; each matrix of
    ENCODER_MATRICES a (packed words, palette [G, 2^bits] f16) pair;
    projected_positions in head-vector-position-vec4 order [8, 32, 2T-1, 4]
    f16; bias_u, bias_v [8, 128] f32; depthwise [9, 1024] f16; bn_scale,
    bn_shift [1024] f32."""
    x: np.ndarray
    layers: list
    valid: np.ndarray
    batch: int
    frames: int
    # Front end (None without it): f32 feature-major fbank [windows, 128,
    # feature_frames], raw lengths, and the weights keyed like
    # pk_encoder_subsampling.
    features: np.ndarray | None = None
    feature_lengths: np.ndarray | None = None
    subsampling: dict | None = None
    # Projector (None without it): (packed, palette [1, 32] f16), f32 bias.
    projector: tuple | None = None
    projector_bias: np.ndarray | None = None

    @property
    def feature_frames(self) -> int:
        return 0 if self.features is None else self.features.shape[2]

    def gemm_flops(self, batch: int | None = None) -> int:
        batch = self.batch if batch is None else batch
        rows = batch * self.frames
        per_layer = sum(2 * rows * k * n for _, k, n, _ in ENCODER_MATRICES.values())
        total = per_layer * len(self.layers)
        if self.subsampling is not None:
            h2 = subsampled_length(self.feature_frames, 2)
            total += 2 * batch * (h2 * 32 + self.frames * 16) * 256 * 256 + 2 * rows * 4096 * 1024
        if self.projector is not None:
            total += 2 * rows * 1024 * self.projector_bias.size
        return total

    def front_end_flops(self, batch: int | None = None) -> int:
        """Multiply-adds x 2 of the three convolutions of the front end."""
        if self.subsampling is None:
            return 0
        batch = self.batch if batch is None else batch
        h1, h2 = subsampled_length(self.feature_frames, 1), subsampled_length(self.feature_frames, 2)
        return 2 * 9 * 256 * batch * (h1 * 64 + h2 * 32 + self.frames * 16)

    def attention_flops(self, batch: int | None = None) -> int:
        batch = self.batch if batch is None else batch
        live = np.minimum(self.valid[:batch].astype(np.int64), self.frames)
        return int((live * live).sum()) * 8 * 128 * 2 * 3 * len(self.layers)

    def weight_bytes(self) -> int:
        """Package bytes the stack reads per pass: packed codes, LUTs,
        positions, norms, biases, depthwise and folded batch norm."""
        total = 0
        for layer in self.layers:
            for name in ENCODER_MATRICES:
                packed, palette = layer[name]
                total += packed.nbytes + palette.nbytes
            for name in ("norm_gamma", "norm_beta", "projected_positions", "bias_u", "bias_v", "depthwise",
                         "bn_scale", "bn_shift"):
                total += layer[name].nbytes
        return total


def encoder_layer_weights(rng: np.random.Generator, frames: int, lut_std: float = 0.02) -> dict:
    layer = {
        "norm_gamma": (1.0 + 0.1 * rng.standard_normal((5, 1024))).astype(np.float32),
        "norm_beta": (0.1 * rng.standard_normal((5, 1024))).astype(np.float32),
    }
    for name, (bits, inner, columns, groups) in ENCODER_MATRICES.items():
        layer[name] = (random_packed_words(rng, bits, inner, columns),
                       normal(rng, (groups, 1 << bits), lut_std, np.float16))
    layer["projected_positions"] = pack_projected_positions(normal(rng, (2 * frames - 1, 1024), 0.6, np.float16))
    layer["bias_u"] = normal(rng, (8, 128), 0.02, np.float32)
    layer["bias_v"] = normal(rng, (8, 128), 0.02, np.float32)
    layer["depthwise"] = normal(rng, (9, 1024), 0.05, np.float16)
    layer["bn_scale"] = (1.0 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    layer["bn_shift"] = (0.1 * rng.standard_normal(1024)).astype(np.float32)
    return layer


def subsampled_length(length: int, steps: int) -> int:
    """Frames after `steps` same-padded stride-2 convolutions."""
    for _ in range(steps):
        length = (length + 1) // 2
    return length


def subsampling_weights(rng: np.random.Generator) -> dict:
    """Front-end weights keyed like pk_encoder_subsampling: conv0 and the
    depthwise kernels [3, 3, 256] f16 ~ N(0, 0.3), biases ~ N(0, 0.05),
    5-bit pointwise 256->256 and flatten 4096->1024 palettes (LUTs ~
    N(0, 0.05) and N(0, 0.08), centred, so the features reach the layers
    at about unit scale)."""
    def kernel():
        return normal(rng, (3, 3, 256), 0.3, np.float16)

    def bias(n):
        return normal(rng, (n,), 0.05, np.float32)
    front = {"conv0_weights": kernel(), "conv0_bias": bias(256), "depthwise2_weights": kernel(),
             "depthwise2_bias": bias(256)}
    def centred_lut(std):
        # These matrices act on ReLU outputs (all >= 0): a LUT mean would add
        # the same offset to every output, so the random LUTs are centred.
        lut = rng.standard_normal((1, 32)) * std
        return (lut - lut.mean()).astype(np.float16)
    front["pointwise3"] = (random_packed_words(rng, 5, 256, 256), centred_lut(0.05))
    front["pointwise3_bias"] = bias(256)
    front["depthwise5_weights"], front["depthwise5_bias"] = kernel(), bias(256)
    front["pointwise6"] = (random_packed_words(rng, 5, 256, 256), centred_lut(0.05))
    front["pointwise6_bias"] = bias(256)
    front["linear"] = (random_packed_words(rng, 5, 4096, 1024), centred_lut(0.08))
    front["linear_bias"] = bias(1024)
    return front


def encoder_stack(seed: int = 0, windows: int = 16, frames: int = 188, layers: int = 24,
                  valid=None, front_end: bool = False, projector: bool = False,
                  feature_lengths=None) -> EncoderStack:
    """Subsampled features [windows x frames x 1024] f16 ~ N(0,1) and
    `layers` random layers (with `front_end`, also an fbank [windows, 128,
    8T-3] f32 ~ N(0,1) with raw lengths uniform in [ceil(F/2), F] from which
    the valid lengths follow, and the front-end weights; with `projector`, a
    5-bit 1024->640 projector, LUT ~ N(0, 0.02), bias ~ N(0, 0.01)): uniform 5/6-bit codes with LUTs ~ N(0, 0.02)
    (QKV with one LUT per Q/K/V block), LayerNorm gamma ~ 1 + N(0, 0.1) and
    beta ~ N(0, 0.1), projected positions ~ N(0, 0.6), u, v ~ N(0, 0.02),
    depthwise ~ N(0, 0.05), folded BN scale ~ 1 + N(0, 0.1) and shift ~
    N(0, 0.1); valid lengths uniform integers in [ceil(T/2), T] unless given."""
    rng = np.random.default_rng(seed)
    x = normal(rng, (windows * frames, 1024), 1.0, np.float16)
    if valid is None:
        valid = rng.integers((frames + 1) // 2, frames + 1, size=windows)
    stack = [encoder_layer_weights(rng, frames) for _ in range(layers)]
    enc = EncoderStack(x, stack, np.asarray(valid, dtype=np.uint32), windows, frames)
    if front_end:
        # 8T - 3 fbank frames subsample to T (1501 -> 751 -> 376 -> 188)
        feature_frames = 8 * frames - 3
        enc.features = rng.standard_normal((windows, 128, feature_frames)).astype(np.float32)
        if feature_lengths is None:
            feature_lengths = rng.integers((feature_frames + 1) // 2, feature_frames + 1, size=windows)
        enc.feature_lengths = np.asarray(feature_lengths, dtype=np.uint32)
        enc.valid = np.array([subsampled_length(int(n), 3) for n in enc.feature_lengths], dtype=np.uint32)
        enc.subsampling = subsampling_weights(rng)
    if projector:
        enc.projector = (random_packed_words(rng, 5, 1024, 640), normal(rng, (1, 32), 0.02, np.float16))
        enc.projector_bias = normal(rng, (640,), 0.01, np.float32)
    return enc


def as_f32_profile(stack: EncoderStack) -> EncoderStack:
    """The same stack for the reference's fp32 profile (encoder.ts:947-1165):
    every f16 tensor (features, palettes, projected positions, depthwise and
    front-end convolution weights) widened to f32, which holds its values
    exactly; packed codes and the f32 per-channel tensors as they are."""
    def widen(v):
        if isinstance(v, np.ndarray) and v.dtype == np.float16:
            return v.astype(np.float32)
        if isinstance(v, tuple):
            return tuple(widen(u) for u in v)
        if isinstance(v, dict):
            return {k: widen(u) for k, u in v.items()}
        return v
    out = EncoderStack(widen(stack.x), [widen(layer) for layer in stack.layers], stack.valid, stack.batch,
                       stack.frames)
    for name in ("features", "feature_lengths", "subsampling", "projector", "projector_bias"):
        if hasattr(stack, name):
            setattr(out, name, widen(getattr(stack, name)))
    return out


@dataclass
class TdtCase:
    """A TDT decoder over random weights (decoder package shapes): weights
    keyed like palette_abi.TDT_WEIGHT_NAMES, the encoder projector's output
    [batch, frames, 640] (f16, or f32 for the f32 profile), encoded
    lengths, decode starts and ends, flush flags."""
    weights: dict
    encoder_projected: np.ndarray
    lengths: np.ndarray
    starts: np.ndarray
    ends: np.ndarray
    flush: np.ndarray

    @property
    def batch(self) -> int:
        return self.encoder_projected.shape[0]

    @property
    def frames(self) -> int:
        return self.encoder_projected.shape[1]


def tdt_weights(rng: np.random.Generator, blank_bias: float = 2.0, precision: str = "f16") -> dict:
    """Embedding ~ N(0, 0.5), LSTM weights ~ N(0, 0.03) and biases ~
    N(0, 0.1), projector ~ N(0, 0.04), head ~ N(0, 0.05) with bias ~
    N(0, 0.1) plus `blank_bias` on the blank (random heads otherwise never
    choose blank); weights in the profile's element (f16 or f32), f32
    biases."""
    wt = np.float32 if precision == "f32" else np.float16

    def n(shape, std, dtype):
        return (rng.standard_normal(shape) * std).astype(dtype)
    head_bias = n(1032, 0.1, np.float32)
    head_bias[1024] += blank_bias
    head_bias[1030:] = 0.0
    head = n((640, 1032), 0.05, wt)
    head[:, 1030:] = 0
    return dict(embedding=n((1025, 640), 0.5, wt), lstm_weight_l0=n((1280, 2560), 0.03, wt),
                lstm_weight_l1=n((1280, 2560), 0.03, wt), lstm_bias_l0=n(2560, 0.1, np.float32),
                lstm_bias_l1=n(2560, 0.1, np.float32), projector_weight=n((640, 640), 0.04, wt),
                projector_bias=n(640, 0.1, np.float32), head_weight=head, head_bias=head_bias)


def tdt_case(seed: int = 0, batch: int = 16, frames: int = 188, *, lengths=None, starts=None, ends=None,
             flush=None, blank_bias: float = 2.0, encoder_std: float = 0.5, precision: str = "f16") -> TdtCase:
    """Encoder projector output ~ N(0, encoder_std) in the profile's element
    (f16 or f32); lengths uniform in [ceil(T/2), T] unless given; starts 0,
    ends T, no flush unless given."""
    rng = np.random.default_rng(seed)
    weights = tdt_weights(rng, blank_bias, precision)
    enc = normal(rng, (batch, frames, 640), encoder_std, np.float32 if precision == "f32" else np.float16)
    if lengths is None:
        lengths = rng.integers((frames + 1) // 2, frames + 1, size=batch)

    def vec(v, default):
        return np.asarray(np.full(batch, default) if v is None else v, dtype=np.uint32)
    return TdtCase(weights, enc, vec(lengths, frames), vec(starts, 0), vec(ends, frames), vec(flush, 0))

"""Pins of the oracle's encoder composition and of its f16 accumulation
order, each against something that can disagree with the oracle.

* One FastConformer layer (encoder.ts:1897-2116) restated through torch's
  library routines in float64 - layer_norm, matmul over dense weights
  unpacked here from the packed bit stream with numpy (not the oracle's
  unpack), silu, the torch attention and convolution restatements of
  test_oracle.py - with every arena tensor stored as f16 like the
  reference's, compared with pko.encoder_layer(gemm_mode="f64"). Planted
  wiring mistakes (a residual from the wrong tensor, a swapped LayerNorm, a
  1 instead of 0.5 scale) each fail the same bar by orders of magnitude.
* The subsampling front end (encoder.ts:2140-2400) restated with torch's
  conv2d (stride 2, padding 1, grouped depthwise), matmul + bias + ReLU and a
  frequency-major flatten, against pko.encoder_front_end(gemm_mode="f64");
  a time-major flatten fails.
* The f16 accumulator of the reference's fp16 GEMM (gemm.ts:1445-1453):
  closed forms that only an increasing-k binary16 chain produces.

The composition runs its LayerNorm, attention, convolution and epilogues in
f32 (the reference's arithmetic), the restatement in float64, and both round
every stored tensor to f16: an f32 difference now and then moves an f16
rounding by one ulp, and the next GEMMs spread those ulps over every
output, so the two agree to 3e-4 (one layer) and 2e-4 (front end)
norm-wise. The bar is 2e-3; the smallest planted mistake (a swapped
LayerNorm) moves the result by 4e-2, the others by 0.2."""
import numpy as np
import pytest

from test_oracle import _torch_conv_module, _torch_relative_attention

THREADS = 8
BAR = 2e-3


def dense_weights(words, bits, palette, inner, columns):
    """[K, N] float64 weights: codes read from the LSB-first bit stream of
    the little-endian words (code i at bit i * bits, convert.py:2119-2156),
    palette group min(n // (N / G), G - 1) (palette-expander.ts:543-549)."""
    stream = np.unpackbits(np.ascontiguousarray(words, dtype="<u4").view(np.uint8), bitorder="little")
    codes = (stream.reshape(-1, bits).astype(np.int64) << np.arange(bits)).sum(axis=1).reshape(inner, columns)
    groups = palette.shape[0]
    group = np.minimum(np.arange(columns) // (columns // groups), groups - 1)
    return palette.astype(np.float64)[group[None, :], codes]


def unpack_positions(packed):
    """[8, 32, 2T-1, 4] head-vector-position-vec4 -> [2T-1, 1024]."""
    heads, vectors, rows, width = packed.shape
    return np.ascontiguousarray(packed.transpose(2, 0, 1, 3).reshape(rows, heads * vectors * width))


class _Attention:
    def __init__(self, qkv, positions, bias_u, bias_v, valid, batch, frames):
        self.qkv, self.positions, self.bias_u, self.bias_v = qkv, positions, bias_u, bias_v
        self.valid, self.batch, self.frames = valid, batch, frames


def torch_encoder_layer(x, layer, valid, batch, frames, mistake=None, storage="f16"):
    """One layer through torch in float64, f16 (or, for the fp32 profile,
    f32) storage between dispatches."""
    import torch
    import torch.nn.functional as F
    stored = torch.float16 if storage == "f16" else torch.float32

    def f16(t):
        return t.to(stored).to(torch.float64)

    def tensor(a):
        return torch.from_numpy(np.asarray(a, dtype=np.float64))
    from parakeet_wgsl_amd.workloads import ENCODER_MATRICES

    def weight(name):
        bits, inner, columns, _ = ENCODER_MATRICES[name]
        words, palette = layer[name]
        return torch.from_numpy(dense_weights(words, bits, palette, inner, columns))

    def norm(i, h):
        if mistake == "swapped-norm" and i in (1, 2):
            i = 3 - i
        return f16(F.layer_norm(h, (1024,), tensor(layer["norm_gamma"][i]), tensor(layer["norm_beta"][i]),
                                eps=1e-5))

    def linear(name, a, activation=None, residual=None, scale=1.0):
        v = a @ weight(name)
        if activation == "silu":
            v = F.silu(v)
        if residual is not None:
            v = residual + scale * v
        return f16(v)

    x = f16(tensor(x))
    ff_scale = 1.0 if mistake == "ff-scale-one" else 0.5
    x1 = linear("ff1_linear2", linear("ff1_linear1", norm(0, x), "silu"), residual=x, scale=ff_scale)
    qkv = linear("qkv", norm(1, x1))
    case = _Attention(qkv.numpy(), unpack_positions(layer["projected_positions"]), layer["bias_u"], layer["bias_v"],
                      valid, batch, frames)
    context = f16(tensor(_torch_relative_attention(case)))
    x2 = linear("o_proj", context, residual=x if mistake == "o-proj-residual-from-x" else x1)
    pointwise = linear("pointwise1", norm(2, x2))
    conv = f16(tensor(_torch_conv_module(pointwise.numpy(), layer["depthwise"], layer["bn_scale"],
                                         layer["bn_shift"], valid, batch, frames)))
    x3 = linear("pointwise2", conv, residual=x2)
    x4 = linear("ff2_linear2", linear("ff2_linear1", norm(3, x3), "silu"), residual=x3, scale=0.5)
    return norm(4, x4).numpy()


@pytest.fixture(scope="module")
def one_layer(workloads):
    stack = workloads.encoder_stack(seed=31, windows=2, frames=64, layers=1, valid=[64, 37])
    return stack


def test_encoder_layer_matches_torch_restatement(oracle, one_layer):
    s = one_layer
    got = oracle.encoder_layer(s.x, s.layers[0], s.valid, batch=s.batch, frames=s.frames, gemm_mode="f64",
                               threads=THREADS)
    want = torch_encoder_layer(s.x, s.layers[0], s.valid, s.batch, s.frames)
    norm, worst = oracle.relative_errors(got, want)
    print(f"encoder layer vs torch float64 restatement: norm {norm:.2e} max {worst:.2e}")
    assert norm <= BAR, (norm, worst)


@pytest.mark.parametrize("mistake", ["o-proj-residual-from-x", "swapped-norm", "ff-scale-one"])
def test_encoder_layer_planted_mistakes_fail(oracle, one_layer, mistake):
    s = one_layer
    got = oracle.encoder_layer(s.x, s.layers[0], s.valid, batch=s.batch, frames=s.frames, gemm_mode="f64",
                               threads=THREADS)
    wrong = torch_encoder_layer(s.x, s.layers[0], s.valid, s.batch, s.frames, mistake=mistake)
    norm, _ = oracle.relative_errors(got, wrong)
    print(f"{mistake}: norm {norm:.2e}")
    assert norm > 10 * BAR, (mistake, norm)


def torch_front_end(oracle, features, front, lengths, mistake=None, storage="f16"):
    """The front end through torch in float64 with the f16 (or f32)
    profile's storage: conv0 + ReLU (rounded to the storage type) +
    depthwise2, pointwise3 + bias + ReLU, depthwise5 over the rows below
    sub(L, 2), pointwise6 + bias + ReLU, rows past sub(L, 3) zeroed, the
    frequency-major flatten and the linear."""
    import torch
    import torch.nn.functional as F
    stored = torch.float16 if storage == "f16" else torch.float32

    def f16(t):
        return t.to(stored).to(torch.float64)

    def kernel(w):  # [3, 3, C] -> [C, 1, 3, 3]
        return torch.from_numpy(np.asarray(w, np.float64)).permute(2, 0, 1).unsqueeze(1)

    def bias(b):
        return torch.from_numpy(np.asarray(b, np.float64))

    def linear(name, a, b, relu):
        words, palette = front[name]
        inner = a.shape[-1]
        columns = b.shape[0]
        v = a @ torch.from_numpy(dense_weights(words, 5, palette, inner, columns)) + bias(b)
        return f16(torch.relu(v) if relu else v)

    batch = features.shape[0]
    sub = oracle.subsampled_length
    x = torch.from_numpy(features.astype(np.float64)).permute(0, 2, 1).unsqueeze(1)  # [B, 1, time, bins]
    c0 = f16(torch.relu(F.conv2d(x, kernel(front["conv0_weights"]), bias(front["conv0_bias"]), stride=2,
                                 padding=1)))
    for b, n in enumerate(lengths):
        c0[b, :, sub(int(n), 1):] = 0
    s2 = F.conv2d(c0, kernel(front["depthwise2_weights"]), bias(front["depthwise2_bias"]), stride=2, padding=1,
                  groups=256)
    for b, n in enumerate(lengths):
        s2[b, :, sub(int(n), 2):] = 0
    s2 = f16(s2.permute(0, 2, 3, 1))  # [B, H2, W2, C]
    p3 = linear("pointwise3", s2, front["pointwise3_bias"], True)
    t = p3.permute(0, 3, 1, 2).clone()
    for b, n in enumerate(lengths):
        t[b, :, sub(int(n), 2):] = 0
    s5 = F.conv2d(t, kernel(front["depthwise5_weights"]), bias(front["depthwise5_bias"]), stride=2, padding=1,
                  groups=256)
    for b, n in enumerate(lengths):
        s5[b, :, sub(int(n), 3):] = 0
    s5 = f16(s5.permute(0, 2, 3, 1))  # [B, H3, W3, C]
    p6 = linear("pointwise6", s5, front["pointwise6_bias"], True)
    for b, n in enumerate(lengths):
        p6[b, sub(int(n), 3):] = 0
    h3, w3 = p6.shape[1], p6.shape[2]
    if mistake == "time-major-flatten":
        flat = p6.permute(0, 1, 3, 2).reshape(batch * h3, w3 * 256)
    else:
        flat = p6.reshape(batch * h3, w3 * 256)
    return linear("linear", flat, front["linear_bias"], False).numpy()


@pytest.fixture(scope="module")
def front_case(workloads):
    return workloads.encoder_stack(seed=32, windows=2, frames=24, layers=0, front_end=True,
                                   feature_lengths=[189, 120])


def test_front_end_matches_torch_restatement(oracle, front_case):
    s = front_case
    got = oracle.encoder_front_end(s.features, s.subsampling, s.feature_lengths, gemm_mode="f64", threads=THREADS)
    want = torch_front_end(oracle, s.features, s.subsampling, s.feature_lengths)
    assert got.shape == want.shape == (2 * 24, 1024)
    norm, worst = oracle.relative_errors(got, want)
    print(f"front end vs torch float64 restatement: norm {norm:.2e} max {worst:.2e}")
    assert norm <= BAR, (norm, worst)
    wrong = torch_front_end(oracle, s.features, s.subsampling, s.feature_lengths, mistake="time-major-flatten")
    bad, _ = oracle.relative_errors(got, wrong)
    print(f"time-major flatten: norm {bad:.2e}")
    assert bad > 10 * BAR


# --------------------------------------------------- f16 accumulation order

def _ones_case(oracle, inner, first):
    """A [1, K] = 2048 at k = `first`, 1 elsewhere; a constant palette of 1.0
    makes every weight 1 whatever the codes."""
    a = np.ones((1, inner), np.float16)
    a[0, first] = 2048.0
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 32, size=inner * 32).astype(np.uint8)
    words = oracle.pack_codes(codes, 5)
    palette = np.ones((1, 32), np.float16)
    return a, words, palette


@pytest.mark.parametrize("inner", [64, 1024])
def test_f16_chain_closed_form_large_term_first(oracle, inner):
    """2048 first, then K - 1 ones: in binary16 every 2048 + 1 is a tie that
    rounds to the even 2048, so an increasing-k f16 chain stays at 2048; the
    exact sum (the f64 mode) is 2047 + K."""
    a, words, palette = _ones_case(oracle, inner, 0)
    got = oracle.gemm(a, words, 5, palette, 32, mode="f16-chain")
    assert (got == 2048.0).all(), got[0, :4]
    exact = oracle.gemm(a, words, 5, palette, 32, mode="f64")
    assert (exact == 2047.0 + inner).all()


def test_f16_chain_closed_form_large_term_last():
    """K - 1 ones first (exact up to 2048), then 2048: the chain holds K - 1
    and rounds 2047 + K once, to the even neighbour (64 -> 2112, not 2111);
    the same inputs in the other order give 2048, so the order is pinned."""
    from oracle import pko
    a, words, palette = _ones_case(pko, 64, 63)
    got = pko.gemm(a, words, 5, palette, 32, mode="f16-chain")
    assert (got == 2112.0).all(), got[0, :4]
    assert np.float16(2111.0) == 2112.0  # the tie 2111 rounds to even


def test_f32_chain_keeps_the_small_terms():
    """The reference's fp32 GEMM (f32 accumulator, gemm.ts:2356-2599) sums
    2048 + 63 ones exactly: 2111."""
    from oracle import pko
    a, words, _ = _ones_case(pko, 64, 0)
    got = pko.gemm(a.astype(np.float32), words, 5, np.ones((1, 32), np.float32), 32, mode="f32-chain")
    assert (got == 2111.0).all()


# The fp32 profile (encoder.ts:947-1165): the same restatements with f32
# storage between dispatches against the oracle's f32 chain; only f32
# arithmetic in the oracle's LayerNorm, attention and convolution separates
# them (measured 2e-6 for the layer and 1e-7 for the front end, norm-wise),
# so the bar is 1e-4, and a planted mistake
# still misses it by orders of magnitude.
BAR32 = 1e-4


def test_encoder_layer_f32_storage_matches_torch_restatement(oracle, one_layer):
    s = one_layer
    got = oracle.encoder_layer(s.x, s.layers[0], s.valid, batch=s.batch, frames=s.frames, gemm_mode="f64",
                               threads=THREADS, dtype=np.float32)
    assert got.dtype == np.float32
    want = torch_encoder_layer(s.x, s.layers[0], s.valid, s.batch, s.frames, storage="f32")
    norm, worst = oracle.relative_errors(got, want)
    print(f"f32 encoder layer vs torch float64 restatement: norm {norm:.2e} max {worst:.2e}")
    assert norm <= BAR32, (norm, worst)
    wrong = torch_encoder_layer(s.x, s.layers[0], s.valid, s.batch, s.frames, mistake="swapped-norm", storage="f32")
    assert oracle.relative_errors(got, wrong)[0] > 10 * BAR32


def test_front_end_f32_storage_matches_torch_restatement(oracle, front_case):
    s = front_case
    got = oracle.encoder_front_end(s.features, s.subsampling, s.feature_lengths, gemm_mode="f64", threads=THREADS,
                                   dtype=np.float32)
    assert got.dtype == np.float32
    want = torch_front_end(oracle, s.features, s.subsampling, s.feature_lengths, storage="f32")
    norm, worst = oracle.relative_errors(got, want)
    print(f"f32 front end vs torch float64 restatement: norm {norm:.2e} max {worst:.2e}")
    assert norm <= BAR32, (norm, worst)
    wrong = torch_front_end(oracle, s.features, s.subsampling, s.feature_lengths, mistake="time-major-flatten",
                            storage="f32")
    assert oracle.relative_errors(got, wrong)[0] > 10 * BAR32

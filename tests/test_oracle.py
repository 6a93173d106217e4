"""Pins for the CPU oracle (oracle/pk_oracle.c) before it is trusted as the
checker of the HIP kernels.

Each check is independent of the formula it pins: the reference's own
known-answer vectors, Python big-integer bit arithmetic, numpy's binary16
conversion, exact integer arithmetic, closed forms and brute force.
"""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def kats():
    with open(os.path.join(GOLDEN, "palette_kats.json")) as f:
        return json.load(f)


def big_int_codes(words, bits, count):
    """Decode a group through one little-endian Python integer."""
    value = 0
    for q, w in enumerate(words):
        value |= int(w) << (32 * q)
    mask = (1 << bits) - 1
    return [(value >> (i * bits)) & mask for i in range(count)]


# ---------------------------------------------------------------- packing


@pytest.mark.parametrize("case", range(2))
def test_pack_matches_reference_known_answers(oracle, case):
    """model/tests/test_convert.py:447-479."""
    kat = kats()["pack_lsb"][case]
    codes = np.array(kat["codes"], dtype=np.uint8)
    words = oracle.pack_codes(codes, kat["bits"])
    assert words.dtype == np.dtype("<u4")
    assert words.shape == (1, len(kat["words"]))
    assert [int(w) for w in words[0]] == kat["words"]
    assert words[0, 0].tobytes() == int(kat["words"][0]).to_bytes(4, "little")
    np.testing.assert_array_equal(oracle.unpack_codes(words, kat["bits"]), codes)


@pytest.mark.parametrize("bits", [5, 6])
def test_unpack_matches_big_integer_bit_positions(oracle, bits):
    rng = np.random.default_rng(bits)
    cpg = oracle.codes_per_group(bits)
    words = rng.integers(0, 2**32, size=(500, oracle.words_per_group(bits)), dtype=np.uint64).astype("<u4")
    codes = oracle.unpack_codes(words, bits).reshape(-1, cpg)
    for g in range(words.shape[0]):
        assert list(codes[g]) == big_int_codes(words[g], bits, cpg)


@pytest.mark.parametrize("bits", [5, 6])
def test_every_code_position_and_value_round_trips(oracle, bits):
    cpg = oracle.codes_per_group(bits)
    for position in range(cpg):
        for value in range(1 << bits):
            codes = np.zeros(cpg, dtype=np.uint8)
            codes[position] = value
            words = oracle.pack_codes(codes, bits)
            assert big_int_codes(words[0], bits, cpg) == list(codes)
            np.testing.assert_array_equal(oracle.unpack_codes(words, bits), codes)


@pytest.mark.parametrize("bits,straddlers", [(5, [6, 12, 19, 25]), (6, [5, 10])])
def test_word_straddling_codes(oracle, bits, straddlers):
    """Codes whose bits cross a u32 boundary keep their high bits in the next
    word (convert.py:2152-2155)."""
    cpg = oracle.codes_per_group(bits)
    assert [i for i in range(cpg) if (i * bits) % 32 + bits > 32] == straddlers
    full = np.full(cpg, (1 << bits) - 1, dtype=np.uint8)
    words = oracle.pack_codes(full, bits)
    assert all(int(w) == 0xFFFFFFFF for w in words[0])  # 160 or 96 bits, all used


@pytest.mark.parametrize("bits", [5, 6])
def test_random_round_trip(oracle, bits):
    rng = np.random.default_rng(10 + bits)
    codes = rng.integers(0, 1 << bits, size=64 * 96, dtype=np.uint8)
    np.testing.assert_array_equal(oracle.unpack_codes(oracle.pack_codes(codes, bits), bits), codes)


def test_pack_rejects_out_of_range_and_unaligned(oracle):
    with pytest.raises(ValueError):
        oracle.pack_codes(np.array([32] + [0] * 31, dtype=np.uint8), 5)
    with pytest.raises(ValueError):
        oracle.pack_codes(np.zeros(31, dtype=np.uint8), 5)


def test_k_major_output_group_fixture(oracle):
    """model/tests/test_convert.py:481-511: the codes of a [K, N] matrix are
    flattened k outer, n inner, across palette groups."""
    fx = kats()["k_major_output_groups"]
    codes = np.array(fx["expected_codes"], dtype=np.uint8)
    words = oracle.pack_codes(codes, fx["bits"])
    assert list(words.shape) == fx["packed_shape"]
    unpacked = oracle.unpack_codes(words, fx["bits"])
    dense = np.array(fx["dense"])
    palettes = np.array(fx["palettes"])
    k, n = dense.shape
    width = fx["output_group_width"]
    for kk in range(k):
        for nn in range(n):
            assert palettes[nn // width][unpacked[kk * n + nn]] == dense[kk, nn]


# ---------------------------------------------------------------- binary16


def test_f16_rounding_every_value_and_midpoint(oracle):
    all_bits = np.arange(0x10000, dtype=np.uint16)
    values = all_bits.view(np.float16)
    finite = np.isfinite(values)
    for b in all_bits[finite][::7]:
        v = float(np.uint16(b).view(np.float16))
        assert oracle.f64_to_f16_bits(v) == int(b)
        assert oracle.f16_bits_to_f64(int(b)) == v
    # midpoints and their neighbours, against numpy's round-to-nearest-even
    pos = values[finite & (values >= 0)].astype(np.float64)
    pos = np.sort(pos)
    mids = (pos[:-1] + pos[1:]) / 2
    probes = np.concatenate([mids, np.nextafter(mids, 0), np.nextafter(mids, np.inf)])
    probes = np.concatenate([probes, -probes, [65519.0, 65520.0, 70000.0, 2.0**-25, 2.0**-26, 3 * 2.0**-26]])
    for p in probes[::5]:
        assert oracle.f64_to_f16_bits(p) == int(np.float16(p).view(np.uint16)), p


def test_f16_round_trip_shortcut_matches_numpy(oracle):
    """pko_round_f16 (the chain GEMM's per-step rounding) against numpy's
    binary16 cast: every midpoint and its neighbours, subnormals, the
    overflow threshold, signed zeros and random doubles."""
    values = np.arange(0x10000, dtype=np.uint16).view(np.float16)
    pos = np.sort(values[np.isfinite(values) & (values >= 0)].astype(np.float64))
    mids = (pos[:-1] + pos[1:]) / 2
    probes = np.concatenate([pos, mids, np.nextafter(mids, 0), np.nextafter(mids, np.inf)])
    rng = np.random.default_rng(5)
    probes = np.concatenate([probes, rng.standard_normal(4000) * 10.0 ** rng.uniform(-9, 5, 4000),
                             [65519.0, 65520.0, 65535.9, 1e300, 2.0**-25, 2.0**-26, 3 * 2.0**-26, 0.0, -0.0]])
    probes = np.concatenate([probes, -probes])
    for p in probes[::3]:
        with np.errstate(over="ignore"):
            want = float(np.float64(np.float16(p)))
        got = oracle.round_f16(p)
        assert got == want and np.signbit(got) == np.signbit(want), (p, got, want)


# ---------------------------------------------------------------- geometry


def test_palette_group_closed_form(oracle):
    for groups, group_columns in [(1, 4096), (3, 1024), (4, 16)]:
        for n in range(0, groups * group_columns, 7):
            assert oracle.palette_group(n, group_columns, groups) == min(n // group_columns, groups - 1)


@pytest.mark.parametrize("tile_columns,columns", [(256, 512), (128, 256)])
def test_tile_major_index_is_a_tile_contiguous_bijection(oracle, tile_columns, columns):
    """runtime-plan.ts:454-490 and the invariants of
    test/model/palette-expander.test.ts:147-247."""
    inner = 64
    seen = np.zeros(inner * columns, dtype=bool)
    for s in range(inner * columns):
        p = oracle.tile_major_index(s, inner, columns, tile_columns)
        assert not seen[p]
        seen[p] = True
        k, n = divmod(s, columns)
        tile = (n // tile_columns) * (inner // 32) + k // 32
        assert tile * 32 * tile_columns <= p < (tile + 1) * 32 * tile_columns
        if s % 4 == 0:
            assert p % 4 == 0
    assert seen.all()


# ---------------------------------------------------------------- expansion


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("bits,groups,columns", [(5, 1, 256), (5, 3, 768), (6, 1, 256), (6, 4, 512)])
def test_expand_one_hot_palette_recovers_codes(oracle, dtype, bits, groups, columns):
    rng = np.random.default_rng(bits * 10 + groups)
    inner = 64
    codes = rng.integers(0, 1 << bits, size=(inner, columns), dtype=np.uint8)
    words = oracle.pack_codes(codes, bits)
    entries = 1 << bits
    palette = (100 * np.arange(groups)[:, None] + np.arange(entries)[None, :]).astype(dtype)
    dense = oracle.expand(words, bits, inner, columns, palette)
    group_of = np.minimum(np.arange(columns) // (columns // groups), groups - 1)
    np.testing.assert_array_equal(dense, (100 * group_of[None, :] + codes).astype(dtype))
    if columns % (256 if dtype == np.float16 else 128) == 0:
        tiled = oracle.expand(words, bits, inner, columns, palette, tile_major=True)
        tile_columns = 256 if dtype == np.float16 else 128
        for s in range(0, inner * columns, 97):
            assert tiled[oracle.tile_major_index(s, inner, columns, tile_columns)] == dense.reshape(-1)[s]


# ---------------------------------------------------------------- GEMM


def _case(rng, rows, inner, columns, bits, dtype, groups=1, int_values=False):
    codes = rng.integers(0, 1 << bits, size=(inner, columns), dtype=np.uint8)
    if int_values:
        a = rng.integers(-2, 3, size=(rows, inner)).astype(dtype)
        palette = rng.integers(-3, 4, size=(groups, 1 << bits)).astype(dtype)
    else:
        a = rng.standard_normal((rows, inner)).astype(dtype)
        palette = (rng.standard_normal((groups, 1 << bits)) * 0.02).astype(dtype)
    return a, codes, palette


def _dense(codes, palette):
    groups = palette.shape[0]
    columns = codes.shape[1]
    g = np.minimum(np.arange(columns) // (columns // groups), groups - 1)
    return palette[g[None, :], codes].astype(np.float64)


@pytest.mark.parametrize("bits,groups", [(5, 1), (6, 3)])
def test_gemm_exact_on_integer_inputs(oracle, bits, groups):
    """Small integers keep every product and partial sum exact in binary16,
    so all three modes equal the integer matmul; the non-square shape
    catches transposed operands and the integer result any dropped term or
    wrong sign."""
    rng = np.random.default_rng(7)
    rows, inner, columns = 5, 64, 96
    a, codes, palette = _case(rng, rows, inner, columns, bits, np.float16, groups, int_values=True)
    words = oracle.pack_codes(codes, bits)
    want = a.astype(np.float64) @ _dense(codes, palette)
    for mode in ["f16-chain", "f32-chain", "f64"]:
        got = oracle.gemm(a, words, bits, palette, columns, mode=mode)
        np.testing.assert_array_equal(got.astype(np.float64), want, err_msg=mode)


def test_gemm_constant_palette_is_row_sum(oracle):
    rng = np.random.default_rng(3)
    a = rng.standard_normal((7, 128)).astype(np.float32)
    codes = rng.integers(0, 32, size=(128, 64), dtype=np.uint8)
    palette = np.full((1, 32), 0.375, dtype=np.float32)
    got = oracle.gemm(a, oracle.pack_codes(codes, 5), 5, palette, 64, mode="f64")
    want = 0.375 * a.astype(np.float64).sum(axis=1, keepdims=True)
    np.testing.assert_allclose(got, np.broadcast_to(want, got.shape), rtol=1e-12, atol=1e-12)


def test_gemm_brute_force_tiny(oracle):
    rng = np.random.default_rng(11)
    rows, inner, columns, bits = 3, 32, 32, 5
    a, codes, palette = _case(rng, rows, inner, columns, bits, np.float32)
    words = oracle.pack_codes(codes, bits)
    # decode through big integers, independent of the oracle's unpack
    flat = []
    for g in range(words.shape[0]):
        flat += big_int_codes(words[g], bits, 32)
    w = [[float(palette[0][flat[k * columns + n]]) for n in range(columns)] for k in range(inner)]
    got = oracle.gemm(a, words, bits, palette, columns, mode="f64")
    for m in range(rows):
        for n in range(columns):
            s = 0.0
            for k in range(inner):
                s += float(a[m, k]) * w[k][n]
            assert abs(got[m, n] - s) <= 1e-12 * max(1.0, abs(s))


def test_f16_chain_is_one_rounding_per_step(oracle):
    """Increasing-k binary16 accumulator with a fused multiply-add
    (gemm.ts:1445-1453): emulate it with numpy's float64->float16 rounding."""
    rng = np.random.default_rng(5)
    rows, inner, columns, bits = 2, 64, 32, 5
    a, codes, palette = _case(rng, rows, inner, columns, bits, np.float16)
    words = oracle.pack_codes(codes, bits)
    w = _dense(codes, palette)
    got = oracle.gemm(a, words, bits, palette, columns, mode="f16-chain")
    for m in range(rows):
        for n in range(columns):
            acc = np.float16(0.0)
            for k in range(inner):
                acc = np.float16(np.float64(a[m, k]) * w[k, n] + np.float64(acc))
            assert got[m, n].view(np.uint16) == acc.view(np.uint16)


def test_f32_chain_is_increasing_k_fma(oracle):
    rng = np.random.default_rng(6)
    rows, inner, columns, bits = 2, 64, 32, 6
    a, codes, palette = _case(rng, rows, inner, columns, bits, np.float32)
    words = oracle.pack_codes(codes, bits)
    w = _dense(codes, palette)
    got = oracle.gemm(a, words, bits, palette, columns, mode="f32-chain")
    for m in range(rows):
        for n in range(columns):
            acc = np.float32(0.0)
            for k in range(inner):
                acc = np.float32(np.float64(a[m, k]) * w[k, n] + np.float64(acc))
            assert got[m, n] == acc


def test_epilogue_order_and_closed_forms(oracle):
    """bias -> activation -> residual + scale * value (gemm.ts:2006-2044)."""
    rng = np.random.default_rng(9)
    rows, inner, columns, bits = 4, 64, 64, 5
    a, codes, palette = _case(rng, rows, inner, columns, bits, np.float32)
    words = oracle.pack_codes(codes, bits)
    plain = oracle.gemm(a, words, bits, palette, columns, mode="f64")
    bias = (rng.standard_normal(columns) * 0.5).astype(np.float32)
    residual = rng.standard_normal((rows, columns)).astype(np.float32)

    def silu(v):
        b = np.clip(v, -20, 20)
        return v / (1 + np.exp(-b))

    got = oracle.gemm(a, words, bits, palette, columns, bias=bias, activation="silu", mode="f64")
    np.testing.assert_allclose(got, silu(plain + bias), rtol=1e-12, atol=1e-14)
    got = oracle.gemm(a, words, bits, palette, columns, bias=bias, activation="relu", mode="f64")
    np.testing.assert_allclose(got, np.maximum(plain + bias, 0), rtol=1e-12, atol=1e-14)
    got = oracle.gemm(a, words, bits, palette, columns, residual=residual, residual_scale=0.5,
                      activation="silu", mode="f64")
    np.testing.assert_allclose(got, residual + 0.5 * silu(plain), rtol=1e-12, atol=1e-14)
    # the bias must act before the activation: a large negative bias zeroes relu
    got = oracle.gemm(a, words, bits, palette, columns, bias=np.full(columns, -1e3, np.float32),
                      activation="relu", mode="f64")
    assert np.all(got == 0)
    # the f32 epilogue matches the double one to f32 precision
    got32 = oracle.gemm(a, words, bits, palette, columns, residual=residual, residual_scale=1.0,
                        activation="silu", mode="f32-chain")
    np.testing.assert_allclose(got32, residual + silu(plain), rtol=1e-5, atol=1e-6)


def test_silu_clamps_its_exponent(oracle):
    """SiLU evaluates exp(-clamp(v, -20, 20)) (gemm.ts:2020-2026): for very
    negative v it is v/(1+e^20), not the exact ~0."""
    rows, inner, columns = 1, 32, 32
    a = np.ones((rows, inner), dtype=np.float32)
    codes = np.zeros((inner, columns), dtype=np.uint8)
    palette = np.zeros((1, 32), dtype=np.float32)
    palette[0, 0] = -2.0  # every output = -64
    got = oracle.gemm(a, oracle.pack_codes(codes, 5), 5, palette, columns, activation="silu", mode="f64")
    np.testing.assert_allclose(got, -64.0 / (1 + np.exp(20.0)), rtol=1e-12)


def test_threads_do_not_change_results(oracle):
    rng = np.random.default_rng(2)
    a, codes, palette = _case(rng, 37, 96, 64, 6, np.float16)
    words = oracle.pack_codes(codes, 6)
    one = oracle.gemm(a, words, 6, palette, 64, mode="f16-chain", threads=1)
    many = oracle.gemm(a, words, 6, palette, 64, mode="f16-chain", threads=5)
    np.testing.assert_array_equal(one.view(np.uint16), many.view(np.uint16))


# ------------------------------------------------------ conformer conv tail


def _conv_case(rng, batch, frames, channels, dtype=np.float32):
    pointwise = rng.standard_normal((batch * frames, 2 * channels)).astype(dtype)
    weights = (rng.standard_normal((9, channels)) * 0.3).astype(dtype)
    scale = (1.0 + 0.1 * rng.standard_normal(channels)).astype(np.float32)
    shift = (0.1 * rng.standard_normal(channels)).astype(np.float32)
    return pointwise, weights, scale, shift


def _torch_conv_module(pointwise, weights, scale, shift, valid, batch, frames):
    """The same tail through torch's library routines in float64: glu over the
    channel axis, masking of frames past each valid length, a same-padded
    grouped conv1d, then silu."""
    import torch
    import torch.nn.functional as F

    channels = weights.shape[1]
    x = torch.from_numpy(pointwise.astype(np.float64)).reshape(batch, frames, 2 * channels)
    glu = F.glu(x, dim=-1)
    live = torch.arange(frames)[None, :] < torch.tensor(valid.astype(np.int64))[:, None]
    glu = glu * live[:, :, None]
    kernel = torch.from_numpy(weights.astype(np.float64)).t().reshape(channels, 1, 9)
    conv = F.conv1d(glu.transpose(1, 2), kernel, padding=4, groups=channels).transpose(1, 2)
    affine = conv * torch.from_numpy(scale.astype(np.float64)) + torch.from_numpy(shift.astype(np.float64))
    return F.silu(affine).reshape(batch * frames, channels).numpy()


def test_conv_matches_torch_grouped_conv1d(oracle):
    """glu (value half first), per-frame masking, same-padded depthwise k9
    (conformer-conv.ts:505-560) equal torch's glu + conv1d(groups=C)."""
    rng = np.random.default_rng(10)
    batch, frames, channels = 3, 23, 16
    pointwise, weights, scale, shift = _conv_case(rng, batch, frames, channels)
    valid = np.array([23, 9, 30], dtype=np.uint32)
    want = _torch_conv_module(pointwise, weights, scale, shift, valid, batch, frames)
    got64 = oracle.conformer_conv(pointwise, weights, scale, shift, valid, batch=batch, frames=frames, mode="f64")
    np.testing.assert_allclose(got64, want, rtol=2e-7, atol=1e-7)
    got32 = oracle.conformer_conv(pointwise, weights, scale, shift, valid, batch=batch, frames=frames)
    np.testing.assert_allclose(got32, want, rtol=2e-6, atol=2e-6)


def test_conv_f16_output_is_one_rounding_of_the_f64_result(oracle):
    rng = np.random.default_rng(11)
    batch, frames, channels = 2, 17, 8
    pointwise, weights, scale, shift = _conv_case(rng, batch, frames, channels, np.float16)
    valid = np.array([17, 12], dtype=np.uint32)
    want = _torch_conv_module(pointwise, weights, scale, shift, valid, batch, frames).astype(np.float16)
    got = oracle.conformer_conv(pointwise, weights, scale, shift, valid, batch=batch, frames=frames, mode="f64")
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("tap", [0, 2, 4, 8])
def test_conv_one_hot_tap_reads_frame_minus_four_plus_tap(oracle, tap):
    """With zero gates (sigmoid 1/2 exactly), unit scale, zero shift and the
    single tap `tap` set to one, the pre-activation at frame f is exactly
    value(f - 4 + tap) / 2, or 0 outside the sequence."""
    batch, frames, channels = 1, 12, 8
    value = np.arange(frames * channels, dtype=np.float32).reshape(frames, channels) % 7 - 3
    pointwise = np.concatenate([value, np.zeros_like(value)], axis=1)
    weights = np.zeros((9, channels), np.float32)
    weights[tap] = 1.0
    got = oracle.conformer_conv(pointwise, weights, np.ones(channels, np.float32), np.zeros(channels, np.float32),
                                np.array([frames], np.uint32), batch=batch, frames=frames)
    pre = np.zeros_like(value, dtype=np.float64)
    for f in range(frames):
        t = f - 4 + tap
        if 0 <= t < frames:
            pre[f] = value[t] / 2.0
    np.testing.assert_allclose(got, pre / (1.0 + np.exp(-pre)), rtol=1e-6, atol=1e-7)


def test_conv_gate_sigmoid_clamps_at_twenty(oracle):
    """sigmoid(gate) uses exp(-clamp(gate, -20, 20)) (conformer-conv.ts:489-492):
    a gate of -30 gives 1/(1+e^20), not 1/(1+e^30)."""
    channels = 8
    pointwise = np.zeros((1, 2 * channels), np.float64)
    pointwise[0, :channels] = 1e6
    pointwise[0, channels:] = -30.0
    weights = np.zeros((9, channels))
    weights[4] = 1.0
    pre = 1e6 / (1.0 + np.exp(20.0))
    for mode in ("f64", "f32-chain"):
        got = oracle.conformer_conv(pointwise.astype(np.float32), weights.astype(np.float32),
                                    np.ones(channels, np.float32), np.zeros(channels, np.float32),
                                    np.array([1], np.uint32), batch=1, frames=1, mode=mode)
        np.testing.assert_allclose(got, pre / (1.0 + np.exp(-pre)), rtol=1e-5)


def test_conv_frames_past_valid_length_read_zero(oracle):
    """A zero valid length leaves only silu(shift) at every frame; lengths at or
    beyond the frame count change nothing."""
    rng = np.random.default_rng(12)
    batch, frames, channels = 2, 10, 8
    pointwise, weights, scale, shift = _conv_case(rng, batch, frames, channels)
    got = oracle.conformer_conv(pointwise, weights, scale, shift, np.array([0, 0], np.uint32),
                                batch=batch, frames=frames, mode="f64")
    s = shift.astype(np.float64)
    np.testing.assert_allclose(got, np.tile(s / (1 + np.exp(-s)), (batch * frames, 1)), rtol=1e-6)
    full = oracle.conformer_conv(pointwise, weights, scale, shift, np.array([frames, frames], np.uint32),
                                 batch=batch, frames=frames)
    beyond = oracle.conformer_conv(pointwise, weights, scale, shift, np.array([frames + 5, 1 << 30], np.uint32),
                                   batch=batch, frames=frames)
    np.testing.assert_array_equal(full, beyond)


def test_conv_batch_items_are_independent(oracle):
    rng = np.random.default_rng(13)
    batch, frames, channels = 2, 9, 8
    pointwise, weights, scale, shift = _conv_case(rng, batch, frames, channels)
    valid = np.array([9, 7], np.uint32)
    one = oracle.conformer_conv(pointwise, weights, scale, shift, valid, batch=batch, frames=frames)
    changed = pointwise.copy()
    changed[frames:] = rng.standard_normal(changed[frames:].shape)
    two = oracle.conformer_conv(changed, weights, scale, shift, valid, batch=batch, frames=frames)
    np.testing.assert_array_equal(one[:frames], two[:frames])
    assert not np.array_equal(one[frames:], two[frames:])


def test_glu_matches_torch_glu(oracle):
    """value half first, gate half second (conformer-conv.ts:520-535), the
    same as torch.nn.functional.glu over the channel axis."""
    import torch
    import torch.nn.functional as F

    rng = np.random.default_rng(14)
    x = rng.standard_normal((37, 48)) * 3
    want = F.glu(torch.from_numpy(x), dim=-1).numpy()
    np.testing.assert_allclose(oracle.glu(x, mode="f64"), want, rtol=1e-14, atol=1e-15)
    np.testing.assert_allclose(oracle.glu(x.astype(np.float32)), want, rtol=2e-6, atol=1e-7)
    got16 = oracle.glu(x.astype(np.float16), mode="f64")
    want16 = F.glu(torch.from_numpy(x.astype(np.float16).astype(np.float64)), dim=-1).numpy().astype(np.float16)
    np.testing.assert_array_equal(got16.view(np.uint16), want16.view(np.uint16))


def test_glu_gate_clamp(oracle):
    x = np.array([[1e6, -30.0]])
    for mode in ("f64", "f32-chain"):
        np.testing.assert_allclose(oracle.glu(x.astype(np.float32) if mode != "f64" else x, mode=mode),
                                   [[1e6 / (1 + np.exp(20.0))]], rtol=1e-5)


def test_glu_is_the_conv_tail_with_a_center_tap(oracle):
    """With the center tap 1, scale 1 and shift 0 the tail is silu(glu): the
    two oracle functions agree on the GLU they form."""
    rng = np.random.default_rng(15)
    x = rng.standard_normal((20, 16)).astype(np.float32)
    w = np.zeros((9, 8), np.float32)
    w[4] = 1.0
    tail = oracle.conformer_conv(x, w, np.ones(8, np.float32), np.zeros(8, np.float32), np.array([20], np.uint32),
                                 batch=1, frames=20, mode="f64")
    g = oracle.glu(x.astype(np.float64), mode="f64")
    np.testing.assert_allclose(tail, g / (1 + np.exp(-g)), rtol=1e-6)


# ------------------------------------------ relative-position attention


def test_relative_position_table_known_answers(workloads):
    """model/tests/test_convert.py:799-815: the T=3, C=4 table by its closed
    form, the 375 x 1024 table's zero-distance row all sin 0 / cos 0."""
    table = workloads.relative_position_table(3, 4)
    positions = np.array([2, 1, 0, -1, -2], dtype=np.float32).reshape(-1, 1)
    div = np.exp(np.arange(0, 4, 2, dtype=np.float32) * np.float32(-(np.log(10_000.0) / 4)))
    want = np.empty((5, 4), np.float32)
    want[:, 0::2] = np.sin(positions * div)
    want[:, 1::2] = np.cos(positions * div)
    np.testing.assert_array_equal(table, want)
    full = workloads.relative_position_table(188)
    assert full.shape == (375, 1024)
    np.testing.assert_array_equal(full[187, 0::2], 0)
    np.testing.assert_array_equal(full[187, 1::2], 1)


def test_pack_projected_positions_known_answers(workloads):
    """model/tests/test_convert.py:828-840: rows inside head vectors."""
    projected = np.arange(16, dtype=np.float16).reshape(2, 8)
    packed = workloads.pack_projected_positions(projected, heads=2)
    assert packed.shape == (2, 1, 2, 4)
    np.testing.assert_array_equal(packed[0, 0, 0], projected[0, 0:4])
    np.testing.assert_array_equal(packed[0, 0, 1], projected[1, 0:4])
    np.testing.assert_array_equal(packed[1, 0, 0], projected[0, 4:8])
    np.testing.assert_array_equal(packed[1, 0, 1], projected[1, 4:8])


def _torch_relative_attention(case):
    """Float64 restatement through torch: scores from einsum over heads with
    the relative keys gathered by index T-1-q+k, a -inf mask, torch.softmax,
    a batched matmul with V, zero rows past the valid length."""
    import torch

    B, T = case.batch, case.frames
    x = torch.from_numpy(case.qkv.astype(np.float64)).reshape(B, T, 3, 8, 128)
    q, k, v = x[:, :, 0], x[:, :, 1], x[:, :, 2]                    # [B, T, H, D]
    u = torch.from_numpy(case.bias_u.astype(np.float64))
    w = torch.from_numpy(case.bias_v.astype(np.float64))
    pos = torch.from_numpy(case.positions.astype(np.float64)).reshape(2 * T - 1, 8, 128)
    idx = (T - 1 - torch.arange(T)[:, None] + torch.arange(T)[None, :])  # [Tq, Tk]
    rel = pos[idx]                                                      # [Tq, Tk, H, D]
    ac = torch.einsum("bqhd,bkhd->bhqk", q + u, k)
    bd = torch.einsum("bqhd,qkhd->bhqk", q + w, rel)
    scores = (ac + bd) / np.sqrt(128.0)
    out = torch.zeros(B, T, 8, 128, dtype=torch.float64)
    for b in range(B):
        live = int(min(case.valid[b], T))
        if live == 0:
            continue
        p = torch.softmax(scores[b, :, :live, :live], dim=-1)          # [H, live, live]
        ctx = torch.matmul(p, v[b, :live].permute(1, 0, 2).contiguous())  # [H, live, D]
        out[b, :live] = ctx.permute(1, 0, 2)
    return out.reshape(B * T, 1024).numpy()


def _attend(oracle, case, mode):
    return oracle.relative_attention(case.qkv, case.packed_positions, case.bias_u, case.bias_v, case.valid,
                                     batch=case.batch, frames=case.frames, mode=mode)


def test_relative_attention_matches_torch(oracle, workloads):
    case = workloads.attention_case(20, 3, 13, dtype=np.float64, valid=[13, 7, 0])
    want = _torch_relative_attention(case)
    np.testing.assert_allclose(_attend(oracle, case, "f64"), want, rtol=1e-11, atol=1e-13)
    case32 = workloads.AttentionCase(case.qkv.astype(np.float32), case.positions.astype(np.float32), case.bias_u,
                                     case.bias_v, case.valid, case.batch, case.frames)
    np.testing.assert_allclose(_attend(oracle, case32, "f32-chain"), want, rtol=2e-5, atol=2e-6)


def test_relative_attention_without_positions_is_plain_attention(oracle, workloads):
    """Zero positions and biases leave scaled dot-product attention (torch's
    scaled_dot_product_attention, default scale 1/sqrt(128))."""
    import torch
    import torch.nn.functional as F

    case = workloads.attention_case(21, 1, 9, dtype=np.float64, valid=[9])
    case.positions[:] = 0
    case.bias_u[:] = 0
    case.bias_v[:] = 0
    x = torch.from_numpy(case.qkv).reshape(9, 3, 8, 128).permute(1, 2, 0, 3)  # [3, H, T, D]
    want = F.scaled_dot_product_attention(x[0], x[1], x[2]).permute(1, 0, 2).reshape(9, 1024).numpy()
    np.testing.assert_allclose(_attend(oracle, case, "f64"), want, rtol=1e-11, atol=1e-13)


def test_relative_shift_direction(oracle, workloads):
    """Q = K = 0, u = 0 and v = beta on one channel of head 0 with R[p] = p on
    that channel: score(q, k) = beta (T-1-q+k) / sqrt(128), so every query's
    weights are softmax(beta k / sqrt(128)) over the keys (the q term
    cancels). Reversing the relative index would flip the sign of k."""
    T, beta = 6, 3.0
    case = workloads.attention_case(22, 1, T, dtype=np.float64, valid=[T])
    case.qkv[:, :2048] = 0
    case.bias_u[:] = 0
    case.bias_v[:] = 0
    case.bias_v[0, 5] = beta
    case.positions[:] = 0
    case.positions[:, 5] = np.arange(2 * T - 1)
    got = _attend(oracle, case, "f64")
    w = np.exp(beta * np.arange(T) / np.sqrt(128.0))
    w /= w.sum()
    want_head0 = w @ case.qkv[:, 2048:2048 + 128]
    for q in range(T):
        np.testing.assert_allclose(got[q, :128], want_head0, rtol=1e-12)
    # the other heads see uniform weights
    np.testing.assert_allclose(got[0, 128:256], case.qkv[:, 2048 + 128:2048 + 256].mean(axis=0), rtol=1e-12)


def test_relative_attention_one_key_and_empty_windows(oracle, workloads):
    case = workloads.attention_case(23, 2, 5, dtype=np.float32, valid=[1, 0])
    got = _attend(oracle, case, "f32-chain")
    np.testing.assert_array_equal(got[0], case.qkv[0, 2048:])  # one key: probability exactly 1
    assert np.all(got[1:5] == 0) and np.all(got[5:] == 0)


# ------------------------------------------------------------- LayerNorm


def test_layernorm_matches_torch(oracle):
    import torch
    import torch.nn.functional as F

    rng = np.random.default_rng(30)
    x = rng.standard_normal((19, 1024)) * 3 + 0.7
    gamma = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(1024)).astype(np.float32)
    want = F.layer_norm(torch.from_numpy(x), (1024,), torch.from_numpy(gamma.astype(np.float64)),
                        torch.from_numpy(beta.astype(np.float64)), eps=1e-5).numpy()
    np.testing.assert_allclose(oracle.layernorm(x, gamma, beta, mode="f64"), want, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(oracle.layernorm(x.astype(np.float32), gamma, beta), want, rtol=1e-4, atol=1e-4)


def test_layernorm_constant_rows_give_beta(oracle):
    """Zero variance: every output is beta (rsqrt(epsilon) times zero)."""
    x = np.full((3, 64), 2.5, np.float32)
    gamma = np.linspace(0.5, 2, 64, dtype=np.float32)
    beta = np.linspace(-1, 1, 64, dtype=np.float32)
    for mode in ("f32-chain", "f64"):
        np.testing.assert_allclose(oracle.layernorm(x, gamma, beta, mode=mode), np.tile(beta, (3, 1)), atol=1e-6)


def test_layernorm_unit_affine_moments(oracle):
    """gamma = 1, beta = 0: each row has mean 0 and variance var / (var + eps)."""
    rng = np.random.default_rng(31)
    x = rng.standard_normal((5, 256)) * np.array([[0.01], [0.1], [1], [10], [100]])
    got = oracle.layernorm(x, np.ones(256, np.float32), np.zeros(256, np.float32), mode="f64")
    var = x.var(axis=1)
    np.testing.assert_allclose(got.mean(axis=1), 0, atol=1e-12)
    # E[x^2] - mean^2 (the reference formula) costs a few 1e-9 at scale 100
    np.testing.assert_allclose(got.var(axis=1), var / (var + 1e-5), rtol=1e-7)


# ---------------------------------------------------------------- subsampling


def test_subsampled_lengths_match_reference_kats(oracle):
    """test/webgpu/subsampling-kernel-shapes.test.ts:27-50."""
    heights, widths = [1501], [128]
    for _ in range(3):
        heights.append(oracle.subsampled_length(heights[-1], 1))
        widths.append(oracle.subsampled_length(widths[-1], 1))
    assert heights == [1501, 751, 376, 188] and widths == [128, 64, 32, 16]
    assert [oracle.subsampled_length(1500, s) for s in (1, 2, 3)] == [750, 375, 188]
    assert [oracle.subsampled_length(799, s) for s in (1, 2, 3)] == [400, 200, 100]
    assert oracle.subsampled_length(1, 3) == 1
    for n in range(1, 300):  # floor((n + 2*1 - 3) / 2) + 1
        assert oracle.subsampled_length(n, 1) == (n + 2 - 3) // 2 + 1


def _torch_subsampling(oracle, features, w0, b0, wd, bd, valid):
    """conv0 + ReLU + depthwise2 with torch.nn.functional.conv2d in float64,
    masking conv0 rows at or past sub(L, 1) and output rows past sub(L, 2)."""
    import torch
    x = torch.tensor(features, dtype=torch.float64).permute(0, 2, 1).unsqueeze(1)  # [B, 1, time, bins]
    channels = w0.shape[-1]
    k0 = torch.tensor(np.asarray(w0, np.float64)).permute(2, 0, 1).unsqueeze(1)  # [C, 1, kh, kw]
    kd = torch.tensor(np.asarray(wd, np.float64)).permute(2, 0, 1).unsqueeze(1)
    c0 = torch.relu(torch.nn.functional.conv2d(x, k0, torch.tensor(b0, dtype=torch.float64), stride=2, padding=1))
    for b, length in enumerate(valid):
        c0[b, :, oracle.subsampled_length(length, 1):] = 0
    out = torch.nn.functional.conv2d(c0, kd, torch.tensor(bd, dtype=torch.float64), stride=2, padding=1,
                                     groups=channels)
    for b, length in enumerate(valid):
        out[b, :, oracle.subsampled_length(length, 2):] = 0
    return out.permute(0, 2, 3, 1).numpy()


def _subsampling_case(seed, batch=3, bins=20, frames=45, channels=8):
    rng = np.random.default_rng(seed)
    features = rng.standard_normal((batch, bins, frames)).astype(np.float32)
    w0 = (rng.standard_normal((3, 3, channels)) * 0.3).astype(np.float16)
    wd = (rng.standard_normal((3, 3, channels)) * 0.3).astype(np.float16)
    b0 = (rng.standard_normal(channels) * 0.1).astype(np.float32)
    bd = (rng.standard_normal(channels) * 0.1).astype(np.float32)
    valid = np.array([frames, 29, 1][:batch], np.uint32)
    return features, w0, b0, wd, bd, valid


def test_subsampling_fused_matches_torch_conv2d(oracle):
    features, w0, b0, wd, bd, valid = _subsampling_case(1)
    want = _torch_subsampling(oracle, features, w0, b0, wd, bd, valid)
    got64 = oracle.subsampling_fused(features, w0, b0, wd, bd, valid, dtype=np.float64)
    assert got64.shape == want.shape == (3, 12, 5, 8)
    np.testing.assert_allclose(got64, want, rtol=0, atol=1e-12)
    got32 = oracle.subsampling_fused(features, w0, b0, wd, bd, valid, dtype=np.float32)
    np.testing.assert_allclose(got32, want, rtol=0, atol=1e-5)
    got16 = oracle.subsampling_fused(features, w0, b0, wd, bd, valid, dtype=np.float16)
    scale = np.abs(want).max()
    assert np.abs(got16.astype(np.float64) - want).max() <= 4e-3 * scale
    # the f16 profile rounds conv0 through f16 before the depthwise sum
    assert not np.array_equal(got16, got32.astype(np.float16))


def test_subsampling_fused_one_hot_taps(oracle):
    """Centre taps of 1 and zero biases: out[y, x] = ReLU(features[4y, 4x])
    on the rows below sub(L, 2), zero past them."""
    features, _, _, _, _, valid = _subsampling_case(2, frames=61, bins=24)
    one_hot = np.zeros((3, 3, 8), np.float16)
    one_hot[1, 1] = 1
    zero = np.zeros(8, np.float32)
    got = oracle.subsampling_fused(features, one_hot, zero, one_hot, zero, valid, dtype=np.float16)
    for b, length in enumerate(valid):
        keep = oracle.subsampled_length(length, 2)
        want = np.maximum(features[b, 0::4, 0::4].T, 0).astype(np.float16)  # [time/4, bins/4]
        np.testing.assert_array_equal(got[b, :keep, :, 0], want[:keep])
        assert not got[b, keep:].any()


def test_subsampling_fused_reads_the_frame_at_an_odd_length(oracle):
    """conv0 is masked by its own valid rows, not the features: for odd L the
    last valid conv0 row reads feature frame L (subsampling.ts:1152-1170)."""
    features, w0, b0, wd, bd, _ = _subsampling_case(3, batch=1, frames=45)
    valid = np.array([29], np.uint32)
    base = oracle.subsampling_fused(features, w0, b0, wd, bd, valid, dtype=np.float64)
    bumped = features.copy()
    bumped[0, :, 29] += 5.0
    assert not np.array_equal(oracle.subsampling_fused(bumped, w0, b0, wd, bd, valid, dtype=np.float64), base)
    later = features.copy()
    later[0, :, 30:] += 5.0
    np.testing.assert_array_equal(oracle.subsampling_fused(later, w0, b0, wd, bd, valid, dtype=np.float64), base)


def test_subsampling_depthwise_matches_torch_conv2d(oracle):
    import torch
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 23, 10, 8))
    w = rng.standard_normal((3, 3, 8)) * 0.3
    bias = (rng.standard_normal(8) * 0.1).astype(np.float32)
    valid = np.array([180, 100, 1], np.uint32)  # raw lengths: stage 3 input rows 23, 13, 1
    got = oracle.subsampling_depthwise(x, w, bias, valid, 3)
    t = torch.tensor(x).permute(0, 3, 1, 2).clone()
    for b, length in enumerate(valid):
        t[b, :, oracle.subsampled_length(length, 2):] = 0
    out = torch.nn.functional.conv2d(t, torch.tensor(w).permute(2, 0, 1).unsqueeze(1),
                                     torch.tensor(bias, dtype=torch.float64), stride=2, padding=1, groups=8)
    for b, length in enumerate(valid):
        out[b, :, oracle.subsampled_length(length, 3):] = 0
    np.testing.assert_allclose(got, out.permute(0, 2, 3, 1).numpy(), rtol=0, atol=1e-12)
    got16 = oracle.subsampling_depthwise(x.astype(np.float16), w, bias, valid, 3)
    np.testing.assert_allclose(got16.astype(np.float64), got, rtol=0, atol=2e-2)


def test_subsampling_mask_zeroes_rows_past_the_length(oracle):
    x = np.arange(2 * 9 * 3 * 4, dtype=np.float32).reshape(2, 9, 3, 4) + 1
    got = oracle.subsampling_mask(x, np.array([60, 33], np.uint32), 3)  # lengths 8 and 5
    np.testing.assert_array_equal(got[0, :8], x[0, :8])
    assert not got[0, 8:].any()
    np.testing.assert_array_equal(got[1, :5], x[1, :5])
    assert not got[1, 5:].any()


# ---------------------------------------------------------------- TDT decoder


def test_decoder_exp_and_tanh_against_the_math_library(oracle):
    rng = np.random.default_rng(7)
    xs = np.concatenate([np.linspace(-20, 20, 4001), rng.uniform(-87, 87, 2000), [0.0, -0.0, 1e-8, -1e-8]])
    for x in xs.astype(np.float32):
        got = oracle.exp_f32(x)
        want = np.exp(np.float64(x))
        assert abs(got - want) <= 2 * np.spacing(np.float32(want)), (x, got, want)
    for x in np.concatenate([np.linspace(-10, 10, 4001), rng.uniform(-10, 10, 2000)]).astype(np.float32):
        assert abs(oracle.tanh_f32(x) - np.tanh(np.float64(x))) <= 2.0 ** -23, x
    assert oracle.tanh_f32(10.0) == pytest.approx(1.0, abs=2.0 ** -23)


def decoder_weights(seed, *, lstm_std=0.03, head_std=0.05):
    rng = np.random.default_rng(seed)

    def n(shape, std, dtype):
        return (rng.standard_normal(shape) * std).astype(dtype)
    return dict(embedding=n((1025, 640), 0.5, np.float16), lstm_weight_l0=n((1280, 2560), lstm_std, np.float16),
                lstm_weight_l1=n((1280, 2560), lstm_std, np.float16), lstm_bias_l0=n(2560, 0.1, np.float32),
                lstm_bias_l1=n(2560, 0.1, np.float32), projector_weight=n((640, 640), 0.04, np.float16),
                projector_bias=n(640, 0.1, np.float32), head_weight=n((640, 1032), head_std, np.float16),
                head_bias=n(1032, 0.1, np.float32))


def torch_lstm_layer(w_k_by_gates, bias, x, h, c):
    """torch.nn.LSTMCell in float64 with the package's k-by-ifgo weight."""
    import torch
    w = torch.tensor(w_k_by_gates.astype(np.float64))
    cell = torch.nn.LSTMCell(640, 640, dtype=torch.float64)
    with torch.no_grad():
        cell.weight_ih.copy_(w[:640].T)
        cell.weight_hh.copy_(w[640:].T)
        cell.bias_ih.copy_(torch.tensor(bias.astype(np.float64)))
        cell.bias_hh.zero_()
        h1, c1 = cell(torch.tensor(x, dtype=torch.float64)[None], (torch.tensor(h, dtype=torch.float64)[None],
                                                                   torch.tensor(c, dtype=torch.float64)[None]))
    return h1[0].numpy(), c1[0].numpy()


def test_decoder_predictor_step_matches_torch_lstm(oracle):
    """One predictor step (two LSTM layers + projector) against torch's
    LSTMCell and a float64 product; the f16 gate chains stay within 1e-2."""
    w = decoder_weights(1)
    rng = np.random.default_rng(2)
    state = (rng.standard_normal((4, 640)) * 0.3).astype(np.float32)
    cand = oracle.tdt_predictor(w, 37, state)
    x = w["embedding"][37].astype(np.float64)
    h0, c0 = torch_lstm_layer(w["lstm_weight_l0"], w["lstm_bias_l0"], x, state[0], state[1])
    h1, c1 = torch_lstm_layer(w["lstm_weight_l1"], w["lstm_bias_l1"], cand[0].astype(np.float64), state[2], state[3])
    proj = cand[2].astype(np.float64) @ w["projector_weight"].astype(np.float64) + w["projector_bias"]
    for got, want in ((cand[0], h0), (cand[1], c0), (cand[2], h1), (cand[3], c1), (cand[4], proj)):
        assert np.abs(got - want).max() <= 1e-2 * max(1.0, np.abs(want).max()), np.abs(got - want).max()
    # the start token: zero input and state, gates are the f16-rounded biases
    start = oracle.tdt_predictor(w, 0, np.zeros((4, 640), np.float32), initial=True)
    g = w["lstm_bias_l0"].astype(np.float16).astype(np.float64)
    sig = lambda v: 1 / (1 + np.exp(-np.clip(v, -20, 20)))  # noqa: E731
    c_closed = sig(g[:640]) * np.tanh(g[1280:1920])
    np.testing.assert_allclose(start[1], c_closed, rtol=0, atol=1e-6)
    np.testing.assert_allclose(start[0], sig(g[1920:]) * np.tanh(c_closed), rtol=0, atol=1e-6)


def test_decoder_joint_matches_a_float64_product(oracle):
    w = decoder_weights(3)
    rng = np.random.default_rng(4)
    row = (rng.standard_normal(640) * 0.5).astype(np.float16)
    proj = (rng.standard_normal(640) * 0.5).astype(np.float32)
    scores, token, duration = oracle.tdt_joint(w, row, proj)
    joint = np.maximum(row.astype(np.float64) + proj, 0)
    want = joint @ w["head_weight"].astype(np.float64) + w["head_bias"]
    assert np.abs(scores[:1030] - want[:1030]).max() <= 2e-2 * np.abs(want).max()
    assert token == int(np.argmax(scores[:1025])) and duration == int(np.argmax(scores[1025:1030]))


def fixed_head(weights, token, duration, *, token_value=5.0):
    """Zero head weights, so every joint returns the bias: `token` (or
    blank, 1024) and `duration` win."""
    w = dict(weights)
    w["head_weight"] = np.zeros((640, 1032), np.float16)
    bias = np.zeros(1032, np.float32)
    bias[token] = token_value
    bias[1025 + duration] = 3.0
    w["head_bias"] = bias
    return w


def test_decoder_control_closed_forms(oracle):
    """The decode loop's rules (tdt-decoder.ts:1740-1810) with a head that
    always answers the same: durations advance time, duration 0 repeats a
    frame up to 10 symbols, blanks advance one frame and emit nothing,
    start/end bound the frames, max_tokens sets the overflow flag."""
    base = decoder_weights(5, lstm_std=0.0)
    enc = np.zeros((1, 12, 640), np.float16)
    r = oracle.tdt_decode(fixed_head(base, 7, 2), enc, [11], max_tokens=64)
    assert r["counts"][0] == 6 and r["status"][0] == 0
    assert list(r["tokens"][0][:6]) == [7] * 6 and list(r["frames"][0][:6]) == [0, 2, 4, 6, 8, 10]
    assert list(r["durations"][0][:6]) == [2] * 6
    r = oracle.tdt_decode(fixed_head(base, 1024, 0), enc, [12], max_tokens=64)
    assert r["counts"][0] == 0
    r = oracle.tdt_decode(fixed_head(base, 3, 0), enc, [4], max_tokens=64)
    assert r["counts"][0] == 40 and list(r["frames"][0][:40]) == sorted([0, 1, 2, 3] * 10)
    r = oracle.tdt_decode(fixed_head(base, 3, 0), enc, [4], max_tokens=25)
    assert r["counts"][0] == 25 and r["status"][0] == 1
    r = oracle.tdt_decode(fixed_head(base, 9, 1), enc, [12], max_tokens=64, starts=[3], ends=[7])
    assert r["counts"][0] == 4 and list(r["frames"][0][:4]) == [3, 4, 5, 6]
    # lengths past the frame count are clamped to it
    r = oracle.tdt_decode(fixed_head(base, 9, 1), enc, [500], max_tokens=64)
    assert r["counts"][0] == 12


def test_decoder_flush_and_ties(oracle):
    """The bounded flush (:1812-1998): a non-blank head emits 10 more tokens
    at the last valid frame; a blank head stops after 5 blanks. Equal
    scores pick the lowest id; a NaN score never wins."""
    base = decoder_weights(6, lstm_std=0.0)
    enc = np.zeros((1, 12, 640), np.float16)
    r = oracle.tdt_decode(fixed_head(base, 4, 1), enc, [6], max_tokens=64, flush=[1])
    assert r["counts"][0] == 16 and list(r["frames"][0][6:16]) == [5] * 10
    r = oracle.tdt_decode(fixed_head(base, 1024, 1), enc, [6], max_tokens=64, flush=[1])
    assert r["counts"][0] == 0
    w = fixed_head(base, 11, 3)
    w["head_bias"][2] = 5.0  # ties token 11
    w["head_bias"][1] = np.nan
    w["head_bias"][1025 + 1] = 3.0  # ties duration 3
    scores, token, duration = oracle.tdt_joint(w, np.zeros(640, np.float16), np.zeros(640, np.float32))
    assert (token, duration) == (2, 1)


# ---------------------------------------------------------------- TDT decoder, f32 profile


def decoder_weights_f32(seed, **kw):
    """The f16 test weights widened to f32, plus f32 detail below f16's
    precision so that an f16 rounding anywhere shows."""
    w = decoder_weights(seed, **kw)
    rng = np.random.default_rng(seed + 1000)
    out = {}
    for k, v in w.items():
        v = v.astype(np.float32)
        if not k.endswith("bias"):
            v = v + (rng.standard_normal(v.shape) * 1e-4 * np.abs(v).max()).astype(np.float32)
        out[k] = v
    return out


def test_decoder_f32_predictor_step_matches_torch_lstm(oracle):
    """The f32 profile's predictor step against torch's LSTMCell and a float64
    projector product at f32 tolerance (an f16 rounding of a chain input, a
    bias or an accumulator would leave errors near 1e-3)."""
    w = decoder_weights_f32(1)
    rng = np.random.default_rng(2)
    state = (rng.standard_normal((4, 640)) * 0.3).astype(np.float32)
    cand = oracle.tdt_predictor(w, 37, state)
    x = w["embedding"][37].astype(np.float64)
    h0, c0 = torch_lstm_layer(w["lstm_weight_l0"], w["lstm_bias_l0"], x, state[0], state[1])
    h1, c1 = torch_lstm_layer(w["lstm_weight_l1"], w["lstm_bias_l1"], cand[0].astype(np.float64), state[2], state[3])
    proj = cand[2].astype(np.float64) @ w["projector_weight"].astype(np.float64) + w["projector_bias"]
    for got, want in ((cand[0], h0), (cand[1], c0), (cand[2], h1), (cand[3], c1), (cand[4], proj)):
        assert np.abs(got - want).max() <= 2e-5 * max(1.0, np.abs(want).max()), np.abs(got - want).max()
    # the start token: the gates are the f32 biases themselves, not f16-rounded
    start = oracle.tdt_predictor(w, 0, np.zeros((4, 640), np.float32), initial=True)
    g = w["lstm_bias_l0"].astype(np.float64)
    sig = lambda v: 1 / (1 + np.exp(-np.clip(v, -20, 20)))  # noqa: E731
    c_closed = sig(g[:640]) * np.tanh(g[1280:1920])
    np.testing.assert_allclose(start[1], c_closed, rtol=0, atol=2e-7)
    np.testing.assert_allclose(start[0], sig(g[1920:]) * np.tanh(c_closed), rtol=0, atol=2e-7)


def test_decoder_f32_joint_matches_a_float64_product(oracle):
    w = decoder_weights_f32(3)
    rng = np.random.default_rng(4)
    row = (rng.standard_normal(640) * 0.5).astype(np.float32)
    proj = (rng.standard_normal(640) * 0.5).astype(np.float32)
    scores, token, duration = oracle.tdt_joint(w, row, proj)
    joint = np.maximum((row + proj).astype(np.float64), 0)
    want = joint @ w["head_weight"].astype(np.float64) + w["head_bias"]
    assert np.abs(scores[:1030] - want[:1030]).max() <= 1e-5 * np.abs(want).max()
    assert token == int(np.argmax(scores[:1025])) and duration == int(np.argmax(scores[1025:1030]))


def test_decoder_f32_chain_order_closed_forms(oracle):
    """Values that only f32 holds fix the f32 chains' order and rounding:
    the head column 2^24, 1, -2^24 over k = 0, 1, 2 with unit inputs gives 0
    in one increasing-k chain with one rounding per fma (2^24 + 1 rounds to
    2^24), where the exact sum is 1 and a decreasing chain gives 1. The
    same values on LSTM rows 0 (even), 1 (odd), 2 (even) of the g gate give
    gate 1 with the even / odd split (even: 2^24 - 2^24 = 0, odd: 1) and 0
    in one chain."""
    w = {k: np.zeros_like(v) for k, v in decoder_weights_f32(9, lstm_std=0.0).items()}
    big = np.float32(2.0 ** 24)
    w["head_weight"][0, 5], w["head_weight"][1, 5], w["head_weight"][2, 5] = big, 1.0, -big
    w["head_weight"][:3, 6] = [1.0, 1.0, 1.0]  # a column the chain sums exactly: 3
    scores, token, _ = oracle.tdt_joint(w, np.ones(640, np.float32), np.zeros(640, np.float32))
    assert scores[5] == 0.0 and scores[6] == 3.0 and token == 6
    # LSTM layer 0, g gate of channel 0 (column 1280): x = embedding row (ones), h0 = 0
    w["embedding"][3] = 1.0
    w["lstm_weight_l0"][0, 1280], w["lstm_weight_l0"][1, 1280], w["lstm_weight_l0"][2, 1280] = big, 1.0, -big
    cand = oracle.tdt_predictor(w, 3, np.zeros((4, 640), np.float32))
    # i = f = o = sigmoid(0) = 1/2, g = tanh(1), c_prev = 0: c = tanh(1) / 2
    assert cand[1, 0] == pytest.approx(0.5 * np.tanh(1.0), abs=2e-7)
    assert cand[1, 1] == 0.0


def test_decoder_f32_control_closed_forms(oracle):
    """The decode loop is shared by both profiles: a fixed f32 head answers
    token 7 with duration 2, and f32 encoder rows are read as f32."""
    base = decoder_weights_f32(5, lstm_std=0.0)
    head = fixed_head({k: v for k, v in base.items()}, 7, 2)
    head["head_weight"] = head["head_weight"].astype(np.float32)
    enc = np.zeros((1, 12, 640), np.float32)
    r = oracle.tdt_decode(head, enc, [11], max_tokens=64)
    assert r["counts"][0] == 6 and list(r["frames"][0][:6]) == [0, 2, 4, 6, 8, 10]
    with pytest.raises(ValueError, match="must be float32"):
        bad = dict(head)
        bad["head_weight"] = bad["head_weight"].astype(np.float16)
        oracle.tdt_decode(bad, enc, [11], max_tokens=64)

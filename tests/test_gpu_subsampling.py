"""Parity of the subsampling front end's convolution stages
(src/webgpu/kernels/subsampling.ts shaders :1092-1430) against the oracle.

The kernels add the same fmaf terms in the same order as the shaders and
the oracle (bias first, taps in (ky, kx) order, out-of-range taps skipped)
and round once to the storage type, so the bar is bit-exact for f16 and f32
storage. Outputs start as a NaN sentinel so an unwritten element shows."""
import numpy as np
import pytest

from test_gpu_parity import Scope

pytestmark = pytest.mark.gpu


@pytest.fixture
def scope(ctx):
    s = Scope(ctx)
    yield s
    s.close()


def fused_case(seed, batch, frames=1501, dtype=np.float16, lengths=None):
    rng = np.random.default_rng(seed)
    features = rng.standard_normal((batch, 128, frames)).astype(np.float32)
    w0 = (rng.standard_normal((3, 3, 256)) * 0.3).astype(dtype)
    wd = (rng.standard_normal((3, 3, 256)) * 0.3).astype(dtype)
    b0 = (rng.standard_normal(256) * 0.05).astype(np.float32)
    bd = (rng.standard_normal(256) * 0.05).astype(np.float32)
    if lengths is None:
        lengths = rng.integers(1, frames + 1, size=batch)
    return features, w0, b0, wd, bd, np.asarray(lengths, np.uint32)


def bits(a):
    return a.view(np.uint16 if a.dtype == np.float16 else np.uint32)


def run_fused(abi, ctx, scope, case, *, active=0, offset=0, lengths_prefix=()):
    features, w0, b0, wd, bd, lengths = case
    batch, _, frames = features.shape
    ho = (((frames + 1) // 2) + 1) // 2
    out = scope.put(np.full((batch, ho, 32, 256), np.nan, w0.dtype))
    valid = scope.put(np.concatenate([np.asarray(lengths_prefix, np.uint32), lengths]).astype(np.uint32))
    op = abi.SubsamplingOp(ctx, "fused", input=scope.put(features), conv0_weights=scope.put(w0),
                           conv0_bias=scope.put(b0), depthwise_weights=scope.put(wd), depthwise_bias=scope.put(bd),
                           output=out, valid_lengths=valid, batch_size=batch, input_height=frames,
                           valid_length_batch_offset=offset)
    try:
        plan = op.plan(active)
        op.enqueue(active)
        ctx.synchronize()
        return out.download(), plan
    finally:
        op.release()


@pytest.mark.parametrize("dtype", [np.float16, np.float32], ids=["f16", "f32"])
def test_fused_conv0_depthwise2_is_bit_exact(abi, ctx, scope, oracle, dtype):
    """[3, 1501, 128, 256] with a full window, an odd length and a one-frame
    window (subsampling-kernel-shapes.test.ts:83-110 plans this B3 shape)."""
    case = fused_case(1, 3, dtype=dtype, lengths=[1501, 799, 1])
    print("fused conv0+depthwise2 [3,1501,128,256]", np.dtype(dtype).name, flush=True)
    got, plan = run_fused(abi, ctx, scope, case)
    assert (plan.output_height, plan.output_width) == (376, 32)
    assert plan.algorithmic_bytes == 3 * 1501 * 128 * 4 + 3 * 376 * 32 * 256 * np.dtype(dtype).itemsize + \
        2 * (9 * 256 * np.dtype(dtype).itemsize + 1024) + 12
    want = oracle.subsampling_fused(*case, dtype=dtype)
    np.testing.assert_array_equal(bits(got), bits(want))
    assert not got[2, 1:].any() and got[1, 200:].max() == 0 and got[1, :200].any()


def test_fused_offset_prefix_and_other_frame_counts(abi, ctx, scope, oracle):
    """validLengthBatchOffset selects the windows' lengths; an active prefix
    leaves the other windows untouched; 6001 frames (60 s windows) work."""
    case = fused_case(2, 3, frames=6001, lengths=[6001, 3333, 17])
    got, _ = run_fused(abi, ctx, scope, case, active=2, offset=2, lengths_prefix=(5, 5))
    want = oracle.subsampling_fused(*case, dtype=np.float16)
    np.testing.assert_array_equal(bits(got[:2]), bits(want[:2]))
    assert np.isnan(got[2]).all()


@pytest.mark.parametrize("dtype", [np.float16, np.float32], ids=["f16", "f32"])
def test_depthwise5_is_bit_exact(abi, ctx, scope, oracle, dtype):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((3, 376, 32, 256)) * 0.7).astype(dtype)
    w = (rng.standard_normal((3, 3, 256)) * 0.3).astype(dtype)
    bias = (rng.standard_normal(256) * 0.05).astype(np.float32)
    lengths = np.array([1501, 799, 1], np.uint32)
    out = scope.put(np.full((3, 188, 16, 256), np.nan, dtype))
    op = abi.SubsamplingOp(ctx, "depthwise", input=scope.put(x), weights=scope.put(w), bias=scope.put(bias),
                           output=out, valid_lengths=scope.put(lengths), batch_size=3, input_height=376,
                           input_width=32, channels=256, steps=3, label="subsampling-depthwise5")
    try:
        op.enqueue()
        ctx.synchronize()
        got = out.download()
    finally:
        op.release()
    want = oracle.subsampling_depthwise(x, w, bias, lengths, 3)
    np.testing.assert_array_equal(bits(got), bits(want))


def test_time_mask_zeroes_exactly_the_rows_past_the_length(abi, ctx, scope, oracle):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 188, 16, 256)).astype(np.float16)
    lengths = np.array([1501, 799, 1, 1500], np.uint32)
    values = scope.put(x)
    op = abi.SubsamplingOp(ctx, "mask", values=values, valid_lengths=scope.put(lengths), batch_size=4, height=188,
                           width=16, channels=256, steps=3)
    try:
        op.enqueue(3)
        ctx.synchronize()
        got = values.download()
    finally:
        op.release()
    want = oracle.subsampling_mask(x[:3], lengths[:3], 3)
    np.testing.assert_array_equal(bits(got[:3]), bits(want))
    np.testing.assert_array_equal(bits(got[3]), bits(x[3]))

"""Parity of the row LayerNorm (layernorm.ts:309-390) against the oracle.

Bars: f16 within one f16 ulp of the oracle's f32 arithmetic rounded to f16,
or within 2^-20 absolute where (x - mean) * rstd * gamma cancels against
beta and leaves a value whose ulp is finer than the f32 statistics (the GPU
sums in a different order and uses v_sqrt/v_rcp); f32 within 1e-5 relative
(norm- and max-wise)."""
import numpy as np
import pytest

from test_gpu_conv import ulp_distance
from test_gpu_parity import Scope

pytestmark = pytest.mark.gpu


@pytest.fixture
def scope(ctx):
    s = Scope(ctx)
    yield s
    s.close()


def assert_f16_close(got, want):
    """One f16 ulp per element, or 2^-20 absolute (cancellation)."""
    far = np.abs(got.astype(np.float64) - want.astype(np.float64)) > 2.0 ** -20
    assert ulp_distance(got[far], want[far]) <= 1


def run_ln(abi, ctx, scope, x, gamma, beta, *, active=0, in_place=False, epsilon=None):
    xin = scope.put(x)
    out = xin if in_place else scope.put(np.full_like(x, 321))
    op = abi.LayerNormOp(ctx, input=xin, gamma=scope.put(gamma), beta=scope.put(beta), output=out, rows=x.shape[0],
                         channels=x.shape[1], epsilon=epsilon)
    try:
        op.enqueue(active)
        ctx.synchronize()
        return out.download()
    finally:
        op.release()


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("rows,channels", [(3008, 1024), (7, 1024), (5, 4), (3, 2048), (2, 4096), (9, 260)])
def test_layernorm_matches_oracle(abi, ctx, scope, oracle, dtype, rows, channels):
    rng = np.random.default_rng(rows + channels)
    x = (rng.standard_normal((rows, channels)) * 2 + 0.5).astype(dtype)
    gamma = (1 + 0.1 * rng.standard_normal(channels)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(channels)).astype(np.float32)
    got = run_ln(abi, ctx, scope, x, gamma, beta)
    want = oracle.layernorm(x, gamma, beta)
    if dtype == np.float16:
        assert_f16_close(got, want)
    else:
        norm, worst = oracle.relative_errors(got, want)
        assert norm <= 1e-5 and worst <= 1e-5, (norm, worst)


def test_layernorm_in_place_active_rows_and_epsilon(abi, ctx, scope, oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((40, 1024)).astype(np.float16)
    gamma, beta = np.ones(1024, np.float32), np.zeros(1024, np.float32)
    got = run_ln(abi, ctx, scope, x, gamma, beta, active=25, in_place=True, epsilon=0.5)
    assert_f16_close(got[:25], oracle.layernorm(x[:25], gamma, beta, epsilon=0.5))
    np.testing.assert_array_equal(got[25:].view(np.uint16), x[25:].view(np.uint16))


@pytest.mark.parametrize("dtype,rows,channels,alias", [
    (np.float16, 3008, 1024, True), (np.float16, 7, 1024, False), (np.float16, 5, 260, True),
    (np.float16, 3, 2048, False), (np.float32, 9, 1024, True), (np.float32, 4, 260, False)])
def test_chained_layernorm_matches_two_launches(abi, ctx, scope, oracle, dtype, rows, channels, alias):
    """A chained LayerNorm writes LN1(x) and LN2(LN1(x)) in one launch,
    bit-identical to two launches (the second over the stored first output),
    with the second output on the input (as the encoder chains it) or in a
    buffer of its own; both within the bars of the oracle's two passes."""
    rng = np.random.default_rng(rows * 7 + channels)
    x = (rng.standard_normal((rows, channels)) * 2 + 0.5).astype(dtype)
    g1, g2 = [(1 + 0.1 * rng.standard_normal(channels)).astype(np.float32) for _ in range(2)]
    b1, b2 = [(0.1 * rng.standard_normal(channels)).astype(np.float32) for _ in range(2)]
    first = run_ln(abi, ctx, scope, x, g1, b1)
    second = run_ln(abi, ctx, scope, first, g2, b2)
    xin = scope.put(x)
    out = scope.put(np.full_like(x, 321))
    nxt = xin if alias else scope.put(np.full_like(x, 123))
    op = abi.LayerNormOp(ctx, input=xin, gamma=scope.put(g1), beta=scope.put(b1), output=out, rows=rows,
                         channels=channels, next_gamma=scope.put(g2), next_beta=scope.put(b2), next_output=nxt)
    try:
        op.enqueue()
        ctx.synchronize()
        got1, got2 = out.download(), nxt.download()
    finally:
        op.release()
    bits = np.uint16 if dtype == np.float16 else np.uint32
    np.testing.assert_array_equal(got1.view(bits), first.view(bits))
    np.testing.assert_array_equal(got2.view(bits), second.view(bits))
    want1 = oracle.layernorm(x, g1, b1)
    want2 = oracle.layernorm(want1, g2, b2)
    if dtype == np.float16:
        assert_f16_close(got1, want1)
        assert_f16_close(got2, oracle.layernorm(got1, g2, b2))
        assert oracle.relative_errors(got2, want2)[0] <= 1e-3
    else:
        assert max(oracle.relative_errors(got1, want1)) <= 1e-5
        assert max(oracle.relative_errors(got2, want2)) <= 1e-5


def test_chained_layernorm_active_rows(abi, ctx, scope):
    """An active prefix writes both outputs of those rows only."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((40, 1024)).astype(np.float16)
    g, b = np.ones(1024, np.float32), np.zeros(1024, np.float32)
    xin, out, nxt = scope.put(x), scope.put(np.full_like(x, 7)), scope.put(np.full_like(x, 9))
    op = abi.LayerNormOp(ctx, input=xin, gamma=scope.put(g), beta=scope.put(b), output=out, rows=40, channels=1024,
                         next_gamma=scope.put(g), next_beta=scope.put(b), next_output=nxt)
    try:
        op.enqueue(25)
        ctx.synchronize()
        got1, got2 = out.download(), nxt.download()
    finally:
        op.release()
    assert (got1[25:] == 7).all() and (got2[25:] == 9).all()
    assert np.isfinite(got1[:25]).all() and np.isfinite(got2[:25]).all()

"""PK_GEMM_POST_NORM: the LayerNorm of a GEMM's finished output rows, written
by the last workgroup of each row band, against the same GEMM tile followed
by a separate LayerNorm launch (layernorm.ts:309-390) through the C ABI.

Bar: bit-identical. The GEMM output, the normalised rows and the chained
second LayerNorm equal those of the separate launches bit for bit (the
band epilogue runs the LayerNorm kernel's arithmetic, pk_rownorm.h, on the
same stored rows); the GEMM itself is checked against the oracle like any
other tile. Rows past an active prefix stay untouched, and repeated
launches (the band counters reset themselves) give the same bits."""
import numpy as np
import pytest

from test_gpu_parity import Scope, assert_f16_parity, variant_names

pytestmark = pytest.mark.gpu


@pytest.fixture
def scope(ctx):
    s = Scope(ctx)
    yield s
    s.close()


def bits(x):
    return x.view(np.uint16)


def affine(rng, n):
    return (1 + 0.1 * rng.standard_normal(n)).astype(np.float32), (0.1 * rng.standard_normal(n)).astype(np.float32)


def run_pair(abi, ctx, scope, workloads, case, *, chain, in_place_chain=False, variant=None, active=0, repeats=1):
    """The post-norm op and, on the same variant, the plain GEMM followed by
    a (chained) LayerNorm launch. Returns both sets of outputs and the
    kernel name."""
    w = case.weight
    rows, n = case.rows, w.columns
    rng = np.random.default_rng(rows + n)
    g, b = affine(rng, n)
    g2, b2 = affine(rng, n)
    sentinel = np.full((rows, n), 77, np.float16)
    dev = {k: scope.put(v) for k, v in dict(a=case.a, packed=w.packed, palette=w.palette, res=case.residual,
                                            g=g, b=b, g2=g2, b2=b2).items() if v is not None}
    common = dict(packed=dev["packed"], palette=dev["palette"], bits=w.bits, rows=rows, inner=w.inner, columns=n,
                  residual=dev.get("res"), residual_scale=case.residual_scale, activation=case.activation)
    out_p, post_p = scope.put(sentinel), scope.put(sentinel)
    next_p = out_p if in_place_chain else scope.put(sentinel)
    extra = dict(post_next_gamma=dev["g2"], post_next_beta=dev["b2"], post_next_output=next_p) if chain else {}
    op = abi.GemmOp(ctx, a=dev["a"], output=out_p, post_gamma=dev["g"], post_beta=dev["b"], post_output=post_p,
                    label="post-norm", **common, **extra)
    try:
        if variant is not None:
            op.set_variant(variant)
        name = op.plan().kernel.decode()
        index = [n.replace("_b5_", f"_b{w.bits}_") for n in variant_names(abi, ctx, scope, workloads)].index(name)
        for _ in range(repeats):
            op.enqueue(active)
        ctx.synchronize()
        got = [out_p.download(), post_p.download()] + ([next_p.download()] if chain and not in_place_chain else [])
    finally:
        op.release()
    # Reference: the plain GEMM on the same tile, then the LayerNorm launch.
    out_r, post_r, next_r = scope.put(sentinel), scope.put(sentinel), scope.put(sentinel)
    plain = abi.GemmOp(ctx, a=dev["a"], output=out_r, label="plain", **common)
    ln_extra = dict(next_gamma=dev["g2"], next_beta=dev["b2"], next_output=next_r) if chain else {}
    ln = abi.LayerNormOp(ctx, input=out_r, gamma=dev["g"], beta=dev["b"], output=post_r, rows=rows, channels=n,
                         **ln_extra)
    try:
        plain.set_variant(index)
        plain.enqueue(active)
        ln.enqueue(active)
        ctx.synchronize()
        want = [out_r.download(), post_r.download()] + ([next_r.download()] if chain else [])
    finally:
        plain.release()
        ln.release()
    if chain and in_place_chain:
        want = [want[2], want[1]]  # the chained rows replace the GEMM output
    return got, want, name


SHAPES = [
    # rows, inner, columns, bits, residual scale
    (3008, 1024, 1024, 6, 1.0),   # o_proj / pointwise-2 + residual, 16 windows
    (3008, 4096, 1024, 5, 0.5),   # FF contract + 0.5 residual
    (333, 1024, 1024, 5, 1.0),    # a partial last band
    (200, 1024, 512, 6, None),    # N = 512, no residual
]


@pytest.mark.parametrize("chain", [False, True])
@pytest.mark.parametrize("rows,inner,columns,bits_,scale", SHAPES)
def test_post_norm_matches_separate_layernorm(abi, ctx, scope, oracle, workloads, rows, inner, columns, bits_,
                                              scale, chain):
    case = workloads.gemm_case(rows + inner + columns, rows, inner, columns, bits_, residual_scale=scale)
    print(f"post norm {rows}x{inner}x{columns} b{bits_} chain={chain}", flush=True)
    got, want, name = run_pair(abi, ctx, scope, workloads, case, chain=chain, repeats=2)
    print(f"  planned {name}", flush=True)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(bits(g), bits(w))
    pick = np.r_[0:64, rows - 64:rows]
    assert_f16_parity(oracle, got[0][pick], case, rows=pick)


def test_post_norm_every_tile(abi, ctx, scope, workloads):
    """Every tile with a post-norm kernel, the chained form written in place
    over the GEMM output as the encoder's last LayerNorm does."""
    case = workloads.gemm_case(7, 700, 1024, 1024, 6, residual_scale=1.0)
    names = variant_names(abi, ctx, scope, workloads)
    tiles = [i for i, n in enumerate(names) if "f16p" in n and ("k2_" in n or "k4_" in n)]
    assert len(tiles) == 7
    for v in tiles:
        print(f"post norm tile {names[v]}", flush=True)
        got, want, name = run_pair(abi, ctx, scope, workloads, case, chain=True, in_place_chain=True, variant=v)
        assert name == names[v].replace("_b5_", "_b6_")
        for g, w in zip(got, want):
            np.testing.assert_array_equal(bits(g), bits(w))


def test_post_norm_active_prefix(abi, ctx, scope, workloads):
    case = workloads.gemm_case(8, 3008, 1024, 1024, 5, residual_scale=1.0)
    got, want, _ = run_pair(abi, ctx, scope, workloads, case, chain=True, active=1000)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(bits(g[:1000]), bits(w[:1000]))
        assert np.all(g[1000:] == np.float16(77))


def test_post_norm_rejects_tiles_without_it(abi, ctx, scope, workloads):
    case = workloads.gemm_case(9, 64, 1024, 1024, 5)
    w = case.weight
    rng = np.random.default_rng(0)
    g, b = affine(rng, 1024)
    op = abi.GemmOp(ctx, a=scope.put(case.a), packed=scope.put(w.packed), palette=scope.put(w.palette),
                    output=scope.empty((64, 1024), np.float16), bits=5, rows=64, inner=1024, columns=1024,
                    post_gamma=scope.put(g), post_beta=scope.put(b), post_output=scope.empty((64, 1024), np.float16),
                    label="post-norm")
    try:
        assert "k2_" in op.plan().kernel.decode() or "k4_" in op.plan().kernel.decode()
        names = variant_names(abi, ctx, scope, workloads)
        for v, n in enumerate(names):
            if "f16p" in n and ("k2_" in n or "k4_" in n):
                continue
            with pytest.raises(abi.PaletteRangeError, match=f"post-norm tile variant {v} has no post-norm epilogue"):
                op.set_variant(v)
    finally:
        op.release()

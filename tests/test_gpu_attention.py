"""Parity of the relative-position attention (attention.ts:418-727) against
the CPU oracle, through the C ABI.

Bars: the f16 kernel within 2e-3 norm-wise of the oracle's reference f32
arithmetic (rounded to f16) and of the fp64 truth — the MFMA path rounds
(q + u), (q + v) and the probabilities to f16 once, which moves results by a
few 1e-4; rows at or past the valid length exactly zero; the f32 kernel
within 1e-4 (norm- and max-wise) of the reference f32 arithmetic.
"""
import numpy as np
import pytest

from test_gpu_parity import F16_TOL_TRUTH, F32_TOL, Scope

pytestmark = pytest.mark.gpu

F16_ATTENTION_TOL = 2e-3


@pytest.fixture
def scope(ctx):
    s = Scope(ctx)
    yield s
    s.close()


def run_attention(abi, ctx, scope, case, *, row_major=False, variant=None, active_batch=0, sentinel=None):
    dtype = case.qkv.dtype
    out = scope.put(np.full((case.batch * case.frames, 1024), sentinel if sentinel is not None else 0, dtype))
    positions = case.positions if row_major else case.packed_positions
    op = abi.RelativeAttentionOp(
        ctx, qkv=scope.put(case.qkv), projected_positions=scope.put(positions), bias_u=scope.put(case.bias_u),
        bias_v=scope.put(case.bias_v), valid_lengths=scope.put(case.valid), output=out, batch_size=case.batch,
        frames=case.frames, positions_row_major=row_major)
    try:
        if variant is not None:
            op.set_variant(variant)
        op.enqueue(active_batch)
        ctx.synchronize()
        return out.download(), op.plan().kernel.decode()
    finally:
        op.release()


def oracle_attention(oracle, case, mode="f32-chain", batch=None):
    batch = case.batch if batch is None else batch
    rows = batch * case.frames
    return oracle.relative_attention(case.qkv[:rows], case.packed_positions, case.bias_u, case.bias_v,
                                     case.valid[:batch], batch=batch, frames=case.frames, mode=mode)


def assert_attention_parity(oracle, got, case, batch=None):
    batch = case.batch if batch is None else batch
    want = oracle_attention(oracle, case, batch=batch)
    if got.dtype == np.float32:
        norm, worst = oracle.relative_errors(got, want)
        assert norm <= F32_TOL and worst <= F32_TOL, (norm, worst)
    else:
        norm, _ = oracle.relative_errors(got, want)
        assert norm <= F16_ATTENTION_TOL, norm
        truth = oracle_attention(oracle, case, mode="f64", batch=batch)
        norm, _ = oracle.relative_errors(got, truth)
        assert norm <= F16_TOL_TRUTH, norm
    for b in range(batch):
        live = min(int(case.valid[b]), case.frames)
        assert np.all(got[b * case.frames + live:(b + 1) * case.frames] == 0)


SHAPES = [
    # batch, frames, valid lengths (None: uniform in [T/2, T])
    (4, 188, None),
    (1, 750, [640]),
    (3, 23, [23, 0, 40]),   # full, empty, longer than the window
    (1, 1, [1]),
    (2, 33, [33, 32]),      # one key past a tile edge
    (2, 64, [64, 1]),
]


@pytest.mark.parametrize("row_major", [False, True])
@pytest.mark.parametrize("batch,frames,valid", SHAPES)
def test_f16_attention_matches_oracle(abi, ctx, scope, oracle, workloads, batch, frames, valid, row_major):
    case = workloads.attention_case(40 + frames, batch, frames, valid=valid)
    print(f"attention f16 B={batch} T={frames} row_major={row_major}", flush=True)
    got, _ = run_attention(abi, ctx, scope, case, row_major=row_major)
    assert_attention_parity(oracle, got, case)


def test_position_layouts_give_identical_results(abi, ctx, scope, workloads):
    case = workloads.attention_case(50, 2, 100, valid=[100, 77])
    packed, _ = run_attention(abi, ctx, scope, case)
    rows, _ = run_attention(abi, ctx, scope, case, row_major=True)
    np.testing.assert_array_equal(packed.view(np.uint16), rows.view(np.uint16))


def test_every_f16_attention_variant_matches(abi, ctx, scope, oracle, workloads):
    case = workloads.attention_case(51, 2, 150, valid=[150, 70])
    for variant in range(abi.attention_variant_count("f16")):
        got, kernel = run_attention(abi, ctx, scope, case, variant=variant)
        print(f"attention variant {variant} {kernel}", flush=True)
        assert_attention_parity(oracle, got, case)


@pytest.mark.parametrize("batch,frames,valid", [(2, 188, [188, 100]), (2, 23, [0, 40]), (1, 200, [200])])
def test_f32_attention_matches_oracle(abi, ctx, scope, oracle, workloads, batch, frames, valid):
    """Both f32 kernels: the planned MFMA flash kernel and the one in the
    reference's own operation order."""
    case = workloads.attention_case(52 + frames, batch, frames, dtype=np.float32, valid=valid)
    names = ["pk_rel_attention_f32_mfma", "pk_rel_attention_f32"]
    assert abi.attention_variant_count("f32") == len(names)
    for row_major in (False, True):
        got, kernel = run_attention(abi, ctx, scope, case, row_major=row_major)
        assert kernel == names[0]
        assert_attention_parity(oracle, got, case)
        for variant, name in enumerate(names):
            print(f"attention f32 B={batch} T={frames} row_major={row_major} variant {variant}", flush=True)
            got, kernel = run_attention(abi, ctx, scope, case, row_major=row_major, variant=variant)
            assert kernel == name
            assert_attention_parity(oracle, got, case)


@pytest.mark.parametrize("batch,frames,valid", [(4, 750, [750, 640, 1, 31]), (3, 64, [64, 33, 32])])
def test_f32_mfma_attention_long_and_edge_windows(abi, ctx, scope, oracle, workloads, batch, frames, valid):
    """The MFMA kernel at T = 750 (24 key tiles, 1499 position rows) and at
    tile edges (valid lengths 1, 31, 32, 33)."""
    case = workloads.attention_case(56 + frames, batch, frames, dtype=np.float32, valid=valid)
    for row_major in (True, False):
        print(f"attention f32 mfma B={batch} T={frames} row_major={row_major}", flush=True)
        got, kernel = run_attention(abi, ctx, scope, case, row_major=row_major)
        assert kernel == "pk_rel_attention_f32_mfma"
        assert_attention_parity(oracle, got, case)


def test_attention_active_batch_prefix(abi, ctx, scope, oracle, workloads):
    """encode(shape.batchSize = 2) of a 4-window dispatch (attention.ts:67-90)."""
    case = workloads.attention_case(53, 4, 60)
    sentinel = np.float16(555.0)
    got, _ = run_attention(abi, ctx, scope, case, active_batch=2, sentinel=sentinel)
    assert_attention_parity(oracle, got[:120], case, batch=2)
    assert np.all(got[120:] == sentinel)


def test_attention_dispatch_errors(abi, ctx, scope, workloads):
    case = workloads.attention_case(54, 2, 20)
    out = scope.empty((40, 1024), np.float16)
    op = abi.RelativeAttentionOp(
        ctx, qkv=scope.put(case.qkv), projected_positions=scope.put(case.packed_positions),
        bias_u=scope.put(case.bias_u), bias_v=scope.put(case.bias_v), valid_lengths=scope.put(case.valid),
        output=out, batch_size=2, frames=20, label="layer5-relative-attention")
    try:
        with pytest.raises(abi.PaletteRangeError, match=r"layer5-relative-attention active batch must be in \[1, 2\]"):
            op.enqueue(3)
        op.destroy()
        op.destroy()
        with pytest.raises(abi.PaletteDestroyedError, match="layer5-relative-attention was destroyed"):
            op.enqueue()
    finally:
        op.release()


# ---------------------------------------------------- the MHA block (C3)


def mha_on_gpu(abi, ctx, scope, mod):
    """QKV GEMM -> rel-pos linear (row-major positions) -> attention -> Wo
    GEMM + residual, on one stream."""
    rows, p = mod.x.shape[0], mod.table.shape[0]
    x = scope.put(mod.x)
    qkv = scope.empty((rows, 3072), np.float16)
    pos = scope.empty((p, 1024), np.float16)
    ctxt = scope.empty((rows, 1024), np.float16)
    y = scope.empty((rows, 1024), np.float16)
    ops = [
        abi.GemmOp(ctx, a=x, packed=scope.put(mod.wqkv.packed), palette=scope.put(mod.wqkv.palette), output=qkv,
                   bits=mod.wqkv.bits, rows=rows, inner=1024, columns=3072, label="attention-qkv"),
        abi.GemmOp(ctx, a=scope.put(mod.table), packed=scope.put(mod.wpos.packed),
                   palette=scope.put(mod.wpos.palette), output=pos, bits=mod.wpos.bits, rows=p, inner=1024,
                   columns=1024, label="attention-relative-positions"),
        abi.RelativeAttentionOp(ctx, qkv=qkv, projected_positions=pos, bias_u=scope.put(mod.bias_u),
                                bias_v=scope.put(mod.bias_v), valid_lengths=scope.put(mod.valid), output=ctxt,
                                batch_size=mod.batch, frames=mod.frames, positions_row_major=True),
        abi.GemmOp(ctx, a=ctxt, packed=scope.put(mod.wo.packed), palette=scope.put(mod.wo.palette), output=y,
                   bits=mod.wo.bits, rows=rows, inner=1024, columns=1024, residual=x, residual_scale=1.0,
                   label="attention-output-residual"),
    ]
    try:
        for op in ops:
            op.enqueue()
        ctx.synchronize()
        return qkv.download(), pos.download(), ctxt.download(), y.download()
    finally:
        for op in ops:
            op.release()


def mha_on_oracle(oracle, workloads, mod, windows, mode):
    """The same chain on the CPU for the given windows: "reference" = f16
    accumulation chains for the GEMMs and the f32 attention, rounded to f16
    between steps; "f64" = every step in double."""
    T = mod.frames
    rows = np.concatenate([np.arange(w * T, (w + 1) * T) for w in windows])
    x = mod.x[rows]
    valid = mod.valid[list(windows)]
    if mode == "reference":
        qkv = oracle.gemm(x, mod.wqkv.packed, 6, mod.wqkv.palette, 3072, mode="f16-chain", threads=8)
        pos = oracle.gemm(mod.table, mod.wpos.packed, 6, mod.wpos.palette, 1024, mode="f16-chain", threads=8)
        c = oracle.relative_attention(qkv, workloads.pack_projected_positions(pos), mod.bias_u, mod.bias_v, valid,
                                      batch=len(windows), frames=T)
        return rows, oracle.gemm(c, mod.wo.packed, 6, mod.wo.palette, 1024, residual=x, residual_scale=1.0,
                                 mode="f16-chain", threads=8)
    qkv = oracle.gemm(x, mod.wqkv.packed, 6, mod.wqkv.palette, 3072, mode="f64", threads=8)
    pos = oracle.gemm(mod.table, mod.wpos.packed, 6, mod.wpos.palette, 1024, mode="f64", threads=8)
    c = oracle.relative_attention(qkv, workloads.pack_projected_positions(pos), mod.bias_u, mod.bias_v, valid,
                                  batch=len(windows), frames=T, mode="f64")
    dense = oracle.expand(mod.wo.packed, 6, 1024, 1024, mod.wo.palette).astype(np.float64)
    return rows, x.astype(np.float64) + c @ dense


@pytest.mark.parametrize("frames,windows", [(188, (0, 3)), (750, (1,))])
def test_mha_block_full_size(abi, ctx, scope, oracle, workloads, frames, windows):
    """4 windows x T frames x 1024 through the four launches; the checked
    windows against the oracle chain (1e-2) and the fp64 truth (2e-3)."""
    mod = workloads.mha_module(0, frames=frames)
    print(f"mha block 4x{frames}x1024", flush=True)
    _, _, _, y = mha_on_gpu(abi, ctx, scope, mod)
    rows, y_ref = mha_on_oracle(oracle, workloads, mod, windows, "reference")
    norm, _ = oracle.relative_errors(y[rows], y_ref)
    assert norm <= 1e-2, norm
    rows, y_truth = mha_on_oracle(oracle, workloads, mod, windows, "f64")
    norm, _ = oracle.relative_errors(y[rows], y_truth)
    assert norm <= F16_TOL_TRUTH, norm


@pytest.mark.parametrize("active", [1, 5])
def test_attention_plan_active_matches_a_dedicated_op(abi, ctx, scope, oracle, workloads, active):
    """PK_ATTENTION_PLAN_ACTIVE: 16 windows x 188 frames, an active prefix
    runs the variant an op created for that many windows plans, bit-identical
    to that op and within tolerance of the oracle; rows past the prefix stay
    untouched."""
    case = workloads.attention_case(71, 16, 188)
    inputs = dict(qkv=scope.put(case.qkv), projected_positions=scope.put(case.packed_positions),
                  bias_u=scope.put(case.bias_u), bias_v=scope.put(case.bias_v), valid_lengths=scope.put(case.valid),
                  frames=case.frames)
    sentinel = np.float16(3.0)
    out = scope.put(np.full((16 * 188, 1024), sentinel, np.float16))
    op = abi.RelativeAttentionOp(ctx, output=out, batch_size=16, plan_active=True, **inputs)
    dedicated_out = scope.put(np.zeros((active * 188, 1024), np.float16))
    dedicated = abi.RelativeAttentionOp(ctx, output=dedicated_out, batch_size=active, **inputs)
    try:
        print("prefix", op.plan(active).kernel.decode(), "dedicated", dedicated.plan().kernel.decode(),
              "capacity", op.plan().kernel.decode(), flush=True)
        assert op.plan(active).kernel == dedicated.plan().kernel
        op.enqueue(active)
        dedicated.enqueue()
        ctx.synchronize()
    finally:
        op.release()
        dedicated.release()
    got = out.download()
    np.testing.assert_array_equal(got[:active * 188].view(np.uint16), dedicated_out.download().view(np.uint16))
    assert (got[active * 188:] == sentinel).all()
    want = oracle_attention(oracle, case, batch=active)
    assert oracle.relative_errors(got[:active * 188], want)[0] <= F16_ATTENTION_TOL

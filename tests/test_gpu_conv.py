"""Parity of the fused Conformer convolution tail (GLU, depthwise k9, folded
batch norm, SiLU) and of the whole convolution module (PW1 GEMM -> tail ->
PW2 GEMM + residual) against the CPU oracle, through the C ABI.

Bars: fp32 tail within 1e-4 relative (norm-wise and max-wise) of the
reference f32 arithmetic; fp16 tail within one f16 ulp of the reference f32
arithmetic rounded to f16 (both compute in f32 and round once), and within
2e-3 norm-wise of the fp64 truth; the module within 1e-2 norm-wise of the
reference chain and 2e-3 of the truth.
"""
import numpy as np
import pytest

from test_gpu_parity import F16_TOL_REFERENCE, F16_TOL_TRUTH, F32_TOL, Scope

pytestmark = pytest.mark.gpu


@pytest.fixture
def scope(ctx):
    s = Scope(ctx)
    yield s
    s.close()


def ulp_distance(got: np.ndarray, want: np.ndarray) -> int:
    """Largest distance in f16 units in the last place (ordered bit patterns)."""
    def ordered(a):
        bits = a.view(np.uint16).astype(np.int32)
        return np.where(bits & 0x8000, 0x8000 - bits, bits + 0x8000)
    return int(np.abs(ordered(got) - ordered(want)).max()) if got.size else 0


def run_conv(abi, ctx, scope, case, *, variant=None, active_batch=0, sentinel=None, repeats=1):
    dtype = case.weights.dtype
    out_host = np.full((case.batch * case.frames, case.channels), sentinel if sentinel is not None else 0, dtype)
    out = scope.put(out_host)
    op = abi.ConformerConvOp(
        ctx, pointwise_input=scope.put(case.pointwise), depthwise_weights=scope.put(case.weights),
        batch_norm_scale=scope.put(case.scale), batch_norm_shift=scope.put(case.shift),
        valid_lengths=scope.put(case.valid), output=out, batch_size=case.batch, frames=case.frames,
        channels=case.channels)
    try:
        if variant is not None:
            op.set_variant(variant)
        for _ in range(repeats):
            op.enqueue(active_batch)
        ctx.synchronize()
        return out.download()
    finally:
        op.release()


def oracle_conv(oracle, case, mode="f32-chain", batch=None):
    batch = case.batch if batch is None else batch
    rows = batch * case.frames
    return oracle.conformer_conv(case.pointwise[:rows], case.weights, case.scale, case.shift,
                                 case.valid[:batch], batch=batch, frames=case.frames, mode=mode)


def assert_conv_parity(oracle, got, case, batch=None):
    want = oracle_conv(oracle, case, batch=batch)
    if got.dtype == np.float32:
        norm, worst = oracle.relative_errors(got, want)
        assert norm <= F32_TOL and worst <= F32_TOL, (norm, worst)
    else:
        assert ulp_distance(got, want) <= 1
        truth = oracle_conv(oracle, case, mode="f64", batch=batch)
        norm, _ = oracle.relative_errors(got, truth)
        assert norm <= F16_TOL_TRUTH, norm


CONV_SHAPES = [
    # batch, frames, channels, valid lengths
    (2, 188, 1024, [188, 150]),
    (3, 23, 64, [23, 0, 40]),      # ragged: full, empty, longer than the window
    (1, 1, 8, [1]),                # a single frame and channel group
    (4, 17, 256, [5, 17, 9, 1]),
    (1, 750, 1024, [701]),          # a long window, many frame runs
]


@pytest.mark.parametrize("precision", ["f16", "f32"])
@pytest.mark.parametrize("batch,frames,channels,valid", CONV_SHAPES)
def test_conv_matches_oracle(abi, ctx, scope, oracle, workloads, precision, batch, frames, channels, valid):
    dtype = np.float16 if precision == "f16" else np.float32
    case = workloads.conv_case(7, batch, frames, channels, dtype=dtype, valid=valid)
    print(f"conv {precision} batch={batch} frames={frames} channels={channels}", flush=True)
    assert_conv_parity(oracle, run_conv(abi, ctx, scope, case), case)


@pytest.mark.parametrize("precision", ["f16", "f32"])
def test_every_conv_variant_matches(abi, ctx, scope, oracle, workloads, precision):
    dtype = np.float16 if precision == "f16" else np.float32
    case = workloads.conv_case(8, 3, 45, 128, dtype=dtype, valid=[45, 30, 3])
    for variant in range(abi.conv_variant_count(precision)):
        print(f"conv {precision} variant {variant}", flush=True)
        assert_conv_parity(oracle, run_conv(abi, ctx, scope, case, variant=variant), case)


def test_conv_active_batch_prefix_leaves_the_tail_untouched(abi, ctx, scope, oracle, workloads):
    """encode(shape.batchSize = 2) of a 4-window dispatch writes windows 0-1 only
    (conformer-conv.ts:134-155)."""
    case = workloads.conv_case(9, 4, 31, 128)
    sentinel = np.float16(1234.0)
    got = run_conv(abi, ctx, scope, case, active_batch=2, sentinel=sentinel)
    rows = 2 * case.frames
    assert_conv_parity(oracle, got[:rows], case, batch=2)
    assert np.all(got[rows:] == sentinel)


def test_conv_is_repeatable(abi, ctx, scope, workloads):
    case = workloads.conv_case(10, 2, 60, 256)
    once = run_conv(abi, ctx, scope, case)
    thrice = run_conv(abi, ctx, scope, case, repeats=3)
    np.testing.assert_array_equal(once.view(np.uint16), thrice.view(np.uint16))


def test_conv_dispatch_errors(abi, ctx, scope, workloads):
    case = workloads.conv_case(11, 2, 20, 64)
    out = scope.empty((case.batch * case.frames, case.channels), np.float16)
    op = abi.ConformerConvOp(
        ctx, pointwise_input=scope.put(case.pointwise), depthwise_weights=scope.put(case.weights),
        batch_norm_scale=scope.put(case.scale), batch_norm_shift=scope.put(case.shift),
        valid_lengths=scope.put(case.valid), output=out, batch_size=2, frames=20, channels=64,
        label="layer3-convolution")
    try:
        with pytest.raises(abi.PaletteRangeError, match=r"layer3-convolution active batch must be in \[1, 2\]"):
            op.enqueue(3)
        with pytest.raises(abi.PaletteRangeError, match="convolution variant"):
            op.set_variant(99)
        op.destroy()
        op.destroy()
        with pytest.raises(abi.PaletteDestroyedError, match="layer3-convolution was destroyed"):
            op.enqueue()
    finally:
        op.release()


def test_conv_timed_enqueue_stamps_the_kernel(abi, ctx, scope, workloads):
    case = workloads.conv_case(12, 4, 188, 1024)
    out = scope.empty((case.batch * case.frames, case.channels), np.float16)
    op = abi.ConformerConvOp(
        ctx, pointwise_input=scope.put(case.pointwise), depthwise_weights=scope.put(case.weights),
        batch_norm_scale=scope.put(case.scale), batch_norm_shift=scope.put(case.shift),
        valid_lengths=scope.put(case.valid), output=out, batch_size=4, frames=188)
    start, end = ctx.event(), ctx.event()
    try:
        op.enqueue(0, None, start, end)
        ctx.synchronize()
        ms = start.elapsed_ms(end)
        assert 0.0 < ms < 50.0
    finally:
        op.release()
        start.destroy()
        end.destroy()


def module_on_gpu(abi, ctx, scope, module, fused_glu=False):
    """PW1 GEMM -> fused conv tail -> PW2 GEMM + residual on one stream.
    fused_glu: PW1 carries the GLU epilogue ([rows, d] output) and the tail
    takes that GLU as its input."""
    x = scope.put(module.x)
    rows, d = module.x.shape
    conv = module.conv
    p = scope.empty((rows, d if fused_glu else 2 * d), np.float16)
    z = scope.empty((rows, d), np.float16)
    y = scope.empty((rows, d), np.float16)
    pw1 = abi.GemmOp(ctx, a=x, packed=scope.put(module.pw1.packed), palette=scope.put(module.pw1.palette),
                     output=p, bits=module.pw1.bits, rows=rows, inner=d, columns=2 * d,
                     label="convolution-pointwise1", glu=fused_glu)
    tail = abi.ConformerConvOp(
        ctx, pointwise_input=p, depthwise_weights=scope.put(conv.weights), batch_norm_scale=scope.put(conv.scale),
        batch_norm_shift=scope.put(conv.shift), valid_lengths=scope.put(conv.valid), output=z,
        batch_size=conv.batch, frames=conv.frames, input_glu=fused_glu)
    pw2 = abi.GemmOp(ctx, a=z, packed=scope.put(module.pw2.packed), palette=scope.put(module.pw2.palette),
                     output=y, bits=module.pw2.bits, rows=rows, inner=d, columns=d, residual=x,
                     residual_scale=1.0, label="convolution-pointwise2-residual")
    try:
        pw1.enqueue()
        tail.enqueue()
        pw2.enqueue()
        ctx.synchronize()
        return p.download(), z.download(), y.download()
    finally:
        pw1.release()
        tail.release()
        pw2.release()


def module_on_oracle(oracle, module, windows, mode):
    """The same chain on the CPU for the given windows (each window only
    reads its own rows). "reference": the f16 GEMM accumulation chain and the
    f32 tail, rounded to f16 between steps like the device; "f64": every
    step in double with no intermediate rounding."""
    frames = module.conv.frames
    rows = np.concatenate([np.arange(w * frames, (w + 1) * frames) for w in windows])
    x = module.x[rows]
    pw1, pw2, conv = module.pw1, module.pw2, module.conv
    valid = conv.valid[list(windows)]
    if mode == "reference":
        p = oracle.gemm(x, pw1.packed, pw1.bits, pw1.palette, pw1.columns, mode="f16-chain", threads=16)
        z = oracle.conformer_conv(p, conv.weights, conv.scale, conv.shift, valid, batch=len(windows),
                                  frames=frames)
        return rows, oracle.gemm(z, pw2.packed, pw2.bits, pw2.palette, pw2.columns, residual=x,
                                 residual_scale=1.0, mode="f16-chain", threads=16)
    p = oracle.gemm(x, pw1.packed, pw1.bits, pw1.palette, pw1.columns, mode="f64", threads=16)
    z = oracle.conformer_conv(p, conv.weights.astype(np.float64), conv.scale, conv.shift, valid,
                              batch=len(windows), frames=frames, mode="f64")
    dense2 = oracle.expand(pw2.packed, pw2.bits, pw2.inner, pw2.columns, pw2.palette).astype(np.float64)
    return rows, x.astype(np.float64) + z @ dense2


_FULL_MODULE = {}


def full_module_on_oracle(oracle, module, mode):
    """module_on_oracle over every window of the seed-0 module, computed once
    per mode for the unfused and the fused-GLU tests (about 10 s of CPU each
    at 16 threads)."""
    if mode not in _FULL_MODULE:
        print("conv module on the oracle:", mode, flush=True)
        _FULL_MODULE[mode] = module_on_oracle(oracle, module, tuple(range(module.conv.batch)), mode)
    return _FULL_MODULE[mode]


def test_conv_module_full_size(abi, ctx, scope, oracle, workloads):
    """16 windows x 188 frames x 1024 on the GPU; every window checked
    against the oracle chain (the reference's f16 GEMM accumulation and f32
    tail) and against the fp64 truth (about 20 s of CPU at 16 threads)."""
    module = workloads.conv_module(0)
    print("conv module 16x188x1024", flush=True)
    p, z, y = module_on_gpu(abi, ctx, scope, module)
    windows = tuple(range(module.conv.batch))
    rows, y_ref = full_module_on_oracle(oracle, module, "reference")
    norm, _ = oracle.relative_errors(y[rows], y_ref)
    assert norm <= F16_TOL_REFERENCE, norm
    rows, y_truth = full_module_on_oracle(oracle, module, "f64")
    norm, _ = oracle.relative_errors(y[rows], y_truth)
    assert norm <= F16_TOL_TRUTH, norm
    # the tail on the GPU's own PW1 output is the oracle's tail of that output
    sub = workloads.ConvCase(p[rows], module.conv.weights, module.conv.scale, module.conv.shift,
                             module.conv.valid[list(windows)], len(windows), module.conv.frames)
    assert ulp_distance(z[rows], oracle_conv(oracle, sub)) <= 1


# ------------------------------------------------ GLU epilogue (fused PW1)


def glu_gemm_on_gpu(abi, ctx, scope, case, variant=None):
    rows, columns = case.rows, case.weight.columns
    out = scope.put(np.full((rows, columns // 2), np.float16(777.0)))
    op = abi.GemmOp(ctx, a=scope.put(case.a), packed=scope.put(case.weight.packed),
                    palette=scope.put(case.weight.palette), output=out, bits=case.weight.bits, rows=rows,
                    inner=case.weight.inner, columns=columns, label="pointwise1-glu", glu=True)
    try:
        if variant is not None:
            op.set_variant(variant)
        op.enqueue()
        ctx.synchronize()
        return out.download(), op.plan().kernel.decode()
    finally:
        op.release()


def assert_glu_parity(oracle, got, case):
    w = case.weight
    p = oracle.gemm(case.a, w.packed, w.bits, w.palette, w.columns, mode="f16-chain", threads=8)
    norm, _ = oracle.relative_errors(got, oracle.glu(p))
    assert norm <= F16_TOL_REFERENCE, norm
    p64 = oracle.gemm(case.a, w.packed, w.bits, w.palette, w.columns, mode="f64", threads=8)
    norm, _ = oracle.relative_errors(got, oracle.glu(p64, mode="f64"))
    assert norm <= F16_TOL_TRUTH, norm


@pytest.mark.parametrize("rows,inner,columns,bits", [
    (376, 1024, 2048, 6),   # two windows of the convolution's pointwise-1
    (300, 512, 256, 5),     # ragged rows
    (64, 256, 128, 6),      # one 64-row tile, small-M plan moved to the pair-code kernels
    (5, 128, 64, 5),        # fewer rows than a tile
])
def test_glu_epilogue_matches_oracle(abi, ctx, scope, oracle, workloads, rows, inner, columns, bits):
    case = workloads.gemm_case(30 + bits, rows, inner, columns, bits)
    print(f"glu gemm {rows}x{inner}x{columns} b{bits}", flush=True)
    got, _ = glu_gemm_on_gpu(abi, ctx, scope, case)
    assert_glu_parity(oracle, got, case)


def test_glu_epilogue_every_pair_code_variant(abi, ctx, scope, oracle, workloads):
    """Every pair-code tile computes the GLU epilogue; other families refuse it."""
    case = workloads.gemm_case(33, 200, 256, 512, 6)
    ran = 0
    for variant in range(abi.variant_count("f16")):
        try:
            got, kernel = glu_gemm_on_gpu(abi, ctx, scope, case, variant)
        except abi.PaletteRangeError as e:
            assert "has no GLU epilogue" in str(e)
            continue
        print(f"glu variant {variant} {kernel}", flush=True)
        assert "_f16p_" in kernel
        assert_glu_parity(oracle, got, case)
        ran += 1
    assert ran >= 8


def test_glu_descriptor_errors(abi, ctx, scope, workloads):
    case = workloads.gemm_case(34, 64, 128, 128, 5)
    a, packed, palette = scope.put(case.a), scope.put(case.weight.packed), scope.put(case.weight.palette)
    out = scope.empty((64, 64), np.float16)
    bias = scope.put(np.zeros(128, np.float32))
    with pytest.raises(abi.PaletteError, match="GLU epilogue needs"):
        abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=out, bits=5, rows=64, inner=128, columns=128,
                   bias=bias, glu=True)
    with pytest.raises(abi.PaletteError, match="output binding must hold"):
        abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=scope.empty((64, 32), np.float16), bits=5,
                   rows=64, inner=128, columns=128, glu=True)


def test_conv_glu_input_matches_oracle(abi, ctx, scope, oracle, workloads):
    """PK_CONV_INPUT_GLU: the tail over a ready [rows, C] GLU equals the oracle
    tail over values g with saturated gates (sigmoid(40) clamps to
    1/(1 + e^-20), 2e-9 from one)."""
    batch, frames, channels = 3, 100, 256
    case = workloads.conv_case(35, batch, frames, channels, valid=[100, 61, 7])
    g = case.pointwise[:, :channels].copy()
    out = scope.put(np.zeros((batch * frames, channels), np.float16))
    op = abi.ConformerConvOp(
        ctx, pointwise_input=scope.put(g), depthwise_weights=scope.put(case.weights),
        batch_norm_scale=scope.put(case.scale), batch_norm_shift=scope.put(case.shift),
        valid_lengths=scope.put(case.valid), output=out, batch_size=batch, frames=frames, channels=channels,
        input_glu=True)
    try:
        op.enqueue()
        ctx.synchronize()
        assert op.plan().kernel.decode().startswith("pk_conformer_conv_glu_")
        got = out.download()
    finally:
        op.release()
    saturated = np.concatenate([g.astype(np.float32), np.full_like(g, 40.0, np.float32)], axis=1)
    want = oracle.conformer_conv(saturated, case.weights.astype(np.float32), case.scale, case.shift, case.valid,
                                 batch=batch, frames=frames).astype(np.float16)
    assert ulp_distance(got, want) <= 1


def test_fused_glu_conv_module_full_size(abi, ctx, scope, oracle, workloads):
    """The convolution module with the GLU fused into PW1's epilogue: within
    1e-2 of the reference chain and 2e-3 of the fp64 truth on every window,
    like the unfused path."""
    module = workloads.conv_module(0)
    print("fused-GLU conv module 16x188x1024", flush=True)
    _, _, y = module_on_gpu(abi, ctx, scope, module, fused_glu=True)
    rows, y_ref = full_module_on_oracle(oracle, module, "reference")
    norm, _ = oracle.relative_errors(y[rows], y_ref)
    assert norm <= F16_TOL_REFERENCE, norm
    rows, y_truth = full_module_on_oracle(oracle, module, "f64")
    norm, _ = oracle.relative_errors(y[rows], y_truth)
    assert norm <= F16_TOL_TRUTH, norm

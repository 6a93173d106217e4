"""Parity of the HIP palette path against the CPU oracle, through the C ABI.

Bars (north star): bit-exact for unpack, expansion and the prepared operand
order; fp32 GEMM within 1e-4 relative (norm-wise and max-wise) of the
reference fp32 chain; fp16 GEMM within 1e-2 norm-wise of the reference f16
accumulator chain (the reference's own rounding, emulated by the oracle) and
within 2e-3 norm-wise of the fp64 truth.
"""
import re

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
F16_TOL_REFERENCE = 1e-2
F16_TOL_TRUTH = 2e-3


class Scope:
    """Frees every device array it handed out."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.arrays = []

    def put(self, host):
        if host is None:
            return None
        arr = self.ctx.array(host)
        self.arrays.append(arr)
        return arr

    def empty(self, shape, dtype):
        arr = self.ctx.empty(shape, dtype)
        self.arrays.append(arr)
        return arr

    def close(self):
        for arr in self.arrays:
            arr.free()


@pytest.fixture
def scope(ctx):
    s = Scope(ctx)
    yield s
    s.close()


def run_case(abi, ctx, scope, case, *, variant=None, splits=None, active_rows=0, sentinel=None,
             prepared=None, capacity=None, repeats=1):
    w = case.weight
    rows = capacity or case.rows
    a_host = case.a if capacity is None else np.concatenate(
        [case.a, np.zeros((capacity - case.rows, w.inner), case.a.dtype)])
    a = scope.put(a_host)
    packed = scope.put(w.packed) if prepared is None else None
    palette = scope.put(w.palette)
    out_host = np.full((rows, w.columns), sentinel if sentinel is not None else 0, dtype=case.a.dtype)
    out = scope.put(out_host)
    bias = scope.put(case.bias)
    residual = None
    if case.residual is not None:
        r = case.residual if capacity is None else np.concatenate(
            [case.residual, np.zeros((capacity - case.rows, w.columns), case.a.dtype)])
        residual = scope.put(r)
    op = abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=out, bits=w.bits, rows=rows,
                    inner=w.inner, columns=w.columns, bias=bias, residual=residual,
                    residual_scale=case.residual_scale, activation=case.activation,
                    prepared=prepared, label=case.name)
    try:
        if variant is not None:
            op.set_variant(variant)
        if splits is not None:
            op.set_splits(splits)
        for _ in range(repeats):
            op.enqueue(active_rows)
        ctx.synchronize()
        return out.download()
    finally:
        op.release()


def variant_names(abi, ctx, scope, workloads, precision="f16"):
    """Kernel name of every compiled tile variant, by index."""
    dtype = np.float16 if precision == "f16" else np.float32
    case = workloads.gemm_case(1, 32, 64, 64, 5, dtype=dtype)
    w = case.weight
    a, packed, palette = scope.put(case.a), scope.put(w.packed), scope.put(w.palette)
    out = scope.empty((case.rows, w.columns), dtype)
    op = abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=out, bits=w.bits, rows=case.rows,
                    inner=w.inner, columns=w.columns, label="variant-names")
    try:
        names = []
        for v in range(abi.variant_count(precision)):
            op.set_variant(v)
            names.append(op.plan().kernel.decode())
        return names
    finally:
        op.release()


def k_split_of(name):
    """Order class of a kernel: pair-code variants add their K-part partial
    tiles at the end (pk_gemm_f16p_b*_n<WN>k<KS>_...); KS = 1 and every
    operand-order variant accumulate all of K in one chain; the small-M
    variants (pk_gemm_f16s_{b*,group,stream}_k<W>_...) add W round-robin K
    partials."""
    m = re.search(r"_f16s_(?:b\d_|group_|stream_)k(\d+)_", name)
    if m:
        return "small-m-k" + m.group(1)
    m = re.search(r"_n\dk(\d)_", name)
    return int(m.group(1)) if m else 1


def pair_code_variants(abi, ctx, scope, workloads):
    return [i for i, n in enumerate(variant_names(abi, ctx, scope, workloads)) if "f16p" in n]


def small_m_variants(abi, ctx, scope, workloads):
    return [i for i, n in enumerate(variant_names(abi, ctx, scope, workloads)) if "f16s" in n]


def oracle_gemm(oracle, case, mode, threads=8, rows=None):
    a = case.a if rows is None else case.a[rows]
    residual = case.residual if (case.residual is None or rows is None) else case.residual[rows]
    return oracle.gemm(a, case.weight.packed, case.weight.bits, case.weight.palette,
                       case.weight.columns, bias=case.bias, residual=residual,
                       residual_scale=case.residual_scale, activation=case.activation,
                       mode=mode, threads=threads)


def assert_f16_parity(oracle, got, case, rows=None, threads=8):
    ref = oracle_gemm(oracle, case, "f16-chain", threads=threads, rows=rows)
    truth = oracle_gemm(oracle, case, "f64", threads=threads, rows=rows)
    assert np.all(np.isfinite(got.astype(np.float32)))
    norm_ref, _ = oracle.relative_errors(got, ref)
    norm_truth, max_truth = oracle.relative_errors(got, truth)
    assert norm_ref <= F16_TOL_REFERENCE, (case.name, norm_ref)
    assert norm_truth <= F16_TOL_TRUTH, (case.name, norm_truth, max_truth)
    return norm_ref, norm_truth


# ------------------------------------------------------------------ codes


@pytest.mark.parametrize("bits", [5, 6])
def test_unpack_is_bit_exact(abi, ctx, scope, oracle, bits):
    rng = np.random.default_rng(100 + bits)
    wpg = abi.words_per_group(bits)
    cpg = abi.codes_per_group(bits)
    random_words = rng.integers(0, 2**32, size=(4099, wpg), dtype=np.uint64).astype("<u4")
    # every code position x every value, one code set per group
    one_hot = []
    for position in range(cpg):
        for value in range(1 << bits):
            codes = np.zeros(cpg, dtype=np.uint8)
            codes[position] = value
            one_hot.append(oracle.pack_codes(codes, bits)[0])
    words = np.concatenate([random_words, np.array(one_hot, dtype="<u4"),
                            np.full((3, wpg), 0xFFFFFFFF, dtype="<u4")])
    dev_words = scope.put(words)
    dev_codes = scope.empty(words.shape[0] * cpg, np.uint8)
    ctx.unpack_codes(bits, dev_words, dev_codes)
    ctx.synchronize()
    np.testing.assert_array_equal(dev_codes.download(), oracle.unpack_codes(words, bits))


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("bits,groups,inner,columns", [
    (5, 1, 1024, 4096), (6, 3, 256, 3072), (6, 1, 96, 512), (5, 2, 64, 1024)])
@pytest.mark.parametrize("layout", ["row-major", "tile-major"])
def test_expansion_is_bit_exact(abi, ctx, scope, oracle, workloads, dtype, bits, groups, inner, columns, layout):
    rng = np.random.default_rng(inner + columns + bits)
    w = workloads.palette_matrix(rng, bits, inner, columns, dtype=dtype, groups=groups)
    if layout == "tile-major" and columns % (256 if dtype == np.float16 else 128):
        pytest.skip("tile-major needs whole column tiles")
    packed = scope.put(w.packed)
    palette = scope.put(w.palette)
    target = scope.empty(inner * columns, dtype)
    ctx.expand(bits, packed, palette, target, inner, columns, layout=layout)
    ctx.synchronize()
    want = oracle.expand(w.packed, bits, inner, columns, w.palette, tile_major=(layout == "tile-major"))
    np.testing.assert_array_equal(target.download().view(np.uint8), want.reshape(-1).view(np.uint8))


@pytest.mark.parametrize("precision", ["f32", "f16", "f16-pair-codes", "f16-pair-codes-k1", "f16-pair-codes-k4",
                                       "f16-small-m"])
@pytest.mark.parametrize("bits,inner,columns,groups", [
    (5, 128, 256, 1), (6, 96, 48, 1), (6, 64, 3072, 3), (5, 160, 640, 1), (6, 32, 16, 1),
    (6, 128, 96, 3)])
def test_prepared_operand_order_is_bit_exact(abi, ctx, scope, oracle, workloads, precision, bits, inner,
                                             columns, groups):
    """A = identity and LUT[g][c] = 64*g + c make the GEMM output each code
    exactly, so this reads back the whole operand-order repack and every
    family's in-register decode (the pair-table fields of the K-split
    kernels included) bit for bit.
    (6, 128, 96, 3) puts three palette groups inside one pair-code tile."""
    variant = None
    if precision.startswith("f16-pair-codes"):
        # one K-split variant per code layout: 2 parts, 1 part, 4 parts
        want = {"f16-pair-codes": 2, "f16-pair-codes-k1": 1, "f16-pair-codes-k4": 4}[precision]
        names = variant_names(abi, ctx, scope, workloads)
        variant = next(i for i in pair_code_variants(abi, ctx, scope, workloads) if k_split_of(names[i]) == want)
        precision = "f16"
    elif precision == "f16-small-m":
        variant = small_m_variants(abi, ctx, scope, workloads)[-1]
        precision = "f16"
    if precision == "f16" and columns % 8:
        pytest.skip("f16 GEMM needs N % 8 == 0")
    dtype = np.float16 if precision == "f16" else np.float32
    rng = np.random.default_rng(inner * 7 + columns)
    codes = rng.integers(0, 1 << bits, size=(inner, columns), dtype=np.uint8)
    weight = workloads.PaletteMatrix(bits, inner, columns, codes, workloads.pack_codes(codes, bits),
                                     (64 * np.arange(groups)[:, None] + np.arange(1 << bits)[None, :]).astype(dtype))
    case = workloads.GemmCase("identity", np.eye(inner, dtype=dtype), weight)
    got = run_case(abi, ctx, scope, case, variant=variant)
    group_of = np.minimum(np.arange(columns) // (columns // groups), groups - 1)
    np.testing.assert_array_equal(got.astype(np.float64), (64 * group_of[None, :] + codes).astype(np.float64))


# ------------------------------------------------------------------ fp32


def test_single_gemm_fp32_full_config(abi, ctx, scope, oracle, workloads):
    """X[256x1024] f32, 6-bit W 1024->4096, 64-entry f32 LUT, bias; seed 0."""
    case = workloads.single_gemm_fp32(0)
    got = run_case(abi, ctx, scope, case)
    ref = oracle_gemm(oracle, case, "f32-chain")
    truth = oracle_gemm(oracle, case, "f64")
    norm, peak = oracle.relative_errors(got, ref)
    assert norm <= F32_TOL and peak <= F32_TOL, (norm, peak)
    norm, peak = oracle.relative_errors(got, truth)
    assert norm <= F32_TOL and peak <= F32_TOL, (norm, peak)


@pytest.mark.parametrize("rows,inner,columns,bits,groups,activation,bias,scale", [
    (1, 1024, 4096, 6, 1, "none", True, None),
    (37, 96, 48, 6, 1, "relu", True, None),
    (200, 1024, 3072, 5, 3, "none", False, None),
    (130, 4096, 1024, 5, 1, "none", False, 0.5),
    (64, 1024, 1024, 6, 1, "silu", False, 1.0),
])
def test_fp32_gemm_parity(abi, ctx, scope, oracle, workloads, rows, inner, columns, bits, groups,
                          activation, bias, scale):
    case = workloads.gemm_case(rows * 31 + inner, rows, inner, columns, bits, dtype=np.float32,
                               groups=groups, activation=activation, bias=bias, residual_scale=scale)
    got = run_case(abi, ctx, scope, case)
    norm, peak = oracle.relative_errors(got, oracle_gemm(oracle, case, "f32-chain"))
    assert norm <= F32_TOL and peak <= F32_TOL, (norm, peak)


# ------------------------------------------------------------------ fp16


@pytest.mark.parametrize("rows,inner,columns,bits,groups,activation,bias,scale", [
    (188, 1024, 4096, 5, 1, "silu", False, None),      # FF expand, one window
    (96, 4096, 1024, 5, 1, "none", False, 0.5),        # FF contract + 0.5 residual
    (752, 1024, 3072, 6, 3, "none", False, None),      # QKV, 3 palette groups
    (64, 1024, 1024, 6, 1, "none", False, 1.0),        # o_proj + residual
    (100, 1024, 640, 5, 1, "none", True, None),        # projector, N = 640
    (300, 256, 256, 5, 1, "relu", True, None),         # subsampling pointwise
    (1, 1024, 4096, 5, 1, "none", False, None),        # M = 1
    (33, 96, 48, 6, 1, "silu", False, None),           # K % 64 = 32, N % 32 = 16
    (260, 512, 2048, 6, 1, "none", False, None),       # conv pointwise expand
])
def test_fp16_gemm_parity(abi, ctx, scope, oracle, workloads, rows, inner, columns, bits, groups,
                          activation, bias, scale):
    case = workloads.gemm_case(rows * 17 + columns, rows, inner, columns, bits, dtype=np.float16,
                               groups=groups, activation=activation, bias=bias, residual_scale=scale)
    got = run_case(abi, ctx, scope, case)
    assert_f16_parity(oracle, got, case)


@pytest.mark.parametrize("rows,kernel", [(24768, "pk_gemm_f16p_b5_n4k1_m6n2"), (50000, "pk_gemm_f16p_b5_n2k2_m3n2")])
def test_subsampling_pointwise_plan(abi, ctx, scope, oracle, workloads, rows, kernel):
    """K = N = 256 at the subsampling's row counts: one round of 192 x 256
    tiles, or the 96 x 128 queue beyond a round (on 256 compute units),
    checked against the oracle on the first, a middle and the last row
    blocks."""
    case = workloads.gemm_case(rows, rows, 256, 256, 5, dtype=np.float16, activation="relu", bias=True)
    w = case.weight
    out = scope.empty((rows, 256), np.float16)
    op = abi.GemmOp(ctx, a=scope.put(case.a), packed=scope.put(w.packed), palette=scope.put(w.palette),
                    output=out, bits=5, rows=rows, inner=256, columns=256, bias=scope.put(case.bias),
                    activation="relu", label="subsampling-pointwise")
    try:
        planned = op.plan().kernel.decode()
        print(f"pointwise rows={rows} planned {planned}", flush=True)
        assert planned == kernel
        op.enqueue()
        ctx.synchronize()
        got = out.download()
    finally:
        op.release()
    pick = np.r_[0:400, rows // 2 - 200:rows // 2 + 200, rows - 400:rows]
    assert_f16_parity(oracle, got[pick], case, rows=pick)


@pytest.mark.parametrize("precision", ["f16", "f32"])
def test_every_tile_variant_matches(abi, ctx, scope, oracle, workloads, precision):
    """Tile shapes with the same K order compute the same sums: every
    variant of one order class (one accumulation chain over K, or KS K parts
    added at the end) agrees bit for bit, and all agree with the oracle."""
    dtype = np.float16 if precision == "f16" else np.float32
    case = workloads.gemm_case(5, 333, 320, 640, 5, dtype=dtype, activation="silu")
    names = variant_names(abi, ctx, scope, workloads, precision)
    first = {}
    for variant, name in enumerate(names):
        got = run_case(abi, ctx, scope, case, variant=variant)
        if precision == "f16":
            assert_f16_parity(oracle, got, case)
        else:
            norm, peak = oracle.relative_errors(got, oracle_gemm(oracle, case, "f32-chain"))
            assert norm <= F32_TOL and peak <= F32_TOL, (variant, norm, peak)
        ref = first.setdefault(k_split_of(name), got)
        np.testing.assert_array_equal(got.view(np.uint8), ref.view(np.uint8), err_msg=name)


@pytest.mark.parametrize("rows,inner,columns,bits,groups,activation,bias,scale", [
    (1504, 1024, 4096, 5, 1, "silu", False, None),     # FF expand, 8 windows
    (333, 1056, 640, 6, 1, "relu", True, None),        # K % 64 = 32, row tail
    (200, 1024, 3072, 6, 3, "none", False, 0.5),       # QKV groups + residual
    (97, 256, 96, 6, 3, "silu", True, None),           # 3 groups inside one tile
    (64, 4096, 1024, 5, 1, "none", False, 0.5),        # FF contract shape
])
def test_pair_code_variants_parity(abi, ctx, scope, oracle, workloads, rows, inner, columns, bits, groups,
                                   activation, bias, scale):
    """Every pair-code K-split variant against the oracle's reference f16
    chain and the fp64 truth, including tails, multi-group tiles and every
    epilogue, with repeated launches bit-identical."""
    case = workloads.gemm_case(rows + inner + columns, rows, inner, columns, bits, dtype=np.float16,
                               groups=groups, activation=activation, bias=bias, residual_scale=scale)
    ref = oracle_gemm(oracle, case, "f16-chain")
    truth = oracle_gemm(oracle, case, "f64")
    for variant in pair_code_variants(abi, ctx, scope, workloads):
        got = run_case(abi, ctx, scope, case, variant=variant, repeats=2)
        assert np.all(np.isfinite(got.astype(np.float32))), variant
        norm_ref, _ = oracle.relative_errors(got, ref)
        norm_truth, _ = oracle.relative_errors(got, truth)
        assert norm_ref <= F16_TOL_REFERENCE and norm_truth <= F16_TOL_TRUTH, (variant, norm_ref, norm_truth)


@pytest.mark.parametrize("rows,inner,columns,bits,groups,activation,bias,scale", [
    (64, 1024, 4096, 5, 1, "silu", False, None),       # FF expand, one third of a window
    (188, 1024, 3072, 6, 3, "none", False, None),      # QKV of one window, 3 groups
    (1, 4096, 1024, 5, 1, "none", False, 0.5),         # FF contract, one row
    (37, 1056, 640, 6, 1, "relu", True, None),         # K % 64 = 32, projector-like N
    (250, 256, 96, 6, 3, "silu", True, None),          # 3 groups of 32 columns
    (130, 512, 2048, 5, 1, "none", False, 1.0),        # rows past a 128-row block
])
def test_small_m_variants_parity(abi, ctx, scope, oracle, workloads, rows, inner, columns, bits, groups,
                                 activation, bias, scale):
    """Every small-M variant (eight wavefronts taking K blocks round robin,
    activations read straight from global memory) against the oracle, with
    repeated launches bit-identical."""
    case = workloads.gemm_case(rows * 3 + inner + columns, rows, inner, columns, bits, dtype=np.float16,
                               groups=groups, activation=activation, bias=bias, residual_scale=scale)
    ref = oracle_gemm(oracle, case, "f16-chain")
    truth = oracle_gemm(oracle, case, "f64")
    for variant in small_m_variants(abi, ctx, scope, workloads):
        got = run_case(abi, ctx, scope, case, variant=variant, repeats=2)
        assert np.all(np.isfinite(got.astype(np.float32))), variant
        norm_ref, _ = oracle.relative_errors(got, ref)
        norm_truth, _ = oracle.relative_errors(got, truth)
        assert norm_ref <= F16_TOL_REFERENCE and norm_truth <= F16_TOL_TRUTH, (variant, norm_ref, norm_truth)


@pytest.mark.parametrize("variant", [0, 1, 3, 5])
def test_split_inner_reduction(abi, ctx, scope, oracle, workloads, variant):
    """Split-K partial tiles are summed in split order by the last
    workgroup of each tile: every split count stays within the parity bars,
    repeated launches (counters reset in-kernel) give identical bits, and a
    K = 32 (mod 64) tail is handled in the last split."""
    case = workloads.gemm_case(77, 300, 1056, 512, 5, activation="silu")
    case_res = workloads.gemm_case(78, 129, 2048, 256, 6, residual_scale=0.5)
    for c in (case, case_res):
        kb = (c.weight.inner + 63) // 64
        for splits in sorted({1, 2, 3, min(5, kb), kb}):
            got = run_case(abi, ctx, scope, c, variant=variant, splits=splits)
            assert_f16_parity(oracle, got, c)
            again = run_case(abi, ctx, scope, c, variant=variant, splits=splits, repeats=3)
            np.testing.assert_array_equal(got.view(np.uint16), again.view(np.uint16),
                                          err_msg=f"{c.name} splits={splits}")


@pytest.mark.parametrize("precision", ["f16", "f32"])
def test_timed_enqueue_stamps_the_kernel(abi, ctx, scope, workloads, precision):
    """pk_gemm_enqueue_timed (encode with timestampWrites): the dispatch
    stamps both events, the elapsed time is positive, and the output equals
    an untimed launch bit for bit."""
    dtype = np.float16 if precision == "f16" else np.float32
    case = workloads.gemm_case(9, 300, 1024, 1024, 5, dtype=dtype, activation="silu")
    w = case.weight
    a, packed, palette = scope.put(case.a), scope.put(w.packed), scope.put(w.palette)
    outs = [scope.empty((case.rows, w.columns), dtype) for _ in range(2)]
    start, end = ctx.event(), ctx.event()
    try:
        for i, out in enumerate(outs):
            op = abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=out, bits=w.bits, rows=case.rows,
                            inner=w.inner, columns=w.columns, activation="silu", label="timed")
            try:
                if i == 0:
                    op.enqueue()
                else:
                    op.enqueue(0, None, start, end)
                ctx.synchronize()
            finally:
                op.release()
        end.synchronize()
        assert start.elapsed_ms(end) > 0.0
        np.testing.assert_array_equal(outs[0].download().view(np.uint8), outs[1].download().view(np.uint8))
    finally:
        start.destroy()
        end.destroy()


def test_active_rows_prefix_leaves_the_tail_untouched(abi, ctx, scope, oracle, workloads):
    """GemmDispatch.encode(shape) re-plans for the active prefix (gemm.ts:427-451)."""
    case = workloads.gemm_case(21, 200, 1024, 1024, 5, activation="silu")
    got = run_case(abi, ctx, scope, case, capacity=600, active_rows=200, sentinel=7.0)
    assert np.all(got[200:] == np.float16(7.0))
    assert_f16_parity(oracle, got[:200], case)


def test_prepared_weight_is_shared_and_outlives_its_owner(abi, ctx, scope, oracle, workloads):
    rng = np.random.default_rng(3)
    w = workloads.palette_matrix(rng, 5, 256, 512)
    packed = scope.put(w.packed)
    prepared = abi.PreparedWeight(ctx, 5, 256, 512, packed, label="shared")
    # one layout: operand-order codes, as many bits per code as the packed format
    assert prepared.nbytes() == 256 * 512 * 5 // 8
    cases = [workloads.GemmCase(f"user{i}", workloads.normal(rng, (64 + 32 * i, 256)), w) for i in range(2)]
    outs, ops = [], []
    for case in cases:
        a = scope.put(case.a)
        palette = scope.put(w.palette)
        out = scope.empty((case.rows, 512), np.float16)
        ops.append(abi.GemmOp(ctx, a=a, packed=None, palette=palette, output=out, bits=5,
                              rows=case.rows, inner=256, columns=512, prepared=prepared,
                              label=case.name))
        outs.append(out)
    prepared.destroy()  # the ops keep the codes alive
    for op in ops:
        op.enqueue()
    ctx.synchronize()
    for case, out in zip(cases, outs):
        assert_f16_parity(oracle, out.download(), case)
    for op in ops:
        op.release()


def test_destroyed_dispatch_raises_and_destroy_is_idempotent(abi, ctx, scope, workloads):
    case = workloads.gemm_case(1, 32, 64, 64, 5)
    a, packed, palette = scope.put(case.a), scope.put(case.weight.packed), scope.put(case.weight.palette)
    out = scope.empty((32, 64), np.float16)
    op = abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=out, bits=5, rows=32, inner=64,
                    columns=64, label="ff-test")
    op.destroy()
    op.destroy()
    with pytest.raises(abi.PaletteDestroyedError, match="ff-test was destroyed"):
        op.enqueue()
    op.release()


def test_descriptor_contract_errors(abi, ctx, scope, workloads):
    """The reference's createDispatch checks (gemm.ts:971-1161), same words."""
    case = workloads.gemm_case(2, 64, 256, 512, 5)
    a, packed, palette = scope.put(case.a), scope.put(case.weight.packed), scope.put(case.weight.palette)
    out = scope.empty((64, 512), np.float16)
    res = scope.empty((64, 512), np.float16)
    bias = scope.put(np.zeros(512, np.float32))
    base = dict(a=a, packed=packed, palette=palette, output=out, bits=5, rows=64, inner=256, columns=512,
                label="lbl")

    def make(**kw):
        args = dict(base)
        args.update(kw)
        return abi.GemmOp(ctx, **args)

    with pytest.raises(abi.PaletteRangeError, match="Unsupported GEMM shape for lbl"):
        make(inner=250)
    with pytest.raises(abi.PaletteError, match="lbl has invalid packed palette indices"):
        make(inner=224)
    with pytest.raises(abi.PaletteError, match="lbl supplies a residual scale without a residual"):
        make(residual_scale=0.5)
    with pytest.raises(abi.PaletteError, match="lbl cannot fuse bias and residual together"):
        make(bias=bias, residual=res)
    with pytest.raises(abi.PaletteError,
                       match="lbl is not a fixed production GEMM signature: M=64, K=256, N=512, "
                             "activation=none, bias=false, residualScale=none"):
        make(production_only=True)
    bad_palette = scope.put(np.zeros((1, 16), np.float16))
    with pytest.raises(abi.PaletteError, match="lbl has invalid transient palette weights"):
        make(palette=bad_palette)
    op = make()
    with pytest.raises(abi.PaletteRangeError, match=r"lbl active rows must be in \[1, 64\]"):
        op.enqueue(65)
    op.release()


def test_production_signature_is_accepted(abi, ctx, scope, workloads):
    rows = 188
    rng = np.random.default_rng(0)
    w = workloads.palette_matrix(rng, 5, 4096, 1024)
    a = scope.put(workloads.normal(rng, (rows, 4096)))
    out = scope.empty((rows, 1024), np.float16)
    bias = scope.put(np.zeros(1024, np.float32))
    op = abi.GemmOp(ctx, a=a, packed=scope.put(w.packed), palette=scope.put(w.palette), output=out,
                    bits=5, rows=rows, inner=4096, columns=1024, bias=bias,
                    label="subsampling-flatten-project", production_only=True)
    op.enqueue()
    ctx.synchronize()
    op.release()


# ------------------------------------------------------------------ FF block at full size


def test_feed_forward_block_full_size(abi, ctx, scope, oracle, workloads):
    """8 windows x 188 frames x 1024: H = SiLU(X W1) and Y = X + 0.5 H W2 run
    back to back on the device; every row of H and Y is checked against the
    oracle (about 15 s of CPU at 16 threads)."""
    ff = workloads.feed_forward_block(0)
    m = ff.x.shape[0]
    x = scope.put(ff.x)
    hidden = scope.empty((m, 4096), np.float16)
    y = scope.empty((m, 1024), np.float16)
    op1 = abi.GemmOp(ctx, a=x, packed=scope.put(ff.w1.packed), palette=scope.put(ff.w1.palette),
                     output=hidden, bits=5, rows=m, inner=1024, columns=4096, activation="silu",
                     label="ff-expand")
    op2 = abi.GemmOp(ctx, a=hidden, packed=scope.put(ff.w2.packed), palette=scope.put(ff.w2.palette),
                     output=y, bits=5, rows=m, inner=4096, columns=1024, residual=x, residual_scale=0.5,
                     label="ff-contract")
    op1.enqueue()
    op2.enqueue()
    ctx.synchronize()
    h = hidden.download()
    out = y.download()
    op1.release()
    op2.release()
    assert np.all(np.isfinite(h.astype(np.float32))) and np.all(np.isfinite(out.astype(np.float32)))
    print("FF block", m, "rows: expand", flush=True)
    assert_f16_parity(oracle, h, ff.expand_case(), threads=16)
    print("FF block: contract", flush=True)
    assert_f16_parity(oracle, out, ff.contract_case(h), threads=16)


def test_feed_forward_block_graph_replay_matches_eager(abi, ctx, workloads):
    """pk_graph_* (no reference counterpart): the FF block's two launches
    captured once and replayed three times, with eager passes on other
    inputs in between, give the eager result bit for bit every time."""
    ff = workloads.feed_forward_block(0)
    m = ff.x.shape[0]
    held = []

    def keep(a):
        held.append(a)
        return a
    try:
        x = keep(ctx.array(ff.x))
        hidden = keep(ctx.empty((m, 4096), np.float16))
        y = keep(ctx.empty((m, 1024), np.float16))
        op1 = abi.GemmOp(ctx, a=x, packed=keep(ctx.array(ff.w1.packed)), palette=keep(ctx.array(ff.w1.palette)),
                         output=hidden, bits=5, rows=m, inner=1024, columns=4096, activation="silu",
                         label="ff-expand")
        op2 = abi.GemmOp(ctx, a=hidden, packed=keep(ctx.array(ff.w2.packed)), palette=keep(ctx.array(ff.w2.palette)),
                         output=y, bits=5, rows=m, inner=4096, columns=1024, residual=x, residual_scale=0.5,
                         label="ff-contract")
        stream = ctx.stream
        op1.enqueue(0, stream)
        op2.enqueue(0, stream)
        ctx.synchronize(stream)
        eager = y.download()
        graph = abi.Graph.capture(ctx, stream)
        with graph:
            op1.enqueue(0, stream)
            op2.enqueue(0, stream)
        try:
            for replay in range(3):
                x.upload(np.flip(ff.x, axis=0).copy())       # other input, eager
                op1.enqueue(0, stream)
                op2.enqueue(0, stream)
                ctx.synchronize(stream)
                x.upload(ff.x)
                y.upload(np.zeros((m, 1024), np.float16))
                graph.launch()
                ctx.synchronize(stream)
                print("graph replay", replay, flush=True)
                np.testing.assert_array_equal(y.download().view(np.uint16), eager.view(np.uint16))
        finally:
            graph.release()
        op1.release()
        op2.release()
    finally:
        for a in held:
            a.free()


@pytest.mark.parametrize("rows,inner,columns,bits,active", [
    (3008, 1024, 4096, 5, 188),    # FF expand: 192 x 256 tile at full rows, a smaller one for one window
    (3008, 4096, 1024, 5, 376),    # FF contract: two-part K split at both row counts
    (3008, 1024, 1024, 6, 752),    # output projection, 6-bit
])
def test_active_prefix_is_replanned_and_bit_identical(abi, ctx, scope, oracle, workloads, rows, inner, columns, bits,
                                                      active):
    """An active prefix runs the tile planned for its own row count (the
    reference re-plans per active batch, gemm.ts:427-451) within the op's
    kernel family and K split, so its rows are bit-identical to the same rows
    of a full launch, and the rows past the prefix stay untouched."""
    case = workloads.gemm_case(61, rows, inner, columns, bits, activation="silu" if columns == 4096 else "none")
    w = case.weight
    a, packed, palette = scope.put(case.a), scope.put(w.packed), scope.put(w.palette)
    full = scope.put(np.zeros((rows, columns), np.float16))
    prefix = scope.put(np.full((rows, columns), 7.0, np.float16))
    ops = [abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=o, bits=bits, rows=rows, inner=inner,
                      columns=columns, activation=case.activation, label="active-prefix") for o in (full, prefix)]
    try:
        plan_full, plan_prefix = ops[0].plan(0), ops[1].plan(active)
        print("full:", plan_full.kernel.decode(), list(plan_full.grid), "prefix:", plan_prefix.kernel.decode(),
              list(plan_prefix.grid), flush=True)
        assert k_split_of(plan_full.kernel.decode()) == k_split_of(plan_prefix.kernel.decode())
        ops[0].enqueue(0)
        ops[1].enqueue(active)
        ctx.synchronize()
    finally:
        for op in ops:
            op.release()
    got_full, got_prefix = full.download(), prefix.download()
    np.testing.assert_array_equal(got_prefix[:active].view(np.uint16), got_full[:active].view(np.uint16))
    assert (got_prefix[active:] == np.float16(7.0)).all()
    sub = workloads.GemmCase("prefix", case.a[:active], w, activation=case.activation)
    assert_f16_parity(oracle, got_prefix[:active], sub)


GROUP_MEMBERS = [  # inner, columns, bits, palette groups, activation, bias, residual scale
    (1024, 4096, 5, 1, "silu", False, None),   # FF expand
    (4096, 1024, 5, 1, "none", False, 0.5),    # FF contract + 0.5 residual
    (1024, 3072, 5, 3, "none", False, None),   # QKV, 3 palette groups
    (1024, 1024, 6, 1, "none", False, 1.0),    # output projection + residual
    (1056, 640, 6, 1, "relu", True, None),     # K % 64 = 32, bias
    (256, 96, 6, 3, "silu", True, None),       # 3 palette groups of 32 columns
]


def group_fixture(abi, ctx, scope, workloads, rows, sentinel=0.0):
    """GEMM cases of GROUP_MEMBERS at `rows`, each bound twice: ops for the
    group and ops for single launches (own outputs), every op on the small-M
    layout."""
    small = small_m_variants(abi, ctx, scope, workloads)
    cases, grouped, single = [], [], []
    for i, (k, n, bits, groups, act, bias, scale) in enumerate(GROUP_MEMBERS):
        case = workloads.gemm_case(rows * 7 + i, rows, k, n, bits, groups=groups, activation=act, bias=bias,
                                   residual_scale=scale)
        cases.append(case)
        a, palette = scope.put(case.a), scope.put(case.weight.palette)
        bias_d, res = scope.put(case.bias), scope.put(case.residual)
        for ops in (grouped, single):
            out = scope.put(np.full((rows, n), sentinel, np.float16))
            op = abi.GemmOp(ctx, a=a, packed=scope.put(case.weight.packed), palette=palette, output=out, bits=bits,
                            rows=rows, inner=k, columns=n, bias=bias_d, residual=res, residual_scale=scale,
                            activation=act, label=f"member-{i}")
            op.set_variant(small[0])  # one K part: the layout group members read
            ops.append((op, out))
    return small, cases, grouped, single


@pytest.mark.parametrize("rows", [16, 64, 188])
def test_gemm_group_matches_single_launches(abi, ctx, scope, oracle, workloads, rows):
    """One group launch of independent GEMMs (5- and 6-bit, several palette
    groups, a K % 64 = 32 tail, every epilogue) gives each member the bits of
    that member launched alone on the same small-M variant, for every
    small-M variant, and the planned launch meets the oracle's bars."""
    small, cases, grouped, single = group_fixture(abi, ctx, scope, workloads, rows)
    group = abi.GemmGroup(ctx, [op for op, _ in grouped], label="parity-group")
    try:
        planned = group.plan()
        print("rows", rows, "planned", planned.kernel.decode(), list(planned.grid), flush=True)
        group.enqueue()
        ctx.synchronize()
        for case, (_, out) in zip(cases, grouped):
            assert_f16_parity(oracle, out.download(), case)
        for variant in small:
            group.set_variant(variant)
            group.enqueue()
            for op, _ in single:
                op.set_variant(variant)
                op.enqueue()
            ctx.synchronize()
            for i, ((_, g_out), (_, s_out)) in enumerate(zip(grouped, single)):
                np.testing.assert_array_equal(g_out.download().view(np.uint16), s_out.download().view(np.uint16),
                                              err_msg=f"variant {variant} member {i}")
    finally:
        group.release()
        for op, _ in grouped + single:
            op.release()


def test_gemm_group_prefix_and_lifetime(abi, ctx, scope, oracle, workloads):
    """An active prefix leaves every member's tail untouched and matches the
    full launch's rows bit for bit; the group outlives the ops it was made
    from (it holds their prepared weights)."""
    rows, active = 96, 40
    small, cases, grouped, single = group_fixture(abi, ctx, scope, workloads, rows, sentinel=7.0)
    group = abi.GemmGroup(ctx, [op for op, _ in grouped])
    try:
        for op, _ in grouped:
            op.release()
        group.enqueue(active)
        for op, _ in single:
            op.enqueue()
        ctx.synchronize()
        for i, ((_, g_out), (_, s_out)) in enumerate(zip(grouped, single)):
            got, full = g_out.download(), s_out.download()
            assert (got[active:] == np.float16(7.0)).all(), i
            sub = workloads.GemmCase("prefix", cases[i].a[:active], cases[i].weight, bias=cases[i].bias,
                                     residual=None if cases[i].residual is None else cases[i].residual[:active],
                                     residual_scale=cases[i].residual_scale, activation=cases[i].activation)
            assert_f16_parity(oracle, got[:active], sub)
    finally:
        group.release()
        for op, _ in single:
            op.release()


# Members a persistent group kernel can run (K a multiple of 512: 64 x four
# wavefronts x two blocks ahead; items inside one palette group): both code
# widths and every epilogue in one launch.
STREAM_MEMBERS = [
    (1024, 4096, 5, 1, "silu", True, None),    # FF expand + SiLU
    (4096, 1024, 5, 1, "none", False, 0.5),    # FF contract + 0.5 residual
    (1024, 3072, 5, 3, "none", False, None),   # QKV, 3 palette groups
    (1024, 1024, 6, 1, "none", False, 1.0),    # output projection + residual
    (2048, 512, 6, 1, "relu", True, None),     # K = 2048, bias, ReLU
]


@pytest.mark.parametrize("rows", [16, 64, 100])
def test_gemm_group_persistent_matches_one_shot(abi, ctx, scope, oracle, workloads, rows):
    """The persistent group kernels (one round of resident workgroups, each
    walking several work items and loading the next item's palette, first
    code blocks and activations while it multiplies the current item's last
    blocks) give every member the bits of a one-shot group launch of the
    same tile and K split (how far ahead codes are loaded changes no sum).
    Copies of the members make about 1,600 items of 128 columns, so that
    every workgroup runs several (the planned grid is checked to be smaller
    than the item count); 100 rows end in a partial row group. One copy of
    each member also meets the oracle's bars."""
    small = small_m_variants(abi, ctx, scope, workloads)
    items_per_copy = sum(-(-n // 128) for _, n, *_ in STREAM_MEMBERS) * -(-rows // 32)
    cases, ops, outs = [], [], []
    for copy in range(-(-1600 // items_per_copy)):
        for i, (k, n, bits, groups, act, bias, scale) in enumerate(STREAM_MEMBERS):
            case = workloads.gemm_case(rows * 53 + copy * 11 + i, rows, k, n, bits, groups=groups, activation=act,
                                       bias=bias, residual_scale=scale)
            out = scope.put(np.full((rows, n), 7.0, np.float16))
            op = abi.GemmOp(ctx, a=scope.put(case.a), packed=scope.put(case.weight.packed),
                            palette=scope.put(case.weight.palette), output=out, bits=bits, rows=rows, inner=k,
                            columns=n, bias=scope.put(case.bias), residual=scope.put(case.residual),
                            residual_scale=scale, activation=act, label=f"stream-{copy}-{i}")
            op.set_variant(small[0])
            cases.append(case)
            ops.append(op)
            outs.append(out)
    group = abi.GemmGroup(ctx, ops, label="stream-group")
    try:
        kinds = {}
        for v in abi.small_m_variants():
            group.set_variant(v)
            plan = group.plan()
            d = abi.describe_variant("f16", v)
            kinds[v] = (plan.kernel.decode(), plan.grid[0], (d.tile_rows, d.tile_columns, d.k_split))
        persistent = [v for v, (name, _, _) in kinds.items() if "_stream_" in name]
        assert persistent, kinds
        for v in persistent:
            name, grid, shape = kinds[v]
            partner = next(p for p, (n, _, s) in kinds.items() if s == shape and "_group_" in n)
            print("rows", rows, name, "grid", grid, "against", kinds[partner][0], "grid", kinds[partner][1],
                  flush=True)
            assert grid < kinds[partner][1], (grid, kinds[partner][1])
            # the persistent kernel twice more (launch after launch)
            results = []
            for variant, launches in ((partner, 1), (v, 1), (v, 2)):
                for out in outs:
                    out.upload(np.full(out.shape, 7.0, np.float16))
                group.set_variant(variant)
                for _ in range(launches):
                    group.enqueue()
                ctx.synchronize()
                results.append([out.download() for out in outs])
            for run in results[1:]:
                for i, (want, got) in enumerate(zip(results[0], run)):
                    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16),
                                                  err_msg=f"{name} member {i}")
        for i in range(len(STREAM_MEMBERS)):
            assert_f16_parity(oracle, results[1][i], cases[i])
    finally:
        group.release()
        for op in ops:
            op.release()


@pytest.mark.parametrize("active", [33, 1])
def test_gemm_group_persistent_prefix(abi, ctx, scope, workloads, active):
    """An active prefix on the planned persistent kernel (a partial last row
    group, or one row): rows past it keep their sentinel, and the prefix
    equals both the full launch's rows and the one-shot launch of the same
    tile bit for bit, over enough items that every workgroup runs several."""
    capacity = 96
    small = small_m_variants(abi, ctx, scope, workloads)
    items_per_copy = sum(-(-n // 128) for _, n, *_ in STREAM_MEMBERS) * -(-active // 32)
    ops, outs = [], []
    for copy in range(-(-1600 // items_per_copy)):
        for i, (k, n, bits, groups, act, bias, scale) in enumerate(STREAM_MEMBERS):
            case = workloads.gemm_case(active * 71 + copy * 13 + i, capacity, k, n, bits, groups=groups,
                                       activation=act, bias=bias, residual_scale=scale)
            out = scope.put(np.full((capacity, n), 7.0, np.float16))
            op = abi.GemmOp(ctx, a=scope.put(case.a), packed=scope.put(case.weight.packed),
                            palette=scope.put(case.weight.palette), output=out, bits=bits, rows=capacity, inner=k,
                            columns=n, bias=scope.put(case.bias), residual=scope.put(case.residual),
                            residual_scale=scale, activation=act, label=f"prefix-{copy}-{i}")
            op.set_variant(small[0])
            ops.append(op)
            outs.append(out)
    group = abi.GemmGroup(ctx, ops, label="stream-prefix")
    try:
        plan = group.plan(active)
        planned = plan.kernel.decode()
        assert "_stream_" in planned, planned
        kinds = {}
        for v in abi.small_m_variants():
            group.set_variant(v)
            e = abi.describe_variant("f16", v)
            kinds[v] = (group.plan(active).kernel.decode(), (e.tile_rows, e.tile_columns, e.k_split))
        group.set_variant(-1)
        shape = next(sh for name, sh in kinds.values() if name == planned)
        partner = next(v for v, (name, sh) in kinds.items() if sh == shape and "_group_" in name)
        print("active", active, planned, "grid", plan.grid[0], flush=True)
        runs = []
        for variant, rows in ((-1, active), (-1, 0), (partner, active)):
            for out in outs:
                out.upload(np.full(out.shape, 7.0, np.float16))
            group.set_variant(variant)
            group.enqueue(rows)
            ctx.synchronize()
            runs.append([out.download() for out in outs])
        group.set_variant(-1)
        for i, (prefix, full, one_shot) in enumerate(zip(*runs)):
            assert (prefix[active:] == np.float16(7.0)).all(), i
            np.testing.assert_array_equal(prefix[:active].view(np.uint16), full[:active].view(np.uint16),
                                          err_msg=f"member {i} prefix against full")
            np.testing.assert_array_equal(prefix.view(np.uint16), one_shot.view(np.uint16),
                                          err_msg=f"member {i} persistent against one-shot")
    finally:
        group.release()
        for op in ops:
            op.release()


def test_gemm_group_errors(abi, ctx, scope, workloads):
    """Members on another code layout, rows past the capacity and variants of
    other kernel families are refused with PK_RANGE_ERROR."""
    case = workloads.gemm_case(3, 188, 1024, 1024, 5)
    a, palette = scope.put(case.a), scope.put(case.weight.palette)
    out = scope.empty((188, 1024), np.float16)
    op = abi.GemmOp(ctx, a=a, packed=scope.put(case.weight.packed), palette=palette, output=out, bits=5, rows=188,
                    inner=1024, columns=1024, label="pair-layout")
    try:
        if k_split_of(op.plan().kernel.decode()) in (2, 4):
            with pytest.raises(abi.PaletteRangeError, match="member 0 \\(pair-layout\\) holds codes split into"):
                abi.GemmGroup(ctx, [op])
        op.set_variant(small_m_variants(abi, ctx, scope, workloads)[0])
        group = abi.GemmGroup(ctx, [op])
        try:
            with pytest.raises(abi.PaletteRangeError, match=r"active rows must be in \[1, 188\]"):
                group.enqueue(189)
            with pytest.raises(abi.PaletteRangeError, match="is not a small-M variant"):
                group.set_variant(0)
        finally:
            group.release()
    finally:
        op.release()


@pytest.mark.parametrize("rows,inner,columns,bits,groups,activation,scale", [
    (3008, 1024, 4096, 5, 1, "silu", None),    # FF expand of the encoder (LayerNorm -> W1 -> SiLU)
    (752, 1024, 3072, 5, 3, "none", None),     # QKV, 3 palette groups of 1024 columns
    (333, 1024, 2048, 6, 1, "none", None),     # row tail, 6-bit
    (188, 2048, 1024, 5, 1, "none", 0.5),      # K = 2048, residual epilogue
])
def test_row_norm_fused_gemm(abi, ctx, scope, oracle, workloads, rows, inner, columns, bits, groups, activation, scale):
    """PK_GEMM_ROW_NORM: the op multiplies LayerNorm(A) without a pass that
    writes it. Against the oracle's LayerNorm (f32 statistics, f16 output,
    layernorm.ts:309-390) followed by the GEMM, in the reference f16 chain
    and in f64, on every pair-code tile (the kernels that run it), with a
    row mean far from zero so the mean-correction term matters."""
    rng = np.random.default_rng(rows + inner)
    case = workloads.gemm_case(rows + inner + columns, rows, inner, columns, bits, groups=groups,
                               activation=activation, residual_scale=scale)
    x = (rng.standard_normal((rows, inner)) * 1.5 + 0.7).astype(np.float16)
    gamma = (1.0 + 0.2 * rng.standard_normal(inner)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(inner)).astype(np.float32)
    ln = oracle.layernorm(x, gamma, beta)
    ref_case = workloads.GemmCase("ln-gemm", ln, case.weight, residual=case.residual, residual_scale=scale,
                                  activation=activation)
    ref = oracle_gemm(oracle, ref_case, "f16-chain")
    truth = oracle_gemm(oracle, ref_case, "f64")
    w = case.weight
    a, palette = scope.put(x), scope.put(w.palette)
    g_d, b_d = scope.put(gamma), scope.put(beta)
    res = scope.put(case.residual)
    out = scope.put(np.zeros((rows, columns), np.float16))
    op = abi.GemmOp(ctx, a=a, packed=scope.put(w.packed), palette=palette, output=out, bits=bits, rows=rows,
                    inner=inner, columns=columns, residual=res, residual_scale=scale, activation=activation,
                    norm_gamma=g_d, norm_beta=b_d, label="row-norm")
    try:
        planned = op.plan().kernel.decode()
        assert planned.startswith("pk_gemm_f16p_"), planned
        variants = [planned] + [n for n in pair_code_names(abi) if n != planned]
        for name in variants:
            op.set_variant(pair_code_index(abi, name))
            op.enqueue()
            ctx.synchronize()
            got = out.download()
            assert np.all(np.isfinite(got.astype(np.float32))), name
            norm_ref, _ = oracle.relative_errors(got, ref)
            norm_truth, _ = oracle.relative_errors(got, truth)
            print(name, f"vs f16 chain {norm_ref:.2e}, vs f64 {norm_truth:.2e}", flush=True)
            assert norm_ref <= F16_TOL_REFERENCE and norm_truth <= F16_TOL_TRUTH, (name, norm_ref, norm_truth)
        with pytest.raises(abi.PaletteRangeError, match="has no fused row norm"):
            op.set_variant(abi.small_m_variants()[0])
    finally:
        op.release()


def pair_code_names(abi):
    return [abi.describe_variant("f16", v).kernel5.decode() for v in range(abi.variant_count("f16"))
            if abi.describe_variant("f16", v).kernel5.decode().startswith("pk_gemm_f16p_")]


def pair_code_index(abi, name5):
    for v in range(abi.variant_count("f16")):
        d = abi.describe_variant("f16", v)
        if d.kernel5.decode() == name5 or d.kernel6.decode() == name5:
            return v
    raise KeyError(name5)


def test_row_norm_contract_errors(abi, ctx, scope, workloads):
    """The fused row norm's own checks: K % 64, no GLU, gamma / beta sizes."""
    case = workloads.gemm_case(4, 64, 1024, 1024, 5)
    w = case.weight
    a, packed, palette = scope.put(case.a), scope.put(w.packed), scope.put(w.palette)
    out = scope.empty((64, 1024), np.float16)
    g = scope.put(np.ones(1024, np.float32))
    short = scope.put(np.ones(512, np.float32))
    with pytest.raises(abi.PaletteError, match="row norm needs gamma and beta"):
        abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=out, bits=5, rows=64, inner=1024,
                   columns=1024, norm_gamma=g, norm_beta=short, label="lbl")
    with pytest.raises(abi.PaletteError, match="row norm needs f16"):
        abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=scope.empty((64, 512), np.float16), bits=5,
                   rows=64, inner=1024, columns=1024, glu=True, norm_gamma=g, norm_beta=g, label="lbl")


@pytest.mark.parametrize("rows,inner,columns,activation,glu", [
    (3008, 1024, 4096, "silu", False),
    (752, 1024, 2048, "none", True),
])
def test_streamed_output_stores_match_plain_stores(abi, ctx, scope, oracle, workloads, rows, inner, columns,
                                                   activation, glu):
    """The f16 pair-code kernels store their output non-temporally unless
    the op keeps it cached (PK_GEMM_CACHED_OUTPUT); both ops run the same
    variant and grid, the streamed instantiation differing only in its
    stores, so the outputs are bit-identical (with the GLU epilogue too),
    and the streamed output is within tolerance of the oracle on sampled
    rows."""
    case = workloads.gemm_case(64, rows, inner, columns, 5, activation=activation)
    w = case.weight
    a, packed, palette = scope.put(case.a), scope.put(w.packed), scope.put(w.palette)
    width = columns // 2 if glu else columns
    outs, plans = {}, {}
    for cached in (False, True):
        outs[cached] = scope.put(np.full((rows, width), 7.0, np.float16))
        op = abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=outs[cached], bits=5, rows=rows,
                        inner=inner, columns=columns, activation=activation, glu=glu, cached_output=cached,
                        label="cached-output" if cached else "streamed-output")
        try:
            plans[cached] = op.plan()
            op.enqueue(0)
            ctx.synchronize()
        finally:
            op.release()
    streamed, plain = plans[False], plans[True]
    print("streamed:", streamed.kernel.decode(), list(streamed.grid), streamed.stream_stores,
          "cached:", plain.kernel.decode(), list(plain.grid), plain.stream_stores, flush=True)
    assert streamed.stream_stores == 1 and plain.stream_stores == 0
    assert streamed.kernel == plain.kernel and list(streamed.grid) == list(plain.grid)
    first, second = outs[False].download(), outs[True].download()
    np.testing.assert_array_equal(first.view(np.uint16), second.view(np.uint16))
    if not glu:
        sample = [0, 1, 191, 192, rows // 2, rows - 2, rows - 1]
        assert_f16_parity(oracle, first[sample], case, rows=sample)


@pytest.mark.parametrize("rows,inner,columns,bits,active", [
    (3008, 1024, 4096, 5, (188, 752)),   # FF expand: a 64 x 64 four-part tile at one window
    (3008, 4096, 1024, 5, (188, 1504)),  # FF contract: the small-M kernel at one window
    (3008, 1024, 1024, 6, (188, 564)),   # output projection, 6-bit
])
def test_prepared_rows_run_the_dedicated_plan(abi, ctx, scope, oracle, workloads, rows, inner, columns, bits,
                                             active):
    """pk_gemm_prepare_rows: a prepared active row count runs the plan of an
    op created for that many rows (its kernel family, K split and a copy of
    the codes in that layout), bit-identical to such a dedicated op, within
    tolerance of the oracle; the rows past the prefix stay untouched, and
    forcing a variant drops the prepared plans."""
    case = workloads.gemm_case(63, rows, inner, columns, bits, activation="silu" if columns == 4096 else "none")
    w = case.weight
    a, packed, palette = scope.put(case.a), scope.put(w.packed), scope.put(w.palette)
    prefix = scope.put(np.full((rows, columns), 7.0, np.float16))
    op = abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=prefix, bits=bits, rows=rows, inner=inner,
                    columns=columns, activation=case.activation, label="prepared-rows")
    try:
        op.prepare_rows(list(active) + [active[0]])  # a repeated count is prepared once
        for m in active:
            dedicated_out = scope.put(np.zeros((m, columns), np.float16))
            dedicated = abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=dedicated_out, bits=bits, rows=m,
                                   inner=inner, columns=columns, activation=case.activation, label="dedicated")
            try:
                plan_d, plan_p = dedicated.plan(0), op.plan(m)
                print(m, "rows: dedicated", plan_d.kernel.decode(), list(plan_d.grid), "prepared",
                      plan_p.kernel.decode(), list(plan_p.grid), flush=True)
                assert plan_d.kernel == plan_p.kernel and list(plan_d.grid) == list(plan_p.grid)
                prefix.upload(np.full((rows, columns), 7.0, np.float16))
                op.enqueue(m)
                dedicated.enqueue(0)
                ctx.synchronize()
            finally:
                dedicated.release()
            got = prefix.download()
            np.testing.assert_array_equal(got[:m].view(np.uint16), dedicated_out.download().view(np.uint16))
            assert (got[m:] == np.float16(7.0)).all()
            assert_f16_parity(oracle, got[:m], workloads.GemmCase("prefix", case.a[:m], w, activation=case.activation))
        op.set_variant(9)  # forced: every row count runs it, the prepared plans are gone
        assert op.plan(active[0]).kernel == op.plan(0).kernel == abi.describe_variant("f16", 9).__getattribute__(
            f"kernel{bits}")
    finally:
        op.release()
    with pytest.raises(abi.PaletteRangeError, match=r"prepared-rows active rows must be in \[1, 3008\]"):
        bad = abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=prefix, bits=bits, rows=rows, inner=inner,
                         columns=columns, activation=case.activation, label="prepared-rows")
        try:
            bad.prepare_rows([rows + 1])
        finally:
            bad.release()

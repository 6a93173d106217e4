"""Parity of the encoder layer stack (pk_encoder: createEncoderLayerDispatches,
src/webgpu/encoder.ts:1868-2135) against the oracle's composition of the
same ops (pko.encoder_layer), with f16 storage between ops as in the
reference's arena.

The oracle runs two chains: "f16-chain" GEMMs accumulate in binary16 as the
reference's fp16 shaders do (gemm.ts:1445-1481); "f64" GEMMs sum exactly and
round once. The device accumulates in f32, so it sits between the two and
much nearer the exact chain. Bars (norm-wise relative error, the fp16
tolerance of the palette GEMM path):
  one layer:  <= 1e-2 against either chain;
  8 layers:   <= 1e-2 against the f64 chain, and no farther from the
              reference's f16 chain than the f64 chain itself is (x1.1);
  24 layers:  <= 1e-2 against the f64 chain.
Everything the stack does per window is independent of the other windows,
so the full-size run also checks a window permutation (bit-exact), the
active prefix, and graph replay against eager launches (bit-exact)."""
import numpy as np
import pytest

from test_gpu_parity import Scope

pytestmark = pytest.mark.gpu

THREADS = 16


@pytest.fixture
def scope(ctx):
    s = Scope(ctx)
    yield s
    s.close()


def upload_layers(scope, layers):
    """Device copies of each layer dict, keyed like pk_encoder_layer."""
    out = []
    for layer in layers:
        d = {"norm_gamma": [scope.put(np.ascontiguousarray(g)) for g in layer["norm_gamma"]],
             "norm_beta": [scope.put(np.ascontiguousarray(b)) for b in layer["norm_beta"]]}
        for key, value in layer.items():
            if key.startswith("norm_"):
                continue
            d[key] = tuple(scope.put(v) for v in value) if isinstance(value, tuple) else scope.put(value)
        out.append(d)
    return out


class Stack:
    """An EncoderOp over uploaded layers with its input, output and lengths
    (and the front end and projector when the stack has them)."""

    def __init__(self, abi, ctx, scope, stack, *, fused_glu=True, fused_norms=False, unchained_norms=False,
                 prefix_same_plan=False):
        precision = "f32" if stack.x.dtype == np.float32 else "f16"
        self.ctx = ctx
        self.valid = scope.put(stack.valid)
        self.output = scope.put(np.full_like(stack.x, 77))
        extra = {}
        if stack.subsampling is not None:
            self.input = scope.put(stack.features)
            self.feature_lengths = scope.put(stack.feature_lengths)
            front = {k: (tuple(scope.put(v) for v in val) if isinstance(val, tuple) else scope.put(val))
                     for k, val in stack.subsampling.items()}
            extra.update(subsampling=front, feature_frames=stack.feature_frames,
                         feature_lengths=self.feature_lengths)
        else:
            self.input = scope.put(stack.x)
        self.projected = None
        if stack.projector is not None:
            channels = stack.projector_bias.size
            self.projected = scope.put(np.full((stack.x.shape[0], channels), 77, stack.x.dtype))
            extra.update(projector=tuple(scope.put(v) for v in stack.projector),
                         projector_bias=scope.put(stack.projector_bias), projected_channels=channels,
                         projected_output=self.projected)
        self.op = abi.EncoderOp(ctx, layers=upload_layers(scope, stack.layers), valid_lengths=self.valid,
                                input=self.input, output=self.output, batch_size=stack.batch, frames=stack.frames,
                                fused_glu=fused_glu, fused_norms=fused_norms, unchained_norms=unchained_norms,
                                prefix_same_plan=prefix_same_plan, precision=precision, **extra)

    def run(self, active=0, graph=False):
        self.op.enqueue(active, graph=graph)
        self.ctx.synchronize()
        return self.output.download()

    def run_both(self, active=0, graph=False):
        out = self.run(active, graph)
        return out, self.projected.download()

    def run_profiled(self, stamped):
        """One eager pass whose launches in `stamped` (slot indices) stamp
        their own events, the others none; returns the output and the
        stamped durations in ms."""
        launches = self.op.info()[0]
        starts = [self.ctx.event() if i in stamped else None for i in range(launches)]
        ends = [self.ctx.event() if i in stamped else None for i in range(launches)]
        self.op.enqueue_profiled(starts, ends)
        self.ctx.synchronize()
        durations = [starts[i].elapsed_ms(ends[i]) for i in sorted(stamped)]
        for ev in starts + ends:
            if ev is not None:
                ev.destroy()
        return self.output.download(), durations

    def release(self):
        self.op.release()


def windows(array, frames, first, count):
    return array[first * frames:(first + count) * frames]


@pytest.mark.parametrize("fused_glu,fused_norms", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["separate-norms", "glu-epilogue", "fused-norms", "glu-epilogue-fused-norms"])
def test_encoder_layer_matches_both_oracle_chains(abi, ctx, scope, oracle, workloads, fused_glu, fused_norms):
    stack = workloads.encoder_stack(seed=11, windows=2, frames=188, layers=1)
    enc = Stack(abi, ctx, scope, stack, fused_glu=fused_glu, fused_norms=fused_norms)
    try:
        assert enc.op.info()[0] == 15
        got = enc.run()
    finally:
        enc.release()
    assert np.isfinite(got).all()
    for mode in ("f16-chain", "f64"):
        want = oracle.encoder(stack.x, stack.layers, stack.valid, batch=2, frames=188, gemm_mode=mode,
                              threads=THREADS)
        norm, worst = oracle.relative_errors(got, want)
        print(f"one layer, fused_glu={fused_glu}, fused_norms={fused_norms}, vs {mode}: norm {norm:.2e} "
              f"max {worst:.2e}", flush=True)
        assert norm <= 1e-2, (mode, norm, worst)


def test_encoder_short_odd_windows(abi, ctx, scope, oracle, workloads):
    """Windows of 37 frames (111 rows: a partial row tile in every GEMM, a
    partial key and query tile in the attention), one full, one half and
    one single-frame window, two layers, under the bar of a stack: within
    1e-2 of the f64 chain and no farther from the f16 chain than the f64
    chain is (on these weights the two chains are 1.2% apart after two
    layers). The graph replay bit for bit."""
    stack = workloads.encoder_stack(seed=18, windows=3, frames=37, layers=2, valid=[37, 20, 1])
    enc = Stack(abi, ctx, scope, stack)
    try:
        got = enc.run()
        graph = enc.run(graph=True)
    finally:
        enc.release()
    np.testing.assert_array_equal(graph.view(np.uint16), got.view(np.uint16))
    assert np.isfinite(got).all()
    truth = oracle.encoder(stack.x, stack.layers, stack.valid, batch=3, frames=37, gemm_mode="f64",
                           threads=THREADS)
    reference = oracle.encoder(stack.x, stack.layers, stack.valid, batch=3, frames=37, gemm_mode="f16-chain",
                               threads=THREADS)
    gap, _ = oracle.relative_errors(truth, reference)
    for w, valid in enumerate(stack.valid):
        rows = slice(w * 37, w * 37 + int(valid))
        norm, worst = oracle.relative_errors(got[rows], truth[rows])
        norm16, _ = oracle.relative_errors(got[rows], reference[rows])
        print(f"window {w} ({valid} frames): vs f64 chain {norm:.2e} (max {worst:.2e}); vs f16 chain "
              f"{norm16:.2e}", flush=True)
        assert norm <= 1e-2, (w, norm, worst)
    norm, worst = oracle.relative_errors(got, truth)
    norm16, _ = oracle.relative_errors(got, reference)
    print(f"two layers of 3 x 37 frames: vs f64 chain {norm:.2e}; vs f16 chain {norm16:.2e}; chains {gap:.2e}",
          flush=True)
    assert norm <= 1e-2, (norm, worst)
    assert norm16 <= 1.1 * gap + 1e-3, (norm16, gap)


def test_encoder_two_layers_at_750_frames(abi, ctx, scope, oracle, workloads):
    """The flash-style attention inside the stack at T=750 (4 x 188 + 2),
    with one short window."""
    stack = workloads.encoder_stack(seed=12, windows=2, frames=750, layers=2, valid=[750, 377])
    enc = Stack(abi, ctx, scope, stack)
    try:
        got = enc.run()
    finally:
        enc.release()
    want = oracle.encoder(stack.x, stack.layers, stack.valid, batch=2, frames=750, gemm_mode="f64",
                          threads=THREADS)
    norm, worst = oracle.relative_errors(got, want)
    print(f"two layers at T=750 vs f64: norm {norm:.2e} max {worst:.2e}", flush=True)
    assert norm <= 1e-2, (norm, worst)


def test_encoder_24_layers_full_size(abi, ctx, scope, oracle, workloads):
    """16 windows x 188 frames x 24 layers: graph replay, the active prefix
    (PK_ENCODER_PREFIX_SAME_PLAN: the capacity's kernel families, so the
    same bits as the full pass's windows) and a window permutation
    bit-exact, then window 0 against the f64 chain."""
    stack = workloads.encoder_stack(seed=13, windows=16, frames=188, layers=24)
    enc = Stack(abi, ctx, scope, stack, prefix_same_plan=True)
    try:
        launches, device_bytes = enc.op.info()
        assert launches == 24 * 15
        eager = enc.run()
        assert np.isfinite(eager).all()
        graph = enc.run(graph=True)
        np.testing.assert_array_equal(graph.view(np.uint16), eager.view(np.uint16))
        graph_again = enc.run(graph=True)
        np.testing.assert_array_equal(graph_again.view(np.uint16), eager.view(np.uint16))

        # active prefix: the first 5 windows alone
        prefix = enc.run(active=5)
        np.testing.assert_array_equal(windows(prefix, 188, 0, 5).view(np.uint16),
                                      windows(eager, 188, 0, 5).view(np.uint16))
        prefix_graph = enc.run(active=5, graph=True)
        np.testing.assert_array_equal(windows(prefix_graph, 188, 0, 5).view(np.uint16),
                                      windows(eager, 188, 0, 5).view(np.uint16))

        # window permutation: outputs move with their windows
        order = np.roll(np.arange(16), 7)
        x_perm = stack.x.reshape(16, 188, 1024)[order].reshape(-1, 1024)
        enc.input.upload(x_perm)
        enc.valid.upload(stack.valid[order])
        permuted = enc.run().reshape(16, 188, 1024)
        np.testing.assert_array_equal(permuted.view(np.uint16), eager.reshape(16, 188, 1024)[order].view(np.uint16))
    finally:
        enc.release()

    x0 = windows(stack.x, 188, 0, 1)
    truth = oracle.encoder(x0, stack.layers, stack.valid[:1], batch=1, frames=188, gemm_mode="f64",
                           threads=THREADS)
    reference = oracle.encoder(x0, stack.layers, stack.valid[:1], batch=1, frames=188, gemm_mode="f16-chain",
                               threads=THREADS)
    got0 = windows(eager, 188, 0, 1)
    norm, worst = oracle.relative_errors(got0, truth)
    norm16, _ = oracle.relative_errors(got0, reference)
    gap, _ = oracle.relative_errors(truth, reference)
    print(f"24 layers: vs f64 chain {norm:.2e} (max {worst:.2e}); vs f16 chain {norm16:.2e}; chains apart {gap:.2e}",
          flush=True)
    assert norm <= 1e-2, (norm, worst)
    # the reference's own f16 accumulation: no farther from it than the exact chain is
    assert norm16 <= 1.1 * gap + 1e-3, (norm16, gap)


def test_encoder_eight_layers_against_the_reference_chain(abi, ctx, scope, oracle, workloads):
    """The reference's own fp16 accumulation drifts from exact sums as layers
    stack (0.6% after one layer, about 2% after eight on these weights); the
    device must be no farther from the f16 chain than the exact chain is."""
    stack = workloads.encoder_stack(seed=16, windows=1, frames=188, layers=8)
    enc = Stack(abi, ctx, scope, stack)
    try:
        got = enc.run()
    finally:
        enc.release()
    truth = oracle.encoder(stack.x, stack.layers, stack.valid, batch=1, frames=188, gemm_mode="f64",
                           threads=THREADS)
    reference = oracle.encoder(stack.x, stack.layers, stack.valid, batch=1, frames=188, gemm_mode="f16-chain",
                               threads=THREADS)
    norm, worst = oracle.relative_errors(got, truth)
    gap, _ = oracle.relative_errors(truth, reference)
    norm16, worst16 = oracle.relative_errors(got, reference)
    print(f"8 layers: vs f64 chain {norm:.2e} (max {worst:.2e}); vs f16 chain {norm16:.2e} (max {worst16:.2e}); "
          f"f64 chain vs f16 chain {gap:.2e}", flush=True)
    assert norm <= 1e-2, (norm, worst)
    assert norm16 <= 1.1 * gap + 1e-3, (norm16, gap)


def test_encoder_fused_glu_matches_unfused(abi, ctx, scope, oracle, workloads):
    """The default GLU epilogue only moves the GLU into PW1 (one more f16
    rounding of the GLU than PK_ENCODER_SEPARATE_GLU, the reference's order);
    4 layers stay within 1e-2 of the unfused stack."""
    stack = workloads.encoder_stack(seed=14, windows=4, frames=188, layers=4)
    outs = []
    for fused in (False, True):
        enc = Stack(abi, ctx, scope, stack, fused_glu=fused)
        try:
            outs.append(enc.run())
        finally:
            enc.release()
    norm, worst = oracle.relative_errors(outs[1], outs[0])
    print(f"fused vs unfused GLU, 4 layers: norm {norm:.2e} max {worst:.2e}", flush=True)
    assert norm <= 1e-2, (norm, worst)


def test_encoder_fused_norms_match_separate_norms(abi, ctx, scope, oracle, workloads):
    """The four LayerNorms that feed a GEMM, run inside it
    (PK_ENCODER_FUSED_NORMS) or as the reference's separate dispatches:
    8 layers agree within 1e-2, both stay within 1e-2 of the f64 chain, and
    the fused stack is no farther from it than the separate one by more than
    the f16 rounding the separate LayerNorm output adds."""
    stack = workloads.encoder_stack(seed=16, windows=4, frames=188, layers=8)
    outs = []
    for fused in (True, False):
        enc = Stack(abi, ctx, scope, stack, fused_norms=fused)
        try:
            outs.append(enc.run())
        finally:
            enc.release()
    want = oracle.encoder(stack.x, stack.layers, stack.valid, batch=4, frames=188, gemm_mode="f64", threads=THREADS)
    norm, worst = oracle.relative_errors(outs[0], outs[1])
    fused_err, _ = oracle.relative_errors(outs[0], want)
    separate_err, _ = oracle.relative_errors(outs[1], want)
    print(f"fused vs separate norms, 8 layers: {norm:.2e} (max {worst:.2e}); vs f64 chain: fused {fused_err:.2e}, "
          f"separate {separate_err:.2e}", flush=True)
    assert norm <= 1e-2, (norm, worst)
    assert fused_err <= 1e-2 and separate_err <= 1e-2
    assert fused_err <= separate_err + 2e-3, (fused_err, separate_err)


def test_encoder_chained_norms_match_unchained(abi, ctx, scope, workloads):
    """Each layer's last LayerNorm also writing the next layer's first one
    in the same launch (the default) gives bit-identical outputs to one
    launch per LayerNorm (PK_ENCODER_UNCHAINED_NORMS), for all windows and
    for an active prefix."""
    stack = workloads.encoder_stack(seed=17, windows=3, frames=188, layers=3)
    outs = []
    for unchained in (False, True):
        enc = Stack(abi, ctx, scope, stack, unchained_norms=unchained)
        try:
            assert enc.op.info()[0] == 15 * 3  # dispatch slots, launching or not
            outs.append((enc.run(), enc.run(active=2)))
        finally:
            enc.release()
    for got, want in zip(outs[0], outs[1]):
        assert np.isfinite(got).all()
        np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


def test_encoder_f32_profile_matches_oracle(abi, ctx, scope, oracle, workloads):
    """The reference's fp32 profile (encoder.ts:947-1165): front end, two
    layers and the projector with f32 activations, palettes, positions and
    depthwise weights (the GLU in the convolution) against the oracle's f32
    chain and the exact one, on the frames below each window's length:
    within 1e-4 of both (measured in the test's output)."""
    stack = workloads.as_f32_profile(workloads.encoder_stack(seed=41, windows=2, frames=188, layers=2,
                                                             front_end=True, projector=True))
    enc = Stack(abi, ctx, scope, stack)
    try:
        got, projected = enc.run_both()
        again, _ = enc.run_both(graph=True)
    finally:
        enc.release()
    assert got.dtype == np.float32 and np.isfinite(got).all()
    np.testing.assert_array_equal(again.view(np.uint32), got.view(np.uint32))
    for mode in ("f32-chain", "f64"):
        want, want_projected = oracle.encoder_graph(None, stack.layers, stack.valid, batch=2, frames=188,
                                                    front=stack.subsampling, features=stack.features,
                                                    feature_lengths=stack.feature_lengths,
                                                    projector=stack.projector, projector_bias=stack.projector_bias,
                                                    gemm_mode=mode, threads=THREADS, dtype=np.float32)
        norm, worst = oracle.relative_errors(valid_rows(got, stack), valid_rows(want, stack))
        pnorm, _ = oracle.relative_errors(valid_rows(projected, stack), valid_rows(want_projected, stack))
        print(f"f32 profile vs {mode}: output norm {norm:.2e} (max {worst:.2e}), projected {pnorm:.2e}", flush=True)
        assert norm <= 1e-4 and pnorm <= 1e-4, (mode, norm, worst, pnorm)


def test_encoder_rejects_bad_active_batch(abi, ctx, scope, workloads):
    stack = workloads.encoder_stack(seed=15, windows=2, frames=188, layers=1)
    enc = Stack(abi, ctx, scope, stack)
    try:
        with pytest.raises(abi.PaletteRangeError, match=r"active batch must be in \[1, 2\]"):
            enc.op.enqueue(3)
    finally:
        enc.release()


def valid_rows(array, stack, count=None):
    """The frames below each window's valid length (what the decoder reads)."""
    count = stack.batch if count is None else count
    parts = [array[b * stack.frames:b * stack.frames + int(stack.valid[b])] for b in range(count)]
    return np.concatenate(parts)


def test_encoder_graph_with_front_end_and_projector(abi, ctx, scope, oracle, workloads):
    """fbank -> subsampling -> 2 layers -> projector (encoder.ts:1690-1706),
    2 windows of 1501 fbank frames, against both oracle chains on the frames
    below each window's length, and graph replay bit-exact."""
    stack = workloads.encoder_stack(seed=21, windows=2, frames=188, layers=2, front_end=True, projector=True,
                                    feature_lengths=[1501, 799])
    enc = Stack(abi, ctx, scope, stack)
    try:
        assert enc.op.info()[0] == 6 + 2 * 15 + 1
        got, projected = enc.run_both()
        graph, graph_projected = enc.run_both(graph=True)
        np.testing.assert_array_equal(graph.view(np.uint16), got.view(np.uint16))
        np.testing.assert_array_equal(graph_projected.view(np.uint16), projected.view(np.uint16))
        # stamped passes (every launch, or a few with the others unstamped, as
        # bench.py's timed steps run) compute the same pass
        launches = enc.op.info()[0]
        for stamped in (set(range(launches)), {7, 8, 8 + 15}):
            profiled, durations = enc.run_profiled(stamped)
            np.testing.assert_array_equal(profiled.view(np.uint16), got.view(np.uint16))
            # (a chained LayerNorm slot launches nothing: its two events are back to back)
            assert len(durations) == len(stamped) and all(d >= 0 for d in durations), durations
            if len(stamped) == 3:
                assert all(d > 0 for d in durations), durations
    finally:
        enc.release()
    assert np.isfinite(got).all() and np.isfinite(projected).all()
    results = {}
    for mode in ("f64", "f16-chain"):
        results[mode] = oracle.encoder_graph(None, stack.layers, stack.valid, batch=2, frames=188,
                                             front=stack.subsampling, features=stack.features,
                                             feature_lengths=stack.feature_lengths, projector=stack.projector,
                                             projector_bias=stack.projector_bias, gemm_mode=mode, threads=THREADS)
    truth, reference = results["f64"], results["f16-chain"]
    for name, g, t, r in (("output", got, truth[0], reference[0]), ("projected", projected, truth[1], reference[1])):
        norm, worst = oracle.relative_errors(valid_rows(g, stack), valid_rows(t, stack))
        gap, _ = oracle.relative_errors(valid_rows(t, stack), valid_rows(r, stack))
        norm16, _ = oracle.relative_errors(valid_rows(g, stack), valid_rows(r, stack))
        every, _ = oracle.relative_errors(g, t)
        print(f"front end + 2 layers, {name}: vs f64 chain {norm:.2e} (max {worst:.2e}, every row {every:.2e}); "
              f"vs f16 chain {norm16:.2e}; chains apart {gap:.2e}", flush=True)
        assert norm <= 1e-2 and every <= 1e-2, (name, norm, every)
        assert norm16 <= 1.1 * gap + 1e-3, (name, norm16, gap)


def first_windows(stack, n):
    """The first n windows of a stack, with the same weights."""
    import copy
    sub = copy.copy(stack)
    sub.x, sub.valid, sub.batch = stack.x[:n * stack.frames], stack.valid[:n], n
    if stack.features is not None:
        sub.features, sub.feature_lengths = stack.features[:n], stack.feature_lengths[:n]
    return sub


def test_encoder_graph_full_size(abi, ctx, scope, oracle, workloads):
    """16 windows x 1501 fbank frames -> 24 layers -> projector: graph replay
    bit-exact; an active prefix of 3 (the default plans of a graph built for
    3 windows, eager and replayed) bit-exact with a 3-window encoder over the
    same weights and within 5e-3 of the full pass's windows; window 0
    against the f64 chain."""
    stack = workloads.encoder_stack(seed=22, windows=16, frames=188, layers=24, front_end=True, projector=True)
    enc = Stack(abi, ctx, scope, stack)
    try:
        launches, device_bytes = enc.op.info()
        assert launches == 6 + 24 * 15 + 1
        eager, eager_projected = enc.run_both()
        graph, graph_projected = enc.run_both(graph=True)
        np.testing.assert_array_equal(graph.view(np.uint16), eager.view(np.uint16))
        np.testing.assert_array_equal(graph_projected.view(np.uint16), eager_projected.view(np.uint16))
        prefix, prefix_projected = enc.run_both(active=3)
        prefix_graph, prefix_graph_projected = enc.run_both(active=3, graph=True)
    finally:
        enc.release()
    small = Stack(abi, ctx, scope, first_windows(stack, 3))
    try:
        dedicated, dedicated_projected = small.run_both(graph=True)
    finally:
        small.release()
    for got, got_projected in ((prefix, prefix_projected), (prefix_graph, prefix_graph_projected)):
        np.testing.assert_array_equal(windows(got, 188, 0, 3).view(np.uint16), dedicated.view(np.uint16))
        np.testing.assert_array_equal(windows(got_projected, 188, 0, 3).view(np.uint16),
                                      dedicated_projected.view(np.uint16))
    for got, full in ((prefix, eager), (prefix_projected, eager_projected)):
        apart, _ = oracle.relative_errors(valid_rows(windows(got, 188, 0, 3), stack, 3),
                                          valid_rows(windows(full, 188, 0, 3), stack, 3))
        print(f"prefix of 3 against the full pass's windows: {apart:.2e}", flush=True)
        assert apart <= 5e-3, apart
    assert np.isfinite(eager).all() and np.isfinite(eager_projected).all()
    chains = {mode: oracle.encoder_graph(None, stack.layers, stack.valid[:1], batch=1, frames=188,
                                         front=stack.subsampling, features=stack.features[:1],
                                         feature_lengths=stack.feature_lengths[:1], projector=stack.projector,
                                         projector_bias=stack.projector_bias, gemm_mode=mode, threads=THREADS)
              for mode in ("f64", "f16-chain")}
    for i, (name, g) in enumerate((("output", windows(eager, 188, 0, 1)),
                                   ("projected", windows(eager_projected, 188, 0, 1)))):
        t, r = chains["f64"][i], chains["f16-chain"][i]
        norm, worst = oracle.relative_errors(valid_rows(g, stack, 1), valid_rows(t, stack, 1))
        norm16, _ = oracle.relative_errors(valid_rows(g, stack, 1), valid_rows(r, stack, 1))
        gap, _ = oracle.relative_errors(valid_rows(t, stack, 1), valid_rows(r, stack, 1))
        print(f"front end + 24 layers, {name}: vs f64 chain {norm:.2e} (max {worst:.2e}); vs f16 chain "
              f"{norm16:.2e}; chains apart {gap:.2e}", flush=True)
        assert norm <= 1e-2, (name, norm, worst)
        assert norm16 <= 1.1 * gap + 1e-3, (name, norm16, gap)

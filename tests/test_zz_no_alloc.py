"""The allocation-free decoder entry point (pk_tdt_decode_static) against
the op path it varies (pk_tdt_create + pk_tdt_enqueue), bit-exact: two calls
in a row, the second over fewer windows, so the second reuses the static team
buffers the first left behind; and the call recorded into a HIP graph,
replayed beside eager work."""
import numpy as np
import pytest

from test_gpu_parity import Scope

pytestmark = pytest.mark.gpu

SENTINEL = 0xDEADBEEF


@pytest.fixture
def scope(ctx):
    s = Scope(ctx)
    yield s
    s.close()


def _slices(scope, case, max_tokens):
    B = case.batch
    return dict(
        tokens=scope.put(np.full((B, max_tokens), SENTINEL, np.uint32)),
        token_frames=scope.put(np.full((B, max_tokens), SENTINEL, np.uint32)),
        token_durations=scope.put(np.full((B, max_tokens), SENTINEL, np.uint32)),
        metadata=scope.put(np.full(2 * B, SENTINEL, np.uint32)),
        state=scope.put(np.zeros((B, 4, 640), np.float32)),
        predictor_scratch=scope.put(np.zeros((B, 5, 640), np.float32)))


def _descriptor(abi, scope, case, max_tokens):
    weights = {k: scope.put(case.weights[k]) for k in abi.TDT_WEIGHT_NAMES}
    inputs = dict(weights=weights, encoder_projected=scope.put(case.encoder_projected),
                  encoded_lengths=scope.put(case.lengths), decode_starts=scope.put(case.starts),
                  decode_ends=scope.put(case.ends), flush_finals=scope.put(case.flush), batch_size=case.batch,
                  frames=case.frames, max_tokens=max_tokens)
    return inputs


def _download(out, batch):
    meta = out["metadata"].download()
    return dict(tokens=out["tokens"].download(), frames=out["token_frames"].download(),
                durations=out["token_durations"].download(), counts=meta[:batch], status=meta[batch:],
                state=out["state"].download(), scratch=out["predictor_scratch"].download())


def _op_decode(abi, ctx, scope, inputs, case, max_tokens):
    out = _slices(scope, case, max_tokens)
    op = abi.TdtDecoderOp(ctx, **inputs, **out)
    try:
        team = op.team_size()
        op.enqueue(0)
        ctx.synchronize()
    finally:
        op.release()
    return _download(out, case.batch), team


def _static_decode(abi, ctx, scope, inputs, case, max_tokens, members):
    out = _slices(scope, case, max_tokens)
    abi.tdt_decode_static(ctx, members, None, **inputs, **out)
    ctx.synchronize()
    return _download(out, case.batch)


def _assert_same(got, want):
    for key in ("counts", "status", "tokens", "frames", "durations"):
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)
    for key in ("state", "scratch"):
        np.testing.assert_array_equal(got[key].view(np.uint32), want[key].view(np.uint32), err_msg=key)


def test_static_decode_matches_the_op_twice(abi, ctx, scope, workloads):
    max_tokens = 1024
    first = workloads.tdt_case(3, 16, 188, flush=[1, 0] * 8)
    inputs = _descriptor(abi, scope, first, max_tokens)
    want, team = _op_decode(abi, ctx, scope, inputs, first, max_tokens)
    print("call 1: 16 windows, op team", team, "counts", want["counts"], flush=True)
    got = _static_decode(abi, ctx, scope, inputs, first, max_tokens, 0)
    _assert_same(got, want)

    second = workloads.tdt_case(4, 5, 120, lengths=[120, 77, 1, 60, 119], flush=[0, 1, 1, 0, 1], blank_bias=0.0)
    inputs = _descriptor(abi, scope, second, 512)
    want, team = _op_decode(abi, ctx, scope, inputs, second, 512)
    print("call 2: 5 windows, op team", team, "counts", want["counts"], flush=True)
    for members in (16, 8, 1):
        got = _static_decode(abi, ctx, scope, inputs, second, 512, members)
        _assert_same(got, want)


def test_static_decode_rejects_more_windows_than_its_buffers(abi, ctx, scope, workloads):
    case = workloads.tdt_case(5, abi.TDT_STATIC_MAX_WINDOWS + 1, 4)
    inputs = _descriptor(abi, scope, case, 16)
    out = _slices(scope, case, 16)
    with pytest.raises(abi.PaletteError, match="exceed the 64 of the static decoder buffers"):
        abi.tdt_decode_static(ctx, 0, None, **inputs, **out)


@pytest.mark.parametrize("members", [16, 1], ids=["team16", "single"])
def test_static_decode_replays_from_a_graph(abi, ctx, scope, workloads, members):
    """pk_tdt_decode_static recorded into a HIP graph (the code it serves):
    three replays, each after eager work on the same stream (another
    decode through the op path and a reset of the outputs), each bit-exact
    with the op path's decode of the captured inputs."""
    max_tokens = 512
    case = workloads.tdt_case(6, 6, 150, lengths=[150, 90, 1, 75, 149, 120], flush=[1, 0, 1, 1, 0, 1],
                              blank_bias=0.5)
    inputs = _descriptor(abi, scope, case, max_tokens)
    want, _ = _op_decode(abi, ctx, scope, inputs, case, max_tokens)
    other = workloads.tdt_case(7, 4, 100)
    other_inputs = _descriptor(abi, scope, other, 256)
    out = _slices(scope, case, max_tokens)
    stream = ctx.stream
    abi.tdt_decode_static(ctx, members, stream, **inputs, **out)  # the device address lookup happens eagerly
    ctx.synchronize(stream)
    graph = abi.Graph.capture(ctx, stream)
    with graph:
        abi.tdt_decode_static(ctx, members, stream, **inputs, **out)
    try:
        for replay in range(3):
            _op_decode(abi, ctx, scope, other_inputs, other, 256)  # eager work between the replays
            for key in ("tokens", "token_frames", "token_durations"):
                out[key].upload(np.full((case.batch, max_tokens), SENTINEL, np.uint32))
            out["metadata"].upload(np.full(2 * case.batch, SENTINEL, np.uint32))
            out["state"].upload(np.full((case.batch, 4, 640), 7.0, np.float32))
            graph.launch()
            ctx.synchronize(stream)
            print("graph replay", replay, "members", members, flush=True)
            _assert_same(_download(out, case.batch), want)
    finally:
        graph.release()

"""Parity of the greedy TDT decoder (PersistentTdtDecoderKernel,
src/webgpu/kernels/tdt-decoder.ts:1133-2010) against the oracle, for one
workgroup per window and for teams of 8 and 16 workgroups per window (f16
profile), and for the f32 profile (:196-218, one workgroup per window).

The kernel evaluates every quantity with the oracle's arithmetic (gate and
head chains in the profile's format with one rounding per fma in increasing
k, f32 cell update, projector and joint, the same exp / tanh), so the bar is
bit-exact: the token, frame and duration sequences, the counts and status
flags, and the final state and predictor scratch of every window."""
import numpy as np
import pytest

from test_gpu_parity import Scope

pytestmark = pytest.mark.gpu


@pytest.fixture
def scope(ctx):
    s = Scope(ctx)
    yield s
    s.close()


def run_decoder(abi, scope, ctx, case, max_tokens, *, active=0, sentinel=0xDEADBEEF, team=None, precision="f16"):
    B, T = case.batch, case.frames
    weights = {k: scope.put(case.weights[k]) for k in abi.TDT_WEIGHT_NAMES}
    outs = {k: scope.put(np.full((B, max_tokens), sentinel, np.uint32)) for k in ("tokens", "frames", "durations")}
    metadata = scope.put(np.full(2 * B, sentinel, np.uint32))
    state = scope.put(np.zeros((B, 4, 640), np.float32))
    scratch = scope.put(np.zeros((B, 5, 640), np.float32))
    op = abi.TdtDecoderOp(ctx, weights=weights, encoder_projected=scope.put(case.encoder_projected),
                          encoded_lengths=scope.put(case.lengths), decode_starts=scope.put(case.starts),
                          decode_ends=scope.put(case.ends), flush_finals=scope.put(case.flush), state=state,
                          predictor_scratch=scratch, tokens=outs["tokens"], token_frames=outs["frames"],
                          token_durations=outs["durations"], metadata=metadata, batch_size=B, frames=T,
                          max_tokens=max_tokens, precision=precision)
    try:
        if team is not None:
            op.set_team_size(team)
        before = op.team_size()
        print("decoder", precision, "team", before, "batch", B, "frames", T, flush=True)
        op.enqueue(active)
        ctx.synchronize()
        # A refused team launch is an error, never a silent change of mode.
        assert op.team_size() == before
        if team:  # 0 lets the op choose
            assert op.team_size() == team
    finally:
        op.release()
    meta = metadata.download()
    got = {k: v.download() for k, v in outs.items()}
    got.update(counts=meta[:B], status=meta[B:], state=state.download(), scratch=scratch.download())
    return got


def oracle_decode(oracle, case, max_tokens, batch=None):
    b = case.batch if batch is None else batch
    return oracle.tdt_decode(case.weights, case.encoder_projected[:b], case.lengths[:b], max_tokens=max_tokens,
                             starts=case.starts[:b], ends=case.ends[:b], flush=case.flush[:b])


def assert_same_decode(got, want, batch):
    np.testing.assert_array_equal(got["counts"][:batch], want["counts"])
    np.testing.assert_array_equal(got["status"][:batch], want["status"])
    for b in range(batch):
        n = int(want["counts"][b])
        for key in ("tokens", "frames", "durations"):
            np.testing.assert_array_equal(got[key][b, :n], want[key][b, :n], err_msg=f"window {b} {key}")


@pytest.mark.parametrize("team", [1, 8, 16], ids=["single", "team8", "team16"])
@pytest.mark.parametrize("blank_bias", [2.0, 0.0], ids=["blank-favoured", "token-heavy"])
def test_decoder_matches_oracle_bit_exact(abi, ctx, scope, oracle, workloads, blank_bias, team):
    """Three windows: a full one with the flush, a bounded [5, 90) one and a
    one-frame window with the flush; with a blank-favoured head and with a
    head that emits at nearly every step (predictor after every joint)."""
    case = workloads.tdt_case(1, 3, 188, lengths=[188, 101, 1], starts=[0, 5, 0], ends=[188, 90, 188],
                              flush=[1, 0, 1], blank_bias=blank_bias)
    got = run_decoder(abi, scope, ctx, case, 512, team=team)
    want = oracle_decode(oracle, case, 512)
    print("counts", got["counts"], "oracle", want["counts"], flush=True)
    assert_same_decode(got, want, 3)
    np.testing.assert_array_equal(got["scratch"].view(np.uint32), want["scratch"].view(np.uint32))
    assert (got["tokens"][0, int(want["counts"][0]):] == 0xDEADBEEF).all()  # nothing past the count


def test_decoder_overflow_and_closed_form(abi, ctx, scope, oracle, workloads):
    """A head that always answers token 7 with duration 2 (zero head weights)
    emits at frames 0, 2, 4, ...; max_tokens below the emissions sets the
    overflow flag and keeps the first max_tokens."""
    case = workloads.tdt_case(2, 2, 40, lengths=[40, 23])
    case.weights["head_weight"][:] = 0
    case.weights["head_bias"][:] = 0
    case.weights["head_bias"][7] = 5.0
    case.weights["head_bias"][1025 + 2] = 3.0
    for team in (1, 16):
        got = run_decoder(abi, scope, ctx, case, 16, team=team)
        assert list(got["counts"]) == [16, 12] and list(got["status"]) == [1, 0]
    assert list(got["frames"][0, :16]) == list(range(0, 32, 2))
    assert (got["tokens"][1, :12] == 7).all() and (got["durations"][1, :12] == 2).all()
    assert_same_decode(got, oracle_decode(oracle, case, 16), 2)


@pytest.mark.parametrize("team", [0, 1], ids=["chosen", "single"])
def test_decoder_full_size_and_active_prefix(abi, ctx, scope, oracle, workloads, team):
    """16 windows x 188 frames, ragged lengths, flush on half of them, bit-exact
    against the oracle with the team the op chooses (16 workgroups per window
    on a 256-CU MI355X) and with one workgroup per window; an active prefix
    of 5 leaves the other windows' outputs untouched."""
    case = workloads.tdt_case(3, 16, 188, flush=[1, 0] * 8)
    got = run_decoder(abi, scope, ctx, case, 1024, team=team)
    want = oracle_decode(oracle, case, 1024)
    print("counts", got["counts"], flush=True)
    assert_same_decode(got, want, 16)
    np.testing.assert_array_equal(got["state"].view(np.uint32), want["state"].view(np.uint32))
    np.testing.assert_array_equal(got["scratch"].view(np.uint32), want["scratch"].view(np.uint32))
    prefix = run_decoder(abi, scope, ctx, case, 1024, active=5, team=team)
    np.testing.assert_array_equal(prefix["counts"][:5], want["counts"][:5])
    for b in range(5):
        n = int(want["counts"][b])
        np.testing.assert_array_equal(prefix["tokens"][b, :n], want["tokens"][b, :n])
    assert (prefix["counts"][5:] == 0xDEADBEEF).all() and (prefix["tokens"][5:] == 0xDEADBEEF).all()


def test_decoder_dispatch_errors(abi, ctx, scope, workloads):
    case = workloads.tdt_case(4, 2, 8)
    weights = {k: scope.put(case.weights[k]) for k in abi.TDT_WEIGHT_NAMES}
    slices = dict(encoder_projected=scope.put(case.encoder_projected), encoded_lengths=scope.put(case.lengths),
                  decode_starts=scope.put(case.starts), decode_ends=scope.put(case.ends),
                  flush_finals=scope.put(case.flush), state=scope.empty((2, 4, 640), np.float32),
                  predictor_scratch=scope.empty((2, 5, 640), np.float32), tokens=scope.empty((2, 4), np.uint32),
                  token_frames=scope.empty((2, 4), np.uint32), token_durations=scope.empty((2, 4), np.uint32),
                  metadata=scope.empty(4, np.uint32))
    op = abi.TdtDecoderOp(ctx, weights=weights, batch_size=2, frames=8, max_tokens=4, label="tdt-errors", **slices)
    try:
        with pytest.raises(abi.PaletteRangeError, match=r"tdt-errors active batch must be in \[1, 2\]"):
            op.enqueue(3)
        with pytest.raises(abi.PaletteRangeError, match="tdt-errors team size must be 0, 1, 8 or 16"):
            op.set_team_size(4)
        assert op.team_size() == 16
        op.destroy()
        op.destroy()
        with pytest.raises(abi.PaletteError, match="tdt-errors was destroyed"):
            op.enqueue()
    finally:
        op.release()


@pytest.mark.parametrize("blank_bias", [2.0, 0.0], ids=["blank-favoured", "token-heavy"])
def test_decoder_f32_profile_matches_oracle_bit_exact(abi, ctx, scope, oracle, workloads, blank_bias):
    """The f32 profile (f32 weights and encoder rows, f32 chains): the three
    edge windows of the f16 test, bit-exact with the oracle's f32 decode."""
    case = workloads.tdt_case(11, 3, 188, lengths=[188, 101, 1], starts=[0, 5, 0], ends=[188, 90, 188],
                              flush=[1, 0, 1], blank_bias=blank_bias, precision="f32")
    assert case.weights["head_weight"].dtype == np.float32 and case.encoder_projected.dtype == np.float32
    got = run_decoder(abi, scope, ctx, case, 512, precision="f32")
    want = oracle_decode(oracle, case, 512)
    print("counts", got["counts"], "oracle", want["counts"], flush=True)
    assert_same_decode(got, want, 3)
    np.testing.assert_array_equal(got["scratch"].view(np.uint32), want["scratch"].view(np.uint32))


def test_decoder_f32_profile_full_size(abi, ctx, scope, oracle, workloads):
    """16 windows x 188 frames in the f32 profile: the op chooses one
    workgroup per window (teams are f16 only) and matches the oracle bit for
    bit, final state included; teams of 8 / 16 are refused."""
    case = workloads.tdt_case(12, 16, 188, flush=[0, 1] * 8, blank_bias=1.0, precision="f32")
    got = run_decoder(abi, scope, ctx, case, 1024, precision="f32")
    want = oracle_decode(oracle, case, 1024)
    print("counts", got["counts"], flush=True)
    assert_same_decode(got, want, 16)
    np.testing.assert_array_equal(got["state"].view(np.uint32), want["state"].view(np.uint32))
    np.testing.assert_array_equal(got["scratch"].view(np.uint32), want["scratch"].view(np.uint32))
    with pytest.raises(abi.PaletteRangeError, match="team decoding is built for the f16 profile"):
        run_decoder(abi, scope, ctx, case, 1024, precision="f32", team=16)

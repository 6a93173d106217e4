"""The Node host (parakeet.wgsl_amd/host over the N-API addon) - the
drop-in for the reference's TypeScript GEMM owners. CPU: exports, record
checks and the descriptor contract with the reference's messages. GPU: one
GEMM driven through HipGpuDevice / arena / createDispatch / encode / submit,
checked against the oracle."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")
ADDON = os.path.join(ROOT, "parakeet.wgsl_amd", "lib", "pk_napi.node")

needs_node = pytest.mark.skipif(NODE is None, reason="node is not installed")


def run_node(script, *args, timeout=120):
    proc = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", script), *args],
                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=timeout)
    assert proc.returncode == 0, proc.stdout
    return proc.stdout


@needs_node
def test_addon_is_built():
    assert os.path.exists(ADDON), "build the addon with `python parakeet.wgsl_amd/build.py`"


@needs_node
def test_node_host_contract_on_cpu():
    assert "host_cpu ok" in run_node("host_cpu.js")


@needs_node
@pytest.mark.gpu
@pytest.mark.parametrize("bits,activation,scale,groups,active", [
    (5, "silu", None, 1, 300),
    (6, "none", 0.5, 3, 211),
])
def test_node_host_gemm_matches_oracle(tmp_path, oracle, workloads, bits, activation, scale, groups, active):
    rows, inner, columns = 300, 1024, 768
    case = workloads.gemm_case(400 + bits, rows, inner, columns, bits, groups=groups, activation=activation,
                               residual_scale=scale)
    files = {}
    for name, arr in (("a", case.a), ("packed", case.weight.packed), ("palette", case.weight.palette),
                      ("residual", case.residual)):
        if arr is None:
            continue
        files[name] = str(tmp_path / f"{name}.bin")
        np.ascontiguousarray(arr).tofile(files[name])
    spec = dict(files, rows=rows, inner=inner, columns=columns, bits=bits, groups=groups, activation=activation,
                residualScale=scale, activeRows=active, output=str(tmp_path / "out.bin"))
    (tmp_path / "case.json").write_text(json.dumps(spec))
    print(run_node("host_gpu.js", str(tmp_path / "case.json")))
    got = np.fromfile(tmp_path / "out.bin", dtype=np.float16).reshape(rows, columns)[:active]
    ref = oracle.gemm(case.a[:active], case.weight.packed, bits, case.weight.palette, columns,
                      residual=None if case.residual is None else case.residual[:active],
                      residual_scale=scale, activation=activation, mode="f16-chain", threads=8)
    truth = oracle.gemm(case.a[:active], case.weight.packed, bits, case.weight.palette, columns,
                        residual=None if case.residual is None else case.residual[:active],
                        residual_scale=scale, activation=activation, mode="f64", threads=8)
    assert oracle.relative_errors(got, ref)[0] <= 1e-2
    assert oracle.relative_errors(got, truth)[0] <= 2e-3


@needs_node
@pytest.mark.gpu
def test_node_host_conv_matches_oracle(tmp_path, oracle, workloads):
    """The conv tail through the Node host (FusedConformerConvKernel) on 3
    windows with an active batch of 2: within one f16 ulp of the oracle."""
    batch, frames = 3, 188
    case = workloads.conv_case(21, batch, frames, 1024, valid=[188, 97, 150])
    files = {}
    for name in ("pointwise", "weights", "scale", "shift", "valid"):
        files[name] = str(tmp_path / f"{name}.bin")
        np.ascontiguousarray(getattr(case, name)).tofile(files[name])
    spec = dict(files, batchSize=batch, frames=frames, activeBatch=2, output=str(tmp_path / "out.bin"))
    (tmp_path / "case.json").write_text(json.dumps(spec))
    print(run_node("host_gpu_conv.js", str(tmp_path / "case.json")))
    got = np.fromfile(tmp_path / "out.bin", dtype=np.float16).reshape(batch * frames, 1024)[:2 * frames]
    want = oracle.conformer_conv(case.pointwise[:2 * frames], case.weights, case.scale, case.shift, case.valid[:2],
                                 batch=2, frames=frames)
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    assert np.all(diff <= ulp * 1.0 + 1e-12)


@needs_node
@pytest.mark.gpu
def test_node_host_attention_matches_oracle(tmp_path, oracle, workloads):
    """The relative attention through the Node host (RelativeAttentionKernel,
    reference package layout for the positions) on 3 windows, active batch 2."""
    batch, frames = 3, 188
    case = workloads.attention_case(60, batch, frames, valid=[188, 120, 150])
    files = {}
    for name, arr in (("qkv", case.qkv), ("positions", case.packed_positions), ("biasU", case.bias_u),
                      ("biasV", case.bias_v), ("valid", case.valid)):
        files[name] = str(tmp_path / f"{name}.bin")
        np.ascontiguousarray(arr).tofile(files[name])
    spec = dict(files, batchSize=batch, frames=frames, activeBatch=2, output=str(tmp_path / "out.bin"))
    (tmp_path / "case.json").write_text(json.dumps(spec))
    print(run_node("host_gpu_attention.js", str(tmp_path / "case.json")))
    got = np.fromfile(tmp_path / "out.bin", dtype=np.float16).reshape(batch * frames, 1024)[:2 * frames]
    want = oracle.relative_attention(case.qkv[:2 * frames], case.packed_positions, case.bias_u, case.bias_v,
                                     case.valid[:2], batch=2, frames=frames)
    assert oracle.relative_errors(got, want)[0] <= 2e-3


def encoder_package_tensors(stack):
    """The stack's tensors under the reference package's names and records
    (model/convert.py:1264-1475, :1608-1702; encoder.ts:2458-2548)."""
    def palette(name, packed, lut, inner, columns, bits):
        groups = lut.shape[0]
        cpg, wpg = (32, 5) if bits == 5 else (16, 3)
        yield name, packed, "uint32", [inner, columns], [inner * columns // cpg, wpg], \
            f"k-by-output-row-major-palette{bits}-lsb-u32"
        yield f"{name}.palette", lut, "float16", [groups, 1 << bits], [groups, 1 << bits], "output-group-by-palette-lut"

    def channel(name, values, layout="channel"):
        yield name, values, "float32", [values.size], [values.size], layout

    frames = stack.frames
    norms = ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out")
    matrices = {"ff1_linear1": "feed_forward1.linear1", "ff1_linear2": "feed_forward1.linear2",
                "qkv": "self_attn.qkv", "o_proj": "self_attn.o_proj", "pointwise1": "conv.pointwise_conv1",
                "pointwise2": "conv.pointwise_conv2", "ff2_linear1": "feed_forward2.linear1",
                "ff2_linear2": "feed_forward2.linear2"}
    from parakeet_wgsl_amd.workloads import ENCODER_MATRICES
    for i, layer in enumerate(stack.layers):
        p = f"encoder.layers.{i}"
        for j, norm in enumerate(norms):
            yield from channel(f"{p}.{norm}.weight", layer["norm_gamma"][j])
            yield from channel(f"{p}.{norm}.bias", layer["norm_beta"][j])
        for key, name in matrices.items():
            bits, inner, columns, _ = ENCODER_MATRICES[key]
            yield from palette(f"{p}.{name}.weight", *layer[key], inner, columns, bits)
        yield f"{p}.self_attn.projected_positions", layer["projected_positions"], "float16", \
            [2 * frames - 1, 1024], [8, 32, 2 * frames - 1, 4], "head-vector-position-vec4"
        for b in ("bias_u", "bias_v"):
            yield f"{p}.self_attn.{b}", layer[b], "float32", [8, 128], [8, 128], "head-by-channel"
        yield f"{p}.conv.depthwise_conv.weight", layer["depthwise"], "float16", [9, 1024], [9, 256, 4], \
            "kernel-channel-vec4"
        yield from channel(f"{p}.conv.norm.scale", layer["bn_scale"])
        yield from channel(f"{p}.conv.norm.shift", layer["bn_shift"])
    f, s = stack.subsampling, "encoder.subsampling"
    for idx, key, layout in ((0, "conv0", "kh-kw-output-channel-vec4"), (2, "depthwise2", "kh-kw-channel-vec4"),
                             (5, "depthwise5", "kh-kw-channel-vec4")):
        yield f"{s}.layers.{idx}.weight", f[f"{key}_weights"], "float16", [3, 3, 256], [3, 3, 64, 4], layout
        yield from channel(f"{s}.layers.{idx}.bias", f[f"{key}_bias"], "output-channel")
    for idx, key in ((3, "pointwise3"), (6, "pointwise6")):
        yield from palette(f"{s}.layers.{idx}.weight", *f[key], 256, 256, 5)
        yield from channel(f"{s}.layers.{idx}.bias", f[f"{key}_bias"], "output-channel")
    yield from palette(f"{s}.linear.weight", *f["linear"], 4096, 1024, 5)
    yield from channel(f"{s}.linear.bias", f["linear_bias"], "output-channel")
    yield from palette("encoder_projector.weight", *stack.projector, 1024, 640, 5)
    yield from channel("encoder_projector.bias", stack.projector_bias, "output-channel")


@needs_node
@pytest.mark.gpu
def test_node_host_encoder_graph(tmp_path, abi, ctx, oracle, workloads):
    """ParakeetEncoderGraph through the Node host (fbank -> front end -> 2
    layers -> projector, 2 windows): eager, graph and profiled passes
    bit-identical to each other and to the C ABI's own run of the same
    weights, and within 1e-2 of the oracle's f64 chain on the valid frames."""
    from test_gpu_encoder import Scope, Stack, valid_rows
    stack = workloads.encoder_stack(seed=31, windows=2, frames=188, layers=2, front_end=True, projector=True,
                                    feature_lengths=[1501, 700])
    tensors = {}
    for k, (name, array, dtype, logical, storage, layout) in enumerate(encoder_package_tensors(stack)):
        path = str(tmp_path / f"t{k}.bin")
        np.ascontiguousarray(array).tofile(path)
        tensors[name] = dict(file=path, dtype=dtype, logicalShape=logical, storageShape=storage, layout=layout)
    np.ascontiguousarray(stack.features).tofile(tmp_path / "features.bin")
    spec = dict(tensors=tensors, features=str(tmp_path / "features.bin"), batchSize=2, layers=2,
                featureLengths=[int(v) for v in stack.feature_lengths],
                encoderLengths=[int(v) for v in stack.valid],
                output=str(tmp_path / "out.bin"), projected=str(tmp_path / "projected.bin"))
    (tmp_path / "case.json").write_text(json.dumps(spec))
    print(run_node("host_gpu_encoder.js", str(tmp_path / "case.json")))
    got = np.fromfile(tmp_path / "out.bin", dtype=np.float16).reshape(-1, 1024)
    projected = np.fromfile(tmp_path / "projected.bin", dtype=np.float16).reshape(-1, 640)
    scope = Scope(ctx)
    try:
        enc = Stack(abi, ctx, scope, stack)
        try:
            want, want_projected = enc.run_both()
        finally:
            enc.release()
    finally:
        scope.close()
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
    np.testing.assert_array_equal(projected.view(np.uint16), want_projected.view(np.uint16))
    truth = oracle.encoder_graph(None, stack.layers, stack.valid, batch=2, frames=188, front=stack.subsampling,
                                 features=stack.features, feature_lengths=stack.feature_lengths,
                                 projector=stack.projector, projector_bias=stack.projector_bias, gemm_mode="f64",
                                 threads=16)
    assert oracle.relative_errors(valid_rows(got, stack), valid_rows(truth[0], stack))[0] <= 1e-2
    assert oracle.relative_errors(valid_rows(projected, stack), valid_rows(truth[1], stack))[0] <= 1e-2


@needs_node
def test_node_host_package_format_on_cpu(tmp_path):
    """parseParakeetManifest / planRuntimePackage / ParakeetGpuPackage.load
    of the Node host over the converter-shaped synthetic inventory (fp16 and
    fp32 manifests, and a zero-filled fp16 package written to disk): the
    reference tests' plan expectations and rejections, the loader's digest,
    length and tokenizer checks with every buffer freed on failure, and the
    decoder's weight-record checks."""
    import package_fixture
    for precision in ("fp16", "fp32"):
        (tmp_path / f"{precision}.json").write_text(json.dumps(package_fixture.manifest(precision)))
    manifest = package_fixture.write_package(str(tmp_path / "package"))
    out = run_node("host_cpu_package.js", str(tmp_path / "fp16.json"), str(tmp_path / "fp32.json"), manifest)
    assert "package checks passed" in out


@needs_node
@pytest.mark.gpu
@pytest.mark.parametrize("precision", ["fp16", "fp32"])
def test_node_host_transcribe_from_package(tmp_path, abi, ctx, oracle, workloads, precision):
    """End to end through the Node host: a converter-shaped synthetic
    package (24 layers, the decoder shard; parakeet-webgpu-v1 or
    parakeet-webgpu-fp32-v1) loaded by ParakeetGpuPackage,
    ParakeetEncoderGraph over its tensors (4 windows of fbank, graph replay)
    and PersistentTdtDecoderKernel over arena slices, in the package's
    execution profile. The projector output is bit-identical to the C ABI
    encoder run with the same weights, and the token, frame and duration
    streams, counts and status flags are bit-identical to the oracle's decode
    of that projector output."""
    import hashlib
    import package_fixture
    from test_gpu_encoder import Scope, Stack
    windows, max_tokens = 4, 2048
    f32 = precision == "fp32"
    stack = workloads.encoder_stack(seed=41, windows=windows, frames=188, layers=24, front_end=True, projector=True,
                                    feature_lengths=[1501, 1200, 801, 37])
    if f32:
        stack = workloads.as_f32_profile(stack)
    tdt = workloads.tdt_weights(np.random.default_rng(42), blank_bias=1.0, precision="f32" if f32 else "f16")
    manifest = package_fixture.write_package(str(tmp_path / "package"), stack, tdt, precision=precision)
    np.ascontiguousarray(stack.features).tofile(tmp_path / "features.bin")
    spec = dict(precision=precision, manifest=manifest,
                manifestSha256=hashlib.sha256(open(manifest, "rb").read()).hexdigest(),
                windows=windows, maxTokens=max_tokens, features=str(tmp_path / "features.bin"),
                featureLengths=[int(v) for v in stack.feature_lengths], projected=str(tmp_path / "projected.bin"),
                decoded=str(tmp_path / "decoded.json"))
    (tmp_path / "case.json").write_text(json.dumps(spec))
    print(run_node("host_gpu_transcribe.js", str(tmp_path / "case.json"), timeout=300), flush=True)
    element = np.float32 if f32 else np.float16
    projected = np.fromfile(tmp_path / "projected.bin", dtype=element).reshape(windows, 188, 640)
    scope = Scope(ctx)
    try:
        enc = Stack(abi, ctx, scope, stack)
        try:
            _, want_projected = enc.run_both()
        finally:
            enc.release()
    finally:
        scope.close()
    bits = np.uint32 if f32 else np.uint16
    np.testing.assert_array_equal(projected.reshape(-1, 640).view(bits), want_projected.view(bits))
    decoded = json.loads((tmp_path / "decoded.json").read_text())
    meta = np.asarray(decoded["metadata"], np.uint32)
    want = oracle.tdt_decode(tdt, projected, stack.valid.astype(np.uint32), max_tokens=max_tokens,
                             starts=np.zeros(windows, np.uint32), ends=np.full(windows, 188, np.uint32),
                             flush=np.ones(windows, np.uint32))
    np.testing.assert_array_equal(meta[:windows], want["counts"])
    np.testing.assert_array_equal(meta[windows:], want["status"])
    assert want["counts"].sum() > 0
    for key, name in (("tokens", "tokens"), ("frames", "tokenFrames"), ("durations", "tokenDurations")):
        got = np.asarray(decoded[name], np.uint32).reshape(windows, max_tokens)
        for b in range(windows):
            n = int(want["counts"][b])
            np.testing.assert_array_equal(got[b, :n], want[key][b, :n], err_msg=f"window {b} {key}")

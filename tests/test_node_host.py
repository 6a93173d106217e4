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

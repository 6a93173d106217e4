"""CPU-only checks of the C-ABI library: it loads, exports exactly what
include/pk_palette.h declares, and the binding covers every entry point.
No compute call is made (this container has no GPU)."""
import ctypes
import json
import os
import re
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pk_palette.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pk_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ["pk_context_create", "pk_gemm_create", "pk_gemm_enqueue", "pk_gemm_destroy",
                     "pk_prepared_weight_create", "pk_palette_expand", "pk_unpack_codes",
                     "pk_gemm_plan", "pk_last_error"]:
        assert required in names


def test_library_exports_every_declared_symbol(abi):
    lib = abi.load()
    exported = subprocess.run(["nm", "-D", "--defined-only", abi.LIB_PATH], check=True,
                              capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (pk_[a-z0-9_]+)$", exported, flags=re.M))
    for name in declared_functions():
        assert name in exported, name
        assert hasattr(lib, name)
    assert set(abi.SIGNATURES) == set(declared_functions())


def test_library_links_only_the_hip_runtime(abi):
    deps = subprocess.run(["ldd", abi.LIB_PATH], capture_output=True, text=True).stdout
    assert "libamdhip64" in deps
    for forbidden in ["liboracle", "libtorch", "libc10", "libpython"]:
        assert forbidden not in deps


def test_struct_layouts_match_the_c_compiler(abi, tmp_path):
    """Every ctypes field offset equals the C compiler's offsetof()."""
    structs = {"pk_weight_desc": abi.WeightDesc, "pk_gemm_desc": abi.GemmDesc,
               "pk_expand_desc": abi.ExpandDesc, "pk_gemm_plan_info": abi.PlanInfo,
               "pk_device_info": abi.DeviceInfo}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "pk_palette.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {}
    for line in out:
        if line:
            cname, field, value = line.split()
            got[(cname, field)] = int(value)
    for cname, cls in structs.items():
        assert got[(cname, "sizeof")] == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert got[(cname, field)] == getattr(cls, field).offset, (cname, field)


def test_abi_version_and_status_names(abi):
    lib = abi.load()
    assert lib.pk_abi_version() == 1
    assert lib.pk_status_name(abi.RANGE_ERROR) == b"PK_RANGE_ERROR"
    assert lib.pk_status_name(99) == b"PK_UNKNOWN"


def test_null_arguments_fail_with_a_message(abi):
    lib = abi.load()
    assert lib.pk_context_create(0, None) == abi.INVALID_ARGUMENT
    assert b"null" in lib.pk_last_error()
    assert lib.pk_gemm_enqueue(None, 0, None) == abi.INVALID_ARGUMENT
    assert lib.pk_gemm_destroy(None) == abi.OK
    assert lib.pk_prepared_weight_destroy(None) == abi.OK
    assert lib.pk_context_destroy(None) == abi.OK


def test_plan_of_variants_is_listed(abi):
    assert abi.variant_count("f16") >= 1
    assert abi.variant_count("f32") >= 1


def test_workload_packer_matches_oracle(oracle, workloads):
    rng = np.random.default_rng(4)
    for bits in (5, 6):
        codes = rng.integers(0, 1 << bits, size=(128, 256), dtype=np.uint8)
        np.testing.assert_array_equal(workloads.pack_codes(codes, bits), oracle.pack_codes(codes, bits))


def test_workload_generators_are_stable(workloads):
    with open(os.path.join(ROOT, "tests", "golden", "workload_draws.json")) as f:
        fx = json.load(f)
    c1 = workloads.single_gemm_fp32(0)
    d = fx["single_gemm_fp32_seed0"]
    assert [float(v) for v in c1.a.reshape(-1)[:8]] == d["x_first8"]
    assert [int(v) for v in c1.weight.codes.reshape(-1)[:8]] == d["codes_first8"]
    assert [int(v) for v in c1.weight.packed.reshape(-1)[:4]] == d["packed_first4"]
    ff = workloads.feed_forward_block(0)
    d = fx["feed_forward_seed0"]
    assert [int(v) for v in ff.x.view("<u2").reshape(-1)[:8]] == d["x_first8_f16_bits"]
    assert [int(v) for v in ff.w1.codes.reshape(-1)[:8]] == d["w1_codes_first8"]
    assert [int(v) for v in ff.w2.codes.reshape(-1)[:8]] == d["w2_codes_first8"]
    assert ff.x.shape == (1504, 1024)
    assert ff.w1.packed.shape == (1024 * 4096 // 32, 5)


def test_algorithmic_bytes_formula(workloads):
    c1 = workloads.single_gemm_fp32(0)
    # 6-bit codes + 64 f32 LUT + X + Y + bias
    assert c1.algorithmic_bytes() == 1024 * 4096 * 6 // 8 + 256 + 256 * 1024 * 4 + 256 * 4096 * 4 + 4096 * 4
    assert c1.flops == 2 * 256 * 1024 * 4096

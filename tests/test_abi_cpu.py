"""CPU-only checks of the C-ABI library: it loads, exports exactly what
include/*.h declares, and the binding covers every entry point. No compute
call is made (this container has no GPU); the host-side contract checks and
launch plans are exercised through the device-free entry points."""
import ctypes
import glob
import json
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
        names.update(re.findall(r"\b(pk_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ["pk_context_create", "pk_gemm_create", "pk_gemm_enqueue", "pk_gemm_destroy",
                     "pk_prepared_weight_create", "pk_palette_expand", "pk_unpack_codes",
                     "pk_gemm_plan", "pk_last_error", "pk_conv_create", "pk_conv_enqueue",
                     "pk_conv_destroy", "pk_conv_plan_shape"]:
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
               "pk_device_info": abi.DeviceInfo, "pk_conv_desc": abi.ConvDesc,
               "pk_conv_plan_info": abi.ConvPlanInfo, "pk_attention_desc": abi.AttentionDesc,
               "pk_attention_plan_info": abi.AttentionPlanInfo, "pk_layernorm_desc": abi.LayerNormDesc,
               "pk_subsampling_fused_desc": abi.SubsamplingFusedDesc,
               "pk_subsampling_depthwise_desc": abi.SubsamplingDepthwiseDesc,
               "pk_subsampling_mask_desc": abi.SubsamplingMaskDesc,
               "pk_subsampling_plan_info": abi.SubsamplingPlanInfo,
               "pk_tdt_weights": abi.TdtWeights, "pk_tdt_desc": abi.TdtDesc,
               "pk_tdt_execution_plan": abi.TdtExecutionPlan,
               "pk_encoder_matrix": abi.EncoderMatrix, "pk_encoder_layer": abi.EncoderLayer,
               "pk_encoder_subsampling": abi.EncoderSubsampling, "pk_encoder_desc": abi.EncoderDesc}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "pk_palette.h"', '#include "pk_conv.h"',
             '#include "pk_attention.h"', '#include "pk_layernorm.h"', '#include "pk_subsampling.h"',
             '#include "pk_encoder.h"', '#include "pk_tdt.h"',
             "int main(void) {"]
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


def test_variant_descriptions(abi):
    """Every compiled variant describes itself without a device: kernel
    names per code width, tile, K split, the code layout it reads, and
    whether a GEMM group can run it (the small-M kernels only)."""
    lib = abi.load()
    groupable = []
    for v in range(abi.variant_count("f16")):
        d = abi.describe_variant("f16", v)
        k5, k6 = d.kernel5.decode(), d.kernel6.decode()
        assert k5.startswith("pk_gemm_f16") and k6.startswith("pk_gemm_f16") and "_b5_" in k5 and "_b6_" in k6, v
        assert d.tile_rows % 32 == 0 and d.tile_columns % 32 == 0 and d.block_threads % 64 == 0, v
        small = k5.startswith("pk_gemm_f16s_")
        assert bool(d.groupable) == small, v
        # pair-code kernels read codes split into their K split's parts; all others one part
        assert d.code_parts == (d.k_split if k5.startswith("pk_gemm_f16p_") else 1), v
        if small:
            groupable.append(v)
    assert groupable == abi.small_m_variants() and groupable
    d = abi.describe_variant("f32", 0)
    assert d.kernel5.decode().startswith("pk_gemm_f32") and not d.groupable and d.code_parts == 1
    assert lib.pk_gemm_variant_describe(abi.PRECISION["f16"], abi.variant_count("f16"), ctypes.byref(d)) \
        == abi.RANGE_ERROR
    assert lib.pk_gemm_group_create(None, None, 0, None, None) == abi.INVALID_ARGUMENT
    assert lib.pk_gemm_group_destroy(None) == abi.OK
    assert lib.pk_gemm_group_set_variant(None, 0) == abi.INVALID_ARGUMENT


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


# ------------------------------------------------------ conformer conv plan


def test_gemm_flags_contract(abi):
    """pk_gemm_validate (no device) accepts every defined GEMM flag alone and
    refuses an unknown bit by name."""
    lib = abi.load()

    def desc(flags):
        d = abi.GemmDesc()
        d.struct_size = ctypes.sizeof(abi.GemmDesc)
        d.flags = flags
        d.label = b"lbl"
        d.precision = abi.PRECISION["f16"]
        d.palette_bits, d.rows, d.inner, d.columns = 5, 64, 256, 512
        d.palette_groups, d.palette_group_columns = 1, 512
        base = 0x2000000000
        d.a, d.a_bytes = base, 64 * 256 * 2
        d.packed, d.packed_bytes = base + (1 << 24), 256 * 512 // 32 * 20
        d.palette, d.palette_bytes = base + (2 << 24), 32 * 2
        d.output, d.output_bytes = base + (3 << 24), 64 * 512 * 2
        d.activation = abi.ACTIVATION["none"]
        return d

    for flags in (0, abi.GEMM_CACHED_OUTPUT):
        abi.check(lib.pk_gemm_validate(ctypes.byref(desc(flags))))
    with pytest.raises(abi.PaletteError, match="lbl has unknown flags 0x10"):
        abi.check(lib.pk_gemm_validate(ctypes.byref(desc(0x10))))


def test_conv_plan_matches_reference_shapes(abi):
    """planFusedConformerConv known answers (test/webgpu/conformer-conv-kernel-shapes.test.ts:18-58):
    batch 2 x 188 frames is 376 rows; byte lengths for fp16 and fp32."""
    for precision, elem in (("f16", 2), ("f32", 4)):
        plan = abi.plan_conformer_conv(2, 188, precision)
        assert plan.rows == 376
        assert plan.input_bytes == 376 * 2048 * elem
        assert plan.output_bytes == 376 * 1024 * elem
        assert plan.valid_lengths_bytes == 2 * 4
        assert plan.depthwise_weight_bytes == 9 * 1024 * elem
        assert plan.affine_bytes == 1024 * 4
        assert plan.algorithmic_bytes == 376 * 3072 * elem + 9 * 1024 * elem + 2 * 4096 + 8
        assert plan.kernel.startswith(b"pk_conformer_conv_" + precision.encode())
        # the grid covers every (window, frame run, channel group) once
        cpt, run = map(int, re.search(rb"_c(\d+)_f(\d+)$", plan.kernel).groups())
        per_item = -(-188 // run) * (1024 // cpt)
        assert plan.grid[0] == 2 * -(-per_item // plan.block_threads)


def test_conv_plan_rejects_non_positive_shapes(abi):
    with pytest.raises(abi.PaletteRangeError, match="batchSize must be a positive integer"):
        abi.plan_conformer_conv(0, 188)
    with pytest.raises(abi.PaletteRangeError, match="frames must be a positive integer"):
        abi.plan_conformer_conv(1, 0)
    with pytest.raises(abi.PaletteRangeError, match="multiple of 8"):
        abi.plan_conformer_conv(1, 4, channels=12)


class _Fake:
    """A device slice stand-in for the host-only checks: an address and a size."""

    def __init__(self, ptr, nbytes, dtype=np.float16):
        self.ptr, self.nbytes, self.dtype = ptr, nbytes, np.dtype(dtype)


def _conv_fakes(batch=2, frames=188, channels=1024, elem=2):
    rows = batch * frames
    dtype = np.float16 if elem == 2 else np.float32
    return dict(
        pointwise_input=_Fake(0x10000000, rows * 2 * channels * elem, dtype),
        depthwise_weights=_Fake(0x20000000, 9 * channels * elem, dtype),
        batch_norm_scale=_Fake(0x30000000, channels * 4, np.float32),
        batch_norm_shift=_Fake(0x30100000, channels * 4, np.float32),
        valid_lengths=_Fake(0x40000000, batch * 4, np.uint32),
        output=_Fake(0x50000000, rows * channels * elem, dtype),
        batch_size=batch, frames=frames, label="layer0-convolution-glu-depthwise-bn-silu")


def _validate(abi, **kw):
    desc = abi.conv_desc(**kw)
    abi.check(abi.load().pk_conv_validate(ctypes.byref(desc)))


def test_conv_validate_accepts_the_reference_descriptor(abi):
    _validate(abi, **_conv_fakes())
    _validate(abi, **_conv_fakes(elem=4))


@pytest.mark.parametrize("role,field,message", [
    ("pointwise input", "pointwise_input", "pointwise input needs 1540096 bytes; arena slice has 1540095"),
    ("output", "output", "output needs 770048 bytes; arena slice has 770047"),
    ("valid lengths", "valid_lengths", "valid lengths needs 8 bytes; arena slice has 7"),
])
def test_conv_validate_arena_capacity_messages(abi, role, field, message):
    """requireArenaCapacity (conformer-conv.ts:390-401) is a RangeError."""
    kw = _conv_fakes()
    kw[field] = _Fake(kw[field].ptr, kw[field].nbytes - 1, kw[field].dtype)
    with pytest.raises(abi.PaletteRangeError, match=re.escape(message)):
        _validate(abi, **kw)


def test_conv_validate_packed_tensor_messages(abi):
    """requirePackedTensor (conformer-conv.ts:403-432) is an Error naming dtype,
    layout, logical and storage shape and byte length."""
    kw = _conv_fakes()
    kw["depthwise_weights"] = _Fake(kw["depthwise_weights"].ptr, 9 * 1024 * 4)
    with pytest.raises(abi.PaletteError, match=re.escape(
            "depthwise weights must be float16 kernel-channel-vec4 logical [9,1024], storage [9,256,4], "
            "18432 bytes")) as err:
        _validate(abi, **kw)
    assert err.value.status == abi.INVALID_ARGUMENT
    kw = _conv_fakes()
    kw["batch_norm_shift"] = _Fake(kw["batch_norm_shift"].ptr, 2048)
    with pytest.raises(abi.PaletteError, match=re.escape(
            "folded batch norm shift must be float32 channel logical [1024], storage [1024], 4096 bytes")):
        _validate(abi, **kw)


def test_conv_validate_rejects_aliasing_and_misalignment(abi):
    kw = _conv_fakes()
    kw["output"] = _Fake(kw["pointwise_input"].ptr + 4096, kw["output"].nbytes)
    with pytest.raises(abi.PaletteError, match="must not overlap"):
        _validate(abi, **kw)
    kw = _conv_fakes()
    kw["output"] = _Fake(kw["output"].ptr + 8, kw["output"].nbytes)
    with pytest.raises(abi.PaletteError, match="aligned"):
        _validate(abi, **kw)
    kw = _conv_fakes()
    kw["batch_size"] = 0
    with pytest.raises(abi.PaletteRangeError, match="batchSize must be a positive integer"):
        _validate(abi, **kw)


def test_conv_null_handles(abi):
    lib = abi.load()
    assert lib.pk_conv_enqueue(None, 0, None) == abi.INVALID_ARGUMENT
    assert lib.pk_conv_destroy(None) == abi.OK
    assert lib.pk_conv_release(None) == abi.OK
    assert abi.conv_variant_count("f16") >= 1 and abi.conv_variant_count("f32") >= 1


# ---------------------------------------------- relative-position attention


def _attention_fakes(batch=2, frames=188, elem=2):
    rows, p = batch * frames, 2 * frames - 1
    dtype = np.float16 if elem == 2 else np.float32
    return dict(
        qkv=_Fake(0x10000000, rows * 3072 * elem, dtype),
        projected_positions=_Fake(0x20000000, p * 1024 * elem, dtype),
        bias_u=_Fake(0x30000000, 4096, np.float32),
        bias_v=_Fake(0x30100000, 4096, np.float32),
        valid_lengths=_Fake(0x40000000, batch * 4, np.uint32),
        output=_Fake(0x50000000, rows * 1024 * elem, dtype),
        batch_size=batch, frames=frames, label="layer0-relative-attention")


def _validate_attention(abi, **kw):
    desc = abi.attention_desc(**kw)
    abi.check(abi.load().pk_attention_validate(ctypes.byref(desc)))


def test_attention_validate_accepts_reference_and_long_windows(abi):
    _validate_attention(abi, **_attention_fakes())
    _validate_attention(abi, **_attention_fakes(elem=4))
    _validate_attention(abi, **_attention_fakes(batch=4, frames=750))


@pytest.mark.parametrize("batch,frames", [(0, 188), (2, 0), (1, 4097)])
def test_attention_shape_is_a_range_error(abi, batch, frames):
    """createDispatch's shape check (attention.ts:222-229)."""
    kw = _attention_fakes()
    kw["batch_size"], kw["frames"] = batch, frames
    with pytest.raises(abi.PaletteRangeError, match="Unsupported attention shape for layer0-relative-attention"):
        _validate_attention(abi, **kw)


@pytest.mark.parametrize("field,message", [
    ("qkv", "layer0-relative-attention QKV needs 2310144 bytes; arena slice has 2310143"),
    ("output", "layer0-relative-attention output needs 770048 bytes; arena slice has 770047"),
    ("valid_lengths", "layer0-relative-attention valid lengths needs 8 bytes; arena slice has 7"),
])
def test_attention_arena_capacity_messages(abi, field, message):
    kw = _attention_fakes()
    kw[field] = _Fake(kw[field].ptr, kw[field].nbytes - 1, kw[field].dtype)
    with pytest.raises(abi.PaletteRangeError, match=re.escape(message)):
        _validate_attention(abi, **kw)


def test_attention_tensor_messages(abi):
    """requireProjectedPositions / requireAttentionBias (attention.ts:323-370)."""
    kw = _attention_fakes()
    kw["projected_positions"] = _Fake(kw["projected_positions"].ptr, 100)
    with pytest.raises(abi.PaletteError, match=re.escape(
            "Projected positions must be float16 head-vector-position-vec4, logical [375,1024], "
            "storage [8,32,375,4]")):
        _validate_attention(abi, **kw)
    kw = _attention_fakes()
    kw["bias_v"] = _Fake(kw["bias_v"].ptr, 2048)
    with pytest.raises(abi.PaletteError, match=re.escape(
            "layer0-relative-attention bias V must be float32 head-by-channel logical/storage [8,128]")):
        _validate_attention(abi, **kw)
    kw = _attention_fakes()
    kw["output"] = _Fake(kw["qkv"].ptr + 1024, kw["output"].nbytes)
    with pytest.raises(abi.PaletteError, match="must not overlap"):
        _validate_attention(abi, **kw)


def test_attention_null_handles(abi):
    lib = abi.load()
    assert lib.pk_attention_enqueue(None, 0, None) == abi.INVALID_ARGUMENT
    assert lib.pk_attention_destroy(None) == abi.OK
    assert abi.attention_variant_count("f16") == 5 and abi.attention_variant_count("f32") == 2


# ---------------------------------------------------------------- LayerNorm


def _ln_fakes(rows=3008, channels=1024, elem=2):
    dtype = np.float16 if elem == 2 else np.float32
    return dict(input=_Fake(0x10000000, rows * channels * elem, dtype), gamma=_Fake(0x20000000, channels * 4),
                beta=_Fake(0x20100000, channels * 4), output=_Fake(0x30000000, rows * channels * elem, dtype),
                rows=rows, channels=channels, label="encoder.layers.0.norm_feed_forward1")


def _validate_ln(abi, **kw):
    desc = abi.layernorm_desc(**kw)
    abi.check(abi.load().pk_layernorm_validate(ctypes.byref(desc)))


def test_layernorm_contract_messages(abi):
    """layernorm.ts:165-281: shape (RangeError), arena capacity (RangeError),
    packed affine tensors (Error); in place is allowed."""
    _validate_ln(abi, **_ln_fakes())
    kw = _ln_fakes()
    kw["output"] = kw["input"]
    _validate_ln(abi, **kw)
    kw = _ln_fakes()
    kw["channels"] = 1022
    with pytest.raises(abi.PaletteRangeError, match="Invalid LayerNorm shape for encoder.layers.0.norm_feed_forward1"):
        _validate_ln(abi, **kw)
    kw = _ln_fakes()
    kw["output"] = _Fake(kw["output"].ptr, 100)
    with pytest.raises(abi.PaletteRangeError, match=re.escape(
            "encoder.layers.0.norm_feed_forward1 output needs 6160384 bytes; arena slice has 100")):
        _validate_ln(abi, **kw)
    kw = _ln_fakes()
    kw["beta"] = _Fake(kw["beta"].ptr, 2048)
    with pytest.raises(abi.PaletteError, match=re.escape(
            "encoder.layers.0.norm_feed_forward1 beta must be float32 channel logical/storage [1024], 4096 bytes")):
        _validate_ln(abi, **kw)


def test_chained_layernorm_contract(abi):
    """A chained LayerNorm (no reference counterpart): rows of at most 4 KB,
    next gamma / beta of C f32 channels, next output capacity, and the next
    output neither overlapping the output nor partly overlapping the input
    (the input itself is allowed)."""
    def chained(**over):
        kw = _ln_fakes(**{k: over.pop(k) for k in ("rows", "channels", "elem") if k in over})
        c = kw["channels"]
        kw.update(next_gamma=_Fake(0x20200000, c * 4), next_beta=_Fake(0x20300000, c * 4),
                  next_output=_Fake(0x40000000, kw["output"].nbytes, kw["output"].dtype))
        kw.update(over)
        return kw
    name = "encoder.layers.0.norm_feed_forward1"
    _validate_ln(abi, **chained())
    kw = chained()
    kw["next_output"] = kw["input"]
    _validate_ln(abi, **kw)
    _validate_ln(abi, **chained(channels=1024, elem=4))
    with pytest.raises(abi.PaletteRangeError, match=f"{name} chained LayerNorm needs rows of at most 4096 bytes"):
        _validate_ln(abi, **chained(channels=2048, elem=4))
    with pytest.raises(abi.PaletteRangeError, match=f"{name} next output needs 6160384 bytes; arena slice has 64"):
        _validate_ln(abi, **chained(next_output=_Fake(0x40000000, 64)))
    with pytest.raises(abi.PaletteError, match=re.escape(f"{name} next gamma and beta must be float32 [1024], 4096")):
        _validate_ln(abi, **chained(next_beta=_Fake(0x20300000, 2048)))
    kw = chained()
    for bad in (kw["output"].ptr + 2048, kw["input"].ptr + 2048):
        with pytest.raises(abi.PaletteError, match="next output must not overlap the output"):
            _validate_ln(abi, **chained(next_output=_Fake(bad, kw["output"].nbytes)))


# ---------------------------------------------------------------- subsampling


def test_subsampling_lengths_match_reference_kats(abi):
    """test/webgpu/subsampling-kernel-shapes.test.ts:27-50."""
    lib = abi.load()
    heights, widths = [1501], [128]
    for _ in range(3):
        heights.append(lib.pk_subsampling_output_dimension(heights[-1]))
        widths.append(lib.pk_subsampling_output_dimension(widths[-1]))
    assert heights == [1501, 751, 376, 188] and widths == [128, 64, 32, 16]
    assert [lib.pk_subsampling_valid_length(1500, s) for s in (1, 2, 3)] == [750, 375, 188]
    assert [lib.pk_subsampling_valid_length(799, s) for s in (1, 2, 3)] == [400, 200, 100]
    assert lib.pk_subsampling_valid_length(1, 3) == 1
    assert lib.pk_subsampling_output_dimension(0) == 0


def _fused_fakes(batch=3, frames=1501, elem=2):
    dtype = np.float16 if elem == 2 else np.float32
    out_rows = abi_lengths(frames, 2)
    return dict(input=_Fake(0x10000000, batch * frames * 128 * 4, np.float32),
                conv0_weights=_Fake(0x20000000, 9 * 256 * elem, dtype), conv0_bias=_Fake(0x20100000, 1024),
                depthwise_weights=_Fake(0x20200000, 9 * 256 * elem, dtype), depthwise_bias=_Fake(0x20300000, 1024),
                output=_Fake(0x40000000, batch * out_rows * 32 * 256 * elem, dtype),
                valid_lengths=_Fake(0x50000000, 4 * batch, np.uint32), batch_size=batch, input_height=frames,
                label="subsampling-fused-conv0-depthwise2-batch-0-size-3")


def abi_lengths(n, steps):
    for _ in range(steps):
        n = (n + 1) // 2
    return n


def _validate_fused(abi, **kw):
    desc = abi.subsampling_fused_desc(**kw)
    abi.check(abi.load().pk_subsampling_fused_validate(ctypes.byref(desc)))


def test_subsampling_fused_contract(abi):
    """planFusedSubsamplingConv0Depthwise2 / createDispatch
    (subsampling.ts:145-206, :334-387): the B3 plan's byte counts
    (subsampling-kernel-shapes.test.ts:83-110) and the reference messages."""
    _validate_fused(abi, **_fused_fakes())
    _validate_fused(abi, **_fused_fakes(elem=4))
    _validate_fused(abi, **_fused_fakes(batch=1, frames=6001))  # longer windows are allowed here
    kw = _fused_fakes()
    kw["output"] = _Fake(kw["output"].ptr, 3 * 376 * 32 * 256 * 2 - 2)
    with pytest.raises(abi.PaletteRangeError, match=re.escape(
            "subsampling-fused-conv0-depthwise2-batch-0-size-3 output needs 18481152 bytes; arena slice has "
            "18481150")):
        _validate_fused(abi, **kw)
    kw = _fused_fakes()
    kw["input"] = _Fake(kw["input"].ptr, 3 * 1501 * 128 * 4 - 4)
    with pytest.raises(abi.PaletteRangeError, match="input needs 2305536 bytes"):
        _validate_fused(abi, **kw)
    kw = _fused_fakes()
    kw["valid_length_batch_offset"] = 3
    with pytest.raises(abi.PaletteRangeError, match="valid lengths needs 24 bytes; arena slice has 12"):
        _validate_fused(abi, **kw)
    kw = _fused_fakes()
    kw["input_width"] = 80
    with pytest.raises(abi.PaletteRangeError, match=re.escape("Fused conv0+depthwise2 requires fixed")):
        _validate_fused(abi, **kw)
    kw = _fused_fakes()
    kw["batch_size"] = 0
    with pytest.raises(abi.PaletteRangeError, match="batchSize must be a positive integer"):
        _validate_fused(abi, **kw)
    kw = _fused_fakes()
    kw["conv0_weights"] = _Fake(kw["conv0_weights"].ptr, 9 * 256 * 4, np.float16)
    with pytest.raises(abi.PaletteError, match=re.escape(
            "conv0 weights must be float16 kh-kw-output-channel-vec4 logical [3,3,256], storage [3,3,64,4], "
            "4608 bytes")):
        _validate_fused(abi, **kw)
    kw = _fused_fakes()
    kw["depthwise_bias"] = _Fake(kw["depthwise_bias"].ptr, 512)
    with pytest.raises(abi.PaletteError, match=re.escape(
            "depthwise2 bias must be float32 output-channel logical [256], storage [256], 1024 bytes")):
        _validate_fused(abi, **kw)


def _dw_fakes(batch=3, elem=2):
    dtype = np.float16 if elem == 2 else np.float32
    return dict(input=_Fake(0x10000000, batch * 376 * 32 * 256 * elem, dtype),
                weights=_Fake(0x20000000, 9 * 256 * elem, dtype), bias=_Fake(0x20100000, 1024),
                output=_Fake(0x40000000, batch * 188 * 16 * 256 * elem, dtype),
                valid_lengths=_Fake(0x50000000, 4 * batch, np.uint32), batch_size=batch, input_height=376,
                input_width=32, channels=256, steps=3, label="subsampling-depthwise5")


def _validate_dw(abi, **kw):
    desc = abi.subsampling_depthwise_desc(**kw)
    abi.check(abi.load().pk_subsampling_depthwise_validate(ctypes.byref(desc)))


def test_subsampling_depthwise_contract(abi):
    """planDepthwise / createDispatch (subsampling.ts:495-531, :795-853) and
    the depthwise5 plan of subsampling-kernel-shapes.test.ts:52-81."""
    _validate_dw(abi, **_dw_fakes())
    _validate_dw(abi, **_dw_fakes(batch=1, elem=4))
    kw = _dw_fakes()
    kw["channels"] = 258
    with pytest.raises(abi.PaletteRangeError, match="Subsampling channels must be divisible by four"):
        _validate_dw(abi, **kw)
    kw = _dw_fakes()
    kw["steps"] = 0
    with pytest.raises(abi.PaletteRangeError,
                       match="subsampling-depthwise5 valid-length subsampling steps must be a positive integer"):
        _validate_dw(abi, **kw)
    kw = _dw_fakes()
    kw["output"] = _Fake(kw["output"].ptr, 100)
    with pytest.raises(abi.PaletteRangeError, match=re.escape(
            "subsampling-depthwise5 output needs 4620288 bytes; arena slice has 100")):
        _validate_dw(abi, **kw)
    kw = _dw_fakes()
    kw["weights"] = _Fake(kw["weights"].ptr, 100)
    with pytest.raises(abi.PaletteError, match=re.escape(
            "subsampling-depthwise5 weights must be float16 kh-kw-channel-vec4 logical [3,3,256], "
            "storage [3,3,64,4], 4608 bytes")):
        _validate_dw(abi, **kw)


def test_subsampling_mask_contract(abi):
    """SubsamplingTimeMaskKernel.createDispatch (subsampling.ts:698-748)."""
    def validate(**kw):
        base = dict(values=_Fake(0x10000000, 3 * 188 * 16 * 256 * 2), valid_lengths=_Fake(0x50000000, 12),
                    batch_size=3, height=188, width=16, channels=256, steps=3,
                    label="subsampling-pointwise6-mask")
        base.update(kw)
        desc = abi.subsampling_mask_desc(**base)
        abi.check(abi.load().pk_subsampling_mask_validate(ctypes.byref(desc)))
    validate()
    with pytest.raises(abi.PaletteRangeError, match="Subsampling mask channels must be divisible by four"):
        validate(channels=6)
    with pytest.raises(abi.PaletteRangeError, match="height must be a positive integer"):
        validate(height=0)
    with pytest.raises(abi.PaletteRangeError, match="values needs 4620288 bytes; arena slice has 64"):
        validate(values=_Fake(0x10000000, 64))
    with pytest.raises(abi.PaletteRangeError, match="valid lengths needs 16 bytes"):
        validate(valid_length_batch_offset=1)


def test_subsampling_null_handles(abi):
    lib = abi.load()
    assert lib.pk_subsampling_enqueue(None, 0, None) == abi.INVALID_ARGUMENT
    assert lib.pk_subsampling_plan(None, 0, None) == abi.INVALID_ARGUMENT
    assert lib.pk_subsampling_destroy(None) == abi.OK
    assert lib.pk_subsampling_release(None) == abi.OK
    assert lib.pk_subsampling_fused_validate(None) == abi.INVALID_ARGUMENT


# ---------------------------------------------------------------- TDT decoder


def _tdt_fakes(batch=16, frames=188, max_tokens=256, elem=2):
    """Nominal addresses and sizes of a decoder descriptor; `elem` is the
    profile's weight and encoder-row element (2: f16, 4: f32)."""
    at = [0x6000000000]

    def take(nbytes):
        addr = at[0]
        at[0] += (nbytes + 0xFFFF) // 0x10000 * 0x10000
        return (addr, nbytes)
    weights = {"embedding": take(1025 * 640 * elem), "lstm_weight_l0": take(1280 * 2560 * elem),
               "lstm_weight_l1": take(1280 * 2560 * elem), "lstm_bias_l0": take(2560 * 4),
               "lstm_bias_l1": take(2560 * 4), "projector_weight": take(640 * 640 * elem),
               "projector_bias": take(640 * 4), "head_weight": take(640 * 1032 * elem), "head_bias": take(1032 * 4)}
    return dict(weights=weights, encoder_projected=take(batch * frames * 640 * elem), encoded_lengths=take(4 * batch),
                decode_starts=take(4 * batch), decode_ends=take(4 * batch), flush_finals=take(4 * batch),
                state=take(batch * 4 * 640 * 4), predictor_scratch=take(batch * 5 * 640 * 4),
                tokens=take(batch * max_tokens * 4), token_frames=take(batch * max_tokens * 4),
                token_durations=take(batch * max_tokens * 4), metadata=take(8 * batch), batch_size=batch,
                frames=frames, max_tokens=max_tokens)


def _validate_tdt(abi, **kw):
    desc = abi.tdt_desc(**kw)
    abi.check(abi.load().pk_tdt_validate(ctypes.byref(desc)))


def test_tdt_plan_and_contract(abi):
    """planTdtDecoderExecution (tdt-decoder.ts:39-52) and validateDescriptor /
    requireDecoderWeights (:378-547) with the reference's messages."""
    plan = abi.plan_tdt_execution(16)
    assert plan.workgroup_count == 16 and plan.predictor_scratch_bytes == 16 * 5 * 640 * 4
    with pytest.raises(abi.PaletteRangeError, match="batchSize must be a positive integer"):
        abi.plan_tdt_execution(0)
    _validate_tdt(abi, **_tdt_fakes())
    for field, message in (("batch_size", "Invalid TDT decoder batchSize"), ("frames", "Invalid TDT decoder frames"),
                           ("max_tokens", "Invalid TDT decoder maxTokens")):
        kw = _tdt_fakes()
        kw[field] = 0
        with pytest.raises(abi.PaletteRangeError, match=message):
            _validate_tdt(abi, **kw)
    kw = _tdt_fakes()
    kw["predictor_scratch"] = (kw["predictor_scratch"][0], 100)
    with pytest.raises(abi.PaletteRangeError, match="predictorScratch is too small for TDT decoding"):
        _validate_tdt(abi, **kw)
    kw = _tdt_fakes()
    kw["weights"]["head_weight"] = (kw["weights"]["head_weight"][0], 640 * 1030 * 2)
    with pytest.raises(abi.PaletteError, match=re.escape("Unexpected decoder tensor k-by-output-row-major-vec4 [640,1032]")):
        _validate_tdt(abi, **kw)
    kw = _tdt_fakes()
    kw["weights"]["lstm_bias_l1"] = (kw["weights"]["lstm_bias_l1"][0], 2560 * 2)
    with pytest.raises(abi.PaletteError, match=re.escape("Unexpected decoder tensor ifgo-gates [2560]")):
        _validate_tdt(abi, **kw)
    lib = abi.load()
    assert lib.pk_gemm_prepare_rows(None, None, 0) == abi.INVALID_ARGUMENT
    assert lib.pk_tdt_enqueue(None, 0, None) == abi.INVALID_ARGUMENT
    assert lib.pk_tdt_destroy(None) == abi.OK


def test_tdt_f32_profile_contract(abi):
    """The f32 profile (tdt-decoder.ts:196-218, :378-405): f32 weights and
    encoder rows are twice the f16 sizes; an f16-sized tensor in an f32
    descriptor, or the reverse, is the reference's "Unexpected decoder
    tensor" error, and a short f32 encoder slice its range error."""
    _validate_tdt(abi, precision="f32", **_tdt_fakes(elem=4))
    kw = _tdt_fakes(elem=2)
    kw["encoder_projected"] = _tdt_fakes(elem=4)["encoder_projected"]  # slices first, then the f16-sized weights
    with pytest.raises(abi.PaletteError, match=re.escape("Unexpected decoder tensor token-by-channel-row-major [1025,640]")):
        _validate_tdt(abi, precision="f32", **kw)
    with pytest.raises(abi.PaletteError, match="Unexpected decoder tensor"):
        _validate_tdt(abi, **_tdt_fakes(elem=4))
    kw = _tdt_fakes(elem=4)
    kw["encoder_projected"] = (kw["encoder_projected"][0], 16 * 188 * 640 * 2)
    with pytest.raises(abi.PaletteRangeError, match="encoderProjected is too small for TDT decoding"):
        _validate_tdt(abi, precision="f32", **kw)
    desc = abi.tdt_desc(**_tdt_fakes())
    desc.precision = 7
    with pytest.raises(abi.PaletteError, match="TDT decoder precision must be f16 or f32"):
        abi.check(abi.load().pk_tdt_validate(ctypes.byref(desc)))


def test_tdt_status_decoding(abi):
    """Overflow and team sync timeout are separate bits of a window's
    status word, counted apart (a timed-out window must be decoded again;
    an overflowed one is complete up to max_tokens)."""
    assert (abi.TDT_OVERFLOW, abi.TDT_SYNC_TIMEOUT) == (1, 2)
    got = abi.decode_tdt_status(np.array([0, 1, 2, 3, 0, 2, 8], np.uint32))
    assert got == {"overflow_windows": 2, "sync_timeout_windows": 3, "unknown_status_windows": 1}
    assert abi.decode_tdt_status([]) == {"overflow_windows": 0, "sync_timeout_windows": 0,
                                         "unknown_status_windows": 0}
    header = open(os.path.join(ROOT, "include", "pk_tdt.h")).read()
    assert re.search(r"#define PK_TDT_OVERFLOW 1u", header) and re.search(r"#define PK_TDT_SYNC_TIMEOUT 2u", header)


# ---------------------------------------------------------------- encoder stack


def _encoder_fakes(layers=2, batch=16, frames=188, elem=2):
    """Nominal, aligned device addresses for every tensor of the stack
    (activations of `elem` bytes)."""
    at = [0x1000000000]

    def take(nbytes=1 << 20):
        addr = at[0]
        at[0] += (nbytes + 0xFFFF) // 0x10000 * 0x10000
        return addr

    stack = []
    for _ in range(layers):
        layer = {"norm_gamma": [take() for _ in range(5)], "norm_beta": [take() for _ in range(5)]}
        for name in ("ff1_linear1", "ff1_linear2", "qkv", "o_proj", "pointwise1", "pointwise2", "ff2_linear1",
                     "ff2_linear2"):
            layer[name] = (take(4 << 20), take())
        for name in ("projected_positions", "bias_u", "bias_v", "depthwise", "bn_scale", "bn_shift"):
            layer[name] = take()
        stack.append(layer)
    rows = batch * frames
    return dict(layers=stack, valid_lengths=take(), input=take(rows * 1024 * elem), output=take(rows * 1024 * elem),
                batch_size=batch, frames=frames)


def _front_fakes(kw, batch=16, feature_frames=1501):
    at = [0x3000000000]

    def take(nbytes=1 << 20):
        addr = at[0]
        at[0] += (nbytes + 0xFFFF) // 0x10000 * 0x10000
        return addr
    front = {name: take() for name in ("conv0_weights", "conv0_bias", "depthwise2_weights", "depthwise2_bias",
                                       "pointwise3_bias", "depthwise5_weights", "depthwise5_bias",
                                       "pointwise6_bias", "linear_bias")}
    for name in ("pointwise3", "pointwise6", "linear"):
        front[name] = (take(4 << 20), take())
    kw.update(subsampling=front, feature_frames=feature_frames, feature_lengths=take(),
              input=take(batch * 128 * feature_frames * 4), projector=(take(4 << 20), take()),
              projector_bias=take(), projected_channels=640, projected_output=take(batch * 188 * 640 * 2))
    return kw


def _validate_encoder(abi, **kw):
    desc = abi.encoder_desc(**kw)
    abi.check(abi.load().pk_encoder_validate(ctypes.byref(desc)))


@pytest.mark.parametrize("fused_glu", [False, True])
def test_encoder_validate_accepts_the_reference_stack(abi, fused_glu):
    """24 layers x 16 windows x 188 frames (encoder.ts:62, :68), and T=750."""
    _validate_encoder(abi, fused_glu=fused_glu, **_encoder_fakes(layers=24))
    _validate_encoder(abi, fused_glu=fused_glu, **_encoder_fakes(layers=1, batch=4, frames=750))


def test_encoder_validate_names_the_failing_op(abi):
    kw = _encoder_fakes()
    kw["layers"][1]["qkv"] = (kw["layers"][1]["qkv"][0], 0)
    with pytest.raises(abi.PaletteError, match=re.escape("encoder.layers.1-self-attention-qkv")):
        _validate_encoder(abi, **kw)
    kw = _encoder_fakes()
    kw["layers"][0]["depthwise"] += 2  # misaligned vec4 tensor
    with pytest.raises(abi.PaletteError, match=re.escape("encoder.layers.0-convolution-glu-depthwise-bn-silu")):
        _validate_encoder(abi, **kw)
    kw = _encoder_fakes(frames=4097)
    with pytest.raises(abi.PaletteError, match="encoder.layers.0-relative-attention"):
        _validate_encoder(abi, **kw)


def test_encoder_validate_stack_fields(abi):
    with pytest.raises(abi.PaletteRangeError, match="Unsupported encoder shape"):
        _validate_encoder(abi, **_encoder_fakes(layers=0))
    kw = _encoder_fakes()
    kw["output"] = kw["input"] + 4096
    with pytest.raises(abi.PaletteError, match="must not overlap its input"):
        _validate_encoder(abi, **kw)
    kw = _encoder_fakes()
    kw["input"] += 8
    with pytest.raises(abi.PaletteError, match="16-byte aligned"):
        _validate_encoder(abi, **kw)
    desc = abi.encoder_desc(**_encoder_fakes())
    desc.precision = 7
    with pytest.raises(abi.PaletteError, match="unsupported precision 7"):
        abi.check(abi.load().pk_encoder_validate(ctypes.byref(desc)))
    desc = abi.encoder_desc(**_encoder_fakes())
    desc.flags = 0x20
    with pytest.raises(abi.PaletteError, match="unknown flags"):
        abi.check(abi.load().pk_encoder_validate(ctypes.byref(desc)))
    desc = abi.encoder_desc(**_encoder_fakes())
    desc.flags = abi.ENCODER_FUSED_GLU | abi.ENCODER_SEPARATE_GLU
    with pytest.raises(abi.PaletteError, match="exclude each other"):
        abi.check(abi.load().pk_encoder_validate(ctypes.byref(desc)))
    desc.flags = abi.ENCODER_FUSED_GLU  # the default, still accepted
    abi.check(abi.load().pk_encoder_validate(ctypes.byref(desc)))
    _validate_encoder(abi, prefix_same_plan=True, **_encoder_fakes())  # prefixes keep the capacity's kernels
    # the fp32 profile: accepted, without the f16-only fusions
    _validate_encoder(abi, precision="f32", **_encoder_fakes(layers=24, elem=4))
    for flags in (abi.ENCODER_FUSED_GLU, abi.ENCODER_FUSED_NORMS):
        desc = abi.encoder_desc(precision="f32", **_encoder_fakes(elem=4))
        desc.flags = flags
        with pytest.raises(abi.PaletteError, match="need f16"):
            abi.check(abi.load().pk_encoder_validate(ctypes.byref(desc)))


def test_encoder_validate_front_end_and_projector(abi):
    """The whole graph of ParakeetEncoderGraph.encode (encoder.ts:1690-1706):
    subsampling front end, 24 layers, projector."""
    _validate_encoder(abi, **_front_fakes(_encoder_fakes(layers=24)))
    kw = _front_fakes(_encoder_fakes(layers=1))
    kw["feature_frames"] = 1500  # 750 -> 375 -> 188 as well
    _validate_encoder(abi, **kw)
    kw["feature_frames"] = 1499  # -> 188 as well ((1499+1)/2 = 750)
    _validate_encoder(abi, **kw)
    kw["feature_frames"] = 1490  # 745 -> 373 -> 187
    with pytest.raises(abi.PaletteRangeError, match="188 encoder frames do not follow from 1490 feature frames"):
        _validate_encoder(abi, **kw)
    kw = _front_fakes(_encoder_fakes(layers=1))
    kw["feature_lengths"] = None
    with pytest.raises(abi.PaletteError, match="needs per-window feature lengths"):
        _validate_encoder(abi, **kw)
    kw = _front_fakes(_encoder_fakes(layers=1))
    kw["subsampling"]["pointwise6"] = (kw["subsampling"]["pointwise6"][0], 0)
    with pytest.raises(abi.PaletteError, match=re.escape("encoder.subsampling-pointwise6")):
        _validate_encoder(abi, **kw)
    kw = _front_fakes(_encoder_fakes(layers=1))
    kw["subsampling"]["conv0_bias"] += 4
    with pytest.raises(abi.PaletteError, match=re.escape("encoder.subsampling-fused-conv0-depthwise2 conv0 bias")):
        _validate_encoder(abi, **kw)
    kw = _front_fakes(_encoder_fakes(layers=1))
    kw["projected_output"] = kw["output"] + 1024
    with pytest.raises(abi.PaletteError, match="projected output must not overlap"):
        _validate_encoder(abi, **kw)
    kw = _front_fakes(_encoder_fakes(layers=1))
    kw["projected_channels"] = 636
    with pytest.raises(abi.PaletteError, match="encoder-projector"):
        _validate_encoder(abi, **kw)


def test_encoder_null_handles(abi):
    lib = abi.load()
    assert lib.pk_encoder_enqueue(None, 0, None, 0) == abi.INVALID_ARGUMENT
    assert lib.pk_encoder_info(None, None, None) == abi.INVALID_ARGUMENT
    assert lib.pk_encoder_destroy(None) == abi.OK
    assert lib.pk_encoder_validate(None) == abi.INVALID_ARGUMENT


def test_tdt_team_size_arguments(abi):
    """The team-size calls (no reference counterpart) reject a null op and a
    null output before touching a device."""
    lib = abi.load()
    out = ctypes.c_uint32()
    with pytest.raises(abi.PaletteError, match="TDT decoder op is null"):
        abi.check(lib.pk_tdt_set_team_size(None, 16))
    with pytest.raises(abi.PaletteError, match="TDT decoder op or output is null"):
        abi.check(lib.pk_tdt_team_size(None, ctypes.byref(out)))

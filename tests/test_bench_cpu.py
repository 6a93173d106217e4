"""CPU tests of bench.py's host logic: the encoder's launch order and the
split of a rocprofv3 kernel trace per launch kind (no GPU, no profiler: the
trace is synthetic)."""
import csv
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from parakeet_wgsl_amd.palette_abi import ENCODER_DISPATCHES  # noqa: E402

KERNEL = {
    "layernorm_kernel": "void pk::(anonymous namespace)::layernorm_kernel<_Float16, 8, 2048, false>(pk::LayerNormArgs)",
    "attention": "void pk::(anonymous namespace)::rel_attention_f16_shared_kernel<4, false>(pk::AttentionArgs)",
    "conformer_conv_kernel": "void pk::(anonymous namespace)::conformer_conv_kernel<_Float16, 2, 8, true>(pk::ConvArgs)",
    "subsampling_": "void pk::(anonymous namespace)::subsampling_depthwise_kernel<_Float16>(pk::SubsamplingArgs)",
    "gemm_f16": "void pk::(anonymous namespace)::gemm_f16k_kernel<5, 2, 2, 3, 2, false, true, 5, false>(pk::GemmArgs)",
}
FUSED = "void pk::(anonymous namespace)::subsampling_fused_kernel<_Float16, 4>(pk::SubsamplingArgs)"
LOOP = "void pk::(anonymous namespace)::gemm_f16k_kernel<5, 4, 1, 6, 2, false, true, 2, false>(pk::GemmArgs)"
PREP = "void pk::(anonymous namespace)::operand_order_kernel<5, 1>(pk::OrderArgs)"


def test_launch_sequence_counts():
    """344 launches per pass at 24 layers: 6 front-end, 15 slots per layer
    less the 23 chained LN ff1 slots, the projector."""
    seq = bench.launch_sequence(24)
    assert len(seq) == 6 + 24 * len(ENCODER_DISPATCHES) - 23 + 1 == 344
    assert seq[0] == "subsampling-fused-conv0-depthwise2" and seq[-1] == "projector"
    assert seq.count("norm_feed_forward1") == 1
    assert len(bench.launch_sequence(24, chained=False)) == 367
    fused = bench.launch_sequence(2, fused_norms=bench.FUSED_NORMS)
    assert not any(n in fused for n in bench.FUSED_NORMS)


def kernel_for(kind):
    if kind == "subsampling-fused-conv0-depthwise2":
        return FUSED
    return KERNEL[bench.kernel_family(kind)]


def write_trace(path, layers, warmup, steps, duration_us, rows=None):
    """A kernel trace of `warmup + PROFILE_PASSES + steps` passes; each
    launch of `kind` lasts duration_us(kind, pass kind) ("profiled" for the
    passes after the warm-up, "stamped" for every TIMING_STRIDE-th timed
    one, "graph" for the rest), then one op preparation and the roofline
    loop."""
    seq = bench.launch_sequence(layers)
    t = 1_000_000
    out = []

    def add(name, us, grid=65536):
        nonlocal t
        out.append({"Kernel_Name": name, "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000),
                    "Grid_Size_X": grid})
        t += int(us * 1000) + 500

    for p in range(warmup + bench.PROFILE_PASSES + steps):
        timed = p - warmup - bench.PROFILE_PASSES
        pass_kind = ("profiled" if warmup <= p < warmup + bench.PROFILE_PASSES else
                     "stamped" if timed >= 0 and timed % bench.TIMING_STRIDE == 0 else "graph")
        for kind in seq:
            add(kernel_for(kind), duration_us(kind, pass_kind))
    add(PREP, 20.0)
    warm, n = bench.ROOFLINE_LOOP
    for i in range(warm + n):
        add(LOOP, 40.0 if i < warm else 30.0)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(out[0]))
        w.writeheader()
        # the profiler writes rows out of start order; the splitter sorts them
        for r in reversed(out):
            w.writerow(r)


def test_split_trace_kinds_and_loop(tmp_path, capsys):
    """Per-kind averages over the profiled passes, the timed stamped steps
    and the graph passes come out as written, and the roofline loop is the
    last ROOFLINE_LOOP[1] GEMM launches, not the op preparation before
    them."""
    path = tmp_path / "trace.csv"
    extra = {"profiled": 2.0, "stamped": 1.0, "graph": 0.0}

    def duration(kind, pass_kind):
        return (10.0 if kind.startswith("norm_") else 20.0) + extra[pass_kind]

    write_trace(path, 2, 3, 10, duration)
    bench.split_trace(str(path), 3, 10, layers=2)
    out = capsys.readouterr().out
    passes = 3 + bench.PROFILE_PASSES + 10
    row = next(line for line in out.splitlines() if line.startswith("| norm_self_att |"))
    cells = [c.strip() for c in row.strip("|").split("|")]
    assert cells[1] == str(2 * passes) and cells[2:5] == ["12.00", "11.00", "10.00"]
    row = next(line for line in out.splitlines() if line.startswith("| feed-forward1-linear1 |"))
    cells = [c.strip() for c in row.strip("|").split("|")]
    assert cells[2:5] == ["22.00", "21.00", "20.00"]
    loop = next(line for line in out.splitlines() if line.startswith("roofline loop"))
    assert "avg 30.00 us" in loop and "operand_order" not in loop and "of 55 " in loop


def test_split_trace_rejects_wrong_pass_count(tmp_path):
    path = tmp_path / "trace.csv"
    write_trace(path, 1, 1, 5, lambda kind, pass_kind: 5.0)
    with pytest.raises(SystemExit, match="passes in the trace"):
        bench.split_trace(str(path), 1, 4, layers=1)


def test_split_trace_checks_kernel_names(tmp_path):
    """A launch whose kernel does not belong to its kind stops the split."""
    path = tmp_path / "trace.csv"
    write_trace(path, 1, 1, 2, lambda kind, pass_kind: 5.0)
    with open(path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    seq = bench.launch_sequence(1)
    i = seq.index("relative-attention")
    rows[i]["Kernel_Name"] = KERNEL["gemm_f16"]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    with pytest.raises(SystemExit, match="relative-attention ran"):
        bench.split_trace(str(path), 1, 2, layers=1)


def write_counters(path, names_values, counter):
    fields = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        for d, (name, value) in enumerate(names_values, 1):
            # two rows per dispatch: the splitter sums them
            for half in (value / 2, value / 2):
                w.writerow({"Dispatch_Id": d, "Kernel_Name": name, "Counter_Name": counter, "Counter_Value": half})


def test_split_counters_scales_by_the_calibration_copy(tmp_path, capsys):
    """HBM bytes per kind = FETCH x (copy KiB / copy FETCH) + WRITE x (copy
    KiB / copy WRITE), from the last pass; the first copy dispatch is
    skipped."""
    layers, warmup, steps = 1, 1, 2
    seq = bench.launch_sequence(layers)
    passes = []
    total = warmup + bench.PROFILE_PASSES + steps
    for p in range(total):
        passes += [(kernel_for(kind), 100.0 * (p + 1)) for kind in seq]
    write_counters(tmp_path / "f.csv", passes, "FETCH_SIZE")
    write_counters(tmp_path / "w.csv", [(n, v / 2) for n, v in passes], "WRITE_SIZE")
    neg = "void at::native::vectorized_elementwise_kernel<neg_kernel>"
    write_counters(tmp_path / "cf.csv", [(neg, 1.0), (neg, bench.COPY_KIB / 2), (neg, bench.COPY_KIB / 2)], "FETCH_SIZE")
    write_counters(tmp_path / "cw.csv", [(neg, bench.COPY_KIB)] * 3, "WRITE_SIZE")
    bench.split_counters(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), str(tmp_path / "cf.csv"),
                         str(tmp_path / "cw.csv"), warmup, steps, layers=layers)
    out = capsys.readouterr().out
    assert "FETCH_SIZE x 2.000, WRITE_SIZE x 1.000" in out
    row = next(line for line in out.splitlines() if line.startswith("| feed-forward1-linear1 |"))
    cells = [c.strip() for c in row.strip("|").split("|")]
    # last pass: FETCH 100 t KiB x 2 + WRITE 50 t KiB x 1 = 250 t KiB
    fetch, write = 100 * total, 50 * total
    assert cells[1] == "1" and cells[2] == f"{fetch:,}" and cells[3] == f"{write:,}"
    assert cells[4] == f"{250 * total * 1024 / 1e6:.1f} MB"
    entries = json.loads(out.split("traffic.json entries:", 1)[1])
    assert entries["encoder-feed-forward1-linear1"]["hbm_bytes_per_launch"] == 250 * total * 1024
    assert "encoder-relative-attention" not in entries


def test_roofline_slots_pick_both_ff_modules():
    """The stamped slots of the timed region are the roofline kind's
    launches in both FF modules of every layer, and nothing else."""
    from parakeet_wgsl_amd.palette_abi import ENCODER_DISPATCHES
    layers = 3
    launches = len(bench.FRONT_DISPATCHES) + len(ENCODER_DISPATCHES) * layers + 1
    dispatches = {k: {"launches_per_pass": layers} for k in ENCODER_DISPATCHES}
    slots = bench.roofline_slots(layers, 1, "feed-forward1-linear2-residual", dispatches, launches)
    kinds = list(bench.FRONT_DISPATCHES) + list(ENCODER_DISPATCHES) * layers + ["projector"]
    assert len(slots) == 2 * layers
    assert {kinds[i] for i in slots} == {"feed-forward1-linear2-residual", "feed-forward2-linear2-residual"}
    # a fused LayerNorm's slot launches nothing and is never stamped
    dispatches["norm_self_att"]["launches_per_pass"] = 0
    assert bench.roofline_slots(layers, 1, "norm_self_att", dispatches, launches) == []
    with pytest.raises(SystemExit, match="dispatch slots"):
        bench.roofline_slots(layers, 1, "projector", dispatches, launches + 1)


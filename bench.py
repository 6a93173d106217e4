"""Benchmark of the MI355X palette-weight GEMM path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Default workload (one step = one encoder pass): the FastConformer encoder in
fp16 over 16 windows of 15 s - the 8x subsampling front end over a 128-bin x
1501-frame fbank, 24 layers at 188 frames x 1024 channels whose eight palette
GEMMs per layer carry every projection, and the 1024->640 projector - with
random-init palette weights at the reference package's widths. Inputs are
seeded synthetic data resident in HBM before timing starts. One JSON line is
printed: encoder audio-sec/sec, the roofline of the dominant palette GEMM
(the average of its launches in the timed region's stamped passes, an event
pair around each on the stream it runs on; the same op launched 50 times
back to back after the timed region beside it), the CPU oracle's throughput on a bounded sample of the same workload at
one thread and at all threads, and, under "ff_block", the palette-GEMM
TFLOP/s of the Conformer feed-forward block (8 windows x 188 frames: H =
SiLU(X W1), 5-bit 1024->4096, then Y = X + 0.5 (H W2), 5-bit 4096->1024).

Other workloads (for profiling; same JSON shape):
  ff-block          the feed-forward block above as the step, TFLOP/s
  single-gemm-fp32  X[256x1024] f32 x 6-bit W 1024->4096 + bias
  small-m           5-bit 1024->4096 f16 GEMM at --rows M (HBM-bound regime)
  layer-gemms       the six palette GEMM shapes of an encoder layer at --rows M
                    (3008 = 16 windows), one launch each per step: FF expand +
                    SiLU, FF contract + 0.5 residual, QKV (3 palette groups),
                    the 6-bit output projection + residual, PW1 + GLU, PW2 +
                    residual; with --variant V every shape that V can run is
                    forced onto it (tile sweeps)
  weight-stream     every palette GEMM of the 24 encoder layers (192 distinct
                    weights, 365 MB packed) at --rows M: one grouped small-M
                    launch per step (value, GB/s), and the same GEMMs as 192
                    single launches replayed from a HIP graph
  conv-module       Conformer convolution module, fp16, 16 windows x 188 x 1024:
                    P = X PW1 (6-bit 1024->2048), Z = SiLU(BN(DW9(GLU(P)))),
                    Y = X + Z PW2 (6-bit 1024->1024); TFLOP/s counts the two
                    GEMMs, the step time includes the fused conv tail
  conv-module-fused the same module with the GLU moved into PW1's epilogue
                    (PW1 writes [rows, 1024] GLU; the tail reads it)
  rel-pos-mha       relative-position MHA block, fp16, 4 windows x --frames (188
                    or 750) x 1024: QKV = X Wqkv (6-bit, 3 palette groups),
                    P = table Wpos (6-bit rel-pos linear over 2T-1 sinusoid
                    rows), C = attention(QKV, P, u, v, valid), Y = X + C Wo;
                    TFLOP/s counts the three GEMMs and the attention products
  encoder           the FastConformer encoder, fp16, 16 windows of 15 s: the
                    8x subsampling front end over a 128-bin x 1501-frame
                    fbank, 24 layers at 188 frames x 1024, the 1024->640
                    projector; random-init palette weights at the reference
                    package's widths; one step = one pass (367 launches,
                    replayed from a HIP graph); value in audio-sec/sec
  transcribe        the encoder pass followed by the greedy TDT decoder over
                    its projector output (LSTM predictor 640, joint to 1024
                    tokens + blank and 5 durations), random-init weights; one
                    step = encoder pass + decode; value in audio-sec/sec
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS = {"f16": 2500.0, "f32": 157.3}  # MI355X dense MFMA
PEAK_HBM_GBS = 8000.0
METRIC = "palette-GEMM TFLOP/s & % roofline; encoder audio-sec/sec at 1 MI355X"
TIMING_STRIDE = 5  # one step in five carries the per-kernel start/end stamps
# Encoder workloads: eager passes with every launch stamped, run after the
# warm-up and before the timed region (the per-dispatch table and the
# dominant launch kind). Stamping all 344 launches of a pass makes it about
# a quarter slower than a graph replay, so inside the timed region the
# stamped steps stamp the dominant kind's launches only.
PROFILE_PASSES = 2
# roofline.traffic is looked up, not measured in the run it is reported with
TRAFFIC_SOURCE = ("looked up in profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of the same "
                  "command, scaled by the counters' reading of a plain copy")


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", default="encoder",
                   choices=["ff-block", "single-gemm-fp32", "small-m", "weight-stream", "conv-module",
                            "conv-module-fused", "rel-pos-mha", "layer-gemms", "encoder", "transcribe"])
    p.add_argument("--frames", type=int, default=188, help="T for --workload rel-pos-mha")
    p.add_argument("--windows", type=int, default=16,
                   help="encoder / transcribe: windows the graph holds (40 is the reference's largest batch)")
    p.add_argument("--active", type=int, default=0,
                   help="encoder / transcribe: active windows of each pass (a prefix; 0 = all)")
    p.add_argument("--rows", type=int, default=64, help="M for --workload small-m and weight-stream")
    p.add_argument("--cpu-sample-rows", type=int, default=0,
                   help="rows of the CPU-oracle sample (0 = workload default)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-dense", action="store_true", help="skip the dense vendor GEMM reference")
    p.add_argument("--no-ff-block", action="store_true", help="encoder workloads: skip the FF block's extra line")
    p.add_argument("--precision", choices=["f16", "f32"], default="f16",
                   help="encoder workload: f32 runs the reference's fp32 profile (f32 activations, palettes, "
                        "positions and depthwise weights)")
    p.add_argument("--separate-glu", action="store_true",
                   help="encoder workloads: the convolution forms the GLU from PW1's values and gates, as the "
                        "reference does (PK_ENCODER_SEPARATE_GLU; default: PW1's epilogue writes the GLU)")
    p.add_argument("--prefix-same-plan", action="store_true",
                   help="encoder workloads with --active below --windows: the prefix keeps the capacity's kernels "
                        "(PK_ENCODER_PREFIX_SAME_PLAN; default: the plans of a graph built for the active windows)")
    p.add_argument("--unchained-norms", action="store_true",
                   help="encoder workloads: launch every LayerNorm on its own (default: each layer's last "
                        "LayerNorm also writes the next layer's first)")
    p.add_argument("--fused-norms", action="store_true",
                   help="encoder workloads: run the four LayerNorms that feed a GEMM inside those GEMMs "
                        "(PK_GEMM_ROW_NORM; default: separate launches, as the reference does)")
    p.add_argument("--graph", action="store_true",
                   help="replay the unstamped steps from a HIP graph (measured slower than eager launches for "
                        "two-launch steps)")
    p.add_argument("--dense-probe", default="", help=argparse.SUPPRESS)
    p.add_argument("--variant", type=int, default=-1, help="force a tile variant (sweeps)")
    p.add_argument("--split-trace", default="",
                   help="CPU only: per launch kind of a rocprofv3 kernel trace (CSV) of the encoder bench run "
                        "with the given --steps / --warmup")
    p.add_argument("--roofline-kind", default="",
                   help="encoder workloads: describe this launch kind in `roofline` instead of the one with the "
                        "most time per pass (to profile the same back-to-back loop as another run's line)")
    p.add_argument("--split-counters", default="",
                   help="CPU only: FETCH,WRITE,COPY_FETCH,COPY_WRITE - four rocprofv3 --pmc counter CSVs (the "
                        "encoder bench run with the given --steps / --warmup, FETCH_SIZE then WRITE_SIZE, and the "
                        "copy of COPY_COMMAND for each counter): HBM bytes per launch kind of the last pass")
    p.add_argument("--bench-json", default="",
                   help="with --split-counters: a bench line of the same workload, for the algorithmic bytes")
    return p.parse_args()


class Kernel:
    """One fused palette GEMM launch of the step and its bookkeeping."""

    def __init__(self, name, op, flops, nbytes, precision, shape=None):
        self.name = name
        self.op = op
        self.flops = flops
        self.nbytes = nbytes
        self.precision = precision
        self.shape = shape  # (M, K, N) of a GEMM launch
        self.times_ms = []

    def summary(self):
        avg = float(np.mean(self.times_ms))
        plan = self.op.plan()
        return {
            "kernel": plan.kernel.decode(),
            "grid": list(plan.grid),
            "avg_us": avg * 1e3,
            "tflops": self.flops / (avg * 1e-3) / 1e12,
            "gbs": self.nbytes / (avg * 1e-3) / 1e9,
            "flops": self.flops,
            "algorithmic_bytes": self.nbytes,
        }


def build_ff_block(abi, ctx, keep):
    import parakeet_wgsl_amd.workloads as wl
    ff = wl.feed_forward_block(0)
    m = ff.x.shape[0]
    x = keep(ctx.array(ff.x))
    hidden = keep(ctx.empty((m, 4096), np.float16))
    y = keep(ctx.empty((m, 1024), np.float16))
    op1 = abi.GemmOp(ctx, a=x, packed=keep(ctx.array(ff.w1.packed)), palette=keep(ctx.array(ff.w1.palette)),
                     output=hidden, bits=5, rows=m, inner=1024, columns=4096, activation="silu",
                     label="ff-expand")
    op2 = abi.GemmOp(ctx, a=hidden, packed=keep(ctx.array(ff.w2.packed)), palette=keep(ctx.array(ff.w2.palette)),
                     output=y, bits=5, rows=m, inner=4096, columns=1024, residual=x, residual_scale=0.5,
                     label="ff-contract")
    e = ff.expand_case()
    c = ff.contract_case(np.zeros((m, 4096), np.float16))
    kernels = [Kernel("ff-expand", op1, e.flops, e.algorithmic_bytes(), "f16", (m, 1024, 4096)),
               Kernel("ff-contract", op2, c.flops, c.algorithmic_bytes(), "f16", (m, 4096, 1024))]
    config = {"workload": "conformer-ff-block-fp16", "windows": 8, "frames": 188, "rows": m,
              "d_model": 1024, "hidden": 4096, "palette_bits": 5, "epilogues": ["silu", "0.5*residual"]}
    return kernels, config, ff


def build_single_gemm(abi, ctx, keep):
    import parakeet_wgsl_amd.workloads as wl
    case = wl.single_gemm_fp32(0)
    out = keep(ctx.empty((case.rows, 4096), np.float32))
    op = abi.GemmOp(ctx, a=keep(ctx.array(case.a)), packed=keep(ctx.array(case.weight.packed)),
                    palette=keep(ctx.array(case.weight.palette)), output=out, bits=6, rows=case.rows,
                    inner=1024, columns=4096, bias=keep(ctx.array(case.bias)), label="single-gemm-fp32")
    config = {"workload": "single-palette-gemm-fp32", "rows": case.rows, "inner": 1024, "columns": 4096,
              "palette_bits": 6, "epilogues": ["bias"]}
    return [Kernel("single-gemm-fp32", op, case.flops, case.algorithmic_bytes(), "f32", (case.rows, 1024, 4096))], \
        config, case


class RotatingOp:
    """Launches a list of same-shape GEMM ops in turn, one per enqueue, so
    consecutive steps read different weights."""

    def __init__(self, ops):
        self.ops = ops
        self.next = 0

    def enqueue(self, *args):
        op = self.ops[self.next]
        self.next = (self.next + 1) % len(self.ops)
        op.enqueue(*args)

    def plan(self, *args):
        return self.ops[0].plan(*args)

    def set_variant(self, variant):
        for op in self.ops:
            op.set_variant(variant)

    def release(self):
        for op in self.ops:
            op.release()


SMALL_M_WEIGHTS = 128  # distinct 2.6 MB weights: 336 MB, past the 256 MB MALL


def build_small_m(abi, ctx, keep, rows):
    """The small-M GEMM over SMALL_M_WEIGHTS distinct weights launched in
    turn: no step finds its weight in the memory-side cache, as a model's
    weights streamed once per token would not."""
    import parakeet_wgsl_amd.workloads as wl
    case = wl.gemm_case(0, rows, 1024, 4096, 5)
    rng = np.random.default_rng(1)
    a = keep(ctx.array(case.a))
    out = keep(ctx.empty((rows, 4096), np.float16))
    ops = []
    for i in range(SMALL_M_WEIGHTS):
        packed = case.weight.packed if i == 0 else wl.random_packed_words(rng, 5, 1024, 4096)
        ops.append(abi.GemmOp(ctx, a=a, packed=keep(ctx.array(packed)),
                              palette=keep(ctx.array(case.weight.palette)), output=out, bits=5, rows=rows,
                              inner=1024, columns=4096, label=f"small-m-{rows}-{i}"))
    config = {"workload": "small-m-palette-gemm-fp16", "rows": rows, "inner": 1024, "columns": 4096,
              "palette_bits": 5, "distinct_weights": SMALL_M_WEIGHTS,
              "rotation": f"each step launches the next of {SMALL_M_WEIGHTS} distinct weights "
                          f"({SMALL_M_WEIGHTS * case.weight.packed.nbytes / 1e6:.0f} MB of packed codes in turn; "
                          "activations and output shared)"}
    return [Kernel(f"small-m-{rows}", RotatingOp(ops), case.flops, case.algorithmic_bytes(), "f16",
                   (rows, 1024, 4096))], config, case


# The palette GEMMs of one encoder layer: name, K, N, bits, palette groups,
# activation, residual scale, GLU epilogue.
LAYER_GEMM_SHAPES = (
    ("ff-expand", 1024, 4096, 5, 1, "silu", None, False),
    ("ff-contract", 4096, 1024, 5, 1, "none", 0.5, False),
    ("qkv", 1024, 3072, 5, 3, "none", None, False),
    ("output-projection", 1024, 1024, 6, 1, "none", 1.0, False),
    ("pointwise1-glu", 1024, 2048, 5, 1, "none", None, True),
    ("pointwise2", 1024, 1024, 5, 1, "none", 1.0, False),
)


def build_layer_gemms(abi, ctx, keep, rows):
    """One launch of each palette GEMM shape of an encoder layer at `rows`
    rows, seeded random operands (the FF expand's case is the CPU leg's)."""
    import parakeet_wgsl_amd.workloads as wl
    kernels, first = [], None
    for seed, (name, inner, columns, bits, groups, activation, scale, glu) in enumerate(LAYER_GEMM_SHAPES):
        case = wl.gemm_case(seed, rows, inner, columns, bits, groups=groups, activation=activation,
                            residual_scale=scale)
        first = first or case
        width = columns // 2 if glu else columns
        out = keep(ctx.empty((rows, width), np.float16))
        op = abi.GemmOp(ctx, a=keep(ctx.array(case.a)), packed=keep(ctx.array(case.weight.packed)),
                        palette=keep(ctx.array(case.weight.palette)), output=out, bits=bits, rows=rows,
                        inner=inner, columns=columns, activation=activation,
                        residual=keep(ctx.array(case.residual)) if scale is not None else None,
                        residual_scale=scale, glu=glu, label=f"layer-{name}")
        nbytes = case.algorithmic_bytes() - (rows * (columns - width) * 2)
        kernels.append(Kernel(name, op, case.flops, nbytes, "f16", (rows, inner, columns)))
    config = {"workload": "encoder-layer-gemms-fp16", "rows": rows,
              "shapes": {n: [k, c] for n, k, c, *_ in LAYER_GEMM_SHAPES}}
    return kernels, config, first


def build_conv_module(abi, ctx, keep, fused_glu=False):
    import parakeet_wgsl_amd.workloads as wl
    mod = wl.conv_module(0)
    m, d = mod.x.shape
    conv = mod.conv
    x = keep(ctx.array(mod.x))
    p = keep(ctx.empty((m, d if fused_glu else 2 * d), np.float16))
    z = keep(ctx.empty((m, d), np.float16))
    y = keep(ctx.empty((m, d), np.float16))
    pw1 = abi.GemmOp(ctx, a=x, packed=keep(ctx.array(mod.pw1.packed)), palette=keep(ctx.array(mod.pw1.palette)),
                     output=p, bits=6, rows=m, inner=d, columns=2 * d, label="conv-pointwise1", glu=fused_glu)
    tail = abi.ConformerConvOp(
        ctx, pointwise_input=p, depthwise_weights=keep(ctx.array(conv.weights)),
        batch_norm_scale=keep(ctx.array(conv.scale)), batch_norm_shift=keep(ctx.array(conv.shift)),
        valid_lengths=keep(ctx.array(conv.valid)), output=z, batch_size=conv.batch, frames=conv.frames,
        label="conv-glu-depthwise-bn-silu", input_glu=fused_glu)
    pw2 = abi.GemmOp(ctx, a=z, packed=keep(ctx.array(mod.pw2.packed)), palette=keep(ctx.array(mod.pw2.palette)),
                     output=y, bits=6, rows=m, inner=d, columns=d, residual=x, residual_scale=1.0,
                     label="conv-pointwise2-residual")
    c1 = mod.pw1_case()
    c2 = mod.pw2_case(np.zeros((m, d), np.float16))
    pw1_bytes = c1.algorithmic_bytes() - (m * d * 2 if fused_glu else 0)  # GLU output is half as wide
    tail_bytes = conv.algorithmic_bytes() - (m * d * 2 if fused_glu else 0)
    kernels = [Kernel("conv-pointwise1", pw1, c1.flops, pw1_bytes, "f16"),
               Kernel("conv-tail", tail, 0, tail_bytes, "f16"),
               Kernel("conv-pointwise2", pw2, c2.flops, c2.algorithmic_bytes(), "f16")]
    config = {"workload": "conformer-conv-module-fp16" + ("-fused-glu" if fused_glu else ""),
              "windows": conv.batch, "frames": conv.frames, "rows": m,
              "d_model": d, "palette_bits": 6, "depthwise_kernel": 9,
              "epilogues": (["pw1+glu", "depthwise9", "batchnorm", "silu", "residual"] if fused_glu
                            else ["glu", "depthwise9", "batchnorm", "silu", "residual"])}
    return kernels, config, mod


def build_mha(abi, ctx, keep, frames):
    import parakeet_wgsl_amd.workloads as wl
    mod = wl.mha_module(0, frames=frames)
    m, p = mod.x.shape[0], mod.table.shape[0]
    x = keep(ctx.array(mod.x))
    qkv = keep(ctx.empty((m, 3072), np.float16))
    pos = keep(ctx.empty((p, 1024), np.float16))
    c = keep(ctx.empty((m, 1024), np.float16))
    y = keep(ctx.empty((m, 1024), np.float16))
    op_qkv = abi.GemmOp(ctx, a=x, packed=keep(ctx.array(mod.wqkv.packed)), palette=keep(ctx.array(mod.wqkv.palette)),
                        output=qkv, bits=6, rows=m, inner=1024, columns=3072, label="attention-qkv")
    op_pos = abi.GemmOp(ctx, a=keep(ctx.array(mod.table)), packed=keep(ctx.array(mod.wpos.packed)),
                        palette=keep(ctx.array(mod.wpos.palette)), output=pos, bits=6, rows=p, inner=1024,
                        columns=1024, label="attention-relative-positions")
    op_att = abi.RelativeAttentionOp(ctx, qkv=qkv, projected_positions=pos, bias_u=keep(ctx.array(mod.bias_u)),
                                     bias_v=keep(ctx.array(mod.bias_v)), valid_lengths=keep(ctx.array(mod.valid)),
                                     output=c, batch_size=mod.batch, frames=frames, positions_row_major=True,
                                     label="relative-attention")
    op_out = abi.GemmOp(ctx, a=c, packed=keep(ctx.array(mod.wo.packed)), palette=keep(ctx.array(mod.wo.palette)),
                        output=y, bits=6, rows=m, inner=1024, columns=1024, residual=x, residual_scale=1.0,
                        label="attention-output-residual")

    def gemm_case(a_rows, w, name, residual=False):
        case = wl.GemmCase(name, np.zeros((a_rows, 1024), np.float16), w)
        extra = a_rows * 1024 * 2 if residual else 0
        return case.flops, case.algorithmic_bytes() + extra
    f_qkv, b_qkv = gemm_case(m, mod.wqkv, "qkv")
    f_pos, b_pos = gemm_case(p, mod.wpos, "pos")
    f_out, b_out = gemm_case(m, mod.wo, "out", residual=True)
    kernels = [Kernel("attention-qkv", op_qkv, f_qkv, b_qkv, "f16"),
               Kernel("attention-relative-positions", op_pos, f_pos, b_pos, "f16"),
               Kernel("relative-attention", op_att, mod.attention_flops(), op_att.plan().algorithmic_bytes, "f16"),
               Kernel("attention-output-residual", op_out, f_out, b_out, "f16")]
    config = {"workload": "relative-position-mha-fp16", "windows": mod.batch, "frames": frames, "rows": m,
              "d_model": 1024, "heads": 8, "head_size": 128, "palette_bits": 6, "position_rows": p,
              "valid_lengths": [int(v) for v in mod.valid]}
    return kernels, config, mod


def host_info():
    """The CPU the baseline runs on: usable threads, logical CPUs, model name."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"nproc": usable, "logical_cpus": os.cpu_count(), "model": model}


def all_threads():
    """Threads of the all-core CPU leg: the usable CPUs, at most 16 (the
    share of one GPU's host)."""
    return max(1, min(host_info()["nproc"], 16))


def cpu_baseline(workload, data, sample_rows, budget_s=10.0, threads=None):
    """The oracle (reference semantics restated in C) on a bounded sample:
    row batches of the same workload until about `budget_s` seconds of wall
    time have passed (or `sample_rows` rows, when given)."""
    from oracle import pko
    threads = threads or all_threads()
    batch = 32
    if workload == "ff-block":
        total_rows, per_row_flops = data.x.shape[0], 2 * 1024 * 4096 * 2

        def run(lo, hi):
            x = data.x[lo:hi]
            h = pko.gemm(x, data.w1.packed, 5, data.w1.palette, 4096, activation="silu", mode="f16-chain",
                         threads=threads)
            pko.gemm(h, data.w2.packed, 5, data.w2.palette, 1024, residual=x, residual_scale=0.5,
                     mode="f16-chain", threads=threads)
        what = "rows of the FF block (W1 + SiLU, W2 + 0.5 residual), f16-accumulator chain (reference fp16 semantics)"
    elif workload == "single-gemm-fp32":
        total_rows, per_row_flops = data.rows, 2 * 1024 * 4096

        def run(lo, hi):
            pko.gemm(data.a[lo:hi], data.weight.packed, 6, data.weight.palette, 4096, bias=data.bias,
                     mode="f32-chain", threads=threads)
        what = "rows, f32 fma chain (reference fp32 semantics)"
    elif workload == "rel-pos-mha":
        # whole windows; the rel-pos linear once, as the step does
        import parakeet_wgsl_amd.workloads as wl
        frames = data.frames
        total_rows, batch = data.x.shape[0], frames
        per_row_flops = (data.gemm_flops() + data.attention_flops()) / total_rows
        pos = pko.gemm(data.table, data.wpos.packed, 6, data.wpos.palette, 1024, mode="f16-chain", threads=threads)
        packed = wl.pack_projected_positions(pos)

        def run(lo, hi):
            x = data.x[lo:hi]
            w = lo // frames
            qkv = pko.gemm(x, data.wqkv.packed, 6, data.wqkv.palette, 3072, mode="f16-chain", threads=threads)
            c = pko.relative_attention(qkv, packed, data.bias_u, data.bias_v, data.valid[w:w + 1], batch=1,
                                       frames=frames)
            pko.gemm(c, data.wo.packed, 6, data.wo.palette, 1024, residual=x, residual_scale=1.0, mode="f16-chain",
                     threads=threads)
        what = (f"rows (whole {frames}-frame windows) of the MHA block: QKV GEMM, relative attention (f32, one "
                "thread), output GEMM + residual; the rel-pos linear once beforehand (reference fp16 semantics)")
    elif workload in ("conv-module", "conv-module-fused"):
        # whole windows: the depthwise convolution spans frames of one window
        frames, conv = data.conv.frames, data.conv
        total_rows, per_row_flops, batch = data.x.shape[0], 2 * 1024 * 2048 + 2 * 1024 * 1024, frames

        def run(lo, hi):
            x = data.x[lo:hi]
            w = lo // frames
            p = pko.gemm(x, data.pw1.packed, 6, data.pw1.palette, 2048, mode="f16-chain", threads=threads)
            zz = pko.conformer_conv(p, conv.weights, conv.scale, conv.shift, conv.valid[w:w + 1], batch=1,
                                    frames=frames)
            pko.gemm(zz, data.pw2.packed, 6, data.pw2.palette, 1024, residual=x, residual_scale=1.0,
                     mode="f16-chain", threads=threads)
        what = ("rows (whole 188-frame windows) of the conv module: PW1, GLU/DW9/BN/SiLU tail, PW2 + residual; "
                "f16-accumulator GEMM chain and f32 tail (reference fp16 semantics)")
    else:
        total_rows, per_row_flops = data.rows, 2 * 1024 * 4096

        def run(lo, hi):
            pko.gemm(data.a[lo:hi], data.weight.packed, 5, data.weight.palette, 4096, mode="f16-chain",
                     threads=threads)
        what = "rows, f16-accumulator chain"
    limit = min(sample_rows, total_rows) if sample_rows else total_rows
    done = 0
    t0 = time.perf_counter()
    while done < limit:
        hi = min(done + batch, limit)
        run(done, hi)
        done = hi
        if not sample_rows and time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    return {"value": done * per_row_flops / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{done} of {total_rows} {what}", "seconds": dt}


WINDOW_SECONDS = 15.0  # audio per encoder window: 1500 fbank frames at 100/s, 8x subsampled to 188


# The LayerNorms that run inside the GEMM after them with --fused-norms.
FUSED_NORMS = ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2")

FRONT_DISPATCHES = ("subsampling-fused-conv0-depthwise2", "subsampling-pointwise3", "subsampling-depthwise5",
                    "subsampling-pointwise6", "subsampling-pointwise6-mask", "subsampling-flatten-project")

# The layer GEMMs as the encoder creates them (dispatch kind -> weight key,
# K, N, palette groups, activation, residual scale): the roofline's
# back-to-back loop rebuilds the dominant kind's op at the pass's shape.
LAYER_GEMMS = {
    "feed-forward1-linear1": ("ff1_linear1", 1024, 4096, 1, "silu", None),
    "feed-forward1-linear2-residual": ("ff1_linear2", 4096, 1024, 1, "none", 0.5),
    "self-attention-qkv": ("qkv", 1024, 3072, 3, "none", None),
    "self-attention-output-residual": ("o_proj", 1024, 1024, 1, "none", 1.0),
    "convolution-pointwise2-residual": ("pointwise2", 1024, 1024, 1, "none", 1.0),
}
ROOFLINE_LOOP = (5, 50)  # warm-up and timed launches of the back-to-back loop


def launch_sequence(layers, chained=True, fused_norms=()):
    """The dispatch kinds of one encoder pass in launch order: the front
    end, every layer's launched slots (a chained LN ff1 of a later layer or
    a fused LayerNorm launches nothing) and the projector."""
    from parakeet_wgsl_amd.palette_abi import ENCODER_DISPATCHES
    seq = list(FRONT_DISPATCHES)
    for layer in range(layers):
        for name in ENCODER_DISPATCHES:
            if chained and layer > 0 and name == "norm_feed_forward1":
                continue
            if name in fused_norms:
                continue
            seq.append(name)
    seq.append("projector")
    return seq


def roofline_slots(layers, projectors, name, dispatches, launches):
    """Dispatch slots of an encoder pass (front end, 15 per layer, the
    projector) whose launch kind is `name`'s, the two FF modules' launches of
    one shape counting as one kind; slots of kinds that launch nothing
    (a LayerNorm inside the next GEMM) are left out."""
    from parakeet_wgsl_amd.palette_abi import ENCODER_DISPATCHES
    slot_kinds = list(FRONT_DISPATCHES) + list(ENCODER_DISPATCHES) * layers + ["projector"] * projectors
    if len(slot_kinds) != launches:
        raise SystemExit(f"{len(slot_kinds)} dispatch slots, the encoder reports {launches}")

    def kind(k):
        return k.replace("feed-forward2-", "feed-forward1-")
    return [i for i, k in enumerate(slot_kinds) if kind(k) == kind(name) and k in dispatches
            and dispatches[k].get("launches_per_pass", 1) > 0]


def kernel_family(kind):
    """Substring the kernel name of a launch of `kind` carries."""
    if kind.startswith("norm_"):
        return "layernorm_kernel"
    if kind == "relative-attention":
        return "attention"
    if kind == "convolution-glu-depthwise-bn-silu":
        return "conformer_conv_kernel"
    if kind in ("subsampling-fused-conv0-depthwise2", "subsampling-depthwise5", "subsampling-pointwise6-mask"):
        return "subsampling_"
    return "gemm_f16"


def split_trace(path, warmup, steps, layers=24):
    """Per launch kind of the encoder bench, from a rocprofv3 kernel trace
    (CSV) of `bench.py --no-cpu --no-dense --no-ff-block --steps S --warmup
    W`: passes start at the fused subsampling kernel; each pass's launches
    are mapped to kinds in launch order (every kernel name checked against
    its kind), the passes split into the profiled passes before the timed
    region (every launch stamped), the timed region's stamped steps (every
    TIMING_STRIDE-th, eager, the roofline kind's launches stamped) and graph
    replays (warm-up and the other timed steps), and the launches after the
    last pass that run the dominant kernel form the roofline's back-to-back
    loop. Prints a markdown table."""
    import csv
    with open(path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    seq = launch_sequence(layers)
    starts = [i for i, r in enumerate(rows) if "subsampling_fused_kernel" in r["Kernel_Name"]]
    if len(starts) != warmup + PROFILE_PASSES + steps:
        raise SystemExit(f"{len(starts)} passes in the trace, expected {warmup + PROFILE_PASSES + steps}")
    per = {"graph": {}, "stamped": {}, "profiled": {}}
    sums = {"graph": [], "stamped": [], "profiled": []}
    for p, i in enumerate(starts):
        seg = rows[i:i + len(seq)]
        timed = p - warmup - PROFILE_PASSES
        kind = ("profiled" if warmup <= p < warmup + PROFILE_PASSES else
                "stamped" if timed >= 0 and timed % TIMING_STRIDE == 0 else "graph")
        total = 0.0
        for name, r in zip(seq, seg):
            if kernel_family(name) not in r["Kernel_Name"]:
                raise SystemExit(f"pass {p}: {name} ran {r['Kernel_Name']}")
            us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            per[kind].setdefault(name, []).append(us)
            total += us
        sums[kind].append(total / 1e3)
    tail = rows[starts[-1] + len(seq):]
    print("| launch kind | launches | profiled passes us | timed stamped steps us | graph passes us | grid |")
    print("|---|---:|---:|---:|---:|---:|")
    grids = {}
    for name, r in zip(seq, rows[starts[-1]:starts[-1] + len(seq)]):
        grids.setdefault(name, r["Grid_Size_X"])
    for name in dict.fromkeys(seq):
        pr, st, gr = (per[k].get(name, []) for k in ("profiled", "stamped", "graph"))
        print(f"| {name} | {len(pr) + len(st) + len(gr)} | {np.mean(pr):.2f} | {np.mean(st):.2f} | "
              f"{np.mean(gr):.2f} | {grids[name]} |")
    print()
    print(f"kernel time per pass: profiled {np.mean(sums['profiled']):.3f} ms, timed stamped "
          f"{np.mean(sums['stamped']):.3f} ms, graph {np.mean(sums['graph']):.3f} ms")
    # the roofline loop: the GEMM launches after the last pass (its op's
    # weight preparation runs before them)
    loop_warm, loop_n = ROOFLINE_LOOP
    gemms = [r for r in tail if "gemm_f16" in r["Kernel_Name"] or "gemm_f32" in r["Kernel_Name"]]
    if len(gemms) >= loop_warm + loop_n:
        loop = gemms[len(gemms) - loop_n:]
        names = {r["Kernel_Name"] for r in loop}
        us = np.array([(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in loop])
        span = (int(loop[-1]["End_Timestamp"]) - int(loop[0]["Start_Timestamp"])) / 1e3 / loop_n
        print(f"roofline loop: the last {loop_n} of {len(gemms)} back-to-back launches of {sorted(names)} "
              f"(grid {loop[-1]['Grid_Size_X']}): avg {us.mean():.2f} us (min {us.min():.2f}, max {us.max():.2f}); "
              f"first start to last end over {loop_n}: {span:.2f} us")


# The calibration copy for the HBM counters: 256 MiB read and 256 MiB
# written per torch.neg dispatch (profiled with one counter per run).
COPY_COMMAND = ("import torch; a=torch.ones(128<<20,dtype=torch.float16,device='cuda'); b=torch.empty_like(a); "
                "[torch.neg(a,out=b) for _ in range(4)]; torch.cuda.synchronize(); print('copy done')")
COPY_KIB = 256 * 1024


def read_counters(path):
    """(dispatch id, kernel name, counter value summed over the rows of the
    dispatch) in dispatch order, from a rocprofv3 --pmc CSV."""
    import csv
    per, names = {}, {}
    with open(path) as f:
        for r in csv.DictReader(f):
            d = int(r["Dispatch_Id"])
            per[d] = per.get(d, 0.0) + float(r["Counter_Value"])
            names[d] = r["Kernel_Name"]
    return [(d, names[d], per[d]) for d in sorted(per)]


def copy_factor(path):
    """True KiB of the calibration copy over what the counter reads for it
    (the torch.neg dispatches after the first)."""
    values = [v for _, name, v in read_counters(path) if "neg" in name]
    if len(values) < 2:
        raise SystemExit(f"{path}: no calibration copy dispatches")
    return COPY_KIB / float(np.mean(values[1:]))


def split_counters(fetch_path, write_path, copy_fetch, copy_write, warmup, steps, bench_json="", layers=24):
    """HBM bytes per launch kind of the encoder bench's last pass, from
    rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs (CSV, KiB per dispatch)
    of `bench.py --no-cpu --no-dense --no-ff-block --steps S --warmup W`,
    each scaled by what the same counter reads for the calibration copy
    (COPY_COMMAND). The pass's launches are mapped to kinds in launch order
    (every kernel name checked against its kind), layer kinds averaged over
    the layers. Prints a markdown table and the traffic.json entries of the
    GEMM kinds."""
    seq = launch_sequence(layers)
    factors = {"fetch": copy_factor(copy_fetch), "write": copy_factor(copy_write)}
    kib = {}
    for counter, path in (("fetch", fetch_path), ("write", write_path)):
        rows = read_counters(path)
        starts = [i for i, (_, name, _) in enumerate(rows) if "subsampling_fused_kernel" in name]
        if len(starts) != warmup + PROFILE_PASSES + steps:
            raise SystemExit(f"{path}: {len(starts)} passes, expected {warmup + PROFILE_PASSES + steps}")
        last = rows[starts[-1]:starts[-1] + len(seq)]
        per = {}
        for kind, (d, name, value) in zip(seq, last):
            if kernel_family(kind) not in name:
                raise SystemExit(f"{path}: dispatch {d} of {kind} ran {name}")
            per.setdefault(kind, []).append(value)
        kib[counter] = {kind: float(np.mean(v)) for kind, v in per.items()}
    algorithmic = {}
    if bench_json:
        with open(bench_json) as f:
            line = json.loads(f.read().strip().splitlines()[-1])
        algorithmic = {k: v["algorithmic_bytes"] for k, v in line["dispatches"].items()}
    print(f"scale: FETCH_SIZE x {factors['fetch']:.3f}, WRITE_SIZE x {factors['write']:.3f} "
          f"(the calibration copy: {COPY_KIB} KiB each way)")
    print()
    print("| launch kind | launches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes | algorithmic | ratio |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    entries = {}
    for kind in dict.fromkeys(seq):
        f, w = kib["fetch"][kind], kib["write"][kind]
        hbm = (f * factors["fetch"] + w * factors["write"]) * 1024
        alg = algorithmic.get(kind)
        ratio = f"{hbm / alg:.2f}" if alg else ""
        alg_text = f"{alg / 1e6:.1f} MB" if alg else ""
        print(f"| {kind} | {seq.count(kind)} | {f:,.0f} | {w:,.0f} | {hbm / 1e6:.1f} MB | {alg_text} | {ratio} |")
        if kernel_family(kind) == "gemm_f16":
            entries[f"encoder-{kind}"] = {"fetch_kib": round(f), "write_kib": round(w),
                                          "fetch_factor": round(factors["fetch"], 3),
                                          "write_factor": round(factors["write"], 3),
                                          "hbm_bytes_per_launch": hbm, "algorithmic_bytes": alg}
    print()
    print("traffic.json entries:", json.dumps(entries))


def roofline_loop(ctx, abi, kind, layer0, a_rows, rows, stream):
    """Average duration of `kind`'s GEMM (rebuilt from LAYER_GEMMS with layer
    0's weights at the pass's shape: `rows` active rows of `a_rows`) over
    ROOFLINE_LOOP back-to-back launches on `stream`, timed by one pair of
    events around the loop: the condition of the graph replay, where every
    launch follows the last with no gap."""
    key, inner, columns, groups, activation, scale = LAYER_GEMMS[kind]
    packed, palette = layer0[key]
    dtype = a_rows.dtype
    a = a_rows if inner == a_rows.shape[1] else ctx.empty((rows, inner), dtype)
    out = ctx.empty((rows, columns), dtype)
    residual = a_rows if scale is not None else None
    op = abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=out, bits=5 if key != "o_proj" else 6,
                    rows=rows, inner=inner, columns=columns, activation=activation, residual=residual,
                    residual_scale=scale, label=f"roofline-loop-{kind}")
    try:
        warm, n = ROOFLINE_LOOP
        for _ in range(warm):
            op.enqueue(0, stream)
        e0, e1 = ctx.event(), ctx.event()
        e0.record(stream)
        for _ in range(n):
            op.enqueue(0, stream)
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_ms(e1) / n * 1e3
    finally:
        op.release()
        if a is not a_rows:
            a.free()
        out.free()


def gemm_cost(rows, inner, columns, bits=5, groups=1, residual=False, bias=False, elem=2):
    """2MKN and compulsory bytes: packed codes, LUT, A, output (+ residual,
    bias), activations and LUT of `elem` bytes."""
    nbytes = inner * columns * bits // 8 + groups * (1 << bits) * elem + rows * inner * elem + rows * columns * elem
    return 2 * rows * inner * columns, nbytes + (rows * columns * elem if residual else 0) + (4 * columns if bias else 0)


def encoder_dispatch_costs(abi, wl, stack, fused_glu=False):
    """(flops, algorithmic bytes) per dispatch kind: the front end's six, one
    layer's fifteen (over all windows) and the projector. LayerNorm reads and
    writes the rows once; the attention and the convolutions count what
    their launches must move. Element bytes follow the stack's precision."""
    rows, frames, batch = stack.x.shape[0], stack.frames, stack.batch
    e = stack.x.dtype.itemsize
    act = rows * 1024 * e
    ln = (0, 2 * act + 2 * 4096)

    def gemm(name, residual=False):
        bits, k, n, groups = wl.ENCODER_MATRICES[name]
        return gemm_cost(rows, k, n, bits, groups, residual, elem=e)
    live = np.minimum(stack.valid.astype(np.int64), frames)
    attention = (int((live * live).sum()) * 8 * 128 * 2 * 3,
                 rows * 3072 * e + (2 * frames - 1) * 1024 * e + 2 * 4096 + 4 * batch + act)
    conv = (0, rows * (1024 if fused_glu else 2048) * e + act + 9 * 1024 * e + 8 * 1024 + 4 * batch)
    pointwise1 = gemm("pointwise1")
    if fused_glu:  # the GLU output is half as wide
        pointwise1 = (pointwise1[0], pointwise1[1] - rows * 1024 * e)
    layer = [ln, gemm("ff1_linear1"), gemm("ff1_linear2", True), ln, gemm("qkv"), attention,
             gemm("o_proj", True), ln, pointwise1, conv, gemm("pointwise2", True), ln,
             gemm("ff2_linear1"), gemm("ff2_linear2", True), ln]
    assert len(layer) == len(abi.ENCODER_DISPATCHES)
    front = []
    if stack.subsampling is not None:
        f = stack.feature_frames
        h1, h2 = wl.subsampled_length(f, 1), wl.subsampled_length(f, 2)
        stage2, stage3 = batch * h2 * 32 * 256 * e, batch * frames * 16 * 256 * e
        kernel = 9 * 256 * e + 1024
        front = [(2 * 9 * 256 * batch * (h1 * 64 + h2 * 32), batch * 128 * f * 4 + stage2 + 2 * kernel + 4 * batch),
                 gemm_cost(batch * h2 * 32, 256, 256, bias=True, elem=e),
                 (2 * 9 * 256 * batch * frames * 16, stage2 + stage3 + kernel + 4 * batch),
                 gemm_cost(batch * frames * 16, 256, 256, bias=True, elem=e),
                 (0, stage3 + 4 * batch),
                 gemm_cost(rows, 4096, 1024, bias=True, elem=e)]
    projector = [gemm_cost(rows, 1024, stack.projector_bias.size, bias=True, elem=e)] \
        if stack.projector is not None else []
    return front, layer, projector


def encoder_cpu_baseline(stack, budget_s=20.0, decoder=None):
    """The oracle (reference fp16 semantics) on window 0 at all threads (the
    front end, then layer after layer for about `budget_s` seconds) and at
    one thread (one layer, the pass extrapolated with the all-thread leg's
    front-end-to-layer ratio); with `decoder` = (weights, projected window
    [188, 640] f16, length), also the oracle's greedy decode of that window
    (one thread in both legs)."""
    from oracle import pko
    main, x0, ratio, decode_s = encoder_cpu_leg(stack, all_threads(), budget_s, decoder)
    t0 = time.perf_counter()
    pko.encoder_layer(x0, stack.layers[0], stack.valid[:1], batch=1, frames=stack.frames, threads=1,
                      dtype=stack.x.dtype)
    layer_s = time.perf_counter() - t0
    pass_s = layer_s * (len(stack.layers) + ratio) + decode_s
    main["single_thread"] = {
        "value": WINDOW_SECONDS / pass_s, "unit": "audio-sec/sec", "cores": 1, "kind": "port",
        "sample": ("one 15-s window: layer 0 timed at one thread, the pass extrapolated to every layer and the "
                   f"front end (front end = {ratio:.2f} layers, from the all-thread leg)"
                   + ("; plus the decode time of the all-thread leg" if decoder is not None else "")),
        "seconds": layer_s}
    main["host"] = host_info()
    return main


def encoder_cpu_leg(stack, threads, budget_s, decoder):
    from oracle import pko
    dtype = stack.x.dtype  # f16: the reference's fp16 chain; f32: its fp32 profile
    t0 = time.perf_counter()
    if stack.subsampling is not None:
        x = pko.encoder_front_end(stack.features[:1], stack.subsampling, stack.feature_lengths[:1], threads=threads,
                                  dtype=dtype)
    else:
        x = stack.x[:stack.frames]
    front_s = time.perf_counter() - t0
    x0 = x
    done = 0
    while done < len(stack.layers) and (done == 0 or time.perf_counter() - t0 < budget_s):
        x = pko.encoder_layer(x, stack.layers[done], stack.valid[:1], batch=1, frames=stack.frames,
                              threads=threads, dtype=dtype)
        done += 1
    layer_s = (time.perf_counter() - t0 - front_s) / done
    # one window's pass: the front end plus every layer at the measured rate
    pass_s = front_s + layer_s * len(stack.layers)
    sample = (f"one 15-s window: the front end and {done} of {len(stack.layers)} layers timed, the pass "
              "extrapolated to every layer " + ("(f16-accumulator GEMM chain, f32 conv, LayerNorm and attention: "
                                                "reference fp16 semantics)" if dtype == np.float16 else
                                                "(f32 storage and arithmetic: the reference's fp32 profile)"))
    decode_s = 0.0
    if decoder is not None:
        weights, projected, length = decoder
        t1 = time.perf_counter()
        pko.tdt_decode(weights, projected[None], [length], max_tokens=1024, flush=[1])
        decode_s = time.perf_counter() - t1
        pass_s += decode_s
        sample += "; then the greedy TDT decode of that window (f16 LSTM and head chains, one thread)"
    leg = {"value": WINDOW_SECONDS / pass_s, "unit": "audio-sec/sec", "cores": threads, "kind": "port",
           "sample": sample, "seconds": time.perf_counter() - t0}
    return leg, x0, front_s / layer_s, decode_s


class ActivePrefix:
    """The first `active` windows of an encoder stack, for the per-pass costs
    of an active-prefix pass."""

    def __init__(self, stack, active):
        self.frames, self.batch = stack.frames, active
        self.x = stack.x[:active * stack.frames]
        self.valid = stack.valid[:active]
        self.layers, self.subsampling = stack.layers, stack.subsampling
        self.feature_frames = stack.feature_frames
        self.projector, self.projector_bias = stack.projector, stack.projector_bias
        self._stack = stack

    def gemm_flops(self):
        return self._stack.gemm_flops() * self.batch // self._stack.batch

    def front_end_flops(self):
        return self._stack.front_end_flops() * self.batch // self._stack.batch

    def attention_flops(self):
        live = np.minimum(self.valid.astype(np.int64), self.frames)
        return int((live * live).sum()) * 8 * 128 * 2 * 3 * len(self.layers)


def run_encoder(args, abi, ctx, decoder=False):
    import parakeet_wgsl_amd.workloads as wl
    stack = wl.encoder_stack(0, windows=args.windows, frames=188, layers=24, front_end=True, projector=True)
    f32 = args.precision == "f32"
    if f32:
        if decoder or args.fused_norms:
            raise SystemExit("--precision f32 runs the encoder workload without the f16-only fusions")
        stack = wl.as_f32_profile(stack)
    active = args.active or stack.batch
    if not 1 <= active <= stack.batch:
        raise SystemExit(f"--active must be in [1, {stack.batch}]")
    held = []

    def put(array):
        held.append(ctx.array(np.ascontiguousarray(array)))
        return held[-1]

    def upload(value):
        return tuple(put(v) for v in value) if isinstance(value, tuple) else put(value)
    layers = []
    for layer in stack.layers:
        d = {"norm_gamma": [put(g) for g in layer["norm_gamma"]], "norm_beta": [put(b) for b in layer["norm_beta"]]}
        d.update({key: upload(value) for key, value in layer.items() if not key.startswith("norm_")})
        layers.append(d)
    front = {key: upload(value) for key, value in stack.subsampling.items()}
    features, feature_lengths, valid = put(stack.features), put(stack.feature_lengths), put(stack.valid)
    out = ctx.empty(stack.x.shape, stack.x.dtype)
    projected = ctx.empty((stack.x.shape[0], stack.projector_bias.size), stack.x.dtype)
    held += [out, projected]
    enc = abi.EncoderOp(ctx, layers=layers, valid_lengths=valid, input=features, output=out, batch_size=stack.batch,
                        frames=stack.frames, subsampling=front, feature_frames=stack.feature_frames,
                        feature_lengths=feature_lengths, projector=upload(stack.projector),
                        projector_bias=put(stack.projector_bias), projected_channels=stack.projector_bias.size,
                        projected_output=projected, fused_norms=args.fused_norms,
                        unchained_norms=args.unchained_norms, prefix_same_plan=args.prefix_same_plan,
                        fused_glu=not args.separate_glu, label="encoder",
                        precision=args.precision)
    launches, device_bytes = enc.info()
    fused_norms = set(FUSED_NORMS) if args.fused_norms else set()
    # the LN ff1 of layers after the first runs in the LN out launch before it
    chained = not (args.fused_norms or args.unchained_norms) and len(stack.layers) > 1
    stream = ctx.stream
    tdt = None
    if decoder:
        # the decoder reads the projector output [windows, 188, 640] as is
        rng = np.random.default_rng(1)
        tdt_weights = {k: put(v) for k, v in wl.tdt_weights(rng).items()}
        B, T, max_tokens = stack.batch, stack.frames, 1024
        zeros = lambda shape, dtype: put(np.zeros(shape, dtype))  # noqa: E731
        tdt_out = dict(state=zeros((B, 4, 640), np.float32), predictor_scratch=zeros((B, 5, 640), np.float32),
                       tokens=zeros((B, max_tokens), np.uint32), token_frames=zeros((B, max_tokens), np.uint32),
                       token_durations=zeros((B, max_tokens), np.uint32), metadata=zeros(2 * B, np.uint32))
        tdt = abi.TdtDecoderOp(ctx, weights=tdt_weights, encoder_projected=projected, encoded_lengths=valid,
                               decode_starts=zeros(B, np.uint32), decode_ends=put(np.full(B, T, np.uint32)),
                               flush_finals=put(np.ones(B, np.uint32)), batch_size=B, frames=T,
                               max_tokens=max_tokens, **tdt_out)
    for _ in range(args.warmup):
        enc.enqueue(active, stream, graph=True)
        if tdt:
            tdt.enqueue(active, stream)
    ctx.synchronize(stream)

    # Profiled passes (before the timed region): every launch stamped.
    profiled = [([ctx.event() for _ in range(launches)], [ctx.event() for _ in range(launches)])
                for _ in range(PROFILE_PASSES)]
    for starts, ends in profiled:
        enc.enqueue_profiled(starts, ends, active, stream)
        if tdt:
            tdt.enqueue(active, stream)
    ctx.synchronize(stream)
    durations = np.array([[a.elapsed_ms(b) for a, b in zip(starts, ends)] for starts, ends in profiled])
    durations = durations.mean(axis=0)  # ms per launch of the pass
    run = ActivePrefix(stack, active)
    front_costs, layer_costs, projector_costs = encoder_dispatch_costs(abi, wl, run, not (args.separate_glu or f32))
    nf, per = len(front_costs), len(abi.ENCODER_DISPATCHES)
    names = list(FRONT_DISPATCHES) + list(abi.ENCODER_DISPATCHES) + ["projector"] * len(projector_costs)
    costs = front_costs + layer_costs + projector_costs
    per_kind_ms = np.concatenate([durations[:nf],
                                  durations[nf:nf + per * len(stack.layers)].reshape(-1, per).mean(axis=0),
                                  durations[nf + per * len(stack.layers):]])
    dispatches = {}
    for name, ms, (flops, nbytes) in zip(names, per_kind_ms, costs):
        us = ms * 1e3
        if chained and name == "norm_feed_forward1":
            # layer 0's own launch; later layers' slots are empty (written by norm_out)
            us = durations[nf + list(abi.ENCODER_DISPATCHES).index(name)] * 1e3
            dispatches[name] = {"avg_us": us, "gbs": nbytes / (us * 1e-6) / 1e9, "flops": 0,
                                "algorithmic_bytes": nbytes, "launches_per_pass": 1,
                                "later_layers_chained_into_norm_out": True}
            continue
        if chained and name == "norm_out":
            # LN out of layer l and LN ff1 of layer l + 1 in one launch: the rows
            # read once and written twice, two gamma / beta pairs (the last
            # layer: LN out alone); averaged over the layers
            n = len(stack.layers)
            act = (nbytes - 2 * 4096) / 2
            both = 3 * act + 4 * 4096
            avg = ((n - 1) * both + nbytes) / n
            dispatches[name] = {"avg_us": us, "gbs": avg / (us * 1e-6) / 1e9, "flops": 0,
                                "algorithmic_bytes": avg, "launches_per_pass": n,
                                "chains_next_norm_feed_forward1": True}
            continue
        if name in fused_norms:
            # runs inside the GEMM after it; the slot's two events are back to back
            dispatches[name] = {"avg_us": us, "fused_into_next_gemm": True, "flops": 0, "algorithmic_bytes": 0,
                                "launches_per_pass": 0}
            continue
        dispatches[name] = {"avg_us": us, "tflops": flops / (us * 1e-6) / 1e12 if flops else 0.0,
                            "gbs": nbytes / (us * 1e-6) / 1e9, "flops": flops, "algorithmic_bytes": nbytes,
                            "launches_per_pass": len(stack.layers) if name in abi.ENCODER_DISPATCHES else 1}
    # dominant kernel: the launch kind with the most time per pass; the two
    # feed-forward modules' launches of one shape count as one kind
    def kind(k):
        return k.replace("feed-forward2-", "feed-forward1-")
    per_kind = {}
    for k, d in dispatches.items():
        per_kind[kind(k)] = per_kind.get(kind(k), 0.0) + d["avg_us"] * d["launches_per_pass"]
    name = max(per_kind, key=per_kind.get)
    if args.roofline_kind:
        if args.roofline_kind not in dispatches:
            raise SystemExit(f"--roofline-kind {args.roofline_kind}: not a launch kind of this pass")
        name = args.roofline_kind
    dom = dispatches[name]
    peak = PEAK_TFLOPS[args.precision]

    # The timed region: graph replays, and every TIMING_STRIDE-th step an
    # eager pass whose launches of the dominant kind stamp events (the
    # roofline's durations); the other launches of that pass stamp nothing.
    stamped_slots = roofline_slots(len(stack.layers), len(projector_costs), name, dispatches, launches)
    stamped = set(stamped_slots)
    timed_steps = list(range(0, args.steps, TIMING_STRIDE))
    marks = {step: ([ctx.event() if i in stamped else None for i in range(launches)],
                    [ctx.event() if i in stamped else None for i in range(launches)])
             for step in timed_steps}
    tdt_marks = {step: (ctx.event(), ctx.event()) for step in timed_steps} if tdt else {}
    start, end = ctx.event(), ctx.event()
    ctx.synchronize(stream)
    wall0 = time.perf_counter()
    start.record(stream)
    for step in range(args.steps):
        if step in marks:
            enc.enqueue_profiled(*marks[step], active, stream)
            if tdt:
                tdt.enqueue(active, stream, *tdt_marks[step])
        else:
            enc.enqueue(active, stream, graph=True)
            if tdt:
                tdt.enqueue(active, stream)
    end.record(stream)
    end.synchronize()
    ctx.synchronize(stream)
    wall = time.perf_counter() - wall0
    ms_per_step = start.elapsed_ms(end) / args.steps
    timed_us = [marks[step][0][i].elapsed_ms(marks[step][1][i]) * 1e3 for step in timed_steps for i in stamped_slots]
    decoder_ms = float(np.mean([a.elapsed_ms(b) for a, b in tdt_marks.values()])) if tdt else None
    # The roofline takes the dominant launch kind's average stamped duration
    # in the timed region (timed_us: an event pair around each of its
    # launches in the stamped steps, whose other launches run unstamped).
    # The same op launched back to back after the timed region is kept
    # beside it: its inputs stay cached between launches, so it runs faster
    # than inside the pass.
    loop_us = None
    if name in LAYER_GEMMS:
        loop_us = roofline_loop(ctx, abi, name, layers[0], out, active * stack.frames, stream)
    us = float(np.mean(timed_us))
    if dom["flops"] / (peak * 1e12) >= dom["algorithmic_bytes"] / (PEAK_HBM_GBS * 1e9):
        achieved = dom["flops"] / (us * 1e-6) / 1e12
        roofline = {"bound": "mfma", "achieved": achieved, "peak": peak, "unit": "TFLOP/s", "frac": achieved / peak}
    else:
        achieved = dom["algorithmic_bytes"] / (us * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": achieved / PEAK_HBM_GBS}
    roofline["avg_us"] = us
    roofline["timing"] = (f"an event pair around each launch of the kind in the timed region's stamped steps (every "
                          f"{TIMING_STRIDE}th step, eager, only this kind's launches stamped), averaged over "
                          f"{len(timed_us)} launches")
    roofline["profiled_passes_us"] = dom["avg_us"]
    if loop_us is not None:
        roofline["back_to_back_us"] = loop_us
        roofline["back_to_back_timing"] = (f"{ROOFLINE_LOOP[1]} launches of the kind's op at the pass's shape after "
                                           "the timed region, one event pair around the loop")
    roofline["kernel"] = f"encoder.layers.*-{name}" if name in abi.ENCODER_DISPATCHES else f"encoder.{name}"
    roofline["traffic"] = read_traffic(f"encoder-{name}", None) if not f32 else None
    roofline["traffic_source"] = TRAFFIC_SOURCE if roofline["traffic"] is not None else None

    total_flops = run.gemm_flops() + run.attention_flops() + run.front_end_flops()
    cpu_decoder = None
    if tdt and not args.no_cpu:
        rng = np.random.default_rng(1)
        window0 = projected.download()[:stack.frames]
        cpu_decoder = (wl.tdt_weights(rng), window0, int(stack.valid[0]))
    cpu = None if args.no_cpu else encoder_cpu_baseline(stack, decoder=cpu_decoder)
    decoded = None
    if tdt:
        meta = tdt_out["metadata"].download()
        decoded = {"avg_ms": decoder_ms, "tokens_per_window": [int(v) for v in meta[:active]],
                   **abi.decode_tdt_status(meta[stack.batch:stack.batch + active]),
                   "kernel": "tdt_team_kernel" if tdt.team_size() > 1 else "tdt_decode_kernel",
                   "workgroups_per_window": tdt.team_size(), "workgroups": active * tdt.team_size(),
                   "max_tokens": 1024}
    dense = None
    if not args.no_dense and not f32:
        rows = active * stack.frames
        shapes = {"feed-forward1-linear1": (1024, 4096), "feed-forward1-linear2-residual": (4096, 1024),
                  "self-attention-qkv": (1024, 3072), "convolution-pointwise1": (1024, 2048),
                  "self-attention-output-residual": (1024, 1024)}
        probes = []
        for k, (inner, columns) in shapes.items():
            probe = Kernel(k, None, 2 * rows * inner * columns, 0, "f16", (rows, inner, columns))
            probe.times_ms = [dispatches[k]["avg_us"] * 1e-3]
            probes.append(probe)
        dense = dense_reference(probes)
    ff_block = None if args.no_ff_block else ff_block_summary(abi, ctx, args)
    line = {
        "metric": METRIC,
        "value": active * WINDOW_SECONDS / (ms_per_step * 1e-3),
        "unit": "audio-sec/sec",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.precision,
        "data": "synthetic (seeded random fbank, palette codes, LUTs, norms and biases)",
        "config": {"workload": "fastconformer-tdt-transcribe-fp16" if tdt else f"fastconformer-encoder-fp{32 if f32 else 16}",
                   "windows": active, "capacity_windows": stack.batch,
                   "window_seconds": WINDOW_SECONDS, "fbank_frames": stack.feature_frames, "mel_bins": 128,
                   "frames": stack.frames, "layers": len(stack.layers), "d_model": 1024, "ff_hidden": 4096,
                   "heads": 8, "subsampling": "dw_striding 8x, 256 channels", "projector": "1024->640",
                   "palette_bits": {"ff/qkv/pointwise/subsampling/projector": 5, "o_proj": 6},
                   "dispatch_slots_per_pass": launches,
                   "launches_per_pass": launches - len(fused_norms) * len(stack.layers) -
                                        (len(stack.layers) - 1 if chained else 0),
                   "layernorms": "four of five per layer inside the GEMM they feed (PK_GEMM_ROW_NORM)"
                                 if args.fused_norms else
                                 "separate launches" if not chained else
                                 "separate launches; each layer's last LayerNorm also writes the next layer's first",
                   "glu": "in the convolution (PK_ENCODER_SEPARATE_GLU)" if args.separate_glu
                          else "in the convolution (the fp32 profile)" if f32 else "in PW1's epilogue",
                   "graph_replay": True,
                   "prefix_plans": None if active == stack.batch else
                                   ("the capacity's kernels" if args.prefix_same_plan else
                                    f"those of a graph built for {active} windows"),
                   "decoder": "greedy TDT, LSTM 2 x 640, joint 1024 + blank, 5 durations" if tdt else None},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "tflops": total_flops / (ms_per_step * 1e-3) / 1e12,
        "gemm_tflops": gemm_tflops(dispatches),
        "ff_block": ff_block,
        "device_bytes": device_bytes,
        "dispatches": dispatches,
        "dense_vendor_reference": dense,
        "decoder": decoded,
        "wall_ms_per_step": wall / args.steps * 1e3,
        "device": ctx.info().name.decode(),
    }
    print(json.dumps(line), flush=True)
    if tdt:
        tdt.release()
    enc.release()
    for arr in held:
        arr.free()
    ctx.close()


WEIGHT_STREAM_EPILOGUES = {"ff1_linear1": ("silu", None), "ff2_linear1": ("silu", None),
                           "ff1_linear2": ("none", 0.5), "ff2_linear2": ("none", 0.5),
                           "o_proj": ("none", 1.0), "pointwise2": ("none", 1.0)}


def copy_bandwidth(ctx, nbytes=1 << 30, reps=10):
    """Device-to-device copy (pk_copy_device = hipMemcpyAsync) of `nbytes`:
    read + write bytes per second, the box's own streaming ceiling."""
    src, dst = ctx.empty((nbytes // 2,), np.float16), ctx.empty((nbytes // 2,), np.float16)
    try:
        for _ in range(2):
            ctx.copy(dst, src)
        e0, e1 = ctx.event(), ctx.event()
        ctx.synchronize()
        e0.record()
        for _ in range(reps):
            ctx.copy(dst, src)
        e1.record()
        e1.synchronize()
        return 2.0 * nbytes * reps / (e0.elapsed_ms(e1) * 1e-3) / 1e9
    finally:
        src.free()
        dst.free()


def run_weight_stream(args, abi, ctx):
    """Every palette GEMM of the 24-layer encoder (8 per layer: 192 distinct
    weights, 365 MB of packed codes, more than the 256 MB last-level cache)
    at --rows rows: the small-M weight-streaming regime. Two steps are timed:
    the 192 GEMMs as one grouped small-M launch (pk_gemm_group), and the 192
    GEMMs as single launches, each on its planned kernel, replayed from a HIP
    graph (a batch-1 pass launches them one by one)."""
    import parakeet_wgsl_amd.workloads as wl
    rows = args.rows
    rng = np.random.default_rng(0)
    held = []

    def put(host):
        held.append(ctx.array(np.ascontiguousarray(host)))
        return held[-1]
    x_host, h_host = wl.normal(rng, (rows, 1024), 1.0), wl.normal(rng, (rows, 4096), 1.0)
    x, h = put(x_host), put(h_host)
    grouped, single, host_layer0 = [], [], []
    flops = nbytes = packed_bytes = 0
    for layer in range(24):
        for name, (bits, inner, columns, groups) in wl.ENCODER_MATRICES.items():
            words = wl.random_packed_words(rng, bits, inner, columns)
            palette_host = wl.normal(rng, (groups, 1 << bits), 0.02)
            if layer == 0:
                host_layer0.append((name, bits, inner, columns, words, palette_host))
            packed, palette = put(words), put(palette_host)
            activation, scale = WEIGHT_STREAM_EPILOGUES.get(name, ("none", None))
            a = x if inner == 1024 else h
            for ops in (grouped, single):
                out = ctx.empty((rows, columns), np.float16)
                held.append(out)
                ops.append(abi.GemmOp(ctx, a=a, packed=packed, palette=palette, output=out, bits=bits, rows=rows,
                                      inner=inner, columns=columns, residual=x if scale is not None else None,
                                      residual_scale=scale, activation=activation, label=f"layer{layer}-{name}"))
            packed_bytes += words.nbytes
            flops += 2 * rows * inner * columns
            nbytes += gemm_cost(rows, inner, columns, bits, groups, residual=scale is not None)[1] - 2 * rows * inner
    # every GEMM reads one of two activation inputs, which count once
    nbytes += 2 * rows * (1024 + 4096)
    small = abi.small_m_variants()
    for op in grouped:
        op.set_variant(small[0])  # the small-M code layout (one K part) that group members read
    group = abi.GemmGroup(ctx, grouped, label="encoder-weights")
    if args.variant >= 0:
        group.set_variant(args.variant)
    for op in grouped:
        op.release()
    stream = ctx.stream

    # grouped: one launch per step, each stamped by its own dispatch
    for _ in range(args.warmup):
        group.enqueue(0, stream)
    marks = [(ctx.event(), ctx.event()) for _ in range(args.steps)]
    start, end = ctx.event(), ctx.event()
    ctx.synchronize(stream)
    start.record(stream)
    for s, e in marks:
        group.enqueue(0, stream, s, e)
    end.record(stream)
    end.synchronize()
    group_ms = start.elapsed_ms(end) / args.steps
    kernel_ms = float(np.mean([s.elapsed_ms(e) for s, e in marks]))
    plan = group.plan()

    # single launches: the 192 GEMMs captured into one graph per step
    for _ in range(2):
        for op in single:
            op.enqueue(0, stream)
    graph = abi.Graph.capture(ctx, stream)
    with graph:
        for op in single:
            op.enqueue(0, stream)
    for _ in range(args.warmup):
        graph.launch()
    ctx.synchronize(stream)
    start.record(stream)
    for _ in range(args.steps):
        graph.launch()
    end.record(stream)
    end.synchronize()
    single_ms = start.elapsed_ms(end) / args.steps
    single_kernels = sorted({op.plan().kernel.decode() for op in single})

    copy_gbs = copy_bandwidth(ctx)
    gbs = nbytes / (kernel_ms * 1e-3) / 1e9
    compute_s, memory_s = flops / (PEAK_TFLOPS["f16"] * 1e12), nbytes / (PEAK_HBM_GBS * 1e9)
    if compute_s >= memory_s:
        tflops = flops / (kernel_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": tflops, "peak": PEAK_TFLOPS["f16"], "unit": "TFLOP/s",
                    "frac": tflops / PEAK_TFLOPS["f16"]}
    else:
        roofline = {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS}
    roofline["kernel"] = plan.kernel.decode()
    roofline["traffic"] = read_traffic(f"weight-stream-{rows}", plan.kernel.decode())
    roofline["traffic_source"] = TRAFFIC_SOURCE if roofline["traffic"] is not None else None

    cpu = None
    if not args.no_cpu:
        cpu = weight_stream_cpu_baseline(host_layer0, x_host, h_host, rows, all_threads())
        cpu["single_thread"] = weight_stream_cpu_baseline(host_layer0, x_host, h_host, rows, 1, budget_s=5.0)
        cpu["host"] = host_info()
    line = {
        "metric": METRIC,
        "value": nbytes / (group_ms * 1e-3) / 1e9,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": group_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded random palette codes, LUTs and activations)",
        "config": {"workload": "encoder-weight-stream-fp16", "rows": rows, "layers": 24,
                   "gemms": len(single), "matrices_per_layer": list(wl.ENCODER_MATRICES),
                   "packed_weight_bytes": packed_bytes, "algorithmic_bytes": nbytes, "flops": flops,
                   "cache_note": "the 192 distinct weights (365 MB packed) exceed the 256 MB last-level cache; "
                                 "each step streams every weight once"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "grouped": {"kernel": plan.kernel.decode(), "grid": list(plan.grid), "block": plan.block_threads,
                    "kernel_us": kernel_ms * 1e3, "gbs": gbs, "frac_of_copy": gbs / copy_gbs,
                    "tflops": flops / (kernel_ms * 1e-3) / 1e12},
        "single_launches": {"ms_per_step": single_ms, "gbs": nbytes / (single_ms * 1e-3) / 1e9,
                            "launches": len(single), "kernels": single_kernels, "graph_replay": True},
        "copy_gbs": copy_gbs,
        "copy_note": "hipMemcpyAsync device-to-device of 1 GiB, read + write bytes",
        "device": ctx.info().name.decode(),
    }
    print(json.dumps(line), flush=True)
    graph.release()
    group.release()
    for op in single:
        op.release()
    for arr in held:
        arr.free()
    ctx.close()


def weight_stream_cpu_baseline(host_layer0, x, h, rows, threads, budget_s=10.0):
    """The oracle (reference fp16 semantics) on layer 0's eight GEMMs at the
    same rows, GEMM after GEMM until about `budget_s` seconds have passed:
    algorithmic bytes per second."""
    from oracle import pko
    done_bytes, done = 0, 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s or done == 0:
        name, bits, inner, columns, words, palette = host_layer0[done % len(host_layer0)]
        activation, scale = WEIGHT_STREAM_EPILOGUES.get(name, ("none", None))
        a = x if inner == 1024 else h
        pko.gemm(a, words, bits, palette, columns, activation=activation,
                 residual=x if scale is not None else None, residual_scale=scale, mode="f16-chain", threads=threads)
        done_bytes += gemm_cost(rows, inner, columns, bits, palette.shape[0], residual=scale is not None)[1]
        done += 1
    dt = time.perf_counter() - t0
    return {"value": done_bytes / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{done} GEMMs of layer 0's eight at {rows} rows (f16-accumulator chain)", "seconds": dt}


def gemm_tflops(dispatches):
    """Palette-GEMM TFLOP/s over the pass: every palette GEMM launch's FLOP
    over the sum of their stamped durations."""
    gemms = {k: d for k, d in dispatches.items()
             if d["flops"] and k not in ("relative-attention", "subsampling-fused-conv0-depthwise2",
                                         "subsampling-depthwise5")}
    flops = sum(d["flops"] * d["launches_per_pass"] for d in gemms.values())
    us = sum(d["avg_us"] * d["launches_per_pass"] for d in gemms.values())
    return flops / (us * 1e-6) / 1e12 if us else None


def ff_block_summary(abi, ctx, args):
    """The FF block (palette-GEMM TFLOP/s of two back-to-back launches) in
    the same process, as the encoder's extra line."""
    held = []

    def keep(arr):
        held.append(arr)
        return arr
    kernels, config, _ = build_ff_block(abi, ctx, keep)
    try:
        step = measure_kernel_step(ctx, kernels, max(args.steps, 20), max(args.warmup, 5))
        return {"value": step["value"], "unit": "TFLOP/s", "ms_per_step": step["ms_per_step"], "config": config,
                "roofline": step["roofline"], "kernels": {k.name: k.summary() for k in kernels}}
    finally:
        for k in kernels:
            k.op.release()
        for arr in held:
            arr.free()


def read_traffic(gemm_name, kernel_name):
    """HBM bytes per launch of one GEMM of the step, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE per dispatch, each
    scaled by what the counter reads for a plain copy of known size), or
    None when no summary of this kernel exists."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        entry = json.load(f).get("kernels", {}).get(gemm_name)
    if entry is None or (kernel_name is not None and entry.get("kernel") != kernel_name):
        return None
    return entry["hbm_bytes_per_launch"]


def dense_reference(kernels, reps=100):
    """The vendor library's dense GEMM (torch.matmul -> hipBLASLt) at each
    GEMM launch's shape and precision with the weights already dense: what
    this shape class reaches without palette decoding, a context for the
    roofline fraction (not the step's work, and not part of `value`). Timed
    in a child process: torch carries its own HIP runtime, which does not
    share a process with this library's."""
    shaped = [k for k in kernels if k.shape is not None]
    if not shaped:
        return None
    request = [{"name": k.name, "shape": list(k.shape), "precision": k.precision} for k in shaped]
    proc = subprocess.run([sys.executable, os.path.abspath(__file__), "--dense-probe", json.dumps(request),
                           "--steps", str(reps)], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                          timeout=300)
    if proc.returncode != 0:
        return {"error": proc.stderr.strip().splitlines()[-1] if proc.stderr.strip() else "failed"}
    out = json.loads(proc.stdout.strip().splitlines()[-1])
    for k in shaped:
        out[k.name]["palette_avg_us"] = float(np.mean(k.times_ms)) * 1e3
    return out


def dense_probe(request, reps):
    import torch
    out = {}
    for item in request:
        m, kk, n = item["shape"]
        dtype = torch.float16 if item["precision"] == "f16" else torch.float32
        a = torch.randn(m, kk, device="cuda", dtype=dtype)
        b = torch.randn(kk, n, device="cuda", dtype=dtype)
        for _ in range(10):
            c = a @ b
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            c = a @ b
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / reps * 1e3
        del a, b, c
        out[item["name"]] = {"shape": [m, kk, n], "avg_us": us, "tflops": 2.0 * m * kk * n / us / 1e6}
    print(json.dumps(out), flush=True)


def measure_kernel_step(ctx, kernels, steps, warmup, use_graph=False):
    """Runs `warmup` then `steps` steps of the kernels' launches in order on
    the context's stream; returns the step time (events around the timed
    region), the per-launch stamped durations and the dominant kernel's
    roofline."""
    import parakeet_wgsl_amd.palette_abi as abi
    stream = ctx.stream
    for _ in range(warmup):
        for k in kernels:
            k.op.enqueue(0, stream)
    ctx.synchronize(stream)
    # With --graph the unstamped steps replay the step's launches from a HIP
    # graph (pk_graph_*); the stamped ones always run eagerly. For the FF
    # block a replay measured 57.8 us per step against 53.1 us for the two
    # eager launches, so eager is the default.
    graph = None
    if use_graph:
        graph = abi.Graph.capture(ctx, stream)
        with graph:
            for k in kernels:
                k.op.enqueue(0, stream)
        graph.launch()
        ctx.synchronize(stream)

    # Per-kernel durations: every TIMING_STRIDE-th step of the timed region,
    # each launch's own dispatch stamps a start and an end event
    # (pk_gemm_enqueue_timed). Stamping costs the stream a few microseconds
    # per launch, so the other steps run unstamped and the step time stays
    # that of the plain launches.
    timed_steps = list(range(0, steps, TIMING_STRIDE))
    marks = {step: [(ctx.event(), ctx.event()) for _ in kernels] for step in timed_steps}
    start, end = ctx.event(), ctx.event()
    ctx.synchronize(stream)
    wall0 = time.perf_counter()
    start.record(stream)
    for step in range(steps):
        stamps = marks.get(step)
        if stamps:
            for i, k in enumerate(kernels):
                k.op.enqueue(0, stream, *stamps[i])
        elif graph is not None:
            graph.launch()
        else:
            for k in kernels:
                k.op.enqueue(0, stream)
    end.record(stream)
    end.synchronize()
    ctx.synchronize(stream)
    wall = time.perf_counter() - wall0

    total_ms = start.elapsed_ms(end)
    for step in timed_steps:
        for i, k in enumerate(kernels):
            k.times_ms.append(marks[step][i][0].elapsed_ms(marks[step][i][1]))
    ms_per_step = total_ms / steps
    flops = sum(k.flops for k in kernels)
    value = flops / (ms_per_step * 1e-3) / 1e12

    dominant = max(kernels, key=lambda k: float(np.mean(k.times_ms)))
    dom = dominant.summary()
    peak = PEAK_TFLOPS[dominant.precision]
    compute_s = dominant.flops / (peak * 1e12)
    memory_s = dominant.nbytes / (PEAK_HBM_GBS * 1e9)
    if compute_s >= memory_s:
        roofline = {"bound": "mfma", "achieved": dom["tflops"], "peak": peak, "unit": "TFLOP/s",
                    "frac": dom["tflops"] / peak}
    else:
        roofline = {"bound": "hbm", "achieved": dom["gbs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": dom["gbs"] / PEAK_HBM_GBS}
    roofline["kernel"] = dom["kernel"]
    roofline["traffic"] = read_traffic(dominant.name, dom["kernel"])
    roofline["traffic_source"] = TRAFFIC_SOURCE if roofline["traffic"] is not None else None

    return {"ms_per_step": ms_per_step, "wall": wall, "value": value, "dominant": dominant, "dom": dom,
            "roofline": roofline, "graph": graph}


def main():
    args = parse_args()
    if args.split_trace:
        split_trace(args.split_trace, args.warmup, args.steps)
        return
    if args.split_counters:
        split_counters(*args.split_counters.split(","), args.warmup, args.steps, args.bench_json)
        return
    if args.dense_probe:
        dense_probe(json.loads(args.dense_probe), args.steps)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the palette path shards by windows with no exchange step)", file=sys.stderr)
        sys.exit(2)

    import parakeet_wgsl_amd.palette_abi as abi
    ctx = abi.Context(0)
    if args.workload in ("encoder", "transcribe"):
        run_encoder(args, abi, ctx, decoder=args.workload == "transcribe")
        return
    if args.workload == "weight-stream":
        run_weight_stream(args, abi, ctx)
        return
    held = []

    def keep(arr):
        held.append(arr)
        return arr

    if args.workload == "ff-block":
        kernels, config, data = build_ff_block(abi, ctx, keep)
    elif args.workload == "single-gemm-fp32":
        kernels, config, data = build_single_gemm(abi, ctx, keep)
    elif args.workload in ("conv-module", "conv-module-fused"):
        kernels, config, data = build_conv_module(abi, ctx, keep, args.workload == "conv-module-fused")
    elif args.workload == "rel-pos-mha":
        kernels, config, data = build_mha(abi, ctx, keep, args.frames)
    elif args.workload == "layer-gemms":
        kernels, config, data = build_layer_gemms(abi, ctx, keep, args.rows)
    else:
        kernels, config, data = build_small_m(abi, ctx, keep, args.rows)
    if args.variant >= 0:
        for k in kernels:
            if isinstance(k.op, (abi.GemmOp, RotatingOp)):
                try:
                    k.op.set_variant(args.variant)
                except abi.PaletteRangeError:
                    if args.workload != "layer-gemms":
                        raise
                    k.name += " (planned: the forced variant cannot run it)"

    step = measure_kernel_step(ctx, kernels, args.steps, args.warmup, args.graph)
    dominant, dom, roofline = step["dominant"], step["dom"], step["roofline"]
    ms_per_step, wall, graph = step["ms_per_step"], step["wall"], step["graph"]
    value = step["value"]

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.workload, data, args.cpu_sample_rows)
        cpu["single_thread"] = cpu_baseline(args.workload, data, args.cpu_sample_rows, threads=1)
        cpu["host"] = host_info()
    dense = None if args.no_dense else dense_reference(kernels)

    line = {
        "metric": METRIC,
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if dominant.precision == "f16" else "f32",
        "data": "synthetic (seeded random palette codes, LUTs and activations)",
        "config": config,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": {k.name: k.summary() for k in kernels},
        "dense_vendor_reference": dense,
        "wall_ms_per_step": wall / args.steps * 1e3,
        "graph_replay": graph is not None,
        "device": ctx.info().name.decode(),
    }
    print(json.dumps(line), flush=True)
    if graph is not None:
        graph.release()
    for k in kernels:
        k.op.release()
    for arr in held:
        arr.free()
    ctx.close()


if __name__ == "__main__":
    main()

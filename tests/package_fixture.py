"""A synthetic parakeet-webgpu-v1 package for the loader tests.

The inventory, tensor order, records and 256-byte alignment are the
converter's (model/convert.py: ShardWriter :156-262, pack_preprocessor
:1231-1262, pack_subsampling :1264-1340, pack_encoder_layer :1343-1475,
pack_decoder :1608-1702, fold_batch_norm :1705-1735, add_matrix /
add_palettized_matrix :1737-1808); the manifest carries the published
source metadata and fixed config (src/model/manifest.ts). Byte totals
therefore equal the published package's (src/model/runtime-plan.ts:10-20),
so the fixed-inventory plan accepts it. The values are the workloads'
seeded weights; nothing of the real model is in it.
"""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np

ALIGNMENT = 256

SOURCE = {
    "repository": "nvidia/parakeet-tdt-0.6b-v2",
    "revision": "ae9ad07059c7c739ffaf932226a8fe64ae2620b0",
    "archive": {"name": "parakeet-tdt-0.6b-v2.nemo", "byteLength": 2472222720,
                "sha256": "d99e39955c9d3d0350d8fb7c75e40c64a2b2eaeb003883d7c941fd2e8747b28c"},
    "weights": {"name": "model_weights.ckpt", "byteLength": 2471920514,
                "sha256": "fb1cbe2765fb80c02c0f874b6ea2c2bd24048c3618c092584fd086c6366e48a9"},
    "license": "CC-BY-4.0",
}


def config(precision: str = "fp16") -> dict:
    return {
        "sampleRate": 16000, "windowSamples": 240000, "windowSeconds": 15, "windowOverlapSeconds": 2,
        "featureBins": 128, "fftSize": 512, "windowSize": 400, "hopSize": 160, "preemphasis": 0.97,
        "logZeroGuard": 2.0 ** -24, "normalizationEpsilon": 1e-5, "subsamplingFactor": 8, "encoderLayers": 24,
        "encoderHiddenSize": 1024, "intermediateSize": 4096, "attentionHeads": 8, "attentionHeadSize": 128,
        "convolutionKernelSize": 9, "decoderHiddenSize": 640, "decoderLayers": 2, "vocabularySize": 1025,
        "blankTokenId": 1024, "jointOutputSize": 1030, "jointStorageOutputSize": 1032,
        "durations": [0, 1, 2, 3, 4], "maxSymbolsPerStep": 10,
        "encoderWeightFormat": f"mixed-palette5-o-proj-palette6-{precision}-lut",
    }


class Entry:
    """One tensor record: name, dtype, logical and storage shape, layout and
    the key of its values (None: seeded filler)."""

    def __init__(self, name, dtype, logical, storage, layout, key=None):
        self.name, self.dtype, self.logical, self.storage, self.layout, self.key = \
            name, dtype, list(logical), list(storage), layout, key

    @property
    def nbytes(self) -> int:
        return int(np.prod(self.storage)) * (2 if self.dtype == "float16" else 4)


def _palette(name, inner, columns, bits, groups, fdtype, key):
    cpg, wpg = (32, 5) if bits == 5 else (16, 3)
    yield Entry(name, "uint32", [inner, columns], [inner * columns // cpg, wpg],
                f"k-by-output-row-major-palette{bits}-lsb-u32", key + (0,))
    yield Entry(f"{name}.palette", fdtype, [groups, 1 << bits], [groups, 1 << bits],
                "output-group-by-palette-lut", key + (1,))


def _channel(name, n, layout, key=None):
    yield Entry(name, "float32", [n], [n], layout, key)


def shard_inventory(precision: str = "fp16", frames: int = 188) -> dict:
    """{shard name: [Entry, ...]} in the converter's write order."""
    f = "float16" if precision == "fp16" else "float32"
    shards = {"preprocessor.bin": [
        Entry("preprocessor.window", "float32", [400], [400], "hann-periodic-false"),
        Entry("preprocessor.mel_filters", "float32", [128, 257], [128, 257], "mel-bin-by-rfft-bin"),
    ]}
    s = "encoder.subsampling"
    sub = []
    for idx, key, layout in ((0, "conv0", "kh-kw-output-channel-vec4"), (2, "depthwise2", "kh-kw-channel-vec4"),
                             (5, "depthwise5", "kh-kw-channel-vec4")):
        sub.append(Entry(f"{s}.layers.{idx}.weight", f, [3, 3, 256], [3, 3, 64, 4], layout,
                         ("sub", f"{key}_weights")))
        sub += _channel(f"{s}.layers.{idx}.bias", 256, "output-channel", ("sub", f"{key}_bias"))
    for idx, key in ((3, "pointwise3"), (6, "pointwise6")):
        sub += _palette(f"{s}.layers.{idx}.weight", 256, 256, 5, 1, f, ("sub", key))
        sub += _channel(f"{s}.layers.{idx}.bias", 256, "output-channel", ("sub", f"{key}_bias"))
    sub += _palette(f"{s}.linear.weight", 4096, 1024, 5, 1, f, ("sub", "linear"))
    sub += _channel(f"{s}.linear.bias", 1024, "output-channel", ("sub", "linear_bias"))
    shards["encoder-subsampling.bin"] = sub
    norms = ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out")
    for i in range(24):
        p = f"encoder.layers.{i}"
        layer = []
        for ff in ("1", "2"):
            layer += _palette(f"{p}.feed_forward{ff}.linear1.weight", 1024, 4096, 5, 1, f, (i, f"ff{ff}_linear1"))
            layer += _palette(f"{p}.feed_forward{ff}.linear2.weight", 4096, 1024, 5, 1, f, (i, f"ff{ff}_linear2"))
        for j, norm in enumerate(norms):
            layer += _channel(f"{p}.{norm}.weight", 1024, "channel", (i, "norm_gamma", j))
            layer += _channel(f"{p}.{norm}.bias", 1024, "channel", (i, "norm_beta", j))
        layer += _palette(f"{p}.self_attn.qkv.weight", 1024, 3072, 5, 3, f, (i, "qkv"))
        layer.append(Entry(f"{p}.self_attn.projected_positions", f, [2 * frames - 1, 1024],
                           [8, 32, 2 * frames - 1, 4], "head-vector-position-vec4", (i, "projected_positions")))
        layer += _palette(f"{p}.self_attn.o_proj.weight", 1024, 1024, 6, 1, f, (i, "o_proj"))
        for b in ("bias_u", "bias_v"):
            layer.append(Entry(f"{p}.self_attn.{b}", "float32", [8, 128], [8, 128], "head-by-channel", (i, b)))
        layer += _palette(f"{p}.conv.pointwise_conv1.weight", 1024, 2048, 5, 1, f, (i, "pointwise1"))
        layer.append(Entry(f"{p}.conv.depthwise_conv.weight", f, [9, 1024], [9, 256, 4], "kernel-channel-vec4",
                           (i, "depthwise")))
        layer += _palette(f"{p}.conv.pointwise_conv2.weight", 1024, 1024, 5, 1, f, (i, "pointwise2"))
        layer += _channel(f"{p}.conv.norm.scale", 1024, "channel", (i, "bn_scale"))
        layer += _channel(f"{p}.conv.norm.shift", 1024, "channel", (i, "bn_shift"))
        shards[f"encoder-layer-{i:02d}.bin"] = layer
    lstm = "input-hidden-k-by-ifgo-row-major-vec4"
    dec = [Entry("decoder.embedding.weight", f, [1025, 640], [1025, 640], "token-by-channel-row-major",
                 ("tdt", "embedding"))]
    for l in (0, 1):
        dec.append(Entry(f"decoder.lstm.weight_l{l}", f, [1280, 2560], [1280, 2560], lstm, ("tdt", f"lstm_weight_l{l}")))
        dec.append(Entry(f"decoder.lstm.bias_l{l}", "float32", [2560], [2560], "ifgo-gates", ("tdt", f"lstm_bias_l{l}")))
    dec.append(Entry("decoder.decoder_projector.weight", f, [640, 640], [640, 640], "k-by-output-row-major-vec4",
                     ("tdt", "projector_weight")))
    dec += _channel("decoder.decoder_projector.bias", 640, "output-channel", ("tdt", "projector_bias"))
    dec += _palette("encoder_projector.weight", 1024, 640, 5, 1, f, ("projector",))
    dec += _channel("encoder_projector.bias", 640, "output-channel", ("projector_bias",))
    dec.append(Entry("joint.head.weight", f, [640, 1030], [640, 1032], "k-by-output-row-major-vec4",
                     ("tdt", "head_weight")))
    dec.append(Entry("joint.head.bias", "float32", [1030], [1032], "output-channel-padded-vec4", ("tdt", "head_bias")))
    shards["decoder.bin"] = dec
    return shards


def _align(n: int) -> int:
    return -(-n // ALIGNMENT) * ALIGNMENT


def layout_records(shards: dict) -> tuple[dict, dict]:
    """Tensor records with ShardWriter offsets, and each shard's byte length
    (padded to the alignment when the writer closes)."""
    tensors, sizes = {}, {}
    for shard, entries in shards.items():
        offset = 0
        for e in entries:
            offset = _align(offset)
            tensors[e.name] = {"shard": shard, "byteOffset": offset, "byteLength": e.nbytes, "dtype": e.dtype,
                               "logicalShape": e.logical, "storageShape": e.storage, "layout": e.layout}
            offset += e.nbytes
        sizes[shard] = _align(offset)
    return tensors, sizes


def manifest(precision: str = "fp16", files: list | None = None, frames: int = 188) -> dict:
    """The manifest of the synthetic package; file digests are zeros unless
    `files` (name, byteLength, sha256 records) is given."""
    tensors, sizes = layout_records(shard_inventory(precision, frames))
    if files is None:
        files = [{"name": n, "byteLength": b, "sha256": "0" * 64} for n, b in sorted(sizes.items())]
    return {"format": "parakeet-webgpu-v1" if precision == "fp16" else "parakeet-webgpu-fp32-v1",
            "source": SOURCE, "config": config(precision), "files": files, "tensors": tensors}


def _values(entry: Entry, stack, tdt: dict, rng) -> np.ndarray:
    key = entry.key
    dtype = {"float16": np.float16, "float32": np.float32, "uint32": np.uint32}[entry.dtype]
    value = None
    if stack is None:
        return np.zeros(entry.storage, dtype)
    if key is None:
        value = rng.standard_normal(int(np.prod(entry.storage))).astype(dtype)
    elif key[0] == "tdt":
        value = tdt[key[1]]
    elif key[0] == "sub":
        v = stack.subsampling[key[1]]
        value = v[key[2]] if len(key) > 2 else v
    elif key[0] == "projector":
        value = stack.projector[key[1]]
    elif key[0] == "projector_bias":
        value = stack.projector_bias
    elif isinstance(key[0], int) and key[0] < len(stack.layers):
        v = stack.layers[key[0]][key[1]]
        value = v[key[2]] if len(key) > 2 else v
    else:  # a layer the stack does not hold: a copy of the last one's values
        v = stack.layers[-1][key[1]]
        value = v[key[2]] if len(key) > 2 else v
    value = np.ascontiguousarray(value)
    if value.dtype != dtype or value.nbytes != entry.nbytes:
        raise ValueError(f"{entry.name}: {value.dtype} {value.nbytes} B, record {entry.dtype} {entry.nbytes} B")
    return value


def write_package(directory: str, stack=None, tdt: dict | None = None, seed: int = 0, frames: int = 188,
                  precision: str = "fp16") -> str:
    """Writes the shards, tokenizer.json and manifest.json of an fp16 or fp32
    package; returns the manifest path. Without a stack every tensor is zero;
    an fp32 package takes an f32-profile stack and f32 decoder weights."""
    os.makedirs(directory, exist_ok=True)
    rng = np.random.default_rng(seed)
    frames = stack.frames if stack is not None else frames
    shards = shard_inventory(precision, frames)
    tensors, sizes = layout_records(shards)
    files = []
    for shard, entries in sorted(shards.items()):
        digest = hashlib.sha256()
        with open(os.path.join(directory, shard), "wb") as out:
            offset = 0
            for e in entries:
                pad = _align(offset) - offset
                if pad:
                    out.write(b"\0" * pad)
                    digest.update(b"\0" * pad)
                    offset += pad
                data = _values(e, stack, tdt, rng).tobytes()
                out.write(data)
                digest.update(data)
                offset += len(data)
            pad = _align(offset) - offset
            if pad:
                out.write(b"\0" * pad)
                digest.update(b"\0" * pad)
                offset += pad
        assert offset == sizes[shard]
        files.append({"name": shard, "byteLength": offset, "sha256": digest.hexdigest()})
    tokenizer = json.dumps({"type": "synthetic", "pieces": [f"<{i}>" for i in range(1024)]}).encode()
    with open(os.path.join(directory, "tokenizer.json"), "wb") as out:
        out.write(tokenizer)
    files.append({"name": "tokenizer.json", "byteLength": len(tokenizer),
                  "sha256": hashlib.sha256(tokenizer).hexdigest()})
    path = os.path.join(directory, "manifest.json")
    with open(path, "w") as out:
        json.dump(manifest(precision, files, frames), out)
    return path

// GPU run of the Node host's encoder graph: the package's tensors (under the
// reference's names and records) become GpuTensors, ParakeetEncoderGraph
// binds them (encoder.ts:1299-1530), uploadFeatures / encode run the front
// end, the layers and the projector (encoder.ts:1690-1706), eagerly, from a
// HIP graph and with per-launch timestamps. Usage: node host_gpu_encoder.js <case.json>.
"use strict";
const assert = require("assert");
const fs = require("fs");
const path = require("path");
const host = require(path.join(__dirname, "..", "..", "parakeet.wgsl_amd", "host"));

function bytesOf(file) {
  const b = fs.readFileSync(file);
  return new Uint8Array(b.buffer, b.byteOffset, b.byteLength);
}

async function main() {
  const spec = JSON.parse(fs.readFileSync(process.argv[2], "utf8"));
  const device = host.HipGpuDevice.create();
  const tensors = new Map();
  for (const [name, t] of Object.entries(spec.tensors)) {
    const record = { dtype: t.dtype, logicalShape: t.logicalShape, storageShape: t.storageShape,
                     byteLength: fs.statSync(t.file).size, layout: t.layout };
    tensors.set(name, host.createGpuTensor(device, { sourceRecord: record, runtimeRecord: record, label: name },
                                           bytesOf(t.file)));
  }
  const model = { tensor(name) {
    const t = tensors.get(name);
    if (t === undefined) throw new Error(`Missing tensor ${name}`);
    return t;
  } };
  const graph = await host.ParakeetEncoderGraph.create(device, model,
                                                       { batchSize: spec.batchSize, layers: spec.layers });
  assert.strictEqual(graph.dispatchCount, 6 + spec.layers * host.ENCODER_LAYER_DISPATCHES + 1);
  const features = bytesOf(spec.features);
  graph.uploadFeatures(new Float32Array(features.buffer, features.byteOffset, features.byteLength / 4));
  const rows = spec.batchSize * host.PARAKEET_ENCODER_FRAMES;
  const read = async (buffer, size) => Buffer.from(await device.queue.readBuffer(buffer, 0, size));

  const outputs = {};
  for (const mode of ["eager", "graph", "profiled"]) {
    const encoder = device.createCommandEncoder({ label: `encode-${mode}` });
    let timestamps = null;
    if (mode === "profiled") {
      timestamps = device.createQuerySet({ type: "timestamp", count: 2 * graph.dispatchCount });
      graph.encode(encoder, spec.featureLengths, { timestamps: { querySet: timestamps } });
    } else {
      const derived = graph.encode(encoder, spec.featureLengths, { useGraph: mode === "graph" });
      assert.deepStrictEqual(Array.from(derived), spec.encoderLengths);
    }
    device.queue.submit([encoder.finish()]);
    await device.queue.onSubmittedWorkDone();
    outputs[mode] = [await read(graph.outputBuffer, rows * 1024 * 2),
                     await read(graph.projectedOutputBuffer, rows * 640 * 2)];
    if (timestamps) {
      let total = 0;
      for (let i = 0; i < graph.dispatchCount; ++i) total += timestamps.elapsedMs(2 * i, 2 * i + 1);
      assert.ok(total > 0, `profiled pass ${total} ms`);
      console.log(`profiled pass: ${graph.dispatchCount} launches, ${total.toFixed(3)} ms of kernel time`);
      timestamps.destroy();
    }
  }
  for (const mode of ["graph", "profiled"]) {
    assert.ok(outputs[mode][0].equals(outputs.eager[0]), `${mode} output differs from the eager pass`);
    assert.ok(outputs[mode][1].equals(outputs.eager[1]), `${mode} projection differs from the eager pass`);
  }
  fs.writeFileSync(spec.output, outputs.eager[0]);
  fs.writeFileSync(spec.projected, outputs.eager[1]);
  assert.throws(() => graph.uploadValidFeatureLengths([1502]), RangeError);
  assert.throws(() => graph.encode(device.createCommandEncoder(), new Array(spec.batchSize + 1).fill(100)),
                /Encoder active batch must be in \[1, /);
  graph.destroy();
  graph.destroy();
  assert.throws(() => graph.encode(device.createCommandEncoder(), [100]), /encoder graph was destroyed/);
  for (const t of tensors.values()) t.buffer.destroy();
  device.destroy();
  console.log("host_gpu_encoder ok");
}

main().catch((e) => { console.error(e); process.exit(1); });

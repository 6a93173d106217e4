// GPU run of the Node host's Conformer convolution tail: the pointwise-1
// output goes into an arena slice, FusedConformerConvKernel.createDispatch
// binds it with the depthwise weights, folded batch norm and valid lengths,
// and encode / submit runs it as the reference's encoder graph does
// (src/webgpu/encoder.ts:2035-2058). Usage: node host_gpu_conv.js <case.json>.
"use strict";
const assert = require("assert");
const fs = require("fs");
const path = require("path");
const host = require(path.join(__dirname, "..", "..", "parakeet.wgsl_amd", "host"));

function bytesOf(file) {
  const b = fs.readFileSync(file);
  return new Uint8Array(b.buffer, b.byteOffset, b.byteLength);
}
function align(n) {
  return Math.ceil(n / 256) * 256;
}

async function main() {
  const spec = JSON.parse(fs.readFileSync(process.argv[2], "utf8"));
  const { batchSize, frames } = spec;
  const rows = batchSize * frames;
  const device = host.HipGpuDevice.create();
  const inBytes = rows * 2048 * 2, outBytes = rows * 1024 * 2;
  const arena = new host.GpuActivationArena(device, align(inBytes) + align(outBytes) + 256);
  const input = arena.slice("pointwise", 0, inBytes);
  const output = arena.slice("conv-out", align(inBytes), outBytes);
  const valid = arena.slice("valid", align(inBytes) + align(outBytes), 4 * batchSize);
  arena.upload(device, input, bytesOf(spec.pointwise));
  arena.upload(device, valid, bytesOf(spec.valid));
  const rec = host.conformerConvTensorRecords();
  const weights = host.createGpuTensor(device, rec.depthwiseWeights, bytesOf(spec.weights));
  const scale = host.createGpuTensor(device, rec.batchNormScale, bytesOf(spec.scale));
  const shift = host.createGpuTensor(device, rec.batchNormShift, bytesOf(spec.shift));
  const kernel = await host.FusedConformerConvKernel.create(device, arena, 64);
  const dispatch = kernel.createDispatch({
    label: "node-host-conv", batchSize, frames, pointwiseInput: input, depthwiseWeights: weights,
    batchNormScale: scale, batchNormShift: shift, validLengths: valid, output,
  });
  assert.strictEqual(dispatch.result.rows, rows);
  const timestamps = device.createQuerySet({ type: "timestamp", count: 2 });
  const encoder = device.createCommandEncoder({ label: "node-host-conv" });
  dispatch.encode(encoder, { querySet: timestamps, beginningOfPassWriteIndex: 0, endOfPassWriteIndex: 1 },
                  { batchSize: spec.activeBatch });
  device.queue.submit([encoder.finish()]);
  await device.queue.onSubmittedWorkDone();
  const result = await device.queue.readBuffer(arena.buffer, output.byteOffset, outBytes);
  fs.writeFileSync(spec.output, Buffer.from(result));
  const ms = timestamps.elapsedMs(0, 1);
  assert.ok(ms > 0, `timestamp ${ms}`);
  assert.throws(() => dispatch.encode(device.createCommandEncoder(), undefined, { batchSize: batchSize + 1 }),
                (e) => e instanceof RangeError && /node-host-conv active batch must be in \[1, /.test(e.message));
  dispatch.destroy();
  dispatch.destroy();
  assert.throws(() => dispatch.encode(device.createCommandEncoder()), /node-host-conv was destroyed/);
  timestamps.destroy();
  arena.destroy();
  for (const t of [weights, scale, shift]) t.buffer.destroy();
  device.destroy();
  console.log(`host_gpu_conv ok ${ms.toFixed(3)} ms`);
}

main().catch((e) => { console.error(e); process.exit(1); });

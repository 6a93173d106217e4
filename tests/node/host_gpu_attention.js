// GPU run of the Node host's relative-position attention: the QKV and
// valid lengths go into arena slices, the projected positions and the u / v
// biases are package tensors with the reference's records, and
// RelativeAttentionKernel.createDispatch / encode / submit runs it as the
// reference's encoder graph does (src/webgpu/encoder.ts:1956-1991).
// Usage: node host_gpu_attention.js <case.json>.
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
  const qkvBytes = rows * 3072 * 2, outBytes = rows * 1024 * 2;
  const arena = new host.GpuActivationArena(device, align(qkvBytes) + align(outBytes) + 256);
  const qkv = arena.slice("qkv", 0, qkvBytes);
  const output = arena.slice("context", align(qkvBytes), outBytes);
  const valid = arena.slice("valid", align(qkvBytes) + align(outBytes), 4 * batchSize);
  arena.upload(device, qkv, bytesOf(spec.qkv));
  arena.upload(device, valid, bytesOf(spec.valid));
  const rec = host.relativeAttentionTensorRecords(frames);
  const positions = host.createGpuTensor(device, rec.projectedPositions, bytesOf(spec.positions));
  const biasU = host.createGpuTensor(device, rec.biasU, bytesOf(spec.biasU));
  const biasV = host.createGpuTensor(device, rec.biasV, bytesOf(spec.biasV));
  const kernel = await host.RelativeAttentionKernel.create(device, arena, 64);
  const dispatch = kernel.createDispatch({
    label: "node-host-attention", qkv, projectedPositions: positions, biasU, biasV, validLengths: valid, output,
    batchSize, frames,
  });
  const timestamps = device.createQuerySet({ type: "timestamp", count: 2 });
  const encoder = device.createCommandEncoder({ label: "node-host-attention" });
  dispatch.encode(encoder, { querySet: timestamps, beginningOfPassWriteIndex: 0, endOfPassWriteIndex: 1 },
                  { batchSize: spec.activeBatch });
  device.queue.submit([encoder.finish()]);
  await device.queue.onSubmittedWorkDone();
  const result = await device.queue.readBuffer(arena.buffer, output.byteOffset, outBytes);
  fs.writeFileSync(spec.output, Buffer.from(result));
  const ms = timestamps.elapsedMs(0, 1);
  assert.ok(ms > 0, `timestamp ${ms}`);
  assert.throws(() => dispatch.encode(device.createCommandEncoder(), undefined, { batchSize: batchSize + 1 }),
                (e) => e instanceof RangeError && /node-host-attention active batch must be in \[1, /.test(e.message));
  dispatch.destroy();
  dispatch.destroy();
  assert.throws(() => dispatch.encode(device.createCommandEncoder()), /node-host-attention was destroyed/);
  timestamps.destroy();
  arena.destroy();
  for (const t of [positions, biasU, biasV]) t.buffer.destroy();
  device.destroy();
  console.log(`host_gpu_attention ok ${ms.toFixed(3)} ms`);
}

main().catch((e) => { console.error(e); process.exit(1); });

// GPU run of the Node host: one palette GEMM through HipGpuDevice /
// GpuActivationArena / F16GemmKernel.createDispatch / encode / submit,
// exactly as the reference's encoder graph drives its GEMM owners.
// Usage: node host_gpu.js <case.json>; the case file names the raw input
// files and where to write the output. Run by tests/test_node_host.py.
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
  const { rows, inner, columns, bits, groups } = spec;
  const device = host.HipGpuDevice.create();
  assert.ok(device.info.arch.startsWith("gfx950"), device.info.arch);
  const aBytes = rows * inner * 2, cBytes = rows * columns * 2;
  const arena = new host.GpuActivationArena(device, align(aBytes) + 2 * align(cBytes));
  const a = arena.slice("a", 0, aBytes);
  const out = arena.slice("out", align(aBytes), cBytes);
  arena.upload(device, a, bytesOf(spec.a));
  const records = host.paletteTensorRecords({ paletteBits: bits, inner, columns, paletteGroups: groups });
  const b = host.createGpuTensor(device, records.weight, bytesOf(spec.packed));
  const palette = host.createGpuTensor(device, records.palette, bytesOf(spec.palette));
  const descriptor = {
    label: "node-host-gemm", a, b, bPalette: palette, paletteGroupColumns: columns / groups, output: out,
    rows, inner, columns, activation: spec.activation,
  };
  let residual;
  if (spec.residual) {
    residual = arena.slice("residual", align(aBytes) + align(cBytes), cBytes);
    arena.upload(device, residual, bytesOf(spec.residual));
    descriptor.residual = residual;
    descriptor.residualScale = spec.residualScale;
  }
  const kernel = await host.F16GemmKernel.create(device, arena, undefined, { allowSyntheticShapes: true });
  const backend = host.createEncoderGemmBackend(kernel);
  const prepared = backend.createPreparedPaletteWeight(descriptor, 0);
  const dispatch = backend.createDispatch(Object.assign({}, descriptor, { preparedPaletteWeight: prepared }));
  const timestamps = device.createQuerySet({ type: "timestamp", count: 2 });
  const encoder = device.createCommandEncoder({ label: "node-host" });
  dispatch.encode(encoder, { querySet: timestamps, beginningOfPassWriteIndex: 0, endOfPassWriteIndex: 1 },
                  { batchSize: 1, rows: spec.activeRows });
  device.queue.submit([encoder.finish()]);
  await device.queue.onSubmittedWorkDone();
  const result = await device.queue.readBuffer(arena.buffer, out.byteOffset, cBytes);
  fs.writeFileSync(spec.output, Buffer.from(result));
  const ms = timestamps.elapsedMs(0, 1);
  assert.ok(ms > 0, `timestamp ${ms}`);
  // the plan names the launch's kernel and whether its output stores are non-temporal
  const plan = dispatch.plan(spec.activeRows);
  assert.strictEqual(typeof plan.kernel, "string");
  assert.strictEqual(typeof plan.streamStores, "boolean");
  // encode after destroy throws the reference's error; destroy is idempotent
  dispatch.destroy();
  dispatch.destroy();
  assert.throws(() => dispatch.encode(device.createCommandEncoder()), /node-host-gemm was destroyed/);
  // an active row count past the capacity is a RangeError (gemm.ts:431-438)
  const again = backend.createDispatch(descriptor);
  assert.throws(() => again.encode(device.createCommandEncoder(), undefined, { batchSize: 1, rows: rows + 1 }),
                (e) => e instanceof RangeError && /active rows must be in \[1, /.test(e.message));
  again.destroy();
  prepared.preparation.destroy();
  timestamps.destroy();
  arena.destroy();
  b.buffer.destroy();
  palette.buffer.destroy();
  device.destroy();
  console.log(`host_gpu ok ${ms.toFixed(3)} ms`);
}

main().catch((e) => { console.error(e); process.exit(1); });

// GPU run of the Node host end to end: ParakeetGpuPackage.load of a
// synthetic package -> ParakeetEncoderGraph (fbank -> 24 layers ->
// projector, graph replay) -> PersistentTdtDecoderKernel over arena slices,
// in the package's execution profile (spec.precision "fp16" or "fp32").
// Writes the projector output and the decoder outputs for
// tests/test_node_host.py to check. argv: <case.json>
"use strict";
const fs = require("fs");
const path = require("path");
const host = require(path.join(__dirname, "..", "..", "parakeet.wgsl_amd", "host"));

async function main() {
  const spec = JSON.parse(fs.readFileSync(process.argv[2], "utf8"));
  const device = host.HipGpuDevice.create();
  const precision = spec.precision || "fp16";
  const executionProfile = { precision };
  const pkg = await host.ParakeetGpuPackage.load(device, spec.manifest, {
    expectedPrecision: precision, manifestSha256: spec.manifestSha256,
  });
  console.log(`loaded ${pkg.memory.runtimeBufferCount} shards, ${pkg.memory.retainedRuntimeBytes} bytes`);
  const windows = spec.windows;
  const graph = await host.ParakeetEncoderGraph.create(device, pkg, { batchSize: windows, executionProfile });
  const features = fs.readFileSync(spec.features);
  graph.uploadFeatures(new Uint8Array(features.buffer, features.byteOffset, features.byteLength));
  let encoder = device.createCommandEncoder({ label: "encode" });
  const lengths = graph.encode(encoder, spec.featureLengths, { useGraph: true });
  device.queue.submit([encoder.finish()]);
  await device.queue.onSubmittedWorkDone();
  const frames = graph.frames;
  const projectedBytes = windows * frames * 640 * (precision === "fp32" ? 4 : 2);
  const projected = await device.queue.readBuffer(graph.projectedOutputBuffer, 0, projectedBytes);
  fs.writeFileSync(spec.projected, Buffer.from(projected));
  console.log("encoded", Array.from(lengths).join(","));

  // Decoder slices in one arena, 256-byte aligned as the reference's arena.
  const sizes = {
    encoderProjected: projectedBytes, encodedLengths: windows * 4, decodeStarts: windows * 4, decodeEnds: windows * 4,
    flushFinals: windows * 4, state: windows * 4 * 640 * 4,
    predictorScratch: host.planTdtDecoderExecution(windows).predictorScratchByteLength,
    tokens: windows * spec.maxTokens * 4, tokenFrames: windows * spec.maxTokens * 4,
    tokenDurations: windows * spec.maxTokens * 4, metadata: windows * 2 * 4,
  };
  let total = 0;
  const offsets = {};
  for (const name of Object.keys(sizes)) {
    offsets[name] = total;
    total += Math.ceil(sizes[name] / 256) * 256;
  }
  const arena = new host.GpuActivationArena(device, total, "decoder-arena");
  const descriptor = { batchSize: windows, frames, maxTokens: spec.maxTokens, label: "transcribe-decode" };
  for (const name of Object.keys(sizes)) descriptor[name] = arena.slice(name, offsets[name], sizes[name]);
  arena.upload(device, descriptor.encoderProjected, new Uint8Array(projected));
  arena.upload(device, descriptor.encodedLengths, lengths);
  arena.upload(device, descriptor.decodeStarts, new Uint32Array(windows));
  arena.upload(device, descriptor.decodeEnds, new Uint32Array(windows).fill(frames));
  arena.upload(device, descriptor.flushFinals, new Uint32Array(windows).fill(1));
  arena.upload(device, descriptor.state, new Float32Array(windows * 4 * 640));
  const kernel = await host.PersistentTdtDecoderKernel.create(device, arena, pkg, executionProfile);
  const dispatch = kernel.createDispatch(descriptor);
  console.log(`decoder team size ${dispatch.teamSize}`);
  encoder = device.createCommandEncoder({ label: "decode" });
  dispatch.encode(encoder);
  device.queue.submit([encoder.finish()]);
  await device.queue.onSubmittedWorkDone();
  const read = (name) => device.queue.readBuffer(arena.buffer, offsets[name], sizes[name]);
  const out = {};
  for (const name of ["tokens", "tokenFrames", "tokenDurations", "metadata"]) {
    out[name] = Array.from(new Uint32Array(await read(name)));
  }
  fs.writeFileSync(spec.decoded, JSON.stringify(out));
  console.log("counts", out.metadata.slice(0, windows).join(","), `team size after the launch ${dispatch.teamSize}`);
  const expectedTeam = precision === "fp32" ? 1 : 16;
  if (dispatch.teamSize !== expectedTeam)
    throw new Error(`decoder ran with team size ${dispatch.teamSize}, expected ${expectedTeam}`);
  dispatch.destroy();
  dispatch.destroy();
  arena.destroy();
  graph.destroy();
  pkg.destroy();
  device.destroy();
  console.log("transcribe ok");
}

main().catch((error) => {
  console.error(error);
  process.exit(1);
});

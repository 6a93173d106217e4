// CPU checks of the Node host (no GPU): exports, record checks and the
// C ABI descriptor contract reached through the N-API addon. Run by
// tests/test_node_host.py; exits non-zero on the first failure.
"use strict";
const assert = require("assert");
const path = require("path");
const host = require(path.join(__dirname, "..", "..", "parakeet.wgsl_amd", "host"));

const native = host.native();
assert.strictEqual(native.abiVersion(), 1);
for (const name of ["contextCreate", "gemmCreate", "gemmValidate", "gemmEnqueue", "gemmDestroy", "gemmPlan",
                    "preparedWeightCreate", "synchronizeAsync", "alloc", "upload", "download"]) {
  assert.strictEqual(typeof native[name], "function", name);
}
assert.strictEqual(host.paletteBitsForLayout("k-by-output-row-major-palette5-lsb-u32"), 5);
assert.strictEqual(host.paletteBitsForLayout("k-by-output-row-major-palette6-lsb-u32"), 6);
assert.strictEqual(host.paletteBitsForLayout("n256-k32-tile-major-f16"), undefined);

// A kernel over a stand-in device and arena: descriptor checks need no GPU.
const fakeBuffer = { address: 1n << 20n, label: "fake" };
const arena = Object.create(host.GpuActivationArena.prototype);
Object.assign(arena, { buffer: fakeBuffer, byteLength: 1 << 30, destroyed: false, label: "arena" });
function tensor(records) {
  return { sourceRecord: records.sourceRecord, runtimeRecord: records.runtimeRecord,
           binding: { buffer: fakeBuffer, offset: 0, size: records.runtimeRecord.byteLength } };
}
function descriptor(over) {
  const rows = over.rows || 7520, inner = over.inner || 1024, columns = over.columns || 4096;
  const bits = over.bits || 5;
  const rec = host.paletteTensorRecords({ paletteBits: bits, inner, columns, paletteGroups: over.groups || 1 });
  const d = {
    label: over.label || "encoder-layer-ff-expand",
    a: arena.slice("a", 0, rows * inner * 2),
    b: tensor(rec.weight),
    bPalette: tensor(rec.palette),
    paletteGroupColumns: columns / (over.groups || 1),
    output: arena.slice("c", 256 * 1024 * 1024, rows * columns * 2),
    rows, inner, columns,
  };
  if (over.activation !== undefined) d.activation = over.activation;
  if (over.residual) d.residual = arena.slice("r", 512 * 1024 * 1024, rows * columns * 2);
  if (over.residualScale !== undefined) d.residualScale = over.residualScale;
  if (over.mutate) over.mutate(d, rec);
  return d;
}

function throwsLike(fn, Kind, text) {
  let caught = null;
  try { fn(); } catch (e) { caught = e; }
  assert.ok(caught, `expected ${Kind.name}: ${text}`);
  assert.ok(caught instanceof Kind, `${caught.constructor.name} is not ${Kind.name}: ${caught.message}`);
  assert.ok(caught.message.includes(text), `"${caught.message}" lacks "${text}"`);
}

host.F16GemmKernel.create({}, arena).then((kernel) => {
  // A production signature passes (gemm.ts:204-356).
  kernel.validateDescriptor(descriptor({ activation: "silu" }));
  kernel.validateDescriptor(descriptor({ label: "encoder-layer-ff-contract", inner: 4096, columns: 1024,
                                         residual: true, residualScale: 0.5 }));
  kernel.validateDescriptor(descriptor({ label: "encoder-layer-attention-qkv", columns: 3072, groups: 3 }));
  // requireGemmShape (gemm.ts:971-1010)
  throwsLike(() => kernel.validateDescriptor(descriptor({ inner: 1000, activation: "silu" })), RangeError,
             "Unsupported GEMM shape for encoder-layer-ff-expand");
  throwsLike(() => kernel.validateDescriptor(descriptor({ columns: 4100, activation: "silu" })), RangeError,
             "Unsupported GEMM shape for encoder-layer-ff-expand");
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu",
      mutate: (d) => { d.b.sourceRecord = Object.assign({}, d.b.sourceRecord, { logicalShape: [2048, 4096] }); } })),
      Error, "weight package does not match K=1024, N=4096");
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu",
      mutate: (d) => { d.b.sourceRecord = Object.assign({}, d.b.sourceRecord, { layout: "n256-k32-tile-major-f16" }); } })),
      Error, "has an unsupported weight format");
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu",
      mutate: (d) => { d.b.sourceRecord = Object.assign({}, d.b.sourceRecord, { byteLength: 4 }); } })),
      Error, "has invalid packed palette indices");
  // requireProductionSpecialization (gemm.ts:1031-1067)
  throwsLike(() => kernel.validateDescriptor(descriptor({})), Error,
             "encoder-layer-ff-expand is not a fixed production GEMM signature: M=7520, K=1024, N=4096, " +
             "activation=none, bias=false, residualScale=none");
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu", residualScale: 0.5 })), Error,
             "supplies a residual scale without a residual");
  // requireRuntimeWeight (gemm.ts:1069-1161)
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu",
      mutate: (d) => { d.bPalette.sourceRecord = Object.assign({}, d.bPalette.sourceRecord, { dtype: "float32" }); } })),
      Error, "has invalid transient palette weights");
  throwsLike(() => kernel.validateDescriptor(descriptor({ activation: "silu", mutate: (d) => { d.paletteGroupColumns = 1024; } })),
      Error, "has invalid transient palette weights");
  // arena.ts slice rules
  throwsLike(() => arena.slice("x", 100, 64), RangeError, "Invalid activation slice x");
  // the counters of a fused kernel: nothing is ever expanded
  const backend = host.createEncoderGemmBackend(kernel);
  assert.strictEqual(backend.transientPaletteDispatchCount, 0);
  assert.strictEqual(backend.transientPaletteExpandedBytes, 0);
  // synthetic shapes are accepted when asked for
  return host.F16GemmKernel.create({}, arena, undefined, { allowSyntheticShapes: true }).then((synthetic) => {
    synthetic.validateDescriptor(descriptor({ rows: 300, inner: 1024, columns: 512, bits: 6 }));
    console.log("host_cpu ok");
  });
}).catch((e) => { console.error(e); process.exit(1); });

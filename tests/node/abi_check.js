"use strict";
// No-GPU checks of the Node-API addon: it loads, exports every entry point,
// turns libafhip's statuses into the reference's exception types, and the
// operators' run() returns a Promise that rejects on invalid input before
// any device work, as the reference's async run() does.
var assert = require("assert");
var fs = require("fs");
var path = require("path");
var afhip = require("../../alphafold2-webgpu_amd/napi/index.js");
var createDeterministicTriangleInput = require("./deterministic.js").createDeterministicTriangleInput;

async function rejects(promise, pattern, kind) {
  assert.ok(promise instanceof Promise, "run() returns a Promise");
  var caught = null;
  try { await promise; } catch (err) { caught = err; }
  assert.ok(caught !== null, "expected a rejection matching " + pattern);
  assert.ok(caught instanceof (kind || RangeError), String(caught));
  assert.ok(pattern.test(caught.message), caught.message);
}

async function main() {
  var native = afhip.addon();
  var expected = ["open", "close", "abiVersion", "deviceReport", "bufferCreate", "bufferDestroy", "bufferWrite",
    "bufferRead", "synchronize", "gemmGrid", "gemmSelect", "gemmCalibrate", "gemmForceVariant", "calibrationLoad",
    "calibrationSave", "gemmPlanCreate", "gemmPlanDestroy", "gemmWorkspaceSize", "gemmRun", "triangleRun", "opmRun",
    "transitionRun", "attentionRun", "timingEnable", "timingReset", "timingReport", "packWeightQ8Block",
    "executionCreate", "executionDestroy", "executionAllocate", "executionUpload", "executionRelease",
    "executionCheckpoint", "executionReleaseSince", "executionNoteSubmitted", "executionSnapshot",
    "executionAddInPlace", "executionPrepareWeights", "executionPairStack", "executionEvoformerBlock",
    "setMemoryBudget", "memoryResident", "calibrationClear", "calibrationInject"];
  expected.forEach(function (n) { assert.strictEqual(typeof native[n], "function", n); });
  assert.strictEqual(native.abiVersion(), 3);

  // gemmGrid known answers (test/gemm-selection.test.ts:239-262, test/gemm.test.ts:37-61).
  assert.deepStrictEqual(afhip.gemmGrid(65536 * 64, 128), [2, 65535]);
  assert.deepStrictEqual(afhip.gemmGrid(100, 300), [3, 2]);
  assert.deepStrictEqual(afhip.gemmGrid(100, 300, 64, 128), [5, 1]);
  assert.throws(function () { afhip.gemmGrid(0, 4); }, RangeError);

  // Selection without a device: f16 operands take the LDS_DMA family, also
  // with a row-contiguous source (the reference's sourceContiguous "row");
  // f32 operands the register-staged one.
  var desc = { rows: 384, inner: 384, columns: 384, batch: 128, precision: 1, aDtype: 1, wDtype: 1, wLayout: 1,
    outDtype: 1 };
  var v = afhip.gemmSelect(desc);
  assert.strictEqual(v.kernel, afhip.KERNEL.lds_dma);
  assert.strictEqual(v.tileRows, 192);
  assert.strictEqual(afhip.gemmSelect(Object.assign({ aLayout: afhip.SOURCE.row }, desc)).kernel,
    afhip.KERNEL.lds_dma);
  assert.strictEqual(afhip.gemmSelect(Object.assign({}, desc, { aLayout: afhip.SOURCE.row, precision: 0, aDtype: 0,
    wDtype: 0, outDtype: 0 })).kernel, afhip.KERNEL.register);
  // An f32 source under f16 precision: LDS_DMA when K is a multiple of 8.
  assert.strictEqual(afhip.gemmSelect(Object.assign({}, desc, { aDtype: 0 })).kernel, afhip.KERNEL.lds_dma);
  assert.strictEqual(afhip.gemmSelect(Object.assign({}, desc, { aDtype: 0, inner: 388 })).kernel,
    afhip.KERNEL.register);

  // Input validation rejects the run's promise before any device work
  // (RangeError, src/triangle/types.ts:42-52, attention.ts:102-141).
  var attInput = { activations: new Float32Array(3 * 4 * 8), mask: new Float32Array(12), batch: 3, queryLength: 4,
    channels: 8, heads: 3, weights: {} };
  await rejects(new afhip.AttentionGpu().run(attInput), /integral head dimension no larger than 32/);
  attInput.heads = 2;
  attInput.mask = new Float32Array(11);
  await rejects(new afhip.AttentionGpu().run(attInput), /mask has 11 values; expected 12/);
  var bad = { shape: { length: 2, cZ: 3, cHidden: 4 }, z: new Float32Array(5), mask: new Float32Array(4),
    weights: {} };
  await rejects(new afhip.TriangleMultiplicationOutgoingGpu().run(bad), /z has 5 values/);
  // The reference's TriangleShape is an object: a tuple's `length` is its
  // array length and it has no cZ, so it is refused as the reference refuses
  // it (const { length, cZ, cHidden } = input.shape, types.ts:55).
  await rejects(new afhip.TriangleMultiplicationOutgoingGpu().run({ shape: [2, 3, 4] }),
    /cZ must be a positive safe integer; received undefined/);
  assert.throws(function () { afhip.validateTriangleInput({ shape: { length: 0, cZ: 3, cHidden: 4 } }); },
    RangeError);
  // The reference's wholeStorage option: an unknown value is refused before
  // any device work; one the backend does not apply is reported once as a
  // Node warning (the run itself then needs the device).
  var valid = createDeterministicTriangleInput({ length: 4, cZ: 8, cHidden: 4 }, 3);
  await rejects(new afhip.TriangleMultiplicationOutgoingGpu().run(valid, { wholeStorage: "f64" }),
    /unknown wholeStorage f64/);
  var warnings = [];
  process.on("warning", function (w) { if (w.code === "AFHIP_OPTION") warnings.push(w.message); });
  try { await new afhip.TriangleMultiplicationOutgoingGpu().run(valid, { wholeStorage: "f16" }); } catch (e) { /* no device */ }
  try { await new afhip.TriangleMultiplicationOutgoingGpu().run(valid, { wholeStorage: "f16" }); } catch (e) { /* no device */ }
  await new Promise(function (resolve) { setImmediate(resolve); });
  assert.strictEqual(warnings.length, 1, JSON.stringify(warnings));
  assert.ok(/wholeStorage "f16" has no effect/.test(warnings[0]), warnings[0]);
  await rejects(new afhip.OuterProductMeanGpu().run({ sequences: 2, length: 0, cM: 4, cOuter: 2, cZ: 3 }),
    /outer product mean dimensions must be positive safe integers/);
  await rejects(new afhip.OuterProductMeanGpu().run({ sequences: 2, length: 3, cM: 4, cOuter: 2, cZ: 3,
    activations: new Float32Array(24), mask: new Float32Array(5), weights: {} }), /mask has 5 values; expected 6/);
  await rejects(new afhip.TransitionGpu().run({ rows: 4, channels: 2, hiddenChannels: 1.5 }),
    /transition dimensions must be positive safe integers/);

  // packWeightQ8Block refuses a block past the C ABI's int32 before any
  // lookup or cast, and checks its handles before any device work.
  assert.throws(function () {
    afhip.packWeightQ8Block(1, 2, Math.pow(2, 31), 0, 4, 4, 3, afhip.DTYPE.f16);
  }, /invalid block/);
  assert.throws(function () { afhip.packWeightQ8Block(999999, 999998, 64, 0, 4, 4, 999997, afhip.DTYPE.f16); },
    /unknown buffer handle/);

  // Execution handles are checked before any device work.
  assert.throws(function () { native.executionSnapshot(424242); }, /unknown execution handle/);

  // errorMetrics (test/cpu-reference.test.ts:36-42).
  var m = afhip.errorMetrics(new Float32Array([1, 3]), new Float32Array([2, 1]));
  assert.deepStrictEqual(m, { meanAbsoluteError: 1.5, maxAbsoluteError: 2, rootMeanSquareError: Math.sqrt(2.5) });

  // The Node tests' createDeterministicTriangleInput against the vectors the
  // reference's own source wrote (tests/golden/generators.json).
  var g = JSON.parse(fs.readFileSync(path.join(__dirname, "..", "golden", "generators.json"), "utf8"));
  g.createDeterministicTriangleInput.forEach(function (c) {
    var inp = createDeterministicTriangleInput(c.shape, c.seed);
    assert.deepStrictEqual(Array.from(inp.z), c.z);
    assert.deepStrictEqual(Array.from(inp.mask), c.mask);
    Object.keys(c.weights).forEach(function (k) { assert.deepStrictEqual(Array.from(inp.weights[k]), c.weights[k], k); });
  });
  var d = g.createDeterministicTriangleInputDefaultSeed;
  assert.deepStrictEqual(Array.from(createDeterministicTriangleInput(d.shape).z), d.z);

  console.log(JSON.stringify({ ok: true, exports: expected.length, node: process.versions.node }));
}

main().catch(function (err) { console.error(err); process.exit(1); });

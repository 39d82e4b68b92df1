"use strict";
// No-GPU checks of the Node-API addon: it loads, exports every entry point,
// and turns libafhip's statuses into the reference's exception types.
var assert = require("assert");
var afhip = require("../../alphafold2-webgpu_amd/napi/index.js");

var native = afhip.addon();
var expected = ["open", "close", "abiVersion", "deviceReport", "bufferCreate", "bufferDestroy", "bufferWrite",
  "bufferRead", "synchronize", "gemmGrid", "gemmSelect", "gemmCalibrate", "gemmForceVariant", "calibrationLoad",
  "calibrationSave", "gemmPlanCreate", "gemmPlanDestroy", "gemmWorkspaceSize", "gemmRun", "triangleRun", "opmRun",
  "transitionRun", "attentionRun", "timingEnable", "timingReset", "timingReport", "packWeightQ8Block", "executionCreate",
  "executionDestroy", "executionAllocate", "executionUpload", "executionRelease", "executionCheckpoint",
  "executionReleaseSince", "executionNoteSubmitted", "executionSnapshot", "executionAddInPlace",
  "executionPrepareWeights", "executionPairStack", "executionEvoformerBlock", "setMemoryBudget", "memoryResident"];
expected.forEach(function (n) { assert.strictEqual(typeof native[n], "function", n); });
assert.strictEqual(native.abiVersion(), 3);

// gemmGrid known answers (test/gemm-selection.test.ts:239-262, test/gemm.test.ts:37-61).
assert.deepStrictEqual(afhip.gemmGrid(65536 * 64, 128), [2, 65535]);
assert.deepStrictEqual(afhip.gemmGrid(100, 300), [3, 2]);
assert.deepStrictEqual(afhip.gemmGrid(100, 300, 64, 128), [5, 1]);
assert.throws(function () { afhip.gemmGrid(0, 4); }, RangeError);

// Selection without a device: f16 operands take the LDS_DMA family.
var v = afhip.gemmSelect({ rows: 384, inner: 384, columns: 384, batch: 128, precision: 1, aDtype: 1, wDtype: 1,
  wLayout: 1, outDtype: 1 });
assert.strictEqual(v.kernel, afhip.KERNEL.lds_dma);
assert.strictEqual(v.tileRows, 192);

// Input validation happens before any device work (RangeError, types.ts:42-52).
var attInput = { activations: new Float32Array(3 * 4 * 8), mask: new Float32Array(12), batch: 3, queryLength: 4,
  channels: 8, heads: 3, weights: {} };
assert.throws(function () { new afhip.AttentionGpu().run(attInput); }, /integral head dimension no larger than 32/);
attInput.heads = 2;
attInput.mask = new Float32Array(11);
assert.throws(function () { new afhip.AttentionGpu().run(attInput); }, /mask has 11 values; expected 12/);
var bad = { shape: [2, 3, 4], z: new Float32Array(5), mask: new Float32Array(4), weights: {} };
assert.throws(function () { new afhip.TriangleMultiplicationOutgoingGpu().run(bad); }, /z has 5 values/);
assert.throws(function () { afhip.validateTriangleInput({ shape: [0, 3, 4] }); }, RangeError);

// packWeightQ8Block checks its handles before any device work.
assert.throws(function () { afhip.packWeightQ8Block(999999, 999998, 64, 0, 4, 4, 999997, afhip.DTYPE.f16); },
  /unknown buffer handle/);

// Execution handles are checked before any device work.
assert.throws(function () { native.executionSnapshot(424242); }, /unknown execution handle/);

// errorMetrics (test/cpu-reference.test.ts:36-42).
var m = afhip.errorMetrics(new Float32Array([1, 3]), new Float32Array([2, 1]));
assert.deepStrictEqual(m, { meanAbsoluteError: 1.5, maxAbsoluteError: 2, rootMeanSquareError: Math.sqrt(2.5) });
console.log(JSON.stringify({ ok: true, exports: expected.length, node: process.versions.node }));

"use strict";
// The TypeScript host's view of afhip.node: classes with the reference's
// operator signatures, so a caller swaps the class and nothing else.
//
//   TriangleMultiplication{Outgoing,Incoming}Gpu(device).run(input, options)
//     src/triangle/webgpu.ts:9-23, :56-214
//   OuterProductMeanGpu(device).run(input, options)
//     src/evoformer/outer-product-mean.ts:21-40, :549-646
//   TransitionGpu(device).run(input, options)
//     src/evoformer/transition.ts:18-31, :264-361
//   AttentionGpu(device).run(input, options)
//     src/evoformer/attention.ts:19-58, :102-201, :1321-1452
//   gemmGrid, the GEMM variant selection and its persisted calibration
//     src/runtime/gemm.ts:213-228, :368-379; src/runtime/gemm-selection.ts:122-125, :560-660
//
// Inputs are the reference's own objects (TriangleMultiplicationInput with
// its TriangleShape {length, cZ, cHidden}, OuterProductMeanInput and
// TransitionInput with their flat dimension fields, AttentionInput); run()
// returns a Promise of {output: Float32Array, elapsedMilliseconds, memory},
// memory being the operator allocator's AllocationSnapshot.
// The loader follows src/runtime/wgpu/backend.ts:80-99: require the addon
// lazily and say how to build it when it is missing.
//
// Written for any Node with Node-API 8 (no ?? or ?. syntax).

var path = require("path");

var native = null;
function addon() {
  if (native) return native;
  var file = path.join(__dirname, "afhip.node");
  try {
    native = require(file);
  } catch (err) {
    var e = new Error("afhip.node is not built (" + file + "): run `make -C alphafold2-webgpu_amd napi`; " +
      "there is no fallback (" + err.message + ")");
    e.cause = err;
    throw e;
  }
  return native;
}

var F32 = 0, F16 = 1, I8 = 2;
var PRECISION = { f32: 0, f16: 1 };
var KERNEL = { register: 0, lds_dma: 1, stream: 2 };
var SOURCE = { k: 0, row: 1 };
var OUTPUT = { row: 0, column: 1 };
var EPILOGUE = { scale: 1, bias: 2, attention: 4, relu: 8, residual: 16 };

var opened = false;
function requestHipDevice(ordinal) {
  // The counterpart of requestAlphaFoldDevice (src/runtime/device.ts:375-467):
  // one context per process.
  if (!opened) {
    addon().open(ordinal === undefined ? 0 : ordinal);
    opened = true;
  }
  return { report: JSON.parse(addon().deviceReport()) };
}

function positiveInteger(name, value) {
  if (typeof value !== "number" || !Number.isSafeInteger(value) || value <= 0) {
    throw new RangeError(name + " must be a positive safe integer; received " + value);
  }
}

function expectLength(name, value, length) {
  if (!value || value.length !== length) {
    throw new RangeError(name + " has " + (value ? value.length : 0) + " values; expected " + length);
  }
}

var TRIANGLE_ORDER = [
  "layerNormInWeight", "layerNormInBias",
  "linearAPWeight", "linearAPBias", "linearAGWeight", "linearAGBias",
  "linearBPWeight", "linearBPBias", "linearBGWeight", "linearBGBias",
  "layerNormOutWeight", "layerNormOutBias",
  "linearZWeight", "linearZBias", "linearGWeight", "linearGBias",
];

function triangleWeightSizes(cZ, cHidden) {
  return {
    layerNormInWeight: cZ, layerNormInBias: cZ,
    linearAPWeight: cHidden * cZ, linearAPBias: cHidden, linearAGWeight: cHidden * cZ, linearAGBias: cHidden,
    linearBPWeight: cHidden * cZ, linearBPBias: cHidden, linearBGWeight: cHidden * cZ, linearBGBias: cHidden,
    layerNormOutWeight: cHidden, layerNormOutBias: cHidden,
    linearZWeight: cZ * cHidden, linearZBias: cZ, linearGWeight: cZ * cZ, linearGBias: cZ,
  };
}

// validateTriangleInput (src/triangle/types.ts:54-89): the reference's
// TriangleShape {length, cZ, cHidden} and its checks and messages.
function validateTriangleInput(input) {
  var shape = input.shape || {};
  var length = shape.length, cZ = shape.cZ, cHidden = shape.cHidden;
  positiveInteger("length", length);
  positiveInteger("cZ", cZ);
  positiveInteger("cHidden", cHidden);
  var pairs = length * length;
  if (!Number.isSafeInteger(pairs * Math.max(cZ, cHidden))) {
    throw new RangeError("tensor dimensions exceed JavaScript's safe integer range");
  }
  expectLength("z", input.z, pairs * cZ);
  expectLength("mask", input.mask, pairs);
  var sizes = triangleWeightSizes(cZ, cHidden);
  TRIANGLE_ORDER.forEach(function (name) { expectLength(name, input.weights[name], sizes[name]); });
  if (input.epsilon !== undefined && (!(input.epsilon > 0) || !isFinite(input.epsilon))) {
    throw new RangeError("epsilon must be finite and positive; received " + input.epsilon);
  }
}

// packWeights (src/triangle/weights.ts:20-34): f32, ORDER, [out][in].
function packTriangleWeights(weights) {
  var total = 0;
  TRIANGLE_ORDER.forEach(function (n) { total += weights[n].length; });
  var out = new Float32Array(total);
  var at = 0;
  TRIANGLE_ORDER.forEach(function (n) { out.set(weights[n], at); at += weights[n].length; });
  return out;
}

function packOrdered(weights, order) {
  var total = 0;
  order.forEach(function (n) { total += weights[n].length; });
  var out = new Float32Array(total);
  var at = 0;
  order.forEach(function (n) { out.set(weights[n], at); at += weights[n].length; });
  return out;
}

function precisionOf(options, fallback) {
  var precision = options && options.precision !== undefined ? options.precision : fallback;
  if (!(precision in PRECISION)) throw new RangeError("unknown precision " + precision);
  return precision;
}

// Every operator object owns one execution: its allocator
// (GpuBufferAllocator, src/runtime/allocator.ts:168-388, one per operator as
// the reference's constructors make one) pools device buffers across runs,
// and `memory` in a result is that allocator's AllocationSnapshot
// (allocator.ts:8-29), taken while the run's tensors are still live.
function Operator(device, options) {
  this.device = device;
  this.options = options || {};
}
Operator.prototype._execution = function () {
  if (this._handle === undefined) {
    requestHipDevice();
    this._handle = addon().executionCreate(0);
  }
  return this._handle;
};
// Starts fn, which validates, copies the host arrays and queues the device
// work (runs of one operator take its execution's lock in turn on the
// worker threads). A synchronous throw in fn (validation) rejects the
// promise, as a throw inside the reference's async run() does.
Operator.prototype._queue = function (fn) {
  var started;
  try {
    started = fn();
  } catch (err) {
    return Promise.reject(err);
  }
  return started.then(function (r) {
    return { output: r.output, elapsedMilliseconds: r.elapsedMilliseconds, memory: JSON.parse(r.memoryJson) };
  });
};
// Frees the operator's pooled device memory (the allocator's destroy).
Operator.prototype.release = function () {
  if (this._handle !== undefined) {
    addon().executionDestroy(this._handle);
    this._handle = undefined;
  }
};

// Options of the reference that this backend takes with another meaning are
// reported once per process as a Node warning (code AFHIP_OPTION), so a
// caller switching backends learns of them without its runs failing.
var warned = {};
function warnOnce(key, message) {
  if (warned[key]) return;
  warned[key] = true;
  process.emitWarning(message, { code: "AFHIP_OPTION" });
}

// The triangle options with no exact counterpart (src/triangle/webgpu.ts:9-15):
// wholeStorage picks the reference's storage of the whole projection; here
// the a/b operands are always stored in the precision's dtype. precision
// "f16" is the reference's f16 weights over an f32 pair; here f16 MFMA
// operands with f32 accumulation.
function triangleOptionNotes(options, precision) {
  if (options.wholeStorage !== undefined) {
    if (options.wholeStorage !== "f32" && options.wholeStorage !== "f16") {
      throw new RangeError("unknown wholeStorage " + options.wholeStorage);
    }
    if (options.wholeStorage !== precision) {
      warnOnce("wholeStorage", "wholeStorage \"" + options.wholeStorage + "\" has no effect on the HIP backend: " +
        "the triangle operands are stored as " + precision + ", the precision's dtype");
    }
  }
  if (precision === "f16") {
    warnOnce("precision-f16", "precision \"f16\" on the HIP backend runs f16 MFMA operands (weights, normalised " +
      "activations and the a/b projections) with f32 accumulation, where the WebGPU backend keeps an f32 pair " +
      "with f16 weights");
  }
}

// TriangleMultiplication{Outgoing,Incoming}Gpu (src/triangle/webgpu.ts:42-214).
// run(input: TriangleMultiplicationInput, {precision, blockRows, wholeStorage})
// -> Promise<{output, elapsedMilliseconds, memory}>.
function TriangleMultiplicationGpu(device, direction) {
  Operator.call(this, device);
  this.direction = direction;
}
TriangleMultiplicationGpu.prototype = Object.create(Operator.prototype);
TriangleMultiplicationGpu.prototype.run = function (input, options) {
  var self = this;
  return this._queue(function () {
    options = options || {};
    validateTriangleInput(input);
    var precision = precisionOf(options, "f32");
    if (options.blockRows !== undefined) positiveInteger("blockRows", options.blockRows);
    triangleOptionNotes(options, precision);
    return addon().triangleRun(self._execution(), {
      length: input.shape.length, cZ: input.shape.cZ, cHidden: input.shape.cHidden,
      direction: self.direction === "incoming" ? 1 : 0,
      precision: PRECISION[precision],
      blockRows: options.blockRows === undefined ? 0 : options.blockRows,
      epsilon: input.epsilon === undefined ? 1e-5 : input.epsilon,
    }, input.z, input.mask, packTriangleWeights(input.weights));
  });
};

function TriangleMultiplicationOutgoingGpu(device) { TriangleMultiplicationGpu.call(this, device, "outgoing"); }
TriangleMultiplicationOutgoingGpu.prototype = Object.create(TriangleMultiplicationGpu.prototype);
function TriangleMultiplicationIncomingGpu(device) { TriangleMultiplicationGpu.call(this, device, "incoming"); }
TriangleMultiplicationIncomingGpu.prototype = Object.create(TriangleMultiplicationGpu.prototype);

var OPM_ORDER = ["layerNormScale", "layerNormOffset", "leftWeight", "leftBias", "rightWeight", "rightBias",
  "outputWeight", "outputBias"];

// validate (src/evoformer/outer-product-mean.ts:45-64).
function validateOuterProductMeanInput(input) {
  var dims = [input.sequences, input.length, input.cM, input.cOuter, input.cZ];
  if (!dims.every(function (v) { return Number.isSafeInteger(v) && v > 0; })) {
    throw new RangeError("outer product mean dimensions must be positive safe integers");
  }
  var w = input.weights;
  var S = input.sequences, L = input.length, cM = input.cM, co = input.cOuter, cZ = input.cZ;
  [["activations", input.activations, S * L * cM], ["mask", input.mask, S * L],
    ["layerNormScale", w.layerNormScale, cM], ["layerNormOffset", w.layerNormOffset, cM],
    ["leftWeight", w.leftWeight, cM * co], ["leftBias", w.leftBias, co],
    ["rightWeight", w.rightWeight, cM * co], ["rightBias", w.rightBias, co],
    ["outputWeight", w.outputWeight, co * co * cZ], ["outputBias", w.outputBias, cZ]].forEach(function (e) {
    expectLength(e[0], e[1], e[2]);
  });
  if (input.rowBlockResidues !== undefined) positiveInteger("rowBlockResidues", input.rowBlockResidues);
}

// OuterProductMeanGpu (src/evoformer/outer-product-mean.ts:538-646).
// run(input: OuterProductMeanInput) with the reference's flat fields
// (sequences, length, cM, cOuter, cZ, rowBlockResidues, layerNormEpsilon,
// normalizationEpsilon; :21-34). Precision: options.precision of the
// constructor or of run (an addition; "f32" by default).
function OuterProductMeanGpu(device, options) { Operator.call(this, device, options); }
OuterProductMeanGpu.prototype = Object.create(Operator.prototype);
OuterProductMeanGpu.prototype.run = function (input, options) {
  var self = this;
  return this._queue(function () {
    validateOuterProductMeanInput(input);
    var precision = precisionOf(options, precisionOf(self.options, "f32"));
    return addon().opmRun(self._execution(), {
      sequences: input.sequences, length: input.length, cM: input.cM, cOuter: input.cOuter, cZ: input.cZ,
      precision: PRECISION[precision],
      rowBlockResidues: input.rowBlockResidues === undefined ? 0 : input.rowBlockResidues,
      layerNormEpsilon: input.layerNormEpsilon === undefined ? 1e-5 : input.layerNormEpsilon,
      normalizationEpsilon: input.normalizationEpsilon === undefined ? 1e-3 : input.normalizationEpsilon,
    }, input.activations, input.mask, packOrdered(input.weights, OPM_ORDER));
  });
};

var TRANSITION_ORDER = ["layerNormScale", "layerNormOffset", "firstWeight", "firstBias", "secondWeight",
  "secondBias"];

// validate (src/evoformer/transition.ts:140-157).
function validateTransitionInput(input) {
  var rows = input.rows, channels = input.channels, hidden = input.hiddenChannels;
  if (![rows, channels, hidden].every(function (v) { return Number.isSafeInteger(v) && v > 0; })) {
    throw new RangeError("transition dimensions must be positive safe integers");
  }
  var w = input.weights;
  [["activations", input.activations, rows * channels], ["layerNormScale", w.layerNormScale, channels],
    ["layerNormOffset", w.layerNormOffset, channels], ["firstWeight", w.firstWeight, channels * hidden],
    ["firstBias", w.firstBias, hidden], ["secondWeight", w.secondWeight, hidden * channels],
    ["secondBias", w.secondBias, channels]].forEach(function (e) { expectLength(e[0], e[1], e[2]); });
}

// TransitionGpu (src/evoformer/transition.ts:247-361). run(input:
// TransitionInput) with {rows, channels, hiddenChannels, epsilon}
// (:18-25).
function TransitionGpu(device, options) { Operator.call(this, device, options); }
TransitionGpu.prototype = Object.create(Operator.prototype);
TransitionGpu.prototype.run = function (input, options) {
  var self = this;
  return this._queue(function () {
    validateTransitionInput(input);
    var precision = precisionOf(options, precisionOf(self.options, "f32"));
    return addon().transitionRun(self._execution(), {
      rows: input.rows, channels: input.channels, hidden: input.hiddenChannels, precision: PRECISION[precision],
      epsilon: input.epsilon === undefined ? 1e-5 : input.epsilon,
    }, input.activations, packOrdered(input.weights, TRANSITION_ORDER));
  });
};

var ATTENTION_ORDER = ["queryNormScale", "queryNormOffset", "queryWeight", "keyWeight", "valueWeight",
  "gatingWeight", "gatingBias", "outputWeight", "outputBias"];
var PAIR_BIAS = { "normalized-input": 1, separate: 2 };

// packAttentionWeights (src/evoformer/attention.ts:179-201): the nine
// tensors, then a separate bias's LayerNorm scale, offset and projection, or
// a normalized-input bias's projection.
function packAttentionWeights(weights, pairBias) {
  var parts = ATTENTION_ORDER.map(function (n) { return weights[n]; });
  if (pairBias !== undefined && pairBias !== null) {
    if (pairBias.source === "separate") {
      parts.push(pairBias.layerNormScale, pairBias.layerNormOffset, pairBias.projectionWeight);
    } else {
      parts.push(pairBias.projectionWeight);
    }
  }
  var total = 0;
  parts.forEach(function (t) { total += t.length; });
  var out = new Float32Array(total);
  var at = 0;
  parts.forEach(function (t) { out.set(t, at); at += t.length; });
  return out;
}

function expectCount(name, value, size) {
  if (value.length !== size) throw new RangeError(name + " has " + value.length + " values; expected " + size);
}

// AttentionGpu (src/evoformer/attention.ts:1321-1452), with validate's
// checks and messages (:102-141). run(input: AttentionInput).
function AttentionGpu(device, options) { Operator.call(this, device, options); }
AttentionGpu.prototype = Object.create(Operator.prototype);
AttentionGpu.prototype.run = function (input, options) {
  var self = this;
  return this._queue(function () {
    var b = input.batch, q = input.queryLength, c = input.channels, h = input.heads;
    [b, q, c, h].forEach(function (v) {
      if (!Number.isSafeInteger(v) || v <= 0) throw new RangeError("attention dimensions must be positive safe integers");
    });
    if (c % h !== 0 || c / h > 32) {
      throw new RangeError("the fused WebGPU attention path requires an integral head dimension no larger than 32");
    }
    var w = input.weights;
    expectCount("activations", input.activations, b * q * c);
    expectCount("mask", input.mask, b * q);
    expectCount("queryNormScale", w.queryNormScale, c);
    expectCount("queryNormOffset", w.queryNormOffset, c);
    ["queryWeight", "keyWeight", "valueWeight", "gatingWeight"].forEach(function (n) { expectCount(n, w[n], c * c); });
    expectCount("gatingBias", w.gatingBias, c);
    expectCount("outputWeight", w.outputWeight, c * c);
    expectCount("outputBias", w.outputBias, c);
    var pair = input.pairBias;
    var pairChannels = 0;
    if (pair !== undefined && pair !== null && pair.source === "separate") {
      pairChannels = pair.channels;
      expectCount("pair activations", pair.activations, q * q * pairChannels);
      expectCount("pair norm scale", pair.layerNormScale, pairChannels);
      expectCount("pair norm offset", pair.layerNormOffset, pairChannels);
      expectCount("pair projection", pair.projectionWeight, pairChannels * h);
    } else if (pair !== undefined && pair !== null && pair.projectionWeight.length !== c * h) {
      throw new RangeError("normalized-input pair projection has an invalid size");
    }
    var precision = precisionOf(options, precisionOf(self.options, "f32"));
    return addon().attentionRun(self._execution(), {
      batch: b, queries: q, channels: c, heads: h, transpose: input.transpose === true ? 1 : 0,
      pairBias: pair === undefined || pair === null ? 0 : PAIR_BIAS[pair.source], pairChannels: pairChannels,
      precision: PRECISION[precision], epsilon: input.epsilon === undefined ? 1e-5 : input.epsilon,
    }, input.activations, input.mask, pairChannels > 0 ? pair.activations : null, packAttentionWeights(w, pair));
  });
};

// gemmGrid (src/runtime/gemm.ts:368-379).
// The execution layer (src/runtime/execution.ts:153-555, allocator.ts:168-388):
// device tensors as buffer handles drawn from a pool that outlives each
// call, and the pair steps of an Evoformer block chained on the device
// (src/evoformer/block.ts:1683-1750). Buffer handles work with gemmRun and
// packWeightQ8Block as well.
function HipExecution(options) {
  requestHipDevice();
  this.handle = addon().executionCreate((options && options.maxPooledBytes) || 0);
}
HipExecution.prototype.upload = function (label, data) { return addon().executionUpload(this.handle, label, data); };
HipExecution.prototype.allocate = function (label, bytes) {
  return addon().executionAllocate(this.handle, label, bytes);
};
HipExecution.prototype.read = function (buffer, target) { addon().synchronize(); addon().bufferRead(buffer, 0, target); return target; };
HipExecution.prototype.releaseTensor = function (buffer) { addon().executionRelease(this.handle, buffer); };
HipExecution.prototype.checkpoint = function () { return addon().executionCheckpoint(this.handle); };
HipExecution.prototype.releaseSince = function (mark) { addon().executionReleaseSince(this.handle, mark); };
HipExecution.prototype.noteSubmitted = function () { addon().executionNoteSubmitted(this.handle); };
HipExecution.prototype.snapshot = function () { return JSON.parse(addon().executionSnapshot(this.handle)); };
HipExecution.prototype.addInPlace = function (base, update, elements, baseDtype, updateDtype) {
  addon().executionAddInPlace(this.handle, base, baseDtype === undefined ? F32 : baseDtype, update,
    updateDtype === undefined ? F32 : updateDtype, elements);
};
// shape: {length, sequences, cM, cZ, cOuter, cHidden, transitionFactor,
// precision, pairDtype, msaDtype, attentionHeads}; weights:
// {outerProductMean, triangleMultiplicationOutgoing,
// triangleMultiplicationIncoming, triangleAttentionStarting,
// triangleAttentionEnding, pairTransition}, each the operator's weight
// object, the attentions as the block's {attention, pairProjectionWeight}
// (src/evoformer/block.ts:1727-1745); a missing one skips that step.
// Returns the prepared weight buffers.
HipExecution.prototype.preparePairStack = function (shape, weights) {
  var native = addon(), h = this.handle, out = {};
  if (weights.outerProductMean) {
    out.outerProductMean = native.executionPrepareWeights(h, "outerProductMean", shape,
      packOrdered(weights.outerProductMean, OPM_ORDER));
  }
  if (weights.triangleMultiplicationOutgoing) {
    out.triangleOutgoing = native.executionPrepareWeights(h, "triangleOutgoing", shape,
      packTriangleWeights(weights.triangleMultiplicationOutgoing));
  }
  if (weights.triangleMultiplicationIncoming) {
    out.triangleIncoming = native.executionPrepareWeights(h, "triangleIncoming", shape,
      packTriangleWeights(weights.triangleMultiplicationIncoming));
  }
  ["triangleAttentionStarting", "triangleAttentionEnding"].forEach(function (kind) {
    var a = weights[kind];
    if (a) {
      out[kind] = native.executionPrepareWeights(h, kind, shape, packAttentionWeights(a.attention,
        { source: "normalized-input", projectionWeight: a.pairProjectionWeight }));
    }
  });
  if (weights.pairTransition) {
    out.pairTransition = native.executionPrepareWeights(h, "pairTransition", shape,
      packOrdered(weights.pairTransition, TRANSITION_ORDER));
  }
  return out;
};
// The whole block (src/evoformer/block.ts:1673-1759). shape: the pair
// stack's plus {msaHeads, msaTransitionFactor, opmFirst}; weights: the pair
// stack's plus {msaRowAttention: {attention, pairLayerNormScale,
// pairLayerNormOffset, pairProjectionWeight}, msaColumnAttention:
// {attention}, msaTransition} (block.ts:86-88).
HipExecution.prototype.prepareEvoformerBlock = function (shape, weights) {
  var native = addon(), h = this.handle, out = this.preparePairStack(shape, weights);
  var row = weights.msaRowAttention;
  if (row) {
    out.msaRowAttention = native.executionPrepareWeights(h, "msaRowAttention", shape, packAttentionWeights(
      row.attention, { source: "separate", layerNormScale: row.pairLayerNormScale,
        layerNormOffset: row.pairLayerNormOffset, projectionWeight: row.pairProjectionWeight }));
  }
  if (weights.msaColumnAttention) {
    out.msaColumnAttention = native.executionPrepareWeights(h, "msaColumnAttention", shape,
      packAttentionWeights(weights.msaColumnAttention.attention));
  }
  if (weights.msaTransition) {
    out.msaTransition = native.executionPrepareWeights(h, "msaTransition", shape,
      packOrdered(weights.msaTransition, TRANSITION_ORDER));
  }
  return out;
};
HipExecution.prototype.evoformerBlock = function (shape, prepared, msa, msaMask, pair, pairMask) {
  addon().executionEvoformerBlock(this.handle, shape, prepared, msa, msaMask, pair, pairMask);
};
HipExecution.prototype.pairStack = function (shape, prepared, pair, pairMask, msa, msaMask) {
  addon().executionPairStack(this.handle, shape, prepared, pair, pairMask, msa === undefined ? null : msa,
    msaMask === undefined ? null : msaMask);
};
HipExecution.prototype.release = function () {
  if (this.handle !== undefined) { addon().executionDestroy(this.handle); this.handle = undefined; }
};

function gemmGrid(rows, columns, tileColumns, tileRows) {
  return addon().gemmGrid(rows, columns, tileColumns === undefined ? 128 : tileColumns,
    tileRows === undefined ? 64 : tileRows);
}

// errorMetrics (src/triangle/types.ts:91-110).
function errorMetrics(actual, expected) {
  if (actual.length !== expected.length || actual.length === 0) {
    throw new RangeError("error metrics require equally sized, non-empty arrays");
  }
  var sum = 0, max = 0, sq = 0;
  for (var i = 0; i < actual.length; i++) {
    var d = Math.abs(actual[i] - expected[i]);
    sum += d;
    sq += d * d;
    if (d > max) max = d;
  }
  return { meanAbsoluteError: sum / actual.length, maxAbsoluteError: max,
    rootMeanSquareError: Math.sqrt(sq / actual.length) };
}

module.exports = {
  addon: addon,
  requestHipDevice: requestHipDevice,
  TriangleMultiplicationOutgoingGpu: TriangleMultiplicationOutgoingGpu,
  TriangleMultiplicationIncomingGpu: TriangleMultiplicationIncomingGpu,
  OuterProductMeanGpu: OuterProductMeanGpu,
  HipExecution: HipExecution,
  setGpuMemoryBudget: function (bytes) { requestHipDevice(); addon().setMemoryBudget(bytes === undefined ? null : bytes); },
  gpuMemoryResident: function () { return addon().memoryResident(); },
  TransitionGpu: TransitionGpu,
  AttentionGpu: AttentionGpu,
  packAttentionWeights: packAttentionWeights,
  validateTriangleInput: validateTriangleInput,
  validateOuterProductMeanInput: validateOuterProductMeanInput,
  validateTransitionInput: validateTransitionInput,
  packTriangleWeights: packTriangleWeights,
  errorMetrics: errorMetrics,
  gemmGrid: gemmGrid,
  gemmSelect: function (desc) { return addon().gemmSelect(desc); },
  calibrateGemmVariant: function (desc) { requestHipDevice(); return addon().gemmCalibrate(desc); },
  forceGemmVariant: function (variant) { addon().gemmForceVariant(variant === undefined ? null : variant); },
  calibrationLoad: function (file) { addon().calibrationLoad(file); },
  calibrationSave: function (file) { addon().calibrationSave(file); },
  calibrationClear: function () { addon().calibrationClear(); },
  // The bundle's mixed-q8 weight (int8 codes and f16 scale bits, in device
  // buffers) decoded straight into a packed GEMM operand buffer.
  packWeightQ8Block: function (codes, scales, block, start, rowsK, columnsN, dst, dtype) {
    addon().packWeightQ8Block(codes, scales, block, start, rowsK, columnsN, dst, dtype);
  },
  TRIANGLE_ORDER: TRIANGLE_ORDER,
  DTYPE: { f32: F32, f16: F16, i8: I8 },
  PRECISION: PRECISION,
  KERNEL: KERNEL,
  SOURCE: SOURCE,
  OUTPUT: OUTPUT,
  EPILOGUE: EPILOGUE,
};

"use strict";
// GPU parity through the Node-API addon, driven as the reference's own GPU
// tests drive its operators: the reference's input objects, `await run()`,
// the reference's tolerances (test/triangle-multiplication-outgoing.gpu.test.ts:30-91,
// test/evoformer-triangle-incoming.gpu.test.ts:42-106,
// test/outer-product-mean-reference.gpu.test.ts:100-135). The float64/f32
// oracle's answers for the generated cases come from the Python test that
// starts this script, in the directory AFHIP_NODE_EXPECTED.
var assert = require("assert");
var fs = require("fs");
var path = require("path");
var afhip = require("../../alphafold2-webgpu_amd/napi/index.js");
var createDeterministicTriangleInput = require("./deterministic.js").createDeterministicTriangleInput;

var expectedDir = process.env.AFHIP_NODE_EXPECTED;
var report = { node: process.versions.node, cases: [] };

function transposePairs(data, L, C) {
  var out = new Float32Array(data.length);
  for (var i = 0; i < L; i++)
    for (var j = 0; j < L; j++)
      for (var c = 0; c < C; c++) out[(j * L + i) * C + c] = data[(i * L + j) * C + c];
  return out;
}

function readF32(name) {
  var bytes = fs.readFileSync(path.join(expectedDir, name));
  return new Float32Array(bytes.buffer.slice(bytes.byteOffset, bytes.byteOffset + bytes.byteLength));
}

// A triangle fixture as the Python side hands it over: <name>.json lists the
// arrays (name, element count) in the order they are packed into <name>.f32,
// plus the shape and epsilon; the result is the reference's operator input
// and the expected output.
function readTriangleFixture(name) {
  var index = JSON.parse(fs.readFileSync(path.join(expectedDir, name + ".json"), "utf8"));
  var data = readF32(name + ".f32");
  var arrays = {}, at = 0;
  index.arrays.forEach(function (entry) {
    arrays[entry[0]] = data.subarray(at, at + entry[1]);
    at += entry[1];
  });
  assert.strictEqual(at, data.length, name + " holds " + data.length + " values, its index " + at);
  var weights = {};
  index.weights.forEach(function (n) { weights[n] = arrays[n]; });
  return { input: { shape: index.shape, epsilon: index.epsilon, z: arrays.z, mask: arrays.mask, weights: weights },
    expected: arrays.expected };
}

function relativeMax(actual, expected) {
  var worst = 0, largest = 0;
  for (var i = 0; i < expected.length; i++) {
    worst = Math.max(worst, Math.abs(actual[i] - expected[i]));
    largest = Math.max(largest, Math.abs(expected[i]));
  }
  return worst / largest;
}

// The AllocationSnapshot fields (src/runtime/allocator.ts:8-29).
function checkSnapshot(memory, labelPrefix) {
  ["currentBytes", "peakBytes", "residentBytes", "peakResidentBytes", "pooledBytes", "allocationCount",
    "bufferCount"].forEach(function (k) { assert.strictEqual(typeof memory[k], "number", k); });
  assert.ok(Array.isArray(memory.peakComposition) && memory.peakComposition.length > 0);
  memory.peakComposition.forEach(function (share) {
    assert.ok(typeof share.label === "string" && share.bytes > 0 && share.count > 0);
  });
  assert.ok(memory.peakComposition.some(function (s) { return s.label.indexOf(labelPrefix) === 0; }));
  assert.ok(memory.currentBytes > 0 && memory.peakBytes >= memory.currentBytes);
  assert.ok(memory.residentBytes >= memory.currentBytes);
}

async function main() {
  afhip.requestHipDevice(0);

  // The reference's triangle fixtures, with their own TriangleShape objects.
  var fixtures = ["openfold-triangle-small", "alphafold-short-9", "alphafold-single-sequence-59", "alphafold-a3m-59"];
  for (var fi = 0; fi < fixtures.length; fi++) {
    var name = fixtures[fi];
    var b = readTriangleFixture(name);
    var L = b.input.shape.length, C = b.input.shape.cZ;
    var op = new afhip.TriangleMultiplicationOutgoingGpu(null);
    var pending = op.run(b.input, { precision: "f32" });
    assert.ok(pending instanceof Promise);
    var out = await pending;
    var m32 = afhip.errorMetrics(out.output, b.expected);
    assert.ok(m32.meanAbsoluteError < 1e-5 && m32.maxAbsoluteError < 1e-4, name + " f32 " + JSON.stringify(m32));
    assert.ok(out.elapsedMilliseconds > 0);
    checkSnapshot(out.memory, "triangle.");
    // A second run on the same operator reuses its pooled buffers.
    var again = await op.run(b.input, { precision: "f32" });
    assert.deepStrictEqual(Buffer.from(again.output.buffer), Buffer.from(out.output.buffer), name + " rerun");
    assert.ok(again.memory.allocationCount > out.memory.allocationCount);
    var out16 = await new afhip.TriangleMultiplicationOutgoingGpu(null).run(b.input, { precision: "f16" });
    var r16 = relativeMax(out16.output, b.expected);
    assert.ok(r16 <= 1e-2, name + " f16 " + r16);
    var blocked = await op.run(b.input, { precision: "f32", blockRows: 2 });
    assert.deepStrictEqual(Buffer.from(blocked.output.buffer), Buffer.from(out.output.buffer), name + " blocking");
    op.release();
    // incoming(z) = T(outgoing(T(z))): the reference's kjc,kic->ijc (src/triangle/shaders.ts:452-495).
    var t = { shape: b.input.shape, epsilon: b.input.epsilon, weights: b.input.weights,
      z: transposePairs(b.input.z, L, C), mask: transposePairs(b.input.mask, L, 1) };
    var results = await Promise.all([new afhip.TriangleMultiplicationIncomingGpu(null).run(b.input),
      new afhip.TriangleMultiplicationOutgoingGpu(null).run(t)]);
    var mi = afhip.errorMetrics(results[0].output, transposePairs(results[1].output, L, C));
    assert.ok(mi.maxAbsoluteError <= 1e-6, name + " incoming " + JSON.stringify(mi));
    report.cases.push({ fixture: name, f32: m32, f16MaxRelative: r16, incomingVsTransposed: mi });
  }

  // release() right after run(), before the run is awaited: the pending run
  // still resolves (its device memory is freed when it has finished), and
  // the operator's next run makes a new execution.
  await (async function () {
    var first = readTriangleFixture(fixtures[0]);
    var op = new afhip.TriangleMultiplicationOutgoingGpu(null);
    var pending = op.run(first.input);
    op.release();
    var done = await pending;
    var m = afhip.errorMetrics(done.output, first.expected);
    assert.ok(m.maxAbsoluteError < 1e-4, "run resolved after release " + JSON.stringify(m));
    var again = await op.run(first.input);
    assert.deepStrictEqual(Buffer.from(again.output.buffer), Buffer.from(done.output.buffer));
    op.release();
    // Two runs pending on two operators while the context closes: both
    // resolve, and the context closes when the second has finished.
    var ops = [new afhip.TriangleMultiplicationOutgoingGpu(null), new afhip.TriangleMultiplicationOutgoingGpu(null)];
    var runs = ops.map(function (o) { return o.run(first.input); });
    afhip.addon().close();
    var both = await Promise.all(runs);
    both.forEach(function (r) {
      assert.deepStrictEqual(Buffer.from(r.output.buffer), Buffer.from(done.output.buffer));
    });
    afhip.addon().open(0);
    report.cases.push({ releaseWhilePending: m });
  })();

  // createDeterministicTriangleInput, both directions, against the oracle;
  // two runs queued on one operator without awaiting the first.
  var det = JSON.parse(fs.readFileSync(path.join(expectedDir, "deterministic.json"), "utf8"));
  var input = createDeterministicTriangleInput(det.shape, det.seed);
  var directions = { outgoing: new afhip.TriangleMultiplicationOutgoingGpu(null),
    incoming: new afhip.TriangleMultiplicationIncomingGpu(null) };
  var detReport = {};
  for (var dir in directions) {
    var first = directions[dir].run(input), second = directions[dir].run(input, { blockRows: 5 });
    var both = await Promise.all([first, second]);
    var expect = readF32("deterministic_" + dir + ".f32");
    var rd = relativeMax(both[0].output, expect);
    assert.ok(rd <= 1e-5, "deterministic " + dir + " " + rd);
    assert.deepStrictEqual(Buffer.from(both[1].output.buffer), Buffer.from(both[0].output.buffer));
    detReport[dir] = rd;
  }
  report.cases.push({ deterministicInput: detReport });

  // The reference test's outer-product-mean input literal
  // (test/outer-product-mean-reference.gpu.test.ts:81-121) and tolerances.
  await (async function () {
    function spread(count, seed) {
      var values = new Float32Array(count);
      for (var index = 0; index < count; index += 1) values[index] = Math.sin((index + 1) * seed) * 0.7;
      return values;
    }
    var sequences = 9, length = 8, cM = 12, cOuter = 32, cZ = 16;
    var mask = new Float32Array(sequences * length).fill(1);
    for (var index = 0; index < sequences * length; index += 3) mask[index] = 0;
    var weights = {
      layerNormScale: spread(cM, 0.31), layerNormOffset: spread(cM, 0.17),
      leftWeight: spread(cM * cOuter, 0.11), leftBias: spread(cOuter, 0.23),
      rightWeight: spread(cM * cOuter, 0.13), rightBias: spread(cOuter, 0.29),
      outputWeight: spread(cOuter * cOuter * cZ, 0.07), outputBias: spread(cZ, 0.37),
    };
    var opmInput = {
      activations: spread(sequences * length * cM, 0.19), mask: mask,
      sequences: sequences, length: length, cM: cM, cOuter: cOuter, cZ: cZ, weights: weights,
      layerNormEpsilon: 1e-5, normalizationEpsilon: 1e-3, rowBlockResidues: 3,
    };
    var actual = await new afhip.OuterProductMeanGpu(null).run(opmInput);
    var error = afhip.errorMetrics(actual.output, readF32("opm_expected.f32"));
    assert.ok(error.meanAbsoluteError < 2e-5 && error.maxAbsoluteError < 2e-4, "opm " + JSON.stringify(error));
    checkSnapshot(actual.memory, "outer-product-mean.");
    report.cases.push({ outerProductMeanReferenceCase: error });

    // TransitionInput {rows, channels, hiddenChannels} (src/evoformer/transition.ts:18-25).
    var rows = 37, channels = 16, hidden = 64;
    var tInput = { rows: rows, channels: channels, hiddenChannels: hidden, activations: spread(rows * channels, 0.41),
      weights: { layerNormScale: spread(channels, 0.53), layerNormOffset: spread(channels, 0.29),
        firstWeight: spread(channels * hidden, 0.17), firstBias: spread(hidden, 0.23),
        secondWeight: spread(hidden * channels, 0.07), secondBias: spread(channels, 0.31) } };
    var tr = await new afhip.TransitionGpu(null).run(tInput);
    var rt = relativeMax(tr.output, readF32("transition_expected.f32"));
    assert.ok(rt <= 1e-5, "transition " + rt);
    checkSnapshot(tr.memory, "transition.");
    report.cases.push({ transitionMaxRelative: rt });
  })();

  var native = afhip.addon();
// The bundle's mixed-q8 weight through device buffers, as a TypeScript host
// holding the bundle would run it: packWeightQ8Block decodes it straight into
// the packed operand W[n][k] (bit-exact against the decode of
// src/reference/dtype.ts:66-99, value = code * f32(scale)), and an f32 plan
// on that operand matches a double-precision product.
await (async function () {
  var K = 96, N = 80, M = 40, block = 64, start = 37;
  var total = start + K * N + 11;
  var codes = new Int8Array(total), scales = new Uint16Array(Math.ceil(total / block));
  for (var i = 0; i < total; i++) codes[i] = ((i * 37) % 255) - 127;
  for (var j = 0; j < scales.length; j++) scales[j] = 0x2000 + (j * 97) % 0x1000;
  function halfToNumber(bits) {
    var e = (bits >> 10) & 31, m = bits & 1023, s = bits & 0x8000 ? -1 : 1;
    if (e === 0) return s * m * Math.pow(2, -24);
    if (e === 31) return m ? NaN : s * Infinity;
    return s * (1 + m / 1024) * Math.pow(2, e - 15);
  }
  var x = new Float32Array(M * K);
  for (var t = 0; t < x.length; t++) x[t] = Math.sin(t * 0.37);
  var bc = native.bufferCreate(total), bs = native.bufferCreate(scales.length * 2);
  var bw = native.bufferCreate(K * N * 4), ba = native.bufferCreate(M * K * 4), bo = native.bufferCreate(M * N * 4);
  native.bufferWrite(bc, 0, codes);
  native.bufferWrite(bs, 0, scales);
  native.bufferWrite(ba, 0, x);
  afhip.packWeightQ8Block(bc, bs, block, start, K, N, bw, afhip.DTYPE.f32);
  var packed = new Float32Array(K * N);
  native.bufferRead(bw, 0, packed);
  var differing = 0;
  for (var k = 0; k < K; k++) for (var n = 0; n < N; n++) {
    var e = start + k * N + n;
    if (packed[n * K + k] !== Math.fround(codes[e] * halfToNumber(scales[Math.floor(e / block)]))) differing++;
  }
  assert.strictEqual(differing, 0, "packed q8 weight differs from the decode");
  var plan = native.gemmPlanCreate({ rows: M, inner: K, columns: N, precision: afhip.PRECISION.f32,
    aDtype: afhip.DTYPE.f32, wDtype: afhip.DTYPE.f32, wLayout: 1, outDtype: afhip.DTYPE.f32 });
  native.gemmRun(plan, { a: ba, w: bw, c: bo });
  native.synchronize();
  var out = new Float32Array(M * N);
  native.bufferRead(bo, 0, out);
  var worst = 0, largest = 0;
  for (var r = 0; r < M; r++) for (var c = 0; c < N; c++) {
    var acc = 0;
    for (var kk = 0; kk < K; kk++) acc += x[r * K + kk] * packed[c * K + kk];
    worst = Math.max(worst, Math.abs(out[r * N + c] - acc));
    largest = Math.max(largest, Math.abs(acc));
  }
  // Operands smaller than the plan reads or writes are refused (WebGPU's
  // binding-size validation).
  var small = native.bufferCreate(16);
  assert.throws(function () { native.gemmRun(plan, { a: small, w: bw, c: bo }); }, /buffer a holds 16 bytes/);
  assert.throws(function () { native.gemmRun(plan, { a: ba, w: bw, c: small }); }, /buffer c holds 16 bytes/);
  assert.throws(function () { native.gemmRun(plan, { a: ba, c: bo }); }, /needs operand w/);
  native.bufferDestroy(small);
  native.gemmPlanDestroy(plan);
  [bc, bs, bw, ba, bo].forEach(function (b) { native.bufferDestroy(b); });
  assert.ok(worst <= 1e-5 * largest, "q8 gemm " + worst / largest);
  report.cases.push({ q8PackedGemmMaxRelative: worst / largest });
})();

// AttentionGpu with zero query and key weights and no bias: every key
// weighs 1/Q, so row (b, q) is mean_k(v[b][k]) * g[b][q], then the output
// projection -- computed here in float64 from the LayerNormed rows.
await (async function () {
  var B = 3, Q = 5, C = 8, H = 2;
  function fill(n, f) { var a = new Float32Array(n); for (var i = 0; i < n; i++) a[i] = f(i); return a; }
  var x = fill(B * Q * C, function (i) { return Math.sin(1.3 * i) + 0.1 * (i % 5); });
  var w = { queryNormScale: fill(C, function () { return 1; }), queryNormOffset: fill(C, function () { return 0; }),
    queryWeight: new Float32Array(C * C), keyWeight: new Float32Array(C * C),
    valueWeight: fill(C * C, function (i) { return 0.3 * Math.cos(0.7 * i); }),
    gatingWeight: fill(C * C, function (i) { return 0.2 * Math.sin(0.4 * i); }),
    gatingBias: fill(C, function (i) { return 0.1 * i; }),
    outputWeight: fill(C * C, function (i) { return 0.25 * Math.sin(0.9 * i + 1); }),
    outputBias: fill(C, function (i) { return 0.01 * i; }) };
  var out = (await new afhip.AttentionGpu().run({ activations: x, mask: fill(B * Q, function () { return 1; }), batch: B,
    queryLength: Q, channels: C, heads: H, weights: w }, { precision: "f32" })).output;
  var worst = 0, largest = 0;
  for (var b = 0; b < B; b++) {
    var xn = [], vmean = new Array(C).fill(0);
    for (var q = 0; q < Q; q++) {
      var row = Array.from(x.subarray((b * Q + q) * C, (b * Q + q + 1) * C));
      var mean = row.reduce(function (s, v) { return s + v; }, 0) / C;
      var vr = row.reduce(function (s, v) { return s + (v - mean) * (v - mean); }, 0) / C;
      xn.push(row.map(function (v) { return (v - mean) / Math.sqrt(vr + 1e-5); }));
    }
    for (q = 0; q < Q; q++)
      for (var c = 0; c < C; c++) for (var k = 0; k < C; k++) vmean[c] += xn[q][k] * w.valueWeight[k * C + c] / Q;
    for (q = 0; q < Q; q++) {
      var o = [];
      for (c = 0; c < C; c++) {
        var g = w.gatingBias[c];
        for (k = 0; k < C; k++) g += xn[q][k] * w.gatingWeight[k * C + c];
        o.push(vmean[c] / (1 + Math.exp(-g)));
      }
      for (c = 0; c < C; c++) {
        var y = w.outputBias[c];
        for (k = 0; k < C; k++) y += o[k] * w.outputWeight[k * C + c];
        worst = Math.max(worst, Math.abs(out[(b * Q + q) * C + c] - y));
        largest = Math.max(largest, Math.abs(y));
      }
    }
  }
  assert.ok(worst <= 1e-5 * largest, "attention closed form " + worst / largest);
  report.cases.push({ attentionClosedFormMaxRelative: worst / largest });
})();

// The execution layer from Node: the pair steps chained on the device
// (HipExecution.pairStack) against the six operators run one by one through
// their host-array entry points, the updates added on the host in the
// block's order (src/evoformer/block.ts:1683-1750).
await (async function () {
  var L = 12, S = 5, cM = 8, cO = 4, cZ = 16, cH = 16, hidden = 4 * cZ;
  function fill(n, f) { var a = new Float32Array(n); for (var i = 0; i < n; i++) a[i] = f(i); return a; }
  function wave(n, scale, phase, center) { return fill(n, function (i) { return (center || 0) + scale * Math.sin(0.7 * i + phase); }); }
  function triangleWeights(phase) {
    var sizes = { layerNormInWeight: cZ, layerNormInBias: cZ, linearAPWeight: cH * cZ, linearAPBias: cH,
      linearAGWeight: cH * cZ, linearAGBias: cH, linearBPWeight: cH * cZ, linearBPBias: cH, linearBGWeight: cH * cZ,
      linearBGBias: cH, layerNormOutWeight: cH, layerNormOutBias: cH, linearZWeight: cZ * cH, linearZBias: cZ,
      linearGWeight: cZ * cZ, linearGBias: cZ };
    var w = {};
    afhip.TRIANGLE_ORDER.forEach(function (n, k) {
      w[n] = n.indexOf("layerNorm") === 0 && n.indexOf("Weight") > 0 ? wave(sizes[n], 0.1, phase + k, 1)
        : wave(sizes[n], n.indexOf("Bias") > 0 ? 0.05 : 0.25, phase + k);
    });
    return w;
  }
  function attentionWeights(phase) {
    return { heads: 2, pairProjectionWeight: wave(cZ * 2, 0.3, phase + 9), attention: {
      queryNormScale: wave(cZ, 0.1, phase, 1), queryNormOffset: wave(cZ, 0.05, phase + 1),
      queryWeight: wave(cZ * cZ, 0.25, phase + 2), keyWeight: wave(cZ * cZ, 0.25, phase + 3),
      valueWeight: wave(cZ * cZ, 0.25, phase + 4), gatingWeight: wave(cZ * cZ, 0.25, phase + 5),
      gatingBias: wave(cZ, 0.1, phase + 6, 1), outputWeight: wave(cZ * cZ, 0.25, phase + 7),
      outputBias: wave(cZ, 0.05, phase + 8) } };
  }
  var weights = {
    outerProductMean: { layerNormScale: wave(cM, 0.1, 1, 1), layerNormOffset: wave(cM, 0.05, 2),
      leftWeight: wave(cM * cO, 0.3, 3), leftBias: wave(cO, 0.05, 4), rightWeight: wave(cM * cO, 0.3, 5),
      rightBias: wave(cO, 0.05, 6), outputWeight: wave(cO * cO * cZ, 0.2, 7), outputBias: wave(cZ, 0.05, 8) },
    triangleMultiplicationOutgoing: triangleWeights(10),
    triangleMultiplicationIncoming: triangleWeights(40),
    triangleAttentionStarting: attentionWeights(50),
    triangleAttentionEnding: attentionWeights(60),
    pairTransition: { layerNormScale: wave(cZ, 0.1, 70, 1), layerNormOffset: wave(cZ, 0.05, 71),
      firstWeight: wave(cZ * hidden, 0.2, 72), firstBias: wave(hidden, 0.05, 73),
      secondWeight: wave(hidden * cZ, 0.1, 74), secondBias: wave(cZ, 0.05, 75) },
  };
  var msa = wave(S * L * cM, 1, 0.3), msaMask = fill(S * L, function (i) { return i % 7 === 3 ? 0 : 1; });
  var pair = wave(L * L * cZ, 1, 0.9), pairMask = fill(L * L, function (i) { return i % 11 === 5 ? 0 : 1; });

  var z = Float32Array.from(pair);
  function addInto(base, update) { for (var i = 0; i < base.length; i++) base[i] = Math.fround(base[i] + update[i]); }
  addInto(z, (await new afhip.OuterProductMeanGpu().run({ sequences: S, length: L, cM: cM, cOuter: cO, cZ: cZ,
    activations: msa, mask: msaMask, weights: weights.outerProductMean })).output);
  addInto(z, (await new afhip.TriangleMultiplicationOutgoingGpu().run({ shape: { length: L, cZ: cZ, cHidden: cH },
    z: z, mask: pairMask, weights: weights.triangleMultiplicationOutgoing })).output);
  addInto(z, (await new afhip.TriangleMultiplicationIncomingGpu().run({ shape: { length: L, cZ: cZ, cHidden: cH },
    z: z, mask: pairMask, weights: weights.triangleMultiplicationIncoming })).output);
  var steps = [["triangleAttentionStarting", false], ["triangleAttentionEnding", true]];
  for (var si = 0; si < steps.length; si++) {
    var a = weights[steps[si][0]];
    addInto(z, (await new afhip.AttentionGpu().run({ activations: z, mask: pairMask, batch: L, queryLength: L,
      channels: cZ, heads: 2, transpose: steps[si][1], weights: a.attention,
      pairBias: { source: "normalized-input", projectionWeight: a.pairProjectionWeight } })).output);
  }
  addInto(z, (await new afhip.TransitionGpu().run({ rows: L * L, channels: cZ, hiddenChannels: hidden,
    activations: z, weights: weights.pairTransition })).output);

  var ex = new afhip.HipExecution();
  var shape = { length: L, sequences: S, cM: cM, cZ: cZ, cOuter: cO, cHidden: cH, transitionFactor: 4,
    precision: afhip.PRECISION.f32, pairDtype: afhip.DTYPE.f32, msaDtype: afhip.DTYPE.f32, attentionHeads: 2 };
  var prepared = ex.preparePairStack(shape, weights);
  var bPair = ex.upload("pair", pair), bMask = ex.upload("pair-mask", pairMask);
  var bMsa = ex.upload("msa", msa), bMsaMask = ex.upload("msa-mask", msaMask);
  ex.pairStack(shape, prepared, bPair, bMask, bMsa, bMsaMask);
  var got = ex.read(bPair, new Float32Array(L * L * cZ));
  var m = afhip.errorMetrics(got, z);
  var largest = 0;
  for (var i = 0; i < z.length; i++) largest = Math.max(largest, Math.abs(z[i]));
  assert.ok(m.maxAbsoluteError <= 1e-5 * largest, "pair stack " + JSON.stringify(m));
  // A prepared-weight handle of another kind, or a plain buffer, is refused
  // before anything runs.
  assert.throws(function () {
    ex.pairStack(shape, { triangleOutgoing: prepared.triangleIncoming }, bPair, bMask);
  }, /must come from executionPrepareWeights\("triangleOutgoing"\); handle \d+ was prepared as "triangleIncoming"/);
  var plainBuffer = afhip.addon().bufferCreate(64);
  assert.throws(function () { ex.pairStack(shape, { pairTransition: plainBuffer }, bPair, bMask); },
    /was prepared as nothing/);
  afhip.addon().bufferDestroy(plainBuffer);
  // (prepared triangle weights pad c_hidden to 32 rows, so the larger shape
  // is c_hidden 64)
  var bigger = Object.assign({}, shape, { cHidden: 64 });
  assert.throws(function () { ex.pairStack(bigger, { triangleOutgoing: prepared.triangleOutgoing }, bPair, bMask); },
    /prepared weights for triangleOutgoing hold \d+ bytes; this shape needs \d+/);
  var snap = ex.snapshot();
  assert.ok(snap.peakComposition.length > 0 && snap.residentBytes >= snap.currentBytes);
  ex.release();
  report.cases.push({ pairStackVsOperators: m });

  // The whole block (HipExecution.evoformerBlock) against its MSA steps run
  // through the host-array operators, followed by the device pair stack
  // checked above (src/evoformer/block.ts:1690-1716).
  var msaW = {
    msaRowAttention: { attention: attentionWeights(80).attention, pairLayerNormScale: wave(cZ, 0.1, 90, 1),
      pairLayerNormOffset: wave(cZ, 0.05, 91), pairProjectionWeight: wave(cZ * 2, 0.3, 92) },
    msaColumnAttention: { attention: attentionWeights(100).attention },
    msaTransition: { layerNormScale: wave(cM, 0.1, 110, 1), layerNormOffset: wave(cM, 0.05, 111),
      firstWeight: wave(cM * 4 * cM, 0.2, 112), firstBias: wave(4 * cM, 0.05, 113),
      secondWeight: wave(4 * cM * cM, 0.1, 114), secondBias: wave(cM, 0.05, 115) },
  };
  // Attention over the MSA needs c_m heads of at most 32 channels: cM = 8 over 2 heads.
  msaW.msaRowAttention.attention = Object.assign({}, msaW.msaRowAttention.attention);
  ["queryNormScale", "queryNormOffset", "gatingBias", "outputBias"].forEach(function (n, k) {
    msaW.msaRowAttention.attention[n] = wave(cM, 0.1, 120 + k, n === "queryNormScale" ? 1 : 0);
    msaW.msaColumnAttention.attention[n] = wave(cM, 0.1, 130 + k, n === "queryNormScale" ? 1 : 0);
  });
  ["queryWeight", "keyWeight", "valueWeight", "gatingWeight", "outputWeight"].forEach(function (n, k) {
    msaW.msaRowAttention.attention[n] = wave(cM * cM, 0.25, 140 + k);
    msaW.msaColumnAttention.attention[n] = wave(cM * cM, 0.25, 150 + k);
  });
  var m2 = Float32Array.from(msa);
  var rw = msaW.msaRowAttention;
  addInto(m2, (await new afhip.AttentionGpu().run({ activations: m2, mask: msaMask, batch: S, queryLength: L,
    channels: cM, heads: 2, weights: rw.attention, pairBias: { source: "separate", activations: pair, channels: cZ,
      layerNormScale: rw.pairLayerNormScale, layerNormOffset: rw.pairLayerNormOffset,
      projectionWeight: rw.pairProjectionWeight } })).output);
  addInto(m2, (await new afhip.AttentionGpu().run({ activations: m2, mask: msaMask, batch: L, queryLength: S,
    channels: cM, heads: 2, transpose: true, weights: msaW.msaColumnAttention.attention })).output);
  addInto(m2, (await new afhip.TransitionGpu().run({ rows: S * L, channels: cM, hiddenChannels: 4 * cM,
    activations: m2, weights: msaW.msaTransition })).output);
  var ex2 = new afhip.HipExecution();
  var ePair = ex2.upload("pair", pair), eMask = ex2.upload("pair-mask", pairMask);
  var eMsa = ex2.upload("msa", m2), eMsaMask = ex2.upload("msa-mask", msaMask);
  ex2.pairStack(shape, ex2.preparePairStack(shape, weights), ePair, eMask, eMsa, eMsaMask);
  var zExpect = ex2.read(ePair, new Float32Array(L * L * cZ));
  var blockShape = Object.assign({ msaHeads: 2 }, shape);
  var preparedBlock = ex2.prepareEvoformerBlock(blockShape, Object.assign({}, weights, msaW));
  var gPair = ex2.upload("pair", pair), gMsa = ex2.upload("msa", msa);
  ex2.evoformerBlock(blockShape, preparedBlock, gMsa, eMsaMask, gPair, eMask);
  var mGot = ex2.read(gMsa, new Float32Array(S * L * cM)), zGot = ex2.read(gPair, new Float32Array(L * L * cZ));
  function rel(a, b) {
    var worst = 0, big = 0;
    for (var i = 0; i < a.length; i++) { worst = Math.max(worst, Math.abs(a[i] - b[i])); big = Math.max(big, Math.abs(b[i])); }
    return worst / big;
  }
  var rm = rel(mGot, m2), rz = rel(zGot, zExpect);
  assert.ok(rm <= 1e-5 && rz <= 1e-5, "evoformer block msa " + rm + " pair " + rz);
  ex2.release();
  report.cases.push({ evoformerBlockVsOperators: { msa: rm, pair: rz } });
})();

  console.log(JSON.stringify(report));
}

main().catch(function (err) { console.error(err); process.exit(1); });

"use strict";
// Test and baseline infrastructure, not product code: the reference's CPU
// path for the triangle multiplication, restated in plain JavaScript so it
// runs under any Node (no ?? or ?. syntax), for bench.py's cpu_baseline leg.
//
// triangleMultiplicationOutgoingReference (src/triangle/cpu-reference.ts:56-100)
// with normalizeRows (:6-31) and project (:33-54): JS doubles for every
// accumulation, each tensor stored to a Float32Array as the reference stores
// it, in the reference's loop order. The input is the reference's
// createDeterministicTriangleInput (src/testing/deterministic-input.ts:7-51).
//
//   node oracle/cpu_reference.js <length> [cZ] [cHidden] [seed] [--output FILE]
// prints one JSON line: node version, CPU count and model, the sample's
// seconds (the operator alone, input generation excluded) and a checksum;
// --output writes the f32 output (little-endian) for tests/test_oracle.py.
var fs = require("fs");
var os = require("os");

function sigmoid(value) { return 1 / (1 + Math.exp(-value)); }

function normalizeRows(input, rowCount, channels, weight, bias, epsilon) {
  var output = new Float32Array(input.length);
  for (var row = 0; row < rowCount; row += 1) {
    var offset = row * channels;
    var mean = 0;
    for (var c = 0; c < channels; c += 1) mean += input[offset + c];
    mean /= channels;
    var variance = 0;
    for (c = 0; c < channels; c += 1) {
      var centered = input[offset + c] - mean;
      variance += centered * centered;
    }
    var inverseStd = 1 / Math.sqrt(variance / channels + epsilon);
    for (c = 0; c < channels; c += 1) {
      output[offset + c] = (input[offset + c] - mean) * inverseStd * weight[c] + bias[c];
    }
  }
  return output;
}

function project(input, rows, inChannels, outChannels, weight, bias) {
  var output = new Float32Array(rows * outChannels);
  for (var row = 0; row < rows; row += 1) {
    for (var out = 0; out < outChannels; out += 1) {
      var value = bias[out];
      var weightOffset = out * inChannels;
      var inputOffset = row * inChannels;
      for (var c = 0; c < inChannels; c += 1) value += input[inputOffset + c] * weight[weightOffset + c];
      output[row * outChannels + out] = value;
    }
  }
  return output;
}

function triangleOutgoing(input) {
  var length = input.shape.length, cZ = input.shape.cZ, cHidden = input.shape.cHidden;
  var pairs = length * length;
  var epsilon = input.epsilon === undefined ? 1e-5 : input.epsilon;
  var w = input.weights;
  var z = normalizeRows(input.z, pairs, cZ, w.layerNormInWeight, w.layerNormInBias, epsilon);
  var ap = project(z, pairs, cZ, cHidden, w.linearAPWeight, w.linearAPBias);
  var ag = project(z, pairs, cZ, cHidden, w.linearAGWeight, w.linearAGBias);
  var bp = project(z, pairs, cZ, cHidden, w.linearBPWeight, w.linearBPBias);
  var bg = project(z, pairs, cZ, cHidden, w.linearBGWeight, w.linearBGBias);
  for (var pair = 0; pair < pairs; pair += 1) {
    var mask = input.mask[pair];
    for (var h = 0; h < cHidden; h += 1) {
      var index = pair * cHidden + h;
      ap[index] = ap[index] * sigmoid(ag[index]) * mask;
      bp[index] = bp[index] * sigmoid(bg[index]) * mask;
    }
  }
  var contracted = new Float32Array(pairs * cHidden);
  for (var i = 0; i < length; i += 1) {
    for (var j = 0; j < length; j += 1) {
      for (h = 0; h < cHidden; h += 1) {
        var value = 0;
        for (var k = 0; k < length; k += 1) value += ap[(i * length + k) * cHidden + h] * bp[(j * length + k) * cHidden + h];
        contracted[(i * length + j) * cHidden + h] = value;
      }
    }
  }
  var normalized = normalizeRows(contracted, pairs, cHidden, w.layerNormOutWeight, w.layerNormOutBias, epsilon);
  var output = project(normalized, pairs, cHidden, cZ, w.linearZWeight, w.linearZBias);
  var gate = project(z, pairs, cZ, cZ, w.linearGWeight, w.linearGBias);
  for (index = 0; index < output.length; index += 1) output[index] = output[index] * sigmoid(gate[index]);
  return output;
}

function deterministicInput(shape, seed) {
  var state = seed >>> 0;
  function random() {
    state = (state + 0x6d2b79f5) >>> 0;
    var value = state;
    value = Math.imul(value ^ (value >>> 15), value | 1);
    value ^= value + Math.imul(value ^ (value >>> 7), value | 61);
    return ((value ^ (value >>> 14)) >>> 0) / 4294967296;
  }
  function values(count, scale, center) {
    var out = new Float32Array(count);
    for (var n = 0; n < count; n++) out[n] = (center || 0) + (random() * 2 - 1) * scale;
    return out;
  }
  var cZ = shape.cZ, cH = shape.cHidden, pairs = shape.length * shape.length;
  var weights = {
    layerNormInWeight: values(cZ, 0.1, 1), layerNormInBias: values(cZ, 0.05),
    linearAPWeight: values(cH * cZ, 0.15 / Math.sqrt(cZ)), linearAPBias: values(cH, 0.03),
    linearAGWeight: values(cH * cZ, 0.15 / Math.sqrt(cZ)), linearAGBias: values(cH, 0.03, 1),
    linearBPWeight: values(cH * cZ, 0.15 / Math.sqrt(cZ)), linearBPBias: values(cH, 0.03),
    linearBGWeight: values(cH * cZ, 0.15 / Math.sqrt(cZ)), linearBGBias: values(cH, 0.03, 1),
    layerNormOutWeight: values(cH, 0.1, 1), layerNormOutBias: values(cH, 0.05),
    linearZWeight: values(cZ * cH, 0.15 / Math.sqrt(cH)), linearZBias: values(cZ, 0.03),
    linearGWeight: values(cZ * cZ, 0.15 / Math.sqrt(cZ)), linearGBias: values(cZ, 0.03, 1),
  };
  var mask = new Float32Array(pairs);
  for (var p = 0; p < pairs; p++) mask[p] = random() > 0.15 ? 1 : 0;
  return { shape: shape, z: values(pairs * cZ, 1), mask: mask, weights: weights };
}

function main(argv) {
  var outputFile = null;
  var positional = [];
  for (var a = 0; a < argv.length; a++) {
    if (argv[a] === "--output") outputFile = argv[++a];
    else positional.push(Number(argv[a]));
  }
  var shape = { length: positional[0] || 32, cZ: positional[1] || 128, cHidden: positional[2] || 128 };
  var input = deterministicInput(shape, positional[3] === undefined ? 7 : positional[3]);
  var start = process.hrtime();
  var output = triangleOutgoing(input);
  var elapsed = process.hrtime(start);
  var checksum = 0;
  for (var n = 0; n < output.length; n++) checksum += output[n];
  if (outputFile) fs.writeFileSync(outputFile, Buffer.from(output.buffer));
  var cpus = os.cpus();
  console.log(JSON.stringify({
    node: process.versions.node, cpus: cpus.length, cpuModel: cpus.length ? cpus[0].model : "unknown",
    threads: 1, shape: shape, seconds: elapsed[0] + elapsed[1] * 1e-9, checksum: checksum,
  }));
}

main(process.argv.slice(2));

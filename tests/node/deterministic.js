"use strict";
// createDeterministicTriangleInput (src/testing/deterministic-input.ts:7-51),
// restated for the Node tests: the reference's generator (state advanced by
// 0x6d2b79f5, three xor-shift-multiply rounds, 32-bit result / 2^32) and its
// draw order (the sixteen weights in ORDER, then the mask, then z).
// tests/node/abi_check.js holds it to tests/golden/generators.json, which
// the reference's own source wrote.
function generator(seed) {
  var state = seed >>> 0;
  return function () {
    state = (state + 0x6d2b79f5) >>> 0;
    var value = state;
    value = Math.imul(value ^ (value >>> 15), value | 1);
    value ^= value + Math.imul(value ^ (value >>> 7), value | 61);
    return ((value ^ (value >>> 14)) >>> 0) / 4294967296;
  };
}

function createDeterministicTriangleInput(shape, seed) {
  var random = generator(seed === undefined ? 7 : seed);
  function values(length, scale, center) {
    var out = new Float32Array(length);
    for (var i = 0; i < length; i++) out[i] = (center || 0) + (random() * 2 - 1) * scale;
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
  for (var i = 0; i < pairs; i++) mask[i] = random() > 0.15 ? 1 : 0;
  return { shape: shape, z: values(pairs * cZ, 1), mask: mask, weights: weights };
}

module.exports = { createDeterministicTriangleInput: createDeterministicTriangleInput };

"use strict";
// Reads a triangle reference bundle (manifest.json + float32 little-endian
// tensors), as src/reference/node.ts:13-42 does.
var fs = require("fs");
var path = require("path");

var WEIGHTS = [
  "layerNormInWeight", "layerNormInBias", "linearAPWeight", "linearAPBias", "linearAGWeight", "linearAGBias",
  "linearBPWeight", "linearBPBias", "linearBGWeight", "linearBGBias", "layerNormOutWeight", "layerNormOutBias",
  "linearZWeight", "linearZBias", "linearGWeight", "linearGBias",
];

function loadTriangleBundle(manifestPath) {
  var manifest = JSON.parse(fs.readFileSync(manifestPath, "utf8"));
  if (manifest.formatVersion !== 1 || manifest.operator !== "TriangleMultiplicationOutgoing") {
    throw new Error("unsupported triangle reference manifest");
  }
  var dir = path.dirname(manifestPath);
  function tensor(name) {
    var rec = manifest.tensors[name];
    if (!rec || rec.dtype !== "float32") throw new Error("missing float32 tensor " + name);
    var buf = fs.readFileSync(path.join(dir, rec.file));
    var count = rec.shape.reduce(function (a, b) { return a * b; }, 1);
    if (buf.length !== count * 4) throw new Error("invalid byte length for tensor " + name);
    var out = new Float32Array(count);
    for (var i = 0; i < count; i++) out[i] = buf.readFloatLE(4 * i);
    return out;
  }
  var weights = {};
  WEIGHTS.forEach(function (n) { weights[n] = tensor(n); });
  return {
    input: {
      shape: [manifest.shape.length, manifest.shape.cZ, manifest.shape.cHidden],
      epsilon: manifest.epsilon === undefined ? 1e-5 : manifest.epsilon,
      z: tensor("z"), mask: tensor("mask"), weights: weights,
    },
    expected: tensor("expected"),
  };
}

module.exports = { loadTriangleBundle: loadTriangleBundle };

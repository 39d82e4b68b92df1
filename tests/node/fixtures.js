"use strict";
// loadTriangleReferenceBundleFromFiles (src/reference/node.ts:13-42): a
// manifest.json plus float32 little-endian tensors; the input carries the
// manifest's own TriangleShape {length, cZ, cHidden} and epsilon, as the
// reference hands them to TriangleMultiplicationGpu.run.
var fs = require("fs");
var path = require("path");

var WEIGHTS = [
  "layerNormInWeight", "layerNormInBias", "linearAPWeight", "linearAPBias", "linearAGWeight", "linearAGBias",
  "linearBPWeight", "linearBPBias", "linearBGWeight", "linearBGBias", "layerNormOutWeight", "layerNormOutBias",
  "linearZWeight", "linearZBias", "linearGWeight", "linearGBias",
];

async function loadTriangleReferenceBundleFromFiles(manifestPath) {
  var manifest = JSON.parse(await fs.promises.readFile(manifestPath, "utf8"));
  if (manifest.formatVersion !== 1 || manifest.operator !== "TriangleMultiplicationOutgoing") {
    throw new Error("unsupported triangle reference manifest");
  }
  var dir = path.dirname(manifestPath);
  async function tensor(name) {
    var rec = manifest.tensors[name];
    if (!rec || rec.dtype !== "float32") throw new Error("missing float32 tensor " + name);
    var bytes = await fs.promises.readFile(path.resolve(dir, rec.file));
    var count = rec.shape.reduce(function (a, b) { return a * b; }, 1);
    if (bytes.byteLength !== count * 4) throw new Error("invalid byte length for tensor " + name);
    return new Float32Array(bytes.buffer.slice(bytes.byteOffset, bytes.byteOffset + bytes.byteLength));
  }
  var weights = {};
  await Promise.all(WEIGHTS.map(async function (n) { weights[n] = await tensor(n); }));
  return {
    source: manifest.source,
    input: { shape: manifest.shape, epsilon: manifest.epsilon, z: await tensor("z"), mask: await tensor("mask"),
      weights: weights },
    expected: await tensor("expected"),
  };
}

module.exports = { loadTriangleReferenceBundleFromFiles: loadTriangleReferenceBundleFromFiles };

"""Triangle reference bundles: manifest.json plus f32 little-endian tensors.

Mirrors src/reference/node.ts:13-42 (loadTriangleReferenceBundleFromFiles)
and the manifest shape of src/reference/bundle.ts: formatVersion 1, operator
"TriangleMultiplicationOutgoing", shape {length, cZ, cHidden}, epsilon, and
a float32 record per tensor.
"""
from __future__ import annotations

import json
import os

import numpy as np

WEIGHT_NAMES = (
    "layerNormInWeight", "layerNormInBias", "linearAPWeight", "linearAPBias",
    "linearAGWeight", "linearAGBias", "linearBPWeight", "linearBPBias",
    "linearBGWeight", "linearBGBias", "layerNormOutWeight", "layerNormOutBias",
    "linearZWeight", "linearZBias", "linearGWeight", "linearGBias",
)


def load_triangle_reference_bundle(manifest_path: str) -> dict:
    """Returns {source, input: {shape, epsilon, z, mask, weights}, expected}.

    Raises ValueError for an unsupported manifest, a missing or non-float32
    tensor, or a file whose byte length disagrees with its shape, as
    node.ts:18-33 does.
    """
    with open(manifest_path, "r", encoding="utf-8") as handle:
        manifest = json.load(handle)
    if manifest.get("formatVersion") != 1 or manifest.get("operator") != "TriangleMultiplicationOutgoing":
        raise ValueError("unsupported triangle reference manifest")
    directory = os.path.dirname(manifest_path)

    def tensor(name: str) -> np.ndarray:
        record = manifest["tensors"].get(name)
        if record is None or record.get("dtype") != "float32":
            raise ValueError(f"missing float32 tensor {name}")
        shape = tuple(int(v) for v in record["shape"])
        with open(os.path.join(directory, record["file"]), "rb") as handle:
            data = handle.read()
        if len(data) != int(np.prod(shape)) * 4:
            raise ValueError(f"invalid byte length for tensor {name}")
        return np.frombuffer(data, dtype="<f4").reshape(shape).astype(np.float32)

    shape = manifest["shape"]
    return {
        "source": manifest.get("source", ""),
        "input": {
            "shape": {"length": int(shape["length"]), "cZ": int(shape["cZ"]), "cHidden": int(shape["cHidden"])},
            "epsilon": float(manifest.get("epsilon", 1e-5)),
            "z": tensor("z"),
            "mask": tensor("mask"),
            "weights": {name: tensor(name) for name in WEIGHT_NAMES},
        },
        "expected": tensor("expected"),
    }

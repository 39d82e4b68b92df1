"""Copies the reference's triangle fixtures into tests/golden/.

The fixtures are data the reference's own tests hold (f32 little-endian .bin
tensors plus a manifest.json, the format read by src/reference/node.ts:13-42).
Run once in a container that has /root/reference; the copies travel with the
repository so the GPU box, which has no reference checkout, can use them.

  python tests/golden/make_golden.py [/root/reference]

openfold-triangle-small: OpenFold deterministic test weights (Apache-2.0).
short-9: activations and parameters of AlphaFold model_3_ptm, block 0; the
AlphaFold parameters are DeepMind's, under CC BY 4.0
(https://github.com/google-deepmind/alphafold/blob/main/WEIGHTS_LICENSE).
model1-reference-59 (single sequence and a3m): AlphaFold model_1 block-0
captures at 59 residues, same licence; 3.9 MB each, copied so the GPU tests
can run them (test/triangle-multiplication-outgoing.gpu.test.ts:30-56).
"""
import os
import shutil
import sys

FIXTURES = {
    "openfold-triangle-small": "test/fixtures/openfold-triangle-small",
    "alphafold-short-9": "test/fixtures/alphafold-single-sequence/short-9",
    "alphafold-single-sequence-59": "test/fixtures/alphafold-single-sequence/model1-reference-59",
    "alphafold-a3m-59": "test/fixtures/alphafold-a3m/model1-reference-59",
}


def main(reference: str = "/root/reference") -> None:
    here = os.path.dirname(os.path.abspath(__file__))
    for name, rel in FIXTURES.items():
        src = os.path.join(reference, rel)
        dst = os.path.join(here, name)
        os.makedirs(dst, exist_ok=True)
        for entry in sorted(os.listdir(src)):
            shutil.copyfile(os.path.join(src, entry), os.path.join(dst, entry))
        print(f"copied {src} -> {dst}")


if __name__ == "__main__":
    main(*sys.argv[1:])

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
The two 59-residue fixtures (3.9 MB each) are not copied; the CPU tests read
them in place when the reference checkout is present.
"""
import os
import shutil
import sys

FIXTURES = {
    "openfold-triangle-small": "test/fixtures/openfold-triangle-small",
    "alphafold-short-9": "test/fixtures/alphafold-single-sequence/short-9",
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

"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

Inputs are not stored: each fixture records the seeds and shapes that regenerate them with numpy's
PCG64 (tests/golden/cases.py), plus the SHA-256 of the generated input bytes so a generator change
is caught. Outputs are stored as arrays. Run from the repository root:
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [HERE, os.path.join(ROOT, "ml-framework_amd"), os.path.join(ROOT, "oracle")]

import cases  # noqa: E402


def main():
    for name in cases.CASES:
        inputs, outputs = cases.build(name)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), input_sha256=np.array(cases.digest(inputs)),
                            **outputs)
        size = os.path.getsize(os.path.join(HERE, f"{name}.npz"))
        print(f"{name}: {', '.join(f'{k}{v.shape}' for k, v in outputs.items())} ({size} bytes)")


if __name__ == "__main__":
    main()

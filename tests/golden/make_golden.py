"""Writes tests/golden/ref_cpu_vectors.json from the reference's own CPU kernels.

The library is oracle/_ref/libfa_cpu_ref.so, compiled by oracle/Makefile from
the reference's frame_analytics/csrc/fa_cpu.cpp.  Inputs are regenerated from
the seeds stored with each case (tests/conftest.py generators), so the file
holds only case parameters and the reference's outputs.

    make -C oracle && python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))

from oracle import ref_cpu  # noqa: E402
from tests.conftest import natural_pair, u8_pair  # noqa: E402

CASES = [
    {"gen": "natural", "h": 64, "w": 64, "kind": "uniform", "noise": 20.0, "seed": 4096},
    {"gen": "natural", "h": 127, "w": 233, "kind": "natural", "noise": 8.0, "seed": 29591},
    {"gen": "natural", "h": 256, "w": 256, "kind": "natural", "noise": 3.0, "seed": 65536},
    {"gen": "natural", "h": 33, "w": 41, "kind": "flat", "noise": 5.0, "seed": 1353},
    {"gen": "natural", "h": 200, "w": 232, "kind": "natural", "noise": 8.0, "seed": 432},
    {"gen": "u8", "shape": [1, 3, 512, 512], "sigma": 8.0, "seed": 0},
    {"gen": "u8", "shape": [3, 2, 70, 90], "sigma": 20.0, "seed": 5},
]


def inputs(case):
    if case["gen"] == "natural":
        a, b = natural_pair(case["h"], case["w"], case["noise"], seed=case["seed"], kind=case["kind"])
        return a.astype(np.uint8)[None, None], b.astype(np.uint8)[None, None]
    return u8_pair(tuple(case["shape"]), case["sigma"], seed=case["seed"])


def main():
    ref_cpu.load(threads=4)
    out = []
    for case in CASES:
        a, b = inputs(case)
        s, cs = ref_cpu.ssim_cs(a, b)
        m, sd = ref_cpu.gmsd(a, b)
        exp = {
            "mse": ref_cpu.pixel_reduce(a, b, "mse"),
            "l1": ref_cpu.pixel_reduce(a, b, "l1"),
            "ssim_per_image": ref_cpu.ssim_per_image(a, b).tolist(),
            "ssim_cs": [s.tolist(), cs.tolist()],
            "gmsd": [m.tolist(), sd.tolist()],
        }
        out.append({**case, "expect": exp})
    dst = Path(__file__).resolve().parent / "ref_cpu_vectors.json"
    dst.write_text(json.dumps({"source": "reference fa_cpu.cpp via oracle/_ref", "cases": out},
                              indent=1))
    print(f"wrote {dst}")


if __name__ == "__main__":
    main()

"""Write tests/golden/oracle_tiny.npz: the oracle's results for the tiny cases of
tests/golden/cases.py (inputs included), as the repository's own golden vectors.

    python tests/golden/make_oracle_vectors.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from tests.golden import cases  # noqa: E402

OUT = os.path.join(HERE, "oracle_tiny.npz")


def oracle_opt(spec):
    return O.Optimiser.adam() if spec[0] == "adam" else O.Optimiser.sgd(spec[1], spec[2])


def oracle_case(name: str, d: dict) -> dict:
    def make(K, N, M, w, half, b, **kw):
        return O.OracleBlock(K, N, M, w, half=half, master_w=w if half else None, b=b, **kw)

    return cases.run(name, d, make, oracle_opt, lambda opt, M, lr: (opt, opt, M, lr, 3.4e38, 1),
                     lambda a, half: a, lambda a: np.asarray(a, np.float32))


def main() -> None:
    arrays = {}
    for name in cases.CASES:
        d = cases.inputs(name)
        for k, v in d.items():
            arrays[f"{name}__in__{k}"] = v
        for k, v in oracle_case(name, d).items():
            arrays[f"{name}__out__{k}"] = v
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}: {len(arrays)} arrays")


if __name__ == "__main__":
    main()

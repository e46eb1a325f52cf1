"""Writes tests/golden/<case>.npz: the inputs stored with each case and the oracle's
outputs (see cases.py). Run from the repository root:

    python tests/golden/make_fixtures.py
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [REPO, os.path.dirname(HERE)]

import numpy as np  # noqa: E402

from golden.cases import CASES, gen_inputs, oracle_outputs, path, weights_digest  # noqa: E402


def main():
    for case in CASES:
        inp = gen_inputs(case)
        out = oracle_outputs(case, inp)
        rec = dict(x_bits=inp["x_bits"], router_w_bits=inp["router_w_bits"],
                   weights_sha256=np.array(weights_digest(inp)))
        if inp["corr_bias"] is not None:
            rec["corr_bias"] = inp["corr_bias"]
        if inp["router_bias"] is not None:
            rec["router_bias"] = inp["router_bias"]
        rec.update(out)
        np.savez_compressed(path(case), **rec)
        print(case, os.path.getsize(path(case)), "bytes", flush=True)


if __name__ == "__main__":
    main()

"""Write tests/golden/kat_<case>.npz: input digest + fp64 brute-force outputs.

    python tests/golden/make_golden.py
"""
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

from golden.cases import CASES, build_case, expected_fp64, input_digest  # noqa: E402


def main():
    for name in CASES:
        case = build_case(name)
        out = expected_fp64(case).astype(np.float32)
        np.savez_compressed(HERE / f"kat_{name}.npz", digest=np.array(input_digest(case)), out=out)
        print(name, out.shape)


if __name__ == "__main__":
    main()

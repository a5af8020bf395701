"""Writes tests/golden/attention_golden.npz: for every case of attention_cases.py, the
SHA-256 of its regenerated inputs and the CPU restatement's output (float64).

    python tests/golden/make_attention_fixtures.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(HERE.parent.parent))

import attention_cases as AC  # noqa: E402
import oracle  # noqa: E402


def main() -> None:
    out = {}
    for name in AC.CASES:
        case = AC.inputs(name)
        out[f"{name}/digest"] = np.array(AC.digest(case))
        out[f"{name}/out"] = AC.expected(oracle, name, case)
        print(name, out[f"{name}/out"].shape, AC.digest(case)[:16])
    np.savez_compressed(HERE / "attention_golden.npz", **out)


if __name__ == "__main__":
    main()

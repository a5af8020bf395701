"""Committed golden attention cases (tests/golden/attention_golden.npz): the CPU
restatement reproduces every stored output from the regenerated inputs, and the
inputs are the ones the outputs were made from (SHA-256)."""
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import attention_cases as AC  # noqa: E402

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "attention_golden.npz")


@pytest.mark.parametrize("name", AC.CASES)
def test_golden_inputs_and_oracle(orc, name):
    case = AC.inputs(name)
    assert str(GOLD[f"{name}/digest"]) == AC.digest(case), "input generator changed"
    np.testing.assert_allclose(AC.expected(orc, name, case), GOLD[f"{name}/out"], rtol=0, atol=1e-12)

"""The library's lineup validator (jq_validate_lineup, host only) against the
oracle's restatement of validate_lineup (setup.py:60-136), which the golden
setup_validation scenarios pin."""

from __future__ import annotations

import json

import numpy as np
import pytest

from oracle import oracle as O
from tests import helpers as H

BITS = {1: "TYPE", 2: "C1", 4: "C2", 8: "C3", 16: "C4", 32: "C5"}


@pytest.fixture(scope="module")
def jl():
    from junqi_amd import _lib
    return _lib


def lib_codes(jl, lineup) -> set[str]:
    a = np.ascontiguousarray(np.asarray(lineup, dtype=np.int8))
    v = jl.lib.jq_validate_lineup(a.ctypes.data)
    assert v >= 0
    return {name for bit, name in BITS.items() if v & bit}


def test_golden_setup_validation_cases(jl):
    for path in H.scenario_files("setup_validation"):
        su = json.loads(path.read_text())["setup_only"]
        lu = [H.TYPE_OF[n] for n in su["lineups"][0]]
        if len(lu) != 30:
            continue   # LENGTH: the C ABI takes exactly 30 slots
        assert lib_codes(jl, lu) == O.validate_lineup(lu), path.stem
        assert (not lib_codes(jl, lu)) == su["expect_valid"], path.stem


def test_random_mutations_agree_with_oracle(jl):
    rng = np.random.default_rng(0)
    for k in range(3000):
        lu = O.random_setup(k)[30 * (k % 4):30 * (k % 4) + 30].astype(np.int64)
        for _ in range(int(rng.integers(0, 3))):
            op = rng.integers(3)
            if op == 0:
                i, j = rng.integers(30, size=2)
                lu[i], lu[j] = lu[j], lu[i]
            elif op == 1:
                lu[rng.integers(30)] = rng.integers(0, 14)
            else:
                lu[rng.integers(30)] = rng.choice([-1, 14, 100])
        assert lib_codes(jl, lu) == O.validate_lineup(lu), (k, lu.tolist())


def test_null_lineup_is_an_argument_error(jl):
    assert jl.lib.jq_validate_lineup(None) == jl.JQ_E_ARG

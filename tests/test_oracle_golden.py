# SPDX-License-Identifier: Unlicense
"""CPU: the oracle against the committed torch-float64 golden outputs of the
reference's own kernel-check cases, and the input generator against the
oracle's C copy of the reference's xorshift64.

These pin the oracle: each generic-op function of oracle/oracle.c must
reproduce a closed form computed independently (torch float64 library
routines) within the reference's bar of 2e-5 (ops_compare.py:26)."""

from pathlib import Path

import numpy as np
import pytest

import opcases
from oracle_lib import fp

GOLDEN = Path(__file__).resolve().parent / "golden" / "ops_check_golden.npz"
CASES = opcases.all_cases()


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


def test_golden_covers_every_case(golden):
    names = {k.split("/")[0] for k in golden.files}
    assert names == {c.name for c in CASES}
    assert len(golden.files) == 41


def test_xorshift_matches_oracle(orc):
    """The Python generator and the oracle's C generator give the same
    stream (both restate ops_check.c:33-42)."""
    r = opcases.XorShift()
    py = r.uniform(1000, -0.3, 0.3)
    orc.orc_rng_seed(opcases.SEED)
    c = np.zeros(1000, np.float32)
    orc.orc_rand_fill(fp(c), 1000, -0.3, 0.3)
    assert np.array_equal(py, c)
    assert orc.orc_rng_state() == r.s


def test_xorshift_known_values():
    """First raw states of xorshift64 (13, 7, 17) from the reference's seed,
    computed independently with Python integers."""
    s = opcases.SEED
    exp = []
    for _ in range(3):
        s ^= (s << 13) & ((1 << 64) - 1)
        s ^= s >> 7
        s ^= (s << 17) & ((1 << 64) - 1)
        exp.append(s)
    got = opcases.XorShift().raw(3)
    assert [int(v) for v in got] == exp


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_oracle_vs_golden(case, orc, golden):
    outs = opcases.oracle_run(orc, case)
    for name, got in outs.items():
        ref = golden[f"{case.name}/{name}"]
        assert got.size == ref.size, name
        assert np.isfinite(got).all()
        err = opcases.rel_err(got, ref)
        assert err <= opcases.TOL, f"{case.name}/{name}: {err:.2e}"


def test_oracle_catches_planted_error(orc, golden):
    """A plausible mistake planted in the oracle's inputs (bias dropped)
    must fail the golden check: the fixture discriminates."""
    c = opcases.all_cases()[0]
    c.inp["bias"] = np.zeros_like(c.inp["bias"])
    got = opcases.oracle_run(orc, c)["out"]
    assert opcases.rel_err(got, golden["gemm_small_nt/out"]) > 1e-2

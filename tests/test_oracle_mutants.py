"""The oracle's tests reject plausible mistakes in the oracle.

Each case plants one mistake in a temporary copy of oracle/jq_oracle.c (a
threshold off by one, a swapped operand, a dropped clause), compiles that copy
with gcc and runs the oracle-level tests against it in a fresh process
(JQ_ORACLE_LIB points the loader at the copy). Every copy must fail them: a
mistake of that kind in the oracle, repeated in the HIP kernels, would
otherwise pass every parity test. The reference facts that catch each one are
the restated known-answer tests (test_oracle_kats.py), the reference games'
vectors (test_oracle_reference_vectors.py) and the oracle's own golden
scenarios and invariants (test_oracle.py).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "oracle" / "jq_oracle.c"

# (area, reference, text in the oracle, planted replacement)
MUTANTS = [
    ("Q10 move-counter draw one early", "rules.py:444; state.py:1721-1724",
     "if (mc >= 4000 || mslc >= 200)", "if (mc >= 3999 || mslc >= 200)"),
    ("Q10 move-counter draw one late", "rules.py:444; state.py:1721-1724",
     "if (mc >= 4000 || mslc >= 200)", "if (mc >= 4001 || mslc >= 200)"),
    ("Q10 move-counter draw dropped", "rules.py:444; state.py:1721-1724",
     "if (mc >= 4000 || mslc >= 200)", "if (mslc >= 200)"),
    ("Q10 no-combat draw one early", "rules.py:445; state.py:1723-1724",
     "if (mc >= 4000 || mslc >= 200)", "if (mc >= 4000 || mslc >= 199)"),
    ("env move cap one late", "junqi_rl/env.py:295-305",
     "if (!term && nmc >= g->max_num_moves)", "if (!term && nmc > g->max_num_moves)"),
    ("engineers do not bomb each other", "rules.py:466-516",
     "if (a == d) return JQO_EV_BOMB;", "if (a == d && a != JQO_GONGB) return JQO_EV_BOMB;"),
    ("rank order inverted", "rules.py:466-516",
     "return a < d ? JQO_EV_EAT : JQO_EV_KILLED;", "return a > d ? JQO_EV_EAT : JQO_EV_KILLED;"),
    ("mine kills engineers too", "rules.py:466-516",
     "if (d == JQO_DILEI) return a == JQO_GONGB ? JQO_EV_EAT : JQO_EV_KILLED;",
     "if (d == JQO_DILEI) return JQO_EV_KILLED;"),
    ("move-counter Zobrist key index masked short", "_zobrist.py:73-122; state.py:1761-1811",
     "Z[ZOFF_MC + (nmc & 0xFFF)]", "Z[ZOFF_MC + (nmc & 0x7FF)]"),
    ("rank floor not raised by propagation", "combat_memory.py:354-569",
     "int prop = vf + 1 < 9 ? vf + 1 : 9;", "int prop = vf < 9 ? vf : 9;"),
    ("R6 names the wrong type", "info_model.py:271-429",
     "g->bcode[o][op] = BC_ONEHOT(JQO_JUNQI - 2);", "g->bcode[o][op] = BC_ONEHOT(JQO_DILEI - 2);"),
    ("left and right enemy swapped", "observation.cu:218-226; observation.py:155-232",
     "int tm = (obs + 2) & 3, le = (obs + 1) & 3, re = (obs + 3) & 3",
     "int tm = (obs + 2) & 3, le = (obs + 3) & 3, re = (obs + 1) & 3"),
    ("turn history from the wrong counter", "observation.py:1000-1021",
     "double dp = (double)g->mslc / 200.0;", "double dp = (double)g->move_counter / 200.0;"),
    ("straight rail run leaves its row", "move_gen.py:127-171",
     "if (sy == dy && ny != sy) continue;", "if (sy == dy && ny != sy && 0) continue;"),
]

TESTS = ["tests/test_oracle_kats.py", "tests/test_oracle_reference_vectors.py", "tests/test_oracle.py"]


CONTROL = ("unchanged copy", "-", "", "")


def _run(case, tmp: Path) -> tuple[int, str]:
    area, _, old, new = case
    src = SRC.read_text()
    if case is not CONTROL:
        assert src.count(old) == 1, f"{area}: the text to mutate is not unique in jq_oracle.c"
    d = tmp / ("control" if case is CONTROL else f"m{MUTANTS.index(case)}")
    d.mkdir()
    c = d / "jq_oracle.c"
    c.write_text(src if case is CONTROL else src.replace(old, new))
    so = d / "libjq_oracle.so"
    subprocess.run(["gcc", "-O1", "-fPIC", "-std=gnu11", "-fopenmp", "-shared", "-I", str(SRC.parent), "-o", str(so),
                    str(c), "-lm"], check=True, capture_output=True)
    env = dict(os.environ, JQ_ORACLE_LIB=str(so), OMP_NUM_THREADS="1")
    try:
        p = subprocess.run(["timeout", "-k", "5", "240", sys.executable, "-m", "pytest", "-q", "-x", "-p",
                            "no:cacheprovider", *TESTS], cwd=ROOT, env=env, capture_output=True, text=True,
                           timeout=260)
    except subprocess.TimeoutExpired:
        return 124, "timeout"
    return p.returncode, p.stdout[-400:]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc to build the oracle copies")
def test_planted_oracle_mistakes_fail_the_tests(tmp_path):
    with ThreadPoolExecutor(4) as ex:
        results = list(ex.map(lambda c: _run(c, tmp_path), [CONTROL] + MUTANTS))
    rc, out = results.pop(0)
    assert rc == 0, f"an unchanged copy of the oracle built the same way must pass: {out}"
    survived = [(case[0], case[1]) for case, (rc, _) in zip(MUTANTS, results) if rc == 0]
    assert not survived, f"planted mistakes the tests did not catch: {survived}"

"""Mutation campaign over the C oracle (run by hand; not collected by pytest).

    python tests/oracle_mutation_campaign.py [--workers 6] [--limit N] [--out DIR]

Every code line of oracle/jq_oracle.c is scanned for comparison operators
(>=, <=, >, <, ==, !=), logical operators (&&, ||), "+ 1" / "- 1" offsets and
"++" increments; each occurrence gives one mutant (>= -> >, < -> <=, == -> !=,
&& -> ||, + 1 -> + 2, ++ -> --, ...). Each mutant is compiled in its own copy
of oracle/ and run against the CPU tests that check the oracle (with -x, in a
fresh process, killed after 150 s: a mutant that hangs counts as caught). A
mutant the tests pass is printed as a survivor. The run writes one JSON line
per mutant to DIR/mutants.jsonl.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import shutil
import subprocess
import sys
import tempfile
from collections import Counter
from concurrent.futures import ProcessPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
SRC = (ROOT / "oracle" / "jq_oracle.c").read_text().split("\n")
OPS = [(r">=", ">"), (r"<=", "<"), (r"(?<![<>=!-])>(?![>=])", ">="), (r"(?<![<>=!])<(?![<=])", "<="),
       (r"==", "!="), (r"!=", "=="), (r"&&", "||"), (r"\|\|", "&&"), (r"\+ 1\b", "+ 2"), (r"- 1\b", "- 2"),
       (r"\+\+", "--")]
TESTS = ["tests/test_oracle_kats.py", "tests/test_oracle_reference_vectors.py", "tests/test_lib_cpu.py",
         "tests/test_oracle.py", "tests/test_oracle_symmetry.py", "tests/test_lib_validate.py",
         "tests/test_replay_cpu.py"]


def sites() -> list[tuple[int, int, int, str]]:
    out = []
    for i, line in enumerate(SRC):
        t = line.strip()
        if t.startswith(("//", "*", "/*", "#")):
            continue
        code = line.split("//")[0]
        for pat, rep in OPS:
            for m in re.finditer(pat, code):
                around = code[max(0, m.start() - 1):m.end() + 1]
                if "<<" in around or ">>" in around or "->" in around:
                    continue
                out.append((i, m.start(), m.end(), rep))
    return out


def run(args) -> list:
    k, (i, s, e, rep), work = args
    d = Path(work) / f"w{os.getpid()}"
    if not d.exists():
        d.mkdir(parents=True)
        for sub in ("oracle", "tests", "junqi_amd"):
            shutil.copytree(ROOT / sub, d / sub, ignore=shutil.ignore_patterns("_build", "__pycache__", "*.so"))
        shutil.copy(ROOT / "pytest.ini", d)
        (d / "junqi_amd" / "_build").mkdir(parents=True, exist_ok=True)
        lib = ROOT / "junqi_amd" / "_build" / "libjunqi_amd.so"
        if lib.exists():
            shutil.copy(lib, d / "junqi_amd" / "_build")
    lines = list(SRC)
    orig = lines[i]
    lines[i] = orig[:s] + rep + orig[e:]
    (d / "oracle" / "jq_oracle.c").write_text("\n".join(lines))
    so = d / "oracle" / "_build" / "libjq_oracle.so"
    so.parent.mkdir(parents=True, exist_ok=True)
    c = subprocess.run(["gcc", "-O1", "-fPIC", "-std=gnu11", "-fopenmp", "-shared", "-o", str(so),
                        str(d / "oracle" / "jq_oracle.c"), "-lm"], capture_output=True)
    if c.returncode:
        return [k, i + 1, orig.strip(), lines[i].strip(), "does not compile", ""]
    env = dict(os.environ, OMP_NUM_THREADS="1")
    try:
        p = subprocess.run(["timeout", "-k", "5", "150", sys.executable, "-m", "pytest", "-q", "-x", "-p",
                            "no:cacheprovider", *TESTS], cwd=d, capture_output=True, text=True, env=env, timeout=170)
    except subprocess.TimeoutExpired:
        return [k, i + 1, orig.strip(), lines[i].strip(), "caught", "hang"]
    if p.returncode in (124, 137):
        return [k, i + 1, orig.strip(), lines[i].strip(), "caught", "hang"]
    if p.returncode == 0:
        return [k, i + 1, orig.strip(), lines[i].strip(), "SURVIVED", ""]
    m = re.search(r"FAILED (\S+)", p.stdout)
    return [k, i + 1, orig.strip(), lines[i].strip(), "caught", m.group(1).split("::")[0] if m else "crash"]


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workers", type=int, default=6)
    ap.add_argument("--limit", type=int, default=0)
    ap.add_argument("--out", default=tempfile.gettempdir())
    a = ap.parse_args()
    out = Path(a.out)
    out.mkdir(parents=True, exist_ok=True)
    ss = sites()
    if a.limit:
        ss = ss[:a.limit]
    print(f"{len(ss)} mutants", flush=True)
    work = tempfile.mkdtemp(prefix="jq_mut_")
    res = []
    with ProcessPoolExecutor(a.workers) as ex, open(out / "mutants.jsonl", "w") as fh:
        for r in ex.map(run, [(k, s, work) for k, s in enumerate(ss)]):
            res.append(r)
            fh.write(json.dumps(r) + "\n")
            fh.flush()
            if r[4] == "SURVIVED":
                print("survivor:", r, flush=True)
    shutil.rmtree(work, ignore_errors=True)
    print(Counter(r[4] for r in res))
    print(Counter(r[5] for r in res if r[4] == "caught").most_common())
    return 1 if any(r[4] == "SURVIVED" for r in res) else 0


if __name__ == "__main__":
    sys.exit(main())

"""The oracle against vectors written by the reference's junqi_core.

tests/golden/reference_vectors.json holds 12 complete random games (seeds
0-3 x BRIGHT / DARK / HALF_DARK, 613-803 plies each, every one played to a
natural end) with, after every ply, the reference GameState's Zobrist hash
the acting seat's legal set before every ply and at the end (its size and a
digest of its sorted world ids, GameState.legal_actions, state.py:1200-1213),
and, at plies 0, 60, 150, 250, 400, 600 and the last, digests of all sixteen
combat-memory fields, every observer's BeliefTensor rows and remaining counts,
and every observer's float32 observation and globals. The file is written by
tests/golden/gen_reference_vectors.py; these are the parts no other fixture or
invariant reaches (Zobrist composition, late-game combat memory, DARK beliefs
after the opening, the W / N / E observations), and here they are compared bit
for bit.
"""

from __future__ import annotations

import hashlib
import json

import numpy as np
import pytest

from oracle import oracle as O
from tests import helpers as H

DOC = json.loads((H.GOLDEN / "reference_vectors.json").read_text())
MODE = {"BRIGHT": 0, "DARK": 1, "HALF_DARK": 2}
CM_MAP = {
    "direct_ate_my_pid_lo": ("cm_direct_lo", np.uint64), "direct_ate_my_pid_hi": ("cm_direct_hi", np.uint64),
    "direct_ate_my_type_mask": ("cm_direct_type", np.uint16), "last_direct_step": ("cm_last_direct", np.int16),
    "direct_other_count": ("cm_other_cnt", np.int16), "chain_pid_lo": ("cm_chain_lo", np.uint64),
    "chain_pid_hi": ("cm_chain_hi", np.uint64), "chain_ate_my_type_mask": ("cm_chain_type", np.uint16),
    "last_chain_step": ("cm_last_chain", np.int16), "eaten_by_pid_lo": ("cm_eaten_lo", np.uint64),
    "eaten_by_pid_hi": ("cm_eaten_hi", np.uint64), "rank_floor": ("cm_floor", np.int8),
    "rank_floor_step": ("cm_floor_step", np.int16), "is_gongb": ("cm_is_gongb", np.bool_),
    "not_gongb": ("cm_not_gongb", np.bool_), "attacked_by_known_gongb": ("cm_atk_gongb", np.bool_),
}


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def legal_digest(ids: np.ndarray) -> str:
    """The generator's digest: SHA-256 of the sorted ids as little-endian int32, 16 hex digits."""
    return sha(np.sort(np.asarray(ids, dtype="<i4")))[:16]


def check_point(g: O.Game, cp: dict, ctx: str) -> None:
    for ref_name, (name, dt) in CM_MAP.items():
        assert sha(np.asarray(g.buf[0][name]).astype(dt)) == cp["cm"][ref_name], f"{ctx}: combat memory {ref_name}"
    for s in range(4):
        probs = np.zeros((120, 12), np.float32)
        for pid in range(120):
            if g.alive[pid]:
                probs[pid] = O.belief_row(int(g.bcode[s, pid]))
        assert sha(probs) == cp["beliefs"][s], f"{ctx}: beliefs of observer {s}"
        rem = np.where(g.rem_tracked[s][:, None] != 0, g.rem[s], 0)
        assert rem.tolist() == cp["remaining"][s], f"{ctx}: remaining counts of observer {s}"
        sp, gl = g.observe(s)
        assert sha(sp) == cp["obs_f32"][s], f"{ctx}: observation of seat {s}"
        assert sha(gl) == cp["glob_f32"][s], f"{ctx}: globals of seat {s}"


@pytest.mark.parametrize("rec", DOC["games"], ids=[f"seed{r['seed']}-{r['show_mode']}" for r in DOC["games"]])
def test_reference_game(rec):
    setup = np.asarray(rec["setup"], np.int8)
    assert np.array_equal(setup, O.random_setup(rec["seed"]))   # the setup stream, too
    g = O.Game(setup, show_mode=MODE[rec["show_mode"]])
    cps = {cp["ply"]: cp for cp in rec["checkpoints"]}
    check_point(g, cps[0], "ply 0")
    for ply, ((src, dst), z) in enumerate(zip(rec["actions"], rec["zobrist"]), start=1):
        ids = g.legal_ids()
        assert len(ids) == rec["legal_count"][ply - 1], f"before ply {ply}: legal count"
        assert legal_digest(ids) == rec["legal_digest"][ply - 1], f"before ply {ply}: legal set"
        rc, _ = g.step(src, dst)
        assert rc == 0, f"ply {ply}: reference action rejected"
        assert format(int(g.zobrist), "016x") == z, f"ply {ply}: Zobrist hash"
        if ply in cps:
            check_point(g, cps[ply], f"ply {ply}")
    assert bool(g.terminated) == rec["terminated"]
    ids = g.legal_ids()
    assert len(rec["legal_count"]) == len(rec["actions"]) + 1
    assert len(ids) == rec["legal_count"][-1] and legal_digest(ids) == rec["legal_digest"][-1], "end position"
    assert len(cps) >= 6

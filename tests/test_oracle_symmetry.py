"""Four-fold rotation symmetry of the rules, checked on the oracle.

The board maps onto itself under the quarter turn R(x, y) = (16 - y, x), which
carries seat s's local index i to seat s + 1's local index i
(board.py:88-102). Relabel every seat s -> s + 1 and every pid p -> p + 30
(mod 120); the two teams swap. The rules (state.py, combat_memory.py,
info_model.py) never refer to an absolute seat or direction, so playing a game
and playing its rotation with rotated actions must stay rotations of each
other at every ply, and the observation of seat s + 1 in the rotated game must
equal the observation of seat s in the original (each is in its observer's
canonical frame). The observation hashes pin the SOUTH observer only; this
carries that pin to WEST, NORTH and EAST: a mistake in one frame (a wrong
rotation, left and right enemy swapped) breaks the equality. The Zobrist hash
is keyed by absolute pids and cells, so it is the one field left out.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O

PID_FIELDS = ("alive", "ptype", "move_count", "active_eat", "passive_surv", "death_reason", "death_step")
CM_SCALAR = ("cm_direct_type", "cm_last_direct", "cm_other_cnt", "cm_chain_type", "cm_last_chain", "cm_floor",
             "cm_floor_step", "cm_is_gongb", "cm_not_gongb", "cm_atk_gongb", "bcode")
CM_SETS = (("cm_direct_lo", "cm_direct_hi"), ("cm_chain_lo", "cm_chain_hi"), ("cm_eaten_lo", "cm_eaten_hi"))
PERM = (np.arange(120) + 30) % 120          # new pid of old pid p


def rot_cell(f: int) -> int:
    if f < 0:
        return f
    x, y = f % 17, f // 17
    return x * 17 + (16 - y)                # R(x, y) = (16 - y, x) -> flat y' * 17 + x'


def rot_set(lo: np.ndarray, hi: np.ndarray):
    """A 120-bit pid set (lo: pids 0-63, hi: 64-119) with every pid p -> p + 30."""
    lo = lo.astype(np.uint64)
    hi = hi.astype(np.uint64)
    nlo = np.zeros_like(lo)
    nhi = np.zeros_like(hi)
    for p in range(120):
        src = (lo >> np.uint64(p)) & np.uint64(1) if p < 64 else (hi >> np.uint64(p - 64)) & np.uint64(1)
        q = int(PERM[p])
        if q < 64:
            nlo |= src << np.uint64(q)
        else:
            nhi |= src << np.uint64(q - 64)
    return nlo, nhi


def rotate_game(g: O.Game) -> O.Game:
    a = g.buf[0]
    r = O.Game(None)
    b = r.buf[0]
    b["show_mode"] = a["show_mode"]
    b["max_num_moves"] = a["max_num_moves"]
    for k in PID_FIELDS:
        b[k][PERM] = a[k]
    b["pseat"][PERM] = np.where(a["pseat"] >= 0, (a["pseat"].astype(np.int32) + 1) % 4, -1)
    for p in range(120):
        q = PERM[p]
        for fx, fy in (("pos_x", "pos_y"), ("zero_x", "zero_y")):
            x, y = int(a[fx][p]), int(a[fy][p])
            if x >= 0 and y >= 0:
                b[fx][q], b[fy][q] = 16 - y, x
            else:
                b[fx][q], b[fy][q] = x, y
        b["death_loc"][q] = rot_cell(int(a["death_loc"][p]))
    b["cell_pid"][:] = -1
    for f in range(289):
        p = int(a["cell_pid"][f])
        if p >= 0:
            b["cell_pid"][rot_cell(f)] = PERM[p]
    b["seat_dead"] = np.roll(a["seat_dead"], 1)
    b["flag_rev"] = np.roll(a["flag_rev"], 1)
    b["turn"] = (int(a["turn"]) + 1) % 4
    b["terminated"] = a["terminated"]
    b["draw"] = a["draw"]
    b["winner"] = -1 if a["winner"] < 0 else 1 - int(a["winner"])
    b["move_counter"] = a["move_counter"]
    b["mslc"] = a["mslc"]
    b["hist_len"] = a["hist_len"]
    for i in range(32):
        b["hist"][i] = [rot_cell(int(a["hist"][i][0])) if i < a["hist_len"] else a["hist"][i][0],
                        rot_cell(int(a["hist"][i][1])) if i < a["hist_len"] else a["hist"][i][1]]
    for k in CM_SCALAR:
        for o in range(4):
            b[k][(o + 1) % 4][PERM] = a[k][o]
    for klo, khi in CM_SETS:
        for o in range(4):
            nlo, nhi = rot_set(a[klo][o], a[khi][o])
            b[klo][(o + 1) % 4][PERM] = nlo
            b[khi][(o + 1) % 4][PERM] = nhi
    for o in range(4):
        for s in range(4):
            b["rem_tracked"][(o + 1) % 4][(s + 1) % 4] = a["rem_tracked"][o][s]
            b["rem"][(o + 1) % 4][(s + 1) % 4] = a["rem"][o][s]
    b["zobrist"] = np.uint64(r.recompute_zobrist())
    return r


def assert_same_state(x: O.Game, y: O.Game, ctx: str) -> None:
    for name in O.GAME_DTYPE.names:
        if name in ("zobrist", "pad_"):
            continue
        if name == "hist":
            n = int(x.buf[0]["hist_len"])
            assert np.array_equal(x.buf[0]["hist"][:n], y.buf[0]["hist"][:n]), f"{ctx}: hist"
            continue
        assert np.array_equal(x.buf[0][name], y.buf[0][name]), f"{ctx}: field {name} differs"


def rot_action(a: int) -> int:
    return rot_cell(a // 289) * 289 + rot_cell(a % 289)


def test_rotation_of_a_new_game_is_the_new_game_of_the_rotated_setup():
    setup = O.random_setup(21)
    g = O.Game(setup, show_mode=2)
    rs = np.roll(setup.reshape(4, 30), 1, axis=0).reshape(120)   # seat s's lineup to seat s + 1
    h = O.Game(rs, show_mode=2)
    r = rotate_game(g)
    h.buf[0]["turn"] = r.buf[0]["turn"]        # a new game starts with SOUTH; the rotation with WEST
    assert_same_state(r, h, "opening")


@pytest.mark.parametrize("seed,show_mode", [(s, m) for s in (1, 2, 3) for m in (0, 1, 2)])
def test_play_commutes_with_rotation(seed, show_mode):
    g = O.Game(O.random_setup(seed), show_mode=show_mode)
    r = rotate_game(g)
    rng = np.random.default_rng(seed)
    for ply in range(260):
        if g.terminated:
            break
        ids = g.legal_ids()
        rids = r.legal_ids()
        assert np.array_equal(np.sort([rot_action(int(a)) for a in ids]), rids), f"ply {ply}: legal sets"
        for s in range(4):
            sp, gl = g.observe(s)
            rsp, rgl = r.observe((s + 1) % 4)
            assert np.array_equal(sp, rsp), f"ply {ply}: observation of seat {s} vs {(s + 1) % 4}"
            assert np.array_equal(gl, rgl), f"ply {ply}: globals of seat {s}"
        a = int(ids[rng.integers(len(ids))])
        rc, res = g.step_id(a)
        rrc, rres = r.step_id(rot_action(a))
        assert rc == rrc == 0
        for k in ("valid", "event", "flag_reveal_src", "flag_reveal_dst", "flag_captured", "terminated", "draw",
                  "gongb_revealed"):
            assert res[k] == rres[k], f"ply {ply}: {k}"
        died = res["seats_died_mask"]
        assert rres["seats_died_mask"] == (((died << 1) | (died >> 3)) & 15)
        assert rres["winner"] == (-1 if res["winner"] < 0 else 1 - res["winner"])
        assert_same_state(rotate_game(g), r, f"ply {ply}")
        assert int(r.zobrist) == r.recompute_zobrist()

"""Known-answer tests of the reference, restated against the C oracle.

Each block follows one reference test file and checks the same facts through
the oracle's own entry points (jqo_world_to_canonical, jqo_validate_lineup,
jqo_cm_apply_event, jqo_step, jqo_observe, the belief codes), so that the
parts the observation hashes cannot reach (the W / N / E frames, combat-memory
rules, belief rules in every show mode, setup validation, the sampler's
generator) are pinned by facts the reference itself asserts:

* rotation: tests/test_rotation.py:35-219
* setup validation: tests/test_setup_validation.py:29-62 over the 8 golden
  setup_validation scenarios
* combat memory v6 (eaten-by reverse projection): tests/test_observation_combat_memory_v6.py:128-329
* combat memory rules A1 / B1 / floor / known-engineer / chain / DARK:
  tests/test_combat_memory.py:46-283
* beliefs I1-I5 and R1-R7: tests/test_info_model.py:79-510,
  tests/test_belief_tensor.py:139-224
* Philox4x32-10: the Random123 known-answer vectors (kat_vectors, philox4x32_10)
"""

from __future__ import annotations

import json

import numpy as np
import pytest

from oracle import oracle as O
from tests import helpers as H

SOUTH, WEST, NORTH, EAST = 0, 1, 2, 3
T = H.TYPE_OF
PIECE_COUNTS = {2: 1, 3: 3, 4: 2, 5: 1, 6: 1, 7: 2, 8: 2, 9: 2, 10: 2, 11: 3, 12: 3, 13: 3}
CH = {}
_c = 0
for _name, _n in H.CHANNEL_GROUPS:
    CH[_name] = (_c, _c + _n)
    _c += _n


@pytest.fixture(scope="module", autouse=True)
def _lib():
    O.lib()


def teammate(s):
    return (s + 2) & 3


def left_enemy(s):
    return (s + 1) & 3


def right_enemy(s):
    return (s + 3) & 3


# ====================================================================== rotation
# tests/test_rotation.py

@pytest.mark.parametrize("seat", range(4))
def test_point_round_trip(seat):
    for y in range(17):
        for x in range(17):
            c = O.world_to_canonical(x, y, seat)
            assert O.canonical_to_world(*c, seat) == (x, y)


@pytest.mark.parametrize("seat,center", [(SOUTH, (8, 13)), (WEST, (3, 8)), (NORTH, (8, 3)), (EAST, (13, 8))])
def test_seat_center_maps_to_canonical_home(seat, center):
    assert O.world_to_canonical(*center, seat) == (8, 13)
    # the centre camp is local index 12 of each seat (board.py:88-102)
    assert O.index_to_pos(seat, 12) == center


@pytest.mark.parametrize("seat", range(4))
def test_teammate_top_enemies_sides(seat):
    _, yc = O.world_to_canonical(*O.index_to_pos(teammate(seat), 0), seat)
    assert yc <= 5
    for enemy in (left_enemy(seat), right_enemy(seat)):
        xc, yc = O.world_to_canonical(*O.index_to_pos(enemy, 0), seat)
        assert 6 <= yc <= 10 and (xc <= 5 or xc >= 11)
    assert O.world_to_canonical(*O.index_to_pos(right_enemy(seat), 0), seat)[0] >= 11
    assert O.world_to_canonical(*O.index_to_pos(left_enemy(seat), 0), seat)[0] <= 5


@pytest.mark.parametrize("seat", range(4))
def test_whole_seats_land_in_their_canonical_zones(seat):
    """Every cell of a seat, not only its corner: own at the bottom, teammate at
    the top, left enemy on the left, right enemy on the right."""
    for i in range(30):
        assert O.world_to_canonical(*O.index_to_pos(seat, i), seat)[1] >= 11
        assert O.world_to_canonical(*O.index_to_pos(teammate(seat), i), seat)[1] <= 5
        assert O.world_to_canonical(*O.index_to_pos(left_enemy(seat), i), seat)[0] <= 5
        assert O.world_to_canonical(*O.index_to_pos(right_enemy(seat), i), seat)[0] >= 11
        # seat-local index i sits at the same canonical cell for every seat
        assert (O.world_to_canonical(*O.index_to_pos(seat, i), seat)
                == O.world_to_canonical(*O.index_to_pos(SOUTH, i), SOUTH))


@pytest.mark.parametrize("seat", range(4))
def test_observation_rotation_is_world_to_canonical(seat):
    """The observation's planes are the world planes moved by world_to_canonical
    (rotate_plane consistency, tests/test_rotation.py:140-158): every own piece
    lights its piece_own plane exactly at its rotated cell."""
    g = O.Game(O.random_setup(11), show_mode=2)
    sp, _ = g.observe(seat)
    own = np.zeros((12, 17, 17), np.float32)
    for pid in range(seat * 30, seat * 30 + 30):
        if g.alive[pid]:
            cx, cy = O.world_to_canonical(int(g.pos_x[pid]), int(g.pos_y[pid]), seat)
            own[int(g.ptype[pid]) - 2, cy, cx] = 1
    assert np.array_equal(sp[0:12], own)


def test_topology_symmetry():
    t = O.tables()
    role = np.zeros(289, np.int8)
    for f in range(289):
        if not t["on_board"][f]:
            role[f] = 0
        elif t["camp"][f]:
            role[f] = 1
        elif t["stronghold"][f]:
            role[f] = 2
        elif t["ninegrid"][f]:
            role[f] = 4
        elif t["rail"][f]:
            role[f] = 3
        else:
            role[f] = 5
    for seat in range(4):
        rot = np.zeros(289, np.int8)
        for f in range(289):
            cx, cy = O.world_to_canonical(f % 17, f // 17, seat)
            rot[cy * 17 + cx] = role[f]
        assert np.array_equal(rot, role)


@pytest.mark.parametrize("seat", range(4))
def test_canonical_action_codec_is_a_bijection(seat):
    """Every (src, dst) pair of on-board cells has one compact canonical id in
    [0, 16641), all distinct, and the id decodes back through canonical_to_world
    (action round trip, tests/test_rotation.py:182-189)."""
    t = O.tables()
    c2f = t["compact_to_flat"]
    on = [f for f in range(289) if t["on_board"][f]]
    seen = set()
    for src in on:
        for dst in on:
            c = O.canonical_id(seat, src * 289 + dst)
            assert 0 <= c < 129 * 129 and c not in seen
            seen.add(c)
            fs, fd = int(c2f[c // 129]), int(c2f[c % 129])
            assert O.canonical_to_world(fs % 17, fs // 17, seat) == (src % 17, src // 17)
            assert O.canonical_to_world(fd % 17, fd // 17, seat) == (dst % 17, dst // 17)
    assert len(seen) == 129 * 129


# ============================================================ setup validation
# tests/test_setup_validation.py over tests/golden/setup_validation/*.json

_SETUP_CASES = H.scenario_files("setup_validation")


@pytest.mark.parametrize("path", _SETUP_CASES, ids=[p.stem for p in _SETUP_CASES])
def test_setup_validation_golden(path):
    su = json.loads(path.read_text())["setup_only"]
    lu = [T[name] for name in su["lineups"][0]]
    got = O.validate_lineup(lu)
    assert (not got) == su["expect_valid"], (path.stem, got)
    assert set(su.get("expect_violations", [])) <= got, (path.stem, got)
    for other in su["lineups"][1:]:   # the template seats are valid
        assert O.validate_lineup([T[n] for n in other]) == set()


def test_setup_validation_each_rule():
    """One violation at a time on a valid lineup: each rule fires alone."""
    good = np.asarray(O.random_setup(5)[:30], np.int64)
    assert O.validate_lineup(good) == set()
    flag = int(np.where(good == T["JUNQI"])[0][0])
    other_sh = 26 if flag == 28 else 28

    def swap(a, i, j):
        b = a.copy()
        b[i], b[j] = b[j], b[i]
        return b

    piece_at_front = int(np.where((good != 0) & (np.arange(30) < 5))[0][0])
    assert O.validate_lineup(swap(good, 6, 0)) >= {"C1"}          # a piece into camp 6
    assert O.validate_lineup(swap(good, flag, 0)) >= {"C2"}       # flag out of the strongholds
    assert O.validate_lineup(swap(good, flag, other_sh)) == set() # the other stronghold is fine
    dilei = int(np.where(good == T["DILEI"])[0][0])
    assert O.validate_lineup(swap(good, dilei, piece_at_front)) >= {"C3"}
    zhadan = int(np.where(good == T["ZHADAN"])[0][0])
    bad = swap(good, zhadan, piece_at_front)
    assert "C4" in O.validate_lineup(bad)
    extra = good.copy()
    extra[int(np.where(good == T["PAIZH"])[0][0])] = T["SILING"]
    assert O.validate_lineup(extra) == {"C5"}
    dark = good.copy()
    dark[int(np.where(good == T["PAIZH"])[0][0])] = T["DARK"]
    assert O.validate_lineup(dark) == {"C5"}
    assert O.validate_lineup(np.where(np.arange(30) == 3, 14, good)) == {"TYPE"}
    assert O.validate_lineup(np.where(np.arange(30) == 3, -1, good)) == {"TYPE"}
    assert O.validate_lineup(good[:29]) == {"LENGTH"}


@pytest.mark.parametrize("seed", range(40))
def test_generated_setups_are_valid(seed):
    s = O.random_setup(seed)
    for seat in range(4):
        assert O.validate_lineup(s[30 * seat:30 * seat + 30]) == set()


# ============================================================ combat memory v6
# tests/test_observation_combat_memory_v6.py

def _bit(pid):
    return (pid < 64, np.uint64(1) << np.uint64(pid if pid < 64 else pid - 64))


def _has(g, field, obs, pid, bit_pid):
    lo, b = _bit(bit_pid)
    arr = g.buf[0][field + ("_lo" if lo else "_hi")]
    return (arr[obs, pid] & b) == b


def _hand_state_after_eat():
    """SOUTH pid 20 (PAIZH) eaten by EAST pid 110 (LIANZH), DARK mode."""
    pieces = [(28, T["JUNQI"], 8, 16), (20, T["PAIZH"], 10, 16), (21, T["PAIZH"], 7, 16),
              (22, T["LIANZH"], 6, 16), (0, T["SILING"], 9, 13), (56, T["JUNQI"], 0, 8),
              (86, T["JUNQI"], 8, 0), (116, T["JUNQI"], 16, 10), (110, T["LIANZH"], 13, 8)]
    g = O.Game.from_pieces(pieces, turn=EAST, move_counter=10, show_mode=1)
    g.cm_apply_event(is_eat=True, attacker_pid=110, defender_pid=20, attacker_seat=EAST, defender_seat=SOUTH,
                     attacker_type=T["LIANZH"], defender_type=T["PAIZH"], step=8)
    return g


def test_eaten_by_pid_writes_killer_bit_for_observer_own_pid():
    g = _hand_state_after_eat()
    assert _has(g, "cm_eaten", SOUTH, 20, 110)
    assert g.cm_eaten_lo[SOUTH, 20] == 0
    for obs in (WEST, NORTH, EAST):
        assert g.cm_eaten_lo[obs, 20] == 0 and g.cm_eaten_hi[obs, 20] == 0


def test_eaten_by_pid_channel_lights_at_victim_cell():
    g = _hand_state_after_eat()
    sp, _ = g.observe(SOUTH)
    e0, e1 = CH["cm_eaten_by_pid"]
    eaten = sp[e0:e1]
    cx, cy = O.world_to_canonical(10, 16, SOUTH)
    assert eaten[50, cy, cx] == 1.0          # right enemy (EAST) slot 20 = pid 110
    assert eaten[:, cy, cx].sum() == 1.0
    for x, y in ((7, 16), (6, 16), (9, 13)):   # innocent SOUTH pids 21, 22, 0
        cx, cy = O.world_to_canonical(x, y, SOUTH)
        assert eaten[:, cy, cx].sum() == 0.0
    assert eaten.sum() == 1.0
    for observer in (WEST, NORTH, EAST):      # DARK boundary: no leak across observers
        sp, _ = g.observe(observer)
        assert sp[e0:e1].sum() == 0.0


def test_eaten_by_pid_chain_propagates_to_new_killer():
    g = O.Game.from_pieces([], show_mode=1)
    g.cm_apply_event(is_eat=True, attacker_pid=110, defender_pid=20, attacker_seat=EAST, defender_seat=SOUTH,
                     attacker_type=T["LIANZH"], defender_type=T["PAIZH"], step=5)
    assert _has(g, "cm_eaten", SOUTH, 20, 110)
    g.cm_apply_event(is_eat=True, attacker_pid=0, defender_pid=110, attacker_seat=SOUTH, defender_seat=EAST,
                     attacker_type=T["SILING"], defender_type=T["LIANZH"], step=12)
    assert _has(g, "cm_eaten", SOUTH, 20, 0)
    assert _has(g, "cm_eaten", SOUTH, 20, 110)
    for obs in (WEST, NORTH, EAST):
        assert g.cm_eaten_lo[obs, 20] == 0 and g.cm_eaten_hi[obs, 20] == 0


def test_dark_boundary_no_eaten_by_pid_for_non_observer_own():
    g = O.Game.from_pieces([], show_mode=1)
    g.cm_apply_event(is_eat=True, attacker_pid=110, defender_pid=40, attacker_seat=EAST, defender_seat=WEST,
                     attacker_type=T["LIANZH"], defender_type=T["PAIZH"], step=5)
    assert _has(g, "cm_eaten", WEST, 40, 110)
    for obs in (SOUTH, NORTH, EAST):
        assert g.cm_eaten_lo[obs, 40] == 0 and g.cm_eaten_hi[obs, 40] == 0


def test_layer4_is_the_final_group():
    e0, e1 = CH["cm_eaten_by_pid"]
    assert e1 == 317 and e1 - e0 == 60 and e0 == CH["cm_recency"][1]


# ============================================================ combat memory v4
# tests/test_combat_memory.py

def _ti(name):
    return 1 << (T[name] - 2)


def _cm():
    return O.Game.from_pieces([], show_mode=1)


def test_eat_my_dilei_marks_killer_as_gongb():
    g = _cm()
    g.cm_apply_event(is_eat=True, attacker_pid=37, defender_pid=12, attacker_seat=WEST, defender_seat=SOUTH,
                     attacker_type=T["GONGB"], defender_type=T["DILEI"], step=10)
    assert g.cm_is_gongb[SOUTH, 37] and not g.cm_not_gongb[SOUTH, 37]
    assert g.cm_floor[SOUTH, 37] == 0
    for other in (WEST, NORTH, EAST):
        assert not g.cm_is_gongb[other, 37]
        assert g.cm_other_cnt[other, 37] == 1


def test_eat_my_paizh_excludes_gongb():
    g = _cm()
    g.cm_apply_event(is_eat=True, attacker_pid=37, defender_pid=12, attacker_seat=WEST, defender_seat=SOUTH,
                     attacker_type=T["LIANZH"], defender_type=T["PAIZH"], step=5)
    assert g.cm_not_gongb[SOUTH, 37] and not g.cm_is_gongb[SOUTH, 37]
    assert g.cm_floor[SOUTH, 37] == 3
    assert g.cm_direct_type[SOUTH, 37] & _ti("PAIZH")
    assert g.cm_direct_lo[SOUTH, 37] == np.uint64(1) << np.uint64(12)


def test_my_paizh_dies_attacking_lifts_floor_to_lianzh():
    g = _cm()
    g.cm_apply_event(is_eat=False, attacker_pid=12, defender_pid=37, attacker_seat=SOUTH, defender_seat=WEST,
                     attacker_type=T["PAIZH"], defender_type=T["SILING"], step=20)
    assert g.cm_floor[SOUTH, 37] == 3
    assert g.cm_direct_type[SOUTH, 37] & _ti("PAIZH")
    assert g.cm_other_cnt[WEST, 37] == 1


def test_known_gongb_attack_flags_defender():
    g = _cm()
    g.cm_path_revealed_gongb(18)
    for obs in range(4):
        assert g.cm_is_gongb[obs, 18] and not g.cm_is_gongb[obs, 0]
    g.cm_apply_event(is_eat=False, attacker_pid=18, defender_pid=44, attacker_seat=SOUTH, defender_seat=WEST,
                     attacker_type=T["GONGB"], defender_type=T["LIANZH"], step=15)
    for obs in range(4):
        assert g.cm_atk_gongb[obs, 44]


def test_unknown_attacker_does_not_flag():
    g = _cm()
    g.cm_apply_event(is_eat=False, attacker_pid=12, defender_pid=44, attacker_seat=SOUTH, defender_seat=WEST,
                     attacker_type=T["PAIZH"], defender_type=T["LIANZH"], step=20)
    for obs in range(4):
        assert not g.cm_atk_gongb[obs, 44]


def test_own_engineer_attack_flags_only_for_its_seat():
    """An unrevealed GONGB attacker is known as one only to its own seat
    (the attacker-seat observer, combat_memory.py:396-408)."""
    g = _cm()
    g.cm_apply_event(is_eat=False, attacker_pid=18, defender_pid=44, attacker_seat=SOUTH, defender_seat=WEST,
                     attacker_type=T["GONGB"], defender_type=T["LIANZH"], step=15)
    assert [bool(g.cm_atk_gongb[o, 44]) for o in range(4)] == [True, False, False, False]


def test_two_step_chain():
    g = _cm()
    g.cm_apply_event(is_eat=True, attacker_pid=37, defender_pid=12, attacker_seat=WEST, defender_seat=SOUTH,
                     attacker_type=T["LIANZH"], defender_type=T["PAIZH"], step=10)
    g.cm_apply_event(is_eat=True, attacker_pid=87, defender_pid=37, attacker_seat=NORTH, defender_seat=WEST,
                     attacker_type=T["YINGZH"], defender_type=T["LIANZH"], step=15)
    assert g.cm_chain_lo[SOUTH, 87] & (np.uint64(1) << np.uint64(12))
    assert g.cm_chain_type[SOUTH, 87] & _ti("PAIZH")
    assert g.cm_floor[SOUTH, 87] >= 4
    for obs in (WEST, NORTH, EAST):
        assert g.cm_chain_lo[obs, 87] & (np.uint64(1) << np.uint64(37))


def test_my_eat_does_not_leak_type_to_others():
    g = _cm()
    g.cm_apply_event(is_eat=True, attacker_pid=11, defender_pid=40, attacker_seat=SOUTH, defender_seat=WEST,
                     attacker_type=T["LIANZH"], defender_type=T["PAIZH"], step=8)
    assert g.cm_direct_type[WEST, 11] & _ti("PAIZH")
    assert g.cm_floor[WEST, 11] == 3
    assert g.cm_direct_type[SOUTH, 11] == 0
    assert g.cm_other_cnt[SOUTH, 11] == 1
    assert g.cm_floor[SOUTH, 11] == 0


@pytest.mark.parametrize("name,floor", [("GONGB", 2), ("PAIZH", 3), ("SHIZH", 8), ("SILING", 9),
                                        ("JUNQI", 0), ("DILEI", 0), ("ZHADAN", 0)])
def test_next_floor_after_eat(name, floor):
    """next_floor_after_eat (combat_memory.py:160-172) as the floor a KILLED
    attacker of that type leaves on the survivor for the attacker's seat."""
    g = _cm()
    g.cm_apply_event(is_eat=False, attacker_pid=12, defender_pid=44, attacker_seat=SOUTH, defender_seat=WEST,
                     attacker_type=T[name], defender_type=T["SILING"], step=3)
    assert g.cm_floor[SOUTH, 44] == floor
    assert g.cm_floor_step[SOUTH, 44] == (3 if floor else -1)


@pytest.mark.parametrize("seat", range(4))
def test_back_two_rows_through_dilei_candidate(seat):
    """is_in_seat_back_two_rows (tests/test_combat_memory.py:222-229): at the
    opening, cm_dilei_candidate marks exactly the enemy pieces on their seat's
    local indices 20-29 and cm_my_dilei_candidate the observer's own."""
    g = O.Game(O.random_setup(3 + seat), show_mode=2)
    sp, _ = g.observe(seat)
    want_enemy = np.zeros((17, 17), np.float32)
    want_own = np.zeros((17, 17), np.float32)
    for s in range(4):
        for i in range(20, 30):
            pid = s * 30 + i
            if not g.alive[pid]:
                continue
            cx, cy = O.world_to_canonical(*O.index_to_pos(s, i), seat)
            if (s & 1) != (seat & 1):
                want_enemy[cy, cx] = 1
            elif s == seat:
                want_own[cy, cx] = 1
    assert np.array_equal(sp[CH["cm_dilei_candidate"][0]], want_enemy)
    assert np.array_equal(sp[CH["cm_my_dilei_candidate"][0]], want_own)


# ================================================================ beliefs
# tests/test_info_model.py, tests/test_belief_tensor.py

def _row(g, obs, pid):
    return O.belief_row(int(g.bcode[obs, pid]))


def _one_hot(v):
    return int((v == 1.0).sum()) == 1 and float(v.sum()) == 1.0


def _rem(g, obs, seat):
    if not g.rem_tracked[obs, seat]:
        return None
    return {t + 2: int(g.rem[obs, seat, t]) for t in range(12)}


def _opening(seed, show_mode=2):
    return O.Game(O.random_setup(seed), show_mode=show_mode)


def _pieces(spec):
    """(seat, type name, x, y) -> (pid, type, x, y): pid = seat*30 + lowest free
    slot in order (state.py:393-427)."""
    used = {s: 0 for s in range(4)}
    out = []
    for s, name, x, y in spec:
        out.append((s * 30 + used[s], T[name], x, y))
        used[s] += 1
    return out


def _pid_at(g, x, y):
    return int(g.cell_pid[y * 17 + x])


def test_initial_sums_to_one_and_own_one_hot():
    g = _opening(42)
    for pid in range(120):
        if g.alive[pid]:
            v = _row(g, SOUTH, pid)
            assert abs(float(v.sum()) - 1.0) < 1e-5 and (v >= 0).all()
    g = _opening(1)
    for pid in range(30):
        if g.alive[pid]:
            v = _row(g, SOUTH, pid)
            assert _one_hot(v) and v[int(g.ptype[pid]) - 2] == 1.0


def test_initial_teammate_one_hot_in_half_dark_and_enemy_distributions():
    g = _opening(2)
    assert sum(_one_hot(_row(g, SOUTH, p)) for p in range(60, 90) if g.alive[p]) == 25
    g = _opening(3)
    nontrivial = 0
    for p in list(range(30, 60)) + list(range(90, 120)):
        if g.alive[p]:
            v = _row(g, SOUTH, p)
            assert v[int(g.ptype[p]) - 2] > 0
            nontrivial += not _one_hot(v)
    assert nontrivial >= 20


def test_initial_bright_all_one_hot_and_dark_hides_teammate():
    g = _opening(4, show_mode=0)
    for obs in range(4):
        assert all(_one_hot(_row(g, obs, p)) for p in range(120) if g.alive[p])
    g = _opening(4, show_mode=1)
    for obs in range(4):
        for p in range(120):
            if g.alive[p]:
                assert _one_hot(_row(g, obs, p)) == (p // 30 == obs)


def test_initial_remaining_only_for_enemies():
    g = _opening(5)
    for obs in range(4):
        for s in range(4):
            if s == obs or (s & 1) == (obs & 1):
                assert _rem(g, obs, s) is None
            else:
                assert _rem(g, obs, s) == PIECE_COUNTS


def test_initial_prior_constraints():
    """Strongholds carry JUNQI mass; DILEI and ZHADAN have none on the front row;
    JUNQI has none off the strongholds (info_model.py:69-138)."""
    for seed in (6, 7, 8, 9):
        g = _opening(seed)
        for enemy in (WEST, EAST):
            for i in range(30):
                pid = enemy * 30 + i
                if not g.alive[pid] or i in (6, 8, 12, 16, 18):
                    continue
                v = _row(g, SOUTH, pid)
                if i in (26, 28):
                    assert v[T["JUNQI"] - 2] > 0
                else:
                    assert v[T["JUNQI"] - 2] == 0
                if i < 5:
                    assert v[T["DILEI"] - 2] == 0 and v[T["ZHADAN"] - 2] == 0


def _hand(spec, turn=SOUTH, show_mode=2):
    return O.Game.from_pieces(_pieces(spec), turn=turn, show_mode=show_mode)


def _move(g, src, dst):
    rc, r = g.step(src[1] * 17 + src[0], dst[1] * 17 + dst[0])
    assert rc == 0
    return r


def test_r1_move_migrates_belief():
    g = _hand([(SOUTH, "PAIZH", 8, 11)])
    _move(g, (8, 11), (8, 12))
    assert _pid_at(g, 8, 11) < 0
    pid = _pid_at(g, 8, 12)
    assert pid >= 0 and _one_hot(_row(g, SOUTH, pid))


def test_r1_eat_migrates_and_keeps_inventory():
    g = _hand([(SOUTH, "SILING", 6, 11), (WEST, "PAIZH", 6, 10), (WEST, "LIANZH", 5, 8)])
    r = _move(g, (6, 11), (6, 10))
    assert r["event"] == 2
    assert _pid_at(g, 6, 11) < 0
    assert _one_hot(_row(g, SOUTH, _pid_at(g, 6, 10)))
    assert _rem(g, SOUTH, WEST)[T["PAIZH"]] == PIECE_COUNTS[T["PAIZH"]]


_KEEP = [(SOUTH, "PAIZH", 10, 11), (WEST, "PAIZH", 5, 6), (NORTH, "PAIZH", 10, 5), (EAST, "PAIZH", 11, 8)]


def test_r1_bomb_and_killed():
    g = _hand([(SOUTH, "SILING", 6, 11), (WEST, "SILING", 6, 10)] + _KEEP)
    r = _move(g, (6, 11), (6, 10))
    assert r["event"] == 3 and _pid_at(g, 6, 11) < 0 and _pid_at(g, 6, 10) < 0
    g = _hand([(SOUTH, "PAIZH", 6, 11), (WEST, "SILING", 6, 10), (SOUTH, "LIANZH", 10, 11)] + _KEEP[1:])
    d = _pid_at(g, 6, 10)
    before = _row(g, SOUTH, d).copy()
    r = _move(g, (6, 11), (6, 10))
    assert r["event"] == 4 and _pid_at(g, 6, 11) < 0 and _pid_at(g, 6, 10) == d
    assert np.array_equal(_row(g, SOUTH, d), before)


def test_r3_siling_reveal_decrements_inventory():
    g = _hand([(SOUTH, "SILING", 6, 11), (WEST, "SILING", 6, 10)] + _KEEP)
    assert _rem(g, SOUTH, WEST)[T["SILING"]] == 1
    r = _move(g, (6, 11), (6, 10))
    assert r["flag_reveal_dst"] == 1
    assert _rem(g, SOUTH, WEST)[T["SILING"]] == 0


def test_r4_flag_capture_clears_inventory():
    g = _hand([(SOUTH, "SILING", 1, 9), (WEST, "JUNQI", 0, 9), (WEST, "PAIZH", 2, 9), (SOUTH, "PAIZH", 10, 16),
               (NORTH, "PAIZH", 6, 0), (EAST, "PAIZH", 11, 8)])
    assert _rem(g, SOUTH, WEST) is not None
    r = _move(g, (1, 9), (0, 9))
    assert r["flag_captured"] == 1
    assert _rem(g, SOUTH, WEST) is None
    assert _pid_at(g, 2, 9) < 0 and not any(g.alive[30:60])


def test_r6_stronghold_eat_reveals_other_stronghold_as_flag():
    g = _hand([(SOUTH, "SILING", 1, 9), (WEST, "PAIZH", 0, 9), (WEST, "JUNQI", 0, 7), (WEST, "DILEI", 1, 7),
               (WEST, "LIANZH", 3, 8), (SOUTH, "PAIZH", 10, 11), (NORTH, "PAIZH", 10, 5), (EAST, "PAIZH", 11, 8)])
    flag = _pid_at(g, 0, 7)
    before = float(_row(g, SOUTH, flag)[T["JUNQI"] - 2])
    assert 0 < before < 1
    r = _move(g, (1, 9), (0, 9))
    assert r["event"] == 2 and not r["flag_captured"] and not (r["seats_died_mask"] >> WEST) & 1
    after = _row(g, SOUTH, flag)
    assert _one_hot(after) and after[T["JUNQI"] - 2] == 1.0


def test_r5_r7_gongb_eats_dilei_reveals_attacker():
    g = _hand([(SOUTH, "GONGB", 6, 11), (WEST, "DILEI", 6, 10)] + _KEEP)
    att = _pid_at(g, 6, 11)
    before = _row(g, EAST, att)
    assert not _one_hot(before) and before[T["GONGB"] - 2] > 0
    r = _move(g, (6, 11), (6, 10))
    assert r["event"] == 2
    after = _row(g, EAST, att)
    assert _one_hot(after) and after[T["GONGB"] - 2] == 1.0
    assert _rem(g, EAST, SOUTH)[T["GONGB"]] == PIECE_COUNTS[T["GONGB"]] - 1


def _play(g, plies, rng):
    for _ in range(plies):
        if g.terminated:
            break
        ids = g.legal_ids()
        if len(ids) == 0:
            break
        rc, _ = g.step_id(int(ids[rng.integers(len(ids))]))
        assert rc == 0


@pytest.mark.parametrize("show_mode", [0, 1, 2])
def test_beliefs_cover_live_pieces_along_games(show_mode):
    """I1-I5 along random games in every show mode: every live piece has a
    probability-vector row for every observer, the observer's own pieces (and in
    BRIGHT / HALF_DARK the teammate's) stay one-hot on their true type, and a
    one-hot row of an enemy piece names its true type (beliefs never lie)."""
    rng = np.random.default_rng(show_mode)
    for seed in range(6):
        g = _opening(100 + seed, show_mode)
        for _ in range(12):
            _play(g, 15, rng)
            for obs in range(4):
                for pid in range(120):
                    if not g.alive[pid]:
                        continue
                    v = _row(g, obs, pid)
                    assert abs(float(v.sum()) - 1.0) < 1e-5 and (v >= 0).all()
                    truth = int(g.ptype[pid]) - 2
                    visible = show_mode == 0 or pid // 30 == obs or (show_mode == 2 and (pid // 30) % 2 == obs % 2)
                    if visible:
                        assert _one_hot(v) and v[truth] == 1.0
                    elif _one_hot(v):
                        assert v[truth] == 1.0
                    else:
                        assert v[truth] > 0


def test_remaining_rows_zero_for_untracked_seats():
    """remaining_arr (tests/test_belief_tensor.py:139-201): a seat whose flag fell
    or that died leaves no tracked inventory, and tracked counts stay within
    [0, PIECE_COUNTS]; in BRIGHT mode every count is untouched until a death."""
    rng = np.random.default_rng(777)
    for seed in range(8):
        g = _opening(777 + seed)
        _play(g, 500, rng)
        for obs in range(4):
            for s in range(4):
                rem = _rem(g, obs, s)
                if g.seat_dead[s] or s == obs or (s & 1) == (obs & 1):
                    assert rem is None
                    continue
                for t, c in rem.items():
                    assert 0 <= c <= PIECE_COUNTS[t]


# ================================================================ Philox
# Random123 known-answer vectors for philox4x32_10 (kat_vectors)

@pytest.mark.parametrize("ctr,key,out", [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
])
def test_philox_known_answers(ctr, key, out):
    assert O.philox4x32_10(ctr, key) == out


def test_uniform_sampler_is_philox_scaled():
    ids = np.arange(100, 137, dtype=np.int32)
    for env in (0, 5, 40000):
        for ply in (0, 1, 2**32 + 3):
            u = O.philox4x32_10((env, ply & 0xFFFFFFFF, ply >> 32, 0), (0x4A51, 0))[0]
            assert O.sample_uniform(ids, env, 0x4A51, ply) == ids[(u * len(ids)) >> 32]
    assert O.sample_uniform(np.zeros(0, np.int32), 0, 1, 1) == -1


def test_logit_sampler_is_argmax_over_legal_canonical_ids():
    """The masked-logit pick equals the argmax of float64 N(0,1) logits
    Phi^-1((u + 1/2) / 2^32) over the legal canonical ids (ties never occur
    here), and it is uniform over the legal set."""
    from scipy.special import ndtri

    g = O.Game(O.random_setup(9), show_mode=2)
    ids = g.legal_ids()
    seat = int(g.turn)
    canon = np.array([O.canonical_id(seat, int(a)) for a in ids])
    counts = np.zeros(len(ids), np.int64)
    for ply in range(3000):
        u = np.array([O.philox4x32_10((7, ply, 0, 1 + int(c)), (0x4A51, 0))[0] for c in canon], np.float64)
        z = ndtri((u + 0.5) / 2.0**32)
        w, c = O.sample_logits(ids, seat, 7, 0x4A51, ply)
        j = int(np.argmax(z))
        assert (w, c) == (int(ids[j]), int(canon[j]))
        counts[j] += 1
    exp = 3000 / len(ids)
    assert ((counts - exp) ** 2 / exp).sum() < 2.0 * len(ids) + 30   # chi-square, generous


def test_reset_pool_index_closed_form():
    for env, seed, size in ((0, 0, 7), (123, 456, 10000), (32767, 2**40 + 3, 977)):
        h = (env * 2654435761 + seed) & (2**64 - 1)
        h ^= h >> 17
        h = (h * 0xBF58476D1CE4E5B9) & (2**64 - 1)
        h ^= h >> 31
        assert O.reset_pool_index(env, seed, size) == h % size


def test_vectorised_philox_helper_equals_oracle():
    """tests/gpu_compare.philox_first_word_np (used over 32,768 envs at once by the
    full-size GPU tests) equals the pinned oracle generator."""
    from tests import gpu_compare as G

    rng = np.random.default_rng(5)
    c0 = rng.integers(0, 2**32, 200, dtype=np.uint64)
    for c1, c2, c3, k0, k1 in ((3, 0, 0, 0x4A51, 0), (2**32 - 1, 7, 9, 1, 2**32 - 1)):
        got = G.philox_first_word_np(c0, c1, c2, c3, k0, k1)
        want = [O.philox4x32_10((int(a), c1, c2, c3), (k0, k1))[0] for a in c0]
        assert got.tolist() == want


# ================================================================ termination
# Q10 draw thresholds (tests/test_state_transitions.py:452-520; rules.py:444-445
# MAX_NUM_MOVES = 4000, MAX_NUM_MOVES_BETWEEN_ATTACKS = 200, applied with >= in
# _check_victory, state.py:1721-1724, before the turn advance, which is skipped
# on termination, state.py:914-941) and the env's move cap
# (tests/test_gpu_rollout.py:211-245; junqi_rl/env.py:295-305, applied after the
# turn advance as game_state.cu:1651-1656 does).

NO_CAP = 2**30   # GameState itself has no env cap
_Q10 = [(SOUTH, "PAIZH", 8, 11), (WEST, "PAIZH", 5, 8), (NORTH, "PAIZH", 8, 0), (EAST, "PAIZH", 11, 8)]


def _q10(mc, mslc, max_num_moves=NO_CAP, spec=_Q10):
    return O.Game.from_pieces(_pieces(spec), turn=SOUTH, move_counter=mc, mslc=mslc,
                              max_num_moves=max_num_moves)


def _assert_draw(g, r, turn):
    assert r["terminated"] == 1 and r["draw"] == 1 and r["winner"] == -1
    assert g.terminated == 1 and g.draw == 1 and g.winner == -1
    assert int(g.turn) == turn
    assert int(g.zobrist) == g.recompute_zobrist()


def _assert_live(g, r, turn):
    assert r["terminated"] == 0 and r["draw"] == 0 and r["winner"] == -1
    assert g.terminated == 0 and g.draw == 0
    assert int(g.turn) == turn
    assert int(g.zobrist) == g.recompute_zobrist()


def test_q10_draw_by_move_counter():
    """move_counter 3999 -> one move -> draw, no winner, rewards 0; the turn stays
    with the mover (no advance on termination)."""
    for cap in (NO_CAP, 4000):
        g = _q10(3999, 0, cap)
        r = _move(g, (8, 11), (8, 12))
        assert r["event"] == 1
        _assert_draw(g, r, SOUTH)
        assert g.move_counter == 4000 and g.mslc == 1


def test_q10_move_counter_below_threshold():
    """A ply ending at move_counter 3999 does not draw; the turn advances."""
    g = _q10(3998, 0)
    r = _move(g, (8, 11), (8, 12))
    _assert_live(g, r, WEST)
    assert g.move_counter == 3999
    rc, r = g.step_id(int(g.legal_ids()[0]))
    assert rc == 0
    _assert_draw(g, r, WEST)


def test_q10_draw_by_no_combat_counter():
    g = _q10(500, 199)
    r = _move(g, (8, 11), (8, 12))
    _assert_draw(g, r, SOUTH)
    assert g.mslc == 200 and g.move_counter == 501


def test_q10_no_combat_counter_below_threshold():
    g = _q10(500, 198)
    r = _move(g, (8, 11), (8, 12))
    _assert_live(g, r, WEST)
    assert g.mslc == 199


def test_q10_draw_not_triggered_by_combat():
    """Combat at moves_since_last_combat 199 resets the counter: no draw."""
    spec = [(SOUTH, "SILING", 6, 11), (WEST, "PAIZH", 6, 10), (NORTH, "PAIZH", 8, 0), (EAST, "PAIZH", 11, 8)]
    g = _q10(500, 199, spec=spec)
    r = _move(g, (6, 11), (6, 10))
    assert r["event"] == 2
    assert g.mslc == 0 and g.move_counter == 501
    # WEST lost its only piece, so it is dead and NORTH moves next
    assert r["seats_died_mask"] == 1 << WEST
    _assert_live(g, r, NORTH)


def test_env_cap_one_and_three_moves():
    """max_num_moves = 1 draws after one step; = 3 is live after one and two
    steps and draws after three (tests/test_gpu_rollout.py:211-245). The cap
    fires after the turn advance, so the turn has moved on."""
    short = _q10(0, 0, 1)
    r = _move(short, (8, 11), (8, 12))
    _assert_draw(short, r, WEST)
    longer = _q10(0, 0, 3)
    for k in range(3):
        seat = int(longer.turn)
        ids = longer.legal_ids()
        rc, r = longer.step_id(int(ids[0]))
        assert rc == 0
        nxt = (seat + 1) & 3
        if k < 2:
            _assert_live(longer, r, nxt)
        else:
            _assert_draw(longer, r, nxt)


@pytest.mark.parametrize("cap", [1, 3, 600])
def test_env_cap_below_and_at_limit(cap):
    """A ply ending at cap - 1 is live; the ply ending at cap draws."""
    g = _q10(cap - 2, 0, cap) if cap >= 2 else None
    if g is not None:
        r = _move(g, (8, 11), (8, 12))
        _assert_live(g, r, WEST)
        assert g.move_counter == cap - 1
    g = _q10(cap - 1, 0, cap)
    r = _move(g, (8, 11), (8, 12))
    _assert_draw(g, r, WEST)


def test_env_cap_survives_new_games():
    """The limit is a property of the game's settings: a fresh game with the same
    cap draws at the same ply again (reset_terminated_device keeps it)."""
    setup = O.random_setup(100)
    for cap, plies in ((1, 1), (3, 3)):
        for _ in range(2):
            g = O.Game(setup, max_num_moves=cap)
            for k in range(plies):
                assert not g.terminated
                rc, r = g.step_id(int(g.legal_ids()[0]))
                assert rc == 0
            assert g.terminated and g.draw and g.winner == -1


def test_rules_draw_and_cap_order():
    """Rules draw (before the advance, turn frozen) vs env cap (after the
    advance): the same ply from move_counter 3999 freezes the turn whatever the
    cap, while a cap reached below 4000 moves the turn on."""
    a = _q10(3999, 5, 4000)
    b = _q10(3999, 5, NO_CAP)
    c = _q10(2999, 5, 3000)
    for g in (a, b, c):
        _move(g, (8, 11), (8, 12))
    assert int(a.turn) == SOUTH and int(b.turn) == SOUTH and int(c.turn) == WEST
    assert int(a.zobrist) == int(b.zobrist)

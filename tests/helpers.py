"""Shared test helpers: fixture loading and scenario construction."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"
TYPE_NAMES = ["NONE", "DARK", "JUNQI", "DILEI", "ZHADAN", "SILING", "JUNZH", "SHIZH",
              "LVZH", "TUANZH", "YINGZH", "LIANZH", "PAIZH", "GONGB"]
TYPE_OF = {n: i for i, n in enumerate(TYPE_NAMES)}
EVENT_OF = {"MOVE": 1, "EAT": 2, "BOMB": 3, "KILLED": 4}
SEAT_OF = {"SOUTH": 0, "WEST": 1, "NORTH": 2, "EAST": 3}


def flat(xy) -> int:
    return int(xy[1]) * 17 + int(xy[0])


def scenario_files(category: str) -> list[Path]:
    return sorted((GOLDEN / "scenarios" / category).glob("*.json"))


def scenario_pieces(pre: dict) -> list[tuple[int, int, int, int]]:
    """(pid, type, x, y) for live pieces; pid = seat*30 + lowest free slot in file
    order, the way junqi_core/state.py:393-427 synthesises ids for hand-built states."""
    used = {s: set() for s in range(4)}
    out = []
    for p in pre["pieces"]:
        if p.get("dead"):
            continue
        s = p["seat"]
        slot = next(i for i in range(30) if i not in used[s])
        used[s].add(slot)
        out.append((s * 30 + slot, TYPE_OF[p["type"]], p["pos"][0], p["pos"][1]))
    return out


def scenario_info(pre: dict):
    dead = [0] * 4
    fr = [0] * 4
    for it in pre["info"]:
        dead[it["seat"]] = int(it["dead"])
        fr[it["seat"]] = int(it["flag_revealed"])
    return dead, fr


def load_replay() -> dict:
    return json.loads((GOLDEN / "replay_recovered.json").read_text())


def replay_setup(doc: dict) -> np.ndarray:
    return np.asarray(doc["lineups"], dtype=np.int8)


def load_obs_hashes() -> list[dict]:
    return json.loads((GOLDEN / "obs_hashes.json").read_text())


def obs_digest(spatial: np.ndarray, glob: np.ndarray) -> str:
    """SHA-256 of the obs quantised to 1e-6 with a shape header
    (the digest of reference tools/gen_obs_golden.py:45-56)."""
    import hashlib
    h = hashlib.sha256()
    for arr in (spatial, glob):
        q = np.rint(arr.astype(np.float64) * 1e6).astype("<i4")
        h.update(np.asarray(arr.shape, dtype="<i4").tobytes())
        h.update(q.tobytes())
    return h.hexdigest()


# Channel group sizes of the 317-channel layout (junqi_core/observation.py:155-196)
CHANNEL_GROUPS = [
    ("piece_own", 12), ("prob_teammate", 12), ("dark_teammate", 1), ("piece_left_side_enemy", 1),
    ("piece_right_side_enemy", 1), ("belief_left_side", 12), ("belief_right_side", 12),
    ("dead_flags", 3), ("flag_revealed", 4), ("board_static", 6), ("turn_history", 2),
    ("move_bucket", 8), ("active_eat_bucket", 8), ("passive_survive_bucket", 8),
    ("death_reason", 12), ("dead_at_zero", 2), ("piece_slot", 25), ("move_history", 32),
    ("cm_kill_mine_type", 12), ("cm_kill_mine_ge", 3), ("cm_kill_other_ge", 3),
    ("cm_chain_type", 12), ("cm_chain_ge", 3), ("cm_floor_ge", 9), ("cm_is_gongb", 1),
    ("cm_not_gongb", 1), ("cm_dilei_candidate", 1), ("cm_my_kill_count_ge", 3),
    ("cm_my_is_gongb", 1), ("cm_my_dilei_candidate", 1), ("cm_kill_mine_count", 12),
    ("cm_kill_mine_slot", 30), ("cm_recency", 4), ("cm_eaten_by_pid", 60),
]
assert sum(s for _, s in CHANNEL_GROUPS) == 317

"""Write tests/golden/reference_vectors.json from the reference's junqi_core.

Run by hand, once, in a checkout that holds the reference repository
(``python tests/golden/gen_reference_vectors.py /path/to/reference``): it
imports ``junqi_core`` from there. Nothing at test time imports the reference;
the tests read only the JSON this writes.

It records what no reference golden file, known-answer test or invariant pins
(the reference's own tests check these only relationally):

* the Zobrist hash of ``GameState`` after every ply (its composition,
  junqi_core/state.py:537-583, 977-1103, 1761-1811);
* combat-memory fields of all four observers late in long games
  (combat_memory.py:354-569; the observation hashes stop at ply 100);
* ``BeliefTensor`` rows and remaining counts of all four observers in
  BRIGHT, DARK and HALF_DARK, including DARK teammate beliefs after the
  opening (info_model.py:218-561);
* bit-exact digests of all four observers' observations
  (observation.py:621-857) at those plies;
* before every ply and at the end, the acting seat's legal set
  (GameState.legal_actions, state.py:1200-1213) as its size and a digest of
  its sorted world ids src_flat*289 + dst_flat (legal_digest below).

Games: setups from generate_random_setup(random.Random(seed)), actions by
random.Random(seed + 1000).choice over GameState.legal_actions(), all four
beliefs updated every ply as junqi_rl/env.py:285-289 does.
"""

from __future__ import annotations

import hashlib
import json
import random
import sys
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "reference_vectors.json"
SEEDS = (0, 1, 2, 3)
MODES = ("BRIGHT", "DARK", "HALF_DARK")
MAX_PLIES = 1000
CHECKPOINTS = (0, 60, 150, 250, 400, 600, 800, 1000)
CM_FIELDS = ("direct_ate_my_pid_lo", "direct_ate_my_pid_hi", "direct_ate_my_type_mask", "last_direct_step",
             "direct_other_count", "chain_pid_lo", "chain_pid_hi", "chain_ate_my_type_mask", "last_chain_step",
             "eaten_by_pid_lo", "eaten_by_pid_hi", "rank_floor", "rank_floor_step", "is_gongb", "not_gongb",
             "attacked_by_known_gongb")


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def legal_digest(ids) -> str:
    """First 16 hex digits of the SHA-256 of the sorted ids as little-endian int32."""
    return sha(np.sort(np.asarray(ids, dtype="<i4")))[:16]


def world_ids(actions) -> list[int]:
    return [(a.src[1] * 17 + a.src[0]) * 289 + a.dst[1] * 17 + a.dst[0] for a in actions]


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from junqi_core.info_model import BeliefTensor
    from junqi_core.observation import build_observation
    from junqi_core.rules import Seat, ShowMode
    from junqi_core.setup import generate_random_setup
    from junqi_core.state import GameState

    games = []
    for seed in SEEDS:
        for mode_name in MODES:
            mode = ShowMode[mode_name]
            setup = generate_random_setup(random.Random(seed))
            state = GameState.new_game(setup, show_mode=mode)
            beliefs = {s: BeliefTensor.initial(state, s) for s in Seat}
            rng = random.Random(seed + 1000)
            rec = {"seed": seed, "show_mode": mode_name,
                   "setup": [int(p) for lu in setup for p in lu],
                   "actions": [], "zobrist": [], "legal_count": [], "legal_digest": [], "checkpoints": []}

            def checkpoint(ply: int) -> None:
                cm = state.combat_memory
                cp = {"ply": ply, "cm": {k: sha(np.asarray(getattr(cm, k))) for k in CM_FIELDS},
                      "beliefs": [], "remaining": [], "obs_f32": [], "glob_f32": []}
                for s in Seat:
                    b = beliefs[s]
                    b.ensure_synced(state)
                    probs = np.zeros((120, 12), np.float32)
                    alive = np.nonzero(state.alive)[0]
                    probs[alive] = b.probs_arr[alive]
                    cp["beliefs"].append(sha(probs))
                    cp["remaining"].append(np.asarray(b.remaining_arr, np.int64).tolist())
                    obs = build_observation(state, b, s)
                    cp["obs_f32"].append(sha(np.asarray(obs.spatial, np.float32)))
                    cp["glob_f32"].append(sha(np.asarray(obs.global_, np.float32)))
                rec["checkpoints"].append(cp)

            def record_legal(legal) -> None:
                ids = world_ids(legal)
                rec["legal_count"].append(len(ids))
                rec["legal_digest"].append(legal_digest(ids))

            checkpoint(0)
            for ply in range(1, MAX_PLIES + 1):
                if state.terminated:
                    break
                legal = state.legal_actions()
                record_legal(legal)
                if not legal:
                    break
                a = rng.choice(legal)
                new_state, result = state.step(a)
                for s in Seat:
                    beliefs[s].update(state, new_state, result)
                state = new_state
                rec["actions"].append([a.src[1] * 17 + a.src[0], a.dst[1] * 17 + a.dst[0]])
                rec["zobrist"].append(format(int(state.zobrist) & (2**64 - 1), "016x"))
                if ply in CHECKPOINTS:
                    checkpoint(ply)
            if len(rec["legal_count"]) == len(rec["actions"]):   # the end position's set (empty once terminated)
                record_legal(state.legal_actions())
            if rec["checkpoints"][-1]["ply"] != len(rec["actions"]):
                checkpoint(len(rec["actions"]))
            rec["terminated"] = bool(state.terminated)
            games.append(rec)
            print(f"seed {seed} {mode_name}: {len(rec['actions'])} plies, terminated={state.terminated}")
    OUT.write_text(json.dumps({"generator": "tests/golden/gen_reference_vectors.py",
                               "checkpoint_plies": list(CHECKPOINTS), "games": games}, separators=(",", ":")))
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")

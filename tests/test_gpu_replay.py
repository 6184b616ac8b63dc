"""Recorded games on an MI355X (junqi_amd.replay).

The recovered 603-ply game (reference replays/recovered_20260815) is replayed
on the device from its .jql action log, and every ply's result and state_after
fields are compared with the reference's moves.jsonl through ply 277 (ply 278
predates RULES 1.1.0: ZHADAN into DILEI is a BOMB now, so the game diverges
there). Random device games are recorded, written as .jql, read back and
replayed on the oracle, which must reach the same positions.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from oracle import oracle as O  # noqa: E402
from tests.helpers import load_replay as recovered_replay  # noqa: E402

FIELDS = ("seat", "src", "dst", "src_type", "dst_type", "event", "flag_reveal_src", "flag_reveal_dst",
          "flag_captured", "seats_died", "terminated", "winner_team", "draw", "turn", "move_counter",
          "moves_since_last_combat", "alive_by_seat", "info")


@pytest.fixture(scope="module")
def jq():
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a visible GPU")
    import junqi_amd
    return junqi_amd


def test_recovered_game_replays_on_device(jq):
    from junqi_amd import replay as R
    d = recovered_replay()
    lineups = np.array(d["lineups"], np.int8).reshape(1, 120)
    acts = R.moves_to_world_ids(np.array(d["jql_moves"]))[None, :]
    recs = R.replay_games(lineups, acts, show_mode=1)[0]
    assert len(recs) >= 277
    for got, want in zip(recs[:277], d["plies"][:277]):
        for k in FIELDS:
            assert got[k] == (list(want[k]) if isinstance(want[k], tuple) else want[k]), (want["step"], k)
    p278 = recs[277]
    assert p278["src_type"] == "ZHADAN" and p278["dst_type"] == "DILEI" and p278["event"] == "BOMB"


def test_recorded_games_round_trip_through_jql(jq):
    from junqi_amd import replay as R
    n, plies, show = 8, 80, 2
    lineups = jq.generate_lineups(123, n)
    b = jq.JunqiBatch(n, show_mode=show, max_num_moves=70)
    b.reset_lineups(lineups)
    rec = R.GameRecorder(lineups)
    for ply in range(plies):
        out = b.legal()
        acts = torch.empty(n, dtype=torch.int32, device=b.device)
        jq._lib.check(jq._lib.lib.jq_sample_uniform(b._h, out["counts"].data_ptr(), out["offsets"].data_ptr(),
                                                    out["values"].data_ptr(), out["values"].numel(), 9, ply,
                                                    acts.data_ptr(), b.stream))
        rec.record(b.step(acts))
    zob = b.get_field("zobrist")[:, 0]
    for i in range(n):
        lu, mv = R.read_jql(rec.jql(i))
        assert np.array_equal(lu.reshape(-1).astype(np.int8), lineups[i])
        g = O.Game(lineups[i], show_mode=show, max_num_moves=70)
        for a in R.moves_to_world_ids(mv):
            rc, _ = g.step_id(int(a))
            assert rc == 0
        assert int(g.zobrist) == int(zob[i]), i
    # the device replay of the recorded logs reproduces the same games
    logs = [rec.world_actions(i) for i in range(n)]
    width = max(len(x) for x in logs)
    acts = np.full((n, width), -1, np.int64)
    for i, x in enumerate(logs):
        acts[i, :len(x)] = x
    recs = R.replay_games(lineups, acts, show_mode=show, max_num_moves=70)
    for i in range(n):
        assert len(recs[i]) == len(logs[i])
        assert recs[i][-1]["move_counter"] == len(logs[i])
    b.close()

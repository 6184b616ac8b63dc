"""The .jql replay format (junqi_amd.replay) without a GPU: the writer
reproduces the reference's recovered replay byte for byte (its SHA-256 is
published in replays/recovered_20260815/README.md), the reader inverts it and
rejects malformed files."""

from __future__ import annotations

import hashlib

import numpy as np
import pytest

from tests.helpers import load_replay as recovered_replay

RECOVERED_JQL_SHA256 = "bbbe3590e6b31928924d4c88e2733e30981c65edcaa0996db3583cef0067124c"


def _replay_module():
    from junqi_amd import replay
    return replay


def test_writer_reproduces_the_recovered_replay():
    R = _replay_module()
    d = recovered_replay()
    raw = R.write_jql(np.array(d["lineups"], np.uint8), np.array(d["jql_moves"], np.uint8))
    assert len(raw) == 8 + 120 + 4 * 603
    assert hashlib.sha256(raw).hexdigest() == RECOVERED_JQL_SHA256
    lu, mv = R.read_jql(raw)
    assert lu.shape == (4, 30) and mv.shape == (603, 4)
    assert np.array_equal(lu.reshape(-1), d["lineups"]) and np.array_equal(mv, d["jql_moves"])


def test_world_id_conversions():
    R = _replay_module()
    d = recovered_replay()
    ids = R.moves_to_world_ids(np.array(d["jql_moves"]))
    # moves.jsonl step 1: (6,13) -> (7,12), chosen_action_id 65814
    assert ids[0] == 65814 == (13 * 17 + 6) * 289 + 12 * 17 + 7
    assert np.array_equal(R.world_ids_to_moves(ids), np.array(d["jql_moves"], np.uint8))
    for p, i in zip(d["plies"][:50], ids[:50]):
        assert list(p["src"]) == [int(i) // 289 % 17, int(i) // 289 // 17]


def test_reader_rejects_malformed_files(tmp_path):
    R = _replay_module()
    d = recovered_replay()
    raw = R.write_jql(np.array(d["lineups"], np.uint8), np.array(d["jql_moves"][:5], np.uint8), tmp_path / "g.jql")
    assert (tmp_path / "g.jql").read_bytes() == raw
    with pytest.raises(ValueError, match="magic"):
        R.read_jql(b"\x00" * 4 + raw[4:])
    with pytest.raises(ValueError, match="bytes"):
        R.read_jql(raw[:-1])
    with pytest.raises(ValueError, match="too short"):
        R.read_jql(raw[:20])
    bad = bytearray(raw)
    bad[8] = 14
    with pytest.raises(ValueError, match="piece type"):
        R.read_jql(bytes(bad))
    with pytest.raises(ValueError, match="17x17"):
        R.write_jql(np.array(d["lineups"], np.uint8), np.array([[0, 0, 17, 0]], np.uint8))
    with pytest.raises(ValueError):
        R.world_ids_to_moves(np.array([289 * 289]))

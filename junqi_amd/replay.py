"""Recorded games.

* The compact ``.jql`` replay format of the reference's native client and RL
  exporter (docs/REPLAY.md "Original GTK native client"; read by
  legacy_gui/src/junqi.c): little-endian ``<II`` header (magic 1111, step
  count), the four 30-slot lineups as piece-type bytes (0 in an empty camp),
  then one ``(sx, sy, dx, dy)`` world-coordinate byte quadruple per step.
* A device replay runner that plays recorded action logs on the MI355X batch
  and reports one record per ply with the engine-derived fields of the
  reference's ``moves.jsonl`` (replays/recovered_20260815/moves.jsonl:
  ``result`` and ``state_after``), so recorded games serve as regressions.
* A recorder that collects the world actions a batch actually applied and
  writes each game as ``.jql``.
"""

from __future__ import annotations

import struct
from pathlib import Path

import numpy as np
import torch

from .batch import JunqiBatch

JQL_MAGIC = 1111
SEAT_NAMES = ("SOUTH", "WEST", "NORTH", "EAST")
# PieceType names (junqi_core/rules.py:49-70), indexed by value
PIECE_NAMES = ("NONE", "DARK", "JUNQI", "DILEI", "ZHADAN", "SILING", "JUNZH", "SHIZH", "LVZH", "TUANZH",
               "YINGZH", "LIANZH", "PAIZH", "GONGB")
EVENT_NAMES = {1: "MOVE", 2: "EAT", 3: "BOMB", 4: "KILLED"}
_SILING = 5


def read_jql(source: bytes | str | Path) -> tuple[np.ndarray, np.ndarray]:
    """(lineups (4, 30) uint8 piece types, moves (T, 4) uint8 sx sy dx dy)."""
    raw = source if isinstance(source, (bytes, bytearray)) else Path(source).read_bytes()
    if len(raw) < 8 + 120:
        raise ValueError(f"jql replay too short: {len(raw)} bytes")
    magic, steps = struct.unpack_from("<II", raw, 0)
    if magic != JQL_MAGIC:
        raise ValueError(f"not a jql replay: magic {magic}, expected {JQL_MAGIC}")
    if len(raw) != 8 + 120 + 4 * steps:
        raise ValueError(f"jql replay of {steps} steps must be {8 + 120 + 4 * steps} bytes, got {len(raw)}")
    lineups = np.frombuffer(raw, np.uint8, 120, 8).reshape(4, 30).copy()
    moves = np.frombuffer(raw, np.uint8, 4 * steps, 128).reshape(steps, 4).copy()
    _check(lineups, moves)
    return lineups, moves


def write_jql(lineups: np.ndarray, moves: np.ndarray, path: str | Path | None = None) -> bytes:
    """Encode a game as ``.jql`` bytes (and write them to ``path`` if given)."""
    lu = np.asarray(lineups).reshape(4, 30)
    mv = np.asarray(moves).reshape(-1, 4)
    _check(lu, mv)
    raw = struct.pack("<II", JQL_MAGIC, mv.shape[0]) + lu.astype(np.uint8).tobytes() + mv.astype(np.uint8).tobytes()
    if path is not None:
        Path(path).write_bytes(raw)
    return raw


def _check(lineups: np.ndarray, moves: np.ndarray) -> None:
    lu = lineups.astype(np.int64)
    if not np.all((lu == 0) | ((lu >= 2) & (lu <= 13))):
        raise ValueError("lineup bytes must be 0 (empty camp) or a piece type 2..13")
    mv = moves.astype(np.int64)
    if mv.size and (mv.min() < 0 or mv.max() > 16):
        raise ValueError("move coordinates must lie on the 17x17 board")


def moves_to_world_ids(moves: np.ndarray) -> np.ndarray:
    """(T, 4) sx sy dx dy -> world action ids (sy*17+sx)*289 + dy*17+dx."""
    mv = np.asarray(moves, np.int64).reshape(-1, 4)
    return ((mv[:, 1] * 17 + mv[:, 0]) * 289 + mv[:, 3] * 17 + mv[:, 2]).astype(np.int32)


def world_ids_to_moves(ids: np.ndarray) -> np.ndarray:
    """World action ids -> (T, 4) uint8 sx sy dx dy."""
    a = np.asarray(ids, np.int64).reshape(-1)
    if a.size and (a.min() < 0 or a.max() >= 289 * 289):
        raise ValueError("world action ids must lie in [0, 289*289)")
    s, d = np.divmod(a, 289)
    return np.stack([s % 17, s // 17, d % 17, d // 17], axis=1).astype(np.uint8)


def _seat_info(dead: int, flag: int) -> dict:
    return {SEAT_NAMES[s]: {"dead": bool((dead >> s) & 1), "flag_revealed": bool((flag >> s) & 1)}
            for s in range(4)}


def replay_games(lineups: np.ndarray, actions: np.ndarray, *, show_mode: int = 2, max_num_moves: int = 4000,
                 device: int = 0) -> list[list[dict]]:
    """Play G recorded games side by side on the device: ``lineups`` (G, 120)
    piece types, ``actions`` (G, T) world ids (-1 = game over). Returns per game
    one record per applied ply with the fields of moves.jsonl's ``result`` and
    ``state_after``; a game's records stop at its first invalid action."""
    lu = np.ascontiguousarray(lineups, np.int8).reshape(-1, 120)
    acts = np.asarray(actions, np.int64).reshape(lu.shape[0], -1)
    g, steps = acts.shape
    b = JunqiBatch(g, show_mode=show_mode, max_num_moves=max_num_moves, device=device)
    try:
        b.reset_lineups(lu)
        out: list[list[dict]] = [[] for _ in range(g)]
        live = np.ones(g, bool)
        for t in range(steps):
            a = np.where(live, acts[:, t], -1).astype(np.int32)
            if not (a >= 0).any():
                break
            turn0 = b.get_field("turn")[:, 0].astype(np.int64)
            ptype = b.get_field("ptype")
            cell = b.get_field("cell")
            r = b.step(torch.from_numpy(a).to(b.device))
            r = {k: v.cpu().numpy() for k, v in r.items()}
            turn = b.get_field("turn")[:, 0]
            mc, mslc = b.get_field("move_counter")[:, 0], b.get_field("mslc")[:, 0]
            dead, flag = b.get_field("seat_dead")[:, 0], b.get_field("flag_rev")[:, 0]
            alive = b.get_field("pos")[:, :120].reshape(g, 4, 30) >= 0
            for i in range(g):
                if a[i] < 0:
                    continue
                if not r["valid"][i]:
                    live[i] = False
                    continue
                src, dst = divmod(int(a[i]), 289)
                sp, dp = int(cell[i, src]), int(cell[i, dst])
                st = int(ptype[i, sp])
                dt = int(ptype[i, dp]) if dp >= 0 else None
                ev = EVENT_NAMES[int(r["event"][i])]
                w = int(r["winner_team"][i])
                out[i].append({
                    "step": t + 1, "seat": int(turn0[i]),
                    "src": [src % 17, src // 17], "dst": [dst % 17, dst // 17],
                    "src_type": PIECE_NAMES[st], "dst_type": None if dt is None else PIECE_NAMES[dt],
                    "event": ev,
                    "flag_reveal_src": st == _SILING and ev in ("KILLED", "BOMB"),
                    "flag_reveal_dst": dt == _SILING and ev in ("EAT", "BOMB"),
                    "flag_captured": bool(r["flag_captured"][i]),
                    "seats_died": [s for s in range(4) if (int(r["seats_died"][i]) >> s) & 1],
                    "terminated": bool(r["terminated"][i]), "winner_team": None if w < 0 else w,
                    "draw": bool(r["draw"][i]), "turn": SEAT_NAMES[int(turn[i])],
                    "move_counter": int(mc[i]), "moves_since_last_combat": int(mslc[i]),
                    "alive_by_seat": {SEAT_NAMES[s]: int(alive[i, s].sum()) for s in range(4)},
                    "info": _seat_info(int(dead[i]), int(flag[i])),
                })
                if r["terminated"][i]:
                    live[i] = False
        return out
    finally:
        b.close()


class GameRecorder:
    """Collects, per env of a JunqiBatch, the lineup it started from and the
    world actions its steps applied, and writes each game as ``.jql``."""

    def __init__(self, lineups: np.ndarray) -> None:
        self.lineups = np.ascontiguousarray(lineups, np.int8).reshape(-1, 120).copy()
        self._moves: list[list[int]] = [[] for _ in range(self.lineups.shape[0])]

    def record(self, step_out: dict) -> None:
        """Append the applied actions of one JunqiBatch.step() result."""
        valid = step_out["valid"].cpu().numpy()
        world = step_out["world_action"].cpu().numpy()
        for i in np.flatnonzero(valid):
            self._moves[i].append(int(world[i]))

    def world_actions(self, env: int) -> np.ndarray:
        return np.asarray(self._moves[env], np.int32)

    def jql(self, env: int, path: str | Path | None = None) -> bytes:
        return write_jql(self.lineups[env].astype(np.uint8).reshape(4, 30),
                         world_ids_to_moves(self.world_actions(env)), path)

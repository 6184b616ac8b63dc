"""Write the committed fixtures under tests/golden/ (run once, in the build container).

It reads only DATA files of the reference repository (JSON scenarios, the
recorded game), parses the canonical lineup tables out of
junqi_core/setup_canonical.py as text (``ast``; nothing is executed) and calls
numpy / the standard library. It imports no reference code. Usage::

    python tests/golden/make_fixtures.py [/path/to/reference]

Outputs
-------
scenarios/<category>/<name>.json   golden step scenarios (reference tests/golden/**)
obs_hashes.json                    reference tests/golden/obs_hashes.json (12 records)
replay_recovered.json              compact per-ply record of
                                   replays/recovered_20260815 (lineups, actions,
                                   per-ply result and state_after fields)
recency_lut_f32.bin                float32 exp(-e/tau) for e in [0,4096) (also written to
                                   junqi_amd/data/, where the library loads it),
                                   tau planes (32, 256, 64, 128), computed the way
                                   junqi_core/observation.py:1561-1562 does
zobrist_sha256.txt                 SHA-256 of the numpy PCG64 Zobrist stream
canonical_lineups.json             the four canonical opening lineups T, D, G, F as
                                   30 seat-local piece types (setup_canonical.py:96-269)
"""

from __future__ import annotations

import ast
import hashlib
import json
import shutil
import struct
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
CATEGORIES = ("battle", "full_game", "inference", "move_gen", "setup_validation",
              "siling_flag", "stronghold")
TYPE_NAMES = ["NONE", "DARK", "JUNQI", "DILEI", "ZHADAN", "SILING", "JUNZH", "SHIZH",
              "LVZH", "TUANZH", "YINGZH", "LIANZH", "PAIZH", "GONGB"]


def recency_lut() -> np.ndarray:
    out = np.zeros((4, 4096), dtype=np.float32)
    for k, tau in enumerate((32.0, 256.0, 64.0, 128.0)):
        elapsed = np.arange(4096, dtype=np.int32).astype(np.float32)
        out[k] = np.exp(-np.maximum(elapsed, 0.0) / tau, dtype=np.float32)
    return out


def zobrist_stream() -> np.ndarray:
    # Same draw order and call as junqi_core/_zobrist.py:80-106.
    rng = np.random.default_rng(0x4A554E51495F5A4F)
    shapes = [(120, 14, 289), (4,), (4096,), (512,), (1,), (3,), (1,), (4,), (4,), (4,)]
    parts = [rng.integers(low=0, high=np.iinfo(np.uint64).max, size=s, dtype=np.uint64,
                          endpoint=True).ravel() for s in shapes]
    return np.concatenate(parts)


def replay(ref: Path) -> dict:
    d = ref / "replays" / "recovered_20260815"
    raw = (d / "victory_team0_seed2026081500.jql").read_bytes()
    magic, steps = struct.unpack_from("<II", raw, 0)
    assert magic == 1111, magic
    lineups = list(raw[8:8 + 120])
    moves = []
    off = 8 + 120
    for _ in range(steps):
        moves.append(list(raw[off:off + 4]))
        off += 4
    plies = []
    with open(d / "moves.jsonl") as fh:
        for line in fh:
            rec = json.loads(line)
            res = rec["result"]
            sa = rec["state_after"]
            plies.append({
                "step": rec["step"],
                "seat": rec["acting_seat"]["id"],
                "src": rec["action"]["src"], "dst": rec["action"]["dst"],
                "src_type": (rec.get("private_before") or {}).get("src", {}).get("type"),
                "dst_type": ((rec.get("private_before") or {}).get("dst") or {}).get("type"),
                "event": res["event"],
                "flag_reveal_src": res["flag_reveal_src"], "flag_reveal_dst": res["flag_reveal_dst"],
                "flag_captured": res["flag_captured"],
                "seats_died": [s["id"] for s in res["seats_died_this_step"]],
                "terminated": sa["terminated"], "winner_team": sa["winner_team"], "draw": sa["draw"],
                "turn": sa["turn"], "move_counter": sa["move_counter"],
                "moves_since_last_combat": sa["moves_since_last_combat"],
                "alive_by_seat": sa["alive"]["by_seat"],
                "info": sa["info"],
            })
    return {"lineups": lineups, "jql_moves": moves, "plies": plies}


def canonical_lineups(ref: Path) -> dict:
    """SETUP_<style> = _make_lineup({slot: PieceType.NAME, ...}) literals of
    setup_canonical.py, read from its syntax tree."""
    tree = ast.parse((ref / "junqi_core" / "setup_canonical.py").read_text())
    out = {}
    for node in ast.walk(tree):
        if not isinstance(node, (ast.Assign, ast.AnnAssign)):
            continue
        target = node.targets[0] if isinstance(node, ast.Assign) else node.target
        if not (isinstance(target, ast.Name) and target.id.startswith("SETUP_")):
            continue
        call = node.value
        assert isinstance(call, ast.Call) and call.func.id == "_make_lineup", target.id
        table = call.args[0]
        row = [0] * 30
        for k, v in zip(table.keys, table.values):
            assert isinstance(v, ast.Attribute) and v.value.id == "PieceType", target.id
            row[k.value] = TYPE_NAMES.index(v.attr)
        out[target.id[len("SETUP_"):]] = row
    assert sorted(out) == ["D", "F", "G", "T"], sorted(out)
    return out


def main() -> None:
    ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    for cat in CATEGORIES:
        src = ref / "tests" / "golden" / cat
        dst = HERE / "scenarios" / cat
        dst.mkdir(parents=True, exist_ok=True)
        for p in sorted(src.glob("*.json")):
            shutil.copyfile(p, dst / p.name)
    shutil.copyfile(ref / "tests" / "golden" / "obs_hashes.json", HERE / "obs_hashes.json")
    (HERE / "replay_recovered.json").write_text(json.dumps(replay(ref)))
    recency_lut().tofile(HERE / "recency_lut_f32.bin")
    recency_lut().tofile(HERE.parent.parent / "junqi_amd" / "data" / "recency_lut_f32.bin")
    z = zobrist_stream()
    (HERE / "zobrist_sha256.txt").write_text(
        f"{hashlib.sha256(z.astype('<u8').tobytes()).hexdigest()}  {z.size} uint64 (little-endian)\n")
    (HERE / "canonical_lineups.json").write_text(json.dumps(canonical_lineups(ref)) + "\n")
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()

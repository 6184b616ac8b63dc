"""ctypes bindings for the C oracle (test infrastructure only).

The oracle is what the HIP path is compared with: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this module. It loads ``oracle/_build/libjq_oracle.so`` (built by
``oracle/build_oracle.py``) and exposes thin numpy-friendly wrappers.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
# JQ_ORACLE_LIB names another build of the oracle: the mutation tests load
# copies with one planted mistake this way, to show the tests reject them.
LIB_PATH = (Path(os.environ["JQ_ORACLE_LIB"]) if os.environ.get("JQ_ORACLE_LIB")
            else _HERE / "_build" / "libjq_oracle.so")
RECENCY_LUT_PATH = _HERE.parent / "tests" / "golden" / "recency_lut_f32.bin"

NC = 289
NP = 120
OBS_C = 317
OBS_G = 28
ONB = 129


class Result(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "valid", "event", "flag_reveal_src", "flag_reveal_dst", "flag_captured",
        "seats_died_mask", "terminated", "winner", "draw", "gongb_revealed")]

    def as_dict(self) -> dict:
        return {n: int(getattr(self, n)) for n, _ in self._fields_}


# Field layout of ``jqo_game`` (must match oracle/jq_oracle.h).
_GAME_FIELDS = [
    ("alive", np.int8, (NP,)), ("ptype", np.int8, (NP,)), ("pseat", np.int8, (NP,)),
    ("pos_x", np.int8, (NP,)), ("pos_y", np.int8, (NP,)), ("zero_x", np.int8, (NP,)),
    ("zero_y", np.int8, (NP,)),
    ("move_count", np.int16, (NP,)), ("active_eat", np.int16, (NP,)), ("passive_surv", np.int16, (NP,)),
    ("death_reason", np.int8, (NP,)), ("death_step", np.int16, (NP,)), ("death_loc", np.int16, (NP,)),
    ("cell_pid", np.int16, (NC,)), ("seat_dead", np.int8, (4,)), ("flag_rev", np.int8, (4,)),
    ("turn", np.int8, ()), ("terminated", np.int8, ()), ("winner", np.int8, ()), ("draw", np.int8, ()),
    ("show_mode", np.int8, ()), ("pad_", np.int8, (3,)),
    ("move_counter", np.int32, ()), ("mslc", np.int32, ()), ("max_num_moves", np.int32, ()),
    ("zobrist", np.uint64, ()),
    ("hist", np.int16, (32, 2)), ("hist_len", np.int32, ()),
    ("cm_direct_lo", np.uint64, (4, NP)), ("cm_direct_hi", np.uint64, (4, NP)),
    ("cm_direct_type", np.uint16, (4, NP)), ("cm_last_direct", np.int16, (4, NP)),
    ("cm_other_cnt", np.int16, (4, NP)),
    ("cm_chain_lo", np.uint64, (4, NP)), ("cm_chain_hi", np.uint64, (4, NP)),
    ("cm_chain_type", np.uint16, (4, NP)), ("cm_last_chain", np.int16, (4, NP)),
    ("cm_eaten_lo", np.uint64, (4, NP)), ("cm_eaten_hi", np.uint64, (4, NP)),
    ("cm_floor", np.int8, (4, NP)), ("cm_floor_step", np.int16, (4, NP)),
    ("cm_is_gongb", np.int8, (4, NP)), ("cm_not_gongb", np.int8, (4, NP)),
    ("cm_atk_gongb", np.int8, (4, NP)),
    ("bcode", np.uint8, (4, NP)), ("rem_tracked", np.int8, (4, 4)), ("rem", np.int16, (4, 4, 12)),
]
GAME_DTYPE = np.dtype([(n, t, s) for n, t, s in _GAME_FIELDS], align=True)

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"oracle library missing: {LIB_PATH} (run oracle/build_oracle.py)")
    L = C.CDLL(str(LIB_PATH))
    P = C.c_void_p
    L.jqo_init.restype = None
    L.jqo_mt_seed.argtypes = [P, C.c_uint64]
    L.jqo_mt_u32.argtypes = [P]; L.jqo_mt_u32.restype = C.c_uint32
    L.jqo_mt_randbelow.argtypes = [P, C.c_uint32]; L.jqo_mt_randbelow.restype = C.c_uint32
    L.jqo_random_lineup.argtypes = [P, P]
    L.jqo_random_setup.argtypes = [C.c_uint64, P]
    L.jqo_setup_pool.argtypes = [C.c_uint64, C.c_int32, P]
    L.jqo_random_lineup.argtypes = [P, P]
    L.jqo_seedseq_state.argtypes = [C.c_uint64, P]
    L.jqo_pcg64_draw.argtypes = [C.c_uint64, C.c_int64, P]
    L.jqo_zobrist_count.restype = C.c_int64
    L.jqo_zobrist_all.restype = C.POINTER(C.c_uint64)
    L.jqo_set_recency_lut.argtypes = [P]
    L.jqo_new_game.argtypes = [P, P, C.c_int, C.c_int]; L.jqo_new_game.restype = C.c_int
    L.jqo_from_pieces.argtypes = [P, C.c_int, P, C.c_int, C.c_int, C.c_int, P, P, C.c_int, C.c_int]
    L.jqo_from_pieces.restype = C.c_int
    L.jqo_is_legal.argtypes = [P, C.c_int, C.c_int, C.c_int]; L.jqo_is_legal.restype = C.c_int
    L.jqo_legal_ids.argtypes = [P, C.c_int, P, C.c_int]; L.jqo_legal_ids.restype = C.c_int
    L.jqo_has_legal.argtypes = [P, C.c_int]; L.jqo_has_legal.restype = C.c_int
    L.jqo_legal_slots.argtypes = [P, C.c_int, P]; L.jqo_legal_slots.restype = C.c_int
    L.jqo_step.argtypes = [P, C.c_int, C.c_int, P]; L.jqo_step.restype = C.c_int
    L.jqo_move_requires_gongb.argtypes = [P, C.c_int, C.c_int]; L.jqo_move_requires_gongb.restype = C.c_int
    L.jqo_observe.argtypes = [P, C.c_int, P, P]
    L.jqo_observe_ext.argtypes = [P, C.c_int, P, P, P]
    L.jqo_recompute_zobrist.argtypes = [P]; L.jqo_recompute_zobrist.restype = C.c_uint64
    L.jqo_belief_row.argtypes = [C.c_int, P]
    L.jqo_sizeof_game.restype = C.c_int
    L.jqo_omp_threads.restype = C.c_int
    L.jqo_batch_new.argtypes = [P, C.c_int, P, C.c_int, C.c_int]
    L.jqo_batch_env_step.argtypes = [P, C.c_int, P, P, P, P, P, C.c_int]
    L.jqo_batch_env_step.restype = C.c_long
    L.jqo_tables_export.argtypes = [P] * 9
    I = C.c_int
    L.jqo_world_to_canonical.argtypes = [I, I, I, P, P]
    L.jqo_canonical_to_world.argtypes = [I, I, I, P, P]
    L.jqo_index_to_pos.argtypes = [I, I, P, P]
    L.jqo_canonical_id.argtypes = [I, I]; L.jqo_canonical_id.restype = I
    L.jqo_validate_lineup.argtypes = [P]; L.jqo_validate_lineup.restype = I
    L.jqo_cm_apply_event.argtypes = [P, I, I, I, I, I, I, I, I]
    L.jqo_cm_path_revealed_gongb.argtypes = [P, I]
    L.jqo_philox4x32_10.argtypes = [P, P, P]
    L.jqo_sample_uniform.argtypes = [P, I, I, C.c_uint64, C.c_uint64]; L.jqo_sample_uniform.restype = C.c_int32
    L.jqo_sample_logits.argtypes = [P, I, I, I, C.c_uint64, C.c_uint64, P]
    L.jqo_sample_logits.restype = C.c_int32
    L.jqo_reset_pool_index.argtypes = [I, C.c_int64, I]; L.jqo_reset_pool_index.restype = C.c_int32
    L.jqo_batch_rollout.argtypes = [P, I, P, I, I, C.c_uint64, C.c_uint64, C.c_int64, I, P, P, P, P, P, P, P]
    L.jqo_batch_rollout.restype = C.c_long
    L.jqo_batch_observe.argtypes = [P, I, I, P, P]
    L.jqo_batch_cpu_env_step.argtypes = [P, I, P, I, I, C.c_uint64, C.c_int64, C.c_int64, P, I, P, P, P, P]
    L.jqo_batch_cpu_env_step.restype = C.c_long
    L.jqo_set_threads.argtypes = [I]
    L.jqo_init()
    assert L.jqo_sizeof_game() == GAME_DTYPE.itemsize, (L.jqo_sizeof_game(), GAME_DTYPE.itemsize)
    if RECENCY_LUT_PATH.exists():
        lut = np.fromfile(RECENCY_LUT_PATH, dtype="<f4")
        assert lut.size == 4 * 4096
        L._lut_keep = np.ascontiguousarray(lut)
        L.jqo_set_recency_lut(L._lut_keep.ctypes.data)
    _lib = L
    return L


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def zobrist_tables() -> np.ndarray:
    L = lib()
    n = L.jqo_zobrist_count()
    ptr = L.jqo_zobrist_all()
    return np.ctypeslib.as_array(ptr, shape=(n,)).copy()


def pcg64_draw(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.uint64)
    lib().jqo_pcg64_draw(seed, n, _p(out))
    return out


def random_setup(seed: int) -> np.ndarray:
    out = np.zeros(120, dtype=np.int8)
    lib().jqo_random_setup(seed, _p(out))
    return out


def setup_pool(seed: int, size: int) -> np.ndarray:
    out = np.zeros((size, 120), dtype=np.int8)
    lib().jqo_setup_pool(seed, size, _p(out))
    return out


class MT:
    """CPython-compatible Mersenne Twister stream (random.Random(seed))."""

    def __init__(self, seed: int):
        self._buf = np.zeros(625, dtype=np.uint32)
        lib().jqo_mt_seed(_p(self._buf), seed)

    def u32(self) -> int:
        return int(lib().jqo_mt_u32(_p(self._buf)))

    def randbelow(self, n: int) -> int:
        return int(lib().jqo_mt_randbelow(_p(self._buf), n))

    def choice(self, seq):
        return seq[self.randbelow(len(seq))]

    def random_lineup(self) -> np.ndarray:
        """generate_random_lineup(rng) (junqi_core/setup.py:162-250) on this stream."""
        out = np.zeros(30, dtype=np.int8)
        lib().jqo_random_lineup(_p(self._buf), _p(out))
        return out


def styled_setups(mode: str, seed: int, count: int, styles, lineups: dict, *, per_game_seed: bool) -> np.ndarray:
    """Canonical / mixed setups (junqi_rl/gpu_rollout.py:278-382 pools from one
    random.Random(seed) stream; :701-728 reset with random.Random(seed + i) per
    game). `lineups` maps a style letter to its 30 seat-local types."""
    out = np.zeros((count, 120), dtype=np.int8)
    shared = MT(seed)
    for i in range(count):
        rng = MT(seed + i) if per_game_seed else shared
        own = np.asarray(lineups[rng.choice(list(styles))], dtype=np.int8)
        for s in range(4):
            if mode == "mixed" and s in (1, 3):
                out[i, 30 * s:30 * s + 30] = rng.random_lineup()
            else:
                out[i, 30 * s:30 * s + 30] = own
    return out


class Game:
    """One oracle game (GameState restatement)."""

    def __init__(self, setup=None, *, show_mode: int = 2, max_num_moves: int = 4000):
        self.buf = np.zeros(1, dtype=GAME_DTYPE)
        if setup is not None:
            s = np.ascontiguousarray(np.asarray(setup, dtype=np.int8).reshape(120))
            rc = lib().jqo_new_game(_p(self.buf), _p(s), show_mode, max_num_moves)
            assert rc == 0

    @classmethod
    def from_pieces(cls, pieces, *, turn=0, move_counter=0, mslc=0, seat_dead=(0, 0, 0, 0),
                    flag_rev=(0, 0, 0, 0), show_mode=2, max_num_moves=4000) -> "Game":
        g = cls(None)
        arr = np.ascontiguousarray(np.asarray(pieces, dtype=np.int32).reshape(-1, 4))
        sd = np.asarray(seat_dead, dtype=np.int8)
        fr = np.asarray(flag_rev, dtype=np.int8)
        rc = lib().jqo_from_pieces(_p(g.buf), len(arr), _p(arr), turn, move_counter, mslc,
                                   _p(sd), _p(fr), show_mode, max_num_moves)
        if rc != 0:
            raise ValueError(f"bad piece list ({rc})")
        return g

    def __getattr__(self, name):
        if name in GAME_DTYPE.names:
            return self.buf[0][name]
        raise AttributeError(name)

    def clone(self) -> "Game":
        g = Game(None)
        g.buf = self.buf.copy()
        return g

    def legal_ids(self, seat: int | None = None) -> np.ndarray:
        seat = int(self.buf[0]["turn"]) if seat is None else seat
        out = np.zeros(8192, dtype=np.int32)
        n = lib().jqo_legal_ids(_p(self.buf), seat, _p(out), 8192)
        assert n >= 0
        return out[:n].copy()

    def legal_slots(self, seat: int | None = None) -> np.ndarray:
        """(120, 80) bool per-piece slot mask (game_state.cu:1964-2197)."""
        seat = int(self.buf[0]["turn"]) if seat is None else seat
        out = np.zeros((120, 80), dtype=np.uint8)
        lib().jqo_legal_slots(_p(self.buf), seat, _p(out))
        return out.astype(bool)

    def is_legal(self, seat: int, src: int, dst: int) -> bool:
        return bool(lib().jqo_is_legal(_p(self.buf), seat, src, dst))

    def has_legal(self, seat: int) -> bool:
        return bool(lib().jqo_has_legal(_p(self.buf), seat))

    def step(self, src: int, dst: int) -> tuple[int, dict]:
        r = Result()
        rc = lib().jqo_step(_p(self.buf), src, dst, C.byref(r))
        return rc, r.as_dict()

    def step_id(self, action_id: int) -> tuple[int, dict]:
        return self.step(action_id // NC, action_id % NC)

    def observe(self, observer: int, beliefs: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
        """Observation of `observer`; `beliefs` (12, 289) float32 world-cell
        beliefs of that observer replace the BeliefTensor belief planes."""
        sp = np.zeros((OBS_C, 17, 17), dtype=np.float32)
        gl = np.zeros(OBS_G, dtype=np.float32)
        if beliefs is None:
            lib().jqo_observe(_p(self.buf), observer, _p(sp), _p(gl))
        else:
            b = np.ascontiguousarray(beliefs, dtype=np.float32).reshape(12, 289)
            lib().jqo_observe_ext(_p(self.buf), observer, _p(b), _p(sp), _p(gl))
        return sp, gl

    def cm_apply_event(self, *, is_eat: bool, attacker_pid: int, defender_pid: int, attacker_seat: int,
                       defender_seat: int, attacker_type: int, defender_type: int, step: int) -> None:
        """apply_combat_event (combat_memory.py:354-569) on this game's memory."""
        lib().jqo_cm_apply_event(_p(self.buf), int(is_eat), attacker_pid, defender_pid, attacker_seat,
                                 defender_seat, attacker_type, defender_type, step)

    def cm_path_revealed_gongb(self, pid: int) -> None:
        lib().jqo_cm_path_revealed_gongb(_p(self.buf), pid)

    def recompute_zobrist(self) -> int:
        return int(lib().jqo_recompute_zobrist(_p(self.buf)))

    @property
    def zobrist_i64(self) -> int:
        return int(np.int64(self.buf[0]["zobrist"].view(np.int64)))


def world_to_canonical(x: int, y: int, seat: int) -> tuple[int, int]:
    """rotation.world_to_canonical (rotation.py:44-61)."""
    cx, cy = C.c_int(), C.c_int()
    lib().jqo_world_to_canonical(x, y, seat, C.byref(cx), C.byref(cy))
    return cx.value, cy.value


def canonical_to_world(x: int, y: int, seat: int) -> tuple[int, int]:
    """rotation.canonical_to_world (rotation.py:64-80)."""
    wx, wy = C.c_int(), C.c_int()
    lib().jqo_canonical_to_world(x, y, seat, C.byref(wx), C.byref(wy))
    return wx.value, wy.value


def index_to_pos(seat: int, i: int) -> tuple[int, int]:
    """board.index_to_pos (board.py:88-102)."""
    x, y = C.c_int(), C.c_int()
    lib().jqo_index_to_pos(seat, i, C.byref(x), C.byref(y))
    return x.value, y.value


def canonical_id(seat: int, world_id: int) -> int:
    return int(lib().jqo_canonical_id(seat, world_id))


# violation bits of validate_lineup (setup.py:60-136)
V_TYPE, V_C1, V_C2, V_C3, V_C4, V_C5 = 1, 2, 4, 8, 16, 32
V_NAMES = {V_TYPE: "TYPE", V_C1: "C1", V_C2: "C2", V_C3: "C3", V_C4: "C4", V_C5: "C5"}


def validate_lineup(lineup) -> set[str]:
    """Violation codes of one seat's 30-entry lineup (empty set = valid)."""
    lu = np.ascontiguousarray(np.asarray(lineup, dtype=np.int64))
    if lu.size != 30:
        return {"LENGTH"}
    if (lu < -128).any() or (lu > 127).any():
        return {"TYPE"}
    v = int(lib().jqo_validate_lineup(_p(np.ascontiguousarray(lu.astype(np.int8)))))
    return {name for bit, name in V_NAMES.items() if v & bit}


def philox4x32_10(ctr, key) -> tuple[int, int, int, int]:
    c = np.asarray(ctr, dtype=np.uint32)
    k = np.asarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().jqo_philox4x32_10(_p(c), _p(k), _p(out))
    return tuple(int(v) for v in out)


def sample_uniform(ids: np.ndarray, env: int, seed: int, ply: int) -> int:
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    return int(lib().jqo_sample_uniform(_p(ids), len(ids), env, seed, ply))


def sample_logits(ids: np.ndarray, seat: int, env: int, seed: int, ply: int) -> tuple[int, int]:
    """(world id, canonical id) of the masked N(0,1)-logit argmax."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    c = C.c_int32(-1)
    w = int(lib().jqo_sample_logits(_p(ids), len(ids), seat, env, seed, ply, C.byref(c)))
    return w, int(c.value)


def reset_pool_index(env: int, seed: int, pool_size: int) -> int:
    return int(lib().jqo_reset_pool_index(env, seed, pool_size))


def belief_row(code: int) -> np.ndarray:
    out = np.zeros(12, dtype=np.float32)
    lib().jqo_belief_row(code, _p(out))
    return out


def tables() -> dict:
    on = np.zeros(NC, np.int8); rail = np.zeros(NC, np.int8); camp = np.zeros(NC, np.int8)
    sh = np.zeros(NC, np.int8); ng = np.zeros(NC, np.int8); cid = np.zeros(NC, np.int8)
    arc = np.zeros(NC, np.int8); c2f = np.zeros(ONB, np.int16); radj = np.zeros((NC, 4), np.int16)
    lib().jqo_tables_export(*(_p(a) for a in (on, rail, camp, sh, ng, cid, arc, c2f, radj)))
    return dict(on_board=on, rail=rail, camp=camp, stronghold=sh, ninegrid=ng, curve=cid,
                arc=arc, compact_to_flat=c2f, rail_adj=radj)


class Batch:
    """N oracle games stepped together (OpenMP over envs); the CPU baseline."""

    def __init__(self, setups: np.ndarray, *, show_mode: int = 2, max_num_moves: int = 4000):
        setups = np.ascontiguousarray(setups, dtype=np.int8).reshape(-1, 120)
        self.n = setups.shape[0]
        self.games = np.zeros(self.n, dtype=GAME_DTYPE)
        lib().jqo_batch_new(_p(self.games), self.n, _p(setups), show_mode, max_num_moves)
        self.counts = np.zeros(self.n, dtype=np.int32)

    def env_step(self, actions: np.ndarray, *, obs: bool = True, mask_bits: np.ndarray | None = None,
                 obs_spatial: np.ndarray | None = None, obs_global: np.ndarray | None = None) -> int:
        actions = np.ascontiguousarray(actions, dtype=np.int32)
        sp = _p(obs_spatial) if obs_spatial is not None else None
        gl = _p(obs_global) if obs_global is not None else None
        mb = _p(mask_bits) if mask_bits is not None else None
        if obs and (sp is None or gl is None):
            raise ValueError("obs=True needs obs_spatial and obs_global buffers")
        return int(lib().jqo_batch_env_step(_p(self.games), self.n, _p(actions), _p(self.counts),
                                            mb, sp, gl, 1 if obs else 0))


LEGAL_DIGEST_P = 0x100000001B3


def legal_digest(ids) -> int:
    """Digest of one legal-id row as the rollout records it: sum ids[j] * P^j mod 2^64."""
    d, w = 0, 1
    for a in np.asarray(ids).tolist():
        d = (d + (a & 0xFFFFFFFF) * w) & (2**64 - 1)
        w = (w * LEGAL_DIGEST_P) & (2**64 - 1)
    return d


def rollout(batch: "Batch", pool: np.ndarray, *, sampler: int, seed: int, ply0: int, reset_seed0: int,
            steps: int, active_from: np.ndarray | None = None) -> dict:
    """jqo_batch_rollout over a Batch: (steps, n) reward / done / hash / actions /
    legal_count / legal_digest."""
    n = batch.n
    pool = np.ascontiguousarray(pool, dtype=np.int8).reshape(-1, 120)
    out = {"reward": np.zeros((steps, n), np.float32), "done": np.zeros((steps, n), np.uint8),
           "hash": np.zeros((steps, n), np.uint64), "actions": np.zeros((steps, n), np.int32),
           "legal_count": np.zeros((steps, n), np.int32), "legal_digest": np.zeros((steps, n), np.uint64)}
    au = None if active_from is None else np.ascontiguousarray(active_from, dtype=np.int32)
    applied = lib().jqo_batch_rollout(_p(batch.games), n, _p(pool), len(pool), sampler, seed, ply0, reset_seed0,
                                      steps, None if au is None else _p(au), _p(out["reward"]), _p(out["done"]),
                                      _p(out["hash"]), _p(out["actions"]), _p(out["legal_count"]),
                                      _p(out["legal_digest"]))
    out["applied"] = int(applied)
    return out


def batch_observe(batch: "Batch", g0: int, g1: int) -> tuple[np.ndarray, np.ndarray]:
    """Acting-seat float32 observations of games [g0, g1)."""
    sp = np.zeros((g1 - g0, OBS_C, 17, 17), np.float32)
    gl = np.zeros((g1 - g0, OBS_G), np.float32)
    lib().jqo_batch_observe(_p(batch.games), g0, g1, _p(sp), _p(gl))
    return sp, gl


class CpuEnv:
    """The CPU baseline: n oracle games stepped with jqo_batch_cpu_env_step."""

    CAP = 1024

    def __init__(self, setups: np.ndarray, pool: np.ndarray, *, show_mode: int = 2, max_num_moves: int = 4000):
        self.batch = Batch(setups, show_mode=show_mode, max_num_moves=max_num_moves)
        self.n = self.batch.n
        self.pool = np.ascontiguousarray(pool, dtype=np.int8).reshape(-1, 120)
        self.ids = np.zeros((self.n, self.CAP), np.int32)
        self.counts = np.zeros(self.n, np.int32)
        self.mask = np.zeros((self.n, 2081), np.uint8)
        self.sp = np.zeros((self.n, OBS_C, 17, 17), np.float32)
        self.gl = np.zeros((self.n, OBS_G), np.float32)
        self.step(-1, sampler=0, seed=0, obs=False)

    def step(self, ply: int, *, sampler: int, seed: int, obs: bool = True) -> int:
        return int(lib().jqo_batch_cpu_env_step(
            _p(self.batch.games), self.n, _p(self.pool), len(self.pool), sampler, seed, ply, ply, _p(self.ids),
            self.CAP, _p(self.counts), _p(self.mask), _p(self.sp) if obs else None, _p(self.gl) if obs else None))


def set_threads(n: int) -> None:
    lib().jqo_set_threads(int(n))


def omp_threads() -> int:
    return int(lib().jqo_omp_threads())

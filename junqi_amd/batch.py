"""Host handle over the HIP library: N games resident in HBM.

``JunqiBatch`` owns one C-ABI handle and the torch device buffers its calls
write. Torch provides device memory and the current HIP stream; every rule,
legal move and observation is computed by the library's kernels.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import torch

from . import _lib as L
from ._lib import check, lib

DATA = Path(__file__).resolve().parent / "data"
ZOBRIST_SEED = 0x4A554E51495F5A4F
_ZOB_SHAPES = [(120, 14, 289), (4,), (4096,), (512,), (1,), (3,), (1,), (4,), (4,), (4,)]


def zobrist_stream() -> np.ndarray:
    """The Zobrist tables in draw order of junqi_core/_zobrist.py:80-106
    (numpy PCG64, the reference's own dependency), as one uint64 array."""
    rng = np.random.default_rng(ZOBRIST_SEED)
    parts = [rng.integers(low=0, high=np.iinfo(np.uint64).max, size=s, dtype=np.uint64,
                          endpoint=True).ravel() for s in _ZOB_SHAPES]
    return np.ascontiguousarray(np.concatenate(parts))


def recency_table() -> np.ndarray:
    """float32[4][4096]: exp(-e/tau) for tau planes (32, 256, 64, 128), the values
    junqi_core/observation.py:1561-1562 produces with numpy."""
    lut = np.fromfile(DATA / "recency_lut_f32.bin", dtype="<f4")
    if lut.size != 4 * 4096:
        raise RuntimeError("corrupt recency table")
    return np.ascontiguousarray(lut)


def generate_lineups(seed_base: int, count: int) -> np.ndarray:
    out = np.zeros((count, 120), dtype=np.int8)
    check(lib.jq_generate_lineups(int(seed_base), int(count), out.ctypes.data))
    return out


def generate_pool(seed: int, size: int) -> np.ndarray:
    out = np.zeros((size, 120), dtype=np.int8)
    check(lib.jq_generate_pool(int(seed), int(size), out.ctypes.data))
    return out


def decode_table() -> np.ndarray:
    out = np.zeros(256, dtype=np.float32)
    check(lib.jq_obs_decode_table(out.ctypes.data))
    return out


def _split_aux(aux):
    """(..., 2320) aux rows -> turn-history floats (..., 2) and recency codes (..., 4, 289)."""
    if isinstance(aux, torch.Tensor):
        turn = aux[..., :8].contiguous().view(torch.float32)
        codes = aux[..., 8:].contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
        return turn, codes.reshape(aux.shape[:-1] + (4, 289))
    a = np.ascontiguousarray(aux)
    return a[..., :8].copy().view(np.float32), a[..., 8:].copy().view(np.uint16).astype(np.int64).reshape(
        a.shape[:-1] + (4, 289))


def decode_u8(spatial, aux):
    """float32 observation (..., 317, 17, 17) from JQ_OBS_U8 codes and aux rows
    (torch tensors on any device, or numpy arrays): codes through the decode
    table, planes 64-65 from the aux floats, planes 253-256 from the recency
    table at the aux codes."""
    if isinstance(spatial, torch.Tensor):
        dev = spatial.device
        dec = torch.from_numpy(decode_table()).to(dev)
        out = dec[spatial.long()]
        turn, codes = _split_aux(aux)
        out[..., 64:66, :, :] = turn[..., :, None, None]
        rl = torch.from_numpy(recency_table().reshape(4, 4096)).to(dev)
        q = torch.arange(4, device=dev).view((1,) * (codes.dim() - 2) + (4, 1)).expand_as(codes)
        vals = torch.where(codes > 0, rl[q, (codes - 1).clamp(min=0)], torch.zeros((), device=dev))
        out[..., 253:257, :, :] = vals.reshape(codes.shape[:-1] + (17, 17))
        return out
    out = decode_table()[np.asarray(spatial)]
    turn, codes = _split_aux(aux)
    out[..., 64:66, :, :] = turn[..., :, None, None]
    rl = recency_table().reshape(4, 4096)
    vals = np.where(codes > 0, rl[np.arange(4)[:, None], np.maximum(codes - 1, 0)], np.float32(0))
    out[..., 253:257, :, :] = vals.reshape(codes.shape[:-1] + (17, 17)).astype(np.float32)
    return out


_CM_FIELDS = ("cm_direct_lo", "cm_direct_hi", "cm_direct_type", "cm_last_direct", "cm_other_count",
              "cm_chain_lo", "cm_chain_hi", "cm_chain_type", "cm_last_chain", "cm_eaten_lo", "cm_eaten_hi",
              "cm_floor", "cm_floor_step", "cm_flags")


class _CudaArrayView:
    """__cuda_array_interface__ wrapper so torch can view library-owned memory."""

    def __init__(self, ptr: int, shape: tuple[int, ...], typestr: str, strides: tuple[int, ...] | None = None):
        self.__cuda_array_interface__ = {"data": (int(ptr), False), "shape": tuple(shape),
                                         "typestr": typestr, "strides": strides, "version": 2}


_TYPESTR = {(1, "i"): "|i1", (1, "u"): "|u1", (2, "i"): "<i2", (2, "u"): "<u2", (4, "i"): "<i4",
            (8, "u"): "<u8"}
_FIELD_KIND = {"hist": "i", "hist_meta": "i", "move_counter": "i", "mslc": "i", "zobrist": "u",
               "belief": "u", "rem_tracked": "u", "cm_direct_lo": "u", "cm_direct_hi": "u",
               "cm_direct_type": "u", "cm_chain_lo": "u", "cm_chain_hi": "u", "cm_chain_type": "u",
               "cm_eaten_lo": "u", "cm_eaten_hi": "u", "cm_flags": "u", "terminated": "u", "draw": "u",
               "seat_dead": "u", "flag_rev": "u"}


class JunqiBatch:
    """N four-player Junqi games on one GPU."""

    def __init__(self, num_envs: int, *, show_mode: int = 2, max_num_moves: int = 4000,
                 device: int = 0, setup_pool: np.ndarray | None = None, pool_seed: int = 42,
                 pool_size: int = 10000):
        if num_envs <= 0:
            raise ValueError(f"num_envs must be positive, got {num_envs}")
        if not torch.cuda.is_available():
            raise RuntimeError("no GPU visible: junqi_amd runs on the device only")
        self.n = int(num_envs)
        self.show_mode = int(show_mode)
        self.device = torch.device("cuda", device)
        h = C.c_void_p()
        with torch.cuda.device(self.device):
            check(lib.jq_create(C.byref(h), self.n, int(max_num_moves), self.show_mode, int(device)))
        self._h = h
        z = zobrist_stream()
        check(lib.jq_upload_zobrist(h, z.ctypes.data, z.size))
        r = recency_table()
        check(lib.jq_upload_recency(h, r.ctypes.data))
        pool = generate_pool(pool_seed, pool_size) if setup_pool is None else np.ascontiguousarray(
            setup_pool, dtype=np.int8).reshape(-1, 120)
        self.upload_setup_pool(pool)
        dev = self.device
        self.counts = torch.zeros(self.n, dtype=torch.int32, device=dev)
        self.offsets = torch.zeros(self.n + 1, dtype=torch.int32, device=dev)
        self.values = torch.zeros(self.n * L.MAX_LEGAL, dtype=torch.int32, device=dev)
        self.mask_words = torch.zeros((self.n, L.MASK_WORDS), dtype=torch.int32, device=dev)

    # ------------------------------------------------------------ lifetime
    def close(self) -> None:
        if getattr(self, "_h", None):
            lib.jq_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    @staticmethod
    def _ptr(t: torch.Tensor | None) -> int | None:
        return None if t is None else t.data_ptr()

    # ------------------------------------------------------------ reset
    def upload_setup_pool(self, pool: np.ndarray) -> None:
        pool = np.ascontiguousarray(pool, dtype=np.int8).reshape(-1, 120)
        check(lib.jq_upload_setup_pool(self._h, pool.ctypes.data, pool.shape[0]))
        self.pool = pool

    def reset(self, seed_base: int = 0) -> None:
        check(lib.jq_reset_seeded(self._h, int(seed_base), self.stream))

    def reset_lineups(self, lineups: np.ndarray) -> None:
        lu = np.ascontiguousarray(lineups, dtype=np.int8).reshape(self.n, 120)
        check(lib.jq_reset_lineups(self._h, lu.ctypes.data, self.stream))

    def reset_terminated(self, seed: int) -> None:
        check(lib.jq_reset_terminated(self._h, int(seed), self.stream))

    # ------------------------------------------------------------ step
    def step(self, actions: torch.Tensor, acting: torch.Tensor | None = None, *,
             canonical: bool = False) -> dict[str, torch.Tensor]:
        a = actions.to(device=self.device, dtype=torch.int32).contiguous()
        if a.shape != (self.n,):
            raise ValueError(f"actions: expected ({self.n},), got {tuple(a.shape)}")
        s = None
        if acting is not None:
            s = acting.to(device=self.device, dtype=torch.int8).contiguous()
            if s.shape != (self.n,):
                raise ValueError(f"acting: expected ({self.n},), got {tuple(s.shape)}")
        if canonical and s is None:
            raise ValueError("canonical actions need the acting seats")
        dev, n = self.device, self.n
        out = {
            "valid": torch.empty(n, dtype=torch.bool, device=dev),
            "event": torch.empty(n, dtype=torch.int8, device=dev),
            "terminated": torch.empty(n, dtype=torch.bool, device=dev),
            "winner_team": torch.empty(n, dtype=torch.int8, device=dev),
            "draw": torch.empty(n, dtype=torch.bool, device=dev),
            "flag_captured": torch.empty(n, dtype=torch.bool, device=dev),
            "seats_died": torch.empty(n, dtype=torch.uint8, device=dev),
            "rewards": torch.empty(n, dtype=torch.float32, device=dev),
            "world_action": torch.empty(n, dtype=torch.int32, device=dev),
        }
        p = self._ptr
        check(lib.jq_step(self._h, a.data_ptr(), p(s), L.ACT_CANONICAL if canonical else L.ACT_WORLD,
                          p(out["valid"]), p(out["event"]), p(out["terminated"]), p(out["winner_team"]),
                          p(out["draw"]), p(out["flag_captured"]), p(out["seats_died"]), p(out["rewards"]),
                          p(out["world_action"]), self.stream))
        return out

    # ------------------------------------------------------------ legal actions
    def legal(self, acting: torch.Tensor | None = None, *, csr: bool = True, mask_words: bool = True,
              mask_bool: bool = False) -> dict[str, torch.Tensor]:
        s = None if acting is None else acting.to(device=self.device, dtype=torch.int8).contiguous()
        mb = torch.empty((self.n, L.ACTION_DIM), dtype=torch.bool, device=self.device) if mask_bool else None
        p = self._ptr
        check(lib.jq_legal(self._h, p(s), self.counts.data_ptr(),
                           self.offsets.data_ptr() if csr else None, self.values.data_ptr() if csr else None,
                           self.values.numel(), self.mask_words.data_ptr() if mask_words else None, p(mb),
                           self.stream))
        out = {"counts": self.counts}
        if csr:
            out["offsets"] = self.offsets
            out["values"] = self.values
        if mask_words:
            out["mask_words"] = self.mask_words
        if mask_bool:
            out["mask_bool"] = mb
        return out

    def legal_slots(self, acting: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
        """(N, 120, 80) bool per-piece slot mask of the acting seats (legal_action_mask_batch,
        game_state.cu:1964-2197)."""
        s = None if acting is None else acting.to(device=self.device, dtype=torch.int8).contiguous()
        shape = (self.n, L.NUM_PIDS, L.SLOTS_PER_PIECE)
        if out is None:
            out = torch.empty(shape, dtype=torch.bool, device=self.device)
        elif tuple(out.shape) != shape or out.dtype != torch.bool or not out.is_contiguous():
            raise ValueError(f"slot mask output must be a contiguous bool tensor of shape {shape}")
        check(lib.jq_legal_slots(self._h, self._ptr(s), out.data_ptr(), self.stream))
        return out

    def legal_csr_numpy(self, acting: torch.Tensor | None = None) -> tuple[np.ndarray, np.ndarray]:
        self.legal(acting, csr=True, mask_words=False)
        offsets = self.offsets.cpu().numpy()
        values = self.values[: int(offsets[-1])].cpu().numpy()
        return offsets, values

    # ------------------------------------------------------------ observations
    def observe(self, observer: torch.Tensor | None = None, *, fmt: str = "f32", all_seats: bool = False,
                out_spatial: torch.Tensor | None = None, out_global: torch.Tensor | None = None,
                out_aux: torch.Tensor | None = None):
        code = {"f32": L.OBS_F32, "bf16": L.OBS_BF16, "u8": L.OBS_U8}[fmt]
        dt = {"f32": torch.float32, "bf16": torch.bfloat16, "u8": torch.uint8}[fmt]
        lead = (self.n, 4) if all_seats else (self.n,)
        if out_spatial is None:
            out_spatial = torch.empty(lead + (L.OBS_CHANNELS, 17, 17), dtype=dt, device=self.device)
        if out_global is None:
            out_global = torch.empty(lead + (L.OBS_GLOBALS,), dtype=torch.float32, device=self.device)
        if fmt == "u8" and out_aux is None:
            out_aux = torch.empty(lead + (L.AUX_BYTES,), dtype=torch.uint8, device=self.device)
        if tuple(out_spatial.shape) != lead + (L.OBS_CHANNELS, 17, 17) or out_spatial.dtype != dt:
            raise ValueError("out_spatial has the wrong shape or dtype")
        s = None if observer is None else observer.to(device=self.device, dtype=torch.int8).contiguous()
        check(lib.jq_observe(self._h, self._ptr(s), code, 1 if all_seats else 0, out_spatial.data_ptr(),
                             self._ptr(out_aux) if fmt == "u8" else None, out_global.data_ptr(), self.stream))
        if fmt == "u8":
            return out_spatial, out_global, out_aux
        return out_spatial, out_global

    def upload_beliefs(self, beliefs) -> None:
        """Observations read their belief planes from (N, 4, 12, 289) float32
        world-cell beliefs (host array or device tensor) until clear_beliefs()."""
        shape = (self.n, 4, 12, 289)
        if isinstance(beliefs, torch.Tensor):
            if tuple(beliefs.shape) != shape:
                raise ValueError(f"beliefs shape must be {shape}, got {tuple(beliefs.shape)}")
            if beliefs.device.type != "cuda":
                beliefs = beliefs.numpy()
            else:
                src = beliefs.to(device=self.device, dtype=torch.float32).contiguous()
                self._bel_src = src   # kept alive until the copy has run
                check(lib.jq_upload_beliefs(self._h, src.data_ptr(), 0, self.stream))
                return
        a = np.ascontiguousarray(beliefs, dtype=np.float32)
        if a.shape != shape:
            raise ValueError(f"beliefs shape must be {shape}, got {a.shape}")
        check(lib.jq_upload_beliefs(self._h, a.ctypes.data, 1, self.stream))
        torch.cuda.synchronize(self.device)   # the host array may go away

    def clear_beliefs(self) -> None:
        """Return observations to the device's own BeliefTensor beliefs."""
        check(lib.jq_clear_beliefs(self._h))

    # ------------------------------------------------------------ sampling / fused step
    def sample_uniform(self, seed: int, ply: int, out: torch.Tensor | None = None) -> torch.Tensor:
        """World action per env, uniform over the current CSR rows (Philox)."""
        if out is None:
            out = torch.empty(self.n, dtype=torch.int32, device=self.device)
        check(lib.jq_sample_uniform(self._h, self.counts.data_ptr(), self.offsets.data_ptr(),
                                    self.values.data_ptr(), self.values.numel(), int(seed), int(ply),
                                    out.data_ptr(), self.stream))
        return out

    def sample_logits(self, seed: int, ply: int, acting: torch.Tensor | None = None,
                      out: torch.Tensor | None = None, canonical_out: torch.Tensor | None = None) -> torch.Tensor:
        """World action per env: argmax of i.i.d. N(0,1) logits (Philox) over the
        acting seat's legal canonical ids of the current CSR rows."""
        if out is None:
            out = torch.empty(self.n, dtype=torch.int32, device=self.device)
        s = None if acting is None else acting.to(device=self.device, dtype=torch.int8).contiguous()
        check(lib.jq_sample_logits(self._h, self._ptr(s), self.counts.data_ptr(), self.offsets.data_ptr(),
                                   self.values.data_ptr(), self.values.numel(), int(seed), int(ply),
                                   out.data_ptr(), self._ptr(canonical_out), self.stream))
        return out

    def env_step(self, *, actions: torch.Tensor | None = None, sampler: str = "uniform", sample_seed: int = 0,
                 ply: int = 0, reset_seed: int = 0, obs_fmt: str = "u8", spatial: torch.Tensor | None = None,
                 aux: torch.Tensor | None = None, glob: torch.Tensor | None = None,
                 terminated: torch.Tensor | None = None, reward: torch.Tensor | None = None,
                 hash_out: torch.Tensor | None = None, actions_out: torch.Tensor | None = None) -> None:
        """One fused env-step (jq_env_step): sample from the current CSR rows
        unless `actions` are given (sampler "uniform" or "logits"), step,
        restart finished games from the pool, next legal sets, observation."""
        code = {"f32": L.OBS_F32, "bf16": L.OBS_BF16, "u8": L.OBS_U8}[obs_fmt]
        smp = {"uniform": L.SAMPLE_UNIFORM, "logits": L.SAMPLE_LOGITS}[sampler]
        p = self._ptr
        check(lib.jq_env_step(self._h, p(actions), smp, int(sample_seed), int(ply), int(reset_seed),
                              self.counts.data_ptr(), self.offsets.data_ptr(), self.values.data_ptr(),
                              self.values.numel(), self.mask_words.data_ptr(), code, p(spatial), p(aux), p(glob),
                              p(terminated), p(reward), p(hash_out), p(actions_out), self.stream))

    # ------------------------------------------------------------ state import / export
    def get_field(self, name: str) -> np.ndarray:
        e, b = L.field_info(name)
        kind = _FIELD_KIND.get(name, "i")
        dt = np.dtype(_TYPESTR[(b, kind)])
        out = np.zeros((self.n, e), dtype=dt)
        check(lib.jq_get_field(self._h, L.FIELDS[name], out.ctypes.data))
        return out

    def set_field(self, name: str, arr: np.ndarray) -> None:
        e, b = L.field_info(name)
        kind = _FIELD_KIND.get(name, "i")
        dt = np.dtype(_TYPESTR[(b, kind)])
        a = np.ascontiguousarray(np.asarray(arr).astype(dt, copy=False).reshape(self.n, e))
        check(lib.jq_set_field(self._h, L.FIELDS[name], a.ctypes.data))

    def finalize_import(self) -> None:
        check(lib.jq_finalize_import(self._h, self.stream))

    def rehash(self) -> None:
        """Zobrist hashes and combat-memory summaries from the current fields;
        beliefs stay as set."""
        check(lib.jq_rehash(self._h, self.stream))
        torch.cuda.synchronize(self.device)

    def _fields_from_dict(self, sd: dict) -> dict[str, np.ndarray]:
        """This handle's per-env fields from the flat SoA dict of the reference's
        DeviceGameStateBatch.copy_from_host (bindings.cpp:73-112; the keys of
        junqi_rl/gpu_rollout.py:447-483): per-piece arrays of N*120,
        cell_piece_id of N*289, seat arrays of N*4, per-env turn / move_counter /
        moves_since_last_combat. Missing keys raise KeyError, wrong sizes ValueError."""
        n = self.n

        def arr(key, shape, dt):
            if key not in sd:
                raise KeyError(f"state dict: missing key {key!r}")
            a = np.asarray(sd[key])
            if a.size != int(np.prod(shape)):
                raise ValueError(f"state dict: {key} has {a.size} elements, expected {int(np.prod(shape))}")
            return a.reshape(shape).astype(dt, copy=False)

        alive = arr("alive", (n, 120), bool)
        ptype = arr("piece_type_arr", (n, 120), np.int16)
        px, py = arr("pos_x", (n, 120), np.int16), arr("pos_y", (n, 120), np.int16)
        zx, zy = arr("zero_x", (n, 120), np.int16), arr("zero_y", (n, 120), np.int16)
        cpid = arr("cell_piece_id", (n, 289), np.int16)

        def pid128(a, fill, dt):
            out = np.full((n, 128), fill, dt)
            out[:, :120] = a
            return out
        cell = np.full((n, 292), -1, np.int8)
        cell[:, :289] = cpid
        bits = np.arange(4, dtype=np.uint8)
        f = {
            "cell": cell,
            "ptype": pid128(np.where(ptype > 0, ptype, -1), -1, np.int8),
            "pos": pid128(np.where(alive & (px >= 0) & (py >= 0), py * 17 + px, -1), -1, np.int16),
            "zero": pid128(np.where((zx >= 0) & (zy >= 0), zy * 17 + zx, -1), -1, np.int16),
            "death_reason": pid128(arr("death_reason_arr", (n, 120), np.int8), -1, np.int8),
            "death_step": pid128(arr("death_step_arr", (n, 120), np.int16), -1, np.int16),
            "death_loc": pid128(arr("death_loc_flat_arr", (n, 120), np.int16), -1, np.int16),
            "seat_dead": (arr("seat_dead_arr", (n, 4), np.uint8) << bits).sum(-1).astype(np.uint8).reshape(n, 1),
            "flag_rev": (arr("seat_flag_revealed_arr", (n, 4), np.uint8) << bits).sum(-1).astype(np.uint8).reshape(n, 1),
            "turn": arr("turn", (n,), np.int8).reshape(n, 1),
            "move_counter": arr("move_counter", (n,), np.int32).reshape(n, 1),
            "mslc": arr("moves_since_last_combat", (n,), np.int32).reshape(n, 1),
        }
        for ours, key in (("move_count", "move_count_arr"), ("active_eat", "active_eat_arr"),
                          ("passive_surv", "passive_surv_arr")):
            f[ours] = pid128(arr(key, (n, 120), np.int16), 0, np.int16)
        return f

    def _clear_history_and_memory(self, rows: np.ndarray | None = None) -> None:
        """Empty combat memory and move history for the envs in `rows` (bool N; all when None)."""
        n = self.n
        for name in _CM_FIELDS + ("hist", "hist_meta"):
            e, _ = L.field_info(name)
            fill = -1 if name in ("cm_last_direct", "cm_last_chain", "cm_floor_step") else 0
            if rows is None:
                self.set_field(name, np.full((n, e), fill, np.int64))
            else:
                cur = self.get_field(name)
                cur[rows] = fill
                self.set_field(name, cur)

    def import_state(self, sd: dict, *, terminated=None, winner_team=None, draw=None,
                     move_history=None) -> None:
        """Load every env from the flat SoA dict that the reference's
        ``DeviceGameStateBatch.copy_from_host`` takes (see _fields_from_dict).
        Combat memory starts empty and beliefs are re-seeded from the board, as
        GameState.__post_init__ does for a state built from arrays
        (state.py:346-483); the Zobrist hash is recomputed. move_history:
        optional list (one per env) of (src_flat, dst_flat) pairs, most recent last."""
        n = self.n
        for name, v in self._fields_from_dict(sd).items():
            self.set_field(name, v)
        self._clear_history_and_memory()
        hist = np.zeros((n, 32), np.int32)
        meta = np.zeros((n, 1), np.int32)
        for i, h in enumerate(move_history or []):
            h = list(h)[-32:]
            for k, (s, d) in enumerate(h):
                hist[i, k] = int(s) | (int(d) << 16)
            meta[i, 0] = len(h) | ((len(h) & 31) << 8)
        self.set_field("hist", hist)
        self.set_field("hist_meta", meta)
        self.set_termination(np.zeros(n, bool) if terminated is None else terminated,
                             np.full(n, -1, np.int8) if winner_team is None else winner_team,
                             np.zeros(n, bool) if draw is None else draw, finalize=False)
        self.finalize_import()

    # ---------------------------------------------- DeviceGameStateBatch host copies
    # The host round trip of the reference's device state (bindings.cpp:73-243)
    # as the v1 PPO collector drives it through GpuRollout.state
    # (junqi_rl/training/gpu_collector.py:375, 538, 602-650).
    def copy_turn_to_host(self) -> np.ndarray:
        """(N,) int8 acting seat per env (py_copy_turn_to_host, bindings.cpp:186-194)."""
        return self.get_field("turn")[:, 0].astype(np.int8)

    def copy_to_host(self) -> dict[str, np.ndarray]:
        """The 21 flat arrays of py_copy_to_host (bindings.cpp:117-183), keys and
        dtypes as there: per-piece arrays N*120, cell_piece_id N*289, seat flags
        N*4, turn / zobrist / move_counter / moves_since_last_combat N."""
        n = self.n
        pos = self.get_field("pos")[:, :120].astype(np.int16)
        alive = pos >= 0
        ptype = self.get_field("ptype")[:, :120].astype(np.int8)
        zero = self.get_field("zero")[:, :120].astype(np.int16)
        seat = np.where(ptype >= 0, np.arange(120, dtype=np.int8)[None, :] // 30, np.int8(-1)).astype(np.int8)
        bits = np.arange(4, dtype=np.uint8)
        flat = lambda a: np.ascontiguousarray(a).reshape(-1)  # noqa: E731
        return {
            "cell_piece_id_per_piece": flat(np.where(alive, pos, -1).astype(np.int16)),
            "piece_seat_arr": flat(seat),
            "piece_type_arr": flat(ptype),
            "alive": flat(alive),
            "pos_x": flat(np.where(alive, pos % 17, -1).astype(np.int8)),
            "pos_y": flat(np.where(alive, pos // 17, -1).astype(np.int8)),
            "zero_x": flat(np.where(zero >= 0, zero % 17, -1).astype(np.int8)),
            "zero_y": flat(np.where(zero >= 0, zero // 17, -1).astype(np.int8)),
            "move_count_arr": flat(self.get_field("move_count")[:, :120].astype(np.int16)),
            "active_eat_arr": flat(self.get_field("active_eat")[:, :120].astype(np.int16)),
            "passive_surv_arr": flat(self.get_field("passive_surv")[:, :120].astype(np.int16)),
            "death_reason_arr": flat(self.get_field("death_reason")[:, :120].astype(np.int8)),
            "death_step_arr": flat(self.get_field("death_step")[:, :120].astype(np.int16)),
            "death_loc_flat_arr": flat(self.get_field("death_loc")[:, :120].astype(np.int16)),
            "cell_piece_id": flat(self.get_field("cell")[:, :289].astype(np.int16)),
            "seat_dead_arr": flat(((self.get_field("seat_dead")[:, :1] >> bits) & 1).astype(bool)),
            "seat_flag_revealed_arr": flat(((self.get_field("flag_rev")[:, :1] >> bits) & 1).astype(bool)),
            "turn": flat(self.get_field("turn")[:, 0].astype(np.int8)),
            "zobrist": flat(self.get_field("zobrist")[:, 0].view(np.int64)),
            "move_counter": flat(self.get_field("move_counter")[:, 0].astype(np.int32)),
            "moves_since_last_combat": flat(self.get_field("mslc")[:, 0].astype(np.int32)),
        }

    def copy_from_host(self, sd: dict) -> None:
        """Write the copy_to_host dict back (py_copy_from_host, bindings.cpp:73-112).
        Envs whose position the dict leaves as it is keep everything; an env
        whose fields it changes (the v1 collector writes fresh games into reset
        slots, gpu_collector.py:596-643) starts from the imported position as a
        GameState built from arrays does (state.py:346-483): empty combat memory
        and move history, beliefs seeded from the board, the Zobrist hash
        recomputed from the fields (the dict's zobrist is not read)."""
        n = self.n
        new = self._fields_from_dict(sd)
        cur = {k: self.get_field(k) for k in new}
        width = {k: (289 if k == "cell" else 120 if v.shape[1] == 128 else v.shape[1]) for k, v in new.items()}
        changed = np.zeros(n, bool)
        for k, v in new.items():   # padding columns (pids 120-127, cells 289-291) are the handle's own
            w = width[k]
            changed |= (cur[k].reshape(n, -1)[:, :w] != v.reshape(n, -1)[:, :w]).any(axis=1)
        if not changed.any():
            return
        for k, v in new.items():
            merged = cur[k].reshape(n, -1).copy()
            w = width[k]
            merged[changed, :w] = v.reshape(n, -1)[changed, :w]
            self.set_field(k, merged)
        self._clear_history_and_memory(changed)
        mask = torch.from_numpy(changed.astype(np.uint8)).to(self.device)
        check(lib.jq_finalize_import_masked(self._h, mask.data_ptr(), self.stream))

    def copy_termination_to_host(self) -> dict[str, np.ndarray]:
        """terminated / winner_team / draw (py_copy_termination_to_host, bindings.cpp:216-231)."""
        return self.termination()

    def copy_termination_from_host(self, terminated, winner_team, draw) -> None:
        """py_copy_termination_from_host (bindings.cpp:201-214); hashes follow."""
        for name, a in (("terminated", terminated), ("winner_team", winner_team), ("draw", draw)):
            if np.asarray(a).size != self.n:
                raise ValueError(f"{name} size mismatch")
        self.set_termination(terminated, winner_team, draw)
        torch.cuda.synchronize(self.device)

    def set_termination(self, terminated, winner_team, draw, *, finalize: bool = True) -> None:
        """Overwrite the per-env terminated / winner_team / draw flags
        (copy_termination_from_host, bindings.cpp:200-243); the Zobrist hash is
        recomputed when `finalize`."""
        n = self.n
        self.set_field("terminated", np.asarray(terminated).reshape(n).astype(np.uint8))
        self.set_field("winner", np.asarray(winner_team).reshape(n).astype(np.int8))
        self.set_field("draw", np.asarray(draw).reshape(n).astype(np.uint8))
        if finalize:
            check(lib.jq_rehash(self._h, self.stream))

    def termination(self) -> dict[str, np.ndarray]:
        """terminated / winner_team / draw on the host (copy_termination_to_host)."""
        return {"terminated": self.get_field("terminated")[:, 0].astype(bool),
                "winner_team": self.get_field("winner")[:, 0].astype(np.int8),
                "draw": self.get_field("draw")[:, 0].astype(bool)}

    def field_tensor(self, name: str, torch_dtype: torch.dtype | None = None) -> torch.Tensor:
        """Zero-copy (strided) device view of a per-env state field, shape (N, elems) or (N,)."""
        e, b = L.field_info(name)
        ptr, es, ls = C.c_void_p(), C.c_int64(), C.c_int64()
        check(lib.jq_field_ptr(self._h, L.FIELDS[name], C.byref(ptr), C.byref(es), C.byref(ls)))
        kind = _FIELD_KIND.get(name, "i")
        ts = _TYPESTR[(b, kind)]
        if torch_dtype is torch.bool:
            ts = "|b1"
        shape, strides = ((self.n,), (es.value,)) if e == 1 else ((self.n, e), (es.value, ls.value))
        return torch.as_tensor(_CudaArrayView(ptr.value, shape, ts, strides), device=self.device)

    def sync(self) -> None:
        torch.cuda.synchronize(self.device)

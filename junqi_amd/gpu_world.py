"""``GpuWorld``: the numpy-facing facade of the reference (junqi_rl/gpu_world.py:97-319)
over the MI355X library.

Same method names, shapes, dtypes and errors (``ValueError`` for bad shapes or
seat dtypes). State arrives from CPU environments exactly as the reference packs
it (``env.state`` GameState SoA arrays, junqi_rl/env_gpu.py:151-236).
"""

from __future__ import annotations

import numpy as np
import torch

from . import _lib as L
from .batch import JunqiBatch
from .gpu_rollout import _dense_from_csr, _show_value


def _pack_state_arrays(envs) -> tuple[dict, dict]:
    """The copy_from_host dict of N CPU environments (each with a GameState at
    ``.state``) plus their termination flags and move histories."""
    states = [e.state for e in envs]
    cat = lambda name: np.concatenate([np.asarray(getattr(s, name)) for s in states])  # noqa: E731
    sd = {k: cat(k) for k in ("alive", "piece_seat_arr", "piece_type_arr", "pos_x", "pos_y", "zero_x", "zero_y",
                              "move_count_arr", "active_eat_arr", "passive_surv_arr", "death_reason_arr",
                              "death_step_arr", "death_loc_flat_arr", "cell_piece_id", "seat_dead_arr",
                              "seat_flag_revealed_arr")}
    sd["turn"] = np.array([int(getattr(s.turn, "value", s.turn)) for s in states], np.int8)
    sd["move_counter"] = np.array([int(s.move_counter) for s in states], np.int32)
    sd["moves_since_last_combat"] = np.array([int(s.moves_since_last_combat) for s in states], np.int32)
    extra = {
        "terminated": np.array([bool(getattr(s, "terminated", False)) for s in states]),
        "winner_team": np.array([-1 if getattr(s, "winner_team", None) is None
                                 else int(getattr(s.winner_team, "value", s.winner_team)) for s in states], np.int8),
        "draw": np.array([bool(getattr(s, "draw", False)) for s in states]),
        "move_history": [list(getattr(s, "move_history", [])) for s in states],
    }
    return sd, extra


class GpuWorld:
    """N Junqi worlds on one GPU (junqi_rl/gpu_world.py:97)."""

    def __init__(self, num_envs: int, *, device_id: int = 0, init_tables: bool = True,
                 show_mode: int = 2, max_num_moves: int = 4000) -> None:
        if num_envs <= 0:
            raise ValueError(f"num_envs must be positive, got {num_envs}")
        if not torch.cuda.is_available() or torch.cuda.device_count() == 0:
            raise RuntimeError("No GPU found")
        self.num_envs = int(num_envs)
        self._device_id = int(device_id)
        self.state = JunqiBatch(self.num_envs, show_mode=_show_value(show_mode), max_num_moves=max_num_moves,
                                device=self._device_id)
        self.device = self.state.device

    # ------------------------------------------------------------ state upload
    def push_state_from_envs(self, envs) -> None:
        """Pack state from N CPU envs and upload it (gpu_world.py:148-157)."""
        if len(envs) != self.num_envs:
            raise ValueError(f"push_state_from_envs: got {len(envs)} envs, expected {self.num_envs}")
        sd, extra = _pack_state_arrays(envs)
        self.state.import_state(sd, terminated=extra["terminated"], winner_team=extra["winner_team"],
                                draw=extra["draw"], move_history=extra["move_history"])

    def push_state_lite(self, envs) -> None:
        """Upload for legal-action queries (gpu_world.py:159-174); the full state
        goes up, which serves the same queries."""
        if len(envs) != self.num_envs:
            raise ValueError(f"push_state_lite: got {len(envs)} envs, expected {self.num_envs}")
        self.push_state_from_envs(envs)

    def push_state_arrays(self, sd: dict, **termination) -> None:
        """Upload a copy_from_host dict directly (JunqiBatch.import_state)."""
        self.state.import_state(sd, **termination)

    # ------------------------------------------------------------ legal actions
    def _validate_acting_seats(self, acting_seats: np.ndarray) -> None:
        if acting_seats.shape != (self.num_envs,):
            raise ValueError(f"acting_seats: expected shape ({self.num_envs},), got {acting_seats.shape}")
        if acting_seats.dtype != np.int8:
            raise ValueError(f"acting_seats: expected int8, got {acting_seats.dtype}")

    def legal_actions_dense(self, acting_seats: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        """(N,512) int32 ids (ascending, -1 padded) and (N,) counts (gpu_world.py:178-188)."""
        self._validate_acting_seats(acting_seats)
        ids, counts = _dense_from_csr(self.state, torch.from_numpy(acting_seats).to(self.device))
        return ids.cpu().numpy(), counts.cpu().numpy()

    def legal_actions_csr(self, acting_seats: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        """(offsets (N+1,) int32, values int32): env i's ascending ids at
        values[offsets[i]:offsets[i+1]] (gpu_world.py:190-206)."""
        self._validate_acting_seats(acting_seats)
        return self.state.legal_csr_numpy(torch.from_numpy(acting_seats).to(self.device))

    def legal_actions_mask(self, acting_seats: np.ndarray) -> np.ndarray:
        """(N, 120, 80) bool per-piece slot mask (gpu_world.py:208-217): slot
        layout of legal_action_mask_batch (game_state.cu:1964-2197)."""
        self._validate_acting_seats(acting_seats)
        return self.state.legal_slots(torch.from_numpy(acting_seats).to(self.device)).cpu().numpy()

    # ------------------------------------------------------------ step
    def step_batch(self, action_ids: np.ndarray) -> dict:
        """One ply per env from world ids src_flat*289 + dst_flat; returns host
        valid / event / terminated / winner_team / draw / flag_captured
        (gpu_world.py:223-253)."""
        action_ids = np.asarray(action_ids)
        if action_ids.shape != (self.num_envs,):
            raise ValueError(f"action_ids: expected shape ({self.num_envs},), got {action_ids.shape}")
        out = self.state.step(torch.from_numpy(action_ids.astype(np.int32, copy=False)).to(self.device))
        return {k: out[k].cpu().numpy() for k in ("valid", "event", "terminated", "winner_team", "draw",
                                                  "flag_captured")}

    def push_termination_state(self, terminated: np.ndarray, winner_team: np.ndarray, draw: np.ndarray) -> None:
        """Overwrite terminated / winner_team / draw (gpu_world.py:255-265)."""
        self.state.set_termination(terminated, winner_team, draw)

    def pull_termination_state(self) -> dict:
        return self.state.termination()

    # ------------------------------------------------------------ observations
    def build_observation(self, beliefs: np.ndarray | None = None, observer_seats: np.ndarray | None = None,
                          show_mode: int = 2) -> tuple[np.ndarray, np.ndarray]:
        """(N,4,317,17,17) and (N,4,28) float32 on the host (gpu_world.py:276-293).
        `beliefs` (N,4,12,289) float32 world-cell beliefs feed the belief planes
        of this call (None: the device's own BeliefTensor beliefs); `show_mode`
        must be the mode the world was created with."""
        if _show_value(show_mode) != self.state.show_mode:
            raise ValueError(f"show_mode {show_mode} differs from the world's show mode {self.state.show_mode}")
        obs = None
        if observer_seats is not None:
            a = np.asarray(observer_seats)
            if a.shape != (self.num_envs, 4):
                raise ValueError(f"observer_seats shape must be ({self.num_envs}, 4), got {a.shape}")
            obs = torch.from_numpy(a.astype(np.int8)).to(self.device)
        if beliefs is not None:
            self.state.upload_beliefs(np.asarray(beliefs, dtype=np.float32))
        try:
            sp, gl = self.state.observe(obs, fmt="f32", all_seats=True)
            return sp.cpu().numpy(), gl.cpu().numpy()
        finally:
            if beliefs is not None:
                self.state.clear_beliefs()

    def release_scratch(self) -> None:
        """No per-call scratch exists (all buffers belong to the handle)."""
        torch.cuda.synchronize(self.device)

    def __repr__(self) -> str:
        return f"GpuWorld(num_envs={self.num_envs}, device_id={self._device_id})"

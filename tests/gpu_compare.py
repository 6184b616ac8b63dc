"""Helpers that line the device state up against oracle games (tests only)."""

from __future__ import annotations

import numpy as np

from oracle import oracle as O

CM_FIELDS = [("cm_direct_lo", "cm_direct_lo"), ("cm_direct_hi", "cm_direct_hi"),
             ("cm_direct_type", "cm_direct_type"), ("cm_last_direct", "cm_last_direct"),
             ("cm_other_count", "cm_other_cnt"), ("cm_chain_lo", "cm_chain_lo"),
             ("cm_chain_hi", "cm_chain_hi"), ("cm_chain_type", "cm_chain_type"),
             ("cm_last_chain", "cm_last_chain"), ("cm_eaten_lo", "cm_eaten_lo"),
             ("cm_eaten_hi", "cm_eaten_hi"), ("cm_floor", "cm_floor"), ("cm_floor_step", "cm_floor_step")]


def flat_pos(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    x = x.astype(np.int32)
    y = y.astype(np.int32)
    return np.where((x >= 0) & (y >= 0), y * 17 + x, -1)


def oracle_fields(games: list) -> dict[str, np.ndarray]:
    """The oracle state laid out the way JunqiBatch.get_field returns it."""
    n = len(games)
    g = np.concatenate([gm.buf for gm in games])
    out = {}
    cell = np.full((n, 292), -1, np.int8)
    cell[:, :289] = g["cell_pid"]
    out["cell"] = cell

    def pid128(a, fill):
        r = np.full((n, 128), fill, a.dtype)
        r[:, :120] = a
        return r
    out["ptype"] = pid128(g["ptype"], -1)
    out["pos"] = pid128(flat_pos(g["pos_x"], g["pos_y"]).astype(np.int16), -1)
    out["zero"] = pid128(flat_pos(g["zero_x"], g["zero_y"]).astype(np.int16), -1)
    for a, b in (("move_count", "move_count"), ("active_eat", "active_eat"), ("passive_surv", "passive_surv")):
        out[a] = pid128(g[b], 0)
    out["death_reason"] = pid128(g["death_reason"], -1)
    out["death_step"] = pid128(g["death_step"], -1)
    out["death_loc"] = pid128(g["death_loc"], -1)

    def obs128(a, fill):
        r = np.full((n, 4, 128), fill, a.dtype)
        r[:, :, :120] = a
        return r.reshape(n, 4 * 128)
    out["belief"] = obs128(g["bcode"], 0)
    out["remaining"] = g["rem"].astype(np.int8).reshape(n, 4 * 48)
    out["rem_tracked"] = (g["rem_tracked"].astype(np.uint8) << np.arange(4, dtype=np.uint8)).sum(-1).astype(np.uint8)
    for dev, orc in CM_FIELDS:
        fill = -1 if orc in ("cm_last_direct", "cm_last_chain", "cm_floor_step") else 0
        out[dev] = obs128(g[orc], fill)
    flags = (g["cm_is_gongb"].astype(np.uint8) | (g["cm_not_gongb"].astype(np.uint8) << 1)
             | (g["cm_atk_gongb"].astype(np.uint8) << 2))
    out["cm_flags"] = obs128(flags, 0)
    out["turn"] = g["turn"].astype(np.int8)
    out["terminated"] = g["terminated"].astype(np.uint8)
    out["winner"] = g["winner"].astype(np.int8)
    out["draw"] = g["draw"].astype(np.uint8)
    bits = np.arange(4, dtype=np.uint8)
    out["seat_dead"] = (g["seat_dead"].astype(np.uint8) << bits).sum(-1).astype(np.uint8)
    out["flag_rev"] = (g["flag_rev"].astype(np.uint8) << bits).sum(-1).astype(np.uint8)
    out["move_counter"] = g["move_counter"].astype(np.int32)
    out["mslc"] = g["mslc"].astype(np.int32)
    out["zobrist"] = g["zobrist"].astype(np.uint64)
    out["hist_list"] = [[(int(s), int(d)) for s, d in gm.hist[: int(gm.hist_len)]] for gm in games]
    return out


def device_fields(batch) -> dict[str, np.ndarray]:
    names = ["cell", "ptype", "pos", "zero", "move_count", "active_eat", "passive_surv", "death_reason",
             "death_step", "death_loc", "belief", "remaining", "rem_tracked"] + [d for d, _ in CM_FIELDS] + [
        "cm_flags", "turn", "terminated", "winner", "draw", "seat_dead", "flag_rev", "move_counter", "mslc",
        "zobrist"]
    out = {}
    for nm in names:
        a = batch.get_field(nm)
        out[nm] = a[:, 0] if a.shape[1] == 1 else a
    hist = batch.get_field("hist")
    meta = batch.get_field("hist_meta")[:, 0]
    lists = []
    for i in range(batch.n):
        cnt, head = int(meta[i] & 0xFF), int((meta[i] >> 8) & 31)
        entries = [int(hist[i, (head - cnt + k) & 31]) for k in range(cnt)]
        lists.append([(e & 0xFFFF, (e >> 16) & 0xFFFF) for e in entries])
    out["hist_list"] = lists
    return out


def compare_state(dev: dict, orc: dict, envs=None, ctx: str = "") -> None:
    for k, v in orc.items():
        if k == "hist_list":
            for i, (a, b) in enumerate(zip(dev[k], v)):
                if envs is not None and i not in envs:
                    continue
                assert a == b, f"{ctx} env {i}: move history differs"
            continue
        d = dev[k]
        if envs is not None:
            d, v = d[envs], v[envs]
        if not np.array_equal(d, v):
            bad = np.argwhere(np.asarray(d != v).reshape(len(d), -1).any(1))[:, 0]
            i = int(bad[0])
            diff = np.nonzero(np.asarray(d[i] != v[i]).ravel())[0][:8] if np.ndim(d) > 1 else []
            raise AssertionError(f"{ctx} field {k} differs in {len(bad)} envs; first env {i} at {diff}: "
                                 f"device {np.ravel(d[i])[diff] if len(diff) else d[i]} "
                                 f"oracle {np.ravel(v[i])[diff] if len(diff) else v[i]}")


def canonical_mask_words(ids: np.ndarray, seat: int, tables: dict) -> np.ndarray:
    """Pack world ids into the (521,) int32 canonical compact mask row."""
    c2f = tables["compact_to_flat"]
    f2c = np.full(289, -1, np.int32)
    f2c[c2f] = np.arange(129)

    def rot(f):
        x, y = f % 17, f // 17
        cx, cy = [(x, y), (y, 16 - x), (16 - x, 16 - y), (16 - y, x)][seat]
        return cy * 17 + cx
    words = np.zeros(521, np.uint32)
    for a in ids.tolist():
        s, d = divmod(a, 289)
        bit = int(f2c[rot(s)]) * 129 + int(f2c[rot(d)])
        words[bit >> 5] |= np.uint32(1 << (bit & 31))
    return words.view(np.int32)


def reset_pool_index(env: int, seed: int, pool_size: int) -> int:
    """Pool pick of the device auto-reset (reference game_state.cu:2997-3001), from the oracle."""
    return O.reset_pool_index(env, seed, pool_size)


def philox_first_word(c0: int, c1: int, c2: int, c3: int, k0: int, k1: int) -> int:
    """Philox4x32-10 first output word, from the oracle (pinned by the Random123 vectors)."""
    return O.philox4x32_10((c0, c1, c2, c3), (k0, k1))[0]


def philox_first_word_np(c0: np.ndarray, c1: int, c2: int, c3: int, k0: int, k1: int) -> np.ndarray:
    """philox_first_word over an array of first counter words."""
    M = np.uint64(0xFFFFFFFF)
    c0 = np.asarray(c0, dtype=np.uint64)
    c1, c2, c3 = (np.full(c0.shape, v, dtype=np.uint64) for v in (c1, c2, c3))
    k0, k1 = np.uint64(k0), np.uint64(k1)
    for _ in range(10):
        p0 = np.uint64(0xD2511F53) * c0
        p1 = np.uint64(0xCD9E8D57) * c2
        c0, c1, c2, c3 = ((p1 >> np.uint64(32)) ^ c1 ^ k0) & M, p1 & M, ((p0 >> np.uint64(32)) ^ c3 ^ k1) & M, p0 & M
        k0 = (k0 + np.uint64(0x9E3779B9)) & M
        k1 = (k1 + np.uint64(0xBB67AE85)) & M
    return c0


def oracle_pack(games: list) -> dict[str, np.ndarray]:
    """The oracle games as the flat dict of DeviceGameStateBatch.copy_to_host /
    _pack_from_batched (bindings.cpp:117-183, junqi_rl/gpu_rollout.py:447-483)."""
    g = np.concatenate([gm.buf for gm in games])
    alive = g["alive"].astype(bool)
    flat = lambda a: np.ascontiguousarray(a).reshape(-1)  # noqa: E731
    return {
        "cell_piece_id_per_piece": flat(np.where(alive, flat_pos(g["pos_x"], g["pos_y"]), -1).astype(np.int16)),
        "piece_seat_arr": flat(g["pseat"].astype(np.int8)),
        "piece_type_arr": flat(g["ptype"].astype(np.int8)),
        "alive": flat(alive),
        "pos_x": flat(g["pos_x"].astype(np.int8)), "pos_y": flat(g["pos_y"].astype(np.int8)),
        "zero_x": flat(g["zero_x"].astype(np.int8)), "zero_y": flat(g["zero_y"].astype(np.int8)),
        "move_count_arr": flat(g["move_count"].astype(np.int16)),
        "active_eat_arr": flat(g["active_eat"].astype(np.int16)),
        "passive_surv_arr": flat(g["passive_surv"].astype(np.int16)),
        "death_reason_arr": flat(g["death_reason"].astype(np.int8)),
        "death_step_arr": flat(g["death_step"].astype(np.int16)),
        "death_loc_flat_arr": flat(g["death_loc"].astype(np.int16)),
        "cell_piece_id": flat(g["cell_pid"].astype(np.int16)),
        "seat_dead_arr": flat(g["seat_dead"].astype(bool)),
        "seat_flag_revealed_arr": flat(g["flag_rev"].astype(bool)),
        "turn": flat(g["turn"].astype(np.int8)),
        "zobrist": flat(g["zobrist"].view(np.int64)),
        "move_counter": flat(g["move_counter"].astype(np.int32)),
        "moves_since_last_combat": flat(g["mslc"].astype(np.int32)),
    }


def oracle_games_from_lineups(lineups: np.ndarray, show_mode: int, max_num_moves: int = 4000) -> list:
    return [O.Game(lu, show_mode=show_mode, max_num_moves=max_num_moves) for lu in lineups]

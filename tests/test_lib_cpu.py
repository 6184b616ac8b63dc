"""CPU-side checks of the HIP library: it loads, exports every declared symbol,
and its host-built tables and lineup streams equal the oracle's."""

from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def jl():
    from junqi_amd import _lib
    return _lib


def test_every_declared_symbol_is_exported(jl):
    header = (ROOT / "include" / "junqi_amd.h").read_text()
    declared = set(re.findall(r"^(?:int|const char \*|int32_t)\s*\*?\s*(jq_\w+)\(", header, re.M))
    assert declared, "no declarations found"
    assert declared == set(jl.exported_symbols())
    lib = C.CDLL(str(jl.LIB_PATH))
    for name in declared:
        assert hasattr(lib, name), name


def test_version_and_errors(jl):
    assert b"gfx950" in jl.lib.jq_version()
    assert jl.lib.jq_field_info(99, None, None) != 0
    assert b"bad field" in jl.lib.jq_last_error()


def _struct(fields):
    """numpy dtype of a C struct: fields (name, dtype, shape[, alignas]) laid out
    with natural alignment, or the given alignas, like the compiler does."""
    names, formats, offsets, off, maxal = [], [], [], 0, 1
    for name, fmt, shape, *al in fields:
        dt = np.dtype((fmt, shape))
        align = al[0] if al else dt.base.alignment
        off = (off + align - 1) // align * align
        names.append(name); formats.append(dt); offsets.append(off)
        off += dt.itemsize
        maxal = max(maxal, align)
    return np.dtype({"names": names, "formats": formats, "offsets": offsets,
                     "itemsize": (off + maxal - 1) // maxal * maxal})


# struct jq::Tables (junqi_amd/csrc/jq_topology.h)
_TABLES = _struct([
    ("cflags", "<u2", (289,)), ("adj", "<i2", (289, 4)), ("diag", "<i2", (289, 4)), ("railidx", "i1", (289,)),
    ("railcell", "<i2", (73,)), ("rnbr", "<u8", (73, 2)), ("rays", "<i2", (73, 4, 12)), ("raylen", "i1", (73, 4)),
    ("crays", "<i2", (73, 2, 11)), ("craylen", "i1", (73, 2)), ("f2c", "<i2", (289,)), ("c2f", "<i2", (129,)),
    ("rot", "<i2", (4, 289)), ("unrot", "<i2", (4, 289)), ("rotc", "u1", (4, 129)), ("home", "<i2", (120,)),
    ("slotch", "i1", (30,)), ("statics", "u1", (289,)), ("sh_other", "<i2", (289,)), ("owner", "i1", (289,)),
    ("localidx", "i1", (289,)),
    ("adjc", "u1", (129, 8), 8), ("adjm", "<u8", (129, 2, 3)), ("raym", "<u8", (73, 4, 3)), ("crayc", "u1", (73, 2, 16), 16),
    ("railc", "u1", (73,)), ("railidxc", "i1", (129,)), ("campm", "<u8", (3,)), ("onm", "<u8", (5,)),
    ("railm", "<u8", (5,)), ("shm", "<u8", (5,)), ("canc", "u1", (4, 289)),
])


def _bits(words, n):
    """The first n bits of a little-endian uint64 word array, as a bool vector."""
    w = np.asarray(words, np.uint64)
    return ((w[np.arange(n) >> 6] >> (np.arange(n) & 63).astype(np.uint64)) & np.uint64(1)).astype(bool)


def _product_tables(jl):
    buf = np.zeros(1, _TABLES)
    assert jl.lib.jq_board_tables(buf.ctypes.data, _TABLES.itemsize) == 0, jl.lib.jq_last_error()
    return buf[0]


def test_board_tables_equal_oracle(jl):
    t = _product_tables(jl)
    o = O.tables()
    fl = t["cflags"]
    assert np.array_equal((fl & 1) > 0, o["on_board"] > 0)
    assert np.array_equal((fl & 2) > 0, o["rail"] > 0)
    assert np.array_equal((fl & 4) > 0, o["camp"] > 0)
    assert np.array_equal((fl & 8) > 0, o["stronghold"] > 0)
    assert np.array_equal((fl & 16) > 0, o["ninegrid"] > 0)
    assert np.array_equal((fl & 32) > 0, o["arc"] > 0)
    assert np.array_equal(fl >> 8, o["curve"])
    assert np.array_equal(t["c2f"], o["compact_to_flat"])
    # world flat -> canonical compact: the composition of f2c and rotc
    on = t["f2c"] >= 0
    for s in range(4):
        assert np.array_equal(t["canc"][s][on], t["rotc"][s][t["f2c"][on]]) and (t["canc"][s][~on] == 255).all()
    # rail graph: the 73-bit neighbour masks against the oracle adjacency lists
    for i in range(73):
        f = int(t["railcell"][i])
        got = {int(t["railcell"][j]) for j in range(73) if (int(t["rnbr"][i][j >> 6]) >> (j & 63)) & 1}
        want = {int(v) for v in o["rail_adj"][f] if v >= 0}
        assert got == want, f
    # straight and curve runs reproduce the oracle's destinations on an empty board
    g = O.Game.from_pieces([(0, 12, 8, 11)])
    for i in range(73):
        f = int(t["railcell"][i])
        runs = set()
        for k in range(4):
            runs |= {int(c) for c in t["rays"][i][k][: t["raylen"][i][k]]}
        for d in range(2):
            runs |= {int(c) for c in t["crays"][i][d][: t["craylen"][i][d]]}
        gg = O.Game.from_pieces([(0, 12, f % 17, f // 17)])
        ids = {int(a) % 289 for a in gg.legal_ids(0)} if not (fl[f] & 8) else set()
        road = {int(c) for c in t["adj"][f] if c >= 0} | {int(c) for c in t["diag"][f] if c >= 0}
        if not (fl[f] & 8):
            assert ids == runs | road, f
    # rotations are bijections and match rotation.py's point map
    for s in range(4):
        assert sorted(t["rot"][s].tolist()) == list(range(289))
        assert np.array_equal(t["unrot"][s][t["rot"][s]], np.arange(289))
    assert t["rot"][1][8 * 17 + 3] == 13 * 17 + 8    # WEST's centre camp (3,8) -> (8,13)
    assert t["rot"][3][8 * 17 + 13] == 13 * 17 + 8   # EAST's centre camp


def test_compact_move_tables(jl):
    """The compact-cell tables of the bitboard move generator against the oracle's
    board (on-board / rail / stronghold / camp cells, compact order) and against
    the flat run and neighbour tables they restate."""
    t = _product_tables(jl)
    o = O.tables()
    c2f = o["compact_to_flat"].astype(np.int64)
    f2c = np.full(289, -1, np.int64)
    f2c[c2f] = np.arange(129)
    assert np.array_equal(_bits(t["onm"], 289), o["on_board"] > 0)
    assert np.array_equal(_bits(t["railm"], 289), o["rail"] > 0)
    assert np.array_equal(_bits(t["shm"], 289), o["stronghold"] > 0)
    assert np.array_equal(_bits(t["campm"], 129), o["camp"][c2f] > 0)
    # ranks in the flat masks are the compact and rail indices
    on, rail = o["on_board"] > 0, o["rail"] > 0
    for f in range(289):
        if on[f]:
            assert int(on[:f].sum()) == f2c[f]
        if rail[f]:
            assert int(rail[:f].sum()) == t["railidx"][f] and t["railcell"][t["railidx"][f]] == f
    assert np.array_equal(t["railc"], f2c[t["railcell"]])
    assert np.array_equal(t["railidxc"], t["railidx"][c2f])
    for c in range(129):
        f = int(c2f[c])
        want = {int(f2c[v]) for v in t["adj"][f] if v >= 0} | {int(f2c[v]) for v in t["diag"][f] if v >= 0}
        got = [int(v) for v in t["adjc"][c] if v != 0xFF]
        assert len(got) == len(set(got)) and set(got) == want, c
        for h in range(2):   # each half's neighbours as a bit set
            half = {int(v) for v in t["adjc"][c][4 * h: 4 * h + 4] if v != 0xFF}
            assert set(np.flatnonzero(_bits(t["adjm"][c][h], 129))) == half, (c, h)
    for i in range(73):
        src = int(f2c[t["railcell"][i]])
        for k in range(4):
            cells = [int(f2c[v]) for v in t["rays"][i][k][: t["raylen"][i][k]]]
            assert set(np.flatnonzero(_bits(t["raym"][i][k], 129))) == set(cells), (i, k)
            # a straight run walks away from its source in compact order: up for +x / +y, down for -x / -y
            seq = [src] + cells
            assert all((b > a) if k in (0, 2) else (b < a) for a, b in zip(seq, seq[1:])), (i, k)
        for d in range(2):
            n = int(t["craylen"][i][d])
            assert np.array_equal(t["crayc"][i][d][:n], f2c[t["crays"][i][d][:n]]), (i, d)
            assert np.all(t["crayc"][i][d][n:] == 0xFF)


@pytest.mark.parametrize("seed", [0, 1, 42, 2026, 123456789])
def test_lineups_equal_oracle(jl, seed):
    from junqi_amd.batch import generate_lineups
    got = generate_lineups(seed, 6)
    for i in range(6):
        assert np.array_equal(got[i], O.random_setup(seed + i))


def test_pool_equals_oracle(jl):
    from junqi_amd.batch import generate_pool
    assert np.array_equal(generate_pool(42, 50), O.setup_pool(42, 50))


def test_decode_table(jl):
    from junqi_amd.batch import decode_table
    d = decode_table()
    assert d[0] == 0 and d[1] == 1 and d[2] == -1
    assert d[3] == np.float32(1) / np.float32(3) and d[4] == np.float32(2) / np.float32(3)
    vals = set(d[:32].tolist())
    for code in list(range(1, 13)) + [16 + s for s in range(30)] + [64]:
        for v in O.belief_row(code):
            assert float(v) in vals


def test_packaged_recency_table_is_the_fixture():
    a = (ROOT / "junqi_amd" / "data" / "recency_lut_f32.bin").read_bytes()
    b = (ROOT / "tests" / "golden" / "recency_lut_f32.bin").read_bytes()
    assert a == b


def test_zobrist_stream_matches_oracle(jl):
    from junqi_amd.batch import zobrist_stream
    assert np.array_equal(zobrist_stream(), O.zobrist_tables())


def test_mirror_helpers_without_gpu():
    """Argument handling of the GpuRollout / GpuWorld mirrors that needs no device."""
    import types

    from junqi_amd.gpu_rollout import _show_value
    from junqi_amd.gpu_world import _pack_state_arrays

    assert _show_value(1) == 1 and _show_value(types.SimpleNamespace(value=2)) == 2
    with pytest.raises(ValueError):
        _show_value(3)
    g = O.Game(O.random_setup(5))
    b = g.buf[0]
    st = types.SimpleNamespace(
        alive=b["alive"].astype(bool), piece_type_arr=b["ptype"], piece_seat_arr=b["pseat"], pos_x=b["pos_x"],
        pos_y=b["pos_y"], zero_x=b["zero_x"], zero_y=b["zero_y"], move_count_arr=b["move_count"],
        active_eat_arr=b["active_eat"], passive_surv_arr=b["passive_surv"], death_reason_arr=b["death_reason"],
        death_step_arr=b["death_step"], death_loc_flat_arr=b["death_loc"], cell_piece_id=b["cell_pid"],
        seat_dead_arr=b["seat_dead"].astype(bool), seat_flag_revealed_arr=b["flag_rev"].astype(bool),
        turn=types.SimpleNamespace(value=2), move_counter=7, moves_since_last_combat=3, terminated=False,
        winner_team=None, draw=False, move_history=[(10, 27)])
    sd, extra = _pack_state_arrays([types.SimpleNamespace(state=st)] * 2)
    assert sd["alive"].shape == (240,) and sd["cell_piece_id"].shape == (578,) and sd["seat_dead_arr"].shape == (8,)
    assert sd["turn"].tolist() == [2, 2] and sd["move_counter"].tolist() == [7, 7]
    assert extra["winner_team"].tolist() == [-1, -1] and extra["move_history"] == [[(10, 27)], [(10, 27)]]


def test_mask_helpers_validate_without_gpu():
    """Argument checks of the legal-support helpers that need no device; the
    helpers refuse host tensors instead of falling back to a host path."""
    import torch

    from junqi_amd.masks import csr_to_dense_selected, dense_mask_to_csr

    m = torch.zeros((4, 16641), dtype=torch.bool)
    with pytest.raises(ValueError, match="2-D bool"):
        dense_mask_to_csr(m.to(torch.uint8), torch.zeros((4, 8), dtype=torch.int32), torch.zeros(4, dtype=torch.int32))
    with pytest.raises(ValueError, match="shapes"):
        dense_mask_to_csr(m, torch.zeros((4, 0), dtype=torch.int32), torch.zeros(4, dtype=torch.int32))
    with pytest.raises(ValueError, match="int32"):
        dense_mask_to_csr(m, torch.zeros((4, 8), dtype=torch.int64), torch.zeros(4, dtype=torch.int32))
    with pytest.raises(ValueError, match="CUDA"):
        dense_mask_to_csr(m, torch.zeros((4, 8), dtype=torch.int32), torch.zeros(4, dtype=torch.int32))
    with pytest.raises(ValueError, match="CUDA"):
        csr_to_dense_selected(torch.zeros((4, 8), dtype=torch.int32), torch.zeros(4, dtype=torch.int32),
                              torch.zeros(2, dtype=torch.int64), 16641)


@pytest.mark.parametrize("mode", ["canonical", "mixed"])
@pytest.mark.parametrize("styles", [("T",), ("T", "D", "G", "F"), ("F", "F", "G")])
def test_styled_setups_match_oracle(jl, mode, styles):
    """jq_generate_styled (host code of the library) equals the oracle's
    restatement of the canonical / mixed pool builders and per-game resets,
    with the lineups taken from the fixture parsed out of setup_canonical.py."""
    import json

    from junqi_amd.setups import canonical_lineup, generate_styled
    from tests import helpers as H

    lu = json.loads((H.GOLDEN / "canonical_lineups.json").read_text())
    for k in "TDGF":
        assert np.array_equal(canonical_lineup(k), np.asarray(lu[k], np.int8))
    for per_game in (False, True):
        got = generate_styled(mode, 42, 64, styles, per_game_seed=per_game)
        want = O.styled_setups(mode, 42, 64, styles, lu, per_game_seed=per_game)
        assert np.array_equal(got, want), (mode, styles, per_game)


def test_styled_setup_errors(jl):
    from junqi_amd.setups import generate_styled

    with pytest.raises(ValueError, match="unknown setup styles"):
        generate_styled("canonical", 0, 4, ("T", "X"), per_game_seed=False)
    with pytest.raises(ValueError, match="non-empty"):
        generate_styled("mixed", 0, 4, (), per_game_seed=False)
    out = np.zeros((1, 120), np.int8)
    assert jl.lib.jq_generate_styled(7, 0, 1, 0, b"T", 1, out.ctypes.data) != 0
    assert b"bad setup mode" in jl.lib.jq_last_error()
    assert jl.lib.jq_generate_styled(1, 0, 1, 0, b"Q", 1, out.ctypes.data) != 0
    assert b"unknown setup style" in jl.lib.jq_last_error()


def test_arrangement_pools():
    """arrangements_to_pool (pool_upload.py:62-150): zip pairing keeps the k-th
    sample of every seat, independent pairing keeps that prefix and draws the
    tail per seat from that seat's samples; vocabulary indices round-trip."""
    import torch

    from junqi_amd.setups import arrangements_to_pool, lineups_to_vocab

    base = O.setup_pool(3, 12)                      # 12 setups -> 48 seat lineups
    vocab = lineups_to_vocab(base)                  # (12, 4, 30)
    assert vocab.max() <= 12 and vocab.min() >= 0
    seats = np.tile(np.arange(4), 12)
    order = np.random.default_rng(0).permutation(48)
    samples = torch.nn.functional.one_hot(torch.from_numpy(vocab.reshape(48, 30)[order]), 13).float()
    seat_idx = torch.from_numpy(seats[order])
    zip_pool = arrangements_to_pool(samples, seat_idx)
    assert zip_pool.shape == (12, 120)
    for s in range(4):
        rows = order[seats[order] == s]             # flat (setup*4 + seat) of seat s samples in order
        assert np.array_equal(zip_pool[:, 30 * s:30 * s + 30], base.reshape(48, 30)[rows])
    big = arrangements_to_pool(samples, seat_idx, pool_size=100, seed=7)
    assert big.shape == (100, 120) and np.array_equal(big[:12], zip_pool)
    assert np.array_equal(big, arrangements_to_pool(samples, seat_idx, pool_size=100, seed=7))
    for s in range(4):
        allowed = {tuple(r) for r in zip_pool[:, 30 * s:30 * s + 30]}
        assert {tuple(r) for r in big[:, 30 * s:30 * s + 30]} <= allowed
    with pytest.raises(ValueError, match="zero arrangement samples"):
        arrangements_to_pool(samples[seat_idx != 2], seat_idx[seat_idx != 2])
    with pytest.raises(ValueError, match="samples must be"):
        arrangements_to_pool(samples[:, :29], seat_idx)

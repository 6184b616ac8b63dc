"""ctypes binding of the C ABI in include/junqi_amd.h.

The shared library is built in-tree by ``junqi_amd/build.py``. If it is missing
this module raises at import time: there is no CPU fallback for any entry point.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_build" / "libjunqi_amd.so"

JQ_OK = 0
JQ_E_ARG, JQ_E_STATE, JQ_E_HIP, JQ_E_OOM, JQ_E_CAPACITY = -1, -2, -3, -4, -5
SAMPLE_UNIFORM, SAMPLE_LOGITS = 0, 1
OBS_F32, OBS_BF16, OBS_U8 = 0, 1, 2
ACT_WORLD, ACT_CANONICAL = 0, 1
NUM_CELLS = 289
NUM_ON_BOARD = 129
NUM_PIDS = 120
ACTION_DIM = 16641
MASK_WORDS = 521
OBS_CHANNELS = 317
OBS_GLOBALS = 28
AUX_BYTES = 2320   # u8 aux row: float32[2] turn history + uint16[4][289] recency codes
MAX_LEGAL = 3200
SLOTS_PER_PIECE = 80
SETUP_CANONICAL, SETUP_MIXED = 1, 2
NOALLOC_MAX_ROWS = 1024
AUX_CHANNELS = (64, 65, 253, 254, 255, 256)

FIELDS = {
    "cell": 0, "ptype": 1, "pos": 2, "zero": 3, "move_count": 4, "active_eat": 5, "passive_surv": 6,
    "death_reason": 7, "death_step": 8, "death_loc": 9, "belief": 10, "remaining": 11, "rem_tracked": 12,
    "cm_direct_lo": 13, "cm_direct_hi": 14, "cm_direct_type": 15, "cm_last_direct": 16,
    "cm_other_count": 17, "cm_chain_lo": 18, "cm_chain_hi": 19, "cm_chain_type": 20,
    "cm_last_chain": 21, "cm_eaten_lo": 22, "cm_eaten_hi": 23, "cm_floor": 24, "cm_floor_step": 25,
    "cm_flags": 26, "hist": 27, "hist_meta": 28, "turn": 29, "terminated": 30, "winner": 31,
    "draw": 32, "seat_dead": 33, "flag_rev": 34, "move_counter": 35, "mslc": 36, "zobrist": 37,
}

_EXPORTS = [
    "jq_last_error", "jq_version", "jq_create", "jq_destroy", "jq_num_envs", "jq_upload_zobrist",
    "jq_upload_recency", "jq_upload_setup_pool", "jq_reset_lineups", "jq_reset_seeded",
    "jq_generate_lineups", "jq_generate_pool", "jq_generate_styled", "jq_board_tables", "jq_reset_terminated", "jq_step",
    "jq_legal", "jq_legal_slots", "jq_observe", "jq_obs_timing", "jq_obs_timing_read", "jq_obs_decode_table",
    "jq_sample_uniform", "jq_sample_logits",
    "jq_env_step", "jq_field_info", "jq_get_field", "jq_set_field", "jq_field_ptr", "jq_finalize_import",
    "jq_finalize_import_masked", "jq_rehash", "jq_validate_lineup",
    "jq_sync", "jq_history_create", "jq_history_destroy", "jq_history_bytes", "jq_history_snapshot",
    "jq_history_reconstruct", "jq_history_reconstruct_noalloc", "jq_mask_count", "jq_mask_to_ids", "jq_ids_to_mask", "jq_upload_beliefs",
    "jq_clear_beliefs",
]


class JunqiError(RuntimeError):
    """A C-ABI call returned an error code."""


class ArgumentError(JunqiError, ValueError):
    """A call was given a bad argument (JQ_E_ARG): also a ValueError, which the
    reference raises for invalid setups and seats."""


class CapacityError(JunqiError):
    """An output buffer was smaller than the result (JQ_E_CAPACITY)."""


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"junqi_amd HIP library not built: {LIB_PATH} is missing "
            "(run `python junqi_amd/build.py` or __graft_entry__.build())")
    return bind(C.CDLL(str(LIB_PATH)))


def bind(L: C.CDLL) -> C.CDLL:
    """Declare the C-ABI signatures of include/junqi_amd.h on a loaded library."""
    P, I32, I64, U64 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64
    sig = {
        "jq_last_error": ([], C.c_char_p), "jq_version": ([], C.c_char_p),
        "jq_create": ([C.POINTER(P), I32, I32, I32, I32], C.c_int),
        "jq_destroy": ([P], C.c_int), "jq_num_envs": ([P], I32),
        "jq_upload_zobrist": ([P, P, I64], C.c_int), "jq_upload_recency": ([P, P], C.c_int),
        "jq_upload_setup_pool": ([P, P, I32], C.c_int), "jq_reset_lineups": ([P, P, P], C.c_int),
        "jq_reset_seeded": ([P, I64, P], C.c_int), "jq_generate_lineups": ([I64, I32, P], C.c_int),
        "jq_generate_pool": ([I64, I32, P], C.c_int),
        "jq_generate_styled": ([I32, I64, I32, I32, C.c_char_p, I32, P], C.c_int), "jq_board_tables": ([P, I64], C.c_int),
        "jq_reset_terminated": ([P, I64, P], C.c_int),
        "jq_step": ([P, P, P, I32, P, P, P, P, P, P, P, P, P, P], C.c_int),
        "jq_legal": ([P, P, P, P, P, I64, P, P, P], C.c_int),
        "jq_legal_slots": ([P, P, P, P], C.c_int),
        "jq_observe": ([P, P, I32, I32, P, P, P, P], C.c_int),
        "jq_obs_decode_table": ([P], C.c_int),
        "jq_obs_timing": ([P, I32], C.c_int),
        "jq_obs_timing_read": ([P, C.POINTER(C.c_double), C.POINTER(I64)], C.c_int),
        "jq_sample_uniform": ([P, P, P, P, I64, U64, U64, P, P], C.c_int),
        "jq_sample_logits": ([P, P, P, P, P, I64, U64, U64, P, P, P], C.c_int),
        "jq_env_step": ([P, P, I32, U64, U64, I64, P, P, P, I64, P, I32, P, P, P, P, P, P, P, P], C.c_int),
        "jq_validate_lineup": ([P], C.c_int),
        "jq_field_info": ([I32, C.POINTER(I32), C.POINTER(I32)], C.c_int),
        "jq_get_field": ([P, I32, P], C.c_int), "jq_set_field": ([P, I32, P], C.c_int),
        "jq_field_ptr": ([P, I32, C.POINTER(P), C.POINTER(I64), C.POINTER(I64)], C.c_int),
        "jq_finalize_import": ([P, P], C.c_int), "jq_finalize_import_masked": ([P, P, P], C.c_int),
        "jq_rehash": ([P, P], C.c_int),
        "jq_sync": ([P], C.c_int),
        "jq_history_create": ([C.POINTER(P), I32, I32, I32, I32], C.c_int),
        "jq_history_destroy": ([P], C.c_int), "jq_history_bytes": ([P, C.POINTER(I64)], C.c_int),
        "jq_history_snapshot": ([P, P, P, I32, P], C.c_int),
        "jq_history_reconstruct": ([P, P, P, I32, I32, P, P, P, P, P, P], C.c_int),
        "jq_history_reconstruct_noalloc": ([P, P, P, I32, I32, P, P, P, P, P, P], C.c_int),
        "jq_mask_count": ([P, I32, I32, P, P], C.c_int), "jq_mask_to_ids": ([P, I32, I32, I32, P, P], C.c_int),
        "jq_ids_to_mask": ([P, P, I64, I32, P, I32, I32, P, P], C.c_int),
        "jq_upload_beliefs": ([P, P, I32, P], C.c_int), "jq_clear_beliefs": ([P], C.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    return L


lib = _load()


def check(rc: int) -> None:
    """Raise for a failed call: ArgumentError (a ValueError) for bad arguments,
    CapacityError for a too small output buffer, JunqiError otherwise."""
    if rc != JQ_OK:
        msg = f"junqi_amd error {rc}: {lib.jq_last_error().decode()}"
        if rc == JQ_E_ARG:
            raise ArgumentError(msg)
        if rc == JQ_E_CAPACITY:
            raise CapacityError(msg)
        raise JunqiError(msg)


def exported_symbols() -> list[str]:
    return list(_EXPORTS)


def field_info(name: str) -> tuple[int, int]:
    e, b = C.c_int32(), C.c_int32()
    check(lib.jq_field_info(FIELDS[name], C.byref(e), C.byref(b)))
    return e.value, b.value

// Device-side state layout, constant tables and wave-level helpers shared by the
// step / legal / reset / observation kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

#include "jq_topology.h"

namespace jq {

constexpr int CELL_STRIDE = 292;   // 289 cells padded to a multiple of 4
constexpr int PID_STRIDE = 128;    // 120 pids padded
constexpr int HIST_LEN = 32;
constexpr int ZN_PIECE = 120 * 14 * 289;
constexpr int ZOFF_TURN = ZN_PIECE, ZOFF_MC = ZOFF_TURN + 4, ZOFF_MSLC = ZOFF_MC + 4096,
              ZOFF_TERM = ZOFF_MSLC + 512, ZOFF_WIN = ZOFF_TERM + 1, ZOFF_DRAW = ZOFF_WIN + 3,
              ZOFF_SDEAD = ZOFF_DRAW + 1, ZOFF_SFLAG = ZOFF_SDEAD + 4, ZOFF_SHOW = ZOFF_SFLAG + 4,
              ZTOTAL = ZOFF_SHOW + 4;

// piece types (reference junqi_core/rules.py:49-70)
enum : int { T_NONE = 0, T_JUNQI = 2, T_DILEI = 3, T_ZHADAN = 4, T_SILING = 5, T_GONGB = 13 };
enum : int { EV_NONE = 0, EV_MOVE = 1, EV_EAT = 2, EV_BOMB = 3, EV_KILLED = 4 };
enum : int { SM_BRIGHT = 0, SM_DARK = 1, SM_HALF_DARK = 2 };
enum : uint8_t { CMF_IS_GONGB = 1, CMF_NOT_GONGB = 2, CMF_ATK_GONGB = 4 };

// belief row codes: 0 zero, 1..12 one-hot(tracked idx+1), 16+slot prior row, 64 uniform
constexpr int BC_PRIOR0 = 16, BC_UNIFORM = 64, BC_COUNT = 65;

// Struct of device pointers; one handle owns all of them. Per-env blocks are
// contiguous so the wave that owns an env reads its rows with coalesced loads.
struct State {
    int32_t n, max_moves, show_mode, pool_size;
    int8_t *cell;          // [n][292]
    int8_t *ptype;         // [n][128]
    int16_t *pos, *zero;   // [n][128]
    int16_t *mcount, *aeat, *psurv;
    int8_t *dreason;
    int16_t *dstep, *dloc;
    uint8_t *bcode;        // [n][4][128]
    int8_t *rem;           // [n][4][4][12]
    uint8_t *remtrk;       // [n][4]
    uint64_t *cm_dlo, *cm_dhi, *cm_clo, *cm_chi, *cm_elo, *cm_ehi;  // [n][4][128]
    uint16_t *cm_dtype, *cm_ctype;
    int16_t *cm_ldir, *cm_ocnt, *cm_lchain, *cm_fstep;
    int8_t *cm_floor;
    uint8_t *cm_flags;
    int32_t *hist;         // [n][32]
    int32_t *hmeta;        // [n]  count | head << 8
    int8_t *turn;
    uint8_t *term;
    int8_t *winner;
    uint8_t *draw, *sdead, *sflag;
    int32_t *mc, *mslc;
    uint64_t *zob;
    const uint64_t *ztab;  // Zobrist stream
    const float *rlut;     // [4][4096]
    const int8_t *pool;    // [pool_size][120]
    // legal-set scratch consumed by the CSR emit kernel
    int16_t *lg_src;       // [n][32]
    uint64_t *lg_mask;     // [n][32][3]
    int32_t *lg_n;         // [n]
    int8_t *lg_seat;       // [n]
};

__device__ __forceinline__ size_t cm_idx(int env, int o, int pid) { return ((size_t)env * 4 + o) * PID_STRIDE + pid; }

}  // namespace jq

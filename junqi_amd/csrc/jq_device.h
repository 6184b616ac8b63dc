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

// One piece id of one env: everything the rules keep per piece, in one 16-byte
// record so a lane fetches it with a single dwordx4 load.
struct alignas(16) PieceRec {
    int16_t pos, zero;       // flat cells (-1 dead / none)
    int16_t dstep, dloc;     // death step and cell (-1 alive)
    int16_t mcount, aeat, psurv;
    int8_t ptype, dreason;   // PieceType (-1 absent), DeathReason (-1 alive)
};
static_assert(sizeof(PieceRec) == 16, "piece record must be 16 bytes");

// CombatMemory v6 of one (observer, pid) (combat_memory.py:251-311), in three
// arrays indexed alike (cm_idx): the record the observation reads for enemy
// pieces, the eaten-by set it reads for the observer's own pieces, and a byte
// summary (kill count capped at 3, flags) it reads where only that is used.
struct alignas(16) CmRec {
    uint64_t dlo, dhi;       // pids killed directly (120-bit set)
    uint64_t clo, chi;       // pids killed directly or by chain
    uint16_t dtype, ctype;   // tracked types killed directly / by chain (12 bits)
    int16_t ldir, ocnt, lchain, fstep;  // last direct step, other count, last chain step, floor step
    int8_t floor;
    uint8_t flags;           // CMF_*
    uint16_t pad;
};
static_assert(sizeof(CmRec) == 48, "combat-memory record must be 48 bytes");
struct alignas(16) CmEat {
    uint64_t elo, ehi;       // pids this (own) piece was eaten by
};
// summary byte: min(|killed directly| + other count, 3) | flags << 2
__device__ __forceinline__ uint8_t cm_summary(const CmRec &c)
{
    const int n = __popcll(c.dlo) + __popcll(c.dhi) + (c.ocnt > 0 ? c.ocnt : 0);
    return (uint8_t)((n < 3 ? n : 3) | ((c.flags & 7) << 2));
}

// What the observation of observer o uses of record (o, pid) for an enemy
// piece, derived from the record: the observer's own pieces it killed
// directly, types killed, floor, flags, counts capped at 3, recency steps.
struct alignas(16) CmView {
    uint32_t kmask;          // bit s: pid o*30 + s killed directly
    uint32_t types;          // dtype | ctype << 12 | floor << 24 | flags << 28
    uint16_t cnts;           // min(|direct|, 3) | min(|chain|, 3) << 2 | min(other, 3) << 4
    int16_t ldir, lchain, fstep;
};
static_assert(sizeof(CmView) == 16, "combat-memory view must be 16 bytes");

__device__ __forceinline__ CmView cm_view(const CmRec &c, int o)
{
    const int b = o * 30;   // the 30 pids of seat o in the 128-bit pid set (dlo, dhi)
    const uint64_t w = b == 0 ? c.dlo : b < 64 ? ((c.dlo >> b) | (c.dhi << (64 - b))) : (c.dhi >> (b - 64));
    const uint32_t k = (uint32_t)w & 0x3FFFFFFFu;
    const int m = __popcll(c.dlo) + __popcll(c.dhi), ch = __popcll(c.clo) + __popcll(c.chi);
    CmView v;
    v.kmask = k;
    const int fl = c.floor < 0 ? 0 : c.floor < 9 ? c.floor : 9;
    v.types = (uint32_t)(c.dtype & 0xFFF) | ((uint32_t)(c.ctype & 0xFFF) << 12) | ((uint32_t)fl << 24) |
              ((uint32_t)(c.flags & 7) << 28);
    const int oc = c.ocnt < 0 ? 0 : c.ocnt < 3 ? c.ocnt : 3;
    v.cnts = (uint16_t)((m < 3 ? m : 3) | ((ch < 3 ? ch : 3) << 2) | (oc << 4));
    v.ldir = c.ldir; v.lchain = c.lchain; v.fstep = c.fstep;
    return v;
}

// Per-env scalars.
struct alignas(16) EnvRec {
    uint64_t zob;
    int32_t mc, mslc;        // move counter, moves since last combat
    int32_t hmeta;           // move-history count | head << 8
    int8_t turn;
    uint8_t term;
    int8_t winner;           // -1 / 0 / 1
    uint8_t draw, sdead, sflag;   // seat bitmasks
    uint8_t remtrk[4];       // per observer: bit s = remaining[s] tracked
    uint8_t pad[2];
};
static_assert(sizeof(EnvRec) == 32, "env record must be 32 bytes");

// Legal-set scratch between k_legal and k_emit: per movable piece (ascending
// source cell) its 129-bit compact destination mask.
struct alignas(16) LegalRec {
    uint64_t mask[32][3];
    int16_t src[32];
    int32_t n, seat;
    int32_t pad[2];
};

// One handle's device arrays. Per-env blocks are contiguous so the wave that
// owns an env reads its rows with coalesced loads.
struct State {
    int32_t n, max_moves, show_mode, pool_size;
    int8_t *cell;          // [n][292]
    PieceRec *piece;       // [n][128]
    CmRec *cm;             // [n][4][128]
    CmEat *cme;            // [n][4][128]
    uint8_t *cmk;          // [n][4][128] cm_summary of cm
    CmView *cmv;           // [n][4][128] cm_view of cm for its observer
    uint8_t *bcode;        // [n][4][128]
    int8_t *rem;           // [n][4][4][12]
    EnvRec *env;           // [n]
    int32_t *hist;         // [n][32]
    LegalRec *lg;          // [n]
    const uint64_t *ztab;  // Zobrist stream
    const float *rlut;     // [4][4096]
    const int8_t *pool;    // [pool_size][120]
};

// Block barrier that orders LDS only. __syncthreads() is a workgroup fence over
// all address spaces, which also waits for every outstanding global store of
// the wave; a kernel that streams stores across LDS phases must not pay that.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Barrier of one wave working alone on its env (the whole block of a 64-thread
// kernel, or one wave of a larger block): orders the wave's LDS and global
// accesses like __syncthreads() without an s_barrier, so the other waves of a
// larger block neither wait for it nor count it.
__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Streaming stores, for outputs that nothing in the same launch reads back.
// Every launch ends by writing back the dirty lines of the XCDs' L2 caches, and
// the next launch on the stream starts only after that: for a kernel that
// streams gigabytes through L2 this writeback took ≈6 µs. With the
// non-temporal hint the lines go out to memory as they are written and leave
// little dirty data behind.
template <typename T>
__device__ __forceinline__ void stream_store(T *p, T v)
{
    __builtin_nontemporal_store(v, p);
}

__device__ __forceinline__ void stream_store(uint4 *p, uint4 v)
{
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 x = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(x, reinterpret_cast<u32x4 *>(p));
}

__device__ __forceinline__ size_t cm_idx(int env, int o, int pid) { return ((size_t)env * 4 + o) * PID_STRIDE + pid; }
__device__ __forceinline__ size_t pc_idx(int env, int pid) { return (size_t)env * PID_STRIDE + pid; }

}  // namespace jq

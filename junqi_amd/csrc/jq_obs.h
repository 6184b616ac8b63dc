// Observation encoder (included into jq_lib.hip's translation unit, which owns
// the constant tables).
//
// Layout and values follow junqi_core/observation.py:155-232 (317 planes in the
// observer's canonical frame, 28 globals) and its writers at :908-1651.
//
// Every element of a row has a u8 value code (cDECODE maps codes to floats).
// Only ~1-2k of the 91,613 elements are nonzero, so a row is built sparsely in
// LDS and then streamed densely:
//   * `bits`: one bit per element, bit 0 of its code (all 0/1 planes), set by
//     LDS atomic-OR scatter from the threads that own a piece or a constant
//     plane; the row-independent board_static words are copied from a template;
//   * `img`: a byte image of the four plane ranges whose codes exceed 1
//     (teammate / enemy beliefs, move history, kill_mine_count), placed so that
//     the 16-byte output chunk at a given address reads an aligned LDS word;
//     zero outside the ranges and in 16-byte margins around them.
// The emit loop gives each lane one aligned 16-byte chunk of the row per
// iteration (a wave covers 1 KB of HBM), expands the chunk's bits to bytes
// (u8), bf16 or f32, merges the image and issues one 16-byte store. Whether a
// wave's 1 KB span touches an image range is decided once per wave.
// The six continuous planes (turn history, recency) are exact floats, computed
// per element in f32 / bf16. The u8 format leaves them zero in the code planes
// and writes one 2,320-byte aux row per observation instead: the two turn
// history values as float32 (each is constant over its plane), then the four
// recency planes as uint16 codes per cell, 0 for 0.0 and 1 + e for the value
// exp(-e / tau) at elapsed step e (entry e of the recency table).
//
// The u8 kernel is persistent (grid = resident blocks): while a block streams
// row i out, its threads already hold the gathered inputs of row i + gridDim.x
// in registers, so the next fill only waits for the recency-table lookups.
// f32 / bf16 rows are 2-4x wider; they run one 256-thread block per row.
#pragma once

namespace jq {

constexpr int OBS_C = 317;
constexpr int OBS_ROW = OBS_C * NC;   // 91,613 elements
constexpr int OBS_THREADS = 256;
constexpr int OBS_BITS_WORDS = 2868;  // >= ceil(91613 / 32) + 1, multiple of 4

// Byte-image ranges [start, end) in elements; each gets 16 zero bytes on either
// side plus 16 bytes of alignment slack.
constexpr int RG0_S = 12 * NC, RG0_E = 24 * NC;    // prob_teammate
constexpr int RG1_S = 27 * NC, RG1_E = 51 * NC;    // belief left / right
constexpr int RG2_S = 129 * NC, RG2_E = 161 * NC;  // move history (+1 dst, -1 src)
constexpr int RG3_S = 211 * NC, RG3_E = 223 * NC;  // kill_mine_count
constexpr int rg_bytes(int s, int e) { return ((e - s) + 48 + 15) & ~15; }
constexpr int RG0_B = 0;
constexpr int RG1_B = RG0_B + rg_bytes(RG0_S, RG0_E);
constexpr int RG2_B = RG1_B + rg_bytes(RG1_S, RG1_E);
constexpr int RG3_B = RG2_B + rg_bytes(RG2_S, RG2_E);
constexpr int IMG_BYTES = RG3_B + rg_bytes(RG3_S, RG3_E);
constexpr int IMG_ZERO = RG0_B;   // 16 bytes that are always zero (range 0's leading margin)
static_assert(IMG_BYTES % 16 == 0, "image must be a whole number of 16-byte words");

// board_static planes 58-63 occupy words 523..577 of `bits`; the template keeps
// 16-byte-aligned words 520..579
constexpr int STAT_Q0 = 130, STAT_NQ = 15;

// continuous planes: 64-65 turn history, 253-256 recency
constexpr int CT0_S = 64 * NC, CT0_E = 66 * NC, CT1_S = 253 * NC, CT1_E = 257 * NC;
// u8 aux row: float32 turn history [2], then uint16 recency codes [4][289]
constexpr int AUXC_ROW = 8 + 4 * NC * 2;   // 2,320 bytes
static_assert(AUXC_ROW % 16 == 0, "aux rows must keep 16-byte alignment");

// u8 codes of the fixed values (the decode table starts 0, 1, -1, 1/3, 2/3)
constexpr uint8_t CODE_ONE = 1, CODE_NEG = 2, CODE_THIRD = 3, CODE_2THIRD = 4;

// thread roles in the build: 0..119 one pid each, 128..159 one move-history
// slot each, 160..166 the whole-plane seat flags
constexpr int T_HIST = PID_STRIDE, T_FLAGS = T_HIST + HIST_LEN, T_END = T_FLAGS + 7;

struct ObsLds {
    alignas(16) uint32_t bits[OBS_BITS_WORDS];
    alignas(16) uint8_t img[IMG_BYTES];
    alignas(16) uint32_t stat[STAT_NQ * 4];   // board_static words of `bits` (row-independent)
    union {
        float rec[PID_STRIDE][4];      // recency values per pid (0 unless an enemy piece on board): f32 / bf16
        uint16_t rcode[PID_STRIDE][4]; // the same as aux codes (0 none, 1 + elapsed): u8
    };
    float dec[32];                   // code -> f32
    uint32_t decb[32];               // code -> bf16 bits
    int8_t cpid[CELL_STRIDE];        // canonical cell -> pid (-1 empty)
    alignas(4) uint8_t bval[BC_COUNT * 12 + 4]; // belief row code x type -> value code
    float turnv[2];
};

// Uploaded beliefs (f32 / bf16 only): the 12 values of each teammate / enemy
// piece, read at its world cell from the observer's (12, 289) slice, and the
// piece's relation (1 teammate, 2 left, 3 right, 0 none).
struct ExtLds {
    float bel[PID_STRIDE][12];
    uint8_t rel[PID_STRIDE];
};

// Byte-image address of element e of the range starting at `start` (image base
// `base`) for a row whose first element sits at element phase m (row address /
// element size, mod 16 / element size).
__device__ __forceinline__ int img_off(int base, int start, int e, int m)
{
    return base + 16 + ((start + m) & 15) + (e - start);
}

// Image range containing element e, as (base, start); false if none.
__device__ __forceinline__ bool img_range(int e, int &base, int &start)
{
    if (e >= RG0_S && e < RG0_E) { base = RG0_B; start = RG0_S; return true; }
    if (e >= RG1_S && e < RG1_E) { base = RG1_B; start = RG1_S; return true; }
    if (e >= RG2_S && e < RG2_E) { base = RG2_B; start = RG2_S; return true; }
    if (e >= RG3_S && e < RG3_E) { base = RG3_B; start = RG3_S; return true; }
    return false;
}

__device__ __forceinline__ bool back_two(int seat, int zero)
{   // observation.py:1376-1383 (zero cell in the owner's two back rows)
    if (zero < 0) return false;
    const int zx = zero % 17, zy = zero / 17;
    switch (seat) {
    case 0: return zy >= 15;
    case 2: return zy <= 1;
    case 1: return zx <= 1;
    default: return zx >= 15;
    }
}

__device__ __forceinline__ void set_el(ObsLds &L, int e) { atomicOr(&L.bits[e >> 5], 1u << (e & 31)); }

__device__ __forceinline__ void set_code(ObsLds &L, int base, int start, int e, int m, uint8_t v)
{
    L.img[img_off(base, start, e, m)] = v;
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f)
{
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Bits [base, base + 30) of the 120-bit pid set (hi:lo), i.e. the 30 pids of one seat.
__device__ __forceinline__ uint32_t seat_bits(uint64_t lo, uint64_t hi, int base)
{
    const uint64_t w = base == 0 ? lo : base < 64 ? ((lo >> base) | (hi << (64 - base))) : (hi >> (base - 64));
    return (uint32_t)w & 0x3FFFFFFFu;
}

// World flat cell -> canonical flat cell of observer s (rotation.py:44-85).
__device__ __forceinline__ int canon_cell(int s, int f)
{
    const int x = f % 17, y = f / 17;
    const int cx = s == 0 ? x : s == 1 ? y : s == 2 ? 16 - x : 16 - y;
    const int cy = s == 0 ? y : s == 1 ? 16 - x : s == 2 ? 16 - y : x;
    return cy * 17 + cx;
}

// Everything one pid contributes, loaded in one batch of independent reads
// before the block's first barrier (observation.py:908-1620 per-piece writers).
struct PieceIn {
    int pos, tp, mcount, aeat, psurv, dstep, dreason, dloc, zero, bcode;
    uint32_t kmask, types, cnts;   // observer's combat memory of an enemy piece (CmView)
    int ldir, lchain, fstep;
    uint64_t elo, ehi;             // eaten_by of the observer's own pieces
    int lsum, rsum;                // left / right enemies' memory of an own piece (cm_summary)
};

__device__ __forceinline__ void piece_load(const State &S, int env, int obs, int pid, PieceIn &P)
{
    const int le = (obs + 1) & 3, re = (obs + 3) & 3, s = pid / 30;
    const PieceRec r = S.piece[pc_idx(env, pid)];
    P.pos = r.pos; P.tp = r.ptype;
    P.mcount = r.mcount; P.aeat = r.aeat; P.psurv = r.psurv;
    P.dstep = r.dstep; P.dreason = r.dreason; P.dloc = r.dloc; P.zero = r.zero;
    P.bcode = S.bcode[((size_t)env * 4 + obs) * PID_STRIDE + pid];
    P.elo = P.ehi = 0;
    P.kmask = P.types = P.cnts = 0;
    P.ldir = P.lchain = P.fstep = -1;
    P.lsum = P.rsum = 0;
    if ((s & 1) != (obs & 1)) {
        const CmView v = S.cmv[cm_idx(env, obs, pid)];
        P.kmask = v.kmask; P.types = v.types; P.cnts = v.cnts;
        P.ldir = v.ldir; P.lchain = v.lchain; P.fstep = v.fstep;
    } else if (s == obs) {
        const CmEat e = S.cme[cm_idx(env, obs, pid)];
        P.elo = e.elo; P.ehi = e.ehi;
        P.lsum = S.cmk[cm_idx(env, le, pid)];
        P.rsum = S.cmk[cm_idx(env, re, pid)];
    }
}

// Scatter one pid's nonzero elements into bits / img.
template <bool EXT = false, bool AUXC = false>
__device__ __forceinline__ void piece_scatter(int show_mode, int obs, int pid, int m, const PieceIn &P,
                                              const float rc[4], const uint16_t rk[4], const uint32_t otb[4],
                                              ObsLds &L, const float *ext = nullptr, ExtLds *X = nullptr)
{
    const int tm = (obs + 2) & 3, le = (obs + 1) & 3, team = obs & 1;
    const int s = pid / 30;
    const int rel = s == obs ? 0 : s == tm ? 1 : s == le ? 2 : 3;
    const bool ours = (s & 1) == team;

    if ((unsigned)P.pos < (unsigned)NC) {
        const int k = canon_cell(obs, P.pos);
        L.cpid[k] = (int8_t)pid;
        // piece_own (0-11), side occupancy (25, 26), dark_teammate (24)
        if (rel == 0 && P.tp >= 2 && P.tp <= 13) set_el(L, (P.tp - 2) * NC + k);
        if (rel == 2) set_el(L, 25 * NC + k);
        if (rel == 3) set_el(L, 26 * NC + k);
        if (rel == 1 && show_mode == SM_DARK) set_el(L, 24 * NC + k);
        // beliefs (12-23 teammate, 27-38 left, 39-50 right)
        if (EXT && rel != 0) {   // uploaded: kept as floats, emitted per element
            for (int j = 0; j < 12; ++j) {
                const float v = ext[j * NC + P.pos];
                X->bel[pid][j] = v > 0.f ? v : 0.f;
            }
            X->rel[pid] = (uint8_t)rel;
        } else if (rel != 0) {
            const int bc = P.bcode < BC_COUNT ? P.bcode : 0;
            const int c0 = rel == 1 ? 12 : rel == 2 ? 27 : 39;
            const int base = rel == 1 ? RG0_B : RG1_B, start = rel == 1 ? RG0_S : RG1_S;
            const uint32_t *bw = reinterpret_cast<const uint32_t *>(&L.bval[bc * 12]);   // the 12 codes
            const uint32_t b3[3] = {bw[0], bw[1], bw[2]};
#pragma unroll
            for (int j = 0; j < 12; ++j) {
                const uint8_t v = (uint8_t)(b3[j >> 2] >> (8 * (j & 3)));
                if (v) set_code(L, base, start, (c0 + j) * NC + k, m, v);
            }
        }
        // move / active_eat / passive_survive buckets (66-89): own team in the
        // first four planes of each group, the other team in the last four
        const int half = ours ? 0 : 4;
        const int mb = min(P.mcount, 3), eb = min(P.aeat, 3), sb = min(P.psurv, 3);
        set_el(L, (66 + half + mb) * NC + k);
        for (int q = 0; q <= eb; ++q) set_el(L, (74 + half + q) * NC + k);
        for (int q = 0; q <= sb; ++q) set_el(L, (82 + half + q) * NC + k);
        // piece_slot (104-128); a camp slot lands on the last plane, like numpy's -1
        const int sc = cT.slotch[pid % 30];
        set_el(L, (104 + (sc < 0 ? 24 : sc)) * NC + k);

        uint64_t cmb = 0;
        if (!ours) {   // combat-memory layers 1 and 3 (observation.py:1292-1387, 1475-1567)
            const int mcnt = P.cnts & 3, ccnt = (P.cnts >> 2) & 3, ocnt = (P.cnts >> 4) & 3;   // capped at 3
            const int floor = (P.types >> 24) & 15, flags = P.types >> 28;
            cmb |= (uint64_t)(P.types & 0xFFF);
            for (int q = 0; q < 3; ++q) {
                if (mcnt >= q + 1) cmb |= 1ull << (12 + q);
                if (ocnt >= q + 1) cmb |= 1ull << (15 + q);
                if (ccnt >= q + 1) cmb |= 1ull << (30 + q);
            }
            cmb |= (uint64_t)((P.types >> 12) & 0xFFF) << 18;
            for (int q = 0; q < 9; ++q) if (floor >= q + 1) cmb |= 1ull << (33 + q);
            if (flags & CMF_IS_GONGB) cmb |= 1ull << 42;
            if (flags & CMF_NOT_GONGB) cmb |= 1ull << 43;
            if (back_two(s, P.zero) && P.mcount == 0 && !(flags & CMF_ATK_GONGB)) cmb |= 1ull << 44;
            // kill_mine_slot (223-252) and kill_mine_count (211-222) over the
            // observer's own pieces this one has killed directly
            uint64_t tcnt = 0;   // 12 counters of 5 bits, one per tracked type
            for (uint32_t hits = P.kmask; hits; hits &= hits - 1) {
                const int sl = __builtin_ctz(hits);
                set_el(L, (223 + sl) * NC + k);
                const int gt = (int)(((otb[0] >> sl) & 1u) | (((otb[1] >> sl) & 1u) << 1) | (((otb[2] >> sl) & 1u) << 2) |
                                     (((otb[3] >> sl) & 1u) << 3));   // the killed piece's type
                if (gt >= 2 && gt <= 13) tcnt += 1ull << (5 * (gt - 2));
            }
#pragma unroll
            for (int q = 0; q < 12; ++q) {
                const int c = (int)((tcnt >> (5 * q)) & 31u);
                if (c) set_code(L, RG3_B, RG3_S, (211 + q) * NC + k, m,
                                c == 1 ? CODE_THIRD : c == 2 ? CODE_2THIRD : CODE_ONE);
            }
        } else if (s == obs) {   // layer 2 (observation.py:1392-1451); counts capped at 3
            const int lc = P.lsum & 3, rcnt = P.rsum & 3;
            const int lflags = P.lsum >> 2, rflags = P.rsum >> 2;
            const int pk = lc < rcnt ? lc : rcnt;
            for (int q = 0; q < 3; ++q) if (pk >= q + 1) cmb |= 1ull << (45 + q);
            if ((lflags & CMF_IS_GONGB) && (rflags & CMF_IS_GONGB)) cmb |= 1ull << 48;
            const bool atk = (lflags & CMF_ATK_GONGB) || (rflags & CMF_ATK_GONGB);
            if (back_two(s, P.zero) && P.mcount == 0 && !atk) cmb |= 1ull << 49;
        }
        while (cmb) {   // combat-memory bit planes 161-210
            const int b = __builtin_ctzll(cmb);
            cmb &= cmb - 1;
            set_el(L, (161 + b) * NC + k);
        }
    }
    for (int q = 0; q < 4; ++q) {
        if (AUXC) L.rcode[pid][q] = rk[q];
        else L.rec[pid][q] = rc[q];
    }

    // death_reason (90-101) and dead_at_zero (102-103), observation.py:1103-1180
    if (P.dstep >= 0) {
        const int grp = rel == 0 ? 0 : rel == 1 ? 3 : rel == 2 ? 6 : 9;
        if (P.dreason >= 0 && P.dreason <= 2 && P.dstep > 0 && (unsigned)P.dloc < (unsigned)NC)
            set_el(L, (90 + grp + P.dreason) * NC + canon_cell(obs, P.dloc));
        if ((unsigned)P.zero < (unsigned)NC) set_el(L, (102 + (ours ? 0 : 1)) * NC + canon_cell(obs, P.zero));
    }
    // eaten_by_pid (257-316), layer 4 (observation.py:1591-1620): the observer's
    // own piece, at its cell or (dead) its zero cell, marks its killers
    if (rel == 0) {
        const int cell = P.pos >= 0 ? P.pos : P.zero;
        if ((unsigned)cell < (unsigned)NC) {
            const int k = canon_cell(obs, cell);
            const int re = (obs + 3) & 3;
            uint64_t hits = (uint64_t)seat_bits(P.elo, P.ehi, le * 30) | ((uint64_t)seat_bits(P.elo, P.ehi, re * 30) << 30);
            for (; hits; hits &= hits - 1) set_el(L, (257 + __builtin_ctzll(hits)) * NC + k);
        }
    }
}


__device__ __forceinline__ int row_env(int row, int all_seats) { return all_seats ? row >> 2 : row; }

// Observer of a row: all_seats rows take observer[env * 4 + k] (k-th slot of the
// env's (N,4) observer map, default seat k); single rows take observer[env] or
// the env's acting seat.
__device__ __forceinline__ int row_obs(const State &S, const int8_t *observer, int all_seats, int row)
{
    if (all_seats) return (observer ? observer[row] : row) & 3;
    return (observer ? observer[row] : S.env[row].turn) & 3;
}

// Seat of the observer's i-th relation in plane order: self, teammate, left, right.
__device__ __forceinline__ int seat_rel(int obs, int i) { return (obs + (i == 0 ? 0 : i == 1 ? 2 : i == 2 ? 1 : 3)) & 3; }

__device__ __forceinline__ float recency_at(const State &S, int mc, int last, int q)
{   // exp(-elapsed / tau) from the table (observation.py:1545-1567)
    if (last < 0) return 0.f;
    int el = mc - last;
    el = el < 0 ? 0 : (el > 4095 ? 4095 : el);
    return S.rlut[q * 4096 + el];
}

__device__ __forceinline__ uint16_t recency_code(int mc, int last)
{   // aux code of recency_at: 0 for no value, else 1 + the clamped elapsed step
    if (last < 0) return 0;
    int el = mc - last;
    el = el < 0 ? 0 : (el > 4095 ? 4095 : el);
    return (uint16_t)(1 + el);
}

// Row-independent LDS content (tables, board_static template) of one buffer.
// All `nthreads` threads of the block call it; it ends with a barrier.
__device__ __forceinline__ void obs_setup(ObsLds &L, int t, int nthreads)
{
    for (int i = t; i < BC_COUNT * 12; i += nthreads) L.bval[i] = cBVAL[i / 12][i % 12];
    if (t < 32) {
        const float d = t < 17 ? cDECODE[t] : 0.f;
        L.dec[t] = d;
        L.decb[t] = f32_to_bf16_rne(d);
    }
    if (t < STAT_NQ * 4) L.stat[t] = 0;
    lds_barrier();
    for (int k = t; k < NC; k += nthreads) {   // board_static (58-63): fixed cell classes
        uint32_t sm = cT.statics[k];
        while (sm) {
            const int b = __builtin_ctz(sm);
            sm &= sm - 1;
            if (b < 6) {
                const int e = (58 + b) * NC + k;
                atomicOr(&L.stat[(e >> 5) - STAT_Q0 * 4], 1u << (e & 31));
            }
        }
    }
    lds_barrier();
}

// Empty row: zero bits except the board_static template, zero image, no pieces.
// Thread t of `nthreads`.
__device__ __forceinline__ void obs_clear(ObsLds &L, int t, int nthreads)
{
    uint4 *w = reinterpret_cast<uint4 *>(L.bits);
    const uint4 *st = reinterpret_cast<const uint4 *>(L.stat);
    for (int i = t; i < OBS_BITS_WORDS / 4; i += nthreads)
        w[i] = (unsigned)(i - STAT_Q0) < (unsigned)STAT_NQ ? st[i - STAT_Q0] : make_uint4(0, 0, 0, 0);
    uint4 *b = reinterpret_cast<uint4 *>(L.img);
    for (int i = t; i < IMG_BYTES / 16; i += nthreads) b[i] = make_uint4(0, 0, 0, 0);
    for (int k = t; k < CELL_STRIDE; k += nthreads) L.cpid[k] = -1;
}

// Producer thread -> pid, grouped by relation so each wave runs one code path:
// wave 0 = own (t 0-29) and teammate (30-59) pieces, wave 1 = left (64-93) and
// right (94-123) enemies. -1 for the threads in between.
__device__ __forceinline__ int piece_of_thread(int t, int obs)
{
    if (t < 30) return obs * 30 + t;
    if (t < 60) return ((obs + 2) & 3) * 30 + (t - 30);
    if (t >= 64 && t < 94) return ((obs + 1) & 3) * 30 + (t - 64);
    if (t >= 94 && t < 124) return ((obs + 3) & 3) * 30 + (t - 94);
    return -1;
}

// One producer thread's inputs of a row (thread roles below), everything that
// depends only on (env, observer): gathered in one round of independent vector
// loads. Nothing here is a scalar load: a kernel that prefetches the next row
// while it works on LDS would otherwise wait for the prefetch at its next LDS
// fence (scalar loads and LDS operations share one wait counter).
struct RowIn {
    PieceIn P;              // t < NP
    int own_tp;             // lane l < 30 of every wave: type of the observer's piece l (& 15)
    uint32_t ew;            // lane l < 8 of every wave: word l of the env record
    int hist;               // T_HIST <= t < T_FLAGS: ring slot t - T_HIST as stored
    int rem;                // t < 24: remaining count behind global feature t
};

// Thread roles: 0..127 one pid each (piece_of_thread) or, for the 8 spare
// threads, one padding recency slot; 128..159 one move-history ring slot each,
// 160..166 the whole-plane seat flags; 0..27 also write the 28 globals.
__device__ __forceinline__ void row_fetch(const State &S, int env, int obs, int t, RowIn &R)
{
    const int l = t & 63;
    R.ew = l < 8 ? reinterpret_cast<const uint32_t *>(&S.env[env])[l] : 0u;
    R.own_tp = l < 30 ? (S.piece[pc_idx(env, obs * 30 + l)].ptype & 15) : 0;
    R.hist = 0;
    R.rem = 0;
    const int pid = t < PID_STRIDE ? piece_of_thread(t, obs) : -1;
    if (pid >= 0) piece_load(S, env, obs, pid, R.P);
    else if (t >= T_HIST && t < T_FLAGS) R.hist = S.hist[(size_t)env * HIST_LEN + (t - T_HIST)];
    if (t < 24) {
        const int seat = t < 12 ? (obs + 1) & 3 : (obs + 3) & 3;
        R.rem = S.rem[((size_t)env * 4 + obs) * 48 + seat * 12 + t % 12];
    }
}

// The observer of `row` (row_obs) as a per-lane vector load: lane 0 holds it,
// the other lanes read a neighbouring entry so the address is not uniform.
// Taken with __builtin_amdgcn_readfirstlane where it is used.
__device__ __forceinline__ int row_obs_prefetch(const State &S, const int8_t *observer, int all_seats, int row,
                                                int nrows)
{
    const int r = min(row + (int)(threadIdx.x & 1), nrows - 1);
    if (all_seats) return observer ? observer[r] : r;
    return observer ? observer[r] : S.env[r].turn;
}

// Fill a cleared buffer with row (env, obs) from the fetched inputs, thread t
// in [0, 256). Only the recency-table gathers are loads here. No thread reads
// what another one writes, so no barrier is needed inside.
// AUXC (the u8 format): recency as aux codes, no table lookups.
template <bool EXT = false, bool AUXC = false>
__device__ __forceinline__ void row_fill(const State &S, int obs, int m, int t, const RowIn &R, ObsLds &L,
                                         float *glob_row, const float *ext = nullptr, ExtLds *X = nullptr)
{
    // env-record fields and the observer's piece types, from the fetched lanes
    const int mc = __builtin_amdgcn_readlane((int)R.ew, 2), mslc = __builtin_amdgcn_readlane((int)R.ew, 3);
    const int hmeta = __builtin_amdgcn_readlane((int)R.ew, 4);
    const uint32_t w6 = (uint32_t)__builtin_amdgcn_readlane((int)R.ew, 6);
    const uint32_t w7 = (uint32_t)__builtin_amdgcn_readlane((int)R.ew, 7);
    const int sdead = w6 & 0xFF, sflag = (w6 >> 8) & 0xFF;
    const int remtrk = (obs < 2 ? w6 >> (16 + 8 * obs) : w7 >> (8 * (obs - 2))) & 0xFF;
    uint32_t otb[4];   // bit planes of the observer's 30 piece types
    for (int b = 0; b < 4; ++b) otb[b] = (uint32_t)__builtin_amdgcn_ballot_w64(((R.own_tp >> b) & 1) != 0);
    const int pid = t < PID_STRIDE ? piece_of_thread(t, obs) : -1;
    if (pid >= 0) {
        float rc[4] = {0.f, 0.f, 0.f, 0.f};
        uint16_t rk[4] = {0, 0, 0, 0};
        if ((unsigned)R.P.pos < (unsigned)NC && t >= 64) {   // enemy pieces on the board
            const int last[4] = {R.P.ldir, R.P.ldir, R.P.lchain, R.P.fstep};
            for (int q = 0; q < 4; ++q) {
                if (AUXC) rk[q] = recency_code(mc, last[q]);
                else rc[q] = recency_at(S, mc, last[q], q);
            }
        }
        piece_scatter<EXT, AUXC>(S.show_mode, obs, pid, m, R.P, rc, rk, otb, L, ext, X);
    } else if (t < PID_STRIDE) {   // the 8 spare threads clear the padding pids' recency
        const int pad = NP + (t < 64 ? t - 60 : t - 120);
        for (int q = 0; q < 4; ++q) {
            if (AUXC) L.rcode[pad][q] = 0;
            else L.rec[pad][q] = 0.f;
        }
    } else if (t < T_FLAGS) {   // move_history (129-160), observation.py:1207-1231
        const int cnt = hmeta & 0xFF, head = (hmeta >> 8) & 31;
        const int d = (head - 1 - (t - T_HIST)) & 31;   // plane of this ring slot (0 = most recent)
        if (d < cnt) {
            const int e = R.hist;
            const int hs = canon_cell(obs, min(e & 0xFFFF, NC - 1));
            const int hd = canon_cell(obs, min((e >> 16) & 0xFFFF, NC - 1));
            if (hs != hd) set_code(L, RG2_B, RG2_S, (129 + d) * NC + hs, m, CODE_NEG);
            set_code(L, RG2_B, RG2_S, (129 + d) * NC + hd, m, CODE_ONE);
        }
    } else if (t < T_END) {   // whole planes: dead_flags 51-53, flag_revealed 54-57
        const int j = t - T_FLAGS;
        const bool on = j < 3 ? ((sdead >> seat_rel(obs, j + 1)) & 1) : ((sflag >> seat_rel(obs, j - 3)) & 1);
        if (on) {
            const int e0 = (51 + j) * NC, e1 = e0 + NC;
            for (int w = e0 >> 5; w <= (e1 - 1) >> 5; ++w) {
                const int lo = max(e0, w * 32) - w * 32, hi = min(e1, w * 32 + 32) - w * 32;
                const uint32_t mask = (hi - lo == 32) ? 0xFFFFFFFFu : (((1u << (hi - lo)) - 1u) << lo);
                atomicOr(&L.bits[w], mask);
            }
        }
    }
    if (t == 0) {   // turn_history: float64 divide, then rounded to float32 (observation.py:1000-1021)
        double dp = (double)mslc / 200.0; if (dp > 1.0) dp = 1.0;
        double mp = (double)mc / 4000.0; if (mp > 1.0) mp = 1.0;
        L.turnv[0] = (float)dp; L.turnv[1] = (float)mp;
    }
    if (glob_row && t < 28) {   // globals (observation.py:1623-1651)
        float v;
        if (t < 24) {   // remaining counts of the left / right enemy
            const int seat = t < 12 ? (obs + 1) & 3 : (obs + 3) & 3;
            v = ((remtrk >> seat) & 1) ? (float)R.rem : 0.f;
        } else {   // flag_revealed of self, teammate, left, right
            v = (float)((sflag >> seat_rel(obs, t - 24)) & 1);
        }
        glob_row[t] = v;
    }
}

// Code of element e (0 <= e < OBS_ROW).
__device__ __forceinline__ uint32_t obs_code_at(const ObsLds &L, int e, int m)
{
    uint32_t c = (L.bits[e >> 5] >> (e & 31)) & 1u;
    int base, start;
    if (img_range(e, base, start)) c |= L.img[img_off(base, start, e, m)];
    return c;
}

// Exact float of a continuous element (plane c in 64, 65, 253..256; cell k).
__device__ __forceinline__ float obs_cont_at(const ObsLds &L, int c, int k)
{
    if (c < 66) return L.turnv[c - 64];
    const int pid = L.cpid[k];
    return pid >= 0 ? L.rec[pid][c - 253] : 0.f;
}

// Belief planes written per element when beliefs are uploaded: 12-23, 27-50.
constexpr int EB0_S = 12 * NC, EB0_E = 24 * NC, EB1_S = 27 * NC, EB1_E = 51 * NC;

// Uploaded belief of plane c (12..23 teammate, 27..38 left, 39..50 right) at cell k.
__device__ __forceinline__ float ext_belief_at(const ObsLds &L, const ExtLds *X, int c, int k)
{
    const int pid = L.cpid[k];
    if (pid < 0) return 0.f;
    const int want = c < 24 ? 1 : c < 39 ? 2 : 3;
    const int j = c < 24 ? c - 12 : c < 39 ? c - 27 : c - 39;
    return X->rel[pid] == want ? X->bel[pid][j] : 0.f;
}

// Value bits of element e in format FMT (0 f32, 1 bf16, 2 u8 code).
template <int FMT, bool EXT = false>
__device__ __forceinline__ uint32_t obs_elem(const ObsLds &L, int e, int m, const ExtLds *X = nullptr)
{
    if (EXT && ((e >= EB0_S && e < EB0_E) || (e >= EB1_S && e < EB1_E))) {
        const int c = e / NC;
        const float v = ext_belief_at(L, X, c, e - c * NC);
        return FMT == 0 ? __float_as_uint(v) : (uint32_t)f32_to_bf16_rne(v);
    }
    if (FMT != 2 && ((e >= CT0_S && e < CT0_E) || (e >= CT1_S && e < CT1_E))) {
        const int c = e / NC;
        const float v = obs_cont_at(L, c, e - c * NC);
        return FMT == 0 ? __float_as_uint(v) : (uint32_t)f32_to_bf16_rne(v);
    }
    const uint32_t code = obs_code_at(L, e, m);
    if (FMT == 2) return code;
    return FMT == 0 ? __float_as_uint(L.dec[code]) : L.decb[code];
}

__device__ __forceinline__ uint32_t bit_window(const ObsLds &L, int e)
{   // bits e .. e+31 of the stream (e >= 0, e + 16 <= OBS_ROW)
    return __builtin_amdgcn_alignbit(L.bits[(e >> 5) + 1], L.bits[e >> 5], e & 31);
}

// One full 16-byte chunk whose first element is e0. `off` is the image offset
// of e0 (IMG_ZERO when the chunk touches no image range).
template <int FMT>
__device__ __forceinline__ uint4 obs_chunk(const ObsLds &L, int e0, int off, bool img)
{
    const uint32_t v = bit_window(L, e0);
    uint32_t w[4];
    if (FMT == 2) {
        for (int i = 0; i < 4; ++i) w[i] = nib_to_bytes(v >> (4 * i));
        if (img) {
            const uint4 b = *reinterpret_cast<const uint4 *>(&L.img[off]);
            w[0] |= b.x; w[1] |= b.y; w[2] |= b.z; w[3] |= b.w;
        }
    } else if (FMT == 1) {
        if (img) {
            const uint2 b = *reinterpret_cast<const uint2 *>(&L.img[off]);
            for (int i = 0; i < 4; ++i) {
                const uint32_t cw = i < 2 ? b.x : b.y;
                const int sh = (i & 1) * 16;
                const uint32_t c0 = ((cw >> sh) & 0xFFu) | ((v >> (2 * i)) & 1u);
                const uint32_t c1 = ((cw >> (sh + 8)) & 0xFFu) | ((v >> (2 * i + 1)) & 1u);
                w[i] = L.decb[c0] | (L.decb[c1] << 16);
            }
        } else {
            for (int i = 0; i < 4; ++i) {   // 2 bits -> two bf16 halves of 0 / 1.0
                const uint32_t t = (v >> (2 * i)) & 3u;
                w[i] = __umul24((t | (t << 15)) & 0x10001u, 0x3F80u);
            }
        }
    } else {
        if (img) {
            const uint32_t cw = *reinterpret_cast<const uint32_t *>(&L.img[off]);
            for (int i = 0; i < 4; ++i) w[i] = __float_as_uint(L.dec[((cw >> (8 * i)) & 0xFFu) | ((v >> i) & 1u)]);
        } else {
            for (int i = 0; i < 4; ++i) w[i] = ((v >> i) & 1u) ? 0x3F800000u : 0u;
        }
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// Elements [e, f) of the row written one by one (row ends, continuous planes).
template <int FMT, bool EXT = false>
__device__ __forceinline__ void obs_elems(const ObsLds &L, uint8_t *row, int e, int f, int m,
                                          const ExtLds *X = nullptr)
{
    for (; e < f; ++e) {
        const uint32_t v = obs_elem<FMT, EXT>(L, e, m, X);
        if (FMT == 2) row[e] = (uint8_t)v;
        else if (FMT == 1) reinterpret_cast<uint16_t *>(row)[e] = (uint16_t)v;
        else reinterpret_cast<uint32_t *>(row)[e] = v;
    }
}

// A 16-byte chunk of a bf16 / f32 row. The bf16 rows go out as streaming
// stores (1.464 -> 1.365 ms per fused bf16 step at 32,768 games); f32 rows
// measured slower that way (2.68 -> 2.71 ms per drop-in step) and keep
// ordinary stores.
template <int FMT>
__device__ __forceinline__ void row_store(uint4 *p, uint4 v)
{
    if constexpr (FMT == 1) stream_store(p, v);
    else *p = v;
}

// Stream the 91,613-element row to `row` (element phase m) in 16-byte chunks:
// chunk q covers row bytes [16q - lead, 16q - lead + 16). A wave iteration
// stores one whole 1 KB-aligned unit of the buffer (the row's first and last
// units in part); each wave owns a contiguous run of units.
template <int FMT, bool EXT = false>
__device__ void obs_emit(const ObsLds &L, uint8_t *row, int m, const ExtLds *X = nullptr)
{
    constexpr int ES = FMT == 0 ? 4 : FMT == 1 ? 2 : 1;
    constexpr int EPC = 16 / ES;
    constexpr int NBYTES = OBS_ROW * ES;
    const int lead = m * ES;
    const int qf = lead ? 1 : 0, ql = (NBYTES + lead) >> 4;   // full chunks [qf, ql)
    const int d0 = RG0_B + 16 + ((RG0_S + m) & 15) - RG0_S, d1 = RG1_B + 16 + ((RG1_S + m) & 15) - RG1_S;
    const int d2 = RG2_B + 16 + ((RG2_S + m) & 15) - RG2_S, d3 = RG3_B + 16 + ((RG3_S + m) & 15) - RG3_S;
    const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    constexpr int NW = OBS_THREADS / 64;
    const uint64_t gbase = (uint64_t)(uintptr_t)(row - lead) >> 4;
    const uint64_t gA = gbase + qf, gB = gbase + ql;
    const uint64_t u0 = gA >> 6, u1 = (gB + 63) >> 6;
    const int nu = (int)(u1 - u0);
    const int per = (nu + NW - 1) / NW;
    const int ka = min(nu, wv * per), kb = min(nu, ka + per);
    const bool back = wv & 1;   // odd waves walk their run from its end, as in obs_emit_u8
    for (int i = ka; i < kb; ++i) {
        const int k = back ? ka + kb - 1 - i : i;
        const int qb = (int)((int64_t)((u0 + k) << 6) - (int64_t)gbase);
        const int s_lo = max(qb, qf) * EPC - m, s_hi = min(qb + 64, ql) * EPC - m;
        const int q = qb + lane;
        const bool ok = q >= qf && q < ql;
        const int e0 = q * EPC - m;
        uint8_t *dst = row + (ptrdiff_t)e0 * ES;
        if (FMT != 2 && ((s_lo < CT0_E && s_hi > CT0_S) || (s_lo < CT1_E && s_hi > CT1_S) ||
                         (EXT && ((s_lo < EB0_E && s_hi > EB0_S) || (s_lo < EB1_E && s_hi > EB1_S))))) {
            if (ok) {   // per-element values, one 16-byte store
                uint32_t w[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (FMT == 0) {
                        w[i] = obs_elem<FMT, EXT>(L, e0 + i, m, X);
                    } else {
                        w[i] = obs_elem<FMT, EXT>(L, e0 + 2 * i, m, X) |
                               (obs_elem<FMT, EXT>(L, e0 + 2 * i + 1, m, X) << 16);
                    }
                }
                row_store<FMT>(reinterpret_cast<uint4 *>(dst), make_uint4(w[0], w[1], w[2], w[3]));
            }
            continue;
        }
        int nov = 0, d = 0, rs = 0, re = 0;
        if (s_lo < RG0_E && s_hi > RG0_S) { ++nov; d = d0; rs = RG0_S; re = RG0_E; }
        if (s_lo < RG1_E && s_hi > RG1_S) { ++nov; d = d1; rs = RG1_S; re = RG1_E; }
        if (s_lo < RG2_E && s_hi > RG2_S) { ++nov; d = d2; rs = RG2_S; re = RG2_E; }
        if (s_lo < RG3_E && s_hi > RG3_S) { ++nov; d = d3; rs = RG3_S; re = RG3_E; }
        if (!ok) continue;
        uint4 out;
        if (nov == 0) {
            out = obs_chunk<FMT>(L, e0, IMG_ZERO, false);
        } else if (nov == 1 && s_lo >= rs - 16 && s_hi - EPC <= re) {
            out = obs_chunk<FMT>(L, e0, e0 + d, true);   // every chunk reads inside range's margins
        } else {
            int off = IMG_ZERO;
            if (e0 < RG0_E && e0 + EPC > RG0_S) off = e0 + d0;
            if (e0 < RG1_E && e0 + EPC > RG1_S) off = e0 + d1;
            if (e0 < RG2_E && e0 + EPC > RG2_S) off = e0 + d2;
            if (e0 < RG3_E && e0 + EPC > RG3_S) off = e0 + d3;
            out = obs_chunk<FMT>(L, e0, off, true);
        }
        row_store<FMT>(reinterpret_cast<uint4 *>(dst), out);
    }
    // partial chunks at the two ends of the row
    if (threadIdx.x == 0 && lead) obs_elems<FMT, EXT>(L, row, 0, EPC - m, m, X);
    if (threadIdx.x == 64 && ((NBYTES + lead) & 15)) obs_elems<FMT, EXT>(L, row, ql * EPC - m, OBS_ROW, m, X);
}

// Image offset of the u8 chunk starting at element e0: inside the range it
// overlaps (ranges are more than 16 elements apart, so at most one), else the
// always-zero word. Branch-free per lane.
__device__ __forceinline__ int u8_img_off(int e0, int d0, int d1, int d2, int d3)
{
    int off = IMG_ZERO;
    off = (e0 < RG0_E && e0 + 16 > RG0_S) ? e0 + d0 : off;
    off = (e0 < RG1_E && e0 + 16 > RG1_S) ? e0 + d1 : off;
    off = (e0 < RG2_E && e0 + 16 > RG2_S) ? e0 + d2 : off;
    off = (e0 < RG3_E && e0 + 16 > RG3_S) ? e0 + d3 : off;
    return off;
}

__device__ __forceinline__ uint4 u8_chunk(const ObsLds &L, int e0, int off)
{
    const uint32_t v = bit_window(L, e0);
    const uint4 b = *reinterpret_cast<const uint4 *>(&L.img[off]);
    return make_uint4(nib_to_bytes(v) | b.x, nib_to_bytes(v >> 4) | b.y, nib_to_bytes(v >> 8) | b.z,
                      nib_to_bytes(v >> 12) | b.w);
}

// Recency aux code j of a row (j = plane * 289 + canonical cell): the code of
// the piece on that cell, 0 on an empty cell.
__device__ __forceinline__ uint32_t rec_code_at(const ObsLds &L, int j)
{
    const int q = j / NC, k = j - q * NC;
    const int pid = L.cpid[k];
    return pid >= 0 ? L.rcode[pid][q] : 0u;
}

// The 2,320-byte aux row of a u8 observation (16-byte aligned): thread ct < 145
// writes bytes [16 ct, 16 ct + 16).
__device__ __forceinline__ void obs_emit_aux_codes(const ObsLds &L, uint8_t *row, int ct)
{
    if (ct >= AUXC_ROW / 16) return;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = ct * 16 + i * 4;
        if (b < 8) {
            w[i] = __float_as_uint(L.turnv[b >> 2]);
        } else {
            const int j = (b - 8) >> 1;
            w[i] = rec_code_at(L, j) | (rec_code_at(L, j + 1) << 16);
        }
    }
    *reinterpret_cast<uint4 *>(row + ct * 16) = make_uint4(w[0], w[1], w[2], w[3]);
}

// u8 row emission: the row's full 16-byte chunks, in 1 KB units of the output
// buffer split into contiguous runs, one per wave. The aux row follows, spread
// over the block.
__device__ __forceinline__ void obs_emit_u8(const ObsLds &L, uint8_t *row, int m, uint8_t *aux, int ct)
{
    const int lead = m;
    const int qf = lead ? 1 : 0, ql = (OBS_ROW + lead) >> 4;   // full chunks [qf, ql)
    const int d0 = RG0_B + 16 + ((RG0_S + m) & 15) - RG0_S, d1 = RG1_B + 16 + ((RG1_S + m) & 15) - RG1_S;
    const int d2 = RG2_B + 16 + ((RG2_S + m) & 15) - RG2_S, d3 = RG3_B + 16 + ((RG3_S + m) & 15) - RG3_S;
    const int wv = __builtin_amdgcn_readfirstlane(ct >> 6);
    const int lane = ct & 63;
    constexpr int NW = OBS_THREADS / 64;
    // chunk q covers row bytes [q*16 - m, q*16 - m + 16): a 16-byte aligned slot
    // of the output, indexed from the aligned address below the row start
    uint4 *__restrict__ slot = reinterpret_cast<uint4 *>(__builtin_assume_aligned(row - m, 16));
    // Each wave iteration stores one whole, 1 KB-aligned unit of the buffer (the
    // row's first and last units in part), and each wave owns a contiguous run
    // of units: a 128-byte line is never split between two store instructions.
    const uint64_t gbase = (uint64_t)(uintptr_t)(row - m) >> 4;   // buffer slot of chunk 0
    const uint64_t gA = gbase + qf, gB = gbase + ql;
    const uint64_t u0 = gA >> 6, u1 = (gB + 63) >> 6;
    const int nu = (int)(u1 - u0);
    const int per = (nu + NW - 1) / NW;
    const int ka = min(nu, wv * per), kb = min(nu, ka + per);
    // Odd waves walk their run from its end: the runs of waves 1 and 2 (and of
    // wave 3 and the next row's wave 0) start side by side and those of waves 0
    // and 1 (2 and 3) end side by side (0.7601 -> 0.7528 ms per fused step at
    // 32,768 games; every wave walking backward 0.7635).
    const bool back = wv & 1;
    for (int i = ka; i < kb; ++i) {
        const int k = back ? ka + kb - 1 - i : i;
        const uint64_t g = ((u0 + k) << 6) + lane;
        if (g >= gA && g < gB) {
            const int q = (int)(g - gbase);
            const int e0 = q * 16 - m;
            stream_store(&slot[q], u8_chunk(L, e0, u8_img_off(e0, d0, d1, d2, d3)));
        }
    }
    // partial chunks at the two ends of the row
    if (ct == 0 && lead) obs_elems<2>(L, row, 0, 16 - m, m);
    if (ct == 64 && ((OBS_ROW + lead) & 15)) obs_elems<2>(L, row, ql * 16 - m, OBS_ROW, m);
    if (aux) obs_emit_aux_codes(L, aux, ct);
}

// nrows = N (one row per env, observer given or the acting seat) or 4N
// (all_seats: row = env * 4 + observer). One 256-thread block per row. EXT
// (f32 / bf16): belief planes from ext, (N, 4, 12, 289) float32 world-cell
// beliefs per (env, observer).
template <int FMT, bool EXT = false>
__global__ __launch_bounds__(OBS_THREADS) void k_observe(State S, const int8_t *__restrict__ observer, int all_seats,
                                                         void *__restrict__ spatial, void *__restrict__ aux,
                                                         float *__restrict__ glob, int nrows,
                                                         const float *__restrict__ ext = nullptr)
{
    __shared__ ObsLds L;
    ExtLds *X = nullptr;
    if constexpr (EXT) {
        __shared__ ExtLds XL;
        X = &XL;
    }
    constexpr int ES = FMT == 0 ? 4 : FMT == 1 ? 2 : 1;
    const int t = threadIdx.x, row = blockIdx.x;
    if (row >= nrows) return;
    const int env = row_env(row, all_seats), obs = row_obs(S, observer, all_seats, row);
    uint8_t *rowp = reinterpret_cast<uint8_t *>(spatial) + (size_t)row * OBS_ROW * ES;
    const int m = (int)(((uintptr_t)rowp / ES) & (16 / ES - 1));
    // Wave issue priority 2 from the block's start through its fill, 0 while
    // streaming: a block that has just started gets its setup, loads and fill
    // issued ahead of the stores of the blocks already streaming on its SIMD,
    // and starts its own stream sooner (32,768 rows, ms per launch: bf16 1.240
    // -> 1.220 with the fill alone raised, 1.182 from the start; f32 2.229 ->
    // 2.210 either way)
    __builtin_amdgcn_s_setprio(2);
    obs_setup(L, t, OBS_THREADS);
    obs_clear(L, t, OBS_THREADS);
    if (EXT && t < PID_STRIDE) X->rel[t] = 0;
    lds_barrier();
    RowIn R;
    row_fetch(S, env, obs, t, R);
    row_fill<EXT, FMT == 2>(S, obs, m, t, R, L, glob ? glob + (size_t)row * 28 : nullptr,
                            EXT ? ext + ((size_t)env * 4 + obs) * 12 * NC : nullptr, X);
    __builtin_amdgcn_s_setprio(0);
    lds_barrier();
    // f32 rows: a short sleep between the fill and the stores (s_sleep 1, 2 or 4:
    // 2.271 -> 2.230-2.237 ms per launch at 32,768 rows, three alternations;
    // 8 / 16 / 32 2.239 / 2.249 / 2.259; bf16 and u8 rows gain nothing)
    if (FMT == 0) __builtin_amdgcn_s_sleep(2);
    if (FMT == 2) obs_emit_u8(L, rowp, m, aux ? static_cast<uint8_t *>(aux) + (size_t)row * AUXC_ROW : nullptr, t);
    else obs_emit<FMT, EXT>(L, rowp, m, X);
}

// u8, persistent single-buffer form: 256 threads, one LDS row. Per row: fill
// from the inputs fetched during the previous row, fetch the next row's inputs
// (in flight during the stores), stream the row, clear the buffer.
__global__ __launch_bounds__(OBS_THREADS) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_observe_u8_persist(
    State S, const int8_t *__restrict__ observer, int all_seats, uint8_t *__restrict__ spatial,
    uint8_t *__restrict__ aux, float *__restrict__ glob, int nrows)
{
    __shared__ ObsLds L;
    const int t = threadIdx.x, G = gridDim.x;
    if ((int)blockIdx.x >= nrows) return;   // uniform per block
    obs_setup(L, t, OBS_THREADS);
    obs_clear(L, t, OBS_THREADS);
    RowIn R;
    int ob = row_obs(S, observer, all_seats, blockIdx.x);
    row_fetch(S, row_env(blockIdx.x, all_seats), ob, t, R);
    int obp = row_obs_prefetch(S, observer, all_seats, blockIdx.x + G, nrows);   // observer of the next row
    lds_barrier();
    for (int row = blockIdx.x; row < nrows; row += G) {
        uint8_t *rowp = spatial + (size_t)row * OBS_ROW;
        const int m = (int)((uintptr_t)rowp & 15);
        // Wave issue priority by phase (s_setprio): 2 while streaming a row,
        // 1 while filling, 0 while fetching, idling and clearing. The SIMD's
        // arbiter then issues a streaming wave's stores ahead of the other
        // blocks' fill and fetch work on the same SIMD (ms per fused step at
        // 32,768 games, three alternations: none 0.7338; stream 1 / 2 / 3
        // 0.717-0.719; stream 2 and fill 1 0.7145; stream 3 without the idle
        // gap below 0.735; priority 2 throughout 0.735: only the difference
        // between phases counts).
        __builtin_amdgcn_s_setprio(1);
        row_fill<false, true>(S, ob, m, t, R, L, glob ? glob + (size_t)row * 28 : nullptr);
        __builtin_amdgcn_s_setprio(0);
        lds_barrier();
        if (row + G < nrows) {
            ob = __builtin_amdgcn_readfirstlane(obp) & 3;
            row_fetch(S, row_env(row + G, all_seats), ob, t, R);
            obp = row_obs_prefetch(S, observer, all_seats, row + 2 * G, nrows);
        }
        __builtin_amdgcn_s_setprio(2);
        obs_emit_u8(L, rowp, m, aux ? aux + (size_t)row * AUXC_ROW : nullptr, t);
        __builtin_amdgcn_s_setprio(0);
        // Each wave idles after issuing its part of the row, before the block
        // clears and refills its buffer: s_sleep 56 = 56 x 64 cycles, about
        // 1.5 us. A longer gap between one block's store phases means fewer
        // rows streaming at once across the GPU, and those reach memory faster
        // (32,768 games, ms per fused step: none 0.755, s_sleep 48 / 56 / 64 /
        // 72 0.734-0.737, 80 0.740, 96 0.749, 127 0.769).
        if (row + G < nrows) __builtin_amdgcn_s_sleep(56);
        lds_barrier();
        obs_clear(L, t, OBS_THREADS);
        lds_barrier();
    }
}

}  // namespace jq

// Observation encoder (included into jq_lib.hip's translation unit, which owns
// the constant tables). One 256-thread block per (env, observer) row.
//
// Layout and values follow junqi_core/observation.py:155-232 (317 planes in the
// observer's canonical frame, 28 globals) and its writers at :908-1651.
//
// Every element of a row has a u8 value code (cDECODE maps codes to floats).
// Only ~1-2k of the 91,613 elements are nonzero, so the block builds the row
// sparsely in LDS and then streams it densely:
//   * `bits`: one bit per element, bit 0 of its code (all 0/1 planes, move
//     history destinations, ...), set by LDS atomic-OR scatter from the threads
//     that own a piece, a history entry or a constant plane;
//   * `img`: a byte image of the four plane ranges whose codes exceed 1
//     (teammate / enemy beliefs, move history, kill_mine_count), placed so that
//     the 16-byte output chunk at a given address reads an aligned 16-byte LDS
//     word; zero outside the ranges.
// The emit loop gives each lane one aligned 16-byte chunk of the row per
// iteration (a wave covers 1 KB of HBM), expands the chunk's bits to bytes
// (u8), to bf16 or to f32, ORs in the image, and issues one 16-byte store.
// The six continuous planes (turn history, recency) are exact floats: they go
// to the aux output in the u8 format and are computed per element in f32 / bf16.
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
static_assert(IMG_BYTES % 16 == 0, "image must be a whole number of 16-byte words");

// continuous planes: 64-65 turn history, 253-256 recency
constexpr int CT0_S = 64 * NC, CT0_E = 66 * NC, CT1_S = 253 * NC, CT1_E = 257 * NC;
constexpr int AUX_ROW = 6 * NC;

// u8 codes of the fixed values (the decode table starts 0, 1, -1, 1/3, 2/3)
constexpr uint8_t CODE_ONE = 1, CODE_NEG = 2, CODE_THIRD = 3, CODE_2THIRD = 4;

struct ObsLds {
    alignas(16) uint32_t bits[OBS_BITS_WORDS];
    alignas(16) uint8_t img[IMG_BYTES];
    float rec[PID_STRIDE][4];        // recency values per pid (0 unless an enemy piece on board)
    float dec[32];                   // code -> f32
    uint32_t decb[32];               // code -> bf16 bits
    int8_t cpid[CELL_STRIDE];        // canonical cell -> pid (-1 empty)
    float turnv[2];
};

// Byte-image address of element e of range r for a row whose first element sits
// at element phase m (row address / element size, mod 16 / element size).
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

// Image range overlapping elements [e, e + len) (len <= 16); false if none.
__device__ __forceinline__ bool img_overlap(int e, int len, int &base, int &start)
{
    const int f = e + len;
    if (e < RG0_E && f > RG0_S) { base = RG0_B; start = RG0_S; return true; }
    if (e < RG1_E && f > RG1_S) { base = RG1_B; start = RG1_S; return true; }
    if (e < RG2_E && f > RG2_S) { base = RG2_B; start = RG2_S; return true; }
    if (e < RG3_E && f > RG3_S) { base = RG3_B; start = RG3_S; return true; }
    return false;
}

__device__ __forceinline__ bool cont_overlap(int e, int len)
{
    const int f = e + len;
    return (e < CT0_E && f > CT0_S) || (e < CT1_E && f > CT1_S);
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

// Stage 1 for one pid: every nonzero element the piece contributes, scattered
// into bits / img (observation.py:908-1620 per-piece writers).
__device__ void obs_scatter_piece(const State &S, int env, int obs, int pid, int m, ObsLds &L)
{
    const int tm = (obs + 2) & 3, le = (obs + 1) & 3, re = (obs + 3) & 3, team = obs & 1;
    const size_t pi = (size_t)env * PID_STRIDE + pid;
    const int pos = S.pos[pi];
    const int tp = S.ptype[pi];
    const int s = pid / 30;
    const int rel = s == obs ? 0 : s == tm ? 1 : s == le ? 2 : 3;
    const bool ours = (s & 1) == team;
    float rc[4] = {0.f, 0.f, 0.f, 0.f};

    if ((unsigned)pos < (unsigned)NC) {
        const int k = cT.rot[obs][pos];
        // piece_own (0-11), side occupancy (25, 26), dark_teammate (24)
        if (rel == 0 && tp >= 2 && tp <= 13) set_el(L, (tp - 2) * NC + k);
        if (rel == 2) set_el(L, 25 * NC + k);
        if (rel == 3) set_el(L, 26 * NC + k);
        if (rel == 1 && S.show_mode == SM_DARK) set_el(L, 24 * NC + k);
        // beliefs (12-23 teammate, 27-38 left, 39-50 right)
        if (rel != 0) {
            int bc = S.bcode[((size_t)env * 4 + obs) * PID_STRIDE + pid];
            bc = bc < BC_COUNT ? bc : 0;
            const int c0 = rel == 1 ? 12 : rel == 2 ? 27 : 39;
            const int base = rel == 1 ? RG0_B : RG1_B, start = rel == 1 ? RG0_S : RG1_S;
            for (int j = 0; j < 12; ++j) {
                const uint8_t v = cBVAL[bc][j];
                if (v) set_code(L, base, start, (c0 + j) * NC + k, m, v);
            }
        }
        // move / active_eat / passive_survive buckets (66-89): own team in the
        // first four planes of each group, the other team in the last four
        const int half = ours ? 0 : 4;
        const int mb = min((int)S.mcount[pi], 3), eb = min((int)S.aeat[pi], 3), sb = min((int)S.psurv[pi], 3);
        set_el(L, (66 + half + mb) * NC + k);
        for (int q = 0; q <= eb; ++q) set_el(L, (74 + half + q) * NC + k);
        for (int q = 0; q <= sb; ++q) set_el(L, (82 + half + q) * NC + k);
        // piece_slot (104-128); a camp slot lands on the last plane, like numpy's -1
        const int sc = cT.slotch[pid % 30];
        set_el(L, (104 + (sc < 0 ? 24 : sc)) * NC + k);

        uint64_t cmb = 0;
        if (!ours) {   // combat-memory layers 1 and 3 (observation.py:1292-1387, 1475-1567)
            const size_t ci = cm_idx(env, obs, pid);
            const uint64_t dlo = S.cm_dlo[ci], dhi = S.cm_dhi[ci];
            const int mcnt = __popcll(dlo) + __popcll(dhi);
            const int ocnt = S.cm_ocnt[ci];
            const int ccnt = __popcll(S.cm_clo[ci]) + __popcll(S.cm_chi[ci]);
            const int fl = S.cm_floor[ci];
            const uint8_t flg = S.cm_flags[ci];
            cmb |= (uint64_t)(S.cm_dtype[ci] & 0xFFF);
            for (int q = 0; q < 3; ++q) {
                if (mcnt >= q + 1) cmb |= 1ull << (12 + q);
                if (ocnt >= q + 1) cmb |= 1ull << (15 + q);
                if (ccnt >= q + 1) cmb |= 1ull << (30 + q);
            }
            cmb |= (uint64_t)(S.cm_ctype[ci] & 0xFFF) << 18;
            for (int q = 0; q < 9; ++q) if (fl >= q + 1) cmb |= 1ull << (33 + q);
            if (flg & CMF_IS_GONGB) cmb |= 1ull << 42;
            if (flg & CMF_NOT_GONGB) cmb |= 1ull << 43;
            if (back_two(s, S.zero[pi]) && S.mcount[pi] == 0 && !(flg & CMF_ATK_GONGB)) cmb |= 1ull << 44;
            // kill_mine_slot (223-252) and kill_mine_count (211-222) over the
            // observer's own pieces this one has killed directly
            uint64_t tcnt = 0;   // 12 counters of 5 bits, one per tracked type
            for (int sl = 0; sl < 30; ++sl) {
                const int gp = obs * 30 + sl;
                const bool hit = gp < 64 ? ((dlo >> gp) & 1) : ((dhi >> (gp - 64)) & 1);
                if (!hit) continue;
                set_el(L, (223 + sl) * NC + k);
                const int gt = S.ptype[(size_t)env * PID_STRIDE + gp];
                if (gt >= 2 && gt <= 13) tcnt += 1ull << (5 * (gt - 2));
            }
            for (int q = 0; q < 12; ++q) {
                const int c = (int)((tcnt >> (5 * q)) & 31u);
                if (c) set_code(L, RG3_B, RG3_S, (211 + q) * NC + k, m,
                                c == 1 ? CODE_THIRD : c == 2 ? CODE_2THIRD : CODE_ONE);
            }
            const int mc = S.mc[env];
            const int ldir = S.cm_ldir[ci], lchain = S.cm_lchain[ci], fstep = S.cm_fstep[ci];
            auto recency = [&](int last, int q) {
                if (last < 0) return 0.f;
                int el = mc - last;
                el = el < 0 ? 0 : (el > 4095 ? 4095 : el);
                return S.rlut[q * 4096 + el];
            };
            rc[0] = recency(ldir, 0);
            rc[1] = recency(ldir, 1);
            rc[2] = recency(lchain, 2);
            rc[3] = recency(fstep, 3);
        } else if (s == obs) {   // layer 2 (observation.py:1392-1451)
            const size_t li = cm_idx(env, le, pid), ri = cm_idx(env, re, pid);
            const int lc = __popcll(S.cm_dlo[li]) + __popcll(S.cm_dhi[li]) + S.cm_ocnt[li];
            const int rcnt = __popcll(S.cm_dlo[ri]) + __popcll(S.cm_dhi[ri]) + S.cm_ocnt[ri];
            const int pk = lc < rcnt ? lc : rcnt;
            for (int q = 0; q < 3; ++q) if (pk >= q + 1) cmb |= 1ull << (45 + q);
            const uint8_t lf = S.cm_flags[li], rf = S.cm_flags[ri];
            if ((lf & CMF_IS_GONGB) && (rf & CMF_IS_GONGB)) cmb |= 1ull << 48;
            const bool atk = (lf & CMF_ATK_GONGB) || (rf & CMF_ATK_GONGB);
            if (back_two(s, S.zero[pi]) && S.mcount[pi] == 0 && !atk) cmb |= 1ull << 49;
        }
        while (cmb) {   // combat-memory bit planes 161-210
            const int b = __builtin_ctzll(cmb);
            cmb &= cmb - 1;
            set_el(L, (161 + b) * NC + k);
        }
    }
    for (int q = 0; q < 4; ++q) L.rec[pid][q] = rc[q];

    // death_reason (90-101) and dead_at_zero (102-103), observation.py:1103-1180
    const int dstp = S.dstep[pi];
    if (dstp >= 0) {
        const int reason = S.dreason[pi], loc = S.dloc[pi], z = S.zero[pi];
        const int grp = rel == 0 ? 0 : rel == 1 ? 3 : rel == 2 ? 6 : 9;
        if (reason >= 0 && reason <= 2 && dstp > 0 && (unsigned)loc < (unsigned)NC)
            set_el(L, (90 + grp + reason) * NC + cT.rot[obs][loc]);
        if ((unsigned)z < (unsigned)NC) set_el(L, (102 + (ours ? 0 : 1)) * NC + cT.rot[obs][z]);
    }
    // eaten_by_pid (257-316), layer 4 (observation.py:1591-1620): the observer's
    // own piece, at its cell or (dead) its zero cell, marks its killers
    if (rel == 0) {
        const int cell = pos >= 0 ? pos : S.zero[pi];
        if ((unsigned)cell < (unsigned)NC) {
            const size_t ci = cm_idx(env, obs, pid);
            const uint64_t elo = S.cm_elo[ci], ehi = S.cm_ehi[ci];
            const int k = cT.rot[obs][cell];
            for (int half = 0; half < 2; ++half) {
                const int opp = half == 0 ? le : re;
                for (int sl = 0; sl < 30; ++sl) {
                    const int gp = opp * 30 + sl;
                    const bool hit = gp < 64 ? ((elo >> gp) & 1) : ((ehi >> (gp - 64)) & 1);
                    if (hit) set_el(L, (257 + half * 30 + sl) * NC + k);
                }
            }
        }
    }
}

// Build the LDS form of row (env, obs); m is the row's element phase.
__device__ void obs_build(const State &S, int env, int obs, int m, ObsLds &L)
{
    const int t = threadIdx.x;
    {
        uint4 *w = reinterpret_cast<uint4 *>(L.bits);
        for (int i = t; i < OBS_BITS_WORDS / 4; i += OBS_THREADS) w[i] = make_uint4(0, 0, 0, 0);
        uint4 *b = reinterpret_cast<uint4 *>(L.img);
        for (int i = t; i < IMG_BYTES / 16; i += OBS_THREADS) b[i] = make_uint4(0, 0, 0, 0);
    }
    const int8_t *cellg = S.cell + (size_t)env * CELL_STRIDE;
    for (int k = t; k < CELL_STRIDE; k += OBS_THREADS) L.cpid[k] = k < NC ? cellg[cT.unrot[obs][k]] : (int8_t)-1;
    if (t < 32) {
        const float d = t < 17 ? cDECODE[t] : 0.f;
        L.dec[t] = d;
        L.decb[t] = f32_to_bf16_rne(d);
    }
    if (t == 0) {   // turn_history: float64 divide, then rounded to float32 (observation.py:1000-1021)
        double dp = (double)S.mslc[env] / 200.0; if (dp > 1.0) dp = 1.0;
        double mp = (double)S.mc[env] / 4000.0; if (mp > 1.0) mp = 1.0;
        L.turnv[0] = (float)dp; L.turnv[1] = (float)mp;
    }
    __syncthreads();
    if (t < PID_STRIDE) {
        if (t < NP) obs_scatter_piece(S, env, obs, t, m, L);
        else for (int q = 0; q < 4; ++q) L.rec[t][q] = 0.f;
    } else if (t < PID_STRIDE + HIST_LEN) {   // move_history (129-160), observation.py:1207-1231
        const int d = t - PID_STRIDE;
        const int meta = S.hmeta[env];
        const int cnt = meta & 0xFF, head = (meta >> 8) & 31;
        if (d < cnt) {
            const int e = S.hist[(size_t)env * HIST_LEN + ((head - 1 - d) & 31)];
            const int hs = cT.rot[obs][min(e & 0xFFFF, NC - 1)];
            const int hd = cT.rot[obs][min((e >> 16) & 0xFFFF, NC - 1)];
            if (hs != hd) set_code(L, RG2_B, RG2_S, (129 + d) * NC + hs, m, CODE_NEG);
            set_code(L, RG2_B, RG2_S, (129 + d) * NC + hd, m, CODE_ONE);
        }
    } else if (t < PID_STRIDE + HIST_LEN + 7) {   // whole planes: dead_flags 51-53, flag_revealed 54-57
        const int j = t - PID_STRIDE - HIST_LEN;
        // seats in plane order: self, teammate, left enemy, right enemy
        auto seat_at = [&](int i) { return (obs + (i == 0 ? 0 : i == 1 ? 2 : i == 2 ? 1 : 3)) & 3; };
        const bool on = j < 3 ? ((S.sdead[env] >> seat_at(j + 1)) & 1) : ((S.sflag[env] >> seat_at(j - 3)) & 1);
        if (on) {
            const int e0 = (51 + j) * NC, e1 = e0 + NC;
            for (int w = e0 >> 5; w <= (e1 - 1) >> 5; ++w) {
                const int lo = max(e0, w * 32) - w * 32, hi = min(e1, w * 32 + 32) - w * 32;
                const uint32_t mask = (hi - lo == 32) ? 0xFFFFFFFFu : (((1u << (hi - lo)) - 1u) << lo);
                atomicOr(&L.bits[w], mask);
            }
        }
    } else {   // board_static (58-63): fixed cell classes of the canonical frame
        for (int k = t - (PID_STRIDE + HIST_LEN + 7); k < NC; k += OBS_THREADS - (PID_STRIDE + HIST_LEN + 7)) {
            uint32_t sm = cT.statics[k];
            while (sm) {
                const int b = __builtin_ctz(sm);
                sm &= sm - 1;
                if (b < 6) set_el(L, (58 + b) * NC + k);
            }
        }
    }
    __syncthreads();
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

// Value bits of element e in format FMT (0 f32, 1 bf16, 2 u8 code).
template <int FMT>
__device__ __forceinline__ uint32_t obs_elem(const ObsLds &L, int e, int m)
{
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

__device__ __forceinline__ uint32_t nib_to_bytes(uint32_t nib)
{   // 4 bits -> 4 bytes of 0/1: the shifted copies land on disjoint bit positions
    return __umul24(nib & 0xFu, 0x00204081u) & 0x01010101u;
}

// Stream the 91,613-element row to `row` (element size ES, 16-byte chunks).
template <int FMT>
__device__ void obs_emit(const ObsLds &L, uint8_t *row, int m)
{
    constexpr int ES = FMT == 0 ? 4 : FMT == 1 ? 2 : 1;
    constexpr int EPC = 16 / ES;
    const uintptr_t B = (uintptr_t)row;
    const uintptr_t A0 = B & ~(uintptr_t)15;
    const uintptr_t E = B + (uintptr_t)OBS_ROW * ES;
    const int nchunks = (int)((E - A0 + 15) >> 4);
    for (int q = threadIdx.x; q < nchunks; q += OBS_THREADS) {
        const uintptr_t A = A0 + (uintptr_t)q * 16;
        if (A < B || A + 16 > E) {   // partial chunk at either end of the row
            const uintptr_t lo = A < B ? B : A, hi = A + 16 > E ? E : A + 16;
            for (uintptr_t p = lo; p < hi; p += ES) {
                const int e = (int)((p - B) / ES);
                const uint32_t v = obs_elem<FMT>(L, e, m);
                if (ES == 1) *reinterpret_cast<uint8_t *>(p) = (uint8_t)v;
                else if (ES == 2) *reinterpret_cast<uint16_t *>(p) = (uint16_t)v;
                else *reinterpret_cast<uint32_t *>(p) = v;
            }
            continue;
        }
        const int e0 = (int)((A - B) / ES);
        uint32_t w[4];
        if (FMT != 2 && cont_overlap(e0, EPC)) {
            for (int i = 0; i < 4; ++i) w[i] = 0;
            for (int i = 0; i < EPC; ++i) {
                const uint32_t v = obs_elem<FMT>(L, e0 + i, m);
                w[(i * ES) >> 2] |= v << (((i * ES) & 3) * 8);
            }
        } else {
            const uint32_t v = bit_window(L, e0);
            int base, start;
            const bool ov = img_overlap(e0, EPC, base, start);
            if (FMT == 2) {
                for (int i = 0; i < 4; ++i) w[i] = nib_to_bytes(v >> (4 * i));
                if (ov) {
                    const uint4 b = *reinterpret_cast<const uint4 *>(&L.img[img_off(base, start, e0, m)]);
                    w[0] |= b.x; w[1] |= b.y; w[2] |= b.z; w[3] |= b.w;
                }
            } else if (FMT == 1) {
                if (ov) {
                    const uint2 b = *reinterpret_cast<const uint2 *>(&L.img[img_off(base, start, e0, m)]);
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t cw = i < 2 ? b.x : b.y;
                        const int sh = (i & 1) * 16;
                        const uint32_t c0 = ((cw >> sh) & 0xFFu) | ((v >> (2 * i)) & 1u);
                        const uint32_t c1 = ((cw >> (sh + 8)) & 0xFFu) | ((v >> (2 * i + 1)) & 1u);
                        w[i] = L.decb[c0] | (L.decb[c1] << 16);
                    }
                } else {
                    for (int i = 0; i < 4; ++i)
                        w[i] = ((v >> (2 * i)) & 1u) * 0x3F80u + ((v >> (2 * i + 1)) & 1u) * 0x3F800000u;
                }
            } else {
                if (ov) {
                    const uint32_t cw = *reinterpret_cast<const uint32_t *>(&L.img[img_off(base, start, e0, m)]);
                    for (int i = 0; i < 4; ++i)
                        w[i] = __float_as_uint(L.dec[((cw >> (8 * i)) & 0xFFu) | ((v >> i) & 1u)]);
                } else {
                    for (int i = 0; i < 4; ++i) w[i] = ((v >> i) & 1u) * 0x3F800000u;
                }
            }
        }
        *reinterpret_cast<uint4 *>(A) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// The six continuous planes of the u8 format as float32 (N, 6, 17, 17).
__device__ void obs_emit_aux(const ObsLds &L, float *row)
{
    const uintptr_t B = (uintptr_t)row;
    const uintptr_t A0 = B & ~(uintptr_t)15;
    const uintptr_t E = B + (uintptr_t)AUX_ROW * 4;
    const int nchunks = (int)((E - A0 + 15) >> 4);
    for (int q = threadIdx.x; q < nchunks; q += OBS_THREADS) {
        const uintptr_t A = A0 + (uintptr_t)q * 16;
        const uintptr_t lo = A < B ? B : A, hi = A + 16 > E ? E : A + 16;
        uint32_t w[4] = {0, 0, 0, 0};
        for (uintptr_t p = lo; p < hi; p += 4) {
            const int e = (int)((p - B) / 4);
            const int j = e / NC, k = e - j * NC;
            w[(p - A) >> 2] = __float_as_uint(obs_cont_at(L, j < 2 ? 64 + j : 251 + j, k));
        }
        if (lo == A && hi == A + 16) *reinterpret_cast<uint4 *>(A) = make_uint4(w[0], w[1], w[2], w[3]);
        else for (uintptr_t p = lo; p < hi; p += 4) *reinterpret_cast<uint32_t *>(p) = w[(p - A) >> 2];
    }
}

template <int FMT>
__global__ __launch_bounds__(OBS_THREADS) void k_observe(State S, const int8_t *__restrict__ observer, int all_seats,
                                                         void *__restrict__ spatial, float *__restrict__ aux,
                                                         float *__restrict__ glob)
{
    __shared__ ObsLds L;
    const int row = blockIdx.x;
    const int env = all_seats ? row >> 2 : row;
    if (env >= S.n) return;
    const int obs = all_seats ? (row & 3) : (observer ? observer[env] : S.turn[env]) & 3;
    constexpr int ES = FMT == 0 ? 4 : FMT == 1 ? 2 : 1;
    uint8_t *rowp = reinterpret_cast<uint8_t *>(spatial) + (size_t)row * OBS_ROW * ES;
    const int m = (int)(((uintptr_t)rowp / ES) & (16 / ES - 1));
    obs_build(S, env, obs, m, L);
    obs_emit<FMT>(L, rowp, m);
    if (FMT == 2 && aux) obs_emit_aux(L, aux + (size_t)row * AUX_ROW);
    if (glob && threadIdx.x < 28) {   // observation.py:1623-1651
        const int t = threadIdx.x;
        const int le = (obs + 1) & 3, re = (obs + 3) & 3;
        float v;
        if (t < 24) {
            const int seat = t < 12 ? le : re, ti = t % 12;
            const bool trk = (S.remtrk[(size_t)env * 4 + obs] >> seat) & 1;
            v = trk ? (float)S.rem[((size_t)env * 4 + obs) * 48 + seat * 12 + ti] : 0.f;
        } else {   // flag_revealed of self, teammate, left enemy, right enemy
            const int i = t - 24;
            const int seat = (obs + (i == 0 ? 0 : i == 1 ? 2 : i == 2 ? 1 : 3)) & 3;
            v = (float)((S.sflag[env] >> seat) & 1);
        }
        glob[(size_t)row * 28 + t] = v;
    }
}

}  // namespace jq

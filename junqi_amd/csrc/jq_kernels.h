// HIP kernels for the batched Junqi environment (gfx950, wave64); included by jq_lib.hip.
//
// Execution model: one wavefront owns one env. Its cell map and piece rows are
// staged in LDS; rules logic that is serial by nature (one ply) runs uniformly on
// all 64 lanes, and the wide parts are spread over lanes: the 30 pieces of a seat
// for move generation, the 73 rail nodes for the engineer's reachability closure
// (two 64-bit ballots per hop), the 120 pids for purges and Zobrist folds, and the
// four observers for combat memory and beliefs.
//
// Reference semantics: junqi_core/state.py::GameState.step_inplace (638-998),
// move_gen.py (SoA generator 1052-1199, legacy predicates 127-376),
// combat_memory.py (339-569), info_model.py (218-429).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "junqi_amd.h"
#include "jq_device.h"
#include "jq_topology.h"

namespace jq {

__constant__ Tables cT;
__constant__ uint8_t cBVAL[BC_COUNT][12];   // belief code x type -> obs value code
__constant__ float cDECODE[256];             // obs value code -> float
constexpr int JQ_MASK_WORDS_PAD = 528;
constexpr int LSCR_WORDS = 12;   // legal_body's per-wave LDS scratch (u64 words)

// ------------------------------------------------------------------ helpers
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ uint32_t nib_to_bytes(uint32_t nib)
{   // 4 bits -> 4 bytes of 0/1: the shifted copies land on disjoint bit positions
    return __umul24(nib & 0xFu, 0x00204081u) & 0x01010101u;
}

// Entry i of a byte or halfword table in cT, read through the aligned 32-bit
// word that holds it. At a wave-uniform index this is a scalar load (there are
// none for bytes or halfwords), which neither waits for nor is waited for by
// the wave's vector stores; at a per-lane index it is an ordinary vector load.
template <typename T>
__device__ __forceinline__ T tab(const T *table, int i)
{
    static_assert(sizeof(T) <= 2, "byte and halfword tables only");
    typedef const __attribute__((address_space(4))) uint32_t *const_word;   // constant memory
    const uintptr_t a = reinterpret_cast<uintptr_t>(table + i);
    const uint32_t w = *reinterpret_cast<const_word>(a & ~uintptr_t(3));
    return (T)(w >> (8 * (a & 3)));
}

__device__ __forceinline__ uint16_t cflags(int f) { return tab(cT.cflags, f); }

// A 32-bit word of global memory at a wave-uniform address, read as a scalar
// load. Only for a word no wave writes before this read in the same kernel
// (an env's CSR count and offset are rewritten only by that env's own wave,
// after it has read them): the scalar cache is not coherent with vector stores.
// Loads through the constant address space count as invariant to the compiler,
// which may then re-issue one at a later use instead of keeping its register;
// after the wave's own store to the word that would read the new value. The
// empty asm takes the loaded word as its output, which the compiler can only
// keep (or spill), never recompute: every later use sees the value read here.
__device__ __forceinline__ int32_t uniform_word_raw(const int32_t *p)
{
    typedef const __attribute__((address_space(4))) int32_t *const_i32;
    return *reinterpret_cast<const_i32>(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ void pin_word(int32_t &v) { asm volatile("" : "+s"(v)); }
__device__ __forceinline__ int32_t uniform_word(const int32_t *p)
{
    int32_t v = uniform_word_raw(p);
    pin_word(v);
    return v;
}

// An env's 32-byte record as one scalar load: only the env's own wave writes it,
// after reading it (at the end of its ply or restart); every field keeps the
// value read here (uniform_word).
__device__ __forceinline__ EnvRec env_record(const State &S, int env)
{
    const int32_t *w = reinterpret_cast<const int32_t *>(S.env + env);
    int32_t v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = uniform_word_raw(w + k);
#pragma unroll
    for (int k = 0; k < 8; ++k) pin_word(v[k]);
    EnvRec E;
    __builtin_memcpy(&E, v, sizeof E);
    return E;
}
__device__ __forceinline__ bool is_on(int f) { return cflags(f) & CF_ON; }
__device__ __forceinline__ bool is_rail(int f) { return cflags(f) & CF_RAIL; }
__device__ __forceinline__ bool is_camp(int f) { return cflags(f) & CF_CAMP; }
__device__ __forceinline__ bool is_sh(int f) { return cflags(f) & CF_SH; }
__device__ __forceinline__ int curve_of(int f) { return cflags(f) >> 8; }
__device__ __forceinline__ int team_of(int pid) { return (pid / 30) & 1; }

__device__ __forceinline__ bool enemy_att(const int8_t *cell, int f, int team)
{   // enemy piece on a non-camp cell (move_gen.py:822-867)
    const int p = cell[f];
    return p >= 0 && team_of(p) != team && !is_camp(f);
}
__device__ __forceinline__ bool landable(const int8_t *cell, int f, int team)
{
    return cell[f] < 0 || enemy_att(cell, f, team);
}

__device__ __forceinline__ void setbit3(uint64_t &m0, uint64_t &m1, uint64_t &m2, int c)
{
    const uint64_t b = 1ull << (c & 63);
    const int w = c >> 6;
    m0 |= (w == 0) ? b : 0ull;
    m1 |= (w == 1) ? b : 0ull;
    m2 |= (w == 2) ? b : 0ull;
}

// Whole-wave reductions (every lane active), from the ROCm device library's
// wavefront reductions (DPP / lane permutes instead of six LDS shuffles).
extern "C" __device__ __attribute__((const)) unsigned long long __ockl_wfred_or_u64(unsigned long long);
extern "C" __device__ __attribute__((const)) unsigned long long __ockl_wfred_xor_u64(unsigned long long);
extern "C" __device__ __attribute__((const)) unsigned long long __ockl_wfred_max_u64(unsigned long long);
extern "C" __device__ __attribute__((const)) int __ockl_wfred_add_i32(int);
__device__ __forceinline__ uint64_t wave_or(uint64_t v) { return __ockl_wfred_or_u64(v); }
__device__ __forceinline__ uint64_t wave_xor(uint64_t v) { return __ockl_wfred_xor_u64(v); }
__device__ __forceinline__ uint64_t wave_max(uint64_t v) { return __ockl_wfred_max_u64(v); }
__device__ __forceinline__ int wave_sum(int v) { return __ockl_wfred_add_i32(v); }

// Reachability closure of an engineer standing on rail index `src_r`: the source
// plus every rail node joined to it through empty rail cells. Lane l evaluates
// nodes l and l+64 each hop; the frontier grows until a hop adds nothing, or
// until it touches a node of the target set (t0, t1) when one is given. A node
// already in the closure may be reported again by its lane: growth is what the
// ballot adds beyond the closure.
__device__ void rail_closure(const int8_t *cell, int src_r, uint64_t &r0, uint64_t &r1, uint64_t t0 = 0,
                             uint64_t t1 = 0)
{
    const int l = lane_id();
    const int v1 = l + 64;
    const bool e0 = cell[cT.railcell[l]] < 0;
    const bool e1 = v1 < NRAIL && cell[cT.railcell[v1 < NRAIL ? v1 : 0]] < 0;
    const uint64_t a0 = cT.rnbr[l][0], a1 = cT.rnbr[l][1];
    const uint64_t b0 = v1 < NRAIL ? cT.rnbr[v1][0] : 0ull, b1 = v1 < NRAIL ? cT.rnbr[v1][1] : 0ull;
    r0 = src_r < 64 ? (1ull << src_r) : 0ull;
    r1 = src_r >= 64 ? (1ull << (src_r - 64)) : 0ull;
    for (int hop = 0; hop < NRAIL; ++hop) {
        if ((r0 & t0) | (r1 & t1)) break;
        const uint64_t g0 = __ballot(e0 && ((a0 & r0) | (a1 & r1)) != 0);
        const uint64_t g1 = __ballot(e1 && ((b0 & r0) | (b1 & r1)) != 0) & 0x1FFull;
        if (!((g0 & ~r0) | (g1 & ~r1))) break;
        r0 |= g0;
        r1 |= g1;
    }
}

// Engineer destinations (move_gen.py:870-895) as a compact-index mask (uniform).
__device__ void engineer_mask(const int8_t *cell, int src, int team, uint64_t &m0, uint64_t &m1, uint64_t &m2)
{
    const int l = lane_id();
    const int sr = cT.railidx[src];
    uint64_t r0, r1;
    rail_closure(cell, sr, r0, r1);
    uint64_t p0 = 0, p1 = 0, p2 = 0;
    for (int v = l; v < NRAIL; v += 64) {
        const bool adj = ((cT.rnbr[v][0] & r0) | (cT.rnbr[v][1] & r1)) != 0;
        const int f = cT.railcell[v];
        if (v != sr && adj && landable(cell, f, team)) setbit3(p0, p1, p2, cT.f2c[f]);
    }
    m0 = wave_or(p0); m1 = wave_or(p1); m2 = wave_or(p2);
}

// ------------------------------------------------------------------ bitboards
// 129-bit sets over compact cells (bit c = compact cell c), three words.
struct BB {
    uint64_t w0, w1, w2;
};
__device__ __forceinline__ bool bb_has(const BB &b, int c)
{
    const uint64_t w = c < 64 ? b.w0 : c < 128 ? b.w1 : b.w2;
    return (w >> (c & 63)) & 1ull;
}
__device__ __forceinline__ BB bb_and(const BB &a, const BB &b) { return {a.w0 & b.w0, a.w1 & b.w1, a.w2 & b.w2}; }
__device__ __forceinline__ BB bb_or(const BB &a, const BB &b) { return {a.w0 | b.w0, a.w1 | b.w1, a.w2 | b.w2}; }
__device__ __forceinline__ bool bb_any(const BB &b) { return (b.w0 | b.w1 | b.w2) != 0; }
__device__ __forceinline__ int bb_lowest(const BB &b)
{
    return b.w0 ? __builtin_ctzll(b.w0) : b.w1 ? 64 + __builtin_ctzll(b.w1) : 128 + __builtin_ctzll(b.w2);
}
__device__ __forceinline__ int bb_highest(const BB &b)
{
    return b.w2 ? 191 - __builtin_clzll(b.w2) : b.w1 ? 127 - __builtin_clzll(b.w1) : 63 - __builtin_clzll(b.w0);
}
__device__ __forceinline__ uint64_t lowmask(int n)
{   // bits [0, n) of a word, n clamped to [0, 64]
    return n <= 0 ? 0ull : n >= 64 ? ~0ull : (1ull << n) - 1ull;
}
__device__ __forceinline__ BB bb_below(int c) { return {lowmask(c), lowmask(c - 64), lowmask(c - 128)}; }
__device__ __forceinline__ BB bb_above(int c) { return {~lowmask(c + 1), ~lowmask(c - 63), ~lowmask(c - 127)}; }

// Number of set bits of the 289-bit flat mask m below bit f (0 <= f < 289):
// with m = on-board cells this is f's compact index, with m = rail cells its
// rail index. The masks are uniform, so they sit in scalar registers.
__device__ __forceinline__ int flat_rank(const uint64_t m[5], int f)
{
    int n = 0;
#pragma unroll
    for (int k = 0; k < 5; ++k) n += __popcll(m[k] & lowmask(f - 64 * k));
    return n;
}
__device__ __forceinline__ bool flat_has(const uint64_t m[5], int f)
{
    const int k = f >> 6;
    const uint64_t w = k == 0 ? m[0] : k == 1 ? m[1] : k == 2 ? m[2] : k == 3 ? m[3] : m[4];
    return (w >> (f & 63)) & 1ull;
}

// Occupied cells and cells holding an enemy of `team` that may be attacked
// (not in a camp) of the env whose board is `cell` (flat, LDS). Uniform.
__device__ __forceinline__ void env_boards(const int8_t *cell, int team, BB &occ, BB &ea)
{
    const int l = lane_id();
    const int p0 = cell[cT.c2f[l]], p1 = cell[cT.c2f[l + 64]], p2 = l == 0 ? cell[cT.c2f[128]] : -1;
    occ = {__ballot(p0 >= 0), __ballot(p1 >= 0), __ballot(p2 >= 0)};
    const BB en = {__ballot(p0 >= 0 && team_of(p0) != team), __ballot(p1 >= 0 && team_of(p1) != team),
                   __ballot(p2 >= 0 && team_of(p2) != team)};
    ea = {en.w0 & ~cT.campm[0], en.w1 & ~cT.campm[1], en.w2 & ~cT.campm[2]};
}

// Road steps and, for non-engineers on a rail, straight runs and curve runs of
// the piece on compact cell sc (rail index r or -1), lane-local
// (move_gen.py:1052-1199 parts a, b, c, e), split in two halves so two lanes
// share one piece: half h takes road / camp neighbours 4h .. 4h + 3 of adjc,
// the +x / -x (h = 0) or +y / -y (h = 1) straight runs, and curve run h. The
// union of both halves is the piece's move set. land = empty or attackable.
__device__ __forceinline__ BB piece_moves_half(int sc, int r, bool engineer, int h, const BB &occ, const BB &ea)
{
    const BB land = {~occ.w0 | ea.w0, ~occ.w1 | ea.w1, (~occ.w2 | ea.w2) & 1ull};
    // this half's road / camp neighbours that are empty or attackable
    const uint64_t *am = cT.adjm[sc][h];
    BB m = {am[0] & land.w0, am[1] & land.w1, am[2] & land.w2};
    if (engineer || r < 0) return m;
#pragma unroll
    for (int j = 0; j < 2; ++j) {   // k = 2h + j; j = 0 runs toward higher compact indices
        const int k = 2 * h + j;
        const BB run = {cT.raym[r][k][0], cT.raym[r][k][1], cT.raym[r][k][2]};
        const BB blk = bb_and(run, occ);
        if (!bb_any(blk)) {
            m = bb_or(m, run);
        } else {   // cells before the first occupied one, plus that one if attackable
            const int f = j ? bb_highest(blk) : bb_lowest(blk);
            m = bb_or(m, bb_and(run, j ? bb_above(f) : bb_below(f)));
            if (bb_has(ea, f)) setbit3(m.w0, m.w1, m.w2, f);
        }
    }
    const uint4 q = *reinterpret_cast<const uint4 *>(cT.crayc[r][h]);
    uint64_t qlo = ((uint64_t)q.y << 32) | q.x, qhi = ((uint64_t)q.w << 32) | q.z;   // cells in walk order
    bool open = true;
    // walk until every lane of the wave has met its run's end or first
    // occupied cell (runs are short and usually blocked early)
    for (int i = 0; i < 12 && __ballot(open) != 0; ++i) {
        const int c = (int)(qlo & 0xFF);
        qlo = (qlo >> 8) | (qhi << 56);
        qhi >>= 8;
        if (!open) continue;
        if (c == 0xFF) { open = false; continue; }
        if (!bb_has(occ, c)) { setbit3(m.w0, m.w1, m.w2, c); continue; }
        if (bb_has(ea, c)) setbit3(m.w0, m.w1, m.w2, c);
        open = false;
    }
    return m;
}

// Rail destinations of up to three engineers at once (move_gen.py:870-895): the
// landable rail nodes adjacent to the closure of engineer j's source (rail
// index sr[j]) through empty rail nodes, OR-ed into the wave's LDS words
// dst[3j .. 3j + 2] (compact cells; zero on entry). Lane v evaluates rail nodes
// v and v + 64 each hop; an engineer whose closure stopped growing is skipped.
__device__ __forceinline__ void engineers_bb(int ne, const int sr[3], const BB &occ, const BB &ea, uint64_t *dst)
{
    const int l = lane_id(), v1 = l + 64;
    const bool has1 = v1 < NRAIL;
    const int c0 = cT.railc[l], c1 = has1 ? cT.railc[v1] : 0;
    const bool e0 = !bb_has(occ, c0), e1 = has1 && !bb_has(occ, c1);
    const bool l0 = e0 || bb_has(ea, c0), l1 = has1 && (e1 || bb_has(ea, c1));   // landable (empty or attackable)
    const uint64_t a0 = cT.rnbr[l][0], a1 = cT.rnbr[l][1];
    const uint64_t b0 = has1 ? cT.rnbr[v1][0] : 0ull, b1 = has1 ? cT.rnbr[v1][1] : 0ull;
    uint64_t r0[3], r1[3];
    bool grow[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        grow[j] = j < ne;
        r0[j] = j < ne && sr[j] < 64 ? 1ull << sr[j] : 0ull;
        r1[j] = j < ne && sr[j] >= 64 ? 1ull << (sr[j] - 64) : 0ull;
    }
    for (int hop = 0; hop < NRAIL && (grow[0] || grow[1] || grow[2]); ++hop) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            if (!grow[j]) continue;
            const uint64_t g0 = __ballot(e0 && ((a0 & r0[j]) | (a1 & r1[j])) != 0);
            const uint64_t g1 = __ballot(e1 && ((b0 & r0[j]) | (b1 & r1[j])) != 0) & 0x1FFull;
            grow[j] = ((g0 & ~r0[j]) | (g1 & ~r1[j])) != 0;
            r0[j] |= g0;
            r1[j] |= g1;
        }
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        if (j >= ne) break;
        if (l != sr[j] && l0 && ((a0 & r0[j]) | (a1 & r1[j])) != 0)
            atomicOr(reinterpret_cast<unsigned long long *>(&dst[3 * j + (c0 >> 6)]), 1ull << (c0 & 63));
        if (has1 && v1 != sr[j] && l1 && ((b0 & r0[j]) | (b1 & r1[j])) != 0)
            atomicOr(reinterpret_cast<unsigned long long *>(&dst[3 * j + (c1 >> 6)]), 1ull << (c1 & 63));
    }
}

// Road steps and (for non-engineers) straight rays and curve runs of one piece,
// computed by the calling lane alone (move_gen.py:1052-1199 parts a, b, c, e).
__device__ void piece_mask_lane(const int8_t *cell, int src, int team, bool engineer,
                                uint64_t &m0, uint64_t &m1, uint64_t &m2)
{
    m0 = m1 = m2 = 0;
    for (int k = 0; k < 4; ++k) {
        const int nb = cT.adj[src][k];
        if (nb >= 0 && landable(cell, nb, team)) setbit3(m0, m1, m2, cT.f2c[nb]);
    }
    for (int k = 0; k < 4; ++k) {
        const int nb = cT.diag[src][k];
        if (nb >= 0 && landable(cell, nb, team)) setbit3(m0, m1, m2, cT.f2c[nb]);
    }
    if (engineer) return;
    const int r = cT.railidx[src];
    if (r < 0) return;
    for (int k = 0; k < 4; ++k) {
        const int len = cT.raylen[r][k];
        for (int i = 0; i < len; ++i) {
            const int nb = cT.rays[r][k][i];
            if (cell[nb] < 0) { setbit3(m0, m1, m2, cT.f2c[nb]); continue; }
            if (enemy_att(cell, nb, team)) setbit3(m0, m1, m2, cT.f2c[nb]);
            break;
        }
    }
    for (int d = 0; d < 2; ++d) {
        const int len = cT.craylen[r][d];
        for (int i = 0; i < len; ++i) {
            const int nb = cT.crays[r][d][i];
            if (cell[nb] < 0) { setbit3(m0, m1, m2, cT.f2c[nb]); continue; }
            if (enemy_att(cell, nb, team)) setbit3(m0, m1, m2, cT.f2c[nb]);
            break;
        }
    }
}

// dst on a straight run (k < 4) or curve run of src with every earlier cell empty
// (move_gen.py:127-171 and 384-423). Wave-uniform: table reads are scalar loads.
// A straight move stays on src's row or column, so only the run toward dst is
// walked; its 12 entries come in with one batch of word loads.
__device__ __forceinline__ bool run_clear(const int8_t *cell, int src, int dst, bool curve)
{
    typedef const __attribute__((address_space(4))) uint32_t *const_word;
    const int r = tab(cT.railidx, src);
    if (r < 0) return false;
    if (!curve) {
        const int sx = src % 17, sy = src / 17, dx = dst % 17, dy = dst / 17;
        const int k = sy == dy ? (dx > sx ? 0 : 1) : (dy > sy ? 2 : 3);   // +x, -x, +y, -y
        const int len = tab(&cT.raylen[r][0], k);
        const_word rw = reinterpret_cast<const_word>(reinterpret_cast<uintptr_t>(cT.rays[r][k]));
        uint32_t w[6];
#pragma unroll
        for (int j = 0; j < 6; ++j) w[j] = rw[j];
        for (int i = 0; i < 12; ++i) {
            if (i >= len) break;
            const int nb = (int16_t)(w[i >> 1] >> (16 * (i & 1)));
            if (nb == dst) return true;
            if (__builtin_amdgcn_readfirstlane(cell[nb]) >= 0) return false;
        }
        return false;
    }
    for (int k = 0; k < 2; ++k) {
        const int len = tab(&cT.craylen[r][0], k);
        for (int i = 0; i < len; ++i) {
            const int nb = tab(&cT.crays[r][k][0], i);
            if (nb == dst) return true;
            if (__builtin_amdgcn_readfirstlane(cell[nb]) >= 0) break;
        }
    }
    return false;
}

__device__ __forceinline__ bool engineer_reaches(const int8_t *cell, int src, int dst)
{   // move_gen.py:186-224: dst is adjacent to the closure of src
    if (!is_rail(src) || !is_rail(dst) || src == dst) return false;
    uint64_t r0, r1;
    const int dr = tab(cT.railidx, dst);
    const uint64_t t0 = cT.rnbr[dr][0], t1 = cT.rnbr[dr][1];
    rail_closure(cell, tab(cT.railidx, src), r0, r1, t0, t1);
    return ((t0 & r0) | (t1 & r1)) != 0;
}

// is_legal_move (move_gen.py:299-376), uniform over the wave.
__device__ __forceinline__ bool legal_pair(const int8_t *cell, const int8_t *ptype, int seat, int src, int dst)
{
    if (src < 0 || src >= NC || dst < 0 || dst >= NC || src == dst) return false;
    if (!is_on(src) || !is_on(dst)) return false;
    const int p = __builtin_amdgcn_readfirstlane(cell[src]);   // LDS reads at uniform cells: uniform values
    if (p < 0 || p / 30 != seat) return false;
    const int t = __builtin_amdgcn_readfirstlane(ptype[p]);
    if (t < T_ZHADAN || t > T_GONGB) return false;   // JUNQI / DILEI never move (no other value is a piece)
    if (is_sh(src)) return false;
    const int q = __builtin_amdgcn_readfirstlane(cell[dst]);   // landable: empty, or an enemy outside a camp
    if (q >= 0 && (team_of(q) == (seat & 1) || is_camp(dst))) return false;
    const int sx = src % 17, sy = src / 17, dx = dst % 17, dy = dst / 17;
    const int adx = abs(sx - dx), ady = abs(sy - dy);
    if (adx <= 1 && ady <= 1) {
        if (adx == 1 && ady == 1) { if (is_camp(src) || is_camp(dst)) return true; }
        else return true;
    }
    if (!(is_rail(src) && is_rail(dst))) return false;
    if (t == T_GONGB) return engineer_reaches(cell, src, dst);
    if (sx == dx || sy == dy) return run_clear(cell, src, dst, false);
    if (curve_of(src) > 0 && curve_of(src) == curve_of(dst)) return run_clear(cell, src, dst, true);
    return false;
}

// move_requires_gongb (move_gen.py:245-296) for a legal engineer move.
__device__ __forceinline__ bool engineer_only(const int8_t *cell, int src, int dst)
{
    const int sx = src % 17, sy = src / 17, dx = dst % 17, dy = dst / 17;
    const int adx = abs(sx - dx), ady = abs(sy - dy);
    if (adx + ady == 1) return false;
    if (adx == 1 && ady == 1 && (is_camp(src) || is_camp(dst))) return false;
    if (!(is_rail(src) && is_rail(dst))) return false;
    if (sx == dx || sy == dy) {
        if (run_clear(cell, src, dst, false)) return false;
        return engineer_reaches(cell, src, dst);
    }
    if (curve_of(src) > 0 && curve_of(src) == curve_of(dst) && run_clear(cell, src, dst, true)) return false;
    return engineer_reaches(cell, src, dst);
}

// Does `seat` have a legal move (the Q12 test, state.py:1139-1165)?
__device__ __forceinline__ bool seat_has_move(const int8_t *cell, const int16_t *pos, const int8_t *ptype, int seat)
{
    const int l = lane_id(), team = seat & 1;
    bool mov = false, quick = false, eng = false;
    int src = -1;
    if (l < 30) {
        const int pid = seat * 30 + l;
        src = pos[pid];
        const int t = ptype[pid];
        // one round of independent table loads (flags and the four road
        // neighbours), then the LDS reads: no load waits on another
        const int s = src >= 0 ? src : 0;
        const uint16_t fl = cT.cflags[s];
        const int n0 = cT.adj[s][0], n1 = cT.adj[s][1], n2 = cT.adj[s][2], n3 = cT.adj[s][3];
        mov = src >= 0 && t != T_JUNQI && t != T_DILEI && !(fl & CF_SH);
        eng = t == T_GONGB;
        const bool e0 = (n0 >= 0) & (cell[n0 >= 0 ? n0 : 0] < 0), e1 = (n1 >= 0) & (cell[n1 >= 0 ? n1 : 0] < 0);
        const bool e2 = (n2 >= 0) & (cell[n2 >= 0 ? n2 : 0] < 0), e3 = (n3 >= 0) & (cell[n3 >= 0 ? n3 : 0] < 0);
        quick = mov & (e0 | e1 | e2 | e3);
    }
    if (__ballot(mov && quick)) return true;
    uint64_t m0 = 0, m1 = 0, m2 = 0;
    if (mov) piece_mask_lane(cell, src, team, eng, m0, m1, m2);
    if (__ballot((m0 | m1 | m2) != 0)) return true;
    uint64_t engs = __ballot(mov && eng && is_rail(src < 0 ? 0 : src));
    while (engs) {
        const int e = __builtin_ctzll(engs);
        engs &= engs - 1;
        const int esrc = __builtin_amdgcn_readlane(src, e);   // e is wave-uniform
        uint64_t e0, e1, e2;
        engineer_mask(cell, esrc, team, e0, e1, e2);
        if (e0 | e1 | e2) return true;
    }
    return false;
}

__device__ __forceinline__ int resolve_combat(int a, int d)
{   // rules.py:466-516, rows in order
    if (a == T_ZHADAN || d == T_ZHADAN) return EV_BOMB;
    if (d == T_JUNQI) return EV_EAT;
    if (d == T_DILEI) return a == T_GONGB ? EV_EAT : EV_KILLED;
    if (a == d) return EV_BOMB;
    return a < d ? EV_EAT : EV_KILLED;
}

// The Zobrist key table is written only by its upload, never by a kernel, so
// kernels read it as constant memory: a wave-uniform key is then a scalar load,
// which does not wait behind the wave's vector stores.
typedef const __attribute__((address_space(4))) uint64_t *KeyTable;
__device__ __forceinline__ KeyTable keys(const uint64_t *z) { return reinterpret_cast<KeyTable>(reinterpret_cast<uintptr_t>(z)); }

__device__ __forceinline__ uint64_t zp(const uint64_t *z, int pid, int t, int f)
{   // indexes come from state rows; out-of-range values read entry 0 instead of faulting
    pid = (unsigned)pid < 120u ? pid : 0;
    t = (unsigned)t < 14u ? t : 0;
    f = (unsigned)f < 289u ? f : 0;
    return keys(z)[((size_t)pid * 14 + t) * 289 + f];
}

__device__ __forceinline__ int tracked(int t) { return (t >= 2 && t <= 13) ? t - 2 : -1; }
__device__ __forceinline__ bool code_onehot(int c) { return c >= 1 && c <= 12; }
__device__ __forceinline__ int rank_floor_next(int t)
{   // combat_memory.py:163-173: ordinary rank GONGB=1..SILING=9, floor = min(rank+1, 9)
    if (t < T_SILING || t > T_GONGB) return 0;
    const int r = T_GONGB - t + 1;
    return r + 1 < 9 ? r + 1 : 9;
}
__device__ __forceinline__ bool sees_truth(int o, int owner, int mode)
{   // info_model.py:568-577
    if (mode == SM_BRIGHT || o == owner) return true;
    return mode == SM_HALF_DARK && ((o & 1) == (owner & 1));
}

// ------------------------------------------------------------------ step
struct StepOut {
    uint8_t *valid; int8_t *event; uint8_t *term; int8_t *winner; uint8_t *draw;
    uint8_t *fcap; uint8_t *died; float *reward; int32_t *world;
    uint64_t *hash;   // Zobrist hash after the ply (unchanged when none was applied)
};

// The values a ply reports (wave-uniform). The caller stores them once its
// own loads are issued: a load issued after a store waits for that store too.
struct StepRes {
    int valid, event, term, winner, draw, fcap, died, world;
    float reward;
    uint64_t hash;
};

__device__ __forceinline__ void write_step_res(const StepOut &O, int env, const StepRes &r)
{
    if (O.valid) O.valid[env] = (uint8_t)r.valid;
    if (O.event) O.event[env] = (int8_t)r.event;
    if (O.term) O.term[env] = (uint8_t)r.term;
    if (O.winner) O.winner[env] = (int8_t)r.winner;
    if (O.draw) O.draw[env] = (uint8_t)r.draw;
    if (O.fcap) O.fcap[env] = (uint8_t)r.fcap;
    if (O.died) O.died[env] = (uint8_t)r.died;
    if (O.reward) O.reward[env] = r.reward;
    if (O.world) O.world[env] = r.world;
    if (O.hash) O.hash[env] = r.hash;
}

// Kill pid at its current cell (state.py:1027-1049). Uniform; lane 0 stores.
__device__ void kill_piece(const State &S, int env, int8_t *cell, int16_t *pos, const int8_t *ptype, int pid,
                           int reason, int loc, int step, uint64_t &zob)
{
    const int cur = __builtin_amdgcn_readfirstlane(pos[pid]);
    if ((unsigned)cur >= (unsigned)NC) return;
    zob ^= zp(S.ztab, pid, __builtin_amdgcn_readfirstlane(ptype[pid]), cur);
    wave_sync();
    if (lane_id() == 0) {
        cell[cur] = -1; pos[pid] = -1;
        PieceRec &r = S.piece[pc_idx(env, pid)];
        r.pos = -1; r.dreason = (int8_t)reason; r.dstep = (int16_t)step; r.dloc = (int16_t)loc;
        S.cell[(size_t)env * CELL_STRIDE + cur] = -1;
    }
    wave_sync();
}

__device__ void move_piece(const State &S, int env, int8_t *cell, int16_t *pos, const int8_t *ptype, int pid,
                           int src, int dst, uint64_t &zob)
{   // state.py:1005-1025
    const int t = __builtin_amdgcn_readfirstlane(ptype[pid]);
    zob ^= zp(S.ztab, pid, t, src) ^ zp(S.ztab, pid, t, dst);
    wave_sync();
    if (lane_id() == 0) {
        cell[src] = -1; cell[dst] = (int8_t)pid; pos[pid] = (int16_t)dst;
        S.cell[(size_t)env * CELL_STRIDE + src] = -1;
        S.cell[(size_t)env * CELL_STRIDE + dst] = (int8_t)pid;
        S.piece[pc_idx(env, pid)].pos = (int16_t)dst;
    }
    wave_sync();
}

// Remove every live piece of `seat` (state.py:1639-1692): KILLED_BY_ENEMY at the
// piece's current cell. Lanes 0..29 take one pid each; Zobrist folded by XOR.
__device__ void purge_seat(const State &S, int env, int8_t *cell, int16_t *pos, const int8_t *ptype, int seat,
                           int step, uint64_t &zob)
{
    const int l = lane_id();
    uint64_t z = 0;
    wave_sync();
    if (l < 30) {
        const int pid = seat * 30 + l;
        const int cur = pos[pid];
        if ((unsigned)cur < (unsigned)NC) {
            z = zp(S.ztab, pid, ptype[pid], cur);
            cell[cur] = -1; pos[pid] = -1;
            PieceRec &r = S.piece[pc_idx(env, pid)];
            r.pos = -1; r.dreason = 0; r.dstep = (int16_t)step; r.dloc = (int16_t)cur;
            S.cell[(size_t)env * CELL_STRIDE + cur] = -1;
        }
    }
    zob ^= wave_xor(z);
    wave_sync();
}

// CombatMemory update for EAT / KILLED (combat_memory.py:354-569). Lane o < 4
// handles observer o; observers never touch each other's records. K is the
// surviving piece, V the killed one; V's own kills cannot include K (K is alive).
__device__ __forceinline__ void cm_apply(const State &S, int env, bool is_eat, int apid, int dpid, int aseat, int dseat,
                         int atype, int dtype, int step)
{
    const int o = lane_id();
    if (o >= 4) return;
    int K, V, Vs, Vt;
    if (is_eat) { K = apid; V = dpid; Vs = dseat; Vt = dtype; }
    else        { K = dpid; V = apid; Vs = aseat; Vt = atype; }
    const size_t kI = cm_idx(env, o, K), vI = cm_idx(env, o, V);
    CmRec k = S.cm[kI];
    const CmRec v = S.cm[vI];
    if (!is_eat) {
        const bool known = (v.flags & CMF_IS_GONGB) || (atype == T_GONGB && o == Vs);
        if (known) k.flags |= CMF_ATK_GONGB;
    }
    k.clo |= v.dlo | v.clo;
    k.chi |= v.dhi | v.chi;
    if (V < 64) k.clo |= 1ull << V; else k.chi |= 1ull << (V - 64);
    k.ctype = (uint16_t)(k.ctype | v.dtype | v.ctype);
    if (v.floor > 0) {
        const int prop = v.floor + 1 < 9 ? v.floor + 1 : 9;
        if (prop > k.floor) { k.floor = (int8_t)prop; k.fstep = (int16_t)step; }
        k.flags |= CMF_NOT_GONGB;
    }
    // v6 reverse projection: observer's own pids V had eaten (directly or by chain),
    // plus V itself when V belongs to the observer, are now eaten by K too.
    {
        // pids 30o .. 30o + 29 as a 128-bit set (o = 0..3: bit offsets 0, 30, 60, 90)
        constexpr uint64_t SEAT30 = 0x3FFFFFFFull;
        const int b0 = o * 30;
        const uint64_t mlo = b0 < 64 ? SEAT30 << b0 : 0ull;
        const uint64_t mhi = b0 == 0 ? 0ull : b0 < 64 ? SEAT30 >> (64 - b0) : SEAT30 << (b0 - 64);
        uint64_t vlo = (v.dlo | v.clo) & mlo, vhi = (v.dhi | v.chi) & mhi;
        if (Vs == o) { if (V < 64) vlo |= 1ull << V; else vhi |= 1ull << (V - 64); }
        const uint64_t klo = K < 64 ? (1ull << K) : 0ull, khi = K >= 64 ? (1ull << (K - 64)) : 0ull;
        while (vlo) { const int b = __builtin_ctzll(vlo); vlo &= vlo - 1; CmEat &t = S.cme[cm_idx(env, o, b)]; t.elo |= klo; t.ehi |= khi; }
        while (vhi) { const int b = __builtin_ctzll(vhi) + 64; vhi &= vhi - 1; CmEat &t = S.cme[cm_idx(env, o, b)]; t.elo |= klo; t.ehi |= khi; }
    }
    if (Vs != o) {
        const int c = k.ocnt + 1;
        k.ocnt = (int16_t)(c < 32767 ? c : 32767);
    } else {
        if (V < 64) k.dlo |= 1ull << V; else k.dhi |= 1ull << (V - 64);
        const int vi = tracked(Vt);
        if (vi >= 0) {
            k.dtype = (uint16_t)(k.dtype | (1u << vi));
            k.ctype = (uint16_t)(k.ctype | (1u << vi));
        }
        if (is_eat) k.flags |= (Vt == T_DILEI) ? CMF_IS_GONGB : CMF_NOT_GONGB;
        if (Vt >= T_SILING && Vt <= T_GONGB) {
            const int pr = rank_floor_next(Vt);
            if (pr > k.floor) { k.floor = (int8_t)pr; k.fstep = (int16_t)step; }
        }
    }
    k.ldir = (int16_t)step;
    k.lchain = (int16_t)step;
    S.cm[kI] = k;
    S.cmk[kI] = cm_summary(k);
    S.cmv[kI] = cm_view(k, o);
}

// BeliefTensor.update for the four observers (info_model.py:271-429). Entries are
// keyed by pid so R1 migration is implicit; lane o < 4 handles observer o.
__device__ __forceinline__ void belief_update(const State &S, int env, const int8_t *cell, int sp, int dp, int ss, int ds,
                              int dt, int dst, int ev, bool rsrc, bool rdst, bool fcap, int died)
{
    const int o = lane_id();
    if (o >= 4) return;
    uint8_t *bc = S.bcode + ((size_t)env * 4 + o) * PID_STRIDE;
    int8_t *rem = S.rem + ((size_t)env * 4 + o) * 48;
    uint8_t trk = S.env[env].remtrk[o];
    auto dec = [&](int seat, int ti) {
        if ((trk >> seat) & 1) { int8_t &c = rem[seat * 12 + ti]; if (c > 0) --c; }
    };
    int acode = bc[sp];
    const int dcode = dp >= 0 ? bc[dp] : 0;
    if (rsrc) dec(ss, T_SILING - 2);
    if (rdst) dec(ds, T_SILING - 2);
    if (ev == EV_EAT && dp >= 0 && dt == T_DILEI && !code_onehot(acode)) {
        acode = 1 + (T_GONGB - 2);
        bc[sp] = (uint8_t)acode;
        dec(ss, T_GONGB - 2);
    }
    if (fcap) {
        trk &= (uint8_t)~(1u << ds);
    } else if (ev == EV_EAT && dp >= 0 && is_sh(dst) && tab(cT.owner, dst) == ds) {
        const int other = tab(cT.sh_other, dst);
        const int op = cell[other];
        if (op >= 0 && !code_onehot(bc[op])) bc[op] = (uint8_t)(1 + (T_JUNQI - 2));
    }
    auto removed = [&](int seat, int code) { if (((trk >> seat) & 1) && code_onehot(code)) dec(seat, code - 1); };
    if (ev == EV_EAT) { if (dp >= 0) removed(ds, dcode); }
    else if (ev == EV_KILLED) removed(ss, acode);
    else if (ev == EV_BOMB) { removed(ss, acode); if (dp >= 0) removed(ds, dcode); }
    trk &= (uint8_t)~died;
    S.env[env].remtrk[o] = trk;
}

// What the env record says after a step (wave-uniform), for work that follows
// the step in the same kernel.
struct TurnAfter {
    int turn;
    bool term;
    uint8_t sdead;
};

// One ply of env `env` by its wave (GameState.step_inplace, state.py:700-1167).
// cell / pos / ptype are the wave's LDS arrays; on return they hold the board
// after the step (unchanged if the action was not applied).
// The board and piece records of one env, lane l's share: the loads of a ply's
// first memory round trip, which a caller can issue early.
struct StepLoad {
    int8_t cv[5];
    PieceRec r0, r1;
};

__device__ __forceinline__ void step_load(const State &S, int env, int l, StepLoad &P)
{
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        const int f = l + 64 * k;
        P.cv[k] = f < NC ? S.cell[(size_t)env * CELL_STRIDE + f] : (int8_t)-1;
    }
    P.r0 = S.piece[pc_idx(env, l)];
    P.r1 = S.piece[pc_idx(env, l + 64)];
}

__device__ void step_env(const State &S, int env, int l, int32_t a, const int8_t *__restrict__ acting, int act_fmt,
                         StepRes &res, int8_t *cell, int16_t *pos, int8_t *ptype, TurnAfter &nx,
                         const StepLoad *pre = nullptr, const EnvRec *pre_rec = nullptr)
{

    // the board, the piece records, the env record and the action are all
    // loaded into registers first (one memory round trip, or `pre` issued
    // earlier by the caller), then staged in LDS; the checks below only decide
    // whether the board is used
    StepLoad ld;
    if (pre) ld = *pre;
    else step_load(S, env, l, ld);
    const int8_t *cv = ld.cv;
    const PieceRec &r0 = ld.r0, &r1 = ld.r1;
    // the env record, read once into scalar registers before any store of the
    // ply (only this wave writes it, at the end), or handed in by the caller
    const EnvRec E = pre_rec ? *pre_rec : env_record(S, env);
#pragma unroll
    for (int k = 0; k < 5; ++k)
        if (l + 64 * k < CELL_STRIDE) cell[l + 64 * k] = cv[k];
    pos[l] = r0.pos; ptype[l] = r0.ptype;
    pos[l + 64] = r1.pos; ptype[l + 64] = r1.ptype;
    const bool was_term = E.term != 0;
    const int seat = E.turn;
    nx.turn = seat; nx.term = was_term; nx.sdead = E.sdead;
    res = {0, 0, was_term ? 1 : 0, (int)E.winner, (int)E.draw, 0, 0, -1, 0.f, E.zob};
    if (was_term) return;

    a = __builtin_amdgcn_readfirstlane(a);   // wave-uniform: the ply's scalar work stays on the SALU
    int src = -1, dst = -1;
    if (act_fmt == 1) {
        const int as = __builtin_amdgcn_readfirstlane(acting ? (int)acting[env] : seat);
        if (a >= 0 && a < NONB * NONB && as >= 0 && as < 4) {
            src = tab(cT.unrot[as], tab(cT.c2f, a / NONB));
            dst = tab(cT.unrot[as], tab(cT.c2f, a % NONB));
        }
    } else if (a >= 0 && a < NC * NC) {
        src = a / NC; dst = a % NC;
    }
    if (src >= 0) res.world = src * NC + dst;
    if (src < 0) return;
    if (acting && acting[env] != seat) return;
    const uint8_t sdead0 = E.sdead;
    if ((sdead0 >> seat) & 1) return;
    wave_sync();
    if (!legal_pair(cell, ptype, seat, src, dst)) return;

    const int mc0 = E.mc, mslc0 = E.mslc;
    uint64_t zob = E.zob;
    const KeyTable Z = keys(S.ztab);
    zob ^= Z[ZOFF_TURN + seat] ^ Z[ZOFF_MC + (mc0 & 0xFFF)] ^ Z[ZOFF_MSLC + (mslc0 & 0x1FF)];
    const int step = mc0 + 1;
    int died = 0;
    uint8_t sdead = sdead0, sflag = E.sflag;
    const int sp = __builtin_amdgcn_readfirstlane(cell[src]), dp = __builtin_amdgcn_readfirstlane(cell[dst]);
    const int st = __builtin_amdgcn_readfirstlane(ptype[sp]), dt = dp >= 0 ? __builtin_amdgcn_readfirstlane(ptype[dp]) : -1;
    const int ss = sp / 30, ds = dp >= 0 ? dp / 30 : -1;

    if (st == T_GONGB && engineer_only(cell, src, dst)) {
        if (l < 4) {
            S.cm[cm_idx(env, l, sp)].flags |= CMF_IS_GONGB;
            S.cmk[cm_idx(env, l, sp)] |= (uint8_t)(CMF_IS_GONGB << 2);
            S.cmv[cm_idx(env, l, sp)].types |= (uint32_t)CMF_IS_GONGB << 28;
        }
    }
    // move history (state.py:673-678)
    const int hcnt = E.hmeta & 0xFF, hhead = (E.hmeta >> 8) & 31;
    if (l == 0) S.hist[(size_t)env * HIST_LEN + hhead] = src | (dst << 16);
    int ev;
    bool rsrc = false, rdst = false, fcap = false;
    auto set_flag = [&](int s) { if (!((sflag >> s) & 1)) { sflag |= (uint8_t)(1u << s); zob ^= Z[ZOFF_SFLAG + s]; } };
    auto set_dead = [&](int s) { if (!((sdead >> s) & 1)) { sdead |= (uint8_t)(1u << s); zob ^= Z[ZOFF_SDEAD + s]; } };
    if (dp < 0) {
        ev = EV_MOVE;
        if (l == 0) S.piece[pc_idx(env, sp)].mcount += 1;
        move_piece(S, env, cell, pos, ptype, sp, src, dst, zob);
    } else {
        ev = resolve_combat(st, dt);
        rsrc = st == T_SILING && (ev == EV_KILLED || ev == EV_BOMB);
        rdst = dt == T_SILING && (ev == EV_EAT || ev == EV_BOMB);
        fcap = dt == T_JUNQI;
        if (rsrc) set_flag(ss);
        if (rdst) set_flag(ds);
        if (ev == EV_EAT) {
            if (l == 0) S.piece[pc_idx(env, sp)].aeat += 1;
            kill_piece(S, env, cell, pos, ptype, dp, 0, dst, step, zob);
            move_piece(S, env, cell, pos, ptype, sp, src, dst, zob);
            cm_apply(S, env, true, sp, dp, ss, ds, st, dt, step);
        } else if (ev == EV_KILLED) {
            if (l == 0) S.piece[pc_idx(env, dp)].psurv += 1;
            kill_piece(S, env, cell, pos, ptype, sp, (dt == T_DILEI || dt == T_ZHADAN) ? 1 : 0, dst, step, zob);
            cm_apply(S, env, false, sp, dp, ss, ds, st, dt, step);
        } else {
            kill_piece(S, env, cell, pos, ptype, sp, 2, dst, step, zob);
            kill_piece(S, env, cell, pos, ptype, dp, 2, dst, step, zob);
        }
    }
    if (fcap && !((sdead >> ds) & 1)) {   // state.py:864-890
        set_dead(ds); set_flag(ds);
        purge_seat(S, env, cell, pos, ptype, ds, step, zob);
        died |= 1 << ds;
    }
    {   // dead sweep (state.py:895-901)
        const int p0 = l, p1 = l + 64;
        const bool a0 = pos[p0] >= 0, a1 = p1 < NP && pos[p1] >= 0;
        for (int s = 0; s < 4; ++s) {
            const bool has = __ballot((a0 && p0 / 30 == s) || (a1 && p1 / 30 == s)) != 0;
            if (!((sdead >> s) & 1) && !has) { set_dead(s); died |= 1 << s; }
        }
    }
    const int nmc = mc0 + 1, nmslc = ev == EV_MOVE ? mslc0 + 1 : 0;
    auto victory = [&](int &term, int &win, int &drw) {   // state.py:1695-1726
        const bool red = !(((sdead >> 0) & 1) && ((sdead >> 2) & 1));
        const bool blue = !(((sdead >> 1) & 1) && ((sdead >> 3) & 1));
        term = 0; win = -1; drw = 0;
        if (!red && !blue) { term = 1; win = seat & 1; return; }
        if (!red) { term = 1; win = 1; return; }
        if (!blue) { term = 1; win = 0; return; }
        if (nmc >= 4000 || nmslc >= 200) { term = 1; drw = 1; }
    };
    int term, win, drw, nturn;
    victory(term, win, drw);
    if (!term) {   // state.py:1109-1167
        int cand = (seat + 1) & 3;
        for (int it = 0; it < 4; ++it) {
            if ((sdead >> cand) & 1) { cand = (cand + 1) & 3; continue; }
            if (seat_has_move(cell, pos, ptype, cand)) break;
            set_dead(cand);
            purge_seat(S, env, cell, pos, ptype, cand, step, zob);
            died |= 1 << cand;
            cand = (cand + 1) & 3;
        }
        nturn = cand;
        victory(term, win, drw);
    } else {
        nturn = seat;
    }
    if (!term && nmc >= S.max_moves) { term = 1; drw = 1; }   // env move cap
    zob ^= Z[ZOFF_TURN + nturn] ^ Z[ZOFF_MC + (nmc & 0xFFF)] ^ Z[ZOFF_MSLC + (nmslc & 0x1FF)];
    if (term) zob ^= Z[ZOFF_TERM];
    if (drw) zob ^= Z[ZOFF_DRAW];
    if (win >= 0) zob ^= Z[ZOFF_WIN] ^ Z[ZOFF_WIN + win + 1];

    belief_update(S, env, cell, sp, dp, ss, ds, dt, dst, ev, rsrc, rdst, fcap, died);

    nx.turn = nturn; nx.term = term != 0; nx.sdead = sdead;
    if (l == 0) {
        EnvRec &W = S.env[env];   // remtrk belongs to belief_update's lanes
        W.zob = zob; W.mc = nmc; W.mslc = nmslc;
        W.hmeta = (hcnt < 32 ? hcnt + 1 : 32) | (((hhead + 1) & 31) << 8);
        W.turn = (int8_t)nturn; W.term = (uint8_t)term; W.winner = (int8_t)win; W.draw = (uint8_t)drw;
        W.sdead = sdead; W.sflag = sflag;
    }
    res.valid = 1; res.event = ev; res.term = term; res.winner = win; res.draw = drw; res.fcap = fcap;
    res.died = died; res.hash = zob;
    res.reward = (term && !drw && win >= 0) ? (((seat & 1) == win) ? 1.f : -1.f) : 0.f;
}

__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_step(State S, const int32_t *__restrict__ actions,
                                             const int8_t *__restrict__ acting, int act_fmt, StepOut O)
{
    const int env = blockIdx.x, l = threadIdx.x;
    if (env >= S.n) return;
    __shared__ int8_t cell[CELL_STRIDE];
    __shared__ int16_t pos[PID_STRIDE];
    __shared__ int8_t ptype[PID_STRIDE];
    TurnAfter nx;
    StepRes res;
    step_env(S, env, l, actions[env], acting, act_fmt, res, cell, pos, ptype, nx);
    if (l == 0) write_step_res(O, env, res);
}

// ------------------------------------------------------------------ reset
// Empty, terminated state of one env (no pieces, empty board, zero beliefs),
// written by threads t of nt.
__device__ __forceinline__ void clear_env(const State &S, int env, int t, int nt)
{
    for (int f = t; f < CELL_STRIDE; f += nt) S.cell[(size_t)env * CELL_STRIDE + f] = -1;
    PieceRec r;
    r.pos = r.zero = r.dstep = r.dloc = -1;
    r.mcount = r.aeat = r.psurv = 0;
    r.ptype = r.dreason = -1;
    CmRec c = {};
    c.ldir = c.lchain = c.fstep = -1;
    const CmEat ce = {};
    const CmView cv = cm_view(c, 0);
    for (int p = t; p < PID_STRIDE; p += nt) {
        S.piece[pc_idx(env, p)] = r;
        for (int o = 0; o < 4; ++o) {
            if (S.cm) S.cm[cm_idx(env, o, p)] = c;   // a rebuild-only state keeps no full records
            S.cme[cm_idx(env, o, p)] = ce;
            S.cmk[cm_idx(env, o, p)] = 0;
            S.cmv[cm_idx(env, o, p)] = cv;
            S.bcode[((size_t)env * 4 + o) * PID_STRIDE + p] = 0;
        }
    }
    for (int k = t; k < 4 * 48; k += nt) S.rem[(size_t)env * 4 * 48 + k] = 0;
    for (int k = t; k < HIST_LEN; k += nt) S.hist[(size_t)env * HIST_LEN + k] = 0;
    if (t == 0) {
        EnvRec E = {};
        E.winner = -1;
        E.term = 1;
        S.env[env] = E;
        S.lg[env].n = 0;
        S.lg[env].seat = 0;
    }
}

// Empty, terminated state for every env (before the first reset).
__global__ __launch_bounds__(64) void k_clear(State S)
{
    const int env = blockIdx.x, l = threadIdx.x;
    if (env >= S.n) return;
    clear_env(S, env, l, 64);
}

// Start an env from a lineup (GameState.new_game, state.py:490-620; beliefs,
// info_model.py:218-265). Zobrist includes every term new_game XORs in. If
// lcell is given, the new board is also staged in the wave's LDS arrays
// lcell / lpos / ltype (as step_env leaves them).
__device__ void init_env(const State &S, int env, const int8_t *types, int8_t *lcell = nullptr,
                         int16_t *lpos = nullptr, int8_t *ltype = nullptr)
{
    const int l = lane_id();
    int8_t *cell = S.cell + (size_t)env * CELL_STRIDE;
    for (int f = l; f < CELL_STRIDE; f += 64) {
        cell[f] = -1;
        if (lcell) lcell[f] = -1;
    }
    wave_sync();
    uint64_t z = 0;
    for (int p = l; p < PID_STRIDE; p += 64) {
        const size_t pi = (size_t)env * PID_STRIDE + p;
        const int t = p < NP ? types[p] : 0;
        const bool alive = t != T_NONE && cT.home[p < NP ? p : 0] >= 0 && p < NP;
        const int h = alive ? cT.home[p] : -1;
        PieceRec r;
        r.ptype = alive ? (int8_t)t : (int8_t)-1;
        r.pos = (int16_t)h; r.zero = (int16_t)h;
        r.mcount = 0; r.aeat = 0; r.psurv = 0;
        r.dreason = -1; r.dstep = -1; r.dloc = -1;
        S.piece[pi] = r;
        if (alive) { cell[h] = (int8_t)p; z ^= zp(S.ztab, p, t, h); }
        if (lcell) {
            if (alive) lcell[h] = (int8_t)p;
            lpos[p] = (int16_t)h;
            ltype[p] = r.ptype;
        }
        for (int o = 0; o < 4; ++o) {
            uint8_t code = 0;
            if (alive) code = sees_truth(o, p / 30, S.show_mode) ? (uint8_t)(1 + t - 2) : (uint8_t)(BC_PRIOR0 + p % 30);
            S.bcode[((size_t)env * 4 + o) * PID_STRIDE + p] = code;
            CmRec c = {};
            c.ldir = -1; c.lchain = -1; c.fstep = -1;
            S.cm[cm_idx(env, o, p)] = c;
            S.cme[cm_idx(env, o, p)] = CmEat{};
            S.cmk[cm_idx(env, o, p)] = 0;
            S.cmv[cm_idx(env, o, p)] = cm_view(c, o);
        }
    }
    z = wave_xor(z);
    static constexpr int8_t kCounts[12] = {1, 3, 2, 1, 1, 2, 2, 2, 2, 3, 3, 3};
    for (int i = l; i < 4 * 48; i += 64) {
        const int o = i / 48, s = (i / 12) % 4, t = i % 12;
        const bool tracked_seat = s != o && ((s & 1) != (o & 1));
        S.rem[(size_t)env * 4 * 48 + i] = tracked_seat ? kCounts[t] : 0;
    }
    if (l < 4) {
        uint8_t trk = 0;
        for (int s = 0; s < 4; ++s) if (s != l && ((s & 1) != (l & 1))) trk |= (uint8_t)(1u << s);
        S.env[env].remtrk[l] = trk;
    }
    if (l == 0) {
        const KeyTable Z = keys(S.ztab);
        z ^= Z[ZOFF_TURN + 0] ^ Z[ZOFF_MC + 0] ^ Z[ZOFF_MSLC + 0] ^ Z[ZOFF_WIN + 0] ^ Z[ZOFF_SHOW + S.show_mode];
        EnvRec &W = S.env[env];
        W.zob = z; W.mc = 0; W.mslc = 0; W.hmeta = 0;
        W.turn = 0; W.term = 0; W.winner = -1; W.draw = 0; W.sdead = 0; W.sflag = 0;
    }
}

__global__ __launch_bounds__(64) void k_reset_lineups(State S, const int8_t *__restrict__ lineups)
{
    const int env = blockIdx.x;
    if (env >= S.n) return;
    init_env(S, env, lineups + (size_t)env * NP);
}

// Pool entry a finished env restarts from: the reference reset kernel's hash
// (game_state.cu:2986-2991).
__device__ __forceinline__ int reset_pool_index(int env, int64_t seed, int pool_size)
{
    uint64_t h = (uint64_t)env * 2654435761ull + (uint64_t)seed;
    h ^= h >> 17;
    h *= 0xbf58476d1ce4e5b9ull;
    h ^= h >> 31;
    return (int)(h % (uint64_t)pool_size);
}

__global__ __launch_bounds__(64) void k_reset_terminated(State S, int64_t seed)
{
    const int env = blockIdx.x;
    if (env >= S.n || !S.env[env].term) return;
    init_env(S, env, S.pool + (size_t)reset_pool_index(env, seed, S.pool_size) * NP);
}

// Recompute Zobrist and (if `beliefs`) re-seed beliefs from the current board
// (hand-built states); only envs whose `mask` entry is nonzero when a mask is given.
__global__ __launch_bounds__(64) void k_finalize(State S, int beliefs, const uint8_t *__restrict__ mask)
{
    const int env = blockIdx.x, l = threadIdx.x;
    if (env >= S.n || (mask && !mask[env])) return;
    uint64_t z = 0;
    for (int p = l; p < NP; p += 64) {
        const size_t pi = (size_t)env * PID_STRIDE + p;
        const PieceRec r = S.piece[pi];
        const int f = r.pos, t = r.ptype;
        if (f >= 0 && t >= 0) z ^= zp(S.ztab, p, t, f);
        for (int o = 0; o < 4; ++o) {
            const CmRec c = S.cm[cm_idx(env, o, p)];
            S.cmk[cm_idx(env, o, p)] = cm_summary(c);
            S.cmv[cm_idx(env, o, p)] = cm_view(c, o);
        }
        for (int o = 0; o < 4 && beliefs; ++o) {
            uint8_t code = 0;
            if (f >= 0 && t >= 2) {
                if (sees_truth(o, p / 30, S.show_mode)) code = (uint8_t)(1 + t - 2);
                else code = (cT.owner[f] == p / 30) ? (uint8_t)(BC_PRIOR0 + cT.localidx[f]) : (uint8_t)BC_UNIFORM;
            }
            S.bcode[((size_t)env * 4 + o) * PID_STRIDE + p] = code;
        }
    }
    z = wave_xor(z);
    static constexpr int8_t kCounts[12] = {1, 3, 2, 1, 1, 2, 2, 2, 2, 3, 3, 3};
    if (beliefs && l < 48) {
        for (int o = 0; o < 4; ++o) {
            const int s = l / 12, t = l % 12;
            const bool tracked_seat = s != o && ((s & 1) != (o & 1));
            S.rem[((size_t)env * 4 + o) * 48 + l] = tracked_seat ? kCounts[t] : 0;
        }
    }
    if (beliefs && l < 4) {
        uint8_t trk = 0;
        for (int s = 0; s < 4; ++s) if (s != l && ((s & 1) != (l & 1))) trk |= (uint8_t)(1u << s);
        S.env[env].remtrk[l] = trk;
    }
    if (l == 0) {
        const KeyTable Z = keys(S.ztab);
        const EnvRec &E = S.env[env];
        const int w = E.winner;
        z ^= Z[ZOFF_TURN + (E.turn & 3)] ^ Z[ZOFF_MC + (E.mc & 0xFFF)] ^ Z[ZOFF_MSLC + (E.mslc & 0x1FF)];
        z ^= Z[ZOFF_WIN + (w < 0 ? 0 : (w & 1) + 1)] ^ Z[ZOFF_SHOW + S.show_mode];
        if (E.term) z ^= Z[ZOFF_TERM];
        if (E.draw) z ^= Z[ZOFF_DRAW];
        for (int s = 0; s < 4; ++s) {
            if ((E.sdead >> s) & 1) z ^= Z[ZOFF_SDEAD + s];
            if ((E.sflag >> s) & 1) z ^= Z[ZOFF_SFLAG + s];
        }
        S.env[env].zob = z;
    }
}

// ------------------------------------------------------------------ legal
// Per env: masks of the acting seat's movable pieces (lanes = pieces), engineer
// closures, counts, the packed canonical mask and the CSR scratch in ascending
// source order (move_gen.py:1199 sorts the ids).
// Legal sets of env `env` for `seat` by its wave (off: none): the board in LDS
// (cell, padded to CELL_STRIDE with -1), bits cleared and, for the canonical
// mask, rotl filled. Piece positions / types come from the LDS arrays lpos /
// ltype when given, else from the piece records.
// lscr: LSCR_WORDS words of the wave's LDS, the compact source cells of the
// movable pieces (words 0-2) and the engineers' rail destinations (3-11).
__device__ __forceinline__ void legal_body(const State &S, int env, int l, int seat, bool off, const int8_t *cell, uint32_t *bits,
                           const uint8_t *rotl, const int16_t *lpos, const int8_t *ltype, uint64_t *lscr,
                           int32_t *__restrict__ counts, int32_t *__restrict__ mask_words, uint8_t *__restrict__ mask_bool)
{
    const int team = seat & 1;
    uint64_t *srcset = lscr, *edst = lscr + 3;
    if (l < 3) srcset[l] = 0;
    BB occ, ea;
    env_boards(cell, team, occ, ea);
    // lanes p and p + 32 share piece p (p < 30), one half of its moves each
    const int h = l >> 5, p = l & 31;
    bool mov = false, eng = false;
    int src = -1, ridx = -1, sc = 0;
    uint64_t m0 = 0, m1 = 0, m2 = 0;
    if (!off && p < 30) {
        const int pid = seat * 30 + p;
        int t;
        if (lpos) {
            src = lpos[pid];
            t = ltype[pid];
        } else {
            const PieceRec r = S.piece[pc_idx(env, pid)];
            src = r.pos;
            t = r.ptype;
        }
        // the source cell's flags, compact index and rail index: one round of
        // independent table loads
        const int f = (unsigned)src < (unsigned)NC ? src : 0;
        const int fl = cT.cflags[f], fc = cT.f2c[f], fr = cT.railidx[f];
        mov = (unsigned)src < (unsigned)NC && t != T_JUNQI && t != T_DILEI && !(fl & CF_SH);
        if (mov) {
            eng = t == T_GONGB;
            sc = fc;
            ridx = fr;
            const BB m = piece_moves_half(sc, ridx, eng, h, occ, ea);
            m0 = m.w0; m1 = m.w1; m2 = m.w2;
        }
    }
    m0 |= (uint64_t)__shfl_xor((long long)m0, 32);
    m1 |= (uint64_t)__shfl_xor((long long)m1, 32);
    m2 |= (uint64_t)__shfl_xor((long long)m2, 32);
    // engineers on a rail, three at a time (a seat has at most three)
    uint64_t engs = __ballot(mov && eng && ridx >= 0 && h == 0);
    while (engs) {
        int lanes[3], sr[3], ne = 0;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            lanes[j] = engs ? __builtin_ctzll(engs) : 64;
            ne += engs ? 1 : 0;
            engs &= engs - 1;
            sr[j] = lanes[j] < 64 ? __builtin_amdgcn_readlane(ridx, lanes[j]) : -1;   // uniform lane
        }
        if (l < 9) edst[l] = 0;
        engineers_bb(ne, sr, occ, ea, edst);
        wave_sync();
#pragma unroll
        for (int j = 0; j < 3; ++j)
            if (p == lanes[j]) { m0 |= edst[3 * j]; m1 |= edst[3 * j + 1]; m2 |= edst[3 * j + 2]; }
        wave_sync();
    }
    const bool lead = mov && h == 0;   // the lane that reports piece p
    const int cnt = __popcll(m0) + __popcll(m1) + __popcll(m2);
    // rank of this piece's source cell among the movable pieces: the movable
    // sources below it in a 129-bit set (compact order is flat order)
    if (lead) atomicOr(reinterpret_cast<unsigned long long *>(&srcset[sc >> 6]), 1ull << (sc & 63));
    wave_sync();
    int rank = 0;
    if (lead) {
        const int w = sc >> 6;
        rank = __popcll(srcset[w] & ((1ull << (sc & 63)) - 1)) + (w > 0 ? __popcll(srcset[0]) : 0) +
               (w > 1 ? __popcll(srcset[1]) : 0);
    }
    const int nmov = __popcll(__ballot(lead));
    const int total = wave_sum(lead ? cnt : 0);
    if (lead) {
        LegalRec &G = S.lg[env];
        G.src[rank] = (int16_t)src;
        G.mask[rank][0] = m0; G.mask[rank][1] = m1; G.mask[rank][2] = m2;
    }
    // canonical compact mask bits (gpu_rollout.py:1220-1238 layout): the two
    // lanes of a piece take alternate destination bits
    if (mov && (mask_words || mask_bool)) {
        const int cs = rotl[sc] * NONB;
        const uint64_t half = h ? 0xAAAAAAAAAAAAAAAAull : 0x5555555555555555ull;
        uint64_t w[3] = {m0 & half, m1 & half, m2 & half};
        for (int q = 0; q < 3; ++q) {
            uint64_t x = w[q];
            while (x) {
                const int b = __builtin_ctzll(x) + 64 * q;
                x &= x - 1;
                const int bit = cs + rotl[b];
                atomicOr(&bits[bit >> 5], 1u << (bit & 31));
            }
        }
    }
    if (l == 0) {
        S.lg[env].n = nmov;
        S.lg[env].seat = seat;
        if (counts) counts[env] = total;
    }
    wave_sync();
    if (mask_words)
        for (int w = l; w < JQ_MASK_WORDS; w += 64) mask_words[(size_t)env * JQ_MASK_WORDS + w] = (int32_t)bits[w];
    if (mask_bool) {
        __builtin_amdgcn_s_setprio(0);
        uint8_t *row = mask_bool + (size_t)env * JQ_ACTION_DIM;
        // bytes until the first 16-byte boundary, then whole 16-byte chunks, then the tail
        const int mis = (int)((uintptr_t)row & 15);
        const int head = mis ? 16 - mis : 0;
        for (int i = l; i < head; i += 64) row[i] = (bits[i >> 5] >> (i & 31)) & 1;
        const int nchunks = (JQ_ACTION_DIM - head) / 16;
        for (int q = l; q < nchunks; q += 64) {
            const int i0 = head + q * 16;   // bits i0 .. i0 + 15 (word (i0 >> 5) + 1 <= 520)
            const uint32_t v = __builtin_amdgcn_alignbit(bits[(i0 >> 5) + 1], bits[i0 >> 5], i0 & 31);
            *reinterpret_cast<uint4 *>(row + i0) =
                make_uint4(nib_to_bytes(v), nib_to_bytes(v >> 4), nib_to_bytes(v >> 8), nib_to_bytes(v >> 12));
        }
        for (int i = head + nchunks * 16 + l; i < JQ_ACTION_DIM; i += 64) row[i] = (bits[i >> 5] >> (i & 31)) & 1;
    }}

__global__ __launch_bounds__(64) void k_legal(State S, const int8_t *__restrict__ acting,
                                              int32_t *__restrict__ counts, int32_t *__restrict__ mask_words,
                                              uint8_t *__restrict__ mask_bool)
{
    const int env = blockIdx.x, l = threadIdx.x;
    if (env >= S.n) return;
    __shared__ int8_t cell[CELL_STRIDE];
    __shared__ uint32_t bits[JQ_MASK_WORDS_PAD];
    __shared__ uint8_t rotl[NONB + 3];   // world compact -> canonical compact of the acting seat
    __shared__ uint64_t lscr[LSCR_WORDS];
    const EnvRec &E = S.env[env];
    const int seat = acting ? acting[env] : E.turn;
    const bool off = E.term || seat < 0 || seat > 3 || ((E.sdead >> (seat & 3)) & 1);
    for (int f = l; f < CELL_STRIDE; f += 64) cell[f] = f < NC ? S.cell[(size_t)env * CELL_STRIDE + f] : -1;
    // wave issue priority 2 through the legal pass, 0 for the bool rows'
    // stores (legal_body lowers it): a wave still computing gets issue slots
    // ahead of the waves that are storing rows (drop-in step at 32,768 games:
    // 2.486 -> 2.474 ms)
    __builtin_amdgcn_s_setprio(2);
    for (int w = l; w < JQ_MASK_WORDS_PAD; w += 64) bits[w] = 0;
    if (mask_words || mask_bool) {
        const int s4 = seat & 3;
        for (int c = l; c < NONB; c += 64) rotl[c] = cT.rotc[s4][c];
    }
    __syncthreads();
    legal_body(S, env, l, seat, off, cell, bits, rotl, nullptr, nullptr, lscr, counts, mask_words, mask_bool);
}

// Exclusive scan of counts into offsets (N+1); one 1024-thread block walks the
// array in tiles of 32768 (one tile at the usual batch sizes). Wave w scans the
// tile's 2048 counts from 2048 w on: lane l holds the four counts at 4 (64 k + l)
// for k < 8, so every 16-byte load and store of the wave covers one contiguous
// 1 KB; eight wave scans give the running sums, the 16 wave totals are scanned
// through LDS, and a carry runs between tiles. The carry is 64-bit: a total
// beyond INT32_MAX (offsets are int32, as the reference's) writes offsets[n] =
// -1, which the host reads as "does not fit" before any id is emitted.
constexpr int SCAN_THREADS = 1024, SCAN_CHUNKS = 8, SCAN_TILE = SCAN_THREADS * 4 * SCAN_CHUNKS;
__global__ __launch_bounds__(SCAN_THREADS) void k_scan(const int32_t *__restrict__ counts, int32_t *__restrict__ offsets,
                                                      int n)
{
    __shared__ int32_t wsum[SCAN_THREADS / 64];
    __shared__ int32_t tile_total;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const bool vec = ((reinterpret_cast<uintptr_t>(counts) | reinterpret_cast<uintptr_t>(offsets)) & 15) == 0;
    int64_t carry = 0;
    for (int base = 0; base < n; base += SCAN_TILE) {
        const int seg = base + w * 64 * 4 * SCAN_CHUNKS;
        int4 v[SCAN_CHUNKS];
        int excl[SCAN_CHUNKS];
        int segsum = 0;
#pragma unroll
        for (int k = 0; k < SCAN_CHUNKS; ++k) {
            const int i = seg + 4 * (64 * k + lane);
            if (vec && i + 4 <= n) {
                v[k] = *reinterpret_cast<const int4 *>(counts + i);
            } else {
                v[k].x = i < n ? counts[i] : 0;
                v[k].y = i + 1 < n ? counts[i + 1] : 0;
                v[k].z = i + 2 < n ? counts[i + 2] : 0;
                v[k].w = i + 3 < n ? counts[i + 3] : 0;
            }
        }
#pragma unroll
        for (int k = 0; k < SCAN_CHUNKS; ++k) {
            const int s4 = v[k].x + v[k].y + v[k].z + v[k].w;
            int incl = s4;
            for (int o = 1; o < 64; o <<= 1) { const int u = __shfl_up(incl, o); if (lane >= o) incl += u; }
            excl[k] = segsum + incl - s4;
            segsum += __builtin_amdgcn_readlane(incl, 63);
        }
        if (lane == 0) wsum[w] = segsum;
        __syncthreads();
        if (w == 0) {
            const int x = lane < SCAN_THREADS / 64 ? wsum[lane] : 0;
            int y = x;
            for (int o = 1; o < SCAN_THREADS / 64; o <<= 1) { const int u = __shfl_up(y, o); if (lane >= o) y += u; }
            if (lane < SCAN_THREADS / 64) wsum[lane] = y - x;   // exclusive wave prefix
            if (lane == SCAN_THREADS / 64 - 1) tile_total = y;
        }
        __syncthreads();
        const int64_t wbase = carry + wsum[w];   // a tile's sums fit int: 32,768 x JQ_MAX_LEGAL < 2^31
#pragma unroll
        for (int k = 0; k < SCAN_CHUNKS; ++k) {
            const int i = seg + 4 * (64 * k + lane);
            int4 o;
            o.x = (int)(wbase + excl[k]);
            o.y = o.x + v[k].x;
            o.z = o.y + v[k].y;
            o.w = o.z + v[k].z;
            if (vec && i + 4 <= n) {
                *reinterpret_cast<int4 *>(offsets + i) = o;
            } else {
                if (i < n) offsets[i] = o.x;
                if (i + 1 < n) offsets[i + 1] = o.y;
                if (i + 2 < n) offsets[i + 2] = o.z;
                if (i + 3 < n) offsets[i + 3] = o.w;
            }
        }
        carry += tile_total;
        __syncthreads();
    }
    if (t == 0) offsets[n] = carry > (int64_t)INT32_MAX ? -1 : (int)carry;
}

// Position of the k-th set bit (k < popcount) of a 64-bit word.
__device__ __forceinline__ int select64(uint64_t x, int k)
{
    int pos = 0;
#pragma unroll
    for (int width = 32; width >= 1; width >>= 1) {
        const int c = __popcll(x & ((1ull << width) - 1ull));
        if (k >= c) { k -= c; x >>= width; pos += width; }
    }
    return pos;
}

// Write each env's ids at its offset: pieces in ascending source order, each
// piece's destinations ascending (compact order = flat order). Two envs per
// wave: half h (lanes 32h .. 32h + 31) takes env 2 * block + h, which fits since
// a seat has at most 30 movable pieces. Lane j of a half produces ids j, j + 32,
// ...: it finds its piece from the running counts, the destination by selecting
// a bit of that piece's mask, and maps it to a flat cell through an LDS copy of
// the compact table.
__global__ __launch_bounds__(64) void k_emit(State S, const int32_t *__restrict__ offsets, int32_t *__restrict__ values,
                                             int64_t cap, int32_t *__restrict__ mask_words)
{
    const int l = threadIdx.x, h = l >> 5, p = l & 31;
    const int env = 2 * (int)blockIdx.x + h;
    const bool live = env < S.n;
    __shared__ int16_t c2f[NONB + 3];
    __shared__ int32_t start[2][33];   // per half: first id of each piece, start[n] = total
    // mask_words: the canonical mask of each half's env is built here, in LDS
    __shared__ uint32_t mbits[2][JQ_MASK_WORDS_PAD];
    __shared__ uint8_t rot[2][NONB + 3];   // world compact -> canonical compact of the env's acting seat
    for (int c = l; c < NONB; c += 64) c2f[c] = cT.c2f[c];
    const int n = live ? min((int)S.lg[env].n, 30) : 0;
    const int seat = live ? (S.lg[env].seat & 3) : 0;
    if (mask_words) {
        for (int w = p; w < JQ_MASK_WORDS_PAD; w += 32) mbits[h][w] = 0;
        for (int c = p; c < NONB; c += 32) rot[h][c] = cT.rotc[seat][c];
    }
    int cnt = 0, src = 0, csrc = 0;   // csrc: the source's canonical compact index
    uint64_t m0 = 0, m1 = 0, m2 = 0;
    if (p < n) {
        const LegalRec &G = S.lg[env];
        src = G.src[p];
        m0 = G.mask[p][0]; m1 = G.mask[p][1]; m2 = G.mask[p][2];
        cnt = __popcll(m0) + __popcll(m1) + __popcll(m2);
        if (mask_words) csrc = cT.canc[seat][src];
    }
    int incl = cnt;
    for (int o = 1; o < 32; o <<= 1) { const int v = __shfl_up(incl, o, 32); if (p >= o) incl += v; }
    if (p < n) start[h][p] = incl - cnt;
    const int total = __shfl(incl, 31, 32);
    if (p == 0) start[h][n] = total;
    const int base = live ? offsets[env] : 0;
    __syncthreads();
    // uniform trip count (the larger half's total): every lane takes the shuffles
    const int trips = max(__builtin_amdgcn_readlane(total, 0), __builtin_amdgcn_readlane(total, 32));
    for (int b = 0; b < trips; b += 32) {
        const int i = b + p;
        int j = 0;   // piece of id i: the last piece whose start is <= i
        for (int step = 16; step >= 1; step >>= 1)
            if (j + step < n && start[h][j + step] <= i) j += step;
        const uint64_t w0 = __shfl(m0, j, 32), w1 = __shfl(m1, j, 32), w2 = __shfl(m2, j, 32);
        const int s = __shfl(src, j, 32), cs = __shfl(csrc, j, 32);
        if (i < total) {
            const int k = i - start[h][j];
            const int c0 = __popcll(w0), c1 = __popcll(w1);
            const int c = k < c0 ? select64(w0, k)
                                 : k < c0 + c1 ? 64 + select64(w1, k - c0) : 128 + select64(w2, k - c0 - c1);
            if (base >= 0 && (int64_t)base + i < cap) values[base + i] = s * NC + c2f[c];
            if (mask_words) {   // canonical bit (rotated source) * 129 + (rotated destination)
                const int bit = cs * NONB + rot[h][c];
                atomicOr(&mbits[h][bit >> 5], 1u << (bit & 31));
            }
        }
    }
    if (mask_words) {
        __syncthreads();
        if (live)
            for (int w = p; w < JQ_MASK_WORDS; w += 32)
                stream_store(mask_words + (size_t)env * JQ_MASK_WORDS + w, (int32_t)mbits[h][w]);
    }
}

// ------------------------------------------------------------------ slot mask
// Per-piece 80-slot legal mask (game_state.cu:1964-2197) from the legal sets
// k_legal left in S.lg. Slots 0-3 are the road steps in table order, 4-7 the
// camp diagonals, 8 + dir*12 + k the k-th cell of a non-engineer's straight
// rail run (road neighbours of the source excepted, they sit in 0-3). The
// reference packs curve-rail destinations (56..67) and an engineer's rail
// destinations (8..79) contiguously in its BFS order, so those sections are a
// run of ones as long as the destinations the earlier slots leave over.
constexpr int JQ_SLOTS = 80;
constexpr int JQ_SLOT_ROW = NP * JQ_SLOTS;   // bytes per env

__device__ __forceinline__ void set_run(uint64_t &lo, uint32_t &hi, int a, int len)
{   // bits [a, a + len) of the 80-bit slot set, a + len <= 80
    if (len <= 0) return;
    const int e = a + len;
    if (a < 64) {
        const int n = (e < 64 ? e : 64) - a;
        lo |= (n == 64 ? ~0ull : ((1ull << n) - 1)) << a;
    }
    if (e > 64) {
        const int ha = a > 64 ? a - 64 : 0;
        hi |= ((1u << (e - 64 - ha)) - 1) << ha;
    }
}

__device__ __forceinline__ uint32_t nibble_bytes(uint32_t nib)
{   // 4 bits -> 4 bytes of 0 / 1
    return (nib * 0x00204081u) & 0x01010101u;
}

__global__ __launch_bounds__(64) void k_slots(State S, uint8_t *__restrict__ out)
{
    const int env = blockIdx.x, l = threadIdx.x;
    if (env >= S.n) return;
    __shared__ uint4 rows[30][JQ_SLOTS / 16];   // the acting seat's 30 piece rows
    const LegalRec &G = S.lg[env];
    const int n = G.n, seat = G.seat;
    for (int q = l; q < 30 * (JQ_SLOTS / 16); q += 64) rows[q / 5][q % 5] = make_uint4(0, 0, 0, 0);
    __syncthreads();
    const int src = l < n ? G.src[l] : -1;
    const int pid = (unsigned)src < (unsigned)NC ? S.cell[(size_t)env * CELL_STRIDE + src] : -1;
    if (l < n && (unsigned)(pid - seat * 30) < 30u) {   // a consistent state always passes
        const BB M{G.mask[l][0], G.mask[l][1], G.mask[l][2]};
        const bool eng = S.piece[pc_idx(env, pid)].ptype == T_GONGB;
        uint64_t lo = 0;
        uint32_t hi = 0;
        int a[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            a[k] = cT.adj[src][k];
            if (a[k] >= 0 && bb_has(M, cT.f2c[a[k]])) lo |= 1ull << k;
            const int d = cT.diag[src][k];
            if (d >= 0 && bb_has(M, cT.f2c[d])) lo |= 1ull << (4 + k);
        }
        const int total = __popcll(M.w0) + __popcll(M.w1) + __popcll(M.w2);
        const int r = cT.railidx[src];
        if (r >= 0 && !eng) {
            for (int d = 0; d < 4; ++d)
                for (int k = 0; k < cT.raylen[r][d]; ++k) {
                    const int f = cT.rays[r][d][k];
                    if (f != a[0] && f != a[1] && f != a[2] && f != a[3] && bb_has(M, cT.f2c[f]))
                        lo |= 1ull << (8 + d * 12 + k);
                }
            const int rest = total - __popcll(lo);
            set_run(lo, hi, 56, rest < 12 ? rest : 12);
        } else if (r >= 0) {
            const int rest = total - __popcll(lo);
            set_run(lo, hi, 8, rest < 72 ? rest : 72);
        }
        uint4 *row = rows[pid - seat * 30];
#pragma unroll
        for (int j = 0; j < JQ_SLOTS / 16; ++j) {
            const uint32_t b = j < 4 ? (uint32_t)(lo >> (16 * j)) & 0xFFFFu : hi & 0xFFFFu;
            row[j] = make_uint4(nibble_bytes(b & 0xF), nibble_bytes((b >> 4) & 0xF),
                                nibble_bytes((b >> 8) & 0xF), nibble_bytes(b >> 12));
        }
    }
    __syncthreads();
    uint4 *dst = reinterpret_cast<uint4 *>(out + (size_t)env * JQ_SLOT_ROW);
    for (int q = l; q < JQ_SLOT_ROW / 16; q += 64) {
        const int p = q / 5 - seat * 30;
        dst[q] = (n > 0 && (unsigned)p < 30u) ? rows[p][q % 5] : make_uint4(0, 0, 0, 0);
    }
}

// ------------------------------------------------------------------ sampler
__device__ __forceinline__ uint32_t philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                                 uint32_t k0, uint32_t k1)
{   // Philox4x32-10 (Salmon et al., SC'11); returns the first output word
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0, hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        c0 = hi1 ^ c1 ^ k0; c1 = lo1; c2 = hi0 ^ c3 ^ k1; c3 = lo0;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
    return c0;
}

// Uniform pick from env's CSR row of c ids at offset off: Philox4x32-10 word 0
// of counter (env, ply lo, ply hi, 0) under key (seed lo, seed hi), scaled to
// the count; -1 for an empty row or one that does not lie inside the values
// buffer.
__device__ __forceinline__ int32_t uniform_pick(int env, int c, int64_t off, const int32_t *__restrict__ values,
                                                int64_t cap, uint64_t seed, uint64_t ply)
{
    if (c <= 0 || off < 0 || off + c > cap) return -1;
    const uint32_t u = philox4x32_10((uint32_t)env, (uint32_t)ply, (uint32_t)(ply >> 32), 0u,
                                     (uint32_t)seed, (uint32_t)(seed >> 32));
    return values[off + (int)(((uint64_t)u * (uint64_t)c) >> 32)];
}

// One env per thread.
__global__ void k_sample(int n, const int32_t *__restrict__ counts, const int32_t *__restrict__ offsets,
                         const int32_t *__restrict__ values, int64_t cap, uint64_t seed, uint64_t ply,
                         int32_t *__restrict__ out)
{
    const int env = blockIdx.x * blockDim.x + threadIdx.x;
    if (env >= n) return;
    out[env] = uniform_pick(env, counts[env], offsets[env], values, cap, seed, ply);
}

// Masked-logit pick by env's wave (lane l): the legal ids of the CSR row, lane
// j taking ids j, j + 64, ...; each id's canonical id c under `seat` draws
// u_c = Philox word 0 of counter (env, ply lo, ply hi, 1 + c). The N(0,1) logit
// Phi^-1((u_c + 1/2) / 2^32) is increasing in u_c, so the argmax over the row is
// the largest u_c, ties to the smallest c: one 64-bit key (u_c, ~c) per lane,
// maximised across the wave. Returns the world id (wave-uniform, -1 for an
// empty or out-of-buffer row) and its canonical id in `canon`.
// `c` and `off` are the env's CSR count and offset (wave-uniform).
__device__ __forceinline__ int32_t sample_logits_wave(int env, int l, int seat, int c, int64_t off,
                                                      const int32_t *__restrict__ values, int64_t cap, uint64_t seed,
                                                      uint64_t ply, int &canon)
{
    canon = -1;
    if (c <= 0 || seat < 0 || seat > 3) return -1;
    if (off < 0 || off + c > cap) return -1;
    uint64_t best = 0;
    int32_t bw = -1;
    for (int j = l; j < c; j += 64) {
        const int32_t w = values[off + j];
        const int src = w / NC, dst = w - src * NC;
        const int cc = (int)cT.canc[seat][src] * NONB + (int)cT.canc[seat][dst];
        const uint32_t u = philox4x32_10((uint32_t)env, (uint32_t)ply, (uint32_t)(ply >> 32), (uint32_t)(1 + cc),
                                         (uint32_t)seed, (uint32_t)(seed >> 32));
        const uint64_t key = ((uint64_t)u << 32) | (uint32_t)~(uint32_t)cc;   // > 0 for every real id
        if (key > best) { best = key; bw = w; }
    }
    const uint64_t m = wave_max(best);
    const uint64_t who = __ballot(best == m && bw >= 0);
    const int src_lane = who ? __builtin_ctzll(who) : 0;
    canon = (int)~(uint32_t)(m & 0xFFFFFFFFu);
    return __builtin_amdgcn_readlane(bw, src_lane);   // src_lane is wave-uniform
}

__global__ __launch_bounds__(64) void k_sample_logits(State S, const int8_t *__restrict__ acting,
                                                      const int32_t *__restrict__ counts,
                                                      const int32_t *__restrict__ offsets,
                                                      const int32_t *__restrict__ values, int64_t cap, uint64_t seed,
                                                      uint64_t ply, int32_t *__restrict__ out,
                                                      int32_t *__restrict__ canon_out)
{
    const int env = blockIdx.x, l = threadIdx.x;
    if (env >= S.n) return;
    const int seat = acting ? acting[env] : S.env[env].turn;
    int32_t c = uniform_word_raw(counts + env), o = uniform_word_raw(offsets + env);
    pin_word(c);
    pin_word(o);
    int cc;
    const int32_t a = sample_logits_wave(env, l, seat, c, o, values, cap, seed, ply, cc);
    if (l == 0) {
        out[env] = a;
        if (canon_out) canon_out[env] = a >= 0 ? cc : -1;
    }
}

// One env-step's state work by one wave per env: the action (given, or the
// Philox pick of k_sample from the env's previous CSR row, read before this
// wave overwrites the env's count), the ply (k_step), the restart
// of a finished game from the setup pool (k_reset_terminated, if do_reset) and
// the legal sets of the next acting seat (k_legal with the current
// turn), on the board the wave keeps in LDS, with no global round trip between
// the three.
// One wave's board while it steps its env: the LDS that step_env, init_env and
// legal_body work on.
struct EnvLds {
    alignas(16) uint32_t bits[JQ_MASK_WORDS_PAD];
    StepRes res;   // the step's reports, parked here across the legal pass
    uint64_t lscr[LSCR_WORDS];
    int16_t pos[PID_STRIDE];
    int8_t ptype[PID_STRIDE];
    int8_t cell[CELL_STRIDE];
    uint8_t rotl[NONB + 3];
};

// Inputs of one env-step beyond the state: the action source (`actions`, else a
// Philox pick from the env's previous CSR row `offsets` / `values` with
// `counts`), the pool restart and the outputs.
struct EnvStepArgs {
    const int32_t *actions; int sampler; uint64_t sample_seed, ply; const int32_t *offsets, *values;
    int64_t values_cap; int32_t *actions_out; StepOut O; int do_reset; int64_t reset_seed;
    int32_t *counts, *mask_words;
};

// The env-step of `env` by one wave (lane l): sample its action, apply the ply,
// restart the env from the setup pool if it ended, then the next seat's legal
// sets and canonical mask, all on the board the wave keeps in E. It synchronises
// only its own wave (wave_sync), so it never waits on other waves of a block.
__device__ __forceinline__ void env_step_wave(const State &S, int env, int l, const EnvStepArgs &A, EnvLds &E)
{
    StepLoad ld;   // the ply's first loads go out before the sampler's
    step_load(S, env, l, ld);
    // the env record and the CSR count and offset in one batch of scalar loads:
    // one wait, then the sampler's only dependent load is its row of ids
    const int32_t *ew = reinterpret_cast<const int32_t *>(S.env + env);
    int32_t v[10];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = uniform_word_raw(ew + k);
    const bool sampled = !A.actions;
    v[8] = sampled ? uniform_word_raw(A.counts + env) : 0;
    v[9] = sampled ? uniform_word_raw(A.offsets + env) : 0;
#pragma unroll
    for (int k = 0; k < 10; ++k) pin_word(v[k]);
    EnvRec E0;
    __builtin_memcpy(&E0, v, sizeof E0);
    int32_t a;
    if (A.actions) {
        a = A.actions[env];
    } else if (A.sampler == 1) {
        int cc;
        a = sample_logits_wave(env, l, E0.turn, v[8], v[9], A.values, A.values_cap, A.sample_seed, A.ply, cc);
    } else {
        a = uniform_pick(env, v[8], v[9], A.values, A.values_cap, A.sample_seed, A.ply);
    }
    if (A.actions_out && l == 0) A.actions_out[env] = a;
    TurnAfter nx;
    {
        StepRes res;
        step_env(S, env, l, a, nullptr, 0, res, E.cell, E.pos, E.ptype, nx, &ld, &E0);
        if (l == 0) E.res = res;
    }
    wave_sync();
    if (A.do_reset && S.pool_size > 0 && nx.term) {
        init_env(S, env, S.pool + (size_t)reset_pool_index(env, A.reset_seed, S.pool_size) * NP, E.cell, E.pos,
                 E.ptype);
        nx.turn = 0; nx.term = false; nx.sdead = 0;
    }
    const int seat = nx.turn;
    const bool off = nx.term || seat < 0 || seat > 3 || ((nx.sdead >> (seat & 3)) & 1);
    if (A.mask_words) {
        for (int w = l; w < JQ_MASK_WORDS_PAD; w += 64) E.bits[w] = 0;
        for (int c = l; c < NONB; c += 64) E.rotl[c] = cT.rotc[seat & 3][c];
    }
    wave_sync();
    legal_body(S, env, l, seat, off, E.cell, E.bits, E.rotl, E.pos, E.ptype, E.lscr, A.counts, A.mask_words,
               nullptr);
    if (l == 0) write_step_res(A.O, env, E.res);   // the step's reports go out last
}

__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(7, 8))) void k_env_step(State S, EnvStepArgs A)
{
    const int env = blockIdx.x;
    if (env >= S.n) return;
    __shared__ EnvLds E;
    env_step_wave(S, env, threadIdx.x, A, E);
}


}  // namespace jq

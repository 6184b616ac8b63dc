/*
 * jq_oracle.c -- CPU restatement of the junqi_core rules. TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * this file, and only as the reference answer / the timed CPU baseline. It shares no
 * code with junqi_amd/ (the product).
 *
 * Citations are reference paths (file:line). The restated behaviour is that
 * of junqi_core/state.py::GameState.step_inplace plus the modules it calls.
 */
#include "jq_oracle.h"

#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define NC JQO_NC
#define NP JQO_NP

/* ======================================================================
 * Board topology (junqi_core/board.py:88-279, rail_topology.py:60-276,
 * _movegen_tables.py:101-467)
 * ====================================================================== */
static int8_t T_on[NC], T_rail[NC], T_camp[NC], T_sh[NC], T_ng[NC], T_curve[NC], T_arc[NC];
static int8_t T_owner[NC], T_sidx[NC];
static int16_t T_adj[NC][4];            /* +x,-x,+y,-y ; -1 none (_movegen_tables.py:155-171) */
static int16_t T_diag[NC][4]; static int T_ndiag[NC];  /* (_movegen_tables.py:180-199) */
static int16_t T_radj[NC][4]; static int T_nradj[NC];  /* sorted (rail_topology.py:200-250) */
static int16_t T_ray[NC][4][12]; static int T_nray[NC][4]; /* (_movegen_tables.py:219-283) */
static int16_t T_cnbr[NC][4]; static int T_ncnbr[NC];      /* (_movegen_tables.py:349-380) */
static int16_t T_f2c[NC], T_c2f[JQO_ONB];
static int T_inited = 0;

static const int8_t PIECE_COUNTS[14] = {0,0,1,3,2,1,1,2,2,2,2,3,3,3}; /* rules.py:131-144 */

static void seat_pos(int seat, int i, int *x, int *y)
{   /* board.py:88-102 */
    int col = i % 5, row = i / 5;
    switch (seat) {
    case 0: *x = 10 - col; *y = 11 + row; break;
    case 1: *x = 5 - row;  *y = 10 - col; break;
    case 2: *x = 6 + col;  *y = 5 - row;  break;
    default:*x = 11 + row; *y = 6 + col;  break;
    }
}
static int is_camp_idx(int i) { return i == 6 || i == 8 || i == 12 || i == 16 || i == 18; }
static int is_sh_idx(int i) { return i == 26 || i == 28; }

static void radj_add(int a, int b)
{
    for (int k = 0; k < T_nradj[a]; k++) if (T_radj[a][k] == b) return;
    T_radj[a][T_nradj[a]++] = (int16_t)b;
}

void jqo_init(void)
{
    if (T_inited) return;
    memset(T_owner, -1, sizeof T_owner); memset(T_sidx, -1, sizeof T_sidx);
    for (int s = 0; s < 4; s++)
        for (int i = 0; i < 30; i++) {
            int x, y; seat_pos(s, i, &x, &y);
            int f = y * 17 + x;
            T_on[f] = 1; T_owner[f] = (int8_t)s; T_sidx[f] = (int8_t)i;
            T_camp[f] = (int8_t)is_camp_idx(i); T_sh[f] = (int8_t)is_sh_idx(i);
            int row = i / 5, col = i % 5;
            T_rail[f] = (int8_t)(i < 25 && (row == 0 || row == 4 || col == 0 || col == 4));
        }
    for (int i = 0; i < 9; i++) {            /* board.py:105-109 */
        int x = 10 - (i % 3) * 2, y = 6 + (i / 3) * 2, f = y * 17 + x;
        T_on[f] = 1; T_rail[f] = 1; T_ng[f] = 1;
    }
    /* curve ids, last write wins (rail_topology.py:173-190) */
    for (int cid = 1; cid <= 4; cid++) {
        int sa = cid - 1, sb = cid % 4;
        for (int j = 0; j < 30; j++) if (j % 5 == 4) {
            int x, y; seat_pos(sa, j, &x, &y); T_curve[y * 17 + x] = (int8_t)cid;
            seat_pos(sb, j - 4, &x, &y); T_curve[y * 17 + x] = (int8_t)cid;
        }
    }
    /* rail adjacency (rail_topology.py:200-243) */
    static const int od[4][2] = {{1,0},{-1,0},{0,1},{0,-1}};
    for (int f = 0; f < NC; f++) if (T_rail[f]) {
        int x = f % 17, y = f / 17;
        for (int k = 0; k < 4; k++) {
            int nx = x + od[k][0], ny = y + od[k][1];
            if (nx < 0 || nx > 16 || ny < 0 || ny > 16) continue;
            int nf = ny * 17 + nx;
            if (T_rail[nf]) { radj_add(f, nf); radj_add(nf, f); }
        }
        if (T_ng[f]) for (int k = 0; k < 4; k++) {
            int nx = x + 2 * od[k][0], ny = y + 2 * od[k][1];
            if (nx < 0 || nx > 16 || ny < 0 || ny > 16) continue;
            int nf = ny * 17 + nx;
            if (T_ng[nf]) { radj_add(f, nf); radj_add(nf, f); }
        }
    }
    static const int spc[4][4] = {{10,11,11,10},{6,11,5,10},{6,5,5,6},{11,6,10,5}};
    for (int e = 0; e < 4; e++) {
        int a = spc[e][1] * 17 + spc[e][0], b = spc[e][3] * 17 + spc[e][2];
        radj_add(a, b); radj_add(b, a);
    }
    for (int f = 0; f < NC; f++)   /* sort ascending */
        for (int a = 0; a < T_nradj[f]; a++)
            for (int b = a + 1; b < T_nradj[f]; b++)
                if (T_radj[f][b] < T_radj[f][a]) { int16_t t = T_radj[f][a]; T_radj[f][a] = T_radj[f][b]; T_radj[f][b] = t; }
    /* arc cells: rail cells with a diagonal rail edge (rail_topology.py:253-276) */
    for (int f = 0; f < NC; f++)
        for (int k = 0; k < T_nradj[f]; k++) {
            int n = T_radj[f][k];
            if (abs(f % 17 - n % 17) == 1 && abs(f / 17 - n / 17) == 1) T_arc[f] = 1;
        }
    /* adjacency, diagonal-into-camp */
    static const int dd[4][2] = {{1,1},{1,-1},{-1,1},{-1,-1}};
    for (int f = 0; f < NC; f++) {
        int x = f % 17, y = f / 17;
        for (int k = 0; k < 4; k++) {
            T_adj[f][k] = -1;
            if (!T_on[f]) continue;
            int nx = x + od[k][0], ny = y + od[k][1];
            if (nx < 0 || nx > 16 || ny < 0 || ny > 16) continue;
            if (T_on[ny * 17 + nx]) T_adj[f][k] = (int16_t)(ny * 17 + nx);
        }
        T_ndiag[f] = 0;
        if (!T_on[f]) continue;
        for (int k = 0; k < 4; k++) {
            int nx = x + dd[k][0], ny = y + dd[k][1];
            if (nx < 0 || nx > 16 || ny < 0 || ny > 16) continue;
            int nf = ny * 17 + nx;
            if (!T_on[nf]) continue;
            if (T_camp[f] || T_camp[nf]) T_diag[f][T_ndiag[f]++] = (int16_t)nf;
        }
    }
    /* straight rail rays: graph walk along one axis (_movegen_tables.py:219-283) */
    for (int f = 0; f < NC; f++) {
        for (int k = 0; k < 4; k++) T_nray[f][k] = 0;
        if (!T_rail[f]) continue;
        int x = f % 17, y = f / 17;
        for (int k = 0; k < 4; k++) {
            int dx = od[k][0], dy = od[k][1];
            int px = x, py = y;
            for (;;) {
                int next = -1, pf = py * 17 + px;
                for (int a = 0; a < T_nradj[pf]; a++) {
                    int nb = T_radj[pf][a], nx = nb % 17, ny = nb / 17;
                    if (dx != 0) { if (ny != y || (nx - px) * dx <= 0) continue; }
                    else         { if (nx != x || (ny - py) * dy <= 0) continue; }
                    if (nb == f) continue;
                    next = nb;
                }
                if (next < 0) break;
                T_ray[f][k][T_nray[f][k]++] = (int16_t)next;
                px = next % 17; py = next / 17;
            }
        }
    }
    /* curve neighbours: rail-graph neighbours with the same curve id */
    for (int f = 0; f < NC; f++) {
        T_ncnbr[f] = 0;
        if (!T_curve[f]) continue;
        for (int a = 0; a < T_nradj[f]; a++)
            if (T_curve[T_radj[f][a]] == T_curve[f]) T_cnbr[f][T_ncnbr[f]++] = T_radj[f][a];
    }
    int c = 0;
    for (int f = 0; f < NC; f++) { T_f2c[f] = -1; if (T_on[f]) { T_f2c[f] = (int16_t)c; T_c2f[c++] = (int16_t)f; } }
    T_inited = 1;
}

void jqo_tables_export(int8_t *on_board, int8_t *is_rail, int8_t *is_camp, int8_t *is_stronghold,
                       int8_t *is_ninegrid, int8_t *curve_id, int8_t *curve_arc,
                       int16_t *compact_to_flat, int16_t *rail_adj4)
{
    jqo_init();
    memcpy(on_board, T_on, NC); memcpy(is_rail, T_rail, NC); memcpy(is_camp, T_camp, NC);
    memcpy(is_stronghold, T_sh, NC); memcpy(is_ninegrid, T_ng, NC); memcpy(curve_id, T_curve, NC);
    memcpy(curve_arc, T_arc, NC);
    memcpy(compact_to_flat, T_c2f, sizeof T_c2f);
    for (int f = 0; f < NC; f++)
        for (int k = 0; k < 4; k++) rail_adj4[f * 4 + k] = k < T_nradj[f] ? T_radj[f][k] : -1;
}

/* ======================================================================
 * Rotation into an acting seat's canonical frame (junqi_core/rotation.py:44-80)
 * and seat-local placement (board.py:88-102)
 * ====================================================================== */
void jqo_world_to_canonical(int x, int y, int seat, int *cx, int *cy)
{
    switch (seat & 3) {
    case 0: *cx = x; *cy = y; break;                 /* SOUTH: identity */
    case 1: *cx = y; *cy = 16 - x; break;            /* WEST: +90 deg */
    case 2: *cx = 16 - x; *cy = 16 - y; break;       /* NORTH: 180 deg */
    default: *cx = 16 - y; *cy = x; break;           /* EAST: -90 deg */
    }
}

void jqo_canonical_to_world(int cx, int cy, int seat, int *x, int *y)
{
    switch (seat & 3) {
    case 0: *x = cx; *y = cy; break;
    case 1: *x = 16 - cy; *y = cx; break;
    case 2: *x = 16 - cx; *y = 16 - cy; break;
    default: *x = cy; *y = 16 - cx; break;
    }
}

void jqo_index_to_pos(int seat, int i, int *x, int *y) { seat_pos(seat & 3, i, x, y); }

int jqo_canonical_id(int seat, int world_id)
{   /* compact canonical action id of `seat` (junqi_rl/action_lut.py:62-170) */
    int src = world_id / NC, dst = world_id % NC, a[2] = {src, dst}, c[2];
    for (int q = 0; q < 2; q++) {
        int cx, cy;
        jqo_world_to_canonical(a[q] % 17, a[q] / 17, seat, &cx, &cy);
        c[q] = T_f2c[cy * 17 + cx];
    }
    return c[0] * JQO_ONB + c[1];
}

/* ======================================================================
 * CPython random.Random (stdlib): MT19937 init_by_array, getrandbits,
 * _randbelow_with_getrandbits, shuffle, choice.
 * ====================================================================== */
static void mt_init_genrand(jqo_mt *r, uint32_t s)
{
    r->mt[0] = s;
    for (int i = 1; i < 624; i++)
        r->mt[i] = 1812433253u * (r->mt[i - 1] ^ (r->mt[i - 1] >> 30)) + (uint32_t)i;
    r->idx = 624;
}

void jqo_mt_seed(jqo_mt *r, uint64_t seed)
{
    uint32_t key[2]; int klen;
    key[0] = (uint32_t)seed; key[1] = (uint32_t)(seed >> 32);
    klen = (seed >> 32) ? 2 : 1;
    mt_init_genrand(r, 19650218u);
    int i = 1, j = 0;
    for (int k = 624 > klen ? 624 : klen; k; k--) {
        r->mt[i] = (r->mt[i] ^ ((r->mt[i - 1] ^ (r->mt[i - 1] >> 30)) * 1664525u)) + key[j] + (uint32_t)j;
        i++; j++;
        if (i >= 624) { r->mt[0] = r->mt[623]; i = 1; }
        if (j >= klen) j = 0;
    }
    for (int k = 623; k; k--) {
        r->mt[i] = (r->mt[i] ^ ((r->mt[i - 1] ^ (r->mt[i - 1] >> 30)) * 1566083941u)) - (uint32_t)i;
        i++;
        if (i >= 624) { r->mt[0] = r->mt[623]; i = 1; }
    }
    r->mt[0] = 0x80000000u;
    r->idx = 624;
}

uint32_t jqo_mt_u32(jqo_mt *r)
{
    uint32_t y;
    if (r->idx >= 624) {
        int kk;
        for (kk = 0; kk < 624 - 397; kk++) {
            y = (r->mt[kk] & 0x80000000u) | (r->mt[kk + 1] & 0x7fffffffu);
            r->mt[kk] = r->mt[kk + 397] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
        }
        for (; kk < 623; kk++) {
            y = (r->mt[kk] & 0x80000000u) | (r->mt[kk + 1] & 0x7fffffffu);
            r->mt[kk] = r->mt[kk + (397 - 624)] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
        }
        y = (r->mt[623] & 0x80000000u) | (r->mt[0] & 0x7fffffffu);
        r->mt[623] = r->mt[396] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
        r->idx = 0;
    }
    y = r->mt[r->idx++];
    y ^= (y >> 11);
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= (y >> 18);
    return y;
}

uint32_t jqo_mt_randbelow(jqo_mt *r, uint32_t n)
{
    int k = 0; while ((n >> k) != 0 && k < 32) k++;   /* n.bit_length() */
    uint32_t v;
    do { v = jqo_mt_u32(r) >> (32 - k); } while (v >= n);
    return v;
}

static void shuffle_i8(jqo_mt *r, int8_t *a, int n)
{
    for (int i = n - 1; i >= 1; i--) {
        int j = (int)jqo_mt_randbelow(r, (uint32_t)(i + 1));
        int8_t t = a[i]; a[i] = a[j]; a[j] = t;
    }
}

void jqo_random_lineup(jqo_mt *r, int8_t lineup[30])
{   /* junqi_core/setup.py:162-250 */
    int flag_slot = jqo_mt_randbelow(r, 2) ? 28 : 26;
    int8_t freeS[30]; int nf = 0;
    for (int i = 0; i < 30; i++) if (!is_camp_idx(i) && i != flag_slot) freeS[nf++] = (int8_t)i;
    shuffle_i8(r, freeS, nf);
    int8_t dv[30], zv[30]; int nd = 0, nz = 0;
    for (int i = 0; i < nf; i++) { if (freeS[i] >= 20) dv[nd++] = freeS[i]; if (freeS[i] >= 5) zv[nz++] = freeS[i]; }
    int8_t place[30]; for (int i = 0; i < 30; i++) place[i] = -1;
    place[flag_slot] = JQO_JUNQI;
    uint8_t used[30] = {0};
    shuffle_i8(r, dv, nd);
    for (int i = 0; i < 3; i++) { place[dv[i]] = JQO_DILEI; used[dv[i]] = 1; }
    int8_t zv2[30]; int nz2 = 0;
    for (int i = 0; i < nz; i++) if (!used[zv[i]]) zv2[nz2++] = zv[i];
    shuffle_i8(r, zv2, nz2);
    for (int i = 0; i < 2; i++) { place[zv2[i]] = JQO_ZHADAN; used[zv2[i]] = 1; }
    int8_t rs[30]; int nr = 0;
    for (int i = 0; i < nf; i++) if (!used[freeS[i]]) rs[nr++] = freeS[i];
    shuffle_i8(r, rs, nr);
    int8_t rp[30]; int np_ = 0;
    for (int t = JQO_SILING; t <= JQO_GONGB; t++)
        for (int c = 0; c < PIECE_COUNTS[t]; c++) rp[np_++] = (int8_t)t;
    shuffle_i8(r, rp, np_);
    for (int i = 0; i < nr; i++) place[rs[i]] = rp[i];
    for (int i = 0; i < 30; i++) lineup[i] = is_camp_idx(i) ? JQO_NONE : place[i];
}

void jqo_random_setup(uint64_t seed, int8_t setup[120])
{
    jqo_mt r; jqo_mt_seed(&r, seed);
    for (int s = 0; s < 4; s++) jqo_random_lineup(&r, setup + 30 * s);
}

void jqo_setup_pool(uint64_t seed, int32_t pool_size, int8_t *pool)
{   /* junqi_rl/gpu_rollout.py:255-275: one shared stream over the whole pool */
    jqo_mt r; jqo_mt_seed(&r, seed);
    for (int p = 0; p < pool_size; p++)
        for (int s = 0; s < 4; s++) jqo_random_lineup(&r, pool + (size_t)p * 120 + 30 * s);
}

/* validate_lineup (junqi_core/setup.py:60-136): violation bits of one seat's
 * 30-entry lineup, 0 when it satisfies C1-C5. A value that is not a PieceType
 * (0..13) is a TYPE violation and stops the check, as PieceType(int(p)) raising
 * does there. */
int jqo_validate_lineup(const int8_t lu[30])
{
    int v = 0, cnt[14] = {0}, nflag = 0, flag_i = -1;
    for (int i = 0; i < 30; i++) if (lu[i] < 0 || lu[i] > JQO_GONGB) return JQO_V_TYPE;
    for (int i = 0; i < 30; i++) {
        int t = lu[i];
        cnt[t]++;
        if (is_camp_idx(i) && t != JQO_NONE) v |= JQO_V_C1;
        if (t == JQO_JUNQI) { nflag++; flag_i = i; }
        if (t == JQO_DILEI && i < 20) v |= JQO_V_C3;        /* BACK_TWO_ROWS = 20..29 */
        if (t == JQO_ZHADAN && i < 5) v |= JQO_V_C4;        /* FRONT_ROW = 0..4 */
    }
    if (nflag != 1 || !is_sh_idx(flag_i)) v |= JQO_V_C2;
    if (cnt[JQO_NONE] != 5) v |= JQO_V_C5;
    for (int t = JQO_JUNQI; t <= JQO_GONGB; t++) if (cnt[t] != PIECE_COUNTS[t]) v |= JQO_V_C5;
    if (cnt[JQO_DARK] != 0) v |= JQO_V_C5;
    return v;
}

/* ======================================================================
 * numpy SeedSequence + PCG64 (third-party, numpy>=1.26; restated from the
 * published algorithm) -> Zobrist tables (junqi_core/_zobrist.py:80-106)
 * ====================================================================== */
static uint32_t ss_hashmix(uint32_t v, uint32_t *hc)
{
    v ^= *hc; *hc *= 0x931e8875u; v *= *hc; v ^= v >> 16; return v;
}
static uint32_t ss_mix(uint32_t x, uint32_t y)
{
    uint32_t r = 0xca01f9ddu * x - 0x4973f715u * y; r ^= r >> 16; return r;
}

void jqo_seedseq_state(uint64_t entropy, uint32_t out8[8])
{
    uint32_t ent[2]; int ne;
    ent[0] = (uint32_t)entropy; ent[1] = (uint32_t)(entropy >> 32);
    ne = (entropy >> 32) ? 2 : 1;
    uint32_t pool[4], hc = 0x43b0d7e5u;
    for (int i = 0; i < 4; i++) pool[i] = ss_hashmix(i < ne ? ent[i] : 0u, &hc);
    for (int s = 0; s < 4; s++)
        for (int d = 0; d < 4; d++)
            if (s != d) pool[d] = ss_mix(pool[d], ss_hashmix(pool[s], &hc));
    uint32_t hb = 0x8b51f9ddu;
    for (int i = 0; i < 8; i++) {
        uint32_t v = pool[i % 4];
        v ^= hb; hb *= 0x58f38dedu; v *= hb; v ^= v >> 16;
        out8[i] = v;
    }
}

typedef unsigned __int128 u128;
void jqo_pcg64_draw(uint64_t seed, int64_t n, uint64_t *out)
{
    uint32_t w[8]; jqo_seedseq_state(seed, w);
    uint64_t v[4];
    for (int i = 0; i < 4; i++) v[i] = (uint64_t)w[2 * i] | ((uint64_t)w[2 * i + 1] << 32);
    u128 initstate = ((u128)v[0] << 64) | v[1];
    u128 initseq = ((u128)v[2] << 64) | v[3];
    const u128 mult = ((u128)0x2360ed051fc65da4ULL << 64) | 0x4385df649fccf645ULL;
    u128 inc = (initseq << 1) | 1u, st = 0;
    st = st * mult + inc; st += initstate; st = st * mult + inc;
    for (int64_t i = 0; i < n; i++) {
        st = st * mult + inc;
        uint64_t hi = (uint64_t)(st >> 64), lo = (uint64_t)st;
        unsigned rot = (unsigned)(st >> 122);
        uint64_t x = hi ^ lo;
        out[i] = (x >> rot) | (x << ((64 - rot) & 63));
    }
}

#define ZN_PIECE (120L * 14 * 289)
#define ZOFF_TURN (ZN_PIECE)
#define ZOFF_MC (ZOFF_TURN + 4)
#define ZOFF_MSLC (ZOFF_MC + 4096)
#define ZOFF_TERM (ZOFF_MSLC + 512)
#define ZOFF_WIN (ZOFF_TERM + 1)
#define ZOFF_DRAW (ZOFF_WIN + 3)
#define ZOFF_SDEAD (ZOFF_DRAW + 1)
#define ZOFF_SFLAG (ZOFF_SDEAD + 4)
#define ZOFF_SHOW (ZOFF_SFLAG + 4)
#define ZTOTAL (ZOFF_SHOW + 4)
static uint64_t *Z = NULL;

static void zob_build(void)
{
    if (Z) return;
    uint64_t *t = (uint64_t *)malloc(sizeof(uint64_t) * ZTOTAL);
    jqo_pcg64_draw(0x4A554E51495F5A4FULL, ZTOTAL, t);
    Z = t;
}
int64_t jqo_zobrist_count(void) { return ZTOTAL; }
const uint64_t *jqo_zobrist_all(void) { zob_build(); return Z; }
#define ZP(pid, t, f) Z[((long)(pid) * 14 + (t)) * 289 + (f)]

/* ======================================================================
 * Recency LUT: float32 exp(-e/tau), tau in {32,256,64,128} plane order,
 * exactly as numpy produced it (observation.py:1552-1567); loaded from the
 * committed fixture.
 * ====================================================================== */
static float RLUT[4][4096];
void jqo_set_recency_lut(const float *lut) { memcpy(RLUT, lut, sizeof RLUT); }

/* ======================================================================
 * Move generation
 * ====================================================================== */
static int team_of_pid(const jqo_game *g, int pid) { return g->pseat[pid] & 1; }
static int occupied(const jqo_game *g, int f) { return g->cell_pid[f] >= 0; }
static int enemy_att(const jqo_game *g, int f, int team)
{   /* move_gen.py:822-867: enemy piece on a non-camp cell */
    int p = g->cell_pid[f];
    return p >= 0 && team_of_pid(g, p) != team && !T_camp[f];
}
static int landable(const jqo_game *g, int f, int team) { return !occupied(g, f) || enemy_att(g, f, team); }

/* Engineer BFS (move_gen.py:870-895). Appends dsts to out. */
static int eng_dests(const jqo_game *g, int src, int team, int16_t *out)
{
    uint8_t vis[NC] = {0}; int16_t q[NC]; int qh = 0, qt = 0, n = 0;
    vis[src] = 1; q[qt++] = (int16_t)src;
    while (qh < qt) {
        int cur = q[qh++];
        for (int a = 0; a < T_nradj[cur]; a++) {
            int nb = T_radj[cur][a];
            if (vis[nb]) continue;
            vis[nb] = 1;
            if (!occupied(g, nb)) { out[n++] = (int16_t)nb; q[qt++] = (int16_t)nb; }
            else if (enemy_att(g, nb, team)) out[n++] = (int16_t)nb;
        }
    }
    return n;
}

/* Curve-rail BFS (move_gen.py:898-920). */
static int curve_dests(const jqo_game *g, int src, int team, int16_t *out)
{
    uint8_t vis[NC] = {0}; int16_t q[NC]; int qh = 0, qt = 0, n = 0;
    vis[src] = 1; q[qt++] = (int16_t)src;
    while (qh < qt) {
        int cur = q[qh++];
        for (int a = 0; a < T_ncnbr[cur]; a++) {
            int nb = T_cnbr[cur][a];
            if (vis[nb]) continue;
            vis[nb] = 1;
            if (!occupied(g, nb)) { out[n++] = (int16_t)nb; q[qt++] = (int16_t)nb; }
            else if (enemy_att(g, nb, team)) out[n++] = (int16_t)nb;
        }
    }
    return n;
}

static int cmp_i32(const void *a, const void *b)
{
    int32_t x = *(const int32_t *)a, y = *(const int32_t *)b; return (x > y) - (x < y);
}

/* Legal action ids for `seat`, sorted unique (move_gen.py:1052-1199). */
static int legal_ids_raw(const jqo_game *g, int seat, int32_t *ids)
{
    int n = 0, team = seat & 1;
    int16_t buf[NC * 2];
    for (int pid = 0; pid < NP; pid++) {
        if (!g->alive[pid] || g->pseat[pid] != seat) continue;
        int t = g->ptype[pid];
        if (t == JQO_JUNQI || t == JQO_DILEI) continue;
        if (g->pos_x[pid] < 0 || g->pos_y[pid] < 0) continue;
        int src = g->pos_y[pid] * 17 + g->pos_x[pid];
        if (T_sh[src]) continue;
        for (int k = 0; k < 4; k++) { int nb = T_adj[src][k]; if (nb >= 0 && landable(g, nb, team)) ids[n++] = src * NC + nb; }
        for (int k = 0; k < T_ndiag[src]; k++) { int nb = T_diag[src][k]; if (landable(g, nb, team)) ids[n++] = src * NC + nb; }
        if (T_rail[src]) {
            if (t == JQO_GONGB) {
                int m = eng_dests(g, src, team, buf);
                for (int i = 0; i < m; i++) ids[n++] = src * NC + buf[i];
            } else {
                for (int k = 0; k < 4; k++)
                    for (int i = 0; i < T_nray[src][k]; i++) {
                        int nb = T_ray[src][k][i];
                        if (!occupied(g, nb)) { ids[n++] = src * NC + nb; continue; }
                        if (enemy_att(g, nb, team)) ids[n++] = src * NC + nb;
                        break;
                    }
            }
        }
        if (T_curve[src] && t != JQO_GONGB) {
            int m = curve_dests(g, src, team, buf);
            for (int i = 0; i < m; i++) ids[n++] = src * NC + buf[i];
        }
    }
    qsort(ids, (size_t)n, sizeof(int32_t), cmp_i32);
    int u = 0;
    for (int i = 0; i < n; i++) if (u == 0 || ids[i] != ids[u - 1]) ids[u++] = ids[i];
    return u;
}

int jqo_legal_ids(const jqo_game *g, int seat, int32_t *out, int cap)
{   /* state.py:1200-1213: empty for a dead seat or a finished game */
    if (g->seat_dead[seat] || g->terminated) return 0;
    int32_t tmp[8192];
    int n = legal_ids_raw(g, seat, tmp);
    if (n > cap) return -n;
    memcpy(out, tmp, sizeof(int32_t) * (size_t)n);
    return n;
}

int jqo_has_legal(const jqo_game *g, int seat)
{
    int32_t tmp[8192];
    return legal_ids_raw(g, seat, tmp) > 0;
}

/* Rail BFS from src over the sorted rail graph, visiting each cell once; a
 * cell that passes `keep` is enqueued when empty. Destinations that are
 * landable and not filtered out by `skip` go to slots [*cur, end).
 * (game_state.cu:2077-2124 with keep = same curve, skip = same axis;
 *  game_state.cu:2150-2195 with keep = all, skip = road neighbour of src) */
static void slot_bfs(const jqo_game *g, int src, int team, int curve_only, uint8_t *row, int *cur, int end)
{
    uint8_t vis[NC] = {0}; int16_t q[NC]; int qh = 0, qt = 0;
    const int sx = src % 17, sy = src / 17;
    vis[src] = 1; q[qt++] = (int16_t)src;
    while (qh < qt) {
        int c = q[qh++];
        for (int a = 0; a < T_nradj[c]; a++) {
            int nb = T_radj[c][a];
            if (vis[nb]) continue;
            vis[nb] = 1;
            if (curve_only && T_curve[nb] != T_curve[src]) continue;
            int skip;
            if (curve_only) skip = (nb % 17 == sx) || (nb / 17 == sy);
            else skip = nb == T_adj[src][0] || nb == T_adj[src][1] || nb == T_adj[src][2] || nb == T_adj[src][3];
            if (!occupied(g, nb)) {
                if (!skip && *cur < end) row[(*cur)++] = 1;
                q[qt++] = (int16_t)nb;
            } else if (!skip && *cur < end && enemy_att(g, nb, team)) {
                row[(*cur)++] = 1;
            }
        }
    }
}

int jqo_legal_slots(const jqo_game *g, int seat, uint8_t *out)
{
    memset(out, 0, (size_t)NP * JQO_SLOTS);
    if (seat < 0 || seat > 3 || g->seat_dead[seat] || g->terminated) return 0;
    const int team = seat & 1;
    int total = 0;
    for (int pid = 0; pid < NP; pid++) {   /* game_state.cu:2005-2018 gate */
        if (!g->alive[pid] || g->pseat[pid] != seat) continue;
        int t = g->ptype[pid];
        if (t == JQO_JUNQI || t == JQO_DILEI) continue;
        if (g->pos_x[pid] < 0 || g->pos_y[pid] < 0) continue;
        int src = g->pos_y[pid] * 17 + g->pos_x[pid];
        if (!T_on[src] || T_sh[src]) continue;
        uint8_t *row = out + (size_t)pid * JQO_SLOTS;
        for (int k = 0; k < 4; k++) {   /* game_state.cu:2032-2043 */
            int nb = T_adj[src][k];
            if (nb >= 0 && landable(g, nb, team)) row[k] = 1;
        }
        for (int k = 0; k < T_ndiag[src]; k++)
            if (landable(g, T_diag[src][k], team)) row[4 + k] = 1;
        if (T_rail[src]) {
            if (t != JQO_GONGB) {   /* game_state.cu:2055-2075 */
                for (int d = 0; d < 4; d++)
                    for (int k = 0; k < T_nray[src][d]; k++) {
                        int nb = T_ray[src][d][k];
                        int ortho = nb == T_adj[src][0] || nb == T_adj[src][1] || nb == T_adj[src][2] || nb == T_adj[src][3];
                        if (!occupied(g, nb)) { if (!ortho) row[8 + d * 12 + k] = 1; continue; }
                        if (!ortho && enemy_att(g, nb, team)) row[8 + d * 12 + k] = 1;
                        break;
                    }
                if (T_curve[src] > 0) { int cur = 56; slot_bfs(g, src, team, 1, row, &cur, 68); }
            } else {
                int cur = 8; slot_bfs(g, src, team, 0, row, &cur, JQO_SLOTS);
            }
        }
        for (int s = 0; s < JQO_SLOTS; s++) total += row[s];
    }
    return total;
}

/* ---- legacy pairwise predicates (move_gen.py:127-376) ---- */
static int straight_rail_clear(const jqo_game *g, int src, int dst)
{   /* move_gen.py:127-171 */
    if (src == dst) return 0;
    int sx = src % 17, sy = src / 17, dx = dst % 17, dy = dst / 17;
    if (sx != dx && sy != dy) return 0;
    uint8_t vis[NC] = {0}; int16_t q[NC]; int qh = 0, qt = 0;
    vis[src] = 1; q[qt++] = (int16_t)src;
    while (qh < qt) {
        int cur = q[qh++];
        for (int a = 0; a < T_nradj[cur]; a++) {
            int nb = T_radj[cur][a];
            if (vis[nb]) continue;
            int nx = nb % 17, ny = nb / 17;
            if (sx == dx && nx != sx) continue;
            if (sy == dy && ny != sy) continue;
            if (nb == dst) return 1;
            if (occupied(g, nb)) continue;
            vis[nb] = 1; q[qt++] = (int16_t)nb;
        }
    }
    return 0;
}

static int same_curve(int a, int b) { return T_curve[a] > 0 && T_curve[a] == T_curve[b]; }

static int curve_rail_clear(const jqo_game *g, int src, int dst)
{   /* move_gen.py:384-423 */
    int cid = T_curve[src];
    if (T_curve[dst] != cid) return 0;
    uint8_t vis[NC] = {0}; int16_t q[NC]; int qh = 0, qt = 0;
    vis[src] = 1; q[qt++] = (int16_t)src;
    while (qh < qt) {
        int cur = q[qh++];
        for (int a = 0; a < T_nradj[cur]; a++) {
            int nb = T_radj[cur][a];
            if (vis[nb] || T_curve[nb] != cid) continue;
            if (nb == dst) return 1;
            if (occupied(g, nb)) continue;
            vis[nb] = 1; q[qt++] = (int16_t)nb;
        }
    }
    return 0;
}

static int engineer_can_reach(const jqo_game *g, int src, int dst)
{   /* move_gen.py:186-224 */
    if (!T_rail[src] || !T_rail[dst] || src == dst) return 0;
    uint8_t vis[NC] = {0}; int16_t q[NC]; int qh = 0, qt = 0;
    vis[src] = 1; q[qt++] = (int16_t)src;
    while (qh < qt) {
        int cur = q[qh++];
        for (int a = 0; a < T_nradj[cur]; a++) {
            int nb = T_radj[cur][a];
            if (vis[nb]) continue;
            if (nb == dst) return 1;
            if (occupied(g, nb)) continue;
            vis[nb] = 1; q[qt++] = (int16_t)nb;
        }
    }
    return 0;
}

int jqo_is_legal(const jqo_game *g, int seat, int src, int dst)
{   /* move_gen.py:299-376 */
    if (src < 0 || src >= NC || dst < 0 || dst >= NC) return 0;
    if (!T_on[src] || !T_on[dst] || src == dst) return 0;
    int p = g->cell_pid[src];
    if (p < 0 || g->pseat[p] != seat) return 0;
    int t = g->ptype[p];
    if (t == JQO_JUNQI || t == JQO_DILEI) return 0;
    if (T_sh[src]) return 0;
    if (!landable(g, dst, seat & 1)) return 0;
    int sx = src % 17, sy = src / 17, dx = dst % 17, dy = dst / 17;
    int adx = abs(sx - dx), ady = abs(sy - dy);
    if (adx <= 1 && ady <= 1) {
        if (adx == 1 && ady == 1) { if (T_camp[src] || T_camp[dst]) return 1; }
        else return 1;
    }
    if (!(T_rail[src] && T_rail[dst])) return 0;
    if (t == JQO_GONGB) return engineer_can_reach(g, src, dst);
    if (sx == dx || sy == dy) return straight_rail_clear(g, src, dst);
    if (same_curve(src, dst)) return curve_rail_clear(g, src, dst);
    return 0;
}

int jqo_move_requires_gongb(const jqo_game *g, int src, int dst)
{   /* move_gen.py:245-296 */
    int sx = src % 17, sy = src / 17, dx = dst % 17, dy = dst / 17;
    if (src == dst) return 0;
    int adx = abs(sx - dx), ady = abs(sy - dy);
    if (adx + ady == 1) return 0;
    if (adx == 1 && ady == 1 && (T_camp[src] || T_camp[dst])) return 0;
    if (!(T_rail[src] && T_rail[dst])) return 0;
    if (sx == dx || sy == dy) {
        if (straight_rail_clear(g, src, dst)) return 0;
        return engineer_can_reach(g, src, dst);
    }
    if (same_curve(src, dst) && curve_rail_clear(g, src, dst)) return 0;
    return engineer_can_reach(g, src, dst);
}

/* ======================================================================
 * Combat (rules.py:466-539)
 * ====================================================================== */
static int resolve_combat(int a, int d)
{
    if (a == JQO_ZHADAN || d == JQO_ZHADAN) return JQO_EV_BOMB;
    if (d == JQO_JUNQI) return JQO_EV_EAT;
    if (d == JQO_DILEI) return a == JQO_GONGB ? JQO_EV_EAT : JQO_EV_KILLED;
    if (a == d) return JQO_EV_BOMB;
    return a < d ? JQO_EV_EAT : JQO_EV_KILLED;
}

/* ======================================================================
 * Belief codes (info_model.py:115-138, 141-145, 218-265)
 * ====================================================================== */
#define BC_ONEHOT(ti) ((uint8_t)(1 + (ti)))
#define BC_PRIOR(slot) ((uint8_t)(16 + (slot)))
#define BC_UNIFORM ((uint8_t)64)
static int tracked_idx(int t) { return (t >= 2 && t <= 13) ? t - 2 : -1; }
static int code_is_onehot(int c) { return c >= 1 && c <= 12; }

static void prior_row(int slot, float out[12])
{   /* info_model.py:69-132: p[t] proportional to count over admissible types */
    float v[12]; for (int i = 0; i < 12; i++) v[i] = 0.f;
    if (!is_camp_idx(slot)) {
        for (int t = 2; t <= 13; t++) {
            int ok;
            if (is_sh_idx(slot)) ok = 1;
            else if (t == JQO_JUNQI) ok = 0;
            else if (t == JQO_DILEI) ok = slot >= 20;
            else if (t == JQO_ZHADAN) ok = slot >= 5;
            else ok = 1;
            if (ok) v[t - 2] = (float)PIECE_COUNTS[t];
        }
    }
    float s = 0.f; for (int i = 0; i < 12; i++) s += v[i];
    for (int i = 0; i < 12; i++) out[i] = s > 0.f ? v[i] / s : 0.f;
}

void jqo_belief_row(int code, float out[12])
{
    for (int i = 0; i < 12; i++) out[i] = 0.f;
    if (code >= 1 && code <= 12) out[code - 1] = 1.f;
    else if (code >= 16 && code < 46) prior_row(code - 16, out);
    else if (code == BC_UNIFORM) for (int i = 0; i < 12; i++) out[i] = (float)(1.0 / 12.0);
}

static int sees_truth(int obs, int owner, int mode)
{   /* info_model.py:568-577 */
    if (mode == JQO_BRIGHT) return 1;
    if (obs == owner) return 1;
    return mode == JQO_HALF_DARK && ((obs & 1) == (owner & 1));
}

static int local_index(int seat, int f)
{
    for (int i = 0; i < 30; i++) { int x, y; seat_pos(seat, i, &x, &y); if (y * 17 + x == f) return i; }
    return -1;
}

static void belief_initial(jqo_game *g)
{   /* info_model.py:218-265, for each of the 4 observers */
    for (int o = 0; o < 4; o++) {
        for (int pid = 0; pid < NP; pid++) {
            g->bcode[o][pid] = 0;
            if (!g->alive[pid]) continue;
            int s = g->pseat[pid], f = g->pos_y[pid] * 17 + g->pos_x[pid];
            if (sees_truth(o, s, g->show_mode)) g->bcode[o][pid] = BC_ONEHOT(tracked_idx(g->ptype[pid]));
            else {
                int li = local_index(s, f);
                g->bcode[o][pid] = li < 0 ? BC_UNIFORM : BC_PRIOR(li);
            }
        }
        for (int s = 0; s < 4; s++) {
            g->rem_tracked[o][s] = (int8_t)(s != o && (s & 1) != (o & 1));
            for (int t = 0; t < 12; t++) g->rem[o][s][t] = g->rem_tracked[o][s] ? PIECE_COUNTS[t + 2] : 0;
        }
    }
}

static void rem_dec(jqo_game *g, int o, int seat, int ti)
{   /* info_model.py:490-495 */
    if (!g->rem_tracked[o][seat]) return;
    if (g->rem[o][seat][ti] > 0) g->rem[o][seat][ti]--;
}
static void on_removed(jqo_game *g, int o, int seat, int code)
{   /* info_model.py:474-488 */
    if (!g->rem_tracked[o][seat]) return;
    if (code_is_onehot(code)) rem_dec(g, o, seat, code - 1);
}

/* BeliefTensor.update for every observer (info_model.py:271-429), pid-keyed:
 * an entry follows its piece, so migration is implicit. */
static void belief_update(jqo_game *g, int src_pid, int dst_pid, int src_seat, int dst_seat,
                          int dst_type, int dst_cell, int event, int rev_src, int rev_dst,
                          int flag_captured, int died_mask)
{
    for (int o = 0; o < 4; o++) {
        int acode = g->bcode[o][src_pid];
        int dcode = dst_pid >= 0 ? g->bcode[o][dst_pid] : 0;
        if (rev_src) rem_dec(g, o, src_seat, JQO_SILING - 2);
        if (rev_dst) rem_dec(g, o, dst_seat, JQO_SILING - 2);
        if (event == JQO_EV_EAT && dst_pid >= 0 && dst_type == JQO_DILEI && !code_is_onehot(acode)) {
            acode = BC_ONEHOT(JQO_GONGB - 2);
            g->bcode[o][src_pid] = (uint8_t)acode;
            rem_dec(g, o, src_seat, JQO_GONGB - 2);
        }
        if (flag_captured) {
            g->rem_tracked[o][dst_seat] = 0;
        } else if (event == JQO_EV_EAT && dst_pid >= 0 && T_sh[dst_cell] && T_owner[dst_cell] == dst_seat) {
            /* R6: the other stronghold of the defender's seat holds the flag */
            int other = -1;
            for (int i = 26; i <= 28; i += 2) { int x, y; seat_pos(dst_seat, i, &x, &y); if (y * 17 + x != dst_cell) other = y * 17 + x; }
            int op = g->cell_pid[other];  /* board before the step */
            if (op >= 0 && !code_is_onehot(g->bcode[o][op])) g->bcode[o][op] = BC_ONEHOT(JQO_JUNQI - 2);
        }
        if (event == JQO_EV_EAT) {
            if (dst_pid >= 0) on_removed(g, o, dst_seat, dcode);
        } else if (event == JQO_EV_KILLED) {
            on_removed(g, o, src_seat, acode);
        } else if (event == JQO_EV_BOMB) {
            on_removed(g, o, src_seat, acode);
            if (dst_pid >= 0) on_removed(g, o, dst_seat, dcode);
        }
        for (int s = 0; s < 4; s++) if (died_mask & (1 << s)) g->rem_tracked[o][s] = 0;
    }
}

/* ======================================================================
 * CombatMemory (combat_memory.py:339-569)
 * ====================================================================== */
static void pid_bit(int pid, uint64_t *lo, uint64_t *hi)
{
    if (pid < 64) *lo |= 1ULL << pid; else *hi |= 1ULL << (pid - 64);
}
static int rank_of(int t)
{   /* ORDINARY_RANKS (combat_memory.py:139-160): GONGB=1 .. SILING=9 */
    return (t >= JQO_SILING && t <= JQO_GONGB) ? (JQO_GONGB - t + 1) : 0;
}
static int next_floor(int t) { int r = rank_of(t); if (r == 0) return 0; return r + 1 < 9 ? r + 1 : 9; }

static void cm_apply(jqo_game *g, int is_eat, int apid, int dpid, int aseat, int dseat,
                     int atype, int dtype, int step)
{
    int K, V, Vs, Vt;
    if (is_eat) { K = apid; V = dpid; Vs = dseat; Vt = dtype; }
    else        { K = dpid; V = apid; Vs = aseat; Vt = atype; }
    if (K < 0 || V < 0) return;
    int vi = tracked_idx(Vt);
    if (!is_eat) {
        for (int o = 0; o < 4; o++) {
            int known = g->cm_is_gongb[o][V] || (atype == JQO_GONGB && o == Vs);
            if (known) g->cm_atk_gongb[o][K] = 1;
        }
    }
    for (int o = 0; o < 4; o++) {
        g->cm_chain_lo[o][K] |= g->cm_direct_lo[o][V] | g->cm_chain_lo[o][V];
        g->cm_chain_hi[o][K] |= g->cm_direct_hi[o][V] | g->cm_chain_hi[o][V];
        pid_bit(V, &g->cm_chain_lo[o][K], &g->cm_chain_hi[o][K]);
        g->cm_chain_type[o][K] |= (uint16_t)(g->cm_direct_type[o][V] | g->cm_chain_type[o][V]);
        g->cm_last_chain[o][K] = (int16_t)step;
        int vf = g->cm_floor[o][V];
        if (vf > 0) {
            int prop = vf + 1 < 9 ? vf + 1 : 9;
            if (prop > g->cm_floor[o][K]) { g->cm_floor[o][K] = (int8_t)prop; g->cm_floor_step[o][K] = (int16_t)step; }
            g->cm_not_gongb[o][K] = 1;
        }
    }
    for (int o = 0; o < 4; o++) {   /* v6 reverse projection */
        uint64_t mlo = 0, mhi = 0;
        for (int s = 0; s < 30; s++) pid_bit(o * 30 + s, &mlo, &mhi);
        uint64_t vlo = (g->cm_direct_lo[o][V] | g->cm_chain_lo[o][V]) & mlo;
        uint64_t vhi = (g->cm_direct_hi[o][V] | g->cm_chain_hi[o][V]) & mhi;
        if (Vs == o) pid_bit(V, &vlo, &vhi);
        for (int b = 0; b < 64; b++) {
            if (vlo >> b & 1) pid_bit(K, &g->cm_eaten_lo[o][b], &g->cm_eaten_hi[o][b]);
            if (vhi >> b & 1) pid_bit(K, &g->cm_eaten_lo[o][64 + b], &g->cm_eaten_hi[o][64 + b]);
        }
    }
    for (int o = 0; o < 4; o++) {
        if (Vs != o) {
            int c = g->cm_other_cnt[o][K] + 1; g->cm_other_cnt[o][K] = (int16_t)(c < 32767 ? c : 32767);
            g->cm_last_direct[o][K] = (int16_t)step;
            continue;
        }
        pid_bit(V, &g->cm_direct_lo[o][K], &g->cm_direct_hi[o][K]);
        if (vi >= 0) {
            g->cm_direct_type[o][K] |= (uint16_t)(1u << vi);
            g->cm_chain_type[o][K] |= (uint16_t)(1u << vi);
        }
        g->cm_last_direct[o][K] = (int16_t)step;
        if (is_eat) {
            if (Vt == JQO_DILEI) g->cm_is_gongb[o][K] = 1; else g->cm_not_gongb[o][K] = 1;
        } else if (Vt >= JQO_SILING && Vt <= JQO_GONGB) {
            int pr = next_floor(Vt);
            if (pr > g->cm_floor[o][K]) { g->cm_floor[o][K] = (int8_t)pr; g->cm_floor_step[o][K] = (int16_t)step; }
        }
        if (is_eat && Vt >= JQO_SILING && Vt <= JQO_GONGB) {
            int pr = next_floor(Vt);
            if (pr > g->cm_floor[o][K]) { g->cm_floor[o][K] = (int8_t)pr; g->cm_floor_step[o][K] = (int16_t)step; }
        }
    }
}

/* apply_combat_event (combat_memory.py:354-569) and apply_path_revealed_gongb
 * (combat_memory.py:339-351) on a game's combat memory, for hand-built cases.
 * The defender's cell argument of the reference is not read by the update. */
void jqo_cm_apply_event(jqo_game *g, int is_eat, int apid, int dpid, int aseat, int dseat, int atype, int dtype,
                        int step)
{
    cm_apply(g, is_eat, apid, dpid, aseat, dseat, atype, dtype, step);
}

void jqo_cm_path_revealed_gongb(jqo_game *g, int pid)
{
    for (int o = 0; o < 4; o++) g->cm_is_gongb[o][pid] = 1;
}

/* ======================================================================
 * GameState construction (state.py:490-620, 346-483)
 * ====================================================================== */
static void game_blank(jqo_game *g, int show_mode, int max_num_moves)
{
    memset(g, 0, sizeof *g);
    memset(g->ptype, -1, sizeof g->ptype); memset(g->pseat, -1, sizeof g->pseat);
    memset(g->pos_x, -1, sizeof g->pos_x); memset(g->pos_y, -1, sizeof g->pos_y);
    memset(g->zero_x, -1, sizeof g->zero_x); memset(g->zero_y, -1, sizeof g->zero_y);
    memset(g->death_reason, -1, sizeof g->death_reason);
    for (int i = 0; i < NP; i++) { g->death_step[i] = -1; g->death_loc[i] = -1; }
    for (int f = 0; f < NC; f++) g->cell_pid[f] = -1;
    for (int o = 0; o < 4; o++) for (int p = 0; p < NP; p++) {
        g->cm_last_direct[o][p] = -1; g->cm_last_chain[o][p] = -1; g->cm_floor_step[o][p] = -1;
    }
    g->winner = -1; g->show_mode = (int8_t)show_mode; g->max_num_moves = max_num_moves;
}

uint64_t jqo_recompute_zobrist(const jqo_game *g)
{   /* state.py:1761-1811 */
    zob_build();
    uint64_t h = 0;
    for (int pid = 0; pid < NP; pid++) {
        if (!g->alive[pid] || g->ptype[pid] < 0) continue;
        h ^= ZP(pid, g->ptype[pid], g->pos_y[pid] * 17 + g->pos_x[pid]);
    }
    h ^= Z[ZOFF_TURN + g->turn];
    h ^= Z[ZOFF_MC + (g->move_counter & 0xFFF)];
    h ^= Z[ZOFF_MSLC + (g->mslc & 0x1FF)];
    h ^= Z[ZOFF_WIN + (g->winner < 0 ? 0 : g->winner + 1)];
    h ^= Z[ZOFF_SHOW + g->show_mode];
    if (g->terminated) h ^= Z[ZOFF_TERM];
    if (g->draw) h ^= Z[ZOFF_DRAW];
    for (int s = 0; s < 4; s++) {
        if (g->seat_dead[s]) h ^= Z[ZOFF_SDEAD + s];
        if (g->flag_rev[s]) h ^= Z[ZOFF_SFLAG + s];
    }
    return h;
}

int jqo_new_game(jqo_game *g, const int8_t setup[120], int show_mode, int max_num_moves)
{
    jqo_init(); zob_build();
    game_blank(g, show_mode, max_num_moves);
    for (int s = 0; s < 4; s++)
        for (int i = 0; i < 30; i++) {
            int t = setup[s * 30 + i];
            if (t == JQO_NONE) continue;
            int pid = s * 30 + i, x, y; seat_pos(s, i, &x, &y);
            g->alive[pid] = 1; g->ptype[pid] = (int8_t)t; g->pseat[pid] = (int8_t)s;
            g->pos_x[pid] = g->zero_x[pid] = (int8_t)x; g->pos_y[pid] = g->zero_y[pid] = (int8_t)y;
            g->cell_pid[y * 17 + x] = (int16_t)pid;
        }
    g->zobrist = jqo_recompute_zobrist(g);
    belief_initial(g);
    return 0;
}

int jqo_from_pieces(jqo_game *g, int n, const int32_t *pc, int turn, int move_counter, int mslc,
                    const int8_t seat_dead[4], const int8_t flag_rev[4], int show_mode, int max_num_moves)
{   /* hand-built positions (state.py:346-483): no zero board, counters zero */
    jqo_init(); zob_build();
    game_blank(g, show_mode, max_num_moves);
    for (int i = 0; i < n; i++) {
        int pid = pc[4 * i], t = pc[4 * i + 1], x = pc[4 * i + 2], y = pc[4 * i + 3];
        if (pid < 0 || pid >= NP || x < 0 || x > 16 || y < 0 || y > 16) return -1;
        if (g->cell_pid[y * 17 + x] >= 0 || g->alive[pid]) return -2;
        g->alive[pid] = 1; g->ptype[pid] = (int8_t)t; g->pseat[pid] = (int8_t)(pid / 30);
        g->pos_x[pid] = (int8_t)x; g->pos_y[pid] = (int8_t)y;
        g->cell_pid[y * 17 + x] = (int16_t)pid;
    }
    g->turn = (int8_t)turn; g->move_counter = move_counter; g->mslc = mslc;
    for (int s = 0; s < 4; s++) { g->seat_dead[s] = seat_dead[s]; g->flag_rev[s] = flag_rev[s]; }
    g->zobrist = jqo_recompute_zobrist(g);
    belief_initial(g);
    return 0;
}

/* ======================================================================
 * step_inplace (state.py:638-998)
 * ====================================================================== */
static void soa_move(jqo_game *g, int pid, int src, int dst)
{   /* state.py:1005-1025 */
    int t = g->ptype[pid];
    g->zobrist ^= ZP(pid, t, src) ^ ZP(pid, t, dst);
    g->cell_pid[src] = -1; g->cell_pid[dst] = (int16_t)pid;
    g->pos_x[pid] = (int8_t)(dst % 17); g->pos_y[pid] = (int8_t)(dst / 17);
}
static void soa_kill(jqo_game *g, int pid, int reason, int loc, int step)
{   /* state.py:1027-1049 */
    if (!g->alive[pid]) return;
    int cur = g->pos_y[pid] * 17 + g->pos_x[pid];
    g->zobrist ^= ZP(pid, g->ptype[pid], cur);
    g->cell_pid[cur] = -1; g->alive[pid] = 0; g->pos_x[pid] = -1; g->pos_y[pid] = -1;
    g->death_reason[pid] = (int8_t)reason; g->death_step[pid] = (int16_t)step; g->death_loc[pid] = (int16_t)loc;
}
static void set_dead(jqo_game *g, int s) { if (!g->seat_dead[s]) { g->seat_dead[s] = 1; g->zobrist ^= Z[ZOFF_SDEAD + s]; } }
static void set_flag(jqo_game *g, int s) { if (!g->flag_rev[s]) { g->flag_rev[s] = 1; g->zobrist ^= Z[ZOFF_SFLAG + s]; } }
static void purge_seat(jqo_game *g, int s, int step)
{   /* state.py:1639-1692 + 1051-1086: KILLED_BY_ENEMY at the piece's current cell */
    for (int pid = 0; pid < NP; pid++)
        if (g->alive[pid] && g->pseat[pid] == s) {
            int cur = g->pos_y[pid] * 17 + g->pos_x[pid];
            soa_kill(g, pid, 0, cur, step);
        }
}
static int seat_has_piece(const jqo_game *g, int s)
{
    for (int pid = 0; pid < NP; pid++) if (g->alive[pid] && g->pseat[pid] == s) return 1;
    return 0;
}
static void check_victory(const jqo_game *g, int attacker, int mc, int mslc, int *term, int *win, int *draw)
{   /* state.py:1695-1726 */
    int red = !(g->seat_dead[0] && g->seat_dead[2]);
    int blue = !(g->seat_dead[1] && g->seat_dead[3]);
    *term = 0; *win = -1; *draw = 0;
    if (!red && !blue) { *term = 1; *win = attacker & 1; return; }
    if (!red) { *term = 1; *win = 1; return; }
    if (!blue) { *term = 1; *win = 0; return; }
    if (mc >= 4000 || mslc >= 200) { *term = 1; *draw = 1; }
}

int jqo_step(jqo_game *g, int src, int dst, jqo_result *res)
{
    memset(res, 0, sizeof *res);
    res->winner = g->winner; res->terminated = g->terminated; res->draw = g->draw;
    if (g->terminated) return -1;
    int seat = g->turn;
    if (g->seat_dead[seat]) return -2;
    if (!jqo_is_legal(g, seat, src, dst)) return -3;

    if (g->hist_len == 32) { memmove(g->hist[0], g->hist[1], sizeof(int16_t) * 2 * 31); g->hist_len = 31; }
    g->hist[g->hist_len][0] = (int16_t)src; g->hist[g->hist_len][1] = (int16_t)dst; g->hist_len++;

    uint64_t zout = Z[ZOFF_TURN + g->turn] ^ Z[ZOFF_MC + (g->move_counter & 0xFFF)] ^ Z[ZOFF_MSLC + (g->mslc & 0x1FF)];
    int step = g->move_counter + 1, died = 0;
    int sp = g->cell_pid[src], dp = g->cell_pid[dst];
    int st = g->ptype[sp], dt = dp >= 0 ? g->ptype[dp] : -1;
    int ss = g->pseat[sp], ds = dp >= 0 ? g->pseat[dp] : -1;

    if (st == JQO_GONGB && jqo_move_requires_gongb(g, src, dst)) {
        for (int o = 0; o < 4; o++) g->cm_is_gongb[o][sp] = 1;
        res->gongb_revealed = 1;
    }
    int ev, rsrc = 0, rdst = 0, fcap = 0;
    if (dp < 0) {
        ev = JQO_EV_MOVE;
        g->move_count[sp]++;
        soa_move(g, sp, src, dst);
    } else {
        ev = resolve_combat(st, dt);
        rsrc = st == JQO_SILING && (ev == JQO_EV_KILLED || ev == JQO_EV_BOMB);
        rdst = dt == JQO_SILING && (ev == JQO_EV_EAT || ev == JQO_EV_BOMB);
        fcap = dt == JQO_JUNQI;
        if (rsrc) set_flag(g, ss);
        if (rdst) set_flag(g, ds);
        if (ev == JQO_EV_EAT) {
            g->active_eat[sp]++;
            soa_kill(g, dp, 0, dst, step);
            soa_move(g, sp, src, dst);
            cm_apply(g, 1, sp, dp, ss, ds, st, dt, step);
        } else if (ev == JQO_EV_KILLED) {
            g->passive_surv[dp]++;
            soa_kill(g, sp, (dt == JQO_DILEI || dt == JQO_ZHADAN) ? 1 : 0, dst, step);
            cm_apply(g, 0, sp, dp, ss, ds, st, dt, step);
        } else {
            soa_kill(g, sp, 2, dst, step);
            soa_kill(g, dp, 2, dst, step);
        }
    }
    if (fcap && !g->seat_dead[ds]) {   /* state.py:864-890 */
        set_dead(g, ds); set_flag(g, ds);
        purge_seat(g, ds, step);
        died |= 1 << ds;
    }
    for (int s = 0; s < 4; s++)       /* state.py:895-901 */
        if (!g->seat_dead[s] && !seat_has_piece(g, s)) { set_dead(g, s); died |= 1 << s; }

    int nmc = g->move_counter + 1, nmslc = ev == JQO_EV_MOVE ? g->mslc + 1 : 0;
    int term, win, drw, nturn;
    check_victory(g, seat, nmc, nmslc, &term, &win, &drw);
    if (!term) {                        /* state.py:1109-1167 */
        int cand = (seat + 1) & 3;
        for (int it = 0; it < 4; it++) {
            if (g->seat_dead[cand]) { cand = (cand + 1) & 3; continue; }
            if (jqo_has_legal(g, cand)) break;
            set_dead(g, cand); purge_seat(g, cand, step); died |= 1 << cand;
            cand = (cand + 1) & 3;
        }
        nturn = cand;
        check_victory(g, seat, nmc, nmslc, &term, &win, &drw);
    } else nturn = g->turn;
    if (!term && nmc >= g->max_num_moves) { term = 1; drw = 1; }   /* env cap */

    g->move_counter = nmc; g->mslc = nmslc; g->turn = (int8_t)nturn;
    uint64_t zin = Z[ZOFF_TURN + nturn] ^ Z[ZOFF_MC + (nmc & 0xFFF)] ^ Z[ZOFF_MSLC + (nmslc & 0x1FF)];
    uint64_t zt = 0;
    if (term != g->terminated) zt ^= Z[ZOFF_TERM];
    if (drw != g->draw) zt ^= Z[ZOFF_DRAW];
    if (win != g->winner) zt ^= Z[ZOFF_WIN + (g->winner < 0 ? 0 : g->winner + 1)] ^ Z[ZOFF_WIN + (win < 0 ? 0 : win + 1)];
    g->terminated = (int8_t)term; g->winner = (int8_t)win; g->draw = (int8_t)drw;
    g->zobrist ^= zout ^ zin ^ zt;

    belief_update(g, sp, dp, ss, ds, dt, dst, ev, rsrc, rdst, fcap, died);

    res->valid = 1; res->event = ev; res->flag_reveal_src = rsrc; res->flag_reveal_dst = rdst;
    res->flag_captured = fcap; res->seats_died_mask = died;
    res->terminated = term; res->winner = win; res->draw = drw;
    return 0;
}

/* ======================================================================
 * Observation (observation.py:621-857, 908-1651)
 * World-frame planes, then rotation into the observer's canonical frame.
 * ====================================================================== */
static int slot_channel(int slot)
{   /* observation.py:272-284 */
    if (is_camp_idx(slot)) return -1;
    int c = 0; for (int i = 0; i < slot; i++) if (!is_camp_idx(i)) c++;
    return c;
}
static int popc64(uint64_t x) { return __builtin_popcountll(x); }
static int in_back_two(int seat, int zx, int zy)
{   /* observation.py:1376-1383 */
    switch (seat) {
    case 0: return zy >= 15 && zy <= 16;
    case 2: return zy >= 0 && zy <= 1;
    case 1: return zx >= 0 && zx <= 1;
    default: return zx >= 15 && zx <= 16;
    }
}

/* ext == NULL: belief planes from the BeliefTensor codes. Otherwise ext is the
 * observer's uploaded (12, 289) belief slice in world cells, read at each
 * teammate / enemy piece's cell where it is > 0 (the reference's uploaded-belief
 * path, src/env/cuda/src/observation.cu:246-372). */
static void observe_impl(const jqo_game *g, int obs, const float *ext, float *out, float *glob);

void jqo_observe(const jqo_game *g, int obs, float *out, float *glob) { observe_impl(g, obs, NULL, out, glob); }

void jqo_observe_ext(const jqo_game *g, int obs, const float *ext, float *out, float *glob)
{
    observe_impl(g, obs, ext, out, glob);
}

static void ext_row(const float *ext, int f, float out[12])
{
    for (int t = 0; t < 12; t++) out[t] = ext[t * NC + f] > 0.f ? ext[t * NC + f] : 0.f;
}

static void observe_impl(const jqo_game *g, int obs, const float *ext, float *out, float *glob)
{
    static const int CH_OWN = 0, CH_PTM = 12, CH_DTM = 24, CH_LE = 25, CH_RE = 26, CH_BL = 27, CH_BR = 39,
        CH_DEAD = 51, CH_FLAG = 54, CH_STATIC = 58, CH_TURN = 64, CH_MOVEB = 66, CH_EATB = 74, CH_SURVB = 82,
        CH_DREASON = 90, CH_DZERO = 102, CH_SLOT = 104, CH_HIST = 129, CH_KMT = 161, CH_KMGE = 173,
        CH_KOGE = 176, CH_CT = 179, CH_CGE = 191, CH_FLOOR = 194, CH_ISG = 203, CH_NOTG = 204, CH_DC = 205,
        CH_MYKC = 206, CH_MYISG = 209, CH_MYDC = 210, CH_KMC = 211, CH_KMS = 223, CH_REC = 253, CH_EAT = 257;
    float *w = (float *)calloc((size_t)JQO_OBS_C * NC, sizeof(float));
#define W(c, f) w[(size_t)(c) * NC + (f)]
    int tm = (obs + 2) & 3, le = (obs + 1) & 3, re = (obs + 3) & 3, team = obs & 1;
    int order[4] = {obs, tm, le, re};
    float brow[12];
    for (int pid = 0; pid < NP; pid++) {
        if (!g->alive[pid]) continue;
        int f = g->pos_y[pid] * 17 + g->pos_x[pid], s = g->pseat[pid], ti = tracked_idx(g->ptype[pid]);
        if (s == obs && ti >= 0) W(CH_OWN + ti, f) = 1.f;
        if (s == tm || s == le || s == re) {
            if (ext) ext_row(ext, f, brow);
            else jqo_belief_row(g->bcode[obs][pid], brow);
        }
        if (s == tm) for (int t = 0; t < 12; t++) W(CH_PTM + t, f) = brow[t];
        if (g->show_mode == JQO_DARKMODE && s == tm) W(CH_DTM, f) = 1.f;
        if (s == le) W(CH_LE, f) = 1.f;
        if (s == re) W(CH_RE, f) = 1.f;
        if (s == le) for (int t = 0; t < 12; t++) W(CH_BL + t, f) = brow[t];
        if (s == re) for (int t = 0; t < 12; t++) W(CH_BR + t, f) = brow[t];
        int ours = (s & 1) == team, half = ours ? 0 : 4;
        int mb = g->move_count[pid] < 3 ? g->move_count[pid] : 3;
        W(CH_MOVEB + half + mb, f) = 1.f;
        int eb = g->active_eat[pid] < 3 ? g->active_eat[pid] : 3;
        for (int k = 0; k <= eb; k++) W(CH_EATB + half + k, f) = 1.f;
        int sb = g->passive_surv[pid] < 3 ? g->passive_surv[pid] : 3;
        for (int k = 0; k <= sb; k++) W(CH_SURVB + half + k, f) = 1.f;
        int sc = slot_channel(pid % 30);
        W(CH_SLOT + (sc < 0 ? 24 : sc), f) = 1.f;   /* numpy's -1 index: last plane */
    }
    for (int k = 0; k < 3; k++) if (g->seat_dead[order[k + 1]]) for (int f = 0; f < NC; f++) W(CH_DEAD + k, f) = 1.f;
    for (int k = 0; k < 4; k++) if (g->flag_rev[order[k]]) for (int f = 0; f < NC; f++) W(CH_FLAG + k, f) = 1.f;
    for (int f = 0; f < NC; f++) {
        W(CH_STATIC + 0, f) = T_camp[f]; W(CH_STATIC + 1, f) = T_sh[f]; W(CH_STATIC + 2, f) = T_rail[f];
        W(CH_STATIC + 3, f) = T_ng[f]; W(CH_STATIC + 4, f) = T_arc[f];
    }
    {   /* turn history: float64 divide, clamp, round to float32 (observation.py:1000-1021) */
        double dp = (double)g->mslc / 200.0; if (dp > 1.0) dp = 1.0;
        double mp = (double)g->move_counter / 4000.0; if (mp > 1.0) mp = 1.0;
        for (int f = 0; f < NC; f++) { W(CH_TURN, f) = (float)dp; W(CH_TURN + 1, f) = (float)mp; }
    }
    for (int pid = 0; pid < NP; pid++) {     /* deaths: D and E groups */
        if (g->death_step[pid] < 0 && g->death_reason[pid] < 0) continue;
        if (g->alive[pid]) continue;
        int s = g->pseat[pid];
        if (g->death_reason[pid] >= 0 && g->death_step[pid] > 0 && g->death_loc[pid] >= 0) {
            int base = s == obs ? 0 : s == tm ? 3 : s == le ? 6 : s == re ? 9 : -1;
            if (base >= 0) W(CH_DREASON + base + g->death_reason[pid], g->death_loc[pid]) = 1.f;
        }
        if (g->zero_x[pid] >= 0 && g->zero_y[pid] >= 0)
            W(CH_DZERO + (((s & 1) == team) ? 0 : 1), g->zero_y[pid] * 17 + g->zero_x[pid]) = 1.f;
    }
    for (int d = 0; d < g->hist_len && d < 32; d++) {
        int e = g->hist_len - 1 - d;
        W(CH_HIST + d, g->hist[e][0]) = -1.f;
        W(CH_HIST + d, g->hist[e][1]) = 1.f;
    }
    /* combat memory layers 1-3 on enemy live pieces */
    int cur = g->move_counter;
    for (int pid = 0; pid < NP; pid++) {
        if (!g->alive[pid]) continue;
        int s = g->pseat[pid], f = g->pos_y[pid] * 17 + g->pos_x[pid];
        if ((s & 1) != team) {
            uint64_t dlo = g->cm_direct_lo[obs][pid], dhi = g->cm_direct_hi[obs][pid];
            int mc = popc64(dlo) + popc64(dhi);
            for (int k = 0; k < 3; k++) if (mc >= k + 1) W(CH_KMGE + k, f) = 1.f;
            for (int t = 0; t < 12; t++) if (g->cm_direct_type[obs][pid] >> t & 1) W(CH_KMT + t, f) = 1.f;
            for (int k = 0; k < 3; k++) if (g->cm_other_cnt[obs][pid] >= k + 1) W(CH_KOGE + k, f) = 1.f;
            int cc = popc64(g->cm_chain_lo[obs][pid]) + popc64(g->cm_chain_hi[obs][pid]);
            for (int k = 0; k < 3; k++) if (cc >= k + 1) W(CH_CGE + k, f) = 1.f;
            for (int t = 0; t < 12; t++) if (g->cm_chain_type[obs][pid] >> t & 1) W(CH_CT + t, f) = 1.f;
            for (int k = 0; k < 9; k++) if (g->cm_floor[obs][pid] >= k + 1) W(CH_FLOOR + k, f) = 1.f;
            if (g->cm_is_gongb[obs][pid]) W(CH_ISG, f) = 1.f;
            if (g->cm_not_gongb[obs][pid]) W(CH_NOTG, f) = 1.f;
            if (in_back_two(s, g->zero_x[pid], g->zero_y[pid]) && g->move_count[pid] == 0 && !g->cm_atk_gongb[obs][pid])
                W(CH_DC, f) = 1.f;
            /* layer 3 */
            int cnt_t[12] = {0};
            for (int sl = 0; sl < 30; sl++) {
                int gp = obs * 30 + sl;
                int hit = gp < 64 ? (int)(dlo >> gp & 1) : (int)(dhi >> (gp - 64) & 1);
                if (!hit) continue;
                W(CH_KMS + sl, f) = 1.f;
                int ti = g->ptype[gp] >= 0 ? tracked_idx(g->ptype[gp]) : -1;
                if (ti >= 0) cnt_t[ti]++;
            }
            for (int t = 0; t < 12; t++) if (cnt_t[t] > 0) {
                float v = (float)cnt_t[t] / 3.0f; W(CH_KMC + t, f) = v < 1.0f ? v : 1.0f;
            }
            int last[4] = {g->cm_last_direct[obs][pid], g->cm_last_direct[obs][pid], g->cm_last_chain[obs][pid], g->cm_floor_step[obs][pid]};
            for (int k = 0; k < 4; k++) {
                if (last[k] < 0) continue;
                int e = cur - last[k]; if (e < 0) e = 0; if (e > 4095) e = 4095;
                float v = RLUT[k][e];
                if (v > 0.f) W(CH_REC + k, f) = v;
            }
        } else if (s == obs) {
            /* layer 2 (observation.py:1392-1451) */
            int lo_ = (obs + 1) & 3, ro_ = (obs + 3) & 3;
            int lc = popc64(g->cm_direct_lo[lo_][pid]) + popc64(g->cm_direct_hi[lo_][pid]) + g->cm_other_cnt[lo_][pid];
            int rc = popc64(g->cm_direct_lo[ro_][pid]) + popc64(g->cm_direct_hi[ro_][pid]) + g->cm_other_cnt[ro_][pid];
            int pk = lc < rc ? lc : rc;
            for (int k = 0; k < 3; k++) if (pk >= k + 1) W(CH_MYKC + k, f) = 1.f;
            if (g->cm_is_gongb[lo_][pid] && g->cm_is_gongb[ro_][pid]) W(CH_MYISG, f) = 1.f;
            int atk = g->cm_atk_gongb[lo_][pid] || g->cm_atk_gongb[ro_][pid];
            if (in_back_two(s, g->zero_x[pid], g->zero_y[pid]) && g->move_count[pid] == 0 && !atk) W(CH_MYDC, f) = 1.f;
        }
    }
    /* layer 4: reverse projection on the observer's own 30 pids */
    for (int sl = 0; sl < 30; sl++) {
        int mp = obs * 30 + sl, px, py;
        if (g->alive[mp]) { px = g->pos_x[mp]; py = g->pos_y[mp]; } else { px = g->zero_x[mp]; py = g->zero_y[mp]; }
        if (px < 0 || py < 0) continue;
        int f = py * 17 + px;
        for (int half = 0; half < 2; half++) {
            int opp = half == 0 ? (obs + 1) & 3 : (obs + 3) & 3;
            for (int s = 0; s < 30; s++) {
                int gp = opp * 30 + s;
                int hit = gp < 64 ? (int)(g->cm_eaten_lo[obs][mp] >> gp & 1) : (int)(g->cm_eaten_hi[obs][mp] >> (gp - 64) & 1);
                if (hit) W(CH_EAT + half * 30 + s, f) = 1.f;
            }
        }
    }
    /* globals (observation.py:1623-1651) */
    for (int t = 0; t < 12; t++) {
        glob[t] = g->rem_tracked[obs][le] ? (float)g->rem[obs][le][t] : 0.f;
        glob[12 + t] = g->rem_tracked[obs][re] ? (float)g->rem[obs][re][t] : 0.f;
    }
    for (int k = 0; k < 4; k++) glob[24 + k] = (float)g->flag_rev[order[k]];
    /* rotate into the canonical frame (rotation.py:44-64, 112-149) */
    for (int c = 0; c < JQO_OBS_C; c++)
        for (int f = 0; f < NC; f++) {
            int cx, cy;
            jqo_world_to_canonical(f % 17, f / 17, obs, &cx, &cy);
            out[(size_t)c * NC + cy * 17 + cx] = W(c, f);
        }
#undef W
    free(w);
}

/* ======================================================================
 * Batch CPU path (the timed CPU baseline)
 * ====================================================================== */
int jqo_sizeof_game(void) { return (int)sizeof(jqo_game); }
int jqo_omp_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void jqo_batch_new(jqo_game *gs, int n, const int8_t *setups, int show_mode, int max_num_moves)
{
    jqo_init(); zob_build();
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; i++) jqo_new_game(&gs[i], setups + (size_t)i * 120, show_mode, max_num_moves);
}

long jqo_batch_env_step(jqo_game *gs, int n, const int32_t *actions, int32_t *legal_counts,
                        uint8_t *mask_bits, float *obs_spatial, float *obs_global, int write_obs)
{
    long total = 0;
#pragma omp parallel for schedule(dynamic, 16) reduction(+:total)
    for (int i = 0; i < n; i++) {
        jqo_game *g = &gs[i];
        jqo_result r;
        if (actions[i] >= 0) jqo_step(g, actions[i] / NC, actions[i] % NC, &r);
        int32_t ids[4096];
        int k = jqo_legal_ids(g, g->turn, ids, 4096);
        uint8_t local[2081];
        uint8_t *bits = mask_bits ? mask_bits + (size_t)i * 2081 : local;
        memset(bits, 0, 2081);
        int s = g->turn;
        for (int j = 0; j < k; j++) {   /* canonical compact bitmask */
            int bit = jqo_canonical_id(s, ids[j]);
            bits[bit >> 3] |= (uint8_t)(1u << (bit & 7));
        }
        legal_counts[i] = k;
        total += k;
        if (write_obs)
            jqo_observe(g, g->turn, obs_spatial + (size_t)i * JQO_OBS_C * NC, obs_global + (size_t)i * JQO_OBS_G);
    }
    return total;
}

/* ======================================================================
 * Samplers (config c2 / c5 action streams; the reference draws its random
 * opponent as the argmax of Gumbel noise over the legal canonical ids,
 * junqi_rl/training/gpu_collector.py:799-810). Philox4x32-10 is the published
 * counter-based generator (Salmon, Moraes, Dror, Shaw, SC'11), restated here
 * and pinned by the Random123 known-answer vectors.
 * ====================================================================== */
void jqo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4])
{
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1; c3 = (uint32_t)p0; c0 = n0; c2 = n2;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

static uint32_t philox_w0(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint64_t seed)
{
    uint32_t ctr[4] = {c0, c1, c2, c3}, key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)}, out[4];
    jqo_philox4x32_10(ctr, key, out);
    return out[0];
}

/* Uniform pick from a legal row: index = (u * n) >> 32 with u = word 0 of
 * Philox(counter (env, ply lo, ply hi, 0), key seed); -1 for an empty row. */
int32_t jqo_sample_uniform(const int32_t *ids, int n, int env, uint64_t seed, uint64_t ply)
{
    if (n <= 0) return -1;
    uint32_t u = philox_w0((uint32_t)env, (uint32_t)ply, (uint32_t)(ply >> 32), 0u, seed);
    return ids[(int)(((uint64_t)u * (uint64_t)n) >> 32)];
}

/* Masked-logit pick: every canonical action id c of the acting seat carries an
 * i.i.d. N(0,1) logit z_c = Phi^-1((u_c + 1/2) / 2^32), u_c = word 0 of
 * Philox(counter (env, ply lo, ply hi, 1 + c), key seed); the action is the
 * argmax of z over the legal set. Phi^-1 is strictly increasing, so that is the
 * argmax of u_c itself (ties to the lowest canonical id, as torch.argmax takes
 * the first maximum). Returns the world id (-1 for an empty row) and the
 * canonical id through *canon. */
int32_t jqo_sample_logits(const int32_t *ids, int n, int seat, int env, uint64_t seed, uint64_t ply, int32_t *canon)
{
    int32_t best = -1, bc = -1;
    uint32_t bu = 0;
    for (int j = 0; j < n; j++) {
        int c = jqo_canonical_id(seat, ids[j]);
        uint32_t u = philox_w0((uint32_t)env, (uint32_t)ply, (uint32_t)(ply >> 32), (uint32_t)(1 + c), seed);
        if (best < 0 || u > bu || (u == bu && c < bc)) { best = ids[j]; bc = c; bu = u; }
    }
    if (canon) *canon = bc;
    return best;
}

/* Pool entry a finished env restarts from (src/env/cuda/src/game_state.cu:2997-3001). */
int32_t jqo_reset_pool_index(int env, int64_t seed, int pool_size)
{
    uint64_t h = (uint64_t)env * 2654435761ull + (uint64_t)seed;
    h ^= h >> 17;
    h *= 0xbf58476d1ce4e5b9ull;
    h ^= h >> 31;
    return (int32_t)(h % (uint64_t)pool_size);
}

/* Digest of a legal-id row: sum of ids[j] * P^j mod 2^64, P = 0x100000001B3. */
static uint64_t row_digest(const int32_t *ids, int m)
{
    uint64_t d = 0, w = 1;
    for (int j = 0; j < m; j++) { d += (uint64_t)(uint32_t)ids[j] * w; w *= 0x100000001B3ull; }
    return d;
}

/* `steps` rollout env-steps of n games (OpenMP over games): at env-step k each
 * game with k >= active_from[i] (all games when active_from is NULL) draws its
 * action from the acting seat's legal ids with `sampler` (0 uniform, 1 masked
 * logits) under (seed, ply0 + k) and applies it; the others take no action.
 * Every game then records the acting team's reward (+-1 on the ply that ends
 * the game), the terminated flag and the Zobrist hash after the ply; a
 * finished game restarts from pool[jqo_reset_pool_index(i, reset_seed0 + k)];
 * and the legal ids of the new acting seat are counted and digested
 * (row_digest). Outputs are (steps, n) row-major; any may be NULL. Returns the
 * number of plies applied. */
long jqo_batch_rollout(jqo_game *gs, int n, const int8_t *pool, int pool_size, int sampler, uint64_t seed,
                       uint64_t ply0, int64_t reset_seed0, int steps, const int32_t *active_from, float *reward,
                       uint8_t *done, uint64_t *hash, int32_t *actions, int32_t *legal_count,
                       uint64_t *legal_digest)
{
    long applied = 0;
#pragma omp parallel for schedule(dynamic, 16) reduction(+:applied)
    for (int i = 0; i < n; i++) {
        jqo_game *g = &gs[i];
        int32_t ids[4096];
        int m = jqo_legal_ids(g, g->turn, ids, 4096);
        for (int k = 0; k < steps; k++) {
            size_t o = (size_t)k * n + i;
            int seat = g->turn;
            int32_t a = -1;
            if (!active_from || k >= active_from[i])
                a = sampler ? jqo_sample_logits(ids, m, seat, i, seed, ply0 + k, NULL)
                            : jqo_sample_uniform(ids, m, i, seed, ply0 + k);
            jqo_result r;
            memset(&r, 0, sizeof r);
            int rc = a >= 0 ? jqo_step(g, a / NC, a % NC, &r) : -1;
            if (rc == 0) applied++;
            if (actions) actions[o] = a;
            if (reward) reward[o] = (rc == 0 && r.terminated && !r.draw && r.winner >= 0)
                                        ? ((seat & 1) == r.winner ? 1.f : -1.f) : 0.f;
            if (done) done[o] = (uint8_t)(g->terminated != 0);
            if (hash) hash[o] = g->zobrist;
            if (g->terminated && pool && pool_size > 0) {
                int p = jqo_reset_pool_index(i, reset_seed0 + k, pool_size);
                jqo_new_game(g, pool + (size_t)p * 120, g->show_mode, g->max_num_moves);
            }
            m = jqo_legal_ids(g, g->turn, ids, 4096);
            if (legal_count) legal_count[o] = m;
            if (legal_digest) legal_digest[o] = row_digest(ids, m);
        }
    }
    return applied;
}

/* Observations of the acting seat of games [g0, g1) (OpenMP), rows from 0. */
void jqo_batch_observe(const jqo_game *gs, int g0, int g1, float *spatial, float *glob)
{
#pragma omp parallel for schedule(dynamic, 8)
    for (int i = g0; i < g1; i++)
        jqo_observe(&gs[i], gs[i].turn, spatial + (size_t)(i - g0) * JQO_OBS_C * NC,
                    glob + (size_t)(i - g0) * JQO_OBS_G);
}

/* The CPU baseline's env-step (OpenMP over games): each game draws its action
 * from the legal ids the previous call left in ids[i] (row cap `cap`, count
 * counts[i]) with `sampler` (0 uniform, 1 masked logits) under (seed, ply),
 * applies it, restarts from pool[jqo_reset_pool_index(i, reset_seed)] when it
 * ended, then writes the new acting seat's legal ids and count, its packed
 * canonical mask (mask_bits: n x 2081 bytes, may be NULL) and its float32
 * observation (obs_spatial / obs_global, may be NULL). Call once with
 * ply < 0 to fill the ids of the opening positions without stepping.
 * Returns the total legal-id count. */
long jqo_batch_cpu_env_step(jqo_game *gs, int n, const int8_t *pool, int pool_size, int sampler, uint64_t seed,
                            int64_t ply, int64_t reset_seed, int32_t *ids, int cap, int32_t *counts,
                            uint8_t *mask_bits, float *obs_spatial, float *obs_global)
{
    long total = 0;
#pragma omp parallel for schedule(dynamic, 16) reduction(+:total)
    for (int i = 0; i < n; i++) {
        jqo_game *g = &gs[i];
        int32_t *row = ids + (size_t)i * cap;
        if (ply >= 0) {
            int m = counts[i], seat = g->turn;
            int32_t a = sampler ? jqo_sample_logits(row, m, seat, i, seed, (uint64_t)ply, NULL)
                                : jqo_sample_uniform(row, m, i, seed, (uint64_t)ply);
            jqo_result r;
            if (a >= 0) jqo_step(g, a / NC, a % NC, &r);
            if (g->terminated && pool && pool_size > 0)
                jqo_new_game(g, pool + (size_t)jqo_reset_pool_index(i, reset_seed, pool_size) * 120, g->show_mode,
                             g->max_num_moves);
        }
        int32_t tmp[4096];
        int k = jqo_legal_ids(g, g->turn, tmp, 4096);
        if (k > cap) k = cap;
        memcpy(row, tmp, sizeof(int32_t) * (size_t)k);
        counts[i] = k;
        total += k;
        if (mask_bits) {
            uint8_t *bits = mask_bits + (size_t)i * 2081;
            memset(bits, 0, 2081);
            for (int j = 0; j < k; j++) {
                int bit = jqo_canonical_id(g->turn, row[j]);
                bits[bit >> 3] |= (uint8_t)(1u << (bit & 7));
            }
        }
        if (obs_spatial && obs_global)
            jqo_observe(g, g->turn, obs_spatial + (size_t)i * JQO_OBS_C * NC, obs_global + (size_t)i * JQO_OBS_G);
    }
    return total;
}

void jqo_set_threads(int n)
{
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

// Board tables and the host lineup generator. See jq_topology.h.
#include "jq_topology.h"

#include <algorithm>
#include <cstring>
#include <vector>

namespace jq {

void seat_cell(int seat, int slot, int &x, int &y)
{
    // seat rectangles (reference board.py:88-102): column = slot % 5, row = slot / 5
    const int col = slot % 5, row = slot / 5;
    switch (seat) {
    case 0: x = 10 - col; y = 11 + row; break;
    case 1: x = 5 - row; y = 10 - col; break;
    case 2: x = 6 + col; y = 5 - row; break;
    default: x = 11 + row; y = 6 + col; break;
    }
}

static bool camp_slot(int s) { return s == 6 || s == 8 || s == 12 || s == 16 || s == 18; }
static bool stronghold_slot(int s) { return s == 26 || s == 28; }
static bool inside(int x, int y) { return x >= 0 && x < 17 && y >= 0 && y < 17; }

void build_tables(Tables &t)
{
    std::memset(&t, 0, sizeof t);
    std::memset(t.owner, -1, sizeof t.owner);
    std::memset(t.localidx, -1, sizeof t.localidx);
    for (int s = 0; s < 4; ++s)
        for (int i = 0; i < 30; ++i) {
            int x, y; seat_cell(s, i, x, y);
            const int f = y * 17 + x;
            uint16_t fl = CF_ON;
            if (camp_slot(i)) fl |= CF_CAMP;
            if (stronghold_slot(i)) fl |= CF_SH;
            const int row = i / 5, col = i % 5;
            if (i < 25 && (row == 0 || row == 4 || col == 0 || col == 4)) fl |= CF_RAIL;
            t.cflags[f] = fl;
            t.owner[f] = (int8_t)s;
            t.localidx[f] = (int8_t)i;
        }
    for (int gx = 0; gx < 3; ++gx)
        for (int gy = 0; gy < 3; ++gy) t.cflags[(6 + 2 * gy) * 17 + 6 + 2 * gx] = CF_ON | CF_RAIL | CF_NG;
    // curve ids: the right column (slot%5==4) of seat c-1 joined to the left
    // column of seat c%4; later ids overwrite earlier ones on shared cells.
    for (int cid = 1; cid <= 4; ++cid)
        for (int j = 4; j < 30; j += 5) {
            int x, y;
            seat_cell(cid - 1, j, x, y);
            t.cflags[y * 17 + x] = (uint16_t)((t.cflags[y * 17 + x] & 0xFF) | (cid << 8));
            seat_cell(cid % 4, j - 4, x, y);
            t.cflags[y * 17 + x] = (uint16_t)((t.cflags[y * 17 + x] & 0xFF) | (cid << 8));
        }
    auto flags = [&](int f) { return t.cflags[f] & 0xFF; };
    auto curve = [&](int f) { return t.cflags[f] >> 8; };

    // rail graph over flat cells
    std::vector<std::vector<int>> g(NC);
    auto link = [&](int a, int b) {
        if (std::find(g[a].begin(), g[a].end(), b) == g[a].end()) g[a].push_back(b);
        if (std::find(g[b].begin(), g[b].end(), a) == g[b].end()) g[b].push_back(a);
    };
    const int dx4[4] = {1, -1, 0, 0}, dy4[4] = {0, 0, 1, -1};
    for (int f = 0; f < NC; ++f) {
        if (!(flags(f) & CF_RAIL)) continue;
        const int x = f % 17, y = f / 17;
        for (int k = 0; k < 4; ++k) {
            const int nx = x + dx4[k], ny = y + dy4[k];
            if (inside(nx, ny) && (flags(ny * 17 + nx) & CF_RAIL)) link(f, ny * 17 + nx);
            const int mx = x + 2 * dx4[k], my = y + 2 * dy4[k];
            if ((flags(f) & CF_NG) && inside(mx, my) && (flags(my * 17 + mx) & CF_NG)) link(f, my * 17 + mx);
        }
    }
    // one arc per inner corner, joining the two front-row end cells that meet there
    const int arcs[4][4] = {{10, 11, 11, 10}, {6, 11, 5, 10}, {6, 5, 5, 6}, {11, 6, 10, 5}};
    for (auto &a : arcs) {
        link(a[1] * 17 + a[0], a[3] * 17 + a[2]);
        t.cflags[a[1] * 17 + a[0]] |= CF_ARC;
        t.cflags[a[3] * 17 + a[2]] |= CF_ARC;
    }
    for (auto &v : g) std::sort(v.begin(), v.end());

    int r = 0;
    std::memset(t.railidx, -1, sizeof t.railidx);
    for (int f = 0; f < NC; ++f)
        if (flags(f) & CF_RAIL) { t.railidx[f] = (int8_t)r; t.railcell[r] = (int16_t)f; ++r; }
    for (int i = 0; i < NRAIL; ++i)
        for (int nb : g[t.railcell[i]]) {
            const int j = t.railidx[nb];
            t.rnbr[i][j >> 6] |= 1ull << (j & 63);
        }

    // road steps
    const int ddx[4] = {1, 1, -1, -1}, ddy[4] = {1, -1, 1, -1};
    for (int f = 0; f < NC; ++f) {
        for (int k = 0; k < 4; ++k) { t.adj[f][k] = -1; t.diag[f][k] = -1; }
        if (!(flags(f) & CF_ON)) continue;
        const int x = f % 17, y = f / 17;
        for (int k = 0; k < 4; ++k) {
            const int nx = x + dx4[k], ny = y + dy4[k];
            if (inside(nx, ny) && (flags(ny * 17 + nx) & CF_ON)) t.adj[f][k] = (int16_t)(ny * 17 + nx);
        }
        int nd = 0;
        for (int k = 0; k < 4; ++k) {
            const int nx = x + ddx[k], ny = y + ddy[k];
            if (!inside(nx, ny)) continue;
            const int nf = ny * 17 + nx;
            if ((flags(nf) & CF_ON) && ((flags(f) & CF_CAMP) || (flags(nf) & CF_CAMP))) t.diag[f][nd++] = (int16_t)nf;
        }
    }

    // straight runs: follow rail edges that stay on the row / column and move on
    std::memset(t.rays, -1, sizeof t.rays);
    std::memset(t.crays, -1, sizeof t.crays);
    for (int i = 0; i < NRAIL; ++i) {
        const int f = t.railcell[i], x0 = f % 17, y0 = f / 17;
        for (int k = 0; k < 4; ++k) {
            int cur = f, n = 0;
            for (;;) {
                const int cx = cur % 17, cy = cur / 17;
                int next = -1;
                for (int nb : g[cur]) {
                    const int nx = nb % 17, ny = nb / 17;
                    const bool along = dx4[k] != 0 ? (ny == y0 && (nx - cx) * dx4[k] > 0)
                                                   : (nx == x0 && (ny - cy) * dy4[k] > 0);
                    if (along) next = nb;
                }
                if (next < 0) break;
                t.rays[i][k][n++] = (int16_t)next;
                cur = next;
            }
            t.raylen[i][k] = (int8_t)n;
        }
        // curve chains: walk rail edges inside the same curve id, both ways
        const int cid = curve(f);
        if (!cid) continue;
        std::vector<int> nbs;
        for (int nb : g[f]) if (curve(nb) == cid) nbs.push_back(nb);
        for (size_t d = 0; d < nbs.size() && d < 2; ++d) {
            int prev = f, cur = nbs[d], n = 0;
            for (;;) {
                t.crays[i][d][n++] = (int16_t)cur;
                int next = -1;
                for (int nb : g[cur]) if (nb != prev && curve(nb) == cid) next = nb;
                if (next < 0) break;
                prev = cur; cur = next;
            }
            t.craylen[i][d] = (int8_t)n;
        }
    }

    int c = 0;
    for (int f = 0; f < NC; ++f) {
        t.f2c[f] = -1;
        if (flags(f) & CF_ON) { t.f2c[f] = (int16_t)c; t.c2f[c++] = (int16_t)f; }
    }
    // canonical frame of observer s (reference rotation.py:44-64)
    for (int s = 0; s < 4; ++s)
        for (int f = 0; f < NC; ++f) {
            const int x = f % 17, y = f / 17;
            int cx, cy;
            switch (s) {
            case 0: cx = x; cy = y; break;
            case 1: cx = y; cy = 16 - x; break;
            case 2: cx = 16 - x; cy = 16 - y; break;
            default: cx = 16 - y; cy = x; break;
            }
            t.rot[s][f] = (int16_t)(cy * 17 + cx);
            t.unrot[s][cy * 17 + cx] = (int16_t)f;
        }
    for (int s = 0; s < 4; ++s) {
        for (int i = 0; i < NONB; ++i) t.rotc[s][i] = (uint8_t)t.f2c[t.rot[s][t.c2f[i]]];
        for (int f = 0; f < NC; ++f) t.canc[s][f] = t.f2c[f] >= 0 ? t.rotc[s][t.f2c[f]] : (uint8_t)0xFF;
    }
    for (int p = 0; p < NP; ++p) {
        const int s = p / 30, i = p % 30;
        int x, y; seat_cell(s, i, x, y);
        t.home[p] = camp_slot(i) ? (int16_t)-1 : (int16_t)(y * 17 + x);
    }
    for (int i = 0, n = 0; i < 30; ++i) t.slotch[i] = camp_slot(i) ? (int8_t)-1 : (int8_t)n++;
    for (int f = 0; f < NC; ++f) {
        const int fl = flags(f);
        t.statics[f] = (uint8_t)(((fl & CF_CAMP) ? 1 : 0) | ((fl & CF_SH) ? 2 : 0) | ((fl & CF_RAIL) ? 4 : 0) |
                                 ((fl & CF_NG) ? 8 : 0) | ((fl & CF_ARC) ? 16 : 0));
        t.sh_other[f] = -1;
    }
    // compact-cell forms
    std::memset(t.adjc, 0xFF, sizeof t.adjc);
    std::memset(t.raym, 0, sizeof t.raym);
    std::memset(t.crayc, 0xFF, sizeof t.crayc);
    std::memset(t.railidxc, -1, sizeof t.railidxc);
    std::memset(t.campm, 0, sizeof t.campm);
    for (int c = 0; c < NONB; ++c) {
        const int f = t.c2f[c];
        int n = 0;
        for (int k = 0; k < 4; ++k) if (t.adj[f][k] >= 0) t.adjc[c][n++] = (uint8_t)t.f2c[t.adj[f][k]];
        for (int k = 0; k < 4; ++k) if (t.diag[f][k] >= 0) t.adjc[c][n++] = (uint8_t)t.f2c[t.diag[f][k]];
        if (flags(f) & CF_CAMP) t.campm[c >> 6] |= 1ull << (c & 63);
        t.railidxc[c] = t.railidx[f];
        for (int h = 0; h < 2; ++h) {
            for (int w = 0; w < 3; ++w) t.adjm[c][h][w] = 0;
            for (int j = 4 * h; j < 4 * h + 4; ++j) {
                const int d = t.adjc[c][j];
                if (d != 0xFF) t.adjm[c][h][d >> 6] |= 1ull << (d & 63);
            }
        }
    }
    std::memset(t.onm, 0, sizeof t.onm);
    std::memset(t.railm, 0, sizeof t.railm);
    std::memset(t.shm, 0, sizeof t.shm);
    for (int f = 0; f < NC; ++f) {
        const int fl = flags(f);
        if (fl & CF_ON) t.onm[f >> 6] |= 1ull << (f & 63);
        if (fl & CF_RAIL) t.railm[f >> 6] |= 1ull << (f & 63);
        if (fl & CF_SH) t.shm[f >> 6] |= 1ull << (f & 63);
    }
    for (int i = 0; i < NRAIL; ++i) {
        t.railc[i] = (uint8_t)t.f2c[t.railcell[i]];
        for (int k = 0; k < 4; ++k)
            for (int j = 0; j < t.raylen[i][k]; ++j) {
                const int c = t.f2c[t.rays[i][k][j]];
                t.raym[i][k][c >> 6] |= 1ull << (c & 63);
            }
        for (int d = 0; d < 2; ++d)
            for (int j = 0; j < t.craylen[i][d]; ++j) t.crayc[i][d][j] = (uint8_t)t.f2c[t.crays[i][d][j]];
    }
    for (int s = 0; s < 4; ++s) {
        int x1, y1, x2, y2;
        seat_cell(s, 26, x1, y1); seat_cell(s, 28, x2, y2);
        t.sh_other[y1 * 17 + x1] = (int16_t)(y2 * 17 + x2);
        t.sh_other[y2 * 17 + x2] = (int16_t)(y1 * 17 + x1);
    }
}

// ---------------------------------------------------------------- lineups
// Mersenne Twister as CPython's random module seeds and draws it.
namespace {
struct MT {
    uint32_t s[624];
    int i = 624;
    explicit MT(uint64_t seed)
    {
        uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
        const int kl = (seed >> 32) ? 2 : 1;
        s[0] = 19650218u;
        for (int k = 1; k < 624; ++k) s[k] = 1812433253u * (s[k - 1] ^ (s[k - 1] >> 30)) + (uint32_t)k;
        int a = 1, b = 0;
        for (int k = 624; k > 0; --k) {
            s[a] = (s[a] ^ ((s[a - 1] ^ (s[a - 1] >> 30)) * 1664525u)) + key[b] + (uint32_t)b;
            if (++a >= 624) { s[0] = s[623]; a = 1; }
            if (++b >= kl) b = 0;
        }
        for (int k = 623; k > 0; --k) {
            s[a] = (s[a] ^ ((s[a - 1] ^ (s[a - 1] >> 30)) * 1566083941u)) - (uint32_t)a;
            if (++a >= 624) { s[0] = s[623]; a = 1; }
        }
        s[0] = 0x80000000u;
    }
    uint32_t next()
    {
        if (i >= 624) {
            for (int k = 0; k < 624; ++k) {
                const uint32_t y = (s[k] & 0x80000000u) | (s[(k + 1) % 624] & 0x7fffffffu);
                s[k] = s[(k + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
            }
            i = 0;
        }
        uint32_t y = s[i++];
        y ^= y >> 11; y ^= (y << 7) & 0x9d2c5680u; y ^= (y << 15) & 0xefc60000u; y ^= y >> 18;
        return y;
    }
    uint32_t below(uint32_t n)  // random._randbelow_with_getrandbits
    {
        int bits = 32 - __builtin_clz(n);
        uint32_t v;
        do { v = next() >> (32 - bits); } while (v >= n);
        return v;
    }
    template <class T> void shuffle(std::vector<T> &v)
    {
        for (int k = (int)v.size() - 1; k >= 1; --k) std::swap(v[k], v[below((uint32_t)k + 1)]);
    }
};

void lineup(MT &rng, int8_t *out)
{
    const int flag = rng.below(2) ? 28 : 26;
    std::vector<int> freeslots;
    for (int i = 0; i < 30; ++i) if (!camp_slot(i) && i != flag) freeslots.push_back(i);
    rng.shuffle(freeslots);
    std::vector<int> mines, bombs;
    for (int i : freeslots) { if (i >= 20) mines.push_back(i); if (i >= 5) bombs.push_back(i); }
    int8_t kind[30];
    std::memset(kind, 0, sizeof kind);
    kind[flag] = 2;
    rng.shuffle(mines);
    bool used[30] = {};
    for (int k = 0; k < 3; ++k) { kind[mines[k]] = 3; used[mines[k]] = true; }
    std::vector<int> b2;
    for (int i : bombs) if (!used[i]) b2.push_back(i);
    rng.shuffle(b2);
    for (int k = 0; k < 2; ++k) { kind[b2[k]] = 4; used[b2[k]] = true; }
    std::vector<int> rest;
    for (int i : freeslots) if (!used[i]) rest.push_back(i);
    rng.shuffle(rest);
    static const int cnt[14] = {0, 0, 0, 0, 0, 1, 1, 2, 2, 2, 2, 3, 3, 3};
    std::vector<int8_t> pieces;
    for (int tp = 5; tp <= 13; ++tp) for (int k = 0; k < cnt[tp]; ++k) pieces.push_back((int8_t)tp);
    rng.shuffle(pieces);
    for (size_t k = 0; k < rest.size(); ++k) kind[rest[k]] = pieces[k];
    std::memcpy(out, kind, 30);
}
// The four canonical opening lineups T, D, G, F in seat-local slots (piece
// types, 0 in the camps), as junqi_core/setup_canonical.py:96-269 defines them.
const int8_t kCanonical[4][30] = {
    {11, 13, 11, 13, 12, 12, 0, 13, 0, 12, 10, 4, 0, 11, 10, 7, 0, 9, 0, 7, 9, 8, 6, 8, 4, 3, 2, 5, 3, 3},
    {13, 11, 13, 11, 13, 12, 0, 12, 0, 12, 10, 11, 0, 10, 4, 7, 0, 9, 0, 8, 8, 9, 7, 6, 4, 5, 2, 3, 3, 3},
    {12, 11, 13, 11, 12, 12, 0, 13, 0, 13, 11, 10, 0, 10, 7, 9, 0, 7, 0, 9, 8, 4, 6, 4, 8, 3, 2, 3, 5, 3},
    {13, 11, 11, 11, 13, 12, 0, 13, 0, 12, 10, 7, 0, 7, 10, 6, 0, 5, 0, 12, 9, 8, 4, 8, 9, 3, 2, 3, 4, 3},
};

// One styled setup: a style by random.choice, then per seat either that
// style's lineup or (mixed, seats 1 and 3) a uniform-random lineup, in seat
// order (gpu_rollout.py:296-305, 360-381).
void styled_setup(MT &rng, int mode, const int8_t *styles, int nstyles, int8_t *out)
{
    const int st = styles[rng.below((uint32_t)nstyles)];
    for (int s = 0; s < 4; ++s) {
        if (mode == SETUP_MIXED && (s & 1)) lineup(rng, out + 30 * s);
        else std::memcpy(out + 30 * s, kCanonical[st], 30);
    }
}
}  // namespace

int canonical_style(char c)
{
    switch (c) {
    case 'T': return 0;
    case 'D': return 1;
    case 'G': return 2;
    case 'F': return 3;
    default: return -1;
    }
}

void generate_styled(int mode, uint64_t seed, int count, bool per_game_seed, const int8_t *styles, int nstyles,
                     int8_t *out)
{
    MT shared(seed);
    for (int i = 0; i < count; ++i) {
        if (per_game_seed) {
            MT rng(seed + (uint64_t)i);
            styled_setup(rng, mode, styles, nstyles, out + (size_t)i * 120);
        } else {
            styled_setup(shared, mode, styles, nstyles, out + (size_t)i * 120);
        }
    }
}

void generate_setup(uint64_t seed, int8_t out[120])
{
    MT rng(seed);
    for (int s = 0; s < 4; ++s) lineup(rng, out + 30 * s);
}

void generate_pool(uint64_t seed, int pool_size, int8_t *out)
{
    MT rng(seed);
    for (int p = 0; p < pool_size; ++p)
        for (int s = 0; s < 4; ++s) lineup(rng, out + (size_t)p * 120 + 30 * s);
}

int validate_lineup(const int8_t *lu)
{   // setup.py:60-136 (validate_lineup): C1-C5 over one seat's 30 slots
    static const int kCount[14] = {0, 0, 1, 3, 2, 1, 1, 2, 2, 2, 2, 3, 3, 3};   // rules.py:131-147
    int cnt[14] = {}, v = 0, nflag = 0, flag_at = -1;
    for (int i = 0; i < 30; ++i)
        if (lu[i] < 0 || lu[i] > 13) return LV_TYPE;   // PieceType(int(p)) raises
    for (int i = 0; i < 30; ++i) {
        const int t = lu[i];
        ++cnt[t];
        if (camp_slot(i) && t != 0) v |= LV_C1;
        if (t == 2) { ++nflag; flag_at = i; }
        if (t == 3 && i < 20) v |= LV_C3;   // landmines only in the back two rows (20..29)
        if (t == 4 && i < 5) v |= LV_C4;    // no bomb in the front row (0..4)
    }
    if (nflag != 1 || !stronghold_slot(flag_at)) v |= LV_C2;
    if (cnt[0] != 5 || cnt[1] != 0) v |= LV_C5;
    for (int t = 2; t <= 13; ++t)
        if (cnt[t] != kCount[t]) v |= LV_C5;
    return v;
}

}  // namespace jq

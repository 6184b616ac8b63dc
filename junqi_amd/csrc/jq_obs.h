// Observation encoder (included into jq_kernels.hip's translation unit, which
// owns the constant tables). One 256-thread block per (env, observer).
//
// Layout and values follow junqi_core/observation.py:155-232 (317 planes in the
// observer's canonical frame, 28 globals) and its writers at :908-1651. The
// block first stages a compact per-piece / per-cell summary in LDS, then streams
// the (317,17,17) row to HBM in aligned 16-byte chunks, computing every element
// from that summary. Values are carried as u8 codes with one decode table; the
// six continuous planes (turn history, recency) are produced as float32.
#pragma once

namespace jq {

constexpr int OBS_C = 317;
constexpr int OBS_ROW = OBS_C * NC;   // 91,613 elements
constexpr int OBS_THREADS = 256;
__constant__ int16_t cAUXCH[6] = {64, 65, 253, 254, 255, 256};

struct ObsLds {
    int8_t cpid[CELL_STRIDE];        // canonical cell -> pid (-1 empty)
    uint8_t rel[PID_STRIDE];         // 0 own, 1 teammate, 2 left enemy, 3 right enemy
    uint8_t tidx[PID_STRIDE];        // tracked type index
    uint8_t bcode[PID_STRIDE];       // observer's belief row code
    uint8_t bkt[PID_STRIDE];         // move bucket | eat top << 2 | surv top << 4 | ours << 6
    int8_t slot[PID_STRIDE];         // piece_slot plane
    uint64_t cmb[PID_STRIDE];        // layer 1 bits 0..44 (enemy) / layer 2 bits 45..49 (own)
    uint64_t l3[PID_STRIDE];         // kill_mine_slot bits 0..29, kill_mine_count 2-bit codes at 32+2t
    float rec[PID_STRIDE][4];        // recency values
    uint32_t dcell[CELL_STRIDE];     // death_reason bits 0..11, dead_at_zero bits 12..13
    unsigned long long ecell[CELL_STRIDE];  // eaten_by planes 0..59
    int16_t hs[HIST_LEN], hd[HIST_LEN];
    float turnv[2];
    uint32_t consts;                 // dead flags 0..2, flag revealed 3..6, dark 7
};

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

__device__ void obs_stage(const State &S, int env, int obs, ObsLds &L)
{
    const int t = threadIdx.x;
    const int tm = (obs + 2) & 3, le = (obs + 1) & 3, re = (obs + 3) & 3, team = obs & 1;
    const int8_t *cellg = S.cell + (size_t)env * CELL_STRIDE;
    for (int k = t; k < CELL_STRIDE; k += OBS_THREADS) {
        L.cpid[k] = k < NC ? cellg[cT.unrot[obs][k]] : (int8_t)-1;
        L.dcell[k] = 0;
        L.ecell[k] = 0;
    }
    if (t < PID_STRIDE) {
        const int pid = t;
        const size_t pi = (size_t)env * PID_STRIDE + pid;
        const int pos = pid < NP ? S.pos[pi] : -1;
        const int tp = pid < NP ? S.ptype[pi] : -1;
        const int s = pid / 30;
        L.rel[pid] = s == obs ? 0 : s == tm ? 1 : s == le ? 2 : 3;
        L.tidx[pid] = (uint8_t)(tp >= 2 ? tp - 2 : 255);
        const int bc = pid < NP ? S.bcode[((size_t)env * 4 + obs) * PID_STRIDE + pid] : 0;
        L.bcode[pid] = (uint8_t)(bc < BC_COUNT ? bc : 0);
        const int ours = (s & 1) == team;
        int mb = 0, eb = 0, sb = 0;
        if (pid < NP) {
            mb = min((int)S.mcount[pi], 3); eb = min((int)S.aeat[pi], 3); sb = min((int)S.psurv[pi], 3);
        }
        L.bkt[pid] = (uint8_t)(mb | (eb << 2) | (sb << 4) | (ours << 6));
        const int sc = cT.slotch[pid % 30];
        L.slot[pid] = (int8_t)(sc < 0 ? 24 : sc);   // a camp slot lands on the last plane, like numpy's -1
        uint64_t cmb = 0, l3 = 0;
        float rc[4] = {0.f, 0.f, 0.f, 0.f};
        if (pos >= 0 && pid < NP) {
            if (!ours) {   // layer 1 and 3 (observation.py:1292-1387, 1475-1567)
                const size_t ci = cm_idx(env, obs, pid);
                const uint64_t dlo = S.cm_dlo[ci], dhi = S.cm_dhi[ci];
                const int mcnt = __popcll(dlo) + __popcll(dhi);
                const int ocnt = S.cm_ocnt[ci];
                const int ccnt = __popcll(S.cm_clo[ci]) + __popcll(S.cm_chi[ci]);
                const int fl = S.cm_floor[ci];
                const uint8_t flg = S.cm_flags[ci];
                cmb |= (uint64_t)(S.cm_dtype[ci] & 0xFFF);
                for (int k = 0; k < 3; ++k) {
                    if (mcnt >= k + 1) cmb |= 1ull << (12 + k);
                    if (ocnt >= k + 1) cmb |= 1ull << (15 + k);
                    if (ccnt >= k + 1) cmb |= 1ull << (30 + k);
                }
                cmb |= (uint64_t)(S.cm_ctype[ci] & 0xFFF) << 18;
                for (int k = 0; k < 9; ++k) if (fl >= k + 1) cmb |= 1ull << (33 + k);
                if (flg & CMF_IS_GONGB) cmb |= 1ull << 42;
                if (flg & CMF_NOT_GONGB) cmb |= 1ull << 43;
                if (back_two(s, S.zero[pi]) && S.mcount[pi] == 0 && !(flg & CMF_ATK_GONGB)) cmb |= 1ull << 44;
                int tcnt[12] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
                for (int sl = 0; sl < 30; ++sl) {
                    const int gp = obs * 30 + sl;
                    const bool hit = gp < 64 ? ((dlo >> gp) & 1) : ((dhi >> (gp - 64)) & 1);
                    if (!hit) continue;
                    l3 |= 1ull << sl;
                    const int gt = S.ptype[(size_t)env * PID_STRIDE + gp];
                    if (gt >= 2 && gt <= 13) tcnt[gt - 2]++;
                }
                for (int k = 0; k < 12; ++k) {
                    const int c = tcnt[k];
                    const uint64_t code = c == 0 ? 0 : c == 1 ? 1 : c == 2 ? 2 : 3;
                    l3 |= code << (32 + 2 * k);
                }
                const int mc = S.mc[env];
                const int last[4] = {S.cm_ldir[ci], S.cm_ldir[ci], S.cm_lchain[ci], S.cm_fstep[ci]};
                for (int k = 0; k < 4; ++k) {
                    if (last[k] < 0) continue;
                    int e = mc - last[k];
                    e = e < 0 ? 0 : (e > 4095 ? 4095 : e);
                    rc[k] = S.rlut[k * 4096 + e];
                }
            } else if (s == obs) {   // layer 2 (observation.py:1392-1451)
                const size_t li = cm_idx(env, le, pid), ri = cm_idx(env, re, pid);
                const int lc = __popcll(S.cm_dlo[li]) + __popcll(S.cm_dhi[li]) + S.cm_ocnt[li];
                const int rcnt = __popcll(S.cm_dlo[ri]) + __popcll(S.cm_dhi[ri]) + S.cm_ocnt[ri];
                const int pk = lc < rcnt ? lc : rcnt;
                for (int k = 0; k < 3; ++k) if (pk >= k + 1) cmb |= 1ull << (45 + k);
                const uint8_t lf = S.cm_flags[li], rf = S.cm_flags[ri];
                if ((lf & CMF_IS_GONGB) && (rf & CMF_IS_GONGB)) cmb |= 1ull << 48;
                const bool atk = (lf & CMF_ATK_GONGB) || (rf & CMF_ATK_GONGB);
                if (back_two(s, S.zero[pi]) && S.mcount[pi] == 0 && !atk) cmb |= 1ull << 49;
            }
        }
        L.cmb[pid] = cmb;
        L.l3[pid] = l3;
        for (int k = 0; k < 4; ++k) L.rec[pid][k] = rc[k];
    }
    if (t < HIST_LEN) {
        const int meta = S.hmeta[env];
        const int cnt = meta & 0xFF, head = (meta >> 8) & 31;
        int16_t hs = -1, hd = -1;
        if (t < cnt) {
            const int e = S.hist[(size_t)env * HIST_LEN + ((head - 1 - t) & 31)];
            hs = cT.rot[obs][min(e & 0xFFFF, NC - 1)];
            hd = cT.rot[obs][min((e >> 16) & 0xFFFF, NC - 1)];
        }
        L.hs[t] = hs; L.hd[t] = hd;
    }
    if (t == 0) {
        const uint8_t sd = S.sdead[env], sf = S.sflag[env];
        const int order[4] = {obs, tm, le, re};
        uint32_t c = 0;
        for (int k = 0; k < 3; ++k) c |= ((sd >> order[k + 1]) & 1u) << k;
        for (int k = 0; k < 4; ++k) c |= ((sf >> order[k]) & 1u) << (3 + k);
        if (S.show_mode == SM_DARK) c |= 1u << 7;
        L.consts = c;
        double dp = (double)S.mslc[env] / 200.0; if (dp > 1.0) dp = 1.0;
        double mp = (double)S.mc[env] / 4000.0; if (mp > 1.0) mp = 1.0;
        L.turnv[0] = (float)dp; L.turnv[1] = (float)mp;
    }
    __syncthreads();
    // death planes (observation.py:1103-1180), anchored in the canonical frame
    if (t < NP) {
        const int pid = t;
        const size_t pi = (size_t)env * PID_STRIDE + pid;
        const int dstp = S.dstep[pi];
        if (dstp >= 0) {
            const int reason = S.dreason[pi], loc = S.dloc[pi], z = S.zero[pi];
            const int s = pid / 30;
            const int grp = s == obs ? 0 : s == tm ? 3 : s == le ? 6 : 9;
            if (reason >= 0 && reason <= 2 && dstp > 0 && (unsigned)loc < (unsigned)NC)
                atomicOr(&L.dcell[cT.rot[obs][loc]], 1u << (grp + reason));
            if ((unsigned)z < (unsigned)NC) atomicOr(&L.dcell[cT.rot[obs][z]], 1u << (12 + (((s & 1) == team) ? 0 : 1)));
        }
    }
    // layer 4 reverse projection (observation.py:1591-1620)
    if (t < 30) {
        const int mp = obs * 30 + t;
        const size_t pi = (size_t)env * PID_STRIDE + mp;
        const int cell = S.pos[pi] >= 0 ? S.pos[pi] : S.zero[pi];
        if ((unsigned)cell < (unsigned)NC) {
            const size_t ci = cm_idx(env, obs, mp);
            const uint64_t elo = S.cm_elo[ci], ehi = S.cm_ehi[ci];
            unsigned long long bits = 0;
            for (int half = 0; half < 2; ++half) {
                const int opp = half == 0 ? le : re;
                for (int s = 0; s < 30; ++s) {
                    const int gp = opp * 30 + s;
                    const bool hit = gp < 64 ? ((elo >> gp) & 1) : ((ehi >> (gp - 64)) & 1);
                    if (hit) bits |= 1ull << (half * 30 + s);
                }
            }
            if (bits) atomicOr(&L.ecell[cT.rot[obs][cell]], bits);
        }
    }
    __syncthreads();
}

// Value of plane c at canonical cell k: a u8 code, or (cont) an exact float.
__device__ __forceinline__ uint32_t obs_code(const ObsLds &L, int c, int k, float &fv, bool &cont)
{
    cont = false;
    const int pid = L.cpid[k];
    const bool has = pid >= 0;
    const int rel = has ? L.rel[pid] : 255;
    if (c < 12) return (rel == 0 && L.tidx[pid] == c) ? 1u : 0u;
    if (c < 24) return rel == 1 ? cBVAL[L.bcode[pid]][c - 12] : 0u;
    if (c == 24) return (rel == 1 && (L.consts & 128u)) ? 1u : 0u;
    if (c == 25) return rel == 2 ? 1u : 0u;
    if (c == 26) return rel == 3 ? 1u : 0u;
    if (c < 39) return rel == 2 ? cBVAL[L.bcode[pid]][c - 27] : 0u;
    if (c < 51) return rel == 3 ? cBVAL[L.bcode[pid]][c - 39] : 0u;
    if (c < 58) return (L.consts >> (c - 51)) & 1u;
    if (c < 64) return (cT.statics[k] >> (c - 58)) & 1u;
    if (c < 66) { cont = true; fv = L.turnv[c - 64]; return 0u; }
    if (c < 90) {
        if (!has) return 0u;
        const int b = L.bkt[pid];
        const int half = (b >> 6) ? 0 : 4;
        const int grp = (c - 66) >> 3, j = (c - 66) & 7;
        if (j < half || j >= half + 4) return 0u;
        const int q = j - half;
        if (grp == 0) return q == (b & 3) ? 1u : 0u;
        const int top = grp == 1 ? ((b >> 2) & 3) : ((b >> 4) & 3);
        return q <= top ? 1u : 0u;
    }
    if (c < 104) return (L.dcell[k] >> (c - 90)) & 1u;
    if (c < 129) return (has && L.slot[pid] == c - 104) ? 1u : 0u;
    if (c < 161) {
        const int d = c - 129;
        if (L.hd[d] == k) return 1u;
        return L.hs[d] == k ? 2u : 0u;
    }
    if (c < 211) return has ? (uint32_t)((L.cmb[pid] >> (c - 161)) & 1u) : 0u;
    if (c < 223) {
        if (!has) return 0u;
        const uint32_t q = (uint32_t)((L.l3[pid] >> (32 + 2 * (c - 211))) & 3u);
        return q == 0 ? 0u : q == 1 ? 3u : q == 2 ? 4u : 1u;
    }
    if (c < 253) return has ? (uint32_t)((L.l3[pid] >> (c - 223)) & 1u) : 0u;
    if (c < 257) { cont = true; fv = has ? L.rec[pid][c - 253] : 0.f; return 0u; }
    return (uint32_t)((L.ecell[k] >> (c - 257)) & 1u);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f)
{
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Element e of the row in the requested format, as raw bits.
template <int FMT>
__device__ __forceinline__ uint32_t obs_elem_bits(const ObsLds &L, int c, int k)
{
    float fv;
    bool cont;
    const uint32_t code = obs_code(L, c, k, fv, cont);
    if (FMT == 2) return code;                       // u8: continuous planes are in aux
    const float v = cont ? fv : cDECODE[code];
    if (FMT == 0) return __float_as_uint(v);
    return f32_to_bf16_rne(v);
}

// Stream `nelem` elements (plane-major, 289 cells per plane) of element size ES
// to `row`, in aligned 16-byte chunks; partial chunks at either end are written
// element by element. `plane_of` maps the local plane index to a channel.
template <int FMT, int ES, bool AUX>
__device__ void obs_emit(const ObsLds &L, uint8_t *row, int nelem)
{
    const uintptr_t B = (uintptr_t)row;
    const uintptr_t E = B + (uintptr_t)nelem * ES;
    const uintptr_t q0 = B >> 4, q1 = (E - 1) >> 4;
    for (uintptr_t q = q0 + threadIdx.x; q <= q1; q += OBS_THREADS) {
        const uintptr_t lo = max(q << 4, B), hi = min((q << 4) + 16, E);
        int e = (int)((lo - B) / ES);
        const int e1 = (int)((hi - B) / ES);
        int p = e / NC, k = e - p * NC;
        if (lo == (q << 4) && hi == (q << 4) + 16) {
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 16 / ES; ++i) {
                const int c = AUX ? cAUXCH[p] : p;
                uint32_t v;
                if (AUX) { float fv; bool cont; (void)obs_code(L, c, k, fv, cont); v = __float_as_uint(fv); }
                else v = obs_elem_bits<FMT>(L, c, k);
                const int bitoff = (i * ES) * 8;
                w[bitoff >> 5] |= v << (bitoff & 31);
                if (++k == NC) { k = 0; ++p; }
            }
            *reinterpret_cast<uint4 *>(q << 4) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (; e < e1; ++e) {
                const int c = AUX ? cAUXCH[p] : p;
                uint32_t v;
                if (AUX) { float fv; bool cont; (void)obs_code(L, c, k, fv, cont); v = __float_as_uint(fv); }
                else v = obs_elem_bits<FMT>(L, c, k);
                uint8_t *dst = row + (size_t)e * ES;
                if (ES == 1) *dst = (uint8_t)v;
                else if (ES == 2) *reinterpret_cast<uint16_t *>(dst) = (uint16_t)v;
                else *reinterpret_cast<uint32_t *>(dst) = v;
                if (++k == NC) { k = 0; ++p; }
            }
        }
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
    obs_stage(S, env, obs, L);
    constexpr int ES = FMT == 0 ? 4 : FMT == 1 ? 2 : 1;
    obs_emit<FMT, ES, false>(L, reinterpret_cast<uint8_t *>(spatial) + (size_t)row * OBS_ROW * ES, OBS_ROW);
    if (FMT == 2 && aux) obs_emit<0, 4, true>(L, reinterpret_cast<uint8_t *>(aux + (size_t)row * 6 * NC), 6 * NC);
    if (glob && threadIdx.x < 28) {   // observation.py:1623-1651
        const int t = threadIdx.x;
        const int le = (obs + 1) & 3, re = (obs + 3) & 3, tm = (obs + 2) & 3;
        float v;
        if (t < 24) {
            const int seat = t < 12 ? le : re, ti = t % 12;
            const bool trk = (S.remtrk[(size_t)env * 4 + obs] >> seat) & 1;
            v = trk ? (float)S.rem[((size_t)env * 4 + obs) * 48 + seat * 12 + ti] : 0.f;
        } else {
            const int order[4] = {obs, tm, le, re};
            v = (float)((S.sflag[env] >> order[t - 24]) & 1);
        }
        glob[(size_t)row * 28 + t] = v;
    }
}

}  // namespace jq

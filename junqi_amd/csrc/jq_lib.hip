// C ABI of the batched Junqi environment: handle lifetime, table upload, state
// import/export and kernel launches. Declarations and contracts live in
// include/junqi_amd.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "junqi_amd.h"
#include "jq_device.h"
#include "jq_kernels.h"
#include "jq_obs.h"
#include "jq_history.h"
#include "jq_masks.h"
#include "jq_topology.h"

using namespace jq;

struct jq_env {
    int device = 0;
    State S{};
    std::vector<void *> allocs;
    bool zob_ready = false, rlut_ready = false;
    int obs_blocks = 0;              // resident u8 observation blocks on the device
    int obs_f32_pad = -1;            // dynamic LDS bytes that hold the f32 observation at 3 blocks per CU
    float *ext_bel = nullptr;        // uploaded (N, 4, 12, 289) beliefs, allocated on first upload
    bool ext_on = false;             // observations read the uploaded beliefs
    int8_t *pool = nullptr;          // setup pool buffer (reused while uploads fit)
    int32_t pool_cap = 0;            // entries the pool buffer holds
    int32_t *total_host = nullptr;   // pinned host word for CSR totals read back
    hipStream_t side = nullptr;      // jq_env_step's CSR pass beside the observation
    hipEvent_t ev_step = nullptr, ev_csr = nullptr;
    bool obs_timing = false;         // jq_obs_timing: events around every observation launch
    std::vector<std::pair<hipEvent_t, hipEvent_t>> obs_ev;
    size_t obs_ev_used = 0;
    hipEvent_t obs_t_end = nullptr;  // end event of a launch whose begin jq_env_step recorded
};

// Rollout history: per-step copies of every per-env state block.
struct jq_history {
    int device = 0;
    int32_t show_mode = 0, max_moves = 0;
    HistState H{};
    std::vector<void *> allocs;
    float *rlut = nullptr;           // recency table copied from the snapshotted handle
    bool rlut_ready = false;
    jq_env *replay = nullptr;        // scratch state of the rebuilt rows
    int32_t replay_cap = 0;
};

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_TRY(expr)                                                                      \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess) return fail(JQ_E_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

std::mutex g_tab_mu;
bool g_tab_done[64] = {};
Tables g_tables;
bool g_host_tables = false;
uint8_t g_bval[BC_COUNT][12];
float g_decode[256];

void prior_row(int slot, float out[12])
{   // info_model.py:115-132: counts over the admissible types, float32 normalised
    static const int cnt[14] = {0, 0, 1, 3, 2, 1, 1, 2, 2, 2, 2, 3, 3, 3};
    const bool camp = slot == 6 || slot == 8 || slot == 12 || slot == 16 || slot == 18;
    const bool sh = slot == 26 || slot == 28;
    float v[12] = {};
    if (!camp)
        for (int t = 2; t <= 13; ++t) {
            bool ok = true;
            if (!sh) {
                if (t == 2) ok = false;
                if (t == 3 && slot < 20) ok = false;
                if (t == 4 && slot < 5) ok = false;
            }
            if (ok) v[t - 2] = (float)cnt[t];
        }
    float s = 0.f;
    for (float x : v) s += x;
    for (int i = 0; i < 12; ++i) out[i] = s > 0.f ? v[i] / s : 0.f;
}

void build_host_tables()
{
    if (g_host_tables) return;
    build_tables(g_tables);
    std::memset(g_decode, 0, sizeof g_decode);
    g_decode[0] = 0.f; g_decode[1] = 1.f; g_decode[2] = -1.f;
    g_decode[3] = 1.0f / 3.0f; g_decode[4] = 2.0f / 3.0f;
    int next = 5;
    for (int code = 0; code < BC_COUNT; ++code) {
        float row[12] = {};
        if (code >= 1 && code <= 12) row[code - 1] = 1.f;
        else if (code >= BC_PRIOR0 && code < BC_PRIOR0 + 30) prior_row(code - BC_PRIOR0, row);
        else if (code == BC_UNIFORM) for (float &x : row) x = (float)(1.0 / 12.0);
        for (int t = 0; t < 12; ++t) {
            int found = -1;
            for (int i = 0; i < next; ++i)
                if (std::memcmp(&g_decode[i], &row[t], 4) == 0) { found = i; break; }
            if (found < 0) { found = next; g_decode[next++] = row[t]; }
            g_bval[code][t] = (uint8_t)found;
        }
    }
    g_host_tables = true;
}

int ensure_device_tables(int device)
{
    std::lock_guard<std::mutex> lk(g_tab_mu);
    build_host_tables();
    if (device < 0 || device >= 64) return fail(JQ_E_ARG, "device %d out of range", device);
    if (g_tab_done[device]) return JQ_OK;
    HIP_TRY(hipMemcpyToSymbol(HIP_SYMBOL(cT), &g_tables, sizeof g_tables));
    HIP_TRY(hipMemcpyToSymbol(HIP_SYMBOL(cBVAL), g_bval, sizeof g_bval));
    HIP_TRY(hipMemcpyToSymbol(HIP_SYMBOL(cDECODE), g_decode, sizeof g_decode));
    g_tab_done[device] = true;
    return JQ_OK;
}

template <class T>
int dalloc(jq_env *e, T *&p, size_t count, int fill_byte)
{
    void *q = nullptr;
    const size_t bytes = count * sizeof(T) + 64;
    if (hipMalloc(&q, bytes) != hipSuccess) return fail(JQ_E_OOM, "hipMalloc(%zu) failed", bytes);
    e->allocs.push_back(q);
    if (hipMemset(q, fill_byte, bytes) != hipSuccess) return fail(JQ_E_HIP, "hipMemset failed");
    p = static_cast<T *>(q);
    return JQ_OK;
}

template <class T>
int halloc(jq_history *h, T *&p, size_t count)
{
    void *q = nullptr;
    const size_t bytes = count * sizeof(T);
    if (hipMalloc(&q, bytes) != hipSuccess) return fail(JQ_E_OOM, "hipMalloc(%zu) failed", bytes);
    h->allocs.push_back(q);
    if (hipMemset(q, 0, bytes) != hipSuccess) return fail(JQ_E_HIP, "hipMemset failed");
    p = static_cast<T *>(q);
    return JQ_OK;
}

// Where field f lives: array, per-env stride, element stride, byte offset of
// element 0 inside its record, element size, elements per env.
enum FieldArr { AR_CELL, AR_PIECE, AR_CM, AR_CME, AR_BCODE, AR_REM, AR_ENV, AR_HIST };
struct FieldDesc { int arr, elems, bytes; size_t env_stride, el_stride, off; };
#define PF(m) {AR_PIECE, PID_STRIDE, (int)sizeof(PieceRec::m), PID_STRIDE * sizeof(PieceRec), sizeof(PieceRec), offsetof(PieceRec, m)}
#define CF(m) {AR_CM, 4 * PID_STRIDE, (int)sizeof(CmRec::m), 4 * PID_STRIDE * sizeof(CmRec), sizeof(CmRec), offsetof(CmRec, m)}
#define CE(m) {AR_CME, 4 * PID_STRIDE, (int)sizeof(CmEat::m), 4 * PID_STRIDE * sizeof(CmEat), sizeof(CmEat), offsetof(CmEat, m)}
#define EF(m) {AR_ENV, 1, (int)sizeof(EnvRec::m), sizeof(EnvRec), sizeof(EnvRec::m), offsetof(EnvRec, m)}
const FieldDesc kFields[JQ_F_COUNT] = {
    {AR_CELL, CELL_STRIDE, 1, CELL_STRIDE, 1, 0},
    PF(ptype), PF(pos), PF(zero), PF(mcount), PF(aeat), PF(psurv), PF(dreason), PF(dstep), PF(dloc),
    {AR_BCODE, 4 * PID_STRIDE, 1, 4 * PID_STRIDE, 1, 0},
    {AR_REM, 4 * 48, 1, 4 * 48, 1, 0},
    {AR_ENV, 4, 1, sizeof(EnvRec), 1, offsetof(EnvRec, remtrk)},
    CF(dlo), CF(dhi), CF(dtype), CF(ldir), CF(ocnt), CF(clo), CF(chi), CF(ctype), CF(lchain), CE(elo), CE(ehi),
    CF(floor), CF(fstep), CF(flags),
    {AR_HIST, HIST_LEN, 4, HIST_LEN * 4, 4, 0},
    EF(hmeta), EF(turn), EF(term), EF(winner), EF(draw), EF(sdead), EF(sflag), EF(mc), EF(mslc), EF(zob),
};
#undef PF
#undef CF
#undef CE
#undef EF

uint8_t *field_array(jq_env *e, int arr)
{
    State &S = e->S;
    switch (arr) {
    case AR_CELL: return reinterpret_cast<uint8_t *>(S.cell);
    case AR_PIECE: return reinterpret_cast<uint8_t *>(S.piece);
    case AR_CM: return reinterpret_cast<uint8_t *>(S.cm);
    case AR_CME: return reinterpret_cast<uint8_t *>(S.cme);
    case AR_BCODE: return S.bcode;
    case AR_REM: return reinterpret_cast<uint8_t *>(S.rem);
    case AR_ENV: return reinterpret_cast<uint8_t *>(S.env);
    default: return reinterpret_cast<uint8_t *>(S.hist);
    }
}

inline hipStream_t strm(void *s) { return reinterpret_cast<hipStream_t>(s); }

// validate_setup (setup.py:139-159) of `count` setups of 120 slot types: the
// first seat lineup that breaks C1-C5 fails the call with its rules named.
int check_setups(const int8_t *host, size_t count, const char *what)
{
    static const char *kRule[6] = {"TYPE", "C1", "C2", "C3", "C4", "C5"};
    for (size_t i = 0; i < count; ++i)
        for (int seat = 0; seat < 4; ++seat) {
            const int v = validate_lineup(host + i * NP + 30 * seat);
            if (!v) continue;
            std::string names;
            for (int b = 0; b < 6; ++b)
                if (v & (1 << b)) names += std::string(names.empty() ? "" : ",") + kRule[b];
            return fail(JQ_E_ARG, "setup violates rules: %s %zu seat %d breaks %s", what, i, seat, names.c_str());
        }
    return JQ_OK;
}

// A values buffer of N * JQ_MAX_LEGAL ids always holds the CSR, and the int32
// offsets cannot overflow while that bound is at most INT32_MAX (N <= 671,088):
// then no read-back is needed.
bool csr_always_fits(const jq_env *e, int64_t cap)
{
    const int64_t bound = (int64_t)e->S.n * JQ_MAX_LEGAL;
    return bound <= (int64_t)INT32_MAX && cap >= bound;
}

// CSR capacity check of jq_legal / jq_env_step: unless csr_always_fits, the
// total (offsets[n], just scanned on `s`; -1 when it exceeds the int32 offsets)
// is read back and must fit.
int csr_fits(jq_env *e, const int32_t *offsets, int64_t cap, hipStream_t s)
{
    if (csr_always_fits(e, cap)) return JQ_OK;
    if (!e->total_host) {
        void *q = nullptr;
        if (hipHostMalloc(&q, sizeof(int32_t)) != hipSuccess) return fail(JQ_E_OOM, "pinned host word");
        e->total_host = static_cast<int32_t *>(q);
    }
    HIP_TRY(hipMemcpyAsync(e->total_host, offsets + e->S.n, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (*e->total_host < 0)
        return fail(JQ_E_CAPACITY, "legal ids exceed the int32 offsets (more than %d in the batch)", INT32_MAX);
    if ((int64_t)*e->total_host > cap)
        return fail(JQ_E_CAPACITY, "legal ids need %d values, the buffer holds %lld", *e->total_host, (long long)cap);
    return JQ_OK;
}

int check_env(jq_env *e)
{
    if (!e) return fail(JQ_E_ARG, "null handle");
    if (hipSetDevice(e->device) != hipSuccess) return fail(JQ_E_HIP, "hipSetDevice(%d) failed", e->device);
    return JQ_OK;
}

int launch_check(const char *what)
{
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(JQ_E_HIP, "%s launch: %s", what, hipGetErrorString(err));
    return JQ_OK;
}

// Persistent grid of the u8 observation kernel: every block the device can
// hold at once.
int obs_u8_grid(jq_env *e)
{
    if (e->obs_blocks > 0) return JQ_OK;
    int per_cu = 0, cus = 0;
    HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_observe_u8_persist, OBS_THREADS, 0));
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, e->device));
    e->obs_blocks = std::max(1, per_cu) * std::max(1, cus);
    return JQ_OK;
}

// The f32 observation (one block per 366,452-byte row) writes faster with at
// most 3 blocks per CU than at the 4 its LDS and registers allow (fewer rows
// streaming at once: 2.377 -> 2.272 ms per launch at 32,768 rows; bf16 rows,
// half as long, are slower at 3). Each block asks for unused dynamic LDS that
// brings it to the midpoint between a third and a quarter of the CU's LDS, so
// a fourth block does not fit and a third still does after the allocation
// rounds up (a pad that left only 0.9 % of slack under the third was rounded
// past it: 2 blocks per CU, 3.06 ms). 0 when the occupancy query does not
// confirm exactly 3.
int obs_f32_pad(jq_env *e, int &pad)
{
    if (e->obs_f32_pad < 0) {
        hipFuncAttributes fa{};
        int lds_cu = 0, per_cu = 0;
        HIP_TRY(hipFuncGetAttributes(&fa, reinterpret_cast<const void *>(&k_observe<0, false>)));
        HIP_TRY(hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, e->device));
        int p = (lds_cu / 3 + lds_cu / 4) / 2 - (int)fa.sharedSizeBytes;
        if (p > 0) {
            HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_observe<0, false>, OBS_THREADS, p));
            if (per_cu != 3) p = 0;
        } else {
            p = 0;
        }
        e->obs_f32_pad = p;
    }
    pad = e->obs_f32_pad;
    return JQ_OK;
}

// The checks of an observation request (format, buffers, tables it needs).
int obs_args(const jq_env *e, int32_t fmt, const void *spatial, const void *aux, const float *global)
{
    if (!spatial) return fail(JQ_E_ARG, "null spatial output");
    if (fmt < JQ_OBS_F32 || fmt > JQ_OBS_U8) return fail(JQ_E_ARG, "bad observation format %d", fmt);
    const int es = fmt == JQ_OBS_F32 ? 4 : fmt == JQ_OBS_BF16 ? 2 : 1;
    if ((uintptr_t)spatial % es || (global && (uintptr_t)global % 4))
        return fail(JQ_E_ARG, "observation buffers must be aligned to their element size");
    if (aux && fmt != JQ_OBS_U8) return fail(JQ_E_ARG, "aux rows belong to the u8 format only");
    if (aux && (uintptr_t)aux % 16) return fail(JQ_E_ARG, "u8 aux rows must be 16-byte aligned");
    if ((fmt != JQ_OBS_U8 || aux) && !e->rlut_ready) return fail(JQ_E_STATE, "recency table not uploaded");
    if (e->ext_on && fmt == JQ_OBS_U8)
        return fail(JQ_E_STATE, "uploaded beliefs are arbitrary floats: observe them as JQ_OBS_F32 or JQ_OBS_BF16");
    return JQ_OK;
}

// With jq_obs_timing on: record the begin event of the next observation launch
// on `stream` and hand back its end event (else *t_end = nullptr).
int obs_timing_begin(jq_env *e, void *stream, hipEvent_t *t_end, hipEvent_t *t_begin = nullptr)
{
    *t_end = nullptr;
    if (t_begin) *t_begin = nullptr;
    if (!e->obs_timing || e->obs_ev_used >= JQ_OBS_TIMING_MAX) return JQ_OK;
    if (e->obs_ev_used == e->obs_ev.size()) {   // a pair per launch, reused after jq_obs_timing_read
        hipEvent_t a = nullptr, b = nullptr;
        HIP_TRY(hipEventCreate(&a));
        if (hipEventCreate(&b) != hipSuccess) {
            (void)hipEventDestroy(a);
            return fail(JQ_E_HIP, "hipEventCreate failed");
        }
        e->obs_ev.emplace_back(a, b);
    }
    const auto &pr = e->obs_ev[e->obs_ev_used++];
    HIP_TRY(hipEventRecord(pr.first, strm(stream)));
    *t_end = pr.second;
    if (t_begin) *t_begin = pr.first;
    return JQ_OK;
}

}  // namespace

extern "C" {

const char *jq_last_error(void) { return g_err.c_str(); }
const char *jq_version(void) { return "junqi_amd 0.1 (gfx950)"; }

int jq_create(jq_env **out, int32_t n, int32_t max_num_moves, int32_t show_mode, int32_t device)
{
    if (!out) return fail(JQ_E_ARG, "out is null");
    *out = nullptr;
    if (n <= 0 || n > (1 << 24)) return fail(JQ_E_ARG, "num_envs %d out of range", n);
    if (max_num_moves <= 0) return fail(JQ_E_ARG, "max_num_moves must be positive");
    if (show_mode < 0 || show_mode > 2) return fail(JQ_E_ARG, "show_mode %d not in {0,1,2}", show_mode);
    int ndev = 0;
    HIP_TRY(hipGetDeviceCount(&ndev));
    if (device < 0 || device >= ndev) return fail(JQ_E_ARG, "device %d not present (%d devices)", device, ndev);
    HIP_TRY(hipSetDevice(device));
    int rc = ensure_device_tables(device);
    if (rc) return rc;
    jq_env *e = new jq_env();
    e->device = device;
    State &S = e->S;
    S.n = n; S.max_moves = max_num_moves; S.show_mode = show_mode; S.pool_size = 0;
    const size_t N = (size_t)n;
#define A(ptr, cnt, fill) do { if ((rc = dalloc(e, ptr, cnt, fill)) != 0) { jq_destroy(e); return rc; } } while (0)
    A(S.cell, N * CELL_STRIDE, 0xFF);
    A(S.piece, N * PID_STRIDE, 0);
    A(S.cm, N * 4 * PID_STRIDE, 0);
    A(S.cme, N * 4 * PID_STRIDE, 0);
    A(S.cmk, N * 4 * PID_STRIDE, 0);
    A(S.cmv, N * 4 * PID_STRIDE, 0);
    A(S.bcode, N * 4 * PID_STRIDE, 0);
    A(S.rem, N * 4 * 48, 0);
    A(S.env, N, 0);
    A(S.hist, N * HIST_LEN, 0);
    A(S.lg, N, 0);
    uint64_t *zt = nullptr; A(zt, (size_t)ZTOTAL, 0); S.ztab = zt;
    float *rl = nullptr; A(rl, 4 * 4096, 0); S.rlut = rl;
    hipLaunchKernelGGL(k_clear, dim3(n), dim3(64), 0, 0, S);
    if ((rc = launch_check("k_clear")) != 0) { jq_destroy(e); return rc; }
    if (hipDeviceSynchronize() != hipSuccess) { jq_destroy(e); return fail(JQ_E_HIP, "state clear failed"); }
#undef A
    *out = e;
    return JQ_OK;
}

int jq_destroy(jq_env *e)
{
    if (!e) return JQ_OK;
    (void)hipSetDevice(e->device);
    // kernels of any stream, the side stream's included, may still use the
    // handle's buffers
    (void)hipDeviceSynchronize();
    for (void *p : e->allocs) (void)hipFree(p);
    if (e->pool) (void)hipFree(e->pool);
    if (e->total_host) (void)hipHostFree(e->total_host);
    if (e->side) (void)hipStreamDestroy(e->side);
    if (e->ev_step) (void)hipEventDestroy(e->ev_step);
    if (e->ev_csr) (void)hipEventDestroy(e->ev_csr);
    for (auto &pr : e->obs_ev) { (void)hipEventDestroy(pr.first); (void)hipEventDestroy(pr.second); }
    delete e;
    return JQ_OK;
}

int32_t jq_num_envs(const jq_env *e) { return e ? e->S.n : 0; }

int jq_upload_zobrist(jq_env *e, const uint64_t *host, int64_t count)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!host || count != ZTOTAL) return fail(JQ_E_ARG, "zobrist table must hold %d uint64 values", ZTOTAL);
    HIP_TRY(hipMemcpy((void *)e->S.ztab, host, sizeof(uint64_t) * ZTOTAL, hipMemcpyHostToDevice));
    e->zob_ready = true;
    return JQ_OK;
}

int jq_upload_recency(jq_env *e, const float *host)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!host) return fail(JQ_E_ARG, "null recency table");
    HIP_TRY(hipMemcpy((void *)e->S.rlut, host, sizeof(float) * 4 * 4096, hipMemcpyHostToDevice));
    e->rlut_ready = true;
    return JQ_OK;
}

int jq_validate_lineup(const int8_t *lineup30)
{
    if (!lineup30) return fail(JQ_E_ARG, "null lineup");
    return validate_lineup(lineup30);
}

int jq_upload_setup_pool(jq_env *e, const int8_t *host, int32_t pool_size)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!host || pool_size <= 0) return fail(JQ_E_ARG, "empty setup pool");
    if ((rc = check_setups(host, (size_t)pool_size, "pool entry")) != 0) return rc;
    // kernels of any stream may still read the old pool: let them finish first
    HIP_TRY(hipDeviceSynchronize());
    if (pool_size > e->pool_cap) {
        if (e->pool) { (void)hipFree(e->pool); e->pool = nullptr; e->pool_cap = 0; e->S.pool = nullptr; e->S.pool_size = 0; }
        void *q = nullptr;
        if (hipMalloc(&q, (size_t)pool_size * NP) != hipSuccess)
            return fail(JQ_E_OOM, "hipMalloc(%zu) for the setup pool failed", (size_t)pool_size * NP);
        e->pool = static_cast<int8_t *>(q);
        e->pool_cap = pool_size;
    }
    HIP_TRY(hipMemcpy(e->pool, host, (size_t)pool_size * NP, hipMemcpyHostToDevice));
    e->S.pool = e->pool;
    e->S.pool_size = pool_size;
    return JQ_OK;
}

int jq_reset_lineups(jq_env *e, const int8_t *host, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!host) return fail(JQ_E_ARG, "null lineups");
    if (!e->zob_ready) return fail(JQ_E_STATE, "upload the Zobrist tables before resetting");
    if ((rc = check_setups(host, (size_t)e->S.n, "env")) != 0) return rc;
    int8_t *d = nullptr;
    const size_t bytes = (size_t)e->S.n * NP;
    HIP_TRY(hipMallocAsync((void **)&d, bytes, strm(stream)));
    HIP_TRY(hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, strm(stream)));
    hipLaunchKernelGGL(k_reset_lineups, dim3(e->S.n), dim3(64), 0, strm(stream), e->S, d);
    rc = launch_check("k_reset_lineups");
    HIP_TRY(hipFreeAsync(d, strm(stream)));
    HIP_TRY(hipStreamSynchronize(strm(stream)));
    return rc;
}

int jq_generate_pool(int64_t seed, int32_t pool_size, int8_t *host_out)
{
    if (!host_out || pool_size < 0) return fail(JQ_E_ARG, "bad pool buffer");
    generate_pool((uint64_t)seed, pool_size, host_out);
    return JQ_OK;
}

int jq_generate_styled(int32_t mode, int64_t seed, int32_t count, int32_t per_game_seed, const char *styles,
                       int32_t nstyles, int8_t *host_out)
{
    if (mode != JQ_SETUP_CANONICAL && mode != JQ_SETUP_MIXED) return fail(JQ_E_ARG, "bad setup mode %d", mode);
    if (!host_out || count < 0) return fail(JQ_E_ARG, "bad setup buffer");
    if (!styles || nstyles <= 0) return fail(JQ_E_ARG, "setup styles must be non-empty");
    std::vector<int8_t> idx((size_t)nstyles);
    for (int32_t k = 0; k < nstyles; ++k) {
        const int v = canonical_style(styles[k]);
        if (v < 0) return fail(JQ_E_ARG, "unknown setup style '%c' (valid: D, F, G, T)", styles[k]);
        idx[(size_t)k] = (int8_t)v;
    }
    generate_styled(mode, (uint64_t)seed, count, per_game_seed != 0, idx.data(), nstyles, host_out);
    return JQ_OK;
}

int jq_board_tables(void *host_out, int64_t nbytes)
{
    std::lock_guard<std::mutex> lk(g_tab_mu);
    build_host_tables();
    if (!host_out || nbytes != (int64_t)sizeof(Tables)) return fail(JQ_E_ARG, "need %zu bytes", sizeof(Tables));
    std::memcpy(host_out, &g_tables, sizeof(Tables));
    return JQ_OK;
}

int jq_generate_lineups(int64_t seed_base, int32_t count, int8_t *host_out)
{
    if (!host_out || count < 0) return fail(JQ_E_ARG, "bad lineup buffer");
    for (int32_t i = 0; i < count; ++i) generate_setup((uint64_t)(seed_base + i), host_out + (size_t)i * NP);
    return JQ_OK;
}

int jq_reset_seeded(jq_env *e, int64_t seed_base, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    std::vector<int8_t> lu((size_t)e->S.n * NP);
    if ((rc = jq_generate_lineups(seed_base, e->S.n, lu.data())) != 0) return rc;
    return jq_reset_lineups(e, lu.data(), stream);
}

int jq_reset_terminated(jq_env *e, int64_t seed, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!e->S.pool || e->S.pool_size <= 0) return fail(JQ_E_STATE, "no setup pool uploaded");
    if (!e->zob_ready) return fail(JQ_E_STATE, "upload the Zobrist tables before resetting");
    hipLaunchKernelGGL(k_reset_terminated, dim3(e->S.n), dim3(64), 0, strm(stream), e->S, seed);
    return launch_check("k_reset_terminated");
}

int jq_step(jq_env *e, const int32_t *actions, const int8_t *acting, int32_t fmt, uint8_t *valid, int8_t *event,
            uint8_t *terminated, int8_t *winner, uint8_t *draw, uint8_t *flag_captured, uint8_t *seats_died,
            float *reward, int32_t *world_action, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!actions) return fail(JQ_E_ARG, "null actions");
    if (fmt != JQ_ACT_WORLD && fmt != JQ_ACT_CANONICAL) return fail(JQ_E_ARG, "bad action format %d", fmt);
    if (!e->zob_ready) return fail(JQ_E_STATE, "upload the Zobrist tables before stepping");
    StepOut O{valid, event, terminated, winner, draw, flag_captured, seats_died, reward, world_action, nullptr};
    hipLaunchKernelGGL(k_step, dim3(e->S.n), dim3(64), 0, strm(stream), e->S, actions, acting, fmt, O);
    return launch_check("k_step");
}

int jq_legal(jq_env *e, const int8_t *acting, int32_t *counts, int32_t *offsets, int32_t *values,
             int64_t values_capacity, int32_t *mask_words, uint8_t *mask_bool, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if ((offsets || values) && !counts) return fail(JQ_E_ARG, "offsets/values need counts");
    if (values && !offsets) return fail(JQ_E_ARG, "values need offsets");
    if (values && values_capacity < 0) return fail(JQ_E_ARG, "negative values capacity");
    hipLaunchKernelGGL(k_legal, dim3(e->S.n), dim3(64), 0, strm(stream), e->S, acting, counts, mask_words, mask_bool);
    if ((rc = launch_check("k_legal")) != 0) return rc;
    if (offsets) {
        hipLaunchKernelGGL(k_scan, dim3(1), dim3(SCAN_THREADS), 0, strm(stream), counts, offsets, e->S.n);
        if ((rc = launch_check("k_scan")) != 0) return rc;
    }
    if (values) {
        if ((rc = csr_fits(e, offsets, values_capacity, strm(stream))) != 0) return rc;
        hipLaunchKernelGGL(k_emit, dim3((e->S.n + 1) / 2), dim3(64), 0, strm(stream), e->S, offsets, values,
                           values_capacity, nullptr);
        if ((rc = launch_check("k_emit")) != 0) return rc;
    }
    return JQ_OK;
}

int jq_legal_slots(jq_env *e, const int8_t *acting, uint8_t *slots, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!slots) return fail(JQ_E_ARG, "null slot mask");
    if ((uintptr_t)slots % 16) return fail(JQ_E_ARG, "slot mask must be 16-byte aligned");
    hipLaunchKernelGGL(k_legal, dim3(e->S.n), dim3(64), 0, strm(stream), e->S, acting, nullptr, nullptr, nullptr);
    if ((rc = launch_check("k_legal")) != 0) return rc;
    hipLaunchKernelGGL(k_slots, dim3(e->S.n), dim3(64), 0, strm(stream), e->S, slots);
    return launch_check("k_slots");
}

int jq_observe(jq_env *e, const int8_t *observer, int32_t fmt, int32_t all_seats, void *spatial, void *aux,
               float *global, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if ((rc = obs_args(e, fmt, spatial, aux, global)) != 0) return rc;
    const int nrows = all_seats ? e->S.n * 4 : e->S.n;
    const dim3 grid(nrows), block(OBS_THREADS);
    const float *x = e->ext_bel;
    if (fmt == JQ_OBS_U8 && (rc = obs_u8_grid(e)) != 0) return rc;
    int f32_pad = 0;
    if (fmt == JQ_OBS_F32 && !e->ext_on && (rc = obs_f32_pad(e, f32_pad)) != 0) return rc;
    hipEvent_t t_end = e->obs_t_end;   // begin already recorded by jq_env_step
    e->obs_t_end = nullptr;
    if (!t_end && (rc = obs_timing_begin(e, stream, &t_end)) != 0) return rc;
    switch (fmt) {
    case JQ_OBS_F32:
        if (e->ext_on)
            hipLaunchKernelGGL((k_observe<0, true>), grid, block, 0, strm(stream), e->S, observer, all_seats, spatial, aux, global, nrows, x);
        else
            hipLaunchKernelGGL((k_observe<0, false>), grid, block, f32_pad, strm(stream), e->S, observer, all_seats, spatial, aux, global, nrows, nullptr);
        break;
    case JQ_OBS_BF16:
        if (e->ext_on)
            hipLaunchKernelGGL((k_observe<1, true>), grid, block, 0, strm(stream), e->S, observer, all_seats, spatial, aux, global, nrows, x);
        else
            hipLaunchKernelGGL((k_observe<1, false>), grid, block, 0, strm(stream), e->S, observer, all_seats, spatial, aux, global, nrows, nullptr);
        break;
    default:
        hipLaunchKernelGGL(k_observe_u8_persist, dim3(std::min(nrows, e->obs_blocks)), dim3(OBS_THREADS), 0,
                           strm(stream), e->S, observer, all_seats, static_cast<uint8_t *>(spatial),
                           static_cast<uint8_t *>(aux), global, nrows);
        break;
    }
    rc = launch_check("k_observe");
    // the end event follows its begin event even when the launch failed, so no
    // later launch is paired with it
    if (t_end) HIP_TRY(hipEventRecord(t_end, strm(stream)));
    return rc;
}

int jq_obs_timing(jq_env *e, int32_t enable)
{
    int rc = check_env(e);
    if (rc) return rc;
    e->obs_timing = enable != 0;
    return JQ_OK;
}

int jq_obs_timing_read(jq_env *e, double *total_ms, int64_t *launches)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!total_ms || !launches) return fail(JQ_E_ARG, "null output");
    double sum = 0.0;
    for (size_t i = 0; i < e->obs_ev_used; ++i) {
        float ms = 0.f;
        HIP_TRY(hipEventSynchronize(e->obs_ev[i].second));
        HIP_TRY(hipEventElapsedTime(&ms, e->obs_ev[i].first, e->obs_ev[i].second));
        sum += ms;
    }
    *total_ms = sum;
    *launches = (int64_t)e->obs_ev_used;
    e->obs_ev_used = 0;
    return JQ_OK;
}

int jq_upload_beliefs(jq_env *e, const void *beliefs, int32_t from_host, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!beliefs) return fail(JQ_E_ARG, "null beliefs");
    const size_t bytes = (size_t)e->S.n * 4 * 12 * NC * sizeof(float);
    if (!e->ext_bel) {
        void *q = nullptr;
        if (hipMalloc(&q, bytes) != hipSuccess) return fail(JQ_E_OOM, "hipMalloc(%zu) for uploaded beliefs failed", bytes);
        e->allocs.push_back(q);
        e->ext_bel = static_cast<float *>(q);
    }
    HIP_TRY(hipMemcpyAsync(e->ext_bel, beliefs, bytes, from_host ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice,
                           strm(stream)));
    e->ext_on = true;
    return JQ_OK;
}

int jq_clear_beliefs(jq_env *e)
{
    int rc = check_env(e);
    if (rc) return rc;
    e->ext_on = false;
    return JQ_OK;
}

int jq_obs_decode_table(float *out)
{
    if (!out) return fail(JQ_E_ARG, "null output");
    std::lock_guard<std::mutex> lk(g_tab_mu);
    build_host_tables();
    std::memcpy(out, g_decode, sizeof g_decode);
    return JQ_OK;
}

int jq_sample_uniform(jq_env *e, const int32_t *counts, const int32_t *offsets, const int32_t *values,
                      int64_t values_capacity, uint64_t seed, uint64_t ply, int32_t *out, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!counts || !offsets || !values || !out) return fail(JQ_E_ARG, "null sampler buffer");
    if (values_capacity < 0) return fail(JQ_E_ARG, "negative values capacity");
    hipLaunchKernelGGL(k_sample, dim3((e->S.n + 255) / 256), dim3(256), 0, strm(stream), e->S.n, counts, offsets,
                       values, values_capacity, seed, ply, out);
    return launch_check("k_sample");
}

int jq_sample_logits(jq_env *e, const int8_t *acting, const int32_t *counts, const int32_t *offsets,
                     const int32_t *values, int64_t values_capacity, uint64_t seed, uint64_t ply, int32_t *out,
                     int32_t *canonical_out, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!counts || !offsets || !values || !out) return fail(JQ_E_ARG, "null sampler buffer");
    if (values_capacity < 0) return fail(JQ_E_ARG, "negative values capacity");
    hipLaunchKernelGGL(k_sample_logits, dim3(e->S.n), dim3(64), 0, strm(stream), e->S, acting, counts, offsets,
                       values, values_capacity, seed, ply, out, canonical_out);
    return launch_check("k_sample_logits");
}

int jq_env_step(jq_env *e, const int32_t *actions, int32_t sampler, uint64_t sample_seed, uint64_t ply,
                int64_t reset_seed, int32_t *counts, int32_t *offsets, int32_t *values, int64_t values_capacity,
                int32_t *mask_words, int32_t obs_fmt, void *spatial, void *aux, float *global, uint8_t *terminated,
                float *reward, uint64_t *hash, int32_t *actions_out, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!counts || !offsets || !values) return fail(JQ_E_ARG, "env_step needs counts, offsets and values");
    if (values_capacity < 0) return fail(JQ_E_ARG, "negative values capacity");
    if (sampler != JQ_SAMPLE_UNIFORM && sampler != JQ_SAMPLE_LOGITS) return fail(JQ_E_ARG, "bad sampler %d", sampler);
    if (!e->zob_ready) return fail(JQ_E_STATE, "upload the Zobrist tables before stepping");
    // the observation's arguments are checked before anything is launched
    if (spatial && (rc = obs_args(e, obs_fmt, spatial, aux, global)) != 0) return rc;
    EnvStepArgs A = {};
    A.actions = actions; A.sampler = sampler; A.sample_seed = sample_seed; A.ply = ply; A.offsets = offsets;
    A.values = values; A.values_cap = values_capacity;
    A.actions_out = actions_out; A.O.term = terminated; A.O.reward = reward; A.O.hash = hash;
    A.do_reset = e->S.pool ? 1 : 0; A.reset_seed = reset_seed; A.counts = counts;
    // The overlapped form moves the CSR pass, and the canonical mask with it,
    // beside the observation (below); the step kernel then skips the mask.
    const bool overlap = spatial && obs_fmt == JQ_OBS_U8 && csr_always_fits(e, values_capacity);
    A.mask_words = overlap ? nullptr : mask_words;
    // sample (unless actions are given), ply, restart from the pool and the
    // next seat's legal sets in one kernel
    hipLaunchKernelGGL(k_env_step, dim3(e->S.n), dim3(64), 0, strm(stream), e->S, A);
    if ((rc = launch_check("k_env_step")) != 0) return rc;
    if (overlap) {
        // The CSR pass (scan + emit, which also builds the canonical mask) reads
        // the legal records and writes offsets / values / mask words; the
        // observation reads the state. Neither touches what the other writes, so
        // the CSR pass runs on a side stream and fills the CUs the persistent
        // observation grid releases as its blocks finish; the caller's stream
        // waits for both before anything it enqueues next.
        if (!e->side) {
            HIP_TRY(hipStreamCreateWithFlags(&e->side, hipStreamNonBlocking));
            HIP_TRY(hipEventCreateWithFlags(&e->ev_step, hipEventDisableTiming));
            HIP_TRY(hipEventCreateWithFlags(&e->ev_csr, hipEventDisableTiming));
        }
        // Each event between two kernels of a stream holds the second back by
        // ≈6 µs, so a timed step's begin event also releases the side stream;
        // an untimed step records the release event alone.
        hipEvent_t t_begin = nullptr;
        if ((rc = obs_timing_begin(e, stream, &e->obs_t_end, &t_begin)) != 0) return rc;
        // Whatever path leaves this block, an end event whose begin was recorded
        // above and that the observation did not take is recorded here, so no
        // later launch pairs with it.
        struct CloseTiming {
            jq_env *e; void *stream;
            ~CloseTiming()
            {
                if (e->obs_t_end) {
                    (void)hipEventRecord(e->obs_t_end, strm(stream));
                    e->obs_t_end = nullptr;
                }
            }
        } close_timing{e, stream};
        if (!t_begin) HIP_TRY(hipEventRecord(e->ev_step, strm(stream)));
        HIP_TRY(hipStreamWaitEvent(e->side, t_begin ? t_begin : e->ev_step, 0));
        hipLaunchKernelGGL(k_scan, dim3(1), dim3(SCAN_THREADS), 0, e->side, counts, offsets, e->S.n);
        if ((rc = launch_check("k_scan")) != 0) return rc;
        hipLaunchKernelGGL(k_emit, dim3((e->S.n + 1) / 2), dim3(64), 0, e->side, e->S, offsets, values,
                           values_capacity, mask_words);
        if ((rc = launch_check("k_emit")) != 0) return rc;
        HIP_TRY(hipEventRecord(e->ev_csr, e->side));
        rc = jq_observe(e, nullptr, obs_fmt, 0, spatial, aux, global, stream);
        HIP_TRY(hipStreamWaitEvent(strm(stream), e->ev_csr, 0));   // joined even if the observation failed
        return rc;
    }
    hipLaunchKernelGGL(k_scan, dim3(1), dim3(SCAN_THREADS), 0, strm(stream), counts, offsets, e->S.n);
    if ((rc = launch_check("k_scan")) != 0) return rc;
    if ((rc = csr_fits(e, offsets, values_capacity, strm(stream))) != 0) return rc;
    hipLaunchKernelGGL(k_emit, dim3((e->S.n + 1) / 2), dim3(64), 0, strm(stream), e->S, offsets, values,
                       values_capacity, nullptr);
    if ((rc = launch_check("k_emit")) != 0) return rc;
    if (spatial && (rc = jq_observe(e, nullptr, obs_fmt, 0, spatial, aux, global, stream)) != 0) return rc;
    return JQ_OK;
}

int jq_field_info(int32_t f, int32_t *elems, int32_t *bytes)
{
    if (f < 0 || f >= JQ_F_COUNT) return fail(JQ_E_ARG, "bad field %d", f);
    if (elems) *elems = kFields[f].elems;
    if (bytes) *bytes = kFields[f].bytes;
    return JQ_OK;
}

int jq_get_field(jq_env *e, int32_t f, void *host)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (f < 0 || f >= JQ_F_COUNT || !host) return fail(JQ_E_ARG, "bad field %d", f);
    const FieldDesc &d = kFields[f];
    const size_t n = (size_t)e->S.n;
    std::vector<uint8_t> tmp(n * d.env_stride);
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(tmp.data(), field_array(e, d.arr), tmp.size(), hipMemcpyDeviceToHost));
    uint8_t *out = static_cast<uint8_t *>(host);
    for (size_t i = 0; i < n; ++i)
        for (int j = 0; j < d.elems; ++j)
            std::memcpy(out + (i * d.elems + j) * d.bytes, tmp.data() + i * d.env_stride + j * d.el_stride + d.off,
                        d.bytes);
    return JQ_OK;
}

int jq_set_field(jq_env *e, int32_t f, const void *host)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (f < 0 || f >= JQ_F_COUNT || !host) return fail(JQ_E_ARG, "bad field %d", f);
    const FieldDesc &d = kFields[f];
    const size_t n = (size_t)e->S.n;
    std::vector<uint8_t> tmp(n * d.env_stride);
    HIP_TRY(hipDeviceSynchronize());
    uint8_t *base = field_array(e, d.arr);
    HIP_TRY(hipMemcpy(tmp.data(), base, tmp.size(), hipMemcpyDeviceToHost));
    const uint8_t *in = static_cast<const uint8_t *>(host);
    for (size_t i = 0; i < n; ++i)
        for (int j = 0; j < d.elems; ++j)
            std::memcpy(tmp.data() + i * d.env_stride + j * d.el_stride + d.off, in + (i * d.elems + j) * d.bytes,
                        d.bytes);
    HIP_TRY(hipMemcpy(base, tmp.data(), tmp.size(), hipMemcpyHostToDevice));
    return JQ_OK;
}

int jq_field_ptr(jq_env *e, int32_t f, void **ptr, int64_t *env_stride, int64_t *el_stride)
{
    if (!e || !ptr || f < 0 || f >= JQ_F_COUNT) return fail(JQ_E_ARG, "bad field %d", f);
    const FieldDesc &d = kFields[f];
    *ptr = field_array(e, d.arr) + d.off;
    if (env_stride) *env_stride = (int64_t)d.env_stride;
    if (el_stride) *el_stride = (int64_t)d.el_stride;
    return JQ_OK;
}

int jq_finalize_import(jq_env *e, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!e->zob_ready) return fail(JQ_E_STATE, "upload the Zobrist tables first");
    hipLaunchKernelGGL(k_finalize, dim3(e->S.n), dim3(64), 0, strm(stream), e->S, 1, nullptr);
    if ((rc = launch_check("k_finalize")) != 0) return rc;
    HIP_TRY(hipStreamSynchronize(strm(stream)));
    return JQ_OK;
}

int jq_finalize_import_masked(jq_env *e, const uint8_t *env_mask, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!env_mask) return fail(JQ_E_ARG, "null env mask");
    if (!e->zob_ready) return fail(JQ_E_STATE, "upload the Zobrist tables first");
    hipLaunchKernelGGL(k_finalize, dim3(e->S.n), dim3(64), 0, strm(stream), e->S, 1, env_mask);
    if ((rc = launch_check("k_finalize")) != 0) return rc;
    HIP_TRY(hipStreamSynchronize(strm(stream)));
    return JQ_OK;
}

int jq_rehash(jq_env *e, void *stream)
{
    int rc = check_env(e);
    if (rc) return rc;
    if (!e->zob_ready) return fail(JQ_E_STATE, "upload the Zobrist tables first");
    hipLaunchKernelGGL(k_finalize, dim3(e->S.n), dim3(64), 0, strm(stream), e->S, 0, nullptr);
    return launch_check("k_finalize");
}

// ---------------------------------------------------------------- history
int jq_history_create(jq_history **out, int32_t num_envs, int32_t num_steps, int32_t show_mode, int32_t device)
{
    if (!out) return fail(JQ_E_ARG, "out is null");
    *out = nullptr;
    if (num_envs <= 0 || num_envs > (1 << 24)) return fail(JQ_E_ARG, "num_envs %d out of range", num_envs);
    if (num_steps <= 0) return fail(JQ_E_ARG, "num_steps must be positive, got %d", num_steps);
    if ((int64_t)num_envs * num_steps > ((int64_t)1 << 31)) return fail(JQ_E_ARG, "num_steps * num_envs too large");
    if (show_mode < 0 || show_mode > 2) return fail(JQ_E_ARG, "show_mode %d not in {0,1,2}", show_mode);
    int ndev = 0;
    HIP_TRY(hipGetDeviceCount(&ndev));
    if (device < 0 || device >= ndev) return fail(JQ_E_ARG, "device %d not present (%d devices)", device, ndev);
    HIP_TRY(hipSetDevice(device));
    jq_history *h = new jq_history();
    h->device = device;
    h->show_mode = show_mode;
    HistState &H = h->H;
    H.steps = num_steps; H.n = num_envs;
    const size_t R = (size_t)num_steps * num_envs;
    int rc;
#define A(ptr, cnt) do { if ((rc = halloc(h, ptr, cnt)) != 0) { jq_history_destroy(h); return rc; } } while (0)
    A(H.cell, R * CELL_STRIDE);
    A(H.piece, R * PID_STRIDE);
    A(H.cm, R * 4 * PID_STRIDE);
    A(H.cme, R * 4 * PID_STRIDE);
    A(H.bcode, R * 4 * PID_STRIDE);
    A(H.rem, R * 4 * 48);
    A(H.env, R);
    A(H.hist, R * HIST_LEN);
    A(h->rlut, 4 * 4096);
#undef A
    *out = h;
    return JQ_OK;
}

int jq_history_destroy(jq_history *h)
{
    if (!h) return JQ_OK;
    (void)hipSetDevice(h->device);
    if (h->replay) jq_destroy(h->replay);
    for (void *p : h->allocs) (void)hipFree(p);
    delete h;
    return JQ_OK;
}

int jq_history_bytes(const jq_history *h, int64_t *bytes)
{
    if (!h || !bytes) return fail(JQ_E_ARG, "null argument");
    *bytes = (int64_t)h->H.steps * h->H.n * (int64_t)HIST_ROW_BYTES;
    return JQ_OK;
}

int jq_history_snapshot(jq_history *h, jq_env *e, const int8_t *acting, int32_t step, void *stream)
{
    (void)acting;
    if (!h || !e) return fail(JQ_E_ARG, "null handle");
    const HistState &H = h->H;
    if (e->S.n != H.n) return fail(JQ_E_ARG, "history/state num_envs mismatch (%d vs %d)", H.n, e->S.n);
    if (e->device != h->device) return fail(JQ_E_ARG, "history and state live on different devices");
    if (e->S.show_mode != h->show_mode) return fail(JQ_E_ARG, "history and state show modes differ");
    if (step < 0 || step >= H.steps) return fail(JQ_E_ARG, "history snapshot step %d out of range [0, %d)", step, H.steps);
    if (!e->rlut_ready) return fail(JQ_E_STATE, "recency table not uploaded to the state handle");
    HIP_TRY(hipSetDevice(h->device));
    hipStream_t s = strm(stream);
    const size_t n = (size_t)H.n, r0 = (size_t)step * n;
    const State &S = e->S;
    HIP_TRY(hipMemcpyAsync(H.cell + r0 * CELL_STRIDE, S.cell, n * CELL_STRIDE, hipMemcpyDeviceToDevice, s));
    HIP_TRY(hipMemcpyAsync(H.piece + r0 * PID_STRIDE, S.piece, n * PID_STRIDE * sizeof(PieceRec), hipMemcpyDeviceToDevice, s));
    HIP_TRY(hipMemcpyAsync(H.cm + r0 * 4 * PID_STRIDE, S.cm, n * 4 * PID_STRIDE * sizeof(CmRec), hipMemcpyDeviceToDevice, s));
    HIP_TRY(hipMemcpyAsync(H.cme + r0 * 4 * PID_STRIDE, S.cme, n * 4 * PID_STRIDE * sizeof(CmEat), hipMemcpyDeviceToDevice, s));
    HIP_TRY(hipMemcpyAsync(H.bcode + r0 * 4 * PID_STRIDE, S.bcode, n * 4 * PID_STRIDE, hipMemcpyDeviceToDevice, s));
    HIP_TRY(hipMemcpyAsync(H.rem + r0 * 4 * 48, S.rem, n * 4 * 48, hipMemcpyDeviceToDevice, s));
    HIP_TRY(hipMemcpyAsync(H.env + r0, S.env, n * sizeof(EnvRec), hipMemcpyDeviceToDevice, s));
    HIP_TRY(hipMemcpyAsync(H.hist + r0 * HIST_LEN, S.hist, n * HIST_LEN * sizeof(int32_t), hipMemcpyDeviceToDevice, s));
    if (!h->rlut_ready) {
        HIP_TRY(hipMemcpyAsync(h->rlut, S.rlut, 4 * 4096 * sizeof(float), hipMemcpyDeviceToDevice, s));
        h->rlut_ready = true;
    }
    h->max_moves = S.max_moves;
    return JQ_OK;
}

int jq_history_reconstruct(jq_history *h, const int64_t *flat, const int8_t *observer, int32_t batch, int32_t fmt,
                           void *spatial, void *aux, float *global, int32_t *mask_words, uint8_t *mask_bool,
                           void *stream)
{
    if (!h) return fail(JQ_E_ARG, "null history");
    if (batch <= 0) return fail(JQ_E_ARG, "cannot reconstruct an empty history minibatch");
    if (!flat || !observer) return fail(JQ_E_ARG, "history reconstruction received a null device pointer");
    if (!h->rlut_ready) return fail(JQ_E_STATE, "history has no snapshot yet");
    HIP_TRY(hipSetDevice(h->device));
    int rc;
    if (h->replay_cap < batch) {   // scratch rows, grown to the largest batch seen
        if (h->replay) { jq_destroy(h->replay); h->replay = nullptr; h->replay_cap = 0; }
        if ((rc = jq_create(&h->replay, batch, std::max(1, h->max_moves), h->show_mode, h->device)) != 0) return rc;
        h->replay_cap = batch;
    }
    jq_env *R = h->replay;
    R->S.n = batch;
    R->S.rlut = h->rlut;
    R->rlut_ready = true;
    hipLaunchKernelGGL(k_history_gather, dim3(batch), dim3(256), 0, strm(stream), h->H, flat, batch, R->S);
    if ((rc = launch_check("k_history_gather")) != 0) return rc;
    if (spatial || aux || global) {
        if (!spatial || !global) return fail(JQ_E_ARG, "spatial and global outputs go together");
        if ((rc = jq_observe(R, observer, fmt, 0, spatial, aux, global, stream)) != 0) return rc;
    }
    if (mask_words || mask_bool)
        if ((rc = jq_legal(R, observer, nullptr, nullptr, nullptr, 0, mask_words, mask_bool, stream)) != 0) return rc;
    return JQ_OK;
}

// ------------------------------------------------ history rebuild without allocation
// Rebuild-only state for jq_history_reconstruct_noalloc: the arrays the gather,
// the observation and the legal masks touch, for at most JQ_NOALLOC_MAX_ROWS
// rows, carved from one file-scope device array (no full combat-memory
// records: the rebuild reads only their summaries, views and eaten-by sets).
// 20,948 bytes per row, 21.45 MB in all on each device the library runs on.
namespace {
constexpr size_t NA_ROWS = JQ_NOALLOC_MAX_ROWS;
constexpr size_t na_up(size_t x) { return (x + 255) & ~size_t(255); }
constexpr size_t NA_CELL = 0;
constexpr size_t NA_PIECE = NA_CELL + na_up(NA_ROWS * CELL_STRIDE);
constexpr size_t NA_CME = NA_PIECE + na_up(NA_ROWS * PID_STRIDE * sizeof(PieceRec));
constexpr size_t NA_CMK = NA_CME + na_up(NA_ROWS * 4 * PID_STRIDE * sizeof(CmEat));
constexpr size_t NA_CMV = NA_CMK + na_up(NA_ROWS * 4 * PID_STRIDE);
constexpr size_t NA_BCODE = NA_CMV + na_up(NA_ROWS * 4 * PID_STRIDE * sizeof(CmView));
constexpr size_t NA_REM = NA_BCODE + na_up(NA_ROWS * 4 * PID_STRIDE);
constexpr size_t NA_ENV = NA_REM + na_up(NA_ROWS * 4 * 48);
constexpr size_t NA_HIST = NA_ENV + na_up(NA_ROWS * sizeof(EnvRec));
constexpr size_t NA_LG = NA_HIST + na_up(NA_ROWS * HIST_LEN * sizeof(int32_t));
constexpr size_t NA_BYTES = NA_LG + na_up(NA_ROWS * sizeof(LegalRec));
}  // namespace

static __device__ __align__(256) uint8_t scratch[NA_BYTES];

namespace {
std::mutex g_na_mu;
uint8_t *g_na_ptr[64] = {};    // device address of `scratch` on each device
jq_env g_na_env[64];           // host view of each device's rebuild state

// Per device, once: the device address of `scratch` (the array's name is a
// host-side stand-in and must never reach a kernel) and the state over it.
int noalloc_state(int device, jq_env *&out)
{
    std::lock_guard<std::mutex> lk(g_na_mu);
    if (device < 0 || device >= 64) return fail(JQ_E_ARG, "device %d out of range", device);
    if (!g_na_ptr[device]) {
        int rc = ensure_device_tables(device);
        if (rc) return rc;
        void *p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !p)
            return fail(JQ_E_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(err));
        uint8_t *b = static_cast<uint8_t *>(p);
        jq_env &e = g_na_env[device];
        e.device = device;
        State &S = e.S;
        S.cell = reinterpret_cast<int8_t *>(b + NA_CELL);
        S.piece = reinterpret_cast<PieceRec *>(b + NA_PIECE);
        S.cm = nullptr;
        S.cme = reinterpret_cast<CmEat *>(b + NA_CME);
        S.cmk = b + NA_CMK;
        S.cmv = reinterpret_cast<CmView *>(b + NA_CMV);
        S.bcode = b + NA_BCODE;
        S.rem = reinterpret_cast<int8_t *>(b + NA_REM);
        S.env = reinterpret_cast<EnvRec *>(b + NA_ENV);
        S.hist = reinterpret_cast<int32_t *>(b + NA_HIST);
        S.lg = reinterpret_cast<LegalRec *>(b + NA_LG);
        S.ztab = nullptr;
        S.pool = nullptr;
        S.pool_size = 0;
        g_na_ptr[device] = b;
    }
    out = &g_na_env[device];
    return JQ_OK;
}
}  // namespace

extern "C" int jq_history_reconstruct_noalloc(jq_history *h, const int64_t *flat, const int8_t *observer,
                                              int32_t batch, int32_t fmt, void *spatial, void *aux, float *global,
                                              int32_t *mask_words, uint8_t *mask_bool, void *stream)
{
    if (!h) return fail(JQ_E_ARG, "null history");
    if (batch <= 0) return fail(JQ_E_ARG, "cannot reconstruct an empty history minibatch");
    if (batch > JQ_NOALLOC_MAX_ROWS)
        return fail(JQ_E_ARG, "batch %d exceeds the %d rows jq_history_reconstruct_noalloc holds", batch,
                    JQ_NOALLOC_MAX_ROWS);
    if (!flat || !observer) return fail(JQ_E_ARG, "history reconstruction received a null device pointer");
    if (!h->rlut_ready) return fail(JQ_E_STATE, "history has no snapshot yet");
    HIP_TRY(hipSetDevice(h->device));
    jq_env *R = nullptr;
    int rc = noalloc_state(h->device, R);
    if (rc) return rc;
    R->S.n = batch;
    R->S.max_moves = std::max(1, h->max_moves);
    R->S.show_mode = h->show_mode;
    R->S.rlut = h->rlut;
    R->rlut_ready = true;
    R->zob_ready = false;
    R->ext_on = false;
    hipLaunchKernelGGL(k_history_gather, dim3(batch), dim3(256), 0, strm(stream), h->H, flat, batch, R->S);
    if ((rc = launch_check("k_history_gather")) != 0) return rc;
    if (spatial || aux || global) {
        if (!spatial || !global) return fail(JQ_E_ARG, "spatial and global outputs go together");
        if ((rc = jq_observe(R, observer, fmt, 0, spatial, aux, global, stream)) != 0) return rc;
    }
    if (mask_words || mask_bool)
        if ((rc = jq_legal(R, observer, nullptr, nullptr, nullptr, 0, mask_words, mask_bool, stream)) != 0) return rc;
    return JQ_OK;
}

// ---------------------------------------------------------------- masks
int jq_mask_count(const uint8_t *mask, int32_t n, int32_t d, int32_t *counts, void *stream)
{
    if (!mask || !counts) return fail(JQ_E_ARG, "null device pointer");
    if (n < 0 || d <= 0) return fail(JQ_E_ARG, "bad mask shape (%d, %d)", n, d);
    if (n == 0) return JQ_OK;
    hipLaunchKernelGGL(k_mask_count, dim3(n), dim3(64), 0, strm(stream), mask, n, d, counts);
    return launch_check("k_mask_count");
}

int jq_mask_to_ids(const uint8_t *mask, int32_t n, int32_t d, int32_t k_max, int32_t *ids, void *stream)
{
    if (!mask || !ids) return fail(JQ_E_ARG, "null device pointer");
    if (n < 0 || d <= 0 || k_max <= 0) return fail(JQ_E_ARG, "bad shapes (n %d, d %d, k_max %d)", n, d, k_max);
    if (n == 0) return JQ_OK;
    hipLaunchKernelGGL(k_mask_to_ids, dim3(n), dim3(64), 0, strm(stream), mask, n, d, k_max, ids);
    return launch_check("k_mask_to_ids");
}

int jq_ids_to_mask(const int32_t *ids, const int32_t *counts, int64_t rows, int32_t k_max, const int64_t *idx,
                   int32_t batch, int32_t d, uint8_t *out, void *stream)
{
    if (!ids || !counts || !idx || !out) return fail(JQ_E_ARG, "null device pointer");
    if (rows < 0 || k_max <= 0 || batch < 0 || d <= 0)
        return fail(JQ_E_ARG, "bad shapes (rows %lld, k_max %d, batch %d, d %d)", (long long)rows, k_max, batch, d);
    if (batch == 0) return JQ_OK;
    hipLaunchKernelGGL(k_ids_to_mask, dim3(batch), dim3(256), 0, strm(stream), ids, counts, rows, k_max, idx, batch, d,
                       out);
    return launch_check("k_ids_to_mask");
}

int jq_sync(void *stream)
{
    HIP_TRY(hipStreamSynchronize(strm(stream)));
    return JQ_OK;
}

}  // extern "C"

// Compact rollout history: every per-env state block of a handle, one copy per
// rollout step, and the gather that rebuilds a batch of (step, env) rows as a
// state from which observations and legal masks are produced again
// (src/env/cuda/src/rollout_history.cu:160-525 keeps the same pre-action state
// per step and rebuilds PPO minibatches from it).
//
// Included into jq_lib.hip's translation unit.
#pragma once

namespace jq {

// Per-env bytes of one history row: board, piece records, all four observers'
// combat memory (records and eaten-by sets; the summary bytes are derived on
// gather) and belief codes, remaining counts, env record, move ring.
constexpr size_t HIST_ROW_BYTES = CELL_STRIDE + PID_STRIDE * sizeof(PieceRec) +
                                  4 * PID_STRIDE * (sizeof(CmRec) + sizeof(CmEat)) + 4 * PID_STRIDE + 4 * 48 +
                                  sizeof(EnvRec) + HIST_LEN * sizeof(int32_t);

// History arrays, row r = step * n + env, each laid out like the State array
// of the same name.
struct HistState {
    int32_t steps, n;
    int8_t *cell;
    PieceRec *piece;
    CmRec *cm;
    CmEat *cme;
    uint8_t *bcode;
    int8_t *rem;
    EnvRec *env;
    int32_t *hist;
};

template <class T>
__device__ __forceinline__ void copy_words(T *__restrict__ dst, const T *__restrict__ src, int count, int t, int nt)
{
    for (int k = t; k < count; k += nt) dst[k] = src[k];
}

// Row i of R <- history row flat[i]; rows outside [0, steps * n) become the
// empty terminated state. One 256-thread block per row, 16-byte copies where
// the blocks allow (the 292-byte board moves in 4-byte words). A state with no
// full combat-memory records (R.cm null) gets only the summaries, views and
// eaten-by sets that observations and legal masks read.
__global__ __launch_bounds__(256) void k_history_gather(HistState H, const int64_t *__restrict__ flat, int batch, State R)
{
    const int i = blockIdx.x, t = threadIdx.x;
    if (i >= batch) return;
    const int64_t f = flat[i];
    if (f < 0 || f >= (int64_t)H.steps * H.n) {
        clear_env(R, i, t, 256);
        return;
    }
    copy_words(reinterpret_cast<uint32_t *>(R.cell + (size_t)i * CELL_STRIDE),
               reinterpret_cast<const uint32_t *>(H.cell + (size_t)f * CELL_STRIDE), CELL_STRIDE / 4, t, 256);
    copy_words(reinterpret_cast<uint4 *>(R.piece + (size_t)i * PID_STRIDE),
               reinterpret_cast<const uint4 *>(H.piece + (size_t)f * PID_STRIDE), PID_STRIDE, t, 256);
    if (R.cm)
        copy_words(reinterpret_cast<uint4 *>(R.cm + (size_t)i * 4 * PID_STRIDE),
                   reinterpret_cast<const uint4 *>(H.cm + (size_t)f * 4 * PID_STRIDE),
                   4 * PID_STRIDE * (int)(sizeof(CmRec) / 16), t, 256);
    copy_words(reinterpret_cast<uint4 *>(R.cme + (size_t)i * 4 * PID_STRIDE),
               reinterpret_cast<const uint4 *>(H.cme + (size_t)f * 4 * PID_STRIDE), 4 * PID_STRIDE, t, 256);
    for (int k = t; k < 4 * PID_STRIDE; k += 256) {   // summaries and views are not stored: derive them
        const CmRec c = H.cm[(size_t)f * 4 * PID_STRIDE + k];
        R.cmk[(size_t)i * 4 * PID_STRIDE + k] = cm_summary(c);
        R.cmv[(size_t)i * 4 * PID_STRIDE + k] = cm_view(c, k / PID_STRIDE);
    }
    copy_words(reinterpret_cast<uint4 *>(R.bcode + (size_t)i * 4 * PID_STRIDE),
               reinterpret_cast<const uint4 *>(H.bcode + (size_t)f * 4 * PID_STRIDE), 4 * PID_STRIDE / 16, t, 256);
    copy_words(reinterpret_cast<uint4 *>(R.rem + (size_t)i * 4 * 48),
               reinterpret_cast<const uint4 *>(H.rem + (size_t)f * 4 * 48), 4 * 48 / 16, t, 256);
    copy_words(reinterpret_cast<uint4 *>(R.env + i), reinterpret_cast<const uint4 *>(H.env + f), 2, t, 256);
    copy_words(reinterpret_cast<uint4 *>(R.hist + (size_t)i * HIST_LEN),
               reinterpret_cast<const uint4 *>(H.hist + (size_t)f * HIST_LEN), HIST_LEN / 4, t, 256);
}

}  // namespace jq

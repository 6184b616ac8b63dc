// Dense bool masks <-> per-row id lists, for rollout buffers that keep the
// legal support as ids (junqi_rl/training/rollout_gpu.py:119-198).
//
// Included into jq_lib.hip's translation unit.
#pragma once

namespace jq {

// Nonzero-byte bits of a 16-byte word (bit k = byte k != 0).
__device__ __forceinline__ uint32_t nz_bytes(uint4 v)
{
    uint32_t m = 0;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int b = 0; b < 4; ++b) m |= (((w[i] >> (8 * b)) & 0xFFu) != 0u ? 1u : 0u) << (4 * i + b);
    return m;
}

// Walk one mask row [base, base + d) in column order, one wave: the bytes up
// to the first 16-byte boundary, whole 16-byte words (64 per step), then the
// tail bytes. f(col, nzbits, nbits) is called by every lane for its piece of
// each step (nbits = 0 for no data), so a caller can take wave prefix sums.
template <class F>
__device__ __forceinline__ void mask_row_walk(const uint8_t *base, int d, F &&f)
{
    const int l = threadIdx.x & 63;
    const uintptr_t b0 = reinterpret_cast<uintptr_t>(base);
    const int head = (int)(min((uintptr_t)d, ((b0 + 15) & ~(uintptr_t)15) - b0));
    const int body = (d - head) / 16;
    {   // head bytes, one lane each
        const bool on = l < head && base[l] != 0;
        f(0, on ? 1u << l : 0u, l < head ? 1 : 0, l);
    }
    const uint4 *w = reinterpret_cast<const uint4 *>(base + head);
    for (int q0 = 0; q0 < body; q0 += 64) {
        const int q = q0 + l;
        const uint32_t m = q < body ? nz_bytes(w[q]) : 0u;
        f(head + 16 * q, m, q < body ? 16 : 0, -1);
    }
    const int t0 = head + 16 * body, tail = d - t0;
    {
        const bool on = l < tail && base[t0 + l] != 0;
        f(t0, on ? 1u << l : 0u, l < tail ? 1 : 0, l);
    }
}

__device__ __forceinline__ int wave_excl(int v, int &total)
{
    const int l = threadIdx.x & 63;
    int incl = v;
    for (int o = 1; o < 64; o <<= 1) { const int u = __shfl_up(incl, o); if (l >= o) incl += u; }
    total = __shfl(incl, 63);
    return incl - v;
}

// counts[r] = nonzero bytes of row r. One wave per row.
__global__ __launch_bounds__(64) void k_mask_count(const uint8_t *__restrict__ mask, int n, int d,
                                                   int32_t *__restrict__ counts)
{
    const int r = blockIdx.x;
    if (r >= n) return;
    int c = 0;
    mask_row_walk(mask + (size_t)r * d, d, [&](int, uint32_t m, int, int) { c += __popc(m); });
    c = wave_sum(c);
    if ((threadIdx.x & 63) == 0) counts[r] = c;
}

// ids[r][0 .. counts[r]) = the nonzero columns of row r in order, the rest of
// the row 0. The caller has checked counts[r] <= k_max. One wave per row.
__global__ __launch_bounds__(64) void k_mask_to_ids(const uint8_t *__restrict__ mask, int n, int d, int k_max,
                                                    int32_t *__restrict__ ids)
{
    const int r = blockIdx.x;
    if (r >= n) return;
    int32_t *out = ids + (size_t)r * k_max;
    int run = 0;
    mask_row_walk(mask + (size_t)r * d, d, [&](int col0, uint32_t m, int, int lane_byte) {
        int tot;
        const int at = run + wave_excl(__popc(m), tot);
        int k = 0;
        for (uint32_t x = m; x; x &= x - 1, ++k) {
            const int b = __builtin_ctz(x);
            // single-byte pieces put the lane's bit at its lane index
            out[at + k] = lane_byte >= 0 ? col0 + lane_byte : col0 + b;
        }
        run += tot;
    });
    for (int j = run + (int)(threadIdx.x & 63); j < k_max; j += 64) out[j] = 0;
}

// out[b] = dense bool row of the id list of row idx[b] (counts[idx[b]] ids of
// ids[idx[b]]); ids outside [0, d) and rows outside [0, rows) contribute
// nothing. One 256-thread block per output row.
__global__ __launch_bounds__(256) void k_ids_to_mask(const int32_t *__restrict__ ids, const int32_t *__restrict__ counts,
                                                     int64_t rows, int k_max, const int64_t *__restrict__ idx, int batch,
                                                     int d, uint8_t *__restrict__ out)
{
    const int b = blockIdx.x, t = threadIdx.x;
    if (b >= batch) return;
    uint8_t *row = out + (size_t)b * d;
    const uintptr_t b0 = reinterpret_cast<uintptr_t>(row);
    const int head = (int)(min((uintptr_t)d, ((b0 + 15) & ~(uintptr_t)15) - b0));
    const int body = (d - head) / 16;
    for (int i = t; i < head; i += 256) row[i] = 0;
    uint4 *w = reinterpret_cast<uint4 *>(row + head);
    for (int q = t; q < body; q += 256) w[q] = make_uint4(0, 0, 0, 0);
    for (int i = head + 16 * body + t; i < d; i += 256) row[i] = 0;
    __syncthreads();
    const int64_t src = idx[b];
    if (src < 0 || src >= rows) return;
    const int cnt = min(counts[src], k_max);
    for (int j = t; j < cnt; j += 256) {
        const int c = ids[(size_t)src * k_max + j];
        if (c >= 0 && c < d) row[c] = 1;
    }
}

}  // namespace jq

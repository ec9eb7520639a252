// Precision guard of the e4m3-MFMA history kernels: the V statistics that
// set each KV head's row threshold, and the merge of the BF16 fixup's split
// partials.
//
// A row's output error from rounding Q and P to e4m3 is a probability-
// weighted sum of relative roundings times the spread of the V values the
// row averages, so it grows as sigma_V / sqrt(W) with W = sum_k 2^(x_k - m)
// the row's probability mass (the effective number of keys, up to a factor
// 2^2.5).  The threshold of KV head h is therefore
//     PCPA_GUARD_MIN_MASS * v_scale^2 * max_d Var_k(V[h, k, d])
// (the variance over the head's valid history keys, per channel d, of the
// e4m3 V codes, times v_scale^2): 384 for unit-variance V, 16 x 384 for V
// of standard deviation 4.  A guarded launch runs, in order:
//   guard_vstats_kernel  the thresholds; zeroes the guard plan's row counts;
//   the e4m3 pass        (one pass) appends each row below its head's
//                        threshold to the guard plan (common.hpp);
//   merge_splits_kernel  (split launch) appends them instead;
//   the BF16 fixup       history_fwd_kernel<..., FIXUP> over the listed rows,
//                        gathered into groups of 128 (the BF16 tile kernel's
//                        4 waves x 32 rows);
//   guard_merge_kernel   the merge of the fixup's range partials.
// Rows are appended by device atomics, in an order that depends on timing,
// which a row's fixup result does not.  Few groups: sparse mode, where the
// fixup splits each group's history walk over as many workgroups as the
// partials hold (guard_ranges) and guard_merge_kernel combines the ranges;
// more: dense mode, one workgroup per group, writing the output directly.
// With no flagged row every fixup and merge workgroup exits at once.
#pragma once

#include "common.hpp"

namespace pcpa {

// KV heads a guard plan handles (the guarded launch is refused beyond).
constexpr int kGuardMaxHeads = 64;
// Capacity of the sparse partials, in query rows over all history ranges:
// [ranges, groups * 128] FP32 rows of D + 1 values (34 MB at head_dim 256).
constexpr int64_t kGuardPartialRows = 32768;

// Sparse mode: the listed rows' range partials ([ranges, listed * 128, D]
// rows in slot order, guard_ranges()) merged by log-sum-exp (as
// merge_splits_kernel) into out (bf16) and lse; workgroup b takes slot rows
// b, b + gridDim.x, ... .  Thread t takes 8 consecutive d (t % d_vec8) of
// the ranges t / d_vec8, t / d_vec8 + groups, ... (at most kGuardMergePer:
// the host caps ranges at 64, and groups >= 8), loads all their log-sum-exps and partials
// at once and sums them against its own largest log-sum-exp; the groups'
// sums meet in LDS, rescaled to the row's largest.  Dense mode: nothing.
constexpr int kGuardMergeThreads = 256;
constexpr int kGuardMergeGroups = 512;  // workgroups of guard_merge_kernel
constexpr int kGuardMergePer = 8;       // ranges per thread at most

__global__ void __launch_bounds__(kGuardMergeThreads) guard_merge_kernel(const float* part_o, const float* part_lse,
                                                                         const int32_t* plan, GuardShape g,
                                                                         int d_vec8, uint8_t* out, float* lse_out) {
    __shared__ float red[kGuardMergeThreads * 8];
    __shared__ float wred[kGuardMergeThreads];
    __shared__ float mred[kGuardMergeThreads];
    const int listed = guard_groups(plan, g.num_kv_heads);
    const int ranges = guard_ranges(listed, g.partial_rows, g.max_ranges);
    if (ranges == 0) return;
    const int64_t stride = (int64_t)listed * kRowsPerGroup;  // rows of one range's partials
    const int D = d_vec8 * 8;
    const int tid = threadIdx.x;
    const int groups = kGuardMergeThreads / d_vec8;  // d_vec8 divides 256 (D = 64, 128, 256)
    const int sg = tid / d_vec8;
    const int d0 = (tid - sg * d_vec8) * 8;
    for (int64_t slot_row = blockIdx.x; slot_row < stride; slot_row += gridDim.x) {
        const int slot = (int)(slot_row / kRowsPerGroup);
        const GuardGroup gg = guard_group(plan, g.num_kv_heads, slot);
        const int idx = gg.first + (int)(slot_row - (int64_t)slot * kRowsPerGroup);
        if (idx >= gg.count) continue;  // the same for the whole workgroup
        float lk[kGuardMergePer];
        v4f lo[kGuardMergePer], hi[kGuardMergePer];
#pragma unroll
        for (int k = 0; k < kGuardMergePer; ++k) {
            const int sp = sg + k * groups;
            lk[k] = -INFINITY;
            lo[k] = hi[k] = v4f{0.f, 0.f, 0.f, 0.f};
            if (sp < ranges) {
                lk[k] = part_lse[sp * stride + slot_row];
                const float* const src = part_o + (sp * stride + slot_row) * D + d0;
                lo[k] = *(const v4f*)src;
                hi[k] = *(const v4f*)(src + 4);
            }
        }
        const int r = plan[guard_list_offset(g.num_kv_heads) + gg.head * guard_head_segment(g.rows_per_head) + idx];
        const int64_t row = guard_row_index(g, gg.head, r);
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < kGuardMergePer; ++k) mx = fmaxf(mx, lk[k]);
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        float wsum = 0.f;
#pragma unroll
        for (int k = 0; k < kGuardMergePer; ++k) {
            const float w = lk[k] == -INFINITY ? 0.f : __expf(lk[k] - mx);
            wsum += w;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc[i] = fmaf(w, lo[k][i], acc[i]);
                acc[4 + i] = fmaf(w, hi[k][i], acc[4 + i]);
            }
        }
        __syncthreads();  // the previous row's sums are read
#pragma unroll
        for (int i = 0; i < 8; ++i) red[tid * 8 + i] = acc[i];
        wred[tid] = wsum;
        mred[tid] = mx;
        __syncthreads();
        if (sg == 0) {
            float m = mx;
            for (int o = 1; o < groups; ++o) m = fmaxf(m, mred[o * d_vec8 + tid]);
            float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            float ws = 0.f;
            for (int o = 0; o < groups; ++o) {
                const int t = o * d_vec8 + tid;
                const float mo = mred[t];
                if (mo == -INFINITY) continue;  // no range of this group has valid keys
                const float f = __expf(mo - m);
#pragma unroll
                for (int i = 0; i < 8; ++i) sum[i] = fmaf(f, red[t * 8 + i], sum[i]);
                ws = fmaf(f, wred[t], ws);
            }
            const float inv = ws > 0.f ? 1.f / ws : 0.f;
            uint32_t wv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const __bf16 x0 = (__bf16)(sum[2 * i] * inv), x1 = (__bf16)(sum[2 * i + 1] * inv);
                wv[i] = (uint32_t)__builtin_bit_cast(uint16_t, x0) | ((uint32_t)__builtin_bit_cast(uint16_t, x1) << 16);
            }
            *(v4i*)(out + (row * D + d0) * 2) = v4i{(int)wv[0], (int)wv[1], (int)wv[2], (int)wv[3]};
            if (lse_out && d0 == 0) lse_out[row] = ws > 0.f ? m + __logf(ws) : -INFINITY;
        }
    }
}


// ---- V statistics and the guard threshold -------------------------------
//
// guard_vstats_kernel: workgroup (KV head h, 16-byte chunk c of a V row)
// sums, for chunk c's 16 channels, the sampled V codes of head h's walk
// (times 2^9) and their squares (times 2^18), and stores
// PCPA_GUARD_MIN_MASS * v_scale^2 times the largest of the 16 variances in
// thr[h * D / 16 + c]; guard_threshold() takes the largest of a head's
// chunks.  A chunk's sums are one workgroup's, so nothing is combined
// across workgroups (no atomics, nothing to zero first).  Every e4m3 value
// is a multiple of 2^-9 of magnitude at most 448: each thread sums its few
// keys' codes (exact) and squares in fp32 over a fixed set of keys, the
// sums are rounded to the fixed-point units and added as integers, so the
// thresholds are the same on every run.
constexpr int kVStatsThreads = 256;
// Keys per KV head the statistics sample at most (every s-th key of each
// page, s the smallest power of two that keeps the walk's valid keys / s
// within it; all keys of a shorter history).
constexpr int kVStatsKeys = 2048;
// Table entries staged in LDS at a time, and the 16-byte loads a thread
// keeps in flight (a sampled walk's kVStatsKeys keys are 8 a thread).
constexpr int kVStatsEntries = 1024;
constexpr int kVStatsBatch = 8;

struct VStatsArgs {
    const uint8_t* kv;
    const int32_t* block_table;
    const int32_t* page_valid_len;
    int64_t page_stride;
    int64_t head_stride;
    int32_t num_entries;
    int32_t table_shift;
    int32_t num_pages;
    int32_t block_size;
    int32_t num_kv_heads;
    float* thr;     // [num_kv_heads * D / 16]
    int32_t* plan;  // the guard plan: its row counts are zeroed
    float scale;    // PCPA_GUARD_MIN_MASS * v_scale^2 / 2^18 (the squares' fixed point)
};

// Page and valid length of table entry e (0 for an empty or out-of-range
// entry).
__device__ __forceinline__ int entry_valid(const VStatsArgs& a, int e, int& page) {
    page = a.block_table[e << a.table_shift];
    if (a.table_shift && a.block_table[2 * e + 1] != 0) page = -1;
    const int n = min(a.page_valid_len[e], a.block_size);
    return n > 0 && (unsigned)page < (unsigned)a.num_pages ? n : 0;
}

// Sum of an int over the workgroup (every thread gets it); `ws` holds one
// int per wave and is free again when the function returns.
template <int T>
__device__ __forceinline__ int block_sum(int x, int* ws) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = x;
    __syncthreads();
    int t = 0;
#pragma unroll
    for (int w = 0; w < T / 64; ++w) t += ws[w];
    __syncthreads();
    return t;
}

// Grid: 8 * ceil(num_kv_heads * D / 16 / 8) workgroups; the chunks of one
// KV head run on one XCD (launch index mod 8), whose L2 then reads the
// head's sampled V rows once.  Table entries are staged kVStatsEntries at
// a time (one table read for a walk of at most that many): their sampled
// key counts ceil(n / s) are scanned in LDS, and thread t reads chunk c of
// the t-th of T contiguous runs of the staged entries' sampled keys, up to
// kVStatsBatch loads in flight (all of them for a sampled walk).
template <int D>
__global__ void __launch_bounds__(kVStatsThreads) guard_vstats_kernel(VStatsArgs a) {
    constexpr int CH = D / 16;  // 16-byte chunks of a V row
    constexpr int T = kVStatsThreads, WAVES = T / 64, EPT = kVStatsEntries / T;
    static_assert(CH == 16 || CH == 8 || CH == 4, "16-byte chunks of a 64, 128 or 256 byte row");
    static_assert(kVStatsEntries % T == 0, "whole entries per thread");
    __shared__ int prefix[kVStatsEntries + 1];
    __shared__ int64_t vbase[kVStatsEntries];
    __shared__ int ws[WAVES];
    __shared__ int64_t s1[16][T], s2[16][T];
    __shared__ float vmax[16];
    const int heads = a.num_kv_heads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (blockIdx.x == 0 && tid < heads) a.plan[tid] = 0;
    const int items = heads * CH;
    const int per_xcd = (items + 7) / 8;
    const int item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (item >= items) return;
    const int head = item / CH, c = item - head * CH;

    // ---- the sampling stride, from the walk's valid keys -------------------
    // (a walk of one staging chunk keeps its entries from this read)
    int n_e[EPT], page_e[EPT];
    const bool one_chunk = a.num_entries <= kVStatsEntries;
    int total = 0;
    if (one_chunk) {
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const int el = tid * EPT + i;
            n_e[i] = el < a.num_entries ? entry_valid(a, el, page_e[i]) : 0;
            total += n_e[i];
        }
    } else {
        for (int e = tid; e < a.num_entries; e += T) {
            int page;
            total += entry_valid(a, e, page);
        }
    }
    total = block_sum<T>(total, ws);
    int stride = 1;
    while (total / stride > kVStatsKeys) stride <<= 1;

    // ---- per-thread fp32 sums of chunk c over its keys ----------------------
    float f1[16], f2[16];
#pragma unroll
    for (int b = 0; b < 16; ++b) f1[b] = f2[b] = 0.f;
    int keys = 0;  // sampled keys of the whole walk
    for (int e0 = 0; e0 < a.num_entries; e0 += kVStatsEntries) {
        const int ne = min(kVStatsEntries, a.num_entries - e0);
        // thread t stages entries EPT t .. EPT t + EPT - 1 of the chunk
        int cnt[EPT], run = 0;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const int el = tid * EPT + i;
            if (!one_chunk) n_e[i] = el < ne ? entry_valid(a, e0 + el, page_e[i]) : 0;
            cnt[i] = (n_e[i] + stride - 1) / stride;  // keys 0, s, 2s, ... of its valid prefix
            run += cnt[i];
            vbase[el] = n_e[i] ? (int64_t)page_e[i] * a.page_stride + (int64_t)(heads + head) * a.head_stride + c * 16
                               : 0;
        }
        int incl = run;  // inclusive scan of the runs over the workgroup
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(incl, off);
            if (lane >= off) incl += y;
        }
        if (lane == 63) ws[wave] = incl;
        __syncthreads();
        int before = 0, chunk_keys = 0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            before += w < wave ? ws[w] : 0;
            chunk_keys += ws[w];
        }
        int excl = before + incl - run;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            prefix[tid * EPT + i] = excl;
            excl += cnt[i];
        }
        if (tid == T - 1) prefix[kVStatsEntries] = excl;
        __syncthreads();
        keys += chunk_keys;
        // this thread's run [k0, k1) of the staged entries' sampled keys,
        // from entry e (the last with prefix[e] <= k0); the cursor's bounds
        // stay in registers and change only at an entry boundary
        const int k0 = (int)((int64_t)chunk_keys * tid / T), k1 = (int)((int64_t)chunk_keys * (tid + 1) / T);
        int e = 0;
        for (int lo = 0, hi = ne - 1; lo < hi;) {
            const int mid = (lo + hi + 1) >> 1;
            if (prefix[mid] <= k0) lo = e = mid;
            else hi = mid - 1;
        }
        int first = prefix[e], next = prefix[e + 1];
        int64_t vb = vbase[e];
        for (int q0 = k0; q0 < k1; q0 += kVStatsBatch) {
            v4i x[kVStatsBatch];
#pragma unroll
            for (int j = 0; j < kVStatsBatch; ++j) {
                const int q = q0 + j;
                x[j] = v4i{0, 0, 0, 0};
                if (q < k1) {
                    while (q >= next) {
                        ++e;
                        first = next;
                        next = prefix[e + 1];
                        vb = vbase[e];
                    }
                    x[j] = *(const v4i*)(a.kv + vb + (int64_t)(q - first) * stride * D);
                }
            }
#pragma unroll
            for (int j = 0; j < kVStatsBatch; ++j)
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(x[j][w], false);
                    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(x[j][w], true);
                    const float v[4] = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        f1[4 * w + i] += v[i];
                        f2[4 * w + i] = fmaf(v[i], v[i], f2[4 * w + i]);
                    }
                }
        }
        __syncthreads();  // prefix, vbase and ws are restaged next
    }

    // ---- fixed point, then channel b's T values: thread (b, p) adds every
    // 16th, the 16 partial sums meet by shuffles ---------------------------
    // (|sum of codes| <= 448 * keys per thread: exact in fp32 for up to
    // 2^24 / 229376 = 73 keys a thread)
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        s1[b][tid] = (int64_t)(f1[b] * 512.f);
        s2[b][tid] = (int64_t)rint((double)f2[b] * 262144.0);
    }
    __syncthreads();
    const int b = tid >> 4, p = tid & 15;
    int64_t t1 = 0, t2 = 0;
#pragma unroll
    for (int k = 0; k < T / 16; ++k) {
        t1 += s1[b][p + 16 * k];
        t2 += s2[b][p + 16 * k];
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
        t1 += __shfl_xor(t1, off);
        t2 += __shfl_xor(t2, off);
    }
    if (p == 0) {
        float var = 0.f;
        if (keys > 0) {
            // Var = E[y^2] - E[y]^2 in units of 2^-18 (y = v * 2^9), in double
            const double mean = (double)t1 / (double)keys;
            const double v = (double)t2 / (double)keys - mean * mean;
            var = v > 0.0 ? (float)v : 0.f;
        }
        vmax[b] = var;
    }
    __syncthreads();
    if (tid == 0) {
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) m = fmaxf(m, vmax[i]);
        a.thr[head * CH + c] = m * a.scale;
    }
}

}  // namespace pcpa

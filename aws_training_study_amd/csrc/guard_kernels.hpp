// Precision guard of the e4m3-MFMA history kernels: the plan of the BF16
// fixup and the merge of its split partials.
//
// The guard plan (common.hpp) lists, per KV head, the query rows whose
// probability mass is below PCPA_GUARD_MIN_MASS.  A one-pass e4m3 launch
// writes one flag byte per row and guard_plan_kernel lists them; a split
// launch's merge appends the rows itself.  The fixup gathers them into groups
// of 128 (the BF16 tile kernel's 4 waves x 32 rows).  Few groups: sparse
// mode, where the fixup splits each group's history walk over several
// workgroups (bounded latency) and guard_merge_kernel combines the ranges;
// many: dense mode, one workgroup per group, writing the output directly.
// With no flagged row every fixup and merge workgroup exits at once.
#pragma once

#include "common.hpp"

namespace pcpa {

constexpr int kGuardPlanThreads = 1024;
// KV heads a guard plan handles (the guarded launch is refused beyond).
constexpr int kGuardMaxHeads = 64;
// Capacity of the sparse partials, in query rows over all history ranges:
// [splits, slots * 128] FP32 rows of D + 1 values (34 MB at head_dim 256).
constexpr int64_t kGuardPartialRows = 32768;

// Block-wide exclusive prefix of x over the workgroup's threads (thread
// order), and the total.  Uses `wave_sum` (kGuardPlanThreads / 64 ints).
__device__ __forceinline__ int block_exclusive_scan(int x, int* wave_sum, int& total) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int incl = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off);
        if (lane >= off) incl += y;
    }
    if (lane == 63) wave_sum[wave] = incl;
    __syncthreads();
    int before = 0;
    total = 0;
    for (int w = 0; w < kGuardPlanThreads / 64; ++w) {
        before += w < wave ? wave_sum[w] : 0;
        total += wave_sum[w];
    }
    __syncthreads();  // wave_sum is rewritten by the next scan
    return before + incl - x;
}

// One workgroup.  Writes the guard plan of the flag bytes: each KV head's
// flagged row count and its list of head rows, in ascending order.
__global__ void __launch_bounds__(kGuardPlanThreads) guard_plan_kernel(const uint8_t* flags, GuardShape g,
                                                                      int32_t* plan) {
    __shared__ int wave_sum[kGuardPlanThreads / 64];
    __shared__ int head_count[kGuardMaxHeads];
    __shared__ int next[kGuardMaxHeads];  // head h's next free list position
    const int tid = threadIdx.x;
    const int heads = g.num_kv_heads;
    const int segment = guard_head_segment(g.rows_per_head);
    for (int i = tid; i < kGuardMaxHeads; i += kGuardPlanThreads) head_count[i] = 0;
    __syncthreads();
    // Rows are visited in [pcp, Hq, local_q] order, `unit` consecutive rows
    // at a time (16 when local_q is a multiple of 16: one 16-byte load, one
    // Q head; else 1); restricted to KV head h that is head h's row order.
    const bool chunked = (g.local_q & 15) == 0;
    const int unit = chunked ? 16 : 1;
    const int64_t units = g.rows_total / unit;
    // flagged rows of unit u, one bit each, and the unit's KV head and head row
    auto load_unit = [&](int64_t u, int& head, int& head_row) -> uint32_t {
        const int64_t row = u * unit;
        uint32_t bits = 0;
        if (chunked) {
            const v4i x = *(const v4i*)(flags + row);
#pragma unroll
            for (int w = 0; w < 4; ++w)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    if (((uint32_t)x[w] >> (8 * b)) & 0xffu) bits |= 1u << (4 * w + b);
        } else {
            bits = flags[row] ? 1u : 0u;
        }
        head_row = guard_head_row(g, row, head);
        return bits;
    };
    // ---- count each head's flagged rows (the common case: none, done) -----
    int any = 0;
    for (int64_t u = tid; u < units; u += kGuardPlanThreads) {
        int head, head_row;
        const uint32_t bits = load_unit(u, head, head_row);
        if (bits) {
            any = 1;
            atomicAdd(&head_count[head], __builtin_popcount(bits));
        }
    }
    const bool flagged = __syncthreads_or(any);
    for (int h = tid; h < heads; h += kGuardPlanThreads) {
        plan[h] = head_count[h];
        next[h] = h * segment;
    }
    if (!flagged) return;
    int32_t* const list = plan + guard_list_offset(heads);
    __syncthreads();
    // ---- write the rows in order: kUnits consecutive units per thread -----
    constexpr int kUnits = 4;
    for (int64_t c0 = 0; c0 < units; c0 += (int64_t)kGuardPlanThreads * kUnits) {
        uint32_t bits[kUnits];
        int head[kUnits], head_row[kUnits];
        bool mine = false;
#pragma unroll
        for (int i = 0; i < kUnits; ++i) {
            const int64_t u = c0 + (int64_t)tid * kUnits + i;
            bits[i] = 0;
            head[i] = -1;
            head_row[i] = 0;
            if (u < units) bits[i] = load_unit(u, head[i], head_row[i]);
            mine |= bits[i] != 0;
        }
        if (!__syncthreads_or(mine)) continue;
        for (int h = 0; h < heads; ++h) {
            int count = 0;
#pragma unroll
            for (int i = 0; i < kUnits; ++i) count += head[i] == h ? __builtin_popcount(bits[i]) : 0;
            int total;
            const int pos = block_exclusive_scan(count, wave_sum, total);
            if (count) {
                int k = next[h] + pos;
#pragma unroll
                for (int i = 0; i < kUnits; ++i)
                    if (head[i] == h)
                        for (uint32_t b = bits[i]; b; b &= b - 1) list[k++] = head_row[i] + __builtin_ctz(b);
            }
            __syncthreads();  // every read of next[h] is done
            if (tid == 0) next[h] += total;
        }
    }
}

// Sparse mode: one workgroup per slot row merges the splits' partials of a
// listed row by log-sum-exp (as merge_splits_kernel) into out (bf16) and
// lse.  Thread t takes 8 consecutive d (t % d_vec8) of the ranges t /
// d_vec8, t / d_vec8 + groups, ...; the groups' sums meet in LDS, so the
// dependent loads per thread are splits / groups rather than splits.
// Dense mode, and slot rows past the listed rows: nothing.
constexpr int kGuardMergeThreads = 256;

__global__ void __launch_bounds__(kGuardMergeThreads) guard_merge_kernel(const float* part_o, const float* part_lse,
                                                                         int splits, const int32_t* plan, GuardShape g,
                                                                         int d_vec8, uint8_t* out, float* lse_out) {
    __shared__ float red[kGuardMergeThreads * 8];
    __shared__ float wred[kGuardMergeThreads];
    const int groups_listed = guard_groups(plan, g.num_kv_heads);
    const int64_t slot_row = blockIdx.x;
    const int slot = (int)(slot_row / kRowsPerGroup);
    if (groups_listed > g.max_sparse || slot >= groups_listed) return;
    const GuardGroup gg = guard_group(plan, g.num_kv_heads, slot);
    const int idx = gg.first + (int)(slot_row - (int64_t)slot * kRowsPerGroup);
    if (idx >= gg.count) return;
    const int r = plan[guard_list_offset(g.num_kv_heads) + gg.head * guard_head_segment(g.rows_per_head) + idx];
    const int64_t row = guard_row_index(g, gg.head, r);
    const int D = d_vec8 * 8;
    const int tid = threadIdx.x;
    const int groups = kGuardMergeThreads / d_vec8;  // d_vec8 divides 256 (D = 64, 128, 256)
    const int sg = tid / d_vec8;
    const int d0 = (tid - sg * d_vec8) * 8;
    const int64_t stride = (int64_t)g.max_sparse * kRowsPerGroup;  // rows of one split's partials
    // every thread finds the largest range lse (few loads, all in flight)
    float mx = -INFINITY;
#pragma unroll 8
    for (int sp = 0; sp < splits; ++sp) mx = fmaxf(mx, part_lse[sp * stride + slot_row]);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float wsum = 0.f;
#pragma unroll 8
    for (int sp = sg; sp < splits; sp += groups) {
        const float l = part_lse[sp * stride + slot_row];
        const float w = l == -INFINITY ? 0.f : __expf(l - mx);
        wsum += w;
        const float* const src = part_o + (sp * stride + slot_row) * D + d0;
        const v4f lo = *(const v4f*)src, hi = *(const v4f*)(src + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[i] = fmaf(w, lo[i], acc[i]);
            acc[4 + i] = fmaf(w, hi[i], acc[4 + i]);
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) red[tid * 8 + i] = acc[i];
    wred[tid] = wsum;
    __syncthreads();
    if (sg != 0) return;
    for (int o = 1; o < groups; ++o) {
        const int t = o * d_vec8 + tid;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += red[t * 8 + i];
        wsum += wred[t];
    }
    const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
    uint32_t wv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const __bf16 x0 = (__bf16)(acc[2 * i] * inv), x1 = (__bf16)(acc[2 * i + 1] * inv);
        wv[i] = (uint32_t)__builtin_bit_cast(uint16_t, x0) | ((uint32_t)__builtin_bit_cast(uint16_t, x1) << 16);
    }
    *(v4i*)(out + (row * D + d0) * 2) = v4i{(int)wv[0], (int)wv[1], (int)wv[2], (int)wv[3]};
    if (lse_out && d0 == 0) lse_out[row] = wsum > 0.f ? mx + __logf(wsum) : -INFINITY;
}

}  // namespace pcpa

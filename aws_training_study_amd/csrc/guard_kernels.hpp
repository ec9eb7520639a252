// Precision guard of the e4m3-MFMA history kernels: the V statistics and
// row threshold, the plan of the BF16 fixup and the merge of its split
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
// of standard deviation 4.  guard_vstats_kernel measures it after the e4m3
// pass.  The guard plan (common.hpp) lists, per KV head, the query rows
// whose mass is below it: a one-pass e4m3 launch writes each row's mass and
// guard_plan_kernel lists them; a split launch's merge appends the rows
// itself.  The fixup gathers them into groups
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

// One workgroup.  Writes the guard plan of the row masses: each KV head's
// count of rows below its threshold and its list of head rows, in ascending
// order.
__global__ void __launch_bounds__(kGuardPlanThreads) guard_plan_kernel(const float* mass, const float* thr,
                                                                      GuardShape g, int32_t* plan) {
    __shared__ int wave_sum[kGuardPlanThreads / 64];
    __shared__ int head_count[kGuardMaxHeads];
    __shared__ int next[kGuardMaxHeads];  // head h's next free list position
    const int tid = threadIdx.x;
    const int heads = g.num_kv_heads;
    const int segment = guard_head_segment(g.rows_per_head);
    for (int i = tid; i < kGuardMaxHeads; i += kGuardPlanThreads) head_count[i] = 0;
    __syncthreads();
    // Rows are visited in [pcp, Hq, local_q] order, `unit` consecutive rows
    // at a time (16 when local_q is a multiple of 16: four 16-byte loads, one
    // Q head; else 1); restricted to KV head h that is head h's row order.
    const bool chunked = (g.local_q & 15) == 0;
    const int unit = chunked ? 16 : 1;
    const int64_t units = g.rows_total / unit;
    // rows of unit u below their head's threshold, one bit each, and the
    // unit's KV head and head row
    auto load_unit = [&](int64_t u, int& head, int& head_row) -> uint32_t {
        const int64_t row = u * unit;
        head_row = guard_head_row(g, row, head);
        const float t = thr[head];
        uint32_t bits = 0;
        if (chunked) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const v4f x = *(const v4f*)(mass + row + 4 * w);
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    if (x[b] < t) bits |= 1u << (4 * w + b);
            }
        } else {
            bits = mass[row] < t ? 1u : 0u;
        }
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


// ---- V statistics and the guard threshold -------------------------------
//
// Layout of the statistics (64-bit words, zeroed by workgroup 0 of the e4m3
// pass): [h][d] sum of the sampled V codes times 2^9 (two's complement),
// [h][d] sum of their squares times 2^18, [h] sampled keys, one arrival
// counter; then the thresholds, one float per KV head.  Every e4m3 value is
// a multiple of 2^-9 of magnitude at most 448, so the sums are exact
// integers and the result does not depend on the order the workgroups add
// them in.
constexpr int kVStatsThreads = 256;
// Keys per KV head the statistics sample at most (every s-th key of each
// page, s the smallest power of two that keeps the walk's valid keys / s
// within it; all keys of a shorter history).
constexpr int kVStatsKeys = 16384;
// Workgroups per KV head (at most one per table entry).
constexpr int kVStatsSlots = 128;

__host__ __device__ __forceinline__ int vstats_words(int num_kv_heads, int head_dim) {
    return num_kv_heads * (2 * head_dim + 1) + 1;
}

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
    uint64_t* stats;  // vstats_words(num_kv_heads, D) words
    float* thr;       // [num_kv_heads]
    float scale;      // PCPA_GUARD_MIN_MASS * v_scale^2 / 2^18 (the squares' fixed point)
};

// Grid: slots * num_kv_heads workgroups (slots <= kVStatsSlots); workgroup b
// takes KV head b % num_kv_heads and every slots-th table entry from b /
// num_kv_heads.  The last workgroup to finish writes every head's threshold
// PCPA_GUARD_MIN_MASS * v_scale^2 * max_d (E[v_d^2] - E[v_d]^2).
template <int D>
__global__ void __launch_bounds__(kVStatsThreads) guard_vstats_kernel(VStatsArgs a) {
    constexpr int CH = D / 16;                // 16-byte chunks of a key row
    constexpr int KL = kVStatsThreads / CH;  // keys read per pass
    __shared__ unsigned long long s1[D], s2[D];
    __shared__ float wmax[kVStatsThreads / 64];
    __shared__ int last;
    const int heads = a.num_kv_heads;
    const int head = blockIdx.x % heads;
    const int slot = blockIdx.x / heads;
    const int slots = gridDim.x / heads;
    const int tid = threadIdx.x;
    const int c = tid % CH, kl = tid / CH;
    for (int i = tid; i < D; i += kVStatsThreads) s1[i] = s2[i] = 0;

    typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
    const const_i32_ptr table = (const_i32_ptr)a.block_table;
    const const_i32_ptr lens = (const_i32_ptr)a.page_valid_len;
    // the sampling stride, from the walk's valid keys
    int total = 0;
    for (int e = 0; e < a.num_entries; ++e) {
        const int page = table_page(table, e, a.table_shift);
        const int n = min(lens[e], a.block_size);
        if (n > 0 && (unsigned)page < (unsigned)a.num_pages) total += n;
    }
    int stride = 1;
    while (total / stride > kVStatsKeys) stride <<= 1;

    int acc1[16];
    unsigned long long acc2[16];
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        acc1[b] = 0;
        acc2[b] = 0;
    }
    int count = 0;
    for (int e = slot; e < a.num_entries; e += slots) {
        const int page = table_page(table, e, a.table_shift);
        const int n = min(lens[e], a.block_size);
        if (n <= 0 || (unsigned)page >= (unsigned)a.num_pages) continue;
        count += (n + stride - 1) / stride;
        const uint8_t* const vbase =
            a.kv + (int64_t)page * a.page_stride + (int64_t)(heads + head) * a.head_stride + c * 16;
        for (int key = kl * stride; key < n; key += KL * stride) {
            const v4i x = *(const v4i*)(vbase + (int64_t)key * D);
            auto add = [&](int b, float v) {
                // v * 2^9 is an integer of magnitude <= 229376
                const float y = v * 512.f;
                const unsigned uv = (unsigned)fabsf(y);
                acc1[b] += (int)y;
                acc2[b] += (unsigned long long)uv * uv;
            };
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(x[w], false);
                const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(x[w], true);
                add(4 * w + 0, lo[0]);
                add(4 * w + 1, lo[1]);
                add(4 * w + 2, hi[0]);
                add(4 * w + 3, hi[1]);
            }
        }
    }
    __syncthreads();  // s1 / s2 zeroed
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        atomicAdd(&s1[c * 16 + b], (unsigned long long)(long long)acc1[b]);
        atomicAdd(&s2[c * 16 + b], acc2[b]);
    }
    __syncthreads();
    uint64_t* const sum1 = a.stats + (int64_t)head * D;
    uint64_t* const sum2 = a.stats + (int64_t)(heads + head) * D;
    uint64_t* const keys = a.stats + (int64_t)2 * heads * D;
    uint64_t* const arrivals = keys + heads;
    for (int i = tid; i < D; i += kVStatsThreads) {
        atomicAdd((unsigned long long*)&sum1[i], s1[i]);
        atomicAdd((unsigned long long*)&sum2[i], s2[i]);
    }
    if (tid == 0) atomicAdd((unsigned long long*)&keys[head], (unsigned long long)count);
    // the last workgroup to arrive sees every other one's sums
    __threadfence();
    __syncthreads();
    if (tid == 0)
        last = atomicAdd((unsigned long long*)arrivals, 1ull) == (unsigned long long)(gridDim.x - 1);
    __syncthreads();
    if (!last) return;
    __threadfence();
    for (int h = 0; h < heads; ++h) {
        const uint64_t nk = __hip_atomic_load(&a.stats[(int64_t)2 * heads * D + h], __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
        float vmax = 0.f;
        for (int i = tid; i < D; i += kVStatsThreads) {
            const long long q1 = (long long)__hip_atomic_load(&a.stats[(int64_t)h * D + i], __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT);
            const uint64_t q2 = __hip_atomic_load(&a.stats[(int64_t)(heads + h) * D + i], __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
            if (nk > 0) {
                // Var = E[y^2] - E[y]^2 in units of 2^-18 (y = v * 2^9), in double
                const double mean = (double)q1 / (double)nk;
                const double var = (double)q2 / (double)nk - mean * mean;
                vmax = fmaxf(vmax, (float)(var > 0.0 ? var : 0.0));
            }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, off));
        if ((tid & 63) == 0) wmax[tid >> 6] = vmax;
        __syncthreads();
        if (tid == 0) {
            float m = wmax[0];
            for (int w = 1; w < kVStatsThreads / 64; ++w) m = fmaxf(m, wmax[w]);
            a.thr[h] = m * a.scale;
        }
        __syncthreads();
    }
}

}  // namespace pcpa

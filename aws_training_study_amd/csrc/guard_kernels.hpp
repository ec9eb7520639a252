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
// guard_list_kernel lists them; a split launch's merge appends the rows
// itself (either way by device atomics, in an order that depends on
// timing, which a row's fixup result does not).  The fixup gathers them into groups
// of 128 (the BF16 tile kernel's 4 waves x 32 rows).  Few groups: sparse
// mode, where the fixup splits each group's history walk over several
// workgroups (bounded latency) and guard_merge_kernel combines the ranges;
// many: dense mode, one workgroup per group, writing the output directly.
// With no flagged row every fixup and merge workgroup exits at once.
#pragma once

#include "common.hpp"

namespace pcpa {

// KV heads a guard plan handles (the guarded launch is refused beyond).
constexpr int kGuardMaxHeads = 64;
// Capacity of the sparse partials, in query rows over all history ranges:
// [splits, slots * 128] FP32 rows of D + 1 values (34 MB at head_dim 256).
constexpr int64_t kGuardPartialRows = 32768;

// Rows per thread and threads per workgroup of guard_list_kernel.
constexpr int kGuardListRows = 4;
constexpr int kGuardListThreads = 256;

// The guard plan of a one-pass launch: every row whose mass (written by the
// e4m3 pass) is below its KV head's threshold is appended to the head's
// list with a device atomic (the e4m3 pass zeroed the counts), as the split
// merge does.  The list order depends on timing, which the fixup's result
// does not.  Grid: ceil(rows / (kGuardListRows * kGuardListThreads)).
__global__ void __launch_bounds__(kGuardListThreads) guard_list_kernel(const float* mass, const float* thr,
                                                                      GuardShape g, int32_t* plan) {
    const int64_t row0 = ((int64_t)blockIdx.x * kGuardListThreads + threadIdx.x) * kGuardListRows;
    if (row0 >= g.rows_total) return;
    float m[kGuardListRows];
    if (row0 + kGuardListRows <= g.rows_total) {
        const v4f x = *(const v4f*)(mass + row0);
#pragma unroll
        for (int i = 0; i < kGuardListRows; ++i) m[i] = x[i];
    } else {
#pragma unroll
        for (int i = 0; i < kGuardListRows; ++i) m[i] = row0 + i < g.rows_total ? mass[row0 + i] : INFINITY;
    }
    int32_t* const list = plan + guard_list_offset(g.num_kv_heads);
    const int segment = guard_head_segment(g.rows_per_head);
#pragma unroll
    for (int i = 0; i < kGuardListRows; ++i) {
        int head;
        const int head_row = guard_head_row(g, row0 + i, head);
        if (m[i] < thr[head]) {
            const int pos = atomicAdd(&plan[head], 1);
            list[head * segment + pos] = head_row;
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
// guard_vstats_kernel: workgroup (group g, KV head h) sums, per channel d,
// the sampled V codes of its share of the walk (times 2^9) and their
// squares (times 2^18) and stores the two int64 rows and its key count in
// its slot [g][h] of the statistics (plain stores: every slot is written on
// every call, so nothing needs zeroing).  guard_threshold_kernel then sums
// the groups' slots per (h, d) and takes the largest variance over d.  Every
// e4m3 value is a multiple of 2^-9 of magnitude at most 448: the sums of
// the codes are exact; the squares are summed in fp32 over a thread's few
// keys and rounded to 2^-18 units before the integer sums, so the result
// does not depend on the order in which workgroups finish.
constexpr int kVStatsThreads = 256;
// Keys per KV head the statistics sample at most (every s-th key of each
// page, s the smallest power of two that keeps the walk's valid keys / s
// within it; all keys of a shorter history).
constexpr int kVStatsKeys = 8192;
// Workgroups per KV head, table entries one workgroup takes at most, and the
// 16-byte loads a thread keeps in flight.
constexpr int kVStatsGroups = 64;
constexpr int kVStatsEntries = 256;
constexpr int kVStatsBatch = 8;
// Channels and threads per workgroup of guard_threshold_kernel.
constexpr int kVStatsFinalChannels = 64;
constexpr int kVStatsFinalThreads = 1024;

// 64-bit words of the statistics: groups x heads slots of 2 D + 1 words.
__host__ __device__ __forceinline__ int64_t vstats_words(int groups, int num_kv_heads, int head_dim) {
    return (int64_t)groups * num_kv_heads * (2 * head_dim + 1);
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
    int32_t groups;             // workgroups per KV head
    int32_t entries_per_group;  // table entries of one group (<= kVStatsEntries)
    int32_t parts;              // groups sharing one entry (its sampled keys dealt round-robin)
    int64_t* stats;             // vstats_words(groups, num_kv_heads, D) words
    float* thr;                 // [num_kv_heads]
    float scale;                // PCPA_GUARD_MIN_MASS * v_scale^2 / 2^18 (the squares' fixed point)
};

// Page and valid length of table entry e (0 for an empty or out-of-range
// entry), read with vector loads (threads take different entries).
__device__ __forceinline__ int entry_valid(const VStatsArgs& a, int e, int& page) {
    page = a.block_table[e << a.table_shift];
    if (a.table_shift && a.block_table[2 * e + 1] != 0) page = -1;
    const int n = min(a.page_valid_len[e], a.block_size);
    return n > 0 && (unsigned)page < (unsigned)a.num_pages ? n : 0;
}

// Grid: groups * num_kv_heads workgroups; workgroup b takes KV head b %
// num_kv_heads and group g = b / num_kv_heads: the table entries [e0, e0 +
// entries_per_group) with e0 = (g / parts) * entries_per_group, and of their
// sampled keys every parts-th one from g % parts.  Thread (key lane kl,
// chunk c) reads chunk c of the group's keys kl, kl + KL, ..., kVStatsBatch
// loads at a time.  Workgroup 0 also zeroes the thresholds, which
// guard_threshold_kernel raises next.
template <int D>
__global__ void __launch_bounds__(kVStatsThreads) guard_vstats_kernel(VStatsArgs a) {
    constexpr int CH = D / 16;                // 16-byte chunks of a key row
    constexpr int KL = kVStatsThreads / CH;  // keys read per pass
    constexpr int WAVES = kVStatsThreads / 64;
    static_assert(CH == 16 || CH == 8 || CH == 4, "16-byte chunks of a 64, 128 or 256 byte row");
    __shared__ int w1[WAVES][D];      // per-wave sums of the codes (times 2^9)
    __shared__ int64_t w2[WAVES][D];  // and of their squares (times 2^18)
    __shared__ int prefix[kVStatsEntries + 1];
    __shared__ int64_t vbase[kVStatsEntries];
    __shared__ int wsum[WAVES];
    const int heads = a.num_kv_heads;
    const int head = blockIdx.x % heads;
    const int group = blockIdx.x / heads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = tid % CH, kl = tid / CH;
    if (blockIdx.x == 0 && tid < heads) a.thr[tid] = 0.f;

    // ---- the sampling stride, from the walk's valid keys -------------------
    int total = 0;
    for (int e = tid; e < a.num_entries; e += kVStatsThreads) {
        int page;
        total += entry_valid(a, e, page);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) total += __shfl_xor(total, off);
    if (lane == 0) wsum[wave] = total;
    // ---- this group's entries: its sampled keys per entry (prefix) ----------
    const int part = group % a.parts;
    const int e0 = group / a.parts * a.entries_per_group;
    const int ne = max(0, min(a.num_entries - e0, a.entries_per_group));
    __syncthreads();
    total = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) total += wsum[w];
    int stride = 1;
    while (total / stride > kVStatsKeys) stride <<= 1;
    if (tid < ne) {
        int page;
        const int n = entry_valid(a, e0 + tid, page);
        const int sampled = (n + stride - 1) / stride;  // this entry's keys 0, s, 2s, ...
        prefix[tid + 1] = sampled > part ? (sampled - part + a.parts - 1) / a.parts : 0;
        vbase[tid] = n ? (int64_t)page * a.page_stride + (int64_t)(heads + head) * a.head_stride : 0;
    }
    __syncthreads();
    if (tid == 0) {
        prefix[0] = 0;
        for (int i = 0; i < ne; ++i) prefix[i + 1] += prefix[i];
    }
    __syncthreads();
    const int keys = prefix[ne];

    // ---- per-thread sums of chunk c over its keys (fp32) --------------------
    float f1[16], f2[16];
#pragma unroll
    for (int b = 0; b < 16; ++b) f1[b] = f2[b] = 0.f;
    int entry = 0;  // the entry of this thread's next key (its keys ascend)
    for (int q0 = kl; q0 < keys; q0 += KL * kVStatsBatch) {
        v4i x[kVStatsBatch];
#pragma unroll
        for (int j = 0; j < kVStatsBatch; ++j) {
            const int q = q0 + j * KL;
            x[j] = v4i{0, 0, 0, 0};
            if (q < keys) {
                while (q >= prefix[entry + 1]) ++entry;
                const int key = ((q - prefix[entry]) * a.parts + part) * stride;
                x[j] = *(const v4i*)(a.kv + vbase[entry] + (int64_t)key * D + c * 16);
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
    // ---- to fixed point, then the lanes of one chunk: l ^ {CH .. 8} by
    // shuffles, l ^ 16, l ^ 32 by lane swaps; then the waves through LDS ------
    // (|sum of codes| <= 448 * keys per thread: exact in fp32 for up to
    // 2^24 / 229376 = 73 keys a thread, which the sampling cap keeps)
    auto swap_sum64 = [](int64_t x) -> int64_t {
        auto pair_sum = [](auto r_lo, auto r_hi) -> int64_t {
            return (int64_t)((uint64_t)r_hi[0] << 32 | r_lo[0]) + (int64_t)((uint64_t)r_hi[1] << 32 | r_lo[1]);
        };
        const uint32_t l0 = (uint32_t)x, h0 = (uint32_t)((uint64_t)x >> 32);
        const int64_t y = pair_sum(__builtin_amdgcn_permlane16_swap(l0, l0, false, false),
                                   __builtin_amdgcn_permlane16_swap(h0, h0, false, false));
        const uint32_t l1 = (uint32_t)y, h1 = (uint32_t)((uint64_t)y >> 32);
        return pair_sum(__builtin_amdgcn_permlane32_swap(l1, l1, false, false),
                        __builtin_amdgcn_permlane32_swap(h1, h1, false, false));
    };
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        int64_t i1 = (int64_t)(f1[b] * 512.f);
        int64_t i2 = (int64_t)rint((double)f2[b] * 262144.0);
        if constexpr (CH < 16) {
#pragma unroll
            for (int off = CH; off < 16; off <<= 1) {
                i1 += __shfl_xor(i1, off);
                i2 += __shfl_xor(i2, off);
            }
        }
        i1 = swap_sum64(i1);
        i2 = swap_sum64(i2);
        if (lane < CH) {
            w1[wave][c * 16 + b] = (int)i1;
            w2[wave][c * 16 + b] = i2;
        }
    }
    __syncthreads();
    int64_t* const slot = a.stats + ((int64_t)group * heads + head) * (2 * D + 1);
    for (int i = tid; i < D; i += kVStatsThreads) {
        int64_t t1 = 0, t2 = 0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            t1 += w1[w][i];
            t2 += w2[w][i];
        }
        slot[i] = t1;
        slot[D + i] = t2;
    }
    if (tid == 0) slot[2 * D] = keys;
}

// Grid: num_kv_heads * (D / kVStatsFinalChannels) workgroups of
// kVStatsFinalThreads; workgroup (h, channel block) sums its channels' slots
// over the groups (kVStatsFinalThreads / kVStatsFinalChannels threads per
// channel, four groups' loads in flight at a time), and raises thr[h] to
// PCPA_GUARD_MIN_MASS * v_scale^2 * its largest variance (non-negative
// floats order like their bits, so the result does not depend on the order
// of the workgroups).
template <int D>
__global__ void __launch_bounds__(kVStatsFinalThreads) guard_threshold_kernel(VStatsArgs a) {
    constexpr int PER = kVStatsFinalThreads / kVStatsFinalChannels;  // threads per channel
    __shared__ int64_t t1[kVStatsFinalThreads], t2[kVStatsFinalThreads];
    __shared__ int64_t nk_part[kVStatsFinalThreads];
    __shared__ float vmax[kVStatsFinalChannels];
    const int blocks = D / kVStatsFinalChannels;
    const int h = blockIdx.x / blocks;
    const int d = (blockIdx.x % blocks) * kVStatsFinalChannels + threadIdx.x % kVStatsFinalChannels;
    const int sub = threadIdx.x / kVStatsFinalChannels;
    const int heads = a.num_kv_heads;
    const int64_t slot_words = 2 * D + 1, group_words = (int64_t)heads * slot_words;
    const int64_t* const base = a.stats + (int64_t)h * slot_words;
    int64_t s1 = 0, s2 = 0, nk = 0;
    int g = sub;
    for (; g + 3 * PER < a.groups; g += 4 * PER) {
        int64_t x1[4], x2[4], xn[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t* const slot = base + (g + k * PER) * group_words;
            x1[k] = slot[d];
            x2[k] = slot[D + d];
            xn[k] = slot[2 * D];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            s1 += x1[k];
            s2 += x2[k];
            nk += xn[k];
        }
    }
    for (; g < a.groups; g += PER) {
        const int64_t* const slot = base + g * group_words;
        s1 += slot[d];
        s2 += slot[D + d];
        nk += slot[2 * D];
    }
    t1[threadIdx.x] = s1;
    t2[threadIdx.x] = s2;
    nk_part[threadIdx.x] = nk;
    __syncthreads();
    if (threadIdx.x < kVStatsFinalChannels) {
        int64_t q1 = 0, q2 = 0, n = 0;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            q1 += t1[threadIdx.x + k * kVStatsFinalChannels];
            q2 += t2[threadIdx.x + k * kVStatsFinalChannels];
            n += nk_part[threadIdx.x + k * kVStatsFinalChannels];
        }
        float var = 0.f;
        if (n > 0) {
            // Var = E[y^2] - E[y]^2 in units of 2^-18 (y = v * 2^9), in double
            const double mean = (double)q1 / (double)n;
            const double v = (double)q2 / (double)n - mean * mean;
            var = v > 0.0 ? (float)v : 0.f;
        }
        vmax[threadIdx.x] = var;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = 0.f;
        for (int i = 0; i < kVStatsFinalChannels; ++i) m = fmaxf(m, vmax[i]);
        atomicMax((unsigned*)&a.thr[h], __float_as_uint(m * a.scale));
    }
}

}  // namespace pcpa

// Precision guard of the e4m3-MFMA history kernels: the plan of the BF16
// fixup and the merge of its split partials.
//
// The e4m3 pass writes one flag byte per query row (probability mass below
// PCPA_GUARD_MIN_MASS).  guard_plan_kernel lists the 128-row tiles (of the
// BF16 tile kernel: 4 waves x 32 rows of one KV head) that hold a flagged
// row.  Few tiles: sparse mode, where the fixup splits each tile's history
// walk over several workgroups (bounded latency) and guard_merge_kernel
// combines the ranges; many tiles: dense mode, one workgroup per tile,
// writing the output directly.  With no flagged row every fixup and merge
// workgroup exits at once.
#pragma once

#include "common.hpp"

namespace pcpa {

constexpr int kGuardPlanThreads = 1024;
constexpr int kTileWindow = 16384;
// Capacity of the sparse partials, in query rows over all history ranges:
// [splits, slots * 128] FP32 rows of D + 1 values (67 MB at head_dim 256).
constexpr int64_t kGuardPartialRows = 65536;

struct GuardShape {
    int64_t rows_total;   // pcp * Hq * local_q
    int32_t rows_per_head;
    int32_t group_rows;   // group * local_q
    int32_t local_q;
    int32_t num_q_heads;
    int32_t group;
    int32_t row_tiles;    // 128-row tiles per KV head
    int32_t tiles_total;  // row_tiles * num_kv_heads
    int32_t max_sparse;   // tiles the sparse partials hold
};

// Flag-array index ([pcp, Hq, local_q] order) of row r of KV head `head`
// (rows of a head in the kernels' order: rank, Q head of the group, token).
__device__ __forceinline__ int64_t guard_row_index(const GuardShape& g, int head, int r) {
    const int rank = r / g.group_rows;
    const int rem = r - rank * g.group_rows;
    const int hig = rem / g.local_q;
    const int tok = rem - hig * g.local_q;
    return ((int64_t)(rank * g.num_q_heads + head * g.group + hig)) * g.local_q + tok;
}

// One workgroup.  plan[0] = listed tiles, plan[1] = mode, plan[4 + i] = tile
// id (KV head * row_tiles + row tile) of the i-th flagged tile, ascending.
__global__ void __launch_bounds__(kGuardPlanThreads) guard_plan_kernel(const uint8_t* flags, GuardShape g,
                                                                      int32_t* plan) {
    __shared__ int wave_count[kGuardPlanThreads / 64];
    const int tid = threadIdx.x;
    // ---- any flag at all (16-byte loads; the common case ends here) ------
    int any = 0;
    const int64_t vecs = g.rows_total / 16;
    for (int64_t i = tid; i < vecs; i += kGuardPlanThreads) {
        const v4i x = *(const v4i*)(flags + 16 * i);
        any |= x[0] | x[1] | x[2] | x[3];
    }
    for (int64_t i = vecs * 16 + tid; i < g.rows_total; i += kGuardPlanThreads) any |= flags[i];
    if (!__syncthreads_or(any)) {
        if (tid == 0) {
            plan[0] = 0;
            plan[1] = kGuardNone;
        }
        return;
    }
    // ---- list the tiles holding a flagged row, in tile order --------------
    // Tile flags are gathered in LDS a window of kTileWindow tiles at a time.
    // When local_q is a multiple of 16, 16 consecutive flag bytes (one Q
    // head's tokens t..t+15 of one rank) belong to one tile and are read as
    // one 16-byte load; otherwise the window's rows are read byte by byte.
    __shared__ uint8_t tile_hit[kTileWindow];
    const int lane = tid & 63, wave = tid >> 6;
    const bool chunked = (g.local_q & 15) == 0;
    int listed = 0;
    for (int w0 = 0; w0 < g.tiles_total; w0 += kTileWindow) {
        const int w1 = min(w0 + kTileWindow, g.tiles_total);
        for (int i = tid; i < kTileWindow; i += kGuardPlanThreads) tile_hit[i] = 0;
        __syncthreads();
        if (chunked) {
            for (int64_t c = tid; c < vecs; c += kGuardPlanThreads) {
                const v4i x = *(const v4i*)(flags + 16 * c);
                if (!(x[0] | x[1] | x[2] | x[3])) continue;
                const int64_t row = 16 * c;  // [pcp, Hq, local_q] index
                const int64_t rh = row / g.local_q;
                const int tok = (int)(row - rh * g.local_q);
                const int rank = (int)(rh / g.num_q_heads);
                const int qh = (int)(rh - (int64_t)rank * g.num_q_heads);
                const int head = qh / g.group;
                const int head_row = (rank * g.group + (qh - head * g.group)) * g.local_q + tok;
                const int id = head * g.row_tiles + head_row / kRowsPerGroup;
                if (id >= w0 && id < w1) tile_hit[id - w0] = 1;
            }
        } else {
            for (int id = w0 + tid; id < w1; id += kGuardPlanThreads) {
                const int head = id / g.row_tiles;
                const int r0 = (id - head * g.row_tiles) * kRowsPerGroup;
                const int r1 = min(r0 + kRowsPerGroup, g.rows_per_head);
                int hit = 0;
                for (int r = r0; r < r1; ++r) hit |= flags[guard_row_index(g, head, r)];
                tile_hit[id - w0] = hit ? 1 : 0;
            }
        }
        __syncthreads();
        for (int base = w0; base < w1; base += kGuardPlanThreads) {
            const int id = base + tid;
            const bool hit = id < w1 && tile_hit[id - w0];
            const uint64_t ballot = __builtin_amdgcn_ballot_w64(hit);
            if (lane == 0) wave_count[wave] = __builtin_popcountll(ballot);
            __syncthreads();
            int before = listed, total = 0;
            for (int w = 0; w < kGuardPlanThreads / 64; ++w) {
                before += w < wave ? wave_count[w] : 0;
                total += wave_count[w];
            }
            if (hit) {
                const uint64_t below = lane ? ballot & (~0ull >> (64 - lane)) : 0ull;
                plan[kGuardPlanHeader + before + __builtin_popcountll(below)] = id;
            }
            listed += total;
            __syncthreads();  // wave_count (and, after the window, tile_hit) is rewritten next
        }
    }
    if (tid == 0) {
        plan[0] = listed;
        plan[1] = listed <= g.max_sparse ? kGuardSparse : kGuardDense;
    }
}

// Sparse mode: one thread per (slot row, 8 consecutive d) merges the splits'
// partials of the listed tiles' rows by log-sum-exp (as merge_splits_kernel)
// into out (bf16) and lse.  Other modes, or slots past the list: nothing.
__global__ void __launch_bounds__(256) guard_merge_kernel(const float* part_o, const float* part_lse, int splits,
                                                          const int32_t* plan, GuardShape g, int d_vec8, uint8_t* out,
                                                          float* lse_out) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (plan[1] != kGuardSparse) return;
    const int64_t slot_row = idx / d_vec8;
    const int slot = (int)(slot_row / kRowsPerGroup);
    if (slot >= plan[0]) return;
    const int id = plan[kGuardPlanHeader + slot];
    const int head = id / g.row_tiles;
    const int r = (id - head * g.row_tiles) * kRowsPerGroup + (int)(slot_row - (int64_t)slot * kRowsPerGroup);
    if (r >= g.rows_per_head) return;
    const int64_t row = guard_row_index(g, head, r);
    const int D = d_vec8 * 8;
    const int d0 = (int)(idx - slot_row * d_vec8) * 8;
    const int64_t stride = (int64_t)g.max_sparse * kRowsPerGroup;  // rows of one split's partials
    float mx = -INFINITY;
    for (int sp = 0; sp < splits; ++sp) mx = fmaxf(mx, part_lse[sp * stride + slot_row]);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float wsum = 0.f;
    for (int sp = 0; sp < splits; ++sp) {
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

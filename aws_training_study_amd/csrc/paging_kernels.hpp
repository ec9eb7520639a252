// Paging kernels: the reference's additive block mask turned into per-page
// valid lengths on the GPU, and the allocation of cache pages to the
// (rank, block) entries that appended history tokens reach.
#pragma once

#include "common.hpp"

namespace pcpa {
namespace paging {

constexpr int kMaskThreads = 256;
constexpr int kAllocThreads = 1024;

// One workgroup per cache block b: its valid length is the number of leading
// keys whose bias is zero (+0 or -0) in the reference's mask
// [max_local_blocks, block_size / 128, 1, 128] bf16 (run_poc.py:137-153,
// consumed by kernel.py:113-118 and 341-358: 0 for a valid key, -9984 for
// padding, always a prefix per block).  Every rank gets the same length
// (the reference shares one mask among its ranks).
__global__ void __launch_bounds__(kMaskThreads) mask_lengths_kernel(const uint16_t* mask, int block_size,
                                                                    int max_local_blocks, int pcp,
                                                                    int32_t* page_valid_len) {
    __shared__ int wave_min[kMaskThreads / 64];
    const int b = blockIdx.x;
    const uint16_t* const bias = mask + (int64_t)b * block_size;
    int first = block_size;
    for (int t = threadIdx.x; t < block_size; t += kMaskThreads)
        if (bias[t] & 0x7fffu) first = min(first, t);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) first = min(first, __shfl_xor(first, off));
    if ((threadIdx.x & 63) == 0) wave_min[threadIdx.x >> 6] = first;
    __syncthreads();
    int n = wave_min[0];
#pragma unroll
    for (int w = 1; w < kMaskThreads / 64; ++w) n = min(n, wave_min[w]);
    for (int r = threadIdx.x; r < pcp; r += kMaskThreads) page_valid_len[(int64_t)r * max_local_blocks + b] = n;
}

// History positions below `pos` owned by `rank` under striping with
// interleave `il` over `pcp` ranks (layout.py:10-16): whole rounds give every
// rank il positions, the tail is dealt il at a time in rank order.
__host__ __device__ __forceinline__ int64_t owned_below(int64_t pos, int rank, int pcp, int il) {
    const int64_t stride = (int64_t)pcp * il;
    const int64_t rounds = pos / stride, rem = pos - rounds * stride;
    const int64_t tail = rem - (int64_t)rank * il;
    return rounds * il + (tail < 0 ? 0 : tail > il ? il : tail);
}

struct AllocArgs {
    int32_t* table;            // [pcp, max_local_blocks] int32 (or int64 as dword pairs, table_shift 1)
    int32_t table_shift;
    const int32_t* free_pages; // the free-page stack
    int32_t* free_count;       // its height (device int32)
    int64_t first_pos;
    int64_t end_pos;           // first_pos + num_tokens
    int32_t pcp, interleave, block_size, max_local_blocks;
};

// One workgroup.  In (rank, block) entry order, every entry that the
// positions [first_pos, end_pos) reach and that holds no page yet (a negative
// table value) takes the next page from the top of the free stack; the
// stack height is lowered by the pages taken.  Entries that find the stack
// empty keep their negative value.  Deterministic: the same appends always
// give the same table.
__global__ void __launch_bounds__(kAllocThreads) page_alloc_kernel(AllocArgs a) {
    __shared__ int wave_count[kAllocThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int height = *a.free_count;
    const int entries = a.pcp * a.max_local_blocks;
    int taken = 0;
    for (int base = 0; base < entries; base += kAllocThreads) {
        const int e = base + tid;
        bool need = false;
        if (e < entries) {
            const int rank = e / a.max_local_blocks;
            const int blk = e - rank * a.max_local_blocks;
            const int64_t lo = owned_below(a.first_pos, rank, a.pcp, a.interleave);
            const int64_t hi = owned_below(a.end_pos, rank, a.pcp, a.interleave);
            const int64_t b0 = (int64_t)blk * a.block_size;
            const bool touched = lo < hi && b0 < hi && b0 + a.block_size > lo;
            if (touched) {
                const int32_t lo_word = a.table[e << a.table_shift];
                const int32_t hi_word = a.table_shift ? a.table[2 * e + 1] : (lo_word < 0 ? -1 : 0);
                need = hi_word < 0;  // a negative (int32 or int64) entry: no page yet
            }
        }
        const uint64_t ballot = __builtin_amdgcn_ballot_w64(need);
        if (lane == 0) wave_count[wave] = __builtin_popcountll(ballot);
        __syncthreads();
        int before = taken, total = 0;
        for (int w = 0; w < kAllocThreads / 64; ++w) {
            before += w < wave ? wave_count[w] : 0;
            total += wave_count[w];
        }
        if (need) {
            const uint64_t below = lane ? ballot & (~0ull >> (64 - lane)) : 0ull;
            const int k = before + __builtin_popcountll(below);
            if (k < height) {
                const int32_t page = a.free_pages[height - 1 - k];
                a.table[e << a.table_shift] = page;
                if (a.table_shift) a.table[2 * e + 1] = 0;
            }
        }
        taken += total;
        __syncthreads();  // wave_count is rewritten by the next chunk
    }
    if (tid == 0) *a.free_count = taken < height ? height - taken : 0;
}

}  // namespace paging
}  // namespace pcpa

// Shared types, constants, launch arguments, LDS layout maps and the
// block-table walk of the history attention kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "pcp_attention_hip.h"

namespace pcpa {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

#define PCPA_LDS(T, p) ((__attribute__((address_space(3))) T*)(p))

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsPerWave = 32;
constexpr int kRowsPerGroup = kWaves * kRowsPerWave;
constexpr int kKeyTile = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kFp8Max = 448.0f;
// FP8 probabilities are computed as 2^(x - m + kPBiasLog2): the largest is 64,
// and values down to 2^-12 of the row max stay in e4m3's normal range.  The
// factor cancels in O / l because l sums the same biased values.
constexpr float kPBiasLog2 = 6.0f;

struct FwdArgs {
    const uint8_t* q;
    const uint8_t* kv;
    const int32_t* block_table;  // int32 entries, or int64 ones read as dword pairs (table_shift 1)
    const int32_t* page_valid_len;
    uint8_t* out;
    int64_t page_stride;   // bytes of one page (K and V of every KV head)
    int64_t head_stride;   // bytes of one head's K (or V) block
    int32_t rows_per_head; // pcp * group * local_q
    int32_t row_tiles;     // ceil(rows_per_head / kRowsPerGroup)
    int32_t group_rows;    // group * local_q
    int32_t local_q;
    int32_t num_q_heads;
    int32_t group;
    int32_t num_kv_heads;
    int32_t num_entries;   // pcp * max_local_blocks
    int32_t table_shift;   // log2 of the table entry size in dwords: 0 (int32) or 1 (int64)
    int32_t num_pages;
    int32_t block_size;
    float score_scale;     // softmax_scale * k_scale * log2(e)
    float v_scale;
    float* lse;            // optional: natural-log sum of exp(score) per row, [pcp, Hq, local_q]
    // Causal current-token attention only (history_fwd_kernel<..., CAUSAL>):
    const uint8_t* merge_o;   // optional history output to merge with, bf16 like `out`
    const float* merge_lse;   // its per-row log-sum-exp
    int32_t interleave;       // striping of the current tokens over ranks
    int32_t pcp;
    // Split history (overlap kernel, SPLIT): the table entries are cut into
    // `splits` equal ranges, one per workgroup of a row tile; each writes its
    // normalised FP32 partial output and log-sum-exp, merged afterwards.
    int32_t splits;
    int32_t part_f16;         // part_o holds fp16 values of O / l before v_scale (the e4m3 overlap kernel)
    float* part_o;            // [splits, pcp * Hq * local_q, D] fp32 (or fp16)
    float* part_lse;          // [splits, pcp * Hq * local_q]
    float* part_m;            // [splits, pcp * Hq * local_q]: each range's reference max (log2)
    // Precision guard of a one-pass e4m3-MFMA launch: each row whose
    // probability mass sum_k 2^(x_k - m) is below its KV head's threshold
    // (guard_threshold over guard_thr, written by guard_vstats_kernel, which
    // also zeroed the plan's row counts) is appended to the guard plan
    // guard_rows.  A split launch leaves both null; its merge appends.
    const float* guard_thr;
    int32_t* guard_rows;
    // The BF16 fixup of a guarded launch (history_fwd_kernel<..., FIXUP>):
    // the guard plan (below), the partials' capacity in rows (part_o /
    // part_lse) and, in `splits`, the most history ranges a group is cut
    // into.  guard_ranges() picks the ranges for the number of groups
    // listed: with two or more the fixup is sparse (each group's walk split
    // over that many workgroups, partials merged by guard_merge_kernel),
    // else dense (one workgroup per group, output written directly).
    const int32_t* guard_plan;
    int32_t guard_partial_rows;
};

// A guard plan: [h] (h < num_kv_heads) the number of flagged rows of KV head
// h, then, from guard_list_offset, one list per KV head of
// guard_head_segment(rows_per_head) entries, whose first [h] are the head's
// flagged rows (head row indices: rank, Q head of the group, token) in any
// order — a row's fixup result does not depend on the rows gathered with
// it.  Head h's rows form ceil([h] / 128) groups of 128, numbered head by
// head.
__host__ __device__ __forceinline__ int guard_list_offset(int num_kv_heads) { return (num_kv_heads + 3) / 4 * 4; }
__host__ __device__ __forceinline__ int guard_head_segment(int rows_per_head) {
    return (rows_per_head + kRowsPerGroup - 1) / kRowsPerGroup * kRowsPerGroup;
}

// Shape of the rows a guard plan indexes.
struct GuardShape {
    int64_t rows_total;   // pcp * Hq * local_q
    int32_t rows_per_head;
    int32_t group_rows;   // group * local_q
    int32_t local_q;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t group;
    int32_t partial_rows;  // rows the sparse fixup's partials hold
    int32_t max_ranges;    // history ranges a sparse group is cut into at most
};

// History ranges of a sparse fixup over `groups` listed 128-row groups: as
// many as the partials hold (partial_rows rows), at most max_ranges; 0
// (dense: one workgroup per group) when fewer than two fit.
__host__ __device__ __forceinline__ int guard_ranges(int groups, int partial_rows, int max_ranges) {
    if (groups <= 0) return 0;
    int r = partial_rows / (kRowsPerGroup * groups);
    r = r < max_ranges ? r : max_ranges;
    return r >= 2 ? r : 0;
}

// The threshold of KV head `head`: the largest of its `chunks` (head_dim /
// 16) per-chunk values (guard_vstats_kernel).
__device__ __forceinline__ float guard_threshold(const float* thr, int head, int chunks) {
    float t = 0.f;
#pragma unroll 16
    for (int c = 0; c < chunks; ++c) t = fmaxf(t, thr[head * chunks + c]);
    return t;
}

// Append head row `row` to KV head `head`'s list of the guard plan (its
// count was zeroed by guard_vstats_kernel earlier in the launch).
__device__ __forceinline__ void guard_append(int32_t* plan, int num_kv_heads, int rows_per_head, int head, int row) {
    const int pos = atomicAdd(&plan[head], 1);
    plan[guard_list_offset(num_kv_heads) + head * guard_head_segment(rows_per_head) + pos] = row;
}

// Flag-array index ([pcp, Hq, local_q] order) of row r of KV head `head`.
__device__ __forceinline__ int64_t guard_row_index(const GuardShape& g, int head, int r) {
    const int rank = r / g.group_rows;
    const int rem = r - rank * g.group_rows;
    const int hig = rem / g.local_q;
    const int tok = rem - hig * g.local_q;
    return ((int64_t)(rank * g.num_q_heads + head * g.group + hig)) * g.local_q + tok;
}

// KV head and head row index of the row at flag-array index `row`.
__device__ __forceinline__ int guard_head_row(const GuardShape& g, int64_t row, int& head) {
    const int64_t rh = row / g.local_q;
    const int tok = (int)(row - rh * g.local_q);
    const int rank = (int)(rh / g.num_q_heads);
    const int qh = (int)(rh - (int64_t)rank * g.num_q_heads);
    head = qh / g.group;
    return (rank * g.group + (qh - head * g.group)) * g.local_q + tok;
}

// Groups of 128 rows in a plan.
__device__ __forceinline__ int guard_groups(const int32_t* plan, int heads) {
    int total = 0;
    for (int h = 0; h < heads; ++h) total += (plan[h] + kRowsPerGroup - 1) / kRowsPerGroup;
    return total;
}

// Group `slot` (< guard_groups) of a plan: its KV head, the list index of its
// first row and the head's row count.
struct GuardGroup {
    int head;
    int first;
    int count;
};
__device__ __forceinline__ GuardGroup guard_group(const int32_t* plan, int heads, int slot) {
    GuardGroup g{0, 0, 0};
    int before = 0;
    for (int h = 0; h < heads; ++h) {
        const int count = plan[h];
        const int n = (count + kRowsPerGroup - 1) / kRowsPerGroup;
        if (slot >= before && slot < before + n) g = GuardGroup{h, (slot - before) * kRowsPerGroup, count};
        before += n;
    }
    return g;
}

// ln(E[(1 + f) / 2^f]) for f uniform in [0, 1): how much the linear-mantissa
// exp2 of the FP8 overlap kernel overestimates a sum of exponentials on
// average (1.04069); subtracted from that kernel's log-sum-exp outputs.
constexpr float kFastLseBias = 0.03987f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// Max / sum of a value over lanes l and l^32 (the two k-groups of a 32x32
// MFMA tile, which hold different keys of the same query).
__device__ __forceinline__ float halves_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Key (within the 64-key tile) held by accumulator register r of score tile t
// in lane half h.  The 32x32 accumulator puts row 8*(r/4) + 4*h + r%4 in
// register r; K rows are ordered so that P^T comes out in PV B-operand order:
//   FP8 (one PV MFMA eats 64 keys, 32 per lane half): key = 32h + 16t + r
//   BF16 (one PV MFMA eats 16 keys, 8 per lane half):
//        key = 32t + 16*(r/8) + 8h + r%8
template <bool FP8>
__device__ __forceinline__ int key_of_acc(int t, int r, int h) {
    return FP8 ? 32 * h + 16 * t + r : 32 * t + 16 * (r >> 3) + 8 * h + (r & 7);
}
// Same map indexed by the A-operand row rho (0..31) of the score MFMA.
template <bool FP8>
__device__ __forceinline__ int key_of_row(int t, int rho) {
    return key_of_acc<FP8>(t, 4 * (rho >> 3) + (rho & 3), (rho >> 2) & 1);
}

// LDS row holding key `key` of a 64-key tile.  FP8 tiles swap key bits 3
// and 5: the 16 score-operand rows a 16-lane group reads (keys 32h+16t+r,
// r < 8) and the 8 keys a transposing V read covers then differ in the low 4
// row bits, and the per-lane part of every K, V and DMA address is the same
// for all tiles t, reads s and DMA blocks.  BF16 tiles keep key order.
template <bool FP8>
__host__ __device__ __forceinline__ constexpr int lds_row(int key) {
    if constexpr (FP8) return (key & ~0x28) | ((key >> 2) & 0x8) | ((key << 2) & 0x20);
    return key;
}

// XOR swizzle of the 16-byte chunk index within LDS row `row`, making the
// score-operand reads (ds_read_b128, 16 rows per 16-lane group) and the
// transposing V reads bank-conflict free (measured with the LDS
// bank-conflict counter on gfx950, per read pattern).  BF16 rows of 128
// bytes (head_dim 64) sit in alternate halves of the 64 banks, so their K
// swizzle spreads even and odd rows over all 8 chunks each.  BF16 rows of
// 512 bytes (head_dim 256) swap the two bit pairs of the row: a bijection
// on the 16 rows a 16-lane score read covers, and distinct in chunk bits
// 2-3 over every 4-row block a 32-lane transposing V read covers, so K and
// V share one swizzle (and one set of lane DMA offsets) with no conflicts.
template <bool FP8, int CHUNKS>
__device__ __forceinline__ int chunk_swizzle(int row) {
    constexpr int mask = (CHUNKS < 16 ? CHUNKS : 16) - 1;
    if constexpr (FP8) return row & 15 & mask;
    if constexpr (CHUNKS == 8) return (row >> 1) & 7;
    if constexpr (CHUNKS == 32) return ((row & 3) << 2) | ((row >> 2) & 3);
    return (((row & 7) << 1) | ((row >> 3) & 1)) & mask;
}
// FP8 V tiles use an even-only swizzle: the two 16-lane groups of a
// transposing read that share rows (d halves 2dt and 2dt+1) then land on
// disjoint chunk sets (even vs odd), so 32 lanes cover all 64 banks once.
// BF16 V tiles of 256-byte rows (head_dim 128): a 32-lane transposing read
// covers 4 consecutive rows x 4 chunks, and rows 4s and 4s + 1 (4s + 2 and
// 4s + 3) would share their chunk block under the score swizzle (2-way
// conflicts, 1.8 extra cycles per read); flipping chunk bit 3 on odd rows
// separates them (GQA-8 workload 1.99 -> 1.97 ms).  Other BF16 rows keep
// the score operand's swizzle: 128-byte rows are conflict-free with it,
// and 512-byte rows have one made for both reads (a flip for V alone
// measured slower there: separate V DMA offsets cost lane-address work).
template <bool FP8, int CHUNKS>
__device__ __forceinline__ int chunk_swizzle_v(int row) {
    constexpr int mask = (CHUNKS < 16 ? CHUNKS : 16) - 1;
    if constexpr (FP8) return (2 * row) & mask & 14;
    if constexpr (CHUNKS == 32) return chunk_swizzle<false, CHUNKS>(row);
    const int s = (((row & 7) << 1) | ((row >> 3) & 1)) & mask;
    if constexpr (CHUNKS == 16) return s ^ ((row & 1) << 3);
    return s;
}

// s = -inf unless K < lim, through vcc alone.  Written as plain C++ over a
// whole score tile, the compiler forms one SGPR-pair mask per element (about
// 64 SGPRs live at once), which pushes the loop's scalar state into VGPR
// lanes; this form needs no SGPR beyond vcc.  (-inf comes from a VGPR: vcc
// and a literal together exceed the one scalar operand a VALU op may read.)
template <int K>
__device__ __forceinline__ float mask_key_at_or_past(float s, int lim, float ninf) {
    static_assert(K >= 0 && K <= 64, "K must be an inline constant");
    asm("v_cmp_lt_i32_e32 vcc, %1, %2\n\t"
        "v_cndmask_b32_e32 %0, %3, %0, vcc"
        : "+v"(s)
        : "i"(K), "v"(lim), "v"(ninf)
        : "vcc");
    return s;
}

// LDS-DMA of one 1 KB block: lane l copies 16 bytes from global memory into
// LDS byte m0v + IMM + 16 l (the instruction offset IMM applies to both
// addresses).  Inline asm rather than the builtin, for the scalar-base form:
// the wave-uniform tile address stays in an SGPR pair and each lane adds one
// 32-bit VGPR offset, where the builtin forms a 64-bit VGPR address per lane
// (registers the kernels' tile loops do not have).  Every LDS-DMA of the
// attention kernels goes through these two helpers, so m0 never holds a
// value of the compiler's own across them; s_nop 0 covers the m0 write
// ahead of the load.
template <int IMM>
__device__ __forceinline__ void dma_sbase(const uint8_t* base, uint32_t lane_off, uint32_t m0v) {
    static_assert(IMM >= -4096 && IMM < 4096, "the instruction offset is 13-bit signed");
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 offset:%3"
                 :
                 : "s"(m0v), "v"(lane_off), "s"(base), "i"(IMM)
                 : "memory", "m0");
}
// The same from a per-lane 64-bit address, without an offset.
__device__ __forceinline__ void dma_vaddr(const uint8_t* addr, uint32_t m0v) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(m0v), "v"(addr)
                 : "memory", "m0");
}

// Four bf16 values (8 bytes) widened exactly from four e4m3 codes (one dword).
__device__ __forceinline__ v2i e4m3x4_to_bf16x4(int codes) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(codes, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(codes, true);
    // e4m3 values are exact in bf16: keep the upper half of each f32.
    const int w0 = (int)((__float_as_uint(lo[0]) >> 16) | (__float_as_uint(lo[1]) & 0xffff0000u));
    const int w1 = (int)((__float_as_uint(hi[0]) >> 16) | (__float_as_uint(hi[1]) & 0xffff0000u));
    return v2i{w0, w1};
}

// s_waitcnt vmcnt(0) with expcnt/lgkmcnt left unconstrained (gfx9 encoding).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// f(std::integral_constant<int, i>{}) for i = I .. N-1, unrolled at compile time.
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Transposing LDS reads as inline asm.  The builtins carry no memory-operand
// information, so the compiler orders them after every in-flight LDS DMA,
// including the prefetch of the *other* buffer, which would serialise the
// pipeline.  Ordering against this buffer's DMA is provided by the
// vmcnt(0) + barrier at the top of each tile; lds_results_ready() makes the
// results usable.  OFF is the instruction's immediate byte offset.
__device__ __forceinline__ uint32_t lds_address(const uint8_t* p) {
    return (uint32_t)(uintptr_t)PCPA_LDS(const uint8_t, p);
}
template <int OFF>
__device__ __forceinline__ v2i ds_read_tr8_b64(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
    v2i r;
    asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
}
template <int OFF>
__device__ __forceinline__ v2i ds_read_tr16_b64(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
    v2i r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
}
// s_waitcnt lgkmcnt(0), with the read results as operands so that no use of
// them (and no copy of the registers) can be scheduled before the wait.
__device__ __forceinline__ void lds_results_ready(v2i (&x)[8]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7]));
}
__device__ __forceinline__ void lds_results_ready(v2i (&x)[4]) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]));
}
__device__ __forceinline__ void lds_results_ready(v2i (&x)[2]) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x[0]), "+v"(x[1]));
}

// Position in the walk over the block table: entry e (rank-major (rank,
// block) order), tile start `base` within the page, the page's valid length
// n, and the byte offset of this KV head's K block in the pool.
struct TileCursor {
    int e;
    int base;
    int n;
    int64_t k_off;
};

// Page of table entry e, or -1 for an int64 entry beyond 32 bits (treated as
// out of range like any other).
template <class P>
__device__ __forceinline__ int table_page(P table, int e, int shift) {
    const int page = table[e << shift];
    return shift && table[2 * e + 1] != 0 ? -1 : page;
}

// The tile after `c`: the next 64 keys of the same page, or the first tile
// of the next table entry with valid tokens and an in-range page.  Entries
// whose page index is outside [0, num_pages) are never read.  The table and
// the valid lengths are read-only for the whole launch, so they are read
// through the constant address space: scalar loads, which do not share the
// vector-memory counter that the LDS-DMA waits count.
__device__ __forceinline__ TileCursor next_tile(const FwdArgs& a, int head, TileCursor c) {
    if (c.base + kKeyTile < c.n) {
        c.base += kKeyTile;
        return c;
    }
    typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
    const const_i32_ptr table = (const_i32_ptr)a.block_table;
    const const_i32_ptr lens = (const_i32_ptr)a.page_valid_len;
    for (int e = c.e + 1; e < a.num_entries; ++e) {
        const int page = table_page(table, e, a.table_shift);
        const int n = min(lens[e], a.block_size);
        if (n > 0 && (unsigned)page < (unsigned)a.num_pages)
            return TileCursor{e, 0, n, (int64_t)page * a.page_stride + (int64_t)head * a.head_stride};
    }
    return TileCursor{a.num_entries, 0, 0, 0};
}

// For a whole workgroup of T threads at once: the cursor of the first key
// tile of range `split` of `splits` equal ranges of the walk's key tiles
// (every entry with valid tokens and an in-range page contributes
// ceil(n / 64)), and in `tiles` the range's tile count (the end cursor for
// an empty range).  Thread t counts the tiles of its block
// of consecutive entries, a scan over the workgroup (`red`: one int per
// wave) places the blocks, and the block holding the range's first tile
// finds its entry and writes the cursor to `shared`.  Every thread of the
// workgroup must call it.
template <int T>
__device__ __forceinline__ TileCursor range_cursor(const FwdArgs& a, int head, int split, int splits, int& tiles,
                                                   int* red, TileCursor* shared) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int per = (a.num_entries + T - 1) / T;
    const int e_lo = min(tid * per, a.num_entries), e_hi = min(e_lo + per, a.num_entries);
    int cnt = 0;
    for (int e = e_lo; e < e_hi; ++e) {
        const int page = table_page(a.block_table, e, a.table_shift);
        const int n = min(a.page_valid_len[e], a.block_size);
        if (n > 0 && (unsigned)page < (unsigned)a.num_pages) cnt += (n + kKeyTile - 1) / kKeyTile;
    }
    int incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off);
        if (lane >= off) incl += y;
    }
    if (lane == 63) red[wave] = incl;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < T / 64; ++w) {
        before += w < wave ? red[w] : 0;
        total += red[w];
    }
    const int first = (int)((int64_t)total * split / splits);
    tiles = (int)((int64_t)total * (split + 1) / splits) - first;
    if (tiles <= 0) return TileCursor{a.num_entries, 0, 0, 0};  // the same for every thread
    const int excl = before + incl - cnt;
    if (first >= excl && first < excl + cnt) {
        int t = first - excl;
        for (int e = e_lo; e < e_hi; ++e) {
            const int page = table_page(a.block_table, e, a.table_shift);
            const int n = min(a.page_valid_len[e], a.block_size);
            if (n <= 0 || (unsigned)page >= (unsigned)a.num_pages) continue;
            const int nt = (n + kKeyTile - 1) / kKeyTile;
            if (t < nt) {
                *shared = TileCursor{e, t * kKeyTile, n,
                                     (int64_t)page * a.page_stride + (int64_t)head * a.head_stride};
                break;
            }
            t -= nt;
        }
    }
    __syncthreads();
    return *shared;
}

// The tile after `c` in the single "page" of the current tokens (CAUSAL
// kernels): entry 0 holds all block_size current tokens in global order;
// there is no block table.
__device__ __forceinline__ TileCursor next_current_tile(const FwdArgs& a, int head, TileCursor c) {
    if (c.e < 0) return TileCursor{0, 0, a.block_size, (int64_t)head * a.head_stride};
    if (c.base + kKeyTile < c.n) {
        c.base += kKeyTile;
        return c;
    }
    return TileCursor{a.num_entries, 0, 0, 0};
}

}  // namespace pcpa

// History-only PCP attention for MI355X (gfx950): kernels and C ABI.
//
// One launch computes, for every logical PCP rank, the attention of that
// rank's current-token Q over the whole paged history (all ranks' cache
// blocks), which the Trainium2 proof of concept computed with a device ring
// (pcp_attention/kernel.py:84-554).  The ring order only changes the order of
// online-softmax updates; here every query row walks the block table in
// table order.
//
// Two kernels share the data layout and operand maps below:
//   * history_fwd_kernel<D, STORE8, FP8>: 4 waves x 32 rows per workgroup,
//     two workgroups per CU, double-buffered tiles; every head dim (64, 128,
//     256) and precision (e4m3 or bf16 MFMAs).
//   * ovl::history_fwd_overlap<256, FAST, LSE>: the e4m3-MFMA path at head_dim 256,
//     8 waves x 32 rows, a two-stage in-wave pipeline with the two waves of a
//     SIMD staggered by half a tile step (see its header).
//
// Work decomposition
//   * A "row" is one (Q head, current token) pair.  Rows that share a KV head
//     (GQA group) are independent and are tiled 32 to a wave; a workgroup's
//     waves take consecutive row tiles of one KV head.
//   * Keys are consumed in 64-key tiles staged through LDS (K tile and V tile,
//     row-major [key][d], 16-byte chunks XOR-swizzled per key so that both the
//     score-operand reads and the transposing V reads are bank-conflict free).
//   * Scores are computed transposed, S^T = K . Q^T, with 32x32 MFMA tiles:
//     K (from LDS) is the A operand, the wave's 32 Q rows are a register-
//     resident B operand.  The accumulator of S^T holds, per lane, 16 keys of
//     one query, which is exactly the B-operand layout of P^T in
//     O^T += V^T . P^T once the K rows are permuted (key_of_row below).  So P
//     goes from the score accumulator to the PV MFMA without leaving the lane,
//     and V^T is read from the row-major V tile with ds_read_b64_tr_b8/b16.
//   * FP8 KV: both GEMMs run as v_mfma_f32_32x32x64_f8f6f4 (e4m3 x e4m3).  Q
//     is quantised to e4m3 per row (scale amax/448) when loaded; P is
//     quantised to e4m3 after exp2.  BF16 KV: v_mfma_f32_32x32x16_bf16.
//   * Online softmax in FP32 registers in the log2 domain: the per-row factor
//     softmax_scale * k_scale * log2(e) (times the Q row scale) is applied in
//     the exp2 argument.
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
    const int32_t* block_table;
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
    float* part_o;            // [splits, pcp * Hq * local_q, D]
    float* part_lse;          // [splits, pcp * Hq * local_q]
};

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
__device__ __forceinline__ int lds_row(int key) {
    if constexpr (FP8) return (key & ~0x28) | ((key >> 2) & 0x8) | ((key << 2) & 0x20);
    return key;
}

// XOR swizzle of the 16-byte chunk index within LDS row `row`, making the
// score-operand reads (16 rows per 16-lane group) and the transposing V
// reads (8 rows x 16 bytes, or 4 rows x 32 bytes) bank-conflict free.
template <bool FP8, int CHUNKS>
__device__ __forceinline__ int chunk_swizzle(int row) {
    constexpr int mask = (CHUNKS < 16 ? CHUNKS : 16) - 1;
    const int s = FP8 ? (row & 15) : (((row & 7) << 1) | ((row >> 3) & 1));
    return s & mask;
}
// FP8 V tiles use an even-only swizzle: the two 16-lane groups of a
// transposing read that share rows (d halves 2dt and 2dt+1) then land on
// disjoint chunk sets (even vs odd), so 32 lanes cover all 64 banks once.
template <bool FP8, int CHUNKS>
__device__ __forceinline__ int chunk_swizzle_v(int row) {
    constexpr int mask = (CHUNKS < 16 ? CHUNKS : 16) - 1;
    if constexpr (FP8) return (2 * row) & mask & 14;
    return chunk_swizzle<FP8, CHUNKS>(row);
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

// Position in the walk over the block table: entry e (rank-major (rank,
// block) order), tile start `base` within the page, the page's valid length
// n, and the byte offset of this KV head's K block in the pool.
struct TileCursor {
    int e;
    int base;
    int n;
    int64_t k_off;
};

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
        const int page = table[e];
        const int n = min(lens[e], a.block_size);
        if (n > 0 && (unsigned)page < (unsigned)a.num_pages)
            return TileCursor{e, 0, n, (int64_t)page * a.page_stride + (int64_t)head * a.head_stride};
    }
    return TileCursor{a.num_entries, 0, 0, 0};
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

// STORE8: the cache holds e4m3 (else bf16).  FP8: the MFMAs run on e4m3
// operands (requires STORE8); otherwise they run on bf16, and an e4m3 cache
// is widened to bf16 while it is staged into LDS.
template <int D, bool STORE8, bool FP8>
struct TileShape {
    static_assert(STORE8 || !FP8, "e4m3 MFMAs need an e4m3 cache");
    static constexpr int ES = FP8 ? 1 : 2;
    static constexpr bool F8 = FP8;
    static constexpr int ROW = D * ES;                 // LDS bytes of one key row
    static constexpr int CHUNKS = ROW / 16;
    static constexpr int TILE = kKeyTile * ROW;        // LDS bytes of one K (or V) tile
    static constexpr int GROW = D * (STORE8 ? 1 : 2);  // cache bytes of one key row
    static constexpr int GCHUNKS = GROW / 16;
    static constexpr bool WIDEN = STORE8 && !FP8;
    // Double-buffered (prefetching) when both buffers fit the 64 KB static
    // LDS limit; the widening path stages synchronously through registers.
    static constexpr int NBUF = (!WIDEN && 4 * TILE <= 65536) ? 2 : 1;
    static constexpr int QK = FP8 ? D / 64 : D / 16;   // k-steps of the score MFMA
    static constexpr int DT = D / 32;                  // 32-row d tiles of O^T
    static constexpr int DMA_PER_WAVE = CHUNKS / 4;    // 1 KB DMA blocks per wave per operand
    // Wave w loads DMA blocks 4i + w.  Block i's lane chunk sits DMA_ROW_DELTA(i)
    // key rows after block 0's, with the same chunk swizzle, except for 512-byte
    // rows (bf16 D=256) whose swizzle changes between blocks: those keep one
    // offset per block (DMA_SPLIT).
    static constexpr bool DMA_SPLIT = ROW == 512;
    static constexpr int K_T1_ROWS = FP8 ? 16 : 32;    // LDS rows from score tile 0 to tile 1
    static constexpr int dma_key_delta(int i) {
        // keys between DMA block i's lane chunk and block 0's (rows are 4i*1024/ROW apart)
        return FP8 ? (ROW == 256 ? 16 * (i & 1) + 8 * (i >> 1) : ROW == 128 ? 8 * i : 0) : i * 4096 / ROW;
    }
    // Lazy rescale: the running max is only raised when a tile's max exceeds
    // it by more than this (log2 units); FP8 probabilities then stay below
    // 2^(kPBiasLog2 + 2.5) = 362 < 448.
    static constexpr float RESCALE_LOG2 = FP8 ? 2.5f : 8.0f;
};

// Per-lane constants of the main loop (LDS offsets are within one buffer).
template <class S>
struct LaneMap {
    uint32_t k_addr;                      // score A operand of tile 0 (tile 1: + K_T1_ROWS rows)
    uint32_t v_addr[S::ES == 1 ? 1 : 2];  // PV A operand base(s)
    uint32_t dma_off[S::DMA_SPLIT ? S::DMA_PER_WAVE : 1];   // global byte offset of the lane's K DMA chunk
    uint32_t dma_off_v[S::DMA_SPLIT ? S::DMA_PER_WAVE : 1]; // same for the V tile (its own swizzle)
};

// Issue asynchronous global->LDS loads of one 64-key K tile and V tile.  The
// tile is split into 1 KB blocks; each wave loads DMA_PER_WAVE blocks of
// each, one 16-byte chunk per lane, landing at block + 16 * lane.  The
// lane's global chunk (dma_off) is chosen so that the swizzled LDS layout
// comes out.
template <class S, int BUF>
__device__ __forceinline__ void stage_tile_async(const FwdArgs& a, const TileCursor& c, uint8_t* lds, int wave,
                                                 const LaneMap<S>& L) {
    const uint8_t* const kt = a.kv + c.k_off + (int64_t)c.base * S::GROW;
    const uint8_t* const vt = kt + (int64_t)a.num_kv_heads * a.head_stride;
    uint8_t* const lk = lds + BUF * 2 * S::TILE;
#pragma unroll
    for (int i = 0; i < S::DMA_PER_WAVE; ++i) {
        const int block = 4 * i + wave;
        const uint32_t koff = L.dma_off[S::DMA_SPLIT ? i : 0];
        const uint32_t voff = L.dma_off_v[S::DMA_SPLIT ? i : 0];
        const int delta = S::DMA_SPLIT ? 0 : S::dma_key_delta(i) * S::GROW;
        __builtin_amdgcn_global_load_lds(kt + delta + koff, PCPA_LDS(void, lk + block * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vt + delta + voff, PCPA_LDS(void, lk + S::TILE + block * 1024), 16, 0, 0);
    }
}

// Synchronous staging through registers into buffer 0, widening e4m3 to
// bf16 when the MFMAs are bf16.  Rows at or beyond `valid` get zero V.
template <class S>
__device__ __forceinline__ void stage_tile_sync(const FwdArgs& a, const TileCursor& c, int valid, uint8_t* lds,
                                                int tid) {
    constexpr int LOADS = kKeyTile * S::GROW / (16 * kThreads);
    static_assert((kKeyTile * S::GROW) % (16 * kThreads) == 0, "tile must split into 16-byte chunks per thread");
    const uint8_t* const kpage = a.kv + c.k_off;
    const uint8_t* const vpage = kpage + (int64_t)a.num_kv_heads * a.head_stride;
    uint8_t* const lds_k = lds;
    uint8_t* const lds_v = lds + S::TILE;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int chunk_id = tid + kThreads * i;
        const int key = chunk_id / S::GCHUNKS;
        const int ch = chunk_id - key * S::GCHUNKS;
        const int64_t goff = (int64_t)(c.base + key) * S::GROW + ch * 16;
        const v4i kc = *(const v4i*)(kpage + goff);
        v4i vc = *(const v4i*)(vpage + goff);
        if (key >= valid) vc = v4i{0, 0, 0, 0};
        const int row = lds_row<S::ES == 1>(key);
        const int sw = chunk_swizzle<S::ES == 1, S::CHUNKS>(row);
        const int swv = chunk_swizzle_v<S::ES == 1, S::CHUNKS>(row);
        if constexpr (S::WIDEN) {
            // 16 e4m3 codes become 32 bytes (LDS chunks 2ch, 2ch+1).
            const v2i k0 = e4m3x4_to_bf16x4(kc[0]), k1 = e4m3x4_to_bf16x4(kc[1]);
            const v2i k2 = e4m3x4_to_bf16x4(kc[2]), k3 = e4m3x4_to_bf16x4(kc[3]);
            const v2i v0 = e4m3x4_to_bf16x4(vc[0]), v1 = e4m3x4_to_bf16x4(vc[1]);
            const v2i v2 = e4m3x4_to_bf16x4(vc[2]), v3 = e4m3x4_to_bf16x4(vc[3]);
            const int lo = row * S::ROW + (((2 * ch) ^ sw) << 4);
            const int hi = row * S::ROW + (((2 * ch + 1) ^ sw) << 4);
            *(v4i*)(lds_k + lo) = v4i{k0[0], k0[1], k1[0], k1[1]};
            *(v4i*)(lds_k + hi) = v4i{k2[0], k2[1], k3[0], k3[1]};
            *(v4i*)(lds_v + lo) = v4i{v0[0], v0[1], v1[0], v1[1]};
            *(v4i*)(lds_v + hi) = v4i{v2[0], v2[1], v3[0], v3[1]};
        } else {
            *(v4i*)(lds_k + row * S::ROW + ((ch ^ sw) << 4)) = kc;
            *(v4i*)(lds_v + row * S::ROW + ((ch ^ swv) << 4)) = vc;
        }
    }
}

// Zero V rows [valid, 64) of a staged tile, so that masked (probability 0)
// keys cannot inject NaN bit patterns from unused cache slots.
template <class S>
__device__ __forceinline__ void zero_masked_v(uint8_t* lds_v, int valid, int tid) {
    for (int idx = tid; idx < (kKeyTile - valid) * S::CHUNKS; idx += kThreads) {
        const int key = valid + idx / S::CHUNKS;
        *(v4i*)(lds_v + lds_row<S::ES == 1>(key) * S::ROW + (idx % S::CHUNKS) * 16) = v4i{0, 0, 0, 0};
    }
}

// Online-softmax state of one lane: running max (log2 domain, times the
// lane's score factor), this lane half's share of the running sum, and the
// O^T accumulator tiles.
template <class S>
struct SoftmaxState {
    float m;
    float l;
    v16f o[S::DT];
};

template <class S>
using QOperand = typename std::conditional<S::ES == 1, v8i, v8bf>::type;

// One 64-key tile held in LDS buffer BUF: S^T = K Q^T, masked online
// softmax, O^T += V^T P^T.
// CAUSAL: `valid` differs per lane (the row's causal limit within the tile,
// possibly <= 0).
template <class S, int BUF, bool CAUSAL = false>
__device__ __forceinline__ void compute_tile(const uint8_t* lds, int valid, const QOperand<S> (&qop)[S::QK],
                                             float cscale, const LaneMap<S>& L, int h, SoftmaxState<S>& st) {
    constexpr bool FP8 = S::ES == 1;
    constexpr int ROW = S::ROW, QK = S::QK, DT = S::DT;
    constexpr int KBASE = BUF * 2 * S::TILE;
    constexpr int VBASE = KBASE + S::TILE;
    const uint8_t* const lk = lds + KBASE;

    // ---- S^T = K . Q^T : two 32-key x 32-query tiles --------------------
    v16f s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        s[t] = v16f{};
#pragma unroll
        for (int c = 0; c < QK; ++c) {
            const uint8_t* const kt = lk + t * S::K_T1_ROWS * ROW;
            if constexpr (FP8) {
                const v4i lo = *(const v4i*)(kt + (L.k_addr ^ ((4 * c) << 4)));
                const v4i hi = *(const v4i*)(kt + (L.k_addr ^ ((4 * c + 1) << 4)));
                const v8i aop = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                s[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(aop, qop[c], s[t], 0, 0, 0, 0, 0, 0);
            } else {
                const v4i x = *(const v4i*)(kt + (L.k_addr ^ ((2 * c) << 4)));
                s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, x), qop[c], s[t], 0, 0, 0);
            }
        }
    }

    // ---- mask, online softmax (lazy rescale) ----------------------------
    // (CAUSAL: only tiles that cross some row's limit, a wave-uniform test)
    if (CAUSAL ? __builtin_amdgcn_ballot_w64(valid < kKeyTile) != 0 : valid < kKeyTile) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (key_of_acc<FP8>(t, r, h) >= valid) s[t][r] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
    const float mxs = halves_max(mx) * cscale;
    if (__builtin_amdgcn_ballot_w64(mxs > st.m + S::RESCALE_LOG2) != 0) {
        const float m_new = fmaxf(st.m, mxs);
        const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
        st.l *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) st.o[dt] *= alpha;
        st.m = m_new;
    }
    float psum = 0.f;
    const float shift = (FP8 ? kPBiasLog2 : 0.f) - st.m;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = __builtin_amdgcn_exp2f(fmaf(s[t][r], cscale, shift));
            s[t][r] = p;
            psum += p;
        }
    st.l += psum;

    // ---- O^T += V^T . P^T -----------------------------------------------
    if constexpr (FP8) {
        v8i pop;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                // The first convert's untouched high half is overwritten by
                // the second, so any register serves as its "old" operand.
                int pk = __builtin_amdgcn_cvt_pk_fp8_f32(s[t][4 * q4], s[t][4 * q4 + 1],
                                                         __float_as_int(s[t][4 * q4]), false);
                pk = __builtin_amdgcn_cvt_pk_fp8_f32(s[t][4 * q4 + 2], s[t][4 * q4 + 3], pk, true);
                pop[4 * t + q4] = pk;
            }
        // A operand lane (d row 16*(grp&1)+gl, k-group grp>>1): keys
        // 32*(grp>>1) + [0, 32) of column d, 8 per transposing read; the
        // d tiles are read two at a time, one pair ahead of the MFMAs.
        constexpr int PAIRS = DT / 2;
        v2i x[2][8];
        auto issue = [&](v2i (&buf)[8], int pair) {
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const uint32_t addr = L.v_addr[0] ^ ((2 * (2 * pair + k)) << 4);
                // keys 32g + 8s + m live in LDS rows (8g + m) + {0, 32, 16, 48}[s]
                buf[4 * k + 0] = ds_read_tr8_b64<VBASE + 0 * ROW>(addr);
                buf[4 * k + 1] = ds_read_tr8_b64<VBASE + 32 * ROW>(addr);
                buf[4 * k + 2] = ds_read_tr8_b64<VBASE + 16 * ROW>(addr);
                buf[4 * k + 3] = ds_read_tr8_b64<VBASE + 48 * ROW>(addr);
            }
        };
        issue(x[0], 0);
#pragma unroll
        for (int pair = 0; pair < PAIRS; ++pair) {
            v2i(&cur)[8] = x[pair & 1];
            lds_results_ready(cur);
            if (pair + 1 < PAIRS) issue(x[(pair + 1) & 1], pair + 1);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const v8i aop = {cur[4 * k][0],     cur[4 * k][1],     cur[4 * k + 1][0], cur[4 * k + 1][1],
                                 cur[4 * k + 2][0], cur[4 * k + 2][1], cur[4 * k + 3][0], cur[4 * k + 3][1]};
                st.o[2 * pair + k] =
                    __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(aop, pop, st.o[2 * pair + k], 0, 0, 0, 0, 0, 0);
            }
        }
    } else {
        v8bf pop[2][2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int e2 = 0; e2 < 8; ++e2) pop[t][u][e2] = (__bf16)s[t][8 * u + e2];
        // A operand lane (d row 16*(grp&1)+gl, k-group grp>>1): for score
        // tile t and half u, keys 32t + 16u + 8*(grp>>1) + [0, 8) of column
        // d, 4 per transposing read.
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const uint32_t a0 = L.v_addr[0] ^ ((4 * dt) << 4);
            const uint32_t a1 = L.v_addr[1] ^ ((4 * dt) << 4);
            v2i x[4];
            x[0] = ds_read_tr16_b64<VBASE>(a0);
            x[1] = ds_read_tr16_b64<VBASE>(a1);
            x[2] = ds_read_tr16_b64<VBASE + 16 * ROW>(a0);
            x[3] = ds_read_tr16_b64<VBASE + 16 * ROW>(a1);
            lds_results_ready(x);
            const v4i aop0 = {x[0][0], x[0][1], x[1][0], x[1][1]};
            const v4i aop1 = {x[2][0], x[2][1], x[3][0], x[3][1]};
            st.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, aop0), pop[0][0], st.o[dt], 0, 0, 0);
            st.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, aop1), pop[0][1], st.o[dt], 0, 0, 0);
            v2i y[4];
            y[0] = ds_read_tr16_b64<VBASE + 32 * ROW>(a0);
            y[1] = ds_read_tr16_b64<VBASE + 32 * ROW>(a1);
            y[2] = ds_read_tr16_b64<VBASE + 48 * ROW>(a0);
            y[3] = ds_read_tr16_b64<VBASE + 48 * ROW>(a1);
            lds_results_ready(y);
            const v4i aop2 = {y[0][0], y[0][1], y[1][0], y[1][1]};
            const v4i aop3 = {y[2][0], y[2][1], y[3][0], y[3][1]};
            st.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, aop2), pop[1][0], st.o[dt], 0, 0, 0);
            st.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, aop3), pop[1][1], st.o[dt], 0, 0, 0);
        }
    }
}

// Wait for tile `cur` (in BUF), start the prefetch of `nxt` into the other
// buffer, then compute `cur`.
template <class S, int BUF, bool CAUSAL>
__device__ __forceinline__ void tile_step(const FwdArgs& a, const TileCursor& cur, const TileCursor& nxt,
                                          uint8_t* lds, int wave, int tid, int h, const LaneMap<S>& L,
                                          const QOperand<S> (&qop)[S::QK], float cscale, SoftmaxState<S>& st,
                                          int row_limit) {
    const int valid = min(kKeyTile, cur.n - cur.base);
    uint8_t* const lds_v = lds + BUF * 2 * S::TILE + S::TILE;
    if constexpr (S::NBUF == 2) {
        wait_vmem();      // this wave's loads of the current tile have landed
        __syncthreads();  // ... and every wave's; the other buffer is free
        if (nxt.e < a.num_entries) stage_tile_async<S, BUF ^ 1>(a, nxt, lds, wave, L);
        if (valid < kKeyTile) {
            zero_masked_v<S>(lds_v, valid, tid);
            __syncthreads();
        }
    } else {
        __syncthreads();  // previous tile fully consumed
        if constexpr (S::WIDEN) {
            stage_tile_sync<S>(a, cur, valid, lds, tid);
        } else {
            stage_tile_async<S, 0>(a, cur, lds, wave, L);
            wait_vmem();
            __syncthreads();
            if (valid < kKeyTile) zero_masked_v<S>(lds_v, valid, tid);
        }
        __syncthreads();
    }
    compute_tile<S, BUF, CAUSAL>(lds, CAUSAL ? min(valid, row_limit - cur.base) : valid, qop, cscale, L, h, st);
}

// CAUSAL: causal attention of the current tokens among themselves (their
// K/V are one page of block_size tokens in global order, no block table):
// row (rank, token) sees current keys up to its own global position.  The
// epilogue can then merge the result with a history output (merge_o,
// merge_lse) by log-sum-exp.
template <int D, bool STORE8, bool FP8, bool CAUSAL = false>
__global__ void __launch_bounds__(kThreads, (D == 256 && !FP8) ? 1 : 2) history_fwd_kernel(FwdArgs a) {
    using S = TileShape<D, STORE8, FP8>;
    constexpr int ROW = S::ROW, CHUNKS = S::CHUNKS, QK = S::QK, DT = S::DT;

    __shared__ __attribute__((aligned(1024))) uint8_t lds[S::NBUF * 2 * S::TILE];
    __shared__ int wave_limit[kWaves];

    // ---- XCD-aware work mapping ------------------------------------------
    // Workgroups are dealt to the 8 XCDs round-robin by launch index; give
    // each XCD a contiguous range of (KV head, row tile) work items so that
    // the workgroups sharing an XCD's L2 stream the same KV head together.
    // CAUSAL: work grows with the row tile (later ranks see more current
    // keys) and the keys fit in L2 anyway, so launch the heaviest tiles
    // first, both heads alike, and let the early finishers take the light
    // ones (longest-first balancing over all XCDs).
    const int items = a.row_tiles * a.num_kv_heads;
    int head, row_tile;
    if constexpr (CAUSAL) {
        const int item = blockIdx.x;
        if (item >= items) return;
        head = item % a.num_kv_heads;
        row_tile = a.row_tiles - 1 - item / a.num_kv_heads;
    } else {
        const int per_xcd = (items + 7) / 8;
        const int item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
        if (item >= items) return;
        head = item / a.row_tiles;
        row_tile = item - head * a.row_tiles;
    }

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31;  // query column of the score tile / A-operand row
    const int h = lane >> 5;  // k-group (lane half)
    const int grp = lane >> 4;
    const int gl = lane & 15;

    // ---- this lane's query row -------------------------------------------
    const int row = row_tile * kRowsPerGroup + wave * kRowsPerWave + j;
    const bool row_ok = row < a.rows_per_head;
    const int rowc = row_ok ? row : a.rows_per_head - 1;
    const int rank = rowc / a.group_rows;
    const int rem = rowc - rank * a.group_rows;
    const int head_in_group = rem / a.local_q;
    const int tok = rem - head_in_group * a.local_q;
    const int64_t row_off =
        ((int64_t)(rank * a.num_q_heads + head * a.group + head_in_group) * a.local_q + tok) * D * 2;
    const uint8_t* const qrow = a.q + row_off;

    // ---- Q^T operand (register resident for the whole history) ------------
    QOperand<S> qop[QK];
    float cscale;
    if constexpr (FP8) {
        // lane (j, h) holds d = 64c + 32h + [0, 32) of its row, as e4m3.
        float amax = 0.f;
#pragma unroll
        for (int c = 0; c < QK; ++c) {
#pragma unroll
            for (int part = 0; part < 4; ++part) {
                const v4i raw = *(const v4i*)(qrow + (64 * c + 32 * h) * 2 + 16 * part);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t u = (uint32_t)raw[w];
                    amax = fmaxf(amax, fabsf(bf16_bits_to_f32(u & 0xffffu)));
                    amax = fmaxf(amax, fabsf(bf16_bits_to_f32(u >> 16)));
                }
            }
        }
        amax = halves_max(amax);
        const float inv = amax > 0.f ? kFp8Max / amax : 1.f;
        const float sigma = amax > 0.f ? amax / kFp8Max : 1.f;
#pragma unroll
        for (int c = 0; c < QK; ++c) {
#pragma unroll
            for (int part = 0; part < 4; ++part) {
                const v4i raw = *(const v4i*)(qrow + (64 * c + 32 * h) * 2 + 16 * part);
#pragma unroll
                for (int w = 0; w < 2; ++w) {
                    const uint32_t u0 = (uint32_t)raw[2 * w], u1 = (uint32_t)raw[2 * w + 1];
                    int pk = __builtin_amdgcn_cvt_pk_fp8_f32(bf16_bits_to_f32(u0 & 0xffffu) * inv,
                                                             bf16_bits_to_f32(u0 >> 16) * inv, 0, false);
                    pk = __builtin_amdgcn_cvt_pk_fp8_f32(bf16_bits_to_f32(u1 & 0xffffu) * inv,
                                                         bf16_bits_to_f32(u1 >> 16) * inv, pk, true);
                    qop[c][2 * part + w] = pk;
                }
            }
        }
        cscale = sigma * a.score_scale;
    } else {
        // lane (j, h) holds d = 16c + 8h + [0, 8) of its row.
#pragma unroll
        for (int c = 0; c < QK; ++c) {
            const v4i raw = *(const v4i*)(qrow + (16 * c + 8 * h) * 2);
            qop[c] = __builtin_bit_cast(v8bf, raw);
        }
        cscale = a.score_scale;
    }

    // ---- per-lane LDS / DMA offsets ---------------------------------------
    // Row offsets are multiples of ROW (a power of two) and the chunk field
    // lies below ROW, so XOR-ing a constant into the chunk field is one v_xor.
    LaneMap<S> L;
    {
        const int row = lds_row<FP8>(key_of_row<FP8>(0, j));
        const int first_chunk = FP8 ? 2 * h : h;
        L.k_addr = row * ROW + ((first_chunk ^ chunk_swizzle<FP8, CHUNKS>(row)) << 4);
    }
    if constexpr (FP8) {
        // key 32*(grp>>1) + (gl>>1) (+ 8s for the other reads) -> row below
        const int row = lds_row<FP8>(32 * (grp >> 1) + (gl >> 1));
        L.v_addr[0] = row * ROW + (((grp & 1) ^ chunk_swizzle_v<FP8, CHUNKS>(row)) << 4) + 8 * (gl & 1);
    } else {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const int vkey = 8 * (grp >> 1) + 4 * s2 + (gl >> 2);  // + 16u + 32t: same swizzle
            const int dbyte = 2 * (16 * (grp & 1) + 4 * (gl & 3));
            L.v_addr[s2] = vkey * ROW + (((dbyte >> 4) ^ chunk_swizzle<FP8, CHUNKS>(vkey)) << 4) + (dbyte & 15);
        }
    }
#pragma unroll
    for (int i = 0; i < (S::DMA_SPLIT ? S::DMA_PER_WAVE : 1); ++i) {
        const int byte = (4 * i + wave) * 1024 + lane * 16;
        const int row = byte / ROW;
        const int pos = (byte % ROW) / 16;
        L.dma_off[i] = lds_row<FP8>(row) * S::GROW + (pos ^ chunk_swizzle<FP8, CHUNKS>(row)) * 16;
        L.dma_off_v[i] = lds_row<FP8>(row) * S::GROW + (pos ^ chunk_swizzle_v<FP8, CHUNKS>(row)) * 16;
    }

    // ---- walk the block table -----------------------------------------------
    SoftmaxState<S> st;
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) st.o[dt] = v16f{};

    // CAUSAL: the row sees current keys [0, g] (g its global current
    // position, layout.py:10-16 inverted); the workgroup stops after the
    // tile holding the largest g of its rows.
    int row_limit = 0, group_limit = 0;
    if constexpr (CAUSAL) {
        row_limit = ((tok / a.interleave) * a.pcp + rank) * a.interleave + tok % a.interleave + 1;
        int w = row_limit;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) w = max(w, __shfl_xor(w, off));
        if (lane == 0) wave_limit[wave] = w;
        __syncthreads();
        group_limit = wave_limit[0];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) group_limit = max(group_limit, wave_limit[i]);
    }
    auto advance = [&](const TileCursor& c) {
        if constexpr (CAUSAL) {
            const TileCursor n = next_current_tile(a, head, c);
            return n.base < group_limit ? n : TileCursor{a.num_entries, 0, 0, 0};
        } else {
            return next_tile(a, head, c);
        }
    };

    TileCursor cur = advance(TileCursor{-1, 0, 0, 0});
    if constexpr (S::NBUF == 2) {
        if (cur.e < a.num_entries) stage_tile_async<S, 0>(a, cur, lds, wave, L);
    }
    while (cur.e < a.num_entries) {
        TileCursor nxt = advance(cur);
        tile_step<S, 0, CAUSAL>(a, cur, nxt, lds, wave, tid, h, L, qop, cscale, st, row_limit);
        cur = nxt;
        if constexpr (S::NBUF == 2) {
            if (cur.e >= a.num_entries) break;
            nxt = advance(cur);
            tile_step<S, 1, CAUSAL>(a, cur, nxt, lds, wave, tid, h, L, qop, cscale, st, row_limit);
            cur = nxt;
        }
    }

    // ---- epilogue: O = O^T / l, bf16; log-sum-exp; merge -------------------
    const float l_tot = halves_sum(st.l);
    float scale = l_tot > 0.f ? a.v_scale / l_tot : 0.f;
    // sum_k exp(score_k) = l * 2^(m - bias): P was 2^(x - m + bias)
    float lse = l_tot > 0.f ? __logf(l_tot) + (st.m - (FP8 ? kPBiasLog2 : 0.f)) * kLn2 : -INFINITY;
    const int64_t row_index = row_off / (D * 2);
    float hist_weight = 0.f;
    if (CAUSAL && a.merge_o) {
        // out = (e^lse_h O_h + e^lse O) / (e^lse_h + e^lse)
        const float lse_h = a.merge_lse[row_index];
        const float mx = fmaxf(lse_h, lse);
        const float wh = lse_h == -INFINITY ? 0.f : __expf(lse_h - mx);
        const float wc = __expf(lse - mx);
        hist_weight = wh / (wh + wc);
        scale *= wc / (wh + wc);
        lse = mx + __logf(wh + wc);
    }
    if (row_ok) {
        uint8_t* const orow = a.out + row_off;
        const uint8_t* const hrow = CAUSAL && a.merge_o ? a.merge_o + row_off : nullptr;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int d = 32 * dt + 8 * r4 + 4 * h;
                float o0 = st.o[dt][4 * r4 + 0] * scale, o1 = st.o[dt][4 * r4 + 1] * scale;
                float o2 = st.o[dt][4 * r4 + 2] * scale, o3 = st.o[dt][4 * r4 + 3] * scale;
                if (CAUSAL && hrow) {
                    const v2i hv = *(const v2i*)(hrow + 2 * d);
                    o0 = fmaf(hist_weight, bf16_bits_to_f32((uint32_t)hv[0] & 0xffffu), o0);
                    o1 = fmaf(hist_weight, bf16_bits_to_f32((uint32_t)hv[0] >> 16), o1);
                    o2 = fmaf(hist_weight, bf16_bits_to_f32((uint32_t)hv[1] & 0xffffu), o2);
                    o3 = fmaf(hist_weight, bf16_bits_to_f32((uint32_t)hv[1] >> 16), o3);
                }
                const __bf16 v0 = (__bf16)o0, v1 = (__bf16)o1, v2 = (__bf16)o2, v3 = (__bf16)o3;
                const uint32_t w0 = (uint32_t)__builtin_bit_cast(uint16_t, v0) |
                                    ((uint32_t)__builtin_bit_cast(uint16_t, v1) << 16);
                const uint32_t w1 = (uint32_t)__builtin_bit_cast(uint16_t, v2) |
                                    ((uint32_t)__builtin_bit_cast(uint16_t, v3) << 16);
                *(v2i*)(orow + 2 * d) = v2i{(int)w0, (int)w1};
            }
        if (a.lse && h == 0) a.lse[row_index] = lse;
    }
}


// ============================================================================
// Helpers of the overlap kernel below.
// ============================================================================
namespace ovl {

// Starting reference max: finite, so that a phantom tile (all scores -inf)
// gives alpha = exp2(0) = 1 and probabilities of 0, and far below any real
// score, so that the first real tile gives alpha = 0.
constexpr float kMaxFloor = -1.0e30f;

// A 16-byte chunk of zeros in global memory: the source of the V rows of a
// partial tile that lie past its valid length.
__device__ __attribute__((aligned(16))) uint8_t zero_chunk[16];

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

template <int OFF>
__device__ __forceinline__ v4i ds_read_b128(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
    v4i r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
}
// s_waitcnt lgkmcnt(N) with the awaited read results as operands, so that
// no use of them is scheduled before the wait.
template <int N>
__device__ __forceinline__ void lds_wait(v4i (&x)[2]) {
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(x[0]), "+v"(x[1]) : "i"(N));
}
template <int N>
__device__ __forceinline__ void lds_wait(v2i (&x)[4]) {
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]) : "i"(N));
}
// max(a, b, c) in one v_max3_f32, without the NaN-quieting moves the
// compiler adds around fmaxf of accumulator reads.  Inputs are scores or
// -inf, never NaN.
__device__ __forceinline__ float max3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
// s_waitcnt vmcnt(N), expcnt/lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmem_le() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Empty asm statements pin a slice's results where the slice is written:
// without them the compiler sinks the probabilities (used only in the next
// iteration) below the PV MFMAs, and nothing overlaps.
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(int& x) { asm volatile("" : "+v"(x)); }

// Scores of keys at or past `valid` become -inf.  Key of accumulator (t, r)
// in lane half h: 32h + 16t + r (key_of_acc), compared as 16t + r against
// valid - 32h so that the per-register side is an inline constant.
__device__ __forceinline__ void mask_tail(v16f (&s)[2], int valid, int h) {
    const int lim = valid - 32 * h;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (16 * t + r >= lim) s[t][r] = -INFINITY;
}

}  // namespace ovl


// ============================================================================
// FP8 kernel with an in-wave MFMA/softmax overlap (head_dim 128 and 256).
//
// gfx950 overlaps an MFMA with independent VALU work of the same wave, but a
// single wave per SIMD issues too slowly to keep the matrix core busy.  So
// this kernel runs two waves per SIMD (8 waves, 256 query rows per
// workgroup; every wave sees the same K/V tiles, which halves the LDS-DMA
// work per row) and splits each wave's tile step into two halves:
//
//   S half:   S^T(t) = K(t) Q^T                              (MFMA only)
//   PV half:  O^T += V^T(t-1) P^T(t-1), interleaved MFMA by MFMA with the
//             softmax of S(t) -> P(t); then O^T is rescaled if tile t raised
//             the running max (lazily, so rarely)
//
// Waves 0-3 run [S(j) | PV(j-1) + softmax(j)] in iteration j and waves 4-7
// run [PV(j-2) + softmax(j-1) | S(j)], so that on every SIMD one wave feeds
// the matrix core alone while the other interleaves its PV MFMAs with its
// softmax.  One barrier per iteration.  K and V tiles live in separate
// four-stage LDS rings (tile t in stage t % 4): K(j+2) and V(j+1) are
// requested at the top of iteration j.  Tiles before the first and after
// the last are "phantom" tiles without valid keys: their scores are masked
// to -inf (P = 0, softmax state unchanged, since the running max starts at
// a finite floor) and their V stages hold zeros (zeroed up front for tiles
// -2 and -1, loaded from zero_chunk afterwards), so every wave runs the same
// loop body until the last real PV.  Everything is register resident in 256
// VGPRs, so the MFMAs write the scores where the softmax reads them.
// ============================================================================
namespace ovl {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsPerGroup = kWaves * 32;
constexpr int kStages = 4;

template <int D>
struct Shape {
    static_assert(D == 128 || D == 256, "overlap kernel covers head_dim 128 and 256");
    static constexpr int ROW = D;            // e4m3 bytes of one key row
    static constexpr int CHUNKS = D / 16;
    static constexpr int TILE = kKeyTile * ROW;
    static constexpr int RING = kStages * TILE;
    static constexpr int QK = D / 64;        // k-steps of the score MFMA
    static constexpr int NX = 2 * QK;        // score MFMAs per tile
    static constexpr int DT = D / 32;        // PV MFMAs per tile
    static constexpr int DPW = TILE / 1024 / kWaves;  // 1 KB DMA blocks per wave per K (or V) tile
    // DMA block 8i + wave lands 32i LDS rows after block `wave` (rows
    // < 32): lds_row maps row bit 5 to key bit 3, so its chunk is 8i keys
    // further on, with the same swizzle.
    static constexpr int DMA_KEY_STEP = 8;
    static_assert(DPW == 1 || 8 * 1024 / ROW == 32, "block rows must step by 32");
    // Softmax micro-slices [pv_begin(i), pv_begin(i+1)) run beside PV MFMA i.
    static constexpr int pv_begin(int i) {
        constexpr int b256[] = {0, 4, 6, 7, 8, 9, 10, 11, 14};
        constexpr int b128[] = {0, 5, 8, 11, 14};
        return D == 256 ? b256[i] : b128[i];
    }
};

struct Lanes {
    uint32_t k_addr;  // score operand, K stage 0, k-step 0, low 16 bytes
    uint32_t v_addr;  // PV operand, V stage 0, d tile 0 (includes the ring offset)
    uint32_t dma_k;   // byte offset of the lane's K chunk of DMA block `wave` in a tile
    uint32_t dma_v;   // same for V (its own swizzle)
};

// Tiles j-1 .. j+2 of iteration j.  e < 0: before the first tile;
// e >= num_entries: after the last (both phantom, valid length 0).
struct Cursors {
    TileCursor cm1, c0, c1, c2;
};

__device__ __forceinline__ bool is_real(const FwdArgs& a, const TileCursor& c) {
    return c.e >= 0 && c.e < a.num_entries;
}

// Per-lane online-softmax state (log2 domain) and the scratch of the
// softmax in progress.  l is the full row sum (both lane halves hold it).
struct SoftmaxRow {
    float cscale;   // Q row scale * softmax_scale * k_scale * log2(e)
    float cscale8;  // 8 * cscale
    float m;        // reference max the probabilities are taken against
    float l;        // running sum of the e4m3 probabilities, same reference
    float alpha;    // rescale factor of the last softmax (1: no change)
    float mx, m_use, shift;
};

// Micro-slice K of the online softmax of one score tile s (32 scores per
// lane, masked keys already -inf), producing P as e4m3 in PV B-operand
// order.  0-3: running max over 8 scores each; 4: new reference max (it lags
// the tile max by at most 2.5, so probabilities stay below 2^(6 + 2.5) =
// 362 < 448) and rescale factor; 5-12: four probabilities each, one dword
// of P; 13: reference update.  The row sum is taken from P by an MFMA.
//
// FAST: P = 2^x (x = s * cscale + 6 - m_use) is produced directly as its
// e4m3 code round(8x + 56), clamped to [0, 255] by v_cvt_pk_u8_f32.  For
// x = n + f that code decodes to 2^n (1 + f) rounded to 3 mantissa bits:
// the exponential is interpolated linearly between powers of two (at most
// 6.1% high, a shape error of +-3% once normalised), which is the e4m3
// rounding step of P itself.  Codes below 8 are the e4m3 subnormals of
// values under 2^-6, i.e. under 2^-14 of the tile max.  Otherwise P =
// v_exp_f32 rounded by v_cvt_pk_fp8_f32.
template <int K, bool FAST>
__device__ __forceinline__ void softmax_slice(const v16f (&s)[2], v8i& p, SoftmaxRow& sm) {
    if constexpr (K < 4) {
        constexpr int t = K >> 1, r = 8 * (K & 1);
        float mx = max3(s[t][r], s[t][r + 1], s[t][r + 2]);
        mx = max3(mx, s[t][r + 3], s[t][r + 4]);
        mx = max3(mx, s[t][r + 5], s[t][r + 6]);
        mx = K == 0 ? max3(mx, s[t][r + 7], s[t][r + 7]) : max3(mx, s[t][r + 7], sm.mx);
        sm.mx = mx;
        pin(sm.mx);
    } else if constexpr (K == 4) {
        const float mxs = halves_max(sm.mx) * sm.cscale;
        sm.m_use = fmaxf(sm.m, mxs - 2.5f);
        sm.alpha = __builtin_amdgcn_exp2f(sm.m - sm.m_use);
        // FAST: 8x + 56 = s * 8 cscale + (8 (6 - m_use) + 56)
        sm.shift = FAST ? fmaf(-8.f, sm.m_use, 8.f * kPBiasLog2 + 56.f) : kPBiasLog2 - sm.m_use;
        pin(sm.m_use);
        pin(sm.alpha);
        pin(sm.shift);
    } else if constexpr (K < 13) {
        constexpr int w = K - 5, t = w >> 2, r0 = 4 * (w & 3);
        int word;
        if constexpr (FAST) {
            word = __builtin_amdgcn_cvt_pk_u8_f32(fmaf(s[t][r0 + 0], sm.cscale8, sm.shift), 0, 0);
            word = __builtin_amdgcn_cvt_pk_u8_f32(fmaf(s[t][r0 + 1], sm.cscale8, sm.shift), 1, word);
            word = __builtin_amdgcn_cvt_pk_u8_f32(fmaf(s[t][r0 + 2], sm.cscale8, sm.shift), 2, word);
            word = __builtin_amdgcn_cvt_pk_u8_f32(fmaf(s[t][r0 + 3], sm.cscale8, sm.shift), 3, word);
        } else {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(s[t][r0 + 0], sm.cscale, sm.shift));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(s[t][r0 + 1], sm.cscale, sm.shift));
            const float p2 = __builtin_amdgcn_exp2f(fmaf(s[t][r0 + 2], sm.cscale, sm.shift));
            const float p3 = __builtin_amdgcn_exp2f(fmaf(s[t][r0 + 3], sm.cscale, sm.shift));
            // The first convert's untouched high half is overwritten by the
            // second, so any register serves as its "old" operand.
            const int pk = __builtin_amdgcn_cvt_pk_fp8_f32(p0, p1, __float_as_int(p0), false);
            word = __builtin_amdgcn_cvt_pk_fp8_f32(p2, p3, pk, true);
        }
        pin(word);
        p[w] = word;
    } else {
        sm.m = sm.m_use;
        pin(sm.m);
    }
}

template <int LO, int HI, bool FAST>
__device__ __forceinline__ void softmax_slices(const v16f (&s)[2], v8i& p, SoftmaxRow& sm) {
    if constexpr (LO < HI) {
        softmax_slice<LO, FAST>(s, p, sm);
        softmax_slices<LO + 1, HI, FAST>(s, p, sm);
    }
}

// Key of the lane's chunk of DMA block i (LDS byte (8i + wave) * 1024 +
// 16 * lane, rows permuted by lds_row).
template <class S>
__device__ __forceinline__ int dma_chunk_key(int i, int wave_off) {
    return lds_row<true>((i * kWaves * 1024 + wave_off + __lane_id() * 16) / S::ROW);
}

// Issue the K tile of cursor c into K stage st.  (Pointers are formed in
// plain variables: address-space casts of expressions that depend on S trip
// the host compilation pass.)
template <class S>
__device__ __forceinline__ void load_k(const FwdArgs& a, const TileCursor& c, uint8_t* lds, int st, int wave_off,
                                       uint32_t off) {
    const uint8_t* const kt = a.kv + c.k_off + (int64_t)c.base * S::ROW + off;
    uint8_t* const dst = lds + st * S::TILE + wave_off;
#pragma unroll
    for (int i = 0; i < S::DPW; ++i) {
        const uint8_t* const src = kt + i * S::DMA_KEY_STEP * S::ROW;
        uint8_t* const d = dst + i * (kWaves * 1024);
        __builtin_amdgcn_global_load_lds(src, PCPA_LDS(void, d), 16, 0, 0);
    }
}

// Issue the V tile of cursor c into V stage st.  Rows past the valid length
// (all rows of a phantom tile) come from zero_chunk, so V stages of masked
// keys hold zeros and the number of loads per tile never changes.
template <class S>
__device__ __forceinline__ void load_v(const FwdArgs& a, const TileCursor& c, uint8_t* lds, int st, int wave_off,
                                       uint32_t off, bool real) {
    const uint8_t* const vt =
        a.kv + c.k_off + (int64_t)c.base * S::ROW + (int64_t)a.num_kv_heads * a.head_stride + off;
    uint8_t* const dst = lds + S::RING + st * S::TILE + wave_off;
    const int valid = real ? c.n - c.base : 0;
    if (valid >= kKeyTile) {
#pragma unroll
        for (int i = 0; i < S::DPW; ++i) {
            const uint8_t* const src = vt + i * S::DMA_KEY_STEP * S::ROW;
            uint8_t* const d = dst + i * (kWaves * 1024);
            __builtin_amdgcn_global_load_lds(src, PCPA_LDS(void, d), 16, 0, 0);
        }
    } else {
        const uint8_t* const zero = zero_chunk;
#pragma unroll
        for (int i = 0; i < S::DPW; ++i) {
            const uint8_t* const src =
                dma_chunk_key<S>(i, wave_off) < valid ? vt + i * S::DMA_KEY_STEP * S::ROW : zero;
            uint8_t* const d = dst + i * (kWaves * 1024);
            __builtin_amdgcn_global_load_lds(src, PCPA_LDS(void, d), 16, 0, 0);
        }
    }
}

// S half: S^T = K Q^T from K stage KST; operand reads one MFMA ahead (the
// other wave on the SIMD covers the latency).  PREFETCH_V: the last slot
// starts the first V-operand read of the PV half that follows (stage VST).
// Also adds to l the row sum of P_last, the probabilities the preceding PV
// half consumed, scaled by the alpha that PV half applied.
template <int D, int KST, bool PREFETCH_V, int VST>
__device__ __forceinline__ void s_half(uint32_t k_addr, uint32_t v_addr, const v8i (&q)[Shape<D>::QK], v16f (&s)[2],
                                       v2i (&xv)[4], const v8i& p_last, SoftmaxRow& sm) {
    using S = Shape<D>;
    // ones (e4m3 1.0) x P_last puts sum_k P_last[k][q] in every accumulator
    // of query column q.  The ones operand is rebuilt from an opaque register
    // instead of occupying 8 VGPRs for good.
    int one = 0x38383838;
    asm volatile("" : "+v"(one));
    const v8i ones = {one, one, one, one, one, one, one, one};
    v16f rowsum = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ones, p_last, v16f{}, 0, 0, 0, 0, 0, 0);
    v4i kr[2][2];
    auto issue_k = [&](auto oc) {
        constexpr int op = decltype(oc)::value, c = op >> 1, t = op & 1;
        constexpr int off = KST * S::TILE + t * 16 * S::ROW;
        kr[op & 1][0] = ds_read_b128<off>(k_addr ^ ((4 * c) << 4));
        kr[op & 1][1] = ds_read_b128<off>(k_addr ^ ((4 * c + 1) << 4));
    };
    issue_k(std::integral_constant<int, 0>{});
    static_for<0, S::NX>([&](auto oc) {
        constexpr int op = decltype(oc)::value, c = op >> 1, t = op & 1;
        lds_wait<0>(kr[op & 1]);
        if constexpr (op + 1 < S::NX) {
            issue_k(std::integral_constant<int, op + 1>{});
        } else if constexpr (PREFETCH_V) {
            // keys 32g + 8s + m of the d tile live in LDS rows (8g + m) + {0, 32, 16, 48}[s]
            constexpr int off = VST * S::TILE;
            xv[0] = ds_read_tr8_b64<off + 0 * S::ROW>(v_addr);
            xv[1] = ds_read_tr8_b64<off + 32 * S::ROW>(v_addr);
            xv[2] = ds_read_tr8_b64<off + 16 * S::ROW>(v_addr);
            xv[3] = ds_read_tr8_b64<off + 48 * S::ROW>(v_addr);
        }
        const v4i lo = kr[op & 1][0], hi = kr[op & 1][1];
        const v8i kop = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        s[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kop, q[c], c == 0 ? v16f{} : s[t], 0, 0, 0, 0, 0, 0);
    });
    // All 16 row-sum registers stay allocated until here: the inline-asm LDS
    // reads above are invisible to the hazard checks and must not be given
    // registers that the in-flight MFMA is still going to write.
    asm volatile("" : "+v"(rowsum));
    sm.l = fmaf(rowsum[0], sm.alpha, sm.l);
}

// PV half: O^T += V^T P_old^T from V stage VST, beside the softmax of s
// (valid keys < valid) into p_new; then the lazy O^T rescale.  PREFETCHED:
// the first V-operand read was issued by the S half.
template <int D, int VST, bool PREFETCHED, bool FAST>
__device__ __forceinline__ void pv_half(uint32_t v_addr, v2i (&xv0)[4], v16f (&o)[Shape<D>::DT], const v8i& p_old,
                                        v16f (&s)[2], v8i& p_new, SoftmaxRow& sm, int valid, int h) {
    using S = Shape<D>;
    if (valid < kKeyTile) mask_tail(s, valid, h);
    v2i xv1[4];
    auto buf = [&](auto dc) -> v2i(&)[4] {
        if constexpr ((decltype(dc)::value & 1) == 0)
            return xv0;
        else
            return xv1;
    };
    auto issue_v = [&](auto dc) {
        constexpr int dt = decltype(dc)::value;
        constexpr int off = VST * S::TILE;
        const uint32_t addr = v_addr ^ ((2 * dt) << 4);
        v2i(&x)[4] = buf(dc);
        x[0] = ds_read_tr8_b64<off + 0 * S::ROW>(addr);
        x[1] = ds_read_tr8_b64<off + 32 * S::ROW>(addr);
        x[2] = ds_read_tr8_b64<off + 16 * S::ROW>(addr);
        x[3] = ds_read_tr8_b64<off + 48 * S::ROW>(addr);
    };
    if constexpr (!PREFETCHED) issue_v(std::integral_constant<int, 0>{});
    static_for<0, S::DT>([&](auto dc) {
        constexpr int dt = decltype(dc)::value;
        v2i(&x)[4] = buf(dc);
        lds_wait<0>(x);
        if constexpr (dt + 1 < S::DT) issue_v(std::integral_constant<int, dt + 1>{});
        const v8i vop = {x[0][0], x[0][1], x[1][0], x[1][1], x[2][0], x[2][1], x[3][0], x[3][1]};
        o[dt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vop, p_old, o[dt], 0, 0, 0, 0, 0, 0);
        softmax_slices<S::pv_begin(dt), S::pv_begin(dt + 1), FAST>(s, p_new, sm);
        __builtin_amdgcn_sched_barrier(0);
    });
    // O^T gained P_old's tile; both O^T and l move to the new reference (l
    // gains P_old's row sum, times this alpha, in the next S half).
    sm.l *= sm.alpha;
    if (__builtin_amdgcn_ballot_w64(sm.alpha < 1.f) != 0) {
#pragma unroll
        for (int dt = 0; dt < S::DT; ++dt) o[dt] *= sm.alpha;
    }
}

// Iteration j, J4 = j mod 4; LATE: waves 4-7 (PV half first, one tile behind).
template <int D, int J4, bool LATE, bool FAST>
__device__ __forceinline__ void iteration(const FwdArgs& a, uint8_t* lds, int wave, int h, const Lanes& L,
                                          const v8i (&q)[Shape<D>::QK], v16f (&s)[2], v8i (&pbuf)[2],
                                          v16f (&o)[Shape<D>::DT], SoftmaxRow& sm, Cursors& cs, int head) {
    using S = Shape<D>;
    constexpr int KST = J4;  // K(j)

    // ---- K(j) and V(j-1) have landed (for every wave) ----------------------
    // Loads issued one iteration ago may be pending: V(j), and K(j+1) if tile
    // j+1 is real.
    if (is_real(a, cs.c1))
        wait_vmem_le<2 * S::DPW>();
    else
        wait_vmem_le<S::DPW>();
    __builtin_amdgcn_s_barrier();
    // K stage (j+2) % 4 held K(j-2) and V stage (j+1) % 4 held V(j-3); both
    // were last read in iteration j-1.  The wave offset and operand bases
    // are made opaque so that the DMA destinations and operand addresses are
    // recomputed in the loop rather than hoisted and spilled.
    int wave_off = wave * 1024;
    uint32_t k_addr = L.k_addr, v_addr = L.v_addr;
    asm volatile("" : "+s"(wave_off), "+v"(k_addr), "+v"(v_addr));
    if (is_real(a, cs.c2)) load_k<S>(a, cs.c2, lds, (J4 + 2) % kStages, wave_off, L.dma_k);
    load_v<S>(a, cs.c1, lds, (J4 + 1) % kStages, wave_off, L.dma_v, is_real(a, cs.c1));

    v2i xv[4];
    if constexpr (!LATE) {
        // S(j), then PV(j-1) beside softmax(j)
        constexpr int VST = (J4 + 3) % kStages;
        s_half<D, KST, true, VST>(k_addr, v_addr, q, s, xv, pbuf[J4 & 1], sm);
        pv_half<D, VST, true, FAST>(v_addr, xv, o, pbuf[(J4 + 1) & 1], s, pbuf[J4 & 1], sm,
                              is_real(a, cs.c0) ? cs.c0.n - cs.c0.base : 0, h);
    } else {
        // PV(j-2) beside softmax(j-1), then S(j)
        constexpr int VST = (J4 + 2) % kStages;
        pv_half<D, VST, false, FAST>(v_addr, xv, o, pbuf[J4 & 1], s, pbuf[(J4 + 1) & 1], sm,
                               is_real(a, cs.cm1) ? cs.cm1.n - cs.cm1.base : 0, h);
        s_half<D, KST, false, 0>(k_addr, v_addr, q, s, xv, pbuf[J4 & 1], sm);
    }

    cs.cm1 = cs.c0;
    cs.c0 = cs.c1;
    cs.c1 = cs.c2;
    if (is_real(a, cs.c2)) cs.c2 = next_tile(a, head, cs.c2);
}

// The loop of one wave group; iteration j runs while j <= T + 1 (T tiles).
template <int D, bool LATE, bool FAST>
__device__ __forceinline__ void walk(const FwdArgs& a, uint8_t* lds, int wave, int h, const Lanes& L,
                                     const v8i (&q)[Shape<D>::QK], v16f (&s)[2], v8i (&pbuf)[2],
                                     v16f (&o)[Shape<D>::DT], SoftmaxRow& sm, Cursors cs, int head) {
    for (;;) {
        // after iteration j the loop ends if tile j-1 was past the last tile
        bool done = cs.cm1.e >= a.num_entries;
        iteration<D, 0, LATE, FAST>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head);
        if (done) break;
        done = cs.cm1.e >= a.num_entries;
        iteration<D, 1, LATE, FAST>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head);
        if (done) break;
        done = cs.cm1.e >= a.num_entries;
        iteration<D, 2, LATE, FAST>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head);
        if (done) break;
        done = cs.cm1.e >= a.num_entries;
        iteration<D, 3, LATE, FAST>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head);
        if (done) break;
    }
}

// LSE: also write each row's log-sum-exp (a separate instantiation, so that
// the plain one keeps its register allocation).
// SPLIT: the workgroup walks only its split's share of the table entries
// and writes a normalised FP32 partial output and log-sum-exp (merged by
// merge_splits_kernel).
template <int D, bool FAST, bool LSE, bool SPLIT = false>
__global__ void __launch_bounds__(kThreads, 1) history_fwd_overlap(FwdArgs a) {
    using S = Shape<D>;
    constexpr int QK = S::QK, DT = S::DT, ROW = S::ROW, CHUNKS = S::CHUNKS;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * S::RING];

    // ---- XCD-aware work mapping (as history_fwd_kernel) ---------------------
    // Items run row tile fastest, so an XCD's workgroups share one (KV head,
    // split) and with it the pages they stream.
    const int splits = SPLIT ? a.splits : 1;
    const int items = a.row_tiles * a.num_kv_heads * splits;
    const int per_xcd = (items + 7) / 8;
    const int item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (item >= items) return;
    const int row_tile = item % a.row_tiles;
    const int head = item / a.row_tiles / splits;
    const int split = item / a.row_tiles - head * splits;
    int entry_begin = 0;
    if constexpr (SPLIT) {
        entry_begin = (int)((int64_t)a.num_entries * split / splits);
        a.num_entries = (int)((int64_t)a.num_entries * (split + 1) / splits);
    }

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j = lane & 31;
    const int h = lane >> 5;
    const int grp = lane >> 4;
    const int gl = lane & 15;

    // ---- this lane's query row and its e4m3 Q^T operand ---------------------
    const int row = row_tile * kRowsPerGroup + wave * 32 + j;
    const bool row_ok = row < a.rows_per_head;
    const int rowc = row_ok ? row : a.rows_per_head - 1;
    const int rank = rowc / a.group_rows;
    const int rem = rowc - rank * a.group_rows;
    const int head_in_group = rem / a.local_q;
    const int tok = rem - head_in_group * a.local_q;
    const int64_t row_off =
        ((int64_t)(rank * a.num_q_heads + head * a.group + head_in_group) * a.local_q + tok) * D * 2;
    const uint8_t* const qrow = a.q + row_off;

    v8i q[QK];
    SoftmaxRow sm;
    {
        // lane (j, h) holds d = 64c + 32h + [0, 32) of its row, as e4m3.
        float amax = 0.f;
#pragma unroll
        for (int c = 0; c < QK; ++c)
#pragma unroll
            for (int part = 0; part < 4; ++part) {
                const v4i raw = *(const v4i*)(qrow + (64 * c + 32 * h) * 2 + 16 * part);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t u = (uint32_t)raw[w];
                    amax = fmaxf(amax, fabsf(bf16_bits_to_f32(u & 0xffffu)));
                    amax = fmaxf(amax, fabsf(bf16_bits_to_f32(u >> 16)));
                }
            }
        amax = halves_max(amax);
        const float inv = amax > 0.f ? kFp8Max / amax : 1.f;
        const float sigma = amax > 0.f ? amax / kFp8Max : 1.f;
#pragma unroll
        for (int c = 0; c < QK; ++c)
#pragma unroll
            for (int part = 0; part < 4; ++part) {
                const v4i raw = *(const v4i*)(qrow + (64 * c + 32 * h) * 2 + 16 * part);
#pragma unroll
                for (int w = 0; w < 2; ++w) {
                    const uint32_t u0 = (uint32_t)raw[2 * w], u1 = (uint32_t)raw[2 * w + 1];
                    int pk = __builtin_amdgcn_cvt_pk_fp8_f32(bf16_bits_to_f32(u0 & 0xffffu) * inv,
                                                             bf16_bits_to_f32(u0 >> 16) * inv, 0, false);
                    pk = __builtin_amdgcn_cvt_pk_fp8_f32(bf16_bits_to_f32(u1 & 0xffffu) * inv,
                                                         bf16_bits_to_f32(u1 >> 16) * inv, pk, true);
                    q[c][2 * part + w] = pk;
                }
            }
        sm.cscale = sigma * a.score_scale;
        sm.cscale8 = 8.f * sm.cscale;
        sm.m = kMaxFloor;
        sm.l = 0.f;
        sm.alpha = 1.f;
    }

    // ---- lane constants ------------------------------------------------------
    Lanes L;
    {
        const uint32_t base = lds_address(lds);
        const int krow = lds_row<true>(key_of_row<true>(0, j));
        L.k_addr = base + krow * ROW + (((2 * h) ^ chunk_swizzle<true, CHUNKS>(krow)) << 4);
        // A operand lane (d row 16*(grp&1)+gl, k-group grp>>1): key 32*(grp>>1) + (gl>>1)
        const int vrow = lds_row<true>(32 * (grp >> 1) + (gl >> 1));
        L.v_addr = base + S::RING + vrow * ROW + (((grp & 1) ^ chunk_swizzle_v<true, CHUNKS>(vrow)) << 4) +
                   8 * (gl & 1);
        // DMA block `wave` lands at LDS byte wave * 1024 + 16 * lane.
        const int byte = wave * 1024 + lane * 16;
        const int drow = byte / ROW;
        const int pos = (byte % ROW) / 16;
        const int key = lds_row<true>(drow);
        L.dma_k = key * ROW + (pos ^ chunk_swizzle<true, CHUNKS>(drow)) * 16;
        L.dma_v = key * ROW + (pos ^ chunk_swizzle_v<true, CHUNKS>(drow)) * 16;
    }

    v16f o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = v16f{};
    v16f s[2];
    v8i pbuf[2] = {v8i{}, v8i{}};

    // ---- pipeline --------------------------------------------------------------
    const TileCursor first = next_tile(a, head, TileCursor{entry_begin - 1, 0, 0, 0});
    if (is_real(a, first)) {
        // V stages 2 and 3 stand for tiles -2 and -1: zeros.
        for (int idx = tid; idx < 2 * S::TILE / 16; idx += kThreads)
            *(v4i*)(lds + S::RING + 2 * S::TILE + 16 * idx) = v4i{0, 0, 0, 0};
        __syncthreads();
        const TileCursor before{-1, 0, 0, 0};
        Cursors cs;
        cs.cm1 = before;
        cs.c0 = first;
        cs.c1 = next_tile(a, head, first);
        cs.c2 = is_real(a, cs.c1) ? next_tile(a, head, cs.c1) : cs.c1;
        // K(0), then V(0) and K(1) as if requested at the top of iteration -1.
        load_k<S>(a, cs.c0, lds, 0, wave * 1024, L.dma_k);
        load_v<S>(a, cs.c0, lds, 0, wave * 1024, L.dma_v, true);
        if (is_real(a, cs.c1)) load_k<S>(a, cs.c1, lds, 1, wave * 1024, L.dma_k);
        if (wave < kWaves / 2)
            walk<D, false, FAST>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head);
        else
            walk<D, true, FAST>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head);
    }

    // ---- epilogue: O = O^T / l, bf16; log-sum-exp ---------------------------
    const float scale = sm.l > 0.f ? a.v_scale / sm.l : 0.f;
    // sum_k exp(score_k) = l * 2^(m - 6), less the average overestimate of
    // the linear-mantissa exp2
    const float lse =
        sm.l > 0.f ? __logf(sm.l) + (sm.m - kPBiasLog2) * kLn2 - (FAST ? kFastLseBias : 0.f) : -INFINITY;
    if constexpr (SPLIT) {
        if (row_ok) {
            const int64_t prow = (int64_t)split * a.rows_per_head * a.num_kv_heads + row_off / (D * 2);
            float* const po = a.part_o + prow * D;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int d = 32 * dt + 8 * r4 + 4 * h;
                    *(v4f*)(po + d) = v4f{o[dt][4 * r4 + 0] * scale, o[dt][4 * r4 + 1] * scale,
                                          o[dt][4 * r4 + 2] * scale, o[dt][4 * r4 + 3] * scale};
                }
            if (h == 0) a.part_lse[prow] = lse;
        }
        return;
    }
    if (LSE && row_ok && h == 0) a.lse[row_off / (D * 2)] = lse;
    if (row_ok) {
        uint8_t* const orow = a.out + row_off;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int d = 32 * dt + 8 * r4 + 4 * h;
                const __bf16 v0 = (__bf16)(o[dt][4 * r4 + 0] * scale);
                const __bf16 v1 = (__bf16)(o[dt][4 * r4 + 1] * scale);
                const __bf16 v2 = (__bf16)(o[dt][4 * r4 + 2] * scale);
                const __bf16 v3 = (__bf16)(o[dt][4 * r4 + 3] * scale);
                const uint32_t w0 = (uint32_t)__builtin_bit_cast(uint16_t, v0) |
                                    ((uint32_t)__builtin_bit_cast(uint16_t, v1) << 16);
                const uint32_t w1 = (uint32_t)__builtin_bit_cast(uint16_t, v2) |
                                    ((uint32_t)__builtin_bit_cast(uint16_t, v3) << 16);
                *(v2i*)(orow + 2 * d) = v2i{(int)w0, (int)w1};
            }
    }
}

}  // namespace ovl

// Merge of split partial outputs by log-sum-exp: one thread per (row, 8
// consecutive d).  out = sum_s w_s O_s / sum_s w_s with w_s = e^(lse_s - max),
// bf16; lse (optional) = max + ln(sum_s w_s).  HBM bound: 4 * D + 4 bytes read
// per row and split, 2 * D written.
__global__ void __launch_bounds__(256) merge_splits_kernel(const float* part_o, const float* part_lse, int splits,
                                                           int64_t rows, int d_vec8, uint8_t* out, float* lse_out) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * d_vec8) return;
    const int64_t row = idx / d_vec8;
    const int d0 = (int)(idx - row * d_vec8) * 8;
    const int D = d_vec8 * 8;
    float mx = -INFINITY;
    for (int sp = 0; sp < splits; ++sp) mx = fmaxf(mx, part_lse[sp * rows + row]);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float wsum = 0.f;
    for (int sp = 0; sp < splits; ++sp) {
        const float l = part_lse[sp * rows + row];
        if (l == -INFINITY) continue;
        const float w = __expf(l - mx);
        wsum += w;
        const float* const src = part_o + (sp * rows + row) * D + d0;
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

// ============================================================================
// C ABI
// ============================================================================

// ============================================================================
// KV-cache producer: per-tensor e4m3 quantisation of K/V and the page write
// in pack_local_kv's format (kernel.py:17-29), i.e. what the reference does
// on the host with shard_history (layout.py:54-98), the float8 cast
// (run_poc.py:96-103) and pack_local_kv, done on the GPU for a range of
// global history positions (a whole history, or tokens appended to it).
// Both kernels are HBM bound: 2 bytes read and 1 (e4m3) or 2 (bf16) bytes
// written per element.
// ============================================================================
namespace pcpa {
namespace cache {

constexpr int kThreads = 256;

// floor(n / d) for 0 <= n < 2^31 by one 64-bit multiply: M = ceil(2^(32+s)/d)
// with 2^s >= d gives the exact quotient for every n < 2^32.
struct FastDiv {
    uint64_t m;
    uint32_t shift;
    uint32_t d;
};
inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t s = 0;
    while ((1ull << s) < d) ++s;
    const unsigned __int128 num = (unsigned __int128)1 << (32 + s);
    return FastDiv{(uint64_t)((num + d - 1) / d), 32 + s, d};
}
__device__ __forceinline__ uint32_t div(uint32_t n, const FastDiv& f) {
    return (uint32_t)(((unsigned __int128)n * f.m) >> f.shift);
}

struct WriteArgs {
    const uint8_t* k;   // [Hkv, n, D] bf16
    const uint8_t* v;
    const int32_t* block_table;
    int32_t* page_valid_len;  // optional
    uint8_t* pages;
    int64_t page_stride;      // bytes of one page
    int64_t head_stride;      // bytes of one head's K (or V) block in a page
    int64_t v_offset;         // bytes from a page's K to its V
    FastDiv chunks_per_row;   // D / 8
    FastDiv interleave;
    FastDiv pcp;
    FastDiv block;            // block_size
    uint32_t log2_cpr, log2_il, log2_pcp, log2_block;  // when POW2
    uint32_t num_tokens;
    uint32_t first_pos;
    int32_t max_local_blocks;
    int32_t num_pages;
    int32_t head_dim;
    float k_scale, v_scale;
};

// e4m3 code of x (round to nearest even; magnitudes above 464 and infinities
// become the NaN code 0x7f with x's sign, like torch's float8_e4m3fn cast;
// v_cvt_pk_fp8_f32 agrees except that it writes 0xff for every NaN input).
__device__ __forceinline__ uint32_t e4m3_codes4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    uint32_t u = (uint32_t)w;
    const float x[4] = {a, b, c, d};
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (__builtin_isnan(x[i])) {
            const uint32_t code = (__float_as_uint(x[i]) >> 31) ? 0xffu : 0x7fu;
            u = (u & ~(0xffu << (8 * i))) | (code << (8 * i));
        }
    return u;
}

// One thread per (token, 8-element chunk) of head blockIdx.y: the token's
// page row comes from the striped layout (owner rank, local position) and
// the block table.  POW2: pcp, interleave, block size and D / 8 are powers
// of two (every configuration in use), so the maps are shifts and masks.
// Tokens whose table entry is outside [0, num_pages) are skipped, as the
// attention kernel skips such pages.
template <bool FP8, bool POW2>
__global__ void __launch_bounds__(kThreads) kv_write_kernel(WriteArgs a, uint32_t row_chunks) {
    const uint32_t gid = blockIdx.x * kThreads + threadIdx.x;
    if (gid >= row_chunks) return;
    const uint32_t head = blockIdx.y;
    uint32_t token, chunk, owner, local, blk, slot;
    const uint32_t p0 = a.first_pos;
    if constexpr (POW2) {
        token = gid >> a.log2_cpr;
        chunk = gid & ((1u << a.log2_cpr) - 1);
        const uint32_t p = p0 + token;
        const uint32_t c = p >> a.log2_il;
        owner = c & ((1u << a.log2_pcp) - 1);
        local = ((c >> a.log2_pcp) << a.log2_il) | (p & ((1u << a.log2_il) - 1));
        blk = local >> a.log2_block;
        slot = local & ((1u << a.log2_block) - 1);
    } else {
        token = div(gid, a.chunks_per_row);
        chunk = gid - token * a.chunks_per_row.d;
        const uint32_t p = p0 + token;
        const uint32_t c = div(p, a.interleave);
        const uint32_t rounds = div(c, a.pcp);
        owner = c - rounds * a.pcp.d;
        local = rounds * a.interleave.d + (p - c * a.interleave.d);
        blk = div(local, a.block);
        slot = local - blk * a.block.d;
    }
    const uint32_t row = head * a.num_tokens + token;
    if (blk >= (uint32_t)a.max_local_blocks) return;  // excluded by the host's capacity check
    const int32_t entry = (int32_t)(owner * a.max_local_blocks + blk);
    const int32_t page = a.block_table[entry];
    if ((uint32_t)page >= (uint32_t)a.num_pages) return;
    if (a.page_valid_len && head == 0 && chunk == 0) atomicMax(a.page_valid_len + entry, (int32_t)slot + 1);

    const int64_t src = ((int64_t)row * a.head_dim + chunk * 8) * 2;  // [Hkv, n, D] bf16
    const v4i kin = *(const v4i*)(a.k + src);
    const v4i vin = *(const v4i*)(a.v + src);
    const int64_t es = FP8 ? 1 : 2;
    uint8_t* const dst = a.pages + (int64_t)page * a.page_stride + head * a.head_stride +
                         ((int64_t)slot * a.head_dim + chunk * 8) * es;
    if constexpr (FP8) {
        float kf[8], vf[8];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            // x / scale with IEEE division, as torch computes (x / scale).to(float8)
            kf[2 * w] = bf16_bits_to_f32((uint32_t)kin[w] & 0xffffu) / a.k_scale;
            kf[2 * w + 1] = bf16_bits_to_f32((uint32_t)kin[w] >> 16) / a.k_scale;
            vf[2 * w] = bf16_bits_to_f32((uint32_t)vin[w] & 0xffffu) / a.v_scale;
            vf[2 * w + 1] = bf16_bits_to_f32((uint32_t)vin[w] >> 16) / a.v_scale;
        }
        *(v2i*)dst = v2i{(int)e4m3_codes4(kf[0], kf[1], kf[2], kf[3]), (int)e4m3_codes4(kf[4], kf[5], kf[6], kf[7])};
        *(v2i*)(dst + a.v_offset) =
            v2i{(int)e4m3_codes4(vf[0], vf[1], vf[2], vf[3]), (int)e4m3_codes4(vf[4], vf[5], vf[6], vf[7])};
    } else {
        *(v4i*)dst = kin;
        *(v4i*)(dst + a.v_offset) = vin;
    }
}

// max |x| over n bf16 values into *out (as the bits of a non-negative float,
// ordered like unsigned integers); *out is cleared first by init_kernel.
__global__ void absmax_init_kernel(uint32_t* out) { *out = 0u; }

// Workgroup b reduces the contiguous span [b * span, (b + 1) * span) with
// four 16-byte loads in flight per thread, then one atomic per workgroup.
__global__ void __launch_bounds__(kThreads) absmax_kernel(const uint16_t* x, int64_t n, int64_t span,
                                                          uint32_t* out) {
    constexpr int kVec = 8, kUnroll = 4, kStep = kThreads * kVec;
    __shared__ float partial[kThreads / 64];
    const int64_t begin = (int64_t)blockIdx.x * span;
    const int64_t end = begin + span < n ? begin + span : n;
    float m[kUnroll] = {0.f, 0.f, 0.f, 0.f};
    int64_t i = begin + threadIdx.x * kVec;
    for (; i + (kUnroll - 1) * kStep + kVec <= end; i += kUnroll * kStep) {
        v4i raw[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) raw[u] = *(const v4i*)(x + i + u * kStep);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                m[u] = fmaxf(m[u], fabsf(bf16_bits_to_f32((uint32_t)raw[u][w] & 0xffffu)));
                m[u] = fmaxf(m[u], fabsf(bf16_bits_to_f32((uint32_t)raw[u][w] >> 16)));
            }
    }
    for (; i < end; i += kStep) {
        if (i + kVec <= end) {
            const v4i raw = *(const v4i*)(x + i);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                m[0] = fmaxf(m[0], fabsf(bf16_bits_to_f32((uint32_t)raw[w] & 0xffffu)));
                m[0] = fmaxf(m[0], fabsf(bf16_bits_to_f32((uint32_t)raw[w] >> 16)));
            }
        } else {
            for (int64_t e = i; e < end; ++e) m[0] = fmaxf(m[0], fabsf(bf16_bits_to_f32(x[e])));
        }
    }
    float r = fmaxf(fmaxf(m[0], m[1]), fmaxf(m[2], m[3]));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) r = fmaxf(r, __shfl_xor(r, off));
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = r;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / 64; ++w) r = fmaxf(r, partial[w]);
        atomicMax(out, __float_as_uint(r));
    }
}

}  // namespace cache
}  // namespace pcpa

namespace pcpa {

// Launch arguments shared by every attention entry point (Q rows, output).
inline FwdArgs common_args(const pcpa_params* p, const void* q, void* out) {
    FwdArgs a{};
    a.q = (const uint8_t*)q;
    a.out = (uint8_t*)out;
    a.group = p->num_q_heads / p->num_kv_heads;
    a.group_rows = a.group * p->local_q_len;
    a.rows_per_head = p->pcp_size * a.group_rows;
    a.row_tiles = (a.rows_per_head + kRowsPerGroup - 1) / kRowsPerGroup;
    a.local_q = p->local_q_len;
    a.num_q_heads = p->num_q_heads;
    a.num_kv_heads = p->num_kv_heads;
    return a;
}

}  // namespace pcpa

extern "C" {

int32_t pcpa_abi_version(void) { return PCPA_ABI_VERSION; }

const char* pcpa_status_string(int32_t status) {
    switch (status) {
        case PCPA_OK: return "ok";
        case PCPA_ERR_NULL_POINTER: return "a required pointer is NULL";
        case PCPA_ERR_ABI_VERSION: return "params.abi_version does not match the library";
        case PCPA_ERR_BAD_SHAPE: return "non-positive or inconsistent sizes";
        case PCPA_ERR_BAD_DTYPE: return "unsupported dtype code";
        case PCPA_ERR_UNSUPPORTED: return "shape not supported by the gfx950 kernel";
        case PCPA_ERR_MISALIGNED: return "tensor pointer is not 16-byte aligned";
        case PCPA_ERR_LAUNCH: return "HIP kernel launch failed";
        case PCPA_ERR_TOO_LARGE: return "sizes overflow the kernel's index arithmetic";
        case PCPA_ERR_BAD_SCALE: return "scales must be finite and positive";
        default: return "unknown status";
    }
}

int32_t pcpa_check_params(const pcpa_params* p) {
    if (p == nullptr) return PCPA_ERR_NULL_POINTER;
    if (p->abi_version != PCPA_ABI_VERSION) return PCPA_ERR_ABI_VERSION;
    if (p->pcp_size <= 0 || p->num_q_heads <= 0 || p->num_kv_heads <= 0 || p->head_dim <= 0 ||
        p->local_q_len <= 0 || p->block_size <= 0 || p->max_local_blocks <= 0 || p->num_pages <= 0)
        return PCPA_ERR_BAD_SHAPE;
    if (p->num_q_heads % p->num_kv_heads) return PCPA_ERR_BAD_SHAPE;
    if (p->flags & ~(uint32_t)(PCPA_FLAG_BF16_MFMA | PCPA_FLAG_EXACT_EXP2)) return PCPA_ERR_BAD_SHAPE;
    if (p->q_dtype != PCPA_DTYPE_BF16 || p->out_dtype != PCPA_DTYPE_BF16) return PCPA_ERR_BAD_DTYPE;
    if (p->kv_dtype != PCPA_DTYPE_BF16 && p->kv_dtype != PCPA_DTYPE_FP8_E4M3FN) return PCPA_ERR_BAD_DTYPE;
    if (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256) return PCPA_ERR_UNSUPPORTED;
    if (p->block_size % pcpa::kKeyTile) return PCPA_ERR_UNSUPPORTED;
    if (!(isfinite(p->softmax_scale) && isfinite(p->k_scale) && isfinite(p->v_scale)) ||
        p->softmax_scale <= 0.f || p->k_scale <= 0.f || p->v_scale <= 0.f)
        return PCPA_ERR_BAD_SCALE;
    const int64_t group = p->num_q_heads / p->num_kv_heads;
    const int64_t rows = (int64_t)p->pcp_size * group * p->local_q_len;
    const int64_t q_elems = (int64_t)p->pcp_size * p->num_q_heads * p->local_q_len * p->head_dim;
    const int64_t entries = (int64_t)p->pcp_size * p->max_local_blocks;
    const int64_t rank_heads = (int64_t)p->pcp_size * p->num_q_heads;
    if (rows > INT32_MAX || entries > INT32_MAX || rank_heads > INT32_MAX || q_elems > (INT64_MAX / 4))
        return PCPA_ERR_TOO_LARGE;
    return PCPA_OK;
}

int32_t pcpa_history_attention_lse(const pcpa_params* p, const void* q, const void* kv_pages,
                                   const int32_t* block_table, const int32_t* page_valid_len, void* out,
                                   float* lse, void* stream) {
    const int32_t st = pcpa_check_params(p);
    if (st != PCPA_OK) return st;
    if (!q || !kv_pages || !block_table || !page_valid_len || !out) return PCPA_ERR_NULL_POINTER;
    if (((uintptr_t)q | (uintptr_t)kv_pages | (uintptr_t)out) & 15u) return PCPA_ERR_MISALIGNED;
    if (((uintptr_t)block_table | (uintptr_t)page_valid_len | (uintptr_t)lse) & 3u) return PCPA_ERR_MISALIGNED;

    const bool store8 = p->kv_dtype == PCPA_DTYPE_FP8_E4M3FN;
    const bool fp8 = store8 && !(p->flags & PCPA_FLAG_BF16_MFMA);
    const int64_t es = store8 ? 1 : 2;
    pcpa::FwdArgs a = pcpa::common_args(p, q, out);
    a.kv = (const uint8_t*)kv_pages;
    a.block_table = block_table;
    a.page_valid_len = page_valid_len;
    a.head_stride = (int64_t)p->block_size * p->head_dim * es;
    a.page_stride = 2 * (int64_t)p->num_kv_heads * a.head_stride;
    a.num_entries = p->pcp_size * p->max_local_blocks;
    a.num_pages = p->num_pages;
    a.block_size = p->block_size;
    a.score_scale = p->softmax_scale * p->k_scale * pcpa::kLog2e;
    a.v_scale = p->v_scale;
    a.lse = lse;

    void* args[] = {&a};
    const void* fn = nullptr;
    if (fp8 && p->head_dim == 256) {
        a.row_tiles = (a.rows_per_head + pcpa::ovl::kRowsPerGroup - 1) / pcpa::ovl::kRowsPerGroup;
        const int oitems = a.row_tiles * p->num_kv_heads;
        const bool exact = p->flags & PCPA_FLAG_EXACT_EXP2;
        if (lse)
            fn = exact ? (const void*)pcpa::ovl::history_fwd_overlap<256, false, true>
                       : (const void*)pcpa::ovl::history_fwd_overlap<256, true, true>;
        else
            fn = exact ? (const void*)pcpa::ovl::history_fwd_overlap<256, false, false>
                       : (const void*)pcpa::ovl::history_fwd_overlap<256, true, false>;
        const hipError_t oerr = hipLaunchKernel(fn, dim3(8 * ((oitems + 7) / 8)), dim3(pcpa::ovl::kThreads), args, 0,
                                                (hipStream_t)stream);
        return oerr == hipSuccess ? PCPA_OK : PCPA_ERR_LAUNCH;
    }
    switch (p->head_dim * 4 + (store8 ? 2 : 0) + (fp8 ? 1 : 0)) {
        case 64 * 4 + 3: fn = (const void*)pcpa::history_fwd_kernel<64, true, true>; break;
        case 128 * 4 + 3: fn = (const void*)pcpa::history_fwd_kernel<128, true, true>; break;
        case 256 * 4 + 3: fn = (const void*)pcpa::history_fwd_kernel<256, true, true>; break;
        case 64 * 4 + 2: fn = (const void*)pcpa::history_fwd_kernel<64, true, false>; break;
        case 128 * 4 + 2: fn = (const void*)pcpa::history_fwd_kernel<128, true, false>; break;
        case 256 * 4 + 2: fn = (const void*)pcpa::history_fwd_kernel<256, true, false>; break;
        case 64 * 4: fn = (const void*)pcpa::history_fwd_kernel<64, false, false>; break;
        case 128 * 4: fn = (const void*)pcpa::history_fwd_kernel<128, false, false>; break;
        case 256 * 4: fn = (const void*)pcpa::history_fwd_kernel<256, false, false>; break;
        default: return PCPA_ERR_UNSUPPORTED;
    }
    const int items = a.row_tiles * p->num_kv_heads;
    const hipError_t err =
        hipLaunchKernel(fn, dim3(8 * ((items + 7) / 8)), dim3(pcpa::kThreads), args, 0, (hipStream_t)stream);
    return err == hipSuccess ? PCPA_OK : PCPA_ERR_LAUNCH;
}

int64_t pcpa_split_workspace_bytes(const pcpa_params* p, int32_t splits) {
    const int32_t st = pcpa_check_params(p);
    if (st != PCPA_OK) return st;
    if (splits < 1 || splits > PCPA_MAX_SPLITS) return PCPA_ERR_BAD_SHAPE;
    const int64_t rows = (int64_t)p->pcp_size * p->num_q_heads * p->local_q_len;
    return (int64_t)splits * rows * ((int64_t)p->head_dim + 1) * 4;
}

int32_t pcpa_history_attention_split(const pcpa_params* p, int32_t splits, const void* q, const void* kv_pages,
                                     const int32_t* block_table, const int32_t* page_valid_len, void* out,
                                     float* lse, void* workspace, int64_t workspace_bytes, void* stream) {
    const int64_t need = pcpa_split_workspace_bytes(p, splits);
    if (need < 0) return (int32_t)need;
    if (splits == 1) return pcpa_history_attention_lse(p, q, kv_pages, block_table, page_valid_len, out, lse, stream);
    if (!q || !kv_pages || !block_table || !page_valid_len || !out || !workspace) return PCPA_ERR_NULL_POINTER;
    if (((uintptr_t)q | (uintptr_t)kv_pages | (uintptr_t)out | (uintptr_t)workspace) & 15u) return PCPA_ERR_MISALIGNED;
    if (((uintptr_t)block_table | (uintptr_t)page_valid_len | (uintptr_t)lse) & 3u) return PCPA_ERR_MISALIGNED;
    if (workspace_bytes < need) return PCPA_ERR_BAD_SHAPE;
    const bool fp8 = p->kv_dtype == PCPA_DTYPE_FP8_E4M3FN && !(p->flags & PCPA_FLAG_BF16_MFMA);
    if (!fp8 || p->head_dim != 256) return PCPA_ERR_UNSUPPORTED;

    pcpa::FwdArgs a = pcpa::common_args(p, q, out);
    a.kv = (const uint8_t*)kv_pages;
    a.block_table = block_table;
    a.page_valid_len = page_valid_len;
    a.head_stride = (int64_t)p->block_size * p->head_dim;
    a.page_stride = 2 * (int64_t)p->num_kv_heads * a.head_stride;
    a.num_entries = p->pcp_size * p->max_local_blocks;
    a.num_pages = p->num_pages;
    a.block_size = p->block_size;
    a.score_scale = p->softmax_scale * p->k_scale * pcpa::kLog2e;
    a.v_scale = p->v_scale;
    a.row_tiles = (a.rows_per_head + pcpa::ovl::kRowsPerGroup - 1) / pcpa::ovl::kRowsPerGroup;
    a.splits = splits;
    const int64_t rows = (int64_t)p->pcp_size * p->num_q_heads * p->local_q_len;
    a.part_o = (float*)workspace;
    a.part_lse = a.part_o + (int64_t)splits * rows * p->head_dim;

    void* args[] = {&a};
    const void* fn = (p->flags & PCPA_FLAG_EXACT_EXP2) ? (const void*)pcpa::ovl::history_fwd_overlap<256, false, false, true>
                                                       : (const void*)pcpa::ovl::history_fwd_overlap<256, true, false, true>;
    const int items = a.row_tiles * p->num_kv_heads * splits;
    hipError_t err = hipLaunchKernel(fn, dim3(8 * ((items + 7) / 8)), dim3(pcpa::ovl::kThreads), args, 0,
                                     (hipStream_t)stream);
    if (err != hipSuccess) return PCPA_ERR_LAUNCH;
    const int d_vec8 = p->head_dim / 8;
    const int64_t threads = rows * d_vec8;
    hipLaunchKernelGGL(pcpa::merge_splits_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const float*)a.part_o, (const float*)a.part_lse, splits, rows, d_vec8,
                       (uint8_t*)out, lse);
    return hipGetLastError() == hipSuccess ? PCPA_OK : PCPA_ERR_LAUNCH;
}

int32_t pcpa_history_attention(const pcpa_params* p, const void* q, const void* kv_pages,
                               const int32_t* block_table, const int32_t* page_valid_len, void* out,
                               void* stream) {
    return pcpa_history_attention_lse(p, q, kv_pages, block_table, page_valid_len, out, nullptr, stream);
}

int32_t pcpa_current_attention(const pcpa_params* p, int32_t interleave, const void* q, const void* kv_current,
                               const void* hist_out, const float* hist_lse, void* out, float* lse,
                               void* stream) {
    const int32_t st = pcpa_check_params(p);
    if (st != PCPA_OK) return st;
    if (!q || !kv_current || !out) return PCPA_ERR_NULL_POINTER;
    if ((hist_out == nullptr) != (hist_lse == nullptr)) return PCPA_ERR_NULL_POINTER;
    if (p->kv_dtype != PCPA_DTYPE_BF16) return PCPA_ERR_BAD_DTYPE;
    if (interleave <= 0 || p->local_q_len % interleave) return PCPA_ERR_BAD_SHAPE;
    const int64_t current = (int64_t)p->pcp_size * p->local_q_len;
    if (current % pcpa::kKeyTile) return PCPA_ERR_UNSUPPORTED;
    if (((uintptr_t)q | (uintptr_t)kv_current | (uintptr_t)out | (uintptr_t)hist_out) & 15u)
        return PCPA_ERR_MISALIGNED;
    if (((uintptr_t)hist_lse | (uintptr_t)lse) & 3u) return PCPA_ERR_MISALIGNED;

    pcpa::FwdArgs a = pcpa::common_args(p, q, out);
    a.kv = (const uint8_t*)kv_current;
    a.head_stride = current * p->head_dim * 2;
    a.page_stride = 2 * (int64_t)p->num_kv_heads * a.head_stride;
    a.num_entries = 1;
    a.num_pages = 1;
    a.block_size = (int32_t)current;
    a.score_scale = p->softmax_scale * pcpa::kLog2e;  // BF16 current K/V: no dequantisation scale
    a.v_scale = 1.f;
    a.lse = lse;
    a.merge_o = (const uint8_t*)hist_out;
    a.merge_lse = hist_lse;
    a.interleave = interleave;
    a.pcp = p->pcp_size;

    void* args[] = {&a};
    const void* fn = nullptr;
    switch (p->head_dim) {
        case 64: fn = (const void*)pcpa::history_fwd_kernel<64, false, false, true>; break;
        case 128: fn = (const void*)pcpa::history_fwd_kernel<128, false, false, true>; break;
        case 256: fn = (const void*)pcpa::history_fwd_kernel<256, false, false, true>; break;
        default: return PCPA_ERR_UNSUPPORTED;
    }
    const int items = a.row_tiles * p->num_kv_heads;
    const hipError_t err =
        hipLaunchKernel(fn, dim3(8 * ((items + 7) / 8)), dim3(pcpa::kThreads), args, 0, (hipStream_t)stream);
    return err == hipSuccess ? PCPA_OK : PCPA_ERR_LAUNCH;
}

int32_t pcpa_absmax_bf16(const void* x, int64_t n, float* amax, void* stream) {
    if (!x || !amax) return PCPA_ERR_NULL_POINTER;
    if (n < 0) return PCPA_ERR_BAD_SHAPE;
    if (((uintptr_t)x & 15u) || ((uintptr_t)amax & 3u)) return PCPA_ERR_MISALIGNED;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(pcpa::cache::absmax_init_kernel, dim3(1), dim3(1), 0, st, (uint32_t*)amax);
    if (hipGetLastError() != hipSuccess) return PCPA_ERR_LAUNCH;
    if (n == 0) return PCPA_OK;
    // spans of whole 8-element groups (the span start stays 16-byte aligned),
    // at least 32 KB each, at most 2048 workgroups
    constexpr int64_t kMinSpan = 16384;
    int64_t span = (n + 2047) / 2048;
    span = span < kMinSpan ? kMinSpan : (span + 7) / 8 * 8;
    const unsigned blocks = (unsigned)((n + span - 1) / span);
    hipLaunchKernelGGL(pcpa::cache::absmax_kernel, dim3(blocks), dim3(pcpa::cache::kThreads), 0, st,
                       (const uint16_t*)x, n, span, (uint32_t*)amax);
    return hipGetLastError() == hipSuccess ? PCPA_OK : PCPA_ERR_LAUNCH;
}

int32_t pcpa_kv_cache_write(const pcpa_params* p, int32_t interleave, int64_t first_pos, int32_t num_tokens,
                            const void* k, const void* v, const int32_t* block_table, void* kv_pages,
                            int32_t* page_valid_len, void* stream) {
    const int32_t st = pcpa_check_params(p);
    if (st != PCPA_OK) return st;
    if (!k || !v || !block_table || !kv_pages) return PCPA_ERR_NULL_POINTER;
    if (interleave <= 0 || first_pos < 0 || num_tokens < 0) return PCPA_ERR_BAD_SHAPE;
    if (((uintptr_t)k | (uintptr_t)v | (uintptr_t)kv_pages) & 15u) return PCPA_ERR_MISALIGNED;
    if (((uintptr_t)block_table | (uintptr_t)page_valid_len) & 3u) return PCPA_ERR_MISALIGNED;
    if (num_tokens == 0) return PCPA_OK;
    // Every position must have a cache block: local index < max_local_blocks *
    // block_size.  The local index grows with the position for each owner
    // rank, so the largest one is among the last pcp_size * interleave
    // positions of the range.
    const int64_t capacity = (int64_t)p->max_local_blocks * p->block_size;  // per rank
    const int64_t last = first_pos + num_tokens - 1;
    const int64_t round_len = (int64_t)p->pcp_size * interleave;
    for (int64_t pos = last; pos >= first_pos && pos > last - round_len; --pos) {
        const int64_t chunk = pos / interleave;
        if ((chunk / p->pcp_size) * interleave + pos % interleave >= capacity) return PCPA_ERR_BAD_SHAPE;
    }
    const int64_t chunks = (int64_t)p->num_kv_heads * num_tokens * (p->head_dim / 8);
    if (last >= INT32_MAX || chunks > INT32_MAX || (int64_t)p->pcp_size * capacity > INT32_MAX)
        return PCPA_ERR_TOO_LARGE;

    const bool fp8 = p->kv_dtype == PCPA_DTYPE_FP8_E4M3FN;
    const int64_t es = fp8 ? 1 : 2;
    pcpa::cache::WriteArgs a;
    a.k = (const uint8_t*)k;
    a.v = (const uint8_t*)v;
    a.block_table = block_table;
    a.page_valid_len = page_valid_len;
    a.pages = (uint8_t*)kv_pages;
    a.head_stride = (int64_t)p->block_size * p->head_dim * es;
    a.v_offset = (int64_t)p->num_kv_heads * a.head_stride;
    a.page_stride = 2 * a.v_offset;
    a.chunks_per_row = pcpa::cache::make_fastdiv((uint32_t)(p->head_dim / 8));
    a.interleave = pcpa::cache::make_fastdiv((uint32_t)interleave);
    a.pcp = pcpa::cache::make_fastdiv((uint32_t)p->pcp_size);
    a.block = pcpa::cache::make_fastdiv((uint32_t)p->block_size);
    auto log2_of = [](uint32_t x) -> int { return (x & (x - 1)) ? -1 : __builtin_ctz(x); };
    const int l_cpr = log2_of((uint32_t)(p->head_dim / 8)), l_il = log2_of((uint32_t)interleave);
    const int l_pcp = log2_of((uint32_t)p->pcp_size), l_blk = log2_of((uint32_t)p->block_size);
    const bool pow2 = l_cpr >= 0 && l_il >= 0 && l_pcp >= 0 && l_blk >= 0;
    a.log2_cpr = pow2 ? l_cpr : 0;
    a.log2_il = pow2 ? l_il : 0;
    a.log2_pcp = pow2 ? l_pcp : 0;
    a.log2_block = pow2 ? l_blk : 0;
    a.num_tokens = (uint32_t)num_tokens;
    a.first_pos = (uint32_t)first_pos;
    a.max_local_blocks = p->max_local_blocks;
    a.num_pages = p->num_pages;
    a.head_dim = p->head_dim;
    a.k_scale = p->k_scale;
    a.v_scale = p->v_scale;
    const uint32_t row_chunks = (uint32_t)num_tokens * (uint32_t)(p->head_dim / 8);
    const dim3 grid((row_chunks + pcpa::cache::kThreads - 1) / pcpa::cache::kThreads, p->num_kv_heads);
    const dim3 block(pcpa::cache::kThreads);
    const hipStream_t hs = (hipStream_t)stream;
    if (fp8 && pow2)
        hipLaunchKernelGGL((pcpa::cache::kv_write_kernel<true, true>), grid, block, 0, hs, a, row_chunks);
    else if (fp8)
        hipLaunchKernelGGL((pcpa::cache::kv_write_kernel<true, false>), grid, block, 0, hs, a, row_chunks);
    else if (pow2)
        hipLaunchKernelGGL((pcpa::cache::kv_write_kernel<false, true>), grid, block, 0, hs, a, row_chunks);
    else
        hipLaunchKernelGGL((pcpa::cache::kv_write_kernel<false, false>), grid, block, 0, hs, a, row_chunks);
    return hipGetLastError() == hipSuccess ? PCPA_OK : PCPA_ERR_LAUNCH;
}

}  // extern "C"

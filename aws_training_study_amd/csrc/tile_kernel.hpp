// history_fwd_kernel: the tile kernel for every head dim and precision, and
// (CAUSAL) the current-token step.
#pragma once

#include "common.hpp"

namespace pcpa {

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
    // Double-buffered (prefetching) when both buffers fit in 128 KB of LDS
    // (gfx950 has 160 KB per CU); the widening path stages synchronously
    // through registers.
    static constexpr int NBUF = (!WIDEN && 4 * TILE <= 131072) ? 2 : 1;
    static constexpr int QK = FP8 ? D / 64 : D / 16;   // k-steps of the score MFMA
    static constexpr int DT = D / 32;                  // 32-row d tiles of O^T
    // BF16 MFMAs at head_dim 256 run eight waves in key-split pairs: the two
    // waves of a SIMD take the same 32 rows and one half of every tile's
    // keys each, with an online softmax and O^T of their own, merged
    // through LDS at the end.  (One wave holding all 64 keys of a tile
    // needs 448 registers, i.e. one wave per SIMD and nothing to overlap
    // the softmax with.)
    static constexpr bool PAIR = D == 256 && !FP8;
    static constexpr int WAVES = PAIR ? 2 * kWaves : kWaves;
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int NT = PAIR ? 1 : 2;            // 32-key score tiles per wave and tile
    static constexpr int DMA_PER_WAVE = CHUNKS / WAVES;  // 1 KB DMA blocks per wave per operand
    // LDS: the tile buffers, which a PAIR workgroup reuses for the partners'
    // O^T (32 KB per pair) after the walk.
    static constexpr int LDS_BYTES = (PAIR && NBUF * 2 * TILE < 4 * 32768) ? 4 * 32768 : NBUF * 2 * TILE;
    // Wave w loads DMA blocks WAVES i + w.  Block i's lane chunk sits
    // dma_key_delta(i) key rows after block 0's, with the same chunk swizzle,
    // except for 512-byte rows (bf16 D=256) loaded by four waves, whose
    // blocks are 8 rows apart and whose swizzle (a function of the row mod
    // 16) changes between blocks: those keep one offset per block
    // (DMA_SPLIT).  Eight waves put a wave's blocks 16 rows apart.
    static constexpr bool DMA_SPLIT = ROW == 512 && WAVES == kWaves;
    static constexpr int K_T1_ROWS = FP8 ? 16 : 32;    // LDS rows from score tile 0 to tile 1
    static constexpr int dma_key_delta(int i) {
        // keys between DMA block i's lane chunk and block 0's (rows are WAVES i 1024 / ROW apart)
        return FP8 ? (ROW == 256 ? 16 * (i & 1) + 8 * (i >> 1) : ROW == 128 ? 8 * i : 0) : i * WAVES * 1024 / ROW;
    }
    // Lazy rescale: the running max is only raised when a tile's max exceeds
    // it by more than this (log2 units); FP8 probabilities then stay below
    // 2^(kPBiasLog2 + 2.5) = 362 < 448.
    static constexpr float RESCALE_LOG2 = FP8 ? 2.5f : 8.0f;
};

// Threads per workgroup of the tile kernel for a head dim and MFMA precision.
__host__ __device__ constexpr int tile_threads(int d, bool fp8) {
    return (d == 256 && !fp8) ? TileShape<256, false, false>::THREADS : kThreads;
}

// Per-lane constants of the main loop (LDS offsets are within one buffer).
template <class S>
struct LaneMap {
    uint32_t k_addr;                      // score A operand of tile 0 (tile 1: + K_T1_ROWS rows)
    uint32_t v_addr[S::ES == 1 ? 1 : 2];  // PV A operand base(s)
    uint32_t dma_off[S::DMA_SPLIT ? S::DMA_PER_WAVE : 1];   // global byte offset of the lane's K DMA chunk
    uint32_t dma_off_v[S::DMA_SPLIT ? S::DMA_PER_WAVE : 1]; // same for the V tile (its own swizzle)
    int rsel;  // e4m3 MFMAs: the row-sum selector operand word (e4m3 1.0 bytes or 0)
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
        const int block = S::WAVES * i + wave;
        const uint32_t koff = L.dma_off[S::DMA_SPLIT ? i : 0];
        const uint32_t voff = L.dma_off_v[S::DMA_SPLIT ? i : 0];
        const int delta = S::DMA_SPLIT ? 0 : S::dma_key_delta(i) * S::GROW;
        dma_sbase<0>(kt + delta, koff, lds_address(lk + block * 1024));
        dma_sbase<0>(vt + delta, voff, lds_address(lk + S::TILE + block * 1024));
    }
}

// Synchronous staging through registers into buffer 0, widening e4m3 to
// bf16 when the MFMAs are bf16.  Rows at or beyond `valid` get zero V.
template <class S>
__device__ __forceinline__ void stage_tile_sync(const FwdArgs& a, const TileCursor& c, int valid, uint8_t* lds,
                                                int tid) {
    constexpr int LOADS = kKeyTile * S::GROW / (16 * S::THREADS);
    static_assert((kKeyTile * S::GROW) % (16 * S::THREADS) == 0, "tile must split into 16-byte chunks per thread");
    const uint8_t* const kpage = a.kv + c.k_off;
    const uint8_t* const vpage = kpage + (int64_t)a.num_kv_heads * a.head_stride;
    uint8_t* const lds_k = lds;
    uint8_t* const lds_v = lds + S::TILE;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int chunk_id = tid + S::THREADS * i;
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
            // (K and V rows have swizzles of their own)
            const int lo = row * S::ROW + (((2 * ch) ^ sw) << 4);
            const int hi = row * S::ROW + (((2 * ch + 1) ^ sw) << 4);
            const int lov = row * S::ROW + (((2 * ch) ^ swv) << 4);
            const int hiv = row * S::ROW + (((2 * ch + 1) ^ swv) << 4);
            *(v4i*)(lds_k + lo) = v4i{k0[0], k0[1], k1[0], k1[1]};
            *(v4i*)(lds_k + hi) = v4i{k2[0], k2[1], k3[0], k3[1]};
            *(v4i*)(lds_v + lov) = v4i{v0[0], v0[1], v1[0], v1[1]};
            *(v4i*)(lds_v + hiv) = v4i{v2[0], v2[1], v3[0], v3[1]};
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
    for (int idx = tid; idx < (kKeyTile - valid) * S::CHUNKS; idx += S::THREADS) {
        const int key = valid + idx / S::CHUNKS;
        *(v4i*)(lds_v + lds_row<S::ES == 1>(key) * S::ROW + (idx % S::CHUNKS) * 16) = v4i{0, 0, 0, 0};
    }
}

// Online-softmax state of one lane: running max (log2 domain, times the
// lane's score factor), the running sum (BF16 MFMAs: this lane half's share;
// e4m3 MFMAs: the whole row's), and the O^T accumulator tiles.
template <class S>
struct SoftmaxState {
    float m;
    float l;
    v16f o[S::DT];
};

template <class S>
using QOperand = typename std::conditional<S::ES == 1, v8i, v8bf>::type;

// One 64-key tile held in LDS buffer BUF (PAIR: this wave's 32 keys of it;
// its operand addresses in L include the half): S^T = K Q^T, masked online
// softmax, O^T += V^T P^T.  `valid`: the valid keys counted from the wave's
// first key.
// CAUSAL: `valid` differs per lane (the row's causal limit within the tile,
// possibly <= 0).
//
// rt_off: a byte offset added to both buffers' addresses at run time (PAIR
// walks alternate buffers with one loop body, BUF 0 and rt_off 0 or
// 2 * TILE; otherwise 0).
template <class S, int BUF, bool CAUSAL = false>
__device__ __forceinline__ void compute_tile(const uint8_t* lds, uint32_t rt_off, int valid,
                                             const QOperand<S> (&qop)[S::QK], float cscale, const LaneMap<S>& L, int h,
                                             SoftmaxState<S>& st) {
    constexpr bool FP8 = S::ES == 1;
    constexpr int ROW = S::ROW, QK = S::QK, DT = S::DT;
    constexpr int KBASE = BUF * 2 * S::TILE;
    constexpr int VBASE = KBASE + S::TILE;
    const uint8_t* const lk = lds + KBASE + rt_off;

    // ---- S^T = K . Q^T : two 32-key x 32-query tiles --------------------
    v16f s[2];
    if constexpr (FP8) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = v16f{};
#pragma unroll
            for (int c = 0; c < QK; ++c) {
                const uint8_t* const kt = lk + t * S::K_T1_ROWS * ROW;
                const v4i lo = *(const v4i*)(kt + (L.k_addr ^ ((4 * c) << 4)));
                const v4i hi = *(const v4i*)(kt + (L.k_addr ^ ((4 * c + 1) << 4)));
                const v8i aop = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                s[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(aop, qop[c], s[t], 0, 0, 0, 0, 0, 0);
            }
        }
    } else {
        // both score tiles advance together, their K operands read one
        // d step ahead of the MFMAs
        const uint8_t* const kt1 = lk + S::K_T1_ROWS * ROW;
        v4i kb[2][2];
        auto load = [&](v4i (&k)[2], int c) {
            k[0] = *(const v4i*)(lk + (L.k_addr ^ ((2 * c) << 4)));
            if constexpr (S::NT > 1) k[1] = *(const v4i*)(kt1 + (L.k_addr ^ ((2 * c) << 4)));
        };
        s[0] = v16f{};
        s[1] = v16f{};
        load(kb[0], 0);
#pragma unroll
        for (int c = 0; c < QK; ++c) {
            if (c + 1 < QK) load(kb[(c + 1) & 1], c + 1);
            // (the barriers keep the reads of step c + 1 ahead of step c's MFMAs)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < S::NT; ++t)
                s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, kb[c & 1][t]), qop[c], s[t], 0,
                                                               0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // Wave priority: the two waves a SIMD holds run the same loop out of
    // phase.  Four-wave workgroups (two per CU, a SIMD's waves from
    // different workgroups) finish sooner when the wave in its softmax
    // issues first (GQA-8 workload 2.018 vs 2.040 ms); key-split pairs
    // (the two waves of one pair on a SIMD) when the wave at its MFMAs does
    // (64-rank BF16 cache 16.43 vs 16.62 ms; interleaved runs on one box).
    __builtin_amdgcn_s_setprio(S::PAIR ? 0 : 1);
    // ---- mask, online softmax (lazy rescale) ----------------------------
    // (CAUSAL: only tiles that cross some row's limit, a wave-uniform test)
    constexpr int KEYS = 32 * S::NT;  // keys of the tile this wave scores
    if (CAUSAL ? __builtin_amdgcn_ballot_w64(valid < KEYS) != 0 : valid < KEYS) {
        // key_of_acc(t, r, h) >= valid, as its lane-independent part against
        // valid less its lane-half part
        const int lim = valid - key_of_acc<FP8>(0, 0, h);
        const float ninf = -INFINITY;
        static_for<0, 16 * S::NT>([&](auto kc) {
            constexpr int t = decltype(kc)::value >> 4, r = decltype(kc)::value & 15;
            constexpr int k = FP8 ? 16 * t + r : 32 * t + 16 * (r >> 3) + (r & 7);
            s[t][r] = mask_key_at_or_past<k>(s[t][r], lim, ninf);
        });
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < S::NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
    const float mxs = halves_max(mx) * cscale;
    const bool raise = mxs > st.m + S::RESCALE_LOG2;
    if (__builtin_amdgcn_ballot_w64(raise) != 0) {
        // only the rows past the margin move (alpha = 1 exactly elsewhere), so
        // a row's result does not depend on the rows that share its wave
        const float m_new = raise ? mxs : st.m;
        const float alpha = raise ? __builtin_amdgcn_exp2f(st.m - m_new) : 1.f;
        st.l *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) st.o[dt] *= alpha;
        st.m = m_new;
    }
    float psum = 0.f;
    const float shift = (FP8 ? kPBiasLog2 : 0.f) - st.m;
#pragma unroll
    for (int t = 0; t < S::NT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = __builtin_amdgcn_exp2f(fmaf(s[t][r], cscale, shift));
            s[t][r] = p;
            if constexpr (!FP8) psum += p;
        }
    // BF16: this lane half's share of the row sum, from the unrounded P (the
    // bf16 rounding of P below is 2^-9 relative).  FP8: the full row sum of
    // the e4m3-rounded P that the PV MFMAs consume, taken by an MFMA below.
    if constexpr (!FP8) st.l += psum;

    __builtin_amdgcn_s_setprio(S::PAIR ? 1 : 0);
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
        // The row sum of exactly the e4m3 probabilities the PV MFMAs weigh V
        // with (so the output weights sum to one), by one 16x16x128 MFMA:
        // read as its B operand, lane 16g + j of P^T holds K group g of
        // column j, keys of query row 16 (g & 1) + j; the selector A operand
        // (lane 16g + i: row i, K group g) is e4m3 1.0 where ((i >> 2) & 1)
        // == (g & 1), so output lane l (rows 4 (l >> 4) + v, column l & 15)
        // holds the sum of query row l & 31 over both key halves.
        int rsel = L.rsel;
        asm volatile("" : "+v"(rsel));
        const v8i sel = {rsel, rsel, rsel, rsel, rsel, rsel, rsel, rsel};
        v4f rowsum = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(sel, pop, v4f{}, 0, 0, 0, 0, 0, 0);
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
        // All 4 row-sum registers stay allocated until here: the inline-asm
        // LDS reads above are invisible to the MFMA hazard checks and must not
        // be given registers the in-flight MFMA is still going to write.
        asm volatile("" : "+v"(rowsum));
        st.l += rowsum[0];
    } else {
        v8bf pop[2][2];
#pragma unroll
        for (int t = 0; t < S::NT; ++t)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int e2 = 0; e2 < 8; ++e2) pop[t][u][e2] = (__bf16)s[t][8 * u + e2];
        // A operand lane (d row 16*(grp&1)+gl, k-group grp>>1): for score
        // tile t and half u, keys 32t + 16u + 8*(grp>>1) + [0, 8) of column
        // d, 4 per transposing read.  Step 2 dt + t takes score tile t of d
        // tile dt (two MFMAs); its four reads are issued one step ahead, so
        // that the LDS latency hides behind the previous step's MFMAs.
        // The second buffer of a 32 KB tile lies beyond the 16-bit immediate:
        // its 64 KB part goes into the address.
        constexpr uint32_t VHI = VBASE & ~0xFFFFu;
        if constexpr (S::PAIR) {
            // One wave's 32 keys: per d tile two MFMAs (keys 0-15, 16-31 of
            // its half), each operand's two reads issued one MFMA ahead (two
            // 4-register buffers: this mode has no registers for more).
            constexpr int SUB = 2 * DT;
            v2i vb[2][2];
            auto issue1 = [&](auto sc) {
                constexpr int sub = decltype(sc)::value, dt = sub >> 1, u = sub & 1;
                constexpr int o = (VBASE + 16 * u * ROW) & 0xFFFF;
                vb[sub & 1][0] = ds_read_tr16_b64<o>((L.v_addr[0] ^ ((4 * dt) << 4)) + (VHI + rt_off));
                vb[sub & 1][1] = ds_read_tr16_b64<o>((L.v_addr[1] ^ ((4 * dt) << 4)) + (VHI + rt_off));
            };
            issue1(std::integral_constant<int, 0>{});
            static_for<0, SUB>([&](auto sc) {
                constexpr int sub = decltype(sc)::value, dt = sub >> 1, u = sub & 1;
                v2i(&x)[2] = vb[sub & 1];
                lds_results_ready(x);
                if constexpr (sub + 1 < SUB) issue1(std::integral_constant<int, sub + 1>{});
                __builtin_amdgcn_sched_barrier(0);
                const v4i aop = {x[0][0], x[0][1], x[1][0], x[1][1]};
                st.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, aop), pop[0][u], st.o[dt], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            });
            return;
        }
        constexpr int STEPS = S::NT * DT;
        v2i buf[2][4];
        auto issue = [&](auto sc) {
            constexpr int step = decltype(sc)::value, dt = step / S::NT, t = step % S::NT;
            constexpr int o0 = (VBASE + 32 * t * ROW) & 0xFFFF, o1 = (VBASE + (32 * t + 16) * ROW) & 0xFFFF;
            const uint32_t a0 = (L.v_addr[0] ^ ((4 * dt) << 4)) + (VHI + rt_off);
            const uint32_t a1 = (L.v_addr[1] ^ ((4 * dt) << 4)) + (VHI + rt_off);
            v2i(&x)[4] = buf[step & 1];
            x[0] = ds_read_tr16_b64<o0>(a0);
            x[1] = ds_read_tr16_b64<o0>(a1);
            x[2] = ds_read_tr16_b64<o1>(a0);
            x[3] = ds_read_tr16_b64<o1>(a1);
        };
        issue(std::integral_constant<int, 0>{});
        static_for<0, STEPS>([&](auto sc) {
            constexpr int step = decltype(sc)::value, dt = step / S::NT, t = step % S::NT;
            v2i(&x)[4] = buf[step & 1];
            lds_results_ready(x);
            if constexpr (step + 1 < STEPS) issue(std::integral_constant<int, step + 1>{});
            __builtin_amdgcn_sched_barrier(0);
            const v4i aop0 = {x[0][0], x[0][1], x[1][0], x[1][1]};
            const v4i aop1 = {x[2][0], x[2][1], x[3][0], x[3][1]};
            st.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, aop0), pop[t][0], st.o[dt], 0, 0, 0);
            st.o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, aop1), pop[t][1], st.o[dt], 0, 0, 0);
            // (the barriers keep the next step's reads ahead of both MFMAs)
            __builtin_amdgcn_sched_barrier(0);
        });
    }
}

// Wait for tile `cur` (in BUF), start the prefetch of `nxt` into the other
// buffer, then compute `cur`.
// PAIR (double-buffered): BUF is 0 and rbuf the buffer of `cur`, so that
// the walk has one loop body (two bodies made the register allocator keep
// copies of O^T across them and spill).
template <class S, int BUF, bool CAUSAL>
__device__ __forceinline__ void tile_step(const FwdArgs& a, const TileCursor& cur, const TileCursor& nxt,
                                          uint8_t* lds, int wave, int tid, int h, const LaneMap<S>& L,
                                          const QOperand<S> (&qop)[S::QK], float cscale, SoftmaxState<S>& st,
                                          int row_limit, int first_key, int rbuf) {
    const int valid = min(kKeyTile, cur.n - cur.base);
    const uint32_t rt_off = S::PAIR && S::NBUF == 2 ? rbuf * 2 * S::TILE : 0;
    uint8_t* const lds_v = lds + BUF * 2 * S::TILE + rt_off + S::TILE;
    if constexpr (S::NBUF == 2) {
        wait_vmem();      // this wave's loads of the current tile have landed
        __syncthreads();  // ... and every wave's; the other buffer is free
        if (nxt.e < a.num_entries) {
            if constexpr (S::PAIR)
                stage_tile_async<S, 0>(a, nxt, lds + (rt_off ^ (2 * S::TILE)), wave, L);
            else
                stage_tile_async<S, BUF ^ 1>(a, nxt, lds, wave, L);
        }
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
    compute_tile<S, BUF, CAUSAL>(lds, rt_off, (CAUSAL ? min(valid, row_limit - cur.base) : valid) - first_key, qop,
                                 cscale, L, h, st);
}

// Query row of lane j of the wave in 32-row slot pw: its index among the
// KV head's rows (FIXUP: entry fix_first + 32 pw + j of the head's list in
// the guard plan, -1 past its fix_count rows), whether it exists, its rank
// and local token, and the byte offset of its Q and output rows in [pcp, Hq,
// local_q, D] bf16.
struct QueryRow {
    int row;
    bool ok;
    int rank;
    int tok;
    int64_t off;
};
template <int D, bool FIXUP>
__device__ __forceinline__ QueryRow query_row(const FwdArgs& a, int head, int row_tile, int pw, int j, int fix_first,
                                              int fix_count) {
    QueryRow r;
    if constexpr (FIXUP) {
        const int idx = fix_first + pw * kRowsPerWave + j;
        r.row = idx < fix_count ? a.guard_plan[guard_list_offset(a.num_kv_heads) +
                                               head * guard_head_segment(a.rows_per_head) + idx]
                                : -1;
    } else
        r.row = row_tile * kRowsPerGroup + pw * kRowsPerWave + j;
    r.ok = FIXUP ? r.row >= 0 : r.row < a.rows_per_head;
    const int rowc = r.ok ? r.row : (FIXUP ? 0 : a.rows_per_head - 1);
    r.rank = rowc / a.group_rows;
    const int rem = rowc - r.rank * a.group_rows;
    const int head_in_group = rem / a.local_q;
    r.tok = rem - head_in_group * a.local_q;
    r.off = ((int64_t)(r.rank * a.num_q_heads + head * a.group + head_in_group) * a.local_q + r.tok) * D * 2;
    return r;
}

// CAUSAL: causal attention of the current tokens among themselves (their
// K/V are one page of block_size tokens in global order, no block table):
// row (rank, token) sees current keys up to its own global position.  The
// epilogue can then merge the result with a history output (merge_o,
// merge_lse) by log-sum-exp.
// SPLIT: the workgroup walks only its split's share of the table entries
// and writes a normalised FP32 partial output and log-sum-exp (merged by
// merge_splits_kernel).
// FIXUP: the BF16-MFMA pass of a precision-guarded launch.  The guard plan
// lists the rows the e4m3 pass flagged, in groups of 128 rows of one KV
// head; in sparse mode (guard_ranges() >= 2 ranges for the listed groups)
// workgroup b takes group b / ranges and walks history range b % ranges
// into the guard partials (merged by guard_merge_kernel), in dense mode it
// takes group b and writes the output directly; workgroups past the plan
// exit at once.
template <int D, bool STORE8, bool FP8, bool CAUSAL = false, bool SPLIT = false, bool FIXUP = false>
__global__ void __launch_bounds__((TileShape<D, STORE8, FP8>::THREADS), (TileShape<D, STORE8, FP8>::PAIR ? 1 : 2))
    history_fwd_kernel(FwdArgs a) {
    static_assert(!(CAUSAL && SPLIT), "the current-token step is not split");
    static_assert(!FIXUP || (!FP8 && !CAUSAL && !SPLIT), "the guard's fixup runs BF16 MFMAs, one launch");
    using S = TileShape<D, STORE8, FP8>;
    constexpr int ROW = S::ROW, CHUNKS = S::CHUNKS, QK = S::QK, DT = S::DT;

    __shared__ __attribute__((aligned(1024))) uint8_t lds[S::LDS_BYTES];
    __shared__ int wave_limit[S::WAVES];
    __shared__ float pair_ml[S::PAIR ? kWaves * 64 * 2 : 1];  // PAIR: the partners' (m, l) per lane

    // ---- XCD-aware work mapping ------------------------------------------
    // Workgroups are dealt to the 8 XCDs round-robin by launch index; give
    // each XCD a contiguous range of (KV head, row tile) work items so that
    // the workgroups sharing an XCD's L2 stream the same KV head together.
    // CAUSAL: work grows with the row tile (later ranks see more current
    // keys) and the keys fit in L2 anyway, so launch the heaviest tiles
    // first, both heads alike, and let the early finishers take the light
    // ones (longest-first balancing over all XCDs).
    // SPLIT: items run row tile fastest, then split, then KV head, so that an
    // XCD's workgroups share one (KV head, split) and its pages.
    int splits = SPLIT ? a.splits : 1;
    const int items = a.row_tiles * a.num_kv_heads * splits;
    int head, row_tile, split = 0, slot = 0, fix_first = 0, fix_count = 0, listed = 0;
    bool sparse = false;
    if constexpr (FIXUP) {
        listed = guard_groups(a.guard_plan, a.num_kv_heads);
        const int ranges = guard_ranges(listed, a.guard_partial_rows, a.splits);
        sparse = ranges > 0;
        if (sparse) {
            if ((int)blockIdx.x >= listed * ranges) return;
            splits = ranges;
            slot = blockIdx.x / splits;
            split = blockIdx.x - slot * splits;
        } else {
            if ((int)blockIdx.x >= listed) return;
            slot = blockIdx.x;
        }
        const GuardGroup gg = guard_group(a.guard_plan, a.num_kv_heads, slot);
        head = gg.head;
        fix_first = gg.first;
        fix_count = gg.count;
        row_tile = 0;
    } else if constexpr (CAUSAL) {
        const int item = blockIdx.x;
        if (item >= items) return;
        head = item % a.num_kv_heads;
        row_tile = a.row_tiles - 1 - item / a.num_kv_heads;
    } else {
        const int per_xcd = (items + 7) / 8;
        const int item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
        if (item >= items) return;
        row_tile = item % a.row_tiles;
        head = item / a.row_tiles / splits;
        split = item / a.row_tiles - head * splits;
    }
    int entry_begin = 0;
    if constexpr (SPLIT) {
        entry_begin = (int)((int64_t)a.num_entries * split / splits);
        a.num_entries = (int)((int64_t)a.num_entries * (split + 1) / splits);
    }
    // FIXUP, sparse: range `split` of `splits` equal ranges of the walk's key
    // tiles (not of table entries: short ranges even for a few large pages),
    // found by the whole workgroup at once
    int tiles_left = -1;
    TileCursor range_first{};
    if constexpr (FIXUP) {
        __shared__ int walk_red[S::THREADS / 64];
        __shared__ TileCursor walk_first;
        if (sparse) range_first = range_cursor<S::THREADS>(a, head, split, splits, tiles_left, walk_red, &walk_first);
    }

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // PAIR: waves w and w + 4 (one SIMD) share 32 rows; wave w + 4 takes the
    // tiles' keys 32..63
    const int pw = S::PAIR ? wave & (kWaves - 1) : wave;  // the wave's 32-row slot
    const int kh = S::PAIR ? wave / kWaves : 0;           // its key half
    const int j = lane & 31;  // query column of the score tile / A-operand row
    const int h = lane >> 5;  // k-group (lane half)
    const int grp = lane >> 4;
    const int gl = lane & 15;

    // ---- this lane's query row -------------------------------------------
    const QueryRow qr = query_row<D, FIXUP>(a, head, row_tile, pw, j, fix_first, fix_count);
    const int rank = qr.rank, tok = qr.tok;
    const uint8_t* const qrow = a.q + qr.off;

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
        L.k_addr = row * ROW + ((first_chunk ^ chunk_swizzle<FP8, CHUNKS>(row)) << 4) + kh * S::K_T1_ROWS * ROW;
    }
    if constexpr (FP8) {
        // key 32*(grp>>1) + (gl>>1) (+ 8s for the other reads) -> row below
        const int row = lds_row<FP8>(32 * (grp >> 1) + (gl >> 1));
        L.v_addr[0] = lds_address(lds) + row * ROW + (((grp & 1) ^ chunk_swizzle_v<FP8, CHUNKS>(row)) << 4) +
                      8 * (gl & 1);
        L.rsel = ((lane ^ (lane >> 2)) & 4) ? 0 : 0x38383838;
    } else {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const int vkey = 8 * (grp >> 1) + 4 * s2 + (gl >> 2);  // + 16u + 32t: same swizzle
            const int dbyte = 2 * (16 * (grp & 1) + 4 * (gl & 3));
            L.v_addr[s2] = lds_address(lds) + vkey * ROW + (((dbyte >> 4) ^ chunk_swizzle_v<FP8, CHUNKS>(vkey)) << 4) +
                           (dbyte & 15) + kh * 32 * ROW;
        }
    }
#pragma unroll
    for (int i = 0; i < (S::DMA_SPLIT ? S::DMA_PER_WAVE : 1); ++i) {
        const int byte = (S::WAVES * i + wave) * 1024 + lane * 16;
        const int row = byte / ROW;
        const int pos = (byte % ROW) / 16;
        L.dma_off[i] = lds_row<FP8>(row) * S::GROW + (pos ^ chunk_swizzle<FP8, CHUNKS>(row)) * 16;
        L.dma_off_v[i] = lds_row<FP8>(row) * S::GROW + (pos ^ chunk_swizzle_v<FP8, CHUNKS>(row)) * 16;
    }

    // ---- walk the block table -----------------------------------------------
    SoftmaxState<S> st;
    // PAIR: a wave can see a whole tile masked before any valid key (its
    // half of a row's first tile); a finite floor keeps the probabilities of
    // such a tile 0 (2^(-inf + 1e30)) instead of NaN (2^(-inf + inf)), and
    // the first real tile rescales by 2^(-1e30 - m) = 0.
    st.m = S::PAIR ? -1.0e30f : -INFINITY;
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
        for (int i = 1; i < S::WAVES; ++i) group_limit = max(group_limit, wave_limit[i]);
    }
    auto advance = [&](const TileCursor& c) {
        if constexpr (CAUSAL) {
            const TileCursor n = next_current_tile(a, head, c);
            return n.base < group_limit ? n : TileCursor{a.num_entries, 0, 0, 0};
        } else {
            if (FIXUP && tiles_left >= 0 && --tiles_left <= 0) return TileCursor{a.num_entries, 0, 0, 0};
            return next_tile(a, head, c);
        }
    };

    TileCursor cur;
    if (FIXUP && sparse)
        cur = range_first;
    else
        cur = advance(TileCursor{entry_begin - 1, 0, 0, 0});
    if constexpr (S::NBUF == 2) {
        if (cur.e < a.num_entries) stage_tile_async<S, 0>(a, cur, lds, wave, L);
    }
    if constexpr (S::PAIR && S::NBUF == 2) {
        for (int rbuf = 0; cur.e < a.num_entries; rbuf ^= 1) {
            const TileCursor nxt = advance(cur);
            tile_step<S, 0, CAUSAL>(a, cur, nxt, lds, wave, tid, h, L, qop, cscale, st, row_limit, 32 * kh, rbuf);
            cur = nxt;
        }
    } else {
        while (cur.e < a.num_entries) {
            TileCursor nxt = advance(cur);
            tile_step<S, 0, CAUSAL>(a, cur, nxt, lds, wave, tid, h, L, qop, cscale, st, row_limit, 32 * kh, 0);
            cur = nxt;
            if constexpr (S::NBUF == 2) {
                if (cur.e >= a.num_entries) break;
                nxt = advance(cur);
                tile_step<S, 1, CAUSAL>(a, cur, nxt, lds, wave, tid, h, L, qop, cscale, st, row_limit, 32 * kh, 0);
                cur = nxt;
            }
        }
    }

    // ---- PAIR: the key halves' results meet in the first wave of the pair --
    if constexpr (S::PAIR) {
        // O^T as [pair][register quad][lane] float4s (conflict-free), m and
        // this lane half's l beside; (m, l) = (-1e30, 0) for a half that saw
        // no valid key (weight 2^(-1e30 - m) = 0 against a real m).
        float* const xo = (float*)lds + pw * (DT * 16 * 64);
        __syncthreads();  // every wave is done with the tile buffers
        if (kh == 1) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    *(v4f*)(xo + ((4 * dt + r4) * 64 + lane) * 4) =
                        v4f{st.o[dt][4 * r4], st.o[dt][4 * r4 + 1], st.o[dt][4 * r4 + 2], st.o[dt][4 * r4 + 3]};
            pair_ml[(pw * 64 + lane) * 2] = st.m;
            pair_ml[(pw * 64 + lane) * 2 + 1] = st.l;
        }
        __syncthreads();
        if (kh == 1) return;
        const float m1 = pair_ml[(pw * 64 + lane) * 2], l1 = pair_ml[(pw * 64 + lane) * 2 + 1];
        const float m = fmaxf(st.m, m1);
        const float w0 = __builtin_amdgcn_exp2f(st.m - m), w1 = __builtin_amdgcn_exp2f(m1 - m);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const v4f x = *(const v4f*)(xo + ((4 * dt + r4) * 64 + lane) * 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) st.o[dt][4 * r4 + i] = fmaf(w1, x[i], w0 * st.o[dt][4 * r4 + i]);
            }
        st.l = fmaf(w1, l1, w0 * st.l);
        st.m = m;
    }

    // ---- epilogue: O = O^T / l, bf16; log-sum-exp; merge -------------------
    // (FP8: st.l is already the whole row's sum, in both lane halves)
    const QueryRow er = qr;
    const bool row_ok = er.ok;
    const int64_t row_off = er.off;
    const float l_tot = FP8 ? st.l : halves_sum(st.l);
    float scale = l_tot > 0.f ? a.v_scale / l_tot : 0.f;
    // sum_k exp(score_k) = l * 2^(m - bias): P was 2^(x - m + bias)
    float lse = l_tot > 0.f ? __logf(l_tot) + (st.m - (FP8 ? kPBiasLog2 : 0.f)) * kLn2 : -INFINITY;
    const int64_t row_index = row_off / (D * 2);
    if (FIXUP && sparse) {
        // guard partials [ranges, listed * 128, D]: slot rows in tile order
        if (row_ok) {
            const int64_t prow = ((int64_t)split * listed + slot) * kRowsPerGroup + pw * kRowsPerWave + j;
            float* const po = a.part_o + prow * D;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int d = 32 * dt + 8 * r4 + 4 * h;
                    *(v4f*)(po + d) = v4f{st.o[dt][4 * r4 + 0] * scale, st.o[dt][4 * r4 + 1] * scale,
                                          st.o[dt][4 * r4 + 2] * scale, st.o[dt][4 * r4 + 3] * scale};
                }
            if (h == 0) a.part_lse[prow] = lse;
        }
        return;
    }
    if constexpr (SPLIT) {
        if (row_ok) {
            const int64_t prow = (int64_t)split * a.rows_per_head * a.num_kv_heads + row_index;
            float* const po = a.part_o + prow * D;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int d = 32 * dt + 8 * r4 + 4 * h;
                    *(v4f*)(po + d) = v4f{st.o[dt][4 * r4 + 0] * scale, st.o[dt][4 * r4 + 1] * scale,
                                          st.o[dt][4 * r4 + 2] * scale, st.o[dt][4 * r4 + 3] * scale};
                }
            if (h == 0) {
                a.part_lse[prow] = lse;
                if (a.part_m) a.part_m[prow] = st.m;
            }
        }
        return;
    }
    // Precision guard (e4m3 MFMAs): l / 2^6 is the row's probability mass
    // sum_k 2^(x_k - m) against the running reference; a row below its KV
    // head's threshold joins the guard plan.
    if (FP8 && a.guard_thr) {
        const float thr = guard_threshold(a.guard_thr, head, D / 16);
        if (row_ok && h == 0 && st.l * (1.f / 64.f) < thr)
            guard_append(a.guard_rows, a.num_kv_heads, a.rows_per_head, head, er.row);
    }
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

}  // namespace pcpa

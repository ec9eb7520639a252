// ovl::history_fwd_overlap: the e4m3 head_dim-256 kernel, and the merge of
// split-history partial outputs.
#pragma once

#include "common.hpp"

namespace pcpa {

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
    const float ninf = -INFINITY;
    static_for<0, 32>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        s[k >> 4][k & 15] = mask_key_at_or_past<k>(s[k >> 4][k & 15], lim, ninf);
    });
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
// requested in iteration j, one 1 KB block per PV MFMA of the PV-first group
// (the LDS-DMA writes then reach the LDS spread over the iteration rather
// than in one burst that stalls every wave's operand reads).  Tiles before the first and after
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
    // Softmax micro-slices [pv_begin(i), pv_begin(i+1)) run beside PV MFMA i.
    static constexpr int pv_begin(int i) {
        constexpr int b256[] = {0, 4, 6, 7, 8, 9, 10, 11, 14};
        constexpr int b128[] = {0, 5, 8, 11, 14};
        return D == 256 ? b256[i] : b128[i];
    }
};

// Who moves the K and V tiles: the last WAVES = kWaves / 2 waves of the
// workgroup, the group that runs PV first (one wave per SIMD), issue the
// LDS-DMA of every K and V tile and each waits for its own blocks; the
// barrier after the waits publishes them to all waves (about 1% faster than
// all eight waves issuing).
template <int D, int WAVES>
struct DmaPlan {
    static_assert(WAVES == kWaves / 2, "the PV-first group issues all DMA");
    static constexpr int ROW = D;
    static constexpr int DPW = kKeyTile * ROW / 1024 / WAVES;  // 1 KB blocks per wave per K (or V) tile
    static constexpr int STRIDE = WAVES * 1024;                // LDS bytes between a wave's blocks
    // A wave's block i lands i * BLOCK_ROWS LDS rows after its block 0
    // (rows < BLOCK_ROWS).  lds_row permutes row bits, so block i holds the
    // keys lds_row(i * BLOCK_ROWS) further on; a multiple of 16 rows keeps
    // the chunk swizzle of block 0.
    static constexpr int BLOCK_ROWS = STRIDE / ROW;
    static_assert(BLOCK_ROWS % 16 == 0, "DMA blocks must share the chunk swizzle");
    // Byte offset of block i's keys; addressed from the middle of their span
    // (MID) they fit the load's 13-bit signed immediate offset.
    static constexpr int offset(int i) { return lds_row<true>(i * BLOCK_ROWS) * ROW; }
    static constexpr int MID = offset(DPW - 1) / 2;
    static_assert(MID < 4096, "DMA block offsets must fit the immediate");
    __device__ static bool issues(int wave) { return wave >= kWaves - WAVES; }
    __device__ static int block(int wave) { return wave - (kWaves - WAVES); }
};

struct Lanes {
    uint32_t k_addr;  // score operand, K stage 0, k-step 0, low 16 bytes
    uint32_t v_addr;  // PV operand, V stage 0, d tile 0 (includes the ring offset)
    uint32_t dma_k;   // byte offset of the lane's K chunk of its DMA block 0 in a tile, plus DmaPlan::MID
    uint32_t dma_v;   // same for V (its own swizzle)
    int rsel;         // row-sum selector operand word (see s_half)
};

__device__ __forceinline__ bool is_real(const FwdArgs& a, const TileCursor& c) {
    return c.e >= 0 && c.e < a.num_entries;
}

// Valid keys of a tile for the softmax: its length if real, 0 before the
// first tile, -1 after the last (phantom tiles; -1 also ends the walk).
__device__ __forceinline__ int tile_keys(const FwdArgs& a, const TileCursor& c) {
    return is_real(a, c) ? c.n - c.base : (c.e < 0 ? 0 : -1);
}

// Tiles j-1 .. j+2 of iteration j.  e < 0: before the first tile;
// e >= num_entries: after the last (both phantom).  Tiles j+1 and j+2 are
// still to be loaded and keep their cursors; of tiles j-1 and j only the
// softmax's valid key counts (tile_keys) are kept, which keeps the loop's
// scalar registers few.
struct Cursors {
    int km1, k0;
    TileCursor c1, c2;
};

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

// Key of the lane's chunk of DMA block i (LDS byte i * P::STRIDE +
// wave_off + 16 * lane, rows permuted by lds_row).
template <class P>
__device__ __forceinline__ int dma_chunk_key(int i, int wave_off) {
    return lds_row<true>((i * P::STRIDE + wave_off + __lane_id() * 16) / P::ROW);
}

// DMA block I of a full tile at `tile` into LDS at `dst` (the LDS address of
// the wave's block 0 in the stage).  lane_mid is the lane's chunk offset in
// the tile plus P::MID: the blocks' offsets from it are the loads'
// immediates, and m0 is taken that much lower (it stays inside the block:
// imm <= MID < STRIDE <= I * STRIDE for I > 0).
template <class P, int I>
__device__ __forceinline__ void dma_block(const uint8_t* tile, uint32_t lane_mid, uint32_t dst) {
    constexpr int imm = P::offset(I) - P::MID;
    static_assert(I == 0 || imm < I * P::STRIDE, "m0 must stay inside the block");
    dma_sbase<imm>(tile, lane_mid, dst + (I * P::STRIDE - imm));
}
template <class P, int I = 0>
__device__ __forceinline__ void dma_blocks(const uint8_t* tile, uint32_t lane_mid, uint32_t dst) {
    if constexpr (I < P::DPW) {
        dma_block<P, I>(tile, lane_mid, dst);
        dma_blocks<P, I + 1>(tile, lane_mid, dst);
    }
}

// Global addresses of cursor c's K and V tiles (wave-uniform).
template <class S>
__device__ __forceinline__ const uint8_t* k_tile(const FwdArgs& a, const TileCursor& c) {
    return a.kv + c.k_off + (int64_t)c.base * S::ROW;
}
template <class S>
__device__ __forceinline__ const uint8_t* v_tile(const FwdArgs& a, const TileCursor& c) {
    return k_tile<S>(a, c) + (int64_t)a.num_kv_heads * a.head_stride;
}

// Issue the K tile of cursor c into K stage st (lds: LDS address of the
// rings).  A phantom tile's cursor reads the pool's first tile (k_off 0),
// so that every iteration issues the same loads.
template <class S, class P>
__device__ __forceinline__ void load_k(const FwdArgs& a, const TileCursor& c, uint32_t lds, int st, int wave_off,
                                       uint32_t lane_mid) {
    dma_blocks<P>(k_tile<S>(a, c), lane_mid, lds + st * S::TILE + wave_off);
}

// The V tile of cursor c with `valid` (< 64) valid keys into V stage st:
// rows past the valid length (all rows of a phantom tile) come from
// zero_chunk, so V stages of masked keys hold zeros.
template <class S, class P>
__device__ __forceinline__ void load_v_partial(const FwdArgs& a, const TileCursor& c, uint32_t lds, int st,
                                               int wave_off, uint32_t lane_mid, int valid) {
    const uint8_t* const vt = v_tile<S>(a, c) + lane_mid;
    const uint32_t dst = lds + S::RING + st * S::TILE + wave_off;
#pragma unroll
    for (int i = 0; i < P::DPW; ++i) {
        const uint8_t* const src = dma_chunk_key<P>(i, wave_off) < valid ? vt + (P::offset(i) - P::MID) : zero_chunk;
        dma_vaddr(src, dst + i * P::STRIDE);
    }
}

// Issue the V tile of cursor c into V stage st (real: c is a tile).
template <class S, class P>
__device__ __forceinline__ void load_v(const FwdArgs& a, const TileCursor& c, uint32_t lds, int st, int wave_off,
                                       uint32_t lane_mid, bool real) {
    const int valid = real ? c.n - c.base : 0;
    if (valid >= kKeyTile)
        dma_blocks<P>(v_tile<S>(a, c), lane_mid, lds + S::RING + st * S::TILE + wave_off);
    else
        load_v_partial<S, P>(a, c, lds, st, wave_off, lane_mid, valid);
}

// The four transposing reads of one PV A operand (d tile of `addr`) from V
// stage VST: keys 32g + 8s + m of the d tile live in LDS rows (8g + m) +
// {0, 32, 16, 48}[s].
template <int D, int VST>
__device__ __forceinline__ void read_v_operand(uint32_t addr, v2i (&x)[4]) {
    constexpr int off = VST * Shape<D>::TILE, ROW = Shape<D>::ROW;
    x[0] = ds_read_tr8_b64<off + 0 * ROW>(addr);
    x[1] = ds_read_tr8_b64<off + 32 * ROW>(addr);
    x[2] = ds_read_tr8_b64<off + 16 * ROW>(addr);
    x[3] = ds_read_tr8_b64<off + 48 * ROW>(addr);
}

// S half: S^T = K Q^T from K stage KST; operand reads one MFMA ahead (the
// other wave on the SIMD covers the latency).  PREFETCH_V: the last slot
// starts the first V-operand read of the PV half that follows (stage VST).
// Also adds to l the row sum of P_last, the probabilities the preceding PV
// half consumed, scaled by the alpha that PV half applied.
//
// The row sum is one 16x16x128 MFMA (half the cycles of a 32x32x64 one):
// read as its B operand, P_last's lane 16g + j holds K group g of column j,
// i.e. keys of query row 16 (g & 1) + j (g >> 1 picks the key half).  The
// selector A operand (lane 16g + i holds row i, K group g) is e4m3 1.0 where
// ((i >> 2) & 1) == (g & 1), else 0, so output row i of column j sums the
// groups of row 16 ((i >> 2) & 1) + j over both key halves.  Output lane l
// holds rows 4 (l >> 4) + v of column l & 15: the sum of query row l & 31,
// the row that lane holds in every other operand.
template <int D, int KST, bool PREFETCH_V, int VST>
__device__ __forceinline__ void s_half(uint32_t k_addr, uint32_t v_addr, const v8i (&q)[Shape<D>::QK], v16f (&s)[2],
                                       v2i (&xv)[4], const v8i& p_last, SoftmaxRow& sm, int rsel) {
    using S = Shape<D>;
    // The selector operand is rebuilt from an opaque register instead of
    // occupying 8 VGPRs for good.
    asm volatile("" : "+v"(rsel));
    const v8i sel = {rsel, rsel, rsel, rsel, rsel, rsel, rsel, rsel};
    v4f rowsum = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(sel, p_last, v4f{}, 0, 0, 0, 0, 0, 0);
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
            read_v_operand<D, VST>(v_addr, xv);
        }
        const v4i lo = kr[op & 1][0], hi = kr[op & 1][1];
        const v8i kop = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        s[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(kop, q[c], c == 0 ? v16f{} : s[t], 0, 0, 0, 0, 0, 0);
        if constexpr (op == 1) {
            // The row sum has long completed (two score MFMAs since): read
            // it, then free its registers.  All 4 stay allocated until the
            // read: the inline-asm LDS reads are invisible to the hazard
            // checks and must not be given registers that the in-flight
            // MFMA is still going to write.  (The read waits for the MFMA;
            // the tie after it keeps the later reads behind it.)
            sm.l = fmaf(rowsum[0], sm.alpha, sm.l);
            asm volatile("" : "+v"(rowsum));
        }
    });
}

// PV half: O^T += V^T P_old^T from V stage VST, beside the softmax of s
// (valid keys < valid) into p_new; then the lazy O^T rescale.  PREFETCHED:
// the first V-operand read was issued by the S half.  after_mfma(dt) runs
// after PV MFMA dt is issued (the DMA-issuing waves spread their tile
// loads over the PV half there, one block per MFMA).
template <int D, int VST, bool PREFETCHED, bool FAST, class Hook>
__device__ __forceinline__ void pv_half(uint32_t v_addr, v2i (&xv0)[4], v16f (&o)[Shape<D>::DT], const v8i& p_old,
                                        v16f (&s)[2], v8i& p_new, SoftmaxRow& sm, int valid, int h,
                                        Hook&& after_mfma) {
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
        read_v_operand<D, VST>(v_addr ^ ((2 * dt) << 4), buf(dc));
    };
    if constexpr (!PREFETCHED) issue_v(std::integral_constant<int, 0>{});
    static_for<0, S::DT>([&](auto dc) {
        constexpr int dt = decltype(dc)::value;
        v2i(&x)[4] = buf(dc);
        lds_wait<0>(x);
        if constexpr (dt + 1 < S::DT) issue_v(std::integral_constant<int, dt + 1>{});
        const v8i vop = {x[0][0], x[0][1], x[1][0], x[1][1], x[2][0], x[2][1], x[3][0], x[3][1]};
        o[dt] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vop, p_old, o[dt], 0, 0, 0, 0, 0, 0);
        after_mfma(dc);
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
template <int D, int J4, bool LATE, bool FAST, int DMAW>
__device__ __forceinline__ void iteration(const FwdArgs& a, uint8_t* lds, int wave, int h, const Lanes& L,
                                          const v8i (&q)[Shape<D>::QK], v16f (&s)[2], v8i (&pbuf)[2],
                                          v16f (&o)[Shape<D>::DT], SoftmaxRow& sm, Cursors& cs, int head,
                                          v2i (&xv)[4]) {
    using S = Shape<D>;
    constexpr int KST = J4;  // K(j)

    // ---- K(j) and V(j-1) have landed (for every wave) ----------------------
    // Loads issued one iteration ago may be pending: V(j) and K(j+1) (a
    // phantom K tile is loaded too).  Each wave that issues DMA waits for its own blocks; the
    // barrier then publishes all of them.
    using P = DmaPlan<D, DMAW>;
    if constexpr (LATE) wait_vmem_le<2 * P::DPW>();
    __builtin_amdgcn_s_barrier();
    // The wave offset and operand bases
    // are made opaque so that the DMA destinations and operand addresses are
    // recomputed in the loop rather than hoisted and spilled.
    int wave_off = P::block(wave) * 1024;
    uint32_t k_addr = L.k_addr, v_addr = L.v_addr;
    asm volatile("" : "+s"(wave_off), "+v"(k_addr), "+v"(v_addr));
    if constexpr (!LATE) {
        // S(j), then PV(j-1) beside softmax(j)
        constexpr int VST = (J4 + 3) % kStages;
        s_half<D, KST, true, VST>(k_addr, v_addr, q, s, xv, pbuf[J4 & 1], sm, L.rsel);
        pv_half<D, VST, true, FAST>(v_addr, xv, o, pbuf[(J4 + 1) & 1], s, pbuf[J4 & 1], sm,
                              cs.k0, h, [](auto) {});
    } else {
        // PV(j-2) beside softmax(j-1), then S(j).  The first V-operand read
        // of PV(j-2) was issued at the end of the previous iteration's S half
        // (V(j-2) landed before the previous barrier), so it is in flight
        // across the barrier; this S half issues the one for PV(j-1).
        constexpr int VST = (J4 + 2) % kStages;
        // This group's DMA of K(j+2) and V(j+1) is spread over its PV half,
        // one block per PV MFMA: K after the first DPW, V after the next DPW
        // (a V tile with masked rows, rare, is issued before the half).  K
        // stage (j+2) % 4 and V stage (j+1) % 4 were last read in iteration
        // j-1, before this iteration's barrier.
        const uint32_t lds_u = lds_address(lds);
        const bool v_real = is_real(a, cs.c1);
        const int v_valid = v_real ? cs.c1.n - cs.c1.base : 0;
        if (v_valid < kKeyTile) load_v_partial<S, P>(a, cs.c1, lds_u, (J4 + 1) % kStages, wave_off, L.dma_v, v_valid);
        const uint8_t* const ktile = k_tile<S>(a, cs.c2);
        const uint32_t kdst = lds_u + ((J4 + 2) % kStages) * S::TILE + wave_off;
        const uint8_t* const vtile = v_tile<S>(a, cs.c1);
        const uint32_t vdst = lds_u + S::RING + ((J4 + 1) % kStages) * S::TILE + wave_off;
        auto dma_step = [&](auto dc) {
            constexpr int i = decltype(dc)::value;
            if constexpr (i < P::DPW) {
                dma_block<P, i>(ktile, L.dma_k, kdst);
            } else if constexpr (i < 2 * P::DPW) {
                if (v_valid >= kKeyTile) dma_block<P, i - P::DPW>(vtile, L.dma_v, vdst);
            }
        };
        // this half carries the group's LDS-DMA issue and softmax VALU work;
        // issuing it ahead of the other wave on the SIMD (whose score MFMAs
        // queue on the matrix core anyway) measured 0.65% faster on the
        // full 64-rank workload (6.79 vs 6.83 ms, interleaved on one box)
        __builtin_amdgcn_s_setprio(1);
        pv_half<D, VST, true, FAST>(v_addr, xv, o, pbuf[J4 & 1], s, pbuf[(J4 + 1) & 1], sm,
                              cs.km1, h, dma_step);
        __builtin_amdgcn_s_setprio(0);
        s_half<D, KST, true, (J4 + 3) % kStages>(k_addr, v_addr, q, s, xv, pbuf[J4 & 1], sm, L.rsel);
    }

    cs.km1 = cs.k0;
    cs.k0 = tile_keys(a, cs.c1);
    cs.c1 = cs.c2;
    if (is_real(a, cs.c2)) cs.c2 = next_tile(a, head, cs.c2);
}

// The loop of one wave group; iteration j runs while j <= T + 1 (T tiles).
template <int D, bool LATE, bool FAST, int DMAW>
__device__ __forceinline__ void walk(const FwdArgs& a, uint8_t* lds, int wave, int h, const Lanes& L,
                                     const v8i (&q)[Shape<D>::QK], v16f (&s)[2], v8i (&pbuf)[2],
                                     v16f (&o)[Shape<D>::DT], SoftmaxRow& sm, Cursors cs, int head) {
    // the first V-operand read of the next PV half (the PV-first waves start
    // with PV(-2): V stage 2, zeros)
    v2i xv[4];
    if constexpr (LATE) read_v_operand<D, 2>(L.v_addr, xv);
    for (;;) {
        // after iteration j the loop ends if tile j-1 was past the last tile
        bool done = cs.km1 < 0;
        iteration<D, 0, LATE, FAST, DMAW>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head, xv);
        if (done) break;
        done = cs.km1 < 0;
        iteration<D, 1, LATE, FAST, DMAW>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head, xv);
        if (done) break;
        done = cs.km1 < 0;
        iteration<D, 2, LATE, FAST, DMAW>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head, xv);
        if (done) break;
        done = cs.km1 < 0;
        iteration<D, 3, LATE, FAST, DMAW>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head, xv);
        if (done) break;
    }
    // the PV-first waves' last S half read an operand of a PV half that does
    // not run: let it land before its registers are reused
    if constexpr (LATE) lds_wait<0>(xv);
}

// Byte offset of query row `row` of KV head `head` (rows past the last are
// clamped to it) in the stacked [pcp, Hq, local_q, D] bf16 Q and output.
template <int D>
__device__ __forceinline__ int64_t query_row_offset(const FwdArgs& a, int row, int head) {
    const int rowc = row < a.rows_per_head ? row : a.rows_per_head - 1;
    const int rank = rowc / a.group_rows;
    const int rem = rowc - rank * a.group_rows;
    const int head_in_group = rem / a.local_q;
    const int tok = rem - head_in_group * a.local_q;
    return ((int64_t)(rank * a.num_q_heads + head * a.group + head_in_group) * a.local_q + tok) * D * 2;
}

// LSE: also write each row's log-sum-exp and/or list the rows of a
// precision-guarded launch whose mass is below their KV head's threshold
// (whichever of a.lse / a.guard_thr is set; a separate instantiation, so
// that the plain one keeps its register allocation).
// SPLIT: the workgroup walks only its split's share of the table entries
// and writes a normalised FP32 partial output and log-sum-exp (merged by
// merge_splits_kernel).
template <int D, bool FAST, bool LSE, bool SPLIT = false>
__global__ void __launch_bounds__(kThreads, 1) history_fwd_overlap(FwdArgs a) {
    using S = Shape<D>;
    constexpr int QK = S::QK, DT = S::DT, ROW = S::ROW, CHUNKS = S::CHUNKS;
    constexpr int DMAW = kWaves / 2;
    using P = DmaPlan<D, DMAW>;
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
    const int q_row = row_tile * kRowsPerGroup + wave * 32 + j;
    const int64_t q_off = query_row_offset<D>(a, q_row, head);
    const uint8_t* const qrow = a.q + q_off;


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
        // A DMA wave's block 0 lands at LDS byte P::block(wave) * 1024 + 16 * lane.
        const int byte = P::block(wave) * 1024 + lane * 16;
        const int drow = byte / ROW;
        const int pos = (byte % ROW) / 16;
        const int key = lds_row<true>(drow);
        L.dma_k = key * ROW + (pos ^ chunk_swizzle<true, CHUNKS>(drow)) * 16 + P::MID;
        L.dma_v = key * ROW + (pos ^ chunk_swizzle_v<true, CHUNKS>(drow)) * 16 + P::MID;
        L.rsel = ((lane ^ (lane >> 2)) & 4) ? 0 : 0x38383838;
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
        cs.km1 = tile_keys(a, before);
        cs.k0 = tile_keys(a, first);
        cs.c1 = next_tile(a, head, first);
        cs.c2 = is_real(a, cs.c1) ? next_tile(a, head, cs.c1) : cs.c1;
        // K(0), then V(0) and K(1) as if requested in iteration -1.
        if (P::issues(wave)) {
            const int wave_off = P::block(wave) * 1024;
            const uint32_t lds_u = lds_address(lds);
            load_k<S, P>(a, first, lds_u, 0, wave_off, L.dma_k);
            load_v<S, P>(a, first, lds_u, 0, wave_off, L.dma_v, true);
            load_k<S, P>(a, cs.c1, lds_u, 1, wave_off, L.dma_k);
        }
        if (wave < kWaves / 2)
            walk<D, false, FAST, DMAW>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head);
        else
            walk<D, true, FAST, DMAW>(a, lds, wave, h, L, q, s, pbuf, o, sm, cs, head);
    }

    // ---- epilogue: O = O^T / l, bf16; log-sum-exp ---------------------------
    // The row and its offset again, from an opaque lane id and opaque
    // divisors: values kept live through the walk (the row offset, the
    // reciprocals of the row maps' divisors) take registers there and spill.
    int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" : "+v"(lane_e));
    FwdArgs ag = a;
    asm volatile("" : "+s"(ag.group_rows), "+s"(ag.local_q));
    const int row = row_tile * kRowsPerGroup + wave * 32 + (lane_e & 31);
    const bool row_ok = row < a.rows_per_head;
    const int64_t row_off = query_row_offset<D>(ag, row, head);
    const float scale = sm.l > 0.f ? a.v_scale / sm.l : 0.f;
    // sum_k exp(score_k) = l * 2^(m - 6), less the average overestimate of
    // the linear-mantissa exp2
    const float lse =
        sm.l > 0.f ? __logf(sm.l) + (sm.m - kPBiasLog2) * kLn2 - (FAST ? kFastLseBias : 0.f) : -INFINITY;
    if constexpr (SPLIT) {
        if (row_ok) {
            const int64_t prow = (int64_t)split * a.rows_per_head * a.num_kv_heads + row_off / (D * 2);
            // fp16 partials of O / l, before the v_scale factor (the merge
            // applies it): a weighted mean of e4m3 V codes, |O / l| <= 448
            // whatever v_scale is, so fp16 keeps its relative precision;
            // half the bytes of fp32 for this kernel to write and the merge
            // to read
            const float inv_l = sm.l > 0.f ? 1.f / sm.l : 0.f;
            _Float16* const po = (_Float16*)a.part_o + prow * D;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int d = 32 * dt + 8 * r4 + 4 * h;
                    uint32_t w[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const _Float16 x0 = (_Float16)(o[dt][4 * r4 + 2 * i] * inv_l);
                        const _Float16 x1 = (_Float16)(o[dt][4 * r4 + 2 * i + 1] * inv_l);
                        w[i] = (uint32_t)__builtin_bit_cast(uint16_t, x0) |
                               ((uint32_t)__builtin_bit_cast(uint16_t, x1) << 16);
                    }
                    *(v2i*)(po + d) = v2i{(int)w[0], (int)w[1]};
                }
            if (h == 0) {
                a.part_lse[prow] = lse;
                if (a.part_m) a.part_m[prow] = sm.m;
            }
        }
        return;
    }
    if constexpr (LSE) {
        if (a.lse && row_ok && h == 0) a.lse[row_off / (D * 2)] = lse;
        // precision guard: l / 2^6 is the row's probability mass sum_k 2^(x_k - m)
        if (a.guard_thr) {
            const float thr = guard_threshold(a.guard_thr, head, D / 16);
            if (row_ok && h == 0 && sm.l * (1.f / 64.f) < thr)
                guard_append(a.guard_rows, a.num_kv_heads, a.rows_per_head, head, row);
        }
    }
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
// consecutive d).  out = part_scale * sum_s w_s O_s / sum_s w_s with w_s =
// e^(lse_s - max), bf16 (part_scale: v_scale for the fp16 partials of the
// e4m3 overlap kernel, which hold O / l before it; else 1); lse (optional)
// = max + ln(sum_s w_s).  HBM bound: 4 * D + 4 bytes
// (2 * D + 4 with fp16 partials) read per row and split, 2 * D written.
// Precision guard (guard_plan set): the row's probability mass against the
// largest range reference m_ref = max_s part_m, sum_s l_s 2^(m_s - m_ref) / 2^6
// = e^(lse + lse_bias - m_ref ln 2) (lse_bias: what the kernel subtracted
// from its log-sum-exps); a row below its KV head's threshold (the largest
// of the head's D / 16 values in guard_thr, from guard_vstats_kernel, which
// also zeroed the plan's counts) is appended to the guard plan.
// NS > 0: exactly NS splits, every load (the guard's inputs, each split's
// log-sum-exp and partial) issued before the first use, one round trip to
// memory instead of three (2-split 16-rank workload: 0.1761 against 0.1792
// ms per call; 8-split 4-rank BF16 workload: 0.0124 against 0.0137 ms);
// NS == 0: any count.
template <int NS>
__global__ void __launch_bounds__(256) merge_splits_kernel(const float* part_o, int part_f16, float part_scale,
                                                           const float* part_lse, int splits, int64_t rows, int d_vec8, uint8_t* out,
                                                           float* lse_out,
                                                           const float* part_m, int32_t* guard_plan, GuardShape g,
                                                           float lse_bias, const float* guard_thr) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * d_vec8) return;
    const int64_t row = idx / d_vec8;
    const int d0 = (int)(idx - row * d_vec8) * 8;
    const int D = d_vec8 * 8;
    if constexpr (NS > 0) splits = NS;
    // the guard's inputs first, so that their loads overlap the partials'
    const bool guard_lane = guard_plan && d0 == 0;
    int head = 0, head_row = 0;
    float thr = 0.f, m_ref = -INFINITY;
    if (guard_lane) {
        head_row = guard_head_row(g, row, head);
        thr = guard_threshold(guard_thr, head, d_vec8 / 2);
#pragma unroll 8
        for (int sp = 0; sp < splits; ++sp) m_ref = fmaxf(m_ref, part_m[sp * rows + row]);
    }
    constexpr int KEEP = NS > 0 ? NS : 1;
    float lk[KEEP];
    v4i raw[KEEP][2];
    float mx = -INFINITY;
    if constexpr (NS > 0) {
#pragma unroll
        for (int sp = 0; sp < NS; ++sp) {
            lk[sp] = part_lse[sp * rows + row];
            if (part_f16) {
                raw[sp][0] = *(const v4i*)((const _Float16*)part_o + (sp * rows + row) * D + d0);
            } else {
                const float* const src = part_o + (sp * rows + row) * D + d0;
                raw[sp][0] = *(const v4i*)src;
                raw[sp][1] = *(const v4i*)(src + 4);
            }
        }
#pragma unroll
        for (int sp = 0; sp < NS; ++sp) mx = fmaxf(mx, lk[sp]);
    } else {
#pragma unroll 8
        for (int sp = 0; sp < splits; ++sp) mx = fmaxf(mx, part_lse[sp * rows + row]);
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float wsum = 0.f;
    auto accumulate = [&](float l, const v4i (&r)[2]) {
        const float w = l == -INFINITY ? 0.f : __expf(l - mx);
        wsum += w;
        float x[8];
        if (part_f16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)((uint32_t)r[0][i] & 0xffffu));
                x[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)((uint32_t)r[0][i] >> 16));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = __int_as_float(r[0][i]);
                x[4 + i] = __int_as_float(r[1][i]);
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = fmaf(w, x[i], acc[i]);
    };
    if constexpr (NS > 0) {
#pragma unroll
        for (int sp = 0; sp < NS; ++sp) accumulate(lk[sp], raw[sp]);
    } else {
#pragma unroll 4
        for (int sp = 0; sp < splits; ++sp) {
            v4i r[2];
            if (part_f16) {
                r[0] = *(const v4i*)((const _Float16*)part_o + (sp * rows + row) * D + d0);
            } else {
                const float* const src = part_o + (sp * rows + row) * D + d0;
                r[0] = *(const v4i*)src;
                r[1] = *(const v4i*)(src + 4);
            }
            accumulate(part_lse[sp * rows + row], r);
        }
    }
    const float inv = wsum > 0.f ? part_scale / wsum : 0.f;
    uint32_t wv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const __bf16 x0 = (__bf16)(acc[2 * i] * inv), x1 = (__bf16)(acc[2 * i + 1] * inv);
        wv[i] = (uint32_t)__builtin_bit_cast(uint16_t, x0) | ((uint32_t)__builtin_bit_cast(uint16_t, x1) << 16);
    }
    *(v4i*)(out + (row * D + d0) * 2) = v4i{(int)wv[0], (int)wv[1], (int)wv[2], (int)wv[3]};
    const float lse = wsum > 0.f ? mx + __logf(wsum) : -INFINITY;
    if (lse_out && d0 == 0) lse_out[row] = lse;
    if (guard_lane) {
        const float mass = wsum > 0.f ? __expf(lse + lse_bias - m_ref * kLn2) : 0.f;
        if (mass < thr) guard_append(guard_plan, g.num_kv_heads, g.rows_per_head, head, head_row);
    }
}

}  // namespace pcpa

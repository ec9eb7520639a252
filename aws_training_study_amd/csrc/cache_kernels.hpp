// KV-cache producer kernels (quantise + page write, absolute maximum).
#pragma once

#include "common.hpp"

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
    const int32_t* block_table;  // int32 entries, or int64 ones as dword pairs (table_shift 1)
    int32_t table_shift;
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
    float k_rcp, v_rcp;  // RN(1 / scale), for div_rn when fast_div
    int32_t fast_div;    // both scales in [2^-80, 2^126]: div_rn instead of the IEEE division
};

// x / d rounded to nearest even, as the IEEE division rounds it, from y =
// RN(1 / d) by Markstein's correction (P. Markstein, IBM J. Res. Develop.
// 34(1), 1990, 111-119): q0 = RN(x y) is within an ulp of
// x / d, the remainder x - d q0 is exact (one FMA), and RN(q0 + r y) is
// RN(x / d).  Three instructions and a sign copy where the IEEE sequence
// takes ten.  Compared with exact quotients for bf16 x with |x| and
// |x / d| >= 2^-100 and d from 2^-80 to 2^126; below that the quotient
// rounds to an e4m3 zero either way, and zeros, infinities, NaNs and
// overflowing quotients give a NaN or a signed zero here where the IEEE
// quotient is an infinity, a NaN or a signed zero: the same e4m3 code (the
// NaN code or zero with x's sign, which copysign keeps).
__device__ __forceinline__ float div_rn(float x, float d, float y) {
    const float q0 = x * y;
    const float r = fmaf(-d, q0, x);
    return copysignf(fmaf(r, y, q0), x);
}

// e4m3 codes of four values (round to nearest even; magnitudes above 464
// and infinities become the NaN code 0x7f with the value's sign, like
// torch's float8_e4m3fn cast).  v_cvt_pk_fp8_f32 gives these codes except
// that it writes 0xff for every NaN; every other code's sign bit is already
// the value's, so each code's bit 7 is set from its value's sign bit (byte 3
// of the float, gathered by two byte permutes).
__device__ __forceinline__ uint32_t e4m3_codes4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    const uint32_t lo = __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x0c0c0703u);
    const uint32_t hi = __builtin_amdgcn_perm(__float_as_uint(d), __float_as_uint(c), 0x07030c0cu);
    return ((uint32_t)w & 0x7f7f7f7fu) | ((lo | hi) & 0x80808080u);
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
    const int32_t page = table_page(a.block_table, entry, a.table_shift);
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
            kf[2 * w] = bf16_bits_to_f32((uint32_t)kin[w] & 0xffffu);
            kf[2 * w + 1] = bf16_bits_to_f32((uint32_t)kin[w] >> 16);
            vf[2 * w] = bf16_bits_to_f32((uint32_t)vin[w] & 0xffffu);
            vf[2 * w + 1] = bf16_bits_to_f32((uint32_t)vin[w] >> 16);
        }
        // x / scale rounded as torch's (x / scale).to(float8) rounds it
        if (a.fast_div) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                kf[i] = div_rn(kf[i], a.k_scale, a.k_rcp);
                vf[i] = div_rn(vf[i], a.v_scale, a.v_rcp);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                kf[i] = kf[i] / a.k_scale;
                vf[i] = vf[i] / a.v_scale;
            }
        }
        // streaming (non-temporal) stores: the pool is written once and read
        // by later launches, so its lines need not stay in this launch's L2
        // (full-fp8 history: 73 -> 59 us with the division above)
        __builtin_nontemporal_store(
            v2i{(int)e4m3_codes4(kf[0], kf[1], kf[2], kf[3]), (int)e4m3_codes4(kf[4], kf[5], kf[6], kf[7])},
            (v2i*)dst);
        __builtin_nontemporal_store(
            v2i{(int)e4m3_codes4(vf[0], vf[1], vf[2], vf[3]), (int)e4m3_codes4(vf[4], vf[5], vf[6], vf[7])},
            (v2i*)(dst + a.v_offset));
    } else {
        __builtin_nontemporal_store(kin, (v4i*)dst);
        __builtin_nontemporal_store(vin, (v4i*)(dst + a.v_offset));
    }
}

// max |x| over n bf16 values into *out (as the bits of a non-negative float,
// ordered like unsigned integers); *out is cleared first by init_kernel.
__global__ void absmax_init_kernel(uint32_t* out) { *out = 0u; }

// |x| of the two bf16 values of a dword, as their 15-bit magnitude patterns.
// Non-negative IEEE values order like their bit patterns, and every NaN
// pattern (exponent all ones, mantissa non-zero) lies above infinity's, so an
// integer maximum of magnitudes is the float maximum with NaN propagated, as
// torch's x.abs().max() computes it.
__device__ __forceinline__ uint32_t abs_bits_max(uint32_t m, uint32_t word) {
    return max(m, max(word & 0x7fffu, (word >> 16) & 0x7fffu));
}

// Workgroup b reduces the contiguous span [b * span, (b + 1) * span) with
// four 16-byte loads in flight per thread, then one atomic per workgroup.
__global__ void __launch_bounds__(kThreads) absmax_kernel(const uint16_t* x, int64_t n, int64_t span,
                                                          uint32_t* out) {
    constexpr int kVec = 8, kUnroll = 4, kStep = kThreads * kVec;
    __shared__ uint32_t partial[kThreads / 64];
    const int64_t begin = (int64_t)blockIdx.x * span;
    const int64_t end = begin + span < n ? begin + span : n;
    uint32_t m[kUnroll] = {0u, 0u, 0u, 0u};
    int64_t i = begin + threadIdx.x * kVec;
    for (; i + (kUnroll - 1) * kStep + kVec <= end; i += kUnroll * kStep) {
        v4i raw[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) raw[u] = *(const v4i*)(x + i + u * kStep);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
#pragma unroll
            for (int w = 0; w < 4; ++w) m[u] = abs_bits_max(m[u], (uint32_t)raw[u][w]);
    }
    for (; i < end; i += kStep) {
        if (i + kVec <= end) {
            const v4i raw = *(const v4i*)(x + i);
#pragma unroll
            for (int w = 0; w < 4; ++w) m[0] = abs_bits_max(m[0], (uint32_t)raw[w]);
        } else {
            for (int64_t e = i; e < end; ++e) m[0] = abs_bits_max(m[0], (uint32_t)x[e]);
        }
    }
    uint32_t r = max(max(m[0], m[1]), max(m[2], m[3]));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) r = max(r, (uint32_t)__shfl_xor((int)r, off));
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = r;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / 64; ++w) r = max(r, partial[w]);
        atomicMax(out, r << 16);  // the float bits of the bf16 magnitude
    }
}

}  // namespace cache
}  // namespace pcpa

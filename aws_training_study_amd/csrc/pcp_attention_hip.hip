// History-only PCP attention for MI355X (gfx950): kernels and C ABI.
//
// One launch computes, for every logical PCP rank, the attention of that
// rank's current-token Q over the whole paged history (all ranks' cache
// blocks), which the Trainium2 proof of concept computed with a device ring
// (pcp_attention/kernel.py:84-554).  The ring order only changes the order of
// online-softmax updates; here every query row walks the block table in
// table order.
//
// Two attention kernels share the data layout and operand maps (common.hpp):
//   * history_fwd_kernel<D, STORE8, FP8, CAUSAL> (tile_kernel.hpp): 4 waves x
//     32 rows per workgroup, two workgroups per CU (one for bf16 MFMAs at
//     head_dim 256), double-buffered tiles; every head
//     dim (64, 128, 256) and precision (e4m3 or bf16 MFMAs) other than e4m3
//     at 256; with CAUSAL, the current tokens' causal step and its
//     log-sum-exp merge.
//   * ovl::history_fwd_overlap<256, FAST, LSE, SPLIT> (overlap_kernel.hpp):
//     the e4m3-MFMA path at head_dim 256, 8 waves x 32 rows, a two-stage
//     in-wave pipeline with the two waves of a SIMD staggered by half a tile
//     step; SPLIT walks one range of the table and writes a partial result
//     for merge_splits_kernel.
// cache_kernels.hpp holds the KV-cache producer.
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
//
// This file holds the C ABI (include/pcp_attention_hip.h).
#include "cache_kernels.hpp"
#include "common.hpp"
#include "overlap_kernel.hpp"
#include "tile_kernel.hpp"

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
    // (e4m3 MFMAs at head_dim 256 took the overlap kernel above)
    switch (p->head_dim * 4 + (store8 ? 2 : 0) + (fp8 ? 1 : 0)) {
        case 64 * 4 + 3: fn = (const void*)pcpa::history_fwd_kernel<64, true, true>; break;
        case 128 * 4 + 3: fn = (const void*)pcpa::history_fwd_kernel<128, true, true>; break;
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
    const bool store8 = p->kv_dtype == PCPA_DTYPE_FP8_E4M3FN;
    const bool fp8 = store8 && !(p->flags & PCPA_FLAG_BF16_MFMA);
    const bool overlap = fp8 && p->head_dim == 256;
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
    const int rows_per_group = overlap ? pcpa::ovl::kRowsPerGroup : pcpa::kRowsPerGroup;
    a.row_tiles = (a.rows_per_head + rows_per_group - 1) / rows_per_group;
    a.splits = splits;
    const int64_t rows = (int64_t)p->pcp_size * p->num_q_heads * p->local_q_len;
    a.part_o = (float*)workspace;
    a.part_lse = a.part_o + (int64_t)splits * rows * p->head_dim;

    void* args[] = {&a};
    const void* fn = nullptr;
    if (overlap) {
        fn = (p->flags & PCPA_FLAG_EXACT_EXP2) ? (const void*)pcpa::ovl::history_fwd_overlap<256, false, false, true>
                                               : (const void*)pcpa::ovl::history_fwd_overlap<256, true, false, true>;
    } else {
        switch (p->head_dim * 4 + (store8 ? 2 : 0) + (fp8 ? 1 : 0)) {
            case 64 * 4 + 3: fn = (const void*)pcpa::history_fwd_kernel<64, true, true, false, true>; break;
            case 128 * 4 + 3: fn = (const void*)pcpa::history_fwd_kernel<128, true, true, false, true>; break;
            case 64 * 4 + 2: fn = (const void*)pcpa::history_fwd_kernel<64, true, false, false, true>; break;
            case 128 * 4 + 2: fn = (const void*)pcpa::history_fwd_kernel<128, true, false, false, true>; break;
            case 256 * 4 + 2: fn = (const void*)pcpa::history_fwd_kernel<256, true, false, false, true>; break;
            case 64 * 4: fn = (const void*)pcpa::history_fwd_kernel<64, false, false, false, true>; break;
            case 128 * 4: fn = (const void*)pcpa::history_fwd_kernel<128, false, false, false, true>; break;
            case 256 * 4: fn = (const void*)pcpa::history_fwd_kernel<256, false, false, false, true>; break;
            default: return PCPA_ERR_UNSUPPORTED;
        }
    }
    const int items = a.row_tiles * p->num_kv_heads * splits;
    hipError_t err = hipLaunchKernel(fn, dim3(8 * ((items + 7) / 8)),
                                     dim3(overlap ? pcpa::ovl::kThreads : pcpa::kThreads), args, 0,
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
    // at least 32 KB each, at most 256 workgroups (one per CU: a 134 MB
    // tensor then reads at 5.8 TB/s, against 3.7 TB/s with 2048 workgroups)
    constexpr int64_t kMinSpan = 16384;
    int64_t span = (n + 255) / 256;
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

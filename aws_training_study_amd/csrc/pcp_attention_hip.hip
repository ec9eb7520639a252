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
//     32 rows per workgroup, two workgroups per CU (bf16 MFMAs at head_dim
//     256: 8 waves in key-split pairs, one workgroup), double-buffered
//     tiles; every head
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
#include "guard_kernels.hpp"
#include "overlap_kernel.hpp"
#include "paging_kernels.hpp"
#include "tile_kernel.hpp"

#include <mutex>

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

// Workspace of a history launch: split partials (outputs, log-sum-exps and
// reference maxima of every range) and, for the precision guard, the
// per-chunk thresholds, the fixup plan and the fixup's range partials.
struct WorkspaceLayout {
    int64_t part_o, part_lse, part_m, thr, plan, gpart_o, gpart_lse, bytes;
    int32_t groups_total;  // 128-row groups the plan can list
    int32_t max_ranges;    // history ranges a sparse fixup group is cut into at most
    int32_t partial_rows;  // rows the fixup's range partials hold
};

// A launch runs e4m3 MFMAs on an e4m3 cache unless PCPA_FLAG_BF16_MFMA.
inline bool e4m3_mfma(const pcpa_params* p) {
    return p->kv_dtype == PCPA_DTYPE_FP8_E4M3FN && !(p->flags & PCPA_FLAG_BF16_MFMA);
}
// The precision guard runs on every e4m3-MFMA launch but an explicitly
// unguarded one.
inline bool guarded(const pcpa_params* p) { return e4m3_mfma(p) && !(p->flags & PCPA_FLAG_E4M3_UNGUARDED); }
// Split partials of the e4m3 overlap kernel (head_dim 256) are FP16 values of
// O / l, before the v_scale factor (|O / l| <= 448, the largest e4m3 V code,
// whatever v_scale is); the merge applies v_scale.  Other kernels: FP32.
inline bool f16_partials(const pcpa_params* p) { return e4m3_mfma(p) && p->head_dim == 256; }

inline int64_t align16(int64_t x) { return (x + 15) / 16 * 16; }

inline WorkspaceLayout workspace_layout(const pcpa_params* p, int splits) {
    const int64_t rows = (int64_t)p->pcp_size * p->num_q_heads * p->local_q_len;
    WorkspaceLayout w{};
    if (splits > 1) {
        w.part_o = 0;
        w.part_lse = align16(w.part_o + (int64_t)splits * rows * p->head_dim * (f16_partials(p) ? 2 : 4));
        w.part_m = w.part_lse + (int64_t)splits * rows * 4;
        w.bytes = w.part_m + (int64_t)splits * rows * 4;
    }
    if (guarded(p)) {
        // fixup: the flagged rows gathered into groups of 128 (at most as
        // many groups as 128-row tiles); a sparse group's history walk is
        // cut into ranges of at least 2 key tiles (128 keys), 64 ranges at
        // most, so that a few flagged rows cost a short walk rather than a
        // whole history's; the partials hold kGuardPartialRows rows, which
        // guard_ranges() shares among the groups listed
        const int64_t entries = (int64_t)p->pcp_size * p->max_local_blocks;
        const int64_t key_tiles = entries * (p->block_size / kKeyTile);
        const int64_t rows_per_head = rows / p->num_q_heads * (p->num_q_heads / p->num_kv_heads);
        w.groups_total = (int32_t)((rows_per_head + kRowsPerGroup - 1) / kRowsPerGroup * p->num_kv_heads);
        constexpr int64_t kMaxRanges = 64;
        static_assert(kMaxRanges <= kGuardMergePer * (kGuardMergeThreads / (256 / 8)),
                      "guard_merge_kernel's threads hold every range at head_dim 256");
        int64_t mr = key_tiles / 2;
        mr = mr < 1 ? 1 : mr > kMaxRanges ? kMaxRanges : mr;
        w.max_ranges = (int32_t)mr;
        int64_t prows = mr >= 2 ? (int64_t)w.groups_total * kRowsPerGroup * mr : 0;
        prows = prows < kGuardPartialRows ? prows : kGuardPartialRows;
        w.partial_rows = (int32_t)prows;
        w.thr = align16(w.bytes);
        w.plan = align16(w.thr + (int64_t)p->num_kv_heads * (p->head_dim / 16) * 4);
        w.gpart_o = align16(w.plan + ((int64_t)guard_list_offset(p->num_kv_heads) +
                                      (int64_t)w.groups_total * kRowsPerGroup) * 4);
        w.gpart_lse = w.gpart_o + prows * p->head_dim * 4;
        w.bytes = w.gpart_lse + prows * 4;
    }
    return w;
}

// Arguments of the history kernels for one launch (everything but the
// split and guard fields).
inline FwdArgs history_args(const pcpa_params* p, const void* q, const void* kv_pages, const void* block_table,
                            const int32_t* page_valid_len, void* out, float* lse) {
    const bool store8 = p->kv_dtype == PCPA_DTYPE_FP8_E4M3FN;
    const int64_t es = store8 ? 1 : 2;
    FwdArgs a = common_args(p, q, out);
    a.kv = (const uint8_t*)kv_pages;
    a.block_table = (const int32_t*)block_table;
    a.page_valid_len = page_valid_len;
    a.head_stride = (int64_t)p->block_size * p->head_dim * es;
    a.page_stride = 2 * (int64_t)p->num_kv_heads * a.head_stride;
    a.num_entries = p->pcp_size * p->max_local_blocks;
    a.table_shift = (p->flags & PCPA_FLAG_TABLE_INT64) ? 1 : 0;
    a.num_pages = p->num_pages;
    a.block_size = p->block_size;
    a.score_scale = p->softmax_scale * p->k_scale * kLog2e;
    a.v_scale = p->v_scale;
    a.lse = lse;
    return a;
}

// The tile kernel instantiation for (head_dim, cache dtype, MFMA precision).
template <bool SPLIT>
inline const void* tile_kernel_for(int head_dim, bool store8, bool fp8) {
    switch (head_dim * 4 + (store8 ? 2 : 0) + (fp8 ? 1 : 0)) {
        case 64 * 4 + 3: return (const void*)history_fwd_kernel<64, true, true, false, SPLIT>;
        case 128 * 4 + 3: return (const void*)history_fwd_kernel<128, true, true, false, SPLIT>;
        case 64 * 4 + 2: return (const void*)history_fwd_kernel<64, true, false, false, SPLIT>;
        case 128 * 4 + 2: return (const void*)history_fwd_kernel<128, true, false, false, SPLIT>;
        case 256 * 4 + 2: return (const void*)history_fwd_kernel<256, true, false, false, SPLIT>;
        case 64 * 4: return (const void*)history_fwd_kernel<64, false, false, false, SPLIT>;
        case 128 * 4: return (const void*)history_fwd_kernel<128, false, false, false, SPLIT>;
        case 256 * 4: return (const void*)history_fwd_kernel<256, false, false, false, SPLIT>;
        default: return nullptr;  // e4m3 MFMAs at head_dim 256 run the overlap kernel
    }
}

// Device memory of the guard scratch (see guard_scratch below), held for
// one call: acquire() makes `stream` wait for the previous call's use of this
// GPU's scratch; the destructor records this call's end for the next one.
// Neither is recorded on a stream under graph capture.
struct GuardLease {
    void* ptr = nullptr;
    int dev = -1;
    bool capturing = false;
    hipStream_t stream = nullptr;
    int32_t acquire(hipStream_t s);
    ~GuardLease();
};

// One history attention call: `splits` ranges of table entries (1: one
// pass), then, for a precision-guarded launch on e4m3 MFMAs, the BF16-MFMA
// pass over the workgroups whose rows the e4m3 pass flagged.  With a lease
// and no workspace, the workspace is the library's guard scratch, taken
// after every argument check.
inline int32_t history_launch(const pcpa_params* p, int splits, const void* q, const void* kv_pages,
                              const void* block_table, const int32_t* page_valid_len, void* out, float* lse,
                              void* workspace, int64_t workspace_bytes, hipStream_t stream,
                              GuardLease* lease = nullptr) {
    const int32_t st = pcpa_check_params(p);
    if (st != PCPA_OK) return st;
    if (splits < 1 || splits > PCPA_MAX_SPLITS) return PCPA_ERR_BAD_SHAPE;
    if (!q || !kv_pages || !block_table || !page_valid_len || !out) return PCPA_ERR_NULL_POINTER;
    if (((uintptr_t)q | (uintptr_t)kv_pages | (uintptr_t)out | (uintptr_t)workspace) & 15u)
        return PCPA_ERR_MISALIGNED;
    if (((uintptr_t)block_table | (uintptr_t)page_valid_len | (uintptr_t)lse) & 3u) return PCPA_ERR_MISALIGNED;
    if ((p->flags & PCPA_FLAG_TABLE_INT64) && ((uintptr_t)block_table & 7u)) return PCPA_ERR_MISALIGNED;
    const bool store8 = p->kv_dtype == PCPA_DTYPE_FP8_E4M3FN;
    const bool fp8 = e4m3_mfma(p);
    const bool overlap = fp8 && p->head_dim == 256;
    const bool guard = guarded(p);
    if (guard && p->num_kv_heads > kGuardMaxHeads) return PCPA_ERR_UNSUPPORTED;
    const WorkspaceLayout w = workspace_layout(p, splits);
    if (w.bytes > 0 && !workspace && lease) {
        if (w.bytes > PCPA_GUARD_SCRATCH_BYTES) return PCPA_ERR_SCRATCH;
        const int32_t ls = lease->acquire(stream);
        if (ls != PCPA_OK) return ls;
        workspace = lease->ptr;
        workspace_bytes = PCPA_GUARD_SCRATCH_BYTES;
    }
    if (w.bytes > 0 && (!workspace || workspace_bytes < w.bytes)) return PCPA_ERR_WORKSPACE;
    uint8_t* const ws = (uint8_t*)workspace;
    int32_t* const plan = guard ? (int32_t*)(ws + w.plan) : nullptr;
    float* const thr = guard ? (float*)(ws + w.thr) : nullptr;
    const bool fast = !(p->flags & PCPA_FLAG_EXACT_EXP2);

    FwdArgs a = history_args(p, q, kv_pages, block_table, page_valid_len, out, lse);
    if (guard) {
        // first the V statistics of the walk: each KV head's threshold (per
        // 16-channel chunk), and the guard plan's row counts set to zero
        VStatsArgs v{};
        v.kv = a.kv;
        v.block_table = a.block_table;
        v.page_valid_len = a.page_valid_len;
        v.page_stride = a.page_stride;
        v.head_stride = a.head_stride;
        v.num_entries = a.num_entries;
        v.table_shift = a.table_shift;
        v.num_pages = a.num_pages;
        v.block_size = a.block_size;
        v.num_kv_heads = a.num_kv_heads;
        v.thr = thr;
        v.plan = plan;
        v.scale = PCPA_GUARD_MIN_MASS * p->v_scale * p->v_scale / 262144.f;
        const void* vfn = p->head_dim == 64    ? (const void*)guard_vstats_kernel<64>
                          : p->head_dim == 128 ? (const void*)guard_vstats_kernel<128>
                                               : (const void*)guard_vstats_kernel<256>;
        void* vargs[] = {&v};
        const int chunks = p->num_kv_heads * (p->head_dim / 16);
        if (hipLaunchKernel(vfn, dim3(8 * ((chunks + 7) / 8)), dim3(kVStatsThreads), vargs, 0, stream) != hipSuccess)
            return PCPA_ERR_LAUNCH;
    }
    const int rows_per_group = overlap ? ovl::kRowsPerGroup : kRowsPerGroup;
    a.row_tiles = (a.rows_per_head + rows_per_group - 1) / rows_per_group;
    const void* fn = nullptr;
    if (splits == 1) {
        // a guarded pass lists its rows below the threshold itself
        a.guard_thr = thr;
        a.guard_rows = plan;
        if (overlap) {
            // the log-sum-exp instantiation also lists the guard's rows
            const bool aux = lse || guard;
            fn = fast ? (aux ? (const void*)ovl::history_fwd_overlap<256, true, true>
                             : (const void*)ovl::history_fwd_overlap<256, true, false>)
                      : (aux ? (const void*)ovl::history_fwd_overlap<256, false, true>
                             : (const void*)ovl::history_fwd_overlap<256, false, false>);
        } else {
            fn = tile_kernel_for<false>(p->head_dim, store8, fp8);
        }
    } else {
        a.splits = splits;
        a.part_o = (float*)(ws + w.part_o);
        a.part_f16 = f16_partials(p) ? 1 : 0;
        a.part_lse = (float*)(ws + w.part_lse);
        a.part_m = guard ? (float*)(ws + w.part_m) : nullptr;
        if (overlap)
            fn = fast ? (const void*)ovl::history_fwd_overlap<256, true, false, true>
                      : (const void*)ovl::history_fwd_overlap<256, false, false, true>;
        else
            fn = tile_kernel_for<true>(p->head_dim, store8, fp8);
    }
    if (!fn) return PCPA_ERR_UNSUPPORTED;
    void* args[] = {&a};
    const int items = a.row_tiles * p->num_kv_heads * splits;
    const int threads = overlap ? ovl::kThreads : tile_threads(p->head_dim, fp8);
    if (hipLaunchKernel(fn, dim3(8 * ((items + 7) / 8)), dim3(threads), args, 0, stream) != hipSuccess)
        return PCPA_ERR_LAUNCH;
    GuardShape g{};
    g.rows_total = (int64_t)p->pcp_size * p->num_q_heads * p->local_q_len;
    g.rows_per_head = a.rows_per_head;
    g.group_rows = a.group_rows;
    g.local_q = a.local_q;
    g.num_q_heads = a.num_q_heads;
    g.num_kv_heads = a.num_kv_heads;
    g.group = a.group;
    g.partial_rows = w.partial_rows;
    g.max_ranges = w.max_ranges;
    if (splits > 1) {
        // the merge also lists the guard's rows
        const int d_vec8 = p->head_dim / 8;
        const int64_t threads = g.rows_total * d_vec8;
        auto merge = splits == 2 ? merge_splits_kernel<2> : splits == 3 ? merge_splits_kernel<3>
                   : splits == 4 ? merge_splits_kernel<4> : splits == 8 ? merge_splits_kernel<8>
                   : merge_splits_kernel<0>;
        hipLaunchKernelGGL(merge, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                           (const float*)a.part_o, a.part_f16, a.part_f16 ? p->v_scale : 1.f,
                           (const float*)a.part_lse, splits, g.rows_total, d_vec8,
                           (uint8_t*)out, lse, (const float*)a.part_m, plan, g, overlap && fast ? kFastLseBias : 0.f,
                           (const float*)thr);
        if (hipGetLastError() != hipSuccess) return PCPA_ERR_LAUNCH;
    }
    if (guard) {
        // the BF16 fixup of the listed rows' 128-row groups (BF16 MFMAs over
        // the exactly widened cache), then the merge of its ranges
        FwdArgs b = history_args(p, q, kv_pages, block_table, page_valid_len, out, lse);
        b.row_tiles = (a.rows_per_head + kRowsPerGroup - 1) / kRowsPerGroup;
        b.guard_plan = plan;
        b.splits = w.max_ranges;
        b.guard_partial_rows = w.partial_rows;
        b.part_o = (float*)(ws + w.gpart_o);
        b.part_lse = (float*)(ws + w.gpart_lse);
        void* bargs[] = {&b};
        const int sparse_items = w.partial_rows / kRowsPerGroup;  // groups x ranges at most
        const int grid = sparse_items > w.groups_total ? sparse_items : w.groups_total;
        const void* fix = nullptr;
        switch (p->head_dim) {
            case 64: fix = (const void*)history_fwd_kernel<64, true, false, false, false, true>; break;
            case 128: fix = (const void*)history_fwd_kernel<128, true, false, false, false, true>; break;
            case 256: fix = (const void*)history_fwd_kernel<256, true, false, false, false, true>; break;
            default: return PCPA_ERR_UNSUPPORTED;
        }
        if (hipLaunchKernel(fix, dim3(grid), dim3(tile_threads(p->head_dim, false)), bargs, 0, stream) != hipSuccess)
            return PCPA_ERR_LAUNCH;
        if (w.partial_rows > 0) {
            hipLaunchKernelGGL(guard_merge_kernel, dim3(kGuardMergeGroups), dim3(kGuardMergeThreads), 0, stream,
                               (const float*)b.part_o, (const float*)b.part_lse, (const int32_t*)plan, g,
                               p->head_dim / 8, (uint8_t*)out, lse);
            if (hipGetLastError() != hipSuccess) return PCPA_ERR_LAUNCH;
        }
    }
    return PCPA_OK;
}

// Scratch of pcpa_history_attention_noalloc: the split partials and guard
// buffers of a launch, in device memory the library owns instead of a
// caller workspace.  One copy per GPU, held until the process ends; every
// call on a GPU shares it (calls that overlap on one GPU race).
static __device__ __align__(256) uint8_t scratch[PCPA_NOALLOC_SCRATCH_BYTES];

// Device address of `scratch` on each GPU (the array's name is a host-side
// stand-in, not a device address), looked up once per device with that
// device current.
constexpr int kMaxDevices = 64;
static void* scratch_ptr[kMaxDevices];
static std::mutex scratch_mutex;

inline int32_t scratch_for_current_device(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return PCPA_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_ptr[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return PCPA_ERR_LAUNCH;
        scratch_ptr[dev] = ptr;
    }
    *out = scratch_ptr[dev];
    return PCPA_OK;
}

// Guard scratch of pcpa_history_attention / _lse: the precision guard's
// flags, row lists and partials of a call that brings no workspace.  One
// copy per GPU, held until the process ends.  Calls are ordered through it
// per GPU: each waits (on the GPU) for the previous call's last kernel.
static __device__ __align__(256) uint8_t guard_scratch[PCPA_GUARD_SCRATCH_BYTES];

struct GuardScratchState {
    std::mutex mutex;     // held from acquire() to the end of the call's launches
    void* ptr = nullptr;  // device address of guard_scratch on this GPU
    hipEvent_t done{};    // the end of the last call that used it
    bool recorded = false;
};
static GuardScratchState guard_state[kMaxDevices];

int32_t GuardLease::acquire(hipStream_t s) {
    int d = -1;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= kMaxDevices) return PCPA_ERR_LAUNCH;
    GuardScratchState& g = guard_state[d];
    g.mutex.lock();
    dev = d;
    stream = s;
    if (!g.ptr) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(guard_scratch)) != hipSuccess || !ptr) return PCPA_ERR_LAUNCH;
        if (hipEventCreateWithFlags(&g.done, hipEventDisableTiming) != hipSuccess) return PCPA_ERR_LAUNCH;
        g.ptr = ptr;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) return PCPA_ERR_LAUNCH;
    capturing = cs != hipStreamCaptureStatusNone;
    if (!capturing && g.recorded && hipStreamWaitEvent(s, g.done, 0) != hipSuccess) return PCPA_ERR_LAUNCH;
    ptr = g.ptr;
    return PCPA_OK;
}

GuardLease::~GuardLease() {
    if (dev < 0) return;
    GuardScratchState& g = guard_state[dev];
    // recorded even after a failed launch: the kernels queued before it
    // still use the scratch
    if (ptr && !capturing && hipEventRecord(g.done, stream) == hipSuccess) g.recorded = true;
    g.mutex.unlock();
}

// pcpa_history_attention / _lse: a guarded launch takes the guard scratch,
// or runs every row on BF16 MFMAs (the guard's own precision) when its
// guard buffers do not fit the scratch.
inline int32_t history_one_pass(const pcpa_params* p, const void* q, const void* kv_pages, const void* block_table,
                                const int32_t* page_valid_len, void* out, float* lse, hipStream_t stream) {
    if (p && p->abi_version == PCPA_ABI_VERSION && pcpa_check_params(p) == PCPA_OK && guarded(p) &&
        workspace_layout(p, 1).bytes > PCPA_GUARD_SCRATCH_BYTES) {
        pcpa_params b = *p;
        b.flags = (b.flags | PCPA_FLAG_BF16_MFMA) & ~(uint32_t)PCPA_FLAG_PRECISION_GUARD;
        return history_launch(&b, 1, q, kv_pages, block_table, page_valid_len, out, lse, nullptr, 0, stream);
    }
    GuardLease lease;
    return history_launch(p, 1, q, kv_pages, block_table, page_valid_len, out, lse, nullptr, 0, stream, &lease);
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
        case PCPA_ERR_WORKSPACE: return "workspace missing or smaller than pcpa_split_workspace_bytes";
        case PCPA_ERR_SCRATCH: return "launch needs more than the library's fixed scratch";
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
    if (p->flags & ~(uint32_t)(PCPA_FLAG_BF16_MFMA | PCPA_FLAG_EXACT_EXP2 | PCPA_FLAG_PRECISION_GUARD |
                               PCPA_FLAG_TABLE_INT64 | PCPA_FLAG_E4M3_UNGUARDED))
        return PCPA_ERR_BAD_SHAPE;
    if ((p->flags & PCPA_FLAG_PRECISION_GUARD) && (p->flags & PCPA_FLAG_E4M3_UNGUARDED)) return PCPA_ERR_BAD_SHAPE;
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
                                   const void* block_table, const int32_t* page_valid_len, void* out,
                                   float* lse, void* stream) {
    return pcpa::history_one_pass(p, q, kv_pages, block_table, page_valid_len, out, lse, (hipStream_t)stream);
}

int64_t pcpa_split_workspace_bytes(const pcpa_params* p, int32_t splits) {
    const int32_t st = pcpa_check_params(p);
    if (st != PCPA_OK) return st;
    if (splits < 1 || splits > PCPA_MAX_SPLITS) return PCPA_ERR_BAD_SHAPE;
    return pcpa::workspace_layout(p, splits).bytes;
}

int32_t pcpa_history_attention_split(const pcpa_params* p, int32_t splits, const void* q, const void* kv_pages,
                                     const void* block_table, const int32_t* page_valid_len, void* out,
                                     float* lse, void* workspace, int64_t workspace_bytes, void* stream) {
    return pcpa::history_launch(p, splits, q, kv_pages, block_table, page_valid_len, out, lse, workspace,
                                workspace_bytes, (hipStream_t)stream);
}

int32_t pcpa_history_attention_noalloc(const pcpa_params* p, int32_t splits, const void* q, const void* kv_pages,
                                       const void* block_table, const int32_t* page_valid_len, void* out, float* lse,
                                       void* stream) {
    const int64_t need = pcpa_split_workspace_bytes(p, splits);
    if (need < 0) return (int32_t)need;
    if (need > PCPA_NOALLOC_SCRATCH_BYTES) return PCPA_ERR_SCRATCH;
    void* ws = nullptr;
    if (need > 0) {
        const int32_t st = pcpa::scratch_for_current_device(&ws);
        if (st != PCPA_OK) return st;
    }
    return pcpa::history_launch(p, splits, q, kv_pages, block_table, page_valid_len, out, lse, ws, need,
                                (hipStream_t)stream);
}

int32_t pcpa_history_attention(const pcpa_params* p, const void* q, const void* kv_pages,
                               const void* block_table, const int32_t* page_valid_len, void* out,
                               void* stream) {
    return pcpa::history_one_pass(p, q, kv_pages, block_table, page_valid_len, out, nullptr, (hipStream_t)stream);
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
        hipLaunchKernel(fn, dim3(8 * ((items + 7) / 8)), dim3(pcpa::tile_threads(p->head_dim, false)), args, 0,
                        (hipStream_t)stream);
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
                            const void* k, const void* v, const void* block_table, void* kv_pages,
                            int32_t* page_valid_len, void* stream) {
    const int32_t st = pcpa_check_params(p);
    if (st != PCPA_OK) return st;
    if (!k || !v || !block_table || !kv_pages) return PCPA_ERR_NULL_POINTER;
    if (interleave <= 0 || first_pos < 0 || num_tokens < 0) return PCPA_ERR_BAD_SHAPE;
    if (((uintptr_t)k | (uintptr_t)v | (uintptr_t)kv_pages) & 15u) return PCPA_ERR_MISALIGNED;
    if (((uintptr_t)block_table | (uintptr_t)page_valid_len) & 3u) return PCPA_ERR_MISALIGNED;
    if ((p->flags & PCPA_FLAG_TABLE_INT64) && ((uintptr_t)block_table & 7u)) return PCPA_ERR_MISALIGNED;
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
    a.block_table = (const int32_t*)block_table;
    a.table_shift = (p->flags & PCPA_FLAG_TABLE_INT64) ? 1 : 0;
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
    a.k_rcp = 1.f / p->k_scale;
    a.v_rcp = 1.f / p->v_scale;
    auto div_ok = [](float d) { return d >= 0x1p-80f && d <= 0x1p126f; };
    a.fast_div = div_ok(p->k_scale) && div_ok(p->v_scale) ? 1 : 0;
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

int32_t pcpa_block_mask_valid_len(const void* mask, int32_t pcp_size, int32_t max_local_blocks, int32_t block_size,
                                  int32_t* page_valid_len, void* stream) {
    if (!mask || !page_valid_len) return PCPA_ERR_NULL_POINTER;
    if (pcp_size <= 0 || max_local_blocks <= 0 || block_size <= 0 || block_size % 128) return PCPA_ERR_BAD_SHAPE;
    if ((int64_t)pcp_size * max_local_blocks > INT32_MAX) return PCPA_ERR_TOO_LARGE;
    if (((uintptr_t)mask & 1u) || ((uintptr_t)page_valid_len & 3u)) return PCPA_ERR_MISALIGNED;
    hipLaunchKernelGGL(pcpa::paging::mask_lengths_kernel, dim3(max_local_blocks), dim3(pcpa::paging::kMaskThreads), 0,
                       (hipStream_t)stream, (const uint16_t*)mask, block_size, max_local_blocks, pcp_size,
                       page_valid_len);
    return hipGetLastError() == hipSuccess ? PCPA_OK : PCPA_ERR_LAUNCH;
}

int32_t pcpa_page_alloc(const pcpa_params* p, int32_t interleave, int64_t first_pos, int32_t num_tokens,
                        void* block_table, const int32_t* free_pages, int32_t* free_count, void* stream) {
    const int32_t st = pcpa_check_params(p);
    if (st != PCPA_OK) return st;
    if (!block_table || !free_pages || !free_count) return PCPA_ERR_NULL_POINTER;
    if (interleave <= 0 || first_pos < 0 || num_tokens < 0) return PCPA_ERR_BAD_SHAPE;
    if (((uintptr_t)block_table | (uintptr_t)free_pages | (uintptr_t)free_count) & 3u) return PCPA_ERR_MISALIGNED;
    if ((p->flags & PCPA_FLAG_TABLE_INT64) && ((uintptr_t)block_table & 7u)) return PCPA_ERR_MISALIGNED;
    if (num_tokens == 0) return PCPA_OK;
    // the positions must fit the cache (as pcpa_kv_cache_write requires);
    // rank 0 owns the most positions of any prefix of the history
    const int64_t end = first_pos + num_tokens;
    const int64_t capacity = (int64_t)p->max_local_blocks * p->block_size;
    if (pcpa::paging::owned_below(end, 0, p->pcp_size, interleave) > capacity) return PCPA_ERR_BAD_SHAPE;
    pcpa::paging::AllocArgs a;
    a.table = (int32_t*)block_table;
    a.table_shift = (p->flags & PCPA_FLAG_TABLE_INT64) ? 1 : 0;
    a.free_pages = free_pages;
    a.free_count = free_count;
    a.first_pos = first_pos;
    a.end_pos = end;
    a.pcp = p->pcp_size;
    a.interleave = interleave;
    a.block_size = p->block_size;
    a.max_local_blocks = p->max_local_blocks;
    hipLaunchKernelGGL(pcpa::paging::page_alloc_kernel, dim3(1), dim3(pcpa::paging::kAllocThreads), 0,
                       (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? PCPA_OK : PCPA_ERR_LAUNCH;
}

}  // extern "C"

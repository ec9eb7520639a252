/*
 * C ABI of the MI355X (gfx950) history-only PCP attention library
 * (libpcp_attention_hip.so).
 *
 * Plain C types only: device pointers are `const void*` / `void*`, the HIP
 * stream is passed as `void*` (a hipStream_t, or NULL for the null stream).
 * The library never synchronises the host: every launch is asynchronous on
 * the given stream.  Status codes are returned, never printed.  Calls are
 * safe from several host threads on different streams.
 *
 * Device memory: the library calls no hipMalloc.  Its code object holds two
 * fixed `__device__` arrays, PCPA_GUARD_SCRATCH_BYTES + PCPA_NOALLOC_SCRATCH_BYTES
 * = 128 MiB on every GPU a process launches any entry point on, held until
 * the process ends:
 *   - the guard scratch of pcpa_history_attention / _lse (the precision
 *     guard's row flags, row lists and partials when the caller gives no
 *     workspace).  The library orders the calls that use it on one GPU (an
 *     event per GPU: a call's first kernel waits for the previous user's
 *     last), except on a stream under graph capture, where no ordering is
 *     recorded: a captured call must not replay while another call on that
 *     GPU uses the guard scratch.
 *   - the array of pcpa_history_attention_noalloc (not ordered by the
 *     library).
 * Every other entry point uses only the memory its caller passes.
 *
 * Reference interface replaced (Trainium2 NKI proof of concept):
 *   pcp_attention/kernel.py:32-556  make_history_attention_kernel(config)
 *       -> history_attention_kernel(q_ref, local_kv_ref, block_valid_mask_ref)
 *   pcp_attention/kernel.py:559-564 wrap_for_native_torch(config)
 * The reference runs one kernel instance per logical PCP rank and rotates
 * KV blocks around a device ring (kernel.py:276-293).  Here every rank's
 * KV blocks sit in one paged pool in HBM and one launch computes all
 * ranks' outputs; the ring becomes a loop over the block table.
 */
#ifndef PCP_ATTENTION_HIP_H
#define PCP_ATTENTION_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PCPA_ABI_VERSION 3

/* Status codes. */
#define PCPA_OK 0
#define PCPA_ERR_NULL_POINTER (-1)  /* a required pointer is NULL            */
#define PCPA_ERR_ABI_VERSION (-2)   /* params.abi_version != PCPA_ABI_VERSION */
#define PCPA_ERR_BAD_SHAPE (-3)     /* non-positive or inconsistent sizes     */
#define PCPA_ERR_BAD_DTYPE (-4)     /* dtype code not supported              */
#define PCPA_ERR_UNSUPPORTED (-5)   /* valid but not implemented (head_dim…) */
#define PCPA_ERR_MISALIGNED (-6)    /* a tensor pointer is not 16-byte aligned */
#define PCPA_ERR_LAUNCH (-7)        /* the HIP launch itself failed          */
#define PCPA_ERR_TOO_LARGE (-8)     /* an index would overflow 32/64-bit maths */
#define PCPA_ERR_BAD_SCALE (-9)     /* a scale is not finite and positive    */
#define PCPA_ERR_WORKSPACE (-10)    /* workspace missing or too small        */
#define PCPA_ERR_SCRATCH (-11)      /* more than PCPA_NOALLOC_SCRATCH_BYTES   */

/* params.flags bits. */
/* Run both GEMMs as BF16 MFMAs even for an e4m3 cache: K/V are widened to
 * bf16 exactly while staged, Q and P stay bf16.  Half the MFMA rate, but no
 * e4m3 rounding of Q and P.  Ignored for a bf16 cache. */
#define PCPA_FLAG_BF16_MFMA 1u
/* FP8 MFMA path at head_dim 256: compute the e4m3 probabilities with
 * v_exp_f32 instead of the default linear-mantissa exp2 (which writes the
 * e4m3 code of 2^x directly; both round P to e4m3, the default interpolates
 * the exponential between powers of two first).  Slower; ignored elsewhere,
 * where P always comes from v_exp_f32. */
#define PCPA_FLAG_EXACT_EXP2 2u
/* Precision guard of the e4m3 MFMAs: ON by default for every launch that
 * runs e4m3 MFMAs (an e4m3 cache without PCPA_FLAG_BF16_MFMA); this bit
 * asks for it explicitly and changes nothing else.
 * e4m3 Q and P carry ~3.6% relative rounding noise per element, which
 * averages away only when many keys share a row's softmax, and the error
 * grows with the spread of V.  A first launch measures, per KV head h, the
 * threshold
 *     thr_h = PCPA_GUARD_MIN_MASS * v_scale^2 * max_d Var_k(V[h, k, d])
 * (the variance per channel of the e4m3 V codes over up to 2048 sampled
 * keys of the walk); the e4m3 pass measures each row's probability mass
 *     W = sum_k 2^(x_k - m)        (x_k the score in log2 units, m the
 *                                    running reference, at most 2.5 below
 *                                    the row's largest x_k)
 * and a later launch recomputes, with BF16 MFMAs on the exactly widened
 * cache (bf16 Q and P), every row with W < thr_h (short histories, peaked
 * score distributions, wide V), the rows gathered 128 to a workgroup.  Its
 * workgroups exit at once when no row is listed.  Its buffers (thresholds,
 * per-head row lists, the recomputation's partials) are in the caller's
 * workspace (pcpa_history_attention_split, sized by
 * pcpa_split_workspace_bytes), the allocation-free array
 * (pcpa_history_attention_noalloc) or, for pcpa_history_attention / _lse,
 * the library's guard scratch; a launch whose guard buffers exceed
 * PCPA_GUARD_SCRATCH_BYTES runs every row on BF16 MFMAs there instead. */
#define PCPA_FLAG_PRECISION_GUARD 4u
#define PCPA_GUARD_MIN_MASS 384.0f
/* e4m3 MFMAs without the precision guard (the fastest path; rows with few
 * effective keys can miss a 2e-2 absolute error bar).  Must not be combined
 * with PCPA_FLAG_PRECISION_GUARD. */
#define PCPA_FLAG_E4M3_UNGUARDED 16u
/* block_table holds int64 entries (torch's default integer type) instead of
 * int32; an entry outside [0, num_pages) is an empty page either way.  Also
 * accepted by pcpa_kv_cache_write. */
#define PCPA_FLAG_TABLE_INT64 8u

/* dtype codes. */
#define PCPA_DTYPE_BF16 1
#define PCPA_DTYPE_FP8_E4M3FN 2 /* OCP e4m3 "fn": bias 7, max 448, no inf */

/*
 * Shapes of one launch.  All ranks are processed together.
 *   q            [pcp_size, num_q_heads, local_q_len, head_dim]   q_dtype
 *   kv_pages     [num_pages, 2, num_kv_heads, block_size, head_dim] kv_dtype
 *                (each row is pack_local_kv's payload, kernel.py:17-29:
 *                 all K of a block, then all V)
 *   block_table  [pcp_size, max_local_blocks] int32 (int64 with
 *                PCPA_FLAG_TABLE_INT64): physical page of (rank, local
 *                block); entries outside [0, num_pages) are treated as empty
 *                pages (never read)
 *   page_valid_len [pcp_size, max_local_blocks] int32: number of valid
 *                leading tokens of that cache block, clamped to
 *                [0, block_size].  Valid tokens of a striped rank always
 *                form a prefix of its local sequence, so this encodes the
 *                reference's additive mask (run_poc.py:137-153) exactly.
 *   out          [pcp_size, num_q_heads, local_q_len, head_dim] bf16
 * Q heads are grouped contiguously per KV head: Q head h reads KV head
 * h / (num_q_heads / num_kv_heads) (reference.py:10-13).
 * Scores are (q . k) * softmax_scale * k_scale; V is multiplied by v_scale
 * (per-tensor dequantisation scales, 1.0 for unscaled storage).
 */
typedef struct pcpa_params {
    int32_t abi_version;
    int32_t pcp_size;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t local_q_len;
    int32_t block_size;
    int32_t max_local_blocks;
    int32_t num_pages;
    int32_t q_dtype;
    int32_t kv_dtype;
    int32_t out_dtype;
    float softmax_scale;
    float k_scale;
    float v_scale;
    uint32_t flags; /* PCPA_FLAG_* bits; other bits must be 0 */
} pcpa_params;

/* Returns PCPA_ABI_VERSION of the loaded library. */
int32_t pcpa_abi_version(void);

/* Static, NUL-terminated description of a status code. */
const char* pcpa_status_string(int32_t status);

/*
 * Validate `params` without launching anything (no HIP call is made).
 * Returns PCPA_OK or the error the launch entry point would return for
 * these parameters (pointer checks excluded).
 */
int32_t pcpa_check_params(const pcpa_params* params);

/*
 * History-only attention over the paged KV pool for every rank's Q.
 * Replaces kernel.py:32-556 (history_attention_kernel) and
 * kernel.py:559-564 (wrap_for_native_torch).  Output is caller-allocated
 * (the reference kernel allocated it, kernel.py:124).
 * flags = 0 on an e4m3 cache runs e4m3 MFMAs with the precision guard, its
 * buffers in the library's guard scratch (calls on one GPU ordered by the
 * library, see the top of this file); PCPA_FLAG_BF16_MFMA and
 * PCPA_FLAG_E4M3_UNGUARDED launches use no scratch.
 */
int32_t pcpa_history_attention(const pcpa_params* params, const void* q, const void* kv_pages,
                               const void* block_table, const int32_t* page_valid_len,
                               void* out, void* stream);

/*
 * pcpa_history_attention that also writes each row's log-sum-exp:
 *   lse  [pcp_size, num_q_heads, local_q_len] float (optional, NULL = none):
 *        natural log of sum_k exp(score_k) over the row's valid history
 *        keys (scores as above), -INFINITY for a row with no valid key.
 * This is what a later merge with other keys (the current tokens) needs.
 * The e4m3 path at head_dim 256 without PCPA_FLAG_EXACT_EXP2 corrects the
 * mean bias of its linear-mantissa exp2 (sum inflated by 1.0407 on average,
 * i.e. lse - 0.0399); its lse is good to about 1e-3 over long histories.
 * No reference counterpart: the reference kernel returns the normalised
 * output only (kernel.py:546-551).
 */
int32_t pcpa_history_attention_lse(const pcpa_params* params, const void* q, const void* kv_pages,
                                   const void* block_table, const int32_t* page_valid_len,
                                   void* out, float* lse, void* stream);

/*
 * History attention with a caller-provided workspace: split history and the
 * precision guard.
 * Split history, for workloads with few query rows: the table entries are cut
 * into `splits` equal ranges, each (row tile, range) pair runs as its own
 * workgroup and writes a normalised partial output (FP32; the e4m3
 * head_dim-256 path: FP16 before the v_scale factor, which the merge
 * applies), log-sum-exp and reference maximum into `workspace`, and a
 * second launch merges the partials by log-sum-exp into `out` (and `lse`,
 * optional).  Results equal
 * pcpa_history_attention_lse's to rounding.  For a launch whose (row tile,
 * KV head) workgroups would leave CUs idle (256 rows and a CU per workgroup
 * for e4m3 MFMAs at head_dim 256, else 128 rows, two per CU).  Every cache
 * dtype, precision and head dim of pcpa_history_attention_lse; splits in
 * [1, PCPA_MAX_SPLITS] (1 = one pass).
 * On e4m3 MFMAs (unless PCPA_FLAG_E4M3_UNGUARDED) the workspace also holds
 * the precision guard's row flags and lists, and the BF16 pass follows the
 * e4m3 one (or the merge).
 * workspace: device memory of at least pcpa_split_workspace_bytes(params,
 * splits) bytes (0 for splits = 1 without the guard, when NULL is
 * accepted), 16-byte aligned; its contents need no initialisation and are
 * left undefined.  The library does not allocate it.  No reference
 * counterpart (the reference's device ring has no split, and its NKI kernel
 * one precision, kernel.py:84-554).
 */
#define PCPA_MAX_SPLITS 64
int64_t pcpa_split_workspace_bytes(const pcpa_params* params, int32_t splits);
int32_t pcpa_history_attention_split(const pcpa_params* params, int32_t splits, const void* q,
                                     const void* kv_pages, const void* block_table,
                                     const int32_t* page_valid_len, void* out, float* lse,
                                     void* workspace, int64_t workspace_bytes, void* stream);

/*
 * pcpa_history_attention_split with no workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The split partials and guard
 * buffers live in a fixed array of PCPA_NOALLOC_SCRATCH_BYTES that the
 * library holds on every GPU it runs on until the process ends; this entry
 * point calls no hipMalloc, hipFree or allocating routine.  A launch whose
 * pcpa_split_workspace_bytes(params, splits) exceeds the array returns
 * PCPA_ERR_SCRATCH.  The array needs no initialisation and keeps the last
 * call's contents; every call on one GPU shares it, so calls that overlap
 * on one GPU (several streams or host threads) race and must be ordered by
 * the caller.  No counterpart in the reference; for callers that cannot
 * allocate.
 */
#define PCPA_NOALLOC_SCRATCH_BYTES (80ll << 20)
/* The guard scratch of pcpa_history_attention / _lse, per GPU. */
#define PCPA_GUARD_SCRATCH_BYTES (48ll << 20)
int32_t pcpa_history_attention_noalloc(const pcpa_params* params, int32_t splits, const void* q,
                                       const void* kv_pages, const void* block_table,
                                       const int32_t* page_valid_len, void* out, float* lse, void* stream);

/*
 * Causal attention of the current tokens among themselves, optionally merged
 * with a history result: the step after the history attention.  The
 * reference stops at history-only attention ("current tokens do not attend
 * to each other yet", README.md:17-18); the semantics here are the standard
 * ones: the query at global current position g sees current keys 0..g.
 *   q           [pcp_size, num_q_heads, local_q_len, head_dim] bf16, striped
 *               as for pcpa_history_attention with `interleave` (the local
 *               token t of rank r is global position
 *               ((t / il) * pcp_size + r) * il + t % il, layout.py:10-16)
 *   kv_current  [2, num_kv_heads, pcp_size * local_q_len, head_dim] bf16:
 *               K then V of the current tokens in global order (one "page"
 *               of block size pcp_size * local_q_len, which must be a
 *               multiple of 64)
 *   hist_out, hist_lse (optional, both or neither): the history output and
 *               log-sum-exp of pcpa_history_attention_lse for the same q.
 *               With them, out = softmax attention over history keys and
 *               causal current keys together (log-sum-exp merge), and lse
 *               covers both.
 *   out         as q; may alias hist_out (each row is read before written)
 *   lse         optional, as for pcpa_history_attention_lse
 * params: kv_dtype must be bf16 here (current K/V are not quantised),
 * k_scale / v_scale / block_size / max_local_blocks / num_pages are unused
 * (validated only).
 */
int32_t pcpa_current_attention(const pcpa_params* params, int32_t interleave, const void* q,
                               const void* kv_current, const void* hist_out, const float* hist_lse,
                               void* out, float* lse, void* stream);

/*
 * KV-cache producer (the step before the attention): quantise K and V of the
 * history tokens at global positions [first_pos, first_pos + num_tokens) and
 * write them into their pages, in pack_local_kv's row format.  Replaces the
 * host chain shard_history (layout.py:54-98) -> float8 cast (run_poc.py:
 * 96-103, here with per-tensor scales) -> pack_local_kv (kernel.py:17-29) ->
 * page placement by the block table, and also serves appends.
 *   k, v        [num_kv_heads, num_tokens, head_dim] bf16 (global token order)
 *   kv_pages    pool as for pcpa_history_attention (params.kv_dtype); only
 *               the rows of the written tokens change
 *   e4m3 pools store round_e4m3(x / params.k_scale) (v_scale for V), bit
 *   for bit torch's (x.float() / scale).to(torch.float8_e4m3fn); bf16 pools
 *   store x unchanged.  Token p belongs to rank (p / interleave) % pcp_size at
 *   local position ((p / interleave) / pcp_size) * interleave + p % interleave
 *   (layout.py:10-16), i.e. block local / block_size, slot local % block_size.
 *   Tokens whose table entry is outside [0, num_pages) are not written.
 *   page_valid_len (optional, int32 [pcp_size, max_local_blocks]): each
 *   written token's entry is raised to at least slot + 1.
 * The q/out fields of params are validated but unused.
 */
int32_t pcpa_kv_cache_write(const pcpa_params* params, int32_t interleave, int64_t first_pos,
                            int32_t num_tokens, const void* k, const void* v,
                            const void* block_table, void* kv_pages, int32_t* page_valid_len,
                            void* stream);

/*
 * max |x| over n bf16 values into *amax (device float): the amax of the
 * per-tensor e4m3 scale amax / 448 (the FP8 configurations' K/V
 * quantisation).  A NaN anywhere in x makes *amax NaN, as torch's
 * x.abs().max() does.  Two launches on `stream`; *amax needs no
 * initialisation.
 */
int32_t pcpa_absmax_bf16(const void* x, int64_t n, float* amax, void* stream);

/*
 * The reference's runtime mask turned into per-page valid lengths on the GPU
 * (no host round trip, so a mask-form call can be captured in a HIP graph).
 *   mask  [max_local_blocks, block_size / 128, 1, 128] bf16, the additive
 *         score bias of make_block_valid_mask (run_poc.py:137-153) that the
 *         NKI kernel takes as block_valid_mask_ref (kernel.py:113-118,
 *         341-358): 0 for a valid key, -9984 for padding, shared by all ranks
 *   page_valid_len [pcp_size, max_local_blocks] int32 (written): for every
 *         rank, the number of leading keys of the block whose bias is zero.
 * The reference's masks are always such prefixes; this kernel does not check
 * that (a host-side conversion can).  block_size must be a multiple of 128.
 */
int32_t pcpa_block_mask_valid_len(const void* mask, int32_t pcp_size, int32_t max_local_blocks,
                                  int32_t block_size, int32_t* page_valid_len, void* stream);

/*
 * Page allocation for appended history tokens, on the GPU: every cache block
 * (rank, local block) that the positions [first_pos, first_pos + num_tokens)
 * reach and whose block_table entry is negative (no page yet) takes a page
 * from the top of a device free-page stack, in (rank, block) entry order:
 *   free_pages  int32 stack of free page indices; entries [0, *free_count)
 *               are free, the top one is free_pages[*free_count - 1]
 *   free_count  device int32, lowered by the pages taken (not below 0;
 *               entries that find the stack empty stay negative, and
 *               pcpa_kv_cache_write then skips their tokens)
 *   block_table int32 (int64 with PCPA_FLAG_TABLE_INT64), updated in place.
 * One workgroup; deterministic (the same appends give the same table).  Call
 * it before pcpa_kv_cache_write for the same positions.  Replaces the
 * reference's host-side placement of every rank's blocks into its padded
 * local cache (run_poc.py:231-237, layout.py:54-98); its pages are what
 * pack_local_kv rows occupy (kernel.py:17-29).  The positions must fit the
 * cache as for pcpa_kv_cache_write (PCPA_ERR_BAD_SHAPE otherwise).
 */
int32_t pcpa_page_alloc(const pcpa_params* params, int32_t interleave, int64_t first_pos, int32_t num_tokens,
                        void* block_table, const int32_t* free_pages, int32_t* free_count, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PCP_ATTENTION_HIP_H */

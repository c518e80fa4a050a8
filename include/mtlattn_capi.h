/*
 * mtlattn C ABI -- the drop-in boundary of the MI355X (gfx950) varlen
 * flash-attention library libmtlattn_hip.so.
 *
 * Every entry point replaces one export of the reference's pybind11 module
 * `mtlattn._C` (src/ext.mm:784-811). Signatures use plain pointers, sizes and
 * an opaque stream handle only (no torch types), so any FFI can bind them; the
 * torch extension mtlattn_amd/csrc/torch_ext.cpp is one such binder.
 *
 * Conventions shared by all entry points:
 *  - Tensors are device pointers. q/k/v/out/dout are [tokens, heads, D] with
 *    the last two dims contiguous (head stride == D) and a free row stride
 *    (in elements), as src/ext.mm:322-325 requires.
 *  - cu_seqlens_{q,kv} are device int32 [num_seqs + 1] cumulative offsets.
 *    Sequence bounds are clamped to [0, total] on the device, so malformed
 *    offsets never address outside the tensors.
 *  - Causal masking is end-aligned: query i sees key j iff
 *    j <= i + (kv_len - q_len); window W > 0 adds j > i + (kv_len - q_len) - W.
 *  - GQA: query head h reads kv head h / (Hq / Hkv).
 *  - The library never allocates device memory. Callers pass scratch space
 *    sized by the matching *_workspace_size() query.
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = the default stream)
 *    of the current device; nothing synchronises with the host.
 *  - Return value: MTLATTN_OK (0) or a negative MTLATTN_ERR_*; the message is
 *    available from mtlattn_last_error() on the calling thread.
 */
#ifndef MTLATTN_CAPI_H
#define MTLATTN_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MTLATTN_ABI_VERSION 2

/* element types of q/k/v/out/dout/dq/dk/dv */
enum {
    MTLATTN_DTYPE_F32 = 0,
    MTLATTN_DTYPE_F16 = 1,
    MTLATTN_DTYPE_BF16 = 2
};

enum {
    MTLATTN_OK = 0,
    MTLATTN_ERR_INVALID = -1,     /* bad argument (shape, stride, null pointer) */
    MTLATTN_ERR_UNSUPPORTED = -2, /* valid request this build has no kernel for */
    MTLATTN_ERR_WORKSPACE = -3,   /* workspace missing or too small */
    MTLATTN_ERR_LAUNCH = -4       /* HIP reported an error at launch */
};

/*
 * Problem description shared by every entry point. Mirrors the scalar part
 * of the reference's kernel argument block `Params` (src/ext.mm:44-57) plus
 * the bias strides of src/ext.mm:348-365.
 */
typedef struct mtlattn_problem {
    int32_t dtype;            /* MTLATTN_DTYPE_* of q/k/v */
    int32_t num_seqs;         /* B; cu_seqlens have B + 1 entries */
    int64_t total_q;          /* rows of q / out / dout */
    int64_t total_kv;         /* rows of k / v */
    int32_t num_heads_q;      /* Hq */
    int32_t num_heads_kv;     /* Hkv; Hq % Hkv == 0 */
    int32_t head_dim;         /* D */
    int32_t max_seqlen_q;     /* caller's bound on q lengths (decode routing only) */
    float scale;              /* logit = scale * q.k (+ bias) */
    int32_t causal;           /* 0 / 1 */
    int32_t window;           /* <= 0: no sliding window */
    const int32_t* cu_seqlens_q;   /* device int32 [B + 1] */
    const int32_t* cu_seqlens_kv;  /* device int32 [B + 1] */
    const float* bias;        /* optional fp32 additive mask, NULL = none */
    int64_t bias_q_stride;    /* elements between query rows of bias */
    int64_t bias_h_stride;    /* elements between heads; 0 = broadcast over heads */
    int64_t bias_kv_cols;     /* size of bias's key dim; keys beyond read as 0 */
    /* Row addressing of bias (no counterpart in the reference, which indexes
     * by global query row): 0 = row of global query r at r * bias_q_stride;
     * 1 = row of query i of sequence s at s * bias_seq_stride +
     * min(i, bias_seq_rows - 1) * bias_q_stride (a dense [B or 1, H or 1,
     * Nq, Nkv] mask used in place, stride 0 for a broadcast batch dim). */
    int32_t bias_seq_local;
    int64_t bias_seq_stride;
    int64_t bias_seq_rows;
} mtlattn_problem;

/* Version of this header the library was built from (== MTLATTN_ABI_VERSION). */
int mtlattn_abi_version(void);

/* Message describing the last failure on this thread ("" if none). */
const char* mtlattn_last_error(void);

/* Compute-unit count of `device` (256 on MI355X); <= 0 on error.
 * Replaces _C.gpu_core_count (src/ext.mm:785). */
int mtlattn_gpu_core_count(int device);

/*
 * Forward: out = softmax(scale * q k^T + bias + mask) v per sequence, plus the
 * natural-log LSE per (row, head) when `lse` is non-NULL.
 * Replaces _C.varlen_attention (src/ext.mm:293-489) including its routing:
 * few-query / long-KV calls go to split-KV decode + combine
 * (src/ext.mm:367-390; here also with a window or a bias, which the
 * reference sends to its flash forward), everything else to the flash
 * forward.
 *   out : contiguous [total_q, Hq, D], same dtype as q
 *   lse : NULL or fp32 [total_q, Hq] (rows with no allowed key get -inf)
 * Workspace: the split-KV partials of calls routed to decode; for fp32
 * problems on the fp32 matrix-core kernels whose grid would leave CUs idle,
 * fp32 partials of 2-8 key splits (a smaller workspace runs them unsplit);
 * otherwise none.
 */
size_t mtlattn_varlen_fwd_workspace_size(const mtlattn_problem* p);
int mtlattn_varlen_fwd(const mtlattn_problem* p,
                       const void* q, int64_t q_row_stride,
                       const void* k, int64_t k_row_stride,
                       const void* v, int64_t v_row_stride,
                       void* out, float* lse,
                       void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * The forward above, allocating nothing and taking no workspace. No
 * counterpart in the reference: for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving (decode) loops,
 * harnesses that forbid allocation. Same routing, kernels and results as
 * mtlattn_varlen_fwd (bitwise); the split-KV partials of calls routed to
 * decode, and the fp32 key-split partials (sized to fit it), live in a
 * static device array of MTLATTN_NOALLOC_SCRATCH_BYTES per
 * GPU, set up on the first call on each GPU (do that call outside capture)
 * and held until the process ends. Calls whose partials would exceed it
 * (mtlattn_varlen_fwd_workspace_size(p) > MTLATTN_NOALLOC_SCRATCH_BYTES)
 * return MTLATTN_ERR_WORKSPACE. Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other threads) race
 * and must be serialised by the caller. Each call rewrites every partial it
 * reads, so nothing carries over from earlier calls.
 */
#define MTLATTN_NOALLOC_SCRATCH_BYTES (64ll << 20)
int mtlattn_varlen_fwd_noalloc(const mtlattn_problem* p,
                               const void* q, int64_t q_row_stride,
                               const void* k, int64_t k_row_stride,
                               const void* v, int64_t v_row_stride,
                               void* out, float* lse,
                               void* stream);

/*
 * Backward: (dq, dk, dv) of the forward above given dout and the forward's
 * out and lse. dk/dv of a kv head are summed over its Hq/Hkv query heads
 * inside the kernels (no atomics; bitwise run-to-run deterministic).
 * Replaces _C.varlen_attention_bwd (src/ext.mm:502-594). The reference needs
 * contiguous inputs (mtlattn/__init__.py:42-45); this entry also takes row
 * strides. dq/dk/dv are written contiguous in the input dtype. The
 * workspace (fp32 [total_q, Hq]) holds delta = rowsum(dO * O) of every row a
 * sequence owns when the call returns; at head dims 64 and 128 the dQ kernel
 * computes it (no separate preprocess launch), bitwise equal to
 * mtlattn_bwd_preprocess. On the fp32 matrix-core kernels the dQ kernel
 * computes delta too (equal to the preprocess up to fp32 rounding); for fp32
 * problems whose dQ or dK/dV grid would leave CUs idle, the size query adds
 * room (after delta, 256-byte aligned) for fp32 partials of 2-8 splits,
 * summed in a fixed order; a workspace of only the delta size runs unsplit.
 */
size_t mtlattn_varlen_bwd_workspace_size(const mtlattn_problem* p);
int mtlattn_varlen_bwd(const mtlattn_problem* p,
                       const void* q, int64_t q_row_stride,
                       const void* k, int64_t k_row_stride,
                       const void* v, int64_t v_row_stride,
                       const void* out, int64_t out_row_stride,
                       const void* dout, int64_t dout_row_stride,
                       const float* lse,
                       void* dq, void* dk, void* dv,
                       void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * delta[row, h] = sum_d dout[row, h, d] * out[row, h, d] in fp32.
 * Replaces the torch reduction at src/ext.mm:518 / bwd_delta_impl
 * (src/attention.metal:724-733). delta: fp32 [total_q, Hq].
 */
int mtlattn_bwd_preprocess(const mtlattn_problem* p,
                           const void* out, int64_t out_row_stride,
                           const void* dout, int64_t dout_row_stride,
                           float* delta, void* stream);

/*
 * dQ alone (test entry). Replaces _C.mpp_bwd_dq (src/ext.mm:656-711).
 * dq_dtype: MTLATTN_DTYPE_F32 (as the reference returns) or p->dtype.
 */
int mtlattn_bwd_dq(const mtlattn_problem* p,
                   const void* q, int64_t q_row_stride,
                   const void* k, int64_t k_row_stride,
                   const void* v, int64_t v_row_stride,
                   const void* dout, int64_t dout_row_stride,
                   const float* lse, const float* delta,
                   void* dq, int32_t dq_dtype, void* stream);

/*
 * dK and dV alone (test entry). Replaces _C.mpp_bwd_dkv (src/ext.mm:597-653).
 * dkv_dtype: MTLATTN_DTYPE_F32 (as the reference returns) or p->dtype.
 */
int mtlattn_bwd_dkv(const mtlattn_problem* p,
                    const void* q, int64_t q_row_stride,
                    const void* k, int64_t k_row_stride,
                    const void* v, int64_t v_row_stride,
                    const void* dout, int64_t dout_row_stride,
                    const float* lse, const float* delta,
                    void* dk, void* dv, int32_t dkv_dtype, void* stream);

/*
 * Split-KV decode with an explicit split count (test entry): each split
 * attends one chunk of every sequence's keys and writes a normalised fp32
 * partial O and its LSE; a combine kernel merges them and also writes the
 * final LSE when `lse` is non-NULL. num_splits == 1 is a plain forward.
 * Replaces _C.attn_splitkv (src/ext.mm:716-773; kernels
 * src/attn_mpp.metal:384-535). Requires fp16/bf16, D in {64, 128},
 * max_seqlen_q <= 16 (query rows of a kv head handled in groups of 16).
 * Bias and window are honoured (the reference's split path has neither);
 * with a window the splits divide only the keys the sequence's rows can see.
 * Workspace: fp32 partial rows of D values plus one LSE each, 16 rows per
 * (kv head, head group, sequence, split).
 */
size_t mtlattn_attn_splitkv_workspace_size(const mtlattn_problem* p, int32_t num_splits);
int mtlattn_attn_splitkv(const mtlattn_problem* p,
                         const void* q, int64_t q_row_stride,
                         const void* k, int64_t k_row_stride,
                         const void* v, int64_t v_row_stride,
                         void* out, float* lse, int32_t num_splits,
                         void* workspace, size_t workspace_bytes,
                         void* stream);

/*
 * Decode over a paged KV cache. No counterpart in the reference (it has no
 * paged KV); the layout is FlashAttention's varlen call with a block table.
 * Same computation as the forward (causal, window, bias, LSE) for
 * max_seqlen_q <= 16, fp16/bf16, D in {64, 128}, through split-KV + combine.
 *   k_cache / v_cache : [num_pages, page_size, Hkv, D], token row strides
 *                       k_row_stride / v_row_stride (elements); a page is
 *                       page_size consecutive token rows
 *   block_table       : int32 [num_seqs, block_table_stride] on the device
 *                       (block_table_stride entries per sequence, all of
 *                       them readable); logical key j of sequence s is row
 *                       j % page_size of page
 *                       block_table[s * block_table_stride + min(j / page_size,
 *                       block_table_stride - 1)] (page indices are clamped
 *                       to [0, num_pages)), so the table needs
 *                       ceil(kv_len / page_size) entries per sequence
 *   p->cu_seqlens_kv  : logical KV lengths (prefix sums); p->total_kv is an
 *                       upper bound on cu_seqlens_kv[num_seqs], the sum of
 *                       the logical lengths (pages may be shared between
 *                       sequences, so it can exceed the cache capacity)
 *   page_size         : a multiple of 16
 *   max_seqlen_kv     : bound on the logical KV lengths (sizes the window
 *                       splits)
 * Work split: fixed KV chunks numbered by the logical prefix sums (slots for
 * p->total_kv keys) as on the contiguous decode path; with a window, equal
 * splits of each sequence's band.
 * Workspace: mtlattn_paged_decode_workspace_size(p, max_seqlen_kv) bytes.
 */
size_t mtlattn_paged_decode_workspace_size(const mtlattn_problem* p, int64_t max_seqlen_kv);
int mtlattn_paged_decode(const mtlattn_problem* p,
                         const void* q, int64_t q_row_stride,
                         const void* k_cache, int64_t k_row_stride,
                         const void* v_cache, int64_t v_row_stride,
                         int32_t page_size, int64_t num_pages,
                         const int32_t* block_table, int64_t block_table_stride,
                         int64_t max_seqlen_kv,
                         void* out, float* lse,
                         void* workspace, size_t workspace_bytes,
                         void* stream);

/* Number of split-KV work-item slots per (kv head, head group) the forward's
 * decode routing would use for `p` (0 = the call is not routed to split-KV).
 * The automatic path cuts each sequence's KV into fixed-length chunks (about
 * 18 work items per CU) rather than a fixed number of splits per sequence,
 * so ragged KV lengths stay balanced; with a window each sequence gets a
 * fixed number of equal splits of its window band instead (slots =
 * num_seqs * splits). Retunes src/ext.mm:372-388. */
int32_t mtlattn_decode_num_splits(const mtlattn_problem* p);

/*
 * Key-padding pack / unpack for the SDPA adapter. No counterpart in the
 * reference's _C: its adapter (mtlattn/__init__.py:202-249) copies each
 * batch's valid prefix in Python after pulling the lengths to the host; these
 * do it on the device with no host synchronisation.
 *
 * mtlattn_pack_padded: dense src [B, H, N, D] (element strides sb, sh, sn of
 * the B, H, N dims; D contiguous) -> packed rows dst [B * N, H, D]. Batch b's
 * first lens[b] tokens (clamped to [0, N]) go to rows cu[b] + n, where
 * cu = prefix sums of the lengths, written to cu_out [B + 1] (int32, device);
 * the padded tokens follow all valid ones. Use dst with cu_out as the varlen
 * q/k/v and cu_seqlens (rows past cu_out[B] belong to no sequence).
 * mtlattn_unpack_padded: packed rows src [B * N, H, D] -> dense dst
 * [B, H, N, D] (strides sb, sh, sn): token (b, n) takes row cu[b] + n when
 * n < lens[b], zeros otherwise.
 * dtype is MTLATTN_DTYPE_*; all pointers are device pointers.
 */
int mtlattn_pack_padded(int32_t dtype, int32_t B, int32_t N, int32_t H, int32_t D,
                        const void* src, int64_t sb, int64_t sh, int64_t sn,
                        const int32_t* lens, int32_t* cu_out, void* dst, void* stream);
int mtlattn_unpack_padded(int32_t dtype, int32_t B, int32_t N, int32_t H, int32_t D,
                          const void* src, const int32_t* lens, const int32_t* cu,
                          void* dst, int64_t sb, int64_t sh, int64_t sn, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MTLATTN_CAPI_H */

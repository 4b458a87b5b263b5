/*
 * mfa.h -- C ABI of the MI355X (gfx950) flash-attention library
 * (libmtlfa_hip.so, built from mtlflashattn_amd/csrc/mfa_fwd.hip and mfa_bwd.hip).
 *
 * This is the drop-in boundary that replaces the reference's per-tier Metal
 * launch calls.  In the reference the Python launcher binds a JIT-compiled
 * Metal library and calls one kernel per tier with device buffers Q, K, V, O
 * plus three small parameter tensors:
 *   SH  int32 shape vector   [B, Hq, Hkv, Lq, Lk, causal(, Lkp)]
 *   PR  fp32 parameter vector [scale, softcap, win_left, win_right, alibi_on]
 *   AL  fp32 [B*Hq] ALiBi slopes (or a 1-element dummy)
 * (metal_flash_attn/_kernel.py:1309-1312 `lib.flash_attn_fwd_v2r_dtype(...)`,
 *  :1333-1337, :1368-1373, :1397-1401, :1416-1419; SH/PR/AL semantics at
 *  :1221-1272).  Here the same information travels in one POD struct, passed
 * by pointer and copied by value into the kernel arguments, so no per-call
 * device parameter tensors exist at all.
 *
 * Contract:
 *  - Every entry point is stateless and re-entrant.  mfa_fwd only enqueues
 *    work on `stream` (a hipStream_t, e.g. torch.cuda.current_stream()
 *    .cuda_stream); it never synchronizes and never allocates.
 *  - Return value 0 = success, negative = error; the message is available
 *    from mfa_last_error() on the same thread.
 *  - All pointers are device pointers.  The head dimension must be
 *    contiguous (element stride 1) in q, k, v and o; every other stride is an
 *    element stride and may describe any layout (views, packed qkv,
 *    heads-second or heads-third), as long as q, k, v and o start at 16-byte
 *    aligned addresses and each of their strides is a multiple of 16 bytes
 *    (8 elements of 16 bits, 4 of fp32); other layouts return
 *    MFA_ERR_INVALID.
 */
#ifndef MTLFA_MFA_H
#define MTLFA_MFA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MFA_ABI_VERSION 7

/* element types (dtype_in / dtype_out) */
#define MFA_DTYPE_F16 0
#define MFA_DTYPE_BF16 1
#define MFA_DTYPE_F32 2

/* error codes */
#define MFA_OK 0
#define MFA_ERR_INVALID -1     /* bad argument (shape, stride, alignment, dtype) */
#define MFA_ERR_UNSUPPORTED -2 /* valid request this build does not implement */
#define MFA_ERR_LAUNCH -3      /* the HIP runtime refused the launch */

#define MFA_MAX_HEAD_DIM 128

/* tile_hint values (bf16/fp16 only; fp32 has one kernel).  Sequences of one
 * query row (and single-row grouped-query decode, whose query heads are
 * computed as the rows of one K/V head) always run the exact-row kernel,
 * whose probabilities carry two 16-bit terms; the hint applies to the rest. */
#define MFA_TILE_AUTO 0     /* library's choice */
#define MFA_TILE_256 1      /* 256-row tiles, 4 wavefronts */
#define MFA_TILE_PINGPONG 2 /* ping-pong tiles, 8 wavefronts: 512 rows at head_dim <= 64,
                               256 rows at head_dim 97..128 (not 65..96) */
#define MFA_TILE_PINGPONG256 3 /* 256-row ping-pong tiles, 8 wavefronts (head_dim <= 64 or
                                  97..128); the library's choice at head_dim <= 64 for causal
                                  calls whose 512-row tiles would leave CUs idle while the
                                  heaviest tiles finish */

/*
 * Forward parameters.  Replaces the SH/PR/AL buffers of the reference
 * (metal_flash_attn/_kernel.py:1221-1272) and the heads-second tensor
 * arguments of flash_attn_forward (metal_flash_attn/_kernel.py:1052-1053).
 *
 * Dense mode (cu_seqlens_q == NULL):
 *   q [batch, seqlen_q, heads_q, head_dim] addressed through the q_*_stride
 *   fields, likewise k/v [batch, seqlen_k, heads_kv, head_dim] and
 *   o [batch, seqlen_q, heads_q, head_dim].
 * Varlen mode (cu_seqlens_q != NULL, metal_flash_attn/__init__.py:102-183):
 *   q [total_q, heads_q, head_dim], k/v [total_k, heads_kv, head_dim],
 *   o [total_q, heads_q, head_dim]; sequence i owns tokens
 *   [cu_seqlens_q[i], cu_seqlens_q[i+1]) of q/o and
 *   [cu_seqlens_k[i], cu_seqlens_k[i+1]) of k/v.  `batch` is the number of
 *   sequences, the *_batch_stride fields are ignored, and seqlen_q/seqlen_k
 *   must hold max_seqlen_q/max_seqlen_k (upper bounds of every sequence).
 *   The kernel and tile choice is made from these bounds (e.g. seqlen_k <= 32
 *   under many query rows selects a kernel that holds one 32-key block per
 *   sequence), so a bound below a sequence's real length gives wrong
 *   results for that sequence; it is not detected on the device.
 *
 * Masking/bias (metal_flash_attn/_kernel.py:32-87): for query row i of a
 * sequence with Lq queries and Lk keys, center = i + (Lk - Lq); key j is
 * valid iff j <= center (causal), j >= center - window_left (window_left >= 0)
 * and j <= center + window_right (window_right >= 0).  Scores are
 * s = scale * q.k; s = softcap * tanh(s / softcap) when softcap > 0;
 * s -= slope * |center - j| when alibi_slopes != NULL, with
 * slope = alibi_slopes[b * alibi_batch_stride + h] (alibi_batch_stride 0 for
 * per-head [Hq] slopes, Hq for [B, Hq]).  Rows with no valid key produce 0.
 */
typedef struct mfa_fwd_params {
    const void* q;
    const void* k;
    const void* v;
    void* o;

    int64_t q_batch_stride, q_seq_stride, q_head_stride;
    int64_t k_batch_stride, k_seq_stride, k_head_stride;
    int64_t v_batch_stride, v_seq_stride, v_head_stride;
    int64_t o_batch_stride, o_seq_stride, o_head_stride;

    int32_t batch;
    int32_t heads_q;
    int32_t heads_kv;
    int32_t seqlen_q;
    int32_t seqlen_k;
    int32_t head_dim;

    const int32_t* cu_seqlens_q; /* NULL = dense */
    const int32_t* cu_seqlens_k; /* NULL = dense */

    float scale;
    float softcap;        /* 0 = off; must be >= 0 */
    int32_t window_left;  /* -1 = unbounded */
    int32_t window_right; /* -1 = unbounded */
    int32_t causal;       /* 0/1, bottom-right aligned */

    const float* alibi_slopes; /* NULL = off; fp32 */
    int32_t alibi_batch_stride;

    int32_t dtype_in;  /* MFA_DTYPE_* of q, k and v */
    int32_t dtype_out; /* == dtype_in, or MFA_DTYPE_F32 (full-precision output) */
    int32_t tile_hint; /* MFA_TILE_AUTO (0); the others force a bf16/fp16 kernel
                          (tests and tuning; results meet the same bars either
                          way) for every sequence of more than one query row */

    /* Softmax log-sum-exp output (optional; the reference raises for it,
     * metal_flash_attn/__init__.py:49-50).  lse = ln(sum_j exp(s_j)) over the
     * row's valid keys, s the transformed score above (natural-log units, as
     * CUDA flash-attn's softmax_lse), -inf for a row with no valid key.  fp32,
     * query rows contiguous: dense lse[b * lse_batch_stride + h *
     * lse_head_stride + i]; varlen lse[h * lse_head_stride + cu_seqlens_q[b]
     * + i] (lse_batch_stride ignored; [heads_q, total_q] when
     * lse_head_stride = total_q). */
    float* softmax_lse; /* NULL = not written */
    int64_t lse_batch_stride;
    int64_t lse_head_stride;

    /* Paged K/V (optional; the reference raises for block_table,
     * metal_flash_attn/__init__.py:130-131).  k and v are
     * [num_pages, page_block_size, heads_kv, head_dim] addressed through
     * k_batch_stride/v_batch_stride (page stride), *_seq_stride and
     * *_head_stride; key j of sequence b is row j % page_block_size of page
     * block_table[b * block_table_batch_stride + j / page_block_size].  The
     * key count of sequence b is seqlen_k (dense) or cu_seqlens_k[b+1] -
     * cu_seqlens_k[b] (varlen; the start offsets are not used for k/v).
     * page_block_size is a positive multiple of 256; a page id outside
     * [0, num_pages) reads as zeros, never out of bounds, but its keys are
     * not masked: they score 0 and take weight in the softmax, so the rows
     * that see them come out wrong (callers validate their tables).  Paged
     * calls run on the 256-row and fp32 kernels: MFA_TILE_PINGPONG with a
     * block_table is MFA_ERR_UNSUPPORTED. */
    const int32_t* block_table; /* NULL = contiguous k/v */
    int64_t block_table_batch_stride;
    int32_t page_block_size;
    int32_t num_pages;

    /* Varlen calls, optional (0 = unknown; ABI 7): 1 when the caller knows
     * that no sequence has exactly one query row.  A varlen call otherwise
     * adds a launch of the exact-row kernel for such sequences (the main
     * launch leaves them to it); 1 skips that launch, so a sequence of one
     * query row would keep its o rows (and lse) unwritten.  Ignored by dense
     * calls.  No counterpart in the reference. */
    int32_t varlen_no_single_rows;
} mfa_fwd_params;

/* Launch geometry of one mfa_fwd call (for profiling/roofline reports). */
typedef struct mfa_launch_info {
    int32_t grid_x;          /* workgroups launched */
    int32_t block_x;         /* threads per workgroup */
    int32_t rows_per_block;  /* query rows per workgroup tile */
    int32_t keys_per_block;  /* keys per K/V block */
    int32_t lds_bytes;       /* LDS bytes per workgroup */
    char kernel_name[96];    /* short name of the kernel instantiation */
} mfa_launch_info;

/* ABI version of the loaded library (MFA_ABI_VERSION).  No counterpart in
 * the reference (its kernels are JIT-compiled from source strings). */
int mfa_abi_version(void);

/* Message of the last failed call on this thread ("" if none).  Replaces
 * the RuntimeError strings of the reference's forced-tier checks
 * (metal_flash_attn/_kernel.py:1083-1140). */
const char* mfa_last_error(void);

/* 1 if mfa_fwd implements (dtype_in, head_dim) on this build, else 0.
 * Replaces the eligibility probes _v1_eligible/_v2_dtype_eligible
 * (metal_flash_attn/_kernel.py:928-936, :896-912). */
int mfa_supported(int32_t dtype_in, int32_t head_dim);

/* Enqueue the attention forward on `stream` (hipStream_t; NULL = default
 * stream).  Replaces the tier launchers _flash_v2r_dtype / _flash_v2_dtype /
 * _flash_v2 / _flash_v1 / _flash_v0 (metal_flash_attn/_kernel.py:1288-1420)
 * and their kernel calls. */
int mfa_fwd(const mfa_fwd_params* params, void* stream);

/* Fill *info with the geometry mfa_fwd would launch for `params`; enqueues
 * nothing.  No counterpart in the reference. */
int mfa_fwd_launch_info(const mfa_fwd_params* params, mfa_launch_info* info);

/* sizeof(mfa_fwd_params) as compiled into the library, so FFI bindings can
 * check their struct mirror.  No counterpart in the reference. */
int mfa_params_size(void);

/* Split-KV forward for decode-like shapes (few query rows, long key ranges):
 * the key range of every sequence is cut into chunks of `split_keys` keys,
 * workgroups compute the chunks in parallel into a caller-provided
 * workspace, and a second kernel merges them (log-sum-exp weighting).  No
 * counterpart in the reference, whose Metal kernels run one threadgroup per
 * query tile over all keys; these three calls are the build's addition for
 * HBM-bound shapes.  bf16/fp16 only; results meet the same bars as mfa_fwd.
 *
 * mfa_fwd_split_keys: the library's choice for `params`, 0 = use mfa_fwd.
 * It is 2048 when seqlen_q (the longest query for varlen) is at most 256 and
 * seqlen_k exceeds 2048, else 0 (fp32 and forced ping-pong tiles: 0); a
 * dense call with batch > 1 and batch * heads_q >= 512 gets 0 too (the
 * single pass already fills the chip).  For varlen and batch = 1 calls the
 * choice depends on the lengths only, so a sequence is chunked alike alone or
 * inside a varlen batch (bit-identical rows either way).
 * mfa_fwd_workspace_bytes: device bytes mfa_fwd_splitkv needs for this call
 * and chunk size (0 for split_keys 0 or an empty problem; < 0 on error).
 * mfa_fwd_splitkv: enqueue both kernels on `stream`; `workspace` is a
 * 256-byte aligned device buffer of at least that many bytes, owned by the
 * caller and reused only after the call's kernels ran (stream order).
 * split_keys must be 0 (same as mfa_fwd) or a positive multiple of 64 (of
 * 256 with a block_table).  softmax_lse and block_table work as in mfa_fwd. */
int32_t mfa_fwd_split_keys(const mfa_fwd_params* params);
int64_t mfa_fwd_workspace_bytes(const mfa_fwd_params* params, int32_t split_keys);
int mfa_fwd_splitkv(const mfa_fwd_params* params, int32_t split_keys, void* workspace, int64_t workspace_bytes,
                    void* stream);

/* Size of the static scratch array behind mfa_fwd_splitkv_static (64 MiB per
 * GPU, held from the library's first use on that GPU until the process
 * ends). */
#define MFA_STATIC_SCRATCH_BYTES (64LL << 20)

/* mfa_fwd_splitkv without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * split-KV partials go to a file-scope device array of
 * MFA_STATIC_SCRATCH_BYTES bytes (one per GPU); a call whose
 * mfa_fwd_workspace_bytes exceeds that returns MFA_ERR_INVALID with a
 * message.  Allocates nothing (no hipMalloc, hipFree or allocating library
 * call); the first call on a GPU looks up the array's device address once.
 * Same kernels, chunks and results as mfa_fwd_splitkv (bit for bit);
 * split_keys 0 behaves as mfa_fwd.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (different streams, or host threads
 * without ordering between them) race and must be serialised by the caller;
 * calls in one stream are ordered and safe.  The array keeps the last call's
 * partials; nothing needs clearing (each call writes every partial it reads). */
int mfa_fwd_splitkv_static(const mfa_fwd_params* params, int32_t split_keys, void* stream);

/*
 * Backward pass (gradients of q, k, v).  No counterpart in the reference,
 * which is forward-only (metal_flash_attn/__init__.py:3-4, README.md:159-161;
 * training callers fall back to other attention).  Same masking and bias
 * semantics as the forward; the forward's O and softmax_lse are inputs:
 *   P = exp(s - lse), dV = P^T dO, dP = dO V^T, Dsum = rowsum(dO * O),
 *   dS = P * (dP - Dsum) [* (1 - tanh^2) under softcap], dQ = scale dS K,
 *   dK = scale dS^T Q.
 * With grouped-query heads, dK/dV of a K/V head sum over its query heads.
 * Deterministic (no atomics): one kernel owns each dK/dV block and loops over
 * every query of its K/V head; another owns each dQ block.
 * fp32 (dtype_in = MFA_DTYPE_F32: q, k, v, o, dout and the gradients fp32)
 * runs fp32 kernels on the vector ALU with the fp32 forward's score transform
 * (strides then multiples of 4 elements; the workspace holds the row sums
 * only).  bf16/fp16 run on the matrix cores.
 */
typedef struct mfa_bwd_params {
    /* q, k, v, o (the forward output), shapes, strides, masks and biases as
     * in the forward; fwd.softmax_lse (+ strides) is the forward's lse and
     * required; fwd.block_table must be NULL; fwd.tile_hint is ignored;
     * fwd.dtype_out is o's dtype and must equal dtype_in. */
    mfa_fwd_params fwd;
    const void* dout; /* dL/dO, laid out like o (its own strides), o's dtype */
    int64_t do_batch_stride, do_seq_stride, do_head_stride;
    void* dq;         /* laid out like q */
    int64_t dq_batch_stride, dq_seq_stride, dq_head_stride;
    void* dk;         /* laid out like k */
    int64_t dk_batch_stride, dk_seq_stride, dk_head_stride;
    void* dv;         /* laid out like v */
    int64_t dv_batch_stride, dv_seq_stride, dv_head_stride;
    int32_t dtype_grad; /* dtype of dq/dk/dv: dtype_in or MFA_DTYPE_F32 */
    int32_t reserved;
    /* Optional gradient of the loss with respect to softmax_lse (fp32, same
     * layout and strides as fwd.softmax_lse; NULL = zero).  Since
     * d lse_i / d s_ij = P_ij, it enters as Dsum_i - dlse_i. */
    const float* dlse;
} mfa_bwd_params;

/* 1 if mfa_bwd implements (dtype_in, head_dim): bf16/fp16/fp32, head_dim a
 * multiple of 8 up to MFA_MAX_HEAD_DIM. */
int mfa_bwd_supported(int32_t dtype_in, int32_t head_dim);
/* Device workspace mfa_bwd needs, 0 for an empty problem, < 0 on error: the
 * fp32 row sums Dsum, and with grouped-query heads (heads_q > heads_kv) the
 * fp32 dK/dV partials of each query head (2 * heads_q * batch * seqlen_k *
 * padded head_dim * 4 bytes) when they fit in 2 GiB -- the query heads of a
 * K/V head then run in parallel workgroups and are summed in head order. */
int64_t mfa_bwd_workspace_bytes(const mfa_bwd_params* params);
/* Enqueue the backward kernels on `stream`; `workspace`: 256-byte aligned
 * device buffer of at least mfa_bwd_workspace_bytes bytes, owned by the
 * caller.  Never synchronizes, never allocates. */
int mfa_bwd(const mfa_bwd_params* params, void* workspace, int64_t workspace_bytes, void* stream);
int mfa_bwd_params_size(void);

#ifdef __cplusplus
}
#endif

#endif /* MTLFA_MFA_H */

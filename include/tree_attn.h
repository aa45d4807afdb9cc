/*
 * tree_attn.h -- C ABI of the MI355X (gfx950) tree-shared decode-attention backend.
 *
 * Replaces the Triton kernels of the reference's src/tree_attention/kernels.py:
 *   _segment (kernels.py:8-55)   -> ta_segment
 *   _merge   (kernels.py:58-83)  -> ta_merge
 *   attention_matrix's launch sequence (kernels.py:152-168) -> ta_attention_matrix
 *
 * Conventions
 *   - Every pointer is a device pointer owned by the caller; the library allocates
 *     nothing, keeps no state between calls and never synchronises the host.
 *   - Launches are asynchronous on `stream` (a hipStream_t; NULL = default stream).
 *   - Return value: 0 on success, a HIP error code from the launch, or one of the
 *     TA_ERR_* argument errors below.  ta_error_string() names any of them.
 *   - dtype: TA_BF16 or TA_FP16, shared by q, kp, vp and out.  Accumulation and
 *     the log-sum-exp values are fp32; partial outputs are stored as fp16 rows
 *     scaled by a power of two (below).
 *   - Layouts (row-major, contiguous, base 16-byte aligned):
 *       q     [nreq, hq, d]        query of each request (kernels.py:157 permutes it;
 *                                  here the kernel indexes it directly)
 *       kp    [hk, d, tcap]        K pool, token-minor (kernels.py:144, qwen.py:27)
 *       vp    [hk, tcap, d]        V pool                 (kernels.py:145, qwen.py:28)
 *       part  [nslot, hq, d] fp16  normalised partial output per (job, request),
 *                                  row-scaled: stored value = (o / z) * 2^-e with e
 *                                  the frexp exponent of the row's largest |o / z|;
 *                                  within a row, element d = 32p + 16h + 4g + i
 *                                  (i < 4) is stored at 32p + 8g + 4h + i
 *       lse   [nslot, hq, 2] fp32  per row: natural-log log-sum-exp, then e
 *       out   [nreq, hq, d]
 *   - Job j covers physical tokens [kstart[j], kstart[j] + klen[j]) for the requests
 *     qids[j*maxr + 0 .. qlen[j]-1]; its partial rows are slots rowbase[j] + i.
 *     klen[j] == 0 yields a zero partial with lse = -inf, which the merge ignores.
 *   - Supported: d in {32, 64, 128}, hq % hk == 0.
 */
#ifndef TREE_ATTN_H
#define TREE_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TA_BF16 0
#define TA_FP16 1

/* segment work-item kinds; items are (job, first query row, kv head) triples */
#define TA_SMALL 0      /* jobs with <= 16 query rows (first row 0), one wave each */
#define TA_LARGE64 1    /* row tiles of 64 rows  */
#define TA_LARGE128 2   /* row tiles of 128 rows */
#define TA_LARGE256 3   /* row tiles of 256 rows */
#define TA_TAIL 4       /* single-request jobs that are their request's only job of
                           <= 16 rows (first row 0): in ta_attention_matrix and
                           ta_tail_merge the item also merges its request's other
                           partial slots and writes out; through ta_segment it
                           writes its partial like TA_SMALL.  The job's own slot
                           is the last of its request's slots. */
#define TA_NKINDS 5

/* attached segments per TA_LARGE256 work item (ta_plan.xtail) */
#define TA_XTAIL_MAX 4
#define TA_XTAIL_STRIDE (1 + 4 * TA_XTAIL_MAX)

#define TA_ERR_ARG 1001      /* null pointer, bad size or unsupported shape */
#define TA_ERR_ALIGN 1002    /* q / kp / vp / part / out not 16-byte aligned, lse not 8-byte */
#define TA_ERR_DTYPE 1003    /* dtype not TA_BF16 / TA_FP16 */
#define TA_ERR_SCRATCH 1004  /* ta_attention_matrix_noalloc: partials beyond TA_NOALLOC_SCRATCH_BYTES */

/* Device memory of ta_attention_matrix_noalloc's partials, per GPU: the plan's
 * nslot * hq * d fp16 partial rows, rounded up to 256 bytes, plus
 * nslot * hq (lse, exponent) fp32 pairs must fit (32 MiB: e.g. 4,096 slots of
 * 32 query heads at d = 128; the 128 x 8192 headline layer needs 17.3 MB). */
#define TA_NOALLOC_SCRATCH_BYTES (32u << 20)

/* Everything one attention_matrix call needs besides q, kp, vp and out.
 * Built once per plan by the host (kernels.py:103-141 `prepare`). */
typedef struct ta_plan {
    const int32_t *qids;      /* [njobs * maxr]                                   */
    const int32_t *kstart;    /* [njobs] first physical token of each job          */
    const int32_t *qlen;      /* [njobs] requests per job                          */
    const int32_t *klen;      /* [njobs] tokens per job (device-updatable; attached
                               * tails keep theirs in xtail, see below)           */
    const int32_t *rowbase;   /* [njobs] first partial slot of each job            */
    const int32_t *slots;     /* [nreq * maxs] partial slots of each request       */
    const int32_t *counts;    /* [nreq] number of slots of each request            */
    const int32_t *items[TA_NKINDS];  /* work-item triples per kind TA_SMALL .. TA_TAIL */
    int32_t n_items[TA_NKINDS];       /* number of triples per kind                 */
    const int32_t *rest;      /* [n_rest] requests without a TA_TAIL job: the ones
                                 the merge kernel of ta_attention_matrix covers;
                                 NULL with n_rest == nreq: every request         */
    void *part;               /* [nslot, hq, d] fp16, row-scaled                   */
    float *lse;               /* [nslot, hq, 2]                                    */
    int32_t njobs, maxr, maxs, nreq, nslot;
    int32_t hq, hk, d, dtype;
    int32_t n_rest;
    /* Attached segments of the TA_LARGE256 items (NULL: none), an execution
     * detail with no counterpart in the reference: xtail_stride
     * (= TA_XTAIL_STRIDE) ints per TA_LARGE256 item -- the number of segments
     * n <= TA_XTAIL_MAX, then (first physical token, tokens, first job row,
     * rows) for each of the n.  A segment's tokens belong to the query rows
     * [first job row, first job row + rows) of the item's job, which lie in
     * one wave (32 rows): a private tail (the group rows of one request) or a
     * node of a few consecutive requests.  The item folds the tokens into those
     * rows' partials, so the segment has no partial slot of its own.  Needs
     * tcap % 8 == 0 (ta_attention_matrix returns TA_ERR_ARG otherwise).
     * Decode steps: a growing tail's length lives in klen[j] when the tail is
     * job j, and in the tokens field (int 2 + 4k of the item's record) of
     * every record that holds it as segment k when it is attached; a caller
     * that lengthens its tails between steps rewrites all of these positions
     * (kernels.PreparedPlan.grow_offsets lists them within the plan's
     * metadata buffer), not klen alone. */
    const int32_t *xtail;
    int32_t xtail_stride;
    /* [njobs] or NULL: the first request id of each job whose requests are
     * consecutive (qids[j*maxr + i] == qbase[j] + i), -1 for the others
     * (cf. the reference's contiguous-Q path, kernels.py:23-26, 138). */
    const int32_t *qbase;
    /* 0, or the stride of an affine slot layout: every merged request r has
     * maxs partial slots, slot k being r + k * slot_stride (slots[r*maxs + k]
     * holds the same values).  The merge then computes the slots instead of
     * loading counts and slot lists. */
    int32_t slot_stride;
} ta_plan;

/* Version string of the library build. */
const char *ta_version(void);

/* Human-readable name of a return code of this library. */
const char *ta_error_string(int code);

/* Grouped partial attention of physical KV segments (replaces _segment,
 * kernels.py:8-55, and its launch at kernels.py:158-165).  Writes the
 * normalised partial output and the log-sum-exp of every (job, request, head)
 * row of the given work items. */
int ta_segment(const void *q, const void *kp, const void *vp,
               const int32_t *qids, const int32_t *kstart, const int32_t *qlen,
               const int32_t *klen, const int32_t *rowbase,
               const int32_t *items, int32_t n_items, int32_t kind,
               void *part, float *lse,
               int32_t nreq, int32_t hq, int32_t hk, int32_t d, int32_t tcap,
               int32_t maxr, int32_t dtype, void *stream);

/* Global log-sum-exp merge of each request's partial outputs (replaces _merge,
 * kernels.py:58-83, and its launch at kernels.py:166-167). */
int ta_merge(const void *part, const float *lse, const int32_t *slots,
             const int32_t *counts, void *out, int32_t nreq, int32_t hq,
             int32_t d, int32_t maxs, int32_t dtype, void *stream);

/* One decode-step attention layer on resident pools (replaces attention_matrix,
 * kernels.py:152-168): the large-job segment launches, the small-job launch,
 * the TA_TAIL launch that merges the requests owning a tail job, and the merge
 * of the remaining requests (`rest`).  Pools whose capacity is not a multiple
 * of 8 take the unfused order: every segment kind, then the merge of all
 * requests. */
int ta_attention_matrix(const void *q, const void *kp, const void *vp,
                        int32_t tcap, const ta_plan *plan, void *out, void *stream);

/* ta_attention_matrix without caller-provided partial buffers.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  The same launches and results as ta_attention_matrix, but
 * the partial rows and log-sum-exp values live in a fixed array of the library
 * (TA_NOALLOC_SCRATCH_BYTES; each GPU the library runs on holds one until the
 * process ends); plan->part and plan->lse are ignored and may be NULL.  The
 * call allocates nothing; a plan whose partials do not fit returns
 * TA_ERR_SCRATCH before any launch.  Every call on one GPU shares that GPU's
 * array, which keeps the last call's contents (each call writes every slot it
 * reads): calls that overlap on one GPU -- other streams, other host threads --
 * race; calls ordered on one stream do not.  The current device must be the
 * stream's device (TA_ERR_ARG otherwise). */
int ta_attention_matrix_noalloc(const void *q, const void *kp, const void *vp,
                                int32_t tcap, const ta_plan *plan, void *out, void *stream);

/* The TA_TAIL launch of ta_attention_matrix on its own: each work item attends
 * its request's tail job and merges the request's other partial slots (written
 * before, on the same stream) into `out`.  No counterpart in the reference: a
 * fusion of _segment (kernels.py:8-55) for these jobs with _merge
 * (kernels.py:58-83).  Needs tcap % 8 == 0 (TA_ERR_ARG otherwise). */
int ta_tail_merge(const void *q, const void *kp, const void *vp,
                  int32_t tcap, const ta_plan *plan, void *out, void *stream);

/* The merge of a prepared plan: every request's partial slots into `out`
 * (kernels.py:166-167), with the plan's affine slot layout (slot_stride) when
 * it has one -- the merge ta_attention_matrix runs, for all nreq requests. */
int ta_merge_plan(const ta_plan *plan, void *out, void *stream);

/* One segment launch of a prepared plan: the work items of `kind`, writing
 * partials (TA_TAIL items included), with the plan's attached segments for
 * TA_LARGE256.  Counterpart of the reference's direct _segment launches in
 * scripts/calibrate_tiles.py:24-29 and scripts/profile_kernel.py:17-20, which
 * pass the prepared plan's tensors; TA_ERR_ARG for a plan with attached
 * segments on pools with tcap % 8 != 0. */
int ta_segment_plan(const void *q, const void *kp, const void *vp, int32_t tcap,
                    const ta_plan *plan, int32_t kind, void *stream);

/* One decode step's per-layer glue of the model adapter in one launch
 * (replaces apply_rotary_pos_emb, the two index_copy_ scatters into the
 * pools and the Q layout copy of qwen.py:86-91 / kernels.py:157).  For each
 * request r: q [nreq, hq, d], k and v [nreq, hk, d] (contiguous rows of the
 * projected, normalised step), cos and sin [d] at cos + r*cs_stride (0 for one
 * row shared by all requests); Q and K are rotated (rotate-half RoPE, each
 * multiply and the add rounded to dtype as the eager ops are), Q is written to
 * q_out [nreq, hq, d], K to kp[h, :, slots[r]] and V to vp[h, slots[r], :]
 * (pools [hk, d, tcap] / [hk, tcap, d]).  A slot outside [0, tcap) writes
 * nothing: a guard only, since the library cannot raise from the device; the
 * Python wrapper range-checks slots given as host data and raises ValueError,
 * as the eager index_copy_ of the reference adapter does.  No counterpart
 * kernel in the reference. */
int ta_decode_append(const void *q, const void *k, const void *v, const void *cos, const void *sin,
                     int32_t cs_stride, const int32_t *slots, void *kp, void *vp, void *q_out,
                     int32_t nreq, int32_t hq, int32_t hk, int32_t d, int32_t tcap, int32_t dtype,
                     void *stream);

/* Kernel timing hook.  No counterpart in the reference, which times kernels
 * with device events around whole launches (scripts/profile_kernel.py:17-33).
 * The next kernel this library launches on the calling host thread records
 * `start_event` when its dispatch begins and `stop_event` when it ends
 * (hipExtLaunchKernel); the hook then clears itself.  Both are hipEvent_t
 * created with timing enabled, or both NULL to clear the hook.  Not for use
 * under stream capture. */
int ta_time_next_launch(void *start_event, void *stop_event);

/* Measurement kernel with no counterpart in the reference: a read-only stream
 * over `bytes` (a multiple of 16) of device memory at `src` (16-byte aligned),
 * `blocks` workgroups of 256 threads in a grid-stride loop of 16-byte loads,
 * folding the data into one word per wave, sink[0 .. 4 * blocks).  Its
 * rate is the read ceiling the memory-bound segment kernels are compared
 * with.  Launches on `stream` (a hipStream_t). */
int ta_read_stream(const void *src, int64_t bytes, uint32_t *sink, int32_t blocks, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TREE_ATTN_H */

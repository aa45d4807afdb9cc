/*
 * tree_plan.h -- C ABI of the host-side grouped planner (libtree_plan.so).
 *
 * Replaces the grouped branch of the reference's schedule()
 * (src/tree_attention/schedule.py:94-151: greedy :103-112, subset DP :113-131)
 * with its cost model (:41-52).  Host code only; no GPU, no allocation visible
 * to the caller, no state kept between calls.
 *
 * The caller passes the tree in CSR form and receives one decision per node;
 * materialising the jobs (split() of every node's remaining requests over its
 * token chain, schedule.py:133-151) stays with the caller, whose plans are then
 * bit-exact with the reference planner's: same jobs, same order, same
 * estimated cost.  Valid when the cost is the reference's formula and every
 * root-to-node id chain is strictly increasing (then a kv_split chunk is one
 * physical job per consecutive run, schedule.py:13-26); other trees go
 * through the Python planner.
 */
#ifndef TREE_PLAN_H
#define TREE_PLAN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TP_GREEDY 0
#define TP_CUBE 1

/*
 * n nodes, node 0 the root; parent[v] (-1 for the root).
 * Children of v, in the tree's child order: child_idx[child_off[v] .. child_off[v+1]).
 * nreq[v]: number of requests whose path passes through v.
 * Node v's token ids as maximal runs of consecutive ids:
 *   (run_start[i], run_len[i]) for i in [run_off[v], run_off[v+1]).
 * fparams: bandwidth (bytes/us), cube_flops (FLOP/us), task_us, merge_us.
 * iparams: cube_rows, key_tile, kv_split, max_query_rows, qheads, kvheads, dim.
 * Outputs: pushed[v] = 1 if, in the plan, v's parent hands v its token chain
 * (SplitQ: v's requests leave the parent's job and attend parent + v tokens
 * together), else 0 (pushed[0] = 0); total[0] = the DP's cost estimate of the
 * root state (for greedy, the sum the reference's greedy pass computes).
 * Returns 0, or 1 for invalid arguments: a table that is not a tree rooted
 * at 0 with every child numbered after its parent, a child with more
 * requests below it than its parent holds, an empty run, or unusable model
 * parameters (qheads % kvheads != 0, nonpositive tile sizes).
 */
int tp_grouped_plan(int32_t method, int32_t n, const int32_t *parent, const int32_t *child_off,
                    const int32_t *child_idx, const int32_t *nreq, const int64_t *run_off,
                    const int64_t *run_start, const int64_t *run_len, const double *fparams,
                    const int64_t *iparams, int8_t *pushed, double *total);

/*
 * Attachment of small segments to 256-row work items, a step of the backend's
 * prepare() with no counterpart in the reference (its jobs each get their own
 * launch work; here a job whose rows fit one wave -- a private tail, or a
 * node of a few requests -- may instead be attended by the wave of a 256-row
 * item of a large job that holds all of its requests at consecutive rows).
 * Candidate jobs, in order, go to the candidate item with the fewest attached
 * tiles, then the fewest on the owning wave, then the lowest large job, within
 * xtail_max segments per item and max(the item's own tile count, min_cap)
 * attached tiles (min_cap lets the one-tile items of decode-sized layers take
 * their requests' tails).
 *   large jobs j < n_large: is256[j] (the job's rows use 256-row items),
 *     tiles[j] (LDS tiles its token run streams), requests
 *     req[req_off[j] .. req_off[j+1]) in row order (group query rows each)
 *   candidate jobs s < n_small: requests sreq[sreq_off[s] .. sreq_off[s+1])
 *     in row order, tiles_s[s], fixed[s] (1: never attached)
 *   requests are ids in [0, nreq); an item covers item_rows rows, a wave
 *     wave_rows of them
 * Outputs: item[s] = index of the item candidate s joined (-1: none),
 * lrow[s] = the first row of its requests in the large job; the item list
 * (item_job[i], item_row0[i]) for i < n_items[0], in large-job order (the
 * caller sizes it: the sum over 256-row jobs of ceil(rows / item_rows)).
 * Returns 0, or 1 for invalid arguments.
 */
int tp_attach_tails(int32_t n_large, const int32_t *is256, const int32_t *tiles, const int32_t *req_off,
                    const int32_t *req, int32_t group, int32_t n_small, const int32_t *sreq_off, const int32_t *sreq,
                    const int32_t *tiles_s, const int8_t *fixed, int32_t nreq, int32_t xtail_max,
                    int32_t wave_rows, int32_t item_rows, int32_t min_cap, int32_t *item, int32_t *lrow,
                    int32_t *item_job, int32_t *item_row0, int32_t *n_items);

/*
 * Device metadata of a prepared plan (the backend's prepare(), cf. the
 * reference's kernels.py:103-141), every int32 section in one buffer:
 *   qids[njobs*maxr] kstart[njobs] qlen[njobs] klen[njobs] slots[nreq*maxs]
 *   counts[nreq] rowbase[njobs] rest[n_rest] xtail[n_l256*xstride, only when
 *   n_att > 0] qbase[njobs] items of kinds TA_SMALL .. TA_TAIL (triples)
 * as struct ta_plan (tree_attn.h) points into them.  Jobs are in execution
 * order, small ones (small_jobs of them) first; a job's requests are
 * req[sum(qlen[0..j)) ..], its tokens [kstart[j], kstart[j] + klen[j]).
 * Attachments: n_att records of xstride ints for the 256-row items of
 * (att_job[a], att_row0[a]).  sizes[13]: maxr, maxs, nslot, n_rest,
 * n_items[5], contiguous (every job's requests span their count), the affine
 * slot stride (0: none), the buffer length, n_l256.  buf == NULL fills sizes
 * only.  Returns 0, 1 for invalid arguments (a request outside [0, nreq)),
 * 2 when buf_len is below the length.
 */
int tp_build_metadata(int32_t njobs, int32_t small_jobs, const int32_t *qlen, const int32_t *req,
                      const int32_t *kstart, const int32_t *klen, int32_t nreq, int32_t group, int32_t kvheads,
                      int32_t tile_rows, int32_t n_att, const int32_t *att_job, const int32_t *att_row0,
                      const int32_t *att_rec, int32_t xstride, int32_t *sizes, int32_t *buf, int64_t buf_len);

#ifdef __cplusplus
}
#endif

#endif /* TREE_PLAN_H */

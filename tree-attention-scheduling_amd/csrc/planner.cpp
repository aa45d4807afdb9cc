// planner.cpp -- host-side restatement of the grouped planners (greedy and
// subset DP) of the reference's src/tree_attention/schedule.py:72-151, with
// the cost model of :29-52.  Host code only (g++), no GPU.
//
// It computes the same decisions as tree_attention/schedule.py's
// _grouped_jobs (which itself is bit-exact with the reference): for every
// tree node, whether its parent's chosen state pushes it (the child inherits
// the parent's token chain, SplitQ) or leaves it alone (SplitK).  The Python
// caller materialises the jobs from those decisions.  Bit-exactness rests on:
//   * the cost expression evaluated in the reference's order in double
//     precision (this file is built with -ffp-contract=off);
//   * every sum a left-to-right accumulation from 0 in the same order as the
//     Python code (split(): request tiles outer, kv_split chunks inner,
//     physical runs innermost);
//   * the DP table kept in insertion order with strict '<' replacement
//     (a replaced entry keeps its position, as a Python dict does) and the
//     final choice by the lexicographic (cost, pushed children) comparison
//     of Python tuples (schedule.py:116-131);
//   * greedy pushing a child only on strict split_q < split_k (:103-112).
// Only the "fast" case is handled: the reference's cost formula and a tree
// whose root-to-node id chains increase (so every chunk's physical runs are
// its consecutive runs); the Python planner covers everything else.
#include "tree_plan.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <unordered_map>
#include <vector>

namespace {

struct Model {
    double bandwidth, cube_flops, task_us, merge_us;
    int64_t cube_rows, key_tile, kv_split, max_query_rows, qheads, kvheads, dim;

    // CostModel._cost_n: one physical job of nreq requests and ntok tokens
    double cost_n(int64_t nreq, int64_t ntok) const {
        if (!nreq || !ntok) return 0.0;
        const int64_t rows = nreq * (qheads / kvheads);
        const bool small = rows <= cube_rows;
        const int64_t q_tile = small ? cube_rows : max_query_rows;
        const int64_t k_tile = small ? key_tile : key_tile / 2;
        // math.ceil(rows / q_tile) on Python floats; exact for these magnitudes
        const int64_t qtiles = (int64_t)std::ceil((double)rows / (double)q_tile);
        const int64_t ktiles = (int64_t)std::ceil((double)ntok / (double)k_tile);
        const int64_t flops = 4 * qtiles * q_tile * ktiles * k_tile * dim * kvheads;
        const int64_t reads = 4 * ntok * dim * kvheads * qtiles;
        const int64_t partial = 4 * nreq * qheads * (dim + 1);
        const double a = (double)flops / cube_flops, b = (double)reads / bandwidth;
        double t = (a < b ? b : a);  // max(a, b): the first if they compare equal
        t = t + task_us * (double)qtiles * (double)kvheads;
        t = t + (double)partial / bandwidth;
        t = t + merge_us * (double)nreq;
        return t;
    }
};

using Runs = std::vector<std::pair<int64_t, int64_t>>;  // (first id, length)

struct Planner {
    const Model &m;
    int n;
    const int32_t *parent, *child_off, *child_idx, *nreq;
    const int64_t *run_off, *run_start, *run_len;
    int64_t req_tile;
    bool cube;

    std::unordered_map<int64_t, Runs> chain_runs;      // key v * (n + 1) + top
    std::unordered_map<int64_t, double> count_memo;    // key (count, v, top)
    struct State {
        double total;
        std::vector<int32_t> pushed;
        bool done = false;
    };
    std::unordered_map<int64_t, State> memo;  // key(v, top); top = -1: nothing inherited
    std::unordered_map<int64_t, std::pair<std::vector<int32_t>, int64_t>> greedy_push;

    int64_t key(int v, int top) const { return (int64_t)v * (n + 1) + (top + 1); }

    Runs own_runs(int v) const {
        Runs r;
        for (int64_t i = run_off[v]; i < run_off[v + 1]; ++i) r.emplace_back(run_start[i], run_len[i]);
        return r;
    }

    static void join(Runs &acc, const Runs &b) {
        for (size_t i = 0; i < b.size(); ++i) {
            if (i == 0 && !acc.empty() && acc.back().first + acc.back().second == b[0].first)
                acc.back().second += b[0].second;
            else
                acc.push_back(b[i]);
        }
    }

    // runs of the chain top -> ... -> v (top = -1 or top == v: v's own).  Walks
    // up to top or to a cached prefix, then joins downwards, caching each
    // intermediate chain (iterative: trees can be deep).
    const Runs &runs(int v, int top) {
        if (top < 0 || top == v) {
            auto it = chain_runs.find(key(v, -1));
            if (it == chain_runs.end()) it = chain_runs.emplace(key(v, -1), own_runs(v)).first;
            return it->second;
        }
        std::vector<int> pending;
        int u = v;
        while (u != top && chain_runs.find(key(u, top)) == chain_runs.end()) {
            pending.push_back(u);
            u = parent[u];
        }
        Runs acc = u == top ? runs(top, -1) : chain_runs.at(key(u, top));
        const Runs *last = nullptr;
        for (auto w = pending.rbegin(); w != pending.rend(); ++w) {
            join(acc, own_runs(*w));
            last = &chain_runs.emplace(key(*w, top), acc).first->second;
        }
        return last ? *last : chain_runs.at(key(v, top));
    }

    // sum(cost(j) for j in physical_jobs(split(range(count), chain tokens)))
    double count_cost(int64_t count, int v, int top) {
        const int64_t k = (count * (int64_t)(n + 1) + v) * (int64_t)(n + 1) + (top + 1);
        auto it = count_memo.find(k);
        if (it != count_memo.end()) return it->second;
        const Runs &r = runs(v, top);
        int64_t ntok = 0;
        std::vector<std::pair<int64_t, int64_t>> edges;
        for (const auto &p : r) {
            edges.emplace_back(ntok, ntok + p.second);
            ntok += p.second;
        }
        std::vector<std::vector<int64_t>> pieces;
        size_t ri = 0;
        for (int64_t kk = 0; kk < ntok; kk += m.kv_split) {
            const int64_t kend = std::min(kk + m.kv_split, ntok);
            std::vector<int64_t> chunk;
            while (edges[ri].second <= kk) ++ri;
            for (size_t j = ri; j < edges.size() && edges[j].first < kend; ++j)
                chunk.push_back(std::min(edges[j].second, kend) - std::max(edges[j].first, kk));
            pieces.push_back(std::move(chunk));
        }
        double total = 0.0;
        for (int64_t q = 0; q < count; q += req_tile) {
            const int64_t nq = std::min(req_tile, count - q);
            for (const auto &chunk : pieces)
                for (int64_t len : chunk) total = total + m.cost_n(nq, len);
        }
        count_memo.emplace(k, total);
        return total;
    }

    int child_top(int v, int top) const { return top < 0 ? v : top; }

    void greedy_choice(int v, int top, int ct, std::vector<int32_t> &pushed, int64_t &remaining) {
        remaining = nreq[v];
        for (int i = child_off[v]; i < child_off[v + 1]; ++i) {
            const int c = child_idx[i];
            const int64_t cnt = nreq[c];
            const double split_k = count_cost(remaining, v, top) + count_cost(cnt, c, c);
            const double split_q = count_cost(remaining - cnt, v, top) + count_cost(cnt, c, ct);
            if (split_q < split_k) {
                pushed.push_back(c);
                remaining -= cnt;
            }
        }
    }

    static bool less_pushed(const std::vector<int32_t> &a, const std::vector<int32_t> &b) {
        return std::lexicographical_compare(a.begin(), a.end(), b.begin(), b.end());
    }

    void evaluate(int v, int top) {
        State &out = memo[key(v, top)];
        const int nc = child_off[v + 1] - child_off[v];
        if (nc == 0) {
            out.total = count_cost(nreq[v], v, top);
            out.done = true;
            return;
        }
        const int ct = child_top(v, top);
        if (!cube) {
            auto &g = greedy_push[key(v, top)];
            double kids = 0.0;
            for (int i = child_off[v]; i < child_off[v + 1]; ++i) {
                const int c = child_idx[i];
                bool p = false;
                for (int32_t x : g.first) p |= x == c;
                kids = kids + memo[key(c, p ? ct : -1)].total;
            }
            out.total = count_cost(g.second, v, top) + kids;
            out.pushed = g.first;
            out.done = true;
            return;
        }
        // Subset DP over the children: a table keyed by requests removed, kept
        // in insertion order.  Each entry's pushed children are a linked list
        // shared with the entry it grew from (links[i] = child, previous link),
        // so extending an entry costs O(1); full lists are built only to break
        // ties between final candidates.
        struct Entry {
            int64_t removed;
            double subtotal;
            int32_t list;  // last link of the pushed children, -1: none
        };
        std::vector<std::pair<int32_t, int32_t>> links;
        std::vector<Entry> table{{0, 0.0, -1}}, nxt;
        std::vector<int32_t> pos((size_t)nreq[v] + 1, -1);
        for (int i = child_off[v]; i < child_off[v + 1]; ++i) {
            const int c = child_idx[i];
            const int64_t cnt = nreq[c];
            const double alone = memo[key(c, -1)].total, joined = memo[key(c, ct)].total;
            nxt.clear();
            for (const Entry &e : table) {
                for (int opt = 0; opt < 2; ++opt) {
                    const int64_t slot = e.removed + (opt ? cnt : 0);
                    const double value = e.subtotal + (opt ? joined : alone);
                    int32_t &at = pos[slot];
                    if (at < 0 || value < nxt[at].subtotal) {
                        int32_t list = e.list;
                        if (opt) {
                            links.emplace_back(c, e.list);
                            list = (int32_t)links.size() - 1;
                        }
                        if (at < 0) {
                            at = (int32_t)nxt.size();
                            nxt.push_back({slot, value, list});
                        } else {
                            nxt[at].subtotal = value;
                            nxt[at].list = list;
                        }
                    }
                }
            }
            for (const Entry &e : nxt) pos[e.removed] = -1;
            std::swap(table, nxt);
        }
        auto unroll = [&](int32_t list) {
            std::vector<int32_t> out;
            for (; list >= 0; list = links[list].second) out.push_back(links[list].first);
            std::reverse(out.begin(), out.end());
            return out;
        };
        int32_t best = -1;
        double best_cost = 0.0;
        for (const Entry &e : table) {
            const double cand = e.subtotal + count_cost(nreq[v] - e.removed, v, top);
            if (best < 0 || cand < best_cost ||
                (cand == best_cost && less_pushed(unroll(e.list), unroll(table[best].list)))) {
                best = (int32_t)(&e - table.data());
                best_cost = cand;
            }
        }
        out.total = best_cost;
        out.pushed = unroll(table[best].list);
        out.done = true;
    }

    // dependencies of state (v, top), as the Python planner visits them
    void deps(int v, int top, std::vector<std::pair<int, int>> &d) {
        d.clear();
        const int nc = child_off[v + 1] - child_off[v];
        if (!nc) return;
        const int ct = child_top(v, top);
        if (cube) {
            for (int i = child_off[v]; i < child_off[v + 1]; ++i) {
                d.emplace_back(child_idx[i], -1);
                d.emplace_back(child_idx[i], ct);
            }
            return;
        }
        auto it = greedy_push.find(key(v, top));
        if (it == greedy_push.end()) {
            std::vector<int32_t> pushed;
            int64_t remaining;
            greedy_choice(v, top, ct, pushed, remaining);
            it = greedy_push.emplace(key(v, top), std::make_pair(pushed, remaining)).first;
        }
        for (int i = child_off[v]; i < child_off[v + 1]; ++i) {
            const int c = child_idx[i];
            bool p = false;
            for (int32_t x : it->second.first) p |= x == c;
            d.emplace_back(c, p ? ct : -1);
        }
    }

    void run() {
        std::vector<std::pair<int, int>> stack{{0, -1}}, d;
        while (!stack.empty()) {
            const auto [v, top] = stack.back();
            if (memo[key(v, top)].done) {
                stack.pop_back();
                continue;
            }
            deps(v, top, d);
            bool missing = false;
            for (auto it = d.rbegin(); it != d.rend(); ++it)
                if (!memo[key(it->first, it->second)].done) {
                    stack.push_back(*it);
                    missing = true;
                }
            if (missing) continue;
            evaluate(v, top);
            stack.pop_back();
        }
    }
};

}  // namespace

// Grouped plan decisions for a tree of n nodes (node 0 is the root).
//   method: 0 greedy, 1 cube (subset DP)
//   parent[n]; children of v: child_idx[child_off[v] .. child_off[v+1])
//   nreq[v]: requests passing through node v
//   node runs: (run_start[i], run_len[i]) for i in [run_off[v], run_off[v+1])
//   model: bandwidth, cube_flops, task_us, merge_us; ints: cube_rows,
//     key_tile, kv_split, max_query_rows, qheads, kvheads, dim
// Writes pushed[v] = 1 if, in the state the materialisation reaches, node v's
// parent pushes it (v inherits the parent's chain), else 0; total[0] = the
// DP's estimate of the root state.  Returns 0, or 1 for invalid arguments.
extern "C" int tp_grouped_plan(int32_t method, int32_t n, const int32_t *parent, const int32_t *child_off,
                    const int32_t *child_idx, const int32_t *nreq, const int64_t *run_off,
                    const int64_t *run_start, const int64_t *run_len, const double *fparams,
                    const int64_t *iparams, int8_t *pushed, double *total) {
    if (n <= 0 || !parent || !child_off || !child_idx || !nreq || !run_off || !run_start || !run_len || !fparams ||
        !iparams || !pushed || !total || (method != 0 && method != 1))
        return 1;
    const Model m{fparams[0], fparams[1], fparams[2], fparams[3], iparams[0], iparams[1], iparams[2],
                  iparams[3], iparams[4], iparams[5], iparams[6]};
    if (m.kv_split <= 0 || m.max_query_rows <= 0 || m.kvheads <= 0 || m.qheads % m.kvheads || m.key_tile <= 0 ||
        m.cube_rows <= 0)
        return 1;
    // the tree's shape: children in range and after their parent, sibling
    // request sets no larger than the parent's (the DP indexes by counts)
    if (parent[0] != -1 || child_off[0] != 0) return 1;
    for (int v = 0; v < n; ++v) {
        if (nreq[v] < 0 || child_off[v + 1] < child_off[v] || run_off[v + 1] < run_off[v]) return 1;
        int64_t below = 0;
        for (int i = child_off[v]; i < child_off[v + 1]; ++i) {
            const int c = child_idx[i];
            if (c <= v || c >= n || parent[c] != v) return 1;
            below += nreq[c];
        }
        if (below > nreq[v]) return 1;
        for (int64_t i = run_off[v]; i < run_off[v + 1]; ++i)
            if (run_len[i] <= 0) return 1;
    }
    if (child_off[n] != n - 1) return 1;
    const int64_t group = m.qheads / m.kvheads;
    Planner p{m, n, parent, child_off, child_idx, nreq, run_off, run_start, run_len,
              std::max<int64_t>(1, m.max_query_rows / group), method == 1};
    p.run();
    // materialise decisions in pre-order from (0, none)
    for (int v = 0; v < n; ++v) pushed[v] = 0;
    std::vector<std::pair<int, int>> todo{{0, -1}};
    while (!todo.empty()) {
        const auto [v, top] = todo.back();
        todo.pop_back();
        const auto &st = p.memo[p.key(v, top)];
        const int ct = p.child_top(v, top);
        for (int i = p.child_off[v]; i < p.child_off[v + 1]; ++i) {
            const int c = p.child_idx[i];
            bool in = false;
            for (int32_t x : st.pushed) in |= x == c;
            pushed[c] = in;
            todo.emplace_back(c, in ? ct : -1);
        }
    }
    total[0] = p.memo[p.key(0, -1)].total;
    return 0;
}

// Attachment of small segments to 256-row work items (tree_attention/kernels.py
// _attach_tails): candidate jobs go, in order, to the candidate item (a 256-row
// item of a large job whose requests include the candidate's, at consecutive
// rows that lie in one wave) with the fewest attached tiles, then the fewest on
// the owning wave, then the lowest large job, within `xtail_max` segments and
// the item's own tile count.
//   large jobs J < n_large: is256[J], tiles[J], requests req[req_off[J] .. req_off[J+1])
//   candidate jobs s < n_small: requests sreq[sreq_off[s] .. sreq_off[s+1]), tiles_s[s], fixed[s]
// Writes item[s] (index into the item list, -1: not attached) and lrow[s]
// (first job row of the candidate's requests), the item list (item_job,
// item_row0) and n_items[0].  Returns 0, or 1 for invalid arguments.
extern "C" int tp_attach_tails(int32_t n_large, const int32_t *is256, const int32_t *tiles, const int32_t *req_off,
                               const int32_t *req, int32_t group, int32_t n_small, const int32_t *sreq_off,
                               const int32_t *sreq, const int32_t *tiles_s, const int8_t *fixed, int32_t nreq,
                               int32_t xtail_max, int32_t wave_rows, int32_t item_rows, int32_t min_cap,
                               int32_t *item, int32_t *lrow, int32_t *item_job, int32_t *item_row0,
                               int32_t *n_items) {
    if (n_large < 0 || n_small < 0 || nreq <= 0 || group <= 0 || xtail_max < 0 || wave_rows <= 0 || min_cap < 0 ||
        item_rows <= 0 || item_rows % wave_rows || (n_large && (!is256 || !tiles || !req_off || !req)) ||
        (n_small && (!sreq_off || !sreq || !tiles_s || !fixed || !item || !lrow)) || !item_job || !item_row0 ||
        !n_items)
        return 1;
    struct Cand {
        int32_t job, item, wave, lrow;
    };
    std::vector<std::vector<Cand>> holders(nreq);
    std::vector<int32_t> own;
    int32_t ni = 0;
    for (int32_t j = 0; j < n_large; ++j) {
        if (req_off[j + 1] < req_off[j]) return 1;
        if (!is256[j]) continue;
        const int64_t rows = (int64_t)(req_off[j + 1] - req_off[j]) * group;
        const int32_t first = ni;
        for (int64_t r0 = 0; r0 < rows; r0 += item_rows) {
            item_job[ni] = j;
            item_row0[ni] = (int32_t)r0;
            own.push_back(tiles[j]);
            ++ni;
        }
        for (int32_t pos = req_off[j]; pos < req_off[j + 1]; ++pos) {
            const int32_t r = req[pos];
            if (r < 0 || r >= nreq) return 1;
            const int32_t lr = (pos - req_off[j]) * group;
            if (lr % wave_rows + group <= wave_rows)
                holders[r].push_back({j, first + lr / item_rows, lr % item_rows / wave_rows, lr});
        }
    }
    n_items[0] = ni;
    const int waves = item_rows / wave_rows;
    std::vector<int32_t> item_tiles(ni, 0), item_segs(ni, 0), wave_tiles((size_t)ni * waves, 0);
    for (int32_t s = 0; s < n_small; ++s) {
        item[s] = -1;
        lrow[s] = 0;
        const int32_t nr = sreq_off[s + 1] - sreq_off[s];
        if (nr <= 0 || fixed[s]) continue;
        const int32_t *sr = sreq + sreq_off[s];
        const int32_t r = sr[0];
        if (r < 0 || r >= nreq) continue;
        const int32_t n = tiles_s[s];
        const Cand *best = nullptr;
        int32_t bt = 0, bw = 0;
        for (const Cand &c : holders[r]) {
            // every request of the candidate at the next rows of the same wave
            if (c.lrow % wave_rows + (int64_t)nr * group > wave_rows) continue;
            const int32_t pos = req_off[c.job] + c.lrow / group;
            if (pos + nr > req_off[c.job + 1]) continue;
            bool same = true;
            for (int32_t i = 1; i < nr && same; ++i) same = req[pos + i] == sr[i];
            if (!same) continue;
            const int32_t t = item_tiles[c.item];
            if (item_segs[c.item] >= xtail_max || t + n > std::max(own[c.item], min_cap)) continue;
            const int32_t w = wave_tiles[(size_t)c.item * waves + c.wave];
            if (!best || t < bt || (t == bt && (w < bw || (w == bw && c.job < best->job)))) {
                best = &c;
                bt = t;
                bw = w;
            }
        }
        if (!best) continue;
        item[s] = best->item;
        lrow[s] = best->lrow;
        item_tiles[best->item] += n;
        item_segs[best->item] += 1;
        wave_tiles[(size_t)best->item * waves + best->wave] += n;
    }
    return 0;
}

// Device metadata of a prepared plan (tree_attention/kernels.py prepare): every
// int32 section the kernels read, in one buffer, in this order --
//   qids[njobs*maxr] kids[njobs] qlen[njobs] klen[njobs] slots[nreq*maxs]
//   counts[nreq] rowbase[njobs] rest[n_rest] xtail[n_l256 * xstride]
//   qbase[njobs] items of kinds 0 .. 4 (triples)
// Jobs 0 .. small_jobs-1 are the small ones.  A small job of one request that
// is its request's only small job is a tail: its items have kind tail and its
// slot goes last in the request's list (its work item merges the others
// first); rest is every other request.  Large jobs get row tiles by their row
// count (64, 128 or 256 rows, at most tile_rows); 256-row items are ordered by
// KV head, then job, then first row, the others by job, head, first row.
// Attachments: n_att records of xstride ints (count, then first token, tokens,
// first job row per segment) for the 256-row items of (att_job, att_row0).
// sizes (out, 13 ints): maxr, maxs, nslot, n_rest, n_items[5], contiguous_q,
// slot_stride, total length, n_l256.  buf == NULL: sizes only.  Returns 0, 1
// for invalid arguments (a request outside [0, nreq)), 2 when buf_len is short.
extern "C" int tp_build_metadata(int32_t njobs, int32_t small_jobs, const int32_t *qlen, const int32_t *req,
                                 const int32_t *kstart, const int32_t *klen, int32_t nreq, int32_t group,
                                 int32_t kvheads, int32_t tile_rows, int32_t n_att, const int32_t *att_job,
                                 const int32_t *att_row0, const int32_t *att_rec, int32_t xstride, int32_t *sizes,
                                 int32_t *buf, int64_t buf_len) {
    if (njobs <= 0 || small_jobs < 0 || small_jobs > njobs || nreq <= 0 || group <= 0 || kvheads <= 0 ||
        xstride <= 0 || n_att < 0 || !qlen || !req || !kstart || !klen || !sizes || (n_att && (!att_job || !att_row0 || !att_rec)))
        return 1;
    std::vector<int64_t> rowbase(njobs);
    int64_t nslot = 0;
    int32_t maxr = 0;
    for (int32_t j = 0; j < njobs; ++j) {
        if (qlen[j] <= 0) return 1;
        rowbase[j] = nslot;
        nslot += qlen[j];
        maxr = std::max(maxr, qlen[j]);
    }
    std::vector<int32_t> counts(nreq, 0);
    for (int64_t s = 0; s < nslot; ++s) {
        if (req[s] < 0 || req[s] >= nreq) return 1;
        ++counts[req[s]];
    }
    int32_t maxs = 1;
    for (int32_t c : counts) maxs = std::max(maxs, c);
    // tails: single-request small jobs whose request has no other small job
    std::vector<int32_t> owners(nreq, 0);
    for (int32_t j = 0; j < small_jobs; ++j)
        for (int64_t s = rowbase[j]; s < rowbase[j] + qlen[j]; ++s) ++owners[req[s]];
    std::vector<char> is_tail(njobs, 0), tail_req(nreq, 0);
    for (int32_t j = 0; j < small_jobs; ++j)
        if (qlen[j] == 1 && owners[req[rowbase[j]]] == 1) {
            is_tail[j] = 1;
            tail_req[req[rowbase[j]]] = 1;
        }
    int32_t n_rest = 0;
    for (int32_t r = 0; r < nreq; ++r) n_rest += !tail_req[r];
    // row tiles of the large jobs
    // jobs of 65 .. 256 rows take 256-row items (the pipelined kernel, which
    // also attends attached segments) unless tile_rows caps the tile lower
    auto kind_of = [&](int64_t rows) {
        if (rows <= 64 || tile_rows <= 64) return 1;
        if (tile_rows <= 128) return 2;
        return 3;
    };
    static const int tile_of[4] = {0, 64, 128, 256};
    int64_t n_items[5] = {0, 0, 0, 0, 0};
    for (int32_t j = 0; j < njobs; ++j) {
        if (j < small_jobs) {
            n_items[is_tail[j] ? 4 : 0] += kvheads;
            continue;
        }
        const int64_t rows = (int64_t)qlen[j] * group;
        const int k = kind_of(rows);
        n_items[k] += (rows + tile_of[k] - 1) / tile_of[k] * kvheads;
    }
    const int64_t n256 = n_items[3];
    const int64_t total = (int64_t)njobs * maxr + 3 * (int64_t)njobs + (int64_t)nreq * maxs + nreq + njobs + n_rest +
                          (n_att ? n256 * xstride : 0) + njobs +
                          3 * (n_items[0] + n_items[1] + n_items[2] + n_items[3] + n_items[4]);
    // qbase and the span test
    bool contiguous = true;
    std::vector<int32_t> qbase(njobs);
    for (int32_t j = 0; j < njobs; ++j) {
        const int32_t *r = req + rowbase[j];
        const int32_t n = qlen[j];
        contiguous &= r[n - 1] - r[0] + 1 == n;
        bool consec = true;
        for (int32_t i = 1; i < n && consec; ++i) consec = r[i] == r[i - 1] + 1;
        qbase[j] = consec ? r[0] : -1;
    }
    // slot lists (positions in job order), the tail slot rotated last
    std::vector<int64_t> start(nreq + 1, 0);
    for (int32_t r = 0; r < nreq; ++r) start[r + 1] = start[r] + counts[r];
    std::vector<int32_t> slot(nslot);
    {
        std::vector<int64_t> fill(start.begin(), start.end() - 1);
        for (int64_t s = 0; s < nslot; ++s) slot[fill[req[s]]++] = (int32_t)s;
    }
    for (int32_t r = 0; r < nreq; ++r)
        if (tail_req[r] && counts[r] > 1) std::rotate(slot.begin() + start[r], slot.begin() + start[r] + 1,
                                                       slot.begin() + start[r + 1]);
    int32_t stride = 0;
    if (maxs > 1) {
        bool even = true;
        for (int32_t c : counts) even &= c == maxs;
        const int32_t st = even ? slot[1] - slot[0] : 0;
        if (st > 0) {
            bool affine = true;
            for (int32_t r = 0; r < nreq && affine; ++r)
                for (int32_t k = 0; k < maxs && affine; ++k) affine = slot[start[r] + k] == r + k * st;
            stride = affine ? st : 0;
        }
    }
    const int32_t out_sizes[13] = {maxr, maxs, (int32_t)nslot, n_rest, (int32_t)n_items[0], (int32_t)n_items[1],
                                   (int32_t)n_items[2], (int32_t)n_items[3], (int32_t)n_items[4], contiguous ? 1 : 0,
                                   stride, (int32_t)total, (int32_t)n256};
    std::copy(out_sizes, out_sizes + 13, sizes);
    if (!buf) return 0;
    if (buf_len < total) return 2;
    std::fill(buf, buf + total, 0);
    int32_t *p = buf;
    for (int32_t j = 0; j < njobs; ++j)  // qids
        std::copy(req + rowbase[j], req + rowbase[j] + qlen[j], p + (int64_t)j * maxr);
    p += (int64_t)njobs * maxr;
    std::copy(kstart, kstart + njobs, p);
    p += njobs;
    std::copy(qlen, qlen + njobs, p);
    p += njobs;
    std::copy(klen, klen + njobs, p);
    p += njobs;
    for (int32_t r = 0; r < nreq; ++r)  // slots
        std::copy(slot.begin() + start[r], slot.begin() + start[r + 1], p + (int64_t)r * maxs);
    p += (int64_t)nreq * maxs;
    std::copy(counts.begin(), counts.end(), p);
    p += nreq;
    for (int32_t j = 0; j < njobs; ++j) p[j] = (int32_t)rowbase[j];
    p += njobs;
    for (int32_t r = 0; r < nreq; ++r)  // rest
        if (!tail_req[r]) *p++ = r;
    // items, then the attachment records of the 256-row items
    int32_t *items[5];
    int32_t *q = p + (n_att ? n256 * xstride : 0) + njobs;
    for (int k = 0; k < 5; ++k) {
        items[k] = q;
        q += 3 * n_items[k];
    }
    auto put = [&](int k, int32_t j, int32_t row0, int32_t h) {
        items[k][0] = j;
        items[k][1] = row0;
        items[k][2] = h;
        items[k] += 3;
    };
    for (int32_t j = 0; j < small_jobs; ++j)
        for (int32_t h = 0; h < kvheads; ++h) put(is_tail[j] ? 4 : 0, j, 0, h);
    for (int32_t j = small_jobs; j < njobs; ++j) {  // 64- and 128-row kinds: job, head, first row
        const int64_t rows = (int64_t)qlen[j] * group;
        const int k = kind_of(rows);
        if (k == 3) continue;
        for (int32_t h = 0; h < kvheads; ++h)
            for (int64_t r0 = 0; r0 < rows; r0 += tile_of[k]) put(k, j, (int32_t)r0, h);
    }
    int32_t *big = items[3];
    for (int32_t h = 0; h < kvheads; ++h)  // 256-row kind: head, job, first row
        for (int32_t j = small_jobs; j < njobs; ++j) {
            const int64_t rows = (int64_t)qlen[j] * group;
            if (kind_of(rows) != 3) continue;
            for (int64_t r0 = 0; r0 < rows; r0 += 256) put(3, j, (int32_t)r0, h);
        }
    if (n_att) {
        for (int64_t i = 0; i < n256; ++i) {
            const int32_t j = big[3 * i], r0 = big[3 * i + 1];
            for (int32_t a = 0; a < n_att; ++a)
                if (att_job[a] == j && att_row0[a] == r0) {
                    std::copy(att_rec + (int64_t)a * xstride, att_rec + (int64_t)(a + 1) * xstride,
                              p + i * xstride);
                    break;
                }
        }
        p += n256 * xstride;
    }
    std::copy(qbase.begin(), qbase.end(), p);
    return 0;
}

// tree_attn.hip -- gfx950 (CDNA4) kernels for tree-shared decode attention.
//
// Replaces the Triton kernels of the reference's src/tree_attention/kernels.py:
//   _segment (kernels.py:8-55): grouped partial attention of one physical KV
//     segment for every request of its job, online softmax in fp32, P rounded
//     to the input dtype before PV (kernels.py:49), writes acc/z and m + ln z.
//   _merge (kernels.py:58-83): per (request, query head) log-sum-exp merge of
//     the request's partial outputs, cast to the input dtype.
//
// Design (MI355X-first, not a translation of the Triton tiling):
//   * K/V of a job are streamed from HBM once per work item in 64-token tiles
//     by all 256 threads (coalesced 16-byte loads), transposed 8x8 in
//     registers and written to LDS as Kt[token][d] and Vt[d][token], the
//     operand orders the MFMA needs.  The next tile's global loads are issued
//     before the current tile is computed.
//   * QK^T is computed transposed, S^T = K Q^T, with
//     v_mfma_f32_16x16x32_{bf16,f16}: the C layout then gives each lane four
//     consecutive tokens of one query row, which is exactly the B operand of
//     the PV product O^T = V^T P^T -- P never leaves registers.
//   * Small jobs (<= 16 query rows, e.g. one request x 4 GQA heads): the four
//     waves split every tile's tokens (16 each), keep private (m, z, O) and
//     combine once through LDS at the end.  PV uses 16x16x16 MFMA.
//   * Large jobs: the four waves split the query rows (NB blocks of 16 rows per
//     wave) and share every staged K/V tile; each K/V fragment read from LDS
//     feeds NB MFMAs.  Work items are (job, row tile, head) and are remapped
//     so that tiles of the same (job, head) land on the same XCD back to back
//     and share its L2.
//   * Softmax runs in base 2 with log2(e)/sqrt(D) folded into one FMA.
//   * Partial rows are stored as fp16 scaled by a power of two per row (the
//     exponent sits next to the log-sum-exp); the merge reads them with
//     8-byte loads, one thread per four head-dim elements, and folds the
//     scale into each slot's weight.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "ta_common.h"
#include "tree_attn.h"

namespace {

using namespace ta;


// ------------------------------------------------------- tile staging (LDS)
// One TTILE-token tile of one KV head: Kt[TTILE][D] (+pad) and Vt[D][TTILE]
// (+pad), built from 8x8 element blocks that NTHR threads load with 16-byte
// global loads, transpose in registers and store with 16-byte LDS writes.
template <int D, int TTILE, int NTHR>
struct Stage {
    // Row strides (elements).  Kt rows are read 16 B per lane, 8 lanes per LDS
    // cycle: D + 8 shifts consecutive rows by 4 banks.  Vt rows are read 8 B per
    // lane, 16 lanes per cycle: TTILE + 4 shifts consecutive rows by 2 banks, so
    // 16 rows cover all 32 banks once.
    static constexpr int KS = D + 8;
    static constexpr int VS = TTILE + 4;
    static constexpr int KELEMS = TTILE * KS;
    static constexpr int ELEMS = KELEMS + D * VS;
    static constexpr int DG = D / 8;
    static constexpr int TG = TTILE / 8;
    static constexpr int KBLK = DG * TG;  // 8x8 blocks per operand
    static constexpr int NBLK = 2 * KBLK;
    static constexpr int BPT = (NBLK + NTHR - 1) / NTHR;  // blocks per thread

    u32x4 r[BPT][8];

    __device__ static u32x4 load_tail(const u16 *p, int valid) {
        u32 w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const u32 lo = (2 * k < valid) ? (u32)p[2 * k] : 0u;
            const u32 hi = (2 * k + 1 < valid) ? (u32)p[2 * k + 1] : 0u;
            w[k] = lo | (hi << 16);
        }
        return u32x4{w[0], w[1], w[2], w[3]};
    }

    // Global -> registers.  Tokens [t0, t0 + nvalid) are read; the rest of the
    // tile is zero (zero V keeps masked columns finite in PV).
    __device__ void load(const u16 *__restrict__ kp, const u16 *__restrict__ vp, int h, int tcap, int t0,
                         int nvalid, bool kaligned, int tid) {
        if (kaligned && nvalid >= TTILE) {
            // full, 16-byte aligned tile: unconditional vector loads (wave-uniform branch)
#pragma unroll
            for (int j = 0; j < BPT; ++j) {
                const int b = tid + j * NTHR;
                if (b < KBLK) {
                    const int dg = b % DG, tg = b / DG;
                    const u16 *base = kp + ((size_t)(h * D + 8 * dg) * tcap + t0 + 8 * tg);
#pragma unroll
                    for (int i = 0; i < 8; ++i) r[j][i] = *(const u32x4 *)(base + (size_t)i * tcap);
                } else if (b < NBLK) {
                    const int u = b - KBLK;
                    const int tg = u % TG, dg = u / TG;
                    const u16 *base = vp + ((size_t)(h * tcap + t0 + 8 * tg) * D + 8 * dg);
#pragma unroll
                    for (int i = 0; i < 8; ++i) r[j][i] = *(const u32x4 *)(base + i * D);
                }
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
            const int b = tid + j * NTHR;
            if (b < KBLK) {
                const int dg = b % DG, tg = b / DG;
                const u16 *base = kp + ((size_t)(h * D + 8 * dg) * tcap + t0 + 8 * tg);
                const int valid = nvalid - 8 * tg;
                if (kaligned && valid >= 8) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) r[j][i] = *(const u32x4 *)(base + (size_t)i * tcap);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) r[j][i] = load_tail(base + (size_t)i * tcap, valid);
                }
            } else if (b < NBLK) {
                const int u = b - KBLK;
                const int tg = u % TG, dg = u / TG;
                const u16 *base = vp + ((size_t)(h * tcap + t0 + 8 * tg) * D + 8 * dg);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    r[j][i] = (8 * tg + i < nvalid) ? *(const u32x4 *)(base + (size_t)i * D) : u32x4{0, 0, 0, 0};
            }
        }
    }

    // 8x8 transpose of 16-bit elements: o[c] = column c of the rows in in[].
    __device__ static void transpose(const u32x4 (&in)[8], u32x4 (&o)[8]) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            u32 w[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const u32 a = in[2 * k][c >> 1], b = in[2 * k + 1][c >> 1];
                w[k] = (c & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
            }
            o[c] = u32x4{w[0], w[1], w[2], w[3]};
        }
    }

    // Registers -> LDS in MFMA operand order.
    __device__ void store(u16 *lds, int tid) const {
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
            const int b = tid + j * NTHR;
            if (b >= NBLK) continue;
            u32x4 o[8];
            transpose(r[j], o);
            if (b < KBLK) {
                const int dg = b % DG, tg = b / DG;
#pragma unroll
                for (int c = 0; c < 8; ++c) *(u32x4 *)(lds + (8 * tg + c) * KS + 8 * dg) = o[c];
            } else {
                const int u = b - KBLK;
                const int tg = u % TG, dg = u / TG;
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    u16 *dst = lds + KELEMS + (8 * dg + c) * VS + 8 * tg;  // 8-byte aligned
                    *(u32x2 *)dst = u32x2{o[c][0], o[c][1]};
                    *(u32x2 *)(dst + 4) = u32x2{o[c][2], o[c][3]};
                }
            }
        }
    }
};

// Query fragment of one 16-row block: lane (row, g4) holds d = 32*ks + 8*g4 .. +7.
template <int D>
__device__ inline void load_q(const SegParams &p, int job, int h, int row, int nrows, int g4,
                              u32x4 (&qf)[D / 32]) {
    if (row < nrows) {
        const int lr = row / p.group, gg = row - lr * p.group;
        const int rq = p.qids[(size_t)job * p.maxr + lr];
        const u16 *src = p.q + ((size_t)rq * p.hq + h * p.group + gg) * D + 8 * g4;
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) qf[ks] = *(const u32x4 *)(src + 32 * ks);
    } else {
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) qf[ks] = u32x4{0, 0, 0, 0};
    }
}

// Online-softmax state of NB 16-row blocks held by one wave.  Lane (row, g4)
// keeps the shared (stale) maximum m of its row, a partial denominator z over
// its own columns and O^T[d = 16*db + 4*g4 + i][row] in o[nb][db][i].
template <int D, int NB>
struct RowState {
    float m[NB], z[NB];
    f32x4 o[NB][D / 16];

    __device__ void reset() {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            m[nb] = NEG_INF;
            z[nb] = 0.f;
#pragma unroll
            for (int db = 0; db < D / 16; ++db) o[nb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
};

// S^T = K Q^T for one 32-token step: s[nb][b][i] is the score of token
// 16*b + 4*g4 + i (relative to kt) against row 16*nb + row.
template <int D, bool FP16, int NB, int KS>
__device__ inline void qk_step(const u16 *kt, int row, int g4, const u32x4 (&qf)[NB][D / 32], f32x4 (&s)[NB][2]) {
    using O = Ops<FP16>;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) s[nb][0] = s[nb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            const u32x4 a = *(const u32x4 *)(kt + (16 * b + row) * KS + 32 * ks + 8 * g4);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) s[nb][b] = O::mma_k32(a, qf[nb][ks], s[nb][b]);
        }
    }
}

// Softmax update and O^T += V^T P^T for one 32-token step with nvs valid
// tokens.  PV k-slot j of lane group g4 is token 4*g4 + j (j < 4) or
// 16 + 4*g4 + j - 4 (j >= 4), which is where the QK output left P.
template <int D, bool FP16, int NB, int VS>
__device__ inline void pv_step(const u16 *vt, int row, int g4, f32x4 (&s)[NB][2], int nvs, float c,
                               RowState<D, NB> &st) {
    using O = Ops<FP16>;
    u32x4 vf[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        const u16 *vr = vt + (16 * db + row) * VS + 4 * g4;
        const u32x2 lo = *(const u32x2 *)vr;
        const u32x2 hi = *(const u32x2 *)(vr + 16);
        vf[db] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
    const bool full = nvs >= 32;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        float x[8];
        float lm = NEG_INF;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v = s[nb][b][i];
                if (!full && 16 * b + 4 * g4 + i >= nvs) v = NEG_INF;
                x[4 * b + i] = v;
                lm = fmaxf(lm, v);
            }
        const bool need = lm * c > st.m[nb] + TAU;
        if (__builtin_amdgcn_ballot_w64(need)) {  // wave-uniform, rare after the first step
            const float mn = fmaxf(st.m[nb], xor_max(lm) * c);
            const float alpha = fast_exp2(st.m[nb] - mn);
            st.z[nb] *= alpha;
#pragma unroll
            for (int db = 0; db < D / 16; ++db) st.o[nb][db] *= alpha;
            st.m[nb] = mn;
        }
        float pr[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) pr[i] = fast_exp2(__builtin_fmaf(x[i], c, -st.m[nb]));
        st.z[nb] += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
        const u32x4 pb = {O::pack(pr[0], pr[1]), O::pack(pr[2], pr[3]), O::pack(pr[4], pr[5]),
                          O::pack(pr[6], pr[7])};
#pragma unroll
        for (int db = 0; db < D / 16; ++db) st.o[nb][db] = O::mma_k32(vf[db], pb, st.o[nb][db]);
    }
}

// Normalise and store the partial rows of NB 16-row blocks (rows >= nrows skipped).
template <int D, int NB>
__device__ inline void store_rows(const SegParams &p, RowState<D, NB> &st, int job, int h, int wrow0, int nrows,
                                  int row, int g4) {
    const int rb = p.rowbase[job];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const float zr = xor_sum(st.z[nb]);
        const int grow = wrow0 + 16 * nb + row;
        if (grow >= nrows) continue;
        const int lr = grow / p.group, gg = grow - lr * p.group;
        const size_t prow = (size_t)(rb + lr) * p.hq + h * p.group + gg;
        store_partial<D / 16>(p.part, p.lse, prow, st.o[nb], st.m[nb], zr, g4);
    }
}

// --------------------------------------------------------- small segments
// Jobs with at most 16 query rows (e.g. one request's private tail).  One
// wave per workgroup walks a strided list of (job, KV head) items; 32-token
// tiles go through wave-private LDS and the next tile -- of the same item or
// of the next one -- is already in flight while the current one is computed.
constexpr int SMALL_TT = 32;
constexpr int SMALL_NT = 64;

template <int D, bool FP16>
__global__ __launch_bounds__(SMALL_NT) void seg_small_kernel(SegParams p) {
    using S = Stage<D, SMALL_TT, SMALL_NT>;
    __shared__ __attribute__((aligned(16))) u16 lds[S::ELEMS];
    const int lane = threadIdx.x;
    const int row = lane & 15, g4 = lane >> 4;
    const int total = p.n_items;
    const float c = p.scale_log2;
    const int stride = gridDim.x;

    struct Item {
        int job, h, kst, ntok, ntiles;
        bool kal;
    };
    auto decode = [&](int idx) {
        Item it;
        it.job = p.items[3 * idx];
        it.h = p.items[3 * idx + 2];
        it.kst = p.kstart[it.job];
        it.ntok = max(0, min(p.klen[it.job], p.tcap - it.kst));
        it.ntiles = (it.ntok + SMALL_TT - 1) / SMALL_TT;
        it.kal = ((p.tcap | it.kst) & 7) == 0;
        return it;
    };

    S st;
    // prefetch cursor: (pidx, ptile) is the tile whose loads sit in st.r
    int pidx = blockIdx.x, ptile = 0;
    Item pit;
    while (pidx < total) {
        pit = decode(pidx);
        if (pit.ntiles > 0) break;
        pidx += stride;
    }
    if (pidx < total)
        st.load(p.kp, p.vp, pit.h, p.tcap, pit.kst, min(pit.ntok, SMALL_TT), pit.kal, lane);

    RowState<D, 1> rs;
    u32x4 qf[1][D / 32];
    for (int idx = blockIdx.x; idx < total; idx += stride) {
        const Item it = decode(idx);
        const int nrows = min(p.qlen[it.job] * p.group, 16);
        load_q<D>(p, it.job, it.h, row, nrows, g4, qf[0]);
        rs.reset();
        for (int t = 0; t < it.ntiles; ++t) {
            __syncthreads();
            st.store(lds, lane);
            __syncthreads();
            // advance the prefetch cursor and issue the next tile's loads
            if (++ptile >= pit.ntiles) {
                ptile = 0;
                for (pidx += stride; pidx < total; pidx += stride) {
                    pit = decode(pidx);
                    if (pit.ntiles > 0) break;
                }
            }
            if (pidx < total) {
                const int t0 = ptile * SMALL_TT;
                st.load(p.kp, p.vp, pit.h, p.tcap, pit.kst + t0, min(pit.ntok - t0, SMALL_TT), pit.kal, lane);
            }
            f32x4 s[1][2];
            qk_step<D, FP16, 1, S::KS>(lds, row, g4, qf, s);
            pv_step<D, FP16, 1, S::VS>(lds + S::KELEMS, row, g4, s, it.ntok - t * SMALL_TT, c, rs);
        }
        store_rows<D, 1>(p, rs, it.job, it.h, 0, nrows, row, g4);
    }
}

// --------------------------------------------------------- large segments
// One workgroup (NW waves) per (job, row tile of 16*NB*NW rows, KV head);
// wave w owns rows [16*NB*w, 16*NB*(w+1)) of the tile.  TT-token K/V tiles
// are double-buffered in LDS (one barrier per tile) and every K/V fragment
// read from LDS feeds NB MFMAs.  Within a tile the next 32-token step's QK is
// issued before the current step's softmax so the matrix cores and the VALU
// have independent work; with 32 rows per wave everything stays in VGPRs and
// two waves share each SIMD.
template <int D, bool FP16, int NB, int NW, int TT>
__global__ __launch_bounds__(64 * NW) void seg_large_kernel(SegParams p) {
    constexpr int NTHR = 64 * NW;
    constexpr int STEPS = TT / 32;
    using S = Stage<D, TT, NTHR>;
    __shared__ __attribute__((aligned(16))) u16 lds[2 * S::ELEMS];

    // Linear block L runs on XCD L % 8; give every XCD a contiguous range of
    // items so neighbouring row tiles of one (job, head) share an L2.
    const int total = gridDim.x;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int q8 = total >> 3, rm = total & 7;
    const int v = xcd * q8 + min(xcd, rm) + slot;
    const int job = p.items[3 * v], row0 = p.items[3 * v + 1], h = p.items[3 * v + 2];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = lane & 15, g4 = lane >> 4;
    const int kst = p.kstart[job];
    const int ntok = max(0, min(p.klen[job], p.tcap - kst));
    const int nrows = p.qlen[job] * p.group;
    const int wrow0 = row0 + 16 * NB * wave;  // first row of this wave
    const bool active = wrow0 < nrows;
    const bool kal = ((p.tcap | kst) & 7) == 0;
    const float c = p.scale_log2;

    u32x4 qf[NB][D / 32];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) load_q<D>(p, job, h, wrow0 + 16 * nb + row, nrows, g4, qf[nb]);
    RowState<D, NB> rs;
    rs.reset();

    const int ntiles = (ntok + TT - 1) / TT;
    S st;
    if (ntiles > 0) {
        st.load(p.kp, p.vp, h, p.tcap, kst, min(ntok, TT), kal, tid);
        st.store(lds, tid);
    }
    if (ntiles > 1) st.load(p.kp, p.vp, h, p.tcap, kst + TT, min(ntok - TT, TT), kal, tid);
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {
        const u16 *cur = lds + (it & 1) * S::ELEMS;
        const int nv = ntok - it * TT;
        if (active) {
            f32x4 sc[2][NB][2];
            qk_step<D, FP16, NB, S::KS>(cur, row, g4, qf, sc[0]);
#pragma unroll
            for (int k = 0; k < STEPS; ++k) {
                const int base = 32 * k;
                if (base >= nv) break;
                if (k + 1 < STEPS && base + 32 < nv)
                    qk_step<D, FP16, NB, S::KS>(cur + (base + 32) * S::KS, row, g4, qf, sc[(k + 1) & 1]);
                pv_step<D, FP16, NB, S::VS>(cur + S::KELEMS + base, row, g4, sc[k & 1], nv - base, c, rs);
            }
        }
        if (it + 1 < ntiles) st.store(lds + ((it + 1) & 1) * S::ELEMS, tid);
        __syncthreads();
        if (it + 2 < ntiles) {
            const int t0 = (it + 2) * TT;
            st.load(p.kp, p.vp, h, p.tcap, kst + t0, min(ntok - t0, TT), kal, tid);
        }
    }
    if (active) store_rows<D, NB>(p, rs, job, h, wrow0, nrows, row, g4);
}

// ------------------------------------------------------------------ merge
// One workgroup of NT threads per (request, group of MH query heads);
// thread (head, d8) owns eight head-dim elements of one query head.  The slot
// list is uniform per workgroup (scalar loads), and each thread reads, for
// MERGE_CHUNK slots at once, the 16-byte partial slice (eight fp16 values) and
// the 8-byte (log-sum-exp, exponent) pair, then merges them online in
// registers: slots -> (lse, partials) is the only chain of dependent memory
// round trips; no LDS and no barriers.  With an affine slot layout
// (slot_stride > 0: slot k of request r is r + k * slot_stride, maxs of them)
// the slots are computed and the partial loads are the first memory access.
constexpr int MERGE_CHUNK = 16;
constexpr int MERGE_NT = 128;
// Below this many workgroups of MERGE_NT threads the merge runs groups of
// MERGE_NT / 2 threads instead (half the heads per workgroup, twice the
// workgroups): one workgroup per CU of the 256 leaves the GPU half empty, and
// a small batch's merge is one round trip of loads per workgroup.
constexpr int MERGE_FILL_BLOCKS = 256;

// SPLIT groups of NT threads split a request's slots into SPLIT
// contiguous ranges, merge them side by side (one round trip of loads per
// MERGE_CHUNK slots each) and combine their running (max, sum, partial sums)
// through LDS; the first group writes the output.  SPLIT = 2 serves plans with
// more than MERGE_CHUNK slots per request: 32 slots wait for one round of loads
// instead of two.  SPLIT = 1 is the single-group kernel described above.
template <int D, bool FP16, int SPLIT, int NT = MERGE_NT>
__global__ __launch_bounds__(NT * SPLIT) void merge_kernel(const u16 *__restrict__ part,
                                                                 const float *__restrict__ lse,
                                                                 const int32_t *__restrict__ slots,
                                                                 const int32_t *__restrict__ counts,
                                                                 const int32_t *__restrict__ reqs,
                                                                 u16 *__restrict__ out, int hq, int maxs,
                                                                 int slot_stride) {
    constexpr int TPH = D / 8;          // threads per head
    constexpr int MH = NT / TPH;  // heads per workgroup
    constexpr float LOG2E = 1.44269504088896341f;
    const int r = reqs ? reqs[blockIdx.x] : blockIdx.x;
    // a group is whole waves: readfirstlane tells the compiler grp is uniform
    const int grp = SPLIT > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x / NT) : 0;
    const int tid = threadIdx.x % NT;
    const int hl = tid / TPH, d8 = tid % TPH;
    const int head = blockIdx.y * MH + hl;
    const bool valid = head < hq;
    if (SPLIT == 1 && !valid) return;
    const int cnt = slot_stride > 0 ? maxs : counts[r];
    const int per = (cnt + SPLIT - 1) / SPLIT;
    const int beg = SPLIT > 1 ? min(cnt, grp * per) : 0, end = SPLIT > 1 ? min(cnt, beg + per) : cnt;
    const int hr = SPLIT > 1 ? min(head, hq - 1) : head;  // the head this lane reads
    const int32_t *slr = slots + (size_t)r * maxs;
    const u16 *src = part + (size_t)hr * D + 8 * d8;
    const float2 *lse2 = reinterpret_cast<const float2 *>(lse) + hr;
    const size_t srow = (size_t)hq * D;

    float M = NEG_INF, Z = 0.f;  // running max (log2 units) and weight sum
    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = lo;
    // the loop bounds stay uniform (so the slot list is read by scalar loads):
    // lanes past hq read head hq - 1 and store nothing
    for (int s0 = beg; s0 < end; s0 += MERGE_CHUNK) {
        float2 le[MERGE_CHUNK];
        u32x4 v[MERGE_CHUNK];
#pragma unroll
        for (int u = 0; u < MERGE_CHUNK; ++u) {
            const int k = min(s0 + u, end - 1);
            const int sl = slot_stride > 0 ? r + k * slot_stride : slr[k];
            // nontemporal: the partials are read once, and leaving them out of L2
            // keeps the next segment launch's metadata, Q and code there
            const f32x2 t = __builtin_nontemporal_load((const f32x2 *)(lse2 + (size_t)sl * hq));
            le[u] = float2(t[0], t[1]);
            v[u] = __builtin_nontemporal_load((const u32x4 *)(src + sl * srow));
        }
        float l[MERGE_CHUNK];
        float cm = M;
#pragma unroll
        for (int u = 0; u < MERGE_CHUNK; ++u) {
            l[u] = s0 + u < end ? le[u].x * LOG2E : NEG_INF;
            cm = fmaxf(cm, l[u]);
        }
        if (cm == NEG_INF) continue;  // every slot so far is empty
        if (cm > M) {
            const float alpha = fast_exp2(M - cm);  // 0 while M is -inf
            Z *= alpha;
            lo *= alpha;
            hi *= alpha;
            M = cm;
        }
#pragma unroll
        for (int u = 0; u < MERGE_CHUNK; ++u) {
            const float w = fast_exp2(l[u] - M);  // 0 for empty slots
            Z += w;
            const float ws = __builtin_amdgcn_ldexpf(w, (int)le[u].y);
            lo += ws * unpack_f16x4(u32x2{v[u][0], v[u][1]});
            hi += ws * unpack_f16x4(u32x2{v[u][2], v[u][3]});
        }
    }
    if constexpr (SPLIT > 1) {
        __shared__ float sh[SPLIT - 1][10][NT];
        if (grp > 0) {
            float *x = &sh[grp - 1][0][tid];
            x[0] = M;
            x[NT] = Z;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[(2 + i) * NT] = lo[i];
                x[(6 + i) * NT] = hi[i];
            }
        }
        __syncthreads();
        if (grp > 0 || !valid) return;
#pragma unroll
        for (int g = 0; g < SPLIT - 1; ++g) {
            const float *x = &sh[g][0][tid];
            const float Mg = x[0];
            if (Mg == NEG_INF) continue;  // an empty range
            const float cm = fmaxf(M, Mg);
            const float alpha = fast_exp2(M - cm), beta = fast_exp2(Mg - cm);  // alpha is 0 while M is -inf
            Z = Z * alpha + x[NT] * beta;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo[i] = lo[i] * alpha + x[(2 + i) * NT] * beta;
                hi[i] = hi[i] * alpha + x[(6 + i) * NT] * beta;
            }
            M = cm;
        }
    }
    if (Z > 0.f) {
        const float inv = 1.f / Z;
        lo *= inv;
        hi *= inv;
    }
    // the slice holds d = 32 (d8 / 4) + 4 (d8 % 4) + {0..3} (lo) and the same + 16 (hi)
    u16 *dst = out + ((size_t)r * hq + head) * D + 32 * (d8 >> 2) + 4 * (d8 & 3);
    *(u32x2 *)dst = u32x2{Ops<FP16>::pack(lo[0], lo[1]), Ops<FP16>::pack(lo[2], lo[3])};
    *(u32x2 *)(dst + 16) = u32x2{Ops<FP16>::pack(hi[0], hi[1]), Ops<FP16>::pack(hi[2], hi[3])};
}

// ------------------------------------------------------------------ read ceiling
// A read-only stream: every lane loads 16-byte chunks in a grid-stride loop
// and folds them into one word per wave, the ceiling against which the
// memory-bound segment kernels are measured (ta_read_stream).
constexpr int READ_NT = 256;

__global__ __launch_bounds__(READ_NT) void read_stream_kernel(const u32x4 *__restrict__ src, int64_t n,
                                                              uint32_t *__restrict__ sink) {
    u32x4 acc = {0u, 0u, 0u, 0u};
    const int64_t step = (int64_t)gridDim.x * READ_NT;
    int64_t i = (int64_t)blockIdx.x * READ_NT + threadIdx.x;
    for (; i + 3 * step < n; i += 4 * step) {
        const u32x4 a = src[i], b = src[i + step], c = src[i + 2 * step], d = src[i + 3 * step];
        acc ^= a ^ b ^ c ^ d;
    }
    for (; i < n; i += step) acc ^= src[i];
    uint32_t w = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    for (int o = 32; o > 0; o >>= 1) w ^= __shfl_xor(w, o);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * (READ_NT / 64) + threadIdx.x / 64] = w;
}

// ------------------------------------------------------------------ launch
// resident one-wave workgroups on 256 CUs (8 per CU by LDS at d = 128)
constexpr int SMALL_MAX_BLOCKS = 2048;

template <int D, bool FP16>
hipError_t launch_segment(const SegParams &sp, int kind, hipStream_t stream) {
    if (sp.n_items <= 0) return hipSuccess;
#ifndef TA_LEGACY_LARGE
    {
        // LDS-transpose kernels (segment_tile.hip) whenever the pool layout allows them
        const hipError_t e = launch_tile(sp, kind, D, FP16, stream);
        if (e != hipErrorNotSupported) return e;
    }
#endif
    switch (kind) {
        case TA_SMALL:
        case TA_TAIL: {  // the fused merge exists only on the LDS-transpose path
            const int blocks = sp.n_items < SMALL_MAX_BLOCKS ? sp.n_items : SMALL_MAX_BLOCKS;
            TA_LAUNCH((seg_small_kernel<D, FP16>), dim3(blocks), dim3(SMALL_NT), stream, sp);
            break;
        }
        case TA_LARGE64:
            TA_LAUNCH((seg_large_kernel<D, FP16, 1, 4, 64>), dim3(sp.n_items), dim3(256), stream, sp);
            break;
        case TA_LARGE128:
            TA_LAUNCH((seg_large_kernel<D, FP16, 2, 4, 64>), dim3(sp.n_items), dim3(256), stream, sp);
            break;
        case TA_LARGE256:
            TA_LAUNCH((seg_large_kernel<D, FP16, 2, 8, 128>), dim3(sp.n_items), dim3(512), stream, sp);
            break;
        default:
            return (hipError_t)TA_ERR_ARG;
    }
    return hipGetLastError();
}

// nreq requests: reqs[0 .. nreq) when reqs is given, else 0 .. nreq-1
template <int D, bool FP16>
hipError_t launch_merge(const void *part, const float *lse, const int32_t *slots, const int32_t *counts,
                        const int32_t *reqs, void *out, int nreq, int hq, int maxs, hipStream_t stream,
                        int slot_stride = 0) {
    constexpr int MH = MERGE_NT / (D / 8), MH2 = MH / 2;
    const bool fill = (long)nreq * ((hq + MH - 1) / MH) < MERGE_FILL_BLOCKS;
    const dim3 grid(nreq, fill ? (hq + MH2 - 1) / MH2 : (hq + MH - 1) / MH);
    const u16 *p16 = static_cast<const u16 *>(part);
    u16 *o16 = static_cast<u16 *>(out);
    if (maxs > MERGE_CHUNK) {
        if (fill)
            TA_LAUNCH((merge_kernel<D, FP16, 2, MERGE_NT / 2>), grid, dim3(MERGE_NT), stream, p16, lse, slots,
                      counts, reqs, o16, hq, maxs, slot_stride);
        else
            TA_LAUNCH((merge_kernel<D, FP16, 2>), grid, dim3(2 * MERGE_NT), stream, p16, lse, slots, counts, reqs,
                      o16, hq, maxs, slot_stride);
    } else {
        if (fill)
            TA_LAUNCH((merge_kernel<D, FP16, 1, MERGE_NT / 2>), grid, dim3(MERGE_NT / 2), stream, p16, lse, slots,
                      counts, reqs, o16, hq, maxs, slot_stride);
        else
            TA_LAUNCH((merge_kernel<D, FP16, 1>), grid, dim3(MERGE_NT), stream, p16, lse, slots, counts, reqs, o16,
                      hq, maxs, slot_stride);
    }
    return hipGetLastError();
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int check_common(int hq, int hk, int d, int dtype) {
    if (dtype != TA_BF16 && dtype != TA_FP16) return TA_ERR_DTYPE;
    if (hq <= 0 || hk <= 0 || hq % hk != 0) return TA_ERR_ARG;
    if (d != 32 && d != 64 && d != 128) return TA_ERR_ARG;
    return 0;
}

#define TA_DISPATCH(d, fp16, CALL)                                         \
    ((d) == 128 ? ((fp16) ? CALL(128, true) : CALL(128, false))           \
     : (d) == 64 ? ((fp16) ? CALL(64, true) : CALL(64, false))            \
                 : ((fp16) ? CALL(32, true) : CALL(32, false)))

}  // namespace

namespace ta {
thread_local LaunchEvents g_launch_events = {nullptr, nullptr};
}  // namespace ta

extern "C" {

const char *ta_version(void) { return "tree_attn gfx950 1.0"; }

const char *ta_error_string(int code) {
    switch (code) {
        case 0: return "success";
        case TA_ERR_ARG: return "tree_attn: invalid argument (null pointer, size or unsupported shape)";
        case TA_ERR_ALIGN: return "tree_attn: q/kp/vp/part/out must be 16-byte aligned, lse 8-byte aligned";
        case TA_ERR_DTYPE: return "tree_attn: dtype must be TA_BF16 or TA_FP16";
        case TA_ERR_SCRATCH:
            return "tree_attn: the plan's partials exceed TA_NOALLOC_SCRATCH_BYTES (use ta_attention_matrix)";
        default: return hipGetErrorString((hipError_t)code);
    }
}

}  // extern "C"

namespace {

void fill_params(SegParams &sp, const void *q, const void *kp, const void *vp, const int32_t *qids,
                 const int32_t *kstart, const int32_t *qlen, const int32_t *klen, const int32_t *rowbase,
                 const int32_t *items, int32_t n_items, void *part, float *lse, int32_t hq, int32_t hk, int32_t d,
                 int32_t tcap, int32_t maxr, const int32_t *slots, const int32_t *counts, void *out, int32_t maxs,
                 const int32_t *xtail, int32_t xtail_stride, const int32_t *qbase);

// One segment launch; with out given (TA_TAIL only) the items merge their
// requests into out.
int segment_launch(const void *q, const void *kp, const void *vp, const int32_t *qids, const int32_t *kstart,
                   const int32_t *qlen, const int32_t *klen, const int32_t *rowbase, const int32_t *items,
                   int32_t n_items, int32_t kind, void *part, float *lse, int32_t nreq, int32_t hq, int32_t hk,
                   int32_t d, int32_t tcap, int32_t maxr, int32_t dtype, const int32_t *slots,
                   const int32_t *counts, void *out, int32_t maxs, const int32_t *xtail, int32_t xtail_stride,
                   const int32_t *qbase, void *stream) {
    if (int e = check_common(hq, hk, d, dtype)) return e;
    if (n_items < 0 || nreq <= 0 || tcap <= 0 || maxr <= 0 || kind < TA_SMALL || kind > TA_TAIL) return TA_ERR_ARG;
    if (n_items == 0) return 0;
    if (!q || !kp || !vp || !qids || !kstart || !qlen || !klen || !rowbase || !items || !part || !lse)
        return TA_ERR_ARG;
    if (!aligned16(q) || !aligned16(kp) || !aligned16(vp) || !aligned16(part)) return TA_ERR_ALIGN;
    if (out) {
#ifdef TA_LEGACY_LARGE
        return TA_ERR_ARG;  // the register-staged kernels have no fused merge
#endif
        if (kind != TA_TAIL || tcap % 8 != 0 || !slots || !counts || maxs <= 0) return TA_ERR_ARG;
        if (!aligned16(out)) return TA_ERR_ALIGN;
    }
    if (xtail) {
#ifdef TA_LEGACY_LARGE
        return TA_ERR_ARG;  // the register-staged kernels take no attached segments
#endif
        if (kind != TA_LARGE256 || tcap % 8 != 0 || xtail_stride != TA_XTAIL_STRIDE) return TA_ERR_ARG;
    }
    SegParams sp;
    fill_params(sp, q, kp, vp, qids, kstart, qlen, klen, rowbase, items, n_items, part, lse, hq, hk, d, tcap, maxr,
                slots, counts, out, maxs, xtail, xtail_stride, qbase);
    const hipStream_t st = static_cast<hipStream_t>(stream);
#define TA_SEG(D, F) launch_segment<D, F>(sp, kind, st)
    return (int)TA_DISPATCH(d, dtype == TA_FP16, TA_SEG);
#undef TA_SEG
}

// The launch arguments every segment kernel shares.
void fill_params(SegParams &sp, const void *q, const void *kp, const void *vp, const int32_t *qids,
                 const int32_t *kstart, const int32_t *qlen, const int32_t *klen, const int32_t *rowbase,
                 const int32_t *items, int32_t n_items, void *part, float *lse, int32_t hq, int32_t hk, int32_t d,
                 int32_t tcap, int32_t maxr, const int32_t *slots, const int32_t *counts, void *out, int32_t maxs,
                 const int32_t *xtail, int32_t xtail_stride, const int32_t *qbase) {
    sp.q = static_cast<const u16 *>(q);
    sp.kp = static_cast<const u16 *>(kp);
    sp.vp = static_cast<const u16 *>(vp);
    sp.qids = qids;
    sp.kstart = kstart;
    sp.qlen = qlen;
    sp.klen = klen;
    sp.rowbase = rowbase;
    sp.items = items;
    sp.part = static_cast<u16 *>(part);
    sp.lse = lse;
    sp.n_items = n_items;
    sp.hq = hq;
    sp.hk = hk;
    sp.group = hq / hk;
    sp.tcap = tcap;
    sp.maxr = maxr;
    sp.scale_log2 = (float)(1.4426950408889634 / __builtin_sqrt((double)d));
    sp.slots = slots;
    sp.counts = counts;
    sp.out = static_cast<u16 *>(out);
    sp.maxs = maxs;
    sp.xtail = xtail;
    sp.xtail_stride = xtail_stride;
    sp.qbase = qbase;
}

int plan_segment(const void *q, const void *kp, const void *vp, int32_t tcap, const ta_plan *plan, int kind,
                 void *out, void *stream) {
    const bool xt = kind == TA_LARGE256 && plan->xtail;
    return segment_launch(q, kp, vp, plan->qids, plan->kstart, plan->qlen, plan->klen, plan->rowbase,
                          plan->items[kind], plan->n_items[kind], kind, plan->part, plan->lse, plan->nreq, plan->hq,
                          plan->hk, plan->d, tcap, plan->maxr, plan->dtype, plan->slots, plan->counts, out,
                          plan->maxs, xt ? plan->xtail : nullptr, xt ? plan->xtail_stride : 0, plan->qbase, stream);
}

// The merge of requests reqs[0 .. n) (reqs == NULL: 0 .. n-1) of a prepared
// plan into out, with the plan's affine slot layout when it has one.
int plan_merge(const ta_plan *plan, const int32_t *reqs, int32_t n, void *out, void *stream) {
    if (!plan->part || !plan->lse || !plan->slots || !plan->counts || n <= 0 || n > plan->nreq) return TA_ERR_ARG;
    if (plan->dtype != TA_BF16 && plan->dtype != TA_FP16) return TA_ERR_DTYPE;
    if (plan->maxs <= 0 || plan->hq <= 0 || (plan->d != 32 && plan->d != 64 && plan->d != 128)) return TA_ERR_ARG;
    if (!aligned16(plan->part) || !aligned16(out) || (reinterpret_cast<uintptr_t>(plan->lse) & 7)) return TA_ERR_ALIGN;
    // an affine slot layout must stay inside the partial slots
    if (plan->slot_stride < 0 ||
        (plan->slot_stride > 0 &&
         (int64_t)(plan->nreq - 1) + (int64_t)(plan->maxs - 1) * plan->slot_stride >= plan->nslot))
        return TA_ERR_ARG;
    const hipStream_t st = static_cast<hipStream_t>(stream);
#define TA_MRG(D, F) \
    launch_merge<D, F>(plan->part, plan->lse, plan->slots, plan->counts, reqs, out, n, plan->hq, plan->maxs, st, \
                       plan->slot_stride)
    return (int)TA_DISPATCH(plan->d, plan->dtype == TA_FP16, TA_MRG);
#undef TA_MRG
}

}  // namespace

extern "C" {

int ta_merge_plan(const ta_plan *plan, void *out, void *stream) {
    if (!plan || !out) return TA_ERR_ARG;
    return plan_merge(plan, nullptr, plan->nreq, out, stream);
}

int ta_segment(const void *q, const void *kp, const void *vp, const int32_t *qids, const int32_t *kstart,
               const int32_t *qlen, const int32_t *klen, const int32_t *rowbase, const int32_t *items,
               int32_t n_items, int32_t kind, void *part, float *lse, int32_t nreq, int32_t hq, int32_t hk,
               int32_t d, int32_t tcap, int32_t maxr, int32_t dtype, void *stream) {
    return segment_launch(q, kp, vp, qids, kstart, qlen, klen, rowbase, items, n_items, kind, part, lse, nreq, hq,
                          hk, d, tcap, maxr, dtype, nullptr, nullptr, nullptr, 0, nullptr, 0, nullptr, stream);
}

int ta_merge(const void *part, const float *lse, const int32_t *slots, const int32_t *counts, void *out,
             int32_t nreq, int32_t hq, int32_t d, int32_t maxs, int32_t dtype, void *stream) {
    if (dtype != TA_BF16 && dtype != TA_FP16) return TA_ERR_DTYPE;
    if (nreq <= 0 || hq <= 0 || maxs <= 0 || (d != 32 && d != 64 && d != 128)) return TA_ERR_ARG;
    if (!part || !lse || !slots || !counts || !out) return TA_ERR_ARG;
    if (!aligned16(part) || !aligned16(out) || (reinterpret_cast<uintptr_t>(lse) & 7)) return TA_ERR_ALIGN;
    const hipStream_t st = static_cast<hipStream_t>(stream);
#define TA_MRG(D, F) launch_merge<D, F>(part, lse, slots, counts, nullptr, out, nreq, hq, maxs, st)
    return (int)TA_DISPATCH(d, dtype == TA_FP16, TA_MRG);
#undef TA_MRG
}

int ta_segment_plan(const void *q, const void *kp, const void *vp, int32_t tcap, const ta_plan *plan, int32_t kind,
                    void *stream) {
    if (!plan || kind < TA_SMALL || kind > TA_TAIL) return TA_ERR_ARG;
    return plan_segment(q, kp, vp, tcap, plan, kind, nullptr, stream);
}

int ta_tail_merge(const void *q, const void *kp, const void *vp, int32_t tcap, const ta_plan *plan, void *out,
                  void *stream) {
    if (!plan || !out || tcap % 8 != 0) return TA_ERR_ARG;
    return plan_segment(q, kp, vp, tcap, plan, TA_TAIL, out, stream);
}

}  // extern "C"

// Partial rows and log-sum-exp values of ta_attention_matrix_noalloc.  Each
// GPU the library runs on holds its own copy until the process ends.  In host
// code the name is a stand-in, not a device address: kernels get the address
// hipGetSymbolAddress returns for the current device (noalloc_scratch).
static __device__ __align__(256) unsigned char scratch[TA_NOALLOC_SCRATCH_BYTES];

namespace {

// The TA_LARGE256, TA_LARGE64 and TA_SMALL items of a plan in one launch
// (seg_mix_kernel), when at least two of those kinds have items and
// TA_LARGE128 has none.  Returns -1 when the plan does not qualify.
int mix_launch(const void *q, const void *kp, const void *vp, int32_t tcap, const ta_plan *plan, void *stream) {
#ifdef TA_LEGACY_LARGE
    return -1;
#endif
    const int n[3] = {plan->n_items[TA_LARGE256], plan->n_items[TA_LARGE64], plan->n_items[TA_SMALL]};
    if ((n[0] > 0) + (n[1] > 0) + (n[2] > 0) < 2 || plan->n_items[TA_LARGE128] > 0 || tcap % 8 != 0) return -1;
    if (n[0] < 0 || n[1] < 0 || n[2] < 0) return TA_ERR_ARG;
    if (int e = check_common(plan->hq, plan->hk, plan->d, plan->dtype)) return e;
    if (plan->nreq <= 0 || tcap <= 0 || plan->maxr <= 0) return TA_ERR_ARG;
    if (!q || !kp || !vp || !plan->qids || !plan->kstart || !plan->qlen || !plan->klen || !plan->rowbase ||
        !plan->part || !plan->lse)
        return TA_ERR_ARG;
    for (int k : {TA_LARGE256, TA_LARGE64, TA_SMALL})
        if (plan->n_items[k] > 0 && !plan->items[k]) return TA_ERR_ARG;
    if (!aligned16(q) || !aligned16(kp) || !aligned16(vp) || !aligned16(plan->part)) return TA_ERR_ALIGN;
    const bool xt = n[0] > 0 && plan->xtail;
    if (xt && plan->xtail_stride != TA_XTAIL_STRIDE) return TA_ERR_ARG;
    SegParams sp;
    fill_params(sp, q, kp, vp, plan->qids, plan->kstart, plan->qlen, plan->klen, plan->rowbase, nullptr, 0,
                plan->part, plan->lse, plan->hq, plan->hk, plan->d, tcap, plan->maxr, plan->slots, plan->counts,
                nullptr, plan->maxs, xt ? plan->xtail : nullptr, xt ? plan->xtail_stride : 0, plan->qbase);
    const int32_t *const items[3] = {plan->items[TA_LARGE256], plan->items[TA_LARGE64], plan->items[TA_SMALL]};
    if (hipError_t e = ta::launch_tile_mix(sp, items, n, plan->d, plan->dtype == TA_FP16,
                                           static_cast<hipStream_t>(stream)))
        return (int)e;
    return 0;
}

int attention_layer(const void *q, const void *kp, const void *vp, int32_t tcap, const ta_plan *plan, void *out,
                    void *stream) {
    if (!plan || !out) return TA_ERR_ARG;
#ifdef TA_LEGACY_LARGE
    const bool fused = false;
#else
    const bool fused = tcap % 8 == 0;  // the LDS-transpose kernels carry the fused merge
#endif
    // attached segments exist only on the LDS-transpose path (pools with tcap % 8 == 0)
    if (plan->xtail && !fused) return TA_ERR_ARG;
    // the partials every merge reads come first: large jobs, then small jobs,
    // in one launch when the kinds allow it
    const int mixed = mix_launch(q, kp, vp, tcap, plan, stream);
    if (mixed > 0) return mixed;
    static const int order[] = {TA_LARGE256, TA_LARGE128, TA_LARGE64, TA_SMALL};
    for (int kind : order) {
        if (mixed == 0 && kind != TA_LARGE128) continue;
        if (plan->n_items[kind] == 0) continue;
        if (int e = plan_segment(q, kp, vp, tcap, plan, kind, nullptr, stream)) return e;
    }
    if (!fused) {
        if (plan->n_items[TA_TAIL] > 0)
            if (int e = plan_segment(q, kp, vp, tcap, plan, TA_TAIL, nullptr, stream)) return e;
        return ta_merge(plan->part, plan->lse, plan->slots, plan->counts, out, plan->nreq, plan->hq, plan->d,
                        plan->maxs, plan->dtype, stream);
    }
    if (plan->n_items[TA_TAIL] > 0)
        if (int e = plan_segment(q, kp, vp, tcap, plan, TA_TAIL, out, stream)) return e;
    if (plan->n_rest <= 0) return 0;
    // rest == NULL with n_rest == nreq: every request
    if (!plan->rest && plan->n_rest != plan->nreq) return TA_ERR_ARG;
    return plan_merge(plan, plan->rest, plan->n_rest, out, stream);
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
unsigned char *g_scratch[kMaxDevices];  // per device: the device address of `scratch`

// The address of `scratch` on the current device, looked up once per device
// (with that device current) and kept.
int noalloc_scratch(unsigned char **ptr) {
    int dev = -1;
    if (hipError_t e = hipGetDevice(&dev)) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return TA_ERR_ARG;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) return (int)e;
        if (!p) return TA_ERR_ARG;
        g_scratch[dev] = static_cast<unsigned char *>(p);
    }
    *ptr = g_scratch[dev];
    return 0;
}

}  // namespace

extern "C" {

int ta_attention_matrix(const void *q, const void *kp, const void *vp, int32_t tcap, const ta_plan *plan,
                        void *out, void *stream) {
    return attention_layer(q, kp, vp, tcap, plan, out, stream);
}

int ta_attention_matrix_noalloc(const void *q, const void *kp, const void *vp, int32_t tcap, const ta_plan *plan,
                                void *out, void *stream) {
    if (!plan || !out) return TA_ERR_ARG;
    if (plan->nslot <= 0 || plan->hq <= 0 || plan->d <= 0) return TA_ERR_ARG;
    // partial rows (fp16) first, then the (lse, exponent) pairs at a 256-byte boundary
    const uint64_t part_bytes = (uint64_t)plan->nslot * (uint64_t)plan->hq * (uint64_t)plan->d * 2u;
    const uint64_t lse_offset = (part_bytes + 255u) & ~(uint64_t)255u;
    const uint64_t lse_bytes = (uint64_t)plan->nslot * (uint64_t)plan->hq * 2u * sizeof(float);
    if (lse_offset + lse_bytes > (uint64_t)TA_NOALLOC_SCRATCH_BYTES) return TA_ERR_SCRATCH;
    unsigned char *base = nullptr;
    if (int e = noalloc_scratch(&base)) return e;
    if (stream) {  // the scratch address belongs to the current device: the stream must be on it
        int cur = -1, sdev = -1;
        if (hipError_t e = hipGetDevice(&cur)) return (int)e;
        if (hipError_t e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev)) return (int)e;
        if (cur != sdev) return TA_ERR_ARG;
    }
    // every partial slot the merge reads is written by a segment launch of the
    // same call first, so nothing in the array needs clearing
    ta_plan local = *plan;
    local.part = base;
    local.lse = reinterpret_cast<float *>(base + lse_offset);
    return attention_layer(q, kp, vp, tcap, &local, out, stream);
}

int ta_read_stream(const void *src, int64_t bytes, uint32_t *sink, int32_t blocks, void *stream) {
    if (!src || !sink || bytes <= 0 || bytes % 16 != 0 || blocks <= 0) return TA_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(src) % 16 != 0) return TA_ERR_ALIGN;
    TA_LAUNCH(read_stream_kernel, dim3(blocks), dim3(READ_NT), static_cast<hipStream_t>(stream),
              static_cast<const u32x4 *>(src), bytes / 16, sink);
    return (int)hipGetLastError();
}

int ta_time_next_launch(void *start_event, void *stop_event) {
    if ((start_event == nullptr) != (stop_event == nullptr)) return TA_ERR_ARG;
    ta::g_launch_events = ta::LaunchEvents{static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event)};
    return 0;
}

}  // extern "C"

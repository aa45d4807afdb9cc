// segment_tile.hip -- gfx950 kernel for large segment jobs (more than 16 query rows).
//
// Replaces the large phase of the reference's Triton _segment
// (src/tree_attention/kernels.py:8-55, launched at :158-165): grouped partial
// attention of one physical KV segment for all requests of a job, online
// softmax in fp32, P rounded to the input dtype before PV (kernels.py:49),
// output acc/z and the natural-log log-sum-exp m + ln z.
//
// One workgroup owns one (job, row tile, KV head) work item: NW waves of
// 16*NB query rows each (jobs with at most 16 rows: one wave, NB = 1).  The
// job's tokens are streamed in 64-token tiles.
//
//  * HBM -> LDS without registers: a tile is D/8 1-KiB blocks of K (8 d-rows
//    x 64 tokens each) and D/8 of V, each copied by one wave with one
//    global_load_lds_dwordx4 (lane i fills bytes 16i..16i+15 of the block).
//    Three LDS stages keep two tiles in flight while one is computed (one-wave
//    workgroups of small jobs use one stage, so that four share a CU); each wave waits for its own copies with s_waitcnt vmcnt
//    and the waves meet at one barrier per tile.
//  * The lane -> 16-byte-chunk assignment inside a block is chosen so that the
//    eight chunks one 16-lane group reads together are 128 contiguous bytes,
//    and odd blocks swap the two 128-byte halves of every 256 bytes so that
//    neighbouring groups land 128 bytes apart (no LDS bank conflicts; see
//    the LDS layout note above struct LdsOfs).
//  * MFMA operands are read with gfx950's transposing LDS load
//    ds_read_b64_tr_b16: within a group of 16 lanes, lane 4a+b receives
//    element b of the 8-byte chunks addressed by lanes a, a+4, a+8, a+12.
//    Lane (g, r) addresses contraction row r/4 (+4) of its group at column
//    4*(r%4), so every lane ends up with four consecutive contraction elements
//    of one output row or column -- the MFMA operand layout -- straight from
//    the pools' own layouts (K [d][token], V [token][d]).
//  * S^T = K Q^T with v_mfma_f32_16x16x32: the C layout gives each lane four
//    consecutive tokens of one query row, which is the B operand of the PV
//    product O^T = V^T P^T, so P never leaves registers.
//  * The softmax denominator is one more PV MFMA against an all-ones A
//    operand, so z sums exactly the rounded P that multiplies V.
//  * Softmax in base 2 with log2(e)/sqrt(D) folded into one FMA; lazy
//    rescaling (the running maximum moves only by more than TAU).
// Requirements (checked by the launcher): tcap % 8 == 0 and 16-byte aligned
// pools, so every 8-token chunk of a K row is one aligned 16-byte copy.
#include "ta_common.h"
#include "tree_attn.h"

namespace ta {
namespace {

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding).
#define TA_VMCNT(n) ((((n)&15) | (7 << 4) | (15 << 8) | ((((n) >> 4) & 3) << 14)))

// Wait until at most n tiles of this wave's copies (BPW each) are in flight
// (n = 0 .. 4; the immediate of s_waitcnt must be a constant).
template <int BPW>
__device__ inline void wait_tiles(int n) {
    static_assert(4 * BPW <= 63, "four tiles of copies fit the vmcnt counter");
    switch (n) {
        case 4: __builtin_amdgcn_s_waitcnt(TA_VMCNT(4 * BPW)); break;
        case 3: __builtin_amdgcn_s_waitcnt(TA_VMCNT(3 * BPW)); break;
        case 2: __builtin_amdgcn_s_waitcnt(TA_VMCNT(2 * BPW)); break;
        case 1: __builtin_amdgcn_s_waitcnt(TA_VMCNT(BPW)); break;
        default: __builtin_amdgcn_s_waitcnt(TA_VMCNT(0)); break;
    }
}

// Two transposing LDS loads -> one 8-element MFMA operand.
__device__ inline u32x4 tr_pair(const u16 *lo, const u16 *hi) {
    const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)lo);
    const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)hi);
    const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
    return u32x4{ua[0], ua[1], ub[0], ub[1]};
}

// LDS layout of one 64-token tile (16-bit elements): KBLK blocks of K, then
// VBLK blocks of V, each a 1 KiB copy unit of 64 16-byte slots.
//   K block b: d-rows 8b..8b+7; the 16-byte chunk c (tokens 8c..8c+7) of
//     d-row 8b+j has logical slot 16*(c>>1) + 8*(j>>2) + 4*(c&1) + (j&3).
//   V block b: token rows VROWS*b ..; chunk s (d = 8s..8s+7) of token row j
//     has logical slot SV*(s>>1) + 8*(j>>2) + 4*(s&1) + (j&3).
// Swizzle: in odd blocks (block index within the tile) logical slot l sits at
// physical slot l ^ 8, i.e. the two 128-byte halves of every 256 bytes are
// swapped.  The four 16-lane groups of a transposing read address blocks of
// alternating parity at equal logical offsets, so the groups land 128 bytes
// apart modulo 256 (disjoint LDS banks) without padding the blocks; a tile is
// 32 KiB and five of them fit the 160 KiB LDS.
struct LdsOfs {  // per-lane element offsets of the transposing reads (swizzle applied)
    int klo, khi;        // K: the two 8-byte halves of a lane's operand
    int vlo[2], vhi[2];  // V: same, by the parity of the 16-row block db of O^T
};

template <int D>
struct Tile {
    static constexpr int TT = 64;
    static constexpr int BLK = 512;         // 1 KiB block
    static constexpr int KBLK = D / 8;
    static constexpr int VROWS = 512 / D;   // token rows per V block
    static constexpr int VBLK = TT / VROWS;
    static constexpr int NBLK = KBLK + VBLK;
    static constexpr int ELEMS = NBLK * BLK;
    static constexpr int SV = 1024 / D;

    // physical element offset of logical in-block offset `e` in block `b`
    __device__ static int swz(int b, int e) { return e ^ (64 * (b & 1)); }

    // Lane (row, g4) of a transposing read addresses, within its block,
    // logical element 8 * (4 * ((row & 3) >> 1) + (row >> 2)) + 4 * (row & 1)
    // (< 64) of the chunk-slot group it reads; the K operand's two halves are
    // 64 elements apart in block 4 ks + g4 (a parity of g4 & 1 for every ks);
    // the V operand's halves are in blocks KBLK + base / VROWS + vb and
    // 16 / VROWS blocks further (base / VROWS is even), at in-block offset
    // 8 SV db + vin, whose bit 6 depends on db only through SV / 8 (odd for
    // D = 128).
    __device__ static LdsOfs offsets(int row, int g4) {
        const int lane_ofs = 8 * (4 * ((row & 3) >> 1) + (row >> 2)) + 4 * (row & 1);
        LdsOfs o;
        o.klo = BLK * g4 + swz(g4, lane_ofs);
        o.khi = BLK * g4 + swz(g4, lane_ofs + 64);
        const int vb = (4 * g4) / VROWS;
        const int vin = 64 * (((4 * g4) % VROWS) >> 2) + lane_ofs;
        const int blo = KBLK + vb, bhi = blo + 16 / VROWS;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int dbo = 8 * SV * e;  // representative db of parity e
            o.vlo[e] = BLK * vb + swz(blo, dbo + vin) - dbo;
            o.vhi[e] = BLK * (vb + 16 / VROWS) + swz(bhi, dbo + vin) - dbo;
        }
        return o;
    }
};

template <int D, bool FP16, int NB, int NW>
struct TileMath {
    static constexpr int DB = D / 16;  // 16-row blocks of O^T
    static constexpr int KS = D / 32;  // 32-wide k slices of QK
    using O = Ops<FP16>;
    using T = Tile<D>;

    f32x4 o[NB][DB], z[NB];
    float m[NB];

    __device__ void reset() {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            m[nb] = NEG_INF;
            z[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int db = 0; db < DB; ++db) o[nb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }

    // One pipeline step: copy the tile at pool token t0n into stage `nxt` (if
    // `copy`), then compute the tile staged in `cur` (if `compute`).  The two
    // stages never alias; declaring them restrict in one function lets the
    // compiler keep the copies in flight across the reads of `cur`.
    __device__ void step(const u16 *__restrict__ cur, u16 *__restrict__ nxt, bool copy, bool compute,
                         const u16 *__restrict__ kp, const u16 *__restrict__ vp, int h, int tcap, int t0n, int kst,
                         int kend, int wave, int lane, const u32x4 (&qf)[NB][KS], const LdsOfs &of, int lo,
                         int hi, int g4, float c) {
        if (copy) this->copy(nxt, kp, vp, h, tcap, t0n, kst, kend, wave, lane);
        if (compute) tile(cur, qf, of, lo, hi, g4, c);
    }

    // Copy the tile at pool token t0n into stage `st` (this wave's blocks).
    // Inside the job (tokens [t0n, t0n + TT) all in [kst, kend)) no index is
    // clamped; at its edges chunks past the pool end read its last chunk and
    // V rows outside the job read a row inside it (finite values; their
    // scores are masked, P = 0).
    __device__ static void copy(u16 *st, const u16 *__restrict__ kp, const u16 *__restrict__ vp, int h,
                                int tcap, int t0n, int kst, int kend, int wave, int lane) {
        const int w = __builtin_amdgcn_readfirstlane(wave);
        if (t0n >= kst && t0n + T::TT <= kend)
            copy_blocks<false>(st, kp, vp, h, tcap, t0n, kst, kend, w, lane);
        else
            copy_blocks<true>(st, kp, vp, h, tcap, t0n, kst, kend, w, lane);
    }

    template <bool CLAMP>
    __device__ static void copy_blocks(u16 *st, const u16 *__restrict__ kp, const u16 *__restrict__ vp, int h,
                                       int tcap, int t0n, int kst, int kend, int w, int lane) {
#pragma unroll
        for (int i = 0; i < T::NBLK / NW; ++i) {
            const int blk = w + i * NW;
            // with KBLK % NW == 0 every wave's i-th block is K for the same i
            const bool isk = T::KBLK % NW == 0 ? i * NW < T::KBLK : blk < T::KBLK;
            const u16 *src;
            const int l = lane ^ (8 * (blk & 1));  // logical slot filled by this lane (swizzle)
            if (isk) {
                const int ck = 2 * (l >> 4) + ((l >> 2) & 1);
                const int d = 8 * blk + 4 * ((l >> 3) & 1) + (l & 3);
                const int tok = t0n + 8 * ck;
                src = kp + (size_t)(h * D + d) * tcap + (CLAMP ? min(tok, tcap - 8) : tok);
            } else {
                const int vb = blk - T::KBLK;
                const int rem = l % T::SV;
                const int s = 2 * (l / T::SV) + ((rem >> 2) & 1);
                const int j = 4 * (rem >> 3) + (rem & 3);
                const int t = t0n + vb * T::VROWS + j;
                src = vp + ((size_t)h * tcap + (CLAMP ? min(max(t, kst), kend - 1) : t)) * D + 8 * s;
            }
            __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(st + blk * T::BLK), 16, 0, 0);
        }
    }

    // K fragments (A operand of QK) of the 32 tokens base .. base+31:
    // kf[b][ks] covers tokens base+16b .. +15, d = 32*ks .. +31.
    __device__ static void load_k(const u16 *__restrict__ cur, const LdsOfs &of, int base, u32x4 (&kf)[2][KS]) {
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                // block 4*ks + g4, chunk pair base/16 + b, block rows 0-3 / 4-7
                const int e = 4 * T::BLK * ks + 8 * (base + 16 * b);
                kf[b][ks] = tr_pair(cur + of.klo + e, cur + of.khi + e);
            }
    }

    // V^T fragments (A operand of PV) of the 32 tokens base .. base+31: PV
    // k-slot j of lane group g4 is token 4*g4+j (j<4) or 16+4*g4+j-4 (j>=4),
    // where the QK output left P.
    __device__ static void load_v(const u16 *__restrict__ st, const LdsOfs &of, int base, u32x4 (&v)[DB]) {
        const u16 *vrow = st + T::BLK * (T::KBLK + base / T::VROWS);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const u16 *va = vrow + 8 * T::SV * db;
            v[db] = tr_pair(va + of.vlo[db & 1], va + of.vhi[db & 1]);
        }
    }

    // S^T = K Q^T: s[nb][b] holds tokens base+16b+4*g4+i of row block nb.
    __device__ static void qk(const u32x4 (&kf)[2][KS], const u32x4 (&qf)[NB][KS], f32x4 (&s)[NB][2]) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) s[nb][0] = s[nb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) s[nb][b] = O::mma_k32(kf[b][ks], qf[nb][ks], s[nb][b]);
    }

    // of: per-lane element offsets of the transposing loads;
    // tokens [lo, hi) of the tile belong to the job.  Software pipeline per
    // 32-token step k: the LDS loads of step k's V and step k+1's K are issued
    // before step k's softmax (which hides their latency), then PV of step k
    // and QK of step k+1 run back to back on the matrix cores.
    __device__ void tile(const u16 *__restrict__ cur, const u32x4 (&qf)[NB][KS], const LdsOfs &of, int lo,
                         int hi, int g4, float c) {
        constexpr int STEPS = T::TT / 32;
        const u32x4 ones = {O::ONE2, O::ONE2, O::ONE2, O::ONE2};
        f32x4 s[NB][2];
        {
            u32x4 kf[2][KS];
            load_k(cur, of, 0, kf);
            qk(kf, qf, s);
        }
#pragma unroll
        for (int k = 0; k < STEPS; ++k) {
            const int base = 32 * k;
            if (base >= hi) break;
            u32x4 vf[DB];
            load_v(cur, of, base, vf);
            const bool more = k + 1 < STEPS && base + 32 < hi;
            u32x4 kf[2][KS];
            if (more) load_k(cur, of, base + 32, kf);
            if (lo > base || hi < base + 32) {  // wave-uniform: first or last step of the job
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int b = 0; b < 2; ++b)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int tok = base + 16 * b + 4 * g4 + i;
                            if (tok < lo || tok >= hi) s[nb][b][i] = NEG_INF;
                        }
            }
            // ---- softmax of every row block -> P^T fragments (B operand of PV)
            u32x4 pb[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                float x[8];
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int i = 0; i < 4; ++i) x[4 * b + i] = s[nb][b][i];
                const float lm = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])),
                                       fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
                const bool need = lm * c > m[nb] + TAU;
                if (__builtin_amdgcn_ballot_w64(need)) {  // wave-uniform, rare after the first step
                    const float mn = fmaxf(m[nb], xor_max(lm) * c);
                    const float alpha = fast_exp2(m[nb] - mn);
                    z[nb] *= alpha;
#pragma unroll
                    for (int db = 0; db < DB; ++db) o[nb][db] *= alpha;
                    m[nb] = mn;
                }
                float pr[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) pr[i] = fast_exp2(__builtin_fmaf(x[i], c, -m[nb]));
                pb[nb] = u32x4{O::pack(pr[0], pr[1]), O::pack(pr[2], pr[3]), O::pack(pr[4], pr[5]),
                               O::pack(pr[6], pr[7])};
            }
            // ---- O^T += V^T P^T (each V^T fragment feeds NB MFMAs), then QK of step k+1
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) o[nb][db] = O::mma_k32(vf[db], pb[nb], o[nb][db]);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) z[nb] = O::mma_k32(ones, pb[nb], z[nb]);
            if (more) qk(kf, qf, s);
        }
    }
};

// Work item of linear block b of n: block b runs on XCD b % 8, and every XCD
// gets a contiguous range of items, so that row tiles of one (job, head)
// share its L2.
__device__ inline int xcd_item(int b, int n) {
    const int xcd = b & 7, slot = b >> 3;
    const int q8 = n >> 3, rm = n & 7;
    return xcd * q8 + min(xcd, rm) + slot;
}

// The waves of a work item meet at a barrier, unless one wave works alone on
// its own LDS stage (SOLO), where its own vmcnt wait orders copy and reads.
template <bool SOLO>
__device__ inline void item_barrier() {
    if constexpr (!SOLO) __builtin_amdgcn_s_barrier();
}

// One work item (job, first row, KV head) of the tile kernels: NW waves, NB
// 16-row blocks per wave, STAGES LDS stages at `lds`.  The item holds rows
// [row0, row0 + item_rows) of its job.  SOLO: one wave alone (tid = its lane).
template <int D, bool FP16, int NB, int NW, int STAGES, bool SOLO = false>
__device__ __forceinline__ void tile_item(const SegParams &p, const int32_t *__restrict__ items, int item,
                                          u16 *lds, int tid, int item_rows) {
    using T = Tile<D>;
    using M = TileMath<D, FP16, NB, NW>;
    constexpr int KS = M::KS;
    constexpr int BPW = T::NBLK / NW;  // copies per wave per tile
    static_assert(T::NBLK % NW == 0, "every wave copies the same number of blocks");
    static_assert(STAGES >= 1 && STAGES <= 3, "one to three LDS stages");
    static_assert(!SOLO || (NW == 1 && STAGES == 1), "a wave alone has one stage");
    const int job = items[3 * item], row0 = items[3 * item + 1], h = items[3 * item + 2];

    const int lane = tid & 63, wave = SOLO ? 0 : tid >> 6;
    const int row = lane & 15, g4 = lane >> 4;
    const int kst = p.kstart[job];
    const int ntok = max(0, min(p.klen[job], p.tcap - kst));
    const int kend = kst + ntok;
    const int nrows = min(p.qlen[job] * p.group, row0 + item_rows);
    const int wrow0 = row0 + 16 * NB * wave;
    const bool active = wrow0 < nrows;

    // Q^T fragments (B operand): lane (row, g4) holds d = 32*ks + 8*g4 .. +7.
    u32x4 qf[NB][KS];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int rr = wrow0 + 16 * nb + row;
        if (rr < nrows) {
            const int lr = rr / p.group, gg = rr - lr * p.group;
            const int rq = p.qids[(size_t)job * p.maxr + lr];
            const u16 *src = p.q + ((size_t)rq * p.hq + h * p.group + gg) * D + 8 * g4;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) qf[nb][ks] = *(const u32x4 *)(src + 32 * ks);
        } else {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) qf[nb][ks] = u32x4{0, 0, 0, 0};
        }
    }
    // Pin the Q fragments: an empty asm that "redefines" them makes the wave
    // wait for the Q loads once, here, and not inside the tile loop behind the
    // copies in flight.
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+v"(qf[nb][ks]));

    M acc;
    acc.reset();
    const LdsOfs of = T::offsets(row, g4);

    const int tb0 = kst & ~7;
    const int ntiles = ntok > 0 ? (kend - tb0 + T::TT - 1) / T::TT : 0;
    if (STAGES == 1) {
        // one stage (one-wave workgroups, four per CU): copy, wait, compute
        for (int it = 0; it < ntiles; ++it) {
            const int t0 = tb0 + it * T::TT;
            if (it > 0) item_barrier<SOLO>();  // every wave is done with the previous tile
            acc.copy(lds, p.kp, p.vp, h, p.tcap, t0, kst, kend, wave, lane);
            __builtin_amdgcn_s_waitcnt(TA_VMCNT(0));
            item_barrier<SOLO>();
            if (active) acc.tile(lds, qf, of, max(0, kst - t0), min(T::TT, kend - t0), g4, p.scale_log2);
        }
    } else {
    // Iteration it copies tile it+STAGES-1 and computes tile it (stage it %
    // STAGES); the first STAGES-1 iterations only copy, so every copy comes
    // from one call site.
    constexpr int AHEAD = STAGES > 1 ? STAGES - 1 : 1;
    int cs = STAGES - AHEAD;  // stage of tile it, starting at it = -AHEAD
    for (int it = -AHEAD; it < ntiles; ++it) {
        if (it >= 0) {
            // this wave's copies of tile it are done once at most those of the
            // tiles after it (issued, at most AHEAD-1 of them) are pending
            if (AHEAD == 2 && it + 1 < ntiles)
                __builtin_amdgcn_s_waitcnt(TA_VMCNT(BPW));
            else
                __builtin_amdgcn_s_waitcnt(TA_VMCNT(0));
            item_barrier<SOLO>();  // every copy of tile it landed; stage of tile it-1 is free
        }
        const int ns = cs == 0 ? STAGES - 1 : cs - 1;  // stage of tile it+AHEAD (that of tile it-1)
        const int t0 = tb0 + it * T::TT;
        acc.step(lds + cs * T::ELEMS, lds + ns * T::ELEMS, it + AHEAD < ntiles, it >= 0 && active, p.kp, p.vp, h,
                 p.tcap, t0 + AHEAD * T::TT, kst, kend, wave, lane, qf, of, max(0, kst - t0),
                 min(T::TT, kend - t0), g4, p.scale_log2);
        cs = cs == STAGES - 1 ? 0 : cs + 1;
    }
    }

    if (!active) return;
    const int rb = p.rowbase[job];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int grow = wrow0 + 16 * nb + row;
        if (grow >= nrows) continue;
        const int lr = grow / p.group, gg = grow - lr * p.group;
        const size_t prow = (size_t)(rb + lr) * p.hq + h * p.group + gg;
        store_partial<M::DB>(p.part, p.lse, prow, acc.o[nb], acc.m[nb], acc.z[nb][0], g4);
    }
}

template <int D, bool FP16, int NB, int NW, int STAGES>
__global__ __launch_bounds__(64 * NW) void seg_tile_kernel(SegParams p) {
    __shared__ __attribute__((aligned(16))) u16 lds[STAGES * Tile<D>::ELEMS];
    tile_item<D, FP16, NB, NW, STAGES>(p, p.items, xcd_item(blockIdx.x, gridDim.x), lds, threadIdx.x, 16 * NB * NW);
}

// ------------------------------------------------------------------------
// Pipelined large-tile kernel.  The 32-token steps of a work item form one
// software pipeline that runs across tile boundaries; within a step the
// matrix cores and the VALU work on different steps:
//
//   block(g):  QK of step g+1 (MFMA)   || exponentials of step g (VALU),
//                                          LDS reads of V(g)
//              PV + row sums of step g  || LDS reads of K(g+2), masking and
//                                          row maxima of step g+1
//
// and the rare online-softmax rescale runs between blocks.  The order inside
// a block is pinned with sched_group_barrier so that MFMAs and VALU
// instructions alternate in each wave's instruction stream.  K/V tiles arrive
// by LDS DMA into five stages: tiles t and t+1 are read while t+2 .. t+4 are
// in flight, with one barrier per tile.
template <int D, bool FP16, int NW, int NB_ = 2>
struct PipeMath {
    static constexpr int NB = NB_;
    static constexpr int DB = D / 16;
    static constexpr int KS = D / 32;
    using O = Ops<FP16>;
    using T = Tile<D>;
    using TM = TileMath<D, FP16, NB, NW>;

    f32x4 o[NB][DB], z[NB];
    float m[NB], lm[NB], thr[NB];  // running max (scaled), raw row max of the staged step, (m + TAU) / c
    f32x4 s[NB][2];      // scores of the step whose exponentials come next
    u32x4 kf[2][KS];     // K fragments of the next QK step
    u32x4 vf[DB];        // V^T fragments of the current PV step

    __device__ void reset() {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            m[nb] = thr[nb] = NEG_INF;
            z[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int db = 0; db < DB; ++db) o[nb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }

    // Scores of a step: mask tokens outside [lo, hi) (if MASK) and take the
    // lane-local row maxima.
    template <bool MASK>
    __device__ void finish_scores(f32x4 (&sn)[NB][2], int lo, int hi, int g4) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            if (MASK) {
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int tok = 16 * b + 4 * g4 + i;
                        if (tok < lo || tok >= hi) sn[nb][b][i] = NEG_INF;
                    }
            }
            float mx = sn[nb][0][0];  // a chain, so that it becomes three-input maxima
#pragma unroll
            for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sn[nb][i >> 2][i & 3]);
            lm[nb] = mx;
            s[nb][0] = sn[nb][0];
            s[nb][1] = sn[nb][1];
        }
    }

    // The running maxima from the job's first scored step: O and z are still
    // zero, so the maxima are set without the pass over O that rescale makes
    // (the values equal rescale's from the initial state).
    __device__ void first_max(float c, float rc) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const float mn = xor_max(lm[nb]) * c;
            m[nb] = mn;
            thr[nb] = (mn + TAU) * rc;
        }
    }

    // Raise the running maxima where a score of the staged step exceeds them
    // by more than TAU (wave-uniform branch, rare after the first step).
    __device__ void rescale(float c, float rc) {  // rc = 1 / c
        bool need = false;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) need |= lm[nb] > thr[nb];
        if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const float mn = fmaxf(m[nb], xor_max(lm[nb]) * c);
                const float alpha = mn == NEG_INF ? 1.f : fast_exp2(m[nb] - mn);
                z[nb] *= alpha;
#pragma unroll
                for (int db = 0; db < DB; ++db) o[nb][db] *= alpha;
                m[nb] = mn;
                thr[nb] = (mn + TAU) * rc;  // raw-score threshold of the next rescale
            }
        }
    }

    // One pipeline block (see above).  vs / vbase: stage and offset of V(g);
    // ks / kbase: of K(g+2) (any resident step when there is none); lo / hi:
    // valid tokens of step g+1.  Every fragment register set is reloaded only
    // after its last reader: V(g) during QK(g+1), K(g+2) during PV(g).
    template <bool MORE, bool MASKN, bool ROWMASK = false>
    __device__ __forceinline__ void block(const u16 *__restrict__ vs, int vbase, const u16 *__restrict__ ks,
                                          int kbase, const u32x4 (&qf)[NB][KS], const LdsOfs &of, int lo,
                                          int hi, int g4, float c, unsigned keep = ~0u) {
        const u32x4 ones = {O::ONE2, O::ONE2, O::ONE2, O::ONE2};
        f32x4 sn[NB][2];
        if (MORE) TM::qk(kf, qf, sn);
        TM::load_v(vs, of, vbase, vf);
        u32x4 pb[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            float pr[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) pr[i] = fast_exp2(__builtin_fmaf(s[nb][i >> 2][i & 3], c, -m[nb]));
            pb[nb] = u32x4{O::pack(pr[0], pr[1]), O::pack(pr[2], pr[3]), O::pack(pr[4], pr[5]),
                           O::pack(pr[6], pr[7])};
            if (ROWMASK && !((keep >> nb) & 1)) pb[nb] = u32x4{0u, 0u, 0u, 0u};
        }
        if (MORE) {
            // 2*KS*NB QK MFMAs; the V reads go out with the first half of them
#pragma unroll
            for (int i = 0; i < 2 * KS * NB; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                if (i < DB) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
                __builtin_amdgcn_sched_group_barrier(0x400, 1, 0);  // transcendental
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // K(g+1) is dead only after QK(g+1)
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) o[nb][db] = O::mma_k32(vf[db], pb[nb], o[nb][db]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) z[nb] = O::mma_k32(ones, pb[nb], z[nb]);
        if (MORE) {
            TM::load_k(ks, of, kbase, kf);
            finish_scores<MASKN>(sn, lo, hi, g4);
        }
        // instruction order: QK MFMAs alternate with the exponentials and the
        // V reads, then PV MFMAs alternate with the K reads and the score epilogue
        if (MORE) {
            // DB*NB PV MFMAs; the K reads go out with the first half of them
#pragma unroll
            for (int i = 0; i < DB * NB; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // MFMA
                if (i < 2 * KS) __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x002, 1, 1);  // VALU
            }
        }
    }

    // One staged tile of an attached private segment (after the pipeline has
    // drained): tokens [lo, hi) of the tile, for this wave's rows [rlo, rhi)
    // only.  Other rows get P = 0 and keep their running maxima, so their
    // state is unchanged.
    __device__ void tail_tile(const u16 *__restrict__ st, const u32x4 (&qf)[NB][KS], const LdsOfs &of, int lo,
                              int hi, int rlo, int rhi, int row, int g4, float c, float rc) {
        unsigned keep = 0;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) keep |= (unsigned)(16 * nb + row >= rlo && 16 * nb + row < rhi) << nb;
#pragma unroll
        for (int k = 0; k < T::TT / 32; ++k) {
            const int base = 32 * k;
            if (base >= hi) break;
            f32x4 sn[NB][2];
            TM::load_k(st, of, base, kf);
            TM::qk(kf, qf, sn);
            if (lo <= base && hi >= base + 32)  // wave-uniform: every token of the step is the segment's
                finish_scores<false>(sn, 0, 32, g4);
            else
                finish_scores<true>(sn, lo - base, hi - base, g4);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                if (!((keep >> nb) & 1)) lm[nb] = NEG_INF;
            rescale(c, rc);
            block<false, false, true>(st, base, st, 0, qf, of, 0, 32, g4, c, keep);
        }
    }
};

#ifndef TA_PIPE_STAGES
#define TA_PIPE_STAGES 5
#endif
#ifndef TA_PIPE_PRO
#define TA_PIPE_PRO 3  // measured: 3 of 5 tiles in the prologue start the loop earliest
#endif

// STAGES LDS tiles; the waves meet at a barrier every SYNC tiles.  While the
// waves work on tiles t .. t+SYNC-1 they read those and the K of tile t+SYNC
// (the pipelined steps read one step ahead), so SYNC+1 tiles are resident
// and STAGES-SYNC-1 more can be in flight.  The prologue issues PRO tiles;
// the first loop barrier issues the rest of the ring.
// One 256-row work item of the pipelined kernel, with its attached segments
// (p.xtail, indexed by the item), STAGES LDS stages at `lds`.
template <int D, bool FP16, int NW, int NB = 2, int STAGES = TA_PIPE_STAGES, int SYNC = 1, int PRO = TA_PIPE_PRO>
__device__ __forceinline__ void pipe_item(const SegParams &p, const int32_t *__restrict__ items, int item, u16 *lds,
                                          int tid) {
    using T = Tile<D>;
    using M = PipeMath<D, FP16, NW, NB>;
    using TM = TileMath<D, FP16, NB, NW>;
    constexpr int KS = M::KS;
    constexpr int BPW = T::NBLK / NW;  // copies per wave per tile
    static_assert(T::NBLK % NW == 0, "every wave copies the same number of blocks");
    static_assert(SYNC >= 1 && STAGES >= 2 * SYNC + 1 && STAGES <= 5,
                  "a group's tiles, the next K and the next group's copies fit the stages");
    static_assert(PRO >= SYNC + 1 && PRO <= STAGES, "the prologue issues the tiles the first group reads");
    const int job = items[3 * item], row0 = items[3 * item + 1], h = items[3 * item + 2];

    const int lane = tid & 63, wave = tid >> 6;
    const int row = lane & 15, g4 = lane >> 4;
    const int kst = p.kstart[job];
    const int ntok = max(0, min(p.klen[job], p.tcap - kst));
    const int kend = kst + ntok;
    const int nrows = p.qlen[job] * p.group;
    const int wrow0 = row0 + 16 * NB * wave;
    const bool active = wrow0 < nrows;
    const float c = p.scale_log2, rc = 1.f / p.scale_log2;
    const int tb0 = kst & ~7;
    const int ntiles = ntok > 0 ? (kend - tb0 + T::TT - 1) / T::TT : 0;
    const int nsteps = ntok > 0 ? (kend - tb0 + 31) / 32 : 0;
    auto tile_stage = [&](int t) { return lds + (t % STAGES) * T::ELEMS; };
    auto stage = [&](int g) { return tile_stage(g >> 1); };  // stage of step g's tile

    // Attached segments (xtail record of this item: count, then (first token,
    // tokens, first job row, rows) for up to TA_XTAIL_MAX segments)
    // follow the job's own tiles in one tile sequence through the same LDS
    // stages.  The record is read at once (constant address space: one batch
    // of scalar loads, no chain of dependent loads) into per-segment values
    // that unrolled loops index with constants.
    constexpr int XM = TA_XTAIL_MAX;
    constexpr int XF = 4;  // fields per segment
    int rec[1 + XF * XM];
    if (p.xtail) {
        const __attribute__((address_space(4))) int32_t *xt =
            (const __attribute__((address_space(4))) int32_t *)(p.xtail + (size_t)item * p.xtail_stride);
#pragma unroll
        for (int i = 0; i < 1 + XF * XM; ++i) rec[i] = xt[i];
    } else {
#pragma unroll
        for (int i = 0; i < 1 + XF * XM; ++i) rec[i] = 0;
    }
    const int nx = min(max(rec[0], 0), XM);
    int xs[XM], xe[XM], xfirst[XM], xn[XM];  // clamped token range, first tile and tiles of each segment
    int ntot = ntiles;
#pragma unroll
    for (int k = 0; k < XM; ++k) {
        xs[k] = max(0, rec[1 + XF * k]);
        xe[k] = xs[k] + max(0, min(rec[2 + XF * k], p.tcap - xs[k]));
        xn[k] = k < nx && xe[k] > xs[k] ? (xe[k] - (xs[k] & ~7) + T::TT - 1) / T::TT : 0;
        xfirst[k] = ntot;
        ntot += xn[k];
    }
    // copy tile t of the sequence into stage st
    auto copy_tile = [&](int t, u16 *st) {
        if (t < ntiles) {
            TM::copy(st, p.kp, p.vp, h, p.tcap, tb0 + t * T::TT, kst, kend, wave, lane);
            return;
        }
        int t0n = 0, cs = 0, ce = 1;
#pragma unroll
        for (int k = 0; k < XM; ++k)
            if (t >= xfirst[k] && t < xfirst[k] + xn[k]) {
                t0n = (xs[k] & ~7) + (t - xfirst[k]) * T::TT;
                cs = xs[k];
                ce = xe[k];
            }
        TM::copy(st, p.kp, p.vp, h, p.tcap, t0n, cs, ce, wave, lane);
    };

    int issued = 0;  // tiles of the sequence whose copies this wave has issued

    // Prologue.  Loads retire in order, and a wait for a load's result also
    // waits for every copy issued before it, so the dependent chain
    // (request ids -> Q rows) is kept short.  A job over consecutive requests
    // (qbase[job] >= 0, cf. the reference's contiguous-Q path,
    // kernels.py:23-26) addresses its Q rows from the first request id, a
    // scalar load beside the job's other metadata: the Q loads go out before
    // tile 0's copies.  Otherwise tile 0's copies go out with the request-id
    // loads (both are needed before the first step), then the Q loads.  Every
    // lane loads a valid row (rows past the job are zeroed afterwards); tiles
    // 1 .. PRO-1 follow.
    const int qb = p.qbase ? p.qbase[job] : -1;
    int rq[NB];
    if (qb < 0 && ntot > 0) copy_tile(0, lds);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int rr = max(0, min(wrow0 + 16 * nb + row, nrows - 1));
        rq[nb] = qb >= 0 ? qb + rr / p.group : p.qids[(size_t)job * p.maxr + rr / p.group];
    }
    u32x4 qf[NB][KS];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int rr = max(0, min(wrow0 + 16 * nb + row, nrows - 1));
        const u16 *src = p.q + ((size_t)rq[nb] * p.hq + h * p.group + rr % p.group) * D + 8 * g4;
#pragma unroll
        for (int k = 0; k < KS; ++k) qf[nb][k] = *(const u32x4 *)(src + 32 * k);
    }
    if (qb >= 0 && ntot > 0) copy_tile(0, lds);  // behind the Q loads: one wait covers both
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const bool valid = wrow0 + 16 * nb + row < nrows;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            if (!valid) qf[nb][k] = u32x4{0, 0, 0, 0};
            asm volatile("" : "+v"(qf[nb][k]));
        }
    }
    for (int t = 1; t < PRO && t < ntot; ++t) copy_tile(t, tile_stage(t));
    issued = min(PRO, ntot);

    M acc;
    acc.reset();
    const LdsOfs of = T::offsets(row, g4);

    wait_tiles<BPW>(issued - 1);  // tile 0 landed (tiles 1 .. PRO-1 may be in flight)
    __builtin_amdgcn_s_barrier();
    if (active && nsteps > 0) {
        f32x4 s0[NB][2];
        TM::load_k(lds, of, 0, acc.kf);
        TM::qk(acc.kf, qf, s0);
        acc.template finish_scores<true>(s0, kst - tb0, kend - tb0, g4);
        acc.first_max(c, rc);
        if (nsteps > 1) TM::load_k(lds, of, 32, acc.kf);
    }

    // Entering tile t (at step 2t): at the start of a group (t % SYNC == 0)
    // tiles t+1 .. t+SYNC must have landed (the earlier ones were waited for
    // at the previous group); the later issued ones may still be in flight.
    // Once every wave passed the barrier the stages of the previous group are
    // free for tiles up to t+STAGES-1.
    auto sync_tile = [&](int t) {
        if (t % SYNC != 0 || t + 1 >= ntot) return;
        wait_tiles<BPW>(max(0, issued - 1 - (t + SYNC)));
        __builtin_amdgcn_s_barrier();
        for (; issued < min(t + STAGES, ntot); ++issued) copy_tile(issued, tile_stage(issued));
    };
    // steady state: steps whose successor is neither the last nor masked
    int g = 0;
    for (; g + 2 < nsteps; ++g) {
        if (!(g & 1)) sync_tile(g >> 1);
        if (active) {
            const int gk = g + 2;
            acc.template block<true, false>(stage(g), 32 * (g & 1), stage(gk), 32 * (gk & 1), qf, of, 0, 32,
                                            g4, c);
            acc.rescale(c, rc);
        }
    }
    // the last two steps: the successor of step nsteps-2 may be masked at its end
    if (g + 1 < nsteps) {
        if (!(g & 1)) sync_tile(g >> 1);
        if (active) {  // one (masked) form for either end of the job keeps the register allocation simple
            acc.template block<true, true>(stage(g), 32 * (g & 1), stage(g + 1), 32 * ((g + 1) & 1), qf, of,
                                           0, kend - (tb0 + 32 * (g + 1)), g4, c);
            acc.rescale(c, rc);
        }
        ++g;
    }
    if (g < nsteps) {
        if (!(g & 1)) sync_tile(g >> 1);
        if (active) acc.template block<false, false>(stage(g), 32 * (g & 1), stage(g), 0, qf, of, 0, 32, g4, c);
    }

    // Attached segments, in rounds of up to STAGES tiles that are resident
    // together: one wait and one barrier per round, then every wave attends
    // the round's tiles of the segments holding its rows, side by side.  The
    // root loop (or the prologue) already issued the first tiles.
    {
        for (int r0 = ntiles; r0 < ntot; r0 += STAGES) {
            const int r1 = min(r0 + STAGES, ntot);
            __builtin_amdgcn_s_barrier();  // every wave is done with the tiles before r0
            for (; issued < r1; ++issued) copy_tile(issued, tile_stage(issued));
            __builtin_amdgcn_s_waitcnt(TA_VMCNT(0));
            __builtin_amdgcn_s_barrier();  // the round's tiles landed
#pragma unroll
            for (int k = 0; k < XM; ++k) {
                // segment rows relative to this wave's: [rlo, rlo + rows); with 16 rows per
                // wave (NB = 1) a segment may span two waves, each attends its own rows
                const int rlo = rec[3 + XF * k] - wrow0;
                if (xn[k] > 0 && active && rlo < 16 * NB && rlo + rec[4 + XF * k] > 0) {
                    for (int i = max(0, r0 - xfirst[k]); i < xn[k] && xfirst[k] + i < r1; ++i) {
                        const int t0 = (xs[k] & ~7) + i * T::TT;
                        acc.tail_tile(tile_stage(xfirst[k] + i), qf, of, max(0, xs[k] - t0), min(T::TT, xe[k] - t0),
                                      rlo, rlo + rec[4 + XF * k], row, g4, c, rc);
                    }
                }
            }
        }
    }

    if (!active) return;
    const int rb = p.rowbase[job];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int grow = wrow0 + 16 * nb + row;
        if (grow >= nrows) continue;
        const int lr = grow / p.group, gg = grow - lr * p.group;
        const size_t prow = (size_t)(rb + lr) * p.hq + h * p.group + gg;
        store_partial<M::DB>(p.part, p.lse, prow, acc.o[nb], acc.m[nb], acc.z[nb][0], g4);
    }
}

// A 256-row work item whose job has at most 8 NW rows from the item's first
// row on runs 16 rows per wave, so that every wave computes (two per SIMD)
// instead of half of them 32 rows each; the arithmetic of every row is the same.
template <int D, bool FP16, int NW>
__device__ __forceinline__ void pipe_item_rows(const SegParams &p, const int32_t *__restrict__ items, int item,
                                               u16 *lds, int tid) {
    const int job = items[3 * item], row0 = items[3 * item + 1];
    if (p.qlen[job] * p.group - row0 <= 16 * NW)
        pipe_item<D, FP16, NW, 1>(p, items, item, lds, tid);
    else
        pipe_item<D, FP16, NW, 2>(p, items, item, lds, tid);
}

template <int D, bool FP16, int NW>
__global__ __launch_bounds__(64 * NW) void seg_pipe_kernel(SegParams p) {
    __shared__ __attribute__((aligned(16))) u16 lds[TA_PIPE_STAGES * Tile<D>::ELEMS];
    pipe_item_rows<D, FP16, NW>(p, p.items, xcd_item(blockIdx.x, gridDim.x), lds, threadIdx.x);
}

// Work items of several kinds of one layer in one launch of 512-thread
// workgroups: blocks [0, base[1]) run 256-row items (with their attached
// segments), blocks [base[1], base[2]) run 64-row items on eight waves (the
// upper four copy and meet at the barriers), and the blocks from base[2] on
// run four small items each, one per wave on its own stage (the upper four
// waves end at once).  The bases are multiples of 8, so that every kind's
// items map to XCDs as in its own kernel; blocks past a kind's item count end
// at once.  The kinds run side by side instead of one launch after another.
template <int D, bool FP16>
__global__ __launch_bounds__(512) void seg_mix_kernel(MixParams mp) {
    using T = Tile<D>;
    __shared__ __attribute__((aligned(16))) u16 lds[TA_PIPE_STAGES * T::ELEMS];
    static_assert(TA_PIPE_STAGES >= 4 && 3 <= TA_PIPE_STAGES, "four small stages and three 64-row stages fit");
    const int b = blockIdx.x, tid = threadIdx.x;
    if (b < mp.base[1]) {
        if (b >= mp.n[0]) return;
        pipe_item_rows<D, FP16, 8>(mp.p, mp.items[0], xcd_item(b, mp.n[0]), lds, tid);
    } else if (b < mp.base[2]) {
        const int lb = b - mp.base[1];
        if (lb >= mp.n[1]) return;
        tile_item<D, FP16, 1, 8, 3>(mp.p, mp.items[1], xcd_item(lb, mp.n[1]), lds, tid, 64);
    } else {
        const int wave = tid >> 6, it = 4 * (b - mp.base[2]) + wave;
        if (wave >= 4 || it >= mp.n[2]) return;
        tile_item<D, FP16, 1, 1, 1, true>(mp.p, mp.items[2], it, lds + wave * T::ELEMS, tid & 63, 16);
    }
}

// ------------------------------------------------------------------------
// Tail kernel with the merge fused in (TA_TAIL items with out given).  One
// two-wave workgroup per (tail job, KV head): the job's single request has
// G = hq/hk query rows for this head, and every other partial slot of the
// request was written by an earlier launch on the stream (the job's own slot
// is the request's last).  The two waves work side by side:
//   wave 0 attends the tail (the small-job tile loop) and leaves its
//          normalised partial and log-sum-exp in LDS;
//   wave 1 loads the other slots, PF float4 registers per round, and merges
//          them by the online log-sum-exp of the merge kernel; lane l owns
//          units u = l + 64k (k < UPL) of the G*D/4 float4 units, unit u =
//          (row u / (D/4), d = 4 (u % (D/4))).
// After one barrier wave 1 merges the own partial and writes the output rows.
template <int D, bool FP16, int UPL>
__global__ __launch_bounds__(128) void seg_tail_kernel(SegParams p) {
    using T = Tile<D>;
    using M = TileMath<D, FP16, 1, 1>;
    constexpr int KS = M::KS, DB = M::DB;
    constexpr int PF = 32;          // units of one merge round
    constexpr int CH = PF / UPL;    // slots per merge round
    constexpr int DU = D / 4;       // units per row
    constexpr float LOG2E = 1.44269504088896341f;
    __shared__ __attribute__((aligned(16))) u16 lds[T::ELEMS];
    float *opart = reinterpret_cast<float *>(lds);  // [G][D] own normalised partial, after the tile loop
    float *olse = opart + 16 * D;                   // [G] own log-sum-exp, log2 units

    const int item = blockIdx.x;
    const int job = p.items[3 * item], h = p.items[3 * item + 2];
    const int G = p.group;
    const int lane = threadIdx.x & 63;
    const int r = p.qids[(size_t)job * p.maxr];

    if (threadIdx.x < 64) {
        // ---- wave 0: the tail's attention
        const int row = lane & 15, g4 = lane >> 4;
        const int kst = p.kstart[job];
        const int ntok = max(0, min(p.klen[job], p.tcap - kst));
        const int kend = kst + ntok;
        const int tb0 = kst & ~7;
        const int ntiles = ntok > 0 ? (kend - tb0 + T::TT - 1) / T::TT : 0;
        if (ntiles > 0) M::copy(lds, p.kp, p.vp, h, p.tcap, tb0, kst, kend, 0, lane);
        u32x4 qf[1][KS];
        {
            const int rr = row < G ? row : 0;  // rows past G repeat row 0 and are never stored
            const u16 *src = p.q + ((size_t)r * p.hq + h * G + rr) * D + 8 * g4;
#pragma unroll
            for (int k = 0; k < KS; ++k) qf[0][k] = *(const u32x4 *)(src + 32 * k);
        }
        M acc;
        acc.reset();
        const LdsOfs of = T::offsets(row, g4);
        for (int it = 0; it < ntiles; ++it) {
            const int t0 = tb0 + it * T::TT;
            if (it > 0) M::copy(lds, p.kp, p.vp, h, p.tcap, t0, kst, kend, 0, lane);
            __builtin_amdgcn_s_waitcnt(TA_VMCNT(0));
            acc.tile(lds, qf, of, max(0, kst - t0), min(T::TT, kend - t0), g4, p.scale_log2);
        }
        // the tile's reads fed the MFMAs above, so the stage is free for the partial
        const bool any = acc.m[0] != NEG_INF;
        const float zr = acc.z[0][0];
        const float inv = any ? 1.f / zr : 0.f;
        if (row < G) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
                *(f32x4 *)(opart + row * D + 16 * db + 4 * g4) = acc.o[0][db] * inv;
            if (g4 == 0) olse[row] = any ? acc.m[0] + __builtin_amdgcn_logf(zr) : NEG_INF;
        }
        __syncthreads();
        return;
    }

    // ---- wave 1: merge the request's other slots
    const int own = p.rowbase[job];
    const int cnt = p.counts[r] - 1;
    const int32_t *slr = p.slots + (size_t)r * p.maxs;
    const int units = G * DU;
    float Mx[UPL], Z[UPL];
    f32x4 o[UPL];
#pragma unroll
    for (int k = 0; k < UPL; ++k) {
        Mx[k] = NEG_INF;
        Z[k] = 0.f;
        o[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int s0 = 0; s0 < cnt; s0 += CH) {
        float l[CH][UPL];
        int e[CH][UPL];
        u32x2 v[CH][UPL];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int si = s0 + c;
            const int sl = slr[min(si, cnt - 1)];
            const bool use = si < cnt && sl != own;
#pragma unroll
            for (int k = 0; k < UPL; ++k) {
                const int u = min(lane + 64 * k, units - 1);
                const size_t prow = (size_t)sl * p.hq + h * G + u / DU;
                const u32x2 x = *(const u32x2 *)(p.part + prow * D + part_pos(u % DU));
                const float lx = p.lse[2 * prow], ex = p.lse[2 * prow + 1];
                l[c][k] = use ? lx * LOG2E : NEG_INF;
                e[c][k] = (int)ex;
                v[c][k] = use ? x : u32x2{0u, 0u};
            }
        }
#pragma unroll
        for (int k = 0; k < UPL; ++k) {
            float cm = Mx[k];
#pragma unroll
            for (int c = 0; c < CH; ++c) cm = fmaxf(cm, l[c][k]);
            const float alpha = Mx[k] == NEG_INF ? 0.f : fast_exp2(Mx[k] - cm);
            Z[k] *= alpha;
            o[k] *= alpha;
            Mx[k] = cm;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const float w = l[c][k] == NEG_INF ? 0.f : fast_exp2(l[c][k] - cm);
                Z[k] += w;
                o[k] += __builtin_amdgcn_ldexpf(w, e[c][k]) * unpack_f16x4(v[c][k]);
            }
        }
    }
    __syncthreads();  // wave 0's partial is in LDS
#pragma unroll
    for (int k = 0; k < UPL; ++k) {
        const int u = lane + 64 * k;
        if (u >= units) continue;
        const float lo = olse[u / DU];
        const f32x4 vo = *(const f32x4 *)(opart + (u / DU) * D + 4 * (u % DU));
        const float cm = fmaxf(Mx[k], lo);
        const float alpha = Mx[k] == NEG_INF ? 0.f : fast_exp2(Mx[k] - cm);
        const float w = lo == NEG_INF ? 0.f : fast_exp2(lo - cm);
        const float zt = Z[k] * alpha + w;
        const f32x4 a = (o[k] * alpha + w * vo) * (zt > 0.f ? 1.f / zt : 0.f);
        u16 *dst = p.out + ((size_t)r * p.hq + h * G + u / DU) * D + 4 * (u % DU);
        *(u32x2 *)dst = u32x2{Ops<FP16>::pack(a[0], a[1]), Ops<FP16>::pack(a[2], a[3])};
    }
}

template <int D, bool FP16>
hipError_t launch_tail_merge(const SegParams &sp, hipStream_t stream) {
    // float4 units per lane: G*D/4 units over 64 lanes
    const int units = sp.group * (D / 4);
    if (units <= 64)
        TA_LAUNCH((seg_tail_kernel<D, FP16, 1>), dim3(sp.n_items), dim3(128), stream, sp);
    else if (units <= 128)
        TA_LAUNCH((seg_tail_kernel<D, FP16, 2>), dim3(sp.n_items), dim3(128), stream, sp);
    else if (units <= 256)
        TA_LAUNCH((seg_tail_kernel<D, FP16, 4>), dim3(sp.n_items), dim3(128), stream, sp);
    else if (units <= 512)
        TA_LAUNCH((seg_tail_kernel<D, FP16, 8>), dim3(sp.n_items), dim3(128), stream, sp);
    else
        return hipErrorNotSupported;
    return hipGetLastError();
}

template <int D, bool FP16>
hipError_t launch_d(const SegParams &sp, int kind, hipStream_t stream) {
    switch (kind) {
        case TA_SMALL:  // one wave per (job, head); one stage so that four fit on a CU
            TA_LAUNCH((seg_tile_kernel<D, FP16, 1, 1, 1>), dim3(sp.n_items), dim3(64), stream, sp);
            break;
        case TA_TAIL:  // as TA_SMALL, merging the request into out when out is given
            if (sp.out) return launch_tail_merge<D, FP16>(sp, stream);
            TA_LAUNCH((seg_tile_kernel<D, FP16, 1, 1, 1>), dim3(sp.n_items), dim3(64), stream, sp);
            break;
        case TA_LARGE64:
            TA_LAUNCH((seg_tile_kernel<D, FP16, 1, 4, 3>), dim3(sp.n_items), dim3(256), stream, sp);
            break;
        case TA_LARGE128:
            TA_LAUNCH((seg_tile_kernel<D, FP16, 2, 4, 3>), dim3(sp.n_items), dim3(256), stream, sp);
            break;
        case TA_LARGE256:
            TA_LAUNCH((seg_pipe_kernel<D, FP16, 8>), dim3(sp.n_items), dim3(512), stream, sp);
            break;
        default:
            return hipErrorNotSupported;
    }
    return hipGetLastError();
}

template <int D, bool FP16>
hipError_t launch_mix_d(const MixParams &mp, int blocks, hipStream_t stream) {
    TA_LAUNCH((seg_mix_kernel<D, FP16>), dim3(blocks), dim3(512), stream, mp);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_tile_mix(const SegParams &sp, const int32_t *const items[3], const int n[3], int d, bool fp16,
                           hipStream_t stream) {
    if (sp.tcap % 8 != 0) return hipErrorNotSupported;
    MixParams mp;
    mp.p = sp;
    int base = 0;
    for (int k = 0; k < 3; ++k) {
        mp.items[k] = items[k];
        mp.n[k] = n[k] > 0 ? n[k] : 0;
        mp.base[k] = base;
        const int blocks = k < 2 ? mp.n[k] : (mp.n[k] + 3) / 4;
        base += (blocks + 7) & ~7;
    }
    const int blocks = mp.base[2] + (mp.n[2] + 3) / 4;
    if (blocks <= 0) return hipSuccess;
    switch (d) {
        case 128: return fp16 ? launch_mix_d<128, true>(mp, blocks, stream) : launch_mix_d<128, false>(mp, blocks, stream);
        case 64: return fp16 ? launch_mix_d<64, true>(mp, blocks, stream) : launch_mix_d<64, false>(mp, blocks, stream);
        case 32: return fp16 ? launch_mix_d<32, true>(mp, blocks, stream) : launch_mix_d<32, false>(mp, blocks, stream);
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_tile(const SegParams &sp, int kind, int d, bool fp16, hipStream_t stream) {
    if (sp.tcap % 8 != 0) return hipErrorNotSupported;
    switch (d) {
        case 128: return fp16 ? launch_d<128, true>(sp, kind, stream) : launch_d<128, false>(sp, kind, stream);
        case 64: return fp16 ? launch_d<64, true>(sp, kind, stream) : launch_d<64, false>(sp, kind, stream);
        case 32: return fp16 ? launch_d<32, true>(sp, kind, stream) : launch_d<32, false>(sp, kind, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace ta

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
// Pipelined 256-row kernel (kind TA_LARGE256) on 32x32x16 MFMAs.
//
// Eight waves own 32 query rows each -- one N block of
// v_mfma_f32_32x32x16_{bf16,f16} -- and share every staged K/V tile.  Per
// 32-token step a wave runs D/16 QK MFMAs (S^T = K Q^T, tokens x rows), D/16
// PV MFMAs (O^T = V^T P^T, d x rows) and two 16x16x32 MFMAs for the softmax
// denominator.  A 32x32 MFMA occupies the matrix core twice as long as a
// 16x16 one and hides about three times the VALU work behind it (measured on
// gfx950: 24 cycles per 32x32 MFMA, 8 per 16x16), which is what the
// exponentials, conversions and maxima of a step need.
//
// The steps form one software pipeline across tile boundaries:
//
//   block(g):  QK of step g+1 (MFMA)   || exponentials and bf16/f16 packing
//                                         of step g, LDS reads of V(g)
//              PV + denominator of g   || LDS reads of K(g+2), masking, row
//                                         maxima and c*s - m of step g+1
//
// The shifted scores t = c*s - m are formed with the running maximum m
// before the lazy-rescale check of their step; when the check raises m (a
// wave-uniform branch, rare after the first step) t is moved by the change
// of m.  The order inside a block is pinned with sched_group_barrier.  K/V
// tiles arrive by LDS DMA into five stages: tiles t and t+1 are read while
// t+2 .. t+4 are in flight, with one barrier per tile.

// LDS layout of one 64-token tile for the 32-row kernel (16-bit elements):
// KBLK 1 KiB blocks of K, then VBLK of V, each a copy unit of 64 16-byte
// slots (one slot per lane of the copying wave).
//   K block b: d-rows 8b + j (j < 8); chunk c (tokens 8c .. 8c+7, c < 8) of
//     d-row 8b + j sits at slot 16u + 8((j >> 2) ^ (u & 1)) + 4(c & 1) +
//     (j & 3), u = c >> 1: a transposing read of 4 d-rows x 16 tokens is one
//     128-byte run, and runs of adjacent 16-token units lie in opposite
//     halves of 256 bytes.
//   V block vb: token rows VROWS vb + jr; a 128-byte unit holds 4 token rows
//     (row quad rq = jr >> 2) x 16 d (unit du = d >> 4) as slots 4 (s & 1) +
//     (jr & 3) for chunk s = d >> 3; unit (rq, du) sits at 128 bytes x
//     vunit(rq, du), whose low bit is (du ^ rq) & 1.
// The four 16-lane groups of a transposing read each take one 128-byte run;
// groups 0/1 and 2/3 land in opposite 128-byte halves of the 64 banks.
template <int D>
struct Tile32 {
    static constexpr int TT = 64;
    static constexpr int BLK = 512;
    static constexpr int KBLK = D / 8;
    static constexpr int VROWS = 512 / D;
    static constexpr int VBLK = TT / VROWS;
    static constexpr int NBLK = KBLK + VBLK;
    static constexpr int ELEMS = NBLK * BLK;
    static constexpr int NDU = D / 16;  // 16-d units of a V row
    static_assert(D % 32 == 0 && D <= 128, "d = 32, 64 or 128");

    __host__ __device__ static constexpr int vunit(int rq, int du) {
        return ((rq * NDU + du) & ~1) | ((du ^ rq) & 1);
    }
    // element offset, within the tile, of the 128-byte V run read by group
    // g's lanes for token rows tau .. tau+3 (tau % 4 == 0) and d unit du
    __host__ __device__ static constexpr int vrun(int tau, int du) {
        return BLK * (KBLK + tau / VROWS) + 64 * vunit((tau % VROWS) >> 2, du);
    }
    // V read of step base sb, 16-token sub-block sub, run r (tokens 8r ..)
    // and d tile dt, relative to the same read at (0, 0, 0, 0); the same for
    // every lane group
    __host__ __device__ static constexpr int vdelta(int sb, int sub, int r, int dt) {
        return vrun(sb + 16 * sub + 8 * r, 2 * dt) - vrun(0, 0);
    }
};

// Per-lane constants of one wave's tile copies and transposing reads.
struct Lane32 {
    int kdma;  // K copy: element offset j * tcap + 8c of this lane's slot
    int vdma;  // V copy: element offset jr * D + 8s of this lane's slot
    int kof0, kof1;  // K reads: element offsets of the two 4-d-row halves
    int vof;         // V reads: element offset at (sb, sub, r, dt) = 0
};

template <int D, bool FP16>
struct Pipe32 {
    static constexpr int DT = D / 32;  // 32-row d tiles of O^T
    static constexpr int KS = D / 16;  // 16-wide d slices of QK
    using T = Tile32<D>;

    f32x16 o[DT];
    f32x4 z;        // denominators: lane r < 16 holds row r (z[0]) and row r + 16 (z[1])
    float m, thr, lm;  // per lane (row lane % 32): running max (scaled), (m + TAU) / c, raw max of the next step
    f32x16 s;       // shifted scores c*s - m of the step whose exponentials come next
    u32x4 kf[KS];   // K fragments of the next QK step
    u32x4 vf[2 * DT];  // V^T fragments of the current PV step: [2 dt + sub]

    __device__ static f32x16 mma32(u32x4 a, u32x4 b, f32x16 c) {
        if constexpr (FP16)
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                          c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                           __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }

    __device__ static Lane32 lane_consts(int lane, int tcap) {
        Lane32 c;
        {  // K copy: slot lane <- chunk c of d-row j
            const int u = lane >> 4, h = ((lane >> 3) & 1) ^ (u & 1);
            const int ch = 2 * u + ((lane >> 2) & 1), j = 4 * h + (lane & 3);
            c.kdma = j * tcap + 8 * ch;
        }
        {  // V copy: slot lane <- chunk s of token row jr
            const int uidx = lane >> 3, sin = lane & 7;
            const int lin_hi = uidx & ~1, rq = lin_hi / T::NDU;
            const int du = ((lin_hi % T::NDU) & ~1) | ((uidx & 1) ^ (rq & 1));
            c.vdma = (4 * rq + (sin & 3)) * D + 8 * (2 * du + (sin >> 2));
        }
        const int g = lane >> 4, i = lane & 15;
        const int in = 32 * ((i >> 1) & 1) + 8 * (i >> 2) + 4 * (i & 1);  // within a 128-byte run
        c.kof0 = T::BLK * (g >> 1) + 128 * (g & 1) + 64 * (g & 1) + in;
        c.kof1 = T::BLK * (g >> 1) + 128 * (g & 1) + 64 * (1 - (g & 1)) + in;
        c.vof = T::vrun(4 * (g >> 1), g & 1) + in;
        return c;
    }

    // Copy the tile at pool token t0n into stage `st` (this wave's blocks of
    // NW waves).  Inside the job (tokens [t0n, t0n + TT) all in [kst, kend))
    // no index is clamped; at its edges chunks past the pool end read its
    // last chunk and V rows outside the job read a row inside it (finite
    // values; their scores are masked, P = 0).
    template <int NW>
    __device__ static void copy(u16 *st, const u16 *__restrict__ kp, const u16 *__restrict__ vp, int h, int tcap,
                                int t0n, int kst, int kend, int wave, int lane, const Lane32 &lc) {
        const int w = __builtin_amdgcn_readfirstlane(wave);
        if (t0n >= kst && t0n + T::TT <= kend)
            copy_blocks<NW, false>(st, kp, vp, h, tcap, t0n, kst, kend, w, lane, lc);
        else
            copy_blocks<NW, true>(st, kp, vp, h, tcap, t0n, kst, kend, w, lane, lc);
    }

    template <int NW, bool CLAMP>
    __device__ static void copy_blocks(u16 *st, const u16 *__restrict__ kp, const u16 *__restrict__ vp, int h,
                                       int tcap, int t0n, int kst, int kend, int w, int lane, const Lane32 &lc) {
        static_assert(T::NBLK % NW == 0, "every wave copies the same number of blocks");
#pragma unroll
        for (int i = 0; i < T::NBLK / NW; ++i) {
            const int blk = w + i * NW;
            const bool isk = T::KBLK % NW == 0 ? i * NW < T::KBLK : blk < T::KBLK;
            const u16 *src;
            if (isk) {
                const u16 *base = kp + (size_t)(h * D + 8 * blk) * tcap;
                if (CLAMP) {
                    const int u = lane >> 4, hh = ((lane >> 3) & 1) ^ (u & 1);
                    const int tok = t0n + 8 * (2 * u + ((lane >> 2) & 1));
                    src = base + (size_t)(4 * hh + (lane & 3)) * tcap + min(tok, tcap - 8);
                } else {
                    src = base + t0n + lc.kdma;
                }
            } else {
                const int t0 = t0n + T::VROWS * (blk - T::KBLK);
                if (CLAMP) {
                    const int jr = lc.vdma / D;
                    const int t = min(max(t0 + jr, kst), kend - 1);
                    src = vp + ((size_t)h * tcap + t) * D + (lc.vdma - jr * D);
                } else {
                    src = vp + ((size_t)h * tcap + t0) * D + lc.vdma;
                }
            }
            __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(st + blk * T::BLK), 16, 0, 0);
        }
    }

    __device__ void reset() {
        m = thr = lm = NEG_INF;
        z = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
    }

    // K fragments (A operand of QK) of the 32 tokens at step base sb (0 or
    // 32) of the tile in `st`: kf[ks] covers d = 16 ks .. +15.
    __device__ static void load_k(const u16 *__restrict__ st, const Lane32 &lc, int sb, u32x4 (&kf)[KS]) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int e = 2 * T::BLK * ks + 8 * sb;
            kf[ks] = tr_pair(st + lc.kof0 + e, st + lc.kof1 + e);
        }
    }

    // S^T = K Q^T of one step: lane l holds query row l % 32 and tokens
    // 8 (e >> 2) + 4 (l >> 5) + (e & 3) in element e.
    __device__ static f32x16 qk(const u32x4 (&kf)[KS], const u32x4 (&qf)[KS]) {
        f32x16 acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) acc = mma32(kf[ks], qf[ks], acc);
        return acc;
    }

    // Mask tokens outside [lo, hi) of the step (if MASK) and take the lane's
    // raw row maximum.
    template <bool MASK>
    __device__ void mask_max(f32x16 &sn, int lo, int hi, int hf) {
        if (MASK) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int tok = 8 * (e >> 2) + 4 * hf + (e & 3);
                if (tok < lo || tok >= hi) sn[e] = NEG_INF;
            }
        }
        float mx = sn[0];  // a chain, so that it becomes three-input maxima
#pragma unroll
        for (int e = 1; e < 16; ++e) mx = fmaxf(mx, sn[e]);
        lm = mx;
    }

    __device__ void shift(const f32x16 &sn, float c) {
#pragma unroll
        for (int e = 0; e < 16; ++e) s[e] = __builtin_fmaf(sn[e], c, -m);
    }

    __device__ void scale(float alpha) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
        z[0] *= alpha;
        z[1] *= __shfl_xor(alpha, 16);  // lanes r < 16: alpha of row r + 16
    }

    // Raise the running maxima where the staged step's raw maximum exceeds
    // them by more than TAU (wave-uniform).  SHIFTED: s already holds
    // c*s - m_old and is moved to c*s - m_new; otherwise the caller shifts.
    template <bool SHIFTED>
    __device__ void rescale(float c, float rc) {
        if (__builtin_amdgcn_ballot_w64(lm > thr)) {
            const float mn = fmaxf(m, fmaxf(lm, __shfl_xor(lm, 32)) * c);
            if (SHIFTED) {
                // m is finite here (the first step of an item is never shifted)
                const float dm = m - mn;
                scale(fast_exp2(dm));
#pragma unroll
                for (int e = 0; e < 16; ++e) s[e] += dm;
            } else {
                scale(mn == NEG_INF ? 1.f : fast_exp2(m - mn));
            }
            m = mn;
            thr = (mn + TAU) * rc;
        }
    }

    // One pipeline block (see above), written as slices of one MFMA each with
    // the work that goes out beside it; a scheduling barrier between slices
    // keeps that order (left free, the compiler issued the QK MFMAs back to
    // back and the exponentials after them).
    //   vsp / vsb: V(g) stage + this lane's V offset, and the step base;
    //   ksp0 / ksp1 / ksb: K(g+2) stage + this lane's two K offsets, step base
    //     (any resident step when there is none);
    //   lo / hi: valid tokens of step g+1;  ROWMASK: only this lane's row if keep.
    template <bool MORE, bool MASKN, bool ROWMASK = false>
    __device__ __forceinline__ void block(const u16 *__restrict__ vsp, int vsb, const u16 *__restrict__ ksp0,
                                          const u16 *__restrict__ ksp1, int ksb, const u32x4 (&qf)[KS],
                                          const u32x4 &zpat, int lo, int hi, int hf, float c, bool keep = true) {
        constexpr int NA = MORE ? KS : 1;  // slices of the QK half
        constexpr int NV = 2 * DT;         // V fragments, read in the first NAV slices
        constexpr int NAV = NA > 1 ? NA / 2 : 1;
        constexpr int NB = 2 * DT + 2;     // slices of the PV half
        constexpr int NBK = KS > 1 ? KS / 2 : 1;  // slices that read K(g+2)
        f32x16 sn;
        u32x4 pb[2];
        __builtin_amdgcn_sched_barrier(0);
        // ---- QK(g+1) || V(g) reads, exponentials and packing of step g
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            if (MORE) {
                if (i == 0) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) sn[e] = 0.f;
                }
                sn = mma32(kf[i], qf[i], sn);
            }
            constexpr int VPS = (NV + NAV - 1) / NAV, XPS = 16 / NA;  // V fragments, exponentials per slice
#pragma unroll
            for (int v2 = 0; v2 < VPS; ++v2) {
                const int v = i * VPS + v2;
                if (i < NAV && v < NV)
                    vf[v] = tr_pair(vsp + T::vdelta(vsb, v & 1, 0, v >> 1), vsp + T::vdelta(vsb, v & 1, 1, v >> 1));
            }
#pragma unroll
            for (int e2 = 0; e2 < XPS; e2 += 2) {
                const int e = i * XPS + e2;
                pb[e >> 3][(e & 7) >> 1] = Ops<FP16>::pack(fast_exp2(s[e]), fast_exp2(s[e + 1]));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (ROWMASK && !keep) pb[0] = pb[1] = u32x4{0u, 0u, 0u, 0u};
        // ---- PV(g) + denominator || K(g+2) reads, masking, maxima and c*s - m of step g+1
        constexpr int NE = MORE ? (16 + NB - 2) / (NB - 1) : 0;  // score elements per slice after the first
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if (j < 2 * DT)
                o[j >> 1] = mma32(vf[j], pb[j & 1], o[j >> 1]);  // d tile j/2, tokens 16 (j&1) ..
            else
                z = Ops<FP16>::mma_k32(zpat, pb[j - 2 * DT], z);
            if (MORE) {
                constexpr int KPS = (KS + NBK - 1) / NBK;  // K fragments per slice
#pragma unroll
                for (int k2 = 0; k2 < KPS; ++k2) {
                    const int k = j * KPS + k2;
                    if (j < NBK && k < KS) {
                        const int e = 2 * T::BLK * k + 8 * ksb;
                        kf[k] = tr_pair(ksp0 + e, ksp1 + e);
                    }
                }
                if (j == 1 && MASKN) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int tok = 8 * (e >> 2) + 4 * hf + (e & 3);
                        if (tok < lo || tok >= hi) sn[e] = NEG_INF;
                    }
                }
                if (j >= 1) {
#pragma unroll
                    for (int e2 = 0; e2 < NE; ++e2) {
                        const int e = (j - 1) * NE + e2;
                        if (e < 16) {
                            mx = e == 0 ? sn[0] : fmaxf(mx, sn[e & 15]);
                            s[e & 15] = __builtin_fmaf(sn[e & 15], c, -m);
                        }
                    }
                    // keeps this slice's maxima in the slice (instruction
                    // selection otherwise gathers the chain after the last MFMA)
                    if ((j - 1) * NE < 16) asm volatile("" : "+v"(mx));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (MORE) lm = ROWMASK && !keep ? NEG_INF : mx;
    }

    // One staged tile of an attached segment (after the pipeline has
    // drained): tokens [lo, hi) of the tile, for this lane's row only if
    // keep.  Rows not kept get P = 0 and keep their running maxima.  The
    // tile's two steps run as a two-step pipeline (the QK of the second step
    // beside the exponentials and PV of the first).
    __device__ void tail_tile(const u16 *__restrict__ st, const u32x4 (&qf)[KS], const Lane32 &lc,
                              const u32x4 &zpat, int lo, int hi, bool keep, int hf, float c, float rc) {
        load_k(st, lc, 0, kf);
        f32x16 sn = qk(kf, qf);
        mask_max<true>(sn, lo, hi, hf);
        if (!keep) lm = NEG_INF;
        rescale<false>(c, rc);
        shift(sn, c);
        if (hi > 32) {
            load_k(st, lc, 32, kf);
            // the K read-ahead of this block has no step to read: it rereads step 0
            block<true, true, true>(st + lc.vof, 0, st + lc.kof0, st + lc.kof1, 0, qf, zpat, lo - 32, hi - 32, hf, c,
                                    keep);
            rescale<true>(c, rc);
            block<false, false, true>(st + lc.vof, 32, st, st, 0, qf, zpat, 0, 32, hf, c, keep);
        } else {
            block<false, false, true>(st + lc.vof, 0, st, st, 0, qf, zpat, 0, 32, hf, c, keep);
        }
    }

    // Store the wave's 32 partial rows (rows row0 + r, r < 32, those below
    // nrows) through the wave's 8 KiB LDS region `stg`, so that every store
    // instruction writes whole 64-byte lines (straight from the registers a
    // row's 256 bytes sit in two lanes, and the nontemporal write path did
    // not combine the two halves of a line written by two instructions).
    // Same format as store_partial: (o / z) 2^-e in fp16 at part_pos order,
    // then (log-sum-exp, e).  In the region, 16-byte chunk c of row r sits at
    // chunk c ^ (r % (D / 8)): the 16 rows a write instruction touches hit
    // distinct banks without padding.
    __device__ void store(u16 *__restrict__ stg, u16 *__restrict__ part, float *__restrict__ lse2,
                          const int32_t *__restrict__ rowbase_job, int row0, int nrows, int hq, int hcol, int group,
                          int lane) {
        constexpr int CPR = D / 8;        // 16-byte chunks per row
        constexpr int RPI = 64 / CPR;     // rows per store instruction
        const int r = lane & 31, hf = lane >> 5;
        const float za = __shfl(z[0], lane & 15), zb = __shfl(z[1], lane & 15);
        const float zr = (lane & 16) ? zb : za;
        const bool any = m != NEG_INF;
        const float inv = any ? 1.f / zr : 0.f;
        float amax = 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int e = 0; e < 16; ++e) amax = fmaxf(amax, __builtin_fabsf(o[dt][e]));
        amax *= inv;
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        const int ex = amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) : 0;
        const float sc = __builtin_amdgcn_ldexpf(inv, -ex);
        // lane (r, hf) holds d = 32 dt + 8 q + 4 hf + i in o[dt][4 q + i]; at
        // part_pos order q = 0 and 2 fill chunk 4 dt + hf, q = 1 and 3 chunk
        // 4 dt + 2 + hf
        u16 *srow = stg + r * D;
        const int sw = r % CPR;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const f32x16 a = o[dt] * sc;
            const u32x4 w0 = {pack_f16(a[0], a[1]), pack_f16(a[2], a[3]), pack_f16(a[8], a[9]),
                              pack_f16(a[10], a[11])};
            const u32x4 w1 = {pack_f16(a[4], a[5]), pack_f16(a[6], a[7]), pack_f16(a[12], a[13]),
                              pack_f16(a[14], a[15])};
            *(u32x4 *)(srow + 8 * ((4 * dt + hf) ^ sw)) = w0;
            *(u32x4 *)(srow + 8 * ((4 * dt + 2 + hf) ^ sw)) = w1;
        }
        const float l = any ? (m + __builtin_amdgcn_logf(zr)) * LN2 : NEG_INF;
        const int grow = row0 + r;
        if (hf == 0 && grow < nrows) {
            const int lr = grow / group;
            const size_t prow = (size_t)(rowbase_job[0] + lr) * hq + hcol + (grow - lr * group);
            __builtin_nontemporal_store(f32x2{l, (float)ex}, (f32x2 *)(lse2 + 2 * prow));
        }
        // the wave reads back its own rows only
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
        const int ck = lane % CPR;
#pragma unroll
        for (int k = 0; k < 32 / RPI; ++k) {
            const int rr = RPI * k + lane / CPR;
            const u32x4 w = *(const u32x4 *)(stg + rr * D + 8 * (ck ^ (rr % CPR)));
            const int gr = row0 + rr;
            if (gr < nrows) {
                const int lr = gr / group;
                const size_t prow = (size_t)(rowbase_job[0] + lr) * hq + hcol + (gr - lr * group);
                __builtin_nontemporal_store(w, (u32x4 *)(part + prow * D + 8 * ck));
            }
        }
    }
};

#ifndef TA_PIPE_STAGES
#define TA_PIPE_STAGES 5
#endif
#ifndef TA_PIPE_PRO
#define TA_PIPE_PRO 3  // measured: 3 of 5 tiles in the prologue start the loop earliest
#endif
#ifndef TA_PIPE_SYNC
#define TA_PIPE_SYNC 1
#endif

// One 256-row work item of the pipelined kernel, with its attached segments
// (p.xtail, indexed by the item), STAGES LDS stages at `lds`.  STAGES LDS
// tiles; the waves meet at a barrier every SYNC tiles.  While the waves work
// on tiles t .. t+SYNC-1 they read those and the K of tile t+SYNC (the
// pipelined steps read one step ahead), so SYNC+1 tiles are resident and
// STAGES-SYNC-1 more can be in flight.  The prologue issues PRO tiles; the
// first loop barrier issues the rest of the ring.
template <int D, bool FP16, int NW, int STAGES = TA_PIPE_STAGES, int PRO = TA_PIPE_PRO, int SYNC = TA_PIPE_SYNC>
__device__ __forceinline__ void pipe_item(const SegParams &p, const int32_t *__restrict__ items, int item, u16 *lds,
                                          int tid) {
    using T = Tile32<D>;
    using M = Pipe32<D, FP16>;
    constexpr int KS = M::KS;
    constexpr int BPW = T::NBLK / NW;  // copies per wave per tile
    static_assert(NW == 8, "eight 32-row waves");
    static_assert(SYNC >= 1 && STAGES >= 2 * SYNC + 1 && STAGES <= 5,
                  "a group's tiles, the next K and the next group's copies fit the stages");
    static_assert(PRO >= SYNC + 1 && PRO <= STAGES, "the prologue issues the tiles the first group reads");
    const int job = items[3 * item], row0 = items[3 * item + 1], h = items[3 * item + 2];

    const int lane = tid & 63, wave = tid >> 6;
    const int hf = lane >> 5;
    const int kst = p.kstart[job];
    const int ntok = max(0, min(p.klen[job], p.tcap - kst));
    const int kend = kst + ntok;
    const int nrows = p.qlen[job] * p.group;
    const int wrow0 = row0 + 32 * wave;
    const bool active = wrow0 < nrows;
    const float c = p.scale_log2, rc = 1.f / p.scale_log2;
    const int tb0 = kst & ~7;
    const int ntiles = ntok > 0 ? (kend - tb0 + T::TT - 1) / T::TT : 0;
    const int nsteps = ntok > 0 ? (kend - tb0 + 31) / 32 : 0;
    auto tile_stage = [&](int t) { return lds + (t % STAGES) * T::ELEMS; };
    auto stage = [&](int g) { return tile_stage(g >> 1); };  // stage of step g's tile
    const Lane32 lc = M::lane_consts(lane, p.tcap);

    // Attached segments (xtail record of this item: count, then (first token,
    // tokens, first job row, rows) for up to TA_XTAIL_MAX segments) follow
    // the job's own tiles in one tile sequence through the same LDS stages.
    // The record is read at once (constant address space: one batch of scalar
    // loads, no chain of dependent loads) into per-segment values that
    // unrolled loops index with constants.
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
            M::template copy<NW>(st, p.kp, p.vp, h, p.tcap, tb0 + t * T::TT, kst, kend, wave, lane, lc);
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
        M::template copy<NW>(st, p.kp, p.vp, h, p.tcap, t0n, cs, ce, wave, lane, lc);
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
    const int rr = max(0, min(wrow0 + (lane & 31), nrows - 1));  // this lane's (clamped) query row
    if (qb < 0 && ntot > 0) copy_tile(0, lds);
    const int rq = qb >= 0 ? qb + rr / p.group : p.qids[(size_t)job * p.maxr + rr / p.group];
    // Q^T fragments (B operand): lane l holds row l % 32, d = 16 ks + 8 (l >> 5) .. +7
    u32x4 qf[KS];
    {
        const u16 *src = p.q + ((size_t)rq * p.hq + h * p.group + rr % p.group) * D + 8 * hf;
#pragma unroll
        for (int k = 0; k < KS; ++k) qf[k] = *(const u32x4 *)(src + 16 * k);
    }
#ifdef TA_PIPE_QFIRST
    __builtin_amdgcn_s_waitcnt(TA_VMCNT(0));
#endif
    if (qb >= 0 && ntot > 0) copy_tile(0, lds);  // behind the Q loads: one wait covers both
    {
        const bool valid = wrow0 + (lane & 31) < nrows;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            if (!valid) qf[k] = u32x4{0, 0, 0, 0};
            asm volatile("" : "+v"(qf[k]));
        }
    }
    for (int t = 1; t < PRO && t < ntot; ++t) copy_tile(t, tile_stage(t));
    issued = min(PRO, ntot);

    // denominator MFMA operand: lane l of the 16x16x32 A operand is row
    // l % 16, k block l / 16; rows 0 and 1 sum the k blocks of 32-row P rows
    // 0-15 and 16-31
    u32x4 zpat;
    {
        const int zr = lane & 15, kb = (lane >> 4) & 1;
        const u32 one = (zr == 0 && kb == 0) || (zr == 1 && kb == 1) ? Ops<FP16>::ONE2 : 0u;
        zpat = u32x4{one, one, one, one};
    }

    M acc;
    acc.reset();

    wait_tiles<BPW>(issued - 1);  // tile 0 landed (tiles 1 .. PRO-1 may be in flight)
    __builtin_amdgcn_s_barrier();
    if (active && nsteps > 0) {
        M::load_k(lds, lc, 0, acc.kf);
        f32x16 s0 = M::qk(acc.kf, qf);
        acc.template mask_max<true>(s0, kst - tb0, kend - tb0, hf);
        acc.template rescale<false>(c, rc);
        acc.shift(s0, c);
        if (nsteps > 1) M::load_k(lds, lc, 32, acc.kf);
    }

    // Entering tile t (at step 2t): at the start of a group (t % SYNC == 0)
    // tiles t+1 .. t+SYNC must have landed (the earlier ones were waited for
    // at the previous group); the later issued ones may still be in flight.
    // Once every wave passed the barrier the stages of the previous group
    // are free for tiles up to t+STAGES-1.
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
            acc.template block<true, false>(stage(g) + lc.vof, 32 * (g & 1), stage(gk) + lc.kof0,
                                            stage(gk) + lc.kof1, 32 * (gk & 1), qf, zpat, 0, 32, hf, c);
            acc.template rescale<true>(c, rc);
        }
    }
    // the last two steps: the successor of step nsteps-2 may be masked at its end
    if (g + 1 < nsteps) {
        if (!(g & 1)) sync_tile(g >> 1);
        if (active) {  // one (masked) form for either end of the job keeps the register allocation simple
            acc.template block<true, true>(stage(g) + lc.vof, 32 * (g & 1), stage(g + 1) + lc.kof0,
                                           stage(g + 1) + lc.kof1, 32 * ((g + 1) & 1), qf, zpat, 0,
                                           kend - (tb0 + 32 * (g + 1)), hf, c);
            acc.template rescale<true>(c, rc);
        }
        ++g;
    }
    if (g < nsteps) {
        if (!(g & 1)) sync_tile(g >> 1);
        if (active)
            acc.template block<false, false>(stage(g) + lc.vof, 32 * (g & 1), stage(g), stage(g), 0, qf, zpat, 0, 32,
                                             hf, c);
    }

    // Attached segments, in rounds of up to STAGES tiles that are resident
    // together: one wait and one barrier per round, then every wave attends
    // the round's tiles of the segments holding its rows, side by side.  The
    // root loop (or the prologue) already issued the first tiles.
    for (int r0 = ntiles; r0 < ntot; r0 += STAGES) {
        const int r1 = min(r0 + STAGES, ntot);
        __builtin_amdgcn_s_barrier();  // every wave is done with the tiles before r0
        for (; issued < r1; ++issued) copy_tile(issued, tile_stage(issued));
        __builtin_amdgcn_s_waitcnt(TA_VMCNT(0));
        __builtin_amdgcn_s_barrier();  // the round's tiles landed
#pragma unroll
        for (int k = 0; k < XM; ++k) {
            const int rlo = rec[3 + XF * k] - wrow0;  // segment rows in this wave: [rlo, rlo + rows)
            if (xn[k] > 0 && active && rlo >= 0 && rlo < 32) {
                const int lr = lane & 31;
                const bool keep = lr >= rlo && lr < rlo + rec[4 + XF * k];
                for (int i = max(0, r0 - xfirst[k]); i < xn[k] && xfirst[k] + i < r1; ++i) {
                    const int t0 = (xs[k] & ~7) + i * T::TT;
                    acc.tail_tile(tile_stage(xfirst[k] + i), qf, lc, zpat, max(0, xs[k] - t0),
                                  min(T::TT, xe[k] - t0), keep, hf, c, rc);
                }
            }
        }
    }

    // Partial rows through LDS.  When the item's attached tiles fit one
    // round with a stage to spare (the stage of its last own tile, which
    // every wave finished before the round) and at most four waves hold no
    // attached rows, those waves stage their rows there (8 KiB each) and the
    // waves with attached rows in the stage of their own last attached tile
    // (no other wave reads it), so no wave waits for another.  Otherwise the
    // waves meet at a barrier and stage at wave * 8 KiB.
    const int nxt = ntot - ntiles;
    int owners = 0;  // waves that hold rows of an attached segment
#pragma unroll
    for (int k = 0; k < XM; ++k) {
        const int ow = (rec[3 + XF * k] - row0) >> 5;
        if (xn[k] > 0 && ow >= 0 && ow < 8) owners |= 1 << ow;
    }
    const int free_waves = 8 - __builtin_popcount(owners);
    const bool spare = ntiles > 0 && nxt > 0 && nxt < STAGES && free_waves <= 4;
    u16 *stg;
    if (spare) {
        if ((owners >> wave) & 1) {
            int last = 0;  // this wave's last attached tile
#pragma unroll
            for (int k = 0; k < XM; ++k)
                if (xn[k] > 0 && ((rec[3 + XF * k] - row0) >> 5) == wave) last = max(last, xfirst[k] + xn[k] - 1);
            stg = tile_stage(last);
        } else {
            const int rank = __builtin_popcount(~owners & ((1 << wave) - 1));  // free waves before this one
            stg = tile_stage(ntiles - 1) + rank * 32 * D;
        }
    } else {
        __builtin_amdgcn_s_barrier();
        stg = lds + wave * 32 * D;
    }
    if (!active) return;
    acc.store(stg, p.part, p.lse, p.rowbase + job, wrow0, nrows, p.hq, h * p.group, p.group, lane);
}

template <int D, bool FP16, int NW>
__global__ __launch_bounds__(64 * NW) void seg_pipe_kernel(SegParams p) {
    __shared__ __attribute__((aligned(16))) u16 lds[TA_PIPE_STAGES * Tile32<D>::ELEMS];
    static_assert(8 * 32 * D <= TA_PIPE_STAGES * Tile32<D>::ELEMS && 4 * 32 * D <= Tile32<D>::ELEMS,
                  "the partial rows fit the stages, four waves' rows one stage");
    pipe_item<D, FP16, NW>(p, p.items, xcd_item(blockIdx.x, gridDim.x), lds, threadIdx.x);
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
        pipe_item<D, FP16, 8>(mp.p, mp.items[0], xcd_item(b, mp.n[0]), lds, tid);
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

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
//   * The merge reads fp32 partials with 16-byte loads, one thread per four
//     head-dim elements.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tree_attn.h"

namespace {

using u16 = unsigned short;
using u32 = unsigned int;
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int TT = 64;          // tokens per staged tile
constexpr int NT = 256;         // threads per workgroup (4 waves)
constexpr float LN2 = 0.69314718055994530942f;
constexpr float NEG_INF = -__builtin_inff();

// ---------------------------------------------------------------- dtype ops
template <bool FP16>
struct Ops;

template <>
struct Ops<false> {  // bfloat16
    __device__ static f32x4 mma_k32(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
    __device__ static f32x4 mma_k16(u32x2 a, u32x2 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                         __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
    }
    __device__ static u32 pack(float lo, float hi) {
        bf16x2 v = {(__bf16)lo, (__bf16)hi};
        return __builtin_bit_cast(u32, v);
    }
};

template <>
struct Ops<true> {  // float16
    __device__ static f32x4 mma_k32(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
    __device__ static f32x4 mma_k16(u32x2 a, u32x2 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                     __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
    }
    __device__ static u32 pack(float lo, float hi) {
        f16x2 v = {(_Float16)lo, (_Float16)hi};
        return __builtin_bit_cast(u32, v);
    }
};

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline float xor_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}

__device__ inline float xor_sum(float v) {
    v += __shfl_xor(v, 16);
    return v + __shfl_xor(v, 32);
}

// Kernel arguments shared by both segment kernels.
struct SegParams {
    const u16 *q, *kp, *vp;
    const int32_t *qids, *kstart, *qlen, *klen, *rowbase, *items;
    float *part, *lse;
    int n_items, hq, hk, group, tcap, maxr;
    float scale_log2;  // log2(e) / sqrt(D)
};

// ------------------------------------------------------- tile staging (LDS)
// One 64-token tile of one KV head: Kt[TT][D] (+pad) and Vt[D][TT] (+pad).
template <int D>
struct Stage {
    static constexpr int KS = D + 8;   // Kt row stride (elements); +16 B breaks bank aliasing
    static constexpr int VS = TT + 8;  // Vt row stride
    static constexpr int KELEMS = TT * KS;
    static constexpr int ELEMS = KELEMS + D * VS;
    static constexpr int DG = D / 8;
    static constexpr int TG = TT / 8;
    static constexpr int KBLK = DG * TG;  // 8x8 blocks per operand
    static constexpr int VBLK = TG * DG;

    u32x4 r[8];

    __device__ static u32x4 load_tail(const u16 *p, int valid) {
        u32 w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            u32 lo = (2 * k < valid) ? (u32)p[2 * k] : 0u;
            u32 hi = (2 * k + 1 < valid) ? (u32)p[2 * k + 1] : 0u;
            w[k] = lo | (hi << 16);
        }
        return u32x4{w[0], w[1], w[2], w[3]};
    }

    // Global -> registers.  Tokens [t0, t0 + nvalid) are read; the rest of the
    // tile is zero (zero V keeps masked columns finite in PV).
    __device__ void load(const u16 *__restrict__ kp, const u16 *__restrict__ vp, int h, int tcap,
                         int t0, int nvalid, bool kaligned, int tid) {
        if (tid < KBLK) {
            const int dg = tid % DG, tg = tid / DG;
            const u16 *base = kp + ((size_t)(h * D + 8 * dg) * tcap + t0 + 8 * tg);
            const int valid = nvalid - 8 * tg;
            if (kaligned && valid >= 8) {
#pragma unroll
                for (int i = 0; i < 8; ++i) r[i] = *(const u32x4 *)(base + (size_t)i * tcap);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) r[i] = load_tail(base + (size_t)i * tcap, valid);
            }
        } else if (tid < KBLK + VBLK) {
            const int u = tid - KBLK;
            const int tg = u % TG, dg = u / TG;
            const u16 *base = vp + ((size_t)(h * tcap + t0 + 8 * tg) * D + 8 * dg);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                r[i] = (8 * tg + i < nvalid) ? *(const u32x4 *)(base + (size_t)i * D) : u32x4{0, 0, 0, 0};
        }
    }

    // 8x8 transpose of 16-bit elements: out[j] = column j of the rows in r.
    __device__ void transpose(u32x4 (&o)[8]) const {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            u32 w[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const u32 a = r[2 * k][j >> 1], b = r[2 * k + 1][j >> 1];
                w[k] = (j & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
            }
            o[j] = u32x4{w[0], w[1], w[2], w[3]};
        }
    }

    // Registers -> LDS in MFMA operand order.
    __device__ void store(u16 *lds, int tid) const {
        if (tid >= KBLK + VBLK) return;
        u32x4 o[8];
        transpose(o);
        if (tid < KBLK) {
            const int dg = tid % DG, tg = tid / DG;
#pragma unroll
            for (int j = 0; j < 8; ++j) *(u32x4 *)(lds + (8 * tg + j) * KS + 8 * dg) = o[j];
        } else {
            const int u = tid - KBLK;
            const int tg = u % TG, dg = u / TG;
#pragma unroll
            for (int j = 0; j < 8; ++j) *(u32x4 *)(lds + KELEMS + (8 * dg + j) * VS + 8 * tg) = o[j];
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

// --------------------------------------------------------- small segments
// One workgroup per (job, KV head) with at most 16 query rows.
template <int D, bool FP16>
__global__ __launch_bounds__(NT) void seg_small_kernel(SegParams p) {
    using S = Stage<D>;
    using O = Ops<FP16>;
    __shared__ __attribute__((aligned(16))) u16 lds[S::ELEMS];

    const int job = p.items[blockIdx.x];
    const int h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = lane & 15, g4 = lane >> 4;
    const int kst = p.kstart[job];
    const int ntok = max(0, min(p.klen[job], p.tcap - kst));
    const int nrows = min(p.qlen[job] * p.group, 16);
    const bool kal = ((p.tcap | kst) & 7) == 0;
    const float c = p.scale_log2;

    u32x4 qf[D / 32];
    load_q<D>(p, job, h, row, nrows, g4, qf);

    float m = NEG_INF, z = 0.f;
    f32x4 o[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int ntiles = (ntok + TT - 1) / TT;
    S st;
    if (ntiles > 0) st.load(p.kp, p.vp, h, p.tcap, kst, min(ntok, TT), kal, tid);
    const int base = 16 * wave;
    for (int it = 0; it < ntiles; ++it) {
        __syncthreads();
        st.store(lds, tid);
        __syncthreads();
        const int t0 = it * TT;
        const int nv = ntok - t0;
        if (it + 1 < ntiles) st.load(p.kp, p.vp, h, p.tcap, kst + t0 + TT, min(nv - TT, TT), kal, tid);
        if (base < nv) {
            f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                const u32x4 a = *(const u32x4 *)(lds + (base + row) * S::KS + 32 * ks + 8 * g4);
                s = O::mma_k32(a, qf[ks], s);
            }
            // s[i] <-> token base + 4*g4 + i of query row `row`
            float sv[4];
            float mx = NEG_INF;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sv[i] = (base + 4 * g4 + i < nv) ? s[i] : NEG_INF;
                mx = fmaxf(mx, sv[i]);
            }
            mx = xor_max(mx);
            const float mn = fmaxf(m, mx * c);
            const float alpha = fast_exp2(m - mn);
            float pr[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) pr[i] = fast_exp2(sv[i] * c - mn);
            z = z * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
            m = mn;
            const u32x2 pb = {O::pack(pr[0], pr[1]), O::pack(pr[2], pr[3])};
#pragma unroll
            for (int db = 0; db < D / 16; ++db) {
                const u32x2 a = *(const u32x2 *)(lds + S::KELEMS + (16 * db + row) * S::VS + base + 4 * g4);
                o[db] = O::mma_k16(a, pb, o[db] * alpha);
            }
        }
    }

    // Combine the four waves' (m, z, O) through LDS.
    const float zr = xor_sum(z);
    __syncthreads();
    float *red = reinterpret_cast<float *>(lds);  // [4 waves][16 rows][D]
    float *mz = red + 4 * 16 * D;                 // [2][4 waves][16 rows]
    static_assert(sizeof(u16) * S::ELEMS >= sizeof(float) * (4 * 16 * D + 128), "LDS reuse");
    if (g4 == 0) {
        mz[wave * 16 + row] = m;
        mz[64 + wave * 16 + row] = zr;
    }
#pragma unroll
    for (int db = 0; db < D / 16; ++db) *(f32x4 *)(red + (wave * 16 + row) * D + 16 * db + 4 * g4) = o[db];
    __syncthreads();
    const int rb = p.rowbase[job];
    for (int cidx = tid; cidx < 16 * (D / 4); cidx += NT) {
        const int r = cidx / (D / 4), d4 = cidx - r * (D / 4);
        if (r >= nrows) continue;
        const int lr = r / p.group, gg = r - lr * p.group;
        const size_t prow = (size_t)(rb + lr) * p.hq + h * p.group + gg;
        float M = NEG_INF;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, mz[w * 16 + r]);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        float Z = 0.f;
        if (M != NEG_INF) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float sc = fast_exp2(mz[w * 16 + r] - M);
                Z += mz[64 + w * 16 + r] * sc;
                acc += sc * *(const f32x4 *)(red + (w * 16 + r) * D + 4 * d4);
            }
            acc *= 1.f / Z;
        }
        *(f32x4 *)(p.part + prow * D + 4 * d4) = acc;
        if (d4 == 0) p.lse[prow] = (M != NEG_INF) ? (M + __builtin_amdgcn_logf(Z)) * LN2 : NEG_INF;
    }
}

// --------------------------------------------------------- large segments
// One workgroup per (job, row tile of 64*NB rows, KV head); wave w owns rows
// [16*NB*w, 16*NB*(w+1)) of the tile.
template <int D, bool FP16, int NB>
__global__ __launch_bounds__(NT) void seg_large_kernel(SegParams p) {
    using S = Stage<D>;
    using O = Ops<FP16>;
    __shared__ __attribute__((aligned(16))) u16 lds[S::ELEMS];

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

    float m[NB], z[NB];
    f32x4 o[NB][D / 16];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        m[nb] = NEG_INF;
        z[nb] = 0.f;
#pragma unroll
        for (int db = 0; db < D / 16; ++db) o[nb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const int ntiles = (ntok + TT - 1) / TT;
    S st;
    if (ntiles > 0) st.load(p.kp, p.vp, h, p.tcap, kst, min(ntok, TT), kal, tid);
    for (int it = 0; it < ntiles; ++it) {
        __syncthreads();
        st.store(lds, tid);
        __syncthreads();
        const int t0 = it * TT;
        const int nv = ntok - t0;
        if (it + 1 < ntiles) st.load(p.kp, p.vp, h, p.tcap, kst + t0 + TT, min(nv - TT, TT), kal, tid);
        if (!active) continue;
#pragma unroll
        for (int hh = 0; hh < TT / 32; ++hh) {
            const int base = 32 * hh;
            if (base >= nv) break;
            f32x4 s[NB][2];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) s[nb][0] = s[nb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
                for (int ks = 0; ks < D / 32; ++ks) {
                    const u32x4 a = *(const u32x4 *)(lds + (base + 16 * b + row) * S::KS + 32 * ks + 8 * g4);
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb) s[nb][b] = O::mma_k32(a, qf[nb][ks], s[nb][b]);
                }
            }
            // V^T fragments; k-slot j <-> token base + 4*g4 + j (j < 4), base + 16 + 4*g4 + j - 4 (j >= 4)
            u32x4 vf[D / 16];
#pragma unroll
            for (int db = 0; db < D / 16; ++db) {
                const u16 *vr = lds + S::KELEMS + (16 * db + row) * S::VS + base + 4 * g4;
                const u32x2 lo = *(const u32x2 *)vr;
                const u32x2 hi = *(const u32x2 *)(vr + 16);
                vf[db] = u32x4{lo[0], lo[1], hi[0], hi[1]};
            }
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                float sv[8];
                float mx = NEG_INF;
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float x = (base + 16 * b + 4 * g4 + i < nv) ? s[nb][b][i] : NEG_INF;
                        sv[4 * b + i] = x;
                        mx = fmaxf(mx, x);
                    }
                mx = xor_max(mx);
                const float mn = fmaxf(m[nb], mx * c);
                const float alpha = fast_exp2(m[nb] - mn);
                float pr[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) pr[i] = fast_exp2(sv[i] * c - mn);
                z[nb] = z[nb] * alpha + (((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7])));
                m[nb] = mn;
                const u32x4 pb = {O::pack(pr[0], pr[1]), O::pack(pr[2], pr[3]), O::pack(pr[4], pr[5]),
                                  O::pack(pr[6], pr[7])};
#pragma unroll
                for (int db = 0; db < D / 16; ++db) o[nb][db] = O::mma_k32(vf[db], pb, o[nb][db] * alpha);
            }
        }
    }

    if (!active) return;
    const int rb = p.rowbase[job];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const float zr = xor_sum(z[nb]);
        const int grow = wrow0 + 16 * nb + row;
        if (grow >= nrows) continue;
        const int lr = grow / p.group, gg = grow - lr * p.group;
        const size_t prow = (size_t)(rb + lr) * p.hq + h * p.group + gg;
        float *dst = p.part + prow * D + 4 * g4;
        const bool any = m[nb] != NEG_INF;
        const float inv = any ? 1.f / zr : 0.f;
#pragma unroll
        for (int db = 0; db < D / 16; ++db) *(f32x4 *)(dst + 16 * db) = o[nb][db] * inv;
        if (g4 == 0) p.lse[prow] = any ? (m[nb] + __builtin_amdgcn_logf(zr)) * LN2 : NEG_INF;
    }
}

// ------------------------------------------------------------------ merge
// One thread per (request, query head, 4 head-dim elements).
template <int D, bool FP16>
__global__ __launch_bounds__(NT) void merge_kernel(const float *__restrict__ part, const float *__restrict__ lse,
                                                   const int32_t *__restrict__ slots,
                                                   const int32_t *__restrict__ counts, u16 *__restrict__ out,
                                                   int hq, int maxs) {
    constexpr int TPH = D / 4;  // threads per head
    constexpr int HPB = NT / TPH;
    const int r = blockIdx.x;
    const int head = blockIdx.y * HPB + threadIdx.x / TPH;
    const int d4 = threadIdx.x % TPH;
    if (head >= hq) return;
    const int cnt = counts[r];
    const int32_t *sl = slots + (size_t)r * maxs;
    float M = NEG_INF;
    for (int s = 0; s < cnt; ++s) M = fmaxf(M, lse[(size_t)sl[s] * hq + head]);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (M != NEG_INF) {
        float Z = 0.f;
        for (int s = 0; s < cnt; ++s) {
            const size_t prow = (size_t)sl[s] * hq + head;
            const float w = fast_exp2((lse[prow] - M) * 1.44269504088896341f);
            Z += w;
            acc += w * *(const f32x4 *)(part + prow * D + 4 * d4);
        }
        acc *= 1.f / Z;
    }
    u16 *dst = out + ((size_t)r * hq + head) * D + 4 * d4;
    const u32x2 packed = {Ops<FP16>::pack(acc[0], acc[1]), Ops<FP16>::pack(acc[2], acc[3])};
    *(u32x2 *)dst = packed;
}

// ------------------------------------------------------------------ launch
template <int D, bool FP16>
hipError_t launch_segment(const SegParams &sp, int kind, hipStream_t stream) {
    if (sp.n_items <= 0) return hipSuccess;
    switch (kind) {
        case TA_SMALL:
            hipLaunchKernelGGL((seg_small_kernel<D, FP16>), dim3(sp.n_items, sp.hk), dim3(NT), 0, stream, sp);
            break;
        case TA_LARGE64:
            hipLaunchKernelGGL((seg_large_kernel<D, FP16, 1>), dim3(sp.n_items), dim3(NT), 0, stream, sp);
            break;
        case TA_LARGE128:
            hipLaunchKernelGGL((seg_large_kernel<D, FP16, 2>), dim3(sp.n_items), dim3(NT), 0, stream, sp);
            break;
        case TA_LARGE256:
            hipLaunchKernelGGL((seg_large_kernel<D, FP16, 4>), dim3(sp.n_items), dim3(NT), 0, stream, sp);
            break;
        default:
            return (hipError_t)TA_ERR_ARG;
    }
    return hipGetLastError();
}

template <int D, bool FP16>
hipError_t launch_merge(const float *part, const float *lse, const int32_t *slots, const int32_t *counts,
                        void *out, int nreq, int hq, int maxs, hipStream_t stream) {
    constexpr int HPB = NT / (D / 4);
    hipLaunchKernelGGL((merge_kernel<D, FP16>), dim3(nreq, (hq + HPB - 1) / HPB), dim3(NT), 0, stream, part,
                       lse, slots, counts, static_cast<u16 *>(out), hq, maxs);
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

extern "C" {

const char *ta_version(void) { return "tree_attn gfx950 1.0"; }

const char *ta_error_string(int code) {
    switch (code) {
        case 0: return "success";
        case TA_ERR_ARG: return "tree_attn: invalid argument (null pointer, size or unsupported shape)";
        case TA_ERR_ALIGN: return "tree_attn: q/kp/vp/part/out must be 16-byte aligned";
        case TA_ERR_DTYPE: return "tree_attn: dtype must be TA_BF16 or TA_FP16";
        default: return hipGetErrorString((hipError_t)code);
    }
}

int ta_segment(const void *q, const void *kp, const void *vp, const int32_t *qids, const int32_t *kstart,
               const int32_t *qlen, const int32_t *klen, const int32_t *rowbase, const int32_t *items,
               int32_t n_items, int32_t kind, float *part, float *lse, int32_t nreq, int32_t hq, int32_t hk,
               int32_t d, int32_t tcap, int32_t maxr, int32_t dtype, void *stream) {
    if (int e = check_common(hq, hk, d, dtype)) return e;
    if (n_items < 0 || nreq <= 0 || tcap <= 0 || maxr <= 0 || kind < TA_SMALL || kind > TA_LARGE256)
        return TA_ERR_ARG;
    if (n_items == 0) return 0;
    if (!q || !kp || !vp || !qids || !kstart || !qlen || !klen || !rowbase || !items || !part || !lse)
        return TA_ERR_ARG;
    if (!aligned16(q) || !aligned16(kp) || !aligned16(vp) || !aligned16(part)) return TA_ERR_ALIGN;
    SegParams sp;
    sp.q = static_cast<const u16 *>(q);
    sp.kp = static_cast<const u16 *>(kp);
    sp.vp = static_cast<const u16 *>(vp);
    sp.qids = qids;
    sp.kstart = kstart;
    sp.qlen = qlen;
    sp.klen = klen;
    sp.rowbase = rowbase;
    sp.items = items;
    sp.part = part;
    sp.lse = lse;
    sp.n_items = n_items;
    sp.hq = hq;
    sp.hk = hk;
    sp.group = hq / hk;
    sp.tcap = tcap;
    sp.maxr = maxr;
    sp.scale_log2 = (float)(1.4426950408889634 / __builtin_sqrt((double)d));
    const hipStream_t st = static_cast<hipStream_t>(stream);
#define TA_SEG(D, F) launch_segment<D, F>(sp, kind, st)
    return (int)TA_DISPATCH(d, dtype == TA_FP16, TA_SEG);
#undef TA_SEG
}

int ta_merge(const float *part, const float *lse, const int32_t *slots, const int32_t *counts, void *out,
             int32_t nreq, int32_t hq, int32_t d, int32_t maxs, int32_t dtype, void *stream) {
    if (dtype != TA_BF16 && dtype != TA_FP16) return TA_ERR_DTYPE;
    if (nreq <= 0 || hq <= 0 || maxs <= 0 || (d != 32 && d != 64 && d != 128)) return TA_ERR_ARG;
    if (!part || !lse || !slots || !counts || !out) return TA_ERR_ARG;
    if (!aligned16(part) || !aligned16(out)) return TA_ERR_ALIGN;
    const hipStream_t st = static_cast<hipStream_t>(stream);
#define TA_MRG(D, F) launch_merge<D, F>(part, lse, slots, counts, out, nreq, hq, maxs, st)
    return (int)TA_DISPATCH(d, dtype == TA_FP16, TA_MRG);
#undef TA_MRG
}

int ta_attention_matrix(const void *q, const void *kp, const void *vp, int32_t tcap, const ta_plan *plan,
                        void *out, void *stream) {
    if (!plan) return TA_ERR_ARG;
    for (int kind = TA_SMALL; kind <= TA_LARGE256; ++kind) {
        const int n = plan->n_items[kind];
        if (n == 0) continue;
        const int e = ta_segment(q, kp, vp, plan->qids, plan->kstart, plan->qlen, plan->klen, plan->rowbase,
                                 plan->items[kind], n, kind, plan->part, plan->lse, plan->nreq, plan->hq,
                                 plan->hk, plan->d, tcap, plan->maxr, plan->dtype, stream);
        if (e) return e;
    }
    return ta_merge(plan->part, plan->lse, plan->slots, plan->counts, out, plan->nreq, plan->hq, plan->d,
                    plan->maxs, plan->dtype, stream);
}

}  // extern "C"

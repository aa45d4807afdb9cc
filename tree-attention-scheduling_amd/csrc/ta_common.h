// ta_common.h -- device helpers and launch arguments shared by the gfx950
// segment kernels of libtree_attn.so (internal; not part of the C ABI).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tree_attn.h"

namespace ta {

using u16 = unsigned short;
using u32 = unsigned int;
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr float LN2 = 0.69314718055994530942f;
constexpr float NEG_INF = -__builtin_inff();

// Lazy rescaling threshold in log2 units: a row's running maximum is only
// raised when a score exceeds it by more than TAU, so exponentials stay
// <= 2^TAU and the accumulator rescale (a pass over all of O) is skipped on
// almost every step.  The final log-sum-exp is exact for any stale maximum.
constexpr float TAU = 8.0f;

// MFMA and packing for one 16-bit input type.
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
    static constexpr u32 ONE2 = 0x3F803F80u;  // two 1.0 values
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
    static constexpr u32 ONE2 = 0x3C003C00u;
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

// Partial outputs.  Row `prow` (= slot * hq + query head) of a segment's
// partial output is stored as D fp16 values of (o / z) * 2^-e, where e is the
// frexp exponent of the row's largest |o / z| (every stored value lies in
// (-1, 1), whatever the range of V), next to lse2[2 prow] = natural-log
// log-sum-exp of the row and lse2[2 prow + 1] = e.  Lane (row, g4) of a
// 16-row MFMA block holds d = 16 db + 4 g4 + i in o[db][i]; the four lanes of
// a row (g4 = 0..3, lanes 16 apart) must all be active.
//
// Within a row the values are stored in the lanes' order: head-dim element
// d = 32 P + 16 h + 4 g + i (i < 4) sits at position 32 P + 8 g + 4 h + i, so
// that a lane writes d blocks 2P and 2P+1 as one 16-byte store and the four
// lanes of a row fill whole 64-byte lines.  part_pos gives the position of
// the four-element chunk starting at d = 4 c.
__device__ constexpr int part_pos(int c) { return 32 * (c >> 3) + 8 * (c & 3) + 4 * ((c >> 2) & 1); }
__device__ inline u32 pack_f16(float lo, float hi) {
    f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(u32, v);
}

// The stores carry the nontemporal hint: the partial lines leave L2 while the
// kernel runs instead of waiting there, dirty, for the end-of-kernel writeback,
// and the merge reads each of them once.
template <int DB>
__device__ inline void store_partial(u16 *part, float *lse2, size_t prow, const f32x4 (&o)[DB], float m, float z,
                                     int g4) {
    constexpr int D = 16 * DB;
    const bool any = m != NEG_INF;
    const float inv = any ? 1.f / z : 0.f;
    float amax = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) amax = fmaxf(amax, __builtin_fabsf(o[db][i]));
    amax *= inv;
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const int e = amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) : 0;
    const float s = __builtin_amdgcn_ldexpf(inv, -e);
    static_assert(DB % 2 == 0, "d blocks are stored in pairs");
    u16 *dst = part + prow * D + 8 * g4;
    u32x4 w[DB / 2];
#pragma unroll
    for (int pr = 0; pr < DB / 2; ++pr) {
        const f32x4 a = o[2 * pr] * s, b = o[2 * pr + 1] * s;
        w[pr] = u32x4{pack_f16(a[0], a[1]), pack_f16(a[2], a[3]), pack_f16(b[0], b[1]), pack_f16(b[2], b[3])};
    }
    const float l = any ? (m + __builtin_amdgcn_logf(z)) * LN2 : NEG_INF;
    // The empty asm statements keep the stores together, after every
    // conversion: left free, the compiler spread them among the conversions
    // and the headline layer ran 6 % longer.
    asm volatile("" ::: "memory");
#pragma unroll
    for (int pr = 0; pr < DB / 2; ++pr) __builtin_nontemporal_store(w[pr], (u32x4 *)(dst + 32 * pr));
    if (g4 == 0) {
        __builtin_nontemporal_store(l, lse2 + 2 * prow);
        __builtin_nontemporal_store((float)e, lse2 + 2 * prow + 1);
    }
    asm volatile("" ::: "memory");
}

// Four fp16 partial values (8 bytes) -> floats.  The whole vector is
// bit-cast: hipcc (ROCm 7.2) lowers a bit_cast of one element of an
// ext_vector (w[1]) as if it were element 0.
__device__ inline f32x4 unpack_f16x4(u32x2 w) {
    const f16x4 h = __builtin_bit_cast(f16x4, w);
    return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}

// Launch arguments of every segment kernel.
struct SegParams {
    const u16 *q, *kp, *vp;
    const int32_t *qids, *kstart, *qlen, *klen, *rowbase, *items;
    u16 *part;   // [nslot, hq, D] fp16, scaled as above
    float *lse;  // [nslot, hq, 2]: log-sum-exp and scale exponent
    int n_items, hq, hk, group, tcap, maxr;
    float scale_log2;  // log2(e) / sqrt(D)
    // TA_TAIL items with a fused merge (out != nullptr): the request's partial
    // slots and the output
    const int32_t *slots, *counts;
    u16 *out;
    int maxs;
    // TA_LARGE256 items only (nullable): per item xtail_stride (=
    // TA_XTAIL_STRIDE) ints -- the number of attached segments (at most
    // TA_XTAIL_MAX), then (first token, tokens, first job row, rows) of each;
    // the item folds them into its rows' partials
    const int32_t *xtail;
    int xtail_stride;
    // nullable: per job the first request id when its requests are
    // consecutive, else -1 (the TA_LARGE256 kernel then skips the qids lookup)
    const int32_t *qbase;
};

// Kernel timing hook (ta_time_next_launch): when set, the next kernel this
// library launches on the calling host thread goes through hipExtLaunchKernel,
// which stamps `start` when the dispatch begins and `stop` when it ends; the
// hook then clears itself.
struct LaunchEvents {
    hipEvent_t start, stop;
};
extern thread_local LaunchEvents g_launch_events;

#define TA_LAUNCH(KERNEL, GRID, BLOCK, STREAM, ...)                                                   \
    do {                                                                                              \
        const ta::LaunchEvents ev_ = ta::g_launch_events;                                             \
        if (ev_.start) {                                                                              \
            ta::g_launch_events = ta::LaunchEvents{nullptr, nullptr};                                 \
            hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, 0, STREAM, ev_.start, ev_.stop, 0, __VA_ARGS__); \
        } else {                                                                                      \
            hipLaunchKernelGGL(KERNEL, GRID, BLOCK, 0, STREAM, __VA_ARGS__);                          \
        }                                                                                             \
    } while (0)

// Work items of several kinds in one launch (segment_tile.hip's
// seg_mix_kernel): p's fields but items / n_items, then per kind --
// TA_LARGE256 (with p.xtail), TA_LARGE64, TA_SMALL -- the item array, its
// count and the first block of the kind (a multiple of 8).
struct MixParams {
    SegParams p;
    const int32_t *items[3];
    int n[3];
    int base[3];
};

// Large-job launcher of segment_tile.hip (gfx950 LDS-transpose kernels).
// Returns hipErrorNotSupported when the shape is outside what it handles.
hipError_t launch_tile(const SegParams &sp, int kind, int d, bool fp16, hipStream_t stream);

// One launch of the TA_LARGE256, TA_LARGE64 and TA_SMALL items items[k]
// (n[k] of each) of one layer, side by side (hipErrorNotSupported unless the
// pool capacity is a multiple of 8).
hipError_t launch_tile_mix(const SegParams &sp, const int32_t *const items[3], const int n[3], int d, bool fp16,
                           hipStream_t stream);

}  // namespace ta

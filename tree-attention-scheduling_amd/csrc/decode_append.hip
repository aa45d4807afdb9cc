// decode_append.hip -- one decode step's per-layer glue in one launch.
//
// Replaces, for every layer of a decode step, the reference adapter's
//   q, k = apply_rotary_pos_emb(q, k, cos, sin)          (qwen.py:86, transformers'
//                                                         rotate-half RoPE)
//   kp.index_copy_(2, slots, k.permute(...))              (qwen.py:89)
//   vp.index_copy_(1, slots, v.permute(...))              (qwen.py:90)
//   q[:, :, 0, :].contiguous() / the Q layout step        (qwen.py:91, kernels.py:157)
// -- about ten small launches -- with one kernel that reads the projected
// (normalised) Q/K/V rows once, rotates Q and K, writes Q in the [R, HQ, D]
// layout attention_matrix takes, and scatters K and V into the pools' step
// columns.
//
// Rounding follows the eager PyTorch ops exactly: in the model dtype, RoPE is
// (x * cos) + (rotate_half(x) * sin), where each multiply and the add is
// computed in fp32 and rounded to the dtype (rotate_half only negates and
// moves values), so the outputs are bit-identical to the unfused path.
// Contraction is off in this file: for fp16 the compiler narrows the
// multiply and add to native half operations (exact), and contracting those
// into an FMA would skip the rounding of the product.
#include "ta_common.h"
#include "tree_attn.h"

#pragma clang fp contract(off)

namespace ta {
namespace {

template <bool FP16>
struct Half;
template <>
struct Half<false> {  // bfloat16
    __device__ static float load(const u16 *p) { return __builtin_bit_cast(float, (u32)*p << 16); }
    __device__ static u16 round(float x) { return __builtin_bit_cast(u16, (__bf16)x); }
    __device__ static float widen(u16 h) { return __builtin_bit_cast(float, (u32)h << 16); }
};
template <>
struct Half<true> {  // float16
    __device__ static float load(const u16 *p) { return (float)__builtin_bit_cast(_Float16, *p); }
    __device__ static u16 round(float x) { return __builtin_bit_cast(u16, (_Float16)x); }
    __device__ static float widen(u16 h) { return (float)__builtin_bit_cast(_Float16, h); }
};

// (x * c) + (r * s) with every operation rounded to the dtype, as the eager ops do
template <bool FP16>
__device__ inline u16 rope(float x, float c, float r, float s) {
    using H = Half<FP16>;
    return H::round(H::widen(H::round(x * c)) + H::widen(H::round(r * s)));
}

// One workgroup per (request, head row): rows 0 .. hq-1 are query heads, rows
// hq .. hq+hk-1 KV heads.  A lane owns rotate-half pairs (i, i + D/2).  Steps
// whose slot lies outside [0, tcap) write nothing to the pools.
template <bool FP16>
__global__ __launch_bounds__(64) void decode_append_kernel(const u16 *__restrict__ q, const u16 *__restrict__ k,
                                                           const u16 *__restrict__ v, const u16 *__restrict__ cos,
                                                           const u16 *__restrict__ sin,
                                                           const int32_t *__restrict__ slots, u16 *__restrict__ kp,
                                                           u16 *__restrict__ vp, u16 *__restrict__ qout, int hq,
                                                           int hk, int d, int tcap, int cs_stride) {
    using H = Half<FP16>;
    const int r = blockIdx.x, row = blockIdx.y, half = d / 2;
    const u16 *cr = cos + (size_t)r * cs_stride, *sr = sin + (size_t)r * cs_stride;
    const bool isq = row < hq;
    const int h = isq ? row : row - hq;
    const int slot = isq ? 0 : slots[r];
    const bool store = isq || (slot >= 0 && slot < tcap);
    const u16 *x = isq ? q + ((size_t)r * hq + h) * d : k + ((size_t)r * hk + h) * d;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float x0 = H::load(x + i), x1 = H::load(x + i + half);
        const float c0 = H::load(cr + i), c1 = H::load(cr + i + half);
        const float s0 = H::load(sr + i), s1 = H::load(sr + i + half);
        // rotate_half(x) = (-x1, x0)
        const u16 y0 = rope<FP16>(x0, c0, -x1, s0), y1 = rope<FP16>(x1, c1, x0, s1);
        if (isq) {
            u16 *dst = qout + ((size_t)r * hq + h) * d;
            dst[i] = y0;
            dst[i + half] = y1;
        } else if (store) {
            kp[((size_t)h * d + i) * tcap + slot] = y0;
            kp[((size_t)h * d + i + half) * tcap + slot] = y1;
            const u16 *vr = v + ((size_t)r * hk + h) * d;
            u16 *vd = vp + ((size_t)h * tcap + slot) * d;
            vd[i] = vr[i];
            vd[i + half] = vr[i + half];
        }
    }
}

}  // namespace
}  // namespace ta

extern "C" int ta_decode_append(const void *q, const void *k, const void *v, const void *cos, const void *sin,
                                int32_t cs_stride, const int32_t *slots, void *kp, void *vp, void *q_out,
                                int32_t nreq, int32_t hq, int32_t hk, int32_t d, int32_t tcap, int32_t dtype,
                                void *stream) {
    using namespace ta;
    if (dtype != TA_BF16 && dtype != TA_FP16) return TA_ERR_DTYPE;
    if (!q || !k || !v || !cos || !sin || !slots || !kp || !vp || !q_out) return TA_ERR_ARG;
    if (nreq <= 0 || hq <= 0 || hk <= 0 || tcap <= 0 || cs_stride < 0 || d < 2 || d % 2 || d > 1024)
        return TA_ERR_ARG;
    const dim3 grid(nreq, hq + hk), block(64);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (dtype == TA_FP16)
        TA_LAUNCH((decode_append_kernel<true>), grid, block, st, static_cast<const u16 *>(q),
                  static_cast<const u16 *>(k), static_cast<const u16 *>(v), static_cast<const u16 *>(cos),
                  static_cast<const u16 *>(sin), slots, static_cast<u16 *>(kp), static_cast<u16 *>(vp),
                  static_cast<u16 *>(q_out), hq, hk, d, tcap, cs_stride);
    else
        TA_LAUNCH((decode_append_kernel<false>), grid, block, st, static_cast<const u16 *>(q),
                  static_cast<const u16 *>(k), static_cast<const u16 *>(v), static_cast<const u16 *>(cos),
                  static_cast<const u16 *>(sin), slots, static_cast<u16 *>(kp), static_cast<u16 *>(vp),
                  static_cast<u16 *>(q_out), hq, hk, d, tcap, cs_stride);
    return (int)hipGetLastError();
}

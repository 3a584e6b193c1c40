// fp8 (e4m3fn) quantize-on-append: the rule and its device helpers, shared by the append
// kernels (kv_append_fp8.hip) and the fp8 decode kernel's fused append (attention.hip), so the
// two write the same bytes and scales by construction.
//
// The reference has no fp8 KV cache (its KV dtype is the model dtype, sdk/kv.py:76-143); this
// is the library's own rule, chosen so the result does not depend on the order of a step's rows:
//   1. The rows of one step that land in one page form a run of consecutive rows (an entry's
//      rows are its newest positions, in order); the run's first row is its leader.
//   2. For each (member m in {K, V}, kv head h) of the page, with t = absmax(run rows) / 448:
//        fresh  = the run writes the page's row 0 (a page is always filled from row 0, so the
//                 old scale and rows belong to a previous owner and are discarded)
//        s_old  = fresh ? 0 : scale[page, m, h]
//        s_new  = t when s_old = 0; s_old * 2^k when t > s_old > 0, k >= 1 the smallest with
//                 s_old * 2^k >= t; s_old otherwise
//        r_new  = 1 / s_new (0 when s_new = 0, and when s_new = inf)
//      When the scale grew (k > 0), every row of the page the run does not write is requantized
//      as q' = e4m3(clamp(f32(q) * 2^-k, +-448)) -- an exponent shift, exact unless the value
//      drops below e4m3's normals. Each run row is quantized as q = e4m3(clamp(x * r_new,
//      +-448)), or q = 0 when r_new = 0 (a run of zeros, or one holding an inf), and
//      scale[page, m, h] = s_new.
// A fresh page's largest element maps to 448; growth by powers of two keeps the e4m3 rounding of
// a decode stream (a row appended per step, the scale growing on many of them) from compounding.
// Products and quotients are single IEEE-754 binary32 operations rounded to nearest even; the
// e4m3 conversion rounds to nearest even.  Dequantized value = f32(q) * scale.  One reciprocal
// per (page, member, head) and a product per value (the form vLLM's scaled fp8 quantization
// uses) keeps the per-value work to a multiply, a clamp and half a conversion instruction.
//
#pragma once

#include "kvpath_device.h"

namespace kvpath {

__device__ __forceinline__ int64_t page_of(int64_t slot, int64_t block, int64_t pool) {
    return (slot >= 0 && slot < pool) ? slot / block : -1;
}

// Two f32 as two e4m3 bytes in the low (hi_word false) or high half of `word`: clamp to
// [-448, 448], then the hardware conversion (round to nearest even; the clamp keeps (448, 464]
// and beyond from becoming NaN).
template <bool HiWord>
__device__ __forceinline__ int cvt2_fp8(float x, float y, int word) {
    x = fminf(fmaxf(x, -kFp8Max), kFp8Max);
    y = fminf(fmaxf(y, -kFp8Max), kFp8Max);
    return __builtin_amdgcn_cvt_pk_fp8_f32(x, y, word, HiWord);
}

// The scale rule for one (page, member, head): s_new and the growth exponent k from the stored
// scale s_old (0 for a fresh page) and t = absmax / 448. Uniform across the lanes that call it.
__device__ __forceinline__ float grow_scale(float s_old, float t, int& k) {
    k = 0;
    if (!(s_old > 0.0f)) return t;
    if (!(t > s_old)) return s_old;
    k = 1;
    while (__builtin_amdgcn_ldexpf(s_old, k) < t) ++k;
    return __builtin_amdgcn_ldexpf(s_old, k);
}

// Eight e4m3 values shifted down by 2^k, requantized (exact for values that stay normal).
__device__ __forceinline__ u32x2 requant8(u32x2 q, int k) {
    const f32x4 lo = fp8x4_to_f32(q[0]), hi = fp8x4_to_f32(q[1]);
    const float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    int w0 = cvt2_fp8<false>(__builtin_amdgcn_ldexpf(x[0], -k), __builtin_amdgcn_ldexpf(x[1], -k), 0);
    w0 = cvt2_fp8<true>(__builtin_amdgcn_ldexpf(x[2], -k), __builtin_amdgcn_ldexpf(x[3], -k), w0);
    int w1 = cvt2_fp8<false>(__builtin_amdgcn_ldexpf(x[4], -k), __builtin_amdgcn_ldexpf(x[5], -k), 0);
    w1 = cvt2_fp8<true>(__builtin_amdgcn_ldexpf(x[6], -k), __builtin_amdgcn_ldexpf(x[7], -k), w1);
    return u32x2{static_cast<uint32_t>(w0), static_cast<uint32_t>(w1)};
}

// Eight values times r as eight e4m3 bytes.
__device__ __forceinline__ u32x2 quantize8(const float (&x)[8], float r) {
    int lo = cvt2_fp8<false>(x[0] * r, x[1] * r, 0);
    lo = cvt2_fp8<true>(x[2] * r, x[3] * r, lo);
    int hi = cvt2_fp8<false>(x[4] * r, x[5] * r, 0);
    hi = cvt2_fp8<true>(x[6] * r, x[7] * r, hi);
    return u32x2{static_cast<uint32_t>(lo), static_cast<uint32_t>(hi)};
}

// Eight bf16 (16 bytes) as eight f32, exact.
__device__ __forceinline__ void widen_bf16x8(u32x4 w, float (&x)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = __uint_as_float(w[i] << 16);
        x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

__device__ __forceinline__ float absmax8(const float (&x)[8]) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(x[i]));
    return m;
}

}  // namespace kvpath

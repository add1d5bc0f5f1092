// Per-head RMSNorm + rotary embedding of one head row held by a group of L
// lanes, 8 consecutive elements per lane -- the arithmetic shared by the
// fused norm/RoPE/KV-write kernel and the decode kernel's fused prologue, so
// that both produce the same bits.
//
// Rounding steps of the reference's eager fp16/bf16 path:
//   rmsnorm: n = T(T(x * rsqrt(mean(x^2) + eps)) * w)  (fallback.py:8-10,
//            elementwise.cu norm_kernel: the normalised value is rounded
//            before the weight multiply);
//   rope:    each product T(a * c) is rounded before the add / subtract, on
//            halves [0, D/2) and [D/2, D) (fallback.py:13-20, data.cu:29-65).
#pragma once

#include "mvme_common.h"

namespace mvme {

template <typename T>
__device__ inline float to_f(uint16_t h) {
    return T::lo((uint32_t)h);
}

template <typename T>
__device__ inline float round_t(float x) {
    return to_f<T>(T::from_float(x));
}

// Row of head_dim = 8 * L (L a power of two in [2, 64]); `sub` = the lane's
// index inside its group of L lanes, which holds elements 8*sub .. 8*sub+7
// in `xv`; `wv` the same elements of the norm weight; `cv` / `sv` the
// cos / sin entries 8*(sub mod L/2) .. +7 of the row's position.  Lane sub
// of the first half pairs with lane sub + L/2 (the same offsets of the
// second half); the partner's normalised values arrive by one lane exchange
// packed two per dword.  Every lane of the wave must call this (the sum of
// squares and the exchange read other lanes); lanes without a row pass zeros.
template <typename T, int L>
__device__ inline u32x4 norm_rope_lanes(u32x4 xv, u32x4 wv, u32x4 cv, u32x4 sv, float eps, int sub) {
    // No multiply-add contraction: once the float arithmetic below is narrowed
    // to fp16 instructions, contraction would fuse n1*c into the subtraction
    // and skip the product's own rounding.
#pragma clang fp contract(off)
    constexpr int kDim = 8 * L;
    constexpr int kHalfLanes = L / 2;
    float x[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        x[2 * j] = T::lo(xv[j]);
        x[2 * j + 1] = T::hi(xv[j]);
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = fmaf(x[j], x[j], ss);
    ss = group_sum<L>(ss);
    const float inv = 1.f / sqrtf(ss / (float)kDim + eps);
    float n[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        // x * inv is rounded to fp32 first, then to T (the reference's two
        // roundings); the empty asm keeps the compiler from turning the pair
        // into one mixed-precision multiply that rounds to T directly.
        float m = x[j] * inv;
        asm volatile("" : "+v"(m));
        const float wj = (j & 1) ? T::hi(wv[j / 2]) : T::lo(wv[j / 2]);
        n[j] = round_t<T>(round_t<T>(m) * wj);
    }
    const bool first = sub < kHalfLanes;
    u32x4 out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t mine = T::pack(n[2 * j], n[2 * j + 1]);
        const uint32_t other = (uint32_t)__builtin_amdgcn_ds_bpermute((__lane_id() ^ kHalfLanes) << 2, (int)mine);
        float o[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float own = n[2 * j + e];
            const float partner = e ? T::hi(other) : T::lo(other);
            const float c = e ? T::hi(cv[j]) : T::lo(cv[j]);
            const float s = e ? T::hi(sv[j]) : T::lo(sv[j]);
            // first half: x1*c - x2*s with x1 = own; second half: x1*s + x2*c with x1 = partner.
            o[e] = first ? round_t<T>(round_t<T>(own * c) - round_t<T>(partner * s))
                         : round_t<T>(round_t<T>(partner * s) + round_t<T>(own * c));
        }
        out[j] = T::pack(o[0], o[1]);
    }
    return out;
}

}  // namespace mvme

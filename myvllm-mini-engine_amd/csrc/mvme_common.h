// Device-side helpers shared by the gfx950 paged-attention kernels:
// element-type traits for fp16/bf16 (conversion, packed dot products,
// MFMA tiles), wave64 cross-lane reductions built on DPP, and the
// host-side error/launch bookkeeping of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/mvme_paged.h"

namespace mvme {

constexpr int kWave = 64;

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Element types.  Values travel as raw 16-bit patterns packed two per dword
// so that 16-byte global loads feed dot2 / MFMA instructions directly.
// ---------------------------------------------------------------------------
struct Half {
    static constexpr int kId = MVME_FP16;
    __device__ static inline float lo(uint32_t w) {
        return (float)__builtin_bit_cast(f16x2, w)[0];
    }
    __device__ static inline float hi(uint32_t w) {
        return (float)__builtin_bit_cast(f16x2, w)[1];
    }
    __device__ static inline uint16_t from_float(float x) {
        return __builtin_bit_cast(uint16_t, (_Float16)x);
    }
    __device__ static inline uint32_t pack(float a, float b) {
        f16x2 v = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(uint32_t, v);
    }
    // a.x*b.x + a.y*b.y + c with fp32 accumulation (v_dot2_f32_f16).
    __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a),
                                      __builtin_bit_cast(f16x2, b), c, false);
    }
    // 16x16x32 MFMA: 8 elements of A and B per lane, fp32 accumulators.
    __device__ static inline f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
};

struct BFloat16 {
    static constexpr int kId = MVME_BF16;
    __device__ static inline float lo(uint32_t w) { return __uint_as_float(w << 16); }
    __device__ static inline float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
    __device__ static inline uint16_t from_float(float x) {
        return __builtin_bit_cast(uint16_t, (__bf16)x);
    }
    __device__ static inline uint32_t pack(float a, float b) {
        bf16x2 v = {(__bf16)a, (__bf16)b};
        return __builtin_bit_cast(uint32_t, v);
    }
    __device__ static inline float dot2(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                               __builtin_bit_cast(bf16x2, b), c, false);
    }
    __device__ static inline f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
};

// ---------------------------------------------------------------------------
// Cross-lane helpers.
// ---------------------------------------------------------------------------
// DPP controls (gfx9 encoding): quad permutations and 16-lane row mirrors.
constexpr int kDppQuadSwap1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141; // lane i <- lane 7-i within 8
constexpr int kDppRowMirror = 0x140;     // lane i <- lane 15-i within 16

template <int CTRL>
__device__ inline float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

__device__ inline float shfl_xor(float v, int mask) {
    const int lane = __lane_id();
    return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}

// Sum over aligned groups of N consecutive lanes; every lane of a group
// receives the group total.  N <= 16 stays inside one DPP row.
template <int N>
__device__ inline float group_sum(float v) {
    if constexpr (N >= 2) v += dpp<kDppQuadSwap1>(v);
    if constexpr (N >= 4) v += dpp<kDppQuadSwap2>(v);
    if constexpr (N >= 8) v += dpp<kDppRowHalfMirror>(v);
    if constexpr (N >= 16) v += dpp<kDppRowMirror>(v);
    if constexpr (N >= 32) v += shfl_xor(v, 16);
    if constexpr (N >= 64) v += shfl_xor(v, 32);
    return v;
}

// Inclusive prefix sum over the 64 lanes of a wave, all in DPP (no LDS
// round trip): shifts by 1, 2, 4, 8 inside each 16-lane row, then the row
// totals carried forward by the row broadcasts of lane 15 (to rows 1 and 3)
// and lane 31 (to rows 2 and 3).  Lanes a shift or a row mask leaves
// unwritten take 0.
__device__ inline int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return x;
}

// Value of lane `l` (wave-uniform index) for every lane.
__device__ inline int lane_value(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ inline int64_t lane_value(int64_t v, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// ---------------------------------------------------------------------------
// Host-side status plumbing.
// ---------------------------------------------------------------------------
void set_error(const std::string& message);
int fail(int code, const std::string& message);
int check_launch(const char* what);

inline bool valid_dtype(int dtype) { return dtype == MVME_FP16 || dtype == MVME_BF16; }

}  // namespace mvme

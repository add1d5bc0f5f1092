// Greedy sampling (argmax over the vocabulary) of logits [batch, vocab] for gfx950.
//
// Semantics of torch.argmax, which the reference's greedy sampler uses
// (mini_engine/sampling.py:22-23) and its CUDA kernel reproduces
// (kernels/csrc/sampling.cu:1-68): the largest value wins; equal values and
// NaNs resolve to the lowest index; NaN ranks above every number, so the
// first NaN of a row wins; -0.0 equals +0.0.
//
// Each (value, index) becomes one 64-bit key whose unsigned order is that
// ranking: the high word is the value's bit pattern mapped to an unsigned
// order (negative values flipped, positive ones offset past them, NaN the
// largest), the low word is the complement of the index.  A row's argmax is
// then a plain unsigned maximum.  Rows are cut into `parts` slices so that
// even a decode batch of one row spreads over the CUs: one 256-lane
// work-group per (slice, row) takes the maximum over 16-byte loads, across
// the wave with lane exchanges and across the waves through LDS, and writes
// its key to the workspace; a second kernel reduces each row's keys.  With a
// single slice the first kernel writes the index directly.  HBM-bound: a
// 151,936-entry bf16 row is 304 KB.
#include <algorithm>

#include "mvme_common.h"

namespace mvme {
namespace {

constexpr int kArgThreads = 256;
constexpr int kArgWaves = kArgThreads / kWave;
constexpr int kArgMinSlice = 2048;   // elements per work-group at least
constexpr int kArgTargetGroups = 512;

__device__ inline uint64_t rank_key(float v, uint32_t index) {
    uint32_t order;
    if (v != v) {
        order = 0xffffffffu;
    } else {
        const uint32_t bits = __float_as_uint(v + 0.f);  // -0.0 + 0.0 = +0.0
        order = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);  // +inf -> 0xff800000 < NaN's rank
    }
    return ((uint64_t)order << 32) | (uint64_t)(0xffffffffu - index);
}

__device__ inline uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ inline uint64_t shfl_xor_u64(uint64_t v, int mask) {
    const int lane = __lane_id();
    const int lo = __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, (int)(uint32_t)v);
    const int hi = __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, (int)(uint32_t)(v >> 32));
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// Element loaders: 16 bytes -> VEC floats.
struct LoadF32 {
    static constexpr int kVec = 4;
    __device__ static void load(const void* p, float (&x)[kVec]) {
        const f32x4 w = *reinterpret_cast<const f32x4*>(p);
        x[0] = w[0]; x[1] = w[1]; x[2] = w[2]; x[3] = w[3];
    }
    __device__ static float one(const void* base, int64_t i) { return static_cast<const float*>(base)[i]; }
    static constexpr int kBytes = 4;
};
template <typename T>
struct Load16 {
    static constexpr int kVec = 8;
    __device__ static void load(const void* p, float (&x)[kVec]) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[2 * j] = T::lo(w[j]);
            x[2 * j + 1] = T::hi(w[j]);
        }
    }
    __device__ static float one(const void* base, int64_t i) {
        return T::lo((uint32_t) static_cast<const uint16_t*>(base)[i]);
    }
    static constexpr int kBytes = 2;
};

// Elements [begin, end) of one row; returns the work-group's maximum key
// (valid in lane 0 of wave 0).
template <typename L, bool VEC>
__device__ inline uint64_t slice_max(const uint8_t* base, int begin, int end, uint64_t* wave_best) {
    uint64_t best = 0;  // below every real key (the lowest, -inf at the last index, is 0x007fffff00000000)
    if constexpr (VEC) {
        constexpr int kVec = L::kVec;
        constexpr int kUnroll = 4;
        // begin is a multiple of kVec (slices are), so vectors never straddle it.
        const int v0 = begin / kVec, v1 = end / kVec;
        int v = v0 + (int)threadIdx.x;
        for (; v + (kUnroll - 1) * kArgThreads < v1; v += kUnroll * kArgThreads) {
            float x[kUnroll][kVec];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) L::load(base + (int64_t)(v + u * kArgThreads) * 16, x[u]);
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
#pragma unroll
                for (int j = 0; j < kVec; ++j)
                    best = max_u64(best, rank_key(x[u][j], (uint32_t)((v + u * kArgThreads) * kVec + j)));
        }
        for (; v < v1; v += kArgThreads) {
            float x[kVec];
            L::load(base + (int64_t)v * 16, x);
#pragma unroll
            for (int j = 0; j < kVec; ++j) best = max_u64(best, rank_key(x[j], (uint32_t)(v * kVec + j)));
        }
        for (int i = v1 * kVec + (int)threadIdx.x; i < end; i += kArgThreads)
            best = max_u64(best, rank_key(L::one(base, i), (uint32_t)i));
    } else {
        for (int i = begin + (int)threadIdx.x; i < end; i += kArgThreads)
            best = max_u64(best, rank_key(L::one(base, i), (uint32_t)i));
    }
#pragma unroll
    for (int mask = 1; mask < kWave; mask <<= 1) best = max_u64(best, shfl_xor_u64(best, mask));
    if ((threadIdx.x & (kWave - 1)) == 0) wave_best[threadIdx.x / kWave] = best;
    __syncthreads();
    uint64_t b = wave_best[0];
#pragma unroll
    for (int w = 1; w < kArgWaves; ++w) b = max_u64(b, wave_best[w]);
    return b;
}

// grid (parts, batch).  parts == 1: writes the index; otherwise the slice's key.
template <typename L, bool VEC>
__global__ __launch_bounds__(kArgThreads) void argmax_slice_kernel(int64_t* out, uint64_t* keys, const void* logits,
                                                                  int vocab, int64_t row_stride, int slice) {
    __shared__ uint64_t wave_best[kArgWaves];
    const int64_t row = blockIdx.y;
    const int part = blockIdx.x;
    const uint8_t* base = static_cast<const uint8_t*>(logits) + row * row_stride * L::kBytes;
    const int begin = part * slice;
    const int end = min(vocab, begin + slice);
    const uint64_t b = slice_max<L, VEC>(base, begin, end, wave_best);
    if (threadIdx.x == 0) {
        if (gridDim.x == 1) out[row] = (int64_t)(0xffffffffu - (uint32_t)b);
        else keys[row * gridDim.x + part] = b;
    }
}

// One wave per row: maximum over the row's slice keys.
__global__ __launch_bounds__(kWave) void argmax_rows_kernel(int64_t* out, const uint64_t* keys, int parts) {
    const int64_t row = blockIdx.x;
    uint64_t best = 0;
    for (int p = threadIdx.x; p < parts; p += kWave) best = max_u64(best, keys[row * parts + p]);
#pragma unroll
    for (int mask = 1; mask < kWave; mask <<= 1) best = max_u64(best, shfl_xor_u64(best, mask));
    if (threadIdx.x == 0) out[row] = (int64_t)(0xffffffffu - (uint32_t)best);
}

// Slices per row: enough work-groups to cover the CUs twice, each at least
// kArgMinSlice elements; slice lengths are multiples of 8 (whole 16-byte
// vectors for every element size).
struct ArgmaxPlan {
    int parts;
    int slice;
};

ArgmaxPlan argmax_plan(int64_t batch, int64_t vocab) {
    const int64_t max_parts = std::max<int64_t>(1, (vocab + kArgMinSlice - 1) / kArgMinSlice);
    int64_t parts = std::min<int64_t>(max_parts, std::max<int64_t>(1, (kArgTargetGroups + batch - 1) / batch));
    int64_t slice = (vocab + parts - 1) / parts;
    slice = (slice + 7) / 8 * 8;
    parts = (vocab + slice - 1) / slice;
    return {(int)parts, (int)slice};
}

template <typename L>
void launch_argmax(int64_t* out, uint64_t* keys, const void* logits, int64_t batch, int64_t vocab,
                   int64_t row_stride, const ArgmaxPlan& plan, hipStream_t s) {
    const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 && (row_stride * L::kBytes) % 16 == 0;
    const dim3 grid((unsigned)plan.parts, (unsigned)batch), block(kArgThreads);
    if (vec)
        hipLaunchKernelGGL((argmax_slice_kernel<L, true>), grid, block, 0, s, out, keys, logits, (int)vocab,
                           row_stride, plan.slice);
    else
        hipLaunchKernelGGL((argmax_slice_kernel<L, false>), grid, block, 0, s, out, keys, logits, (int)vocab,
                           row_stride, plan.slice);
}

}  // namespace
}  // namespace mvme

using namespace mvme;

extern "C" size_t mvme_greedy_argmax_workspace_size(int64_t batch, int64_t vocab) {
    if (batch <= 0 || vocab <= 0 || batch > 65535 || vocab > 2147483647) return 0;
    const ArgmaxPlan plan = argmax_plan(batch, vocab);
    return plan.parts > 1 ? (size_t)batch * (size_t)plan.parts * sizeof(uint64_t) : 0;
}

extern "C" int mvme_greedy_argmax(int64_t* out, const void* logits, int64_t batch, int64_t vocab, int64_t row_stride,
                                  int dtype, void* workspace, size_t workspace_bytes, void* stream) {
    if (dtype != MVME_FP16 && dtype != MVME_BF16 && dtype != MVME_FP32)
        return fail(MVME_EINVAL, "greedy supports FP32/FP16/BF16");
    if (batch < 0 || vocab <= 0) return fail(MVME_EINVAL, "greedy logits must be [batch, nonempty vocab]");
    if (batch > 65535 || vocab > 2147483647) return fail(MVME_EINVAL, "greedy logits shape too large");
    if (row_stride < vocab) return fail(MVME_EINVAL, "greedy logits row stride smaller than the vocabulary");
    if (batch == 0) return MVME_OK;
    if (!out || !logits) return fail(MVME_EINVAL, "greedy argmax received a null pointer");
    const ArgmaxPlan plan = argmax_plan(batch, vocab);
    const size_t need = plan.parts > 1 ? (size_t)batch * (size_t)plan.parts * sizeof(uint64_t) : 0;
    if (need > 0 && (!workspace || workspace_bytes < need))
        return fail(MVME_EWORKSPACE, "greedy argmax workspace too small");
    if (need > 0 && (reinterpret_cast<uintptr_t>(workspace) & 7u) != 0)
        return fail(MVME_EWORKSPACE, "greedy argmax workspace must be 8-byte aligned");
    uint64_t* keys = static_cast<uint64_t*>(workspace);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == MVME_FP32) launch_argmax<LoadF32>(out, keys, logits, batch, vocab, row_stride, plan, s);
    else if (dtype == MVME_FP16) launch_argmax<Load16<Half>>(out, keys, logits, batch, vocab, row_stride, plan, s);
    else launch_argmax<Load16<BFloat16>>(out, keys, logits, batch, vocab, row_stride, plan, s);
    if (plan.parts > 1)
        hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)batch), dim3(kWave), 0, s, out, keys, plan.parts);
    return check_launch("greedy argmax");
}

// Linear layer for a few rows (the decode batch): out[M, N] = x[M, K] W[N, K]^T
// (+ bias) with nn.Linear's weight layout, for M <= 64, on gfx950 MFMA.
//
// The reference's CudaLinear (mini_engine/kernels/linear.py:14-30) calls
// torch.mm(x, weight.t()); at decode sizes (M = batch, K = N = 2048 for the
// attention output projection) that GEMM reads the 8 MB weight at a small
// fraction of HBM bandwidth, because a library tile sized for large M leaves
// most CUs idle.  Here the weight is the only large operand and is read
// once: one work-group per 16 output features, its 16 waves splitting K,
// each wave computing D[n, m] = W[n, k-slice] x[m, k-slice]^T for every
// 16-row block of x with v_mfma_f32_16x16x32 (fp32 accumulation), then the
// 16 partial tiles are summed through LDS and rounded once to the output type.
#include "mvme_common.h"

namespace mvme {
namespace {

constexpr int kLinWaves = 16;
constexpr int kLinThreads = kLinWaves * kWave;
constexpr int kLinMaxRows = 64;
constexpr int kLinMaxBlocks = kLinMaxRows / 16;

struct LinearArgs {
    void* out;
    const void* x;
    const void* weight;
    const void* bias;  // nullptr: none
    int rows;          // M
    int in_features;   // K, a multiple of 32
    int out_features;  // N, a multiple of 16
    int64_t x_stride;  // elements between rows of x
};

// A operand: W rows n0 + (lane % 16), k = k0 + 8 * (lane / 16) .. +8.
// B operand: x rows 16 * mb + (lane % 16), same k.  D: lane holds output
// feature n0 + 4 * (lane / 16) + i (i < 4) for row 16 * mb + lane % 16.
template <typename T, int MB>
__global__ __launch_bounds__(kLinThreads) void linear_rows_kernel(LinearArgs a) {
    __shared__ f32x4 sm_part[kLinWaves][MB][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int n0 = blockIdx.x * 16;
    const int li = lane & 15, lg = lane >> 4;
    const int ksteps = a.in_features / 32;
    const uint16_t* wrow = static_cast<const uint16_t*>(a.weight) + (int64_t)(n0 + li) * a.in_features + 8 * lg;
    const uint16_t* xbase = static_cast<const uint16_t*>(a.x) + 8 * lg;
    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Rows of x past M read row 0 (in bounds) and are masked to zero.
    bool row_ok[MB];
    const uint16_t* xrow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int r = 16 * mb + li;
        row_ok[mb] = r < a.rows;
        xrow[mb] = xbase + (int64_t)(row_ok[mb] ? r : 0) * a.x_stride;
    }
    // This wave's k-steps: wave, wave + 16, ...  Four in flight at a time (all
    // of them at K = 2048).
    constexpr int kBatch = 4;
    for (int s0 = wave; s0 < ksteps; s0 += kLinWaves * kBatch) {
        u32x4 wv[kBatch], xv[kBatch][MB];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int s = min(s0 + j * kLinWaves, ksteps - 1);  // past the end: re-read the last, unused
            wv[j] = *reinterpret_cast<const u32x4*>(wrow + 32 * s);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) xv[j][mb] = *reinterpret_cast<const u32x4*>(xrow[mb] + 32 * s);
        }
        // No branch between the loads and the products (a branch would make
        // the compiler wait for each step's loads before issuing the next):
        // steps past the end multiply a zero operand.
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const bool step_ok = s0 + j * kLinWaves < ksteps;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const u32x4 b = (row_ok[mb] && step_ok) ? xv[j][mb] : u32x4{0u, 0u, 0u, 0u};
                acc[mb] = T::mfma16x16x32(wv[j], b, acc[mb]);
            }
        }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) sm_part[wave][mb][lane] = acc[mb];
    __syncthreads();
    // Thread t sums the waves' partials of one (row block, lane) slot.
    for (int slot = threadIdx.x; slot < MB * kWave; slot += kLinThreads) {
        const int mb = slot / kWave, l = slot % kWave;
        // Every partial is read before any is added (the reads overlap).
        f32x4 part[kLinWaves];
#pragma unroll
        for (int w = 0; w < kLinWaves; ++w) part[w] = sm_part[w][mb][l];
#pragma unroll
        for (int stride = kLinWaves / 2; stride > 0; stride /= 2)
#pragma unroll
            for (int w = 0; w < stride; ++w) part[w] += part[w + stride];
        const f32x4 sum = part[0];
        const int row = 16 * mb + (l & 15);
        if (row >= a.rows) continue;
        const int nb = n0 + 4 * (l >> 4);
        float v[4] = {sum[0], sum[1], sum[2], sum[3]};
        if (a.bias) {
            const uint16_t* bias = static_cast<const uint16_t*>(a.bias) + nb;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] += T::lo((uint32_t)bias[i]);
        }
        const u32x2 packed = {T::pack(v[0], v[1]), T::pack(v[2], v[3])};
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + (int64_t)row * a.out_features + nb) = packed;
    }
}

template <typename T>
void launch_linear_rows(const LinearArgs& a, hipStream_t s) {
    const dim3 grid((unsigned)(a.out_features / 16)), block(kLinThreads);
    const int mb = (a.rows + 15) / 16;
    if (mb == 1) hipLaunchKernelGGL((linear_rows_kernel<T, 1>), grid, block, 0, s, a);
    else if (mb == 2) hipLaunchKernelGGL((linear_rows_kernel<T, 2>), grid, block, 0, s, a);
    else if (mb == 3) hipLaunchKernelGGL((linear_rows_kernel<T, 3>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((linear_rows_kernel<T, 4>), grid, block, 0, s, a);
}

}  // namespace
}  // namespace mvme

using namespace mvme;

extern "C" int mvme_linear_rows(void* out, const void* x, const void* weight, const void* bias, int64_t rows,
                                int64_t in_features, int64_t out_features, int64_t x_row_stride, int dtype,
                                void* stream) {
    if (dtype != MVME_FP16 && dtype != MVME_BF16) return fail(MVME_EINVAL, "linear rows supports FP16/BF16");
    if (rows < 0 || rows > kLinMaxRows) return fail(MVME_EINVAL, "linear rows supports at most 64 rows");
    if (in_features <= 0 || in_features % 32 != 0 || in_features > 2147483647)
        return fail(MVME_EINVAL, "linear rows needs in_features a positive multiple of 32");
    if (out_features <= 0 || out_features % 16 != 0 || out_features / 16 > 2147483647)
        return fail(MVME_EINVAL, "linear rows needs out_features a positive multiple of 16");
    if (x_row_stride < in_features || x_row_stride % 8 != 0)
        return fail(MVME_EINVAL, "linear rows needs a row stride >= in_features and a multiple of 8");
    if (rows == 0) return MVME_OK;
    if (!out || !x || !weight) return fail(MVME_EINVAL, "linear rows received a null pointer");
    const auto misaligned = [](const void* p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & m) != 0; };
    if (misaligned(x, 15) || misaligned(weight, 15) || misaligned(out, 7) || (bias && misaligned(bias, 1)))
        return fail(MVME_EINVAL, "linear rows needs 16-byte aligned x and weight and 8-byte aligned out");
    LinearArgs a{};
    a.out = out;
    a.x = x;
    a.weight = weight;
    a.bias = bias;
    a.rows = (int)rows;
    a.in_features = (int)in_features;
    a.out_features = (int)out_features;
    a.x_stride = x_row_stride;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == MVME_FP16) launch_linear_rows<Half>(a, s);
    else launch_linear_rows<BFloat16>(a, s);
    return check_launch("linear rows");
}

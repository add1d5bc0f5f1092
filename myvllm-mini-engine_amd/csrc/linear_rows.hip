// Linear layer for a few rows (the decode batch): out[M, N] = x[M, K] W[N, K]^T
// (+ bias) with nn.Linear's weight layout, for M <= 64, on gfx950 MFMA.
//
// The reference's CudaLinear (mini_engine/kernels/linear.py:14-30) calls
// torch.mm(x, weight.t()); at decode sizes (M = batch, K = N = 2048 for the
// attention output projection) that GEMM reads the 8 MB weight at a small
// fraction of HBM bandwidth, because a library tile sized for large M leaves
// most CUs idle.  Here the weight is the only large operand and is read
// once.  Two kernels:
// * staged (K a multiple of 512, N of 8, operands within 160 KB of LDS --
//   the decode batch): one work-group per 8 output features, x and the
//   weight slab copied global->LDS in whole 1 KiB segments;
// * register (any other shape): one work-group per 16 output features, each
//   lane loading its operands straight into registers.
// In both, the 16 waves split K, each wave computing D[n, m] = W[n, k-slice]
// x[m, k-slice]^T for every 16-row block of x with v_mfma_f32_16x16x32 (fp32
// accumulation), then the 16 partial tiles are summed through LDS and
// rounded once to the output type.  Measured over 28 layers' distinct
// 2048 x 2048 bf16 weights at 32 rows: register kernel 7.8 us per call,
// staged kernel 5.5 us (x re-read from L2 by every work-group dominated the
// register kernel: 5.6 us with the weight loads removed, 4.3 us with the
// x loads removed; with 8 features per work-group, as the staged kernel
// has, it took 7.7 us).
#include <mutex>

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

// Staged variant for the decode batch (K a multiple of 512, N of 8, x and an
// 8-feature weight slab fitting in LDS): one work-group per 8 output
// features, 256 work-groups at N = 2048, so every CU streams its share of
// the weight.  Both operands reach LDS by direct global->LDS copies of whole
// 1 KiB row segments (coalesced, no VGPR staging): the x rows [16*MB][K]
// with 16-byte chunk c of row r at chunk c ^ (r & 15), the weight rows
// n0..n0+7 [8][K] at c ^ (r & 7), so the operand reads (16 rows x one chunk
// per MFMA) hit distinct banks.  The A operand of the 16x16x32 product
// takes weight row li & 7 (rows 8..15 repeat 0..7; their outputs are
// dropped); each wave then accumulates its k-steps as the register kernel
// does, and the wave partials are summed through LDS (aliasing the x rows).
constexpr int kStagedFeat = 8;
constexpr size_t kStagedMaxLds = 160 * 1024;

__device__ inline void lds_copy16(const void* gptr, uint32_t lds_base) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_base);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gptr), "s"(base) : "m0");
}

template <typename P>
__device__ inline uint32_t lds_offset(P* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)p;
}

size_t staged_lds_bytes(int mb, int64_t in_features) {
    const size_t operands = (size_t)(16 * mb + kStagedFeat) * in_features * 2;
    const size_t partials = (size_t)kLinWaves * mb * kWave * sizeof(f32x4);
    return operands > partials ? operands : partials;
}

template <typename T, int MB>
__global__ __launch_bounds__(kLinThreads) void linear_rows_staged_kernel(LinearArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int n0 = blockIdx.x * kStagedFeat;
    const int li = lane & 15, lg = lane >> 4;
    const int K = a.in_features;
    const int row_chunks = K / 8;          // 16-byte chunks per row
    const int row_instr = row_chunks / 64;  // 1 KiB copies per row
    uint8_t* xs = smem;
    uint8_t* ws = smem + (size_t)16 * MB * K * 2;
    // The weight slab first: its copies come from HBM, x's from L2 (every
    // work-group reads the same x), so the longer latency starts first
    // (5.9 -> 5.5 us per call at 32 x 2048 x 2048).
    for (int i = wave; i < kStagedFeat * row_instr; i += kLinWaves) {
        const int r = i / row_instr, cbase = (i % row_instr) * 64;
        const int c = (cbase + lane) ^ (r & 7);
        const uint16_t* src = static_cast<const uint16_t*>(a.weight) + (int64_t)(n0 + r) * K + 8 * c;
        lds_copy16(src, lds_offset(ws) + (uint32_t)(r * row_chunks + cbase) * 16);
    }
    // Rows of x past M copy row 0 (in bounds); their products are dropped.
    for (int i = wave; i < 16 * MB * row_instr; i += kLinWaves) {
        const int r = i / row_instr, cbase = (i % row_instr) * 64;
        const int c = (cbase + lane) ^ (r & 15);
        const uint16_t* src = static_cast<const uint16_t*>(a.x) + (int64_t)(r < a.rows ? r : 0) * a.x_stride + 8 * c;
        lds_copy16(src, lds_offset(xs) + (uint32_t)(r * row_chunks + cbase) * 16);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies landed
    __syncthreads();                // everyone's
    f32x4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int wr = li & 7;
    for (int st = wave; st < K / 32; st += kLinWaves) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(ws + (size_t)(wr * row_chunks + ((4 * st + lg) ^ wr)) * 16);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int r = 16 * mb + li;
            u32x4 x = *reinterpret_cast<const u32x4*>(xs + (size_t)(r * row_chunks + ((4 * st + lg) ^ (r & 15))) * 16);
            if (r >= a.rows) x = u32x4{0u, 0u, 0u, 0u};
            acc[mb] = T::mfma16x16x32(w, x, acc[mb]);
        }
    }
    __syncthreads();  // the operand rows are no longer read
    f32x4* part = reinterpret_cast<f32x4*>(smem);  // [wave][MB][lane]
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) part[(wave * MB + mb) * kWave + lane] = acc[mb];
    __syncthreads();
    // Thread t sums the waves' partials of one (row block, lane) slot whose
    // features are real (lanes 0..31 of the tile hold features 0..7).
    for (int slot = threadIdx.x; slot < MB * kWave; slot += kLinThreads) {
        const int mb = slot / kWave, l = slot % kWave;
        if ((l >> 4) >= kStagedFeat / 4) continue;
        f32x4 p[kLinWaves];
#pragma unroll
        for (int w = 0; w < kLinWaves; ++w) p[w] = part[(w * MB + mb) * kWave + l];
#pragma unroll
        for (int stride = kLinWaves / 2; stride > 0; stride /= 2)
#pragma unroll
            for (int w = 0; w < stride; ++w) p[w] += p[w + stride];
        const int row = 16 * mb + (l & 15);
        if (row >= a.rows) continue;
        const int nb = n0 + 4 * (l >> 4);
        float v[4] = {p[0][0], p[0][1], p[0][2], p[0][3]};
        if (a.bias) {
            const uint16_t* bias = static_cast<const uint16_t*>(a.bias) + nb;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] += T::lo((uint32_t)bias[i]);
        }
        const u32x2 packed = {T::pack(v[0], v[1]), T::pack(v[2], v[3])};
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + (int64_t)row * a.out_features + nb) = packed;
    }
}

template <typename T, int MB>
int launch_staged(const LinearArgs& a, hipStream_t s) {
    const size_t lds = staged_lds_bytes(MB, a.in_features);
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute(reinterpret_cast<const void*>(linear_rows_staged_kernel<T, MB>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)kStagedMaxLds);
    });
    if (attr != hipSuccess) return fail(MVME_ELAUNCH, std::string("linear rows: LDS size attribute: ") +
                                                      hipGetErrorString(attr));
    hipLaunchKernelGGL((linear_rows_staged_kernel<T, MB>), dim3((unsigned)(a.out_features / kStagedFeat)),
                       dim3(kLinThreads), lds, s, a);
    return MVME_OK;
}

template <typename T>
int launch_linear_staged(const LinearArgs& a, int mb, hipStream_t s) {
    if (mb == 1) return launch_staged<T, 1>(a, s);
    if (mb == 2) return launch_staged<T, 2>(a, s);
    if (mb == 3) return launch_staged<T, 3>(a, s);
    return launch_staged<T, 4>(a, s);
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
    const int mb = (int)((rows + 15) / 16);
    if (in_features % 512 == 0 && out_features % kStagedFeat == 0 &&
        staged_lds_bytes(mb, in_features) <= kStagedMaxLds) {
        const int rc = dtype == MVME_FP16 ? launch_linear_staged<Half>(a, mb, s) : launch_linear_staged<BFloat16>(a, mb, s);
        if (rc != MVME_OK) return rc;
        return check_launch("linear rows");
    }
    if (dtype == MVME_FP16) launch_linear_rows<Half>(a, s);
    else launch_linear_rows<BFloat16>(a, s);
    return check_launch("linear rows");
}

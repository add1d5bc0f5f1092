// GQA paged decode attention for gfx950: launch plan, split-K merge and
// the C entry points.  The attention kernel and its design notes are in
// paged_decode_kernel.h.
#include <mutex>

#include "paged_decode_kernel.h"

namespace mvme {
namespace {

// Split-K combine: out = sum_p acc_p 2^(m_p - M) / sum_p l_p 2^(m_p - M).
// Partitions that never saw a valid token carry m = -inf and contribute 0;
// an all-empty sequence produces 0.
// One work-group of whole waves per (sequence, query head), D rounded up to
// 64 threads; thread t < D owns output dim t.  Threads past D take part in
// the partition-maximum and weight loops and feed the identities (-inf for
// the maximum, 0 for the sums) into the reductions, so a wave never reads a
// lane that does not exist.  Every step loads many partitions at once: the
// partition maxima one per thread, then (per window of partitions) the
// weights 2^(m_p - ref) into LDS and each dim's partials eight at a time.
constexpr int kMergeWindow = 2048;  // partition weights held in LDS at once

template <int D>
constexpr int merge_threads() { return (D + kWave - 1) / kWave * kWave; }

template <typename T, int D>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeArgs a) {
    static_assert(D <= 256, "one thread per output dim");
    constexpr int kThreads = merge_threads<D>();
    __shared__ float sm_red[kThreads / kWave];
    __shared__ float sm_w[kMergeWindow];
    const int64_t bh = blockIdx.x;
    const int b = (int)(bh / a.q_heads);
    const int len = seq_tokens(a.lens[b], a.capacity);
    const int nparts = len > 0 ? (len + a.partition - 1) / a.partition : 1;
    if (nparts == 1) return;  // written directly by the attention kernel
    const float* ml = a.ws_ml + bh * a.max_parts * 2;
    const float* acc = a.ws_acc + bh * a.max_parts * D;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1), wave = tid / kWave;
    constexpr int kWaves = kThreads / kWave;
    const bool owns_dim = tid < D;
    auto block_reduce = [&](float v, bool is_max) __attribute__((always_inline)) {
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) {
            const float o = __shfl_xor(v, off);
            v = is_max ? fmaxf(v, o) : v + o;
        }
        __syncthreads();  // earlier reads of sm_red are done
        if (lane == 0) sm_red[wave] = v;
        __syncthreads();
        v = sm_red[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) v = is_max ? fmaxf(v, sm_red[w]) : v + sm_red[w];
        return v;
    };
    float mx = kNegInf;
    for (int p = tid; p < nparts; p += kThreads) mx = fmaxf(mx, ml[2 * p]);
    mx = block_reduce(mx, true);
    const float ref = mx == kNegInf ? 0.f : mx;
    constexpr int kBatch = 8;
    float o = 0.f, sum = 0.f;
    for (int w0 = 0; w0 < nparts; w0 += kMergeWindow) {
        const int n = min(kMergeWindow, nparts - w0);
        __syncthreads();  // the previous window's weights are no longer read
        for (int p = tid; p < n; p += kThreads) {
            const float w = fast_exp2(ml[2 * (w0 + p)] - ref);
            sm_w[p] = w;
            sum += ml[2 * (w0 + p) + 1] * w;
        }
        __syncthreads();
        if (!owns_dim) continue;
        const float* accw = acc + (int64_t)w0 * D + tid;
        for (int p0 = 0; p0 < n; p0 += kBatch) {
            // Indices past the window's last partition re-read it; the
            // select drops them.
            float av[kBatch], wv[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int pk = min(p0 + k, n - 1);
                av[k] = accw[(int64_t)pk * D];
                wv[k] = sm_w[pk];
            }
#pragma unroll
            for (int k = 0; k < kBatch; ++k) o += p0 + k < n ? av[k] * wv[k] : 0.f;
        }
    }
    sum = block_reduce(sum, false);
    if (owns_dim) static_cast<uint16_t*>(a.out)[bh * D + tid] = T::from_float(sum > 0.f ? o / sum : 0.f);
}

// Merge of the balanced walk: work-group l merges the unit its share's
// descriptor names (one that began in an earlier share and ends in this
// one).  The unit's pieces are the shares from p0, the one holding its first
// chunk, up to l; share p0 wrote its piece in row slot `slot0` (1 when the
// unit was its last segment), every later one as its first segment (slot 0).
// Shares left empty (fewer chunks than work-groups) wrote nothing: they get
// weight 0 and read the merging share's own row instead, so every load is
// unconditional.  A unit has at most one piece per work-group of the walk:
// thread t reads piece t's (reference, sum) pairs, the block maximum gives
// the reference, and the weights and row offsets go to LDS; each output dim
// then sums its pieces in order, kBatch loads at a time (the same sums, in
// the same order, as one piece after the other; a zero weight adds nothing).
// Work-group g merges share (g mod 8) * kFlatGroups/8 + g/8, the share the
// attention kernel's work-group g computed, so the merge runs on the XCD
// whose L2 holds that share's partials.  Measured against the first version
// (one piece after the other, each a dependent load, and the walk's prefix
// sums recomputed before the first load; µs per call): one sequence of
// 32768 keys 32.0 -> 29.7, two of 8192 27.5 -> 18.3, 8 of 512 11.9 -> 9.6.
template <typename T, int D, int G>
__global__ __launch_bounds__(kLptMax) void paged_decode_flat_merge_kernel(DecodeArgs a) {
    __shared__ float sm_red[G][kLptMax / kWave];
    __shared__ float sm_w[G][kLptMax];
    __shared__ float sm_lw[G][kLptMax];
    __shared__ int64_t sm_row[kLptMax];
    const int64_t l = (blockIdx.x & 7) * (kFlatGroups >> 3) + (blockIdx.x >> 3);
    const FlatMergeDesc dsc = a.ws_flat[l];
    if (dsc.b < 0) return;
    const int64_t total = dsc.total;
    const int64_t p0 = dsc.p0;
    const int n = (int)(l - p0 + 1);
    const int kvh = dsc.r / a.gtiles;
    const int h0 = kvh * a.group + (dsc.r - kvh * a.gtiles) * G;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int64_t p = p0 + tid;
    const bool live = tid < n && flat_share_start(p, total) < flat_share_start(p + 1, total);
    const int64_t row = (p * 2 + (tid == 0 ? dsc.slot0 : 0)) * G;
    float m[G], lsum[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = live ? a.ws_ml[(row + g) * 2] : kNegInf;
        lsum[g] = live ? a.ws_ml[(row + g) * 2 + 1] : 0.f;
        float v = m[g];
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
        if (lane == 0) sm_red[g][wave] = v;
    }
    // Empty pieces read the merging share's own row (always written) and
    // are dropped by their zero weight.
    if (tid < n) sm_row[tid] = live ? row : (l * 2) * G;
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float mx = sm_red[g][0];
#pragma unroll
        for (int w = 1; w < kLptMax / kWave; ++w) mx = fmaxf(mx, sm_red[g][w]);
        const float ref = mx == kNegInf ? 0.f : mx;
        const float w = live ? fast_exp2(m[g] - ref) : 0.f;
        if (tid < n) {
            sm_w[g][tid] = w;
            sm_lw[g][tid] = live ? lsum[g] * w : 0.f;
        }
    }
    __syncthreads();
    constexpr int kBatch = 16;
    for (int idx = tid; idx < G * D; idx += kLptMax) {
        const int g = idx / D;
        const int d = idx - g * D;
        float sum = 0.f, o = 0.f;
        for (int t0 = 0; t0 < n; t0 += kBatch) {
            float av[kBatch];
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                av[k] = a.ws_acc[(sm_row[min(t0 + k, n - 1)] + g) * D + d];
            }
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int t = min(t0 + k, n - 1);
                const bool use = t0 + k < n && sm_w[g][t] != 0.f;
                sum += use ? sm_lw[g][t] : 0.f;
                o += use ? av[k] * sm_w[g][t] : 0.f;
            }
        }
        static_cast<uint16_t*>(a.out)[((int64_t)dsc.b * a.q_heads + h0 + g) * D + d] =
            T::from_float(sum > 0.f ? o / sum : 0.f);
    }
}

struct DecodePlan {
    int partition;
    int max_parts;
    int gtile;  // G of the kernel instance
    int waves;  // waves per work-group (kSplitWaves or kWholeWaves; kFlatWaves in the walk)
    bool stream;  // non-temporal K/V loads
    int flat_groups;  // > 0: balanced walk with this many work-groups
};


constexpr int64_t kStreamBytes = int64_t(64) << 20;  // K+V bytes within capacity above which loads stream

int decode_tile_tokens(int64_t head_dim) {
    switch (head_dim) {
        case 16: return DecodeShape<16>::kTpi;
        case 32: return DecodeShape<32>::kTpi;
        case 64: return DecodeShape<64>::kTpi;
        case 80: return DecodeShape<80>::kTpi;
        case 96: return DecodeShape<96>::kTpi;
        case 128: return DecodeShape<128>::kTpi;
        case 192: return DecodeShape<192>::kTpi;
        case 256: return DecodeShape<256>::kTpi;
        default: return 0;
    }
}

constexpr int64_t kDeviceCUs = 256;  // MI355X compute units

// Host-side plan (lengths stay on the device, so it depends on the table
// capacity only).  Long units (kLongUnitBytes of K+V capacity) numbering at
// most one per CU take the balanced walk.  Otherwise, enough (sequence, kv
// head) units to occupy every CU, a capacity of one 16-wave step, or two
// steps with more than a quarter of the CUs' worth of units: one work-group
// per unit over the whole context, merged in LDS (8 waves; with two
// work-groups per CU holding every unit, long sequences paired with short
// ones; below two 16-wave steps, 4 waves when the units outnumber the CUs).
// (A "16-wave step" is 16 wave iterations of tokens, the unit the
// thresholds were measured in.)  Otherwise split-K into partitions of 4-wave
// work-groups, sized to give every CU about two work-groups (at least one
// 4-wave step each), plus a merge kernel.  `requested` > 0 forces split-K
// with that partition length (rounded to the wave tiling), -1 the balanced
// walk (batch <= 256).
//
// Measured at head_dim 128 (bf16, block 16, 16/8 heads, µs per call in a
// graph): whole-sequence against split-K at 64/128/256 keys.
// * ctx 128: whole 4.9-5.1, any split about 2 µs more (the merge launch).
// * ctx 256: level up to 64 units; whole ahead from 128 units.
// * ctx 512: split at 64 ahead up to 64 units (1 unit 7.96 -> 6.87, 64 units
//   8.18 -> 7.82); whole ahead from 128 units (128 units 9.01 vs 9.98).
// * ctx 1024-4096 with 8-64 units: the best partition gives about 512
//   work-groups (1024 keys x 8 units: 256-key parts 9.69, 64-key 7.30; 1024
//   x 64: 11.61 -> 9.93 at 128; 2048 x 32: 11.56 -> 10.48 at 128); the
//   earlier plan took at least 256 keys for a target of 1024 work-groups.
DecodePlan make_decode_plan(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                            int64_t block_size, int64_t table_width, int64_t requested) {
    DecodePlan p{};
    const int64_t group = q_heads / kv_heads;
    p.gtile = group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    const int64_t tile = decode_tile_tokens(head_dim);
    const int64_t cap = table_width * block_size;
    const int64_t units = batch * kv_heads * (group / p.gtile);
    const int64_t split_step = tile * kSplitWaves;
    const int64_t whole_step = tile * 16;  // the capacity unit the thresholds below were measured in
    int64_t part;
    const bool whole = units >= kDeviceCUs - kDeviceCUs / 16 || cap <= whole_step ||
                       (cap <= 2 * whole_step && units > kDeviceCUs / 4);
    if (requested <= 0 && whole) {
        // Below two whole steps (512 tokens at D=128): 8 waves (a 128-token
        // context in one iteration of loads) while the units fit the CUs, 4
        // beyond (more work-groups per CU).  µs per call: B1 / ctx 128 fp16 4.85 -> 4.77,
        // B4 / ctx 256 6.82 -> 6.00, B32 / ctx 256 bf16 8.76 -> 7.32; but
        // B64 / ctx 128 7.18 -> 7.39 (512 units), hence 4 there.
        const int short_waves = units <= kDeviceCUs ? kWholeWaves : kSplitWaves;
        p.waves = cap < 2 * whole_step ? short_waves : kWholeWaves;
        part = (cap + tile - 1) / tile * tile;
    } else {
        p.waves = kSplitWaves;
        if (requested > 0) {
            part = requested;
        } else {
            constexpr int64_t kTargetGroups = 2 * kDeviceCUs;
            part = (cap * units + kTargetGroups - 1) / kTargetGroups;
        }
        part = (part + split_step - 1) / split_step * split_step;
        const int64_t cap_steps = (cap + split_step - 1) / split_step * split_step;
        if (part > cap_steps) part = cap_steps;
    }
    p.partition = (int)part;
    p.max_parts = (int)((cap + part - 1) / part);
    // Long units (kLongUnitBytes of K+V capacity or more) numbering at most
    // one per CU, or a request (requested == -1), take the balanced walk.
    // With one work-group per unit the CUs holding the shortest units idle
    // while the longest stream alone, whatever the order: 32 sequences of
    // contexts U[1,4096] (fp16, block 256) 70.5 -> 62.5 µs per call, all 4096
    // tokens 84.3 -> 84.6.  Fewer units, which split-K cuts into partitions
    // sized by capacity, leave ragged batches with empty partitions and
    // uneven CUs (bf16, block 16 unless noted, µs per call, split-K ->
    // walk): 24 sequences U[1,4096] 60.8 -> 47.3, 16 U[1,8192] 58.1 -> 46.4,
    // 8 U[1,8192] fp16 block 256 30.1 -> 27.4, 4 U[1,32768] block 256 61.5
    // -> 56.9; equal lengths cost the walk 2-6 % (8 x 4096 26.2 -> 27.7, 1 x
    // 32768 block 256 28.5 -> 29.7) and short capacities more (8 x 512 8.4
    // -> 9.6), so those keep split-K.  With two or more units per CU the
    // longest-first order already balances the CUs, and the walk was slower
    // (64 sequences U[1,4096] sharing a 1024-token prefix, bf16, block 16:
    // 88.1 -> 90.5 µs; 128 sequences U[1,4096]: 166.4 -> 169.2).
    const bool long_units = (double)cap * (double)head_dim * 4.0 >= (double)kLongUnitBytes;
    const bool flat = batch <= kLptMax &&
                      (requested == -1 || (requested <= 0 && long_units && units <= kDeviceCUs));
    if (flat) {
        p.flat_groups = kFlatGroups;
        p.waves = kFlatWaves;
        p.max_parts = 1;
    }
    // In floating point: the size query runs before any shape check, where the
    // integer product could overflow.  The walk's kernels always load with the
    // non-temporal hint.
    p.stream = flat || (double)batch * (double)cap * (double)kv_heads * (double)head_dim * 4.0 > (double)kStreamBytes;
    return p;
}

template <typename T, int D, int G, int NW, bool STREAM>
void launch_decode_kernel_pro(const DecodeArgs& a, dim3 grid, bool page_uniform, hipStream_t s) {
    if constexpr (decode_fused_capable<D>()) {
        if (a.prologue != 0) {
            launch_decode_fused<T, D, G, NW, STREAM>(a, grid, page_uniform, s);
            return;
        }
    }
    launch_decode_kernel<T, D, G, NW, STREAM, false>(a, grid, page_uniform, s);
}

template <typename T, int D, int G, int NW>
void launch_decode_nw(const DecodeArgs& a, int units, bool page_uniform, bool stream, hipStream_t s) {
    const dim3 grid(a.flat_groups > 0 ? a.flat_groups : units, a.max_parts);
    if (stream) {
        launch_decode_kernel_pro<T, D, G, NW, true>(a, grid, page_uniform, s);
        return;
    }
    launch_decode_kernel_pro<T, D, G, NW, false>(a, grid, page_uniform, s);
}

template <typename T, int D, int G>
void launch_decode(const DecodeArgs& a, const DecodePlan& p, int units, bool page_uniform, hipStream_t s) {
    if (p.waves == kWholeWaves) launch_decode_nw<T, D, G, kWholeWaves>(a, units, page_uniform, p.stream, s);
    else launch_decode_nw<T, D, G, kSplitWaves>(a, units, page_uniform, p.stream, s);
    if (a.flat_groups > 0)
        hipLaunchKernelGGL((paged_decode_flat_merge_kernel<T, D, G>), dim3(a.flat_groups), dim3(kLptMax), 0, s, a);
    else if (a.max_parts > 1)
        hipLaunchKernelGGL((paged_decode_merge_kernel<T, D>), dim3(units / a.kv_heads / a.gtiles * a.q_heads),
                           dim3(merge_threads<D>()), 0, s, a);
}

template <typename T, int D>
void launch_decode_g(const DecodeArgs& a, const DecodePlan& p, int units, bool page_uniform, hipStream_t s) {
    if (p.gtile == 4) launch_decode<T, D, 4>(a, p, units, page_uniform, s);
    else if (p.gtile == 2) launch_decode<T, D, 2>(a, p, units, page_uniform, s);
    else launch_decode<T, D, 1>(a, p, units, page_uniform, s);
}

template <typename T>
void launch_decode_d(const DecodeArgs& a, int64_t head_dim, const DecodePlan& p, int units, bool pu,
                     hipStream_t s) {
    switch (head_dim) {
        case 16: launch_decode_g<T, 16>(a, p, units, pu, s); break;
        case 32: launch_decode_g<T, 32>(a, p, units, pu, s); break;
        case 64: launch_decode_g<T, 64>(a, p, units, pu, s); break;
        case 80: launch_decode_g<T, 80>(a, p, units, pu, s); break;
        case 96: launch_decode_g<T, 96>(a, p, units, pu, s); break;
        case 128: launch_decode_g<T, 128>(a, p, units, pu, s); break;
        case 192: launch_decode_g<T, 192>(a, p, units, pu, s); break;
        case 256: launch_decode_g<T, 256>(a, p, units, pu, s); break;
    }
}

constexpr int64_t kMaxCapacity = 1048576;     // tokens a block table may address
constexpr int64_t kMaxBatchHeads = 2147483647; // batch * q_heads

int check_decode_shapes(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                        int64_t num_blocks, int64_t block_size, int64_t table_width, int dtype) {
    if (!valid_dtype(dtype)) return fail(MVME_EINVAL, "FP16/BF16 required");
    if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || num_blocks <= 0)
        return fail(MVME_EINVAL, "empty batch/heads/cache");
    if (block_size <= 0) return fail(MVME_EINVAL, "block size mismatch");
    if (q_heads % kv_heads != 0) return fail(MVME_EINVAL, "head dimension or GQA mismatch");
    if (decode_tile_tokens(head_dim) == 0)
        return fail(MVME_EINVAL, "supported head_dim: 16,32,64,80,96,128,192,256");
    if (table_width <= 0) return fail(MVME_EINVAL, "invalid block table");
    if (block_size > kMaxCapacity || table_width > kMaxCapacity || table_width * block_size > kMaxCapacity)
        return fail(MVME_EINVAL, "maximum table capacity is 1M tokens");
    if (batch > kMaxBatchHeads || q_heads > kMaxBatchHeads || batch * q_heads > kMaxBatchHeads)
        return fail(MVME_EINVAL, "batch/head product too large");
    return MVME_OK;
}

}  // namespace
}  // namespace mvme

using namespace mvme;

extern "C" size_t mvme_paged_attention_workspace_size(int64_t batch, int64_t q_heads, int64_t kv_heads,
                                                      int64_t head_dim, int64_t block_size,
                                                      int64_t table_width, int64_t partition_tokens) {
    if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0 || block_size <= 0 ||
        table_width <= 0 || decode_tile_tokens(head_dim) == 0)
        return 0;
    // The limits mvme_paged_attention enforces; inside them every product of
    // the plan fits its type.
    if (block_size > kMaxCapacity || table_width > kMaxCapacity || table_width * block_size > kMaxCapacity ||
        batch > kMaxBatchHeads || q_heads > kMaxBatchHeads || batch * q_heads > kMaxBatchHeads)
        return 0;
    const DecodePlan p = make_decode_plan(batch, q_heads, kv_heads, head_dim, block_size, table_width,
                                          partition_tokens);
    if (p.flat_groups > 0)
        return (size_t)p.flat_groups * 2 * p.gtile * (head_dim + 2) * sizeof(float) +
               (size_t)p.flat_groups * sizeof(FlatMergeDesc);
    if (p.max_parts <= 1) return 0;
    return (size_t)batch * q_heads * p.max_parts * (head_dim + 2) * sizeof(float);
}

namespace mvme {
namespace {

// The fused prologue's inputs (mode 0: none).
struct DecodePrologue {
    int mode;
    const void* new_k;
    const void* new_v;
    int64_t k_stride, v_stride, q_stride;
    const void* q_weight;
    const void* k_weight;
    const void* cos;
    const void* sin;
    void* q_out;
    float eps;
};

// Shapes checked, workspace sized: plan the call and launch its kernels.
int launch_paged_attention(void* out, const void* query, const void* key_cache, const void* value_cache,
                           const int64_t* block_tables, const int64_t* context_lens, int64_t batch,
                           int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t num_blocks,
                           int64_t block_size, int64_t table_width, int64_t partition_tokens, int dtype,
                           size_t need, void* workspace, void* stream, const DecodePrologue* pro = nullptr) {
    const DecodePlan p = make_decode_plan(batch, q_heads, kv_heads, head_dim, block_size, table_width,
                                          partition_tokens);
    const int64_t group = q_heads / kv_heads;
    const int64_t units = batch * kv_heads * (group / p.gtile);
    if (units > 2147483647) return fail(MVME_EINVAL, "batch/head product too large");
    DecodeArgs a{};
    a.out = out;
    a.query = query;
    a.key_cache = key_cache;
    a.value_cache = value_cache;
    a.tables = block_tables;
    a.lens = context_lens;
    if (need > 0) {
        a.ws_acc = static_cast<float*>(workspace);
        a.ws_ml = a.ws_acc + (p.flat_groups > 0 ? (int64_t)p.flat_groups * 2 * p.gtile
                                                 : batch * q_heads * p.max_parts) * head_dim;
        // After the partial rows (a multiple of 16 bytes: 256 shares x 2 x G
        // x (D + 2) floats).
        if (p.flat_groups > 0) {
            if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
                return fail(MVME_EINVAL, "the balanced walk needs a 16-byte aligned workspace");
            a.ws_flat = reinterpret_cast<FlatMergeDesc*>(a.ws_ml + (int64_t)p.flat_groups * 2 * p.gtile * 2);
        }
    }
    a.q_heads = (int)q_heads;
    a.kv_heads = (int)kv_heads;
    a.group = (int)group;
    a.gtiles = (int)(group / p.gtile);
    a.num_blocks = num_blocks;
    a.block_size = (int)block_size;
    a.block_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctzll((unsigned long long)block_size) : -1;
    a.table_width = (int)table_width;
    a.capacity = (int)(table_width * block_size);
    a.partition = p.partition;
    a.max_parts = p.max_parts;
    a.lpt_batch = p.flat_groups == 0 && p.max_parts == 1 && batch >= 2 && batch <= kLptMax ? (int)batch : 0;
    // Two 8-wave work-groups per CU hold every unit at once (units in
    // (CUs, 2 CUs]): pair long sequences with short ones.  Longest first
    // alone put the k-th and the (k + batch/2)-th longest on one CU: 64
    // sequences of contexts U[1,2048] (bf16, block 16) 54.8 -> 47.8 µs.
    a.lpt_pair = a.lpt_batch > 0 && p.waves == kWholeWaves && units > kDeviceCUs && units <= 2 * kDeviceCUs;
    a.flat_groups = p.flat_groups;
    a.batch = (int)batch;
    a.scale_log2 = kLog2e / sqrtf((float)head_dim);
    if (pro && pro->mode != 0) {
        a.prologue = pro->mode;
        a.new_k = static_cast<const uint16_t*>(pro->new_k);
        a.new_v = static_cast<const uint16_t*>(pro->new_v);
        a.k_stride = pro->k_stride;
        a.v_stride = pro->v_stride;
        a.q_stride = pro->q_stride;
        a.q_weight = static_cast<const uint16_t*>(pro->q_weight);
        a.k_weight = static_cast<const uint16_t*>(pro->k_weight);
        a.cos = static_cast<const uint16_t*>(pro->cos);
        a.sin = static_cast<const uint16_t*>(pro->sin);
        a.q_out = static_cast<uint16_t*>(pro->q_out);
        a.eps = pro->eps;
    }
    const bool page_uniform = block_size % decode_tile_tokens(head_dim) == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == MVME_FP16) launch_decode_d<Half>(a, head_dim, p, (int)units, page_uniform, s);
    else launch_decode_d<BFloat16>(a, head_dim, p, (int)units, page_uniform, s);
    return check_launch("paged attention");
}

// Split-K scratch of the allocation-free entry point: one array per device,
// held until the process ends.  The kernels write every partial they later
// read, so nothing in it needs clearing between calls.
constexpr size_t kScratchBytes = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of `scratch` on each device, resolved on the first call made
// with that device current (the host-side name is only a handle).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices] = {};

int device_scratch(void** ptr) {
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices)
        return fail(MVME_ELAUNCH, "paged attention (no-alloc): no usable current HIP device");
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    if (g_scratch_ptr[device] == nullptr) {
        void* address = nullptr;
        const hipError_t err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
        if (err != hipSuccess || address == nullptr)
            return fail(MVME_ELAUNCH, std::string("paged attention (no-alloc): scratch address: ") +
                                          hipGetErrorString(err));
        g_scratch_ptr[device] = address;
    }
    *ptr = g_scratch_ptr[device];
    return MVME_OK;
}

}  // namespace
}  // namespace mvme

extern "C" int mvme_paged_attention(void* out, const void* query, const void* key_cache,
                                    const void* value_cache, const int64_t* block_tables,
                                    const int64_t* context_lens, int64_t batch, int64_t q_heads,
                                    int64_t kv_heads, int64_t head_dim, int64_t num_blocks,
                                    int64_t block_size, int64_t table_width, int64_t partition_tokens,
                                    int dtype, void* workspace, size_t workspace_bytes, void* stream) {
    if (int rc = check_decode_shapes(batch, q_heads, kv_heads, head_dim, num_blocks, block_size,
                                     table_width, dtype))
        return rc;
    if (!out || !query || !key_cache || !value_cache || !block_tables || !context_lens)
        return fail(MVME_EINVAL, "paged attention received a null pointer");
    const size_t need = mvme_paged_attention_workspace_size(batch, q_heads, kv_heads, head_dim, block_size,
                                                            table_width, partition_tokens);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(MVME_EWORKSPACE, "paged attention workspace too small: need " + std::to_string(need) +
                                         " bytes, got " + std::to_string(workspace_bytes));
    return launch_paged_attention(out, query, key_cache, value_cache, block_tables, context_lens, batch,
                                  q_heads, kv_heads, head_dim, num_blocks, block_size, table_width,
                                  partition_tokens, dtype, need, workspace, stream);
}

namespace {
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
}  // namespace

extern "C" int mvme_paged_attention_decode_write(
    void* out, const void* query, void* key_cache, void* value_cache, const int64_t* block_tables,
    const int64_t* context_lens, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
    int64_t num_blocks, int64_t block_size, int64_t table_width, int64_t partition_tokens, int dtype,
    const void* new_key, const void* new_value, int64_t key_token_stride, int64_t value_token_stride,
    const void* q_weight, const void* k_weight, const void* cos, const void* sin, float eps,
    int64_t query_token_stride, void* q_out, void* workspace, size_t workspace_bytes, void* stream) {
    if (int rc = check_decode_shapes(batch, q_heads, kv_heads, head_dim, num_blocks, block_size,
                                     table_width, dtype))
        return rc;
    if (!out || !query || !key_cache || !value_cache || !block_tables || !context_lens || !new_key || !new_value)
        return fail(MVME_EINVAL, "paged decode with KV write received a null pointer");
    if (head_dim != 16 && head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)
        return fail(MVME_EINVAL, "paged decode with KV write supports head_dim 16,32,64,128,256");
    const bool rope = q_weight != nullptr;
    if (rope && (!k_weight || !cos || !sin))
        return fail(MVME_EINVAL, "paged decode with norm/RoPE needs q_weight, k_weight, cos and sin");
    if (rope && (!(eps > 0.f) || !__builtin_isfinite(eps)))
        return fail(MVME_EINVAL, "eps must be positive, finite and representable in FP32");
    if (key_token_stride < kv_heads * head_dim || value_token_stride < kv_heads * head_dim ||
        (rope && query_token_stride < q_heads * head_dim))
        return fail(MVME_EINVAL, "Q/K/V token stride smaller than a row");
    const bool aligned = aligned16(query) && aligned16(key_cache) && aligned16(value_cache) &&
                         aligned16(new_key) && aligned16(new_value) && key_token_stride % 8 == 0 &&
                         value_token_stride % 8 == 0 &&
                         (!rope || (aligned16(q_weight) && aligned16(k_weight) && aligned16(cos) &&
                                    aligned16(sin) && query_token_stride % 8 == 0 &&
                                    (q_out == nullptr || aligned16(q_out))));
    if (!aligned) return fail(MVME_EINVAL, "paged decode with KV write needs 16-byte aligned rows");
    if (rope && q_out != nullptr) {
        // Every wave (and every split-K partition) reads the raw query rows
        // while the first partition writes the rotated rows to q_out, so the
        // two byte ranges must be disjoint (an in-place rotation belongs to
        // the two-launch sequence).
        const uintptr_t q_lo = reinterpret_cast<uintptr_t>(query);
        const uintptr_t q_hi = q_lo + (uintptr_t)(((batch - 1) * query_token_stride + q_heads * head_dim) * 2);
        const uintptr_t o_lo = reinterpret_cast<uintptr_t>(q_out);
        const uintptr_t o_hi = o_lo + (uintptr_t)(batch * q_heads * head_dim * 2);
        if (o_lo < q_hi && q_lo < o_hi)
            return fail(MVME_EINVAL, "q_out must not overlap the raw query rows");
    }
    const size_t need = mvme_paged_attention_workspace_size(batch, q_heads, kv_heads, head_dim, block_size,
                                                            table_width, partition_tokens);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(MVME_EWORKSPACE, "paged attention workspace too small: need " + std::to_string(need) +
                                         " bytes, got " + std::to_string(workspace_bytes));
    DecodePrologue pro{};
    pro.mode = rope ? 2 : 1;
    pro.new_k = new_key;
    pro.new_v = new_value;
    pro.k_stride = key_token_stride;
    pro.v_stride = value_token_stride;
    pro.q_stride = rope ? query_token_stride : q_heads * head_dim;
    pro.q_weight = q_weight;
    pro.k_weight = k_weight;
    pro.cos = cos;
    pro.sin = sin;
    pro.q_out = rope ? q_out : nullptr;
    pro.eps = eps;
    return launch_paged_attention(out, query, key_cache, value_cache, block_tables, context_lens, batch,
                                  q_heads, kv_heads, head_dim, num_blocks, block_size, table_width,
                                  partition_tokens, dtype, need, workspace, stream, &pro);
}

extern "C" int mvme_paged_attention_noalloc(void* out, const void* query, const void* key_cache,
                                            const void* value_cache, const int64_t* block_tables,
                                            const int64_t* context_lens, int64_t batch, int64_t q_heads,
                                            int64_t kv_heads, int64_t head_dim, int64_t num_blocks,
                                            int64_t block_size, int64_t table_width, int64_t partition_tokens,
                                            int dtype, void* stream) {
    if (int rc = check_decode_shapes(batch, q_heads, kv_heads, head_dim, num_blocks, block_size,
                                     table_width, dtype))
        return rc;
    if (!out || !query || !key_cache || !value_cache || !block_tables || !context_lens)
        return fail(MVME_EINVAL, "paged attention received a null pointer");
    const size_t need = mvme_paged_attention_workspace_size(batch, q_heads, kv_heads, head_dim, block_size,
                                                            table_width, partition_tokens);
    if (need > kScratchBytes)
        return fail(MVME_EWORKSPACE, "paged attention (no-alloc) needs " + std::to_string(need) +
                                         " bytes of split-K scratch, above its fixed " +
                                         std::to_string(kScratchBytes) + "; use mvme_paged_attention");
    void* workspace = nullptr;
    if (need > 0)
        if (int rc = device_scratch(&workspace)) return rc;
    return launch_paged_attention(out, query, key_cache, value_cache, block_tables, context_lens, batch,
                                  q_heads, kv_heads, head_dim, num_blocks, block_size, table_width,
                                  partition_tokens, dtype, need, workspace, stream);
}

// GQA paged decode attention for gfx950.
//
// Work decomposition: one work-group of NW waves per
// (sequence, kv head, G-query-head tile, partition of `partition` tokens).
// All G query heads that share a kv head are served by the same loads, so
// every K/V byte of a partition is fetched from HBM exactly once.  When the
// (sequence, kv head) units alone fill the GPU, a 16-wave work-group covers a
// whole sequence and merges its waves in LDS: one kernel, no workspace.
// Otherwise the context is split into partitions of 4-wave work-groups
// (split-K) whose fp32 partials a second, small kernel merges.
//
// Lane layout inside a wave: a token row of one kv head is head_dim*2 bytes
// = D/8 16-byte chunks; LPT (next power of two >= D/8) consecutive lanes
// cover one token, so one global_load_dwordx4 per lane moves 64/LPT whole
// token rows (1 KiB for D=128: four 256-byte rows).  Each wave issues four
// K loads and four V loads per iteration before touching any of them.
//
// Scores: packed dot2 (fp16/bf16 products, fp32 accumulation) on the lane's
// 8 elements, then a DPP reduction across the LPT lanes of the token.
// Softmax: online, fp32, base-2 exponent with log2(e)/sqrt(D) folded into
// the scale.  Each token group of lanes keeps its own running max/sum/acc;
// groups, then waves (through LDS), are merged at the end.  Sequences that
// fit one partition write the output directly from the attention kernel.
#include <mutex>

#include "mvme_common.h"

namespace mvme {
namespace {

constexpr int kSplitWaves = 4;   // waves per work-group in split-K mode
constexpr int kWholeWaves = 16;  // waves per work-group covering a whole sequence
constexpr int kLptMax = 256;     // largest batch whose units go longest context first
static_assert(kSplitWaves * kWave >= kLptMax, "one thread per sequence key");
constexpr int kDecodeLoads = 4;  // K (and V) loads per lane per iteration

template <int D>
struct DecodeShape {
    static constexpr int kChunks = D / 8;  // 16-byte chunks per token row
    static constexpr int kLpt = kChunks <= 1 ? 1 : kChunks <= 2 ? 2 : kChunks <= 4 ? 4
                              : kChunks <= 8 ? 8 : kChunks <= 16 ? 16 : kChunks <= 32 ? 32 : 64;
    static constexpr int kTpl = kWave / kLpt;          // tokens per load
    static constexpr int kTpi = kTpl * kDecodeLoads;   // tokens per wave iteration
};

struct DecodeArgs {
    void* out;
    const void* query;
    const void* key_cache;
    const void* value_cache;
    const int64_t* tables;
    const int64_t* lens;
    float* ws_acc;  // [batch*q_heads, max_parts, D]
    float* ws_ml;   // [batch*q_heads, max_parts, 2]  (max in log2 units, sum)
    int q_heads;
    int kv_heads;
    int group;      // q_heads / kv_heads
    int gtiles;     // group / G
    int64_t num_blocks;
    int block_size;
    int block_shift;  // log2(block_size) when it is a power of two, else -1
    int table_width;
    int capacity;   // table_width * block_size
    int partition;  // tokens per partition (multiple of the wave tile)
    int max_parts;
    int lpt_batch;  // batch size when units go longest sequence first (<= kLptMax), else 0
    float scale_log2;
};

// K/V rows are read once per call, by one work-group.  When a call's rows
// can exceed the caches (more than 64 MiB of K/V within the tables'
// capacity) the loads carry the non-temporal hint (`nt`), so that streamed
// rows do not displace cache lines that are reused (page tables, the query,
// rows other waves still need): on the 28-layer B32 / ctx 2048 fp16 headline
// step a call went from 49.7 to 45.4 us, the ragged B64 case from 99.7 to
// 93.7 us, and split-K calls of 512 MiB (B1 / ctx 128k, B4 / ctx 32k,
// B16 / ctx 8k, bf16) from 101-106 to 89-94 us.  Smaller calls keep ordinary loads,
// so that their rows can stay cached from one call to the next: with the
// hint a repeated B8 / ctx 512 bf16 call (16 MiB) went from 10.4 to 11.7 us.
template <bool STREAM>
__device__ inline u32x4 kv_load(const uint8_t* p) {
    if constexpr (STREAM) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    else return *reinterpret_cast<const u32x4*>(p);
}

// Number of partitions a sequence of context length `len64` occupies; 0
// tokens still owns partition 0 so that its (zero) output gets written.
__device__ inline int seq_tokens(int64_t len64, int capacity) {
    return (len64 > 0 && len64 <= capacity) ? (int)len64 : 0;
}

template <typename T, int D, int G, bool PAGE_UNIFORM, int NW, bool STREAM>
__global__ __launch_bounds__(NW * kWave) void paged_decode_kernel(DecodeArgs a) {
    using S = DecodeShape<D>;
    constexpr int L = kDecodeLoads;
    constexpr int kStep = S::kTpi * NW;  // tokens per work-group iteration
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int tl = lane / S::kLpt;  // token slot inside one load
    const int c = lane % S::kLpt;   // 16-byte chunk of the token row
    const bool chunk_ok = c < S::kChunks;

    const int unit = blockIdx.x;
    const int part = blockIdx.y;
    const int per_seq = a.kv_heads * a.gtiles;
    int b = unit / per_seq;
    const int r = unit - b * per_seq;
    int len;
    if (a.lpt_batch > kWave) {
        // As below for 64 < batch <= kLptMax: thread s keeps sequence s's key
        // in LDS and counts the larger keys with broadcast reads.
        __shared__ int lpt_keys[kLptMax];
        __shared__ int lpt_pick;
        const int n = a.lpt_batch;
        const int tid = threadIdx.x;
        const int key = tid < n ? (seq_tokens(a.lens[tid], a.capacity) << 8) | (kLptMax - 1 - tid) : -1;
        if (tid < ((n + 3) & ~3)) lpt_keys[tid] = key;  // -1 pads the last group of four
        __syncthreads();
        if (tid < n) {
            int g0 = 0, g1 = 0, g2 = 0, g3 = 0;
            for (int t = 0; t < n; t += 4) {
                const int4 kv = *reinterpret_cast<const int4*>(&lpt_keys[t]);
                g0 += kv.x > key ? 1 : 0;
                g1 += kv.y > key ? 1 : 0;
                g2 += kv.z > key ? 1 : 0;
                g3 += kv.w > key ? 1 : 0;
            }
            if (g0 + g1 + g2 + g3 == b) lpt_pick = tid;
        }
        __syncthreads();
        b = __builtin_amdgcn_readfirstlane(lpt_pick);
        len = lpt_keys[b] >> 8;
    } else if (a.lpt_batch > 0) {
        // Whole-sequence mode (batch <= 64): the k-th group of units takes
        // the sequence with the k-th longest context (ties by index), so the
        // longest sequences start first and the short ones fill the CUs that
        // free up (longest-processing-time-first list scheduling).  Lane s
        // holds a key unique to sequence s; its rank is the number of larger
        // keys.  Equal lengths keep the identity order without the count.
        const int n = a.lpt_batch;
        const int key = lane < n ? (seq_tokens(a.lens[lane], a.capacity) << 6) | (63 - lane) : -1;
        const int len0 = __builtin_amdgcn_readlane(key, 0) >> 6;
        if (__ballot(lane < n && (key >> 6) != len0) != 0) {
            int g0 = 0, g1 = 0, g2 = 0, g3 = 0;
            int t = 0;
            for (; t + 4 <= n; t += 4) {
                g0 += __builtin_amdgcn_readlane(key, t) > key ? 1 : 0;
                g1 += __builtin_amdgcn_readlane(key, t + 1) > key ? 1 : 0;
                g2 += __builtin_amdgcn_readlane(key, t + 2) > key ? 1 : 0;
                g3 += __builtin_amdgcn_readlane(key, t + 3) > key ? 1 : 0;
            }
            for (; t < n; ++t) g0 += __builtin_amdgcn_readlane(key, t) > key ? 1 : 0;
            b = __builtin_ctzll(__ballot(lane < n && g0 + g1 + g2 + g3 == b));
        }
        len = __builtin_amdgcn_readlane(key, b) >> 6;
    } else {
        len = seq_tokens(a.lens[b], a.capacity);
    }
    const int kvh = r / a.gtiles;
    const int h0 = kvh * a.group + (r - kvh * a.gtiles) * G;

    const int nparts = len > 0 ? (len + a.partition - 1) / a.partition : 1;
    if (part >= nparts) return;
    const int start = part * a.partition;
    const int end = min(start + a.partition, len);

    // Query slice of this lane for every head of the tile (8 elements each).
    uint32_t q[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        u32x4 w = {0u, 0u, 0u, 0u};
        if (chunk_ok)
            w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.query) +
                                                ((int64_t)b * a.q_heads + h0 + g) * D + 8 * c);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[g][i] = w[i];
    }

    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = kNegInf;
        l[g] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
    }

    const int64_t row_elems = (int64_t)a.kv_heads * D;
    const int64_t page_elems = (int64_t)a.block_size * row_elems;
    const uint16_t* kbase = static_cast<const uint16_t*>(a.key_cache) + kvh * D + 8 * c;
    const uint16_t* vbase = static_cast<const uint16_t*>(a.value_cache) + kvh * D + 8 * c;
    const int64_t* table = a.tables + (int64_t)b * a.table_width;

    // Page-uniform iterations: the iteration's tokens lie in one page, whose
    // id is a scalar load issued one iteration ahead (its latency hides
    // behind the current iteration); the loads are a scalar page base plus
    // 32-bit per-lane offsets, with no per-load branches.
    typedef __attribute__((address_space(4))) const int64_t const_i64;
    const const_i64* ctable = (const const_i64*)table;
    const int row_bytes = (int)(row_elems * 2);
    uint32_t lane_off[L];
#pragma unroll
    for (int u = 0; u < L; ++u) lane_off[u] = (uint32_t)((u * S::kTpl + tl) * row_bytes + (kvh * D + 8 * c) * 2);
    auto page_of = [&](int t) __attribute__((always_inline)) -> int64_t {
        if (t >= end) return -1;
        return ctable[a.block_shift >= 0 ? t >> a.block_shift : t / a.block_size];
    };
    int it = __builtin_amdgcn_readfirstlane(start + wave * S::kTpi);
    int64_t page_next = 0;
    if constexpr (PAGE_UNIFORM) page_next = page_of(it);
    for (; it < end; it += kStep) {
        u32x4 kk[L], vv[L];
        bool ok[L];
        if constexpr (PAGE_UNIFORM) {
            const int64_t page = page_next;
            page_next = page_of(it + kStep);
            const bool page_ok = page >= 0 && page < a.num_blocks;
            const int in_page = a.block_shift >= 0 ? it & (a.block_size - 1) : it % a.block_size;
#pragma unroll
            for (int u = 0; u < L; ++u) {
                ok[u] = page_ok && it + u * S::kTpl + tl < end;
                kk[u] = vv[u] = u32x4{0u, 0u, 0u, 0u};
            }
            if (page_ok) {  // wave-uniform
                const int64_t base = (page * a.block_size + in_page) * (int64_t)row_bytes;
                const uint8_t* kp = static_cast<const uint8_t*>(a.key_cache) + base;
                const uint8_t* vp = static_cast<const uint8_t*>(a.value_cache) + base;
#pragma unroll
                for (int u = 0; u < L; ++u) {
                    // In-page rows past the context are loaded (in bounds) and zeroed below.
                    if constexpr (S::kChunks == S::kLpt) {
                        kk[u] = kv_load<STREAM>(kp + lane_off[u]);
                        vv[u] = kv_load<STREAM>(vp + lane_off[u]);
                    } else if (chunk_ok) {
                        kk[u] = kv_load<STREAM>(kp + lane_off[u]);
                        vv[u] = kv_load<STREAM>(vp + lane_off[u]);
                    }
                }
#pragma unroll
                for (int u = 0; u < L; ++u)
                    if (!ok[u]) vv[u] = u32x4{0u, 0u, 0u, 0u};  // 0 * (stale NaN) must not reach acc
            }
        } else {
#pragma unroll
            for (int u = 0; u < L; ++u) {
                const int t = it + u * S::kTpl + tl;
                int64_t page = -1;
                if (t < end) page = table[t / a.block_size];
                ok[u] = page >= 0 && page < a.num_blocks;
                const int64_t off = page * page_elems + (int64_t)(t % a.block_size) * row_elems;
                kk[u] = vv[u] = u32x4{0u, 0u, 0u, 0u};
                if (ok[u] && chunk_ok) {
                    kk[u] = kv_load<STREAM>(reinterpret_cast<const uint8_t*>(kbase + off));
                    vv[u] = kv_load<STREAM>(reinterpret_cast<const uint8_t*>(vbase + off));
                }
            }
        }

#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s[L];
#pragma unroll
            for (int u = 0; u < L; ++u) {
                float d = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) d = T::dot2(kk[u][i], q[g][i], d);
                d = group_sum<S::kLpt>(d) * a.scale_log2;
                s[u] = ok[u] ? d : kNegInf;
            }
            float mx = s[0];
#pragma unroll
            for (int u = 1; u < L; ++u) mx = fmaxf(mx, s[u]);
            const float mn = fmaxf(m[g], mx);
            const float ref = mn == kNegInf ? 0.f : mn;
            const float alpha = fast_exp2(m[g] - ref);
            float p[L];
            float psum = 0.f;
#pragma unroll
            for (int u = 0; u < L; ++u) {
                p[u] = fast_exp2(s[u] - ref);
                psum += p[u];
            }
            l[g] = l[g] * alpha + psum;
            m[g] = mn;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[g][i] *= alpha;
#pragma unroll
            for (int u = 0; u < L; ++u) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[g][2 * i] = fmaf(p[u], T::lo(vv[u][i]), acc[g][2 * i]);
                    acc[g][2 * i + 1] = fmaf(p[u], T::hi(vv[u][i]), acc[g][2 * i + 1]);
                }
            }
        }
    }

    // Merge the token groups of this wave (lanes with equal chunk index).
#pragma unroll
    for (int mask = S::kLpt; mask < kWave; mask <<= 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mo = shfl_xor(m[g], mask);
            const float lo = shfl_xor(l[g], mask);
            const float mn = fmaxf(m[g], mo);
            const float ref = mn == kNegInf ? 0.f : mn;
            const float a1 = fast_exp2(m[g] - ref);
            const float a2 = fast_exp2(mo - ref);
            l[g] = l[g] * a1 + lo * a2;
            m[g] = mn;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float ao = shfl_xor(acc[g][i], mask);
                acc[g][i] = acc[g][i] * a1 + ao * a2;
            }
        }
    }

    // Merge the waves through LDS.
    __shared__ float sm_acc[NW][G][D];
    __shared__ float sm_ml[NW][G][2];
    if (tl == 0 && chunk_ok) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int i = 0; i < 8; ++i) sm_acc[wave][g][8 * c + i] = acc[g][i];
            if (c == 0) {
                sm_ml[wave][g][0] = m[g];
                sm_ml[wave][g][1] = l[g];
            }
        }
    }
    __syncthreads();

    for (int idx = threadIdx.x; idx < G * D; idx += NW * kWave) {
        const int g = idx / D;
        const int d = idx - g * D;
        float mx = sm_ml[0][g][0];
#pragma unroll
        for (int w = 1; w < NW; ++w) mx = fmaxf(mx, sm_ml[w][g][0]);
        const float ref = mx == kNegInf ? 0.f : mx;
        float sum = 0.f, o = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float f = fast_exp2(sm_ml[w][g][0] - ref);
            sum += sm_ml[w][g][1] * f;
            o += sm_acc[w][g][d] * f;
        }
        const int64_t bh = (int64_t)b * a.q_heads + h0 + g;
        if (nparts == 1) {
            static_cast<uint16_t*>(a.out)[bh * D + d] = T::from_float(sum > 0.f ? o / sum : 0.f);
        } else {
            const int64_t row = bh * a.max_parts + part;
            a.ws_acc[row * D + d] = o;
            if (d == 0) {
                a.ws_ml[row * 2] = mx;
                a.ws_ml[row * 2 + 1] = sum;
            }
        }
    }
}

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

struct DecodePlan {
    int partition;
    int max_parts;
    int gtile;  // G of the kernel instance
    int waves;  // waves per work-group (kSplitWaves or kWholeWaves)
    bool stream;  // non-temporal K/V loads
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
// capacity only).  Enough (sequence, kv head) units to occupy every CU, or a
// short capacity: one work-group per unit over the whole context, merged in
// LDS.  Otherwise split-K into partitions of 4-wave work-groups, sized to
// give every CU about four work-groups, plus a merge kernel.  `requested` > 0
// forces split-K with that partition length (rounded to the wave tiling).
DecodePlan make_decode_plan(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                            int64_t block_size, int64_t table_width, int64_t requested) {
    DecodePlan p{};
    const int64_t group = q_heads / kv_heads;
    p.gtile = group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    const int64_t tile = decode_tile_tokens(head_dim);
    const int64_t cap = table_width * block_size;
    const int64_t units = batch * kv_heads * (group / p.gtile);
    const int64_t split_step = tile * kSplitWaves;
    const int64_t whole_step = tile * kWholeWaves;
    int64_t part;
    if (requested <= 0 && (units >= kDeviceCUs - kDeviceCUs / 16 || cap <= 2 * whole_step)) {
        // Whole-sequence work-groups; also when the capacity is at most two
        // 16-wave steps (launch- and latency-bound, a merge would only add a
        // launch).  Longer contexts with few units split instead, so that a
        // few work-groups do not each walk a long context alone.
        p.waves = cap >= 2 * whole_step ? kWholeWaves : kSplitWaves;
        part = (cap + tile - 1) / tile * tile;
    } else {
        p.waves = kSplitWaves;
        if (requested > 0) {
            part = requested;
        } else {
            constexpr int64_t kTargetGroups = 4 * kDeviceCUs;
            part = (cap * units + kTargetGroups - 1) / kTargetGroups;
            if (part < 256) part = 256;  // short partitions only add merge traffic
        }
        part = (part + split_step - 1) / split_step * split_step;
        const int64_t cap_steps = (cap + split_step - 1) / split_step * split_step;
        if (part > cap_steps) part = cap_steps;
    }
    p.partition = (int)part;
    p.max_parts = (int)((cap + part - 1) / part);
    // In floating point: the size query runs before any shape check, where the
    // integer product could overflow.
    p.stream = (double)batch * (double)cap * (double)kv_heads * (double)head_dim * 4.0 > (double)kStreamBytes;
    return p;
}

template <typename T, int D, int G, int NW, bool STREAM>
void launch_decode_kernel(const DecodeArgs& a, dim3 grid, bool page_uniform, hipStream_t s) {
    if (page_uniform)
        hipLaunchKernelGGL((paged_decode_kernel<T, D, G, true, NW, STREAM>), grid, dim3(NW * kWave), 0, s, a);
    else
        hipLaunchKernelGGL((paged_decode_kernel<T, D, G, false, NW, STREAM>), grid, dim3(NW * kWave), 0, s, a);
}

template <typename T, int D, int G, int NW>
void launch_decode_nw(const DecodeArgs& a, int units, bool page_uniform, bool stream, hipStream_t s) {
    const dim3 grid(units, a.max_parts);
    if (stream) {
        launch_decode_kernel<T, D, G, NW, true>(a, grid, page_uniform, s);
        return;
    }
    launch_decode_kernel<T, D, G, NW, false>(a, grid, page_uniform, s);
}

template <typename T, int D, int G>
void launch_decode(const DecodeArgs& a, const DecodePlan& p, int units, bool page_uniform, hipStream_t s) {
    if (p.waves == kWholeWaves) launch_decode_nw<T, D, G, kWholeWaves>(a, units, page_uniform, p.stream, s);
    else launch_decode_nw<T, D, G, kSplitWaves>(a, units, page_uniform, p.stream, s);
    if (a.max_parts > 1)
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
    if (p.max_parts <= 1) return 0;
    return (size_t)batch * q_heads * p.max_parts * (head_dim + 2) * sizeof(float);
}

namespace mvme {
namespace {

// Shapes checked, workspace sized: plan the call and launch its kernels.
int launch_paged_attention(void* out, const void* query, const void* key_cache, const void* value_cache,
                           const int64_t* block_tables, const int64_t* context_lens, int64_t batch,
                           int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t num_blocks,
                           int64_t block_size, int64_t table_width, int64_t partition_tokens, int dtype,
                           size_t need, void* workspace, void* stream) {
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
        a.ws_ml = a.ws_acc + batch * q_heads * p.max_parts * head_dim;
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
    a.lpt_batch = p.max_parts == 1 && batch >= 2 && batch <= kLptMax ? (int)batch : 0;
    a.scale_log2 = kLog2e / sqrtf((float)head_dim);
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

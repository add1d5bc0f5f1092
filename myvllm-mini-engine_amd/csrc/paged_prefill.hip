// Ragged chunked paged prefill for gfx950.
//
// Packed queries q[T, Hq, D]; sequence s owns packed rows
// [cu[s], cu[s+1]), row i of s sits at absolute position starts[s] + i and
// attends keys [0, starts[s] + i] of s through its block table.
//
// MFMA path (D = 128, G = Hq/Hkv in {1,2,4,8,16}):
//   One work-group (4 waves) per (sequence, kv head, block of 64/G query
//   tokens): 64 query rows = (token, head-of-group) pairs that share every
//   K/V tile.  Wave w owns rows 16w..16w+15.  K/V tiles of 64 keys are
//   gathered from the pages into LDS (K row-major, V transposed), the next
//   tile's global loads are in flight while the current tile is multiplied.
//
//   Scores are computed transposed, S^T = K Q^T (v_mfma_f32_16x16x32), so
//   that each lane ends up holding 16 scores of ONE query row: the online
//   softmax needs only two cross-lane max exchanges per tile, and the
//   probabilities are already in the B-operand layout of O^T = V^T P^T
//   (keys are assigned to MFMA k-slots by a fixed permutation applied to
//   both operands).  Accumulation, softmax and normalisation are fp32.
//
// Generic path (any D <= 1024, any G): one wave per (query row, head),
// online softmax over 64-key tiles, fp32 throughout.
#include "mvme_common.h"

namespace mvme {
namespace {

constexpr int kPfWaves = 4;
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kPfRows = 64;    // query rows per work-group
constexpr int kPfKeys = 64;    // keys per LDS tile
constexpr int kPfD = 128;
constexpr int kKStride = 136;  // K tile row stride in elements (272 B, 16 B aligned)
constexpr int kVStride = 68;   // V^T tile row stride in elements (136 B = 34 dwords)

struct PrefillArgs {
    void* out;
    const void* q;
    const void* key_cache;
    const void* value_cache;
    const int64_t* cu;
    const int64_t* starts;
    const int64_t* tables;
    const int64_t* lens;
    int num_seqs;
    int q_heads;
    int kv_heads;
    int group;
    int qb;  // query tokens per work-group (kPfRows / group)
    int head_dim;
    int64_t num_blocks;
    int block_size;
    int table_width;
    float scale_log2;
};

// Locate (sequence, first query token) of query block `blk`, counting
// ceil(rows/qb) blocks per sequence in order.  Returns false past the end.
__device__ inline bool find_block(const PrefillArgs& a, int blk, int& seq, int& q0) {
    int rem = blk;
    for (int s = 0; s < a.num_seqs; ++s) {
        const int64_t n = a.cu[s + 1] - a.cu[s];
        const int nb = n > 0 ? (int)((n + a.qb - 1) / a.qb) : 0;
        if (rem < nb) {
            seq = s;
            q0 = rem * a.qb;
            return true;
        }
        rem -= nb;
    }
    return false;
}

template <typename T>
__global__ __launch_bounds__(kPfThreads) void paged_prefill_mfma_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t sm_k[kPfKeys * kKStride];
    __shared__ __attribute__((aligned(16))) uint16_t sm_vt[kPfD * kVStride];
    __shared__ __attribute__((aligned(16))) float sm_bias[kPfKeys];

    int seq, q0;
    if (!find_block(a, blockIdx.x, seq, q0)) return;
    const int kvh = blockIdx.y;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int li = lane & 15;  // MFMA column / row index
    const int lg = lane >> 4;  // MFMA k-group (0..3)

    const int64_t row0 = a.cu[seq];
    const int qlen = (int)(a.cu[seq + 1] - row0);
    const int64_t start = a.starts[seq];
    const int64_t ctx = a.lens[seq];
    const int64_t cap = (int64_t)a.table_width * a.block_size;
    const int64_t* table = a.tables + (int64_t)seq * a.table_width;

    // This lane's query row.
    const int r = wave * 16 + li;
    const int qi = q0 + r % a.qb;
    const int head = kvh * a.group + r / a.qb;
    const int64_t pos = start + qi;
    const bool row_ok = qi < qlen && start >= 0 && pos < ctx && pos < cap;

    // Keys needed by the block: [0, kv_end).
    const int last_qi = min(q0 + a.qb, qlen) - 1;
    int64_t kv_end = start + last_qi + 1;
    if (kv_end > ctx) kv_end = ctx;
    if (kv_end > cap) kv_end = cap;
    const int ntiles = kv_end > 0 ? (int)((kv_end + kPfKeys - 1) / kPfKeys) : 0;

    // Q^T operand: lane holds row r, d = 32*dc + 8*lg .. +8.
    u32x4 qop[4];
    {
        const uint16_t* qrow = static_cast<const uint16_t*>(a.q) + ((row0 + qi) * a.q_heads + head) * kPfD;
#pragma unroll
        for (int dc = 0; dc < 4; ++dc) {
            qop[dc] = u32x4{0u, 0u, 0u, 0u};
            if (row_ok) qop[dc] = *reinterpret_cast<const u32x4*>(qrow + 32 * dc + 8 * lg);
        }
    }

    float m_run = kNegInf, l_part = 0.f;
    f32x4 o[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Tile loader mapping: load j of lane -> key 16*wave + li, chunk 4*j + lg.
    const int64_t row_elems = (int64_t)a.kv_heads * kPfD;
    const uint16_t* kcache = static_cast<const uint16_t*>(a.key_cache) + kvh * kPfD;
    const uint16_t* vcache = static_cast<const uint16_t*>(a.value_cache) + kvh * kPfD;
    const int ld_key = 16 * wave + li;
    u32x4 pk[4], pv[4];
    bool pvalid = false;

    auto load_tile = [&](int tile) {
        const int64_t key = (int64_t)tile * kPfKeys + ld_key;
        int64_t page = -1;
        if (key < kv_end) page = table[key / a.block_size];
        pvalid = page >= 0 && page < a.num_blocks;
        const int64_t off = (page * a.block_size + key % a.block_size) * row_elems;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            pk[j] = pv[j] = u32x4{0u, 0u, 0u, 0u};
            if (pvalid) {
                pk[j] = *reinterpret_cast<const u32x4*>(kcache + off + 8 * (4 * j + lg));
                pv[j] = *reinterpret_cast<const u32x4*>(vcache + off + 8 * (4 * j + lg));
            }
        }
    };

    auto store_tile = [&]() {
        // K row-major.
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<u32x4*>(&sm_k[ld_key * kKStride + 8 * (4 * j + lg)]) = pk[j];
        // V transposed: lanes li, li^1 hold keys 2m, 2m+1 of the same chunk;
        // exchange half a chunk so each lane writes (V[2m][d], V[2m+1][d])
        // dwords for 4 of the chunk's 8 dims.
        const bool odd = li & 1;
        const int kpair = ld_key & ~1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // Even lane keeps dims 0..3 (dwords 0,1) and sends dwords 2,3.
            const uint32_t send0 = odd ? pv[j][0] : pv[j][2];
            const uint32_t send1 = odd ? pv[j][1] : pv[j][3];
            const uint32_t keep0 = odd ? pv[j][2] : pv[j][0];
            const uint32_t keep1 = odd ? pv[j][3] : pv[j][1];
            const uint32_t recv0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)send0, kDppQuadSwap1, 0xf, 0xf, false);
            const uint32_t recv1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)send1, kDppQuadSwap1, 0xf, 0xf, false);
            // mine/partner words hold dims (2e, 2e+1) of keys kpair+odd / kpair+!odd.
            const uint32_t e_lo0 = odd ? recv0 : keep0;  // key 2m, dims base+0,1
            const uint32_t e_lo1 = odd ? recv1 : keep1;  // key 2m, dims base+2,3
            const uint32_t e_hi0 = odd ? keep0 : recv0;  // key 2m+1, dims base+0,1
            const uint32_t e_hi1 = odd ? keep1 : recv1;  // key 2m+1, dims base+2,3
            const int dbase = 8 * (4 * j + lg) + (odd ? 4 : 0);
            const uint32_t w0 = (e_lo0 & 0xffffu) | (e_hi0 << 16);
            const uint32_t w1 = (e_lo0 >> 16) | (e_hi0 & 0xffff0000u);
            const uint32_t w2 = (e_lo1 & 0xffffu) | (e_hi1 << 16);
            const uint32_t w3 = (e_lo1 >> 16) | (e_hi1 & 0xffff0000u);
            *reinterpret_cast<uint32_t*>(&sm_vt[(dbase + 0) * kVStride + kpair]) = w0;
            *reinterpret_cast<uint32_t*>(&sm_vt[(dbase + 1) * kVStride + kpair]) = w1;
            *reinterpret_cast<uint32_t*>(&sm_vt[(dbase + 2) * kVStride + kpair]) = w2;
            *reinterpret_cast<uint32_t*>(&sm_vt[(dbase + 3) * kVStride + kpair]) = w3;
        }
        if (lg == 0) sm_bias[ld_key] = pvalid ? 0.f : kNegInf;
    };

    if (ntiles > 0) load_tile(0);
    for (int tile = 0; tile < ntiles; ++tile) {
        __syncthreads();  // previous tile fully consumed
        store_tile();
        __syncthreads();
        if (tile + 1 < ntiles) load_tile(tile + 1);

        // S^T = K Q^T for the 4 key sub-tiles of 16.
        f32x4 s[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int dc = 0; dc < 4; ++dc) {
                const u32x4 kop = *reinterpret_cast<const u32x4*>(&sm_k[(16 * kt + li) * kKStride + 32 * dc + 8 * lg]);
                s[kt] = T::mfma16x16x32(kop, qop[dc], s[kt]);
            }
        }

        // Online softmax for this lane's row over its 16 keys.
        const int64_t tile0 = (int64_t)tile * kPfKeys;
        float mx = kNegInf;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            const f32x4 bias = *reinterpret_cast<const f32x4*>(&sm_bias[16 * kt + 4 * lg]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t key = tile0 + 16 * kt + 4 * lg + j;
                float v = s[kt][j] * a.scale_log2 + bias[j];
                if (!row_ok || key > pos) v = kNegInf;
                s[kt][j] = v;
                mx = fmaxf(mx, v);
            }
        }
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        const float mn = fmaxf(m_run, mx);
        const float ref = mn == kNegInf ? 0.f : mn;
        const float alpha = fast_exp2(m_run - ref);
        m_run = mn;
        float psum = 0.f;
        uint32_t pp[8];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            float p[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                p[j] = fast_exp2(s[kt][j] - ref);
                psum += p[j];
            }
            pp[2 * kt] = T::pack(p[0], p[1]);
            pp[2 * kt + 1] = T::pack(p[2], p[3]);
        }
        l_part = l_part * alpha + psum;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;

        // O^T += V^T P^T over two 32-key chunks.
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const u32x4 pop = {pp[4 * c], pp[4 * c + 1], pp[4 * c + 2], pp[4 * c + 3]};
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
                const uint16_t* vrow = &sm_vt[(16 * dt + li) * kVStride + 32 * c + 4 * lg];
                const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
                const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 16);
                const u32x4 vop = {lo[0], lo[1], hi[0], hi[1]};
                o[dt] = T::mfma16x16x32(vop, pop, o[dt]);
            }
        }
    }

    // Row sum across the four k-groups holding this row's keys.
    float l_row = l_part + shfl_xor(l_part, 16);
    l_row += shfl_xor(l_row, 32);
    if (qi >= qlen) return;
    const float inv = (row_ok && l_row > 0.f) ? 1.f / l_row : 0.f;
    uint16_t* orow = static_cast<uint16_t*>(a.out) + ((row0 + qi) * a.q_heads + head) * kPfD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
        const u32x2 w = {T::pack(o[dt][0] * inv, o[dt][1] * inv), T::pack(o[dt][2] * inv, o[dt][3] * inv)};
        *reinterpret_cast<u32x2*>(orow + 16 * dt + 4 * lg) = w;
    }
}

// ---------------------------------------------------------------------------
// Generic path: one wave per (packed query row, query head).
// ---------------------------------------------------------------------------
constexpr int kGenMaxD = 1024;

template <typename T>
__device__ inline float elem_to_float(uint16_t h) {
    return T::lo((uint32_t)h);
}

template <typename T>
__global__ __launch_bounds__(kWave) void paged_prefill_generic_kernel(PrefillArgs a) {
    __shared__ float sm_q[kGenMaxD];
    __shared__ float sm_p[kWave];
    __shared__ int64_t sm_off[kWave];
    const int64_t token = blockIdx.x;
    const int head = blockIdx.y;
    const int lane = threadIdx.x;
    const int D = a.head_dim;
    uint16_t* orow = static_cast<uint16_t*>(a.out) + (token * a.q_heads + head) * D;

    // Sequence owning this packed row (cu is monotone).
    int lo = 0, hi = a.num_seqs;
    while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (a.cu[mid + 1] <= token) lo = mid + 1;
        else hi = mid;
    }
    bool ok = lo < a.num_seqs && token >= a.cu[lo];
    int64_t pos = 0;
    const int64_t cap = (int64_t)a.table_width * a.block_size;
    if (ok) {
        pos = a.starts[lo] + token - a.cu[lo];
        ok = a.starts[lo] >= 0 && pos < a.lens[lo] && pos < cap;
    }
    if (!ok) {
        for (int d = lane; d < D; d += kWave) orow[d] = 0;
        return;
    }
    const int kvh = head / a.group;
    const int64_t* table = a.tables + (int64_t)lo * a.table_width;
    const int64_t row_elems = (int64_t)a.kv_heads * D;
    const uint16_t* qrow = static_cast<const uint16_t*>(a.q) + (token * a.q_heads + head) * D;
    for (int d = lane; d < D; d += kWave) sm_q[d] = elem_to_float<T>(qrow[d]);
    __syncthreads();

    constexpr int kPer = kGenMaxD / kWave;
    float acc[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) acc[i] = 0.f;
    float m_run = kNegInf, l_run = 0.f;
    const uint16_t* kcache = static_cast<const uint16_t*>(a.key_cache) + (int64_t)kvh * D;
    const uint16_t* vcache = static_cast<const uint16_t*>(a.value_cache) + (int64_t)kvh * D;

    for (int64_t k0 = 0; k0 <= pos; k0 += kWave) {
        const int64_t key = k0 + lane;
        int64_t page = -1;
        if (key <= pos) page = table[key / a.block_size];
        const bool kv_ok = page >= 0 && page < a.num_blocks;
        const int64_t off = kv_ok ? (page * a.block_size + key % a.block_size) * row_elems : -1;
        float s = kNegInf;
        if (kv_ok) {
            const uint16_t* krow = kcache + off;
            float d = 0.f;
            for (int e = 0; e < D; ++e) d = fmaf(sm_q[e], elem_to_float<T>(krow[e]), d);
            s = d * a.scale_log2;
        }
        float mx = s;
#pragma unroll
        for (int mask = 1; mask < kWave; mask <<= 1) mx = fmaxf(mx, shfl_xor(mx, mask));
        const float mn = fmaxf(m_run, mx);
        const float ref = mn == kNegInf ? 0.f : mn;
        const float alpha = fast_exp2(m_run - ref);
        const float p = fast_exp2(s - ref);
        float ps = p;
#pragma unroll
        for (int mask = 1; mask < kWave; mask <<= 1) ps += shfl_xor(ps, mask);
        l_run = l_run * alpha + ps;
        m_run = mn;
        __syncthreads();
        sm_p[lane] = p;
        sm_off[lane] = off;
        __syncthreads();
        const int nk = (int)min<int64_t>(kWave, pos + 1 - k0);
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int d = lane + i * kWave;
            if (d < D) {
                float w = 0.f;
                for (int k = 0; k < nk; ++k) {
                    const int64_t vo = sm_off[k];
                    if (vo >= 0) w = fmaf(sm_p[k], elem_to_float<T>(vcache[vo + d]), w);
                }
                acc[i] = acc[i] * alpha + w;
            }
        }
    }
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int d = lane + i * kWave;
        if (d < D) orow[d] = T::from_float(acc[i] * inv);
    }
}

int check_prefill(int64_t num_seqs, int64_t total_tokens, int64_t q_heads, int64_t kv_heads,
                  int64_t head_dim, int64_t num_blocks, int64_t block_size, int64_t table_width,
                  int dtype) {
    if (!valid_dtype(dtype)) return fail(MVME_EINVAL, "paged prefill requires FP16/BF16");
    if (block_size <= 0 || num_blocks <= 0 || kv_heads <= 0 || head_dim <= 0)
        return fail(MVME_EINVAL, "paged prefill cache/block size mismatch");
    if (q_heads <= 0 || q_heads % kv_heads != 0 || head_dim > kGenMaxD)
        return fail(MVME_EINVAL, "paged prefill GQA/head_dim mismatch (maximum head_dim 1024)");
    if (num_seqs < 0 || total_tokens < 0 || table_width < 0)
        return fail(MVME_EINVAL, "paged prefill metadata shape mismatch");
    if (total_tokens * q_heads > 2147483647) return fail(MVME_EINVAL, "too many paged prefill rows");
    if (num_seqs > 65535 * 16) return fail(MVME_EINVAL, "too many paged prefill sequences");
    return MVME_OK;
}

}  // namespace
}  // namespace mvme

using namespace mvme;

extern "C" int mvme_paged_prefill_attention(void* out, const void* q, const void* key_cache,
                                            const void* value_cache, const int64_t* cu_seqlens_q,
                                            const int64_t* query_starts, const int64_t* block_tables,
                                            const int64_t* context_lens, int64_t num_seqs,
                                            int64_t total_tokens, int64_t q_heads, int64_t kv_heads,
                                            int64_t head_dim, int64_t num_blocks, int64_t block_size,
                                            int64_t table_width, int dtype, void* stream) {
    if (int rc = check_prefill(num_seqs, total_tokens, q_heads, kv_heads, head_dim, num_blocks,
                               block_size, table_width, dtype))
        return rc;
    if (total_tokens == 0) return MVME_OK;
    if (num_seqs == 0 || table_width == 0) return fail(MVME_EINVAL, "paged prefill metadata shape mismatch");
    if (!out || !q || !key_cache || !value_cache || !cu_seqlens_q || !query_starts || !block_tables ||
        !context_lens)
        return fail(MVME_EINVAL, "paged prefill received a null pointer");
    PrefillArgs a{};
    a.out = out;
    a.q = q;
    a.key_cache = key_cache;
    a.value_cache = value_cache;
    a.cu = cu_seqlens_q;
    a.starts = query_starts;
    a.tables = block_tables;
    a.lens = context_lens;
    a.num_seqs = (int)num_seqs;
    a.q_heads = (int)q_heads;
    a.kv_heads = (int)kv_heads;
    a.group = (int)(q_heads / kv_heads);
    a.head_dim = (int)head_dim;
    a.num_blocks = num_blocks;
    a.block_size = (int)block_size;
    a.table_width = (int)table_width;
    a.scale_log2 = kLog2e / sqrtf((float)head_dim);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool mfma = head_dim == kPfD && kPfRows % a.group == 0 && a.group <= 16;
    if (mfma) {
        a.qb = kPfRows / a.group;
        const int64_t blocks = (total_tokens + a.qb - 1) / a.qb + num_seqs;
        if (blocks > 2147483647 || kv_heads > 65535) return fail(MVME_EINVAL, "paged prefill grid too large");
        const dim3 grid((unsigned)blocks, (unsigned)kv_heads);
        if (dtype == MVME_FP16)
            hipLaunchKernelGGL((paged_prefill_mfma_kernel<Half>), grid, dim3(kPfThreads), 0, s, a);
        else
            hipLaunchKernelGGL((paged_prefill_mfma_kernel<BFloat16>), grid, dim3(kPfThreads), 0, s, a);
    } else {
        if (q_heads > 65535) return fail(MVME_EINVAL, "paged prefill grid too large");
        const dim3 grid((unsigned)total_tokens, (unsigned)q_heads);
        if (dtype == MVME_FP16)
            hipLaunchKernelGGL((paged_prefill_generic_kernel<Half>), grid, dim3(kWave), 0, s, a);
        else
            hipLaunchKernelGGL((paged_prefill_generic_kernel<BFloat16>), grid, dim3(kWave), 0, s, a);
    }
    return check_launch("paged prefill");
}

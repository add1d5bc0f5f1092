// Fused per-head q/k RMSNorm + rotary embedding + KV page write for gfx950.
//
// For every token t (packed rows of one prefill batch, or one row per
// sequence of a decode batch):
//   q_out[t, h]           = rope(rmsnorm(q[t, h], q_weight), cos[t], sin[t])   h < q_heads
//   key_cache[slot(t), h] = rope(rmsnorm(k[t, h], k_weight), cos[t], sin[t])   h < kv_heads
//   value_cache[slot(t), h] = v[t, h]                                           (bit-exact copy)
// with the eager fp16/bf16 rounding steps of the reference's torch path:
//   rmsnorm: n = T(x * rsqrt(mean(x^2) + eps)) then T(n * w) (fallback.py:8-10,
//            elementwise.cu norm_kernel: the normalised value is rounded
//            before the weight multiply);
//   rope:    each product T(a * c) is rounded before the add / subtract, on
//            halves [0, D/2) and [D/2, D) (fallback.py:13-20, data.cu:29-65).
// Two kernels: a vector kernel for head_dim 16, 32, ..., 512 with 16-byte
// aligned rows (16-byte loads, rows of all tokens spread over the grid), and
// a general one for any even head_dim <= 512 (one 256-lane work-group per
// token; each wave takes whole head rows and a lane holds the rotation pairs
// (p, p + D/2) for p = lane, lane + 64, ..., so the rotation never leaves the
// lane).  Rows whose slot is out of range skip the cache write (q_out is
// always written).
#include "norm_rope.h"

namespace mvme {
namespace {

constexpr int kRopeThreads = 256;
constexpr int kRopeMaxHalf = 256;  // head_dim <= 512
constexpr int kRopePairs = kRopeMaxHalf / kWave;

struct RopeArgs {
    uint16_t* q_out;
    uint16_t* key_cache;
    uint16_t* value_cache;
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const uint16_t* q_weight;
    const uint16_t* k_weight;
    const uint16_t* cos;
    const uint16_t* sin;
    const int64_t* slots;      // [tokens] or null (decode mode)
    const int64_t* tables;     // decode mode: [tokens, table_width]
    const int64_t* positions;  // decode mode: [tokens]
    int64_t q_stride, k_stride, v_stride;  // elements between consecutive tokens
    int64_t num_blocks, block_size, table_width;
    int q_heads, kv_heads, dim;
    float eps;
};

// Physical slot of token t or -1 (slot rule of batch.py:110-112, data.cu:88-107).
__device__ inline int64_t rope_slot(const RopeArgs& a, int64_t t) {
    const int64_t capacity = a.num_blocks * a.block_size;
    if (a.slots) {
        const int64_t slot = a.slots[t];
        return slot >= 0 && slot < capacity ? slot : -1;
    }
    const int64_t pos = a.positions[t];
    if (pos < 0 || pos >= a.table_width * a.block_size) return -1;
    const int64_t page = a.tables[t * a.table_width + pos / a.block_size];
    if (page < 0 || page >= a.num_blocks) return -1;
    return page * a.block_size + pos % a.block_size;
}

// RMSNorm + RoPE of one head row `src` (dim elements) into `dst`.
template <typename T>
__device__ inline void norm_rope_row(const RopeArgs& a, const uint16_t* src, const uint16_t* weight,
                                     const uint16_t* cs, const uint16_t* sn, uint16_t* dst, int lane) {
    // No multiply-add contraction: once the float arithmetic below is narrowed
    // to fp16 instructions, contraction would fuse n1*c into the subtraction
    // and skip the product's own rounding.
#pragma clang fp contract(off)
    const int half = a.dim / 2;
    float x1[kRopePairs], x2[kRopePairs];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kRopePairs; ++i) {
        const int p = lane + i * kWave;
        x1[i] = x2[i] = 0.f;
        if (p < half) {
            x1[i] = to_f<T>(src[p]);
            x2[i] = to_f<T>(src[p + half]);
        }
        ss = fmaf(x1[i], x1[i], ss);
        ss = fmaf(x2[i], x2[i], ss);
    }
#pragma unroll
    for (int mask = 1; mask < kWave; mask <<= 1) ss += shfl_xor(ss, mask);
    const float inv = 1.f / sqrtf(ss / (float)a.dim + a.eps);
#pragma unroll
    for (int i = 0; i < kRopePairs; ++i) {
        const int p = lane + i * kWave;
        if (p >= half) continue;
        // x * inv is rounded to fp32 first, then to T (the reference's two
        // roundings); the empty asm keeps the compiler from turning the pair
        // into one mixed-precision multiply that rounds to T directly.
        float m1 = x1[i] * inv, m2 = x2[i] * inv;
        asm volatile("" : "+v"(m1), "+v"(m2));
        const float n1 = round_t<T>(round_t<T>(m1) * to_f<T>(weight[p]));
        const float n2 = round_t<T>(round_t<T>(m2) * to_f<T>(weight[p + half]));
        const float c = to_f<T>(cs[p]), s = to_f<T>(sn[p]);
        dst[p] = T::from_float(round_t<T>(n1 * c) - round_t<T>(n2 * s));
        dst[p + half] = T::from_float(round_t<T>(n1 * s) + round_t<T>(n2 * c));
    }
}

template <typename T>
__global__ __launch_bounds__(kRopeThreads) void qk_norm_rope_kernel(RopeArgs a) {
    const int64_t t = blockIdx.x;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    constexpr int kWaves = kRopeThreads / kWave;
    const int64_t slot = rope_slot(a, t);
    const int half = a.dim / 2;
    const uint16_t* cs = a.cos + t * half;
    const uint16_t* sn = a.sin + t * half;
    const int64_t row_elems = (int64_t)a.kv_heads * a.dim;
    const int rows = a.q_heads + 2 * a.kv_heads;
    for (int r = wave; r < rows; r += kWaves) {
        if (r < a.q_heads) {
            norm_rope_row<T>(a, a.q + t * a.q_stride + (int64_t)r * a.dim, a.q_weight, cs, sn,
                             a.q_out + (t * a.q_heads + r) * a.dim, lane);
        } else if (r < a.q_heads + a.kv_heads) {
            if (slot < 0) continue;
            const int h = r - a.q_heads;
            norm_rope_row<T>(a, a.k + t * a.k_stride + (int64_t)h * a.dim, a.k_weight, cs, sn,
                             a.key_cache + slot * row_elems + (int64_t)h * a.dim, lane);
        } else {
            if (slot < 0) continue;
            const int h = r - a.q_heads - a.kv_heads;
            const uint16_t* src = a.v + t * a.v_stride + (int64_t)h * a.dim;
            uint16_t* dst = a.value_cache + slot * row_elems + (int64_t)h * a.dim;
            for (int d = lane; d < a.dim; d += kWave) dst[d] = src[d];
        }
    }
}

// Vector form for head_dim = 8 * L with L a power of two in [2, 64]
// (head_dim 16 .. 512): a head row spans L lanes, each holding 8 consecutive
// elements in one 16-byte load, so a wave covers 64 / L rows at once (4 rows
// of 128).  Rows of all tokens are numbered q rows, k rows, v rows per token
// and spread over the grid, one row per L lanes, which keeps many rows in
// flight per CU instead of walking a token's rows one after another.  Lane i
// of the first half of a row pairs with lane i + L/2 (the same offsets of the
// second half), so the rotation partner arrives by one lane exchange of the
// normalised values, packed two per dword.  Every lane runs the reductions
// and exchanges (v rows and rows past the end compute on zeros and store
// nothing), so no shuffle reads a lane that branched away.
constexpr int kVecThreads = 256;

template <typename T, int L>
__global__ __launch_bounds__(kVecThreads) void qk_norm_rope_vec_kernel(RopeArgs a, int rows_per_token,
                                                                       int total_rows) {
#pragma clang fp contract(off)
    constexpr int kDim = 8 * L;
    constexpr int kHalfLanes = L / 2;
    const int sub = threadIdx.x % L;
    const int grow = (int)((blockIdx.x * kVecThreads + threadIdx.x) / L);
    const bool live = grow < total_rows;
    const int t = live ? grow / rows_per_token : 0;
    const int r = live ? grow - t * rows_per_token : 0;
    const bool is_q = r < a.q_heads;
    const bool is_k = !is_q && r < a.q_heads + a.kv_heads;
    const int h = is_q ? r : is_k ? r - a.q_heads : r - a.q_heads - a.kv_heads;
    const uint16_t* src = is_q ? a.q + t * a.q_stride : is_k ? a.k + t * a.k_stride : a.v + t * a.v_stride;
    src += (int64_t)h * kDim + sub * 8;
    const u32x4 zero = {0u, 0u, 0u, 0u};
    // Lanes past the last row read row 0 of q (in bounds) and discard it: an
    // unconditional load keeps all loads in flight together.
    const u32x4 xraw = *reinterpret_cast<const u32x4*>(src);
    const u32x4 xv = live ? xraw : zero;
    const u32x4 wv = *reinterpret_cast<const u32x4*>((is_q ? a.q_weight : a.k_weight) + sub * 8);
    const int64_t trig = (int64_t)t * (kDim / 2) + (sub % kHalfLanes) * 8;
    const u32x4 cv = *reinterpret_cast<const u32x4*>(a.cos + trig);
    const u32x4 sv = *reinterpret_cast<const u32x4*>(a.sin + trig);
    // The cache slot (one or two dependent metadata loads) after the row
    // loads, so that their latencies overlap instead of adding up.
    const int64_t slot = live && !is_q ? rope_slot(a, t) : -1;

    const u32x4 out = norm_rope_lanes<T, L>(xv, wv, cv, sv, a.eps, sub);
    if (!live) return;
    const int64_t cache_row = slot * (int64_t)a.kv_heads * kDim + (int64_t)h * kDim + sub * 8;
    if (is_q) {
        *reinterpret_cast<u32x4*>(a.q_out + ((int64_t)t * a.q_heads + h) * kDim + sub * 8) = out;
    } else if (slot >= 0) {
        *reinterpret_cast<u32x4*>((is_k ? a.key_cache : a.value_cache) + cache_row) = is_k ? out : xv;
    }
}

template <typename T>
void launch_vec(const RopeArgs& a, int lanes, int rows_per_token, int total_rows, hipStream_t s) {
    const dim3 grid((unsigned)(((int64_t)total_rows * lanes + kVecThreads - 1) / kVecThreads)), block(kVecThreads);
    switch (lanes) {
    case 2: hipLaunchKernelGGL((qk_norm_rope_vec_kernel<T, 2>), grid, block, 0, s, a, rows_per_token, total_rows); break;
    case 4: hipLaunchKernelGGL((qk_norm_rope_vec_kernel<T, 4>), grid, block, 0, s, a, rows_per_token, total_rows); break;
    case 8: hipLaunchKernelGGL((qk_norm_rope_vec_kernel<T, 8>), grid, block, 0, s, a, rows_per_token, total_rows); break;
    case 16: hipLaunchKernelGGL((qk_norm_rope_vec_kernel<T, 16>), grid, block, 0, s, a, rows_per_token, total_rows); break;
    case 32: hipLaunchKernelGGL((qk_norm_rope_vec_kernel<T, 32>), grid, block, 0, s, a, rows_per_token, total_rows); break;
    default: hipLaunchKernelGGL((qk_norm_rope_vec_kernel<T, 64>), grid, block, 0, s, a, rows_per_token, total_rows); break;
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace mvme

using namespace mvme;

extern "C" int mvme_qk_norm_rope_write_kv(void* q_out, void* key_cache, void* value_cache, int64_t num_blocks,
                                          int64_t block_size, int64_t kv_heads, int64_t head_dim,
                                          const int64_t* slot_mapping, const int64_t* block_tables,
                                          int64_t table_width, const int64_t* positions, const void* q,
                                          const void* k, const void* v, int64_t q_token_stride,
                                          int64_t k_token_stride, int64_t v_token_stride, const void* q_weight,
                                          const void* k_weight, const void* cos, const void* sin,
                                          int64_t tokens, int64_t q_heads, float eps, int dtype, void* stream) {
    if (!valid_dtype(dtype)) return fail(MVME_EINVAL, "RoPE requires FP16/BF16 Q/K");
    if (num_blocks <= 0 || block_size <= 0 || kv_heads <= 0 || head_dim <= 0)
        return fail(MVME_EINVAL, "cache shape mismatch");
    if (head_dim % 2 != 0 || head_dim / 2 > kRopeMaxHalf)
        return fail(MVME_EINVAL, "RoPE cos/sin shape mismatch (head_dim must be even and at most 512)");
    if (q_heads <= 0 || q_heads % kv_heads != 0) return fail(MVME_EINVAL, "RoPE GQA head mismatch");
    if (q_heads + 2 * kv_heads > (1 << 20)) return fail(MVME_EINVAL, "too many RoPE heads");
    if (!(eps > 0.f) || !__builtin_isfinite(eps)) return fail(MVME_EINVAL, "eps must be positive, finite and representable in FP32");
    if (tokens < 0 || tokens > 2147483647) return fail(MVME_EINVAL, "too many RoPE tokens");
    if (q_token_stride < q_heads * head_dim || k_token_stride < kv_heads * head_dim ||
        v_token_stride < kv_heads * head_dim)
        return fail(MVME_EINVAL, "Q/K/V token stride smaller than a row");
    if (tokens == 0) return MVME_OK;
    if (!q_out || !key_cache || !value_cache || !q || !k || !v || !q_weight || !k_weight || !cos || !sin)
        return fail(MVME_EINVAL, "qk_norm_rope received a null pointer");
    if (!slot_mapping && (!block_tables || !positions || table_width <= 0))
        return fail(MVME_EINVAL, "qk_norm_rope needs a slot mapping or block tables with positions");
    RopeArgs a{};
    a.q_out = static_cast<uint16_t*>(q_out);
    a.key_cache = static_cast<uint16_t*>(key_cache);
    a.value_cache = static_cast<uint16_t*>(value_cache);
    a.q = static_cast<const uint16_t*>(q);
    a.k = static_cast<const uint16_t*>(k);
    a.v = static_cast<const uint16_t*>(v);
    a.q_weight = static_cast<const uint16_t*>(q_weight);
    a.k_weight = static_cast<const uint16_t*>(k_weight);
    a.cos = static_cast<const uint16_t*>(cos);
    a.sin = static_cast<const uint16_t*>(sin);
    a.slots = slot_mapping;
    a.tables = block_tables;
    a.positions = positions;
    a.q_stride = q_token_stride;
    a.k_stride = k_token_stride;
    a.v_stride = v_token_stride;
    a.num_blocks = num_blocks;
    a.block_size = block_size;
    a.table_width = table_width;
    a.q_heads = (int)q_heads;
    a.kv_heads = (int)kv_heads;
    a.dim = (int)head_dim;
    a.eps = eps;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // Vector kernel: head_dim = 8 * lanes with lanes a power of two in [2, 64],
    // 16-byte aligned rows, and a row count whose lane index fits 32 bits.
    const int64_t lanes = head_dim / 8;
    const int64_t rows_per_token = q_heads + 2 * kv_heads;
    const bool vec_shape = head_dim % 8 == 0 && lanes >= 2 && lanes <= 64 && (lanes & (lanes - 1)) == 0;
    const bool vec_align = aligned16(q_out) && aligned16(key_cache) && aligned16(value_cache) && aligned16(q) &&
                           aligned16(k) && aligned16(v) && aligned16(q_weight) && aligned16(k_weight) &&
                           aligned16(cos) && aligned16(sin) && q_token_stride % 8 == 0 &&
                           k_token_stride % 8 == 0 && v_token_stride % 8 == 0;
    const bool vec_size = tokens * rows_per_token * lanes <= 2147483647;
    if (vec_shape && vec_align && vec_size) {
        const int total_rows = (int)(tokens * rows_per_token);
        if (dtype == MVME_FP16) launch_vec<Half>(a, (int)lanes, (int)rows_per_token, total_rows, s);
        else launch_vec<BFloat16>(a, (int)lanes, (int)rows_per_token, total_rows, s);
        return check_launch("qk norm + rope + KV write");
    }
    const dim3 grid((unsigned)tokens), block(kRopeThreads);
    if (dtype == MVME_FP16) hipLaunchKernelGGL(qk_norm_rope_kernel<Half>, grid, block, 0, s, a);
    else hipLaunchKernelGGL(qk_norm_rope_kernel<BFloat16>, grid, block, 0, s, a);
    return check_launch("qk norm + rope + KV write");
}

// KV scatter / gather on the paged cache [num_blocks, block_size, kv_heads, head_dim].
//
// All variants are byte copies of whole token rows (kv_heads*head_dim
// elements): one work-group per token row, 16-byte vector copies when every
// address is 16-byte aligned, 2-byte copies otherwise.  The destination slot
// of a token is computed from the metadata inside the kernel, so the host
// never reads device metadata.  Rows whose slot or page id is out of range
// are skipped (scatter) or zero-filled (gather), never dereferenced.
#include "mvme_common.h"

namespace mvme {
namespace {

constexpr int kCopyThreads = 256;

enum SlotMode { kModeSlots = 0, kModeBatch = 1, kModeRange = 2 };

struct ScatterArgs {
    uint8_t* key_cache;
    uint8_t* value_cache;
    const uint8_t* key;
    const uint8_t* value;
    const int64_t* index;    // slots | block tables | block ids
    const int64_t* offsets;  // per-sequence token offsets (batch mode)
    int64_t row_bytes;
    int64_t key_stride_bytes;
    int64_t value_stride_bytes;
    int64_t num_blocks;
    int64_t block_size;
    int64_t index_width;     // table width (batch) or number of ids (range)
    int64_t token_offset;    // first logical position (range mode)
};

// Physical slot of token `t`, or -1 when the metadata does not name a valid
// slot.  Follows the slot rule page * block_size + pos % block_size of
// mini_engine/engine/batch.py:110-112 and csrc/data.cu:88-107, :67-86.
template <int MODE>
__device__ inline int64_t token_slot(const ScatterArgs& a, int64_t t) {
    const int64_t capacity = a.num_blocks * a.block_size;
    if constexpr (MODE == kModeSlots) {
        const int64_t slot = a.index[t];
        return (slot >= 0 && slot < capacity) ? slot : -1;
    } else {
        const int64_t pos = MODE == kModeBatch ? a.offsets[t] : a.token_offset + t;
        if (pos < 0) return -1;
        const int64_t block = pos / a.block_size;
        if (block >= a.index_width) return -1;
        const int64_t page = MODE == kModeBatch ? a.index[t * a.index_width + block] : a.index[block];
        if (page < 0 || page >= a.num_blocks) return -1;
        return page * a.block_size + pos % a.block_size;
    }
}

template <int MODE, bool VEC16>
__global__ __launch_bounds__(kCopyThreads) void kv_scatter_kernel(ScatterArgs a) {
    const int64_t t = blockIdx.x;
    const int64_t slot = token_slot<MODE>(a, t);
    if (slot < 0) return;
    uint8_t* dk = a.key_cache + slot * a.row_bytes;
    uint8_t* dv = a.value_cache + slot * a.row_bytes;
    const uint8_t* sk = a.key + t * a.key_stride_bytes;
    const uint8_t* sv = a.value + t * a.value_stride_bytes;
    if constexpr (VEC16) {
        const int n = (int)(a.row_bytes / 16);
        for (int i = threadIdx.x; i < 2 * n; i += kCopyThreads) {
            const bool is_v = i >= n;
            const int j = is_v ? i - n : i;
            const u32x4 w = reinterpret_cast<const u32x4*>(is_v ? sv : sk)[j];
            reinterpret_cast<u32x4*>(is_v ? dv : dk)[j] = w;
        }
    } else {
        const int n = (int)(a.row_bytes / 2);
        for (int i = threadIdx.x; i < 2 * n; i += kCopyThreads) {
            const bool is_v = i >= n;
            const int j = is_v ? i - n : i;
            reinterpret_cast<uint16_t*>(is_v ? dv : dk)[j] =
                reinterpret_cast<const uint16_t*>(is_v ? sv : sk)[j];
        }
    }
}

struct GatherArgs {
    uint8_t* key_out;
    uint8_t* value_out;
    const uint8_t* key_cache;
    const uint8_t* value_cache;
    const int64_t* block_ids;
    int64_t row_bytes;
    int64_t num_blocks;
    int64_t block_size;
    int64_t num_ids;
};

template <bool VEC16>
__global__ __launch_bounds__(kCopyThreads) void kv_gather_kernel(GatherArgs g) {
    const int64_t n = blockIdx.x;
    const int64_t block = n / g.block_size;
    const int64_t page = block < g.num_ids ? g.block_ids[block] : -1;
    const bool valid = page >= 0 && page < g.num_blocks;
    const int64_t src_row = valid ? page * g.block_size + n % g.block_size : 0;
    const uint8_t* sk = g.key_cache + src_row * g.row_bytes;
    const uint8_t* sv = g.value_cache + src_row * g.row_bytes;
    uint8_t* dk = g.key_out + n * g.row_bytes;
    uint8_t* dv = g.value_out + n * g.row_bytes;
    if constexpr (VEC16) {
        const int count = (int)(g.row_bytes / 16);
        for (int i = threadIdx.x; i < 2 * count; i += kCopyThreads) {
            const bool is_v = i >= count;
            const int j = is_v ? i - count : i;
            u32x4 w = {0u, 0u, 0u, 0u};
            if (valid) w = reinterpret_cast<const u32x4*>(is_v ? sv : sk)[j];
            reinterpret_cast<u32x4*>(is_v ? dv : dk)[j] = w;
        }
    } else {
        const int count = (int)(g.row_bytes / 2);
        for (int i = threadIdx.x; i < 2 * count; i += kCopyThreads) {
            const bool is_v = i >= count;
            const int j = is_v ? i - count : i;
            uint16_t w = 0;
            if (valid) w = reinterpret_cast<const uint16_t*>(is_v ? sv : sk)[j];
            reinterpret_cast<uint16_t*>(is_v ? dv : dk)[j] = w;
        }
    }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_geometry(int64_t num_blocks, int64_t block_size, int64_t kv_heads, int64_t head_dim, int dtype) {
    if (num_blocks <= 0 || block_size <= 0 || kv_heads <= 0 || head_dim <= 0)
        return fail(MVME_EINVAL, "KV cache dimensions must be positive");
    if (!valid_dtype(dtype)) return fail(MVME_EINVAL, "KV cache requires FP16/BF16");
    if (kv_heads * head_dim > (int64_t(1) << 24))
        return fail(MVME_EINVAL, "KV row (kv_heads*head_dim) too large");
    return MVME_OK;
}

template <int MODE>
int launch_scatter(const ScatterArgs& a, int64_t tokens, hipStream_t stream) {
    if (tokens == 0) return MVME_OK;
    const bool vec = a.row_bytes % 16 == 0 && a.key_stride_bytes % 16 == 0 &&
                     a.value_stride_bytes % 16 == 0 && aligned16(a.key_cache) &&
                     aligned16(a.value_cache) && aligned16(a.key) && aligned16(a.value);
    const dim3 grid((unsigned)tokens);
    if (vec)
        hipLaunchKernelGGL((kv_scatter_kernel<MODE, true>), grid, dim3(kCopyThreads), 0, stream, a);
    else
        hipLaunchKernelGGL((kv_scatter_kernel<MODE, false>), grid, dim3(kCopyThreads), 0, stream, a);
    return check_launch("KV scatter");
}

}  // namespace
}  // namespace mvme

using namespace mvme;

extern "C" int mvme_write_kv_cache_slots(void* key_cache, void* value_cache, int64_t num_blocks,
                                         int64_t block_size, int64_t kv_heads, int64_t head_dim,
                                         const int64_t* slot_mapping, const void* key,
                                         const void* value, int64_t tokens,
                                         int64_t key_token_stride, int64_t value_token_stride,
                                         int dtype, void* stream) {
    if (int rc = check_geometry(num_blocks, block_size, kv_heads, head_dim, dtype)) return rc;
    if (tokens < 0 || tokens > 2147483647) return fail(MVME_EINVAL, "too many packed KV rows");
    if (tokens == 0) return MVME_OK;
    const int64_t row = kv_heads * head_dim;
    if (!key_cache || !value_cache || !slot_mapping || !key || !value)
        return fail(MVME_EINVAL, "packed KV write received a null pointer");
    if (key_token_stride < row || value_token_stride < row)
        return fail(MVME_EINVAL, "packed key/value token stride smaller than a KV row");
    ScatterArgs a{};
    a.key_cache = static_cast<uint8_t*>(key_cache);
    a.value_cache = static_cast<uint8_t*>(value_cache);
    a.key = static_cast<const uint8_t*>(key);
    a.value = static_cast<const uint8_t*>(value);
    a.index = slot_mapping;
    a.row_bytes = row * 2;
    a.key_stride_bytes = key_token_stride * 2;
    a.value_stride_bytes = value_token_stride * 2;
    a.num_blocks = num_blocks;
    a.block_size = block_size;
    return launch_scatter<kModeSlots>(a, tokens, static_cast<hipStream_t>(stream));
}

extern "C" int mvme_write_kv_cache_batch(void* key_cache, void* value_cache, int64_t num_blocks,
                                         int64_t block_size, int64_t kv_heads, int64_t head_dim,
                                         const int64_t* block_tables, int64_t table_width,
                                         const int64_t* token_offsets, const void* key,
                                         const void* value, int64_t batch, int dtype,
                                         void* stream) {
    if (int rc = check_geometry(num_blocks, block_size, kv_heads, head_dim, dtype)) return rc;
    if (batch < 0 || batch > 2147483647) return fail(MVME_EINVAL, "batch KV write: batch out of range");
    if (table_width <= 0) return fail(MVME_EINVAL, "batch table shape mismatch");
    if (batch == 0) return MVME_OK;
    if (!key_cache || !value_cache || !block_tables || !token_offsets || !key || !value)
        return fail(MVME_EINVAL, "batch KV write received a null pointer");
    const int64_t row = kv_heads * head_dim;
    ScatterArgs a{};
    a.key_cache = static_cast<uint8_t*>(key_cache);
    a.value_cache = static_cast<uint8_t*>(value_cache);
    a.key = static_cast<const uint8_t*>(key);
    a.value = static_cast<const uint8_t*>(value);
    a.index = block_tables;
    a.offsets = token_offsets;
    a.row_bytes = row * 2;
    a.key_stride_bytes = a.row_bytes;
    a.value_stride_bytes = a.row_bytes;
    a.num_blocks = num_blocks;
    a.block_size = block_size;
    a.index_width = table_width;
    return launch_scatter<kModeBatch>(a, batch, static_cast<hipStream_t>(stream));
}

extern "C" int mvme_write_kv_cache(void* key_cache, void* value_cache, int64_t num_blocks,
                                   int64_t block_size, int64_t kv_heads, int64_t head_dim,
                                   const int64_t* block_ids, int64_t num_ids, int64_t token_offset,
                                   const void* key, const void* value, int64_t tokens, int dtype,
                                   void* stream) {
    if (int rc = check_geometry(num_blocks, block_size, kv_heads, head_dim, dtype)) return rc;
    if (tokens < 0 || tokens > 2147483647) return fail(MVME_EINVAL, "KV write: too many tokens");
    if (num_ids < 0 || token_offset < 0 || token_offset + tokens > num_ids * block_size)
        return fail(MVME_EINVAL, "KV write exceeds block table");
    if (tokens == 0) return MVME_OK;
    if (!key_cache || !value_cache || !block_ids || !key || !value)
        return fail(MVME_EINVAL, "KV write received a null pointer");
    const int64_t row = kv_heads * head_dim;
    ScatterArgs a{};
    a.key_cache = static_cast<uint8_t*>(key_cache);
    a.value_cache = static_cast<uint8_t*>(value_cache);
    a.key = static_cast<const uint8_t*>(key);
    a.value = static_cast<const uint8_t*>(value);
    a.index = block_ids;
    a.row_bytes = row * 2;
    a.key_stride_bytes = a.row_bytes;
    a.value_stride_bytes = a.row_bytes;
    a.num_blocks = num_blocks;
    a.block_size = block_size;
    a.index_width = num_ids;
    a.token_offset = token_offset;
    return launch_scatter<kModeRange>(a, tokens, static_cast<hipStream_t>(stream));
}

extern "C" int mvme_gather_kv_cache(void* key_out, void* value_out, const void* key_cache,
                                    const void* value_cache, int64_t num_blocks,
                                    int64_t block_size, int64_t kv_heads, int64_t head_dim,
                                    const int64_t* block_ids, int64_t num_ids,
                                    int64_t token_count, int dtype, void* stream) {
    if (int rc = check_geometry(num_blocks, block_size, kv_heads, head_dim, dtype)) return rc;
    if (token_count < 0 || num_ids < 0 || token_count > num_ids * block_size)
        return fail(MVME_EINVAL, "token_count exceeds supplied block table capacity");
    if (token_count > 2147483647) return fail(MVME_EINVAL, "gather: too many tokens");
    if (token_count == 0) return MVME_OK;
    if (!key_out || !value_out || !key_cache || !value_cache || !block_ids)
        return fail(MVME_EINVAL, "gather received a null pointer");
    GatherArgs g{};
    g.key_out = static_cast<uint8_t*>(key_out);
    g.value_out = static_cast<uint8_t*>(value_out);
    g.key_cache = static_cast<const uint8_t*>(key_cache);
    g.value_cache = static_cast<const uint8_t*>(value_cache);
    g.block_ids = block_ids;
    g.row_bytes = kv_heads * head_dim * 2;
    g.num_blocks = num_blocks;
    g.block_size = block_size;
    g.num_ids = num_ids;
    const bool vec = g.row_bytes % 16 == 0 && aligned16(key_out) && aligned16(value_out) &&
                     aligned16(key_cache) && aligned16(value_cache);
    const dim3 grid((unsigned)token_count);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (vec)
        hipLaunchKernelGGL((kv_gather_kernel<true>), grid, dim3(kCopyThreads), 0, s, g);
    else
        hipLaunchKernelGGL((kv_gather_kernel<false>), grid, dim3(kCopyThreads), 0, s, g);
    return check_launch("KV gather");
}

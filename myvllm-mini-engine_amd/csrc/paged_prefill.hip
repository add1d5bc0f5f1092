// Ragged chunked paged prefill for gfx950.
//
// Packed queries q[T, Hq, D]; sequence s owns packed rows
// [cu[s], cu[s+1]), row i of s sits at absolute position starts[s] + i and
// attends keys [0, starts[s] + i] of s through its block table.
//
// MFMA path (D a multiple of 8 up to 256, any G = Hq/Hkv up to the tile's
// rows; described for the D = 128 tile shape, PfShape below gives the 256 one):
//   Work item = (sequence, kv head, block of floor(256/G) query tokens, chunk
//   of `chunk` keys).  The 256 query rows of an item = (token, head-of-group)
//   pairs that share every K/V tile (rows past tokens * G idle); each of the
//   8 waves (two per SIMD) owns 32 rows (two 16-row MFMA column blocks).
//   Head dims below the shape's are zero-padded in LDS.  Long contexts with few query
//   blocks are cut into key chunks so that the work items spread over all
//   CUs; items of a query block that needs several chunks write partials
//   (the output normalised by its own probability sum -- bf16 for bf16
//   inputs, fp32 for fp16 -- with the fp32 reference and sum) that a merge
//   kernel combines.  Items are enumerated densely from the metadata on the device,
//   so grid position i is the i-th real item (work-groups past the end exit);
//   within a sequence the query blocks are enumerated from the last (longest
//   key range) to the first, so that the work-groups dispatched last are the
//   short ones.
//
//   K/V tiles of 64 keys move from the pages straight into LDS with
//   global_load_lds_dwordx4 (no VGPR staging) into a ring of 4 stages, in
//   pairs: one barrier per pair of tiles both publishes the two landed tiles
//   and retires the previous pair's stages, which the copies of the next
//   pair (issued right after the barrier) overwrite.  Each 256-byte key row is stored with its 16-byte
//   chunks XOR-swizzled by the row index (K) or twice the row index (V),
//   which keeps both the K reads and the transposing V reads below free of
//   bank conflicts.
//
//   Scores are computed transposed, S^T = K Q^T (v_mfma_f32_16x16x32), so
//   each lane holds scores of ONE query row (four lanes share a row) and the
//   probabilities already sit in the B-operand layout of O^T = V^T P^T.  The
//   V^T operand (8 consecutive keys of one dim per lane) is read from the
//   row-major V tile with two ds_read_b64_tr_b16 transposing loads.  Keys are
//   assigned to MFMA k-slots by one permutation applied to both operands.
//   Every accumulator takes its products back to back (the four d-slices of
//   a score block; both halves of a tile for an output block): the matrix
//   core forwards a result into the next product of the same accumulator,
//   while alternating accumulators costs issue slots.
//   The online softmax keeps a per-row reference m and computes
//   p = 2^(s*scale - m) without a row maximum; the sum of a lane's 8
//   probabilities of a half tile (which any probability above 2^8, inf or
//   NaN pushes past 256) triggers the exact step: the row maximum across the
//   four lanes (permlane swaps), a rescale of the accumulators, and new
//   probabilities.  It runs when a row sees its first key and when a row's
//   scores grow by several binary orders, so the accumulators are rescaled
//   rarely and probabilities stay below 2^8.  Tiles that are complete and
//   entirely below the causal diagonal skip masking.  Accumulation, softmax
//   and normalisation are fp32.
//
// Generic path (any D <= 1024, any G): one wave per (query row, head),
// online softmax over 64-key tiles, fp32 throughout.
//
// Dense mode (the dense suffix prefill of [B, H, T, D] tensors, at the end of
// this file): the same kernels with batch entry b as sequence b, whose keys
// are one page read through explicit strides, and no metadata arrays.  In
// the MFMA kernel it is a template flag, so the paged instantiations keep
// their code.
#include "mvme_common.h"

#include <algorithm>

namespace mvme {
namespace {

constexpr int kPfWaves = 8;
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kPfStages = 4;              // LDS ring of K/V tiles
constexpr int kArriveSpinLimit = 1 << 18; // polls (each with a 64-cycle sleep) of a split-barrier wait
constexpr int kTileBytes = 16384;         // one K (or V) tile in LDS, every tile shape
constexpr int kPfMaxKeys = 64;            // keys per tile, largest tile shape

// Tile shape of the MFMA kernel by padded head dim: 128 (head_dim 128 and
// narrower multiples of 8) or 256.  Every tile is 16 KiB of K (and of V) in
// LDS; at 256 a wave holds one 16-row block (the accumulators of 256 dims
// fill the registers two blocks used) and a tile has 32 keys.
template <int HD>
struct PfShape {
    static_assert(HD == 128 || HD == 256, "padded head dim 128 or 256");
    static constexpr int kD = HD;
    static constexpr int kNb = HD == 128 ? 2 : 1;      // 16-row MFMA column blocks per wave
    static constexpr int kRows = kPfWaves * kNb * 16;  // query rows per work-group
    static constexpr int kKeys = HD == 128 ? 64 : 32;  // keys per LDS tile
    static constexpr int kHalves = kKeys / 32;         // 32-key halves per tile
    static constexpr int kRowBytes = HD * 2;           // bytes per K/V row in LDS
    static constexpr int kChunks = HD / 8;             // 16-byte chunks per row
    static constexpr int kRowsPerInst = 1024 / kRowBytes;  // rows per 1 KiB copy instruction
    static constexpr int kIpw = kKeys * kRowBytes / 1024 / kPfWaves;  // copy instructions per wave per tile
    static constexpr int kDc = HD / 32;  // 32-dim slices of a score product
    static constexpr int kDt = HD / 16;  // 16-dim output blocks
    static_assert(kKeys * kRowBytes == kTileBytes, "one tile = 16 KiB");
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Finite source for key rows that are absent (out-of-range page, beyond the
// context): loading zeros keeps every LDS slot finite without predication.
__device__ __attribute__((aligned(16))) const uint32_t kZeroChunk[4] = {0u, 0u, 0u, 0u};

struct PrefillArgs {
    void* out;
    const void* q;
    const void* key_cache;
    const void* value_cache;
    const int64_t* cu;
    const int64_t* starts;
    const int64_t* tables;
    const int64_t* lens;
    void* ws_o;    // [max_chunks, T*Hq, part_dim] partial outputs normalised by their sum (PartialOf<T>)
    float* ws_ml;  // [max_chunks, T*Hq, 2] (running max in log2 units, sum)
    int64_t ws_rows;  // T*Hq: one plane of partials per chunk index
    int64_t total_tokens;  // T: packed query rows (every row a sequence covers lies below it)
    int* ws_tok;   // [T] chunks of the token's query block (written by its chunk-0 items)
    int item_stride;  // 0: one item per work-group; else items walked per work-group
    int num_seqs;
    int q_heads;
    int kv_heads;
    int group;
    int qb;        // query tokens per item (rows of the tile shape / group, rounded down)
    int chunk;     // keys per item (multiple of the tile's keys)
    int max_chunks;
    int chunk_choice;  // 1: a walk with more than one round of items may take a larger chunk
    int head_dim;
    int part_dim;  // elements per partial row: the tile shape's padded head dim
    int64_t num_blocks;
    int block_size;
    int block_shift;  // log2(block_size) when a power of two, else -1
    int table_width;
    float scale_log2;
    // Memory layout.  Key row k of page p, kv head h starts at byte
    // p*kv_page_bytes + (k mod block_size)*kv_row_bytes + h*kv_head_bytes of
    // the K (and V) base.  Query / output row (packed row r of sequence s,
    // head h) starts at element s*x_seq + r*x_tok + h*x_head.
    int64_t kv_page_bytes, kv_row_bytes, kv_head_bytes;
    int64_t q_seq, q_tok, q_head;
    int64_t o_seq, o_tok, o_head;
    // Dense mode (tables == nullptr): every sequence has dense_tokens queries
    // starting at position dense_start and context dense_start +
    // dense_tokens; sequence s owns packed rows [s*dense_tokens, (s+1)*dense_tokens)
    // and its keys are page s.  The metadata arrays are not read.
    int dense_tokens;
    int dense_start;
};

// Sequence of a packed row in dense mode (0 otherwise: the layouts of the
// paged mode have no per-sequence term).
__device__ inline int64_t dense_seq(const PrefillArgs& a, int64_t row) {
    return a.dense_tokens > 0 ? row / a.dense_tokens : 0;
}

// Keys a query block [q0, q0+qb) of sequence s needs: [0, kv_end).
__device__ inline int64_t block_kv_end(const PrefillArgs& a, int64_t start, int64_t ctx, int64_t qlen, int64_t q0) {
    const int64_t cap = (int64_t)a.table_width * a.block_size;
    int64_t e = start + min(q0 + (int64_t)a.qb, qlen);
    if (e > ctx) e = ctx;
    if (e > cap) e = cap;
    return e > 0 ? e : 0;
}

// ceil(e / d) for 0 < e, d < 2^31: a float estimate of the quotient,
// corrected to the exact ceiling with integer products -- cheaper than an
// integer division by a run-time divisor.  The estimate's relative error is
// a few ulps, so below 2^20 it is within one of e / d: its truncation is
// floor(e/d) - 1, floor(e/d) or (only when that is the ceiling)
// floor(e/d) + 1, and at most two steps up reach the ceiling.  Larger
// quotients take the integer division.
__device__ inline uint32_t ceil_div_u32(uint32_t e, uint32_t d) {
    uint32_t q = (uint32_t)((float)e * __builtin_amdgcn_rcpf((float)d));
    if (q >= (1u << 20)) return (e - 1u) / d + 1u;
    if (q * d < e) ++q;
    if (q * d < e) ++q;
    return q;
}

// Query blocks of a sequence with n packed queries (n < 2^31: offsets are
// clamped to the packed rows), by the float-corrected quotient rather than a
// 64-bit division (a long instruction sequence on the lookup's critical path).
__device__ inline int query_blocks(const PrefillArgs& a, int64_t n) {
    return n > 0 ? (int)ceil_div_u32((uint32_t)n, (uint32_t)a.qb) : 0;
}

// kv_end <= table capacity < 2^31, so 32-bit unsigned arithmetic is exact.
__device__ inline int chunks_of(int chunk_len, int64_t kv_end) {
    return kv_end > 0 ? (int)ceil_div_u32((uint32_t)kv_end, (uint32_t)chunk_len) : 1;
}

// Items (query block x key chunk) of a sequence with n packed queries;
// every query block owns at least one item so its rows always get written.
// Without key splitting every block is exactly one item.
__device__ inline int seq_items(const PrefillArgs& a, int chunk_len, int64_t n, int64_t start, int64_t ctx) {
    if (n <= 0) return 0;
    if (a.max_chunks == 1) return query_blocks(a, n);
    int count = 0;
    for (int64_t b0 = 0; b0 < n; b0 += a.qb) count += chunks_of(chunk_len, block_kv_end(a, start, ctx, n, b0));
    return count;
}

// Element type of the key-chunk partial outputs.  They are normalised by
// their own probability sum (a convex combination of V rows), so bf16 keeps
// them as accurately as the bf16 output; fp16 inputs keep fp32 partials.
template <typename T> struct PartialOf { using type = float; };
template <> struct PartialOf<BFloat16> { using type = uint16_t; };

struct PrefillItem {
    int seq, q0, chunk, nchunks, chunk_len;
    int64_t kv_end;
    int64_t row0, qlen, start, ctx;  // the sequence's metadata
};

// One sequence's metadata per lane (lane s: sequence s0 + s).
struct SeqMeta {
    int64_t row0, n, start, ctx;
};
// Offsets are clamped to the packed rows, so that metadata that is not
// monotone (unchecked in trusted mode) can neither send a write past the
// output nor make a lookup loop over an absurd number of query blocks.
template <bool DENSE>
__device__ inline SeqMeta load_meta(const PrefillArgs& a, int s) {
    SeqMeta m{0, 0, 0, 0};
    if (DENSE && s < a.num_seqs) {
        m.row0 = (int64_t)s * a.dense_tokens;
        m.n = a.dense_tokens;
        m.start = a.dense_start;
        m.ctx = (int64_t)a.dense_start + a.dense_tokens;
    } else if (!DENSE && s < a.num_seqs) {
        const int64_t lo = min(max(a.cu[s], (int64_t)0), a.total_tokens);
        const int64_t hi = min(max(a.cu[s + 1], lo), a.total_tokens);
        m.row0 = lo;
        m.n = hi - lo;
        m.start = a.starts[s];
        m.ctx = a.lens[s];
    }
    return m;
}

// Item `item` -> sequence, first query token, chunk, and the sequence's
// metadata, with key chunks of chunk_len keys.  `first` (optional) holds the
// first 64 sequences' metadata, already loaded.  Lane-parallel: each lane loads one sequence's metadata and
// counts its items, a wave prefix sum locates the sequence, the lane that
// owns it hands its metadata over by shuffles, and that one sequence's query
// blocks are walked.  Every wave of the work-group computes the same answer.
template <bool DENSE>
__device__ inline bool find_item(const PrefillArgs& a, int chunk_len, int item, PrefillItem& it,
                                 int* total_items = nullptr, const SeqMeta* first = nullptr) {
    const int lane = __lane_id();
    int base = 0;
    bool found = false;
    for (int s0 = 0; s0 < a.num_seqs; s0 += kWave) {
        const SeqMeta m = (first && s0 == 0) ? *first : load_meta<DENSE>(a, s0 + lane);
        const int64_t row0 = m.row0, n = m.n, start = m.start, ctx = m.ctx;
        const int cnt = seq_items(a, chunk_len, n, start, ctx);
        const int incl = wave_incl_scan(cnt);
        const int total = lane_value(incl, kWave - 1);
        if (!found && item >= base && item < base + total) {
            const uint64_t hit = __ballot(base + incl > item);
            const int sel = __builtin_ctzll(hit);
            it.seq = s0 + sel;
            int rem = item - base - (lane_value(incl, sel) - lane_value(cnt, sel));
            it.row0 = lane_value(row0, sel);
            it.qlen = lane_value(n, sel);
            it.start = lane_value(start, sel);
            it.ctx = lane_value(ctx, sel);
            // Query blocks from the last (longest key range) to the first, so
            // that the work-groups dispatched last are the short ones.
            const int64_t nblocks = query_blocks(a, it.qlen);
            it.chunk_len = chunk_len;
            if (a.max_chunks == 1) {  // one item per block: no search
                const int64_t b0 = (nblocks - 1 - rem) * a.qb;
                it.q0 = (int)b0;
                it.chunk = 0;
                it.kv_end = block_kv_end(a, it.start, it.ctx, it.qlen, b0);
                it.nchunks = 1;
                found = true;
                if (!total_items) return true;
                base += total;
                continue;
            }
            for (int64_t bi = nblocks - 1; bi >= 0; --bi) {
                const int64_t b0 = bi * a.qb;
                const int64_t e = block_kv_end(a, it.start, it.ctx, it.qlen, b0);
                const int nc = chunks_of(chunk_len, e);
                if (rem < nc) {
                    it.q0 = (int)b0;
                    it.chunk = rem;
                    it.chunk_len = chunk_len;
                    it.kv_end = e;
                    it.nchunks = nc;
                    found = true;
                    break;
                }
                rem -= nc;
            }
            if (!total_items) return found;  // (not found only if the counts are inconsistent)
        }
        base += total;
    }
    if (total_items) *total_items = base;
    return found;
}

// Direct global -> LDS copy of 16 bytes per lane: lane i's bytes land at LDS
// address `lds_base + 16*i` (lds_base is wave-uniform, passed through M0).
// Issued as inline assembly so that the compiler does not serialise it
// against unrelated LDS reads; the kernel orders it with explicit
// s_waitcnt vmcnt(0) + s_barrier before the destination stage is read.
// M0 is declared clobbered (the compiler sets it again where it needs it).
__device__ inline void lds_dma16(const void* gptr, uint32_t lds_base) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_base);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gptr), "s"(base) : "m0");
}

template <typename P>
__device__ inline uint32_t lds_addr(P* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)p;
}

// A lane's 8 probabilities of one half tile sum to at most this before the
// row's reference is raised (some probability above 2^5 .. 2^8 triggers it):
// probabilities stay far inside fp16/bf16/fp32 range, and the final division
// by the row sum makes the result independent of the reference.
constexpr float kPSumLimit = 256.f;

// Full wait issued through the builtin, which the compiler's own wait
// insertion understands (it then knows earlier loads have completed).
__device__ inline void wait_vmcnt_all() { __builtin_amdgcn_s_waitcnt(0); }

// Every load and LDS access of this wave complete, then the work-group
// barrier (with a compiler memory fence).  The wait goes through the builtin
// so that the compiler knows the Q operand loads have landed too: written in
// the barrier's inline assembly instead, it is invisible to the compiler,
// which then adds its own vmcnt(0) before the first use of Q in every tile --
// and that wait also covers the copies issued right after the barrier, so
// every pair of tiles waited for the next pair's copies to land.
__device__ inline void landed_barrier() {
    wait_vmcnt_all();
    asm volatile("s_barrier" : : : "memory");
}

// Max / sum over the four lanes {l, l^16, l^32, l^48} (the 4 MFMA k-groups
// holding one query row) with gfx950 lane swaps -- no LDS round trip.
__device__ inline float row4_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float row4_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Direct global -> LDS copy from a wave-uniform base plus a per-lane 32-bit
// byte offset (the SGPR-base form of global_load_lds_dwordx4: no 64-bit
// per-lane address arithmetic).  M0 (the LDS destination) is declared
// clobbered instead of saved and restored: the compiler sets it again where
// it needs it.
__device__ inline void lds_dma16_s(const uint8_t* sbase, uint32_t voff, uint32_t lds_base) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_base);
    const uint64_t g = (uint64_t)(uintptr_t)sbase;
    const uint64_t gu = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(g >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)g);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(gu), "s"(base) : "m0");
}

// Minimum over the 64 lanes of a wave, returned to every lane: each 16-lane
// row's minimum by DPP (quad swaps, then the half-row and row mirrors), then
// the four rows' by readlane.
__device__ inline uint32_t wave_min_u32(uint32_t x) {
    x = min(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppQuadSwap1, 0xf, 0xf, false));
    x = min(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppQuadSwap2, 0xf, 0xf, false));
    x = min(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowHalfMirror, 0xf, 0xf, false));
    x = min(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowMirror, 0xf, 0xf, false));
    const uint32_t lo = min((uint32_t)lane_value((int)x, 0), (uint32_t)lane_value((int)x, 16));
    const uint32_t hi = min((uint32_t)lane_value((int)x, 32), (uint32_t)lane_value((int)x, 48));
    return min(lo, hi);
}

constexpr int kPagesPerLane = 0;
constexpr int kPagesPerRows = 1;
constexpr int kPagesPerTile = 2;

// How page ids are found (PAGES):
//   kPagesPerTile: block_size is a power of two >= 64, so a 64-key tile lies
//     in one page: one scalar page lookup per tile, and a full tile's copies
//     are a scalar base plus precomputed per-lane offsets -- a few scalar
//     instructions per tile, which matters because the scalar unit is shared
//     by all waves of the CU.
//   kPagesPerRows: see below; the fallback for partial tiles as well.
// SCALAR_PAGES: block_size is a multiple of 4, so the 4 key rows one copy
// instruction covers sit in one page and the page id is wave-uniform (a
// scalar load).  Then the vector-memory counter only ever holds the tile
// copies, and "tile t has landed" is exactly vmcnt <= 2 tiles of copies.
// Otherwise page ids are per-lane vector loads and every tile waits for
// all outstanding copies (correct, shallower pipeline).
struct PrefillLds {
    alignas(16) uint8_t k[kPfStages][kTileBytes];
    alignas(16) uint8_t v[kPfStages][kTileBytes];
    // Key biases (0 or -inf) of partial tiles: the pipelined loop indexes
    // them by tile mod 8, the other loop by its ring stage.
    alignas(16) float b[2 * kPfStages][kPfMaxKeys];
    alignas(16) int full[kPfStages][kPfWaves];
    int arrive;  // pipelined loop: arrivals of the item's waves (see wait_arrivals)
    uint64_t pick[kPfWaves];  // chunk choice: each wave's best (cost, candidate)
    // The walk's index (num_seqs <= 64): sequence s's metadata, item count
    // and inclusive prefix of item counts.
    SeqMeta meta[kWave];
    int cnt[kWave];
    int incl[kWave];
};

// Item counts of the sequences held one per lane (lane s: sequence s), as
// seq_items.  A lane walking a long sequence's query blocks one after the
// other costs about 0.1 us per block (a dependent chain of integer and
// reciprocal arithmetic); when some sequence has more than 8 blocks the wave
// counts one sequence at a time instead, one block per lane, and sums
// across the lanes.  The counts are the same either way.
__device__ inline int wave_seq_items(const PrefillArgs& a, int chunk_len, const SeqMeta& m) {
    const int lane = __lane_id();
    const int64_t nb = query_blocks(a, m.n);
    if (a.max_chunks == 1 || __builtin_amdgcn_ballot_w64(nb > 8) == 0)
        return seq_items(a, chunk_len, m.n, m.start, m.ctx);
    int mine = 0;
    const int held = min(a.num_seqs, kWave);
    for (int s = 0; s < held; ++s) {
        const int64_t n = lane_value(m.n, s);
        if (n <= 0) continue;
        const int64_t start = lane_value(m.start, s), ctx = lane_value(m.ctx, s);
        const int64_t blocks = query_blocks(a, n);
        int part = 0;
        for (int64_t b = lane; b < blocks; b += kWave)
            part += chunks_of(chunk_len, block_kv_end(a, start, ctx, n, b * a.qb));
        const int total = lane_value(wave_incl_scan(part), kWave - 1);
        if (lane == s) mine = total;
    }
    return mine;
}

// The walk's index when every sequence fits one wave (num_seqs <= 64): lane
// s keeps sequence s's metadata, item count and inclusive prefix of counts,
// computed once per chunk length, so that a lookup is a ballot over the
// prefixes plus a lane-parallel search over the sequence's query blocks.
// walk_index returns the item total; wave 0 stores the index in LDS (read
// after the next barrier).
__device__ inline int walk_index(const PrefillArgs& a, int chunk_len, const SeqMeta& m, PrefillLds& lds,
                                int& cnt, int& incl) {
    const int lane = __lane_id();
    cnt = wave_seq_items(a, chunk_len, m);
    incl = wave_incl_scan(cnt);
    if (threadIdx.x < kWave) {
        lds.meta[lane] = m;
        lds.cnt[lane] = cnt;
        lds.incl[lane] = incl;
    }
    return lane_value(incl, kWave - 1);
}

// Lookup from the index values every wave holds in its lanes (lane s:
// sequence s's metadata, item count and inclusive prefix).
__device__ inline bool find_item_lanes(const PrefillArgs& a, int chunk_len, int total, const SeqMeta& m, int cnt,
                                       int incl_s, int item, PrefillItem& it) {
    if (item >= total) return false;
    const int lane = __lane_id();
    const int sel = __builtin_ctzll(__ballot(incl_s > item));
    int rem = item - (lane_value(incl_s, sel) - lane_value(cnt, sel));
    it.seq = sel;
    it.row0 = lane_value(m.row0, sel);
    it.qlen = lane_value(m.n, sel);
    it.start = lane_value(m.start, sel);
    it.ctx = lane_value(m.ctx, sel);
    it.chunk_len = chunk_len;
    // Query blocks from the last to the first (as find_item), 64 at a time:
    // lane l takes the l-th block of the group.  A sequence of one query
    // block (a short prefill chunk) has its chunks as its items.
    const int64_t nblocks = query_blocks(a, it.qlen);
    if (nblocks == 1) {
        it.q0 = 0;
        it.chunk = rem;
        it.kv_end = block_kv_end(a, it.start, it.ctx, it.qlen, 0);
        it.nchunks = lane_value(cnt, sel);
        return true;
    }
    for (int64_t g0 = 0; g0 < nblocks; g0 += kWave) {
        const int64_t bi = nblocks - 1 - (g0 + lane);
        int64_t e = 0;
        int nc = 0;
        if (bi >= 0) {
            e = block_kv_end(a, it.start, it.ctx, it.qlen, bi * a.qb);
            nc = chunks_of(chunk_len, e);
        }
        const int incl = wave_incl_scan(nc);
        const int group = lane_value(incl, kWave - 1);
        if (rem < group) {
            const int l = __builtin_ctzll(__ballot(incl > rem));
            it.q0 = (int)((nblocks - 1 - (g0 + l)) * a.qb);
            it.chunk = rem - (lane_value(incl, l) - lane_value(nc, l));
            it.kv_end = lane_value(e, l);
            it.nchunks = lane_value(nc, l);
            return true;
        }
        rem -= group;
    }
    return false;  // (only if the counts are inconsistent)
}

__device__ inline bool find_item_indexed(const PrefillArgs& a, int chunk_len, int total, const PrefillLds& lds,
                                         int item, PrefillItem& it) {
    const int lane = __lane_id();
    return find_item_lanes(a, chunk_len, total, lds.meta[lane], lds.cnt[lane], lds.incl[lane], item, it);
}


// One work item, computed by the whole work-group, in tiles of
// PfShape<HD>.  NARROW: head_dim is a multiple of 8 below HD; rows are
// zero-padded to HD in LDS (the copies skip the padded 16-byte chunks,
// which stay zero), the queries' padded dims are zero, and only head_dim
// output dims are stored.
template <typename T, int PAGES, bool NARROW, int HD, bool DENSE>
__device__ __attribute__((always_inline)) void prefill_item(const PrefillArgs& a, const PrefillItem& item,
                                                            PrefillLds& lds) {
    using SH = PfShape<HD>;
    constexpr bool SCALAR_PAGES = PAGES != kPagesPerLane;
    // The software-pipelined loop serves whole-tile pages of the 128 shape.
    constexpr bool PIPE = PAGES == kPagesPerTile && !NARROW && HD == 128 && !DENSE;
    const int hd = NARROW ? a.head_dim : SH::kD;  // elements per K/V/Q/output row in memory
    const int dchunks = hd / 8;                 // 16-byte chunks per row
    auto& sm_k = lds.k;
    auto& sm_v = lds.v;
    auto& sm_b = lds.b;
    auto& sm_full = lds.full;
    // The item is the same for every lane: keep it in scalar registers.
    // Context positions fit in 31 bits (table capacity <= 2^31 keys), and so
    // do the packed row index and query count (T*Hq < 2^31).
    const int seq = __builtin_amdgcn_readfirstlane(item.seq);
    const int q0 = __builtin_amdgcn_readfirstlane(item.q0);
    const int chunk = __builtin_amdgcn_readfirstlane(item.chunk);
    const int nchunks = __builtin_amdgcn_readfirstlane(item.nchunks);
    const int64_t kv_end64 = __builtin_amdgcn_readfirstlane((int)item.kv_end);
    const int64_t row0 = __builtin_amdgcn_readfirstlane((int)item.row0);
    const int qlen = __builtin_amdgcn_readfirstlane((int)item.qlen);
    const int64_t ctx = item.ctx;
    const int kvh = blockIdx.x % a.kv_heads;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int li = lane & 15;  // MFMA row / column index
    const int lg = lane >> 4;  // MFMA k-group (0..3)

    const int cap = a.table_width * a.block_size;
    // A row is valid only at positions in [0, cap); clamping start to
    // [-1, cap] keeps every row's validity and its position in 32 bits.
    const int start = __builtin_amdgcn_readfirstlane(
        (int)(item.start < -1 ? -1 : (item.start > cap ? (int64_t)cap : item.start)));
    // Dense mode has no table: every key of sequence seq is in page seq.
    constexpr bool ident = DENSE;
    const int64_t* table = ident ? nullptr : a.tables + (int64_t)seq * a.table_width;
    const int kv_end = (int)kv_end64;
    const int chunk_len = __builtin_amdgcn_readfirstlane(item.chunk_len);
    const int chunk_start = chunk * chunk_len;
    const int chunk_end = min(chunk_start + chunk_len, kv_end);
    const int t_begin = chunk_start / SH::kKeys;
    const int t_end = chunk_end > chunk_start ? (chunk_end + SH::kKeys - 1) / SH::kKeys : t_begin;

    // The SH::kNb 16-row column blocks of this wave.  Row r is token r % qb of
    // the block and head r / qb of the group; when the group does not divide
    // the tile's rows, those from qb * group on are idle (placed past the block's
    // tokens, so nothing reads or writes for them).
    int qi[SH::kNb], head[SH::kNb], pos[SH::kNb];
    bool row_ok[SH::kNb];
    int wave_last = -1, wave_first = 0x7fffffff;
    const int rows_used = a.qb * a.group;
#pragma unroll
    for (int nb = 0; nb < SH::kNb; ++nb) {
        const int r = wave * (16 * SH::kNb) + nb * 16 + li;
        const bool in_block = r < rows_used;
        qi[nb] = in_block ? q0 + r % a.qb : qlen;
        head[nb] = kvh * a.group + (in_block ? r / a.qb : 0);
        const int64_t p64 = (int64_t)start + qi[nb];
        row_ok[nb] = qi[nb] < qlen && start >= 0 && p64 < ctx && p64 < cap;
        pos[nb] = (int)p64;
        if (row_ok[nb]) {
            wave_last = max(wave_last, pos[nb]);
            wave_first = min(wave_first, pos[nb]);
        } else {
            pos[nb] = -1;
        }
    }
    // Wave maximum / minimum: the lanes of one MFMA row index li hold the
    // same rows, so lanes 0..15 cover every row of the wave: a reduction
    // inside one 16-lane DPP row (quad swaps, then the half-row and row
    // mirrors), read from lane 0.
    {
        int hi = wave_last, lo = wave_first;
        hi = max(hi, __builtin_amdgcn_update_dpp(0, hi, kDppQuadSwap1, 0xf, 0xf, false));
        lo = min(lo, __builtin_amdgcn_update_dpp(0, lo, kDppQuadSwap1, 0xf, 0xf, false));
        hi = max(hi, __builtin_amdgcn_update_dpp(0, hi, kDppQuadSwap2, 0xf, 0xf, false));
        lo = min(lo, __builtin_amdgcn_update_dpp(0, lo, kDppQuadSwap2, 0xf, 0xf, false));
        hi = max(hi, __builtin_amdgcn_update_dpp(0, hi, kDppRowHalfMirror, 0xf, 0xf, false));
        lo = min(lo, __builtin_amdgcn_update_dpp(0, lo, kDppRowHalfMirror, 0xf, 0xf, false));
        hi = max(hi, __builtin_amdgcn_update_dpp(0, hi, kDppRowMirror, 0xf, 0xf, false));
        lo = min(lo, __builtin_amdgcn_update_dpp(0, lo, kDppRowMirror, 0xf, 0xf, false));
        wave_last = __builtin_amdgcn_readfirstlane(hi);
        wave_first = __builtin_amdgcn_readfirstlane(lo);
    }


    // m_run: the row's reference (log2 units, -inf until the row sees a key);
    // nref = -m_run, or 0 while there is no reference (masked keys then give
    // 2^-inf = 0 rather than NaN).
    float m_run[SH::kNb], nref[SH::kNb], l_part[SH::kNb];
    f32x4 o[SH::kNb][SH::kDt];
#pragma unroll
    for (int nb = 0; nb < SH::kNb; ++nb) {
        m_run[nb] = kNegInf;
        nref[nb] = 0.f;
        l_part[nb] = 0.f;
#pragma unroll
        for (int dt = 0; dt < SH::kDt; ++dt) o[nb][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // Swizzled LDS offsets this lane reads (independent of the tile):
    // K chunk 4*dc + lg of row 16*kt + li, and the transposing V reads of
    // rows 32*c + 4*lg + li/4 (+16), dims 16*dt + 4*(li%4) .. +4.  K rows
    // store global chunk c in slot c ^ (row & 15); V rows in slot
    // c ^ (2*row & 15), so that the 16 lanes of a transposing read (4 rows x
    // 2 adjacent chunks) hit 8 different 16-byte bank groups.
    int koff[SH::kDc];
#pragma unroll
    for (int dc = 0; dc < SH::kDc; ++dc) koff[dc] = li * SH::kRowBytes + 16 * ((4 * dc + lg) ^ li);
    const int vrow = 4 * lg + (li >> 2);
    int voff[SH::kDt];
#pragma unroll
    for (int dt = 0; dt < SH::kDt; ++dt)
        voff[dt] = vrow * SH::kRowBytes + 16 * ((2 * dt + ((li & 3) >> 1)) ^ ((2 * vrow) & 15)) + 8 * (li & 1);

    // Copy plan: a tile's K (and V) is 16 instructions of 1 KiB; wave w issues
    // instructions j = SH::kIpw*w + i, each covering key rows 4j..4j+3 (lane ->
    // row 4j + lane/16, LDS slot lane%16 = global chunk (lane%16)^(row&15) for
    // K, (lane%16)^(2*row&15) for V).
    // Paged mode: the cache layout [pages, block_size, kv_heads, hd] (the
    // strides follow from the shapes, nothing more is held in registers).
    const int64_t row_bytes_g = DENSE ? a.kv_row_bytes : (int64_t)a.kv_heads * hd * 2;
    const int64_t page_bytes_g = DENSE ? a.kv_page_bytes : (int64_t)a.block_size * row_bytes_g;
    const int64_t head_bytes_g = DENSE ? a.kv_head_bytes : (int64_t)hd * 2;
    const uint8_t* kcache = static_cast<const uint8_t*>(a.key_cache) + kvh * head_bytes_g;
    const uint8_t* vcache = static_cast<const uint8_t*>(a.value_cache) + kvh * head_bytes_g;
    const int bs_shift = a.block_shift;
    const int lrow = lane / SH::kChunks;  // row inside the instruction's rows
    const int lslot = lane % SH::kChunks;  // LDS slot of the lane's 16 bytes in that row
    uint32_t tile_off[SH::kIpw], tile_off_v[SH::kIpw];  // per-lane byte offsets of whole-tile copies from row 0
    bool kchunk_ok[SH::kIpw], vchunk_ok[SH::kIpw];      // the lane's global chunk lies inside the row
#pragma unroll
    for (int i = 0; i < SH::kIpw; ++i) {
        const int row = SH::kRowsPerInst * (SH::kIpw * wave + i) + lrow;
        const int kc = lslot ^ (row & 15), vc = lslot ^ ((2 * row) & 15);
        kchunk_ok[i] = !NARROW || kc < dchunks;
        vchunk_ok[i] = !NARROW || vc < dchunks;
        tile_off[i] = (uint32_t)(row * row_bytes_g) + 16u * (uint32_t)(kchunk_ok[i] ? kc : 0);
        tile_off_v[i] = (uint32_t)(row * row_bytes_g) + 16u * (uint32_t)(vchunk_ok[i] ? vc : 0);
    }

    // The table is read-only here: reading it through the constant address
    // space lets wave-uniform lookups become scalar loads.
    typedef __attribute__((address_space(4))) const int64_t const_i64;
    const const_i64* ctable = (const const_i64*)table;
    auto page_at = [&](int key) -> int {
        const int kc = key < cap ? key : cap - 1;
        const int idx = bs_shift >= 0 ? kc >> bs_shift : kc / a.block_size;
        const int64_t page = ident ? seq : ctable[idx];
        return (key < chunk_end && page >= 0 && page < a.num_blocks) ? (int)page : -1;
    };
    // Page-per-tile mode: the page ids of a window of 64 consecutive tiles,
    // one per lane (lane j: tile tile_base + j; -1 when absent or past the
    // chunk), read with readlane -- the tile loop never waits for a table
    // lookup.  The next window is loaded one window ahead (right after the
    // copies that follow a switch), so by its first use a barrier's full wait
    // has retired it.  Windows start at t_begin + 64 k: both tiles of a pair
    // lie in one window.
    // Raw table entries are kept (validated at use), so that nothing waits for
    // the window's load before the tile loop needs it.
    int tile_base = t_begin;
    int64_t tile_pages = -1, next_pages = -1;
    auto window_pages = [&](int base) -> int64_t {
        const int key0 = (base + lane) * SH::kKeys;
        int64_t raw = -1;
        if (key0 < chunk_end) raw = ident ? seq : table[key0 >> bs_shift];
        return raw;
    };
    auto page_of_tile = [&](int tile) -> int {
        const int64_t page = lane_value(tile_pages, tile - tile_base);
        return (page >= 0 && page < a.num_blocks) ? (int)page : -1;
    };
    if constexpr (PAGES == kPagesPerTile) tile_pages = window_pages(t_begin);
    // Bit st: the tile in ring stage st lies in one present page with all of
    // its 64 keys in the chunk (set by every wave when it issues the copies).
    uint32_t full_stages = 0;
    int pg_next[SH::kIpw];  // pages for the next tile to issue
    auto lookup = [&](int tile) {
        if constexpr (PAGES == kPagesPerTile) {
            const int pg = page_of_tile(tile);
#pragma unroll
            for (int i = 0; i < SH::kIpw; ++i) pg_next[i] = pg;
        } else {
#pragma unroll
            for (int i = 0; i < SH::kIpw; ++i) {
                const int row = SH::kRowsPerInst * (SH::kIpw * wave + i) + (SCALAR_PAGES ? 0 : lrow);
                pg_next[i] = page_at(tile * SH::kKeys + row);
            }
        }
    };
    auto issue = [&](int tile, int st) {
        if constexpr (PAGES == kPagesPerTile) {
            const int key0 = tile * SH::kKeys;
            const bool full = pg_next[0] >= 0 && key0 + SH::kKeys - 1 < chunk_end;
            full_stages = full ? (full_stages | (1u << st)) : (full_stages & ~(1u << st));
            if (full) {
                // Full tile in one page: one scalar base for all copies.
                const int64_t base =
                    (int64_t)pg_next[0] * page_bytes_g + (int64_t)(key0 & (a.block_size - 1)) * row_bytes_g;
                const uint32_t lk = lds_addr(&sm_k[st][0]), lv = lds_addr(&sm_v[st][0]);
#pragma unroll
                for (int i = 0; i < SH::kIpw; ++i) {
                    const int j = SH::kIpw * wave + i;
                    if (kchunk_ok[i]) lds_dma16_s(kcache + base, tile_off[i], lk + 1024 * j);
                    if (vchunk_ok[i]) lds_dma16_s(vcache + base, tile_off_v[i], lv + 1024 * j);
                }
                return;
            }
        }
        bool all_ok = true;
#pragma unroll
        for (int i = 0; i < SH::kIpw; ++i) {
            const int j = SH::kIpw * wave + i;
            const int row = SH::kRowsPerInst * j + lrow;
            const int key = tile * SH::kKeys + row;
            const int cidx = lslot ^ (row & 15);
            const int cidx_v = lslot ^ ((2 * row) & 15);
            const int page = pg_next[i];
            // Rows past the chunk inside a valid first-row page are masked too.
            const bool ok = page >= 0 && key < chunk_end;
            all_ok = all_ok && ok;
            const uint8_t* gk = reinterpret_cast<const uint8_t*>(kZeroChunk);
            const uint8_t* gv = gk;
            if (ok) {
                const int in_page = bs_shift >= 0 ? key & (a.block_size - 1) : key % a.block_size;
                const int64_t off = (int64_t)page * page_bytes_g + (int64_t)in_page * row_bytes_g;
                // Padded chunks of narrow rows copy zeros.
                if (!NARROW || cidx < dchunks) gk = kcache + off + 16 * cidx;
                if (!NARROW || cidx_v < dchunks) gv = vcache + off + 16 * cidx_v;
            }
            lds_dma16(gk, lds_addr(&sm_k[st][0]) + 1024 * j);
            lds_dma16(gv, lds_addr(&sm_v[st][0]) + 1024 * j);
            if (lslot == 0) sm_b[st][row] = ok ? 0.f : kNegInf;
        }
        const bool wave_full = __builtin_amdgcn_ballot_w64(!all_ok) == 0;
        if (lane == 0) sm_full[st][wave] = wave_full ? 1 : 0;
    };

    // Q^T operands: row (nb, li), d = 32*dc + 8*lg .. +8.  Their latency
    // overlaps the first pair's copies: the first pair barrier waits for the
    // whole vector-memory counter.
    u32x4 qop[SH::kNb][SH::kDc];
#pragma unroll
    for (int nb = 0; nb < SH::kNb; ++nb) {
        const uint16_t* qrow = static_cast<const uint16_t*>(a.q) +
                               (DENSE ? seq * a.q_seq + (row0 + qi[nb]) * a.q_tok + head[nb] * a.q_head
                                      : ((row0 + qi[nb]) * a.q_heads + head[nb]) * hd);
#pragma unroll
        for (int dc = 0; dc < SH::kDc; ++dc) {
            qop[nb][dc] = u32x4{0u, 0u, 0u, 0u};
            if (row_ok[nb] && (!NARROW || 32 * dc + 8 * lg < hd))
                qop[nb][dc] = *reinterpret_cast<const u32x4*>(qrow + 32 * dc + 8 * lg);
        }
    }

    // Dense mode: output row offsets (elements), formed here so that the
    // layout's strides are not held in scalar registers across the tile loop.
    int64_t out_off[SH::kNb];
#pragma unroll
    for (int nb = 0; nb < SH::kNb; ++nb)
        out_off[nb] = DENSE ? seq * a.o_seq + (row0 + qi[nb]) * a.o_tok + head[nb] * a.o_head : 0;

    // Row sums accumulated on the matrix core (pipelined loop only): a
    // block of ones times P^T gives every lane its row's full sum.
    f32x4 osum[SH::kNb];
#pragma unroll
    for (int nb = 0; nb < SH::kNb; ++nb) osum[nb] = f32x4{0.f, 0.f, 0.f, 0.f};

    if constexpr (PIPE) {
        // Software-pipelined tile loop.  Step i computes S^T of tile i+1,
        // then O^T += V^T P^T of tile i, then the probabilities of tile
        // i+1, so each wave's products of two tiles run back to back and the
        // softmax of one tile follows the products of the previous one.  K
        // is therefore needed one tile before V: the K copies run one tile
        // ahead of the V copies, both in 4-stage rings (tile i: K and V
        // stage i mod 4, i counted from t_begin).
        //
        // The queries are pre-scaled by scale*log2(e) and each score product
        // starts from the row's -reference (the MFMA's C input), so a
        // probability is one exp2 of the product.
        const u32x4 ones = {T::pack(1.f, 1.f), T::pack(1.f, 1.f), T::pack(1.f, 1.f), T::pack(1.f, 1.f)};
        const int ntiles = t_end - t_begin;
        f32x4 sc[SH::kHalves][SH::kNb][2];
        u32x4 pops[SH::kHalves][SH::kNb];
        // Per lane j: byte offset (from the kv head's base) of tile
        // tile_base + j's first key row when the tile is whole (present page,
        // all of its keys in the chunk), else -1.
        int64_t tile_offs = -1;
        auto window_offsets = [&](int64_t raw, int base) -> int64_t {
            const int key0 = (base + lane) * SH::kKeys;
            const bool whole = raw >= 0 && raw < a.num_blocks && key0 + SH::kKeys <= chunk_end;
            return whole ? raw * page_bytes_g + (int64_t)(key0 & (a.block_size - 1)) * row_bytes_g : (int64_t)-1;
        };
        // Moves to the next window (loaded a window ago, retired by a landed
        // barrier's full wait since) and loads the one after it.  Called at
        // one place per issue phase: two consecutive tiles never both cross
        // a window boundary, and a second call site would read the load the
        // first one just issued.
        auto next_window = [&]() {
            tile_pages = next_pages;
            tile_base += kWave;
            tile_offs = window_offsets(tile_pages, tile_base);
            if (tile_base + kWave < t_end) next_pages = window_pages(tile_base + kWave);
        };
        // Row-by-row copies of a tile that is not whole: absent rows load
        // zeros (finite in both rings) and, for K, get a -inf bias.
        auto issue_rows = [&](int tile, int st, bool is_k) {
            const int key0 = tile * SH::kKeys;
            const int64_t page = ctable[(key0 < cap ? key0 : cap - 1) >> bs_shift];
            const bool pg_ok = key0 < chunk_end && page >= 0 && page < a.num_blocks;
            const int64_t base = pg_ok ? page * page_bytes_g : 0;
            const uint8_t* cache = is_k ? kcache : vcache;
            const uint32_t lds0 = lds_addr(is_k ? &sm_k[st][0] : &sm_v[st][0]);
#pragma unroll
            for (int i = 0; i < SH::kIpw; ++i) {
                const int j = SH::kIpw * wave + i;
                const int row = SH::kRowsPerInst * j + lrow;
                const int key = key0 + row;
                const int cidx = is_k ? lslot ^ (row & 15) : lslot ^ ((2 * row) & 15);
                const bool ok = pg_ok && key < chunk_end;
                const uint8_t* g = reinterpret_cast<const uint8_t*>(kZeroChunk);
                if (ok) g = cache + base + (int64_t)(key & (a.block_size - 1)) * row_bytes_g + 16 * cidx;
                lds_dma16(g, lds0 + 1024 * j);
                if (is_k && lslot == 0) sm_b[(tile - t_begin) & (2 * kPfStages - 1)][row] = ok ? 0.f : kNegInf;
            }
        };
        auto issue_k = [&](int tile, int st, int64_t off) {
            if (off >= 0) {
                full_stages |= 1u << st;
                const uint32_t lk = lds_addr(&sm_k[st][0]);
#pragma unroll
                for (int i = 0; i < SH::kIpw; ++i) lds_dma16_s(kcache + off, tile_off[i], lk + 1024 * (SH::kIpw * wave + i));
            } else {
                full_stages &= ~(1u << st);
                issue_rows(tile, st, true);
            }
        };
        auto issue_v = [&](int tile, int st, int64_t off) {
            if (off >= 0) {
                const uint32_t lv = lds_addr(&sm_v[st][0]);
#pragma unroll
                for (int i = 0; i < SH::kIpw; ++i)
                    lds_dma16_s(vcache + off, tile_off_v[i], lv + 1024 * (SH::kIpw * wave + i));
            } else {
                issue_rows(tile, st, false);
            }
        };
        // S^T of a tile (K stage st), starting from -reference.
        auto s_product = [&](int st) __attribute__((always_inline)) {
            const uint8_t* smk = &sm_k[st][0];
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int h = 0; h < SH::kHalves; ++h) {
                u32x4 kop[2][SH::kDc];
#pragma unroll
                for (int dc = 0; dc < SH::kDc; ++dc) {
                    kop[0][dc] = *reinterpret_cast<const u32x4*>(smk + 32 * h * SH::kRowBytes + koff[dc]);
                    kop[1][dc] = *reinterpret_cast<const u32x4*>(smk + (32 * h + 16) * SH::kRowBytes + koff[dc]);
                }
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                    for (int nb = 0; nb < SH::kNb; ++nb) {
                        f32x4 c = {nref[nb], nref[nb], nref[nb], nref[nb]};
#pragma unroll
                        for (int dc = 0; dc < SH::kDc; ++dc) c = T::mfma16x16x32(kop[kk][dc], qop[nb][dc], c);
                        sc[h][nb][kk] = c;
                        __builtin_amdgcn_sched_barrier(0);  // keep the chain contiguous
                    }
            }
            __builtin_amdgcn_s_setprio(0);
        };
        // O^T += V^T P^T of a tile (V stage st), and the row sums.
        auto pv_product = [&](int st) __attribute__((always_inline)) {
            typedef __attribute__((address_space(3))) uint8_t lds_u8;
            lds_u8* vbase = (lds_u8*)&sm_v[st][0];
            auto vread = [&](int dt, u32x4 (&vop)[SH::kHalves]) __attribute__((always_inline)) {
#pragma unroll
                for (int h = 0; h < SH::kHalves; ++h) {
                    const s16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_s16x4*)(vbase + 32 * h * SH::kRowBytes + voff[dt]));
                    const s16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_s16x4*)(vbase + (32 * h + 16) * SH::kRowBytes + voff[dt]));
                    const u32x2 w0 = __builtin_bit_cast(u32x2, t0);
                    const u32x2 w1 = __builtin_bit_cast(u32x2, t1);
                    vop[h] = u32x4{w0[0], w0[1], w1[0], w1[1]};
                }
            };
            __builtin_amdgcn_s_setprio(1);
            u32x4 vcur[SH::kHalves], vnext[SH::kHalves];
            vread(0, vcur);
#pragma unroll
            for (int dt = 0; dt < SH::kDt; ++dt) {
                if (dt + 1 < SH::kDt) vread(dt + 1, vnext);
#pragma unroll
                for (int nb = 0; nb < SH::kNb; ++nb) {
#pragma unroll
                    for (int h = 0; h < SH::kHalves; ++h) o[nb][dt] = T::mfma16x16x32(vcur[h], pops[h][nb], o[nb][dt]);
                    __builtin_amdgcn_sched_barrier(0);  // keep the products back to back
                }
#pragma unroll
                for (int h = 0; h < SH::kHalves; ++h) vcur[h] = vnext[h];
            }
#pragma unroll
            for (int nb = 0; nb < SH::kNb; ++nb) {
#pragma unroll
                for (int h = 0; h < SH::kHalves; ++h) osum[nb] = T::mfma16x16x32(ones, pops[h][nb], osum[nb]);
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_s_setprio(0);
        };
        // Probabilities of a tile whose S^T is in sc (K stage st): masked and
        // biased first unless every key is present and visible to every row
        // of the wave.  p = 2^sc; the exact step (row maxima, rescale of what
        // is accumulated, new probabilities) runs when a row sees its first
        // key or some probability, rounded to the operand type, exceeds 2^8
        // (inf and NaN included: as 16-bit patterns of non-negative values
        // they order above 256, so an unsigned maximum of the packed halves
        // decides).  `first`:
        // the item's first tile, where nothing is accumulated yet (every
        // rescale factor is 1, so the rescale is skipped).
        auto softmax_tile = [&](int tile, int st, bool first) __attribute__((always_inline)) {
            const int tile0 = tile * SH::kKeys;
            const bool full = ((full_stages >> st) & 1u) != 0;
            const bool fast = full && tile0 + SH::kKeys - 1 <= wave_first;
            const float* smb = &sm_b[(tile - t_begin) & (2 * kPfStages - 1)][0];
            if (!fast) {
#pragma unroll
                for (int h = 0; h < SH::kHalves; ++h)
#pragma unroll
                    for (int nb = 0; nb < SH::kNb; ++nb) {
                        const int lim = pos[nb] - tile0 - 32 * h - 4 * lg;  // key (16*kk + j) must be <= lim
#pragma unroll
                        for (int kk = 0; kk < 2; ++kk) {
                            const f32x4 bias = full ? f32x4{0.f, 0.f, 0.f, 0.f}
                                                    : *reinterpret_cast<const f32x4*>(&smb[32 * h + 16 * kk + 4 * lg]);
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                                sc[h][nb][kk][j] = 16 * kk + j > lim ? kNegInf : sc[h][nb][kk][j] + bias[j];
                        }
                    }
            }
            bool need = false;
#pragma unroll
            for (int nb = 0; nb < SH::kNb; ++nb) need = need | ((m_run[nb] == kNegInf) & (pos[nb] >= tile0));
#pragma unroll
            for (int h = 0; h < SH::kHalves; ++h)
#pragma unroll
                for (int nb = 0; nb < SH::kNb; ++nb) {
                    float p[8];
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                        for (int j = 0; j < 4; ++j) p[4 * kk + j] = fast_exp2(sc[h][nb][kk][j]);
                    pops[h][nb] = u32x4{T::pack(p[0], p[1]), T::pack(p[2], p[3]), T::pack(p[4], p[5]), T::pack(p[6], p[7])};
                    {
                        typedef unsigned short us2 __attribute__((ext_vector_type(2)));
                        us2 m = __builtin_elementwise_max(__builtin_bit_cast(us2, pops[h][nb][0]),
                                                          __builtin_bit_cast(us2, pops[h][nb][1]));
                        m = __builtin_elementwise_max(m, __builtin_bit_cast(us2, pops[h][nb][2]));
                        m = __builtin_elementwise_max(m, __builtin_bit_cast(us2, pops[h][nb][3]));
                        const uint32_t lim = T::pack(kPSumLimit, 0.f) & 0xffffu;
                        need = need | ((uint32_t)max(m.x, m.y) > lim);
                    }
                }
            if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
                for (int nb = 0; nb < SH::kNb; ++nb) {
                    float r = kNegInf;
#pragma unroll
                    for (int h = 0; h < SH::kHalves; ++h)
#pragma unroll
                        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                            for (int j = 0; j < 4; ++j) r = fmaxf(r, sc[h][nb][kk][j] - nref[nb]);
                    const float mn = fmaxf(m_run[nb], row4_max(r));
                    const float alpha = (m_run[nb] == kNegInf || mn == kNegInf) ? 1.f : fast_exp2(m_run[nb] - mn);
                    const float shift = mn == kNegInf ? 0.f : nref[nb] + mn;
                    m_run[nb] = mn;
                    nref[nb] = mn == kNegInf ? 0.f : -mn;
                    if (!first) {
                        osum[nb] *= alpha;
#pragma unroll
                        for (int dt = 0; dt < SH::kDt; ++dt) o[nb][dt] *= alpha;
                    }
#pragma unroll
                    for (int h = 0; h < SH::kHalves; ++h) {
                        float p[8];
#pragma unroll
                        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                            for (int j = 0; j < 4; ++j) p[4 * kk + j] = fast_exp2(sc[h][nb][kk][j] - shift);
                        pops[h][nb] =
                            u32x4{T::pack(p[0], p[1]), T::pack(p[2], p[3]), T::pack(p[4], p[5]), T::pack(p[6], p[7])};
                    }
                }
            }
        };

        // Split barrier of the loop.  A wave arrives (one LDS count) once its
        // copies issued at the top of the pair have landed and its LDS
        // reads of the pair's last products have returned; at the top of
        // the next pair it waits for all arrivals.  Between the two it runs
        // its last softmax, so waves may drift apart by that much without
        // waiting (a work-group barrier per pair keeps them in lockstep,
        // and the two waves of a SIMD then contend for the matrix core and
        // the vector ALU at the same moments).  The wait is bounded: past
        // the bound the wave goes on (never reached while every wave runs
        // the loop, which always arrives).
        auto arrive_pair = [&]() {
            wait_vmcnt_all();  // this wave's copies and LDS reads complete
            asm volatile("" : : : "memory");
            if (lane == 0) __hip_atomic_fetch_add(&lds.arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        };
        auto wait_arrivals = [&](int target) {
            for (int spin = 0; spin < kArriveSpinLimit; ++spin) {
                const int n = __builtin_amdgcn_readfirstlane(
                    __hip_atomic_load(&lds.arrive, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
                if (n >= target) break;
                __builtin_amdgcn_s_sleep(1);
            }
            asm volatile("" : : : "memory");  // no LDS access or copy moves above the wait
        };

        // Step i: S^T of tile i+1, O^T += V^T P^T of tile i (step 0: done
        // in the prologue), then the probabilities of tile i+1 (products
        // skipped for tiles past the wave's last visible key).  `last`: the
        // pair's second step, which arrives after its products.
        auto step = [&](int i, bool pv, bool last) __attribute__((always_inline)) {
            const int tile = t_begin + i;
            const bool next_vis = i + 1 < ntiles && (tile + 1) * SH::kKeys <= wave_last;
            if (next_vis) s_product((i + 1) & (kPfStages - 1));
            if (pv && tile * SH::kKeys <= wave_last) pv_product(i & (kPfStages - 1));
            if (last) arrive_pair();
            if (next_vis) softmax_tile(tile + 1, (i + 1) & (kPfStages - 1), false);
        };

        if (ntiles > 0) {
            // Prologue: K and V of tile 0 (its page by a scalar lookup: the
            // window's vector load is first needed after the barrier) land
            // with the queries; tile 0 is then computed whole while K of
            // tiles 1, 2 and V of tile 1 are in flight.
            const int key0 = t_begin * SH::kKeys;
            const int64_t page0 = ctable[key0 >> bs_shift];
            const bool whole0 = key0 + SH::kKeys <= chunk_end && page0 >= 0 && page0 < a.num_blocks;
            const int64_t off0 =
                whole0 ? page0 * page_bytes_g + (int64_t)(key0 & (a.block_size - 1)) * row_bytes_g : (int64_t)-1;
            issue_k(t_begin, 0, off0);
            issue_v(t_begin, 0, off0);
            if (t_begin + kWave < t_end) next_pages = window_pages(t_begin + kWave);
            if (threadIdx.x == 0) lds.arrive = 0;  // no wave counts before the next barrier
            landed_barrier();
            tile_offs = window_offsets(tile_pages, tile_base);
            int64_t pend = -1;  // offset of the last K tile issued, whose V is still to come
            if (ntiles > 1) {  // tiles 1 and 2 lie in the first window
                const int64_t off1 = lane_value(tile_offs, 1);
                issue_k(t_begin + 1, 1, off1);
                if (ntiles > 2) {
                    pend = lane_value(tile_offs, 2);
                    issue_k(t_begin + 2, 2, pend);
                }
                issue_v(t_begin + 1, 1, off1);
            }
            // Queries scaled by scale*log2(e) (they landed at the barrier).
#pragma unroll
            for (int nb = 0; nb < SH::kNb; ++nb)
#pragma unroll
                for (int dc = 0; dc < SH::kDc; ++dc)
#pragma unroll
                    for (int w = 0; w < 4; ++w)
                        qop[nb][dc][w] = T::pack(T::lo(qop[nb][dc][w]) * a.scale_log2, T::hi(qop[nb][dc][w]) * a.scale_log2);
            if (key0 <= wave_last) {
                s_product(0);
                softmax_tile(t_begin, 0, true);
            }
            // The prologue's arrival: this wave's copies of K 1, 2 and V 1
            // have landed and its reads of K 0 are done.  Tile 0's O^T
            // product follows, so the first pair waits for no wave's O^T
            // (V 0's stage is next refilled two pairs on).
            arrive_pair();
            if (key0 <= wave_last) pv_product(0);
            // Pairs of steps (i0, i0+1), i0 even: the arrivals at the top
            // (the prologue's for the first pair, then the previous pair's)
            // publish K of i0+1, i0+2 and V of i0, i0+1; then the copies of
            // K i0+3, i0+4 and V i0+2, i0+3 go out: their stages were last
            // read by products that every wave finished before arriving.  Partial-tile biases are written at
            // issue time into slot tile mod 8: K i0+4's bias then replaces
            // tile i0-4's, not tile i0's (read by softmax i0, which a wave
            // runs after its arrival).
            for (int i0 = 0; i0 < ntiles; i0 += 2) {
                wait_arrivals(kPfWaves * (i0 / 2 + 1));
                if (i0 + 2 < ntiles) {
                    int64_t off3 = -1, off4 = -1;
                    if (i0 + 3 < ntiles) {
                        const int t3 = t_begin + i0 + 3, last = i0 + 4 < ntiles ? t3 + 1 : t3;
                        const int base0 = tile_base;
                        if (t3 < base0 + kWave) off3 = lane_value(tile_offs, t3 - base0);
                        if (last >= base0 + kWave) next_window();
                        if (t3 >= base0 + kWave) off3 = lane_value(tile_offs, t3 - tile_base);
                        if (i0 + 4 < ntiles) off4 = lane_value(tile_offs, t3 + 1 - tile_base);
                        issue_k(t3, (i0 + 3) & (kPfStages - 1), off3);
                    }
                    if (i0 + 4 < ntiles) issue_k(t_begin + i0 + 4, (i0 + 4) & (kPfStages - 1), off4);
                    issue_v(t_begin + i0 + 2, (i0 + 2) & (kPfStages - 1), pend);
                    if (i0 + 3 < ntiles) issue_v(t_begin + i0 + 3, (i0 + 3) & (kPfStages - 1), off3);
                    pend = off4;
                }
                step(i0, i0 > 0, false);
                if (i0 + 1 < ntiles) step(i0 + 1, true, true);
            }
        }
    } else {
    // Prologue: only the first tile in flight, so the first products wait
    // for the queries and one tile; the pairs that follow are (t, t+1) with
    // t - t_begin odd, each issued one pair ahead.
    if (t_begin < t_end) {
        if constexpr (PAGES == kPagesPerTile) {
            // A scalar lookup: the window's vector load is first needed after
            // the first barrier, so nothing waits for it (or for the queries)
            // before these copies go out.
            const int key0 = t_begin * SH::kKeys;
            const int64_t page = ident ? seq : ctable[key0 >> bs_shift];
            const int pg = (key0 < chunk_end && page >= 0 && page < a.num_blocks) ? (int)page : -1;
#pragma unroll
            for (int i = 0; i < SH::kIpw; ++i) pg_next[i] = pg;
        } else {
            lookup(t_begin);
        }
        issue(t_begin, 0);
    }
    if constexpr (PAGES == kPagesPerTile)
        if (t_begin + kWave < t_end) next_pages = window_pages(t_begin + kWave);
    for (int tp = t_begin - 1; tp < t_end; tp += 2) {
        const int st0 = (tp - t_begin) & (kPfStages - 1);
        // Both tiles of the pair have landed (this lane's copies, then every
        // lane's through the barrier), and every wave is done with the
        // previous pair, whose stages the copies below refill.
        landed_barrier();
        bool switched = false;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int tile = tp + 2 + k;
            if (tile < t_end) {  // stages of tiles past the chunk are never read
                if constexpr (PAGES == kPagesPerTile) {
                    // The next window was loaded a window ago; the barrier's
                    // full wait has retired it.
                    if (tile >= tile_base + kWave) {
                        tile_pages = next_pages;
                        tile_base += kWave;
                        switched = true;
                    }
                }
                lookup(tile);
                issue(tile, (st0 + 2 + k) & (kPfStages - 1));
            }
        }
        if constexpr (PAGES == kPagesPerTile)
            if (switched && tile_base + kWave < t_end) next_pages = window_pages(tile_base + kWave);
        // Unrolled: with this loop left rolled, the compiler's wait insertion
        // puts a full vmcnt(0) at its head (before the first product of every
        // tile), and that wait also covers the copies issued just above, so
        // each pair of tiles would wait for the next pair to land.
#pragma unroll
        for (int k = 0; k < 2 && tp + k < t_end; ++k) {
            const int tile = tp + k;
            if (tile < t_begin) continue;  // the prologue's virtual first slot
            const int st = (st0 + k) & (kPfStages - 1);
            const int tile0 = tile * SH::kKeys;
            if (tile0 <= wave_last) {
                const uint8_t* smk = &sm_k[st][0];
                const float* smb = &sm_b[st][0];
                // Every key of the tile present and visible to every row of the
                // wave: no bias and no causal mask needed.
                bool full;
                if constexpr (PAGES == kPagesPerTile) {
                    full = ((full_stages >> st) & 1u) != 0;
                } else {
                    static_assert(kPfWaves == 8, "two int4 flag reads below");
                    const int4 fa = *reinterpret_cast<const int4*>(&sm_full[st][0]);
                    const int4 fb = *reinterpret_cast<const int4*>(&sm_full[st][4]);
                    full = (fa.x & fa.y & fa.z & fa.w & fb.x & fb.y & fb.z & fb.w) != 0;
                }
                const bool fast = full && tile0 + SH::kKeys - 1 <= wave_first;
                typedef __attribute__((address_space(3))) uint8_t lds_u8;
                lds_u8* vbase = (lds_u8*)&sm_v[st][0];
                // Two halves of 32 keys: S^T -> probabilities each, then
                // O^T += V^T P^T over the whole tile, two products back to back
                // per accumulator.
                u32x4 pops[SH::kHalves][SH::kNb];
#pragma unroll
                for (int h = 0; h < SH::kHalves; ++h) {
                    // S^T = K Q^T for key sub-tiles 2h, 2h+1: 8 independent accumulators.
                    f32x4 sc[SH::kNb][2];
#pragma unroll
                    for (int nb = 0; nb < SH::kNb; ++nb) sc[nb][0] = sc[nb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
                    // Each accumulator takes its four products back to back: the
                    // matrix core forwards a result straight into the next
                    // product of the same accumulator, while alternating between
                    // accumulators costs issue slots.
                    // Raised wave priority over the matrix products: while a wave
                    // issues MFMAs, the other wave of its SIMD runs softmax VALU
                    // work in the gaps rather than competing for the same slots.
                    __builtin_amdgcn_s_setprio(1);
                    u32x4 kop[2][SH::kDc];
#pragma unroll
                    for (int dc = 0; dc < SH::kDc; ++dc) {
                        kop[0][dc] = *reinterpret_cast<const u32x4*>(smk + 32 * h * SH::kRowBytes + koff[dc]);
                        kop[1][dc] = *reinterpret_cast<const u32x4*>(smk + (32 * h + 16) * SH::kRowBytes + koff[dc]);
                    }
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                        for (int nb = 0; nb < SH::kNb; ++nb) {
#pragma unroll
                            for (int dc = 0; dc < SH::kDc; ++dc)
                                sc[nb][kk] = T::mfma16x16x32(kop[kk][dc], qop[nb][dc], sc[nb][kk]);
                            __builtin_amdgcn_sched_barrier(0);  // keep the chain contiguous
                        }
                    // Scores -> probabilities against the running reference m_run.
                    // Fast tiles keep raw scores and scale inside the exponent;
                    // edge tiles are scaled, biased and masked in place first.
                    __builtin_amdgcn_s_setprio(0);
                    if (!fast) {
#pragma unroll
                        for (int nb = 0; nb < SH::kNb; ++nb) {
                            const int lim = pos[nb] - tile0 - 32 * h - 4 * lg;  // key (16*kk + j) must be <= lim
#pragma unroll
                            for (int kk = 0; kk < 2; ++kk) {
                                // Full tiles leave the bias unwritten: every key row is present.
                                const f32x4 bias = full ? f32x4{0.f, 0.f, 0.f, 0.f}
                                                        : *reinterpret_cast<const f32x4*>(&smb[32 * h + 16 * kk + 4 * lg]);
#pragma unroll
                                for (int j = 0; j < 4; ++j) {
                                    const float v = sc[nb][kk][j] * a.scale_log2 + bias[j];
                                    sc[nb][kk][j] = 16 * kk + j > lim ? kNegInf : v;
                                }
                            }
                        }
                    }
                    const float mult = fast ? a.scale_log2 : 1.f;
                    // No row maximum on the common path: the reference only has to
                    // keep every probability small, which the sum of a lane's
                    // probabilities checks after the fact (inf and NaN included).
                    float p[SH::kNb][8], dl[SH::kNb];
                    bool need = false;
#pragma unroll
                    for (int nb = 0; nb < SH::kNb; ++nb) {
#pragma unroll
                        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                            for (int j = 0; j < 4; ++j)
                                p[nb][4 * kk + j] = fast_exp2(fmaf(sc[nb][kk][j], mult, nref[nb]));
                        dl[nb] = ((p[nb][0] + p[nb][1]) + (p[nb][2] + p[nb][3])) +
                                 ((p[nb][4] + p[nb][5]) + (p[nb][6] + p[nb][7]));
                        // A row without a reference yet needs one as soon as it
                        // sees a key (key 32h of the tile is at or before its position).
                        need = need | !(dl[nb] <= kPSumLimit) | ((m_run[nb] == kNegInf) & (pos[nb] >= tile0 + 32 * h));
                    }
                    if (__builtin_amdgcn_ballot_w64(need)) {
                        // Exact step: row maxima over the 4 lanes of each row,
                        // rescale what is accumulated, recompute the probabilities.
#pragma unroll
                        for (int nb = 0; nb < SH::kNb; ++nb) {
                            float r = kNegInf;
#pragma unroll
                            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                                for (int j = 0; j < 4; ++j) r = fmaxf(r, sc[nb][kk][j] * mult);
                            const float mn = fmaxf(m_run[nb], row4_max(r));
                            const float alpha = mn == kNegInf ? 1.f : fast_exp2(m_run[nb] - mn);
                            m_run[nb] = mn;
                            l_part[nb] *= alpha;
#pragma unroll
                            for (int dt = 0; dt < SH::kDt; ++dt) o[nb][dt] *= alpha;
                            if (h == 1) {
                                // The first half's products are still to be accumulated.
#pragma unroll
                                for (int w = 0; w < 4; ++w)
                                    pops[0][nb][w] =
                                        T::pack(T::lo(pops[0][nb][w]) * alpha, T::hi(pops[0][nb][w]) * alpha);
                            }
                            nref[nb] = mn == kNegInf ? 0.f : -mn;
#pragma unroll
                            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                                for (int j = 0; j < 4; ++j)
                                    p[nb][4 * kk + j] = fast_exp2(fmaf(sc[nb][kk][j], mult, nref[nb]));
                            dl[nb] = ((p[nb][0] + p[nb][1]) + (p[nb][2] + p[nb][3])) +
                                     ((p[nb][4] + p[nb][5]) + (p[nb][6] + p[nb][7]));
                        }
                    }
                    // Packed as the B operand of the PV products:
                    // k-slot 4*kk + j <-> key 32h + 16kk + 4*lg + j.
#pragma unroll
                    for (int nb = 0; nb < SH::kNb; ++nb) {
                        l_part[nb] += dl[nb];
                        pops[h][nb] = u32x4{T::pack(p[nb][0], p[nb][1]), T::pack(p[nb][2], p[nb][3]),
                                            T::pack(p[nb][4], p[nb][5]), T::pack(p[nb][6], p[nb][7])};
                    }
                }
                // O^T += V^T P^T over the tile; V^T operands by transposing reads,
                // one dim block ahead of the products that use them.
                auto vread = [&](int dt, u32x4 (&vop)[SH::kHalves]) __attribute__((always_inline)) {
#pragma unroll
                    for (int h = 0; h < SH::kHalves; ++h) {
                        const s16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (lds_s16x4*)(vbase + 32 * h * SH::kRowBytes + voff[dt]));
                        const s16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (lds_s16x4*)(vbase + (32 * h + 16) * SH::kRowBytes + voff[dt]));
                        const u32x2 w0 = __builtin_bit_cast(u32x2, t0);
                        const u32x2 w1 = __builtin_bit_cast(u32x2, t1);
                        vop[h] = u32x4{w0[0], w0[1], w1[0], w1[1]};
                    }
                };
                __builtin_amdgcn_s_setprio(1);
                u32x4 vcur[SH::kHalves], vnext[SH::kHalves];
                vread(0, vcur);
#pragma unroll
                for (int dt = 0; dt < SH::kDt; ++dt) {
                    if (dt + 1 < SH::kDt) vread(dt + 1, vnext);
#pragma unroll
                    for (int nb = 0; nb < SH::kNb; ++nb) {
#pragma unroll
                        for (int h = 0; h < SH::kHalves; ++h)
                            o[nb][dt] = T::mfma16x16x32(vcur[h], pops[h][nb], o[nb][dt]);
                        __builtin_amdgcn_sched_barrier(0);  // keep the products back to back
                    }
#pragma unroll
                    for (int h = 0; h < SH::kHalves; ++h) vcur[h] = vnext[h];
                }
                __builtin_amdgcn_s_setprio(0);
            }
        }
    }
    }  // old loop
    // Drain the trailing copies before the work-group's LDS can be reassigned.
    wait_vmcnt_all();

#pragma unroll
    for (int nb = 0; nb < SH::kNb; ++nb) {
        // The pipelined loop's sums come from the matrix core, whole per lane.
        const float l_row = PIPE ? osum[nb][0] : row4_sum(l_part[nb]);
        if (qi[nb] >= qlen) continue;
        const int64_t rowid = (row0 + qi[nb]) * a.q_heads + head[nb];
        if (nchunks == 1) {
            const float inv = (row_ok[nb] && l_row > 0.f) ? __builtin_amdgcn_rcpf(l_row) : 0.f;
            uint16_t* orow = static_cast<uint16_t*>(a.out) + (DENSE ? out_off[nb] : rowid * hd);
#pragma unroll
            for (int dt = 0; dt < SH::kDt; ++dt) {
                const u32x2 w = {T::pack(o[nb][dt][0] * inv, o[nb][dt][1] * inv),
                                 T::pack(o[nb][dt][2] * inv, o[nb][dt][3] * inv)};
                if (!NARROW || 16 * dt + 4 * lg < hd) *reinterpret_cast<u32x2*>(orow + 16 * dt + 4 * lg) = w;
            }
        } else {
            const int64_t slot = (int64_t)chunk * a.ws_rows + rowid;
            const float inv = (row_ok[nb] && l_row > 0.f) ? __builtin_amdgcn_rcpf(l_row) : 0.f;
            using P = typename PartialOf<T>::type;
            P* po = static_cast<P*>(a.ws_o) + slot * SH::kD;
#pragma unroll
            for (int dt = 0; dt < SH::kDt; ++dt) {
                if constexpr (sizeof(P) == 4) {
                    *reinterpret_cast<f32x4*>(po + 16 * dt + 4 * lg) = o[nb][dt] * inv;
                } else {
                    const u32x2 w = {T::pack(o[nb][dt][0] * inv, o[nb][dt][1] * inv),
                                     T::pack(o[nb][dt][2] * inv, o[nb][dt][3] * inv)};
                    *reinterpret_cast<u32x2*>(po + 16 * dt + 4 * lg) = w;
                }
            }
            if (lg == 0) {
                a.ws_ml[slot * 2] = row_ok[nb] ? m_run[nb] : kNegInf;
                a.ws_ml[slot * 2 + 1] = row_ok[nb] ? l_row : 0.f;
            }
        }
    }
    // With key splitting, the first chunk's item of kv head 0 tells the merge
    // how many chunks each of its block's tokens has (1: written directly).
    if (a.max_chunks > 1 && chunk == 0 && kvh == 0) {
        for (int t = threadIdx.x; t < a.qb && q0 + t < qlen; t += kPfThreads) a.ws_tok[row0 + q0 + t] = nchunks;
    }
}

// Chunk choice for a walk (the caller's chunk is the smallest allowed: it
// bounds the workspace).  The best chunk puts the item count just under a
// multiple of the walkers, and which chunk that is depends on the lengths,
// which only the device sees.  Every work-group evaluates the same
// candidates a.chunk + 64*step*c (c < 128, or c < 512 when there are fewer
// than 16 query blocks; up to the capacity) against the same estimate of
// the makespan (in tile times) of walking one kv head's items with W
// work-groups:
//   max(ceil(items / W) * (F + chunk / 64), (tiles + F * items) / W),
// rounds of full items, never below the perfectly balanced total, with F
// the fixed cost of an item in a walk (lookup, first page, Q and first-tile
// latency, partial stores and the drained pipeline: about 5 tile times,
// fitted to walks of one 2048- or 4096-token causal prompt timed at chunks
// of 256 to 1024 keys), and all take the cheapest (ties: the smaller chunk).
// Thread t counts candidate t % 128 over every fourth query block (t / 128
// picks which), so the count costs a quarter of the blocks per thread; with
// fewer than 16 blocks (a few long requests: large capacities, so a coarse
// step) thread t counts candidate t over all of them, which puts the
// candidates 4 times closer.  The sums meet in the V ring, which the first
// copies fill only after the final barrier here.  (The V ring, not the K ring: with heads narrower than the
// tile the K ring's padded slots must stay zero, as they multiply the
// queries' zero dims; the V ring's padded slots only reach output dims that
// are never read.)
constexpr float kItemFixedTiles = 5.0f;  // in 64-key tiles
constexpr int kChoiceCands = 128;
constexpr int kChoiceSlices = kPfThreads / kChoiceCands;
constexpr int kChoiceWideBlocks = 16;    // below this many blocks: one candidate per thread
constexpr int kChoiceListOffset = 1024;  // uint32 offset of the block-end list in the V ring (after the sums)
constexpr int kChoiceMaxBlocks = 8192;   // blocks the list holds (32 KiB)
static_assert((kChoiceListOffset + kChoiceMaxBlocks) * 4 <= kPfStages * kTileBytes, "list inside the V ring");
static_assert(kChoiceSlices * kChoiceCands + kChoiceSlices <= kChoiceListOffset, "sums before the list");

template <int KEYS, bool DENSE>
__device__ int choose_chunk(const PrefillArgs& a, PrefillLds& lds, const SeqMeta& first) {
    constexpr float kFixed = kItemFixedTiles * 64.f / KEYS;  // an item's fixed cost in tiles of KEYS keys
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    // 64-bit: the capacity may be up to 2^31 - 1 keys, and candidates past it
    // are formed (and rejected) too.
    const int64_t cap = (int64_t)a.table_width * a.block_size;
    const int64_t cmax = (cap + KEYS - 1) / KEYS * KEYS;
    const int span = (int)((cmax - a.chunk) / KEYS);  // candidate steps above the minimum
    uint32_t items = 0, tiles = 0;
    // Up to 64 sequences (lane j of every wave holds sequence j) the key
    // ends of all query blocks go into one list in LDS first, each computed
    // once, so that a thread's count is one read and one quotient per block;
    // the list sits behind the sums' scratch in the V ring.  With more
    // blocks than the list holds, each thread reads the walk index's
    // metadata from LDS and computes the ends itself.
    const bool indexed = a.num_seqs <= kWave;
    uint32_t* blk_end = reinterpret_cast<uint32_t*>(&lds.v[0][0]) + kChoiceListOffset;
    int total_blocks = 0;
    bool flat = false;
    if (indexed) {
        __syncthreads();  // the index's LDS copy is complete
        const int nb = first.n > 0 ? (int)ceil_div_u32((uint32_t)first.n, (uint32_t)a.qb) : 0;
        const int incl = wave_incl_scan(nb);
        total_blocks = lane_value(incl, kWave - 1);
        flat = total_blocks <= kChoiceMaxBlocks;
        if (flat) {
            for (int j = wave; j < a.num_seqs; j += kPfWaves) {
                const int64_t n = lane_value(first.n, j), start = lane_value(first.start, j);
                const int64_t ctx = lane_value(first.ctx, j);
                const int nbj = lane_value(nb, j), off = lane_value(incl, j) - nbj;
                for (int b = lane; b < nbj; b += kWave)
                    blk_end[off + b] = (uint32_t)block_kv_end(a, start, ctx, n, (int64_t)b * a.qb);
            }
            __syncthreads();
        }
    }
    // Uniform over the work-group: every wave derives total_blocks from the
    // same metadata.
    const bool wide = flat && total_blocks < kChoiceWideBlocks;
    const int cands = wide ? kPfThreads : kChoiceCands;
    const int slices = wide ? 1 : kChoiceSlices;
    const int ci = tid % cands, slice = tid / cands;
    const int step = max(1, (span + cands - 1) / cands);
    const int64_t cand64 = a.chunk + (int64_t)KEYS * step * ci;
    const bool valid = cand64 <= cmax && cand64 <= 2147483647;  // candidate 0, the minimum, always is
    const int cand = valid ? (int)cand64 : a.chunk;
    if (flat) {
        if (__builtin_amdgcn_ballot_w64(valid) != 0) {  // wave-uniform
            for (int b = slice; b < total_blocks; b += slices) {
                const uint32_t e = blk_end[b];
                items += e > 0 ? ceil_div_u32(e, (uint32_t)cand) : 1;
                tiles += (e + KEYS - 1) / KEYS;
            }
        }
    } else if (indexed && __builtin_amdgcn_ballot_w64(valid) != 0) {
        int blk = 0;  // query blocks of the sequences before (uniform)
        for (int j = 0; j < a.num_seqs; ++j) {
            const SeqMeta mj = lds.meta[j];
            const int nb = mj.n > 0 ? (int)ceil_div_u32((uint32_t)mj.n, (uint32_t)a.qb) : 0;
            for (int k = ((slice - blk) % kChoiceSlices + kChoiceSlices) % kChoiceSlices; k < nb; k += kChoiceSlices) {
                const uint32_t e = (uint32_t)block_kv_end(a, mj.start, mj.ctx, mj.n, (int64_t)k * a.qb);
                items += e > 0 ? ceil_div_u32(e, (uint32_t)cand) : 1;
                tiles += (e + KEYS - 1) / KEYS;
            }
            blk += nb;
        }
    } else if (!indexed && __builtin_amdgcn_ballot_w64(valid) != 0) {  // wave-uniform
        int blk = 0;  // query blocks of the sequences before (uniform)
        for (int s0 = 0; s0 < a.num_seqs; s0 += kWave) {
            // One sequence's metadata per lane, then every lane walks them all.
            const SeqMeta m = s0 == 0 ? first : load_meta<DENSE>(a, s0 + lane);
            const int64_t n = m.n, start = m.start, ctx = m.ctx;
            const int cnt = min(kWave, a.num_seqs - s0);
            for (int j = 0; j < cnt; ++j) {
                const int64_t nj = __shfl(n, j), sj = __shfl(start, j), cj = __shfl(ctx, j);
                const int nb = query_blocks(a, nj);
                for (int k = ((slice - blk) % kChoiceSlices + kChoiceSlices) % kChoiceSlices; k < nb;
                     k += kChoiceSlices) {
                    const uint32_t e = (uint32_t)block_kv_end(a, sj, cj, nj, (int64_t)k * a.qb);
                    items += e > 0 ? ceil_div_u32(e, (uint32_t)cand) : 1;
                    tiles += (e + KEYS - 1) / KEYS;
                }
                blk += nb;
            }
        }
    }
    uint32_t* sc_items = reinterpret_cast<uint32_t*>(&lds.v[0][0]);  // [slice][candidate]
    uint32_t* sc_tiles = sc_items + kPfThreads;                       // [slice]
    sc_items[slice * cands + ci] = items;
    if (ci == 0) sc_tiles[slice] = tiles;
    __syncthreads();
    // Slice 0 (candidate ci = thread: waves 0 and 1, or every wave when
    // wide) prices the candidates; each of those waves takes its cheapest
    // (the lowest lane among equal costs: the smaller chunk).  Non-negative
    // floats order like their bit patterns; a candidate past the capacity
    // costs all ones.
    static_assert(kChoiceCands == 2 * kWave, "slice 0 is waves 0 and 1");
    static_assert(kChoiceSlices * kChoiceCands == kPfThreads, "one candidate slot per thread");
    const int pricing_waves = wide ? kPfWaves : 2;
    if (wave < pricing_waves) {
        uint32_t cost_bits = 0xffffffffu;
        if (valid) {
            uint32_t it_sum = 0, tl_sum = 0;
#pragma unroll
            for (int k = 0; k < kChoiceSlices; ++k) {
                if (k >= slices) break;
                it_sum += sc_items[k * cands + ci];
                tl_sum += sc_tiles[k];
            }
            const uint32_t w = (uint32_t)a.item_stride;
            const float rounds = (float)((it_sum + w - 1) / w);
            const float cost = fmaxf(rounds * (kFixed + (float)(cand / KEYS)),
                                     ((float)tl_sum + kFixed * (float)it_sum) / (float)w);
            cost_bits = __float_as_uint(cost);
        }
        const uint32_t least = wave_min_u32(cost_bits);
        const uint64_t hit = __builtin_amdgcn_ballot_w64(cost_bits == least);
        if (lane == 0) lds.pick[wave] = ((uint64_t)least << 32) | (uint32_t)(wave * kWave + __builtin_ctzll(hit));
    }
    // The sums and the block list (V ring) are read before this barrier, so
    // the copies that follow may overwrite them; the picks are not in a ring.
    __syncthreads();
    uint64_t best = lds.pick[0];
    for (int w = 1; w < pricing_waves; ++w) best = lds.pick[w] < best ? lds.pick[w] : best;
    return (int)(a.chunk + (int64_t)KEYS * step * (int)(uint32_t)best);  // a valid candidate: below 2^31
}

// Items are enumerated densely.  WALK = false: one item per work-group (the
// grid covers every possible item; work-groups past the end exit).  WALK =
// true: one work-group per CU slot, each walking items idx, idx +
// item_stride, ... below the item count (a separate instantiation, so that
// the one-item kernel keeps its register allocation).
template <typename T, int PAGES, bool WALK, bool NARROW, int HD, bool DENSE>
__global__ __launch_bounds__(kPfThreads, 1) void paged_prefill_mfma_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) PrefillLds lds;
    if constexpr (NARROW && PAGES == kPagesPerTile) {
        // Whole-tile copies skip the padded chunks of narrow rows: those LDS
        // slots (the same in every stage and item) must hold zeros.
        u32x4* ring = reinterpret_cast<u32x4*>(&lds.k[0][0]);
        static_assert(offsetof(PrefillLds, v) == offsetof(PrefillLds, k) + sizeof(lds.k), "K and V rings adjacent");
        constexpr int n16 = (int)(sizeof(lds.k) + sizeof(lds.v)) / 16;
        for (int i = threadIdx.x; i < n16; i += kPfThreads) ring[i] = u32x4{0u, 0u, 0u, 0u};
        __syncthreads();
    }
    if constexpr (!WALK) {
        PrefillItem item;
        if (!find_item<DENSE>(a, a.chunk, blockIdx.x / a.kv_heads, item)) return;
        prefill_item<T, PAGES, NARROW, HD, DENSE>(a, item, lds);
    } else {
        // The first lookup also counts the items, so that the walk ends
        // without a lookup past the end.
        int total = 0;
        int idx = blockIdx.x / a.kv_heads;
        PrefillItem item;
        // Up to 64 sequences: their metadata and item counts go to LDS once,
        // and every lookup reads them there (nothing held in registers
        // across the tile loop).
        const bool indexed = a.num_seqs <= kWave;
        int chunk_len = a.chunk;
        bool ok = false;
        if (indexed) {
            const SeqMeta m = load_meta<DENSE>(a, (int)(threadIdx.x & (kWave - 1)));
            int cnt, incl;
            total = walk_index(a, chunk_len, m, lds, cnt, incl);
            if (a.chunk_choice && total > a.item_stride) {
                // More than one round of items: the lengths decide the chunk.
                chunk_len = choose_chunk<PfShape<HD>::kKeys, DENSE>(a, lds, m);
                total = walk_index(a, chunk_len, m, lds, cnt, incl);
            }
            // The first lookup uses this wave's own copy of the index; wave 0's
            // LDS copy serves the later ones (after the barrier between items).
            ok = find_item_lanes(a, chunk_len, total, m, cnt, incl, idx, item);
        } else {
            ok = find_item<DENSE>(a, chunk_len, idx, item, &total);
            if (a.chunk_choice && total > a.item_stride) {
                const SeqMeta m = load_meta<DENSE>(a, (int)(threadIdx.x & (kWave - 1)));
                chunk_len = choose_chunk<PfShape<HD>::kKeys, DENSE>(a, lds, m);
                ok = find_item<DENSE>(a, chunk_len, idx, item, &total);
            }
        }
        while (ok) {
            prefill_item<T, PAGES, NARROW, HD, DENSE>(a, item, lds);
            idx += a.item_stride;
            if (idx >= total) break;
            __syncthreads();  // every wave is done with the LDS ring before the next item refills it
            ok = indexed ? find_item_indexed(a, chunk_len, total, lds, idx, item)
                         : find_item<DENSE>(a, chunk_len, idx, item);
        }
    }
}

// Combines the key-chunk partials of rows whose query block needed several
// chunks: with o_c the chunk's normalised output, l_c its probability sum and
// m_c its reference, out = sum_c w_c o_c / sum_c w_c, w_c = l_c 2^(m_c - M).
// One work-group per packed token (its chunk count comes from the attention
// kernel); a thread handles 8 dims of one head.  Partial rows are part_dim
// wide (heads narrower than the tile shape are zero-padded there); the output has
// head_dim.
constexpr int kMergeThreads = 256;

// One chunk's partial: 8 dims of the row (two 16-byte words for fp32
// partials, one for bf16) and its (reference, sum) pair.
template <typename T>
struct MergePart {
    u32x4 raw[2];
    float2 ml;
};

template <typename T>
__device__ inline MergePart<T> merge_load(const PrefillArgs& a, int64_t rowid, int d0, int c) {
    using P = typename PartialOf<T>::type;
    MergePart<T> part;
    const int64_t slot = (int64_t)c * a.ws_rows + rowid;  // chunk c's slot: c * ws_rows + rowid
    const u32x4* po = reinterpret_cast<const u32x4*>(static_cast<const P*>(a.ws_o) + slot * a.part_dim + d0);
    part.raw[0] = po[0];
    if constexpr (sizeof(P) == 4) part.raw[1] = po[1];
    part.ml = reinterpret_cast<const float2*>(a.ws_ml)[slot];
    return part;
}

// Folds G chunks into the running (reference, sum, acc); entries with
// live = false get weight zero.  The reference moves (with a rescale) only
// when the group holds a larger maximum.
template <typename T, int G>
__device__ inline void merge_absorb(const MergePart<T> (&parts)[G], const bool (&live)[G], float& mref, float& sum,
                                    float (&acc)[8]) {
    using P = typename PartialOf<T>::type;
    float m[G];
    float gmax = kNegInf;
#pragma unroll
    for (int k = 0; k < G; ++k) {
        m[k] = live[k] ? parts[k].ml.x : kNegInf;
        gmax = fmaxf(gmax, m[k]);
    }
    if (gmax > mref) {
        const float scale = mref == kNegInf ? 0.f : fast_exp2(mref - gmax);
        sum *= scale;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] *= scale;
        mref = gmax;
    }
    const float ref = mref == kNegInf ? 0.f : mref;
#pragma unroll
    for (int k = 0; k < G; ++k) {
        f32x4 x0, x1;
        if constexpr (sizeof(P) == 4) {
            x0 = __builtin_bit_cast(f32x4, parts[k].raw[0]);
            x1 = __builtin_bit_cast(f32x4, parts[k].raw[1]);
        } else {
            const u32x4 w = parts[k].raw[0];
            x0 = f32x4{T::lo(w[0]), T::hi(w[0]), T::lo(w[1]), T::hi(w[1])};
            x1 = f32x4{T::lo(w[2]), T::hi(w[2]), T::lo(w[3]), T::hi(w[3])};
        }
        // Chunk weight: its probability sum at the common reference.
        const float w = m[k] == kNegInf ? 0.f : parts[k].ml.y * fast_exp2(m[k] - ref);
        sum += w;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[i] = fmaf(x0[i], w, acc[i]);
            acc[4 + i] = fmaf(x1[i], w, acc[4 + i]);
        }
    }
}

// Chunks c0 .. c0+G-1 below nchunks, every load of the group in flight
// together (loads guarded one by one, each followed by its use, would each
// wait for the previous one): chunks past the last re-read the last one --
// in bounds and cached -- and get weight zero.
template <typename T, int G>
__device__ inline void merge_group(const PrefillArgs& a, int64_t rowid, int d0, int c0, int nchunks, float& mref,
                                   float& sum, float (&acc)[8]) {
    MergePart<T> parts[G];
    bool live[G];
#pragma unroll
    for (int k = 0; k < G; ++k) {
        parts[k] = merge_load<T>(a, rowid, d0, min(c0 + k, nchunks - 1));
        live[k] = c0 + k < nchunks;
    }
    merge_absorb<T, G>(parts, live, mref, sum, acc);
}

// Grid: (packed token, group of kMergeThreads (head, 8-dim) pairs).
template <typename T>
__global__ __launch_bounds__(kMergeThreads) void paged_prefill_merge_kernel(PrefillArgs a) {
    const int64_t token = blockIdx.x;
    // Every token of consistent metadata is written by its block's first
    // item; the clamp keeps reads inside the workspace for any other value.
    // The count is a scalar load; the first two chunks' partials (every
    // merged row has at least two, and the workspace holds at least two
    // chunks whenever this kernel runs) are requested before it is used, so
    // that the count and the data cost one memory round trip, not two.
    const int counted = a.ws_tok[token];
    const int dgroups = a.head_dim / 8;
    const int idx = blockIdx.y * kMergeThreads + threadIdx.x;
    if (idx >= a.q_heads * dgroups) return;
    const int head = idx / dgroups;
    const int d0 = 8 * (idx - head * dgroups);
    const int64_t rowid = token * a.q_heads + head;
    const MergePart<T> first[2] = {merge_load<T>(a, rowid, d0, 0), merge_load<T>(a, rowid, d0, 1)};
    // Keeps the two loads above the count test (the compiler would
    // otherwise move them below it, after the count's round trip).
    asm volatile("" : : : "memory");
    const int nchunks = min(counted, a.max_chunks);
    if (nchunks <= 1) return;
    float mref = kNegInf, sum = 0.f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // The rest in one group of 4 or 8 when it fits (a group's re-reads of
    // the last chunk cost cache bandwidth, not HBM traffic).
    if (nchunks > 2) {
        if (nchunks <= 6) {
            merge_group<T, 4>(a, rowid, d0, 2, nchunks, mref, sum, acc);
        } else {
            for (int c0 = 2; c0 < nchunks; c0 += 8) merge_group<T, 8>(a, rowid, d0, c0, nchunks, mref, sum, acc);
        }
    }
    const bool both[2] = {true, true};
    merge_absorb<T, 2>(first, both, mref, sum, acc);
    const float inv = sum > 0.f ? 1.f / sum : 0.f;
    const u32x4 wv = {T::pack(acc[0] * inv, acc[1] * inv), T::pack(acc[2] * inv, acc[3] * inv),
                      T::pack(acc[4] * inv, acc[5] * inv), T::pack(acc[6] * inv, acc[7] * inv)};
    uint16_t* orow =
        static_cast<uint16_t*>(a.out) + dense_seq(a, token) * a.o_seq + token * a.o_tok + head * a.o_head;
    *reinterpret_cast<u32x4*>(orow + d0) = wv;
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
    const int64_t dseq = dense_seq(a, token);
    uint16_t* orow = static_cast<uint16_t*>(a.out) + dseq * a.o_seq + token * a.o_tok + head * a.o_head;

    // Sequence owning this packed row (cu is monotone; dense mode: every
    // sequence has dense_tokens rows).
    int lo = 0;
    bool ok;
    int64_t pos = 0;
    const int64_t cap = (int64_t)a.table_width * a.block_size;
    if (a.dense_tokens > 0) {
        lo = (int)dseq;
        pos = a.dense_start + token - dseq * a.dense_tokens;
        ok = lo < a.num_seqs && pos < cap;
    } else {
        int hi = a.num_seqs;
        while (lo < hi) {
            const int mid = (lo + hi) / 2;
            if (a.cu[mid + 1] <= token) lo = mid + 1;
            else hi = mid;
        }
        ok = lo < a.num_seqs && token >= a.cu[lo];
        if (ok) {
            pos = a.starts[lo] + token - a.cu[lo];
            ok = a.starts[lo] >= 0 && pos < a.lens[lo] && pos < cap;
        }
    }
    if (!ok) {
        for (int d = lane; d < D; d += kWave) orow[d] = 0;
        return;
    }
    const int kvh = head / a.group;
    const bool ident = a.tables == nullptr;
    const int64_t* table = ident ? nullptr : a.tables + (int64_t)lo * a.table_width;
    const int64_t page_elems = a.kv_page_bytes / 2, row_elems = a.kv_row_bytes / 2;
    const uint16_t* qrow = static_cast<const uint16_t*>(a.q) + dseq * a.q_seq + token * a.q_tok + head * a.q_head;
    for (int d = lane; d < D; d += kWave) sm_q[d] = elem_to_float<T>(qrow[d]);
    __syncthreads();

    constexpr int kPer = kGenMaxD / kWave;
    float acc[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) acc[i] = 0.f;
    float m_run = kNegInf, l_run = 0.f;
    const uint16_t* kcache = static_cast<const uint16_t*>(a.key_cache) + kvh * (a.kv_head_bytes / 2);
    const uint16_t* vcache = static_cast<const uint16_t*>(a.value_cache) + kvh * (a.kv_head_bytes / 2);

    for (int64_t k0 = 0; k0 <= pos; k0 += kWave) {
        const int64_t key = k0 + lane;
        int64_t page = -1;
        if (key <= pos) page = ident ? lo : table[key / a.block_size];
        const bool kv_ok = page >= 0 && page < a.num_blocks;
        const int64_t off = kv_ok ? page * page_elems + (key % a.block_size) * row_elems : -1;
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

constexpr int64_t kMaxPrefillRows = 2147483647;  // packed rows x heads, table capacity
constexpr int64_t kMaxPrefillSeqs = 65535 * 16;

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
    if (total_tokens > kMaxPrefillRows || q_heads > kMaxPrefillRows || total_tokens * q_heads > kMaxPrefillRows)
        return fail(MVME_EINVAL, "too many paged prefill rows");
    if (num_seqs > kMaxPrefillSeqs) return fail(MVME_EINVAL, "too many paged prefill sequences");
    return MVME_OK;
}

struct PrefillPlan {
    bool mfma;
    bool narrow;  // head_dim below the tile shape's, zero-padded in LDS
    int hd;       // tile shape: padded head dim (128 or 256)
    int keys;     // keys per tile of that shape
    int qb;
    int chunk;
    int max_chunks;
    int64_t items_bound;
};

constexpr int64_t kPrefillCUs = 256;

// Host plan from shapes only (lengths stay on the device).  Enough query
// blocks to occupy the GPU 1.5 times over: no key split.  Otherwise split
// the keys into chunks of at least 512 (and at most 32 chunks per block,
// which bounds the workspace), which spreads long contexts over all CUs at
// the cost of partials and a merge; a walk over more than one round of
// items then takes a larger chunk on the device when the lengths favour it.
PrefillPlan make_prefill_plan(int64_t num_seqs, int64_t total_tokens, int64_t q_heads, int64_t kv_heads,
                              int64_t head_dim, int64_t block_size, int64_t table_width, int64_t chunk_tokens) {
    PrefillPlan p{};
    const int64_t group = q_heads / kv_heads;
    // MFMA tiles for every multiple of 8 up to 256: the 128 shape for head
    // dims up to 128, the 256 shape above; dims below the shape's are padded
    // with zeros in LDS (zero dims add nothing to the scores and give zero
    // outputs).
    const bool wide = head_dim > 128;
    p.hd = wide ? 256 : 128;
    p.narrow = head_dim < p.hd;
    p.keys = wide ? PfShape<256>::kKeys : PfShape<128>::kKeys;
    const int rows = wide ? PfShape<256>::kRows : PfShape<128>::kRows;
    p.mfma = group <= rows && head_dim % 8 == 0 && head_dim >= 8 && head_dim <= 256;
    if (!p.mfma) return p;
    p.qb = (int)(rows / group);
    const int64_t keys = p.keys;
    const int64_t cap = table_width * block_size;
    const int64_t cap_tiles = (cap + keys - 1) / keys * keys;
    const int64_t blocks_bound = (total_tokens + p.qb - 1) / p.qb + num_seqs;
    int64_t chunk;
    if (chunk_tokens > 0) chunk = (chunk_tokens + keys - 1) / keys * keys;
    // The split test counts the query blocks the tokens fill at least (the
    // bound above adds one partial block per sequence): near the threshold,
    // ragged contexts make whole-context items uneven, and the walk's chunk
    // choice can still take chunks as long as the capacity.
    else if ((total_tokens + p.qb - 1) / p.qb * kv_heads >= kPrefillCUs + kPrefillCUs / 2) chunk = cap_tiles;
    else chunk = std::max<int64_t>(512, ((cap + 31) / 32 + keys - 1) / keys * keys);
    if (chunk > cap_tiles) chunk = cap_tiles;
    if (chunk < keys) chunk = keys;
    p.chunk = (int)chunk;
    p.max_chunks = (int)((cap + chunk - 1) / chunk);
    if (p.max_chunks < 1) p.max_chunks = 1;
    p.items_bound = blocks_bound * p.max_chunks;
    return p;
}

// Key-chunk workspace: the partial outputs [max_chunks][rows][D] in the
// partial type (bf16 for bf16 inputs, fp32 for fp16), their (reference,
// sum) pairs [max_chunks][rows][2] fp32, then one int per packed token; each
// region 16-byte aligned.
struct PrefillWorkspace {
    size_t ml_offset, tok_offset, bytes;
};
PrefillWorkspace prefill_workspace_layout(int64_t rows, int64_t max_chunks, int64_t tokens, int dtype,
                                          int64_t part_dim) {
    const size_t part_elem = dtype == MVME_BF16 ? sizeof(uint16_t) : sizeof(float);
    auto align16 = [](size_t n) { return (n + 15) / 16 * 16; };
    PrefillWorkspace w{};
    w.ml_offset = align16((size_t)max_chunks * rows * part_dim * part_elem);
    w.tok_offset = w.ml_offset + align16((size_t)max_chunks * rows * 2 * sizeof(float));
    w.bytes = w.tok_offset + align16((size_t)tokens * sizeof(int));
    return w;
}

// Launches the attention kernel (and the merge of split query blocks) for
// arguments whose layout and metadata fields are filled in; `need` is the
// plan's workspace size, already checked against the caller's buffer.
int launch_prefill(PrefillArgs a, const PrefillPlan& p, int64_t total_tokens, int64_t chunk_tokens, int dtype,
                   size_t need, void* workspace, hipStream_t s, const char* what) {
    const int64_t q_heads = a.q_heads, kv_heads = a.kv_heads, table_width = a.table_width;
    if (p.mfma) {
        if (table_width * a.block_size > 2147483647)
            return fail(MVME_EINVAL, "paged prefill table capacity exceeds 2^31 tokens");
        a.qb = p.qb;
        a.part_dim = p.hd;
        a.chunk = p.chunk;
        a.max_chunks = p.max_chunks;
        a.ws_rows = total_tokens * q_heads;
        a.total_tokens = total_tokens;
        a.chunk_choice = chunk_tokens <= 0 ? 1 : 0;
        if (need > 0) {
            const PrefillWorkspace w = prefill_workspace_layout(total_tokens * q_heads, p.max_chunks, total_tokens,
                                                                dtype, p.hd);
            a.ws_o = workspace;
            a.ws_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + w.ml_offset);
            a.ws_tok = reinterpret_cast<int*>(static_cast<uint8_t*>(workspace) + w.tok_offset);
        }
        // The item count depends on lengths that stay on the device, so the
        // grid is sized from a bound.  With key splitting that bound is loose
        // (every block counted with the most chunks) and surplus work-groups
        // would queue behind the real ones (one work-group fits a CU): there
        // the grid is one work-group per CU slot, each walking its items.
        int64_t item_slots = p.items_bound;
        a.item_stride = 0;
        if (p.max_chunks > 1) {
            const int64_t slots = std::max<int64_t>(1, kPrefillCUs / kv_heads);
            if (p.items_bound > slots) {
                item_slots = slots;
                a.item_stride = (int)slots;
            }
        }
        const int64_t groups = item_slots * kv_heads;
        if (groups > 2147483647) return fail(MVME_EINVAL, "paged prefill grid too large");
        // Whole-tile pages: a tile lies in one page (power-of-two blocks of at
        // least a tile's keys) and per-lane offsets inside a tile fit 32 bits.
        const bool tile_pages = a.block_shift >= 0 && a.block_size >= p.keys &&
                                a.kv_row_bytes * p.keys < (int64_t(1) << 31);
        const int64_t block_size = a.block_size;
        const bool dense = a.tables == nullptr;
        if (dense && !tile_pages) return fail(MVME_EINVAL, "prefill key/value token stride too large");
        int pages = tile_pages ? kPagesPerTile : (block_size % 4 == 0 ? kPagesPerRows : kPagesPerLane);
        if (p.narrow && pages == kPagesPerRows) pages = kPagesPerLane;  // no narrow instantiation of that mode
        const dim3 grid((unsigned)groups), block(kPfThreads);
        auto launch = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, 0, s, a); };
        auto launch_walk = [&](auto one, auto walk) {
            if (a.item_stride > 0) launch(walk);
            else launch(one);
        };
        auto launch_type = [&](auto type_tag) {
            using T = decltype(type_tag);
            if (dense) {
                // Dense mode: one power-of-two page per sequence, whole-tile copies.
                if (p.hd == 256 && p.narrow)
                    launch_walk(paged_prefill_mfma_kernel<T, kPagesPerTile, false, true, 256, true>,
                                paged_prefill_mfma_kernel<T, kPagesPerTile, true, true, 256, true>);
                else if (p.hd == 256)
                    launch_walk(paged_prefill_mfma_kernel<T, kPagesPerTile, false, false, 256, true>,
                                paged_prefill_mfma_kernel<T, kPagesPerTile, true, false, 256, true>);
                else if (p.narrow)
                    launch_walk(paged_prefill_mfma_kernel<T, kPagesPerTile, false, true, 128, true>,
                                paged_prefill_mfma_kernel<T, kPagesPerTile, true, true, 128, true>);
                else
                    launch_walk(paged_prefill_mfma_kernel<T, kPagesPerTile, false, false, 128, true>,
                                paged_prefill_mfma_kernel<T, kPagesPerTile, true, false, 128, true>);
            } else if (p.hd == 256 && p.narrow) {
                if (pages == kPagesPerTile)
                    launch_walk(paged_prefill_mfma_kernel<T, kPagesPerTile, false, true, 256, false>,
                                paged_prefill_mfma_kernel<T, kPagesPerTile, true, true, 256, false>);
                else
                    launch_walk(paged_prefill_mfma_kernel<T, kPagesPerLane, false, true, 256, false>,
                                paged_prefill_mfma_kernel<T, kPagesPerLane, true, true, 256, false>);
            } else if (p.hd == 256) {
                if (pages == kPagesPerTile)
                    launch_walk(paged_prefill_mfma_kernel<T, kPagesPerTile, false, false, 256, false>,
                                paged_prefill_mfma_kernel<T, kPagesPerTile, true, false, 256, false>);
                else if (pages == kPagesPerRows)
                    launch_walk(paged_prefill_mfma_kernel<T, kPagesPerRows, false, false, 256, false>,
                                paged_prefill_mfma_kernel<T, kPagesPerRows, true, false, 256, false>);
                else
                    launch_walk(paged_prefill_mfma_kernel<T, kPagesPerLane, false, false, 256, false>,
                                paged_prefill_mfma_kernel<T, kPagesPerLane, true, false, 256, false>);
            } else if (p.narrow) {
                if (pages == kPagesPerTile)
                    launch_walk(paged_prefill_mfma_kernel<T, kPagesPerTile, false, true, 128, false>,
                                paged_prefill_mfma_kernel<T, kPagesPerTile, true, true, 128, false>);
                else
                    launch_walk(paged_prefill_mfma_kernel<T, kPagesPerLane, false, true, 128, false>,
                                paged_prefill_mfma_kernel<T, kPagesPerLane, true, true, 128, false>);
            } else if (pages == kPagesPerTile) {
                launch_walk(paged_prefill_mfma_kernel<T, kPagesPerTile, false, false, 128, false>,
                            paged_prefill_mfma_kernel<T, kPagesPerTile, true, false, 128, false>);
            } else if (pages == kPagesPerRows) {
                launch_walk(paged_prefill_mfma_kernel<T, kPagesPerRows, false, false, 128, false>,
                            paged_prefill_mfma_kernel<T, kPagesPerRows, true, false, 128, false>);
            } else {
                launch_walk(paged_prefill_mfma_kernel<T, kPagesPerLane, false, false, 128, false>,
                            paged_prefill_mfma_kernel<T, kPagesPerLane, true, false, 128, false>);
            }
        };
        if (dtype == MVME_FP16) launch_type(Half{});
        else launch_type(BFloat16{});
        if (p.max_chunks > 1) {
            const int64_t pairs = q_heads * (a.head_dim / 8);
            const dim3 grid((unsigned)total_tokens, (unsigned)((pairs + kMergeThreads - 1) / kMergeThreads));
            if (dtype == MVME_FP16)
                hipLaunchKernelGGL((paged_prefill_merge_kernel<Half>), grid, dim3(kMergeThreads), 0, s, a);
            else
                hipLaunchKernelGGL((paged_prefill_merge_kernel<BFloat16>), grid, dim3(kMergeThreads), 0, s, a);
        }
    } else {
        if (q_heads > 65535) return fail(MVME_EINVAL, "paged prefill grid too large");
        const dim3 grid((unsigned)total_tokens, (unsigned)q_heads);
        if (dtype == MVME_FP16)
            hipLaunchKernelGGL((paged_prefill_generic_kernel<Half>), grid, dim3(kWave), 0, s, a);
        else
            hipLaunchKernelGGL((paged_prefill_generic_kernel<BFloat16>), grid, dim3(kWave), 0, s, a);
    }
    return check_launch(what);
}

}  // namespace
}  // namespace mvme

using namespace mvme;

extern "C" size_t mvme_paged_prefill_workspace_size(int64_t num_seqs, int64_t total_tokens, int64_t q_heads,
                                                    int64_t kv_heads, int64_t head_dim, int64_t block_size,
                                                    int64_t table_width, int64_t chunk_tokens, int dtype) {
    if (num_seqs <= 0 || total_tokens <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0 ||
        block_size <= 0 || table_width <= 0 || !valid_dtype(dtype))
        return 0;
    // The limits the entry point enforces; inside them no product overflows.
    if (total_tokens > kMaxPrefillRows || q_heads > kMaxPrefillRows || total_tokens * q_heads > kMaxPrefillRows ||
        block_size > kMaxPrefillRows || table_width > kMaxPrefillRows ||
        table_width * block_size > kMaxPrefillRows || num_seqs > kMaxPrefillSeqs)
        return 0;
    const PrefillPlan p = make_prefill_plan(num_seqs, total_tokens, q_heads, kv_heads, head_dim, block_size,
                                            table_width, chunk_tokens);
    if (!p.mfma || p.max_chunks <= 1) return 0;
    return prefill_workspace_layout(total_tokens * q_heads, p.max_chunks, total_tokens, dtype, p.hd).bytes;
}

extern "C" int mvme_paged_prefill_attention(void* out, const void* q, const void* key_cache,
                                            const void* value_cache, const int64_t* cu_seqlens_q,
                                            const int64_t* query_starts, const int64_t* block_tables,
                                            const int64_t* context_lens, int64_t num_seqs,
                                            int64_t total_tokens, int64_t q_heads, int64_t kv_heads,
                                            int64_t head_dim, int64_t num_blocks, int64_t block_size,
                                            int64_t table_width, int64_t chunk_tokens, int dtype,
                                            void* workspace, size_t workspace_bytes, void* stream) {
    if (int rc = check_prefill(num_seqs, total_tokens, q_heads, kv_heads, head_dim, num_blocks,
                               block_size, table_width, dtype))
        return rc;
    if (total_tokens == 0) return MVME_OK;
    if (num_seqs == 0 || table_width == 0) return fail(MVME_EINVAL, "paged prefill metadata shape mismatch");
    if (!out || !q || !key_cache || !value_cache || !cu_seqlens_q || !query_starts || !block_tables ||
        !context_lens)
        return fail(MVME_EINVAL, "paged prefill received a null pointer");
    const size_t need = mvme_paged_prefill_workspace_size(num_seqs, total_tokens, q_heads, kv_heads, head_dim,
                                                          block_size, table_width, chunk_tokens, dtype);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(MVME_EWORKSPACE, "paged prefill workspace too small: need " + std::to_string(need) +
                                         " bytes, got " + std::to_string(workspace_bytes));
    const PrefillPlan p = make_prefill_plan(num_seqs, total_tokens, q_heads, kv_heads, head_dim, block_size,
                                            table_width, chunk_tokens);
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
    a.block_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctzll((unsigned long long)block_size) : -1;
    a.table_width = (int)table_width;
    a.scale_log2 = kLog2e / sqrtf((float)head_dim);
    // Paged layout: [pages, block_size, kv_heads, head_dim] caches, packed
    // [tokens, q_heads, head_dim] queries and outputs.
    a.kv_row_bytes = kv_heads * head_dim * 2;
    a.kv_page_bytes = block_size * a.kv_row_bytes;
    a.kv_head_bytes = head_dim * 2;
    a.q_tok = a.o_tok = q_heads * head_dim;
    a.q_head = a.o_head = head_dim;
    return launch_prefill(a, p, total_tokens, chunk_tokens, dtype, need, workspace,
                          static_cast<hipStream_t>(stream), "paged prefill");
}

// ---------------------------------------------------------------------------
// Dense suffix prefill: q [B, Hq, T, D], k and v [B, Hkv, S, D], any strides
// with a dense innermost dim; row (b, h, t) attends keys [0, query_start + t]
// of batch entry b.  The paged kernels run in dense mode: batch entry b is
// sequence b with T queries, its keys are one page (the entry itself, read
// through the strides), and no metadata arrays exist.
// ---------------------------------------------------------------------------
namespace {

constexpr int64_t kMaxDenseContext = 1048576;  // query_start + T

// The one page holding a sequence's keys: a power of two >= the context and
// >= a tile's keys, so that the whole-tile copy mode applies.
int64_t dense_block(int64_t ctx) {
    int64_t bs = 64;
    while (bs < ctx) bs *= 2;
    return bs;
}

bool dense_shapes_ok(int64_t batch, int64_t q_tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                     int64_t query_start) {
    return batch > 0 && q_tokens > 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0 && head_dim > 0 &&
           head_dim <= kGenMaxD && query_start >= 0 && query_start <= kMaxDenseContext &&
           q_tokens <= kMaxDenseContext && query_start + q_tokens <= kMaxDenseContext &&
           batch <= kMaxPrefillSeqs && batch * q_tokens <= kMaxPrefillRows / q_heads;
}

// Largest element offset a strided [n0, n1, n2, d] view can reach, plus the
// intermediate products the kernels form (rows of every batch entry times
// the token stride), kept below 2^60.
bool strided_span_ok(int64_t n0, int64_t s0, int64_t n1, int64_t s1, int64_t n2, int64_t s2, int64_t d) {
    if (s0 < 0 || s1 < 0 || s2 < 0) return false;
    const __int128 span = (__int128)n0 * s0 + (__int128)n0 * n2 * s2 + (__int128)n1 * s1 + d;
    return span < ((__int128)1 << 60);
}

// No two elements of a [n0, n1, n2, d] view (innermost stride 1, strides
// non-negative) share an address: taken by increasing stride, every
// dimension of more than one element steps past all the offsets the smaller
// ones reach.  (Holds for every layout torch makes without expand().)
bool view_disjoint(int64_t n0, int64_t s0, int64_t n1, int64_t s1, int64_t n2, int64_t s2, int64_t d) {
    int64_t n[3] = {n0, n1, n2}, s[3] = {s0, s1, s2};
    for (int i = 0; i < 3; ++i)
        for (int j = i + 1; j < 3; ++j)
            if (s[j] < s[i]) {
                std::swap(n[i], n[j]);
                std::swap(s[i], s[j]);
            }
    __int128 reach = d;  // offsets [0, reach) are taken
    for (int i = 0; i < 3; ++i) {
        if (n[i] <= 1) continue;
        if ((__int128)s[i] < reach) return false;
        reach += (__int128)s[i] * (n[i] - 1);
    }
    return true;
}

}  // namespace

extern "C" size_t mvme_prefill_attention_workspace_size(int64_t batch, int64_t q_tokens, int64_t q_heads,
                                                        int64_t kv_heads, int64_t head_dim, int64_t query_start,
                                                        int dtype) {
    if (!valid_dtype(dtype) || !dense_shapes_ok(batch, q_tokens, q_heads, kv_heads, head_dim, query_start))
        return 0;
    const int64_t rows = batch * q_tokens;
    const PrefillPlan p = make_prefill_plan(batch, rows, q_heads, kv_heads, head_dim,
                                            dense_block(query_start + q_tokens), 1, 0);
    if (!p.mfma || p.max_chunks <= 1) return 0;
    return prefill_workspace_layout(rows * q_heads, p.max_chunks, rows, dtype, p.hd).bytes;
}

extern "C" int mvme_prefill_attention(void* out, const void* q, const void* key, const void* value, int64_t batch,
                                      int64_t q_heads, int64_t kv_heads, int64_t q_tokens, int64_t kv_tokens,
                                      int64_t head_dim, int64_t query_start, int64_t q_batch_stride,
                                      int64_t q_head_stride, int64_t q_token_stride, int64_t kv_batch_stride,
                                      int64_t kv_head_stride, int64_t kv_token_stride, int64_t out_batch_stride,
                                      int64_t out_head_stride, int64_t out_token_stride, int dtype, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    if (!valid_dtype(dtype)) return fail(MVME_EINVAL, "prefill requires FP16/BF16");
    if (batch <= 0 || head_dim <= 0 || kv_tokens <= 0) return fail(MVME_EINVAL, "prefill shape mismatch");
    if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0) return fail(MVME_EINVAL, "prefill GQA mismatch");
    if (head_dim > kGenMaxD) return fail(MVME_EINVAL, "prefill supports head_dim up to 1024");
    if (query_start < 0 || q_tokens <= 0 || query_start > kv_tokens || q_tokens > kv_tokens - query_start)
        return fail(MVME_EINVAL, "prefill query range exceeds KV sequence");
    if (!dense_shapes_ok(batch, q_tokens, q_heads, kv_heads, head_dim, query_start))
        return fail(MVME_EINVAL, "prefill context exceeds 1048576 tokens or too many rows");
    if (!out || !q || !key || !value) return fail(MVME_EINVAL, "prefill received a null pointer");
    if (!strided_span_ok(batch, q_batch_stride, q_heads, q_head_stride, q_tokens, q_token_stride, head_dim) ||
        !strided_span_ok(batch, out_batch_stride, q_heads, out_head_stride, q_tokens, out_token_stride, head_dim) ||
        !strided_span_ok(batch, kv_batch_stride, kv_heads, kv_head_stride, kv_tokens, kv_token_stride, head_dim))
        return fail(MVME_EINVAL, "prefill strides out of range");
    if (!view_disjoint(batch, out_batch_stride, q_heads, out_head_stride, q_tokens, out_token_stride, head_dim))
        return fail(MVME_EINVAL, "prefill output rows overlap");
    const int64_t ctx = query_start + q_tokens;
    const int64_t bs = dense_block(ctx);
    const int64_t rows = batch * q_tokens;
    const PrefillPlan p = make_prefill_plan(batch, rows, q_heads, kv_heads, head_dim, bs, 1, 0);
    // The MFMA path moves rows in 16-byte pieces (the generic kernel reads elements).
    const int64_t align = p.mfma ? 16 : 2;
    const int64_t stride_mult = align / 2;
    for (const void* ptr : {static_cast<const void*>(out), q, key, value})
        if (reinterpret_cast<uintptr_t>(ptr) % align != 0)
            return fail(MVME_EINVAL, "prefill tensors must be " + std::to_string(align) + "-byte aligned");
    for (int64_t st : {q_batch_stride, q_head_stride, q_token_stride, kv_batch_stride, kv_head_stride,
                       kv_token_stride, out_batch_stride, out_head_stride, out_token_stride})
        if (st % stride_mult != 0)
            return fail(MVME_EINVAL, "prefill strides must be multiples of " + std::to_string(stride_mult) +
                                         " elements");
    const size_t need =
        mvme_prefill_attention_workspace_size(batch, q_tokens, q_heads, kv_heads, head_dim, query_start, dtype);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(MVME_EWORKSPACE, "prefill workspace too small: need " + std::to_string(need) + " bytes, got " +
                                         std::to_string(workspace_bytes));
    PrefillArgs a{};
    a.out = out;
    a.q = q;
    a.key_cache = key;
    a.value_cache = value;
    a.num_seqs = (int)batch;
    a.q_heads = (int)q_heads;
    a.kv_heads = (int)kv_heads;
    a.group = (int)(q_heads / kv_heads);
    a.head_dim = (int)head_dim;
    a.num_blocks = batch;
    a.block_size = (int)bs;
    a.block_shift = __builtin_ctzll((unsigned long long)bs);
    a.table_width = 1;
    a.scale_log2 = kLog2e / sqrtf((float)head_dim);
    a.dense_tokens = (int)q_tokens;
    a.dense_start = (int)query_start;
    a.kv_page_bytes = kv_batch_stride * 2;
    a.kv_row_bytes = kv_token_stride * 2;
    a.kv_head_bytes = kv_head_stride * 2;
    // Packed row r = b*T + t: s*x_seq + r*x_tok = b*batch_stride + t*token_stride.
    a.q_seq = q_batch_stride - q_tokens * q_token_stride;
    a.q_tok = q_token_stride;
    a.q_head = q_head_stride;
    a.o_seq = out_batch_stride - q_tokens * out_token_stride;
    a.o_tok = out_token_stride;
    a.o_head = out_head_stride;
    return launch_prefill(a, p, rows, 0, dtype, need, workspace, static_cast<hipStream_t>(stream), "prefill");
}

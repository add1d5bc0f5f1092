// GQA paged decode attention for gfx950: the attention kernel, shared by
// paged_decode.hip (plain instantiations, plan, merge, entry points) and
// paged_decode_fused.hip (instantiations with the fused prologue).
//
// Work decomposition: one work-group of NW waves per
// (sequence, kv head, G-query-head tile, partition of `partition` tokens).
// All G query heads that share a kv head are served by the same loads, so
// every K/V byte of a partition is fetched from HBM exactly once.  When the
// (sequence, kv head) units alone fill the GPU, one work-group (4 or 8 waves
// by the context's length) covers a whole sequence and merges its waves
// in LDS: one kernel, no workspace.
// Otherwise the context is split into partitions of 4-wave work-groups
// (split-K) whose fp32 partials a second, small kernel merges.  A third
// mode, the balanced walk, lays the units end to end and gives every
// work-group an equal share of their tokens (several short units, or a piece
// of a long one); the units cut by a share boundary are merged the same way.
//
// Lane layout inside a wave: a token row of one kv head is head_dim*2 bytes
// = D/8 16-byte chunks; LPT (next power of two >= D/8) consecutive lanes
// cover one token, so one global_load_dwordx4 per lane moves 64/LPT whole
// token rows (1 KiB for D=128: four 256-byte rows).  Each wave issues four
// K loads and four V loads per iteration before touching any of them.
//
// Fused prologue (optional, head_dim 16/32/64/128/256): before attention,
// each work-group writes its sequence's new token -- at position len - 1 --
// into the kv head's cache row, either as given (the decode-batch KV write)
// or after per-head RMSNorm + RoPE of k, with the query heads of its tile
// normalised and rotated the same way.  The row is written by the one wave
// that later reads that position (in every work-group whose token range
// holds it: identical bytes from each G-tile), so no barrier is needed.
//
// Scores: packed dot2 (fp16/bf16 products, fp32 accumulation) on the lane's
// 8 elements, then a DPP reduction across the LPT lanes of the token.
// Softmax: online, fp32, base-2 exponent with log2(e)/sqrt(D) folded into
// the scale.  Each token group of lanes keeps its own running max/sum/acc;
// groups, then waves (through LDS), are merged at the end.  Sequences that
// fit one partition write the output directly from the attention kernel.
#pragma once

#include "norm_rope.h"

namespace mvme {

constexpr int kSplitWaves = 4;   // waves per work-group in split-K mode
// Waves per work-group covering a whole sequence.  Uniform decode at head_dim
// 128 (fp16, block 256, us per call), 16 waves against 8: B32/ctx2048 43.7 ->
// 42.9 (45.2 at 12); B128/ctx1024 91.4 -> 83.9; B64/ctx2048 83.8 -> 83.3.  A
// plain streaming read of a 256 MiB layer likewise peaks at 8 waves per CU
// (6.8 TB/s; 16 waves 6.4).  Long units (kLongUnitBytes of K+V or more) once
// took 16 waves, which were ahead only where 8-wave work-groups sat badly
// paired on the CUs or a round of units was unbalanced; the paired order and
// the balanced walk now serve those shapes (ragged B64 / ctx 4096, block 16:
// 88.0 at 16 -> 81.1; ragged B128 165.8 -> 161.3; ragged B256 349.5 ->
// 333.1; uniform B128 / ctx 4096 328.8 -> 327.1).
constexpr int kWholeWaves = 8;
constexpr int64_t kLongUnitBytes = int64_t(2) << 20;
constexpr int kLptMax = 256;     // largest batch whose units go longest context first
static_assert(kSplitWaves * kWave >= kLptMax, "one thread per sequence key");
constexpr int kDecodeLoads = 4;  // K (and V) loads per lane per iteration
// Balanced walk: waves per work-group (its own kernel instances, with
// non-temporal loads: the plan takes the walk for calls of 480 MiB or more).
constexpr int kFlatWaves = kWholeWaves;

template <int D>
struct DecodeShape {
    static constexpr int kChunks = D / 8;  // 16-byte chunks per token row
    static constexpr int kLpt = kChunks <= 1 ? 1 : kChunks <= 2 ? 2 : kChunks <= 4 ? 4
                              : kChunks <= 8 ? 8 : kChunks <= 16 ? 16 : kChunks <= 32 ? 32 : 64;
    static constexpr int kTpl = kWave / kLpt;          // tokens per load
    static constexpr int kTpi = kTpl * kDecodeLoads;   // tokens per wave iteration
};

// Balanced walk: the merge duty of share l, written by the attention
// kernel's work-group for that share on every call and read by the merge
// kernel's work-group l.  A share merges the unit it began with when that
// unit started in an earlier share and ends inside this one.
struct FlatMergeDesc {
    int b;          // the unit's sequence, -1 when the share merges nothing
    int r;          // the unit's column (kv head * gtiles + query-head tile)
    int p0;         // share holding the unit's first piece
    int slot0;      // row slot of that piece (1: its share's last segment)
    int64_t total;  // chunks of the call, for the empty-share test
    int64_t pad;
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
    FlatMergeDesc* ws_flat;  // balanced walk: [flat_groups] merge duties
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
    // With two work-groups resident per CU for the whole call: the second
    // half of the unit groups takes the ranks in reverse (shortest first), so
    // that each CU pairs a long sequence with a short one.
    int lpt_pair;
    // Balanced walk (flat_groups > 0, batch <= kLptMax): `flat_groups`
    // (kFlatGroups) work-groups, each taking an equal share of the call's
    // token chunks.
    int flat_groups;
    int batch;
    float scale_log2;
    // Fused prologue: 0 none; 1 write new_k / new_v rows at position len - 1;
    // 2 RMSNorm + RoPE of the query heads (query = raw rows, q_stride apart)
    // and of new_k, then write.  cos / sin: [batch, D/2] at that position.
    int prologue;
    const uint16_t* new_k;  // [batch, kv_heads, D], token rows k_stride apart
    const uint16_t* new_v;  // token rows v_stride apart
    int64_t k_stride, v_stride, q_stride;
    const uint16_t* q_weight;  // [D]
    const uint16_t* k_weight;  // [D]
    const uint16_t* cos;
    const uint16_t* sin;
    uint16_t* q_out;  // [batch, q_heads, D] rotated queries, or nullptr
    float eps;
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

// Balanced walk.  The call's units are laid end to end, column by column (a
// column is one (kv head, query-head tile) across every sequence, sequences
// in index order), each unit cut into chunks of `chunk` tokens (at least one
// chunk, so that an empty sequence still writes its zero output).  With W
// chunks in all, logical work-group l of NG takes chunks [l*W/NG, (l+1)*W/NG):
// every work-group streams the same number of K/V rows whatever the lengths,
// and only the units cut by a share boundary leave partials to merge.
//
// Every thread of the work-group (at least kLptMax of them) calls this; it
// fills len[b] (the sequence's valid context) and pref[b] (chunks of the
// sequences before b in a column, pref[batch] = chunks per column), and ends
// with a barrier.
__device__ inline void flat_prefix(const DecodeArgs& a, int chunk, int* len, int* pref, int* wave_tot) {
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1), wave = tid / kWave;
    const int n = a.batch;
    int w = 0;
    if (tid < n) {
        const int ln = seq_tokens(a.lens[tid], a.capacity);
        len[tid] = ln;
        w = ln > 0 ? (ln + chunk - 1) / chunk : 1;
    }
    const int incl = wave_incl_scan(w);
    constexpr int kScanWaves = kLptMax / kWave;
    if (wave < kScanWaves && lane == kWave - 1) wave_tot[wave] = incl;
    __syncthreads();
    if (tid < n) {
        int before = 0;
        for (int v = 0; v < wave; ++v) before += wave_tot[v];
        pref[tid + 1] = before + incl;
    }
    if (tid == 0) pref[0] = 0;
    __syncthreads();
}

// Sequence whose chunks hold position `cin` of a column (pref as above):
// the number of sequences that end at or before it.  Wave-uniform.
__device__ inline int flat_seq_of(const int* pref, int n, int64_t cin) {
    const int lane = threadIdx.x & (kWave - 1);
    int count = 0;
    for (int base = 0; base < n; base += kWave) {
        const int idx = base + lane;
        count += __builtin_popcountll(__ballot(idx < n && pref[idx + 1] <= cin));
    }
    return count;
}

// Work-groups of the walk: a multiple of 8, the XCD count, kFlatWaves waves
// each, and a power of two (share bounds are a shift).  Measured on 32
// sequences of contexts U[1,4096] (fp16, block 256, µs per call): 256 x 8
// waves 62.5, 256 x 16 63.3, 512 x 8 63.3, 1024 x 4 67.9.
constexpr int kFlatShift = 8;
constexpr int kFlatGroups = 1 << kFlatShift;
static_assert(kFlatGroups <= kLptMax, "one merge thread per piece");

// First chunk of logical work-group l's share.
__device__ inline int64_t flat_share_start(int64_t l, int64_t total) { return (l * total) >> kFlatShift; }

// PRO: the kernel runs the fused prologue (a.prologue 1 or 2); without it
// the prologue's code is not compiled in.  FLAT: the balanced walk (its
// segment loop would cost the other modes about 20 VGPRs).
template <typename T, int D, int G, bool PAGE_UNIFORM, int NW, bool STREAM, bool PRO, bool FLAT>
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
    // The segment this work-group computes: tokens [start, end) of the unit
    // (sequence b, column r = kv head * gtiles + query-head tile); `direct`
    // segments hold the whole unit and write its output, the others write
    // partials for the merge kernel.
    int b, r, len, start, end;
    bool direct;
    __shared__ int fl_len[kLptMax];
    __shared__ int fl_pref[kLptMax + 1];
    __shared__ int fl_tot[kLptMax / kWave];
    int64_t fl_wc = 0, fl_pos = 0, fl_stop = 0, fl_row = 0, fl_row_later = 0;
    if constexpr (FLAT) {
        flat_prefix(a, S::kTpi, fl_len, fl_pref, fl_tot);
        constexpr int ng = kFlatGroups;
        // Work-groups go to the 8 XCDs round robin; consecutive shares run
        // on one XCD, so a column's rows (and the pages its sequences
        // share) meet in one L2.
        const int l = (unit & 7) * (ng >> 3) + (unit >> 3);
        // LDS reads are wave-uniform here; readfirstlane keeps the segment
        // bounds in scalar registers (uniform loop control, as for the other
        // modes).
        fl_wc = __builtin_amdgcn_readfirstlane(fl_pref[a.batch]);
        const int64_t total = fl_wc * per_seq;
        fl_pos = flat_share_start(l, total);
        fl_stop = flat_share_start(l + 1, total);
        if (fl_pos >= fl_stop) {
            if (threadIdx.x == 0) a.ws_flat[l] = FlatMergeDesc{-1, 0, 0, 0, total, 0};
            return;
        }
        r = (int)(fl_pos / fl_wc);
        b = flat_seq_of(fl_pref, a.batch, fl_pos - r * fl_wc);
        if (threadIdx.x == 0) {
            // The unit this share begins with: merged here when it began in
            // an earlier share and ends in this one.
            const int64_t first = (int64_t)r * fl_wc + fl_pref[b];
            const int64_t last = (int64_t)r * fl_wc + fl_pref[b + 1];
            FlatMergeDesc d{-1, 0, 0, 0, total, 0};
            if (first < fl_pos && last <= fl_stop) {
                const int64_t p0 = ((first + 1) * ng - 1) / total;  // share holding chunk `first`
                d.b = b;
                d.r = r;
                d.p0 = (int)p0;
                d.slot0 = flat_share_start(p0, total) < first ? 1 : 0;
            }
            a.ws_flat[l] = d;
        }
        // Partial rows: the share's first segment, then its last.
        fl_row = (int64_t)l * 2 * G;
        fl_row_later = fl_row + G;
        len = start = end = 0;
        direct = false;
    } else {
        b = unit / per_seq;
        r = unit - b * per_seq;
        if (a.lpt_batch > kWave) {
            // As below for 64 < batch <= kLptMax: thread s keeps sequence s's key
            // in LDS and counts the larger keys with broadcast reads.
            __shared__ int lpt_keys[kLptMax];
            __shared__ int lpt_pick;
            const int n = a.lpt_batch;
            const int half = (n + 1) / 2;
            const int rank = a.lpt_pair && b >= half ? n - 1 - (b - half) : b;
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
                if (g0 + g1 + g2 + g3 == rank) lpt_pick = tid;
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
            const int half = (n + 1) / 2;
            const int rank = a.lpt_pair && b >= half ? n - 1 - (b - half) : b;
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
                b = __builtin_ctzll(__ballot(lane < n && g0 + g1 + g2 + g3 == rank));
            }
            len = __builtin_amdgcn_readlane(key, b) >> 6;
        } else {
            len = seq_tokens(a.lens[b], a.capacity);
        }
        const int nparts = len > 0 ? (len + a.partition - 1) / a.partition : 1;
        if (part >= nparts) return;
        start = part * a.partition;
        end = min(start + a.partition, len);
        direct = nparts == 1;
    }

    for (;;) {
        if constexpr (FLAT) {
            // Chunks [first, last) of the column are this unit's.
            const int64_t first = (int64_t)r * fl_wc + __builtin_amdgcn_readfirstlane(fl_pref[b]);
            const int64_t last = (int64_t)r * fl_wc + __builtin_amdgcn_readfirstlane(fl_pref[b + 1]);
            len = __builtin_amdgcn_readfirstlane(fl_len[b]);
            start = (int)(fl_pos - first) * S::kTpi;
            end = min((int)(min(fl_stop, last) - first) * S::kTpi, len);
            direct = fl_pos == first && last <= fl_stop;
        }
        const int kvh = r / a.gtiles;
        const int h0 = kvh * a.group + (r - kvh * a.gtiles) * G;

        static_assert(!PRO || (S::kLpt == S::kChunks && S::kLpt >= 2), "prologue needs head_dim 16/32/64/128/256");
        // Fused prologue, with no barrier: the wave whose iterations hold the new
        // position writes its K/V row (and waits for that store before it loads
        // the row again); in mode 2 every wave rotates the tile's query rows
        // itself, into its own slice of LDS.  One row per kLpt lanes.
        __shared__ __attribute__((aligned(16))) uint16_t sm_q[PRO ? NW : 1][PRO ? G : 1][PRO ? D : 8];
        const int pos = len - 1;
        // Token t is read by wave ((t - start) / kTpi) mod NW.
        const bool owner = PRO && pos >= start && pos < end && ((pos - start) / S::kTpi) % NW == wave;
        if constexpr (PRO) {
            int64_t slot = -1;
            if (owner) {
                const int64_t page = a.tables[(int64_t)b * a.table_width +
                                              (a.block_shift >= 0 ? pos >> a.block_shift : pos / a.block_size)];
                if (page >= 0 && page < a.num_blocks)
                    slot = page * a.block_size + (a.block_shift >= 0 ? pos & (a.block_size - 1) : pos % a.block_size);
            }
            const int64_t cache_row = slot * a.kv_heads * D + (int64_t)kvh * D + 8 * c;
            const uint16_t* kv_src = a.new_k + (int64_t)b * a.k_stride + kvh * D + 8 * c;
            const uint16_t* v_src = a.new_v + (int64_t)b * a.v_stride + kvh * D + 8 * c;
            uint16_t* kdst = static_cast<uint16_t*>(const_cast<void*>(a.key_cache)) + cache_row;
            uint16_t* vdst = static_cast<uint16_t*>(const_cast<void*>(a.value_cache)) + cache_row;
            if (a.prologue == 1) {
                if (slot >= 0 && tl == 0) {
                    const u32x4 kx = *reinterpret_cast<const u32x4*>(kv_src);
                    const u32x4 vx = *reinterpret_cast<const u32x4*>(v_src);
                    *reinterpret_cast<u32x4*>(kdst) = kx;
                    *reinterpret_cast<u32x4*>(vdst) = vx;
                }
            } else {
                // Rows 0 .. G-1: the tile's query heads; row G (owner only): the new K.
                constexpr int kRowsPerWave = kWave / S::kLpt;
                const int rows = G + (slot >= 0 ? 1 : 0);
                for (int r0 = 0; r0 < rows; r0 += kRowsPerWave) {
                    const int row = r0 + tl;
                    const bool live = row < rows;
                    const bool is_k = row == G;
                    // Lanes past the list compute on zeros and store nothing (the
                    // sum of squares and the rotation exchange read every lane).
                    const uint16_t* src = is_k ? kv_src
                                               : static_cast<const uint16_t*>(a.query) + (int64_t)b * a.q_stride +
                                                     (int64_t)(h0 + (live ? row : 0)) * D + 8 * c;
                    const u32x4 zero = {0u, 0u, 0u, 0u};
                    const u32x4 xraw = *reinterpret_cast<const u32x4*>(src);
                    const u32x4 xv = live ? xraw : zero;
                    const u32x4 wv = *reinterpret_cast<const u32x4*>((is_k ? a.k_weight : a.q_weight) + 8 * c);
                    const int64_t trig = (int64_t)b * (D / 2) + (c % (S::kLpt / 2)) * 8;
                    const u32x4 cv = *reinterpret_cast<const u32x4*>(a.cos + trig);
                    const u32x4 sv = *reinterpret_cast<const u32x4*>(a.sin + trig);
                    const u32x4 rot = norm_rope_lanes<T, S::kLpt>(xv, wv, cv, sv, a.eps, c);
                    if (!live) continue;
                    if (is_k) {
                        const u32x4 vx = *reinterpret_cast<const u32x4*>(v_src);
                        *reinterpret_cast<u32x4*>(kdst) = rot;
                        *reinterpret_cast<u32x4*>(vdst) = vx;
                    } else {
                        *reinterpret_cast<u32x4*>(&sm_q[wave][row][8 * c]) = rot;
                        if (a.q_out && start == 0 && wave == 0)
                            *reinterpret_cast<u32x4*>(a.q_out + ((int64_t)b * a.q_heads + h0 + row) * D + 8 * c) = rot;
                    }
                }
            }
        }

        // Query slice of this lane for every head of the tile (8 elements each).
        uint32_t q[G][4];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            u32x4 w = {0u, 0u, 0u, 0u};
            if (PRO && a.prologue == 2) {
                if (chunk_ok) w = *reinterpret_cast<const u32x4*>(&sm_q[PRO ? wave : 0][PRO ? g : 0][PRO ? 8 * c : 0]);
            } else if (chunk_ok)
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
            // The owner's store of the new row completes before the row is read.
            if constexpr (PRO)
                if (owner && it <= pos && pos < it + S::kTpi) __builtin_amdgcn_s_waitcnt(0);
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
            if (direct) {
                static_cast<uint16_t*>(a.out)[bh * D + d] = T::from_float(sum > 0.f ? o / sum : 0.f);
            } else {
                const int64_t row = FLAT ? fl_row + g : bh * a.max_parts + part;
                a.ws_acc[row * D + d] = o;
                if (d == 0) {
                    a.ws_ml[row * 2] = mx;
                    a.ws_ml[row * 2 + 1] = sum;
                }
            }
        }
        if constexpr (!FLAT) return;
        // The share's next unit: the column's next sequence, or the first
        // sequence of the next column.
        fl_pos = (int64_t)r * fl_wc + __builtin_amdgcn_readfirstlane(fl_pref[b + 1]);
        if (fl_pos >= fl_stop) return;
        fl_row = fl_row_later;
        if (++b == a.batch) {
            b = 0;
            ++r;
        }
        __syncthreads();  // the next segment rewrites the wave-merge LDS
    }
}

template <typename T, int D, int G, int NW, bool STREAM, bool PRO>
void launch_decode_kernel(const DecodeArgs& a, dim3 grid, bool page_uniform, hipStream_t s) {
    if constexpr (NW == kFlatWaves && STREAM) {
        if (a.flat_groups > 0) {
            if (page_uniform)
                hipLaunchKernelGGL((paged_decode_kernel<T, D, G, true, NW, true, PRO, true>), grid, dim3(NW * kWave),
                                   0, s, a);
            else
                hipLaunchKernelGGL((paged_decode_kernel<T, D, G, false, NW, true, PRO, true>), grid, dim3(NW * kWave),
                                   0, s, a);
            return;
        }
    }
    if (page_uniform)
        hipLaunchKernelGGL((paged_decode_kernel<T, D, G, true, NW, STREAM, PRO, false>), grid, dim3(NW * kWave), 0, s,
                           a);
    else
        hipLaunchKernelGGL((paged_decode_kernel<T, D, G, false, NW, STREAM, PRO, false>), grid, dim3(NW * kWave), 0,
                           s, a);
}

// Head dims with a fused-prologue instantiation (one 16-byte chunk per lane).
template <int D>
constexpr bool decode_fused_capable() {
    return DecodeShape<D>::kLpt == DecodeShape<D>::kChunks && DecodeShape<D>::kLpt >= 2;
}

// The prologue instantiations, compiled in their own translation unit
// (paged_decode_fused.hip) so that the two halves build in parallel.
template <typename T, int D, int G, int NW, bool STREAM>
void launch_decode_fused(const DecodeArgs& a, dim3 grid, bool page_uniform, hipStream_t s);

}  // namespace mvme

/*
 * paged_ref.c -- C restatement of the paged-attention hot path.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (through oracle/c_oracle.py) as
 * an independent checker of the torch oracle and of the HIP kernels.  Never
 * linked into or called by the product library.
 *
 * Scalar loops with float64 accumulation; inputs are the exact fp32 values
 * of the fp16/bf16 data (converted by the bit-level routines below), so the
 * result is the real-number attention up to float64 rounding.
 *
 * Follows (reference dandan20031031/myvllm-mini-engine):
 *   decode   -- mini_engine/kernels/fallback.py:27-64 (semantics),
 *               benchmarks/compare_paged_backends.py:58-72 (fp32 oracle)
 *   prefill  -- mini_engine/kernels/prefill.py:114-131 (mask k <= start+i)
 *   scatter  -- mini_engine/kernels/data.py:120-125 (index_copy_ of rows)
 *   slots    -- mini_engine/engine/batch.py:110-112
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* IEEE binary16 -> binary32, exact (normals, subnormals, inf, nan). */
float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t exp = (h >> 10) & 0x1f;
    const uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float v = (float)man * (1.0f / 16777216.0f);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* bfloat16 -> binary32 is a 16-bit shift. */
float oracle_bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

void oracle_convert(const uint16_t* src, float* dst, int64_t n, int is_bf16) {
    for (int64_t i = 0; i < n; ++i)
        dst[i] = is_bf16 ? oracle_bf16_to_f32(src[i]) : oracle_f16_to_f32(src[i]);
}

/* Physical row (page*block_size + offset) of logical token t, or -1. */
static int64_t token_row(const int64_t* table, int64_t width, int64_t t, int64_t block_size,
                         int64_t num_blocks) {
    const int64_t block = t / block_size;
    if (block >= width) return -1;
    const int64_t page = table[block];
    if (page < 0 || page >= num_blocks) return -1;
    return page * block_size + t % block_size;
}

/* Attention of one query row over keys [0, n) of one sequence/kv head. */
static void attend(double* out, const float* q, const float* kc, const float* vc,
                   const int64_t* table, int64_t width, int64_t n, int64_t kvh, int64_t kv_heads,
                   int64_t d, int64_t block_size, int64_t num_blocks, double* scores) {
    const double scale = 1.0 / sqrt((double)d);
    double mx = -INFINITY;
    for (int64_t t = 0; t < n; ++t) {
        const int64_t row = token_row(table, width, t, block_size, num_blocks);
        if (row < 0) { scores[t] = -INFINITY; continue; }
        const float* k = kc + (row * kv_heads + kvh) * d;
        double s = 0.0;
        for (int64_t e = 0; e < d; ++e) s += (double)q[e] * (double)k[e];
        scores[t] = s * scale;
        if (scores[t] > mx) mx = scores[t];
    }
    for (int64_t e = 0; e < d; ++e) out[e] = 0.0;
    if (mx == -INFINITY) return;
    double sum = 0.0;
    for (int64_t t = 0; t < n; ++t) {
        const double p = scores[t] == -INFINITY ? 0.0 : exp(scores[t] - mx);
        scores[t] = p;
        sum += p;
    }
    for (int64_t t = 0; t < n; ++t) {
        if (scores[t] == 0.0) continue;
        const int64_t row = token_row(table, width, t, block_size, num_blocks);
        const float* v = vc + (row * kv_heads + kvh) * d;
        for (int64_t e = 0; e < d; ++e) out[e] += scores[t] * (double)v[e];
    }
    for (int64_t e = 0; e < d; ++e) out[e] /= sum;
}

/*
 * Decode: out[b, h, :] over the first lens[b] tokens of sequence b.
 * Sequences with lens <= 0 or beyond the table capacity give zeros.
 * `scratch` holds at least width*block_size doubles.
 */
void oracle_paged_decode(double* out, const float* q, const float* kc, const float* vc,
                         const int64_t* tables, const int64_t* lens, int64_t batch, int64_t q_heads,
                         int64_t kv_heads, int64_t d, int64_t num_blocks, int64_t block_size,
                         int64_t width, double* scratch) {
    const int64_t group = q_heads / kv_heads;
    for (int64_t b = 0; b < batch; ++b) {
        int64_t n = lens[b];
        if (n <= 0 || n > width * block_size) n = 0;
        for (int64_t h = 0; h < q_heads; ++h)
            attend(out + (b * q_heads + h) * d, q + (b * q_heads + h) * d, kc, vc, tables + b * width,
                   width, n, h / group, kv_heads, d, block_size, num_blocks, scratch);
    }
}

/*
 * Ragged paged prefill: packed row i of sequence s attends keys
 * [0, starts[s] + i] (only those < lens[s]).
 */
void oracle_paged_prefill(double* out, const float* q, const float* kc, const float* vc,
                          const int64_t* cu, const int64_t* starts, const int64_t* tables,
                          const int64_t* lens, int64_t num_seqs, int64_t q_heads, int64_t kv_heads,
                          int64_t d, int64_t num_blocks, int64_t block_size, int64_t width,
                          double* scratch) {
    const int64_t group = q_heads / kv_heads;
    for (int64_t s = 0; s < num_seqs; ++s) {
        for (int64_t row = cu[s]; row < cu[s + 1]; ++row) {
            const int64_t pos = starts[s] + (row - cu[s]);
            int64_t n = pos + 1;
            if (pos < 0 || pos >= lens[s] || pos >= width * block_size) n = 0;
            for (int64_t h = 0; h < q_heads; ++h)
                attend(out + (row * q_heads + h) * d, q + (row * q_heads + h) * d, kc, vc,
                       tables + s * width, width, n, h / group, kv_heads, d, block_size, num_blocks,
                       scratch);
        }
    }
}

/* Row scatter by slot (bit copy); out-of-range slots are skipped. */
void oracle_scatter_slots(uint16_t* kc, uint16_t* vc, const int64_t* slots, const uint16_t* k,
                          const uint16_t* v, int64_t tokens, int64_t capacity, int64_t row) {
    for (int64_t t = 0; t < tokens; ++t) {
        const int64_t s = slots[t];
        if (s < 0 || s >= capacity) continue;
        memcpy(kc + s * row, k + t * row, (size_t)row * 2);
        memcpy(vc + s * row, v + t * row, (size_t)row * 2);
    }
}

/* Slot of each packed prefill token (batch.py:110-112 rule). */
void oracle_prefill_slots(int64_t* slots, const int64_t* cu, const int64_t* starts,
                          const int64_t* tables, int64_t num_seqs, int64_t width, int64_t block_size) {
    for (int64_t s = 0; s < num_seqs; ++s)
        for (int64_t row = cu[s]; row < cu[s + 1]; ++row) {
            const int64_t pos = starts[s] + (row - cu[s]);
            slots[row] = tables[s * width + pos / block_size] * block_size + pos % block_size;
        }
}

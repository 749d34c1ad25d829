/*
 * CPU oracle for the paged KV-cache + attention path. TEST INFRASTRUCTURE
 * ONLY: the checker for tests/, smoke() and bench.py's CPU baseline. The
 * product never links or calls it. See oracle.h for the contract of each
 * function and the reference lines it restates.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- 16-bit float conversions ------------------------------------------ */

static uint32_t f32_bits(float value)
{
    uint32_t bits;
    memcpy(&bits, &value, sizeof bits);
    return bits;
}

static float bits_f32(uint32_t bits)
{
    float value;
    memcpy(&value, &bits, sizeof value);
    return value;
}

/* src/tensor/types.h:60-75: NaN keeps its upper payload with the quiet bit
 * forced; everything else rounds to nearest, ties to even, by adding
 * 0x7FFF + lsb before truncating. */
uint16_t orc_bf16_from_f32(float value)
{
    uint32_t bits = f32_bits(value);
    if ((bits & 0x7FFFFFFFu) > 0x7F800000u)
        return (uint16_t)((bits >> 16) | 0x0040u);
    bits += 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

/* src/tensor/types.h:83-88: the bf16 bits are the upper half of an f32. */
float orc_bf16_to_f32(uint16_t bits)
{
    return bits_f32((uint32_t)bits << 16);
}

/* IEEE 754 binary16 from binary32, round to nearest even. NaN keeps the top
 * ten payload bits and is made quiet. */
uint16_t orc_f16_from_f32(float value)
{
    const uint32_t bits = f32_bits(value);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t exponent = (bits >> 23) & 0xFFu;
    const uint32_t mantissa = bits & 0x7FFFFFu;
    if (exponent == 0xFFu) {
        if (mantissa)
            return (uint16_t)(sign | 0x7C00u | 0x0200u | (mantissa >> 13));
        return (uint16_t)(sign | 0x7C00u);
    }
    const int e = (int)exponent - 127 + 15; /* biased binary16 exponent */
    if (e >= 31)
        return (uint16_t)(sign | 0x7C00u);
    if (e >= 1) {
        /* normal: keep 10 mantissa bits, round the 13 dropped bits; a carry
         * out of the mantissa correctly bumps the exponent (up to infinity) */
        uint32_t result = ((uint32_t)e << 10) | (mantissa >> 13);
        const uint32_t dropped = mantissa & 0x1FFFu;
        if (dropped > 0x1000u || (dropped == 0x1000u && (result & 1u)))
            ++result;
        return (uint16_t)(sign | result);
    }
    if (exponent == 0)
        return sign; /* binary32 zero or subnormal: far below 2^-25 */
    /* subnormal binary16: value = full * 2^(exponent-150); unit is 2^-24 */
    const uint32_t full = mantissa | 0x800000u;
    const int shift = 126 - (int)exponent; /* = 14 - e, at least 14 */
    if (shift >= 25)
        return sign; /* below half of the smallest subnormal */
    uint32_t q = full >> shift;
    const uint32_t rest = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rest > half || (rest == half && (q & 1u)))
        ++q;
    return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t bits)
{
    const uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    const uint32_t exponent = (bits >> 10) & 0x1Fu;
    const uint32_t mantissa = bits & 0x3FFu;
    if (exponent == 0x1Fu)
        return bits_f32(sign | 0x7F800000u | (mantissa << 13));
    if (exponent == 0) {
        /* zero or subnormal: mantissa * 2^-24 is exact in binary32 */
        const float magnitude = (float)mantissa * 0x1p-24f;
        return sign ? -magnitude : magnitude;
    }
    return bits_f32(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

size_t orc_dtype_size(int dtype)
{
    return dtype == ORC_F32 ? 4 : 2;
}

static float load_value(const void* base, size_t index, int dtype)
{
    switch (dtype) {
    case ORC_F32:
        return ((const float*)base)[index];
    case ORC_BF16:
        return orc_bf16_to_f32(((const uint16_t*)base)[index]);
    default:
        return orc_f16_to_f32(((const uint16_t*)base)[index]);
    }
}

static void store_value(void* base, size_t index, int dtype, float value)
{
    switch (dtype) {
    case ORC_F32:
        ((float*)base)[index] = value;
        break;
    case ORC_BF16:
        ((uint16_t*)base)[index] = orc_bf16_from_f32(value);
        break;
    default:
        ((uint16_t*)base)[index] = orc_f16_from_f32(value);
        break;
    }
}

void orc_convert_from_f32(const float* in, void* out, size_t n, int dtype)
{
    for (size_t i = 0; i < n; ++i)
        store_value(out, i, dtype, in[i]);
}

void orc_convert_to_f32(const void* in, float* out, size_t n, int dtype)
{
    for (size_t i = 0; i < n; ++i)
        out[i] = load_value(in, i, dtype);
}

/* ---- mt19937_64 ---------------------------------------------------------- */
/* Parameters of std::mt19937_64 ([rand.predef] in the C++ standard):
 * w=64 n=312 m=156 r=31 a=0xB5026F5AA96619E9 u=29 d=0x5555555555555555
 * s=17 b=0x71D67FFFEDA60000 t=37 c=0xFFF7EEE000000000 l=43
 * f=6364136223846793005. */
#define MT_N 312
#define MT_M 156

void orc_mt64_seed(orc_mt64* rng, uint64_t seed)
{
    rng->state[0] = seed;
    for (size_t i = 1; i < MT_N; ++i) {
        const uint64_t prev = rng->state[i - 1];
        rng->state[i] = 6364136223846793005ULL * (prev ^ (prev >> 62)) + (uint64_t)i;
    }
    rng->index = MT_N;
}

static void mt64_twist(orc_mt64* rng)
{
    const uint64_t upper = 0xFFFFFFFF80000000ULL;
    const uint64_t lower = 0x7FFFFFFFULL;
    for (size_t i = 0; i < MT_N; ++i) {
        const uint64_t y = (rng->state[i] & upper) | (rng->state[(i + 1) % MT_N] & lower);
        uint64_t next = rng->state[(i + MT_M) % MT_N] ^ (y >> 1);
        if (y & 1u)
            next ^= 0xB5026F5AA96619E9ULL;
        rng->state[i] = next;
    }
    rng->index = 0;
}

uint64_t orc_mt64_next(orc_mt64* rng)
{
    if (rng->index >= MT_N)
        mt64_twist(rng);
    uint64_t x = rng->state[rng->index++];
    x ^= (x >> 29) & 0x5555555555555555ULL;
    x ^= (x << 17) & 0x71D67FFFEDA60000ULL;
    x ^= (x << 37) & 0xFFF7EEE000000000ULL;
    x ^= x >> 43;
    return x;
}

double orc_uniform(orc_mt64* rng)
{
    return (double)(orc_mt64_next(rng) >> 11) * 0x1p-53;
}

void orc_fill_normal(orc_mt64* rng, void* out, size_t n, int dtype)
{
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = orc_uniform(rng);
        const double u2 = orc_uniform(rng);
        const double radius = sqrt(-2.0 * log(1.0 - u1));
        const double angle = two_pi * u2;
        store_value(out, i, dtype, (float)(radius * cos(angle)));
        if (i + 1 < n)
            store_value(out, i + 1, dtype, (float)(radius * sin(angle)));
    }
}

void orc_permutation(orc_mt64* rng, uint32_t* out, size_t n)
{
    for (size_t i = 0; i < n; ++i)
        out[i] = (uint32_t)i;
    for (size_t i = n; i > 1; --i) {
        const size_t j = (size_t)(orc_mt64_next(rng) % (uint64_t)i);
        const uint32_t t = out[i - 1];
        out[i - 1] = out[j];
        out[j] = t;
    }
}

uint64_t orc_uniform_int(orc_mt64* rng, uint64_t lo, uint64_t hi)
{
    return lo + orc_mt64_next(rng) % (hi - lo + 1);
}

/* ---- Page allocator ------------------------------------------------------ */

struct orc_block_manager {
    size_t block_count;
    size_t block_size;
    size_t max_sequences;
    uint32_t* ring; /* free list as a ring buffer of block_count entries */
    size_t head;
    size_t size;
    uint32_t** tables;
    size_t* lengths;
    size_t* capacities;
};

int orc_bm_make(size_t block_count, size_t block_size, size_t max_sequences,
                orc_block_manager** out)
{
    if (!block_count)
        return 1;
    if (!block_size)
        return 2;
    if (block_count - 1 > (size_t)UINT32_MAX)
        return 3;
    orc_block_manager* bm = calloc(1, sizeof *bm);
    bm->block_count = block_count;
    bm->block_size = block_size;
    bm->max_sequences = max_sequences;
    bm->ring = malloc(block_count * sizeof(uint32_t));
    for (size_t i = 0; i < block_count; ++i)
        bm->ring[i] = (uint32_t)i; /* src/block_manager.cc:21-22 */
    bm->head = 0;
    bm->size = block_count;
    bm->tables = calloc(max_sequences, sizeof(uint32_t*));
    bm->lengths = calloc(max_sequences, sizeof(size_t));
    bm->capacities = calloc(max_sequences, sizeof(size_t));
    *out = bm;
    return 0;
}

void orc_bm_destroy(orc_block_manager* bm)
{
    if (!bm)
        return;
    for (size_t i = 0; i < bm->max_sequences; ++i)
        free(bm->tables[i]);
    free(bm->tables);
    free(bm->lengths);
    free(bm->capacities);
    free(bm->ring);
    free(bm);
}

/* src/block_manager.cc:32-53 */
int orc_bm_reserve(orc_block_manager* bm, size_t seq, size_t tokens)
{
    if (!tokens)
        return 2;
    const size_t required = 1 + (tokens - 1) / bm->block_size;
    const size_t existing = bm->lengths[seq];
    if (required <= existing)
        return 0;
    const size_t extra = required - existing;
    if (extra > bm->size)
        return 1;
    if (bm->capacities[seq] < required) {
        bm->tables[seq] = realloc(bm->tables[seq], required * sizeof(uint32_t));
        bm->capacities[seq] = required;
    }
    for (size_t i = 0; i < extra; ++i) {
        bm->tables[seq][existing + i] = bm->ring[bm->head];
        bm->head = (bm->head + 1) % bm->block_count;
        --bm->size;
    }
    bm->lengths[seq] = required;
    return 0;
}

/* src/block_manager.cc:55-64 */
void orc_bm_release(orc_block_manager* bm, size_t seq)
{
    for (size_t i = 0; i < bm->lengths[seq]; ++i) {
        bm->ring[(bm->head + bm->size) % bm->block_count] = bm->tables[seq][i];
        ++bm->size;
    }
    bm->lengths[seq] = 0;
}

size_t orc_bm_free_count(const orc_block_manager* bm)
{
    return bm->size;
}

int orc_prepare_paged_batch(size_t n_items, const uint32_t* token_count,
                            const uint32_t* tables, const size_t* table_start,
                            const uint32_t* table_len, const uint32_t* positions,
                            size_t max_positions, size_t block_count, size_t block_size,
                            uint32_t* flat_table, uint32_t* slots, uint32_t* offsets,
                            uint32_t* lengths)
{
    /* src/model_batch.cc:132-139: empty batch, zero geometry */
    if (!n_items || !block_size || !block_count)
        return 1;
    size_t flat = 0, row = 0;
    for (size_t i = 0; i < n_items; ++i) {
        /* :151-160: the item's rows and its table */
        if (!token_count[i] || !table_len[i] || flat > UINT32_MAX
            || table_len[i] > UINT32_MAX - flat)
            return 1;
        const uint32_t* table = tables + table_start[i];
        const uint32_t offset = (uint32_t)flat;
        /* :162-169: append the table, every entry < block_count */
        for (size_t b = 0; b < table_len[i]; ++b) {
            if (table[b] >= block_count)
                return 1;
            flat_table[flat++] = table[b];
        }
        /* :171-192: one slot, offset and length per row */
        for (size_t t = 0; t < token_count[i]; ++t, ++row) {
            const uint32_t position = positions[row];
            if (position >= max_positions)
                return 1;
            const size_t logical = position / block_size;
            if (logical >= table_len[i])
                return 1;
            const size_t slot = (size_t)table[logical] * block_size + position % block_size;
            if (slot > UINT32_MAX)
                return 1;
            slots[row] = (uint32_t)slot;
            offsets[row] = offset;
            lengths[row] = table_len[i];
        }
    }
    return 0;
}

int orc_decode_step_host(orc_block_manager* bm, size_t n, uint32_t* lengths,
                         uint32_t* scratch_tables, size_t* scratch_start, uint32_t* scratch_len,
                         uint32_t* token_count, uint32_t* flat_table, uint32_t* slots,
                         uint32_t* offsets, uint32_t* row_lengths, size_t block_count,
                         size_t block_size)
{
    size_t at = 0;
    for (size_t s = 0; s < n; ++s) {
        if (orc_bm_reserve(bm, s, (size_t)lengths[s] + 1))
            return 1;
        scratch_start[s] = at;
        scratch_len[s] = (uint32_t)orc_bm_table(bm, s, scratch_tables + at, (size_t)-1);
        at += scratch_len[s];
        token_count[s] = 1;
    }
    /* the new token of sequence s sits at position lengths[s] */
    if (orc_prepare_paged_batch(n, token_count, scratch_tables, scratch_start, scratch_len,
                                lengths, (size_t)UINT32_MAX, block_count, block_size, flat_table,
                                slots, offsets, row_lengths))
        return 1;
    for (size_t s = 0; s < n; ++s)
        lengths[s] += 1;
    return 0;
}

size_t orc_bm_table(const orc_block_manager* bm, size_t seq, uint32_t* out, size_t cap)
{
    const size_t n = bm->lengths[seq];
    for (size_t i = 0; i < n && i < cap; ++i)
        out[i] = bm->tables[seq][i];
    return n;
}

/* ---- Slots and addressing ------------------------------------------------ */

int orc_slot(const uint32_t* table, size_t table_length, uint32_t position, uint32_t block_size,
             uint32_t* slot)
{
    const size_t logical = position / block_size;
    if (logical >= table_length)
        return -1;
    const uint64_t value = (uint64_t)table[logical] * block_size + position % block_size;
    if (value > UINT32_MAX)
        return -1;
    *slot = (uint32_t)value;
    return 0;
}

int orc_element_offset(const orc_geometry* g, size_t layer, size_t block, size_t token,
                       size_t head, size_t feature, size_t* offset)
{
    if (layer >= g->layers)
        return 7;
    if (block >= g->blocks)
        return 8;
    if (token >= g->block_size)
        return 9;
    if (head >= g->kv_heads)
        return 10;
    if (feature >= g->head_dim)
        return 11;
    *offset = (((layer * g->blocks + block) * g->block_size + token) * g->kv_heads + head)
            * g->head_dim
        + feature;
    return 0;
}

/* ---- Append and gather --------------------------------------------------- */

void orc_store_kv(void* key_cache, void* value_cache, const void* keys, const void* values,
                  const uint32_t* slots, size_t rows, size_t feature_count, size_t layer,
                  size_t slot_count, size_t elem_size)
{
    const size_t row_bytes = feature_count * elem_size;
    for (size_t row = 0; row < rows; ++row) {
        if (slots[row] >= slot_count)
            continue;
        const size_t target = (layer * slot_count + slots[row]) * row_bytes;
        memcpy((char*)key_cache + target, (const char*)keys + row * row_bytes, row_bytes);
        memcpy((char*)value_cache + target, (const char*)values + row * row_bytes, row_bytes);
    }
}

void orc_gather(const void* key_cache, const void* value_cache, const uint32_t* table,
                size_t n_tokens, size_t layer, size_t slot_count, size_t block_size,
                size_t feature_count, size_t elem_size, void* out_keys, void* out_values)
{
    const size_t row_bytes = feature_count * elem_size;
    for (size_t token = 0; token < n_tokens; ++token) {
        const size_t slot = (size_t)table[token / block_size] * block_size + token % block_size;
        const size_t source = (layer * slot_count + slot) * row_bytes;
        memcpy((char*)out_keys + token * row_bytes, (const char*)key_cache + source, row_bytes);
        memcpy((char*)out_values + token * row_bytes, (const char*)value_cache + source,
               row_bytes);
    }
}

/* ---- Attention ------------------------------------------------------------- */

/* The row checks of attention.metal:70-78 (kernel early return). */
static int row_valid(const orc_attention_args* a, size_t row)
{
    const uint32_t position = a->positions[row];
    const uint32_t offset = a->offsets[row];
    const uint32_t length = a->lengths[row];
    return offset <= a->table_entries && length <= a->table_entries - offset
        && position / a->g->block_size < length;
}

static size_t cache_base(const orc_attention_args* a, size_t row, size_t token, size_t kv_head)
{
    const orc_geometry* g = a->g;
    const size_t block = a->table[a->offsets[row] + token / g->block_size];
    const size_t slot = block * g->block_size + token % g->block_size;
    return ((a->layer * g->blocks * g->block_size + slot) * g->kv_heads + kv_head) * g->head_dim;
}

static float dot_f32(const orc_attention_args* a, size_t q_base, size_t k_base)
{
    float score = 0.0f;
    for (size_t f = 0; f < a->g->head_dim; ++f)
        score += load_value(a->queries, q_base + f, a->q_dtype)
            * load_value(a->key_cache, k_base + f, a->cache_dtype);
    return score;
}

/* One (row, q_head) of paged_attention_f32, tokens [begin, end). Writes the
 * running max, denominator and unnormalised accumulator. */
static void online_range(const orc_attention_args* a, size_t row, size_t head, size_t begin,
                         size_t end, float* max_out, float* sum_out, float* acc)
{
    const size_t D = a->g->head_dim;
    const size_t kv_head = head / (a->q_heads / a->g->kv_heads);
    const size_t q_base = (row * a->q_heads + head) * D;
    float running_max = -INFINITY, running_sum = 0.0f;
    for (size_t f = 0; f < D; ++f)
        acc[f] = 0.0f;
    for (size_t token = begin; token < end; ++token) {
        const size_t base = cache_base(a, row, token, kv_head);
        const float score = dot_f32(a, q_base, base) * a->scale;
        const float new_max = running_max > score ? running_max : score;
        const float rescale = expf(running_max - new_max);
        const float weight = expf(score - new_max);
        running_max = new_max;
        running_sum = running_sum * rescale + weight;
        for (size_t f = 0; f < D; ++f)
            acc[f] = acc[f] * rescale + load_value(a->value_cache, base + f, a->cache_dtype) * weight;
    }
    *max_out = running_max;
    *sum_out = running_sum;
}

int orc_attention_online(const orc_attention_args* a, float* out)
{
    const size_t D = a->g->head_dim;
    int status = 0;
    for (size_t row = 0; row < a->rows; ++row) {
        if (!row_valid(a, row)) {
            status = -1;
            continue;
        }
        for (size_t head = 0; head < a->q_heads; ++head) {
            float m, l;
            float* acc = out + (row * a->q_heads + head) * D;
            online_range(a, row, head, 0, (size_t)a->positions[row] + 1, &m, &l, acc);
            for (size_t f = 0; f < D; ++f)
                acc[f] /= l;
        }
    }
    return status;
}

int orc_attention_reference(const orc_attention_args* a, double* out)
{
    const size_t D = a->g->head_dim;
    int status = 0;
    double* scores = NULL;
    size_t capacity = 0;
    for (size_t row = 0; row < a->rows; ++row) {
        if (!row_valid(a, row)) {
            status = -1;
            continue;
        }
        const size_t count = (size_t)a->positions[row] + 1;
        if (count > capacity) {
            scores = realloc(scores, count * sizeof(double));
            capacity = count;
        }
        for (size_t head = 0; head < a->q_heads; ++head) {
            const size_t kv_head = head / (a->q_heads / a->g->kv_heads);
            const size_t q_base = (row * a->q_heads + head) * D;
            double maximum = -INFINITY;
            for (size_t token = 0; token < count; ++token) {
                const size_t base = cache_base(a, row, token, kv_head);
                double score = 0.0;
                for (size_t f = 0; f < D; ++f)
                    score += (double)load_value(a->queries, q_base + f, a->q_dtype)
                        * (double)load_value(a->key_cache, base + f, a->cache_dtype);
                scores[token] = score * (double)a->scale;
                if (scores[token] > maximum)
                    maximum = scores[token];
            }
            double* o = out + q_base;
            for (size_t f = 0; f < D; ++f)
                o[f] = 0.0;
            double denominator = 0.0;
            for (size_t token = 0; token < count; ++token) {
                const double weight = exp(scores[token] - maximum);
                denominator += weight;
                const size_t base = cache_base(a, row, token, kv_head);
                for (size_t f = 0; f < D; ++f)
                    o[f] += weight * (double)load_value(a->value_cache, base + f, a->cache_dtype);
            }
            for (size_t f = 0; f < D; ++f)
                o[f] /= denominator;
        }
    }
    free(scores);
    return status;
}

int orc_attention_split(const orc_attention_args* a, size_t chunk_size, float* out)
{
    const size_t D = a->g->head_dim;
    int status = 0;
    float* partial_acc = NULL;
    float* partial_max = NULL;
    float* partial_sum = NULL;
    size_t capacity = 0;
    for (size_t row = 0; row < a->rows; ++row) {
        if (!row_valid(a, row)) {
            status = -1;
            continue;
        }
        const size_t end = (size_t)a->positions[row] + 1;
        const size_t chunks = (size_t)a->positions[row] / chunk_size + 1;
        if (chunks > capacity) {
            partial_acc = realloc(partial_acc, chunks * D * sizeof(float));
            partial_max = realloc(partial_max, chunks * sizeof(float));
            partial_sum = realloc(partial_sum, chunks * sizeof(float));
            capacity = chunks;
        }
        for (size_t head = 0; head < a->q_heads; ++head) {
            /* attention.metal:492-509: each chunk covers
             * [c*chunk, min(pos + 1, c*chunk + chunk)); empty chunks are (-inf, 0, 0) */
            for (size_t c = 0; c < chunks; ++c) {
                const size_t begin = c * chunk_size;
                const size_t stop = end < begin + chunk_size ? end : begin + chunk_size;
                if (begin >= stop) {
                    partial_max[c] = -INFINITY;
                    partial_sum[c] = 0.0f;
                    for (size_t f = 0; f < D; ++f)
                        partial_acc[c * D + f] = 0.0f;
                    continue;
                }
                online_range(a, row, head, begin, stop, &partial_max[c], &partial_sum[c],
                             partial_acc + c * D);
            }
            /* attention.metal:588-614 */
            float global_max = -INFINITY;
            for (size_t c = 0; c < chunks; ++c)
                if (partial_max[c] > global_max)
                    global_max = partial_max[c];
            float denominator = 0.0f;
            float* o = out + (row * a->q_heads + head) * D;
            for (size_t f = 0; f < D; ++f)
                o[f] = 0.0f;
            for (size_t c = 0; c < chunks; ++c) {
                const float scale = expf(partial_max[c] - global_max);
                denominator += partial_sum[c] * scale;
                for (size_t f = 0; f < D; ++f)
                    o[f] += partial_acc[c * D + f] * scale;
            }
            for (size_t f = 0; f < D; ++f)
                o[f] /= denominator;
        }
    }
    free(partial_acc);
    free(partial_max);
    free(partial_sum);
    return status;
}

size_t orc_query_tiles(const uint32_t* positions, const uint32_t* offsets,
                       const uint32_t* lengths, size_t rows, uint32_t* starts,
                       uint32_t* tile_lengths, int* shared)
{
    const size_t max_rows = 8;
    size_t count = 0;
    *shared = 0;
    size_t row = 0;
    while (row < rows) {
        size_t n = 1;
        while (n < max_rows && row + n < rows && offsets[row + n] == offsets[row]
               && lengths[row + n] == lengths[row]
               && positions[row + n] == positions[row + n - 1] + 1)
            ++n;
        starts[count] = (uint32_t)row;
        tile_lengths[count] = (uint32_t)n;
        ++count;
        if (n > 1)
            *shared = 1;
        row += n;
    }
    return count;
}

int orc_attention_prefill_tiles(const orc_attention_args* a, const uint32_t* tile_starts,
                                const uint32_t* tile_lengths, size_t tile_count, float* out)
{
    enum { QT = 8, KT = 16 };
    const size_t D = a->g->head_dim;
    float* acc = malloc(QT * D * sizeof(float));
    float* keys = malloc(KT * D * sizeof(float));
    float* vals = malloc(KT * D * sizeof(float));
    int status = 0;
    for (size_t tile = 0; tile < tile_count; ++tile) {
        const size_t start = tile_starts[tile];
        const size_t n_rows = tile_lengths[tile];
        if (!n_rows || n_rows > QT || start >= a->rows || n_rows > a->rows - start) {
            status = -1;
            continue;
        }
        const size_t final_position = a->positions[start + n_rows - 1];
        /* the tile uses the first row's table (attention.metal:290-291) */
        if (!(a->offsets[start] <= a->table_entries
              && a->lengths[start] <= a->table_entries - a->offsets[start]
              && final_position / a->g->block_size < a->lengths[start])) {
            status = -1;
            continue;
        }
        for (size_t head = 0; head < a->q_heads; ++head) {
            const size_t kv_head = head / (a->q_heads / a->g->kv_heads);
            float running_max[QT], running_sum[QT], scores[QT][KT];
            for (size_t q = 0; q < QT; ++q) {
                running_max[q] = -INFINITY;
                running_sum[q] = 0.0f;
            }
            for (size_t i = 0; i < n_rows * D; ++i)
                acc[i] = 0.0f;
            for (size_t begin = 0; begin <= final_position; begin += KT) {
                const size_t n_keys = final_position + 1 - begin < KT ? final_position + 1 - begin
                                                                      : KT;
                for (size_t k = 0; k < n_keys; ++k) {
                    const size_t base = cache_base(a, start, begin + k, kv_head);
                    for (size_t f = 0; f < D; ++f) {
                        keys[k * D + f] = load_value(a->key_cache, base + f, a->cache_dtype);
                        vals[k * D + f] = load_value(a->value_cache, base + f, a->cache_dtype);
                    }
                }
                for (size_t q = 0; q < n_rows; ++q) {
                    const size_t q_base = ((start + q) * a->q_heads + head) * D;
                    for (size_t k = 0; k < n_keys; ++k) {
                        float s = 0.0f;
                        for (size_t f = 0; f < D; ++f)
                            s += load_value(a->queries, q_base + f, a->q_dtype) * keys[k * D + f];
                        s *= a->scale;
                        scores[q][k] = begin + k <= a->positions[start + q] ? s : -INFINITY;
                    }
                    float tile_max = -INFINITY;
                    for (size_t k = 0; k < n_keys; ++k)
                        if (scores[q][k] > tile_max)
                            tile_max = scores[q][k];
                    const float new_max = running_max[q] > tile_max ? running_max[q] : tile_max;
                    const float rescale = expf(running_max[q] - new_max);
                    float tile_sum = 0.0f;
                    for (size_t k = 0; k < n_keys; ++k) {
                        scores[q][k] = expf(scores[q][k] - new_max);
                        tile_sum += scores[q][k];
                    }
                    running_max[q] = new_max;
                    running_sum[q] = running_sum[q] * rescale + tile_sum;
                    for (size_t f = 0; f < D; ++f) {
                        float value = acc[q * D + f] * rescale;
                        for (size_t k = 0; k < n_keys; ++k)
                            value += scores[q][k] * vals[k * D + f];
                        acc[q * D + f] = value;
                    }
                }
            }
            for (size_t q = 0; q < n_rows; ++q) {
                float* o = out + ((start + q) * a->q_heads + head) * D;
                for (size_t f = 0; f < D; ++f)
                    o[f] = acc[q * D + f] / running_sum[q];
            }
        }
    }
    free(acc);
    free(keys);
    free(vals);
    return status;
}

/* ---- Checkpoints and page copies ------------------------------------------ */

void orc_copy_prefix(void* paged, void* packed, const uint32_t* blocks, const orc_geometry* g,
                     size_t tokens, size_t elem_size, int restore)
{
    const size_t token_bytes = g->kv_heads * g->head_dim * elem_size;
    const size_t block_bytes = g->block_size * token_bytes;
    const size_t layer_bytes = g->blocks * block_bytes;
    for (size_t layer = 0; layer < g->layers; ++layer) {
        for (size_t token = 0; token < tokens; token += g->block_size) {
            const size_t paged_offset = layer * layer_bytes + blocks[token / g->block_size] * block_bytes;
            const size_t packed_offset = (layer * tokens + token) * token_bytes;
            const size_t count = tokens - token < g->block_size ? tokens - token : g->block_size;
            if (restore)
                memcpy((char*)paged + paged_offset, (const char*)packed + packed_offset,
                       count * token_bytes);
            else
                memcpy((char*)packed + packed_offset, (const char*)paged + paged_offset,
                       count * token_bytes);
        }
    }
}

void orc_copy_blocks(void* key_cache, void* value_cache, const orc_geometry* g,
                     const uint32_t* src, const uint32_t* dst, size_t n, size_t elem_size)
{
    const size_t block_bytes = g->block_size * g->kv_heads * g->head_dim * elem_size;
    const size_t layer_bytes = g->blocks * block_bytes;
    for (size_t layer = 0; layer < g->layers; ++layer) {
        for (size_t i = 0; i < n; ++i) {
            const size_t from = layer * layer_bytes + src[i] * block_bytes;
            const size_t to = layer * layer_bytes + dst[i] * block_bytes;
            memmove((char*)key_cache + to, (const char*)key_cache + from, block_bytes);
            memmove((char*)value_cache + to, (const char*)value_cache + from, block_bytes);
        }
    }
}

/* ---- Rotary position embedding ---------------------------------------------- */

void orc_rope_frequencies(float theta, size_t rotary_dim, float* out)
{
    for (size_t pair = 0; pair < rotary_dim / 2; ++pair) {
        const float exponent = -2.0f * (float)pair / (float)rotary_dim;
        out[pair] = powf(theta, exponent);
    }
}

int orc_rope(const void* in, void* out, int dtype, size_t rows, size_t heads, size_t head_dim,
             const uint32_t* positions, float theta, size_t rotary_dim)
{
    if (rotary_dim == 0)
        rotary_dim = head_dim;
    if (head_dim % 2 || rotary_dim % 2 || rotary_dim > head_dim || !isfinite(theta)
        || theta <= 0.0f)
        return -1;
    const size_t width = heads * head_dim;
    float* x = malloc(rows * width * sizeof(float));
    float* y = malloc(rows * width * sizeof(float));
    float* freq = malloc((rotary_dim / 2 + 1) * sizeof(float));
    if (!x || !y || !freq) {
        free(x);
        free(y);
        free(freq);
        return -1;
    }
    orc_convert_to_f32(in, x, rows * width, dtype);
    orc_rope_frequencies(theta, rotary_dim, freq);
    const size_t half = rotary_dim / 2;
    for (size_t row = 0; row < rows; ++row) {
        for (size_t head = 0; head < heads; ++head) {
            const size_t base = row * width + head * head_dim;
            for (size_t pair = 0; pair < head_dim / 2; ++pair) {
                if (pair >= half) { /* the unrotated tail, two elements per pair */
                    const size_t tail = base + rotary_dim + 2 * (pair - half);
                    y[tail] = x[tail];
                    y[tail + 1] = x[tail + 1];
                    continue;
                }
                const float angle = (float)positions[row] * freq[pair];
                const float cosine = cosf(angle);
                const float sine = sinf(angle);
                const float first = x[base + pair];
                const float second = x[base + pair + half];
                y[base + pair] = first * cosine - second * sine;
                y[base + pair + half] = second * cosine + first * sine;
            }
        }
    }
    orc_convert_from_f32(y, out, rows * width, dtype);
    free(x);
    free(y);
    free(freq);
    return 0;
}

/* ---- Attention-output gate -------------------------------------------------- */

/* silu_mul_f32 with sigmoid_only (src/metal/kernels/tensor_ops.metal:108-124):
 * out = (1 / (1 + exp(-gate))) * in, in float, elementwise. */
void orc_sigmoid_mul(const void* gate, const void* in, void* out, size_t n, int dtype)
{
    float* g = malloc((n ? n : 1) * sizeof(float));
    float* x = malloc((n ? n : 1) * sizeof(float));
    if (!g || !x) {
        free(g);
        free(x);
        return;
    }
    orc_convert_to_f32(gate, g, n, dtype);
    orc_convert_to_f32(in, x, n, dtype);
    for (size_t i = 0; i < n; ++i)
        x[i] = (1.0f / (1.0f + expf(-g[i]))) * x[i];
    orc_convert_from_f32(x, out, n, dtype);
    free(g);
    free(x);
}

/* ---- Threaded CPU baseline -------------------------------------------------- */

typedef struct {
    const orc_attention_args* a;
    float* out;
    size_t next; /* shared work counter, guarded by lock */
    pthread_mutex_t lock;
    int status;
} pool_state;

/* (row, kv_head) task: the q heads of the group walk the tokens together, each
 * with its own online-softmax state; arithmetic per q head equals
 * online_range. */
static void group_task(const orc_attention_args* a, size_t row, size_t kv_head, float* out)
{
    const size_t D = a->g->head_dim;
    const size_t group = a->q_heads / a->g->kv_heads;
    float running_max[64], running_sum[64];
    float* q = malloc(group * D * sizeof(float));
    float* acc = out; /* rows of the group are contiguous in out */
    float* kv = malloc(2 * D * sizeof(float));
    for (size_t h = 0; h < group; ++h) {
        running_max[h] = -INFINITY;
        running_sum[h] = 0.0f;
        const size_t q_base = (row * a->q_heads + kv_head * group + h) * D;
        for (size_t f = 0; f < D; ++f) {
            q[h * D + f] = load_value(a->queries, q_base + f, a->q_dtype);
            acc[h * D + f] = 0.0f;
        }
    }
    const size_t count = (size_t)a->positions[row] + 1;
    for (size_t token = 0; token < count; ++token) {
        const size_t base = cache_base(a, row, token, kv_head);
        for (size_t f = 0; f < D; ++f) {
            kv[f] = load_value(a->key_cache, base + f, a->cache_dtype);
            kv[D + f] = load_value(a->value_cache, base + f, a->cache_dtype);
        }
        for (size_t h = 0; h < group; ++h) {
            float score = 0.0f;
            for (size_t f = 0; f < D; ++f)
                score += q[h * D + f] * kv[f];
            score *= a->scale;
            const float new_max = running_max[h] > score ? running_max[h] : score;
            const float rescale = expf(running_max[h] - new_max);
            const float weight = expf(score - new_max);
            running_max[h] = new_max;
            running_sum[h] = running_sum[h] * rescale + weight;
            for (size_t f = 0; f < D; ++f)
                acc[h * D + f] = acc[h * D + f] * rescale + kv[D + f] * weight;
        }
    }
    for (size_t h = 0; h < group; ++h)
        for (size_t f = 0; f < D; ++f)
            acc[h * D + f] /= running_sum[h];
    free(q);
    free(kv);
}

static void* pool_worker(void* arg)
{
    pool_state* s = arg;
    const orc_attention_args* a = s->a;
    const size_t tasks = a->rows * a->g->kv_heads;
    const size_t group = a->q_heads / a->g->kv_heads;
    for (;;) {
        pthread_mutex_lock(&s->lock);
        const size_t task = s->next++;
        pthread_mutex_unlock(&s->lock);
        if (task >= tasks)
            break;
        const size_t row = task / a->g->kv_heads;
        const size_t kv_head = task % a->g->kv_heads;
        if (!row_valid(a, row)) {
            s->status = -1;
            continue;
        }
        group_task(a, row, kv_head,
                   s->out + (row * a->q_heads + kv_head * group) * a->g->head_dim);
    }
    return NULL;
}

int orc_attention_online_threads(const orc_attention_args* a, float* out, int threads)
{
    if (a->q_heads / a->g->kv_heads > 64)
        return -1;
    pool_state s = { a, out, 0, PTHREAD_MUTEX_INITIALIZER, 0 };
    if (threads < 1)
        threads = 1;
    pthread_t* ids = malloc((size_t)threads * sizeof(pthread_t));
    for (int i = 0; i < threads; ++i)
        pthread_create(&ids[i], NULL, pool_worker, &s);
    for (int i = 0; i < threads; ++i)
        pthread_join(ids[i], NULL);
    free(ids);
    return s.status;
}

/*
 * CPU oracle for the paged KV-cache + attention path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libckv, the C++ host layer,
 * the chibillm_amd package) links, loads or calls this library. Only tests/,
 * __graft_entry__.smoke() and bench.py's CPU-baseline leg use it, and only as
 * the checker / the timed CPU baseline.
 *
 * Each function restates the reference algorithm it names (paths relative to
 * the chibillm source tree). The reference itself cannot be built here: its
 * host code needs <expected> (absent from libstdc++ 11) and its kernels are
 * Metal. Where only a Metal kernel exists, the kernel's arithmetic is written
 * out as scalar C with fp32 accumulation, in the kernel's own order.
 *
 * Pinning (tests/test_oracle.py): every function below is checked against
 * the reference's own known-answer tests, a closed form, a brute-force
 * double-precision computation, or an exhaustive enumeration.
 */
#ifndef CHIBILLM_ORACLE_H
#define CHIBILLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of cache, query and output arrays. Same numbering as ckv.h. */
enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_F16 = 2 };

/* ---- 16-bit float conversions ------------------------------------------ */
uint16_t orc_bf16_from_f32(float value);   /* src/tensor/types.h:60-75 (RNE, NaN quieting) */
float orc_bf16_to_f32(uint16_t bits);      /* src/tensor/types.h:83-88 */
uint16_t orc_f16_from_f32(float value);    /* IEEE 754 binary16, round to nearest even */
float orc_f16_to_f32(uint16_t bits);       /* IEEE 754 binary16, exact */
void orc_convert_from_f32(const float* in, void* out, size_t n, int dtype);
void orc_convert_to_f32(const void* in, float* out, size_t n, int dtype);
size_t orc_dtype_size(int dtype);

/* ---- Seeded inputs ------------------------------------------------------ */
/* std::mt19937_64 (the engine is fully specified by the C++ standard). */
typedef struct {
    uint64_t state[312];
    size_t index;
} orc_mt64;
void orc_mt64_seed(orc_mt64* rng, uint64_t seed);
uint64_t orc_mt64_next(orc_mt64* rng);
/* (x >> 11) * 2^-53: a double in [0, 1). */
double orc_uniform(orc_mt64* rng);
/* N(0,1) by Box-Muller in double, both outputs of each pair used in order,
 * then rounded to f32 and, for 16-bit types, to that type (RNE). */
void orc_fill_normal(orc_mt64* rng, void* out, size_t n, int dtype);
/* Fisher-Yates: out = a permutation of 0..n-1 (i from n-1 down to 1,
 * j = next() % (i + 1)). */
void orc_permutation(orc_mt64* rng, uint32_t* out, size_t n);
/* Uniform integer in [lo, hi] as lo + next() % (hi - lo + 1). */
uint64_t orc_uniform_int(orc_mt64* rng, uint64_t lo, uint64_t hi);

/* ---- Page allocator (src/block_manager.cc:5-64) ------------------------- */
/* FIFO free list 0..N-1; reserve pops from the front, release pushes to the
 * back. Sequence ids are dense small integers < max_sequences here. */
typedef struct orc_block_manager orc_block_manager;
/* status codes follow block_manager_errc / state_errc numbering:
 *   make: 0 ok, 1 invalid_block_count, 2 invalid_block_size, 3 too_many_blocks
 *   reserve: 0 ok, 1 capacity_exhausted, 2 invalid_reservation */
int orc_bm_make(size_t block_count, size_t block_size, size_t max_sequences,
                orc_block_manager** out);
void orc_bm_destroy(orc_block_manager* bm);
int orc_bm_reserve(orc_block_manager* bm, size_t seq, size_t tokens);
void orc_bm_release(orc_block_manager* bm, size_t seq);
size_t orc_bm_free_count(const orc_block_manager* bm);
/* Copies at most cap entries of seq's table; returns the table length. */
size_t orc_bm_table(const orc_block_manager* bm, size_t seq, uint32_t* out, size_t cap);

/* ---- Slot mapping (src/model_batch.cc:178-185) -------------------------- */
/* slot = table[pos / bs] * bs + pos % bs; returns 0 or -1 when pos is beyond
 * the table or the slot does not fit in u32. */
int orc_slot(const uint32_t* table, size_t table_length, uint32_t position, uint32_t block_size,
             uint32_t* slot);

/* ---- prepare_paged_batch (src/model_batch.cc:127-204) ------------------ */
/* Items are runs of token rows: item i has token_count[i] rows starting at
 * row sum(token_count[0..i)), and its block table is
 * tables[table_start[i] .. table_start[i] + table_len[i]). For every row:
 * slot = table[pos / bs] * bs + pos % bs, table offset = the item's start in
 * the flat table, table length = the item's table length; the flat table is
 * the items' tables concatenated. Returns 0, or 1 (inconsistent_batch) for the
 * reference's checks: no items or rows, block_size or block_count 0, an item
 * with no tokens or an empty table, a table entry >= block_count, a position
 * >= max_positions or past its table, or a slot beyond u32. flat_table needs
 * sum(table_len) entries; slots, offsets and lengths one per row. */
int orc_prepare_paged_batch(size_t n_items, const uint32_t* token_count,
                            const uint32_t* tables, const size_t* table_start,
                            const uint32_t* table_len, const uint32_t* positions,
                            size_t max_positions, size_t block_count, size_t block_size,
                            uint32_t* flat_table, uint32_t* slots, uint32_t* offsets,
                            uint32_t* lengths);
/* One decode step's host work for n sequences (ids 0..n-1) that each append
 * one token: block_manager reserve(seq, lengths[seq] + 1), then
 * prepare_paged_batch over one row per sequence at position lengths[seq];
 * lengths[] is advanced by one. scratch_tables needs the sum of the table
 * lengths after the step. Returns 0, 1 (capacity exhausted or inconsistent). */
int orc_decode_step_host(orc_block_manager* bm, size_t n, uint32_t* lengths,
                         uint32_t* scratch_tables, size_t* scratch_start, uint32_t* scratch_len,
                         uint32_t* token_count, uint32_t* flat_table, uint32_t* slots,
                         uint32_t* offsets, uint32_t* row_lengths, size_t block_count,
                         size_t block_size);

/* ---- Cache addressing (src/metal/metal_kv_cache.cc:150-179) ------------- */
/* Layout [layer, block, token_in_block, kv_head, feature]. Returns 0, or the
 * kv_cache_errc value (7 layer, 8 block, 9 token, 10 head, 11 feature). */
typedef struct {
    size_t layers, blocks, block_size, kv_heads, head_dim;
} orc_geometry;
int orc_element_offset(const orc_geometry* g, size_t layer, size_t block, size_t token,
                       size_t head, size_t feature, size_t* offset);

/* ---- KV append (src/metal/kernels/attention.metal:3-33) ----------------- */
/* key_cache[(layer*slot_count + slot)*F + f] = keys[row*F + f]; rows whose slot
 * is >= slot_count are skipped. elem_size is the byte size of one element. */
void orc_store_kv(void* key_cache, void* value_cache, const void* keys, const void* values,
                  const uint32_t* slots, size_t rows, size_t feature_count, size_t layer,
                  size_t slot_count, size_t elem_size);
/* Reads tokens 0..n-1 of one sequence back through its table (the inverse of
 * store_kv on the same slots). */
void orc_gather(const void* key_cache, const void* value_cache, const uint32_t* table,
                size_t n_tokens, size_t layer, size_t slot_count, size_t block_size,
                size_t feature_count, size_t elem_size, void* out_keys, void* out_values);

/* ---- Decode attention ---------------------------------------------------- */
/* Common arguments: q is [rows, q_heads*D] of q_dtype; caches are the flat
 * [L, B, bs, Hkv, D] arrays of cache_dtype; output is f32 [rows, q_heads*D].
 * Row r attends to logical positions 0..positions[r] through
 * table[offsets[r] .. offsets[r]+lengths[r]). kv_head = q_head / (Hq / Hkv).
 * Returns 0, or -1 on metadata the reference kernel would skip. */
typedef struct {
    const orc_geometry* g;
    const void* key_cache;
    const void* value_cache;
    int cache_dtype;
    const void* queries;
    int q_dtype;
    const uint32_t* positions;
    const uint32_t* table;
    size_t table_entries;
    const uint32_t* offsets;
    const uint32_t* lengths;
    size_t rows;
    size_t q_heads;
    size_t layer;
    float scale;
} orc_attention_args;

/* paged_attention_f32 (src/metal/kernels/attention.metal:35-159): per token,
 * score = (q . k) * scale, one online-softmax update per token in fp32. */
int orc_attention_online(const orc_attention_args* a, float* out);
/* Two-pass softmax in double (tests/tensor_ops_test.cc:908-936). */
int orc_attention_reference(const orc_attention_args* a, double* out);
/* paged_attention_partial_f32 + paged_attention_reduce_f32
 * (src/metal/kernels/attention.metal:446-615): chunks of chunk_size tokens,
 * partial (m, l, acc) per chunk, merged with e^{m_c - M}. */
int orc_attention_split(const orc_attention_args* a, size_t chunk_size, float* out);
/* paged_flash_attention_prefill_f32 (src/metal/kernels/attention.metal:246-444)
 * over the query tiles of orc_query_tiles: 16-key tiles, per-row online softmax,
 * keys past the row's position masked to -inf. */
int orc_attention_prefill_tiles(const orc_attention_args* a, const uint32_t* tile_starts,
                                const uint32_t* tile_lengths, size_t tile_count, float* out);

/* Query tiles (src/tensor/attention.cc:142-167): runs of <= 8 rows with the
 * same table offset/length and consecutive positions. Returns the tile count;
 * *shared is set when some tile has more than one row. */
size_t orc_query_tiles(const uint32_t* positions, const uint32_t* offsets,
                       const uint32_t* lengths, size_t rows, uint32_t* starts,
                       uint32_t* tile_lengths, int* shared);

/* ---- Checkpoint pack / restore (src/metal/metal_kv_cache.cc:14-35) ------ */
/* Packed layout [layer, token, kv_head, feature]; only the first `tokens`
 * tokens are copied (the tail page is copied partially). restore != 0 copies
 * packed -> paged. */
void orc_copy_prefix(void* paged, void* packed, const uint32_t* blocks, const orc_geometry* g,
                     size_t tokens, size_t elem_size, int restore);

/* ---- Page copy (copy-on-write target of a shared page) ------------------ */
/* For every layer: page dst[i] := page src[i], keys and values. */
void orc_copy_blocks(void* key_cache, void* value_cache, const orc_geometry* g,
                     const uint32_t* src, const uint32_t* dst, size_t n, size_t elem_size);

/* ---- Rotary position embedding (src/metal/kernels/tensor_ops.metal:158-195) */
/* inv_freq[j] = theta^(-2j/rotary_dim) in float (src/metal/metal_kernels.mm:186-191). */
void orc_rope_frequencies(float theta, size_t rotary_dim, float* out);
/* Split-half rotation of [rows, heads*head_dim] rows of dtype at positions;
 * rotary_dim 0 means head_dim. Returns -1 on invalid arguments. */
int orc_rope(const void* in, void* out, int dtype, size_t rows, size_t heads, size_t head_dim,
             const uint32_t* positions, float theta, size_t rotary_dim);

/* ---- Attention-output gate (src/metal/kernels/tensor_ops.metal:108-124) -- */
/* out = (1 / (1 + exp(-gate))) * in, float math, rounded once; out may be in. */
void orc_sigmoid_mul(const void* gate, const void* in, void* out, size_t n, int dtype);

/* ---- Timing helper for the CPU baseline --------------------------------- */
/* Decode attention for every row, parallel over (row, kv_head) on `threads`
 * host threads, same arithmetic as orc_attention_online but the two q heads of
 * a GQA group share each K/V read. Returns 0 or -1. */
int orc_attention_online_threads(const orc_attention_args* a, float* out, int threads);

#ifdef __cplusplus
}
#endif
#endif

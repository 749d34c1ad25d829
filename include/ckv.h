/*
 * ckv.h - C ABI of the MI355X paged KV-cache + attention path (libckv.so).
 *
 * The library replaces chibillm's Metal KV-cache path: the KV tensors and
 * dispatches of metal_kv_cache / metal_kernels (src/metal/metal_kv_cache.h:75-122,
 * src/metal/metal_kernels.h:76-123) and the host checks of store_kv /
 * paged_attention (src/tensor/tensor_ops.cc:412-463, src/tensor/attention.cc:8-254).
 * The C++ host layer (block_manager, scheduler, prefix_cache, model_batch,
 * hip_model_state) calls these functions; so can a ctypes or other FFI binding.
 *
 * Conventions
 *  - Every function returns an int status: 0 on success, else one of the
 *    CKV_E_* codes below. ckv_error_name(code) gives the reference's
 *    "namespace.name" string for it.
 *  - Pointers named in device memory (keys, values, queries, output,
 *    checkpoint buffers) are HIP device pointers. Metadata arrays (tables,
 *    slots, positions, block ids) are host pointers, borrowed only for the
 *    duration of the call; the library validates them on the host and uploads
 *    them with one pinned host-to-device copy.
 *  - All work is enqueued on the context's stream, in call order. ckv_sync is
 *    the single wait (the role of end_compute_pass, src/metal/metal_context.h:99-110).
 *  - A context and its pools are not thread-safe; one thread drives them
 *    (src/serving_runtime.cc:364-392 has exactly one engine thread).
 *
 * KV layout in HBM (one allocation each for keys and values):
 *   [layer][block][token_in_block][kv_head][feature]
 * exactly the reference's element_offset order (src/metal/metal_kv_cache.cc:150-179),
 * stored as f32, bf16 or fp16 (the reference stores f32).
 */
#ifndef CHIBILLM_CKV_H
#define CHIBILLM_CKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CKV_ABI_VERSION 1

typedef struct ckv_context ckv_context;
typedef struct ckv_pool ckv_pool;

/* Element types. f32 and bf16 follow src/tensor/types.h:90-95; fp16 is new. */
enum ckv_dtype { CKV_F32 = 0, CKV_BF16 = 1, CKV_F16 = 2 };

/* Status codes. 1xx = tensor_op_errc + 100 (src/tensor/tensor_ops.h:18-48),
 * 2xx = kv_cache_errc + 200 (src/metal/metal_kv_cache.h:42-55),
 * 3xx = state_errc + 300 (src/model_state.h:10-15), 4xx = this library. */
enum ckv_status {
    CKV_OK = 0,
    CKV_E_TENSOR_ALLOCATION_FAILED = 101,
    CKV_E_INVALID_RANK = 107,
    CKV_E_UNSUPPORTED_DTYPE = 108,
    CKV_E_INPUT_SHAPE_MISMATCH = 109,
    CKV_E_OUTPUT_SHAPE_MISMATCH = 111,
    CKV_E_POSITION_COUNT_MISMATCH = 114,
    CKV_E_INVALID_HEAD_COUNT = 115,
    CKV_E_INVALID_HEAD_DIMENSION = 116,
    CKV_E_INVALID_ROPE_THETA = 117,
    CKV_E_CACHE_SLOT_COUNT_MISMATCH = 118,
    CKV_E_CACHE_FEATURE_COUNT_MISMATCH = 119,
    CKV_E_CACHE_LAYER_OUT_OF_RANGE = 120,
    CKV_E_CACHE_SLOT_OUT_OF_RANGE = 121,
    CKV_E_BLOCK_TABLE_METADATA_COUNT_MISMATCH = 122,
    CKV_E_BLOCK_TABLE_RANGE_OUT_OF_BOUNDS = 123,
    CKV_E_CACHE_BLOCK_OUT_OF_RANGE = 124,
    CKV_E_CACHE_HEAD_DIMENSION_MISMATCH = 125,
    CKV_E_INVALID_KV_HEAD_MAPPING = 126,
    CKV_E_BACKEND_FAILURE = 127,
    CKV_E_UNSUPPORTED_ALIASING = 128,
    CKV_E_INVALID_LAYER_COUNT = 200,
    CKV_E_INVALID_BLOCK_COUNT = 201,
    CKV_E_INVALID_BLOCK_SIZE = 202,
    CKV_E_INVALID_KV_HEAD_COUNT = 203,
    CKV_E_INVALID_HEAD_DIMENSION_KV = 204,
    CKV_E_LAYOUT_SIZE_OVERFLOW = 205,
    CKV_E_KV_ALLOCATION_FAILED = 206,
    CKV_E_LAYER_OUT_OF_RANGE = 207,
    CKV_E_BLOCK_OUT_OF_RANGE = 208,
    CKV_E_TOKEN_OFFSET_OUT_OF_RANGE = 209,
    CKV_E_KV_HEAD_OUT_OF_RANGE = 210,
    CKV_E_HEAD_FEATURE_OUT_OF_RANGE = 211,
    CKV_E_STATE_CAPACITY_EXHAUSTED = 300,
    CKV_E_STATE_INVALID_RESERVATION = 301,
    CKV_E_STATE_BACKEND_FAILURE = 302,
    CKV_E_STATE_ALLOCATION_FAILED = 303,
    CKV_E_INVALID_ARGUMENT = 400, /* null pointer or zero where a value is required */
    CKV_E_HIP_FAILURE = 401,      /* a HIP runtime call failed; see ckv_last_error */
    CKV_E_NO_DEVICE = 402,
    CKV_E_NO_TABLES = 403,        /* an op needs metadata that was never uploaded */
};

/* Name of a status code, e.g. "tensor_op.cache_slot_out_of_range".
 * Replaces error_name() of each reference enum (src/tensor/tensor_ops.h:50-86,
 * src/metal/metal_kv_cache.h:57-70, src/model_state.h:17-28). */
const char* ckv_error_name(int code);
/* Detail text of the last failure on this context (HIP error string, etc.);
 * the role of error<Code>::detail (src/error.h:13-31). Never NULL. */
const char* ckv_last_error(const ckv_context* ctx);
int ckv_abi_version(void);

/* ---- Context: device + stream (src/metal/metal_context.h:87-120) ---------- */
int ckv_context_create(int device, ckv_context** out);
int ckv_context_destroy(ckv_context* ctx);
/* Enqueue on hip_stream from now on, e.g. a framework's current stream so
 * that ckv work is ordered after the framework's writes of its inputs. NULL
 * is the device's null (default) stream. Work already enqueued on the
 * previous stream is drained first. */
int ckv_context_set_stream(ckv_context* ctx, void* hip_stream);
/* The stream currently used, and the stream the context created for itself
 * (used until ckv_context_set_stream is called). */
void* ckv_context_stream(const ckv_context* ctx);
void* ckv_context_own_stream(const ckv_context* ctx);
/* Waits for all work enqueued on the context's stream. */
int ckv_sync(ckv_context* ctx);

/* Device buffers for callers without their own HIP binding (the role of
 * metal_context::make_shared_buffer, src/metal/metal_context.h:87-120, but
 * device memory: the host reaches it only through the copies below).
 * The copies are synchronous with respect to the context stream. */
int ckv_device_alloc(ckv_context* ctx, size_t bytes, void** out);
int ckv_device_free(ckv_context* ctx, void* ptr);
/* Pinned (page-locked) host memory, for spilled checkpoints (ckv_checkpoint_export):
 * copies to and from it run asynchronously on the context stream. Free waits for
 * the stream first. */
int ckv_host_alloc(ckv_context* ctx, size_t bytes, void** out);
int ckv_host_free(ckv_context* ctx, void* ptr);
int ckv_copy_to_device(ckv_context* ctx, void* device_dst, const void* host_src, size_t bytes);
int ckv_copy_to_host(ckv_context* ctx, void* host_dst, const void* device_src, size_t bytes);

/* Per-kernel GPU timing, the role of CHIBILLM_PROFILE
 * (src/metal/metal_context.mm:94-169): when enabled, every launch is bracketed
 * by HIP events on the launch stream and its duration is added under the
 * kernel's name. Query synchronises the stream. Names: "store_kv",
 * "gather_kv", "paged_attention_decode", "paged_attention_merge", "append_decode",
 * "paged_attention_prefill", "copy_blocks", "checkpoint_pack",
 * "checkpoint_unpack", "tables_patch", "tables_fill", "batch_expand", "rope",
 * "rope_append", "rope_append_decode", "sigmoid_mul", "checkpoint_export",
 * "checkpoint_import". */
int ckv_profile_enable(ckv_context* ctx, int enabled);
int ckv_profile_query(ckv_context* ctx, const char* kernel, double* total_ms,
                      uint64_t* launches);
int ckv_profile_reset(ckv_context* ctx);

/* ---- KV pool (metal_kv_cache::make, src/metal/metal_kv_cache.cc:38-82) ----- */
/* Allocates keys and values, each layers*blocks*block_size*kv_heads*head_dim
 * elements of dtype. Geometry checks and their order follow the reference:
 * invalid_layer_count, invalid_block_count, invalid_block_size,
 * invalid_kv_head_count, invalid_head_dimension, layout_size_overflow,
 * allocation_failed. Slots (blocks*block_size) must fit in u32. */
int ckv_pool_create(ckv_context* ctx, size_t layers, size_t blocks, size_t block_size,
                    size_t kv_heads, size_t head_dim, int dtype, ckv_pool** out);
/* Same geometry checks, over caller-owned device memory (not freed by the pool). */
int ckv_pool_wrap(ckv_context* ctx, size_t layers, size_t blocks, size_t block_size,
                  size_t kv_heads, size_t head_dim, int dtype, void* keys, void* values,
                  ckv_pool** out);
int ckv_pool_destroy(ckv_pool* pool);
int ckv_pool_buffers(const ckv_pool* pool, void** keys, void** values, size_t* bytes_each);
/* metal_kv_cache::element_offset (src/metal/metal_kv_cache.cc:150-179): the
 * element index into either tensor, or layer/block/token/head/feature
 * _out_of_range. */
int ckv_element_offset(const ckv_pool* pool, size_t layer, size_t block, size_t token_offset,
                       size_t kv_head, size_t head_feature, size_t* offset);

/* ---- Device-resident metadata ------------------------------------------------ */
/* Uploads the batch metadata of prepare_paged_batch (src/model_batch.cc:127-204):
 * the flat block table, per-row table offset/length, positions and slots,
 * after the host checks of prepared_attention_batch::make
 * (src/tensor/attention.cc:110-137) and store_kv (src/tensor/tensor_ops.cc:445-453):
 *   block_table_range_out_of_bounds  a row's [offset, offset+length) leaves the
 *                                    table, or position/block_size >= length
 *   cache_block_out_of_range         a table entry >= blocks
 *   cache_slot_out_of_range          a slot >= blocks*block_size
 * slots may be NULL when no append follows. The query tiles of
 * prepared_attention_batch::make (src/tensor/attention.cc:142-167) are derived
 * here, once per batch, and reused by every layer; so is the decode kernel's
 * row order when every tile is a single row. The split-KV decode work list
 * (and the row order of other batches) are derived and uploaded by the
 * batch's first decode launch that needs them. A batch that fails the checks
 * leaves the previous batch current; one that fails after them (device
 * allocation or copy) leaves no batch: launches report no_tables until the
 * next upload succeeds. The same holds for ckv_batch_upload. */
int ckv_tables_upload(ckv_pool* pool, const uint32_t* block_table, size_t n_entries,
                      const uint32_t* offsets, const uint32_t* lengths,
                      const uint32_t* positions, const uint32_t* slots, size_t rows);
/* Device-side delta update of the uploaded block table: table[idx[i]] = val[i],
 * so a block_manager change is mirrored without re-sending the table. Rows'
 * offsets/lengths and the uploaded slots are unchanged; every idx must be
 * < n_entries (block_table_range_out_of_bounds) and every val < blocks
 * (cache_block_out_of_range). A patch that moves the page holding a row's own
 * position away from that row's uploaded slot leaves ckv_append_decode on its
 * unfused form (ckv_append to the uploaded slot, then the attention through
 * the patched table), as store_kv followed by paged_attention would. */
int ckv_tables_patch(ckv_pool* pool, const uint32_t* idx, const uint32_t* val, size_t n);

/* ---- Device-resident sequence tables (prepare_paged_batch on the device) ----
 * The alternative to ckv_tables_upload for a serving loop: every live
 * sequence's block table stays in a device arena of max_sequences rows of
 * pages_per_sequence entries (entry (s, i) at s*pages_per_sequence + i), and
 * only its changes cross PCIe. A batch is then given per item (sequence,
 * first position, token count) and its per-row offsets, lengths, positions
 * and slots are expanded on the device: the loop of prepare_paged_batch
 * (src/model_batch.cc:127-204) that concatenates each item's block table
 * and computes slot = table[position / block_size] * block_size +
 * position % block_size for every row. */

/* Allocates the arena (kept until the pool is destroyed; a second call
 * resizes it) and sets every entry to page 0 and every table length to 0.
 * A batch uploaded from the previous arena must be uploaded again (launches
 * report no_tables until then). */
int ckv_seq_tables_reserve(ckv_pool* pool, size_t max_sequences, size_t pages_per_sequence);
/* Mirrors block_manager changes (src/block_manager.cc:5-64: pages appended
 * to a reservation, a release; and a copy-on-write page replacement):
 * entry (seq[i], index[i]) = block[i] for i < n, then table length of
 * len_seq[j] = length[j] for j < m. Host work only: the written entries are
 * pending (a later write of one entry wins) and reach the device with the
 * next ckv_batch_upload, in its single copy. Checks, before anything changes:
 *   block_table_range_out_of_bounds  seq >= max_sequences, index or length
 *                                    > pages_per_sequence (index ==)
 *   cache_block_out_of_range         block >= blocks
 *   no_tables                        before ckv_seq_tables_reserve */
int ckv_seq_tables_update(ckv_pool* pool, const uint32_t* seq, const uint32_t* index,
                          const uint32_t* block, size_t n, const uint32_t* len_seq,
                          const uint32_t* length, size_t m);
/* Uploads a batch of n_items items; item i is token_count[i] rows of
 * sequence seq[i] at positions first_position[i] + j, rows numbered in item
 * order (model_batch::items, src/model_batch.h). Equivalent to
 * ckv_tables_upload with the sequences' tables as the flat table, offsets
 * seq*pages_per_sequence, lengths the sequences' table lengths, and (when
 * with_slots) the slots of prepare_paged_batch. Checks (the row checks of
 * src/model_batch.cc:151-185 and src/tensor/attention.cc:110-137):
 *   invalid_argument                 an item with no tokens
 *   block_table_range_out_of_bounds  seq >= max_sequences, or the item's
 *                                    last position / block_size >= the
 *                                    sequence's table length
 * Table entries are checked when they are written (ckv_seq_tables_update),
 * so slots cannot leave the pool. ckv_tables_patch is refused while such a
 * batch is current. */
int ckv_batch_upload(ckv_pool* pool, const uint32_t* seq, const uint32_t* first_position,
                     const uint32_t* token_count, size_t n_items, int with_slots);

/* The fast decode's plan of the current batch (deriving it if a decode launch
 * has not yet): pages per workgroup (0 when every (row, kv head) is one
 * workgroup), work items (rows or row pieces; a workgroup may take several)
 * and partial records. Rows are cut when one workgroup per (row, kv head)
 * would leave the batch bound by its longest rows: the batch's pages are then
 * dealt out evenly to as many workgroups as the GPU holds at once, and a
 * row's pieces are merged as
 * paged_attention_reduce_f32 merges (src/metal/kernels/attention.metal:567-615).
 * A diagnostic with no counterpart in the reference, for tests and tuning. */
int ckv_decode_plan(ckv_pool* pool, uint32_t* split_pages, uint32_t* work_items,
                    uint32_t* records);
/* The number of device and pinned host allocations and frees (hipMalloc,
 * hipFree, hipHostMalloc, hipHostFree) the library has made on this context:
 * pools, their metadata and scratch buffers, staging, ckv_device_alloc and
 * ckv_host_alloc. A diagnostic with no counterpart in the reference, for tests
 * of ckv_append_decode_noalloc, which must leave it unchanged. */
int ckv_debug_allocations(const ckv_context* ctx, uint64_t* count);

/* ---- Ops -------------------------------------------------------------------------- */
/* store_kv (src/tensor/tensor_ops.cc:412-463; kernel src/metal/kernels/attention.metal:3-33):
 * keys/values are device [rows, kv_heads*head_dim] of the pool dtype; row r is
 * copied bit-for-bit to slot slots[r] of `layer`. rows must equal the uploaded
 * row count (cache_slot_count_mismatch); layer < layers
 * (cache_layer_out_of_range); slots must have been uploaded (no_tables). */
int ckv_append(ckv_pool* pool, size_t layer, const void* keys, const void* values,
               size_t rows);
/* Reads tokens 0..n_tokens-1 of one sequence back through the uploaded table
 * entries [table_offset, table_offset+table_length) into device
 * [n_tokens, kv_heads*head_dim] arrays (the inverse of ckv_append). */
int ckv_gather(ckv_pool* pool, size_t layer, size_t table_offset, size_t table_length,
               size_t n_tokens, void* out_keys, void* out_values);
/* paged_attention (src/tensor/attention.cc:188-254) for rows that each attend
 * to logical positions 0..positions[r] through their table range:
 * out = softmax(q . k * scale) . v with fp32 accumulation. queries and
 * output are device [rows, q_heads*head_dim] of the pool dtype.
 * Decode form: the q heads of a GQA group share every K/V read. Pools with
 * head_dim 128, 16-token pages and 1, 2, 4 or 8 q heads per kv head (f32 pools
 * with 8 in two passes of 4) take one workgroup per (row, kv_head),
 * or per page chunk of rows the batch plan cuts (ckv_decode_plan), the chunks
 * merged by the last to finish; other geometries take split-KV over token
 * chunks and a merge launch. Both are the split-K of
 * paged_attention_partial_f32 / paged_attention_reduce_f32
 * (src/metal/kernels/attention.metal:446-615), generalised to every row.
 * Checks: invalid_head_count, invalid_kv_head_mapping (q_heads % kv_heads),
 * cache_layer_out_of_range, position_count_mismatch (rows != uploaded rows). */
int ckv_decode_attention(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads,
                         float scale, void* output, size_t rows);
/* store_kv followed by the decode form, in one launch where possible: the
 * `run_attention` pair of src/qwen/qwen_layer.cc:32-50 (store_kv, then
 * paged_attention). Each workgroup reads its row's new token from keys/values,
 * writes it into the row's slot and attends to it in the same pass, which
 * applies when every uploaded slot is the slot of its row's position and no
 * two rows share a table range (a decode batch); otherwise ckv_append then
 * ckv_decode_attention run. Results are those of the two calls in sequence.
 * Checks: those of ckv_append, then those of ckv_decode_attention. */
int ckv_append_decode(ckv_pool* pool, size_t layer, const void* keys, const void* values,
                      const void* queries, size_t q_heads, float scale, void* output, size_t rows);
/* Prefill form (paged_flash_attention_prefill_f32,
 * src/metal/kernels/attention.metal:246-444): query tiles of consecutive
 * positions of one sequence share every K/V tile; QK^T and PV run on the
 * matrix cores for head_dim 128, 16-token pages, 1, 2, 4 or 8 q heads per kv
 * head and scale > 0 (bf16/fp16 products for 16-bit pools, exact fp32
 * products for f32 pools); other geometries and scales take the decode form
 * row by row, with the same results. A launch too small to fill the GPU
 * splits each long tile's keys between workgroups and merges their partial states
 * in the pool's scratch (grown on first use, like the decode's split-K
 * records); the merge order is fixed, so results do not depend on timing.
 * Same arguments and checks as ckv_decode_attention. */
int ckv_prefill_attention(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads,
                          float scale, void* output, size_t rows);
/* Kernel selection of dispatch_paged_attention_f32 / paged_attention
 * (src/metal/metal_kernels_attention.mm:143-298, src/tensor/attention.cc:290-309):
 * the prefill form when some query tile has more than one row, else decode. */
int ckv_attention(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads,
                  float scale, void* output, size_t rows);

/* ckv_append_decode for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): no
 * counterpart in the reference. Same arguments, checks and results as
 * ckv_append_decode, bit for bit, but it calls no hipMalloc, hipFree or other
 * allocating routine: the partial records and arrival counters of rows the
 * batch plan cuts into chunks go to a fixed 16 MiB device array of the
 * library (one per GPU, held until the process ends) instead of pool buffers,
 * and its launches are not timed by ckv_profile_*. The array's first 256 KiB
 * are the counters (zero when the library loads; every call leaves them zero),
 * the rest the records. It needs what the allocating calls already set up:
 * a batch of single-row query tiles uploaded with ckv_tables_upload or
 * ckv_batch_upload (its plan goes up with it), and the fast decode's geometry
 * (head_dim 128, 16-token pages, 1, 2, 4 or 8 q heads per kv head, 16-byte
 * aligned pools, queries and output); a batch with a multi-row query
 * tile is refused whatever ran on it before. Otherwise, and when the batch's
 * records exceed the array (n_records * q_heads * 528 bytes > 16 MiB - 256 KiB
 * or n_records * kv_heads * 4 bytes > 256 KiB, see ckv_decode_plan), it
 * returns invalid_argument with a reason in ckv_last_error. Every call on one
 * GPU shares that GPU's array: calls that may overlap on one GPU (other
 * threads, other streams) race, on the outputs and on the counters, which can
 * then stay wrong for later calls; a caller serialises them, as one stream
 * does. */
int ckv_append_decode_noalloc(ckv_pool* pool, size_t layer, const void* keys, const void* values,
                              const void* queries, size_t q_heads, float scale, void* output,
                              size_t rows);

/* ---- The attention output's consumer: the Qwen3.5 sigmoid gate ---------------
 * src/qwen/qwen_layer.cc:183-206 splits the projected query into query and
 * gate (split_heads), attends, then sigmoid_mul(gate, attended, attended) and
 * feeds the result to linear_add. The gated forms apply the gate in the
 * attention epilogue, to the float result before its one rounding:
 * output = attention * 1 / (1 + e^-gate) (silu_mul_f32 with sigmoid_only,
 * src/metal/kernels/tensor_ops.metal:108-124). gate is a device array shaped
 * like output ([rows, q_heads * head_dim], pool dtype); it must not be the
 * queries' or the output's memory (unsupported_aliasing), and is required when
 * rows > 0 (invalid_argument). Otherwise as ckv_attention / ckv_append_decode. */
int ckv_attention_gated(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads,
                        float scale, const void* gate, void* output, size_t rows);
int ckv_append_decode_gated(ckv_pool* pool, size_t layer, const void* keys, const void* values,
                            const void* queries, size_t q_heads, float scale, const void* gate,
                            void* output, size_t rows);
/* sigmoid_mul (src/tensor/tensor_ops.h:131-135, src/tensor/tensor_ops.cc:289-296):
 * output[i] = input[i] * sigmoid(gate[i]) over count device elements of dtype,
 * computed in float; output may be input. The unfused form of the gate.
 * Checks: unsupported_dtype, invalid_argument (null arrays with count > 0). */
int ckv_sigmoid_mul(ckv_context* ctx, int dtype, const void* gate, const void* input,
                    void* output, size_t count);

/* ---- Rotary position embedding ------------------------------------------------------ */
/* rope (src/tensor/tensor_ops.cc:356-410; kernel rope_f32,
 * src/metal/kernels/tensor_ops.metal:158-195) on device rows
 * [rows, heads*head_dim] of the pool dtype and head_dim, each at its uploaded
 * position: within every head, pair j < rotary_dim/2 rotates elements j and
 * j + rotary_dim/2 by position * theta^(-2j/rotary_dim); the rest is copied.
 * rotary_dim 0 means head_dim. input may equal output (in place). Checks, in
 * the reference's order: position_count_mismatch (rows != uploaded rows),
 * invalid_head_count, invalid_head_dimension (odd head_dim or rotary_dim,
 * rotary_dim > head_dim, or rotary_dim > 1024), invalid_rope_theta (not
 * positive and finite). */
int ckv_rope(ckv_pool* pool, const void* input, void* output, size_t heads, float theta,
             size_t rotary_dim, size_t rows);
/* rope of the key rows fused with ckv_append: the apply_rope + store_kv pair
 * of src/qwen/qwen_layer.cc:20-30, :43 in one pass. keys/values are device
 * [rows, kv_heads*head_dim] rows of the pool dtype; keys are read unrotated
 * and are not modified; the rotated keys and the values land in the
 * uploaded slots of `layer`. Checks: those of ckv_append, then those of
 * ckv_rope. */
int ckv_rope_append(ckv_pool* pool, size_t layer, const void* keys, const void* values,
                    float theta, size_t rotary_dim, size_t rows);
/* The decode step of an attention layer from unrotated rows: rope of the
 * queries and of the new keys, store_kv, paged_attention (and, with a gate,
 * sigmoid_mul) — src/qwen/qwen_layer.cc:20-30, :43-49 (Qwen3) and :183-206
 * (Qwen3.5 full attention) — in one launch where ckv_append_decode's fused
 * kernel applies, the pool is bf16 or fp16 and rotary_dim (0 = head_dim) is
 * 16, 32, 64 or 128; otherwise
 * as ckv_rope into a pool-owned buffer, ckv_rope_append and the attention.
 * keys/values: [rows, kv_heads*head_dim]; queries: [rows, q_heads*head_dim];
 * queries and keys are read unrotated and not modified; gate may be NULL (no
 * gate), else as ckv_append_decode_gated's. The rotated keys and the values
 * land in the uploaded slots of `layer`: values bit-exact, rotated 16-bit
 * elements within one unit in the last place of ckv_rope_append's (both
 * within one of rope_f32 in float, rounded). Checks: those of
 * ckv_append_decode, unsupported_aliasing for the gate, then those of ckv_rope
 * (with q_heads). */
int ckv_rope_append_decode(ckv_pool* pool, size_t layer, const void* keys, const void* values,
                           const void* queries, size_t q_heads, float scale, float theta,
                           size_t rotary_dim, const void* gate, void* output, size_t rows);

/* ---- Pages: copy-on-write and checkpoints ------------------------------------------ */
/* For every layer, keys and values: page dst[i] := page src[i]. The copy-on-write
 * step for a shared page (new; the reference never shares pages). Checks:
 * cache_block_out_of_range; unsupported_aliasing when a dst repeats or is
 * also a src. */
int ckv_copy_blocks(ckv_pool* pool, const uint32_t* src, const uint32_t* dst, size_t n);
/* metal_kv_cache::checkpoint / restore (src/metal/metal_kv_cache.cc:14-35, :225-253):
 * packed device buffers [layer][token][kv_head][feature] of the pool dtype;
 * only the first `tokens` tokens are copied (the tail page partially).
 * blocks must hold at least ceil(tokens/block_size) ids < blocks
 * (state.invalid_reservation otherwise, as valid_prefix, :205-223). */
int ckv_checkpoint_pack(ckv_pool* pool, const uint32_t* blocks, size_t n_blocks, size_t tokens,
                        void* packed_keys, void* packed_values);
int ckv_checkpoint_unpack(ckv_pool* pool, const uint32_t* blocks, size_t n_blocks,
                          size_t tokens, const void* packed_keys, const void* packed_values);
/* The same packed prefix in host memory: a prefix checkpoint that outlives its
 * pages (the reference's kv_cache_checkpoint holds it in host byte vectors,
 * src/metal/metal_kv_cache.h:24-40, and the byte-bounded prefix cache,
 * src/prefix_cache.cc:42-73, keeps it after the pages are reused). Host
 * buffers hold layers*tokens*kv_heads*head_dim elements each, in the layout of
 * ckv_checkpoint_pack. The copies run on the context stream through a device
 * staging buffer of at most 64 MiB per tensor, whole layers at a time; they are
 * asynchronous when the host buffers are pinned (ckv_host_alloc): do not read an
 * exported buffer, or change or free an imported one, before ckv_sync. Checks as
 * ckv_checkpoint_pack. Profile names "checkpoint_export", "checkpoint_import". */
int ckv_checkpoint_export(ckv_pool* pool, const uint32_t* blocks, size_t n_blocks, size_t tokens,
                          void* host_keys, void* host_values);
int ckv_checkpoint_import(ckv_pool* pool, const uint32_t* blocks, size_t n_blocks,
                          size_t tokens, const void* host_keys, const void* host_values);

#ifdef __cplusplus
}
#endif
#endif

// Internal declarations of libckv: context/pool state and kernel launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "ckv.h"

namespace ckv {

// Geometry of one KV tensor as the kernels see it. Element index of
// (layer, slot, kv_head, feature) is (layer*slot_count + slot)*F + kv_head*D + feature.
struct pool_view {
    void* keys;
    void* values;
    uint64_t layer_elems; // blocks * block_size * F
    uint32_t blocks;
    uint32_t block_size;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t features; // kv_heads * head_dim
    uint32_t elem_size;
    int dtype; // ckv_dtype
};

// Device pointers into the uploaded metadata block (one H2D copy per upload).
struct meta_view {
    const uint32_t* table;
    const uint32_t* offsets;
    const uint32_t* lengths;
    const uint32_t* positions;
    const uint32_t* slots;
    const uint32_t* items; // decode work list: (row, chunk) pairs
    const uint32_t* row_first; // first work item of each row
    const uint32_t* row_count; // work items (chunks) of each row
    // prefill query tiles, tile_entry_words each: (first row, row count, the
    // first row's position, the rows' table offset)
    const uint32_t* tiles;
    // fast decode plan, plan_entry_words per entry: a segment (pages
    // [first, end) of a row) per entry, (row, the segment's chunk index in
    // the row, the row's position, the flat table index of page `first`,
    // first, end, the row's chunk count, the workgroup's next entry or
    // plan_last). Workgroup w (per kv head) starts at entry w. A workgroup
    // needs nothing else from the batch to issue its first page loads.
    const uint32_t* plan;
    const uint32_t* split_first; // first partial record of each row cut into chunks
    const uint32_t* cut;         // the rows cut into chunks
    uint32_t n_entries;
    uint32_t rows;
    uint32_t n_items;
    uint32_t chunk; // tokens per decode work item, a multiple of 16
    uint32_t n_tiles;
    uint32_t tile_blocks; // 32-key blocks the batch's shortest query tile attends (host side)
    uint32_t mean_pages; // pages attended per row, mean over the batch (host side)
    uint32_t n_plan;      // workgroups per kv head of the fast decode (the entries they start at)
    uint32_t n_segments;  // entries of plan
    uint32_t split_pages; // the plan's pages per chunk or per workgroup; 0: one row per workgroup
    uint32_t n_records;   // partial records of the rows cut into chunks
    uint32_t n_cut;       // rows cut into chunks
};

// Device scratch of the fast decode's cut rows: a partial record
// [max, denominator, 0, 0, acc[head_dim]] per (record, q head), written by the
// chunks, and an arrival counter per (record, kv head), of which a cut row
// uses the one at (its first record, kv head). The counters must be zero
// before a launch and every launch leaves them zero (the row's last chunk
// resets its counter), so they are cleared once, when allocated.
struct split_scratch {
    float* records;
    uint32_t* arrivals;
};

constexpr size_t tile_entry_words = 4;

// Device scratch of a prefill launch whose tiles' key blocks are split
// between workgroups: a record [max, denominator, 0, 0, acc[128]] per (share,
// query vector), and an arrival counter per (tile, workgroup row range, kv
// head), zero before a launch and left zero by it. n_split = 1: no split;
// a tile's keys are cut into at most n_split ranges of at least min_blocks
// 32-key blocks.
struct prefill_split {
    float* records;
    uint32_t* arrivals;
    uint32_t n_split;
    uint32_t min_blocks;
};
constexpr uint32_t prefill_record_floats = 128 + 4;
constexpr uint32_t split_min_blocks = 8; // default of prefill_split::min_blocks
constexpr uint32_t split_max = 8;        // shares a tile's keys are split into at most

// A tile (or a workgroup's rows of it) whose keys span n_blocks 32-key
// blocks is cut into at most n_split ranges of at least min_blocks each;
// prefill_range_count gives how many. A tile shorter than three ranges' worth
// is not cut (1): the handoff's round trips would cost more than the blocks
// it takes off the longest range. n_split and min_blocks are at least 1
// (prefill_plan).
__host__ __device__ inline uint32_t prefill_range_count(uint32_t n_blocks, uint32_t n_split,
                                                        uint32_t min_blocks)
{
    const uint32_t by_length = n_blocks / min_blocks;
    return n_blocks >= 3 * min_blocks ? (by_length < n_split ? by_length : n_split) : 1;
}

// The key blocks [begin, end) of range `part` of n ranges. Range 0 starts at
// block 0, so every query of the tile attends some key of it. 32-bit:
// n_blocks < 2^27 (positions are 32-bit) and part < split_max.
__host__ __device__ inline void prefill_range_bounds(uint32_t n_blocks, uint32_t n, uint32_t part,
                                                     uint32_t& begin, uint32_t& end)
{
    begin = part * n_blocks / n;
    end = (part + 1) * n_blocks / n;
}

// Largest query tile, in rows (positions): the prefill kernel covers a tile
// with G workgroups of 256/G rows for GQA group size G.
constexpr uint32_t prefill_tile_rows = 256;

// Inverse RoPE frequencies of one (theta, rotary width), by value as a kernel
// argument; head_dim is at most 1024, so rotary/2 <= 512.
constexpr uint32_t max_rope_pairs = 512;
struct rope_table {
    float inv_freq[max_rope_pairs];
};
// The first 64 of them, all that a 128-wide head uses: the fused decode's
// kernel argument.
struct rope_table64 {
    float inv_freq[64];
};

// One rotary pair (a, b) -> (a cos - b sin, b cos + a sin), written once with
// explicit fused multiply-adds for every kernel that rotates (ckv_rope,
// ckv_rope_append, the fused decode).
__device__ __forceinline__ void rope_pair(float a, float b, float c, float s, float& ra, float& rb)
{
    ra = __builtin_fmaf(a, c, -(b * s));
    rb = __builtin_fmaf(b, c, a * s);
}

struct pending_timing {
    const char* name;
    hipEvent_t start;
    hipEvent_t stop;
};

struct profile_total {
    double ms = 0.0;
    uint64_t launches = 0;
};

// ---- elementwise (kernels_rope.hip) ------------------------------------------------
// out[i] = in[i] * sigmoid(gate[i]) over n elements of dtype (src/tensor/tensor_ops.cc:289-296)
hipError_t launch_sigmoid_mul(hipStream_t s, int dtype, const void* gate, const void* in,
                              void* out, uint64_t n);

// ---- launchers (kernels_rope.hip) --------------------------------------------------
// theta^(-2j/rotary) in float for j < rotary/2 (src/metal/metal_kernels.mm:186-191)
void rope_frequencies(float theta, uint32_t rotary, rope_table& out);
// rows of `heads` heads of the pool's head_dim and dtype, at the uploaded positions
hipError_t launch_rope(hipStream_t s, const pool_view& p, const meta_view& m, const void* in,
                       void* out, uint32_t rows, uint32_t heads, uint32_t rotary,
                       const rope_table& freq);
// rotated key rows and the value rows into the uploaded slots of `layer`
hipError_t launch_rope_append(hipStream_t s, const pool_view& p, const meta_view& m,
                              uint32_t layer, const void* keys, const void* values, uint32_t rows,
                              uint32_t rotary, const rope_table& freq);

} // namespace ckv

struct ckv_context {
    int device = 0;
    int cu_count = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string last_error;

    // pinned staging for metadata uploads: a ring of slots, each reused once
    // the copy last made from it has completed, so the host can prepare the
    // next uploads while earlier ones wait in the stream behind kernels
    static constexpr int staging_slots = 4;
    struct staging_slot {
        void* pinned = nullptr;
        size_t bytes = 0;
        hipEvent_t done = nullptr;
        bool pending = false;
    };
    staging_slot staging[staging_slots];
    int staging_next = 0; // the slot stage() hands out

    // this device's copy of the no-allocation entry point's scratch array
    // (its device address, from hipGetSymbolAddress at context creation; null
    // if that failed)
    void* noalloc_scratch = nullptr;

    // device and pinned host allocations and frees made by the library on
    // this context (ckv_debug_allocations)
    uint64_t allocations = 0;

    bool profile = false;
    std::vector<ckv::pending_timing> pending;
    std::vector<hipEvent_t> spare_events;
    std::map<std::string, ckv::profile_total> totals;
};

struct ckv_pool {
    ckv_context* ctx = nullptr;
    size_t layers = 0, blocks = 0, block_size = 0, kv_heads = 0, head_dim = 0;
    int dtype = CKV_BF16;
    size_t elem_size = 2;
    void* keys = nullptr;
    void* values = nullptr;
    size_t bytes_each = 0;
    bool owned = false;

    // host state of the current batch
    bool uploaded = false;
    bool has_slots = false;
    size_t n_entries = 0; // entries of the table the rows index
    size_t slot_rows = 0; // rows with an uploaded slot (0 without slots)
    std::vector<uint32_t> positions;
    std::vector<uint32_t> row_offsets; // each row's table offset (the decode plan's entries)
    bool shared_tile = false;
    bool fusable = false; // slots are the rows' own positions, one row per table range
    // while fusable: each row's own table index (offset + position / block_size)
    // and its uploaded slot, so a table patch can tell whether the fused
    // append still writes where ckv_append would
    std::vector<uint32_t> own_index, own_slot;
    // derived when a decode launch first needs them: the fast decode's plan
    // (uploaded with the batch when the batch goes to the decode kernel
    // anyway) and the generic path's split-KV work list
    bool plan_ready = false;
    bool work_ready = false;
    bool work_multi = false; // some row has more than one chunk: partials are merged
    std::vector<uint32_t> scratch; // host staging of the derived arrays
    std::vector<uint64_t> sort_keys;
    std::vector<uint32_t> stamp; // distinctness checks (all_distinct)
    uint32_t stamp_generation = 0;
    // pages the fused append writes, by page id: the generation that marked
    // them and the table index each is written through (own_pages_clash)
    std::vector<uint32_t> own_stamp, own_at;
    uint32_t own_generation = 0;

    // device copies
    uint32_t* d_meta = nullptr;
    size_t d_meta_words = 0;
    uint32_t* d_plan = nullptr; // the plan of a batch uploaded without it
    size_t d_plan_words = 0;
    uint32_t* d_work = nullptr;
    size_t d_work_words = 0;
    ckv::meta_view meta {};

    // device-resident sequence tables (ckv_seq_tables_*): seq_max rows of
    // seq_cap page ids. The host keeps a mirror of the entries and the rows'
    // lengths; entries written since the last batch upload are pending
    // (listed once each in `dirty`) and go up with the next batch.
    bool device_tables = false; // the current batch indexes the sequence tables
    uint32_t* d_seq = nullptr;
    size_t d_seq_words = 0;
    size_t seq_max = 0, seq_cap = 0;
    std::vector<uint32_t> seq_len, seq_host, dirty;
    std::vector<uint8_t> seq_dirty;

    // device scratch
    float* d_partials = nullptr;
    size_t d_partials_bytes = 0;
    uint32_t* d_arrivals = nullptr; // the fast decode's arrival counters (zero between launches)
    size_t d_arrivals_words = 0;
    float* d_pre_records = nullptr; // the split prefill's records
    size_t d_pre_records_floats = 0;
    uint32_t* d_pre_arrivals = nullptr; // its arrival counters (zero between launches)
    size_t d_pre_arrivals_words = 0;
    uint32_t* d_pairs = nullptr; // block-id pairs / patch pairs
    size_t d_pairs_words = 0;
    char* d_spill = nullptr; // staging of checkpoint export/import
    size_t d_spill_bytes = 0;
    char* d_rope_q = nullptr; // rotated queries of the unfused ckv_rope_append_decode
    size_t d_rope_q_bytes = 0;
};

namespace ckv {

// ---- launchers (kernels_copy.hip) ------------------------------------------
hipError_t launch_store_kv(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                           const void* keys, const void* values, uint32_t rows);
hipError_t launch_gather(hipStream_t s, const pool_view& p, const uint32_t* table,
                         uint32_t layer, uint32_t n_tokens, void* out_keys, void* out_values);
hipError_t launch_copy_blocks(hipStream_t s, const pool_view& p, uint32_t layers,
                              const uint32_t* pairs, uint32_t n);
hipError_t launch_checkpoint(hipStream_t s, const pool_view& p, uint32_t layers,
                             const uint32_t* blocks, uint32_t tokens, void* packed_keys,
                             void* packed_values, bool unpack);
hipError_t launch_table_patch(hipStream_t s, uint32_t* table, const uint32_t* pairs, uint32_t n);
// dst[0..n) = value (a kernel, not hipMemsetAsync: callers may capture it)
hipError_t launch_fill(hipStream_t s, uint32_t* dst, uint32_t value, uint32_t n);
// Expands a batch given as items into per-row metadata. `items` holds five
// sections of n_items words: sequence, first position, token count, first
// row, table length. Rows get offset seq*cap, the item's length, position
// first + j and (with_slots) slot seq_table[seq*cap + pos/bs]*bs + pos%bs.
hipError_t launch_expand_batch(hipStream_t s, const uint32_t* items, uint32_t n_items,
                               uint32_t rows, const uint32_t* seq_table, uint32_t cap,
                               uint32_t block_size, bool with_slots, uint32_t* offsets,
                               uint32_t* lengths, uint32_t* positions, uint32_t* slots);

// ---- decode plan (kernels_decode.hip) -------------------------------------------
// The fast decode's plan of a batch, from its rows' positions: which pages
// each workgroup covers, as segments of rows, and each cut row's first
// partial record. A row per workgroup (longest first) while that keeps every
// compute unit busy; otherwise, when one workgroup per (row, kv head) would
// leave the batch bound by its longest rows (a row holds more than half of
// one compute unit's share of the batch's pages), the batch's pages in row
// order are dealt out evenly to as many workgroups as the GPU holds at once,
// each taking a run of whole rows and row pieces (balanced). The fixed form
// cuts each row into chunks of split_pages pages, a workgroup per chunk.
// CKV_DECODE_SPLIT=<pages> forces the fixed form (0: no cut),
// CKV_DECODE_BALANCE=<pages> the balanced form with that many pages per
// workgroup.
struct decode_plan_shape {
    uint32_t split_pages; // pages per chunk (fixed) or per workgroup (balanced); 0: no cut
    uint32_t n_items;     // plan entries (segments)
    uint32_t n_records;
    uint32_t n_cut;
    uint32_t n_wgs;       // workgroups per kv head
    uint32_t n_deal;      // balanced: the workgroups per kv head the pages are dealt to
    uint64_t deal_work;   // balanced: the work dealt out (pages and segment costs)
    bool balanced;
};
decode_plan_shape shape_decode_plan(const std::vector<uint32_t>& positions, uint32_t block_size,
                                    uint32_t kv_heads, int cu_count);
// Waves per workgroup of the fast decode for a launch of `units` (plan
// workgroup, kv head) workgroups: a plan's split_pages (0 when no row is cut)
// and the batch's mean row pages decide it; CKV_DECODE_WAVES overrides.
uint32_t decode_fast_waves(uint32_t group, int dtype, uint32_t units, int cu_count,
                           uint32_t mean_pages, uint32_t split_pages);
constexpr size_t plan_entry_words = 8;
constexpr uint32_t plan_last = 0xFFFFFFFFu; // no next entry
// Writes shape.n_items plan entries to plan, rows words to split_first and the
// shape.n_cut cut rows to cut; offsets are the rows' table offsets.
void write_decode_plan(const std::vector<uint32_t>& positions,
                       const std::vector<uint32_t>& offsets, uint32_t block_size,
                       const decode_plan_shape& shape, std::vector<uint64_t>& sort_keys,
                       uint32_t* plan, uint32_t* split_first, uint32_t* cut);

// ---- launchers (kernels_decode.hip) ------------------------------------------
// Returns hipErrorInvalidValue when no kernel fits the geometry. The fast
// path (decode_fast_applies) merges a chunk's waves in the workgroup; when the
// plan cuts rows into chunks it needs `split` (records of m.n_records x q_heads)
// and launches a merge of the cut rows after the chunks; the generic path
// writes partials for rows with several chunks and needs a merge launch.
// gate (optional, same shape and dtype as out): out = attention * sigmoid(gate),
// the sigmoid_mul of src/qwen/qwen_layer.cc:204 in the epilogue.
hipError_t launch_decode(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                         const void* q, uint32_t q_heads, float scale, void* out,
                         float* partials, int cu_count, const void* gate = nullptr,
                         split_scratch split = {});
bool decode_fast_applies(const pool_view& p, uint32_t q_heads, const void* q, const void* out);
// store_kv + fast decode in one launch; the caller has checked
// decode_fast_applies, 16-byte aligned inputs, and that every row's slot is
// its position's slot with no two rows on one table range.
// With `rope` (rotary a multiple of 16 up to 128, rotary/16 a power of two)
// the queries and the new keys are rotated inside the kernel first.
hipError_t launch_append_decode(hipStream_t s, const pool_view& p, const meta_view& m,
                                uint32_t layer, const void* k_in, const void* v_in, const void* q,
                                uint32_t q_heads, float scale, void* out, const void* gate,
                                int cu_count, split_scratch split, const rope_table* rope = nullptr,
                                uint32_t rotary = 0);
hipError_t launch_merge(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t q_heads,
                        void* out, const float* partials, const void* gate = nullptr);
bool decode_uses_fast_path(const pool_view& p, uint32_t q_heads);
// Floats per (work item, q head) partial record: [max, denominator, 0, 0, acc[head_dim]].
uint32_t partial_record_floats(uint32_t head_dim);

// ---- launchers (kernels_prefill.hip, kernels_prefill_f32.hip) -----------------
// MFMA prefill: head_dim 128, 16-token pages, GQA group 1/2/4/8, 16-byte
// aligned pools, queries and output; bf16/fp16 products on
// v_mfma_f32_32x32x16, f32 ones on v_mfma_f32_32x32x2_f32.
bool prefill_supported(const pool_view& p, uint32_t q_heads, const void* q, const void* out);
// How a 16-bit prefill launch runs: workgroup waves (8, or 4 when 8-wave
// workgroups would not give every compute unit one) and the key split of the
// 4-wave form (1: none), with the records and counters that split needs.
struct prefill_shape_info {
    uint32_t waves;
    uint32_t n_split;
    uint32_t min_blocks;
    uint64_t records_floats;
    uint64_t counters;
};
prefill_shape_info prefill_plan(const pool_view& p, const meta_view& m, uint32_t q_heads,
                                int cu_count);
hipError_t launch_prefill(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                          const void* q, uint32_t q_heads, float scale, void* out,
                          const void* gate, const prefill_shape_info& plan,
                          prefill_split split);
hipError_t launch_prefill_f32(hipStream_t s, const pool_view& p, const meta_view& m,
                              uint32_t layer, const void* q, uint32_t q_heads, float scale,
                              void* out, const void* gate, prefill_split split);

// ---- launchers (kernels_rope.hip) --------------------------------------------------
// theta^(-2j/rotary) in float for j < rotary/2 (src/metal/metal_kernels.mm:186-191)
void rope_frequencies(float theta, uint32_t rotary, rope_table& out);
// rows of `heads` heads of the pool's head_dim and dtype, at the uploaded positions
hipError_t launch_rope(hipStream_t s, const pool_view& p, const meta_view& m, const void* in,
                       void* out, uint32_t rows, uint32_t heads, uint32_t rotary,
                       const rope_table& freq);
// rotated key rows and the value rows into the uploaded slots of `layer`
hipError_t launch_rope_append(hipStream_t s, const pool_view& p, const meta_view& m,
                              uint32_t layer, const void* keys, const void* values, uint32_t rows,
                              uint32_t rotary, const rope_table& freq);

} // namespace ckv

// C ABI of libckv: context, pool, metadata upload and op entry points.
//
// Every op validates on the host from the caller's arrays (the host cannot
// read device memory the way the reference reads Metal shared buffers), then
// enqueues HIP work on the context stream. Metadata goes up with one pinned
// host-to-device copy per call.
#include "ckv_internal.h"

#include <cmath>

#include <algorithm>
#include <array>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <unordered_map>
#include <unordered_set>

using namespace ckv;

// Scratch of ckv_append_decode_noalloc: the arrival counters (the first
// noalloc_counter_bytes; zero when the library loads, and every call leaves
// them zero) and then the partial records of the rows its batch plan cuts into
// chunks. Every GPU the library runs on holds its own copy of this array until
// the process ends. In host code `noalloc_scratch` is a host-side stand-in, not
// a device address: kernels are given the address hipGetSymbolAddress returns
// for the current device (ckv_context::noalloc_scratch).
constexpr size_t noalloc_scratch_bytes = (size_t)16 << 20;
constexpr size_t noalloc_counter_bytes = (size_t)256 << 10;
constexpr size_t noalloc_record_bytes = noalloc_scratch_bytes - noalloc_counter_bytes;
static __device__ __align__(256) unsigned char noalloc_scratch[noalloc_scratch_bytes];

namespace {

// hipGetSymbolAddress once per device, under a lock (contexts of different
// threads may be created at once); the result is kept per device ordinal.
constexpr int max_scratch_devices = 64;
std::mutex scratch_lock;
std::array<void*, max_scratch_devices> scratch_address {};
std::array<bool, max_scratch_devices> scratch_looked_up {};

// With `device` current: this device's address of noalloc_scratch, or null.
void* device_scratch(int device)
{
    if (device < 0 || device >= max_scratch_devices)
        return nullptr;
    std::lock_guard<std::mutex> hold(scratch_lock);
    if (!scratch_looked_up[device]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(noalloc_scratch));
        if (e != hipSuccess) {
            (void)hipGetLastError();
            ptr = nullptr;
        }
        scratch_address[device] = ptr;
        scratch_looked_up[device] = true;
    }
    return scratch_address[device];
}

int set_error(ckv_context* ctx, int code, const std::string& detail)
{
    if (ctx)
        ctx->last_error = detail;
    return code;
}

int hip_error(ckv_context* ctx, hipError_t e, const char* what)
{
    return set_error(ctx, CKV_E_HIP_FAILURE, std::string(what) + ": " + hipGetErrorString(e));
}

bool mul_fits(size_t a, size_t b, size_t* out)
{
    return !__builtin_mul_overflow(a, b, out);
}

pool_view view_of(const ckv_pool* p)
{
    pool_view v {};
    v.keys = p->keys;
    v.values = p->values;
    v.layer_elems = (uint64_t)p->blocks * p->block_size * p->kv_heads * p->head_dim;
    v.blocks = (uint32_t)p->blocks;
    v.block_size = (uint32_t)p->block_size;
    v.kv_heads = (uint32_t)p->kv_heads;
    v.head_dim = (uint32_t)p->head_dim;
    v.features = (uint32_t)(p->kv_heads * p->head_dim);
    v.elem_size = (uint32_t)p->elem_size;
    v.dtype = p->dtype;
    return v;
}

hipEvent_t take_event(ckv_context* ctx)
{
    if (!ctx->spare_events.empty()) {
        hipEvent_t e = ctx->spare_events.back();
        ctx->spare_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess)
        return nullptr;
    return e;
}

// Launches through `launch`, bracketing it with timing events when profiling.
template <class Launch>
int run_kernel(ckv_context* ctx, const char* name, Launch&& launch)
{
    hipEvent_t start = nullptr, stop = nullptr;
    if (ctx->profile) {
        start = take_event(ctx);
        stop = take_event(ctx);
        if (start && stop)
            (void)hipEventRecord(start, ctx->stream);
    }
    const hipError_t e = launch();
    if (start && stop) {
        (void)hipEventRecord(stop, ctx->stream);
        ctx->pending.push_back({ name, start, stop });
    }
    if (e != hipSuccess)
        return hip_error(ctx, e, name);
    return CKV_OK;
}

// Every device and pinned host allocation and free the library makes goes
// through these, which count them per context (ckv_debug_allocations): the
// no-allocation entry point is checked by that count staying put.
hipError_t dev_malloc(ckv_context* ctx, void** ptr, size_t bytes)
{
    ++ctx->allocations;
    return hipMalloc(ptr, bytes);
}

hipError_t dev_free(ckv_context* ctx, void* ptr)
{
    ++ctx->allocations;
    return hipFree(ptr);
}

hipError_t host_malloc(ckv_context* ctx, void** ptr, size_t bytes)
{
    ++ctx->allocations;
    return hipHostMalloc(ptr, bytes, hipHostMallocDefault);
}

hipError_t host_free(ckv_context* ctx, void* ptr)
{
    ++ctx->allocations;
    return hipHostFree(ptr);
}

// Returns pinned staging memory of at least `bytes`: the ring's next slot,
// after the copy last made from it has completed. upload_staged copies from
// this slot and advances the ring.
int stage(ckv_context* ctx, size_t bytes, void** host)
{
    auto& slot = ctx->staging[ctx->staging_next];
    if (slot.pending) {
        const hipError_t e = hipEventSynchronize(slot.done);
        if (e != hipSuccess)
            return hip_error(ctx, e, "staging wait");
        slot.pending = false;
    }
    if (bytes > slot.bytes) {
        if (slot.pinned)
            (void)host_free(ctx, slot.pinned);
        slot.pinned = nullptr;
        slot.bytes = 0;
        const size_t size = std::max<size_t>(bytes, 1 << 20);
        const hipError_t e = host_malloc(ctx, &slot.pinned, size);
        if (e != hipSuccess)
            return hip_error(ctx, e, "pinned staging allocation");
        slot.bytes = size;
    }
    *host = slot.pinned;
    return CKV_OK;
}

int upload_staged(ckv_context* ctx, void* device, size_t bytes)
{
    auto& slot = ctx->staging[ctx->staging_next];
    hipError_t e = hipMemcpyAsync(device, slot.pinned, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess)
        return hip_error(ctx, e, "metadata upload");
    e = hipEventRecord(slot.done, ctx->stream);
    if (e != hipSuccess)
        return hip_error(ctx, e, "metadata upload event");
    slot.pending = true;
    ctx->staging_next = (ctx->staging_next + 1) % ckv_context::staging_slots;
    return CKV_OK;
}

// Grow-only device buffer; the stream is drained before an old buffer is freed.
template <class T>
int ensure_device(ckv_context* ctx, T** ptr, size_t* capacity, size_t needed, const char* what)
{
    if (needed <= *capacity)
        return CKV_OK;
    // grow by half again at least: a batch a little larger than the last
    // must not reallocate (and drain the stream) every step
    const size_t count = std::max({ needed, *capacity + *capacity / 2, (size_t)1024 });
    if (*ptr) {
        (void)hipStreamSynchronize(ctx->stream);
        (void)dev_free(ctx, *ptr);
        *ptr = nullptr;
        *capacity = 0;
    }
    const hipError_t e = dev_malloc(ctx, reinterpret_cast<void**>(ptr), count * sizeof(T));
    if (e != hipSuccess)
        return hip_error(ctx, e, what);
    *capacity = count;
    return CKV_OK;
}

// Tokens per decode work item: enough (chunk, kv_head) waves for about 64 per
// compute unit, a multiple of 16 tokens, between 32 and 4096. CKV_DECODE_CHUNK
// overrides it (rounded to a multiple of 16).
uint32_t choose_chunk(uint64_t token_heads, int cu_count)
{
    if (const char* forced = std::getenv("CKV_DECODE_CHUNK")) {
        const long v = std::strtol(forced, nullptr, 10);
        if (v >= 16)
            return (uint32_t)((v + 15) / 16 * 16);
    }
    const uint64_t target = (uint64_t)std::max(cu_count, 1) * 64;
    uint64_t chunk = (token_heads + target - 1) / target;
    chunk = (chunk + 15) / 16 * 16;
    return (uint32_t)std::clamp<uint64_t>(chunk, 32, 4096);
}

size_t round4(size_t words)
{
    return (words + 3) & ~(size_t)3;
}

int check_attention(const ckv_pool* pool, size_t layer, const void* queries, size_t q_heads,
                    const void* output, size_t rows)
{
    ckv_context* ctx = pool->ctx;
    if (rows && (!queries || !output))
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "queries and output are required");
    // the order of validate_shapes (src/tensor/attention.cc:32-87)
    if (!pool->uploaded)
        return set_error(ctx, CKV_E_NO_TABLES, "attention before ckv_tables_upload");
    if (rows != pool->positions.size())
        return set_error(ctx, CKV_E_POSITION_COUNT_MISMATCH, "rows != uploaded positions");
    if (q_heads == 0)
        return set_error(ctx, CKV_E_INVALID_HEAD_COUNT, "q_heads == 0");
    if (q_heads % pool->kv_heads != 0)
        return set_error(ctx, CKV_E_INVALID_KV_HEAD_MAPPING, "q_heads % kv_heads != 0");
    if (layer >= pool->layers)
        return set_error(ctx, CKV_E_CACHE_LAYER_OUT_OF_RANGE, "layer >= layers");
    return CKV_OK;
}

// Whether keys[0..n) (each < bound) are distinct: a generation-stamped
// table, cleared only when the generation counter wraps.
bool all_distinct(ckv_pool* pool, const uint32_t* keys, size_t n, size_t bound)
{
    if (pool->stamp.size() < bound)
        pool->stamp.assign(bound, 0);
    if (++pool->stamp_generation == 0) {
        std::fill(pool->stamp.begin(), pool->stamp.end(), 0);
        pool->stamp_generation = 1;
    }
    const uint32_t g = pool->stamp_generation;
    for (size_t i = 0; i < n; ++i) {
        if (pool->stamp[keys[i]] == g)
            return false;
        pool->stamp[keys[i]] = g;
    }
    return true;
}

// The fused append + decode writes each row's new token into its own page
// while the batch's workgroups read their rows' pages: it keeps the semantics
// of store_kv followed by paged_attention only if no row reads a row's own
// page through any other table entry. own_pages_clash marks every row's own
// page (own(r): its table index) and scans the entries each row reads
// (entries(r): the first and one-past-last table index), reporting whether an
// own page is reached through an index other than its own.
template <class Own, class Entries>
bool own_pages_clash(ckv_pool* pool, const uint32_t* table, size_t rows, Own own, Entries entries)
{
    if (pool->own_stamp.size() < pool->blocks) {
        pool->own_stamp.assign(pool->blocks, 0);
        pool->own_at.assign(pool->blocks, 0);
    }
    if (++pool->own_generation == 0) {
        std::fill(pool->own_stamp.begin(), pool->own_stamp.end(), 0);
        pool->own_generation = 1;
    }
    const uint32_t g = pool->own_generation;
    for (size_t r = 0; r < rows; ++r) {
        const uint32_t at = own(r), page = table[at];
        if (pool->own_stamp[page] == g && pool->own_at[page] != at)
            return true; // two rows append into one page
        pool->own_stamp[page] = g;
        pool->own_at[page] = at;
    }
    for (size_t r = 0; r < rows; ++r) {
        const auto [first, end] = entries(r);
        for (uint32_t i = first; i < end; ++i)
            if (pool->own_stamp[table[i]] == g && pool->own_at[table[i]] != i)
                return true;
    }
    return false;
}

// Query tiles heaviest first, ties in their order: the prefill's workgroups
// start in tile order as compute units free up, so the launch's last round
// holds the lightest tiles. A tile of n rows from position p attends
// n (p + 1) + n (n - 1) / 2 keys.
void heaviest_first(std::vector<uint32_t>& tiles)
{
    const size_t n = tiles.size() / tile_entry_words;
    if (n < 2)
        return;
    std::vector<std::pair<uint64_t, uint32_t>> work(n);
    for (size_t t = 0; t < n; ++t) {
        const uint64_t rows = tiles[tile_entry_words * t + 1];
        const uint64_t first = tiles[tile_entry_words * t + 2];
        work[t] = { rows * (first + 1) + rows * (rows - 1) / 2, (uint32_t)t };
    }
    std::stable_sort(work.begin(), work.end(),
                     [](const auto& a, const auto& b) { return a.first > b.first; });
    std::vector<uint32_t> sorted(tiles.size());
    for (size_t t = 0; t < n; ++t)
        std::copy_n(tiles.begin() + tile_entry_words * work[t].second, tile_entry_words,
                    sorted.begin() + tile_entry_words * t);
    tiles.swap(sorted);
}

// The 32-key blocks the batch's shortest query tile attends (through its last
// row).
uint32_t shortest_tile_blocks(const std::vector<uint32_t>& tiles)
{
    const size_t n = tiles.size() / tile_entry_words;
    uint64_t least = n ? UINT64_MAX : 0;
    for (size_t t = 0; t < n; ++t) {
        const uint64_t rows = tiles[tile_entry_words * t + 1];
        const uint64_t first = tiles[tile_entry_words * t + 2];
        least = std::min<uint64_t>(least, (first + rows - 1) / 32 + 1);
    }
    return (uint32_t)least;
}

// Words of the fast decode plan in the metadata block: the segments'
// entries, each row's first partial record, then the cut rows.
size_t plan_words(const decode_plan_shape& shape, size_t rows)
{
    return round4(plan_entry_words * shape.n_items) + round4(rows) + shape.n_cut;
}

// Writes the plan at `words` (plan_words long) and points the batch's
// meta_view at `device`, its device copy.
void put_plan(ckv_pool* pool, const decode_plan_shape& shape, uint32_t* words,
              const uint32_t* device)
{
    const size_t s_first = round4(plan_entry_words * shape.n_items);
    const size_t s_cut = s_first + round4(pool->positions.size());
    write_decode_plan(pool->positions, pool->row_offsets, (uint32_t)pool->block_size, shape,
                      pool->sort_keys, words, words + s_first, words + s_cut);
    meta_view& m = pool->meta;
    m.plan = device;
    m.split_first = device + s_first;
    m.cut = device + s_cut;
    m.n_plan = shape.n_wgs;
    m.n_segments = shape.n_items;
    m.split_pages = shape.split_pages;
    m.n_records = shape.n_records;
    m.n_cut = shape.n_cut;
}

// The fast decode plan of a batch uploaded without it (one served by the
// prefill kernel), at its first decode launch.
int ensure_plan(ckv_pool* pool)
{
    if (pool->plan_ready)
        return CKV_OK;
    ckv_context* ctx = pool->ctx;
    const decode_plan_shape shape = shape_decode_plan(
        pool->positions, (uint32_t)pool->block_size, (uint32_t)pool->kv_heads, ctx->cu_count);
    const size_t words = std::max<size_t>(plan_words(shape, pool->positions.size()), 4);
    void* host = nullptr;
    int status = stage(ctx, words * sizeof(uint32_t), &host);
    if (status)
        return status;
    status = ensure_device(ctx, &pool->d_plan, &pool->d_plan_words, words, "decode plan");
    if (status)
        return status;
    put_plan(pool, shape, static_cast<uint32_t*>(host), pool->d_plan);
    status = upload_staged(ctx, pool->d_plan, words * sizeof(uint32_t));
    if (status)
        return status;
    pool->plan_ready = true;
    return CKV_OK;
}

// Scratch of the fast decode when its plan cuts rows into chunks: a partial
// record for every (record, q head) and an arrival counter for every
// (record, kv head). The counters have a buffer of their own (the generic
// decode writes its partials over d_partials) and are zeroed by a fill
// kernel whenever it is allocated; launches leave them zero.
int ensure_split(ckv_pool* pool, size_t q_heads, split_scratch& split)
{
    split = {};
    const meta_view& m = pool->meta;
    if (!m.n_cut)
        return CKV_OK;
    ckv_context* ctx = pool->ctx;
    size_t capacity_floats = pool->d_partials_bytes / sizeof(float);
    const size_t floats = (size_t)m.n_records * q_heads
        * partial_record_floats((uint32_t)pool->head_dim);
    int status = ensure_device(ctx, &pool->d_partials, &capacity_floats, floats,
                               "decode partials");
    pool->d_partials_bytes = capacity_floats * sizeof(float);
    if (status)
        return status;
    const size_t counters = (size_t)m.n_records * pool->kv_heads;
    if (counters > pool->d_arrivals_words) {
        status = ensure_device(ctx, &pool->d_arrivals, &pool->d_arrivals_words, counters,
                               "decode arrival counters");
        if (status)
            return status;
        status = run_kernel(ctx, "fill", [&] {
            return launch_fill(ctx->stream, pool->d_arrivals, 0,
                               (uint32_t)pool->d_arrivals_words);
        });
        if (status) {
            // not known to be zero: allocate and clear again next time
            (void)dev_free(ctx, pool->d_arrivals);
            pool->d_arrivals = nullptr;
            pool->d_arrivals_words = 0;
            return status;
        }
    }
    split.records = pool->d_partials;
    split.arrivals = pool->d_arrivals;
    return CKV_OK;
}

// The split-KV work list, at the batch's first split decode launch: each
// row's range 0..position cut into chunks of `chunk` tokens, (row, chunk)
// pairs, plus each row's first item and item count.
int ensure_work(ckv_pool* pool)
{
    if (pool->work_ready)
        return CKV_OK;
    ckv_context* ctx = pool->ctx;
    const std::vector<uint32_t>& positions = pool->positions;
    const size_t rows = positions.size();
    uint64_t token_heads = 0, n_items = 0;
    for (const uint32_t p : positions)
        token_heads += ((uint64_t)p + 1) * pool->kv_heads;
    const uint32_t chunk = choose_chunk(token_heads, ctx->cu_count);
    for (const uint32_t p : positions)
        n_items += p / chunk + 1;
    if (n_items > UINT32_MAX / pool->kv_heads)
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "too many decode work items");
    const size_t s_first = round4(2 * n_items);
    const size_t s_count = s_first + round4(rows);
    const size_t words = std::max<size_t>(s_count + rows, 4);
    void* host = nullptr;
    int status = stage(ctx, words * sizeof(uint32_t), &host);
    if (status)
        return status;
    auto* w = static_cast<uint32_t*>(host);
    bool multi = false;
    for (size_t r = 0, item = 0; r < rows; ++r) {
        const uint32_t n = positions[r] / chunk + 1;
        w[s_first + r] = (uint32_t)item;
        w[s_count + r] = n;
        multi = multi || n > 1;
        for (uint32_t c = 0; c < n; ++c, ++item) {
            w[2 * item] = (uint32_t)r;
            w[2 * item + 1] = c;
        }
    }
    status = ensure_device(ctx, &pool->d_work, &pool->d_work_words, words, "decode work list");
    if (status)
        return status;
    status = upload_staged(ctx, pool->d_work, words * sizeof(uint32_t));
    if (status)
        return status;
    meta_view& m = pool->meta;
    m.items = pool->d_work;
    m.row_first = pool->d_work + s_first;
    m.row_count = pool->d_work + s_count;
    m.n_items = (uint32_t)n_items;
    m.chunk = chunk;
    pool->work_multi = multi;
    pool->work_ready = true;
    return CKV_OK;
}

int run_decode(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads, float scale,
               void* output, const void* gate = nullptr)
{
    ckv_context* ctx = pool->ctx;
    const pool_view view = view_of(pool);
    float* partials = nullptr;
    split_scratch split {};
    const bool fast = decode_fast_applies(view, (uint32_t)q_heads, queries, output);
    int status = fast ? ensure_plan(pool) : ensure_work(pool);
    if (!status && fast)
        status = ensure_split(pool, q_heads, split);
    if (status)
        return status;
    const bool needs_merge = !fast && pool->work_multi;
    if (needs_merge) {
        size_t capacity_floats = pool->d_partials_bytes / sizeof(float);
        const size_t needed = (size_t)pool->meta.n_items * q_heads
            * partial_record_floats((uint32_t)pool->head_dim);
        status = ensure_device(ctx, &pool->d_partials, &capacity_floats, needed,
                               "decode partials");
        // stored whatever the outcome: a failed regrow leaves no buffer and
        // no capacity, so the next launch allocates again
        pool->d_partials_bytes = capacity_floats * sizeof(float);
        if (status)
            return status;
        partials = pool->d_partials;
    }
    status = run_kernel(ctx, "paged_attention_decode", [&] {
        return launch_decode(ctx->stream, view, pool->meta, (uint32_t)layer, queries,
                             (uint32_t)q_heads, scale, output, partials, ctx->cu_count, gate,
                             split);
    });
    if (status || !needs_merge)
        return status;
    return run_kernel(ctx, "paged_attention_merge", [&] {
        return launch_merge(ctx->stream, view, pool->meta, (uint32_t)q_heads, output, partials,
                            gate);
    });
}

int stage_pairs(ckv_pool* pool, const uint32_t* a, const uint32_t* b, size_t n)
{
    ckv_context* ctx = pool->ctx;
    void* host = nullptr;
    int status = stage(ctx, 2 * n * sizeof(uint32_t), &host);
    if (status)
        return status;
    auto* words = static_cast<uint32_t*>(host);
    for (size_t i = 0; i < n; ++i) {
        words[2 * i] = a[i];
        words[2 * i + 1] = b[i];
    }
    status = ensure_device(ctx, &pool->d_pairs, &pool->d_pairs_words, 2 * n, "pair buffer");
    if (status)
        return status;
    return upload_staged(ctx, pool->d_pairs, 2 * n * sizeof(uint32_t));
}

// Uploads a plain u32 list into the pool's pair buffer.
int stage_list(ckv_pool* pool, const uint32_t* list, size_t n)
{
    ckv_context* ctx = pool->ctx;
    void* host = nullptr;
    int status = stage(ctx, n * sizeof(uint32_t), &host);
    if (status)
        return status;
    std::memcpy(host, list, n * sizeof(uint32_t));
    status = ensure_device(ctx, &pool->d_pairs, &pool->d_pairs_words, n, "block list");
    if (status)
        return status;
    return upload_staged(ctx, pool->d_pairs, n * sizeof(uint32_t));
}

int validate_prefix(const ckv_pool* pool, const uint32_t* blocks, size_t n_blocks, size_t tokens)
{
    // metal_kv_cache::valid_prefix (src/metal/metal_kv_cache.cc:205-223)
    if (!tokens || tokens > pool->blocks * pool->block_size)
        return CKV_E_STATE_INVALID_RESERVATION;
    const size_t required = 1 + (tokens - 1) / pool->block_size;
    if (!blocks || n_blocks < required)
        return CKV_E_STATE_INVALID_RESERVATION;
    for (size_t i = 0; i < required; ++i)
        if (blocks[i] >= pool->blocks)
            return CKV_E_STATE_INVALID_RESERVATION;
    return CKV_OK;
}

int run_checkpoint(ckv_pool* pool, const uint32_t* blocks, size_t n_blocks, size_t tokens,
                   const void* packed_keys, const void* packed_values, bool unpack)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    int status = validate_prefix(pool, blocks, n_blocks, tokens);
    if (status)
        return set_error(ctx, status, "invalid checkpoint prefix");
    if (!packed_keys || !packed_values)
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "packed buffers are required");
    const size_t required = 1 + (tokens - 1) / pool->block_size;
    status = stage_list(pool, blocks, required);
    if (status)
        return status;
    const pool_view view = view_of(pool);
    return run_kernel(ctx, unpack ? "checkpoint_unpack" : "checkpoint_pack", [&] {
        return launch_checkpoint(ctx->stream, view, (uint32_t)pool->layers, pool->d_pairs,
                                 (uint32_t)tokens, const_cast<void*>(packed_keys),
                                 const_cast<void*>(packed_values), unpack);
    });
}

// Packed prefix <-> host memory, through a device staging buffer of at most
// spill_chunk_bytes per tensor: whole layers at a time, pack then copy down
// (export), or copy up then unpack (import). The packed layout is that of
// ckv_checkpoint_pack, so a layer range is one contiguous span of it.
constexpr size_t spill_chunk_bytes = 64u << 20;

int run_transfer(ckv_pool* pool, const uint32_t* blocks, size_t n_blocks, size_t tokens,
                 void* host_keys, void* host_values, bool import)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    int status = validate_prefix(pool, blocks, n_blocks, tokens);
    if (status)
        return set_error(ctx, status, "invalid checkpoint prefix");
    if (!host_keys || !host_values)
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "host buffers are required");
    const size_t required = 1 + (tokens - 1) / pool->block_size;
    status = stage_list(pool, blocks, required);
    if (status)
        return status;
    const size_t layer_bytes = tokens * pool->kv_heads * pool->head_dim * pool->elem_size;
    const size_t per_chunk = std::clamp<size_t>(spill_chunk_bytes / layer_bytes, 1, pool->layers);
    const size_t chunk_bytes = per_chunk * layer_bytes;
    status = ensure_device(ctx, &pool->d_spill, &pool->d_spill_bytes, 2 * chunk_bytes,
                           "spill staging");
    if (status)
        return status;
    char* stage_k = pool->d_spill;
    char* stage_v = pool->d_spill + chunk_bytes;
    auto* hk = static_cast<char*>(host_keys);
    auto* hv = static_cast<char*>(host_values);
    const size_t page_layer_bytes = pool->blocks * pool->block_size * pool->kv_heads
        * pool->head_dim * pool->elem_size;
    for (size_t l0 = 0; l0 < pool->layers; l0 += per_chunk) {
        const size_t n = std::min(per_chunk, pool->layers - l0);
        const size_t bytes = n * layer_bytes, at = l0 * layer_bytes;
        pool_view view = view_of(pool); // layers l0 .. l0 + n
        view.keys = static_cast<char*>(view.keys) + l0 * page_layer_bytes;
        view.values = static_cast<char*>(view.values) + l0 * page_layer_bytes;
        auto copy = [&](void* dst, const void* src, hipMemcpyKind kind) {
            const hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, ctx->stream);
            return e == hipSuccess ? CKV_OK : hip_error(ctx, e, "checkpoint host copy");
        };
        if (import) {
            status = copy(stage_k, hk + at, hipMemcpyHostToDevice);
            if (!status)
                status = copy(stage_v, hv + at, hipMemcpyHostToDevice);
        }
        if (!status)
            status = run_kernel(ctx, import ? "checkpoint_import" : "checkpoint_export", [&] {
                return launch_checkpoint(ctx->stream, view, (uint32_t)n, pool->d_pairs,
                                         (uint32_t)tokens, stage_k, stage_v, import);
            });
        if (!status && !import) {
            status = copy(hk + at, stage_k, hipMemcpyDeviceToHost);
            if (!status)
                status = copy(hv + at, stage_v, hipMemcpyDeviceToHost);
        }
        if (status)
            return status;
    }
    return CKV_OK;
}

int create_pool(ckv_context* ctx, size_t layers, size_t blocks, size_t block_size,
                size_t kv_heads, size_t head_dim, int dtype, void* keys, void* values,
                ckv_pool** out)
{
    if (!ctx || !out)
        return CKV_E_INVALID_ARGUMENT;
    *out = nullptr;
    // metal_kv_cache::make (src/metal/metal_kv_cache.cc:38-82)
    if (layers == 0)
        return set_error(ctx, CKV_E_INVALID_LAYER_COUNT, "layers == 0");
    if (blocks == 0)
        return set_error(ctx, CKV_E_INVALID_BLOCK_COUNT, "blocks == 0");
    if (block_size == 0)
        return set_error(ctx, CKV_E_INVALID_BLOCK_SIZE, "block_size == 0");
    if (kv_heads == 0)
        return set_error(ctx, CKV_E_INVALID_KV_HEAD_COUNT, "kv_heads == 0");
    if (head_dim == 0)
        return set_error(ctx, CKV_E_INVALID_HEAD_DIMENSION_KV, "head_dim == 0");
    if (dtype != CKV_F32 && dtype != CKV_BF16 && dtype != CKV_F16)
        return set_error(ctx, CKV_E_UNSUPPORTED_DTYPE, "dtype must be f32, bf16 or f16");
    const size_t elem = dtype == CKV_F32 ? 4 : 2;
    size_t elements = layers, bytes = 0, slots = 0, features = 0;
    if (!mul_fits(elements, blocks, &elements) || !mul_fits(elements, block_size, &elements)
        || !mul_fits(elements, kv_heads, &elements) || !mul_fits(elements, head_dim, &elements)
        || !mul_fits(elements, elem, &bytes) || !mul_fits(blocks, block_size, &slots)
        || slots > UINT32_MAX || !mul_fits(kv_heads, head_dim, &features)
        || features > UINT32_MAX || layers > UINT32_MAX)
        return set_error(ctx, CKV_E_LAYOUT_SIZE_OVERFLOW, "KV layout does not fit");
    auto* pool = new (std::nothrow) ckv_pool;
    if (!pool)
        return set_error(ctx, CKV_E_KV_ALLOCATION_FAILED, "pool object");
    pool->ctx = ctx;
    pool->layers = layers;
    pool->blocks = blocks;
    pool->block_size = block_size;
    pool->kv_heads = kv_heads;
    pool->head_dim = head_dim;
    pool->dtype = dtype;
    pool->elem_size = elem;
    pool->bytes_each = bytes;
    if (keys || values) {
        if (!keys || !values) {
            delete pool;
            return set_error(ctx, CKV_E_INVALID_ARGUMENT, "both buffers are required");
        }
        pool->keys = keys;
        pool->values = values;
        pool->owned = false;
    } else {
        (void)hipSetDevice(ctx->device);
        hipError_t e = dev_malloc(ctx, &pool->keys, bytes);
        if (e == hipSuccess)
            e = dev_malloc(ctx, &pool->values, bytes);
        if (e != hipSuccess) {
            if (pool->keys)
                (void)dev_free(ctx, pool->keys);
            delete pool;
            (void)hipGetLastError();
            return set_error(ctx, CKV_E_KV_ALLOCATION_FAILED,
                             std::string("KV allocation: ") + hipGetErrorString(e));
        }
        pool->owned = true;
    }
    *out = pool;
    return CKV_OK;
}

} // namespace

extern "C" {

int ckv_abi_version(void)
{
    return CKV_ABI_VERSION;
}

const char* ckv_error_name(int code)
{
    static const char* tensor_op[] = {
        "tensor_op.tensor_creation_failed",
        "tensor_op.allocation_failed",
        "tensor_op.empty_tokens",
        "tensor_op.empty_logits_indices",
        "tensor_op.invalid_hidden_states",
        "tensor_op.logits_index_out_of_range",
        "tensor_op.token_id_overflow",
        "tensor_op.invalid_rank",
        "tensor_op.unsupported_dtype",
        "tensor_op.input_shape_mismatch",
        "tensor_op.inner_dimension_mismatch",
        "tensor_op.output_shape_mismatch",
        "tensor_op.token_out_of_range",
        "tensor_op.invalid_epsilon",
        "tensor_op.position_count_mismatch",
        "tensor_op.invalid_head_count",
        "tensor_op.invalid_head_dimension",
        "tensor_op.invalid_rope_theta",
        "tensor_op.cache_slot_count_mismatch",
        "tensor_op.cache_feature_count_mismatch",
        "tensor_op.cache_layer_out_of_range",
        "tensor_op.cache_slot_out_of_range",
        "tensor_op.block_table_metadata_count_mismatch",
        "tensor_op.block_table_range_out_of_bounds",
        "tensor_op.cache_block_out_of_range",
        "tensor_op.cache_head_dimension_mismatch",
        "tensor_op.invalid_kv_head_mapping",
        "tensor_op.backend_failure",
        "tensor_op.unsupported_aliasing",
    };
    static const char* kv_cache[] = {
        "kv_cache.invalid_layer_count",    "kv_cache.invalid_block_count",
        "kv_cache.invalid_block_size",     "kv_cache.invalid_kv_head_count",
        "kv_cache.invalid_head_dimension", "kv_cache.layout_size_overflow",
        "kv_cache.allocation_failed",      "kv_cache.layer_out_of_range",
        "kv_cache.block_out_of_range",     "kv_cache.token_offset_out_of_range",
        "kv_cache.kv_head_out_of_range",   "kv_cache.head_feature_out_of_range",
    };
    static const char* state[] = {
        "state.capacity_exhausted",
        "state.invalid_reservation",
        "state.backend_failure",
        "state.allocation_failed",
    };
    static const char* own[] = {
        "ckv.invalid_argument",
        "ckv.hip_failure",
        "ckv.no_device",
        "ckv.no_tables",
    };
    if (code == 0)
        return "ok";
    if (code >= 100 && code < 100 + (int)(sizeof tensor_op / sizeof *tensor_op))
        return tensor_op[code - 100];
    if (code >= 200 && code < 200 + (int)(sizeof kv_cache / sizeof *kv_cache))
        return kv_cache[code - 200];
    if (code >= 300 && code < 300 + (int)(sizeof state / sizeof *state))
        return state[code - 300];
    if (code >= 400 && code < 400 + (int)(sizeof own / sizeof *own))
        return own[code - 400];
    return "ckv.unknown_error";
}

const char* ckv_last_error(const ckv_context* ctx)
{
    return ctx ? ctx->last_error.c_str() : "";
}

int ckv_context_create(int device, ckv_context** out)
{
    if (!out)
        return CKV_E_INVALID_ARGUMENT;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) {
        (void)hipGetLastError();
        return CKV_E_NO_DEVICE;
    }
    auto* ctx = new (std::nothrow) ckv_context;
    if (!ctx)
        return CKV_E_INVALID_ARGUMENT;
    ctx->device = device;
    hipError_t e = hipSetDevice(device);
    hipDeviceProp_t props {};
    if (e == hipSuccess)
        e = hipGetDeviceProperties(&props, device);
    if (e == hipSuccess)
        e = hipStreamCreate(&ctx->own_stream);
    for (auto& slot : ctx->staging)
        if (e == hipSuccess)
            e = hipEventCreateWithFlags(&slot.done, hipEventDisableTiming);
    if (e != hipSuccess) {
        for (auto& slot : ctx->staging)
            if (slot.done)
                (void)hipEventDestroy(slot.done);
        if (ctx->own_stream)
            (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return CKV_E_HIP_FAILURE;
    }
    ctx->cu_count = props.multiProcessorCount;
    ctx->stream = ctx->own_stream;
    // the device is current: its copy of the no-allocation scratch
    ctx->noalloc_scratch = device_scratch(device);
    // room for any detail text, so that storing one never allocates
    ctx->last_error.reserve(512);
    *out = ctx;
    return CKV_OK;
}

int ckv_context_destroy(ckv_context* ctx)
{
    if (!ctx)
        return CKV_E_INVALID_ARGUMENT;
    (void)hipStreamSynchronize(ctx->stream);
    for (auto& p : ctx->pending) {
        (void)hipEventDestroy(p.start);
        (void)hipEventDestroy(p.stop);
    }
    for (auto e : ctx->spare_events)
        (void)hipEventDestroy(e);
    for (auto& slot : ctx->staging) {
        if (slot.pinned)
            (void)host_free(ctx, slot.pinned);
        (void)hipEventDestroy(slot.done);
    }
    (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return CKV_OK;
}

int ckv_context_set_stream(ckv_context* ctx, void* hip_stream)
{
    if (!ctx)
        return CKV_E_INVALID_ARGUMENT;
    // work already enqueued on the old stream finishes before the switch
    (void)hipStreamSynchronize(ctx->stream);
    ctx->stream = static_cast<hipStream_t>(hip_stream);
    return CKV_OK;
}

void* ckv_context_stream(const ckv_context* ctx)
{
    return ctx ? ctx->stream : nullptr;
}

void* ckv_context_own_stream(const ckv_context* ctx)
{
    return ctx ? ctx->own_stream : nullptr;
}

int ckv_sync(ckv_context* ctx)
{
    if (!ctx)
        return CKV_E_INVALID_ARGUMENT;
    const hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess)
        return hip_error(ctx, e, "stream synchronize");
    return CKV_OK;
}

int ckv_debug_allocations(const ckv_context* ctx, uint64_t* count)
{
    if (!ctx || !count)
        return CKV_E_INVALID_ARGUMENT;
    *count = ctx->allocations;
    return CKV_OK;
}

int ckv_device_alloc(ckv_context* ctx, size_t bytes, void** out)
{
    if (!ctx || !out)
        return CKV_E_INVALID_ARGUMENT;
    *out = nullptr;
    (void)hipSetDevice(ctx->device);
    const hipError_t e = dev_malloc(ctx, out, bytes ? bytes : 1);
    if (e != hipSuccess) {
        *out = nullptr;
        return hip_error(ctx, e, "device buffer allocation");
    }
    return CKV_OK;
}

int ckv_device_free(ckv_context* ctx, void* ptr)
{
    if (!ctx)
        return CKV_E_INVALID_ARGUMENT;
    if (!ptr)
        return CKV_OK;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess)
        e = dev_free(ctx, ptr);
    if (e != hipSuccess)
        return hip_error(ctx, e, "device buffer free");
    return CKV_OK;
}

int ckv_host_alloc(ckv_context* ctx, size_t bytes, void** out)
{
    if (!ctx || !out)
        return CKV_E_INVALID_ARGUMENT;
    *out = nullptr;
    (void)hipSetDevice(ctx->device);
    const hipError_t e = host_malloc(ctx, out, bytes ? bytes : 1);
    if (e != hipSuccess) {
        *out = nullptr;
        return hip_error(ctx, e, "pinned host allocation");
    }
    return CKV_OK;
}

int ckv_host_free(ckv_context* ctx, void* ptr)
{
    if (!ctx)
        return CKV_E_INVALID_ARGUMENT;
    if (!ptr)
        return CKV_OK;
    // copies to or from the buffer may still be queued
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess)
        e = host_free(ctx, ptr);
    if (e != hipSuccess)
        return hip_error(ctx, e, "pinned host free");
    return CKV_OK;
}

int ckv_copy_to_device(ckv_context* ctx, void* device_dst, const void* host_src, size_t bytes)
{
    if (!ctx || (bytes && (!device_dst || !host_src)))
        return CKV_E_INVALID_ARGUMENT;
    hipError_t e = hipMemcpyAsync(device_dst, host_src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess)
        return hip_error(ctx, e, "copy to device");
    return CKV_OK;
}

int ckv_copy_to_host(ckv_context* ctx, void* host_dst, const void* device_src, size_t bytes)
{
    if (!ctx || (bytes && (!host_dst || !device_src)))
        return CKV_E_INVALID_ARGUMENT;
    hipError_t e = hipMemcpyAsync(host_dst, device_src, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess)
        return hip_error(ctx, e, "copy to host");
    return CKV_OK;
}

int ckv_profile_enable(ckv_context* ctx, int enabled)
{
    if (!ctx)
        return CKV_E_INVALID_ARGUMENT;
    ctx->profile = enabled != 0;
    return CKV_OK;
}

int ckv_profile_query(ckv_context* ctx, const char* kernel, double* total_ms, uint64_t* launches)
{
    if (!ctx || !kernel)
        return CKV_E_INVALID_ARGUMENT;
    for (auto& p : ctx->pending) {
        hipError_t e = hipEventSynchronize(p.stop);
        float ms = 0.0f;
        if (e == hipSuccess)
            e = hipEventElapsedTime(&ms, p.start, p.stop);
        if (e != hipSuccess)
            return hip_error(ctx, e, "profile events");
        auto& total = ctx->totals[p.name];
        total.ms += ms;
        total.launches += 1;
        ctx->spare_events.push_back(p.start);
        ctx->spare_events.push_back(p.stop);
    }
    ctx->pending.clear();
    const auto found = ctx->totals.find(kernel);
    if (total_ms)
        *total_ms = found == ctx->totals.end() ? 0.0 : found->second.ms;
    if (launches)
        *launches = found == ctx->totals.end() ? 0 : found->second.launches;
    return CKV_OK;
}

int ckv_profile_reset(ckv_context* ctx)
{
    if (!ctx)
        return CKV_E_INVALID_ARGUMENT;
    double ms;
    uint64_t n;
    const int status = ckv_profile_query(ctx, "", &ms, &n); // drains pending events
    ctx->totals.clear();
    return status;
}

int ckv_pool_create(ckv_context* ctx, size_t layers, size_t blocks, size_t block_size,
                    size_t kv_heads, size_t head_dim, int dtype, ckv_pool** out)
{
    return create_pool(ctx, layers, blocks, block_size, kv_heads, head_dim, dtype, nullptr,
                       nullptr, out);
}

int ckv_pool_wrap(ckv_context* ctx, size_t layers, size_t blocks, size_t block_size,
                  size_t kv_heads, size_t head_dim, int dtype, void* keys, void* values,
                  ckv_pool** out)
{
    if (!keys || !values)
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "both buffers are required");
    return create_pool(ctx, layers, blocks, block_size, kv_heads, head_dim, dtype, keys, values,
                       out);
}

int ckv_pool_destroy(ckv_pool* pool)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    (void)hipStreamSynchronize(ctx->stream);
    if (pool->owned) {
        (void)dev_free(ctx, pool->keys);
        (void)dev_free(ctx, pool->values);
    }
    if (pool->d_meta)
        (void)dev_free(ctx, pool->d_meta);
    if (pool->d_partials)
        (void)dev_free(ctx, pool->d_partials);
    if (pool->d_arrivals)
        (void)dev_free(ctx, pool->d_arrivals);
    if (pool->d_pre_records)
        (void)dev_free(ctx, pool->d_pre_records);
    if (pool->d_pre_arrivals)
        (void)dev_free(ctx, pool->d_pre_arrivals);
    if (pool->d_pairs)
        (void)dev_free(ctx, pool->d_pairs);
    if (pool->d_seq)
        (void)dev_free(ctx, pool->d_seq);
    if (pool->d_plan)
        (void)dev_free(ctx, pool->d_plan);
    if (pool->d_work)
        (void)dev_free(ctx, pool->d_work);
    if (pool->d_spill)
        (void)dev_free(ctx, pool->d_spill);
    if (pool->d_rope_q)
        (void)dev_free(ctx, pool->d_rope_q);
    delete pool;
    return CKV_OK;
}

int ckv_pool_buffers(const ckv_pool* pool, void** keys, void** values, size_t* bytes_each)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    if (keys)
        *keys = pool->keys;
    if (values)
        *values = pool->values;
    if (bytes_each)
        *bytes_each = pool->bytes_each;
    return CKV_OK;
}

int ckv_element_offset(const ckv_pool* pool, size_t layer, size_t block, size_t token_offset,
                       size_t kv_head, size_t head_feature, size_t* offset)
{
    if (!pool || !offset)
        return CKV_E_INVALID_ARGUMENT;
    if (layer >= pool->layers)
        return CKV_E_LAYER_OUT_OF_RANGE;
    if (block >= pool->blocks)
        return CKV_E_BLOCK_OUT_OF_RANGE;
    if (token_offset >= pool->block_size)
        return CKV_E_TOKEN_OFFSET_OUT_OF_RANGE;
    if (kv_head >= pool->kv_heads)
        return CKV_E_KV_HEAD_OUT_OF_RANGE;
    if (head_feature >= pool->head_dim)
        return CKV_E_HEAD_FEATURE_OUT_OF_RANGE;
    *offset = (((layer * pool->blocks + block) * pool->block_size + token_offset) * pool->kv_heads
               + kv_head)
            * pool->head_dim
        + head_feature;
    return CKV_OK;
}

namespace {

// The host state of a batch just uploaded; the work list (and, unless it
// was uploaded, the decode plan) are derived on first use.
void adopt_batch(ckv_pool* pool, size_t rows, size_t n_entries, bool with_slots, bool shared,
                 bool fusable, bool plan_uploaded, bool device_tables)
{
    meta_view& m = pool->meta;
    m.n_entries = (uint32_t)n_entries;
    m.rows = (uint32_t)rows;
    uint64_t pages = 0;
    for (const uint32_t position : pool->positions)
        pages += position / pool->block_size + 1;
    m.mean_pages = rows ? (uint32_t)(pages / rows) : 0;
    m.items = m.row_first = m.row_count = nullptr;
    m.n_items = 0;
    m.chunk = 0;
    if (!plan_uploaded) {
        m.plan = m.split_first = m.cut = nullptr;
        m.n_plan = m.n_segments = m.split_pages = m.n_records = m.n_cut = 0;
    }
    pool->has_slots = with_slots;
    pool->slot_rows = with_slots ? rows : 0;
    pool->n_entries = n_entries;
    pool->device_tables = device_tables;
    pool->shared_tile = shared;
    pool->fusable = fusable;
    pool->plan_ready = plan_uploaded;
    pool->work_ready = false;
    pool->uploaded = true;
}

} // namespace

int ckv_tables_upload(ckv_pool* pool, const uint32_t* block_table, size_t n_entries,
                      const uint32_t* offsets, const uint32_t* lengths,
                      const uint32_t* positions, const uint32_t* slots, size_t rows)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if ((n_entries && !block_table) || (rows && (!offsets || !lengths || !positions)))
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "metadata arrays are required");
    if (n_entries > UINT32_MAX || rows > UINT32_MAX)
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "metadata exceeds u32 counts");
    const size_t bs = pool->block_size;
    // prepared_attention_batch::make (src/tensor/attention.cc:110-137): row ranges
    // first, then every table entry
    for (size_t r = 0; r < rows; ++r) {
        const size_t required = positions[r] / bs + 1;
        if (offsets[r] > n_entries || lengths[r] > n_entries - offsets[r] || required > lengths[r])
            return set_error(ctx, CKV_E_BLOCK_TABLE_RANGE_OUT_OF_BOUNDS,
                             "row " + std::to_string(r) + " table range");
    }
    for (size_t i = 0; i < n_entries; ++i)
        if (block_table[i] >= pool->blocks)
            return set_error(ctx, CKV_E_CACHE_BLOCK_OUT_OF_RANGE,
                             "table entry " + std::to_string(i));
    // store_kv's slot check (src/tensor/tensor_ops.cc:445-453)
    const size_t slot_count = pool->blocks * bs;
    if (slots)
        for (size_t r = 0; r < rows; ++r)
            if (slots[r] >= slot_count)
                return set_error(ctx, CKV_E_CACHE_SLOT_OUT_OF_RANGE,
                                 "slot of row " + std::to_string(r));

    // query tiles: runs of consecutive positions sharing a table range
    // (src/tensor/attention.cc:142-167), up to prefill_tile_rows rows
    std::vector<uint32_t>& tiles = pool->scratch;
    tiles.clear();
    bool shared = false;
    for (size_t r = 0; r < rows;) {
        size_t n = 1;
        while (n < prefill_tile_rows && r + n < rows && offsets[r + n] == offsets[r]
               && lengths[r + n] == lengths[r] && positions[r + n] == positions[r + n - 1] + 1)
            ++n;
        tiles.insert(tiles.end(), { (uint32_t)r, (uint32_t)n, positions[r], offsets[r] });
        shared = shared || n > 1;
        r += n;
    }
    heaviest_first(tiles);

    // append + decode can run as one launch when every row appends the token at
    // its own position and no two rows attend through the same table range
    bool fusable = slots != nullptr;
    for (size_t r = 0; r < rows && fusable; ++r) {
        const uint64_t own = (uint64_t)block_table[offsets[r] + positions[r] / bs] * bs
            + positions[r] % bs;
        fusable = own == slots[r];
    }
    fusable = fusable && all_distinct(pool, offsets, rows, n_entries + 1);
    fusable = fusable
        && !own_pages_clash(
            pool, block_table, rows,
            [&](size_t r) { return (uint32_t)(offsets[r] + positions[r] / bs); },
            [&](size_t r) {
                return std::pair<uint32_t, uint32_t> { offsets[r],
                                                       (uint32_t)(offsets[r] + positions[r] / bs + 1) };
            });
    // the checks passed: from here the batch's host state and device metadata
    // are replaced, so until this batch is adopted launches report no tables
    // (never the previous batch's pointers with this batch's positions)
    pool->uploaded = false;
    pool->positions.assign(positions, positions + rows);
    pool->row_offsets.assign(offsets, offsets + rows);
    if (fusable) {
        pool->own_index.resize(rows);
        for (size_t r = 0; r < rows; ++r)
            pool->own_index[r] = (uint32_t)(offsets[r] + positions[r] / bs);
        pool->own_slot.assign(slots, slots + rows);
    }
    // a batch of single-row tiles goes to the decode kernel: its plan goes
    // up now
    const bool with_plan = !shared;
    const decode_plan_shape plan_shape = with_plan
        ? shape_decode_plan(pool->positions, (uint32_t)bs, (uint32_t)pool->kv_heads, ctx->cu_count)
        : decode_plan_shape {};

    // pack: table | offsets | lengths | positions | slots | tiles | plan
    const size_t s_table = 0;
    const size_t s_offsets = s_table + round4(n_entries);
    const size_t s_lengths = s_offsets + round4(rows);
    const size_t s_positions = s_lengths + round4(rows);
    const size_t s_slots = s_positions + round4(rows);
    const size_t s_tiles = s_slots + round4(rows);
    const size_t s_plan = s_tiles + round4(tiles.size());
    const size_t words = std::max<size_t>(s_plan + (with_plan ? plan_words(plan_shape, rows) : 0), 4);
    void* host = nullptr;
    int status = stage(ctx, words * sizeof(uint32_t), &host);
    if (status)
        return status;
    auto* w = static_cast<uint32_t*>(host);
    auto put = [&](size_t at, const uint32_t* src, size_t n) {
        if (n)
            std::memcpy(w + at, src, n * sizeof(uint32_t));
    };
    put(s_table, block_table, n_entries);
    put(s_offsets, offsets, rows);
    put(s_lengths, lengths, rows);
    put(s_positions, positions, rows);
    if (slots)
        put(s_slots, slots, rows);
    put(s_tiles, tiles.data(), tiles.size());
    status = ensure_device(ctx, &pool->d_meta, &pool->d_meta_words, words, "metadata buffer");
    if (status)
        return status;
    if (with_plan)
        put_plan(pool, plan_shape, w + s_plan, pool->d_meta + s_plan);
    status = upload_staged(ctx, pool->d_meta, words * sizeof(uint32_t));
    if (status)
        return status;

    meta_view& m = pool->meta;
    m.table = pool->d_meta + s_table;
    m.offsets = pool->d_meta + s_offsets;
    m.lengths = pool->d_meta + s_lengths;
    m.positions = pool->d_meta + s_positions;
    m.slots = pool->d_meta + s_slots;
    m.tiles = pool->d_meta + s_tiles;
    m.n_tiles = (uint32_t)(tiles.size() / tile_entry_words);
    m.tile_blocks = shortest_tile_blocks(tiles);
    adopt_batch(pool, rows, n_entries, slots != nullptr, shared, fusable, with_plan, false);
    return CKV_OK;
}

int ckv_tables_patch(ckv_pool* pool, const uint32_t* idx, const uint32_t* val, size_t n)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if (!n)
        return CKV_OK;
    if (!idx || !val)
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "patch arrays are required");
    if (!pool->uploaded)
        return set_error(ctx, CKV_E_NO_TABLES, "patch before ckv_tables_upload");
    if (pool->device_tables)
        return set_error(ctx, CKV_E_INVALID_ARGUMENT,
                         "the batch indexes the sequence tables: use ckv_seq_tables_update");
    for (size_t i = 0; i < n; ++i) {
        if (idx[i] >= pool->n_entries)
            return set_error(ctx, CKV_E_BLOCK_TABLE_RANGE_OUT_OF_BOUNDS, "patch index");
        if (val[i] >= pool->blocks)
            return set_error(ctx, CKV_E_CACHE_BLOCK_OUT_OF_RANGE, "patch value");
    }
    int status = stage_pairs(pool, idx, val, n);
    if (status)
        return status;
    uint32_t* table = pool->d_meta; // the table section starts the metadata block
    status = run_kernel(ctx, "tables_patch", [&] {
        return launch_table_patch(ctx->stream, table, pool->d_pairs, (uint32_t)n);
    });
    if (status) {
        pool->uploaded = false; // the device table may hold part of the patch
        return status;
    }
    // The fused append writes a row's token through the table (its own
    // position's page), ckv_append through the uploaded slot: once a patch
    // moves a row's own page elsewhere, only the unfused pair keeps the
    // semantics of store_kv followed by paged_attention. The last write of
    // an index wins, as on the device.
    // A patch that points another entry at a row's own page would have that
    // page read while the fused append writes it: the batch then takes the
    // unfused pair as well.
    if (pool->fusable) {
        std::unordered_map<uint32_t, uint32_t> patched;
        for (size_t i = 0; i < n; ++i)
            patched[idx[i]] = val[i];
        const size_t bs = pool->block_size;
        std::unordered_map<uint32_t, uint32_t> own_page; // page -> its own table index
        for (size_t r = 0; r < pool->own_index.size() && pool->fusable; ++r) {
            const auto at = patched.find(pool->own_index[r]);
            if (at != patched.end())
                pool->fusable = (uint64_t)at->second * bs + pool->positions[r] % bs
                    == pool->own_slot[r];
            own_page[(uint32_t)(pool->own_slot[r] / bs)] = pool->own_index[r];
        }
        for (const auto& [index, page] : patched) {
            if (!pool->fusable)
                break;
            const auto own = own_page.find(page);
            if (own != own_page.end() && own->second != index)
                pool->fusable = false;
        }
    }
    return CKV_OK;
}

int ckv_seq_tables_reserve(ckv_pool* pool, size_t max_sequences, size_t pages_per_sequence)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if (!max_sequences || !pages_per_sequence
        || (uint64_t)max_sequences * pages_per_sequence > UINT32_MAX)
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "sequence table arena size");
    const size_t words = max_sequences * pages_per_sequence;
    if (pool->device_tables)
        pool->uploaded = false; // the batch indexes the arena, which may be replaced
    int status = ensure_device(ctx, &pool->d_seq, &pool->d_seq_words, words, "sequence tables");
    if (status)
        return status;
    // every entry starts as page 0: a valid page id, whatever a range reads
    uint32_t* arena = pool->d_seq;
    status = run_kernel(ctx, "tables_fill",
                        [&] { return launch_fill(ctx->stream, arena, 0, (uint32_t)words); });
    if (status)
        return status;
    pool->seq_max = max_sequences;
    pool->seq_cap = pages_per_sequence;
    pool->seq_len.assign(max_sequences, 0);
    pool->seq_host.assign(words, 0);
    pool->seq_dirty.assign(words, 0);
    pool->dirty.clear();
    return CKV_OK;
}

int ckv_seq_tables_update(ckv_pool* pool, const uint32_t* seq, const uint32_t* index,
                          const uint32_t* block, size_t n, const uint32_t* len_seq,
                          const uint32_t* length, size_t m)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if ((n && (!seq || !index || !block)) || (m && (!len_seq || !length)))
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "update arrays are required");
    if (!pool->d_seq)
        return set_error(ctx, CKV_E_NO_TABLES, "update before ckv_seq_tables_reserve");
    for (size_t i = 0; i < n; ++i) {
        if (seq[i] >= pool->seq_max || index[i] >= pool->seq_cap)
            return set_error(ctx, CKV_E_BLOCK_TABLE_RANGE_OUT_OF_BOUNDS,
                             "entry " + std::to_string(i) + " outside the arena");
        if (block[i] >= pool->blocks)
            return set_error(ctx, CKV_E_CACHE_BLOCK_OUT_OF_RANGE,
                             "entry " + std::to_string(i) + " page id");
    }
    for (size_t j = 0; j < m; ++j)
        if (len_seq[j] >= pool->seq_max || length[j] > pool->seq_cap)
            return set_error(ctx, CKV_E_BLOCK_TABLE_RANGE_OUT_OF_BOUNDS,
                             "length " + std::to_string(j) + " outside the arena");
    // pending until the next batch upload; a later write of an entry wins
    for (size_t i = 0; i < n; ++i) {
        const size_t at = (size_t)seq[i] * pool->seq_cap + index[i];
        pool->seq_host[at] = block[i];
        if (!pool->seq_dirty[at]) {
            pool->seq_dirty[at] = 1;
            pool->dirty.push_back((uint32_t)at);
        }
    }
    for (size_t j = 0; j < m; ++j)
        pool->seq_len[len_seq[j]] = length[j];
    return CKV_OK;
}

int ckv_batch_upload(ckv_pool* pool, const uint32_t* seq, const uint32_t* first_position,
                     const uint32_t* token_count, size_t n_items, int with_slots)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if (n_items && (!seq || !first_position || !token_count))
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "item arrays are required");
    if (!pool->d_seq)
        return set_error(ctx, CKV_E_NO_TABLES, "batch upload before ckv_seq_tables_reserve");
    const size_t bs = pool->block_size;
    // rows, and the checks of prepared_attention_batch::make
    // (src/tensor/attention.cc:110-137) against the sequences' table lengths
    uint64_t rows = 0;
    for (size_t i = 0; i < n_items; ++i) {
        if (!token_count[i])
            return set_error(ctx, CKV_E_INVALID_ARGUMENT, "item with no tokens");
        const uint64_t last = (uint64_t)first_position[i] + token_count[i] - 1;
        if (seq[i] >= pool->seq_max || last > UINT32_MAX
            || last / bs >= pool->seq_len[seq[i]])
            return set_error(ctx, CKV_E_BLOCK_TABLE_RANGE_OUT_OF_BOUNDS,
                             "item " + std::to_string(i) + " table range");
        rows += token_count[i];
    }
    if (rows > UINT32_MAX || n_items > UINT32_MAX)
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "batch exceeds u32 counts");

    // query tiles: items of one sequence at consecutive positions, up to
    // prefill_tile_rows rows (the rule of src/tensor/attention.cc:142-167)
    std::vector<uint32_t>& tiles = pool->scratch;
    tiles.clear();
    bool shared = false;
    for (size_t i = 0, first_row = 0; i < n_items;) {
        size_t end = i + 1, span = token_count[i]; // items [i, end) continue one another
        while (end < n_items && seq[end] == seq[i]
               && first_position[end]
                   == (uint64_t)first_position[end - 1] + token_count[end - 1])
            span += token_count[end++];
        for (size_t at = 0; at < span; at += prefill_tile_rows) {
            const size_t n = std::min<size_t>(prefill_tile_rows, span - at);
            tiles.insert(tiles.end(), { (uint32_t)(first_row + at), (uint32_t)n,
                                        (uint32_t)(first_position[i] + at),
                                        seq[i] * (uint32_t)pool->seq_cap });
            shared = shared || n > 1;
        }
        first_row += span;
        i = end;
    }
    heaviest_first(tiles);
    // one decode row per sequence at its own position's slot: fusable
    bool fusable = with_slots != 0 && rows == n_items; // every item a single row
    fusable = fusable && all_distinct(pool, seq, n_items, pool->seq_max);
    const size_t cap = pool->seq_cap;
    fusable = fusable
        && !own_pages_clash(
            pool, pool->seq_host.data(), n_items,
            [&](size_t i) { return (uint32_t)(seq[i] * cap + first_position[i] / bs); },
            [&](size_t i) {
                return std::pair<uint32_t, uint32_t> {
                    (uint32_t)(seq[i] * cap), (uint32_t)(seq[i] * cap + first_position[i] / bs + 1)
                };
            });
    // the checks passed: from here the batch's host state and device metadata
    // are replaced, so until this batch is adopted launches report no tables
    pool->uploaded = false;
    std::vector<uint32_t>& positions = pool->positions;
    positions.resize(rows);
    pool->row_offsets.resize(rows);
    for (size_t i = 0, r = 0; i < n_items; ++i)
        for (uint32_t j = 0; j < token_count[i]; ++j, ++r) {
            positions[r] = first_position[i] + j;
            pool->row_offsets[r] = seq[i] * (uint32_t)pool->seq_cap; // the sequence's arena slot
        }
    const bool with_plan = !shared;
    const decode_plan_shape plan_shape = with_plan
        ? shape_decode_plan(positions, (uint32_t)bs, (uint32_t)pool->kv_heads, ctx->cu_count)
        : decode_plan_shape {};

    // d_meta: offsets | lengths | positions | slots (written by the expand
    // kernel) | pending (index, block) pairs | items (5 sections) | tiles | plan;
    // the upload starts at the pairs
    const size_t n_pairs = pool->dirty.size();
    const size_t s_offsets = 0;
    const size_t s_lengths = s_offsets + round4(rows);
    const size_t s_positions = s_lengths + round4(rows);
    const size_t s_slots = s_positions + round4(rows);
    const size_t s_pairs = s_slots + round4(rows);
    const size_t s_batch = s_pairs + round4(2 * n_pairs);
    const size_t s_tiles = s_batch + round4(5 * n_items);
    const size_t s_plan = s_tiles + round4(tiles.size());
    const size_t words = s_plan + (with_plan ? plan_words(plan_shape, rows) : 0);
    const size_t up_words = std::max<size_t>(words - s_pairs, 4);
    void* host = nullptr;
    int status = stage(ctx, up_words * sizeof(uint32_t), &host);
    if (status)
        return status;
    // staging holds d_meta[s_pairs, words)
    const auto section = [&](size_t at) { return static_cast<uint32_t*>(host) + (at - s_pairs); };
    uint32_t* pairs = section(s_pairs);
    for (size_t k = 0; k < n_pairs; ++k) {
        const uint32_t at = pool->dirty[k];
        pairs[2 * k] = at;
        pairs[2 * k + 1] = pool->seq_host[at];
    }
    uint32_t* b = section(s_batch);
    for (size_t i = 0, r = 0; i < n_items; ++i) {
        b[i] = seq[i];
        b[n_items + i] = first_position[i];
        b[2 * n_items + i] = token_count[i];
        b[3 * n_items + i] = (uint32_t)r;
        b[4 * n_items + i] = pool->seq_len[seq[i]];
        r += token_count[i];
    }
    if (!tiles.empty())
        std::memcpy(section(s_tiles), tiles.data(), tiles.size() * sizeof(uint32_t));
    status = ensure_device(ctx, &pool->d_meta, &pool->d_meta_words, s_pairs + up_words,
                           "metadata buffer");
    if (status)
        return status;
    uint32_t* d = pool->d_meta;
    if (with_plan)
        put_plan(pool, plan_shape, section(s_plan), d + s_plan);
    status = upload_staged(ctx, d + s_pairs, up_words * sizeof(uint32_t));
    if (status)
        return status;
    uint32_t* arena = pool->d_seq;
    if (n_pairs) {
        status = run_kernel(ctx, "tables_patch", [&] {
            return launch_table_patch(ctx->stream, arena, d + s_pairs, (uint32_t)n_pairs);
        });
        if (status)
            return status;
        // the entries are on their way: no longer pending (a failure before
        // this point leaves them pending for the next upload)
        for (size_t k = 0; k < n_pairs; ++k)
            pool->seq_dirty[pool->dirty[k]] = 0;
        pool->dirty.clear();
    }
    status = run_kernel(ctx, "batch_expand", [&] {
        return launch_expand_batch(ctx->stream, d + s_batch, (uint32_t)n_items, (uint32_t)rows,
                                   arena, (uint32_t)pool->seq_cap, (uint32_t)bs, with_slots != 0,
                                   d + s_offsets, d + s_lengths, d + s_positions, d + s_slots);
    });
    if (status)
        return status;

    meta_view& m = pool->meta;
    m.table = arena;
    m.offsets = d + s_offsets;
    m.lengths = d + s_lengths;
    m.positions = d + s_positions;
    m.slots = d + s_slots;
    m.tiles = d + s_tiles;
    m.n_tiles = (uint32_t)(tiles.size() / tile_entry_words);
    m.tile_blocks = shortest_tile_blocks(tiles);
    adopt_batch(pool, rows, pool->seq_max * pool->seq_cap, with_slots != 0, shared, fusable,
                with_plan, true);
    return CKV_OK;
}

int ckv_decode_plan(ckv_pool* pool, uint32_t* split_pages, uint32_t* work_items,
                    uint32_t* records)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    if (!pool->uploaded)
        return set_error(pool->ctx, CKV_E_NO_TABLES, "plan before ckv_tables_upload");
    const int status = ensure_plan(pool);
    if (status)
        return status;
    if (split_pages)
        *split_pages = pool->meta.split_pages;
    if (work_items)
        *work_items = pool->meta.n_segments;
    if (records)
        *records = pool->meta.n_records;
    return CKV_OK;
}

int ckv_append(ckv_pool* pool, size_t layer, const void* keys, const void* values, size_t rows)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if (rows && (!keys || !values))
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "keys and values are required");
    if (!pool->uploaded || !pool->has_slots)
        return set_error(ctx, CKV_E_NO_TABLES, "append before slots were uploaded");
    if (rows != pool->slot_rows)
        return set_error(ctx, CKV_E_CACHE_SLOT_COUNT_MISMATCH, "rows != uploaded slots");
    if (layer >= pool->layers)
        return set_error(ctx, CKV_E_CACHE_LAYER_OUT_OF_RANGE, "layer >= layers");
    const pool_view view = view_of(pool);
    return run_kernel(ctx, "store_kv", [&] {
        return launch_store_kv(ctx->stream, view, pool->meta, (uint32_t)layer, keys, values,
                               (uint32_t)rows);
    });
}

namespace {

// Host checks of rope (src/tensor/tensor_ops.cc:375-399) after the row count;
// fills the frequency table and the effective rotary width.
int check_rope(ckv_pool* pool, size_t heads, float theta, size_t rotary_dim,
               ckv::rope_table& freq, uint32_t& rotary)
{
    ckv_context* ctx = pool->ctx;
    if (heads == 0)
        return set_error(ctx, CKV_E_INVALID_HEAD_COUNT, "heads == 0");
    const size_t head_dim = pool->head_dim;
    if (rotary_dim == 0)
        rotary_dim = head_dim;
    if (head_dim % 2 != 0 || rotary_dim % 2 != 0 || rotary_dim > head_dim)
        return set_error(ctx, CKV_E_INVALID_HEAD_DIMENSION,
                         "head_dim and rotary_dim must be even, rotary_dim <= head_dim");
    // the kernels take the frequencies of at most max_rope_pairs pairs
    if (rotary_dim / 2 > ckv::max_rope_pairs)
        return set_error(ctx, CKV_E_INVALID_HEAD_DIMENSION,
                         "rotary_dim must be at most " + std::to_string(2 * ckv::max_rope_pairs));
    if (!std::isfinite(theta) || theta <= 0.0f)
        return set_error(ctx, CKV_E_INVALID_ROPE_THETA, "theta must be positive and finite");
    if ((uint64_t)heads * head_dim > UINT32_MAX)
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "row too wide");
    rotary = (uint32_t)rotary_dim;
    ckv::rope_frequencies(theta, rotary, freq);
    return CKV_OK;
}

} // namespace

int ckv_rope(ckv_pool* pool, const void* input, void* output, size_t heads, float theta,
             size_t rotary_dim, size_t rows)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if (rows && (!input || !output))
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "input and output are required");
    if (!pool->uploaded)
        return set_error(ctx, CKV_E_NO_TABLES, "rope before ckv_tables_upload");
    if (rows != pool->positions.size())
        return set_error(ctx, CKV_E_POSITION_COUNT_MISMATCH, "rows != uploaded positions");
    ckv::rope_table freq;
    uint32_t rotary = 0;
    if (const int status = check_rope(pool, heads, theta, rotary_dim, freq, rotary))
        return status;
    const pool_view view = view_of(pool);
    return run_kernel(ctx, "rope", [&] {
        return launch_rope(ctx->stream, view, pool->meta, input, output, (uint32_t)rows,
                           (uint32_t)heads, rotary, freq);
    });
}

int ckv_rope_append(ckv_pool* pool, size_t layer, const void* keys, const void* values,
                    float theta, size_t rotary_dim, size_t rows)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if (rows && (!keys || !values))
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "keys and values are required");
    if (!pool->uploaded || !pool->has_slots)
        return set_error(ctx, CKV_E_NO_TABLES, "append before slots were uploaded");
    if (rows != pool->slot_rows)
        return set_error(ctx, CKV_E_CACHE_SLOT_COUNT_MISMATCH, "rows != uploaded slots");
    if (layer >= pool->layers)
        return set_error(ctx, CKV_E_CACHE_LAYER_OUT_OF_RANGE, "layer >= layers");
    ckv::rope_table freq;
    uint32_t rotary = 0;
    if (const int status = check_rope(pool, pool->kv_heads, theta, rotary_dim, freq, rotary))
        return status;
    const pool_view view = view_of(pool);
    return run_kernel(ctx, "rope_append", [&] {
        return launch_rope_append(ctx->stream, view, pool->meta, (uint32_t)layer, keys, values,
                                  (uint32_t)rows, rotary, freq);
    });
}

int ckv_gather(ckv_pool* pool, size_t layer, size_t table_offset, size_t table_length,
               size_t n_tokens, void* out_keys, void* out_values)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if (n_tokens && (!out_keys || !out_values))
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "outputs are required");
    if (!pool->uploaded)
        return set_error(ctx, CKV_E_NO_TABLES, "gather before ckv_tables_upload");
    if (layer >= pool->layers)
        return set_error(ctx, CKV_E_CACHE_LAYER_OUT_OF_RANGE, "layer >= layers");
    if (table_offset > pool->n_entries || table_length > pool->n_entries - table_offset
        || n_tokens > table_length * pool->block_size)
        return set_error(ctx, CKV_E_BLOCK_TABLE_RANGE_OUT_OF_BOUNDS, "gather range");
    const pool_view view = view_of(pool);
    const uint32_t* table = pool->meta.table + table_offset;
    return run_kernel(ctx, "gather_kv", [&] {
        return launch_gather(ctx->stream, view, table, (uint32_t)layer, (uint32_t)n_tokens,
                             out_keys, out_values);
    });
}

namespace {

// The gate of the gated forms: [rows, q_heads * head_dim] of the pool dtype,
// not the queries' or the output's memory (the epilogue reads it while other
// workgroups still read queries).
int check_gate(const ckv_pool* pool, const void* gate, const void* queries, const void* output,
               size_t rows)
{
    if (rows && !gate)
        return set_error(pool->ctx, CKV_E_INVALID_ARGUMENT, "gate is required");
    if (gate && (gate == queries || gate == output))
        return set_error(pool->ctx, CKV_E_UNSUPPORTED_ALIASING, "gate overlaps queries or output");
    return CKV_OK;
}

int decode_impl(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads, float scale,
                void* output, size_t rows, const void* gate)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    const int status = check_attention(pool, layer, queries, q_heads, output, rows);
    if (status || !rows)
        return status;
    return run_decode(pool, layer, queries, q_heads, scale, output, gate);
}

int append_decode_impl(ckv_pool* pool, size_t layer, const void* keys, const void* values,
                       const void* queries, size_t q_heads, float scale, void* output,
                       size_t rows, const void* gate)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if (rows && (!keys || !values))
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "keys and values are required");
    if (!pool->uploaded || !pool->has_slots)
        return set_error(ctx, CKV_E_NO_TABLES, "append before slots were uploaded");
    if (rows != pool->slot_rows)
        return set_error(ctx, CKV_E_CACHE_SLOT_COUNT_MISMATCH, "rows != uploaded slots");
    int status = check_attention(pool, layer, queries, q_heads, output, rows);
    if (status || !rows)
        return status;
    const pool_view view = view_of(pool);
    const auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (pool->fusable && decode_fast_applies(view, (uint32_t)q_heads, queries, output)
        && aligned(keys) && aligned(values)) {
        split_scratch split {};
        status = ensure_plan(pool);
        if (!status)
            status = ensure_split(pool, q_heads, split);
        if (status)
            return status;
        return run_kernel(ctx, "append_decode", [&] {
            return launch_append_decode(ctx->stream, view, pool->meta, (uint32_t)layer, keys,
                                        values, queries, (uint32_t)q_heads, scale, output, gate,
                                        ctx->cu_count, split);
        });
    }
    status = ckv_append(pool, layer, keys, values, rows);
    if (status)
        return status;
    return run_decode(pool, layer, queries, q_heads, scale, output, gate);
}

int prefill_impl(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads, float scale,
                 void* output, size_t rows, const void* gate)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    const int status = check_attention(pool, layer, queries, q_heads, output, rows);
    if (status || !rows)
        return status;
    const pool_view view = view_of(pool);
    const auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    // the MFMA kernel tracks maxima of the unscaled scores, which needs scale > 0;
    // the decode kernels scale first and take any scale, one row at a time
    if (!prefill_supported(view, (uint32_t)q_heads, queries, output) || (gate && !aligned(gate))
        || !(scale > 0.0f))
        return run_decode(pool, layer, queries, q_heads, scale, output, gate);
    ckv_context* ctx = pool->ctx;
    const prefill_shape_info plan = prefill_plan(view, pool->meta, (uint32_t)q_heads, ctx->cu_count);
    prefill_split split { nullptr, nullptr, plan.n_split, plan.min_blocks };
    if (plan.n_split > 1) {
        int status = ensure_device(ctx, &pool->d_pre_records, &pool->d_pre_records_floats,
                                   (size_t)plan.records_floats, "prefill split records");
        if (status)
            return status;
        if (plan.counters > pool->d_pre_arrivals_words) {
            status = ensure_device(ctx, &pool->d_pre_arrivals, &pool->d_pre_arrivals_words,
                                   (size_t)plan.counters, "prefill split counters");
            if (status)
                return status;
            status = run_kernel(ctx, "fill", [&] {
                return launch_fill(ctx->stream, pool->d_pre_arrivals, 0,
                                   (uint32_t)pool->d_pre_arrivals_words);
            });
            if (status) {
                // not known to be zero: allocate and clear again next time
                (void)dev_free(ctx, pool->d_pre_arrivals);
                pool->d_pre_arrivals = nullptr;
                pool->d_pre_arrivals_words = 0;
                return status;
            }
        }
        split.records = pool->d_pre_records;
        split.arrivals = pool->d_pre_arrivals;
    }
    return run_kernel(ctx, "paged_attention_prefill", [&] {
        return launch_prefill(ctx->stream, view, pool->meta, (uint32_t)layer, queries,
                              (uint32_t)q_heads, scale, output, gate, plan, split);
    });
}

int attention_impl(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads, float scale,
                   void* output, size_t rows, const void* gate)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    // src/tensor/attention.cc:290-309: tiles are used when some run of rows
    // shares a query tile and head_dim <= 128
    if (pool->shared_tile && pool->head_dim <= 128)
        return prefill_impl(pool, layer, queries, q_heads, scale, output, rows, gate);
    return decode_impl(pool, layer, queries, q_heads, scale, output, rows, gate);
}

} // namespace

int ckv_decode_attention(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads,
                         float scale, void* output, size_t rows)
{
    return decode_impl(pool, layer, queries, q_heads, scale, output, rows, nullptr);
}

int ckv_append_decode(ckv_pool* pool, size_t layer, const void* keys, const void* values,
                      const void* queries, size_t q_heads, float scale, void* output, size_t rows)
{
    return append_decode_impl(pool, layer, keys, values, queries, q_heads, scale, output, rows,
                              nullptr);
}

int ckv_prefill_attention(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads,
                          float scale, void* output, size_t rows)
{
    return prefill_impl(pool, layer, queries, q_heads, scale, output, rows, nullptr);
}

int ckv_attention(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads,
                  float scale, void* output, size_t rows)
{
    return attention_impl(pool, layer, queries, q_heads, scale, output, rows, nullptr);
}

int ckv_attention_gated(ckv_pool* pool, size_t layer, const void* queries, size_t q_heads,
                        float scale, const void* gate, void* output, size_t rows)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    const int status = check_gate(pool, gate, queries, output, rows);
    if (status)
        return status;
    return attention_impl(pool, layer, queries, q_heads, scale, output, rows, gate);
}

int ckv_append_decode_gated(ckv_pool* pool, size_t layer, const void* keys, const void* values,
                            const void* queries, size_t q_heads, float scale, const void* gate,
                            void* output, size_t rows)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    const int status = check_gate(pool, gate, queries, output, rows);
    if (status)
        return status;
    return append_decode_impl(pool, layer, keys, values, queries, q_heads, scale, output, rows,
                              gate);
}

int ckv_rope_append_decode(ckv_pool* pool, size_t layer, const void* keys, const void* values,
                           const void* queries, size_t q_heads, float scale, float theta,
                           size_t rotary_dim, const void* gate, void* output, size_t rows)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if (rows && (!keys || !values))
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "keys and values are required");
    if (!pool->uploaded || !pool->has_slots)
        return set_error(ctx, CKV_E_NO_TABLES, "append before slots were uploaded");
    if (rows != pool->slot_rows)
        return set_error(ctx, CKV_E_CACHE_SLOT_COUNT_MISMATCH, "rows != uploaded slots");
    int status = check_attention(pool, layer, queries, q_heads, output, rows);
    if (status)
        return status;
    if (gate && (gate == queries || gate == output))
        return set_error(ctx, CKV_E_UNSUPPORTED_ALIASING, "gate overlaps queries or output");
    ckv::rope_table freq;
    uint32_t rotary = 0;
    status = check_rope(pool, q_heads, theta, rotary_dim, freq, rotary);
    if (status || !rows)
        return status;
    const pool_view view = view_of(pool);
    const auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    // the fused kernel rotates 16-bit pages in lane pairs part ^ (rotary / 16)
    // of a 128-wide head
    const bool lane_pairs = view.dtype != CKV_F32 && rotary >= 16 && rotary <= 128
        && (rotary & (rotary - 1)) == 0;
    if (pool->fusable && lane_pairs && decode_fast_applies(view, (uint32_t)q_heads, queries, output)
        && aligned(keys) && aligned(values) && (!gate || aligned(gate))) {
        split_scratch split {};
        status = ensure_plan(pool);
        if (!status)
            status = ensure_split(pool, q_heads, split);
        if (status)
            return status;
        return run_kernel(ctx, "rope_append_decode", [&] {
            return launch_append_decode(ctx->stream, view, pool->meta, (uint32_t)layer, keys,
                                        values, queries, (uint32_t)q_heads, scale, output, gate,
                                        ctx->cu_count, split, &freq, rotary);
        });
    }
    // unfused: queries rotated into a pool buffer, keys rotated into their
    // slots, then the attention over the rotated queries
    const size_t q_bytes = rows * q_heads * pool->head_dim * pool->elem_size;
    status = ensure_device(ctx, &pool->d_rope_q, &pool->d_rope_q_bytes, q_bytes, "rotated queries");
    if (status)
        return status;
    status = ckv_rope(pool, queries, pool->d_rope_q, q_heads, theta, rotary_dim, rows);
    if (status)
        return status;
    status = ckv_rope_append(pool, layer, keys, values, theta, rotary_dim, rows);
    if (status)
        return status;
    return run_decode(pool, layer, pool->d_rope_q, q_heads, scale, output, gate);
}

namespace {

// A status with a fixed detail text, stored in the context's reserved
// string: no allocation.
int fail_fixed(ckv_context* ctx, int code, const char* text)
{
    ctx->last_error.assign(text);
    return code;
}

} // namespace

int ckv_append_decode_noalloc(ckv_pool* pool, size_t layer, const void* keys, const void* values,
                              const void* queries, size_t q_heads, float scale, void* output,
                              size_t rows)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    // the checks of ckv_append_decode, in its order, with fixed texts
    if (rows && (!keys || !values))
        return fail_fixed(ctx, CKV_E_INVALID_ARGUMENT, "keys and values are required");
    if (!pool->uploaded || !pool->has_slots)
        return fail_fixed(ctx, CKV_E_NO_TABLES, "append before slots were uploaded");
    if (rows != pool->slot_rows)
        return fail_fixed(ctx, CKV_E_CACHE_SLOT_COUNT_MISMATCH, "rows != uploaded slots");
    if (rows && (!queries || !output))
        return fail_fixed(ctx, CKV_E_INVALID_ARGUMENT, "queries and output are required");
    if (rows != pool->positions.size())
        return fail_fixed(ctx, CKV_E_POSITION_COUNT_MISMATCH, "rows != uploaded positions");
    if (q_heads == 0)
        return fail_fixed(ctx, CKV_E_INVALID_HEAD_COUNT, "q_heads == 0");
    if (q_heads % pool->kv_heads != 0)
        return fail_fixed(ctx, CKV_E_INVALID_KV_HEAD_MAPPING, "q_heads % kv_heads != 0");
    if (layer >= pool->layers)
        return fail_fixed(ctx, CKV_E_CACHE_LAYER_OUT_OF_RANGE, "layer >= layers");
    if (!rows)
        return CKV_OK;
    // what only this entry point requires
    const pool_view view = view_of(pool);
    if (!decode_fast_applies(view, (uint32_t)q_heads, queries, output))
        return fail_fixed(ctx, CKV_E_INVALID_ARGUMENT,
                          "no-allocation decode: needs head_dim 128, 16-token pages, 1, 2, 4 "
                          "or 8 q heads per kv head and 16-byte aligned pools, queries and "
                          "output");
    // a batch of multi-row query tiles is refused whatever ran on it before
    // (a decode launch or ckv_decode_plan would have derived its plan)
    if (pool->shared_tile || !pool->plan_ready)
        return fail_fixed(ctx, CKV_E_INVALID_ARGUMENT,
                          "no-allocation decode: the batch has multi-row query tiles, so its "
                          "decode plan was not uploaded with it");
    const meta_view& m = pool->meta;
    const uint64_t need = (uint64_t)m.n_records * q_heads * partial_record_floats(128) * sizeof(float);
    const uint64_t counters = (uint64_t)m.n_records * pool->kv_heads * sizeof(uint32_t);
    if (need > noalloc_record_bytes || counters > noalloc_counter_bytes)
        return fail_fixed(ctx, CKV_E_INVALID_ARGUMENT,
                          "no-allocation decode: the batch's partial records exceed the "
                          "scratch (16 MiB less 256 KiB of counters; fewer or shorter rows "
                          "cut into chunks fit)");
    if (m.n_cut && !ctx->noalloc_scratch)
        return fail_fixed(ctx, CKV_E_HIP_FAILURE,
                          "no-allocation decode: the scratch array has no device address");
    unsigned char* const scratch = static_cast<unsigned char*>(ctx->noalloc_scratch);
    const split_scratch split { reinterpret_cast<float*>(scratch + noalloc_counter_bytes),
                                reinterpret_cast<uint32_t*>(scratch) };
    const bool fused = pool->fusable && reinterpret_cast<uintptr_t>(keys) % 16 == 0
        && reinterpret_cast<uintptr_t>(values) % 16 == 0;
    hipError_t e = hipSuccess;
    if (fused) {
        e = launch_append_decode(ctx->stream, view, m, (uint32_t)layer, keys, values, queries,
                                 (uint32_t)q_heads, scale, output, nullptr, ctx->cu_count, split);
    } else {
        e = launch_store_kv(ctx->stream, view, m, (uint32_t)layer, keys, values, (uint32_t)rows);
        if (e == hipSuccess)
            e = launch_decode(ctx->stream, view, m, (uint32_t)layer, queries, (uint32_t)q_heads,
                              scale, output, nullptr, ctx->cu_count, nullptr, split);
    }
    if (e != hipSuccess)
        return fail_fixed(ctx, CKV_E_HIP_FAILURE, hipGetErrorString(e));
    return CKV_OK;
}

int ckv_sigmoid_mul(ckv_context* ctx, int dtype, const void* gate, const void* input,
                    void* output, size_t count)
{
    if (!ctx)
        return CKV_E_INVALID_ARGUMENT;
    if (dtype != CKV_F32 && dtype != CKV_BF16 && dtype != CKV_F16)
        return set_error(ctx, CKV_E_UNSUPPORTED_DTYPE, "dtype");
    if (count && (!gate || !input || !output))
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "gate, input and output are required");
    return run_kernel(ctx, "sigmoid_mul", [&] {
        return launch_sigmoid_mul(ctx->stream, dtype, gate, input, output, count);
    });
}

int ckv_copy_blocks(ckv_pool* pool, const uint32_t* src, const uint32_t* dst, size_t n)
{
    if (!pool)
        return CKV_E_INVALID_ARGUMENT;
    ckv_context* ctx = pool->ctx;
    if (!n)
        return CKV_OK;
    if (!src || !dst)
        return set_error(ctx, CKV_E_INVALID_ARGUMENT, "block lists are required");
    std::unordered_set<uint32_t> targets, sources(src, src + n);
    for (size_t i = 0; i < n; ++i) {
        if (src[i] >= pool->blocks || dst[i] >= pool->blocks)
            return set_error(ctx, CKV_E_CACHE_BLOCK_OUT_OF_RANGE, "copy block id");
        if (!targets.insert(dst[i]).second || sources.count(dst[i]))
            return set_error(ctx, CKV_E_UNSUPPORTED_ALIASING, "copy targets overlap");
    }
    int status = stage_pairs(pool, src, dst, n);
    if (status)
        return status;
    const pool_view view = view_of(pool);
    return run_kernel(ctx, "copy_blocks", [&] {
        return launch_copy_blocks(ctx->stream, view, (uint32_t)pool->layers, pool->d_pairs,
                                  (uint32_t)n);
    });
}

int ckv_checkpoint_pack(ckv_pool* pool, const uint32_t* blocks, size_t n_blocks, size_t tokens,
                        void* packed_keys, void* packed_values)
{
    return run_checkpoint(pool, blocks, n_blocks, tokens, packed_keys, packed_values, false);
}

int ckv_checkpoint_unpack(ckv_pool* pool, const uint32_t* blocks, size_t n_blocks,
                          size_t tokens, const void* packed_keys, const void* packed_values)
{
    return run_checkpoint(pool, blocks, n_blocks, tokens, packed_keys, packed_values, true);
}

int ckv_checkpoint_export(ckv_pool* pool, const uint32_t* blocks, size_t n_blocks, size_t tokens,
                          void* host_keys, void* host_values)
{
    return run_transfer(pool, blocks, n_blocks, tokens, host_keys, host_values, false);
}

int ckv_checkpoint_import(ckv_pool* pool, const uint32_t* blocks, size_t n_blocks,
                          size_t tokens, const void* host_keys, const void* host_values)
{
    return run_transfer(pool, blocks, n_blocks, tokens, const_cast<void*>(host_keys),
                        const_cast<void*>(host_values), true);
}

} // extern "C"

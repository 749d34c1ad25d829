// GPU tests of the C++ host layer over libckv: the KV cache and tensor-op
// known answers of the reference (tests/metal_kv_cache_test.cc,
// tests/tensor_ops_test.cc), shared-prefix checkpoints with copy-on-write of
// the partial tail page, and engine runs on the device KV path in which a
// restored prefix must give the same attention as a cold prefill.
#include <algorithm>
#include <array>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <deque>
#include <numeric>
#include <unordered_map>

#include "check.h"
#include "hip_model_state.h"
#include "inference_engine.h"
#include "tensor_ops.h"

using namespace chibillm;

namespace {

hip_context&
gpu()
{
    static hip_context ctx = [] {
        auto c = hip_context::make(0);
        if (!c)
            throw std::runtime_error("no GPU context: " + describe_error(c.error()));
        return std::move(*c);
    }();
    return ctx;
}

device_buffer
upload(const void* host, std::size_t bytes)
{
    auto b = device_buffer::make(gpu(), bytes);
    REQUIRE(b);
    REQUIRE(b->upload(host, bytes));
    return std::move(*b);
}

template <typename T>
std::vector<T>
download(const device_buffer& b, std::size_t count)
{
    std::vector<T> out(count);
    REQUIRE(b.download(out.data(), count * sizeof(T)));
    return out;
}

template <typename T>
std::vector<T>
read_cache(const hip_kv_cache& c, void* ptr)
{
    std::vector<T> out(c.element_count());
    REQUIRE(ckv_copy_to_host(gpu().get(), out.data(), ptr, out.size() * sizeof(T)) == 0);
    return out;
}

template <typename T>
void
write_cache(const hip_kv_cache& c, void* ptr, const std::vector<T>& values)
{
    REQUIRE(values.size() == c.element_count());
    REQUIRE(ckv_copy_to_device(gpu().get(), ptr, values.data(), values.size() * sizeof(T)) == 0);
}

template <typename R, typename C>
bool
error_is(const R& r, C code)
{
    return !r.has_value() && r.error() == code;
}

std::uint16_t
to_bf16(float x)
{
    std::uint32_t b;
    std::memcpy(&b, &x, 4);
    b += 0x7FFFu + ((b >> 16) & 1u);
    return static_cast<std::uint16_t>(b >> 16);
}

float
from_bf16(std::uint16_t h)
{
    const std::uint32_t b = static_cast<std::uint32_t>(h) << 16;
    float x;
    std::memcpy(&x, &b, 4);
    return x;
}

device_tensor
view(const device_buffer& b, dtype t, std::vector<std::size_t> dims)
{
    return device_tensor { b.data(), t, std::move(dims) };
}

hip_kv_cache
make_cache(kv_cache_config c, kv_dtype t = kv_dtype::f32)
{
    auto cache = hip_kv_cache::make(gpu(), c, t);
    REQUIRE(cache);
    return std::move(*cache);
}

} // namespace

// ---- hip_kv_cache (tests/metal_kv_cache_test.cc) -----------------------------------

TEST("kv cache: allocates matching key and value tensors")
{
    auto c = make_cache({ 2, 3, 4, 2, 8 });
    CHECK(c.layer_count() == 2 && c.block_count() == 3 && c.block_size() == 4);
    CHECK(c.kv_head_count() == 2 && c.head_dimension() == 8);
    CHECK(c.elements_per_token() == 16 && c.elements_per_block() == 64);
    CHECK(c.elements_per_layer() == 192 && c.element_count() == 384);
    CHECK(c.keys() != nullptr && c.values() != nullptr && c.keys() != c.values());
}

TEST("kv cache: rejects zero and overflowing dimensions")
{
    const kv_cache_config good { 2, 3, 4, 2, 8 };
    auto bad = [&](auto edit, kv_cache_errc want) {
        auto c = good;
        edit(c);
        CHECK(error_is(hip_kv_cache::make(gpu(), c), want));
    };
    bad([](auto& c) { c.layer_count = 0; }, kv_cache_errc::invalid_layer_count);
    bad([](auto& c) { c.block_count = 0; }, kv_cache_errc::invalid_block_count);
    bad([](auto& c) { c.block_size = 0; }, kv_cache_errc::invalid_block_size);
    bad([](auto& c) { c.kv_head_count = 0; }, kv_cache_errc::invalid_kv_head_count);
    bad([](auto& c) { c.head_dimension = 0; }, kv_cache_errc::invalid_head_dimension);
    bad([](auto& c) { c.layer_count = std::numeric_limits<std::size_t>::max(); },
        kv_cache_errc::layout_size_overflow);
}

TEST("kv cache: flattens coordinates in layout order and rejects invalid coordinates")
{
    auto c = make_cache({ 2, 3, 4, 2, 8 });
    CHECK(*c.element_offset(0, 0, 0, 0, 0) == 0 && *c.element_offset(0, 0, 0, 0, 1) == 1);
    CHECK(*c.element_offset(0, 0, 0, 1, 0) == 8 && *c.element_offset(0, 0, 1, 0, 0) == 16);
    CHECK(*c.element_offset(0, 1, 0, 0, 0) == 64 && *c.element_offset(1, 0, 0, 0, 0) == 192);
    CHECK(*c.element_offset(1, 2, 3, 1, 7) == 383);
    CHECK(error_is(c.element_offset(2, 0, 0, 0, 0), kv_cache_errc::layer_out_of_range));
    CHECK(error_is(c.element_offset(0, 3, 0, 0, 0), kv_cache_errc::block_out_of_range));
    CHECK(error_is(c.element_offset(0, 0, 4, 0, 0), kv_cache_errc::token_offset_out_of_range));
    CHECK(error_is(c.element_offset(0, 0, 0, 2, 0), kv_cache_errc::kv_head_out_of_range));
    CHECK(error_is(c.element_offset(0, 0, 0, 0, 8), kv_cache_errc::head_feature_out_of_range));
}

TEST("kv cache: checkpoints remap fragmented pages and copy only the committed tail")
{
    auto c = make_cache({ 2, 3, 4, 2, 8 });
    std::vector<float> keys(c.element_count()), values(c.element_count());
    std::iota(keys.begin(), keys.end(), 1.0f);
    std::iota(values.begin(), values.end(), 1001.0f);
    write_cache(c, c.keys(), keys);
    write_cache(c, c.values(), values);
    const std::vector<block_id> source { 2, 0 }, target { 0, 1 };
    auto saved = c.checkpoint(source, 5);
    REQUIRE(saved);
    CHECK((*saved)->size_bytes() == c.checkpoint_bytes(5));
    const std::vector<float> zeros(c.element_count(), 0.0f);
    write_cache(c, c.keys(), zeros);
    write_cache(c, c.values(), zeros);
    REQUIRE(c.restore(target, **saved));
    const auto rk = read_cache<float>(c, c.keys());
    const auto rv = read_cache<float>(c, c.values());
    for (std::size_t layer = 0; layer < 2; ++layer)
        for (std::size_t token = 0; token < 8; ++token)
            for (std::size_t f = 0; f < 16; ++f) {
                const std::size_t dst = layer * 192 + token * 16 + f;
                const std::size_t src = layer * 192 + source[token / 4] * 64 + (token % 4) * 16 + f;
                CHECK(rk[dst] == (token < 5 ? keys[src] : 0.0f));
                CHECK(rv[dst] == (token < 5 ? values[src] : 0.0f));
            }
    CHECK_FALSE(c.checkpoint(std::vector<block_id> { 3 }, 1));
    CHECK_FALSE(c.checkpoint(source, 9));
}

// ---- tensor ops (tests/tensor_ops_test.cc) ---------------------------------------------

namespace {
kv_cache_config
tiny()
{
    return { 2, 2, 2, 1, 2 };
}
} // namespace

TEST("tensor ops: store writes rows into selected physical slots")
{
    auto c = make_cache(tiny());
    write_cache(c, c.keys(), std::vector<float>(16, -1.0f));
    write_cache(c, c.values(), std::vector<float>(16, -1.0f));
    const std::array<float, 4> k { 1, 2, 3, 4 }, v { 5, 6, 7, 8 };
    auto kb = upload(k.data(), 16), vb = upload(v.data(), 16);
    const std::vector<std::uint32_t> pos { 0, 0 }, slots { 1, 3 }, table { 0, 1 }, off { 0, 0 },
        len { 2, 2 };
    REQUIRE(upload_attention_metadata(c, { pos, slots, table, off, len }));
    REQUIRE(store_kv(c, view(kb, dtype::f32, { 2, 2 }), view(vb, dtype::f32, { 2, 2 }), 1));
    const auto rk = read_cache<float>(c, c.keys());
    const auto rv = read_cache<float>(c, c.values());
    const std::vector<float> want_k { -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, 1, 2, -1, -1, 3, 4 };
    const std::vector<float> want_v { -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, 5, 6, -1, -1, 7, 8 };
    CHECK(rk == want_k);
    CHECK(rv == want_v);
}

TEST("tensor ops: store validates inputs, shapes and slots")
{
    auto c = make_cache(tiny());
    auto b = device_buffer::make(gpu(), 64);
    REQUIRE(b);
    const std::vector<std::uint32_t> pos { 0, 0 }, slots { 0, 1 }, table { 0, 1 }, off { 0, 0 },
        len { 2, 2 };
    REQUIRE(upload_attention_metadata(c, { pos, slots, table, off, len }));
    auto t = [&](dtype type, std::vector<std::size_t> dims) { return view(*b, type, dims); };
    const auto keys = t(dtype::f32, { 2, 2 });
    CHECK(error_is(store_kv(c, t(dtype::f32, { 4 }), keys, 0), tensor_op_errc::invalid_rank));
    CHECK(error_is(store_kv(c, keys, t(dtype::f32, { 4 }), 0), tensor_op_errc::invalid_rank));
    CHECK(error_is(store_kv(c, t(dtype::bf16, { 2, 2 }), keys, 0), tensor_op_errc::unsupported_dtype));
    CHECK(error_is(store_kv(c, keys, t(dtype::bf16, { 2, 2 }), 0), tensor_op_errc::unsupported_dtype));
    CHECK(error_is(store_kv(c, keys, t(dtype::f32, { 1, 2 }), 0), tensor_op_errc::input_shape_mismatch));
    CHECK(error_is(store_kv(c, t(dtype::f32, { 1, 2 }), t(dtype::f32, { 1, 2 }), 0),
                   tensor_op_errc::cache_slot_count_mismatch));
    CHECK(error_is(store_kv(c, t(dtype::f32, { 2, 3 }), t(dtype::f32, { 2, 3 }), 0),
                   tensor_op_errc::cache_feature_count_mismatch));
    CHECK(error_is(store_kv(c, keys, keys, 2), tensor_op_errc::cache_layer_out_of_range));
    const std::vector<std::uint32_t> bad_slots { 0, 4 };
    CHECK(error_is(upload_attention_metadata(c, { pos, bad_slots, table, off, len }),
                   tensor_op_errc::cache_slot_out_of_range));
}

TEST("tensor ops: paged attention follows block tables and shares kv heads")
{
    auto c = make_cache(tiny());
    write_cache(c, c.keys(), std::vector<float> { 1, 1, 0, 0, 1, 0, 0, 1, 0, 0, 0, 0, 0, 0, 0, 0 });
    write_cache(c, c.values(), std::vector<float> { 30, 3, 0, 0, 10, 1, 20, 2, 0, 0, 0, 0, 0, 0, 0, 0 });
    const std::array<float, 4> q { 1, 0, 0, 1 };
    auto qb = upload(q.data(), 16);
    auto ob = device_buffer::make(gpu(), 16);
    REQUIRE(ob);
    const std::vector<std::uint32_t> pos { 2 }, table { 1, 0 }, off { 0 }, len { 2 };
    REQUIRE(upload_attention_metadata(c, { pos, {}, table, off, len }));
    auto out = view(*ob, dtype::f32, { 1, 4 });
    REQUIRE(paged_attention(c, view(qb, dtype::f32, { 1, 4 }), 0, 2, out));
    const float e = std::exp(1.0f / std::sqrt(2.0f));
    const float d = 2 * e + 1;
    const std::array<float, 4> want { (40 * e + 20) / d, (4 * e + 2) / d, (10 + 50 * e) / d,
                                      (1 + 5 * e) / d };
    const auto got = download<float>(*ob, 4);
    for (int i = 0; i < 4; ++i)
        CHECK(std::fabs(got[i] - want[i]) <= 1e-5f * std::fabs(want[i]));
}

TEST("tensor ops: paged attention validates inputs and metadata")
{
    auto c = make_cache(tiny());
    auto b = device_buffer::make(gpu(), 64);
    REQUIRE(b);
    auto t = [&](dtype type, std::vector<std::size_t> dims) { return view(*b, type, dims); };
    const std::vector<std::uint32_t> pos { 0 }, table { 0 }, off { 0 }, len { 1 };
    REQUIRE(upload_attention_metadata(c, { pos, {}, table, off, len }));
    auto q = t(dtype::f32, { 1, 2 });
    auto out = t(dtype::f32, { 1, 2 });
    auto rank1 = t(dtype::f32, { 2 });
    CHECK(error_is(paged_attention(c, rank1, 0, 1, out), tensor_op_errc::invalid_rank));
    auto i32 = t(dtype::i32, { 1, 2 });
    CHECK(error_is(paged_attention(c, i32, 0, 1, out), tensor_op_errc::unsupported_dtype));
    CHECK(error_is(paged_attention(c, q, 0, 0, out), tensor_op_errc::invalid_head_count));
    auto dim5 = t(dtype::f32, { 1, 5 });
    CHECK(error_is(paged_attention(c, dim5, 0, 2, dim5), tensor_op_errc::invalid_head_dimension));
    auto dim3 = t(dtype::f32, { 1, 3 });
    CHECK(error_is(paged_attention(c, dim3, 0, 1, dim3), tensor_op_errc::cache_head_dimension_mismatch));
    auto bad_out = t(dtype::f32, { 2, 1 });
    CHECK(error_is(paged_attention(c, q, 0, 1, bad_out), tensor_op_errc::output_shape_mismatch));
    CHECK(error_is(paged_attention(c, q, 2, 1, out), tensor_op_errc::cache_layer_out_of_range));
    auto q2 = t(dtype::f32, { 2, 2 });
    auto out2 = t(dtype::f32, { 2, 2 });
    CHECK(error_is(paged_attention(c, q2, 0, 1, out2), tensor_op_errc::position_count_mismatch));
    const std::vector<std::uint32_t> two { 0, 0 };
    CHECK(error_is(upload_attention_metadata(c, { pos, {}, table, two, len }),
                   tensor_op_errc::block_table_metadata_count_mismatch));
    auto gqa = make_cache({ 1, 1, 1, 2, 2 });
    REQUIRE(upload_attention_metadata(gqa, { pos, {}, table, off, len }));
    auto dim6 = t(dtype::f32, { 1, 6 });
    CHECK(error_is(paged_attention(gqa, dim6, 0, 3, dim6), tensor_op_errc::invalid_kv_head_mapping));
    // block table bounds and ids
    const std::vector<std::uint32_t> pos2 { 2 };
    CHECK(error_is(upload_attention_metadata(c, { pos2, {}, table, off, len }),
                   tensor_op_errc::block_table_range_out_of_bounds));
    const std::vector<std::uint32_t> t2 { 0, 1 }, off1 { 1 }, len2 { 2 };
    CHECK(error_is(upload_attention_metadata(c, { pos, {}, t2, off1, len2 }),
                   tensor_op_errc::block_table_range_out_of_bounds));
    const std::vector<std::uint32_t> bad_block { 2 };
    CHECK(error_is(upload_attention_metadata(c, { pos, {}, bad_block, off, len }),
                   tensor_op_errc::cache_block_out_of_range));
}

TEST("tensor ops: attention gates use sigmoid and apply in the attention epilogue")
{
    // tests/tensor_ops_test.cc:513-539: sigmoid_mul of the gate {0, 1, -1, 2, -1000, 1000, 0, -2}
    // on {1..8}, in place
    auto c = make_cache(tiny());
    const std::array<float, 8> g { 0, 1, -1, 2, -1000, 1000, 0, -2 };
    const std::array<float, 8> x { 1, 2, 3, 4, 5, 6, 7, 8 };
    auto gb = upload(g.data(), 32), xb = upload(x.data(), 32);
    auto xv = view(xb, dtype::f32, { 2, 4 });
    REQUIRE(sigmoid_mul(c, view(gb, dtype::f32, { 2, 4 }), xv, xv));
    const auto got = download<float>(xb, 8);
    const std::array<float, 8> want { 0.5f, 2 / (1 + std::exp(-1.0f)), 3 / (1 + std::exp(1.0f)),
                                      4 / (1 + std::exp(-2.0f)), 0.0f, 6.0f, 3.5f,
                                      8 / (1 + std::exp(2.0f)) };
    for (int i = 0; i < 8; ++i)
        CHECK(std::fabs(got[i] - want[i]) <= 1e-5f * std::fabs(want[i]));
    CHECK(got[4] == 0.0f && got[5] == 6.0f);
    auto packed = view(gb, dtype::f32, { 1, 8 });
    CHECK(error_is(sigmoid_mul(c, packed, xv, xv), tensor_op_errc::input_shape_mismatch));
    auto short_out = view(xb, dtype::f32, { 1, 4 });
    CHECK(error_is(sigmoid_mul(c, view(gb, dtype::f32, { 2, 4 }), xv, short_out),
                   tensor_op_errc::output_shape_mismatch));
    CHECK(error_is(sigmoid_mul(c, view(gb, dtype::bf16, { 2, 4 }), xv, xv),
                   tensor_op_errc::unsupported_dtype));

    // the gated attention of the known answer above: output * sigmoid(gate)
    write_cache(c, c.keys(), std::vector<float> { 1, 1, 0, 0, 1, 0, 0, 1, 0, 0, 0, 0, 0, 0, 0, 0 });
    write_cache(c, c.values(), std::vector<float> { 30, 3, 0, 0, 10, 1, 20, 2, 0, 0, 0, 0, 0, 0, 0, 0 });
    const std::array<float, 4> q { 1, 0, 0, 1 }, gate { 0, 1, -1, 1000 };
    auto qb = upload(q.data(), 16), gateb = upload(gate.data(), 16);
    auto ob = device_buffer::make(gpu(), 16);
    REQUIRE(ob);
    const std::vector<std::uint32_t> pos { 2 }, table { 1, 0 }, off { 0 }, len { 2 };
    REQUIRE(upload_attention_metadata(c, { pos, {}, table, off, len }));
    auto out = view(*ob, dtype::f32, { 1, 4 });
    REQUIRE(paged_attention_gated(c, view(qb, dtype::f32, { 1, 4 }),
                                  view(gateb, dtype::f32, { 1, 4 }), 0, 2, out));
    const float e = std::exp(1.0f / std::sqrt(2.0f));
    const float d = 2 * e + 1;
    const std::array<float, 4> plain { (40 * e + 20) / d, (4 * e + 2) / d, (10 + 50 * e) / d,
                                       (1 + 5 * e) / d };
    const auto o = download<float>(*ob, 4);
    for (int i = 0; i < 4; ++i) {
        const float w = plain[i] / (1 + std::exp(-gate[i]));
        CHECK(std::fabs(o[i] - w) <= 1e-5f * std::fabs(w));
    }
    CHECK(error_is(paged_attention_gated(c, view(qb, dtype::f32, { 1, 4 }),
                                         view(gateb, dtype::f32, { 1, 2 }), 0, 2, out),
                   tensor_op_errc::input_shape_mismatch));
}

// ---- shared prefixes on the device --------------------------------------------------------

namespace {

constexpr kv_cache_config shared_geometry { 3, 32, 16, 2, 128 };

// Deterministic bf16 K/V row of (sequence token, position) so that equal
// prefixes write equal bytes.
std::vector<std::uint16_t>
kv_rows(std::span<const token_id> tokens, std::span<const position_id> positions,
        std::size_t features, std::uint32_t salt)
{
    std::vector<std::uint16_t> rows(tokens.size() * features);
    for (std::size_t r = 0; r < tokens.size(); ++r) {
        std::uint32_t h = static_cast<std::uint32_t>(tokens[r]) * 2654435761u ^ positions[r] * 40503u
            ^ salt * 97u;
        for (std::size_t f = 0; f < features; ++f) {
            h ^= h << 13;
            h ^= h >> 17;
            h ^= h << 5;
            rows[r * features + f] = to_bf16(static_cast<float>(h % 2001) / 1000.0f - 1.0f);
        }
    }
    return rows;
}

// A model stand-in that runs the real device KV path: per batch it uploads
// prepare_paged_batch's metadata, writes each token's K/V row for every
// layer through store_kv and attends with paged_attention; it keeps the
// attention output of each sampled row and samples a fixed token.
struct kv_path_runner final : model_runner {
    mutable hip_model_state* state = nullptr;
    prefix_sharing sharing = prefix_sharing::shared_pages;
    std::unordered_map<seq_id, std::vector<std::vector<float>>> outputs; // per sample
    std::size_t prefill_tokens = 0;
    bool device_tables = false; // tables kept on the device instead of prepare_paged_batch

    const model_info& info() const noexcept override
    {
        static const model_info value { "kv-path", 512, -1 };
        return value;
    }
    result<std::unique_ptr<model_state>, model_runner_error> make_state(
        scheduler_config config) const override
    {
        auto s = hip_model_state::make(gpu(), shared_geometry, kv_dtype::bf16, sharing);
        if (!s)
            return fail(model_runner_errc::backend_failure, s.error());
        state = s->get();
        if (device_tables) {
            auto on = state->enable_device_tables(config.max_sequences, 512 / 16);
            if (!on)
                return fail(model_runner_errc::backend_failure, on.error());
        }
        return std::unique_ptr<model_state>(std::move(*s));
    }
    result<std::vector<token_id>, model_runner_error> execute(const model_batch& batch,
                                                              model_state&) override
    {
        auto& cache = state->cache();
        const std::size_t F = cache.elements_per_token();
        const std::size_t qf = 4 * cache.head_dimension(); // 4 q heads over 2 KV heads
        if (batch.phase == batch_phase::prefill)
            prefill_tokens += batch.tokens.size();
        const std::size_t rows = batch.tokens.size();
        if (device_tables) {
            auto up = state->tables()->upload(batch, 512, true);
            if (!up)
                return fail(model_runner_errc::backend_failure, up.error());
        } else {
            auto md = prepare_paged_batch(batch, 512, cache.block_count(), cache.block_size());
            if (!md)
                return fail(model_runner_errc::inconsistent_batch, md.error());
            std::vector<std::uint32_t> positions(batch.positions.begin(), batch.positions.end());
            auto up = upload_attention_metadata(cache, { positions, md->slots, md->block_table,
                                                         md->table_offsets, md->table_lengths });
            if (!up)
                return fail(model_runner_errc::backend_failure, up.error());
        }
        auto out = device_buffer::make(gpu(), rows * qf * 2);
        if (!out)
            return fail(model_runner_errc::backend_failure, out.error());
        std::vector<float> last_out;
        for (std::size_t layer = 0; layer < cache.layer_count(); ++layer) {
            const auto k = kv_rows(batch.tokens, batch.positions, F, 1 + layer * 2);
            const auto v = kv_rows(batch.tokens, batch.positions, F, 2 + layer * 2);
            const auto q = kv_rows(batch.tokens, batch.positions, qf, 100 + layer);
            auto kb = upload(k.data(), k.size() * 2), vb = upload(v.data(), v.size() * 2);
            auto qb = upload(q.data(), q.size() * 2);
            auto stored = store_kv(cache, view(kb, dtype::bf16, { rows, F }),
                                   view(vb, dtype::bf16, { rows, F }), layer);
            if (!stored)
                return fail(model_runner_errc::backend_failure, stored.error());
            auto o = view(*out, dtype::bf16, { rows, qf });
            auto attended = paged_attention(cache, view(qb, dtype::bf16, { rows, qf }), layer, 4, o);
            if (!attended)
                return fail(model_runner_errc::backend_failure, attended.error());
        }
        const auto bits = download<std::uint16_t>(*out, rows * qf);
        std::vector<token_id> samples;
        for (const auto& item : batch.items) {
            if (!item.logits_index)
                continue;
            std::vector<float> row(qf);
            for (std::size_t f = 0; f < qf; ++f)
                row[f] = from_bf16(bits[*item.logits_index * qf + f]);
            outputs[item.id].push_back(std::move(row));
            samples.push_back(7);
        }
        return samples;
    }
};

scheduler_config
shared_config()
{
    scheduler_config c;
    c.max_sequences = 4;
    c.max_batch_tokens = 256;
    c.kv_block_count = shared_geometry.block_count;
    c.kv_block_size = 16;
    c.prefill_chunk_tokens = 256;
    c.prefix_cache_bytes = 64ull << 20;
    c.prefix_cache_min_tokens = 8;
    return c;
}

std::vector<token_id>
prompt_of(std::size_t length, token_id first)
{
    std::vector<token_id> p(length);
    std::iota(p.begin(), p.end(), first);
    return p;
}

void
run_all(inference_engine& engine)
{
    while (!engine.is_finished()) {
        auto stepped = engine.step();
        REQUIRE(stepped);
    }
}

bool
close_rows(const std::vector<std::vector<float>>& a, const std::vector<std::vector<float>>& b)
{
    if (a.size() != b.size())
        return false;
    for (std::size_t i = 0; i < a.size(); ++i)
        for (std::size_t f = 0; f < a[i].size(); ++f)
            if (std::fabs(a[i][f] - b[i][f]) > 2e-2f + 1e-2f * std::fabs(b[i][f]))
                return false;
    return true;
}

} // namespace

TEST("shared prefix: a restored prefix attends like a cold prefill and copies only its tail")
{
    for (std::size_t prefix : { 40, 48 }) { // a partial tail page, then an exact page boundary
        for (auto sharing : { prefix_sharing::shared_pages, prefix_sharing::packed_copy,
                              prefix_sharing::host_copy }) {
            kv_path_runner warm;
            warm.sharing = sharing;
            auto engine = inference_engine::make(shared_config(), warm);
            REQUIRE(engine);
            auto base = prompt_of(prefix + 5, 1000);
            auto first = seq::make(1, base, generation_params { 3 }, { prefix });
            REQUIRE(first);
            REQUIRE(engine->add(std::move(*first)));
            run_all(*engine);
            CHECK(engine->engine_scheduler().prefixes().entry_count() == 1);
            // two branches of the cached prefix
            for (seq_id id : { 2, 3 }) {
                auto p = prompt_of(prefix, 1000);
                for (int i = 0; i < 7; ++i)
                    p.push_back(static_cast<token_id>(5000 + id * 10 + i));
                auto s = seq::make(id, p, generation_params { 3 }, { prefix });
                REQUIRE(s);
                REQUIRE(engine->add(std::move(*s)));
                CHECK(engine->find_sequence(id)->cached_token_count() == prefix);
            }
            const std::size_t prefill_before = warm.prefill_tokens;
            run_all(*engine);
            CHECK(warm.prefill_tokens - prefill_before == 14); // only the suffixes ran
            if (sharing == prefix_sharing::shared_pages)
                CHECK(warm.state->cow_copies() == (prefix % 16 ? 2u : 0u));

            kv_path_runner cold;
            auto cold_config = shared_config();
            cold_config.prefix_cache_bytes = 0;
            auto reference = inference_engine::make(cold_config, cold);
            REQUIRE(reference);
            for (seq_id id : { 2, 3 }) {
                auto p = prompt_of(prefix, 1000);
                for (int i = 0; i < 7; ++i)
                    p.push_back(static_cast<token_id>(5000 + id * 10 + i));
                auto s = seq::make(id, p, generation_params { 3 });
                REQUIRE(s);
                REQUIRE(reference->add(std::move(*s)));
            }
            run_all(*reference);
            for (seq_id id : { 2, 3 })
                CHECK(close_rows(warm.outputs[id], cold.outputs[id]));
        }
    }
}

TEST("device tables: an engine run over device-resident tables equals the host-uploaded run")
{
    // shared prefixes (page sharing + copy-on-write tails), several live
    // sequences with ragged prompts, rows reused after sequences finish
    std::unordered_map<seq_id, std::vector<std::vector<float>>> runs[2];
    std::size_t live_rows = 0;
    for (int mode = 0; mode < 2; ++mode) {
        kv_path_runner runner;
        runner.device_tables = mode == 1;
        auto engine = inference_engine::make(shared_config(), runner);
        REQUIRE(engine);
        auto base = seq::make(1, prompt_of(45, 1000), generation_params { 4 }, { 40 });
        REQUIRE(base);
        REQUIRE(engine->add(std::move(*base)));
        run_all(*engine);
        const std::size_t lengths[] = { 47, 9, 130, 61, 23 };
        std::deque<seq> pending;
        for (seq_id id = 2; id < 7; ++id) {
            auto p = prompt_of(lengths[id - 2], id < 4 ? 1000 : 3000 + 200 * id);
            std::vector<std::size_t> marks; // a prefix checkpoint where the prompt has one
            if (p.size() > 40)
                marks.push_back(40);
            auto s = seq::make(id, p, generation_params { 3 + id % 3 }, marks);
            REQUIRE(s);
            pending.push_back(std::move(*s));
        }
        // admitted as pages free up: later sequences take finished ones' rows
        while (!pending.empty() || !engine->is_finished()) {
            while (!pending.empty()) {
                auto r = engine->try_add(pending.front());
                REQUIRE(r);
                if (*r == admission_result::deferred)
                    break;
                REQUIRE(*r == admission_result::admitted);
                pending.pop_front();
            }
            if (!engine->is_finished())
                REQUIRE(engine->step());
        }
        if (mode == 1)
            live_rows = runner.state->tables()->live_sequences();
        runs[mode] = runner.outputs;
    }
    CHECK(live_rows == 0); // every finished sequence gave its row back
    REQUIRE(runs[0].size() == 6 && runs[1].size() == 6);
    for (const auto& [id, rows] : runs[0]) {
        REQUIRE(runs[1].count(id) == 1);
        CHECK(runs[1][id] == rows); // bit-exact: same kernels, same metadata
    }
}

TEST("shared prefix: refcounts keep shared pages until the last holder lets go")
{
    auto made = hip_model_state::make(gpu(), shared_geometry, kv_dtype::bf16);
    REQUIRE(made);
    auto& state = **made;
    const auto& pages = state.pages();
    REQUIRE(state.reserve(1, 40)); // 3 pages
    auto cp = state.checkpoint(1, 40);
    REQUIRE(cp);
    CHECK((*cp)->size_bytes() == 3 * state.cache().page_bytes_all_layers());
    const auto owned = state.resources(1).blocks;
    const std::vector<block_id> first(owned.begin(), owned.end());
    for (block_id b : first)
        CHECK(pages.refcount(b) == 2);
    REQUIRE(state.reserve(2, 1));
    REQUIRE(state.restore(2, **cp));
    const auto t2 = state.resources(2).blocks;
    REQUIRE(t2.size() == 3);
    CHECK(t2[0] == first[0] && t2[1] == first[1] && t2[2] != first[2]);
    CHECK(pages.refcount(first[0]) == 3 && pages.refcount(first[2]) == 2);
    CHECK(state.cow_copies() == 1);
    state.release(1);
    CHECK(pages.refcount(first[0]) == 2 && pages.refcount(first[2]) == 1);
    cp->reset(); // the checkpoint lets go
    CHECK(pages.refcount(first[0]) == 1 && pages.refcount(first[2]) == 0);
    state.release(2);
    CHECK(pages.free_block_count() == pages.block_count());
    // a restore needs a fresh one-page reservation
    REQUIRE(state.reserve(3, 40));
    auto cp3 = state.checkpoint(3, 16);
    REQUIRE(cp3);
    REQUIRE(state.reserve(4, 20));
    CHECK(error_is(state.restore(4, **cp3), state_errc::invalid_reservation));
}

TEST("shared prefix: the copy-on-write tail page equals its source bit for bit")
{
    auto made = hip_model_state::make(gpu(), shared_geometry, kv_dtype::bf16);
    REQUIRE(made);
    auto& state = **made;
    auto& cache = state.cache();
    std::vector<std::uint16_t> k(cache.element_count()), v(cache.element_count());
    for (std::size_t i = 0; i < k.size(); ++i) {
        k[i] = static_cast<std::uint16_t>(i * 7919u);
        v[i] = static_cast<std::uint16_t>(i * 104729u);
    }
    write_cache(cache, cache.keys(), k);
    write_cache(cache, cache.values(), v);
    REQUIRE(state.reserve(1, 21)); // pages 0, 1
    auto cp = state.checkpoint(1, 21);
    REQUIRE(cp);
    REQUIRE(state.reserve(2, 1));
    const block_id own = state.resources(2).blocks[0];
    REQUIRE(state.restore(2, **cp));
    const auto rk = read_cache<std::uint16_t>(cache, cache.keys());
    const auto rv = read_cache<std::uint16_t>(cache, cache.values());
    const std::size_t per_page = cache.elements_per_block();
    const block_id tail = state.resources(1).blocks[1];
    for (std::size_t layer = 0; layer < cache.layer_count(); ++layer) {
        const std::size_t base = layer * cache.elements_per_layer();
        CHECK(std::equal(rk.begin() + base + own * per_page, rk.begin() + base + (own + 1) * per_page,
                         k.begin() + base + tail * per_page));
        CHECK(std::equal(rv.begin() + base + own * per_page, rv.begin() + base + (own + 1) * per_page,
                         v.begin() + base + tail * per_page));
    }
    // nothing else changed
    std::size_t changed = 0;
    for (std::size_t i = 0; i < rk.size(); ++i)
        changed += rk[i] != k[i];
    CHECK(changed <= cache.layer_count() * per_page);
}

TEST("spill: an exhausted pool moves a lone prefix checkpoint to host memory and restores it")
{
    auto made = hip_model_state::make(gpu(), shared_geometry, kv_dtype::bf16);
    REQUIRE(made);
    auto& state = **made;
    auto& cache = state.cache();
    std::vector<std::uint16_t> k(cache.element_count()), v(cache.element_count());
    for (std::size_t i = 0; i < k.size(); ++i) {
        k[i] = static_cast<std::uint16_t>(i * 7919u + 3);
        v[i] = static_cast<std::uint16_t>(i * 104729u + 5);
    }
    write_cache(cache, cache.keys(), k);
    write_cache(cache, cache.values(), v);
    REQUIRE(state.reserve(1, 40)); // 3 pages
    const auto first = state.resources(1).blocks;
    const std::vector<block_id> held(first.begin(), first.end());
    auto cp = state.checkpoint(1, 40);
    REQUIRE(cp);
    state.release(1); // the checkpoint alone holds the 3 pages
    // the whole pool for one sequence: the checkpoint must leave
    REQUIRE(state.reserve(2, 32 * 16));
    CHECK(state.spills() == 1);
    CHECK(state.spilled_pages() == 3);
    CHECK(state.pages().free_block_count() == 0);
    // the pages are reused and overwritten
    std::vector<std::uint16_t> junk(cache.element_count(), 0x7F80);
    write_cache(cache, cache.keys(), junk);
    write_cache(cache, cache.values(), junk);
    state.release(2);
    REQUIRE(state.reserve(3, 1));
    REQUIRE(state.restore(3, **cp)); // copied in from host memory
    const auto own = state.resources(3).blocks;
    REQUIRE(own.size() == 3);
    const auto rk = read_cache<std::uint16_t>(cache, cache.keys());
    const auto rv = read_cache<std::uint16_t>(cache, cache.values());
    const std::size_t per_token = cache.elements_per_token();
    const std::size_t per_page = cache.elements_per_block();
    std::size_t mismatches = 0;
    for (std::size_t layer = 0; layer < cache.layer_count(); ++layer) {
        const std::size_t base = layer * cache.elements_per_layer();
        for (std::size_t t = 0; t < 40; ++t) {
            const std::size_t to = base + own[t / 16] * per_page + (t % 16) * per_token;
            const std::size_t from = base + held[t / 16] * per_page + (t % 16) * per_token;
            mismatches += !std::equal(rk.begin() + to, rk.begin() + to + per_token,
                                      k.begin() + from);
            mismatches += !std::equal(rv.begin() + to, rv.begin() + to + per_token,
                                      v.begin() + from);
        }
    }
    CHECK(mismatches == 0);
}

TEST("spill: a sequence that needs the pool spills a cached prefix; a later hit restores it")
{
    std::unordered_map<seq_id, std::vector<std::vector<float>>> outputs[2];
    std::size_t spills = 0, spilled_pages = 0;
    for (int cold = 0; cold < 2; ++cold) {
        kv_path_runner runner;
        auto config = shared_config();
        if (cold)
            config.prefix_cache_bytes = 0;
        auto engine = inference_engine::make(config, runner);
        REQUIRE(engine);
        if (!cold) { // caches a 40-token prefix, which then holds 3 pages alone
            auto first = seq::make(1, prompt_of(45, 1000), generation_params { 2 }, { 40 });
            REQUIRE(first);
            REQUIRE(engine->add(std::move(*first)));
            run_all(*engine);
            REQUIRE(engine->engine_scheduler().prefixes().entry_count() == 1);
            CHECK(runner.state->pages().free_block_count() == 29);
        }
        // 30 pages of budget: only fits once the prefix's pages are spilled
        auto big = seq::make(2, prompt_of(470, 9000), generation_params { 3 });
        REQUIRE(big);
        REQUIRE(engine->add(std::move(*big)));
        run_all(*engine);
        auto p = prompt_of(40, 1000);
        for (int i = 0; i < 9; ++i)
            p.push_back(static_cast<token_id>(7000 + i));
        auto hit = seq::make(3, p, generation_params { 3 }, { 40 });
        REQUIRE(hit);
        REQUIRE(engine->add(std::move(*hit)));
        if (!cold)
            CHECK(engine->find_sequence(3)->cached_token_count() == 40);
        run_all(*engine);
        if (!cold) {
            spills = runner.state->spills();
            spilled_pages = runner.state->spilled_pages();
        }
        outputs[cold] = runner.outputs;
    }
    // the 40-token prefix (3 pages) makes room for sequence 2; sequence 2's
    // own prompt checkpoint (469 tokens, 30 pages, the default boundary)
    // then makes room for sequence 3's restore
    CHECK(spills == 2);
    CHECK(spilled_pages == 33);
    for (seq_id id : { 2, 3 })
        CHECK(close_rows(outputs[0][id], outputs[1][id]));
}

// tests/qwen3_5_model_state_test.cc:329-417 without the DeltaNet layers: two-token batches over
// two-token pages; every attempted batch writes K = V = position + 1 for its rows at every layer
// through store_kv. After an abort, every committed position still holds its value, and the
// retried batch rewrites the same slots.
TEST("transactions: an aborted append never overwrites the committed KV prefix")
{
    auto made = hip_model_state::make(gpu(), kv_cache_config { 2, 8, 2, 1, 2 }, kv_dtype::f32,
                                      prefix_sharing::shared_pages);
    REQUIRE(made);
    hip_model_state* state = made->get();
    auto& cache = state->cache();
    write_cache(cache, cache.keys(), std::vector<float>(cache.element_count(), 0.0f));
    write_cache(cache, cache.values(), std::vector<float>(cache.element_count(), 0.0f));
    scheduler_config config;
    config.max_sequences = 2;
    config.max_batch_tokens = 2;
    config.kv_block_count = 8;
    config.kv_block_size = 2;
    auto engine = scheduler::make(config, 99, std::move(*made));
    REQUIRE(engine);
    auto sequence = seq::make(1, { 1, 2, 3 }, { .max_new_tokens = 2 });
    REQUIRE(sequence);
    REQUIRE(engine->add(std::move(*sequence)));

    const auto execute = [&](const model_batch& batch) {
        auto md = prepare_paged_batch(batch, 512, cache.block_count(), cache.block_size());
        REQUIRE(md);
        const std::vector<std::uint32_t> positions(batch.positions.begin(), batch.positions.end());
        REQUIRE(upload_attention_metadata(cache, { positions, md->slots, md->block_table,
                                                   md->table_offsets, md->table_lengths }));
        const std::size_t rows = batch.tokens.size();
        std::vector<float> rows_kv(rows * 2);
        for (std::size_t r = 0; r < rows; ++r)
            rows_kv[2 * r] = rows_kv[2 * r + 1] = float(batch.positions[r] + 1);
        auto kb = upload(rows_kv.data(), rows_kv.size() * 4);
        auto vb = upload(rows_kv.data(), rows_kv.size() * 4);
        for (std::size_t layer = 0; layer < 2; ++layer)
            REQUIRE(store_kv(cache, view(kb, dtype::f32, { rows, 2 }), view(vb, dtype::f32, { rows, 2 }),
                             layer));
    };
    const auto committed_prefix_intact = [&](std::size_t committed) {
        const auto keys = read_cache<float>(cache, cache.keys());
        const auto values = read_cache<float>(cache, cache.values());
        const auto table = state->resources(1).blocks;
        for (std::size_t layer = 0; layer < 2; ++layer)
            for (std::size_t pos = 0; pos < committed; ++pos)
                for (std::size_t f = 0; f < 2; ++f) {
                    const auto offset = cache.element_offset(layer, table[pos / 2], pos % 2, 0, f);
                    REQUIRE(offset);
                    CHECK(keys[*offset] == float(pos + 1));
                    CHECK(values[*offset] == float(pos + 1));
                }
    };

    // a partial prefill, aborted, then retried and committed
    auto scheduled = engine->schedule();
    REQUIRE(scheduled);
    auto batch = build_model_batch(*scheduled, *engine);
    REQUIRE(batch);
    REQUIRE(engine->begin_execution(*batch));
    execute(*batch);
    REQUIRE(engine->abort(scheduled->id));
    CHECK(engine->find_sequence(1)->processed_token_count() == 0);
    scheduled = engine->schedule();
    REQUIRE(scheduled);
    batch = build_model_batch(*scheduled, *engine);
    REQUIRE(batch);
    REQUIRE(engine->begin_execution(*batch));
    execute(*batch);
    REQUIRE(engine->complete(scheduled->id, {}));
    CHECK(engine->find_sequence(1)->processed_token_count() == 2);
    committed_prefix_intact(2);

    // the rest of the prefill, then one decode; each attempted once and aborted first
    for (int step = 0; step < 2; ++step) {
        scheduled = engine->schedule();
        REQUIRE(scheduled);
        batch = build_model_batch(*scheduled, *engine);
        REQUIRE(batch);
        const std::size_t committed = engine->find_sequence(1)->processed_token_count();
        REQUIRE(engine->begin_execution(*batch));
        execute(*batch);
        REQUIRE(engine->abort(scheduled->id));
        CHECK(engine->find_sequence(1)->processed_token_count() == committed);
        committed_prefix_intact(committed);
        scheduled = engine->schedule();
        REQUIRE(scheduled);
        batch = build_model_batch(*scheduled, *engine);
        REQUIRE(batch);
        REQUIRE(engine->begin_execution(*batch));
        execute(*batch);
        const std::vector<token_id> samples { 42 };
        REQUIRE(engine->complete(scheduled->id, samples));
    }
    // the sequence has finished: its pages are released
    CHECK(engine->state().resources(1).blocks.empty());
}

// Continuous-batching churn trace on the device KV path (the config-5
// workload): seeded Poisson arrivals, lognormal prompt and output lengths,
// the C++ scheduler and refcounted page allocator over a large device pool,
// and every engine step running the KV path for all layers: the batch's
// metadata uploaded once (tables mirrored on the device), then per layer the
// append of every row plus paged attention (prefill tiles on the matrix
// cores for prefill batches; the fused append + decode kernel for decode
// batches). K/V/Q rows are synthetic bf16 N(0,1) values resident in HBM: each
// layer has its own rows (twice the batch cap, drawn once from a counter-based
// generator), and each step takes its rows from a window at a seeded offset, so
// every layer and step appends and attends different values and any appended
// row can be regenerated on the host.
//
// Prints one JSON line: steps/s, tokens/s (prefill + decode rows), and the
// algorithmic HBM bytes of the path per second against the 8 TB/s peak.
//
// --check <dir> checks the trace as it runs and stops at the first failure
// (exit status 3): every --check-every steps, the page accounting (each live
// sequence's pages are held once, reference counts sum to the pages in tables,
// free + used = pool) and the K/V of sampled sequences, packed back from the
// pool for all layers, against the rows the trace appended for them; and at
// the first decode step and the first prefill step after --dump-after, the
// K/V (regenerated on the host from the rows the trace appended), queries and
// outputs of layers 0 and L - 1 are written to <dir> for a CPU check of the
// attention: up to eight decode rows (decode_rows.json) and one prefill chunk
// (prefill_rows.json), with raw bf16 .bin files.
//
// --log-steps <file> writes one line per engine step with its batch's shape
// (phase, rows, items, attended tokens, the longest item, and for decode steps
// the fast decode's plan), to be read beside a kernel trace of the run.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <fstream>
#include <random>
#include <string>
#include <thread>
#include <unordered_map>
#include <unordered_set>

#include "hip_model_state.h"
#include "inference_engine.h"
#include "tensor_ops.h"

using namespace chibillm;

namespace {

struct options {
    std::size_t steps = 5000;
    std::uint64_t seed = 0;
    double pool_gb = 160.0;
    std::size_t max_live = 512;
    double arrival_mean = 8.0;
    double prompt_median = 512, output_median = 256, sigma = 1.0;
    std::size_t prompt_min = 16, prompt_max = 16384, output_min = 1, output_max = 4096;
    std::size_t layers = 28, kv_heads = 8, q_heads = 16, head_dim = 128, block_size = 16;
    std::size_t max_batch_tokens = 2048, prefill_chunk = 512;
    bool profile = false;
    bool device_tables = false; // sequence tables kept on the device (device_tables)
    bool host_timing = false;   // drain the GPU before each step's metadata work and time it
    std::string check_dir;      // --check: verify the trace and dump one decode step here
    std::string log_steps;      // --log-steps: one line per step with its batch's shape
    std::size_t check_every = 250;
    std::size_t dump_after = 1000;
};

// Sequences whose K/V the check follows: every 50th id.
bool sampled(seq_id id)
{
    return id % 50 == 7;
}

// Seeded draws: std::mt19937_64 (fully specified) with explicit transforms.
struct draws {
    std::mt19937_64 rng;
    explicit draws(std::uint64_t seed)
        : rng(seed)
    {}
    double uniform() { return (rng() >> 11) * 0x1.0p-53; } // [0, 1)
    double normal()                                         // Box-Muller, one output
    {
        const double u1 = 1.0 - uniform(), u2 = uniform();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * M_PI * u2);
    }
    std::size_t poisson(double mean) // Knuth's product of uniforms
    {
        const double limit = std::exp(-mean);
        std::size_t k = 0;
        for (double p = uniform(); p > limit; p *= uniform())
            ++k;
        return k;
    }
    std::size_t lognormal(double median, double sigma, std::size_t lo, std::size_t hi)
    {
        const double x = std::exp(std::log(median) + sigma * normal());
        const auto v = static_cast<std::size_t>(std::llround(x));
        return v < lo ? lo : v > hi ? hi : v;
    }
};

// Counter-based N(0,1) draws rounded to bf16: value i of stream s is a
// Box-Muller transform of two splitmix64 outputs keyed by (seed, s, i), so any
// value can be drawn again on its own.
std::uint64_t
mix64(std::uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

std::uint16_t
normal_bf16(std::uint64_t seed, std::uint64_t stream, std::uint64_t i)
{
    const std::uint64_t a = mix64(seed ^ mix64(stream * 0x100000001B3ull ^ (2 * i)));
    const std::uint64_t b = mix64(a ^ (2 * i + 1));
    const double u1 = ((a >> 11) + 1) * 0x1.0p-53, u2 = (b >> 11) * 0x1.0p-53;
    const float x = static_cast<float>(std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * M_PI * u2));
    std::uint32_t bits;
    std::memcpy(&bits, &x, 4);
    bits += 0x7FFFu + ((bits >> 16) & 1u);
    return static_cast<std::uint16_t>(bits >> 16);
}

// n values of one stream, on the host's threads
std::vector<std::uint16_t>
draw_stream(std::size_t n, std::uint64_t seed, std::uint64_t stream)
{
    std::vector<std::uint16_t> out(n);
    const std::size_t workers = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> pool;
    for (std::size_t w = 0; w < workers; ++w)
        pool.emplace_back([&, w] {
            for (std::size_t i = w * n / workers, e = (w + 1) * n / workers; i < e; ++i)
                out[i] = normal_bf16(seed, stream, i);
        });
    for (auto& t : pool)
        t.join();
    return out;
}

// Streams of the row buffers: K, V and Q of each layer.
std::uint64_t
row_stream(std::size_t layer, int tensor)
{
    return 3 * layer + static_cast<std::uint64_t>(tensor) + 1;
}

struct totals {
    std::size_t prefill_steps = 0, decode_steps = 0;
    std::size_t prefill_rows = 0, decode_rows = 0;
    double kv_read_bytes = 0, append_bytes = 0, metadata_bytes = 0, qo_bytes = 0;
    double decode_bytes = 0; // the decode steps' share: K/V read, appends, Q and O
    double h2d_bytes = 0;    // metadata sent over PCIe
    double metadata_host_s = 0;
    std::size_t timed_steps = 0;
};

// The model stand-in: runs the KV path of every layer for each batch.
class churn_runner final : public model_runner {
public:
    churn_runner(const options& opt, hip_context& ctx)
        : opt_(opt)
        , ctx_(ctx)
    {
        if (!opt_.log_steps.empty())
            step_log_ = std::fopen(opt_.log_steps.c_str(), "w");
    }
    ~churn_runner() override
    {
        if (step_log_)
            std::fclose(step_log_);
    }
    churn_runner(const churn_runner&) = delete;
    churn_runner& operator=(const churn_runner&) = delete;
    bool step_log_open() const noexcept { return opt_.log_steps.empty() || step_log_; }

    const model_info& info() const noexcept override { return info_; }

    result<std::unique_ptr<model_state>, model_runner_error> make_state(
        scheduler_config config) const override
    {
        const kv_cache_config geometry { opt_.layers, config.kv_block_count, config.kv_block_size,
                                         opt_.kv_heads, opt_.head_dim };
        auto s = hip_model_state::make(ctx_, geometry, kv_dtype::bf16);
        if (!s)
            return fail(model_runner_errc::backend_failure, s.error(), "device KV pool");
        state_ = s->get();
        if (opt_.device_tables) {
            const std::size_t longest = opt_.prompt_max + opt_.output_max;
            auto on = state_->enable_device_tables(config.max_sequences,
                                                   (longest + config.kv_block_size - 1)
                                                           / config.kv_block_size
                                                       + 1);
            if (!on)
                return fail(model_runner_errc::backend_failure, on.error(), "device tables");
        }
        return std::unique_ptr<model_state>(std::move(*s));
    }

    // The row buffers: per layer, K, V and Q rows for twice the batch cap (a
    // step's rows are a window of them), drawn from the layer's own streams;
    // kept on the host too when the trace is checked.
    result<void, std::string> allocate(bool keep_host)
    {
        window_rows_ = 2 * opt_.max_batch_tokens;
        const std::size_t F = opt_.kv_heads * opt_.head_dim, QF = opt_.q_heads * opt_.head_dim;
        auto fill = [&](device_buffer& b, std::size_t n, std::uint64_t stream,
                        std::vector<std::uint16_t>* keep) -> bool {
            auto made = device_buffer::make(ctx_, n * 2);
            if (!made)
                return false;
            b = std::move(*made);
            auto host = draw_stream(n, opt_.seed, stream);
            const bool ok = b.upload(host.data(), n * 2).has_value();
            if (keep)
                *keep = std::move(host);
            return ok;
        };
        k_.resize(opt_.layers);
        v_.resize(opt_.layers);
        q_.resize(opt_.layers);
        if (keep_host) {
            k_host_.resize(opt_.layers);
            v_host_.resize(opt_.layers);
            q_host_.resize(opt_.layers);
            checking_ = true;
        }
        for (std::size_t l = 0; l < opt_.layers; ++l)
            if (!fill(k_[l], window_rows_ * F, row_stream(l, 0), keep_host ? &k_host_[l] : nullptr)
                || !fill(v_[l], window_rows_ * F, row_stream(l, 1), keep_host ? &v_host_[l] : nullptr)
                || !fill(q_[l], window_rows_ * QF, row_stream(l, 2), keep_host ? &q_host_[l] : nullptr))
                return fail(std::string("row buffers"));
        auto out = device_buffer::make(ctx_, opt_.max_batch_tokens * QF * 2);
        if (!out)
            return fail(std::string("output buffer"));
        o_ = std::move(*out);
        return {};
    }

    result<std::vector<token_id>, model_runner_error> execute(const model_batch& batch,
                                                              model_state&) override
    {
        auto& cache = state_->cache();
        const std::size_t rows = batch.tokens.size();
        if (opt_.host_timing)
            (void)ctx_.sync();
        const auto t0 = std::chrono::steady_clock::now();
        double h2d = 0;
        if (auto* tables = state_->tables()) {
            const std::size_t sent = tables->entries_sent();
            auto up = tables->upload(batch, info_.max_context_tokens, true);
            if (!up)
                return fail(model_runner_errc::backend_failure, up.error());
            // (seq, index, block) per changed entry, 5 words per item
            h2d = 4.0 * (3.0 * (tables->entries_sent() - sent) + 5.0 * batch.items.size());
        } else {
            auto md = prepare_paged_batch(batch, info_.max_context_tokens, cache.block_count(),
                                          cache.block_size());
            if (!md)
                return fail(model_runner_errc::inconsistent_batch, md.error());
            positions_.assign(batch.positions.begin(), batch.positions.end());
            auto up = upload_attention_metadata(cache, { positions_, md->slots, md->block_table,
                                                         md->table_offsets, md->table_lengths });
            if (!up)
                return fail(model_runner_errc::backend_failure, up.error());
            h2d = 4.0 * (md->block_table.size() + 4.0 * rows);
        }
        if (opt_.host_timing) {
            totals_.metadata_host_s +=
                std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
            ++totals_.timed_steps;
        }
        const std::size_t F = opt_.kv_heads * opt_.head_dim, QF = opt_.q_heads * opt_.head_dim;
        // this step's rows: a window of every layer's row buffers at a seeded offset
        offset_ = mix64(opt_.seed ^ (0xC0FFEEull + step_)) % opt_.max_batch_tokens;
        ++step_;
        device_tensor o { o_.data(), dtype::bf16, { rows, QF } };
        const bool decode = batch.phase == batch_phase::decode;
        const bool dumping = checking_ && (decode ? dump_decode_wanted_ : dump_prefill_wanted_);
        std::vector<std::uint16_t> out_first; // layer 0's outputs of a dumped step
        for (std::size_t layer = 0; layer < opt_.layers; ++layer) {
            auto* kb = static_cast<std::uint16_t*>(k_[layer].data()) + offset_ * F;
            auto* vb = static_cast<std::uint16_t*>(v_[layer].data()) + offset_ * F;
            auto* qb = static_cast<std::uint16_t*>(q_[layer].data()) + offset_ * QF;
            const device_tensor k { kb, dtype::bf16, { rows, F } };
            const device_tensor v { vb, dtype::bf16, { rows, F } };
            const device_tensor q { qb, dtype::bf16, { rows, QF } };
            if (layer == 1 && dumping) {
                out_first.resize(rows * QF);
                if (!o_.download(out_first.data(), rows * QF * 2))
                    return fail(model_runner_errc::backend_failure, "check: output download");
            }
            if (decode) {
                auto done = store_kv_and_attend(cache, k, v, q, layer, opt_.q_heads, o);
                if (!done)
                    return fail(model_runner_errc::backend_failure, done.error());
            } else {
                auto stored = store_kv(cache, k, v, layer);
                if (!stored)
                    return fail(model_runner_errc::backend_failure, stored.error());
                auto attended = paged_attention(cache, q, layer, opt_.q_heads, o);
                if (!attended)
                    return fail(model_runner_errc::backend_failure, attended.error());
            }
        }
        account(batch, h2d);
        if (step_log_)
            log_step(cache.pool(), batch);
        if (checking_) {
            auto recorded = record(batch);
            if (recorded && dumping) {
                if (out_first.empty()) { // one layer: layer 0 is the last
                    out_first.resize(rows * QF);
                    if (!o_.download(out_first.data(), rows * QF * 2))
                        return fail(model_runner_errc::backend_failure, "check: output download");
                }
                recorded = decode ? dump_decode(batch, out_first) : dump_prefill(batch, out_first);
                (decode ? dump_decode_wanted_ : dump_prefill_wanted_) = false;
                (decode ? dumped_decode_ : dumped_prefill_) = recorded.has_value();
            }
            if (!recorded) {
                check_error_ = recorded.error();
                return fail(model_runner_errc::backend_failure, "check: " + check_error_);
            }
        }
        return std::vector<token_id>(batch.sample_count(), 7);
    }

    const totals& stats() const noexcept { return totals_; }
    hip_model_state* state() const noexcept { return state_; }

    // ---- --check ------------------------------------------------------------
    void forget(seq_id id) { appended_.erase(id); }
    void request_dumps()
    {
        dump_decode_wanted_ = !dumped_decode_;
        dump_prefill_wanted_ = !dumped_prefill_;
    }
    bool dumped() const noexcept { return dumped_decode_ && dumped_prefill_; }
    bool dumped_decode() const noexcept { return dumped_decode_; }
    bool dumped_prefill() const noexcept { return dumped_prefill_; }
    std::size_t kv_tokens_checked() const noexcept { return kv_tokens_checked_; }

    // Page accounting over the live sequences: no page in two tables or twice
    // in one, each table page held exactly once (no prefix sharing in this
    // trace), the reference counts summing to the pages in tables, and free +
    // used = the pool.
    result<void, std::string> check_pages(const std::unordered_set<seq_id>& live) const
    {
        const block_manager& pages = state_->pages();
        std::vector<std::uint8_t> seen(pages.block_count(), 0);
        std::size_t in_tables = 0;
        for (const seq_id id : live) {
            for (const block_id b : pages.resources(id).blocks) {
                if (b >= pages.block_count() || seen[b])
                    return fail("page " + std::to_string(b) + " held twice (sequence "
                                + std::to_string(id) + ")");
                seen[b] = 1;
                if (pages.refcount(b) != 1)
                    return fail("page " + std::to_string(b) + " has "
                                + std::to_string(pages.refcount(b)) + " references");
                ++in_tables;
            }
        }
        std::uint64_t refs = 0;
        for (std::size_t b = 0; b < pages.block_count(); ++b)
            refs += pages.refcount(static_cast<block_id>(b));
        if (refs != in_tables)
            return fail("reference counts sum to " + std::to_string(refs) + ", tables hold "
                        + std::to_string(in_tables));
        if (pages.free_block_count() + in_tables != pages.block_count())
            return fail("free " + std::to_string(pages.free_block_count()) + " + used "
                        + std::to_string(in_tables) + " != pool "
                        + std::to_string(pages.block_count()));
        return {};
    }

    // Every appended token of up to `limit` followed sequences, all layers,
    // packed back from their pages and compared bit for bit with the row the
    // trace appended at that position.
    result<void, std::string> check_kv(std::size_t limit)
    {
        const std::size_t F = opt_.kv_heads * opt_.head_dim;
        std::vector<seq_id> ids;
        for (const auto& [id, rows] : appended_)
            if (sampled(id) && !rows.empty())
                ids.push_back(id);
        std::sort(ids.begin(), ids.end());
        // `limit` of them per check, rotating through the followed sequences
        const std::size_t count = std::min(limit, ids.size());
        for (std::size_t i = 0; i < count; ++i) {
            const seq_id id = ids[(check_round_ * limit + i) % ids.size()];
            const auto& rows = appended_.at(id);
            const std::size_t n = rows.size();
            std::vector<std::uint16_t> pk, pv;
            if (auto packed = pack(id, n, pk, pv); !packed)
                return packed;
            for (std::size_t layer = 0; layer < opt_.layers; ++layer)
                for (std::size_t t = 0; t < n; ++t) {
                    const std::size_t at = (layer * n + t) * F;
                    const std::size_t src = static_cast<std::size_t>(rows[t]) * F;
                    if (std::memcmp(&pk[at], &k_host_[layer][src], F * 2) != 0
                        || std::memcmp(&pv[at], &v_host_[layer][src], F * 2) != 0)
                        return fail("sequence " + std::to_string(id) + " layer "
                                    + std::to_string(layer) + " token " + std::to_string(t)
                                    + " differs from the row appended");
                }
            kv_tokens_checked_ += n * opt_.layers;
        }
        ++check_round_;
        return {};
    }

private:
    // The sequence's first n tokens of every layer, [layer][token][feature].
    result<void, std::string> pack(seq_id id, std::size_t n, std::vector<std::uint16_t>& k,
                                   std::vector<std::uint16_t>& v) const
    {
        const std::size_t F = opt_.kv_heads * opt_.head_dim;
        const std::size_t bytes = opt_.layers * n * F * 2;
        auto dk = device_buffer::make(ctx_, bytes);
        auto dv = device_buffer::make(ctx_, bytes);
        if (!dk || !dv)
            return fail(std::string("check buffers"));
        const auto blocks = state_->pages().resources(id).blocks;
        const int rc = ckv_checkpoint_pack(state_->cache().pool(), blocks.data(), blocks.size(), n,
                                           dk->data(), dv->data());
        if (rc)
            return fail(std::string("pack: ") + ckv_error_name(rc));
        k.resize(bytes / 2);
        v.resize(bytes / 2);
        if (!dk->download(k.data(), bytes) || !dv->download(v.data(), bytes))
            return fail(std::string("check download"));
        return {};
    }

    // Rows of the batch that append each sequence's tokens: position -> row of
    // the layers' row buffers (the step's window offset plus the batch row).
    // A position appended again (a sequence computed anew after losing its
    // pages) replaces what followed it.
    result<void, std::string> record(const model_batch& batch)
    {
        for (const auto& item : batch.items) {
            auto& rows = appended_[item.id];
            for (std::size_t t = 0; t < item.token_count; ++t) {
                const std::size_t r = item.token_offset + t;
                const std::size_t position = batch.positions[r];
                if (position > rows.size())
                    return fail("sequence " + std::to_string(item.id) + " appends position "
                                + std::to_string(position) + " after "
                                + std::to_string(rows.size()) + " tokens");
                rows.resize(position);
                rows.push_back(static_cast<std::uint32_t>(offset_ + r));
            }
        }
        return {};
    }

    // A sequence's first n tokens of one layer as the trace appended them,
    // [token][feature], from the host copies of the row buffers.
    void regenerate(seq_id id, std::size_t n, std::size_t layer, std::vector<std::uint16_t>& k,
                    std::vector<std::uint16_t>& v) const
    {
        const std::size_t F = opt_.kv_heads * opt_.head_dim;
        const auto& rows = appended_.at(id);
        k.resize(n * F);
        v.resize(n * F);
        for (std::size_t t = 0; t < n; ++t) {
            const std::size_t src = static_cast<std::size_t>(rows[t]) * F;
            std::memcpy(&k[t * F], &k_host_[layer][src], F * 2);
            std::memcpy(&v[t * F], &v_host_[layer][src], F * 2);
        }
    }

    bool write_bin(const std::string& name, const std::uint16_t* p, std::size_t n) const
    {
        std::ofstream f(opt_.check_dir + "/" + name, std::ios::binary);
        f.write(reinterpret_cast<const char*>(p), static_cast<std::streamsize>(n * 2));
        return static_cast<bool>(f);
    }

    std::string layers_json() const
    {
        return "\"layers\": [0, " + std::to_string(opt_.layers - 1)
            + "], \"kv_heads\": " + std::to_string(opt_.kv_heads)
            + ", \"q_heads\": " + std::to_string(opt_.q_heads)
            + ", \"head_dim\": " + std::to_string(opt_.head_dim);
    }

    // Up to eight rows of this decode batch (spread over it), at layers 0 and
    // L - 1: each row's sequence K/V regenerated from the rows the trace
    // appended, its query and the kernel's output, for a CPU check.
    result<void, std::string> dump_decode(const model_batch& batch,
                                          const std::vector<std::uint16_t>& out_first)
    {
        const std::size_t QF = opt_.q_heads * opt_.head_dim;
        const std::size_t rows = batch.tokens.size();
        const std::size_t n_dump = std::min<std::size_t>(rows, 8);
        std::vector<std::uint16_t> out_last(rows * QF);
        if (!o_.download(out_last.data(), rows * QF * 2))
            return fail(std::string("output download"));
        std::string json = "{" + layers_json() + ", \"rows\": [";
        const std::size_t layers[2] = { 0, opt_.layers - 1 };
        for (int li = 0; li < 2; ++li) {
            const std::size_t layer = layers[li];
            const auto& out = li == 0 ? out_first : out_last;
            std::vector<std::uint16_t> q, o;
            for (std::size_t i = 0; i < n_dump; ++i) {
                const std::size_t r = i * rows / n_dump;
                const auto& item = batch.items[r];
                const std::size_t n = batch.positions[r] + 1;
                std::vector<std::uint16_t> k, v;
                regenerate(item.id, n, layer, k, v);
                const std::string tag = std::to_string(layer) + "_" + std::to_string(i);
                if (!write_bin("dk_" + tag + ".bin", k.data(), k.size())
                    || !write_bin("dv_" + tag + ".bin", v.data(), v.size()))
                    return fail(std::string("dump write"));
                const std::size_t qrow = offset_ + r;
                q.insert(q.end(), q_host_[layer].begin() + qrow * QF,
                         q_host_[layer].begin() + (qrow + 1) * QF);
                o.insert(o.end(), out.begin() + r * QF, out.begin() + (r + 1) * QF);
                if (li == 0)
                    json += (i ? ", " : "") + std::string("{\"seq\": ") + std::to_string(item.id)
                        + ", \"position\": " + std::to_string(n - 1) + ", \"row\": "
                        + std::to_string(r) + "}";
            }
            const std::string l = std::to_string(layer);
            if (!write_bin("dq_" + l + ".bin", q.data(), q.size())
                || !write_bin("dout_" + l + ".bin", o.data(), o.size()))
                return fail(std::string("dump write"));
        }
        json += "]}\n";
        std::ofstream(opt_.check_dir + "/decode_rows.json") << json;
        return {};
    }

    // One chunk of this prefill batch (the item attending the fewest keys of
    // those of at least 16 rows, else the largest), at layers 0 and L - 1: the
    // sequence's K/V up to the chunk's last position regenerated from the rows
    // the trace appended, the chunk's queries and the kernel's outputs.
    result<void, std::string> dump_prefill(const model_batch& batch,
                                           const std::vector<std::uint16_t>& out_first)
    {
        const std::size_t QF = opt_.q_heads * opt_.head_dim;
        const std::size_t rows = batch.tokens.size();
        std::vector<std::uint16_t> out_last(rows * QF);
        if (!o_.download(out_last.data(), rows * QF * 2))
            return fail(std::string("output download"));
        std::size_t best = 0;
        double best_cost = -1;
        for (std::size_t i = 0; i < batch.items.size(); ++i) {
            const auto& it = batch.items[i];
            const double keys = static_cast<double>(batch.positions[it.token_offset + it.token_count - 1] + 1);
            const double cost = it.token_count >= 16 ? keys * it.token_count : 1e30 - it.token_count;
            if (best_cost < 0 || cost < best_cost) {
                best = i;
                best_cost = cost;
            }
        }
        const auto& item = batch.items[best];
        const std::size_t first = item.token_offset, count = item.token_count;
        const std::size_t n = batch.positions[first + count - 1] + 1;
        std::string json = "{" + layers_json() + ", \"seq\": " + std::to_string(item.id)
            + ", \"first_position\": " + std::to_string(batch.positions[first])
            + ", \"rows\": " + std::to_string(count) + ", \"tokens\": " + std::to_string(n)
            + "}\n";
        const std::size_t layers[2] = { 0, opt_.layers - 1 };
        for (int li = 0; li < 2; ++li) {
            const std::size_t layer = layers[li];
            const auto& out = li == 0 ? out_first : out_last;
            std::vector<std::uint16_t> k, v;
            regenerate(item.id, n, layer, k, v);
            const std::string l = std::to_string(layer);
            const std::size_t qrow = offset_ + first;
            if (!write_bin("pk_" + l + ".bin", k.data(), k.size())
                || !write_bin("pv_" + l + ".bin", v.data(), v.size())
                || !write_bin("pq_" + l + ".bin", &q_host_[layer][qrow * QF], count * QF)
                || !write_bin("pout_" + l + ".bin", &out[first * QF], count * QF))
                return fail(std::string("dump write"));
        }
        std::ofstream(opt_.check_dir + "/prefill_rows.json") << json;
        return {};
    }

private:
    // --log-steps: phase (d or p), rows, items, attended tokens (every row's
    // for decode, every tile's last row's for prefill), the longest item's,
    // and for decode steps the fast decode's plan (pages per workgroup, work
    // items, partial records; ckv_decode_plan)
    void log_step(ckv_pool* pool, const model_batch& batch)
    {
        std::size_t attended = 0, longest = 0;
        for (const auto& item : batch.items) {
            const std::size_t a = batch.positions[item.token_offset + item.token_count - 1] + 1;
            attended += a;
            longest = std::max(longest, a);
        }
        const bool decode = batch.phase == batch_phase::decode;
        std::uint32_t split_pages = 0, work_items = 0, records = 0;
        if (decode)
            (void)ckv_decode_plan(pool, &split_pages, &work_items, &records);
        std::fprintf(step_log_, "%zu %c %zu %zu %zu %zu %u %u %u\n", step_ - 1, decode ? 'd' : 'p',
                     batch.tokens.size(), batch.items.size(), attended, longest, split_pages,
                     work_items, records);
    }

    // Algorithmic bytes of one step, all layers: K+V of every attended token
    // (once per decode row; once per prefill tile, whose rows share it), the
    // appended rows, Q and O, and the uploaded metadata.
    void account(const model_batch& batch, double h2d)
    {
        const double L = static_cast<double>(opt_.layers);
        const double row_kv = 2.0 * opt_.kv_heads * opt_.head_dim * 2.0;
        const double row_q = opt_.q_heads * opt_.head_dim * 2.0;
        double attended = 0;
        for (const auto& item : batch.items) {
            // a tile's rows attend keys up to its last row: count those once
            const std::size_t last = batch.positions[item.token_offset + item.token_count - 1];
            attended += static_cast<double>(last + 1);
        }
        const std::size_t rows = batch.tokens.size();
        const double kv = L * attended * row_kv;
        const double append = L * rows * row_kv * 2.0; // read the new rows, write the pages
        const double qo = L * rows * row_q * 2.0;
        totals_.kv_read_bytes += kv;
        totals_.append_bytes += append;
        totals_.qo_bytes += qo;
        // the per-row metadata the kernels read (offset, length, position, slot)
        totals_.metadata_bytes += h2d + 16.0 * rows;
        totals_.h2d_bytes += h2d;
        if (batch.phase == batch_phase::decode) {
            totals_.decode_bytes += kv + append + qo;
            ++totals_.decode_steps;
            totals_.decode_rows += rows;
        } else {
            ++totals_.prefill_steps;
            totals_.prefill_rows += rows;
        }
    }

    const options& opt_;
    hip_context& ctx_;
    model_info info_ { "churn", 1u << 20, -1 };
    mutable hip_model_state* state_ = nullptr;
    std::vector<device_buffer> k_, v_, q_; // per layer, window_rows_ rows each
    device_buffer o_;
    std::size_t window_rows_ = 0, step_ = 0, offset_ = 0;
    std::vector<std::uint32_t> positions_;
    totals totals_;
    // --check
    bool checking_ = false;
    std::FILE* step_log_ = nullptr;
    bool dump_decode_wanted_ = false, dump_prefill_wanted_ = false;
    bool dumped_decode_ = false, dumped_prefill_ = false;
    std::vector<std::vector<std::uint16_t>> k_host_, v_host_, q_host_; // per layer
    std::unordered_map<seq_id, std::vector<std::uint32_t>> appended_;
    std::size_t check_round_ = 0, kv_tokens_checked_ = 0;
    std::string check_error_;

public:
    const std::string& check_error() const noexcept { return check_error_; }
};

bool
parse(int argc, char** argv, options& o)
{
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&]() -> const char* { return i + 1 < argc ? argv[++i] : nullptr; };
        const char* v = nullptr;
        if (a == "--profile") {
            o.profile = true;
            continue;
        }
        if (a == "--device-tables") {
            o.device_tables = true;
            continue;
        }
        if (a == "--host-timing") {
            o.host_timing = true;
            continue;
        }
        if (!(v = next()))
            return false;
        if (a == "--check")
            o.check_dir = v;
        else if (a == "--check-every")
            o.check_every = std::strtoull(v, nullptr, 10);
        else if (a == "--dump-after")
            o.dump_after = std::strtoull(v, nullptr, 10);
        else if (a == "--steps")
            o.steps = std::strtoull(v, nullptr, 10);
        else if (a == "--seed")
            o.seed = std::strtoull(v, nullptr, 10);
        else if (a == "--pool-gb")
            o.pool_gb = std::strtod(v, nullptr);
        else if (a == "--max-live")
            o.max_live = std::strtoull(v, nullptr, 10);
        else if (a == "--arrival-mean")
            o.arrival_mean = std::strtod(v, nullptr);
        else if (a == "--layers")
            o.layers = std::strtoull(v, nullptr, 10);
        else if (a == "--max-batch-tokens")
            o.max_batch_tokens = std::strtoull(v, nullptr, 10);
        else if (a == "--prefill-chunk")
            o.prefill_chunk = std::strtoull(v, nullptr, 10);
        else if (a == "--sigma")
            o.sigma = std::strtod(v, nullptr);
        else if (a == "--log-steps")
            o.log_steps = v;
        else
            return false;
    }
    return o.steps > 0 && o.layers > 0 && o.max_live > 0 && o.pool_gb > 0;
}

} // namespace

int
main(int argc, char** argv)
{
    options opt;
    if (!parse(argc, argv, opt)) {
        std::fprintf(stderr,
                     "usage: churn [--steps N] [--seed S] [--pool-gb G] [--max-live N] "
                     "[--arrival-mean M] [--layers L] [--max-batch-tokens T] "
                     "[--prefill-chunk C] [--sigma S] [--profile] [--device-tables] "
                     "[--host-timing] [--check DIR [--check-every N] [--dump-after STEP]] "
                     "[--log-steps FILE]\n");
        return 2;
    }
    auto ctx = hip_context::make(0);
    if (!ctx) {
        std::fprintf(stderr, "no device: %s\n", describe_error(ctx.error()).c_str());
        return 1;
    }
    const double page_bytes = 2.0 * opt.layers * opt.block_size * opt.kv_heads * opt.head_dim * 2.0;
    scheduler_config config;
    config.max_sequences = opt.max_live;
    config.max_batch_tokens = opt.max_batch_tokens;
    config.kv_block_count = static_cast<std::size_t>(opt.pool_gb * 1e9 / page_bytes);
    config.kv_block_size = opt.block_size;
    config.prefill_chunk_tokens = opt.prefill_chunk;
    config.prefix_cache_bytes = 0;

    churn_runner runner(opt, *ctx);
    if (!runner.step_log_open()) {
        std::fprintf(stderr, "cannot write %s\n", opt.log_steps.c_str());
        return 1;
    }
    auto engine = inference_engine::make(config, runner);
    if (!engine) {
        std::fprintf(stderr, "engine: %s\n", describe_error(engine.error()).c_str());
        return 1;
    }
    const bool check = !opt.check_dir.empty();
    if (auto a = runner.allocate(check); !a) {
        std::fprintf(stderr, "allocation failed: %s\n", a.error().c_str());
        return 1;
    }
    std::unordered_set<seq_id> live;
    std::size_t checks = 0;
    // the trace's checks; a failure ends the run with status 3
    auto run_checks = [&](std::size_t step) -> bool {
        auto pages = runner.check_pages(live);
        if (pages)
            pages = runner.check_kv(4);
        if (!pages) {
            std::fprintf(stderr, "[churn] check failed at step %zu: %s\n", step,
                         pages.error().c_str());
            return false;
        }
        ++checks;
        std::fprintf(stderr, "[churn] step %zu: checks passed (%zu live, %zu K/V tokens so far)\n",
                     step, live.size(), runner.kv_tokens_checked());
        return true;
    };
    if (opt.profile)
        ckv_profile_enable(ctx->get(), 1);
    std::fprintf(stderr, "[churn] pool %zu pages (%.1f GB), %zu layers, live cap %zu, %zu steps\n",
                 config.kv_block_count, config.kv_block_count * page_bytes / 1e9, opt.layers,
                 opt.max_live, opt.steps);

    draws rng(opt.seed);
    std::deque<seq> pending;
    seq_id next_id = 1;
    std::size_t arrived = 0, admitted = 0, finished = 0, rejected = 0, peak_live = 0;
    std::vector<token_id> prompt;
    const auto t0 = std::chrono::steady_clock::now();
    auto last_report = t0;
    for (std::size_t step = 0; step < opt.steps; ++step) {
        const std::size_t arrivals = rng.poisson(opt.arrival_mean);
        for (std::size_t a = 0; a < arrivals; ++a) {
            const std::size_t plen = rng.lognormal(opt.prompt_median, opt.sigma, opt.prompt_min,
                                                   opt.prompt_max);
            const std::size_t olen = rng.lognormal(opt.output_median, opt.sigma, opt.output_min,
                                                   opt.output_max);
            prompt.resize(plen);
            for (std::size_t t = 0; t < plen; ++t)
                prompt[t] = static_cast<token_id>((next_id * 7919 + t) % 151000 + 1);
            auto s = seq::make(next_id++, prompt, generation_params { olen, true });
            if (!s) {
                std::fprintf(stderr, "seq: %s\n", describe_error(s.error()).c_str());
                return 1;
            }
            pending.push_back(std::move(*s));
            ++arrived;
        }
        while (!pending.empty()) {
            const seq_id id = pending.front().id(); // try_add may move the sequence
            auto r = engine->try_add(pending.front());
            if (!r) {
                std::fprintf(stderr, "admission: %s\n", describe_error(r.error()).c_str());
                return 1;
            }
            if (*r == admission_result::deferred)
                break;
            if (*r == admission_result::too_large) {
                ++rejected;
            } else {
                ++admitted;
                live.insert(id);
            }
            pending.pop_front();
        }
        const auto& sched = engine->engine_scheduler();
        peak_live = std::max(peak_live, sched.running_count() + sched.waiting_count());
        if (sched.running_count() + sched.waiting_count() == 0)
            continue;
        if (check && step >= opt.dump_after && !runner.dumped())
            runner.request_dumps();
        auto updates = engine->step();
        if (!updates) {
            std::fprintf(stderr, "step %zu: %s\n", step, describe_error(updates.error()).c_str());
            return runner.check_error().empty() ? 1 : 3;
        }
        for (const auto& u : *updates)
            if (u.reason != finish_reason::none) {
                if (auto removed = engine->remove(u.id); !removed) {
                    std::fprintf(stderr, "remove: %s\n", describe_error(removed.error()).c_str());
                    return 1;
                }
                live.erase(u.id);
                runner.forget(u.id);
                ++finished;
            }
        if (check && (step + 1) % opt.check_every == 0 && !run_checks(step))
            return 3;
        const auto now = std::chrono::steady_clock::now();
        if (now - last_report > std::chrono::seconds(10)) {
            last_report = now;
            std::fprintf(stderr, "[churn] step %zu: live %zu, pending %zu, finished %zu\n", step,
                         sched.running_count() + sched.waiting_count(), pending.size(), finished);
        }
    }
    if (auto synced = ctx->sync(); !synced) {
        std::fprintf(stderr, "sync: %s\n", describe_error(synced.error()).c_str());
        return 1;
    }
    if (check && !run_checks(opt.steps))
        return 3;
    const double seconds =
        std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    const auto& t = runner.stats();
    const double bytes = t.kv_read_bytes + t.append_bytes + t.qo_bytes + t.metadata_bytes;
    const double rows = static_cast<double>(t.prefill_rows + t.decode_rows);
    std::printf("{\"steps\": %zu, \"seconds\": %.4f, \"steps_per_s\": %.2f, \"tokens_per_s\": %.1f, "
                "\"prefill_tokens\": %zu, \"decode_tokens\": %zu, \"prefill_steps\": %zu, "
                "\"decode_steps\": %zu, \"hbm_bytes\": %.6e, \"hbm_gbs\": %.2f, "
                "\"hbm_frac\": %.4f, \"kv_read_bytes\": %.6e, \"append_bytes\": %.6e, "
                "\"decode_step_bytes\": %.6e, "
                "\"arrived\": %zu, \"admitted\": %zu, \"finished\": %zu, \"rejected\": %zu, "
                "\"pending_at_end\": %zu, \"peak_live\": %zu, \"pool_pages\": %zu, "
                "\"device_tables\": %s, \"h2d_bytes_per_step\": %.1f",
                opt.steps, seconds, opt.steps / seconds, rows / seconds, t.prefill_rows,
                t.decode_rows, t.prefill_steps, t.decode_steps, bytes, bytes / seconds / 1e9,
                bytes / seconds / 8e12, t.kv_read_bytes, t.append_bytes, t.decode_bytes, arrived,
                admitted,
                finished, rejected, pending.size(), peak_live, config.kv_block_count,
                opt.device_tables ? "true" : "false",
                t.h2d_bytes / std::max<std::size_t>(1, t.prefill_steps + t.decode_steps));
    if (check)
        std::printf(", \"check\": {\"checks\": %zu, \"kv_tokens_checked\": %zu, "
                    "\"dumped_decode\": %s, \"dumped_prefill\": %s}",
                    checks, runner.kv_tokens_checked(), runner.dumped_decode() ? "true" : "false",
                    runner.dumped_prefill() ? "true" : "false");
    if (opt.host_timing)
        std::printf(", \"metadata_host_us_per_step\": %.2f",
                    1e6 * t.metadata_host_s / std::max<std::size_t>(1, t.timed_steps));
    if (opt.profile) {
        std::printf(", \"kernels_ms\": {");
        const char* names[] = { "append_decode", "paged_attention_decode", "paged_attention_merge",
                                "paged_attention_prefill", "store_kv" };
        for (std::size_t i = 0; i < 5; ++i) {
            double ms = 0;
            std::uint64_t n = 0;
            ckv_profile_query(ctx->get(), names[i], &ms, &n);
            std::printf("%s\"%s\": [%.3f, %llu]", i ? ", " : "", names[i], ms,
                        static_cast<unsigned long long>(n));
        }
        std::printf("}");
    }
    std::printf("}\n");
    return 0;
}

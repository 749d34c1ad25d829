// Continuous-batching churn trace on the device KV path (the config-5
// workload): seeded Poisson arrivals, lognormal prompt and output lengths,
// the C++ scheduler and refcounted page allocator over a large device pool,
// and every engine step running the KV path for all layers: the batch's
// metadata uploaded once (tables mirrored on the device), then per layer the
// append of every row plus paged attention (prefill tiles on the matrix
// cores for prefill batches; the fused append + decode kernel for decode
// batches). K/V/Q rows are synthetic bf16 N(0,1) values resident in HBM.
//
// Prints one JSON line: steps/s, tokens/s (prefill + decode rows), and the
// algorithmic HBM bytes of the path per second against the 8 TB/s peak.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <random>
#include <string>

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
};

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

std::vector<std::uint16_t>
random_bf16(std::size_t n, std::uint64_t seed)
{
    draws d(seed);
    std::vector<std::uint16_t> out(n);
    for (auto& v : out) {
        const float x = static_cast<float>(d.normal());
        std::uint32_t b;
        std::memcpy(&b, &x, 4);
        b += 0x7FFFu + ((b >> 16) & 1u);
        v = static_cast<std::uint16_t>(b >> 16);
    }
    return out;
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
    {}

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

    result<void, std::string> allocate()
    {
        const std::size_t rows = opt_.max_batch_tokens;
        const std::size_t F = opt_.kv_heads * opt_.head_dim, QF = opt_.q_heads * opt_.head_dim;
        auto fill = [&](device_buffer& b, std::size_t n, std::uint64_t seed) -> bool {
            auto made = device_buffer::make(ctx_, n * 2);
            if (!made)
                return false;
            b = std::move(*made);
            const auto host = random_bf16(n, seed);
            return b.upload(host.data(), n * 2).has_value();
        };
        if (!fill(k_, rows * F, 11) || !fill(v_, rows * F, 12) || !fill(q_, rows * QF, 13)
            || !fill(o_, rows * QF, 14))
            return fail(std::string("row buffers"));
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
        const device_tensor k { k_.data(), dtype::bf16, { rows, F } };
        const device_tensor v { v_.data(), dtype::bf16, { rows, F } };
        const device_tensor q { q_.data(), dtype::bf16, { rows, QF } };
        device_tensor o { o_.data(), dtype::bf16, { rows, QF } };
        const bool decode = batch.phase == batch_phase::decode;
        for (std::size_t layer = 0; layer < opt_.layers; ++layer) {
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
        return std::vector<token_id>(batch.sample_count(), 7);
    }

    const totals& stats() const noexcept { return totals_; }
    hip_model_state* state() const noexcept { return state_; }

private:
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
    device_buffer k_, v_, q_, o_;
    std::vector<std::uint32_t> positions_;
    totals totals_;
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
        if (a == "--steps")
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
                     "[--host-timing]\n");
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
    auto engine = inference_engine::make(config, runner);
    if (!engine) {
        std::fprintf(stderr, "engine: %s\n", describe_error(engine.error()).c_str());
        return 1;
    }
    if (auto a = runner.allocate(); !a) {
        std::fprintf(stderr, "allocation failed: %s\n", a.error().c_str());
        return 1;
    }
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
            auto r = engine->try_add(pending.front());
            if (!r) {
                std::fprintf(stderr, "admission: %s\n", describe_error(r.error()).c_str());
                return 1;
            }
            if (*r == admission_result::deferred)
                break;
            if (*r == admission_result::too_large)
                ++rejected;
            else
                ++admitted;
            pending.pop_front();
        }
        const auto& sched = engine->engine_scheduler();
        peak_live = std::max(peak_live, sched.running_count() + sched.waiting_count());
        if (sched.running_count() + sched.waiting_count() == 0)
            continue;
        auto updates = engine->step();
        if (!updates) {
            std::fprintf(stderr, "step %zu: %s\n", step, describe_error(updates.error()).c_str());
            return 1;
        }
        for (const auto& u : *updates)
            if (u.reason != finish_reason::none) {
                if (auto removed = engine->remove(u.id); !removed) {
                    std::fprintf(stderr, "remove: %s\n", describe_error(removed.error()).c_str());
                    return 1;
                }
                ++finished;
            }
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

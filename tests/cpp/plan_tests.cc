// The fast decode's batch planner (shape_decode_plan / write_decode_plan in
// libckv), on the CPU: every plan covers each row's pages exactly once, in
// segments whose chunk indices, chunk counts, table offsets and partial
// records agree; each workgroup's entries link from entry w through its
// segments; the balanced plan evens out the work; the fixed and forced forms
// follow their definitions. The plans' outputs on the GPU are checked against
// the oracle by the -m gpu tests.
#include <algorithm>
#include <cstdlib>
#include <random>
#include <utility>

#include "check.h"
#include "ckv_internal.h"

namespace {

constexpr uint32_t bs = 16;

struct plan_view {
    ckv::decode_plan_shape shape;
    std::vector<uint32_t> entries, split_first, cut;
    std::vector<std::vector<uint32_t>> wg_segments; // entry indices per workgroup
    std::vector<uint64_t> wg_pages;
};

uint32_t pages_of(uint32_t position)
{
    return position / bs + 1;
}

// Builds the plan of `positions` (rows' table offsets packed in row order)
// and checks every structural property; returns it for further checks.
plan_view plan_and_check(const std::vector<uint32_t>& positions, uint32_t kv_heads, int cus)
{
    plan_view v;
    v.shape = ckv::shape_decode_plan(positions, bs, kv_heads, cus);
    std::vector<uint32_t> offsets(positions.size());
    uint32_t at = 0;
    for (size_t r = 0; r < positions.size(); ++r) {
        offsets[r] = at;
        at += pages_of(positions[r]);
    }
    const auto& s = v.shape;
    v.entries.assign(ckv::plan_entry_words * s.n_items, 0xDEADBEEFu);
    v.split_first.assign(positions.size(), 0xDEADBEEFu);
    v.cut.assign(s.n_cut, 0xDEADBEEFu);
    std::vector<uint64_t> scratch;
    ckv::write_decode_plan(positions, offsets, bs, s, scratch, v.entries.data(),
                           v.split_first.data(), v.cut.data());
    REQUIRE(s.n_wgs >= 1 && s.n_wgs <= s.n_items);
    // walk every workgroup's links; each entry is reached once
    std::vector<int> seen(s.n_items, 0);
    std::vector<std::vector<std::pair<uint32_t, uint32_t>>> cover(positions.size());
    std::vector<uint32_t> chunk_count(positions.size(), 0);
    for (uint32_t w = 0; w < s.n_wgs; ++w) {
        std::vector<uint32_t> segs;
        uint64_t pages = 0;
        for (uint32_t e = w;;) {
            REQUIRE(e < s.n_items);
            REQUIRE(!seen[e]);
            seen[e] = 1;
            segs.push_back(e);
            const uint32_t* x = &v.entries[ckv::plan_entry_words * e];
            const uint32_t row = x[0];
            REQUIRE(row < positions.size());
            CHECK(x[2] == positions[row]);
            REQUIRE(x[4] < x[5] && x[5] <= pages_of(positions[row]));
            CHECK(x[3] == offsets[row] + x[4]);
            REQUIRE(x[1] < x[6]);
            cover[row].push_back({ x[4], x[5] });
            chunk_count[row] = x[6];
            pages += x[5] - x[4];
            if (x[7] == ckv::plan_last)
                break;
            e = x[7];
        }
        v.wg_segments.push_back(segs);
        v.wg_pages.push_back(pages);
    }
    for (uint32_t e = 0; e < s.n_items; ++e)
        CHECK(seen[e]);
    // each row: pages 0..n covered once, by its n_chunks pieces in chunk order
    uint32_t records = 0, n_cut = 0;
    std::vector<std::pair<uint32_t, uint32_t>> record_ranges;
    for (size_t r = 0; r < positions.size(); ++r) {
        auto c = cover[r];
        std::sort(c.begin(), c.end());
        uint32_t pg = 0;
        for (const auto& piece : c) {
            CHECK(piece.first == pg);
            pg = piece.second;
        }
        CHECK(pg == pages_of(positions[r]));
        CHECK(chunk_count[r] == c.size());
        if (c.size() > 1) {
            records += (uint32_t)c.size();
            CHECK(v.cut[n_cut] == r);
            ++n_cut;
            record_ranges.push_back({ v.split_first[r], v.split_first[r] + (uint32_t)c.size() });
        }
    }
    CHECK(records == s.n_records);
    CHECK(n_cut == s.n_cut);
    // the cut rows' records are disjoint ranges inside [0, n_records)
    std::sort(record_ranges.begin(), record_ranges.end());
    for (size_t i = 0; i < record_ranges.size(); ++i) {
        CHECK(record_ranges[i].second <= s.n_records);
        if (i)
            CHECK(record_ranges[i - 1].second <= record_ranges[i].first);
    }
    // chunk c of a row covers the row's c-th range of pages
    for (uint32_t e = 0; e < s.n_items; ++e) {
        const uint32_t* x = &v.entries[ckv::plan_entry_words * e];
        auto c = cover[x[0]];
        std::sort(c.begin(), c.end());
        CHECK(c[x[1]].first == x[4]);
    }
    return v;
}

std::vector<uint32_t> uniform_rows(std::mt19937_64& g, size_t n, uint32_t lo, uint32_t hi)
{
    std::vector<uint32_t> p(n);
    for (auto& x : p)
        x = lo + (uint32_t)(g() % (hi - lo + 1)) - 1; // positions of rows of lo..hi tokens
    return p;
}

struct env_guard {
    const char* name;
    env_guard(const char* n, const char* value) : name(n) { setenv(n, value, 1); }
    ~env_guard() { unsetenv(name); }
};

} // namespace

TEST("config-2 batch: balanced, every workgroup within a few pages of its share")
{
    std::mt19937_64 g(0);
    const auto p = uniform_rows(g, 32, 256, 4096);
    const auto v = plan_and_check(p, 8, 256);
    CHECK(v.shape.balanced);
    CHECK(v.shape.n_wgs == 64); // two 8-wave workgroups per compute unit, 8 kv heads
    // work per workgroup (pages plus 4 per segment): all within 16 of each
    // other (a row's short rest stays with its neighbour), 60 of the 64 within
    // 2 of the median
    std::vector<uint64_t> work;
    for (size_t w = 0; w < v.wg_pages.size(); ++w)
        work.push_back(v.wg_pages[w] + 4 * v.wg_segments[w].size());
    std::sort(work.begin(), work.end());
    const uint64_t median = work[work.size() / 2];
    CHECK(work.back() - work.front() <= 16);
    size_t near = 0;
    for (const uint64_t x : work)
        near += x + 2 >= median && x <= median + 2;
    CHECK(near >= 60);
    for (const auto& segs : v.wg_segments)
        CHECK(segs.size() <= 3);
}

TEST("uniform rows: whole rows when they fill the GPU, balanced pieces when they do not")
{
    for (uint32_t tokens : { 1024u, 4096u, 16384u }) {
        // 32 rows x 8 kv heads = one (row, kv head) unit per compute unit
        const auto v = plan_and_check(std::vector<uint32_t>(32, tokens - 1), 8, 256);
        CHECK(!v.shape.balanced && v.shape.split_pages == 0 && v.shape.n_items == 32);
    }
    for (uint32_t tokens : { 4096u, 16384u }) {
        // 16 rows leave half the compute units without a unit: each row in 4 pieces
        const auto v = plan_and_check(std::vector<uint32_t>(16, tokens - 1), 8, 256);
        CHECK(v.shape.balanced);
        CHECK(v.shape.n_wgs == 64); // two 8-wave workgroups per compute unit, 8 kv heads
        for (size_t w = 0; w < v.wg_pages.size(); ++w) {
            CHECK(v.wg_segments[w].size() == 1);
            CHECK(v.wg_pages[w] == pages_of(tokens - 1) / 4);
        }
    }
}

TEST("rows near the share stay whole, far longer ones are cut")
{
    // 32 rows of U[512, 1536] tokens: longest 96 pages against a share of about 64
    std::mt19937_64 g(3);
    auto p = uniform_rows(g, 32, 512, 1536);
    p[0] = 1535;
    auto v = plan_and_check(p, 8, 256);
    CHECK(v.shape.split_pages == 0 && v.shape.n_items == 32);
    // one row of 5,000 tokens among them exceeds 9/8 of the share by more than 47 pages
    p[0] = 4999;
    v = plan_and_check(p, 8, 256);
    CHECK(v.shape.n_records > 0);
}

TEST("short rows, small batches and many rows keep the fixed plan")
{
    // one page per row: a row per workgroup
    auto v = plan_and_check(std::vector<uint32_t>(32, 15), 8, 256);
    CHECK(!v.shape.balanced && v.shape.split_pages == 0 && v.shape.n_wgs == 32);
    // 32 rows of 16 pages fill the GPU with whole rows
    v = plan_and_check(std::vector<uint32_t>(32, 255), 8, 256);
    CHECK(!v.shape.balanced && v.shape.split_pages == 0 && v.shape.n_items == 32);
    // 8 of them do not, and are too little work to balance: fixed chunks of 12 pages
    v = plan_and_check(std::vector<uint32_t>(8, 255), 8, 256);
    CHECK(!v.shape.balanced && v.shape.split_pages == 12 && v.shape.n_items == 16);
    // 128 rows of 1K-8K tokens fill the GPU with whole rows
    std::mt19937_64 g(1);
    v = plan_and_check(uniform_rows(g, 128, 1024, 8192), 8, 256);
    CHECK(!v.shape.balanced && v.shape.split_pages == 0 && v.shape.n_items == 128);
    // hundreds of rows with one far longer: more rows than workgroups, so fixed chunks
    auto many = uniform_rows(g, 300, 1, 600);
    many.push_back(200000);
    v = plan_and_check(many, 8, 256);
    CHECK(!v.shape.balanced && v.shape.split_pages > 0);
    for (const auto& segs : v.wg_segments)
        CHECK(segs.size() == 1);
}

TEST("one long row: at most 32 pieces")
{
    for (uint32_t tokens : { 5000u, 32768u, 40960u, 1000000u }) {
        const auto v = plan_and_check({ tokens - 1 }, 8, 256);
        CHECK(v.shape.n_items <= 32);
        CHECK(v.shape.n_records == v.shape.n_items);
        CHECK(v.shape.n_cut == 1);
    }
}

TEST("fixed chunks follow their definition (CKV_DECODE_SPLIT)")
{
    const env_guard e("CKV_DECODE_SPLIT", "5");
    const std::vector<uint32_t> p = { 2999, 699, 63, 2499, 0, 79 };
    const auto v = plan_and_check(p, 8, 256);
    CHECK(!v.shape.balanced && v.shape.split_pages == 5);
    uint32_t items = 0, records = 0;
    for (const uint32_t x : p) {
        const uint32_t n = (pages_of(x) + 4) / 5;
        items += n;
        records += n > 1 ? n : 0;
    }
    CHECK(v.shape.n_items == items && v.shape.n_wgs == items && v.shape.n_records == records);
    for (size_t w = 0; w < v.wg_pages.size(); ++w)
        CHECK(v.wg_pages[w] <= 5);
}

TEST("forced balance: several rows and pieces to a workgroup (CKV_DECODE_BALANCE)")
{
    const std::vector<uint32_t> p = { 0, 15, 16, 31, 32, 111, 112, 126, 499, 1998 };
    {
        const env_guard e("CKV_DECODE_BALANCE", "40");
        const auto v = plan_and_check(p, 8, 256);
        CHECK(v.shape.balanced && v.shape.split_pages == 40);
        size_t most = 0;
        for (const auto& segs : v.wg_segments)
            most = std::max(most, segs.size());
        CHECK(most >= 3);
    }
    {
        const env_guard e("CKV_DECODE_BALANCE", "100000");
        const auto v = plan_and_check(p, 8, 256);
        CHECK(v.shape.n_wgs == 1 && v.shape.n_items == p.size() && v.shape.n_records == 0);
    }
    for (const char* t : { "1", "2", "7" }) {
        const env_guard e("CKV_DECODE_BALANCE", t);
        plan_and_check(p, 8, 256);
    }
}

TEST("random batches at random GPU sizes: every plan is well formed")
{
    std::mt19937_64 g(7);
    for (int t = 0; t < 1500; ++t) {
        std::vector<uint32_t> p(1 + g() % 70);
        for (auto& x : p)
            x = (uint32_t)(g() % ((g() % 3) ? 2000 : 20000));
        const uint32_t heads = 1 + (uint32_t)(g() % 16);
        const int cus = 1 + (int)(g() % 320);
        if (t % 3 == 1) {
            const env_guard e("CKV_DECODE_BALANCE", std::to_string(1 + g() % 90).c_str());
            plan_and_check(p, heads, cus);
        } else if (t % 3 == 2) {
            const env_guard e("CKV_DECODE_SPLIT", std::to_string(g() % 40).c_str());
            plan_and_check(p, heads, cus);
        } else {
            plan_and_check(p, heads, cus);
        }
    }
}

TEST("decode waves per workgroup: cut plans of one workgroup per compute unit take 12")
{
    auto waves = [](const std::vector<uint32_t>& positions, uint32_t group, int dtype) {
        const auto shape = ckv::shape_decode_plan(positions, bs, 8, 256);
        uint64_t pages = 0;
        for (const uint32_t p : positions)
            pages += pages_of(p);
        const uint32_t n_wgs = shape.n_wgs ? shape.n_wgs : (uint32_t)positions.size();
        return ckv::decode_fast_waves(group, dtype, n_wgs * 8, 256,
                                      (uint32_t)(pages / positions.size()), shape.split_pages);
    };
    CHECK(waves({ 32767 }, 2, CKV_BF16) == 12);  // 32 pieces of 64 pages, one per CU
    CHECK(waves({ 65535 }, 2, CKV_BF16) == 12);  // 128 pages each
    CHECK(waves({ 16383 }, 2, CKV_BF16) == 8);   // 32 pages each: under the floor
    CHECK(waves({ 32767 }, 1, CKV_F16) == 12);
    CHECK(waves({ 32767 }, 8, CKV_BF16) == 8);   // wide lanes: 8 at most
    CHECK(waves({ 32767 }, 2, CKV_F32) == 4);
    std::vector<uint32_t> two(2, 40959);         // two long rows: two workgroups per CU
    CHECK(waves(two, 2, CKV_BF16) == 8);
    std::mt19937_64 rng(7);
    std::vector<uint32_t> c2(32), c3(128), churn(512);
    for (auto& p : c2)
        p = 256 + (uint32_t)(rng() % 3841);
    for (auto& p : c3)
        p = 1024 + (uint32_t)(rng() % 7169);
    for (auto& p : churn)
        p = 256 + (uint32_t)(rng() % 1945);
    CHECK(waves(c2, 2, CKV_BF16) == 8);   // config 2: two 8-wave workgroups per CU
    CHECK(waves(c3, 2, CKV_BF16) == 10);  // config 3: whole rows, long on average
    CHECK(waves(churn, 2, CKV_BF16) == 8); // many short whole rows
    {
        const env_guard e("CKV_DECODE_WAVES", "6");
        CHECK(waves({ 32767 }, 2, CKV_BF16) == 6);
    }
}

// ---- the prefill's launch shape and key ranges ---------------------------

namespace {

ckv::prefill_shape_info prefill_shape_for(uint32_t n_tiles, uint32_t kv_heads, uint32_t q_heads,
                                          int cus, int dtype = CKV_BF16, uint32_t tile_blocks = 75)
{
    ckv::pool_view p {};
    p.kv_heads = kv_heads;
    p.head_dim = 128;
    p.block_size = 16;
    p.features = kv_heads * 128;
    p.dtype = dtype;
    ckv::meta_view m {};
    m.n_tiles = n_tiles;
    m.tile_blocks = tile_blocks;
    return ckv::prefill_plan(p, m, q_heads, cus);
}

} // namespace

TEST("prefill key ranges: a partition of the tile's blocks, each range long enough")
{
    for (uint32_t n_blocks = 1; n_blocks <= 1200; ++n_blocks)
        for (uint32_t n_split = 1; n_split <= ckv::split_max; ++n_split)
            for (uint32_t least : { 1u, 2u, 3u, 8u, 16u }) {
                const uint32_t n = ckv::prefill_range_count(n_blocks, n_split, least);
                REQUIRE(n >= 1 && n <= n_split);
                if (n_blocks < 3 * least)
                    CHECK(n == 1);
                uint32_t next = 0;
                for (uint32_t part = 0; part < n; ++part) {
                    uint32_t b = 0, e = 0;
                    ckv::prefill_range_bounds(n_blocks, n, part, b, e);
                    CHECK(b == next);         // contiguous, starting at block 0
                    CHECK(e > b);             // never empty
                    if (n > 1)
                        CHECK(e - b >= least); // at least min_blocks each
                    next = e;
                }
                CHECK(next == n_blocks); // covering every block once
            }
}

TEST("prefill launch shape: 8-wave workgroups when they fill the GPU")
{
    // config 4: 64 sequences x 512 rows = 128 tiles, 8 kv heads, 16 q heads
    const auto c4 = prefill_shape_for(128, 8, 16, 256);
    CHECK(c4.waves == 8 && c4.n_split == 1 && c4.records_floats == 0 && c4.counters == 0);
    // exactly one 8-wave workgroup per compute unit, or whole rounds of them: 8-wave
    CHECK(prefill_shape_for(16, 8, 16, 256).waves == 8);
    CHECK(prefill_shape_for(32, 8, 16, 256).waves == 8);
    CHECK(prefill_shape_for(48, 8, 16, 256).waves == 8);
    // a last round 3/4 full (448 = 1.75 rounds): 8-wave
    CHECK(prefill_shape_for(28, 8, 16, 256).waves == 8);
    // a last round at most 5/8 full under three rounds: 4-wave, no key split
    for (uint32_t tiles : { 18u, 24u, 34u, 40u }) {
        const auto s = prefill_shape_for(tiles, 8, 16, 256);
        CHECK(s.waves == 4 && s.n_split == 1 && s.records_floats == 0);
    }
    // from three rounds on: 8-wave (56 tiles = 3.5 rounds)
    CHECK(prefill_shape_for(56, 8, 16, 256).waves == 8);
    // GQA groups of 8 always take 8-wave workgroups, and f32 pools their own kernel
    CHECK(prefill_shape_for(1, 8, 64, 256).waves == 8);
    CHECK(prefill_shape_for(1, 8, 16, 256, CKV_F32).waves == 8);
    // f32: 8-wave workgroups two to a compute unit; at most one to each splits
    const auto f32_small = prefill_shape_for(1, 8, 16, 256, CKV_F32); // 16 workgroups
    CHECK(f32_small.n_split == ckv::split_max && f32_small.counters == 16);
    CHECK(f32_small.records_floats == 16ull * ckv::split_max * 256 * ckv::prefill_record_floats);
    CHECK(prefill_shape_for(8, 8, 16, 256, CKV_F32).n_split == 4);  // 128 workgroups
    CHECK(prefill_shape_for(16, 8, 16, 256, CKV_F32).n_split == 2); // 256: one per CU
    CHECK(prefill_shape_for(17, 8, 16, 256, CKV_F32).n_split == 1); // 272
    CHECK(prefill_shape_for(128, 8, 16, 256, CKV_F32).n_split == 1); // config 4
}

TEST("prefill launch shape: small launches take 4-wave workgroups and split keys to fill")
{
    // one sequence's 512-row chunk: 2 tiles x 2 x 8 = 32 eight-wave units for 256 CUs
    const auto one = prefill_shape_for(2, 8, 16, 256);
    CHECK(one.waves == 4 && one.n_split == 8 && one.min_blocks == ckv::split_min_blocks);
    // 64 (tile rows, kv head) pairs of 4-wave workgroups, 8 ranges of 128 query vectors
    CHECK(one.counters == 64);
    CHECK(one.records_floats == 64ull * 8 * 128 * ckv::prefill_record_floats);
    // four sequences: 8 tiles -> 256 pairs, two ranges each fill two per compute unit
    const auto four = prefill_shape_for(8, 8, 16, 256);
    CHECK(four.waves == 4 && four.n_split == 2 && four.counters == 256);
    // never more than split_max ranges
    CHECK(prefill_shape_for(1, 1, 1, 256).n_split == ckv::split_max);
    // past half a round (240 units: 480 pairs, no split): 4-wave for short tiles only
    const auto full = prefill_shape_for(15, 8, 16, 256, CKV_BF16, 30);
    CHECK(full.waves == 4 && full.n_split == 1 && full.records_floats == 0);
    CHECK(prefill_shape_for(15, 8, 16, 256, CKV_BF16, 75).waves == 8);
    CHECK(prefill_shape_for(12, 8, 16, 256, CKV_BF16, 40).waves == 4);
    CHECK(prefill_shape_for(12, 8, 16, 256, CKV_BF16, 41).waves == 8);
    // up to half a round: 4-wave whatever the tiles' lengths
    CHECK(prefill_shape_for(8, 8, 16, 256, CKV_BF16, 500).waves == 4);
}

TEST("prefill launch shape: the environment overrides")
{
    {
        const env_guard e("CKV_PREFILL_SPLIT", "3");
        CHECK(prefill_shape_for(2, 8, 16, 256).n_split == 3);
    }
    {
        const env_guard e("CKV_PREFILL_SPLIT", "50");
        CHECK(prefill_shape_for(2, 8, 16, 256).n_split == ckv::split_max);
    }
    {
        const env_guard e("CKV_PREFILL_SPLIT", "0");
        CHECK(prefill_shape_for(2, 8, 16, 256).n_split == 1);
    }
    {
        const env_guard e("CKV_PREFILL_SPLIT_MIN", "2");
        CHECK(prefill_shape_for(2, 8, 16, 256).min_blocks == 2);
    }
    {
        const env_guard e("CKV_PREFILL_WAVES", "8");
        const auto s = prefill_shape_for(2, 8, 16, 256);
        CHECK(s.waves == 8 && s.n_split == 1);
    }
    {
        const env_guard e("CKV_PREFILL_WAVES", "4");
        const auto s = prefill_shape_for(128, 8, 16, 256); // config 4 forced to 4 waves
        CHECK(s.waves == 4 && s.n_split == 1);
    }
}

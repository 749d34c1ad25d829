// In-process A/B of two libckv builds (measurement only): both libraries are
// opened with dlopen, wrap the same device pool and alternate rounds of
// launches on one stream, so the box's own drift cancels out (separate bench
// runs on one box differ by up to several per cent).
//   ab_libckv libA libB [rounds] [launches] [decode|prefill] [layers]
//             [hash|zero|normal] [rows] [lo] [hi]
// decode: rows (default 128) of U[lo, hi] tokens (default config 3's
// [1024, 8192]), or lognormal lengths with LOGNORMAL=median:sigma:max, on
// permuted pages, through ckv_append_decode; prefill: config 4's 64 x 512 rows
// over a 2,000-token prefix (PREFILL_SHAPE=seqs:chunk:prefix for another)
// through ckv_prefill_attention. AB_ENV_A/AB_ENV_B set environment settings
// for one side's launches only. Prints each
// library's time per launch and how many outputs differ.
#include <hip/hip_runtime.h>
#include <dlfcn.h>
#include <cstdio>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <vector>
#include <algorithm>
#include <cmath>
#include <string>

#define CHECK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("hip error %s at %d\n", hipGetErrorString(e), __LINE__); exit(1); } } while (0)

struct ckv_context;
struct ckv_pool;
struct Lib {
    void* h;
    int (*context_create)(int, ckv_context**);
    int (*context_set_stream)(ckv_context*, void*);
    int (*pool_wrap)(ckv_context*, size_t, size_t, size_t, size_t, size_t, int, void*, void*, ckv_pool**);
    int (*tables_upload)(ckv_pool*, const uint32_t*, size_t, const uint32_t*, const uint32_t*, const uint32_t*, const uint32_t*, size_t);
    int (*append_decode)(ckv_pool*, size_t, const void*, const void*, const void*, size_t, float, void*, size_t);
    int (*decode)(ckv_pool*, size_t, const void*, size_t, float, void*, size_t);
    int (*prefill)(ckv_pool*, size_t, const void*, size_t, float, void*, size_t);
    ckv_context* ctx;
    ckv_pool* pool;
};

template <class F> void sym(void* h, F& f, const char* n)
{
    f = reinterpret_cast<F>(dlsym(h, n));
    if (!f) { printf("missing %s\n", n); exit(1); }
}

Lib open_lib(const char* path)
{
    Lib l{};
    l.h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!l.h) { printf("dlopen %s: %s\n", path, dlerror()); exit(1); }
    sym(l.h, l.context_create, "ckv_context_create");
    sym(l.h, l.context_set_stream, "ckv_context_set_stream");
    sym(l.h, l.pool_wrap, "ckv_pool_wrap");
    sym(l.h, l.tables_upload, "ckv_tables_upload");
    sym(l.h, l.append_decode, "ckv_append_decode");
    sym(l.h, l.decode, "ckv_decode_attention");
    sym(l.h, l.prefill, "ckv_prefill_attention");
    return l;
}

__device__ int g_fill_mode = 0; // 0 hash, 1 zero, 2 normal (Box-Muller), bf16
__global__ void fill(uint16_t* p, size_t n, uint32_t seed)
{
    if (g_fill_mode == 1) {
        for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
        return;
    }
    if (g_fill_mode == 2) {
        for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
            uint32_t x = (uint32_t)i * 2654435761u ^ seed, y = (uint32_t)(i >> 32) * 40503u + (uint32_t)i * 2246822519u + seed;
            x ^= x >> 15; x *= 2246822519u; x ^= x >> 13; y ^= y >> 16; y *= 3266489917u; y ^= y >> 15;
            const float u1 = ((x >> 8) + 1) * (1.0f / 16777217.0f), u2 = (y >> 8) * (1.0f / 16777216.0f);
            const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.2831853f * u2);
            uint32_t b; memcpy(&b, &z, 4);
            p[i] = (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
        }
        return;
    }
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        uint32_t x = (uint32_t)i * 2654435761u ^ seed;
        x ^= x >> 15; x *= 2246822519u; x ^= x >> 13;
        // bf16 in about [-2, 2]: sign, exponent 126..128, random mantissa
        p[i] = (uint16_t)(((x & 1) << 15) | ((126 + (x >> 1) % 3) << 7) | ((x >> 8) & 0x7F));
    }
}

int main(int argc, char** argv)
{
    if (argc < 3) { printf("usage: abtest libA libB [rounds] [launches]\n"); return 1; }
    const int rounds = argc > 3 ? atoi(argv[3]) : 10;
    const int launches = argc > 4 ? atoi(argv[4]) : 20;
    const bool pre = argc > 5 && !strcmp(argv[5], "prefill");
    const uint32_t L = argc > 6 ? (uint32_t)atoi(argv[6]) : 1;
    const int fill_mode = argc > 7 ? (!strcmp(argv[7], "zero") ? 1 : !strcmp(argv[7], "normal") ? 2 : 0) : 0;
    CHECK(hipMemcpyToSymbol(HIP_SYMBOL(g_fill_mode), &fill_mode, sizeof(int)));
    const uint32_t H = 8, D = 128, Hq = 16, BS = 16, F = H * D;
    uint64_t s = 12345;
    auto rnd = [&]() { s = s * 6364136223846793005ull + 1442695040888963407ull; return (uint32_t)(s >> 33); };
    std::vector<uint32_t> len, table, off, lens, pos, slot;
    size_t blocks = 0;
    uint32_t B = 0;
    double kv_bytes = 0, flops = 0;
    if (!pre) {
        B = argc > 8 ? (uint32_t)atoi(argv[8]) : 128;
        const uint32_t lo = argc > 9 ? (uint32_t)atoi(argv[9]) : 1024, hi = argc > 10 ? (uint32_t)atoi(argv[10]) : 8192;
        len.resize(B);
        size_t pages = 0;
        // LOGNORMAL=median:sigma:max: churn-like lengths instead of U[lo, hi]
        const char* ln = getenv("LOGNORMAL");
        double med = 0, sig = 0, mx = 0;
        if (ln) sscanf(ln, "%lf:%lf:%lf", &med, &sig, &mx);
        for (auto& n : len) {
            if (ln) {
                double u1 = (rnd() + 1.0) / 2147483649.0, u2 = rnd() / 2147483648.0;
                double z = sqrt(-2 * log(u1)) * cos(6.283185307 * u2);
                n = (uint32_t)std::min(mx, std::max(16.0, med * exp(sig * z)));
            } else n = lo + rnd() % (hi - lo + 1);
            pages += (n + BS - 1) / BS;
        }
        blocks = pages + 64;
        std::vector<uint32_t> perm(blocks);
        for (size_t i = 0; i < blocks; ++i) perm[i] = (uint32_t)i;
        for (size_t i = blocks - 1; i > 0; --i) std::swap(perm[i], perm[rnd() % (i + 1)]);
        off.resize(B); lens.resize(B); pos.resize(B); slot.resize(B);
        size_t at = 0;
        for (uint32_t r = 0; r < B; ++r) {
            const uint32_t np = (len[r] + BS - 1) / BS;
            off[r] = (uint32_t)table.size();
            lens[r] = np;
            for (uint32_t p = 0; p < np; ++p) table.push_back(perm[at++]);
            pos[r] = len[r] - 1;
            slot[r] = table[off[r] + pos[r] / BS] * BS + pos[r] % BS;
        }
        for (auto n : len) kv_bytes += (double)n * F * 2 * 2;
    } else {
        // config 4: 64 sequences x 512 rows at positions 2000..2511 over a shared 125-page prefix;
        // PREFILL_SHAPE=seqs:chunk:prefix (multiples of 16) for another shape
        uint32_t seqs = 64, chunk = 512, prefix = 2000;
        if (const char* shape = getenv("PREFILL_SHAPE"))
            sscanf(shape, "%u:%u:%u", &seqs, &chunk, &prefix);
        const uint32_t pp = prefix / BS, cp = chunk / BS;
        blocks = pp + (size_t)seqs * cp;
        std::vector<uint32_t> seq_table(seqs * (pp + cp));
        for (uint32_t q = 0; q < seqs; ++q)
            for (uint32_t p = 0; p < pp + cp; ++p)
                seq_table[q * (pp + cp) + p] = p < pp ? p : pp + q * cp + (p - pp);
        table = seq_table;
        B = seqs * chunk;
        for (uint32_t q = 0; q < seqs; ++q)
            for (uint32_t r = 0; r < chunk; ++r) {
                off.push_back(q * (pp + cp));
                lens.push_back(pp + cp);
                pos.push_back(prefix + r);
                flops += 4.0 * D * Hq * (prefix + r + 1);
            }
        slot.clear();
    }
    const size_t elems = (size_t)L * blocks * BS * F;
    void *kp, *vp, *kin, *vin, *q, *outA, *outB;
    CHECK(hipMalloc(&kp, elems * 2));
    CHECK(hipMalloc(&vp, elems * 2));
    CHECK(hipMalloc(&kin, (size_t)B * F * 2));
    CHECK(hipMalloc(&vin, (size_t)B * F * 2));
    CHECK(hipMalloc(&q, (size_t)B * Hq * D * 2));
    CHECK(hipMalloc(&outA, (size_t)B * Hq * D * 2));
    CHECK(hipMalloc(&outB, (size_t)B * Hq * D * 2));
    hipLaunchKernelGGL(fill, dim3(16384), dim3(256), 0, 0, (uint16_t*)kp, elems, 1u);
    hipLaunchKernelGGL(fill, dim3(16384), dim3(256), 0, 0, (uint16_t*)vp, elems, 2u);
    hipLaunchKernelGGL(fill, dim3(256), dim3(256), 0, 0, (uint16_t*)kin, (size_t)B * F, 3u);
    hipLaunchKernelGGL(fill, dim3(256), dim3(256), 0, 0, (uint16_t*)vin, (size_t)B * F, 4u);
    hipLaunchKernelGGL(fill, dim3(256), dim3(256), 0, 0, (uint16_t*)q, (size_t)B * Hq * D, 5u);
    CHECK(hipDeviceSynchronize());
    hipStream_t st;
    CHECK(hipStreamCreate(&st));
    Lib libs[2] = { open_lib(argv[1]), open_lib(argv[2]) };
    void* outs[2] = { outA, outB };
    // AB_ENV_A / AB_ENV_B = "NAME=value,NAME=value": set before that library's
    // launches and cleared before the other's (the libraries read such
    // settings at each launch), so one library can be compared with itself
    // under two settings
    auto apply_env = [&](int i) {
        for (int pass = 0; pass < 2; ++pass) { // clear the other side's names, then set ours
            const char* spec = getenv(pass ? (i ? "AB_ENV_B" : "AB_ENV_A") : (i ? "AB_ENV_A" : "AB_ENV_B"));
            if (!spec)
                continue;
            std::string all(spec);
            size_t at = 0;
            while (at < all.size()) {
                size_t end = all.find(',', at);
                if (end == std::string::npos)
                    end = all.size();
                const std::string item = all.substr(at, end - at);
                const size_t eq = item.find('=');
                if (eq != std::string::npos) {
                    const std::string name = item.substr(0, eq);
                    if (pass)
                        setenv(name.c_str(), item.substr(eq + 1).c_str(), 1);
                    else
                        unsetenv(name.c_str());
                }
                at = end + 1;
            }
        }
    };
    // each side's settings apply from its pool's table upload on (the decode
    // plan is built there)
    for (int i = 0; i < 2; ++i) {
        Lib& l = libs[i];
        apply_env(i);
        if (l.context_create(0, &l.ctx) || l.context_set_stream(l.ctx, st)
            || l.pool_wrap(l.ctx, L, blocks, BS, H, D, 1, kp, vp, &l.pool)
            || l.tables_upload(l.pool, table.data(), table.size(), off.data(), lens.data(), pos.data(), pre ? nullptr : slot.data(), B)) {
            printf("setup failed\n");
            return 1;
        }
    }
    if (!pre)
        for (int i = 0; i < 2; ++i) {
            auto plan = reinterpret_cast<int (*)(void*, uint32_t*, uint32_t*, uint32_t*)>(
                dlsym(libs[i].h, "ckv_decode_plan"));
            uint32_t sp = 0, wi = 0, rec = 0;
            if (plan && plan(libs[i].pool, &sp, &wi, &rec) == 0)
                printf("%s plan: %u pages per workgroup, %u work items, %u records\n",
                       i ? "B" : "A", sp, wi, rec);
        }
    const float scale = 0.08838834764831845f;
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    double tot[2] = { 0, 0 };
    for (int r = -1; r < rounds; ++r) {
        for (int k = 0; k < 2; ++k) {
            const int i = (r & 1) ? 1 - k : k; // alternate which goes first
            apply_env(i);
            CHECK(hipEventRecord(e0, st));
            for (int j = 0; j < launches; ++j)
                if (pre ? libs[i].prefill(libs[i].pool, j % L, q, Hq, scale, outs[i], B)
                        : libs[i].append_decode(libs[i].pool, j % L, kin, vin, q, Hq, scale, outs[i], B)) { printf("launch failed\n"); return 1; }
            CHECK(hipEventRecord(e1, st));
            CHECK(hipEventSynchronize(e1));
            float ms;
            CHECK(hipEventElapsedTime(&ms, e0, e1));
            if (r >= 0) tot[i] += ms;
        }
    }
    if (const char* dump = getenv("DUMP_TS")) {
        auto f = reinterpret_cast<int (*)(void*, size_t)>(dlsym(libs[0].h, "ckv_debug_times"));
        if (f) {
            std::vector<unsigned long long> ts(65536 * 4);
            CHECK(hipDeviceSynchronize());
            if (f(ts.data(), 65536) == 0) {
                FILE* fo = fopen(dump, "wb");
                fwrite(ts.data(), 8, ts.size(), fo);
                fclose(fo);
                printf("timestamps written to %s\n", dump);
            }
        }
    }
    std::vector<uint16_t> ha((size_t)B * Hq * D), hb((size_t)B * Hq * D);
    CHECK(hipMemcpy(ha.data(), outA, ha.size() * 2, hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(hb.data(), outB, hb.size() * 2, hipMemcpyDeviceToHost));
    size_t diff = 0;
    double maxd = 0, maxv = 0;
    auto bf = [](uint16_t b) { uint32_t u = (uint32_t)b << 16; float f; memcpy(&f, &u, 4); return (double)f; };
    for (size_t i = 0; i < ha.size(); ++i) {
        diff += ha[i] != hb[i];
        maxd = std::max(maxd, std::fabs(bf(ha[i]) - bf(hb[i])));
        maxv = std::max(maxv, std::fabs(bf(ha[i])));
    }
    printf("max |A-B| %.3g (max |A| %.3g)\n", maxd, maxv);
    for (int i = 0; i < 2; ++i) {
        const double us = tot[i] * 1e3 / (rounds * launches);
        if (pre)
            printf("%s: %.2f us per launch, %.1f TFLOP/s\n", i ? "B" : "A", us, flops / (us * 1e-6) / 1e12);
        else
            printf("%s: %.2f us per launch, %.1f GB/s KV\n", i ? "B" : "A", us, kv_bytes / (us * 1e-6) / 1e9);
    }
    printf("B/A time ratio %.4f; outputs differing: %zu of %zu\n", tot[1] / tot[0], diff, ha.size());
    return 0;
}

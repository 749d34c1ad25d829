// The chunked prefill's instruction mix without its dependences (measurement
// only, outside libckv): per group of 4 MFMAs (4 independent accumulators),
// B ds_read_b128, T pairs of ds_read_b64_tr_b16, NV v_fma_f32 and NE
// v_exp_f32, all independent of one another. "A" is the per-wave mix of
// prefill_kernel (per 32-key block: 16 MFMAs, 8 K and 16 transposed V reads,
// about 62 vector instructions and 16 exponentials) at 2 waves per SIMD; "B"
// the mix of one wave per SIMD holding two 32-query blocks (the K and V reads
// shared by both). Prints the MFMA utilisation each mix allows.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <vector>
#include <algorithm>
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
#define CHECK(x) do { hipError_t e=(x); if(e!=hipSuccess){printf("err %s line %d\n",hipGetErrorString(e),__LINE__); return 1;} } while(0)

template <int B, int T, int NV, int NE>
__global__ __launch_bounds__(512) void mix(float* out, unsigned long long* ts, int iters)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    for (int i = threadIdx.x; i < 32768; i += blockDim.x) reinterpret_cast<int*>(lds)[i] = i;
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    i32x4 a = {(int)threadIdx.x, 1, 2, 3}, b = {4, 5, (int)threadIdx.x, 7};
    float x[8];
    for (int i = 0; i < 8; ++i) x[i] = threadIdx.x * 0.001f + i;
    const float y = out[0], z = out[1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds + lane * 16 + (wave & 3) * 8192;
    __syncthreads();
    unsigned long long t0 = __builtin_readcyclecounter();
    unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
            asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c0) : "v"(a), "v"(b));
#pragma unroll
            for (int j = 0; j < B; ++j) { i32x4 v; asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(base + ((grp * B + j) & 7) * 1024)); }
            asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c1) : "v"(a), "v"(b));
#pragma unroll
            for (int j = 0; j < T; ++j) { i32x2 lo, hi; asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(lo) : "v"(base + ((grp + j) & 7) * 512)); asm volatile("ds_read_b64_tr_b16 %0, %1 offset:256" : "=v"(hi) : "v"(base + ((grp + j) & 7) * 512)); }
#pragma unroll
            for (int j = 0; j < NV / 2; ++j) asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x[j & 7]) : "v"(y), "v"(z));
#pragma unroll
            for (int j = 0; j < NE / 2; ++j) asm volatile("v_exp_f32 %0, %0" : "+v"(x[(j + 3) & 7]));
            asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c2) : "v"(a), "v"(b));
#pragma unroll
            for (int j = 0; j < NV - NV / 2; ++j) asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x[(j + 5) & 7]) : "v"(y), "v"(z));
            asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c3) : "v"(a), "v"(b));
#pragma unroll
            for (int j = 0; j < NE - NE / 2; ++j) asm volatile("v_exp_f32 %0, %0" : "+v"(x[(j + 1) & 7]));
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    unsigned long long t1 = __builtin_readcyclecounter();
    unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    f32x16 t = c0 + c1 + c2 + c3;
    float s = 0;
    for (int i = 0; i < 8; ++i) s += x[i];
    for (int i = 0; i < 16; ++i) s += t[i];
    if (s == 1234.5f) out[2 + threadIdx.x] = s;
    if (lane == 0) {
        unsigned long long* p = ts + 4 * (blockIdx.x * 16 + wave);
        p[0] = t0; p[1] = t1; p[2] = r0; p[3] = r1;
    }
}

template <int B, int T, int NV, int NE>
int run(int wps, float* out, unsigned long long* ts, const char* name)
{
    const int iters = 1000, threads = 256 * wps;
    const size_t shm = 128 * 1024;
    auto k = mix<B, T, NV, NE>;
    CHECK(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, shm));
    hipLaunchKernelGGL(k, dim3(256), dim3(threads), shm, 0, out, ts, 50);
    CHECK(hipDeviceSynchronize());
    hipLaunchKernelGGL(k, dim3(256), dim3(threads), shm, 0, out, ts, iters);
    CHECK(hipDeviceSynchronize());
    std::vector<unsigned long long> h(256 * 16 * 4);
    CHECK(hipMemcpy(h.data(), ts, h.size() * 8, hipMemcpyDeviceToHost));
    double span = 0;
    for (int g = 0; g < 256; ++g) {
        unsigned long long a0 = ~0ull, a1 = 0;
        for (int w = 0; w < 4 * wps; ++w) { const unsigned long long* p = &h[4 * (g * 16 + w)]; a0 = std::min(a0, p[0]); a1 = std::max(a1, p[1]); }
        span += a1 - a0;
    }
    span /= 256;
    // one iteration = 16 MFMAs per wave; per SIMD wps*16 MFMAs (512 cycles each 16)
    const double per_iter = span / iters;
    printf("%-10s wps=%d B=%d T=%d NV=%2d NE=%d : %7.1f cyc/iter/SIMD for %d MFMA -> MFMA util %.1f%%\n",
           name, wps, B, T, NV, NE, per_iter, 16 * wps, 100.0 * 32 * 16 * wps / per_iter);
    fflush(stdout);
    return 0;
}

int main()
{
    float* out; unsigned long long* ts;
    CHECK(hipMalloc(&out, 1 << 20)); CHECK(hipMemset(out, 0, 1 << 20));
    CHECK(hipMalloc(&ts, 256 * 16 * 4 * 8));
    // A: today's mix per wave (per 4 MFMA: 2 b128, 2 tr pairs, ~16 VALU, 4 exp), 2 waves/SIMD
    run<2, 2, 16, 4>(2, out, ts, "A today");
    run<0, 0, 16, 4>(2, out, ts, "A no LDS");
    run<2, 2, 0, 0>(2, out, ts, "A no VALU");
    // B: v2 mix (per 4 MFMA: 1 b128, 1 tr pair, 16 VALU, 4 exp), 1 wave/SIMD
    run<1, 1, 16, 4>(1, out, ts, "B v2");
    run<1, 1, 12, 4>(1, out, ts, "B v2 -4v");
    run<0, 0, 16, 4>(1, out, ts, "B no LDS");
    // C: v2 mix on 2 waves/SIMD (if registers allowed)
    run<1, 1, 16, 4>(2, out, ts, "C");
    printf("done\n");
    return 0;
}

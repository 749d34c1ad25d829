// Whether LDS operand reads overlap v_mfma_f32_32x32x16_bf16 on gfx950
// (measurement only, outside libckv). One workgroup of 8 waves (2 per SIMD)
// per compute unit; per wave and iteration 8 MFMAs (4 independent
// accumulators) and, per MFMA, R reads of 1 KiB per wave, either ds_read_b128
// or two ds_read_b64_tr_b16 (the prefill's transposed V read), to addresses
// inside a 128 KiB LDS array; one lgkmcnt wait per iteration. Prints cycles
// per iteration per SIMD and the LDS bytes per clock per compute unit.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <vector>
#include <algorithm>
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
#define CHECK(x) do { hipError_t e=(x); if(e!=hipSuccess){printf("err %s line %d\n",hipGetErrorString(e),__LINE__); return 1;} } while(0)

template <int R, int ACC, bool MF, int TR>  // R LDS reads per MFMA; TR: 0 b128, 1 two tr_b64
__global__ __launch_bounds__(512) void mb(float* out, unsigned long long* ts, int iters)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    for (int i = threadIdx.x; i < 32768; i += blockDim.x) reinterpret_cast<int*>(lds)[i] = i;
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    i32x4 a = {(int)threadIdx.x, 1, 2, 3}, b = {4, 5, (int)threadIdx.x, 7};
    i32x4 acc4 = {};
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds + lane * 16 + (wave & 3) * 8192;
    __syncthreads();
    unsigned long long t0 = __builtin_readcyclecounter();
    unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            if constexpr (MF) {
#define MF1(c) do { if constexpr (ACC) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b)); \
                    else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b)); } while (0)
                if ((m & 3) == 0) MF1(c0); else if ((m & 3) == 1) MF1(c1); else if ((m & 3) == 2) MF1(c2); else MF1(c3);
            }
#pragma unroll
            for (int j = 0; j < R; ++j) {
                i32x4 v;
                const uint32_t addr = base + ((m * R + j) & 7) * 1024;
                if constexpr (TR == 0) {
                    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
                } else {
                    i32x2 lo, hi;
                    asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(lo) : "v"(addr));
                    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:256" : "=v"(hi) : "v"(addr));
                    v = i32x4 {lo.x, lo.y, hi.x, hi.y};
                }
                acc4 ^= v; // consumed late: forces a wait only at the next use
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    unsigned long long t1 = __builtin_readcyclecounter();
    unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    f32x16 t = c0 + c1 + c2 + c3;
    float s = (float)(acc4.x + acc4.y + acc4.z + acc4.w);
    for (int i = 0; i < 16; ++i) s += t[i];
    if (s == 1234.5f) out[2 + threadIdx.x] = s;
    if (lane == 0) {
        unsigned long long* p = ts + 4 * (blockIdx.x * 16 + wave);
        p[0] = t0; p[1] = t1; p[2] = r0; p[3] = r1;
    }
}

template <int R, int ACC, bool MF, int TR>
int run(float* out, unsigned long long* ts, const char* name)
{
    const int iters = 2000, threads = 512;
    const size_t shm = 128 * 1024;
    auto k = mb<R, ACC, MF, TR>;
    CHECK(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, shm));
    hipLaunchKernelGGL(k, dim3(256), dim3(threads), shm, 0, out, ts, 100);
    CHECK(hipDeviceSynchronize());
    hipLaunchKernelGGL(k, dim3(256), dim3(threads), shm, 0, out, ts, iters);
    CHECK(hipDeviceSynchronize());
    std::vector<unsigned long long> h(256 * 16 * 4);
    CHECK(hipMemcpy(h.data(), ts, h.size() * 8, hipMemcpyDeviceToHost));
    double span = 0, rspan = 0;
    for (int g = 0; g < 256; ++g) {
        unsigned long long a0 = ~0ull, a1 = 0, b0 = ~0ull, b1 = 0;
        for (int w = 0; w < 8; ++w) {
            const unsigned long long* p = &h[4 * (g * 16 + w)];
            a0 = std::min(a0, p[0]); a1 = std::max(a1, p[1]);
            b0 = std::min(b0, p[2]); b1 = std::max(b1, p[3]);
        }
        span += a1 - a0; rspan += b1 - b0;
    }
    span /= 256; rspan /= 256;
    const double per_iter = span / iters;
    const double kb = 2.0 * 8 * R * 1024 * 4; // bytes per iteration per CU: 4 SIMDs x 2 waves x 8R KiB
    printf("%-18s R=%d acc=%s tr=%d : %7.1f cyc/iter per SIMD (16 MFMA = 512 at peak), LDS %6.1f B/clk/CU, %.2f GHz\n",
           name, R, ACC ? "a" : "v", TR, per_iter, MF || R ? kb / per_iter : 0.0, span / (rspan * 10.0));
    fflush(stdout);
    return 0;
}

int main()
{
    float* out; unsigned long long* ts;
    CHECK(hipMalloc(&out, 1 << 20)); CHECK(hipMemset(out, 0, 1 << 20));
    CHECK(hipMalloc(&ts, 256 * 16 * 4 * 8));
    run<0, 0, true, 0>(out, ts, "mfma only");
    run<1, 0, false, 0>(out, ts, "lds b128 only");
    run<2, 0, false, 0>(out, ts, "lds b128 only");
    run<1, 0, false, 1>(out, ts, "lds tr only");
    run<1, 0, true, 0>(out, ts, "mfma+lds b128");
    run<1, 1, true, 0>(out, ts, "mfma+lds b128");
    run<2, 0, true, 0>(out, ts, "mfma+lds b128");
    run<2, 1, true, 0>(out, ts, "mfma+lds b128");
    run<1, 0, true, 1>(out, ts, "mfma+lds tr");
    run<1, 1, true, 1>(out, ts, "mfma+lds tr");
    printf("done\n");
    return 0;
}

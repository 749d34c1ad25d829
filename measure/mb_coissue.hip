// How much vector work a gfx950 SIMD issues while its matrix core runs
// v_mfma_f32_32x32x16_bf16 (measurement only, outside libckv; the prefill's
// schedule is judged against it). One workgroup per compute unit of 1, 2 or 4
// waves per SIMD; per wave and iteration 8 MFMAs (4 independent accumulators)
// and, per MFMA, NV independent v_fma_f32 and NE v_exp_f32:
//   mfma only / fma only / exp only: each unit alone;
//   mixed: every wave issues both;
//   split: waves 0-3 (and 8-11) the MFMAs only, waves 4-7 (and 12-15) the
//          vector work only (a wave and the wave four above it share a SIMD).
// Prints the workgroup span per iteration in shader cycles (s_memtime), the
// fastest and slowest wave, and the clock against s_memrealtime (100 MHz).
// Operands are registers; the MFMA results are not read back, so nothing
// depends on their values.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <vector>
#include <algorithm>
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
#define CHECK(x) do { hipError_t e=(x); if(e!=hipSuccess){printf("err %s line %d\n",hipGetErrorString(e),__LINE__); return 1;} } while(0)

template <int NV, int NE, bool DO_MF, bool DO_V>
__device__ __forceinline__ void body(int iters, f32x16& c0, f32x16& c1, f32x16& c2, f32x16& c3, i32x4 a, i32x4 b, float (&x)[8], float y, float z)
{
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            if constexpr (DO_MF) {
                if ((m & 3) == 0) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c0) : "v"(a), "v"(b));
                else if ((m & 3) == 1) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c1) : "v"(a), "v"(b));
                else if ((m & 3) == 2) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c2) : "v"(a), "v"(b));
                else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c3) : "v"(a), "v"(b));
            }
            if constexpr (DO_V) {
#pragma unroll
                for (int j = 0; j < NV; ++j)
                    asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x[j & 7]) : "v"(y), "v"(z));
#pragma unroll
                for (int j = 0; j < NE; ++j)
                    asm volatile("v_exp_f32 %0, %0" : "+v"(x[(j + 3) & 7]));
            }
        }
    }
}

template <int NV, int NE, int MODE> // MODE 0 mixed, 1 split, 2 mfma only, 3 valu only
__global__ __launch_bounds__(1024) void mb(float* out, unsigned long long* ts, int iters)
{
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    i32x4 a = {(int)threadIdx.x, 1, 2, 3}, b = {4, 5, (int)threadIdx.x, 7};
    float x[8];
    for (int i = 0; i < 8; ++i) x[i] = threadIdx.x * 0.001f + i;
    const float y = out[0], z = out[1];
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    unsigned long long t0 = __builtin_readcyclecounter();
    unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    if constexpr (MODE == 0) body<NV, NE, true, true>(iters, c0, c1, c2, c3, a, b, x, y, z);
    else if constexpr (MODE == 2) body<NV, NE, true, false>(iters, c0, c1, c2, c3, a, b, x, y, z);
    else if constexpr (MODE == 3) body<NV, NE, false, true>(iters, c0, c1, c2, c3, a, b, x, y, z);
    else {
        if ((wave >> 2) & 1) body<NV, NE, false, true>(iters, c0, c1, c2, c3, a, b, x, y, z);
        else body<NV, NE, true, false>(iters, c0, c1, c2, c3, a, b, x, y, z);
    }
    unsigned long long t1 = __builtin_readcyclecounter();
    unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0;
    for (int i = 0; i < 8; ++i) s += x[i];
    f32x16 t = c0 + c1 + c2 + c3;
    for (int i = 0; i < 16; ++i) s += t[i];
    if (s == 1234.5f) out[2 + threadIdx.x] = s;
    if ((threadIdx.x & 63) == 0) {
        unsigned long long* p = ts + 4 * (blockIdx.x * 16 + wave);
        p[0] = t0; p[1] = t1; p[2] = r0; p[3] = r1;
    }
}

template <int NV, int NE, int MODE>
int run(int wps, float* out, unsigned long long* ts, const char* name)
{
    const int iters = 4000;
    const int threads = 256 * wps;
    const size_t shm = 100 * 1024;
    auto k = mb<NV, NE, MODE>;
    CHECK(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, shm));
    hipLaunchKernelGGL(k, dim3(256), dim3(threads), shm, 0, out, ts, 200);
    CHECK(hipDeviceSynchronize());
    hipLaunchKernelGGL(k, dim3(256), dim3(threads), shm, 0, out, ts, iters);
    CHECK(hipDeviceSynchronize());
    std::vector<unsigned long long> h(256 * 16 * 4);
    CHECK(hipMemcpy(h.data(), ts, h.size() * 8, hipMemcpyDeviceToHost));
    double span = 0, rspan = 0, wmin = 0, wmax = 0;
    const int nw = 4 * wps;
    for (int g = 0; g < 256; ++g) {
        unsigned long long a0 = ~0ull, a1 = 0, b0 = ~0ull, b1 = 0, dmin = ~0ull, dmax = 0;
        for (int w = 0; w < nw; ++w) {
            const unsigned long long* p = &h[4 * (g * 16 + w)];
            a0 = std::min(a0, p[0]); a1 = std::max(a1, p[1]);
            b0 = std::min(b0, p[2]); b1 = std::max(b1, p[3]);
            dmin = std::min(dmin, p[1] - p[0]); dmax = std::max(dmax, p[1] - p[0]);
        }
        span += a1 - a0; rspan += b1 - b0; wmin += dmin; wmax += dmax;
    }
    span /= 256; rspan /= 256; wmin /= 256; wmax /= 256;
    // per SIMD per iteration: wps waves' MFMAs (mixed) or the MFMA waves' (split: wps/2 per SIMD)
    const double per_iter = span / iters;
    printf("%-22s wps=%d NV=%2d NE=%d : span %7.1f cyc/iter (waves %6.1f..%6.1f), %.2f GHz\n",
           name, wps, NV, NE, per_iter, wmin / iters, wmax / iters, span / (rspan * 10.0));
    fflush(stdout);
    return 0;
}

int main()
{
    float* out; unsigned long long* ts;
    CHECK(hipMalloc(&out, 1 << 20)); CHECK(hipMemset(out, 0, 1 << 20));
    CHECK(hipMalloc(&ts, 256 * 16 * 4 * 8));
    printf("mixed: each wave 8 MFMA/iter + NV fma + NE exp per MFMA; split: half the waves MFMA only, half VALU only\n");
    for (int wps = 1; wps <= 4; wps *= 2) {
        run<0, 0, 2>(wps, out, ts, "mfma only");
        run<8, 0, 3>(wps, out, ts, "fma only");
        run<0, 4, 3>(wps, out, ts, "exp only");
        run<4, 0, 0>(wps, out, ts, "mixed fma");
        run<6, 0, 0>(wps, out, ts, "mixed fma");
        run<8, 0, 0>(wps, out, ts, "mixed fma");
        run<12, 0, 0>(wps, out, ts, "mixed fma");
        run<4, 2, 0>(wps, out, ts, "mixed fma+exp");
        run<3, 1, 0>(wps, out, ts, "mixed fma+exp");
        if (wps >= 2) {
            run<4, 0, 1>(wps, out, ts, "split fma");
            run<6, 0, 1>(wps, out, ts, "split fma");
            run<8, 0, 1>(wps, out, ts, "split fma");
            run<12, 0, 1>(wps, out, ts, "split fma");
            run<16, 0, 1>(wps, out, ts, "split fma");
            run<4, 2, 1>(wps, out, ts, "split fma+exp");
            run<8, 4, 1>(wps, out, ts, "split fma+exp");
        }
    }
    printf("done\n");
    return 0;
}

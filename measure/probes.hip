// Hardware ceilings the kernels are judged against, measured on the part
// itself: libckv_probes.so, outside the libckv boundary (no counterpart in the
// reference; `bench.py --workload ceiling` drives it).
//
//   ckv_probe_read   one pass over a buffer with 16-byte loads (plain or
//                    nontemporal): the HBM read rate a streaming kernel reaches.
//   ckv_probe_pages  the decode's access pattern without its arithmetic: each
//                    workgroup walks a list of pages of a K and a V tensor and
//                    reads one slice of every token row (a kv head's 256 bytes
//                    of a 2 KiB row, or the whole row), its waves taking pages
//                    in turn, two pages in flight per wave, nontemporal.
//   ckv_probe_mfma   back-to-back v_mfma_f32_32x32x16_bf16 on register operands:
//                    the matrix cores' rate at this clock.
//
// Every kernel reduces what it reads into one word that is stored only when it
// equals a constant, so the loads cannot be dropped and nothing is written.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr uint32_t never = 0x9E3779B9u;

__device__ __forceinline__ uint32_t fold(u32x4_t x)
{
    return x.x ^ x.y ^ x.z ^ x.w;
}

template <bool NT>
__device__ __forceinline__ u32x4_t load16(const u32x4_t* p)
{
    if constexpr (NT)
        return __builtin_nontemporal_load(p);
    else
        return *p;
}

// Grid-stride pass, four independent 16-byte loads per lane per step.
template <bool NT>
__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4_t* __restrict__ src,
                                                         size_t n16, uint32_t* sink)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4_t a = load16<NT>(src + i), b = load16<NT>(src + i + stride);
        const u32x4_t c = load16<NT>(src + i + 2 * stride), d = load16<NT>(src + i + 3 * stride);
        acc ^= fold(a) ^ fold(b) ^ fold(c) ^ fold(d);
    }
    for (; i < n16; i += stride)
        acc ^= fold(load16<NT>(src + i));
    if (acc == never)
        sink[0] = acc;
}

// Workgroup b: pages [g * per_wg, (g + 1) * per_wg) of the list (g = b / slices)
// and slice b % slices of every token row; chunk c of a page (16 bytes) is
// row c / cpr, 16-byte column c % cpr of the slice. chunks (rows x cpr) is a
// multiple of 256, so each lane takes four chunks per step.
__global__ __launch_bounds__(1024) void probe_pages_kernel(
    const uint8_t* __restrict__ keys, const uint8_t* __restrict__ values, uint32_t pool_pages,
    const uint32_t* __restrict__ pages, uint32_t n_pages, uint32_t page_bytes, uint32_t row_bytes,
    uint32_t slice_bytes, uint32_t per_wg, uint32_t* sink)
{
    extern __shared__ uint32_t reserved[]; // held only to cap the workgroups per CU
    const uint32_t slices = row_bytes / slice_bytes;
    const uint32_t g = blockIdx.x / slices, s = blockIdx.x % slices;
    const uint32_t first = g * per_wg;
    const uint32_t end = min(first + per_wg, n_pages);
    const uint32_t W = blockDim.x >> 6;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t cpr = slice_bytes / 16;
    const uint32_t chunks = (page_bytes / row_bytes) * cpr;
    auto offset = [&](uint32_t c) { return (c / cpr) * row_bytes + s * slice_bytes + (c % cpr) * 16; };
    uint32_t acc = 0;
    for (uint32_t i = first + wave; i < end; i += 2 * W) {
        const bool two = i + W < end;
        // a list entry past the pool would be a caller's error: clamp it
        const uint64_t p0 = (uint64_t)min(pages[i], pool_pages - 1) * page_bytes;
        const uint64_t p1 = (uint64_t)min(pages[two ? i + W : i], pool_pages - 1) * page_bytes;
        for (uint32_t c0 = 0; c0 < chunks; c0 += 256) {
            u32x4_t k0[4], v0[4], k1[4], v1[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t off = offset(c0 + lane + 64 * j);
                k0[j] = load16<true>(reinterpret_cast<const u32x4_t*>(keys + p0 + off));
                v0[j] = load16<true>(reinterpret_cast<const u32x4_t*>(values + p0 + off));
            }
            if (two) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t off = offset(c0 + lane + 64 * j);
                    k1[j] = load16<true>(reinterpret_cast<const u32x4_t*>(keys + p1 + off));
                    v1[j] = load16<true>(reinterpret_cast<const u32x4_t*>(values + p1 + off));
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc ^= fold(k1[j]) ^ fold(v1[j]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc ^= fold(k0[j]) ^ fold(v0[j]);
        }
    }
    if (acc == never)
        sink[0] = acc;
}

// `chains` independent accumulation chains of `iters` products per wave.
template <int CHAINS>
__global__ __launch_bounds__(1024) void probe_mfma_kernel(uint32_t iters, float* sink)
{
    const uint32_t lane = threadIdx.x & 63;
    u32x4_t bits = { lane * 0x00010001u, lane ^ 0x3F803F80u, 0x3F003F00u + lane, 0x3E803E80u };
    const bf16x8_t a = __builtin_bit_cast(bf16x8_t, bits);
    bits.x ^= 0x00400040u;
    const bf16x8_t b = __builtin_bit_cast(bf16x8_t, bits);
    f32x16_t c[CHAINS];
#pragma unroll
    for (int k = 0; k < CHAINS; ++k)
        c[k] = f32x16_t {};
    for (uint32_t i = 0; i < iters; ++i)
#pragma unroll
        for (int k = 0; k < CHAINS; ++k)
            c[k] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[k], 0, 0, 0);
    float x = 0.0f;
#pragma unroll
    for (int k = 0; k < CHAINS; ++k)
        x += c[k][0] + c[k][15];
    if (x == 1234.5f)
        sink[0] = x;
}

bool aligned16(const void* p)
{
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

} // namespace

extern "C" {

// One pass over `bytes` (a multiple of 16) at `src` (16-byte aligned) with
// `grid` workgroups of 256 threads. `sink`: one device word, never written
// in practice. Returns a hipError_t.
int ckv_probe_read(const void* src, size_t bytes, int nontemporal, uint32_t grid, void* sink,
                   void* stream)
{
    if (!src || !sink || !aligned16(src) || bytes % 16 || !grid)
        return hipErrorInvalidValue;
    const auto s = static_cast<hipStream_t>(stream);
    const auto* p = static_cast<const u32x4_t*>(src);
    auto* k = static_cast<uint32_t*>(sink);
    if (nontemporal)
        hipLaunchKernelGGL(probe_read_kernel<true>, dim3(grid), dim3(256), 0, s, p, bytes / 16, k);
    else
        hipLaunchKernelGGL(probe_read_kernel<false>, dim3(grid), dim3(256), 0, s, p, bytes / 16, k);
    return hipGetLastError();
}

// Reads, for the n_pages entries of the device list `pages` (each below
// pool_pages), slice after slice of every token row of that page of `keys`
// and of `values` (tensors of pool_pages pages of page_bytes, rows of
// row_bytes): (n_pages / per_wg rounded up) x (row_bytes / slice_bytes)
// workgroups of `waves` waves. slice_bytes divides row_bytes, row_bytes
// divides page_bytes, and (page_bytes / row_bytes) x (slice_bytes / 16) is a
// multiple of 256. lds_bytes of LDS (unused) are reserved per workgroup, which
// caps how many share a compute unit (160 KiB each): 0 leaves it to the
// registers. Returns a hipError_t.
int ckv_probe_pages(const void* keys, const void* values, uint32_t pool_pages,
                    const uint32_t* pages, uint32_t n_pages, uint32_t page_bytes,
                    uint32_t row_bytes, uint32_t slice_bytes, uint32_t per_wg, uint32_t waves,
                    uint32_t lds_bytes, void* sink, void* stream)
{
    if (lds_bytes > 160 * 1024)
        return hipErrorInvalidValue;
    if (!keys || !values || !pages || !sink || !pool_pages || !n_pages || !per_wg)
        return hipErrorInvalidValue;
    if (!aligned16(keys) || !aligned16(values) || waves < 1 || waves > 16)
        return hipErrorInvalidValue;
    if (!slice_bytes || slice_bytes % 16 || !row_bytes || row_bytes % slice_bytes
        || !page_bytes || page_bytes % row_bytes)
        return hipErrorInvalidValue;
    const uint64_t chunks = (uint64_t)(page_bytes / row_bytes) * (slice_bytes / 16);
    if (chunks % 256)
        return hipErrorInvalidValue;
    const uint64_t groups = ((uint64_t)n_pages + per_wg - 1) / per_wg;
    const uint64_t grid = groups * (row_bytes / slice_bytes);
    if (grid > 0x7FFFFFFFull)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(probe_pages_kernel, dim3((uint32_t)grid), dim3(64 * waves), lds_bytes,
                       static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(keys),
                       static_cast<const uint8_t*>(values), pool_pages, pages, n_pages,
                       page_bytes, row_bytes, slice_bytes, per_wg, static_cast<uint32_t*>(sink));
    return hipGetLastError();
}

// grid workgroups of `waves` waves, each wave running `chains` (1, 2 or 4)
// independent chains of `iters` v_mfma_f32_32x32x16_bf16 (32,768 FLOPs each).
int ckv_probe_mfma(uint32_t iters, uint32_t chains, uint32_t waves, uint32_t grid, void* sink,
                   void* stream)
{
    if (!sink || !grid || waves < 1 || waves > 16)
        return hipErrorInvalidValue;
    const auto s = static_cast<hipStream_t>(stream);
    auto* k = static_cast<float*>(sink);
    const dim3 g(grid), b(64 * waves);
    if (chains == 1)
        hipLaunchKernelGGL(probe_mfma_kernel<1>, g, b, 0, s, iters, k);
    else if (chains == 2)
        hipLaunchKernelGGL(probe_mfma_kernel<2>, g, b, 0, s, iters, k);
    else if (chains == 4)
        hipLaunchKernelGGL(probe_mfma_kernel<4>, g, b, 0, s, iters, k);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

} // extern "C"

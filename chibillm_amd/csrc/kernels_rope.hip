// Rotary position embedding over device rows, and its fusion with the KV
// append.
//
// rope_f32 (src/metal/kernels/tensor_ops.metal:158-195): within each head of
// a row at position p, pair j < rotary/2 rotates elements j and j + rotary/2
// by the angle float(p) * inv_freq[j]; elements past the rotary width are
// copied. inv_freq is theta^(-2j/rotary) in float, computed on the host as
// src/metal/metal_kernels.mm:186-191 does. The angle is reduced by the
// device library's sincosf (positions reach 10^4..10^5 radians).
//
// The fused form rotates the key rows and scatters them, with the value
// rows, straight into their pages: the apply_rope + store_kv pair of
// src/qwen/qwen_layer.cc:20-30, :43 without the rotated keys' round trip
// through HBM. One thread per (row, head, pair) touches both elements of its
// pair, so consecutive threads read and write consecutive elements.
#include "ckv_internal.h"

#include <algorithm>
#include <cmath>

namespace ckv {
namespace {

constexpr uint32_t block_threads = 256;

template <int DT>
struct element;

template <>
struct element<CKV_F32> {
    using type = float;
    static __device__ __forceinline__ float load(type v) { return v; }
    static __device__ __forceinline__ type store(float v) { return v; }
};

template <>
struct element<CKV_BF16> {
    using type = uint16_t;
    static __device__ __forceinline__ float load(type v)
    {
        return __builtin_bit_cast(float, static_cast<uint32_t>(v) << 16);
    }
    // round to nearest even, NaN quieted (src/tensor/types.h:60-75)
    static __device__ __forceinline__ type store(float v)
    {
        uint32_t b = __builtin_bit_cast(uint32_t, v);
        if ((b & 0x7FFFFFFFu) > 0x7F800000u)
            return static_cast<type>((b >> 16) | 0x40u);
        b += 0x7FFFu + ((b >> 16) & 1u);
        return static_cast<type>(b >> 16);
    }
};

template <>
struct element<CKV_F16> {
    using type = uint16_t;
    static __device__ __forceinline__ float load(type v)
    {
        return static_cast<float>(__builtin_bit_cast(_Float16, v));
    }
    static __device__ __forceinline__ type store(float v)
    {
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
    }
};

// Grid: x covers the row's (head, pair) threads, y strides over rows.
// APPEND: `out` is ignored; rotated keys and the values go to the rows'
// slots of `layer`.
template <int DT, bool APPEND>
__global__ __launch_bounds__(block_threads) void rope_kernel(
    const void* in, void* out, uint32_t rows, uint32_t heads,
    uint32_t head_dim, uint32_t rotary, rope_table freq, const uint32_t* __restrict__ positions,
    pool_view p, const uint32_t* __restrict__ slots, uint32_t layer,
    const void* __restrict__ values)
{
    using E = element<DT>;
    using T = typename E::type;
    const uint32_t half_dim = head_dim / 2, half = rotary / 2;
    const uint32_t t = blockIdx.x * block_threads + threadIdx.x;
    if (t >= heads * half_dim)
        return;
    const uint32_t head = t / half_dim, pair = t % half_dim;
    const uint64_t width = (uint64_t)heads * head_dim;
    // the pair's two elements within the head
    const uint32_t a = pair < half ? pair : rotary + 2 * (pair - half);
    const uint32_t b = pair < half ? pair + half : a + 1;
    for (uint32_t row = blockIdx.y; row < rows; row += gridDim.y) {
        const T* src = static_cast<const T*>(in) + row * width + head * head_dim;
        float x1 = E::load(src[a]), x2 = E::load(src[b]);
        if (pair < half) {
            const float angle = static_cast<float>(positions[row]) * freq.inv_freq[pair];
            float sine, cosine;
            sincosf(angle, &sine, &cosine);
            float r1, r2;
            rope_pair(x1, x2, cosine, sine, r1, r2);
            x1 = r1;
            x2 = r2;
        }
        if constexpr (APPEND) {
            const uint64_t dst = layer * p.layer_elems + (uint64_t)slots[row] * p.features
                + head * head_dim;
            T* kc = static_cast<T*>(p.keys) + dst;
            T* vc = static_cast<T*>(p.values) + dst;
            const T* vs = static_cast<const T*>(values) + row * width + head * head_dim;
            kc[a] = E::store(x1);
            kc[b] = E::store(x2);
            vc[a] = vs[a];
            vc[b] = vs[b];
        } else {
            T* dst = static_cast<T*>(out) + row * width + head * head_dim;
            dst[a] = E::store(x1);
            dst[b] = E::store(x2);
        }
    }
}

// 16-bit rows with rotary == head_dim and half a head a multiple of 8: a
// thread rotates 8 consecutive pairs, reading and writing 16 bytes of each
// half (two 128-bit loads and stores per tensor instead of sixteen 2-byte
// accesses). A row's angles are the same for every head, so the workgroup
// computes the (cosine, sine) of each (row, pair) its threads touch into LDS,
// one sincosf per entry instead of one per (row, head, pair), while its
// threads' loads are in flight.
template <int DT, bool APPEND>
__global__ __launch_bounds__(block_threads) void rope_kernel_x8(
    const void* in, void* out, uint32_t rows, uint32_t heads, uint32_t head_dim,
    rope_table freq, const uint32_t* __restrict__ positions, pool_view p,
    const uint32_t* __restrict__ slots, uint32_t layer, const void* __restrict__ values)
{
    using E = element<DT>;
    extern __shared__ float2 angles[]; // (cosine, sine) per (row of the workgroup, pair)
    const uint32_t half = head_dim / 2, groups = half / 8;
    const uint32_t per_row = heads * groups;
    const uint64_t total = (uint64_t)rows * per_row;
    const uint64_t first = (uint64_t)blockIdx.x * block_threads;
    // the rows this workgroup's items fall in: first_row .. last_row
    const uint32_t first_row = (uint32_t)(first / per_row);
    const uint32_t last_row = (uint32_t)((min(first + block_threads, total) - 1) / per_row);
    const uint32_t entries = (last_row - first_row + 1) * half;
    // this thread's item (its loads go out before the angles are computed)
    const uint64_t t = min(first + threadIdx.x, total - 1);
    const uint32_t row = (uint32_t)(t / per_row), rest = (uint32_t)(t % per_row);
    const uint32_t head = rest / groups, p0 = (rest % groups) * 8;
    const uint64_t width = (uint64_t)heads * head_dim;
    const uint64_t src = row * width + head * head_dim + p0;
    const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(in) + src);
    const uint4 b = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(in) + src + half);
    uint4 va = make_uint4(0, 0, 0, 0), vb = va;
    if constexpr (APPEND) {
        const uint16_t* vs = static_cast<const uint16_t*>(values) + src;
        va = *reinterpret_cast<const uint4*>(vs);
        vb = *reinterpret_cast<const uint4*>(vs + half);
    }
    for (uint32_t e = threadIdx.x; e < entries; e += block_threads) {
        const uint32_t r = first_row + e / half, pair = e % half;
        float sine, cosine;
        sincosf(static_cast<float>(positions[r]) * freq.inv_freq[pair], &sine, &cosine);
        angles[e] = make_float2(cosine, sine);
    }
    __syncthreads();
    if (first + threadIdx.x >= total)
        return;
    const float2* cs = angles + (row - first_row) * half + p0;
    const uint32_t wa[4] = { a.x, a.y, a.z, a.w }, wb[4] = { b.x, b.y, b.z, b.w };
    uint32_t ra[4], rb[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t oa = 0, ob = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float x1 = E::load(static_cast<uint16_t>(wa[d] >> (16 * h)));
            const float x2 = E::load(static_cast<uint16_t>(wb[d] >> (16 * h)));
            const float2 c = cs[2 * d + h];
            float r1, r2;
            rope_pair(x1, x2, c.x, c.y, r1, r2);
            oa |= static_cast<uint32_t>(E::store(r1)) << (16 * h);
            ob |= static_cast<uint32_t>(E::store(r2)) << (16 * h);
        }
        ra[d] = oa;
        rb[d] = ob;
    }
    uint16_t* dst;
    if constexpr (APPEND) {
        const uint64_t off = layer * p.layer_elems + (uint64_t)slots[row] * p.features
            + head * head_dim + p0;
        dst = static_cast<uint16_t*>(p.keys) + off;
        uint16_t* vd = static_cast<uint16_t*>(p.values) + off;
        *reinterpret_cast<uint4*>(vd) = va;
        *reinterpret_cast<uint4*>(vd + half) = vb;
    } else {
        dst = static_cast<uint16_t*>(out) + src;
    }
    *reinterpret_cast<uint4*>(dst) = make_uint4(ra[0], ra[1], ra[2], ra[3]);
    *reinterpret_cast<uint4*>(dst + half) = make_uint4(rb[0], rb[1], rb[2], rb[3]);
}

bool aligned16(const void* ptr)
{
    return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0;
}

template <bool APPEND>
hipError_t launch(hipStream_t s, int dtype, const void* in, void* out, uint32_t rows,
                  uint32_t heads, uint32_t head_dim, uint32_t rotary, const rope_table& freq,
                  const uint32_t* positions, const pool_view& p, const uint32_t* slots,
                  uint32_t layer, const void* values)
{
    if (!rows)
        return hipSuccess;
    const bool x8 = dtype != CKV_F32 && rotary == head_dim && (head_dim / 2) % 8 == 0
        && aligned16(in) && (APPEND ? aligned16(values) && aligned16(p.keys) && aligned16(p.values)
                                    : aligned16(out));
    if (x8) {
        const uint32_t per_row = heads * (head_dim / 16);
        const uint64_t total = (uint64_t)rows * per_row;
        const uint64_t blocks = (total + block_threads - 1) / block_threads;
        if (blocks > 0x7FFFFFFFull)
            return hipErrorInvalidValue;
        const dim3 grid((uint32_t)blocks);
        // the angle table: the rows a workgroup's items fall in, half a head each
        const uint32_t table_rows = std::min<uint32_t>(rows, (block_threads - 1) / per_row + 2);
        const size_t lds = (size_t)table_rows * (head_dim / 2) * sizeof(float2);
        if (dtype == CKV_BF16)
            rope_kernel_x8<CKV_BF16, APPEND><<<grid, block_threads, lds, s>>>(
                in, out, rows, heads, head_dim, freq, positions, p, slots, layer, values);
        else
            rope_kernel_x8<CKV_F16, APPEND><<<grid, block_threads, lds, s>>>(
                in, out, rows, heads, head_dim, freq, positions, p, slots, layer, values);
        return hipGetLastError();
    }
    const uint32_t threads = heads * (head_dim / 2);
    const dim3 grid((threads + block_threads - 1) / block_threads, rows < 65535 ? rows : 65535);
    switch (dtype) {
    case CKV_F32:
        rope_kernel<CKV_F32, APPEND><<<grid, block_threads, 0, s>>>(
            in, out, rows, heads, head_dim, rotary, freq, positions, p, slots, layer, values);
        break;
    case CKV_BF16:
        rope_kernel<CKV_BF16, APPEND><<<grid, block_threads, 0, s>>>(
            in, out, rows, heads, head_dim, rotary, freq, positions, p, slots, layer, values);
        break;
    default:
        rope_kernel<CKV_F16, APPEND><<<grid, block_threads, 0, s>>>(
            in, out, rows, heads, head_dim, rotary, freq, positions, p, slots, layer, values);
        break;
    }
    return hipGetLastError();
}

// out = in * sigmoid(gate), elementwise in float (silu_mul_f32 with
// sigmoid_only, src/metal/kernels/tensor_ops.metal:108-124); out may be in.
template <int DT>
__global__ __launch_bounds__(block_threads) void sigmoid_mul_kernel(const void* gate,
                                                                   const void* in, void* out,
                                                                   uint64_t n)
{
    using E = element<DT>;
    using T = typename E::type;
    const uint64_t stride = (uint64_t)gridDim.x * block_threads;
    for (uint64_t i = (uint64_t)blockIdx.x * block_threads + threadIdx.x; i < n; i += stride) {
        const float g = E::load(static_cast<const T*>(gate)[i]);
        const float x = E::load(static_cast<const T*>(in)[i]);
        static_cast<T*>(out)[i] = E::store(1.0f / (1.0f + __expf(-g)) * x);
    }
}

// The same with 16 bytes of each tensor per thread and step (8 16-bit or 4
// f32 elements, the same arithmetic per element), the last n % per elements
// one at a time; gate, in and out 16-byte aligned.
template <int DT>
__global__ __launch_bounds__(block_threads) void sigmoid_mul_x16_kernel(const void* gate,
                                                                       const void* in, void* out,
                                                                       uint64_t n)
{
    using E = element<DT>;
    using T = typename E::type;
    constexpr uint32_t per = 16 / sizeof(T);
    const uint64_t stride = (uint64_t)gridDim.x * block_threads;
    const uint64_t vecs = n / per;
    union lanes {
        uint4 v;
        T e[per];
    };
    for (uint64_t i = (uint64_t)blockIdx.x * block_threads + threadIdx.x; i < vecs; i += stride) {
        lanes g, x, o;
        g.v = static_cast<const uint4*>(gate)[i];
        x.v = static_cast<const uint4*>(in)[i];
#pragma unroll
        for (uint32_t e = 0; e < per; ++e)
            o.e[e] = E::store(1.0f / (1.0f + __expf(-E::load(g.e[e]))) * E::load(x.e[e]));
        static_cast<uint4*>(out)[i] = o.v;
    }
    for (uint64_t i = vecs * per + (uint64_t)blockIdx.x * block_threads + threadIdx.x; i < n;
         i += stride) {
        const float gv = E::load(static_cast<const T*>(gate)[i]);
        const float xv = E::load(static_cast<const T*>(in)[i]);
        static_cast<T*>(out)[i] = E::store(1.0f / (1.0f + __expf(-gv)) * xv);
    }
}

} // namespace

hipError_t launch_sigmoid_mul(hipStream_t s, int dtype, const void* gate, const void* in,
                              void* out, uint64_t n)
{
    if (!n)
        return hipSuccess;
    const bool x16 = aligned16(gate) && aligned16(in) && aligned16(out);
    const uint64_t per = x16 ? (dtype == CKV_F32 ? 4 : 8) : 1;
    const uint64_t want = (n / per + block_threads - 1) / block_threads;
    const dim3 grid((uint32_t)std::clamp<uint64_t>(want, 1, 65536));
    switch (dtype) {
    case CKV_F32:
        if (x16)
            sigmoid_mul_x16_kernel<CKV_F32><<<grid, block_threads, 0, s>>>(gate, in, out, n);
        else
            sigmoid_mul_kernel<CKV_F32><<<grid, block_threads, 0, s>>>(gate, in, out, n);
        break;
    case CKV_BF16:
        if (x16)
            sigmoid_mul_x16_kernel<CKV_BF16><<<grid, block_threads, 0, s>>>(gate, in, out, n);
        else
            sigmoid_mul_kernel<CKV_BF16><<<grid, block_threads, 0, s>>>(gate, in, out, n);
        break;
    default:
        if (x16)
            sigmoid_mul_x16_kernel<CKV_F16><<<grid, block_threads, 0, s>>>(gate, in, out, n);
        else
            sigmoid_mul_kernel<CKV_F16><<<grid, block_threads, 0, s>>>(gate, in, out, n);
        break;
    }
    return hipGetLastError();
}

void rope_frequencies(float theta, uint32_t rotary, rope_table& out)
{
    for (uint32_t pair = 0; pair < rotary / 2; ++pair) {
        const float exponent = -2.0f * static_cast<float>(pair) / static_cast<float>(rotary);
        out.inv_freq[pair] = std::pow(theta, exponent);
    }
}

hipError_t launch_rope(hipStream_t s, const pool_view& p, const meta_view& m, const void* in,
                       void* out, uint32_t rows, uint32_t heads, uint32_t rotary,
                       const rope_table& freq)
{
    return launch<false>(s, p.dtype, in, out, rows, heads, p.head_dim, rotary, freq,
                         m.positions, p, nullptr, 0, nullptr);
}

hipError_t launch_rope_append(hipStream_t s, const pool_view& p, const meta_view& m,
                              uint32_t layer, const void* keys, const void* values, uint32_t rows,
                              uint32_t rotary, const rope_table& freq)
{
    return launch<true>(s, p.dtype, keys, nullptr, rows, p.kv_heads, p.head_dim, rotary, freq,
                        m.positions, p, m.slots, layer, values);
}

} // namespace ckv

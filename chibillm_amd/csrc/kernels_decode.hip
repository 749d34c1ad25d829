// Paged GQA decode attention: split-KV partials + merge.
//
// Work decomposition (built on the host at upload, reused by every layer):
// each row's logical range 0..position is cut into chunks of m.chunk tokens
// (a multiple of 16); one wave64 owns one (chunk, kv_head) and serves all
// q heads of that KV head's GQA group, so every K/V byte is read once.
// A row with a single chunk writes its output directly; otherwise each wave
// writes (max, denominator, accumulator) and merge_kernel combines them with
// weights 2^(m_c - M), the reduction of paged_attention_reduce_f32
// (src/metal/kernels/attention.metal:567-615).
//
// Fast path (16-bit K/V, head_dim 128, block_size % 4 == 0): the wave reads
// four token rows per load instruction, 16 lanes x 16 bytes per 256-byte
// row, so lane l holds features 8*(l%16).. of token 4j + l/16. A score is a
// bf16/fp16 dot2 chain over the lane's 8 features followed by a 16-lane DPP
// all-reduce (4 VALU ops). Each 16-lane row group keeps its own online-softmax
// state over its tokens; the four states are merged once per chunk. Scores
// are kept in the log2 domain (scale * log2(e)) so every exponential is one
// v_exp_f32.
#include "ckv_internal.h"

#include <cmath>

namespace ckv {
namespace {

constexpr float log2e = 1.4426950408889634f;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float fast_exp2(float x)
{
    return __builtin_amdgcn_exp2f(x);
}

// f32 -> bf16 round to nearest even, NaN quieted (src/tensor/types.h:60-75).
__device__ __forceinline__ uint32_t bf16_bits(float x)
{
    uint32_t b = __builtin_bit_cast(uint32_t, x);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u)
        return (b >> 16) | 0x40u;
    b += 0x7FFFu + ((b >> 16) & 1u);
    return b >> 16;
}

__device__ __forceinline__ uint32_t f16_bits(float x)
{
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

template <bool F16>
struct half2_ops;

template <>
struct half2_ops<false> { // bf16
    static __device__ __forceinline__ float lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
    static __device__ __forceinline__ float hi(uint32_t w)
    {
        return __builtin_bit_cast(float, w & 0xFFFF0000u);
    }
    static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c)
    {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                               __builtin_bit_cast(bf16x2_t, b), c, false);
    }
    static __device__ __forceinline__ uint32_t pack(float a, float b)
    {
        return bf16_bits(a) | (bf16_bits(b) << 16);
    }
};

template <>
struct half2_ops<true> { // fp16
    static __device__ __forceinline__ float lo(uint32_t w)
    {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
    }
    static __device__ __forceinline__ float hi(uint32_t w)
    {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
    }
    static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c)
    {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a),
                                      __builtin_bit_cast(f16x2_t, b), c, false);
    }
    static __device__ __forceinline__ uint32_t pack(float a, float b)
    {
        return f16_bits(a) | (f16_bits(b) << 16);
    }
};

template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __builtin_amdgcn_update_dpp(0.0f, v, CTRL, 0xF, 0xF, false);
}

// Sum over each row of 16 lanes, result in every lane of the row.
__device__ __forceinline__ float row16_sum(float v)
{
    v += dpp<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);  // quad_perm [2,3,0,1]
    v += dpp<0x141>(v); // row_half_mirror
    v += dpp<0x140>(v); // row_mirror
    return v;
}

// Partial record per (work item, q head): [max, denominator, 0, 0, acc[D]].
__host__ __device__ constexpr uint32_t record_floats(uint32_t head_dim)
{
    return head_dim + 4;
}

template <int G, bool F16>
__global__ __launch_bounds__(64) void decode_d128_kernel(pool_view p, meta_view m, uint32_t layer,
                                                         const uint16_t* __restrict__ q,
                                                         uint32_t q_heads, float scale_log2,
                                                         uint16_t* __restrict__ out,
                                                         float* __restrict__ partials)
{
    using ops = half2_ops<F16>;
    constexpr uint32_t D = 128;
    const uint32_t H = p.kv_heads;
    const uint32_t kv_head = blockIdx.x % H;
    const uint32_t item = blockIdx.x / H;
    const uint32_t row = m.items[2 * item];
    const uint32_t chunk_index = m.items[2 * item + 1];
    const uint32_t position = m.positions[row];
    const uint32_t table_base = m.offsets[row];
    const uint32_t begin = chunk_index * m.chunk;
    const uint32_t end = min(position + 1, begin + m.chunk);
    const uint32_t lane = threadIdx.x;
    const uint32_t group = lane >> 4; // token of a 4-token step
    const uint32_t part = lane & 15;  // features 8*part .. 8*part + 7
    const uint32_t bs = p.block_size;
    const uint64_t F = p.features;
    const uint16_t* kbase = static_cast<const uint16_t*>(p.keys) + (uint64_t)layer * p.layer_elems
        + kv_head * D + part * 8;
    const uint16_t* vbase = static_cast<const uint16_t*>(p.values)
        + (uint64_t)layer * p.layer_elems + kv_head * D + part * 8;

    uint4 qv[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
        qv[g] = *reinterpret_cast<const uint4*>(
            q + ((uint64_t)row * q_heads + kv_head * G + g) * D + part * 8);

    float mx[G], den[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        mx[g] = -INFINITY;
        den[g] = 0.0f;
#pragma unroll
        for (int f = 0; f < 8; ++f)
            acc[g][f] = 0.0f;
    }

    for (uint32_t t0 = begin; t0 < end; t0 += 16) {
        uint4 kr[4], vr[4];
        bool ok[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t step = t0 + 4 * j;         // wave-uniform
            const uint32_t last = min(step, end - 1); // a token this row owns
            const uint32_t page = m.table[table_base + last / bs];
            const uint32_t token = step + group;
            ok[j] = token < end;
            // invalid lanes re-read the row's own token `last`: in bounds and written
            const uint32_t in_page = ok[j] ? token % bs : last % bs;
            const uint64_t slot = (uint64_t)page * bs + in_page;
            kr[j] = *reinterpret_cast<const uint4*>(kbase + slot * F);
            vr[j] = *reinterpret_cast<const uint4*>(vbase + slot * F);
        }

        float vf[4][8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            vf[j][0] = ops::lo(vr[j].x);
            vf[j][1] = ops::hi(vr[j].x);
            vf[j][2] = ops::lo(vr[j].y);
            vf[j][3] = ops::hi(vr[j].y);
            vf[j][4] = ops::lo(vr[j].z);
            vf[j][5] = ops::hi(vr[j].z);
            vf[j][6] = ops::lo(vr[j].w);
            vf[j][7] = ops::hi(vr[j].w);
        }

#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float d = ops::dot2(qv[g].x, kr[j].x, 0.0f);
                d = ops::dot2(qv[g].y, kr[j].y, d);
                d = ops::dot2(qv[g].z, kr[j].z, d);
                d = ops::dot2(qv[g].w, kr[j].w, d);
                s[j] = ok[j] ? row16_sum(d) * scale_log2 : -INFINITY;
            }
            const float tile = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
            const float nm = fmaxf(mx[g], tile);
            const bool none = nm == -INFINITY; // this row group has no token yet
            const float alpha = none ? 1.0f : fast_exp2(mx[g] - nm);
            float pw[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                pw[j] = ok[j] ? fast_exp2(s[j] - nm) : 0.0f;
            den[g] = den[g] * alpha + ((pw[0] + pw[1]) + (pw[2] + pw[3]));
#pragma unroll
            for (int f = 0; f < 8; ++f) {
                float a = acc[g][f] * alpha;
                a += pw[0] * vf[0][f];
                a += pw[1] * vf[1][f];
                a += pw[2] * vf[2][f];
                a += pw[3] * vf[3][f];
                acc[g][f] = a;
            }
            mx[g] = nm;
        }
    }

    // merge the four row-group states (lanes l, l^16, l^32, l^48)
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float M = fmaxf(mx[g], __shfl_xor(mx[g], 16));
        M = fmaxf(M, __shfl_xor(M, 32));
        const float w = mx[g] == -INFINITY ? 0.0f : fast_exp2(mx[g] - M);
        float d = den[g] * w;
        d += __shfl_xor(d, 16);
        d += __shfl_xor(d, 32);
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            float a = acc[g][f] * w;
            a += __shfl_xor(a, 16);
            a += __shfl_xor(a, 32);
            acc[g][f] = a;
        }
        den[g] = d;
        mx[g] = M;
    }

    if (group != 0)
        return;
    const bool single = m.row_count[row] == 1;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const uint32_t qh = kv_head * G + g;
        if (single) {
            const float inv = 1.0f / den[g];
            uint4 o;
            o.x = ops::pack(acc[g][0] * inv, acc[g][1] * inv);
            o.y = ops::pack(acc[g][2] * inv, acc[g][3] * inv);
            o.z = ops::pack(acc[g][4] * inv, acc[g][5] * inv);
            o.w = ops::pack(acc[g][6] * inv, acc[g][7] * inv);
            *reinterpret_cast<uint4*>(out + ((uint64_t)row * q_heads + qh) * D + part * 8) = o;
        } else {
            float* rec = partials + ((uint64_t)item * q_heads + qh) * record_floats(D);
            float4* dst = reinterpret_cast<float4*>(rec + 4 + part * 8);
            dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
            dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
            if (part == 0) {
                rec[0] = mx[g];
                rec[1] = den[g];
            }
        }
    }
}

// ---- generic path: any head_dim <= 1024, f32 / bf16 / fp16 ---------------------

template <int DT>
__device__ __forceinline__ float load_elem(const void* base, uint64_t i)
{
    if constexpr (DT == CKV_F32)
        return static_cast<const float*>(base)[i];
    else if constexpr (DT == CKV_BF16)
        return __builtin_bit_cast(float, (uint32_t)static_cast<const uint16_t*>(base)[i] << 16);
    else
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(base)[i]));
}

template <int DT>
__device__ __forceinline__ void store_elem(void* base, uint64_t i, float x)
{
    if constexpr (DT == CKV_F32)
        static_cast<float*>(base)[i] = x;
    else if constexpr (DT == CKV_BF16)
        static_cast<uint16_t*>(base)[i] = static_cast<uint16_t>(bf16_bits(x));
    else
        static_cast<uint16_t*>(base)[i] = static_cast<uint16_t>(f16_bits(x));
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1)
        v += __shfl_xor(v, mask);
    return v;
}

constexpr int generic_max_features_per_lane = 16; // head_dim <= 1024

// One wave per (work item, kv_head); the group's q heads are processed one
// after another, each with the per-token online softmax of
// paged_attention_f32 (src/metal/kernels/attention.metal:101-155), lanes
// striding the features.
template <int DT>
__global__ __launch_bounds__(64) void decode_generic_kernel(pool_view p, meta_view m, uint32_t layer,
                                                            const void* __restrict__ q,
                                                            uint32_t q_heads, float scale_log2,
                                                            void* __restrict__ out,
                                                            float* __restrict__ partials)
{
    constexpr int NF = generic_max_features_per_lane;
    const uint32_t H = p.kv_heads;
    const uint32_t D = p.head_dim;
    const uint32_t kv_head = blockIdx.x % H;
    const uint32_t item = blockIdx.x / H;
    const uint32_t row = m.items[2 * item];
    const uint32_t chunk_index = m.items[2 * item + 1];
    const uint32_t position = m.positions[row];
    const uint32_t table_base = m.offsets[row];
    const uint32_t begin = chunk_index * m.chunk;
    const uint32_t end = min(position + 1, begin + m.chunk);
    const uint32_t lane = threadIdx.x;
    const uint32_t G = q_heads / H;
    const uint32_t bs = p.block_size;
    const uint64_t slot_count = (uint64_t)p.blocks * bs;
    const bool single = m.row_count[row] == 1;

    for (uint32_t g = 0; g < G; ++g) {
        const uint32_t qh = kv_head * G + g;
        const uint64_t q_base = ((uint64_t)row * q_heads + qh) * D;
        float qf[NF], acc[NF];
#pragma unroll
        for (int k = 0; k < NF; ++k) {
            const uint32_t f = lane + 64 * k;
            qf[k] = f < D ? load_elem<DT>(q, q_base + f) : 0.0f;
            acc[k] = 0.0f;
        }
        float mx = -INFINITY, den = 0.0f;
        for (uint32_t t = begin; t < end; ++t) {
            const uint64_t slot = (uint64_t)m.table[table_base + t / bs] * bs + t % bs;
            const uint64_t base = ((uint64_t)layer * slot_count + slot) * p.features + kv_head * D;
            float d = 0.0f;
#pragma unroll
            for (int k = 0; k < NF; ++k) {
                const uint32_t f = lane + 64 * k;
                if (f < D)
                    d += qf[k] * load_elem<DT>(p.keys, base + f);
            }
            const float score = wave_sum(d) * scale_log2;
            const float nm = fmaxf(mx, score);
            const float alpha = fast_exp2(mx - nm);
            const float w = fast_exp2(score - nm);
            den = den * alpha + w;
#pragma unroll
            for (int k = 0; k < NF; ++k) {
                const uint32_t f = lane + 64 * k;
                if (f < D)
                    acc[k] = acc[k] * alpha + w * load_elem<DT>(p.values, base + f);
            }
            mx = nm;
        }
        if (single) {
            for (int k = 0; k < NF; ++k) {
                const uint32_t f = lane + 64 * k;
                if (f < D)
                    store_elem<DT>(out, q_base + f, acc[k] / den);
            }
        } else {
            float* rec = partials + ((uint64_t)item * q_heads + qh) * record_floats(D);
            for (int k = 0; k < NF; ++k) {
                const uint32_t f = lane + 64 * k;
                if (f < D)
                    rec[4 + f] = acc[k];
            }
            if (lane == 0) {
                rec[0] = mx;
                rec[1] = den;
            }
        }
    }
}

// One wave per (row, q head) of rows with more than one chunk.
template <int DT>
__global__ __launch_bounds__(64) void merge_kernel(meta_view m, uint32_t q_heads, uint32_t D,
                                                   const float* __restrict__ partials,
                                                   void* __restrict__ out)
{
    const uint32_t row = blockIdx.x / q_heads;
    const uint32_t qh = blockIdx.x % q_heads;
    const uint32_t n = m.row_count[row];
    if (n <= 1)
        return;
    const uint32_t first = m.row_first[row];
    const uint32_t stride = record_floats(D);
    const float* rec0 = partials + ((uint64_t)first * q_heads + qh) * stride;
    const uint64_t item_stride = (uint64_t)q_heads * stride;
    float M = -INFINITY;
    for (uint32_t c = 0; c < n; ++c)
        M = fmaxf(M, rec0[c * item_stride]);
    float den = 0.0f;
    for (uint32_t c = 0; c < n; ++c)
        den += rec0[c * item_stride + 1] * fast_exp2(rec0[c * item_stride] - M);
    const float inv = 1.0f / den;
    const uint64_t o_base = ((uint64_t)row * q_heads + qh) * D;
    for (uint32_t f = threadIdx.x; f < D; f += 64) {
        float a = 0.0f;
        for (uint32_t c = 0; c < n; ++c)
            a += rec0[c * item_stride + 4 + f] * fast_exp2(rec0[c * item_stride] - M);
        store_elem<DT>(out, o_base + f, a * inv);
    }
}

bool aligned16(const void* ptr)
{
    return reinterpret_cast<uintptr_t>(ptr) % 16 == 0;
}

template <int G>
hipError_t launch_fast(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                       const void* q, uint32_t q_heads, float scale_log2, void* out,
                       float* partials, bool f16)
{
    const dim3 grid(m.n_items * p.kv_heads), block(64);
    const auto qq = static_cast<const uint16_t*>(q);
    const auto oo = static_cast<uint16_t*>(out);
    if (f16)
        decode_d128_kernel<G, true><<<grid, block, 0, s>>>(p, m, layer, qq, q_heads, scale_log2, oo,
                                                           partials);
    else
        decode_d128_kernel<G, false><<<grid, block, 0, s>>>(p, m, layer, qq, q_heads, scale_log2,
                                                            oo, partials);
    return hipGetLastError();
}

} // namespace

bool decode_uses_fast_path(const pool_view& p, uint32_t q_heads)
{
    const uint32_t G = q_heads / p.kv_heads;
    return p.dtype != CKV_F32 && p.head_dim == 128 && p.block_size % 4 == 0
        && (G == 1 || G == 2 || G == 4 || G == 8) && aligned16(p.keys) && aligned16(p.values);
}

hipError_t launch_decode(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                         const void* q, uint32_t q_heads, float scale, void* out,
                         float* partials)
{
    if (!m.n_items)
        return hipSuccess;
    const float scale_log2 = scale * log2e;
    if (decode_uses_fast_path(p, q_heads) && aligned16(q) && aligned16(out)) {
        const bool f16 = p.dtype == CKV_F16;
        switch (q_heads / p.kv_heads) {
        case 1:
            return launch_fast<1>(s, p, m, layer, q, q_heads, scale_log2, out, partials, f16);
        case 2:
            return launch_fast<2>(s, p, m, layer, q, q_heads, scale_log2, out, partials, f16);
        case 4:
            return launch_fast<4>(s, p, m, layer, q, q_heads, scale_log2, out, partials, f16);
        default:
            return launch_fast<8>(s, p, m, layer, q, q_heads, scale_log2, out, partials, f16);
        }
    }
    if (p.head_dim > 64u * generic_max_features_per_lane)
        return hipErrorInvalidValue;
    const dim3 grid(m.n_items * p.kv_heads), block(64);
    switch (p.dtype) {
    case CKV_F32:
        decode_generic_kernel<CKV_F32><<<grid, block, 0, s>>>(p, m, layer, q, q_heads, scale_log2,
                                                              out, partials);
        break;
    case CKV_BF16:
        decode_generic_kernel<CKV_BF16><<<grid, block, 0, s>>>(p, m, layer, q, q_heads,
                                                               scale_log2, out, partials);
        break;
    default:
        decode_generic_kernel<CKV_F16><<<grid, block, 0, s>>>(p, m, layer, q, q_heads, scale_log2,
                                                              out, partials);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_merge(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t q_heads,
                        void* out, const float* partials)
{
    const dim3 grid(m.rows * q_heads), block(64);
    switch (p.dtype) {
    case CKV_F32:
        merge_kernel<CKV_F32><<<grid, block, 0, s>>>(m, q_heads, p.head_dim, partials, out);
        break;
    case CKV_BF16:
        merge_kernel<CKV_BF16><<<grid, block, 0, s>>>(m, q_heads, p.head_dim, partials, out);
        break;
    default:
        merge_kernel<CKV_F16><<<grid, block, 0, s>>>(m, q_heads, p.head_dim, partials, out);
        break;
    }
    return hipGetLastError();
}

uint32_t partial_record_floats(uint32_t head_dim)
{
    return record_floats(head_dim);
}

} // namespace ckv

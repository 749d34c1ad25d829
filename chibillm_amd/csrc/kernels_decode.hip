// Paged GQA decode attention.
//
// Fast path (head_dim 128, 16-token pages, 1/2/4/8 q heads per KV head; f32
// pages up to 4): one workgroup per (plan workgroup, kv_head) serves every q
// head of the KV head's GQA group, so each K/V byte is read once. A wave reads
// four token rows per load instruction, 16 lanes per row, so lane l holds 8
// features of token 4j + l/16: 8*(l%16).. of a bf16/fp16 row (16 bytes), or
// 4*(l%16).. and 64 + 4*(l%16).. of an f32 row (two 16-byte words, each
// instruction reading 256 contiguous bytes). A score is a dot chain over the lane's 8 features
// (v_dot2 for 16-bit pairs) followed by a 16-lane DPP all-reduce (4 VALU ops).
// Each 16-lane row group keeps its own online-softmax state over its tokens;
// the four states are merged once per segment. Scores are kept in the log2
// domain (scale * log2(e)) so every exponential is one v_exp_f32. Rows the
// batch plan cuts are merged in the same launch with weights 2^(m_c - M), the
// reduction of paged_attention_reduce_f32
// (src/metal/kernels/attention.metal:567-615).
//
// Generic path (any head_dim <= 1024, any page size): split-KV over token
// chunks, one wave per (chunk, kv_head), and a merge launch.
#include "ckv_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>

namespace ckv {
namespace {

constexpr float log2e = 1.4426950408889634f;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// K/V pages are read once per decode step: nontemporal loads stream them
// past the caches (measured on MI355X: plain 16-byte streaming reads top out
// near 6.4 TB/s, nontemporal ones near 6.9 TB/s).
__device__ __forceinline__ uint4 load_stream(const void* p)
{
    const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}

// The eight elements of one K, V or query head row a lane of the fast decode
// holds: lane part p (of 16) takes the 16 bytes at 16p, features 8p..8p+7 of
// a 16-bit row; of an f32 row (the reference's storage,
// src/metal/metal_kv_cache.cc:57-69) also the 16 bytes at 256 + 16p, so its
// features are 4p..4p+3 and 64+4p..64+4p+3. Either way each 16-byte load
// instruction of 16 lanes reads 256 contiguous bytes of the row.
template <int DT>
struct lane8 {
    static constexpr uint32_t words = DT == CKV_F32 ? 2 : 1;
    static constexpr uint32_t elem = DT == CKV_F32 ? 4 : 2; // bytes per element
    static constexpr uint32_t stride = 256;                 // bytes between the words
    uint4 w[words];
    // the head feature of the lane's element i (of 8), for lane part p
    static __device__ __forceinline__ uint32_t feature(uint32_t p, uint32_t i)
    {
        return DT == CKV_F32 ? (i < 4 ? 4 * p + i : 64 + 4 * p + (i - 4)) : 8 * p + i;
    }
};

template <int DT>
__device__ __forceinline__ lane8<DT> load8_stream(const char* p)
{
    lane8<DT> x;
#pragma unroll
    for (uint32_t i = 0; i < lane8<DT>::words; ++i)
        x.w[i] = load_stream(p + lane8<DT>::stride * i);
    return x;
}

template <int DT>
__device__ __forceinline__ lane8<DT> load8(const char* p)
{
    lane8<DT> x;
#pragma unroll
    for (uint32_t i = 0; i < lane8<DT>::words; ++i)
        x.w[i] = *reinterpret_cast<const uint4*>(p + lane8<DT>::stride * i);
    return x;
}

template <int DT>
__device__ __forceinline__ void store8(char* p, const lane8<DT>& x)
{
#pragma unroll
    for (uint32_t i = 0; i < lane8<DT>::words; ++i)
        *reinterpret_cast<uint4*>(p + lane8<DT>::stride * i) = x.w[i];
}

__device__ __forceinline__ float fast_exp2(float x)
{
    return __builtin_amdgcn_exp2f(x);
}

// The split-K handoff between workgroups (a cut row's chunks store partial
// records, count themselves in, and the last to arrive merges) is a protocol
// of this target's memory system, not a release/acquire pair of the HIP
// memory model:
//   - records are written with relaxed agent-scope atomic stores and read
//     with relaxed agent-scope atomic loads; on gfx950 (the GFX942 rows of
//     LLVM's AMDGPU memory model) these are global_store/global_load with sc1,
//     which write through and bypass any L2 line that could be stale, so
//     every XCD sees them in memory without an L2 writeback;
//   - each writer waits with s_waitcnt vmcnt(0) for its stores to complete
//     (on GFX9-family parts vmcnt counts stores too) before one thread's
//     relaxed agent-scope fetch-add counts the chunk in; the last arriver's
//     loads are issued after that RMW returns.
// A model-level handoff costs far more here: an agent-scope release lowers to
// buffer_wbl2 sc1, a writeback of the XCD's L2 (a release RMW +27 % and an
// acq_rel RMW +29 % on config 2's decode; a separate merge launch +1.3 %;
// an acquire fence in the last arriver alone +1.5 %). The guard below keeps
// the protocol off targets where the vmcnt wait would not cover stores
// (GFX10+, which count them with vscnt) or where sc1 means something else.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "kernels_decode.hip's split-K handoff relies on gfx950's memory system; build for gfx950"
#endif

// Relaxed agent-scope accesses: coherent across the XCDs on their own (the
// store writes through, the load misses any cache line that could be stale),
// so data passed this way between workgroups needs no L2 writeback, only
// the writer's wait for its stores to complete before it signals.
__device__ __forceinline__ void agent_store(float* p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float agent_load(const float* p)
{
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until every vector memory access this wave issued (stores included)
// has completed; a compiler barrier too.
__device__ __forceinline__ void wait_vector_memory()
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
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

// 1 / (1 + e^-g) in float, the gate of silu_mul_f32 with sigmoid_only
// (src/metal/kernels/tensor_ops.metal:108-124): 0 and 1 at the extremes.
__device__ __forceinline__ float sigmoid(float g)
{
    return 1.0f / (1.0f + fast_exp2(-g * log2e));
}

template <bool F16>
__device__ __forceinline__ float half_value(uint16_t bits)
{
    if constexpr (F16)
        return static_cast<float>(__builtin_bit_cast(_Float16, bits));
    else
        return __builtin_bit_cast(float, static_cast<uint32_t>(bits) << 16);
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

// Workgroups whose lanes need more than 128 registers (more than two q heads
// per KV head, or f32 pages, whose double-buffered K/V words alone take 128)
// run at most 8 waves, two per SIMD, with up to 256 registers a lane.
__host__ __device__ constexpr bool wide_lanes(uint32_t group, int dtype)
{
    return group > 2 || dtype == CKV_F32;
}

// Eight q heads of f32 pages do not fit 256 registers a lane (the kernel
// would spill): such pools run the four-head kernel twice (launch_fast<8>).
__host__ __device__ constexpr bool fast_fits(uint32_t group, int dtype)
{
    return !(group == 8 && dtype == CKV_F32);
}

// q . k over a lane's eight elements (16-bit pairs by v_dot2 with fp32
// accumulation; f32 by fused multiply-adds), and a V row widened to floats.
template <int DT>
__device__ __forceinline__ float dot8(const lane8<DT>& q, const lane8<DT>& k)
{
    if constexpr (DT == CKV_F32) {
        float d = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < 2; ++i) {
            d = __builtin_fmaf(__builtin_bit_cast(float, q.w[i].x), __builtin_bit_cast(float, k.w[i].x), d);
            d = __builtin_fmaf(__builtin_bit_cast(float, q.w[i].y), __builtin_bit_cast(float, k.w[i].y), d);
            d = __builtin_fmaf(__builtin_bit_cast(float, q.w[i].z), __builtin_bit_cast(float, k.w[i].z), d);
            d = __builtin_fmaf(__builtin_bit_cast(float, q.w[i].w), __builtin_bit_cast(float, k.w[i].w), d);
        }
        return d;
    } else {
        using ops = half2_ops<DT == CKV_F16>;
        float d = ops::dot2(q.w[0].x, k.w[0].x, 0.0f);
        d = ops::dot2(q.w[0].y, k.w[0].y, d);
        d = ops::dot2(q.w[0].z, k.w[0].z, d);
        return ops::dot2(q.w[0].w, k.w[0].w, d);
    }
}

template <int DT>
__device__ __forceinline__ void widen8(const lane8<DT>& v, float (&f)[8])
{
    if constexpr (DT == CKV_F32) {
#pragma unroll
        for (uint32_t i = 0; i < 2; ++i) {
            f[4 * i + 0] = __builtin_bit_cast(float, v.w[i].x);
            f[4 * i + 1] = __builtin_bit_cast(float, v.w[i].y);
            f[4 * i + 2] = __builtin_bit_cast(float, v.w[i].z);
            f[4 * i + 3] = __builtin_bit_cast(float, v.w[i].w);
        }
    } else {
        using ops = half2_ops<DT == CKV_F16>;
        const uint4 w = v.w[0];
        f[0] = ops::lo(w.x); f[1] = ops::hi(w.x); f[2] = ops::lo(w.y); f[3] = ops::hi(w.y);
        f[4] = ops::lo(w.z); f[5] = ops::hi(w.z); f[6] = ops::lo(w.w); f[7] = ops::hi(w.w);
    }
}

// One element of a pool-dtype row (gate, output, generic-path operands) as
// float, and back (one rounding, to nearest even).
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

// Fast path, one workgroup per (plan workgroup, kv_head), W waves. A
// workgroup runs its plan segments one after another: each a row, or a piece
// (a run of pages) of a row that the plan cuts (the split-K of
// paged_attention_partial_f32 / paged_attention_reduce_f32,
// src/metal/kernels/attention.metal:446-615, for any row). With FUSED, the
// row's new token (position = the row's last) is taken from k_in/v_in rows
// instead of the cache and stored into its slot by the wave that owns the
// last page: the append of store_kv and the attention in one pass. Wave w
// walks pages first+w, first+w+W, ... of its segment (16-token pages, one
// scalar table read per page); the next page's K/V loads are issued before the
// current page is processed. Lane 16*group + part reads features 8*part..8*part+7 of token
// 4j + group of the page (j = 0..3): four 1 KiB wave loads per page for K and
// four for V. The wave's four row-group softmax states are merged with
// shuffles, the W wave states through LDS, and the workgroup writes the
// normalised output of the group's q heads. GATED multiplies it by
// sigmoid(gate) first; the gate values are loaded when the workgroup starts,
// so their latency hides behind the page loads. A chunk of a cut row writes
// its unnormalised state instead (a partial record per q head) with
// agent-scope stores and counts itself in; the chunk that arrives last merges
// the row's records in the same launch. (An agent-scope release fence per
// workgroup would write back the XCD's whole L2, measured at about 1.9 us per
// workgroup per XCD; stores that are coherent on their own need only a wait
// for completion before the count.) ROPE (with FUSED) rotates the
// queries and the new token's key by the row's position first, as rope_f32
// (src/metal/kernels/tensor_ops.metal:158-195) would: feature f < rotary/2
// pairs with f + rotary/2, which sits in the lane part ^ (rotary/16) of the
// same 16-lane group, so one lane exchange per register rotates a head.
template <int G, int DT, bool FUSED, bool GATED, bool ROPE>
__global__ __launch_bounds__(wide_lanes(G, DT) ? 512 : 1024, wide_lanes(G, DT) ? 2 : 4) void decode_wg_kernel(
    pool_view p, meta_view m, uint32_t layer, const char* __restrict__ q, uint32_t q_heads,
    float scale_log2, void* __restrict__ out, const char* __restrict__ k_in,
    const char* __restrict__ v_in, const void* __restrict__ gate, rope_table64 freq,
    uint32_t rotary, split_scratch split, uint32_t group_stride, uint32_t head_base)
{
    static_assert(!(ROPE && DT == CKV_F32), "the fused rotation works on 16-bit pairs");
    constexpr bool F16 = DT == CKV_F16;
    using ops = half2_ops<F16>;
    using row8 = lane8<DT>;
    constexpr uint32_t ES = row8::elem;
    constexpr uint32_t D = 128;
    constexpr uint32_t BS = 16;
    extern __shared__ float lds[];
    const uint32_t W = blockDim.x >> 6;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // a scalar
    const uint32_t H = p.kv_heads;
    const uint32_t kv_head = blockIdx.x % H;
    // the workgroup's q heads: qh0 .. qh0 + G - 1 (group_stride = G and
    // head_base = 0, or one of the passes over half of a larger group)
    const uint32_t qh0 = kv_head * group_stride + head_base;
    const uint32_t row_bytes = p.features * ES;
    const uint64_t page_bytes = (uint64_t)BS * row_bytes;
    const char* kl = static_cast<const char*>(p.keys) + (uint64_t)layer * p.layer_elems * ES;
    const char* vl = static_cast<const char*>(p.values) + (uint64_t)layer * p.layer_elems * ES;
    // the layer's bases and the table are known from the arguments alone: load
    // them now, beside the plan entry, not after it
    asm volatile("" ::"s"(kl), "s"(vl), "s"(m.table), "s"(row_bytes), "s"(q));

    // One segment: pages [pg_first, pg_end) of a row, chunk `chunk` of the
    // row's n_chunks (e0 = row, chunk, the row's position, the flat table
    // index of page pg_first; e1 = pg_first, pg_end, n_chunks, next entry).
    auto segment = [&](const uint4 e0, const uint4 e1) {
        // The lane's index, computed anew in each segment (a volatile asm, so it
        // is not held in a register across the segment loop), and the thread's.
        uint32_t lane;
        asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
        const uint32_t tid = wave * 64 + lane;
        const uint32_t group = lane >> 4;
        const uint32_t part = lane & 15;
        const uint32_t head_off = kv_head * (D * ES) + part * 16u; // the lane's first word
        const uint32_t row = e0.x;
        const uint32_t chunk = e0.y;
        const uint32_t position = e0.z;
        const uint32_t n_pages = position / BS + 1;
        const uint32_t last_in_page = position % BS;
        const uint32_t pg_first = e1.x;
        const uint32_t pg_end = e1.y;
        const uint32_t n_chunks = e1.z;
        float gate_early = 0.0f; // the first epilogue iteration's gate value (one register)
        if constexpr (GATED) {
            if (tid < G * D)
                gate_early = load_elem<DT>(gate, ((uint64_t)row * q_heads + qh0) * D + tid);
        }
        const uint32_t* tbl = m.table + (e0.w - pg_first); // the row's table

        row8 qv[G];
#pragma unroll
        for (int g = 0; g < G; ++g)
            qv[g] = load8<DT>(q + ((uint64_t)row * q_heads + qh0 + g) * D * ES + part * 16);

        // ROPE: this lane's 8 features (pairs j0 .. j0 + 7) and their rotation;
        // every lane of the wave takes part in the exchanges. The queries and the
        // new token's key share the row's position: both are rotated while the
        // wave's first page loads, and the rotated key (this lane's 16 bytes of
        // it) takes the new token's place when the last page is processed. The
        // row's rotary/2 angles are computed once, by wave 0, into LDS past the
        // merge area.
        const uint32_t rot_mask = ROPE ? rotary / 16 : 1; // lane parts per half of the rotary width
        const bool rot_on = ROPE && part < 2 * rot_mask;
        const bool rot_first = part < rot_mask;
        auto angles = [&](float (&rc)[8], float (&rs)[8]) {
            float* table = lds + W * G * (D + 2); // (cos, sin) per pair
            if (wave == 0 && lane < rotary / 2) {
                float sn, cs;
                sincosf(static_cast<float>(position) * freq.inv_freq[lane], &sn, &cs);
                table[2 * lane] = cs;
                table[2 * lane + 1] = sn;
            }
            __syncthreads();
            const uint32_t j0 = 8 * (part & (rot_mask - 1));
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                rc[e] = rot_on ? table[2 * (j0 + e)] : 1.0f;
                rs[e] = rot_on ? table[2 * (j0 + e) + 1] : 0.0f;
            }
        };
        auto rotate = [&](const uint4& w, const float (&rc)[8], const float (&rs)[8]) {
            const uint32_t in[4] = { w.x, w.y, w.z, w.w };
            uint32_t r[4];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t pw = __shfl_xor(in[d], (int)rot_mask);
                const float own[2] = { ops::lo(in[d]), ops::hi(in[d]) };
                const float par[2] = { ops::lo(pw), ops::hi(pw) };
                float x[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float ra, rb;
                    rope_pair(rot_first ? own[h] : par[h], rot_first ? par[h] : own[h],
                              rc[2 * d + h], rs[2 * d + h], ra, rb);
                    x[h] = rot_first ? ra : rb;
                }
                r[d] = rot_on ? ops::pack(x[0], x[1]) : in[d];
            }
            return make_uint4(r[0], r[1], r[2], r[3]);
        };
        const uint64_t in_row = (uint64_t)row * row_bytes + head_off;
        uint4 k_new = make_uint4(0, 0, 0, 0); // ROPE: the new token's key, rotated once loaded
        if constexpr (ROPE)
            k_new = load8<DT>(k_in + in_row).w[0];

        float mx[G], den[G], acc[G][8];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            mx[g] = -INFINITY;
            den[g] = 0.0f;
#pragma unroll
            for (int f = 0; f < 8; ++f)
                acc[g][f] = 0.0f;
        }

        // rows past the row's last token re-read that token (in bounds, written)
        auto load_page = [&](uint32_t pg, row8* k, row8* v) {
            const uint64_t base = (uint64_t)tbl[pg] * page_bytes;
            const char* kb = kl + base;
            const char* vb = vl + base;
            const bool last_page = pg == n_pages - 1;
            const uint32_t last = last_page ? last_in_page : BS - 1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t r = min(4u * j + group, last);
                const uint32_t off = r * row_bytes + head_off;
                const bool fresh = FUSED && last_page && r == last_in_page;
                // ROPE: the new token's slot is read too and replaced in process
                k[j] = load8_stream<DT>(fresh && !ROPE ? k_in + in_row : kb + off);
                v[j] = load8_stream<DT>(fresh ? v_in + in_row : vb + off);
            }
        };

        auto process = [&](row8* k, const row8* v, uint32_t pg) {
            const uint32_t valid = pg == n_pages - 1 ? last_in_page + 1 : BS;
            if (FUSED && pg == n_pages - 1) {
                if constexpr (ROPE) {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (4u * j + group == last_in_page)
                            k[j].w[0] = k_new;
                }
                // append: the lanes holding the new token write it into its slot
                const uint64_t base = (uint64_t)tbl[pg] * page_bytes;
                const uint32_t off = last_in_page * row_bytes + head_off;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (4u * j + group == last_in_page) {
                        store8<DT>(const_cast<char*>(kl) + base + off, k[j]);
                        store8<DT>(const_cast<char*>(vl) + base + off, v[j]);
                    }
                }
            }
            bool ok[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                ok[j] = 4u * j + group < valid;
            float pw[G][4];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float s[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float r = row16_sum(dot8<DT>(qv[g], k[j])) * scale_log2;
                    s[j] = ok[j] ? r : -INFINITY;
                }
                const float nm = fmaxf(mx[g], fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
                // rescale only when some lane's running max grew (alpha is 1 elsewhere)
                if (__builtin_amdgcn_ballot_w64(nm > mx[g])) {
                    const float alpha = nm == -INFINITY ? 1.0f : fast_exp2(mx[g] - nm);
                    den[g] *= alpha;
#pragma unroll
                    for (int f = 0; f < 8; ++f)
                        acc[g][f] *= alpha;
                    mx[g] = nm;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    pw[g][j] = ok[j] ? fast_exp2(s[j] - mx[g]) : 0.0f;
                den[g] += (pw[g][0] + pw[g][1]) + (pw[g][2] + pw[g][3]);
            }
            // token by token: widen the V row once, accumulate it into every q head
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float vf[8];
                widen8<DT>(v[j], vf);
#pragma unroll
                for (int g = 0; g < G; ++g)
#pragma unroll
                    for (int f = 0; f < 8; ++f)
                        acc[g][f] += pw[g][j] * vf[f];
            }
        };

        row8 ka[4], va[4], kb[4], vb[4];
        uint32_t pg = pg_first + wave;
        if (pg < pg_end)
            load_page(pg, ka, va);
        // ROPE: rotate the queries and the new key while the first page loads
        if constexpr (ROPE) {
            float rc[8], rs[8];
            angles(rc, rs);
#pragma unroll
            for (int g = 0; g < G; ++g)
                qv[g].w[0] = rotate(qv[g].w[0], rc, rs);
            k_new = rotate(k_new, rc, rs);
        }
        // Issue arbitration favours older waves: with a fixed priority the
        // workgroup's youngest waves finish their pages last while the others
        // wait (in config 3's workgroups, 13.6 us median between wave 0's last
        // page and the workgroup's end). Each wave steps through the four
        // priority levels page by page, starting at its own index, so every
        // wave takes its turn at the top (5.1 us; launches 1.2-2 % shorter).
        // The pages each wave reads, and so the results, do not change.
        uint32_t turn = wave;
        auto rotate_priority = [&]() {
            switch (turn++ & 3) {
            case 0:
                __builtin_amdgcn_s_setprio(0);
                break;
            case 1:
                __builtin_amdgcn_s_setprio(1);
                break;
            case 2:
                __builtin_amdgcn_s_setprio(2);
                break;
            default:
                __builtin_amdgcn_s_setprio(3);
                break;
            }
        };
        while (pg < pg_end) {
            uint32_t next = pg + W;
            rotate_priority();
            if (next < pg_end)
                load_page(next, kb, vb);
            process(ka, va, pg);
            pg = next;
            if (pg >= pg_end)
                break;
            next = pg + W;
            rotate_priority();
            if (next < pg_end)
                load_page(next, ka, va);
            process(kb, vb, pg);
            pg = next;
        }
        __builtin_amdgcn_s_setprio(0); // the merge at the default priority

        // merge the wave's four row-group states (lanes l, l^16, l^32, l^48)
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
        // LDS: acc [W][G][D], then (max, denominator) [W][G][2]
        float* lds_acc = lds;
        float* lds_ml = lds + W * G * D;
        if (group == 0) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float* dst = lds_acc + (wave * G + g) * D;
                *reinterpret_cast<float4*>(dst + row8::feature(part, 0)) =
                    make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
                *reinterpret_cast<float4*>(dst + row8::feature(part, 4)) =
                    make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
                if (part == 0) {
                    lds_ml[(wave * G + g) * 2] = mx[g];
                    lds_ml[(wave * G + g) * 2 + 1] = den[g];
                }
            }
        }
        __syncthreads();
        // the workgroup's state of q head g, feature f: the W wave states merged
        auto wg_state = [&](uint32_t g, uint32_t f, float& M, float& d, float& a) {
            M = -INFINITY;
            for (uint32_t w = 0; w < W; ++w)
                M = fmaxf(M, lds_ml[(w * G + g) * 2]);
            d = 0.0f;
            a = 0.0f;
            for (uint32_t w = 0; w < W; ++w) {
                const float mw = lds_ml[(w * G + g) * 2];
                const float weight = mw == -INFINITY ? 0.0f : fast_exp2(mw - M);
                d += lds_ml[(w * G + g) * 2 + 1] * weight;
                a += lds_acc[(w * G + g) * D + f] * weight;
            }
        };
        auto emit = [&](uint32_t g, uint32_t f, uint32_t it, float o) {
            const uint64_t at = ((uint64_t)row * q_heads + qh0 + g) * D + f;
            if constexpr (GATED)
                o *= sigmoid(it == 0 ? gate_early : load_elem<DT>(gate, at));
            store_elem<DT>(out, at, o);
        };
        if (n_chunks == 1) {
            uint32_t it = 0;
            for (uint32_t t = tid; t < G * D; t += blockDim.x, ++it) {
                float M, d, a;
                wg_state(t / D, t % D, M, d, a);
                emit(t / D, t % D, it, a / d);
            }
            return;
        }
        // a chunk of a cut row: record [max, denominator, 0, 0, acc[D]] per q head,
        // stored at agent scope (through to where every XCD reads it)
        constexpr uint32_t RF = D + 4;
        const uint64_t record_stride = (uint64_t)q_heads * RF; // between a row's chunks
        float* const records = split.records
            + ((uint64_t)m.split_first[row] * q_heads + qh0) * RF;
        for (uint32_t t = tid; t < G * D; t += blockDim.x) {
            const uint32_t g = t / D, f = t % D;
            float M, d, a;
            wg_state(g, f, M, d, a);
            float* rec = records + chunk * record_stride + g * RF;
            agent_store(rec + 4 + f, a);
            if (f == 0) {
                agent_store(rec, M);
                agent_store(rec + 1, d);
            }
        }
        // Arrival: every wave waits until its record stores are complete, then
        // one thread counts the chunk in. The chunk that arrives last resets the
        // counter and merges the row's records (agent-scope loads, so none comes
        // from a stale cache line); the others are done.
        wait_vector_memory();
        __syncthreads();
        uint32_t* const arrivals = split.arrivals + (uint64_t)m.split_first[row] * H + kv_head;
        uint32_t* const last_flag = reinterpret_cast<uint32_t*>(lds_ml); // lds_ml is read out
        if (tid == 0) {
            const uint32_t before =
                __hip_atomic_fetch_add(arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t last = before == n_chunks - 1;
            if (last)
                __hip_atomic_store(arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *last_flag = last;
        }
        __syncthreads();
        if (!*last_flag)
            return;
        // Thread (slice, g, f) folds chunks slice, slice + S, ... of q head g with
        // weights 2^(m_c - M) (paged_attention_reduce_f32,
        // src/metal/kernels/attention.metal:567-615, done online); the S slices are
        // folded through LDS and the result normalised, gated and rounded once.
        const uint32_t S = blockDim.x >= G * D ? blockDim.x / (G * D) : 1;
        for (uint32_t t = tid; t < S * G * D; t += blockDim.x) {
            const uint32_t slice = t / (G * D), g = (t / D) % G, f = t % D;
            const float* rec = records + g * RF;
            float M = -INFINITY, d = 0.0f, a = 0.0f;
            auto fold = [&](float mc, float dc, float ac) {
                const float nm = fmaxf(M, mc);
                const float keep = M == -INFINITY ? 0.0f : fast_exp2(M - nm);
                const float take = fast_exp2(mc - nm);
                d = d * keep + dc * take;
                a = a * keep + ac * take;
                M = nm;
            };
            uint32_t c = slice;
            for (; c + 3 * S < n_chunks; c += 4 * S) {
                float mc[4], dc[4], ac[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float* r = rec + (c + u * S) * record_stride;
                    mc[u] = agent_load(r);
                    dc[u] = agent_load(r + 1);
                    ac[u] = agent_load(r + 4 + f);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    fold(mc[u], dc[u], ac[u]);
            }
            for (; c < n_chunks; c += S) {
                const float* r = rec + c * record_stride;
                fold(agent_load(r), agent_load(r + 1), agent_load(r + 4 + f));
            }
            if (S == 1) {
                emit(g, f, 1, a / d);
                continue;
            }
            lds_acc[(slice * G + g) * D + f] = a;
            if (f == 0) {
                lds_ml[2 + (slice * G + g) * 2] = M;
                lds_ml[2 + (slice * G + g) * 2 + 1] = d;
            }
        }
        if (S == 1)
            return;
        __syncthreads();
        for (uint32_t t = tid; t < G * D; t += blockDim.x) {
            const uint32_t g = t / D, f = t % D;
            float M = -INFINITY;
            for (uint32_t sl = 0; sl < S; ++sl)
                M = fmaxf(M, lds_ml[2 + (sl * G + g) * 2]);
            float d = 0.0f, a = 0.0f;
            for (uint32_t sl = 0; sl < S; ++sl) {
                const float ms = lds_ml[2 + (sl * G + g) * 2];
                // a slice may hold no chunk
                const float w = ms == -INFINITY ? 0.0f : fast_exp2(ms - M);
                d += lds_ml[2 + (sl * G + g) * 2 + 1] * w;
                a += lds_acc[(sl * G + g) * D + f] * w;
            }
            emit(g, f, 1, a / d);
        }
    };

    // Workgroup blockIdx.x / H starts at that plan entry and follows the
    // entries' links through its segments.
    uint32_t at = blockIdx.x / H;
    for (;;) {
        // scalar loads (the plan is constant during the launch)
        using c4 = const __attribute__((address_space(4))) u32x4_t;
        const auto* e = (c4*)(uintptr_t)(m.plan + plan_entry_words * at);
        const u32x4_t a = e[0], b = e[1];
        const uint4 e0 = make_uint4(a.x, a.y, a.z, a.w);
        const uint4 e1 = make_uint4(b.x, b.y, b.z, b.w);
        segment(e0, e1);
        at = e1.w;
        if (at == plan_last)
            break;
        __syncthreads(); // the next segment's merge reuses the LDS
    }
}

// ---- generic path: any head_dim <= 1024, f32 / bf16 / fp16 ---------------------

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1)
        v += __shfl_xor(v, mask);
    return v;
}

constexpr int generic_max_features_per_lane = 16; // head_dim <= 1024

// Cut rows (shape_decode_plan). The balanced plan deals the batch's pages to
// split_wgs_per_cu workgroups of split_waves waves per compute unit (all of
// them resident at once), with a segment costing split_segment_pages pages
// and no piece shorter than split_min_piece; no more workgroups than rows
// where pieces would fall under split_min_pages, and no row in more than
// split_max_chunks pieces (the merge of a row reads its pieces' records:
// measured on MI355X, a 32K-token row cut into 128 chunks of 16 pages
// decodes in 24 us and merges in 7.5 us, in 32 chunks of 64 pages the pair
// takes 29 us in all). With more rows than workgroups, or under
// split_balance_min_pages pages per workgroup, the round trips of the
// segments a workgroup runs one after another cost more than the balance
// gains, and rows are cut into fixed chunks of a quarter of a compute unit's
// share instead (the config-5 churn took 3 % longer dealing its batches of
// hundreds of rows).
// Measured on one MI355X layer (bf16, 8 kv heads, fused append + decode,
// against fixed chunks throughout): batch 32 of U[256, 4096] tokens -2.8 %
// time (-0.7 % unfused), 32 rows of 1,024 tokens -14 %, of 4,096 -1.3 %,
// 64 rows of U[64, 2048] and one 32K-token row within 0.6 %.
constexpr uint64_t split_wgs_per_cu = 2;
constexpr uint64_t split_min_pages = 12;
constexpr uint64_t split_min_piece = 4;
constexpr uint64_t split_balance_min_pages = 32;
constexpr uint64_t split_per_share = 4;
constexpr uint64_t split_segment_pages = 4;
constexpr uint64_t split_max_chunks = 32;
constexpr uint32_t split_waves = 8;
// Waves per workgroup of a cut plan whose workgroups fit one per compute unit
// and hold at least split_alone_min_pages pages each (one long row's pieces):
// each wave holds one page in flight, and more waves per compute unit read
// faster (one 32K-token row, 64 pages per workgroup, 2.1-2.3 % faster than
// at 8 waves, a 64K-token row 1.3-2.4 %; 16 waves no faster than 8; at 32
// pages per workgroup even, at 16 pages 1.6-2.1 % slower)
constexpr uint32_t split_waves_alone = 12;
constexpr uint32_t split_alone_min_pages = 48;
// Pages (about 12 us of one workgroup's reads) by which the longest row may
// exceed 9/8 of a compute unit's share and still stay whole, for batches of
// one or two (row, kv head) units per compute unit. Measured on one
// MI355X layer (fused, bf16, 8 kv heads) against cutting: 32 rows of
// U[512, 1536] tokens -15 %, U[768, 1280] -9 %, 1,024 tokens -7 %, 2,048 -6 %,
// 64 rows of U[64, 2048] -5 %, 48 rows of U[256, 4096] -3.5 %; config 2's 32
// rows of U[256, 4096] (longest 256 pages, share 144) still cut, as do batches
// of fewer (row, kv head) units than compute units (8 rows of 1,024 tokens
// whole: +36 %).
constexpr uint64_t split_uncut_slack = 47;

// One wave per (work item, kv_head); the group's q heads are processed one
// after another, each with the per-token online softmax of
// paged_attention_f32 (src/metal/kernels/attention.metal:101-155), lanes
// striding the features.
template <int DT>
__global__ __launch_bounds__(64) void decode_generic_kernel(pool_view p, meta_view m, uint32_t layer,
                                                            const void* __restrict__ q,
                                                            uint32_t q_heads, float scale_log2,
                                                            void* __restrict__ out,
                                                            float* __restrict__ partials,
                                                            const void* __restrict__ gate)
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
                if (f < D) {
                    float o = acc[k] / den;
                    if (gate)
                        o *= sigmoid(load_elem<DT>(gate, q_base + f));
                    store_elem<DT>(out, q_base + f, o);
                }
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
                                                   void* __restrict__ out,
                                                   const void* __restrict__ gate)
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
        float o = a * inv;
        if (gate)
            o *= sigmoid(load_elem<DT>(gate, o_base + f));
        store_elem<DT>(out, o_base + f, o);
    }
}

bool aligned16(const void* ptr)
{
    return reinterpret_cast<uintptr_t>(ptr) % 16 == 0;
}

// Waves per workgroup of the fast path. With one or two q heads per KV head
// and at least one (row, kv head) unit per compute unit: 10 waves (one
// workgroup per CU), except for batches of at least 6 units per CU whose rows
// average under 256 pages, which take 8 (two workgroups per CU, so one's
// start and merge overlap the other's page reads). Measured on MI355X (one
// layer): with 6-16 units per CU, 8 waves is 0.6-9.5 % faster for mean rows
// of 50-160 pages, the two tie at 256 pages and 10 is 2.7 % faster at 288
// (config 3); with 1-2 units per CU, 8 waves is 7-16 % slower. A smaller
// batch takes the maximum (16, or 8 for wide lanes) so each row streams
// as fast as one CU allows. Chunks of cut rows take split_waves (a chunk is
// short, and several of them share a CU), or split_waves_alone when the
// plan's workgroups fit one per CU with enough pages each. f32 pages take 4 waves, two
// workgroups per CU at their two waves per SIMD: on config 2's shape 4, 6 and
// 8 waves measured 90.9, 97.9 and 96.6 us per launch, on config 3's 770, 768
// and 779 us (one box).
// CKV_DECODE_WAVES overrides.
uint32_t fast_waves(uint32_t group, int dtype, uint32_t units, int cu_count,
                    uint32_t mean_pages, uint32_t split_pages)
{
    const uint32_t limit = wide_lanes(group, dtype) ? 8u : 16u;
    if (const char* forced = std::getenv("CKV_DECODE_WAVES")) {
        const long v = std::strtol(forced, nullptr, 10);
        if (v >= 1 && v <= (long)limit)
            return (uint32_t)v;
    }
    if (dtype == CKV_F32)
        return 4;
    if (split_pages) {
        const bool alone = units <= (uint32_t)std::max(cu_count, 1)
            && split_pages >= split_alone_min_pages;
        return std::min(limit, alone ? split_waves_alone : split_waves);
    }
    if (limit > 10 && cu_count > 0 && units >= (uint32_t)cu_count)
        return units / (uint32_t)cu_count >= 6 && mean_pages < 256 ? 8 : 10;
    return limit;
}

template <int G>
hipError_t launch_fast(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                       const void* q, uint32_t q_heads, float scale_log2, void* out, int dt,
                       const void* k_in, const void* v_in, const void* gate, int cu_count,
                       split_scratch split, const rope_table* rope = nullptr,
                       uint32_t rotary = 0, uint32_t group_stride = G, uint32_t head_base = 0)
{
    if (!m.plan || (m.n_cut && (!split.records || !split.arrivals)))
        return hipErrorInvalidValue;
    if constexpr (G == 8) {
        // f32 pages at 8 q heads per kv head: two passes over 4 heads each (one
        // pass holds twice the registers its 512-lane workgroups allow); each
        // reads the K/V once more, the fused append writes the same token twice
        if (dt == CKV_F32) {
            hipError_t e = launch_fast<4>(s, p, m, layer, q, q_heads, scale_log2, out, dt, k_in,
                                          v_in, gate, cu_count, split, rope, rotary, 8, 0);
            if (e == hipSuccess)
                e = launch_fast<4>(s, p, m, layer, q, q_heads, scale_log2, out, dt, k_in, v_in,
                                   gate, cu_count, split, rope, rotary, 8, 4);
            return e;
        }
    }
    const uint32_t units = m.n_plan * p.kv_heads;
    const uint32_t waves = fast_waves(G, dt, units, cu_count, m.mean_pages, m.split_pages);
    const dim3 grid(units), block(64 * waves);
    // the merge's (acc, max, denominator) per wave, then the rope angle table
    const size_t lds = ((size_t)waves * G * (128 + 2) + (rope ? 2 * 64 : 0)) * sizeof(float);
    const auto qq = static_cast<const char*>(q);
    const auto ki = static_cast<const char*>(k_in);
    const auto vi = static_cast<const char*>(v_in);
    rope_table64 f64 = {};
    if (rope)
        for (uint32_t j = 0; j < rotary / 2; ++j)
            f64.inv_freq[j] = rope->inv_freq[j];
    // one instantiation per (dtype, fused, gated, rope); rope only when fused
    // and on 16-bit pages
    const int variant = (rope ? 16 : 0) | (dt << 2) | (k_in ? 2 : 0) | (gate ? 1 : 0);
    switch (variant) {
#define CKV_FAST_CASE(DT_, FUSED_, GATED_, ROPE_)                                              \
    case (ROPE_ ? 16 : 0) | (DT_ << 2) | (FUSED_ ? 2 : 0) | (GATED_ ? 1 : 0):                  \
        if constexpr (fast_fits(G, DT_))                                                       \
            decode_wg_kernel<G, DT_, FUSED_, GATED_, ROPE_><<<grid, block, lds, s>>>(          \
                p, m, layer, qq, q_heads, scale_log2, out, ki, vi, gate, f64, rotary, split,   \
                group_stride, head_base);                                                      \
        else                                                                                   \
            return hipErrorInvalidValue;                                                       \
        break;
        CKV_FAST_CASE(CKV_F32, false, false, false)
        CKV_FAST_CASE(CKV_F32, false, true, false)
        CKV_FAST_CASE(CKV_F32, true, false, false)
        CKV_FAST_CASE(CKV_F32, true, true, false)
        CKV_FAST_CASE(CKV_BF16, false, false, false)
        CKV_FAST_CASE(CKV_BF16, false, true, false)
        CKV_FAST_CASE(CKV_BF16, true, false, false)
        CKV_FAST_CASE(CKV_BF16, true, true, false)
        CKV_FAST_CASE(CKV_F16, false, false, false)
        CKV_FAST_CASE(CKV_F16, false, true, false)
        CKV_FAST_CASE(CKV_F16, true, false, false)
        CKV_FAST_CASE(CKV_F16, true, true, false)
        CKV_FAST_CASE(CKV_BF16, true, false, true)
        CKV_FAST_CASE(CKV_BF16, true, true, true)
        CKV_FAST_CASE(CKV_F16, true, false, true)
        CKV_FAST_CASE(CKV_F16, true, true, true)
#undef CKV_FAST_CASE
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Pages of a row at `position`, and the batch's total and longest.
void batch_pages(const std::vector<uint32_t>& positions, uint32_t block_size, uint64_t& total,
                 uint64_t& longest)
{
    total = longest = 0;
    for (const uint32_t p : positions) {
        const uint64_t pages = p / block_size + 1;
        total += pages;
        longest = std::max(longest, pages);
    }
}

// The balanced plan's segments: the batch's pages, row after row, dealt to
// `n` workgroups. A segment costs split_segment_pages pages of work besides
// its pages (its first loads and its merge wait on memory round trips), so
// the work dealt out (balanced_work) is the pages plus that cost for every
// segment, and workgroup k ends at ceil((k + 1) * work / n) of it. No row is
// cut into a piece shorter than split_min_piece pages (a workgroup takes such
// a rest with it, or ends early and leaves the row to the next one). Calls
// emit(row, first page, end page, workgroup) in row order; returns the
// workgroups used (at most n).
template <class Emit>
uint32_t balanced_segments(const std::vector<uint32_t>& positions, uint32_t block_size,
                           uint64_t work, uint64_t n, Emit&& emit)
{
    auto cut = [&](uint64_t i) { return (work * (i + 1) + n - 1) / n; };
    uint64_t k = 0; // the current workgroup's end, as an index of the cuts
    uint64_t end = cut(0), done = 0;
    uint32_t wg = 0;
    bool empty = true;
    auto next_wg = [&]() {
        ++wg;
        empty = true;
        if (k + 1 < n)
            end = cut(++k);
        while (k + 1 < n && end <= done)
            end = cut(++k);
    };
    for (size_t r = 0; r < positions.size(); ++r) {
        const uint64_t pages = positions[r] / block_size + 1;
        uint64_t pg = 0;
        while (pg < pages) {
            const uint64_t left = pages - pg;
            uint64_t take = left;
            if (k + 1 < n) { // the last workgroup takes what is left
                const uint64_t cost = done + split_segment_pages;
                take = std::min(left, end > cost ? end - cost : 0);
                if (take < left && take < split_min_piece) { // too short a piece to cut off
                    if (!empty) {
                        next_wg();
                        continue;
                    }
                    take = std::min(left, split_min_piece);
                }
                if (left - take < split_min_piece) // nor leave a short rest
                    take = left;
            }
            emit((uint32_t)r, (uint32_t)pg, (uint32_t)(pg + take), wg);
            empty = false;
            pg += take;
            done += take + split_segment_pages;
            if (k + 1 < n && done >= end)
                next_wg();
        }
    }
    return empty ? wg : wg + 1;
}

// The work balanced_segments deals out: the batch's pages plus the segment
// cost of as many segments as dealing that work makes (every row and every
// workgroup has one; found by dealing again until the count holds, at most
// four times), so the last workgroup's share comes out like the others.
uint64_t balanced_work(const std::vector<uint32_t>& positions, uint32_t block_size,
                       uint64_t total, uint64_t n)
{
    uint64_t segments = std::max<uint64_t>(positions.size(), n);
    for (int round = 0; round < 4; ++round) {
        uint64_t count = 0;
        balanced_segments(positions, block_size, total + split_segment_pages * segments, n,
                          [&](uint32_t, uint32_t, uint32_t, uint32_t) { ++count; });
        if (count == segments)
            break;
        segments = count;
    }
    return total + split_segment_pages * segments;
}

uint64_t forced_pages(const char* name, bool& set)
{
    const char* v = std::getenv(name);
    set = v != nullptr;
    return v ? (uint64_t)std::max(0L, std::strtol(v, nullptr, 10)) : 0;
}

} // namespace

uint32_t decode_fast_waves(uint32_t group, int dtype, uint32_t units, int cu_count,
                           uint32_t mean_pages, uint32_t split_pages)
{
    return fast_waves(group, dtype, units, cu_count, mean_pages, split_pages);
}

decode_plan_shape shape_decode_plan(const std::vector<uint32_t>& positions, uint32_t block_size,
                                    uint32_t kv_heads, int cu_count)
{
    const uint32_t rows = (uint32_t)positions.size();
    decode_plan_shape shape { 0, rows, 0, 0, rows, 0, 0, false };
    uint64_t total, longest;
    batch_pages(positions, block_size, total, longest);
    bool fixed_set, balanced_set;
    uint64_t span = forced_pages("CKV_DECODE_SPLIT", fixed_set);
    const uint64_t target = forced_pages("CKV_DECODE_BALANCE", balanced_set);
    uint64_t deal = 0; // workgroups per kv head the balanced plan deals the pages to
    if (balanced_set) {
        deal = target ? (total + target - 1) / target : 0;
    } else if (!fixed_set) {
        // a compute unit's share of the batch, in (page, kv head) units
        const uint64_t cus = (uint64_t)std::max(cu_count, 1);
        const uint64_t share = total * kv_heads / cus;
        // Rows stay whole when they give every compute unit one or two (row,
        // kv head) units and the longest is within split_uncut_slack of the
        // share: a cut costs its merge and second segment, about 12 us, and
        // the cut plan's pages run about 12 % slower than a whole row's. With
        // more units per compute unit the fixed chunks balance better (the
        // config-5 churn's batches of hundreds of rows: 1.5 % faster cut).
        const uint64_t units = (uint64_t)rows * kv_heads;
        const bool fill = units >= cus && units <= 2 * cus;
        if (2 * longest > share
            && (!fill || longest > share + share / 8 + split_uncut_slack)) {
            // as many workgroups as the GPU holds at once, but no more than a
            // row each where rows are short (pieces of at least
            // split_min_pages), nor more than split_max_chunks to a row
            const uint64_t slots = std::max<uint64_t>(1, cus * split_wgs_per_cu / kv_heads);
            const uint64_t piece = std::max(split_min_pages,
                                            (longest + split_max_chunks - 1) / split_max_chunks);
            deal = std::max<uint64_t>(1, std::min(slots, std::max<uint64_t>(rows, total / piece)));
            // More rows than workgroups (the balanced plan would run several
            // whole rows one after another in a workgroup, each paying its
            // round trips) or too little work per workgroup to pay for a
            // second segment: fixed chunks instead, a quarter of a compute
            // unit's share, dispatched longest first.
            if (rows > deal || total < deal * split_balance_min_pages) {
                deal = 0;
                span = std::max({ split_min_pages, (share + split_per_share - 1) / split_per_share,
                                  (longest + split_max_chunks - 1) / split_max_chunks });
                fixed_set = true;
            }
        }
    }
    uint64_t items = 0, records = 0, cut = 0, wgs = 0, per_wg = 0;
    if (deal) {
        uint32_t run_row = UINT32_MAX;
        uint64_t run = 0;
        auto close_run = [&]() {
            records += run > 1 ? run : 0;
            cut += run > 1 ? 1 : 0;
        };
        shape.deal_work = balanced_work(positions, block_size, total, deal);
        wgs = balanced_segments(positions, block_size, shape.deal_work, deal,
                                [&](uint32_t r, uint32_t, uint32_t, uint32_t) {
                                    ++items;
                                    if (r != run_row) {
                                        close_run();
                                        run_row = r;
                                        run = 0;
                                    }
                                    ++run;
                                });
        close_run();
        shape.balanced = true;
        per_wg = balanced_set ? target : (total + deal - 1) / deal;
    } else if (fixed_set && span && span < longest) {
        for (const uint32_t p : positions) {
            const uint64_t n = (p / block_size + span) / span; // chunks of (p / bs + 1) pages
            items += n;
            records += n > 1 ? n : 0;
            cut += n > 1 ? 1 : 0;
        }
        wgs = items;
        per_wg = span;
    } else {
        return shape; // a row per workgroup
    }
    if (items > UINT32_MAX / plan_entry_words || wgs > UINT32_MAX / kv_heads
        || records > UINT32_MAX / kv_heads)
        return decode_plan_shape { 0, rows, 0, 0, rows, 0, 0, false };
    shape.split_pages = (uint32_t)per_wg;
    shape.n_deal = (uint32_t)deal;
    shape.n_items = (uint32_t)items;
    shape.n_records = (uint32_t)records;
    shape.n_cut = (uint32_t)cut;
    shape.n_wgs = (uint32_t)wgs;
    return shape;
}

void write_decode_plan(const std::vector<uint32_t>& positions,
                       const std::vector<uint32_t>& offsets, uint32_t block_size,
                       const decode_plan_shape& shape, std::vector<uint64_t>& sort_keys,
                       uint32_t* plan, uint32_t* split_first, uint32_t* cut)
{
    const size_t rows = positions.size();
    const uint32_t span = shape.split_pages;
    auto entry = [&](size_t at, uint32_t r, uint32_t chunk, uint32_t first, uint32_t end,
                     uint32_t n_chunks, uint32_t next) {
        uint32_t* e = plan + plan_entry_words * at;
        e[0] = r;
        e[1] = chunk;
        e[2] = positions[r];
        e[3] = offsets[r] + first;
        e[4] = first;
        e[5] = end;
        e[6] = n_chunks;
        e[7] = next;
    };
    auto pages_of = [&](size_t r) { return positions[r] / block_size + 1; };
    if (!span) {
        // rows by decreasing position (ties in row order): the longest first
        sort_keys.resize(rows);
        for (size_t r = 0; r < rows; ++r)
            sort_keys[r] = ((uint64_t)(UINT32_MAX - positions[r]) << 32) | r;
        std::sort(sort_keys.begin(), sort_keys.end());
        for (size_t r = 0; r < rows; ++r) {
            const uint32_t row = (uint32_t)sort_keys[r];
            entry(r, row, 0, 0, pages_of(row), 1, plan_last);
            split_first[r] = 0;
        }
        return;
    }
    if (shape.balanced) {
        // the segments in row order, two words each: (row, first), (end, workgroup)
        sort_keys.clear();
        balanced_segments(positions, block_size, shape.deal_work, shape.n_deal,
                          [&](uint32_t r, uint32_t first, uint32_t end, uint32_t wg) {
                              sort_keys.push_back(((uint64_t)r << 32) | first);
                              sort_keys.push_back(((uint64_t)end << 32) | wg);
                          });
        // Dealt workgroup w runs as plan workgroup slot_of[w]: its first
        // segment is entry slot_of[w], its others follow the first segments in
        // order, each entry linking to the next.
        const size_t n = sort_keys.size() / 2;
        auto row_at = [&](size_t i) { return (uint32_t)(sort_keys[2 * i] >> 32); };
        auto wg_at = [&](size_t i) { return (uint32_t)sort_keys[2 * i + 1]; };
        // Workgroups with more segments take the lower slots: workgroups start
        // in slot order, one per compute unit before a second, and the second
        // to start on a compute unit loses issue to the first, so a workgroup
        // paying an extra segment's round trips should not also be the younger
        // (bit-identical; 32 rows of U[384, 3072] tokens 6 % faster, U[256,
        // 2560] 4 %, config 2 0.3 %).
        std::vector<uint32_t> segs(shape.n_wgs, 0), slot_of(shape.n_wgs);
        for (size_t i = 0; i < n; ++i)
            ++segs[wg_at(i)];
        {
            std::vector<uint32_t> order(shape.n_wgs);
            for (uint32_t w = 0; w < shape.n_wgs; ++w)
                order[w] = w;
            std::stable_sort(order.begin(), order.end(),
                             [&](uint32_t a, uint32_t b) { return segs[a] > segs[b]; });
            for (uint32_t k = 0; k < shape.n_wgs; ++k)
                slot_of[order[k]] = k;
        }
        std::fill(split_first, split_first + rows, 0u);
        size_t more = shape.n_wgs, n_cut = 0;
        uint32_t record = 0, run = 0, chunk = 0;
        for (size_t i = 0; i < n; ++i) {
            const uint32_t r = row_at(i), wg = wg_at(i);
            if (i == 0 || r != row_at(i - 1)) { // a row's first segment: count its segments
                run = 1;
                while (i + run < n && row_at(i + run) == r)
                    ++run;
                chunk = 0;
                if (run > 1) {
                    split_first[r] = record;
                    record += run;
                    cut[n_cut++] = r;
                }
            }
            const size_t at = i == 0 || wg != wg_at(i - 1) ? slot_of[wg] : more++;
            const uint32_t next = i + 1 < n && wg_at(i + 1) == wg ? (uint32_t)more : plan_last;
            const uint32_t first = (uint32_t)sort_keys[2 * i];
            const uint32_t end = (uint32_t)(sort_keys[2 * i + 1] >> 32);
            entry(at, r, chunk++, first, end, run, next);
        }
        return;
    }
    // fixed chunks by decreasing page count: the full chunks of every row (row
    // after row), then the short last chunks, longest first
    uint32_t record = 0;
    size_t at = 0, n_cut = 0;
    auto chunk_entry = [&](size_t at, uint32_t r, uint32_t c) {
        const uint32_t pages = pages_of(r);
        entry(at, r, c, c * span, std::min(c * span + span, pages), (pages + span - 1) / span,
              plan_last);
    };
    sort_keys.clear();
    for (size_t r = 0; r < rows; ++r) {
        const uint32_t pages = pages_of(r);
        const uint32_t n = (pages + span - 1) / span, full = pages / span;
        split_first[r] = n > 1 ? record : 0;
        record += n > 1 ? n : 0;
        if (n > 1)
            cut[n_cut++] = (uint32_t)r;
        for (uint32_t c = 0; c < full; ++c, ++at)
            chunk_entry(at, (uint32_t)r, c);
        if (full < n)
            sort_keys.push_back(((uint64_t)(span - (pages - full * span)) << 32) | r);
    }
    std::sort(sort_keys.begin(), sort_keys.end());
    for (const uint64_t key : sort_keys) {
        const uint32_t r = (uint32_t)key;
        chunk_entry(at++, r, pages_of(r) / span); // the last chunk
    }
}

bool decode_uses_fast_path(const pool_view& p, uint32_t q_heads)
{
    const uint32_t G = q_heads / p.kv_heads;
    // f32 at G = 8 runs as two passes of G = 4 (launch_fast<8>)
    return p.head_dim == 128 && p.block_size == 16
        && (G == 1 || G == 2 || G == 4 || G == 8)
        && (fast_fits(G, p.dtype) || (G == 8 && p.dtype == CKV_F32)) && aligned16(p.keys)
        && aligned16(p.values);
}

bool decode_fast_applies(const pool_view& p, uint32_t q_heads, const void* q, const void* out)
{
    return decode_uses_fast_path(p, q_heads) && aligned16(q) && aligned16(out);
}

hipError_t launch_decode(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                         const void* q, uint32_t q_heads, float scale, void* out,
                         float* partials, int cu_count, const void* gate, split_scratch split)
{
    if (!m.rows)
        return hipSuccess;
    const float scale_log2 = scale * log2e;
    if (decode_fast_applies(p, q_heads, q, out)) {
        const int dt = p.dtype;
        switch (q_heads / p.kv_heads) {
        case 1:
            return launch_fast<1>(s, p, m, layer, q, q_heads, scale_log2, out, dt, nullptr,
                                  nullptr, gate, cu_count, split);
        case 2:
            return launch_fast<2>(s, p, m, layer, q, q_heads, scale_log2, out, dt, nullptr,
                                  nullptr, gate, cu_count, split);
        case 4:
            return launch_fast<4>(s, p, m, layer, q, q_heads, scale_log2, out, dt, nullptr,
                                  nullptr, gate, cu_count, split);
        default:
            return launch_fast<8>(s, p, m, layer, q, q_heads, scale_log2, out, dt, nullptr,
                                  nullptr, gate, cu_count, split);
        }
    }
    if (p.head_dim > 64u * generic_max_features_per_lane)
        return hipErrorInvalidValue;
    const dim3 grid(m.n_items * p.kv_heads), block(64);
    switch (p.dtype) {
    case CKV_F32:
        decode_generic_kernel<CKV_F32><<<grid, block, 0, s>>>(p, m, layer, q, q_heads, scale_log2,
                                                              out, partials, gate);
        break;
    case CKV_BF16:
        decode_generic_kernel<CKV_BF16><<<grid, block, 0, s>>>(p, m, layer, q, q_heads,
                                                               scale_log2, out, partials, gate);
        break;
    default:
        decode_generic_kernel<CKV_F16><<<grid, block, 0, s>>>(p, m, layer, q, q_heads, scale_log2,
                                                              out, partials, gate);
        break;
    }
    return hipGetLastError();
}

hipError_t launch_append_decode(hipStream_t s, const pool_view& p, const meta_view& m,
                                uint32_t layer, const void* k_in, const void* v_in, const void* q,
                                uint32_t q_heads, float scale, void* out, const void* gate,
                                int cu_count, split_scratch split, const rope_table* rope,
                                uint32_t rotary)
{
    if (!m.rows)
        return hipSuccess;
    if (rope && (rotary < 16 || rotary > 128 || (rotary & (rotary - 1)) != 0))
        return hipErrorInvalidValue;
    const float scale_log2 = scale * log2e;
    const int dt = p.dtype;
    switch (q_heads / p.kv_heads) {
    case 1:
        return launch_fast<1>(s, p, m, layer, q, q_heads, scale_log2, out, dt, k_in, v_in, gate,
                              cu_count, split, rope, rotary);
    case 2:
        return launch_fast<2>(s, p, m, layer, q, q_heads, scale_log2, out, dt, k_in, v_in, gate,
                              cu_count, split, rope, rotary);
    case 4:
        return launch_fast<4>(s, p, m, layer, q, q_heads, scale_log2, out, dt, k_in, v_in, gate,
                              cu_count, split, rope, rotary);
    default:
        return launch_fast<8>(s, p, m, layer, q, q_heads, scale_log2, out, dt, k_in, v_in, gate,
                              cu_count, split, rope, rotary);
    }
}

hipError_t launch_merge(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t q_heads,
                        void* out, const float* partials, const void* gate)
{
    const dim3 grid(m.rows * q_heads), block(64);
    switch (p.dtype) {
    case CKV_F32:
        merge_kernel<CKV_F32><<<grid, block, 0, s>>>(m, q_heads, p.head_dim, partials, out, gate);
        break;
    case CKV_BF16:
        merge_kernel<CKV_BF16><<<grid, block, 0, s>>>(m, q_heads, p.head_dim, partials, out, gate);
        break;
    default:
        merge_kernel<CKV_F16><<<grid, block, 0, s>>>(m, q_heads, p.head_dim, partials, out, gate);
        break;
    }
    return hipGetLastError();
}

uint32_t partial_record_floats(uint32_t head_dim)
{
    return record_floats(head_dim);
}

} // namespace ckv

// Chunked-prefill causal attention over f32 pages on the matrix cores (gfx950).
//
// The maths of paged_flash_attention_prefill_f32
// (src/metal/kernels/attention.metal:246-444) in f32 throughout, as the
// reference computes it: q.k, the softmax and P.V in fp32, the products on
// v_mfma_f32_32x32x2_f32 (exact fp32 products, fp32 accumulation).
//
// Decomposition as for 16-bit pools: one workgroup of eight waves owns
// (256/G rows of a query tile, one kv head) and all G query heads of the
// head's GQA group; wave w holds the q-block (head w % G, rows 32*(w/G)..+31).
// Per 32-key block (two pages) and wave:
//   S^T[key][query] = K . Q^T   64 products of 2 features: A = K from LDS
//                                (lane (m, h) gives features 64h + j of key m),
//                                B = Q^T held in registers (lane (n, h):
//                                features 64h + j of query n), in two
//                                independent accumulator chains.
//   softmax                     lane (n, h) holds query n's scores of keys
//                                8*(r/4) + 4h + r%4 (its accumulator element
//                                r); the lane 32 apart holds the other 16.
//   O^T[feature][query] += V^T . P^T   step i takes key 8*(i/4) + 4h + i%4 in
//                                lane half h, so the B operand is the lane's
//                                own probability i; the A operand of
//                                accumulator c (0..3) is V[key][4m + c], so one
//                                16-byte LDS read feeds four products and row m
//                                of accumulator c is feature 4m + c.
// A product takes 64 cycles, so a block's 128 per wave (8,192 cycles) bound
// the kernel: the softmax's vector work and the LDS reads (32 KiB per wave and
// block) hide behind them.
//
// Staging: each block's K and V rows pass through registers into LDS (two
// stages; rows padded to 528 bytes, so the 32 key rows one K read touches
// start 16 bytes apart in the banks), the next block's loads in flight while
// the current one is multiplied, one barrier per block. Keys past the tile's
// last position are staged as zeros and never read from the pool.
//
// A launch that leaves compute units idle splits each long tile's key blocks
// between up to 8 workgroups, as the 16-bit kernel does (kernels_prefill.hip):
// each stores its unnormalised state as 16-byte records, and the last to
// arrive folds them in range order.
#include "ckv_internal.h"
#include "prefill_records.h"

namespace ckv {
namespace {

constexpr float log2e = 1.4426950408889634f;

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr uint32_t dim = 128;
constexpr uint32_t page_tokens = 16;
constexpr uint32_t block_keys = 32;
constexpr uint32_t waves = 8;
constexpr uint32_t row_pitch = dim * 4 + 16;              // bytes per staged key row
constexpr uint32_t tensor_bytes = block_keys * row_pitch; // one block of K (or V)
constexpr uint32_t stage_bytes = 2 * tensor_bytes;        // K, then V
constexpr uint32_t n_stages = 2;

__device__ __forceinline__ f32x16_t mfma(float a, float b, const f32x16_t& c)
{
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// 1 / (1 + e^-g) in float (src/metal/kernels/tensor_ops.metal:108-124 with sigmoid_only)
__device__ __forceinline__ float sigmoid(float g)
{
    return 1.0f / (1.0f + __builtin_amdgcn_exp2f(-g * log2e));
}

template <int G>
__global__ __launch_bounds__(64 * waves, 2) void prefill_f32_kernel(
    pool_view p, meta_view md, uint32_t layer, const float* __restrict__ q,
    float* __restrict__ out, uint32_t q_heads, float c, const float* __restrict__ gate,
    prefill_split split_scratch)
{
    __shared__ __attribute__((aligned(16))) uint8_t lds[n_stages * stage_bytes];
    constexpr uint32_t tile_rows = 256 / G;

    const uint32_t kv_heads = p.kv_heads;
    const uint32_t kvh = blockIdx.x % kv_heads;
    // key ranges vary slowest: every tile's first range is dispatched first
    const uint32_t n_split = split_scratch.n_split;
    const uint32_t n_rest = md.n_tiles * G;
    const uint32_t rest = blockIdx.x / kv_heads % n_rest;
    const uint32_t part = blockIdx.x / kv_heads / n_rest; // this workgroup's range of the keys
    const uint32_t sub = rest % G;
    const uint32_t tile = rest / G;
    // the tile: first row, rows, first position, table offset
    const uint4 te = *reinterpret_cast<const uint4*>(md.tiles + tile_entry_words * tile);
    const uint32_t count = te.y;
    const uint32_t r0 = sub * tile_rows;
    if (r0 >= count)
        return;
    const uint32_t nrows = min(tile_rows, count - r0);
    const uint32_t row0 = te.x + r0;
    const uint32_t pos0 = te.z + r0; // positions are consecutive inside a tile
    const uint32_t pos_last = pos0 + nrows - 1;
    const uint32_t* table = md.table + te.w;
    const uint32_t n_blocks = pos_last / block_keys + 1;
    const uint32_t last_entry = pos_last / page_tokens;
    // key blocks [kb_begin, kb_end) of this workgroup
    const uint32_t n_parts = prefill_range_count(n_blocks, n_split, split_scratch.min_blocks);
    if (part >= n_parts)
        return;
    uint32_t kb_begin, kb_end;
    prefill_range_bounds(n_blocks, n_parts, part, kb_begin, kb_end);

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const uint32_t n = lane & 31, h = lane >> 5;
    const uint64_t q_stride = (uint64_t)q_heads * dim;

    // this wave's q-block: head kvh * G + wave % G, tile rows 32 * (wave / G) + n
    const uint32_t head = kvh * G + wave % G;
    const uint32_t row = (wave / G) * 32 + n;
    const bool valid = row < nrows;
    const uint32_t qpos = pos0 + min(row, nrows - 1);
    const uint64_t qoff = (uint64_t)(row0 + min(row, nrows - 1)) * q_stride + (uint64_t)head * dim;
    // the q-block's first position, wave-uniform: blocks ending before it need
    // no mask (a scalar branch; 1.2 % faster on config 4)
    const uint32_t pos_lo = __builtin_amdgcn_readfirstlane(pos0 + (wave / G) * 32);

    // Q^T operands: features 64h .. 64h + 63 of query n
    float qr[64];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        const float4 v = valid ? *reinterpret_cast<const float4*>(q + qoff + 64 * h + 4 * t)
                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        qr[4 * t] = v.x;
        qr[4 * t + 1] = v.y;
        qr[4 * t + 2] = v.z;
        qr[4 * t + 3] = v.w;
    }

    // Staging: thread t moves 16 bytes of key rows t/32 and t/32 + 16 of the
    // block (one of each page), of K and of V.
    const uint64_t page_bytes = (uint64_t)page_tokens * p.features * 4;
    const uint64_t layer_bytes = p.layer_elems * 4;
    const uint8_t* kbase = static_cast<const uint8_t*>(p.keys) + layer * layer_bytes + kvh * dim * 4;
    const uint8_t* vbase = static_cast<const uint8_t*>(p.values) + layer * layer_bytes + kvh * dim * 4;
    const uint32_t sr = tid >> 5;
    const uint32_t scol = (tid & 31) * 16;
    const uint64_t srow = (uint64_t)sr * p.features * 4 + scol;
    uint4 k_a, k_b, v_a, v_b; // the staged 16 bytes of each page's K and V row
    auto fetch = [&](uint32_t kb) __attribute__((always_inline)) {
        const uint32_t key0 = kb * block_keys;
        const uint64_t pa = table[2 * kb];
        const uint64_t pb = table[min(2 * kb + 1, last_entry)];
        k_a = k_b = v_a = v_b = make_uint4(0, 0, 0, 0);
        if (key0 + sr <= pos_last) {
            k_a = *reinterpret_cast<const uint4*>(kbase + pa * page_bytes + srow);
            v_a = *reinterpret_cast<const uint4*>(vbase + pa * page_bytes + srow);
        }
        if (key0 + 16 + sr <= pos_last) {
            k_b = *reinterpret_cast<const uint4*>(kbase + pb * page_bytes + srow);
            v_b = *reinterpret_cast<const uint4*>(vbase + pb * page_bytes + srow);
        }
    };
    auto store = [&](uint32_t kb) __attribute__((always_inline)) {
        uint8_t* st = lds + (kb % n_stages) * stage_bytes + sr * row_pitch + scol;
        *reinterpret_cast<uint4*>(st) = k_a;
        *reinterpret_cast<uint4*>(st + 16 * row_pitch) = k_b;
        *reinterpret_cast<uint4*>(st + tensor_bytes) = v_a;
        *reinterpret_cast<uint4*>(st + tensor_bytes + 16 * row_pitch) = v_b;
    };

    f32x16_t o[4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
        o[a] = f32x16_t {};
    float m = -__builtin_inff(), l = 0.0f; // running maximum (log2 units), denominator share

    auto attend = [&](uint32_t kb) __attribute__((always_inline)) {
        const uint8_t* st = lds + (kb % n_stages) * stage_bytes;
        // S^T = K . Q^T
        const uint8_t* kr = st + n * row_pitch + h * 256;
        f32x16_t s0 = {}, s1 = {};
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const float4 kv = *reinterpret_cast<const float4*>(kr + 16 * t);
            s0 = mfma(kv.x, qr[4 * t], s0);
            s1 = mfma(kv.y, qr[4 * t + 1], s1);
            s0 = mfma(kv.z, qr[4 * t + 2], s0);
            s1 = mfma(kv.w, qr[4 * t + 3], s1);
        }
        // causal mask, scores in log2 units, the block maximum of the query
        const uint32_t key0 = kb * block_keys;
        float s[16];
        float mx = -__builtin_inff();
        if (key0 + block_keys - 1 <= pos_lo) { // every key precedes every query
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[r] = (s0[r] + s1[r]) * c;
                mx = fmaxf(mx, s[r]);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t key = key0 + 8 * (r >> 2) + 4 * h + (r & 3);
                s[r] = key <= qpos ? (s0[r] + s1[r]) * c : -__builtin_inff();
                mx = fmaxf(mx, s[r]);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        if (__any(mx > m)) {
            const float m_new = fmaxf(m, mx);
            const float alpha = m_new == -__builtin_inff() ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
            l *= alpha;
#pragma unroll
            for (int a = 0; a < 4; ++a)
                o[a] *= alpha;
            m = m_new;
        }
        // a range of the keys may hold none a query attends yet (m = -inf)
        const float mm = m == -__builtin_inff() ? 0.0f : m;
        float sum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s[r] = __builtin_amdgcn_exp2f(s[r] - mm);
            sum += s[r];
        }
        l += sum;
        // O^T += V^T . P^T
        const uint8_t* vr = st + tensor_bytes + 16 * n;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t key = 8 * (i >> 2) + 4 * h + (i & 3);
            const float4 vv = *reinterpret_cast<const float4*>(vr + key * row_pitch);
            o[0] = mfma(vv.x, s[i], o[0]);
            o[1] = mfma(vv.y, s[i], o[1]);
            o[2] = mfma(vv.z, s[i], o[2]);
            o[3] = mfma(vv.w, s[i], o[3]);
        }
    };

    fetch(kb_begin);
    store(kb_begin);
    __syncthreads();
    for (uint32_t kb = kb_begin; kb < kb_end; ++kb) {
        const bool more = kb + 1 < kb_end; // workgroup-uniform
        if (more)
            fetch(kb + 1);
        attend(kb);
        if (more)
            store(kb + 1); // stage (kb + 1) % 2 was last read in iteration kb - 1
        __syncthreads();
    }

    float lt = l + __shfl_xor(l, 32); // the query's denominator (both lane halves)
    if (n_parts > 1) {
        // A range of a split tile: its record is 33 chunks of 4 floats per query
        // vector, chunk 0 = [max (log2 units), denominator, 0, 0] and chunk
        // 1 + j = features 4j .. 4j + 3 (lane half h, element r of the four
        // accumulators: chunk 1 + 8 (r / 4) + 4h + r % 4), chunk-major with the
        // workgroup's 256 query vectors consecutive. The range that arrives
        // last folds every range's record in range order, two per round trip,
        // with weights 2^(m_s - M).
        const uint32_t pair = rest * kv_heads + kvh;
        const uint32_t qv = wave * 32 + n;
        constexpr uint32_t QV = 32 * waves, chunks = prefill_record_floats / 4;
        const __amdgpu_buffer_rsrc_t rs = record_rsrc(
            split_scratch.records + (uint64_t)pair * n_split * (chunks * QV * 4),
            n_split * chunks * QV * 16);
        auto off = [&](uint32_t share, uint32_t chunk) {
            return ((share * chunks + chunk) * QV + qv) * 16u;
        };
#pragma unroll
        for (int r = 0; r < 16; ++r)
            agent_store4(rs, off(part, 1 + 8 * (r >> 2) + 4 * h + (r & 3)), o[0][r], o[1][r],
                         o[2][r], o[3][r]);
        if (h == 0)
            agent_store4(rs, off(part, 0), m, lt, 0.0f, 0.0f);
        wait_vector_memory();
        __syncthreads(); // also: every wave is past its LDS reads
        uint32_t* const last_flag = reinterpret_cast<uint32_t*>(lds);
        if (tid == 0) {
            const uint32_t before = __hip_atomic_fetch_add(split_scratch.arrivals + pair, 1u,
                                                           __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t last = before == n_parts - 1;
            if (last)
                __hip_atomic_store(split_scratch.arrivals + pair, 0u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            *last_flag = last;
        }
        __syncthreads();
        if (!*last_flag)
            return;
        auto weight = [&](float ms, float to) { // 0 for a range that attended nothing
            return ms == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(ms - to);
        };
        float M = -__builtin_inff();
        lt = 0.0f;
#pragma unroll
        for (int a = 0; a < 4; ++a)
            o[a] = f32x16_t {};
        for (uint32_t sh = 0; sh < n_parts; sh += 2) {
            const uint32_t s1 = min(sh + 1, n_parts - 1);
            const u32x4_t ha = agent_load4(rs, off(sh, 0)), hb = agent_load4(rs, off(s1, 0));
            u32x4_t va[16], vb[16];
#pragma unroll
            for (int r = 0; r < 16; ++r)
                va[r] = agent_load4(rs, off(sh, 1 + 8 * (r >> 2) + 4 * h + (r & 3)));
#pragma unroll
            for (int r = 0; r < 16; ++r)
                vb[r] = agent_load4(rs, off(s1, 1 + 8 * (r >> 2) + 4 * h + (r & 3)));
            const float ma = __uint_as_float(ha[0]);
            const float mb = sh + 1 < n_parts ? __uint_as_float(hb[0]) : -__builtin_inff();
            const float m_new = fmaxf(M, fmaxf(ma, mb));
            const float keep = weight(M, m_new), wa = weight(ma, m_new), wb = weight(mb, m_new);
            M = m_new;
            lt = lt * keep + __uint_as_float(ha[1]) * wa;
            lt += __uint_as_float(hb[1]) * wb;
#pragma unroll
            for (int r = 0; r < 16; ++r)
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    float acc = o[a][r] * keep;
                    acc += __uint_as_float(va[r][a]) * wa;
                    o[a][r] = acc + __uint_as_float(vb[r][a]) * wb;
                }
        }
        // lt > 0 for a valid row: the tile's first range attends key 0
    }

    if (!valid)
        return;
    const float inv = 1.0f / lt;
    float* dst = out + qoff;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        // features 4 * (8 * (r / 4) + 4h + r % 4) + 0..3: accumulators 0..3
        const uint32_t f = 32 * (r >> 2) + 16 * h + 4 * (r & 3);
        float x[4] = { o[0][r] * inv, o[1][r] * inv, o[2][r] * inv, o[3][r] * inv };
        if (gate) { // sigmoid_mul (src/qwen/qwen_layer.cc:204) in the epilogue
            const float4 gv = *reinterpret_cast<const float4*>(gate + qoff + f);
            x[0] *= sigmoid(gv.x);
            x[1] *= sigmoid(gv.y);
            x[2] *= sigmoid(gv.z);
            x[3] *= sigmoid(gv.w);
        }
        *reinterpret_cast<float4*>(dst + f) = make_float4(x[0], x[1], x[2], x[3]);
    }
}

template <int G>
hipError_t launch_g(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                    const void* q, uint32_t q_heads, float c, void* out, uint32_t grid,
                    const void* gate, prefill_split split)
{
    hipLaunchKernelGGL((prefill_f32_kernel<G>), dim3(grid), dim3(64 * waves), 0, s, p, m, layer,
                       static_cast<const float*>(q), static_cast<float*>(out), q_heads, c,
                       static_cast<const float*>(gate), split);
    return hipGetLastError();
}

} // namespace

hipError_t launch_prefill_f32(hipStream_t s, const pool_view& p, const meta_view& m,
                              uint32_t layer, const void* q, uint32_t q_heads, float scale,
                              void* out, const void* gate, prefill_split split)
{
    const uint32_t group = q_heads / p.kv_heads;
    if (split.n_split < 1 || split.min_blocks < 1
        || (split.n_split > 1 && (!split.records || !split.arrivals)))
        return hipErrorInvalidValue;
    const uint64_t grid = (uint64_t)m.n_tiles * group * p.kv_heads * split.n_split;
    if (!grid)
        return hipSuccess;
    if (grid > 0x7FFFFFFFull)
        return hipErrorInvalidValue;
    const float c = scale * log2e;
    switch (group) {
    case 1:
        return launch_g<1>(s, p, m, layer, q, q_heads, c, out, (uint32_t)grid, gate, split);
    case 2:
        return launch_g<2>(s, p, m, layer, q, q_heads, c, out, (uint32_t)grid, gate, split);
    case 4:
        return launch_g<4>(s, p, m, layer, q, q_heads, c, out, (uint32_t)grid, gate, split);
    case 8:
        return launch_g<8>(s, p, m, layer, q, q_heads, c, out, (uint32_t)grid, gate, split);
    default:
        return hipErrorInvalidValue;
    }
}

} // namespace ckv

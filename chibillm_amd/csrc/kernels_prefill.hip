// Chunked-prefill causal attention over paged KV with MFMA tiles (gfx950).
//
// Maths of paged_flash_attention_prefill_f32 (src/metal/kernels/attention.metal:246-444):
// a query row at position p attends keys 0..p of its sequence through the
// block table, softmax(q.k * scale) weighted sum of v, with an online softmax
// over key blocks. The reference walks 8 query rows x 16-key tiles with
// scalar FMAs; here the dense products run on the matrix cores.
//
// Decomposition. A query tile is a run of rows of one sequence at consecutive
// positions (built at upload, at most 256 rows). One workgroup of four waves
// owns (256/G rows of a tile, one kv head) and all G query heads of that
// head's GQA group: 256 query vectors, 64 per wave in two q-blocks of 32
// (q-block b: head b % G, rows 32*(b / G)..). Every K/V byte of a key block
// is staged once per workgroup in LDS and used by all 256 query vectors.
//
// Per 32-key block (two pages) and q-block:
//   S^T[key][query] = K . Q^T    8 x v_mfma_f32_32x32x16 (A = K rows from
//                                LDS, B = Q held in registers)
//   online softmax              lane-local: lane l holds query l%32 and 16
//                                of the 32 keys, lane l^32 the other 16
//   O^T[feature][query] += V^T . P^T   8 x v_mfma_f32_32x32x16 (A = V^T
//                                from LDS, B = P^T straight from registers)
// With the 32x32 accumulator layout (element r of lane l sits at row
// 8*(r/4) + 4*(l/32) + r%4, column l%32), the S^T rows are mapped to
// physical keys with bits 2 and 3 swapped. Then the 8 probabilities a lane
// needs as the B operand of the next product (k = 8*(l/32) + e) are its own
// accumulator elements r = 8*step + e, physical keys 16*step + 8*(l/32) + e:
// no data moves between S and P. K rows are stored at row key_row(key);
// V is stored transposed ([feature][key], 2 keys per dword).
//
// Keys past the tile's last position are zero-filled (never read from the
// pool), so no page outside a row's table is touched and masked keys carry
// finite zeros into P.V.
#include "ckv_internal.h"

namespace ckv {
namespace {

constexpr float log2e = 1.4426950408889634f;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr uint32_t dim = 128;
constexpr uint32_t page_tokens = 16;
constexpr uint32_t block_keys = 32;
constexpr uint32_t threads = 256;
constexpr uint32_t k_row_bytes = 272;  // 256 + 16: rows 0..7 start in distinct 16-byte bank groups
constexpr uint32_t vt_row_bytes = 80;  // 64 + 16: likewise for 8 consecutive feature rows
constexpr uint32_t k_bytes = block_keys * k_row_bytes;
constexpr uint32_t vt_bytes = dim * vt_row_bytes;
constexpr uint32_t stage_bytes = k_bytes + vt_bytes;

// LDS row of physical key `key` in a block (an involution: bits 2 and 3 swapped).
__device__ __forceinline__ uint32_t key_row(uint32_t key)
{
    return (key & ~12u) | ((key & 4u) << 1) | ((key & 8u) >> 1);
}

// LDS row of feature f in the transposed V tile: rotated inside each group of
// 8 by the group index, so the 16 chunks written by one instruction spread
// over the banks while 8 consecutive features still occupy 8 distinct rows.
__device__ __forceinline__ uint32_t vt_row(uint32_t f)
{
    return (f & ~7u) | ((f + (f >> 3)) & 7u);
}

template <bool F16>
__device__ __forceinline__ f32x16_t mfma(uint4 a, uint4 b, f32x16_t c)
{
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Two floats to a packed 16-bit pair, round to nearest even.
template <bool F16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi)
{
    const f32x2_t v = { lo, hi };
    if constexpr (F16)
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
    else
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// One q-block's online-softmax step over the 16 scores this lane holds.
// Scores are raw q.k; c = scale * log2(e) so every exponential is one exp2.
// Returns the factor the accumulator must be multiplied by.
__device__ __forceinline__ float softmax_step(f32x16_t& s, float& m, float& l, float c)
{
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r)
        mx = fmaxf(mx, s[r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx);
    const float mc = m_new * c;
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        s[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, -mc));
        sum += s[r];
    }
    const float alpha = __builtin_amdgcn_exp2f((m - m_new) * c); // m = -inf at the start: 0
    l = l * alpha + sum;
    m = m_new;
    return alpha;
}

template <int G, bool F16>
__global__ __launch_bounds__(threads, 1) void prefill_kernel(pool_view p, meta_view md,
                                                             uint32_t layer,
                                                             const uint16_t* __restrict__ q,
                                                             uint16_t* __restrict__ out,
                                                             uint32_t q_heads, float c)
{
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * stage_bytes];
    constexpr uint32_t tile_rows = 256 / G;

    const uint32_t kv_heads = p.kv_heads;
    const uint32_t kvh = blockIdx.x % kv_heads; // consecutive workgroups: different heads/XCDs
    const uint32_t rest = blockIdx.x / kv_heads;
    const uint32_t sub = rest % G;
    const uint32_t tile = rest / G;
    const uint32_t count = md.tiles[2 * tile + 1];
    const uint32_t r0 = sub * tile_rows;
    if (r0 >= count)
        return;
    const uint32_t nrows = min(tile_rows, count - r0);
    const uint32_t row0 = md.tiles[2 * tile] + r0;
    const uint32_t pos0 = md.positions[row0];
    const uint32_t pos_last = pos0 + nrows - 1; // positions are consecutive inside a tile
    const uint32_t* table = md.table + md.offsets[row0];
    const uint32_t n_blocks = pos_last / block_keys + 1;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const uint32_t n = lane & 31, g = lane >> 5;
    const uint32_t F = p.features;
    const size_t q_stride = (size_t)q_heads * dim;

    // this wave's two q-blocks
    uint32_t head[2], qpos[2];
    size_t qoff[2];
    bool valid[2];
    uint32_t row_lo = ~0u, row_hi = 0;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const uint32_t b = 2 * wave + s;
        const uint32_t rb = b / G;
        head[s] = kvh * G + b % G;
        const uint32_t row = rb * 32 + n;
        valid[s] = row < nrows;
        qpos[s] = pos0 + min(row, nrows - 1);
        qoff[s] = (size_t)(row0 + min(row, nrows - 1)) * q_stride + (size_t)head[s] * dim;
        row_lo = min(row_lo, rb * 32);
        row_hi = max(row_hi, rb * 32 + 31);
    }
    const bool active = row_lo < nrows;
    const uint32_t pos_lo = pos0 + row_lo;
    const uint32_t pos_hi = pos0 + min(row_hi, nrows - 1);

    // Q^T operands: lane (n, g) holds features 16*ks + 8*g .. +7 of its query
    uint4 qr[2][8];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            qr[s][ks] = valid[s] && active
                ? *reinterpret_cast<const uint4*>(q + qoff[s] + ks * 16 + g * 8)
                : make_uint4(0, 0, 0, 0);

    const uint16_t* kbase = static_cast<const uint16_t*>(p.keys) + layer * p.layer_elems + kvh * dim;
    const uint16_t* vbase = static_cast<const uint16_t*>(p.values) + layer * p.layer_elems + kvh * dim;
    // staging roles: K row t/16 (+16), chunk t%16; V key pair t/16, chunk t%16
    const uint32_t srow = tid >> 4, chunk = tid & 15;

    uint4 kr[2], vr[2];
    auto load_block = [&](uint32_t kb) {
        const uint32_t key0 = kb * block_keys;
        const uint32_t pg0 = table[2 * kb];
        const uint32_t pg1 = key0 + page_tokens <= pos_last ? table[2 * kb + 1] : 0;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t key = 16 * i + srow;
            const size_t slot = (size_t)(i ? pg1 : pg0) * page_tokens + srow;
            kr[i] = key0 + key <= pos_last
                ? *reinterpret_cast<const uint4*>(kbase + slot * F + chunk * 8)
                : make_uint4(0, 0, 0, 0);
        }
        const uint32_t vpg = srow < 8 ? pg0 : pg1;
        const uint32_t vtok = (2 * srow) & 15;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const size_t slot = (size_t)vpg * page_tokens + vtok + i;
            vr[i] = key0 + 2 * srow + i <= pos_last
                ? *reinterpret_cast<const uint4*>(vbase + slot * F + chunk * 8)
                : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_block = [&](uint8_t* st) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            *reinterpret_cast<uint4*>(st + key_row(16 * i + srow) * k_row_bytes + chunk * 16) = kr[i];
        uint8_t* vt = st + k_bytes;
        const uint32_t w0[4] = { vr[0].x, vr[0].y, vr[0].z, vr[0].w };
        const uint32_t w1[4] = { vr[1].x, vr[1].y, vr[1].z, vr[1].w };
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            // features 8*chunk + 2d (low halves) and + 2d + 1 (high halves), keys (2*srow, +1)
            const uint32_t even = __builtin_amdgcn_perm(w1[d], w0[d], 0x05040100u);
            const uint32_t odd = __builtin_amdgcn_perm(w1[d], w0[d], 0x07060302u);
            const uint32_t f = 8 * chunk + 2 * d;
            *reinterpret_cast<uint32_t*>(vt + vt_row(f) * vt_row_bytes + 4 * srow) = even;
            *reinterpret_cast<uint32_t*>(vt + vt_row(f + 1) * vt_row_bytes + 4 * srow) = odd;
        }
    };

    f32x16_t o[2][4];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
            o[s][mt] = f32x16_t {};
    float m[2] = { -__builtin_inff(), -__builtin_inff() };
    float l[2] = { 0.0f, 0.0f };

    load_block(0);
    store_block(lds);
    __syncthreads();

    for (uint32_t kb = 0; kb < n_blocks; ++kb) {
        const bool more = kb + 1 < n_blocks;
        if (more)
            load_block(kb + 1);
        const uint8_t* st = lds + (kb & 1) * stage_bytes;
        const uint32_t key0 = kb * block_keys;
        if (active && key0 <= pos_hi) {
            f32x16_t sc[2] = { f32x16_t {}, f32x16_t {} };
            const uint8_t* krow = st + n * k_row_bytes + g * 16;
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const uint4 a = *reinterpret_cast<const uint4*>(krow + ks * 32);
                sc[0] = mfma<F16>(a, qr[0][ks], sc[0]);
                sc[1] = mfma<F16>(a, qr[1][ks], sc[1]);
            }
            if (key0 + block_keys - 1 > pos_lo) { // the causal diagonal crosses this block
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t kpos = key0 + 16 * (r >> 3) + 8 * g + (r & 7);
#pragma unroll
                    for (int s = 0; s < 2; ++s)
                        if (kpos > qpos[s])
                            sc[s][r] = -__builtin_inff();
                }
            }
            uint4 pt[2][2];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const float alpha = softmax_step(sc[s], m[s], l[s], c);
                if (__any(alpha != 1.0f)) {
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt)
                        o[s][mt] *= alpha;
                }
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    pt[s][h] = make_uint4(pack2<F16>(sc[s][8 * h + 0], sc[s][8 * h + 1]),
                                          pack2<F16>(sc[s][8 * h + 2], sc[s][8 * h + 3]),
                                          pack2<F16>(sc[s][8 * h + 4], sc[s][8 * h + 5]),
                                          pack2<F16>(sc[s][8 * h + 6], sc[s][8 * h + 7]));
            }
            const uint8_t* vt = st + k_bytes + g * 16;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const uint8_t* vrow = vt + vt_row(32 * mt + n) * vt_row_bytes;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint4 a = *reinterpret_cast<const uint4*>(vrow + h * 32);
                    o[0][mt] = mfma<F16>(a, pt[0][h], o[0][mt]);
                    o[1][mt] = mfma<F16>(a, pt[1][h], o[1][mt]);
                }
            }
        }
        if (more)
            store_block(lds + ((kb + 1) & 1) * stage_bytes);
        __syncthreads();
    }

    if (!active)
        return;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const float inv = 1.0f / (l[s] + __shfl_xor(l[s], 32));
        if (!valid[s])
            continue;
        uint16_t* dst = out + qoff[s];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int quad = 0; quad < 4; ++quad) {
                const uint32_t f = 32 * mt + 8 * quad + 4 * g;
                const f32x16_t& acc = o[s][mt];
                *reinterpret_cast<uint2*>(dst + f) =
                    make_uint2(pack2<F16>(acc[4 * quad] * inv, acc[4 * quad + 1] * inv),
                               pack2<F16>(acc[4 * quad + 2] * inv, acc[4 * quad + 3] * inv));
            }
    }
}

template <int G>
hipError_t launch_g(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                    const void* q, uint32_t q_heads, float c, void* out, uint32_t grid)
{
    const auto* qq = static_cast<const uint16_t*>(q);
    auto* oo = static_cast<uint16_t*>(out);
    if (p.dtype == CKV_F16)
        hipLaunchKernelGGL((prefill_kernel<G, true>), dim3(grid), dim3(threads), 0, s, p, m, layer,
                           qq, oo, q_heads, c);
    else
        hipLaunchKernelGGL((prefill_kernel<G, false>), dim3(grid), dim3(threads), 0, s, p, m,
                           layer, qq, oo, q_heads, c);
    return hipGetLastError();
}

bool aligned16(const void* ptr)
{
    return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0;
}

} // namespace

bool prefill_supported(const pool_view& p, uint32_t q_heads, const void* q, const void* out)
{
    if (p.dtype == CKV_F32 || p.head_dim != dim || p.block_size != page_tokens)
        return false;
    if (!p.kv_heads || q_heads % p.kv_heads)
        return false;
    const uint32_t group = q_heads / p.kv_heads;
    if (group != 1 && group != 2 && group != 4 && group != 8)
        return false;
    return aligned16(p.keys) && aligned16(p.values) && aligned16(q) && aligned16(out);
}

hipError_t launch_prefill(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                          const void* q, uint32_t q_heads, float scale, void* out)
{
    const uint32_t group = q_heads / p.kv_heads;
    const uint64_t grid = (uint64_t)m.n_tiles * group * p.kv_heads;
    if (!grid)
        return hipSuccess;
    if (grid > 0x7FFFFFFFull)
        return hipErrorInvalidValue;
    const float c = scale * log2e;
    switch (group) {
    case 1:
        return launch_g<1>(s, p, m, layer, q, q_heads, c, out, (uint32_t)grid);
    case 2:
        return launch_g<2>(s, p, m, layer, q, q_heads, c, out, (uint32_t)grid);
    case 4:
        return launch_g<4>(s, p, m, layer, q, q_heads, c, out, (uint32_t)grid);
    case 8:
        return launch_g<8>(s, p, m, layer, q, q_heads, c, out, (uint32_t)grid);
    default:
        return hipErrorInvalidValue;
    }
}

} // namespace ckv

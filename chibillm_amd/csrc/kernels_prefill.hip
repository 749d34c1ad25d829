// Chunked-prefill causal attention over paged KV with MFMA tiles (gfx950).
//
// Maths of paged_flash_attention_prefill_f32 (src/metal/kernels/attention.metal:246-444):
// a query row at position p attends keys 0..p of its sequence through the
// block table, softmax(q.k * scale) weighted sum of v, with an online softmax
// over key blocks. The reference walks 8 query rows x 16-key tiles with
// scalar FMAs; here the dense products run on the matrix cores.
//
// Decomposition. A query tile is a run of rows of one sequence at consecutive
// positions (built at upload, at most 256 rows). One workgroup of eight waves
// (two per SIMD) owns (256/G rows of a tile, one kv head) and all G query
// heads of that head's GQA group: 256 query vectors, one q-block of 32 per
// wave (wave w: head w % G, rows 32*(w / G)..). Every K/V byte of a key block
// is staged once per workgroup in LDS and used by all 256 query vectors.
// Launches too small to give every compute unit such a workgroup take four
// waves per workgroup instead (128/G rows, GQA groups up to 4), two to a
// compute unit.
//
// Per 32-key block (two pages) and wave:
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
// no data moves between S and P.
//
// Staging. K and V reach LDS by DMA (global_load_lds_dwordx4): each wave
// moves one 1 KiB K region and one V row group per block, no registers
// involved. Eight LDS stages; block kb + 4 is loaded while block kb is
// scored, and one barrier every two blocks publishes the next two, so each
// load has two to three iterations in flight. The block table entries are
// scalar loads, issued a block before their use; a page's address is a 32-bit
// offset from the layer's base (64-bit only for layers beyond 4 GiB).
//
// Keys past the tile's last position are read from a zero row (never from
// the pool), so no page outside a row's table is touched and masked keys
// carry finite zeros into P.V.
#include "ckv_internal.h"
#include "prefill_records.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace ckv {
namespace {

constexpr float log2e = 1.4426950408889634f;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t dim = 128;
constexpr uint32_t page_tokens = 16;
constexpr uint32_t block_keys = 32;

// K stage: already in the A-operand order of S^T = K.Q^T. Region ks (1 KiB)
// holds, at 16-byte slot l, what lane l = 32g + n reads for step ks:
// features 16ks + 8g .. +7 of LDS row n (physical key key_row(n)). Each wave
// fills one region with one DMA instruction, and every operand read is
// lane * 16 + ks * 1024, 256 contiguous bytes per 16 lanes.
constexpr uint32_t k_stage_bytes = 8 * 1024;
// V stage: the natural [key][feature] layout, read transposed
// (ds_read_b64_tr_b16) into the A operand of O^T += V^T P^T. A block's 32 key
// rows sit in 8 DMA groups of 4 rows (one 1 KiB wave instruction each) with
// 64 bytes after each group: key k is row (k/4)%4 of group k%4 + 4*(k/16),
// so the 8 keys one transposed read touches start at 4 different bank offsets.
constexpr uint32_t vg_bytes = 1024 + 64;
constexpr uint32_t v_stage_bytes = 8 * vg_bytes;
constexpr uint32_t stage_bytes = k_stage_bytes + v_stage_bytes;

// The source of masked (past the tile's last position) K and V rows: zeros,
// so that their zero probabilities multiply finite values.
__device__ const uint4 zero_row[16] = {};

// One 16-byte LDS DMA per lane: lane l's 16 bytes at `src` land at LDS byte
// address lds + 16 * l. Written out rather than through the compiler builtin,
// which makes the compiler wait for every outstanding DMA before any later
// LDS read; here completion is awaited explicitly (vmcnt) before the barrier
// that publishes the data. M0 (the LDS base) is saved and restored around
// the load, with the wait state its write needs before the load reads it.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds)
{
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %2\n\t"
                 "s_nop 0\n\t"
                 "global_load_lds_dwordx4 %1, off\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds)));
}

// The same with a scalar 64-bit base and a per-lane 32-bit byte offset: no
// vector address arithmetic.
__device__ __forceinline__ void dma16_s(const void* base, uint32_t voff, uint32_t lds)
{
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %3\n\t"
                 "s_nop 0\n\t"
                 "global_load_lds_dwordx4 %1, %2\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(voff), "s"(base), "s"(__builtin_amdgcn_readfirstlane(lds)));
}

// The K and V DMAs of one block, each with a scalar 64-bit base and a per-lane
// 32-bit byte offset, under one save and restore of M0.
__device__ __forceinline__ void dma16_pair(const void* kb, uint32_t koff, uint32_t klds,
                                           const void* vb, uint32_t voff, uint32_t vlds)
{
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %3\n\t"
                 "s_nop 0\n\t"
                 "global_load_lds_dwordx4 %1, %2\n\t"
                 "s_mov_b32 m0, %6\n\t"
                 "s_nop 0\n\t"
                 "global_load_lds_dwordx4 %4, %5\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(koff), "s"(kb), "s"(__builtin_amdgcn_readfirstlane(klds)), "v"(voff), "s"(vb),
                   "s"(__builtin_amdgcn_readfirstlane(vlds)));
}

// vmcnt wait (the other counters left alone) that lets `outstanding` of this
// wave's newest DMA loads (a K and a V load per region it stages per block)
// stay in flight.
__device__ __forceinline__ void wait_dma(uint32_t outstanding)
{
    if (outstanding >= 8)
        __builtin_amdgcn_s_waitcnt(0x0F78); // vmcnt(8)
    else if (outstanding >= 4)
        __builtin_amdgcn_s_waitcnt(0x0F74); // vmcnt(4)
    else if (outstanding >= 2)
        __builtin_amdgcn_s_waitcnt(0x0F72); // vmcnt(2)
    else
        __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0)
}

__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* ptr)
{
    const uint64_t v = (uint64_t)(uintptr_t)ptr;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const uint8_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// LDS row of physical key `key` in a block (an involution: bits 2 and 3 swapped).
__device__ __forceinline__ uint32_t key_row(uint32_t key)
{
    return (key & ~12u) | ((key & 4u) << 1) | ((key & 8u) >> 1);
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

template <bool F16>
__device__ __forceinline__ float half_value(uint16_t bits)
{
    if constexpr (F16)
        return static_cast<float>(__builtin_bit_cast(_Float16, bits));
    else
        return __builtin_bit_cast(float, static_cast<uint32_t>(bits) << 16);
}

// 1 / (1 + e^-g) in float (src/metal/kernels/tensor_ops.metal:108-124 with sigmoid_only)
__device__ __forceinline__ float sigmoid(float g)
{
    return 1.0f / (1.0f + __builtin_amdgcn_exp2f(-g * log2e));
}

// Growth of the running maximum (log2 units) that forces a rescale. Below it
// the probabilities keep using the older, smaller maximum and may reach
// 2^rescale_log2 (exact in fp32 and in the 16-bit P operand's exponent
// range); the final division by the denominator, accumulated with the same
// maximum, removes the offset exactly. Skipping the rescale of 64 fp32
// accumulators per block matters because on random data some lane of a
// 32-query block sees a new maximum in most key blocks.
constexpr float rescale_log2 = 8.0f;

// Maxima by v_maximum3_f32 (IEEE 754-2019 maximum: a NaN propagates, so the
// scores the matrix core writes need no quieting first, which fmaxf's maxNum
// would make the compiler insert).
__device__ __forceinline__ float max2(float a, float b)
{
    return __builtin_elementwise_maximum(a, b);
}

// The maximum of the 16 scores a lane holds, as a tree of three-input maxima
// (depth 3 instead of a chain of 8). Both lanes of a query compare their own
// maximum with the query's rescale threshold; only a rescale needs the pair's.
__device__ __forceinline__ float lane_max(const f32x16_t& s)
{
    const float a = max2(max2(s[0], s[1]), s[2]), b = max2(max2(s[3], s[4]), s[5]);
    const float d = max2(max2(s[6], s[7]), s[8]), e = max2(max2(s[9], s[10]), s[11]);
    const float f = max2(max2(s[12], s[13]), s[14]);
    return max2(max2(max2(a, b), d), max2(max2(e, f), s[15]));
}

// The maximum of a lane's value and its partner lane's (lane l ^ 32, the same
// query's other 16 keys). The partner is read with v_permlane32_swap, which
// exchanges the two 32-lane halves inside the VALU: of its two results, lanes
// 0-31 find the upper half's value in the second and lanes 32-63 the lower
// half's in the first, while the other result holds the lane's own value, so
// the maximum of all three is the pair's. A ds_bpermute would put an LDS
// round trip on the chain from the scores to the next block's exponentials.
__device__ __forceinline__ float pair_max(float mx)
{
    const uint32_t bits = __builtin_bit_cast(uint32_t, mx);
    const auto sw = __builtin_amdgcn_permlane32_swap(bits, bits, false, false);
    return max2(max2(mx, __builtin_bit_cast(float, (uint32_t)sw[0])),
                __builtin_bit_cast(float, (uint32_t)sw[1]));
}

// Probabilities of one q-block against the running maximum m (raw q.k
// units; c = scale * log2(e) so every exponential is one exp2), added to
// this lane's share of the denominator.
template <bool GUARD>
__device__ __forceinline__ void exponentiate(f32x16_t& s, float m, float& l, float c)
{
    // GUARD: a workgroup that attends only part of the keys may have seen no
    // unmasked key of a query yet (m = -inf); its probabilities are then 0
    const float mc = GUARD && m == -__builtin_inff() ? 0.0f : m * c;
#pragma unroll
    for (int r = 0; r < 16; ++r)
        s[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, -mc));
    // a tree of sums (depth 4 instead of a chain of 15)
    float q4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        q4[i] = (s[4 * i] + s[4 * i + 1]) + (s[4 * i + 2] + s[4 * i + 3]);
    l += (q4[0] + q4[1]) + (q4[2] + q4[3]);
}

// W waves per workgroup: 8 (two per SIMD, eight LDS stages), or 4 for
// launches that would leave compute units idle (one per SIMD, four stages,
// so two workgroups share a compute unit and twice as many run at once).
template <int W>
struct prefill_shape {
    static constexpr uint32_t stages = W == 8 ? 8 : 4;   // block kb in stage kb % stages
    static constexpr uint32_t regions = 8 / W;           // K regions and V groups a wave stages
    static constexpr uint32_t dmas = 2 * regions;        // DMA loads per block and wave
};

template <int G, bool F16, bool WIDE, int W>
__global__ __launch_bounds__(64 * W, 2) void prefill_kernel(
    pool_view p, meta_view md, uint32_t layer, const uint16_t* __restrict__ q,
    uint16_t* __restrict__ out, uint32_t q_heads, float c, const uint16_t* __restrict__ gate,
    prefill_split split_scratch)
{
    static_assert(W == 8 || (W == 4 && G <= 4), "a workgroup covers every q head of its group");
    // 4-wave workgroups may split a tile's key blocks between workgroups
    constexpr bool SPLIT = W == 4;
    using shape = prefill_shape<W>;
    constexpr uint32_t n_stages = shape::stages;
    constexpr uint32_t R = shape::regions;
    __shared__ __attribute__((aligned(16))) uint8_t lds[n_stages * stage_bytes];
    constexpr uint32_t tile_rows = 32 * W / G;
    constexpr uint32_t subs = 256 / tile_rows; // workgroups per (tile, kv head)

    const uint32_t kv_heads = p.kv_heads;
    const uint32_t kvh = blockIdx.x % kv_heads; // consecutive workgroups: different heads/XCDs
    // key ranges vary slowest: every tile's first range is dispatched before
    // any second one (ranges interleaved with the rows placed the ranges that
    // find no keys, and the long ones, unevenly: +5 to +29 % launch time)
    const uint32_t n_split = SPLIT ? split_scratch.n_split : 1;
    const uint32_t n_rest = md.n_tiles * subs;
    const uint32_t rest = blockIdx.x / kv_heads % n_rest;
    const uint32_t part = blockIdx.x / kv_heads / n_rest; // this workgroup's range of the keys
    const uint32_t sub = rest % subs;
    const uint32_t tile = rest / subs;
    // one scalar load gives the tile: first row, rows, first position, table offset
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
    // Key blocks [kb_begin, kb_end) of this workgroup: the tile's blocks cut
    // into n_parts ranges of at least min_blocks (uniform over the tile's
    // workgroups), range `part`.
    uint32_t n_parts = 1, kb_begin = 0, kb_end = n_blocks;
    if constexpr (SPLIT) {
        n_parts = prefill_range_count(n_blocks, n_split, split_scratch.min_blocks);
        if (part >= n_parts)
            return;
        prefill_range_bounds(n_blocks, n_parts, part, kb_begin, kb_end);
    } else {
        (void)part;
    }

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const uint32_t n = lane & 31, g = lane >> 5;
    const uint32_t F = p.features;
    const size_t q_stride = (size_t)q_heads * dim;

    // this wave's q-block: head kvh * G + wave % G, tile rows 32 * (wave / G) + n
    const uint32_t rb = wave / G;
    const uint32_t head = kvh * G + wave % G;
    const uint32_t row = rb * 32 + n;
    const bool valid = row < nrows;
    const bool active = rb * 32 < nrows;
    const uint32_t qpos = pos0 + min(row, nrows - 1);
    const size_t qoff = (size_t)(row0 + min(row, nrows - 1)) * q_stride + (size_t)head * dim;
    // the q-block's first position, wave-uniform: the diagonal test is a scalar branch
    const uint32_t pos_lo = __builtin_amdgcn_readfirstlane(pos0 + rb * 32);

    // Q^T operands: lane (n, g) holds features 16*ks + 8*g .. +7 of its query
    uint4 qr[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
        qr[ks] = valid ? *reinterpret_cast<const uint4*>(q + qoff + ks * 16 + g * 8)
                       : make_uint4(0, 0, 0, 0);

    const uint16_t* kbase = static_cast<const uint16_t*>(p.keys) + layer * p.layer_elems + kvh * dim;
    const uint16_t* vbase = static_cast<const uint16_t*>(p.values) + layer * p.layer_elems + kvh * dim;
    // K DMA: this lane's key (LDS row lane % 32) and features in the wave's
    // regions wave, wave + W, ...
    const uint32_t k_key = key_row(lane & 31);
    const bool k_hi = (lane & 31) >= 16; // the key is in the block's second page
    uint32_t k_feat[R], k_off[R], vd_key[R], v_off[R];
#pragma unroll
    for (uint32_t r = 0; r < R; ++r) {
        const uint32_t region = wave + r * W;
        k_feat[r] = 16 * region + 8 * (lane >> 5);
        k_off[r] = ((k_key & 15) * F + k_feat[r]) * 2; // bytes into the key's page
        // V DMA: this lane's key of the wave's group `region`
        vd_key[r] = 16 * (region >> 2) + 4 * (lane >> 4) + (region & 3);
        v_off[r] = ((vd_key[r] & 15) * F + (lane & 15) * 8) * 2;
    }
    const uint32_t vr_off = ((lane & 15) >> 2) * vg_bytes + (lane >> 5) * 512
        + ((lane >> 4) & 1) * 32 + (lane & 3) * 8;
    // DMA operands that do not change from block to block
    const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
    const uint32_t wave_u = __builtin_amdgcn_readfirstlane(wave);
    const size_t page_bytes = (size_t)page_tokens * F * 2;
    const uint32_t page_bytes32 = __builtin_amdgcn_readfirstlane((uint32_t)page_bytes);
    const uint8_t* kbytes = uniform_ptr(reinterpret_cast<const uint8_t*>(kbase));
    const uint8_t* vbytes = uniform_ptr(reinterpret_cast<const uint8_t*>(vbase));
    const uint8_t* zbytes = reinterpret_cast<const uint8_t*>(zero_row);
    auto stage_of = [&](uint32_t kb) { return lds + (kb % n_stages) * stage_bytes; };

    // Block table entries through the constant address space (scalar loads),
    // read one block before that block's loads are issued.
    uint32_t page_a = 0, page_b = 0;
    const uint32_t last_entry = pos_last / page_tokens; // the tile's last table entry
    auto fetch_pages_unchecked = [&](uint32_t kb) {
        using c32 = const __attribute__((address_space(4))) uint32_t;
        const auto* cb = (const __attribute__((address_space(4))) uint8_t*)(uintptr_t)table;
        page_a = *(c32*)(cb + 8 * kb);
        // the block's second page, or its first when the tile ends in the first
        page_b = *(c32*)(cb + 4 * min(2 * kb + 1, last_entry));
    };
    auto fetch_pages = [&](uint32_t kb) {
        if (kb < n_blocks)
            fetch_pages_unchecked(kb);
    };
    // K region `wave` and V group `wave` of block kb, into its stage
    // The K region `wave` and V group `wave` of a block whose 32 keys are all
    // in the tile, from pages pg0 and pg1, into LDS stage address st. A layer
    // spanning at most 4 GiB takes 32-bit page offsets from its base (two
    // scalar multiplies); a WIDE one 64-bit page addresses.
    auto load_full = [&](uint32_t pg0, uint32_t pg1, uint32_t st) {
#pragma unroll
        for (uint32_t r = 0; r < R; ++r) {
            const uint32_t region = wave_u + r * W;
            if constexpr (WIDE) {
                const uint8_t* k0 = kbytes + pg0 * page_bytes;
                const uint8_t* k1 = kbytes + pg1 * page_bytes;
                const uint8_t* vp = vbytes + (region >= 4 ? pg1 : pg0) * page_bytes;
                dma16((k_hi ? k1 : k0) + k_off[r], st + region * 1024);
                dma16_s(vp, v_off[r], st + k_stage_bytes + region * vg_bytes);
            } else {
                const uint32_t off0 = pg0 * page_bytes32, off1 = pg1 * page_bytes32;
                dma16_pair(kbytes, (k_hi ? off1 : off0) + k_off[r], st + region * 1024, vbytes,
                           (region >= 4 ? off1 : off0) + v_off[r],
                           st + k_stage_bytes + region * vg_bytes);
            }
        }
    };
    // load_block for a block whose keys are all in the tile and whose
    // successor exists (the page fetch needs no check)
    auto load_block_steady = [&](uint32_t kb) {
        const uint32_t pg0 = __builtin_amdgcn_readfirstlane(page_a);
        const uint32_t pg1 = __builtin_amdgcn_readfirstlane(page_b);
        fetch_pages_unchecked(kb + 1);
        load_full(pg0, pg1, lds_base + (kb % n_stages) * stage_bytes);
    };
    auto load_block = [&](uint32_t kb) {
        const uint32_t key0 = kb * block_keys;
        const uint32_t pg0 = __builtin_amdgcn_readfirstlane(page_a);
        const uint32_t pg1 = __builtin_amdgcn_readfirstlane(page_b);
        fetch_pages(kb + 1);
        const uint32_t st = lds_base + (kb % n_stages) * stage_bytes;
        if (key0 + block_keys - 1 <= pos_last) { // every key of the block is in the tile
            load_full(pg0, pg1, st);
        } else {
            const uint8_t* k0 = kbytes + pg0 * page_bytes;
            const uint8_t* k1 = kbytes + pg1 * page_bytes;
#pragma unroll
            for (uint32_t r = 0; r < R; ++r) {
                const uint32_t region = wave_u + r * W;
                const uint8_t* vp = vbytes + (region >= 4 ? pg1 : pg0) * page_bytes;
                const uint8_t* ksrc = key0 + k_key <= pos_last ? (k_hi ? k1 : k0) + k_off[r]
                                                               : zbytes + k_feat[r] * 2;
                dma16(ksrc, st + region * 1024);
                const uint8_t* vsrc = key0 + vd_key[r] <= pos_last ? vp + v_off[r]
                                                                   : zbytes + (lane & 15) * 16;
                dma16(vsrc, st + k_stage_bytes + region * vg_bytes);
            }
        }
    };

    f32x16_t o[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
        o[mt] = f32x16_t {};
    float m = -__builtin_inff(), l = 0.0f;
    // the running maximum past which a block's maxima force a rescale
    float m_limit = -__builtin_inff();
    const float rescale_raw = rescale_log2 / c;

    // Software pipeline over key blocks. Iteration kb issues S(kb) = K(kb) Q^T
    // on the matrix core while the vector ALU turns S(kb-1) into
    // probabilities, then P.V(kb-1) on the matrix core while the vector ALU
    // masks S(kb) and takes its maxima. The two halves of each iteration have
    // no dependence between their matrix and vector work, so one wave keeps
    // both units busy.
    f32x16_t sc; // S^T(kb), written by the matrix core
    f32x16_t sp; // S^T(kb - 1), its maxima taken, awaiting exponentials
    float mx = 0.0f;
    auto qk = [&](const uint4 (&ka)[8]) {
        sc = f32x16_t {};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            sc = mfma<F16>(ka[ks], qr[ks], sc);
    };
    auto read_k = [&](uint32_t kb, uint4 (&ka)[8]) {
        const uint8_t* kl = stage_of(kb) + lane * 16;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
            ka[ks] = *reinterpret_cast<const uint4*>(kl + ks * 1024);
    };
    auto read_v = [&](uint32_t kb, uint4 (&va)[4][2]) {
        // lane (n, g) of the A operand: features 32mt + n, keys 16h + 8g + 0..7,
        // two transposed reads of keys 4 at a time; one base register per
        // block, the 16 reads add immediate offsets
        uint32_t vaddr = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) uint8_t*)(
                             stage_of(kb) + k_stage_bytes))
            + vr_off;
        asm volatile("" : "+v"(vaddr));
        auto* vb = (__attribute__((address_space(3))) uint8_t*)(uintptr_t)vaddr;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) i16x4_t*)(vb + 4 * h * vg_bytes + 64 * mt));
                const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) i16x4_t*)(vb + 4 * h * vg_bytes + 256 + 64 * mt));
                const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
                va[mt][h] = make_uint4(l2.x, l2.y, h2.x, h2.y);
            }
    };
    auto probabilities = [&](uint4 (&pt)[2]) {
        exponentiate<SPLIT>(sp, m, l, c);
#pragma unroll
        for (int h = 0; h < 2; ++h)
            pt[h] = make_uint4(pack2<F16>(sp[8 * h + 0], sp[8 * h + 1]),
                               pack2<F16>(sp[8 * h + 2], sp[8 * h + 3]),
                               pack2<F16>(sp[8 * h + 4], sp[8 * h + 5]),
                               pack2<F16>(sp[8 * h + 6], sp[8 * h + 7]));
    };
    auto pv = [&](const uint4 (&va)[4][2], const uint4 (&pt)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                o[mt] = mfma<F16>(va[mt][h], pt[h], o[mt]);
    };
    // causal mask and maxima of S(kb); moves it to sp; true when some lane's
    // maximum grew past the rescale threshold (m = -inf before block 0).
    // `clear`: block kb is known to end before the q-block's first position.
    auto stats = [&](uint32_t kb, bool clear) {
        const uint32_t key0 = kb * block_keys;
        if (!clear && key0 + block_keys - 1 > pos_lo) { // the diagonal crosses this block
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t kpos = key0 + 16 * (r >> 3) + 8 * g + (r & 7);
                if (kpos > qpos)
                    sc[r] = -__builtin_inff();
            }
        }
        sp = sc;
        // the lane's own maximum decides: both halves of a query share m_limit
        mx = lane_max(sp);
        return __any(mx > m_limit);
    };
    auto rescale = [&]() {
        const float m_new = fmaxf(m, pair_max(mx));
        float alpha = __builtin_amdgcn_exp2f((m - m_new) * c); // 0 at the start
        if constexpr (SPLIT)
            alpha = m_new == -__builtin_inff() ? 1.0f : alpha; // nothing attended yet
        l *= alpha;
        m = m_new;
        m_limit = m_new + rescale_raw;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
            o[mt] *= alpha;
    };

    // This wave's loads newer than block b once it has issued block `last`.
    auto newer = [&](uint32_t b, uint32_t last) {
        const uint32_t top = min(last, kb_end - 1);
        return top > b ? shape::dmas * (top - b) : 0u;
    };
    if constexpr (W == 8) {
    // Blocks are loaded four ahead and published two at a time: the barrier
    // after an odd iteration kb waits for blocks kb + 1 and kb + 2, which the
    // next two iterations read. Block b is loaded in iteration b - 4 into the
    // stage of block b - 8, whose last read (V, iteration b - 7) precedes the
    // barrier after iteration b - 7 or b - 6.
    fetch_pages(0);
    for (uint32_t b = 0; b < 4; ++b)
        if (b < n_blocks)
            load_block(b);
    wait_dma(newer(1, 3));
    __syncthreads();
    // block 0: its scores and maxima (the first block always sets the maxima)
    {
        if (4 < n_blocks)
            load_block(4);
        uint4 ka[8];
        read_k(0, ka);
        qk(ka);
        stats(0, false);
        rescale();
    }
    // Iteration kb finishes block kb - 1 and scores block kb. The steady
    // state runs iterations in pairs (kb odd, kb + 1) while kb + 8 < n_blocks:
    // the blocks such a pair loads (kb + 4, kb + 5) hold only keys inside the
    // tile and the pages it fetches (blocks kb + 6, kb + 7) exist, so its loads,
    // fetches and waits take no checks, and the barrier's place is fixed (ODD).
    // Cutting the per-block scalar work this way (with the 32-bit page
    // offsets) made config 4's prefill 4.6 % faster.
    // A steady iteration's blocks end at least 193 positions before the tile's
    // last one ((kb + 2) * 32 <= (n_blocks - 7) * 32 <= pos_last - 192), so
    // with tiles of at most 128 rows (G >= 2) they end before the tile's first
    // position and need no mask: the scores' maxima then follow P.V in the
    // same basic block (1.2 % faster on config 4).
    constexpr bool steady_clear = G >= 2;
    auto iteration = [&](uint32_t kb, auto steady, auto odd, auto prio, uint32_t pa, uint32_t pb) {
        constexpr bool STEADY = decltype(steady)::value;
        if constexpr (STEADY)
            load_full(__builtin_amdgcn_readfirstlane(pa), __builtin_amdgcn_readfirstlane(pb),
                      lds_base + ((kb + 4) % n_stages) * stage_bytes);
        else if (kb + 4 < n_blocks)
            load_block(kb + 4);
        // The two waves of a SIMD (w and w + 4) take turns at the higher issue
        // priority block by block; with a fixed one the older runs ahead and
        // waits at the barrier (0.7 % faster on config 4; levels 0 and 3, four
        // levels, or turns every two blocks were 0.4 % faster to 1.8 % slower).
        // `prio` is the level when the caller knows it (0 or 1), else 2: the
        // level follows from the wave and the block, a branch per block.
        if constexpr (decltype(prio)::value == 1)
            __builtin_amdgcn_s_setprio(1);
        else if constexpr (decltype(prio)::value == 0)
            __builtin_amdgcn_s_setprio(0);
        else if (((wave_u >> 2) + kb) & 1)
            __builtin_amdgcn_s_setprio(1);
        else
            __builtin_amdgcn_s_setprio(0);
        uint4 ka[8], va[4][2];
        uint4 pt[2];
        read_k(kb, ka);
        // the K operand reads go out before the exponentials
        __builtin_amdgcn_sched_barrier(0);
        probabilities(pt); // vector: block kb - 1
        qk(ka);            // matrix: block kb
        read_v(kb - 1, va);
        pv(va, pt);                  // matrix: block kb - 1
        const bool grew = stats(kb, STEADY && steady_clear); // vector: block kb
        if (STEADY ? decltype(odd)::value : (kb & 1) != 0) {
            // this wave's loads of blocks kb + 1, kb + 2 (in the steady state
            // those of kb + 3 and kb + 4 stay in flight)
            wait_dma(STEADY ? 4u : newer(kb + 2, kb + 4));
            __syncthreads();
        }
        if (grew)
            rescale(); // before block kb's probabilities are formed
    };
    using yes = std::true_type;
    using no = std::false_type;
    using p0 = std::integral_constant<int, 0>;
    using p1 = std::integral_constant<int, 1>;
    using prt = std::integral_constant<int, 2>;
    uint32_t kb = 1;
    // The steady loop in two copies, one per half of the workgroup, so each
    // sets its priority levels without a branch (kb odd: waves 0-3 at 1, then
    // 0 at kb + 1; waves 4-7 the reverse): config 4 0.9-1.4 % faster. Its
    // pairs load blocks kb + 4 and kb + 5 from pages fetched by the pair
    // before; kb + 8 < n_blocks keeps those blocks inside the tile and the
    // fetched pages (blocks kb + 6 and kb + 7, neither the last) in the table.
    if (kb + 8 < n_blocks) {
        // pages of blocks kb + 4 (fetched by block 4's load) and kb + 5
        uint32_t a0 = page_a, b0 = page_b;
        fetch_pages_unchecked(kb + 5);
        uint32_t a1 = page_a, b1 = page_b;
        auto pairs = [&](auto first, auto second) {
            for (; kb + 8 < n_blocks; kb += 2) { // kb odd: a barrier follows it
                iteration(kb, yes {}, yes {}, first, a0, b0);
                iteration(kb + 1, yes {}, no {}, second, a1, b1);
                // the next pair's pages, carried into it: a fetch used in the
                // same trip is moved next to its use by the compiler, its
                // latency exposed once per pair (0.7-0.9 % slower)
                using c32 = const __attribute__((address_space(4))) uint32_t;
                const auto* cb = (const __attribute__((address_space(4))) uint8_t*)(uintptr_t)table;
                a0 = *(c32*)(cb + 8 * (kb + 6));
                b0 = *(c32*)(cb + 8 * (kb + 6) + 4);
                a1 = *(c32*)(cb + 8 * (kb + 7));
                b1 = *(c32*)(cb + 8 * (kb + 7) + 4);
            }
        };
        if (wave_u < 4)
            pairs(p1 {}, p0 {});
        else
            pairs(p0 {}, p1 {});
        page_a = a0; // block kb + 4, for the checked iterations
        page_b = b0;
    }
    for (; kb < n_blocks; ++kb)
        iteration(kb, no {}, no {}, prt {}, 0u, 0u);
    } else {
        // Four stages, loads two blocks ahead, a barrier after every block:
        // block b is loaded in iteration b - 2 into the stage of block b - 4,
        // whose last read (V, iteration b - 3) precedes the barrier after
        // iteration b - 3; the barrier after iteration kb waits for block
        // kb + 1, the next iteration's K.
        fetch_pages(kb_begin);
        load_block(kb_begin);
        if (kb_begin + 1 < kb_end)
            load_block(kb_begin + 1);
        wait_dma(0);
        __syncthreads();
        {
            if (kb_begin + 2 < kb_end)
                load_block(kb_begin + 2);
            uint4 ka[8];
            read_k(kb_begin, ka);
            qk(ka);
            stats(kb_begin, false);
            rescale();
        }
        // A steady iteration loads a block wholly inside the tile whose
        // successor's pages exist (kb + 3 < n_blocks) and inside its range, so
        // the load, the page fetch and the wait take no checks. (Skipping the
        // diagonal test as well, for G >= 2, was 0.3-0.7 % slower.)
        auto iteration4 = [&](uint32_t kb, auto steady) {
            constexpr bool STEADY = decltype(steady)::value;
            if constexpr (STEADY)
                load_block_steady(kb + 2);
            else if (kb + 2 < kb_end)
                load_block(kb + 2);
            uint4 ka[8], va[4][2];
            uint4 pt[2];
            read_k(kb, ka);
            __builtin_amdgcn_sched_barrier(0);
            probabilities(pt); // vector: block kb - 1
            qk(ka);            // matrix: block kb
            read_v(kb - 1, va);
            pv(va, pt); // matrix: block kb - 1
            const bool grew = stats(kb, false);
            wait_dma(STEADY ? shape::dmas : newer(kb + 1, kb + 2));
            __syncthreads();
            if (grew)
                rescale();
        };
        uint32_t kb = kb_begin + 1;
        for (; kb + 2 < kb_end && kb + 3 < n_blocks; ++kb)
            iteration4(kb, std::true_type {});
        for (; kb < kb_end; ++kb)
            iteration4(kb, std::false_type {});
    }
    // the last block's probabilities and product
    {
        uint4 va[4][2];
        uint4 pt[2];
        probabilities(pt);
        read_v(kb_end - 1, va);
        pv(va, pt);
    }

    float lt = l + __shfl_xor(l, 32); // the query's denominator (both lane halves)
    if (SPLIT && n_parts > 1) {
        // A share of a split tile: its record is 33 chunks of 4 floats per
        // query vector, chunk 0 = [max, denominator, 0, 0] and chunk 1 + j =
        // acc[4j .. 4j + 3], chunk-major with the workgroup's 128 query vectors
        // consecutive, so the 32 lanes of a wave half fill 512 contiguous
        // bytes per access. The share that arrives last folds every share's
        // record, its own included, in share order (the result does not
        // depend on the order of arrival), with weights 2^(m_s - M).
        const uint32_t pair = (tile * subs + sub) * kv_heads + kvh;
        const uint32_t qv = wave * 32 + n; // this lane's query vector in the workgroup
        constexpr uint32_t QV = 32 * W, chunks = prefill_record_floats / 4;
        const __amdgpu_buffer_rsrc_t rs = record_rsrc(
            split_scratch.records + (uint64_t)pair * n_split * (chunks * QV * 4),
            n_split * chunks * QV * 16);
        auto off = [&](uint32_t share, uint32_t chunk) {
            return ((share * chunks + chunk) * QV + qv) * 16u;
        };
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int quad = 0; quad < 4; ++quad) {
                const f32x16_t& acc = o[mt];
                agent_store4(rs, off(part, 1 + 8 * mt + 2 * quad + g), acc[4 * quad],
                             acc[4 * quad + 1], acc[4 * quad + 2], acc[4 * quad + 3]);
            }
        if (g == 0)
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
        // online over the shares, two per round trip: the running state
        // (M, lt, o) is rescaled by 2^(M - M') when a share raises the maximum
        float M = -__builtin_inff();
        auto weight = [&](float ms, float to) { // 0 for a share that attended nothing
            return ms == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f((ms - to) * c);
        };
        lt = 0.0f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
            o[mt] = f32x16_t {};
        for (uint32_t s = 0; s < n_parts; s += 2) {
            const uint32_t s1 = min(s + 1, n_parts - 1);
            u32x4_t ha = agent_load4(rs, off(s, 0)), hb = agent_load4(rs, off(s1, 0));
            u32x4_t va[16], vb[16];
#pragma unroll
            for (int j = 0; j < 16; ++j)
                va[j] = agent_load4(rs, off(s, 1 + 2 * j + g));
#pragma unroll
            for (int j = 0; j < 16; ++j)
                vb[j] = agent_load4(rs, off(s1, 1 + 2 * j + g));
            const float ma = __uint_as_float(ha[0]);
            const float mb = s + 1 < n_parts ? __uint_as_float(hb[0]) : -__builtin_inff();
            const float m_new = fmaxf(M, fmaxf(ma, mb));
            const float keep = weight(M, m_new), wa = weight(ma, m_new), wb = weight(mb, m_new);
            M = m_new;
            lt = lt * keep + __uint_as_float(ha[1]) * wa;
            lt += __uint_as_float(hb[1]) * wb;
#pragma unroll
            for (int j = 0; j < 16; ++j) // chunk 1 + 2j + g = features 32mt + 8quad + 4g + e
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float acc = o[j / 4][4 * (j % 4) + e] * keep;
                    acc += __uint_as_float(va[j][e]) * wa;
                    o[j / 4][4 * (j % 4) + e] = acc + __uint_as_float(vb[j][e]) * wb;
                }
        }
        // lt > 0 for a valid row: the tile's first share attends key 0
    }

    if (!active || !valid)
        return;
    const float inv = 1.0f / lt;
    uint16_t* dst = out + qoff;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int quad = 0; quad < 4; ++quad) {
            const uint32_t f = 32 * mt + 8 * quad + 4 * g;
            const f32x16_t& acc = o[mt];
            float x[4] = { acc[4 * quad] * inv, acc[4 * quad + 1] * inv,
                           acc[4 * quad + 2] * inv, acc[4 * quad + 3] * inv };
            if (gate) { // sigmoid_mul (src/qwen/qwen_layer.cc:204) in the epilogue
                const uint2 gv = *reinterpret_cast<const uint2*>(gate + qoff + f);
                const uint32_t w[2] = { gv.x, gv.y };
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    x[e] *= sigmoid(half_value<F16>((uint16_t)(w[e / 2] >> (16 * (e % 2)))));
            }
            *reinterpret_cast<uint2*>(dst + f) =
                make_uint2(pack2<F16>(x[0], x[1]), pack2<F16>(x[2], x[3]));
        }
}

template <int G, int W>
hipError_t launch_gw(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                     const void* q, uint32_t q_heads, float c, void* out, const void* gate,
                     prefill_split split)
{
    const uint64_t grid = (uint64_t)m.n_tiles * (256 / (32 * W / G)) * p.kv_heads
        * (W == 4 ? split.n_split : 1);
    if (!grid)
        return hipSuccess;
    if (grid > 0x7FFFFFFFull)
        return hipErrorInvalidValue;
    const auto* qq = static_cast<const uint16_t*>(q);
    auto* oo = static_cast<uint16_t*>(out);
    const auto* gg = static_cast<const uint16_t*>(gate);
    // a layer's K (or V) span beyond 4 GiB needs 64-bit page addresses
    const bool wide = p.layer_elems * 2 > 0xFFFFFFFFull;
    const bool f16 = p.dtype == CKV_F16;
    const dim3 g((uint32_t)grid), b(64 * W);
    if (f16 && wide)
        hipLaunchKernelGGL((prefill_kernel<G, true, true, W>), g, b, 0, s, p, m, layer, qq, oo,
                           q_heads, c, gg, split);
    else if (f16)
        hipLaunchKernelGGL((prefill_kernel<G, true, false, W>), g, b, 0, s, p, m, layer, qq, oo,
                           q_heads, c, gg, split);
    else if (wide)
        hipLaunchKernelGGL((prefill_kernel<G, false, true, W>), g, b, 0, s, p, m, layer, qq, oo,
                           q_heads, c, gg, split);
    else
        hipLaunchKernelGGL((prefill_kernel<G, false, false, W>), g, b, 0, s, p, m, layer, qq, oo,
                           q_heads, c, gg, split);
    return hipGetLastError();
}

template <int G>
hipError_t launch_g(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                    const void* q, uint32_t q_heads, float c, void* out, const void* gate,
                    const prefill_shape_info& plan, prefill_split split)
{
    if constexpr (G <= 4) {
        if (plan.waves == 4)
            return launch_gw<G, 4>(s, p, m, layer, q, q_heads, c, out, gate, split);
    }
    split.n_split = 1;
    return launch_gw<G, 8>(s, p, m, layer, q, q_heads, c, out, gate, split);
}

bool aligned16(const void* ptr)
{
    return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0;
}

} // namespace

bool prefill_supported(const pool_view& p, uint32_t q_heads, const void* q, const void* out)
{
    if (p.head_dim != dim || p.block_size != page_tokens)
        return false;
    if (!p.kv_heads || q_heads % p.kv_heads)
        return false;
    const uint32_t group = q_heads / p.kv_heads;
    if (group != 1 && group != 2 && group != 4 && group != 8)
        return false;
    return aligned16(p.keys) && aligned16(p.values) && aligned16(q) && aligned16(out);
}

// A launch of 8-wave workgroups (one per compute unit: their LDS stages take
// 135 KB) that would not give every compute unit one, or would end on a
// partial round, takes 4-wave workgroups instead, two to a compute unit (GQA
// groups up to 4); if those still leave
// compute units idle, each tile's key blocks are split between as many
// workgroups as fill them (at most split_max, each attending at least
// split_min_blocks blocks; the kernel takes fewer for short tiles).
// CKV_PREFILL_WAVES (4 or 8), CKV_PREFILL_SPLIT and CKV_PREFILL_SPLIT_MIN (blocks) override.
// a launch of more than half a round of 8-wave workgroups, and less than one,
// takes 4-wave workgroups unless its shortest tile attends more 32-key blocks
constexpr uint32_t sub_round_max_blocks = 40;

prefill_shape_info prefill_plan(const pool_view& p, const meta_view& m, uint32_t q_heads,
                                int cu_count)
{
    prefill_shape_info plan { 8, 1, split_min_blocks, 0, 0 };
    const uint32_t group = p.kv_heads ? q_heads / p.kv_heads : 0;
    if (const char* forced = std::getenv("CKV_PREFILL_SPLIT_MIN"))
        plan.min_blocks = (uint32_t)std::max(1L, std::strtol(forced, nullptr, 10));
    if (p.dtype == CKV_F32) {
        // f32 pools: 8-wave workgroups, two to a compute unit; a launch that
        // gives at most one to each splits its long tiles' keys to fill them
        const uint64_t grid = (uint64_t)m.n_tiles * group * p.kv_heads;
        uint64_t split = grid && cu_count > 0 && grid <= (uint64_t)cu_count
            ? 2 * (uint64_t)cu_count / grid
            : 1;
        if (const char* forced = std::getenv("CKV_PREFILL_SPLIT"))
            split = (uint64_t)std::max(1L, std::strtol(forced, nullptr, 10));
        plan.n_split = (uint32_t)std::min<uint64_t>(std::max<uint64_t>(split, 1), split_max);
        if (plan.n_split > 1) {
            plan.records_floats = grid * plan.n_split * 256 * prefill_record_floats;
            plan.counters = grid;
        }
        return plan;
    }
    if (group == 0 || group > 4)
        return plan;
    const uint64_t grid8 = (uint64_t)m.n_tiles * group * p.kv_heads;
    const uint64_t cus = cu_count > 0 ? (uint64_t)cu_count : 0;
    // Fewer 8-wave workgroups than compute units; or, under three rounds of
    // them, a last round at most 5/8 full, whose compute units would wait
    // out the others' tiles (4-wave workgroups, half the rows each, pack it:
    // 9-12 sequences of config 4's shape 5-7 % faster, 17 and 20 3.5-6 %;
    // full rounds or a last round 3/4 full are 3.5-8 % slower in 4-wave form).
    // Under one round, 4-wave workgroups fill the compute units, and split
    // long tiles' keys while at most half of them hold an 8-wave workgroup;
    // past half, without a split, they lose to 8-wave workgroups when every
    // tile is long (6 sequences of 512 rows over 0 or 512 tokens 15 % and 7 %
    // faster in 4-wave form, over 1,008, 2,000 and 6,000 tokens 1 %, 5 % and
    // 12 % slower); batches that mix short and long tiles (the churn's) keep
    // the 4-wave form, whose smaller workgroups even out the tiles' lengths.
    const uint64_t rem = cus ? grid8 % cus : 0;
    bool small = false;
    if (cus && grid8 < cus)
        small = 2 * grid8 <= cus || m.tile_blocks <= sub_round_max_blocks;
    else if (cus)
        small = grid8 < 3 * cus && rem > 0 && rem * 8 <= cus * 5;
    if (const char* forced = std::getenv("CKV_PREFILL_WAVES"))
        small = std::strtol(forced, nullptr, 10) == 4;
    if (!small)
        return plan;
    plan.waves = 4;
    const uint64_t pairs = grid8 * 2; // 4-wave workgroups
    uint64_t split = pairs && cu_count > 0 ? 2 * (uint64_t)cu_count / pairs : 1;
    if (const char* forced = std::getenv("CKV_PREFILL_SPLIT"))
        split = (uint64_t)std::max(1L, std::strtol(forced, nullptr, 10));
    plan.n_split = (uint32_t)std::min<uint64_t>(std::max<uint64_t>(split, 1), split_max);
    if (plan.n_split > 1) {
        plan.records_floats = pairs * plan.n_split * 128 * prefill_record_floats;
        plan.counters = pairs;
    }
    return plan;
}

hipError_t launch_prefill(hipStream_t s, const pool_view& p, const meta_view& m, uint32_t layer,
                          const void* q, uint32_t q_heads, float scale, void* out,
                          const void* gate, const prefill_shape_info& plan,
                          prefill_split split)
{
    if (plan.n_split > 1 && (!split.records || !split.arrivals))
        return hipErrorInvalidValue;
    split.n_split = plan.n_split;
    split.min_blocks = plan.min_blocks;
    if (p.dtype == CKV_F32)
        return launch_prefill_f32(s, p, m, layer, q, q_heads, scale, out, gate, split);
    const float c = scale * log2e;
    switch (q_heads / p.kv_heads) {
    case 1:
        return launch_g<1>(s, p, m, layer, q, q_heads, c, out, gate, plan, split);
    case 2:
        return launch_g<2>(s, p, m, layer, q, q_heads, c, out, gate, plan, split);
    case 4:
        return launch_g<4>(s, p, m, layer, q, q_heads, c, out, gate, plan, split);
    case 8:
        return launch_g<8>(s, p, m, layer, q, q_heads, c, out, gate, plan, split);
    default:
        return hipErrorInvalidValue;
    }
}

} // namespace ckv

// chunked_prefill.hip -- causal paged attention for prefill chunks on gfx950
// bf16 MFMA (FlashAttention-2 style, online softmax, fp32 accumulation).
//
// Math: crates/engine/src/backend/cpu/attention.rs:5-16 (prefill path,
// cpu/mod.rs:287-312).  Row t of sequence s sits at position p = ctx_s + i
// and attends to keys 0..p of its sequence through the block table; the
// cached context is fully visible and the chunk is causal because row t is
// given only p + 1 keys (attention.rs:16).
//
// Work split.  A work item is a 64-row query tile of one sequence (host
// plan, longest first).  A workgroup owns R 32-row groups of one item and one
// KV head k, with one wavefront per (row group, query head of k's GQA group):
// R = 2 for groups up to 4 heads (8 waves), R = 1 with two workgroups per item
// for 8 heads, so that every K/V tile staged in LDS serves 64 rows x G heads
// and the pool is read once per 64 query rows.  The workgroup walks the
// 64-key KV tiles 0 .. p_max/64 of its sequence; tiles past its last row are
// never touched, tiles wholly before a wave's first row need no mask.  The
// grid runs KV heads fastest: workgroups are dealt to the 8 XCDs round-robin,
// so with 8 (or 16 ..) KV heads every (sequence, KV head) stream stays in one
// XCD's L2 and its q tiles, which walk the same KV tiles at the same pace,
// share the loads.
//
// Per wavefront and KV tile (keys j0 .. j0+63), with c = lane % 32 the query
// row of the lane within its row group and gl = lane / 32:
//   S^T = K . Q^T    v_mfma_f32_32x32x16_bf16, A = 32 keys x 16 dims of K
//                    from LDS, B = Q^T (the wave's 32 query rows, kept in
//                    registers for the whole kernel); two 32-key halves,
//                    head_dim/16 steps each.  A-row i reads key pi(i), pi =
//                    swap of bits 2 and 3, so that the result register r of
//                    lane l holds key 32*half + 16*(r>>3) + 8*gl + (r&7).
//   softmax          each lane holds 32 scores of its own query row; the row
//                    max is a local max plus one lane^32 exchange.  The
//                    probabilities are exp2(s*scale*log2e - m) with m a
//                    running row max that is only raised when the tile max
//                    exceeds it by more than kLazyLog2 (the accumulators are
//                    rescaled then); otherwise the tile reuses the stale m,
//                    which leaves numerator and denominator scaled alike and
//                    keeps P <= 2^kLazyLog2.  The DMA kernel first runs with
//                    m fixed at the tile-0 max (no max or rescale after tile
//                    0) and falls back to the running max for a workgroup
//                    whose row sums leave the range that proves it exact.
//   O^T += V^T . P^T B = P^T is then exactly the lane's own probabilities:
//                    16-key step j uses registers 8*(j&1) .. +7 of half j>>1.
//                    A = 32 dims x 16 keys of V^T from LDS.  Output rows are
//                    dims and columns query rows, so the rescale is
//                    lane-local.  Tile 0, where rows with few keys live,
//                    feeds P as bf16 hi + lo parts (two MFMAs) so that short
//                    rows keep rtol 1e-2 / atol 2e-3; later tiles feed the
//                    rounded P and sum the same rounded values into the
//                    denominator (v_dot2c_f32_bf16).
//
// Staging.  A KV tile is 4 blocks x head_dim/32 (block, 32-dim chunk) pairs of
// 1 KiB for K and for V; each wave loads whole pairs (64 lanes x 16 bytes,
// contiguous in the pool) into registers and writes them to LDS after the
// current tile's MFMAs.  LDS rows are padded by 16 bytes (K: [64 keys]
// [head_dim + 8], V^T: [head_dim][64 + 8 keys]) so that the 16 lanes of a
// ds_read_b128 phase cover all 64 banks; two buffers, one barrier per tile.
// The block-table entries of tile t+2 are loaded while tile t is computed
// (lane b < 4 holds block b of the tile) and broadcast with v_readlane, so the
// K/V load addresses of the next tile are scalar and ready.
//
// Roofline: bf16 MFMA.  Algorithmic FLOPs = sum over rows of (keys) * heads *
// 4 * head_dim (Q.K^T and P.V, causal-aware).
#include <cmath>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "vo_device.hpp"
#include "vo_kernels.hpp"

namespace vo {
namespace kernels {

namespace {

constexpr int kBS = 16;          // block size of the MFMA path
constexpr int kQT = 64;          // query rows per work item
constexpr int kRG = 32;          // query rows per wavefront
constexpr int kKT = 64;          // keys per KV tile (4 blocks)
constexpr float kLazyLog2 = 8.0f;  // growth of a row max (log2 units) absorbed without a rescale
// Row sum below which a fixed-offset pass provably kept every P and O in
// range (2^40; see prefill_dma_kernel).
constexpr float kOverflowSum = 1099511627776.0f;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ floatx16 mfma32x32x16(bf16x8 a, bf16x8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Swap bits 2 and 3: the A-row -> key order of the Q.K^T MFMA.
__device__ __forceinline__ uint32_t key_perm(uint32_t i) {
    return (i & ~0xCu) | ((i & 4u) << 1) | ((i & 8u) >> 1);
}

// Sum of the eight bf16 values of v, accumulated onto acc in fp32.
__device__ __forceinline__ float sum8(bf16x8 v, float acc) {
    const bf16x2 one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 0, 1), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 2, 3), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 4, 5), one, acc, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 6, 7), one, acc, false);
}

// True when every element of the DT accumulator blocks is finite: fma(x, 0,
// acc) keeps acc at exactly +0 for finite x and turns it into NaN for an
// infinite or NaN x.  (One VALU op per element; a chain of v_cmp_class
// lane masks ANDed on the scalar unit waits on every VALU result.)
template <int DT>
__device__ __forceinline__ bool all_finite(const floatx16 (&o)[DT]) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r & 3] = __builtin_fmaf(o[dt][r], 0.0f, acc[r & 3]);
    return (acc[0] + acc[1]) + (acc[2] + acc[3]) == 0.0f;
}

template <int HD, int W>
struct TileShape {
    static constexpr int KS = HD / 16;               // Q.K^T k-steps
    static constexpr int DT = HD / 32;               // P.V output tiles (32 dims)
    static constexpr int CH = HD / 32;               // 32-dim chunks of a block tile
    static constexpr int KSTR = HD * 2 + 16;         // bytes per K row in LDS
    static constexpr int VSTR = kKT * 2 + 16;        // bytes per V^T row in LDS
    static constexpr int KBYTES = kKT * KSTR;
    static constexpr int BUF = KBYTES + HD * VSTR;   // one K + V^T buffer
    static constexpr int PAIRS = (kKT / kBS) * CH;   // (block, chunk) pairs per tile
    static constexpr int UPT = PAIRS / W;            // pairs per wave per tile
    static_assert(PAIRS % W == 0, "pairs must divide over the waves");

    // Pair i of wave w: block b of the tile and 32-dim chunk ch, both
    // wave-uniform; the waves of one step cover distinct pairs.
    __device__ static __forceinline__ void pair(uint32_t w, int i, uint32_t &b, uint32_t &ch) {
        if constexpr (W >= CH) {
            b = w / CH + (W / CH) * i;
            ch = w % CH;
        } else {
            b = i / (CH / W);
            ch = w + W * (i % (CH / W));
        }
    }
};

template <int HD, int G, int R>
__global__ __launch_bounds__(64 * G * R) __attribute__((amdgpu_waves_per_eu(2))) void prefill_mfma_kernel(
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool, uint32_t kv_heads,
    const uint32_t *__restrict__ table_off, const uint32_t *__restrict__ tables,
    const uint32_t *__restrict__ work, const uint16_t *__restrict__ q,
    uint16_t *__restrict__ out, uint32_t num_heads, float scale_log2) {
    constexpr int HALVES = kQT / (kRG * R);  // workgroups per (item, KV head)
    using S = TileShape<HD, G * R>;
    constexpr int KS = S::KS;
    constexpr int DT = S::DT;
    constexpr int UPT = S::UPT;
    constexpr uint32_t kTile = kBS * HD;  // elements per (block, kv head) tile

    __shared__ __align__(16) uint8_t lds[2 * S::BUF];

    const uint32_t kvh = blockIdx.x % kv_heads;
    const uint32_t rest = blockIdx.x / kv_heads;
    const uint32_t item = rest / HALVES;
    const uint32_t wg_row0 = (rest % HALVES) * (kRG * R);  // first item row of the workgroup
    const uint32_t item_rows = work[4 * item + 1];
    if (wg_row0 >= item_rows) return;  // whole workgroup, before any barrier
    const uint32_t row_begin = work[4 * item] + wg_row0;
    const uint32_t nrows = min(item_rows - wg_row0, static_cast<uint32_t>(kRG * R));
    const uint32_t p_min = work[4 * item + 2] + wg_row0;
    const uint32_t seq = work[4 * item + 3];
    const uint32_t p_max = p_min + nrows - 1;
    const uint32_t n_tiles = p_max / kKT + 1;
    const uint32_t nblk = p_max / kBS + 1;
    const uint32_t *table = tables + table_off[seq];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t head = wave % G;  // query head of the wave within the group
    const uint32_t rg = wave / G;    // row group of the wave
    const uint32_t c = lane & 31;    // query row of this lane within the row group
    const uint32_t gl = lane >> 5;
    const uint32_t qhead = kvh * G + head;
    const uint32_t lr = kRG * rg + c;  // row within the workgroup
    const bool row_ok = lr < nrows;
    const uint32_t p_row = p_min + lr;
    // Positions of the wave's first and last rows (wave-uniform).
    const uint32_t wp_min = p_min + kRG * rg;
    const uint32_t wp_max = min(wp_min + kRG - 1, p_max);

    // Q^T operand, k-step kk: dims 16*kk + 8*gl .. +7 of row lr.
    bf16x8 qv[KS];
    {
        const uint16_t *qp =
            q + (static_cast<uint64_t>(row_begin + lr) * num_heads + qhead) * HD + 8 * gl;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
            qv[kk] = row_ok ? __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(qp + 16 * kk))
                            : bf16x8{};
    }

    // Lane b < 4 of the result holds the physical block of slot b of tile t.
    auto load_table = [&](uint32_t t) -> uint32_t { return table[min(4 * t + (lane & 3), nblk - 1)]; };

    // Global -> register staging of one KV tile.  K pair: lane = (key
    // lane&15, 8-dim quarter lane>>4); V pair: lane = (dim lane&31, 8-key half
    // lane>>5); both read 1 KiB that is contiguous in the pool.
    const uint32_t k_lane = (lane & 15) * 32 + (lane >> 4) * 8;
    const uint32_t v_lane = (lane & 31) * kBS + (lane >> 5) * 8;
    u32x4 kreg[UPT], vreg[UPT];
    auto gload = [&](uint32_t tbv) {
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
            uint32_t b, ch;
            S::pair(wave, i, b, ch);
            const uint32_t blk = __builtin_amdgcn_readlane(tbv, b);
            const uint64_t base = (static_cast<uint64_t>(blk) * kv_heads + kvh) * kTile + ch * (kBS * 32);
            kreg[i] = *reinterpret_cast<const u32x4 *>(k_pool + base + k_lane);
            vreg[i] = *reinterpret_cast<const u32x4 *>(v_pool + base + v_lane);
        }
    };
    // Register -> LDS: K row 16b + key at byte 64*ch + 16*quarter; V^T row
    // 32*ch + dim at byte 32*b + 16*half.
    const uint32_t k_st = (lane & 15) * S::KSTR + (lane >> 4) * 16;
    const uint32_t v_st = S::KBYTES + (lane & 31) * S::VSTR + (lane >> 5) * 16;
    auto lstore = [&](uint8_t *base) {
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
            uint32_t b, ch;
            S::pair(wave, i, b, ch);
            *reinterpret_cast<u32x4 *>(base + k_st + (kBS * b) * S::KSTR + 64 * ch) = kreg[i];
            *reinterpret_cast<u32x4 *>(base + v_st + (32 * ch) * S::VSTR + 32 * b) = vreg[i];
        }
    };

    float m_run = 0.0f;  // set by tile 0
    float l_run = 0.0f;
    floatx16 o_acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o_acc[dt] = floatx16{};

    // Per-lane LDS read offsets: K A-row c reads key key_perm(c) (+32),
    // 16-byte unit 2*kk + gl; V^T A-row c reads dim 32*dt + c, unit 2*j + gl.
    const uint32_t k_rd = key_perm(c) * S::KSTR + gl * 16;
    const uint32_t v_rd = S::KBYTES + c * S::VSTR + gl * 16;

    auto step = [&](auto buf_c, auto first_c, uint32_t t, uint32_t &tbv) {
        constexpr int buf = decltype(buf_c)::value;
        constexpr bool first = decltype(first_c)::value;
        const bool more = t + 1 < n_tiles;
        if (more) {
            gload(tbv);
            tbv = load_table(t + 2);
        }
        const uint8_t *tile = lds + buf * S::BUF;
        const uint32_t j0 = t * kKT;
        // A row group that ends before this tile (the workgroup's other row
        // group reaches further) has nothing to add.
        if (wp_min >= nrows + p_min || j0 > wp_max) goto staged;
        {
        // S^T = K . Q^T for the two 32-key halves.
        floatx16 s0 = {}, s1 = {};
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            const bf16x8 a0 = *reinterpret_cast<const bf16x8 *>(tile + k_rd + 32 * kk);
            const bf16x8 a1 = *reinterpret_cast<const bf16x8 *>(tile + k_rd + 32 * S::KSTR + 32 * kk);
            s0 = mfma32x32x16(a0, qv[kk], s0);
            s1 = mfma32x32x16(a1, qv[kk], s1);
        }

        float sc[32];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            sc[r] = s0[r];
            sc[16 + r] = s1[r];
        }
        if (j0 + kKT - 1 > wp_min) {
            // Diagonal tile: key j is visible to this row iff j <= p_row.
#pragma unroll
            for (int r = 0; r < 32; ++r) {
                const uint32_t key = j0 + 32 * (r >> 4) + 16 * ((r >> 3) & 1) + 8 * gl + (r & 7);
                sc[r] = (key <= p_row) ? sc[r] : -INFINITY;
            }
        }
        float mx = sc[0];
#pragma unroll
        for (int r = 1; r < 32; ++r) mx = fmaxf(mx, sc[r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mt = mx * scale_log2;  // finite: tile 0 holds key 0 for every row
        if constexpr (first) {
            m_run = mt;
        } else if (__builtin_amdgcn_ballot_w64(mt > m_run + kLazyLog2) != 0) {
            const float m_new = fmaxf(m_run, mt);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o_acc[dt] *= alpha;
            m_run = m_new;
        }
        const float nm = -m_run;
#pragma unroll
        for (int r = 0; r < 32; ++r) sc[r] = __builtin_amdgcn_exp2f(fmaf(sc[r], scale_log2, nm));

        // O^T += V^T . P^T over four 16-key steps.
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bf16x8 pb_hi, pb_lo;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float p = sc[16 * (j >> 1) + 8 * (j & 1) + i];
                const __bf16 hi = static_cast<__bf16>(p);
                pb_hi[i] = hi;
                if constexpr (first) {
                    pb_lo[i] = static_cast<__bf16>(p - static_cast<float>(hi));
                    l_run += p;
                }
            }
            if constexpr (!first) l_run = sum8(pb_hi, l_run);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const bf16x8 a = *reinterpret_cast<const bf16x8 *>(tile + v_rd + 32 * dt * S::VSTR + 32 * j);
                if constexpr (first) o_acc[dt] = mfma32x32x16(a, pb_lo, o_acc[dt]);
                o_acc[dt] = mfma32x32x16(a, pb_hi, o_acc[dt]);
            }
        }

        }
    staged:
        if (more) lstore(lds + (buf ^ 1) * S::BUF);
        __syncthreads();
    };

    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using First = std::integral_constant<bool, true>;
    using Rest = std::integral_constant<bool, false>;

    uint32_t tbv = load_table(0);
    gload(tbv);
    tbv = load_table(1);
    lstore(lds);
    __syncthreads();
    step(B0{}, First{}, 0, tbv);
    for (uint32_t t = 1; t < n_tiles; t += 2) {
        step(B1{}, Rest{}, t, tbv);
        if (t + 1 >= n_tiles) break;
        step(B0{}, Rest{}, t + 1, tbv);
    }

    l_run += __shfl_xor(l_run, 32, 64);
    if (!row_ok) return;
    const float inv = 1.0f / l_run;
    uint16_t *op = out + (static_cast<uint64_t>(row_begin + lr) * num_heads + qhead) * HD + 4 * gl;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            u32x2 packed;
            packed[0] = f32_to_bf16_bits(o_acc[dt][4 * r4] * inv) |
                        (static_cast<uint32_t>(f32_to_bf16_bits(o_acc[dt][4 * r4 + 1] * inv)) << 16);
            packed[1] = f32_to_bf16_bits(o_acc[dt][4 * r4 + 2] * inv) |
                        (static_cast<uint32_t>(f32_to_bf16_bits(o_acc[dt][4 * r4 + 3] * inv)) << 16);
            *reinterpret_cast<u32x2 *>(op + 32 * dt + 8 * r4) = packed;
        }
    }
}

// ---------------------------------------------------------------------------
// The same kernel with the KV tiles staged by LDS DMA (gfx950
// buffer_load_dwordx4 ... lds: each lane's 16 bytes go from its own global
// address straight into LDS at base + 16 * lane) through a ring of three LDS
// stages, so the tile two ahead is in flight while this one is computed and
// no registers or ds_write instructions carry the staging.
//
// A stage keeps the pool's own tile layout, block after block: K as
// [4 blocks][head_dim/32][16 keys][32 dims] and V as [4 blocks][head_dim]
// [16 keys], so every DMA instruction copies 1 KiB of one (block, KV head)
// tile.  A DMA instruction cannot pad, so bank conflicts are avoided by a
// permutation of the 16-byte units inside each 256-byte line, chosen per
// lane on the global side: the unit U of a block tile is stored at
//   K: U ^ ((U >> 4) & 3)        V: U ^ ((U >> 4) & 1).
// A ds_read_b128 phase (16 lanes) of the Q.K^T A operand reads 16 keys of
// one block at one (chunk, 8-dim unit): U = 64 ch + 4 key + s, which the K
// map spreads over all 16 units of a line; the P.V A operand reads 16 dims
// at one 8-key half: U = 2 dim + half, which the V map spreads likewise.
// Both maps leave the per-lane read address independent of the MFMA step,
// so the steps are immediate offsets.
//
// The block table of the item's sequence is copied to LDS first, so the
// per-tile block ids are LDS reads: no global load joins the DMA
// instructions in the vector-memory counter.  Stage s of tile t is read
// after an explicit s_waitcnt that leaves only the wave's newest DMA
// instructions (tile t + 1's) outstanding, then a barrier; compiler-only
// fences keep LDS reads on their side of it.
constexpr uint32_t kTableLds = 4096;  // block-table entries the DMA kernel stages

template <int HD, int W>
struct DmaShape {
    static constexpr int BT = HD * kBS * 2;       // bytes of one (block, KV head) tile
    static constexpr int IPB = BT / 1024;         // DMA instructions per block tile
    static constexpr int KBYTES = 4 * BT;
    static constexpr int STAGE = 2 * KBYTES;      // K then V
    static constexpr int NK = 4 * IPB;            // K DMA instructions per KV tile
    static constexpr int DPW = 2 * NK / W;        // per wave: DPW/2 for K, DPW/2 for V
    static_assert((2 * NK) % W == 0 && DPW % 2 == 0 && DPW <= 15, "DMA split");
};

// Occupancy target: two wavefronts per SIMD, except at head_dim 128 with 4
// wavefronts per workgroup, where the 112 KiB of LDS leaves one workgroup per
// CU and so one wavefront per SIMD.
template <int HD, int G, int R>
__global__ __launch_bounds__(64 * G * R) __attribute__((amdgpu_waves_per_eu(
    (HD == 128 && G * R == 4) ? 1 : 2))) void prefill_dma_kernel(
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool, uint32_t kv_heads,
    const uint32_t *__restrict__ table_off, const uint32_t *__restrict__ tables,
    const uint32_t *__restrict__ work, const uint16_t *__restrict__ q,
    uint16_t *__restrict__ out, uint32_t num_heads, float scale_log2, uint32_t fixed_offset,
    uint32_t pool_bytes) {
    constexpr int W = G * R;
    constexpr int HALVES = kQT / (kRG * R);
    using D = DmaShape<HD, W>;
    constexpr int KS = HD / 16;
    constexpr int DT = HD / 32;
    constexpr int DPW = D::DPW;
    constexpr uint32_t kTile = kBS * HD;

    __shared__ uint32_t tbl[kTableLds];
    __shared__ __align__(1024) uint8_t st0[D::STAGE];
    __shared__ __align__(1024) uint8_t st1[D::STAGE];
    __shared__ __align__(1024) uint8_t st2[D::STAGE];
    __shared__ uint32_t redo;  // bit g: a row of row group g left the fixed-offset range

    const uint32_t kvh = blockIdx.x % kv_heads;
    const uint32_t rest = blockIdx.x / kv_heads;
    const uint32_t item = rest / HALVES;
    const uint32_t wg_row0 = (rest % HALVES) * (kRG * R);
    const uint32_t item_rows = work[4 * item + 1];
    if (wg_row0 >= item_rows) return;  // whole workgroup, before any barrier
    const uint32_t row_begin = work[4 * item] + wg_row0;
    const uint32_t nrows = min(item_rows - wg_row0, static_cast<uint32_t>(kRG * R));
    const uint32_t p_min = work[4 * item + 2] + wg_row0;
    const uint32_t seq = work[4 * item + 3];
    const uint32_t p_max = p_min + nrows - 1;
    const uint32_t n_tiles = p_max / kKT + 1;
    const uint32_t nblk = p_max / kBS + 1;  // <= kTableLds (longer items run on the register kernel)
    const uint32_t *table = tables + table_off[seq];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t head = wave % G;
    const uint32_t rg = wave / G;
    const uint32_t c = lane & 31;
    const uint32_t gl = lane >> 5;
    const uint32_t qhead = kvh * G + head;
    const uint32_t lr = kRG * rg + c;
    const bool row_ok = lr < nrows;
    const uint32_t p_row = p_min + lr;
    const uint32_t wp_min = p_min + kRG * rg;
    const uint32_t wp_max = min(wp_min + kRG - 1, p_max);

    for (uint32_t i = tid; i < nblk; i += 64 * W) tbl[i] = table[i];
    if (tid == 0) redo = 0u;

    bf16x8 qv[KS];
    {
        const uint16_t *qp =
            q + (static_cast<uint64_t>(row_begin + lr) * num_heads + qhead) * HD + 8 * gl;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
            qv[kk] = row_ok ? __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(qp + 16 * kk))
                            : bf16x8{};
    }
    wait_barrier<0>();  // the table copy

    // DMA sources: wave instruction i is K instruction i * W + wave for
    // i < DPW/2, V instruction (i - DPW/2) * W + wave after; instruction qi
    // copies 1 KiB number qi % IPB of block qi / IPB.  Lane L writes physical
    // unit P = 64 (qi % IPB) + L of the block tile and reads logical unit U.
    uint32_t dma_off[DPW];
#pragma unroll
    for (int i = 0; i < DPW; ++i) {
        const uint32_t qi = (i % (DPW / 2)) * W + wave;
        const uint32_t P = 64 * (qi % D::IPB) + lane;
        const uint32_t U = i < DPW / 2 ? P ^ ((P >> 4) & 3u) : P ^ ((P >> 4) & 1u);
        dma_off[i] = U * 16;
    }
    // K instruction i and V instruction i + NB copy from the same block, so
    // a wave touches NB blocks of each tile: slot s is block (s W + wave) / IPB
    // of the tile.  One buffer resource per pool spans the layer from KV head
    // kvh's first tile on; a block's byte offset goes in the instruction's
    // scalar offset, so a DMA costs one s_mov to m0 besides the load.
    constexpr int NB = DPW / 2;
    const auto k_rsrc = buffer_rsrc(k_pool + kvh * kTile, pool_bytes - kvh * D::BT);
    const auto v_rsrc = buffer_rsrc(v_pool + kvh * kTile, pool_bytes - kvh * D::BT);
    const uint32_t blk_stride = kv_heads * D::BT;  // bytes from a block to the next
    auto dma_tile = [&](uint8_t *stage, const uint32_t (&boff)[NB]) {
#pragma unroll
        for (int i = 0; i < DPW; ++i) {
            const bool is_k = i < NB;
            const uint32_t qi = (i % NB) * W + wave;
            dma16_at(is_k ? k_rsrc : v_rsrc, stage + (is_k ? 0 : D::KBYTES) + qi * 1024, dma_off[i],
                     boff[i % NB]);
        }
    };
    // Byte offsets of tile t's blocks in this wave's slots.
    auto blk_offs = [&](uint32_t t, uint32_t (&boff)[NB]) {
#pragma unroll
        for (int s = 0; s < NB; ++s) {
            const uint32_t slot = (static_cast<uint32_t>(s) * W + wave) / D::IPB;
            boff[s] = uniform_u32(tbl[min(4 * t + slot, nblk - 1)]) * blk_stride;
        }
    };

    float m_run = 0.0f;
    float l_run = 0.0f;  // the f32 sum of the lane's p, then (after the pass) the row's
    floatx16 o_acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o_acc[dt] = floatx16{};

    // LDS read offsets.  K: A-row c reads key kp = key_perm(c) of block kp/16
    // (+2 blocks for the second 32-key half), chunk kk/2, unit 2(kk%2) + gl,
    // stored at unit ^ ((kp % 16) >> 2).  V: A-row c reads dim 32 dt + c of
    // block j, half gl, stored at half ^ ((c >> 3) & 1).
    const uint32_t kp = key_perm(c);
    const uint32_t kx = ((kp & 15) >> 2) & 3;
    const uint32_t k_rd0 = (kp / 16) * D::BT + (kp & 15) * 64 + 16 * (gl ^ kx);
    const uint32_t k_rd1 = (kp / 16) * D::BT + (kp & 15) * 64 + 16 * ((gl ^ kx) ^ 2);
    const uint32_t v_rd = D::KBYTES + c * 32 + 16 * (gl ^ ((c >> 3) & 1));

    uint32_t nxt[NB];  // block offsets of tile t + 2 while step t runs
    // A wave that is not live in the second pass issues its share of the DMA
    // and meets every barrier, but computes nothing and keeps its state.
    bool live = true;
    // The stage read and the stage filled are passed as restrict pointers, so
    // the compiler knows this step's DMA does not write what it reads (it
    // then inserts no wait for that DMA before the reads).
    auto body = [&](auto fixed_c, auto first_c, uint32_t t, const uint8_t *__restrict__ tile,
                    uint8_t *__restrict__ ahead) __attribute__((always_inline)) {
        constexpr bool fixed = decltype(fixed_c)::value;
        constexpr bool first = decltype(first_c)::value;
        // Every step issues its DMA, past the last tile too (block ids clamp
        // to the table's last entry), so that every step has the same number
        // of DMA instructions in flight and the compiler's wait tracking
        // stays exact through the loop.
        dma_tile(ahead, nxt);
        blk_offs(t + 3, nxt);
        const uint32_t j0 = t * kKT;
        if ((!fixed && !live) || wp_min >= nrows + p_min || j0 > wp_max) goto staged;
        {
        // K fragments are read four k-steps ahead of their MFMAs (the
        // scheduling fence keeps the first four reads ahead of every MFMA),
        // and the tile's V fragments are all read right after the Q.K^T
        // MFMAs, so they land while the exps run.
        constexpr int KA = KS < 4 ? KS : 4;
        floatx16 s0 = {}, s1 = {};
        bf16x8 ka[KS], kb[KS];
        auto read_k = [&](int kk) __attribute__((always_inline)) {
            const uint32_t off = (kk / 2) * (kBS * 64) + ((kk & 1) ? k_rd1 : k_rd0);
            ka[kk] = *reinterpret_cast<const bf16x8 *>(tile + off);
            kb[kk] = *reinterpret_cast<const bf16x8 *>(tile + off + 2 * D::BT);
        };
#pragma unroll
        for (int kk = 0; kk < KA; ++kk) read_k(kk);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            if (kk + KA < KS) read_k(kk + KA);
            s0 = mfma32x32x16(ka[kk], qv[kk], s0);
            s1 = mfma32x32x16(kb[kk], qv[kk], s1);
        }
        bf16x8 vf[4][DT];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                vf[j][dt] = *reinterpret_cast<const bf16x8 *>(tile + v_rd + j * D::BT + dt * 1024);

        float sc[32];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            sc[r] = s0[r];
            sc[16 + r] = s1[r];
        }
        if (j0 + kKT - 1 > wp_min) {
#pragma unroll
            for (int r = 0; r < 32; ++r) {
                const uint32_t key = j0 + 32 * (r >> 4) + 16 * ((r >> 3) & 1) + 8 * gl + (r & 7);
                sc[r] = (key <= p_row) ? sc[r] : -INFINITY;
            }
        }
        // Row max of the tile, in the exp2 domain (both lanes of the row).
        auto tile_max = [&]() __attribute__((always_inline)) {
            float mx = sc[0];
#pragma unroll
            for (int r = 1; r < 32; ++r) mx = fmaxf(mx, sc[r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            return mx * scale_log2;
        };
        if constexpr (first) {
            m_run = tile_max();  // finite: every row sees key 0
        } else if constexpr (!fixed) {
            const float mt = tile_max();
            if (__builtin_amdgcn_ballot_w64(mt > m_run + kLazyLog2) != 0) {
                const float m_new = fmaxf(m_run, mt);
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o_acc[dt] *= alpha;
                m_run = m_new;
            }
        }
        const float nm = -m_run;
#pragma unroll
        for (int r = 0; r < 32; ++r) sc[r] = __builtin_amdgcn_exp2f(fmaf(sc[r], scale_log2, nm));

#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bf16x8 pb_hi, pb_lo;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float p = sc[16 * (j >> 1) + 8 * (j & 1) + i];
                const __bf16 hi = static_cast<__bf16>(p);
                pb_hi[i] = hi;
                if constexpr (first) pb_lo[i] = static_cast<__bf16>(p - static_cast<float>(hi));
                l_run += p;
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                if constexpr (first) o_acc[dt] = mfma32x32x16(vf[j][dt], pb_lo, o_acc[dt]);
                o_acc[dt] = mfma32x32x16(vf[j][dt], pb_hi, o_acc[dt]);
            }
        }
        }
    staged:
        // Tile t + 1 must have landed; tile t + 2 (this step's DMA) may fly on.
        wait_barrier<DPW>();
    };
    auto step = [&](auto fixed_c, auto buf_c, auto first_c, uint32_t t) {
        constexpr int buf = decltype(buf_c)::value;
        if constexpr (buf == 0) body(fixed_c, first_c, t, st0, st2);
        else if constexpr (buf == 1) body(fixed_c, first_c, t, st1, st0);
        else body(fixed_c, first_c, t, st2, st1);
    };

    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using B2 = std::integral_constant<int, 2>;
    using First = std::integral_constant<bool, true>;
    using Rest = std::integral_constant<bool, false>;

    // One pass over the item's KV tiles; a live wave's m_run, l_run and
    // o_acc start afresh.
    auto pass = [&](auto fixed_c) __attribute__((always_inline)) {
        constexpr bool fixed = decltype(fixed_c)::value;  // the first pass: every wave live
        if (fixed || live) {
            m_run = 0.0f;
            l_run = 0.0f;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o_acc[dt] = floatx16{};
        }
        blk_offs(0, nxt);
        dma_tile(st0, nxt);
        blk_offs(1, nxt);
        dma_tile(st1, nxt);
        blk_offs(2, nxt);
        wait_barrier<DPW>();
        step(fixed_c, B0{}, First{}, 0);
        for (uint32_t t = 1; t < n_tiles; t += 3) {
            step(fixed_c, B1{}, Rest{}, t);
            if (t + 1 >= n_tiles) break;
            step(fixed_c, B2{}, Rest{}, t + 1);
            if (t + 2 >= n_tiles) break;
            step(fixed_c, B0{}, Rest{}, t + 2);
        }
        // The DMA of the tiles past the end is still in flight: it must land
        // before the stages are refilled or the workgroup's LDS is released.
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
        if (fixed || live) l_run += __shfl_xor(l_run, 32, 64);
    };

    // Fixed softmax offset: m_run stays at the row's tile-0 max.  A later
    // score above it gives P = 2^(s c - m) > 1, which bf16 and the f32 sums
    // hold with the same relative precision, and O / l does not depend on
    // the offset; so later tiles need neither a row max nor a rescale.  Only
    // the range can fail: every P is a term of l, and |O| <= l max |V|, so a
    // row with l below kOverflowSum and a finite O lost nothing.  If a row of
    // a 32-row group is past that, the group's rows are recomputed with the
    // running max (raised by more than kLazyLog2 at a time, per wave) in a
    // second pass, in which the waves of the other groups stay idle and keep
    // their first-pass results.  The decision is per row group, never per
    // workgroup, so a row's result does not depend on whether its group
    // shares a workgroup with the item's other group (which a plan of few
    // items avoids): the same rows give the same bits in any batch.
    if (fixed_offset) {
        pass(std::true_type{});
        const bool ok = l_run < kOverflowSum && all_finite(o_acc);  // false for inf and NaN too
        if (__builtin_amdgcn_ballot_w64(row_ok && !ok) != 0 && lane == 0) atomicOr(&redo, 1u << rg);
    } else if (tid == 0) {
        redo = (1u << R) - 1;
    }
    wait_barrier<0>();
    const uint32_t again = uniform_u32(redo);
    if (again != 0) {
        live = ((again >> rg) & 1u) != 0;
        pass(std::false_type{});
    }
    // Every wave's DMA has landed and its stage reads are done: the stages
    // can hold the output.
    wait_barrier<0>();

    // The output goes out through LDS.  A wave's MFMA results put 8 dims of
    // one row in a lane pair, so direct stores would write 16-byte pieces of
    // 32 rows per instruction; the workgroup's rows hold its G heads side by
    // side in memory (G * HD * 2 contiguous bytes per row), so staged in LDS
    // each store instruction writes whole rows.  Wave w's 32 x HD tile sits
    // in stage w / WPS, 16-byte chunk q of row c at chunk q ^ (c % CH) (no
    // bank conflicts on the writes).
    constexpr int ROWB = HD * 2;         // bytes of one (row, head)
    constexpr int CH = HD / 8;           // 16-byte chunks of one (row, head)
    constexpr int WTILE = kRG * ROWB;    // one wave's output tile
    constexpr int WPS = D::STAGE / WTILE;
    static_assert(W <= 2 * WPS, "the output tiles fit two stages");
    {
        const float inv = 1.0f / l_run;
        uint8_t *tile = (wave < WPS ? st0 : st1) + (wave % WPS) * WTILE + c * ROWB + 8 * gl;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                u32x2 packed;
                packed[0] = f32_to_bf16_bits(o_acc[dt][4 * r4] * inv) |
                            (static_cast<uint32_t>(f32_to_bf16_bits(o_acc[dt][4 * r4 + 1] * inv)) << 16);
                packed[1] = f32_to_bf16_bits(o_acc[dt][4 * r4 + 2] * inv) |
                            (static_cast<uint32_t>(f32_to_bf16_bits(o_acc[dt][4 * r4 + 3] * inv)) << 16);
                const uint32_t q4 = static_cast<uint32_t>(4 * dt + r4) ^ (c % CH);
                *reinterpret_cast<u32x2 *>(tile + 16 * q4) = packed;
            }
        }
    }
    wait_barrier<0>();
    constexpr uint32_t kRowChunks = G * CH;  // 16-byte chunks of a row's G heads
    uint16_t *obase = out + (static_cast<uint64_t>(row_begin) * num_heads + kvh * G) * HD;
    for (uint32_t k = tid; k < nrows * kRowChunks; k += 64 * W) {
        const uint32_t row = k / kRowChunks;
        const uint32_t h = (k % kRowChunks) / CH;
        const uint32_t q4 = k % CH;
        const uint32_t w = h + G * (row / kRG);
        const uint32_t cr = row % kRG;
        const u32x4 v = *reinterpret_cast<const u32x4 *>((w < WPS ? st0 : st1) + (w % WPS) * WTILE +
                                                         cr * ROWB + 16 * (q4 ^ (cr % CH)));
        *reinterpret_cast<u32x4 *>(obase + static_cast<uint64_t>(row) * num_heads * HD + h * HD +
                                   8 * q4) = v;
    }
}

// ---------------------------------------------------------------------------
// Head_dim 128 with GQA 4 (the Llama-3-8B shape): the same work item (64
// query rows x the 4 query heads of KV head k) served by 4 wavefronts, one
// per query head and one per SIMD, each holding both 32-row groups.  Every
// K or V fragment read from LDS then feeds two MFMAs (half the LDS reads per
// MFMA of the 8-wavefront kernel), and the steady-state KV tiles run a
// software pipeline written as one inline-asm loop (prefill_pipe_loop.inc,
// generated by gen_prefill_pipe.py): iteration t issues the Q.K^T MFMAs of
// tile t + 1 between the softmax instructions of tile t, then tile t's P.V.
// On gfx950 VALU instructions co-issue with a running 32-cycle MFMA, so the
// softmax no longer takes turns with the MFMAs.
//
// Four LDS stages (the tile in P.V, the tile in Q.K^T, and two in flight):
// the DMA of tile t + 3 is issued at iteration t, after a barrier that
// follows the wait for tile t + 1.  The generated code also runs tile 0
// (whose max becomes the fixed softmax offset and whose P goes in as bf16
// hi + lo) and the causal masks; the overflow check, the running-max
// recompute and the output run as ordinary code between items.  Per row the
// arithmetic is the 32-row kernels' operation for operation (same MFMAs in
// the same order from the same LDS bytes, same VALU operations), so a row
// gets the same bits here as in prefill_dma_kernel<128, 4, 1>, which serves
// the same items on small grids.  The kernel is persistent (below): one
// workgroup per CU runs a slot's items through one LDS ring.
#include "prefill_pipe_loop.inc"

// The four words of a raw buffer resource, for an inline-asm operand.
__device__ __forceinline__ u32x4 rsrc_words(const void *base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return u32x4{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xffffu, bytes,
                 kBufferRsrcWord3};
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t *)p));
}

constexpr int kPipeStage = 32768;  // one stage: K (16 KiB) then V (16 KiB)
constexpr int kPipeBT = 4096;      // one (block, KV head) tile at head_dim 128

// One work item of prefill_pipe_kernel, from its descriptor (first row, rows,
// position of the first row, offset of the sequence's block table).
struct PipeItem {
    uint32_t row_begin, nrows, p_min, n_tiles, nblk;
    const uint32_t *table;
};

__device__ __forceinline__ PipeItem pipe_item(const uint32_t *desc, const uint32_t *tables) {
    PipeItem it;
    it.row_begin = desc[0];
    it.nrows = desc[1];
    it.p_min = desc[2];
    it.table = tables + desc[3];
    const uint32_t p_max = it.p_min + it.nrows - 1;
    it.n_tiles = p_max / kKT + 1;
    it.nblk = p_max / kBS + 1;  // <= kTableLds
    return it;
}

// Persistent: workgroup w serves KV head w % kv_heads and runs the items of
// slot w / kv_heads (plan[slot] .. plan[slot + 1] - 1 of the descriptors at
// plan + num_slots + 1) back to back.  The four LDS stages form one ring
// across the items: item k's tile t sits in stage (T_k + t) % 4 with
// T_k+1 = T_k + n_k, and the block table in LDS continues past an item's
// last tile with the next item's first twelve block ids, so the DMAs the
// loop issues past the end (tiles n .. n + 2) fetch the next item's tiles
// 0-2 while this one finishes.  Its Q and block table load while this
// item's output is written.  Each wave writes its own head's rows through
// the one stage that holds no prefetched tile.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void prefill_pipe_kernel(
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool, uint32_t kv_heads,
    const uint32_t *__restrict__ tables, const uint32_t *__restrict__ plan, uint32_t num_slots,
    const uint16_t *__restrict__ q, uint16_t *__restrict__ out, uint32_t num_heads, float scale_log2,
    uint32_t fixed_offset, uint32_t pool_bytes) {
    constexpr int HD = 128, G = 4, KS = 8, DT = 4;
    constexpr uint32_t kTile = kBS * HD;

    // The table gets 16 entries past an item's last tile: the next item's
    // first twelve block ids (or copies of the last one), since the DMA runs
    // up to three tiles past the last one and the loop reads the ids of the
    // tile after that.
    __shared__ __align__(16) uint32_t tbl[kTableLds + 16];
    __shared__ __align__(1024) uint8_t st[4 * kPipeStage];
    // Overflow flags, alternating between consecutive items: item k sets
    // redo[k % 2]; redo[(k + 1) % 2] is cleared after item k's first
    // barrier, when every wave has read it for item k - 1.
    __shared__ uint32_t redo[2];

    const uint32_t kvh = blockIdx.x % kv_heads;
    const uint32_t slot = blockIdx.x / kv_heads;
    // The slot's first record (its first item's descriptor, that item's
    // tiles 0-2 block ids, the next item's first twelve) sits at an address
    // that depends only on the slot, so the first DMAs, Q loads and table
    // copy wait for one load.
    const uint32_t *first = plan + num_slots + 1 + kPipeFirstWords * slot;
    const uint32_t *descs = plan + num_slots + 1 + kPipeFirstWords * num_slots;
    uint32_t i = plan[slot];
    const uint32_t i_end = plan[slot + 1];
    if (i >= i_end) return;  // the host plan gives every slot an item

    const uint32_t head = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t qhead = kvh * G + head;

    // Per-lane values.  They are rebuilt after the pipelined loop from a
    // copy of the thread id that the compiler cannot see through, so that
    // of all of them only that id stays live across the loop's asm (which
    // leaves 63 VGPRs to the compiler).
    struct Lane {
        uint32_t tid, lane, c, gl, dma_k, dma_v, k_rd0, k_rd1, v_rd;
    };
    auto make_lane = [&](uint32_t t) __attribute__((always_inline)) {
        Lane L;
        L.tid = t;
        L.lane = t & 63;
        L.c = L.lane & 31;
        L.gl = L.lane >> 5;
        // DMA: the wave copies 1 KiB (part `head` of 4) of each of the
        // tile's four blocks, K then V; lane L reads logical unit U of
        // physical unit P = 64 head + L, as prefill_dma_kernel's stage
        // layout has it.
        const uint32_t dma_unit = 64 * head + L.lane;
        L.dma_k = (dma_unit ^ ((dma_unit >> 4) & 3u)) * 16;
        L.dma_v = (dma_unit ^ ((dma_unit >> 4) & 1u)) * 16;
        // LDS read offsets within a stage (prefill_dma_kernel's): K A-row c
        // reads key key_perm(c); V A-row c reads dim 32 dt + c.
        const uint32_t kp = key_perm(L.c);
        const uint32_t kx = ((kp & 15) >> 2) & 3;
        L.k_rd0 = (kp / 16) * kPipeBT + (kp & 15) * 64 + 16 * (L.gl ^ kx);
        L.k_rd1 = (kp / 16) * kPipeBT + (kp & 15) * 64 + 16 * ((L.gl ^ kx) ^ 2);
        L.v_rd = 4 * kPipeBT + L.c * 32 + 16 * (L.gl ^ ((L.c >> 3) & 1));
        return L;
    };
    Lane ln = make_lane(threadIdx.x);
    const u32x4 krs = rsrc_words(k_pool + kvh * kTile, pool_bytes - kvh * kPipeBT);
    const u32x4 vrs = rsrc_words(v_pool + kvh * kTile, pool_bytes - kvh * kPipeBT);
    const uint32_t stride = kv_heads * kPipeBT;
    const uint32_t st0 = lds_addr(st);
    const uint32_t wbase = st0 + 1024 * head;

    // The current item, the next (its first block ids go into the current
    // item's table) and the one after (loaded a hand-over ahead of its use).
    PipeItem A = pipe_item(first, tables);
    bool has_b = i + 1 < i_end;
    PipeItem B = pipe_item(descs + 4 * (has_b ? i + 1 : i), tables);
    bool has_c = i + 2 < i_end;
    PipeItem C = pipe_item(descs + 4 * (has_c ? i + 2 : i), tables);
    uint32_t T = 0;  // stage of the current item's tile 0

    // LDS DMA of a tile with block byte offsets b into `stage`.
    auto dma_raw = [&](uint32_t stage, const uint32_t (&b)[4]) __attribute__((always_inline)) {
        const uint32_t w = uniform_u32(wbase + stage * kPipeStage);
        asm volatile(
            "s_mov_b32 m0, %[w]\n s_nop 0\n buffer_load_dwordx4 %[dk], %[krs], %[b0] offen lds\n"
            "s_add_u32 m0, %[w], 4096\n s_nop 0\n buffer_load_dwordx4 %[dk], %[krs], %[b1] offen lds\n"
            "s_add_u32 m0, %[w], 8192\n s_nop 0\n buffer_load_dwordx4 %[dk], %[krs], %[b2] offen lds\n"
            "s_add_u32 m0, %[w], 12288\n s_nop 0\n buffer_load_dwordx4 %[dk], %[krs], %[b3] offen lds\n"
            "s_add_u32 m0, %[w], 16384\n s_nop 0\n buffer_load_dwordx4 %[dv], %[vrs], %[b0] offen lds\n"
            "s_add_u32 m0, %[w], 20480\n s_nop 0\n buffer_load_dwordx4 %[dv], %[vrs], %[b1] offen lds\n"
            "s_add_u32 m0, %[w], 24576\n s_nop 0\n buffer_load_dwordx4 %[dv], %[vrs], %[b2] offen lds\n"
            "s_add_u32 m0, %[w], 28672\n s_nop 0\n buffer_load_dwordx4 %[dv], %[vrs], %[b3] offen lds\n"
            :
            : [w] "s"(w), [krs] "s"(krs), [vrs] "s"(vrs), [dk] "v"(ln.dma_k), [dv] "v"(ln.dma_v),
              [b0] "s"(b[0]), [b1] "s"(b[1]), [b2] "s"(b[2]), [b3] "s"(b[3])
            : "m0", "scc", "memory");  // s_add_u32 writes scc
    };
    // The current item's tile t, block ids from the LDS table.
    auto dma = [&](uint32_t t) __attribute__((always_inline)) {
        uint32_t b[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) b[k] = uniform_u32(tbl[4 * t + k]) * stride;
        dma_raw((T + t) % 4, b);
    };
    // The first item's tile t (0-2) with the ids from the slot's record,
    // before the LDS copy exists.
    auto dma_first = [&](uint32_t t) __attribute__((always_inline)) {
        uint32_t b[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) b[k] = uniform_u32(first[4 + 4 * t + k]) * stride;
        dma_raw((T + t) % 4, b);
    };
    // The item's block ids into the LDS table, then the next item's first
    // twelve (or copies of the last id when there is none).
    auto copy_table = [&](const PipeItem &it, bool has_next, const PipeItem &nx)
                          __attribute__((always_inline)) {
        const uint32_t n4 = 4 * it.n_tiles;
        const uint32_t ntbl = min(n4 + 16, static_cast<uint32_t>(kTableLds + 16));
        for (uint32_t k = ln.tid; k < ntbl; k += 256)
            tbl[k] = (k < n4 || !has_next) ? it.table[min(k, it.nblk - 1)]
                                           : nx.table[min(k - n4, nx.nblk - 1)];
    };

    // Q of an item's rows; a lane past the item's last row loads that row
    // instead (its results are not stored, and each MFMA column is one
    // row), so every lane loads and no register is written before its load.
    bf16x8 qv[2][KS];
    auto load_q = [&](const PipeItem &it) __attribute__((always_inline)) {
#pragma unroll
        for (int rg = 0; rg < 2; ++rg) {
            const uint32_t row = it.row_begin + min(kRG * rg + ln.c, it.nrows - 1);
            const uint16_t *qp = q + (static_cast<uint64_t>(row) * num_heads + qhead) * HD + 8 * ln.gl;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
                qv[rg][kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(qp + 16 * kk));
        }
    };

    // The first item: its first three tiles' DMA goes out first, then Q,
    // then the table copy, so that their latencies overlap behind one wait.
    if (fixed_offset) {
        dma_first(0);
        dma_first(1);
        dma_first(2);
    }
    load_q(A);
    {
        // the first item's ids, then the next item's first twelve from the
        // record (the entries after them are never used for a DMA)
        const uint32_t n4 = 4 * A.n_tiles;
        const uint32_t ntbl = min(n4 + 16, static_cast<uint32_t>(kTableLds + 16));
        for (uint32_t k = ln.tid; k < ntbl; k += 256)
            tbl[k] = k < n4 ? A.table[min(k, A.nblk - 1)] : first[16 + min(k - n4, 11u)];
    }
    if (ln.tid == 0) {
        redo[0] = 0u;
        redo[1] = 0u;
    }
    wait_barrier<0>();  // the table copy, Q and (fixed offset) tiles 0-2
    // Tiles 0-2 of the current item are in their stages (issued and waited
    // for, or in flight from the previous item's DMAs past its end).
    bool ready = fixed_offset != 0;

    using True = std::true_type;
    using False = std::false_type;
    const bool both[2] = {true, true};

    for (uint32_t k_item = 0;; ++k_item) {
        const uint32_t n_tiles = A.n_tiles;
        uint32_t *const my_redo = &redo[k_item & 1];
        if (ln.tid == 0) redo[(k_item + 1) & 1] = 0u;

        floatx16 o_acc[2][DT];
        float m_run[2], l_run[2];

        // One KV tile as ordinary code for both row groups: Q.K^T, the
        // causal mask, the softmax (fixed offset, or the running max when
        // `running`), P.V.  first: tile 0 (the offset is its max; P as bf16
        // hi + lo; the row sum adds the f32 P).
        auto tile_step = [&](auto first_c, auto running_c, uint32_t t, const bool (&live)[2])
                             __attribute__((always_inline)) {
            constexpr bool first = decltype(first_c)::value;
            constexpr bool running = decltype(running_c)::value;
            const uint8_t *tile = st + ((T + t) % 4) * kPipeStage;
            const uint32_t j0 = t * kKT;
#pragma unroll
            for (int rg = 0; rg < 2; ++rg) {
                if (!live[rg]) continue;
                const uint32_t p_row = A.p_min + kRG * rg + ln.c;
                const uint32_t wp_min = A.p_min + kRG * rg;
                floatx16 s0 = {}, s1 = {};
#pragma unroll
                for (int kk = 0; kk < KS; ++kk) {
                    const uint32_t off = (kk / 2) * (kBS * 64) + ((kk & 1) ? ln.k_rd1 : ln.k_rd0);
                    const bf16x8 ka = *reinterpret_cast<const bf16x8 *>(tile + off);
                    const bf16x8 kb = *reinterpret_cast<const bf16x8 *>(tile + off + 2 * kPipeBT);
                    s0 = mfma32x32x16(ka, qv[rg][kk], s0);
                    s1 = mfma32x32x16(kb, qv[rg][kk], s1);
                }
                float sc[32];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    sc[r] = s0[r];
                    sc[16 + r] = s1[r];
                }
                if (j0 + kKT - 1 > wp_min) {
#pragma unroll
                    for (int r = 0; r < 32; ++r) {
                        const uint32_t key = j0 + 32 * (r >> 4) + 16 * ((r >> 3) & 1) + 8 * ln.gl + (r & 7);
                        sc[r] = (key <= p_row) ? sc[r] : -INFINITY;
                    }
                }
                auto tile_max = [&]() __attribute__((always_inline)) {
                    float mx = sc[0];
#pragma unroll
                    for (int r = 1; r < 32; ++r) mx = fmaxf(mx, sc[r]);
                    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                    return mx * scale_log2;
                };
                if constexpr (first) {
                    m_run[rg] = tile_max();
                } else if constexpr (running) {
                    const float mt = tile_max();
                    if (__builtin_amdgcn_ballot_w64(mt > m_run[rg] + kLazyLog2) != 0) {
                        const float m_new = fmaxf(m_run[rg], mt);
                        const float alpha = __builtin_amdgcn_exp2f(m_run[rg] - m_new);
                        l_run[rg] *= alpha;
#pragma unroll
                        for (int dt = 0; dt < DT; ++dt) o_acc[rg][dt] *= alpha;
                        m_run[rg] = m_new;
                    }
                }
                const float nm = -m_run[rg];
#pragma unroll
                for (int r = 0; r < 32; ++r) sc[r] = __builtin_amdgcn_exp2f(fmaf(sc[r], scale_log2, nm));
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    bf16x8 pb_hi, pb_lo;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float p = sc[16 * (j >> 1) + 8 * (j & 1) + e];
                        const __bf16 hi = static_cast<__bf16>(p);
                        pb_hi[e] = hi;
                        if constexpr (first) pb_lo[e] = static_cast<__bf16>(p - static_cast<float>(hi));
                        l_run[rg] += p;
                    }
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) {
                        const bf16x8 vf =
                            *reinterpret_cast<const bf16x8 *>(tile + ln.v_rd + j * kPipeBT + dt * 1024);
                        if constexpr (first) o_acc[rg][dt] = mfma32x32x16(vf, pb_lo, o_acc[rg][dt]);
                        o_acc[rg][dt] = mfma32x32x16(vf, pb_hi, o_acc[rg][dt]);
                    }
                }
            }
        };

        // One pass as ordinary code, for the row groups in `live`: running
        // max (the recompute) or the fixed offset (when the pipelined loop
        // is off).  Its tiles 0-2 are issued here; the caller has waited for
        // every DMA in flight.
        auto plain_pass = [&](auto running_c, const bool (&live)[2]) __attribute__((always_inline)) {
            // every group's state starts over (a group not in `live` keeps
            // zeros, unused), so nothing of the first pass stays live here
#pragma unroll
            for (int rg = 0; rg < 2; ++rg) {
                m_run[rg] = 0.0f;
                l_run[rg] = 0.0f;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) o_acc[rg][dt] = floatx16{};
            }
            dma(0);
            dma(1);
            dma(2);
            wait_barrier<16>();
            dma(3);
            tile_step(True{}, running_c, 0, live);
            for (uint32_t t = 1; t < n_tiles; ++t) {
                wait_barrier<16>();
                dma(t + 3);
                tile_step(False{}, running_c, t, live);
            }
            // vmcnt(0): the DMA past the end (the next item's tiles 0-2)
            __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
#pragma unroll
            for (int rg = 0; rg < 2; ++rg)
                if (live[rg]) l_run[rg] += __shfl_xor(l_run[rg], 32, 64);
        };

        // A row group's output as bf16, O scaled by 1 / l, made as soon as
        // the group's pass ends: the accumulators are read once and are dead
        // across the barrier and the output that follow.
        bf16x4 packed[2][DT][4];
        auto pack_out = [&](int rg) __attribute__((always_inline)) {
            const float inv = 1.0f / l_run[rg];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        packed[rg][dt][r4][e] = static_cast<__bf16>(o_acc[rg][dt][4 * r4 + e] * inv);
        };

        // Tiles nA .. nA + 2 of this item's ring positions carry the next
        // item's tiles 0-2 when each was issued from the LDS table.
        bool next_ready = true;
        if (fixed_offset) {
            // Tile 0 here, tiles 1 .. n - 1 in the pipelined loop.
            if (!ready) {
                dma(0);
                dma(1);
                dma(2);
                wait_barrier<0>();
            }
            next_ready = n_tiles >= 3 || !ready;
            {
                // The whole item in the generated code: tile 0 (its max
                // becomes the fixed offset), then tiles 1 .. n - 1.  Tiles
                // from `tmask` (a key index) on need the causal mask: the
                // first is the one holding row group 0's first row's last
                // visible key + 1.
                l_run[0] = 0.0f;
                l_run[1] = 0.0f;
                const uint32_t tmask = kKT * ((A.p_min + 1) / kKT);
                const uint32_t tend = T + n_tiles;
                uint32_t vtbl = lds_addr(tbl) + 16 * 3;  // the ids of tile 3
                const int32_t pr0 = static_cast<int32_t>(A.p_min + ln.c - 8 * ln.gl);
                const int32_t pr1 = static_cast<int32_t>(A.p_min + kRG + ln.c - 8 * ln.gl);
                uint32_t t_reg, j0_reg, b0, b1, b2, b3;
                uint64_t mk0, mk1, mk2;
                asm volatile(VO_PREFILL_PIPE_LOOP
                             : "={a[0:15]}"(o_acc[0][0]), "={a[16:31]}"(o_acc[0][1]),
                               "={a[32:47]}"(o_acc[0][2]), "={a[48:63]}"(o_acc[0][3]),
                               "={a[64:79]}"(o_acc[1][0]), "={a[80:95]}"(o_acc[1][1]),
                               "={a[96:111]}"(o_acc[1][2]), "={a[112:127]}"(o_acc[1][3]),
                               "+{v166}"(l_run[0]), "+{v167}"(l_run[1]), "+{v189}"(vtbl),
                               [t] "=&s"(t_reg), [j0] "=&s"(j0_reg), [b0] "=&s"(b0), [b1] "=&s"(b1),
                               [b2] "=&s"(b2), [b3] "=&s"(b3), [m0] "=&s"(mk0), [m1] "=&s"(mk1),
                               [m2] "=&s"(mk2)
                             : "{a[128:131]}"(qv[0][0]), "{a[132:135]}"(qv[0][1]),
                               "{a[136:139]}"(qv[0][2]), "{a[140:143]}"(qv[0][3]),
                               "{a[144:147]}"(qv[0][4]), "{a[148:151]}"(qv[0][5]),
                               "{a[152:155]}"(qv[0][6]), "{a[156:159]}"(qv[0][7]),
                               "{a[160:163]}"(qv[1][0]), "{a[164:167]}"(qv[1][1]),
                               "{a[168:171]}"(qv[1][2]), "{a[172:175]}"(qv[1][3]),
                               "{a[176:179]}"(qv[1][4]), "{a[180:183]}"(qv[1][5]),
                               "{a[184:187]}"(qv[1][6]), "{a[188:191]}"(qv[1][7]),
                               "{v181}"(st0 + ln.k_rd0), "{v182}"(st0 + ln.k_rd1), "{v185}"(st0 + ln.v_rd),
                               "{v187}"(ln.dma_k), "{v188}"(ln.dma_v), "{v190}"(pr0), "{v191}"(pr1),
                               [krs] "s"(krs), [vrs] "s"(vrs), [wbase] "s"(wbase), [stride] "s"(stride),
                               [tbase] "s"(T), [tend] "s"(tend), [tmask] "s"(tmask),
                               [scale] "s"(scale_log2)
                             : VO_PREFILL_PIPE_CLOBBERS, "m0", "scc", "memory");
                uint32_t t2 = ln.tid;
                asm volatile("" : "+v"(t2));
                ln = make_lane(t2);
            }
#pragma unroll
            for (int rg = 0; rg < 2; ++rg) {
                l_run[rg] += __shfl_xor(l_run[rg], 32, 64);
                const bool ok = l_run[rg] < kOverflowSum && all_finite(o_acc[rg]);  // false for inf, NaN
                if (__builtin_amdgcn_ballot_w64(kRG * rg + ln.c < A.nrows && !ok) != 0 && ln.lane == 0)
                    atomicOr(my_redo, 1u << rg);
                pack_out(rg);
            }
        } else {
            // every row group runs in the pass below, which packs it
            if (ln.tid == 0) *my_redo = 3u;
        }
        // Output of one row group: each wave its own head's rows, through
        // 8 KiB of the stage that holds no prefetched tile (this item's last
        // tile's); chunk q of row c at q ^ (c % 16).  The stores are
        // non-temporal: the output is not read again by this kernel, and
        // lines left dirty in L2 are written back when the kernel ends.
        auto write_out = [&](int rg) __attribute__((always_inline)) {
            constexpr int ROWB = HD * 2;
            constexpr int CH = HD / 8;
            uint8_t *wst = st + ((T + n_tiles + 3) % 4) * kPipeStage + head * (kRG * ROWB);
            uint8_t *row_at = wst + ln.c * ROWB + 8 * ln.gl;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const uint32_t q4 = static_cast<uint32_t>(4 * dt + r4) ^ (ln.c % CH);
                    *reinterpret_cast<bf16x4 *>(row_at + 16 * q4) = packed[rg][dt][r4];
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            uint8_t *obase = reinterpret_cast<uint8_t *>(
                out + (static_cast<uint64_t>(A.row_begin + kRG * rg) * num_heads + qhead) * HD);
            // every chunk read first (one wait), then the stores of the
            // item's rows; lane L stores chunk L % 16 of rows L / 16 + 4 k
            constexpr int NK = kRG * CH / 64;
            const uint32_t row_bytes = num_heads * HD * 2;
            const uint32_t row0 = ln.lane / CH;
            const uint32_t q4 = ln.lane % CH;
            const uint32_t voff = row0 * row_bytes + 16 * q4;
            u32x4 vals[NK];
#pragma unroll
            for (int k = 0; k < NK; ++k) {
                const uint32_t row = row0 + (64 / CH) * k;
                vals[k] = *reinterpret_cast<const u32x4 *>(wst + row * ROWB + 16 * (q4 ^ (row % CH)));
            }
#pragma unroll
            for (int k = 0; k < NK; ++k) {
                const uint32_t row = row0 + (64 / CH) * k;
                if (kRG * rg + row < A.nrows)
                    __builtin_nontemporal_store(
                        vals[k], reinterpret_cast<u32x4 *>(obase + (voff + (64 / CH) * k * row_bytes)));
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        };

        wait_barrier<63>();  // the flags; every wave is done with this item's tiles
        const uint32_t again = uniform_u32(*my_redo);
        if (again != 0) {
            // The recompute with the running max for the 32-row groups that
            // left the fixed-offset range (prefill_dma_kernel's second pass),
            // after the DMAs in flight (the next item's tiles) have landed.
            // A group kept from the first pass is written first, so that no
            // packed output is held across the pass.
            const bool live[2] = {(again & 1u) != 0, (again & 2u) != 0};
#pragma unroll
            for (int rg = 0; rg < 2; ++rg)
                if (!live[rg]) write_out(rg);
            wait_barrier<0>();  // also every wave's staging reads, before the DMA rewrites the stages
            plain_pass(True{}, live);
            next_ready = true;
#pragma unroll
            for (int rg = 0; rg < 2; ++rg) {
                if (live[rg]) {
                    pack_out(rg);
                } else {
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                        for (int r4 = 0; r4 < 4; ++r4) packed[rg][dt][r4] = bf16x4{};  // written above
                }
            }
            wait_barrier<63>();  // every wave is done with the stages
        }

        // The next item's Q (this item's is no longer needed).
        if (has_b) load_q(B);

        // The row groups not written above, one at a time.
#pragma unroll
        for (int rg = 0; rg < 2; ++rg)
            if (again == 0 || ((again >> rg) & 1u) != 0) write_out(rg);
        if (!has_b) break;
        // The next item: its table (and the first ids of the one after),
        // then one wait for its Q, its table and its tiles 0-2; the barrier
        // also orders every wave's output reads before the DMA of its tile 3
        // rewrites that stage.
        copy_table(B, has_c, C);
        T = (T + n_tiles) % 4;
        ready = next_ready;
        A = B;
        B = C;
        has_b = has_c;
        ++i;
        has_c = i + 2 < i_end;
        C = pipe_item(descs + 4 * (has_c ? i + 2 : i), tables);  // waited for by the barrier
        wait_barrier<0>();
    }
    // The last item's DMAs past its end write LDS: they land before the
    // workgroup ends.
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
}

// VO_PREFILL_STAGING=regs selects the register-staged kernel above (A/B).
bool prefill_use_dma() {
    static const bool dma = [] {
        const char *v = std::getenv("VO_PREFILL_STAGING");
        return !(v && std::string(v) == "regs");
    }();
    return dma;
}

// VO_PREFILL_OFFSET=running runs the DMA kernel with the running row max
// from the start instead of the fixed tile-0 offset (A/B).  Read at every
// launch.
bool prefill_fixed_offset() {
    const char *v = std::getenv("VO_PREFILL_OFFSET");
    return !(v && std::string(v) == "running");
}

// VO_PREFILL_NARROW=0 keeps 64-row workgroups on small grids (A/B).  Read at
// every launch.
bool prefill_narrow_enabled() {
    const char *v = std::getenv("VO_PREFILL_NARROW");
    return !(v && std::string(v) == "0");
}

// VO_PREFILL_PIPE=0 runs the 8-wavefront DMA kernel instead of the
// pipelined one at head_dim 128, GQA 4 (A/B).  Read at every launch.
bool prefill_pipe_enabled() {
    const char *v = std::getenv("VO_PREFILL_PIPE");
    return !(v && std::string(v) == "0");
}

template <int HD, int G, int R>
hipError_t launch_gr(const PoolLayer &pool, const MetaView &meta, const PrefillPlan &plan,
                     const uint16_t *q, uint16_t *out, uint32_t num_heads, float scale_log2,
                     hipStream_t stream) {
    constexpr int HALVES = kQT / (kRG * R);
    const uint64_t grid = static_cast<uint64_t>(plan.num_items) * HALVES * pool.kv_heads;
    if (grid > 0x7fffffffull || plan.num_long > plan.num_items) return hipErrorInvalidValue;
    // The DMA kernel stages a sequence's whole block table in LDS, and its
    // three 32 KiB stages at head_dim 128 leave room for one workgroup per
    // CU, which takes 8 wavefronts to fill the SIMDs -- or 4 when the grid
    // has fewer workgroups than CUs anyway (32-row workgroups below).  Its
    // items are those past the plan's num_long; the others (rows past its
    // table) run on the register-staged kernel, launched first.
    uint32_t regs_items = plan.num_items;
    constexpr bool dma_shape = HD == 64 || G * R == 8 || (G == 4 && R == 1);
    if constexpr (dma_shape) {
        if (prefill_use_dma() && pool.elems != 0 && pool.elems * 2 <= 0xffffffffull)
            regs_items = plan.num_long;
    }
    const uint32_t per_item = HALVES * pool.kv_heads;
    // Each launch is timed (when profiling is on) under the name of its
    // kernel instance, so that a caller can tell which one ran.
    if (regs_items != 0) {
        KernelTimer timer("prefill_regs", stream);
        hipLaunchKernelGGL((prefill_mfma_kernel<HD, G, R>), dim3(regs_items * per_item),
                           dim3(64 * G * R), 0, stream, pool.k, pool.v, pool.kv_heads,
                           meta.table_off, meta.tables, plan.work, q, out, num_heads, scale_log2);
        if (hipError_t err = hipGetLastError(); err != hipSuccess) return err;
    }
    if constexpr (HD == 128 && G == 4 && R == 2) {
        // 64-row workgroups at the Llama-3-8B shape: the pipelined kernel.
        if (regs_items < plan.num_items && plan.pipe != nullptr && plan.pipe_slots != 0 &&
            prefill_pipe_enabled()) {
            KernelTimer timer("prefill_pipe", stream);
            hipLaunchKernelGGL(prefill_pipe_kernel, dim3(plan.pipe_slots * pool.kv_heads), dim3(256), 0,
                               stream, pool.k, pool.v, pool.kv_heads, meta.tables, plan.pipe,
                               plan.pipe_slots, q, out, num_heads, scale_log2,
                               prefill_fixed_offset() ? 1u : 0u, static_cast<uint32_t>(pool.elems * 2));
            return hipGetLastError();
        }
    }
    if constexpr (dma_shape) {
        if (regs_items < plan.num_items) {
            KernelTimer timer(G == 4 && R == 1 ? "prefill_dma_narrow" : "prefill_dma", stream);
            hipLaunchKernelGGL((prefill_dma_kernel<HD, G, R>),
                               dim3((plan.num_items - regs_items) * per_item), dim3(64 * G * R), 0,
                               stream, pool.k, pool.v, pool.kv_heads, meta.table_off, meta.tables,
                               plan.work + 4 * static_cast<uint64_t>(regs_items), q, out, num_heads,
                               scale_log2, prefill_fixed_offset() ? 1u : 0u,
                               static_cast<uint32_t>(pool.elems * 2));
            return hipGetLastError();
        }
    }
    return hipSuccess;
}

template <int HD, int G>
hipError_t launch_g(const PoolLayer &pool, const MetaView &meta, const PrefillPlan &plan,
                    const uint16_t *q, uint16_t *out, uint32_t num_heads, float scale_log2,
                    uint32_t num_cus, hipStream_t stream) {
    // Eight waves per workgroup: two row groups for up to 4 heads, one for 8.
    // A grid of fewer 64-row workgroups than CUs (a few long chunks, as in a
    // mixed serving step) leaves CUs idle while its longest items run; 32-row
    // workgroups of 4 wavefronts then double the grid and halve each
    // workgroup's MFMA work per KV tile.
    if constexpr (G == 4) {
        if (prefill_narrow_enabled() &&
            static_cast<uint64_t>(plan.num_items) * pool.kv_heads < num_cus)
            return launch_gr<HD, 4, 1>(pool, meta, plan, q, out, num_heads, scale_log2, stream);
    }
    return launch_gr<HD, G, (G <= 4 ? 2 : 1)>(pool, meta, plan, q, out, num_heads, scale_log2,
                                              stream);
}

template <int HD>
hipError_t launch_hd(const PoolLayer &pool, const MetaView &meta, const PrefillPlan &plan,
                     const uint16_t *q, uint16_t *out, uint32_t num_heads, float scale_log2,
                     uint32_t num_cus, hipStream_t stream) {
    switch (num_heads / pool.kv_heads) {
        case 2: return launch_g<HD, 2>(pool, meta, plan, q, out, num_heads, scale_log2, num_cus, stream);
        case 4: return launch_g<HD, 4>(pool, meta, plan, q, out, num_heads, scale_log2, num_cus, stream);
        case 8: return launch_g<HD, 8>(pool, meta, plan, q, out, num_heads, scale_log2, num_cus, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool prefill_mfma_supported(uint32_t head_dim, uint32_t block_size, uint32_t group) {
    return (head_dim == 64 || head_dim == 128) && block_size == kBS &&
           (group == 2 || group == 4 || group == 8);
}

uint32_t prefill_rows_per_tile() { return kQT; }

uint32_t prefill_dma_max_keys() { return kTableLds * kBS; }

hipError_t launch_prefill_mfma(const PoolLayer &pool, const MetaView &meta,
                               const PrefillPlan &plan, const uint16_t *q, uint16_t *out,
                               uint32_t num_heads, float scale, uint32_t num_cus,
                               hipStream_t stream) {
    if (plan.num_items == 0) return hipSuccess;
    const float scale_log2 = scale * 1.4426950408889634f;
    switch (pool.head_dim) {
        case 64: return launch_hd<64>(pool, meta, plan, q, out, num_heads, scale_log2, num_cus, stream);
        case 128: return launch_hd<128>(pool, meta, plan, q, out, num_heads, scale_log2, num_cus, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace kernels
}  // namespace vo

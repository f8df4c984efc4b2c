// chunked_prefill.hip -- causal paged attention for prefill chunks on gfx950
// bf16 MFMA (FlashAttention-2 style, online softmax, fp32 accumulation).
//
// Math: crates/engine/src/backend/cpu/attention.rs:5-16 (prefill path,
// cpu/mod.rs:287-312).  Row t of sequence s sits at position p = ctx_s + i
// and attends to keys 0..p of its sequence through the block table; the
// cached context is fully visible and the chunk is causal because row t is
// given only p + 1 keys (attention.rs:16).
//
// Work split.  A workgroup owns one 32-row query tile of one sequence and one
// KV head k, with one wavefront per query head of k's GQA group (G waves), so
// every K/V tile staged in LDS serves all G heads.  It walks the 64-key KV
// tiles 0 .. p_max/64 of its sequence; tiles past the tile's last row are
// never touched, tiles wholly before its first row need no mask.  Work items
// are ordered longest first (host plan), so the long tiles start early.
//
// Per wavefront and KV tile (keys j0 .. j0+63), with c = lane % 32 the query
// row of the lane and gl = lane / 32:
//   S^T = K . Q^T    v_mfma_f32_32x32x16_bf16, A = 32 keys x 16 dims of K
//                    from LDS, B = Q^T (the wave's 32 query rows, kept in
//                    registers for the whole kernel); two 32-key halves,
//                    head_dim/16 steps each.  A-row i reads key pi(i), pi =
//                    swap of bits 2 and 3, so that the result register r of
//                    lane l holds key 32*half + 16*(r>>3) + 8*gl + (r&7).
//   softmax          each lane holds 32 scores of its own query row; the row
//                    max is a local max plus one lane^32 exchange.
//   O^T += V^T . P^T B = P^T is then exactly the lane's own probabilities:
//                    16-key step j uses registers 8*(j&1) .. +7 of half j>>1.
//                    A = 32 dims x 16 keys of V^T from LDS.  Output rows are
//                    dims and columns query rows, so the rescale by the new
//                    max is lane-local.  The first KV tile, where rows with
//                    few keys live, feeds P as bf16 hi + lo parts (two
//                    MFMAs) so that short rows keep rtol 1e-2 / atol 2e-3.
//
// LDS: K tile [64 keys][head_dim] and V^T tile [head_dim][64 keys], 16-byte
// units XOR-swizzled by row so that the 16 lanes of one ds_read_b128 phase
// hit 16 different 16-byte slots of a 256-byte bank sweep; two buffers, the
// next tile's global loads are in flight while the current one is computed.
//
// Roofline: bf16 MFMA.  Algorithmic FLOPs = sum over rows of (keys) * heads *
// 4 * head_dim (Q.K^T and P.V, causal-aware).
#include <cmath>

#include "vo_device.hpp"
#include "vo_kernels.hpp"

namespace vo {
namespace kernels {

namespace {

constexpr int kBS = 16;  // block size of the MFMA path
constexpr int kQT = 32;  // query rows per tile
constexpr int kKT = 64;  // keys per KV tile (4 blocks)

__device__ __forceinline__ floatx16 mfma32x32x16(bf16x8 a, bf16x8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 16-byte slot of unit u in LDS row `row` (see the header comment).
template <int UNITS_PER_ROW>
__device__ __forceinline__ uint32_t swizzle(uint32_t u, uint32_t row) {
    if constexpr (UNITS_PER_ROW == 16)
        return u ^ (row & 15u);
    else
        return u ^ ((row >> 1) & 7u);
}

// Swap bits 2 and 3: the A-row -> key order of the Q.K^T MFMA.
__device__ __forceinline__ uint32_t key_perm(uint32_t i) {
    return (i & ~0xCu) | ((i & 4u) << 1) | ((i & 8u) >> 1);
}

template <int HD, int G>
__global__ __launch_bounds__(64 * G) __attribute__((amdgpu_waves_per_eu(2))) void prefill_mfma_kernel(
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool, uint32_t kv_heads,
    const uint32_t *__restrict__ table_off, const uint32_t *__restrict__ tables,
    const uint32_t *__restrict__ work, uint32_t num_items, const uint16_t *__restrict__ q,
    uint16_t *__restrict__ out, uint32_t num_heads, float scale_log2) {
    constexpr int KS = HD / 16;                 // Q.K^T k-steps
    constexpr int DT = HD / 32;                 // P.V output tiles
    constexpr int KROW = HD * 2;                // bytes of one K row in LDS
    constexpr int KUPR = HD / 8;                // 16-byte units per K row
    constexpr int TILE_BYTES = kKT * HD * 2;    // K (or V) tile in LDS
    constexpr int UNITS = kKT * HD / 8;         // 16-byte units per K (or V) tile
    constexpr int THREADS = 64 * G;
    constexpr int UPT = UNITS / THREADS;        // units per thread per tile
    constexpr int BLOCK_UNITS = 2 * HD;         // units per (block, kv head) tile
    constexpr uint32_t kTile = kBS * HD;        // elements per (block, kv head) tile
    static_assert(UNITS % THREADS == 0, "tile units must divide over the workgroup");

    __shared__ __align__(16) uint8_t lds[2][2][TILE_BYTES];  // [buffer][K|V]

    const uint32_t item = blockIdx.x % num_items;
    const uint32_t kvh = blockIdx.x / num_items;
    const uint32_t row_begin = work[4 * item];
    const uint32_t nrows = work[4 * item + 1];
    const uint32_t p_min = work[4 * item + 2];
    const uint32_t seq = work[4 * item + 3];
    const uint32_t p_max = p_min + nrows - 1;
    const uint32_t n_tiles = p_max / kKT + 1;
    const uint32_t nblk = p_max / kBS + 1;
    const uint32_t *table = tables + table_off[seq];

    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t c = lane & 31;  // query row of this lane within the tile
    const uint32_t gl = lane >> 5;
    const uint32_t qhead = kvh * G + wave;
    const bool row_ok = c < nrows;
    const uint32_t p_row = p_min + c;

    // Q^T operand, k-step kk: dims 16*kk + 8*gl .. +7 of row c.
    bf16x8 qv[KS];
    {
        const uint16_t *qp =
            q + (static_cast<uint64_t>(row_begin + c) * num_heads + qhead) * HD + 8 * gl;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
            qv[kk] = row_ok ? __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(qp + 16 * kk))
                            : bf16x8{};
    }

    // Global -> register staging of one KV tile, then register -> LDS.
    u32x4 kreg[UPT], vreg[UPT];
    auto gload = [&](uint32_t t) {
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
            const uint32_t U = tid + THREADS * i;
            const uint32_t b = U / BLOCK_UNITS;
            const uint32_t o = U % BLOCK_UNITS;
            const uint32_t blk = table[min(4 * t + b, nblk - 1)];
            const uint64_t base = (static_cast<uint64_t>(blk) * kv_heads + kvh) * kTile + 8 * o;
            kreg[i] = *reinterpret_cast<const u32x4 *>(k_pool + base);
            vreg[i] = *reinterpret_cast<const u32x4 *>(v_pool + base);
        }
    };
    auto lstore = [&](int buf) {
        uint8_t *kl = lds[buf][0];
        uint8_t *vl = lds[buf][1];
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
            const uint32_t U = tid + THREADS * i;
            const uint32_t b = U / BLOCK_UNITS;
            const uint32_t o = U % BLOCK_UNITS;
            // K pool tile [HD/32][16 keys][32 dims]: unit o = (chunk, key, quarter).
            const uint32_t key = kBS * b + (o / 4) % kBS;
            const uint32_t ku = (o / 64) * 4 + o % 4;
            *reinterpret_cast<u32x4 *>(kl + key * KROW + swizzle<KUPR>(ku, key) * 16) = kreg[i];
            // V pool tile [HD dims][16 keys]: unit o = (dim, half).
            const uint32_t d = o / 2;
            const uint32_t vu = 2 * b + o % 2;
            *reinterpret_cast<u32x4 *>(vl + d * (kKT * 2) + swizzle<8>(vu, d) * 16) = vreg[i];
        }
    };

    float m_run = -INFINITY;
    float l_run = 0.0f;
    floatx16 o_acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o_acc[dt] = floatx16{};

    const uint32_t ka = key_perm(c);  // A-row c of the Q.K^T MFMA reads key ka (+32)

    gload(0);
    lstore(0);
    __syncthreads();

    for (uint32_t t = 0; t < n_tiles; ++t) {
        const int buf = t & 1;
        const bool more = t + 1 < n_tiles;
        if (more) gload(t + 1);

        const uint8_t *kl = lds[buf][0];
        const uint8_t *vl = lds[buf][1];

        // S^T = K . Q^T for the two 32-key halves.
        floatx16 s0 = {}, s1 = {};
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            const uint32_t u = 2 * kk + gl;
            const bf16x8 a0 = *reinterpret_cast<const bf16x8 *>(kl + ka * KROW + swizzle<KUPR>(u, ka) * 16);
            const bf16x8 a1 =
                *reinterpret_cast<const bf16x8 *>(kl + (32 + ka) * KROW + swizzle<KUPR>(u, 32 + ka) * 16);
            s0 = mfma32x32x16(a0, qv[kk], s0);
            s1 = mfma32x32x16(a1, qv[kk], s1);
        }

        // Online softmax for this lane's query row.
        float sc[32];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            sc[r] = s0[r] * scale_log2;
            sc[16 + r] = s1[r] * scale_log2;
        }
        const uint32_t j0 = t * kKT;
        if (j0 + kKT - 1 > p_min) {
            // Diagonal tile: key j is visible to this row iff j <= p_row.
#pragma unroll
            for (int r = 0; r < 32; ++r) {
                const uint32_t key = j0 + 32 * (r >> 4) + 16 * ((r >> 3) & 1) + 8 * gl + (r & 7);
                sc[r] = (key <= p_row) ? sc[r] : -INFINITY;
            }
        }
        float mt = sc[0];
#pragma unroll
        for (int r = 1; r < 32; ++r) mt = fmaxf(mt, sc[r]);
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float m_new = fmaxf(m_run, mt);  // finite: tile 0 holds key 0 for every row
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        float ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 32; ++r) {
            sc[r] = __builtin_amdgcn_exp2f(sc[r] - m_new);
            ps += sc[r];
        }
        l_run = l_run * alpha + ps;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o_acc[dt] *= alpha;

        // O^T += V^T . P^T over four 16-key steps.
        const bool split_p = (t == 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bf16x8 pb_hi, pb_lo;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float p = sc[16 * (j >> 1) + 8 * (j & 1) + i];
                const __bf16 hi = static_cast<__bf16>(p);
                pb_hi[i] = hi;
                pb_lo[i] = static_cast<__bf16>(p - static_cast<float>(hi));
            }
            const uint32_t vu = 2 * j + gl;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const uint32_t d = 32 * dt + c;
                const bf16x8 a =
                    *reinterpret_cast<const bf16x8 *>(vl + d * (kKT * 2) + swizzle<8>(vu, d) * 16);
                if (split_p) o_acc[dt] = mfma32x32x16(a, pb_lo, o_acc[dt]);
                o_acc[dt] = mfma32x32x16(a, pb_hi, o_acc[dt]);
            }
        }

        if (more) lstore(buf ^ 1);
        __syncthreads();
    }

    l_run += __shfl_xor(l_run, 32, 64);
    if (!row_ok) return;
    const float inv = 1.0f / l_run;
    uint16_t *op = out + (static_cast<uint64_t>(row_begin + c) * num_heads + qhead) * HD + 4 * gl;
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

template <int HD, int G>
hipError_t launch_g(const PoolLayer &pool, const MetaView &meta, const PrefillPlan &plan,
                    const uint16_t *q, uint16_t *out, uint32_t num_heads, float scale_log2,
                    hipStream_t stream) {
    const uint64_t grid = static_cast<uint64_t>(plan.num_items) * pool.kv_heads;
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
    KernelTimer timer("prefill_mfma", stream);
    hipLaunchKernelGGL((prefill_mfma_kernel<HD, G>), dim3(static_cast<uint32_t>(grid)),
                       dim3(64 * G), 0, stream, pool.k, pool.v, pool.kv_heads, meta.table_off,
                       meta.tables, plan.work, plan.num_items, q, out, num_heads, scale_log2);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const PoolLayer &pool, const MetaView &meta, const PrefillPlan &plan,
                     const uint16_t *q, uint16_t *out, uint32_t num_heads, float scale_log2,
                     hipStream_t stream) {
    switch (num_heads / pool.kv_heads) {
        case 2: return launch_g<HD, 2>(pool, meta, plan, q, out, num_heads, scale_log2, stream);
        case 4: return launch_g<HD, 4>(pool, meta, plan, q, out, num_heads, scale_log2, stream);
        case 8: return launch_g<HD, 8>(pool, meta, plan, q, out, num_heads, scale_log2, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool prefill_mfma_supported(uint32_t head_dim, uint32_t block_size, uint32_t group) {
    return (head_dim == 64 || head_dim == 128) && block_size == kBS &&
           (group == 2 || group == 4 || group == 8);
}

uint32_t prefill_rows_per_tile() { return kQT; }

hipError_t launch_prefill_mfma(const PoolLayer &pool, const MetaView &meta,
                               const PrefillPlan &plan, const uint16_t *q, uint16_t *out,
                               uint32_t num_heads, float scale, hipStream_t stream) {
    if (plan.num_items == 0) return hipSuccess;
    const float scale_log2 = scale * 1.4426950408889634f;
    switch (pool.head_dim) {
        case 64: return launch_hd<64>(pool, meta, plan, q, out, num_heads, scale_log2, stream);
        case 128: return launch_hd<128>(pool, meta, plan, q, out, num_heads, scale_log2, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace kernels
}  // namespace vo

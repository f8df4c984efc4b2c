// rope.hip -- rotary position embedding on bf16 rows, alone (Backend::rope)
// and fused with the paged KV-cache write.
//
// Math (crates/engine/src/backend/cpu/rope.rs:86-100): each head vector of
// width d = 2*half splits into x1 = x[..half], x2 = x[half..]; pair i at
// position p uses the precomputed cos/sin of table row p:
//   x1'[i] = x1[i]*cos - x2[i]*sin,   x2'[i] = x2[i]*cos + x1[i]*sin.
// Every product and sum is a separately rounded f32 operation in that order
// (no contraction into FMA), as the reference
// computes, so the f32 result equals the reference's on the same inputs; it
// is then rounded to bf16 (round to nearest even).
//
// rope_rows_kernel: one thread per (row, head, 8 pairs), or per pair when
// half is not a multiple of 8; 16-byte loads and stores in the first case.
// rope_cache_kernel: the layer's "rope(q); rope(k); write_kv(k, v)"
// (model.rs:307-311) as one launch over the step's write plan: one workgroup
// per (run of rows with consecutive slots in one block, KV head), and in it
// one wavefront per RPI rows of the run (4 at head_dim 128), so that each
// wavefront waits for one chain of loads.  A lane owns 8 dims of a row; its
// rotation partner (the other half of the head) is the lane UPR/2 away in
// the same row, reached with a lane shuffle.  The wavefront rotates its rows'
// q for the G query heads of its KV head in place, writes the rotated K into
// the key-major tile and V into the dim-major tile (transposed in registers:
// per dim the wavefront's RPI keys, 2 RPI bytes, in a whole block's run),
// reading each row's cos/sin once.  q may be read from one buffer
// and written to another (the rows of a fused QKV projection output are
// strided: q_in_ld, kv_ld), or rotated in place (q_in == q_out).
//
// Roofline: HBM.  Bytes per row = q read + written, k and v read and written
// to the pool, cos/sin 2*half*4*2 (mostly cache hits).
#include "vo_device.hpp"
#include "vo_kernels.hpp"

namespace vo {
namespace kernels {

namespace {

__device__ __forceinline__ float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return static_cast<uint32_t>(f32_to_bf16_bits(a)) |
           (static_cast<uint32_t>(f32_to_bf16_bits(b)) << 16);
}

// x1' (first half) and x2' (second half) of rope.rs:95-96.  HIP compiles
// with contraction on, which would fuse a product into the following add
// (an FMA rounds once where the reference rounds twice); the pragma keeps
// each product and sum rounded on its own.
__device__ __forceinline__ float rot_first(float a, float b, float c, float s) {
#pragma clang fp contract(off)
    const float ac = a * c;
    const float bs = b * s;
    return ac - bs;
}
__device__ __forceinline__ float rot_second(float a, float b, float c, float s) {
#pragma clang fp contract(off)
    const float bc = b * c;
    const float as = a * s;
    return bc + as;
}

// 8 pairs: x1 = a (8 bf16), x2 = b (8 bf16) -> rotated in place.
__device__ __forceinline__ void rotate8(u32x4 &a, u32x4 &b, const float *c, const float *s) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float a0 = lo_f(a[k]), a1 = hi_f(a[k]);
        const float b0 = lo_f(b[k]), b1 = hi_f(b[k]);
        const float c0 = c[2 * k], c1 = c[2 * k + 1], s0 = s[2 * k], s1 = s[2 * k + 1];
        a[k] = pack2(rot_first(a0, b0, c0, s0), rot_first(a1, b1, c1, s1));
        b[k] = pack2(rot_second(a0, b0, c0, s0), rot_second(a1, b1, c1, s1));
    }
}

template <bool WIDE>
__global__ __launch_bounds__(256) void rope_rows_kernel(uint16_t *__restrict__ x, uint32_t rows,
                                                        uint32_t cols, uint32_t half,
                                                        const uint32_t *__restrict__ positions,
                                                        const float *__restrict__ cos_tab,
                                                        const float *__restrict__ sin_tab) {
    constexpr uint32_t PW = WIDE ? 8 : 1;  // pairs per thread
    const uint32_t chunks = half / PW;
    const uint32_t heads = cols / (2 * half);
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<uint64_t>(rows) * heads * chunks) return;
    const uint32_t row = static_cast<uint32_t>(idx / (static_cast<uint64_t>(heads) * chunks));
    const uint32_t rem = static_cast<uint32_t>(idx % (static_cast<uint64_t>(heads) * chunks));
    const uint32_t head = rem / chunks;
    const uint32_t p0 = (rem % chunks) * PW;
    uint16_t *h = x + static_cast<uint64_t>(row) * cols + static_cast<uint64_t>(head) * 2 * half;
    const uint64_t t = static_cast<uint64_t>(positions[row]) * half + p0;
    if constexpr (WIDE) {
        float c[8], s[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            c[k] = cos_tab[t + k];
            s[k] = sin_tab[t + k];
        }
        u32x4 a = *reinterpret_cast<const u32x4 *>(h + p0);
        u32x4 b = *reinterpret_cast<const u32x4 *>(h + half + p0);
        rotate8(a, b, c, s);
        *reinterpret_cast<u32x4 *>(h + p0) = a;
        *reinterpret_cast<u32x4 *>(h + half + p0) = b;
    } else {
        const float c = cos_tab[t], s = sin_tab[t];
        const float a = bf16_bits_to_f32(h[p0]), b = bf16_bits_to_f32(h[half + p0]);
        h[p0] = f32_to_bf16_bits(rot_first(a, b, c, s));
        h[half + p0] = f32_to_bf16_bits(rot_second(a, b, c, s));
    }
}

template <int HD>
__global__ __launch_bounds__(64 * (16 / (64 / (HD / 8)))) void rope_cache_kernel(
    uint16_t *__restrict__ k_pool, uint16_t *__restrict__ v_pool, uint32_t kv_heads,
    const uint16_t *q_in, uint32_t q_in_ld, uint16_t *q_out, uint32_t q_out_ld, uint32_t group,
    const uint16_t *__restrict__ keys, const uint16_t *__restrict__ values, uint32_t kv_ld,
    const uint32_t *__restrict__ segments,
    const uint32_t *__restrict__ positions, const float *__restrict__ cos_tab,
    const float *__restrict__ sin_tab, uint32_t num_items) {
    constexpr uint32_t BS = 16;
    constexpr uint32_t HALF = HD / 2;
    constexpr int DPL = HD / 64;        // V dims per lane
    constexpr uint32_t UPR = HD / 8;    // 16-byte units per row of one head
    constexpr uint32_t RPI = 64 / UPR;  // rows per pass (one instruction covers them)
    // One workgroup per (run, KV head); wavefront w takes the run's rows
    // RPI w .. RPI w + RPI - 1, so a wavefront's loads form one dependent
    // chain (position, then cos/sin, K, Q) instead of one per pass.
    const uint32_t item = blockIdx.x;
    if (item >= num_items) return;
    const uint32_t pass = threadIdx.x >> 6;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t seg = item / kv_heads;
    const uint32_t kvh = item % kv_heads;
    const uint32_t row0 = segments[3 * seg];
    const uint32_t n = segments[3 * seg + 1];  // 1 .. BS
    const uint32_t slot0 = segments[3 * seg + 2];
    if (RPI * pass >= n) return;  // whole wavefront: no row of the run in this pass
    // A superseded row (slot kSkipSlot) only has its q rotated.
    const bool cache = slot0 != kSkipSlot;
    const uint32_t off0 = cache ? slot0 % BS : 0;
    const uint64_t width = kv_ld;
    const uint64_t tile = cache ? (static_cast<uint64_t>(slot0 / BS) * kv_heads + kvh) * (BS * HD) : 0;

    // V of this pass's rows (dims DPL lane .. + DPL - 1), loaded first: it
    // depends on nothing else.  Rows past the run load its last row (not
    // stored), so the loads go out together, without a branch between them.
    uint16_t vv[DPL][RPI];
    {
        const uint16_t *vsrc = values + static_cast<uint64_t>(row0) * width + kvh * HD + DPL * lane;
#pragma unroll
        for (uint32_t ii = 0; ii < RPI; ++ii) {
            const uint32_t iv = min(RPI * pass + ii, n - 1);
            if constexpr (DPL == 2) {
                const uint32_t w = *reinterpret_cast<const uint32_t *>(vsrc + iv * width);
                vv[0][ii] = static_cast<uint16_t>(w & 0xffffu);
                vv[1][ii] = static_cast<uint16_t>(w >> 16);
            } else {
                vv[0][ii] = vsrc[iv * width];
            }
        }
    }

    const uint32_t u = lane % UPR;
    const bool first_half = u < UPR / 2;
    const uint32_t d = 8 * u;
    const uint32_t p0 = 8 * (u % (UPR / 2));  // first pair of the lane's 8 dims
    const uint32_t i = lane / UPR + RPI * pass;

    // Rotates a lane's 8 dims with its partner lane's (the other half).
    auto rot = [&](u32x4 own, const float *c, const float *s) -> u32x4 {
        u32x4 other;
#pragma unroll
        for (int k = 0; k < 4; ++k) other[k] = __shfl_xor(own[k], UPR / 2, 64);
        u32x4 a = first_half ? own : other;
        u32x4 b = first_half ? other : own;
        rotate8(a, b, c, s);
        return first_half ? a : b;
    };

    {
        // Every lane of a row takes part in the shuffles, so rows past the
        // run clamp to its last row and skip only the stores.
        const bool live = i < n;
        const uint32_t row = row0 + min(i, n - 1);
        // K and the first four query heads need only the row: they load
        // beside the position, before the cos/sin that wait for it.  Later
        // heads (G > 4) load after the first ones' stores (q may be rotated
        // in place).
        const u32x4 kin = *reinterpret_cast<const u32x4 *>(keys + row * width + kvh * HD + d);
        auto load_q4 = [&](uint32_t h0, u32x4 (&qin)[4]) {
#pragma unroll
            for (uint32_t hh = 0; hh < 4; ++hh) {
                const uint32_t h = min(h0 + hh, group - 1);
                const uint32_t col = (kvh * group + h) * HD + d;
                qin[hh] = *reinterpret_cast<const u32x4 *>(q_in + static_cast<uint64_t>(row) * q_in_ld + col);
            }
        };
        u32x4 qfirst[4];
        load_q4(0, qfirst);
        const uint64_t t = static_cast<uint64_t>(positions[row]) * HALF + p0;
        float c[8], s[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            c[k] = cos_tab[t + k];
            s[k] = sin_tab[t + k];
        }
        const u32x4 kout = rot(kin, c, s);
        if (live && cache)
            *reinterpret_cast<u32x4 *>(k_pool + tile + (d / 32) * (BS * 32) + (off0 + i) * 32 + d % 32) = kout;
        // The G query heads four at a time, loads first, so that four loads
        // are in flight rather than one.
        for (uint32_t h0 = 0; h0 < group; h0 += 4) {
            u32x4 qin[4];
            if (h0 == 0) {
#pragma unroll
                for (uint32_t hh = 0; hh < 4; ++hh) qin[hh] = qfirst[hh];
            } else {
                load_q4(h0, qin);
            }
#pragma unroll
            for (uint32_t hh = 0; hh < 4; ++hh) {
                const uint32_t col = (kvh * group + h0 + hh) * HD + d;
                const u32x4 qout = rot(qin[hh], c, s);
                if (live && h0 + hh < group)
                    *reinterpret_cast<u32x4 *>(q_out + static_cast<uint64_t>(row) * q_out_ld + col) = qout;
            }
        }
    }

    if (!cache) return;
    // This pass's RPI keys of each of the lane's dims in the dim-major V
    // tile: one 2 RPI-byte store per dim for a whole run, else key by key.
    uint16_t *vdst = v_pool + tile + static_cast<uint64_t>(DPL * lane) * BS;
    if (n == BS) {
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
            uint32_t w[RPI / 2];
#pragma unroll
            for (uint32_t p = 0; p < RPI / 2; ++p)
                w[p] = static_cast<uint32_t>(vv[e][2 * p]) | (static_cast<uint32_t>(vv[e][2 * p + 1]) << 16);
            if constexpr (RPI == 4)
                *reinterpret_cast<u32x2 *>(vdst + e * BS + RPI * pass) = u32x2{w[0], w[1]};
            else
                *reinterpret_cast<u32x4 *>(vdst + e * BS + RPI * pass) = u32x4{w[0], w[1], w[2], w[3]};
        }
    } else {
#pragma unroll
        for (uint32_t ii = 0; ii < RPI; ++ii) {
            const uint32_t iv = RPI * pass + ii;
            if (iv < n) {
#pragma unroll
                for (int e = 0; e < DPL; ++e) vdst[e * BS + off0 + iv] = vv[e][ii];
            }
        }
    }
}

}  // namespace

hipError_t launch_rope_rows(uint16_t *x, uint32_t rows, uint32_t cols, uint32_t half,
                            const uint32_t *positions, const float *cos_tab, const float *sin_tab,
                            hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    if (half == 0 || cols % (2 * half) != 0) return hipErrorInvalidValue;
    const bool wide = half % 8 == 0;
    const uint64_t per_row = static_cast<uint64_t>(cols / (2 * half)) * (wide ? half / 8 : half);
    const uint64_t grid = (static_cast<uint64_t>(rows) * per_row + 255) / 256;
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
    KernelTimer timer("rope", stream);
    if (wide)
        hipLaunchKernelGGL((rope_rows_kernel<true>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                           stream, x, rows, cols, half, positions, cos_tab, sin_tab);
    else
        hipLaunchKernelGGL((rope_rows_kernel<false>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                           stream, x, rows, cols, half, positions, cos_tab, sin_tab);
    return hipGetLastError();
}

hipError_t launch_rope_cache(const PoolLayer &pool, const uint16_t *q_in, uint32_t q_in_ld,
                             uint16_t *q_out, uint32_t q_out_ld, uint32_t group,
                             const uint16_t *keys, const uint16_t *values, uint32_t kv_ld,
                             const WritePlan &plan, const uint32_t *positions,
                             const float *cos_tab, const float *sin_tab, hipStream_t stream) {
    if (plan.num_segments == 0) return hipSuccess;
    if (!cache_write_supported(pool.head_dim, pool.block_size)) return hipErrorInvalidValue;
    const uint64_t items = static_cast<uint64_t>(plan.num_segments) * pool.kv_heads;
    const uint64_t grid = items;  // one workgroup per (run, KV head)
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
    KernelTimer timer("rope_cache", stream);
    // block 16 rows: head_dim 128 takes 4 rows per pass (4 wavefronts), 64 takes 8 (2)
    if (pool.head_dim == 128)
        hipLaunchKernelGGL((rope_cache_kernel<128>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                           stream, pool.k, pool.v, pool.kv_heads, q_in, q_in_ld, q_out, q_out_ld, group,
                           keys, values, kv_ld, plan.segments, positions, cos_tab, sin_tab,
                           static_cast<uint32_t>(items));
    else
        hipLaunchKernelGGL((rope_cache_kernel<64>), dim3(static_cast<uint32_t>(grid)), dim3(128), 0,
                           stream, pool.k, pool.v, pool.kv_heads, q_in, q_in_ld, q_out, q_out_ld, group,
                           keys, values, kv_ld, plan.segments, positions, cos_tab, sin_tab,
                           static_cast<uint32_t>(items));
    return hipGetLastError();
}

}  // namespace kernels
}  // namespace vo

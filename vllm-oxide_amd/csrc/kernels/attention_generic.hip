// attention_generic.hip -- paged GQA attention for any shape.
//
// Math (crates/engine/src/backend/cpu/attention.rs:5-16, :76-128), per query
// row t at position p and query head h:
//   kv_head = h / (heads / kv_heads)
//   s_j     = (q_h . K[slot(j), kv_head]) * scale,   j in 0..row_num_keys[t]
//   out_h   = sum_j softmax(s)_j * V[slot(j), kv_head]
// with scale = 1/sqrt(head_dim) in f32 (attention.rs:88).  A row with zero
// keys produces zeros, as the reference's empty loops do.
//
// This kernel is the fallback for shapes outside the MFMA kernels (any
// head_dim that is a multiple of 8, any block size, any GQA group).  It is
// written for clarity, not speed: one workgroup per (row, head), keys taken
// 256 at a time (one per thread for the score), an online softmax across
// chunks (exact in real arithmetic; the reference's two passes and this one
// differ only by rounding), and threads striding over head_dim for P.V.
// Bottleneck: K and V are re-read once per query head of a group.
#include <cmath>

#include "vo_device.hpp"
#include "vo_kernels.hpp"

namespace vo {
namespace kernels {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__global__ __launch_bounds__(kThreads) void attention_generic_kernel(
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool, PoolDims dims,
    const uint32_t *__restrict__ table_off, const uint32_t *__restrict__ tables,
    const uint32_t *__restrict__ row_seq, const uint32_t *__restrict__ row_num_keys,
    const uint16_t *__restrict__ q, uint16_t *__restrict__ out, uint32_t num_heads,
    float scale) {
    extern __shared__ float smem[];
    const uint32_t hd = dims.head_dim;
    float *q_s = smem;                     // [hd]
    float *acc_s = q_s + hd;               // [hd]
    float *p_s = acc_s + hd;               // [kThreads]
    uint32_t *slot_s = reinterpret_cast<uint32_t *>(p_s + kThreads);  // [kThreads]
    float *red_s = reinterpret_cast<float *>(slot_s + kThreads);      // [kWaves]

    const uint32_t row = blockIdx.x;
    const uint32_t head = blockIdx.y;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const uint32_t group = num_heads / dims.kv_heads;
    const uint32_t kvh = head / group;
    const uint32_t seq = row_seq[row];
    const uint32_t nk = row_num_keys[row];
    const uint32_t *table = tables + table_off[seq];
    const uint64_t row_base = static_cast<uint64_t>(row) * num_heads * hd + head * hd;

    for (uint32_t d = tid; d < hd; d += kThreads) {
        q_s[d] = bf16_bits_to_f32(q[row_base + d]);
        acc_s[d] = 0.0f;
    }
    __syncthreads();

    float m_run = -INFINITY;
    float l_run = 0.0f;
    for (uint32_t c0 = 0; c0 < nk; c0 += kThreads) {
        const uint32_t j = c0 + tid;
        const bool valid = j < nk;
        float s = -INFINITY;
        uint32_t slot = 0;
        if (valid) {
            const uint32_t block = table[j / dims.block_size];
            const uint32_t t = j % dims.block_size;
            slot = block * dims.block_size + t;
            const uint16_t *kp = k_pool + k_offset(dims, block, kvh, 0, 0);
            float dot = 0.0f;
            for (uint32_t d = 0; d < hd; ++d)
                dot += q_s[d] * bf16_bits_to_f32(kp[k_tile_offset(dims, t, d)]);
            s = dot * scale;
        }
        slot_s[tid] = slot;

        // Chunk max over the workgroup.
        float cm = wave_max(s);
        if (lane == 0) red_s[wave] = cm;
        __syncthreads();
        cm = red_s[0];
        for (int w = 1; w < kWaves; ++w) cm = fmaxf(cm, red_s[w]);
        __syncthreads();

        const float m_new = fmaxf(m_run, cm);
        const float alpha = (m_run == -INFINITY) ? 0.0f : expf(m_run - m_new);
        const float p = valid ? expf(s - m_new) : 0.0f;
        p_s[tid] = p;
        float cs = wave_sum(p);
        if (lane == 0) red_s[wave] = cs;
        __syncthreads();
        cs = 0.0f;
        for (int w = 0; w < kWaves; ++w) cs += red_s[w];
        l_run = l_run * alpha + cs;
        m_run = m_new;

        const uint32_t n = min(static_cast<uint32_t>(kThreads), nk - c0);
        for (uint32_t d = tid; d < hd; d += kThreads) {
            float a = acc_s[d] * alpha;
            for (uint32_t jj = 0; jj < n; ++jj) {
                const uint32_t sl = slot_s[jj];
                const uint32_t block = sl / dims.block_size;
                const uint32_t t = sl % dims.block_size;
                a += p_s[jj] * bf16_bits_to_f32(v_pool[v_offset(dims, block, kvh, t, d)]);
            }
            acc_s[d] = a;
        }
        __syncthreads();
    }

    const float inv = (nk > 0) ? 1.0f / l_run : 0.0f;
    for (uint32_t d = tid; d < hd; d += kThreads)
        out[row_base + d] = f32_to_bf16_bits(nk > 0 ? acc_s[d] * inv : 0.0f);
}

}  // namespace

hipError_t launch_attention_generic(const PoolLayer &pool, const MetaView &meta,
                                    const uint16_t *q, uint16_t *out, uint32_t num_heads,
                                    float scale, hipStream_t stream) {
    if (meta.num_rows == 0 || num_heads == 0) return hipSuccess;
    const PoolDims dims{pool.kv_heads, pool.head_dim, pool.block_size};
    const size_t smem = (2 * static_cast<size_t>(pool.head_dim) + 2 * kThreads + kWaves) * 4;
    if (smem > 64 * 1024) return hipErrorInvalidValue;
    KernelTimer timer("attention_generic", stream);
    hipLaunchKernelGGL(attention_generic_kernel, dim3(meta.num_rows, num_heads), dim3(kThreads),
                       smem, stream, pool.k, pool.v, dims, meta.table_off, meta.tables,
                       meta.row_seq, meta.row_num_keys, q, out, num_heads, scale);
    return hipGetLastError();
}

}  // namespace kernels
}  // namespace vo

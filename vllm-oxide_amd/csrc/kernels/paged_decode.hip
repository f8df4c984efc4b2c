// paged_decode.hip -- split-K paged decode attention on gfx950 MFMA, and the
// reduce kernel that merges the split-K partials.
//
// Math: crates/engine/src/backend/cpu/attention.rs:5-16 (one query row per
// sequence at decode, cpu/mod.rs:314-339).  For query row t, KV head k and
// the G = heads/kv_heads query heads h of k's group:
//   s[j,h] = (K[slot(j),k] . Q[t,kG+h]) * scale          j < row_num_keys[t]
//   out[t,kG+h] = sum_j softmax_j(s[.,h]) V[slot(j),k]
// computed as an online softmax in the exp2 domain (scores pre-multiplied by
// scale*log2 e), fp32 accumulation, bf16 I/O.
//
// Work split.  The keys of each row are cut into splits of `split_keys`
// (a multiple of 32).  Workgroup (item, k) owns one (row, split) for one KV
// head and all G heads of its group, so every K/V byte is read from HBM once:
// the algorithmic minimum.  Its W wavefronts take the split's 32-key chunks
// round robin and merge through LDS at the end.  A row with one split writes
// its bf16 output directly; otherwise the workgroup writes an fp32 partial
// (m, l, acc[head_dim]) per head and decode_reduce_kernel merges them.
//
// One 32-key chunk (two 16-key blocks b0, b1) of one wavefront:
//   Q.K^T: S^T[key, h] = K[key, :] . Q[h, :] with v_mfma_f32_16x16x32_bf16,
//          A = 16 keys x 32 dims of K (one 16-byte load per lane from the
//          key-major tile), B = Q^T with the G heads in columns 0..G-1 and
//          zeros elsewhere; head_dim/32 MFMAs per 16 keys, two key sets.
//          The A-row -> key assignment is chosen so that lane l ends up
//          holding the scores of head l%16 for keys 8*(l/16) .. +7 of the
//          chunk, in order.
//   softmax: per head, max over the lane's 8 keys and over the 4 lane groups
//          (two xor-shuffles); exp2; the running sum stays per lane and is
//          reduced once at the end.
//   P.V:   O^T[d, h] += V^T[d, key] . P^T[key, h] with 16x16x32 MFMAs:
//          A = 16 dims x 32 keys of V -- lane l reads the 8 keys 8*(l/16)..+7
//          of dim l%16, which are 16 contiguous bytes of the dim-major V tile
//          -- and B = P^T, which is exactly the lane's own 8 probabilities,
//          split into bf16 hi and lo parts (two MFMAs) so P keeps ~16 bits.
//          Output rows are dims, columns heads, so the softmax rescale of the
//          accumulator is lane-local.
// Per chunk and KV head a wavefront moves 16 KiB (hd 128) through 16 global
// loads of 16 bytes per lane and issues 24 MFMAs.
//
// Roofline: HBM.  Algorithmic bytes per row = keys * kv_heads * head_dim * 2 B
// * 2 (K and V) + q and out rows + block-table entries.  The MFMA work is
// <10% of gfx950's bf16 rate even with 12 of 16 head columns padding.
#include <cmath>

#include "vo_device.hpp"
#include "vo_kernels.hpp"

namespace vo {
namespace kernels {

namespace {

constexpr int kBS = 16;     // block size of the MFMA path
constexpr int kChunk = 32;  // keys per wavefront iteration

__device__ __forceinline__ floatx4 mfma16x16x32(bf16x8 a, bf16x8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t *p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}

template <int HD, int W>
__global__ __launch_bounds__(64 * W) void decode_splitk_kernel(
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool,
    uint32_t kv_heads, const uint32_t *__restrict__ table_off,
    const uint32_t *__restrict__ tables, const uint32_t *__restrict__ row_seq,
    const uint32_t *__restrict__ row_num_keys, const uint32_t *__restrict__ work,
    const uint32_t *__restrict__ row_part, uint32_t split_keys,
    const uint16_t *__restrict__ q, uint16_t *__restrict__ out, float *__restrict__ part_acc,
    float *__restrict__ part_ml, uint32_t num_heads, uint32_t group, float scale_log2) {
    constexpr int KK = HD / 32;  // QK MFMAs per 16 keys
    constexpr int DT = HD / 16;  // PV output tiles
    constexpr uint32_t kTile = kBS * HD;

    const uint32_t item = blockIdx.x;
    const uint32_t kvh = blockIdx.y;
    const uint32_t row = work[2 * item];
    const uint32_t split = work[2 * item + 1];
    const uint32_t seq = row_seq[row];
    const uint32_t nk = row_num_keys[row];
    const uint32_t *table = tables + table_off[seq];
    const uint32_t k_begin = split * split_keys;
    const uint32_t k_end = min(nk, k_begin + split_keys);
    const uint32_t nsplit = (nk + split_keys - 1) / split_keys;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane & 15;   // head column of this lane
    const int g = lane >> 4;   // lane group: keys 8g..8g+7 of a chunk
    const bool head_ok = h < static_cast<int>(group);
    const uint32_t qhead = kvh * group + h;

    // Q^T operand: column h, dims 32*kk + 8g .. +7.
    bf16x8 qv[KK];
    {
        const uint16_t *qp = q + (static_cast<uint64_t>(row) * num_heads + qhead) * HD + 8 * g;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            if (head_ok)
                qv[kk] = load_bf16x8(qp + 32 * kk);
            else
                qv[kk] = bf16x8{};
        }
    }

    // Q.K^T A-row assignment: row m = lane%16 reads block (m>>3) and key
    // 8*((m>>2)&1) + (m&3) (+4 for the second key set).  With the MFMA output
    // layout (lane l holds rows 4*(l/16)+i) this puts keys 8g+0..3 in the first
    // result and 8g+4..7 in the second.
    const int mrow = lane & 15;
    const int k_sel = mrow >> 3;
    const int k_t = 8 * ((mrow >> 2) & 1) + (mrow & 3);
    const int v_sel = g >> 1;
    const int v_t = 8 * (g & 1);

    float m_run = -INFINITY;
    float l_run = 0.0f;
    floatx4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

    const uint32_t nchunks = (k_end - k_begin + kChunk - 1) / kChunk;
    const uint64_t head_stride = static_cast<uint64_t>(kvh) * kTile;

    for (uint32_t c = wave; c < nchunks; c += W) {
        const uint32_t j0 = k_begin + c * kChunk;
        const uint32_t lb = j0 / kBS;
        const uint32_t phys0 = table[lb];
        const uint32_t phys1 = (j0 + kBS < k_end) ? table[lb + 1] : phys0;

        const uint32_t pk = k_sel ? phys1 : phys0;
        const uint16_t *kp = k_pool + static_cast<uint64_t>(pk) * kv_heads * kTile + head_stride +
                             k_t * HD + 8 * g;
        bf16x8 ka[KK], kb[KK];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            ka[kk] = load_bf16x8(kp + 32 * kk);
            kb[kk] = load_bf16x8(kp + 4 * HD + 32 * kk);
        }
        const uint32_t pv = v_sel ? phys1 : phys0;
        const uint16_t *vp = v_pool + static_cast<uint64_t>(pv) * kv_heads * kTile + head_stride +
                             mrow * kBS + v_t;
        bf16x8 va[DT];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) va[dt] = load_bf16x8(vp + dt * 16 * kBS);

        floatx4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            s0 = mfma16x16x32(ka[kk], qv[kk], s0);
            s1 = mfma16x16x32(kb[kk], qv[kk], s1);
        }

        // Scores of keys j0 + 8g + i, i = 0..7.
        const uint32_t jg = j0 + 8 * g;
        float sc[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sc[i] = (jg + i < k_end) ? s0[i] * scale_log2 : -INFINITY;
            sc[4 + i] = (jg + 4 + i < k_end) ? s1[i] * scale_log2 : -INFINITY;
        }
        float mt = sc[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) mt = fmaxf(mt, sc[i]);
        mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float m_new = fmaxf(m_run, mt);  // finite: the chunk has a valid key
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        // P goes to the MFMA as two bf16 parts, hi = bf16(p) and lo = bf16(p - hi),
        // so the probabilities keep ~16 significant bits instead of bf16's 8;
        // bf16 P alone exceeds rtol 1e-2 / atol 2e-3 on rows whose weight sits
        // on a few keys.
        float ps = 0.0f;
        bf16x8 pb_hi, pb_lo;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float p = __builtin_amdgcn_exp2f(sc[i] - m_new);
            ps += p;
            const __bf16 hi = static_cast<__bf16>(p);
            pb_hi[i] = hi;
            pb_lo[i] = static_cast<__bf16>(p - static_cast<float>(hi));
        }
        l_run = l_run * alpha + ps;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;

        if (j0 + kChunk > k_end) {
            // Tail chunk: keys past k_end have p = 0; zero their V as well so
            // that whatever the pool holds there cannot turn 0*x into NaN.
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    if (jg + i >= k_end) va[dt][i] = static_cast<__bf16>(0.0f);
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            acc[dt] = mfma16x16x32(va[dt], pb_lo, acc[dt]);
            acc[dt] = mfma16x16x32(va[dt], pb_hi, acc[dt]);
        }
    }

    // The running sums are per lane group; the max is already per head.
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);

    const uint64_t out_base = static_cast<uint64_t>(row) * num_heads * HD;

    if constexpr (W == 1) {
        if (!head_ok) return;
        if (nsplit == 1) {
            const float inv = 1.0f / l_run;
            uint16_t *op = out + out_base + static_cast<uint64_t>(qhead) * HD + 4 * g;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                u32x2 packed;
                packed[0] = f32_to_bf16_bits(acc[dt][0] * inv) |
                            (static_cast<uint32_t>(f32_to_bf16_bits(acc[dt][1] * inv)) << 16);
                packed[1] = f32_to_bf16_bits(acc[dt][2] * inv) |
                            (static_cast<uint32_t>(f32_to_bf16_bits(acc[dt][3] * inv)) << 16);
                *reinterpret_cast<u32x2 *>(op + 16 * dt) = packed;
            }
        } else {
            const uint64_t part = static_cast<uint64_t>(row_part[row] + split) * num_heads + qhead;
            float *ap = part_acc + part * HD + 4 * g;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<floatx4 *>(ap + 16 * dt) = acc[dt];
            if (g == 0) {
                part_ml[2 * part] = m_run;
                part_ml[2 * part + 1] = l_run;
            }
        }
    } else {
        // Merge the W wavefronts' (m, l, acc) through LDS.
        extern __shared__ float smem[];
        float *sm_m = smem;                  // [W][16]
        float *sm_l = sm_m + W * 16;         // [W][16]
        float *sm_acc = sm_l + W * 16;       // [W][group][HD]
        if (head_ok) {
            if (g == 0) {
                sm_m[wave * 16 + h] = m_run;
                sm_l[wave * 16 + h] = l_run;
            }
            float *ap = sm_acc + (static_cast<uint32_t>(wave) * group + h) * HD + 4 * g;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<floatx4 *>(ap + 16 * dt) = acc[dt];
        }
        __syncthreads();
        const uint32_t total = group * HD;
        for (uint32_t idx = threadIdx.x; idx < total; idx += 64 * W) {
            const uint32_t hh = idx / HD;
            const uint32_t d = idx % HD;
            float mx = -INFINITY;
#pragma unroll
            for (int w = 0; w < W; ++w) mx = fmaxf(mx, sm_m[w * 16 + hh]);
            float num = 0.0f, den = 0.0f;
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float mw = sm_m[w * 16 + hh];
                if (mw != -INFINITY) {
                    const float e = __builtin_amdgcn_exp2f(mw - mx);
                    num += e * sm_acc[(w * group + hh) * HD + d];
                    den += e * sm_l[w * 16 + hh];
                }
            }
            const uint32_t qh = kvh * group + hh;
            if (nsplit == 1) {
                out[out_base + static_cast<uint64_t>(qh) * HD + d] = f32_to_bf16_bits(num / den);
            } else {
                const uint64_t part = static_cast<uint64_t>(row_part[row] + split) * num_heads + qh;
                part_acc[part * HD + d] = num;
                if (d == 0) {
                    part_ml[2 * part] = mx;
                    part_ml[2 * part + 1] = den;
                }
            }
        }
    }
}

// Merge the split-K partials of one (row, head):
//   M = max_i m_i,  out = sum_i 2^(m_i - M) acc_i / sum_i 2^(m_i - M) l_i
// (log2 domain, matching the split kernel).  Rows with one split were
// written by the split kernel; rows with zero keys get zeros (the
// reference's empty softmax leaves the zero-filled output, attention.rs:119).
template <int HD>
__global__ __launch_bounds__(64) void decode_reduce_kernel(
    const uint32_t *__restrict__ row_num_keys, const uint32_t *__restrict__ row_part,
    uint32_t split_keys, const float *__restrict__ part_acc, const float *__restrict__ part_ml,
    uint16_t *__restrict__ out, uint32_t num_heads) {
    const uint32_t row = blockIdx.x;
    const uint32_t head = blockIdx.y;
    const uint32_t nk = row_num_keys[row];
    const uint32_t nsplit = (nk + split_keys - 1) / split_keys;
    if (nsplit == 1) return;
    uint16_t *op = out + (static_cast<uint64_t>(row) * num_heads + head) * HD;
    if (nsplit == 0) {
        for (uint32_t d = threadIdx.x; d < HD; d += 64) op[d] = 0;
        return;
    }
    const uint64_t p0 = static_cast<uint64_t>(row_part[row]) * num_heads + head;
    float mx = -INFINITY;
    for (uint32_t i = 0; i < nsplit; ++i) mx = fmaxf(mx, part_ml[2 * (p0 + i * num_heads)]);
    float den = 0.0f;
    float num[HD / 64];
#pragma unroll
    for (int r = 0; r < HD / 64; ++r) num[r] = 0.0f;
    for (uint32_t i = 0; i < nsplit; ++i) {
        const uint64_t p = p0 + static_cast<uint64_t>(i) * num_heads;
        const float e = __builtin_amdgcn_exp2f(part_ml[2 * p] - mx);
        den += e * part_ml[2 * p + 1];
#pragma unroll
        for (int r = 0; r < HD / 64; ++r) num[r] += e * part_acc[p * HD + threadIdx.x + 64 * r];
    }
    const float inv = 1.0f / den;
#pragma unroll
    for (int r = 0; r < HD / 64; ++r) op[threadIdx.x + 64 * r] = f32_to_bf16_bits(num[r] * inv);
}

template <int HD, int W>
hipError_t launch_split(const PoolLayer &pool, const MetaView &meta, const DecodePlan &plan,
                        const uint16_t *q, uint16_t *out, uint32_t num_heads, float scale_log2,
                        hipStream_t stream) {
    const uint32_t group = num_heads / pool.kv_heads;
    const size_t smem = (W == 1) ? 0 : (2 * W * 16 + static_cast<size_t>(W) * group * HD) * 4;
    KernelTimer timer("decode_splitk", stream);
    hipLaunchKernelGGL((decode_splitk_kernel<HD, W>), dim3(plan.num_work, pool.kv_heads),
                       dim3(64 * W), smem, stream, pool.k, pool.v, pool.kv_heads, meta.table_off,
                       meta.tables, meta.row_seq, meta.row_num_keys, plan.work, plan.row_part,
                       plan.split_keys, q, out, plan.part_acc, plan.part_ml, num_heads, group,
                       scale_log2);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const PoolLayer &pool, const MetaView &meta, const DecodePlan &plan,
                     const uint16_t *q, uint16_t *out, uint32_t num_heads, float scale_log2,
                     int waves, hipStream_t stream) {
    hipError_t err = hipSuccess;
    if (plan.num_work > 0) {
        switch (waves) {
            case 1: err = launch_split<HD, 1>(pool, meta, plan, q, out, num_heads, scale_log2, stream); break;
            case 2: err = launch_split<HD, 2>(pool, meta, plan, q, out, num_heads, scale_log2, stream); break;
            default: err = launch_split<HD, 4>(pool, meta, plan, q, out, num_heads, scale_log2, stream); break;
        }
        if (err != hipSuccess) return err;
    }
    if (!plan.needs_reduce) return hipSuccess;
    KernelTimer timer("decode_reduce", stream);
    hipLaunchKernelGGL((decode_reduce_kernel<HD>), dim3(meta.num_rows, num_heads), dim3(64), 0,
                       stream, meta.row_num_keys, plan.row_part, plan.split_keys, plan.part_acc,
                       plan.part_ml, out, num_heads);
    return hipGetLastError();
}

}  // namespace

bool decode_mfma_supported(uint32_t head_dim, uint32_t block_size, uint32_t group) {
    return (head_dim == 64 || head_dim == 128) && block_size == kBS && group >= 1 && group <= 16;
}

hipError_t launch_decode_mfma(const PoolLayer &pool, const MetaView &meta,
                              const DecodePlan &plan, const uint16_t *q, uint16_t *out,
                              uint32_t num_heads, float scale, int waves_per_group,
                              hipStream_t stream) {
    if (meta.num_rows == 0) return hipSuccess;
    const float scale_log2 = scale * 1.4426950408889634f;
    switch (pool.head_dim) {
        case 64: return launch_hd<64>(pool, meta, plan, q, out, num_heads, scale_log2, waves_per_group, stream);
        case 128: return launch_hd<128>(pool, meta, plan, q, out, num_heads, scale_log2, waves_per_group, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace kernels
}  // namespace vo

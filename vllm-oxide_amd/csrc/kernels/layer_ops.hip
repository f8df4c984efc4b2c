// layer_ops.hip -- the Llama layer's ops around attention (model.rs:269-356):
// embedding lookup, RMSNorm (alone or over the step's last rows), row gather,
// residual add, SwiGLU's silu(gate) * up, and greedy argmax.
//
// Numerics: the residual stream is f32 (as the reference's workspace);
// projections' inputs and outputs that feed a GEMM are bf16.  Every op
// computes in f32.  Reductions (RMSNorm's sum of squares, argmax) run as a
// tree over the 256 threads of a workgroup rather than the reference's
// 16-lane dot: the sum differs from the reference's in the last bits, the
// argmax result does not (ties resolve to the lowest index).
//
// Roofline: all HBM-bound.  Algorithmic bytes per row:
//   embed     2*hidden (table row) + 4*hidden (f32 out)
//   rmsnorm   4*hidden (x) + 2*hidden (out) (+ the weight, cache-resident)
//   gather    2 * row bytes (read, written)
//   add       4*cols (sum read) + 4*cols (written) + 2 or 4*cols (x)
//   silu_mul  2*2*cols (gate, up) + 2*cols (out)
//   argmax    4*cols (f32 logits) or 2*cols (bf16)
#include "vo_device.hpp"
#include "vo_kernels.hpp"

namespace vo {
namespace kernels {

namespace {

constexpr int kThreads = 256;
constexpr int kNormRegIt = 4;  // rmsnorm rows up to kThreads * 8 * 4 columns stay in registers

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum over the 256 threads of the workgroup; every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float *lds4) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) lds4[wave] = v;
    __syncthreads();
    const float t = (lds4[0] + lds4[1]) + (lds4[2] + lds4[3]);
    return t;
}

// 8 bf16 (one 16-byte word) -> 8 f32.
__device__ __forceinline__ void unpack8(const u32x4 w, float *f) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        f[2 * k] = __uint_as_float(w[k] << 16);
        f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
}

__device__ __forceinline__ u32x4 pack8(const float *f) {
    u32x4 w;
#pragma unroll
    for (int k = 0; k < 4; ++k)
        w[k] = static_cast<uint32_t>(f32_to_bf16_bits(f[2 * k])) |
               (static_cast<uint32_t>(f32_to_bf16_bits(f[2 * k + 1])) << 16);
    return w;
}

// Backend::embed (cpu/mod.rs:172-180): out[r] = table[tokens[r]], widened to
// f32 (exact).  One workgroup per row.  V8: 16-byte loads (hidden % 8 == 0).
template <bool V8>
__global__ __launch_bounds__(kThreads) void embed_kernel(const uint16_t *__restrict__ table,
                                                         uint32_t hidden,
                                                         const uint32_t *__restrict__ tokens,
                                                         float *__restrict__ out) {
    const uint32_t r = blockIdx.x;
    const uint16_t *src = table + static_cast<uint64_t>(tokens[r]) * hidden;
    float *dst = out + static_cast<uint64_t>(r) * hidden;
    if constexpr (V8) {
        for (uint32_t c = threadIdx.x * 8; c < hidden; c += kThreads * 8) {
            float f[8];
            unpack8(*reinterpret_cast<const u32x4 *>(src + c), f);
            *reinterpret_cast<floatx4 *>(dst + c) = floatx4{f[0], f[1], f[2], f[3]};
            *reinterpret_cast<floatx4 *>(dst + c + 4) = floatx4{f[4], f[5], f[6], f[7]};
        }
    } else {
        for (uint32_t c = threadIdx.x; c < hidden; c += kThreads) dst[c] = bf16_bits_to_f32(src[c]);
    }
}

// Backend::gather_rows (cpu/mod.rs:360-368): out row i = x row rows[i], a
// byte copy of row_words 4-byte words per row.  One workgroup per output
// row.  V4: 16-byte accesses (row_words % 4 == 0, both bases 16-byte aligned).
template <bool V4>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(const uint32_t *__restrict__ x,
                                                               uint32_t row_words,
                                                               const uint32_t *__restrict__ rows,
                                                               uint32_t *__restrict__ out) {
    const uint32_t i = blockIdx.x;
    const uint32_t *src = x + static_cast<uint64_t>(rows[i]) * row_words;
    uint32_t *dst = out + static_cast<uint64_t>(i) * row_words;
    if constexpr (V4) {
        for (uint32_t c = threadIdx.x * 4; c < row_words; c += kThreads * 4)
            *reinterpret_cast<u32x4 *>(dst + c) = *reinterpret_cast<const u32x4 *>(src + c);
    } else {
        for (uint32_t c = threadIdx.x; c < row_words; c += kThreads) dst[c] = src[c];
    }
}

// Backend::rmsnorm (cpu/mod.rs:182-197): out = w * (x * (1 / sqrt(mean(x^2)
// + eps))), the reference's (and HF's) order.  Row i of out normalises row
// rows_idx[i] of x (the LM head's gather_rows, model.rs:334-340), or row i
// when rows_idx is null.  One workgroup per output row; x is read once and
// held in registers for rows up to kThreads * 8 * kNormRegIt columns, longer
// rows are read twice, the second time from cache.
template <bool V8>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float *__restrict__ x,
                                                           uint32_t hidden,
                                                           const uint16_t *__restrict__ w,
                                                           float eps,
                                                           const uint32_t *__restrict__ rows_idx,
                                                           uint16_t *__restrict__ out) {
    __shared__ float lds4[4];
    const uint32_t i = blockIdx.x;
    const uint32_t r = rows_idx ? rows_idx[i] : i;
    const float *src = x + static_cast<uint64_t>(r) * hidden;
    uint16_t *dst = out + static_cast<uint64_t>(i) * hidden;
    float ss = 0.0f;
    if constexpr (V8) {
        if (hidden <= kThreads * 8 * kNormRegIt) {
            // The row stays in registers between the two passes, and the
            // weights load before the reduction; a thread's sum adds the same
            // terms in the same order as the loop below.  Columns past the
            // row load its last 8 (not used), so the loads need no branch.
            floatx4 a[kNormRegIt], b[kNormRegIt];
            u32x4 wv[kNormRegIt];
#pragma unroll
            for (int it = 0; it < kNormRegIt; ++it) {
                const uint32_t c = min(threadIdx.x * 8 + it * kThreads * 8, hidden - 8);
                a[it] = *reinterpret_cast<const floatx4 *>(src + c);
                b[it] = *reinterpret_cast<const floatx4 *>(src + c + 4);
                wv[it] = *reinterpret_cast<const u32x4 *>(w + c);
            }
#pragma unroll
            for (int it = 0; it < kNormRegIt; ++it) {
                if (threadIdx.x * 8 + it * kThreads * 8 < hidden) {
                    ss += a[it][0] * a[it][0] + a[it][1] * a[it][1] + a[it][2] * a[it][2] + a[it][3] * a[it][3];
                    ss += b[it][0] * b[it][0] + b[it][1] * b[it][1] + b[it][2] * b[it][2] + b[it][3] * b[it][3];
                }
            }
            const float mean_square = block_sum(ss, lds4) / static_cast<float>(hidden);
            const float inv_rms = 1.0f / sqrtf(mean_square + eps);
#pragma unroll
            for (int it = 0; it < kNormRegIt; ++it) {
                const uint32_t c = threadIdx.x * 8 + it * kThreads * 8;
                if (c < hidden) {
                    float wf[8], o[8];
                    unpack8(wv[it], wf);
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        o[k] = wf[k] * (a[it][k] * inv_rms);
                        o[4 + k] = wf[4 + k] * (b[it][k] * inv_rms);
                    }
                    *reinterpret_cast<u32x4 *>(dst + c) = pack8(o);
                }
            }
            return;
        }
        for (uint32_t c = threadIdx.x * 8; c < hidden; c += kThreads * 8) {
            const floatx4 a = *reinterpret_cast<const floatx4 *>(src + c);
            const floatx4 b = *reinterpret_cast<const floatx4 *>(src + c + 4);
            ss += a[0] * a[0] + a[1] * a[1] + a[2] * a[2] + a[3] * a[3];
            ss += b[0] * b[0] + b[1] * b[1] + b[2] * b[2] + b[3] * b[3];
        }
    } else {
        for (uint32_t c = threadIdx.x; c < hidden; c += kThreads) ss += src[c] * src[c];
    }
    const float mean_square = block_sum(ss, lds4) / static_cast<float>(hidden);
    const float inv_rms = 1.0f / sqrtf(mean_square + eps);
    if constexpr (V8) {
        for (uint32_t c = threadIdx.x * 8; c < hidden; c += kThreads * 8) {
            const floatx4 a = *reinterpret_cast<const floatx4 *>(src + c);
            const floatx4 b = *reinterpret_cast<const floatx4 *>(src + c + 4);
            float wf[8], o[8];
            unpack8(*reinterpret_cast<const u32x4 *>(w + c), wf);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                o[k] = wf[k] * (a[k] * inv_rms);
                o[4 + k] = wf[4 + k] * (b[k] * inv_rms);
            }
            *reinterpret_cast<u32x4 *>(dst + c) = pack8(o);
        }
    } else {
        for (uint32_t c = threadIdx.x; c < hidden; c += kThreads)
            dst[c] = f32_to_bf16_bits(bf16_bits_to_f32(w[c]) * (src[c] * inv_rms));
    }
}

// Backend::add (cpu/mod.rs:351-358): sum += x, x bf16 (widened) or f32.
template <bool XBF16>
__global__ __launch_bounds__(kThreads) void add_kernel(float *__restrict__ sum,
                                                       const void *__restrict__ x, uint64_t n) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) {
        const float v = XBF16 ? bf16_bits_to_f32(static_cast<const uint16_t *>(x)[i])
                              : static_cast<const float *>(x)[i];
        sum[i] += v;
    }
}

__device__ __forceinline__ float silu_mul1(float g, float u) {
    // silu(g) = g * sigmoid(g) = g / (1 + e^-g); times up (cpu/mod.rs:341-349).
    // e^-g = 2^(-g log2 e) on the hardware exp2 and the quotient through the
    // hardware reciprocal (about an ulp each): the f32 value is within ~2^-20
    // of the correctly rounded one, far inside the bf16 rounding of the
    // output, and the kernel stays bound by HBM rather than by an exact
    // exp and divide per element.  Infinities and NaN come out as the exact
    // form's: g = -inf gives -inf * 0 = NaN, as -inf / inf does.
    constexpr float kLog2e = 1.44269504088896341f;
    const float e = __builtin_amdgcn_exp2f(-g * kLog2e);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// Backend::silu_mul: out = silu(gate) * up, rows with their own strides;
// out may be gate itself (the reference's in-place form).  V8: 8 columns per
// thread with 16-byte accesses (cols and strides % 8 == 0).
template <bool V8>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const uint16_t *gate, uint32_t gate_ld,
                                                            const uint16_t *up, uint32_t up_ld,
                                                            uint32_t rows, uint32_t cols,
                                                            uint16_t *out, uint32_t out_ld) {
    constexpr uint32_t V = V8 ? 8 : 1;
    const uint32_t per_row = cols / V;
    const uint64_t n = static_cast<uint64_t>(rows) * per_row;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) {
        const uint32_t r = static_cast<uint32_t>(i / per_row);
        const uint32_t c = static_cast<uint32_t>(i % per_row) * V;
        const uint16_t *gp = gate + static_cast<uint64_t>(r) * gate_ld + c;
        const uint16_t *upp = up + static_cast<uint64_t>(r) * up_ld + c;
        uint16_t *op = out + static_cast<uint64_t>(r) * out_ld + c;
        if constexpr (V8) {
            float g[8], u[8], o[8];
            unpack8(*reinterpret_cast<const u32x4 *>(gp), g);
            unpack8(*reinterpret_cast<const u32x4 *>(upp), u);
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = silu_mul1(g[k], u[k]);
            *reinterpret_cast<u32x4 *>(op) = pack8(o);
        } else {
            *op = f32_to_bf16_bits(silu_mul1(bf16_bits_to_f32(*gp), bf16_bits_to_f32(*upp)));
        }
    }
}

// (value, index) of a running maximum; index 0xffffffff = no element yet.
struct ArgBest {
    float v;
    uint32_t i;
};

// `o` beats `b`: larger, or equal at a lower index -- the first maximum
// wins (cpu/mod.rs:370-388; torch's rule).
__device__ __forceinline__ bool beats(const ArgBest &o, const ArgBest &b) {
    return o.v > b.v || (o.v == b.v && o.i < b.i);
}

__device__ __forceinline__ float load_logit(const void *p, uint64_t k, bool f32) {
    return f32 ? static_cast<const float *>(p)[k]
               : bf16_bits_to_f32(static_cast<const uint16_t *>(p)[k]);
}

// Backend::argmax: ids[r] = first index of row r's maximum, or 0xffffffff
// when the row holds a NaN (EngineError::NaN, reported by the host).  One
// workgroup per row; each thread scans its columns in increasing order with
// a strict '>', then the (value, index) pairs merge by `beats`.  V4: f32
// rows read as 16-byte words (cols % 4 == 0).
template <bool F32, bool V4>
__global__ __launch_bounds__(kThreads) void argmax_kernel(const void *__restrict__ logits,
                                                          uint32_t cols,
                                                          uint32_t *__restrict__ ids) {
    __shared__ float lds_v[4];
    __shared__ uint32_t lds_i[4];
    __shared__ int lds_nan[4];
    const uint32_t r = blockIdx.x;
    const uint64_t base = static_cast<uint64_t>(r) * cols;
    ArgBest b{-__builtin_inff(), 0xffffffffu};
    bool nan = false;
    if constexpr (F32 && V4) {
        const floatx4 *row = reinterpret_cast<const floatx4 *>(static_cast<const float *>(logits) + base);
        for (uint32_t q = threadIdx.x; q < cols / 4; q += kThreads) {
            const floatx4 v = row[q];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                nan |= v[k] != v[k];
                const ArgBest o{v[k], 4 * q + k};
                if (b.i == 0xffffffffu || o.v > b.v) b = o;
            }
        }
    } else {
        for (uint32_t c = threadIdx.x; c < cols; c += kThreads) {
            const float v = load_logit(logits, base + c, F32);
            nan |= v != v;
            if (b.i == 0xffffffffu || v > b.v) b = ArgBest{v, c};
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const ArgBest x{__shfl_xor(b.v, o, 64), static_cast<uint32_t>(__shfl_xor(static_cast<int>(b.i), o, 64))};
        if (beats(x, b)) b = x;
    }
    const int any_nan = __any(nan) ? 1 : 0;
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        lds_v[wave] = b.v;
        lds_i[wave] = b.i;
        lds_nan[wave] = any_nan;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        ArgBest t{lds_v[0], lds_i[0]};
        int n = lds_nan[0];
        for (int k = 1; k < 4; ++k) {
            const ArgBest x{lds_v[k], lds_i[k]};
            if (beats(x, t)) t = x;
            n |= lds_nan[k];
        }
        ids[r] = n ? 0xffffffffu : t.i;
    }
}

// Backend::matmul for shapes the library GEMM does not take (rows of x or
// of the weight not a whole number of 16-byte words): out[r][o] = sum_k
// x[r][k] * w[o][k] in f32, k ascending, then out = acc (+ out when
// accumulating), stored as f32 or bf16.  One thread per output element;
// meant for the reference's tiny test shapes, not for throughput.
template <bool OUT_F32>
__global__ __launch_bounds__(kThreads) void matmul_generic_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ w, uint32_t rows, uint32_t n,
    uint32_t k, void *__restrict__ out, bool accumulate) {
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (idx >= static_cast<uint64_t>(rows) * n) return;
    const uint32_t r = static_cast<uint32_t>(idx / n), o = static_cast<uint32_t>(idx % n);
    const uint16_t *xr = x + static_cast<uint64_t>(r) * k;
    const uint16_t *wr = w + static_cast<uint64_t>(o) * k;
    float acc = 0.0f;
    for (uint32_t j = 0; j < k; ++j) acc += bf16_bits_to_f32(xr[j]) * bf16_bits_to_f32(wr[j]);
    if constexpr (OUT_F32) {
        float *d = static_cast<float *>(out) + idx;
        *d = accumulate ? *d + acc : acc;
    } else {
        uint16_t *d = static_cast<uint16_t *>(out) + idx;
        *d = f32_to_bf16_bits(accumulate ? bf16_bits_to_f32(*d) + acc : acc);
    }
}

// Backend::matmul for 1..4 rows (small decode batches): streaming the
// weight is the whole cost.  A workgroup owns 16 weight rows (outputs) and
// splits K over its 8 wavefronts; each wavefront runs
// v_mfma_f32_16x16x32_bf16 with A = 16 weight rows x 32 k (one non-temporal
// 16-byte load per lane) and B = x^T (the batch rows in columns 0..rows-1;
// columns past the batch repeat its last row and are not stored, so no lane
// branches), 8 steps of loads issued before their MFMAs.  The 8 partial
// tiles are summed through LDS in wavefront order, so an output depends
// only on its own row of x, whatever the batch size.  Beyond 4 rows the
// repeated x reads (every workgroup reads all of x) make hipBLASLt faster.
// MODE 0: bf16 out, 1: f32 out, 2: f32 out += .
constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyU = 8;     // 32-k steps per load batch
constexpr int kSkinnyRows = 4;  // largest batch the kernel is used for

template <int MODE>
__global__ __launch_bounds__(64 * kSkinnyWaves) void skinny_gemm_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ w, uint32_t rows, uint32_t n,
    uint32_t k, void *__restrict__ out) {
    constexpr int U = kSkinnyU;
    __shared__ floatx4 part[kSkinnyWaves][64];
    const uint32_t n0 = blockIdx.x * 16;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t kw = k / kSkinnyWaves;  // a multiple of 32 * U
    const uint32_t r = lane & 15, kg = lane >> 4;
    const uint16_t *wp = w + static_cast<uint64_t>(n0 + r) * k + wave * kw + 8 * kg;
    const bool live = r < rows;
    const uint16_t *xp = x + static_cast<uint64_t>(min(r, rows - 1)) * k + wave * kw + 8 * kg;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t kk = 0; kk < kw; kk += 32 * U) {
        u32x4 a[U], b[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            a[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wp + kk + 32 * u));
            b[u] = *reinterpret_cast<const u32x4 *>(xp + kk + 32 * u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[u]),
                                                          __builtin_bit_cast(bf16x8, b[u]), acc,
                                                          0, 0, 0);
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    floatx4 t = part[0][lane];
#pragma unroll
    for (int v = 1; v < kSkinnyWaves; ++v) t += part[v][lane];
    // Lane l holds outputs n0 + 4 (l / 16) + e, e = 0..3, of batch row l % 16.
    if (!live) return;
    const uint64_t o = static_cast<uint64_t>(r) * n + n0 + 4 * kg;
    if constexpr (MODE == 0) {
        u32x2 p;
        p[0] = static_cast<uint32_t>(f32_to_bf16_bits(t[0])) |
               (static_cast<uint32_t>(f32_to_bf16_bits(t[1])) << 16);
        p[1] = static_cast<uint32_t>(f32_to_bf16_bits(t[2])) |
               (static_cast<uint32_t>(f32_to_bf16_bits(t[3])) << 16);
        *reinterpret_cast<u32x2 *>(static_cast<uint16_t *>(out) + o) = p;
    } else {
        floatx4 *d = reinterpret_cast<floatx4 *>(static_cast<float *>(out) + o);
        if constexpr (MODE == 2) t += *d;
        *d = t;
    }
}

uint32_t grid_for(uint64_t items) {
    const uint64_t g = (items + kThreads - 1) / kThreads;
    return static_cast<uint32_t>(g < 65536 ? (g ? g : 1) : 65536);
}

}  // namespace

hipError_t launch_embed(const uint16_t *table, uint32_t hidden, const uint32_t *tokens,
                        uint32_t rows, float *out, hipStream_t stream) {
    if (rows == 0 || hidden == 0) return hipSuccess;
    KernelTimer timer("embed", stream);
    if (hidden % 8 == 0)
        hipLaunchKernelGGL((embed_kernel<true>), dim3(rows), dim3(kThreads), 0, stream, table, hidden,
                           tokens, out);
    else
        hipLaunchKernelGGL((embed_kernel<false>), dim3(rows), dim3(kThreads), 0, stream, table, hidden,
                           tokens, out);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, uint32_t hidden, const uint16_t *weight, float eps,
                          const uint32_t *rows_idx, uint32_t rows, uint16_t *out,
                          hipStream_t stream) {
    if (rows == 0 || hidden == 0) return hipSuccess;
    KernelTimer timer("rmsnorm", stream);
    if (hidden % 8 == 0)
        hipLaunchKernelGGL((rmsnorm_kernel<true>), dim3(rows), dim3(kThreads), 0, stream, x, hidden,
                           weight, eps, rows_idx, out);
    else
        hipLaunchKernelGGL((rmsnorm_kernel<false>), dim3(rows), dim3(kThreads), 0, stream, x, hidden,
                           weight, eps, rows_idx, out);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const void *x, uint32_t row_words, const uint32_t *rows,
                              uint32_t num_rows, void *out, bool vec4, hipStream_t stream) {
    if (num_rows == 0 || row_words == 0) return hipSuccess;
    KernelTimer timer("gather_rows", stream);
    const uint32_t *src = static_cast<const uint32_t *>(x);
    uint32_t *dst = static_cast<uint32_t *>(out);
    if (vec4)
        hipLaunchKernelGGL((gather_rows_kernel<true>), dim3(num_rows), dim3(kThreads), 0, stream, src,
                           row_words, rows, dst);
    else
        hipLaunchKernelGGL((gather_rows_kernel<false>), dim3(num_rows), dim3(kThreads), 0, stream,
                           src, row_words, rows, dst);
    return hipGetLastError();
}

hipError_t launch_add(float *sum, const void *x, bool x_bf16, uint64_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    KernelTimer timer("add", stream);
    const uint32_t grid = grid_for(n);
    if (x_bf16)
        hipLaunchKernelGGL((add_kernel<true>), dim3(grid), dim3(kThreads), 0, stream, sum, x, n);
    else
        hipLaunchKernelGGL((add_kernel<false>), dim3(grid), dim3(kThreads), 0, stream, sum, x, n);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const uint16_t *gate, uint32_t gate_ld, const uint16_t *up,
                           uint32_t up_ld, uint32_t rows, uint32_t cols, uint16_t *out,
                           uint32_t out_ld, bool vec8, hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    KernelTimer timer("silu_mul", stream);
    const uint64_t items = static_cast<uint64_t>(rows) * (vec8 ? cols / 8 : cols);
    const uint32_t grid = grid_for(items);
    if (vec8)
        hipLaunchKernelGGL((silu_mul_kernel<true>), dim3(grid), dim3(kThreads), 0, stream, gate,
                           gate_ld, up, up_ld, rows, cols, out, out_ld);
    else
        hipLaunchKernelGGL((silu_mul_kernel<false>), dim3(grid), dim3(kThreads), 0, stream, gate,
                           gate_ld, up, up_ld, rows, cols, out, out_ld);
    return hipGetLastError();
}

hipError_t launch_argmax(const void *logits, bool f32, uint32_t rows, uint32_t cols, uint32_t *ids,
                         hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    KernelTimer timer("argmax", stream);
    const bool v4 = f32 && cols % 4 == 0;
    if (f32 && v4)
        hipLaunchKernelGGL((argmax_kernel<true, true>), dim3(rows), dim3(kThreads), 0, stream, logits,
                           cols, ids);
    else if (f32)
        hipLaunchKernelGGL((argmax_kernel<true, false>), dim3(rows), dim3(kThreads), 0, stream,
                           logits, cols, ids);
    else
        hipLaunchKernelGGL((argmax_kernel<false, false>), dim3(rows), dim3(kThreads), 0, stream,
                           logits, cols, ids);
    return hipGetLastError();
}

}  // namespace kernels
}  // namespace vo

namespace vo {
namespace kernels {

hipError_t launch_matmul_generic(const uint16_t *x, const uint16_t *w, uint32_t rows, uint32_t n,
                                 uint32_t k, void *out, bool out_f32, bool accumulate,
                                 hipStream_t stream) {
    const uint64_t items = static_cast<uint64_t>(rows) * n;
    if (items == 0) return hipSuccess;
    const uint64_t grid = (items + kThreads - 1) / kThreads;
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
    KernelTimer timer("matmul_generic", stream);
    if (out_f32)
        hipLaunchKernelGGL((matmul_generic_kernel<true>), dim3(static_cast<uint32_t>(grid)),
                           dim3(kThreads), 0, stream, x, w, rows, n, k, out, accumulate);
    else
        hipLaunchKernelGGL((matmul_generic_kernel<false>), dim3(static_cast<uint32_t>(grid)),
                           dim3(kThreads), 0, stream, x, w, rows, n, k, out, accumulate);
    return hipGetLastError();
}

}  // namespace kernels
}  // namespace vo

namespace vo {
namespace kernels {

bool skinny_gemm_supported(uint64_t rows, uint64_t n, uint64_t k) {
    return rows >= 1 && rows <= kSkinnyRows && n % 16 == 0 &&
           k % (kSkinnyWaves * 32 * kSkinnyU) == 0 && n / 16 <= 0x7fffffffull;
}

hipError_t launch_skinny_gemm(const uint16_t *x, const uint16_t *w, uint32_t rows, uint32_t n,
                              uint32_t k, void *out, bool out_f32, bool accumulate,
                              hipStream_t stream) {
    if (!skinny_gemm_supported(rows, n, k)) return hipErrorInvalidValue;
    KernelTimer timer("matmul_skinny", stream);
    const dim3 grid(n / 16), block(64 * kSkinnyWaves);
    if (!out_f32)
        hipLaunchKernelGGL((skinny_gemm_kernel<0>), grid, block, 0, stream, x, w, rows, n, k, out);
    else if (!accumulate)
        hipLaunchKernelGGL((skinny_gemm_kernel<1>), grid, block, 0, stream, x, w, rows, n, k, out);
    else
        hipLaunchKernelGGL((skinny_gemm_kernel<2>), grid, block, 0, stream, x, w, rows, n, k, out);
    return hipGetLastError();
}

}  // namespace kernels
}  // namespace vo

// reshape_and_cache.hip -- write this step's K/V rows into their paged slots,
// and the debug gather that reads a sequence back through its block table.
//
// Math (Backend::write_kv, crates/engine/src/backend/mod.rs:107-119; CPU
// reference cpu/mod.rs:257-285):  pool.K[slot[t]] = keys[t],
// pool.V[slot[t]] = values[t], a bitwise copy of kv_heads*head_dim bf16 per
// row.  Slots were range-checked on the host before launch.
//
// cache_write_kernel (block size 16, head_dim 64/128) works from the step's
// write plan: runs of rows whose slots are consecutive inside one block.  A
// prefill chunk's whole blocks are written tile by tile with full-width
// stores, which matters because the V tile is dim-major (a key's values are
// 32 bytes apart).  reshape_and_cache_kernel covers every other shape: one
// thread per (row, kv_head, 8-dim chunk), 16-byte K stores and 2-byte V
// stores.  At decode (one row per sequence) either is launch-latency bound:
// 256 KiB per direction at a 64-row step.
#include "vo_device.hpp"
#include "vo_kernels.hpp"

namespace vo {
namespace kernels {

namespace {

__global__ void reshape_and_cache_kernel(uint16_t *__restrict__ k_pool,
                                         uint16_t *__restrict__ v_pool, PoolDims dims,
                                         const uint16_t *__restrict__ keys,
                                         const uint16_t *__restrict__ values,
                                         const uint32_t *__restrict__ slot_mapping,
                                         uint32_t rows) {
    const uint32_t chunks_per_head = dims.head_dim / 8;
    const uint32_t chunks_per_row = dims.kv_heads * chunks_per_head;
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<uint64_t>(rows) * chunks_per_row) return;
    const uint32_t row = static_cast<uint32_t>(idx / chunks_per_row);
    const uint32_t c = static_cast<uint32_t>(idx % chunks_per_row);
    const uint32_t kvh = c / chunks_per_head;
    const uint32_t d0 = (c % chunks_per_head) * 8;

    const uint32_t slot = slot_mapping[row];
    if (slot == kSkipSlot) return;
    const uint32_t block = slot / dims.block_size;
    const uint32_t t = slot % dims.block_size;

    const uint64_t src = static_cast<uint64_t>(row) * chunks_per_row * 8 + kvh * dims.head_dim + d0;
    const u32x4 kv = *reinterpret_cast<const u32x4 *>(keys + src);
    const u32x4 vv = *reinterpret_cast<const u32x4 *>(values + src);

    *reinterpret_cast<u32x4 *>(k_pool + k_offset(dims, block, kvh, t, d0)) = kv;

    uint16_t *vdst = v_pool + v_offset(dims, block, kvh, t, d0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        vdst[(2 * i) * dims.block_size] = static_cast<uint16_t>(vv[i] & 0xffffu);
        vdst[(2 * i + 1) * dims.block_size] = static_cast<uint16_t>(vv[i] >> 16);
    }
}

// One wavefront per (run of rows with consecutive slots in one block, KV
// head); four per workgroup.  Needs block size 16 and head_dim 64 or 128.
//   K: lane = (row, 16-byte unit); each store puts 8 dims of one key into the
//      key-major tile, and the 4 units of one (key, 32-dim chunk) are one
//      64-byte run.
//   V: lane = HD/64 consecutive dims; each row's values for the head are one
//      contiguous load across the wavefront.  A run that fills its block (16
//      rows from offset 0, every whole block of a prefill chunk) then writes
//      each dim's 16 keys as two 16-byte stores, so the wavefront writes the
//      4 KiB dim-major tile contiguously; shorter runs (chunk ends, decode
//      rows) write 2-byte elements.
template <int HD>
__global__ __launch_bounds__(256) void cache_write_kernel(
    uint16_t *__restrict__ k_pool, uint16_t *__restrict__ v_pool, uint32_t kv_heads,
    const uint16_t *__restrict__ keys, const uint16_t *__restrict__ values,
    const uint32_t *__restrict__ segments, uint32_t num_items) {
    constexpr uint32_t BS = 16;
    constexpr int DPL = HD / 64;            // V dims per lane
    constexpr uint32_t UPR = HD / 8;        // 16-byte K units per row
    constexpr uint32_t RPI = 64 / UPR;      // K rows per load instruction
    const uint32_t item = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= num_items) return;  // whole wavefront
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t seg = item / kv_heads;
    const uint32_t kvh = item % kv_heads;
    const uint32_t row0 = segments[3 * seg];
    const uint32_t n = segments[3 * seg + 1];  // 1 .. BS
    const uint32_t slot0 = segments[3 * seg + 2];
    if (slot0 == kSkipSlot) return;  // a superseded row: nothing to cache
    const uint32_t off0 = slot0 % BS;
    const uint64_t width = static_cast<uint64_t>(kv_heads) * HD;
    const uint64_t tile = (static_cast<uint64_t>(slot0 / BS) * kv_heads + kvh) * (BS * HD);

    // Every load of the run is issued before the first store.
    const uint32_t u = lane % UPR;
    const uint32_t d = 8 * u;
    const uint32_t i0 = lane / UPR;
    constexpr uint32_t KI = BS / RPI;  // K load instructions for a whole block
    u32x4 kreg[KI];
#pragma unroll
    for (uint32_t j = 0; j < KI; ++j) {
        const uint32_t i = i0 + RPI * j;
        if (i < n) kreg[j] = *reinterpret_cast<const u32x4 *>(keys + (row0 + i) * width + kvh * HD + d);
    }

    uint16_t vv[DPL][BS];
    const uint16_t *vsrc = values + static_cast<uint64_t>(row0) * width + kvh * HD + DPL * lane;
#pragma unroll
    for (uint32_t i = 0; i < BS; ++i) {
        if (i < n) {
            if constexpr (DPL == 2) {
                const uint32_t w = *reinterpret_cast<const uint32_t *>(vsrc + i * width);
                vv[0][i] = static_cast<uint16_t>(w & 0xffffu);
                vv[1][i] = static_cast<uint16_t>(w >> 16);
            } else {
                vv[0][i] = vsrc[i * width];
            }
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < KI; ++j) {
        const uint32_t i = i0 + RPI * j;
        if (i < n)
            *reinterpret_cast<u32x4 *>(k_pool + tile + (d / 32) * (BS * 32) + (off0 + i) * 32 + d % 32) =
                kreg[j];
    }
    uint16_t *vdst = v_pool + tile + static_cast<uint64_t>(DPL * lane) * BS;
    if (n == BS) {  // off0 == 0: the run is the whole block
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
            u32x4 lo, hi;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                lo[p] = static_cast<uint32_t>(vv[e][2 * p]) | (static_cast<uint32_t>(vv[e][2 * p + 1]) << 16);
                hi[p] = static_cast<uint32_t>(vv[e][8 + 2 * p]) |
                        (static_cast<uint32_t>(vv[e][8 + 2 * p + 1]) << 16);
            }
            *reinterpret_cast<u32x4 *>(vdst + e * BS) = lo;
            *reinterpret_cast<u32x4 *>(vdst + e * BS + 8) = hi;
        }
    } else {
#pragma unroll
        for (uint32_t i = 0; i < BS; ++i) {
            if (i < n) {
#pragma unroll
                for (int e = 0; e < DPL; ++e) vdst[e * BS + off0 + i] = vv[e][i];
            }
        }
    }
}

// Block copies of every layer (the block manager's copy on write): workgroup
// (pair, layer, K|V) copies one block's tiles of all KV heads, which are
// contiguous in each layer's region, with 16-byte loads and stores.
__global__ __launch_bounds__(256) void copy_blocks_kernel(uint16_t *__restrict__ base,
                                                          uint64_t layer_elems,
                                                          uint64_t block_elems,
                                                          BlockPairs pairs) {
    const uint32_t pair = blockIdx.x;
    const uint32_t layer = blockIdx.y >> 1;
    const uint32_t which = blockIdx.y & 1;  // 0 = K, 1 = V
    uint16_t *region = base + (static_cast<uint64_t>(layer) * 2 + which) * layer_elems;
    const u32x4 *src = reinterpret_cast<const u32x4 *>(region + pairs.src[pair] * block_elems);
    u32x4 *dst = reinterpret_cast<u32x4 *>(region + pairs.dst[pair] * block_elems);
    const uint64_t n = block_elems / 8;
    for (uint64_t i = threadIdx.x; i < n; i += 256) dst[i] = src[i];
}

__global__ void gather_kv_kernel(const uint16_t *__restrict__ k_pool,
                                 const uint16_t *__restrict__ v_pool, PoolDims dims,
                                 const uint32_t *__restrict__ table, uint32_t num_keys,
                                 uint16_t *__restrict__ out_k, uint16_t *__restrict__ out_v) {
    const uint32_t chunks_per_head = dims.head_dim / 8;
    const uint32_t chunks_per_row = dims.kv_heads * chunks_per_head;
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<uint64_t>(num_keys) * chunks_per_row) return;
    const uint32_t j = static_cast<uint32_t>(idx / chunks_per_row);
    const uint32_t c = static_cast<uint32_t>(idx % chunks_per_row);
    const uint32_t kvh = c / chunks_per_head;
    const uint32_t d0 = (c % chunks_per_head) * 8;

    // slot_of (paged.rs:48-52), split back into (block, offset).
    const uint32_t block = table[j / dims.block_size];
    const uint32_t t = j % dims.block_size;

    const uint64_t dst = static_cast<uint64_t>(j) * chunks_per_row * 8 + kvh * dims.head_dim + d0;
    *reinterpret_cast<u32x4 *>(out_k + dst) =
        *reinterpret_cast<const u32x4 *>(k_pool + k_offset(dims, block, kvh, t, d0));

    const uint16_t *vsrc = v_pool + v_offset(dims, block, kvh, t, d0);
    u32x4 vv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        vv[i] = static_cast<uint32_t>(vsrc[(2 * i) * dims.block_size]) |
                (static_cast<uint32_t>(vsrc[(2 * i + 1) * dims.block_size]) << 16);
    }
    *reinterpret_cast<u32x4 *>(out_v + dst) = vv;
}

}  // namespace

hipError_t launch_reshape_and_cache(const PoolLayer &pool, const uint16_t *keys,
                                    const uint16_t *values, const uint32_t *slot_mapping,
                                    uint32_t rows, hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    const PoolDims dims{pool.kv_heads, pool.head_dim, pool.block_size};
    const uint64_t threads = static_cast<uint64_t>(rows) * pool.kv_heads * (pool.head_dim / 8);
    const uint32_t block = 256;
    const uint64_t grid = (threads + block - 1) / block;
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
    KernelTimer timer("reshape_and_cache", stream);
    hipLaunchKernelGGL(reshape_and_cache_kernel, dim3(static_cast<uint32_t>(grid)), dim3(block),
                       0, stream, pool.k, pool.v, dims, keys, values, slot_mapping, rows);
    return hipGetLastError();
}

bool cache_write_supported(uint32_t head_dim, uint32_t block_size) {
    return block_size == 16 && (head_dim == 64 || head_dim == 128);
}

hipError_t launch_cache_write(const PoolLayer &pool, const uint16_t *keys, const uint16_t *values,
                              const WritePlan &plan, hipStream_t stream) {
    if (plan.num_segments == 0) return hipSuccess;
    if (!cache_write_supported(pool.head_dim, pool.block_size)) return hipErrorInvalidValue;
    const uint64_t items = static_cast<uint64_t>(plan.num_segments) * pool.kv_heads;
    const uint64_t grid = (items + 3) / 4;
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
    KernelTimer timer("reshape_and_cache", stream);
    if (pool.head_dim == 128)
        hipLaunchKernelGGL((cache_write_kernel<128>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                           stream, pool.k, pool.v, pool.kv_heads, keys, values, plan.segments,
                           static_cast<uint32_t>(items));
    else
        hipLaunchKernelGGL((cache_write_kernel<64>), dim3(static_cast<uint32_t>(grid)), dim3(256), 0,
                           stream, pool.k, pool.v, pool.kv_heads, keys, values, plan.segments,
                           static_cast<uint32_t>(items));
    return hipGetLastError();
}

hipError_t launch_copy_blocks(uint16_t *base, uint64_t num_layers, uint64_t layer_elems,
                              uint64_t block_elems, const BlockPairs &pairs, uint32_t count,
                              hipStream_t stream) {
    if (count == 0) return hipSuccess;
    if (count > kMaxBlockPairs || block_elems % 8 != 0 || num_layers * 2 > 65535)
        return hipErrorInvalidValue;
    KernelTimer timer("copy_blocks", stream);
    hipLaunchKernelGGL(copy_blocks_kernel, dim3(count, static_cast<uint32_t>(num_layers * 2)),
                       dim3(256), 0, stream, base, layer_elems, block_elems, pairs);
    return hipGetLastError();
}

hipError_t launch_gather_kv(const PoolLayer &pool, const uint32_t *table, uint32_t num_keys,
                            uint16_t *out_k, uint16_t *out_v, hipStream_t stream) {
    if (num_keys == 0) return hipSuccess;
    const PoolDims dims{pool.kv_heads, pool.head_dim, pool.block_size};
    const uint64_t threads = static_cast<uint64_t>(num_keys) * pool.kv_heads * (pool.head_dim / 8);
    const uint32_t block = 256;
    const uint64_t grid = (threads + block - 1) / block;
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
    KernelTimer timer("gather_kv", stream);
    hipLaunchKernelGGL(gather_kv_kernel, dim3(static_cast<uint32_t>(grid)), dim3(block), 0,
                       stream, pool.k, pool.v, dims, table, num_keys, out_k, out_v);
    return hipGetLastError();
}

}  // namespace kernels
}  // namespace vo

// reshape_and_cache.hip -- write this step's K/V rows into their paged slots,
// and the debug gather that reads a sequence back through its block table.
//
// Math (Backend::write_kv, crates/engine/src/backend/mod.rs:107-119; CPU
// reference cpu/mod.rs:257-285):  pool.K[slot[t]] = keys[t],
// pool.V[slot[t]] = values[t], a bitwise copy of kv_heads*head_dim bf16 per
// row.  Slots were range-checked on the host before launch.
//
// Launch: one thread per (row, kv_head, 8-dim chunk).  Each thread does one
// 16-byte load of K and of V.  K goes out as one 16-byte store (a key's dims
// are contiguous in the key-major tile); V goes out as 8 two-byte stores at a
// stride of block_size (the dim-major tile).  The op moves 2*rows*kv_heads*
// head_dim*2 bytes each way: 256 KiB per direction at a 64-row decode step,
// so at decode it is launch-latency bound, not bandwidth bound.
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

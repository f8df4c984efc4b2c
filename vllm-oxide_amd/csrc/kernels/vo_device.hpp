// vo_device.hpp -- device-side types and the physical KV-pool layout.
//
// Pool layout (backend-private; the reference leaves the bytes to the
// backend, crates/engine/src/backend/mod.rs:10-12).  Per layer:
//
//   K: [num_blocks][kv_heads][head_dim/CW][block_size][CW]  bf16  ("key-major tile")
//   V: [num_blocks][kv_heads][head_dim][block_size]         bf16  ("dim-major tile")
//
// with CW = 32 dims when head_dim is a multiple of 32, else 8.  One
// (block, kv_head) tile is block_size*head_dim*2 bytes contiguous for K and
// for V (4 KiB at bs 16, hd 128).  K keeps 32 consecutive dims of a key
// together (64 bytes), the row operand of one Q.K^T MFMA step, and puts the
// block's keys for the same 32 dims next to each other, so one load
// instruction of the decode kernel reads whole 128-byte lines; V keeps a
// dim's block_size keys together, the row operand of the V^T.P MFMA.  The
// logical slot semantics are the reference's: slot = block*bs + offset
// (crates/engine/src/backend/paged.rs:25-28).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vo {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Widening bf16 -> f32 is exact: the bf16 bits are the top half of the f32.
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even f32 -> bf16 (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

struct PoolDims {
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t block_size;
};

// Dims per K chunk (see the layout above).
__host__ __device__ __forceinline__ uint32_t k_chunk_dims(uint32_t head_dim) {
    return (head_dim % 32 == 0) ? 32u : 8u;
}

// Element offset of key t, dim d inside one K tile.  Eight consecutive dims
// starting at a multiple of 8 are contiguous.
__device__ __forceinline__ uint32_t k_tile_offset(const PoolDims &p, uint32_t t, uint32_t d) {
    const uint32_t cw = k_chunk_dims(p.head_dim);
    return (d / cw) * (p.block_size * cw) + t * cw + d % cw;
}

// Element offset of K[block][kvh][key t][dim d] within one layer's K region.
__device__ __forceinline__ uint64_t k_offset(const PoolDims &p, uint32_t block, uint32_t kvh,
                                             uint32_t t, uint32_t d) {
    return (static_cast<uint64_t>(block) * p.kv_heads + kvh) * (p.block_size * p.head_dim) +
           k_tile_offset(p, t, d);
}

// Element offset of V[block][kvh][d][t] within one layer's V region.
__device__ __forceinline__ uint64_t v_offset(const PoolDims &p, uint32_t block, uint32_t kvh,
                                             uint32_t t, uint32_t d) {
    return (static_cast<uint64_t>(block) * p.kv_heads + kvh) * (p.block_size * p.head_dim) +
           static_cast<uint64_t>(d) * p.block_size + t;
}

// Word 3 of a raw buffer resource on gfx950 (32-bit data format, no swizzle).
constexpr uint32_t kBufferRsrcWord3 = 0x00020000u;

// LDS DMA of 16 bytes per lane: bytes [voff, voff + 16) of the buffer at base
// (wave-uniform, `bytes` long) to lds + 16 * lane.  The MUBUF form is used
// rather than global_load_lds: the compiler counts a pending FLAT-encoded LDS
// DMA against the LDS counter too and then waits for every outstanding LDS
// read (lgkmcnt(0)) wherever it needs one, while a MUBUF DMA counts only in
// vmcnt and the ds_read waits stay partial.
__device__ __forceinline__ void dma16(const void *base, uint32_t bytes, void *lds, uint32_t voff) {
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, kBufferRsrcWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)lds,
                                             16, voff, 0, 0, 0);
}

// A raw buffer resource over `bytes` bytes from base (wave-uniform).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, kBufferRsrcWord3);
}

// LDS DMA of 16 bytes per lane from bytes [soff + voff, soff + voff + 16) of
// the buffer rsrc to lds + 16 * lane; soff is wave-uniform (the scalar
// offset of the instruction), voff per lane.
__device__ __forceinline__ void dma16_at(__amdgpu_buffer_rsrc_t rsrc, void *lds, uint32_t voff,
                                         uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)lds,
                                             16, voff, soff, 0, 0);
}

__device__ __forceinline__ uint32_t uniform_u32(uint32_t x) {
    return __builtin_amdgcn_readfirstlane(x);
}

// s_waitcnt vmcnt(N) lgkmcnt(0), then a workgroup barrier.
template <int N>
__device__ __forceinline__ void wait_barrier() {
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace vo

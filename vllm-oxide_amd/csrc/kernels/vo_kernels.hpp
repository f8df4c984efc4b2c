// vo_kernels.hpp -- host-side launchers of the gfx950 kernels.
//
// Callers (vo_backend.cpp) validate every input on the host first; the
// launchers assume in-bounds metadata and only check launch-shape limits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vo {
namespace kernels {

// Brackets one kernel launch with HIP events on `stream` when profiling is
// enabled (vo_profiling_enable); a no-op otherwise.  Declare it in the scope
// of the launch; the stop event is recorded when it goes out of scope.
class KernelTimer {
   public:
    KernelTimer(const char *name, hipStream_t stream);
    ~KernelTimer();
    KernelTimer(const KernelTimer &) = delete;
    KernelTimer &operator=(const KernelTimer &) = delete;

   private:
    const char *name_;
    hipStream_t stream_;
    hipEvent_t start_ = nullptr;
};

// One layer of the pool: K and V regions plus the dims that index them.
struct PoolLayer {
    uint16_t *k;
    uint16_t *v;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t block_size;
    uint64_t elems = 0;  // elements of the layer's K (and of its V)
};

// Device metadata of one step (all u32, device pointers).
struct MetaView {
    const uint32_t *table_off;     // [S+1]
    const uint32_t *tables;        // [entries]
    const uint32_t *row_seq;       // [T]
    const uint32_t *row_num_keys;  // [T]
    const uint32_t *slot_mapping;  // [T]
    const uint32_t *positions;     // [T] (RoPE); null for a slots-only upload
    uint32_t num_rows;
    uint32_t num_seqs;
};

// Write plan of one step's write_kv: runs of rows whose slots are
// consecutive inside one block (rows never cross a block boundary).
struct WritePlan {
    const uint32_t *segments;  // [num_segments][3]: (first row, rows, first slot)
    uint32_t num_segments;
};

// True when the block-run cache writer covers this shape.
bool cache_write_supported(uint32_t head_dim, uint32_t block_size);

// reshape_and_cache over a write plan: one wavefront per (run, KV head); K
// goes out in 16-byte stores, V is transposed in registers so that a whole
// block writes each dim's keys as one 32-byte run.
hipError_t launch_cache_write(const PoolLayer &pool, const uint16_t *keys, const uint16_t *values,
                              const WritePlan &plan, hipStream_t stream);

// RoPE (rope.rs:86-100) in place on x [rows, cols] bf16, heads of width
// 2*half, row r at positions[r]; cos/sin [max_len][half] f32.
hipError_t launch_rope_rows(uint16_t *x, uint32_t rows, uint32_t cols, uint32_t half,
                            const uint32_t *positions, const float *cos_tab, const float *sin_tab,
                            hipStream_t stream);

// rope(q) (q_in -> q_out, which may be the same rows) + rope(k) and v into
// the pool over the write plan.  Row strides in elements: q_in_ld, q_out_ld,
// kv_ld (keys and values).
hipError_t launch_rope_cache(const PoolLayer &pool, const uint16_t *q_in, uint32_t q_in_ld,
                             uint16_t *q_out, uint32_t q_out_ld, uint32_t group,
                             const uint16_t *keys, const uint16_t *values, uint32_t kv_ld,
                             const WritePlan &plan, const uint32_t *positions,
                             const float *cos_tab, const float *sin_tab, hipStream_t stream);

// reshape_and_cache: pool[slot_mapping[t]] = keys[t], values[t].
// keys/values: [rows, kv_heads*head_dim] bf16.  Rows whose slot is
// kSkipSlot (0xffffffff) are superseded by a later row and not written.
constexpr uint32_t kSkipSlot = 0xffffffffu;
hipError_t launch_reshape_and_cache(const PoolLayer &pool, const uint16_t *keys,
                                    const uint16_t *values, const uint32_t *slot_mapping,
                                    uint32_t rows, hipStream_t stream);

// Up to kMaxBlockPairs (src, dst) block pairs, passed by value.
constexpr uint32_t kMaxBlockPairs = 128;
struct BlockPairs {
    uint32_t src[kMaxBlockPairs];
    uint32_t dst[kMaxBlockPairs];
};

// dst[i] := src[i] for whole blocks of every layer's K and V.  base is the
// pool's [layers][K|V][layer_elems]; block_elems = kv_heads*block_size*head_dim.
hipError_t launch_copy_blocks(uint16_t *base, uint64_t num_layers, uint64_t layer_elems,
                              uint64_t block_elems, const BlockPairs &pairs, uint32_t count,
                              hipStream_t stream);

// Gather keys 0..num_keys of one sequence, whose block table is the device
// array `table`, into [num_keys, kv_heads*head_dim] (the reference's layout).
hipError_t launch_gather_kv(const PoolLayer &pool, const uint32_t *table, uint32_t num_keys,
                            uint16_t *out_k, uint16_t *out_v, hipStream_t stream);

// Generic paged attention for any shape: one workgroup per (row, head),
// online softmax over 256-key chunks, fp32 accumulation.
hipError_t launch_attention_generic(const PoolLayer &pool, const MetaView &meta,
                                    const uint16_t *q, uint16_t *out, uint32_t num_heads,
                                    float scale, hipStream_t stream);

// PrefillMeta::new / DecodeMeta::new on the device (paged.rs:117-143,
// 189-209): per-row positions, slots, sequences and key counts from the
// per-sequence row starts, context lengths and CSR block tables (all device
// u32 arrays).  Uncovered positions get slot 0xffffffff and set *errors = 1.
hipError_t launch_build_rows(const uint32_t *seq_row_starts, const uint32_t *context_lens,
                             const uint32_t *table_off, const uint32_t *tables, uint32_t num_seqs,
                             uint32_t num_rows, uint32_t block_size, uint32_t *positions,
                             uint32_t *slot_mapping, uint32_t *row_seq, uint32_t *row_num_keys,
                             uint32_t *errors, hipStream_t stream);

// The layer's ops around attention (layer_ops.hip).  rows_idx (device, may
// be null) selects the rows of x that rmsnorm normalises.
hipError_t launch_embed(const uint16_t *table, uint32_t hidden, const uint32_t *tokens,
                        uint32_t rows, float *out, hipStream_t stream);
hipError_t launch_rmsnorm(const float *x, uint32_t hidden, const uint16_t *weight, float eps,
                          const uint32_t *rows_idx, uint32_t rows, uint16_t *out,
                          hipStream_t stream);
// out row i = x row rows[i], rows of row_words 4-byte words (device rows[]).
hipError_t launch_gather_rows(const void *x, uint32_t row_words, const uint32_t *rows,
                              uint32_t num_rows, void *out, bool vec4, hipStream_t stream);
hipError_t launch_add(float *sum, const void *x, bool x_bf16, uint64_t n, hipStream_t stream);
hipError_t launch_silu_mul(const uint16_t *gate, uint32_t gate_ld, const uint16_t *up,
                           uint32_t up_ld, uint32_t rows, uint32_t cols, uint16_t *out,
                           uint32_t out_ld, bool vec8, hipStream_t stream);
hipError_t launch_argmax(const void *logits, bool f32, uint32_t rows, uint32_t cols, uint32_t *ids,
                         hipStream_t stream);
// Weight-streaming GEMM for 1..4 rows (small decode batches): n % 16 == 0,
// k % 2048 == 0.
bool skinny_gemm_supported(uint64_t rows, uint64_t n, uint64_t k);
hipError_t launch_skinny_gemm(const uint16_t *x, const uint16_t *w, uint32_t rows, uint32_t n,
                              uint32_t k, void *out, bool out_f32, bool accumulate,
                              hipStream_t stream);
hipError_t launch_matmul_generic(const uint16_t *x, const uint16_t *w, uint32_t rows, uint32_t n,
                                 uint32_t k, void *out, bool out_f32, bool accumulate,
                                 hipStream_t stream);

// Largest split the decode kernel takes (its block-table slice lives in LDS).
constexpr uint32_t kMaxSplitKeys = 4096;

// Split-K work plan for the MFMA decode kernel.
struct DecodePlan {
    const uint32_t *work;         // [num_work][4]: (row, split, index of the split's first
                                  // block id in `tables`, the row's keys); 16-byte aligned,
                                  // launch_work records readable; a zero-key row has one item
    const uint32_t *row_info;     // [T][2]: (first partial index, number of splits); (0, 0) for
                                  // rows the plan does not cover
    const uint32_t *reduce_rows;  // [num_reduce_rows]: rows with more than one split
    uint32_t num_work;
    uint32_t num_reduce_rows;
    uint32_t split_keys;          // keys per split, a multiple of 32, <= kMaxSplitKeys
    float *part_acc;              // [parts][num_heads][head_dim]
    float *part_ml;               // [parts][num_heads][2]: (max, sum), log2 domain
    bool streaming;               // no KV block is read by two rows: non-temporal K/V loads
    const uint32_t *counts;       // device [2]: num_work, num_reduce_rows; the kernels stop there
    uint32_t launch_work;         // work items launched (>= num_work; = num_work unless fixed)
    uint32_t launch_reduce;       // reduce rows launched (>= num_reduce_rows)
    // Row packing: item i also serves the rows mates[(pack-1)*i .. +pack-2]
    // (kNoMate where its pack is short), rows whose split reads the same
    // blocks; the pack * group head columns fit one 16-column MFMA tile, or
    // two (the kernel then runs both tiles on every item).
    // pack == 1: no mates (mates may be null).
    const uint32_t *mates;
    uint32_t pack;
    // Items 0 .. num_shared - 1 are shared packs (mates over one full split):
    // the workgroup stages each chunk in LDS once and its W wavefronts take
    // 16 / group rows each, so pack <= W * (16 / group); every other item
    // then has no mates.  0: no shared packs.
    uint32_t num_shared;
    // Shared packs in wavefront pairs: two wavefronts per 16-column tile,
    // each keeping two of the tile's four softmax states, so pack <= W / 2 *
    // (16 / group) and each wavefront walks half of the split's chunks.
    bool shared_pairs;
};

constexpr uint32_t kNoMate = 0xffffffffu;


// True when the MFMA decode kernel covers this shape.
bool decode_mfma_supported(uint32_t head_dim, uint32_t block_size, uint32_t group);

// MFMA split-K decode (one launch) and, when a row has several splits, the
// reduce kernel (a second launch).
// The step's new keys, for a decode launch that also caches them (the
// write_kv before decode_attention, in the same launch): the item holding a
// row's last key writes row r of k and v ([rows][kv_heads * head_dim] bf16)
// to the pool at slots[r] and takes that key's K/V from k and v instead of
// the pool.  The caller guarantees that no slot repeats and that no other
// row of the step reads a block these slots are in (so a packed item, whose
// blocks several rows read, holds no row's last key).
struct NewKeys {
    const uint16_t *k;
    const uint16_t *v;
    const uint32_t *slots;  // [rows]
};

hipError_t launch_decode_mfma(const PoolLayer &pool, const MetaView &meta,
                              const DecodePlan &plan, const uint16_t *q, uint16_t *out,
                              uint32_t num_heads, float scale, int waves_per_group,
                              hipStream_t stream, const NewKeys *new_keys = nullptr);

constexpr uint32_t kPipeFirstWords = 28;

// Work plan of the MFMA prefill kernel: one item per 32-row query tile of a
// sequence, longest first.
struct PrefillPlan {
    const uint32_t *work;  // [num_items][4]: (first row, rows, position of first row, sequence)
    uint32_t num_items;
    uint32_t max_keys;     // largest key count of any row (position + 1) in the plan
    // Items 0 .. num_long - 1 have rows past prefill_dma_max_keys() keys (the
    // order is longest first, so they lead); they run on the register-staged
    // kernel, the others on the DMA kernel.  The choice is made per item, from
    // the item's own rows, so a sequence's result does not depend on the
    // other sequences of the batch.
    uint32_t num_long = 0;
    // The pipelined kernel's plan for items num_long .. num_items - 1, dealt
    // to persistent workgroup slots: pipe[0 .. pipe_slots] are the slots'
    // first descriptor indices, then each slot's first record
    // (kPipeFirstWords words: its first item's descriptor, the block ids of
    // that item's tiles 0-2 and the next item's first twelve), then
    // [num_items - num_long][4] descriptors (first row, rows, position of
    // first row, offset of the sequence's block table) ordered by slot.
    const uint32_t *pipe = nullptr;
    uint32_t pipe_slots = 0;
};

// Keys the DMA prefill kernel takes per row (its block table lives in LDS).
uint32_t prefill_dma_max_keys();

// True when the MFMA prefill kernel covers this shape.
bool prefill_mfma_supported(uint32_t head_dim, uint32_t block_size, uint32_t group);
// Query rows per work item of the MFMA prefill kernel.
uint32_t prefill_rows_per_tile();

// num_cus: compute units of the device (0 if unknown); a plan with fewer
// 64-row workgroups than CUs runs on 32-row workgroups.
hipError_t launch_prefill_mfma(const PoolLayer &pool, const MetaView &meta,
                               const PrefillPlan &plan, const uint16_t *q, uint16_t *out,
                               uint32_t num_heads, float scale, uint32_t num_cus,
                               hipStream_t stream);

}  // namespace kernels
}  // namespace vo

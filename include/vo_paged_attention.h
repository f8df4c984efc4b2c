/*
 * vo_paged_attention.h -- C ABI of the MI355X (gfx950) paged-attention backend.
 *
 * This is the drop-in boundary for vllm-oxide's attention path.  The Rust
 * engine's `Backend` trait (crates/engine/src/backend/mod.rs:61-182) is
 * op-level: the engine owns block tables and slot mappings, the backend owns
 * the KV bytes (mod.rs:10-12).  Each trait op on the attention path has one
 * entry point here, with the same argument meaning and the same error classes
 * (crates/engine/src/error.rs:8-56):
 *
 *   Backend::alloc_kv_pool   (mod.rs:73-74)   -> vo_kv_pool_create
 *   Backend::kv_layout       (mod.rs:75)      -> vo_kv_pool_layout
 *   Backend::rope            (mod.rs:105)     -> vo_rope_positions (host positions);
 *                                                  vo_rope (the step upload's)
 *   Backend::write_kv        (mod.rs:107-119) -> vo_write_kv_slots (host slots);
 *                                                  vo_write_kv (the step upload's)
 *   Backend::prefill_attention (mod.rs:121-135) -> vo_step_meta_sync_prefill +
 *                                                  vo_prefill_attention
 *   Backend::decode_attention  (mod.rs:137-149) -> vo_step_meta_sync_decode +
 *                                                  vo_decode_attention
 *   Backend::gather_rows     (mod.rs:167)     -> vo_gather_rows
 *   Backend::embed, rmsnorm, matmul, silu_mul, add, argmax (mod.rs:84-175)
 *                                             -> vo_embed, vo_rmsnorm, vo_matmul,
 *                                                  vo_silu_mul, vo_add, vo_argmax
 *   Backend::read            (mod.rs:177-181) -> vo_workspace_read; vo_gather_kv
 *                                                  reads the pool (both debug/test only)
 *   Backend::alloc_workspace (mod.rs:76-77)   -> vo_workspace_create
 *   Backend::workspace_elems (mod.rs:78)      -> vo_workspace_elems
 *   Backend::upload          (mod.rs:69-70)   -> vo_weight_upload
 *   Backend::weight_shape    (mod.rs:71-72)   -> vo_weight_shape
 *
 * plus the paged-KV addressing of crates/engine/src/backend/paged.rs
 * (slot_of, PrefillMeta::new, DecodeMeta::new, last_rows) as host functions,
 * and a device-resident copy of one step's metadata (vo_step_meta) so that
 * block tables and slot mappings cross host->device once per step, not once
 * per layer.
 *
 * Conventions
 *  - Every function returns vo_status (0 = VO_OK).  All validation happens on
 *    the host, before anything is enqueued, exactly as the reference checks
 *    before it writes (cpu/mod.rs:265-272, attention.rs:130-147,
 *    arena/ops.rs:191-214, paged.rs:64-80).  On failure nothing is enqueued and
 *    vo_last_error() describes the error.  No C++ exception crosses the ABI.
 *  - Activations (queries, keys, values, outputs) are device pointers to
 *    row-major bf16 matrices, the GPU counterpart of the reference's f32
 *    workspace `Region {offset, rows, cols}` (mod.rs:31-38).  Accumulation is
 *    fp32.  Block tables, slots and lengths are host arrays, borrowed for the
 *    duration of the call only.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *    Every device op is asynchronous and stream-ordered; no call synchronises
 *    the device (the reference's one sync per step is argmax, mod.rs:169-175).
 *  - Safety contract (mod.rs:49-60): device regions are in bounds for the
 *    shapes given, and an output region overlaps no input region.  The
 *    library checks the overlap it can see (q vs out) and returns
 *    VO_ERR_SHAPE.
 *  - Not thread-safe per object: one engine thread owns a pool and a meta
 *    (the reference's "one engine thread owns the CUDA context").
 */
#ifndef VO_PAGED_ATTENTION_H
#define VO_PAGED_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ */
/* Status codes: one per EngineError variant on this path              */
/* (error.rs:8-56), plus the device and argument classes a C ABI needs. */
/* ------------------------------------------------------------------ */
typedef enum vo_status {
    VO_OK = 0,
    VO_ERR_SHAPE = 1,                  /* EngineError::Shape            error.rs:11-12 */
    VO_ERR_CAPACITY = 2,               /* EngineError::Capacity         error.rs:13-18 */
    VO_ERR_BLOCK_TABLE_TOO_SHORT = 3,  /* EngineError::BlockTable       error.rs:21-22 */
    VO_ERR_SLOT_OUT_OF_RANGE = 4,      /* EngineError::SlotOutOfRange   error.rs:23-28 */
    VO_ERR_BLOCK_OUT_OF_RANGE = 5,     /* EngineError::BlockOutOfRange  error.rs:29-34 */
    VO_ERR_DEVICE = 6,                 /* HIP runtime failure (no reference counterpart) */
    VO_ERR_INVALID_ARGUMENT = 7,       /* NULL pointer or zero size where one is required */
    VO_ERR_UNSUPPORTED = 8,            /* shape outside what the kernels are built for */
    VO_ERR_POSITION_OUT_OF_RANGE = 9,  /* EngineError::PositionOutOfRange error.rs:52-53 */
    VO_ERR_NAN = 10,                   /* EngineError::NaN              error.rs:54-55 */
    VO_ERR_OUTSIDE_WORKSPACE = 11      /* EngineError::OutsideWorkspace error.rs:47-48 */
} vo_status;

/* Element type of an activation buffer or a weight. */
typedef enum vo_dtype { VO_DTYPE_BF16 = 0, VO_DTYPE_F32 = 1 } vo_dtype;

/* Detail of the last failed call on the calling thread.  The numeric fields
 * carry what the reference's error variant carries:
 *   BlockTableTooShort {op, tokens, needed, have}       (paged.rs:57-62)
 *   SlotOutOfRange     {op, slot -> value, num_slots -> limit}
 *   BlockOutOfRange    {op, block -> value, num_blocks -> limit}
 *   Capacity           {what -> op, need -> value, limit}
 * `seq` is the sequence index for per-sequence errors.  `message` is the
 * reference's Display text for the variant. */
typedef struct vo_error_info {
    int32_t status;
    char op[48];
    uint64_t seq;
    uint64_t tokens;
    uint64_t needed;
    uint64_t have;
    uint64_t value;
    uint64_t limit;
    char message[256];
} vo_error_info;

/* Fills *out with the last error of this thread and returns its status
 * (VO_OK if the last call succeeded).  `out` may be NULL. */
int32_t vo_last_error(vo_error_info *out);
const char *vo_status_name(int32_t status);
const char *vo_version(void);

/* ------------------------------------------------------------------ */
/* Device memory the engine gets from the backend (mod.rs:61-78)       */
/* ------------------------------------------------------------------ */

/* Opaque.  The activation workspace (Backend::alloc_workspace, mod.rs:76-77):
 * one device allocation of `elems` 4-byte elements, zero-filled (the
 * reference's f32 workspace, cpu/mod.rs:163-166), allocated once at startup.
 * The engine's arena carves it into Regions {offset, rows, cols} in elements
 * (mod.rs:31-38); vo_workspace_region turns one into the device address the
 * ops take.  A Region's address is base + 4 * offset whatever the element type
 * the op keeps there: the ops on this path read and write bf16 activations
 * (2 bytes per value, so such a region uses the first half of its bytes) and
 * f32 for the residual stream and the logits. */
typedef struct vo_workspace vo_workspace;

int32_t vo_workspace_create(int32_t device, uint64_t elems, vo_workspace **out);
void vo_workspace_destroy(vo_workspace *ws);
/* Backend::workspace_elems (mod.rs:78); 0 for NULL. */
uint64_t vo_workspace_elems(const vo_workspace *ws);
/* Device address of Region {offset, rows, cols}.  VO_ERR_OUTSIDE_WORKSPACE
 * when offset + rows * cols > elems (cpu/mod.rs:57-62). */
int32_t vo_workspace_region(const vo_workspace *ws, uint64_t offset, uint64_t rows, uint64_t cols,
                            void **ptr);
/* Backend::read (mod.rs:177-181): the Region's rows * cols values of `dtype`
 * (VO_DTYPE_BF16 widened exactly, or VO_DTYPE_F32) into host_out as f32.
 * Waits for `stream` first; debug and tests only, never in the hot loop.
 * VO_ERR_OUTSIDE_WORKSPACE as vo_workspace_region. */
int32_t vo_workspace_read(const vo_workspace *ws, uint64_t offset, uint64_t rows, uint64_t cols,
                          int32_t dtype, float *host_out, void *stream);

/* Opaque.  A weight resident on one device (Backend::Weight, mod.rs:64-66). */
typedef struct vo_weight vo_weight;

/* Backend::upload (mod.rs:69-70): the host Weight (weights.rs:20-24: f32,
 * row-major, matrices [out_features, in_features]) of `ndim` dimensions
 * `shape` to `device`, as bf16 (VO_DTYPE_BF16: rounded to nearest even; what
 * the ops take) or f32.  Synchronous: `data` may be freed on return. */
int32_t vo_weight_upload(int32_t device, const float *data, const uint64_t *shape, uint64_t ndim,
                         int32_t dtype, vo_weight **out);
/* One weight holding `count` uploaded matrices of the same dtype, device and
 * column count, stacked by rows (a device copy).  No counterpart in the
 * reference, whose Llama::new uploads q/k/v and gate/up one by one
 * (model.rs:157-165): stacked, each group is one GEMM over the same input
 * (vo_qkv_rope_write_kv reads the [q | k | v] rows of such a product). */
int32_t vo_weight_concat_rows(const vo_weight *const *parts, uint64_t count, vo_weight **out);
void vo_weight_destroy(vo_weight *w);
/* Backend::weight_shape (mod.rs:71-72): *ndim dimensions, the first
 * `capacity` of them into shape (shape may be NULL to ask for ndim). */
int32_t vo_weight_shape(const vo_weight *w, uint64_t *shape, uint64_t capacity, uint64_t *ndim);
/* The device address and element type (vo_dtype) the ops take. */
const void *vo_weight_data(const vo_weight *w);
int32_t vo_weight_dtype(const vo_weight *w);

/* ------------------------------------------------------------------ */
/* Paged-KV addressing, host side (paged.rs)                          */
/* ------------------------------------------------------------------ */

/* KvLayout (paged.rs:25-45).  Per layer, K and V each hold
 * num_blocks * block_size slots of kv_heads x head_dim values. */
typedef struct vo_kv_layout {
    uint64_t num_layers;
    uint64_t num_blocks;
    uint64_t block_size;
    uint64_t kv_heads;
    uint64_t head_dim;
} vo_kv_layout;

/* KvLayout::num_slots (paged.rs:38-40) and ::layer_elems (paged.rs:42-44). */
uint64_t vo_kv_layout_num_slots(const vo_kv_layout *layout);
uint64_t vo_kv_layout_layer_elems(const vo_kv_layout *layout);

/* slot_of (paged.rs:48-52): table[pos / bs] * bs + pos % bs.  The reference
 * panics on an index past the table; here that is VO_ERR_BLOCK_TABLE_TOO_SHORT. */
int32_t vo_slot_of(const uint32_t *block_table, uint64_t table_len, uint64_t pos,
                   uint64_t block_size, uint32_t *out_slot);

/* One sequence of a prefill step (PrefillSeq, paged.rs:84-92). */
typedef struct vo_prefill_seq {
    uint64_t context_len;
    uint64_t num_new;
    const uint32_t *block_table;
    uint64_t block_table_len;
} vo_prefill_seq;

/* One sequence of a decode step (DecodeSeq, paged.rs:164-168). */
typedef struct vo_decode_seq {
    uint64_t context_len;
    const uint32_t *block_table;
    uint64_t block_table_len;
} vo_decode_seq;

/* PrefillMeta::new (paged.rs:117-143) into caller-sized arrays:
 * seq_row_starts [S+1]; positions, slot_mapping, row_seq, row_num_keys [T]
 * with T = sum num_new.  Any output pointer may be NULL.  Fails with
 * VO_ERR_BLOCK_TABLE_TOO_SHORT {op "prefill", tokens, needed, have, seq}. */
int32_t vo_prefill_meta_build(const vo_prefill_seq *seqs, uint64_t num_seqs,
                              uint64_t block_size, uint64_t *seq_row_starts,
                              uint32_t *positions, uint32_t *slot_mapping,
                              uint64_t *row_seq, uint64_t *row_num_keys);

/* DecodeMeta::new (paged.rs:189-209): outputs [S].  Fails with
 * VO_ERR_BLOCK_TABLE_TOO_SHORT {op "decode", ...}. */
int32_t vo_decode_meta_build(const vo_decode_seq *seqs, uint64_t num_seqs,
                             uint64_t block_size, uint32_t *positions,
                             uint32_t *slot_mapping, uint64_t *row_seq,
                             uint64_t *row_num_keys);

/* PrefillMeta::new (paged.rs:117-143) on the device.  No counterpart in the
 * reference, which builds a step's metadata on the host: this is for callers
 * that keep a batch's per-sequence state in device memory (context lengths,
 * CSR block tables) and want the per-row arrays without a host round trip.
 * Inputs, all device u32 arrays: seq_row_starts [S+1] (row offsets, from 0
 * to num_rows), context_lens [S], table_off [S+1], tables [table_off[S]].
 * Outputs, device u32 arrays [num_rows]: positions, slot_mapping, row_seq,
 * row_num_keys, exactly the values vo_prefill_meta_build returns.  A decode
 * step (DecodeMeta::new, paged.rs:189-209) is seq_row_starts[s] = s.
 * The coverage check of paged.rs:64-80 runs on the device: a row whose
 * position lies past its sequence's table gets slot 0xffffffff and sets
 * *errors (a device u32 the call does not clear) to 1, so the caller checks
 * the flag where the reference would return BlockTableTooShort.
 * Asynchronous on `stream`; the caller keeps the arrays alive until it ends. */
int32_t vo_prefill_meta_build_device(const uint32_t *seq_row_starts, const uint32_t *context_lens,
                                     const uint32_t *table_off, const uint32_t *tables,
                                     uint64_t num_seqs, uint64_t num_rows, uint64_t block_size,
                                     uint32_t *positions, uint32_t *slot_mapping,
                                     uint32_t *row_seq, uint32_t *row_num_keys, uint32_t *errors,
                                     void *stream);

/* PrefillMeta::last_rows (paged.rs:154-159): out[s] = seq_row_starts[s+1]-1. */
int32_t vo_last_rows(const uint64_t *seq_row_starts, uint64_t num_seqs, uint32_t *out);

/* ------------------------------------------------------------------ */
/* KV pool (Backend::KvPool, mod.rs:64-75)                             */
/* ------------------------------------------------------------------ */

/* Opaque.  Device memory for all layers' K and V, bf16, zero-filled at
 * creation (the reference's calloc, cpu/mod.rs:148-157).  The physical
 * layout is private to the backend (ADR 0003); logical slot semantics are the
 * reference's: slot = block * block_size + offset. */
typedef struct vo_kv_pool vo_kv_pool;

/* Backend::alloc_kv_pool (mod.rs:73-74): allocate once at startup on
 * `device`.  head_dim must be a multiple of 8; the fast kernels cover
 * head_dim 64/128 with block_size 16, every other shape runs on the generic
 * kernels. */
int32_t vo_kv_pool_create(const vo_kv_layout *layout, int32_t device, vo_kv_pool **out);
void vo_kv_pool_destroy(vo_kv_pool *pool);
/* Backend::kv_layout (mod.rs:75). */
int32_t vo_kv_pool_layout(const vo_kv_pool *pool, vo_kv_layout *out);
/* Bytes of device memory the pool holds. */
uint64_t vo_kv_pool_bytes(const vo_kv_pool *pool);

/* ------------------------------------------------------------------ */
/* Step metadata, device resident                                      */
/* ------------------------------------------------------------------ */

/* Opaque.  Preallocated at startup for a maximum batch, then refilled once
 * per step with a PrefillMeta, a DecodeMeta or a bare slot list.  Holds a
 * host copy for validation and a device copy for the kernels, plus the
 * split-K work plan and the fp32 partial buffers the decode kernels use.
 * Nothing is allocated after creation (CLAUDE.md:70 "no allocation in the
 * hot loop"). */
typedef struct vo_step_meta vo_step_meta;

/* max_rows: rows (tokens) per step; max_seqs: sequences per step;
 * max_table_entries: sum of block-table lengths per step; max_query_heads:
 * the largest num_heads an attention call will use. */
int32_t vo_step_meta_create(const vo_kv_pool *pool, uint64_t max_seqs, uint64_t max_rows,
                            uint64_t max_table_entries, uint64_t max_query_heads,
                            vo_step_meta **out);
void vo_step_meta_destroy(vo_step_meta *meta);

/* Upload a PrefillMeta (paged.rs:97-114) built by vo_prefill_meta_build or by
 * the engine.  Tables are CSR: table s is tables[table_off[s] ..
 * table_off[s+1]).  Fails with VO_ERR_CAPACITY when the batch exceeds the
 * sizes given at creation.  Enqueues host->device copies on `stream`; the
 * host arrays may be reused as soon as the call returns. */
int32_t vo_step_meta_upload_prefill(vo_step_meta *meta, uint64_t block_size, uint64_t num_seqs,
                                    const uint64_t *table_off, const uint32_t *tables,
                                    const uint64_t *context_lens,
                                    const uint64_t *seq_row_starts, uint64_t num_rows,
                                    const uint32_t *positions, const uint32_t *slot_mapping,
                                    const uint64_t *row_seq, const uint64_t *row_num_keys,
                                    void *stream);

/* Upload a DecodeMeta (paged.rs:173-186): one row per sequence. */
int32_t vo_step_meta_upload_decode(vo_step_meta *meta, uint64_t block_size, uint64_t num_seqs,
                                   const uint64_t *table_off, const uint32_t *tables,
                                   const uint32_t *positions, const uint32_t *slot_mapping,
                                   const uint64_t *row_seq, const uint64_t *row_num_keys,
                                   void *stream);

/* Fixed launch shapes, so that a decode step can be recorded once as a HIP
 * graph and replayed for later steps (no counterpart in the reference; for
 * engines that capture the decode step to take the per-launch host cost out
 * of small-batch decoding).  Takes the last upload, which must be a decode
 * step of S sequences, and uploads it again in a layout where every array
 * has a fixed device address, sized for S sequences, the current table
 * entries + entry_headroom and the current split-K work items +
 * work_headroom; the decode kernels are then launched for that many work
 * items and S reduce rows and read the step's own counts from the device.
 * While fixed, every launch of a decode step through this meta has the same
 * arguments and grid, and vo_step_meta_upload_decode accepts only steps that
 * fit (else VO_ERR_SHAPE / VO_ERR_CAPACITY with nothing changed: unfix,
 * upload, fix and record again); prefill and slot uploads are refused.  The
 * first call of each GEMM shape (vo_matmul) must happen before recording. */
int32_t vo_step_meta_fix_launch(vo_step_meta *meta, uint64_t work_headroom,
                                uint64_t entry_headroom, void *stream);
/* Back to packed uploads from the next upload on. */
int32_t vo_step_meta_unfix_launch(vo_step_meta *meta);

/* The split-K plan of the last upload (diagnostic; no counterpart in the
 * reference, whose CPU backend has no launch plan): work items launched per
 * KV head, split-K partials (one per (row, split)), and the row-packing
 * factor P -- with P > 1, full splits of up to P rows that read the same
 * physical blocks (a shared prefix) run as one work item.  VO_ERR_ARGUMENT
 * when the last upload planned no decode rows. */
int32_t vo_step_meta_decode_plan(const vo_step_meta *meta, uint64_t *work_items,
                                 uint64_t *partials, uint32_t *pack);

/* Upload only a slot list, for write_kv calls whose slots are not a step's
 * slot mapping (the reference's tests write ad-hoc ranges, cpu/tests.rs:210-230). */
int32_t vo_step_meta_upload_slots(vo_step_meta *meta, const uint32_t *slots, uint64_t num_slots,
                                  void *stream);

/* The trait's form of the two uploads: Backend::prefill_attention and
 * decode_attention (mod.rs:121-149) take `meta: &PrefillMeta` / `&DecodeMeta`
 * at every layer, so an implementation of the trait calls these with the
 * meta's arrays before each attention call.  Same arguments, checks and
 * errors as vo_step_meta_upload_prefill / _decode; when the meta's last
 * upload is a step of the same kind whose every array holds the same values
 * (compared on the host, element by element: the caller may refill the same
 * buffers for the next step), nothing is uploaded or planned again and the
 * call returns VO_OK. */
int32_t vo_step_meta_sync_prefill(vo_step_meta *meta, uint64_t block_size, uint64_t num_seqs,
                                  const uint64_t *table_off, const uint32_t *tables,
                                  const uint64_t *context_lens, const uint64_t *seq_row_starts,
                                  uint64_t num_rows, const uint32_t *positions,
                                  const uint32_t *slot_mapping, const uint64_t *row_seq,
                                  const uint64_t *row_num_keys, void *stream);
int32_t vo_step_meta_sync_decode(vo_step_meta *meta, uint64_t block_size, uint64_t num_seqs,
                                 const uint64_t *table_off, const uint32_t *tables,
                                 const uint32_t *positions, const uint32_t *slot_mapping,
                                 const uint64_t *row_seq, const uint64_t *row_num_keys,
                                 void *stream);

/* ------------------------------------------------------------------ */
/* Ops                                                                 */
/* ------------------------------------------------------------------ */

/* Backend::write_kv (mod.rs:107-119; CPU: cpu/mod.rs:257-285) -- the
 * reshape_and_cache kernel.  Stores row t of keys/values ([rows, cols] bf16,
 * cols = kv_heads * head_dim) at slot slot_mapping[t] of `layer`, where the
 * slot mapping is the one last uploaded into `meta`.  Checks first, as
 * arena/ops.rs:102-131 and cpu/mod.rs:265-272 do: rows == number of slots,
 * cols == kv_heads * head_dim, layer < num_layers (VO_ERR_SHAPE), then every
 * slot < num_slots (VO_ERR_SLOT_OUT_OF_RANGE).  Slots must be distinct within
 * one call: the reference's "later row wins" (cpu/mod.rs:277-283) has no
 * ordering guarantee on a GPU. */
int32_t vo_write_kv(vo_kv_pool *pool, uint64_t layer, const void *keys, const void *values,
                    uint64_t rows, uint64_t cols, const vo_step_meta *meta, void *stream);

/* Backend::write_kv with the trait's own arguments (mod.rs:107-119:
 * `slots: &[u32]`): the slots [num_slots] are host values.  Checks rows ==
 * num_slots, cols and layer first (VO_ERR_SHAPE, nothing uploaded).  When
 * the meta's last upload holds exactly these slots (the model passes the
 * step's slot mapping, model.rs:289-292) it runs vo_write_kv on them;
 * otherwise it uploads them as vo_step_meta_upload_slots does (replacing the
 * meta's last upload; a later vo_step_meta_sync_* uploads the step again)
 * and then runs vo_write_kv.  Errors: those of vo_write_kv. */
int32_t vo_write_kv_slots(vo_kv_pool *pool, uint64_t layer, const void *keys, const void *values,
                          uint64_t rows, uint64_t cols, const uint32_t *slots, uint64_t num_slots,
                          vo_step_meta *meta, void *stream);

/* write_kv followed by decode_attention on the same decode step
 * (model.rs:310-316: the step's new keys are cached, then attended), in one
 * launch where the step allows it: the split-K workgroup holding a row's
 * last key writes that key's K/V to the pool and uses the new rows directly.
 * Results (the output and the pool) are bitwise those of vo_write_kv then
 * vo_decode_attention, which run instead when a slot repeats, rows alias
 * the block of another row's new slot, or the launch shapes are fixed.  No
 * counterpart in the reference, whose CPU backend runs the two ops; for
 * engines that decode with write_kv and decode_attention back to back.
 * Arguments and errors: those of the two ops. */
int32_t vo_decode_attention_write_kv(const void *queries, uint64_t rows, uint64_t cols,
                                     const void *keys, const void *values, uint64_t kv_cols,
                                     vo_kv_pool *pool, uint64_t layer, const vo_step_meta *meta,
                                     void *out, void *stream);

/* Backend::prefill_attention (mod.rs:121-135; CPU: cpu/mod.rs:287-312).
 * queries, out: [rows, num_heads * head_dim] bf16 with num_heads = cols /
 * head_dim.  Row t attends to row_num_keys[t] keys of sequence row_seq[t]
 * through its block table; causality comes from the key counts
 * (attention.rs:16).  Checks: arena/ops.rs:191-214 (VO_ERR_SHAPE), then
 * every table entry < num_blocks (VO_ERR_BLOCK_OUT_OF_RANGE,
 * attention.rs:130-147).  `meta` must hold a prefill upload. */
int32_t vo_prefill_attention(const void *queries, uint64_t rows, uint64_t cols,
                             const vo_kv_pool *pool, uint64_t layer, const vo_step_meta *meta,
                             void *out, void *stream);

/* Backend::decode_attention (mod.rs:137-149; CPU: cpu/mod.rs:314-339): one
 * query row per sequence.  Split-K over the keys with an fp32 partial per
 * split and a reduce kernel.  `meta` must hold a decode upload. */
int32_t vo_decode_attention(const void *queries, uint64_t rows, uint64_t cols,
                            const vo_kv_pool *pool, uint64_t layer, const vo_step_meta *meta,
                            void *out, void *stream);

/* Decode attention that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The op is
 * Backend::decode_attention (mod.rs:137-149) on the kernels of
 * vo_decode_attention, and its output is bitwise that entry point's; but the
 * decode step's metadata is read from device memory the caller owns, in
 * DecodeMeta::new's layout (paged.rs:189-209: row s is sequence s): table_off
 * [rows+1] CSR offsets into tables [num_entries], row_num_keys [rows]
 * (context + 1), all device u32 arrays, and no vo_step_meta is needed.  The
 * split-K plan and partials live in a fixed 32 MiB device array per GPU,
 * which bounds a call: rows <= 4096 and rows * ceil(max_keys / 2048) work
 * items of partials (num_heads * head_dim fp32 each) within 32 MiB, else
 * VO_ERR_CAPACITY before anything is enqueued (e.g. 256 rows of up to 8192
 * keys at 32 heads of 128 dims fit).  max_keys bounds every row's key count.
 * The host checks shapes and sizes; the device checks, before any pool read,
 * what vo_decode_attention checks on the host -- coverage (paged.rs:64-80),
 * every table entry < num_blocks (attention.rs:130-147) -- plus keys <=
 * max_keys and offsets ascending within num_entries; on a failure it sets
 * *errors (a device u32 the call does not clear) to 1 and writes zero rows.
 * Calls that overlap on one GPU (other streams, other threads) share its
 * array and race.  Needs block size 16, head_dim 64 or 128, group <= 16. */
int32_t vo_decode_attention_static(const void *queries, uint64_t rows, uint64_t cols,
                                   const vo_kv_pool *pool, uint64_t layer, const uint32_t *table_off,
                                   const uint32_t *tables, uint64_t num_entries,
                                   const uint32_t *row_num_keys, uint64_t max_keys, void *out,
                                   uint32_t *errors, void *stream);

/* Debug and test only (the counterpart of Backend::read, mod.rs:177-181):
 * gather keys 0..num_keys of sequence `seq` of the last upload in `meta` from
 * `layer` into out_keys and out_values, each [num_keys, kv_heads * head_dim]
 * bf16 in the reference's logical layout (paged.rs:25-28): row j is the
 * pool entry at slot_of(table, j).  The kernel reads the block table from
 * the meta's device copy, as the attention kernels do.  Checks seq range
 * (VO_ERR_SHAPE), coverage (VO_ERR_BLOCK_TABLE_TOO_SHORT) and block range
 * (VO_ERR_BLOCK_OUT_OF_RANGE) first. */
int32_t vo_gather_kv(const vo_kv_pool *pool, uint64_t layer, const vo_step_meta *meta,
                     uint64_t seq, uint64_t num_keys, void *out_keys, void *out_values,
                     void *stream);

/* ------------------------------------------------------------------ */
/* KV block manager and prefix cache (host side)                       */
/* ------------------------------------------------------------------ */

/* No counterpart in the reference snapshot: it plans the block manager (the
 * owner's M2) and the prefix cache (M4) (README.md:14, CLAUDE.md:26,
 * docs/process.md:43-47) and fixes their invariant (CLAUDE.md:71): every
 * block is free or referenced by >= 1 block table, its refcount equals the
 * number of references, nothing is freed while a sequence uses it.  It
 * replaces the M0 driver's block counter (generate.rs:4-7).  Host only; it
 * makes no HIP call.  Block tables it returns feed PrefillSeq / DecodeSeq.
 *
 * Prefix caching shares whole blocks: block i of a sequence is identified by
 * a hash chained over the token ids of blocks 0..i, and a hit also compares
 * the stored token ids.  A prompt reuses its longest run of cached leading
 * blocks, never the block holding its last token.  Blocks whose sequences
 * are all freed stay cached (least recently used first out) until a new
 * block is needed.  An empty pool is VO_ERR_CAPACITY and changes nothing
 * (preemption is the scheduler's policy, docs/grill-log.md:86-88). */
typedef struct vo_block_manager vo_block_manager;

typedef struct vo_bm_stats {
    uint64_t hit_blocks;          /* prompt blocks served from the prefix cache */
    uint64_t lookup_blocks;       /* prompt blocks that could have been served */
    uint64_t evictions;           /* cached idle blocks reused for new contents */
    uint64_t copies;              /* copy-on-write block copies handed out */
    uint64_t free_blocks;         /* on the free list now */
    uint64_t cached_idle_blocks;  /* refcount 0, still cached, now */
    uint64_t sequences;           /* live sequences now */
} vo_bm_stats;

int32_t vo_bm_create(uint64_t num_blocks, uint64_t block_size, int32_t prefix_caching,
                     vo_block_manager **out);
void vo_bm_destroy(vo_block_manager *bm);
/* Test hook, no reference counterpart: with on != 0 a block's hash covers
 * its own tokens only, so that equal blocks after different prefixes collide
 * on purpose (the tests of the prefix cache's collision handling).  Only
 * before the first sequence; VO_ERR_INVALID_ARGUMENT otherwise. */
int32_t vo_bm_test_unchained_hash(vo_block_manager *bm, int32_t on);
/* Admits a sequence with its prompt and gives it ceil(n / bs) blocks;
 * *cached_tokens = prompt tokens whose KV the prefix cache already holds
 * (a multiple of bs; the step computes the rest). */
int32_t vo_bm_add_sequence(vo_block_manager *bm, uint64_t seq_id, const uint32_t *tokens,
                           uint64_t num_tokens, uint64_t *cached_tokens);
/* Appends one token: a new block on a block boundary; a copy of the last
 * block when a fork shares it, reported as *copy_src -> *copy_dst (else both
 * 0xffffffff) for vo_kv_copy_blocks.  *slot is the token's KV slot. */
int32_t vo_bm_append_token(vo_block_manager *bm, uint64_t seq_id, uint32_t token, uint32_t *slot,
                           uint32_t *copy_src, uint32_t *copy_dst);
/* The child shares every block of the parent (one more reference each). */
int32_t vo_bm_fork(vo_block_manager *bm, uint64_t parent, uint64_t child);
/* Drops the sequence's references. */
int32_t vo_bm_free_sequence(vo_block_manager *bm, uint64_t seq_id);
/* Copies the sequence's block table into out[capacity] (out may be NULL to
 * query *len); *num_tokens = its token count. */
int32_t vo_bm_block_table(const vo_block_manager *bm, uint64_t seq_id, uint32_t *out,
                          uint64_t capacity, uint64_t *len, uint64_t *num_tokens);
/* Blocks a new sequence could take now (free + cached idle). */
uint64_t vo_bm_num_available(const vo_block_manager *bm);
int32_t vo_bm_get_stats(const vo_block_manager *bm, vo_bm_stats *out);
/* Checks CLAUDE.md:71 and the manager's bookkeeping exhaustively; VO_OK or
 * VO_ERR_SHAPE with the first violation in vo_last_error's message. */
int32_t vo_bm_check_invariants(const vo_block_manager *bm);

/* Copies whole blocks of every layer's K and V in the pool: for each i,
 * block dst[i] := block src[i] (the block manager's copy-on-write).  Block
 * ids are checked against the pool (VO_ERR_BLOCK_OUT_OF_RANGE); a
 * destination may not repeat or also be a source (VO_ERR_SHAPE).
 * Asynchronous on `stream`; the id arrays are host arrays. */
int32_t vo_kv_copy_blocks(vo_kv_pool *pool, const uint32_t *src, const uint32_t *dst,
                          uint64_t count, void *stream);

/* ------------------------------------------------------------------ */
/* Rotary position embedding (Backend::rope, mod.rs:105; rope.rs)      */
/* ------------------------------------------------------------------ */

/* The RoPE fields of ModelConfig (config.rs:9-34): head_dim, rope_theta and
 * the llama3 rope_scaling block. */
typedef struct vo_rope_config {
    uint64_t head_dim;
    double rope_theta;
    double factor;
    double low_freq_factor;
    double high_freq_factor;
    uint64_t original_max_position_embeddings;
} vo_rope_config;

/* Opaque: RopeTable (rope.rs:24-31) on one device, cos and sin
 * [max_len][head_dim/2] f32, computed on the host in the reference's f32
 * order (llama3_inv_freq rope.rs:36-60, RopeTable::new rope.rs:62-84) and
 * copied to the device once (CpuBackend::new builds it once, cpu/mod.rs:53). */
typedef struct vo_rope_table vo_rope_table;

int32_t vo_rope_table_create(const vo_rope_config *config, uint64_t max_len, int32_t device,
                             vo_rope_table **out);
void vo_rope_table_destroy(vo_rope_table *table);

/* Backend::rope (mod.rs:105; cpu/mod.rs:231-255; shape checks
 * arena/ops.rs:83-99): rotates x [rows, cols] bf16 in place, every head of
 * width head_dim, row r at the position the step metadata gives it
 * (vo_step_meta_upload_prefill / _decode positions; rows == the meta's rows).
 * f32 arithmetic in the reference's order, result rounded to bf16.
 * Errors: VO_ERR_SHAPE (positions != rows, head_dim odd or zero or not
 * dividing cols, or head_dim != the table's), VO_ERR_POSITION_OUT_OF_RANGE
 * {value = pos, limit = max_len} for the first position past the table. */
int32_t vo_rope(const vo_rope_table *table, void *x, uint64_t rows, uint64_t cols,
                uint64_t head_dim, const vo_step_meta *meta, void *stream);

/* Backend::rope with the trait's own arguments (mod.rs:105: `positions:
 * &[u32]`): positions [num_positions] are host values.  Checks and errors
 * as vo_rope, on these positions.  When the meta's last upload holds exactly
 * these positions the kernel reads the meta's device copy; otherwise they
 * go to a device array of the meta's own (at most max_rows values,
 * VO_ERR_CAPACITY), copied from pinned staging on `stream` only when the
 * values differ from that array's last contents.  The meta's last upload is
 * left as it is.  Calls on one meta are ordered by `stream`. */
int32_t vo_rope_positions(const vo_rope_table *table, void *x, uint64_t rows, uint64_t cols,
                          uint64_t head_dim, const uint32_t *positions, uint64_t num_positions,
                          vo_step_meta *meta, void *stream);

/* The layer's "rope(q); rope(k); write_kv(k, v)" (model.rs:307-311) as one
 * launch.  No counterpart in the reference's op list: it fuses three of its
 * ops.  queries [rows, q_cols] are rotated in place (as Backend::rope leaves
 * them); keys [rows, kv_cols] are read, rotated and written to the pool with
 * values; the caller's keys buffer itself is left unrotated (the reference
 * never reads k after write_kv).  Checks are those of vo_rope on both
 * operands and of vo_write_kv, in that order, all before the launch.
 * Needs block size 16 and head_dim 64 or 128 (else VO_ERR_UNSUPPORTED; use
 * vo_rope twice and vo_write_kv). */
int32_t vo_rope_write_kv(vo_kv_pool *pool, uint64_t layer, const vo_rope_table *table,
                         void *queries, uint64_t q_cols, const void *keys, const void *values,
                         uint64_t rows, uint64_t kv_cols, const vo_step_meta *meta, void *stream);

/* ------------------------------------------------------------------ */
/* The rest of the layer (Llama::forward, model.rs:269-356)            */
/* ------------------------------------------------------------------ */

/* The step's token ids (Llama::prefill / decode `tokens`, model.rs:221-243),
 * kept apart from the attention metadata: a host copy for embed's check and
 * a device copy (one async copy from pinned staging on `stream`).  At most
 * max_rows ids (VO_ERR_CAPACITY). */
int32_t vo_step_meta_upload_tokens(vo_step_meta *meta, const uint32_t *tokens,
                                   uint64_t num_tokens, void *stream);

/* Backend::embed (mod.rs:84; cpu/mod.rs:172-180): row r of out [rows,
 * hidden] f32 = row tokens[r] of table [vocab, hidden] bf16 (widened, exact),
 * tokens being the meta's last upload_tokens.  Checks (arena/ops.rs:30-44):
 * rows == number of tokens, then the first token >= vocab fails with
 * VO_ERR_SHAPE "embed: token {t} >= vocab {v}". */
int32_t vo_embed(const void *table, uint64_t vocab, uint64_t hidden, const vo_step_meta *meta,
                 uint64_t rows, float *out, void *stream);

/* Backend::rmsnorm (mod.rs:91-96; cpu/mod.rs:182-197): out [rows, cols] bf16 =
 * weight * (x * 1/sqrt(mean(x^2) + eps)) per row, x [rows, cols] f32 (the
 * residual stream), weight [weight_len] bf16.  Check (arena/ops.rs:47-62):
 * weight_len == cols (VO_ERR_SHAPE). */
int32_t vo_rmsnorm(const float *x, uint64_t rows, uint64_t cols, const void *weight,
                   uint64_t weight_len, float eps, void *out, void *stream);

/* The LM head's input (model.rs:334-343): gather_rows(x, meta.last_rows())
 * then rmsnorm, in one pass.  out [num_seqs, cols] bf16: row s normalises
 * the last row of sequence s (PrefillMeta::last_rows, paged.rs:153-159); for
 * a decode upload every row.  Checks: weight_len == cols, rows == the meta's
 * rows, and the upload is a prefill or decode one whose sequences all have
 * rows (VO_ERR_SHAPE). */
int32_t vo_rmsnorm_last_rows(const float *x, uint64_t rows, uint64_t cols, const void *weight,
                             uint64_t weight_len, float eps, const vo_step_meta *meta, void *out,
                             void *stream);

/* Backend::gather_rows (mod.rs:167; cpu/mod.rs:360-368): row i of out
 * [num_rows_idx, cols] = row row_idx[i] of x [rows, cols], both of `dtype`
 * (VO_DTYPE_F32 for the residual stream, or VO_DTYPE_BF16); row_idx are host
 * values.  Check (arena/ops.rs:242-244): the first index >= rows fails with
 * VO_ERR_SHAPE "gather_rows: row {r} of x [rows, cols]".  Rows must be whole
 * 4-byte words (a bf16 row of odd width is VO_ERR_ARGUMENT) and out must not
 * overlap x.  When row_idx are the meta's last rows (PrefillMeta::last_rows,
 * paged.rs:153-159) the kernel reads the meta's device copy; otherwise a
 * device array of the meta's own, refilled from pinned staging on `stream`
 * when the values change (at most max_rows, VO_ERR_CAPACITY). */
int32_t vo_gather_rows(const void *x, int32_t dtype, uint64_t rows, uint64_t cols,
                       const uint32_t *row_idx, uint64_t num_rows_idx, vo_step_meta *meta,
                       void *out, void *stream);

/* Backend::add (mod.rs:161; cpu/mod.rs:351-358): sum [rows, cols] f32 += x
 * [rows, cols] of x_dtype.  The model's residual adds also run fused into
 * vo_matmul (accumulate = 1). */
int32_t vo_add(float *sum, const void *x, int32_t x_dtype, uint64_t rows, uint64_t cols,
               void *stream);

/* Backend::silu_mul (mod.rs:155; cpu/mod.rs:341-349): out = silu(gate) * up
 * = gate / (1 + e^-gate) * up, all [rows, cols] bf16 with row strides (in
 * elements) gate_ld, up_ld, out_ld >= cols.  out may be gate itself (the
 * reference's in-place form); gate and up may be the two halves of one
 * fused gate/up projection ([rows, 2*cols], gate_ld = up_ld = 2*cols).
 * e^-gate and the quotient use the GPU's exp2 and reciprocal: the f32 value
 * is within ~2^-20 of the exact one, each output within one bf16 ulp of the
 * reference's f32 result. */
int32_t vo_silu_mul(const void *gate, uint64_t gate_ld, const void *up, uint64_t up_ld,
                    uint64_t rows, uint64_t cols, void *out, uint64_t out_ld, void *stream);

/* Backend::argmax (mod.rs:175; cpu/mod.rs:370-388): ids[r] = index of the
 * first maximum of row r of logits [rows, cols] (dtype bf16 or f32).  ids is
 * a device array [rows]; a row with a NaN gets 0xffffffff.  With host_ids
 * non-NULL the call also copies the ids there, waits for `stream`, and
 * returns VO_ERR_NAN {op "argmax"} if a row held a NaN -- the step's one
 * device-to-host synchronisation, as in the reference (arena/ops.rs:252-253). */
int32_t vo_argmax(const void *logits, int32_t dtype, uint64_t rows, uint64_t cols, uint32_t *ids,
                  uint32_t *host_ids, void *stream);

/* The layer's "q, k, v = matmul(...); rope(q); rope(k); write_kv(k, v)"
 * (model.rs:303-311) over one fused QKV projection output: qkv [rows,
 * q_cols + 2*kv_cols] bf16, each row [q | k | v].  Writes rotated q to q_out
 * [rows, q_cols] (a contiguous operand for attention), rotates k and writes
 * k and v to the pool at the meta's slots, in one launch.  Checks and limits
 * are vo_rope_write_kv's. */
int32_t vo_qkv_rope_write_kv(vo_kv_pool *pool, uint64_t layer, const vo_rope_table *table,
                             const void *qkv, uint64_t rows, uint64_t q_cols, uint64_t kv_cols,
                             const vo_step_meta *meta, void *q_out, void *stream);

/* Dense projections: Backend::matmul (mod.rs:98; cpu/mod.rs:199-229) on
 * hipBLASLt.  Opaque: one hipBLASLt handle, a workspace and a cache of
 * per-shape algorithm choices on one device.  hipBLASLt is loaded at
 * vo_gemm_create (the copy the process already has, else libhipblaslt.so.1);
 * VO_ERR_UNSUPPORTED when it cannot be. */
typedef struct vo_gemm vo_gemm;
int32_t vo_gemm_create(int32_t device, uint64_t workspace_bytes, vo_gemm **out);
void vo_gemm_destroy(vo_gemm *gemm);

/* out [rows, out_features] = x [rows, x_cols] . weight^T, weight [out_features,
 * in_features] bf16 (the reference's Weight layout), x bf16, fp32
 * accumulation, out of out_dtype.  accumulate = 1: out += x . weight^T (the
 * model's add(residual, matmul(..)), model.rs:320-321 and :330-331, fused
 * into the GEMM's epilogue).  Check (arena/ops.rs:65-81): in_features ==
 * x_cols (VO_ERR_SHAPE "x [r, c], weight [o, i]"). */
int32_t vo_matmul(vo_gemm *gemm, const void *x, uint64_t rows, uint64_t x_cols, const void *weight,
                  uint64_t out_features, uint64_t in_features, void *out, int32_t out_dtype,
                  int32_t accumulate, void *stream);

/* ------------------------------------------------------------------ */
/* Opt-in kernel timing (the reference's opt-in per-op timing,         */
/* arena.rs:82-87 OpStat, :129-136 enable_profiling)                   */
/* ------------------------------------------------------------------ */

/* Per-kernel totals since the last reset. */
typedef struct vo_kernel_stat {
    char name[48];
    uint64_t calls;
    double total_ms;
    double min_ms;
    double max_ms;
} vo_kernel_stat;

/* While enabled, every kernel launch is bracketed by HIP events on its
 * stream.  Recording never waits on the device. */
int32_t vo_profiling_enable(int32_t on);
/* Waits for the recorded events (call outside the hot loop), folds them into
 * the per-kernel totals and copies up to `capacity` entries to `out`;
 * `*count` receives the number of kernels seen. */
int32_t vo_profile_read(vo_kernel_stat *out, uint64_t capacity, uint64_t *count);
/* Drops all totals and pending events. */
void vo_profile_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* VO_PAGED_ATTENTION_H */

/*
 * vo_oracle.h -- CPU restatement of vllm-oxide's paged-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the correctness oracle and the
 * CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker.  The product library
 * (libvo_paged_attention.so) never links, loads or calls anything here.
 *
 * Every function restates one item of the Rust reference (KamdynS/vLLM-oxide,
 * crates/engine/src/...) and cites the file:line it follows.  Numerics follow
 * the reference bit for bit where C allows it: f32 throughout, the 16-lane
 * partial-sum dot, the two-pass softmax in index order, glibc expf/sqrtf, and
 * no FMA contraction (built with -ffp-contract=off).
 *
 * Integer widths: Rust `usize` is uint64_t here, `u32` is uint32_t.
 * Block tables are passed in CSR form: table s is
 * tables[table_off[s] .. table_off[s+1]), which is the flattening of the
 * reference's `Vec<Vec<u32>>` (paged.rs:99-100).
 *
 * Status codes returned by the checking functions mirror EngineError
 * (error.rs:8-56): 0 = Ok, VO_ORACLE_BLOCK_TABLE_TOO_SHORT,
 * VO_ORACLE_SLOT_OUT_OF_RANGE, VO_ORACLE_BLOCK_OUT_OF_RANGE, VO_ORACLE_NAN.
 */
#ifndef VO_ORACLE_H
#define VO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    VO_ORACLE_OK = 0,
    VO_ORACLE_BLOCK_TABLE_TOO_SHORT = 3,
    VO_ORACLE_SLOT_OUT_OF_RANGE = 4,
    VO_ORACLE_BLOCK_OUT_OF_RANGE = 5,
};

/* Error payload: which sequence / value failed and the numbers the
 * reference's error variants carry (paged.rs:57-62, error.rs:23-34). */
typedef struct {
    uint64_t seq;     /* sequence index (meta builders, block-table check) */
    uint64_t tokens;  /* BlockTableTooShort.tokens */
    uint64_t needed;  /* BlockTableTooShort.needed */
    uint64_t have;    /* BlockTableTooShort.have */
    uint64_t value;   /* offending slot or block id */
    uint64_t limit;   /* num_slots or num_blocks */
} vo_oracle_err;

/* ---- testutil.rs ---------------------------------------------------- */

/* testutil.rs:34-44: uniform values in [-1, 1) from Knuth's MMIX LCG. */
void vo_oracle_rand_vec(uint64_t seed, uint64_t n, float *out);

/* testutil.rs:94-98: max|a-b| / max(max|b|, 1e-30), folded in f32. */
float vo_oracle_max_rel_diff(const float *a, const float *b, uint64_t n);

/* ---- backend/paged.rs ---------------------------------------------- */

/* paged.rs:48-52 */
uint32_t vo_oracle_slot_of(const uint32_t *table, uint64_t pos, uint64_t block_size);

/* paged.rs:64-80: 0 if the table covers `tokens`, else
 * VO_ORACLE_BLOCK_TABLE_TOO_SHORT with needed/have filled in. */
int vo_oracle_check_covers(uint64_t table_len, uint64_t tokens, uint64_t block_size,
                           vo_oracle_err *err);

/* paged.rs:117-143 (PrefillMeta::new).  Output arrays are sized by the
 * caller: seq_row_starts [S+1], positions/slot_mapping/row_seq/row_num_keys
 * [T] with T = sum(num_new). */
int vo_oracle_prefill_meta(uint64_t num_seqs, const uint64_t *context_lens,
                           const uint64_t *num_new, const uint64_t *table_off,
                           const uint32_t *tables, uint64_t block_size,
                           uint64_t *seq_row_starts, uint32_t *positions,
                           uint32_t *slot_mapping, uint64_t *row_seq,
                           uint64_t *row_num_keys, vo_oracle_err *err);

/* paged.rs:154-159 (PrefillMeta::last_rows). */
void vo_oracle_last_rows(const uint64_t *seq_row_starts, uint64_t num_seqs, uint32_t *out);

/* paged.rs:189-209 (DecodeMeta::new).  Outputs are [S]. */
int vo_oracle_decode_meta(uint64_t num_seqs, const uint64_t *context_lens,
                          const uint64_t *table_off, const uint32_t *tables,
                          uint64_t block_size, uint32_t *positions,
                          uint32_t *slot_mapping, uint64_t *row_seq,
                          uint64_t *row_num_keys, vo_oracle_err *err);

/* ---- backend/cpu/mod.rs and backend/cpu/attention.rs --------------- */

/* cpu/mod.rs:95-110: 16 independent partial sums, summed in lane order,
 * then the scalar remainder. */
float vo_oracle_dot(const float *a, const float *b, uint64_t n);

/* cpu/mod.rs:257-285 (write_kv).  Pool layer is [num_slots, slot_width]
 * (paged.rs:25-28).  All slots are range-checked before any write. */
int vo_oracle_write_kv(float *pool_keys, float *pool_values, uint64_t num_slots,
                       uint64_t slot_width, const float *keys, const float *values,
                       const uint32_t *slots, uint64_t rows, vo_oracle_err *err);

/* attention.rs:132-147: every entry of every table < num_blocks. */
int vo_oracle_check_block_tables(uint64_t num_seqs, const uint64_t *table_off,
                                 const uint32_t *tables, uint64_t num_blocks,
                                 vo_oracle_err *err);

/* attention.rs:44-128 (paged_attention + attend_one_row).  queries/output
 * [rows, num_heads*head_dim]; pool_keys/pool_values are one layer,
 * [num_slots, kv_heads*head_dim].  Rows run on `threads` worker threads
 * (rayon's row parallelism, attention.rs:54-71); results do not depend on
 * the thread count. */
void vo_oracle_paged_attention(const float *queries, float *output,
                               const float *pool_keys, const float *pool_values,
                               uint64_t num_heads, uint64_t num_kv_heads,
                               uint64_t head_dim, uint64_t block_size,
                               const uint64_t *table_off, const uint32_t *tables,
                               const uint64_t *row_seq, const uint64_t *row_num_keys,
                               uint64_t rows, int threads);

/* cpu/tests.rs:184-208 (naive_attend), with the shape as parameters:
 * naive causal GQA attention in f64 for one query row at `pos` over one
 * sequence's contiguous K/V [len, kv_heads*head_dim].  out [num_heads*head_dim]. */
void vo_oracle_naive_attend_f64(const float *q, const float *seq_k, const float *seq_v,
                                uint64_t pos, uint64_t num_heads, uint64_t num_kv_heads,
                                uint64_t head_dim, float *out);

/* Split-K combine (no reference counterpart; the math of merging softmax
 * partials).  For one (row, head): m[i], l[i] and acc[i][head_dim] are the
 * running max, exp-sum and unnormalised output of split i, all in the
 * natural-exp domain.  out = sum_i e^{m_i-M} acc_i / sum_i e^{m_i-M} l_i. */
void vo_oracle_splitk_combine(uint64_t splits, uint64_t head_dim, const float *m,
                              const float *l, const float *acc, float *out);

/* ---- backend/cpu/rope.rs --------------------------------------------- */

/* rope.rs:36-60 (llama3_inv_freq): out[i], i < head_dim/2, the Llama 3 scaled
 * inverse frequencies.  theta, factor, low, high are the config's f64
 * values, narrowed to f32 as the reference does; old_ctx is
 * original_max_position_embeddings. */
void vo_oracle_rope_inv_freq(uint64_t head_dim, double theta, double factor, double low,
                             double high, uint64_t old_ctx, float *out);

/* rope.rs:62-84 (RopeTable::new): cos, sin [max_len][half], theta = p * f. */
void vo_oracle_rope_table(const float *inv_freq, uint64_t half, uint64_t max_len, float *cos_out,
                          float *sin_out);

/* rope.rs:86-100 (RopeTable::apply) on rows [rows][cols]: each head of width
 * 2*half rotated at positions[r]. */
void vo_oracle_rope_apply(float *x, uint64_t rows, uint64_t cols, const uint32_t *positions,
                          const float *cos_tab, const float *sin_tab, uint64_t half);

/* ---- the rest of the layer: backend/cpu/mod.rs ---------------------- */

enum { VO_ORACLE_NAN = 10 };

/* cpu/mod.rs:172-180 (embed): out[r] = table[tokens[r]], table [vocab, hidden]. */
void vo_oracle_embed(const float *table, uint64_t hidden, const uint32_t *tokens, uint64_t rows,
                     float *out);

/* cpu/mod.rs:182-197 (rmsnorm): mean_square = dot(x, x) / hidden (the 16-lane
 * dot), inv_rms = 1 / sqrt(mean_square + eps), out = w * (x * inv_rms). */
void vo_oracle_rmsnorm(const float *x, uint64_t rows, uint64_t hidden, const float *w, float eps,
                       float *out);

/* cpu/mod.rs:199-229 (matmul): out[r][o] = dot(x[r], w[o]) for x [rows, in],
 * w [out_features, in].  Output columns are split over `threads` workers
 * (rayon's weight-row chunks); each element is one dot, so the result does
 * not depend on the thread count. */
void vo_oracle_matmul(const float *x, uint64_t rows, uint64_t in_features, const float *w,
                      uint64_t out_features, float *out, int threads);

/* cpu/mod.rs:341-349 (silu_mul): gate[i] = gate[i] / (1 + exp(-gate[i])) * up[i]. */
void vo_oracle_silu_mul(float *gate, const float *up, uint64_t n);

/* cpu/mod.rs:351-358 (add): sum[i] += x[i]. */
void vo_oracle_add(float *sum, const float *x, uint64_t n);

/* cpu/mod.rs:360-368 (gather_rows): out[i] = x[rows[i]], rows of width cols. */
void vo_oracle_gather_rows(const float *x, uint64_t cols, const uint32_t *rows, uint64_t n,
                           float *out);

/* cpu/mod.rs:370-388 (argmax): per row the first index of the maximum
 * (strict '>' from index 0); VO_ORACLE_NAN when a NaN is met, scanning rows
 * in order and each row from its start. */
int vo_oracle_argmax(const float *x, uint64_t rows, uint64_t cols, uint32_t *out);

#ifdef __cplusplus
}
#endif

#endif /* VO_ORACLE_H */

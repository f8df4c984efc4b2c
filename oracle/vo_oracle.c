/*
 * vo_oracle.c -- CPU restatement of vllm-oxide's paged-attention path.
 *
 * TEST INFRASTRUCTURE ONLY (see vo_oracle.h).  Built with
 * -O3 -ffp-contract=off and without -ffast-math so that every f32 operation
 * happens in the order and rounding the Rust reference uses.
 *
 * Reference files (crates/engine/src/ in KamdynS/vLLM-oxide):
 *   testutil.rs           rand_vec, max_rel_diff
 *   backend/paged.rs      slot_of, check_covers, PrefillMeta, DecodeMeta
 *   backend/cpu/mod.rs    dot, write_kv
 *   backend/cpu/attention.rs  paged_attention, attend_one_row,
 *                             check_block_tables
 *   backend/cpu/tests.rs  naive_attend (the reference's f64 test oracle)
 *   backend/cpu/rope.rs   llama3_inv_freq, RopeTable::new / apply
 *   backend/cpu/mod.rs    embed, rmsnorm, matmul, silu_mul, add, gather_rows,
 *                         argmax (the layer around attention)
 */
#include "vo_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ---- testutil.rs ---------------------------------------------------- */

/* testutil.rs:34-44.  The state update wraps mod 2^64, which is what
 * uint64_t arithmetic does in C. */
void vo_oracle_rand_vec(uint64_t seed, uint64_t n, float *out) {
    uint64_t s = seed * 0x9E3779B97F4A7C15ull + 1ull;
    for (uint64_t i = 0; i < n; ++i) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        float top24 = (float)(s >> 40);
        out[i] = (top24 / 16777216.0f) * 2.0f - 1.0f;
    }
}

/* testutil.rs:94-98.  Rust's f32::max returns the non-NaN operand, as
 * fmaxf does. */
float vo_oracle_max_rel_diff(const float *a, const float *b, uint64_t n) {
    float scale = 0.0f;
    for (uint64_t i = 0; i < n; ++i) scale = fmaxf(scale, fabsf(b[i]));
    scale = fmaxf(scale, 1e-30f);
    float diff = 0.0f;
    for (uint64_t i = 0; i < n; ++i) diff = fmaxf(diff, fabsf(a[i] - b[i]));
    return diff / scale;
}

/* ---- backend/paged.rs ---------------------------------------------- */

/* paged.rs:48-52: table[pos / bs] * bs + pos % bs, in u32. */
uint32_t vo_oracle_slot_of(const uint32_t *table, uint64_t pos, uint64_t block_size) {
    uint32_t block = table[pos / block_size];
    uint32_t offset_in_block = (uint32_t)(pos % block_size);
    return block * (uint32_t)block_size + offset_in_block;
}

/* paged.rs:64-80: needed = ceil(tokens / bs). */
int vo_oracle_check_covers(uint64_t table_len, uint64_t tokens, uint64_t block_size,
                           vo_oracle_err *err) {
    uint64_t needed = (tokens + block_size - 1) / block_size;
    if (table_len < needed) {
        if (err) {
            err->tokens = tokens;
            err->needed = needed;
            err->have = table_len;
        }
        return VO_ORACLE_BLOCK_TABLE_TOO_SHORT;
    }
    return VO_ORACLE_OK;
}

/* paged.rs:117-143.  Rows are laid out sequence after sequence; for each
 * sequence the coverage check of context_len + num_new comes first, then one
 * row per new position. */
int vo_oracle_prefill_meta(uint64_t num_seqs, const uint64_t *context_lens,
                           const uint64_t *num_new, const uint64_t *table_off,
                           const uint32_t *tables, uint64_t block_size,
                           uint64_t *seq_row_starts, uint32_t *positions,
                           uint32_t *slot_mapping, uint64_t *row_seq,
                           uint64_t *row_num_keys, vo_oracle_err *err) {
    uint64_t t = 0;
    seq_row_starts[0] = 0;
    for (uint64_t s = 0; s < num_seqs; ++s) {
        const uint32_t *table = tables + table_off[s];
        uint64_t table_len = table_off[s + 1] - table_off[s];
        uint64_t total_len = context_lens[s] + num_new[s];
        int rc = vo_oracle_check_covers(table_len, total_len, block_size, err);
        if (rc != VO_ORACLE_OK) {
            if (err) err->seq = s;
            return rc;
        }
        for (uint64_t pos = context_lens[s]; pos < total_len; ++pos, ++t) {
            positions[t] = (uint32_t)pos;
            slot_mapping[t] = vo_oracle_slot_of(table, pos, block_size);
            row_seq[t] = s;
            row_num_keys[t] = pos + 1;
        }
        seq_row_starts[s + 1] = t;
    }
    return VO_ORACLE_OK;
}

/* paged.rs:154-159 */
void vo_oracle_last_rows(const uint64_t *seq_row_starts, uint64_t num_seqs, uint32_t *out) {
    for (uint64_t s = 0; s < num_seqs; ++s) out[s] = (uint32_t)(seq_row_starts[s + 1] - 1);
}

/* paged.rs:189-209 */
int vo_oracle_decode_meta(uint64_t num_seqs, const uint64_t *context_lens,
                          const uint64_t *table_off, const uint32_t *tables,
                          uint64_t block_size, uint32_t *positions,
                          uint32_t *slot_mapping, uint64_t *row_seq,
                          uint64_t *row_num_keys, vo_oracle_err *err) {
    for (uint64_t s = 0; s < num_seqs; ++s) {
        const uint32_t *table = tables + table_off[s];
        uint64_t table_len = table_off[s + 1] - table_off[s];
        uint64_t pos = context_lens[s];
        int rc = vo_oracle_check_covers(table_len, pos + 1, block_size, err);
        if (rc != VO_ORACLE_OK) {
            if (err) err->seq = s;
            return rc;
        }
        positions[s] = (uint32_t)pos;
        slot_mapping[s] = vo_oracle_slot_of(table, pos, block_size);
        row_seq[s] = s;
        row_num_keys[s] = pos + 1;
    }
    return VO_ORACLE_OK;
}

/* ---- backend/cpu/mod.rs -------------------------------------------- */

#define DOT_LANES 16 /* cpu/mod.rs:26-29 */

/* cpu/mod.rs:95-110.  Rust's f32 `Sum` folds from -0.0; the partials are
 * never -0.0 (they start at +0.0 and x + (-x) rounds to +0.0), so the start
 * value does not change any result. */
float vo_oracle_dot(const float *a, const float *b, uint64_t n) {
    float partial[DOT_LANES];
    for (int lane = 0; lane < DOT_LANES; ++lane) partial[lane] = 0.0f;
    uint64_t chunks = n / DOT_LANES;
    for (uint64_t c = 0; c < chunks; ++c) {
        const float *ac = a + c * DOT_LANES;
        const float *bc = b + c * DOT_LANES;
        for (int lane = 0; lane < DOT_LANES; ++lane) partial[lane] += ac[lane] * bc[lane];
    }
    float sum = -0.0f;
    for (int lane = 0; lane < DOT_LANES; ++lane) sum += partial[lane];
    for (uint64_t i = chunks * DOT_LANES; i < n; ++i) sum += a[i] * b[i];
    return sum;
}

/* cpu/mod.rs:257-285.  The range check covers every slot before the first
 * copy; copies go in row order, so a repeated slot keeps the later row. */
int vo_oracle_write_kv(float *pool_keys, float *pool_values, uint64_t num_slots,
                       uint64_t slot_width, const float *keys, const float *values,
                       const uint32_t *slots, uint64_t rows, vo_oracle_err *err) {
    for (uint64_t r = 0; r < rows; ++r) {
        if ((uint64_t)slots[r] >= num_slots) {
            if (err) {
                err->value = slots[r];
                err->limit = num_slots;
            }
            return VO_ORACLE_SLOT_OUT_OF_RANGE;
        }
    }
    for (uint64_t r = 0; r < rows; ++r) {
        uint64_t dst = (uint64_t)slots[r] * slot_width;
        memcpy(pool_keys + dst, keys + r * slot_width, slot_width * sizeof(float));
        memcpy(pool_values + dst, values + r * slot_width, slot_width * sizeof(float));
    }
    return VO_ORACLE_OK;
}

/* ---- backend/cpu/attention.rs -------------------------------------- */

/* attention.rs:132-147: the whole of every table, not just the used prefix. */
int vo_oracle_check_block_tables(uint64_t num_seqs, const uint64_t *table_off,
                                 const uint32_t *tables, uint64_t num_blocks,
                                 vo_oracle_err *err) {
    for (uint64_t s = 0; s < num_seqs; ++s) {
        for (uint64_t i = table_off[s]; i < table_off[s + 1]; ++i) {
            if ((uint64_t)tables[i] >= num_blocks) {
                if (err) {
                    err->seq = s;
                    err->value = tables[i];
                    err->limit = num_blocks;
                }
                return VO_ORACLE_BLOCK_OUT_OF_RANGE;
            }
        }
    }
    return VO_ORACLE_OK;
}

typedef struct {
    const float *queries;
    float *output;
    const float *keys;
    const float *values;
    uint64_t num_heads, num_kv_heads, head_dim, block_size;
    const uint64_t *table_off;
    const uint32_t *tables;
    const uint64_t *row_seq;
    const uint64_t *row_num_keys;
    uint64_t rows;
    uint64_t max_keys;
    atomic_uint_fast64_t next_row;
} attention_job;

/* attention.rs:76-128 for one row, all heads.  `scores` holds num_keys f32. */
static void attend_one_row(const attention_job *job, uint64_t row, float *scores) {
    const uint64_t head_dim = job->head_dim;
    const uint64_t heads_per_kv_head = job->num_heads / job->num_kv_heads;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const uint64_t slot_width = job->num_kv_heads * head_dim;
    const uint64_t row_width = job->num_heads * head_dim;
    const float *query_row = job->queries + row * row_width;
    float *out_row = job->output + row * row_width;
    const uint64_t seq = job->row_seq[row];
    const uint32_t *block_table = job->tables + job->table_off[seq];
    const uint64_t num_keys = job->row_num_keys[row];

    for (uint64_t head = 0; head < job->num_heads; ++head) {
        const uint64_t kv_head = head / heads_per_kv_head;
        const float *query = query_row + head * head_dim;

        /* Pass 1: a score per key (attention.rs:102-107). */
        for (uint64_t j = 0; j < num_keys; ++j) {
            uint64_t slot = vo_oracle_slot_of(block_table, j, job->block_size);
            const float *key = job->keys + slot * slot_width + kv_head * head_dim;
            scores[j] = vo_oracle_dot(query, key, head_dim) * scale;
        }

        /* Softmax with the max subtracted (attention.rs:109-115). */
        float max_score = -INFINITY;
        for (uint64_t j = 0; j < num_keys; ++j) max_score = fmaxf(max_score, scores[j]);
        float total = 0.0f;
        for (uint64_t j = 0; j < num_keys; ++j) {
            scores[j] = expf(scores[j] - max_score);
            total += scores[j];
        }

        /* Pass 2: weighted sum of values (attention.rs:117-126). */
        float *out_head = out_row + head * head_dim;
        for (uint64_t d = 0; d < head_dim; ++d) out_head[d] = 0.0f;
        for (uint64_t j = 0; j < num_keys; ++j) {
            float weight = scores[j] / total;
            uint64_t slot = vo_oracle_slot_of(block_table, j, job->block_size);
            const float *value = job->values + slot * slot_width + kv_head * head_dim;
            for (uint64_t d = 0; d < head_dim; ++d) out_head[d] += weight * value[d];
        }
    }
}

/* Row-parallel worker: rows are handed out one at a time, as rayon's work
 * stealing over par_chunks_mut(row_width) does (attention.rs:54-71).  Each
 * worker owns one scores buffer, as for_each_init gives each rayon worker. */
static void *attention_worker(void *arg) {
    attention_job *job = (attention_job *)arg;
    float *scores = (float *)malloc((job->max_keys ? job->max_keys : 1) * sizeof(float));
    if (!scores) return NULL;
    for (;;) {
        uint64_t row = atomic_fetch_add(&job->next_row, 1);
        if (row >= job->rows) break;
        attend_one_row(job, row, scores);
    }
    free(scores);
    return NULL;
}

void vo_oracle_paged_attention(const float *queries, float *output,
                               const float *pool_keys, const float *pool_values,
                               uint64_t num_heads, uint64_t num_kv_heads,
                               uint64_t head_dim, uint64_t block_size,
                               const uint64_t *table_off, const uint32_t *tables,
                               const uint64_t *row_seq, const uint64_t *row_num_keys,
                               uint64_t rows, int threads) {
    attention_job job;
    job.queries = queries;
    job.output = output;
    job.keys = pool_keys;
    job.values = pool_values;
    job.num_heads = num_heads;
    job.num_kv_heads = num_kv_heads;
    job.head_dim = head_dim;
    job.block_size = block_size;
    job.table_off = table_off;
    job.tables = tables;
    job.row_seq = row_seq;
    job.row_num_keys = row_num_keys;
    job.rows = rows;
    job.max_keys = 0;
    for (uint64_t r = 0; r < rows; ++r)
        if (row_num_keys[r] > job.max_keys) job.max_keys = row_num_keys[r];
    atomic_init(&job.next_row, 0);

    if (threads < 1) threads = 1;
    if ((uint64_t)threads > rows) threads = rows ? (int)rows : 1;
    if (threads == 1) {
        attention_worker(&job);
        return;
    }
    pthread_t *tids = (pthread_t *)malloc((size_t)threads * sizeof(pthread_t));
    int started = 0;
    for (int i = 0; i < threads; ++i) {
        if (pthread_create(&tids[i], NULL, attention_worker, &job) == 0) ++started;
    }
    if (started == 0) attention_worker(&job);
    for (int i = 0; i < started; ++i) pthread_join(tids[i], NULL);
    free(tids);
}

/* cpu/tests.rs:184-208, shape-parametrised: scores and weights in f64,
 * summed in key order, each output cast to f32 once at the end. */
void vo_oracle_naive_attend_f64(const float *q, const float *seq_k, const float *seq_v,
                                uint64_t pos, uint64_t num_heads, uint64_t num_kv_heads,
                                uint64_t head_dim, float *out) {
    const uint64_t w = num_kv_heads * head_dim;
    const uint64_t group = num_heads / num_kv_heads;
    const uint64_t n = pos + 1;
    double *scores = (double *)malloc(n * sizeof(double));
    if (!scores) return;
    for (uint64_t h = 0; h < num_heads; ++h) {
        const uint64_t g = h / group;
        for (uint64_t j = 0; j < n; ++j) {
            double acc = 0.0;
            for (uint64_t d = 0; d < head_dim; ++d)
                acc += (double)q[h * head_dim + d] * (double)seq_k[j * w + g * head_dim + d];
            scores[j] = acc / sqrt((double)head_dim);
        }
        double m = -INFINITY;
        for (uint64_t j = 0; j < n; ++j) m = fmax(m, scores[j]);
        double z = 0.0;
        for (uint64_t j = 0; j < n; ++j) {
            scores[j] = exp(scores[j] - m);
            z += scores[j];
        }
        for (uint64_t d = 0; d < head_dim; ++d) {
            double acc = 0.0;
            for (uint64_t j = 0; j < n; ++j)
                acc += scores[j] / z * (double)seq_v[j * w + g * head_dim + d];
            out[h * head_dim + d] = (float)acc;
        }
    }
    free(scores);
}

/* Merge of softmax partials, computed in f64.  A split with m = -inf holds
 * no keys and contributes nothing. */
void vo_oracle_splitk_combine(uint64_t splits, uint64_t head_dim, const float *m,
                              const float *l, const float *acc, float *out) {
    double big = -INFINITY;
    for (uint64_t i = 0; i < splits; ++i) big = fmax(big, (double)m[i]);
    double denom = 0.0;
    for (uint64_t i = 0; i < splits; ++i)
        if (m[i] != -INFINITY) denom += exp((double)m[i] - big) * (double)l[i];
    for (uint64_t d = 0; d < head_dim; ++d) {
        double num = 0.0;
        for (uint64_t i = 0; i < splits; ++i)
            if (m[i] != -INFINITY) num += exp((double)m[i] - big) * (double)acc[i * head_dim + d];
        out[d] = (float)(num / denom);
    }
}


/* ---- backend/cpu/rope.rs --------------------------------------------- */

/* rope.rs:36-60.  Every operation is the reference's f32 operation in the
 * reference's order: `1.0 / base.powf((2 * i) as f32 / d as f32)`,
 * `2.0 * PI / inv`, and `(1.0 - smooth) * inv / factor + smooth * inv`
 * evaluated left to right (no contraction: -ffp-contract=off). */
void vo_oracle_rope_inv_freq(uint64_t head_dim, double theta, double factor, double low,
                             double high, uint64_t old_ctx, float *out) {
    const float d = (float)head_dim;
    const float base = (float)theta;
    const float f = (float)factor;
    const float lo = (float)low;
    const float hi = (float)high;
    const float ctx = (float)old_ctx;
    const float low_freq_wavelen = ctx / lo;
    const float high_freq_wavelen = ctx / hi;
    const float pi = 3.14159265358979323846f; /* std::f32::consts::PI */
    for (uint64_t i = 0; i < head_dim / 2; ++i) {
        const float inv = 1.0f / powf(base, (float)(2 * i) / d);
        const float wavelen = 2.0f * pi / inv;
        float r;
        if (wavelen < high_freq_wavelen) {
            r = inv;
        } else if (wavelen > low_freq_wavelen) {
            r = inv / f;
        } else {
            const float smooth = (ctx / wavelen - lo) / (hi - lo);
            r = (1.0f - smooth) * inv / f + smooth * inv;
        }
        out[i] = r;
    }
}

/* rope.rs:62-84: theta = p as f32 * inv_freq[i]; cos and sin from libm. */
void vo_oracle_rope_table(const float *inv_freq, uint64_t half, uint64_t max_len, float *cos_out,
                          float *sin_out) {
    for (uint64_t p = 0; p < max_len; ++p) {
        for (uint64_t i = 0; i < half; ++i) {
            const float th = (float)p * inv_freq[i];
            cos_out[p * half + i] = cosf(th);
            sin_out[p * half + i] = sinf(th);
        }
    }
}

/* rope.rs:86-100: x1' = a*cos - b*sin, x2' = b*cos + a*sin per pair. */
void vo_oracle_rope_apply(float *x, uint64_t rows, uint64_t cols, const uint32_t *positions,
                          const float *cos_tab, const float *sin_tab, uint64_t half) {
    for (uint64_t r = 0; r < rows; ++r) {
        const float *c = cos_tab + (uint64_t)positions[r] * half;
        const float *sn = sin_tab + (uint64_t)positions[r] * half;
        for (uint64_t h0 = 0; h0 + 2 * half <= cols; h0 += 2 * half) {
            float *x1 = x + r * cols + h0;
            float *x2 = x1 + half;
            for (uint64_t i = 0; i < half; ++i) {
                const float a = x1[i], b = x2[i];
                x1[i] = a * c[i] - b * sn[i];
                x2[i] = b * c[i] + a * sn[i];
            }
        }
    }
}

/* ---- the rest of the layer: backend/cpu/mod.rs ---------------------- */

/* cpu/mod.rs:172-180. */
void vo_oracle_embed(const float *table, uint64_t hidden, const uint32_t *tokens, uint64_t rows,
                     float *out) {
    for (uint64_t r = 0; r < rows; ++r)
        memcpy(out + r * hidden, table + (uint64_t)tokens[r] * hidden, hidden * sizeof(float));
}

/* cpu/mod.rs:182-197.  `dot(x_row, x_row) / hidden as f32`, then
 * `1.0 / (mean_square + eps).sqrt()`, then `w * (x * inv_rms)`. */
void vo_oracle_rmsnorm(const float *x, uint64_t rows, uint64_t hidden, const float *w, float eps,
                       float *out) {
    for (uint64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * hidden;
        float *o = out + r * hidden;
        float mean_square = vo_oracle_dot(xr, xr, hidden) / (float)hidden;
        float inv_rms = 1.0f / sqrtf(mean_square + eps);
        for (uint64_t j = 0; j < hidden; ++j) o[j] = w[j] * (xr[j] * inv_rms);
    }
}

typedef struct {
    const float *x, *w;
    float *out;
    uint64_t rows, in, out_f, o_begin, o_end;
} matmul_job;

static void *matmul_worker(void *arg) {
    const matmul_job *j = (const matmul_job *)arg;
    for (uint64_t o = j->o_begin; o < j->o_end; ++o) {
        const float *wr = j->w + o * j->in;
        for (uint64_t r = 0; r < j->rows; ++r)
            j->out[r * j->out_f + o] = vo_oracle_dot(j->x + r * j->in, wr, j->in);
    }
    return NULL;
}

/* cpu/mod.rs:199-229: element [r][o] = dot(x_row r, weight_row o). */
void vo_oracle_matmul(const float *x, uint64_t rows, uint64_t in_features, const float *w,
                      uint64_t out_features, float *out, int threads) {
    if (threads < 1) threads = 1;
    if ((uint64_t)threads > out_features) threads = out_features ? (int)out_features : 1;
    matmul_job jobs[64];
    pthread_t tid[64];
    if (threads > 64) threads = 64;
    uint64_t per = (out_features + (uint64_t)threads - 1) / (uint64_t)threads;
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        uint64_t b = (uint64_t)t * per, e = b + per;
        if (e > out_features) e = out_features;
        if (b >= e) break;
        jobs[t] = (matmul_job){x, w, out, rows, in_features, out_features, b, e};
        if (t == 0 || pthread_create(&tid[t], NULL, matmul_worker, &jobs[t]) != 0) {
            if (t != 0) matmul_worker(&jobs[t]);
            tid[t] = 0;
        }
        started = t + 1;
    }
    if (started > 0) matmul_worker(&jobs[0]);
    for (int t = 1; t < started; ++t)
        if (tid[t]) pthread_join(tid[t], NULL);
}

/* cpu/mod.rs:341-349: `*g = *g / (1.0 + (-*g).exp()) * u`. */
void vo_oracle_silu_mul(float *gate, const float *up, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) gate[i] = gate[i] / (1.0f + expf(-gate[i])) * up[i];
}

/* cpu/mod.rs:351-358. */
void vo_oracle_add(float *sum, const float *x, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) sum[i] += x[i];
}

/* cpu/mod.rs:360-368. */
void vo_oracle_gather_rows(const float *x, uint64_t cols, const uint32_t *rows, uint64_t n,
                           float *out) {
    for (uint64_t i = 0; i < n; ++i)
        memcpy(out + i * cols, x + (uint64_t)rows[i] * cols, cols * sizeof(float));
}

/* cpu/mod.rs:370-388.  The reference chunks rows*cols elements by
 * `cols.max(1)`: with cols == 0 there are no elements and no rows. */
int vo_oracle_argmax(const float *x, uint64_t rows, uint64_t cols, uint32_t *out) {
    if (cols == 0) return VO_ORACLE_OK;
    for (uint64_t r = 0; r < rows; ++r) {
        const float *row = x + r * cols;
        uint64_t best = 0;
        for (uint64_t i = 0; i < cols; ++i) {
            if (isnan(row[i])) return VO_ORACLE_NAN;
            if (row[i] > row[best]) best = i;
        }
        out[r] = (uint32_t)best;
    }
    return VO_ORACLE_OK;
}

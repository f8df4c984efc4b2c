// vo_layer.cpp -- the C ABI of the Llama layer's ops around attention:
// token upload, embed, rmsnorm (alone and over the LM head's rows),
// gather_rows, add, silu_mul and argmax.  Checks mirror crates/engine/src/arena/ops.rs and
// backend/cpu/mod.rs; kernels are in kernels/layer_ops.hip.
#include <algorithm>
#include <cstring>
#include <string>

#include "vo_backend.hpp"

using namespace vo;

namespace {

std::string shape2(uint64_t r, uint64_t c) {
    return "[" + std::to_string(r) + ", " + std::to_string(c) + "]";
}

vo_status check_u32(const char *what, uint64_t v) {
    if (v > 0xffffffffull) return fail_capacity(what, v, 0xffffffffull);
    return VO_OK;
}

}  // namespace

extern "C" int32_t vo_step_meta_upload_tokens(vo_step_meta *m, const uint32_t *tokens,
                                              uint64_t num_tokens, void *stream) {
    const char *op = "embed";
    if (!m) return fail_argument(op, "null meta");
    if (num_tokens > m->max_rows) return fail_capacity("tokens per step", num_tokens, m->max_rows);
    if (num_tokens && !tokens) return fail_argument(op, "null tokens");
    DeviceGuard guard(m->device);
    m->tokens.assign(tokens, tokens + num_tokens);
    m->has_tokens = true;
    if (num_tokens) {
        // Double-buffered pinned staging: waits only if the copy out of this
        // buffer, two uploads ago, has not run yet.
        uint8_t *host;
        hipError_t err = m->tokens_stage.acquire(&host);
        if (err == hipSuccess) {
            std::memcpy(host, tokens, num_tokens * sizeof(uint32_t));
            err = m->tokens_stage.commit(m->d_tokens, num_tokens * sizeof(uint32_t),
                                         static_cast<hipStream_t>(stream));
        }
        if (err != hipSuccess) return fail_device(op, err, hipGetErrorString(err));
    }
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_embed(const void *table, uint64_t vocab, uint64_t hidden,
                            const vo_step_meta *m, uint64_t rows, float *out, void *stream) {
    const char *op = "embed";
    if (!m) return fail_argument(op, "null meta");
    if (!m->has_tokens || rows != m->tokens.size())
        return fail_shape(op, "out has " + std::to_string(rows) + " rows, " +
                                  std::to_string(m->has_tokens ? m->tokens.size() : 0) +
                                  " tokens uploaded");
    // arena/ops.rs:33-38: the first token past the vocabulary.
    for (uint32_t t : m->tokens)
        if (t >= vocab)
            return fail_shape(op, "token " + std::to_string(t) + " >= vocab " + std::to_string(vocab));
    if (rows == 0 || hidden == 0) {
        clear_error();
        return VO_OK;
    }
    if (!table || !out) return fail_argument(op, "null table or output");
    if (vo_status rc = check_u32("hidden size (u32)", hidden)) return rc;
    if (vo_status rc = check_u32("rows (u32)", rows)) return rc;
    if (hidden % 8 == 0 && (!aligned16(table) || !aligned16(out)))
        return fail_argument(op, "table and output must be 16-byte aligned");
    DeviceGuard guard(m->device);
    return device_status(op, kernels::launch_embed(static_cast<const uint16_t *>(table),
                                                   static_cast<uint32_t>(hidden), m->d_tokens,
                                                   static_cast<uint32_t>(rows), out,
                                                   static_cast<hipStream_t>(stream)));
}

namespace {

vo_status rmsnorm_common(const char *op, const float *x, uint64_t rows, uint64_t cols,
                         const void *weight, uint64_t weight_len, const void *out,
                         uint64_t out_rows) {
    // arena/ops.rs:50-56
    if (weight_len != cols)
        return fail_shape(op, "x " + shape2(rows, cols) + ", weight [" + std::to_string(weight_len) + "]");
    if (out_rows == 0 || cols == 0) return VO_OK;
    if (!x || !weight || !out) return fail_argument(op, "null x, weight or output");
    if (vo_status rc = check_u32("hidden size (u32)", cols)) return rc;
    if (vo_status rc = check_u32("rows (u32)", std::max(rows, out_rows))) return rc;
    if (cols % 8 == 0 && (!aligned16(x) || !aligned16(weight) || !aligned16(out)))
        return fail_argument(op, "x, weight and output must be 16-byte aligned");
    if (overlaps(x, rows * cols * 4, out, out_rows * cols * 2))
        return fail_shape(op, "output overlaps x");
    return VO_OK;
}

}  // namespace

extern "C" int32_t vo_rmsnorm(const float *x, uint64_t rows, uint64_t cols, const void *weight,
                              uint64_t weight_len, float eps, void *out, void *stream) {
    const char *op = "rmsnorm";
    if (vo_status rc = rmsnorm_common(op, x, rows, cols, weight, weight_len, out, rows)) return rc;
    if (rows == 0 || cols == 0) {
        clear_error();
        return VO_OK;
    }
    return device_status(op, kernels::launch_rmsnorm(x, static_cast<uint32_t>(cols),
                                                     static_cast<const uint16_t *>(weight), eps,
                                                     nullptr, static_cast<uint32_t>(rows),
                                                     static_cast<uint16_t *>(out),
                                                     static_cast<hipStream_t>(stream)));
}

extern "C" int32_t vo_rmsnorm_last_rows(const float *x, uint64_t rows, uint64_t cols,
                                        const void *weight, uint64_t weight_len, float eps,
                                        const vo_step_meta *m, void *out, void *stream) {
    const char *op = "rmsnorm";
    if (!m) return fail_argument(op, "null meta");
    if ((m->kind != kPrefill && m->kind != kDecode) || !m->last_rows_ok || rows != m->num_rows)
        return fail_shape("gather_rows", "x " + shape2(rows, cols) + ", metadata of " +
                                             std::to_string(m->num_rows) +
                                             " rows without a last row for every sequence");
    if (vo_status rc = rmsnorm_common(op, x, rows, cols, weight, weight_len, out, m->num_seqs))
        return rc;
    if (m->num_seqs == 0 || cols == 0) {
        clear_error();
        return VO_OK;
    }
    DeviceGuard guard(m->device);
    return device_status(op, kernels::launch_rmsnorm(x, static_cast<uint32_t>(cols),
                                                     static_cast<const uint16_t *>(weight), eps,
                                                     m->d_last_rows,
                                                     static_cast<uint32_t>(m->num_seqs),
                                                     static_cast<uint16_t *>(out),
                                                     static_cast<hipStream_t>(stream)));
}

namespace {

// Whether rows [n] are the meta's last rows (PrefillMeta::last_rows,
// paged.rs:153-159; in a decode step every row), so that the meta's device
// copy serves vo_gather_rows.
bool are_last_rows(const vo_step_meta *m, const uint32_t *rows, uint64_t n) {
    if ((m->kind != kPrefill && m->kind != kDecode) || !m->last_rows_ok || !m->d_last_rows ||
        n != m->num_seqs)
        return false;
    for (uint64_t s = 0; s < n; ++s) {
        const uint64_t last = m->kind == kDecode ? s : m->seq_row_starts[s + 1] - 1;
        if (rows[s] != last) return false;
    }
    return true;
}

}  // namespace

extern "C" int32_t vo_gather_rows(const void *x, int32_t dtype, uint64_t rows, uint64_t cols,
                                  const uint32_t *idx, uint64_t num_idx, vo_step_meta *m,
                                  void *out, void *stream) {
    const char *op = "gather_rows";
    if (!m) return fail_argument(op, "null meta");
    if (dtype != VO_DTYPE_BF16 && dtype != VO_DTYPE_F32)
        return fail_argument(op, "dtype must be VO_DTYPE_BF16 or VO_DTYPE_F32");
    if (num_idx && !idx) return fail_argument(op, "null rows");
    // arena/ops.rs:242-244: the first row past x.
    for (uint64_t i = 0; i < num_idx; ++i)
        if (idx[i] >= rows)
            return fail_shape(op, "row " + std::to_string(idx[i]) + " of x " + shape2(rows, cols));
    const uint64_t esize = dtype == VO_DTYPE_BF16 ? 2 : 4;
    const uint64_t row_bytes = cols * esize;
    if (num_idx == 0 || row_bytes == 0) {
        clear_error();
        return VO_OK;
    }
    if (!x || !out) return fail_argument(op, "null x or out");
    if (overlaps(x, rows * row_bytes, out, num_idx * row_bytes))
        return fail_shape(op, "out overlaps x");
    if (num_idx > kU32Limit) return fail_capacity("gather_rows rows (u32)", num_idx, kU32Limit);
    // The kernel copies 4-byte words; a bf16 row of odd width is not whole words.
    if (row_bytes % 4 != 0 || row_bytes / 4 > kU32Limit || (reinterpret_cast<uintptr_t>(x) & 3) ||
        (reinterpret_cast<uintptr_t>(out) & 3))
        return fail_argument(op, "rows must be whole, 4-byte aligned 4-byte words");
    DeviceGuard guard(m->device);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const uint32_t *d_rows = m->d_last_rows;
    if (!are_last_rows(m, idx, num_idx)) {
        if (vo_status rc = aux_upload(m, m->aux_rows, m->aux_rows_valid, m->d_aux_rows, idx,
                                      num_idx, st, op))
            return rc;
        d_rows = m->d_aux_rows;
    }
    const bool vec4 = row_bytes % 16 == 0 && aligned16(x) && aligned16(out);
    return device_status(op, kernels::launch_gather_rows(
                                 x, static_cast<uint32_t>(row_bytes / 4), d_rows,
                                 static_cast<uint32_t>(num_idx), out, vec4, st));
}

extern "C" int32_t vo_add(float *sum, const void *x, int32_t x_dtype, uint64_t rows, uint64_t cols,
                          void *stream) {
    const char *op = "add";
    if (x_dtype != VO_DTYPE_BF16 && x_dtype != VO_DTYPE_F32)
        return fail_argument(op, "x_dtype must be VO_DTYPE_BF16 or VO_DTYPE_F32");
    const uint64_t n = rows * cols;
    if (n == 0) {
        clear_error();
        return VO_OK;
    }
    if (!sum || !x) return fail_argument(op, "null sum or x");
    const uint64_t xb = n * (x_dtype == VO_DTYPE_BF16 ? 2 : 4);
    if (sum != x && overlaps(sum, n * 4, x, xb)) return fail_shape(op, "x overlaps sum");
    return device_status(op, kernels::launch_add(sum, x, x_dtype == VO_DTYPE_BF16, n,
                                                 static_cast<hipStream_t>(stream)));
}

extern "C" int32_t vo_silu_mul(const void *gate, uint64_t gate_ld, const void *up, uint64_t up_ld,
                               uint64_t rows, uint64_t cols, void *out, uint64_t out_ld,
                               void *stream) {
    const char *op = "silu_mul";
    if (gate_ld < cols || up_ld < cols || out_ld < cols)
        return fail_shape(op, "row strides " + std::to_string(gate_ld) + ", " +
                                  std::to_string(up_ld) + ", " + std::to_string(out_ld) +
                                  " below " + std::to_string(cols) + " columns");
    if (rows == 0 || cols == 0) {
        clear_error();
        return VO_OK;
    }
    if (!gate || !up || !out) return fail_argument(op, "null gate, up or output");
    if (vo_status rc = check_u32("silu_mul strides (u32)", std::max({gate_ld, up_ld, out_ld})))
        return rc;
    if (vo_status rc = check_u32("rows (u32)", rows)) return rc;
    const uint64_t span_out = ((rows - 1) * out_ld + cols) * 2;
    const uint64_t span_up = ((rows - 1) * up_ld + cols) * 2;
    const uint64_t span_gate = ((rows - 1) * gate_ld + cols) * 2;
    // The in-place form (out == gate, same stride) is the reference's; any
    // other overlap of out with an input is refused.
    const bool in_place = out == gate && out_ld == gate_ld;
    if ((!in_place && overlaps(out, span_out, gate, span_gate)) || overlaps(out, span_out, up, span_up))
        return fail_shape(op, "output overlaps an input");
    const bool vec8 = cols % 8 == 0 && gate_ld % 8 == 0 && up_ld % 8 == 0 && out_ld % 8 == 0 &&
                      aligned16(gate) && aligned16(up) && aligned16(out);
    return device_status(
        op, kernels::launch_silu_mul(static_cast<const uint16_t *>(gate), static_cast<uint32_t>(gate_ld),
                                     static_cast<const uint16_t *>(up), static_cast<uint32_t>(up_ld),
                                     static_cast<uint32_t>(rows), static_cast<uint32_t>(cols),
                                     static_cast<uint16_t *>(out), static_cast<uint32_t>(out_ld), vec8,
                                     static_cast<hipStream_t>(stream)));
}

extern "C" int32_t vo_argmax(const void *logits, int32_t dtype, uint64_t rows, uint64_t cols,
                             uint32_t *ids, uint32_t *host_ids, void *stream) {
    const char *op = "argmax";
    if (dtype != VO_DTYPE_BF16 && dtype != VO_DTYPE_F32)
        return fail_argument(op, "dtype must be VO_DTYPE_BF16 or VO_DTYPE_F32");
    if (rows == 0) {
        clear_error();
        return VO_OK;
    }
    if (cols == 0) return fail_shape(op, "logits " + shape2(rows, cols) + " have no columns");
    if (!logits || !ids) return fail_argument(op, "null logits or ids");
    if (vo_status rc = check_u32("rows (u32)", rows)) return rc;
    if (cols >= 0xffffffffull) return fail_capacity("argmax columns (u32)", cols, 0xfffffffeull);
    const bool f32 = dtype == VO_DTYPE_F32;
    if (f32 && cols % 4 == 0 && !aligned16(logits))
        return fail_argument(op, "logits must be 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t err = kernels::launch_argmax(logits, f32, static_cast<uint32_t>(rows),
                                            static_cast<uint32_t>(cols), ids, s);
    if (err != hipSuccess || !host_ids) return device_status(op, err);
    err = hipMemcpyAsync(host_ids, ids, rows * sizeof(uint32_t), hipMemcpyDeviceToHost, s);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
    if (err != hipSuccess) return fail_device(op, err, hipGetErrorString(err));
    for (uint64_t r = 0; r < rows; ++r) {
        if (host_ids[r] == 0xffffffffu) {
            Error e;
            e.status = VO_ERR_NAN;
            e.op = op;
            e.message = "argmax: NaN in input";
            return fail(e);
        }
    }
    clear_error();
    return VO_OK;
}

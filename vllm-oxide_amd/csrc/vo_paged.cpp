// vo_paged.cpp -- paged-KV metadata builders and the error state of the C ABI.
//
// Follows crates/engine/src/backend/paged.rs (slot_of :47-52, check_covers
// :64-80, PrefillMeta::new :117-143, last_rows :154-159, DecodeMeta::new
// :189-209) and the error texts of crates/engine/src/error.rs:8-56.
#include "vo_paged.hpp"

#include <cstdio>
#include <cstring>

namespace vo {

namespace {
thread_local Error g_last_error;
}

vo_status fail(const Error &e) {
    g_last_error = e;
    return e.status;
}

void clear_error() { g_last_error = Error{}; }

const Error &last_error() { return g_last_error; }

vo_status fail_shape(const char *op, const std::string &msg) {
    Error e;
    e.status = VO_ERR_SHAPE;
    e.op = op;
    e.message = std::string(op) + ": " + msg;  // error.rs:11 "{op}: {msg}"
    return fail(e);
}

vo_status fail_capacity(const char *what, uint64_t need, uint64_t limit) {
    Error e;
    e.status = VO_ERR_CAPACITY;
    e.op = what;
    e.value = need;
    e.limit = limit;
    // error.rs:13 "{what}: need {need}, limit {limit}"
    e.message = std::string(what) + ": need " + std::to_string(need) + ", limit " +
                std::to_string(limit);
    return fail(e);
}

vo_status fail_device(const char *op, int hip_error, const char *what) {
    Error e;
    e.status = VO_ERR_DEVICE;
    e.op = op;
    e.value = static_cast<uint64_t>(hip_error);
    e.message = std::string(op) + ": HIP error " + std::to_string(hip_error) + " (" +
                (what ? what : "?") + ")";
    return fail(e);
}

vo_status fail_argument(const char *op, const std::string &msg) {
    Error e;
    e.status = VO_ERR_INVALID_ARGUMENT;
    e.op = op;
    e.message = std::string(op) + ": " + msg;
    return fail(e);
}

vo_status fail_unsupported(const char *op, const std::string &msg) {
    Error e;
    e.status = VO_ERR_UNSUPPORTED;
    e.op = op;
    e.message = std::string(op) + ": " + msg;
    return fail(e);
}

vo_status check_covers(const char *op, uint64_t table_len, uint64_t tokens,
                       uint64_t block_size, uint64_t seq) {
    const uint64_t needed = (tokens + block_size - 1) / block_size;
    if (table_len < needed) {
        Error e;
        e.status = VO_ERR_BLOCK_TABLE_TOO_SHORT;
        e.op = op;
        e.seq = seq;
        e.tokens = tokens;
        e.needed = needed;
        e.have = table_len;
        // paged.rs:56
        e.message = std::string(op) + ": block table too short: " + std::to_string(tokens) +
                    " tokens need " + std::to_string(needed) + " blocks, table has " +
                    std::to_string(table_len);
        return fail(e);
    }
    return VO_OK;
}

vo_status check_block_tables(const char *op, uint64_t num_seqs, const uint64_t *table_off,
                             const uint32_t *tables, uint64_t num_blocks) {
    for (uint64_t s = 0; s < num_seqs; ++s) {
        for (uint64_t i = table_off[s]; i < table_off[s + 1]; ++i) {
            if (static_cast<uint64_t>(tables[i]) >= num_blocks) {
                Error e;
                e.status = VO_ERR_BLOCK_OUT_OF_RANGE;
                e.op = op;
                e.seq = s;
                e.value = tables[i];
                e.limit = num_blocks;
                // error.rs:29
                e.message = std::string(op) + ": block " + std::to_string(tables[i]) +
                            " out of range (pool has " + std::to_string(num_blocks) + ")";
                return fail(e);
            }
        }
    }
    return VO_OK;
}

}  // namespace vo

// ---------------------------------------------------------------------------
// C ABI: addressing and metadata builders.
// ---------------------------------------------------------------------------
using namespace vo;

extern "C" uint64_t vo_kv_layout_num_slots(const vo_kv_layout *layout) {
    return layout ? layout->num_blocks * layout->block_size : 0;  // paged.rs:38-40
}

extern "C" uint64_t vo_kv_layout_layer_elems(const vo_kv_layout *layout) {
    // paged.rs:42-44
    return layout ? vo_kv_layout_num_slots(layout) * layout->kv_heads * layout->head_dim : 0;
}

extern "C" int32_t vo_slot_of(const uint32_t *block_table, uint64_t table_len, uint64_t pos,
                              uint64_t block_size, uint32_t *out_slot) {
    if (!block_table || !out_slot || block_size == 0)
        return fail_argument("slot_of", "null table/output or block_size 0");
    if (vo_status rc = check_covers("slot_of", table_len, pos + 1, block_size, 0)) return rc;
    *out_slot = slot_of(block_table, pos, block_size);
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_prefill_meta_build(const vo_prefill_seq *seqs, uint64_t num_seqs,
                                         uint64_t block_size, uint64_t *seq_row_starts,
                                         uint32_t *positions, uint32_t *slot_mapping,
                                         uint64_t *row_seq, uint64_t *row_num_keys) {
    if ((!seqs && num_seqs) || block_size == 0)
        return fail_argument("prefill", "null sequences or block_size 0");
    uint64_t t = 0;
    if (seq_row_starts) seq_row_starts[0] = 0;
    for (uint64_t s = 0; s < num_seqs; ++s) {
        const vo_prefill_seq &seq = seqs[s];
        const uint64_t total_len = seq.context_len + seq.num_new;
        if (vo_status rc = check_covers("prefill", seq.block_table_len, total_len, block_size, s))
            return rc;
        if (seq.block_table_len && !seq.block_table)
            return fail_argument("prefill", "null block table");
        for (uint64_t pos = seq.context_len; pos < total_len; ++pos, ++t) {
            if (positions) positions[t] = static_cast<uint32_t>(pos);
            if (slot_mapping) slot_mapping[t] = slot_of(seq.block_table, pos, block_size);
            if (row_seq) row_seq[t] = s;
            if (row_num_keys) row_num_keys[t] = pos + 1;
        }
        if (seq_row_starts) seq_row_starts[s + 1] = t;
    }
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_decode_meta_build(const vo_decode_seq *seqs, uint64_t num_seqs,
                                        uint64_t block_size, uint32_t *positions,
                                        uint32_t *slot_mapping, uint64_t *row_seq,
                                        uint64_t *row_num_keys) {
    if ((!seqs && num_seqs) || block_size == 0)
        return fail_argument("decode", "null sequences or block_size 0");
    for (uint64_t s = 0; s < num_seqs; ++s) {
        const vo_decode_seq &seq = seqs[s];
        const uint64_t pos = seq.context_len;
        if (vo_status rc = check_covers("decode", seq.block_table_len, pos + 1, block_size, s))
            return rc;
        if (!seq.block_table) return fail_argument("decode", "null block table");
        if (positions) positions[s] = static_cast<uint32_t>(pos);
        if (slot_mapping) slot_mapping[s] = slot_of(seq.block_table, pos, block_size);
        if (row_seq) row_seq[s] = s;
        if (row_num_keys) row_num_keys[s] = pos + 1;
    }
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_last_rows(const uint64_t *seq_row_starts, uint64_t num_seqs,
                                uint32_t *out) {
    if ((!seq_row_starts || !out) && num_seqs)
        return fail_argument("last_rows", "null input or output");
    for (uint64_t s = 0; s < num_seqs; ++s) {
        if (seq_row_starts[s + 1] == 0)
            return fail_shape("last_rows", "sequence " + std::to_string(s) + " has no rows");
        out[s] = static_cast<uint32_t>(seq_row_starts[s + 1] - 1);
    }
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_last_error(vo_error_info *out) {
    const Error &e = last_error();
    if (out) {
        std::memset(out, 0, sizeof(*out));
        out->status = e.status;
        std::snprintf(out->op, sizeof(out->op), "%s", e.op.c_str());
        out->seq = e.seq;
        out->tokens = e.tokens;
        out->needed = e.needed;
        out->have = e.have;
        out->value = e.value;
        out->limit = e.limit;
        std::snprintf(out->message, sizeof(out->message), "%s", e.message.c_str());
    }
    return e.status;
}

extern "C" const char *vo_status_name(int32_t status) {
    switch (status) {
        case VO_OK: return "VO_OK";
        case VO_ERR_SHAPE: return "VO_ERR_SHAPE";
        case VO_ERR_CAPACITY: return "VO_ERR_CAPACITY";
        case VO_ERR_BLOCK_TABLE_TOO_SHORT: return "VO_ERR_BLOCK_TABLE_TOO_SHORT";
        case VO_ERR_SLOT_OUT_OF_RANGE: return "VO_ERR_SLOT_OUT_OF_RANGE";
        case VO_ERR_BLOCK_OUT_OF_RANGE: return "VO_ERR_BLOCK_OUT_OF_RANGE";
        case VO_ERR_DEVICE: return "VO_ERR_DEVICE";
        case VO_ERR_INVALID_ARGUMENT: return "VO_ERR_INVALID_ARGUMENT";
        case VO_ERR_UNSUPPORTED: return "VO_ERR_UNSUPPORTED";
        case VO_ERR_POSITION_OUT_OF_RANGE: return "VO_ERR_POSITION_OUT_OF_RANGE";
        case VO_ERR_NAN: return "VO_ERR_NAN";
        case VO_ERR_OUTSIDE_WORKSPACE: return "VO_ERR_OUTSIDE_WORKSPACE";
        default: return "VO_ERR_UNKNOWN";
    }
}

extern "C" const char *vo_version(void) { return "vo_paged_attention 0.1.0 gfx950"; }

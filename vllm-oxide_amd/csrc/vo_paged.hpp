// vo_paged.hpp -- paged-KV addressing and per-step metadata, host side.
//
// C++ counterpart of crates/engine/src/backend/paged.rs.  Token `pos` of a
// sequence lives at slot table[pos / bs] * bs + pos % bs (paged.rs:47-52).
// A step's tokens are rows, sequence after sequence with no padding; each row
// has a position, a slot, a sequence and a key count = position + 1
// (paged.rs:14-21).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "vo_paged_attention.h"

namespace vo {

// Error state of one failed call, mirroring EngineError (error.rs:8-56).
struct Error {
    vo_status status = VO_OK;
    std::string op;
    uint64_t seq = 0, tokens = 0, needed = 0, have = 0, value = 0, limit = 0;
    std::string message;
};

// Records `e` as the calling thread's last error and returns its status.
vo_status fail(const Error &e);
// Marks the calling thread's last call as successful.
void clear_error();
// The calling thread's last error.
const Error &last_error();

vo_status fail_shape(const char *op, const std::string &msg);
vo_status fail_capacity(const char *what, uint64_t need, uint64_t limit);
vo_status fail_device(const char *op, int hip_error, const char *what);
vo_status fail_argument(const char *op, const std::string &msg);
vo_status fail_unsupported(const char *op, const std::string &msg);

// paged.rs:48-52.  u32 arithmetic, as the reference.
inline uint32_t slot_of(const uint32_t *table, uint64_t pos, uint64_t block_size) {
    const uint32_t block = table[pos / block_size];
    const uint32_t offset_in_block = static_cast<uint32_t>(pos % block_size);
    return block * static_cast<uint32_t>(block_size) + offset_in_block;
}

// paged.rs:64-80: VO_ERR_BLOCK_TABLE_TOO_SHORT {op, tokens, needed, have}
// when the table does not cover `tokens` keys.
vo_status check_covers(const char *op, uint64_t table_len, uint64_t tokens,
                       uint64_t block_size, uint64_t seq);

// attention.rs:130-147: every entry of every CSR table < num_blocks.
vo_status check_block_tables(const char *op, uint64_t num_seqs, const uint64_t *table_off,
                             const uint32_t *tables, uint64_t num_blocks);

}  // namespace vo

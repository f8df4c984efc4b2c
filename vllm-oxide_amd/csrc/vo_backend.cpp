// vo_backend.cpp -- the HIP backend behind the C ABI: KV pool, device-resident
// step metadata, and the attention-path ops with the reference's checks.
//
// Each op validates on the host, in the reference's order, before anything is
// enqueued (crates/engine/src/arena/ops.rs:102-214, backend/cpu/mod.rs:257-339,
// backend/cpu/attention.rs:130-147), then launches the kernels on the
// caller's stream without synchronising.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <queue>
#include <string>
#include <unordered_map>
#include <vector>

#include "vo_backend.hpp"

using namespace vo;

// ---------------------------------------------------------------------------
// KV pool
// ---------------------------------------------------------------------------

extern "C" int32_t vo_kv_pool_create(const vo_kv_layout *layout, int32_t device,
                                     vo_kv_pool **out) {
    if (!layout || !out) return fail_argument("alloc_kv_pool", "null layout or output");
    *out = nullptr;
    const vo_kv_layout &L = *layout;
    if (L.num_layers == 0 || L.num_blocks == 0 || L.block_size == 0 || L.kv_heads == 0 ||
        L.head_dim == 0)
        return fail_shape("alloc_kv_pool", "every layout dimension must be non-zero");
    if (L.head_dim % 8 != 0)
        return fail_unsupported("alloc_kv_pool",
                                "head_dim " + std::to_string(L.head_dim) +
                                    " is not a multiple of 8 (16-byte rows)");
    if (L.num_blocks * L.block_size > 0xffffffffull)
        return fail_capacity("kv slots (u32 slot ids)", L.num_blocks * L.block_size,
                             0xffffffffull);
    DeviceGuard guard(device);
    if (!guard.ok()) return fail_device("alloc_kv_pool", hipErrorInvalidDevice, "hipSetDevice");
    vo_kv_pool *pool = new (std::nothrow) vo_kv_pool();
    if (!pool) return fail_argument("alloc_kv_pool", "out of host memory");
    pool->layout = L;
    pool->device = device;
    pool->layer_elems = vo_kv_layout_layer_elems(&L);
    pool->bytes = L.num_layers * 2 * pool->layer_elems * sizeof(uint16_t);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0)
        pool->num_cus = prop.multiProcessorCount;
    hipError_t err = hipMalloc(reinterpret_cast<void **>(&pool->base), pool->bytes);
    if (err != hipSuccess) {
        delete pool;
        return fail_device("alloc_kv_pool", err, hipGetErrorString(err));
    }
    // Zero-filled, as the reference's calloc'd pool (cpu/mod.rs:148-157).
    err = hipMemset(pool->base, 0, pool->bytes);
    if (err != hipSuccess) {
        (void)hipFree(pool->base);
        delete pool;
        return fail_device("alloc_kv_pool", err, hipGetErrorString(err));
    }
    *out = pool;
    clear_error();
    return VO_OK;
}

extern "C" void vo_kv_pool_destroy(vo_kv_pool *pool) {
    if (!pool) return;
    DeviceGuard guard(pool->device);
    (void)hipFree(pool->base);
    delete pool;
}

extern "C" int32_t vo_kv_pool_layout(const vo_kv_pool *pool, vo_kv_layout *out) {
    if (!pool || !out) return fail_argument("kv_layout", "null pool or output");
    *out = pool->layout;
    clear_error();
    return VO_OK;
}

extern "C" uint64_t vo_kv_pool_bytes(const vo_kv_pool *pool) { return pool ? pool->bytes : 0; }

// ---------------------------------------------------------------------------
// Step metadata
// ---------------------------------------------------------------------------

namespace {

// Packs u32 arrays back to back (256-byte aligned) into the staging buffer and
// records each array's device address.  With fixed launch shapes, each region
// goes to its fixed offset instead (so its device address is the same in
// every upload).  The buffer is sized at creation for the declared
// capacities; should a request still not fit, the arrays go to a host-side
// sink and fits() reports it, so nothing is written out of bounds.
class Packer {
   public:
    explicit Packer(vo_step_meta *m, bool fixed = false) : m_(m), fixed_(fixed) {
        if (fixed_) off_ = m_->fixed.bytes;
    }
    uint32_t *add(Region region, uint64_t count, const uint32_t **device_ptr) {
        uint64_t at;
        if (fixed_) {
            at = m_->fixed.offset[region];
            if (count > m_->fixed.cap[region]) overflow_ = true;
        } else {
            off_ = align_up(off_, 256);
            at = off_;
            off_ = at + count * sizeof(uint32_t);
            if (off_ > m_->buf_bytes) overflow_ = true;
        }
        if (overflow_) {
            sinks_.emplace_back(count + 1);
            *device_ptr = nullptr;
            return sinks_.back().data();
        }
        *device_ptr = reinterpret_cast<const uint32_t *>(m_->d_buf + at);
        return reinterpret_cast<uint32_t *>(m_->stage.current() + at);
    }
    uint64_t used() const { return off_; }
    bool fits() const { return !overflow_; }
    bool fixed() const { return fixed_; }

   private:
    vo_step_meta *m_;
    bool fixed_;
    uint64_t off_ = 0;
    bool overflow_ = false;
    std::vector<std::vector<uint32_t>> sinks_;
};

// Takes the staging buffer this upload fills (double-buffered: the host
// waits only if the copy out of it, two uploads ago, has not run yet).
vo_status acquire_staging(vo_step_meta *m, const char *op) {
    uint8_t *host;
    const hipError_t err = m->stage.acquire(&host);
    if (err != hipSuccess) return fail_device(op, err, hipGetErrorString(err));
    return VO_OK;
}

vo_status finish_upload(vo_step_meta *m, const Packer &pk, hipStream_t stream, const char *op) {
    if (pk.used() > 0) {
        const hipError_t err = m->stage.commit(m->d_buf, pk.used(), stream);
        if (err != hipSuccess) return fail_device(op, err, hipGetErrorString(err));
    }
    return VO_OK;
}

// CSR block tables: offsets start at 0 and never decrease.
vo_status check_tables(const char *op, uint64_t num_seqs, const uint64_t *table_off,
                       const uint32_t *tables, uint64_t max_entries) {
    if (!table_off) return fail_argument(op, "null table offsets");
    if (table_off[0] != 0) return fail_shape(op, "table offsets must start at 0");
    for (uint64_t s = 0; s < num_seqs; ++s)
        if (table_off[s + 1] < table_off[s])
            return fail_shape(op, "table offsets decrease at sequence " + std::to_string(s));
    const uint64_t entries = table_off[num_seqs];
    if (entries > max_entries) return fail_capacity("block-table entries per step", entries, max_entries);
    if (entries && !tables) return fail_argument(op, "null block tables");
    return VO_OK;
}

// Rows: sequence index in range; key count covered by the sequence's table
// (what PrefillMeta::new / DecodeMeta::new guarantee, paged.rs:130, :200).
vo_status check_rows(const char *op, uint64_t num_rows, uint64_t num_seqs, uint64_t block_size,
                     const uint64_t *table_off, const uint64_t *row_seq,
                     const uint64_t *row_num_keys) {
    if (num_rows && (!row_seq || !row_num_keys)) return fail_argument(op, "null row arrays");
    for (uint64_t r = 0; r < num_rows; ++r) {
        if (row_seq[r] >= num_seqs)
            return fail_shape(op, "row " + std::to_string(r) + " names sequence " +
                                      std::to_string(row_seq[r]) + " of " +
                                      std::to_string(num_seqs));
        if (row_num_keys[r] > kU32Limit)
            return fail_capacity("keys per row", row_num_keys[r], kU32Limit);
        const uint64_t s = row_seq[r];
        if (vo_status rc = check_covers(op, table_off[s + 1] - table_off[s], row_num_keys[r],
                                        block_size, s))
            return rc;
    }
    return VO_OK;
}

// Common part of the prefill and decode uploads.
vo_status upload_common(vo_step_meta *m, MetaKind kind, const char *op, uint64_t block_size,
                        uint64_t num_seqs, const uint64_t *table_off, const uint32_t *tables,
                        uint64_t num_rows, const uint32_t *slot_mapping, const uint64_t *row_seq,
                        const uint64_t *row_num_keys, const uint32_t *positions, Packer &pk) {
    if (block_size == 0) return fail_shape(op, "block_size 0");
    if (num_seqs > m->max_seqs) return fail_capacity("sequences per step", num_seqs, m->max_seqs);
    if (num_rows > m->max_rows) return fail_capacity("tokens per step", num_rows, m->max_rows);
    if (vo_status rc = check_tables(op, num_seqs, table_off, tables, m->max_entries)) return rc;
    if (kind != kSlots) {
        if (vo_status rc =
                check_rows(op, num_rows, num_seqs, block_size, table_off, row_seq, row_num_keys))
            return rc;
    }
    if (num_rows && !slot_mapping) return fail_argument(op, "null slot mapping");
    if (vo_status rc = acquire_staging(m, op)) return rc;

    const uint64_t entries = table_off[num_seqs];
    m->kind = kind;
    m->block_size = block_size;
    m->num_seqs = num_seqs;
    m->num_rows = num_rows;
    m->table_off.assign(table_off, table_off + num_seqs + 1);
    m->tables.assign(tables, tables + entries);
    m->slots.assign(slot_mapping, slot_mapping + num_rows);
    m->row_seq.resize(num_rows);
    m->row_num_keys.resize(num_rows);
    m->max_block = 0;
    for (uint32_t b : m->tables) m->max_block = std::max(m->max_block, b);
    m->max_slot = 0;
    for (uint32_t s : m->slots) m->max_slot = std::max(m->max_slot, s);

    const uint32_t *dp;
    // The split-K counts the kernels read; plan_decode_rows fills them.
    m->h_counts = pk.add(kRegCounts, 2, &dp);
    m->h_counts[0] = m->h_counts[1] = 0;
    m->d_counts = dp;
    uint32_t *h = pk.add(kRegTableOff, num_seqs + 1, &dp);
    for (uint64_t s = 0; s <= num_seqs; ++s) h[s] = static_cast<uint32_t>(table_off[s]);
    m->view.table_off = dp;
    h = pk.add(kRegTables, entries, &dp);
    if (entries) std::memcpy(h, tables, entries * sizeof(uint32_t));
    m->view.tables = dp;
    h = pk.add(kRegRowSeq, num_rows, &dp);
    for (uint64_t r = 0; r < num_rows; ++r)
        h[r] = m->row_seq[r] = row_seq ? static_cast<uint32_t>(row_seq[r]) : 0u;
    m->view.row_seq = dp;
    h = pk.add(kRegRowKeys, num_rows, &dp);
    for (uint64_t r = 0; r < num_rows; ++r)
        h[r] = m->row_num_keys[r] = row_num_keys ? static_cast<uint32_t>(row_num_keys[r]) : 0u;
    m->view.row_num_keys = dp;
    // Positions (RoPE): kept only when the caller gave them.
    m->has_positions = positions != nullptr || num_rows == 0;
    m->max_position = 0;
    m->positions.clear();
    m->view.positions = nullptr;
    if (positions) {
        m->positions.assign(positions, positions + num_rows);
        h = pk.add(kRegPositions, num_rows, &dp);
        for (uint64_t r = 0; r < num_rows; ++r) {
            h[r] = positions[r];
            m->max_position = std::max(m->max_position, positions[r]);
        }
        m->view.positions = dp;
    }
    // Write slots: a slot that appears again later keeps only its last row,
    // the reference's "later row wins" copy order (cpu/mod.rs:277-283).
    h = pk.add(kRegSlots, num_rows, &dp);
    {
        std::unordered_map<uint32_t, uint64_t> last;
        bool dup = false;
        last.reserve(num_rows * 2);
        for (uint64_t r = 0; r < num_rows; ++r) {
            auto it = last.find(slot_mapping[r]);
            if (it != last.end()) dup = true;
            last[slot_mapping[r]] = r;
        }
        for (uint64_t r = 0; r < num_rows; ++r)
            h[r] = (!dup || last[slot_mapping[r]] == r) ? slot_mapping[r] : kSkipSlot;
        m->slots_repeat = dup;
    }
    m->d_write_slots = dp;
    m->view.slot_mapping = dp;
    // Write plan: maximal runs of rows whose slots are consecutive inside one
    // block of the pool, as (first row, rows, first slot).  A prefill chunk
    // becomes whole blocks plus partial ends, a decode step one-row runs.  A
    // superseded row is a one-row run with slot kSkipSlot: nothing is cached
    // for it, but the fused RoPE write still rotates its q row.
    {
        const uint32_t *ws = h;
        const uint64_t pbs = m->pool_block_size ? m->pool_block_size : 1;
        auto run_end = [&](uint64_t r) {
            uint64_t e = r + 1;
            if (ws[r] == kSkipSlot) return e;
            while (e < num_rows && ws[e] != kSkipSlot && ws[e] == ws[e - 1] + 1 && ws[e] % pbs != 0)
                ++e;
            return e;
        };
        uint64_t nseg = 0;
        for (uint64_t r = 0; r < num_rows; r = run_end(r)) ++nseg;
        uint32_t *seg = pk.add(kRegSegments, 3 * nseg, &dp);
        uint64_t k = 0;
        for (uint64_t r = 0; r < num_rows;) {
            const uint64_t e = run_end(r);
            seg[3 * k] = static_cast<uint32_t>(r);
            seg[3 * k + 1] = static_cast<uint32_t>(e - r);
            seg[3 * k + 2] = ws[r];
            ++k;
            r = e;
        }
        m->write_plan.segments = dp;
        m->write_plan.num_segments = static_cast<uint32_t>(nseg);
    }
    m->view.num_rows = static_cast<uint32_t>(num_rows);
    m->view.num_seqs = static_cast<uint32_t>(num_seqs);
    m->decode_planned = false;
    m->d_last_rows = nullptr;
    m->last_rows_ok = false;
    return VO_OK;
}

// Whether the n values at `given` equal `held` (same count, same values).
template <class H, class G>
bool same_array(const std::vector<H> &held, const G *given, uint64_t n) {
    if (held.size() != n) return false;
    if (n && !given) return false;
    for (uint64_t i = 0; i < n; ++i)
        if (static_cast<uint64_t>(held[i]) != static_cast<uint64_t>(given[i])) return false;
    return true;
}

// Whether the meta's last upload is a `kind` step with exactly these inputs
// (the common part of the prefill and decode uploads).
bool holds_step(const vo_step_meta *m, MetaKind kind, uint64_t block_size, uint64_t num_seqs,
                const uint64_t *table_off, const uint32_t *tables, uint64_t num_rows,
                const uint32_t *positions, const uint32_t *slot_mapping, const uint64_t *row_seq,
                const uint64_t *row_num_keys) {
    if (m->kind != kind || m->block_size != block_size || m->num_seqs != num_seqs ||
        m->num_rows != num_rows || !table_off)
        return false;
    if (!same_array(m->table_off, table_off, num_seqs + 1) ||
        !same_array(m->tables, tables, table_off[num_seqs]) ||
        !same_array(m->slots, slot_mapping, num_rows) ||
        !same_array(m->row_seq, row_seq, num_rows) ||
        !same_array(m->row_num_keys, row_num_keys, num_rows))
        return false;
    if (positions) return m->has_positions && same_array(m->positions, positions, num_rows);
    return m->positions.empty() && m->has_positions == (num_rows == 0);
}

// Split-K plan.  Every row's keys are cut into splits of L keys (a multiple
// of 32, default kDefaultSplit).  L does not depend on the rest of the batch,
// so a row's arithmetic -- which keys each wavefront accumulates, in which
// order, and how the partials merge -- is the same alone or in any batch:
// the reference's batch-invariance invariant (CLAUDE.md "Batch invariance",
// model.rs:539-584).  VO_DECODE_SPLIT overrides L (a tuning knob).
// 2048: on the isolated decode, prefix-shared decode and mixed-step
// benchmarks it measured 1.8% / 1.5% / 2% faster than 1024 keys on one box
// (fewer workgroup starts and partials); 8 wavefronts per workgroup were
// slower on the last two.
constexpr uint64_t kDefaultSplit = 2048;

}  // namespace

uint64_t vo::decode_split_keys() {
    const int env = env_int("VO_DECODE_SPLIT", 0);
    return (env >= 32 && env % 32 == 0 && env <= static_cast<int>(kernels::kMaxSplitKeys))
               ? static_cast<uint64_t>(env)
               : kDefaultSplit;
}

namespace {

// True when no physical block is read by two sequences of this step (no
// prefix sharing through aliased table entries): the decode kernel then
// streams K/V with non-temporal loads.  When blocks are shared, the cached
// loads let later rows hit the shared prefix in L2 / MALL.  Either way the
// arithmetic is identical.  Each sequence's used table prefix is checked
// once (its last row has the most keys).  VO_DECODE_NT=0/1 forces the choice.
bool decode_streaming(vo_step_meta *m) {
    const int env = env_int("VO_DECODE_NT", -1);
    if (env == 0 || env == 1) return env == 1;
    const uint64_t bs = m->block_size;
    const uint64_t S = m->num_seqs;
    m->seq_keys.assign(S, 0);
    for (uint64_t r = 0; r < m->num_rows; ++r)
        m->seq_keys[m->row_seq[r]] = std::max<uint64_t>(m->seq_keys[m->row_seq[r]], m->row_num_keys[r]);
    m->block_seen.assign(static_cast<size_t>(m->max_block) + 1, 0);
    for (uint64_t seq = 0; seq < S; ++seq) {
        const uint64_t used = (m->seq_keys[seq] + bs - 1) / bs;
        const uint32_t *t = m->tables.data() + m->table_off[seq];
        for (uint64_t i = 0; i < used; ++i) {
            if (m->block_seen[t[i]]) return false;
            m->block_seen[t[i]] = 1;
        }
    }
    return true;
}

// Rows with zero keys still get one work item (it writes the zero output).
uint64_t row_splits(uint64_t keys, uint64_t L) { return keys ? (keys + L - 1) / L : 1; }

// Row packing.  The split kernel computes 16 head columns per MFMA tile, of
// which one row's KV-head group uses G = query heads / KV heads.  Full splits
// of different rows that read the same physical blocks (aliased block-table
// entries: a shared prefix) go to one workgroup, so those blocks are read
// once per pack instead of once per row.  Each row keeps its own columns,
// softmax and partial, so its result is bitwise the one it gets unpacked.
// Modes (VO_DECODE_PACK): 0 off; 1 one tile per item (16 / G rows, the
// register path); 2 (default) shared packs: the workgroup stages each chunk
// in LDS once and each of its 4 wavefronts takes one tile, 4 * (16 / G)
// rows.  The limits use the largest group the metadata admits, so any call's
// group fits; the staging buffer is sized for the largest
// (decode_pack_limit).
enum PackMode : uint32_t { kPackOff = 0, kPackOneTile = 1, kPackShared = 2 };

uint64_t max_group(const vo_step_meta *m) {
    return std::max<uint64_t>(1, (m->max_heads + m->kv_heads - 1) / m->kv_heads);
}

// Rows per item with `tiles` 16-column tiles shared by all rows.
uint32_t decode_pack_rows(const vo_step_meta *m, uint32_t tiles) {
    if (m->kv_heads == 0) return 1;
    const uint64_t p = 16 * tiles / max_group(m);
    return p >= 2 ? static_cast<uint32_t>(p) : 1u;
}

// Rows per shared pack: 16 / G per wavefront.
uint32_t decode_shared_rows(const vo_step_meta *m, uint32_t waves) {
    if (m->kv_heads == 0) return 1;
    const uint64_t p = waves * (16 / max_group(m));
    return p >= 2 ? static_cast<uint32_t>(p) : 1u;
}

// The mates buffer is sized for the larger packs (one wavefront per tile),
// whichever form a later plan takes.
uint32_t decode_pack_limit(const vo_step_meta *m) {
    return std::max(decode_pack_rows(m, 1), decode_shared_rows(m, 4));
}

// Shared packs in wavefront pairs (two wavefronts per tile, each walking
// half of the split's chunks; half the rows per pack).  VO_DECODE_SHARED_PAIRS
// = 0 keeps one wavefront per tile (a tuning knob, read per plan).
bool decode_shared_pairs() { return env_int("VO_DECODE_SHARED_PAIRS", 1) != 0; }

// With shared packs, the blocks several rows read go through the packs'
// LDS stages, so the other items stream their (mostly private) blocks with
// non-temporal loads, which keeps the shared blocks in L2 for the packs.
// VO_DECODE_PACK_NT = 0 keeps cached loads (a tuning knob, read per plan).
bool decode_pack_nt() { return env_int("VO_DECODE_PACK_NT", 1) != 0; }

uint32_t decode_pack_mode() {
    const int v = env_int("VO_DECODE_PACK", kPackShared);
    return (v <= 0) ? kPackOff : static_cast<uint32_t>(std::min(v, static_cast<int>(kPackShared)));
}

// Moves the packs of two or more rows (pack_fill >= 2) in front of the rest,
// keeping order within both; returns their number.  Records hold (row,
// split) in their first two words; mates rows move along.
uint64_t shared_packs_first(vo_step_meta *m, uint32_t *work, uint64_t n, uint32_t P,
                            uint32_t *mates) {
    std::vector<uint32_t> w(2 * n), mt(static_cast<size_t>(P - 1) * n);
    uint64_t at = 0, ns = 0;
    for (int pass = 0; pass < 2; ++pass)
        for (uint64_t i = 0; i < n; ++i) {
            if ((m->pack_fill[i] >= 2) != (pass == 0)) continue;
            w[2 * at] = work[4 * i];
            w[2 * at + 1] = work[4 * i + 1];
            std::copy(mates + (P - 1) * i, mates + (P - 1) * (i + 1), mt.begin() + (P - 1) * at);
            ++at;
            if (pass == 0) ++ns;
        }
    for (uint64_t i = 0; i < n; ++i) {
        work[4 * i] = w[2 * i];
        work[4 * i + 1] = w[2 * i + 1];
    }
    std::copy(mt.begin(), mt.end(), mates);
    return ns;
}

// Packs work[0 .. nfull) (full splits; (row, split) in the first two words
// of each record) in place: items
// with the same split index over the same block list join the first open
// pack of that list (its leader keeps the item's place, the others become
// its mates).  Returns the number of packed items; mates gets P - 1 entries
// per packed item, kNoMate where a pack is short.
uint64_t pack_full_splits(vo_step_meta *m, uint32_t *work, uint64_t nfull, uint64_t L,
                          uint32_t P, uint32_t *mates) {
    const uint64_t nb = L / m->block_size;
    auto blocks_of = [&](uint32_t row, uint32_t split) {
        return m->tables.data() + m->table_off[m->row_seq[row]] + split * nb;
    };
    m->pack_open.clear();
    m->pack_fill.clear();
    uint64_t n = 0;
    for (uint64_t f = 0; f < nfull; ++f) {
        const uint32_t row = work[4 * f], split = work[4 * f + 1];
        const uint32_t *b = blocks_of(row, split);
        uint64_t hsh = 0xcbf29ce484222325ull ^ split;  // FNV-1a over (split, blocks)
        for (uint64_t i = 0; i < nb; ++i) hsh = (hsh ^ b[i]) * 0x100000001b3ull;
        auto it = m->pack_open.find(hsh);
        if (it != m->pack_open.end()) {
            const uint32_t lead = it->second;
            const uint32_t lrow = work[4 * lead];
            if (work[4 * lead + 1] == split &&
                std::memcmp(blocks_of(lrow, split), b, nb * sizeof(uint32_t)) == 0) {
                mates[(P - 1) * lead + m->pack_fill[lead] - 1] = row;
                if (++m->pack_fill[lead] == P) m->pack_open.erase(it);
                continue;
            }
        }
        // A new pack (a hash collision just starts another one).
        work[4 * n] = row;
        work[4 * n + 1] = split;
        std::fill(mates + (P - 1) * n, mates + (P - 1) * (n + 1), kernels::kNoMate);
        m->pack_fill.push_back(1);
        m->pack_open[hsh] = static_cast<uint32_t>(n);
        ++n;
    }
    return n;
}

// Every row of the upload is the one DecodeMeta::new (paged.rs:189-209)
// gives a sequence: one row per sequence, at least one key (the new one),
// and the slot of its last key, slot_of(table, keys - 1) (paged.rs:47-52,
// u32 arithmetic).  The upload accepts any rows, as the reference's pub
// fields do; the one-launch write_kv + decode_attention needs these.
bool canonical_decode_rows(vo_step_meta *m) {
    const uint64_t bs = m->block_size;
    m->block_seen.assign(m->num_seqs, 0);  // here: rows per sequence
    for (uint64_t r = 0; r < m->num_rows; ++r) {
        const uint32_t seq = m->row_seq[r];
        const uint32_t nk = m->row_num_keys[r];
        if (nk == 0 || m->block_seen[seq]) return false;
        m->block_seen[seq] = 1;
        // check_rows already made sure the table covers nk keys.
        if (m->slots[r] != slot_of(m->tables.data() + m->table_off[seq], nk - 1, bs)) return false;
    }
    return true;
}

// Split-K plan over the rows listed in `rows` (every row of the step when
// rows is null).  Rows outside the plan get row_info (0, 0).
vo_status plan_decode_rows(vo_step_meta *m, Packer &pk, const std::vector<uint32_t> *rows) {
    const uint64_t T = m->num_rows;
    const uint64_t L = decode_split_keys();
    const uint64_t R = rows ? rows->size() : T;
    auto row_at = [&](uint64_t i) -> uint64_t { return rows ? (*rows)[i] : i; };
    uint64_t parts = 0;
    for (uint64_t i = 0; i < R; ++i) parts += row_splits(m->row_num_keys[row_at(i)], L);
    if (parts > m->max_parts) return fail_capacity("split-K partials per step", parts, m->max_parts);

    const uint32_t *dp;
    uint32_t *work = pk.add(kRegWork, 4 * parts, &dp);
    m->plan.work = dp;
    uint32_t *row_info = pk.add(kRegRowInfo, 2 * T, &dp);
    m->plan.row_info = dp;
    uint32_t *reduce_rows = pk.add(kRegReduceRows, R, &dp);
    m->plan.reduce_rows = dp;
    // Work order, longest first: every full split (L keys) in row order, then
    // each row's shorter last split by descending length.  The hardware deals
    // workgroups out in grid order as slots free up, so the short items fill
    // the gaps at the end instead of a full split starting last and running
    // alone.  Partials are addressed by (row, split), so the order changes no
    // arithmetic.
    if (rows) std::fill(row_info, row_info + 2 * T, 0u);
    uint64_t n = 0, nred = 0;
    for (uint64_t i = 0; i < R; ++i) {
        const uint64_t r = row_at(i);
        const uint64_t ns = row_splits(m->row_num_keys[r], L);
        row_info[2 * r] = static_cast<uint32_t>(n);
        row_info[2 * r + 1] = static_cast<uint32_t>(ns);
        n += ns;
        if (ns > 1) reduce_rows[nred++] = static_cast<uint32_t>(r);
    }
    m->tail_items.clear();
    uint64_t f = 0;
    const bool streaming = pk.fixed() ? m->fixed.streaming : decode_streaming(m);
    // Packing needs shared blocks, so a streaming plan never packs; a fixed
    // launch keeps one item per (row, split).
    uint32_t mode = (pk.fixed() || streaming || L % m->block_size != 0) ? kPackOff : decode_pack_mode();
    const int waves = decode_waves();
    // Shared packs need 4 wavefronts (the kernel keeps one softmax state per
    // wavefront in registers and stages four chunks).
    if (mode == kPackShared && waves != 4) mode = kPackOneTile;
    const bool pairs = mode == kPackShared && decode_shared_pairs();
    uint32_t P = mode == kPackOff      ? 1u
                 : mode == kPackShared ? decode_shared_rows(m, static_cast<uint32_t>(pairs ? waves / 2 : waves))
                                       : decode_pack_rows(m, 1);
    uint32_t *mates = nullptr;
    m->plan.mates = nullptr;
    m->plan.num_shared = 0;
    m->plan.shared_pairs = pairs;
    if (P > 1) {
        mates = pk.add(kRegMates, (P - 1) * parts, &dp);
        m->plan.mates = dp;
    }
    auto full_splits = [&]() {
        uint64_t nf = 0;
        for (uint64_t i = 0; i < R; ++i) {
            const uint64_t r = row_at(i);
            for (uint64_t sp = 0; sp < m->row_num_keys[r] / L; ++sp, ++nf) {
                work[4 * nf] = static_cast<uint32_t>(r);
                work[4 * nf + 1] = static_cast<uint32_t>(sp);
            }
        }
        return nf;
    };
    f = full_splits();
    for (uint64_t i = 0; i < R; ++i) {
        const uint64_t r = row_at(i);
        const uint64_t nk = m->row_num_keys[r];
        if (nk % L != 0 || nk == 0)
            m->tail_items.push_back({static_cast<uint32_t>(nk % L), static_cast<uint32_t>(r),
                                     static_cast<uint32_t>(nk / L)});
    }
    if (P > 1) {
        const uint64_t nfull = f;
        f = pack_full_splits(m, work, nfull, L, P, mates);
        if (mode == kPackShared) {
            // Shared packs first; the other items run as single rows.  With
            // no pack of two rows there is nothing to share.
            uint32_t fullest = 0;
            for (uint32_t fill : m->pack_fill) fullest = std::max(fullest, fill);
            if (fullest >= 2) {
                m->plan.num_shared = static_cast<uint32_t>(shared_packs_first(m, work, f, P, mates));
            } else {
                P = 1;
                f = full_splits();
            }
        }
    }
    std::stable_sort(m->tail_items.begin(), m->tail_items.end(),
                     [](const TailItem &a, const TailItem &b) { return a.keys > b.keys; });
    for (const TailItem &t : m->tail_items) {
        work[4 * f] = t.row;
        work[4 * f + 1] = t.split;
        if (P > 1) std::fill(mates + (P - 1) * f, mates + (P - 1) * (f + 1), kernels::kNoMate);
        ++f;
    }
    const uint64_t num_work = f;  // = parts unless packed
    // The rest of each record: where the split's block ids start in the
    // tables, and the (leading) row's key count.
    for (uint64_t i = 0; i < num_work; ++i) {
        const uint32_t row = work[4 * i];
        const uint64_t split = work[4 * i + 1];
        work[4 * i + 2] =
            static_cast<uint32_t>(m->table_off[m->row_seq[row]] + split * L / m->block_size);
        work[4 * i + 3] = m->row_num_keys[row];
    }
    m->decode_parts = parts;
    m->plan.pack = P;
    m->plan.num_work = static_cast<uint32_t>(num_work);
    m->plan.num_reduce_rows = static_cast<uint32_t>(nred);
    m->plan.split_keys = static_cast<uint32_t>(L);
    m->plan.part_acc = m->d_part_acc;
    m->plan.part_ml = m->d_part_ml;
    m->h_counts[0] = static_cast<uint32_t>(num_work);
    m->h_counts[1] = static_cast<uint32_t>(nred);
    m->plan.counts = m->d_counts;
    if (pk.fixed()) {
        // The same launches every step: capacity-sized grids, the kernels stop
        // at the counts; the load policy stays the one fixed (it changes no
        // arithmetic).
        m->plan.streaming = streaming;
        m->plan.launch_work = static_cast<uint32_t>(m->fixed.work_cap);
        m->plan.launch_reduce = static_cast<uint32_t>(m->fixed.seqs);
    } else {
        m->plan.streaming = streaming || (m->plan.num_shared != 0 && decode_pack_nt());
        m->plan.launch_work = static_cast<uint32_t>(num_work);
        m->plan.launch_reduce = static_cast<uint32_t>(nred);
    }
    m->decode_planned = true;
    // New keys cached by the decode launch: a whole decode step without
    // repeated slots or a fixed launch, and no block holding a new slot read
    // by another sequence (with a streaming plan no block is shared at all).
    // A packed item's blocks are read by several rows, so under these
    // conditions it never holds a row's last key.  Every row must also be
    // the canonical decode row DecodeMeta::new builds (paged.rs:189-209):
    // its own sequence, at least one key, and its slot the one of its last
    // key.  Only then is the workgroup holding that key the one place that
    // reads the slot, so taking K/V from the new rows and writing the slot at
    // the end equals write_kv followed by decode_attention.
    m->fused_write_ok = false;
    if (!rows && !pk.fixed() && !m->slots_repeat && m->kind == kDecode) {
        bool ok = canonical_decode_rows(m);
        if (ok && !streaming) {
            const uint64_t bs = m->block_size;
            m->seq_keys.assign(m->num_seqs, 0);
            for (uint64_t r = 0; r < T; ++r)
                m->seq_keys[m->row_seq[r]] =
                    std::max<uint64_t>(m->seq_keys[m->row_seq[r]], m->row_num_keys[r]);
            m->block_seen.assign(static_cast<size_t>(m->max_block) + 1, 0);  // readers, up to 2
            for (uint64_t seq = 0; seq < m->num_seqs; ++seq) {
                const uint64_t used = (m->seq_keys[seq] + bs - 1) / bs;
                const uint32_t *t = m->tables.data() + m->table_off[seq];
                for (uint64_t i = 0; i < used; ++i)
                    if (m->block_seen[t[i]] < 2) ++m->block_seen[t[i]];
            }
            for (uint64_t r = 0; r < T && ok; ++r) ok = m->block_seen[m->slots[r] / bs] < 2;
        }
        m->fused_write_ok = ok;
    }
    return VO_OK;
}

vo_status plan_decode(vo_step_meta *m, Packer &pk) { return plan_decode_rows(m, pk, nullptr); }

// Prefill plan.  It needs the layout PrefillMeta::new produces
// (paged.rs:128-141): the rows of sequence s are seq_row_starts[s] ..
// seq_row_starts[s+1], row i of them at position context_lens[s] + i with
// i + 1 + context_lens[s] keys; other layouts run on the generic kernel.
// A mixed continuous-batching step carries decode sequences (one new row) and
// chunks in one call: a sequence with one row goes to the split-K decode
// kernel, with the same split plan a decode call gives it, so its result is
// bitwise the one decode_attention returns; sequences with more rows become
// 64-row items of the MFMA prefill kernel, sorted by KV tiles, longest first,
// so that the long ones are scheduled early.  Both kernels cover the same
// shapes, and each row is written by exactly one of them.  Items with rows
// past prefill_dma_max_keys() keys (a multiple of 64, so exactly the items of
// more tiles than that / 64) lead the order and are counted in num_long.
// Per-item cost of the pipelined prefill kernel's slot plan, in KV tiles
// (measured: an item's tile 0, overflow check, output and hand-over take
// about five tiles' time).
constexpr uint64_t kPipeItemCost = 5;

// Persistent slots per KV head for the pipelined prefill kernel: the CUs'
// share of one KV head (one workgroup fills a CU), at most one per item.
// VO_PREFILL_PIPE_SLOTS=n sets the count (tests: long item chains per slot).
uint32_t pipe_slot_count(const vo_step_meta *m, uint64_t items) {
    uint64_t s = (m->num_cus && m->kv_heads) ? m->num_cus / m->kv_heads : 1;
    const int forced = env_int("VO_PREFILL_PIPE_SLOTS", 0);
    if (forced > 0) s = static_cast<uint64_t>(forced);
    return static_cast<uint32_t>(std::max<uint64_t>(1, std::min<uint64_t>(s, items)));
}

vo_status plan_prefill(vo_step_meta *m, Packer &pk, const uint64_t *context_lens,
                       const uint64_t *seq_row_starts) {
    m->prefill_planned = false;
    m->decode_planned = false;
    const uint64_t S = m->num_seqs;
    for (uint64_t s = 0; s < S; ++s) {
        for (uint64_t r = seq_row_starts[s]; r < seq_row_starts[s + 1]; ++r) {
            const uint64_t i = r - seq_row_starts[s];
            if (m->row_seq[r] != s || m->row_num_keys[r] != context_lens[s] + i + 1) return VO_OK;
        }
    }
    const uint32_t QT = kernels::prefill_rows_per_tile();
    struct Item { uint32_t row, rows, pos, seq, tiles; };
    std::vector<Item> items;
    m->decode_rows.clear();
    // VO_PREFILL_DECODE_ROWS=0 keeps one-row sequences on the prefill kernel
    // (a measurement switch).
    const bool route_decode_rows = env_int("VO_PREFILL_DECODE_ROWS", 1) != 0;
    for (uint64_t s = 0; s < S; ++s) {
        const uint64_t n = seq_row_starts[s + 1] - seq_row_starts[s];
        if (n == 1 && route_decode_rows) {
            m->decode_rows.push_back(static_cast<uint32_t>(seq_row_starts[s]));
            continue;
        }
        for (uint64_t q0 = 0; q0 < n; q0 += QT) {
            Item it;
            it.row = static_cast<uint32_t>(seq_row_starts[s] + q0);
            it.rows = static_cast<uint32_t>(std::min<uint64_t>(QT, n - q0));
            it.pos = static_cast<uint32_t>(context_lens[s] + q0);
            it.seq = static_cast<uint32_t>(s);
            it.tiles = (it.pos + it.rows - 1) / 64 + 1;
            items.push_back(it);
        }
    }
    std::stable_sort(items.begin(), items.end(),
                     [](const Item &a, const Item &b) { return a.tiles > b.tiles; });
    const uint32_t *dp;
    uint32_t *w = pk.add(kRegPrefillWork, 4 * items.size(), &dp);
    for (size_t i = 0; i < items.size(); ++i) {
        w[4 * i] = items[i].row;
        w[4 * i + 1] = items[i].rows;
        w[4 * i + 2] = items[i].pos;
        w[4 * i + 3] = items[i].seq;
    }
    m->prefill_plan.work = dp;
    m->prefill_plan.num_items = static_cast<uint32_t>(items.size());
    uint32_t max_keys = 0, num_long = 0;
    for (const Item &it : items) {
        max_keys = std::max(max_keys, it.pos + it.rows);
        num_long += it.pos + it.rows > kernels::prefill_dma_max_keys();
    }
    m->prefill_plan.max_keys = max_keys;
    m->prefill_plan.num_long = num_long;
    // The pipelined kernel's persistent slots (one workgroup per slot and
    // KV head): its items, longest first, each to the slot with the least
    // work so far, counted in KV tiles plus kPipeItemCost per item (its
    // tile 0 and the hand-over between items); ties go to the lower slot.
    // Which slot runs an item changes no bit of its rows.
    m->prefill_plan.pipe = nullptr;
    m->prefill_plan.pipe_slots = 0;
    const uint64_t n_pipe = items.size() - num_long;
    if (n_pipe > 0) {
        const uint32_t S = pipe_slot_count(m, n_pipe);
        std::vector<uint32_t> slot_of(items.size()), count(S, 0);
        using Load = std::pair<uint64_t, uint32_t>;
        std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
        for (uint32_t s = 0; s < S; ++s) heap.push({0, s});
        for (size_t k = num_long; k < items.size(); ++k) {
            const Load top = heap.top();
            heap.pop();
            slot_of[k] = top.second;
            ++count[top.second];
            heap.push({top.first + items[k].tiles + kPipeItemCost, top.second});
        }
        const uint32_t *pp;
        uint32_t *pw = pk.add(kRegPrefillPipe,
                              S + 1 + kernels::kPipeFirstWords * S + 4 * n_pipe, &pp);
        std::vector<uint32_t> at(S);
        uint32_t sum = 0;
        for (uint32_t s = 0; s < S; ++s) {
            pw[s] = at[s] = sum;
            sum += count[s];
        }
        pw[S] = sum;
        uint32_t *const descs = pw + S + 1 + kernels::kPipeFirstWords * S;
        for (size_t k = num_long; k < items.size(); ++k) {
            uint32_t *d = descs + 4 * static_cast<uint64_t>(at[slot_of[k]]++);
            d[0] = items[k].row;
            d[1] = items[k].rows;
            d[2] = items[k].pos;
            d[3] = static_cast<uint32_t>(m->table_off[items[k].seq]);
        }
        // Each slot's first record: its first item's descriptor, the block
        // ids of that item's tiles 0-2, and the next item's first twelve
        // (copies of the item's last id when the slot has one item), each
        // clamped to the item's last block -- what the kernel's first DMAs
        // and block table need, at an address that depends only on the slot.
        // (nblk at the step's block size: the rows' checked table coverage)
        auto block_id = [&](const uint32_t *d, uint32_t k) {
            const uint64_t nblk = (static_cast<uint64_t>(d[2]) + d[1] - 1) / m->block_size + 1;
            return m->tables[d[3] + std::min<uint64_t>(k, nblk - 1)];
        };
        for (uint32_t s = 0; s < S; ++s) {
            uint32_t *f = pw + S + 1 + kernels::kPipeFirstWords * static_cast<uint64_t>(s);
            const uint32_t *d0 = descs + 4 * static_cast<uint64_t>(pw[s]);
            const uint32_t *d1 = count[s] > 1 ? d0 + 4 : nullptr;
            for (int w = 0; w < 4; ++w) f[w] = d0[w];
            for (uint32_t k = 0; k < 12; ++k) f[4 + k] = block_id(d0, k);
            for (uint32_t k = 0; k < 12; ++k) f[16 + k] = d1 ? block_id(d1, k) : block_id(d0, 0xffffffffu);
        }
        m->prefill_plan.pipe = pp;
        m->prefill_plan.pipe_slots = S;
    }
    if (!m->decode_rows.empty())
        if (vo_status rc = plan_decode_rows(m, pk, &m->decode_rows)) return rc;
    m->prefill_planned = true;
    return VO_OK;
}

// VO_MIXED_OVERLAP=0 runs a mixed step's decode rows after its chunks on the
// caller's stream (A/B).
bool mixed_overlap_enabled() {
    static const bool on = env_int("VO_MIXED_OVERLAP", 1) != 0;
    return on;
}

}  // namespace

int vo::decode_waves() {
    int w = env_int("VO_DECODE_WAVES", 4);
    return (w == 1 || w == 2 || w == 4 || w == 8) ? w : 4;
}

namespace {


}  // namespace

namespace {

vo_status refuse_if_fixed(const vo_step_meta *m, const char *op) {
    if (!m->fixed.on) return VO_OK;
    return fail_shape(op, "the metadata has fixed launch shapes for decode steps of " +
                              std::to_string(m->fixed.seqs) +
                              " sequences; vo_step_meta_unfix_launch first");
}

// A decode upload fits the fixed launch shapes: same sequence count, table
// entries and split-K work items within the capacities, positions given iff
// they were when the shapes were fixed.  Checked before anything changes.
vo_status check_fixed_decode(const vo_step_meta *m, uint64_t num_seqs, const uint64_t *table_off,
                             const uint32_t *positions, const uint64_t *row_num_keys) {
    const FixedLaunch &f = m->fixed;
    const char *what = "fixed-launch decode step";
    if (num_seqs != f.seqs || (positions != nullptr) != f.has_positions || !table_off ||
        (num_seqs && !row_num_keys))
        return fail_shape("decode", "a fixed-launch decode step takes " + std::to_string(f.seqs) +
                                        " sequences" +
                                        (f.has_positions ? " with positions" : " without positions") +
                                        ", got " + std::to_string(num_seqs));
    if (table_off[num_seqs] > f.entries_cap) return fail_capacity(what, table_off[num_seqs], f.entries_cap);
    const uint64_t L = decode_split_keys();
    uint64_t parts = 0;
    for (uint64_t r = 0; r < num_seqs; ++r) parts += row_splits(row_num_keys[r], L);
    if (parts > f.work_cap) return fail_capacity(what, parts, f.work_cap);
    return VO_OK;
}

}  // namespace

extern "C" int32_t vo_step_meta_create(const vo_kv_pool *pool, uint64_t max_seqs,
                                       uint64_t max_rows, uint64_t max_table_entries,
                                       uint64_t max_query_heads, vo_step_meta **out) {
    const char *op = "step_meta_create";
    if (!pool || !out) return fail_argument(op, "null pool or output");
    *out = nullptr;
    if (max_seqs == 0 || max_rows == 0 || max_query_heads == 0)
        return fail_argument(op, "capacities must be non-zero");
    if (max_seqs > kU32Limit || max_rows > kU32Limit || max_table_entries > kU32Limit)
        return fail_capacity("step metadata entries (u32)", std::max({max_seqs, max_rows, max_table_entries}),
                             kU32Limit);
    DeviceGuard guard(pool->device);
    if (!guard.ok()) return fail_device(op, hipErrorInvalidDevice, "hipSetDevice");
    vo_step_meta *m = new (std::nothrow) vo_step_meta();
    if (!m) return fail_argument(op, "out of host memory");
    m->device = pool->device;
    m->num_cus = pool->num_cus;
    m->pool_block_size = pool->layout.block_size;
    m->kv_heads = pool->layout.kv_heads;
    m->head_dim = pool->layout.head_dim;
    m->max_seqs = max_seqs;
    m->max_rows = max_rows;
    m->max_entries = max_table_entries;
    m->max_heads = max_query_heads;
    // Decode partials: one per (row, split).  With one row per sequence the
    // keys of a step are at most entries * block_size, so rows + keys / L
    // bounds the splits (L as configured when the meta is created).
    m->max_parts = max_rows + (max_table_entries * pool->layout.block_size) / decode_split_keys();

    const uint64_t u32s = (max_seqs + 1) + max_table_entries + 3 * max_rows  // offsets, tables, row arrays
                          + max_rows                                         // write slots
                          + 3 * max_rows                                     // write plan
                          + max_rows                                         // positions
                          + 4 * m->max_parts + 3 * max_rows                  // decode plan
                          + 4 * (max_rows + max_seqs)                        // prefill plan
                          + (5 + kernels::kPipeFirstWords) * (max_rows + max_seqs) + 1  // its slot plan
                          + max_seqs                                         // last rows
                          + (decode_pack_limit(m) - 1) * m->max_parts        // row-packing mates
                          + 10 * 64;                                         // alignment slack
    m->buf_bytes = align_up(u32s * sizeof(uint32_t), 4096);
    hipError_t err = hipMalloc(reinterpret_cast<void **>(&m->d_buf), m->buf_bytes);
    if (err == hipSuccess) err = m->stage.create(m->buf_bytes);
    if (err == hipSuccess)
        err = hipMalloc(reinterpret_cast<void **>(&m->d_part_acc),
                        m->max_parts * max_query_heads * m->head_dim * sizeof(float));
    if (err == hipSuccess)
        err = hipMalloc(reinterpret_cast<void **>(&m->d_part_ml),
                        m->max_parts * max_query_heads * 2 * sizeof(float));
    if (err == hipSuccess)
        err = hipMalloc(reinterpret_cast<void **>(&m->d_tokens), max_rows * sizeof(uint32_t));
    if (err == hipSuccess) err = m->tokens_stage.create(max_rows * sizeof(uint32_t));
    if (err == hipSuccess)
        err = hipMalloc(reinterpret_cast<void **>(&m->d_aux_pos), max_rows * sizeof(uint32_t));
    if (err == hipSuccess)
        err = hipMalloc(reinterpret_cast<void **>(&m->d_aux_rows), max_rows * sizeof(uint32_t));
    if (err == hipSuccess) err = m->aux_stage.create(max_rows * sizeof(uint32_t));
    // Default priority, like every stream here.
    if (err == hipSuccess) err = hipStreamCreateWithFlags(&m->side, hipStreamNonBlocking);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&m->fork, hipEventDisableTiming);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&m->join, hipEventDisableTiming);
    if (err != hipSuccess) {
        vo_status rc = fail_device(op, err, hipGetErrorString(err));
        if (m->d_tokens) (void)hipFree(m->d_tokens);
        m->tokens_stage.destroy();
        if (m->d_aux_pos) (void)hipFree(m->d_aux_pos);
        if (m->d_aux_rows) (void)hipFree(m->d_aux_rows);
        m->aux_stage.destroy();
        if (m->d_buf) (void)hipFree(m->d_buf);
        m->stage.destroy();
        if (m->d_part_acc) (void)hipFree(m->d_part_acc);
        if (m->d_part_ml) (void)hipFree(m->d_part_ml);
        if (m->side) (void)hipStreamDestroy(m->side);
        if (m->fork) (void)hipEventDestroy(m->fork);
        if (m->join) (void)hipEventDestroy(m->join);
        delete m;
        return rc;
    }
    *out = m;
    clear_error();
    return VO_OK;
}

extern "C" void vo_step_meta_destroy(vo_step_meta *m) {
    if (!m) return;
    DeviceGuard guard(m->device);
    m->stage.destroy();
    m->tokens_stage.destroy();
    m->aux_stage.destroy();
    (void)hipFree(m->d_tokens);
    (void)hipFree(m->d_aux_pos);
    (void)hipFree(m->d_aux_rows);
    (void)hipFree(m->d_buf);
    (void)hipFree(m->d_part_acc);
    (void)hipFree(m->d_part_ml);
    if (m->side) {
        (void)hipStreamSynchronize(m->side);
        (void)hipStreamDestroy(m->side);
    }
    if (m->fork) (void)hipEventDestroy(m->fork);
    if (m->join) (void)hipEventDestroy(m->join);
    delete m;
}

extern "C" int32_t vo_step_meta_upload_prefill(
    vo_step_meta *m, uint64_t block_size, uint64_t num_seqs, const uint64_t *table_off,
    const uint32_t *tables, const uint64_t *context_lens, const uint64_t *seq_row_starts,
    uint64_t num_rows, const uint32_t *positions, const uint32_t *slot_mapping,
    const uint64_t *row_seq, const uint64_t *row_num_keys, void *stream) {
    const char *op = "prefill";
    if (!m) return fail_argument(op, "null meta");
    if (vo_status rc = refuse_if_fixed(m, op)) return rc;
    if (num_seqs && (!context_lens || !seq_row_starts))
        return fail_argument(op, "null context_lens or seq_row_starts");
    if (seq_row_starts && (seq_row_starts[0] != 0 || seq_row_starts[num_seqs] != num_rows))
        return fail_shape(op, "seq_row_starts must run from 0 to num_rows");
    for (uint64_t s = 0; s < num_seqs; ++s)
        if (seq_row_starts[s + 1] < seq_row_starts[s])
            return fail_shape(op, "seq_row_starts decrease at sequence " + std::to_string(s));
    DeviceGuard guard(m->device);
    Packer pk(m);
    if (vo_status rc = upload_common(m, kPrefill, op, block_size, num_seqs, table_off, tables,
                                     num_rows, slot_mapping, row_seq, row_num_keys, positions, pk))
        return rc;
    if (vo_status rc = plan_prefill(m, pk, context_lens, seq_row_starts)) {
        m->kind = kNone;
        return rc;
    }
    m->context_lens.assign(context_lens, context_lens + num_seqs);
    m->seq_row_starts.assign(seq_row_starts, seq_row_starts + num_seqs + 1);
    {
        // PrefillMeta::last_rows (paged.rs:153-159).
        const uint32_t *dp;
        uint32_t *h = pk.add(kRegLastRows, num_seqs, &dp);
        m->last_rows_ok = true;
        for (uint64_t s = 0; s < num_seqs; ++s) {
            if (seq_row_starts[s + 1] == seq_row_starts[s]) m->last_rows_ok = false;
            h[s] = seq_row_starts[s + 1] ? static_cast<uint32_t>(seq_row_starts[s + 1] - 1) : 0u;
        }
        m->d_last_rows = dp;
    }
    if (!pk.fits()) {
        m->kind = kNone;
        return fail_capacity("step metadata bytes", pk.used(), m->buf_bytes);
    }
    if (vo_status rc = finish_upload(m, pk, static_cast<hipStream_t>(stream), op)) return rc;
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_step_meta_upload_decode(vo_step_meta *m, uint64_t block_size,
                                              uint64_t num_seqs, const uint64_t *table_off,
                                              const uint32_t *tables, const uint32_t *positions,
                                              const uint32_t *slot_mapping,
                                              const uint64_t *row_seq,
                                              const uint64_t *row_num_keys, void *stream) {
    const char *op = "decode";
    if (!m) return fail_argument(op, "null meta");
    if (m->fixed.on)
        if (vo_status rc = check_fixed_decode(m, num_seqs, table_off, positions, row_num_keys))
            return rc;
    DeviceGuard guard(m->device);
    Packer pk(m, m->fixed.on);
    if (vo_status rc = upload_common(m, kDecode, op, block_size, num_seqs, table_off, tables,
                                     num_seqs, slot_mapping, row_seq, row_num_keys, positions, pk))
        return rc;
    if (m->fixed.on && m->write_plan.num_segments != num_seqs) {
        m->kind = kNone;
        return fail_shape(op, "two rows of a fixed-launch decode step share a slot");
    }
    if (vo_status rc = plan_decode(m, pk)) {
        m->kind = kNone;
        return rc;
    }
    {
        // Decode: every row is its sequence's last (model.rs:342).
        const uint32_t *dp;
        uint32_t *h = pk.add(kRegLastRows, num_seqs, &dp);
        for (uint64_t s = 0; s < num_seqs; ++s) h[s] = static_cast<uint32_t>(s);
        m->d_last_rows = dp;
        m->last_rows_ok = true;
    }
    if (!pk.fits()) {
        m->kind = kNone;
        return fail_capacity("step metadata bytes", pk.used(), m->buf_bytes);
    }
    if (vo_status rc = finish_upload(m, pk, static_cast<hipStream_t>(stream), op)) return rc;
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_step_meta_upload_slots(vo_step_meta *m, const uint32_t *slots,
                                             uint64_t num_slots, void *stream) {
    const char *op = "write_kv";
    if (!m) return fail_argument(op, "null meta");
    if (vo_status rc = refuse_if_fixed(m, op)) return rc;
    DeviceGuard guard(m->device);
    const uint64_t zero = 0;
    Packer pk(m);
    if (vo_status rc = upload_common(m, kSlots, op, m->pool_block_size ? m->pool_block_size : 1, 0,
                                     &zero, nullptr, num_slots, slots, nullptr, nullptr, nullptr, pk))
        return rc;
    if (!pk.fits()) {
        m->kind = kNone;
        return fail_capacity("step metadata bytes", pk.used(), m->buf_bytes);
    }
    if (vo_status rc = finish_upload(m, pk, static_cast<hipStream_t>(stream), op)) return rc;
    clear_error();
    return VO_OK;
}

namespace vo {

vo_status aux_upload(vo_step_meta *m, std::vector<uint32_t> &held, bool &valid, uint32_t *dev,
                     const uint32_t *values, uint64_t n, hipStream_t stream, const char *op) {
    if (valid && same_array(held, values, n)) return VO_OK;
    if (n > m->max_rows) return fail_capacity("rows per step", n, m->max_rows);
    if (n == 0) {
        held.clear();
        valid = true;
        return VO_OK;
    }
    uint8_t *host;
    hipError_t err = m->aux_stage.acquire(&host);
    if (err == hipSuccess) {
        std::memcpy(host, values, n * sizeof(uint32_t));
        err = m->aux_stage.commit(dev, n * sizeof(uint32_t), stream);
    }
    if (err != hipSuccess) {
        valid = false;
        return fail_device(op, err, hipGetErrorString(err));
    }
    held.assign(values, values + n);
    valid = true;
    return VO_OK;
}

}  // namespace vo

extern "C" int32_t vo_step_meta_sync_prefill(
    vo_step_meta *m, uint64_t block_size, uint64_t num_seqs, const uint64_t *table_off,
    const uint32_t *tables, const uint64_t *context_lens, const uint64_t *seq_row_starts,
    uint64_t num_rows, const uint32_t *positions, const uint32_t *slot_mapping,
    const uint64_t *row_seq, const uint64_t *row_num_keys, void *stream) {
    if (!m) return fail_argument("prefill", "null meta");
    if (holds_step(m, kPrefill, block_size, num_seqs, table_off, tables, num_rows, positions,
                   slot_mapping, row_seq, row_num_keys) &&
        same_array(m->context_lens, context_lens, num_seqs) &&
        same_array(m->seq_row_starts, seq_row_starts, num_seqs + 1)) {
        clear_error();
        return VO_OK;
    }
    return vo_step_meta_upload_prefill(m, block_size, num_seqs, table_off, tables, context_lens,
                                       seq_row_starts, num_rows, positions, slot_mapping, row_seq,
                                       row_num_keys, stream);
}

extern "C" int32_t vo_step_meta_sync_decode(vo_step_meta *m, uint64_t block_size,
                                            uint64_t num_seqs, const uint64_t *table_off,
                                            const uint32_t *tables, const uint32_t *positions,
                                            const uint32_t *slot_mapping, const uint64_t *row_seq,
                                            const uint64_t *row_num_keys, void *stream) {
    if (!m) return fail_argument("decode", "null meta");
    if (holds_step(m, kDecode, block_size, num_seqs, table_off, tables, num_seqs, positions,
                   slot_mapping, row_seq, row_num_keys)) {
        clear_error();
        return VO_OK;
    }
    return vo_step_meta_upload_decode(m, block_size, num_seqs, table_off, tables, positions,
                                      slot_mapping, row_seq, row_num_keys, stream);
}

extern "C" int32_t vo_step_meta_fix_launch(vo_step_meta *m, uint64_t work_headroom,
                                           uint64_t entry_headroom, void *stream) {
    const char *op = "fix_launch";
    if (!m) return fail_argument(op, "null meta");
    if (m->kind != kDecode || !m->decode_planned)
        return fail_shape(op, "the last upload must be a decode step");
    FixedLaunch f;
    f.on = true;
    f.seqs = m->num_seqs;
    f.entries_cap = std::min<uint64_t>(m->tables.size() + entry_headroom, m->max_entries);
    f.work_cap = std::min<uint64_t>(m->decode_parts + work_headroom, m->max_parts);
    f.has_positions = !m->positions.empty() || (m->num_rows == 0 && m->has_positions);
    f.streaming = m->plan.streaming;
    const uint64_t S = f.seqs;
    const uint64_t caps[kNumRegions] = {
        2, S + 1, f.entries_cap, S, S, f.has_positions ? S : 0, S, 3 * S,
        4 * f.work_cap, 2 * S, S, S, 0, 0, 0};
    uint64_t off = 0;
    for (int r = 0; r < kNumRegions; ++r) {
        off = align_up(off, 256);
        f.offset[r] = off;
        f.cap[r] = caps[r];
        off += caps[r] * sizeof(uint32_t);
    }
    f.bytes = off;
    if (f.bytes > m->buf_bytes) return fail_capacity("fixed-launch metadata bytes", f.bytes, m->buf_bytes);
    // Upload the current step again, in the fixed layout.
    const std::vector<uint64_t> table_off = m->table_off;
    const std::vector<uint32_t> tables = m->tables, slots = m->slots, positions = m->positions;
    std::vector<uint64_t> row_seq(m->row_seq.begin(), m->row_seq.end());
    std::vector<uint64_t> row_keys(m->row_num_keys.begin(), m->row_num_keys.end());
    const FixedLaunch saved = m->fixed;
    m->fixed = f;
    const int32_t rc = vo_step_meta_upload_decode(
        m, m->block_size, S, table_off.data(), tables.empty() ? nullptr : tables.data(),
        f.has_positions ? positions.data() : nullptr, slots.data(), row_seq.data(),
        row_keys.data(), stream);
    if (rc != VO_OK) m->fixed = saved;
    return rc;
}

extern "C" int32_t vo_step_meta_decode_plan(const vo_step_meta *m, uint64_t *work_items,
                                            uint64_t *partials, uint32_t *pack) {
    if (!m || !work_items || !partials || !pack) return fail_argument("decode_plan", "null argument");
    if (!m->decode_planned) return fail_argument("decode_plan", "the last upload has no decode plan");
    *work_items = m->plan.num_work;
    *partials = m->decode_parts;
    *pack = m->plan.pack ? m->plan.pack : 1;
    clear_error();
    return VO_OK;
}

extern "C" int32_t vo_step_meta_unfix_launch(vo_step_meta *m) {
    if (!m) return fail_argument("fix_launch", "null meta");
    m->fixed.on = false;
    clear_error();
    return VO_OK;
}

// ---------------------------------------------------------------------------
// Ops
// ---------------------------------------------------------------------------
namespace {

std::string layout_text(const vo_kv_layout &L) {
    return "KvLayout { num_layers: " + std::to_string(L.num_layers) +
           ", num_blocks: " + std::to_string(L.num_blocks) +
           ", block_size: " + std::to_string(L.block_size) +
           ", kv_heads: " + std::to_string(L.kv_heads) +
           ", head_dim: " + std::to_string(L.head_dim) + " }";
}

// arena/ops.rs:191-214 (check_attention) plus the pointer checks a C ABI needs.
vo_status check_attention(const char *op, const void *queries, uint64_t rows, uint64_t cols,
                          const vo_kv_pool *pool, uint64_t layer, const vo_step_meta *m,
                          const void *out, MetaKind want) {
    if (!pool || !m) return fail_argument(op, "null pool or meta");
    const vo_kv_layout &L = pool->layout;
    const bool shape_ok = rows == m->num_rows && cols % L.head_dim == 0 &&
                          (cols / L.head_dim) % L.kv_heads == 0 && layer < L.num_layers &&
                          m->block_size == L.block_size;
    if (!shape_ok || m->kind != want) {
        std::string msg = "queries [" + std::to_string(rows) + ", " + std::to_string(cols) + "], " +
                          std::to_string(m->num_rows) + " rows in metadata, block size " +
                          std::to_string(m->block_size) + ", layer " + std::to_string(layer) +
                          ", pool " + layout_text(L);
        if (m->kind != want)
            msg += want == kPrefill ? "; metadata is not a prefill upload"
                                    : "; metadata is not a decode upload";
        return fail_shape(op, msg);
    }
    if (rows == 0) return VO_OK;
    if (!queries || !out) return fail_argument(op, "null queries or output");
    if (!aligned16(queries) || !aligned16(out))
        return fail_argument(op, "queries and output must be 16-byte aligned");
    const uint64_t bytes = rows * cols * sizeof(uint16_t);
    if (overlaps(queries, bytes, out, bytes)) return fail_shape(op, "output overlaps queries");
    const uint64_t heads = cols / L.head_dim;
    if (heads > m->max_heads) return fail_capacity("query heads", heads, m->max_heads);
    if (heads > 0xffffull) return fail_capacity("query heads", heads, 0xffff);
    // attention.rs:130-147, against this pool's block count.
    if (m->max_block >= L.num_blocks)
        return check_block_tables(op, m->num_seqs, m->table_off.data(), m->tables.data(),
                                  L.num_blocks);
    return VO_OK;
}


}  // namespace

namespace {

// write_kv's checks: arena/ops.rs:116-127 (shape), cpu/mod.rs:265-272 (every
// slot in range before any write).
vo_status check_write(const vo_kv_pool *pool, uint64_t layer, uint64_t rows, uint64_t cols,
                      const vo_step_meta *m) {
    const char *op = "write_kv";
    const vo_kv_layout &L = pool->layout;
    const uint64_t slot_width = L.kv_heads * L.head_dim;
    // arena/ops.rs:116-127
    const bool shape_ok = rows == m->num_rows && cols == slot_width && layer < L.num_layers;
    if (!shape_ok || m->kind == kNone)
        return fail_shape(op, "keys [" + std::to_string(rows) + ", " + std::to_string(cols) +
                                  "], values [" + std::to_string(rows) + ", " +
                                  std::to_string(cols) + "], " + std::to_string(m->num_rows) +
                                  " slots, layer " + std::to_string(layer) + ", pool " +
                                  layout_text(L));
    // The write plan's runs were cut at the block size of the pool the
    // metadata was created for.
    if (m->pool_block_size != L.block_size)
        return fail_shape(op, "step metadata was created for a pool with block size " +
                                  std::to_string(m->pool_block_size) + ", pool " + layout_text(L));
    // cpu/mod.rs:265-272: every slot in range before any write.
    const uint64_t num_slots = vo_kv_layout_num_slots(&L);
    if (rows && m->max_slot >= num_slots) {
        for (uint32_t s : m->slots) {
            if (s >= num_slots) {
                Error e;
                e.status = VO_ERR_SLOT_OUT_OF_RANGE;
                e.op = op;
                e.value = s;
                e.limit = num_slots;
                e.message = std::string(op) + ": slot " + std::to_string(s) +
                            " out of range (pool has " + std::to_string(num_slots) + ")";
                return fail(e);
            }
        }
    }
    return VO_OK;
}

}  // namespace

extern "C" int32_t vo_write_kv(vo_kv_pool *pool, uint64_t layer, const void *keys,
                               const void *values, uint64_t rows, uint64_t cols,
                               const vo_step_meta *m, void *stream) {
    const char *op = "write_kv";
    if (!pool || !m) return fail_argument(op, "null pool or meta");
    const vo_kv_layout &L = pool->layout;
    if (vo_status rc = check_write(pool, layer, rows, cols, m)) return rc;
    if (rows == 0) {
        clear_error();
        return VO_OK;
    }
    if (!keys || !values) return fail_argument(op, "null keys or values");
    if (!aligned16(keys) || !aligned16(values))
        return fail_argument(op, "keys and values must be 16-byte aligned");
    DeviceGuard guard(pool->device);
    hipError_t err;
    if (kernels::cache_write_supported(static_cast<uint32_t>(L.head_dim),
                                       static_cast<uint32_t>(L.block_size)))
        err = kernels::launch_cache_write(pool->layer(layer), static_cast<const uint16_t *>(keys),
                                          static_cast<const uint16_t *>(values), m->write_plan,
                                          static_cast<hipStream_t>(stream));
    else
        err = kernels::launch_reshape_and_cache(
            pool->layer(layer), static_cast<const uint16_t *>(keys),
            static_cast<const uint16_t *>(values), m->d_write_slots, static_cast<uint32_t>(rows),
            static_cast<hipStream_t>(stream));
    return device_status(op, err);
}

extern "C" int32_t vo_write_kv_slots(vo_kv_pool *pool, uint64_t layer, const void *keys,
                                     const void *values, uint64_t rows, uint64_t cols,
                                     const uint32_t *slots, uint64_t num_slots, vo_step_meta *m,
                                     void *stream) {
    const char *op = "write_kv";
    if (!pool || !m) return fail_argument(op, "null pool or meta");
    if (num_slots && !slots) return fail_argument(op, "null slots");
    const vo_kv_layout &L = pool->layout;
    // arena/ops.rs:116-127, before anything is uploaded.
    if (rows != num_slots || cols != L.kv_heads * L.head_dim || layer >= L.num_layers)
        return fail_shape(op, "keys [" + std::to_string(rows) + ", " + std::to_string(cols) +
                                  "], values [" + std::to_string(rows) + ", " +
                                  std::to_string(cols) + "], " + std::to_string(num_slots) +
                                  " slots, layer " + std::to_string(layer) + ", pool " +
                                  layout_text(L));
    // The step's own slot mapping (the model passes meta.slot_mapping,
    // model.rs:289-292) is written through the step's plan; other slots
    // are uploaded first, replacing the meta's last upload.
    if (m->kind == kNone || !same_array(m->slots, slots, num_slots))
        if (int32_t rc = vo_step_meta_upload_slots(m, slots, num_slots, stream)) return rc;
    return vo_write_kv(pool, layer, keys, values, rows, cols, m, stream);
}

// ---------------------------------------------------------------------------
// RoPE
// ---------------------------------------------------------------------------

namespace {

// llama3_inv_freq (rope.rs:36-60) and RopeTable::new (rope.rs:62-84): every
// operation is the reference's f32 operation in its order, with no
// contraction, and cos/sin/pow come from the host libm as in the reference.
void rope_host_table(const vo_rope_config &c, uint64_t max_len, std::vector<float> &cos_t,
                     std::vector<float> &sin_t) {
#pragma clang fp contract(off)
    const uint64_t d_i = c.head_dim;
    const uint64_t half = d_i / 2;
    const float d = static_cast<float>(d_i);
    const float base = static_cast<float>(c.rope_theta);
    const float factor = static_cast<float>(c.factor);
    const float low = static_cast<float>(c.low_freq_factor);
    const float high = static_cast<float>(c.high_freq_factor);
    const float old_ctx = static_cast<float>(c.original_max_position_embeddings);
    const float low_freq_wavelen = old_ctx / low;
    const float high_freq_wavelen = old_ctx / high;
    const float pi = 3.14159265358979323846f;  // std::f32::consts::PI
    std::vector<float> inv(half);
    for (uint64_t i = 0; i < half; ++i) {
        const float raw = 1.0f / powf(base, static_cast<float>(2 * i) / d);
        const float wavelen = 2.0f * pi / raw;
        float r;
        if (wavelen < high_freq_wavelen) {
            r = raw;
        } else if (wavelen > low_freq_wavelen) {
            r = raw / factor;
        } else {
            const float smooth = (old_ctx / wavelen - low) / (high - low);
            r = (1.0f - smooth) * raw / factor + smooth * raw;
        }
        inv[i] = r;
    }
    cos_t.resize(max_len * half);
    sin_t.resize(max_len * half);
    for (uint64_t p = 0; p < max_len; ++p) {
        for (uint64_t i = 0; i < half; ++i) {
            const float th = static_cast<float>(p) * inv[i];
            cos_t[p * half + i] = cosf(th);
            sin_t[p * half + i] = sinf(th);
        }
    }
}

// cpu/mod.rs:232-247 and arena/ops.rs:86-96 for one operand of rope, whose
// positions are num_positions host values with maximum max_position (has:
// whether there are positions at all).
vo_status check_rope(const char *op, const vo_rope_table *t, uint64_t rows, uint64_t cols,
                     uint64_t head_dim, bool has, uint64_t num_positions,
                     const uint32_t *positions, uint32_t max_position) {
    const bool shape_ok = has && rows == num_positions && head_dim > 0 && head_dim % 2 == 0 &&
                          cols % head_dim == 0;
    if (!shape_ok)
        return fail_shape(op, "x [" + std::to_string(rows) + ", " + std::to_string(cols) + "], " +
                                  (has ? std::to_string(num_positions) : std::string("no")) +
                                  " positions, head_dim " + std::to_string(head_dim));
    if (head_dim != 2 * t->half)
        return fail_shape(op, "head_dim " + std::to_string(head_dim) + ", table built for " +
                                  std::to_string(2 * t->half));
    if (rows && max_position >= t->max_len) {
        // The first position past the table, in row order (cpu/mod.rs:241).
        uint64_t pos = max_position;
        for (uint64_t r = 0; r < num_positions; ++r) {
            if (positions[r] >= t->max_len) {
                pos = positions[r];
                break;
            }
        }
        Error e;
        e.status = VO_ERR_POSITION_OUT_OF_RANGE;
        e.op = "rope";
        e.value = pos;
        e.limit = t->max_len;
        e.message = "rope: position " + std::to_string(pos) + " beyond the precomputed table (" +
                    std::to_string(t->max_len) + ")";
        return fail(e);
    }
    return VO_OK;
}

// The device positions for rope over `positions` [rows]: the meta's own when
// its last upload holds exactly these, else its aux copy.
vo_status device_positions(vo_step_meta *m, const uint32_t *positions, uint64_t rows,
                           hipStream_t stream, const char *op, const uint32_t **out) {
    if (m->kind != kNone && m->has_positions && m->view.positions &&
        same_array(m->positions, positions, rows)) {
        *out = m->view.positions;
        return VO_OK;
    }
    if (vo_status rc = aux_upload(m, m->aux_pos, m->aux_pos_valid, m->d_aux_pos, positions, rows,
                                  stream, op))
        return rc;
    *out = m->d_aux_pos;
    return VO_OK;
}

// check_rope on the positions of the meta's last upload.
vo_status check_rope(const char *op, const vo_rope_table *t, uint64_t rows, uint64_t cols,
                     uint64_t head_dim, const vo_step_meta *m) {
    return check_rope(op, t, rows, cols, head_dim, m->has_positions, m->num_rows,
                      m->positions.data(), m->max_position);
}

}  // namespace

extern "C" int32_t vo_rope_table_create(const vo_rope_config *config, uint64_t max_len,
                                        int32_t device, vo_rope_table **out) {
    const char *op = "rope_table_create";
    if (!config || !out) return fail_argument(op, "null config or output");
    *out = nullptr;
    if (config->head_dim == 0 || config->head_dim % 2 != 0 || max_len == 0)
        return fail_shape(op, "head_dim must be even and non-zero, max_len non-zero");
    if (max_len > 0xffffffffull) return fail_capacity("rope positions (u32)", max_len, 0xffffffffull);
    DeviceGuard guard(device);
    if (!guard.ok()) return fail_device(op, hipErrorInvalidDevice, "hipSetDevice");
    std::vector<float> cos_t, sin_t;
    rope_host_table(*config, max_len, cos_t, sin_t);
    vo_rope_table *t = new (std::nothrow) vo_rope_table();
    if (!t) return fail_argument(op, "out of host memory");
    t->device = device;
    t->head_dim = config->head_dim;
    t->half = config->head_dim / 2;
    t->max_len = max_len;
    const size_t bytes = cos_t.size() * sizeof(float);
    hipError_t err = hipMalloc(reinterpret_cast<void **>(&t->d_cos), bytes);
    if (err == hipSuccess) err = hipMalloc(reinterpret_cast<void **>(&t->d_sin), bytes);
    if (err == hipSuccess) err = hipMemcpy(t->d_cos, cos_t.data(), bytes, hipMemcpyHostToDevice);
    if (err == hipSuccess) err = hipMemcpy(t->d_sin, sin_t.data(), bytes, hipMemcpyHostToDevice);
    if (err != hipSuccess) {
        vo_status rc = fail_device(op, err, hipGetErrorString(err));
        if (t->d_cos) (void)hipFree(t->d_cos);
        if (t->d_sin) (void)hipFree(t->d_sin);
        delete t;
        return rc;
    }
    *out = t;
    clear_error();
    return VO_OK;
}

extern "C" void vo_rope_table_destroy(vo_rope_table *t) {
    if (!t) return;
    DeviceGuard guard(t->device);
    (void)hipFree(t->d_cos);
    (void)hipFree(t->d_sin);
    delete t;
}

extern "C" int32_t vo_rope(const vo_rope_table *t, void *x, uint64_t rows, uint64_t cols,
                           uint64_t head_dim, const vo_step_meta *m, void *stream) {
    const char *op = "rope";
    if (!t || !m) return fail_argument(op, "null table or meta");
    if (vo_status rc = check_rope(op, t, rows, cols, head_dim, m)) return rc;
    if (rows == 0 || cols == 0) {
        clear_error();
        return VO_OK;
    }
    if (!x) return fail_argument(op, "null x");
    if (rows > kU32Limit || cols > kU32Limit) return fail_capacity("rope rows/cols (u32)", std::max(rows, cols), kU32Limit);
    if (t->half % 8 == 0 && !aligned16(x)) return fail_argument(op, "x must be 16-byte aligned");
    DeviceGuard guard(t->device);
    const hipError_t err = kernels::launch_rope_rows(
        static_cast<uint16_t *>(x), static_cast<uint32_t>(rows), static_cast<uint32_t>(cols),
        static_cast<uint32_t>(t->half), m->view.positions, t->d_cos, t->d_sin,
        static_cast<hipStream_t>(stream));
    return device_status(op, err);
}

extern "C" int32_t vo_rope_positions(const vo_rope_table *t, void *x, uint64_t rows,
                                     uint64_t cols, uint64_t head_dim, const uint32_t *positions,
                                     uint64_t num_positions, vo_step_meta *m, void *stream) {
    const char *op = "rope";
    if (!t || !m) return fail_argument(op, "null table or meta");
    if (num_positions && !positions) return fail_argument(op, "null positions");
    uint32_t max_position = 0;
    for (uint64_t r = 0; r < num_positions; ++r) max_position = std::max(max_position, positions[r]);
    if (vo_status rc = check_rope(op, t, rows, cols, head_dim, true, num_positions, positions,
                                  max_position))
        return rc;
    if (rows == 0 || cols == 0) {
        clear_error();
        return VO_OK;
    }
    if (!x) return fail_argument(op, "null x");
    if (rows > kU32Limit || cols > kU32Limit) return fail_capacity("rope rows/cols (u32)", std::max(rows, cols), kU32Limit);
    if (t->half % 8 == 0 && !aligned16(x)) return fail_argument(op, "x must be 16-byte aligned");
    DeviceGuard guard(t->device);
    const uint32_t *d_positions = nullptr;
    if (vo_status rc = device_positions(m, positions, rows, static_cast<hipStream_t>(stream),
                                        op, &d_positions))
        return rc;
    const hipError_t err = kernels::launch_rope_rows(
        static_cast<uint16_t *>(x), static_cast<uint32_t>(rows), static_cast<uint32_t>(cols),
        static_cast<uint32_t>(t->half), d_positions, t->d_cos, t->d_sin,
        static_cast<hipStream_t>(stream));
    return device_status(op, err);
}

extern "C" int32_t vo_rope_write_kv(vo_kv_pool *pool, uint64_t layer, const vo_rope_table *t,
                                    void *queries, uint64_t q_cols, const void *keys,
                                    const void *values, uint64_t rows, uint64_t kv_cols,
                                    const vo_step_meta *m, void *stream) {
    const char *op = "rope_write_kv";
    if (!pool || !t || !m) return fail_argument(op, "null pool, table or meta");
    const vo_kv_layout &L = pool->layout;
    if (vo_status rc = check_rope("rope", t, rows, q_cols, L.head_dim, m)) return rc;
    if (vo_status rc = check_rope("rope", t, rows, kv_cols, L.head_dim, m)) return rc;
    if (!kernels::cache_write_supported(static_cast<uint32_t>(L.head_dim),
                                        static_cast<uint32_t>(L.block_size)))
        return fail_unsupported(op, "the fused write needs block size 16 and head_dim 64 or 128");
    // write_kv's checks (arena/ops.rs:116-127, cpu/mod.rs:265-272).
    if (vo_status rc = check_write(pool, layer, rows, kv_cols, m)) return rc;
    if (q_cols % (L.kv_heads * L.head_dim) != 0)
        return fail_shape(op, "q_cols " + std::to_string(q_cols) + " is not a multiple of kv_heads * head_dim");
    if (rows == 0) {
        clear_error();
        return VO_OK;
    }
    if (!queries || !keys || !values) return fail_argument(op, "null queries, keys or values");
    if (!aligned16(queries) || !aligned16(keys) || !aligned16(values))
        return fail_argument(op, "queries, keys and values must be 16-byte aligned");
    if (overlaps(queries, rows * q_cols * 2, keys, rows * kv_cols * 2) ||
        overlaps(queries, rows * q_cols * 2, values, rows * kv_cols * 2))
        return fail_shape(op, "queries overlap keys or values");
    DeviceGuard guard(pool->device);
    const uint32_t group = static_cast<uint32_t>(q_cols / L.head_dim / L.kv_heads);
    const hipError_t err = kernels::launch_rope_cache(
        pool->layer(layer), static_cast<const uint16_t *>(queries), static_cast<uint32_t>(q_cols),
        static_cast<uint16_t *>(queries), static_cast<uint32_t>(q_cols), group,
        static_cast<const uint16_t *>(keys), static_cast<const uint16_t *>(values),
        static_cast<uint32_t>(kv_cols), m->write_plan, m->view.positions, t->d_cos, t->d_sin,
        static_cast<hipStream_t>(stream));
    return device_status(op, err);
}

extern "C" int32_t vo_qkv_rope_write_kv(vo_kv_pool *pool, uint64_t layer, const vo_rope_table *t,
                                        const void *qkv, uint64_t rows, uint64_t q_cols,
                                        uint64_t kv_cols, const vo_step_meta *m, void *q_out,
                                        void *stream) {
    const char *op = "rope_write_kv";
    if (!pool || !t || !m) return fail_argument(op, "null pool, table or meta");
    const vo_kv_layout &L = pool->layout;
    if (vo_status rc = check_rope("rope", t, rows, q_cols, L.head_dim, m)) return rc;
    if (vo_status rc = check_rope("rope", t, rows, kv_cols, L.head_dim, m)) return rc;
    if (!kernels::cache_write_supported(static_cast<uint32_t>(L.head_dim),
                                        static_cast<uint32_t>(L.block_size)))
        return fail_unsupported(op, "the fused write needs block size 16 and head_dim 64 or 128");
    if (vo_status rc = check_write(pool, layer, rows, kv_cols, m)) return rc;
    if (q_cols % (L.kv_heads * L.head_dim) != 0)
        return fail_shape(op, "q_cols " + std::to_string(q_cols) + " is not a multiple of kv_heads * head_dim");
    const uint64_t ld = q_cols + 2 * kv_cols;
    if (ld > kU32Limit) return fail_capacity("qkv columns (u32)", ld, kU32Limit);
    if (rows == 0) {
        clear_error();
        return VO_OK;
    }
    if (!qkv || !q_out) return fail_argument(op, "null qkv or q_out");
    if (!aligned16(qkv) || !aligned16(q_out))
        return fail_argument(op, "qkv and q_out must be 16-byte aligned");
    if (overlaps(qkv, rows * ld * 2, q_out, rows * q_cols * 2))
        return fail_shape(op, "q_out overlaps qkv");
    DeviceGuard guard(pool->device);
    const uint32_t group = static_cast<uint32_t>(q_cols / L.head_dim / L.kv_heads);
    const uint16_t *base = static_cast<const uint16_t *>(qkv);
    const hipError_t err = kernels::launch_rope_cache(
        pool->layer(layer), base, static_cast<uint32_t>(ld), static_cast<uint16_t *>(q_out),
        static_cast<uint32_t>(q_cols), group, base + q_cols, base + q_cols + kv_cols,
        static_cast<uint32_t>(ld), m->write_plan, m->view.positions, t->d_cos, t->d_sin,
        static_cast<hipStream_t>(stream));
    return device_status(op, err);
}

extern "C" int32_t vo_prefill_attention(const void *queries, uint64_t rows, uint64_t cols,
                                        const vo_kv_pool *pool, uint64_t layer,
                                        const vo_step_meta *m, void *out, void *stream) {
    const char *op = "prefill_attention";
    if (vo_status rc = check_attention(op, queries, rows, cols, pool, layer, m, out, kPrefill))
        return rc;
    if (rows == 0) {
        clear_error();
        return VO_OK;
    }
    const vo_kv_layout &L = pool->layout;
    const uint32_t heads = static_cast<uint32_t>(cols / L.head_dim);
    const float scale = 1.0f / std::sqrt(static_cast<float>(L.head_dim));  // attention.rs:88
    const uint32_t group = heads / static_cast<uint32_t>(L.kv_heads);
    DeviceGuard guard(pool->device);
    hipError_t err;
    if (m->prefill_planned &&
        kernels::prefill_mfma_supported(static_cast<uint32_t>(L.head_dim),
                                        static_cast<uint32_t>(L.block_size), group)) {
        // A mixed step's chunks and decode rows write disjoint rows of `out`
        // and read the pool only.  The decode rows (sequences with one new
        // row) run on the metadata's side stream, forked before the prefill
        // launch and joined after, so that the HBM-bound split-K workgroups
        // fill the wavefront slots the MFMA-bound prefill workgroups leave
        // free.
        const hipStream_t st = static_cast<hipStream_t>(stream);
        const bool overlap = m->decode_planned && mixed_overlap_enabled();
        if (overlap) {
            err = hipEventRecord(m->fork, st);
            if (err == hipSuccess) err = hipStreamWaitEvent(m->side, m->fork, 0);
            if (err != hipSuccess) return fail_device("prefill_attention", err, "stream fork");
        }
        err = kernels::launch_prefill_mfma(pool->layer(layer), m->view, m->prefill_plan,
                                           static_cast<const uint16_t *>(queries),
                                           static_cast<uint16_t *>(out), heads, scale,
                                           pool->num_cus, st);
        if (err == hipSuccess && m->decode_planned)
            err = kernels::launch_decode_mfma(pool->layer(layer), m->view, m->plan,
                                              static_cast<const uint16_t *>(queries),
                                              static_cast<uint16_t *>(out), heads, scale,
                                              decode_waves(), overlap ? m->side : st);
        if (overlap) {
            // Joined whatever happened above, so the caller's stream never
            // runs ahead of work left on the side stream.
            hipError_t j = hipEventRecord(m->join, m->side);
            if (j == hipSuccess) j = hipStreamWaitEvent(st, m->join, 0);
            if (err == hipSuccess) err = j;
        }
    } else {
        err = kernels::launch_attention_generic(
            pool->layer(layer), m->view, static_cast<const uint16_t *>(queries),
            static_cast<uint16_t *>(out), heads, scale, static_cast<hipStream_t>(stream));
    }
    return device_status(op, err);
}

extern "C" int32_t vo_decode_attention(const void *queries, uint64_t rows, uint64_t cols,
                                       const vo_kv_pool *pool, uint64_t layer,
                                       const vo_step_meta *m, void *out, void *stream) {
    const char *op = "decode_attention";
    if (vo_status rc = check_attention(op, queries, rows, cols, pool, layer, m, out, kDecode))
        return rc;
    if (rows == 0) {
        clear_error();
        return VO_OK;
    }
    const vo_kv_layout &L = pool->layout;
    const uint32_t heads = static_cast<uint32_t>(cols / L.head_dim);
    const uint32_t group = heads / static_cast<uint32_t>(L.kv_heads);
    const float scale = 1.0f / std::sqrt(static_cast<float>(L.head_dim));  // attention.rs:88
    DeviceGuard guard(pool->device);
    hipError_t err;
    if (kernels::decode_mfma_supported(static_cast<uint32_t>(L.head_dim),
                                       static_cast<uint32_t>(L.block_size), group) &&
        m->decode_planned) {
        err = kernels::launch_decode_mfma(pool->layer(layer), m->view, m->plan,
                                          static_cast<const uint16_t *>(queries),
                                          static_cast<uint16_t *>(out), heads, scale,
                                          decode_waves(), static_cast<hipStream_t>(stream));
    } else {
        err = kernels::launch_attention_generic(
            pool->layer(layer), m->view, static_cast<const uint16_t *>(queries),
            static_cast<uint16_t *>(out), heads, scale, static_cast<hipStream_t>(stream));
    }
    return device_status(op, err);
}

extern "C" int32_t vo_decode_attention_write_kv(const void *queries, uint64_t rows,
                                                uint64_t cols, const void *keys,
                                                const void *values, uint64_t kv_cols,
                                                vo_kv_pool *pool, uint64_t layer,
                                                const vo_step_meta *m, void *out, void *stream) {
    const char *op = "decode_attention_write_kv";
    if (!pool || !m) return fail_argument(op, "null pool or meta");
    if (vo_status rc = check_write(pool, layer, rows, kv_cols, m)) return rc;
    if (vo_status rc = check_attention(op, queries, rows, cols, pool, layer, m, out, kDecode))
        return rc;
    if (rows == 0) {
        clear_error();
        return VO_OK;
    }
    if (!keys || !values) return fail_argument(op, "null keys or values");
    if (!aligned16(keys) || !aligned16(values))
        return fail_argument(op, "keys and values must be 16-byte aligned");
    const vo_kv_layout &L = pool->layout;
    const uint32_t heads = static_cast<uint32_t>(cols / L.head_dim);
    const uint32_t group = heads / static_cast<uint32_t>(L.kv_heads);
    if (m->fused_write_ok && m->decode_planned &&
        kernels::decode_mfma_supported(static_cast<uint32_t>(L.head_dim),
                                       static_cast<uint32_t>(L.block_size), group)) {
        DeviceGuard guard(pool->device);
        const float scale = 1.0f / std::sqrt(static_cast<float>(L.head_dim));  // attention.rs:88
        const kernels::NewKeys nk{static_cast<const uint16_t *>(keys),
                                  static_cast<const uint16_t *>(values), m->d_write_slots};
        const hipError_t err = kernels::launch_decode_mfma(
            pool->layer(layer), m->view, m->plan, static_cast<const uint16_t *>(queries),
            static_cast<uint16_t *>(out), heads, scale, decode_waves(),
            static_cast<hipStream_t>(stream), &nk);
        return device_status(op, err);
    }
    // Otherwise the two ops in sequence, with the same results.
    if (const int32_t rc = vo_write_kv(pool, layer, keys, values, rows, kv_cols, m, stream))
        return rc;
    return vo_decode_attention(queries, rows, cols, pool, layer, m, out, stream);
}

extern "C" int32_t vo_prefill_meta_build_device(
    const uint32_t *seq_row_starts, const uint32_t *context_lens, const uint32_t *table_off,
    const uint32_t *tables, uint64_t num_seqs, uint64_t num_rows, uint64_t block_size,
    uint32_t *positions, uint32_t *slot_mapping, uint32_t *row_seq, uint32_t *row_num_keys,
    uint32_t *errors, void *stream) {
    const char *op = "prefill_meta_build_device";
    if (num_rows == 0) {
        clear_error();
        return VO_OK;
    }
    if (!seq_row_starts || !context_lens || !table_off || !tables || !positions ||
        !slot_mapping || !row_seq || !row_num_keys || !errors)
        return fail_argument(op, "null device array");
    if (num_seqs == 0 || block_size == 0) return fail_shape(op, "rows need a sequence and a block size");
    if (num_seqs > kU32Limit || num_rows > kU32Limit || block_size > kU32Limit)
        return fail_capacity("step metadata entries (u32)", std::max({num_seqs, num_rows, block_size}),
                             kU32Limit);
    const hipError_t err = kernels::launch_build_rows(
        seq_row_starts, context_lens, table_off, tables, static_cast<uint32_t>(num_seqs),
        static_cast<uint32_t>(num_rows), static_cast<uint32_t>(block_size), positions,
        slot_mapping, row_seq, row_num_keys, errors, static_cast<hipStream_t>(stream));
    return device_status(op, err);
}

extern "C" int32_t vo_kv_copy_blocks(vo_kv_pool *pool, const uint32_t *src, const uint32_t *dst,
                                     uint64_t count, void *stream) {
    const char *op = "copy_blocks";
    if (!pool) return fail_argument(op, "null pool");
    if (count == 0) {
        clear_error();
        return VO_OK;
    }
    if (!src || !dst) return fail_argument(op, "null block ids");
    const vo_kv_layout &L = pool->layout;
    std::vector<uint8_t> is_dst(L.num_blocks, 0);
    for (uint64_t i = 0; i < count; ++i) {
        for (uint32_t b : {src[i], dst[i]}) {
            if (b >= L.num_blocks) {
                Error e;
                e.status = VO_ERR_BLOCK_OUT_OF_RANGE;
                e.op = op;
                e.value = b;
                e.limit = L.num_blocks;
                e.message = std::string(op) + ": block " + std::to_string(b) +
                            " out of range (pool has " + std::to_string(L.num_blocks) + ")";
                return fail(e);
            }
        }
        if (is_dst[dst[i]]) return fail_shape(op, "block " + std::to_string(dst[i]) + " is a destination twice");
        is_dst[dst[i]] = 1;
    }
    for (uint64_t i = 0; i < count; ++i)
        if (is_dst[src[i]]) return fail_shape(op, "block " + std::to_string(src[i]) + " is both a source and a destination");
    DeviceGuard guard(pool->device);
    const uint64_t block_elems = L.kv_heads * L.block_size * L.head_dim;
    hipError_t err = hipSuccess;
    for (uint64_t i0 = 0; i0 < count && err == hipSuccess; i0 += kernels::kMaxBlockPairs) {
        kernels::BlockPairs pairs{};
        const uint32_t n = static_cast<uint32_t>(std::min<uint64_t>(kernels::kMaxBlockPairs, count - i0));
        for (uint32_t j = 0; j < n; ++j) {
            pairs.src[j] = src[i0 + j];
            pairs.dst[j] = dst[i0 + j];
        }
        err = kernels::launch_copy_blocks(pool->base, L.num_layers, pool->layer_elems, block_elems,
                                          pairs, n, static_cast<hipStream_t>(stream));
    }
    return device_status(op, err);
}

extern "C" int32_t vo_gather_kv(const vo_kv_pool *pool, uint64_t layer, const vo_step_meta *m,
                                uint64_t seq, uint64_t num_keys, void *out_keys,
                                void *out_values, void *stream) {
    const char *op = "read";
    if (!pool || !m) return fail_argument(op, "null pool or meta");
    const vo_kv_layout &L = pool->layout;
    if (layer >= L.num_layers || seq >= m->num_seqs || m->block_size != L.block_size ||
        (m->kind != kPrefill && m->kind != kDecode))
        return fail_shape(op, "layer " + std::to_string(layer) + ", sequence " +
                                  std::to_string(seq) + " of " + std::to_string(m->num_seqs) +
                                  ", pool " + layout_text(L));
    const uint64_t t0 = m->table_off[seq], t1 = m->table_off[seq + 1];
    if (vo_status rc = check_covers(op, t1 - t0, num_keys, L.block_size, seq)) return rc;
    const uint64_t one_off[2] = {0, t1 - t0};
    if (vo_status rc = check_block_tables(op, 1, one_off, m->tables.data() + t0, L.num_blocks))
        return rc;
    if (num_keys > kU32Limit) return fail_capacity("keys", num_keys, kU32Limit);
    if (num_keys == 0) {
        clear_error();
        return VO_OK;
    }
    if (!out_keys || !out_values) return fail_argument(op, "null outputs");
    if (!aligned16(out_keys) || !aligned16(out_values))
        return fail_argument(op, "outputs must be 16-byte aligned");
    DeviceGuard guard(pool->device);
    hipError_t err = kernels::launch_gather_kv(pool->layer(layer), m->view.tables + t0,
                                               static_cast<uint32_t>(num_keys),
                                               static_cast<uint16_t *>(out_keys),
                                               static_cast<uint16_t *>(out_values),
                                               static_cast<hipStream_t>(stream));
    return device_status(op, err);
}

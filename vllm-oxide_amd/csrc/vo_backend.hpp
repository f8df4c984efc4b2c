// vo_backend.hpp -- private to the library: the opaque C types behind the
// ABI (KV pool, step metadata, RoPE table) and the helpers the op files share.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <string>
#include <unordered_map>
#include <vector>

#include "kernels/vo_kernels.hpp"
#include "vo_paged.hpp"

namespace vo {

constexpr uint32_t kSkipSlot = 0xffffffffu;  // row superseded by a later row
constexpr uint64_t kU32Limit = 0x7fffffffull;

// Makes `device` current for the scope and restores the caller's device.
class DeviceGuard {
   public:
    explicit DeviceGuard(int device) {
        if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
        if (prev_ != device) ok_ = hipSetDevice(device) == hipSuccess;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev_ >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev_) (void)hipSetDevice(prev_);
    }
    bool ok() const { return ok_; }

   private:
    int prev_ = -1;
    bool ok_ = true;
};

inline uint64_t align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

inline int env_int(const char *name, int fallback) {
    const char *v = std::getenv(name);
    if (!v || !*v) return fallback;
    return std::atoi(v);
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline bool overlaps(const void *a, uint64_t a_bytes, const void *b, uint64_t b_bytes) {
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a_bytes && b_bytes && a0 < b0 + b_bytes && b0 < a0 + a_bytes;
}

inline vo_status device_status(const char *op, hipError_t err) {
    if (err != hipSuccess) return fail_device(op, err, hipGetErrorString(err));
    clear_error();
    return VO_OK;
}

enum MetaKind { kNone = 0, kPrefill = 1, kDecode = 2, kSlots = 3 };

// The arrays of one upload in the metadata buffer.  Ordinary uploads pack
// them back to back; with fixed launch shapes each has a fixed offset.
enum Region {
    kRegCounts = 0,  // [2]: split-K work items, rows to reduce (read by the kernels)
    kRegTableOff,
    kRegTables,
    kRegRowSeq,
    kRegRowKeys,
    kRegPositions,
    kRegSlots,
    kRegSegments,
    kRegWork,
    kRegRowInfo,
    kRegReduceRows,
    kRegLastRows,
    kRegPrefillWork,
    kRegPrefillPipe,
    kRegMates,
    kNumRegions
};

// Fixed launch shapes (vo_step_meta_fix_launch): decode uploads of `seqs`
// sequences put every array at a fixed offset of the metadata buffer, sized
// by these capacities, and the decode kernels are launched for `work_cap`
// work items and `seqs` rows to reduce, reading the step's real counts from
// the device.  Every launch the step makes then has the same arguments and
// grid from one step to the next, so a HIP graph recorded once replays them.
struct FixedLaunch {
    bool on = false;
    uint64_t seqs = 0;
    uint64_t entries_cap = 0;
    uint64_t work_cap = 0;
    bool has_positions = false;
    bool streaming = false;
    uint64_t offset[kNumRegions] = {};  // bytes
    uint64_t cap[kNumRegions] = {};     // u32 elements
    uint64_t bytes = 0;
};

// Keys per split-K split of the decode kernels (a multiple of 32; the same
// for every row and batch, so a row's arithmetic does not depend on the
// batch) and wavefronts per decode workgroup.  VO_DECODE_SPLIT and
// VO_DECODE_WAVES override them (tuning knobs).
uint64_t decode_split_keys();
int decode_waves();

// A row's last, shorter split in the decode work order (keys < split size).
struct TailItem {
    uint32_t keys, row, split;
};

// Pinned host staging of one kind of upload, double-buffered.  The host fills
// one buffer while the copy out of the other may still be in flight, so an
// upload waits on the host only when both buffers' copies are still pending
// (a third upload before the first one's copy ran).
struct Staging {
    uint8_t *buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
    int cur = 0;

    hipError_t create(uint64_t bytes) {
        for (int i = 0; i < 2; ++i) {
            hipError_t err = hipHostMalloc(reinterpret_cast<void **>(&buf[i]), bytes, hipHostMallocDefault);
            if (err == hipSuccess) err = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
            if (err != hipSuccess) return err;
        }
        return hipSuccess;
    }
    void destroy() {
        for (int i = 0; i < 2; ++i) {
            if (pending[i] && done[i]) (void)hipEventSynchronize(done[i]);
            if (done[i]) (void)hipEventDestroy(done[i]);
            if (buf[i]) (void)hipHostFree(buf[i]);
            buf[i] = nullptr;
            done[i] = nullptr;
            pending[i] = false;
        }
    }
    // The buffer the next upload fills.  Its last copy was enqueued two
    // uploads ago; the host waits only if that copy has not run yet.
    hipError_t acquire(uint8_t **host) {
        if (pending[cur]) {
            hipError_t err = hipEventQuery(done[cur]);
            if (err == hipErrorNotReady) err = hipEventSynchronize(done[cur]);
            if (err != hipSuccess) return err;
            pending[cur] = false;
        }
        *host = buf[cur];
        return hipSuccess;
    }
    uint8_t *current() const { return buf[cur]; }
    // Copies the first `bytes` of the current buffer to `dst` on `stream`
    // and moves on to the other buffer.
    hipError_t commit(void *dst, uint64_t bytes, hipStream_t stream) {
        hipError_t err = hipMemcpyAsync(dst, buf[cur], bytes, hipMemcpyHostToDevice, stream);
        if (err == hipSuccess) err = hipEventRecord(done[cur], stream);
        if (err != hipSuccess) return err;
        pending[cur] = true;
        cur ^= 1;
        return hipSuccess;
    }
};

}  // namespace vo

struct vo_kv_pool {
    vo_kv_layout layout{};
    int device = 0;
    int num_cus = 256;
    uint16_t *base = nullptr;   // [layers][K|V][layer_elems] bf16
    uint64_t layer_elems = 0;   // elements of one layer's K (or V)
    uint64_t bytes = 0;

    vo::kernels::PoolLayer layer(uint64_t l) const {
        vo::kernels::PoolLayer p;
        p.k = base + l * 2 * layer_elems;
        p.v = p.k + layer_elems;
        p.kv_heads = static_cast<uint32_t>(layout.kv_heads);
        p.head_dim = static_cast<uint32_t>(layout.head_dim);
        p.block_size = static_cast<uint32_t>(layout.block_size);
        p.elems = layer_elems;
        return p;
    }
};

struct vo_step_meta {
    int device = 0;
    int num_cus = 256;
    uint64_t pool_block_size = 0;
    uint64_t kv_heads = 0;
    uint64_t head_dim = 0;

    uint64_t max_seqs = 0, max_rows = 0, max_entries = 0, max_heads = 0, max_parts = 0;

    vo::MetaKind kind = vo::kNone;
    uint64_t block_size = 0;
    uint64_t num_seqs = 0;
    uint64_t num_rows = 0;

    // Host copies, for validation with the reference's error semantics.
    std::vector<uint64_t> table_off;    // [S+1]
    std::vector<uint32_t> tables;       // [entries]
    std::vector<uint32_t> slots;        // [T] as given
    std::vector<uint32_t> row_seq;      // [T]
    std::vector<uint32_t> row_num_keys; // [T]
    uint32_t max_block = 0;             // max table entry (0 if none)
    uint32_t max_slot = 0;              // max slot (0 if none)
    bool has_positions = false;         // positions were uploaded (RoPE needs them)
    std::vector<uint32_t> positions;    // [T] when uploaded
    uint32_t max_position = 0;          // largest position (0 if none)

    // Device buffer and its pinned staging (two buffers of the same size).
    uint8_t *d_buf = nullptr;
    vo::Staging stage;
    uint64_t buf_bytes = 0;
    // A mixed step's decode rows run on `side`, forked from and joined back
    // into the caller's stream, beside the prefill chunks.
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;

    // Split-K partials (fp32).
    float *d_part_acc = nullptr;
    float *d_part_ml = nullptr;

    vo::kernels::MetaView view{};
    const uint32_t *d_write_slots = nullptr;  // slots with superseded rows = kSkipSlot
    vo::kernels::WritePlan write_plan{};      // runs of consecutive slots inside one block
    vo::kernels::DecodePlan plan{};
    bool decode_planned = false;
    bool slots_repeat = false;  // a slot appears in two rows of the step
    // Decode step whose new keys can be cached by the decode launch itself
    // (vo_decode_attention_write_kv): no slot repeats and no row reads a
    // block holding another row's new slot.
    bool fused_write_ok = false;
    std::vector<vo::TailItem> tail_items;  // scratch of plan_decode (capacity kept across steps)
    std::vector<uint8_t> block_seen;   // scratch of plan_decode: one byte per physical block
    std::vector<uint64_t> seq_keys;    // scratch of plan_decode: keys read per sequence
    std::vector<uint32_t> decode_rows; // rows of a prefill step planned on the decode kernel
    uint64_t decode_parts = 0;         // split-K partials of the plan (work items before packing)
    std::unordered_map<uint64_t, uint32_t> pack_open;  // scratch of plan_decode: open packs by hash
    std::vector<uint32_t> pack_fill;                   // scratch of plan_decode: rows per pack
    vo::kernels::PrefillPlan prefill_plan{};
    bool prefill_planned = false;  // rows are regular: one contiguous run per sequence

    vo::FixedLaunch fixed;
    const uint32_t *d_counts = nullptr;  // [2] device copy of the plan's counts
    uint32_t *h_counts = nullptr;        // their place in the staging buffer

    // Rows the LM head reads (PrefillMeta::last_rows, paged.rs:153-159): each
    // sequence's last row for a prefill upload, every row for a decode upload.
    const uint32_t *d_last_rows = nullptr;  // [num_seqs]
    bool last_rows_ok = false;              // false: a sequence has no rows

    // Token ids of the step (Llama::prefill/decode `tokens`, model.rs:221-243),
    // uploaded apart from the metadata: host copy for embed's check, device
    // copy for the kernel, pinned staging for the copy.
    std::vector<uint32_t> tokens;
    uint32_t *d_tokens = nullptr;   // [max_rows]
    vo::Staging tokens_stage;       // 2 x [max_rows], pinned
    bool has_tokens = false;

    // A prefill upload's per-sequence inputs, kept to compare a later
    // vo_step_meta_sync_prefill with.
    std::vector<uint64_t> context_lens;    // [S]
    std::vector<uint64_t> seq_row_starts;  // [S+1]

    // Arrays the trait-shaped ops bring with each call (vo_rope_positions'
    // positions, vo_gather_rows' rows) when they are not the current
    // upload's: device copies of their own, refilled only when the content
    // changes (compared with the host copies), through pinned staging.
    std::vector<uint32_t> aux_pos;       // host copy of d_aux_pos
    bool aux_pos_valid = false;
    uint32_t *d_aux_pos = nullptr;       // [max_rows]
    std::vector<uint32_t> aux_rows;      // host copy of d_aux_rows
    bool aux_rows_valid = false;
    uint32_t *d_aux_rows = nullptr;      // [max_rows]
    vo::Staging aux_stage;               // 2 x [max_rows] u32, pinned
};

namespace vo {

// A device copy of the n host values `values` in `dev` (one of the meta's
// aux arrays, of max_rows entries), whose host copy is `held`: refilled by
// one async copy from the meta's pinned staging on `stream` when the content
// differs, else left as it is.  VO_ERR_CAPACITY past max_rows.
vo_status aux_upload(vo_step_meta *m, std::vector<uint32_t> &held, bool &valid, uint32_t *dev,
                     const uint32_t *values, uint64_t n, hipStream_t stream, const char *op);

}  // namespace vo

struct vo_rope_table {
    int device = 0;
    uint64_t head_dim = 0, half = 0, max_len = 0;
    float *d_cos = nullptr;  // [max_len][half]
    float *d_sin = nullptr;
};

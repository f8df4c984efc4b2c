// vo_decode_static.hip -- decode attention that allocates nothing
// (vo_decode_attention_static): the split-K work plan and the fp32 partials
// live in one file-scope device array, and the step's metadata is read from
// device memory the caller owns.
//
// For callers that cannot allocate device memory: code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc.  It is
// Backend::decode_attention (crates/engine/src/backend/mod.rs:137-149) on the
// same kernels as vo_decode_attention, with DecodeMeta::new's canonical rows
// (paged.rs:189-209: row s is sequence s) given as device u32 arrays:
// CSR table offsets [S+1], tables [entries], key counts [S] (context + 1).
//
// Scratch.  `scratch` holds, per call: the plan's two counts, row_info [S][2],
// reduce_rows [S], work [cap][4] and the partials (m, l) [cap][heads][2] and
// acc [cap][heads][head_dim] fp32, cap = S * ceil(max_keys / split) work
// items.  Each GPU holds its own copy, whose address hipGetSymbolAddress
// gives once per device (the array's name is not a device address in host
// code).  Every call on a GPU shares that copy: calls that overlap on one GPU
// (two streams, two threads) race, and a call reads nothing an earlier call
// left there -- the plan kernel writes every count, row record and work item
// before the decode kernels read them, and each partial is written before it
// is read.
//
// Plan on the device (decode_static_plan_kernel, one workgroup): checks what
// the host checks for vo_decode_attention -- coverage (paged.rs:64-80), every
// table entry < num_blocks (attention.rs:130-147), plus the bounds this call
// relies on (keys <= max_keys, offsets ascending and within num_entries) --
// and on any failure sets *errors = 1 and plans every row as zero keys, so
// the decode kernels read no pool memory and write zeros.  Otherwise row s
// gets ceil(keys / split) items in row order and the same split size as
// vo_decode_attention, so its output is bitwise that entry point's.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>

#include "vo_backend.hpp"

using namespace vo;

namespace {

// 32 MiB per device: e.g. 256 sequences of up to 8192 keys at 32 query heads
// of 128 dims (1280 work items: 21 MB of partials), or 64 of up to 4096 keys
// at 64 heads.
constexpr uint64_t kScratchBytes = 32ull << 20;
constexpr uint64_t kMaxSeqs = 4096;
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

std::mutex g_scratch_mutex;
uint8_t *g_scratch_ptr[kMaxDevices] = {};

// The device address of this device's `scratch`, looked up on the first call
// on each device (with that device current) and kept.
vo_status scratch_of(int device, const char *op, uint8_t **out) {
    if (device < 0 || device >= kMaxDevices)
        return fail_capacity("device ordinal", static_cast<uint64_t>(device), kMaxDevices - 1);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[device]) {
        void *p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !p) return fail_device(op, err, "hipGetSymbolAddress(scratch)");
        g_scratch_ptr[device] = static_cast<uint8_t *>(p);
    }
    *out = g_scratch_ptr[device];
    return VO_OK;
}

// Byte offsets of the plan's arrays inside the scratch for S sequences, cap
// work items, `heads` query heads of hd dims; total = bytes used.
struct ScratchLayout {
    uint64_t counts, row_info, reduce_rows, work, part_ml, part_acc, total;
    ScratchLayout(uint64_t S, uint64_t cap, uint64_t heads, uint64_t hd) {
        uint64_t at = 0;
        auto take = [&](uint64_t bytes) {
            const uint64_t o = at;
            at = align_up(at + bytes, 256);
            return o;
        };
        counts = take(2 * 4);
        row_info = take(2 * S * 4);
        reduce_rows = take(S * 4);
        work = take(4 * cap * 4);
        part_ml = take(cap * heads * 2 * 4);
        part_acc = take(cap * heads * hd * 4);
        total = at;
    }
};

constexpr int kPlanThreads = 1024;

// Inclusive prefix sum over the workgroup (kPlanThreads threads), in
// thread order; *total receives the sum of all values.
__device__ uint32_t block_scan(uint32_t v, uint32_t *s_wave, uint32_t *total) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (uint32_t off = 1; off < 64; off <<= 1) {
        const uint32_t u = __shfl_up(v, off, 64);
        if (lane >= off) v += u;
    }
    if (lane == 63) s_wave[wave] = v;
    __syncthreads();
    uint32_t before = 0, all = 0;
    for (uint32_t w = 0; w < kPlanThreads / 64; ++w) {
        const uint32_t x = s_wave[w];
        if (w < wave) before += x;
        all += x;
    }
    __syncthreads();  // s_wave is reused by the next scan
    *total = all;
    return v + before;
}

__global__ __launch_bounds__(kPlanThreads) void decode_static_plan_kernel(
    const uint32_t *__restrict__ table_off, const uint32_t *__restrict__ tables,
    const uint32_t *__restrict__ row_num_keys, uint32_t num_seqs, uint32_t num_entries,
    uint32_t num_blocks, uint32_t block_size, uint32_t split_keys, uint32_t max_keys,
    uint32_t *__restrict__ counts, uint32_t *__restrict__ row_info,
    uint32_t *__restrict__ reduce_rows, uint32_t *__restrict__ work,
    uint32_t *__restrict__ errors) {
    __shared__ uint32_t s_err;
    __shared__ uint32_t s_wave[kPlanThreads / 64];
    const uint32_t tid = threadIdx.x;
    if (tid == 0) s_err = 0;
    __syncthreads();
    // Per-sequence bounds: offsets ascending and inside the tables, keys
    // within max_keys and covered by the table (paged.rs:64-80).
    for (uint32_t s = tid; s < num_seqs; s += kPlanThreads) {
        const uint32_t o0 = table_off[s], o1 = table_off[s + 1];
        const uint32_t nk = row_num_keys[s];
        const bool bad = o1 < o0 || o1 > num_entries || nk > max_keys ||
                         o1 - o0 < (nk + block_size - 1) / block_size;
        if (bad) atomicOr(&s_err, 1u);
    }
    __syncthreads();
    // Every entry of every table < num_blocks (attention.rs:130-147); only
    // read once the offsets are known to lie inside the tables.
    if (s_err == 0) {
        const uint32_t e0 = table_off[0], e1 = table_off[num_seqs];
        for (uint32_t i = e0 + tid; i < e1; i += kPlanThreads)
            if (tables[i] >= num_blocks) atomicOr(&s_err, 1u);
    }
    __syncthreads();
    const bool err = s_err != 0;
    if (err && tid == 0) errors[0] = 1u;

    // Contiguous rows per thread, so the scans keep row order.
    const uint32_t per = (num_seqs + kPlanThreads - 1) / kPlanThreads;
    const uint32_t r0 = min(tid * per, num_seqs), r1 = min(r0 + per, num_seqs);
    auto splits = [&](uint32_t s) -> uint32_t {
        const uint32_t nk = err ? 0u : row_num_keys[s];
        return nk ? (nk + split_keys - 1) / split_keys : 1u;
    };
    uint32_t my_items = 0, my_red = 0;
    for (uint32_t s = r0; s < r1; ++s) {
        const uint32_t n = splits(s);
        my_items += n;
        my_red += n > 1;
    }
    uint32_t total_items, total_red;
    uint32_t item = block_scan(my_items, s_wave, &total_items) - my_items;
    uint32_t red = block_scan(my_red, s_wave, &total_red) - my_red;
    const uint32_t blocks_per_split = split_keys / block_size;
    for (uint32_t s = r0; s < r1; ++s) {
        const uint32_t n = splits(s);
        const uint32_t nk = err ? 0u : row_num_keys[s];
        const uint32_t base = err ? 0u : table_off[s];
        row_info[2 * s] = item;
        row_info[2 * s + 1] = n;
        for (uint32_t sp = 0; sp < n; ++sp, ++item) {
            uint32_t *w = work + 4 * static_cast<uint64_t>(item);
            w[0] = s;
            w[1] = sp;
            w[2] = base + sp * blocks_per_split;
            w[3] = nk;
        }
        if (n > 1) reduce_rows[red++] = s;
    }
    if (tid == 0) {
        counts[0] = total_items;
        counts[1] = total_red;
    }
}

}  // namespace

extern "C" int32_t vo_decode_attention_static(const void *queries, uint64_t rows, uint64_t cols,
                                              const vo_kv_pool *pool, uint64_t layer,
                                              const uint32_t *table_off, const uint32_t *tables,
                                              uint64_t num_entries, const uint32_t *row_num_keys,
                                              uint64_t max_keys, void *out, uint32_t *errors,
                                              void *stream) {
    const char *op = "decode_attention";
    if (!pool) return fail_argument(op, "null pool");
    const vo_kv_layout &L = pool->layout;
    // arena/ops.rs:191-214 on what the host knows: the shapes.
    if (cols % L.head_dim != 0 || (cols / L.head_dim) % L.kv_heads != 0 || layer >= L.num_layers)
        return fail_shape(op, "queries [" + std::to_string(rows) + ", " + std::to_string(cols) +
                                  "], layer " + std::to_string(layer) + ", pool of " +
                                  std::to_string(L.num_layers) + " layers, " +
                                  std::to_string(L.kv_heads) + " KV heads of " +
                                  std::to_string(L.head_dim));
    if (rows == 0) {
        clear_error();
        return VO_OK;
    }
    const uint64_t heads = cols / L.head_dim;
    const uint32_t group = static_cast<uint32_t>(heads / L.kv_heads);
    if (!kernels::decode_mfma_supported(static_cast<uint32_t>(L.head_dim),
                                        static_cast<uint32_t>(L.block_size), group))
        return fail_unsupported(op, "needs block size 16, head_dim 64 or 128 and at most 16 query "
                                    "heads per KV head");
    if (!queries || !out || !table_off || !tables || !row_num_keys || !errors)
        return fail_argument(op, "null queries, output, metadata or errors");
    if (!aligned16(queries) || !aligned16(out))
        return fail_argument(op, "queries and output must be 16-byte aligned");
    const uint64_t qbytes = rows * cols * sizeof(uint16_t);
    if (overlaps(queries, qbytes, out, qbytes)) return fail_shape(op, "output overlaps queries");
    if (rows > kMaxSeqs) return fail_capacity("sequences per static decode call", rows, kMaxSeqs);
    if (num_entries > kU32Limit) return fail_capacity("block-table entries (u32)", num_entries, kU32Limit);
    if (max_keys > kU32Limit) return fail_capacity("keys per row (u32)", max_keys, kU32Limit);
    const uint64_t split = decode_split_keys();
    if (split % L.block_size != 0) return fail_unsupported(op, "split size not a multiple of the block size");
    const uint64_t cap = rows * std::max<uint64_t>(1, (max_keys + split - 1) / split);
    const ScratchLayout sl(rows, cap, heads, L.head_dim);
    if (sl.total > kScratchBytes)
        return fail_capacity("static decode scratch bytes", sl.total, kScratchBytes);
    DeviceGuard guard(pool->device);
    if (!guard.ok()) return fail_device(op, hipErrorInvalidDevice, "hipSetDevice");
    uint8_t *base = nullptr;
    if (vo_status rc = scratch_of(pool->device, op, &base)) return rc;

    const hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t *counts = reinterpret_cast<uint32_t *>(base + sl.counts);
    uint32_t *row_info = reinterpret_cast<uint32_t *>(base + sl.row_info);
    uint32_t *reduce_rows = reinterpret_cast<uint32_t *>(base + sl.reduce_rows);
    uint32_t *work = reinterpret_cast<uint32_t *>(base + sl.work);
    hipLaunchKernelGGL(decode_static_plan_kernel, dim3(1), dim3(kPlanThreads), 0, st, table_off,
                       tables, row_num_keys, static_cast<uint32_t>(rows),
                       static_cast<uint32_t>(num_entries), static_cast<uint32_t>(L.num_blocks),
                       static_cast<uint32_t>(L.block_size), static_cast<uint32_t>(split),
                       static_cast<uint32_t>(max_keys), counts, row_info, reduce_rows, work,
                       errors);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail_device(op, err, hipGetErrorString(err));

    // The decode kernels of vo_decode_attention, launched for the capacity;
    // they stop at the plan's counts, which the plan kernel wrote.
    kernels::MetaView view{};
    view.tables = tables;
    view.num_rows = static_cast<uint32_t>(rows);
    view.num_seqs = static_cast<uint32_t>(rows);
    kernels::DecodePlan plan{};
    plan.work = work;
    plan.row_info = row_info;
    plan.reduce_rows = reduce_rows;
    plan.num_work = static_cast<uint32_t>(cap);
    plan.num_reduce_rows = static_cast<uint32_t>(rows);
    plan.split_keys = static_cast<uint32_t>(split);
    plan.part_acc = reinterpret_cast<float *>(base + sl.part_acc);
    plan.part_ml = reinterpret_cast<float *>(base + sl.part_ml);
    plan.streaming = false;  // blocks may be shared; either load path gives the same bits
    plan.counts = counts;
    plan.launch_work = static_cast<uint32_t>(cap);
    plan.launch_reduce = static_cast<uint32_t>(rows);
    plan.mates = nullptr;
    plan.pack = 1;
    const float scale = 1.0f / std::sqrt(static_cast<float>(L.head_dim));  // attention.rs:88
    err = kernels::launch_decode_mfma(pool->layer(layer), view, plan,
                                      static_cast<const uint16_t *>(queries),
                                      static_cast<uint16_t *>(out), static_cast<uint32_t>(heads),
                                      scale, decode_waves(), st);
    return device_status(op, err);
}

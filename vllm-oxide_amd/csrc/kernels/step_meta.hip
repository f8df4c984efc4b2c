// step_meta.hip -- a step's per-row paged-KV metadata, built on the device.
//
// PrefillMeta::new (crates/engine/src/backend/paged.rs:117-143) flattens a
// step's sequences into rows: the rows of sequence s are seq_row_starts[s] ..
// seq_row_starts[s+1], row i of them sits at position context_lens[s] + i,
// reads position + 1 keys, and its new K/V go to slot_of(table_s, position)
// = table_s[position / bs] * bs + position % bs (paged.rs:47-52, u32
// arithmetic).  DecodeMeta::new (paged.rs:189-209) is the case of one row per
// sequence.  The reference builds these arrays on the host every step; a
// caller that keeps its batch state in device memory builds them here with
// no host round trip.
//
// One thread per row finds its sequence by binary search over
// seq_row_starts.  The coverage check of paged.rs:64-80 runs per row: a
// position past its sequence's table gets slot 0xffffffff and sets *errors to
// 1 (a plain store; every writer stores the same value).
//
// Roofline: HBM / launch latency; 16 bytes written per row plus a table read.
#include "vo_device.hpp"
#include "vo_kernels.hpp"

namespace vo {
namespace kernels {

namespace {

__global__ __launch_bounds__(256) void build_rows_kernel(
    const uint32_t *__restrict__ seq_row_starts, const uint32_t *__restrict__ context_lens,
    const uint32_t *__restrict__ table_off, const uint32_t *__restrict__ tables,
    uint32_t num_seqs, uint32_t num_rows, uint32_t block_size, uint32_t *__restrict__ positions,
    uint32_t *__restrict__ slot_mapping, uint32_t *__restrict__ row_seq,
    uint32_t *__restrict__ row_num_keys, uint32_t *__restrict__ errors) {
    const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= num_rows) return;
    // Largest s with seq_row_starts[s] <= row; empty sequences (equal
    // consecutive starts) are skipped because the search keeps the last one.
    uint32_t lo = 0, hi = num_seqs;  // invariant: starts[lo] <= row < starts[hi]
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) / 2;
        if (seq_row_starts[mid] <= row)
            lo = mid;
        else
            hi = mid;
    }
    const uint32_t s = lo;
    const uint32_t pos = context_lens[s] + (row - seq_row_starts[s]);
    const uint32_t idx = pos / block_size;
    const uint32_t len = table_off[s + 1] - table_off[s];
    uint32_t slot = 0xffffffffu;
    if (idx < len)
        slot = tables[table_off[s] + idx] * block_size + pos % block_size;
    else
        *errors = 1u;
    positions[row] = pos;
    slot_mapping[row] = slot;
    row_seq[row] = s;
    row_num_keys[row] = pos + 1;
}

}  // namespace

hipError_t launch_build_rows(const uint32_t *seq_row_starts, const uint32_t *context_lens,
                             const uint32_t *table_off, const uint32_t *tables, uint32_t num_seqs,
                             uint32_t num_rows, uint32_t block_size, uint32_t *positions,
                             uint32_t *slot_mapping, uint32_t *row_seq, uint32_t *row_num_keys,
                             uint32_t *errors, hipStream_t stream) {
    if (num_rows == 0) return hipSuccess;
    if (num_seqs == 0 || block_size == 0) return hipErrorInvalidValue;
    const uint32_t grid = (num_rows + 255) / 256;
    KernelTimer timer("build_rows", stream);
    hipLaunchKernelGGL(build_rows_kernel, dim3(grid), dim3(256), 0, stream, seq_row_starts,
                       context_lens, table_off, tables, num_seqs, num_rows, block_size, positions,
                       slot_mapping, row_seq, row_num_keys, errors);
    return hipGetLastError();
}

}  // namespace kernels
}  // namespace vo

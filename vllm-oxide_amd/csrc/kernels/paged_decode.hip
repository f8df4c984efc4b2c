// paged_decode.hip -- split-K paged decode attention on gfx950 MFMA, and the
// reduce kernel that merges the split-K partials.
//
// Math: crates/engine/src/backend/cpu/attention.rs:5-16 (one query row per
// sequence at decode, cpu/mod.rs:314-339).  For query row t, KV head k and
// the G = heads/kv_heads query heads h of k's group:
//   s[j,h] = (K[slot(j),k] . Q[t,kG+h]) * scale          j < row_num_keys[t]
//   out[t,kG+h] = sum_j softmax_j(s[.,h]) V[slot(j),k]
// computed as an online softmax in the exp2 domain (scores pre-multiplied by
// scale*log2 e), fp32 accumulation, bf16 I/O.
//
// Work split.  The keys of each row are cut into splits of `split_keys`
// (a multiple of 32, at most kMaxSplitKeys).  Workgroup (item, k) owns one
// (row, split) for one KV head and all G heads of its group, so every K/V
// byte is read from HBM once: the algorithmic minimum.  An item is one
// 16-byte record (row, split, where the split's block ids start, keys), so
// the workgroup starts its loads after one dependent read.  Its W wavefronts
// take the split's 32-key chunks round robin; block ids are wave-uniform and
// come from scalar loads.  Each wavefront issues all 16 loads of its next
// chunk before it waits for the current one (two register buffers), so two
// chunks are in flight per wavefront.  The wavefronts merge through LDS at
// the end.  A row with one
// split writes its bf16 output directly; otherwise the workgroup writes an
// fp32 partial (m, l, acc[head_dim]) per head, and decode_reduce_kernel
// merges them:
//   M = max_i m_i,  out = sum_i 2^(m_i-M) acc_i / sum_i 2^(m_i-M) l_i.
// (Merging in the last workgroup to finish a row instead needs an
// agent-scope release/acquire per workgroup; on gfx950 that is an L2
// writeback and invalidate each time, which measured 5-9x slower than the
// separate launch.)
// Workgroups are numbered KV head fastest, so the KV heads of one block are
// read at about the same time.
//
// Row packing.  One row's group fills G of the MFMA tile's 16 head columns.
// When the plan finds full splits of several rows over the same physical
// blocks (aliased block-table entries: a shared prefix), one work item
// serves several of them (`pack`; the others are listed in `mates`), and the
// blocks are read once per pack instead of once per row.  Either up to 16 / G
// rows share the tile (column c takes head c % G of row slot c / G), or, in a
// shared pack (shared_split), the workgroup stages each chunk in LDS once and
// each of its 4 wavefronts takes 16 / G rows in its own tile.  MFMA output
// columns and the per-column softmax never mix, and a shared pack keeps the
// register path's per-wavefront states and merge, so every row's result is
// bitwise the one it gets unpacked.
//
// One 32-key chunk (two 16-key blocks b0, b1) of one wavefront:
//   Q.K^T: S^T[key, h] = K[key, :] . Q[h, :] with v_mfma_f32_16x16x32_bf16,
//          A = 16 keys x 32 dims of K (one 16-byte load per lane from the
//          key-major tile), B = Q^T with the G heads in columns 0..G-1 and
//          zeros elsewhere; head_dim/32 MFMAs per 16 keys, two key sets.
//          The A-row -> key assignment is chosen so that lane l ends up
//          holding the scores of head l%16 for keys 8*(l/16) .. +7 of the
//          chunk, in order.
//   softmax: per head, max over the lane's 8 keys and over the 4 lane groups
//          (two xor-shuffles); exp2; the running sum stays per lane and is
//          reduced once at the end.
//   P.V:   O^T[d, h] += V^T[d, key] . P^T[key, h] with 16x16x32 MFMAs:
//          A = 16 dims x 32 keys of V -- lane l reads the 8 keys 8*(l/16)..+7
//          of dim l%16, which are 16 contiguous bytes of the dim-major V tile
//          -- and B = P^T, which is exactly the lane's own 8 probabilities,
//          split into bf16 hi and lo parts (two MFMAs) so P keeps ~16 bits.
//          Output rows are dims, columns heads, so the softmax rescale of the
//          accumulator is lane-local.
// Per chunk and KV head a wavefront moves 16 KiB (hd 128) through 16 global
// loads of 16 bytes per lane and issues 24 MFMAs.
//
// Roofline: HBM.  Algorithmic bytes per row = keys * kv_heads * head_dim * 2 B
// * 2 (K and V) + q and out rows + block-table entries.  The MFMA work is
// <10% of gfx950's bf16 rate even with 12 of 16 head columns padding.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "vo_device.hpp"
#include "vo_kernels.hpp"

namespace vo {
namespace kernels {

namespace {

constexpr int kBS = 16;     // block size of the MFMA path
constexpr int kChunk = 32;  // keys per wavefront iteration

__device__ __forceinline__ floatx4 mfma16x16x32(bf16x8 a, bf16x8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t *p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}

// K/V tile load.  NT = non-temporal (streaming) loads: on MI355X they raise
// random 4 KiB-tile read bandwidth from ~5.7 to ~6.4 TB/s; used when no KV
// block is read by more than one row of the step, so nothing is lost by not
// keeping the lines in L2.
template <bool NT>
__device__ __forceinline__ bf16x8 load_kv(const uint16_t *p) {
    const u32x4 *v = reinterpret_cast<const u32x4 *>(p);
    if constexpr (NT)
        return __builtin_bit_cast(bf16x8, __builtin_nontemporal_load(v));
    else
        return __builtin_bit_cast(bf16x8, *v);
}

// One chunk's K and V operands, in registers.
template <int HD>
struct Chunk {
    bf16x8 ka[HD / 32];  // first key set (keys 8g + 0..3 land in its result)
    bf16x8 kb[HD / 32];  // second key set (keys 8g + 4..7)
    bf16x8 va[HD / 16];  // V^T rows: dims 16*dt + l%16, keys 8g .. 8g+7
};

// Per-lane element offsets inside one (block, kv head) tile.  K tiles are
// [head_dim/32][16 keys][32 dims] (vo_device.hpp).
struct LaneMap {
    uint32_t k_off;  // Q.K^T A-row m = l%16: key 8*((m>>2)&1) + (m&3), dims 8*(l/16)..
    uint32_t v_off;  // P.V A-row d = l%16: keys 8*(g&1) .. +7 of block g>>1
    bool k_hi;       // A-row m reads block b1 (m >= 8)
    bool v_hi;       // lane group g reads block b1 (g >= 2)
};

template <int HD, bool NT>
__device__ __forceinline__ void load_chunk(Chunk<HD> &r, const uint16_t *k_head,
                                           const uint16_t *v_head, uint64_t block_stride,
                                           uint32_t phys0, uint32_t phys1, const LaneMap &lm) {
    const uint16_t *kp =
        k_head + static_cast<uint64_t>(lm.k_hi ? phys1 : phys0) * block_stride + lm.k_off;
#pragma unroll
    for (int kk = 0; kk < HD / 32; ++kk) {
        r.ka[kk] = load_kv<NT>(kp + kk * (kBS * 32));
        r.kb[kk] = load_kv<NT>(kp + 4 * 32 + kk * (kBS * 32));
    }
    const uint16_t *vp =
        v_head + static_cast<uint64_t>(lm.v_hi ? phys1 : phys0) * block_stride + lm.v_off;
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) r.va[dt] = load_kv<NT>(vp + dt * 16 * kBS);
}

// The step's new key is chunk key kc of r: take its K and V from the new
// rows (nk_row, nv_row: this KV head's head_dim values) instead of the pool,
// which this launch writes them to.  Lane l's K rows are chunk keys
// 16*(m>=8) + 8*((m>>2)&1) + (m&3) (ka) and that + 4 (kb), m = l%16, dims
// 8*(l/16) + 32*kk; its V registers hold keys 8*(l/16) .. +7 of dims
// 16*dt + m (the LaneMap above).
template <int HD>
__device__ __forceinline__ void take_new_key(Chunk<HD> &r, uint32_t kc, const uint16_t *nk_row,
                                             const uint16_t *nv_row, int lane) {
    const uint32_t m = lane & 15;
    const uint32_t g = lane >> 4;
    const uint32_t ka_key = 16 * (m >= 8) + 8 * ((m >> 2) & 1) + (m & 3);
    if (ka_key == kc) {
#pragma unroll
        for (int kk = 0; kk < HD / 32; ++kk)
            r.ka[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(nk_row + 32 * kk + 8 * g));
    }
    if (ka_key + 4 == kc) {
#pragma unroll
        for (int kk = 0; kk < HD / 32; ++kk)
            r.kb[kk] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(nk_row + 32 * kk + 8 * g));
    }
    if ((kc >> 3) == g) {
        const uint32_t i = kc & 7;
#pragma unroll
        for (int dt = 0; dt < HD / 16; ++dt) {
            u32x4 w = __builtin_bit_cast(u32x4, r.va[dt]);
            const uint32_t val = nv_row[16 * dt + m];
            const uint32_t sh = 16 * (i & 1);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (q == static_cast<int>(i >> 1)) w[q] = (w[q] & ~(0xffffu << sh)) | (val << sh);
            r.va[dt] = __builtin_bit_cast(bf16x8, w);
        }
    }
}

// One chunk of the online softmax, in two parts: the scores (chunk_qk), then
// the softmax update and P.V (chunk_update).  `nv` = valid keys of this
// lane's group (0..8); the last chunk of a split passes tail = true, with V
// already masked.  Every product and sum is rounded on its own (no fused
// multiply-adds), so that a chunk gets the same bits in every inlined copy:
// the fusion the compiler chooses otherwise depends on the surrounding code
// (whether a product has other uses, as in a tail chunk's masking).
template <int HD>
__device__ __forceinline__ void chunk_qk(const bf16x8 (&ka)[HD / 32], const bf16x8 (&kb)[HD / 32],
                                         const bf16x8 (&qv)[HD / 32], floatx4 &s0, floatx4 &s1) {
    s0 = floatx4{0.f, 0.f, 0.f, 0.f};
    s1 = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < HD / 32; ++kk) {
        s0 = mfma16x16x32(ka[kk], qv[kk], s0);
        s1 = mfma16x16x32(kb[kk], qv[kk], s1);
    }
}

// Keys past the end get p = 0; zero their V too, so whatever the pool holds
// there cannot turn 0*x into NaN.
template <int HD>
__device__ __forceinline__ void mask_tail_v(bf16x8 (&va)[HD / 16], int nv) {
    u32x4 mask;
#pragma unroll
    for (int p = 0; p < 4; ++p)
        mask[p] = ((2 * p < nv) ? 0x0000ffffu : 0u) | ((2 * p + 1 < nv) ? 0xffff0000u : 0u);
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt)
        va[dt] = __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, va[dt]) & mask);
}

template <int HD>
__device__ __forceinline__ void chunk_update(const floatx4 &s0, const floatx4 &s1,
                                             const bf16x8 (&va)[HD / 16], bool tail, int nv,
                                             float scale_log2, float &m_run, float &l_run,
                                             floatx4 (&acc)[HD / 16]) {
#pragma clang fp contract(off)
    float sc[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sc[i] = s0[i] * scale_log2;
        sc[4 + i] = s1[i] * scale_log2;
    }
    if (tail) {
#pragma unroll
        for (int i = 0; i < 8; ++i) sc[i] = (i < nv) ? sc[i] : -INFINITY;
    }
    float mt = sc[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mt = fmaxf(mt, sc[i]);
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt);  // finite: every chunk has a valid key
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    // P goes to the MFMA as two bf16 parts, hi = bf16(p) and lo = bf16(p - hi),
    // so the probabilities keep ~16 significant bits instead of bf16's 8;
    // bf16 P alone exceeds rtol 1e-2 / atol 2e-3 on rows whose weight sits on
    // a few keys.
    float ps = 0.0f;
    bf16x8 pb_hi, pb_lo;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float p = __builtin_amdgcn_exp2f(sc[i] - m_new);
        ps += p;
        const __bf16 hi = static_cast<__bf16>(p);
        pb_hi[i] = hi;
        pb_lo[i] = static_cast<__bf16>(p - static_cast<float>(hi));
    }
    l_run = l_run * alpha + ps;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < HD / 16; ++dt) {
        acc[dt] *= alpha;
        acc[dt] = mfma16x16x32(va[dt], pb_lo, acc[dt]);
        acc[dt] = mfma16x16x32(va[dt], pb_hi, acc[dt]);
    }
}

template <int HD>
__device__ __forceinline__ void compute_chunk(Chunk<HD> &r, const bf16x8 (&qv)[HD / 32], bool tail,
                                              int nv, float scale_log2, float &m_run, float &l_run,
                                              floatx4 (&acc)[HD / 16]) {
    floatx4 s0, s1;
    chunk_qk<HD>(r.ka, r.kb, qv, s0, s1);
    if (tail) mask_tail_v<HD>(r.va, nv);
    chunk_update<HD>(s0, s1, r.va, tail, nv, scale_log2, m_run, l_run, acc);
}

// Keeps the scheduler from moving instructions across this point: the next
// chunk's loads are all issued before the current chunk's first wait.
__device__ __forceinline__ void issue_fence() { __builtin_amdgcn_sched_barrier(0); }

// A shared pack: one full split whose blocks the rows of a pack all read
// (an aliased prefix), for up to W * (16 / G) rows.  Each wavefront owns one
// 16-column tile (rows w * 16/G ..) and walks every chunk of the split, so
// the workgroup reads each K/V byte once for all of its rows instead of once
// per wavefront.  A chunk (two blocks: K b0, K b1, V b0, V b1, one tile
// each) is copied into LDS by LDS DMA, 16 bytes per lane from the lane's own
// global address, through a ring of four stages; the workgroup takes one
// chunk per barrier while the next three load.  The wavefronts then read their operands from LDS at
// the positions the register path loads from the pool and run its
// compute_chunk; chunk c updates state c % W, the state the register path's
// wavefront c % W keeps, and the W states are merged as that path merges its
// wavefronts, so every column's result is the register path's, bit for bit.
//
// LDS bank spread: within a tile, 16-byte unit x sits at unit swz(x).  K
// unit x = 64 kk + 4 key + j (dims 8 j.. of 32-dim chunk kk): j ^= 2 (key >>
// 3) ^ (block & 1), so the 16 lanes of one read phase (keys 0-3 and 8-11 of
// two blocks) fill 16 distinct 4-bank groups.  V unit x = 2 dim + half:
// half ^= (dim >> 3) & 1.  Both are involutions on the low bits, so the DMA
// reads global unit swz(u) into LDS unit u.
// Floats per column of the wavefronts' merge buffer: 4 more than head_dim, so
// that the 16 columns of one store phase fall into 16 different bank groups.
template <int HD>
constexpr uint32_t kAccStride = HD + 4;

// A shared pack keeps W softmax states per wavefront (W x 32 registers at
// head_dim 128), and its four stages also hold the register path's merge:
// exactly 4 wavefronts (with 2 the four-stage loop no longer fits two
// wavefronts per SIMD).
constexpr int kSharedWaves = 4;

template <int HD>
struct SharedStage {
    static constexpr uint32_t TB = kBS * HD * 2;   // bytes of one (block, KV head) tile
    static constexpr uint32_t BYTES = 4 * TB;      // K b0, K b1, V b0, V b1
    __device__ static __forceinline__ uint32_t swz_k(uint32_t x, uint32_t b) {
        return x ^ (((x >> 5) & 1u) << 1) ^ (b & 1u);
    }
    __device__ static __forceinline__ uint32_t swz_v(uint32_t x) { return x ^ ((x >> 4) & 1u); }
};

template <int HD, int W>
__device__ __forceinline__ void shared_split(
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool, uint32_t kv_heads,
    uint32_t kvh, uint32_t item, const u32x4 rec, const uint32_t *__restrict__ tables,
    const uint32_t *__restrict__ row_info, uint32_t split_keys, const uint16_t *__restrict__ q,
    uint16_t *__restrict__ out, float *__restrict__ part_acc, float *__restrict__ part_ml,
    uint32_t num_heads, uint32_t group, float scale_log2, const uint32_t *__restrict__ mates,
    uint32_t pack, uint8_t *__restrict__ st0, uint8_t *__restrict__ st1,
    uint8_t *__restrict__ st2, uint8_t *__restrict__ st3) {
#pragma clang fp contract(off)  // the merge below rounds as the register path's does
    constexpr int KK = HD / 32;
    constexpr int DT = HD / 16;
    using S = SharedStage<HD>;
    constexpr uint32_t kTile = kBS * HD;
    constexpr int NI = S::BYTES / 1024 / W;  // DMA instructions per wavefront and chunk
    static_assert(S::BYTES % (1024 * W) == 0 && NI <= 15, "chunk DMA split");
    constexpr uint32_t KIB_PER_TILE = S::TB / 1024;

    const uint32_t row = uniform_u32(rec[0]);
    const uint32_t split = uniform_u32(rec[1]);
    const uint32_t *table = tables + uniform_u32(rec[2]);
    const uint32_t nchunks = split_keys / kChunk;  // a full split
    // The split's block ids (at most kMaxSplitKeys / 16 = 256), 64 per
    // register across the lanes, read before the first DMA; a chunk's two ids
    // are then v_readlane'd.  (Loads from the table after an LDS DMA would be
    // vector loads, and every wait for one would also wait for the DMA.)
    constexpr int TV = kMaxSplitKeys / kBS / 64;
    const uint32_t nblk = 2 * nchunks;
    uint32_t tv[TV];
#pragma unroll
    for (int k = 0; k < TV; ++k) {
        const uint32_t i = 64 * k + static_cast<uint32_t>(threadIdx.x & 63);
        tv[k] = i < nblk ? table[i] : 0u;
    }
    auto block_id = [&](uint32_t i) {  // i < nblk, wave-uniform
        uint32_t b = __builtin_amdgcn_readlane(tv[0], i & 63);
#pragma unroll
        for (int k = 1; k < TV; ++k) {
            const uint32_t bk = __builtin_amdgcn_readlane(tv[k], i & 63);
            b = (i >> 6) == static_cast<uint32_t>(k) ? bk : b;
        }
        return b;
    };
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane & 15;
    const int g = lane >> 4;

    // This wavefront's columns: row slot wave * R + h / G, head h % G, with
    // R = ceil(pack / W) <= 16 / G rows per wavefront.
    const uint32_t per_wave = (pack + W - 1) / W;
    const uint32_t hslot = static_cast<uint32_t>(h) / group;
    const uint32_t pslot = static_cast<uint32_t>(wave) * per_wave + hslot;
    const uint32_t hh = static_cast<uint32_t>(h) - hslot * group;
    uint32_t crow = kNoMate;
    if (hslot < per_wave) {
        if (pslot == 0)
            crow = row;
        else if (pslot < pack)
            crow = mates[(pack - 1) * item + pslot - 1];
    }
    const bool head_ok = crow != kNoMate;
    // Whether any column of this wavefront is live (wave-uniform).
    const bool wave_live = __builtin_amdgcn_ballot_w64(head_ok) != 0;
    const uint32_t qhead = kvh * group + hh;
    bf16x8 qv[KK];
    {
        const uint16_t *qp = q + (static_cast<uint64_t>(head_ok ? crow : row) * num_heads + qhead) * HD + 8 * g;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qv[kk] = head_ok ? load_bf16x8(qp + 32 * kk) : bf16x8{};
    }
    u32x2 cinfo = {0u, 0u};
    if (head_ok) cinfo = *reinterpret_cast<const u32x2 *>(row_info + 2 * static_cast<uint64_t>(crow));

    // DMA: instruction i of wavefront w copies KiB qi = i * W + w of the
    // stage: tile qi / KIB_PER_TILE (K b0, K b1, V b0, V b1), its KiB qi %
    // KIB_PER_TILE; lane unit u of that tile reads global unit swz(u).
    uint32_t dma_off[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const uint32_t qi = static_cast<uint32_t>(i * W + wave);
        const uint32_t t = qi / KIB_PER_TILE;
        const uint32_t u = (qi % KIB_PER_TILE) * 64 + lane;
        dma_off[i] = 16 * (t < 2 ? S::swz_k(u, t) : S::swz_v(u));
    }
    const uint64_t block_stride = static_cast<uint64_t>(kv_heads) * kTile;
    auto dma_chunk = [&](uint8_t *stage, uint32_t c) {
        const uint32_t b0 = block_id(2 * c);
        const uint32_t b1 = block_id(2 * c + 1);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t qi = static_cast<uint32_t>(i * W + wave);
            const uint32_t t = qi / KIB_PER_TILE;
            const uint16_t *pool = t < 2 ? k_pool : v_pool;
            const uint32_t blk = (t & 1) ? b1 : b0;
            dma16(pool + static_cast<uint64_t>(blk) * block_stride + static_cast<uint64_t>(kvh) * kTile,
                  S::TB, stage + qi * 1024, dma_off[i]);
        }
    };

    // LDS read offsets of this lane (the register path's LaneMap positions,
    // swizzled): K A-row m = l % 16 reads key 8((m >> 2) & 1) + (m & 3) of
    // block m >= 8, dims 8 g .. of chunk kk (+64 kk units) and the key + 4
    // (+16 units); V lane reads dim 16 dt + m (+32 dt units), keys 8 (g & 1)
    // .. +7 of block g >= 2.
    const uint32_t m = static_cast<uint32_t>(h);
    const uint32_t kb_hi = m >= 8 ? 1u : 0u;
    const uint32_t kx = (8 * ((m >> 2) & 1) + (m & 3)) * 4 + static_cast<uint32_t>(g);
    const uint32_t k_rd = kb_hi * S::TB + 16 * S::swz_k(kx, kb_hi);
    const uint32_t vb_hi = g >= 2 ? 1u : 0u;
    const uint32_t vx = 2 * m + static_cast<uint32_t>(g & 1);
    const uint32_t v_rd = (2 + vb_hi) * S::TB + 16 * S::swz_v(vx);

    // Chunk c goes to state c % W: the (m, l, acc) the register path's
    // wavefront c % W keeps, in the same order, merged at the end as that
    // path merges its wavefronts.  So a row's bits do not depend on whether
    // it was packed.
    float ms[W], ls[W];
    floatx4 as[W][DT];
#pragma unroll
    for (int w = 0; w < W; ++w) {
        ms[w] = -INFINITY;
        ls[w] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) as[w][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

    // Chunk c (stage c % 4) updates state c % 4.
    auto read_k = [&](const uint8_t *cur, bf16x8 (&ka)[KK], bf16x8 (&kb)[KK])
        __attribute__((always_inline)) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            ka[kk] = *reinterpret_cast<const bf16x8 *>(cur + k_rd + 1024 * kk);
            kb[kk] = *reinterpret_cast<const bf16x8 *>(cur + k_rd + 1024 * kk + 256);
        }
    };
    auto read_v = [&](const uint8_t *cur, bf16x8 (&va)[DT]) __attribute__((always_inline)) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) va[dt] = *reinterpret_cast<const bf16x8 *>(cur + v_rd + 512 * dt);
    };
    // One chunk per step: step c waits for chunk c (the DMA of chunks c + 1
    // and c + 2 may fly on) and for every wavefront to be done with chunk
    // c - 1, refills that stage with chunk c + 3 and computes chunk c into
    // state c % 4.  Every step issues its DMA (past the last chunk the block
    // ids repeat the split's last blocks), so the wait count stays uniform.
    auto one = [&](auto s_c, uint32_t c) __attribute__((always_inline)) {
        constexpr int sidx = decltype(s_c)::value;
        uint8_t *__restrict__ cur = sidx == 0 ? st0 : sidx == 1 ? st1 : sidx == 2 ? st2 : st3;
        uint8_t *__restrict__ nxt = sidx == 0 ? st3 : sidx == 1 ? st0 : sidx == 2 ? st1 : st2;
        wait_barrier<2 * NI>();
        dma_chunk(nxt, min(c + 3, nchunks - 1));
        if (!wave_live) return;
        bf16x8 ka[KK], kb[KK], va[DT];
        floatx4 sa0, sa1;
        read_k(cur, ka, kb);
        chunk_qk<HD>(ka, kb, qv, sa0, sa1);
        read_v(cur, va);
        chunk_update<HD>(sa0, sa1, va, false, 8, scale_log2, ms[sidx], ls[sidx], as[sidx]);
    };
    static_assert(W == 4, "state index = stage index");
    dma_chunk(st0, 0);
    dma_chunk(st1, min(1u, nchunks - 1));
    dma_chunk(st2, min(2u, nchunks - 1));
    for (uint32_t c = 0; c < nchunks; c += 4) {
        one(std::integral_constant<int, 0>{}, c);
        if (c + 1 >= nchunks) break;
        one(std::integral_constant<int, 1>{}, c + 1);
        if (c + 2 >= nchunks) break;
        one(std::integral_constant<int, 2>{}, c + 2);
        if (c + 3 >= nchunks) break;
        one(std::integral_constant<int, 3>{}, c + 3);
    }
    // The DMA past the last chunk must land before the workgroup's LDS is
    // released.
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));

    if (!head_ok) return;
    // The register path's merge of its W wavefronts, per element.
#pragma unroll
    for (int w = 0; w < W; ++w) {
        ls[w] += __shfl_xor(ls[w], 16, 64);
        ls[w] += __shfl_xor(ls[w], 32, 64);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) mx = fmaxf(mx, ms[w]);
    float den = 0.0f;
    floatx4 num[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) num[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < W; ++w) {
        const float mw = ms[w];
        if (mw != -INFINITY) {
            const float e = __builtin_amdgcn_exp2f(mw - mx);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int j = 0; j < 4; ++j) num[dt][j] += e * as[w][dt][j];
            den += e * ls[w];
        }
    }
    if (cinfo[1] == 1) {
        uint16_t *op = out + static_cast<uint64_t>(crow) * num_heads * HD +
                       static_cast<uint64_t>(qhead) * HD + 4 * g;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) op[16 * dt + j] = f32_to_bf16_bits(num[dt][j] / den);
    } else {
        const uint64_t part = static_cast<uint64_t>(cinfo[0] + split) * num_heads + qhead;
        float *ap = part_acc + part * HD + 4 * g;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<floatx4 *>(ap + 16 * dt) = num[dt];
        if (g == 0) {
            part_ml[2 * part] = mx;
            part_ml[2 * part + 1] = den;
        }
    }
}

// A shared pack in wavefront pairs.  The same staged chunks and the same
// four softmax states as shared_split, but each 16-column tile has two
// wavefronts: the one of parity 0 keeps states 0 and 2 (chunks 4k and
// 4k + 2), the one of parity 1 states 1 and 3 (chunks 4k + 1, 4k + 3).  One
// step stages two chunks (2j in stage 2(j % 2), 2j + 1 in the next) and each
// wavefront of a pair computes one of them, so a wavefront walks half of the
// split's chunks.  The workgroup holds W / 2 tiles, so a pack has W / 2 *
// (16 / G) rows.  Every state still takes its chunks in increasing order,
// and the four states are merged in the order 0..3 with the register path's
// arithmetic, so a row's bits are the register path's, as in shared_split.
// Two chunks are consumed per step, so the DMA of a step's pair is issued
// one step ahead (the four stages hold two pairs).
template <int HD, int W>
__device__ __forceinline__ void shared_split_pairs(
    const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool, uint32_t kv_heads,
    uint32_t kvh, uint32_t item, const u32x4 rec, const uint32_t *__restrict__ tables,
    const uint32_t *__restrict__ row_info, uint32_t split_keys, const uint16_t *__restrict__ q,
    uint16_t *__restrict__ out, float *__restrict__ part_acc, float *__restrict__ part_ml,
    uint32_t num_heads, uint32_t group, float scale_log2, const uint32_t *__restrict__ mates,
    uint32_t pack, uint8_t *__restrict__ st0, uint8_t *__restrict__ st1,
    uint8_t *__restrict__ st2, uint8_t *__restrict__ st3) {
#pragma clang fp contract(off)  // the merge below rounds as the register path's does
    constexpr int KK = HD / 32;
    constexpr int DT = HD / 16;
    using S = SharedStage<HD>;
    constexpr uint32_t kTile = kBS * HD;
    constexpr int NI = S::BYTES / 1024 / W;  // DMA instructions per wavefront and chunk
    static_assert(W == 4 && S::BYTES % (1024 * W) == 0 && 2 * NI <= 15, "chunk DMA split");
    constexpr uint32_t KIB_PER_TILE = S::TB / 1024;
    constexpr uint32_t kTiles = W / 2;
    // The partner's two states go through the stages: per tile, DT x 64
    // lanes of floatx4 per state (one stage), and (m, l) per state and lane.
    static_assert(2 * DT * 64 * 16 <= S::BYTES && kTiles * 4 * 64 * 4 <= S::BYTES,
                  "pair exchange fits the stages");
    // The packs set the launch's length and share each CU with a
    // register-path workgroup that has slack: their wavefronts win the
    // SIMDs' issue arbitration.
    __builtin_amdgcn_s_setprio(3);

    const uint32_t row = uniform_u32(rec[0]);
    const uint32_t split = uniform_u32(rec[1]);
    const uint32_t *table = tables + uniform_u32(rec[2]);
    const uint32_t nchunks = split_keys / kChunk;  // a full split
    constexpr int TV = kMaxSplitKeys / kBS / 64;
    const uint32_t nblk = 2 * nchunks;
    uint32_t tv[TV];
#pragma unroll
    for (int k = 0; k < TV; ++k) {
        const uint32_t i = 64 * k + static_cast<uint32_t>(threadIdx.x & 63);
        tv[k] = i < nblk ? table[i] : 0u;
    }
    auto block_id = [&](uint32_t i) {  // i < nblk, wave-uniform
        uint32_t b = __builtin_amdgcn_readlane(tv[0], i & 63);
#pragma unroll
        for (int k = 1; k < TV; ++k) {
            const uint32_t bk = __builtin_amdgcn_readlane(tv[k], i & 63);
            b = (i >> 6) == static_cast<uint32_t>(k) ? bk : b;
        }
        return b;
    };
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane & 15;
    const int g = lane >> 4;
    const uint32_t tile = static_cast<uint32_t>(wave) >> 1;
    const uint32_t par = static_cast<uint32_t>(wave) & 1;

    // This tile's columns: row slot tile * R + h / G, head h % G, with
    // R = ceil(pack / tiles) <= 16 / G rows per tile.
    const uint32_t per_tile = (pack + kTiles - 1) / kTiles;
    const uint32_t hslot = static_cast<uint32_t>(h) / group;
    const uint32_t pslot = tile * per_tile + hslot;
    const uint32_t hh = static_cast<uint32_t>(h) - hslot * group;
    uint32_t crow = kNoMate;
    if (hslot < per_tile) {
        if (pslot == 0)
            crow = row;
        else if (pslot < pack)
            crow = mates[(pack - 1) * item + pslot - 1];
    }
    const bool head_ok = crow != kNoMate;
    const bool wave_live = __builtin_amdgcn_ballot_w64(head_ok) != 0;
    const uint32_t qhead = kvh * group + hh;
    bf16x8 qv[KK];
    {
        const uint16_t *qp = q + (static_cast<uint64_t>(head_ok ? crow : row) * num_heads + qhead) * HD + 8 * g;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qv[kk] = head_ok ? load_bf16x8(qp + 32 * kk) : bf16x8{};
    }
    u32x2 cinfo = {0u, 0u};
    if (head_ok) cinfo = *reinterpret_cast<const u32x2 *>(row_info + 2 * static_cast<uint64_t>(crow));

    // DMA as in shared_split: instruction i of wavefront w copies KiB i * W
    // + w of a chunk's stage.
    uint32_t dma_off[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const uint32_t qi = static_cast<uint32_t>(i * W + wave);
        const uint32_t t = qi / KIB_PER_TILE;
        const uint32_t u = (qi % KIB_PER_TILE) * 64 + lane;
        dma_off[i] = 16 * (t < 2 ? S::swz_k(u, t) : S::swz_v(u));
    }
    const uint64_t block_stride = static_cast<uint64_t>(kv_heads) * kTile;
    auto dma_chunk = [&](uint8_t *stage, uint32_t c) {
        const uint32_t b0 = block_id(2 * c);
        const uint32_t b1 = block_id(2 * c + 1);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t qi = static_cast<uint32_t>(i * W + wave);
            const uint32_t t = qi / KIB_PER_TILE;
            const uint16_t *pool = t < 2 ? k_pool : v_pool;
            const uint32_t blk = (t & 1) ? b1 : b0;
            dma16(pool + static_cast<uint64_t>(blk) * block_stride + static_cast<uint64_t>(kvh) * kTile,
                  S::TB, stage + qi * 1024, dma_off[i]);
        }
    };

    // LDS read offsets: shared_split's.
    const uint32_t m = static_cast<uint32_t>(h);
    const uint32_t kb_hi = m >= 8 ? 1u : 0u;
    const uint32_t kx = (8 * ((m >> 2) & 1) + (m & 3)) * 4 + static_cast<uint32_t>(g);
    const uint32_t k_rd = kb_hi * S::TB + 16 * S::swz_k(kx, kb_hi);
    const uint32_t vb_hi = g >= 2 ? 1u : 0u;
    const uint32_t vx = 2 * m + static_cast<uint32_t>(g & 1);
    const uint32_t v_rd = (2 + vb_hi) * S::TB + 16 * S::swz_v(vx);

    // Local state i is state par + 2 i.
    float ms[2], ls[2];
    floatx4 as[2][DT];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        ms[i] = -INFINITY;
        ls[i] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) as[i][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    auto compute = [&](const uint8_t *cur, int i) __attribute__((always_inline)) {
        bf16x8 ka[KK], kb[KK], va[DT];
        floatx4 sa0, sa1;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            ka[kk] = *reinterpret_cast<const bf16x8 *>(cur + k_rd + 1024 * kk);
            kb[kk] = *reinterpret_cast<const bf16x8 *>(cur + k_rd + 1024 * kk + 256);
        }
        chunk_qk<HD>(ka, kb, qv, sa0, sa1);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) va[dt] = *reinterpret_cast<const bf16x8 *>(cur + v_rd + 512 * dt);
        chunk_update<HD>(sa0, sa1, va, false, 8, scale_log2, ms[i], ls[i], as[i]);
    };
    // Step j: wait for chunks 2j and 2j + 1 (the only DMA in flight), then
    // for every wavefront to be done with step j - 1's pair, refill that
    // pair with chunks 2j + 2 and 2j + 3, and compute chunk 2j + par into
    // local state j % 2 (state (2j + par) % 4).  Each stage is named in its
    // own branch, so that the compiler tells the stage being read from the
    // ones the DMA fills.  Every step issues its DMA (past the last chunk
    // the block ids repeat the split's last blocks).
    auto step = [&](auto s_pair, uint32_t j) __attribute__((always_inline)) {
        constexpr int sp = decltype(s_pair)::value;
        wait_barrier<0>();
        dma_chunk(sp ? st0 : st2, min(2 * j + 2, nchunks - 1));
        dma_chunk(sp ? st1 : st3, min(2 * j + 3, nchunks - 1));
        if (!wave_live || 2 * j + par >= nchunks) return;
        if (par == 0)
            compute(sp ? st2 : st0, sp);
        else
            compute(sp ? st3 : st1, sp);
    };
    const uint32_t nsteps = (nchunks + 1) / 2;
    dma_chunk(st0, 0);
    dma_chunk(st1, min(1u, nchunks - 1));
    for (uint32_t j = 0; j < nsteps; j += 2) {
        step(std::integral_constant<int, 0>{}, j);
        if (j + 1 >= nsteps) break;
        step(std::integral_constant<int, 1>{}, j + 1);
    }
    // The DMA past the last chunk must land before the stages are reused.
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
    // The running sums are per lane group (the four lanes of a column are
    // all live or all not).
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        ls[i] += __shfl_xor(ls[i], 16, 64);
        ls[i] += __shfl_xor(ls[i], 32, 64);
    }
    // The parity-1 wavefront hands its states to its partner through the
    // stages, once every wavefront is done reading them.
    __syncthreads();
    floatx4 *xa = reinterpret_cast<floatx4 *>(tile == 0 ? st0 : st1);  // [2][DT][64]
    float *xml = reinterpret_cast<float *>(st2) + tile * 4 * 64;     // [2][m, l][64]
    if (par == 1 && head_ok) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) xa[(i * DT + dt) * 64 + lane] = as[i][dt];
            xml[(2 * i) * 64 + lane] = ms[i];
            xml[(2 * i + 1) * 64 + lane] = ls[i];
        }
    }
    __syncthreads();
    if (par == 1 || !head_ok) return;

    // The register path's merge of its W = 4 wavefronts' states, in order
    // 0..3: state 2i is this wavefront's local state i, state 2i + 1 the
    // partner's.
    float sm[4], sl[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        sm[2 * i] = ms[i];
        sl[2 * i] = ls[i];
        sm[2 * i + 1] = xml[(2 * i) * 64 + lane];
        sl[2 * i + 1] = xml[(2 * i + 1) * 64 + lane];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, sm[w]);
    float den = 0.0f;
    floatx4 num[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) num[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float mw = sm[w];
        if (mw != -INFINITY) {
            const float e = __builtin_amdgcn_exp2f(mw - mx);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const floatx4 a = (w & 1) ? xa[((w >> 1) * DT + dt) * 64 + lane] : as[w >> 1][dt];
#pragma unroll
                for (int j = 0; j < 4; ++j) num[dt][j] += e * a[j];
            }
            den += e * sl[w];
        }
    }
    if (cinfo[1] == 1) {
        uint16_t *op = out + static_cast<uint64_t>(crow) * num_heads * HD +
                       static_cast<uint64_t>(qhead) * HD + 4 * g;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) op[16 * dt + j] = f32_to_bf16_bits(num[dt][j] / den);
    } else {
        const uint64_t part = static_cast<uint64_t>(cinfo[0] + split) * num_heads + qhead;
        float *ap = part_acc + part * HD + 4 * g;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<floatx4 *>(ap + 16 * dt) = num[dt];
        if (g == 0) {
            part_ml[2 * part] = mx;
            part_ml[2 * part + 1] = den;
        }
    }
}

template <int HD, int W, bool NT>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2))) void
decode_splitk_kernel(const uint16_t *__restrict__ k_pool, const uint16_t *__restrict__ v_pool,
                     uint32_t kv_heads, const uint32_t *__restrict__ tables,
                     const uint32_t *__restrict__ work,
                     const uint32_t *__restrict__ row_info, uint32_t split_keys,
                     const uint16_t *__restrict__ q, uint16_t *__restrict__ out,
                     float *__restrict__ part_acc, float *__restrict__ part_ml, uint32_t num_heads,
                     uint32_t group, float scale_log2, const uint32_t *__restrict__ counts,
                     const uint32_t *__restrict__ mates, uint32_t pack, uint16_t *__restrict__ k_w,
                     uint16_t *__restrict__ v_w, const uint16_t *__restrict__ new_k,
                     const uint16_t *__restrict__ new_v, const uint32_t *__restrict__ new_slots,
                     uint32_t num_shared, uint32_t shared_pairs) {
#pragma clang fp contract(off)  // the wavefronts' merge rounds as a shared pack's does
    constexpr int KK = HD / 32;
    constexpr int DT = HD / 16;
    constexpr uint32_t kTile = kBS * HD;
    __shared__ uint32_t s_col[3][16];  // per column: row, first partial, splits
    extern __shared__ float smem[];  // the wavefronts' merge (without stages)
    // The stages of a shared pack (four objects of their own, so that the
    // compiler can tell one stage's DMA from another stage's reads and waits
    // for neither); the register path's merge keeps wavefront w's
    // accumulators in stage w.
    constexpr bool kStages = W == kSharedWaves;
    constexpr uint32_t kStageBytes = kStages ? SharedStage<HD>::BYTES : 16;
    __shared__ __align__(1024) uint8_t sh0[kStageBytes];
    __shared__ __align__(1024) uint8_t sh1[kStageBytes];
    __shared__ __align__(1024) uint8_t sh2[kStageBytes];
    __shared__ __align__(1024) uint8_t sh3[kStageBytes];
    __shared__ float s_ml[kStages ? 2 * W * 16 : 1];
    static_assert(!kStages || 16 * kAccStride<HD> * 4 <= kStageBytes, "merge fits a stage");

    const uint32_t item = blockIdx.x / kv_heads;
    const uint32_t kvh = blockIdx.x % kv_heads;
    // The item's record loads beside the step's count: every launched item
    // has a readable record.  The grid may be sized for more work than this
    // step has (fixed launch shapes); the step's own count is on the device.
    const u32x4 rec = *reinterpret_cast<const u32x4 *>(work + 4 * static_cast<uint64_t>(item));
    if (item >= counts[0]) return;
    const uint32_t row = rec[0];
    const uint32_t split = rec[1];
    const uint32_t *table = tables + rec[2];  // this split's block ids
    const uint32_t nk = rec[3];
    const uint64_t out_base = static_cast<uint64_t>(row) * num_heads * HD;

    if (nk == 0) {
        // The reference's empty softmax leaves the zero-filled output
        // (attention.rs:119); one work item covers such a row.
        for (uint32_t idx = threadIdx.x; idx < group * HD; idx += 64 * W)
            out[out_base + static_cast<uint64_t>(kvh) * group * HD + idx] = 0;
        return;
    }
    if constexpr (kStages) {
        if (item < num_shared) {
            if (shared_pairs)
                shared_split_pairs<HD, W>(k_pool, v_pool, kv_heads, kvh, item, rec, tables,
                                          row_info, split_keys, q, out, part_acc, part_ml,
                                          num_heads, group, scale_log2, mates, pack, sh0, sh1,
                                          sh2, sh3);
            else
                shared_split<HD, W>(k_pool, v_pool, kv_heads, kvh, item, rec, tables, row_info,
                                    split_keys, q, out, part_acc, part_ml, num_heads, group,
                                    scale_log2, mates, pack, sh0, sh1, sh2, sh3);
            return;
        }
    }
    // In a plan with shared packs every item with mates is one of them.
    if (num_shared != 0) pack = 1;

    const uint32_t k_begin = split * split_keys;
    const uint32_t k_end = min(nk, k_begin + split_keys);
    const uint32_t nblk = (k_end - k_begin + kBS - 1) / kBS;
    const uint32_t nchunks = (k_end - k_begin + kChunk - 1) / kChunk;
    // With new keys given, the item holding the row's last key caches it
    // and takes it from new_k / new_v (see NewKeys).
    const bool take_new = new_k != nullptr && k_end == nk;
    const uint16_t *nk_row = take_new ? new_k + (static_cast<uint64_t>(row) * kv_heads + kvh) * HD : nullptr;
    const uint16_t *nv_row = take_new ? new_v + (static_cast<uint64_t>(row) * kv_heads + kvh) * HD : nullptr;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane & 15;  // MFMA column of this lane
    const int g = lane >> 4;  // lane group: keys 8g..8g+7 of a chunk

    LaneMap lm;
    {
        const int m = lane & 15;
        lm.k_off = (8 * ((m >> 2) & 1) + (m & 3)) * 32 + 8 * g;
        lm.k_hi = m >= 8;
        lm.v_off = m * kBS + 8 * (g & 1);
        lm.v_hi = g >= 2;
    }
    const uint64_t block_stride = static_cast<uint64_t>(kv_heads) * kTile;
    const uint16_t *k_head = k_pool + static_cast<uint64_t>(kvh) * kTile;
    const uint16_t *v_head = v_pool + static_cast<uint64_t>(kvh) * kTile;

    // Column h holds query head kvh*group + hh of row slot h / group: slot 0
    // is the item's own row, slot j > 0 its j-th mate (a row whose split
    // reads the same blocks); columns past the pack stay zero.  MFMA output
    // columns and the per-column softmax never mix, so a packed row gets the
    // same bits as it would alone.
    const uint32_t pslot = static_cast<uint32_t>(h) / group;
    const uint32_t hh = static_cast<uint32_t>(h) - pslot * group;
    uint32_t crow = kNoMate;
    if (pslot == 0)
        crow = row;
    else if (pslot < pack)
        crow = mates[(pack - 1) * item + pslot - 1];
    const bool head_ok = crow != kNoMate;
    const uint32_t qhead = kvh * group + hh;

    // Q^T operand: column h, dims 32*kk + 8g .. +7.
    bf16x8 qv[KK];
    {
        const uint16_t *qp =
            q + (static_cast<uint64_t>(head_ok ? crow : row) * num_heads + qhead) * HD + 8 * g;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qv[kk] = head_ok ? load_bf16x8(qp + 32 * kk) : bf16x8{};
    }
    // The column's output place (first partial, splits), loaded now so that
    // the end of the item waits on no load.
    u32x2 cinfo = {0u, 0u};
    if (head_ok) cinfo = *reinterpret_cast<const u32x2 *>(row_info + 2 * static_cast<uint64_t>(crow));

    // Block ids of chunk cc: wave-uniform, so scalar loads from the table
    // (no LDS copy, no VGPR).  Load order: mates, Q and column info, first
    // chunk, so that each wait for a value (vmcnt counts in issue order)
    // leaves the later loads in flight.  Every wave issues its first chunk,
    // a wave without one from the split's last block, so that no branch
    // leaves the compiler's wait counting unsure.
    auto load = [&](Chunk<HD> &r, uint32_t cc) {
        const uint32_t b0 = min(2 * cc, nblk - 1);
        const uint32_t p0 = table[b0];
        const uint32_t p1 = (b0 + 1 < nblk) ? table[b0 + 1] : p0;
        load_chunk<HD, NT>(r, k_head, v_head, block_stride, p0, p1, lm);
        issue_fence();
    };
    Chunk<HD> bufA, bufB;
    // This wavefront's chunks: wave + k W for k < mine.
    const uint32_t mine = nchunks > static_cast<uint32_t>(wave) ? (nchunks - wave + W - 1) / W : 0;
    auto chunk = [&](uint32_t k) { return static_cast<uint32_t>(wave) + k * W; };
    load(bufA, chunk(0));

    float m_run = -INFINITY;
    float l_run = 0.0f;
    floatx4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

    // A chunk computed inside the loop has a successor, so it is full: only
    // the chunks computed at the loop's exits can be the split's tail, and
    // only they carry the masking code.
    auto run = [&](Chunk<HD> &r, uint32_t cc, bool may_tail) {
        const uint32_t j0 = k_begin + cc * kChunk;
        if (may_tail && take_new && cc + 1 == nchunks)
            take_new_key<HD>(r, nk - 1 - j0, nk_row, nv_row, lane);
        const bool tail = may_tail && j0 + kChunk > k_end;
        const int nv = max(0, min(8, static_cast<int>(k_end) - static_cast<int>(j0 + 8 * g)));
        compute_chunk<HD>(r, qv, tail, nv, scale_log2, m_run, l_run, acc);
    };

    // Two register buffers: the loads of chunk k + 1 are all issued (the
    // fence in `load`) before the first wait for chunk k, so each wavefront
    // has two chunks in flight while it waits.  The loop has one exit and
    // the last one or two chunks follow it: with an early exit inside the
    // loop, the control-flow structurizer routes that exit back through the
    // loop header, where the compiler then waits for every load in flight.
    uint32_t k = 0;
    for (; k + 2 < mine; k += 2) {
        load(bufB, chunk(k + 1));
        run(bufA, chunk(k), false);
        load(bufA, chunk(k + 2));
        run(bufB, chunk(k + 1), false);
    }
    if (k + 1 < mine) {
        load(bufB, chunk(k + 1));
        run(bufA, chunk(k), false);
        run(bufB, chunk(k + 1), true);
    } else if (k < mine) {
        run(bufA, chunk(k), true);
    }

    // Cache the new key (nothing in this launch reads its slot from the pool).
    if (take_new) {
        const uint32_t slot = new_slots[row];
        const uint64_t tile = static_cast<uint64_t>(slot / kBS) * block_stride + static_cast<uint64_t>(kvh) * kTile;
        const uint32_t t = slot % kBS;
        for (uint32_t u = threadIdx.x; u < HD / 8; u += 64 * W) {
            const uint32_t d = 8 * u;
            *reinterpret_cast<u32x4 *>(k_w + tile + (d / 32) * (kBS * 32) + t * 32 + d % 32) =
                *reinterpret_cast<const u32x4 *>(nk_row + d);
        }
        for (uint32_t d = threadIdx.x; d < HD; d += 64 * W) v_w[tile + d * kBS + t] = nv_row[d];
    }

    // The running sums are per lane group; the max is already per head.
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);

    if constexpr (W == 1) {
        if (head_ok) {
            const uint32_t nsplit = cinfo[1];
            const uint64_t part_base = static_cast<uint64_t>(cinfo[0] + split) * num_heads;
            if (nsplit == 1) {
                const float inv = 1.0f / l_run;
                uint16_t *op = out + static_cast<uint64_t>(crow) * num_heads * HD +
                               static_cast<uint64_t>(qhead) * HD + 4 * g;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    u32x2 packed;
                    packed[0] = f32_to_bf16_bits(acc[dt][0] * inv) |
                                (static_cast<uint32_t>(f32_to_bf16_bits(acc[dt][1] * inv)) << 16);
                    packed[1] = f32_to_bf16_bits(acc[dt][2] * inv) |
                                (static_cast<uint32_t>(f32_to_bf16_bits(acc[dt][3] * inv)) << 16);
                    *reinterpret_cast<u32x2 *>(op + 16 * dt) = packed;
                }
            } else {
                const uint64_t part = part_base + qhead;
                float *ap = part_acc + part * HD + 4 * g;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<floatx4 *>(ap + 16 * dt) = acc[dt];
                if (g == 0) {
                    part_ml[2 * part] = m_run;
                    part_ml[2 * part + 1] = l_run;
                }
            }
        }
    } else {
        // Merge the W wavefronts' (m, l, acc) through LDS.
        float *sm_m = kStages ? s_ml : smem;  // [W][16]
        float *sm_l = sm_m + W * 16;          // [W][16]
        // [W][cols][HD]: wavefront w's block at sm_acc_w(w)
        float *sm_acc = kStages ? nullptr : sm_l + W * 16;
        const uint32_t cols = pack * group;
        auto sm_acc_w = [&](int w) -> float * {
            if constexpr (kStages)
                return reinterpret_cast<float *>(w == 0 ? sh0 : (w == 1 ? sh1 : (w == 2 ? sh2 : sh3)));
            else
                return sm_acc + static_cast<uint32_t>(w) * cols * kAccStride<HD>;
        };
        if (wave == 0 && g == 0) {
            s_col[0][h] = crow;
            s_col[1][h] = cinfo[0];
            s_col[2][h] = cinfo[1];
        }
        if (head_ok) {
            if (g == 0) {
                sm_m[wave * 16 + h] = m_run;
                sm_l[wave * 16 + h] = l_run;
            }
            float *ap = sm_acc_w(wave) + h * kAccStride<HD> + 4 * g;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<floatx4 *>(ap + 16 * dt) = acc[dt];
        }
        __syncthreads();
        for (uint32_t idx = threadIdx.x; idx < cols * HD; idx += 64 * W) {
            const uint32_t col = idx / HD;
            const uint32_t d = idx % HD;
            const uint32_t r = s_col[0][col];
            if (r == kNoMate) continue;  // a short pack
            float mx = -INFINITY;
#pragma unroll
            for (int w = 0; w < W; ++w) mx = fmaxf(mx, sm_m[w * 16 + col]);
            float num = 0.0f, den = 0.0f;
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float mw = sm_m[w * 16 + col];
                if (mw != -INFINITY) {
                    const float e = __builtin_amdgcn_exp2f(mw - mx);
                    num += e * sm_acc_w(w)[col * kAccStride<HD> + d];
                    den += e * sm_l[w * 16 + col];
                }
            }
            const uint32_t qh = kvh * group + (col % group);
            const uint32_t nsplit = s_col[2][col];
            if (nsplit == 1) {
                out[static_cast<uint64_t>(r) * num_heads * HD + static_cast<uint64_t>(qh) * HD + d] =
                    f32_to_bf16_bits(num / den);
            } else {
                const uint64_t part = static_cast<uint64_t>(s_col[1][col] + split) * num_heads + qh;
                part_acc[part * HD + d] = num;
                if (d == 0) {
                    part_ml[2 * part] = mx;
                    part_ml[2 * part + 1] = den;
                }
            }
        }
    }
}

// Merge the split-K partials of one (row, query head) for the rows listed in
// reduce_rows (those with more than one split; rows with one split were
// written by the split kernel).  The 256 threads are HD/4 dim quads x P
// split lanes: lane p folds splits p, p + P, ... with a running max (its
// loads are independent of each other), and the P lane results are merged
// through LDS in lane order.  The merge order depends only on the row's
// number of splits, so the result is the same in any batch.  With P lanes a
// 64-split row costs 8 dependent load rounds instead of 64.
template <int HD>
__global__ __launch_bounds__(256) void decode_reduce_kernel(
    const uint32_t *__restrict__ row_info, const uint32_t *__restrict__ reduce_rows,
    const float *__restrict__ part_acc, const float *__restrict__ part_ml,
    uint16_t *__restrict__ out, uint32_t num_heads, const uint32_t *__restrict__ counts) {
    constexpr int NQ = HD / 4;     // dim quads of one head
    constexpr int P = 256 / NQ;    // split lanes
    __shared__ float s_m[P][NQ];
    __shared__ float s_l[P][NQ];
    __shared__ floatx4 s_acc[P][NQ];

    if (blockIdx.x / num_heads >= counts[1]) return;  // past this step's rows (fixed launch)
    const uint32_t row = reduce_rows[blockIdx.x / num_heads];
    const uint32_t qh = blockIdx.x % num_heads;
    const uint32_t first = row_info[2 * row];
    const uint32_t nsplit = row_info[2 * row + 1];
    const uint32_t dq = threadIdx.x % NQ;
    const uint32_t p = threadIdx.x / NQ;
    const uint32_t d = 4 * dq;

    float mx = -INFINITY, den = 0.0f;
    floatx4 num = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
    for (uint32_t i = p; i < nsplit; i += P) {
        const uint64_t part = static_cast<uint64_t>(first + i) * num_heads + qh;
        const float m = part_ml[2 * part];  // finite: a split holds >= 1 key
        const float l = part_ml[2 * part + 1];
        const floatx4 a = *reinterpret_cast<const floatx4 *>(part_acc + part * HD + d);
        const float m_new = fmaxf(mx, m);
        const float scale_old = __builtin_amdgcn_exp2f(mx - m_new);
        const float e = __builtin_amdgcn_exp2f(m - m_new);
        den = den * scale_old + e * l;
        num = num * scale_old + a * e;
        mx = m_new;
    }
    s_m[p][dq] = mx;
    s_l[p][dq] = den;
    s_acc[p][dq] = num;
    __syncthreads();
    if (p != 0) return;
    float M = s_m[0][dq];
#pragma unroll
    for (int j = 1; j < P; ++j) M = fmaxf(M, s_m[j][dq]);
    float L = 0.0f;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < P; ++j) {
        const float mj = s_m[j][dq];
        if (mj == -INFINITY) continue;  // lane j had no split
        const float e = __builtin_amdgcn_exp2f(mj - M);
        L += e * s_l[j][dq];
        acc += s_acc[j][dq] * e;
    }
    const float inv = 1.0f / L;
    u32x2 packed;
    packed[0] = f32_to_bf16_bits(acc[0] * inv) |
                (static_cast<uint32_t>(f32_to_bf16_bits(acc[1] * inv)) << 16);
    packed[1] = f32_to_bf16_bits(acc[2] * inv) |
                (static_cast<uint32_t>(f32_to_bf16_bits(acc[3] * inv)) << 16);
    const uint64_t out_off = (static_cast<uint64_t>(row) * num_heads + qh) * HD + d;
    *reinterpret_cast<u32x2 *>(out + out_off) = packed;
}

template <int HD, int W, bool NT>
hipError_t launch_split(const PoolLayer &pool, const MetaView &meta, const DecodePlan &plan,
                        const uint16_t *q, uint16_t *out, uint32_t num_heads, float scale_log2,
                        hipStream_t stream, const NewKeys *nkeys) {
    const uint32_t group = num_heads / pool.kv_heads;
    const uint32_t pack = plan.pack ? plan.pack : 1;
    const uint32_t shared = plan.num_shared;
    // Shared packs: W wavefronts of up to 16 / G rows; the other items then
    // carry no mates.  (A shared pack never holds a row's new key: its blocks
    // are read by another row, so a plan with new keys has none there.)
    const uint32_t shared_tiles = plan.shared_pairs ? W / 2 : W;
    if (shared != 0 && (W != kSharedWaves || group > 16 ||
                        pack > shared_tiles * (16 / group) || plan.split_keys % kChunk != 0))
        return hipErrorInvalidValue;
    const uint32_t item_pack = shared ? 1u : pack;
    if (item_pack * group > 16 || (pack > 1 && plan.mates == nullptr)) return hipErrorInvalidValue;
    // With 4 wavefronts (not streaming) the merge lives in the shared-pack
    // stages (at most 16 columns of HD floats per wavefront, 8 KiB at
    // head_dim 128).
    constexpr bool kStages = W == kSharedWaves;
    const size_t smem =
        (W == 1 || kStages) ? 0
                            : (2 * W * 16 + static_cast<size_t>(W) * item_pack * group * kAccStride<HD>) * 4;
    const uint64_t grid = static_cast<uint64_t>(plan.launch_work) * pool.kv_heads;
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
    KernelTimer timer("decode_splitk", stream);
    hipLaunchKernelGGL((decode_splitk_kernel<HD, W, NT>), dim3(static_cast<uint32_t>(grid)),
                       dim3(64 * W), smem, stream, pool.k, pool.v, pool.kv_heads, meta.tables,
                       plan.work, plan.row_info,
                       plan.split_keys, q, out, plan.part_acc, plan.part_ml, num_heads, group,
                       scale_log2, plan.counts, plan.mates, pack, pool.k, pool.v,
                       nkeys ? nkeys->k : nullptr, nkeys ? nkeys->v : nullptr,
                       nkeys ? nkeys->slots : nullptr, shared, plan.shared_pairs ? 1u : 0u);
    return hipGetLastError();
}

template <int HD>
hipError_t launch_hd(const PoolLayer &pool, const MetaView &meta, const DecodePlan &plan,
                     const uint16_t *q, uint16_t *out, uint32_t num_heads, float scale_log2,
                     int waves, hipStream_t stream, const NewKeys *nkeys) {
    hipError_t err;
    const bool nt = plan.streaming;
#define VO_SPLIT(Wv)                                                                            \
    (nt ? launch_split<HD, Wv, true>(pool, meta, plan, q, out, num_heads, scale_log2, stream,  \
                                     nkeys)                                                  \
        : launch_split<HD, Wv, false>(pool, meta, plan, q, out, num_heads, scale_log2, stream, \
                                      nkeys))
    switch (waves) {
        case 1: err = VO_SPLIT(1); break;
        case 2: err = VO_SPLIT(2); break;
        case 8: err = VO_SPLIT(8); break;
        default: err = VO_SPLIT(4); break;
    }
#undef VO_SPLIT
    if (err != hipSuccess || plan.launch_reduce == 0) return err;
    const uint64_t grid = static_cast<uint64_t>(plan.launch_reduce) * num_heads;
    if (grid > 0x7fffffffull) return hipErrorInvalidValue;
    KernelTimer timer("decode_reduce", stream);
    hipLaunchKernelGGL((decode_reduce_kernel<HD>), dim3(static_cast<uint32_t>(grid)), dim3(256),
                       0, stream, plan.row_info, plan.reduce_rows, plan.part_acc, plan.part_ml,
                       out, num_heads, plan.counts);
    return hipGetLastError();
}

}  // namespace

bool decode_mfma_supported(uint32_t head_dim, uint32_t block_size, uint32_t group) {
    return (head_dim == 64 || head_dim == 128) && block_size == kBS && group >= 1 && group <= 16;
}

hipError_t launch_decode_mfma(const PoolLayer &pool, const MetaView &meta,
                              const DecodePlan &plan, const uint16_t *q, uint16_t *out,
                              uint32_t num_heads, float scale, int waves_per_group,
                              hipStream_t stream, const NewKeys *new_keys) {
    if (plan.launch_work == 0) return hipSuccess;
    // New keys need exactly the plan's items (not a fixed launch's grid).
    if (new_keys && plan.launch_work != plan.num_work) return hipErrorInvalidValue;
    if (plan.split_keys == 0 || plan.split_keys % kChunk != 0 || plan.split_keys > kMaxSplitKeys)
        return hipErrorInvalidValue;
    const float scale_log2 = scale * 1.4426950408889634f;
    switch (pool.head_dim) {
        case 64:
            return launch_hd<64>(pool, meta, plan, q, out, num_heads, scale_log2, waves_per_group,
                                 stream, new_keys);
        case 128:
            return launch_hd<128>(pool, meta, plan, q, out, num_heads, scale_log2,
                                  waves_per_group, stream, new_keys);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace kernels
}  // namespace vo

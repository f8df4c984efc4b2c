"""Generates prefill_pipe_loop.inc: the KV-tile loop of prefill_pipe_kernel
(chunked_prefill.hip) as one inline-asm string.

    python3 gen_prefill_pipe.py > prefill_pipe_loop.inc

One wavefront per SIMD holds 64 query rows (row groups rg 0 and 1, 32 rows
each) of one query head, head_dim 128.  Tile 0 runs before the loop (its
max is the fixed softmax offset m); the loop covers tiles 1 .. n - 1.
Tile t of the item sits in LDS stage (tbase + t) % 4: the persistent kernel
runs several items back to back through one ring, and an item's tile 0
follows the previous item's last tile.  The tile counter t of the loop is
tbase + (the tile's index in the item); keys are indexed from the item's
first key.  Before the loop, the fill computes S of tile 1 (masked if
needed) and P of its first 16 keys.  Iteration t then issues, in MFMA order,

    P1  P.V of tile t, keys 0-15   ( 8 MFMAs; V fragments and P ready)
    P2  Q.K^T of tile t + 1        (32 MFMAs; K from LDS stage (t+1) % 4)
    P3  P.V of tile t, keys 16-63  (24 MFMAs; V from stage t % 4)

and between them the VALU work: the softmax of tile t's keys 16-63 in P1
and P2; in P3 the causal mask of tile t + 1 when it needs one and the
softmax of its keys 0-15.  The row sums add each f32 probability in key
order (one v_add_f32 chain per lane and row group; a v_dot2 would block the
MFMA pipe).  On gfx950 independent VALU
instructions co-issue with a running 32-cycle v_mfma_f32_32x32x16_bf16, so
the softmax runs under the MFMAs.  Iteration t starts with the wait for tile
t + 1's DMA and a barrier (after which stage (t+3) % 4 is free: every wave
has left iteration t - 1), then issues the DMA of tile t + 3 under P1's
MFMAs.  The last tile (t = n - 1) takes a variant without Q.K^T; its DMA,
like those of the two iterations before it, fetches a tile past the item's
end: the block table in LDS continues there with the next item's first
three tiles, which so arrive while this item finishes.

Each K or V fragment read from LDS feeds two MFMAs (the two row groups).
Per row the arithmetic is the 32-row kernels' operation for operation: S
accumulates the eight 16-dim k-steps in order from zero, masked scores are
-inf, p = exp2(fma(s, scale, -m)), P is rounded to bf16 (nearest even), the
row sum adds the f32 p in key order (each lane its 32 keys of the tile),
and O accumulates a tile's four 16-key steps in order.

Register map (physical; the kernel pins its operands to these):
    a[0:127]    O: block (rg, dt) at a[16 (4 rg + dt)] (32 dims x 32 rows)
    a[128:191]  Q: fragment (rg, kk) at a[128 + 4 (8 rg + kk)]
    a[192:223]  K fragment slots (8)       a[224:255]  V fragment slots (8)
    v[0:63]     S buffer 0, v[64:127] S buffer 1; block (rg, h) at +16 (2 h + rg)
    v[128:159]  P: (rg, j) at v[128 + 16 rg + 4 j] (bf16 pairs)
    v[160:163]  block ids of the tile whose DMA the next iteration issues
    v164, v165  -m (rg 0, 1)           v166, v167  row sums (rg 0, 1; per lane)
    v180        -inf
    v181, v182  K read address at stage 0 (even / odd k-steps); v183, v184 + 64 KiB
    v185        V read address at stage 0; v186 + 64 KiB
    v187, v188  per-lane DMA source offsets (K, V)
    v189        LDS address of the next block-id quad
    v190, v191  p_row - 8 (lane / 32) for rg 0, 1 (the mask's per-lane bound)
    v192        scratch of the mask

Stage s of the four-stage ring sits at s x 32 KiB (K at +0, V at +16 KiB).
The wave's LDS DMA copies 1 KiB of each of a tile's four blocks, K then V,
to m0 = wbase + s x 32 KiB (+ 16 KiB) + 4 KiB x block.

Hazards the code keeps by construction (the compiler does not see inside
the asm): a packed P is read by an MFMA at least 3 instructions later
(s_nop otherwise); scores are read by VALU at least three MFMAs after the
MFMA that wrote them; a v_cmp lane mask is read by v_cndmask three
instructions later; m0 is written one instruction before its LDS DMA;
LDS reads are waited for with exact lgkmcnt counts (LDS returns in order).
"""

STAGE = 32768
VOFF = 16384
BT = 4096  # bytes of one (block, KV head) tile at head_dim 128

K_AHEAD = 8   # MFMA slots between a K fragment's read and its first use
V_AHEAD = 7   # the same for V fragments
DMA_SPREAD = 4  # MFMA slots between the tile DMA's eight loads (the last
                # tile's iteration: half).  Each buffer load with a VGPR
                # address costs about 20 cycles of MFMA issue on gfx950; the
                # four wavefronts issue theirs at the same slots, and spread
                # out they overlap the running MFMAs better (-1 to -2%).


def O(rg, dt):
    b = 16 * (4 * rg + dt)
    return f"a[{b}:{b + 15}]"


def Q(rg, kk):
    b = 128 + 4 * (8 * rg + kk)
    return f"a[{b}:{b + 3}]"


def S(buf, rg, h):
    return 64 * buf + 16 * (2 * h + rg)


def P(rg, j):
    return 128 + 16 * rg + 4 * j


def kslot(n):
    b = 192 + 4 * (n % 8)
    return f"a[{b}:{b + 3}]"


def vslot(n):
    b = 224 + 4 * (n % 8)
    return f"a[{b}:{b + 3}]"


def k_read(stage, n):
    """K fragment n = 2 kk + h of the tile in `stage`, into slot n."""
    kk, h = n // 2, n % 2
    base = ("v181" if kk % 2 == 0 else "v182") if stage < 2 else ("v183" if kk % 2 == 0 else "v184")
    off = (stage % 2) * STAGE + (kk // 2) * 1024 + h * 2 * BT
    return f"ds_read_b128 {kslot(n)}, {base} offset:{off}"


def v_read(stage, n):
    """V fragment n = 4 j + dt of the tile in `stage`, into slot n."""
    j, dt = n // 4, n % 4
    base = "v185" if stage < 2 else "v186"
    off = (stage % 2) * STAGE + j * BT + dt * 1024
    return f"ds_read_b128 {vslot(n)}, {base} offset:{off}"


def qk_mfma(buf, n, rg):
    kk, h = n // 2, n % 2
    dst = S(buf, rg, h)
    src_c = "0" if kk == 0 else f"v[{dst}:{dst + 15}]"
    return f"v_mfma_f32_32x32x16_bf16 v[{dst}:{dst + 15}], {kslot(n)}, {Q(rg, kk)}, {src_c}"


def pv_mfma(n, rg):
    j, dt = n // 4, n % 4
    return f"v_mfma_f32_32x32x16_bf16 {O(rg, dt)}, {vslot(n)}, v[{P(rg, j)}:{P(rg, j) + 3}], {O(rg, dt)}"


def softmax_j(buf, j):
    """fma + exp + row-sum add + bf16 pack of the 16 scores (8 per row
    group) of 16-key step j of the S buffer into P(rg, j).  The two row groups' chains are
    interleaved and each exp trails its fma by two ops, so exps (the
    slow VALU op) spread out; a pack follows its second exp by at least
    two ops (a transcendental result needs one wait state)."""
    base = [S(buf, rg, j >> 1) + 8 * (j & 1) for rg in range(2)]
    fm = [f"v_fma_f32 v{base[rg] + i}, v{base[rg] + i}, %[scale], v{164 + rg}"
          for i in range(8) for rg in range(2)]
    ex = [f"v_exp_f32 v{base[rg] + i}, v{base[rg] + i}" for i in range(8) for rg in range(2)]
    pk = {(rg, i): f"v_cvt_pk_bf16_f32 v{P(rg, j) + i // 2}, v{base[rg] + i}, v{base[rg] + i + 1}"
          for rg in range(2) for i in range(0, 8, 2)}
    ad = [f"v_add_f32 v{166 + rg}, v{166 + rg}, v{base[rg] + i}" for i in range(8) for rg in range(2)]
    ops = fm[:4]
    pend = []  # (ops to wait, pack)

    def push(op):
        ops.append(op)
        for q in pend:
            q[0] -= 1
        while pend and pend[0][0] <= 0:
            ops.append(pend.pop(0)[1])
            for q in pend:
                q[0] -= 1

    for k in range(16):
        if k + 4 < 16:
            push(fm[k + 4])
        push(ex[k])
        i, rg = k // 2, k % 2
        pend.append([2, ad[k]])
        if i % 2 == 1:
            pend.append([2, pk[(rg, i - 1)]])
    while pend:
        ops.append(pend.pop(0)[1])
    return ops


def mask_ops(buf):
    """Causal mask of the S buffer for the tile starting at key %[j0]: score
    r of block (rg, h) is key j0 + 32 h + 16 (r >> 3) + 8 (lane / 32) +
    (r & 7) and stays when that key <= p_row, i.e. when its lane-free part
    32 h + 16 (r >> 3) + (r & 7) <= p_row - 8 (lane / 32) - j0 (signed)."""
    ops = []
    pairs = ["%[m0]", "%[m1]", "%[m2]"]
    for rg in range(2):
        ops.append(f"v_subrev_u32 v192, %[j0], v{190 + rg}")
        cm = []
        for h in range(2):
            for r in range(16):
                cm.append((S(buf, rg, h) + r, 32 * h + 16 * (r >> 3) + (r & 7)))
        pend = []
        for i, (reg, off) in enumerate(cm):
            ops.append(f"v_cmp_lt_i32_e64 {pairs[i % 3]}, v192, {off}")
            pend.append((i, reg))
            if len(pend) == 3:
                k, rk = pend.pop(0)
                ops.append(f"v_cndmask_b32_e64 v{rk}, v{rk}, v180, {pairs[k % 3]}")
        ops.append("s_nop 1")
        for k, rk in pend:
            ops.append(f"v_cndmask_b32_e64 v{rk}, v{rk}, v180, {pairs[k % 3]}")
    return ops


class Body:
    """One code path: lines plus the LDS reads issued so far, so that each
    wait names exactly the reads issued after the one needed."""

    def __init__(self):
        self.lines = []
        self.lds_n = 0
        self.lds_done = 0

    def emit(self, s):
        self.lines.append(s)

    def lds(self, s):
        self.lines.append(s)
        self.lds_n += 1
        return self.lds_n

    def wait(self, seq):
        if seq > self.lds_done:
            self.lines.append(f"s_waitcnt lgkmcnt({min(self.lds_n - seq, 15)})")
            self.lds_done = seq


# Issue cost (cycles) of VALU ops, and the VALU budget of one 32-cycle MFMA
# slot.  Spreading the softmax evenly over the MFMAs (about 14 cycles of
# VALU per slot here) runs a tile in ~2,355 cycles against ~2,515 when each
# slot is filled to 28 cycles first (probe of this loop with static LDS,
# MFMA floor 2,176): co-issued VALU still costs about a cycle per op, more
# when bunched.
COST = {"v_exp_f32": 9, "s_nop": 2, "WAITALL": 0}
BUDGET = 16


def cost(op):
    return COST.get(op.split()[0], 4)


def run_slots(b, mfmas, reads, valu, side, first_use):
    """Emits the MFMAs in order with the other work between them.
    mfmas: (text, fragment key or None, P registers read)
    reads: (key, text, ahead): issued once the slot reaches first_use - ahead
    valu:  (op, earliest slot, deadline slot), kept in list order; after
           each MFMA, ops up to the slot's cycle budget, more only when a
           deadline needs them
    side:  (op, earliest slot), at most 6 per slot, in list order"""
    seqs = {}
    ri = vi = si = 0
    last_pack = {}

    def issue_reads(slot):
        nonlocal ri
        while ri < len(reads):
            key, text, ahead = reads[ri]
            if first_use[key] - ahead > slot:
                break
            seqs[key] = b.lds(text)
            ri += 1

    def put_valu(op):
        if op == "WAITALL":
            b.emit("s_waitcnt lgkmcnt(0)")
            b.lds_done = b.lds_n
            return
        b.emit(op)
        if op.startswith("v_cvt_pk_bf16_f32"):
            reg = int(op.split()[1].rstrip(",")[1:])
            last_pack[reg - reg % 4] = len(b.lines)

    for slot, (text, rkey, pneed) in enumerate(mfmas):
        k = 0
        while si < len(side) and side[si][1] <= slot and k < 6:
            op = side[si][0]
            if op.startswith("ds_"):
                b.lds(op)
            else:
                b.emit(op)
            si += 1
            k += 1
        issue_reads(slot)
        if rkey is not None:
            b.wait(seqs[rkey])
        for preg in pneed:
            if preg in last_pack and len(b.lines) - last_pack[preg] < 3:
                b.emit("s_nop 1")
        b.emit(text)
        spent = 0
        quota = cnt = 0
        for i in range(vi, len(valu)):
            cnt += 1
            quota = max(quota, -(-cnt // max(valu[i][2] - slot, 1)))
        emitted = 0
        while vi < len(valu) and valu[vi][1] <= slot:
            c = cost(valu[vi][0])
            if emitted >= quota and spent + c > BUDGET:
                break
            put_valu(valu[vi][0])
            spent += c
            vi += 1
            emitted += 1
    while si < len(side):
        op = side[si][0]
        if op.startswith("ds_"):
            b.lds(op)
        else:
            b.emit(op)
        si += 1
    while vi < len(valu):
        put_valu(valu[vi][0])
        vi += 1


def dma_side(stage_dma):
    ops = [f"v_readfirstlane_b32 %[b{i}], v{160 + i}" for i in range(4)]
    ops += [f"s_mul_i32 %[b{i}], %[b{i}], %[stride]" for i in range(4)]
    for side, rs, voff in (("k", "%[krs]", "v187"), ("v", "%[vrs]", "v188")):
        for i in range(4):
            off = stage_dma * STAGE + (VOFF if side == "v" else 0) + i * BT
            ops.append(f"s_add_u32 m0, %[wbase], {off}")
            ops.append("s_nop 0")
            ops.append(f"buffer_load_dwordx4 {voff}, {rs}, %[b{i}] offen lds")
    return ops


def iteration(stage, masked_next, last):
    """Tile t with t % 4 == stage.  masked_next: tile t + 1 needs the causal
    mask.  last: t is the last tile (no Q.K^T of a next tile, no block ids
    to read)."""
    b = Body()
    cur, nxt = stage % 2, (stage + 1) % 2
    kst = (stage + 1) % 4
    b.emit("s_waitcnt vmcnt(8) lgkmcnt(0)")
    b.emit("s_barrier")
    mfmas, first_use = [], {}

    def pv_block(j):
        for nv in range(4 * j, 4 * j + 4):
            for rg in range(2):
                key = ("v", nv) if nv >= 4 else None
                if key:
                    first_use.setdefault(key, len(mfmas))
                mfmas.append((pv_mfma(nv, rg), key, [P(rg, j)]))

    pv_block(0)
    if not last:
        for n in range(16):
            for rg in range(2):
                first_use.setdefault(("k", n), len(mfmas))
                mfmas.append((qk_mfma(nxt, n, rg), ("k", n), []))
    p3 = len(mfmas)
    for j in (1, 2, 3):
        pv_block(j)
    end = len(mfmas)
    reads = []
    if not last:
        reads += [(("k", n), k_read(kst, n), K_AHEAD) for n in range(16)]
    reads += [(("v", nv), v_read(stage, nv), V_AHEAD) for nv in range(4, 16)]
    dops = dma_side((stage + 3) % 4)
    side = [(op, 0) for op in dops[:8]]
    spread = DMA_SPREAD if not last else DMA_SPREAD // 2
    side += [(op, spread * (i // 3)) for i, op in enumerate(dops[8:])]
    if not last:
        side += [("ds_read_b128 v[160:163], v189", 1), ("v_add_u32 v189, 16, v189", 1)]
        # the next tile's first V fragments, once slots 0-3 (fragments
        # 8-11 of this tile) have been read by their MFMAs
        pre = first_use[("v", 11)] + 2
        side += [(v_read(kst, nv), pre) for nv in range(4)]
    side.sort(key=lambda e: e[1])
    valu = []
    for j in (1, 2, 3):
        valu += [(op, 0, first_use[("v", 4 * j)] - 1) for op in softmax_j(cur, j)]
    if not last:
        ready = p3 + 3  # three MFMAs after the last Q.K^T
        if masked_next:
            valu += [(op, ready, end) for op in mask_ops(nxt)]
        valu += [(op, ready, end) for op in softmax_j(nxt, 0)]
    run_slots(b, mfmas, reads, valu, side, first_use)
    return b.lines


def max_ops(buf):
    """Row max of tile 0's scores (S buffer `buf`, masked): per lane and row
    group a tree of v_max_f32 over its 32 scores into the P registers (free
    until tile 0's packs), the address of lane ^ 32 for the exchange (v192),
    and, after the exchange, -max * scale into v164 / v165."""
    tree = []
    for rg in range(2):
        t = 128 + 16 * rg
        src = [S(buf, rg, h) + r for h in range(2) for r in range(16)]
        lvl = [(f"v_max_f32 v{t + i}, v{src[2 * i]}, v{src[2 * i + 1]}", rg) for i in range(16)]
        tree.append(lvl)
    ops = []
    # level 1 of both row groups interleaved, then the in-place levels
    for i in range(16):
        for rg in range(2):
            ops.append(tree[rg][i][0])
    n = 16
    while n > 1:
        n //= 2
        for i in range(n):
            for rg in range(2):
                t = 128 + 16 * rg
                ops.append(f"v_max_f32 v{t + i}, v{t + 2 * i}, v{t + 2 * i + 1}")
    ops += ["v_mbcnt_lo_u32_b32 v192, -1, 0", "v_mbcnt_hi_u32_b32 v192, -1, v192",
            "v_xor_b32 v192, 32, v192", "v_lshlrev_b32 v192, 2, v192"]
    return ops


def exchange_side():
    return ["ds_bpermute_b32 v130, v192, v128", "ds_bpermute_b32 v146, v192, v144"]


def nm_ops():
    return ["WAITALL", "v_max_f32 v128, v128, v130", "v_max_f32 v144, v144, v146",
            "v_mul_f32_e64 v164, -v128, %[scale]", "v_mul_f32_e64 v165, -v144, %[scale]"]


def LO(buf, rg, j):
    """Tile 0's bf16 lo packs of (rg, j): the first four registers of the
    eight scores they come from."""
    return S(buf, rg, j >> 1) + 8 * (j & 1)


def softmax0_j(buf, j):
    """Tile 0's softmax of 16-key step j: p = exp2(fma(s, scale, -m)), the
    row sum adds p in key order, P as bf16 hi (P registers) + lo, lo =
    bf16(p - hi) (the hi as f32 from its pack; v192 / v193 as scratch for
    row group 0 / 1)."""
    ops = []
    base = [LO(buf, rg, j) for rg in range(2)]
    for i in range(8):
        for rg in range(2):
            ops.append(f"v_fma_f32 v{base[rg] + i}, v{base[rg] + i}, %[scale], v{164 + rg}")
            ops.append(f"v_exp_f32 v{base[rg] + i}, v{base[rg] + i}")
    for k in range(4):
        for rg in range(2):
            b, hi, tmp = base[rg], P(rg, j) + k, 192 + rg
            ops += [f"v_add_f32 v{166 + rg}, v{166 + rg}, v{b + 2 * k}",
                    f"v_add_f32 v{166 + rg}, v{166 + rg}, v{b + 2 * k + 1}",
                    f"v_cvt_pk_bf16_f32 v{hi}, v{b + 2 * k}, v{b + 2 * k + 1}",
                    f"v_lshlrev_b32 v{tmp}, 16, v{hi}",
                    f"v_sub_f32 v{b + 2 * k}, v{b + 2 * k}, v{tmp}",
                    f"v_and_b32 v{tmp}, 0xffff0000, v{hi}",
                    f"v_sub_f32 v{b + 2 * k + 1}, v{b + 2 * k + 1}, v{tmp}",
                    f"v_cvt_pk_bf16_f32 v{b + k}, v{b + 2 * k}, v{b + 2 * k + 1}"]
    return ops


def pv0_mfma(n, rg, buf, lo):
    """P.V of tile 0 for V fragment n = 4 j + dt: P lo (first, from zero at
    j = 0) or hi."""
    j, dt = n // 4, n % 4
    preg = LO(buf, rg, j) if lo else P(rg, j)
    src_c = "0" if (lo and j == 0) else O(rg, dt)
    return f"v_mfma_f32_32x32x16_bf16 {O(rg, dt)}, {vslot(n)}, v[{preg}:{preg + 3}], {src_c}", preg


def head(stage, single):
    """Tile 0 (in `stage`) of the item, and unless `single` the start of
    tile 1: the DMA of tile 3; Q.K^T of tile 0; Q.K^T of tile 1 with tile
    0's mask, max and softmax (P as hi + lo) under it; P.V of tile 0 (lo,
    then hi, per 16-key step) with tile 1's mask and the P of its keys 0-15
    under it; tile 1's first V fragments.  Tiles 0 and 1 always take the
    causal mask (it keeps every key a row sees).  Leaves the state the loop
    expects at tile 1 (or, single, the item's result)."""
    b = Body()
    b0 = stage % 2
    st1 = (stage + 1) % 4
    b1 = st1 % 2
    # the ids of tile 3, its DMA, then the ids of tile 4
    seq = b.lds("ds_read_b128 v[160:163], v189")
    b.emit("v_add_u32 v189, 16, v189")
    b.wait(seq)
    b.lines += dma_side((stage + 3) % 4)
    b.lds("ds_read_b128 v[160:163], v189")
    b.emit("v_add_u32 v189, 16, v189")
    b.emit("s_mov_b32 %[j0], 0")
    mfmas, first_use, reads = [], {}, []
    for n in range(16):
        for rg in range(2):
            first_use.setdefault(("k0", n), len(mfmas))
            mfmas.append((qk_mfma(b0, n, rg), ("k0", n), []))
    reads += [(("k0", n), k_read(stage, n), K_AHEAD) for n in range(16)]
    z1 = len(mfmas)
    if not single:
        for n in range(16):
            for rg in range(2):
                first_use.setdefault(("k1", n), len(mfmas))
                mfmas.append((qk_mfma(b1, n, rg), ("k1", n), []))
        reads += [(("k1", n), k_read(st1, n), K_AHEAD) for n in range(16)]
    z3 = len(mfmas)
    if single:
        # nothing to overlap tile 0's softmax with
        run_slots(b, mfmas, reads, [], [], first_use)
        b.lines += ["s_nop 7", "s_nop 7", "s_nop 7"]
        b.lines += mask_ops(b0)
        b.lines += max_ops(b0)
        for op in exchange_side():
            b.lds(op)
        for op in nm_ops():
            if op == "WAITALL":
                b.emit("s_waitcnt lgkmcnt(0)")
                b.lds_done = b.lds_n
            else:
                b.emit(op)
        for j in range(4):
            b.lines += softmax0_j(b0, j)
        b.lines += ["s_nop 1"]
        mfmas, first_use, reads = [], {}, []
        z3 = 0
    pv = []
    for j in range(4):
        for lo in (True, False):
            for dt in range(4):
                for rg in range(2):
                    n = 4 * j + dt
                    text, preg = pv0_mfma(n, rg, b0, lo)
                    first_use.setdefault(("v0", n), len(mfmas))
                    mfmas.append((text, ("v0", n), [preg]))
    reads += [(("v0", n), v_read(stage, n), V_AHEAD) for n in range(16)]
    end = len(mfmas)
    valu, side = [], []
    if not single:
        ready0 = z1 + 3  # three MFMAs after the last Q.K^T of tile 0
        mx = mask_ops(b0) + max_ops(b0)
        xs = ready0 + 20  # the exchange, once the tree is done
        valu += [(op, ready0, xs - 1) for op in mx]
        side += [(op, xs) for op in exchange_side()]
        valu += [(op, xs + 2, z3) for op in nm_ops()]
        for j in range(4):
            valu += [(op, xs + 2, z3 + 16 * j - 1) for op in softmax0_j(b0, j)]
        # tile 1's mask and its keys 0-15, once P(rg, 0) has been read by
        # tile 0's hi MFMAs of step 0
        late = z3 + 16 + 4
        valu += [("s_mov_b32 %[j0], 64", late, end)]
        valu += [(op, late, end) for op in mask_ops(b1)]
        valu += [(op, late, end) for op in softmax_j(b1, 0)]
        # tile 1's first V fragments, once slots 0-3 (fragments 8-11 of
        # tile 0) have been read by their last MFMAs
        side += [(v_read(st1, nv), z3 + 3 * 16 + 2) for nv in range(4)]
    run_slots(b, mfmas, reads, valu, side, first_use)
    return b.lines


def loop_text():
    L = []
    # MFMA and VALU results written before the asm (O, Q) are read by the
    # loop's MFMAs; the compiler does not see them as MFMA operands.
    L += ["s_nop 7", "s_nop 7"]
    L += ["v_mov_b32 v180, 0xff800000",
          "v_add_u32 v183, 0x10000, v181", "v_add_u32 v184, 0x10000, v182",
          "v_add_u32 v186, 0x10000, v185"]
    # the head: dispatch on tile 0's stage and on a single-tile item
    L += ["s_and_b32 %[b0], %[tbase], 3", "s_add_u32 %[t], %[tbase], 1",
          "s_cmp_ge_u32 %[t], %[tend]", "s_cbranch_scc1 48f"]
    for stage in range(4):
        L += [f"s_cmp_eq_u32 %[b0], {stage}", f"s_cbranch_scc1 {40 + stage}f"]
    L += ["48:"]
    for stage in range(4):
        L += [f"s_cmp_eq_u32 %[b0], {stage}", f"s_cbranch_scc1 {44 + stage}f"]
    for single in (False, True):
        for stage in range(4):
            L += [f"{40 + 4 * single + stage}:"]
            L += head(stage, single)
            if single:
                L += ["s_branch 99f"]
            else:
                L += ["s_add_u32 %[t], %[tbase], 1", "s_branch 70f"]
    # dispatch on the last tile, t % 4 and the mask of tile t + 1 (key
    # index j0 = 64 (t + 1 - tbase))
    L += ["70:", "s_add_u32 %[j0], %[t], 1", "s_cmp_ge_u32 %[j0], %[tend]", "s_cbranch_scc1 71f",
          "s_sub_u32 %[j0], %[j0], %[tbase]", "s_lshl_b32 %[j0], %[j0], 6", "s_and_b32 %[b0], %[t], 3"]
    for stage in range(4):
        L += [f"s_cmp_eq_u32 %[b0], {stage}", f"s_cbranch_scc1 {80 + stage}f"]
    for stage in range(4):
        L += [f"{80 + stage}:", "s_cmp_ge_u32 %[j0], %[tmask]", f"s_cbranch_scc1 {84 + stage}f"]
        L += iteration(stage, False, False)
        L += ["s_add_u32 %[t], %[t], 1", "s_branch 70b", f"{84 + stage}:"]
        L += iteration(stage, True, False)
        L += ["s_add_u32 %[t], %[t], 1", "s_branch 70b"]
    L += ["71:", "s_and_b32 %[b0], %[t], 3"]
    for stage in range(4):
        L += [f"s_cmp_eq_u32 %[b0], {stage}", f"s_cbranch_scc1 {90 + stage}f"]
    for stage in range(4):
        L += [f"{90 + stage}:"]
        L += iteration(stage, False, True)
        L += ["s_branch 99f"]
    # the last MFMAs' results (O) are read after the asm
    L += ["99:", "s_nop 7", "s_nop 7", "s_nop 7"]
    return L


def main():
    lines = loop_text()
    print("// Generated by gen_prefill_pipe.py; do not edit.")
    print("// The KV-tile loop of prefill_pipe_kernel (chunked_prefill.hip).")
    print(f"// {sum(1 for l in lines if 'v_mfma' in l)} MFMAs, "
          f"{sum(1 for l in lines if l.startswith('ds_read'))} LDS reads, "
          f"{len(lines)} lines.")
    print("#define VO_PREFILL_PIPE_LOOP \\")
    for l in lines:
        print(f'    "{l}\\n" \\')
    print('    ""')
    clob = ([f'"v{i}"' for i in range(0, 166)] +
            ['"v180"', '"v183"', '"v184"', '"v186"', '"v192"', '"v193"'] +
            [f'"a{i}"' for i in range(192, 256)])
    print("#define VO_PREFILL_PIPE_CLOBBERS " + ", ".join(clob))


if __name__ == "__main__":
    main()

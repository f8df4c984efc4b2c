"""Synthetic paged-KV workloads shared by the GPU parity tests and bench.py.

A workload is one layer's paged KV state plus one step's queries, built the
way the reference engine builds it: block tables are disjoint slices of a
seeded permutation of the physical pool (cpu/tests.rs:242-244 uses shuffled,
non-identity tables for the same reason), the cached context is written
through write_kv, then this step's new K/V are written through write_kv at the
step's slot mapping before attention reads them (model.rs:309-311).

K, V and Q are bf16 ~ N(0, 1) drawn on the GPU from a seeded generator.  The
oracle receives exactly the same values widened to f32.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

FILL_ROWS = 8192  # rows per write_kv call when filling cached context


def split_tables(rng, lengths_blocks, num_blocks, shared_prefix_blocks=0, shared_count=0):
    """Disjoint tables from a permutation of the pool.  The first
    ``shared_count`` sequences start with the same ``shared_prefix_blocks``
    blocks (prefix sharing through aliased table entries)."""
    perm = rng.permutation(num_blocks).astype(np.uint32)
    pos = 0
    prefix = perm[pos:pos + shared_prefix_blocks]
    pos += shared_prefix_blocks
    tables = []
    for i, nb in enumerate(lengths_blocks):
        if i < shared_count:
            own = nb - shared_prefix_blocks
            t = np.concatenate([prefix, perm[pos:pos + own]])
            pos += own
        else:
            t = perm[pos:pos + nb]
            pos += nb
        if pos > num_blocks:
            raise ValueError("pool too small for the tables")
        tables.append(t.copy())
    return tables


@dataclass
class Workload:
    kind: str                      # "decode" or "prefill"
    heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    layer: int
    tables: List[np.ndarray]
    context_lens: np.ndarray       # cached keys per sequence before this step
    num_new: np.ndarray            # new tokens per sequence this step
    meta: object = None            # PrefillMeta / DecodeMeta (product)
    pool: object = None            # KvPool (device)
    q: object = None               # [T, heads*hd] bf16 device
    k_new: object = None           # [T, kvh*hd] bf16 device
    v_new: object = None
    ctx_kv: list = field(default_factory=list)  # per seq (k, v) cached context, device bf16
    host: Optional[dict] = None    # f32 copies for the oracle

    @property
    def rows(self) -> int:
        return int(self.num_new.sum())

    def row_num_keys(self) -> np.ndarray:
        return np.asarray(self.meta.row_num_keys, dtype=np.int64)

    def decode_bytes(self) -> int:
        """Algorithmic HBM bytes of decode attention: K+V of every key read
        once per KV head, q and out rows, and the table entries read."""
        keys = self.row_num_keys()
        kv = int(keys.sum()) * self.kv_heads * self.head_dim * 2 * 2
        qo = 2 * self.rows * self.heads * self.head_dim * 2
        tab = int(np.sum(-(-keys // self.block_size))) * 4
        return kv + qo + tab

    def decode_unique_bytes(self) -> int:
        """decode_bytes with every physical block's keys counted once (the
        HBM bytes when rows that alias a shared prefix hit it in cache):
        per block, the most keys any sequence uses in it."""
        keys = self.row_num_keys()
        bs = self.block_size
        used = {}
        for s, t in enumerate(self.tables):
            n = int(keys[s])
            for i in range(-(-n // bs)):
                b = int(t[i])
                used[b] = max(used.get(b, 0), min(bs, n - i * bs))
        kv = sum(used.values()) * self.kv_heads * self.head_dim * 2 * 2
        qo = 2 * self.rows * self.heads * self.head_dim * 2
        tab = int(np.sum(-(-keys // bs))) * 4
        return kv + qo + tab

    def attention_flops(self) -> int:
        """Q.K^T plus P.V over each row's own keys (causal-aware)."""
        return int(self.row_num_keys().sum()) * self.heads * 4 * self.head_dim


def _randn(torch, shape, gen, device):
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)


def build(vo, backend, *, kind, heads, kv_heads, head_dim, block_size, num_blocks,
          context_lens, num_new=None, seed=0, layer=0, num_layers=1, shared_prefix=0,
          shared_count=0, extra_blocks=0, keep_host=True, device=0, fill_layers=None,
          tables=None):
    """Build a workload on ``backend`` (a vo.HipBackend).  ``fill_layers``
    (default: just ``layer``) lists the pool layers that receive the same
    cached context and new tokens.  ``tables`` (default: disjoint tables from
    a seeded permutation of the pool) gives each sequence's block ids."""
    fill_layers = [layer] if fill_layers is None else list(fill_layers)
    import torch
    dev = f"cuda:{device}"
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    S = len(context_lens)
    context_lens = np.asarray(context_lens, dtype=np.int64)
    if num_new is None:
        num_new = np.ones(S, np.int64)
    num_new = np.asarray(num_new, dtype=np.int64)
    totals = context_lens + num_new
    nblocks = [int(-(-int(t) // block_size)) + extra_blocks for t in totals]
    shared_blocks = shared_prefix // block_size
    if tables is None:
        tables = split_tables(rng, nblocks, num_blocks, shared_blocks, shared_count)
    else:
        tables = [np.asarray(t, dtype=np.uint32) for t in tables]
        if any(len(t) < nb for t, nb in zip(tables, nblocks)) or len(tables) != S:
            raise ValueError("a table is shorter than its sequence")

    layout = vo.KvLayout(num_layers, num_blocks, block_size, kv_heads, head_dim)
    pool = backend.alloc_kv_pool(layout)
    width = kv_heads * head_dim
    wl = Workload(kind, heads, kv_heads, head_dim, block_size, num_blocks, layer, tables,
                  context_lens, num_new, pool=pool)

    # Cached context, written the way earlier steps would have (cpu/tests.rs:210-230).
    # A shared prefix is written once, by its first owner.
    host_ctx = []
    pending_k, pending_v, pending_s = [], [], []
    written_prefix = False
    for s in range(S):
        c = int(context_lens[s])
        k = _randn(torch, (c, width), gen, dev)
        v = _randn(torch, (c, width), gen, dev)
        if shared_count and s < shared_count and written_prefix:
            # aliased prefix positions hold the first owner's values
            k[:shared_prefix] = wl.ctx_kv[0][0][:shared_prefix]
            v[:shared_prefix] = wl.ctx_kv[0][1][:shared_prefix]
            lo = shared_prefix
        else:
            lo = 0
        if shared_count and s < shared_count:
            written_prefix = True
        wl.ctx_kv.append((k, v))
        slots = [int(tables[s][p // block_size]) * block_size + p % block_size for p in range(lo, c)]
        if c > lo:
            pending_k.append(k[lo:])
            pending_v.append(v[lo:])
            pending_s.extend(slots)
    if pending_s:
        kk = torch.cat(pending_k)
        vv = torch.cat(pending_v)
        ss = np.asarray(pending_s, np.uint32)
        for lay in fill_layers:
            for a in range(0, len(ss), FILL_ROWS):
                b = min(a + FILL_ROWS, len(ss))
                backend.write_kv(pool, lay, kk[a:b].contiguous(), vv[a:b].contiguous(), ss[a:b])

    # This step.
    if kind == "decode":
        wl.meta = vo.DecodeMeta.new(
            [vo.DecodeSeq(int(context_lens[s]), tables[s]) for s in range(S)], block_size)
    else:
        wl.meta = vo.PrefillMeta.new(
            [vo.PrefillSeq(int(context_lens[s]), int(num_new[s]), tables[s]) for s in range(S)],
            block_size)
    T = wl.rows
    wl.k_new = _randn(torch, (T, width), gen, dev)
    wl.v_new = _randn(torch, (T, width), gen, dev)
    wl.q = _randn(torch, (T, heads * head_dim), gen, dev)
    for lay in fill_layers:
        backend.write_kv(pool, lay, wl.k_new, wl.v_new, wl.meta)

    if keep_host:
        wl.host = dict(
            ctx=[(k.float().cpu().numpy(), v.float().cpu().numpy()) for k, v in wl.ctx_kv],
            k_new=wl.k_new.float().cpu().numpy(), v_new=wl.v_new.float().cpu().numpy(),
            q=wl.q.float().cpu().numpy())
    torch.cuda.synchronize()
    return wl


def oracle_pool(orc, wl: Workload, num_layers=1):
    """The same KV state in the oracle's f32 pool, written through its write_kv."""
    pool = orc.Pool(max(num_layers, wl.layer + 1), wl.num_blocks, wl.block_size, wl.kv_heads,
                    wl.head_dim)
    bs = wl.block_size
    for s, (k, v) in enumerate(wl.host["ctx"]):
        c = k.shape[0]
        if c:
            slots = [int(wl.tables[s][p // bs]) * bs + p % bs for p in range(c)]
            pool.write_kv(wl.layer, k, v, slots)
    pool.write_kv(wl.layer, wl.host["k_new"], wl.host["v_new"], wl.meta.slot_mapping)
    return pool


def oracle_attention(orc, wl: Workload, pool=None, rows=None, threads=None):
    """Oracle output for all rows (or the given row indices)."""
    if pool is None:
        pool = oracle_pool(orc, wl)
    q = wl.host["q"]
    rseq = np.asarray(wl.meta.row_seq)
    rkeys = np.asarray(wl.meta.row_num_keys)
    if rows is not None:
        q, rseq, rkeys = q[rows], rseq[rows], rkeys[rows]
    return pool.attention(q, wl.layer, wl.tables, rseq, rkeys, threads=threads)


def cfg2_context_lens(seed=2, num_seqs=64, lo=512, hi=4096):
    """context lengths uniform in [lo, hi]; the new token
    makes keys = ctx + 1."""
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, num_seqs)


def cfg3_context_lens(seed=3, num_seqs=8, hi=8192):
    """cached context uniform in [0, hi], 512 new rows each."""
    rng = np.random.default_rng(seed)
    return rng.integers(0, hi + 1, num_seqs)


def cfg4_attention_lens(seed=4, num_decode=256, median=1024, sigma=1.0, lo=128, hi=8192,
                        chunk_ctx=(0, 1536), chunk=512):
    """The attention part of BASELINE config 4's mixed step: 256 decode
    sequences with context lognormal (median 1024, sigma 1.0 -- BASELINE
    leaves sigma open) clipped to [128, 8192], plus two 512-row prefill
    chunks, one at the start of its prompt and one continuing a prompt whose
    first 1536 tokens are cached.  Returns (context_lens, num_new)."""
    rng = np.random.default_rng(seed)
    dec = np.clip(np.round(np.exp(np.log(median) + sigma * rng.standard_normal(num_decode))),
                  lo, hi).astype(np.int64)
    ctx = np.concatenate([dec, np.asarray(chunk_ctx, np.int64)])
    new = np.concatenate([np.ones(num_decode, np.int64), np.full(len(chunk_ctx), chunk, np.int64)])
    return ctx, new


def cfg5_context_lens(seed=5, num_seqs=64, prefix=4096, lo=256, hi=1024, long_ctx=32768):
    """64 sequences share a 4096-token prefix and add a
    suffix uniform in [256, 1024]; one more sequence at 32768 context."""
    rng = np.random.default_rng(seed)
    ctx = prefix + rng.integers(lo, hi + 1, num_seqs)
    return np.concatenate([ctx, [long_ctx]])


# ---- model configurations ----------------------------------------------------

class ModelCfg:
    """The ModelConfig fields (config.rs:9-34) with RopeScaling as a dict,
    plus head_dim (config.rs:74-76).  Host-only, for the oracle and tests."""

    def __init__(self, **kw):
        self.__dict__.update(kw)
        self.head_dim = self.hidden_size // self.num_attention_heads


def tiny_config():
    """testutil.rs:10-30: the reference's own test model."""
    return ModelCfg(hidden_size=48, intermediate_size=80, num_hidden_layers=2,
                    num_attention_heads=6, num_key_value_heads=2, vocab_size=37,
                    max_position_embeddings=256, rms_norm_eps=1e-5, rope_theta=10000.0,
                    rope_scaling=dict(factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                                      original_max_position_embeddings=64))


def cfg1_config():
    """the tiny Llama-style decoder (2 layers, hidden 256,
    4 q / 2 kv heads, head_dim 64, FFN 688, vocab 1024, eps 1e-5, theta
    10000).  Its rope_scaling block is the reference test model's
    (testutil.rs:21-26): the reference's config always carries one."""
    return ModelCfg(hidden_size=256, intermediate_size=688, num_hidden_layers=2,
                    num_attention_heads=4, num_key_value_heads=2, vocab_size=1024,
                    max_position_embeddings=256, rms_norm_eps=1e-5, rope_theta=10000.0,
                    rope_scaling=dict(factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                                      original_max_position_embeddings=64))


def llama3_8b_config(num_hidden_layers=32):
    """Llama-3-8B shape (32 layers, hidden 4096, 32 q / 8 kv
    heads, head_dim 128, FFN 14336, vocab 128256, theta 500000).  Llama 3 8B
    has no rope_scaling; factor 1 with the 1-4 bands leaves every frequency
    at its raw value up to the blend's rounding."""
    return ModelCfg(hidden_size=4096, intermediate_size=14336,
                    num_hidden_layers=num_hidden_layers, num_attention_heads=32,
                    num_key_value_heads=8, vocab_size=128256, max_position_embeddings=8192,
                    rms_norm_eps=1e-5, rope_theta=500000.0,
                    rope_scaling=dict(factor=1.0, low_freq_factor=1.0, high_freq_factor=4.0,
                                      original_max_position_embeddings=8192))


def normal_weights(cfg, seed, std=0.02):
    """BASELINE configs 1 and 4: weights ~ N(0, std) (f32 numpy, seeded),
    norm weights 1."""
    rng = np.random.default_rng(seed)
    h, hd = cfg.hidden_size, cfg.head_dim
    qd, kvd, f = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd, cfg.intermediate_size

    def m(o, i):
        return (rng.standard_normal((o, i), np.float32) * np.float32(std)).astype(np.float32)

    layers = [dict(attn_norm=np.ones(h, np.float32), wq=m(qd, h), wk=m(kvd, h), wv=m(kvd, h),
                   wo=m(h, qd), mlp_norm=np.ones(h, np.float32), w_gate=m(f, h), w_up=m(f, h),
                   w_down=m(h, f)) for _ in range(cfg.num_hidden_layers)]
    return dict(embed=m(cfg.vocab_size, h), layers=layers, final_norm=np.ones(h, np.float32))


def round_bf16(a):
    """f32 -> nearest bf16 (ties to even) -> f32, on the host."""
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def bf16_weights(w):
    """The same weights rounded to bf16 (what the GPU model holds), as f32."""
    return dict(embed=round_bf16(w["embed"]), final_norm=round_bf16(w["final_norm"]),
                layers=[{k: round_bf16(v) for k, v in L.items()} for L in w["layers"]])


def ref_prompt(n, seed):
    """model.rs:385-389: the reference's test prompts over a 37-token vocab."""
    return [(i * 7 + seed * 13 + 3) % 37 for i in range(n)]

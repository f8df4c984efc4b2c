"""CPU oracle for the paged-attention path -- TEST INFRASTRUCTURE ONLY.

numpy wrappers over ``oracle/build/libvo_oracle_v{3,4}.so`` (built from
``vo_oracle.c`` by ``oracle/Makefile``), the C restatement of the reference's
CPU backend and paged metadata (citations in vo_oracle.h / vo_oracle.c).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may
import this module, and only as the checker or the timed CPU baseline.  The
product library never calls it.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
from typing import List, Sequence, Tuple

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent


def _has_avx512() -> bool:
    try:
        flags = pathlib.Path("/proc/cpuinfo").read_text()
    except OSError:
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512dq", "avx512vl"))


VARIANT = "v4" if _has_avx512() else "v3"
LIB_PATH = _HERE / "build" / f"libvo_oracle_{VARIANT}.so"

_u64 = ctypes.c_uint64
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_f32p = ctypes.POINTER(ctypes.c_float)

OK = 0
BLOCK_TABLE_TOO_SHORT = 3
SLOT_OUT_OF_RANGE = 4
BLOCK_OUT_OF_RANGE = 5
NAN = 10


class Err(ctypes.Structure):
    _fields_ = [("seq", _u64), ("tokens", _u64), ("needed", _u64), ("have", _u64),
                ("value", _u64), ("limit", _u64)]


class OracleError(Exception):
    def __init__(self, code: int, err: Err):
        self.code = code
        self.seq, self.tokens, self.needed = int(err.seq), int(err.tokens), int(err.needed)
        self.have, self.value, self.limit = int(err.have), int(err.value), int(err.limit)
        super().__init__(f"oracle error {code}: seq {self.seq} tokens {self.tokens} "
                         f"needed {self.needed} have {self.have} value {self.value} "
                         f"limit {self.limit}")


def _load():
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
    h = ctypes.CDLL(str(LIB_PATH))
    sig = {
        "vo_oracle_rand_vec": (None, [_u64, _u64, _f32p]),
        "vo_oracle_max_rel_diff": (ctypes.c_float, [_f32p, _f32p, _u64]),
        "vo_oracle_slot_of": (ctypes.c_uint32, [_u32p, _u64, _u64]),
        "vo_oracle_check_covers": (ctypes.c_int, [_u64, _u64, _u64, ctypes.POINTER(Err)]),
        "vo_oracle_prefill_meta": (ctypes.c_int, [_u64, _u64p, _u64p, _u64p, _u32p, _u64,
                                                  _u64p, _u32p, _u32p, _u64p, _u64p,
                                                  ctypes.POINTER(Err)]),
        "vo_oracle_last_rows": (None, [_u64p, _u64, _u32p]),
        "vo_oracle_decode_meta": (ctypes.c_int, [_u64, _u64p, _u64p, _u32p, _u64, _u32p, _u32p,
                                                 _u64p, _u64p, ctypes.POINTER(Err)]),
        "vo_oracle_dot": (ctypes.c_float, [_f32p, _f32p, _u64]),
        "vo_oracle_write_kv": (ctypes.c_int, [_f32p, _f32p, _u64, _u64, _f32p, _f32p, _u32p,
                                              _u64, ctypes.POINTER(Err)]),
        "vo_oracle_check_block_tables": (ctypes.c_int, [_u64, _u64p, _u32p, _u64,
                                                        ctypes.POINTER(Err)]),
        "vo_oracle_paged_attention": (None, [_f32p, _f32p, _f32p, _f32p, _u64, _u64, _u64, _u64,
                                             _u64p, _u32p, _u64p, _u64p, _u64, ctypes.c_int]),
        "vo_oracle_naive_attend_f64": (None, [_f32p, _f32p, _f32p, _u64, _u64, _u64, _u64,
                                              _f32p]),
        "vo_oracle_splitk_combine": (None, [_u64, _u64, _f32p, _f32p, _f32p, _f32p]),
        "vo_oracle_rope_inv_freq": (None, [_u64, ctypes.c_double, ctypes.c_double,
                                           ctypes.c_double, ctypes.c_double, _u64, _f32p]),
        "vo_oracle_rope_table": (None, [_f32p, _u64, _u64, _f32p, _f32p]),
        "vo_oracle_rope_apply": (None, [_f32p, _u64, _u64, _u32p, _f32p, _f32p, _u64]),
        "vo_oracle_embed": (None, [_f32p, _u64, _u32p, _u64, _f32p]),
        "vo_oracle_rmsnorm": (None, [_f32p, _u64, _u64, _f32p, ctypes.c_float, _f32p]),
        "vo_oracle_matmul": (None, [_f32p, _u64, _u64, _f32p, _u64, _f32p, ctypes.c_int]),
        "vo_oracle_silu_mul": (None, [_f32p, _f32p, _u64]),
        "vo_oracle_add": (None, [_f32p, _f32p, _u64]),
        "vo_oracle_gather_rows": (None, [_f32p, _u64, _u32p, _u64, _f32p]),
        "vo_oracle_argmax": (ctypes.c_int, [_f32p, _u64, _u64, _u32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    return h


lib = _load()


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def _u64a(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint64))


def _pf(a):
    return a.ctypes.data_as(_f32p)


def _p32(a):
    return a.ctypes.data_as(_u32p)


def _p64(a):
    return a.ctypes.data_as(_u64p)


def csr(tables: Sequence[Sequence[int]]) -> Tuple[np.ndarray, np.ndarray]:
    off = np.zeros(len(tables) + 1, np.uint64)
    if len(tables):
        off[1:] = np.cumsum([len(t) for t in tables])
    flat = np.concatenate([_u32(t) for t in tables]) if len(tables) and off[-1] else np.zeros(1, np.uint32)
    return off, _u32(flat)


# ---- testutil.rs ----------------------------------------------------------

def rand_vec(seed: int, n: int) -> np.ndarray:
    out = np.zeros(max(n, 1), np.float32)
    lib.vo_oracle_rand_vec(seed, n, _pf(out))
    return out[:n]


def max_rel_diff(a, b) -> float:
    a, b = _f32(a).ravel(), _f32(b).ravel()
    assert a.shape == b.shape
    return float(lib.vo_oracle_max_rel_diff(_pf(a), _pf(b), a.size))


# ---- paged.rs -------------------------------------------------------------

def slot_of(table, pos: int, block_size: int) -> int:
    t = _u32(table)
    return int(lib.vo_oracle_slot_of(_p32(t), pos, block_size))


def prefill_meta(seqs: Sequence[Tuple[int, int, Sequence[int]]], block_size: int) -> dict:
    """seqs = [(context_len, num_new, table)] -> PrefillMeta fields."""
    ctx = _u64a([s[0] for s in seqs])
    new = _u64a([s[1] for s in seqs])
    off, flat = csr([s[2] for s in seqs])
    T = int(new.sum()) if len(seqs) else 0
    starts = np.zeros(len(seqs) + 1, np.uint64)
    pos = np.zeros(max(T, 1), np.uint32)
    slots = np.zeros(max(T, 1), np.uint32)
    rseq = np.zeros(max(T, 1), np.uint64)
    rkeys = np.zeros(max(T, 1), np.uint64)
    err = Err()
    rc = lib.vo_oracle_prefill_meta(len(seqs), _p64(ctx if len(seqs) else np.zeros(1, np.uint64)),
                                    _p64(new if len(seqs) else np.zeros(1, np.uint64)), _p64(off),
                                    _p32(flat), block_size, _p64(starts), _p32(pos), _p32(slots),
                                    _p64(rseq), _p64(rkeys), ctypes.byref(err))
    if rc != OK:
        raise OracleError(rc, err)
    last = np.zeros(max(len(seqs), 1), np.uint32)
    lib.vo_oracle_last_rows(_p64(starts), len(seqs), _p32(last))
    return dict(seq_row_starts=starts, positions=pos[:T], slot_mapping=slots[:T],
                row_seq=rseq[:T], row_num_keys=rkeys[:T], last_rows=last[:len(seqs)],
                table_off=off, tables=flat, context_lens=ctx)


def decode_meta(seqs: Sequence[Tuple[int, Sequence[int]]], block_size: int) -> dict:
    """seqs = [(context_len, table)] -> DecodeMeta fields."""
    n = len(seqs)
    ctx = _u64a([s[0] for s in seqs]) if n else np.zeros(1, np.uint64)
    off, flat = csr([s[1] for s in seqs])
    pos = np.zeros(max(n, 1), np.uint32)
    slots = np.zeros(max(n, 1), np.uint32)
    rseq = np.zeros(max(n, 1), np.uint64)
    rkeys = np.zeros(max(n, 1), np.uint64)
    err = Err()
    rc = lib.vo_oracle_decode_meta(n, _p64(ctx), _p64(off), _p32(flat), block_size, _p32(pos),
                                   _p32(slots), _p64(rseq), _p64(rkeys), ctypes.byref(err))
    if rc != OK:
        raise OracleError(rc, err)
    return dict(positions=pos[:n], slot_mapping=slots[:n], row_seq=rseq[:n],
                row_num_keys=rkeys[:n], table_off=off, tables=flat)


# ---- cpu/mod.rs, cpu/attention.rs -------------------------------------------

def dot(a, b) -> float:
    a, b = _f32(a), _f32(b)
    return float(lib.vo_oracle_dot(_pf(a), _pf(b), a.size))


class Pool:
    """CpuKvPool (cpu/mod.rs:31-37): f32 [layers][num_slots, kv_heads*head_dim]."""

    def __init__(self, num_layers, num_blocks, block_size, kv_heads, head_dim):
        self.num_layers, self.num_blocks, self.block_size = num_layers, num_blocks, block_size
        self.kv_heads, self.head_dim = kv_heads, head_dim
        self.num_slots = num_blocks * block_size
        w = kv_heads * head_dim
        self.keys = [np.zeros((self.num_slots, w), np.float32) for _ in range(num_layers)]
        self.values = [np.zeros((self.num_slots, w), np.float32) for _ in range(num_layers)]

    def write_kv(self, layer, keys, values, slots) -> None:
        k, v, s = _f32(keys), _f32(values), _u32(slots)
        err = Err()
        rc = lib.vo_oracle_write_kv(_pf(self.keys[layer]), _pf(self.values[layer]),
                                    self.num_slots, self.kv_heads * self.head_dim, _pf(k), _pf(v),
                                    _p32(s), len(s), ctypes.byref(err))
        if rc != OK:
            raise OracleError(rc, err)

    def check_block_tables(self, tables) -> None:
        off, flat = csr(tables)
        err = Err()
        rc = lib.vo_oracle_check_block_tables(len(tables), _p64(off), _p32(flat),
                                              self.num_blocks, ctypes.byref(err))
        if rc != OK:
            raise OracleError(rc, err)

    def attention(self, queries, layer, tables, row_seq, row_num_keys, threads=None):
        """prefill_attention / decode_attention (cpu/mod.rs:287-339)."""
        self.check_block_tables(tables)
        q = _f32(queries)
        rows = q.shape[0]
        out = np.zeros_like(q)
        off, flat = csr(tables)
        rs, rk = _u64a(row_seq), _u64a(row_num_keys)
        num_heads = q.shape[1] // self.head_dim
        if threads is None:
            threads = os.cpu_count() or 1
        lib.vo_oracle_paged_attention(_pf(q), _pf(out), _pf(self.keys[layer]),
                                      _pf(self.values[layer]), num_heads, self.kv_heads,
                                      self.head_dim, self.block_size, _p64(off), _p32(flat),
                                      _p64(rs if rows else np.zeros(1, np.uint64)),
                                      _p64(rk if rows else np.zeros(1, np.uint64)), rows,
                                      int(threads))
        return out


def paged_attention_raw(queries, pool_k, pool_v, num_kv_heads, head_dim, block_size, table_off,
                        tables, row_seq, row_num_keys, threads=None) -> np.ndarray:
    """attention.rs:44-128 on caller-owned arrays (pool_k/pool_v: [slots, kvh*hd] f32)."""
    q = _f32(queries)
    out = np.zeros_like(q)
    rows = q.shape[0]
    if threads is None:
        threads = os.cpu_count() or 1
    lib.vo_oracle_paged_attention(_pf(q), _pf(out), _pf(pool_k), _pf(pool_v),
                                  q.shape[1] // head_dim, num_kv_heads, head_dim, block_size,
                                  _p64(_u64a(table_off)), _p32(_u32(tables)),
                                  _p64(_u64a(row_seq)), _p64(_u64a(row_num_keys)), rows,
                                  int(threads))
    return out


def naive_attend_f64(q, seq_k, seq_v, pos, num_heads, num_kv_heads, head_dim) -> np.ndarray:
    """cpu/tests.rs:184-208."""
    q, k, v = _f32(q), _f32(seq_k), _f32(seq_v)
    out = np.zeros(num_heads * head_dim, np.float32)
    lib.vo_oracle_naive_attend_f64(_pf(q), _pf(k), _pf(v), pos, num_heads, num_kv_heads,
                                   head_dim, _pf(out))
    return out


def splitk_combine(m, l, acc) -> np.ndarray:
    m, l, acc = _f32(m), _f32(l), _f32(acc)
    hd = acc.shape[-1]
    out = np.zeros(hd, np.float32)
    lib.vo_oracle_splitk_combine(len(m), hd, _pf(m), _pf(l), _pf(acc), _pf(out))
    return out


# ---- cpu/rope.rs ------------------------------------------------------------

# config.rs:41-56 (LLAMA_3_2_1B) rope_scaling; BASELINE's models use theta
# 10000 (config 1) and 500000 (config 4) with the same scaling block.
LLAMA3_SCALING = dict(factor=32.0, low_freq_factor=1.0, high_freq_factor=4.0,
                      original_max_position_embeddings=8192)


def rope_inv_freq(head_dim: int, theta: float, factor=32.0, low_freq_factor=1.0,
                  high_freq_factor=4.0, original_max_position_embeddings=8192) -> np.ndarray:
    """rope.rs:36-60 (llama3_inv_freq)."""
    out = np.zeros(head_dim // 2, np.float32)
    lib.vo_oracle_rope_inv_freq(head_dim, theta, factor, low_freq_factor, high_freq_factor,
                                original_max_position_embeddings, _pf(out))
    return out


def rope_table(inv_freq, max_len: int):
    """rope.rs:62-84 (RopeTable::new): (cos, sin), each [max_len, half] f32."""
    inv = _f32(inv_freq)
    half = inv.size
    c = np.zeros((max_len, half), np.float32)
    sn = np.zeros((max_len, half), np.float32)
    lib.vo_oracle_rope_table(_pf(inv), half, max_len, _pf(c), _pf(sn))
    return c, sn


def rope_apply(x, positions, cos_tab, sin_tab) -> np.ndarray:
    """rope.rs:86-100 (RopeTable::apply) on every row of x [rows, cols]; a copy."""
    x = _f32(x).copy()
    pos = _u32(positions)
    c, sn = _f32(cos_tab), _f32(sin_tab)
    lib.vo_oracle_rope_apply(_pf(x), x.shape[0], x.shape[1], _p32(pos), _pf(c), _pf(sn),
                             c.shape[1])
    return x


# ---- cpu/mod.rs: the layer around attention -----------------------------------

def embed(table, tokens) -> np.ndarray:
    """cpu/mod.rs:172-180."""
    t, ids = _f32(table), _u32(tokens)
    out = np.zeros((len(ids), t.shape[1]), np.float32)
    if len(ids):
        lib.vo_oracle_embed(_pf(t), t.shape[1], _p32(ids), len(ids), _pf(out))
    return out


def rmsnorm(x, w, eps: float) -> np.ndarray:
    """cpu/mod.rs:182-197."""
    x, w = _f32(x), _f32(w)
    out = np.zeros_like(x)
    if x.size:
        lib.vo_oracle_rmsnorm(_pf(x), x.shape[0], x.shape[1], _pf(w), eps, _pf(out))
    return out


def matmul(x, w, threads=None) -> np.ndarray:
    """cpu/mod.rs:199-229: x [rows, in] . w[out, in]^T, each element the 16-lane dot."""
    x, w = _f32(x), _f32(w)
    out = np.zeros((x.shape[0], w.shape[0]), np.float32)
    if threads is None:
        threads = min(os.cpu_count() or 1, 64)
    if out.size:
        lib.vo_oracle_matmul(_pf(x), x.shape[0], x.shape[1], _pf(w), w.shape[0], _pf(out),
                             int(threads))
    return out


def silu_mul(gate, up) -> np.ndarray:
    """cpu/mod.rs:341-349, on a copy of gate."""
    g, u = _f32(gate).copy(), _f32(up)
    lib.vo_oracle_silu_mul(_pf(g), _pf(u), g.size)
    return g


def add(total, x) -> np.ndarray:
    """cpu/mod.rs:351-358, on a copy of total."""
    s, v = _f32(total).copy(), _f32(x)
    lib.vo_oracle_add(_pf(s), _pf(v), s.size)
    return s


def gather_rows(x, rows) -> np.ndarray:
    """cpu/mod.rs:360-368."""
    x, r = _f32(x), _u32(rows)
    out = np.zeros((len(r), x.shape[1]), np.float32)
    if len(r):
        lib.vo_oracle_gather_rows(_pf(x), x.shape[1], _p32(r), len(r), _pf(out))
    return out


def argmax(x) -> np.ndarray:
    """cpu/mod.rs:370-388; raises OracleError(NAN) on a NaN."""
    x = _f32(x)
    out = np.zeros(max(x.shape[0], 1), np.uint32)
    rc = lib.vo_oracle_argmax(_pf(x), x.shape[0], x.shape[1], _p32(out))
    if rc != OK:
        raise OracleError(rc, Err())
    return out[:x.shape[0] if x.shape[1] else 0]


# ---- testutil.rs: random_weights ------------------------------------------------

def rand_weight(seed: int, shape, scale: float) -> np.ndarray:
    """testutil.rs:46-53: rand_vec(seed, n) * scale, in f32."""
    n = int(np.prod(shape))
    return (rand_vec(seed, n) * np.float32(scale)).astype(np.float32).reshape(shape)


def random_weights(cfg, seed: int) -> dict:
    """testutil.rs:57-91: matrices ~U[-1,1)/sqrt(in), norms 1 + 0.1 U[-1,1).
    ``cfg`` has the ModelConfig fields (config.rs:9-22) and ``head_dim``."""
    h, hd = cfg.hidden_size, cfg.head_dim
    qd, kvd, ffn = cfg.num_attention_heads * hd, cfg.num_key_value_heads * hd, cfg.intermediate_size

    def m(s, o, i):
        return rand_weight(seed * 1000 + s, (o, i), np.float32(1.0) / np.sqrt(np.float32(i)))

    def norm(s):
        return (np.float32(1.0) + np.float32(0.1) * rand_vec(seed * 1000 + s, h)).astype(np.float32)

    layers = []
    for l in range(cfg.num_hidden_layers):
        b = 10 + l * 10
        layers.append(dict(attn_norm=norm(b), wq=m(b + 1, qd, h), wk=m(b + 2, kvd, h),
                           wv=m(b + 3, kvd, h), wo=m(b + 4, h, qd), mlp_norm=norm(b + 5),
                           w_gate=m(b + 6, ffn, h), w_up=m(b + 7, ffn, h),
                           w_down=m(b + 8, h, ffn)))
    return dict(embed=rand_weight(seed * 1000, (cfg.vocab_size, h), 1.0), layers=layers,
                final_norm=norm(999))


# ---- model.rs: Llama::forward ------------------------------------------------------

class Llama:
    """Llama<CpuBackend> (model.rs:269-356) on the oracle's ops: f32 weights
    (dict as random_weights returns), f32 KV pool, RoPE table of max_len rows
    (CpuBackend::new builds it for max_model_len, cpu/mod.rs:53)."""

    def __init__(self, cfg, weights: dict, num_blocks: int, block_size: int, max_len: int,
                 threads=None):
        self.cfg, self.w, self.threads = cfg, weights, threads
        hd = cfg.head_dim
        self.pool = Pool(cfg.num_hidden_layers, num_blocks, block_size,
                         cfg.num_key_value_heads, hd)
        inv = rope_inv_freq(hd, cfg.rope_theta, **cfg.rope_scaling)
        self.cos, self.sin = rope_table(inv, max_len)

    def forward(self, tokens, positions, slots, tables, row_seq, row_num_keys, last_rows=None):
        """One step.  ``last_rows`` None: decode (every row feeds the LM head).
        Returns (next token ids, logits [S, vocab])."""
        cfg, W = self.cfg, self.w
        eps = np.float32(cfg.rms_norm_eps)
        hd = cfg.head_dim
        residual = embed(W["embed"], tokens)
        for li, L in enumerate(W["layers"]):
            normed = rmsnorm(residual, L["attn_norm"], eps)
            q = matmul(normed, L["wq"], self.threads)
            k = matmul(normed, L["wk"], self.threads)
            v = matmul(normed, L["wv"], self.threads)
            q = rope_apply(q, positions, self.cos, self.sin)
            k = rope_apply(k, positions, self.cos, self.sin)
            self.pool.write_kv(li, k, v, slots)
            attn = self.pool.attention(q, li, tables, row_seq, row_num_keys, self.threads)
            residual = add(residual, matmul(attn, L["wo"], self.threads))
            normed = rmsnorm(residual, L["mlp_norm"], eps)
            gate = matmul(normed, L["w_gate"], self.threads)
            up = matmul(normed, L["w_up"], self.threads)
            residual = add(residual, matmul(silu_mul(gate, up), L["w_down"], self.threads))
        last = residual if last_rows is None else gather_rows(residual, last_rows)
        normed = rmsnorm(last, W["final_norm"], eps)
        logits = matmul(normed, W["embed"], self.threads)
        return argmax(logits), logits

    def prefill(self, tokens, seqs, block_size: int):
        """seqs = [(context_len, num_new, table)] (PrefillSeq, paged.rs:84-92)."""
        m = prefill_meta(seqs, block_size)
        return self.forward(tokens, m["positions"], m["slot_mapping"], [s[2] for s in seqs],
                            m["row_seq"], m["row_num_keys"], m["last_rows"])

    def decode(self, tokens, seqs, block_size: int):
        """seqs = [(context_len, table)] (DecodeSeq, paged.rs:164-168)."""
        m = decode_meta(seqs, block_size)
        return self.forward(tokens, m["positions"], m["slot_mapping"], [s[1] for s in seqs],
                            m["row_seq"], m["row_num_keys"], None)

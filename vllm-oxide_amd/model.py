"""Llama forward (crates/engine/src/model.rs:269-356) on the HIP backend.

``Llama`` mirrors the reference's ``Llama<B>``: a config (config.rs:9-34),
weights uploaded once, activation buffers sized once for ``max_batch_tokens``
rows and ``max_seqs`` sequences (the reference's arena, model.rs:81-90; no
allocation in the hot loop), and ``prefill`` / ``decode`` with the
reference's batch checks (model.rs:245-267) and op order:

    residual = embed(tokens)                                  (f32)
    per layer:
      normed = rmsnorm(residual, attn_norm)                   (bf16)
      qkv    = matmul(normed, [wq; wk; wv])                   one GEMM
      rope(q), rope(k), write_kv(k, v)                        one launch
      attn   = prefill_attention / decode_attention(q)
      residual += matmul(attn, wo)                            GEMM epilogue add
      normed = rmsnorm(residual, mlp_norm)
      gu     = matmul(normed, [w_gate; w_up])                 one GEMM
      act    = silu(gate) * up
      residual += matmul(act, w_down)                         GEMM epilogue add
    normed = rmsnorm(gather_rows(residual, last_rows), final_norm)  one pass
    logits = matmul(normed, embed)                            (f32, tied)
    tokens = argmax(logits)                                   the one sync

Every op is a call into libvo_paged_attention.so on the caller's (torch's
current) stream; there is no other compute path.  Weights and activations
are bf16 on the device, the residual stream and the logits f32.  q/k/v and
gate/up are concatenated row-wise at upload so that each pair or triple is
one GEMM over the same input; the attention output projection and the down
projection add into the residual inside the GEMM (beta = 1).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

from . import (VO_DTYPE_BF16, VO_DTYPE_F32, CapacityError, DecodeMeta, HipBackend, KvLayout,
               KvPool, PrefillMeta, RopeTable, ShapeError, _check, _engine_error, _stream_ptr,
               _vp, lib, VO_ERR_CAPACITY, VO_ERR_SHAPE)


@dataclass(frozen=True)
class ModelConfig:
    """config.rs:9-34 (ModelConfig with its RopeScaling block flattened)."""
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    vocab_size: int
    max_position_embeddings: int
    rms_norm_eps: float
    rope_theta: float
    rope_scaling: dict = field(default_factory=lambda: dict(
        factor=32.0, low_freq_factor=1.0, high_freq_factor=4.0,
        original_max_position_embeddings=8192))

    @property
    def head_dim(self) -> int:
        """config.rs:74-76."""
        return self.hidden_size // self.num_attention_heads

    def kv_bytes_per_token(self, dtype_bytes: int = 2) -> int:
        """config.rs:99-101 at the pool's element size (bf16 here)."""
        return (2 * self.num_hidden_layers * self.num_key_value_heads * self.head_dim
                * dtype_bytes)


@dataclass(frozen=True)
class EngineConfig:
    """model.rs:38-54 (num_blocks stands for kv_pool_bytes, model.rs:201-212)."""
    max_batch_tokens: int = 2048
    max_seqs: int = 32
    max_model_len: int = 8192
    block_size: int = 16
    num_blocks: int = 2048


@dataclass
class StepOutput:
    """model.rs:113-118: the next token of every sequence, logits on request."""
    tokens: List[int]
    logits: Optional[np.ndarray] = None


def _ptr(t) -> _vp:
    return _vp(t.data_ptr())


class Llama:
    """Llama<HipBackend>.  ``weights`` is the reference's ModelWeights as a
    dict of float arrays (numpy or torch): embed [vocab, hidden], layers
    [{attn_norm, wq, wk, wv, wo, mlp_norm, w_gate, w_up, w_down}], final_norm
    (testutil.rs:57-91 field names); they are rounded to bf16 on upload."""

    def __init__(self, backend: HipBackend, config: ModelConfig, engine: EngineConfig,
                 weights: dict, gemm_workspace: int = 128 << 20):
        import torch
        self.backend, self.config, self.engine = backend, config, engine
        self.dev = torch.device(f"cuda:{backend.device}")
        c = config
        hd = c.head_dim
        self.qd, self.kvd = c.num_attention_heads * hd, c.num_key_value_heads * hd
        self.ffn = c.intermediate_size

        def up(a):
            if isinstance(a, torch.Tensor):
                return a.to(device=self.dev, dtype=torch.bfloat16).contiguous()
            return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(
                device=self.dev, dtype=torch.bfloat16).contiguous()

        def cat(*xs):
            return torch.cat([up(x) for x in xs], dim=0).contiguous()

        self.embed = up(weights["embed"])
        self.final_norm = up(weights["final_norm"])
        self.layers = []
        for L in weights["layers"]:
            self.layers.append(dict(
                attn_norm=up(L["attn_norm"]), wqkv=cat(L["wq"], L["wk"], L["wv"]),
                wo=up(L["wo"]), mlp_norm=up(L["mlp_norm"]), wgu=cat(L["w_gate"], L["w_up"]),
                wd=up(L["w_down"])))
        if len(self.layers) != c.num_hidden_layers:
            raise ValueError("weights have a different layer count than the config")
        self.rope = RopeTable(hd, c.rope_theta, engine.max_model_len, backend.device,
                              **c.rope_scaling)
        self._workspace = gemm_workspace
        self.lanes = [_Lane(self, engine.max_batch_tokens, engine.max_seqs)]
        lane = self.lanes[0]
        self.gemm = lane.gemm
        self.logits, self.ids, self.ids_host = lane.logits, lane.ids, lane.ids_host

    def kv_layout(self) -> KvLayout:
        """model.rs:201-212, with the engine's block count."""
        c = self.config
        return KvLayout(c.num_hidden_layers, self.engine.num_blocks, self.engine.block_size,
                        c.num_key_value_heads, c.head_dim)

    def alloc_kv_pool(self) -> KvPool:
        """model.rs:214-217."""
        return self.backend.alloc_kv_pool(self.kv_layout())

    def close(self) -> None:
        for lane in getattr(self, "lanes", []):
            lane.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # model.rs:221-243
    def prefill(self, pool: KvPool, tokens: Sequence[int], meta: PrefillMeta,
                want_logits: bool = False, stream=None) -> StepOutput:
        self._check_batch(len(tokens), meta.num_rows(), meta.num_seqs())
        return self._forward(pool, tokens, meta, True, want_logits, stream)

    def decode(self, pool: KvPool, tokens: Sequence[int], meta: DecodeMeta,
               want_logits: bool = False, stream=None) -> StepOutput:
        self._check_batch(len(tokens), meta.num_seqs(), meta.num_seqs())
        return self._forward(pool, tokens, meta, False, want_logits, stream)

    def _check_batch(self, tokens: int, meta_rows: int, sequences: int) -> None:
        """model.rs:245-267."""
        if tokens != meta_rows:
            raise _engine_error(ShapeError, VO_ERR_SHAPE, "forward",
                                f"forward: {tokens} tokens, metadata describes {meta_rows}")
        if tokens > self.engine.max_batch_tokens:
            raise _engine_error(CapacityError, VO_ERR_CAPACITY, "tokens per step",
                                f"tokens per step: need {tokens}, "
                                f"limit {self.engine.max_batch_tokens}",
                                value=tokens, limit=self.engine.max_batch_tokens)
        if sequences > self.engine.max_seqs:
            raise _engine_error(CapacityError, VO_ERR_CAPACITY, "sequences per step",
                                f"sequences per step: need {sequences}, "
                                f"limit {self.engine.max_seqs}",
                                value=sequences, limit=self.engine.max_seqs)

    def _forward(self, pool: KvPool, tokens, meta, prefill: bool, want_logits: bool, stream):
        self.enqueue(pool, tokens, meta, prefill, stream)
        return self.finish(meta.num_seqs(), want_logits, stream)

    def enqueue(self, pool: KvPool, tokens, meta, prefill: bool, stream=None) -> None:
        """Everything of one step up to the logits, enqueued without a wait."""
        m = self.backend._meta_for(pool, meta, stream)
        m.upload_tokens(tokens, stream)
        self._launch(pool, m, len(tokens), meta.num_seqs(), prefill, stream)

    def _launch(self, pool: KvPool, m, T: int, S: int, prefill: bool, stream=None,
                lane=None) -> None:
        """The step's device work, from the embedding to the logits, for the
        metadata and tokens already uploaded into ``m``, in ``lane``'s buffers
        (default: the model's own)."""
        c = self.config
        B = self.lanes[0] if lane is None else lane
        s = _stream_ptr(stream)
        H, V, hd = c.hidden_size, c.vocab_size, c.head_dim
        qd, kvd, F = self.qd, self.kvd, self.ffn
        eps = float(c.rms_norm_eps)
        mh = m.handle
        res, nrm, qkv, q, attn = (_ptr(B.residual), _ptr(B.normed), _ptr(B.qkv), _ptr(B.q),
                                  _ptr(B.attn))
        gu, act = _ptr(B.gu), _ptr(B.act)
        g = B.gemm
        bf, f32 = VO_DTYPE_BF16, VO_DTYPE_F32
        fused = pool.layout.block_size == 16 and hd in (64, 128)
        attention = lib.vo_prefill_attention if prefill else lib.vo_decode_attention
        _check(lib.vo_embed(_ptr(self.embed), V, H, mh, T, res, s))
        for li, L in enumerate(self.layers):
            _check(lib.vo_rmsnorm(res, T, H, _ptr(L["attn_norm"]), H, eps, nrm, s))
            _check(lib.vo_matmul(g, nrm, T, H, _ptr(L["wqkv"]), qd + 2 * kvd, H, qkv, bf, 0, s))
            if fused:
                _check(lib.vo_qkv_rope_write_kv(pool.handle, li, self.rope.handle, qkv, T, qd,
                                                kvd, mh, q, s))
            else:
                self._rope_write_unfused(pool, li, T, m, stream, B)
            _check(attention(q, T, qd, pool.handle, li, mh, attn, s))
            _check(lib.vo_matmul(g, attn, T, qd, _ptr(L["wo"]), H, qd, res, f32, 1, s))
            _check(lib.vo_rmsnorm(res, T, H, _ptr(L["mlp_norm"]), H, eps, nrm, s))
            _check(lib.vo_matmul(g, nrm, T, H, _ptr(L["wgu"]), 2 * F, H, gu, bf, 0, s))
            gu_up = _vp(B.gu.data_ptr() + F * 2)
            _check(lib.vo_silu_mul(gu, 2 * F, gu_up, 2 * F, T, F, act, F, s))
            _check(lib.vo_matmul(g, act, T, F, _ptr(L["wd"]), H, F, res, f32, 1, s))
        _check(lib.vo_rmsnorm_last_rows(res, T, H, _ptr(self.final_norm), H, eps, mh,
                                        _ptr(B.last), s))
        _check(lib.vo_matmul(g, _ptr(B.last), S, H, _ptr(self.embed), V, H,
                             _ptr(B.logits), f32, 0, s))

    # -- decode steps as a HIP graph ---------------------------------------
    def capture_decode(self, pool: KvPool, tokens, meta: DecodeMeta, work_headroom=None,
                       entry_headroom=None) -> "DecodeGraph":
        """Records the decode step of ``meta``'s sequences (the same count for
        every later step) as a HIP graph: the metadata is fixed to stable device
        addresses and capacity-sized launches (vo_step_meta_fix_launch), one
        eager step builds every GEMM plan, then the device work of a step --
        embed to argmax into a device buffer -- is recorded.  Replays upload the
        new step's metadata and tokens, replay, and copy the ids back."""
        import torch
        S = meta.num_seqs()
        self._check_batch(len(tokens), S, S)
        m = self.backend.step_meta(pool)
        m.unfix_launch()
        m.upload(meta)
        m.fix_launch(S if work_headroom is None else work_headroom,
                     4 * S + 64 if entry_headroom is None else entry_headroom)
        m.holds = meta
        m.upload_tokens(tokens)
        self._launch(pool, m, S, S, False)
        self._argmax_device(S)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._launch(pool, m, S, S, False)
            self._argmax_device(S)
        return DecodeGraph(self, pool, m, graph, S)

    def _argmax_device(self, S: int, stream=None) -> None:
        _check(lib.vo_argmax(_ptr(self.logits), VO_DTYPE_F32, S, self.config.vocab_size,
                             ctypes.cast(ctypes.c_void_p(self.ids.data_ptr()),
                                         ctypes.POINTER(ctypes.c_uint32)), None,
                             _stream_ptr(stream)))

    def finish(self, num_seqs: int, want_logits: bool, stream=None) -> StepOutput:
        """argmax (the step's one device-to-host wait) and the logits on request."""
        s = _stream_ptr(stream)
        V = self.config.vocab_size
        ids_host = ctypes.cast(ctypes.c_void_p(self.ids_host.data_ptr()),
                               ctypes.POINTER(ctypes.c_uint32))
        _check(lib.vo_argmax(_ptr(self.logits), VO_DTYPE_F32, num_seqs, V,
                             ctypes.cast(ctypes.c_void_p(self.ids.data_ptr()),
                                         ctypes.POINTER(ctypes.c_uint32)), ids_host, s))
        toks = [int(x) for x in self.ids_host[:num_seqs].tolist()]
        logits = self.logits[:num_seqs].cpu().numpy().copy() if want_logits else None
        return StepOutput(toks, logits)

    def _rope_write_unfused(self, pool: KvPool, li: int, T: int, m, stream, L) -> None:
        """Shapes the fused launch does not cover (the reference's tiny test
        model: head_dim 8, block size 4): rope(q), rope(k), write_kv(k, v) as
        three calls on contiguous copies of the q/k/v column blocks."""
        qd, kvd, hd = self.qd, self.kvd, self.config.head_dim
        s = _stream_ptr(stream)
        L.q[:T].copy_(L.qkv[:T, :qd])
        k = L.qkv[:T, qd:qd + kvd].contiguous()
        v = L.qkv[:T, qd + kvd:].contiguous()
        _check(lib.vo_rope(self.rope.handle, _ptr(L.q), T, qd, hd, m.handle, s))
        _check(lib.vo_rope(self.rope.handle, _ptr(k), T, kvd, hd, m.handle, s))
        _check(lib.vo_write_kv(pool.handle, li, _ptr(k), _ptr(v), T, kvd, m.handle, s))


class DecodeGraph:
    """A recorded decode step (Llama.capture_decode) for a fixed number of
    sequences.  ``run`` serves any later decode step of those sequences whose
    metadata fits the fixed capacities; otherwise the upload raises
    ShapeError / CapacityError and the step must be recorded again."""

    def __init__(self, model: Llama, pool: KvPool, meta_holder, graph, num_seqs: int):
        self.model, self.pool, self.m, self.graph, self.num_seqs = (model, pool, meta_holder,
                                                                   graph, num_seqs)

    def run(self, tokens: Sequence[int], meta: DecodeMeta, want_logits: bool = False) -> StepOutput:
        """Llama::decode (model.rs:234-243) by replaying the recorded launches."""
        import torch
        from . import NaNError, VO_ERR_NAN
        model, S = self.model, self.num_seqs
        model._check_batch(len(tokens), meta.num_seqs(), meta.num_seqs())
        if meta.num_seqs() != S:
            raise _engine_error(ShapeError, VO_ERR_SHAPE, "decode",
                                f"decode: graph recorded for {S} sequences, step has "
                                f"{meta.num_seqs()}")
        if self.m.holds is not meta:
            self.m.upload(meta)
            self.m.holds = meta
        self.m.upload_tokens(tokens)
        self.graph.replay()
        model.ids_host[:S].copy_(model.ids[:S])
        torch.cuda.current_stream().synchronize()
        ids = model.ids_host[:S].tolist()
        if any(i == -1 for i in ids):  # 0xffffffff: a row with a NaN
            raise _engine_error(NaNError, VO_ERR_NAN, "argmax", "argmax: NaN in input")
        logits = model.logits[:S].cpu().numpy().copy() if want_logits else None
        return StepOutput([int(i) for i in ids], logits)


class _Lane:
    """Activation buffers and a GEMM handle (with its hipBLASLt workspace) for
    the steps of one stream, allocated once for max_batch_tokens rows and
    max_seqs sequences."""

    def __init__(self, model: Llama, T: int, S: int):
        import torch
        c, dev = model.config, model.dev
        H = c.hidden_size
        bf, f32 = torch.bfloat16, torch.float32
        self.gemm = _vp()
        _check(lib.vo_gemm_create(model.backend.device, model._workspace, ctypes.byref(self.gemm)))
        self.residual = torch.empty((T, H), dtype=f32, device=dev)
        self.normed = torch.empty((T, H), dtype=bf, device=dev)
        self.qkv = torch.empty((T, model.qd + 2 * model.kvd), dtype=bf, device=dev)
        self.q = torch.empty((T, model.qd), dtype=bf, device=dev)
        self.attn = torch.empty((T, model.qd), dtype=bf, device=dev)
        self.gu = torch.empty((T, 2 * model.ffn), dtype=bf, device=dev)
        self.act = torch.empty((T, model.ffn), dtype=bf, device=dev)
        self.last = torch.empty((S, H), dtype=bf, device=dev)
        self.logits = torch.empty((S, c.vocab_size), dtype=f32, device=dev)
        self.ids = torch.empty((S,), dtype=torch.int32, device=dev)
        self.ids_host = torch.empty((S,), dtype=torch.int32, pin_memory=True)

    def close(self) -> None:
        if self.gemm:
            lib.vo_gemm_destroy(self.gemm)
            self.gemm = _vp()

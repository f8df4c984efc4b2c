"""vllm-oxide paged attention for MI355X (gfx950).

Python view of ``libvo_paged_attention.so`` (C ABI in
``include/vo_paged_attention.h``).  The names and argument meanings mirror the
reference engine's Rust interface:

* ``KvLayout``, ``slot_of``, ``PrefillSeq``/``PrefillMeta.new``,
  ``DecodeSeq``/``DecodeMeta.new``, ``last_rows`` --
  crates/engine/src/backend/paged.rs:25-209
* ``HipBackend.alloc_kv_pool``, ``kv_layout``, ``write_kv``,
  ``prefill_attention``, ``decode_attention``, ``read_kv`` --
  the attention-path ops of ``trait Backend``,
  crates/engine/src/backend/mod.rs:61-182
* ``EngineError`` and its subclasses -- crates/engine/src/error.rs:8-56

All compute runs in the HIP library.  Importing this package loads the
library and raises ``ImportError`` when it is missing; there is no CPU path.
torch is used only for device memory and streams.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import weakref
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

__all__ = [
    "LIB_PATH", "lib", "KvLayout", "slot_of", "PrefillSeq", "PrefillMeta", "DecodeSeq",
    "DecodeMeta", "EngineError", "ShapeError", "CapacityError", "BlockTableTooShort",
    "SlotOutOfRange", "BlockOutOfRange", "DeviceError", "InvalidArgument", "Unsupported",
    "HipBackend", "KvPool", "StepMeta", "Workspace", "Weight", "Region", "OutsideWorkspace",
]

_HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = pathlib.Path(os.environ.get("VO_LIB_PATH", _HERE / "libvo_paged_attention.so"))

# ---------------------------------------------------------------------------
# C ABI
# ---------------------------------------------------------------------------
VO_OK = 0
VO_ERR_SHAPE = 1
VO_ERR_CAPACITY = 2
VO_ERR_BLOCK_TABLE_TOO_SHORT = 3
VO_ERR_SLOT_OUT_OF_RANGE = 4
VO_ERR_BLOCK_OUT_OF_RANGE = 5
VO_ERR_DEVICE = 6
VO_ERR_INVALID_ARGUMENT = 7
VO_ERR_UNSUPPORTED = 8
VO_ERR_POSITION_OUT_OF_RANGE = 9
VO_ERR_NAN = 10
VO_ERR_OUTSIDE_WORKSPACE = 11
VO_DTYPE_BF16 = 0
VO_DTYPE_F32 = 1

_u64 = ctypes.c_uint64
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_vp = ctypes.c_void_p


class vo_error_info(ctypes.Structure):
    _fields_ = [
        ("status", ctypes.c_int32), ("op", ctypes.c_char * 48), ("seq", _u64),
        ("tokens", _u64), ("needed", _u64), ("have", _u64), ("value", _u64),
        ("limit", _u64), ("message", ctypes.c_char * 256),
    ]


class vo_kv_layout(ctypes.Structure):
    _fields_ = [("num_layers", _u64), ("num_blocks", _u64), ("block_size", _u64),
                ("kv_heads", _u64), ("head_dim", _u64)]


class vo_kernel_stat(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("calls", _u64), ("total_ms", ctypes.c_double),
                ("min_ms", ctypes.c_double), ("max_ms", ctypes.c_double)]


class vo_rope_config(ctypes.Structure):
    _fields_ = [("head_dim", _u64), ("rope_theta", ctypes.c_double), ("factor", ctypes.c_double),
                ("low_freq_factor", ctypes.c_double), ("high_freq_factor", ctypes.c_double),
                ("original_max_position_embeddings", _u64)]


class vo_bm_stats(ctypes.Structure):
    _fields_ = [("hit_blocks", _u64), ("lookup_blocks", _u64), ("evictions", _u64),
                ("copies", _u64), ("free_blocks", _u64), ("cached_idle_blocks", _u64),
                ("sequences", _u64)]


class vo_prefill_seq(ctypes.Structure):
    _fields_ = [("context_len", _u64), ("num_new", _u64), ("block_table", _u32p),
                ("block_table_len", _u64)]


class vo_decode_seq(ctypes.Structure):
    _fields_ = [("context_len", _u64), ("block_table", _u32p), ("block_table_len", _u64)]


# Every exported symbol of the C ABI with its ctypes signature.
SIGNATURES = {
    "vo_last_error": (ctypes.c_int32, [ctypes.POINTER(vo_error_info)]),
    "vo_status_name": (ctypes.c_char_p, [ctypes.c_int32]),
    "vo_version": (ctypes.c_char_p, []),
    "vo_kv_layout_num_slots": (_u64, [ctypes.POINTER(vo_kv_layout)]),
    "vo_kv_layout_layer_elems": (_u64, [ctypes.POINTER(vo_kv_layout)]),
    "vo_slot_of": (ctypes.c_int32, [_u32p, _u64, _u64, _u64, _u32p]),
    "vo_prefill_meta_build": (ctypes.c_int32, [ctypes.POINTER(vo_prefill_seq), _u64, _u64,
                                               _u64p, _u32p, _u32p, _u64p, _u64p]),
    "vo_decode_meta_build": (ctypes.c_int32, [ctypes.POINTER(vo_decode_seq), _u64, _u64,
                                              _u32p, _u32p, _u64p, _u64p]),
    "vo_last_rows": (ctypes.c_int32, [_u64p, _u64, _u32p]),
    "vo_kv_pool_create": (ctypes.c_int32, [ctypes.POINTER(vo_kv_layout), ctypes.c_int32,
                                           ctypes.POINTER(_vp)]),
    "vo_kv_pool_destroy": (None, [_vp]),
    "vo_kv_pool_layout": (ctypes.c_int32, [_vp, ctypes.POINTER(vo_kv_layout)]),
    "vo_kv_pool_bytes": (_u64, [_vp]),
    "vo_step_meta_create": (ctypes.c_int32, [_vp, _u64, _u64, _u64, _u64, ctypes.POINTER(_vp)]),
    "vo_step_meta_destroy": (None, [_vp]),
    "vo_step_meta_upload_prefill": (ctypes.c_int32, [_vp, _u64, _u64, _u64p, _u32p, _u64p,
                                                     _u64p, _u64, _u32p, _u32p, _u64p, _u64p,
                                                     _vp]),
    "vo_step_meta_upload_decode": (ctypes.c_int32, [_vp, _u64, _u64, _u64p, _u32p, _u32p,
                                                    _u32p, _u64p, _u64p, _vp]),
    "vo_step_meta_upload_slots": (ctypes.c_int32, [_vp, _u32p, _u64, _vp]),
    "vo_step_meta_sync_prefill": (ctypes.c_int32, [_vp, _u64, _u64, _u64p, _u32p, _u64p,
                                                   _u64p, _u64, _u32p, _u32p, _u64p, _u64p,
                                                   _vp]),
    "vo_step_meta_sync_decode": (ctypes.c_int32, [_vp, _u64, _u64, _u64p, _u32p, _u32p,
                                                  _u32p, _u64p, _u64p, _vp]),
    "vo_write_kv": (ctypes.c_int32, [_vp, _u64, _vp, _vp, _u64, _u64, _vp, _vp]),
    "vo_write_kv_slots": (ctypes.c_int32, [_vp, _u64, _vp, _vp, _u64, _u64, _u32p, _u64, _vp,
                                           _vp]),
    "vo_prefill_attention": (ctypes.c_int32, [_vp, _u64, _u64, _vp, _u64, _vp, _vp, _vp]),
    "vo_decode_attention": (ctypes.c_int32, [_vp, _u64, _u64, _vp, _u64, _vp, _vp, _vp]),
    "vo_decode_attention_static": (ctypes.c_int32, [_vp, _u64, _u64, _vp, _u64, _vp, _vp, _u64,
                                                    _vp, _u64, _vp, _vp, _vp]),
    "vo_gather_kv": (ctypes.c_int32, [_vp, _u64, _vp, _u64, _u64, _vp, _vp, _vp]),
    "vo_prefill_meta_build_device": (ctypes.c_int32, [_vp, _vp, _vp, _vp, _u64, _u64, _u64,
                                                      _vp, _vp, _vp, _vp, _vp, _vp]),
    "vo_bm_create": (ctypes.c_int32, [_u64, _u64, ctypes.c_int32, ctypes.POINTER(_vp)]),
    "vo_bm_destroy": (None, [_vp]),
    "vo_bm_test_unchained_hash": (ctypes.c_int32, [_vp, ctypes.c_int32]),
    "vo_bm_add_sequence": (ctypes.c_int32, [_vp, _u64, _u32p, _u64, _u64p]),
    "vo_bm_append_token": (ctypes.c_int32, [_vp, _u64, ctypes.c_uint32, _u32p, _u32p, _u32p]),
    "vo_bm_fork": (ctypes.c_int32, [_vp, _u64, _u64]),
    "vo_bm_free_sequence": (ctypes.c_int32, [_vp, _u64]),
    "vo_bm_block_table": (ctypes.c_int32, [_vp, _u64, _u32p, _u64, _u64p, _u64p]),
    "vo_bm_num_available": (_u64, [_vp]),
    "vo_bm_get_stats": (ctypes.c_int32, [_vp, ctypes.POINTER(vo_bm_stats)]),
    "vo_bm_check_invariants": (ctypes.c_int32, [_vp]),
    "vo_kv_copy_blocks": (ctypes.c_int32, [_vp, _u32p, _u32p, _u64, _vp]),
    "vo_rope_table_create": (ctypes.c_int32, [ctypes.POINTER(vo_rope_config), _u64,
                                              ctypes.c_int32, ctypes.POINTER(_vp)]),
    "vo_rope_table_destroy": (None, [_vp]),
    "vo_rope": (ctypes.c_int32, [_vp, _vp, _u64, _u64, _u64, _vp, _vp]),
    "vo_rope_positions": (ctypes.c_int32, [_vp, _vp, _u64, _u64, _u64, _u32p, _u64, _vp, _vp]),
    "vo_rope_write_kv": (ctypes.c_int32, [_vp, _u64, _vp, _vp, _u64, _vp, _vp, _u64, _u64, _vp,
                                          _vp]),
    "vo_qkv_rope_write_kv": (ctypes.c_int32, [_vp, _u64, _vp, _vp, _u64, _u64, _u64, _vp, _vp,
                                              _vp]),
    "vo_step_meta_upload_tokens": (ctypes.c_int32, [_vp, _u32p, _u64, _vp]),
    "vo_step_meta_fix_launch": (ctypes.c_int32, [_vp, _u64, _u64, _vp]),
    "vo_step_meta_unfix_launch": (ctypes.c_int32, [_vp]),
    "vo_step_meta_decode_plan": (ctypes.c_int32, [_vp, _vp, _vp, _vp]),
    "vo_decode_attention_write_kv": (ctypes.c_int32, [_vp, _u64, _u64, _vp, _vp, _u64, _vp, _u64,
                                                      _vp, _vp, _vp]),
    "vo_embed": (ctypes.c_int32, [_vp, _u64, _u64, _vp, _u64, _vp, _vp]),
    "vo_rmsnorm": (ctypes.c_int32, [_vp, _u64, _u64, _vp, _u64, ctypes.c_float, _vp, _vp]),
    "vo_rmsnorm_last_rows": (ctypes.c_int32, [_vp, _u64, _u64, _vp, _u64, ctypes.c_float, _vp,
                                              _vp, _vp]),
    "vo_gather_rows": (ctypes.c_int32, [_vp, ctypes.c_int32, _u64, _u64, _u32p, _u64, _vp, _vp,
                                        _vp]),
    "vo_add": (ctypes.c_int32, [_vp, _vp, ctypes.c_int32, _u64, _u64, _vp]),
    "vo_silu_mul": (ctypes.c_int32, [_vp, _u64, _vp, _u64, _u64, _u64, _vp, _u64, _vp]),
    "vo_argmax": (ctypes.c_int32, [_vp, ctypes.c_int32, _u64, _u64, _u32p, _u32p, _vp]),
    "vo_gemm_create": (ctypes.c_int32, [ctypes.c_int32, _u64, ctypes.POINTER(_vp)]),
    "vo_gemm_destroy": (None, [_vp]),
    "vo_matmul": (ctypes.c_int32, [_vp, _vp, _u64, _u64, _vp, _u64, _u64, _vp, ctypes.c_int32,
                                   ctypes.c_int32, _vp]),
    "vo_workspace_create": (ctypes.c_int32, [ctypes.c_int32, _u64, ctypes.POINTER(_vp)]),
    "vo_workspace_destroy": (None, [_vp]),
    "vo_workspace_elems": (_u64, [_vp]),
    "vo_workspace_region": (ctypes.c_int32, [_vp, _u64, _u64, _u64, ctypes.POINTER(_vp)]),
    "vo_workspace_read": (ctypes.c_int32, [_vp, _u64, _u64, _u64, ctypes.c_int32,
                                           ctypes.POINTER(ctypes.c_float), _vp]),
    "vo_weight_upload": (ctypes.c_int32, [ctypes.c_int32, ctypes.POINTER(ctypes.c_float), _u64p,
                                          _u64, ctypes.c_int32, ctypes.POINTER(_vp)]),
    "vo_weight_concat_rows": (ctypes.c_int32, [ctypes.POINTER(_vp), _u64, ctypes.POINTER(_vp)]),
    "vo_weight_destroy": (None, [_vp]),
    "vo_weight_shape": (ctypes.c_int32, [_vp, _u64p, _u64, _u64p]),
    "vo_weight_data": (_vp, [_vp]),
    "vo_weight_dtype": (ctypes.c_int32, [_vp]),
    "vo_profiling_enable": (ctypes.c_int32, [ctypes.c_int32]),
    "vo_profile_read": (ctypes.c_int32, [ctypes.POINTER(vo_kernel_stat), _u64, _u64p]),
    "vo_profile_reset": (None, []),
}


def _hip_runtimes_mapped() -> List[str]:
    try:
        maps = pathlib.Path("/proc/self/maps").read_text()
    except OSError:
        return []
    return sorted({line.split()[-1] for line in maps.splitlines()
                   if "libamdhip64.so" in line and "/" in line})


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
            f"g.build()'` (make -C vllm-oxide_amd/csrc).  There is no fallback path.")
    # PyTorch-ROCm wheels carry their own HIP runtime (SONAME libamdhip64.so.7).
    # Loading torch first makes the loader bind this library to that same
    # runtime, so torch's device pointers and streams are valid here.  Loaded
    # the other way round, two HIP runtimes would coexist in the process.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    handle = ctypes.CDLL(str(LIB_PATH))
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        raise ImportError(
            "two HIP runtimes are loaded in this process (" + ", ".join(runtimes) + "); "
            "import torch before anything that loads /opt/rocm's libamdhip64")
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle


lib = _load()

# ---------------------------------------------------------------------------
# Errors (error.rs:8-56)
# ---------------------------------------------------------------------------


class EngineError(Exception):
    """A failed C-ABI call; fields are the reference variant's fields."""

    def __init__(self, info: vo_error_info):
        self.status = int(info.status)
        self.op = info.op.decode()
        self.seq = int(info.seq)
        self.tokens = int(info.tokens)
        self.needed = int(info.needed)
        self.have = int(info.have)
        self.value = int(info.value)
        self.limit = int(info.limit)
        self.message = info.message.decode()
        super().__init__(f"{lib.vo_status_name(self.status).decode()}: {self.message}")


class ShapeError(EngineError): pass
class CapacityError(EngineError): pass
class BlockTableTooShort(EngineError): pass
class SlotOutOfRange(EngineError): pass
class BlockOutOfRange(EngineError): pass
class DeviceError(EngineError): pass
class InvalidArgument(EngineError): pass
class Unsupported(EngineError): pass
class PositionOutOfRange(EngineError): pass
class NaNError(EngineError): pass
class OutsideWorkspace(EngineError): pass


_ERROR_CLASSES = {
    VO_ERR_SHAPE: ShapeError, VO_ERR_CAPACITY: CapacityError,
    VO_ERR_BLOCK_TABLE_TOO_SHORT: BlockTableTooShort, VO_ERR_SLOT_OUT_OF_RANGE: SlotOutOfRange,
    VO_ERR_BLOCK_OUT_OF_RANGE: BlockOutOfRange, VO_ERR_DEVICE: DeviceError,
    VO_ERR_INVALID_ARGUMENT: InvalidArgument, VO_ERR_UNSUPPORTED: Unsupported,
    VO_ERR_POSITION_OUT_OF_RANGE: PositionOutOfRange, VO_ERR_NAN: NaNError,
    VO_ERR_OUTSIDE_WORKSPACE: OutsideWorkspace,
}


def _engine_error(cls, status: int, op: str, message: str, value: int = 0, limit: int = 0):
    """An EngineError raised by host code above the C ABI (the model's batch
    checks, model.rs:245-267), with the same fields as one from the library."""
    info = vo_error_info()
    info.status = status
    info.op = op.encode()[:47]
    info.value, info.limit = value, limit
    info.message = message.encode()[:255]
    return cls(info)


def _check(rc: int) -> None:
    if rc != VO_OK:
        info = vo_error_info()
        lib.vo_last_error(ctypes.byref(info))
        raise _ERROR_CLASSES.get(rc, EngineError)(info)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def _u64a(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint64))


def _p32(a: np.ndarray):
    return a.ctypes.data_as(_u32p)


def _p64(a: np.ndarray):
    return a.ctypes.data_as(_u64p)


# ---------------------------------------------------------------------------
# paged.rs
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class KvLayout:
    """paged.rs:25-45."""
    num_layers: int
    num_blocks: int
    block_size: int
    kv_heads: int
    head_dim: int

    def _c(self) -> vo_kv_layout:
        return vo_kv_layout(self.num_layers, self.num_blocks, self.block_size, self.kv_heads,
                            self.head_dim)

    def num_slots(self) -> int:
        return int(lib.vo_kv_layout_num_slots(ctypes.byref(self._c())))

    def layer_elems(self) -> int:
        return int(lib.vo_kv_layout_layer_elems(ctypes.byref(self._c())))


def slot_of(block_table: Sequence[int], pos: int, block_size: int) -> int:
    """paged.rs:48-52."""
    t = _u32(block_table)
    out = ctypes.c_uint32()
    _check(lib.vo_slot_of(_p32(t), len(t), pos, block_size, ctypes.byref(out)))
    return int(out.value)


@dataclass
class PrefillSeq:
    """paged.rs:84-92."""
    context_len: int
    num_new: int
    block_table: Sequence[int]


@dataclass
class DecodeSeq:
    """paged.rs:164-168."""
    context_len: int
    block_table: Sequence[int]


def _csr(tables: List[np.ndarray]):
    off = np.zeros(len(tables) + 1, dtype=np.uint64)
    if tables:
        off[1:] = np.cumsum([len(t) for t in tables])
    flat = np.concatenate(tables).astype(np.uint32) if tables and off[-1] else np.zeros(1, np.uint32)
    return off, flat


def _frozen(a, dtype) -> np.ndarray:
    """A read-only copy of `a` as a flat array of `dtype`."""
    out = np.array(a, dtype=dtype, copy=True).reshape(-1)
    out.setflags(write=False)
    return out


@dataclass(frozen=True)
class PrefillMeta:
    """paged.rs:97-114, built by the library's PrefillMeta::new restatement.

    Immutable: every array is a read-only copy, so a meta object names one
    step's contents and HipBackend may upload it once for all the layers
    that receive it.  A changed step is a new object
    (``dataclasses.replace``)."""
    block_size: int
    block_tables: List[np.ndarray]
    context_lens: np.ndarray
    seq_row_starts: np.ndarray
    positions: np.ndarray
    slot_mapping: np.ndarray
    row_seq: np.ndarray
    row_num_keys: np.ndarray
    kind: str = field(default="prefill", repr=False)

    def __post_init__(self):
        put = object.__setattr__
        put(self, "block_tables", tuple(_frozen(t, np.uint32) for t in self.block_tables))
        put(self, "context_lens", _frozen(self.context_lens, np.uint64))
        put(self, "seq_row_starts", _frozen(self.seq_row_starts, np.uint64))
        put(self, "positions", _frozen(self.positions, np.uint32))
        put(self, "slot_mapping", _frozen(self.slot_mapping, np.uint32))
        put(self, "row_seq", _frozen(self.row_seq, np.uint64))
        put(self, "row_num_keys", _frozen(self.row_num_keys, np.uint64))

    @staticmethod
    def new(seqs: Sequence[PrefillSeq], block_size: int) -> "PrefillMeta":
        tables = [_u32(s.block_table) for s in seqs]
        cseqs = (vo_prefill_seq * max(len(seqs), 1))()
        for i, (s, t) in enumerate(zip(seqs, tables)):
            cseqs[i] = vo_prefill_seq(s.context_len, s.num_new, _p32(t), len(t))
        rows = int(sum(s.num_new for s in seqs))
        starts = np.zeros(len(seqs) + 1, np.uint64)
        pos = np.zeros(max(rows, 1), np.uint32)
        slots = np.zeros(max(rows, 1), np.uint32)
        rseq = np.zeros(max(rows, 1), np.uint64)
        rkeys = np.zeros(max(rows, 1), np.uint64)
        _check(lib.vo_prefill_meta_build(cseqs, len(seqs), block_size, _p64(starts), _p32(pos),
                                         _p32(slots), _p64(rseq), _p64(rkeys)))
        return PrefillMeta(block_size, tables,
                           np.array([s.context_len for s in seqs], np.uint64), starts,
                           pos[:rows], slots[:rows], rseq[:rows], rkeys[:rows])

    def num_seqs(self) -> int:
        return len(self.context_lens)

    def num_rows(self) -> int:
        return len(self.positions)

    def last_rows(self) -> np.ndarray:
        """paged.rs:154-159."""
        out = np.zeros(max(self.num_seqs(), 1), np.uint32)
        starts = _u64a(self.seq_row_starts)
        _check(lib.vo_last_rows(_p64(starts), self.num_seqs(), _p32(out)))
        return out[: self.num_seqs()]


@dataclass(frozen=True)
class DecodeMeta:
    """paged.rs:173-186, built by the library's DecodeMeta::new restatement.
    Immutable, as PrefillMeta."""
    block_size: int
    block_tables: List[np.ndarray]
    positions: np.ndarray
    slot_mapping: np.ndarray
    row_seq: np.ndarray
    row_num_keys: np.ndarray
    kind: str = field(default="decode", repr=False)

    def __post_init__(self):
        put = object.__setattr__
        put(self, "block_tables", tuple(_frozen(t, np.uint32) for t in self.block_tables))
        put(self, "positions", _frozen(self.positions, np.uint32))
        put(self, "slot_mapping", _frozen(self.slot_mapping, np.uint32))
        put(self, "row_seq", _frozen(self.row_seq, np.uint64))
        put(self, "row_num_keys", _frozen(self.row_num_keys, np.uint64))

    @staticmethod
    def new(seqs: Sequence[DecodeSeq], block_size: int) -> "DecodeMeta":
        tables = [_u32(s.block_table) for s in seqs]
        cseqs = (vo_decode_seq * max(len(seqs), 1))()
        for i, (s, t) in enumerate(zip(seqs, tables)):
            cseqs[i] = vo_decode_seq(s.context_len, _p32(t), len(t))
        n = len(seqs)
        pos = np.zeros(max(n, 1), np.uint32)
        slots = np.zeros(max(n, 1), np.uint32)
        rseq = np.zeros(max(n, 1), np.uint64)
        rkeys = np.zeros(max(n, 1), np.uint64)
        _check(lib.vo_decode_meta_build(cseqs, n, block_size, _p32(pos), _p32(slots), _p64(rseq),
                                        _p64(rkeys)))
        return DecodeMeta(block_size, tables, pos[:n], slots[:n], rseq[:n], rkeys[:n])

    def num_seqs(self) -> int:
        return len(self.positions)


# ---------------------------------------------------------------------------
# Opt-in kernel timing (arena.rs:129-136 enable_profiling / profile)
# ---------------------------------------------------------------------------


def enable_profiling(on: bool = True) -> None:
    _check(lib.vo_profiling_enable(1 if on else 0))


def profile() -> dict:
    """{kernel: {"calls", "total_ms", "min_ms", "max_ms", "avg_ms"}}; waits for
    the recorded events."""
    n = ctypes.c_uint64()
    _check(lib.vo_profile_read(None, 0, ctypes.byref(n)))
    arr = (vo_kernel_stat * max(n.value, 1))()
    _check(lib.vo_profile_read(arr, n.value, ctypes.byref(n)))
    out = {}
    for i in range(n.value):
        s = arr[i]
        out[s.name.decode()] = dict(calls=int(s.calls), total_ms=s.total_ms, min_ms=s.min_ms,
                                    max_ms=s.max_ms,
                                    avg_ms=s.total_ms / s.calls if s.calls else 0.0)
    return out


def profile_reset() -> None:
    lib.vo_profile_reset()


# ---------------------------------------------------------------------------
# Backend (mod.rs:61-182, attention path)
# ---------------------------------------------------------------------------


class KvPool:
    """Backend::KvPool: an opaque device pool (bf16)."""

    def __init__(self, layout: KvLayout, device: int):
        self.layout = layout
        self.device = device
        self._h = _vp()
        _check(lib.vo_kv_pool_create(ctypes.byref(layout._c()), device, ctypes.byref(self._h)))

    @property
    def handle(self):
        return self._h

    def nbytes(self) -> int:
        return int(lib.vo_kv_pool_bytes(self._h))

    def close(self) -> None:
        if self._h:
            lib.vo_kv_pool_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class StepMeta:
    """Device-resident step metadata (vo_step_meta)."""

    def __init__(self, pool: KvPool, max_seqs: int, max_rows: int, max_table_entries: int,
                 max_query_heads: int):
        self._h = _vp()
        _check(lib.vo_step_meta_create(pool.handle, max_seqs, max_rows, max_table_entries,
                                       max_query_heads, ctypes.byref(self._h)))
        self.capacity = (max_seqs, max_rows, max_table_entries, max_query_heads)
        self.holds = None  # the host meta object last uploaded

    @property
    def handle(self):
        return self._h

    def upload(self, meta, stream=None) -> None:
        off, flat = _csr(meta.block_tables)
        if isinstance(meta, PrefillMeta):
            ctx = _u64a(meta.context_lens)
            starts = _u64a(meta.seq_row_starts)
            pos = _u32(meta.positions)
            slots = _u32(meta.slot_mapping)
            rseq = _u64a(meta.row_seq)
            rkeys = _u64a(meta.row_num_keys)
            _check(lib.vo_step_meta_upload_prefill(
                self._h, meta.block_size, meta.num_seqs(), _p64(off), _p32(flat), _p64(ctx),
                _p64(starts), meta.num_rows(), _p32(pos), _p32(slots), _p64(rseq), _p64(rkeys),
                _stream_ptr(stream)))
        elif isinstance(meta, DecodeMeta):
            pos = _u32(meta.positions)
            slots = _u32(meta.slot_mapping)
            rseq = _u64a(meta.row_seq)
            rkeys = _u64a(meta.row_num_keys)
            _check(lib.vo_step_meta_upload_decode(
                self._h, meta.block_size, meta.num_seqs(), _p64(off), _p32(flat), _p32(pos),
                _p32(slots), _p64(rseq), _p64(rkeys), _stream_ptr(stream)))
        else:
            raise TypeError(f"cannot upload {type(meta).__name__}")
        self.holds = meta

    def sync(self, meta, stream=None) -> None:
        """vo_step_meta_sync_prefill / _decode: upload ``meta`` unless the last
        upload holds exactly its values (compared in the library, element by
        element, so a meta refilled in place is seen)."""
        off, flat = _csr(meta.block_tables)
        pos = _u32(meta.positions)
        slots = _u32(meta.slot_mapping)
        rseq = _u64a(meta.row_seq)
        rkeys = _u64a(meta.row_num_keys)
        if isinstance(meta, PrefillMeta):
            _check(lib.vo_step_meta_sync_prefill(
                self._h, meta.block_size, meta.num_seqs(), _p64(off), _p32(flat),
                _p64(_u64a(meta.context_lens)), _p64(_u64a(meta.seq_row_starts)),
                meta.num_rows(), _p32(pos), _p32(slots), _p64(rseq), _p64(rkeys),
                _stream_ptr(stream)))
        elif isinstance(meta, DecodeMeta):
            _check(lib.vo_step_meta_sync_decode(
                self._h, meta.block_size, meta.num_seqs(), _p64(off), _p32(flat), _p32(pos),
                _p32(slots), _p64(rseq), _p64(rkeys), _stream_ptr(stream)))
        else:
            raise TypeError(f"cannot upload {type(meta).__name__}")
        self.holds = meta

    def upload_tokens(self, tokens, stream=None) -> None:
        """The step's token ids (vo_step_meta_upload_tokens)."""
        t = _u32(tokens) if len(tokens) else np.zeros(1, np.uint32)
        _check(lib.vo_step_meta_upload_tokens(self._h, _p32(t), len(tokens),
                                              _stream_ptr(stream)))

    def fix_launch(self, work_headroom: int, entry_headroom: int, stream=None) -> None:
        """vo_step_meta_fix_launch: the last upload (a decode step) again, in
        fixed-launch layout, ready to be recorded as a graph."""
        _check(lib.vo_step_meta_fix_launch(self._h, work_headroom, entry_headroom,
                                           _stream_ptr(stream)))

    def unfix_launch(self) -> None:
        _check(lib.vo_step_meta_unfix_launch(self._h))

    def decode_plan(self) -> tuple:
        """vo_step_meta_decode_plan: (work items, split-K partials, row-packing
        factor) of the last upload's decode plan."""
        w, p, k = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint32()
        _check(lib.vo_step_meta_decode_plan(self._h, ctypes.byref(w), ctypes.byref(p),
                                            ctypes.byref(k)))
        return w.value, p.value, k.value

    def upload_slots(self, slots, stream=None) -> None:
        s = _u32(slots)
        _check(lib.vo_step_meta_upload_slots(self._h, _p32(s), len(s), _stream_ptr(stream)))
        self.holds = None

    def close(self) -> None:
        if self._h:
            lib.vo_step_meta_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _stream_ptr(stream):
    if stream is None:
        import torch
        return _vp(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return _vp(stream)
    return _vp(stream.cuda_stream)


def _dev_ptr(t) -> _vp:
    import torch
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError("expected a device tensor")
    if t.dtype != torch.bfloat16 or not t.is_contiguous():
        raise TypeError("expected a contiguous bfloat16 tensor")
    return _vp(t.data_ptr())


def _any_ptr(t, dtype) -> _vp:
    """Device pointer of a contiguous tensor of the given torch dtype."""
    import torch
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError("expected a device tensor")
    if t.dtype != dtype or not t.is_contiguous():
        raise TypeError(f"expected a contiguous {dtype} tensor, got {t.dtype}")
    return _vp(t.data_ptr())


@dataclass(frozen=True)
class Region:
    """mod.rs:31-38: a [rows, cols] matrix at ``offset`` elements of the workspace."""
    offset: int
    rows: int
    cols: int

    def __len__(self) -> int:
        return self.rows * self.cols


class Workspace:
    """Backend::alloc_workspace / workspace_elems / read (mod.rs:76-78,
    177-181): the activation workspace, ``elems`` 4-byte elements of device
    memory owned by the library (vo_workspace)."""

    def __init__(self, elems: int, device: int = 0):
        self._h = _vp()
        _check(lib.vo_workspace_create(device, elems, ctypes.byref(self._h)))

    @property
    def handle(self):
        return self._h

    def elems(self) -> int:
        return int(lib.vo_workspace_elems(self._h))

    def ptr(self, region: Region) -> _vp:
        """Device address of a region (OutsideWorkspace past the end)."""
        out = _vp()
        _check(lib.vo_workspace_region(self._h, region.offset, region.rows, region.cols,
                                       ctypes.byref(out)))
        return out

    def read(self, region: Region, dtype: int = VO_DTYPE_F32, stream=0) -> np.ndarray:
        """Backend::read: the region's values as f32 [rows, cols] (waits for ``stream``)."""
        out = np.zeros(max(len(region), 1), np.float32)
        _check(lib.vo_workspace_read(self._h, region.offset, region.rows, region.cols, dtype,
                                     out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                     _vp(stream) if isinstance(stream, int) else _stream_ptr(stream)))
        return out[:len(region)].reshape(region.rows, region.cols)

    def close(self) -> None:
        if self._h:
            lib.vo_workspace_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Weight:
    """Backend::upload / weight_shape (mod.rs:69-72): a weight the library
    holds on the device (vo_weight), bf16 by default."""

    def __init__(self, data=None, device: int = 0, dtype: int = VO_DTYPE_BF16, _handle=None):
        self._h = _vp()
        if _handle is not None:
            self._h = _handle
            return
        a = np.ascontiguousarray(np.asarray(data, np.float32))
        shape = _u64a(a.shape)
        _check(lib.vo_weight_upload(device, a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                    _p64(shape), a.ndim, dtype, ctypes.byref(self._h)))

    @staticmethod
    def concat_rows(parts: Sequence["Weight"]) -> "Weight":
        arr = (_vp * len(parts))(*[p.handle for p in parts])
        h = _vp()
        _check(lib.vo_weight_concat_rows(arr, len(parts), ctypes.byref(h)))
        return Weight(_handle=h)

    @property
    def handle(self):
        return self._h

    @property
    def ptr(self) -> _vp:
        return _vp(lib.vo_weight_data(self._h))

    def shape(self) -> tuple:
        n = ctypes.c_uint64()
        _check(lib.vo_weight_shape(self._h, None, 0, ctypes.byref(n)))
        dims = np.zeros(max(n.value, 1), np.uint64)
        _check(lib.vo_weight_shape(self._h, _p64(dims), n.value, ctypes.byref(n)))
        return tuple(int(d) for d in dims[:n.value])

    def dtype(self) -> int:
        return int(lib.vo_weight_dtype(self._h))

    def close(self) -> None:
        if self._h:
            lib.vo_weight_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class BlockManager:
    """KV block manager with refcounted blocks and a full-block prefix cache
    (the reference's planned M2/M4 components; invariant CLAUDE.md:71).
    Host only: no GPU needed."""

    NONE = 0xFFFFFFFF

    def __init__(self, num_blocks: int, block_size: int, prefix_caching: bool = True):
        self._h = _vp()
        _check(lib.vo_bm_create(num_blocks, block_size, int(prefix_caching), ctypes.byref(self._h)))
        self.num_blocks, self.block_size = num_blocks, block_size

    def test_unchained_hash(self, on: bool = True) -> None:
        """Test hook: block hashes cover a block's own tokens only, so equal
        blocks after different prefixes collide on purpose.  Only before the
        first sequence."""
        _check(lib.vo_bm_test_unchained_hash(self._h, int(on)))

    def add_sequence(self, seq_id: int, tokens) -> int:
        """Admit a sequence with its prompt; returns the prompt tokens already cached."""
        t = _u32(tokens) if len(tokens) else np.zeros(1, np.uint32)
        cached = ctypes.c_uint64(0)
        _check(lib.vo_bm_add_sequence(self._h, seq_id, _p32(t), len(tokens), ctypes.byref(cached)))
        return cached.value

    def append_token(self, seq_id: int, token: int):
        """Returns (slot, copy) with copy = (src, dst) block ids or None."""
        slot, src, dst = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
        _check(lib.vo_bm_append_token(self._h, seq_id, token, ctypes.byref(slot),
                                      ctypes.byref(src), ctypes.byref(dst)))
        return slot.value, (None if src.value == self.NONE else (src.value, dst.value))

    def fork(self, parent: int, child: int) -> None:
        _check(lib.vo_bm_fork(self._h, parent, child))

    def free(self, seq_id: int) -> None:
        _check(lib.vo_bm_free_sequence(self._h, seq_id))

    def block_table(self, seq_id: int) -> np.ndarray:
        n, toks = ctypes.c_uint64(), ctypes.c_uint64()
        _check(lib.vo_bm_block_table(self._h, seq_id, None, 0, ctypes.byref(n), ctypes.byref(toks)))
        out = np.zeros(max(n.value, 1), np.uint32)
        _check(lib.vo_bm_block_table(self._h, seq_id, _p32(out), len(out), ctypes.byref(n),
                                     ctypes.byref(toks)))
        return out[:n.value]

    def num_tokens(self, seq_id: int) -> int:
        n, toks = ctypes.c_uint64(), ctypes.c_uint64()
        _check(lib.vo_bm_block_table(self._h, seq_id, None, 0, ctypes.byref(n), ctypes.byref(toks)))
        return toks.value

    def available(self) -> int:
        return int(lib.vo_bm_num_available(self._h))

    def stats(self) -> dict:
        st = vo_bm_stats()
        _check(lib.vo_bm_get_stats(self._h, ctypes.byref(st)))
        return {f: int(getattr(st, f)) for f, _ in vo_bm_stats._fields_}

    def check(self) -> None:
        """Raises ShapeError with the first violated invariant."""
        _check(lib.vo_bm_check_invariants(self._h))

    def close(self) -> None:
        if self._h:
            lib.vo_bm_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class RopeTable:
    """RopeTable (rope.rs:24-100) on one device: Llama 3 scaled frequencies,
    cos/sin for positions 0 .. max_len-1.  Defaults are LLAMA_3_2_1B's
    rope_scaling block (config.rs:41-56)."""

    def __init__(self, head_dim: int, rope_theta: float, max_len: int, device: int = 0,
                 factor: float = 32.0, low_freq_factor: float = 1.0,
                 high_freq_factor: float = 4.0, original_max_position_embeddings: int = 8192):
        cfg = vo_rope_config(head_dim, rope_theta, factor, low_freq_factor, high_freq_factor,
                             original_max_position_embeddings)
        self._h = _vp()
        _check(lib.vo_rope_table_create(ctypes.byref(cfg), max_len, device, ctypes.byref(self._h)))
        self.head_dim, self.max_len = head_dim, max_len

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if self._h:
            lib.vo_rope_table_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipBackend:
    """The attention-path ops of ``trait Backend`` (mod.rs:61-182) on one GPU.

    Activations are contiguous ``torch.bfloat16`` device tensors (the GPU
    counterpart of the reference's f32 workspace regions).  Block tables and
    slot mappings come from ``PrefillMeta``/``DecodeMeta``; the backend uploads
    a meta to its device-resident copy the first time it sees it, so a step's
    metadata crosses to the device once for all layers.
    """

    def __init__(self, device: int = 0, max_seqs: int = 512, max_rows: int = 8192,
                 max_table_entries: int = 1 << 16, max_query_heads: int = 64):
        self.device = device
        self._caps = (max_seqs, max_rows, max_table_entries, max_query_heads)
        # pool -> {slot name: StepMeta}; keyed by the pool object itself (weakly),
        # so a meta never outlives its pool or serves a later pool.
        self._metas = weakref.WeakKeyDictionary()

    def name(self) -> str:
        return "hip-gfx950"

    # mod.rs:73-75
    def alloc_kv_pool(self, layout: KvLayout) -> KvPool:
        return KvPool(layout, self.device)

    def kv_layout(self, pool: KvPool) -> KvLayout:
        out = vo_kv_layout()
        _check(lib.vo_kv_pool_layout(pool.handle, ctypes.byref(out)))
        return KvLayout(out.num_layers, out.num_blocks, out.block_size, out.kv_heads,
                        out.head_dim)

    def step_meta(self, pool: KvPool, slot: str = "step") -> StepMeta:
        per_pool = self._metas.setdefault(pool, {})
        m = per_pool.get(slot)
        if m is None:
            m = StepMeta(pool, *self._caps)
            per_pool[slot] = m
        return m

    def _meta_for(self, pool: KvPool, meta, stream, slot: str = "step") -> StepMeta:
        # A PrefillMeta / DecodeMeta is immutable, so the object names its
        # contents: the step's upload serves every layer that receives it.
        m = self.step_meta(pool, slot)
        if m.holds is not meta:
            m.upload(meta, stream)
        return m

    # mod.rs:107-119
    def write_kv(self, pool: KvPool, layer: int, keys, values, slots, stream=None) -> None:
        """``slots`` is a PrefillMeta/DecodeMeta (its slot mapping) or a slot list."""
        if isinstance(slots, (PrefillMeta, DecodeMeta)):
            m = self._meta_for(pool, slots, stream)
        else:
            m = self.step_meta(pool, "slots")
            m.upload_slots(slots, stream)
        rows = keys.shape[0] if keys.dim() == 2 else 0
        cols = keys.shape[1] if keys.dim() == 2 else 0
        if tuple(values.shape) != tuple(keys.shape):
            raise ValueError("keys and values must have the same shape")
        _check(lib.vo_write_kv(pool.handle, layer, _dev_ptr(keys), _dev_ptr(values), rows, cols,
                               m.handle, _stream_ptr(stream)))

    def _attention(self, fn, queries, pool: KvPool, layer: int, meta, out, stream):
        import torch
        m = self._meta_for(pool, meta, stream)
        if out is None:
            out = torch.empty_like(queries)
        _check(fn(_dev_ptr(queries), queries.shape[0], queries.shape[1], pool.handle, layer,
                  m.handle, _dev_ptr(out), _stream_ptr(stream)))
        return out

    def copy_blocks(self, pool: KvPool, pairs, stream=None) -> None:
        """Block copies of every layer: pairs = [(src, dst), ...] (copy on write)."""
        if not pairs:
            return
        src = _u32([p[0] for p in pairs])
        dst = _u32([p[1] for p in pairs])
        _check(lib.vo_kv_copy_blocks(pool.handle, _p32(src), _p32(dst), len(pairs),
                                     _stream_ptr(stream)))

    # mod.rs:105
    def rope(self, table: RopeTable, x, pool: KvPool, meta, head_dim: int, stream=None) -> None:
        """Backend::rope: rotates x [rows, cols] in place at the meta's positions."""
        m = self._meta_for(pool, meta, stream)
        _check(lib.vo_rope(table.handle, _dev_ptr(x), x.shape[0], x.shape[1], head_dim, m.handle,
                           _stream_ptr(stream)))

    def rope_positions(self, table: RopeTable, x, pool: KvPool, positions, head_dim: int,
                       stream=None) -> None:
        """Backend::rope with the trait's arguments: rotates x [rows, cols] in
        place at host ``positions`` [rows] (vo_rope_positions)."""
        m = self.step_meta(pool)
        p = _u32(positions) if len(positions) else np.zeros(1, np.uint32)
        _check(lib.vo_rope_positions(table.handle, _dev_ptr(x), x.shape[0], x.shape[1], head_dim,
                                     _p32(p), len(positions), m.handle, _stream_ptr(stream)))

    def rope_write_kv(self, pool: KvPool, layer: int, table: RopeTable, queries, keys, values,
                      meta, stream=None) -> None:
        """rope(q); rope(k); write_kv(k, v) in one launch (q rotated in place)."""
        m = self._meta_for(pool, meta, stream)
        if tuple(values.shape) != tuple(keys.shape):
            raise ValueError("keys and values must have the same shape")
        _check(lib.vo_rope_write_kv(pool.handle, layer, table.handle, _dev_ptr(queries),
                                    queries.shape[1], _dev_ptr(keys), _dev_ptr(values),
                                    keys.shape[0], keys.shape[1], m.handle, _stream_ptr(stream)))

    # mod.rs:121-135
    def prefill_attention(self, queries, pool: KvPool, layer: int, meta: PrefillMeta, out=None,
                          stream=None):
        return self._attention(lib.vo_prefill_attention, queries, pool, layer, meta, out, stream)

    # mod.rs:137-149
    def decode_attention(self, queries, pool: KvPool, layer: int, meta: DecodeMeta, out=None,
                         stream=None):
        return self._attention(lib.vo_decode_attention, queries, pool, layer, meta, out, stream)

    def decode_attention_write_kv(self, queries, keys, values, pool: KvPool, layer: int,
                                  meta: DecodeMeta, out=None, stream=None):
        """write_kv(keys, values, meta) then decode_attention(queries), as one
        launch where the step allows it (vo_decode_attention_write_kv)."""
        import torch
        m = self._meta_for(pool, meta, stream)
        if out is None:
            out = torch.empty_like(queries)
        _check(lib.vo_decode_attention_write_kv(
            _dev_ptr(queries), queries.shape[0], queries.shape[1], _dev_ptr(keys),
            _dev_ptr(values), keys.shape[1], pool.handle, layer, m.handle, _dev_ptr(out),
            _stream_ptr(stream)))
        return out

    # ---- the rest of the layer (model.rs:269-356) ------------------------
    def embed(self, table, tokens, meta_holder: StepMeta, stream=None):
        """Backend::embed: [T, hidden] f32 rows of the bf16 table."""
        import torch
        meta_holder.upload_tokens(tokens, stream)
        out = torch.empty((len(tokens), table.shape[1]), dtype=torch.float32,
                          device=f"cuda:{self.device}")
        _check(lib.vo_embed(_dev_ptr(table), table.shape[0], table.shape[1], meta_holder.handle,
                            len(tokens), _any_ptr(out, torch.float32), _stream_ptr(stream)))
        return out

    def rmsnorm(self, x, weight, eps: float, stream=None):
        """Backend::rmsnorm: x [T, H] f32, weight [H] bf16 -> [T, H] bf16."""
        import torch
        out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
        _check(lib.vo_rmsnorm(_any_ptr(x, torch.float32), x.shape[0], x.shape[1],
                              _dev_ptr(weight), weight.numel(), eps, _dev_ptr(out),
                              _stream_ptr(stream)))
        return out

    def rmsnorm_last_rows(self, x, weight, eps: float, pool: KvPool, meta, stream=None):
        """gather_rows(x, meta.last_rows()) then rmsnorm, one pass -> [S, H] bf16."""
        import torch
        m = self._meta_for(pool, meta, stream)
        out = torch.empty((meta.num_seqs(), x.shape[1]), dtype=torch.bfloat16, device=x.device)
        _check(lib.vo_rmsnorm_last_rows(_any_ptr(x, torch.float32), x.shape[0], x.shape[1],
                                        _dev_ptr(weight), weight.numel(), eps, m.handle,
                                        _dev_ptr(out), _stream_ptr(stream)))
        return out

    def gather_rows(self, x, rows, pool: KvPool, out=None, stream=None):
        """Backend::gather_rows: out[i] = x[rows[i]], x [T, H] f32 or bf16,
        host ``rows`` (vo_gather_rows)."""
        import torch
        m = self.step_meta(pool)
        if out is None:
            out = torch.empty((len(rows), x.shape[1]), dtype=x.dtype, device=x.device)
        dt = VO_DTYPE_BF16 if x.dtype == torch.bfloat16 else VO_DTYPE_F32
        r = _u32(rows) if len(rows) else np.zeros(1, np.uint32)
        _check(lib.vo_gather_rows(_any_ptr(x, x.dtype), dt, x.shape[0], x.shape[1], _p32(r),
                                  len(rows), m.handle, _any_ptr(out, x.dtype),
                                  _stream_ptr(stream)))
        return out

    def add(self, total, x, stream=None) -> None:
        """Backend::add: total (f32) += x (bf16 or f32), in place."""
        import torch
        if tuple(total.shape) != tuple(x.shape):
            raise ValueError("add: shapes differ")
        dt = VO_DTYPE_BF16 if x.dtype == torch.bfloat16 else VO_DTYPE_F32
        _check(lib.vo_add(_any_ptr(total, torch.float32), _any_ptr(x, x.dtype), dt,
                          total.shape[0], total.shape[1], _stream_ptr(stream)))

    def silu_mul(self, gate, up, out=None, stream=None):
        """Backend::silu_mul: out = silu(gate) * up (out=gate: in place); 2-D
        bf16 tensors whose rows may be strided."""
        import torch
        if out is None:
            out = torch.empty(gate.shape, dtype=torch.bfloat16, device=gate.device)
        for t in (gate, up, out):
            if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1:
                raise TypeError("silu_mul takes 2-D bfloat16 tensors with unit column stride")
        _check(lib.vo_silu_mul(_vp(gate.data_ptr()), gate.stride(0), _vp(up.data_ptr()),
                               up.stride(0), gate.shape[0], gate.shape[1], _vp(out.data_ptr()),
                               out.stride(0), _stream_ptr(stream)))
        return out

    def argmax(self, logits, stream=None) -> np.ndarray:
        """Backend::argmax: first index of each row's maximum; NaNError on a NaN."""
        import torch
        rows = logits.shape[0]
        ids = torch.empty((max(rows, 1),), dtype=torch.int32, device=logits.device)
        host = np.zeros(max(rows, 1), np.uint32)
        dt = VO_DTYPE_F32 if logits.dtype == torch.float32 else VO_DTYPE_BF16
        _check(lib.vo_argmax(_any_ptr(logits, logits.dtype), dt, rows, logits.shape[1],
                             ctypes.cast(ctypes.c_void_p(ids.data_ptr()), _u32p), _p32(host),
                             _stream_ptr(stream)))
        return host[:rows]

    def gemm(self) -> "Gemm":
        g = getattr(self, "_gemm", None)
        if g is None:
            g = self._gemm = Gemm(self.device)
        return g

    def matmul(self, x, weight, out_dtype=None, out=None, accumulate=False, stream=None):
        """Backend::matmul: x [T, in] bf16 . weight [out, in]^T (bf16) on hipBLASLt;
        accumulate: out += (out f32 or bf16)."""
        return self.gemm().matmul(x, weight, out_dtype, out, accumulate, stream)

    def read_kv(self, pool: KvPool, layer: int, meta, seq: int, num_keys: int, stream=None):
        """Keys and values 0..num_keys of sequence ``seq``, [num_keys, kv_heads*head_dim]."""
        import torch
        m = self._meta_for(pool, meta, stream)
        width = pool.layout.kv_heads * pool.layout.head_dim
        k = torch.empty((max(num_keys, 1), width), dtype=torch.bfloat16,
                        device=f"cuda:{self.device}")
        v = torch.empty_like(k)
        _check(lib.vo_gather_kv(pool.handle, layer, m.handle, seq, num_keys, _dev_ptr(k),
                                _dev_ptr(v), _stream_ptr(stream)))
        return k[:num_keys], v[:num_keys]


class Gemm:
    """vo_gemm: hipBLASLt handle, workspace and per-shape plans on one device."""

    def __init__(self, device: int = 0, workspace_bytes: int = 128 << 20):
        self._h = _vp()
        _check(lib.vo_gemm_create(device, workspace_bytes, ctypes.byref(self._h)))

    @property
    def handle(self):
        return self._h

    def matmul(self, x, weight, out_dtype=None, out=None, accumulate=False, stream=None):
        import torch
        if out_dtype is None:
            out_dtype = out.dtype if out is not None else torch.bfloat16
        if out is None:
            if accumulate:
                raise ValueError("accumulate needs an output to add into")
            out = torch.empty((x.shape[0], weight.shape[0]), dtype=out_dtype, device=x.device)
        dt = VO_DTYPE_F32 if out_dtype == torch.float32 else VO_DTYPE_BF16
        _check(lib.vo_matmul(self._h, _dev_ptr(x), x.shape[0], x.shape[1], _dev_ptr(weight),
                             weight.shape[0], weight.shape[1], _any_ptr(out, out_dtype), dt,
                             int(bool(accumulate)), _stream_ptr(stream)))
        return out

    def close(self) -> None:
        if self._h:
            lib.vo_gemm_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def prefill_meta_build_device(seq_row_starts, context_lens, table_off, tables, block_size: int,
                              num_rows: int, stream=None):
    """PrefillMeta::new (paged.rs:117-143) on the device from device ``torch.int32``
    tensors (read as u32): seq_row_starts [S+1], context_lens [S], table_off [S+1],
    tables [entries].  Returns (positions, slot_mapping, row_seq, row_num_keys, errors)
    as device int32 tensors (u32 bit patterns); ``errors[0]`` is 1 when some row's
    position lies past its table (the reference's BlockTableTooShort)."""
    import torch
    for t in (seq_row_starts, context_lens, table_off, tables):
        if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.int32
                and t.is_contiguous()):
            raise TypeError("expected contiguous int32 device tensors")
    dev = seq_row_starts.device
    S = seq_row_starts.numel() - 1
    outs = [torch.empty(max(num_rows, 1), dtype=torch.int32, device=dev) for _ in range(4)]
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    _check(lib.vo_prefill_meta_build_device(
        _vp(seq_row_starts.data_ptr()), _vp(context_lens.data_ptr()), _vp(table_off.data_ptr()),
        _vp(tables.data_ptr()), S, num_rows, block_size, *[_vp(o.data_ptr()) for o in outs],
        _vp(err.data_ptr()), _stream_ptr(stream)))
    return tuple(o[:num_rows] for o in outs) + (err,)

"""ctypes binding of include/dr_attn.h (lib/libdr_attn.so).

Python mirror of the reference's attention interface for the tests and the
bench: ``AttnShape``/``Rows``/``attention()`` follow
``src/model/attention.rs:10-27, 65-70, 106`` (same names, same argument
meaning; a failed call raises ``DrError`` where the reference panics), and
``StepCache``/``Pass`` wrap the device-resident KV cache (``cache.rs:25-115``)
and per-pass row metadata (``PassRows``, ``attention.rs:79-85``).

The library is the only compute path: if it is missing ``load()`` raises, and
on a host without a GPU every compute call raises ``DrError`` with
``DR_ERR_NO_DEVICE``.  Nothing here computes attention on the CPU.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import re
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "lib" / "libdr_attn.so"
HEADER_PATH = HERE.parent / "include" / "dr_attn.h"

DR_OK, DR_ERR_INVALID, DR_ERR_NO_DEVICE, DR_ERR_OOM, DR_ERR_HIP, DR_ERR_UNSUPPORTED, DR_ERR_BUSY = range(7)
KERNEL_AUTO, KERNEL_STAGED, KERNEL_STREAMS, KERNEL_HILO = range(4)
DTYPE_F32, DTYPE_BF16 = 0, 1
PRECISION_BF16, PRECISION_HILO = 0, 1  # dr_cache_set_precision
STATUS_NAMES = {
    DR_OK: "DR_OK",
    DR_ERR_INVALID: "DR_ERR_INVALID",
    DR_ERR_NO_DEVICE: "DR_ERR_NO_DEVICE",
    DR_ERR_OOM: "DR_ERR_OOM",
    DR_ERR_HIP: "DR_ERR_HIP",
    DR_ERR_UNSUPPORTED: "DR_ERR_UNSUPPORTED",
    DR_ERR_BUSY: "DR_ERR_BUSY",
}

c_size_p = ctypes.POINTER(ctypes.c_size_t)


class OptUsize(ctypes.Structure):
    _fields_ = [("value", ctypes.c_size_t), ("present", ctypes.c_uint8)]


class CAttnShape(ctypes.Structure):
    _fields_ = [
        ("nq", ctypes.c_size_t),
        ("nk", ctypes.c_size_t),
        ("n_head", ctypes.c_size_t),
        ("n_head_kv", ctypes.c_size_t),
        ("head_dim", ctypes.c_size_t),
        ("sliding_window", OptUsize),
        ("causal_prefix", OptUsize),
        ("scale", ctypes.c_float),
    ]


class CRows(ctypes.Structure):
    _fields_ = [
        ("pos", c_size_p),
        ("pos_len", ctypes.c_size_t),
        ("seq", c_size_p),
        ("seq_len", ctypes.c_size_t),
        ("prefix", c_size_p),
        ("prefix_len", ctypes.c_size_t),
    ]


class CBatchItem(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("out", ctypes.c_void_p), ("pass_", ctypes.c_void_p)]


class CStepItem(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("out", ctypes.c_void_p), ("pass_", ctypes.c_void_p),
                ("k", ctypes.c_void_p), ("v", ctypes.c_void_p)]


class CStepItemRows(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("out", ctypes.c_void_p), ("pass_", ctypes.c_void_p),
                ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("q_stride", ctypes.c_size_t),
                ("kv_stride", ctypes.c_size_t)]


class CEpilogue(ctypes.Structure):
    _fields_ = [("bq", ctypes.c_void_p), ("bk", ctypes.c_void_p), ("bv", ctypes.c_void_p),
                ("q_norm_w", ctypes.c_void_p), ("k_norm_w", ctypes.c_void_p),
                ("v_norm", ctypes.c_int), ("eps", ctypes.c_float), ("rope", ctypes.c_void_p)]


class CLaunchInfo(ctypes.Structure):
    _fields_ = [
        ("n_split", ctypes.c_int),
        ("n_workgroups", ctypes.c_int),
        ("waves_per_wg", ctypes.c_int),
        ("block_n", ctypes.c_int),
        ("head_dim_tile", ctypes.c_int),
        ("row_blocks", ctypes.c_int),
        ("key_groups", ctypes.c_int),
        ("rows_per_wave", ctypes.c_int),
        ("kernel", ctypes.c_int),
        ("split_merge", ctypes.c_int),
    ]


class DrError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


_LIB: Optional[ctypes.CDLL] = None

_VP = ctypes.c_void_p
_SZ = ctypes.c_size_t
_I = ctypes.c_int
_F = ctypes.c_float
_SIGS = {
    "dr_last_error": (ctypes.c_char_p, []),
    "dr_version": (ctypes.c_char_p, []),
    "dr_device_count": (_I, []),
    "dr_attention": (_I, [_VP, _SZ, _VP, _SZ, _VP, _SZ, _VP, _SZ, CAttnShape, CRows, CRows]),
    "dr_ctx_create": (_I, [_I, ctypes.POINTER(_VP)]),
    "dr_ctx_set_stream": (_I, [_VP, _VP]),
    "dr_ctx_stream": (_VP, [_VP]),
    "dr_ctx_synchronize": (_I, [_VP]),
    "dr_ctx_destroy": (None, [_VP]),
    "dr_ctx_last_launch": (_I, [_VP, ctypes.POINTER(CLaunchInfo)]),
    "dr_ctx_set_split": (_I, [_VP, _I]),
    "dr_ctx_set_wave_rows": (_I, [_VP, _I]),
    "dr_ctx_set_kernel": (_I, [_VP, _I]),
    "dr_ctx_set_q_dtype": (_I, [_VP, _I]),
    "dr_ctx_set_o_dtype": (_I, [_VP, _I]),
    "dr_ctx_set_split_merge": (_I, [_VP, _I]),
    "dr_rope_create": (_I, [_VP, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_float, _VP,
                            ctypes.POINTER(ctypes.c_void_p)]),
    "dr_rope_destroy": (None, [_VP]),
    "dr_attention_step_epi": (_I, [_VP, ctypes.c_size_t, ctypes.POINTER(CStepItem), ctypes.c_size_t,
                                   ctypes.c_size_t, OptUsize, OptUsize, ctypes.c_float,
                                   ctypes.POINTER(CEpilogue)]),
    "dr_attention_step_rows": (_I, [_VP, ctypes.c_size_t, ctypes.POINTER(CStepItemRows), ctypes.c_size_t,
                                    ctypes.c_size_t, OptUsize, OptUsize, ctypes.c_float, ctypes.POINTER(CEpilogue)]),
    "dr_qkv_epilogue": (_I, [_VP, _VP, _VP, _VP, _VP, ctypes.c_size_t, ctypes.c_size_t,
                             ctypes.c_size_t, _VP, _VP, _VP, _VP, _VP, _I, ctypes.c_float, _VP]),
    "dr_ctx_set_tuning": (_I, [_VP, _I, _I, _I]),
    "dr_pass_create": (_I, [_VP, c_size_p, _SZ, ctypes.POINTER(_VP)]),
    "dr_pass_set": (_I, [_VP, c_size_p, _SZ]),
    "dr_pass_len": (_SZ, [_VP]),
    "dr_pass_positions": (_I, [_VP, c_size_p, _SZ]),
    "dr_qmatmul": (_I, [_VP, _I, _VP, _SZ, _SZ, _VP, _SZ, _VP, _VP]),
    "dr_qmatmul_expert": (_I, [_VP, _I, _VP, _SZ, _SZ, _SZ, _SZ, _VP, _SZ, _VP, _VP]),
    "dr_quantize_q8k": (_I, [_VP, _VP, _SZ, _SZ, _VP]),
    "dr_quantize_q8_0": (_I, [_VP, _VP, _SZ, _SZ, _VP]),
    "dr_qmatmul_post_norm": (_I, [_VP, _I, _VP, _SZ, _SZ, _VP, _SZ, _VP, _VP, _VP, _F]),
    "dr_pass_destroy": (None, [_VP]),
    "dr_cache_create": (_I, [_VP, _SZ, _SZ, c_size_p, c_size_p, _SZ, ctypes.POINTER(_VP)]),
    "dr_cache_create_layers": (_I, [_VP, _SZ, _SZ, c_size_p, c_size_p, _VP, _SZ, ctypes.POINTER(_VP)]),
    "dr_cache_destroy": (None, [_VP]),
    "dr_cache_set_precision": (_I, [_VP, _SZ, _I]),
    "dr_cache_store": (_I, [_VP, _SZ, _SZ, _VP, _VP, _VP, _VP, _F]),
    "dr_cache_gather": (_I, [_VP, _SZ, _SZ, c_size_p, _SZ, _VP, _VP]),
    "dr_cache_update_seq": (_I, [_VP, _SZ, _VP, _SZ]),
    "dr_cache_split_active": (_I, [_VP, _SZ, _VP, _VP, _SZ, _SZ, c_size_p, c_size_p, c_size_p, c_size_p]),
    "dr_split_active": (_I, [_VP, _VP, _VP, _VP, _SZ, _SZ, _SZ, c_size_p, c_size_p, c_size_p, c_size_p]),
    "dr_cache_set_vicinity": (_I, [_VP, _SZ, _SZ]),
    "dr_cache_update_seq_dev": (_I, [_VP, _SZ, _VP, _SZ]),
    "dr_cache_split_active_dev": (_I, [_VP, _SZ, _VP, _VP, _SZ, _SZ, _VP, _VP, c_size_p, c_size_p]),
    "dr_cache_initialized": (_I, [_VP, _SZ]),
    "dr_attention_cached": (_I, [_VP, _SZ, ctypes.POINTER(CBatchItem), _SZ, _SZ, OptUsize, OptUsize, _F, _VP, _F]),
    "dr_attention_cached_noalloc": (_I, [_VP, _SZ, ctypes.POINTER(CBatchItem), _SZ, _SZ, OptUsize, OptUsize, _F,
                                         _VP, _F]),
    "dr_attention_step": (_I, [_VP, _SZ, ctypes.POINTER(CStepItem), _SZ, _SZ, OptUsize, OptUsize, _F, _VP, _F, _VP, _F]),
    "dr_debug_alloc_count": (ctypes.c_long, []),
    "dr_debug_ring_tiles": (_I, [_SZ, _SZ, _SZ, ctypes.c_longlong, ctypes.c_longlong, ctypes.c_longlong, _SZ,
                                 ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
}


def header_functions(path: pathlib.Path = HEADER_PATH) -> list:
    """Names of every function declared in include/dr_attn.h."""
    text = path.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dr_[a-z0-9_]+)\s*\(", text)))


def load(path: Optional[os.PathLike] = None) -> ctypes.CDLL:
    """Load the HIP library.  Raises if it has not been built: there is no
    fallback implementation."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = pathlib.Path(path) if path else LIB_PATH
    # torch ships its own HIP runtime under the soname libamdhip64.so.7.  When
    # this library was loaded (and bound ROCm's copy of that runtime) before
    # torch in the same process, torch then saw no GPU; loading torch first
    # makes both use torch's runtime, and device pointers and streams are
    # shared between them.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not p.exists():
        raise FileNotFoundError(
            f"{p} not built (run `python -c 'import __graft_entry__ as g; g.build()'`)")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def _check(rc: int) -> None:
    if rc != DR_OK:
        raise DrError(rc, load().dr_last_error().decode())


def device_count() -> int:
    return load().dr_device_count()


def _opt(v: Optional[int]) -> OptUsize:
    return OptUsize(0, 0) if v is None else OptUsize(int(v), 1)


def _usize_array(xs) -> tuple:
    a = np.ascontiguousarray(np.asarray(xs, dtype=np.uint64).reshape(-1)).astype(np.uintp, copy=False)
    return a, (a.ctypes.data_as(c_size_p) if a.size else None), a.size


# --------------------------------------------------------------------------
# attention(): reference-shaped drop-in


@dataclass
class AttnShape:
    """AttnShape (attention.rs:10-27)."""

    nq: int
    nk: int
    n_head: int
    n_head_kv: int
    head_dim: int
    sliding_window: Optional[int] = None
    causal_prefix: Optional[int] = None
    scale: float = 1.0

    def c(self) -> CAttnShape:
        return CAttnShape(self.nq, self.nk, self.n_head, self.n_head_kv, self.head_dim,
                          _opt(self.sliding_window), _opt(self.causal_prefix), self.scale)


@dataclass
class Rows:
    """Rows (attention.rs:65-70): per-row sequence position, optional
    sequence id (empty = all 0) and optional per-row causal prefix (empty =
    the shape's causal_prefix)."""

    pos: Sequence[int]
    seq: Sequence[int] = field(default_factory=tuple)
    prefix: Sequence[int] = field(default_factory=tuple)

    def c(self, keep: list) -> CRows:
        parts = []
        for xs in (self.pos, self.seq, self.prefix):
            arr, ptr, n = _usize_array(xs)
            keep.append(arr)
            parts += [ptr, n]
        return CRows(*parts)


def idpos(n: int) -> Rows:
    """Single-sequence rows at positions 0..n (tests.rs:4-11)."""
    return Rows(pos=range(n))


def attention(out: np.ndarray, q: np.ndarray, k: np.ndarray, v: np.ndarray, s: AttnShape,
              qr: Rows, kr: Rows) -> None:
    """Drop-in for ``attention(out, q, k, v, s, qr, kr)`` (attention.rs:106):
    float32 numpy arrays, ``out`` overwritten in place."""
    lib = load()
    for name, a in (("out", out), ("q", q), ("k", k), ("v", v)):
        if a.dtype != np.float32 or not a.flags.c_contiguous:
            raise TypeError(f"{name} must be a C-contiguous float32 array")
    keep: list = []
    rc = lib.dr_attention(out.ctypes.data, out.size, q.ctypes.data, q.size, k.ctypes.data,
                          k.size, v.ctypes.data, v.size, s.c(), qr.c(keep), kr.c(keep))
    _check(rc)


def split_active(prev_seq: np.ndarray, last_changed: np.ndarray, seq, is_masked, step: int,
                 vicinity: int = 0) -> tuple:
    """Stateless StepCache::split_active (cache.rs:85-114).  ``last_changed``
    (int32) is updated in place.  Returns (active, cached) position lists."""
    lib = load()
    n = len(seq)
    seq_a = np.ascontiguousarray(seq, dtype=np.int32)
    m_a = np.ascontiguousarray(is_masked, dtype=np.uint8)
    prev = np.ascontiguousarray(prev_seq, dtype=np.int32)
    assert last_changed.dtype == np.int32 and last_changed.flags.c_contiguous
    act = np.zeros(max(n, 1), dtype=np.uintp)
    cac = np.zeros(max(n, 1), dtype=np.uintp)
    na, nc = ctypes.c_size_t(), ctypes.c_size_t()
    _check(lib.dr_split_active(prev.ctypes.data, last_changed.ctypes.data, seq_a.ctypes.data,
                               m_a.ctypes.data, n, step, vicinity, act.ctypes.data_as(c_size_p),
                               ctypes.byref(na), cac.ctypes.data_as(c_size_p), ctypes.byref(nc)))
    return [int(x) for x in act[: na.value]], [int(x) for x in cac[: nc.value]]


# --------------------------------------------------------------------------
# device-resident path


class Context:
    """dr_ctx: one device and one HIP stream.  (Passes, RoPE tables and
    caches made on it hold the C context alive, so the garbage collector may
    finalize these objects in any order.)"""

    def __init__(self, device: int = 0):
        self.lib = load()
        h = ctypes.c_void_p()
        _check(self.lib.dr_ctx_create(device, ctypes.byref(h)))
        self.h = h

    def set_stream(self, stream_ptr: int) -> None:
        _check(self.lib.dr_ctx_set_stream(self.h, ctypes.c_void_p(stream_ptr)))

    @property
    def stream(self) -> int:
        return self.lib.dr_ctx_stream(self.h) or 0

    def synchronize(self) -> None:
        _check(self.lib.dr_ctx_synchronize(self.h))

    def set_split(self, n_split: int) -> None:
        _check(self.lib.dr_ctx_set_split(self.h, n_split))

    def set_wave_rows(self, rows: int) -> None:
        _check(self.lib.dr_ctx_set_wave_rows(self.h, rows))

    def set_kernel(self, kernel: int) -> None:
        """KERNEL_AUTO, KERNEL_STAGED, KERNEL_STREAMS or KERNEL_HILO (dr_ctx_set_kernel)."""
        _check(self.lib.dr_ctx_set_kernel(self.h, kernel))

    def set_q_dtype(self, dtype: int) -> None:
        """DTYPE_F32 or DTYPE_BF16: the element type of the Q rows of later
        cached attention calls (dr_ctx_set_q_dtype)."""
        _check(self.lib.dr_ctx_set_q_dtype(self.h, dtype))

    def set_o_dtype(self, dtype: int) -> None:
        """DTYPE_F32 or DTYPE_BF16: the element type of the output rows of
        later cached attention calls (dr_ctx_set_o_dtype)."""
        _check(self.lib.dr_ctx_set_o_dtype(self.h, dtype))

    def set_split_merge(self, in_kernel: bool) -> None:
        """Key splits of the STREAMS kernel merge in-kernel (True, the
        default) or in a second kernel (dr_ctx_set_split_merge)."""
        _check(self.lib.dr_ctx_set_split_merge(self.h, 1 if in_kernel else 0))

    def set_tuning(self, row_blocks: int = 0, key_groups: int = 0, n_split: int = 0) -> None:
        _check(self.lib.dr_ctx_set_tuning(self.h, row_blocks, key_groups, n_split))

    def last_launch(self) -> dict:
        info = CLaunchInfo()
        _check(self.lib.dr_ctx_last_launch(self.h, ctypes.byref(info)))
        return {f: getattr(info, f) for f, _ in CLaunchInfo._fields_}

    def close(self) -> None:
        if self.h:
            self.lib.dr_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Pass:
    """dr_pass: a forward pass's active positions, resident on the device."""

    def __init__(self, ctx: Context, active: Sequence[int]):
        self.ctx = ctx
        arr, ptr, n = _usize_array(active)
        h = ctypes.c_void_p()
        _check(ctx.lib.dr_pass_create(ctx.h, ptr, n, ctypes.byref(h)))
        self.h = h

    def set(self, active: Sequence[int]) -> None:
        arr, ptr, n = _usize_array(active)
        _check(self.ctx.lib.dr_pass_set(self.h, ptr, n))

    def __len__(self) -> int:
        return self.ctx.lib.dr_pass_len(self.h)

    def positions(self) -> list:
        n = len(self)
        out = np.zeros(max(n, 1), dtype=np.uintp)
        _check(self.ctx.lib.dr_pass_positions(self.h, out.ctypes.data_as(c_size_p), out.size))
        return [int(x) for x in out[:n]]

    def close(self) -> None:
        if self.h:
            self.ctx.lib.dr_pass_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Rope:
    """dr_rope: build_rope_cache_ff's (sin, cos) table (ops.rs:396-417) on the device."""

    def __init__(self, ctx: "Context", max_len: int, rope_dim: int, theta: float,
                 freq_factors=None):
        self.ctx = ctx
        ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, np.float32)
        h = ctypes.c_void_p()
        _check(ctx.lib.dr_rope_create(ctx.h, max_len, rope_dim, theta,
                                      ff.ctypes.data if ff is not None else None, ctypes.byref(h)))
        self.h = h
        self.rope_dim = rope_dim

    def close(self) -> None:
        if self.h:
            self.ctx.lib.dr_rope_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def qkv_epilogue(ctx: "Context", p: "Pass", q, k, v, n_head: int, n_head_kv: int, head_dim: int,
                 bq=None, bk=None, bv=None, q_norm_w=None, k_norm_w=None, v_norm: bool = False,
                 eps: float = 1e-6, rope: "Rope | None" = None) -> None:
    """attention_block's Q/K/V epilogue (forward.rs:291-310) in place on device
    rows: bias, QK-norm, Gemma V-norm, RoPE at the pass's positions."""
    _check(ctx.lib.dr_qkv_epilogue(ctx.h, p.h, _ptr(q), _ptr(k), _ptr(v), n_head, n_head_kv,
                                   head_dim, _ptr(bq) or None, _ptr(bk) or None, _ptr(bv) or None,
                                   _ptr(q_norm_w) or None, _ptr(k_norm_w) or None,
                                   1 if v_norm else 0, eps, rope.h if rope is not None else None))


def _ptr(t) -> int:
    """Device pointer of a torch tensor (or an int) -- torch is only used as
    device-memory plumbing."""
    if t is None:
        return 0
    if isinstance(t, int):
        return t
    return t.data_ptr()


class StepCache:
    """dr_step_cache: per-layer bf16 K/V for every position, in HBM."""

    def __init__(self, ctx: Context, n_total: int, n_head_kv: Sequence[int],
                 head_dim: Sequence[int], n_batch: int = 1, precision: Optional[Sequence[int]] = None):
        """precision: per-layer PRECISION_BF16 / PRECISION_HILO
        (dr_cache_create_layers); None: every layer bf16 (dr_cache_create)."""
        self.ctx = ctx
        hkv, hkv_p, n_layer = _usize_array(n_head_kv)
        hd, hd_p, n2 = _usize_array(head_dim)
        assert n2 == n_layer
        h = ctypes.c_void_p()
        if precision is None:
            _check(ctx.lib.dr_cache_create(ctx.h, n_total, n_layer, hkv_p, hd_p, n_batch,
                                           ctypes.byref(h)))
        else:
            prec = np.ascontiguousarray(precision, dtype=np.int32)
            assert prec.size == n_layer
            _check(ctx.lib.dr_cache_create_layers(ctx.h, n_total, n_layer, hkv_p, hd_p, prec.ctypes.data,
                                                  n_batch, ctypes.byref(h)))
        self.h = h
        self.n_total = n_total
        self.n_batch = n_batch

    def set_precision(self, layer: int, precision: int) -> None:
        """PRECISION_BF16 or PRECISION_HILO for one layer (dr_cache_set_precision):
        HILO keeps K's lo half and gives the layer f32-accurate scores."""
        _check(self.ctx.lib.dr_cache_set_precision(self.h, layer, precision))

    def store(self, layer: int, p: Pass, k, v, k_norm_w=None, eps: float = 1e-6, batch: int = 0):
        _check(self.ctx.lib.dr_cache_store(self.h, layer, batch, p.h, _ptr(k), _ptr(v),
                                           _ptr(k_norm_w) or None, eps))

    def gather(self, layer: int, positions: Sequence[int], out_k, out_v, batch: int = 0):
        arr, ptr, n = _usize_array(positions)
        _check(self.ctx.lib.dr_cache_gather(self.h, layer, batch, ptr, n, _ptr(out_k),
                                            _ptr(out_v)))

    def update_seq(self, seq, batch: int = 0) -> None:
        a = np.ascontiguousarray(seq, dtype=np.int32)
        _check(self.ctx.lib.dr_cache_update_seq(self.h, batch, a.ctypes.data, a.size))

    def split_active(self, seq, is_masked, step: int, batch: int = 0) -> tuple:
        n = len(seq)
        seq_a = np.ascontiguousarray(seq, dtype=np.int32)
        m_a = np.ascontiguousarray(is_masked, dtype=np.uint8)
        act = np.zeros(max(n, 1), dtype=np.uintp)
        cac = np.zeros(max(n, 1), dtype=np.uintp)
        na, nc = ctypes.c_size_t(), ctypes.c_size_t()
        _check(self.ctx.lib.dr_cache_split_active(
            self.h, batch, seq_a.ctypes.data, m_a.ctypes.data, n, step,
            act.ctypes.data_as(c_size_p), ctypes.byref(na), cac.ctypes.data_as(c_size_p),
            ctypes.byref(nc)))
        return [int(x) for x in act[: na.value]], [int(x) for x in cac[: nc.value]]

    def update_seq_dev(self, seq, batch: int = 0) -> None:
        """update_seq from a device int32 tensor of n_total tokens."""
        _check(self.ctx.lib.dr_cache_update_seq_dev(self.h, batch, _ptr(seq), self.n_total))

    def split_active_dev(self, seq, is_masked, n: int, step: int, active: Pass, cached: Pass,
                         batch: int = 0) -> tuple:
        """split_active on the device (cache.rs:85-114): seq (int32) and
        is_masked (uint8) are device tensors of n entries; the active and cached
        positions land in the two passes.  Returns (n_active, n_cached)."""
        na, nc = ctypes.c_size_t(), ctypes.c_size_t()
        _check(self.ctx.lib.dr_cache_split_active_dev(
            self.h, batch, _ptr(seq), _ptr(is_masked), n, step, active.h, cached.h,
            ctypes.byref(na), ctypes.byref(nc)))
        return na.value, nc.value

    def set_vicinity(self, vicinity: int, batch: int = 0) -> None:
        _check(self.ctx.lib.dr_cache_set_vicinity(self.h, batch, vicinity))

    def initialized(self, batch: int = 0) -> bool:
        return bool(self.ctx.lib.dr_cache_initialized(self.h, batch))

    def attention(self, layer: int, items: Sequence[tuple], n_head: int,
                  sliding_window: Optional[int] = None, causal_prefix: Optional[int] = None,
                  scale: float = 1.0, q_norm_w=None, q_norm_eps: float = 1e-6,
                  noalloc: bool = False) -> None:
        """items: sequence of (q, out, Pass) per batch slot (device tensors).
        noalloc: dr_attention_cached_noalloc (the library's fixed device
        scratch instead of the context's workspace)."""
        arr = (CBatchItem * len(items))()
        for i, (q, out, p) in enumerate(items):
            arr[i] = CBatchItem(_ptr(q), _ptr(out), p.h)
        fn = self.ctx.lib.dr_attention_cached_noalloc if noalloc else self.ctx.lib.dr_attention_cached
        _check(fn(self.h, layer, arr, len(items), n_head, _opt(sliding_window), _opt(causal_prefix),
                  scale, _ptr(q_norm_w) or None, q_norm_eps))

    def step(self, layer: int, items: Sequence[tuple], n_head: int,
             sliding_window: Optional[int] = None, causal_prefix: Optional[int] = None,
             scale: float = 1.0, q_norm_w=None, q_norm_eps: float = 1e-6, k_norm_w=None,
             k_norm_eps: float = 1e-6) -> None:
        """One denoise-step layer: items = (q, out, Pass, k, v) per batch slot
        (device tensors; k/v the pass's active rows).  Stores k/v into the
        cache and runs the attention (one kernel where the pass allows)."""
        arr = (CStepItem * len(items))()
        for i, (q, out, p, k, v) in enumerate(items):
            arr[i] = CStepItem(_ptr(q), _ptr(out), p.h, _ptr(k), _ptr(v))
        _check(self.ctx.lib.dr_attention_step(
            self.h, layer, arr, len(items), n_head, _opt(sliding_window), _opt(causal_prefix),
            scale, _ptr(q_norm_w) or None, q_norm_eps, _ptr(k_norm_w) or None, k_norm_eps))

    def step_epi(self, layer: int, items: Sequence[tuple], n_head: int,
                 sliding_window: Optional[int] = None, causal_prefix: Optional[int] = None,
                 scale: float = 1.0, bq=None, bk=None, bv=None, q_norm_w=None, k_norm_w=None,
                 v_norm: bool = False, eps: float = 1e-6, rope: "Rope | None" = None) -> None:
        """step() with the Q/K/V epilogue (forward.rs:291-310) folded into the
        store and the attention; the item buffers are only read."""
        arr = (CStepItem * len(items))()
        for i, (q, out, p, k, v) in enumerate(items):
            arr[i] = CStepItem(_ptr(q), _ptr(out), p.h, _ptr(k), _ptr(v))
        epi = CEpilogue(_ptr(bq) or None, _ptr(bk) or None, _ptr(bv) or None,
                        _ptr(q_norm_w) or None, _ptr(k_norm_w) or None, 1 if v_norm else 0, eps,
                        rope.h.value if rope is not None else None)
        _check(self.ctx.lib.dr_attention_step_epi(
            self.h, layer, arr, len(items), n_head, _opt(sliding_window), _opt(causal_prefix),
            scale, ctypes.byref(epi)))

    def step_rows(self, layer: int, items: Sequence[tuple], n_head: int, q_stride: int, kv_stride: int,
                  sliding_window: Optional[int] = None, causal_prefix: Optional[int] = None,
                  scale: float = 1.0, bq=None, bk=None, bv=None, q_norm_w=None, k_norm_w=None,
                  v_norm: bool = False, eps: float = 1e-6, rope: "Rope | None" = None) -> None:
        """step_epi() on strided rows (dr_attention_step_rows): items = (q, out,
        Pass, k, v) with q / k / v device addresses (ints or tensors) whose rows
        are q_stride / kv_stride floats apart, e.g. the Q, K and V parts of
        fused QKV rows."""
        arr = (CStepItemRows * len(items))()
        for i, (q, out, p, k, v) in enumerate(items):
            arr[i] = CStepItemRows(_ptr(q), _ptr(out), p.h, _ptr(k), _ptr(v), q_stride, kv_stride)
        epi = CEpilogue(_ptr(bq) or None, _ptr(bk) or None, _ptr(bv) or None,
                        _ptr(q_norm_w) or None, _ptr(k_norm_w) or None, 1 if v_norm else 0, eps,
                        rope.h.value if rope is not None else None)
        _check(self.ctx.lib.dr_attention_step_rows(
            self.h, layer, arr, len(items), n_head, _opt(sliding_window), _opt(causal_prefix),
            scale, ctypes.byref(epi)))

    def close(self) -> None:
        if self.h:
            self.ctx.lib.dr_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


WTYPE_Q4K, WTYPE_Q6K = 12, 14
WTYPE_Q4_0, WTYPE_Q5_0, WTYPE_Q8_0 = 2, 6, 8


def qmatmul(ctx: Context, wtype: int, w, rows: int, cols: int, act, n: int, out,
            residual=None) -> None:
    """Wo on k-quant weights (matmul.rs:94-148) + residual_add (ops.rs:365-370):
    device tensors; w holds rows * cols/256 GGUF blocks."""
    _check(ctx.lib.dr_qmatmul(ctx.h, wtype, _ptr(w), rows, cols, _ptr(act), n, _ptr(out),
                              _ptr(residual) or None))


def qmatmul_expert(ctx: Context, wtype: int, w, n_expert: int, expert: int, rows: int, cols: int,
                   act, n: int, out, residual=None) -> None:
    """ExpertMat::forward_expert (matmul.rs:176-213): qmatmul on one expert's
    slice of a [n_expert][rows][cols] block stack."""
    _check(ctx.lib.dr_qmatmul_expert(ctx.h, wtype, _ptr(w), n_expert, expert, rows, cols, _ptr(act), n,
                                     _ptr(out), _ptr(residual) or None))


def quantize_q8k(ctx: Context, act, n: int, cols: int, out) -> None:
    """quantize_rows_q8_k (kernels.rs:79-122) into n * cols/256 BlockQ8K
    (292 bytes each) at device pointer / tensor out."""
    _check(ctx.lib.dr_quantize_q8k(ctx.h, _ptr(act), n, cols, _ptr(out)))


def alloc_count() -> int:
    """Device and pinned host allocations the library has made in this
    process (dr_debug_alloc_count)."""
    return int(load().dr_debug_alloc_count())


def ring_tiles(head_dim: int, nk: int, cap: int, window: Optional[int], qmin: int, qmax: int,
               n_split: int) -> tuple:
    """(min tile, max tile, partition ok) over every DMA the stream kernel's
    waves issue for one workgroup (dr_debug_ring_tiles); host-only."""
    lo, hi, ok = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _check(load().dr_debug_ring_tiles(head_dim, nk, cap, -1 if window is None else window, qmin, qmax,
                                      n_split, ctypes.byref(lo), ctypes.byref(hi), ctypes.byref(ok)))
    return lo.value, hi.value, bool(ok.value)


def qmatmul_post_norm(ctx: Context, wtype: int, w, rows: int, cols: int, act, n: int, out, norm_w,
                      eps: float, residual=None) -> None:
    """Wo, Gemma's post-attention RMSNorm of each output row, then the
    residual (forward.rs:346-350; dr_qmatmul_post_norm)."""
    _check(ctx.lib.dr_qmatmul_post_norm(ctx.h, wtype, _ptr(w), rows, cols, _ptr(act), n, _ptr(out),
                                        _ptr(residual) or None, _ptr(norm_w), eps))


def quantize_q8_0(ctx: Context, act, n: int, cols: int, out) -> None:
    """quantize_row_q8_0 (matmul.rs:73-82) into n * cols/32 BlockQ8_0
    (34 bytes each) at device pointer / tensor out."""
    _check(ctx.lib.dr_quantize_q8_0(ctx.h, _ptr(act), n, cols, _ptr(out)))

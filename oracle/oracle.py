"""ctypes binding of the CPU oracle (oracle/attn_oracle.c).

TEST INFRASTRUCTURE ONLY: a C restatement of diffuse-rs's attention path
(src/model/attention.rs, ops.rs, cache.rs) used as the parity checker by
tests/, __graft_entry__.smoke() and as the timed CPU baseline in bench.py.
The product library (diffuse-rs_amd/lib/libdr_attn.so) never calls it.

The API mirrors the reference: ``attention(out, q, k, v, s, qr, kr)`` with
the same AttnShape / Rows meaning (attention.rs:10-27, 65-70).
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess
from typing import Optional, Sequence

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_attn.so"

c_size_p = ctypes.POINTER(ctypes.c_size_t)
c_float_p = ctypes.POINTER(ctypes.c_float)


class OrShape(ctypes.Structure):
    _fields_ = [
        ("nq", ctypes.c_size_t),
        ("nk", ctypes.c_size_t),
        ("n_head", ctypes.c_size_t),
        ("n_head_kv", ctypes.c_size_t),
        ("head_dim", ctypes.c_size_t),
        ("window", ctypes.c_size_t),
        ("has_window", ctypes.c_int),
        ("prefix", ctypes.c_size_t),
        ("has_prefix", ctypes.c_int),
        ("scale", ctypes.c_float),
    ]


class OrRows(ctypes.Structure):
    _fields_ = [("pos", c_size_p), ("seq", c_size_p), ("prefix", c_size_p)]


_LIB: Optional[ctypes.CDLL] = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    P = ctypes.c_void_p
    row_sig = [P, P, P, P, ctypes.POINTER(OrShape), ctypes.POINTER(OrRows),
               ctypes.POINTER(OrRows), ctypes.c_size_t, ctypes.c_size_t]
    lib.or_attention_row_scalar.argtypes = row_sig
    lib.or_attention_row_avx2.argtypes = row_sig
    lib.or_attention.argtypes = [P, P, P, P, ctypes.POINTER(OrShape), ctypes.POINTER(OrRows),
                                 ctypes.POINTER(OrRows), ctypes.c_int, ctypes.c_int]
    lib.or_visible.argtypes = [ctypes.c_size_t] * 4 + [ctypes.c_int, ctypes.c_size_t,
                                                       ctypes.c_int, ctypes.c_size_t]
    lib.or_visible.restype = ctypes.c_int
    lib.or_max_threads.restype = ctypes.c_int
    lib.or_rms_norm_inplace.argtypes = [P, P, ctypes.c_size_t, ctypes.c_float]
    lib.or_norm_heads.argtypes = [P, ctypes.c_size_t, P, ctypes.c_size_t, ctypes.c_float]
    lib.or_rms_norm_noscale.argtypes = [P, ctypes.c_size_t, ctypes.c_float]
    lib.or_add_bias.argtypes = [P, P, ctypes.c_size_t, ctypes.c_size_t]
    lib.or_rope_table.argtypes = [P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_float, P]
    lib.or_rotate_rows.argtypes = [P, P, c_size_p, ctypes.c_size_t, ctypes.c_size_t,
                                   ctypes.c_size_t, ctypes.c_size_t]
    lib.or_cache_store.argtypes = [P, P, ctypes.c_size_t, c_size_p, ctypes.c_size_t, P, P]
    lib.or_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.or_f16_to_f32.restype = ctypes.c_float
    lib.or_quantize_q8k.argtypes = [P, ctypes.c_size_t, ctypes.c_size_t, P]
    lib.or_dequant_q4k.argtypes = [P, ctypes.c_size_t, P]
    lib.or_dequant_q6k.argtypes = [P, ctypes.c_size_t, P]
    lib.or_vec_dot_q4k_q8k.argtypes = [P, P, ctypes.c_size_t]
    lib.or_vec_dot_q4k_q8k.restype = ctypes.c_float
    lib.or_vec_dot_q6k_q8k.argtypes = [P, P, ctypes.c_size_t]
    lib.or_vec_dot_q6k_q8k.restype = ctypes.c_float
    lib.or_qmatmul.argtypes = [ctypes.c_int, P, ctypes.c_size_t, ctypes.c_size_t, P, ctypes.c_size_t,
                               P, P]
    for nm in ("or_dequant_q4_0", "or_dequant_q5_0", "or_dequant_q8_0"):
        getattr(lib, nm).argtypes = [P, ctypes.c_size_t, P]
    lib.or_f32_to_f16.argtypes = [ctypes.c_float]
    lib.or_f32_to_f16.restype = ctypes.c_uint16
    lib.or_quantize_q8_0.argtypes = [P, ctypes.c_size_t, ctypes.c_size_t, P]
    for nm in ("or_vec_dot_q4_0_q8_0", "or_vec_dot_q5_0_q8_0", "or_vec_dot_q8_0_q8_0"):
        getattr(lib, nm).argtypes = [P, P, ctypes.c_size_t]
        getattr(lib, nm).restype = ctypes.c_float
    lib.or_post_norm_residual.argtypes = [P, P, P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_float]
    lib.or_cache_gather.argtypes = [P, P, ctypes.c_size_t, c_size_p, ctypes.c_size_t, P, P]
    lib.or_split_active.argtypes = [P, P, P, P, ctypes.c_size_t, ctypes.c_size_t,
                                    ctypes.c_size_t, c_size_p, c_size_p, c_size_p, c_size_p]
    _LIB = lib
    return lib


def _shape(s) -> OrShape:
    return OrShape(s.nq, s.nk, s.n_head, s.n_head_kv, s.head_dim,
                   0 if s.sliding_window is None else s.sliding_window,
                   int(s.sliding_window is not None),
                   0 if s.causal_prefix is None else s.causal_prefix,
                   int(s.causal_prefix is not None), s.scale)


def _arr(xs, keep):
    if xs is None or len(xs) == 0:
        return None
    a = np.ascontiguousarray(np.asarray(xs, dtype=np.uint64)).astype(np.uintp, copy=False)
    keep.append(a)
    return a.ctypes.data_as(c_size_p)


def _rows(r, n: int, keep) -> OrRows:
    """Rows -> OrRows.  A ``seq`` shorter than the rows is padded with 0, as
    Rows::seq_at (attention.rs:73-76) reads missing ids as 0."""
    seq = None
    if r.seq is not None and len(r.seq) > 0:
        seq = list(r.seq)[:n] + [0] * max(0, n - len(r.seq))
    return OrRows(_arr(r.pos, keep), _arr(seq, keep), _arr(r.prefix, keep))


def _f32(a: np.ndarray) -> np.ndarray:
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a


def attention(out: np.ndarray, q: np.ndarray, k: np.ndarray, v: np.ndarray, s, qr, kr,
              threads: int = 0, avx2: bool = True) -> None:
    """attention() (attention.rs:106): fills ``out`` in place."""
    lib = load()
    assert out.size == s.nq * s.n_head * s.head_dim
    assert len(qr.pos) == s.nq and len(kr.pos) == s.nk
    keep: list = []
    sh = _shape(s)
    lib.or_attention(_f32(out).ctypes.data, _f32(q).ctypes.data, _f32(k).ctypes.data,
                     _f32(v).ctypes.data, ctypes.byref(sh), ctypes.byref(_rows(qr, s.nq, keep)),
                     ctypes.byref(_rows(kr, s.nk, keep)), threads, int(avx2))


def attention_row(kind: str, out, q, k, v, s, qr, kr, head: int, i: int) -> None:
    """One (head, query) row via attention_row_scalar or attention_row_avx2."""
    lib = load()
    keep: list = []
    fn = lib.or_attention_row_avx2 if kind == "avx2" else lib.or_attention_row_scalar
    sh = _shape(s)
    fn(_f32(out).ctypes.data, _f32(q).ctypes.data, _f32(k).ctypes.data, _f32(v).ctypes.data,
       ctypes.byref(sh), ctypes.byref(_rows(qr, s.nq, keep)), ctypes.byref(_rows(kr, s.nk, keep)),
       head, i)


def visible(qpos, kpos, qseq, kseq, window=None, prefix=None) -> bool:
    return bool(load().or_visible(qpos, kpos, qseq, kseq, int(window is not None), window or 0,
                                  int(prefix is not None), prefix or 0))


def max_threads() -> int:
    return load().or_max_threads()


def rms_norm_inplace(x: np.ndarray, w: np.ndarray, eps: float) -> None:
    load().or_rms_norm_inplace(_f32(x).ctypes.data, _f32(w).ctypes.data, x.size, eps)


def norm_heads(x: np.ndarray, w: np.ndarray, eps: float) -> None:
    load().or_norm_heads(_f32(x).ctypes.data, x.size, _f32(w).ctypes.data, w.size, eps)


def rms_norm_noscale(x: np.ndarray, eps: float) -> None:
    load().or_rms_norm_noscale(_f32(x).ctypes.data, x.size, eps)


def add_bias(x: np.ndarray, b: np.ndarray, n: int) -> None:
    load().or_add_bias(_f32(x).ctypes.data, _f32(b).ctypes.data, b.size, n)


def rope_table(max_len: int, rope_dim: int, theta: float, freq_factors=None) -> np.ndarray:
    """(max_len, rope_dim/2, 2) float32: (sin, cos) per position and pair."""
    out = np.zeros((max_len, rope_dim // 2, 2), np.float32)
    ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, np.float32)
    load().or_rope_table(out.ctypes.data, max_len, rope_dim, ctypes.c_float(theta),
                         ff.ctypes.data if ff is not None else None)
    return out


def rotate_rows(x: np.ndarray, table: np.ndarray, positions: Sequence[int], heads: int, hd: int,
                rot: int) -> None:
    keep: list = []
    t = np.ascontiguousarray(table, np.float32)
    load().or_rotate_rows(_f32(x).ctypes.data, t.ctypes.data, _arr(positions, keep), len(positions),
                          heads, hd, rot)


def cache_store(ck: np.ndarray, cv: np.ndarray, stride: int, positions: Sequence[int],
                k: np.ndarray, v: np.ndarray) -> None:
    keep: list = []
    load().or_cache_store(_f32(ck).ctypes.data, _f32(cv).ctypes.data, stride,
                          _arr(positions, keep), len(positions), _f32(k).ctypes.data,
                          _f32(v).ctypes.data)


def cache_gather(ck, cv, stride: int, positions: Sequence[int], out_k, out_v) -> None:
    keep: list = []
    load().or_cache_gather(_f32(ck).ctypes.data, _f32(cv).ctypes.data, stride,
                           _arr(positions, keep), len(positions), _f32(out_k).ctypes.data,
                           _f32(out_v).ctypes.data)


def split_active(prev_seq, last_changed: np.ndarray, seq, is_masked, step: int,
                 vicinity: int = 0) -> tuple:
    n = len(seq)
    prev = np.ascontiguousarray(prev_seq, dtype=np.int32)
    seq_a = np.ascontiguousarray(seq, dtype=np.int32)
    m_a = np.ascontiguousarray(is_masked, dtype=np.uint8)
    act = np.zeros(max(n, 1), dtype=np.uintp)
    cac = np.zeros(max(n, 1), dtype=np.uintp)
    na, nc = ctypes.c_size_t(), ctypes.c_size_t()
    load().or_split_active(prev.ctypes.data, last_changed.ctypes.data, seq_a.ctypes.data,
                           m_a.ctypes.data, n, step, vicinity, act.ctypes.data_as(c_size_p),
                           ctypes.byref(na), cac.ctypes.data_as(c_size_p), ctypes.byref(nc))
    return [int(x) for x in act[: na.value]], [int(x) for x in cac[: nc.value]]


# ---- quantized matmul (src/kernels.rs, src/model/matmul.rs) -----------------

QK_K = 256
Q4K_BYTES, Q6K_BYTES = 144, 210
WTYPE_Q4K, WTYPE_Q6K = 12, 14  # GGML type ids
# the legacy 32-value block types (GGML ids) and their block bytes
QK0 = 32
WTYPE_Q4_0, WTYPE_Q5_0, WTYPE_Q8_0 = 2, 6, 8
LEGACY_BYTES = {WTYPE_Q4_0: 18, WTYPE_Q5_0: 22, WTYPE_Q8_0: 34}
# Q8_0 block, 34 bytes (f16 d, int8 qs[32])
Q80_DTYPE = np.dtype([("d", "<u2"), ("qs", "i1", (QK0,))])
assert Q80_DTYPE.itemsize == 34
# Q8_K block, 292 bytes (src/kernels.rs:37-41)
Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", (QK_K,)), ("bsums", "<i2", (QK_K // 16,))])
assert Q8K_DTYPE.itemsize == 292


def f16_to_f32(h: int) -> float:
    return float(load().or_f16_to_f32(h))


def quantize_q8k(x: np.ndarray, n: int, cols: int) -> np.ndarray:
    """quantize_rows_q8_k: n rows of cols f32 -> n * cols / 256 Q8_K blocks."""
    src = np.ascontiguousarray(x, np.float32)
    out = np.zeros(n * cols // QK_K, Q8K_DTYPE)
    load().or_quantize_q8k(src.ctypes.data, n, cols, out.ctypes.data)
    return out


def dequant(wtype: int, blocks: np.ndarray, nb: int) -> np.ndarray:
    """nb blocks of wtype to f32 (QK_K values per k-quant block, QK0 per
    legacy block)."""
    b = np.ascontiguousarray(blocks, np.uint8)
    lib = load()
    fn = {WTYPE_Q4K: lib.or_dequant_q4k, WTYPE_Q6K: lib.or_dequant_q6k, WTYPE_Q4_0: lib.or_dequant_q4_0,
          WTYPE_Q5_0: lib.or_dequant_q5_0, WTYPE_Q8_0: lib.or_dequant_q8_0}[wtype]
    out = np.zeros(nb * (QK0 if wtype in LEGACY_BYTES else QK_K), np.float32)
    fn(b.ctypes.data, nb, out.ctypes.data)
    return out


def f32_to_f16(x: float) -> int:
    return int(load().or_f32_to_f16(x))


def quantize_q8_0(x: np.ndarray, n: int, cols: int) -> np.ndarray:
    """quantize_row_q8_0: n rows of cols f32 -> n * cols / 32 Q8_0 blocks."""
    src = np.ascontiguousarray(x, np.float32)
    out = np.zeros(n * cols // QK0, Q80_DTYPE)
    load().or_quantize_q8_0(src.ctypes.data, n, cols, out.ctypes.data)
    return out


def vec_dot_legacy(wtype: int, x_blocks: np.ndarray, y_blocks: np.ndarray, nb: int) -> float:
    """Q4_0 / Q5_0 / Q8_0 weight blocks . Q8_0 activation blocks."""
    xb = np.ascontiguousarray(x_blocks, np.uint8)
    yb = np.ascontiguousarray(y_blocks, Q80_DTYPE)
    lib = load()
    fn = {WTYPE_Q4_0: lib.or_vec_dot_q4_0_q8_0, WTYPE_Q5_0: lib.or_vec_dot_q5_0_q8_0,
          WTYPE_Q8_0: lib.or_vec_dot_q8_0_q8_0}[wtype]
    return float(fn(xb.ctypes.data, yb.ctypes.data, nb))


def post_norm_residual(cur: np.ndarray, w: np.ndarray, residual, n: int, e: int, eps: float) -> None:
    """Gemma's post-attention norm then residual add (forward.rs:346-350), in place."""
    assert cur.dtype == np.float32 and cur.flags.c_contiguous
    res = None if residual is None else np.ascontiguousarray(residual, np.float32)
    ww = np.ascontiguousarray(w, np.float32)
    load().or_post_norm_residual(cur.ctypes.data, ww.ctypes.data, None if res is None else res.ctypes.data, n, e,
                                 eps)


def vec_dot(wtype: int, x_blocks: np.ndarray, y_blocks: np.ndarray, nb: int) -> float:
    xb = np.ascontiguousarray(x_blocks, np.uint8)
    yb = np.ascontiguousarray(y_blocks, Q8K_DTYPE)
    fn = load().or_vec_dot_q4k_q8k if wtype == WTYPE_Q4K else load().or_vec_dot_q6k_q8k
    return float(fn(xb.ctypes.data, yb.ctypes.data, nb))


def qmatmul(wtype: int, w: np.ndarray, rows: int, cols: int, act: np.ndarray, n: int,
            residual: "np.ndarray | None" = None) -> np.ndarray:
    """native_matmul + residual_add: out[t, r] = vec_dot(w row r, q8k(act row t)) (+ residual)."""
    wb = np.ascontiguousarray(w, np.uint8)
    a = np.ascontiguousarray(act, np.float32)
    out = np.zeros(n * rows, np.float32)
    res = None if residual is None else np.ascontiguousarray(residual, np.float32)
    load().or_qmatmul(wtype, wb.ctypes.data, rows, cols, a.ctypes.data, n, out.ctypes.data,
                      None if res is None else res.ctypes.data)
    return out

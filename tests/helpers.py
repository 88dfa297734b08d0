"""Shared test helpers: input generators, a float64 brute-force attention and
the benchmark configurations.

The brute force is deliberately a different algorithm from the reference's
online softmax (attention.rs:289-331): it materialises the full visibility
matrix and score matrix in float64 and normalises in three passes, like the
reference's own test oracle ``softmax_row_scalar`` (ops.rs:267-280) used by
``test_attention_matches_naive_reference`` (tests.rs:154-186).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np


@dataclass
class Shape:
    """Same fields as AttnShape (attention.rs:10-27)."""

    nq: int
    nk: int
    n_head: int
    n_head_kv: int
    head_dim: int
    sliding_window: Optional[int] = None
    causal_prefix: Optional[int] = None
    scale: float = 1.0


@dataclass
class RowsSpec:
    pos: Sequence[int]
    seq: Sequence[int] = ()
    prefix: Sequence[int] = ()


def closed_form(n: int, mul: int, mod: int, off: float, div: float) -> np.ndarray:
    """((x*mul % mod) - off) / div for x in 0..n -- the input family of the
    reference's attention tests (tests.rs:80-82, 108-110, 124-128, 159-161)."""
    x = np.arange(n, dtype=np.int64)
    return (((x * mul) % mod).astype(np.float32) - np.float32(off)) / np.float32(div)


def visibility(s: Shape, qr: RowsSpec, kr: RowsSpec) -> np.ndarray:
    """[nq, nk] bool: the key/query visibility rules stated in the
    reference's AttnShape and Rows docs (attention.rs:17-24, 29-35, 59-64)."""
    qpos = np.asarray(qr.pos, dtype=np.int64)[:, None]
    kpos = np.asarray(kr.pos, dtype=np.int64)[None, :]

    def ids(r, n):
        a = np.zeros(n, dtype=np.int64)
        if len(r.seq):
            m = min(n, len(r.seq))
            a[:m] = np.asarray(r.seq, dtype=np.int64)[:m]
        return a

    vis = ids(qr, s.nq)[:, None] == ids(kr, s.nk)[None, :]
    if s.sliding_window is not None:
        vis &= np.abs(qpos - kpos) < s.sliding_window
    if len(qr.prefix):
        pref = np.asarray(qr.prefix, dtype=np.int64)[:, None]
    elif s.causal_prefix is not None:
        pref = np.full((s.nq, 1), s.causal_prefix, dtype=np.int64)
    else:
        pref = None
    if pref is not None:
        prompt_row = qpos < pref
        vis &= ~prompt_row | (kpos <= qpos)
    return vis


def brute_force(q, k, v, s: Shape, qr: RowsSpec, kr: RowsSpec) -> np.ndarray:
    """float64 three-pass attention.  Rows with no visible key are NaN."""
    h, hkv, hd = s.n_head, s.n_head_kv, s.head_dim
    Q = np.asarray(q, dtype=np.float64).reshape(s.nq, h, hd)
    K = np.asarray(k, dtype=np.float64).reshape(s.nk, hkv, hd)
    V = np.asarray(v, dtype=np.float64).reshape(s.nk, hkv, hd)
    vis = visibility(s, qr, kr)
    out = np.full((s.nq, h, hd), np.nan)
    group = h // hkv
    live = vis.any(axis=1)
    for head in range(h):
        g = head // group
        sc = (Q[:, head] @ K[:, g].T) * float(np.float32(s.scale))
        sc = np.where(vis, sc, -np.inf)
        m = np.max(sc, axis=1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        p = np.where(vis, np.exp(sc - m), 0.0)
        l = p.sum(axis=1)
        o = (p @ V[:, g]) / np.where(l > 0, l, 1.0)[:, None]
        out[live, head] = o[live]
    return out.reshape(s.nq, h * hd)


def make_input(spec: dict, n: int) -> np.ndarray:
    """A golden-case input: explicit values or closed_form(n, *gen)."""
    if "values" in spec:
        a = np.asarray(spec["values"], dtype=np.float32)
        assert a.size == n
        return a
    return closed_form(n, *spec["gen"])


def materialise(c: dict):
    """(shape, qrows, krows, q, k, v) of a case from tests/golden/cases.json."""
    s = Shape(**c["shape"])
    qr = RowsSpec(**c["qrows"])
    kr = RowsSpec(**c["krows"])
    q = make_input(c["q"], s.nq * s.n_head * s.head_dim)
    k = make_input(c["k"], s.nk * s.n_head_kv * s.head_dim)
    v = make_input(c["v"], s.nk * s.n_head_kv * s.head_dim)
    return s, qr, kr, q, k, v


def golden_cases() -> list:
    """[(case dict, expected float64 [nq, h*hd])] from tests/golden/."""
    import json
    import pathlib

    d = pathlib.Path(__file__).resolve().parent / "golden"
    cases = json.loads((d / "cases.json").read_text())
    exp = np.load(d / "expected.npz")
    return [(c, exp[c["name"]]) for c in cases]


def rms_norm_f64(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """Per-head RMSNorm in float64 over the last axis (ops.rs:106-114)."""
    x64 = np.asarray(x, dtype=np.float64)
    r = np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + eps)
    return x64 / r * np.asarray(w, dtype=np.float64)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


LOG2E = 1.4426950408889634


def as_kernel_sees(q, k, v, scale: float):
    """The operands the bf16 path multiplies, widened back to f32: K and V as
    stored in the bf16 cache, Q as bf16(q * scale * log2 e) / (scale * log2 e).
    The oracle on these isolates the kernel's own arithmetic (bf16 P, f32
    accumulation) from the input rounding."""
    c = np.float32(np.float32(scale) * np.float32(LOG2E))
    qb = (bf16_round(np.asarray(q, np.float32) * c).astype(np.float64) / float(c)).astype(np.float32)
    return qb, bf16_round(k), bf16_round(v)


def normal(rng: np.random.Generator, *shape) -> np.ndarray:
    return rng.standard_normal(shape, dtype=np.float32)


def err_stats(got: np.ndarray, want: np.ndarray) -> tuple:
    """(max-abs, mean-abs) error over finite expected entries; NaN positions
    must coincide."""
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    want = np.asarray(want, dtype=np.float64).reshape(-1)
    nan_w, nan_g = np.isnan(want), np.isnan(got)
    assert np.array_equal(nan_w, nan_g), "NaN pattern differs"
    d = np.abs(got[~nan_w] - want[~nan_w])
    if d.size == 0:
        return 0.0, 0.0
    return float(d.max()), float(d.mean())


# Tolerance of the bf16-MFMA path against the f32 reference (BASELINE.json
# north_star): max-abs <= 1e-2 and mean-abs <= 1e-3.
TOL_MAX = 1e-2
TOL_MEAN = 1e-3


@dataclass
class Config:
    """One BASELINE.json config as a cached denoise-step attention problem."""

    name: str
    n_head: int
    n_head_kv: int
    head_dim: int
    n_prompt: int
    n_canvas: int
    batch: int = 1
    window: Optional[int] = None
    qk_norm: bool = False
    scale: Optional[float] = None

    @property
    def n_total(self) -> int:
        return self.n_prompt + self.n_canvas

    @property
    def attn_scale(self) -> float:
        return self.scale if self.scale is not None else 1.0 / math.sqrt(self.head_dim)

    def visible_keys(self) -> int:
        """sum over canvas queries of |visible keys| (one head, one batch)."""
        total = 0
        for qp in range(self.n_prompt, self.n_total):
            if self.window is None:
                total += self.n_total
            else:
                lo = max(0, qp - self.window + 1)
                hi = min(self.n_total, qp + self.window)
                total += hi - lo
        return total

    def flops(self) -> float:
        """4 * h * hd * sum_q |visible(q)| per batch slot (QK^T + PV)."""
        return 4.0 * self.n_head * self.head_dim * self.visible_keys() * self.batch


CONFIGS = {
    # 64 prompt + 64 canvas, all 128 rows are queries (no cache)
    "C1": Config("llada8b_128x128", 32, 32, 128, 0, 128),
    # the headline denoise step
    "C2": Config("llada8b_step_512c+256q", 32, 32, 128, 512, 256),
    "C3": Config("dream7b_gqa_cfg_1024c+256q_b2", 28, 4, 128, 1024, 256, batch=2),
    "C4": Config("lladamoe_qknorm_2048c+512q", 16, 16, 128, 2048, 512, qk_norm=True),
    "C5S": Config("gemma_sliding_w1024_4096c+256q", 16, 8, 256, 4096, 256, window=1024),
    "C5G": Config("gemma_global_4096c+256q", 16, 8, 256, 4096, 256),
}

# Shapes outside BASELINE.json's configs that the path also serves.
# G512: a real DiffusionGemma global layer (docs/diffusiongemma.md:11-12): 16
# query heads over 2 KV heads at head dim 512, full attention, C5's context.
EXTRA_CONFIGS = {
    "G512": Config("diffusiongemma_global_hd512_4096c+256q", 16, 2, 512, 4096, 256),
}


def config_seed(cfg_id: int, step: int = 0) -> int:
    return 0xD1FF0000 + cfg_id + 1000 * step


# ---- k-quant Wo (native_matmul, matmul.rs:120-148) test inputs and bound

def kquant_weights(rng: np.random.Generator, wtype: int, rows: int, cols: int) -> np.ndarray:
    """rows * cols/256 random GGUF blocks (Q4_K = 12: 144 bytes, Q6_K = 14: 210)
    with sane positive f16 d (and dmin); the quant bytes are arbitrary."""
    nb = cols // 256
    bb = 144 if wtype == 12 else 210
    w = rng.integers(0, 256, (rows * nb, bb), dtype=np.uint8)
    dpos = 0 if wtype == 12 else 208
    w[:, dpos:dpos + 2] = np.float16(rng.uniform(1e-4, 0.02, rows * nb)).view(np.uint8).reshape(-1, 2)
    if wtype == 12:
        w[:, 2:4] = np.float16(rng.uniform(1e-4, 0.02, rows * nb)).view(np.uint8).reshape(-1, 2)
    return w.reshape(-1)


def kquant_acts(rng: np.random.Generator, n: int, cols: int) -> np.ndarray:
    """Activations with an all-zero block (d = 0; n > 1), a negative extreme
    and tied largest magnitudes (the first one sets the scale; n > 2)."""
    x = rng.standard_normal((n, cols)).astype(np.float32)
    if n > 1:
        x[0, :256] = 0.0
    if n > 2:
        x[2, 300 % cols] = -40.0
        x[1, 7] = x[1, 9] = 9.0
        x[1, 8] = -9.0
    return x


def kquant_dequant_f64(orc, wtype: int, w: np.ndarray, rows: int, cols: int, magnitude: bool = False):
    """[rows][cols] float64 of dequantize_q4k/q6k_row (kernels.rs:129-215).
    magnitude=True: |d sc q| + |dmin mn| per value instead (Q4_K: the same
    blocks with dmin negated, d and dmin > 0; Q6_K: |value|)."""
    nb = cols // 256
    wb = np.array(w, np.uint8).reshape(rows * nb, -1)
    if magnitude and wtype == 12:
        wb = wb.copy()
        wb[:, 3] ^= 0x80  # sign bit of the f16 dmin
    deq = orc.dequant(wtype, wb.reshape(-1), rows * nb).astype(np.float64).reshape(rows, cols)
    return np.abs(deq) if magnitude else deq


def kquant_acts_f64(orc, x: np.ndarray, n: int, cols: int) -> np.ndarray:
    """[n][cols] float64 of the Q8_K activations d * qs (quantize_rows_q8_k,
    kernels.rs:79-122)."""
    q = orc.quantize_q8k(x, n, cols)
    nb = cols // 256
    return (q["qs"].astype(np.float64) * q["d"].astype(np.float64)[:, None]).reshape(n, nb * 256)


def kquant_bound(orc, wtype: int, w, rows: int, cols: int, x: np.ndarray, n: int, res=None) -> np.ndarray:
    """[n][rows] bound on |a k-quant Wo output - another one|.  Every integer
    of a block dot is exact; the f32 combine of the per-block integers with d
    and dmin, however ordered, is within (nb + 12) * 2^-24 * S of the exact
    value, S = sum over blocks of |d dot| + |dmin mins dot| <= T = sum_i (|d sc
    q_i| + |dmin mn|) |d_x qs_i|.  Two such computations differ by at most
    twice that; the residual add rounds once on each side (|res| counted in)."""
    nb = cols // 256
    T = np.abs(kquant_acts_f64(orc, x, n, cols)) @ kquant_dequant_f64(orc, wtype, w, rows, cols, True).T
    r = 0.0 if res is None else np.abs(np.asarray(res, np.float64).reshape(n, rows))
    return 2.0 * (nb + 12) * 2.0 ** -24 * (T + r)


def legacy_weights(rng: np.random.Generator, wtype: int, rows: int, cols: int) -> np.ndarray:
    """rows * cols/32 random legacy blocks (Q4_0 = 2: 18 bytes, Q5_0 = 6: 22,
    Q8_0 = 8: 34) with a sane positive f16 d at bytes 0..1; the quant bytes
    are arbitrary."""
    bb = {2: 18, 6: 22, 8: 34}[wtype]
    nb = cols // 32
    w = rng.integers(0, 256, (rows * nb, bb), dtype=np.uint8)
    w[:, 0:2] = np.float16(rng.uniform(1e-3, 0.05, rows * nb)).view(np.uint8).reshape(-1, 2)
    return w.reshape(-1)


def legacy_dequant_f64(orc, wtype: int, w: np.ndarray, rows: int, cols: int, magnitude: bool = False):
    """[rows][cols] float64 of the dequantized legacy blocks (|.| with magnitude)."""
    nb = cols // 32
    deq = orc.dequant(wtype, np.asarray(w, np.uint8), rows * nb).astype(np.float64).reshape(rows, cols)
    return np.abs(deq) if magnitude else deq


def legacy_acts_f64(orc, x: np.ndarray, n: int, cols: int) -> np.ndarray:
    """[n][cols] float64 of the Q8_0 activations f16(d) * qs (quantize_row_q8_0)."""
    q = orc.quantize_q8_0(x, n, cols)
    d = q["d"].view(np.float16).astype(np.float64)
    return (q["qs"].astype(np.float64) * d[:, None]).reshape(n, cols)


def legacy_bound(orc, wtype: int, w, rows: int, cols: int, x: np.ndarray, n: int, res=None) -> np.ndarray:
    """[n][rows] bound on |a legacy-type Wo output - another one|: every block's
    integer dot is exact; its f32 combine with d_w and d_a, however ordered,
    is within (nb + 12) * 2^-24 * T of the exact value, T = sum_i |w_i| |x_i|
    (dequantized values); twice that between two computations, plus the
    residual add's rounding on each side."""
    nb = cols // 32
    T = np.abs(legacy_acts_f64(orc, x, n, cols)) @ legacy_dequant_f64(orc, wtype, w, rows, cols, True).T
    r = 0.0 if res is None else np.abs(np.asarray(res, np.float64).reshape(n, rows))
    return 2.0 * (nb + 12) * 2.0 ** -24 * (T + r)


# Raw-input bar of the bf16 cached path.  Rows that see at least RAW_MIN_KEYS
# keys meet the standard bar against the oracle on the unrounded f32 inputs.
# A row that averages fewer V rows inherits more of the bf16 rounding of K and
# V (2^-9 relative: up to ~9e-3 at |v| ~ 4.5 with one key, plus the weight
# shift of bf16 P times the V spread with two or three): such rows are held
# to RAW_FEW_KEYS_MAX instead, and their measured error is reported.
RAW_MIN_KEYS = 64
RAW_FEW_KEYS_MAX = 3e-2


def check_raw(orc, got, q, k, v, s: Shape, qr: RowsSpec, kr: RowsSpec, label: str, say=print):
    """The bf16 cached path's output `got` against the oracle on the raw f32
    inputs q, k, v (already QK-normed where the call normed them): the
    standard bar over rows with >= RAW_MIN_KEYS visible keys, RAW_FEW_KEYS_MAX
    over the others (NaN rows, which see no key, must be NaN in both).
    Returns (max-abs over many-key rows, max-abs over few-key rows, fewest
    keys of a row)."""
    want = np.zeros(s.nq * s.n_head * s.head_dim, np.float32)
    orc.attention(want, np.ascontiguousarray(q, np.float32), np.ascontiguousarray(k, np.float32),
                  np.ascontiguousarray(v, np.float32), s, qr, kr, threads=0)
    keys = visibility(s, qr, kr).sum(1)
    g = np.asarray(got, np.float32).reshape(s.nq, -1)
    w = want.reshape(s.nq, -1)
    assert np.array_equal(np.isnan(g), np.isnan(w)), label
    seen = keys > 0
    many, few = seen & (keys >= RAW_MIN_KEYS), seen & (keys < RAW_MIN_KEYS)
    err = np.abs(g.astype(np.float64) - w.astype(np.float64))
    mx_many = float(err[many].max()) if many.any() else 0.0
    mean_many = float(err[many].mean()) if many.any() else 0.0
    mx_few = float(err[few].max()) if few.any() else 0.0
    fewest = int(keys[seen].min()) if seen.any() else 0
    say(f"  {label} vs oracle on raw f32 inputs: rows >= {RAW_MIN_KEYS} keys max-abs {mx_many:.3e} "
        f"mean-abs {mean_many:.3e}; {int(few.sum())} rows below (fewest {fewest} keys) max-abs {mx_few:.3e}")
    assert mx_many <= TOL_MAX and mean_many <= TOL_MEAN, (label, mx_many, mean_many)
    assert mx_few <= RAW_FEW_KEYS_MAX, (label, mx_few, fewest)
    return mx_many, mx_few, fewest

"""Parity of the HIP path (diffuse-rs_amd/lib/libdr_attn.so, through its C
ABI) with the CPU oracle and the golden fixtures.  Needs an MI355X.

Bar: max-abs <= 1e-2 and mean-abs <= 1e-3 against
the f32 reference on identical inputs; NaN exactly where the reference
produces NaN (a query with no visible key); bit-exact for the integer
bookkeeping (cache positions, split lists) and for bf16-representable data
moved through the cache.
"""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

import dr_attn as dr
import oracle as orc
from helpers import (CONFIGS, TOL_MAX, TOL_MEAN, Config, RowsSpec, Shape, as_kernel_sees, check_raw,
                     closed_form, config_seed, err_stats, golden_cases, materialise)

pytestmark = pytest.mark.gpu

try:  # import at collection: the first torch import on a fresh box is slow
    import torch as _torch  # noqa: F401
except ImportError:  # pragma: no cover
    _torch = None


def say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as t
    if not t.cuda.is_available() or dr.device_count() == 0:
        pytest.skip(f"no GPU visible (torch: {t.cuda.is_available()}, "
                    f"library: {dr.device_count()})")
    dr.load()  # raises if the library is not built: no fallback
    return t


class Dev:
    """A dr context bound to a dedicated torch stream, so torch's copies and
    the library's kernels are ordered."""

    def __init__(self, torch):
        self.t = torch
        self.stream = torch.cuda.Stream()
        self.ctx = dr.Context(0)
        self.ctx.set_stream(self.stream.cuda_stream)

    def put(self, a: np.ndarray):
        with self.t.cuda.stream(self.stream):
            return self.t.from_numpy(np.ascontiguousarray(a)).to("cuda", non_blocking=False)

    def empty(self, n: int):
        with self.t.cuda.stream(self.stream):
            return self.t.full((n,), float("nan"), dtype=self.t.float32, device="cuda")

    def get(self, x) -> np.ndarray:
        self.stream.synchronize()
        return x.cpu().numpy()


@pytest.fixture(scope="module")
def dev(torch):
    return Dev(torch)


def oracle_run(s, qr, kr, q, k, v):
    out = np.zeros(s.nq * s.n_head * s.head_dim, np.float32)
    orc.attention(out, q, k, v, s, qr, kr, threads=0)
    return out


def check(got, want, label, tol_max=TOL_MAX, tol_mean=TOL_MEAN):
    mx, mean = err_stats(got, want)
    say(f"  {label}: max-abs {mx:.3e} mean-abs {mean:.3e}")
    assert mx <= tol_max and mean <= tol_mean, (label, mx, mean)
    return mx, mean


# ------------------------------------------------------------- drop-in path

@pytest.mark.parametrize("case,want", golden_cases(), ids=[c["name"] for c, _ in golden_cases()])
def test_golden_dropin(torch, case, want):
    say(f"golden {case['name']}")
    s, qr, kr, q, k, v = materialise(case)
    out = np.zeros(s.nq * s.n_head * s.head_dim, np.float32)
    dr.attention(out, q, k, v, dr.AttnShape(**s.__dict__), dr.Rows(**qr.__dict__),
                 dr.Rows(**kr.__dict__))
    check(out, want, case["name"])


def test_uniform_scores_exact(torch):
    # tests.rs:104-114; every value is bf16-exact, so the answer is exact
    out = np.zeros(2, np.float32)
    dr.attention(out, np.array([1, 0], np.float32), np.array([1, 0, 1, 0], np.float32),
                 np.array([0, 2, 4, 6], np.float32), dr.AttnShape(1, 2, 1, 1, 2),
                 dr.idpos(1), dr.idpos(2))
    assert out.tolist() == [2.0, 4.0]


def test_gqa_equals_repeated_kv(torch):
    # tests.rs:116-152 at a realistic head dim
    rng = np.random.default_rng(21)
    nq, nk, h, hkv, hd = 40, 150, 8, 2, 128
    q = rng.standard_normal(nq * h * hd).astype(np.float32)
    k = rng.standard_normal(nk * hkv * hd).astype(np.float32)
    v = rng.standard_normal(nk * hkv * hd).astype(np.float32)
    rep = lambda x: np.repeat(x.reshape(nk, hkv, hd), h // hkv, axis=1).reshape(-1).copy()  # noqa
    a = np.zeros(nq * h * hd, np.float32)
    b = np.zeros_like(a)
    sc = 1 / math.sqrt(hd)
    dr.attention(a, q, k, v, dr.AttnShape(nq, nk, h, hkv, hd, scale=sc), dr.idpos(nq), dr.idpos(nk))
    dr.attention(b, q, rep(k), rep(v), dr.AttnShape(nq, nk, h, h, hd, scale=sc), dr.idpos(nq),
                 dr.idpos(nk))
    assert np.max(np.abs(a - b)) < 1e-5


def test_block_diagonal_equals_separate(torch):
    """tests.rs:70-102 at hd 128: sequences batched in one call (seq ids) give
    each sequence's separate answer.  The two GPU runs use different launch
    plans (so bf16 rounding of P differs slightly); each is held to the parity
    bar against the oracle of the separate problems, and any cross-sequence
    leak would be O(0.1)."""
    rng = np.random.default_rng(22)
    hd, na, nb = 128, 37, 70
    n = na + nb
    q = rng.standard_normal(n * hd).astype(np.float32)
    k = rng.standard_normal(n * hd).astype(np.float32)
    v = rng.standard_normal(n * hd).astype(np.float32)
    pos = list(range(na)) + list(range(nb))
    seq = [0] * na + [1] * nb
    S = lambda m: dr.AttnShape(m, m, 1, 1, hd, scale=0.09)  # noqa: E731
    bat = np.zeros(n * hd, np.float32)
    dr.attention(bat, q, k, v, S(n), dr.Rows(pos, seq), dr.Rows(pos, seq))
    parts = []
    for lo, m in ((0, na), (na, nb)):
        sl = slice(lo * hd, (lo + m) * hd)
        sep = np.zeros(m * hd, np.float32)
        dr.attention(sep, q[sl].copy(), k[sl].copy(), v[sl].copy(), S(m), dr.idpos(m),
                     dr.idpos(m))
        want = oracle_run(Shape(m, m, 1, 1, hd, scale=0.09), RowsSpec(list(range(m))),
                          RowsSpec(list(range(m))), q[sl].copy(), k[sl].copy(), v[sl].copy())
        check(sep, want, f"separate rows {lo}..{lo + m}")
        check(bat[sl], want, f"batched rows {lo}..{lo + m}")
        parts.append(sep)
    assert np.max(np.abs(bat - np.concatenate(parts))) < TOL_MAX


def test_c1_dropin_vs_oracle(torch):
    # 32/32 heads, hd 128, 128 queries x 128 keys, no mask
    say("C1 drop-in")
    rng = np.random.default_rng(config_seed(0))
    nq = nk = 128
    h, hd = 32, 128
    q = rng.standard_normal(nq * h * hd).astype(np.float32)
    k = rng.standard_normal(nk * h * hd).astype(np.float32)
    v = rng.standard_normal(nk * h * hd).astype(np.float32)
    s = Shape(nq, nk, h, h, hd, scale=1 / math.sqrt(hd))
    want = oracle_run(s, RowsSpec(list(range(nq))), RowsSpec(list(range(nk))), q, k, v)
    got = np.zeros_like(want)
    dr.attention(got, q, k, v, dr.AttnShape(**s.__dict__), dr.idpos(nq), dr.idpos(nk))
    check(got, want, "C1")


def test_dropin_random_masks_vs_oracle(torch):
    # arbitrary key order, windows, prefixes and sequence ids at hd 64/128/256
    rng = np.random.default_rng(23)
    for trial, hd in enumerate((64, 128, 256, 40)):
        h, hkv = 4, 2
        nq, nk = 70, 200
        kpos = rng.permutation(nk).tolist()
        qpos = sorted(rng.choice(nk, nq, replace=False).tolist())
        seq_k = (np.asarray(kpos) >= 150).astype(int).tolist()
        seq_q = (np.asarray(qpos) >= 150).astype(int).tolist()
        s = Shape(nq, nk, h, hkv, hd, sliding_window=int(rng.integers(3, 60)),
                  causal_prefix=int(rng.integers(0, 120)), scale=1 / math.sqrt(hd))
        qr, kr = RowsSpec(qpos, seq_q), RowsSpec(kpos, seq_k)
        q = rng.standard_normal(nq * h * hd).astype(np.float32)
        k = rng.standard_normal(nk * hkv * hd).astype(np.float32)
        v = rng.standard_normal(nk * hkv * hd).astype(np.float32)
        say(f"random mask trial {trial} hd {hd} window {s.sliding_window} prefix {s.causal_prefix}")
        want = oracle_run(s, qr, kr, q, k, v)
        got = np.zeros_like(want)
        dr.attention(got, q, k, v, dr.AttnShape(**s.__dict__), dr.Rows(qpos, seq_q),
                     dr.Rows(kpos, seq_k))
        # Raw f32 inputs, the standard bar.  With windows of 3..60 keys and
        # causal prompt rows that see a single key, an output averages only a
        # few V rows, so bf16 operands alone would move it by up to ~1e-2
        # (2^-9 of |v| <= ~4.5, plus a ~0.3 % weight shift times a V spread of
        # ~6); the drop-in runs the hi/lo kernel on its f32 inputs instead.
        mx, _ = check(got, want, f"trial {trial} vs oracle on f32 inputs")
        assert mx < 2e-3, mx  # f32-accurate, well inside the bar


def test_no_visible_key_is_nan(torch):
    s = dr.AttnShape(3, 8, 1, 1, 128, sliding_window=2, scale=0.1)
    q = np.ones(3 * 128, np.float32)
    k = np.ones(8 * 128, np.float32)
    v = np.ones(8 * 128, np.float32)
    out = np.zeros(3 * 128, np.float32)
    dr.attention(out, q, k, v, s, dr.Rows([0, 20, 7]), dr.idpos(8))
    out = out.reshape(3, 128)
    assert np.all(np.isnan(out[1])) and not np.any(np.isnan(out[[0, 2]]))
    # nk == 0: every row is NaN
    out0 = np.zeros(2 * 128, np.float32)
    dr.attention(out0, np.ones(256, np.float32), np.zeros(0, np.float32), np.zeros(0, np.float32),
                 dr.AttnShape(2, 0, 1, 1, 128, scale=0.1), dr.idpos(2), dr.Rows([]))
    assert np.all(np.isnan(out0))


# ------------------------------------------------------------- cached path

def _cached_problem(dev, cfg, cfg_id, batch=1, step=0):
    """Stores prompt + canvas K/V of `batch` streams and attends with the
    canvas queries.  Returns (outputs, inputs) with inputs as numpy."""
    rng = np.random.default_rng(config_seed(cfg_id, step))
    kvs = cfg.n_head_kv * cfg.head_dim
    n_tot = cfg.n_total
    cache = dr.StepCache(dev.ctx, n_tot, [cfg.n_head_kv], [cfg.head_dim], n_batch=batch)
    canvas = list(range(cfg.n_prompt, n_tot))
    p_all = dr.Pass(dev.ctx, list(range(n_tot)))
    p_can = dr.Pass(dev.ctx, canvas)
    qn = kn = None
    if cfg.qk_norm:
        g = np.random.default_rng(config_seed(cfg_id) + 100)
        qn = g.uniform(0.5, 1.5, cfg.head_dim).astype(np.float32)
        kn = g.uniform(0.5, 1.5, cfg.head_dim).astype(np.float32)
    ins, outs, items = [], [], []
    for b in range(batch):
        K = rng.standard_normal((n_tot, kvs), dtype=np.float32)
        V = rng.standard_normal((n_tot, kvs), dtype=np.float32)
        Q = rng.standard_normal((cfg.n_canvas, cfg.n_head * cfg.head_dim), dtype=np.float32)
        cache.store(0, p_all, dev.put(K), dev.put(V), dev.put(kn) if kn is not None else None,
                    1e-6, batch=b)
        out = dev.empty(cfg.n_canvas * cfg.n_head * cfg.head_dim)
        qd = dev.put(Q)
        items.append((qd, out, p_can))
        outs.append(out)
        ins.append((Q, K, V))
    cache.attention(0, items, cfg.n_head, sliding_window=cfg.window, scale=cfg.attn_scale,
                    q_norm_w=dev.put(qn) if qn is not None else None, q_norm_eps=1e-6)
    got = [dev.get(o) for o in outs]
    return got, ins, (qn, kn), cache


def _oracle_cfg(cfg, Q, K, V, qn=None, kn=None):
    Q = Q.reshape(-1).copy()
    K = K.reshape(-1).copy()
    if qn is not None:
        orc.norm_heads(Q, qn, 1e-6)
        orc.norm_heads(K, kn, 1e-6)
    s = Shape(cfg.n_canvas, cfg.n_total, cfg.n_head, cfg.n_head_kv, cfg.head_dim,
              sliding_window=cfg.window, scale=cfg.attn_scale)
    qr = RowsSpec(list(range(cfg.n_prompt, cfg.n_total)))
    kr = RowsSpec(list(range(cfg.n_total)))
    return oracle_run(s, qr, kr, Q, K, V.reshape(-1).copy())


@pytest.mark.parametrize("cid", ["C2", "C3", "C4", "C5S", "C5G"])
def test_config_cached_vs_oracle(dev, cid):
    cfg = CONFIGS[cid]
    say(f"config {cid} ({cfg.name})")
    got, ins, (qn, kn), _ = _cached_problem(dev, cfg, list(CONFIGS).index(cid), batch=cfg.batch)
    say(f"  launch {dev.ctx.last_launch()}")
    for b in range(cfg.batch):
        Q, K, V = ins[b]
        want = _oracle_cfg(cfg, Q, K, V, qn, kn)
        check(got[b], want, f"{cid} batch {b}")


def test_gemma_scale_one_hilo_layer(dev):
    """Gemma's real kq_scale is 1.0 (forward.rs:338-341): with N(0,1) inputs
    at hd 256 the score std is 16 and the softmax is close to one-hot, so a
    bf16 Q/K path errs by ~0.15.  On a layer kept at DR_PRECISION_HILO the
    scores and values are f32-accurate and C5S's shape at scale 1.0 meets the
    north-star tolerance (tests/test_gpu_hilo.py covers QK-normed inputs,
    hd 512 and the bf16 contrast)."""
    cfg = CONFIGS["C5S"]
    rng = np.random.default_rng(config_seed(4))
    h, hkv, hd, n_p, n_c = cfg.n_head, cfg.n_head_kv, cfg.head_dim, 1024, cfg.n_canvas
    n_t = n_p + n_c
    K = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
    V = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
    Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    cache.set_precision(0, dr.PRECISION_HILO)
    cache.store(0, dr.Pass(dev.ctx, range(n_t)), dev.put(K), dev.put(V))
    out = dev.empty(n_c * h * hd)
    cache.attention(0, [(dev.put(Q), out, dr.Pass(dev.ctx, range(n_p, n_t)))], h,
                    sliding_window=cfg.window, scale=1.0)
    assert dev.ctx.last_launch()["kernel"] == dr.KERNEL_HILO
    s = Shape(n_c, n_t, h, hkv, hd, sliding_window=cfg.window, scale=1.0)
    want = oracle_run(s, RowsSpec(list(range(n_p, n_t))), RowsSpec(list(range(n_t))),
                      Q.reshape(-1).copy(), K.reshape(-1).copy(), V.reshape(-1).copy())
    check(dev.get(out), want, "Gemma scale 1.0 (hd 256, N(0,1)), hi/lo layer")


@pytest.mark.parametrize("hd", [128, 256, 512])
@pytest.mark.parametrize("window,prefix", [(None, None), (64, None), (None, 250), (37, 180)])
def test_wave_rows_16_and_32_vs_oracle(dev, hd, window, prefix):
    """Both compute-wave shapes of head dims 128, 256 and 512 (32 query rows
    per wave, or two waves of 16 on 16x16x32 MFMAs; at 512 each also split
    over the head dim) against the oracle, unmasked and with windows /
    causal prefixes, on a GQA problem with a ragged last tile and a ragged
    last row block."""
    rng = np.random.default_rng(31)
    h, hkv, n_p, n_c = 8, 2, 200, 93
    n_t = n_p + n_c
    K = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
    V = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
    Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    cache.store(0, dr.Pass(dev.ctx, range(n_t)), dev.put(K), dev.put(V))
    pc = dr.Pass(dev.ctx, range(n_p, n_t))
    scale = 1 / math.sqrt(hd)
    s = Shape(n_c, n_t, h, hkv, hd, sliding_window=window, causal_prefix=prefix, scale=scale)
    qr, kr = RowsSpec(list(range(n_p, n_t))), RowsSpec(list(range(n_t)))
    want = oracle_run(s, qr, kr, *as_kernel_sees(Q.reshape(-1).copy(), K.reshape(-1).copy(),
                                                 V.reshape(-1).copy(), scale))
    got = {}
    try:
        for rows in (16, 32):
            dev.ctx.set_wave_rows(rows)
            out = dev.empty(n_c * h * hd)
            cache.attention(0, [(dev.put(Q), out, pc)], h, sliding_window=window,
                            causal_prefix=prefix, scale=scale)
            assert dev.ctx.last_launch()["rows_per_wave"] == rows
            got[rows] = dev.get(out)
            check(got[rows], want, f"rows {rows} window {window} prefix {prefix}")
            check_raw(orc, got[rows], Q.reshape(-1), K.reshape(-1), V.reshape(-1), s, qr, kr,
                      f"rows {rows} window {window} prefix {prefix}", say)
    finally:
        dev.ctx.set_wave_rows(0)
    assert np.max(np.abs(got[16] - got[32])) < 1e-5


@pytest.mark.parametrize("n_split", [1, 2, 3, 5, 8])
def test_split_count_does_not_change_result(dev, n_split):
    """Key splits merged by the last workgroup of each row group give the
    unsplit result."""
    cfg = CONFIGS["C2"]
    say(f"C2 with forced n_split={n_split}")
    dev.ctx.set_split(n_split)
    try:
        got, ins, _, _ = _cached_problem(dev, cfg, 1)
        assert dev.ctx.last_launch()["n_split"] == n_split
    finally:
        dev.ctx.set_split(0)
    Q, K, V = ins[0]
    check(got[0], _oracle_cfg(cfg, Q, K, V), f"split {n_split}")


def test_c2_sixteen_denoise_steps(dev):
    """the prompt K/V is stored once; each of 16 steps stores fresh
    canvas K/V and attends with fresh canvas queries (forward.rs:312-343)."""
    cfg = CONFIGS["C2"]
    kvs = cfg.n_head_kv * cfg.head_dim
    rng = np.random.default_rng(config_seed(1))
    Kp = rng.standard_normal((cfg.n_prompt, kvs), dtype=np.float32)
    Vp = rng.standard_normal((cfg.n_prompt, kvs), dtype=np.float32)
    cache = dr.StepCache(dev.ctx, cfg.n_total, [cfg.n_head_kv], [cfg.head_dim])
    cache.store(0, dr.Pass(dev.ctx, range(cfg.n_prompt)), dev.put(Kp), dev.put(Vp))
    p_can = dr.Pass(dev.ctx, range(cfg.n_prompt, cfg.n_total))
    out = dev.empty(cfg.n_canvas * cfg.n_head * cfg.head_dim)
    for step in range(16):
        r = np.random.default_rng(config_seed(1, step + 1))
        Kc = r.standard_normal((cfg.n_canvas, kvs), dtype=np.float32)
        Vc = r.standard_normal((cfg.n_canvas, kvs), dtype=np.float32)
        Q = r.standard_normal((cfg.n_canvas, cfg.n_head * cfg.head_dim), dtype=np.float32)
        cache.store(0, p_can, dev.put(Kc), dev.put(Vc))
        cache.attention(0, [(dev.put(Q), out, p_can)], cfg.n_head, scale=cfg.attn_scale)
        if step in (0, 7, 15):
            got = dev.get(out)
            want = _oracle_cfg(cfg, Q, np.concatenate([Kp, Kc]), np.concatenate([Vp, Vc]))
            check(got, want, f"C2 step {step}")


# Ragged shapes of the step (not BASELINE configs).
STEP_RAGGED = {
    "R1": Config("ragged_gqa_qknorm_96c+77q_b2", 8, 2, 128, 96, 77, batch=2, qk_norm=True),
    "R2": Config("hd64_all_fresh_0c+50q", 4, 4, 64, 0, 50),
    "R3": Config("prompt128_128c+100q", 8, 8, 128, 128, 100),
}


def _step_problem(dev, cfg, cfg_id, n_split=0):
    """Prompt K/V stored once, then one denoise-step layer through
    StepCache.step (store of the canvas rows + attention).  Returns outputs,
    inputs, norms, the cache and the launch info."""
    rng = np.random.default_rng(config_seed(cfg_id, 7))
    kvs = cfg.n_head_kv * cfg.head_dim
    n_tot = cfg.n_total
    cache = dr.StepCache(dev.ctx, n_tot, [cfg.n_head_kv], [cfg.head_dim], n_batch=cfg.batch)
    p_pr = dr.Pass(dev.ctx, list(range(cfg.n_prompt)))
    p_can = dr.Pass(dev.ctx, list(range(cfg.n_prompt, n_tot)))
    qn = kn = None
    if cfg.qk_norm:
        g = np.random.default_rng(config_seed(cfg_id) + 100)
        qn = g.uniform(0.5, 1.5, cfg.head_dim).astype(np.float32)
        kn = g.uniform(0.5, 1.5, cfg.head_dim).astype(np.float32)
    knd = dev.put(kn) if kn is not None else None
    ins, outs, items = [], [], []
    for b in range(cfg.batch):
        K = rng.standard_normal((n_tot, kvs), dtype=np.float32)
        V = rng.standard_normal((n_tot, kvs), dtype=np.float32)
        Q = rng.standard_normal((cfg.n_canvas, cfg.n_head * cfg.head_dim), dtype=np.float32)
        if cfg.n_prompt:
            cache.store(0, p_pr, dev.put(K[:cfg.n_prompt].copy()), dev.put(V[:cfg.n_prompt].copy()),
                        knd, 1e-6, batch=b)
        out = dev.empty(cfg.n_canvas * cfg.n_head * cfg.head_dim)
        items.append((dev.put(Q), out, p_can, dev.put(K[cfg.n_prompt:].copy()),
                      dev.put(V[cfg.n_prompt:].copy())))
        outs.append(out)
        ins.append((Q, K, V))
    dev.ctx.set_split(n_split)
    try:
        cache.step(0, items, cfg.n_head, sliding_window=cfg.window, scale=cfg.attn_scale,
                   q_norm_w=dev.put(qn) if qn is not None else None, q_norm_eps=1e-6,
                   k_norm_w=knd, k_norm_eps=1e-6)
        launch = dev.ctx.last_launch()
    finally:
        dev.ctx.set_split(0)
    got = [dev.get(o) for o in outs]
    return got, ins, (qn, kn), cache, launch


def _normed_bf16(dev, x, w):
    x = x.reshape(-1).copy()
    if w is not None:
        orc.norm_heads(x, w, 1e-6)
    t = dev.t
    return t.from_numpy(x).to(t.bfloat16).to(t.float32).numpy()


@pytest.mark.parametrize("cid,n_split", [
    ("C2", 0), ("C2", 2), ("C3", 0), ("C4", 0), ("C5S", 0), ("C5G", 0), ("R1", 0), ("R1", 3),
    ("R2", 0), ("R3", 0)])
def test_step_vs_oracle_and_cache(dev, cid, n_split):
    """StepCache.step = norm_heads(k) + cache.store(canvas) + attention over
    [prompt | canvas] (forward.rs:296-343): the outputs meet the parity bar
    against the oracle, and afterwards the cache holds bf16 of the (K-normed)
    canvas rows and still the prompt rows, bit for bit.  R1-R3 are ragged
    cases: a partial last tile (rows past the pass stored as zeros), every
    key fresh (head dim 64, no prompt), and a prompt of 128 rows."""
    cfg = CONFIGS.get(cid) or STEP_RAGGED[cid]
    cfg_id = list(CONFIGS).index(cid) if cid in CONFIGS else 100 + list(STEP_RAGGED).index(cid)
    say(f"step {cid} split {n_split} ({cfg.name})")
    got, ins, (qn, kn), cache, launch = _step_problem(dev, cfg, cfg_id, n_split)
    say(f"  launch {launch}")
    if n_split:
        assert launch["n_split"] == n_split
    kvs = cfg.n_head_kv * cfg.head_dim
    for b in range(cfg.batch):
        Q, K, V = ins[b]
        check(got[b], _oracle_cfg(cfg, Q, K, V, qn, kn), f"{cid} batch {b}")
        ok, ov = dev.empty(cfg.n_total * kvs), dev.empty(cfg.n_total * kvs)
        cache.gather(0, list(range(cfg.n_total)), ok, ov, batch=b)
        assert np.array_equal(dev.get(ok), _normed_bf16(dev, K, kn)), f"{cid} K cache, batch {b}"
        assert np.array_equal(dev.get(ov), _normed_bf16(dev, V, None)), f"{cid} V cache, batch {b}"


def test_step_sixteen_denoise_steps(dev):
    """configs[1] through StepCache.step: 16 steps with fresh canvas K/V and
    queries; each step's output against the oracle, and the cache after the
    last step against its canvas rows."""
    cfg = CONFIGS["C2"]
    kvs = cfg.n_head_kv * cfg.head_dim
    rng = np.random.default_rng(config_seed(1))
    Kp = rng.standard_normal((cfg.n_prompt, kvs), dtype=np.float32)
    Vp = rng.standard_normal((cfg.n_prompt, kvs), dtype=np.float32)
    cache = dr.StepCache(dev.ctx, cfg.n_total, [cfg.n_head_kv], [cfg.head_dim])
    cache.store(0, dr.Pass(dev.ctx, range(cfg.n_prompt)), dev.put(Kp), dev.put(Vp))
    p_can = dr.Pass(dev.ctx, range(cfg.n_prompt, cfg.n_total))
    out = dev.empty(cfg.n_canvas * cfg.n_head * cfg.head_dim)
    for step in range(16):
        r = np.random.default_rng(config_seed(1, step + 1))
        Kc = r.standard_normal((cfg.n_canvas, kvs), dtype=np.float32)
        Vc = r.standard_normal((cfg.n_canvas, kvs), dtype=np.float32)
        Q = r.standard_normal((cfg.n_canvas, cfg.n_head * cfg.head_dim), dtype=np.float32)
        cache.step(0, [(dev.put(Q), out, p_can, dev.put(Kc), dev.put(Vc))], cfg.n_head,
                   scale=cfg.attn_scale)
        if step in (0, 7, 15):
            want = _oracle_cfg(cfg, Q, np.concatenate([Kp, Kc]), np.concatenate([Vp, Vc]))
            check(dev.get(out), want, f"C2 step {step}")
    ok, ov = dev.empty(cfg.n_total * kvs), dev.empty(cfg.n_total * kvs)
    cache.gather(0, list(range(cfg.n_total)), ok, ov)
    assert np.array_equal(dev.get(ok), _normed_bf16(dev, np.concatenate([Kp, Kc]), None))
    assert np.array_equal(dev.get(ov), _normed_bf16(dev, np.concatenate([Vp, Vc]), None))


def test_step_scattered_pass(dev):
    """A pass that is not one block ending at n_total (the ActiveSplit of a
    later step): the result is the reference's [cached | active]
    concatenation (forward.rs:312-343)."""
    rng = np.random.default_rng(43)
    n_tot, h, hkv, hd = 300, 8, 4, 128
    kvs = hkv * hd
    K = rng.standard_normal((n_tot, kvs), dtype=np.float32)
    V = rng.standard_normal((n_tot, kvs), dtype=np.float32)
    cache = dr.StepCache(dev.ctx, n_tot, [hkv], [hd])
    cache.store(0, dr.Pass(dev.ctx, range(n_tot)), dev.put(K), dev.put(V))
    active = sorted(rng.choice(n_tot, 61, replace=False).tolist())
    cached = [p for p in range(n_tot) if p not in set(active)]
    Ka = rng.standard_normal((len(active), kvs), dtype=np.float32)
    Va = rng.standard_normal((len(active), kvs), dtype=np.float32)
    Q = rng.standard_normal((len(active), h * hd), dtype=np.float32)
    pa = dr.Pass(dev.ctx, active)
    out = dev.empty(len(active) * h * hd)
    cache.step(0, [(dev.put(Q), out, pa, dev.put(Ka), dev.put(Va))], h, scale=0.1)
    Kf = np.concatenate([K[cached], Ka]).reshape(-1).copy()
    Vf = np.concatenate([V[cached], Va]).reshape(-1).copy()
    s = Shape(len(active), n_tot, h, hkv, hd, scale=0.1)
    want = oracle_run(s, RowsSpec(active), RowsSpec(cached + active), Q.reshape(-1).copy(), Kf, Vf)
    check(dev.get(out), want, "scattered pass via step")


def test_cache_store_gather_roundtrip(dev):
    # tests.rs:55-68: values are bf16-exact, so the round trip is exact
    cache = dr.StepCache(dev.ctx, 3, [1], [4])
    k = np.arange(8, dtype=np.float32)
    v = np.arange(100, 108, dtype=np.float32)
    cache.store(0, dr.Pass(dev.ctx, [0, 2]), dev.put(k[[4, 5, 6, 7, 0, 1, 2, 3]].copy()),
                dev.put(v[[4, 5, 6, 7, 0, 1, 2, 3]].copy()))
    ok, ov = dev.empty(8), dev.empty(8)
    cache.gather(0, [0, 2], ok, ov)
    assert dev.get(ok).tolist() == [4, 5, 6, 7, 0, 1, 2, 3]
    assert dev.get(ov).tolist() == [104, 105, 106, 107, 100, 101, 102, 103]


def test_cache_gather_is_bf16_of_store(dev):
    rng = np.random.default_rng(31)
    n, hkv, hd = 100, 3, 96
    cache = dr.StepCache(dev.ctx, 130, [hkv], [hd])
    pos = sorted(rng.choice(130, n, replace=False).tolist())
    K = rng.standard_normal((n, hkv * hd), dtype=np.float32)
    V = rng.standard_normal((n, hkv * hd), dtype=np.float32)
    cache.store(0, dr.Pass(dev.ctx, pos), dev.put(K), dev.put(V))
    ok, ov = dev.empty(n * hkv * hd), dev.empty(n * hkv * hd)
    cache.gather(0, pos, ok, ov)
    t = dev.t
    bf = lambda a: t.from_numpy(a).to(t.bfloat16).to(t.float32).numpy().reshape(-1)  # noqa: E731
    assert np.array_equal(dev.get(ok), bf(K))
    assert np.array_equal(dev.get(ov), bf(V))


@pytest.mark.parametrize("hd,hkv,p0,n,n_batch", [(128, 32, 512, 256, 1), (128, 3, 0, 96, 2), (64, 5, 32, 64, 1),
                                                 (256, 8, 4096, 256, 1), (256, 2, 64, 32, 2), (96, 2, 32, 64, 1)])
def test_cache_store_whole_tiles_is_bf16(dev, hd, hkv, p0, n, n_batch):
    """Rows that fill whole 32-key tiles at contiguous positions (the canvas
    rows of a denoise step; their own store kernel at head dim 64/128/256,
    the general one at 96): gather returns bf16 of every stored row bit for
    bit (cache.rs:62-82), in the last layer of a three-layer cache and in
    every batch slot, and the rows stored before, around the tiles, keep
    their values."""
    rng = np.random.default_rng(hd + p0 + n)
    n_tot = p0 + n + 40
    cache = dr.StepCache(dev.ctx, n_tot, [hkv] * 3, [hd] * 3, n_batch=n_batch)
    t = dev.t
    bf = lambda a: t.from_numpy(a).to(t.bfloat16).to(t.float32).numpy().reshape(-1)  # noqa: E731
    every = list(range(n_tot))
    for b in range(n_batch):
        K0 = rng.standard_normal((n_tot, hkv * hd), dtype=np.float32)
        V0 = rng.standard_normal((n_tot, hkv * hd), dtype=np.float32)
        cache.store(2, dr.Pass(dev.ctx, every), dev.put(K0), dev.put(V0), batch=b)  # ragged: the general kernel
        K = rng.standard_normal((n, hkv * hd), dtype=np.float32)
        V = rng.standard_normal((n, hkv * hd), dtype=np.float32)
        cache.store(2, dr.Pass(dev.ctx, range(p0, p0 + n)), dev.put(K), dev.put(V), batch=b)
        wk, wv = K0.copy(), V0.copy()
        wk[p0:p0 + n], wv[p0:p0 + n] = K, V
        ok, ov = dev.empty(n_tot * hkv * hd), dev.empty(n_tot * hkv * hd)
        cache.gather(2, every, ok, ov, batch=b)
        assert np.array_equal(dev.get(ok), bf(wk)), b
        assert np.array_equal(dev.get(ov), bf(wv)), b


@pytest.mark.parametrize("hd,hkv,n,n_tot,n_batch", [(128, 32, 256, 768, 1), (128, 3, 173, 400, 2), (64, 5, 40, 90, 1),
                                                 (256, 8, 100, 4352, 1), (256, 2, 7, 64, 2), (96, 2, 77, 200, 1)])
def test_cache_store_position_list_is_bf16(dev, hd, hkv, n, n_tot, n_batch):
    """Rows stored at sorted scattered positions (split_active's active rows,
    on kv_store_kernel's position-list V^T path): gather returns bf16 of every
    stored row bit for bit (cache.rs:62-82), and every other position keeps
    its value."""
    rng = np.random.default_rng(hd * 7 + n + n_tot)
    cache = dr.StepCache(dev.ctx, n_tot, [hkv] * 2, [hd] * 2, n_batch=n_batch)
    t = dev.t
    bf = lambda a: t.from_numpy(a).to(t.bfloat16).to(t.float32).numpy().reshape(-1)  # noqa: E731
    every = list(range(n_tot))
    for b in range(n_batch):
        K0 = rng.standard_normal((n_tot, hkv * hd), dtype=np.float32)
        V0 = rng.standard_normal((n_tot, hkv * hd), dtype=np.float32)
        cache.store(1, dr.Pass(dev.ctx, every), dev.put(K0), dev.put(V0), batch=b)
        pos = sorted(rng.choice(n_tot, size=n, replace=False).tolist())
        K = rng.standard_normal((n, hkv * hd), dtype=np.float32)
        V = rng.standard_normal((n, hkv * hd), dtype=np.float32)
        cache.store(1, dr.Pass(dev.ctx, pos), dev.put(K), dev.put(V), batch=b)
        wk, wv = K0.copy(), V0.copy()
        wk[pos], wv[pos] = K, V
        ok, ov = dev.empty(n_tot * hkv * hd), dev.empty(n_tot * hkv * hd)
        cache.gather(1, every, ok, ov, batch=b)
        assert np.array_equal(dev.get(ok), bf(wk)), b
        assert np.array_equal(dev.get(ov), bf(wv)), b


@pytest.mark.parametrize("hd,hkv,h,n_p,n_c,bias,norm,v_norm,rot", [
    (128, 16, 16, 512, 256, False, True, False, 0),   # C4-like QK-norm
    (128, 16, 16, 512, 256, True, True, False, 128),  # the same with the biases and RoPE
    (256, 8, 16, 256, 128, True, True, True, 256),    # Gemma-like: biases, K norm, V norm, RoPE
    (64, 4, 8, 64, 96, True, False, False, 0),        # biases only
    (128, 2, 8, 96, 64, False, False, True, 0),       # V norm only
    (128, 4, 8, 64, 64, True, True, False, 64),       # partial rotary
    (64, 2, 4, 32, 32, False, False, False, 24),      # RoPE only, rot / 2 not a multiple of 8
])
def test_cache_store_whole_tiles_epilogue(dev, hd, hkv, h, n_p, n_c, bias, norm, v_norm, rot):
    """The Q/K/V epilogue's K and V part (forward.rs:291-310) on the whole-tile
    store (canvas rows at contiguous positions), through
    dr_attention_step_epi: add_bias (ops.rs:373-382), then K's RMSNorm with
    its gain (ops.rs:106-114) and V's without one (ops.rs:116-124), then RoPE
    on K (rotate_rows, ops.rs:433-452).  The gathered rows equal bf16 of the
    oracle's rows bit for bit."""
    rng = np.random.default_rng(hd + n_c + 10 * bias + 100 * norm + 1000 * v_norm + rot)
    eps = 1e-6
    n_t, kvs = n_p + n_c, hkv * hd
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    K = (rng.standard_normal((n_c, kvs)) * 2).astype(np.float32)
    V = rng.standard_normal((n_c, kvs)).astype(np.float32)
    Q = rng.standard_normal((n_c, h * hd)).astype(np.float32)
    bk = (0.1 * rng.standard_normal(kvs)).astype(np.float32) if bias else None
    bv = (0.1 * rng.standard_normal(kvs)).astype(np.float32) if bias else None
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norm else None
    put = lambda x: dev.put(x) if x is not None else None  # noqa: E731
    out = dev.empty(n_c * h * hd)
    p_c = dr.Pass(dev.ctx, range(n_p, n_t))
    rope = dr.Rope(dev.ctx, n_t, rot, 10000.0) if rot else None
    cache.step_epi(0, [(dev.put(Q), out, p_c, dev.put(K), dev.put(V))], h, scale=1 / math.sqrt(hd),
                   bk=put(bk), bv=put(bv), k_norm_w=put(kn), v_norm=v_norm, eps=eps, rope=rope)
    wk, wv = K.reshape(-1).copy(), V.reshape(-1).copy()
    if bias:
        orc.add_bias(wk, bk, n_c)
        orc.add_bias(wv, bv, n_c)
    for o in range(0, wk.size, hd):
        if norm:
            seg = wk[o:o + hd].copy()
            orc.rms_norm_inplace(seg, kn, eps)
            wk[o:o + hd] = seg
        if v_norm:
            seg = wv[o:o + hd].copy()
            orc.rms_norm_noscale(seg, eps)
            wv[o:o + hd] = seg
    if rot:
        orc.rotate_rows(wk, orc.rope_table(n_t, rot, 10000.0), list(range(n_p, n_t)), hkv, hd, rot)
    ok, ov = dev.empty(n_c * kvs), dev.empty(n_c * kvs)
    cache.gather(0, list(range(n_p, n_t)), ok, ov)
    t = dev.t
    bf = lambda a: t.from_numpy(a).to(t.bfloat16).to(t.float32).numpy().reshape(-1)  # noqa: E731
    assert np.array_equal(dev.get(ok), bf(wk))
    assert np.array_equal(dev.get(ov), bf(wv))


@pytest.mark.parametrize("hd,n,n_tot", [(64, 70, 200), (96, 129, 150), (128, 64, 64),
                                        (256, 33, 90), (512, 70, 100), (320, 17, 40)])
def test_cache_store_k_norm_is_bf16_of_oracle(dev, hd, n, n_tot):
    """norm_heads(k, k_norm) + cache.store (forward.rs:300-302, 318-320): the
    gathered K equals bf16 of the oracle's rms_norm_inplace (ops.rs:106-114)
    per (row, kv head), bit for bit; V is stored unnormalised."""
    rng = np.random.default_rng(hd * 1000 + n)
    hkv, eps = 3, 1e-6
    cache = dr.StepCache(dev.ctx, n_tot, [hkv], [hd])
    pos = sorted(rng.choice(n_tot, n, replace=False).tolist())
    K = rng.standard_normal((n, hkv * hd), dtype=np.float32) * 3
    V = rng.standard_normal((n, hkv * hd), dtype=np.float32)
    w = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    cache.store(0, dr.Pass(dev.ctx, pos), dev.put(K), dev.put(V), k_norm_w=dev.put(w), eps=eps)
    ok, ov = dev.empty(n * hkv * hd), dev.empty(n * hkv * hd)
    cache.gather(0, pos, ok, ov)
    Kn = K.reshape(-1).copy()
    for o in range(0, Kn.size, hd):
        seg = Kn[o:o + hd].copy()
        orc.rms_norm_inplace(seg, w, eps)
        Kn[o:o + hd] = seg
    t = dev.t
    bf = lambda a: t.from_numpy(a).to(t.bfloat16).to(t.float32).numpy().reshape(-1)  # noqa: E731
    assert np.array_equal(dev.get(ok), bf(Kn))
    assert np.array_equal(dev.get(ov), bf(V))


def test_cache_split_active_reference_case(dev):
    # tests.rs:39-53 through the StepCache object
    cache = dr.StepCache(dev.ctx, 4, [1], [8])
    assert not cache.initialized()
    cache.update_seq([10, 20, -1, -1])
    assert cache.initialized()
    act, cac = cache.split_active([10, 21, -1, -1], [0, 0, 1, 1], 5)
    assert act == [1, 2, 3] and cac == [0]
    cache.update_seq([10, 21, -1, -1])
    act, cac = cache.split_active([10, 21, -1, -1], [0, 0, 1, 1], 8)
    assert act == [2, 3] and cac == [0, 1]


def test_partial_active_split_vs_dropin(dev):
    """A denoise step with a non-trivial ActiveSplit: the cached path (keys
    read by position from the cache) equals the reference's [cached | active]
    concatenation through the drop-in (forward.rs:312-343)."""
    rng = np.random.default_rng(41)
    n_tot, h, hkv, hd = 300, 8, 4, 128
    kvs = hkv * hd
    K = rng.standard_normal((n_tot, kvs), dtype=np.float32)
    V = rng.standard_normal((n_tot, kvs), dtype=np.float32)
    cache = dr.StepCache(dev.ctx, n_tot, [hkv], [hd])
    cache.store(0, dr.Pass(dev.ctx, range(n_tot)), dev.put(K), dev.put(V))
    active = sorted(rng.choice(n_tot, 77, replace=False).tolist())
    cached = [p for p in range(n_tot) if p not in set(active)]
    Ka = rng.standard_normal((len(active), kvs), dtype=np.float32)
    Va = rng.standard_normal((len(active), kvs), dtype=np.float32)
    Q = rng.standard_normal((len(active), h * hd), dtype=np.float32)
    pa = dr.Pass(dev.ctx, active)
    cache.store(0, pa, dev.put(Ka), dev.put(Va))
    out = dev.empty(len(active) * h * hd)
    cache.attention(0, [(dev.put(Q), out, pa)], h, sliding_window=40, scale=0.1)
    got = dev.get(out)
    # reference key order: gather(cached) ++ active rows (forward.rs:312-317)
    Kf = np.concatenate([K[cached], Ka]).reshape(-1).copy()
    Vf = np.concatenate([V[cached], Va]).reshape(-1).copy()
    s = Shape(len(active), n_tot, h, hkv, hd, sliding_window=40, scale=0.1)
    want = oracle_run(s, RowsSpec(active), RowsSpec(cached + active), Q.reshape(-1).copy(), Kf, Vf)
    check(got, want, "partial split")


# ------------------------------------------------------------- Q/K/V epilogue

def _epilogue_oracle(q, k, v, pos, h, hkv, hd, bq, bk, bv, qn, kn, v_norm, eps, table, rot):
    """forward.rs:291-310 with the oracle's restatement of each step."""
    q, k, v = q.copy(), k.copy(), v.copy()
    n = len(pos)
    for x, b in ((q, bq), (k, bk), (v, bv)):
        if b is not None:
            orc.add_bias(x, b, n)
    if qn is not None:
        orc.norm_heads(q, qn, eps)
    if kn is not None:
        orc.norm_heads(k, kn, eps)
    if v_norm:
        for r in range(n * hkv):
            seg = v[r * hd:(r + 1) * hd].copy()
            orc.rms_norm_noscale(seg, eps)
            v[r * hd:(r + 1) * hd] = seg
    if table is not None:
        orc.rotate_rows(q, table, pos, h, hd, rot)
        orc.rotate_rows(k, table, pos, hkv, hd, rot)
    return q, k, v


@pytest.mark.parametrize("hd,rot,h,hkv,bias,norm,v_norm,ff", [
    (128, 128, 8, 2, True, True, False, False),
    (128, 64, 4, 4, True, False, False, False),
    (128, 128, 4, 2, False, False, False, False),
    (256, 256, 4, 2, False, True, True, True),
    (64, 64, 2, 2, True, True, False, False),
    (96, 32, 3, 1, True, True, True, False),
    (512, 256, 4, 2, False, True, True, False),
])
def test_qkv_epilogue_vs_oracle(dev, hd, rot, h, hkv, bias, norm, v_norm, ff):
    """The epilogue kernel against the oracle's add_bias / norm_heads /
    rms_norm_noscale / rotate_rows (bias and rotation are exact: no fused
    multiply-adds on either side; a norm's f64 sum runs in another order,
    which may move its f32 scale by an ulp)."""
    rng = np.random.default_rng(hd * 7 + rot)
    n, max_len, eps = 37, 3000, 1e-6
    pos = sorted(rng.choice(max_len, n, replace=False).tolist())
    q = rng.standard_normal(n * h * hd).astype(np.float32)
    k = rng.standard_normal(n * hkv * hd).astype(np.float32)
    v = rng.standard_normal(n * hkv * hd).astype(np.float32)
    mk = lambda m: rng.standard_normal(m).astype(np.float32) if bias else None  # noqa: E731
    bq, bk, bv = mk(h * hd), mk(hkv * hd), mk(hkv * hd)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norm else None
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norm else None
    ffv = rng.uniform(1.0, 8.0, rot // 2).astype(np.float32) if ff else None
    theta = 10000.0 if hd != 256 else 1e6
    table = orc.rope_table(max_len, rot, theta, ffv)
    want = _epilogue_oracle(q, k, v, pos, h, hkv, hd, bq, bk, bv, qn, kn, v_norm, eps, table, rot)
    say(f"epilogue hd {hd} rot {rot} h {h}/{hkv} bias {bias} norm {norm} v_norm {v_norm} ff {ff}")
    rope = dr.Rope(dev.ctx, max_len, rot, theta, ffv)
    p = dr.Pass(dev.ctx, pos)
    dq, dk, dv = dev.put(q), dev.put(k), dev.put(v)
    put = lambda x: dev.put(x) if x is not None else None  # noqa: E731
    dr.qkv_epilogue(dev.ctx, p, dq, dk, dv, h, hkv, hd, put(bq), put(bk), put(bv), put(qn),
                    put(kn), v_norm, eps, rope)
    for name, g, w in zip("qkv", (dev.get(dq), dev.get(dk), dev.get(dv)), want):
        if not (norm or (v_norm and name == "v")):
            assert np.array_equal(g, w), name
        else:
            rel = np.abs(g - w) / np.maximum(np.abs(w), 1e-30)
            assert np.max(rel) <= 2.0**-22 or np.max(np.abs(g - w)) < 1e-6, (name, np.max(rel))
            say(f"  {name}: {np.count_nonzero(g != w)} of {g.size} differ by an ulp")


def test_qkv_epilogue_then_step_vs_oracle(dev):
    """C4-like layer (16/16 heads, hd 128, QK-norm) with biases and RoPE:
    epilogue, then the step (store + attention without norms), against the
    oracle's epilogue and attention; the cache then holds bf16 of the
    oracle's K and V rows, bit for bit."""
    rng = np.random.default_rng(41)
    h, hkv, hd, n_p, n_c, eps = 16, 16, 128, 512, 256, 1e-6
    n_t = n_p + n_c
    kvs = hkv * hd
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    bq = (0.1 * rng.standard_normal(h * hd)).astype(np.float32)
    bk = (0.1 * rng.standard_normal(kvs)).astype(np.float32)
    bv = (0.1 * rng.standard_normal(kvs)).astype(np.float32)
    table = orc.rope_table(n_t, hd, 10000.0)
    rope = dr.Rope(dev.ctx, n_t, hd, 10000.0)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    K = rng.standard_normal(n_t * kvs).astype(np.float32)
    V = rng.standard_normal(n_t * kvs).astype(np.float32)
    Q = rng.standard_normal(n_c * h * hd).astype(np.float32)
    put = dev.put
    kp, vp = K[:n_p * kvs].copy(), V[:n_p * kvs].copy()
    kc, vc = K[n_p * kvs:].copy(), V[n_p * kvs:].copy()
    # prompt pass through the same epilogue (its q rows are not needed)
    p_pr = dr.Pass(dev.ctx, range(n_p))
    qdummy = np.zeros(n_p * h * hd, np.float32)
    _, kp_o, vp_o = _epilogue_oracle(qdummy, kp, vp, list(range(n_p)), h, hkv, hd, bq, bk, bv,
                                     qn, kn, False, eps, table, hd)
    dq0, dkp, dvp = put(qdummy), put(kp), put(vp)
    dr.qkv_epilogue(dev.ctx, p_pr, dq0, dkp, dvp, h, hkv, hd, put(bq), put(bk), put(bv), put(qn),
                    put(kn), False, eps, rope)
    cache.store(0, p_pr, dkp, dvp)
    # canvas step
    canvas = list(range(n_p, n_t))
    p_c = dr.Pass(dev.ctx, canvas)
    q_o, kc_o, vc_o = _epilogue_oracle(Q, kc, vc, canvas, h, hkv, hd, bq, bk, bv, qn, kn, False,
                                       eps, table, hd)
    dq, dk, dv = put(Q), put(kc), put(vc)
    dr.qkv_epilogue(dev.ctx, p_c, dq, dk, dv, h, hkv, hd, put(bq), put(bk), put(bv), put(qn),
                    put(kn), False, eps, rope)
    out = dev.empty(n_c * h * hd)
    cache.step(0, [(dq, out, p_c, dk, dv)], h, scale=1 / math.sqrt(hd))
    s = Shape(n_c, n_t, h, hkv, hd, scale=1 / math.sqrt(hd))
    Kf = np.concatenate([kp_o, kc_o])
    Vf = np.concatenate([vp_o, vc_o])
    want = oracle_run(s, RowsSpec(canvas), RowsSpec(list(range(n_t))), q_o, Kf, Vf)
    check(dev.get(out), want, "epilogue + step vs oracle")
    ok, ov = dev.empty(n_t * kvs), dev.empty(n_t * kvs)
    cache.gather(0, list(range(n_t)), ok, ov)
    # bf16 of the oracle's rows (an ulp of f32 from the norm's sum order can
    # move a bf16 rounding only at an exact tie, which these inputs avoid)
    assert np.array_equal(dev.get(ok), _normed_bf16(dev, Kf, None))
    assert np.array_equal(dev.get(ov), _normed_bf16(dev, Vf, None))


@pytest.mark.parametrize("h,hkv,hd,rot,n_p,n_c,batch,norm,v_norm,window,theta", [
    (16, 16, 128, 128, 512, 256, 1, True, False, None, 10000.0),   # C4-like, QK-norm
    (8, 2, 128, 64, 200, 93, 2, False, False, None, 500000.0),     # GQA, partial rotary, CFG pair
    (8, 4, 256, 256, 300, 120, 1, True, True, 128, 10000.0),       # Gemma-like: V-norm, window
])
def test_step_epi_vs_oracle(dev, h, hkv, hd, rot, n_p, n_c, batch, norm, v_norm, window, theta):
    """dr_attention_step_epi (the Q/K/V epilogue folded into the cache store
    and the attention prologue) against the oracle's epilogue + attention,
    and the cache against bf16 of the oracle's K / V rows."""
    rng = np.random.default_rng(hd + rot + batch)
    eps = 1e-6
    n_t = n_p + n_c
    kvs = hkv * hd
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norm else None
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if norm else None
    bq = (0.1 * rng.standard_normal(h * hd)).astype(np.float32)
    bk = (0.1 * rng.standard_normal(kvs)).astype(np.float32)
    bv = (0.1 * rng.standard_normal(kvs)).astype(np.float32)
    table = orc.rope_table(n_t, rot, theta)
    rope = dr.Rope(dev.ctx, n_t, rot, theta)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd], n_batch=batch)
    p_pr = dr.Pass(dev.ctx, range(n_p))
    canvas = list(range(n_p, n_t))
    p_c = dr.Pass(dev.ctx, canvas)
    put = lambda x: dev.put(x) if x is not None else None  # noqa: E731
    scale = 1 / math.sqrt(hd)
    items, outs, wants = [], [], []
    for b in range(batch):
        K = rng.standard_normal(n_t * kvs).astype(np.float32)
        V = rng.standard_normal(n_t * kvs).astype(np.float32)
        Q = rng.standard_normal(n_c * h * hd).astype(np.float32)
        kp, vp = K[:n_p * kvs].copy(), V[:n_p * kvs].copy()
        kc, vc = K[n_p * kvs:].copy(), V[n_p * kvs:].copy()
        # the prompt rows go through the two-pass path: epilogue, then store
        qd = np.zeros(n_p * h * hd, np.float32)
        dq0, dkp, dvp = put(qd), put(kp), put(vp)
        dr.qkv_epilogue(dev.ctx, p_pr, dq0, dkp, dvp, h, hkv, hd, put(bq), put(bk), put(bv),
                        put(qn), put(kn), v_norm, eps, rope)
        cache.store(0, p_pr, dkp, dvp, batch=b)
        _, kp_o, vp_o = _epilogue_oracle(qd, kp, vp, list(range(n_p)), h, hkv, hd, bq, bk, bv, qn,
                                         kn, v_norm, eps, table, rot)
        q_o, kc_o, vc_o = _epilogue_oracle(Q, kc, vc, canvas, h, hkv, hd, bq, bk, bv, qn, kn,
                                           v_norm, eps, table, rot)
        s = Shape(n_c, n_t, h, hkv, hd, sliding_window=window, scale=scale)
        Kf, Vf = np.concatenate([kp_o, kc_o]), np.concatenate([vp_o, vc_o])
        wants.append((oracle_run(s, RowsSpec(canvas), RowsSpec(list(range(n_t))), q_o, Kf, Vf),
                      Kf, Vf))
        out = dev.empty(n_c * h * hd)
        outs.append(out)
        items.append((put(Q), out, p_c, put(kc), put(vc)))
    say(f"step_epi h {h}/{hkv} hd {hd} rot {rot} batch {batch} norm {norm} v_norm {v_norm} "
        f"window {window}")
    cache.step_epi(0, items, h, sliding_window=window, scale=scale, bq=put(bq), bk=put(bk),
                   bv=put(bv), q_norm_w=put(qn), k_norm_w=put(kn), v_norm=v_norm, eps=eps,
                   rope=rope)
    # full rotary folds into the per-wave-stream kernel's Q load; partial
    # rotary (a dim's partner in another lane) runs on the staged kernel
    launch = dev.ctx.last_launch()
    say(f"  launch {launch}")
    assert launch["kernel"] == (dr.KERNEL_STREAMS if rot == hd else dr.KERNEL_STAGED)
    for b in range(batch):
        want, Kf, Vf = wants[b]
        check(dev.get(outs[b]), want, f"batch {b} vs oracle")
        ok, ov = dev.empty(n_t * kvs), dev.empty(n_t * kvs)
        cache.gather(0, list(range(n_t)), ok, ov, batch=b)
        gk, gv = dev.get(ok), dev.get(ov)
        wk, wv = _normed_bf16(dev, Kf, None), _normed_bf16(dev, Vf, None)
        # bf16 of the same f32 rows; a norm's f64 sum in another order can
        # move an f32 value by an ulp, which changes its bf16 rounding only
        # at an exact tie
        for name, g_, w_ in (("K", gk, wk), ("V", gv, wv)):
            bad = np.count_nonzero(g_ != w_)
            assert bad <= 2 and np.max(np.abs(g_ - w_)) <= 2.0**-7 * np.max(np.abs(w_)), (name, bad)


@pytest.mark.parametrize("h,hkv,hd,batch,window,prefix", [
    (28, 4, 128, 2, 96, None),    # 448 one-row-block workgroups: the RB 2 x KQ 4 shape, masked
    (28, 4, 128, 2, None, 700),   # the same shape under a causal prefix
    (8, 4, 256, 2, None, None),   # 16-row waves at hd 256, two batch slots
    (16, 2, 512, 2, 300, None),   # hd 512 split waves with a window, two batch slots
])
def test_batched_plans_vs_oracle(dev, h, hkv, hd, batch, window, prefix):
    """Launch shapes the planner picks for batched (CFG-pair) problems, under
    masks, against the oracle per batch slot."""
    rng = np.random.default_rng(h * 1000 + hd + (window or 0))
    n_p, n_c = 600, 256
    n_t = n_p + n_c
    kvs = hkv * hd
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd], n_batch=batch)
    p_all = dr.Pass(dev.ctx, range(n_t))
    pc = dr.Pass(dev.ctx, range(n_p, n_t))
    scale = 1 / math.sqrt(hd)
    items, ins, outs = [], [], []
    for b in range(batch):
        K = rng.standard_normal((n_t, kvs), dtype=np.float32)
        V = rng.standard_normal((n_t, kvs), dtype=np.float32)
        Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
        cache.store(0, p_all, dev.put(K), dev.put(V), batch=b)
        out = dev.empty(n_c * h * hd)
        items.append((dev.put(Q), out, pc))
        ins.append((Q, K, V))
        outs.append(out)
    cache.attention(0, items, h, sliding_window=window, causal_prefix=prefix, scale=scale)
    info = dev.ctx.last_launch()
    say(f"h {h}/{hkv} hd {hd} batch {batch} window {window} prefix {prefix}: launch {info}")
    s = Shape(n_c, n_t, h, hkv, hd, sliding_window=window, causal_prefix=prefix, scale=scale)
    qr, kr = RowsSpec(list(range(n_p, n_t))), RowsSpec(list(range(n_t)))
    for b in range(batch):
        Q, K, V = ins[b]
        want = oracle_run(s, qr, kr, *as_kernel_sees(Q.reshape(-1).copy(), K.reshape(-1).copy(),
                                                     V.reshape(-1).copy(), scale))
        got = dev.get(outs[b])
        check(got, want, f"batch {b}")
        check_raw(orc, got, Q.reshape(-1), K.reshape(-1), V.reshape(-1), s, qr, kr, f"batch {b}", say)

"""Cached attention with bf16 Q rows (dr_ctx_set_q_dtype; no counterpart in
the reference, whose attention() takes f32: for callers whose projections
produce bf16).  The per-wave-stream kernel widens each bf16 piece exactly to
f32 and then runs the f32 path, so its outputs must equal, bit for bit, the
f32 path fed with the same values; they also meet the standard bar against
the oracle of attention() (src/model/attention.rs:101-186) on those values.
Calls the kernel cannot run fail before any store.  Needs an MI355X.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import dr_attn as dr
import oracle as orc
from helpers import CONFIGS, RowsSpec, Shape, config_seed

from test_gpu_parity import _epilogue_oracle, check, dev, oracle_run, say, torch  # noqa: F401

pytestmark = pytest.mark.gpu


def _bf16(dev, x: np.ndarray):
    """(device bf16 tensor, its values as f32 numpy)"""
    t = dev.t
    with t.cuda.stream(dev.stream):
        b = t.from_numpy(np.ascontiguousarray(x)).to("cuda").to(t.bfloat16)
    return b, dev.get(b.float()).reshape(x.shape)


def _with_q_dtype(dev, dtype, fn):
    dev.ctx.set_q_dtype(dtype)
    try:
        return fn()
    finally:
        dev.ctx.set_q_dtype(dr.DTYPE_F32)


@pytest.mark.parametrize("cid", ["C2", "C4", "C5S"])
def test_bf16_q_equals_f32_path_and_oracle(dev, cid):
    cfg = CONFIGS[cid]
    rng = np.random.default_rng(config_seed(list(CONFIGS).index(cid), 3))
    h, hkv, hd, n_t, n_c = cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.n_total, cfg.n_canvas
    kvs = hkv * hd
    K = rng.standard_normal((n_t, kvs), dtype=np.float32)
    V = rng.standard_normal((n_t, kvs), dtype=np.float32)
    Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
    qn = kn = None
    if cfg.qk_norm:
        qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
        kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    cache.store(0, dr.Pass(dev.ctx, range(n_t)), dev.put(K), dev.put(V),
                dev.put(kn) if kn is not None else None, 1e-6)
    pc = dr.Pass(dev.ctx, range(cfg.n_prompt, n_t))
    qb, qv = _bf16(dev, Q)
    qnd = dev.put(qn) if qn is not None else None

    def run(q):
        out = dev.empty(n_c * h * hd)
        cache.attention(0, [(q, out, pc)], h, sliding_window=cfg.window, scale=cfg.attn_scale,
                        q_norm_w=qnd, q_norm_eps=1e-6)
        return dev.get(out), dev.ctx.last_launch()

    got_b, launch = _with_q_dtype(dev, dr.DTYPE_BF16, lambda: run(qb))
    got_f, _ = run(dev.put(qv))
    say(f"{cid} bf16 Q: launch {launch}")
    assert launch["kernel"] == dr.KERNEL_STREAMS
    assert np.array_equal(got_b.view(np.uint32), got_f.view(np.uint32)), cid
    q_o, k_o = qv.reshape(-1).copy(), K.reshape(-1).copy()
    if qn is not None:
        orc.norm_heads(q_o, qn, 1e-6)
        orc.norm_heads(k_o, kn, 1e-6)
    s = Shape(n_c, n_t, h, hkv, hd, sliding_window=cfg.window, scale=cfg.attn_scale)
    want = oracle_run(s, RowsSpec(list(range(cfg.n_prompt, n_t))), RowsSpec(list(range(n_t))), q_o, k_o,
                      V.reshape(-1).copy())
    check(got_b, want, f"{cid} bf16 Q vs oracle")


def test_bf16_q_step_epi_full_rotary(dev):
    """The folded epilogue (bias, QK-norm, full-rotary RoPE on Q) on bf16 Q
    rows: the same bits as on f32 rows of the same values, and the cache
    rows the step stores are those of the f32 step."""
    rng = np.random.default_rng(77)
    h, hkv, hd, n_p, n_c = 16, 16, 128, 384, 128
    n_t, kvs, eps = n_p + n_c, hkv * hd, 1e-6
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    bq = (0.1 * rng.standard_normal(h * hd)).astype(np.float32)
    K = rng.standard_normal((n_t, kvs), dtype=np.float32)
    V = rng.standard_normal((n_t, kvs), dtype=np.float32)
    Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
    rope = dr.Rope(dev.ctx, n_t, hd, 10000.0)
    qb, qv = _bf16(dev, Q)
    outs, caches = [], []
    for q, dtype in ((qb, dr.DTYPE_BF16), (dev.put(qv), dr.DTYPE_F32)):
        cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
        cache.store(0, dr.Pass(dev.ctx, range(n_p)), dev.put(K[:n_p].copy()), dev.put(V[:n_p].copy()))
        out = dev.empty(n_c * h * hd)
        item = (q, out, dr.Pass(dev.ctx, range(n_p, n_t)), dev.put(K[n_p:].copy()), dev.put(V[n_p:].copy()))
        _with_q_dtype(dev, dtype, lambda: cache.step_epi(0, [item], h, scale=1 / math.sqrt(hd), bq=dev.put(bq),
                                                          q_norm_w=dev.put(qn), k_norm_w=dev.put(kn), eps=eps,
                                                          rope=rope))
        assert dev.ctx.last_launch()["kernel"] == dr.KERNEL_STREAMS
        outs.append(dev.get(out))
        ok, ov = dev.empty(n_t * kvs), dev.empty(n_t * kvs)
        cache.gather(0, list(range(n_t)), ok, ov)
        caches.append((dev.get(ok), dev.get(ov)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.array_equal(caches[0][0], caches[1][0]) and np.array_equal(caches[0][1], caches[1][1])
    table = orc.rope_table(n_t, hd, 10000.0)
    q_o, kc_o, vc_o = _epilogue_oracle(qv.reshape(-1).copy(), K[n_p:].reshape(-1).copy(),
                                       V[n_p:].reshape(-1).copy(), list(range(n_p, n_t)), h, hkv, hd, bq,
                                       None, None, qn, kn, False, eps, table, hd)
    s = Shape(n_c, n_t, h, hkv, hd, scale=1 / math.sqrt(hd))
    want = oracle_run(s, RowsSpec(list(range(n_p, n_t))), RowsSpec(list(range(n_t))), q_o,
                      np.concatenate([K[:n_p].reshape(-1), kc_o]), np.concatenate([V[:n_p].reshape(-1), vc_o]))
    check(outs[0], want, "bf16 Q step_epi vs oracle")


def test_bf16_q_refused_where_the_stream_kernel_cannot_run(dev):
    """Head dim 64 (no stream kernel), partial rotary (a RoPE partner in
    another lane): DR_ERR_UNSUPPORTED, and the step stored nothing."""
    rng = np.random.default_rng(5)
    q = _bf16(dev, rng.standard_normal((32, 4 * 64), dtype=np.float32))[0]
    cache = dr.StepCache(dev.ctx, 96, [4], [64])
    with pytest.raises(dr.DrError) as ei:
        _with_q_dtype(dev, dr.DTYPE_BF16, lambda: cache.attention(0, [(q, dev.empty(32 * 256), dr.Pass(dev.ctx, range(64, 96)))],
                                                                  4, scale=0.125))
    assert ei.value.status == dr.DR_ERR_UNSUPPORTED
    # partial rotary: refused before the store
    h, hd, n_t = 4, 128, 96
    cache = dr.StepCache(dev.ctx, n_t, [h], [hd])
    before = (dev.empty(n_t * h * hd), dev.empty(n_t * h * hd))
    cache.gather(0, list(range(n_t)), *before)
    before = [dev.get(x) for x in before]
    qb = _bf16(dev, rng.standard_normal((32, h * hd), dtype=np.float32))[0]
    kv = dev.put(rng.standard_normal((32, h * hd), dtype=np.float32))
    rope = dr.Rope(dev.ctx, n_t, 64, 10000.0)
    item = (qb, dev.empty(32 * h * hd), dr.Pass(dev.ctx, range(64, 96)), kv, kv)
    with pytest.raises(dr.DrError) as ei:
        _with_q_dtype(dev, dr.DTYPE_BF16, lambda: cache.step_epi(0, [item], h, scale=0.1, rope=rope))
    assert ei.value.status == dr.DR_ERR_UNSUPPORTED
    after = (dev.empty(n_t * h * hd), dev.empty(n_t * h * hd))
    cache.gather(0, list(range(n_t)), *after)
    assert all(np.array_equal(x, dev.get(y), equal_nan=True) for x, y in zip(before, after))
    with pytest.raises(dr.DrError) as ei:
        dev.ctx.set_q_dtype(7)
    assert ei.value.status == dr.DR_ERR_INVALID


@pytest.mark.parametrize("cid,n_split,in_kernel", [("C2", 0, True), ("C4", 0, True), ("C5S", 0, True),
                                                   ("C2", 3, True), ("C2", 2, False)])
def test_bf16_out_is_the_f32_output_rounded(dev, cid, n_split, in_kernel):
    """bf16 output rows (dr_ctx_set_o_dtype): each element is the f32 path's
    output rounded to nearest even, bit for bit, unsplit, with key splits
    merged in-kernel and by split_merge_kernel; and within the bar of the
    oracle."""
    t = dev.t
    cfg = CONFIGS[cid]
    rng = np.random.default_rng(config_seed(list(CONFIGS).index(cid), 5))
    h, hkv, hd, n_t, n_c = cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.n_total, cfg.n_canvas
    kvs = hkv * hd
    K = rng.standard_normal((n_t, kvs), dtype=np.float32)
    V = rng.standard_normal((n_t, kvs), dtype=np.float32)
    Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
    qn = kn = None
    if cfg.qk_norm:
        qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
        kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    cache.store(0, dr.Pass(dev.ctx, range(n_t)), dev.put(K), dev.put(V),
                dev.put(kn) if kn is not None else None, 1e-6)
    pc = dr.Pass(dev.ctx, range(cfg.n_prompt, n_t))
    qd = dev.put(Q)
    qnd = dev.put(qn) if qn is not None else None
    dev.ctx.set_split(n_split)
    dev.ctx.set_split_merge(in_kernel)
    try:
        out_f = dev.empty(n_c * h * hd)
        cache.attention(0, [(qd, out_f, pc)], h, sliding_window=cfg.window, scale=cfg.attn_scale,
                        q_norm_w=qnd, q_norm_eps=1e-6)
        with t.cuda.stream(dev.stream):
            out_b = t.full((n_c * h * hd,), float("nan"), dtype=t.bfloat16, device="cuda")
        dev.ctx.set_o_dtype(dr.DTYPE_BF16)
        try:
            cache.attention(0, [(qd, out_b, pc)], h, sliding_window=cfg.window, scale=cfg.attn_scale,
                            q_norm_w=qnd, q_norm_eps=1e-6)
            launch = dev.ctx.last_launch()
        finally:
            dev.ctx.set_o_dtype(dr.DTYPE_F32)
    finally:
        dev.ctx.set_split(0)
        dev.ctx.set_split_merge(True)
    say(f"{cid} bf16 out (split {n_split}, in-kernel {in_kernel}): launch {launch}")
    assert launch["kernel"] == dr.KERNEL_STREAMS
    if n_split:
        assert launch["n_split"] == n_split and launch["split_merge"] == (2 if in_kernel else 1)
    got_f = dev.get(out_f)
    with t.cuda.stream(dev.stream):
        want_bits = out_f.to(t.bfloat16).view(t.int16)
        got_bits = out_b.view(t.int16)
    assert np.array_equal(dev.get(got_bits), dev.get(want_bits)), cid
    q_o, k_o = Q.reshape(-1).copy(), K.reshape(-1).copy()
    if qn is not None:
        orc.norm_heads(q_o, qn, 1e-6)
        orc.norm_heads(k_o, kn, 1e-6)
    s = Shape(n_c, n_t, h, hkv, hd, sliding_window=cfg.window, scale=cfg.attn_scale)
    want = oracle_run(s, RowsSpec(list(range(cfg.n_prompt, n_t))), RowsSpec(list(range(n_t))), q_o, k_o,
                      V.reshape(-1).copy())
    with t.cuda.stream(dev.stream):
        got_b32 = out_b.float()
    check(dev.get(got_b32), want, f"{cid} bf16 out vs oracle")
    assert not np.any(np.isnan(got_f))

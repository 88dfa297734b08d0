"""Head dim 512 (DiffusionGemma's global layers: 16 query heads over 2 KV
heads, full attention, RoPE over all 512 dims with theta 1e6, K reused as V
when the layer has no attn_v; docs/diffusiongemma.md:11-12,
src/model/loader.rs:381-397, src/model/forward.rs:291-343) through the C ABI,
against the CPU oracle.  The reference handles any head_dim
(attention.rs:135-138 keeps the accumulator on the heap above 256); the
kernel splits the head dim over a pair of waves.  Needs an MI355X.
"""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

import dr_attn as dr
import oracle as orc
from helpers import RowsSpec, Shape, as_kernel_sees, err_stats

from test_gpu_parity import _epilogue_oracle, _normed_bf16, check, dev, oracle_run, say, torch  # noqa: F401

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hd", [512, 384, 260])
def test_hd512_dropin_random_masks_vs_oracle(torch, hd):
    """The drop-in at head dims that take the 512 tile (384 and 260: a
    ragged head dim inside it), with arbitrary key order, windows, causal
    prefixes and sequence ids, and without a mask."""
    rng = np.random.default_rng(5120 + hd)
    h, hkv = 4, 2
    nq, nk = 70, 200
    sc = 1 / math.sqrt(hd)
    q = rng.standard_normal(nq * h * hd).astype(np.float32)
    k = rng.standard_normal(nk * hkv * hd).astype(np.float32)
    v = rng.standard_normal(nk * hkv * hd).astype(np.float32)
    # unmasked
    s = Shape(nq, nk, h, hkv, hd, scale=sc)
    qr, kr = RowsSpec(list(range(nq))), RowsSpec(list(range(nk)))
    got = np.zeros(nq * h * hd, np.float32)
    say(f"hd {hd} drop-in, no mask")
    dr.attention(got, q, k, v, dr.AttnShape(**s.__dict__), dr.idpos(nq), dr.idpos(nk))
    check(got, oracle_run(s, qr, kr, q, k, v), f"hd {hd} no mask")
    # masked, keys in arbitrary order with sequence ids
    kpos = rng.permutation(nk).tolist()
    qpos = sorted(rng.choice(nk, nq, replace=False).tolist())
    seq_k = (np.asarray(kpos) >= 150).astype(int).tolist()
    seq_q = (np.asarray(qpos) >= 150).astype(int).tolist()
    s = Shape(nq, nk, h, hkv, hd, sliding_window=int(rng.integers(20, 60)),
              causal_prefix=int(rng.integers(0, 120)), scale=sc)
    qr, kr = RowsSpec(qpos, seq_q), RowsSpec(kpos, seq_k)
    say(f"hd {hd} drop-in, window {s.sliding_window} prefix {s.causal_prefix}")
    got = np.zeros(nq * h * hd, np.float32)
    dr.attention(got, q, k, v, dr.AttnShape(**s.__dict__), dr.Rows(qpos, seq_q), dr.Rows(kpos, seq_k))
    # windows of 20..60 keys average few V rows; the drop-in's hi/lo scores
    # and values hold the f32 comparison to the standard bar
    check(got, oracle_run(s, qr, kr, q, k, v), f"hd {hd} masked (f32 inputs)")


@pytest.mark.parametrize("n_split", [0, 1, 3])
def test_hd512_global_layer_cached_vs_oracle(dev, n_split):
    """The global layer's geometry (16/2 heads, group 8, hd 512) over a 1024
    prompt + 256 canvas cache: store by position, attend with the canvas
    queries, at the automatic key split and at forced ones."""
    rng = np.random.default_rng(512)
    h, hkv, hd, n_p, n_c = 16, 2, 512, 1024, 256
    n_t = n_p + n_c
    kvs = hkv * hd
    K = rng.standard_normal((n_t, kvs), dtype=np.float32)
    V = rng.standard_normal((n_t, kvs), dtype=np.float32)
    Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    cache.store(0, dr.Pass(dev.ctx, range(n_t)), dev.put(K), dev.put(V))
    pc = dr.Pass(dev.ctx, range(n_p, n_t))
    scale = 1 / math.sqrt(hd)
    s = Shape(n_c, n_t, h, hkv, hd, scale=scale)
    want = oracle_run(s, RowsSpec(list(range(n_p, n_t))), RowsSpec(list(range(n_t))),
                      Q.reshape(-1).copy(), K.reshape(-1).copy(), V.reshape(-1).copy())
    out = dev.empty(n_c * h * hd)
    say(f"hd 512 global layer, n_split {n_split}")
    dev.ctx.set_split(n_split)
    try:
        cache.attention(0, [(dev.put(Q), out, pc)], h, scale=scale)
        info = dev.ctx.last_launch()
    finally:
        dev.ctx.set_split(0)
    say(f"  launch {info}")
    assert info["head_dim_tile"] == 512 and info["waves_per_wg"] == 8 and info["rows_per_wave"] == 16
    if n_split:
        assert info["n_split"] == n_split
    check(dev.get(out), want, f"global layer split {info['n_split']}")
    # the cache holds bf16 of the stored rows
    ok, ov = dev.empty(n_t * kvs), dev.empty(n_t * kvs)
    cache.gather(0, list(range(n_t)), ok, ov)
    assert np.array_equal(dev.get(ok), _normed_bf16(dev, K.reshape(-1), None))
    assert np.array_equal(dev.get(ov), _normed_bf16(dev, V.reshape(-1), None))


def test_hd512_step_epi_k_as_v_vs_oracle(dev):
    """A global layer's whole attention block from the raw projections:
    K reused as V (the same device buffer passed as k and v), K's RMSNorm
    with its gain and RoPE over all 512 dims at theta 1e6, Gemma's unweighted
    V-norm, Q's norm and RoPE, folded into the cache store and the attention
    (dr_attention_step_epi), against the oracle's epilogue + attention."""
    rng = np.random.default_rng(5121)
    h, hkv, hd, n_p, n_c, eps, theta = 16, 2, 512, 768, 256, 1e-6, 1e6
    n_t = n_p + n_c
    kvs = hkv * hd
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    table = orc.rope_table(n_t, hd, theta)
    rope = dr.Rope(dev.ctx, n_t, hd, theta)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    K = rng.standard_normal(n_t * kvs).astype(np.float32)
    Q = rng.standard_normal(n_c * h * hd).astype(np.float32)
    kp, kc = K[:n_p * kvs].copy(), K[n_p * kvs:].copy()
    put = dev.put
    # prompt rows: the two-pass path (epilogue in place, then store), with
    # separate K and V copies of the same projection
    p_pr = dr.Pass(dev.ctx, range(n_p))
    qd = np.zeros(n_p * h * hd, np.float32)
    dq0, dkp, dvp = put(qd), put(kp), put(kp)
    dr.qkv_epilogue(dev.ctx, p_pr, dq0, dkp, dvp, h, hkv, hd, None, None, None, put(qn), put(kn),
                    True, eps, rope)
    cache.store(0, p_pr, dkp, dvp)
    _, kp_o, vp_o = _epilogue_oracle(qd, kp, kp, list(range(n_p)), h, hkv, hd, None, None, None,
                                     qn, kn, True, eps, table, hd)
    canvas = list(range(n_p, n_t))
    p_c = dr.Pass(dev.ctx, canvas)
    q_o, kc_o, vc_o = _epilogue_oracle(Q, kc, kc, canvas, h, hkv, hd, None, None, None, qn, kn,
                                       True, eps, table, hd)
    scale = 1 / math.sqrt(hd)
    s = Shape(n_c, n_t, h, hkv, hd, scale=scale)
    Kf, Vf = np.concatenate([kp_o, kc_o]), np.concatenate([vp_o, vc_o])
    want = oracle_run(s, RowsSpec(canvas), RowsSpec(list(range(n_t))), q_o, Kf, Vf)
    dk = put(kc)
    out = dev.empty(n_c * h * hd)
    say("hd 512 step_epi, K as V")
    cache.step_epi(0, [(put(Q), out, p_c, dk, dk)], h, scale=scale, q_norm_w=put(qn),
                   k_norm_w=put(kn), v_norm=True, eps=eps, rope=rope)
    check(dev.get(out), want, "hd 512 step_epi K-as-V")
    # the raw projection was only read
    assert np.array_equal(dev.get(dk), kc)
    ok, ov = dev.empty(n_t * kvs), dev.empty(n_t * kvs)
    cache.gather(0, list(range(n_t)), ok, ov)
    for name, g_, w_ in (("K", dev.get(ok), _normed_bf16(dev, Kf, None)),
                         ("V", dev.get(ov), _normed_bf16(dev, Vf, None))):
        bad = np.count_nonzero(g_ != w_)
        assert bad <= 2 and np.max(np.abs(g_ - w_)) <= 2.0**-7 * np.max(np.abs(w_)), (name, bad)


def test_hd512_scale_one_hilo_layer(dev):
    """Gemma's real kq_scale is 1.0 (forward.rs:338-341).  With N(0,1) inputs
    at hd 512 the score std is ~23 and the softmax is nearly one-hot: bf16
    Q/K err by ~0.25.  A layer kept at DR_PRECISION_HILO (f32-accurate scores
    and values) meets the north-star tolerance."""
    rng = np.random.default_rng(5122)
    h, hkv, hd, n_t, n_c = 16, 2, 512, 512, 128
    n_p = n_t - n_c
    K = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
    V = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
    Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    cache.set_precision(0, dr.PRECISION_HILO)
    cache.store(0, dr.Pass(dev.ctx, range(n_t)), dev.put(K), dev.put(V))
    out = dev.empty(n_c * h * hd)
    cache.attention(0, [(dev.put(Q), out, dr.Pass(dev.ctx, range(n_p, n_t)))], h, scale=1.0)
    assert dev.ctx.last_launch()["kernel"] == dr.KERNEL_HILO
    s = Shape(n_c, n_t, h, hkv, hd, scale=1.0)
    want = oracle_run(s, RowsSpec(list(range(n_p, n_t))), RowsSpec(list(range(n_t))),
                      Q.reshape(-1).copy(), K.reshape(-1).copy(), V.reshape(-1).copy())
    check(dev.get(out), want, "hd 512 scale 1.0 (N(0,1)), hi/lo layer")

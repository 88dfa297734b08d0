"""dr_attention_step_rows on the rows of a fused QKV projection (Qkv::Fused,
src/model/forward.rs:281-289: [n][n_head*hd + 2*n_head_kv*hd] per active
row, which the reference copies apart into b.q / b.k / b.v before the
epilogue).  Read in place through row strides, the step must give the same
bits -- outputs and cache contents -- as dr_attention_step_epi on the copied
Q, K and V, on every path the strides touch: the per-wave-stream kernel's Q
load with the folded epilogue, the staged kernel's (partial rotary), the
hi/lo kernel's Q copy, the whole-tile store and the position-list store, two
batch slots.  Needs an MI355X.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import dr_attn as dr

from test_gpu_parity import dev, say, torch  # noqa: F401

pytestmark = pytest.mark.gpu

# (h, hkv, hd, n_prompt, canvas positions, batch, rope dims, precision, epilogue)
CASES = {
    "streams_full_epi": (16, 16, 128, 256, list(range(256, 384)), 1, 128, None, True),
    "staged_partial_rotary": (8, 2, 128, 200, list(range(200, 264)), 1, 64, None, True),
    "hilo_gqa_epi": (8, 4, 256, 300, list(range(300, 364)), 1, 256, dr.PRECISION_HILO, True),
    "scattered_batch2": (8, 4, 128, 0, sorted(np.random.default_rng(0).choice(320, 90, replace=False).tolist()),
                         2, 128, None, True),
    "no_epilogue": (4, 4, 64, 64, list(range(64, 96)), 1, 0, None, False),
}


@pytest.mark.parametrize("name", list(CASES))
def test_fused_qkv_rows_equal_copied_rows(dev, name):
    t = dev.t
    h, hkv, hd, n_p, pos, batch, rot, prec, use_epi = CASES[name]
    rng = np.random.default_rng(sum(map(ord, name)))
    n_t = max(n_p, max(pos) + 1)
    n = len(pos)
    qs, kvs = h * hd, hkv * hd
    fused = qs + 2 * kvs
    eps = 1e-6
    kw = dict(scale=1 / math.sqrt(hd))
    if use_epi:
        kw.update(bq=dev.put((0.1 * rng.standard_normal(qs)).astype(np.float32)),
                  bk=dev.put((0.1 * rng.standard_normal(kvs)).astype(np.float32)),
                  bv=dev.put((0.1 * rng.standard_normal(kvs)).astype(np.float32)),
                  q_norm_w=dev.put(rng.uniform(0.5, 1.5, hd).astype(np.float32)),
                  k_norm_w=dev.put(rng.uniform(0.5, 1.5, hd).astype(np.float32)), eps=eps,
                  rope=dr.Rope(dev.ctx, n_t, rot, 10000.0) if rot else None)
    prompt = [(rng.standard_normal((n_p, kvs), dtype=np.float32), rng.standard_normal((n_p, kvs), dtype=np.float32))
              for _ in range(batch)]
    rows = [rng.standard_normal((n, fused), dtype=np.float32) for _ in range(batch)]
    p = dr.Pass(dev.ctx, pos)
    results = []
    for mode in ("copied", "fused"):
        cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd], n_batch=batch,
                             precision=None if prec is None else [prec])
        if n_p:
            for b in range(batch):
                cache.store(0, dr.Pass(dev.ctx, range(n_p)), dev.put(prompt[b][0]), dev.put(prompt[b][1]), batch=b)
        outs, keep = [], []
        if mode == "copied":
            items = []
            for b in range(batch):
                out = dev.empty(n * qs)
                q, k, v = (dev.put(rows[b][:, :qs].copy()), dev.put(rows[b][:, qs:qs + kvs].copy()),
                           dev.put(rows[b][:, qs + kvs:].copy()))
                items.append((q, out, p, k, v))
                outs.append(out)
            cache.step_epi(0, items, h, **kw)
        else:
            items = []
            for b in range(batch):
                out = dev.empty(n * qs)
                r = dev.put(rows[b])
                keep.append(r)
                base = r.data_ptr()
                items.append((base, out, p, base + 4 * qs, base + 4 * (qs + kvs)))
                outs.append(out)
            cache.step_rows(0, items, h, fused, fused, **kw)
        launch = dev.ctx.last_launch()
        got = [dev.get(o) for o in outs]
        cache_rows = []
        for b in range(batch):
            ok, ov = dev.empty(n_t * kvs), dev.empty(n_t * kvs)
            cache.gather(0, list(range(n_t)), ok, ov, batch=b)
            cache_rows.append((dev.get(ok), dev.get(ov)))
        results.append((got, cache_rows, launch))
    (g0, c0, l0), (g1, c1, l1) = results
    say(f"{name}: launch {l1}")
    assert l0["kernel"] == l1["kernel"]
    if prec is not None:
        assert l1["kernel"] == dr.KERNEL_HILO
    for b in range(batch):
        assert not np.any(np.isnan(g0[b]))
        assert np.array_equal(g0[b].view(np.uint32), g1[b].view(np.uint32)), (name, b)
        assert np.array_equal(c0[b][0], c1[b][0]) and np.array_equal(c0[b][1], c1[b][1]), (name, b)


def test_step_rows_rejects_bad_strides(dev):
    h, hd, n_t = 4, 64, 64
    cache = dr.StepCache(dev.ctx, n_t, [h], [hd])
    p = dr.Pass(dev.ctx, range(32, 64))
    buf = dev.put(np.zeros((32, 3 * h * hd + 4), np.float32))
    base = buf.data_ptr()
    item = (base, dev.empty(32 * h * hd), p, base + 4 * h * hd, base + 8 * h * hd)
    for qst, kvst in ((h * hd - 4, 3 * h * hd), (3 * h * hd + 2, 3 * h * hd), (3 * h * hd, h * hd - 1)):
        with pytest.raises(dr.DrError) as ei:
            cache.step_rows(0, [item], h, qst, kvst, scale=0.1)
        assert ei.value.status == dr.DR_ERR_INVALID

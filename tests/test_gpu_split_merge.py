"""Key splits of the per-wave-stream kernel merged in-kernel
(dr_ctx_set_split_merge): the last split of each 32-row block to finish
merges the partials, which every split writes and reads with agent-scope
accesses, and resets the block's ticket.  The merge is the softmax-state
merge of attention() split over key ranges (src/model/attention.rs:101-186):
it must give the values of the separate merge kernel (the same operations in
the same split order), meet the oracle bar, repeat bit for bit, leave every
ticket at zero for the next call (later calls of other shapes, graph
replays) and handle splits that see no key tile.  Needs an MI355X.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import dr_attn as dr
from helpers import TOL_MAX, TOL_MEAN, err_stats

from test_gpu_kernels import CASES, CASES_256, _run, dev, say  # noqa: F401

pytestmark = pytest.mark.gpu


def _with(dev, in_kernel, fn):
    dev.ctx.set_split_merge(in_kernel)
    try:
        return fn()
    finally:
        dev.ctx.set_split_merge(True)


def _forced(dev, name, hd, n_split, in_kernel):
    table = CASES if hd == 128 else CASES_256
    saved = table[name]
    table[name] = saved[:8] + (n_split,)
    try:
        return _with(dev, in_kernel, lambda: _run(dev, name, dr.KERNEL_STREAMS, hd))
    finally:
        table[name] = saved


# (head dim, case, splits): MHA and GQA, batch slots, ragged key and row
# tails, windows and causal prefixes whose bands leave some splits of some
# row blocks without a key tile, QK-norm
MERGE_CASES = [
    (128, "mha", 2), (128, "mha", 3), (128, "mha", 4),
    (128, "mha_ragged", 4), (128, "gqa_batch2", 2), (128, "window", 4),
    (128, "prefix", 3), (128, "window_prefix", 4), (128, "qk_norm", 2),
    (256, "mha", 2), (256, "ragged", 2), (256, "gqa_batch2", 2),
    (256, "window", 2), (256, "window_prefix", 2), (256, "qk_norm", 2),
]


@pytest.mark.parametrize("hd,name,n_split", MERGE_CASES,
                         ids=[f"hd{h}-{n}-s{s}" for h, n, s in MERGE_CASES])
def test_in_kernel_merge_equals_merge_kernel_and_oracle(dev, hd, name, n_split):
    got_k, wants, info_k = _forced(dev, name, hd, n_split, False)
    got_i, _, info_i = _forced(dev, name, hd, n_split, True)
    say(f"hd {hd} {name} split {n_split}: in-kernel {info_i}")
    assert info_i["kernel"] == dr.KERNEL_STREAMS and info_i["n_split"] == n_split
    assert info_i["split_merge"] == 2 and info_k["split_merge"] == 1
    for b, (gi, gk, w) in enumerate(zip(got_i, got_k, wants)):
        assert np.array_equal(gi, gk, equal_nan=True), (name, b)
        mx, mean = err_stats(gi, w)
        say(f"  batch {b}: max-abs {mx:.3e} mean-abs {mean:.3e}")
        assert mx <= TOL_MAX and mean <= TOL_MEAN, (name, b, mx, mean)
    # tickets back at zero: the same call again, bit for bit
    again, _, _ = _forced(dev, name, hd, n_split, True)
    for x, y in zip(got_i, again):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_more_splits_than_registers_use_the_merge_kernel(dev):
    """Splits beyond what the kernel merges in registers (3 at hd 256) fall
    back to the merge kernel, with the same result."""
    got, wants, info = _forced(dev, "split3_window", 256, 3, True)
    assert info["n_split"] == 3 and info["split_merge"] == 1
    for g, w in zip(got, wants):
        mx, mean = err_stats(g, w)
        assert mx <= TOL_MAX and mean <= TOL_MEAN


def test_tickets_reset_across_shapes(dev):
    """Calls of different shapes in a row share the context's tickets: a
    large split call, a smaller one (fewer row blocks), then the large one
    again give what each gives alone."""
    first, _, _ = _forced(dev, "mha", 128, 4, True)
    small, small_want, _ = _forced(dev, "mha_ragged", 128, 2, True)
    third, _, _ = _forced(dev, "mha", 128, 4, True)
    for x, y in zip(first, third):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    for g, w in zip(small, small_want):
        mx, mean = err_stats(g, w)
        assert mx <= TOL_MAX and mean <= TOL_MEAN


def test_graph_replays_of_in_kernel_merge(dev):
    """One split attention call captured in a HIP graph and replayed
    several times, with eager calls and synchronisations between the
    replays: every replay equals the eager result (the kernel resets its
    own tickets; nothing is cleared by a memset node)."""
    t = dev.t
    h, hkv, hd, n_p, n_c = 8, 8, 128, 900, 128
    n_t = n_p + n_c
    rng = np.random.default_rng(2024)
    K = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
    V = rng.standard_normal((n_t, hkv * hd), dtype=np.float32)
    Q = rng.standard_normal((n_c, h * hd), dtype=np.float32)
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    cache.store(0, dr.Pass(dev.ctx, range(n_t)), dev.put(K), dev.put(V))
    pc = dr.Pass(dev.ctx, range(n_p, n_t))
    q = dev.put(Q)
    out = dev.empty(n_c * h * hd)
    dev.ctx.set_kernel(dr.KERNEL_STREAMS)
    dev.ctx.set_split(3)
    try:
        cache.attention(0, [(q, out, pc)], h, scale=1 / math.sqrt(hd))
        assert dev.ctx.last_launch()["split_merge"] == 2
        eager = dev.get(out).copy()
        g = t.cuda.CUDAGraph()
        with t.cuda.graph(g, stream=dev.stream, capture_error_mode="thread_local"):
            cache.attention(0, [(q, out, pc)], h, scale=1 / math.sqrt(hd))
        dev.stream.synchronize()
        for i in range(4):
            with t.cuda.stream(dev.stream):
                out.fill_(float("nan"))
                g.replay()
            got = dev.get(out)
            assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), i
            # an eager call of another shape between the replays
            small = dev.empty(64 * h * hd)
            cache.attention(0, [(q[:64], small, dr.Pass(dev.ctx, range(n_p, n_p + 64)))], h,
                            scale=1 / math.sqrt(hd))
            dev.stream.synchronize()
    finally:
        dev.ctx.set_kernel(dr.KERNEL_AUTO)
        dev.ctx.set_split(0)
    say("graph replays: equal to the eager call")


def test_planner_splits_gemma_sliding_layer_in_kernel(dev):
    """DiffusionGemma's sliding layer (C5 sliding: canvas rows at the end, a
    band of 1279 keys at head dim 256) runs 16-row waves, 256 workgroups with
    no key split, whether the in-kernel merge is on or off.  The same window
    over canvas rows in the middle of the sequence (a band of 2302 keys)
    keeps the 32-row kernel: two key splits merged in-kernel, and unsplit when
    the in-kernel merge is off (the separate merge kernel made the split
    lose)."""
    from helpers import CONFIGS
    cfg = CONFIGS["C5S"]
    h, hkv, hd, n_t, n_c = cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.n_total, cfg.n_canvas
    cache = dr.StepCache(dev.ctx, n_t, [hkv], [hd])
    z = dev.put(np.zeros((n_t, hkv * hd), np.float32))
    cache.store(0, dr.Pass(dev.ctx, range(n_t)), z, z)
    q = dev.put(np.zeros((n_c, h * hd), np.float32))
    for first, want_on, want_off in ((cfg.n_prompt, (16, 1, 0), (16, 1, 0)), (2048, (32, 2, 2), (32, 1, 0))):
        item = [(q, dev.empty(n_c * h * hd), dr.Pass(dev.ctx, range(first, first + n_c)))]
        cache.attention(0, item, h, sliding_window=cfg.window, scale=cfg.attn_scale)
        info = dev.ctx.last_launch()
        assert info["kernel"] == dr.KERNEL_STREAMS, info
        assert (info["rows_per_wave"], info["n_split"], info["split_merge"]) == want_on, (first, info)
        _with(dev, False, lambda: cache.attention(0, item, h, sliding_window=cfg.window, scale=cfg.attn_scale))
        info = dev.ctx.last_launch()
        assert info["kernel"] == dr.KERNEL_STREAMS, info
        assert (info["rows_per_wave"], info["n_split"], info["split_merge"]) == want_off, (first, info)

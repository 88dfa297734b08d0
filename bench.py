#!/usr/bin/env python3
"""Benchmark: denoise-step attention on one MI355X (BASELINE.json metric).

Workload ("C2"): LLaDA-8B shape, 32 query heads =
32 KV heads, head_dim 128, 512 cached prompt rows + 256 canvas rows, batch 1,
bidirectional, scale 1/sqrt(128).  The cache holds LLaDA-8B's 32 layers
(32 x 12 MiB of bf16 K/V, more than the 256 MB Infinity Cache), each with the
prompt K/V stored once.  Step i works on layer i mod 32: store the step's 256
fresh canvas K/V rows into that layer's cache (f32 -> bf16, by position) +
attention of the 256 canvas queries over all 768 keys (the attention_block
sequence of forward.rs:312-343).  Inputs (16 distinct canvas sets, f32
N(0,1), seeded) are resident in HBM before the timed region.

value = algorithmic attention FLOPs of K steps / wall time of the K steps,
all of them graph replays (a graph of 32 steps, and one of the remainder),
FLOPs = 4 * h * hd * sum_q |visible keys| = 3.221 GFLOP per step (softmax,
masking and the store excluded).  roofline = the attention kernel alone:
the same FLOPs / its mean launch duration over a graph of 32 back-to-back
calls, one per layer (so K/V come from HBM, as in a real step), timed with
HIP events on the library's stream, against 2516.6 TFLOP/s dense bf16 MFMA;
its traffic is the HBM bytes per launch from the rocprofv3 FETCH_SIZE /
WRITE_SIZE record in profiles/.  other_configs_attention_only = the same
timing for configs[2..4] (C5 also as its 6-layer S,S,S,S,S,G set).
cpu_baseline = the C restatement of the reference's AVX2 attention (oracle/,
"port") timed on this host's cores on a bounded sample of the same workload;
its output also checks the GPU result.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode eager|graph]
       python bench.py --only CFG [--calls N]   (one config's attention, for profiling)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "diffuse-rs_amd"))
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "tests"))

METRIC = "attn TFLOP/s & % bf16 MFMA peak per denoise step, LLaDA-8B shape, 1 MI355X"
PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0
PEAK_INT8_TOPS = 5000.0  # dense int8 MFMA


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def measured_traffic(cfg_name: str):
    """HBM bytes per attention launch at a config, as measured by the two
    rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) recorded in
    profiles/attn_<cfg>_traffic.txt, or (None, None) if that record is absent."""
    path = ROOT / "profiles" / f"attn_{cfg_name}_traffic.txt"
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch"):
                return int(float(line.split("=")[1])), path.name
    except (OSError, ValueError, IndexError):
        pass
    return None, None


def attention_only_ms(torch, stream, call, n_calls: int, reps: int):
    """Mean duration of one call(i), i < n_calls: the calls are captured in a
    graph, replayed `reps` times between two events on `stream`."""
    with torch.cuda.stream(stream):
        for i in range(n_calls):
            call(i)
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
        for i in range(n_calls):
            call(i)
    stream.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for _ in range(2):
            g.replay()
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
    stream.synchronize()
    return e0.elapsed_time(e1) / (reps * n_calls), g


def _config_cache(torch, dr, ctx, stream, cfg, gen, n_layer: int = 1, windows=None, precision=None):
    """A cache of n_layer layers of cfg's geometry with random K/V stored in
    every layer and batch slot, and the attention items of its canvas rows."""
    h, hkv, hd = cfg.n_head, cfg.n_head_kv, cfg.head_dim
    n_t, n_c = cfg.n_total, cfg.n_canvas
    cache = dr.StepCache(ctx, n_t, [hkv] * n_layer, [hd] * n_layer, n_batch=cfg.batch)
    if precision is not None:
        for layer in range(n_layer):
            cache.set_precision(layer, precision)
    p_all = dr.Pass(ctx, range(n_t))
    p_can = dr.Pass(ctx, range(cfg.n_prompt, n_t))
    qn = kn = None
    with torch.cuda.stream(stream):
        if cfg.qk_norm:
            qn = torch.rand(hd, device="cuda", generator=gen) + 0.5
            kn = torch.rand(hd, device="cuda", generator=gen) + 0.5
        Q = [torch.randn(n_c, h * hd, device="cuda", generator=gen) for _ in range(cfg.batch)]
        O = [torch.empty(n_c * h * hd, device="cuda") for _ in range(cfg.batch)]
    for layer in range(n_layer):
        for b in range(cfg.batch):
            with torch.cuda.stream(stream):
                K = torch.randn(n_t, hkv * hd, device="cuda", generator=gen)
                V = torch.randn(n_t, hkv * hd, device="cuda", generator=gen)
            cache.store(layer, p_all, K, V, k_norm_w=kn, batch=b)
    stream.synchronize()
    items = [(Q[b], O[b], p_can) for b in range(cfg.batch)]
    return cache, items, qn, (p_all, p_can)


def other_configs(torch, dr, ctx, stream, CONFIGS, reps: int) -> dict:
    """Attention-only TFLOP/s of the other BASELINE.json configs, of C5 as
    the 6-layer set it states (5 sliding + 1 global layer), and of a real
    DiffusionGemma global layer at head dim 512 (synthetic N(0,1) inputs;
    graph bursts of 4 calls on one layer's cache, as the roofline's warm
    figure; the C5 set is one graph of its 6 layers)."""
    res = {}
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    from helpers import EXTRA_CONFIGS
    for name in ("C3", "C4", "C5S", "C5G", "G512"):
        cfg = CONFIGS[name] if name in CONFIGS else EXTRA_CONFIGS[name]
        cache, items, qn, _ = _config_cache(torch, dr, ctx, stream, cfg, gen)

        def call(i):
            cache.attention(0, items, cfg.n_head, sliding_window=cfg.window, scale=cfg.attn_scale,
                            q_norm_w=qn)
        ms, _ = attention_only_ms(torch, stream, call, 4, reps)
        fl = cfg.flops()
        traffic, src = measured_traffic(name)
        res[name] = {"workload": cfg.name, "us_per_call": round(ms * 1e3, 3),
                     "tflops": round(fl / (ms / 1e3) / 1e12, 2),
                     "pct_of_peak": round(100 * fl / (ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 2),
                     "traffic": traffic, "traffic_source": src,
                     "launch": ctx.last_launch()}
        log(f"{name}: {res[name]}")
        stream.synchronize()
        del cache
    # C5 as stated: layers S,S,S,S,S,G of one cache, one call each
    cs, cg = CONFIGS["C5S"], CONFIGS["C5G"]
    cache, items, _, _ = _config_cache(torch, dr, ctx, stream, cs, gen, n_layer=6)

    def six(i):
        layer = i % 6
        cache.attention(layer, items, cs.n_head, sliding_window=cs.window if layer < 5 else None,
                        scale=cs.attn_scale)
    ms6, _ = attention_only_ms(torch, stream, six, 6, max(2, reps // 2))
    fl6 = 5 * cs.flops() + cg.flops()
    t6 = ms6 * 6 / 1e3  # seconds per 6-layer set
    res["C5_6layer"] = {"workload": "C5: 6 layers S,S,S,S,S,G (window 1024 / global), 16/8 heads, "
                                    "hd 256, 4096 cached + 256 canvas",
                        "us_per_6_layers": round(t6 * 1e6, 3), "tflops": round(fl6 / t6 / 1e12, 2),
                        "pct_of_peak": round(100 * fl6 / t6 / 1e12 / PEAK_BF16_TFLOPS, 2),
                        "gflop": round(fl6 / 1e9, 3)}
    log(f"C5_6layer: {res['C5_6layer']}")
    stream.synchronize()
    del cache
    return res


def hilo_timing(torch, dr, ctx, stream, CONFIGS, reps: int) -> dict:
    """The cost of hi/lo-precision layers (dr_cache_set_precision), which
    Gemma's kq_scale 1.0 needs: C5's sliding and global layers and the hd 512
    global layer at scale 1.0 with QK-norm, each on a bf16 layer and on a
    hi/lo layer (attention only, graph bursts as other_configs; the accuracy
    of both is in tests/test_gpu_hilo.py)."""
    import dataclasses
    from helpers import EXTRA_CONFIGS
    res = {}
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4321)
    for name in ("C5S", "C5G", "G512"):
        base = CONFIGS[name] if name in CONFIGS else EXTRA_CONFIGS[name]
        cfg = dataclasses.replace(base, scale=1.0, qk_norm=True)
        entry = {"workload": cfg.name + ", scale 1.0, QK-norm"}
        for label, prec in (("bf16", None), ("hilo", dr.PRECISION_HILO)):
            cache, items, qn, _ = _config_cache(torch, dr, ctx, stream, cfg, gen, precision=prec)

            def call(i):
                cache.attention(0, items, cfg.n_head, sliding_window=cfg.window, scale=1.0, q_norm_w=qn)
            # (a bf16 layer refuses scale 1.0 unless a kernel family is
            # forced: the one the planner picks for its shape at the usual
            # scale -- the stream kernel at head dim 256, C5's sliding and
            # global layers; the staged kernel at 512)
            if prec is None:
                ctx.set_kernel(dr.KERNEL_STREAMS if cfg.head_dim in (128, 256) else dr.KERNEL_STAGED)
            try:
                ms, _ = attention_only_ms(torch, stream, call, 4, reps)
                entry[f"{label}_kernel"] = ctx.last_launch()["kernel"]
            finally:
                ctx.set_kernel(dr.KERNEL_AUTO)
            entry[f"{label}_us_per_call"] = round(ms * 1e3, 3)
            stream.synchronize()
            del cache
        entry["hilo_over_bf16"] = round(entry["hilo_us_per_call"] / entry["bf16_us_per_call"], 3)
        res[name] = entry
        log(f"hilo {name}: {entry}")
    return res


def dropin_timing(torch, dr, CONFIGS) -> dict:
    """The literal drop-in, dr_attention() (attention.rs:106): host f32 Q/K/V
    in, host f32 out, synchronous (upload, pack K/V to bf16, attend,
    download), at C1 and C2 (C2 with all 768 keys passed as rows, the
    reference's [cached | active] assembly).  Host wall time per call."""
    import numpy as np
    res = {}
    for name in ("C1", "C2"):
        cfg = CONFIGS[name]
        h, hkv, hd = cfg.n_head, cfg.n_head_kv, cfg.head_dim
        nq, nk = cfg.n_canvas, cfg.n_total
        rng = np.random.default_rng(5)
        q = rng.standard_normal(nq * h * hd, dtype=np.float32)
        k = rng.standard_normal(nk * hkv * hd, dtype=np.float32)
        v = rng.standard_normal(nk * hkv * hd, dtype=np.float32)
        out = np.zeros(nq * h * hd, np.float32)
        s = dr.AttnShape(nq, nk, h, hkv, hd, scale=cfg.attn_scale)
        qr, kr = dr.Rows(list(range(cfg.n_prompt, nk))), dr.idpos(nk)
        for _ in range(3):
            dr.attention(out, q, k, v, s, qr, kr)
        reps = 20
        t = time.perf_counter()
        for _ in range(reps):
            dr.attention(out, q, k, v, s, qr, kr)
        us = (time.perf_counter() - t) / reps * 1e6
        fl = cfg.flops()
        res[name] = {"us_per_call": round(us, 1), "tflops": round(fl / (us / 1e6) / 1e12, 3),
                     "bytes_host_to_device": int(4 * (q.size + k.size + v.size)),
                     "bytes_device_to_host": int(4 * out.size)}
    log(f"drop-in dr_attention: {res}")
    return res


def qkv_epilogue_timing(torch, dr, ctx, stream, CONFIGS, reps: int) -> dict:
    """The Q/K/V epilogue (bias + QK-norm + RoPE, forward.rs:291-310) on the
    C4 layer's 512 canvas rows, in graph bursts.  HBM-bound: every element of
    q, k and v is read and written once (the bias, gains and table rows stay
    in L2), so GB/s = 2 * 4 * n * (h + 2 hkv) * hd / time."""
    cfg = CONFIGS["C4"]
    h, hkv, hd, n = cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.n_canvas
    gen = torch.Generator(device="cuda")
    gen.manual_seed(99)
    with torch.cuda.stream(stream):
        q = torch.randn(n, h * hd, device="cuda", generator=gen)
        k = torch.randn(n, hkv * hd, device="cuda", generator=gen)
        v = torch.randn(n, hkv * hd, device="cuda", generator=gen)
        bq = 0.1 * torch.randn(h * hd, device="cuda", generator=gen)
        bk = 0.1 * torch.randn(hkv * hd, device="cuda", generator=gen)
        bv = 0.1 * torch.randn(hkv * hd, device="cuda", generator=gen)
        qn = torch.rand(hd, device="cuda", generator=gen) + 0.5
        kn = torch.rand(hd, device="cuda", generator=gen) + 0.5
    rope = dr.Rope(ctx, cfg.n_total, hd, 10000.0)
    p_can = dr.Pass(ctx, range(cfg.n_prompt, cfg.n_total))

    def call(i):
        dr.qkv_epilogue(ctx, p_can, q, k, v, h, hkv, hd, bq, bk, bv, qn, kn, False, 1e-6, rope)
    ms, _ = attention_only_ms(torch, stream, call, 4, reps)
    nbytes = 2 * 4 * n * (h + 2 * hkv) * hd
    gbs = nbytes / (ms / 1e3) / 1e9
    # the whole C4 layer step: plain (no epilogue), the epilogue folded into
    # the store and the attention, and the separate pass followed by the step
    n_t = cfg.n_total
    with torch.cuda.stream(stream):
        Kp = torch.randn(n_t, hkv * hd, device="cuda", generator=gen)
        Vp = torch.randn(n_t, hkv * hd, device="cuda", generator=gen)
        out = torch.empty(n * h * hd, device="cuda")
    cache = dr.StepCache(ctx, n_t, [hkv], [hd])
    cache.store(0, dr.Pass(ctx, range(n_t)), Kp, Vp, k_norm_w=kn)
    sc = cfg.attn_scale
    item = [(q, out, p_can, k, v)]
    plain, _ = attention_only_ms(torch, stream, lambda i: cache.step(
        0, item, h, scale=sc, q_norm_w=qn, k_norm_w=kn), 4, reps)
    folded, _ = attention_only_ms(torch, stream, lambda i: cache.step_epi(
        0, item, h, scale=sc, bq=bq, bk=bk, bv=bv, q_norm_w=qn, k_norm_w=kn, rope=rope), 4, reps)

    def two_pass(i):
        dr.qkv_epilogue(ctx, p_can, q, k, v, h, hkv, hd, bq, bk, bv, qn, kn, False, 1e-6, rope)
        cache.step(0, item, h, scale=sc)
    both, _ = attention_only_ms(torch, stream, two_pass, 4, reps)
    res = {"workload": f"C4 layer epilogue: {n} rows, {h}+{hkv}+{hkv} heads x {hd}, "
                       "bias + QK-norm + RoPE (f32, in place)",
           "us_per_call": round(ms * 1e3, 3), "bytes": nbytes, "gbs": round(gbs, 1),
           "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
           "c4_step_us": {"no_epilogue": round(plain * 1e3, 3),
                          "epilogue_in_store_and_attention": round(folded * 1e3, 3),
                          "epilogue_pass_then_step": round(both * 1e3, 3)}}
    log(f"qkv epilogue: {res}")
    stream.synchronize()
    del cache
    rope.close()
    return res


def split_active_timing(torch, dr, ctx, stream, reps: int = 200) -> dict:
    """StepCache::split_active (cache.rs:85-114) per call, host wall time:
    on the device from device tokens (the two counts come back by one small
    copy), against the host split of host tokens plus the upload of the
    active list into a pass (what a step needs before its launches)."""
    import time
    res = {}
    for n in (768, 4352):
        rng = torch.Generator()
        rng.manual_seed(n)
        seq = torch.randint(5, 30000, (n,), generator=rng, dtype=torch.int32)
        seq[n // 3:] = 4
        prev = seq.clone()
        prev[n // 3::7] = 9  # a seventh of the canvas changed since the last step
        mask = (seq == 4).to(torch.uint8)
        cache = dr.StepCache(ctx, n, [1], [64])
        with torch.cuda.stream(stream):
            d_seq, d_mask, d_prev = seq.cuda(), mask.cuda(), prev.cuda()
        pa, pc = dr.Pass(ctx, []), dr.Pass(ctx, [])
        cache.update_seq_dev(d_prev)
        stream.synchronize()
        for _ in range(10):
            cache.split_active_dev(d_seq, d_mask, n, 5, pa, pc)
        t0 = time.perf_counter()
        for _ in range(reps):
            na, _ = cache.split_active_dev(d_seq, d_mask, n, 5, pa, pc)
        dev_us = (time.perf_counter() - t0) / reps * 1e6
        cache.update_seq(prev.numpy())
        seq_h, mask_h = seq.numpy(), mask.numpy()
        ph = dr.Pass(ctx, [])
        for _ in range(10):
            act, _ = cache.split_active(seq_h, mask_h, 5)
        t0 = time.perf_counter()
        for _ in range(reps):
            act, _ = cache.split_active(seq_h, mask_h, 5)
            ph.set(act)
        host_us = (time.perf_counter() - t0) / reps * 1e6
        res[str(n)] = {"n_active": na, "device_us": round(dev_us, 1),
                       "host_split_and_upload_us": round(host_us, 1)}
        del cache
    log(f"split_active: {res}")
    return res


def _wo_inputs(torch, stream):
    """LLaDA-8B's Wo at the C2 step: synthetic Q4_K blocks (sane f16 scales)
    for 4096 x 4096, 256 activation rows, a residual; host and device copies."""
    import numpy as np
    n, rows, cols = 256, 4096, 4096
    rng = np.random.default_rng(7)
    nb = cols // 256
    w = rng.integers(0, 256, (rows * nb, 144), dtype=np.uint8)
    w[:, 0:4] = np.float16(rng.uniform(1e-4, 0.02, (rows * nb, 2))).view(np.uint8).reshape(-1, 4)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    res = rng.standard_normal((n, rows)).astype(np.float32)
    with torch.cuda.stream(stream):
        dw = torch.from_numpy(w.reshape(-1)).cuda()
        dx = torch.from_numpy(x).cuda()
        dres = torch.from_numpy(res).cuda()
        out = torch.empty(n * rows, device="cuda")
    stream.synchronize()
    return n, rows, cols, nb, w, x, res, dw, dx, dres, out


def _wo_extra_inputs(torch, stream, rows, cols):
    """Q4_0 blocks (sane f16 scales) for the same Wo, and a post-norm gain."""
    import numpy as np
    rng = np.random.default_rng(8)
    w0 = rng.integers(0, 256, (rows * (cols // 32), 18), dtype=np.uint8)
    w0[:, 0:2] = np.float16(rng.uniform(1e-3, 0.05, rows * (cols // 32))).view(np.uint8).reshape(-1, 2)
    g = rng.uniform(0.5, 1.5, rows).astype(np.float32)
    with torch.cuda.stream(stream):
        dw0 = torch.from_numpy(w0.reshape(-1)).cuda()
        dg = torch.from_numpy(g).cuda()
    stream.synchronize()
    return dw0, dg


def qmatmul_timing(torch, dr, ctx, stream, reps: int) -> dict:
    """Wo + residual on Q4_K weights (dr_qmatmul) at LLaDA-8B's shape for the
    C2 step: 256 canvas rows x 4096 x 4096, synthetic blocks.  Ops = 2 * n *
    rows * cols (the int8 products and their sums), against MI355X's dense
    int8 MFMA peak; bytes = Q4_K weights + f32 activations in + residual in +
    out.  The CPU baseline leg times the oracle on the same call."""
    n, rows, cols, nb, w, x, res, dw, dx, dres, out = _wo_inputs(torch, stream)

    def call(i):
        dr.qmatmul(ctx, dr.WTYPE_Q4K, dw, rows, cols, dx, n, out, dres)
    ms, _ = attention_only_ms(torch, stream, call, 4, reps)
    ops = 2.0 * n * rows * cols
    nbytes = rows * nb * 144 + 4 * n * cols + 8 * n * rows
    res_d = {"workload": f"LLaDA-8B Wo + residual: {n} rows x {rows} x {cols}, Q4_K weights, Q8_K activations",
             "us_per_call": round(ms * 1e3, 3), "int_tops": round(ops / (ms / 1e3) / 1e12, 2),
             "frac_of_int8_mfma_peak": round(ops / (ms / 1e3) / 1e12 / PEAK_INT8_TOPS, 4),
             "bytes": nbytes, "gbs": round(nbytes / (ms / 1e3) / 1e9, 1)}
    # the same Wo on Q4_0 weights (MatWeight::Q40, Q8_0 activations), and the
    # Q4_K Wo with Gemma's post-attention RMSNorm before the residual add
    dw0, dg = _wo_extra_inputs(torch, stream, rows, cols)

    def call0(i):
        dr.qmatmul(ctx, dr.WTYPE_Q4_0, dw0, rows, cols, dx, n, out, dres)
    ms0, _ = attention_only_ms(torch, stream, call0, 4, reps)
    nbytes0 = rows * (cols // 32) * 18 + 4 * n * cols + 8 * n * rows
    res_d["q4_0"] = {"us_per_call": round(ms0 * 1e3, 3), "int_tops": round(ops / (ms0 / 1e3) / 1e12, 2),
                     "frac_of_int8_mfma_peak": round(ops / (ms0 / 1e3) / 1e12 / PEAK_INT8_TOPS, 4),
                     "bytes": nbytes0, "gbs": round(nbytes0 / (ms0 / 1e3) / 1e9, 1)}

    def call_pn(i):
        dr.qmatmul_post_norm(ctx, dr.WTYPE_Q4K, dw, rows, cols, dx, n, out, dg, 1e-6, dres)
    ms_pn, _ = attention_only_ms(torch, stream, call_pn, 4, reps)
    res_d["q4k_post_norm"] = {"us_per_call": round(ms_pn * 1e3, 3),
                              "timing": "Wo, then the row RMSNorm and residual add (forward.rs:346-350)"}
    del dw0, dg
    log(f"qmatmul: {res_d}")
    return res_d, (w.reshape(-1), rows, cols, x, n, res)


N_LAYERS = 32  # LLaDA-8B


def profile_only(args, torch, dr, CONFIGS) -> int:
    """--only CFG: `calls` eager attention calls of one config (for rocprofv3
    runs: kernel trace and counters of that config's launches).  --only wo:
    `calls` dr_qmatmul calls at LLaDA-8B's Wo (wo_q40: on Q4_0 weights;
    wo_pn: Q4_K with Gemma's post-attention norm).  --precision hilo: the config
    on a hi/lo-precision layer at scale 1.0 with QK-norm (Gemma's operating
    point)."""
    import dataclasses
    from helpers import EXTRA_CONFIGS
    stream = torch.cuda.Stream()
    ctx = dr.Context(0)
    ctx.set_stream(stream.cuda_stream)
    if args.calib_mib > 0:  # the copy kernel of known size that scales FETCH_SIZE / WRITE_SIZE
        n_el = args.calib_mib * (1 << 20) // 4
        with torch.cuda.stream(stream):
            src = torch.ones(n_el, dtype=torch.float32, device="cuda")
            dst = torch.empty_like(src)
            for _ in range(3):
                torch.neg(src, out=dst)
        stream.synchronize()
        del src, dst
    if args.only in ("wo", "wo_q40", "wo_pn"):
        n, rows, cols, nb, w, x, res, dw, dx, dres, out = _wo_inputs(torch, stream)
        dw0, dg = _wo_extra_inputs(torch, stream, rows, cols)
        with torch.cuda.stream(stream):
            for _ in range(args.calls):
                if args.only == "wo":
                    dr.qmatmul(ctx, dr.WTYPE_Q4K, dw, rows, cols, dx, n, out, dres)
                elif args.only == "wo_q40":
                    dr.qmatmul(ctx, dr.WTYPE_Q4_0, dw0, rows, cols, dx, n, out, dres)
                else:
                    dr.qmatmul_post_norm(ctx, dr.WTYPE_Q4K, dw, rows, cols, dx, n, out, dg, 1e-6, dres)
        stream.synchronize()
        print(json.dumps({"only": args.only, "calls": args.calls}), flush=True)
        return 0
    cfg = CONFIGS[args.only] if args.only in CONFIGS else EXTRA_CONFIGS[args.only]
    prec = None
    if args.precision == "hilo":
        cfg = dataclasses.replace(cfg, scale=1.0, qk_norm=True)
        prec = dr.PRECISION_HILO
    gen = torch.Generator(device="cuda")
    gen.manual_seed(99)
    cache, items, qn, _ = _config_cache(torch, dr, ctx, stream, cfg, gen, precision=prec)
    with torch.cuda.stream(stream):
        for _ in range(args.calls):
            cache.attention(0, items, cfg.n_head, sliding_window=cfg.window, scale=cfg.attn_scale,
                            q_norm_w=qn)
    stream.synchronize()
    print(json.dumps({"only": args.only, "calls": args.calls, "launch": ctx.last_launch()}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--mode", choices=["eager", "graph"], default="graph")
    ap.add_argument("--split", type=int, default=0, help="force key splits (0 = automatic)")
    ap.add_argument("--cpu-reps", type=int, default=0, help="oracle reps (0 = auto ~15 s)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-others", action="store_true",
                    help="skip the attention-only timing of the other configs")
    ap.add_argument("--only", default="", help="profile one config's attention and exit")
    ap.add_argument("--calls", type=int, default=64, help="calls of --only")
    ap.add_argument("--precision", choices=["bf16", "hilo"], default="bf16",
                    help="--only: the layer's precision (hilo: at scale 1.0 with QK-norm)")
    ap.add_argument("--calib-mib", type=int, default=0,
                    help="also run a plain streaming kernel (out = -in) over this many MiB, "
                         "three times: the calibration for rocprofv3 FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1"}))
        return 2

    import numpy as np
    import torch

    import dr_attn as dr
    from helpers import CONFIGS, config_seed

    torch.cuda.init()
    if args.only:
        return profile_only(args, torch, dr, CONFIGS)

    cfg = CONFIGS["C2"]
    h, hkv, hd = cfg.n_head, cfg.n_head_kv, cfg.head_dim
    n_p, n_c, n_t = cfg.n_prompt, cfg.n_canvas, cfg.n_total
    flops = cfg.flops()
    kvs = hkv * hd
    n_sets = 16

    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    ctx = dr.Context(0)
    ctx.set_stream(stream.cuda_stream)
    if args.split:
        ctx.set_split(args.split)

    rng = np.random.default_rng(config_seed(1))
    Kp = rng.standard_normal((n_p, kvs), dtype=np.float32)
    Vp = rng.standard_normal((n_p, kvs), dtype=np.float32)
    sets = []
    for s in range(n_sets):
        r = np.random.default_rng(config_seed(1, s + 1))
        sets.append((r.standard_normal((n_c, kvs), dtype=np.float32),
                     r.standard_normal((n_c, kvs), dtype=np.float32),
                     r.standard_normal((n_c, h * hd), dtype=np.float32)))
    with torch.cuda.stream(stream):
        dKp, dVp = torch.from_numpy(Kp).to(dev), torch.from_numpy(Vp).to(dev)
        dsets = [tuple(torch.from_numpy(x).to(dev) for x in st) for st in sets]
        out = torch.empty(n_c * h * hd, dtype=torch.float32, device=dev)
    cache = dr.StepCache(ctx, n_t, [hkv] * N_LAYERS, [hd] * N_LAYERS)
    p_prompt = dr.Pass(ctx, range(n_p))
    p_canvas = dr.Pass(ctx, range(n_p, n_t))
    for layer in range(N_LAYERS):
        cache.store(layer, p_prompt, dKp, dVp)
    scale = cfg.attn_scale

    # one denoise step of one layer: dr_attention_step, the store of the 256
    # canvas K/V rows and the attention of attention_block (forward.rs:312-343)
    def step(i: int) -> None:
        Kc, Vc, Q = dsets[i % n_sets]
        cache.step(i % N_LAYERS, [(Q, out, p_canvas, Kc, Vc)], h, scale=scale)

    with torch.cuda.stream(stream):
        step(0)
    stream.synchronize()
    launch = ctx.last_launch()
    log(f"launch: {launch}")

    if args.calib_mib > 0:
        n_el = args.calib_mib * (1 << 20) // 4
        with torch.cuda.stream(stream):
            src = torch.ones(n_el, dtype=torch.float32, device=dev)
            dst = torch.empty_like(src)
            for _ in range(3):
                torch.neg(src, out=dst)
        stream.synchronize()
        log(f"calibration: 3 x neg over {args.calib_mib} MiB (reads and writes that much)")
        del src, dst

    # ---- roofline: the attention call alone.  32 calls, one per layer (the
    # K/V of a real denoise step, 384 MiB, more than the Infinity Cache), are
    # captured in one graph and replayed back to back between two HIP events
    # on the library's stream; the mean launch duration is the elapsed time
    # over the number of calls.  The warm figure replays 16 calls on one
    # layer's cache (its 12 MiB stay in the Infinity Cache).
    reps = max(2, min(64, args.steps // N_LAYERS))
    attn_mean_ms, _ = attention_only_ms(
        torch, stream,
        lambda i: cache.attention(i % N_LAYERS, [(dsets[i % n_sets][2], out, p_canvas)], h, scale=scale),
        N_LAYERS, reps)
    warm_mean_ms, _ = attention_only_ms(
        torch, stream, lambda i: cache.attention(0, [(dsets[i][2], out, p_canvas)], h, scale=scale),
        n_sets, reps)
    log(f"attention call: {attn_mean_ms * 1e3:.2f} us over 32 layers, {warm_mean_ms * 1e3:.2f} us on one layer")

    # ---- the same attention call with Q rows in bf16 (dr_ctx_set_q_dtype):
    # the kernel-only figure for a caller whose projections emit bf16
    # (Q 2 bytes per element instead of 4; cache on the device either way).
    bf16_q = None
    if launch.get("kernel") == dr.KERNEL_STREAMS:
        with torch.cuda.stream(stream):
            qb = [st[2].to(torch.bfloat16) for st in dsets]
        stream.synchronize()
        ctx.set_q_dtype(dr.DTYPE_BF16)
        try:
            b_mean_ms, _ = attention_only_ms(
                torch, stream,
                lambda i: cache.attention(i % N_LAYERS, [(qb[i % n_sets], out, p_canvas)], h, scale=scale),
                N_LAYERS, reps)
            b_warm_ms, _ = attention_only_ms(
                torch, stream, lambda i: cache.attention(0, [(qb[i], out, p_canvas)], h, scale=scale),
                n_sets, reps)
            b_launch = ctx.last_launch()
        finally:
            ctx.set_q_dtype(dr.DTYPE_F32)
        bf16_q = {"launch_us_mean": round(b_mean_ms * 1e3, 3),
                  "tflops": round(flops / (b_mean_ms / 1e3) / 1e12, 2),
                  "launch_us_one_layer_warm": round(b_warm_ms * 1e3, 3),
                  "tflops_one_layer_warm": round(flops / (b_warm_ms / 1e3) / 1e12, 2),
                  "kernel": b_launch.get("kernel"),
                  "timing": "as the roofline's launch timing, Q rows bf16 (values of the f32 sets "
                            "rounded to bf16), out f32"}
        # ... and with bf16 output rows as well (dr_ctx_set_o_dtype): Q and O
        # 2 bytes per element, the boundary at which the HBM ceiling of C2
        # rises from 48.8 % to 61 % of the MFMA peak
        with torch.cuda.stream(stream):
            out_b = torch.empty(n_c * h * hd, dtype=torch.bfloat16, device=dev)
        ctx.set_q_dtype(dr.DTYPE_BF16)
        ctx.set_o_dtype(dr.DTYPE_BF16)
        try:
            o_mean_ms, _ = attention_only_ms(
                torch, stream,
                lambda i: cache.attention(i % N_LAYERS, [(qb[i % n_sets], out_b, p_canvas)], h, scale=scale),
                N_LAYERS, reps)
            o_warm_ms, _ = attention_only_ms(
                torch, stream, lambda i: cache.attention(0, [(qb[i], out_b, p_canvas)], h, scale=scale),
                n_sets, reps)
            o_launch = ctx.last_launch()
        finally:
            ctx.set_q_dtype(dr.DTYPE_F32)
            ctx.set_o_dtype(dr.DTYPE_F32)
        bf16_q["bf16_q_and_out"] = {
            "launch_us_mean": round(o_mean_ms * 1e3, 3),
            "tflops": round(flops / (o_mean_ms / 1e3) / 1e12, 2),
            "pct_of_peak": round(100 * flops / (o_mean_ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 3),
            "launch_us_one_layer_warm": round(o_warm_ms * 1e3, 3),
            "tflops_one_layer_warm": round(flops / (o_warm_ms / 1e3) / 1e12, 2),
            "kernel": o_launch.get("kernel"),
            "algorithmic_bytes_per_launch": 2 * n_c * h * hd * 2 + 2 * n_t * kvs * 2,
            "timing": "as above, Q and output rows bf16 (dr_ctx_set_o_dtype)"}
        del qb, out_b
        log(f"attention call, bf16 Q (and bf16 Q + out): {bf16_q}")

    # ---- timed region: K whole steps, every one a graph replay (a graph of
    # 32 steps, one per layer, and a graph of the remainder)
    graphs = {}
    mode = args.mode

    def capture(n: int):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
            for i in range(n):
                step(i)
        stream.synchronize()
        return g

    if mode == "graph":
        try:
            with torch.cuda.stream(stream):
                for i in range(3):
                    step(i)
            stream.synchronize()
            graphs["full"] = capture(N_LAYERS)
            for n in {args.steps % N_LAYERS, args.warmup % N_LAYERS} - {0}:
                graphs[n] = capture(n)
        except Exception as e:  # graph capture unavailable: measure eagerly
            log(f"graph capture failed ({e}); timing eagerly")
            graphs = {}
            mode = "eager"

    def run(n: int) -> None:
        with torch.cuda.stream(stream):
            if graphs:
                for _ in range(n // N_LAYERS):
                    graphs["full"].replay()
                if n % N_LAYERS:
                    graphs[n % N_LAYERS].replay()
            else:
                for i in range(n):
                    step(i)

    run(args.warmup)
    with torch.cuda.stream(stream):
        for g in graphs.values():  # (a graph's first replay is slower than the next ones)
            g.replay()
    torch.cuda.synchronize()
    stream.synchronize()
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    run(args.steps)
    e1.record(stream)
    torch.cuda.synchronize()  # (covers the stream: a second wait only added its own latency)
    wall = time.perf_counter() - t0
    gpu_ms = e0.elapsed_time(e1)
    total_s = max(wall, gpu_ms / 1e3)
    ms_per_step = total_s * 1e3 / args.steps
    value = flops * args.steps / total_s / 1e12

    # ---- step-inclusive with the host upload: the canvas K, V and Q rows
    # (f32, 12 MiB) copied from pinned host memory on the library's stream,
    # then store + attention; eager, events around `h2d_steps` steps
    h2d = None
    if not args.no_others:
        h2d_steps = 20
        pins = [tuple(torch.from_numpy(x).pin_memory() for x in st) for st in sets[:2]]
        with torch.cuda.stream(stream):
            dst = tuple(torch.empty_like(x) for x in dsets[0])

        def h2d_step(i: int) -> None:
            for d, hsrc in zip(dst, pins[i % 2]):
                d.copy_(hsrc, non_blocking=True)
            cache.step(i % N_LAYERS, [(dst[2], out, p_canvas, dst[0], dst[1])], h, scale=scale)

        with torch.cuda.stream(stream):
            for i in range(3):
                h2d_step(i)
            h0, h1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            h0.record(stream)
            for i in range(h2d_steps):
                h2d_step(i)
            h1.record(stream)
        stream.synchronize()
        h2d_ms = h0.elapsed_time(h1) / h2d_steps
        up = sum(x.numel() * 4 for x in dsets[0])
        h2d = {"us_per_step": round(h2d_ms * 1e3, 2), "tflops": round(flops / (h2d_ms / 1e3) / 1e12, 3),
               "bytes_host_to_device": up, "h2d_gbs": round(up / (h2d_ms / 1e3) / 1e9, 1),
               "timing": f"eager, HIP events around {h2d_steps} steps: pinned-host copies of the canvas "
                         "K, V, Q rows (f32) on the library's stream, then store + attention"}
        log(f"step with host upload: {h2d}")
        del pins, dst

    # ---- a C2 step whose active rows are a scattered split_active set
    # (StepCache::split_active, cache.rs:85-114): mid-denoise, about half of
    # the canvas still masked at random positions and a seventh of the rest
    # changed since the previous step.  Those rows are the step's queries and
    # the rows it stores (at scattered positions: the position-list store
    # kernel), attending over all 768 keys of the 32-layer cache.
    scattered = None
    if not args.no_others:
        rs = np.random.default_rng(config_seed(1, 99))
        seq = rs.integers(5, 30000, n_t).astype(np.int32)
        masked = np.zeros(n_t, np.uint8)
        masked[n_p:] = rs.random(n_c) < 0.5
        seq[masked.astype(bool)] = 4
        prev = seq.copy()
        changed = (masked == 0) & (np.arange(n_t) >= n_p) & (rs.random(n_t) < 1 / 7)
        prev[changed] = 9
        act, _ = dr.split_active(prev, np.zeros(n_t, np.int32), seq, masked, 5)
        n_a = len(act)
        runs = 1 + sum(1 for x, y in zip(act, act[1:]) if y != x + 1)
        p_act = dr.Pass(ctx, act)
        with torch.cuda.stream(stream):
            kq, kk, kv = dsets[0][2][:n_a].contiguous(), dsets[0][0][:n_a].contiguous(), dsets[0][1][:n_a].contiguous()
            oa = torch.empty(n_a * h * hd, dtype=torch.float32, device=dev)
        stream.synchronize()
        reps_s = max(2, min(64, args.steps // N_LAYERS))
        s_ms, _ = attention_only_ms(
            torch, stream, lambda i: cache.step(i % N_LAYERS, [(kq, oa, p_act, kk, kv)], h, scale=scale),
            N_LAYERS, reps_s)
        fl_s = 4.0 * h * hd * n_a * n_t
        scattered = {"n_active": n_a, "contiguous_runs": runs, "us_per_step": round(s_ms * 1e3, 3),
                     "tflops": round(fl_s / (s_ms / 1e3) / 1e12, 2),
                     "timing": "HIP events around graph replays of 32 steps, one per layer: the store of the "
                               "active rows (position list) and their attention over 768 keys"}
        log(f"step with scattered active rows: {scattered}")
        del kq, kk, kv, oa

    achieved = flops / (attn_mean_ms / 1e3) / 1e12
    traffic, traffic_src = measured_traffic("C2")
    algo_bytes = (n_c * h * hd * 4) * 2 + 2 * n_t * kvs * 2  # Q f32 + O f32 + K,V bf16
    kernel_name = ("attn_ring_kernel" if launch.get("kernel") == dr.KERNEL_STREAMS else "attn_fwd_kernel")
    roofline = {
        "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
        "traffic_source": traffic_src,
        "kernel": f"{kernel_name} (one launch per attention call)",
        "flops_per_launch": flops, "launch_us_mean": round(attn_mean_ms * 1e3, 3),
        "launch_timing": "HIP events around graph replays of 32 back-to-back calls, one per layer "
                         "(K/V from HBM)",
        "achieved_one_layer_warm": round(flops / (warm_mean_ms / 1e3) / 1e12, 2),
        "launch_us_one_layer_warm": round(warm_mean_ms * 1e3, 3),
        "algorithmic_bytes_per_launch": algo_bytes,
        "hbm_ceiling_frac": round(min(1.0, flops / algo_bytes * PEAK_HBM_GBS * 1e9 / 1e12
                                      / PEAK_BF16_TFLOPS), 4),
    }

    others = epi = split = qmm = qmm_inputs = dropin = hilo = None
    if not args.no_others:
        r2 = max(4, min(64, args.steps // 32))
        others = other_configs(torch, dr, ctx, stream, CONFIGS, r2)
        epi = qkv_epilogue_timing(torch, dr, ctx, stream, CONFIGS, r2)
        split = split_active_timing(torch, dr, ctx, stream)
        qmm, qmm_inputs = qmatmul_timing(torch, dr, ctx, stream, r2)
        dropin = dropin_timing(torch, dr, CONFIGS)
        hilo = hilo_timing(torch, dr, ctx, stream, CONFIGS, r2)

    # ---- CPU baseline: the C restatement of the reference's attention on this
    # host's cores, on step 0's inputs (layer 0); its output also checks the
    # GPU result of that step.
    cpu, parity = None, None
    if not args.no_cpu:
        import oracle as orc
        from helpers import RowsSpec, Shape
        with torch.cuda.stream(stream):
            step(0)
        stream.synchronize()
        got = out.cpu().numpy()
        Kc, Vc, Q = sets[0]
        s = Shape(n_c, n_t, h, hkv, hd, scale=scale)
        qr, kr = RowsSpec(list(range(n_p, n_t))), RowsSpec(list(range(n_t)))
        qf = Q.reshape(-1).copy()
        kf = np.concatenate([Kp, Kc]).reshape(-1).copy()
        vf = np.concatenate([Vp, Vc]).reshape(-1).copy()
        threads = orc.max_threads()
        out_c = np.zeros(n_c * h * hd, np.float32)
        t = time.perf_counter()
        orc.attention(out_c, qf, kf, vf, s, qr, kr, threads=threads)
        one = time.perf_counter() - t
        err = np.abs(got.astype(np.float64) - out_c)
        parity = {"max_abs": float(err.max()), "mean_abs": float(err.mean()),
                  "ok": bool(err.max() <= 1e-2 and err.mean() <= 1e-3)}
        log(f"parity of step 0 vs the CPU reference: {parity}")
        reps = args.cpu_reps or max(1, min(200, int(15.0 / max(one, 1e-3))))
        t = time.perf_counter()
        for _ in range(reps):
            orc.attention(out_c, qf, kf, vf, s, qr, kr, threads=threads)
        per = (time.perf_counter() - t) / reps
        t = time.perf_counter()
        orc.attention(out_c, qf, kf, vf, s, qr, kr, threads=1)
        per1 = time.perf_counter() - t
        if qmm is not None:
            # the same Wo call through the oracle's native_matmul + residual_add
            t = time.perf_counter()
            orc.qmatmul(orc.WTYPE_Q4K, *qmm_inputs)
            qmm["cpu_oracle_ms"] = round((time.perf_counter() - t) * 1e3, 1)
            qmm["cpu_oracle_threads"] = threads
        cpu = {"value": round(flops / per / 1e12, 5), "unit": "TFLOP/s", "cores": threads,
               "kind": "port",
               "sample": f"{reps} C2 attention calls (256 q x 768 k x 32 heads, hd 128, f32) "
                         f"with the C restatement of attention()+attention_row_avx2 on "
                         f"{threads} OpenMP threads; {per * 1e3:.1f} ms/call",
               "ms_per_call": round(per * 1e3, 3),
               "value_1thread": round(flops / per1 / 1e12, 5),
               "ms_per_call_1thread": round(per1 * 1e3, 2)}
        log(f"cpu baseline: {cpu}")

    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "C2: LLaDA-8B denoise step, 32/32 heads, hd 128, 512 cached + "
                               "256 canvas, batch 1 (dr_attention_step: store canvas K/V + "
                               "attention; step i on layer i mod 32 of a 32-layer cache)",
                   "global_batch": 1, "seq_len": n_t, "parallelism": "none (1 GPU)",
                   "timing": mode, "accumulate": "fp32", "q_out_dtype": "f32",
                   "kv_cache_dtype": "bf16", "layers": N_LAYERS},
        "pct_of_peak": round(100 * value / PEAK_BF16_TFLOPS, 3),
        "attention_call_pct_of_peak": round(100 * achieved / PEAK_BF16_TFLOPS, 3),
        "gpu_event_ms": round(gpu_ms, 4), "wall_s": round(wall, 4),
        "launch": launch, "parity": parity, "roofline": roofline, "cpu_baseline": cpu,
        "attention_bf16_q": bf16_q,
        "step_with_host_upload": h2d,
        "other_configs_attention_only": others,
        "dropin_dr_attention": dropin,
        "qkv_epilogue": epi,
        "split_active": split,
        "scattered_step": scattered,
        "wo_qmatmul": qmm,
        "precision_hilo": hilo,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

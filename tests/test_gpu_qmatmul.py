"""The projection after the attention on GGUF k-quant weights (dr_qmatmul:
Wo, src/model/forward.rs:345-350): activations quantized to Q8_K
(src/kernels.rs:79-122), Q4_K / Q6_K x Q8_K block dots (src/kernels.rs:228-347)
on the int8 matrix cores, and residual_add (ops.rs:365-370), against the
oracle's or_qmatmul (pinned by tests/test_oracle.py against a float64
dequantize-and-dot).

Bar: the quantization is bit-exact (dr_quantize_q8k against the oracle's
quantize_rows_q8_k); every integer of a block dot is exact; the f32 combine
of the per-block integers with d and dmin rounds in another order than the
reference's scalar dot, so each output must lie within
2 (nb + 12) 2^-24 (T + |residual|) of the oracle's, T = sum_i (|d sc q_i| +
|dmin mn|) |d_x qs_i| (helpers.kquant_bound).  The bound is checked to be
tight enough to see one block of 256 values.  Needs an MI355X.
"""
from __future__ import annotations

import numpy as np
import pytest

import dr_attn as dr
import oracle as orc
from helpers import kquant_acts, kquant_bound, kquant_weights

from test_gpu_parity import dev, say, torch  # noqa: F401

pytestmark = pytest.mark.gpu


def _check(got, want, tol, what):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ratio = float(np.max(np.divide(err, tol, out=np.zeros_like(err), where=tol > 0)))
    bad = int(np.count_nonzero(err > tol))
    assert np.max(np.abs(want)) > 0  # not a vacuous comparison
    say(f"  {what}: max |err| / bound {ratio:.3e} ({bad} outside); "
        f"max |err| {float(np.max(err)):.3e}, max |want| {float(np.max(np.abs(want))):.3e}")
    assert bad == 0


def _run(dev, wtype, w, rows, cols, x, n, res=None):
    out = dev.put(res.reshape(-1)) if res is not None else dev.empty(n * rows)
    dr.qmatmul(dev.ctx, wtype, dev.put(w), rows, cols, dev.put(x), n, out,
               out if res is not None else None)
    return dev.get(out).reshape(n, rows)


@pytest.mark.parametrize("wtype", [orc.WTYPE_Q4K, orc.WTYPE_Q6K])
@pytest.mark.parametrize("rows,cols,n", [(192, 512, 37), (100, 1024, 5), (64, 256, 1), (257, 768, 70),
                                         (33, 1792, 130)])
def test_qmatmul_vs_oracle(dev, wtype, rows, cols, n):
    rng = np.random.default_rng(rows * 7 + cols + n + wtype)
    w = kquant_weights(rng, wtype, rows, cols)
    x = kquant_acts(rng, n, cols)
    res = rng.standard_normal((n, rows)).astype(np.float32)
    say(f"qmatmul wtype {wtype} rows {rows} cols {cols} n {n}")
    want = orc.qmatmul(wtype, w, rows, cols, x, n).reshape(n, rows)
    tol = kquant_bound(orc, wtype, w, rows, cols, x, n)
    _check(_run(dev, wtype, w, rows, cols, x, n), want, tol, "no residual")
    # the residual add in place (residual == out, as attention_block's b.cur)
    want_r = orc.qmatmul(wtype, w, rows, cols, x, n, res).reshape(n, rows)
    tol_r = kquant_bound(orc, wtype, w, rows, cols, x, n, res)
    _check(_run(dev, wtype, w, rows, cols, x, n, res), want_r, tol_r, "residual in place")
    # negative control: the bound sees a missing last block
    w_drop = w.reshape(rows, cols // 256, -1).copy()
    dpos = 0 if wtype == orc.WTYPE_Q4K else 208
    w_drop[:, -1, dpos:dpos + (4 if wtype == orc.WTYPE_Q4K else 2)] = 0  # d (and dmin) = 0
    want_drop = orc.qmatmul(wtype, w_drop.reshape(-1), rows, cols, x, n).reshape(n, rows)
    assert np.any(np.abs(want_drop - want) > tol)


def test_quantize_q8k_bit_exact(dev):
    """dr_quantize_q8k against quantize_rows_q8_k: d, all 256 qs and the 16
    bsums of every block, with an all-zero block, ties of the largest
    magnitude, a NaN, values that round half away from zero, and the +127 cap
    (a positive extreme of -128 / -max scale)."""
    rng = np.random.default_rng(81)
    n, cols = 9, 1024
    x = kquant_acts(rng, n, cols)
    x[3, 40] = np.nan
    x[4, :256] = np.linspace(-2.0, 2.0, 256, dtype=np.float32)  # symmetric: +max hits the cap
    x[5, 256:512] = (np.arange(256, dtype=np.float32) - 127.5) / 127.5 * 3.0
    x[6, 512:768] = np.float32(0.5) * (np.arange(256) % 5 - 2)  # exact halves after scaling
    want = orc.quantize_q8k(x, n, cols)
    nbk = n * cols // 256
    t = dev.t
    with t.cuda.stream(dev.stream):
        buf = t.zeros(nbk * orc.Q8K_DTYPE.itemsize, dtype=t.uint8, device="cuda")
    dr.quantize_q8k(dev.ctx, dev.put(x), n, cols, buf)
    got = np.frombuffer(dev.get(buf).tobytes(), orc.Q8K_DTYPE)
    assert np.array_equal(got["qs"], want["qs"])
    assert np.array_equal(got["bsums"], want["bsums"])
    assert np.array_equal(got["d"].view(np.uint32), want["d"].view(np.uint32))
    assert np.any(want["qs"] == 127) and np.any(want["qs"] == -128)


def test_qmatmul_llada8b_wo_vs_oracle(dev):
    """LLaDA-8B's Wo at the C2 step: 256 canvas rows, 4096 x 4096, Q4_K, with
    the residual add in place."""
    rng = np.random.default_rng(4096)
    rows = cols = 4096
    n = 256
    w = kquant_weights(rng, orc.WTYPE_Q4K, rows, cols)
    x = kquant_acts(rng, n, cols)
    res = rng.standard_normal((n, rows)).astype(np.float32)
    want = orc.qmatmul(orc.WTYPE_Q4K, w, rows, cols, x, n, res).reshape(n, rows)
    tol = kquant_bound(orc, orc.WTYPE_Q4K, w, rows, cols, x, n, res)
    say("LLaDA-8B Wo 256 x 4096 x 4096 Q4_K")
    _check(_run(dev, orc.WTYPE_Q4K, w, rows, cols, x, n, res), want, tol, "LLaDA-8B Wo")


def test_qmatmul_repeat_calls_bit_identical(dev):
    """Each output's partial sums meet in a fixed order: repeated calls (and a
    call after a different shape on the same workspace) give the same bits."""
    rng = np.random.default_rng(5)
    rows, cols, n = 300, 2048, 200
    w = dev.put(kquant_weights(rng, orc.WTYPE_Q4K, rows, cols))
    x = dev.put(kquant_acts(rng, n, cols))
    outs = []
    for i in range(3):
        if i == 2:  # a smaller call in between
            dr.qmatmul(dev.ctx, orc.WTYPE_Q4K, w, 50, 1024, x, 7, dev.empty(7 * 50))
        out = dev.empty(n * rows)
        dr.qmatmul(dev.ctx, orc.WTYPE_Q4K, w, rows, cols, x, n, out)
        outs.append(dev.get(out))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


@pytest.mark.parametrize("wtype", [orc.WTYPE_Q4K, orc.WTYPE_Q6K])
def test_qmatmul_expert_slice(dev, wtype):
    """ExpertMat::forward_expert (matmul.rs:176-213): expert e's matmul is
    native_matmul on bytes [e * size, (e + 1) * size) of the
    [n_expert][rows][cols] stack; each expert matches the oracle on its own
    slice (and differs from its neighbours'); expert >= n_expert is an error."""
    rng = np.random.default_rng(31 + wtype)
    n_expert, rows, cols, n = 3, 96, 768, 24
    stack = kquant_weights(rng, wtype, n_expert * rows, cols)
    x = kquant_acts(rng, n, cols)
    per = stack.size // n_expert
    dw, dx = dev.put(stack), dev.put(x)
    prev = None
    for e in range(n_expert):
        sl = stack[e * per:(e + 1) * per]
        want = orc.qmatmul(wtype, sl, rows, cols, x, n).reshape(n, rows)
        tol = kquant_bound(orc, wtype, sl, rows, cols, x, n)
        out = dev.empty(n * rows)
        dr.qmatmul_expert(dev.ctx, wtype, dw, n_expert, e, rows, cols, dx, n, out)
        got = dev.get(out).reshape(n, rows)
        _check(got, want, tol, f"expert {e}")
        if prev is not None:
            assert np.any(np.abs(got - prev) > tol)
        prev = got
    with pytest.raises(dr.DrError) as ei:
        dr.qmatmul_expert(dev.ctx, wtype, dw, n_expert, n_expert, rows, cols, dx, n, dev.empty(n * rows))
    assert ei.value.status == dr.DR_ERR_INVALID


def test_qmatmul_rejects_bad_shapes(dev):
    w = np.zeros(144, np.uint8)
    x = np.zeros(256, np.float32)
    out = dev.empty(1)
    with pytest.raises(dr.DrError):
        dr.qmatmul(dev.ctx, 13, dev.put(w), 1, 256, dev.put(x), 1, out)  # Q5_K: not built
    with pytest.raises(dr.DrError):
        dr.qmatmul(dev.ctx, orc.WTYPE_Q4K, dev.put(w), 1, 200, dev.put(x), 1, out)  # cols % 256
    w2 = dev.put(np.zeros(160, np.uint8))
    with pytest.raises(dr.DrError):  # Q4_K blocks off a 16-byte boundary
        dr.qmatmul(dev.ctx, orc.WTYPE_Q4K, w2.data_ptr() + 4, 1, 256, dev.put(x), 1, out)

"""Wo on the legacy 32-value GGUF block types (dr_qmatmul with Q4_0 / Q5_0 /
Q8_0 weights: MatWeight::Q40 and ExpertMat::{Q40, Q50, Q80},
src/model/matmul.rs:103-106, 156-158, 192-194), the Q8_0 activation
quantization they run on (ActScratch::q80, matmul.rs:73-82), and Gemma's
post-attention RMSNorm before the residual add (forward.rs:346-350,
dr_qmatmul_post_norm), against the oracle (pinned by tests/test_oracle.py:
the reference's Q8_0 dequantization vector, closed forms of the block
layouts, numpy's f16 rounding and a float64 dequantize-and-dot with negative
controls).

Bar: the quantization is bit-exact (dr_quantize_q8_0 against the oracle's
quantize_row_q8_0); every block's integer dot is exact and only the f32
combine with the block scales rounds in another order, so each output lies
within helpers.legacy_bound of the oracle's; the post-norm outputs within a
relative 1e-5 of the oracle's (its f64 sum of squares runs in another
order).  Needs an MI355X.
"""
from __future__ import annotations

import numpy as np
import pytest

import dr_attn as dr
import oracle as orc
from helpers import kquant_acts, kquant_bound, kquant_weights, legacy_bound, legacy_weights

from test_gpu_parity import dev, say, torch  # noqa: F401
from test_gpu_qmatmul import _check, _run

pytestmark = pytest.mark.gpu

LEGACY = [orc.WTYPE_Q4_0, orc.WTYPE_Q5_0, orc.WTYPE_Q8_0]


@pytest.mark.parametrize("wtype", LEGACY)
@pytest.mark.parametrize("rows,cols,n", [(192, 512, 37), (100, 96, 5), (64, 32, 1), (257, 800, 70),
                                         (33, 1792, 130)])
def test_qmatmul_legacy_vs_oracle(dev, wtype, rows, cols, n):
    rng = np.random.default_rng(rows * 11 + cols + n + wtype)
    w = legacy_weights(rng, wtype, rows, cols)
    x = kquant_acts(rng, n, cols) if cols >= 256 else rng.standard_normal((n, cols)).astype(np.float32)
    res = rng.standard_normal((n, rows)).astype(np.float32)
    say(f"qmatmul wtype {wtype} rows {rows} cols {cols} n {n}")
    want = orc.qmatmul(wtype, w, rows, cols, x, n).reshape(n, rows)
    _check(_run(dev, wtype, w, rows, cols, x, n), want, legacy_bound(orc, wtype, w, rows, cols, x, n),
           "no residual")
    want_r = orc.qmatmul(wtype, w, rows, cols, x, n, res).reshape(n, rows)
    tol_r = legacy_bound(orc, wtype, w, rows, cols, x, n, res)
    _check(_run(dev, wtype, w, rows, cols, x, n, res), want_r, tol_r, "residual in place")
    # negative control: the bound sees a missing last block (its d = 0)
    w_drop = w.reshape(rows, cols // 32, -1).copy()
    w_drop[:, -1, 0:2] = 0
    want_drop = orc.qmatmul(wtype, w_drop.reshape(-1), rows, cols, x, n).reshape(n, rows)
    assert np.any(np.abs(want_drop - want) > tol_r)


def test_quantize_q8_0_bit_exact(dev):
    """dr_quantize_q8_0 against quantize_row_q8_0: the f16 d and all 32 qs of
    every block, with an all-zero block, a NaN, exact halves after scaling
    (round half away from zero) and a negative extreme."""
    rng = np.random.default_rng(83)
    n, cols = 7, 320
    x = (rng.standard_normal((n, cols)) * rng.uniform(0.01, 20, (n, cols))).astype(np.float32)
    x[1, 32:64] = 0.0
    x[2, 5] = np.nan
    x[3, :32] = np.float32(127.0) * (np.arange(32) - 16) / np.float32(16.0)  # exact q = k * 127/16
    x[4, 64:96] = np.float32(2.0) * ((np.arange(32) % 5) - 2) + np.float32(0.5)
    x[5, 100] = -1e4
    want = orc.quantize_q8_0(x, n, cols)
    t = dev.t
    with t.cuda.stream(dev.stream):
        buf = t.zeros(want.size * orc.Q80_DTYPE.itemsize, dtype=t.uint8, device="cuda")
    dr.quantize_q8_0(dev.ctx, dev.put(x), n, cols, buf)
    got = np.frombuffer(dev.get(buf).tobytes(), orc.Q80_DTYPE)
    assert np.array_equal(got["d"], want["d"])
    assert np.array_equal(got["qs"], want["qs"])
    assert np.any(want["qs"] == 127) and np.any(want["qs"] == -127)


def test_qmatmul_llada8b_wo_q4_0_vs_oracle(dev):
    """LLaDA-8B's Wo at the C2 step on Q4_0 weights (MatWeight::Q40): 256
    canvas rows, 4096 x 4096, residual in place."""
    rng = np.random.default_rng(4097)
    rows = cols = 4096
    n = 256
    w = legacy_weights(rng, orc.WTYPE_Q4_0, rows, cols)
    x = kquant_acts(rng, n, cols)
    res = rng.standard_normal((n, rows)).astype(np.float32)
    want = orc.qmatmul(orc.WTYPE_Q4_0, w, rows, cols, x, n, res).reshape(n, rows)
    tol = legacy_bound(orc, orc.WTYPE_Q4_0, w, rows, cols, x, n, res)
    _check(_run(dev, orc.WTYPE_Q4_0, w, rows, cols, x, n, res), want, tol, "LLaDA-8B Wo Q4_0")


@pytest.mark.parametrize("wtype", LEGACY)
def test_qmatmul_legacy_expert_slice(dev, wtype):
    """ExpertMat::forward_expert on the legacy types (matmul.rs:192-194,
    201-213): each expert's slice of the stack against the oracle on that
    slice, neighbours differing; expert >= n_expert is an error."""
    rng = np.random.default_rng(41 + wtype)
    n_expert, rows, cols, n = 3, 96, 384, 24
    stack = legacy_weights(rng, wtype, n_expert * rows, cols)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    per = stack.size // n_expert
    dw, dx = dev.put(stack), dev.put(x)
    prev = None
    for e in range(n_expert):
        sl = stack[e * per:(e + 1) * per]
        want = orc.qmatmul(wtype, sl, rows, cols, x, n).reshape(n, rows)
        tol = legacy_bound(orc, wtype, sl, rows, cols, x, n)
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


@pytest.mark.parametrize("wtype", [orc.WTYPE_Q4K, orc.WTYPE_Q4_0])
@pytest.mark.parametrize("rows,shift", [(768, 0), (4100, 0), (770, 0), (768, 1)])
def test_qmatmul_post_norm_vs_oracle(dev, wtype, rows, shift):
    """Gemma's step after the attention (forward.rs:345-350): Wo, the
    post-attention RMSNorm of each output row (norm_rows_inplace), then the
    residual; against the oracle's qmatmul followed by its post-norm, with
    and without a residual.  A norm over the wrong axis (per column) or
    without the gain is caught by the bar.  Rows of 768 and 4100 values take
    the norm's 16-byte path (4100: a second pass over the row and a partial
    last piece); 770 values, and an output / residual buffer that starts one
    float past a 16-byte boundary (shift 1), take its per-value path."""
    rng = np.random.default_rng(51 + wtype + rows)
    cols, n, eps = 512, 40, 1e-6
    if wtype == orc.WTYPE_Q4K:
        w = kquant_weights(rng, wtype, rows, cols)
    else:
        w = legacy_weights(rng, wtype, rows, cols)
    x = kquant_acts(rng, n, cols)
    g = rng.uniform(0.5, 1.5, rows).astype(np.float32)
    res = rng.standard_normal((n, rows)).astype(np.float32)
    mm = orc.qmatmul(wtype, w, rows, cols, x, n).reshape(n, rows)
    bound = (kquant_bound if wtype == orc.WTYPE_Q4K else legacy_bound)(orc, wtype, w, rows, cols, x, n)
    rms = np.sqrt((mm.astype(np.float64) ** 2).mean(1, keepdims=True) + eps)
    for residual in (res, None):
        want = mm.copy()
        orc.post_norm_residual(want, g, residual, n, rows, eps)
        say(f"post-norm wtype {wtype} rows {rows} shift {shift} residual {residual is not None}")
        if residual is not None:
            buf = dev.put(np.concatenate([np.zeros(shift, np.float32), residual.reshape(-1)]))
        else:
            buf = dev.empty(n * rows + shift)
        out = buf[shift:]
        dr.qmatmul_post_norm(dev.ctx, wtype, dev.put(w), rows, cols, dev.put(x), n, out, dev.put(g), eps,
                             out if residual is not None else None)
        got = dev.get(out).reshape(n, rows)
        err = np.abs(got.astype(np.float64) - want)
        # the matmul's own bound carried through the norm (x g / rms), plus a
        # few ulp of the norm's scale, of the products and of the residual add
        tol = bound / rms * g + 1e-6 * (np.abs(want) + (np.abs(residual) if residual is not None else 0)) + 1e-7
        say(f"  post-norm wtype {wtype} residual {residual is not None}: max err / bound "
            f"{float(np.max(err / tol)):.2e}, max err {float(np.max(err)):.2e}")
        assert np.all(err <= tol)
        wrong_axis = mm / np.sqrt((mm.astype(np.float64) ** 2).mean(0, keepdims=True) + eps) * g
        assert np.max(np.abs(got - wrong_axis - (residual if residual is not None else 0))) > 1e-2
        no_gain = mm / np.sqrt((mm.astype(np.float64) ** 2).mean(1, keepdims=True) + eps)
        assert np.max(np.abs(got - no_gain - (residual if residual is not None else 0))) > 1e-2


def test_qmatmul_legacy_rejects_bad_shapes(dev):
    x = dev.put(np.zeros(64, np.float32))
    out = dev.empty(2)
    w = dev.put(np.zeros(64, np.uint8))
    with pytest.raises(dr.DrError) as ei:
        dr.qmatmul(dev.ctx, orc.WTYPE_Q4_0, w, 1, 48, x, 1, out)  # cols % 32
    assert ei.value.status == dr.DR_ERR_INVALID
    with pytest.raises(dr.DrError) as ei:
        dr.qmatmul(dev.ctx, 3, w, 1, 32, x, 1, out)  # Q4_1: not a type the reference runs natively
    assert ei.value.status == dr.DR_ERR_UNSUPPORTED
    with pytest.raises(dr.DrError) as ei:
        dr.qmatmul(dev.ctx, orc.WTYPE_Q8_0, w.data_ptr() + 1, 1, 32, x, 1, out)  # odd address
    assert ei.value.status == dr.DR_ERR_INVALID

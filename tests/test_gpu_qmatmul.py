"""The projection after the attention on GGUF k-quant weights (dr_qmatmul:
Wo, src/model/forward.rs:345-350): activations quantized to Q8_K
(src/kernels.rs:79-122), Q4_K / Q6_K x Q8_K block dots (the reference's
scalar vec_dot, src/kernels.rs:228-347) and residual_add (ops.rs:365-370),
against the oracle's or_qmatmul, which tests/test_oracle.py pins.  Each
output runs the same integer and f32 operations in the same order, so the
bar is bit-exact.  Needs an MI355X.
"""
from __future__ import annotations

import numpy as np
import pytest

import dr_attn as dr
import oracle as orc

from test_gpu_parity import dev, say, torch  # noqa: F401

pytestmark = pytest.mark.gpu


def _weights(rng, wtype: int, rows: int, cols: int) -> np.ndarray:
    """Random GGUF blocks with sane f16 scales (the quant bytes are arbitrary)."""
    nb = cols // 256
    bb = orc.Q4K_BYTES if wtype == orc.WTYPE_Q4K else orc.Q6K_BYTES
    w = rng.integers(0, 256, (rows * nb, bb), dtype=np.uint8)
    dpos = 0 if wtype == orc.WTYPE_Q4K else 208
    w[:, dpos:dpos + 2] = np.float16(rng.uniform(1e-4, 0.02, rows * nb)).view(np.uint8).reshape(-1, 2)
    if wtype == orc.WTYPE_Q4K:
        w[:, 2:4] = np.float16(rng.uniform(1e-4, 0.02, rows * nb)).view(np.uint8).reshape(-1, 2)
    return w.reshape(-1)


def _acts(rng, n: int, cols: int) -> np.ndarray:
    x = rng.standard_normal((n, cols)).astype(np.float32)
    x[0, :256] = 0.0  # an all-zero block: d = 0
    if n > 2:
        x[2, 300] = -40.0  # a negative extreme
        x[1, 7] = x[1, 9] = 9.0  # tied largest magnitudes: the first one counts
        x[1, 8] = -9.0
    return x


@pytest.mark.parametrize("wtype", [orc.WTYPE_Q4K, orc.WTYPE_Q6K])
@pytest.mark.parametrize("rows,cols,n", [(192, 512, 37), (100, 1024, 5), (64, 256, 1), (257, 768, 70)])
def test_qmatmul_bit_exact_vs_oracle(dev, wtype, rows, cols, n):
    rng = np.random.default_rng(rows * 7 + cols + n + wtype)
    w = _weights(rng, wtype, rows, cols)
    x = _acts(rng, n, cols)
    res = rng.standard_normal((n, rows)).astype(np.float32)
    want = orc.qmatmul(wtype, w, rows, cols, x, n)
    want_r = orc.qmatmul(wtype, w, rows, cols, x, n, res)
    dw, dx = dev.put(w), dev.put(x)
    out = dev.empty(n * rows)
    say(f"qmatmul wtype {wtype} rows {rows} cols {cols} n {n}")
    dr.qmatmul(dev.ctx, wtype, dw, rows, cols, dx, n, out)
    got = dev.get(out)
    bad = np.count_nonzero(got != want)
    say(f"  {bad} of {got.size} differ; max rel {np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)):.3e}")
    assert bad == 0
    # with the residual add, in place (residual == out, as attention_block's b.cur)
    io = dev.put(res.reshape(-1))
    dr.qmatmul(dev.ctx, wtype, dw, rows, cols, dx, n, io, io)
    assert np.array_equal(dev.get(io), want_r)


def test_qmatmul_llada8b_wo_vs_oracle(dev):
    """LLaDA-8B's Wo at the C2 step: 256 canvas rows, 4096 x 4096, Q4_K."""
    rng = np.random.default_rng(4096)
    rows = cols = 4096
    n = 256
    w = _weights(rng, orc.WTYPE_Q4K, rows, cols)
    x = _acts(rng, n, cols)
    res = rng.standard_normal((n, rows)).astype(np.float32)
    want = orc.qmatmul(orc.WTYPE_Q4K, w, rows, cols, x, n, res)
    io = dev.put(res.reshape(-1))
    dr.qmatmul(dev.ctx, orc.WTYPE_Q4K, dev.put(w), rows, cols, dev.put(x), n, io, io)
    got = dev.get(io)
    bad = np.count_nonzero(got != want)
    say(f"LLaDA-8B Wo: {bad} of {got.size} differ")
    assert bad == 0


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

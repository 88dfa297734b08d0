"""Pins the CPU oracle (oracle/attn_oracle.c) before it is trusted as the
parity checker.  CPU only.

What pins what:
  * the reference's own attention tests, same inputs and tolerances
    (src/model/tests.rs:70-237): known answer, GQA == repeated MHA,
    block-diagonal == separate runs, online == naive, AVX2 == scalar;
  * a float64 three-pass brute force (tests/helpers.py) and the committed
    golden fixtures it produced (tests/golden/);
  * torch.nn.functional.scaled_dot_product_attention on the CPU (a library
    routine, independent of both);
  * invariants: key-permutation invariance, thread-count determinism;
  * the StepCache tests (tests.rs:39-68) and closed forms for RMSNorm;
  * negative controls: a plausible mistake (dropped window, wrong prefix,
    wrong GQA mapping, wrong scale) must fail the same checks.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle as orc
from helpers import (RowsSpec, Shape, brute_force, closed_form, golden_cases, materialise,
                     rms_norm_f64)


def run(s, qr, kr, q, k, v, **kw):
    out = np.zeros(s.nq * s.n_head * s.head_dim, dtype=np.float32)
    orc.attention(out, q, k, v, s, qr, kr, **kw)
    return out.reshape(s.nq, s.n_head * s.head_dim)


def idrows(n):
    return RowsSpec(pos=list(range(n)))


# ---------------------------------------------------------------- visible()

def test_visible_known_cases():
    # attention.rs:17-24, 29-35: different sequences never see each other.
    assert not orc.visible(3, 3, 0, 1)
    # symmetric band, strict: |q - k| < w
    assert orc.visible(10, 14, 0, 0, window=5)
    assert orc.visible(14, 10, 0, 0, window=5)
    assert not orc.visible(10, 15, 0, 0, window=5)
    assert not orc.visible(15, 10, 0, 0, window=5)
    # window 0 hides everything (|d| >= 0)
    assert not orc.visible(4, 4, 0, 0, window=0)
    # prompt rows (qpos < prefix) are causal; canvas rows see all
    assert orc.visible(5, 5, 0, 0, prefix=8)
    assert not orc.visible(5, 6, 0, 0, prefix=8)
    assert orc.visible(5, 0, 0, 0, prefix=8)
    assert orc.visible(8, 20, 0, 0, prefix=8)
    assert orc.visible(9, 2, 0, 0, prefix=8)


def test_visible_matches_visibility_matrix():
    s = Shape(nq=9, nk=12, n_head=1, n_head_kv=1, head_dim=1, sliding_window=4, causal_prefix=6)
    qr = RowsSpec(pos=[0, 2, 5, 6, 7, 11, 3, 8, 1], seq=[0, 0, 0, 0, 1, 1, 0, 1, 0])
    kr = RowsSpec(pos=list(range(12)), seq=[0] * 6 + [1] * 6)
    from helpers import visibility
    m = visibility(s, qr, kr)
    for i in range(s.nq):
        for j in range(s.nk):
            assert bool(m[i, j]) == orc.visible(qr.pos[i], kr.pos[j], qr.seq[i], kr.seq[j], 4, 6)


# --------------------------------------------- the reference's own tests

@pytest.mark.parametrize("avx2", [False, True])
def test_uniform_scores_known_answer(avx2):
    # tests.rs:104-114
    s = Shape(nq=1, nk=2, n_head=1, n_head_kv=1, head_dim=2)
    q = np.array([1.0, 0.0], np.float32)
    k = np.array([1.0, 0.0, 1.0, 0.0], np.float32)
    v = np.array([0.0, 2.0, 4.0, 6.0], np.float32)
    out = run(s, idrows(1), idrows(2), q, k, v, avx2=avx2).reshape(-1)
    assert abs(out[0] - 2.0) < 1e-6 and abs(out[1] - 4.0) < 1e-6


@pytest.mark.parametrize("avx2", [False, True])
def test_matches_naive_reference(avx2):
    # tests.rs:154-186 -- online softmax == three-pass softmax, 1e-5
    s = Shape(nq=4, nk=6, n_head=2, n_head_kv=2, head_dim=8)
    q = closed_form(4 * 2 * 8, 37, 101, 50, 25)
    k = closed_form(6 * 2 * 8, 53, 97, 48, 24)
    v = closed_form(6 * 2 * 8, 71, 89, 44, 44)
    out = run(s, idrows(4), idrows(6), q, k, v, avx2=avx2)
    want = brute_force(q, k, v, s, idrows(4), idrows(6))
    assert np.max(np.abs(out - want)) < 1e-5


@pytest.mark.parametrize("avx2", [False, True])
def test_gqa_matches_repeated_kv(avx2):
    # tests.rs:116-152
    nq, nk, hd = 3, 5, 8
    gqa = Shape(nq=nq, nk=nk, n_head=4, n_head_kv=2, head_dim=hd)
    mha = Shape(nq=nq, nk=nk, n_head=4, n_head_kv=4, head_dim=hd)
    q = closed_form(nq * 4 * hd, 37, 101, 50, 50)
    k = closed_form(nk * 2 * hd, 53, 97, 48, 48)
    v = closed_form(nk * 2 * hd, 71, 89, 44, 44)

    def repeat(x):
        return np.repeat(x.reshape(nk, 2, hd), 2, axis=1).reshape(-1).copy()

    a = run(gqa, idrows(nq), idrows(nk), q, k, v, avx2=avx2)
    b = run(mha, idrows(nq), idrows(nk), q, repeat(k), repeat(v), avx2=avx2)
    assert np.max(np.abs(a - b)) < 1e-5


@pytest.mark.parametrize("avx2", [False, True])
def test_block_diagonal_batches(avx2):
    # tests.rs:70-102
    hd, na, nb = 4, 2, 3
    s = lambda n: Shape(nq=n, nk=n, n_head=1, n_head_kv=1, head_dim=hd)  # noqa: E731
    q = closed_form((na + nb) * hd, 37, 101, 50, 50)
    k = q.copy()
    v = closed_form((na + nb) * hd, 71, 89, 44, 44)
    br = RowsSpec(pos=[0, 1, 0, 1, 2], seq=[0, 0, 1, 1, 1])
    batched = run(s(na + nb), br, br, q, k, v, avx2=avx2).reshape(-1)
    sep_a = run(s(na), idrows(na), idrows(na), q[: na * hd].copy(), k[: na * hd].copy(),
                v[: na * hd].copy(), avx2=avx2).reshape(-1)
    sep_b = run(s(nb), idrows(nb), idrows(nb), q[na * hd:].copy(), k[na * hd:].copy(),
                v[na * hd:].copy(), avx2=avx2).reshape(-1)
    assert np.max(np.abs(batched[: na * hd] - sep_a)) < 1e-5
    assert np.max(np.abs(batched[na * hd:] - sep_b)) < 1e-5


def test_avx2_matches_scalar():
    # tests.rs:188-213, row by row
    s = Shape(nq=3, nk=3, n_head=2, n_head_kv=2, head_dim=16)
    n = 3 * 2 * 16
    q, k, v = closed_form(n, 37, 101, 50, 50), closed_form(n, 53, 97, 48, 48), closed_form(n, 71, 89, 44, 44)
    a = np.zeros(n, np.float32)
    b = np.zeros(n, np.float32)
    for head in range(2):
        for i in range(3):
            orc.attention_row("scalar", a, q, k, v, s, idrows(3), idrows(3), head, i)
            orc.attention_row("avx2", b, q, k, v, s, idrows(3), idrows(3), head, i)
    assert np.max(np.abs(a - b)) < 1e-5


# ------------------------------------------------- golden fixtures

@pytest.mark.parametrize("avx2", [False, True])
@pytest.mark.parametrize("case,want", golden_cases(), ids=[c["name"] for c, _ in golden_cases()])
def test_golden(case, want, avx2):
    s, qr, kr, q, k, v = materialise(case)
    got = run(s, qr, kr, q, k, v, avx2=avx2)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    tol = 1e-5 * max(1.0, float(np.max(np.abs(want[ok])))) if ok.any() else 0
    assert np.max(np.abs(got[ok] - want[ok]), initial=0.0) <= tol


# ------------------------------------------------- independent cross-checks

def test_torch_sdpa_crosscheck():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    h, hkv, hd, nq, nk = 8, 2, 128, 16, 96
    s = Shape(nq=nq, nk=nk, n_head=h, n_head_kv=hkv, head_dim=hd, scale=1 / math.sqrt(hd))
    q = rng.standard_normal(nq * h * hd).astype(np.float32)
    k = rng.standard_normal(nk * hkv * hd).astype(np.float32)
    v = rng.standard_normal(nk * hkv * hd).astype(np.float32)
    got = run(s, RowsSpec(pos=list(range(nk - nq, nk))), idrows(nk), q, k, v)
    Q = torch.from_numpy(q.astype(np.float64)).view(nq, h, hd).transpose(0, 1)
    K = torch.from_numpy(k.astype(np.float64)).view(nk, hkv, hd).transpose(0, 1)
    V = torch.from_numpy(v.astype(np.float64)).view(nk, hkv, hd).transpose(0, 1)
    K = K.repeat_interleave(h // hkv, dim=0)
    V = V.repeat_interleave(h // hkv, dim=0)
    ref = torch.nn.functional.scaled_dot_product_attention(Q, K, V, scale=s.scale)
    ref = ref.transpose(0, 1).reshape(nq, h * hd).numpy()
    assert np.max(np.abs(got - ref)) < 1e-5


def test_key_permutation_invariance():
    # Masking is by position, so the [cached | active] key order of the cache
    # (forward.rs:91-101) must not change the result beyond rounding.
    rng = np.random.default_rng(3)
    h, hkv, hd, nq, nk = 4, 2, 64, 6, 50
    s = Shape(nq=nq, nk=nk, n_head=h, n_head_kv=hkv, head_dim=hd, sliding_window=9,
              causal_prefix=20, scale=0.125)
    q = rng.standard_normal(nq * h * hd).astype(np.float32)
    k = rng.standard_normal((nk, hkv * hd)).astype(np.float32)
    v = rng.standard_normal((nk, hkv * hd)).astype(np.float32)
    qr = RowsSpec(pos=[3, 15, 19, 20, 33, 49])
    a = run(s, qr, idrows(nk), q, k.reshape(-1), v.reshape(-1))
    perm = rng.permutation(nk)
    b = run(s, qr, RowsSpec(pos=[int(p) for p in perm]), q, k[perm].reshape(-1).copy(),
            v[perm].reshape(-1).copy())
    assert np.max(np.abs(a - b)) < 1e-5


def test_threads_bit_identical():
    # each (head, query) task is sequential: the pool size cannot change bits
    rng = np.random.default_rng(5)
    h, hd, nq, nk = 8, 128, 32, 64
    s = Shape(nq=nq, nk=nk, n_head=h, n_head_kv=h, head_dim=hd, scale=0.1)
    q = rng.standard_normal(nq * h * hd).astype(np.float32)
    k = rng.standard_normal(nk * h * hd).astype(np.float32)
    v = rng.standard_normal(nk * h * hd).astype(np.float32)
    a = run(s, idrows(nq), idrows(nk), q, k, v, threads=1)
    b = run(s, idrows(nq), idrows(nk), q, k, v, threads=0)
    assert np.array_equal(a, b)


# ------------------------------------------------- negative controls

def _dense_case():
    rng = np.random.default_rng(11)
    h, hkv, hd, nq, nk = 4, 2, 32, 5, 40
    q = rng.standard_normal(nq * h * hd).astype(np.float32)
    k = rng.standard_normal(nk * hkv * hd).astype(np.float32)
    v = rng.standard_normal(nk * hkv * hd).astype(np.float32)
    return h, hkv, hd, nq, nk, q, k, v


def test_checks_catch_plausible_mistakes():
    h, hkv, hd, nq, nk, q, k, v = _dense_case()
    qr = RowsSpec(pos=[2, 10, 21, 30, 39])
    good = Shape(nq=nq, nk=nk, n_head=h, n_head_kv=hkv, head_dim=hd, sliding_window=6,
                 causal_prefix=15, scale=0.2)
    want = brute_force(q, k, v, good, qr, idrows(nk))
    assert np.max(np.abs(run(good, qr, idrows(nk), q, k, v) - want)) < 1e-5
    mistakes = [
        Shape(**{**good.__dict__, "sliding_window": None}),   # dropped window
        Shape(**{**good.__dict__, "sliding_window": 7}),      # off-by-one band
        Shape(**{**good.__dict__, "causal_prefix": None}),    # dropped prefix
        Shape(**{**good.__dict__, "causal_prefix": 3}),       # wrong prefix
        Shape(**{**good.__dict__, "scale": 0.1}),             # wrong scale
    ]
    for bad in mistakes:
        assert np.max(np.abs(run(bad, qr, idrows(nk), q, k, v) - want)) > 1e-3, bad
    # wrong GQA mapping (head % n_head_kv instead of head / group): swapping
    # the two KV heads' data changes the answer
    ks = k.reshape(nk, hkv, hd)[:, ::-1].reshape(-1).copy()
    vs = v.reshape(nk, hkv, hd)[:, ::-1].reshape(-1).copy()
    assert np.max(np.abs(run(good, qr, idrows(nk), q, ks, vs) - want)) > 1e-3


# ------------------------------------------------- QK-norm

def test_rms_norm_closed_forms():
    w = np.linspace(0.5, 1.5, 128).astype(np.float32)
    # all-equal vector c: rms = |c| -> x = sign(c) * w / sqrt(1 + eps/c^2)
    for c in (3.0, -0.25):
        x = np.full(128, c, np.float32)
        orc.rms_norm_inplace(x, w, 1e-6)
        want = np.sign(c) * w / math.sqrt(1 + 1e-6 / c**2)
        assert np.max(np.abs(x - want)) < 1e-6
    # positive rescaling invariance (eps -> 0)
    rng = np.random.default_rng(0)
    x = rng.standard_normal(128).astype(np.float32)
    y = (x * 37.0).astype(np.float32)
    orc.rms_norm_inplace(x, w, 0.0)
    orc.rms_norm_inplace(y, w, 0.0)
    assert np.max(np.abs(x - y)) < 1e-5


def test_norm_heads_matches_f64():
    rng = np.random.default_rng(1)
    hd, n = 128, 12
    x = rng.standard_normal(n * hd).astype(np.float32)
    w = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    want = rms_norm_f64(x.reshape(n, hd), w, 1e-6).reshape(-1)
    orc.norm_heads(x, w, 1e-6)
    assert np.max(np.abs(x - want)) < 1e-5


# ------------------------------------------------- QKV epilogue: bias, V-norm, RoPE

def test_rms_norm_noscale_closed_forms():
    # ops.rs:116-124: all-equal c -> sign(c) / sqrt(1 + eps/c^2); unit RMS and
    # a positive multiple of the input for random rows
    for c in (2.5, -0.125):
        x = np.full(256, c, np.float32)
        orc.rms_norm_noscale(x, 1e-6)
        assert np.max(np.abs(x - np.sign(c) / math.sqrt(1 + 1e-6 / c**2))) < 1e-6
    rng = np.random.default_rng(5)
    x0 = rng.standard_normal(256).astype(np.float32) * 3.0
    x = x0.copy()
    orc.rms_norm_noscale(x, 0.0)
    assert abs(math.sqrt(np.mean(x.astype(np.float64) ** 2)) - 1.0) < 1e-6
    ratio = x / x0
    assert np.all(ratio > 0) and np.ptp(ratio) < 1e-6


def test_add_bias_is_rowwise_addition():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((7, 96)).astype(np.float32)
    b = rng.standard_normal(96).astype(np.float32)
    want = x + b
    y = x.reshape(-1).copy()
    orc.add_bias(y, b, 7)
    assert np.array_equal(y.reshape(7, 96), want)


def test_rope_table_matches_f64_trig():
    # ops.rs:396-417: freq_i = theta^(-2i/d) (/ ff_i), angle t*freq_i.  The
    # f32 angle carries a relative rounding error of ~2^-23 per operation,
    # so the bound grows with the angle.
    d, theta, T = 128, 10000.0, 4096
    tab = orc.rope_table(T, d, theta)
    i = np.arange(d // 2, dtype=np.float64)
    freq = theta ** (-2.0 * i / d)
    t = np.arange(T, dtype=np.float64)[:, None]
    ang = t * freq[None, :]
    tol = 4 * 2.0**-23 * (ang + 1.0) + 1e-7
    assert np.all(np.abs(tab[:, :, 0] - np.sin(ang)) <= tol)
    assert np.all(np.abs(tab[:, :, 1] - np.cos(ang)) <= tol)
    # freq factors divide the frequency: the angle at 2t with factor 2 is the
    # plain angle at t
    ff = np.full(d // 2, 2.0, np.float32)
    tab2 = orc.rope_table(T, d, theta, ff)
    assert np.max(np.abs(tab2[0:T:2] - tab[: T // 2])) < 1e-3
    assert np.array_equal(tab[0, :, 0], np.zeros(d // 2, np.float32))
    assert np.array_equal(tab[0, :, 1], np.ones(d // 2, np.float32))


def test_rotate_rows_pairs_signs_and_invariants():
    d, rot, heads = 128, 128, 3
    tab = orc.rope_table(512, rot, 10000.0)
    half = rot // 2
    # unit vectors: e_i -> cos at i, sin at i+half; e_{half+i} -> -sin at i,
    # cos at i+half (the pairing (i, i+half) and the rotation's sign)
    for i in (0, 5, half - 1):
        for pos in (1, 77, 300):
            x = np.zeros(d, np.float32)
            x[i] = 1.0
            orc.rotate_rows(x, tab, [pos], 1, d, rot)
            sn, cs = tab[pos, i]
            nz = np.flatnonzero(x)
            assert set(nz.tolist()) <= {i, half + i}
            assert x[i] == cs and x[half + i] == sn
            y = np.zeros(d, np.float32)
            y[half + i] = 1.0
            orc.rotate_rows(y, tab, [pos], 1, d, rot)
            assert y[i] == -sn and y[half + i] == cs
    rng = np.random.default_rng(7)
    x0 = rng.standard_normal((4, heads, d)).astype(np.float32)
    pos = [0, 3, 200, 511]
    x = x0.reshape(-1).copy()
    orc.rotate_rows(x, tab, pos, heads, d, rot)
    x = x.reshape(4, heads, d)
    assert np.array_equal(x[0], x0[0])  # position 0 is the identity
    n0 = x0[..., :half] ** 2 + x0[..., half:] ** 2
    n1 = x[..., :half] ** 2 + x[..., half:] ** 2
    assert np.max(np.abs(n1 - n0) / (n0 + 1e-3)) < 1e-5  # pair norms kept
    # relative position: <R(q, m), R(k, n)> depends only on m - n
    q0 = rng.standard_normal(d).astype(np.float32)
    k0 = rng.standard_normal(d).astype(np.float32)

    def dot_at(m, n):
        q = q0.copy()
        k = k0.copy()
        orc.rotate_rows(q, tab, [m], 1, d, rot)
        orc.rotate_rows(k, tab, [n], 1, d, rot)
        return float(np.dot(q.astype(np.float64), k.astype(np.float64)))
    for m, n, s in ((10, 3, 40), (50, 60, 7), (5, 5, 100)):
        assert abs(dot_at(m, n) - dot_at(m + s, n + s)) < 2e-3 * math.sqrt(d)
    assert abs(dot_at(10, 3) - dot_at(10, 4)) > 1e-2  # and it does depend on m - n


def test_rotate_rows_partial_rotary():
    d, rot = 128, 64
    tab = orc.rope_table(64, rot, 500.0)
    rng = np.random.default_rng(8)
    x0 = rng.standard_normal((2, 2, d)).astype(np.float32)
    x = x0.reshape(-1).copy()
    orc.rotate_rows(x, tab, [9, 33], 2, d, rot)
    x = x.reshape(2, 2, d)
    assert np.array_equal(x[..., rot:], x0[..., rot:])  # the rest untouched
    assert np.max(np.abs(x[..., :rot] - x0[..., :rot])) > 1e-2
    # a rotation by the table's angle in each (i, i + rot/2) plane
    a, b = x0[1, 1, :rot // 2], x0[1, 1, rot // 2:rot]
    sn, cs = tab[33, :, 0], tab[33, :, 1]
    assert np.max(np.abs(x[1, 1, :rot // 2] - (a * cs - b * sn))) < 1e-6
    assert np.max(np.abs(x[1, 1, rot // 2:rot] - (a * sn + b * cs))) < 1e-6


# ------------------------------------------------- StepCache

def test_cache_store_gather_roundtrip():
    # tests.rs:55-68
    stride = 4
    ck = np.zeros(3 * stride, np.float32)
    cv = np.zeros(3 * stride, np.float32)
    k = np.arange(8, dtype=np.float32)
    v = np.arange(100, 108, dtype=np.float32)
    orc.cache_store(ck, cv, stride, [2, 0], k, v)
    ok = np.zeros(8, np.float32)
    ov = np.zeros(8, np.float32)
    orc.cache_gather(ck, cv, stride, [0, 2], ok, ov)
    assert ok.tolist() == [4, 5, 6, 7, 0, 1, 2, 3]
    assert ov.tolist() == [104, 105, 106, 107, 100, 101, 102, 103]


def test_split_active_reference_case():
    # tests.rs:39-53
    prev = np.array([10, 20, -1, -1], np.int32)
    last = np.full(4, -1, np.int32)
    act, cac = orc.split_active(prev, last, [10, 21, -1, -1], [0, 0, 1, 1], 5)
    assert act == [1, 2, 3] and cac == [0]
    prev = np.array([10, 21, -1, -1], np.int32)
    act, cac = orc.split_active(prev, last, [10, 21, -1, -1], [0, 0, 1, 1], 5 + 2 + 1)
    assert act == [2, 3] and cac == [0, 1]


def test_split_active_vicinity_and_decay():
    n = 12
    prev = np.full(n, 7, np.int32)
    last = np.full(n, -1, np.int32)
    masked = np.zeros(n, np.uint8)
    masked[6] = 1
    act, cac = orc.split_active(prev, last, prev, masked, 3, vicinity=2)
    assert act == [4, 5, 6, 7, 8]
    assert cac == [0, 1, 2, 3, 9, 10, 11]
    # position 1 changes at step 3 and stays active through step 5 (<= 2 later)
    seq = prev.copy()
    seq[1] = 9
    act, _ = orc.split_active(prev, last, seq, np.zeros(n, np.uint8), 3)
    assert act == [1]
    for step, expect in ((4, [1]), (5, [1]), (6, [])):
        act, _ = orc.split_active(seq, last, seq, np.zeros(n, np.uint8), step)
        assert act == expect, step


def test_bf16_round_known_values():
    """The test-side bf16 rounding used to build the kernel's operand view:
    ties go to even, and values already in bf16 are fixed points."""
    from helpers import bf16_round
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -2.5, 0.0],
                 np.float32)
    want = np.array([1.0, 1.0, 1.0 + 2 ** -6, 1.0 + 2 ** -7, -2.5, 0.0], np.float32)
    assert np.array_equal(bf16_round(x), want)
    r = bf16_round(np.random.default_rng(0).standard_normal(1000).astype(np.float32))
    assert np.array_equal(bf16_round(r), r)
    assert np.all(r.view(np.uint32) & 0xFFFF == 0)


# ---- quantized matmul pieces (src/kernels.rs, src/model/matmul.rs) ----------

def test_f16_to_f32_reference_vectors():
    # kernels.rs:350-372 (test_f16_to_f32): numpy float16 reference values
    cases = [(0x0000, 0.0), (0x0001, 5.9604645e-8), (0x0200, 3.0517578e-5), (0x03FF, 6.097555e-5),
             (0x0400, 6.1035156e-5), (0x3C00, 1.0), (0xC000, -2.0), (0x8001, -5.9604645e-8)]
    for h, want in cases:
        got = orc.f16_to_f32(h)
        assert abs(got - want) <= abs(want) * 1e-6, (hex(h), got, want)
        # and numpy's own decode of every one of them
        assert got == float(np.array([h], np.uint16).view(np.float16)[0])
    assert math.isinf(orc.f16_to_f32(0x7C00)) and math.isnan(orc.f16_to_f32(0x7C01))
    allh = np.arange(0, 0x7C00, 97, dtype=np.uint16)
    assert all(orc.f16_to_f32(int(h)) == float(np.float16(allh.view(np.float16)[i]))
               for i, h in enumerate(allh))


def test_q8k_quantize_invariants():
    rng = np.random.default_rng(81)
    x = (rng.standard_normal(4 * 512) * rng.uniform(0.01, 50, 4 * 512)).astype(np.float32)
    x[256:512] = 0.0  # an all-zero block
    x[777] = -3.0 * np.abs(x[768:1024]).max()  # its block's largest magnitude, negative
    q = orc.quantize_q8k(x, 4, 512)
    assert orc.Q8K_DTYPE.itemsize == 292  # kernels.rs:374-379
    xb = x.reshape(-1, 256)
    for b in range(q.size):
        d, qs = float(q["d"][b]), q["qs"][b].astype(np.int32)
        if not np.any(xb[b]):
            assert d == 0.0 and not np.any(qs)
            continue
        i = int(np.argmax(np.abs(xb[b])))  # first index of the largest magnitude
        assert qs[i] == -128
        assert np.all(np.abs(xb[b] - d * qs) <= abs(d) * 0.5 * (1 + 1e-5) + 1e-30)
        assert np.array_equal(q["bsums"][b], qs.reshape(16, 16).sum(1).astype(np.int16))
    assert q["d"][3] > 0  # a negative extreme gives a positive d (iscale = -128 / max)


def _q4k_ref_block():
    # kernels.rs:425-437 (test_q4k_nonzero)
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(0x3800).tobytes(), np.uint8)
    b[4:16] = [(i * 5 + 1) & 0x3F for i in range(12)]
    b[16:] = [(i * 7 + 3) & 0xFF for i in range(128)]
    return b


def _q6k_ref_block():
    # kernels.rs:398-423 (test_q6k_vs_dequantize)
    b = np.zeros(210, np.uint8)
    b[:128] = [(i * 7 + 3) & 0xFF for i in range(128)]
    b[128:192] = [(i * 13 + 5) & 0xFF for i in range(64)]
    b[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    return b


def _ref_q8():
    q = np.zeros(1, orc.Q8K_DTYPE)
    q["d"] = np.float32(1.0 / 127.0)
    qs = np.clip(np.arange(256) * 3 - 128, -128, 127).astype(np.int8)
    q["qs"][0] = qs
    q["bsums"][0] = qs.astype(np.int16).reshape(16, 16).sum(1)
    return q


@pytest.mark.parametrize("wtype", [orc.WTYPE_Q4K, orc.WTYPE_Q6K])
def test_quantized_dot_equals_dequantized_dot(wtype):
    """The reference's own cross-check (kernels.rs:398-437): the integer dot
    equals dequantize-then-dot, on its block patterns and on random blocks."""
    nbytes = orc.Q4K_BYTES if wtype == orc.WTYPE_Q4K else orc.Q6K_BYTES
    blocks = [_q4k_ref_block() if wtype == orc.WTYPE_Q4K else _q6k_ref_block()]
    ys = [_ref_q8()]
    rng = np.random.default_rng(82 + wtype)
    for _ in range(6):
        b = rng.integers(0, 256, nbytes, dtype=np.uint8)
        dpos = 0 if wtype == orc.WTYPE_Q4K else 208
        b[dpos:dpos + 2] = np.frombuffer(np.float16(rng.uniform(0.001, 0.05)).tobytes(), np.uint8)
        if wtype == orc.WTYPE_Q4K:
            b[2:4] = np.frombuffer(np.float16(rng.uniform(0.001, 0.05)).tobytes(), np.uint8)
        blocks.append(b)
        ys.append(orc.quantize_q8k(rng.standard_normal(256).astype(np.float32), 1, 256))
    for b, y in zip(blocks, ys):
        got = orc.vec_dot(wtype, b, y, 1)
        w = orc.dequant(wtype, b, 1).astype(np.float64)
        want = float(np.dot(w, y["qs"][0].astype(np.float64)) * float(y["d"][0]))
        assert np.isfinite(got) and abs(got) > 1e-6
        assert abs(got - want) <= 1e-4 * max(abs(want), 1e-3), (got, want)


def test_q4k_scales_and_mins_closed_form():
    """Q4_K with every nibble q, d = 1, dmin = 1 and per-sub-block scale s_j and
    min m_j dequantizes to s_j * q - m_j; sub-block j's scale lands on it (a
    transposed unpack of the 12 packed bytes would not)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    sc = [1, 2, 3, 4, 5, 6, 7, 63]
    mn = [0, 1, 2, 3, 10, 20, 30, 40]
    pk = np.zeros(12, np.uint8)  # get_scale_min_k4 packing
    for j in range(4):
        pk[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        pk[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        pk[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    b[4:16] = pk
    b[16:] = 0x53  # low nibble 3, high nibble 5
    w = orc.dequant(orc.WTYPE_Q4K, b, 1)
    for j in range(8):
        q = 3 if j % 2 == 0 else 5
        assert np.all(w[32 * j:32 * j + 32] == np.float32(sc[j] * q - mn[j])), j


@pytest.mark.parametrize("wtype", [orc.WTYPE_Q4K, orc.WTYPE_Q6K])
def test_qmatmul_composition_vs_f64_dequant(wtype):
    """or_qmatmul (native_matmul, matmul.rs:120-148, over Q8_K activations,
    matmul.rs:64-71) against an independent float64 composition: out[t, r] =
    sum_i dequant(W)[r, i] * d_t,b * qs_t,i + residual, with three blocks per
    row and rows != n, within the stated f32 bound.  Negative controls: the
    same composition with the output transposed (out[r * n + t]), with two
    weight rows swapped, with two activation rows swapped, or without the
    last block, each breaks the bound."""
    from helpers import kquant_acts, kquant_acts_f64, kquant_bound, kquant_dequant_f64, kquant_weights
    rng = np.random.default_rng(7 + wtype)
    rows, cols, n = 7, 768, 4
    w = kquant_weights(rng, wtype, rows, cols)
    x = kquant_acts(rng, n, cols)
    res = rng.standard_normal((n, rows)).astype(np.float32)
    got = orc.qmatmul(wtype, w, rows, cols, x, n, res).reshape(n, rows).astype(np.float64)
    W = kquant_dequant_f64(orc, wtype, w, rows, cols)
    X = kquant_acts_f64(orc, x, n, cols)
    want = X @ W.T + res
    # dequant's own f32 rounding (d * sc * q - dmin * mn: 3 roundings) on top
    tol = kquant_bound(orc, wtype, w, rows, cols, x, n, res) + \
        3 * 2.0 ** -24 * (np.abs(X) @ kquant_dequant_f64(orc, wtype, w, rows, cols, True).T)
    err = np.abs(got - want)
    assert np.all(err <= tol), float(np.max(err / tol))
    assert np.max(np.abs(want)) > 1.0  # not a vacuous comparison
    bad_t = (X @ W.T + res).reshape(-1)[np.arange(n * rows).reshape(rows, n).T.reshape(-1)].reshape(n, rows)
    W_sw = W[[1, 0] + list(range(2, rows))]
    X_sw = X[[1, 0] + list(range(2, n))]
    X_drop = X.copy()
    X_drop[:, 512:] = 0.0
    for name, wrong in (("transposed", bad_t), ("weight rows swapped", X @ W_sw.T + res),
                        ("activation rows swapped", X_sw @ W.T + res), ("last block dropped", X_drop @ W.T + res)):
        assert np.any(np.abs(got - wrong) > tol), name


def test_q6k_values_bijective_and_scale_per_16():
    """Q6_K (dequantize_q6k_row, kernels.rs:129-163): every one of the 256
    6-bit fields (a 4-bit ql nibble + a 2-bit qh pair) feeds exactly one value,
    and sub-block j (values 16 j .. 16 j + 15) takes scale j: with all fields
    zero each value is d * sc_j * -32; raising one field's low bit moves
    exactly one value by d * sc_j."""
    b = np.zeros(210, np.uint8)
    sc = np.arange(1, 17, dtype=np.int8)
    b[192:208] = sc.view(np.uint8)
    b[208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    base = orc.dequant(orc.WTYPE_Q6K, b, 1)
    assert np.array_equal(base, np.repeat(sc.astype(np.float32) * -32.0, 16))
    hit = np.zeros(256, int)
    for byte in range(128):  # ql: two nibbles per byte
        for shift in (0, 4):
            bb = b.copy()
            bb[byte] = 1 << shift
            d = orc.dequant(orc.WTYPE_Q6K, bb, 1) - base
            (idx,) = np.nonzero(d)
            assert len(idx) == 1 and d[idx[0]] == sc[idx[0] // 16], (byte, shift)
            hit[idx[0]] += 1
    for byte in range(128, 192):  # qh: four 2-bit pairs per byte; +16 per pair
        for pair in range(4):
            bb = b.copy()
            bb[byte] = 1 << (2 * pair)
            d = orc.dequant(orc.WTYPE_Q6K, bb, 1) - base
            (idx,) = np.nonzero(d)
            assert len(idx) == 1 and d[idx[0]] == 16 * int(sc[idx[0] // 16]), (byte, pair)
    assert np.all(hit == 1)


# ---- the legacy 32-value block types and Q8_0 activations

def test_dequantize_q8_0_reference_vector():
    """kernels.rs:382-395 (test_dequantize_q8_0_row): two blocks, d = 0.5
    (0x3800), quants blk * 32 + i - 40: value i is 0.5 * (i - 40)."""
    b = bytearray()
    for blk in range(2):
        b += (0x3800).to_bytes(2, "little")
        b += bytes(((blk * 32 + i - 40) & 0xFF) for i in range(32))
    out = orc.dequant(orc.WTYPE_Q8_0, np.frombuffer(bytes(b), np.uint8), 2)
    assert np.array_equal(out, (0.5 * (np.arange(64) - 40)).astype(np.float32))


def test_q4_0_nibble_order_closed_form():
    """dequantize_q4_0_row (kernels.rs:165-173): byte i's low nibble is value
    i, its high nibble value i + 16, each minus 8, times d (a swapped nibble
    order or a missing -8 fails)."""
    b = np.zeros(18, np.uint8)
    b[0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    lo, hi = np.arange(16) % 16, (np.arange(16) * 7 + 3) % 16
    b[2:] = (hi << 4) | lo
    out = orc.dequant(orc.WTYPE_Q4_0, b, 1)
    want = np.concatenate([lo - 8, hi - 8]).astype(np.float32) * np.float32(0.25)
    assert np.array_equal(out, want)


def test_q5_0_fields_bijective():
    """Q5_0 (ggml's layout: f16 d, 32 high bits, 16 nibble bytes): with every
    field zero each value is -16 d; raising a nibble's low bit moves exactly
    one value by d, raising one of the 32 high bits exactly one value by 16 d,
    and value j takes high bit j (nibbles as Q4_0's)."""
    b = np.zeros(22, np.uint8)
    b[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    base = orc.dequant(orc.WTYPE_Q5_0, b, 1)
    assert np.array_equal(base, np.full(32, -16.0, np.float32))
    hit = np.zeros(32, int)
    for byte in range(16):
        for shift in (0, 4):
            bb = b.copy()
            bb[6 + byte] = 1 << shift
            (idx,) = np.nonzero(orc.dequant(orc.WTYPE_Q5_0, bb, 1) - base)
            assert list(idx) == [byte + (16 if shift else 0)]
            hit[idx[0]] += 1
    for bit in range(32):
        bb = b.copy()
        bb[2 + bit // 8] = 1 << (bit % 8)
        d = orc.dequant(orc.WTYPE_Q5_0, bb, 1) - base
        (idx,) = np.nonzero(d)
        assert list(idx) == [bit] and d[bit] == 16.0
    assert np.all(hit == 1)


def test_f32_to_f16_is_round_to_nearest_even():
    """The oracle's f16 rounding of the Q8_0 scale against numpy's (IEEE round
    to nearest even), over normals, subnormals, exact ties and overflow."""
    rng = np.random.default_rng(90)
    xs = np.concatenate([rng.uniform(-1, 1, 2000) * 10.0 ** rng.integers(-9, 5, 2000),
                         np.array([0.0, -0.0, 6.1e-5, 5.96e-8, 2.98e-8, 65504.0, 65519.0, 65520.0, 1e-30])])
    # exact ties of f16 (a value halfway between two neighbours)
    f = np.float16(rng.uniform(0.001, 1000, 200))
    nxt = np.nextafter(f, np.float16(np.inf))
    xs = np.concatenate([xs, ((f.astype(np.float64) + nxt.astype(np.float64)) / 2)])
    xs = xs.astype(np.float32)
    got = np.array([orc.f32_to_f16(float(x)) for x in xs], np.uint16)
    want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want), xs[got != want][:5]


def test_q8_0_quantize_invariants():
    """quantize_row_q8_0: d = f16(amax / 127), the largest magnitude maps to
    +-127, every q is round(x / d32) (half away from zero, d32 = amax / 127 in
    f32), an all-zero block has d = 0 and zero quants."""
    rng = np.random.default_rng(91)
    x = (rng.standard_normal(6 * 64) * rng.uniform(0.01, 30, 6 * 64)).astype(np.float32)
    x[32:64] = 0.0
    x[70] = -5.0 * np.abs(x[64:96]).max()
    q = orc.quantize_q8_0(x, 6, 64)
    xb = x.reshape(-1, 32)
    for b in range(q.size):
        amax = np.float32(np.abs(xb[b]).max())
        d32 = np.float32(amax / np.float32(127.0))
        assert q["d"][b] == np.float32(d32).astype(np.float16).view(np.uint16)
        if amax == 0:
            assert not np.any(q["qs"][b])
            continue
        inv = np.float32(np.float32(1.0) / d32)
        prod = (xb[b] * inv).astype(np.float32)
        want = np.sign(prod) * np.floor(np.abs(prod) + 0.5)  # round half away from zero
        assert np.array_equal(q["qs"][b].astype(np.float32), want)
        assert abs(int(q["qs"][b][int(np.argmax(np.abs(xb[b])))])) == 127
    assert q["qs"][2][70 - 64] == -127


@pytest.mark.parametrize("wtype", [orc.WTYPE_Q4_0, orc.WTYPE_Q5_0, orc.WTYPE_Q8_0])
def test_legacy_dot_equals_dequantized_dot(wtype):
    """Each legacy block dot equals the float64 dot of the dequantized blocks
    with the Q8_0 activations, within the f32 bound, on random blocks."""
    from helpers import legacy_weights
    rng = np.random.default_rng(92 + wtype)
    nb = 6
    w = legacy_weights(rng, wtype, 1, 32 * nb)
    x = rng.standard_normal(32 * nb).astype(np.float32)
    y = orc.quantize_q8_0(x, 1, 32 * nb)
    got = orc.vec_dot_legacy(wtype, w, y, nb)
    wv = orc.dequant(wtype, w, nb).astype(np.float64)
    yv = y["qs"].astype(np.float64) * y["d"].view(np.float16).astype(np.float64)[:, None]
    want = float(np.dot(wv, yv.reshape(-1)))
    T = float(np.dot(np.abs(wv), np.abs(yv.reshape(-1))))
    assert abs(got - want) <= (nb + 12) * 2.0 ** -24 * T, (got, want)
    assert abs(want) > 1e-3


@pytest.mark.parametrize("wtype", [orc.WTYPE_Q4_0, orc.WTYPE_Q5_0, orc.WTYPE_Q8_0])
def test_qmatmul_legacy_composition_vs_f64_dequant(wtype):
    """or_qmatmul on Q4_0 / Q5_0 / Q8_0 weights (matmul.rs:103-106, 192-194,
    over Q8_0 activations) against a float64 composition X @ W^T + residual,
    within the bound; the transposed output, swapped weight rows, swapped
    activation rows and a dropped last block each break it."""
    from helpers import legacy_acts_f64, legacy_bound, legacy_dequant_f64, legacy_weights
    rng = np.random.default_rng(17 + wtype)
    rows, cols, n = 9, 160, 5
    w = legacy_weights(rng, wtype, rows, cols)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    x[1, :32] = 0.0
    res = rng.standard_normal((n, rows)).astype(np.float32)
    got = orc.qmatmul(wtype, w, rows, cols, x, n, res).reshape(n, rows).astype(np.float64)
    W = legacy_dequant_f64(orc, wtype, w, rows, cols)
    X = legacy_acts_f64(orc, x, n, cols)
    want = X @ W.T + res
    tol = legacy_bound(orc, wtype, w, rows, cols, x, n, res) + \
        2.0 ** -24 * (np.abs(X) @ legacy_dequant_f64(orc, wtype, w, rows, cols, True).T)
    err = np.abs(got - want)
    assert np.all(err <= tol), float(np.max(err / tol))
    assert np.max(np.abs(want)) > 0.1
    bad_t = want.reshape(-1)[np.arange(n * rows).reshape(rows, n).T.reshape(-1)].reshape(n, rows)
    X_drop = X.copy()
    X_drop[:, -32:] = 0.0
    for name, wrong in (("transposed", bad_t), ("weight rows swapped", X @ W[[1, 0] + list(range(2, rows))].T + res),
                        ("activation rows swapped", X[[1, 0] + list(range(2, n))] @ W.T + res),
                        ("last block dropped", X_drop @ W.T + res)):
        assert np.any(np.abs(got - wrong) > tol), name


def test_post_norm_residual_closed_form_and_f64():
    """forward.rs:346-350: a row of equal values c normalises to
    sign(c) / sqrt(1 + eps / c^2) * w, then the residual is added; random rows
    match a float64 RMSNorm within a few ulp; without the residual the rows are
    only normalised; a forgotten gain or residual is caught."""
    e, eps = 96, 1e-6
    w = np.linspace(0.5, 1.5, e).astype(np.float32)
    cur = np.full((1, e), 3.0, np.float32)
    res = np.arange(e, dtype=np.float32).reshape(1, e)
    orc.post_norm_residual(cur, w, res, 1, e, eps)
    want = (1.0 / np.sqrt(1.0 + eps / 9.0)) * w.astype(np.float64) + res.astype(np.float64)
    assert np.allclose(cur, want, rtol=3e-7, atol=1e-6)
    rng = np.random.default_rng(93)
    x = (rng.standard_normal((4, e)) * 7).astype(np.float32)
    r = rng.standard_normal((4, e)).astype(np.float32)
    got = x.copy()
    orc.post_norm_residual(got, w, r, 4, e, eps)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + eps) * w + r
    assert np.max(np.abs(got - ref)) <= 1e-5
    assert np.max(np.abs(got - (ref - r))) > 0.1 and np.max(np.abs(got - (ref - r) / w - r)) > 0.1
    only = x.copy()
    orc.post_norm_residual(only, w, None, 4, e, eps)
    assert np.max(np.abs(only - (ref - r))) <= 1e-5

"""The C ABI without a GPU: the library loads, exports every symbol declared
in include/dr_attn.h, validates arguments with the reference's contract, and
refuses (rather than computes) when no device is visible.  CPU only."""
from __future__ import annotations

import ctypes
import subprocess

import numpy as np
import pytest

import dr_attn as dr
import oracle as orc


@pytest.fixture(scope="module")
def lib():
    return dr.load()


def test_exports_every_header_symbol(lib):
    names = dr.header_functions()
    assert len(names) >= 20
    nm = subprocess.run(["nm", "-D", "--defined-only", str(dr.LIB_PATH)], capture_output=True,
                        text=True, check=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if line.strip()}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        assert hasattr(lib, n)
    # every header function has a ctypes signature in the binding
    assert set(names) <= set(dr._SIGS)


def test_version_and_device_count(lib):
    assert lib.dr_version().decode().count(".") == 2
    assert dr.device_count() >= 0


def _call(s, nq_len=None, out_len=None, qpos=None, kpos=None, qprefix=()):
    out = np.zeros(max(1, s.nq * s.n_head * s.head_dim), np.float32)
    q = np.zeros(max(1, s.nq * s.n_head * s.head_dim), np.float32)
    k = np.zeros(max(1, s.nk * s.n_head_kv * s.head_dim), np.float32)
    v = np.zeros_like(k)
    lib = dr.load()
    keep = []
    qr = dr.Rows(pos=qpos if qpos is not None else range(s.nq), prefix=qprefix)
    kr = dr.Rows(pos=kpos if kpos is not None else range(s.nk))
    rc = lib.dr_attention(out.ctypes.data, out_len if out_len is not None else s.nq * s.n_head * s.head_dim,
                          q.ctypes.data, q.size, k.ctypes.data, k.size, v.ctypes.data, v.size,
                          s.c(), qr.c(keep), kr.c(keep))
    return rc, lib.dr_last_error().decode()


def test_invalid_shapes_rejected(lib):
    S = dr.AttnShape
    # out.len() != nq*n_head*head_dim (debug_assert attention.rs:107)
    rc, msg = _call(S(2, 3, 2, 2, 8), out_len=5)
    assert rc == dr.DR_ERR_INVALID and "out.len()" in msg
    # qr.pos.len() != nq (:108)
    rc, _ = _call(S(2, 3, 2, 2, 8), qpos=[0])
    assert rc == dr.DR_ERR_INVALID
    # kr.pos.len() != nk (:109)
    rc, _ = _call(S(2, 3, 2, 2, 8), kpos=[0, 1])
    assert rc == dr.DR_ERR_INVALID
    # n_head not a multiple of n_head_kv (the reference indexes out of bounds)
    rc, msg = _call(S(2, 3, 3, 2, 8))
    assert rc == dr.DR_ERR_INVALID and "multiple" in msg
    # per-row prefix shorter than nq (the reference's qr.prefix[i] panics)
    rc, _ = _call(S(2, 3, 2, 2, 8), qprefix=[1])
    assert rc == dr.DR_ERR_INVALID
    # head_dim > 512 is valid for the reference but not built here
    rc, _ = _call(S(1, 1, 1, 1, 516))
    assert rc == dr.DR_ERR_UNSUPPORTED


def test_empty_problems_are_noops(lib):
    # nq == 0 / head_dim == 0: no (head, query) task runs (attention.rs:116)
    assert _call(dr.AttnShape(0, 3, 2, 2, 8))[0] == dr.DR_OK
    assert _call(dr.AttnShape(2, 3, 2, 2, 0))[0] == dr.DR_OK


def test_no_device_is_an_error_not_a_fallback(lib):
    if dr.device_count() > 0:
        pytest.skip("host has a GPU")
    rc, msg = _call(dr.AttnShape(2, 3, 2, 2, 8, scale=0.5))
    assert rc == dr.DR_ERR_NO_DEVICE, msg
    with pytest.raises(dr.DrError) as e:
        dr.Context(0)
    assert e.value.status == dr.DR_ERR_NO_DEVICE


def test_split_active_reference_case(lib):
    # tests.rs:39-53 through the library's stateless split
    prev = np.array([10, 20, -1, -1], np.int32)
    last = np.full(4, -1, np.int32)
    act, cac = dr.split_active(prev, last, [10, 21, -1, -1], [0, 0, 1, 1], 5)
    assert act == [1, 2, 3] and cac == [0]
    prev = np.array([10, 21, -1, -1], np.int32)
    act, cac = dr.split_active(prev, last, [10, 21, -1, -1], [0, 0, 1, 1], 8)
    assert act == [2, 3] and cac == [0, 1]


def test_split_active_matches_oracle_random(lib):
    rng = np.random.default_rng(9)
    n = 200
    prev_a = rng.integers(0, 5, n).astype(np.int32)
    prev_b = prev_a.copy()
    last_a = np.full(n, -1, np.int32)
    last_b = last_a.copy()
    for step in range(12):
        seq = prev_a.copy()
        flip = rng.random(n) < 0.1
        seq[flip] = rng.integers(0, 5, flip.sum())
        masked = (rng.random(n) < 0.2).astype(np.uint8)
        vic = int(step % 3)
        got = dr.split_active(prev_a, last_a, seq, masked, step, vic)
        want = orc.split_active(prev_b, last_b, seq, masked, step, vic)
        assert got == want
        assert np.array_equal(last_a, last_b)
        prev_a, prev_b = seq.copy(), seq.copy()


def test_ring_kernel_dma_stays_inside_the_cache_plane(lib):
    """Every tile the stream kernel's waves request (a wave without tiles too)
    lies inside the kv head's cache plane, and each split's waves multiply
    each tile of its range exactly once.  The tile base is the DMA's scalar
    offset, which the buffer range check does not cover, so a tile past the
    plane would read the next allocation.  Host evaluation of the kernel's
    own tile-assignment code (dr_debug_ring_tiles)."""
    rng = np.random.default_rng(7)
    cases = [(128, 32, 64, None, 0, 0, 1), (256, 1, 64, None, 0, 0, 1), (128, 768, 768, None, 0, 0, 1),
             (256, 4352, 4352, 1024, 4096, 4351, 2), (128, 100, 4096, 16, 40, 60, 3)]
    for _ in range(400):
        hd = int(rng.choice([128, 256]))
        n_total = int(rng.integers(1, 5000))
        nk = int(rng.integers(1, n_total + 1))
        cap = (n_total + 63) // 64 * 64
        window = None if rng.random() < 0.4 else int(rng.integers(1, 2048))
        qmin = int(rng.integers(0, nk))
        qmax = int(rng.integers(qmin, min(nk, qmin + 300)))
        cases.append((hd, nk, cap, window, qmin, qmax, int(rng.integers(1, 5))))
    for hd, nk, cap, window, qmin, qmax, n_split in cases:
        lo, hi, ok = dr.ring_tiles(hd, nk, cap, window, qmin, qmax, n_split)
        assert ok, (hd, nk, cap, window, qmin, qmax, n_split)
        assert 0 <= lo <= hi < cap // 32, (hd, nk, cap, window, qmin, qmax, n_split, lo, hi)
    # one 32-key tile: seven of eight waves own none; their DMA is clamped to
    # the plane's last tile (unclamped it would be tile 7 of a 2-tile plane)
    assert dr.ring_tiles(128, 32, 64, None, 0, 0, 1) == (0, 1, True)
    with pytest.raises(dr.DrError):
        dr.ring_tiles(64, 32, 64, None, 0, 0, 1)  # no stream kernel at hd 64


def test_alloc_counter_counts_no_device_calls(lib):
    """The allocation counter is host-side state: readable without a GPU and
    unchanged by calls that fail before allocating."""
    before = dr.alloc_count()
    assert before >= 0
    rc, _ = _call(dr.AttnShape(2, 3, 2, 2, 8), out_len=5)
    assert rc == dr.DR_ERR_INVALID
    assert dr.alloc_count() == before

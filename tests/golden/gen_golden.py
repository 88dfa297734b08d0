"""Writes tests/golden/cases.json and tests/golden/expected.npz.

Every case is an attention problem whose inputs are closed-form (the
reference's own test inputs, tests.rs:70-237, or the same formula family at
larger head dims), so only the expected outputs are stored.  Expected values
come from the float64 three-pass brute force in tests/helpers.py; the first
case is additionally the reference's known answer (tests.rs:104-114).

Run: python tests/golden/gen_golden.py
"""
from __future__ import annotations

import json
import math
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

from helpers import brute_force, materialise  # noqa: E402

Q_GEN = [37, 101, 50.0, 50.0]
K_GEN = [53, 97, 48.0, 48.0]
V_GEN = [71, 89, 44.0, 44.0]


def case(name, shape, qrows, krows, q, k, v, note):
    return {"name": name, "shape": shape, "qrows": qrows, "krows": krows, "q": q, "k": k, "v": v,
            "note": note}


def sh(nq, nk, h, hkv, hd, window=None, prefix=None, scale=1.0):
    return {"nq": nq, "nk": nk, "n_head": h, "n_head_kv": hkv, "head_dim": hd,
            "sliding_window": window, "causal_prefix": prefix, "scale": scale}


def rows(pos, seq=(), prefix=()):
    return {"pos": list(pos), "seq": list(seq), "prefix": list(prefix)}


CASES = [
    case("ref_uniform_scores", sh(1, 2, 1, 1, 2), rows(range(1)), rows(range(2)),
         {"values": [1.0, 0.0]}, {"values": [1.0, 0.0, 1.0, 0.0]},
         {"values": [0.0, 2.0, 4.0, 6.0]},
         "tests.rs:104-114: identical keys -> mean of values = [2, 4]"),
    case("ref_naive_reference", sh(4, 6, 2, 2, 8), rows(range(4)), rows(range(6)),
         {"gen": [37, 101, 50.0, 25.0]}, {"gen": [53, 97, 48.0, 24.0]}, {"gen": V_GEN},
         "tests.rs:154-186 inputs"),
    case("ref_gqa", sh(3, 5, 4, 2, 8), rows(range(3)), rows(range(5)),
         {"gen": Q_GEN}, {"gen": K_GEN}, {"gen": V_GEN}, "tests.rs:116-152 inputs (GQA 4/2)"),
    case("ref_block_diagonal", sh(5, 5, 1, 1, 4), rows([0, 1, 0, 1, 2], [0, 0, 1, 1, 1]),
         rows([0, 1, 0, 1, 2], [0, 0, 1, 1, 1]),
         {"gen": Q_GEN}, {"gen": Q_GEN}, {"gen": V_GEN}, "tests.rs:70-102 batched rows"),
    case("ref_avx2_scalar", sh(3, 3, 2, 2, 16), rows(range(3)), rows(range(3)),
         {"gen": Q_GEN}, {"gen": K_GEN}, {"gen": V_GEN}, "tests.rs:188-213 inputs"),
    case("hd128_dense_canvas", sh(8, 40, 4, 2, 128, scale=1 / math.sqrt(128)),
         rows(range(32, 40)), rows(range(40)),
         {"gen": Q_GEN}, {"gen": K_GEN}, {"gen": V_GEN},
         "8 canvas queries (pos 32..39) over 40 keys, GQA 4/2, hd 128"),
    case("hd128_window_reordered", sh(8, 40, 4, 2, 128, window=5, scale=1 / math.sqrt(128)),
         rows([3, 9, 17, 20, 25, 31, 36, 39]),
         rows([0, 1, 2, 4, 5, 6, 7, 8, 10, 11, 12, 13, 14, 15, 16, 18, 19, 21, 22, 23, 24, 26,
               27, 28, 29, 30, 32, 33, 34, 35, 37, 38, 3, 9, 17, 20, 25, 31, 36, 39]),
         {"gen": Q_GEN}, {"gen": K_GEN}, {"gen": V_GEN},
         "sliding window 5 with keys in [cached | active] order (forward.rs:91-101)"),
    case("hd128_causal_prefix", sh(10, 30, 2, 2, 128, prefix=20, scale=1 / math.sqrt(128)),
         rows([0, 3, 7, 11, 19, 20, 21, 25, 28, 29]), rows(range(30)),
         {"gen": Q_GEN}, {"gen": K_GEN}, {"gen": V_GEN},
         "Gemma dual mode: prompt rows (< 20) causal, canvas rows bidirectional"),
    case("hd128_rowprefix_seq", sh(9, 9, 2, 1, 128, scale=0.125),
         rows([0, 1, 2, 3, 0, 1, 2, 3, 4], [0, 0, 0, 0, 1, 1, 1, 1, 1], [2, 2, 2, 2, 3, 3, 3, 3, 3]),
         rows([0, 1, 2, 3, 0, 1, 2, 3, 4], [0, 0, 0, 0, 1, 1, 1, 1, 1]),
         {"gen": Q_GEN}, {"gen": K_GEN}, {"gen": V_GEN},
         "two batched sequences, per-row causal prefix (forward.rs:153-160)"),
    case("hd256_gemma_window_prefix", sh(6, 70, 2, 1, 256, window=16, prefix=60, scale=1 / 16),
         rows([10, 40, 59, 60, 64, 69]), rows(range(70)),
         {"gen": Q_GEN}, {"gen": K_GEN}, {"gen": V_GEN},
         "hd 256, sliding window 16 and causal prefix 60"),
    case("hd64_all_masked_rows", sh(4, 12, 2, 2, 64, window=1, scale=0.125),
         rows([0, 3, 50, 11]), rows(range(12)),
         {"gen": Q_GEN}, {"gen": K_GEN}, {"gen": V_GEN},
         "window 1: query at position 50 sees no key -> NaN row (attention.rs:181-185)"),
    case("hd96_gqa3_padded", sh(7, 33, 3, 1, 96, scale=1 / math.sqrt(96)),
         rows(range(26, 33)), rows(range(33)),
         {"gen": Q_GEN}, {"gen": K_GEN}, {"gen": V_GEN},
         "head_dim 96 (not a tile size) with 3 query heads per KV head"),
    case("hd128_scale1_gemma", sh(4, 64, 2, 1, 128, scale=1.0),
         rows(range(60, 64)), rows(range(64)),
         {"gen": Q_GEN}, {"gen": K_GEN}, {"gen": V_GEN},
         "unscaled scores (Gemma kq_scale 1.0, forward.rs:338-341): score std ~4"),
]


def main():
    expected = {}
    for c in CASES:
        s, qr, kr, q, k, v = materialise(c)
        expected[c["name"]] = brute_force(q, k, v, s, qr, kr).astype(np.float64)
    # the reference's known answer
    assert np.allclose(expected["ref_uniform_scores"].reshape(-1), [2.0, 4.0])
    (HERE / "cases.json").write_text(json.dumps(CASES, indent=1) + "\n")
    np.savez_compressed(HERE / "expected.npz", **expected)
    print(f"wrote {len(CASES)} cases")


if __name__ == "__main__":
    main()

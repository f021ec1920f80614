"""The committed golden fixture (``tests/golden/q4_small.npz``) against the
oracle and against what fixes it independently of the oracle.

The fixture was written by ``tests/golden/make_golden.py``; this file checks
that the oracle still reproduces it bit for bit, that its e4m3 bytes (from
torch, the encoder ``src/vk_engine.py:136`` calls) and int32 accumulators
(int64 matmul) agree with the oracle's own, and a few hand-computed entries.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import q4_oracle as O

FIX = Path(__file__).resolve().parent / "golden" / "q4_small.npz"


@pytest.fixture(scope="module")
def gold():
    with np.load(FIX, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def test_oracle_reproduces_fixture(gold):
    from tests.golden.make_golden import build

    fresh = build()
    assert set(fresh) == set(gold)
    for k, v in fresh.items():
        assert v.dtype == gold[k].dtype and v.shape == gold[k].shape, k
        assert (np.asarray(v).reshape(-1).view(np.uint8) == gold[k].reshape(-1).view(np.uint8)).all(), k


def test_fixture_formats_round_trip(gold):
    N = int(gold["N"])
    assert (O.unpack_ref(gold["wp_ref"], N) == gold["q"]).all()
    assert (gold["scb16_ref"] == gold["sc"].T.astype(np.float16)).all()
    # torch's e4m3 bytes decode to the lifted scales within e4m3 precision and
    # equal the oracle's encoder output
    shift = int(gold["e4m3_shift"])
    lifted = np.clip(gold["sc"] * np.float32(2.0 ** shift), 0, 448)
    assert (O.e4m3_encode(lifted) == gold["e8"]).all()
    assert float(gold["e4m3_inv"]) == 2.0 ** -shift


def test_fixture_accumulators_independent(gold):
    assert (O.int_matmul_exact(gold["A"], gold["W8"]) == gold["C_w8a8"]).all()
    assert (O.int_matmul_exact(gold["A"], gold["W8_w4a8"]) == gold["C_w4a8"]).all()


def test_fixture_known_answers(gold):
    # row 1: block scale exactly 2^-6, quotients 7, 3.5, -2.5, 0.5, -0.5, 1.5, -7, 2.5 (ties to even)
    assert gold["sc"][1, 0] == np.float32(2.0 ** -6)
    assert list(gold["q"][1, :8]) == [15, 12, 6, 8, 8, 10, 1, 10]
    assert gold["sc"][0, 0] == np.float32(1e-8) and (gold["q"][0, :32] == 8).all()
    # activation rows: zero row -> 1e-12 floor, all codes 0; row 1 -> s = 1/16, ties to even
    assert gold["sa"][0] == np.float32(1e-12) and (gold["A"][0] == 0).all()
    assert gold["sa"][1] == np.float32(1.0 / 16.0)
    assert list(gold["A"][1, :4]) == [127, -126, -124, -124]
    # float64 brute force of one GEMV output and one W4A16 output
    q, s16, x = gold["q"].astype(np.float64) - 8, gold["scb16_ref"].T.astype(np.float64), gold["x"].astype(np.float64)
    y5 = sum(q[5, k] * s16[5, k // 32] * x[k] for k in range(q.shape[1]))
    assert abs(y5 - gold["y_f16s"][5]) <= 1e-5 * max(1.0, abs(y5))
    X = gold["X"].astype(np.float64)
    y37 = sum(X[3, k] * q[7, k] * s16[7, k // 32] for k in range(q.shape[1]))
    assert abs(y37 - gold["Y_w4a16"][3, 7]) <= 1e-5 * max(1.0, abs(y37))

"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each check is chosen so that a plausible slip in the restatement fails it:
reciprocal-multiply instead of true division, round-half-away instead of
half-to-even, quantizing with the fp32 scale instead of the fp16 one, a wrong
nibble order, a lost sign restore, a dropped padding column, a wrong fp16
subnormal rounding.  The reference's own known answers
(Kshipra tests/test_quantization.py) are restated here as well.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from oracle import quant
from cases import adversarial_rows
from exact_ref import (F16, exact_f16, exact_quantize_int4, exact_quantize_int8,
                       round_to_format)


# ---------------------------------------------------------------------- #
# fp16 conversion
# ---------------------------------------------------------------------- #


def test_f32_to_f16_matches_numpy_on_every_boundary_and_tie():
    """Every fp16 value, its neighbours' midpoints (ties) and one ulp either
    side, plus the subnormal/underflow and overflow edges, against numpy's
    independent RNE conversion."""
    h = np.arange(0, 0x7C00, dtype=np.uint16)                   # all finite positive fp16
    v = h.view(np.float16).astype(np.float64)
    nxt = np.append(v[1:], 65520.0)
    mids = ((v + nxt) / 2).astype(np.float32)                    # exact ties (representable in f32)
    f = np.concatenate([v.astype(np.float32), mids,
                        np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(np.inf)),
                        np.array([2.0 ** -25, 2.0 ** -26, 1e-8, 65504, 65519.99, 65520, 1e9],
                                 np.float32)])
    f = np.concatenate([f, -f])
    got = quant.c_f32_to_f16_bits(f)
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f32_to_f16_matches_exact_rational_rounding():
    rng = np.random.default_rng(7)
    f = (rng.standard_normal(2000) * 10.0 ** rng.integers(-9, 5, 2000)).astype(np.float32)
    got = quant.c_f32_to_f16_bits(f).view(np.float16).astype(np.float64)
    want = np.array([exact_f16(float(x)) for x in f])
    assert np.array_equal(got, want)


def test_f16_to_f32_is_exact_for_all_65536_patterns():
    L = quant.lib()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([L.kqo_f16_to_f32(int(b)) for b in h], np.float32)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])


# ---------------------------------------------------------------------- #
# Quantize: exact rational arithmetic vs both restatements
# ---------------------------------------------------------------------- #


@pytest.mark.parametrize("k", [1, 7, 128, 200])
def test_int8_matches_exact_rational(k):
    w = adversarial_rows(np.random.default_rng(k), k)
    qe, se = exact_quantize_int8(w)
    qc, sc = quant.c_quantize_int8(w)
    qn, sn = quant.np_quantize_int8(w)
    assert np.array_equal(se.view(np.uint16), sc.view(np.uint16))
    assert np.array_equal(se.view(np.uint16), sn.view(np.uint16))
    assert np.array_equal(qe, qc)
    assert np.array_equal(qe, qn)


@pytest.mark.parametrize("k,g", [(1, 128), (100, 128), (128, 128), (300, 128), (96, 32), (130, 2), (500, 256)])
def test_int4_matches_exact_rational(k, g):
    w = adversarial_rows(np.random.default_rng(k + g), k)
    qe, se = exact_quantize_int4(w, g)
    pc, sc, kp = quant.c_quantize_int4(w, g)
    pn, sn, kpn = quant.np_quantize_int4(w, g)
    assert kp == kpn == qe.shape[1]
    assert np.array_equal(se.view(np.uint16), sc.view(np.uint16))
    assert np.array_equal(se.view(np.uint16), sn.view(np.uint16))
    assert np.array_equal(quant.np_unpack_int4(pc), qe)
    assert np.array_equal(pc, pn)


def test_ties_round_half_to_even():
    """w / s == j + 0.5 exactly must round to the even neighbour."""
    w = np.array([[127 * 2.0 ** -7, 0.5 * 2 ** -7, 1.5 * 2 ** -7, 2.5 * 2 ** -7, -2.5 * 2 ** -7,
                   125.5 * 2 ** -7, 126.5 * 2 ** -7]], np.float32)
    q, s = quant.c_quantize_int8(w)
    assert float(s[0]) == 2.0 ** -7
    assert q[0].tolist() == [127, 0, 2, 2, -2, 126, 126]


def _near_tie_row(m: float) -> np.ndarray:
    """A row with max |w| = m and many entries a few ulps from (j + 0.5) * s,
    where the rounding of w / s decides q."""
    s = np.float32(np.float16(np.float32(m) / np.float32(127)))
    j = np.arange(0, 126, dtype=np.float64)
    base = ((j + 0.5) * float(s)).astype(np.float32)
    cands = [base]
    for d in range(1, 4):
        cands.append(np.nextafter(base, np.float32(np.inf)))
        cands.append(np.nextafter(base, np.float32(0)))
        base = cands[-2]
    row = np.concatenate([[np.float32(m)], np.concatenate(cands)])
    return row.astype(np.float32)


def test_true_division_not_reciprocal_multiply():
    """A reciprocal-multiply variant of the oracle (a plausible slip) is caught
    by the exact-rational restatement on near-tie inputs."""
    rows = [_near_tie_row(m) for m in (0.9, 0.77, 1.3, 0.031, 5.5)]
    w = np.stack(rows)
    qe, se = exact_quantize_int8(w)
    q, s = quant.c_quantize_int8(w)
    assert np.array_equal(q, qe) and np.array_equal(s.view(np.uint16), se.view(np.uint16))
    s32 = s.astype(np.float32)[:, None]
    q_recip = np.clip(np.rint(w * (np.float32(1) / s32)), -127, 127).astype(np.int8)
    assert (q_recip != qe).any(), "planted reciprocal-multiply slip must be detected"


def test_fp16_scale_is_the_quantization_scale():
    """Quantizing with the fp32 scale while storing the fp16 one (the slip the
    reference warns about at engine/quantization.py:209-214) breaks the
    half-scale bound on some rows; the oracle must not."""
    rng = np.random.default_rng(11)
    w = rng.standard_normal((4096, 64)).astype(np.float32)
    q, s = quant.c_quantize_int8(w)
    s32 = s.astype(np.float32)[:, None]
    err = np.abs(w - q.astype(np.float32) * s32).max(axis=1)
    assert (err <= s.astype(np.float32) / 2).all()
    # planted slip, on the CPU: divide by the fp32 scale
    m = np.abs(w).max(axis=1)
    sf = np.maximum(m / np.float32(127), np.float32(1e-8))
    q_bad = np.clip(np.rint(w / sf[:, None]), -127, 127)
    err_bad = np.abs(w - q_bad * sf.astype(np.float16).astype(np.float32)[:, None]).max(axis=1)
    assert (err_bad > s.astype(np.float32) / 2).any()


def test_max_element_maps_to_127_and_sign_symmetry():
    w = np.random.default_rng(5).standard_normal((256, 300)).astype(np.float32) * 0.02
    q, s = quant.c_quantize_int8(w)
    idx = np.abs(w).argmax(axis=1)
    assert (np.abs(q[np.arange(256), idx]) == 127).all()
    qn, sn = quant.c_quantize_int8(-w)
    assert np.array_equal(qn, -q) and np.array_equal(sn, s)
    p4, s4, _ = quant.c_quantize_int4(w, 128)
    p4n, s4n, _ = quant.c_quantize_int4(-w, 128)
    assert np.array_equal(quant.np_unpack_int4(p4n), -quant.np_unpack_int4(p4))
    assert np.array_equal(s4n, s4)


def test_ranges():
    w = adversarial_rows(np.random.default_rng(2), 256)
    q, _ = quant.c_quantize_int8(w)
    assert q.min() >= -127 and q.max() <= 127
    p, _, _ = quant.c_quantize_int4(w, 128)
    u = quant.np_unpack_int4(p)
    assert u.min() >= -8 and u.max() <= 7
    # -8 appears only through the +-inf case (fp16 scale 0): row 3 of adversarial_rows
    rows_with_m8 = np.unique(np.nonzero(u == -8)[0])
    assert set(rows_with_m8.tolist()) <= {3}


# ---------------------------------------------------------------------- #
# Packing
# ---------------------------------------------------------------------- #


def test_pack_unpack_all_256_bytes():
    b = np.arange(256, dtype=np.uint8).reshape(1, 256)
    u = quant.np_unpack_int4(b)                                   # [1, 512]
    lo, hi = u[0, 0::2].astype(int), u[0, 1::2].astype(int)
    for byte in range(256):
        ln, hn = byte & 0xF, byte >> 4
        assert lo[byte] == (ln - 16 if ln >= 8 else ln)
        assert hi[byte] == (hn - 16 if hn >= 8 else hn)
    repacked = ((u[:, 0::2].view(np.uint8) & 0xF) | ((u[:, 1::2].view(np.uint8) & 0xF) << 4))
    assert np.array_equal(repacked, b)


def test_low_nibble_is_even_column():
    """q = [1, -2] packs to 0xE1 (engine/quantization.py:259-270)."""
    s = 2.0 ** -5
    w = np.zeros((1, 128), np.float32)
    w[0, 0], w[0, 1], w[0, 2] = 1 * s, -2 * s, 7 * s              # max 7s -> scale s
    p, sc, _ = quant.c_quantize_int4(w, 128)
    assert float(sc[0, 0]) == s
    assert p[0, 0] == 0xE1 and p[0, 1] == 0x07


# ---------------------------------------------------------------------- #
# The reference tests' known answers (Kshipra tests/test_quantization.py)
# ---------------------------------------------------------------------- #


def test_one_by_one_weight():
    """:212-218: 1.5 -> q = 127, s = fp16(1.5 / 127)."""
    q, s = quant.c_quantize_int8(np.array([[1.5]], np.float32))
    assert q[0, 0] == 127
    assert float(s[0]) == float(np.float16(np.float32(1.5) / np.float32(127)))
    w_hat = quant.c_dequantize_int8(q, s)
    assert abs(w_hat[0, 0] - 1.5) / 1.5 < 1e-3


def test_zero_row():
    """:234-239: an all-zero row dequantizes to 0; its fp16 scale is +0."""
    q, s = quant.c_quantize_int8(np.zeros((4, 128), np.float32))
    assert (q == 0).all() and (s.view(np.uint16) == 0).all()
    assert (quant.c_dequantize_int8(q, s) == 0).all()


def test_in_features_one_and_padding():
    """:221-225 and :107-117, :189-197."""
    p, s, kp = quant.c_quantize_int4(np.array([[0.5], [-0.3]], np.float32), 128)
    assert kp == 128 and p.shape == (2, 64) and s.shape == (2, 1)
    assert quant.c_dequantize_int4(p, s, 1, 128).shape == (2, 1)
    w = np.random.default_rng(3).standard_normal((16, 500)).astype(np.float32)
    p, s, kp = quant.c_quantize_int4(w, 128)
    assert kp == 512
    u = quant.np_unpack_int4(p)
    assert (u[:, 500:] == 0).all()                                  # padding quantizes to 0
    w_hat = quant.c_dequantize_int4(p, s, 500, 128)
    assert w_hat.shape == (16, 500)
    assert np.linalg.norm(w_hat - w) / np.linalg.norm(w) < 0.25


def test_storage_accounting():
    """:37-76: INT8 N*K + 2N bytes; INT4 N*K/2 + 2*N*K/128, 4.125 bits/weight."""
    n = k = 4096
    assert quant.algorithmic_bytes(0, n, k, "int8") == n * k + 2 * n
    w4 = quant.algorithmic_bytes(0, n, k, "int4", 128)
    assert w4 == n * k // 2 + n * (k // 128) * 2
    assert (n * (k // 128) * 2) / (n * k // 2) == pytest.approx(0.03125, rel=1e-12)
    assert w4 * 8 / (n * k) == pytest.approx(4.125, abs=1e-3)
    assert w4 < n * k * 2 / 3


def test_half_scale_bounds():
    """:84-104: per-row / per-group |w - w_hat| <= s / 2 (+1e-6)."""
    rng = np.random.default_rng(1)
    w = rng.standard_normal((64, 512)).astype(np.float32)
    q, s = quant.c_quantize_int8(w)
    err = np.abs(w - quant.c_dequantize_int8(q, s)).max(axis=1)
    assert (err <= s.astype(np.float32) / 2 + 1e-6).all()
    w = rng.standard_normal((32, 512)).astype(np.float32)
    p, s, _ = quant.c_quantize_int4(w, 128)
    err = np.abs(w - quant.c_dequantize_int4(p, s, 512, 128)).reshape(32, 4, 128).max(axis=-1)
    assert (err <= s.astype(np.float32) / 2 + 1e-6).all()


def test_dequantize_is_exact_product():
    """q * s is exact in fp32 (at most 7 + 11 significant bits); the C and numpy
    dequantizers agree bit for bit and with the rational product."""
    w = adversarial_rows(np.random.default_rng(9), 256)
    q, s = quant.c_quantize_int8(w)
    a, b = quant.c_dequantize_int8(q, s), quant.np_dequantize_int8(q, s)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    for r in range(w.shape[0]):
        for c in (0, 17, 255):
            if np.isfinite(s[r]):
                assert Fraction(float(a[r, c])) == Fraction(int(q[r, c])) * Fraction(float(s[r]))
    p, s4, _ = quant.c_quantize_int4(w, 64)
    a, b = quant.c_dequantize_int4(p, s4, 256, 64), quant.np_dequantize_int4(p, s4, 256, 64)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("shape,g", [((64, 512), 128), ((33, 4864), 128), ((17, 896), 32), ((5, 1000), 256)])
def test_c_and_numpy_restatements_agree(shape, g):
    w = (np.random.default_rng(shape[0]).standard_normal(shape) * 0.02).astype(np.float32)
    qc, sc = quant.c_quantize_int8(w)
    qn, sn = quant.np_quantize_int8(w)
    assert np.array_equal(qc, qn) and np.array_equal(sc.view(np.uint16), sn.view(np.uint16))
    pc, s4c, _ = quant.c_quantize_int4(w, g)
    pn, s4n, _ = quant.np_quantize_int4(w, g)
    assert np.array_equal(pc, pn) and np.array_equal(s4c.view(np.uint16), s4n.view(np.uint16))


def test_count_nonfinite():
    w = np.ones((3, 5), np.float32)
    assert quant.c_count_nonfinite(w) == 0
    w[1, 2], w[2, 4] = np.nan, -np.inf
    assert quant.c_count_nonfinite(w) == 2


# ---------------------------------------------------------------------- #
# Linear
# ---------------------------------------------------------------------- #


def test_linear_f64_matches_exact_sum():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 40)).astype(np.float32)
    w = rng.standard_normal((5, 40)).astype(np.float32) * 0.02
    b = rng.standard_normal(5).astype(np.float32)
    q, s = quant.c_quantize_int8(w)
    w_hat = quant.c_dequantize_int8(q, s)
    y = quant.linear_f64(x, w_hat, b)
    for i in range(3):
        for j in range(5):
            exact = sum(Fraction(float(a)) * Fraction(float(c)) for a, c in zip(x[i], w_hat[j]))
            exact += Fraction(float(b[j]))
            assert abs(float(exact) - y[i, j]) <= 1e-15 * (1 + abs(float(exact)))


def test_linear_f32_close_to_f64():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((16, 512)).astype(np.float32)
    w = rng.standard_normal((512, 512)).astype(np.float32) * 0.02
    w_hat = quant.c_dequantize_int4(*quant.c_quantize_int4(w, 128)[:2], 512, 128)
    y32, y64 = quant.linear_f32(x, w_hat), quant.linear_f64(x, w_hat)
    assert np.abs(y32 - y64).max() / np.abs(y64).max() < 1e-5


def test_round_to_format_self_check():
    """The exact helper itself: known fp16 facts."""
    assert round_to_format(Fraction(65504), F16) == 65504
    assert round_to_format(Fraction(65520), F16) == float("inf")
    assert round_to_format(Fraction(1, 2 ** 25), F16) == 0                 # tie -> even (0)
    assert round_to_format(Fraction(3, 2 ** 26), F16) == Fraction(1, 2 ** 24)
    assert round_to_format(Fraction(1, 2 ** 24), F16) == Fraction(1, 2 ** 24)

"""The oracle's 24-bit rounding (or_round24) against its closed form.

The default per-token forward stores fc1's dequantised output rounded to
its top 24 bits (sign, exponent, 15 mantissa bits) for the GELU +
quantisation pass to read. The oracle restates that rounding on the bit
pattern (add 0x80, clear the low byte). Here it is checked against the
arithmetic definition, evaluated in float64: round |x| to a multiple of its
ulp at 15 mantissa bits, 2^(e - 15) for 2^e <= |x| < 2^(e + 1) (2^-141 in
the subnormal range), ties away from zero; values that round to 2^128 become
infinity; NaN becomes the quiet NaN. A dropped carry, a wrong tie direction or a wrong
bit count fails it.
"""
import numpy as np
import pytest


def round24_closed_form(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float32)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        a = np.abs(x.astype(np.float64))
        _, E = np.frexp(a)  # a = m 2^E, m in [0.5, 1)
        e = np.where(a < 2.0 ** -126, -126, E - 1)
        ulp = np.ldexp(1.0, e - 15)
        r = np.floor(a / ulp + 0.5) * ulp
        out = (np.sign(x.astype(np.float64)) * r).astype(np.float32)
        out = np.where(a == 0, x, out)  # keeps the sign of zero
        out = np.where(np.isinf(x), x, out)
        return np.where(np.isnan(x), np.float32(np.nan), out).astype(np.float32)


def _from_bits(b):
    return np.asarray(b, np.uint32).view(np.float32)


def _check(oracle, x):
    got, want = oracle.round24(x), round24_closed_form(x)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    gb, wb = got.view(np.uint32), want.view(np.uint32)
    bad = ~nan & (gb != wb)
    assert not bad.any(), (x[bad][:4], got[bad][:4], want[bad][:4])
    assert np.all(gb & 0xFF == 0)


def test_round24_dense_bit_patterns(oracle):
    """Every 251st float32 bit pattern (17.1 M values, all exponents and
    both signs), NaNs and infinities included."""
    bits = np.arange(0, 1 << 32, 251, dtype=np.uint64).astype(np.uint32)
    _check(oracle, _from_bits(bits))


def test_round24_ties_and_neighbours(oracle):
    """Low bytes 0x7f, 0x80 (the tie) and 0x81 under 200 000 random upper
    parts: below, at and above every rounding boundary."""
    r = np.random.default_rng(24)
    hi = r.integers(0, 1 << 24, size=200_000, dtype=np.uint64).astype(np.uint32) << 8
    for low in (0x7F, 0x80, 0x81, 0x00, 0xFF):
        _check(oracle, _from_bits(hi | np.uint32(low)))


@pytest.mark.parametrize("bits,want", [
    (0x3F800080, 0x3F800100),  # 1 + 2^-16: a tie, away from zero
    (0x3F80007F, 0x3F800000),  # just below the tie
    (0xBF800080, 0xBF800100),  # negative tie: away from zero
    (0x3FFFFF80, 0x40000000),  # carry into the exponent
    (0x7F7FFF80, 0x7F800000),  # rounds past the largest float: infinity
    (0x7F7FFF7F, 0x7F7FFF00),
    (0x00000080, 0x00000100),  # subnormal tie
    (0x807FFF80, 0x80800000),  # subnormal rounding up to the smallest normal
    (0x7F800000, 0x7F800000),  # infinity
    (0x80000000, 0x80000000),  # -0
])
def test_round24_special_values(oracle, bits, want):
    got = oracle.round24(_from_bits([bits])).view(np.uint32)[0]
    assert got == want, hex(int(got))


@pytest.mark.parametrize("bits", [0x7F800001, 0x7FFFFFFF, 0xFFFFFFFF, 0x7FC00000, 0xFF800080])
def test_round24_keeps_nan(oracle, bits):
    """A plain add of 0x80 would turn 0x7fffffff into -0.0 and 0x7f800001
    into infinity; the rounding keeps every NaN a NaN."""
    got = oracle.round24(_from_bits([bits]))
    assert np.isnan(got[0])
    assert got.view(np.uint32)[0] == 0x7FC00000  # the quiet NaN, as the GPU epilogue writes

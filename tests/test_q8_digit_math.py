"""CPU check of the integer-digit Q8_0 matvec's arithmetic (emulated exactly in q8_digits.py)
against f64 dequantize-then-matvec, on ordinary and adversarial blocks: an outlier next to small
values (the outlier's quant 0, so the small values carry the whole dot product), values spread
over many binades, denormals, and all-zero blocks. The bound checked is the one the header
states: 2^-30 of the block's largest |x| times sum |d q|, plus f32 rounding."""
import numpy as np
import pytest

from q8_digits import block_bound, block_values


def _case(kind, rng, rows=16, nb=64):
    x = rng.standard_normal((nb, 32)).astype(np.float32)
    q = rng.integers(-127, 128, size=(rows, nb, 32)).astype(np.int8)
    d = rng.uniform(0.001, 0.02, (rows, nb)).astype(np.float16)
    if kind == "outlier":
        x[:, 1:] = (rng.standard_normal((nb, 31)) * 1e-3).astype(np.float32)
        x[:, 0] = 1000.0
        q[:, :, 0] = 0
    elif kind == "binades":
        x *= np.float32(2.0) ** rng.integers(-60, 60, size=(nb, 32)).astype(np.float32)
    elif kind == "denormal":
        x = (x * np.float32(1e-40)).astype(np.float32)
    elif kind == "zero":
        x[::3] = 0.0
    return x, q, d


@pytest.mark.parametrize("kind", ["normal", "outlier", "binades", "denormal", "zero"])
def test_digit_block_values_within_stated_bound(kind):
    rng = np.random.default_rng(5)
    x, q, d = _case(kind, rng)
    got = block_values(x, q, d).astype(np.float64)
    exact = np.einsum("rbi,bi->rb", q.astype(np.float64), x.astype(np.float64)) * d.astype(np.float64)
    assert np.all(np.abs(got - exact) <= block_bound(x, q, d))


def test_outlier_block_is_accurate_relative_to_its_small_values():
    """The case the earlier 3-digit (2^-22) form lost: 1000 beside N(0, 1e-3) values with the
    outlier's quant 0. The 4-digit form's error stays below 1e-3 of the small values' dot product
    (the 3-digit form's was about 40% of it)."""
    rng = np.random.default_rng(9)
    x, q, d = _case("outlier", rng, rows=64, nb=16)
    got = block_values(x, q, d).astype(np.float64)
    exact = np.einsum("rbi,bi->rb", q.astype(np.float64), x.astype(np.float64)) * d.astype(np.float64)
    scale = np.abs(q.astype(np.float64)).sum(axis=2) * np.abs(d.astype(np.float64)) * 1e-3
    assert np.all(np.abs(got - exact) <= 1e-3 * scale)

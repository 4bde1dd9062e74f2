"""Pins for oracle/canon.py (the canonical reduction orders)."""
from fractions import Fraction

import numpy as np

from oracle import canon


def _scalar_wave_sum(x):
    """Direct transcription of the lane loop + butterfly, one scalar at a time."""
    lanes = [0.0] * 64
    for i, v in enumerate(x):
        lanes[i % 64] = lanes[i % 64] + float(v)
    for off in (32, 16, 8, 4, 2, 1):
        lanes = [lanes[j] + lanes[j ^ off] for j in range(64)]
    assert len(set(lanes)) == 1  # every lane ends with the same value
    return lanes[0]


def test_wave_sum_matches_scalar_restatement():
    rng = np.random.default_rng(0)
    for n in (1, 63, 64, 65, 130, 1000, 2072):
        x = (rng.standard_normal(n) * 10.0 ** rng.integers(-20, 20, n)).astype(np.float32)
        assert canon.wave_sum(x) == _scalar_wave_sum(x)


def test_sums_exact_when_float64_is_exact():
    rng = np.random.default_rng(1)
    x = rng.integers(-2 ** 20, 2 ** 20, (7, 513)).astype(np.float32) / np.float32(1024)
    exact = [float(sum(Fraction(float(v)) for v in row)) for row in x]
    assert np.array_equal(canon.wave_sum(x, axis=-1), exact)
    assert np.array_equal(canon.seq_sum(x, axis=-1), exact)


def test_order_matters_and_is_fixed():
    # 1 + 2^-53 + ... : sequential order loses the small terms, the
    # lane/butterfly order keeps some of them; the two definitions must differ
    x = np.array([1.0] + [2.0 ** -53] * 127, dtype=np.float64)
    seq = canon.seq_sum(x)
    wav = canon.wave_sum(x)
    assert seq == 1.0
    assert wav != seq
    # a butterfly missing its last stage would not be lane-invariant
    lanes = np.arange(64, dtype=np.float64) * 2.0 ** -40 + 1.0
    full = canon.wave_sum(lanes)
    partial = lanes.copy()
    for off in (32, 16, 8, 4, 2):
        partial = partial + partial[np.arange(64) ^ off]
    assert len(set(partial.tolist())) > 1 and full == _scalar_wave_sum(lanes)


def test_order_key_is_monotone_and_folds_zero():
    vals = np.array([-np.inf, -3.0, -1e-30, -0.0, 0.0, 1e-45, 1e-30, 1.0, 2.0, np.finfo(np.float32).max, np.inf,
                     np.nan], dtype=np.float32)
    keys = canon.order_key(vals).astype(np.int64)
    assert keys[3] == keys[4]                       # -0 == +0
    assert np.all(np.diff(np.delete(keys, 3)) > 0)  # strictly increasing otherwise; NaN on top


def test_clamps_propagate_nan_like_torch():
    import torch
    x = np.array([np.nan, -1.0, 0.5, 2.0, -0.0], dtype=np.float32)
    t = torch.from_numpy(x)
    np.testing.assert_array_equal(canon.clamp01(x), t.clamp(0, 1).numpy())
    got = canon.clamp_min0(x)
    assert np.isnan(got[0]) and got[1] == 0 and got[2] == 0.5 and got[4] == 0 and not np.signbit(got[4])

"""Calibration table derivation (run_statequant.py:81-83), host only.

The table orders each (layer, group) row's 128 coordinates by decreasing mean
|FP16 carry|; equal means keep coordinate order.  Checked against a brute-force
selection (repeatedly take the first maximum of what is left), which fixes both
the direction and the tie rule independently of any sort routine.
"""
import numpy as np
import pytest
import torch

from mamba2_recall import state_codec
from mamba2_recall.state_quant import permutations_from_statistics


def brute_order(row):
    left = list(range(len(row)))
    out = []
    while left:
        best = left[0]
        for i in left[1:]:
            if row[i] > row[best]:   # strictly greater: the first of equal maxima wins
                best = i
        out.append(best)
        left.remove(best)
    return out


def test_order_direction_and_ties_match_brute_force():
    rng = np.random.default_rng(3)
    # few distinct values, so most rows hold many ties
    mean = rng.integers(0, 6, size=(3, 8, 128)).astype(np.float64) * 0.25
    mean[0, 0] = 1.0                       # all equal: identity order
    mean[0, 1] = np.arange(128)[::-1]      # already descending: identity order
    mean[0, 2] = np.arange(128)            # ascending: reversed order
    stats = {"mean_abs": torch.from_numpy(mean)}
    table = permutations_from_statistics(stats)
    assert table.dtype == torch.uint8 and tuple(table.shape) == (3, 8, 128)
    for layer in range(3):
        state_codec.validate_permutation(table[layer], 8)
        for g in range(8):
            assert table[layer, g].tolist() == brute_order(mean[layer, g].tolist())
    assert table[0, 0].tolist() == list(range(128))
    assert table[0, 1].tolist() == list(range(128))
    assert table[0, 2].tolist() == list(range(127, -1, -1))


def test_accepts_tensor_and_signed_zero_ties():
    mean = torch.zeros(1, 1, 128, dtype=torch.float64)
    mean[0, 0, 1::2] = -0.0                # -0 == +0: still one tie class
    mean[0, 0, 100] = 2.0
    table = permutations_from_statistics(mean)
    assert table[0, 0, 0].item() == 100
    assert table[0, 0, 1:].tolist() == [i for i in range(128) if i != 100]


@pytest.mark.parametrize("bad", [float("nan"), float("inf")])
def test_nonfinite_statistics_raise(bad):
    mean = torch.ones(2, 8, 128, dtype=torch.float64)
    mean[1, 3, 7] = bad
    with pytest.raises(RuntimeError, match="Nonfinite calibration statistics"):
        permutations_from_statistics({"mean_abs": mean})


def test_shape_is_checked():
    with pytest.raises(ValueError, match="mean_abs"):
        permutations_from_statistics(torch.ones(8, 128))

"""Pins the oracle's top-k selection (CPU only).

The selection contract: exact 32-bit order, ties -> lowest position,
ascending output, -1 padding, seq_len <= k selects everything
(csrc/attention/sm70_mla_decode.cu:1187-1212).  The numpy (lexsort) and C
(qsort) restatements are checked against each other and against hand cases.
"""
import numpy as np
import pytest
import torch

from oracle import cref
from oracle import dsa_oracle as O


def test_hand_case():
    s = torch.tensor([[0.5, 3.0, -1.0, 3.0, 2.0, 3.0, float("-inf"), 7.0]])
    sl = torch.tensor([8], dtype=torch.int32)
    # k=3: 7.0 (pos 7), then the 3.0s at the lowest positions 1 and 3
    want = torch.tensor([[1, 3, 7]], dtype=torch.int32)
    assert torch.equal(O.topk_rows(s, sl, 3), want)
    assert torch.equal(cref.topk_rows(s, sl, 3), want)
    # seq_len 5 hides positions >= 5: 3.0@1, 3.0@3, 2.0@4
    sl5 = torch.tensor([5], dtype=torch.int32)
    want5 = torch.tensor([[1, 3, 4]], dtype=torch.int32)
    assert torch.equal(O.topk_rows(s, sl5, 3), want5)
    assert torch.equal(cref.topk_rows(s, sl5, 3), want5)


def test_short_rows_select_all_and_pad():
    s = torch.randn(3, 10)
    sl = torch.tensor([0, 4, 10], dtype=torch.int32)
    got = cref.topk_rows(s, sl, 6)
    assert got[0].tolist() == [-1] * 6
    assert got[1].tolist() == [0, 1, 2, 3, -1, -1]
    assert torch.equal(got, O.topk_rows(s, sl, 6))


def test_negative_zero_below_positive_zero():
    s = torch.tensor([[-0.0, 0.0, -0.0]])
    sl = torch.tensor([3], dtype=torch.int32)
    assert cref.topk_rows(s, sl, 1).tolist() == [[1]]
    assert O.topk_rows(s, sl, 1).tolist() == [[1]]


@pytest.mark.parametrize("seed", range(4))
def test_c_matches_numpy_random(seed):
    g = torch.Generator().manual_seed(seed)
    R, W, K = 6, 5000, 257
    s = torch.randn(R, W, generator=g)
    # heavy ties: quantize half the rows
    s[::2] = torch.round(s[::2] * 4) / 4
    sl = torch.randint(0, W + 50, (R,), generator=g, dtype=torch.int32)
    a = cref.topk_rows(s, sl, K)
    b = O.topk_rows(s, sl, K)
    assert torch.equal(a, b)


def test_selection_property():
    """Brute-force definition: every selected key >= every unselected one,
    and among equal keys at the boundary the selected positions are lowest."""
    g = torch.Generator().manual_seed(7)
    s = torch.round(torch.randn(1, 3000, generator=g) * 3) / 3
    sl = torch.tensor([2900], dtype=torch.int32)
    K = 500
    idx = cref.topk_rows(s, sl, K)[0].numpy()
    assert np.all(np.diff(idx) > 0)
    keys = O.mono_key(s[0, :2900]).numpy()
    sel = np.zeros(2900, bool)
    sel[idx] = True
    kmin_sel = keys[sel].min()
    assert np.all(keys[~sel] <= kmin_sel)
    tie = np.nonzero(keys == kmin_sel)[0]
    assert np.all(sel[tie[: sel[tie].sum()]])  # the selected ties are a prefix


def test_all_equal_row():
    s = torch.full((1, 4096), 1.5)
    sl = torch.tensor([4000], dtype=torch.int32)
    got = cref.topk_rows(s, sl, 2048)
    assert got[0].tolist() == list(range(2048))

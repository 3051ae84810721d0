"""Pin the C oracle's dispatch permutation (oracle/combine_ref.c: oracle_permute) -- CPU only.

The permutation restates src/fastmoe/models/tiny_model.py:108-138 with a stable sort.  Checks that
fail for a plausible mistake (an unstable or reversed tie order, an off-by-one offset, a wrong
token of a slot, a dropped slot):
  * equality with the reference's own torch code path run with ``stable=True`` (argsort,
    arange().repeat_interleave()[order], bincount);
  * closed forms: k = 1 with a permutation of experts is that permutation's inverse; all slots to
    one expert is the identity order; offsets are the exclusive cumsum of the counts;
  * invariants: rev[slot_pos[i]] == i // k for every slot, slot_pos is a permutation of [0, N),
    every expert's rows are contiguous and in ascending slot order;
  * ids outside [0, E) form one bucket after every expert, in slot order.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cref


def _reference_torch(ids: torch.Tensor, E: int):
    """tiny_model.py:108-138 as the reference writes it, with a stable argsort."""
    T, k = ids.shape
    flat = ids.reshape(-1)
    order = torch.argsort(flat, stable=True)
    rev = torch.arange(T).repeat_interleave(k)[order]
    counts = torch.bincount(flat[order], minlength=E)
    return order, rev, counts


@pytest.mark.parametrize("T,k,E,seed", [(64, 2, 8, 0), (200, 8, 256, 1), (33, 3, 5, 2), (1, 4, 3, 3)])
def test_matches_reference_torch_path(T, k, E, seed):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=g)
    ids = torch.topk(logits, min(k, E), dim=-1).indices
    order, rev_t, counts_t = _reference_torch(ids, E)
    counts, offsets, rev, slot_pos, bad = cref.permute(ids.numpy(), E)
    assert bad == 0
    np.testing.assert_array_equal(rev, rev_t.numpy())
    np.testing.assert_array_equal(counts, counts_t.numpy())
    np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]))
    inv = np.empty_like(slot_pos)
    inv[slot_pos] = np.arange(len(slot_pos))
    np.testing.assert_array_equal(inv, order.numpy())


def test_closed_forms():
    perm = np.random.default_rng(5).permutation(16)
    counts, offsets, rev, slot_pos, _ = cref.permute(perm[:, None], 16)
    np.testing.assert_array_equal(slot_pos, perm)                 # expert e holds token argwhere
    np.testing.assert_array_equal(rev, np.argsort(perm))
    assert (counts == 1).all()
    counts, offsets, rev, slot_pos, _ = cref.permute(np.full((10, 3), 2), 4)
    np.testing.assert_array_equal(slot_pos, np.arange(30))        # one expert: identity
    np.testing.assert_array_equal(counts, [0, 0, 30, 0])
    np.testing.assert_array_equal(offsets, [0, 0, 0, 30, 30])


def test_invariants_and_invalid_bucket():
    rng = np.random.default_rng(7)
    ids = rng.integers(-2, 9, size=(50, 4))   # ids -2, -1 and 8 are outside [0, 8)
    E = 8
    counts, offsets, rev, slot_pos, bad = cref.permute(ids, E)
    flat = ids.reshape(-1)
    invalid = (flat < 0) | (flat >= E)
    assert bad == invalid.sum() and offsets[E] == len(flat) - bad
    assert sorted(slot_pos.tolist()) == list(range(len(flat)))
    np.testing.assert_array_equal(rev[slot_pos], np.arange(len(flat)) // 4)
    for e in range(E):
        rows = slot_pos[flat == e]
        np.testing.assert_array_equal(rows, np.arange(offsets[e], offsets[e] + counts[e]))
    np.testing.assert_array_equal(slot_pos[invalid], np.arange(offsets[E], len(flat)))


def _mutant(ids, E, mistake):
    """Python copies of the oracle's counting sort with one planted mistake (CPU only)."""
    T, k = ids.shape
    flat = ids.reshape(-1)
    cnt = np.bincount(flat, minlength=E)
    off = np.concatenate([[0], np.cumsum(cnt)])[:E]
    if mistake == "offset_off_by_one":
        off = off + (np.arange(E) > 0)
    cur = off.copy()
    rev = np.zeros(len(flat), np.int64)
    order = range(len(flat))
    if mistake == "reverse_ties":
        order = reversed(order)
    for i in order:
        pos = cur[flat[i]] % len(flat)
        cur[flat[i]] += 1
        rev[pos] = i // k if mistake != "wrong_token" else i % T
    if mistake == "drop_slot":
        rev[-1] = 0
    return rev


@pytest.mark.parametrize("mistake", ["reverse_ties", "offset_off_by_one", "wrong_token", "drop_slot"])
def test_pinning_rejects_planted_mistakes(mistake):
    ids = torch.topk(torch.randn(40, 6, generator=torch.Generator().manual_seed(9)), 3).indices
    _, rev_t, _ = _reference_torch(ids, 6)
    np.testing.assert_array_equal(_mutant(ids.numpy(), 6, None), rev_t.numpy())
    assert not np.array_equal(_mutant(ids.numpy(), 6, mistake), rev_t.numpy())

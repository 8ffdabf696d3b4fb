"""The prompt-lookup draft rule of qe_decode_lookup (host code; runs without a GPU)."""
import pytest

import qe


@pytest.mark.parametrize("history,ngram,k_max,want", [
    ([1, 2, 3, 4], 3, 4, []),                      # no suffix recurs
    ([1, 2, 3, 9, 1, 2, 3], 3, 4, [9, 1, 2, 3]),   # 3-gram match, continuation up to the end
    ([1, 2, 3, 9, 1, 2, 3], 3, 2, [9, 1]),         # capped at k_max
    ([5, 7, 1, 5, 8, 2, 5], 1, 2, [8, 2]),         # the most recent occurrence with k_max followers
    ([5, 7, 1, 5, 8, 2, 5], 1, 4, [7, 1, 5, 8]),   # ... else the earliest (longest continuation)
    ([4, 2, 3, 7, 8, 3], 3, 2, [7, 8]),            # 3- and 2-grams do not recur: falls back to 1
    ([6, 6, 6], 3, 4, [6]),                        # overlapping repeat; g capped at n - 1
    ([1, 2, 1, 2], 3, 0, []),                      # k_max 0: nothing to draft
    ([7], 3, 4, []),                               # too short
])
def test_lookup_draft(history, ngram, k_max, want):
    assert qe.lookup_draft(history, ngram, k_max) == want


def test_longest_ngram_is_preferred():
    # the 1-gram [3] recurs most recently at index 4 (followed by 5), but the 2-gram [2, 3]
    # recurs at index 1 (followed by 9): the longer match decides
    h = [0, 2, 3, 9, 3, 5, 2, 3]
    assert qe.lookup_draft(h, 2, 1) == [9]
    assert qe.lookup_draft(h, 1, 1) == [5]

"""CPU checks of the speculative-verification host logic.

The oracle restates greedy_sample (main.cu:326-335) and one round of the
verification loop (main_speculative.cu:474-510, bread_step replaced by a
lookup of the target's predictions).  They are pinned here by hand-derived
known answers and, for the argmax, by numpy's first-occurrence argmax; then
the library's bread_spec_accept (no device involved) must agree with the
oracle round on every small case."""
import itertools

import numpy as np
import pytest

import breadv2_amd as B
from oracle import oracle as O

EOS = 2


@pytest.mark.parametrize(
    "pred,draft,total,max_tokens,want",
    [
        # all drafts accepted: the bonus is the prediction after the last draft
        ([5, 6, 7, 9], [5, 6, 7], 1, 100, (3, 9, 5)),
        # first draft rejected: bonus = the first prediction
        ([4, 6, 7, 9], [5, 6, 7], 1, 100, (0, 4, 2)),
        # mismatch at draft 2
        ([5, 6, 8, 9], [5, 6, 7], 1, 100, (2, 8, 4)),
        # the prediction equals a draft but is EOS: not accepted, and no bonus
        ([EOS, 6], [EOS], 1, 100, (0, EOS, 1)),
        # budget spent after one acceptance: no further step, no bonus
        ([5, 6, 7, 9], [5, 6, 7], 9, 10, (1, 5, 10)),
        # budget leaves room for exactly the bonus
        ([5, 6, 7, 9], [5, 6, 7], 6, 10, (3, 9, 10)),
        # no drafts
        ([3], [], 1, 100, (0, 3, 2)),
    ],
)
def test_oracle_round_known_answers(pred, draft, total, max_tokens, want):
    assert O.spec_round(pred, draft, EOS, total, max_tokens) == want


def test_oracle_greedy_pins():
    rng = np.random.default_rng(1)
    for n in (1, 7, 100, 4096):
        for _ in range(20):
            a = rng.integers(-20, 20, n).astype(np.float16)  # many ties
            assert O.greedy_f16(a) == int(np.argmax(a))
    nan, inf = np.float16(np.nan), np.float16(np.inf)
    assert O.greedy_f16(np.array([nan, 5, 9], np.float16)) == 0
    assert O.greedy_f16(np.array([1, nan, 9, nan], np.float16)) == 2
    assert O.greedy_f16(np.array([-inf, -inf], np.float16)) == 0
    assert O.greedy_f16(np.array([1, inf, inf], np.float16)) == 1
    assert O.greedy_f16(np.array([-0.0, 0.0], np.float16)) == 0
    assert O.greedy_f16(np.array([0.0, -0.0], np.float16)) == 0


def test_spec_accept_matches_oracle_exhaustively():
    """Tokens from {0, 1, 2 = EOS}, up to 3 drafts, every budget."""
    n_cases = 0
    for n in range(0, 4):
        for pred in itertools.product(range(3), repeat=n + 1):
            for draft in itertools.product(range(3), repeat=n):
                for left in range(1, n + 3):
                    total, max_tokens = 10, 10 + left
                    a, nx, _ = O.spec_round(pred, draft, EOS, total, max_tokens)
                    assert B.spec_accept(pred, draft, EOS, left) == (a, nx), (pred, draft, left)
                    n_cases += 1
    assert n_cases > 5000


def test_spec_accept_rejects_bad_arguments():
    with pytest.raises(B.BreadError):
        B.spec_accept([1, 2], [1], EOS, 0)

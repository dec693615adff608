"""The greedy check's comparison rule (tests/qwen3_harness.GreedyComparison)
on synthetic logits: a flip at a margin above the bound fails, a flip below
it is recorded (and on the fed-back row both runs continue with the
oracle's token), and logits outside the tolerance fail."""
import pytest
import torch

from qwen3_harness import GreedyComparison

TOL = dict(atol=0.25, rtol=2e-2)


def rows(*tops, vocab=16):
    """Logit rows whose token 0 and 1 lead by the given margins over the rest."""
    out = torch.zeros(len(tops), vocab)
    for r, (a, b) in enumerate(tops):
        out[r, 0], out[r, 1] = a, b
    return out


def test_identical_rows_pass():
    c = GreedyComparison(0.2, TOL)
    assert c.check(0, 0, rows((5.0, 3.0)), rows((5.0, 3.0))) == 0
    assert c.n_rows == 1 and not c.forced and not c.flips


def test_flip_above_the_bound_fails():
    c = GreedyComparison(0.2, TOL)
    with pytest.raises(AssertionError, match="top-2 margin"):
        c.check(3, 1, rows((5.0, 5.02)), rows((5.0, 4.75)))    # oracle margin 0.25 >= 0.2


def test_flip_below_the_bound_feeds_back_the_oracle_token():
    c = GreedyComparison(0.2, TOL)
    assert c.check(2, 1, rows((5.0, 5.05)), rows((5.0, 4.95))) == 0   # margin 0.05: both runs continue with 0
    assert c.forced == [(2, 1)] and c.ties == 1 and len(c.flips) == 1
    # the sequence is still compared afterwards
    with pytest.raises(AssertionError):
        c.check(3, 1, rows((5.0, 5.3)), rows((5.3, 5.0)))       # margin 0.3


def test_flip_on_a_verification_row_is_recorded():
    c = GreedyComparison(0.2, TOL)
    assert c.check(7, 0, rows((5.0, 3.0), (4.0, 4.1)), rows((5.0, 3.0), (4.0, 3.9))) == 0
    assert not c.forced and len(c.flips) == 1 and c.flips[0][:3] == (7, 0, 1)
    with pytest.raises(AssertionError):
        c.check(8, 0, rows((5.0, 3.0), (4.0, 4.5)), rows((5.0, 3.0), (4.5, 4.0)))  # margin 0.5


def test_logits_outside_the_tolerance_fail():
    c = GreedyComparison(0.2, TOL)
    with pytest.raises(AssertionError, match="logits differ"):
        c.check(0, 0, rows((5.0, 3.0)), rows((6.0, 3.0)))

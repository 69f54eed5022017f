"""The adaptive depth policy (q35_mtp_policy_*, the reference's mtpadapt::Tracker,
engine/mtp_adaptive.h:1-254) on known-answer sequences worked out by hand from the rule the
reference states: estimate = emitted / (rounds x cost) over the last 32 rounds, cost 1.90 at
k = 2 and 1.58 at k = 1; demote 2 -> 1 below 0.95 after 16 rounds, abandon 1 -> 0 below 0.90
after 24 rounds; the window clears on a change; no re-promotion; abandonment is sticky.
Host code only (no GPU): runs in the CPU suite through the built library."""
import pytest

from qwen35 import EngineError, MtpPolicy


def _feed(p, k, emitted, n):
    """Feed n rounds; returns (note index 1..n of the first change, change, est at it)."""
    for i in range(1, n + 1):
        ch, est = p.note(k, emitted)
        if ch:
            return i, ch, est
    return None, None, est


def test_zero_accept_demotes_at_16_then_abandons_at_24():
    p = MtpPolicy(2)
    i, ch, est = _feed(p, 2, 1, 40)
    assert (i, ch) == (16, (2, 1, 16)) and est == pytest.approx(1 / 1.9)
    assert p.k == 1
    i, ch, est = _feed(p, 1, 1, 40)
    assert (i, ch) == (24, (1, 0, 24)) and est == pytest.approx(1 / 1.58)
    assert p.k == 0
    for _ in range(100):                       # sticky: nothing walks it back
        assert p.note(2, 3)[0] is None
    assert p.k == 0
    p.close()


def test_break_even_rounds_keep_depth():
    p = MtpPolicy(2)
    assert _feed(p, 2, 2, 200)[0] is None      # 2 / 1.90 = 1.053 >= 0.95
    assert p.k == 2
    q = MtpPolicy(2)
    # alternating 2, 1: 1.5 / 1.9 = 0.789 < 0.95 -> demotes as soon as 16 rounds are seen
    for r in range(1, 17):
        ch, est = q.note(2, 2 if r % 2 else 1)
        assert (ch is None) == (r < 16)
    assert ch == (2, 1, 16) and est == pytest.approx(1.5 / 1.9)
    # at k = 1 a round emitting 2 (one accept) is worth 2 / 1.58 = 1.27 -> stays
    assert _feed(q, 1, 2, 100)[0] is None and q.k == 1


def test_window_evicts_old_rounds():
    """16 rounds emitting 3, then rounds emitting 1: while the window still fills (32 rounds)
    the good rounds hold the estimate up; once it is full the j-th bad round leaves
    (96 - 2j) / 60.8, which first drops below 0.95 at j = 20 (note 36)."""
    p = MtpPolicy(2)
    assert _feed(p, 2, 3, 16)[0] is None
    i, ch, est = _feed(p, 2, 1, 30)
    assert i == 20 and ch == (2, 1, 32) and est == pytest.approx((96 - 40) / 60.8)


def test_start_at_k1_and_costs():
    p = MtpPolicy(1)
    i, ch, _ = _feed(p, 1, 1, 30)
    assert (i, ch) == (24, (1, 0, 24))
    # own cost figures: a round billed at 1.0 step that emits 1 token is exactly break-even
    q = MtpPolicy(2, cost_k1=1.0, cost_k2=1.0)
    assert _feed(q, 2, 1, 100)[0] is None and q.k == 2
    r = MtpPolicy(0)
    assert r.k == 0


def test_bad_arguments():
    with pytest.raises(EngineError, match="start_k is 0, 1 or 2"):
        MtpPolicy(3)
    p = MtpPolicy(2)
    with pytest.raises(EngineError, match="k_round is 0 .. 2"):
        p.note(3, 1)
    with pytest.raises(EngineError, match="emitted >= 0"):
        p.note(2, -1)

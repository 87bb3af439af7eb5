"""Online MTP depth selection (gfxinfer_depth_policy_*), host only."""
from __future__ import annotations

import pytest


def _policy(depth):
    from gfxinfer_amd.runtime import DepthPolicy
    return DepthPolicy(depth)


def test_tries_every_candidate_shallowest_first(gx):
    p = _policy(8)
    seen = []
    for _ in range(6):
        d = p.choose(8)
        seen.append(d)
        p.record(d, 1, 1.0)
    assert seen == [1, 2, 3, 4, 6, 8]
    p.close()


def test_picks_best_tokens_per_millisecond_and_remeasures_the_others(gx):
    p = _policy(31)
    # rate: depth 8 emits 4 tokens in 2 ms (2 tok/ms); deeper is slower per token,
    # shallower emits too few.
    rates = {1: (1, 1.0), 2: (1.5, 1.1), 3: (2, 1.2), 4: (2.5, 1.3), 6: (3, 1.6), 8: (4, 2.0),
             12: (4.2, 2.8), 16: (4.3, 3.6), 24: (4.3, 5.2), 31: (4.3, 6.6)}
    choices = []
    for _ in range(64):
        d = p.choose(31)
        choices.append(d)
        tokens, ms = rates[d]
        p.record(d, int(round(tokens)), ms)
    # the policy's round counter starts at 1: rounds 16, 32, 48, 64 re-measure the
    # other candidates in turn (1, 2, 3, 4 here), every other round takes depth 8
    probes = [i for i in range(10, len(choices)) if (i + 1) % 16 == 0]
    assert [choices[i] for i in probes] == [1, 2, 3, 4]
    assert all(choices[i] == 8 for i in range(10, len(choices)) if i not in probes)
    p.close()


def test_adapts_when_a_depth_gets_better(gx):
    p = _policy(4)
    for d in (1, 2, 3, 4):
        assert p.choose(4) == d
        p.record(d, 1, 1.0 if d == 1 else 2.0)  # depth 1 best at first
    assert p.choose(4) == 1
    # depth 4 now accepts everything, the rest nothing; each other depth is re-measured
    # every third probe (every 48 rounds), and two good rounds lift depth 4 past depth 1
    for _ in range(200):
        d = p.choose(4)
        p.record(d, d + 1 if d == 4 else 1, 2.0 if d != 1 else 1.0)
    assert p.choose(4) == 4
    p.close()


def test_limit_and_validation(gx):
    p = _policy(16)
    assert p.choose(1) == 1
    assert p.choose(5) in (1, 2, 3, 4)  # candidates within the limit only
    from gfxinfer_amd import GfxinferError
    with pytest.raises(GfxinferError):
        p.record(4, 6, 1.0)   # more tokens than depth + 1
    with pytest.raises(GfxinferError):
        p.record(4, 1, 0.0)   # no time
    p.close()
    with pytest.raises(GfxinferError):
        _policy(0)
    with pytest.raises(GfxinferError):
        _policy(32)
    q = _policy(5)            # a maximum that is not a listed depth is a candidate too
    seen = []
    for _ in range(5):
        d = q.choose(5)
        seen.append(d)
        q.record(d, 1, 1.0)
    assert seen == [1, 2, 3, 4, 5]
    q.close()

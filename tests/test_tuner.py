"""The autotuner's UCB1 bandit, pinned (host only, no GPU).

The engine's bandit (seeml_hip_ucb1_run over the C-ABI) against the
reference's own Ucb1Bandit (compiler/backend/tuner/bandit.cc, compiled into
oracle/_ref from the reference sources): the same reward sequence must give
the same selections, pull counts, means (bit for bit) and best arm. Then the
reference's tuner suite (test/compiler/backend/tuner_test.cc:67-145) is
restated against the engine's bandit: every arm once before exploiting,
convergence on the best arm, all-negative rewards, and the injected-reward
autotune that finds the fastest candidate."""
import ctypes as C
import math

import numpy as np
import pytest

from seeml_amd import _lib

REWARD = C.CFUNCTYPE(C.c_double, C.c_void_p, C.c_uint64)


def run_engine(arms, trials, fn, exploration=1.0):
    budget = max(trials, arms)
    picks = (C.c_uint64 * budget)()
    pulls = (C.c_uint64 * arms)()
    means = (C.c_double * arms)()
    best = C.c_uint64()
    cb = REWARD(lambda ctx, arm: fn(arm))
    rc = _lib.lib().seeml_hip_ucb1_run(arms, exploration, trials, C.cast(cb, C.c_void_p), None,
                                       C.addressof(picks), C.addressof(pulls),
                                       C.addressof(means), C.addressof(best))
    assert rc == 0
    return list(picks), list(pulls), np.array(means, np.float64), best.value


def run_ref(ref, arms, trials, fn, exploration=1.0):
    budget = max(trials, arms)
    picks = (C.c_uint64 * budget)()
    pulls = (C.c_uint64 * arms)()
    means = (C.c_double * arms)()
    best = C.c_uint64()
    cb = REWARD(lambda ctx, arm: fn(arm))
    ref.ucb1_run(arms, exploration, trials, C.cast(cb, C.c_void_p).value, None,
                 C.addressof(picks), C.addressof(pulls), C.addressof(means), C.addressof(best))
    return list(picks), list(pulls), np.array(means, np.float64), best.value


def _reward_models():
    """Deterministic reward sources of several kinds: fixed per arm, ties,
    all negative, and pull-dependent noise (a fixed per-(arm, pull) table)."""
    rng = np.random.default_rng(2024)
    models = []
    for arms in (1, 2, 3, 7, 13):
        base = rng.uniform(0.1, 1.0, arms)
        models.append((f"fixed{arms}", arms, lambda a, b=base: float(b[a])))
        table = rng.normal(0.5, 0.2, (arms, 512))
        count = [0] * arms

        def noisy(a, t=table, c=count):
            v = float(t[a, c[a] % 512])
            c[a] += 1
            return v
        models.append((f"noisy{arms}", arms, noisy))
    models.append(("ties", 4, lambda a: 0.5 if a in (1, 3) else 0.25))
    models.append(("negative", 3, lambda a: (-10.0, -5.0, -7.5)[a]))
    models.append(("zero", 3, lambda a: 0.0))
    return models


@pytest.mark.parametrize("exploration", [1.0, math.sqrt(2) / 2, 2.0])
@pytest.mark.parametrize("trials", [0, 5, 64, 300])
def test_engine_bandit_equals_reference_bandit(ref, exploration, trials):
    for name, arms, _ in _reward_models():
        # each side gets a fresh copy of the reward source (the noisy ones
        # are stateful)
        fn_e = dict((n, f) for n, _, f in _reward_models())[name]
        fn_r = dict((n, f) for n, _, f in _reward_models())[name]
        e = run_engine(arms, trials, fn_e, exploration)
        r = run_ref(ref, arms, trials, fn_r, exploration)
        assert e[0] == r[0], (name, "selection sequence")
        assert e[1] == r[1], (name, "pulls")
        assert np.array_equal(e[2].view(np.uint64), r[2].view(np.uint64)), (name, "means")
        assert e[3] == r[3], (name, "best arm")


def test_pulls_every_arm_once_before_exploiting():
    # tuner_test.cc:67-75
    picks, pulls, _, _ = run_engine(3, 3, lambda a: 1.0)
    assert picks == [0, 1, 2]
    assert sum(pulls) == 3


def test_converges_on_the_best_arm():
    # tuner_test.cc:77-91
    reward = [0.2, 0.9, 0.4]
    _, pulls, means, best = run_engine(3, 200, lambda a: reward[a])
    assert best == 1
    assert pulls[1] > 100 and pulls[0] > 1 and pulls[2] > 1
    assert abs(means[1] - 0.9) <= 1e-9


def test_selects_argmax_when_every_reward_is_negative():
    # tuner_test.cc:93-105: after pulling arm 0 (-10) and arm 1 (-5), the
    # next selection and the best arm are arm 1
    picks, _, _, best = run_engine(2, 3, lambda a: (-10.0, -5.0)[a])
    assert picks[:2] == [0, 1] and picks[2] == 1
    assert best == 1


def test_injected_reward_autotune_finds_the_fastest_candidate():
    # tuner_test.cc:130-145: 7 candidates (the halve/double neighbourhood),
    # reward 10 for the last one, 1 otherwise, budget 8 per candidate
    n = 7
    _, pulls, _, best = run_engine(n, n * 8, lambda a: 10.0 if a == n - 1 else 1.0)
    assert best == n - 1
    assert all(p > 0 for p in pulls)


def test_budget_is_raised_to_cover_every_arm():
    # autotuner.cc:66-71: the budget is at least the number of candidates
    picks, pulls, _, _ = run_engine(5, 2, lambda a: float(a))
    assert len(picks) == 5 and all(p == 1 for p in pulls)

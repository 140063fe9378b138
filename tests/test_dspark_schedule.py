"""The adaptive prefix scheduler (snowllm_amd.dspark_schedule) on the CPU: the scenarios and
expected results of the reference's own tests (tests/test_dspark_schedule.py), and a brute-force
check of the capacity search and of the prefixes it hands out."""
import itertools
import random

import pytest

from snowllm_amd import dspark_schedule as S


def test_greedy_capacity_walk_on_random_confidences():
    """Before any history the capacity grows while expected tokens per second improve
    (tests/test_dspark_schedule.py:15-29)."""
    rng = random.Random(12)

    def cost(rows):
        return .01 + .001 * rows ** 1.5
    for _ in range(100):
        confidence = [[rng.random() for _ in range(5)] for _ in range(3)]
        limits = [rng.randrange(6) for _ in range(3)]
        ranked = S.ranked_prefixes(confidence, limits)
        expected, best, count = 3.0, 3 / cost(3), 0
        for survival, _, _ in ranked:
            expected += survival
            rate = expected / cost(4 + count)
            if rate <= best:
                break
            best, count = rate, count + 1
        got = S.PrefixScheduler(256).choose([0, 1, 2], confidence, limits, cost)
        assert got == S.prefix_lengths(ranked, count, 3)


def test_capacity_from_two_steps_back_lengths_from_now():
    """tests/test_dspark_schedule.py:31-39."""
    sched = S.PrefixScheduler(256)
    table = {2: 1., 3: 1.3, 4: 1.5, 5: 2., 6: 3.}
    sched.choose([0, 1], [[.99, .99], [.01, .01]], [2, 2], table.__getitem__)
    sched.choose([0, 1], [[.01] * 2] * 2, [2, 2], table.__getitem__)
    assert sched.choose([0, 1], [[.01, .01], [.99, .99]], [2, 2], table.__getitem__) == [0, 2]


def test_cost_cliff_found_only_with_history():
    """tests/test_dspark_schedule.py:41-47: the early stop misses a cheaper larger step; the
    historical full search finds it; a new cohort starts over."""
    table = {1: 1., 2: 2., 3: 1.2}
    sched = S.PrefixScheduler(256)
    assert sched.choose([0], [[.8, 1.]], [2], table.__getitem__) == [0]
    assert sched.choose([0], [[.8, 1.]], [2], table.__getitem__) == [0]
    assert sched.choose([0], [[.01, .01]], [2], table.__getitem__) == [2]
    assert sched.choose([1], [[.8, 1.]], [2], table.__getitem__) == [0]


def test_row_cap_ties_and_zero_confidence():
    """tests/test_dspark_schedule.py:49-56."""
    sched = S.PrefixScheduler(5)
    assert sched.choose([0, 1], [[1.] * 5] * 2, [1, 5], lambda _: 1.) == [1, 2]
    sched.reset()
    assert sched.choose([0], [[0., 1.]], [2], lambda _: 1.) == [0]
    sched.reset()
    assert sched.choose([0], [[1.] * 5], [0], lambda _: 1.) == [0]


def test_planning_leaves_history_alone():
    sched = S.PrefixScheduler(256)
    for _ in range(3):
        sched.choose([0], [[.9]], [1], lambda _: 1., remember=False)
    assert len(sched.history) == 0
    sched.choose([0], [[.9]], [1], lambda _: 1.)
    assert len(sched.history) == 1


def test_step_cost_graph_only_at_its_bucket():
    """tests/test_dspark_schedule.py:66-72."""
    cost = S.StepCost({2: 2., 4: 4., 6: 6.}, {4: .5}, .1)
    assert cost(4) == pytest.approx(.6)
    assert cost(3) == pytest.approx(3.1)
    assert cost(5) == pytest.approx(5.1)
    with pytest.raises(ValueError):
        cost(7)
    for bad in (({}, {}, 0.), ({1: 0.}, {}, 0.), ({1: 1.}, {2: float("inf")}, 0.),
                ({1: 1.}, {}, -1.), ({1: 1.}, {}, float("nan"))):
        with pytest.raises(ValueError):
            S.StepCost(*bad)


@pytest.mark.parametrize("value", [float("nan"), float("inf"), -.1, 1.1])
def test_invalid_confidence(value):
    with pytest.raises(ValueError):
        S.ranked_prefixes([[value]], [1])


def test_against_brute_force():
    """The full search picks the k that maximises expected tokens / cost over all k; the
    candidates it takes are whole prefixes of each request; survivals are the running
    products."""
    rng = random.Random(3)
    for _ in range(200):
        n = rng.randrange(1, 4)
        confidence = [[rng.choice([rng.random(), 1.0, 0.5]) for _ in range(4)] for _ in range(n)]
        limits = [rng.randrange(5) for _ in range(n)]
        slope = rng.random()

        def cost(rows):
            return 1.0 + slope * rows + (0.7 if rows % 3 == 0 else 0.0)
        ranked = S.ranked_prefixes(confidence, limits)
        for survival, r, j in ranked:
            prod = 1.0
            for s in confidence[r][:j + 1]:
                prod *= s
            assert survival == prod
        row_limit = n + rng.randrange(0, 9)
        k = S.best_capacity(ranked, n, row_limit, cost, early_stop=False)
        rates = [(n + sum(s for s, _, _ in ranked[:i])) / cost(n + i)
                 for i in range(min(len(ranked), row_limit - n) + 1)]
        assert rates[k] == max(rates) and k == rates.index(max(rates))
        lengths = S.prefix_lengths(ranked, k, n)
        taken = {(r, j) for _, r, j in ranked[:k]}
        assert taken == {(r, j) for r in range(n) for j in range(lengths[r])}
        for r in range(n):
            assert lengths[r] <= limits[r]
    assert list(itertools.islice(S.ranked_prefixes([[.5, .5]], [2]), 2)) == [(.5, 0, 0),
                                                                        (.25, 0, 1)]


def test_even_lengths_match_the_reference_decode_shapes():
    """Rows per request of a profiled batch step: the spread of the reference's decode shapes
    (snowllm/engine/spec_decode.py:149-156: (q + 1,) * rem + (q,) * (n - rem))."""
    from snowllm_amd.dspark_schedule import even_lengths
    assert even_lengths(9, 1) == [9]
    assert even_lengths(36, 4) == [9, 9, 9, 9]
    assert even_lengths(10, 4) == [3, 3, 2, 2]
    assert even_lengths(4, 4) == [1, 1, 1, 1]
    for total in range(3, 80):
        for n in range(1, min(total, 8) + 1):
            got = even_lengths(total, n)
            assert sum(got) == total and len(got) == n and max(got) - min(got) <= 1
            assert got == sorted(got, reverse=True)

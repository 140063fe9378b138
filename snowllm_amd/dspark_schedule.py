# SPDX-License-Identifier: Apache-2.0
# The function names, arguments, results, error texts and the steps of the algorithm here follow
# snowllm/engine/dspark_schedule.py (SPDX-FileCopyrightText: Copyright contributors to the
# SnowLLM project), which this module keeps so that the reference's callers choose the same
# prefixes with it.
"""Adaptive verify-prefix scheduling for DSpark drafts (snowllm/engine/dspark_schedule.py:7-85,
used by snowllm/engine/spec_decode.py:143-166), with the same functions, arguments, results and
errors, on step costs measured on this build's verify step (profile_step_costs).

Each request r offers up to limits[r] drafted tokens with per-token confidences c[r][j]; the
chance that the prefix up to j survives verification is prod_{i <= j} c[r][i]. Verifying k of
the drafted tokens beyond the one row every request always verifies yields
requests + (the k largest survivals) tokens in expectation at cost(requests + k); the scheduler
picks the k with the best expected tokens per second and hands out the k best prefix positions.
The capacity k is searched on the confidences of two steps back once two steps of one cohort
are remembered (so the search does not look at the proposal it is scheduling), and on the
current ones, stopping at the first step that does not improve, before that. The prefix lengths
always come from the current confidences.
"""
import itertools
import math
import statistics
import time
from collections import deque


def _check_confidence(score):
    if not (math.isfinite(score) and 0.0 <= score <= 1.0):
        raise ValueError(f"invalid DSpark confidence: {score}")


def ranked_prefixes(confidence, limits):
    """[(survival, request, position)] of every prefix position with a positive survival,
    best first; equal survivals go by request, then position."""
    out = []
    for r, (scores, limit) in enumerate(zip(confidence, limits)):
        head = list(scores[:limit])
        for j, survival in enumerate(itertools.accumulate(head, lambda acc, s: acc * s,
                                                          initial=1.0)):
            if j == 0:
                continue                      # the empty prefix
            _check_confidence(head[j - 1])
            if survival <= 0.0:
                break
            out.append((survival, r, j - 1))
    out.sort(key=lambda c: (-c[0], c[1], c[2]))
    return out


def prefix_lengths(candidates, count, requests):
    """Drafted tokens to verify per request when the best `count` candidates are taken."""
    lengths = [0] * requests
    for _, r, j in candidates[:count]:
        lengths[r] = max(lengths[r], j + 1)
    return lengths


def best_capacity(candidates, requests, row_limit, cost, *, early_stop):
    """The number of candidates k (rows beyond one per request, at most row_limit - requests)
    that maximises expected tokens / cost(requests + k)."""
    expected = float(requests)
    best_rate, best_k = expected / cost(requests), 0
    for k, (survival, _, _) in enumerate(candidates[:max(0, row_limit - requests)], start=1):
        expected += survival
        rate = expected / cost(requests + k)
        if rate > best_rate:
            best_rate, best_k = rate, k
        elif early_stop:
            break
    return best_k


class PrefixScheduler:
    """Chooses how many drafted tokens of each request the next verify step checks."""

    def __init__(self, row_limit):
        self.row_limit = row_limit
        self.history = deque(maxlen=2)
        self.cohort = ()

    def reset(self):
        self.cohort = ()
        self.history.clear()

    def choose(self, cohort, confidence, limits, cost, *, remember=True):
        cohort = tuple(cohort)
        if cohort != self.cohort:             # a new set of requests: forget the history
            self.reset()
            self.cohort = cohort
        n = len(cohort)
        current = ranked_prefixes(confidence, limits)
        if len(self.history) == 2:
            k = best_capacity(ranked_prefixes(self.history[0], limits), n,
                              max(n, self.row_limit), cost, early_stop=False)
        else:
            k = best_capacity(current, n, max(n, self.row_limit), cost, early_stop=True)
        if remember:
            self.history.append(tuple(tuple(row) for row in confidence))
        return prefix_lengths(current, k, n)


class StepCost:
    """Seconds of one verify step of `rows` query rows plus the draft's time: a profiled
    graph time when one was captured at exactly that row count, else the eager time,
    interpolated linearly between profiled row counts."""

    def __init__(self, eager, graphs, draft):
        times = list(eager.values()) + list(graphs.values())
        if not eager or not math.isfinite(draft) or draft < 0 or \
                any(not math.isfinite(t) or t <= 0 for t in times):
            raise ValueError("DSpark profiling needs positive, finite step times")
        self.eager, self.graphs, self.draft = dict(eager), dict(graphs), draft
        self.points = sorted(self.eager)

    def __call__(self, rows):
        if rows in self.graphs:
            return self.draft + self.graphs[rows]
        if rows in self.eager:
            return self.draft + self.eager[rows]
        for lo, hi in zip(self.points, self.points[1:]):
            if lo < rows < hi:
                return self.draft + (self.eager[lo] * (hi - rows)
                                     + self.eager[hi] * (rows - lo)) / (hi - lo)
        raise ValueError(f"unprofiled DSpark batch size: {rows}")


def _median_seconds(run, reps):
    import torch
    samples = []
    for _ in range(reps):
        torch.cuda.synchronize()
        start = time.perf_counter()
        run()
        torch.cuda.synchronize()
        samples.append(time.perf_counter() - start)
    return statistics.median(samples)


def share_weights(source):
    """A VerifyModel weights installer that reuses `source`'s weights (no copy)."""
    def install(model):
        for name in ("layers", "embed", "lm_head", "final_norm", "head_wt", "head_fmt",
                     "embed_q4k"):
            setattr(model, name, getattr(source, name))
    return install


def even_lengths(total, requests):
    """Rows per request of a step of `total` rows over `requests` requests, spread as evenly as
    the reference's profiled decode shapes spread them (snowllm/engine/spec_decode.py:149-156)."""
    q, rem = divmod(total, requests)
    return [q + 1] * rem + [q] * (requests - rem)


def profile_step_costs(source, rows, *, requests=1, draft_seconds=0.0, seed=0, reps=5,
                       graph_reps=20):
    """StepCost of this build's verify step (snowllm_amd.verify.VerifyModel.forward) on the
    weights of the VerifyModel `source`, for `requests` sequences of n query rows in all (spread
    by even_lengths) at the source's context, for each n in `rows`: the eager time and the time
    of one replay of the step captured as a HIP graph (the reference's
    snowllm/engine/dspark_profile.py measures its engine the same two ways, one cost table per
    request count)."""
    import torch
    from dataclasses import replace
    from .verify import VerifyModel
    eager, graphs = {}, {}
    for n in rows:
        if n < requests:
            raise ValueError(f"{n} rows cannot hold {requests} requests")
        lengths = even_lengths(n, requests)
        T = max(lengths)
        m = VerifyModel(replace(source.cfg, block=T, tree_parents=()), seed=seed,
                        weights=share_weights(source), batch=requests)
        ids = (torch.arange(requests * T) * 7 + 1).view(requests, T)
        if requests == 1:
            m.set_block(ids[0])
        else:
            m.set_batch(ids, [source.cfg.context] * requests, lengths)
        m.forward()
        eager[n] = _median_seconds(m.forward, reps)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            m.forward()
            with torch.cuda.graph(graph, stream=stream):
                m.forward()
        torch.cuda.current_stream().wait_stream(stream)

        def replays():
            for _ in range(graph_reps):
                graph.replay()
        graphs[n] = _median_seconds(replays, reps) / graph_reps
        del graph, m
        torch.cuda.synchronize()
    return StepCost(eager, graphs, draft_seconds)

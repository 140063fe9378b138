"""Host logic of the sampler mirror (snowllm_amd/sampler.py): the penalty lists a batch of
verify rows stages, against the reference tests' own per-row construction
(tests/test_runtime_buffers.py:108-143). CPU only: nothing is launched."""
from collections import Counter
from types import SimpleNamespace

import pytest

from snowllm_amd.errors import SnowLLMError
from snowllm_amd.sampler import SamplingParams, penalty_plan


def _per_row(rows):
    """tests/test_runtime_buffers.py:121-126: every row on its own -- the counts of the
    request's output plus its drafts before the row, over sorted(prompt | counted ids)."""
    depths, out = {}, {}
    for i, r in enumerate(rows):
        depth = depths.get(id(r), 0)
        depths[id(r)] = depth + 1
        if not r.params.penalized():
            continue
        counts = Counter(r.out)
        counts.update(r.drafts[:depth])
        ids = sorted(set(r.prompt) | counts.keys())
        out[i] = {t: counts.get(t, 0) for t in ids}
    return out


def test_shared_ids_match_independent_rows():
    a = SimpleNamespace(params=SamplingParams(presence_penalty=.4, frequency_penalty=.2,
                                              repetition_penalty=1.3),
                        prompt=[1, 2, 1], out=[3, 3], drafts=[4, 1, 5])
    b = SimpleNamespace(params=SamplingParams(presence_penalty=-.2, frequency_penalty=.1,
                                              repetition_penalty=.9),
                        prompt=[6, 7], out=[], drafts=[8])
    c = SimpleNamespace(params=SamplingParams(), prompt=[9], out=[9], drafts=[9])
    rows = [a, b, a, b, c, a, a]
    plan = penalty_plan(rows, 17, 2)
    got = {i: dict(zip(ids, counts)) for i, _, ids, counts, _ in plan}
    assert got == _per_row(rows)
    assert sorted(got) == [0, 1, 2, 3, 5, 6]
    # one shared id list per request, in sorted-then-first-occurrence order
    lists = {key: ids for _, key, ids, _, _ in plan}
    assert sorted(map(tuple, lists.values())) == [(1, 2, 3, 4, 5), (6, 7, 8)]


def test_future_drafts_are_not_seen():
    # tests/test_runtime_buffers.py:136-143: row d sees the drafts before d only
    row = SimpleNamespace(params=SamplingParams(repetition_penalty=2), prompt=[1], out=[],
                          drafts=[2, 3])
    plan = penalty_plan([row] * 3, 9, 1)
    seen = [dict(zip(ids, counts)) for _, _, ids, counts, _ in plan]
    assert seen == [{1: 0}, {1: 0, 2: 1}, {1: 0, 2: 1, 3: 1}]


def test_capacity_is_checked_before_anything():
    # tests/test_runtime_buffers.py:145-152
    row = SimpleNamespace(params=SamplingParams(repetition_penalty=1.1), prompt=list(range(9)),
                          out=[], drafts=[])
    with pytest.raises(SnowLLMError):
        penalty_plan([row], 8, 1)
    a = SimpleNamespace(params=SamplingParams(presence_penalty=1.), prompt=[1], out=[], drafts=[])
    b = SimpleNamespace(params=SamplingParams(presence_penalty=1.), prompt=[2], out=[], drafts=[])
    with pytest.raises(SnowLLMError):
        penalty_plan([a, b], 8, 1)


def test_sampling_params_kernel_forms():
    # snowllm/engine/request.py:25-35
    from snowllm_amd.sampling import SAMPLING_MAX_K
    assert SamplingParams(temperature=0).kernel_top_k() == 1
    assert SamplingParams(top_k=0).kernel_top_k() == SAMPLING_MAX_K
    assert SamplingParams(top_k=2000).kernel_top_k() == 2000
    assert SamplingParams(temperature=-1).kernel_temperature() == 1.0
    assert not SamplingParams().penalized()
    assert SamplingParams(repetition_penalty=1.1).penalized()

# SPDX-License-Identifier: Apache-2.0
# The class and method names, the request parameters, the staging rules of the penalty ids and
# counts, and the error texts here follow snowllm/engine/sampler.py and snowllm/engine/request.py
# (SPDX-FileCopyrightText: Copyright contributors to the SnowLLM project), which this module
# keeps so that the reference's verify drivers can use it unchanged.
"""The sampler of the verify step: penalties, no-repeat-n-gram masks, then greedy argmax,
top-k/top-p sampling or the probability lists of rejection sampling
(snowllm/engine/sampler.py:17-220, parameters snowllm/engine/request.py:12-35).

Per-row parameters and the penalty ids/counts are staged through pinned host buffers that are
reserved once and reused: a write waits for the previous copy out of the same buffer (an event)
and then copies asynchronously, so a step allocates nothing on the device.
"""
from collections import Counter
from dataclasses import dataclass

import numpy as np
import torch

from .errors import SnowLLMError
from .ngram import banned_ngram_tokens
from .sampling import (SAMPLING_MAX_K, argmax, penalties, probabilities, sample,
                       sample_workspace_bytes)


@dataclass
class SamplingParams:
    """Per-request sampling parameters (snowllm/engine/request.py:12-35)."""
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0
    max_new_tokens: int = 32
    stop_token_ids: tuple = ()
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    repetition_penalty: float = 1.0
    no_repeat_ngram_size: int = 0

    def penalized(self) -> bool:
        return bool(self.presence_penalty or self.frequency_penalty
                    or self.repetition_penalty != 1.0)

    def kernel_top_k(self) -> int:
        if self.temperature <= 0.0:
            return 1
        return self.top_k if 0 < self.top_k <= SAMPLING_MAX_K else SAMPLING_MAX_K

    def kernel_temperature(self) -> float:
        return self.temperature if self.temperature > 0.0 else 1.0


class Staged:
    """A pinned host buffer and its device copy, reused for every write: a write waits until
    the previous copy out of the host buffer has run, fills it and copies asynchronously."""

    def __init__(self, n, dtype):
        self.host = torch.empty(max(int(n), 1), dtype=dtype, pin_memory=True)
        self.device = torch.empty(max(int(n), 1), dtype=dtype, device="cuda")
        self.done = torch.cuda.Event()
        self.pending = False

    def write(self, values, offset=0):
        """values: a sequence or a numpy array; returns the device view of what was written."""
        n = len(values)
        if offset + n > self.host.numel():
            raise SnowLLMError("staging capacity exceeded")
        if self.pending:
            self.done.synchronize()
            self.pending = False
        if n:
            self.host.numpy()[offset:offset + n] = values
            self.device[offset:offset + n].copy_(self.host[offset:offset + n], non_blocking=True)
            self.done.record()
            self.pending = True
        return self.device[offset:offset + n]


def penalty_plan(rows, limit, max_requests):
    """The penalty lists of a batch of logit rows (snowllm/engine/sampler.py:187-220): for each
    penalised row i, (i, request key, ids, counts, params). A request's ids are its prompt and
    output ids, sorted, followed by its drafts in order of first occurrence; its row at verify
    depth d sees the first ids up to the d-th draft, with counts over its output plus its
    first d drafts (a row never sees its own or later drafts). Every list is checked before
    anything is written."""
    groups = {}
    for i, r in enumerate(rows):
        if r.params.penalized():
            groups.setdefault(id(r), (r, []))[1].append(i)
    if len(groups) > max_requests:
        raise SnowLLMError('penalty request capacity exceeded')
    plan = []
    for key, (r, indices) in groups.items():
        counts = Counter(r.out)
        ids = sorted(set(r.prompt) | set(counts))
        known = set(ids)
        ends = [len(ids)]
        for token in r.drafts[:len(indices) - 1]:
            if token not in known:
                known.add(token)
                ids.append(token)
            ends.append(len(ids))
        if len(ids) > limit:
            raise SnowLLMError('penalty token capacity exceeded')
        for depth, i in enumerate(indices):
            if 0 < depth <= len(r.drafts):
                counts[r.drafts[depth - 1]] += 1
            n = ends[min(depth, len(ends) - 1)]
            plan.append((i, key, ids, [counts.get(t, 0) for t in ids[:n]], r.params))
    return plan


class Sampler:
    """Sampling over a batch of logit rows, each row belonging to a request (a row object with
    .params, and for penalties/n-grams .prompt, .out, .drafts). Several rows of one request
    are its verify rows: row d of the request sees its first d drafts as already emitted."""

    def __init__(self, stop_token_ids=frozenset(), seed=None):
        self.stop_token_ids = stop_token_ids
        self.rng = torch.Generator(device="cuda")
        if seed is not None:
            self.rng.manual_seed(seed)
        self._rows = 0

    def reserve(self, rows, vocab, *, max_tokens=None, max_requests=None):
        """Device and staging buffers for up to `rows` logit rows of width `vocab`, penalty
        lists of up to `max_tokens` ids for up to `max_requests` requests."""
        limit = vocab if max_tokens is None else min(vocab, max_tokens)
        requests = rows if max_requests is None else max_requests
        if not 0 < requests <= rows or limit <= 0:
            raise SnowLLMError('invalid penalty buffer dimensions')
        self._rows, self._vocab = rows, vocab
        self._width = min(vocab, SAMPLING_MAX_K)
        self.workspace = torch.empty(sample_workspace_bytes(rows, vocab, self._width),
                                     dtype=torch.uint8, device="cuda")
        self.uniforms = torch.empty(rows, dtype=torch.float32, device="cuda")
        self.top_k = Staged(rows, torch.int32)
        self.top_p = Staged(rows, torch.float32)
        self.temperature = Staged(rows, torch.float32)
        self._penalty_requests, self._penalty_limit = requests, limit
        self.penalty_ids = Staged(requests * limit, torch.int64)
        self.penalty_counts = Staged(rows * limit, torch.int32)
        self.ngram_ids = Staged(rows * limit, torch.int64)

    # -- parameters ------------------------------------------------------------------------
    def _parameters(self, rows, vocab):
        ks = [r.params.kernel_top_k() for r in rows]
        top_k = self.top_k.write(np.asarray(ks, dtype=np.int32))
        top_p = self.top_p.write(np.asarray([r.params.top_p for r in rows], dtype=np.float32))
        temp = self.temperature.write(np.asarray([r.params.kernel_temperature() for r in rows],
                                                 dtype=np.float32))
        return top_k, top_p, temp, min(max(ks), vocab)

    def _uniform(self, n):
        return torch.rand(n, generator=self.rng, out=self.uniforms[:n])

    def prepare(self, logits, rows):
        """Penalties, then the no-repeat-n-gram masks, applied to the logits in place
        (snowllm/engine/sampler.py:87-90, 108-111)."""
        if len(rows) > self._rows:
            raise SnowLLMError('penalty row capacity exceeded')
        if any(r.params.penalized() for r in rows):
            self._penalize(logits, rows)
        if any(r.params.no_repeat_ngram_size for r in rows):
            self._mask_ngrams(logits, rows)

    # -- sampling (sampler.py:84-104) ------------------------------------------------------
    def sample(self, logits, rows, *, out=None):
        self.prepare(logits, rows)
        if all(r.params.temperature <= 0 for r in rows):
            return argmax(logits, out=out)
        top_k, top_p, temp, width = self._parameters(rows, logits.shape[1])
        uniform = self._uniform(len(rows))
        return sample(logits, top_k, top_p, temp, width, uniform=uniform, out=out,
                      workspace=self.workspace)

    def probabilities(self, logits, rows, out, indices, *, prepared=False):
        """Probability lists of width min(largest top-k, V) per row (sampler.py:106-117):
        values/ids are views of `out`/`indices`. prepared: the penalties and n-gram masks are
        already on the logits."""
        if not prepared:
            self.prepare(logits, rows)
        top_k, top_p, temp, width = self._parameters(rows, logits.shape[1])
        n = len(rows) * width
        values, ids = out[:n].view(-1, width), indices[:n].view(-1, width)
        probabilities(logits, top_k, top_p, temp, width, values, ids, self.workspace)
        return values, ids

    # -- penalties (sampler.py:146-220) ----------------------------------------------------
    def _penalize(self, logits, rows):
        plan = penalty_plan(rows, self._penalty_limit, self._penalty_requests)
        if not plan:
            return
        # requests' ids and rows' counts packed back to back, one staging copy each
        id_lists, seen, id_at, count_at, launches = [], {}, 0, 0, []
        for i, key, ids, counts, params in plan:
            if key not in seen:
                seen[key] = id_at
                id_lists.append(ids)
                id_at += len(ids)
            launches.append((i, seen[key], count_at, len(counts), params))
            count_at += len(counts)
        d_ids = self.penalty_ids.write(np.asarray([t for ids in id_lists for t in ids],
                                                  dtype=np.int64))
        d_counts = self.penalty_counts.write(np.asarray([c for _, _, _, cs, _ in plan for c in cs],
                                                        dtype=np.int32))
        for i, ia, ca, n, p in launches:
            penalties(logits[i], d_ids[ia:ia + n], d_counts[ca:ca + n], p.presence_penalty,
                      p.frequency_penalty, p.repetition_penalty)

    def _mask_ngrams(self, logits, rows):
        L = self._penalty_limit
        depth_of = Counter()
        staged, fills = [], []
        for row, r in enumerate(rows):
            size = r.params.no_repeat_ngram_size
            depth = depth_of[id(r)]
            depth_of[id(r)] += 1
            if not size:
                continue
            banned = banned_ngram_tokens(list(r.prompt) + list(r.out) + list(r.drafts[:depth]),
                                         size)
            if not banned:
                continue
            if len(banned) > L:
                raise SnowLLMError('n-gram token capacity exceeded')
            fills.append((row, len(staged), len(banned)))
            staged.extend(banned)
        if not fills:
            return
        d = self.ngram_ids.write(np.asarray(staged, dtype=np.int64))
        for row, at, n in fills:
            logits[row].index_fill_(0, d[at:at + n], float('-inf'))

    # -- emission (sampler.py:226-237) -----------------------------------------------------
    def append(self, r, tok):
        r.out.append(tok)
        if tok in self.stop_token_ids or tok in r.params.stop_token_ids:
            r.done, r.finish_reason = True, "stop"
        elif len(r.out) >= r.params.max_new_tokens:
            r.done, r.finish_reason = True, "length"

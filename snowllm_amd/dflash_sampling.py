"""The DFlash/DSpark verify-side acceptance and its dispatch (snowllm/engine/dflash_sampling.py:
8-69), on this build's kernels.

Per verify step, for a batch of requests each holding k drafts (block width k + 1), after the
sampler's penalties and no-repeat-n-gram masks on the logits (snowllm/engine/sampler.py:
84-117):

- every request greedy (temperature <= 0): argmax of every row, then 1 + leading matches
  (snowllm/engine/dflash_sampling.py:56-59, where Sampler.sample takes ops.argmax when every
  row is greedy) -- one launch (snowverify_accept_greedy);
- otherwise target probabilities with each request's sampling parameters, then rejection
  sampling against the draft's 16-candidate proposal, read at the request's stable slot
  (snowllm/engine/dflash_sampling.py:60-69): `valid` is 1 when the request's drafts are the
  proposal remembered for its slot, uniforms are drawn as [count, width]. When every request
  keeps the whole vocabulary (top-k covering it, top-p 1) this runs straight from the logits
  without materialising probabilities (snowverify_accept_reject, three launches); otherwise
  the sampler's probability lists (snowllm_sampling_softmax + _topk_topp, any top-k and
  top-p) and snowllm_draft_reject.

Per-step parameters go through pinned staging buffers reserved once (sampler.Staged).
"""
from dataclasses import dataclass, field

import numpy as np
import torch

from . import ops
from ._capi import SnowLLMError
from .dflash import SELECTOR_TOP_K, accept_greedy, accept_reject, reject, select_path
from .sampler import Sampler, SamplingParams, Staged  # noqa: F401  (SamplingParams re-exported)


@dataclass(eq=False)
class VerifyRequest:
    """One request of a verify batch: its stable slot, sampling parameters and drafts, and
    the prompt and output ids the penalties and n-gram masks read."""
    slot: int
    params: SamplingParams
    drafts: tuple = ()
    prompt: tuple = ()
    out: list = field(default_factory=list)


class DFlashAcceptance:
    """Host side of the DFlash verify acceptance (snowllm/engine/dflash_sampling.py:8-69):
    device buffers sized for max_seqs requests of `block` rows, the stable-slot proposal
    pool the selector fills, and the verify dispatch."""

    def __init__(self, max_seqs: int, block: int, vocab: int, *, seed: int = 0,
                 selector_top_k: int = SELECTOR_TOP_K, sampler: Sampler = None,
                 max_tokens: int = 4096):
        dev = "cuda"
        self.block, self.length, self.vocab = block, block - 1, vocab
        if sampler is None:
            sampler = Sampler(seed=seed)
            sampler.reserve(max_seqs * block, vocab, max_tokens=max_tokens,
                            max_requests=max_seqs)
        self.sampler = sampler
        self.rng = sampler.rng
        self.proposals = [None] * max_seqs
        self.temperature = torch.zeros(max_seqs, dtype=torch.float32, device=dev)
        self.slots = torch.arange(max_seqs, dtype=torch.int32, device=dev)
        self.uniform = torch.zeros(max_seqs, self.length, dtype=torch.float32, device=dev)
        self.candidates = torch.zeros(max_seqs, self.length, selector_top_k, dtype=torch.int64,
                                      device=dev)
        self.q = torch.zeros(max_seqs, self.length, selector_top_k, dtype=torch.float32,
                             device=dev)
        rows = max_seqs * block
        self.width_max = min(vocab, ops.SAMPLING_MAX_K)
        self.p = torch.empty(rows * self.width_max, dtype=torch.float32, device=dev)
        self.p_ids = torch.empty(rows * self.width_max, dtype=torch.int64, device=dev)
        self.tokens = torch.empty(rows, dtype=torch.int64, device=dev)
        self.staged_temp = Staged(max_seqs, torch.float32)
        self.staged_slots = Staged(max_seqs, torch.int32)
        self.verify_slots = Staged(max_seqs, torch.int32)
        self.verify_valid = Staged(max_seqs, torch.int32)
        self.verify_temp = Staged(rows, torch.float32)
        self.accepted = torch.empty(max_seqs, dtype=torch.int64, device=dev)
        self.verify_uniform = torch.empty(rows, dtype=torch.float32, device=dev)
        self.path = None  # which branch the last verify took: "greedy", "fused", "lists"

    # -- drafting side (dflash_sampling.py:28-52) ------------------------------------------
    def stage(self, batch):
        """Temperatures and stable slots of the batch; selector uniforms when any request
        samples."""
        count = len(batch)
        temps = [r.params.temperature for r in batch]
        self.temperature[:count].copy_(self.staged_temp.write(np.asarray(temps, np.float32)))
        self.slots[:count].copy_(self.staged_slots.write(
            np.asarray([r.slot for r in batch], np.int32)))
        if any(t > 0 for t in temps):
            self.uniform[:count].uniform_(generator=self.rng)

    def propose(self, hp, logits, pred, succ, anchor, path):
        """The selector walk at each request's temperature; its 16-candidate lists and
        probabilities land at the requests' stable slots."""
        count = path.shape[0]
        select_path(hp, logits, pred, succ, anchor, path, self.select_scratch(logits.shape[0]),
                    temperature=self.temperature[:count], uniform=self.uniform[:count],
                    slots=self.slots[:count], candidate_ids=self.candidates,
                    probabilities=self.q)

    def select_scratch(self, n):
        need = ops.dflash.select_scratch_bytes(n)
        if getattr(self, "_sel_scratch", None) is None or self._sel_scratch.numel() < need:
            self._sel_scratch = torch.empty(need, dtype=torch.uint8, device="cuda")
        return self._sel_scratch

    def remember(self, batch, drafts):
        for request, tokens in zip(batch, drafts):
            self.proposals[request.slot] = tuple(int(t) for t in tokens)

    def release(self, request):
        self.proposals[request.slot] = None

    # -- verify (dflash_sampling.py:54-69) ---------------------------------------------------
    def verify(self, logits, batch, drafts):
        """logits [count * width, V] of the verify block (penalties and n-gram masks are
        applied to them in place), drafts [count, width - 1] int64 on the device ->
        (tokens [count, width], accepted [count])."""
        count, width = len(batch), self.block
        if logits.shape != (count * width, self.vocab):
            raise SnowLLMError(f"verify logits must be [{count * width}, {self.vocab}]")
        tokens = self.tokens[:count * width].view(count, width)
        accepted = self.accepted[:count]
        rows = [r for r in batch for _ in range(width)]
        if all(r.params.temperature <= 0 for r in batch):
            self.path = "greedy"
            self.sampler.prepare(logits, rows)
            if not accept_greedy(logits, drafts, tokens, accepted):
                ops.argmax(logits, out=tokens.view(-1))
                ops.spec_accept(tokens, drafts, out=accepted)
            return tokens, accepted
        valid = self.verify_valid.write(np.asarray(
            [int(tuple(r.drafts) == self.proposals[r.slot]) for r in batch], np.int32))
        slots = self.verify_slots.write(np.asarray([r.slot for r in batch], np.int32))
        uniform = self.verify_uniform[:count * width].view(count, width)
        uniform.uniform_(generator=self.rng)
        ks = [r.params.kernel_top_k() for r in rows]
        whole = all(k >= self.vocab for k in ks) and all(r.params.top_p >= 1.0 for r in rows)
        self.sampler.prepare(logits, rows)
        if whole:
            temp = self.verify_temp.write(np.asarray([r.params.kernel_temperature() for r in rows],
                                                     np.float32))
            if accept_reject(logits, drafts, self.candidates, self.q, slots, valid, uniform,
                             tokens, accepted, temperature=temp):
                self.path = "fused"
                return tokens, accepted
        self.path = "lists"
        p, ids = self.sampler.probabilities(logits, rows, self.p, self.p_ids, prepared=True)
        reject(p, ids, drafts, self.candidates, self.q, slots, valid, uniform, tokens, accepted)
        return tokens, accepted

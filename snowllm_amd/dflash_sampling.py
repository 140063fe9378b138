"""The DFlash/DSpark verify-side acceptance and its dispatch (snowllm/engine/dflash_sampling.py:
8-69), on this build's kernels.

Per verify step, for a batch of requests each holding k drafts (block width k + 1):

- every request greedy (temperature <= 0): argmax of every row, then 1 + leading matches
  (snowllm/engine/dflash_sampling.py:56-59) -- one launch (snowverify_accept_greedy);
- otherwise target probabilities with each request's sampling parameters, then rejection
  sampling against the draft's 16-candidate proposal, read at the request's stable slot
  (snowllm/engine/dflash_sampling.py:60-69): `valid` is 1 when the request's drafts are the
  proposal remembered for its slot, uniforms are drawn as [count, width]. When every request
  keeps the whole vocabulary (top-k covering it, top-p 1) this runs straight from the logits
  without materialising probabilities (snowverify_accept_reject, three launches); otherwise
  snowllm_sampling_softmax + _topk_topp and snowllm_draft_reject.

The argmax of the greedy branch is the logits' (NaN as -inf, ties to the first index, as
ops.argmax); the reference's branch samples each row's top-1 list, which names the same token
except where two probabilities round to the same value.
"""
from dataclasses import dataclass

import torch

from . import ops
from ._capi import SnowLLMError
from .dflash import SELECTOR_TOP_K, accept_greedy, accept_reject, reject, select_path


@dataclass
class SamplingParams:
    """The per-request parameters the verify dispatch reads (snowllm/engine/request.py:
    12-35)."""
    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 1.0

    def kernel_top_k(self) -> int:                       # request.py:29-32
        if self.temperature <= 0.0:
            return 1
        return self.top_k if 0 < self.top_k <= ops.SAMPLING_MAX_K else ops.SAMPLING_MAX_K

    def kernel_temperature(self) -> float:               # request.py:34-35
        return self.temperature if self.temperature > 0.0 else 1.0


@dataclass(eq=False)
class VerifyRequest:
    """One request of a verify batch: its stable slot, sampling parameters and drafts."""
    slot: int
    params: SamplingParams
    drafts: tuple = ()


class DFlashAcceptance:
    """Host side of the DFlash verify acceptance (snowllm/engine/dflash_sampling.py:8-69):
    device buffers sized for max_seqs requests of `block` rows, the stable-slot proposal
    pool the selector fills, and the verify dispatch."""

    def __init__(self, max_seqs: int, block: int, vocab: int, *, seed: int = 0,
                 selector_top_k: int = SELECTOR_TOP_K):
        dev = "cuda"
        self.block, self.length, self.vocab = block, block - 1, vocab
        self.rng = torch.Generator(device=dev).manual_seed(seed)
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
        self.ws = torch.empty(ops.sample_workspace_bytes(rows, vocab, self.width_max),
                              dtype=torch.uint8, device=dev)
        self.tokens = torch.empty(rows, dtype=torch.int64, device=dev)
        self.accepted = torch.empty(max_seqs, dtype=torch.int64, device=dev)
        self.verify_uniform = torch.empty(rows, dtype=torch.float32, device=dev)
        self.path = None  # which branch the last verify took: "greedy", "fused", "lists"

    # -- drafting side (dflash_sampling.py:28-52) ------------------------------------------
    def stage(self, batch):
        """Temperatures and stable slots of the batch; selector uniforms when any request
        samples."""
        count = len(batch)
        temps = [r.params.temperature for r in batch]
        self.temperature[:count].copy_(torch.tensor(temps, dtype=torch.float32))
        self.slots[:count].copy_(torch.tensor([r.slot for r in batch], dtype=torch.int32))
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
        """logits [count * width, V] of the verify block, drafts [count, width - 1] int64 on
        the device -> (tokens [count, width], accepted [count])."""
        count, width = len(batch), self.block
        if logits.shape != (count * width, self.vocab):
            raise SnowLLMError(f"verify logits must be [{count * width}, {self.vocab}]")
        tokens = self.tokens[:count * width].view(count, width)
        accepted = self.accepted[:count]
        if all(r.params.temperature <= 0 for r in batch):
            self.path = "greedy"
            if not accept_greedy(logits, drafts, tokens, accepted):
                ops.argmax(logits, out=tokens.view(-1))
                ops.spec_accept(tokens, drafts, out=accepted)
            return tokens, accepted
        rows = [r for r in batch for _ in range(width)]
        valid = torch.tensor([int(tuple(r.drafts) == self.proposals[r.slot]) for r in batch],
                             dtype=torch.int32, device="cuda")
        slots = torch.tensor([r.slot for r in batch], dtype=torch.int32, device="cuda")
        uniform = self.verify_uniform[:count * width].view(count, width)
        uniform.uniform_(generator=self.rng)
        temp = torch.tensor([r.params.kernel_temperature() for r in rows], dtype=torch.float32,
                            device="cuda")
        ks = [r.params.kernel_top_k() for r in rows]
        whole = all(k >= self.vocab for k in ks) and all(r.params.top_p >= 1.0 for r in rows)
        if whole and accept_reject(logits, drafts, self.candidates, self.q, slots, valid,
                                   uniform, tokens, accepted, temperature=temp):
            self.path = "fused"
            return tokens, accepted
        self.path = "lists"
        width_p = min(max(ks), self.vocab)
        n = len(rows) * width_p
        p, ids = self.p[:n].view(-1, width_p), self.p_ids[:n].view(-1, width_p)
        top_k = torch.tensor(ks, dtype=torch.int32, device="cuda")
        top_p = torch.tensor([r.params.top_p for r in rows], dtype=torch.float32, device="cuda")
        ops.probabilities(logits, top_k, top_p, temp, width_p, p, ids, self.ws)
        reject(p, ids, drafts, self.candidates, self.q, slots, valid, uniform, tokens, accepted)
        return tokens, accepted

"""Draft-side proposal heads that feed the verify step: the DFlash 2 candidate selector fed by
its hidden projection (snowllm/models/qwen3_5/dflash_draft.py:187-204) and the DSpark Markov
head (snowllm/models/qwen3_5/dspark_draft.py:12-44). The draft backbone that produces the
hidden rows and logits is not part of this build; these take them as inputs."""
import torch

from . import dflash
from .dflash import Proj
from .dspark import dspark_markov, dspark_markov_workspace_bytes, dspark_pack_weight
from .errors import SnowLLMError


class _Shape:
    def __init__(self, hidden):
        self.hidden = hidden


class SelectorHead:
    """hp = SELECTOR_HIDDEN(hidden) [n, 256] bf16, then the selector walk over the draft logits
    with the predecessor / successor codebooks. sel_hidden: bf16 [256, hidden] or GGUF blocks
    (with fmt) of that matrix; pred / succ: bf16 [V, 256]."""

    def __init__(self, hidden_size: int, sel_hidden, sel_pred, sel_succ, fmt: int = 0):
        dflash.select(_Shape(hidden_size))
        if fmt:
            self.w_hidden = dflash.proj_shuffle_w_kquant(Proj.SELECTOR_HIDDEN, sel_hidden, fmt)
        else:
            self.w_hidden = dflash.proj_shuffle_w(Proj.SELECTOR_HIDDEN, sel_hidden)
        self.pred, self.succ = sel_pred, sel_succ
        self._proj_ws = self._sel_ws = None

    def project(self, hidden: torch.Tensor, hp: torch.Tensor = None) -> torch.Tensor:
        n = hidden.shape[0]
        if hp is None:
            hp = torch.empty(n, dflash.proj_shape(Proj.SELECTOR_HIDDEN)[0], dtype=torch.bfloat16,
                             device="cuda")
        need = dflash.proj_workspace_bytes(Proj.SELECTOR_HIDDEN, self.w_hidden, n)
        if need and (self._proj_ws is None or self._proj_ws.numel() < need):
            self._proj_ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        dflash.proj(Proj.SELECTOR_HIDDEN, hidden, self.w_hidden, self._proj_ws if need else None,
                    hp)
        return hp

    def propose(self, hidden, logits, anchor, path, *, temperature=None, uniform=None,
                slots=None, candidate_ids=None, probabilities=None):
        hp = self.project(hidden)
        need = dflash.select_scratch_bytes(hidden.shape[0])
        if self._sel_ws is None or self._sel_ws.numel() < need:
            self._sel_ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        dflash.select_path(hp, logits, self.pred, self.succ, anchor, path, self._sel_ws,
                           temperature=temperature, uniform=uniform, slots=slots,
                           candidate_ids=candidate_ids, probabilities=probabilities)
        return hp


class MarkovHead:
    """The DSpark head: w1, w2 bf16 [V, rank] (w2 is packed here), conf_weight f32
    [hidden + rank] and an optional scalar conf_bias."""

    def __init__(self, w1: torch.Tensor, w2: torch.Tensor, conf_weight=None, conf_bias=None):
        if w1.shape != w2.shape:
            raise SnowLLMError("DSpark W1 and W2 shapes differ")
        self.w1, self.w2 = w1.contiguous(), dspark_pack_weight(w2.contiguous())
        self.conf_weight = None if conf_weight is None else conf_weight.float().reshape(-1)
        self.conf_bias = None if conf_bias is None else conf_bias.float().reshape(-1)
        self._ws = None

    def propose(self, hidden, logits, anchor, path, confidence=None, fp32_bias=False):
        b, block = path.shape
        if logits.shape[0] != b * block:
            raise SnowLLMError("DSpark logits rows do not match its proposal block")
        need = dspark_markov_workspace_bytes(b, self.w1.shape[0], self.w1.shape[1], block)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        return dspark_markov(logits, self.w1, self.w2, anchor, block,
                             pre_head=hidden if confidence is not None else None,
                             conf_weight=self.conf_weight if confidence is not None else None,
                             conf_bias=self.conf_bias if confidence is not None else None,
                             confidence=confidence, workspace=self._ws, out=path,
                             fp32_bias=fp32_bias)

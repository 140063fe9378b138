"""torch restatements of the reference's own CPU semantics -- TEST INFRASTRUCTURE ONLY.

These follow the reference's tests line by line, in torch fp32 as they are written there.
They are the independent check that pins the canonical C oracle (accept.c) to the reference
semantics, and they are the "reference CPU path" timed by bench.py's cpu_baseline leg.
"""
import torch


def reference_reject(p, ids, drafts, q_ids, q, slots, valid, uniform):
    """tests/test_dflash_sampling.py:94-119 (rejection sampling with residual resample)."""
    output, lengths = [], []
    for b in range(drafts.shape[0]):
        length = drafts.shape[1]
        chosen = []
        for j in range(length):
            token = drafts[b, j]
            pt = p[b, j][ids[b, j] == token].sum()
            qt = q[slots[b], j][q_ids[slots[b], j] == token].sum() if valid[b] else 1.
            if uniform[b, j] * qt >= pt:
                break
            chosen.append(token.item())
        first = len(chosen)
        residual = p[b, first].clone()
        if first < length:
            for k, token in enumerate(ids[b, first]):
                qt = (q[slots[b], first][q_ids[slots[b], first] == token].sum() if valid[b]
                      else float(token == drafts[b, first]))
                residual[k] = (residual[k] - qt).clamp_min(0)
        if residual.sum() == 0:
            residual = p[b, first].clone()
        cdf = residual.cumsum(-1)
        pick = (uniform[b, -1] * residual.sum() >= cdf).sum().clamp_max(len(cdf) - 1)
        chosen.append(ids[b, first, pick].item())
        output.append(chosen + [-1] * (length + 1 - len(chosen)))
        lengths.append(len(chosen))
    return torch.tensor(output), torch.tensor(lengths)


def reference_reject_identity(p, drafts, q, uniform):
    """reference_reject specialised to full-vocabulary candidate lists (ids = 0..V-1 for
    both p and q, one request slot per row, valid proposals) -- BASELINE config 1. The
    residual loop of the generic form is O(V^2) there; this is the same arithmetic written
    with tensor ops: p [b, k+1, V], q [b, k, V], drafts [b, k], uniform [b, k+1]."""
    output, lengths = [], []
    for b in range(drafts.shape[0]):
        length = drafts.shape[1]
        chosen = []
        for j in range(length):
            token = drafts[b, j]
            pt = p[b, j, token]
            qt = q[b, j, token]
            if uniform[b, j] * qt >= pt:
                break
            chosen.append(token.item())
        first = len(chosen)
        residual = p[b, first].clone()
        if first < length:
            residual = (residual - q[b, first]).clamp_min(0)
        if residual.sum() == 0:
            residual = p[b, first].clone()
        cdf = residual.cumsum(-1)
        pick = (uniform[b, -1] * residual.sum() >= cdf).sum().clamp_max(len(cdf) - 1)
        chosen.append(pick.item())
        output.append(chosen + [-1] * (length + 1 - len(chosen)))
        lengths.append(len(chosen))
    return torch.tensor(output), torch.tensor(lengths)


def reference_greedy(logits, drafts):
    """Greedy verify: argmax with NaN as -inf (tests/test_sampling_argmax.py:29-30), then
    accepted = 1 + leading matches (snowllm/engine/spec_decode.py:203-206)."""
    tokens = logits.nan_to_num(nan=float('-inf'), posinf=float('inf'),
                               neginf=float('-inf')).argmax(-1)
    b, k = drafts.shape
    tv = tokens.view(b, k + 1)
    acc = []
    for i in range(b):
        a = 1
        while a < k + 1 and tv[i, a - 1] == drafts[i, a - 1]:
            a += 1
        acc.append(a)
    return tv, torch.tensor(acc)


def target_probabilities(logits, temperature, top_k, top_p):
    """tests/test_dflash_sampling.py:199-209 as a dense [rows, V] distribution."""
    expected = torch.zeros_like(logits)
    for i in range(logits.shape[0]):
        if temperature[i] <= 0:
            expected[i, logits[i].argmax()] = 1.
            continue
        k = int(top_k[i]) if 0 < int(top_k[i]) <= logits.shape[1] else logits.shape[1]
        scores, candidates = logits[i].topk(k)
        probabilities = (scores / float(temperature[i])).softmax(-1)
        probabilities *= probabilities.cumsum(-1) - probabilities < float(top_p[i])
        expected[i, candidates] = probabilities / probabilities.sum()
    return expected


def dense_attention(q, k, v, scale, mask=None):
    """fp32 masked softmax attention (tests/test_draft_window.py:62-67,
    tests/test_lfm2_long_attention.py:36-44): q [T, H, d], k/v [L, Hkv, d] -> [T, H, d].
    mask [T, L] bool (True = visible) or None."""
    T, H, d = q.shape
    Hkv = k.shape[1]
    g = H // Hkv
    qf = q.float().view(T, Hkv, g, d)
    kf, vf = k.float(), v.float()
    out = torch.empty(T, Hkv, g, d)
    for h in range(Hkv):
        s = torch.einsum("tgd,ld->tgl", qf[:, h], kf[:, h]) * scale
        if mask is not None:
            s = s.masked_fill(~mask[:, None, :], float("-inf"))
        out[:, h] = torch.einsum("tgl,ld->tgd", s.softmax(-1), vf[:, h])
    return out.view(T, H, d)

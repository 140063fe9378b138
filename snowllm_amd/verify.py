"""The speculative-decoding verify step on one MI355X.

One verify step runs the target model over a block of T = k+1 rows (the last accepted token
plus k draft tokens) against the paged KV cache and then accepts a prefix of the drafts:

  embed -> [norm -> QKV -> QK-norm/RoPE/KV write -> paged attention -> O] ->
           [norm -> MoE (router, top-k, experts, shared expert) | SwiGLU MLP]  x L
  -> final norm -> LM head -> target probabilities -> rejection sampling (or argmax + prefix)

Layer order and fusions follow the reference's Qwen3.5 model (snowllm/models/qwen3_5/
qwen3_5.py:32-78, layers.py:75-228) and its verify drivers (snowllm/engine/spec_decode.py:
263-309, 527-581). Every launch goes to torch's current stream and nothing allocates or
synchronises inside step(), so the step can be captured in one HIP graph.

Weights are either random-initialised on the GPU from seeded generators, in the formats of
the BASELINE configs (Q4_K/Q8_0 GGUF blocks repacked with snowllm_gemm_kquant_shuffle_b, fp16
embedding and LM head, bf16 router and norms), or read from a GGUF checkpoint
(snowllm_amd.checkpoint: bf16 or Q4_K embedding, bf16 or k-quant head).
"""
from dataclasses import dataclass, field, replace
import math

import torch

from . import layers as Lops
from . import ops
from ._capi import SnowLLMError

Q4_K, Q5_K, Q6_K, Q8_0 = 4, 5, 6, 8
HEAD_KQUANT = -1   # VerifyModel.head_wt for a Q4_K / Q8_0 head (lm_head = (quant, meta))
# rows of one verify step over all its requests (SPEC_MAX_STEP_ROWS, snowllm/defaults.py:9)
MAX_STEP_ROWS = 256


@dataclass
class VerifyConfig:
    name: str
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    rot_half: int            # rotated pairs per head (rotary dims / 2)
    rope_theta: float
    vocab: int
    context: int             # prior tokens in the KV cache
    block: int               # T = k + 1 query rows
    ffn: int = 0             # dense SwiGLU width (0 for MoE)
    experts: int = 0
    expert_ffn: int = 0
    topk: int = 0
    shared_expert: bool = True
    attn_fmt: int = Q4_K
    ffn_fmt: int = Q4_K
    down_fmt: int = 0        # format of the down projections when it differs (0: ffn_fmt)
    v_fmt: int = 0           # V rows in their own format, q|k in attn_fmt (0: one q|k|v weight)
    tree_parents: tuple = ()  # non-empty: tree block (ancestor mask) instead of a chain
    eps: float = 1e-6
    page: int = 16
    qk_norm: bool = True
    centered: bool = True    # zero-mean Q4_K model weights (gguf_random); False: config 2's

    @property
    def moe(self):
        return self.experts > 0

    @property
    def qkv_n(self):
        return (self.heads + 2 * self.kv_heads) * self.head_dim


# BASELINE.json configs. RoPE: config 3 rotates the full head (theta 1e6); the 35B-A3B shape
# rotates 64 of 256 dims (partial_rotary_factor 0.25, as the reference's Qwen3.5 loader
# requires at snowllm/models/qwen3_5/qwen3_5_weights.py:443-445) with theta 1e7.
# Config 3's linear weights are Q4_K "as in config 2" (its generator exactly); the MoE shapes
# use zero-mean blocks so that the router logits stay ~N(0, 1) per row (gguf_random).
CONFIG3 = VerifyConfig("config3_dense8b", layers=36, hidden=4096, heads=32, kv_heads=8,
                       head_dim=128, rot_half=64, rope_theta=1e6, vocab=151936, context=8192,
                       block=9, ffn=14336, centered=False)
CONFIG4 = VerifyConfig("config4_moe35b_a3b", layers=40, hidden=2048, heads=16, kv_heads=2,
                       head_dim=256, rot_half=32, rope_theta=1e7, vocab=151936, context=8192,
                       block=9, experts=256, expert_ffn=512, topk=8)
CONFIG5 = replace(CONFIG4, name="config5_moe35b_a3b_220k_tree", context=220000, block=11,
                  attn_fmt=Q8_0, tree_parents=(-1, 0, 1, 2, 3, 4, 0, 6, 7, 8, 9))
CONFIGS = {"config3": CONFIG3, "config4": CONFIG4, "config5": CONFIG5}


def geometry_fields(cfg: VerifyConfig) -> dict:
    """The BuildGeometry fields of a config, for ops.define_geometry (the reference-signature
    entry points and the checkpoint repacks read their shapes from the active geometry)."""
    d, moe = cfg.head_dim, cfg.moe
    return dict(
        hidden=cfg.hidden, num_heads=cfg.heads, num_kv_heads=cfg.kv_heads, head_size=d,
        block_size=cfg.page, vocab_size=cfg.vocab, qkv_proj_n=cfg.qkv_n, qkv_q_head_stride=d,
        qkv_off_k=cfg.heads * d, qkv_off_v=(cfg.heads + cfg.kv_heads) * d,
        moe_num_experts=cfg.experts if moe else 0, moe_shared_expert=int(moe),
        moe_topk=cfg.topk if moe else 0, moe_topk_all=cfg.topk + 1 if moe else 0,
        moe_inter=cfg.expert_ffn if moe else 0, sampling_max_k=1 << 19,
        lm_head_decode_max_m=256, mlp_inter=0 if moe else cfg.ffn,
        mlp_gate_up_n=0 if moe else 2 * cfg.ffn)


def tree_masks(parents):
    masks = []
    for i, p in enumerate(parents):
        masks.append((1 << i) | (masks[p] if p >= 0 else 0))
    return masks


def tree_depths(parents):
    d = []
    for p in parents:
        d.append(0 if p < 0 else d[p] + 1)
    return d


# ---------------------------------------------------------------------------------------
# random-init weights (GPU)
# ---------------------------------------------------------------------------------------
def gguf_random(fmt, n, k, seed, device="cuda", centered=False):
    """Seeded random GGUF blocks for an [n, k] weight: Q4_K with 6-bit scales/mins and nibbles
    uniform and d, dmin = fp16(|N(0, 1e-3^2)|); Q8_0 with int8 uniform in
    -127..127 and d = fp16(|N(0, 1e-2^2)|).

    centered (model weights): Q4_K blocks whose dequantised values are zero-mean, as GGUF
    blocks quantised from a trained matrix are (the min offsets one sub-block's range):
    d = fp16(|N(0, (2e-4)^2)|), dmin = fp16(8 d), m_j = round(0.9375 sc_j), so that
    w = d sc_j q - dmin m_j ~ d sc_j (q - 7.5). Uniform raw mins put a common-mode component
    into every projection, which makes all rows of a block route to the same experts."""
    g = torch.Generator(device=device).manual_seed(seed)
    if fmt == Q4_K:
        nb = n * k // 256
        raw = torch.randint(0, 256, (nb, 144), dtype=torch.uint8, device=device, generator=g)
        if not centered:
            dd = (torch.randn(nb, 2, device=device, generator=g) * 1e-3).abs().half()
            raw[:, 0:4] = dd.view(torch.uint8).view(nb, 4)
            return raw.view(-1)
        d = (torch.randn(nb, device=device, generator=g) * 2e-4).abs()
        dd = torch.stack([d, 8 * d], 1).half()
        raw[:, 0:4] = dd.view(torch.uint8).view(nb, 4)
        sc = torch.randint(0, 64, (nb, 8), dtype=torch.int32, device=device, generator=g)
        mn = torch.round(sc.float() * 0.9375).int().clamp_(0, 63)
        lo = (sc[:, :4] & 63) | ((sc[:, 4:] >> 4) << 6)
        mid = (mn[:, :4] & 63) | ((mn[:, 4:] >> 4) << 6)
        hi = (sc[:, 4:] & 15) | ((mn[:, 4:] & 15) << 4)
        raw[:, 4:16] = torch.cat([lo, mid, hi], 1).to(torch.uint8)
        return raw.view(-1)
    if fmt == Q5_K:
        # Q4_K's form with a fifth bit (qh uniform); centered: dmin = 16 d, m_j = round(0.96875
        # sc_j), so that w ~ d sc_j (q - 15.5)
        nb = n * k // 256
        raw = torch.randint(0, 256, (nb, 176), dtype=torch.uint8, device=device, generator=g)
        dstd = 8e-5 if centered else 1e-3
        d = (torch.randn(nb, device=device, generator=g) * dstd).abs()
        dd = torch.stack([d, 16 * d if centered else d], 1).half()
        raw[:, 0:4] = dd.view(torch.uint8).view(nb, 4)
        if centered:
            sc = torch.randint(0, 64, (nb, 8), dtype=torch.int32, device=device, generator=g)
            mn = torch.round(sc.float() * 0.96875).int().clamp_(0, 63)
            lo = (sc[:, :4] & 63) | ((sc[:, 4:] >> 4) << 6)
            mid = (mn[:, :4] & 63) | ((mn[:, 4:] >> 4) << 6)
            hi = (sc[:, 4:] & 15) | ((mn[:, 4:] & 15) << 4)
            raw[:, 4:16] = torch.cat([lo, mid, hi], 1).to(torch.uint8)
        return raw.view(-1)
    if fmt == Q6_K:
        # ql/qh uniform, int8 scales uniform in -64..64, d = fp16(|N(0, s^2)|): w = d sc (q - 32)
        nb = n * k // 256
        raw = torch.randint(0, 256, (nb, 210), dtype=torch.uint8, device=device, generator=g)
        sc = torch.randint(-64, 65, (nb, 16), dtype=torch.int8, device=device, generator=g)
        raw[:, 192:208] = sc.view(torch.uint8)
        d = (torch.randn(nb, device=device, generator=g) * (3.5e-5 if centered else 1e-4)).abs()
        raw[:, 208:210] = d.half().view(torch.uint8).view(nb, 2)
        return raw.view(-1)
    if fmt == Q8_0:
        nb = n * k // 32
        raw = torch.empty(nb, 34, dtype=torch.uint8, device=device)
        q = torch.randint(-127, 128, (nb, 32), dtype=torch.int8, device=device, generator=g)
        d = (torch.randn(nb, device=device, generator=g) * 1e-2).abs().half()
        raw[:, 0:2] = d.view(torch.uint8).view(nb, 2)
        raw[:, 2:] = q.view(torch.uint8)
        return raw.view(-1)
    raise SnowLLMError(f"unknown format {fmt}")


def packed_random(fmt, n, k, seed, keep_raw=False, centered=True, stack=1):
    """(quant, meta, raw GGUF bytes or None) of a seeded random [n, k] weight; stack > 1: n
    rows of `stack` equal weights (an expert stack), each repacked on its own."""
    raw = gguf_random(fmt, n, k, seed, centered=centered)
    if stack > 1:
        quant, meta = ops.kquant_shuffle_stack(fmt, raw, stack, n // stack, k)
    else:
        quant, meta = ops.gemm_kquant_shuffle_b(fmt, raw, n, k)
    return (quant, meta, raw if keep_raw else None)


@dataclass
class LayerWeights:
    in_norm: torch.Tensor
    post_norm: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    qkv: tuple
    o: tuple
    router: torch.Tensor = None      # shuffled bf16 [E+1, H]
    gu: tuple = None                 # stacked experts (MoE) or the dense MLP gate/up
    dn: tuple = None
    sh_gu: tuple = None
    sh_dn: tuple = None
    raw: dict = field(default_factory=dict)  # unshuffled copies kept for parity checks
    # formats of this layer's matrices where a checkpoint stores them differently from the
    # config's attn_fmt / ffn_fmt (0: the config's)
    qkv_fmt: int = 0
    o_fmt: int = 0
    gu_fmt: int = 0
    dn_fmt: int = 0
    # V rows of the attention projection in their own format (then qkv holds the q|k rows):
    # GGUF files keep attn_v wider than attn_q / attn_k in some layers
    v: tuple = None
    v_fmt: int = 0


class VerifyModel:
    """Weights, KV pools and step buffers of one verify-step configuration."""

    def __init__(self, cfg: VerifyConfig, seed: int = 0, keep_raw=False, kv_std: float = 1.0,
                 weights=None, batch: int = 1):
        """keep_raw: keep the unshuffled GGUF bytes (and the router / LM head) for parity
        checks -- True for every layer, an int n for the first n layers, or a collection of
        layer indices. weights: None for seeded random weights, else a callable that installs
        layers / embed / lm_head / head_wt / final_norm on the model (a checkpoint loader).
        batch: requests verified together, each with cfg.block rows (at most cfg.block for a
        ragged batch, see set_batch) and its own pages of the KV pools; batch * block <=
        MAX_STEP_ROWS."""
        if batch < 1 or batch * cfg.block > MAX_STEP_ROWS:
            raise SnowLLMError(f"a verify step holds at most {MAX_STEP_ROWS} rows")
        self.batch = batch
        self.cfg = c = cfg
        self.keep_raw = keep_raw
        dev = "cuda"
        torch.cuda.synchronize()
        self.head_wt = Lops.WT_F16   # or WT_BF16, or HEAD_KQUANT with self.head_fmt
        self.head_fmt = 0
        # MoE layers: post-attention norm, router and routing/plan in one launch where the
        # fused kernel takes the shape (False: the three separate launches, the same bits)
        # the MoE and the 16-bit GEMVs take at most 16 rows per launch: a step of more rows
        # runs them on row chunks (the fused router on chunks whose rows fit its LDS)
        M = batch * c.block
        self.rows = M
        self.row_chunks = [(r0, min(16, M - r0)) for r0 in range(0, M, 16)]
        # one MoE plan per 64 rows (an expert with more than 16 of them takes a slot per 16),
        # so each expert's weights are read once per 16 of its rows across the whole batch
        R = Lops.MOE_MAX_ROWS
        self.moe_chunks = [(r0, min(R, M - r0)) for r0 in range(0, M, R)]
        # norm + router + routing/plan in one launch holds up to 16 rows
        chunk = max(n for _, n in self.moe_chunks)
        self.fuse_router = bool(c.moe and chunk <= 16 and c.hidden % 512 == 0 and
                                c.hidden <= 4096 and chunk * (c.hidden + 8) * 2 <= 131072 and
                                chunk * (c.experts + 1) * 4 <= 131072)
        self.embed_q4k = False       # True: self.embed holds Q4_K blocks [V, H / 256 * 144]
        self.lm_head_raw = None
        if weights is None:
            self._random_weights(seed, keep_raw)
        else:
            weights(self)
        self.inv_freq = (1.0 / (c.rope_theta ** (torch.arange(c.rot_half, device=dev,
                                                             dtype=torch.float32) / c.rot_half)))
        # KV cache: context + block pages per request, random page table (prior tokens ~
        # N(0, kv_std^2))
        T = c.block
        self.pages = (c.context + T + c.page - 1) // c.page
        self.blocks = batch * self.pages + 8
        kvg = torch.Generator(device=dev).manual_seed(seed + 7)
        shape_k = (self.blocks, c.kv_heads, c.head_dim // 16, c.page, 16)
        shape_v = (self.blocks, c.kv_heads, c.page // 4, c.head_dim, 4)
        self.k_pools, self.v_pools = [], []
        for _ in range(c.layers):
            k = torch.empty(shape_k, dtype=torch.bfloat16, device=dev)
            v = torch.empty(shape_v, dtype=torch.bfloat16, device=dev)
            k.normal_(0, kv_std, generator=kvg)
            v.normal_(0, kv_std, generator=kvg)
            self.k_pools.append(k)
            self.v_pools.append(v)
        perm = torch.randperm(self.blocks, device=dev, generator=kvg)[:batch * self.pages]
        self.table = perm.int().view(batch, -1).contiguous()
        self._alloc_step_buffers()

    def _random_weights(self, seed, keep_raw):
        c, dev = self.cfg, "cuda"
        gen = torch.Generator(device=dev).manual_seed(seed)
        H, V = c.hidden, c.vocab

        def gamma(n):
            return (1.0 + 0.02 * torch.randn(n, device=dev, generator=gen)).bfloat16()

        def sub(i, j):
            return seed * 100003 + i * 101 + j

        self.layers = []
        for i in range(c.layers):
            if isinstance(keep_raw, bool):
                kr = keep_raw
            elif isinstance(keep_raw, int):
                kr = i < keep_raw
            else:
                kr = i in keep_raw

            def pk(fmt, n, k, j, stack=1):
                return packed_random(fmt, n, k, sub(i, j), kr, c.centered, stack)

            nqk = (c.heads + c.kv_heads) * c.head_dim
            lw = LayerWeights(in_norm=gamma(H), post_norm=gamma(H), q_norm=gamma(c.head_dim),
                              k_norm=gamma(c.head_dim),
                              qkv=pk(c.attn_fmt, nqk if c.v_fmt else c.qkv_n, H, 0),
                              o=pk(c.attn_fmt, H, c.heads * c.head_dim, 1))
            if c.v_fmt:
                lw.v, lw.v_fmt = pk(c.v_fmt, c.qkv_n - nqk, H, 6), c.v_fmt
            if c.moe:
                E, F = c.experts, c.expert_ffn
                router = (torch.randn(E + 1, H, device=dev, generator=gen) / math.sqrt(H)).bfloat16()
                lw.router = Lops.dense_shuffle(router)
                lw.gu = pk(c.ffn_fmt, E * 2 * F, H, 2, E)
                lw.dn = pk(c.down_fmt or c.ffn_fmt, E * H, F, 3, E)
                lw.sh_gu = pk(c.ffn_fmt, 2 * F, H, 4)
                lw.sh_dn = pk(c.down_fmt or c.ffn_fmt, H, F, 5)
                if kr:
                    lw.raw["router"] = router
            else:
                lw.gu = pk(c.ffn_fmt, 2 * c.ffn, H, 2)
                lw.dn = pk(c.down_fmt or c.ffn_fmt, H, c.ffn, 3)
            lw.dn_fmt = c.down_fmt
            self.layers.append(lw)
        self.embed = (0.02 * torch.randn(V, H, device=dev, generator=gen)).half()
        head = (0.02 * torch.randn(V, H, device=dev, generator=gen)).half()
        self.lm_head = Lops.dense_shuffle(head)
        self.lm_head_raw = head if (keep_raw is not False and keep_raw != 0) else None
        self.final_norm = gamma(H)

    # -----------------------------------------------------------------------------------
    def _alloc_step_buffers(self):
        c, dev = self.cfg, "cuda"
        T = self.rows            # all rows of the step: batch * block
        B = self.batch
        H = c.hidden
        bf = torch.bfloat16
        self.ids = torch.zeros(T, dtype=torch.int64, device=dev)
        self.positions = torch.zeros(T, dtype=torch.int64, device=dev)
        self.slots = torch.zeros(T, dtype=torch.int32, device=dev)
        self.lens = torch.zeros(B, dtype=torch.int32, device=dev)
        self.lengths = [c.block] * B   # rows per request (ragged batches: set_batch)
        self.tree = None
        if c.tree_parents:
            self.tree = torch.tensor([m - (1 << 64) if m >= 1 << 63 else m
                                      for m in tree_masks(c.tree_parents)] * B,
                                     dtype=torch.int64, device=dev)
        self._chain_tree = None  # ancestor masks of a ragged chain batch (set_batch)
        self.cos = torch.empty(T, c.rot_half, dtype=torch.float32, device=dev)
        self.sin = torch.empty_like(self.cos)
        self.x = torch.empty(T, H, dtype=bf, device=dev)         # layer input (block output)
        self.res = [torch.empty(T, H, dtype=bf, device=dev) for _ in range(2)]
        self.proj = torch.empty(T, c.qkv_n, dtype=bf, device=dev)
        self.q = torch.empty(T, c.heads, c.head_dim, dtype=bf, device=dev)
        self.attn = torch.empty(T, c.heads, c.head_dim, dtype=bf, device=dev)
        self.o = torch.empty(T, H, dtype=bf, device=dev)
        self.h2 = torch.empty(T, H, dtype=bf, device=dev)
        wsH = ops.gemm_kquant_a_ws_bytes(T, H)
        self.ws_h = torch.empty(wsH, dtype=torch.uint8, device=dev)
        self.ws_h2 = torch.empty(wsH, dtype=torch.uint8, device=dev)
        self.ws_a = torch.empty(ops.gemm_kquant_a_ws_bytes(T, c.heads * c.head_dim),
                                dtype=torch.uint8, device=dev)
        self.attn_scratch = torch.empty(
            ops.paged_attention_explicit_scratch_bytes(B, c.block, c.heads, c.kv_heads,
                                                       c.head_dim),
            dtype=torch.uint8, device=dev)
        self.ws_tile = ops.gemm_kquant_a_ws_bytes(16, H)   # one 16-row tile of ws_h / ws_h2
        if c.moe:
            E, F, K = c.experts, c.expert_ffn, c.topk
            self.router_logits = torch.empty(T, E + 1, dtype=torch.float32, device=dev)
            self.route_w = torch.empty(T, K, dtype=torch.float32, device=dev)
            self.route_ids = torch.empty(T, K, dtype=torch.int32, device=dev)
            self.shared_w = torch.empty(T, dtype=torch.float32, device=dev)
            self.plans = [torch.empty(Lops.MOE_PLAN_BYTES, dtype=torch.uint8, device=dev)
                          for _ in self.moe_chunks]
            self.plan = self.plans[0]
            self.moe_slots = [Lops.moe_max_slots(n, K, E) for _, n in self.moe_chunks]
            self.moe_act = torch.empty(max(self.moe_slots), 16, F, dtype=bf, device=dev)
            self.pairs = torch.empty(T * K, H, dtype=torch.float32, device=dev)
            self.shared_out = torch.empty(T, H, dtype=torch.float32, device=dev)
        else:
            self.act = torch.empty(T, c.ffn, dtype=bf, device=dev)
            self.ws_act = torch.empty(ops.gemm_kquant_a_ws_bytes(T, c.ffn), dtype=torch.uint8,
                                      device=dev)
        self.ws_f = torch.empty(wsH, dtype=torch.uint8, device=dev)
        self.logits = torch.empty(T, c.vocab, dtype=torch.float32, device=dev)

    def set_block(self, ids, context=None):
        """Stage one block: ids [T] (last token + drafts) at positions context..context+T-1
        (tree blocks: context + depth). Host-side, outside the timed/captured step. A batched
        model stages every request with the same block (set_batch for anything else)."""
        B = self.batch
        ids = torch.as_tensor(ids, dtype=torch.int64).view(1, -1).expand(B, -1)
        ctx = self.cfg.context if context is None else context
        self.set_batch(ids, [ctx] * B)

    def set_batch(self, ids, contexts, lengths=None):
        """Stage a batch: ids [batch, T] (each request's last token + drafts; a ragged request
        uses its first lengths[b] ids), request b's rows at positions contexts[b] + t (tree
        blocks: + depth) with its K/V written at those positions of its pages. Ragged batches
        (a length below the block) keep the padded layout [batch, T]: the padding rows write no
        cache (slot -1) and see only themselves, the real rows never see them (ancestor masks
        of the chain), and their logits are ignored. Host-side, outside the captured step; a
        graph captured with one ragged/uniform shape must be replayed with the same kind."""
        c, B, T = self.cfg, self.batch, self.cfg.block
        dev = "cuda"
        ids = torch.as_tensor(ids, dtype=torch.int64).view(B, T)
        lengths = [T] * B if lengths is None else [int(n) for n in lengths]
        if len(contexts) != B or len(lengths) != B or not all(1 <= n <= T for n in lengths):
            raise SnowLLMError("set_batch: one context and a length in 1..block per request")
        if any(n < T for n in lengths) and (c.tree_parents or T > 64):
            raise SnowLLMError("set_batch: ragged lengths apply to chain blocks of <= 64 rows")
        if any(x < 0 or x + T > self.pages * c.page for x in contexts):
            raise SnowLLMError("set_batch: a request's block runs past its pages")
        depth = tree_depths(c.tree_parents) if c.tree_parents else list(range(T))
        tbl = self.table.cpu().long()
        pos, slots = [], []
        for b in range(B):
            for t in range(T):
                p = contexts[b] + t
                pos.append(contexts[b] + depth[t])
                slots.append(int(tbl[b, p // c.page]) * c.page + p % c.page if t < lengths[b]
                             else -1)
        self.ids.copy_(ids.reshape(-1).to(dev))
        self.positions.copy_(torch.tensor(pos, dtype=torch.int64, device=dev))
        self.slots.copy_(torch.tensor(slots, dtype=torch.int32, device=dev))
        self.lens.copy_(torch.tensor([x + T for x in contexts], dtype=torch.int32, device=dev))
        self.lengths = lengths
        if not c.tree_parents:
            if all(n == T for n in lengths):
                self.tree = None
            else:
                masks = [((2 << t) - 1) if t < n else (1 << t) for n in lengths for t in range(T)]
                self._chain_tree = torch.tensor([m - (1 << 64) if m >= 1 << 63 else m
                                                 for m in masks], dtype=torch.int64, device=dev)
                self.tree = self._chain_tree

    # -----------------------------------------------------------------------------------
    def forward(self, *, upto_layer=None, record_slots=None):
        """Target model over the staged block -> self.logits [T, V] f32. record_slots: optional
        int32 [layers] device tensor that receives each MoE layer's unique routed experts over
        all rows + the shared expert, for byte accounting; it adds a count per layer, so timed
        steps leave it out."""
        c, T = self.cfg, self.rows
        H = c.hidden
        if self.embed_q4k:
            from .embedding import gather_embedding_q4_k
            gather_embedding_q4_k(self.ids, self.embed, self.x)
        else:
            Lops.gather_embedding(self.ids, self.embed, self.x)
        Lops.rope_cos_sin(self.positions, self.inv_freq, self.cos, self.sin)
        res_in, res_out = None, self.res[0]
        n_layers = c.layers if upto_layer is None else upto_layer
        moe_out = False  # the previous layer's MoE output is still in (pairs, shared_out)

        def norm(gamma, ws, y_out=None):
            # residual update + norm fused with the GEMV operand prep; after a MoE layer the
            # experts' combine is fused in too (self.x still receives the layer output)
            if moe_out:
                Lops.norm_prep_moe(self.pairs, self.shared_out, c.topk, gamma, ws, c.eps,
                                   x_out=self.x, res_in=res_in, res_out=res_out, y_out=y_out)
            else:
                Lops.norm_prep(self.x, gamma, ws, c.eps, res_in=res_in, res_out=res_out,
                               y_out=y_out)

        for i in range(n_layers):
            lw = self.layers[i]
            # attention block
            norm(lw.in_norm, self.ws_h)
            if lw.v is None:
                ops.gemm_kquant_a_prepared(lw.qkv_fmt or c.attn_fmt, lw.qkv[0], lw.qkv[1],
                                           self.proj, T, c.qkv_n, H, self.ws_h)
            else:   # q|k and v in their formats, into their columns of proj
                nqk = (c.heads + c.kv_heads) * c.head_dim
                ops.gemm_kquant_a_prepared(lw.qkv_fmt or c.attn_fmt, lw.qkv[0], lw.qkv[1],
                                           self.proj, T, nqk, H, self.ws_h, col=0)
                ops.gemm_kquant_a_prepared(lw.v_fmt, lw.v[0], lw.v[1], self.proj, T,
                                           c.qkv_n - nqk, H, self.ws_h, col=nqk)
            if c.rot_half <= ops.FUSED_QK_MAX_HALF:
                # QK-norm + RoPE + the block's K/V cache write inside the attention's launches
                # with 256-wide heads the merge also writes the O projection's operands
                ws_o = self.ws_a if c.head_dim == 256 else None
                ops.paged_attention_qk(self.proj, lw.q_norm, lw.k_norm, self.cos, self.sin,
                                       c.eps, self.slots, self.k_pools[i], self.v_pools[i],
                                       self.attn, self.table, self.lens, c.head_dim ** -0.5,
                                       self.attn_scratch, num_heads=c.heads,
                                       num_kv_heads=c.kv_heads, tree=self.tree, q_out=self.q,
                                       ws_out=ws_o)
            else:
                Lops.qk_norm_rope_cache(self.proj, lw.q_norm, lw.k_norm, self.cos, self.sin,
                                        self.q, self.k_pools[i], self.v_pools[i], self.slots,
                                        c.eps)
                ops.paged_attention_explicit(self.q, self.k_pools[i], self.v_pools[i], self.attn,
                                             self.table, self.lens, c.head_dim ** -0.5,
                                             self.attn_scratch, tree=self.tree)
            if c.rot_half <= ops.FUSED_QK_MAX_HALF and c.head_dim == 256:
                ops.gemm_kquant_a_prepared(lw.o_fmt or c.attn_fmt, lw.o[0], lw.o[1], self.o, T,
                                           H, c.heads * c.head_dim, self.ws_a)
            else:
                ops.gemm_kquant_a(lw.o_fmt or c.attn_fmt, self.attn.view(T, -1), lw.o[0], lw.o[1],
                                  self.o, T, H, c.heads * c.head_dim, self.ws_a)
            # feed-forward block
            res_in, res_out = res_out, self.res[1] if res_out is self.res[0] else self.res[0]
            gu_fmt = lw.gu_fmt or c.ffn_fmt
            dn_fmt = lw.dn_fmt or c.down_fmt or c.ffn_fmt
            if c.moe:
                # the router, routing and experts on row chunks of at most 16 rows (one chunk
                # for a single block); chunk j's operands are its rows' tiles of ws_h2
                if not self.fuse_router:
                    Lops.norm_prep(self.o, lw.post_norm, self.ws_h2, c.eps, res_in=res_in,
                                   res_out=res_out, y_out=self.h2)
                K = c.topk
                for j, (r0, n) in enumerate(self.moe_chunks):
                    rs = slice(r0, r0 + n)
                    ws = self._ws_rows(self.ws_h2, r0)
                    plan = self.plans[j]
                    if self.fuse_router:
                        # post-attention norm + router GEMV + routing and plan: one launch
                        Lops.norm_router_plan(self.o[rs], lw.post_norm, ws, c.eps, lw.router,
                                              self.router_logits[rs], K, self.route_w[rs],
                                              self.route_ids[rs], self.shared_w[rs], plan,
                                              res_in=res_in[rs], res_out=res_out[rs],
                                              y_out=self.h2[rs])
                    else:
                        Lops.dense_gemv(Lops.WT_BF16, lw.router, self.h2[rs],
                                        self.router_logits[rs], n, c.experts + 1, H)
                        Lops.moe_route_plan(self.router_logits[rs], c.experts, K,
                                            self.route_w[rs], self.route_ids[rs],
                                            self.shared_w[rs], plan)

                    # gate/up and down in one launch: a slot's down starts when its gate/up
                    # is done
                    Lops.moe_gate_up_down(gu_fmt | dn_fmt << 8, lw.gu, lw.dn, lw.sh_gu, lw.sh_dn, plan,
                                          ws, self.route_w[rs], self.shared_w[rs],
                                          self.moe_act, self.pairs[r0 * K:(r0 + n) * K],
                                          self.shared_out[rs], n, self.moe_slots[j],
                                          c.experts, H, c.expert_ffn)
                if record_slots is not None:
                    # unique routed experts of the whole step + the shared expert
                    used = torch.bincount(self.route_ids.view(-1).long(), minlength=c.experts)
                    record_slots[i:i + 1].copy_((used > 0).sum().view(1) + 1)
                moe_out = True
            else:
                Lops.norm_prep(self.o, lw.post_norm, self.ws_h2, c.eps, res_in=res_in,
                               res_out=res_out)
                for r0, n in self.row_chunks:
                    Lops.gate_up_swiglu(gu_fmt, lw.gu[0], lw.gu[1],
                                        self._ws_rows(self.ws_h2, r0), self.act[r0:r0 + n], n,
                                        c.ffn, H)
                ops.gemm_kquant_a(dn_fmt, self.act, lw.dn[0], lw.dn[1], self.x, T,
                                  H, c.ffn, self.ws_act)
            res_in, res_out = res_out, self.res[1] if res_out is self.res[0] else self.res[0]
        self.layer_residual = res_in  # residual stream entering the next layer (with self.x)
        # final norm + LM head (fp16 weights, f32 logits)
        if self.head_wt == Lops.WT_BF16:
            # the bf16 head GEMV reads the normalised rows themselves
            norm(self.final_norm, self.ws_f, y_out=self.h2)
            Lops.dense_gemv(Lops.WT_BF16, self.lm_head, self.h2, self.logits, T, c.vocab, H)
        else:
            norm(self.final_norm, self.ws_f)
            if self.head_wt == HEAD_KQUANT:
                ops.gemm_kquant_a_prepared(self.head_fmt, self.lm_head[0], self.lm_head[1],
                                           self.logits, T, c.vocab, H, self.ws_f)
            else:
                Lops.dense_gemv(Lops.WT_F16, self.lm_head, self.ws_f, self.logits, T, c.vocab, H)
        self.final_residual = res_out
        return self.logits

    def _ws_rows(self, ws, r0):
        """The operand-workspace view whose first tile is rows r0.. (r0 a multiple of 16 or
        0): the workspace is laid out per 16-row tile."""
        if r0 % 16:
            raise SnowLLMError("row chunks start on 16-row tiles")
        return ws[(r0 // 16) * self.ws_tile:]


class Acceptance:
    """Rejection-sampling acceptance of the block against draft probabilities q (the draft
    side's proposal) over the full vocabulary at temperature 1 (snowllm/engine/
    dflash_sampling.py:60-69): straight from the logits (ops.dflash.accept_reject), which
    gives the bits of ops.sampling.probabilities + ops.dflash.reject. For a tree block the
    chain rows[0..k] is accepted. batch: requests of `block` rows each (logits [batch * block,
    V]), request b's chain at rows b * block + rows. The batch dispatch (greedy / whole
    vocabulary / candidate lists) lives in snowllm_amd.dflash_sampling."""

    def __init__(self, vocab, chain_rows, batch=1, block=None):
        dev = "cuda"
        self.rows = list(chain_rows)
        T = len(self.rows)
        k = T - 1
        B = batch
        block = T if block is None else block
        self.V, self.T, self.B, self.block = vocab, T, B, block
        n = B * T
        self.top_k = torch.full((n,), ops.SAMPLING_MAX_K, dtype=torch.int32, device=dev)
        self.top_p = torch.ones(n, device=dev)
        self.temp = torch.ones(n, device=dev)
        self.p = torch.empty(n, vocab, device=dev)
        self.pid = torch.empty(n, vocab, dtype=torch.int64, device=dev)
        self.ws = torch.empty(ops.sample_workspace_bytes(n, vocab, vocab), dtype=torch.uint8, device=dev)
        self.q = torch.empty(B, k, vocab, device=dev)
        self.qid = torch.arange(vocab, dtype=torch.int64, device=dev).repeat(B, k, 1).contiguous()
        self.drafts = torch.zeros(B, k, dtype=torch.int64, device=dev)
        self.uniform = torch.zeros(B, T, device=dev)
        self.slot = torch.arange(B, dtype=torch.int32, device=dev)
        self.valid = torch.ones(B, dtype=torch.int32, device=dev)
        self.out = torch.empty(B, T, dtype=torch.int64, device=dev)
        self.accepted = torch.empty(B, dtype=torch.int64, device=dev)
        self.chain_logits = None
        if self.rows != list(range(block)) or B * T != B * block:
            self.chain_logits = torch.empty(n, vocab, device=dev)
            self.chain_index = torch.tensor([b * block + r for b in range(B) for r in self.rows],
                                            dtype=torch.int64, device=dev)

    def set_draft(self, draft_logits, drafts, uniform):
        """Draft side (outside the step): q = softmax(draft logits) over the vocabulary.
        draft_logits [batch * k, V], drafts [batch, k], uniform [batch, k + 1]."""
        k, B = self.T - 1, self.B
        ones = torch.ones(B * k, device="cuda")
        qid = torch.empty(B * k, self.V, dtype=torch.int64, device="cuda")
        q = self.q.view(B * k, self.V)
        ops.probabilities(draft_logits, self.top_k[:B * k], ones, ones, self.V, q, qid, self.ws)
        self.drafts.copy_(drafts.view(B, k))
        self.uniform.copy_(uniform.view(B, self.T))

    def set_selector(self, hp, draft_logits, pred, succ, anchor, temperature, select_uniform,
                     uniform):
        """Draft side inside the step: the DFlash 2 selector walks the draft logits and
        proposes the drafts with their 16-candidate probabilities (snowllm/engine/
        dflash_sampling.py:44-48); the rejection step then reads those candidate lists by
        request slot. hp [k, rank], draft_logits [k, V], codebooks [V, rank], anchor [1],
        temperature [1], select_uniform [1, k], uniform [1, k + 1]."""
        k, B = self.T - 1, self.B
        dev = "cuda"
        self.sel = dict(hp=hp, logits=draft_logits, pred=pred, succ=succ,
                        anchor=anchor.view(B), temperature=temperature.view(B),
                        uniform=select_uniform.view(B, k))
        self.q = torch.empty(B, k, 16, device=dev)
        self.qid = torch.empty(B, k, 16, dtype=torch.int64, device=dev)
        self.sel_scratch = torch.empty(ops.dflash.select_scratch_bytes(B * k), dtype=torch.uint8,
                                       device=dev)
        self.uniform.copy_(uniform.view(B, self.T))

    def propose(self, block_ids=None):
        """Run the selector: drafts, candidate ids and q for this step; block_ids [k + 1], if
        given, receives anchor + drafts (the verify block's input ids)."""
        s = self.sel
        if block_ids is not None and self.B == 1:
            # the walk writes the drafts straight into the block's ids (after the anchor), and
            # the acceptance reads them there: no copy in the step
            self.drafts = block_ids[1:].view(1, self.T - 1)
        ops.dflash.select_path(s["hp"], s["logits"], s["pred"], s["succ"], s["anchor"],
                               self.drafts, self.sel_scratch, temperature=s["temperature"],
                               uniform=s["uniform"], slots=self.slot, candidate_ids=self.qid,
                               probabilities=self.q)
        if block_ids is not None and self.B > 1:
            # each request's block: its anchor, then its drafts
            block_ids.view(self.B, self.block)[:, 1:self.T].copy_(self.drafts)
        return self.drafts

    def __call__(self, logits):
        src = logits
        if self.chain_logits is not None:
            torch.index_select(logits, 0, self.chain_index, out=self.chain_logits)
            src = self.chain_logits
        elif logits.shape[0] != self.B * self.T:
            src = logits[:self.B * self.T]  # chain = leading rows (contiguous view)
        # the whole vocabulary at T = 1: straight from the logits (the same bits as
        # probabilities + reject, which runs when the shape is beyond the fused kernel)
        if ops.dflash.accept_reject(src, self.drafts, self.qid, self.q, self.slot, self.valid,
                                    self.uniform, self.out, self.accepted,
                                    temperature=self.temp):
            return self.out, self.accepted
        ops.probabilities(src, self.top_k, self.top_p, self.temp, self.V, self.p, self.pid, self.ws)
        ops.dflash.reject(self.p, self.pid, self.drafts, self.qid, self.q, self.slot, self.valid,
                          self.uniform, self.out, self.accepted)
        return self.out, self.accepted

"""Test helpers: build paged KV pools in the reference layout from dense K/V and read them
back (the reader restates tests/test_lfm2_dspark_reference.py:30-36)."""
import torch

from oracle.model import cache_rows  # noqa: F401  (re-exported for the tests)

PAGE = 16


def pools_from_dense(k, v, table, num_blocks):
    """k, v: bf16 [L, Hkv, D] -> (k_pool [blocks, Hkv, D/16, 16, 16], v_pool [blocks, Hkv, 4, D, 4])."""
    L, H, D = k.shape
    npages = (L + PAGE - 1) // PAGE
    pad = npages * PAGE - L
    if pad:
        k = torch.cat([k, k.new_zeros(pad, H, D)])
        v = torch.cat([v, v.new_zeros(pad, H, D)])
    kp = torch.zeros(num_blocks, H, D // 16, PAGE, 16, dtype=k.dtype, device=k.device)
    vp = torch.zeros(num_blocks, H, PAGE // 4, D, 4, dtype=v.dtype, device=v.device)
    blocks = table[:npages].long()
    kp[blocks] = k.view(npages, PAGE, H, D // 16, 16).permute(0, 2, 3, 1, 4)
    vp[blocks] = v.view(npages, PAGE // 4, 4, H, D).permute(0, 3, 1, 4, 2)
    return kp, vp


def tree_masks(parents):
    """Ancestor bit masks for a block given each row's parent (-1 for the root)."""
    masks = []
    for i, p in enumerate(parents):
        m = 1 << i
        if p >= 0:
            m |= masks[p]
        masks.append(m)
    return masks


def to_i64(masks):
    """uint64 bit patterns as int64 values (same bits)."""
    return [m - (1 << 64) if m >= 1 << 63 else m for m in masks]

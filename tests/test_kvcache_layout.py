"""CPU: the pool writer used by the tests inverts the reference's own pool reader."""
import torch

from tests.kvcache import cache_rows, pools_from_dense, tree_masks


def test_pools_roundtrip_through_reference_reader():
    g = torch.Generator().manual_seed(0)
    L, H, D = 100, 2, 64
    k = torch.randn(L, H, D, generator=g).bfloat16()
    v = torch.randn(L, H, D, generator=g).bfloat16()
    npages = (L + 15) // 16
    table = torch.randperm(20, generator=g)[:npages].int()
    kp, vp = pools_from_dense(k, v, table, 20)
    assert torch.equal(cache_rows(kp, table.long(), H, D, 16, key=True)[:L], k)
    assert torch.equal(cache_rows(vp, table.long(), H, D, 16, key=False)[:L], v)


def test_tree_masks_width2_depth5():
    parents = [-1, 0, 1, 2, 3, 4, 0, 6, 7, 8, 9]
    m = tree_masks(parents)
    assert m[0] == 1 and m[5] == 0b111111 and m[6] == 0b1000001 and m[10] == 0b11111000001

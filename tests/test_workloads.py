"""Host-side checks of the synthetic workload helpers the bench and the GPU tests build on."""

import torch

from kvskip_amd import workloads as W


def test_paged_pools_hold_every_token_at_its_table_page():
    """paged_pools: token t of sequence b (each copy) is row t % 64 of page table[b, t // 64]; the
    table's pages are distinct; rows past T and unused pages are zero."""
    g = torch.Generator().manual_seed(3)
    B, Hkv, T, D = 2, 3, 200, 8
    ks = [torch.randn(B, Hkv, T, D, generator=g) for _ in range(2)]
    vs = [torch.randn(B, Hkv, T, D, generator=g) for _ in range(2)]
    table, kps, vps = W.paged_pools(ks, vs, seed=5, extra=3)
    nb = (T + 63) // 64
    assert table.dtype == torch.int32 and tuple(table.shape) == (B, nb)
    assert len(set(table.flatten().tolist())) == B * nb
    for c in range(2):
        assert tuple(kps[c].shape) == (B * nb + 3, Hkv, 64, D)
        for b in range(B):
            for t in range(T):
                pg = int(table[b, t // 64])
                assert torch.equal(kps[c][pg, :, t % 64], ks[c][b, :, t])
                assert torch.equal(vps[c][pg, :, t % 64], vs[c][b, :, t])
            last = int(table[b, nb - 1])
            assert (kps[c][last, :, T - 64 * (nb - 1):] == 0).all()
        unused = sorted(set(range(B * nb + 3)) - set(table.flatten().tolist()))
        assert len(unused) == 3 and (kps[c][unused] == 0).all() and (vps[c][unused] == 0).all()

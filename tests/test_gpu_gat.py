"""GPU parity: HIP GAT attention forward/backward vs the oracle (PyG GATConv semantics)."""

import pytest
import torch

import oracle
from grinnder_amd.aggregation import gat_attention
from grinnder_amd.data.adjacency import Adjacency
from tests.graphs import TOL, max_abs_norm_err, random_bipartite

pytestmark = pytest.mark.gpu

CASES = [
    # (B, E, avg_deg, long_rows, heads, channels, concat)
    (200, 300, 6, 0, 1, 16, True),
    (300, 500, 10, 2, 1, 256, True),
    (300, 420, 8, 1, 1, 19, False),
    (250, 400, 9, 1, 8, 4, True),
    (250, 400, 9, 0, 4, 7, False),
    (150, 260, 12, 2, 2, 64, True),
    (100, 140, 5, 0, 3, 100, True),
]


@pytest.mark.parametrize("B,E,deg,longs,H,C,concat", CASES)
def test_gat_forward_backward_matches_oracle(gpu, B, E, deg, longs, H, C, concat):
    print(f"case B={B} E={E} H={H} C={C} concat={concat}", flush=True)
    rowptr, col, val = random_bipartite(B, E, deg, seed=B * 7 + C, long_rows=longs,
                                        long_len=1200)
    adj = Adjacency(rowptr, col, val, (B, E), seg_len=512)
    g = torch.Generator().manual_seed(H * 100 + C)
    hs = torch.randn(E, H * C, generator=g)
    att_src = torch.randn(1, H, C, generator=g) * 0.5
    att_dst = torch.randn(1, H, C, generator=g) * 0.5
    out_w = H * C if concat else C
    bias = torch.randn(out_w, generator=g)
    gy = torch.randn(B, out_w, generator=g)

    hs_d = hs.to(gpu).requires_grad_(True)
    as_d = att_src.to(gpu).requires_grad_(True)
    ad_d = att_dst.to(gpu).requires_grad_(True)
    b_d = bias.to(gpu).requires_grad_(True)
    y = gat_attention(hs_d, adj, as_d, ad_d, b_d, H, C, concat)
    y.backward(gy.to(gpu))
    torch.cuda.synchronize()

    ref_y, alpha, tpre = oracle.gat_forward(rowptr, col, hs, H, C, att_src, att_dst, bias, concat)
    dhs, das, dad, db = oracle.gat_backward(rowptr, col, hs, H, C, att_src, att_dst, concat,
                                            alpha, tpre, gy)
    assert max_abs_norm_err(y.detach(), ref_y) <= TOL
    assert max_abs_norm_err(hs_d.grad, dhs) <= TOL
    assert max_abs_norm_err(as_d.grad.reshape(-1), das) <= TOL
    assert max_abs_norm_err(ad_d.grad.reshape(-1), dad) <= TOL
    assert max_abs_norm_err(b_d.grad, db) <= TOL


def test_gat_deterministic(gpu):
    rowptr, col, val = random_bipartite(400, 600, 20, seed=11, long_rows=3, long_len=2500)
    adj = Adjacency(rowptr, col, val, (400, 600), seg_len=256)
    g = torch.Generator().manual_seed(5)
    hs = torch.randn(600, 64, generator=g).to(gpu).requires_grad_(True)
    a_s = torch.randn(1, 1, 64, generator=g).to(gpu).requires_grad_(True)
    a_d = torch.randn(1, 1, 64, generator=g).to(gpu).requires_grad_(True)
    outs = []
    for _ in range(2):
        hs.grad = None
        y = gat_attention(hs, adj, a_s, a_d, None, 1, 64, True)
        y.sum().backward()
        outs.append((y.detach().clone(), hs.grad.clone()))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])

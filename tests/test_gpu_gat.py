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
    # one head, narrow: several rows (forward) / columns (backward) per wavefront
    (2000, 2600, 7, 3, 1, 20, True),
    (1500, 1800, 4, 2, 1, 8, True),
    (1200, 1300, 11, 1, 1, 64, True),
    (900, 1000, 6, 2, 1, 3, True),
    (700, 900, 9, 1, 1, 13, True),
    (600, 800, 3, 0, 1, 48, True),
    # rows and columns on both sides of the narrow kernels' length limits
    # (16 edges for at most 4 vectors, 32 otherwise)
    (700, 800, 30, 2, 1, 20, True),
    (600, 600, 16, 1, 1, 12, True),
    (650, 700, 31, 1, 1, 13, True),
    # packed-line kernels (one head, a multiple of 4 up to 24 channels) at
    # their widest and narrowest
    (800, 800, 9, 2, 1, 24, True),
    (500, 700, 6, 1, 1, 4, True),
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


@pytest.mark.parametrize("C,long_len,seg", [(256, 1200, 512), (19, 700, 256), (3, 300, 128),
                                            (64, 2000, 512), (300, 900, 512), (301, 600, 512),
                                            (1024, 0, 512)])
def test_gat_forward_fused_matches_two_pass(gpu, C, long_len, seg):
    """gr_gat_forward (one fused pass for one head) against gr_gat_softmax_stats
    + gr_gat_aggregate through the C ABI: m, den, alpha and O bit-identical on
    whole rows; split rows (combined with rescaled partials) within TOL."""
    from grinnder_amd import _lib
    B, E = 300, 420
    print(f"case C={C} long_len={long_len} seg={seg}", flush=True)
    rowptr, col, val = random_bipartite(B, E, 9, seed=C, long_rows=3 if long_len else 0,
                                        long_len=long_len)
    adj = Adjacency(rowptr, col, val, (B, E), seg_len=seg)
    plan = adj.device_plan(gpu)
    f = plan.fwd
    g = torch.Generator().manual_seed(C)
    hs = torch.randn(E, C, generator=g).to(gpu)
    s = (torch.randn(E, 1, generator=g) * 2).to(gpu)
    d = (torch.randn(B, 1, generator=g) * 2).to(gpu)
    bias = torch.randn(C, generator=g).to(gpu)
    nnz = plan.nnz
    st = _lib.stream_handle()
    fixp = f.fixups.data_ptr() if f.n_fix else None
    c4 = (C + 3) // 4 * 4
    outs = []
    for fused in (False, True):
        m = torch.full((B, 1), float("nan"), device=gpu)
        den = torch.full((B, 1), float("nan"), device=gpu)
        alpha = torch.full((max(nnz, 1), 1), float("nan"), device=gpu)
        o = torch.full((B, C), float("nan"), device=gpu)
        y = torch.full((B, C), float("nan"), device=gpu)
        ws = torch.empty(max(1, f.n_slots) * (c4 + 4), device=gpu)
        if fused:
            _lib.call("gr_gat_forward", f.units.data_ptr(), f.n_units, fixp, f.n_fix,
                      plan.idx.data_ptr(), hs.data_ptr(), C, s.data_ptr(), d.data_ptr(), B, 1, C,
                      bias.data_ptr(), m.data_ptr(), den.data_ptr(), alpha.data_ptr(),
                      o.data_ptr(), y.data_ptr(), C, ws.data_ptr(), ws.numel(), f.n_slots, st)
        else:
            _lib.call("gr_gat_softmax_stats", f.units.data_ptr(), f.n_units, fixp, f.n_fix,
                      plan.idx.data_ptr(), s.data_ptr(), d.data_ptr(), 1, m.data_ptr(),
                      den.data_ptr(), alpha.data_ptr(), ws.data_ptr(), f.n_slots, st)
            _lib.call("gr_gat_aggregate", f.units.data_ptr(), f.n_units, fixp, f.n_fix,
                      plan.idx.data_ptr(), hs.data_ptr(), C, alpha.data_ptr(), B, 1, C,
                      bias.data_ptr(), o.data_ptr(), y.data_ptr(), C, ws.data_ptr(), f.n_slots,
                      st)
        torch.cuda.synchronize()
        outs.append([t.cpu() for t in (m, den, alpha[:nnz], o, y)])
    deg = rowptr[1:] - rowptr[:-1]
    split = deg > seg
    edge_split = torch.repeat_interleave(split, deg)
    assert (f.n_fix > 0) == bool(split.any())
    (m0, den0, a0, o0, y0), (m1, den1, a1, o1, y1) = outs
    for t in (m1, den1, a1, o1, y1):
        assert not torch.isnan(t).any()
    whole = ~split
    # Narrow rows (at most 16 vectors) run several per wavefront and sum in
    # groups of lanes, not in a 64-lane tree: the same values up to rounding.
    narrow = (C % 4 == 0 and C // 4 <= 16) or C <= 16
    if narrow:
        assert torch.equal(m0[whole], m1[whole])
        for a, b in ((den0[whole], den1[whole]), (a0[~edge_split], a1[~edge_split]),
                     (o0[whole], o1[whole]), (y0[whole], y1[whole])):
            assert max_abs_norm_err(b, a.double()) <= TOL
    else:
        assert torch.equal(m0[whole], m1[whole]) and torch.equal(den0[whole], den1[whole])
        assert torch.equal(a0[~edge_split], a1[~edge_split])
        assert torch.equal(o0[whole], o1[whole]) and torch.equal(y0[whole], y1[whole])
    # Split rows: the same statistics formula, O from rescaled partial sums.
    assert torch.equal(m0[split], m1[split]) and torch.equal(den0[split], den1[split])
    assert max_abs_norm_err(a1[edge_split], a0[edge_split].double()) <= TOL
    assert max_abs_norm_err(o1, o0.double()) <= TOL
    assert max_abs_norm_err(y1, y0.double()) <= TOL
    # Rows without edges: m = 0, den = 1, O = 0, Y = bias.
    empty = deg == 0
    assert bool(empty.any())
    assert torch.equal(m1[empty], torch.zeros(int(empty.sum()), 1))
    assert torch.equal(den1[empty], torch.ones(int(empty.sum()), 1))
    assert torch.equal(o1[empty], torch.zeros(int(empty.sum()), C))
    assert torch.equal(y1[empty], bias.cpu().expand(int(empty.sum()), C))


@pytest.mark.parametrize("H,C", [(1, 256), (1, 20), (1, 7), (2, 16)])
def test_gat_hub_source_matches_oracle(gpu, H, C):
    """A source column shared by most destination rows (an R-MAT hub):
    its CSC column is longer than the segment length, so the backward's
    split-column fixup runs, next to short columns."""
    print(f"case hub H={H} C={C}", flush=True)
    B, E = 900, 1500
    rowptr, col, val = random_bipartite(B, E, 6, seed=C + H, long_rows=1, long_len=700)
    rows = torch.repeat_interleave(torch.arange(B), rowptr[1:] - rowptr[:-1])
    g = torch.Generator().manual_seed(3)
    hub = (torch.rand(col.numel(), generator=g) < 0.5) & (rows % 3 != 0)
    col = torch.where(hub, torch.full_like(col, 11), col)
    adj = Adjacency(rowptr, col, val, (B, E), seg_len=128)
    assert int((col == 11).sum()) > 128
    hs = torch.randn(E, H * C, generator=g)
    att_src = torch.randn(1, H, C, generator=g) * 0.5
    att_dst = torch.randn(1, H, C, generator=g) * 0.5
    bias = torch.randn(H * C, generator=g)
    gy = torch.randn(B, H * C, generator=g)
    hs_d = hs.to(gpu).requires_grad_(True)
    as_d = att_src.to(gpu).requires_grad_(True)
    ad_d = att_dst.to(gpu).requires_grad_(True)
    b_d = bias.to(gpu).requires_grad_(True)
    y = gat_attention(hs_d, adj, as_d, ad_d, b_d, H, C, True)
    y.backward(gy.to(gpu))
    torch.cuda.synchronize()
    ref_y, alpha, tpre = oracle.gat_forward(rowptr, col, hs, H, C, att_src, att_dst, bias, True)
    dhs, das, dad, db = oracle.gat_backward(rowptr, col, hs, H, C, att_src, att_dst, True,
                                            alpha, tpre, gy)
    assert max_abs_norm_err(y.detach(), ref_y) <= TOL
    assert max_abs_norm_err(hs_d.grad, dhs) <= TOL
    assert max_abs_norm_err(as_d.grad.reshape(-1), das) <= TOL
    assert max_abs_norm_err(ad_d.grad.reshape(-1), dad) <= TOL
    assert max_abs_norm_err(b_d.grad, db) <= TOL


@pytest.mark.parametrize("rows,H,C", [(1000, 1, 256), (777, 1, 20), (500, 4, 64), (300, 3, 7),
                                      (5, 1, 1024), (0, 1, 8)])
def test_gat_row_dot_matches_fp64(gpu, rows, H, C):
    """cdot[r,h] = <a[r,h,:], b[r,h,:]> (the backward's <GO_i, O_i>)."""
    from grinnder_amd import _lib
    g = torch.Generator().manual_seed(rows + C)
    a = torch.randn(rows, H * C + 4, generator=g)[:, :H * C]   # row stride H*C + 4
    b = torch.randn(rows, H * C, generator=g)
    a_d, b_d = a.to(gpu), b.to(gpu)
    out = torch.full((max(rows, 1), H), float("nan"), device=gpu)
    _lib.call("gr_gat_row_dot", a_d.data_ptr(), a_d.stride(0), b_d.data_ptr(), H * C, rows, H,
              C, out.data_ptr(), _lib.stream_handle())
    torch.cuda.synchronize()
    if rows == 0:
        return
    ref = (a.double().view(rows, H, C) * b.double().view(rows, H, C)).sum(-1)
    assert max_abs_norm_err(out.cpu(), ref) <= TOL


@pytest.mark.parametrize("C,big", [(256, False), (128, False), (256, True)])
def test_gat_attention_in_place_matches_gathered(gpu, C, big):
    """One head read in place (the projected flow's ProjectedSink: edge
    sources as global rows of Z, dHs added into dZ at the partition's rows)
    gives the same output, dZ, att_dst and bias gradients, bit for bit, as
    the same partition on its gathered rows of Z with the gradient scattered
    back.  The in-place backward forms att_src's gradient from per-wavefront
    partial sums (the same sum, re-associated): within TOL of the gathered
    form's and of a float64 sum over the edges.  `big`: more source columns
    than the GPU holds wavefronts, so each wavefront takes several, and hub
    columns split into several units."""
    from grinnder_amd.aggregation import ProjectedSink, gat_scores
    if big:
        N, B, E, lo = 150_000, 20_000, 70_000, 40_000
    else:
        N, B, E, lo = 3000, 500, 1400, 700
    print(f"case C={C} N={N} B={B} E={E}", flush=True)
    rowptr, col, val = random_bipartite(B, E, 9, seed=C, long_rows=2, long_len=900)
    if big:
        # Three hub source columns of about 2,000 edges each (split in the CSC plan).
        g0 = torch.Generator().manual_seed(7)
        hub = torch.rand(col.numel(), generator=g0) < 6000 / col.numel()
        col[hub] = torch.tensor([B + 11, B + 23, B + 37])[torch.randint(0, 3, (int(hub.sum()),),
                                                                          generator=g0)]
    adj = Adjacency(rowptr, col, val, (B, E), seg_len=512)
    g = torch.Generator().manual_seed(C)
    others = torch.cat([torch.arange(0, lo), torch.arange(lo + B, N)])
    rows = torch.cat([torch.arange(lo, lo + B),
                      others[torch.randperm(others.numel(), generator=g)[:E - B]]])
    z = torch.randn(N, C, generator=g).to(gpu)
    att_s = (0.5 * torch.randn(1, 1, C, generator=g)).to(gpu)
    att_d = (0.5 * torch.randn(1, 1, C, generator=g)).to(gpu)
    bias = torch.randn(C, generator=g).to(gpu)
    gy = torch.randn(B, C, generator=g).to(gpu)
    s_all, d_all = gat_scores(z, att_s, att_d, 1, C, N)
    rg = rows.to(gpu)
    outs = []
    for in_place in (False, True):
        a_s = att_s.clone().requires_grad_(True)
        a_d = att_d.clone().requires_grad_(True)
        b = bias.clone().requires_grad_(True)
        dz = torch.zeros(N, C, device=gpu)
        if in_place:
            sink = ProjectedSink(dz, rows[col].to(torch.int32).to(gpu), rg.to(torch.int32),
                                 torch.zeros(0, device=gpu, requires_grad=True), lo)
            y = gat_attention(z, adj, a_s, a_d, b, 1, C, True,
                              scores=(s_all, d_all[lo:lo + B]), sink=sink)
            y.backward(gy)
        else:
            hs = z[rg].clone().requires_grad_(True)
            y = gat_attention(hs, adj, a_s, a_d, b, 1, C, True,
                              scores=(s_all[rg], d_all[lo:lo + B]))
            y.backward(gy)
            dz.index_add_(0, rg, hs.grad)
        torch.cuda.synchronize()
        outs.append((y.detach(), dz, a_s.grad, a_d.grad, b.grad))
    (y0, dz0, as0, ad0, b0), (y1, dz1, as1, ad1, b1) = outs
    for t0, t1 in ((y0, y1), (dz0, dz1), (ad0, ad1), (b0, b1)):
        assert torch.equal(t0, t1)
    assert max_abs_norm_err(as1, as0.double()) <= TOL
    if big:
        return
    # float64: the oracle's backward on the gathered rows.  (The big case
    # leaves it out: among its 190k edges a LeakyReLU tie, a logit within
    # fp32 rounding of 0, may take the other slope in float64.)
    hs64 = z[rg].cpu()
    ref_o, alpha, tpre = oracle.gat_forward(rowptr, col, hs64, 1, C, att_s.cpu(), att_d.cpu(),
                                            bias.cpu(), True)
    back = oracle.gat_backward(rowptr, col, hs64, 1, C, att_s.cpu(), att_d.cpu(), True, alpha,
                               tpre, gy.cpu())
    assert max_abs_norm_err(as1.view(-1), torch.as_tensor(back[1]).view(-1)) <= TOL


@pytest.mark.parametrize("C,square,with_bias", [(20, True, True), (20, False, True),
                                                (24, True, True), (8, False, True),
                                                (20, False, False), (4, True, False)])
def test_gat_narrow_path_runs_and_matches_oracle_with_scores(gpu, C, square, with_bias,
                                                             monkeypatch):
    """One head of C <= 24 channels (a multiple of 4) runs the packed-line
    kernels (gr_gat_narrow_forward / _backward), not the general ones, with
    the logit halves formed inside, given (as the projected flow gives
    them, gat_scores over all rows), or given with the packed lines
    (gat_scores(packed=True), as a merged layer gives them): all three give
    the same bits, and match the oracle, including split rows and columns
    (hub rows of 1500 edges at a 256-edge segment), rows past the
    destinations (E > B), and a layer without bias (O itself is the output
    and what the backward reads)."""
    from grinnder_amd import _lib
    from grinnder_amd.aggregation import gat_scores

    B, E = (900, 900) if square else (700, 1000)
    rowptr, col, val = random_bipartite(B, E, 10, seed=C + int(square), long_rows=3,
                                        long_len=1500)
    adj = Adjacency(rowptr, col, val, (B, E), seg_len=256)
    g = torch.Generator().manual_seed(C)
    hs = torch.randn(E, C, generator=g)
    a_s = torch.randn(1, 1, C, generator=g) * 0.5
    a_d = torch.randn(1, 1, C, generator=g) * 0.5
    b = torch.randn(C, generator=g)
    gy = torch.randn(B, C, generator=g)
    called = []
    real = _lib.call
    monkeypatch.setattr(_lib, "call", lambda name, *a: (called.append(name), real(name, *a))[1])
    results = []
    for given in ("inside", "scores", "packed"):
        leaves = [t.to(gpu).requires_grad_(True) for t in (hs, a_s, a_d, b)]
        scores = None
        if given != "inside":
            scores = gat_scores(leaves[0].detach(), leaves[1], leaves[2], 1, C, B,
                                packed=given == "packed")
            assert len(scores) == (3 if given == "packed" else 2)
        out = gat_attention(leaves[0], adj, leaves[1], leaves[2],
                            leaves[3] if with_bias else None, 1, C, True, scores=scores)
        out.backward(gy.to(gpu))
        torch.cuda.synchronize()
        results.append([out.detach()] + [t.grad for t in leaves[:3]]
                       + ([leaves[3].grad] if with_bias else []))
    assert "gr_gat_narrow_forward" in called and "gr_gat_narrow_backward" in called
    assert "gr_gat_narrow_pack" in called
    assert "gr_gat_forward" not in called
    for other in results[1:]:
        for a, c in zip(results[0], other):
            assert torch.equal(a, c)
    ref_o, alpha, tpre = oracle.gat_forward(rowptr, col, hs, 1, C, a_s, a_d,
                                            b if with_bias else None, True)
    refs = oracle.gat_backward(rowptr, col, hs, 1, C, a_s, a_d, True, alpha, tpre, gy)
    got = results[0]
    assert max_abs_norm_err(got[0], ref_o) <= TOL
    for t, r in zip(got[1:], refs):
        assert max_abs_norm_err(t.reshape(-1), torch.as_tensor(r).reshape(-1)) <= TOL


@pytest.mark.parametrize("C,longs", [(256, 3), (132, 0), (1024, 1)])
def test_gat_attention_ln_matches_attention_then_epilogue(gpu, C, longs):
    """gat_attention_ln (the attention kernel storing act(LN(O + bias))
    straight from its accumulators, gr_gat_forward_ln) against the two-step
    form it replaces in the GAT model, gat_attention then bias_ln_act: output
    and every gradient (hs, attention vectors, conv bias, LayerNorm gamma and
    beta) within TOL, and with whole rows only (no split rows) the output
    bit-identical, since both form the row statistics with the same code
    from the same h.  Split rows (longs > 0: hub rows of 1500 edges at a
    256-edge segment) finish in their own fixup."""
    from grinnder_amd.aggregation import RowDotSink, gat_attention_ln
    from grinnder_amd.dense import bias_ln_act

    B, E = 600, 900
    rowptr, col, val = random_bipartite(B, E, 12, seed=C, long_rows=longs, long_len=1500)
    adj = Adjacency(rowptr, col, val, (B, E), seg_len=256)
    g = torch.Generator().manual_seed(C)
    hs = torch.randn(E, C, generator=g)
    a_s = torch.randn(1, 1, C, generator=g) / C ** 0.5
    a_d = torch.randn(1, 1, C, generator=g) / C ** 0.5
    b = torch.randn(C, generator=g)
    gamma = 1 + 0.1 * torch.randn(C, generator=g)
    beta = 0.1 * torch.randn(C, generator=g)
    gy = torch.randn(B, C, generator=g)
    res = []
    for fused in (True, False):
        leaves = [t.to(gpu).requires_grad_(True) for t in (hs, a_s, a_d, b, gamma, beta)]
        if fused:
            out = gat_attention_ln(leaves[0], adj, leaves[1], leaves[2], leaves[3], leaves[4],
                                   leaves[5], 1e-5, "elu")
        else:
            dot = RowDotSink()
            x = gat_attention(leaves[0], adj, leaves[1], leaves[2], None, 1, C, True,
                              rowdot_sink=dot)
            out = bias_ln_act(x, leaves[3], leaves[4], leaves[5], 1e-5, "elu", dot)
        out.backward(gy.to(gpu))
        torch.cuda.synchronize()
        res.append([out.detach()] + [t.grad for t in leaves])
    names = ["out", "hs", "att_src", "att_dst", "bias", "gamma", "beta"]
    for name, a, c in zip(names, res[0], res[1]):
        err = max_abs_norm_err(a.reshape(-1), c.reshape(-1))
        print(f"C={C} longs={longs} {name}: {err:.1e}", flush=True)
        assert err <= TOL, name
    if longs == 0:
        assert torch.equal(res[0][0], res[1][0])

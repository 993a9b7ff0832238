"""GPU: the dense per-layer transform — split-K weight-gradient GEMM
(gr_gemm_tn), the forward / input-gradient GEMM (gr_gemm_nt), the Linear
autograd function built on them, and the dense
bias + LayerNorm + ReLU/ELU epilogue (gr_bias_ln_act) — against float64 torch.
fp32 tolerance: max-abs-normalised error <= 1e-5 (TOL)."""

import pytest
import torch

from grinnder_amd import _lib
from grinnder_amd.dense import (bias_ln_act, bias_ln_relu, gemm_nt, gemm_tn, gemm_tn_splits,
                                linear)
from tests.graphs import TOL, max_abs_norm_err

pytestmark = pytest.mark.gpu


def _randn(*shape, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dev)


@pytest.mark.parametrize("k,m,n", [(0, 5, 7), (1, 1, 1), (37, 3, 5), (1000, 47, 256),
                                   (5000, 256, 100), (3001, 130, 129), (200_000, 256, 256),
                                   (70_000, 47, 256), (20_000, 256, 48), (20_000, 48, 100),
                                   (5000, 64, 256), (0, 48, 256), (20_000, 256, 20),
                                   (30_000, 19, 256), (5000, 32, 300), (777, 130, 3)])
def test_gemm_tn_matches_fp64(gpu, k, m, n):
    """Covers 128-, 64- and 32-column tiles and the transposed narrow path
    (m <= 64 < n), 32-column tiles with 4-byte loads of the narrow side.  At
    these K the 128- and 64-column tiles run on 32 x 32 blocks (ragged at
    130 x 129); the 16 x 16 form of the 128-column tiles is taken past
    2^22 rows (the K = 10M test below)."""
    a = _randn(k, m, seed=k + m, dev=gpu)
    b = _randn(k, n, seed=k + n + 1, dev=gpu)
    c = gemm_tn(a, b)
    ref = a.double().t() @ b.double()
    if k == 0:
        assert torch.equal(c.cpu(), torch.zeros(m, n))
    else:
        assert max_abs_norm_err(c, ref) <= TOL


@pytest.mark.parametrize("m,n", [(256, 256), (20, 256)])
def test_gemm_tn_at_ten_million_rows(gpu, m, n):
    """dW = dZᵀ X over K = 10,000,000 node rows, the reduction length of the
    merged layers' weight gradients at C4/C5 (256-wide layer 1, and the
    20-wide padded last layer in its transposed narrow form).  Operands are
    generated on the device; the float64 reference is summed over 1M-row
    slices."""
    k = 10_000_000
    g = torch.Generator(device=gpu).manual_seed(m + n)
    a = torch.randn(k, m, device=gpu, generator=g)
    b = torch.randn(k, n, device=gpu, generator=g)
    c = gemm_tn(a, b)
    ref = torch.zeros(m, n, dtype=torch.float64, device=gpu)
    for lo in range(0, k, 1 << 20):
        ref += a[lo:lo + (1 << 20)].double().t() @ b[lo:lo + (1 << 20)].double()
    err = max_abs_norm_err(c, ref)
    print(f"gemm_tn K={k} {m}x{n}: {err:.1e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("splits", [1, 3, 8, 64, 1000])
def test_gemm_tn_split_counts(gpu, splits):
    """Any split count gives the same product (chunks of 16-row steps)."""
    a = _randn(20_000, 64, seed=1, dev=gpu)
    b = _randn(20_000, 200, seed=2, dev=gpu)
    c = gemm_tn(a, b, splits=splits)
    assert max_abs_norm_err(c, a.double().t() @ b.double()) <= TOL


def test_gemm_tn_strided_beta_and_determinism(gpu):
    big_a = _randn(9000, 300, seed=3, dev=gpu)
    big_b = _randn(9000, 260, seed=4, dev=gpu)
    a, b = big_a[:, 17:273], big_b[:, :256]  # lda = 300, ldb = 260, offset rows
    c0 = _randn(256, 256, seed=5, dev=gpu)
    c = c0.clone()
    gemm_tn(a, b, out=c, beta=0.5)
    ref = 0.5 * c0.double() + a.double().t() @ b.double()
    assert max_abs_norm_err(c, ref) <= TOL
    again = gemm_tn(a, b)
    assert torch.equal(again, gemm_tn(a, b))  # fixed reduction order


def test_gemm_tn_workspace_checked(gpu):
    a = torch.zeros(100, 8, device=gpu)
    b = torch.zeros(100, 8, device=gpu)
    c = torch.empty(8, 8, device=gpu)
    ws = torch.empty(8 * 8 * 2, device=gpu)
    with pytest.raises(_lib.GrError, match="workspace"):
        _lib.call("gr_gemm_tn", a.data_ptr(), 8, b.data_ptr(), 8, 8, 8, 100, 0.0,
                  c.data_ptr(), ws.data_ptr(), ws.numel(), 7, _lib.stream_handle())


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (37, 7, 3), (1000, 20, 256), (777, 48, 100),
                                   (5000, 256, 1024), (300, 300, 64), (129, 65, 33),
                                   (4096, 16, 20), (70_000, 256, 48), (3000, 1024, 256),
                                   (2500, 47, 256), (513, 130, 1), (100_003, 256, 19),
                                   (5000, 512, 20), (2001, 602, 47), (64, 64, 31), (1, 256, 63),
                                   (70_001, 256, 256), (65_536, 20, 256), (200_003, 48, 100),
                                   (66_000, 128, 12), (70_000, 200, 60), (80_000, 4, 40),
                                   (70_003, 48, 256), (66_001, 100, 256), (65_536, 200, 64),
                                   (131_071, 64, 32), (70_000, 36, 128), (100_000, 128, 32),
                                   (1000, 300, 300), (777, 130, 513), (20_000, 256, 1024)])
@pytest.mark.parametrize("bias", [False, True])
def test_gemm_nt_matches_fp64(gpu, m, n, k, bias):
    """Every tile shape (n > 64, 33..64, 17..32, <= 16), K not a multiple of
    the 32-wide step or of 4 (scalar loads), ragged row and column tiles; the
    short-reduction kernel (k <= 64 not a multiple of 4, n >= 64) with one to
    five 128-column blocks, 8-byte and element stores, k just under its 32
    and 64 register limits; row counts past 65536 with one and two column
    tiles, a partial second tile (n = 200), k below one step and not a
    multiple of the step; the resident-B kernels (m >= 65536, k a multiple
    of 32 up to 256: 16 x 16 blocks for 33..64 columns, 32 x 32 blocks for
    65..256) with one 32-k chunk to eight, one and two column blocks,
    partial blocks (n = 36, 100, 200) and ragged row blocks."""
    a = _randn(m, k, seed=m + k, dev=gpu)
    b = _randn(n, k, seed=n + k + 1, dev=gpu)
    bv = _randn(n, seed=n, dev=gpu) if bias else None
    c = gemm_nt(a, b, bv)
    ref = a.double() @ b.double().t()
    if bias:
        ref += bv.double()
    assert max_abs_norm_err(c, ref) <= TOL


def test_gemm_nt_strided_and_in_place(gpu):
    """Strided a and b rows, an unaligned a (scalar path), and a column slice
    of a wider buffer as `out` (ldc > n): the columns around it are untouched;
    the same call twice gives the same bits."""
    big_a = _randn(9000, 300, seed=3, dev=gpu)
    big_b = _randn(200, 260, seed=4, dev=gpu)
    a, b = big_a[:, 16:272], big_b[:, :256]  # lda = 300, ldb = 260
    buf = _randn(9000, 320, seed=5, dev=gpu)
    before = buf.clone()
    gemm_nt(a, b, out=buf[:, 40:240])
    ref = a.double() @ b.double().t()
    assert max_abs_norm_err(buf[:, 40:240], ref) <= TOL
    assert torch.equal(buf[:, :40], before[:, :40]) and torch.equal(buf[:, 240:], before[:, 240:])
    again = gemm_nt(a, b)
    assert torch.equal(again, gemm_nt(a, b))
    odd = big_a[:, 1:257]  # 4-byte aligned only
    assert max_abs_norm_err(gemm_nt(odd, b), odd.double() @ b.double().t()) <= TOL
    assert gemm_nt(a[:0], b).shape == (0, 200)
    # Short reduction (k = 19) with strided, unaligned a and b, into column
    # slices whose start is 16-byte aligned (vector stores) or not.
    sa, sb = big_a[:, 5:24], big_b[:, 3:22]
    ref = sa.double() @ sb.double().t()
    for c0 in (40, 41):
        buf = _randn(9000, 320, seed=6, dev=gpu)
        before = buf.clone()
        gemm_nt(sa, sb, out=buf[:, c0:c0 + 200])
        assert max_abs_norm_err(buf[:, c0:c0 + 200], ref) <= TOL
        assert torch.equal(buf[:, :c0], before[:, :c0])
        assert torch.equal(buf[:, c0 + 200:], before[:, c0 + 200:])
    with pytest.raises(ValueError, match="out must be"):
        gemm_nt(a, b, out=torch.empty(9000, 199, device=gpu))
    # 70k rows (the resident-B kernel) with strided rows of a and b, a bias,
    # and a column slice of a wider buffer as out.
    big_a = _randn(70_000, 300, seed=7, dev=gpu)
    a = big_a[:, 16:272]
    buf = _randn(70_000, 320, seed=8, dev=gpu)
    before = buf.clone()
    bv = _randn(200, seed=9, dev=gpu)
    gemm_nt(a, b, bv, out=buf[:, 40:240])
    ref = a.double() @ b.double().t() + bv.double()
    assert max_abs_norm_err(buf[:, 40:240], ref) <= TOL
    assert torch.equal(buf[:, :40], before[:, :40]) and torch.equal(buf[:, 240:], before[:, 240:])
    assert torch.equal(gemm_nt(a, b, bv), gemm_nt(a, b, bv))


@pytest.mark.parametrize("rows,fin,fout,bias", [(5000, 100, 256, True), (777, 256, 47, False),
                                                (0, 16, 32, True)])
def test_linear_autograd_matches_fp64(gpu, rows, fin, fout, bias):
    x = _randn(rows, fin, seed=rows, dev=gpu).requires_grad_(True)
    w = _randn(fout, fin, seed=fin, dev=gpu).mul_(0.1).requires_grad_(True)
    b = _randn(fout, seed=fout, dev=gpu).requires_grad_(True) if bias else None
    go = _randn(rows, fout, seed=7, dev=gpu)
    y = linear(x, w, b)
    y.backward(go)
    xd = x.detach().double().requires_grad_(True)
    wd = w.detach().double().requires_grad_(True)
    bd = b.detach().double().requires_grad_(True) if bias else None
    yd = torch.nn.functional.linear(xd, wd, bd)
    yd.backward(go.double())
    if rows == 0:
        assert y.shape == (0, fout) and torch.equal(w.grad.cpu(), torch.zeros(fout, fin))
        return
    assert max_abs_norm_err(y, yd) <= TOL
    assert max_abs_norm_err(x.grad, xd.grad) <= TOL
    assert max_abs_norm_err(w.grad, wd.grad) <= TOL
    if bias:
        assert max_abs_norm_err(b.grad, bd.grad) <= TOL


@pytest.mark.parametrize("rows,dim,bias", [(4000, 256, True), (1500, 47, True), (300, 100, False),
                                           (0, 64, True)])
def test_bias_ln_relu_matches_fp64(gpu, rows, dim, bias):
    z = _randn(rows, dim, seed=dim, dev=gpu).requires_grad_(True)
    b = _randn(dim, seed=1, dev=gpu).requires_grad_(True) if bias else None
    gamma = (1 + 0.1 * _randn(dim, seed=2, dev=gpu)).requires_grad_(True)
    beta = (0.1 * _randn(dim, seed=3, dev=gpu)).requires_grad_(True)
    go = _randn(rows, dim, seed=4, dev=gpu)
    out = bias_ln_relu(z, b, gamma, beta, 1e-5)
    out.backward(go)
    zd = z.detach().double().requires_grad_(True)
    bd = b.detach().double().requires_grad_(True) if bias else None
    gd = gamma.detach().double().requires_grad_(True)
    btd = beta.detach().double().requires_grad_(True)
    h = zd + bd if bias else zd
    ref = torch.relu(torch.nn.functional.layer_norm(h, (dim,), gd, btd, 1e-5))
    ref.backward(go.double())
    if rows == 0:
        assert out.shape == (0, dim)
        return
    assert max_abs_norm_err(out, ref) <= TOL
    assert max_abs_norm_err(z.grad, zd.grad) <= TOL
    assert max_abs_norm_err(gamma.grad, gd.grad) <= TOL
    assert max_abs_norm_err(beta.grad, btd.grad) <= TOL
    if bias:
        assert max_abs_norm_err(b.grad, bd.grad) <= TOL


def test_bias_ln_relu_in_place_h(gpu):
    """h may overwrite z (ldz == dim): same out and h as the out-of-place call."""
    rows, dim = 999, 128
    z = _randn(rows, dim, seed=9, dev=gpu)
    bias = _randn(dim, seed=10, dev=gpu)
    gamma = torch.ones(dim, device=gpu)
    beta = torch.zeros(dim, device=gpu)
    outs = []
    for in_place in (False, True):
        zz = z.clone()
        h = zz if in_place else torch.empty_like(z)
        out = torch.empty_like(z)
        mean = torch.empty(rows, device=gpu)
        rstd = torch.empty(rows, device=gpu)
        _lib.call("gr_bias_ln_act", zz.data_ptr(), dim, bias.data_ptr(), gamma.data_ptr(),
                  beta.data_ptr(), 1e-5, 0, rows, dim, h.data_ptr(), out.data_ptr(),
                  mean.data_ptr(), rstd.data_ptr(), _lib.stream_handle())
        outs.append((h.clone(), out.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][0], z + bias)


def test_default_splits_shape(gpu):
    s, ws = gemm_tn_splits(256, 256, 2_449_029)
    assert s % 8 == 0 and ws == s * 256 * 256


@pytest.mark.parametrize("rows,dim,bias", [(3000, 256, True), (800, 20, False)])
def test_bias_ln_elu_matches_fp64(gpu, rows, dim, bias):
    """The GAT epilogue: ELU(LayerNorm(z + b)) and its gradients."""
    z = _randn(rows, dim, seed=dim + 1, dev=gpu).requires_grad_(True)
    b = _randn(dim, seed=5, dev=gpu).requires_grad_(True) if bias else None
    gamma = (1 + 0.1 * _randn(dim, seed=6, dev=gpu)).requires_grad_(True)
    beta = (0.1 * _randn(dim, seed=7, dev=gpu)).requires_grad_(True)
    go = _randn(rows, dim, seed=8, dev=gpu)
    out = bias_ln_act(z, b, gamma, beta, 1e-5, "elu")
    out.backward(go)
    zd = z.detach().double().requires_grad_(True)
    bd = b.detach().double().requires_grad_(True) if bias else None
    gd = gamma.detach().double().requires_grad_(True)
    btd = beta.detach().double().requires_grad_(True)
    h = zd + bd if bias else zd
    ref = torch.nn.functional.elu(torch.nn.functional.layer_norm(h, (dim,), gd, btd, 1e-5))
    ref.backward(go.double())
    assert max_abs_norm_err(out, ref) <= TOL
    assert max_abs_norm_err(z.grad, zd.grad) <= TOL
    assert max_abs_norm_err(gamma.grad, gd.grad) <= TOL
    assert max_abs_norm_err(beta.grad, btd.grad) <= TOL
    if bias:
        assert max_abs_norm_err(b.grad, bd.grad) <= TOL


@pytest.mark.parametrize("rows,dim,shift", [(3000, 256, True), (777, 48, False), (50, 300, True),
                                            (130, 7, True)])
def test_ln_act_backward_row_dot(gpu, rows, dim, shift):
    """gr_ln_act_backward's row dot <gh_r, h_r - shift> against the same dot of
    its own gh in float64 (16-byte and scalar rows, several chunks a row)."""
    from grinnder_amd.aggregation import ln_act_backward
    h = _randn(rows, dim, seed=dim, dev=gpu)
    g = _randn(rows, dim, seed=dim + 1, dev=gpu)
    mean = h.mean(1)
    rstd = 1.0 / (h.var(1, unbiased=False) + 1e-5).sqrt()
    gamma = 1 + 0.1 * _randn(dim, seed=2, dev=gpu)
    beta = 0.1 * _randn(dim, seed=3, dev=gpu)
    sh = _randn(dim, seed=4, dev=gpu) if shift else None
    rowdot = torch.empty(rows, device=gpu)
    gh, dgamma, dbeta, _ = ln_act_backward(g, h, mean, rstd, gamma, beta, False, "elu",
                                           shift=sh, rowdot=rowdot)
    gh0, dgamma0, dbeta0, _ = ln_act_backward(g, h, mean, rstd, gamma, beta, False, "elu")
    assert torch.equal(gh, gh0) and torch.equal(dgamma, dgamma0) and torch.equal(dbeta, dbeta0)
    z = h.double() - (sh.double() if shift else 0.0)
    terms = gh.double() * z
    # Without a shift the dot cancels (a LayerNorm input gradient is
    # orthogonal to its input up to eps), so the error is bounded by the
    # size of the terms, as for any fp32 dot product.
    err = (rowdot.double() - terms.sum(1)).abs() / terms.abs().sum(1).clamp_min(1e-30)
    assert float(err.max()) <= TOL
    if shift:
        assert max_abs_norm_err(rowdot, terms.sum(1)) <= TOL


def test_gat_layer_row_dot_handoff(gpu):
    """A GAT attention whose output feeds bias_ln_act through a RowDotSink
    takes c_i from the LayerNorm's backward: same gradients as without the
    sink (where the attention forms c_i itself), and the hand-off is used."""
    from grinnder_amd.aggregation import RowDotSink, gat_attention
    from grinnder_amd.data.adjacency import Adjacency
    from tests.graphs import random_bipartite
    B, E, C = 600, 900, 64
    rowptr, col, val = random_bipartite(B, E, 9, seed=3, long_rows=2, long_len=700)
    adj = Adjacency(rowptr, col, val, (B, E), seg_len=512)
    grads = []
    for use_sink in (False, True):
        hs = _randn(E, C, seed=1, dev=gpu).requires_grad_(True)
        a_s = (0.5 * _randn(1, 1, C, seed=2, dev=gpu)).requires_grad_(True)
        a_d = (0.5 * _randn(1, 1, C, seed=3, dev=gpu)).requires_grad_(True)
        b = _randn(C, seed=4, dev=gpu).requires_grad_(True)
        gamma = (1 + 0.1 * _randn(C, seed=5, dev=gpu)).requires_grad_(True)
        beta = (0.1 * _randn(C, seed=6, dev=gpu)).requires_grad_(True)
        sink = RowDotSink() if use_sink else None
        x = gat_attention(hs, adj, a_s, a_d, None, 1, C, True, rowdot_sink=sink)
        out = bias_ln_act(x, b, gamma, beta, 1e-5, "elu", sink)
        out.backward(_randn(B, C, seed=7, dev=gpu))
        if use_sink:
            assert sink.cdot is None  # handed over and consumed
        grads.append([t.grad.clone() for t in (hs, a_s, a_d, b, gamma, beta)])
    for g0, g1 in zip(*grads):
        assert max_abs_norm_err(g1, g0.double()) <= TOL


@pytest.mark.parametrize("rows,din,dout,act", [
    (5000, 100, 256, "relu"), (777, 37, 48, "elu"), (64, 3, 16, "relu"), (0, 8, 32, "relu"),
    # dout 256 with k tails of 4/8/12 past the 16-k chunks, no full chunk,
    # eight full chunks, ragged and single rows, and 70k rows.  The large
    # cases take ELU: among millions of ReLU inputs a few fall within fp32
    # rounding of 0 and take the other slope in the float64 reference, a
    # difference of the test, not of the kernel.
    (70001, 100, 256, "elu"), (33, 4, 256, "elu"), (1000, 12, 256, "elu"),
    (517, 128, 256, "elu"), (1, 24, 256, "relu"), (16, 16, 256, "relu"),
    # The resident form (dout 256, din <= 100 a multiple of 4, >= 65536
    # rows): 16-k groups with tails of 0-3 four-k steps (din 96: LDS row
    # stride 100; 92: 92; 64: 68; 8 and 4: tail only), row counts a multiple
    # of 16 and ragged.
    (65536, 92, 256, "elu"), (100_003, 96, 256, "elu"), (66_000, 8, 256, "elu"),
    (65_537, 64, 256, "elu"), (70_001, 4, 256, "elu")])
def test_linear_ln_act_matches_fp64(gpu, rows, din, dout, act):
    """act(LayerNorm(x Wᵀ + b)) with the LayerNorm in the MFMA GEMM epilogue."""
    from grinnder_amd.dense import linear_ln_act
    x = _randn(rows, din, seed=din, dev=gpu).requires_grad_(True)
    w = (0.2 * _randn(dout, din, seed=dout, dev=gpu)).requires_grad_(True)
    b = _randn(dout, seed=1, dev=gpu).requires_grad_(True)
    gamma = (1 + 0.1 * _randn(dout, seed=2, dev=gpu)).requires_grad_(True)
    beta = (0.1 * _randn(dout, seed=3, dev=gpu)).requires_grad_(True)
    go = _randn(rows, dout, seed=4, dev=gpu)
    out = linear_ln_act(x, w, b, gamma, beta, 1e-5, act)
    out.backward(go)
    ps = [t.detach().double().requires_grad_(True) for t in (x, w, b, gamma, beta)]
    f = torch.relu if act == "relu" else torch.nn.functional.elu
    ref = f(torch.nn.functional.layer_norm(ps[0] @ ps[1].t() + ps[2], (dout,), ps[3], ps[4],
                                           1e-5))
    ref.backward(go.double())
    if rows == 0:
        assert out.shape == (0, dout)
        return
    assert max_abs_norm_err(out, ref) <= TOL
    for got, want in zip((x, w, b, gamma, beta), ps):
        assert max_abs_norm_err(got.grad, want.grad) <= TOL


@pytest.mark.parametrize("din,act", [(100, "relu"), (92, "elu"), (8, "relu"), (64, "relu")])
def test_linear_ln_act_resident_form_matches_tiled_form_bit_for_bit(gpu, din, act):
    """The resident form (taken from 65536 rows) sums the same products in
    the same order as the tiled kernel (taken below), and rows are
    independent: the first and last 1000 rows of a 70,001-row call equal
    1000-row calls on those rows bit for bit."""
    from grinnder_amd.dense import linear_ln_act
    rows = 70_001
    x = _randn(rows, din, seed=din + 7, dev=gpu)
    w = 0.2 * _randn(256, din, seed=5, dev=gpu)
    b = _randn(256, seed=6, dev=gpu)
    gamma = 1 + 0.1 * _randn(256, seed=7, dev=gpu)
    beta = 0.1 * _randn(256, seed=8, dev=gpu)
    with torch.no_grad():
        full = linear_ln_act(x, w, b, gamma, beta, 1e-5, act)
        head = linear_ln_act(x[:1000].contiguous(), w, b, gamma, beta, 1e-5, act)
        tail = linear_ln_act(x[-1000:].contiguous(), w, b, gamma, beta, 1e-5, act)
    assert torch.equal(full[:1000], head)
    assert torch.equal(full[-1000:], tail)


def test_fused_epilogues_write_into_output_block(gpu):
    """The fused epilogues' `dest` (the trainer passes the next layer's
    HBM-resident input rows): the output is a view of the block with the
    same bits as a freshly allocated output, the gradients are unchanged,
    and a block of the wrong shape is refused."""
    from grinnder_amd.aggregation import gcn_aggregate_ln_relu
    from grinnder_amd.data.adjacency import Adjacency
    from grinnder_amd.dense import OutputRows, linear_ln_act
    from tests.graphs import random_bipartite

    rows, din, dout = 700, 64, 256
    block = torch.full((rows + 300, dout), 7.0, device=gpu)
    x = _randn(rows, din, seed=11, dev=gpu)
    w = 0.2 * _randn(dout, din, seed=12, dev=gpu)
    b = _randn(dout, seed=13, dev=gpu)
    gamma = 1 + 0.1 * _randn(dout, seed=14, dev=gpu)
    beta = 0.1 * _randn(dout, seed=15, dev=gpu)
    go = _randn(rows, dout, seed=16, dev=gpu)
    rowptr, col, val = random_bipartite(rows, 900, 12, seed=5, long_rows=2)
    adj = Adjacency(rowptr, col, val, (rows, 900), seg_len=64)
    z = _randn(900, dout, seed=17, dev=gpu)

    def run(fn, inputs, dest):
        ps = [t.clone().requires_grad_(True) for t in inputs]
        out = fn(*ps, dest)
        out.backward(go)
        return out.detach().clone(), [p.grad for p in ps], out

    cases = [
        ("bias_ln_act", lambda zz, bb, dst: bias_ln_act(zz, bb, gamma, beta, 1e-5, "elu",
                                                       dest=dst), (x @ w.t(), b)),
        ("linear_ln_act", lambda xx, ww, dst: linear_ln_act(xx, ww, b, gamma, beta, 1e-5,
                                                           "relu", dest=dst), (x, w)),
        ("gcn_aggregate_ln_relu", lambda zz, bb, dst: gcn_aggregate_ln_relu(
            zz, adj, bb, gamma, beta, 1e-5, dest=dst), (z, b)),
    ]
    for name, fn, inputs in cases:
        print(f"case {name}", flush=True)
        ref, ref_grads, _ = run(fn, inputs, None)
        lo = 100
        got, grads, view = run(fn, inputs, OutputRows(block[lo:lo + rows]))
        assert view.data_ptr() == block[lo].data_ptr(), name
        assert torch.equal(got, ref), name
        assert torch.equal(block[lo:lo + rows], ref), name
        for g0, g1 in zip(ref_grads, grads):
            assert torch.equal(g0, g1), name
        with pytest.raises(ValueError):
            fn(*inputs, OutputRows(block[:rows, :dout - 4]))
    assert torch.all(block[:100] == 7.0) and torch.all(block[100 + rows:] == 7.0)


@pytest.mark.parametrize("rows,k,dim,act,bias,dot", [(5000, 48, 256, "relu", True, False),
                                                     (3001, 20, 256, "elu", False, False),
                                                     (3001, 20, 256, "elu", True, True),
                                                     (777, 64, 128, "relu", True, True),
                                                     (995, 32, 192, "elu", False, True),
                                                     (17, 4, 64, "elu", True, False),
                                                     (0, 48, 256, "relu", True, True),
                                                     (100_003, 20, 256, "elu", True, True),
                                                     (70_001, 48, 256, "elu", True, False),
                                                     (65_537, 64, 128, "elu", False, True)])
def test_ln_act_backward_product_matches_fp64(gpu, rows, k, dim, act, bias, dot):
    """The LayerNorm/activation backward with dL/dout = dz B formed inside the
    pass, against float64 autograd of act(LayerNorm(h)) with that gradient;
    with `dot`, also rowdot[r] = <dL/dh_r, h_r - shift> (the c_i a GAT
    attention backward takes when its output, shifted by the bias, feeds the
    LayerNorm).  The large cases give each workgroup many 32-row steps and
    take ELU, whose derivative has no jump for fp32 rounding to straddle."""
    from grinnder_amd.aggregation import ln_act_backward_product

    h = _randn(rows, dim, seed=dim + k, dev=gpu)
    gamma = 1 + 0.1 * _randn(dim, seed=1, dev=gpu)
    beta = 0.1 * _randn(dim, seed=2, dev=gpu)
    dz = _randn(rows, k, seed=3, dev=gpu)
    b = 0.2 * _randn(k, dim, seed=4, dev=gpu)
    shift = 0.3 * _randn(dim, seed=5, dev=gpu)
    rowdot = torch.full((rows,), float("nan"), device=gpu) if dot else None
    h64 = h.double()
    if rows:
        mean = h64.mean(1)
        rstd = 1.0 / torch.sqrt(h64.var(1, unbiased=False) + 1e-5)
    else:  # no rows: empty statistics (var over an empty row set only warns)
        mean = rstd = torch.zeros(0, dtype=torch.float64, device=gpu)
    gh, dg, db_, dbias = ln_act_backward_product(dz, b, h, mean.float().contiguous(),
                                                 rstd.float().contiguous(), gamma, beta,
                                                 bias, act, shift=shift if dot else None,
                                                 rowdot=rowdot)
    torch.cuda.synchronize()
    if rows == 0:
        assert gh.shape == (0, dim)
        return
    hh = h64.clone().requires_grad_(True)
    g64 = gamma.double().requires_grad_(True)
    b64 = beta.double().requires_grad_(True)
    f = torch.relu if act == "relu" else torch.nn.functional.elu
    out = f(torch.nn.functional.layer_norm(hh, (dim,), g64, b64, 1e-5))
    out.backward(dz.double() @ b.double())
    assert max_abs_norm_err(gh, hh.grad) <= TOL
    assert max_abs_norm_err(dg, g64.grad) <= TOL
    assert max_abs_norm_err(db_, b64.grad) <= TOL
    if bias:
        assert max_abs_norm_err(dbias, hh.grad.sum(0)) <= TOL
    else:
        assert dbias is None
    if dot:
        ref = (hh.grad * (h64 - shift.double())).sum(1)
        assert max_abs_norm_err(rowdot, ref) <= TOL


@pytest.mark.parametrize("rows", [1, 17, 31, 33, 4099])
def test_ln_act_backward_product_writes_no_row_past_the_last(gpu, rows):
    """gh leaves the kernel through a buffer resource that ends at each step's
    last row, the rows past it sent beyond the end to be dropped: with gh the
    first rows of a larger buffer filled with a sentinel, every row past the
    last keeps the sentinel, and the rows written match the float64 result."""
    dim, k = 256, 48
    h = _randn(rows, dim, seed=rows, dev=gpu)
    gamma = 1 + 0.1 * _randn(dim, seed=1, dev=gpu)
    beta = 0.1 * _randn(dim, seed=2, dev=gpu)
    dz = _randn(rows, k, seed=3, dev=gpu)
    b = 0.2 * _randn(k, dim, seed=4, dev=gpu)
    h64 = h.double()
    mean = h64.mean(1).float().contiguous()
    rstd = (1.0 / torch.sqrt(h64.var(1, unbiased=False) + 1e-5)).float().contiguous()
    pad = 40  # rows of sentinel after the last row (a whole 32-row step and more)
    gh = torch.full((rows + pad, dim), 12345.0, device=gpu)
    dgamma = torch.empty(dim, device=gpu)
    dbeta = torch.empty(dim, device=gpu)
    nwaves = (min(8192, max(4, (rows + 15) // 16)) + 3) // 4 * 4
    ws = torch.empty((2 * nwaves + 1) * dim, device=gpu)
    _lib.call("gr_ln_act_backward_product", dz.data_ptr(), k, k, b.data_ptr(), h.data_ptr(),
              mean.data_ptr(), rstd.data_ptr(), gamma.data_ptr(), beta.data_ptr(),
              _lib.ACTIVATIONS["relu"], rows, dim, gh.data_ptr(), dgamma.data_ptr(),
              dbeta.data_ptr(), None, None, None, ws.data_ptr(), ws.numel(),
              _lib.stream_handle())
    torch.cuda.synchronize()
    assert torch.all(gh[rows:] == 12345.0)
    hh = h64.clone().requires_grad_(True)
    out = torch.relu(torch.nn.functional.layer_norm(hh, (dim,), gamma.double(),
                                                    beta.double(), 1e-5))
    out.backward(dz.double() @ b.double())
    assert max_abs_norm_err(gh[:rows], hh.grad) <= TOL


@pytest.mark.parametrize("extra_consumer", [False, True])
def test_layernorm_takes_narrow_product_gradient(gpu, extra_consumer):
    """A fused LayerNorm/ReLU output consumed by a narrow padded GCN product
    (47 outputs, the C2 last layer's shape) hands its input gradient to the
    LayerNorm as dZ W: every gradient equals the same model built without the
    handoff (the LayerNorm output copied first, so it carries no sink), to
    TOL against each other and against float64.  With a second consumer of
    the output the LayerNorm receives autograd's sum and completes it."""
    from grinnder_amd.aggregation import gcn_aggregate_ln_relu, gcn_linear_aggregate
    from grinnder_amd.data.adjacency import Adjacency
    from tests.graphs import random_bipartite

    n, d, c = 3000, 256, 47
    rowptr, col, val = random_bipartite(n, n, 10, seed=9, long_rows=2, long_len=700)
    adj = Adjacency(rowptr, col, val, (n, n), seg_len=256)
    z = _randn(n, d, seed=5, dev=gpu)
    params = [_randn(d, seed=6, dev=gpu), 1 + 0.1 * _randn(d, seed=7, dev=gpu),
              0.1 * _randn(d, seed=8, dev=gpu), 0.1 * _randn(c, d, seed=9, dev=gpu),
              _randn(c, seed=10, dev=gpu)]
    go = _randn(n, c, seed=11, dev=gpu)
    grads = []
    for handoff in (True, False):
        zz = z.clone().requires_grad_(True)
        b1, g1, be1, w2, b2 = [p.clone().requires_grad_(True) for p in params]
        out1 = gcn_aggregate_ln_relu(zz, adj, b1, g1, be1)
        x2 = out1 if handoff else out1 * 1.0
        y = gcn_linear_aggregate(x2, w2, adj, b2)
        loss = (y * go).sum()
        if extra_consumer:
            loss = loss + out1[:, :3].square().sum()
        loss.backward()
        torch.cuda.synchronize()
        grads.append([t.grad for t in (zz, b1, g1, be1, w2, b2)])
    for g0, g1 in zip(*grads):
        assert max_abs_norm_err(g0, g1.double()) <= TOL

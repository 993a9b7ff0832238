"""GPU: fused masked cross-entropy + accuracy (gr_xent_forward) against
float64 torch (F.cross_entropy on the masked rows, argmax accuracy).
Loss and gradient: max-abs-normalised error <= 1e-5; counts: exact."""

import pytest
import torch
import torch.nn.functional as F

from grinnder_amd.loss import check_stats, mask_codes, masked_cross_entropy
from tests.graphs import TOL, max_abs_norm_err

pytestmark = pytest.mark.gpu


def _case(rows, classes, seed, dev, frac=(0.5, 0.3, 0.3)):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(rows, classes, generator=g) * 3).to(dev)
    y = torch.randint(0, classes, (rows,), generator=g).to(dev)
    tr = torch.rand(rows, generator=g) < frac[0]
    va = torch.rand(rows, generator=g) < frac[1]  # may overlap train: counted independently
    te = torch.rand(rows, generator=g) < frac[2]
    return logits, y, tr, va, te


def _acc_counts(logits, y, m):
    pred = logits.argmax(-1)
    return int((pred[m] == y[m]).sum()), int(m.sum())


@pytest.mark.parametrize("rows,classes", [(1000, 1), (5000, 10), (4000, 19), (20000, 47),
                                          (3000, 100), (700, 300)])
@pytest.mark.parametrize("reduction", ["sum", "mean"])
def test_masked_xent_matches_fp64(gpu, rows, classes, reduction):
    logits, y, tr, va, te = _case(rows, classes, rows + classes, gpu)
    codes = mask_codes(tr, va, te).to(gpu)
    x = logits.clone().requires_grad_(True)
    loss, stats = masked_cross_entropy(x, y, codes, reduction)
    go = torch.tensor(0.75, device=gpu)
    loss.backward(go)
    xd = logits.double().cpu().requires_grad_(True)
    trc = tr.cpu()
    ref = F.cross_entropy(xd[trc], y.cpu()[trc], reduction=reduction)
    (ref * 0.75).backward()
    assert max_abs_norm_err(loss.detach().reshape(1), ref.detach().reshape(1)) <= TOL
    assert max_abs_norm_err(x.grad, xd.grad) <= TOL
    st = stats.tolist()
    vc, vn = _acc_counts(logits.cpu(), y.cpu(), va)
    tc, tn = _acc_counts(logits.cpu(), y.cpu(), te)
    assert st == [int(tr.sum()), vc, vn, tc, tn, 0]


@pytest.mark.parametrize("rows,classes,ld", [(20_003, 47, 48), (4_000, 19, 20), (777, 10, 12),
                                             (300, 3, 4), (513, 47, 52)])
def test_padded_logit_rows_match_fp64(gpu, rows, classes, ld):
    """Logits held zero-padded to a multiple of 4 columns (the trainer's
    [rows, 48] and [rows, 20] blocks): the first `classes` columns of a
    16-byte aligned [rows, ld] buffer, read as 16-byte pieces.  The buffer
    ends at the last row's last class (no pad after it), and its pad
    columns hold large values that must not reach the loss."""
    logits, y, tr, va, te = _case(rows, classes, rows + ld, gpu)
    flat = torch.full(((rows - 1) * ld + classes,), 1e4, device=gpu)
    x = flat.as_strided((rows, classes), (ld, 1))
    x.copy_(logits)
    x.requires_grad_(True)
    codes = mask_codes(tr, va, te).to(gpu)
    loss, stats = masked_cross_entropy(x, y, codes, "sum")
    loss.backward()
    xd = logits.double().cpu().requires_grad_(True)
    trc = tr.cpu()
    ref = F.cross_entropy(xd[trc], y.cpu()[trc], reduction="sum")
    ref.backward()
    assert max_abs_norm_err(loss.detach().reshape(1), ref.detach().reshape(1)) <= TOL
    assert max_abs_norm_err(x.grad, xd.grad) <= TOL
    vc, vn = _acc_counts(logits.cpu(), y.cpu(), va)
    tc, tn = _acc_counts(logits.cpu(), y.cpu(), te)
    assert stats.tolist() == [int(tr.sum()), vc, vn, tc, tn, 0]


def test_strided_logits_and_ties(gpu):
    """ld > C (a column slice) and tied maxima: the first maximal index wins."""
    wide = torch.randn(600, 64, device=gpu)
    logits = wide[:, 5:52]  # 47 classes, row stride 64
    logits[::3, 10] = 100.0
    logits[::3, 30] = 100.0  # tie between 10 and 30 on every third row
    y = torch.full((600,), 10, dtype=torch.int64, device=gpu)
    y[1::3] = 30
    every = torch.ones(600, dtype=torch.bool)
    codes = mask_codes(every, every, every).to(gpu)
    loss, stats = masked_cross_entropy(logits, y, codes, "sum")
    ref = F.cross_entropy(logits.double().cpu(), y.cpu(), reduction="sum")
    assert max_abs_norm_err(loss.reshape(1), ref.reshape(1)) <= TOL
    vc, vn = _acc_counts(logits.cpu(), y.cpu(), every)
    assert stats.tolist()[1:3] == [vc, vn]


def test_no_train_rows_zero_loss_and_grad(gpu):
    logits, y, _, va, te = _case(500, 7, 3, gpu)
    codes = mask_codes(torch.zeros(500, dtype=torch.bool), va, te).to(gpu)
    x = logits.clone().requires_grad_(True)
    for red in ("sum", "mean"):
        x.grad = None
        loss, stats = masked_cross_entropy(x, y, codes, red)
        loss.backward()
        assert float(loss.detach()) == 0.0 and stats.tolist()[0] == 0
        assert torch.count_nonzero(x.grad) == 0


def test_empty_and_bad_labels(gpu):
    x = torch.empty(0, 5, device=gpu)
    loss, stats = masked_cross_entropy(x, torch.empty(0, dtype=torch.int64, device=gpu),
                                       torch.empty(0, dtype=torch.uint8, device=gpu), "sum")
    assert float(loss) == 0.0 and stats.tolist() == [0] * 6
    logits, y, tr, va, te = _case(300, 5, 4, gpu)
    y[7] = 5  # out of range on a selected row
    codes = mask_codes(torch.ones(300, dtype=torch.bool), va, te).to(gpu)
    _, stats = masked_cross_entropy(logits, y, codes, "sum")
    st = stats.tolist()
    assert st[5] == 1
    with pytest.raises(IndexError):
        check_stats(st)


def test_deterministic(gpu):
    logits, y, tr, va, te = _case(200_000, 47, 5, gpu)
    codes = mask_codes(tr, va, te).to(gpu)
    a = masked_cross_entropy(logits, y, codes, "mean")[0]
    b = masked_cross_entropy(logits, y, codes, "mean")[0]
    assert torch.equal(a, b)

"""gr_gcn_aggregate_noalloc (the entry point that allocates nothing) against
gr_gcn_aggregate with a caller workspace, through the C ABI: the same
kernels on the same inputs, so the outputs must be bit-identical.  Two calls
in a row, the second with a smaller input (the scratch keeps the first
call's contents), in both directions (CSR forward plan, CSC backward plan),
split rows included; and the size limit is refused before any launch."""

import pytest
import torch

from grinnder_amd import _lib
from grinnder_amd.data.adjacency import Adjacency
from tests.graphs import random_bipartite

pytestmark = pytest.mark.gpu

SCRATCH_FLOATS = 8 << 20  # GR_NOALLOC_SCRATCH_FLOATS


def _args(plan, idx, val, x, y, bias, rows, dim):
    return (plan.units.data_ptr(), plan.n_units,
            plan.fixups.data_ptr() if plan.n_fix else None, plan.n_fix, idx.data_ptr(),
            val.data_ptr(), x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0),
            _lib.ptr(bias), rows, dim)


def _both(plan, idx, val, x, bias, rows, dim, device):
    y_ref = torch.full((rows, dim), float("nan"), device=device)
    ws = torch.empty(max(1, plan.n_slots * dim), device=device)
    _lib.call("gr_gcn_aggregate", *_args(plan, idx, val, x, y_ref, bias, rows, dim),
              ws.data_ptr(), plan.n_slots, _lib.stream_handle())
    y = torch.full((rows, dim), float("nan"), device=device)
    _lib.call("gr_gcn_aggregate_noalloc", *_args(plan, idx, val, x, y, bias, rows, dim),
              plan.n_slots, _lib.stream_handle())
    torch.cuda.synchronize()
    return y, y_ref


@pytest.mark.parametrize("dim", [256, 47])
def test_noalloc_matches_workspace_entry_twice(gpu, dim):
    for B, E, longs, seed in ((3000, 4200, 8, 1), (700, 900, 3, 2)):
        print(f"noalloc dim={dim} B={B} E={E}", flush=True)
        rowptr, col, val = random_bipartite(B, E, 12, seed=seed + dim, long_rows=longs,
                                            long_len=2500)
        adj = Adjacency(rowptr, col, val, (B, E), seg_len=256)
        plan = adj.device_plan(gpu)
        assert plan.fwd.n_fix > 0 and plan.fwd.n_slots * dim <= SCRATCH_FLOATS
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(E, dim, generator=g).to(gpu)
        bias = torch.randn(dim, generator=g).to(gpu)
        gy = torch.randn(B, dim, generator=g).to(gpu)
        y, y_ref = _both(plan.fwd, plan.idx, plan.val, x, bias, B, dim, gpu)
        assert torch.equal(y, y_ref)
        dz, dz_ref = _both(plan.bwd, plan.row_idx, plan.val_t, gy, None, E, dim, gpu)
        assert torch.equal(dz, dz_ref)


def test_noalloc_refuses_more_than_the_scratch(gpu):
    rowptr, col, val = random_bipartite(50, 60, 4, seed=3, long_rows=1, long_len=600)
    adj = Adjacency(rowptr, col, val, (50, 60), seg_len=128)
    plan = adj.device_plan(gpu)
    dim = 256
    x = torch.randn(60, dim, device=gpu)
    y = torch.zeros(50, dim, device=gpu)
    too_many = SCRATCH_FLOATS // dim + 1
    with pytest.raises(_lib.GrError, match="scratch"):
        _lib.call("gr_gcn_aggregate_noalloc",
                  *_args(plan.fwd, plan.idx, plan.val, x, y, None, 50, dim), too_many,
                  _lib.stream_handle())
    torch.cuda.synchronize()
    assert bool((y == 0).all())

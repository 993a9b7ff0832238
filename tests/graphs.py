"""Seeded sparse test inputs shared by the test modules (test infrastructure)."""

from __future__ import annotations

import torch


def random_bipartite(num_dst: int, num_src: int, avg_deg: float, seed: int,
                     long_rows: int = 0, long_len: int = 1500, empty_frac: float = 0.05,
                     self_loops: bool = True):
    """CSR [num_dst x num_src] with Poisson-ish degrees, some empty rows and
    `long_rows` rows of `long_len` edges (exercises the split/fixup path).
    Row i gets the self-loop column i first when `self_loops` (i < num_src).
    Returns (rowptr int64, col int64, val fp32)."""
    g = torch.Generator().manual_seed(seed)
    deg = torch.poisson(torch.full((num_dst,), float(avg_deg)), generator=g).to(torch.int64)
    empty = torch.rand(num_dst, generator=g) < empty_frac
    deg[empty] = 0
    if long_rows:
        which = torch.randperm(num_dst, generator=g)[:long_rows]
        deg[which] = long_len
    cols = []
    for i in range(num_dst):
        d = int(deg[i])
        c = torch.randint(0, num_src, (d,), generator=g)
        if self_loops and d > 0 and i < num_src:
            c[0] = i
        cols.append(c)
    col = torch.cat(cols) if cols else torch.zeros(0, dtype=torch.int64)
    rowptr = torch.zeros(num_dst + 1, dtype=torch.int64)
    rowptr[1:] = deg.cumsum(0)
    val = torch.rand(col.numel(), generator=g) * 2 - 1
    return rowptr, col, val.to(torch.float32)


def max_abs_norm_err(got, ref) -> float:
    """max|got - ref| / max|ref| (the north-star tolerance metric)."""
    got = torch.as_tensor(got, dtype=torch.float64).detach().cpu()
    ref = torch.as_tensor(ref, dtype=torch.float64).detach().cpu()
    if ref.numel() == 0:
        return 0.0
    scale = float(ref.abs().max())
    diff = float((got - ref).abs().max())
    return diff / scale if scale > 0 else diff


def grad_errs(grads, ref_grads, floor_frac: float = 1e-2):
    """Per-parameter max-abs error normalised by max(|ref param|max,
    floor_frac * largest |ref| gradient of the model).

    The floor matters for parameters whose true gradient is (nearly) zero by
    an invariance — e.g. GAT's destination attention vector, which only acts
    through the LeakyReLU kink because softmax is shift-invariant — where
    per-tensor normalisation would divide fp32 rounding noise by ~0.  With the
    1e-5 bound, such a parameter may be off by at most 1e-7 of the model's
    largest gradient (about two fp32 ulps of it)."""
    scale = max(float(torch.as_tensor(r).abs().max()) for r in ref_grads.values())
    out = {}
    for k, r in ref_grads.items():
        r = torch.as_tensor(r, dtype=torch.float64).cpu()
        g = torch.as_tensor(grads[k], dtype=torch.float64).cpu()
        denom = max(float(r.abs().max()), floor_frac * scale)
        out[k] = float((g - r).abs().max()) / denom
    return out


TOL = 1e-5

"""Torch restatements of the reference models on the unpartitioned graph, for
the epoch-level GPU tests (test infrastructure).

They follow the reference's layer definitions, with PyG's conv semantics:

- GCN (grinnder/nn/gcn.py:52-73): ``A (X Wᵀ) + b``, then LayerNorm and ReLU
  on every layer but the last.
- GAT (grinnder/nn/gat.py:53-78, one head): Hs = X Wᵀ, logits
  LeakyReLU_0.2(<Hs_j, att_src> + <Hs_i, att_dst>) over row i's edges,
  softmax with PyG's + 1e-16 in the denominator, O_i = sum_j alpha_ij Hs_j
  + b, then LayerNorm and ELU on every layer but the last.

The adjacency is the pipeline's: self-loops appended, rows from
edge_index[0] (grinnder/data/partition.py:79-87), fp32 sym-norm weights
(grinnder/data/datasets.py:334-362) for GCN; GAT ignores the weights.  In
float64 these are the checkers' reference; in float32 they are the
reference's own arithmetic (torch sparse and dense kernels, what PyG runs),
whose distance from float64 says how well conditioned a gradient is.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from grinnder_amd.data.datasets import append_self_loops, compute_gcn_norm


def _model_in(make, state, dtype, device):
    model = make().to(dtype).to(device)
    model.load_state_dict({k: v.to(dtype) for k, v in state.items()})
    return model


def gcn_layers(model, a, h):
    for i, conv in enumerate(model.convs):
        h = torch.sparse.mm(a, h @ conv.lin.weight.t()) + conv.bias
        if i < len(model.convs) - 1:
            if model.norms is not None:
                h = model.norms[i](h)
            h = torch.relu(h)
    return h


def gat_attention_full(hs, att_src, att_dst, bias, dst, src, n):
    """One head of PyG's GATConv over edges (src j -> dst i), [n, C] rows."""
    s = hs @ att_src.reshape(-1)
    d = hs @ att_dst.reshape(-1)
    t = F.leaky_relu(s.index_select(0, src) + d.index_select(0, dst), 0.2)
    m = torch.full((n,), float("-inf"), dtype=hs.dtype, device=hs.device)
    m = m.scatter_reduce(0, dst, t, "amax")
    ex = torch.exp(t - m.index_select(0, dst))
    den = torch.zeros(n, dtype=hs.dtype, device=hs.device).index_add(0, dst, ex)
    alpha = ex / (den.index_select(0, dst) + 1e-16)
    msg = hs.index_select(0, src) * alpha.unsqueeze(1)
    out = torch.zeros_like(hs).index_add(0, dst, msg)
    return out + bias


def gat_layers(model, dst, src, n, h):
    for i, conv in enumerate(model.convs):
        h = gat_attention_full(h @ conv.lin.weight.t(), conv.att_src, conv.att_dst, conv.bias,
                               dst, src, n)
        if i < len(model.convs) - 1:
            if model.norms is not None:
                h = model.norms[i](h)
            h = F.elu(h)
    return h


def model_epoch(kind, ei, x, y, train, state, make, device, dtype=torch.float64):
    """Loss (CE mean over the train rows) and every parameter gradient of one
    full-graph step of the `kind` ('gcn' or 'gat') model from `state`.
    Loss and gradients do not depend on the node order."""
    n = x.size(0)
    model = _model_in(make, state, dtype, device)
    h = x.to(dtype).to(device)
    full = append_self_loops(ei, n)
    if kind == "gcn":
        w = compute_gcn_norm(ei, n, add_self_loops=True)
        a = torch.sparse_coo_tensor(full.to(device), w.to(dtype).to(device), (n, n)).coalesce()
        a = a.to_sparse_csr()
        del w
        out = gcn_layers(model, a, h)
    else:
        dst, src = full[0].to(device), full[1].to(device)
        out = gat_layers(model, dst, src, n, h)
    del full
    tr = train.to(device)
    loss = F.cross_entropy(out[tr], y.to(device)[tr])
    loss.backward()
    result = (float(loss.detach()),
              {k: p.grad.double().cpu() for k, p in model.named_parameters()})
    del model, out, loss, h
    torch.cuda.empty_cache()
    return result

"""GPU: models, autograd hooks and the Trainer (reference tests test_models.py,
test_autograd.py, test_trainer.py, test_gradient_identity.py), with the
reference's tolerances tightened to the north-star 1e-5 where it applies."""

import copy

import pytest
import torch
from torch.autograd.graph import saved_tensors_hooks

from grinnder_amd.autograd.checkpoint import HongtuCheckpoint, ScatteredCheckpoint
from grinnder_amd.autograd.grad_offload import GradOffload
from grinnder_amd.buffer.device import DeviceBuffer
from grinnder_amd.buffer.host import HostBuffer
from grinnder_amd.config import GriNNderConfig
from grinnder_amd.data.adjacency import Adjacency
from grinnder_amd.data.datasets import append_self_loops, compute_gcn_norm
from grinnder_amd.data.partition import build_partitioned_graph
from grinnder_amd.data.synthetic import banded_graph
from grinnder_amd.engine.streams import StreamManager
from grinnder_amd.engine.trainer import Trainer
from grinnder_amd.nn import GAT, GCN
from tests.graphs import TOL, grad_errs

pytestmark = pytest.mark.gpu


# -------------------------------------------------------------- models --

@pytest.fixture
def small_adj():
    """tests/test_models.py:13-20: 4 dst nodes, 7 source nodes."""
    row = torch.tensor([0, 0, 1, 1, 2, 3, 3])
    col = torch.tensor([0, 4, 1, 5, 2, 3, 6])
    rowptr = torch.zeros(5, dtype=torch.long)
    rowptr[1:] = torch.bincount(row, minlength=4).cumsum(0)
    return Adjacency(rowptr, col, None, (4, 7))


def test_model_shapes(gpu, small_adj):
    m = GCN(16, 32, 7, num_layers=3).to(gpu)
    assert m.forward_layer(0, torch.randn(7, 16, device=gpu), small_adj).shape == (4, 32)
    assert m.layer_dims() == [16, 32, 32, 7]
    g = GAT(16, 4, 7, num_layers=2, heads=8).to(gpu)
    assert g.forward_layer(0, torch.randn(7, 16, device=gpu), small_adj).shape == (4, 32)
    assert g.forward_layer(1, torch.randn(7, 32, device=gpu), small_adj).shape == (4, 7)


def test_stream_manager(gpu):
    sm = StreamManager(pool_size=2, device="cuda:0")
    assert len(sm.h2d) == 2 and len(sm.d2h) == 2 and len(sm.act_h2d) == 2
    assert sm.compute is not None


def test_device_buffer(gpu):
    buf = DeviceBuffer(3, [10, 15, 12], 8)
    assert not buf.is_allocated(0)
    buf.allocate(0)
    assert buf.is_allocated(0) and buf[0].shape == (10, 8)
    buf.allocate(1)
    buf.reset()
    assert buf.allocated_pids() == []


# ------------------------------------------------------------ autograd --

def test_grad_offload(gpu):
    """tests/test_autograd.py:14-74."""
    x = torch.randn(10, 4, device=gpu, requires_grad=True)
    hg = HostBuffer(2, [10, 8], 4)
    out = GradOffload.apply(x, 1, 0, hg, [None, torch.tensor([0, 1, 2])], torch.cuda.Stream(),
                            torch.cuda.current_stream())
    assert torch.equal(out, x)

    hg = HostBuffer(2, [5, 8], 4, pin_memory=True)
    hg.initialize_zeros()
    d2h = torch.cuda.Stream()
    x = torch.randn(8, 4, device=gpu, requires_grad=True)
    out = GradOffload.apply(x, 1, 0, hg, [None, torch.tensor([0, 2, 4])], d2h,
                            torch.cuda.current_stream())
    (out * 2).sum().backward()
    hg.d2h_synchronize(d2h)
    assert torch.equal(hg[0], torch.full((5, 4), 2.0))
    assert hg[1][[0, 2, 4]].eq(2.0).all() and hg[1][[1, 3, 5, 6, 7]].eq(0).all()
    assert x.grad is None

    hg = HostBuffer(2, [5, 5], 4)
    hg.initialize_zeros()
    x = torch.randn(5, 4, device=gpu, requires_grad=True)
    out = GradOffload.apply(x, 0, 0, hg, [None, torch.empty(0, dtype=torch.long)],
                            torch.cuda.Stream(), torch.cuda.current_stream())
    out.sum().backward()
    torch.cuda.synchronize()
    assert hg[0].abs().sum() == 0 and x.grad is None


def test_checkpoint_hooks(gpu):
    """tests/test_autograd.py:77-106."""
    from torch.utils.checkpoint import checkpoint

    buf = DeviceBuffer(1, [5], 4)
    buf.allocate(0)
    assert isinstance(ScatteredCheckpoint(0, buf, torch.cuda.Stream()), saved_tensors_hooks)
    x = torch.randn(5, 4, device=gpu, requires_grad=True)
    with HongtuCheckpoint(0, buf):
        y = checkpoint(lambda t: t * 3, x, use_reentrant=True)
    y.sum().backward()
    assert torch.equal(x.grad, torch.full((5, 4), 3.0, device=gpu))


# ------------------------------------------------------------- trainer --

def _graph_data(n=20, reach=2, feat=8, classes=3, seed=42, train_all=True):
    """tests/test_gradient_identity.py:27-45 (banded graph, seed 42)."""
    torch.manual_seed(seed)
    ei = banded_graph(n, reach)
    x = torch.randn(n, feat)
    y = torch.randint(0, classes, (n,))
    train = torch.ones(n, dtype=torch.bool) if train_all else torch.arange(n) < int(0.7 * n)
    val = torch.zeros(n, dtype=torch.bool) if train_all else (torch.arange(n) >= int(0.7 * n))
    test = torch.zeros(n, dtype=torch.bool)
    return ei, x, y, train, val, test


def _step(data, state, make_model, num_parts, mode, pool_size=2):
    ei, x, y, tr, va, te = data
    config = GriNNderConfig(num_parts=num_parts, mode=mode, pool_size=pool_size)
    graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
    model = make_model().cuda()
    model.load_state_dict(state)
    trainer = Trainer(model, graph, config)
    opt = torch.optim.SGD(model.parameters(), lr=0.1)
    metrics = trainer.train_epoch(opt, torch.nn.CrossEntropyLoss())
    grads = {n: p.grad.detach().clone() for n, p in model.named_parameters()
             if p.grad is not None}
    return metrics["loss"], grads, trainer, graph


def _vanilla(data, state, make_model):
    """Dense float64 full-batch GCN (the reference's 'vanilla PyG' step)."""
    ei, x, y, tr, _, _ = data
    n = x.size(0)
    w = compute_gcn_norm(ei, n, True).double()
    full = append_self_loops(ei, n)
    a = torch.zeros(n, n, dtype=torch.float64)
    a.index_put_((full[0], full[1]), w, accumulate=True)
    model = make_model().double()
    model.load_state_dict({k: v.double() for k, v in state.items()})
    h = x.double()
    for i, conv in enumerate(model.convs):
        h = a @ (h @ conv.lin.weight.t()) + conv.bias
        if i < len(model.convs) - 1:
            if model.norms is not None:
                h = model.norms[i](h)
            h = torch.relu(h)
    loss = torch.nn.functional.cross_entropy(h[tr], y[tr])
    loss.backward()
    return float(loss.detach()), {k: p.grad for k, p in model.named_parameters()}


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("feat,hidden", [(8, 16), (24, 16)])
def test_gcn_matches_dense_vanilla(gpu, norm, feat, hidden):
    """feat < hidden: the first layer aggregates first, (A X) W^T; feat >
    hidden: it multiplies first, A (X W^T), as PyG does."""
    data = _graph_data(feat=feat)
    torch.manual_seed(7)
    make = lambda: GCN(feat, hidden, 3, num_layers=2, dropout=0.0, norm=norm)  # noqa: E731
    state = make().state_dict()
    ref_loss, ref_grads = _vanilla(data, state, make)
    for parts, mode in [(1, "grinnder"), (4, "grinnder"), (4, "hongtu")]:
        loss, grads, *_ = _step(data, state, make, parts, mode)
        assert abs(loss - ref_loss) < 1e-5, (parts, mode, loss, ref_loss)
        for k, err in grad_errs(grads, ref_grads).items():
            assert err <= 1e-5, (parts, mode, k, err)


def test_fast_path_rejects_bad_labels_before_stepping(gpu):
    """A selected row whose label is outside [0, C) raises, as F.cross_entropy
    does, before the optimizer changes any weight."""
    ei, x, y, tr, va, te = _graph_data()
    y = y.clone()
    y[3] = 99
    config = GriNNderConfig(num_parts=1)
    graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
    model = GCN(8, 16, 3, num_layers=2).cuda()
    before = {k: v.clone() for k, v in model.state_dict().items()}
    trainer = Trainer(model, graph, config)
    with pytest.raises(IndexError):
        trainer.train_epoch(torch.optim.SGD(model.parameters(), lr=0.1),
                            torch.nn.CrossEntropyLoss())
    assert all(torch.equal(before[k], v) for k, v in model.state_dict().items())


def _vanilla_gat(data, state, make_model):
    """Dense float64 full-batch GAT with the same layer structure."""
    from tests.test_oracle import _dense_gat

    ei, x, y, tr, _, _ = data
    n = x.size(0)
    full = append_self_loops(ei, n)
    mask = torch.zeros(n, n, dtype=torch.float64)
    mask.index_put_((full[0], full[1]), torch.ones(full.size(1), dtype=torch.float64),
                    accumulate=True)
    model = make_model().double()
    model.load_state_dict({k: v.double() for k, v in state.items()})
    h = x.double()
    for i, conv in enumerate(model.convs):
        hs = h @ conv.lin.weight.t()
        h = _dense_gat(mask, hs, conv.att_src, conv.att_dst, conv.bias, conv.heads,
                       conv.out_channels, conv.concat)
        if i < len(model.convs) - 1:
            if model.norms is not None:
                h = model.norms[i](h)
            h = torch.nn.functional.elu(h)
    loss = torch.nn.functional.cross_entropy(h[tr], y[tr])
    loss.backward()
    return float(loss.detach()), {k: p.grad for k, p in model.named_parameters()}


@pytest.mark.parametrize("heads,hidden,classes", [(1, 8, 4), (2, 8, 4), (1, 6, 3)])
def test_gat_matches_dense_vanilla(gpu, heads, hidden, classes):
    """(1, 6, 3): single-head layers of 6 and 3 channels run padded to 8 and 4."""
    data = _graph_data(n=40, reach=3, feat=12, classes=classes, train_all=False)
    torch.manual_seed(11)
    make = lambda: GAT(12, hidden, classes, num_layers=3, heads=heads, dropout=0.0,  # noqa
                       norm=True)
    state = make().state_dict()
    ref_loss, ref_grads = _vanilla_gat(data, state, make)
    for parts, mode in [(1, "grinnder"), (4, "grinnder"), (4, "hongtu")]:
        loss, grads, *_ = _step(data, state, make, parts, mode)
        assert abs(loss - ref_loss) < 1e-5, (parts, mode, loss, ref_loss)
        for k, err in grad_errs(grads, ref_grads).items():
            print(f"parts={parts} mode={mode} {k}: {err:.2e}")
            assert err <= 1e-5, (parts, mode, k, err)


@pytest.mark.parametrize("model_kind", ["gcn", "gat"])
@pytest.mark.parametrize("pool_size", [1, 2])
def test_partition_invariance(gpu, model_kind, pool_size):
    """tests/test_gradient_identity.py:290-410 (atol 1e-4 there): 1 partition vs
    2/4/5 partitions at the north-star 1e-5 (max-abs normalised, see grad_errs);
    both sides are also pinned to float64 by the *_vanilla tests."""
    tol = 1e-5
    data = _graph_data(n=50, reach=3, feat=16, classes=4, train_all=False)
    torch.manual_seed(7)
    if model_kind == "gcn":
        make = lambda: GCN(16, 32, 4, num_layers=3, dropout=0.0, norm=True)  # noqa: E731
    else:
        make = lambda: GAT(16, 8, 4, num_layers=3, heads=2, dropout=0.0, norm=True)  # noqa
    state = make().state_dict()
    loss1, g1, *_ = _step(data, state, make, 1, "grinnder")
    for parts in (2, 4, 5):
        for mode in ("grinnder", "hongtu"):
            loss, g, *_ = _step(data, state, make, parts, mode, pool_size)
            assert abs(loss - loss1) < 1e-5, (parts, mode)
            for k, err in grad_errs(g, g1).items():
                assert err <= tol, (parts, mode, k, err)
                assert torch.allclose(g[k], g1[k], atol=1e-4)


def test_buffers_released_and_loss_decreases(gpu):
    """tests/test_gradient_identity.py:412-456 and tests/test_trainer.py (5 epochs)."""
    data = _graph_data(n=50, reach=3, feat=16, classes=4, train_all=False)
    torch.manual_seed(0)
    for make in (lambda: GCN(16, 32, 4, num_layers=2),
                 lambda: GAT(16, 8, 4, num_layers=2, heads=2)):
        ei, x, y, tr, va, te = data
        config = GriNNderConfig(num_parts=4)
        graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
        model = make().cuda()
        trainer = Trainer(model, graph, config)
        opt = torch.optim.Adam(model.parameters(), lr=0.01)
        losses = [trainer.train_epoch(opt, torch.nn.CrossEntropyLoss())["loss"]
                  for _ in range(5)]
        assert losses[-1] < losses[0]
        for buf in trainer.device_features:
            assert buf.allocated_pids() == []
            assert all(buf[p].grad is None for p in range(4))
        for buf in trainer.device_gradients:
            if buf is not None:
                assert buf.allocated_pids() == []
        ev = trainer.evaluate(torch.nn.CrossEntropyLoss())
        assert 0.0 <= ev["val_acc"] <= 1.0


def _limit_resident_inputs(monkeypatch, keep):
    """Plans projected layers as usual but keeps only the inputs of layers in
    `keep` in HBM, as when HBM has no room for the others: their dW then
    comes from uploads (a second one, for layer 0)."""
    plan = Trainer._plan_projection

    def limited(self):
        out = plan(self)
        self._xin = {l for l in self._xin if l in keep}
        last = self.model.num_layers - 1
        self._keep = {l for l in self._keep if l + 1 in self._xin or l == last}
        return out
    monkeypatch.setattr(Trainer, "_plan_projection", limited)


@pytest.mark.parametrize("model_kind", ["gcn", "gat", "gat2"])
@pytest.mark.parametrize("pool_size", [1, 2])
@pytest.mark.parametrize("resident", ["all", "above0", "none"])
def test_projected_layers_match_gathered(gpu, model_kind, pool_size, resident, monkeypatch):
    """config.project_first: every layer runs on projected rows Z = x Wᵀ held
    in HBM (narrowing, equal and widening projections), with the layer inputs
    kept in HBM for the epoch (all, those above layer 0, or none: uploads);
    loss and gradients equal those of the reference flow that gathers input
    rows (project_first='off') within the 1e-5 bound, and evaluate() agrees
    too."""
    kept = {"all": [0, 1, 2], "above0": [1, 2], "none": []}[resident]
    if resident != "all":
        _limit_resident_inputs(monkeypatch, set(kept))
    data = _graph_data(n=60, reach=3, feat=24, classes=4, train_all=False)
    torch.manual_seed(3)
    if model_kind == "gcn":
        make = lambda: GCN(24, 16, 4, num_layers=3, dropout=0.0, norm=True)  # noqa: E731
    else:
        heads = 2 if model_kind == "gat2" else 1
        make = lambda: GAT(24, 8, 4, num_layers=3, heads=heads, dropout=0.0, norm=True)  # noqa
    state = make().state_dict()
    ei, x, y, tr, va, te = data
    runs = {}
    for proj in ("off", "auto"):
        config = GriNNderConfig(num_parts=4, pool_size=pool_size, project_first=proj)
        graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
        model = make().cuda()
        model.load_state_dict(state)
        trainer = Trainer(model, graph, config)
        opt = torch.optim.SGD(model.parameters(), lr=0.0)
        metrics = trainer.train_epoch(opt, torch.nn.CrossEntropyLoss())
        assert trainer.projected_layers == ([0, 1, 2] if proj == "auto" else [])
        assert trainer.resident_inputs == (kept if proj == "auto" else [])
        grads = {n: p.grad.detach().clone() for n, p in model.named_parameters()
                 if p.grad is not None}
        ev = trainer.evaluate(torch.nn.CrossEntropyLoss())
        runs[proj] = (metrics["loss"], grads, ev)
    (l0, g0, e0), (l1, g1, e1) = runs["off"], runs["auto"]
    assert abs(l0 - l1) < 1e-5
    assert set(g0) == set(g1)
    for k, err in grad_errs(g1, g0).items():
        assert err <= 1e-5, (k, err)
    assert e0["val_acc"] == e1["val_acc"]


@pytest.mark.parametrize("model_kind", ["gcn", "gat", "gat2"])
def test_merged_layers_match_per_partition(gpu, model_kind):
    """config.merge_partitions: layers run as one pass over the whole graph's
    adjacency ('auto': every layer here, GCN's widening first layer in place;
    'last': the last layer, with one loss and one dW product), against the
    per-partition passes ('off') of the same flow, on a 20k-node graph with
    a hub destination and a hub source of 3000 edges each (their rows and
    columns split into several work units): loss, metrics and every
    gradient within 1e-5, evaluate() alike, and repeated merged epochs and
    runs bit-identical.  The forward's per-row sums run over the same edges
    in the same order either way; the backward's per-source sums and the
    last layer's dW differ only in fp32 association."""
    from grinnder_amd.data import synthetic

    n, classes = 20_000, 5
    ei = synthetic.uniform_graph(n, 200_000, seed=9)
    hub = torch.arange(2, 3002)
    ei = torch.cat([ei, torch.stack([hub, torch.zeros_like(hub)]),
                    torch.stack([torch.ones_like(hub), hub + 3000])], 1)
    nd = synthetic.node_data(n, 24, classes, seed=9)
    torch.manual_seed(5)
    if model_kind == "gcn":
        make = lambda: GCN(24, 32, classes, num_layers=3, dropout=0.0, norm=True)  # noqa: E731
    else:
        heads = 2 if model_kind == "gat2" else 1
        make = lambda: GAT(24, 16, classes, num_layers=2, heads=heads, dropout=0.0,  # noqa
                           norm=True)
    state = make().state_dict()
    runs = {}
    for merge in ("off", "last", "auto", "auto"):
        config = GriNNderConfig(num_parts=6, merge_partitions=merge)
        graph = build_partitioned_graph(ei, nd.x, nd.y, nd.train_mask, nd.val_mask,
                                        nd.test_mask, config)
        model = make().cuda()
        model.load_state_dict(state)
        trainer = Trainer(model, graph, config)
        opt = torch.optim.SGD(model.parameters(), lr=0.0)
        metrics = trainer.train_epoch(opt, torch.nn.CrossEntropyLoss())
        last = model.num_layers - 1
        expect = {"off": [], "last": [last], "auto": list(range(model.num_layers))}[merge]
        assert trainer.merged_layers == expect
        grads = {k: p.grad.detach().clone() for k, p in model.named_parameters()
                 if p.grad is not None}
        opt.zero_grad()
        again = trainer.train_epoch(opt, torch.nn.CrossEntropyLoss())
        grads2 = {k: p.grad.detach().clone() for k, p in model.named_parameters()
                  if p.grad is not None}
        ev = trainer.evaluate(torch.nn.CrossEntropyLoss())
        runs.setdefault(merge, []).append((metrics, grads, again, grads2, ev))
        del trainer, model, graph
    (m0, g0, _, _, e0), = runs["off"]
    for m1, g1, a1, g12, e1 in runs["last"] + runs["auto"]:
        assert abs(m0["loss"] - m1["loss"]) <= 1e-5 * max(1.0, abs(m0["loss"]))
        assert m0["val_acc"] == m1["val_acc"] and m0["test_acc"] == m1["test_acc"]
        assert set(g0) == set(g1)
        for k, err in grad_errs(g1, g0).items():
            assert err <= 1e-5, (k, err)
        assert a1["loss"] == m1["loss"]
        assert all(torch.equal(g1[k], g12[k]) for k in g1)
        assert abs(e0["loss"] - e1["loss"]) <= 1e-5 * max(1.0, abs(e0["loss"]))
        assert e0["val_acc"] == e1["val_acc"]
    (_, ga, _, _, _), (_, gb, _, _, _) = runs["auto"]
    assert all(torch.equal(ga[k], gb[k]) for k in ga)


def test_projected_layers_match_dense_vanilla(gpu):
    """The projected flow (layer 0 24 -> 16, last layer 16 -> 3, padded to 4)
    against the float64 dense GCN, and a widening first layer (8 -> 16)."""
    data = _graph_data(feat=24)
    torch.manual_seed(7)
    make = lambda: GCN(24, 16, 3, num_layers=2, dropout=0.0, norm=True)  # noqa: E731
    state = make().state_dict()
    ref_loss, ref_grads = _vanilla(data, state, make)
    loss, grads, trainer, _ = _step(data, state, make, 4, "grinnder")
    assert trainer.projected_layers == [0, 1]
    assert abs(loss - ref_loss) < 1e-5
    for k, err in grad_errs(grads, ref_grads).items():
        assert err <= 1e-5, (k, err)
    data = _graph_data(feat=8)
    make = lambda: GCN(8, 16, 3, num_layers=2, dropout=0.0, norm=True)  # noqa: E731
    state = make().state_dict()
    ref_loss, ref_grads = _vanilla(data, state, make)
    loss, grads, trainer, _ = _step(data, state, make, 4, "grinnder")
    # The widening first layer aggregates its narrower input in place.
    assert trainer.projected_layers == [1] and trainer.inplace_layers == [0]
    assert abs(loss - ref_loss) < 1e-5
    for k, err in grad_errs(grads, ref_grads).items():
        assert err <= 1e-5, (k, err)


@pytest.mark.parametrize("project_first", ["off", "auto"])
def test_dropped_trainer_releases_pinned_memory(gpu, project_first):
    """A Trainer's pinned host buffers are released when the last reference
    to it goes, by reference counting alone (the cyclic collector is off
    here), so a second trainer in the same process does not find the
    first one's pinned memory still mapped."""
    import gc

    from grinnder_amd.buffer.host import PINNED_STATS

    data = _graph_data(n=60, reach=3, feat=24, classes=4)
    make = lambda: GCN(24, 16, 4, num_layers=3, dropout=0.0, norm=True)  # noqa: E731
    gc.collect()
    before = dict(PINNED_STATS)
    gc.disable()
    try:
        ei, x, y, tr, va, te = data
        config = GriNNderConfig(num_parts=4, project_first=project_first)
        graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
        model = make().cuda()
        trainer = Trainer(model, graph, config)
        trainer.train_epoch(torch.optim.SGD(model.parameters(), lr=0.1),
                            torch.nn.CrossEntropyLoss())
        torch.cuda.synchronize()
        assert PINNED_STATS["bytes"] > before["bytes"]
        del trainer, model, graph
        assert PINNED_STATS["bytes"] == before["bytes"]
        assert PINNED_STATS["blocks"] == before["blocks"]
    finally:
        gc.enable()


@pytest.mark.parametrize("model_kind", ["gcn", "gat"])
@pytest.mark.parametrize("resident", [True, False])
def test_projected_layers_match_gathered_at_scale(gpu, model_kind, resident, monkeypatch):
    """The projected flow against the reference flow on a graph large enough
    that the dW pass's uploads run while compute work is still queued
    (300k nodes, 8 partitions, widths 128/256), with the layer inputs kept
    in HBM for the epoch or uploaded again for dW, both against a float64
    torch restatement of the model on the unpartitioned graph
    (tests/restate.py):

    - the loss of each flow is within 1e-5 of float64, and the two flows'
      losses agree within 1e-5;
    - every gradient of each flow is within 1e-5 of float64, or no further
      from it than 1.5x the distance of the reference's own fp32 arithmetic
      (the same restatement in float32: torch sparse / index ops and torch
      GEMMs) - each weight gradient sums ~180k training rows' contributions
      that cancel, which no fp32 arithmetic resolves to 1e-5;
    - the two flows' gradients agree within 1e-5 (grad_errs), or, where
      both are that far from float64, within twice the fp32 restatement's
      distance (each is within 1.5x of it).  That case is the first GCN
      layer with its inputs uploaded again for dW: the reference flow's
      GCNConv aggregates the 128-wide input first ((A X) Wᵀ) while the
      default flow projects first (A (X Wᵀ)), so the two weight gradients
      sum the same terms in another order (both ~6-9e-5 from float64, as
      torch's fp32 is 6.3e-5);
    - two projected epochs give bit-identical gradients."""
    from grinnder_amd.data import synthetic
    from tests.restate import model_epoch

    if not resident:
        _limit_resident_inputs(monkeypatch, set())
    n = 300_000
    ei = synthetic.uniform_graph(n, 3_000_000, seed=5)
    nd = synthetic.node_data(n, 128, 16, seed=5)
    torch.manual_seed(11)
    if model_kind == "gcn":
        make = lambda: GCN(128, 256, 16, num_layers=3, dropout=0.0, norm=True)  # noqa: E731
    else:
        make = lambda: GAT(128, 256, 16, num_layers=2, heads=1, dropout=0.0, norm=True)  # noqa
    state = make().state_dict()
    ref_loss, ref_grads = model_epoch(model_kind, ei, nd.x, nd.y, nd.train_mask, state, make,
                                      gpu)
    t32_loss, t32_grads = model_epoch(model_kind, ei, nd.x, nd.y, nd.train_mask, state, make,
                                      gpu, dtype=torch.float32)
    t32_err = grad_errs(t32_grads, ref_grads)
    print(f"{model_kind} 300k: float64 loss {ref_loss:.8f}, torch fp32 {t32_loss:.8f}; torch "
          f"fp32 grads vs float64 {({k: f'{v:.1e}' for k, v in t32_err.items()})}", flush=True)
    runs = []
    for proj in ("off", "auto", "auto"):
        config = GriNNderConfig(num_parts=8, project_first=proj)
        graph = build_partitioned_graph(ei, nd.x, nd.y, nd.train_mask, nd.val_mask,
                                        nd.test_mask, config)
        model = make().cuda()
        model.load_state_dict(state)
        trainer = Trainer(model, graph, config)
        metrics = trainer.train_epoch(torch.optim.SGD(model.parameters(), lr=0.0),
                                      torch.nn.CrossEntropyLoss())
        n_fast = len(trainer.projected_layers) + len(trainer.inplace_layers)
        assert n_fast == (0 if proj == "off" else model.num_layers)
        # GCN's first layer widens (128 -> 256): in place when its input is in HBM.
        assert trainer.inplace_layers == ([0] if proj == "auto" and resident
                                          and model_kind == "gcn" else [])
        runs.append((metrics["loss"], {k: p.grad.detach().clone()
                                       for k, p in model.named_parameters()}))
        del trainer, model, graph
    (l0, g0), (l1, g1), (l2, g2) = runs
    for name, loss, grads in (("off", l0, g0), ("auto", l1, g1)):
        err = grad_errs({k: v.cpu() for k, v in grads.items()}, ref_grads)
        print(f"{model_kind} 300k {name}: loss rel err {abs(loss - ref_loss) / abs(ref_loss):.1e}"
              f"; grads vs float64 {({k: f'{v:.1e}' for k, v in err.items()})}", flush=True)
        assert abs(loss - ref_loss) / abs(ref_loss) <= TOL
        for k, e in err.items():
            assert e <= max(TOL, 1.5 * t32_err[k]), (name, k, e, t32_err[k])
    assert abs(l0 - l1) / abs(l0) <= TOL
    flows = grad_errs(g1, g0)
    print(f"{model_kind} 300k auto vs off: {({k: f'{v:.1e}' for k, v in flows.items()})}",
          flush=True)
    for k, e in flows.items():
        assert e <= max(TOL, 2.0 * t32_err[k]), (k, e, t32_err[k])
    assert all(torch.equal(g1[k], g2[k]) for k in g1)


@pytest.mark.parametrize("keep_products", [True, False])
def test_gathered_layers_match_reference_flow_at_scale(gpu, keep_products, monkeypatch):
    """GAT with input dropout 0.6 on the 300k-node graph (8 partitions,
    widths 128 -> 256 -> 16, two heads in the first layer): every layer is
    gathered from HBM, against the reference flow from the same seed.  The
    two flows run the same kernels on the same rows with the same dropout
    masks, and add each input-gradient row in the same partition order, so
    the loss and every gradient are bit-identical, whether the recompute
    takes each partition's projection product kept by its forward
    (forward_gathered) or forms it again."""
    from grinnder_amd.data import synthetic

    plan = Trainer._plan_projection
    compute_losses = Trainer._compute_losses
    kept_counts = []

    def planned(self):
        out = plan(self)
        if not keep_products:
            self._gkept_left = 0
        return out

    def losses(self):
        kept_counts.append(len(self._gkept))
        return compute_losses(self)
    monkeypatch.setattr(Trainer, "_plan_projection", planned)
    monkeypatch.setattr(Trainer, "_compute_losses", losses)
    n = 300_000
    ei = synthetic.uniform_graph(n, 3_000_000, seed=6)
    nd = synthetic.node_data(n, 128, 16, seed=6)
    torch.manual_seed(12)
    make = lambda: GAT(128, 128, 16, num_layers=3, heads=2, dropout=0.6, norm=True)  # noqa
    state = make().state_dict()
    runs = {}
    for proj in ("off", "auto"):
        config = GriNNderConfig(num_parts=8, project_first=proj)
        graph = build_partitioned_graph(ei, nd.x, nd.y, nd.train_mask, nd.val_mask,
                                        nd.test_mask, config)
        model = make().cuda()
        model.load_state_dict(state)
        trainer = Trainer(model, graph, config)
        torch.manual_seed(77)
        metrics = trainer.train_epoch(torch.optim.SGD(model.parameters(), lr=0.0),
                                      torch.nn.CrossEntropyLoss())
        assert trainer.gathered_layers == ([] if proj == "off" else [0, 1, 2])
        assert trainer._gkept == {}
        runs[proj] = (metrics["loss"], {k: p.grad.detach().clone()
                                        for k, p in model.named_parameters()})
        del trainer, model, graph
    # Every layer of every partition kept its product for the recompute.
    assert kept_counts == [0, 3 * 8 if keep_products else 0]
    (l0, g0), (l1, g1) = runs["off"], runs["auto"]
    assert l0 == l1
    for k in g0:
        assert torch.equal(g0[k], g1[k]), (k, grad_errs({k: g1[k]}, {k: g0[k]}))


def _no_kept_graphs(monkeypatch):
    """Plans as usual but recomputes every projected layer in its backward."""
    plan = Trainer._plan_projection

    def recompute(self):
        out = plan(self)
        self._keep = set()
        return out
    monkeypatch.setattr(Trainer, "_plan_projection", recompute)


@pytest.mark.parametrize("flow", ["reference", "kept_graph", "recompute", "gathered",
                                  "gat_reference"])
def test_dropout_gradient_matches_finite_difference(gpu, flow, monkeypatch):
    """With dropout active, the backward must see the masks the forward drew:
    the reference flow's checkpoint restores the RNG state, a projected layer
    either keeps its forward graph or recomputes from the RNG state its
    forward started from, and so does a gathered layer (GAT with input
    dropout, gathered from HBM).  Every epoch below starts from the same
    seed, so its forward draws the same masks and the reported loss is one
    smooth function of the weights: its central difference along the
    gradient must equal the gradient's norm (a backward that drew new masks
    is off by tens of percent)."""
    data = _graph_data(n=60, reach=3, feat=24, classes=4)
    ei, x, y, tr, va, te = data
    if flow == "recompute":
        _no_kept_graphs(monkeypatch)
    torch.manual_seed(5)
    if flow in ("gathered", "gat_reference"):
        model = GAT(24, 8, 4, num_layers=3, heads=2, dropout=0.5, norm=True).cuda()
    else:
        model = GCN(24, 32, 4, num_layers=3, dropout=0.5, norm=True).cuda()
    reference = flow in ("reference", "gat_reference")
    config = GriNNderConfig(num_parts=4, project_first="off" if reference else "auto")
    graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
    trainer = Trainer(model, graph, config)
    opt = torch.optim.SGD(model.parameters(), lr=0.0)
    crit = torch.nn.CrossEntropyLoss()

    def epoch():
        torch.manual_seed(123)
        return trainer.train_epoch(opt, crit)["loss"]

    epoch()
    if reference:
        assert trainer.projected_layers == [] and trainer.gathered_layers == []
    elif flow == "gathered":
        assert trainer.projected_layers == [] and trainer.gathered_layers == [0, 1, 2]
    else:
        # 24 -> 32 widens: the first layer reads its input rows in place.
        assert trainer.projected_layers == [1, 2] and trainer.inplace_layers == [0]
        assert sorted(trainer._keep) == ([0, 1, 2] if flow == "kept_graph" else [])
    w = model.convs[1].lin.weight
    g = w.grad.detach().clone()
    v = g / g.norm()
    # GAT's attention logits pass a LeakyReLU, whose kinks the step can
    # cross: at 1e-2 the central difference is 0.8% off in both flows alike.
    delta = 1e-3 if model.__class__ is GAT else 1e-2
    with torch.no_grad():
        w.add_(delta * v)
    up = epoch()
    with torch.no_grad():
        w.sub_(2 * delta * v)
    down = epoch()
    with torch.no_grad():
        w.add_(delta * v)
    fd = (up - down) / (2 * delta)
    assert abs(fd - float(g.norm())) <= 2e-3 * float(g.norm()) + 1e-4, (fd, float(g.norm()))


@pytest.mark.parametrize("model_kind", ["gcn", "gat", "gat_dropout"])
def test_layer0_prefetch_across_epochs_is_exact(gpu, model_kind, monkeypatch):
    """Layer 0's input rows for the next epoch stream into a second buffer
    while an epoch computes: three training epochs (weights changing) and an
    evaluate() in between give bit-identical weights and metrics with and
    without that prefetch.  With GAT's input dropout, layer 0 is gathered
    from those rows in training and projected from them in evaluate()."""
    data = _graph_data(n=60, reach=3, feat=24, classes=4, train_all=False)
    ei, x, y, tr, va, te = data
    torch.manual_seed(4)
    if model_kind == "gcn":
        make = lambda: GCN(24, 32, 4, num_layers=3, dropout=0.0, norm=True)  # noqa: E731
    else:
        p = 0.5 if model_kind == "gat_dropout" else 0.0
        make = lambda: GAT(24, 8, 4, num_layers=2, heads=1, dropout=p, norm=True)  # noqa
    state = make().state_dict()
    plan = Trainer._plan_projection
    runs = []
    for prefetch in (True, False):
        if not prefetch:
            def single(self):
                out = plan(self)
                self._x0double = False
                self._drop_prefetch()
                return out
            monkeypatch.setattr(Trainer, "_plan_projection", single)
        config = GriNNderConfig(num_parts=4)
        graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
        model = make().cuda()
        model.load_state_dict(state)
        trainer = Trainer(model, graph, config)
        opt = torch.optim.SGD(model.parameters(), lr=0.5)
        crit = torch.nn.CrossEntropyLoss()
        metrics = []
        for i, step in enumerate(("train", "eval", "train", "train")):
            torch.manual_seed(300 + i)
            metrics.append(trainer.train_epoch(opt, crit) if step == "train"
                           else trainer.evaluate(crit))
        assert len(trainer._x0bufs) == (2 if prefetch else 1)
        if model_kind == "gat_dropout":
            assert trainer.gathered_layers == [0, 1]
        runs.append((metrics, {k: v.detach().clone() for k, v in model.state_dict().items()}))
    (m0, w0), (m1, w1) = runs
    assert [m["loss"] for m in m0] == [m["loss"] for m in m1]
    assert all(torch.equal(w0[k], w1[k]) for k in w0)


@pytest.mark.parametrize("num_parts,model_kind", [(1, "gcn"), (1, "gcn_narrow"), (4, "gcn"),
                                                  (4, "gat")])
def test_input_residency_stream_equals_resident(gpu, num_parts, model_kind):
    """input_residency 'stream' (features uploaded every epoch, the next
    epoch's upload overlapped) and 'resident' (uploaded once): four steps
    with the weights changing and an evaluate() in between give
    bit-identical metrics and weights, on the single-partition path and on
    the partitioned projected flow."""
    data = _graph_data(n=60, reach=3, feat=24, classes=4, train_all=False)
    ei, x, y, tr, va, te = data
    torch.manual_seed(5)
    if model_kind == "gcn":
        make = lambda: GCN(24, 32, 4, num_layers=3, dropout=0.0, norm=True)  # noqa: E731
    elif model_kind == "gcn_narrow":  # layer 0 projects first: autograd keeps x for dW
        make = lambda: GCN(24, 16, 4, num_layers=2, dropout=0.0, norm=True)  # noqa: E731
    else:
        make = lambda: GAT(24, 8, 4, num_layers=2, heads=1, dropout=0.0, norm=True)  # noqa
    state = make().state_dict()
    runs = []
    for residency in ("stream", "resident"):
        config = GriNNderConfig(num_parts=num_parts, input_residency=residency)
        graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
        model = make().cuda()
        model.load_state_dict(state)
        trainer = Trainer(model, graph, config)
        opt = torch.optim.Adam(model.parameters(), lr=0.05)
        crit = torch.nn.CrossEntropyLoss()
        metrics = [trainer.train_epoch(opt, crit) if step == "train" else trainer.evaluate(crit)
                   for step in ("train", "eval", "train", "train")]
        if num_parts == 1:
            assert (trainer._uploads is not None) == (residency == "stream")
        else:
            assert 0 in trainer.resident_inputs or 0 in trainer.inplace_layers
            assert len(trainer._x0bufs) == (2 if residency == "stream" else 1)
        runs.append((metrics, {k: v.detach().clone() for k, v in model.state_dict().items()}))
    (m0, w0), (m1, w1) = runs
    assert m0 == m1
    assert all(torch.equal(w0[k], w1[k]) for k in w0)


@pytest.mark.parametrize("pool_size", [1, 2])
@pytest.mark.parametrize("resident", ["all", "projected", "none"])
def test_mixed_flows_match_reference(gpu, pool_size, resident, monkeypatch):
    """A residual GCN whose 16 -> 16 layers cannot be projected (the residual
    add needs x itself): layers 0 and 3 run projected, layers 1 and 2 are
    gathered from HBM (all inputs resident) or take the reference flow's host
    buffers (only the projected layers' inputs resident, or none), so outputs
    and gradients cross between the flows in both directions (device Z rows,
    resident inputs and host buffers forward; host gradient buffers, dL/dx
    buffers and dZ W backward).  Loss, gradients and evaluate() equal those of
    the reference flow throughout within the 1e-5 bound, over two epochs."""
    kept = {"all": [0, 1, 2, 3], "projected": [0, 3], "none": []}[resident]
    if resident != "all":
        _limit_resident_inputs(monkeypatch, set(kept))
    data = _graph_data(n=60, reach=3, feat=24, classes=4, train_all=False)
    ei, x, y, tr, va, te = data
    torch.manual_seed(6)
    make = lambda: GCN(24, 16, 4, num_layers=4, dropout=0.0, norm=True,  # noqa: E731
                       residual=True)
    state = make().state_dict()
    runs = {}
    for proj in ("off", "auto"):
        config = GriNNderConfig(num_parts=4, pool_size=pool_size, project_first=proj)
        graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
        model = make().cuda()
        model.load_state_dict(state)
        trainer = Trainer(model, graph, config)
        opt = torch.optim.SGD(model.parameters(), lr=0.0)
        crit = torch.nn.CrossEntropyLoss()
        losses = [trainer.train_epoch(opt, crit)["loss"]]
        grads = {n: p.grad.detach().clone() for n, p in model.named_parameters()}
        losses.append(trainer.train_epoch(opt, crit)["loss"])
        ev = trainer.evaluate(crit)
        if proj == "auto":
            assert trainer.projected_layers == [0, 3]
            assert trainer.resident_inputs == kept
            assert trainer.gathered_layers == [l for l in kept if l in (1, 2)]
        runs[proj] = (losses, grads, ev)
    (l0, g0, e0), (l1, g1, e1) = runs["off"], runs["auto"]
    assert all(abs(a - b) < 1e-5 for a, b in zip(l0, l1))
    for k, err in grad_errs(g1, g0).items():
        assert err <= 1e-5, (k, err)
    assert e0["val_acc"] == e1["val_acc"]


@pytest.mark.parametrize("heads", [1, 2])
@pytest.mark.parametrize("pool_size", [1, 2])
@pytest.mark.parametrize("resident", ["all", "above0", "none"])
def test_gathered_layers_match_reference_flow(gpu, heads, pool_size, resident, monkeypatch):
    """GAT with input dropout (0.6, the model's default): no layer can run
    projected in training, so every layer is gathered from HBM when its input
    rows stay there (all layers, those above layer 0, or none: the reference
    flow's host buffers).  Over two seeded epochs the loss, the gradients and
    evaluate() (which runs projected: dropout is off) equal the reference
    flow's within the 1e-5 bound."""
    kept = {"all": [0, 1, 2], "above0": [1, 2], "none": []}[resident]
    if resident != "all":
        _limit_resident_inputs(monkeypatch, set(kept))
    data = _graph_data(n=60, reach=3, feat=24, classes=4, train_all=False)
    ei, x, y, tr, va, te = data
    torch.manual_seed(9)
    make = lambda: GAT(24, 8, 4, num_layers=3, heads=heads, norm=True)  # noqa: E731
    state = make().state_dict()
    runs = {}
    for proj in ("off", "auto"):
        config = GriNNderConfig(num_parts=4, pool_size=pool_size, project_first=proj)
        graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
        model = make().cuda()
        model.load_state_dict(state)
        assert model.dropout == 0.6
        trainer = Trainer(model, graph, config)
        opt = torch.optim.SGD(model.parameters(), lr=0.0)
        crit = torch.nn.CrossEntropyLoss()
        torch.manual_seed(200)
        losses = [trainer.train_epoch(opt, crit)["loss"]]
        grads = {n: p.grad.detach().clone() for n, p in model.named_parameters()}
        if proj == "auto":
            assert trainer.projected_layers == [] and trainer.gathered_layers == kept
        torch.manual_seed(201)
        losses.append(trainer.train_epoch(opt, crit)["loss"])
        ev = trainer.evaluate(crit)
        if proj == "auto":
            assert trainer.projected_layers == [0, 1, 2] and trainer.gathered_layers == []
        runs[proj] = (losses, grads, ev)
    (l0, g0, e0), (l1, g1, e1) = runs["off"], runs["auto"]
    assert all(abs(a - b) < 1e-5 for a, b in zip(l0, l1)), (l0, l1)
    for k, err in grad_errs(g1, g0).items():
        assert err <= 1e-5, (k, err)
    assert e0["val_acc"] == e1["val_acc"]


@pytest.mark.parametrize("budget_parts", [0, 1, 3])
def test_gathered_partial_keep_budget_is_exact(gpu, budget_parts, monkeypatch):
    """When HBM holds the forward's projection products of only some
    partitions (a budget of 0, 1 or 3 partitions' worth), those recompute
    from the kept product and the others form it again: the loss and the
    gradients are bit-identical to keeping every partition's product."""
    data = _graph_data(n=60, reach=3, feat=24, classes=4, train_all=False)
    ei, x, y, tr, va, te = data
    torch.manual_seed(19)
    make = lambda: GAT(24, 8, 4, num_layers=2, heads=2, dropout=0.6, norm=True)  # noqa
    state = make().state_dict()
    plan = Trainer._plan_projection
    compute_losses = Trainer._compute_losses
    budget = {"bytes": None}
    kept = []

    def planned(self):
        out = plan(self)
        if budget["bytes"] is not None:
            self._gkept_left = budget["bytes"]
        return out

    def losses(self):
        kept.append(len(self._gkept))
        return compute_losses(self)
    monkeypatch.setattr(Trainer, "_plan_projection", planned)
    monkeypatch.setattr(Trainer, "_compute_losses", losses)
    runs = []
    for limited in (False, True):
        config = GriNNderConfig(num_parts=4)
        graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
        if limited:
            # Layer 0's products of `budget_parts` average partitions.
            per_part = sum(graph.expanded_sizes) // graph.num_parts * 16 * 4
            budget["bytes"] = budget_parts * per_part
        model = make().cuda()
        model.load_state_dict(state)
        trainer = Trainer(model, graph, config)
        torch.manual_seed(33)
        loss = trainer.train_epoch(torch.optim.SGD(model.parameters(), lr=0.0),
                                   torch.nn.CrossEntropyLoss())["loss"]
        assert trainer.gathered_layers == [0, 1]
        runs.append((loss, {k: p.grad.detach().clone() for k, p in model.named_parameters()}))
    (l0, g0), (l1, g1) = runs
    # Two layers of four partitions: all eight kept without a limit, fewer
    # with one (none for a zero budget).
    assert kept[0] == 8 and (kept[1] == 0 if budget_parts == 0 else 0 < kept[1] < 8)
    assert l0 == l1
    assert all(torch.equal(g0[k], g1[k]) for k in g0)


@pytest.mark.parametrize("model_kind", ["gcn_widening", "gcn_narrowing"])
def test_training_trajectory_matches_reference_flow(gpu, model_kind):
    """Three Adam epochs (weight decay, dropout 0.5 on layer outputs) from the
    same weights in the reference flow and the default (projected / in place)
    flow: every epoch's loss agrees within 1e-5 and the final weights within
    1e-4 of their largest entry.  Each partition draws its dropout mask over
    its own output rows in partition order in both flows, so the masks agree."""
    data = _graph_data(n=60, reach=3, feat=24, classes=4, train_all=False)
    ei, x, y, tr, va, te = data
    hidden = 32 if model_kind == "gcn_widening" else 16
    torch.manual_seed(8)
    make = lambda: GCN(24, hidden, 4, num_layers=3, dropout=0.5, norm=True)  # noqa: E731
    state = make().state_dict()
    runs = {}
    for proj in ("off", "auto"):
        config = GriNNderConfig(num_parts=4, project_first=proj)
        graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
        model = make().cuda()
        model.load_state_dict(state)
        trainer = Trainer(model, graph, config)
        opt = torch.optim.Adam(model.parameters(), lr=0.01, weight_decay=5e-4)
        crit = torch.nn.CrossEntropyLoss()
        losses = []
        for ep in range(3):
            torch.manual_seed(100 + ep)
            losses.append(trainer.train_epoch(opt, crit)["loss"])
        if proj == "auto":
            assert trainer.projected_layers + trainer.inplace_layers != []
        runs[proj] = (losses, {k: v.detach().clone() for k, v in model.state_dict().items()})
    (l0, w0), (l1, w1) = runs["off"], runs["auto"]
    assert all(abs(a - b) < 1e-5 for a, b in zip(l0, l1)), (l0, l1)
    for k, err in grad_errs(w1, w0).items():
        assert err <= 1e-4, (k, err)


@pytest.mark.parametrize("model_kind", ["gcn", "gat", "gat_dropout", "gcn_residual"])
def test_empty_partitions_match_reference_flow(gpu, model_kind):
    """A 12-node graph cut into 8 partitions, two of them empty: every flow
    (projected and in place for GCN, projected GAT, gathered GAT with input
    dropout, gathered residual GCN) gives the reference flow's loss,
    gradients and evaluate() within the 1e-5 bound, in both modes."""
    n = 12
    src = torch.tensor([0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 0, 3])
    dst = torch.tensor([1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 5, 9])
    ei = torch.stack([torch.cat([src, dst]), torch.cat([dst, src])])
    g = torch.Generator().manual_seed(3)
    x = torch.randn(n, 8, generator=g)
    y = torch.randint(0, 3, (n,), generator=g)
    tr = torch.zeros(n, dtype=torch.bool)
    tr[::2] = True
    va, te = ~tr, torch.zeros(n, dtype=torch.bool)
    torch.manual_seed(13)
    make = {
        "gcn": lambda: GCN(8, 16, 3, num_layers=2, dropout=0.0, norm=True),
        "gat": lambda: GAT(8, 4, 3, num_layers=2, heads=2, dropout=0.0, norm=True),
        "gat_dropout": lambda: GAT(8, 4, 3, num_layers=2, heads=2, dropout=0.5, norm=True),
        "gcn_residual": lambda: GCN(8, 8, 3, num_layers=3, dropout=0.0, norm=True,
                                    residual=True),
    }[model_kind]
    state = make().state_dict()
    for mode in ("grinnder", "hongtu"):
        runs = {}
        for proj in ("off", "auto"):
            config = GriNNderConfig(num_parts=8, mode=mode, project_first=proj)
            graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
            assert 0 in graph.partition_sizes
            model = make().cuda()
            model.load_state_dict(state)
            trainer = Trainer(model, graph, config)
            torch.manual_seed(21)
            loss = trainer.train_epoch(torch.optim.SGD(model.parameters(), lr=0.0),
                                       torch.nn.CrossEntropyLoss())["loss"]
            grads = {k: p.grad.detach().clone() for k, p in model.named_parameters()}
            runs[proj] = (loss, grads, trainer.evaluate(torch.nn.CrossEntropyLoss()))
        (l0, g0, e0), (l1, g1, e1) = runs["off"], runs["auto"]
        assert abs(l0 - l1) < 1e-5, (mode, l0, l1)
        for k, err in grad_errs(g1, g0).items():
            assert err <= 1e-5, (mode, k, err)
        assert abs(e0["loss"] - e1["loss"]) < 1e-5
        assert (e0["val_acc"], e0["test_acc"]) == (e1["val_acc"], e1["test_acc"])


def _random_config(seed):
    import random
    r = random.Random(seed)
    kind = r.choice(["gcn", "gat"])
    layers = r.randint(2, 4)
    feat = r.choice([3, 8, 12, 20])
    hidden = r.choice([4, 8, 12, 16])
    classes = r.choice([3, 4, 5])
    norm = r.random() < 0.7
    parts = r.choice([2, 3, 5])
    pool = r.choice([1, 2])
    if kind == "gcn":
        residual = r.random() < 0.4
        make = lambda: GCN(feat, hidden, classes, num_layers=layers, dropout=0.0,  # noqa: E731
                           norm=norm, residual=residual)
        desc = f"gcn L={layers} {feat}->{hidden}->{classes} norm={norm} residual={residual}"
    else:
        heads = r.choice([1, 2])
        # Active input dropout keeps GAT layers off the projected flow: they
        # run gathered from HBM.
        dropout = r.choice([0.0, 0.0, 0.5])
        make = lambda: GAT(feat, hidden, classes, num_layers=layers, heads=heads,  # noqa: E731
                           dropout=dropout, norm=norm)
        desc = f"gat L={layers} {feat}->{hidden}x{heads}->{classes} norm={norm} dropout={dropout}"
    return make, feat, classes, parts, pool, f"{desc} P={parts} pool={pool}"


@pytest.mark.parametrize("seed", range(24))
def test_random_configs_match_reference_flow(gpu, seed):
    """Seeded random models and partitionings (GCN / GAT, 2-4 layers, widths
    that are and are not multiples of 4, widening and narrowing first layers,
    residual layers that cannot be projected, GAT with and without input
    dropout, 1-2 heads, 2-5 partitions, both pool sizes): the default flow's
    loss, gradients and evaluate() equal the reference flow's within the 1e-5
    bound."""
    make, feat, classes, parts, pool, desc = _random_config(seed)
    print(f"config {seed}: {desc}", flush=True)
    data = _graph_data(n=50, reach=3, feat=feat, classes=classes, seed=seed,
                       train_all=False)
    ei, x, y, tr, va, te = data
    torch.manual_seed(seed)
    state = make().state_dict()
    runs = {}
    for proj in ("off", "auto"):
        config = GriNNderConfig(num_parts=parts, pool_size=pool, project_first=proj)
        graph = build_partitioned_graph(ei, x, y, tr, va, te, config)
        model = make().cuda()
        model.load_state_dict(state)
        trainer = Trainer(model, graph, config)
        opt = torch.optim.SGD(model.parameters(), lr=0.0)
        crit = torch.nn.CrossEntropyLoss()
        torch.manual_seed(1000 + seed)
        loss = trainer.train_epoch(opt, crit)["loss"]
        grads = {n: p.grad.detach().clone() for n, p in model.named_parameters()
                 if p.grad is not None}
        ev = trainer.evaluate(crit)
        runs[proj] = (loss, grads, ev)
    (l0, g0, e0), (l1, g1, e1) = runs["off"], runs["auto"]
    assert abs(l0 - l1) < 1e-5, desc
    assert set(g0) == set(g1), desc
    for k, err in grad_errs(g1, g0).items():
        assert err <= 1e-5, (desc, k, err)
    assert e0["val_acc"] == e1["val_acc"], desc

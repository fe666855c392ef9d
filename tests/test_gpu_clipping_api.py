"""GPU parity of the clipping API: the materialised-leaf seam, ``clipped_grad`` /
``clipped_fun`` / ``auto_clipped_grad`` and model-level ghost clipping, each
against the CPU oracle on the same inputs.

Tolerances: the reference's own fused-kernel contract
(packages/opake-patches/tests/kernels/test_clip_sum.py:167-195: norms rtol
1e-6, clipped norms rtol 1e-5, sums ``assert_close`` defaults) for the leaf
kernels; 1e-5 relative (fp32) / 2e-2 relative (bf16) for the ghost path.
"""

from __future__ import annotations

import math

import pytest
import torch

from opake_amd import clipping as cl
from opake_amd.exceptions import OperationError
from opake_amd.noise import gaussian_noise
from opake_amd.random import key
from opake_amd.types import ClippedPytree, NoisedPytree
from oracle import clip_oracle, ghost_oracle

pytestmark = pytest.mark.gpu


class _Scale:
    def __init__(self, kind, gamma=0.0):
        self.kind, self.gamma = kind, gamma


def _reduce(x):
    acc = torch.float32 if x.dtype in (torch.bfloat16, torch.float16) else None
    return torch.sum(x, dim=0, dtype=acc).to(x.dtype)


def _rel(got, want):
    got, want = got.double().cpu(), want.double().cpu()
    return ((got - want).norm() / want.norm().clamp_min(1e-300)).item()


# --- materialised-leaf seam -------------------------------------------------------


def _values(gen, B, dtypes):
    shapes = [(5, 7), (3000,), (11,), (64, 70), (1,)]
    tree = {}
    for i, shape in enumerate(shapes):
        dt = dtypes[i % len(dtypes)]
        scale = torch.exp(torch.randn(B, *([1] * len(shape)), generator=gen))
        tree[f"p{i}"] = (torch.randn(B, *shape, generator=gen) * scale * 0.1).to(dt)
    return tree


@pytest.mark.parametrize("dtypes", [[torch.float32], [torch.bfloat16],
                                    [torch.float32, torch.bfloat16]])
@pytest.mark.parametrize("kind", ["fixed", "auto_s"])
def test_leaf_backend_matches_streaming_oracle(dev, dtypes, kind):
    gen = torch.Generator().manual_seed(len(dtypes) * 7 + (kind == "auto_s"))
    B = 9
    tree = _values(gen, B, dtypes)
    tree["p1"][2, 17] = math.nan
    tree["p3"][4, 0, 3] = math.inf
    names = sorted(tree)
    C = clip_oracle.conservative_bound(0.5)
    gamma = 0.01 if kind == "auto_s" else 0.0
    res = clip_oracle.stream_clip_and_sum([tree[n] for n in names], C, kind=kind, gamma=gamma,
                                          return_aux=True)
    dev_tree = {k: v.to(dev) for k, v in tree.items()}
    reduced, markers, sq, sqm, diag = cl.fused_stream_clip_and_sum(
        dev_tree, torch.tensor(C, device=dev), scale=_Scale(kind, gamma), batch_size=B,
        reduce_leaf=_reduce, compute_dtype=None, second_moment=False, return_aux=True,
        return_stats=False)
    assert sq == () and sqm == ()
    for i, n in enumerate(names):
        assert reduced[n].dtype == tree[n].dtype
        assert markers[n].dtype == tree[n].dtype and markers[n].dim() == 0
        torch.testing.assert_close(reduced[n].cpu(), res.reduced[i])
    torch.testing.assert_close(diag["norms"].cpu().double(), res.norms, rtol=1e-6, atol=0)
    torch.testing.assert_close(diag["clipped_norms"].cpu().double(),
                               res.clipped_norms.double(), rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("second_moment", [False, True])
def test_leaf_kernels_whole_ragged_and_unaligned_tiles(dev, dtype, second_moment):
    """Leaves that exercise every path of the leaf kernels: whole 2048-element
    tiles read with 16-byte loads, a ragged last tile, rows that do not start
    16-byte aligned (n * elem_size % 16 != 0), output offsets that are not
    16-byte aligned, and a batch that is not a multiple of the apply kernel's
    4-example unroll."""
    gen = torch.Generator().manual_seed(11 + second_moment)
    B = 19
    shapes = [(4096,), (2049,), (8, 1031), (3,), (16392,), (2, 2048)]
    tree = {}
    for i, shape in enumerate(shapes):
        scale = torch.exp(torch.randn(B, *([1] * len(shape)), generator=gen))
        tree[f"p{i}"] = (torch.randn(B, *shape, generator=gen) * scale * 0.02).to(dtype)
    tree["p4"][7, 5000] = math.nan
    tree["p0"][18, 3] = -math.inf
    names = sorted(tree)
    C = clip_oracle.conservative_bound(1.0)
    res = clip_oracle.stream_clip_and_sum([tree[n] for n in names], C, return_aux=True,
                                          second_moment=second_moment)
    dev_tree = {k: v.to(dev) for k, v in tree.items()}
    reduced, _, sq, _, diag = cl.fused_stream_clip_and_sum(
        dev_tree, torch.tensor(C, device=dev), scale=_Scale("fixed"), batch_size=B,
        reduce_leaf=_reduce, compute_dtype=None, second_moment=second_moment, return_aux=True,
        return_stats=False)
    for i, n in enumerate(names):
        torch.testing.assert_close(reduced[n].cpu(), res.reduced[i])
        if second_moment:
            torch.testing.assert_close(sq[n].cpu(), res.squared[i])
    torch.testing.assert_close(diag["norms"].cpu().double(), res.norms, rtol=1e-6, atol=0)
    torch.testing.assert_close(diag["clipped_norms"].cpu().double(),
                               res.clipped_norms.double(), rtol=1e-5, atol=1e-7)


def test_leaf_backend_boundary_pin(dev):
    # [[3,4],[0.6,0.8]], C = 1 -> [1.2, 1.6] (test_clip_sum.py:156-161).
    batch = {"w": torch.tensor([[3.0, 4.0], [0.6, 0.8]], device=dev)}
    reduced, *_ = cl.fused_stream_clip_and_sum(
        batch, torch.tensor(1.0, device=dev), scale=_Scale("fixed"), batch_size=2,
        reduce_leaf=_reduce, compute_dtype=None, second_moment=False, return_aux=False,
        return_stats=False)
    torch.testing.assert_close(reduced["w"].cpu(), torch.tensor([1.2, 1.6]))


def test_leaf_backend_many_leaves_and_stored_bound(dev):
    gen = torch.Generator().manual_seed(3)
    B = 4
    tree = {f"l{i:03d}": (torch.randn(B, 64, generator=gen) * 10).to(torch.bfloat16)
            for i in range(120)}
    dev_tree = {k: v.to(dev) for k, v in tree.items()}
    # Per-example stored values: run with B = 1 slices; every stored norm <= C.
    for b in range(B):
        one = {k: v[b:b + 1] for k, v in dev_tree.items()}
        red, *_ = cl.fused_stream_clip_and_sum(
            one, torch.tensor(1.0, device=dev), scale=_Scale("fixed"), batch_size=1,
            reduce_leaf=_reduce, compute_dtype=None, second_moment=False, return_aux=False,
            return_stats=False)
        norm = math.sqrt(sum(float((v.double().cpu() ** 2).sum()) for v in red.values()))
        assert norm <= 1.0


def test_leaf_backend_unsupported_raises_or_falls_back(dev):
    # Integer leaves have no kernel (the reference's torch path serves them).
    tree = {"w": torch.arange(12, device=dev, dtype=torch.int32).reshape(3, 4)}
    kw = dict(scale=_Scale("fixed"), batch_size=3, reduce_leaf=_reduce, compute_dtype=None,
              second_moment=False, return_aux=False, return_stats=False)
    with pytest.raises(OperationError, match="int32"):
        cl.fused_stream_clip_and_sum(tree, torch.tensor(1.0, device=dev), **kw)
    called = {}

    def fallback(values, clipping_norm, **kwargs):
        called["yes"] = True
        return "fallback"

    backend = cl.make_fused_backend(fallback)
    assert backend(tree, torch.tensor(1.0, device=dev), **kw) == "fallback"
    assert called


def test_register_backend_roundtrip():
    cl.register_fused_clip_backend(cl.fused_stream_clip_and_sum)
    assert cl.get_fused_clip_backend() is cl.fused_stream_clip_and_sum
    cl.register_fused_clip_backend(None)


# --- clipped_grad / clipped_fun ------------------------------------------------------


def test_clipped_grad_docstring_closed_form(dev):
    f = lambda p, d: 0.5 * ((d - p) ** 2).mean()  # noqa: E731
    g, st = cl.clipped_grad(f, clipping_norm=float("inf"), return_aux=True)
    (res, aux), st2 = g(torch.tensor(3.0, device=dev), torch.tensor([0.0, 7.0, -2.0], device=dev),
                        state=st)
    assert isinstance(res, ClippedPytree) and st2 is st
    assert res.pytree.item() == pytest.approx(4.0)
    torch.testing.assert_close(aux.loss_values.cpu(), torch.tensor([4.5, 8.0, 12.5]))
    torch.testing.assert_close(aux.grad_norms.cpu(), torch.tensor([3.0, 4.0, 5.0]))
    assert aux.clipping_rate == 0.0 and aux.batch_size == 3


def test_clipped_fun_mean_closed_form(dev):
    # _clipped_fun.py:524-531: clipped_fun(torch.mean, C=1) over [0..5] -> 5.0, max_norm 1.0.
    fn, st = cl.clipped_fun(torch.mean, clipping_norm=1.0)
    out, _ = fn(torch.arange(6.0, device=dev).reshape(6, 1), state=st)
    assert out.max_norm == 1.0
    assert out.pytree.item() == pytest.approx(5.0)


@pytest.mark.parametrize("microbatch", [None, 100])
def test_clipped_grad_mlp_config1_matches_oracle(dev, microbatch):
    torch.manual_seed(0)
    model = ghost_oracle.MLP()
    params = {k: v.detach() for k, v in model.named_parameters()}
    gen = torch.Generator().manual_seed(1)
    B = 256
    x = torch.randn(B, 784, generator=gen)
    y = torch.randint(0, 10, (B,), generator=gen)
    per = ghost_oracle.mlp_per_example_grads(model, params, x, y)
    names = sorted(per)
    res = clip_oracle.stream_clip_and_sum([per[n] for n in names], clip_oracle.conservative_bound(1.0))

    dmodel = ghost_oracle.MLP().to(dev)
    dmodel.load_state_dict(model.state_dict())
    dparams = {k: v.detach() for k, v in dmodel.named_parameters()}

    def loss_fn(p, xb, yb):
        logits = torch.func.functional_call(dmodel, p, (xb.unsqueeze(0),))
        return torch.nn.functional.cross_entropy(logits, yb.unsqueeze(0))

    g, st = cl.clipped_grad(loss_fn, clipping_norm=1.0, normalize_by=float(B), return_stats=True,
                            batch_argnums=(1, 2), microbatch_size=microbatch)
    (out, stats), _ = g(dparams, x.to(dev), y.to(dev), state=st)
    assert out.max_norm == pytest.approx(1.0 / B)
    for i, n in enumerate(names):
        assert _rel(out.pytree[n], res.reduced[i] / B) < 1e-5, n
    assert stats.num_clipped == clip_oracle.num_clipped(res.norms.float(), 1.0)


def test_auto_clipped_grad_formula(dev):
    f = lambda p, d: (p * d).sum()  # noqa: E731  per-example grad = d
    g, st = cl.auto_clipped_grad(f, R=1.0, gamma=0.01)
    d = torch.tensor([[3.0, 4.0], [0.3, 0.4]], device=dev)
    out, _ = g(torch.zeros(2, device=dev), d, state=st)
    want = d[0].cpu() / 5.01 + d[1].cpu() / 0.51
    torch.testing.assert_close(out.pytree.cpu(), want, rtol=1e-6, atol=1e-7)


# --- model-level ghost clipping ----------------------------------------------------------


def _mlp_oracle(model, x, y, C, nb):
    params = {k: v.detach() for k, v in model.named_parameters()}
    per = ghost_oracle.mlp_per_example_grads(model, params, x, y)
    names = sorted(per)
    res = clip_oracle.stream_clip_and_sum([per[n] for n in names], clip_oracle.conservative_bound(C))
    return names, [r / nb for r in res.reduced], res


def test_ghost_clipped_grad_mlp_config1(dev):
    torch.manual_seed(0)
    model = ghost_oracle.MLP()
    gen = torch.Generator().manual_seed(2)
    B = 256
    x = torch.randn(B, 784, generator=gen)
    y = torch.randint(0, 10, (B,), generator=gen)
    names, want, res = _mlp_oracle(model, x, y, 1.0, float(B))
    dmodel = ghost_oracle.MLP().to(dev)
    dmodel.load_state_dict(model.state_dict())
    loss = lambda out, t: torch.nn.functional.cross_entropy(out, t, reduction="none")  # noqa: E731
    g, st = cl.ghost_clipped_grad(dmodel, loss, clipping_norm=1.0, normalize_by=float(B),
                                  return_aux=True)
    (out, aux), _ = g(x.to(dev), y.to(dev), state=st)
    assert sorted(out.pytree) == names and list(out.pytree) == names
    for i, n in enumerate(names):
        assert _rel(out.pytree[n], want[i]) < 1e-5, n
    torch.testing.assert_close(aux.grad_norms.cpu().double(), res.norms, rtol=1e-5, atol=0)
    assert int(aux.num_clipped.item()) == clip_oracle.num_clipped(res.norms.float(), 1.0)
    assert all(p.grad is None for p in dmodel.parameters())


@pytest.mark.parametrize("stream", ["reference", "device"])
def test_ghost_clipped_grad_fused_noise_equals_separate_noise(dev, stream):
    torch.manual_seed(1)
    model = ghost_oracle.MLP(64, 32, 10).to(dev)
    x = torch.randn(16, 64, device=dev)
    y = torch.randint(0, 10, (16,), device=dev)
    loss = lambda out, t: torch.nn.functional.cross_entropy(out, t, reduction="none")  # noqa: E731
    g, st = cl.ghost_clipped_grad(model, loss, clipping_norm=1.0, normalize_by=16.0)
    noise_fn, nstate = gaussian_noise(noise_multiplier=1.3, key=key(5), stream=stream)
    fused, _, nstate2 = g(x, y, state=st, noise_fn=noise_fn, noise_state=nstate)
    assert isinstance(fused, NoisedPytree) and nstate2._step_counter == 1
    center, _ = g(x, y, state=st)
    sep, _ = noise_fn(center, nstate)
    for n in sep.pytree:
        assert torch.equal(fused.pytree[n], sep.pytree[n]), n
    assert fused.noise_stddev == pytest.approx(1.3 / 16.0)


def test_ghost_clipped_grad_sequence_bf16(dev):
    torch.manual_seed(2)
    B, T, d = 4, 128, 64
    model = torch.nn.Sequential(torch.nn.Linear(d, 96), torch.nn.GELU(),
                                torch.nn.Linear(96, d, bias=False))
    x = torch.randn(B, T, d)
    tgt = torch.randn(B, T, d)

    def loss(out, t):
        return ((out.float() - t.float()) ** 2).mean(dim=(1, 2))

    # Oracle: per-example grads by vmap(grad) in float64 on the same bf16 weights.
    mb = model.to(torch.bfloat16)
    params = {k: v.detach().double() for k, v in mb.named_parameters()}
    m64 = torch.nn.Sequential(torch.nn.Linear(d, 96), torch.nn.GELU(),
                              torch.nn.Linear(96, d, bias=False)).double()

    def loss_one(p, xi, ti):
        out = torch.func.functional_call(m64, p, (xi.unsqueeze(0),))
        return ((out - ti.unsqueeze(0)) ** 2).mean()

    xb = x.to(torch.bfloat16)
    per = torch.func.vmap(torch.func.grad(loss_one), in_dims=(None, 0, 0))(
        params, xb.double(), tgt.double())
    names = sorted(per)
    res = clip_oracle.stream_clip_and_sum([per[n].to(torch.bfloat16) for n in names],
                                          clip_oracle.conservative_bound(0.05))
    dmodel = mb.to(dev)
    g, st = cl.ghost_clipped_grad(dmodel, loss, clipping_norm=0.05, return_aux=True)
    (out, aux), _ = g(xb.to(dev), tgt.to(dev), state=st)
    for i, n in enumerate(names):
        assert _rel(out.pytree[n], res.reduced[i]) < 2e-2, n
    torch.testing.assert_close(aux.grad_norms.cpu().double(), res.norms, rtol=2e-2, atol=0)


# --- per-group clipping ------------------------------------------------------------------


def _per_group(names, assignment, values):
    from opake_amd.types import PerGroup
    return PerGroup({n: assignment[n] for n in names}, values)


@pytest.mark.parametrize("kind", ["fixed", "auto_s"])
def test_leaf_backend_per_group_matches_streaming_oracle(dev, kind):
    gen = torch.Generator().manual_seed(11 + (kind == "auto_s"))
    B = 7
    tree = _values(gen, B, [torch.float32, torch.bfloat16])
    tree["p3"][1, 2, 5] = math.nan
    names = sorted(tree)
    assignment = {"p0": "attn", "p1": "mlp", "p2": "attn", "p3": "emb", "p4": "mlp"}
    values = {"attn": 0.3, "mlp": 0.05, "emb": 2.0}
    cons = {g: clip_oracle.conservative_bound(v) for g, v in values.items()}
    gamma = 0.01 if kind == "auto_s" else 0.0
    res = clip_oracle.stream_clip_and_sum(
        [tree[n] for n in names], None, kind=kind, gamma=gamma,
        groups=[assignment[n] for n in names], group_values=cons, return_aux=True)
    pg = _per_group(names, assignment, values)
    dev_tree = {k: v.to(dev) for k, v in tree.items()}
    reduced, _, _, _, diag = cl.fused_stream_clip_and_sum(
        dev_tree, pg, scale=_Scale(kind, gamma), batch_size=B, reduce_leaf=_reduce,
        compute_dtype=None, second_moment=False, return_aux=True, return_stats=False)
    for i, n in enumerate(names):
        assert reduced[n].dtype == tree[n].dtype
        torch.testing.assert_close(reduced[n].cpu(), res.reduced[i])
    torch.testing.assert_close(diag["norms"].cpu().double(), res.norms, rtol=1e-6, atol=0)
    assert set(diag["group_norms"]) == set(values)
    for g in values:
        torch.testing.assert_close(diag["group_norms"][g].cpu().double(), res.group_norms[g],
                                   rtol=1e-6, atol=0)
    torch.testing.assert_close(diag["clipped_norms"].cpu().double(),
                               res.clipped_norms.double(), rtol=1e-5, atol=1e-7)


def test_clip_pytree_per_group_closed_form(dev):
    # attn = [3, 4] with C_attn = 1 -> [0.6, 0.8]; mlp = [0.3, 0.4] with C_mlp = 1 unchanged.
    tree = {"attn": torch.tensor([3.0, 4.0], device=dev),
            "mlp": torch.tensor([0.3, 0.4], device=dev)}
    pg = _per_group(["attn", "mlp"], {"attn": "a", "mlp": "m"}, {"a": 1.0, "m": 1.0})
    out, aux = cl.clip_pytree(tree, pg)
    torch.testing.assert_close(out["attn"].cpu(), torch.tensor([0.6, 0.8]), rtol=1e-6, atol=0)
    assert torch.equal(out["mlp"].cpu(), tree["mlp"].cpu())
    assert aux.group_norms["a"].item() == pytest.approx(5.0)
    assert aux.group_norms["m"].item() == pytest.approx(0.5)
    assert aux.norm.item() == pytest.approx(math.sqrt(25.25))


def test_per_group_path_mismatch_raises(dev):
    from opake_amd.exceptions import ConfigurationError
    tree = {"a": torch.ones(2, 3, device=dev), "b": torch.ones(2, 3, device=dev)}
    pg = _per_group(["a"], {"a": "g"}, {"g": 1.0})
    with pytest.raises(ConfigurationError, match="Leaves with no group assignment"):
        cl.fused_stream_clip_and_sum(
            tree, pg, scale=_Scale("fixed"), batch_size=2, reduce_leaf=_reduce,
            compute_dtype=None, second_moment=False, return_aux=False, return_stats=False)


@pytest.mark.parametrize("microbatch", [None, 3])
def test_clipped_grad_per_group_stats_and_aux(dev, microbatch):
    gen = torch.Generator().manual_seed(5)
    B = 8
    d_w, d_b = torch.randn(B, 6, generator=gen) * 2, torch.randn(B, 3, generator=gen) * 0.1

    def loss(p, dw, db):  # per-example grads: w -> dw, b -> db
        return (p["w"] * dw).sum() + (p["b"] * db).sum()

    params = {"w": torch.zeros(6, device=dev), "b": torch.zeros(3, device=dev)}
    pg = _per_group(["w", "b"], {"w": "weights", "b": "bias"}, {"weights": 1.5, "bias": 0.2})
    cons = {"weights": clip_oracle.conservative_bound(1.5),
            "bias": clip_oracle.conservative_bound(0.2)}
    res = clip_oracle.stream_clip_and_sum([d_b, d_w], None, groups=["bias", "weights"],
                                          group_values=cons, return_aux=True)
    g, st = cl.clipped_grad(loss, clipping_norm=pg, normalize_by=2.0, batch_argnums=(1, 2),
                            return_aux=True, microbatch_size=microbatch)
    (out, aux), _ = g(params, d_w.to(dev), d_b.to(dev), state=st)
    assert out.max_norm.values == {"weights": 0.75, "bias": 0.1}
    torch.testing.assert_close(out.pytree["b"].cpu(), res.reduced[0] / 2.0)
    torch.testing.assert_close(out.pytree["w"].cpu(), res.reduced[1] / 2.0)
    assert aux.clipping_rate is None and aux.batch_size == B
    for gname in ("weights", "bias"):
        torch.testing.assert_close(aux.group_norms[gname].cpu().double(), res.group_norms[gname],
                                   rtol=1e-6, atol=0)
    g2, st2 = cl.clipped_grad(loss, clipping_norm=pg, batch_argnums=(1, 2), return_stats=True,
                              microbatch_size=microbatch)
    (_, stats), _ = g2(params, d_w.to(dev), d_b.to(dev), state=st2)
    want = {gname: float((res.group_norms[gname].float() > v).sum())
            for gname, v in (("weights", 1.5), ("bias", 0.2))}
    assert stats.num_clipped == want
    assert stats.clipping_rate == {k: v / B for k, v in want.items()}
    assert stats.batch_size == B


# --- single-pytree clipping ----------------------------------------------------------------


def test_clip_pytree_closed_forms(dev):
    x = {"w": torch.tensor([3.0, 4.0], device=dev)}
    out, aux = cl.clip_pytree(x, 0.0)
    assert torch.equal(out["w"].cpu(), torch.zeros(2)) and aux.norm.item() == 5.0
    out, _ = cl.clip_pytree(x, float("inf"))
    assert torch.equal(out["w"].cpu(), x["w"].cpu())
    out, aux = cl.clip_pytree(x, 1.0)
    assert float(out["w"].double().norm()) == pytest.approx(1.0, rel=1e-6)
    assert float(out["w"].double().norm()) <= 1.0
    small = {"w": torch.tensor([0.3, 0.4], device=dev)}
    out, _ = cl.clip_pytree(small, 1.0)
    assert torch.equal(out["w"].cpu(), small["w"].cpu())
    bad = {"w": torch.tensor([math.nan, math.inf, 2.0], device=dev)}
    out, aux = cl.clip_pytree(bad, 10.0)
    assert torch.equal(out["w"].cpu(), torch.tensor([0.0, 0.0, 2.0])) and aux.norm.item() == 2.0
    out, _ = cl.clip_pytree(x, 1.0, return_zero=True)
    assert torch.equal(out["w"].cpu(), torch.zeros(2))
    zero = {"w": torch.zeros(4, device=dev)}
    out, _ = cl.clip_pytree(zero, 1.0)
    assert torch.equal(out["w"].cpu(), torch.zeros(4))
    # AUTO-S: [3,4], R=1, gamma=0.01 -> x / 5.01; zeros stay zeros (test_auto.py:24-62).
    out, aux = cl.auto_scale_pytree(x, R=1.0, gamma=0.01)
    torch.testing.assert_close(out["w"].cpu(), torch.tensor([3.0, 4.0]) / 5.01, rtol=1e-6,
                               atol=0)
    out, _ = cl.auto_scale_pytree(zero, R=1.0, gamma=0.01)
    assert torch.equal(out["w"].cpu(), torch.zeros(4))
    from opake_amd.exceptions import ConfigurationError
    with pytest.raises(ConfigurationError):
        cl.auto_scale_pytree(x, R=1.0, gamma=0.0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_clip_pytree_matches_oracle(dev, dtype):
    gen = torch.Generator().manual_seed(21)
    tree = {"a": (torch.randn(37, 5, generator=gen) * 3).to(dtype),
            "b": (torch.randn(9000, generator=gen)).to(dtype), "c": 1.5}
    names = ["a", "b"]
    for C in (0.7, 1e6):
        want, want_norm = clip_oracle.clip_pytree_scalar([tree[n] for n in names], C)
        out, aux = cl.clip_pytree({k: (v.to(dev) if torch.is_tensor(v) else v)
                                   for k, v in tree.items()}, C)
        assert out["c"] == 1.5
        for n, w in zip(names, want):
            torch.testing.assert_close(out[n].cpu(), w)
        torch.testing.assert_close(aux.norm.cpu(), want_norm, rtol=1e-6, atol=0)
    want, _ = clip_oracle.auto_scale_scalar([tree[n] for n in names], 0.5, 0.01)
    out, _ = cl.auto_scale_pytree({n: tree[n].to(dev) for n in names}, R=0.5, gamma=0.01)
    for n, w in zip(names, want):
        torch.testing.assert_close(out[n].cpu(), w)


# --- second moment ----------------------------------------------------------------------


@pytest.mark.parametrize("per_group", [False, True])
def test_leaf_backend_second_moment_matches_oracle(dev, per_group):
    gen = torch.Generator().manual_seed(31 + per_group)
    B = 6
    tree = _values(gen, B, [torch.float32, torch.bfloat16])
    names = sorted(tree)
    if per_group:
        assignment = {"p0": "a", "p1": "b", "p2": "a", "p3": "b", "p4": "a"}
        values = {"a": 0.4, "b": 0.1}
        C = _per_group(names, assignment, values)
        res = clip_oracle.stream_clip_and_sum(
            [tree[n] for n in names], None, groups=[assignment[n] for n in names],
            group_values={g: clip_oracle.conservative_bound(v) for g, v in values.items()},
            second_moment=True)
    else:
        C = torch.tensor(clip_oracle.conservative_bound(0.3), device=dev)
        res = clip_oracle.stream_clip_and_sum([tree[n] for n in names], float(C),
                                              second_moment=True)
    reduced, markers, squared, sq_markers, _ = cl.fused_stream_clip_and_sum(
        {k: v.to(dev) for k, v in tree.items()}, C, scale=_Scale("fixed"), batch_size=B,
        reduce_leaf=_reduce, compute_dtype=None, second_moment=True, return_aux=False,
        return_stats=False)
    for i, n in enumerate(names):
        assert squared[n].dtype == tree[n].dtype and sq_markers[n].dtype == tree[n].dtype
        torch.testing.assert_close(reduced[n].cpu(), res.reduced[i])
        torch.testing.assert_close(squared[n].cpu(), res.squared[i])


@pytest.mark.parametrize("microbatch", [None, 2])
def test_clipped_grad_second_moment_and_paired_noise(dev, microbatch):
    from opake_amd.types import SecondMomentClippingOutput, SecondMomentNoiseOutput

    gen = torch.Generator().manual_seed(41)
    d = torch.randn(5, 12, generator=gen) * 0.7

    def loss(p, db):  # per-example gradient = db
        return (p * db).sum()

    g, st = cl.clipped_grad(loss, clipping_norm=1.5, normalize_by=5.0, batch_argnums=1,
                            second_moment=True, microbatch_size=microbatch)
    out, _ = g(torch.zeros(12, device=dev), d.to(dev), state=st)
    assert isinstance(out, SecondMomentClippingOutput)
    assert out.grads.max_norm == pytest.approx(1.5 / 5.0)
    assert out.squared_grads.max_norm == pytest.approx(1.5 * 1.5 / 5.0)
    res = clip_oracle.stream_clip_and_sum([d], clip_oracle.conservative_bound(1.5),
                                          second_moment=True)
    assert _rel(out.grads.pytree, res.reduced[0] / 5.0) < 1e-6
    assert _rel(out.squared_grads.pytree, res.squared[0] / 5.0) < 1e-6
    noise_fn, nstate = gaussian_noise(noise_multiplier=1.0, key=key(3), stream="device")
    noisy, _ = noise_fn(out, nstate)
    assert isinstance(noisy, SecondMomentNoiseOutput)
    assert not torch.equal(noisy.noisy_grads.pytree, out.grads.pytree)


# --- microbatching in ghost_clipped_grad ---------------------------------------------------


def test_ghost_clipped_grad_microbatch_matches_full_batch(dev):
    torch.manual_seed(0)
    model = ghost_oracle.MLP()
    gen = torch.Generator().manual_seed(2)
    B = 256
    x = torch.randn(B, 784, generator=gen)
    y = torch.randint(0, 10, (B,), generator=gen)
    names, want, res = _mlp_oracle(model, x, y, 1.0, float(B))
    dmodel = ghost_oracle.MLP().to(dev)
    dmodel.load_state_dict(model.state_dict())
    loss = lambda out, t: torch.nn.functional.cross_entropy(out, t, reduction="none")  # noqa: E731
    g, st = cl.ghost_clipped_grad(dmodel, loss, clipping_norm=1.0, normalize_by=float(B),
                                  return_aux=True, microbatch_size=100)
    (out, aux), _ = g(x.to(dev), y.to(dev), state=st)
    for i, n in enumerate(names):
        assert _rel(out.pytree[n], want[i]) < 1e-5, n
    assert aux.batch_size == B and aux.loss_values.shape == (B,)
    torch.testing.assert_close(aux.grad_norms.cpu().double(), res.norms, rtol=1e-5, atol=0)
    assert int(aux.num_clipped.item()) == clip_oracle.num_clipped(res.norms.float(), 1.0)
    noise_fn, nstate = gaussian_noise(noise_multiplier=1.0, key=key(4), stream="device")
    noisy, st2, nstate2 = g(x.to(dev), y.to(dev), state=st, noise_fn=noise_fn, noise_state=nstate)
    assert isinstance(noisy[0], NoisedPytree) and nstate2._step_counter == 1

"""Pins of the per-example gradient oracle (oracle/ghost_oracle.py) -- CPU only.

The reference materialises per-example gradients with ``vmap(grad)``
(packages/opake-engine/src/opake/api/engine/clipping/_clipped_grad.py:278-296).
The oracle's closed form ``G_i^T A_i`` (+ ``sum_t G_i[t]`` for a bias) is
checked against torch.func on the surrogate loss and against a per-example
autograd loop through a real ``nn.Linear``; the Gram identity
``||G_i^T A_i||^2 = <A_i A_i^T, G_i G_i^T>`` is checked against the
materialised norm.  The config-1 MLP's vmap(grad) is checked against a loop of
single-example backward passes.
"""

from __future__ import annotations

import torch

from oracle import ghost_oracle


def test_linear_closed_form_matches_vmap_grad():
    g = torch.Generator().manual_seed(0)
    A = torch.randn(3, 5, 7, generator=g, dtype=torch.float64)
    G = torch.randn(3, 5, 4, generator=g, dtype=torch.float64)
    closed = ghost_oracle.linear_per_example_grads(A, G)[0]
    vm = ghost_oracle.surrogate_per_example_grads(A, G)
    torch.testing.assert_close(closed, vm, rtol=1e-12, atol=1e-12)


def test_linear_closed_form_matches_autograd_loop_with_bias():
    g = torch.Generator().manual_seed(1)
    B, T, din, dout = 4, 6, 5, 3
    A = torch.randn(B, T, din, generator=g, dtype=torch.float64)
    lin = torch.nn.Linear(din, dout).double()
    targets = torch.randn(B, T, dout, generator=g, dtype=torch.float64)
    ws, bs, Gs = [], [], []
    for i in range(B):
        lin.zero_grad()
        y = lin(A[i])
        y.retain_grad()
        loss = 0.5 * ((y - targets[i]) ** 2).sum()
        loss.backward()
        ws.append(lin.weight.grad.clone())
        bs.append(lin.bias.grad.clone())
        Gs.append(y.grad.clone())
    G = torch.stack(Gs)
    b, w = ghost_oracle.linear_per_example_grads(A, G, with_bias=True)
    torch.testing.assert_close(w, torch.stack(ws), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(b, torch.stack(bs), rtol=1e-12, atol=1e-12)


def test_gram_identity():
    g = torch.Generator().manual_seed(2)
    A = torch.randn(3, 9, 6, generator=g, dtype=torch.float64)
    G = torch.randn(3, 9, 4, generator=g, dtype=torch.float64)
    w = ghost_oracle.linear_per_example_grads(A, G)[0]
    direct = (w * w).sum(dim=(1, 2))
    gram = ((A @ A.transpose(1, 2)) * (G @ G.transpose(1, 2))).sum(dim=(1, 2))
    torch.testing.assert_close(gram, direct, rtol=1e-12, atol=0)
    # Flat inputs (T == 1): ||a||^2 ||g||^2.
    a, gg = A[:, :1], G[:, :1]
    w1 = ghost_oracle.linear_per_example_grads(a, gg)[0]
    torch.testing.assert_close((w1 * w1).sum(dim=(1, 2)),
                               (a[:, 0] ** 2).sum(1) * (gg[:, 0] ** 2).sum(1), rtol=1e-12, atol=0)


def test_mlp_vmap_grad_matches_loop():
    torch.manual_seed(0)
    model = ghost_oracle.MLP(12, 8, 3).double()
    params = {k: v.detach() for k, v in model.named_parameters()}
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 12, generator=g, dtype=torch.float64)
    y = torch.randint(0, 3, (5,), generator=g)
    got = ghost_oracle.mlp_per_example_grads(model, params, x, y)
    for i in range(5):
        model.zero_grad()
        loss = torch.nn.functional.cross_entropy(model(x[i:i + 1]), y[i:i + 1])
        loss.backward()
        for k, p in model.named_parameters():
            torch.testing.assert_close(got[k][i], p.grad, rtol=1e-10, atol=1e-12)


def test_per_example_loop_matches_vmap_grad_mlp():
    torch.manual_seed(3)
    model = ghost_oracle.MLP(12, 9, 4).double()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(5, 12, generator=g, dtype=torch.float64)
    y = torch.randint(0, 4, (5,), generator=g)
    params = {k: v.detach() for k, v in model.named_parameters()}
    vm = ghost_oracle.mlp_per_example_grads(model, params, x, y)
    loop = ghost_oracle.per_example_grads_loop(
        model, lambda out, t: torch.nn.functional.cross_entropy(out, t, reduction="none"),
        (x,), y)
    for k in vm:
        torch.testing.assert_close(loop[k], vm[k], rtol=1e-12, atol=1e-12)


def _moe_setup(seed=0, B=3, T=7, d=6, inter=5, E=4, k=2):
    from opake_amd.moe import TopKMoE

    torch.manual_seed(seed)
    model = TopKMoE(d, inter, E, k, dtype=torch.float64)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(B, T, d, generator=g, dtype=torch.float64)
    logits = torch.randn(B, T, E, generator=g, dtype=torch.float64)
    target = torch.randn(B, T, d, generator=g, dtype=torch.float64)
    return model, x, logits, target


def _mse(out, t):
    return ((out - t) ** 2).sum(dim=(1, 2))


def test_moe_matches_dense_reference_forward():
    # moe.py:74-103 of the reference: dense loop over experts with route weights.
    model, x, logits, _ = _moe_setup()
    out = model(x, logits)
    top_v, top_i = torch.topk(logits, model.top_k, dim=-1)
    w = torch.softmax(top_v, dim=-1)
    ref = torch.zeros_like(x)
    for e, ex in enumerate(model.experts):
        gu = x @ ex.gate_up.weight.T
        h = torch.nn.functional.silu(gu[..., :model.inter]) * gu[..., model.inter:]
        y = h @ ex.down.weight.T
        route = torch.where(top_i == e, w, torch.zeros_like(w)).sum(-1, keepdim=True)
        ref = ref + y * route
    # The module (as the reference) accumulates the expert outputs and takes
    # the SiLU in float32.
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-6)


def test_segment_grads_are_the_per_example_expert_grads():
    # The rows of expert e are its examples' tokens in example order, so the
    # per-segment G_v^T A_v are the per-example gradients of that expert.
    model, x, logits, target = _moe_setup(seed=5)
    caps = {}

    def hook(name):
        def fn(mod, inp, out):
            caps[name] = (inp[0].detach(), out, list(mod.dpc_row_segments))
        return fn

    handles = [m.register_forward_hook(hook(n)) for n, m in model.named_modules()
               if isinstance(m, torch.nn.Linear) and m.weight.requires_grad]
    losses = _mse(model(x, logits), target)
    names = list(caps)
    outs = torch.autograd.grad(losses.sum(), [caps[n][1] for n in names])
    for h in handles:
        h.remove()
    loop = ghost_oracle.per_example_grads_loop(model, _mse, (x, logits), target)
    for n, G in zip(names, outs):
        A, _, seg = caps[n]
        assert len(seg) == x.shape[0] and sum(seg) == A.shape[0]
        got = ghost_oracle.segment_grads(A, G.detach(), seg)
        # The forward takes the SiLU and the output sum in float32, so a batch
        # of one and the full batch agree to float32 rounding.
        torch.testing.assert_close(got, loop[f"{n}.weight"], rtol=1e-6, atol=1e-8)

"""DP metadata of ClippedPytree / NoisedPytree / PerGroup (opake_amd/types.py) -- CPU.

The reference types (packages/opake-engine/src/opake/api/engine/types.py:71-477)
carry the sensitivity with the value: ``sensitivity`` (``max_norm``, or a
PerGroup's effective ``sqrt(sum C_k^2)``), ``noise_stddev_for`` (scalar
``nm * C``; PerGroup "optimal" ``nm * sqrt(C_k * sum_j C_j)``, "isotropic"
``nm * effective``), public-scalar ``*`` and ``/`` that rescale the values and
``|s| * max_norm`` (and a NoisedPytree's ``noise_stddev``), negation, and
``+``, ``-``, ``**``, reverse division raising ``InputTypeError`` (a
``TypeError``).  The reference's own pins: the per-group sigmas 4.0 and
2 sqrt(12) of packages/opake-dpsgd/tests/noise/test_noise.py:206-228.
"""

from __future__ import annotations

import math

import pytest
import torch

from opake_amd.exceptions import ConfigurationError, InputTypeError
from opake_amd.types import ClippedPytree, NoisedPytree, PerGroup, clipped, noised


def _tree():
    return {"b": torch.tensor([1.0, -2.0]), "w": torch.ones(2, 3), "meta": "keep"}


def test_sensitivity_scalar_and_per_group():
    assert clipped(_tree(), max_norm=0.5).sensitivity == 0.5
    pg = PerGroup({"w": "a", "b": "b"}, {"a": 3.0, "b": 4.0})
    assert clipped(_tree(), max_norm=pg).sensitivity == pytest.approx(5.0)
    assert pg.num_groups == 2 and pg.for_path("w") == 3.0 and pg.for_path(("b",)) == 4.0


def test_noise_stddev_for():
    c = clipped(_tree(), max_norm=2.0)
    assert c.noise_stddev_for(noise_multiplier=1.5) == 3.0
    assert c.noise_stddev_for(noise_multiplier=1.5, allocation="isotropic") == 3.0
    assert c.noise_stddev_for(noise_multiplier=0.0) == 0.0
    # The reference's per-group pin: C = {2, 6} -> sigma_k = nm sqrt(C_k (2 + 6)).
    pg = PerGroup({"w": "a", "b": "b"}, {"a": 2.0, "b": 6.0})
    sig = clipped(_tree(), max_norm=pg).noise_stddev_for(noise_multiplier=1.0)
    assert isinstance(sig, PerGroup)
    assert sig.values["a"] == pytest.approx(4.0)
    assert sig.values["b"] == pytest.approx(6.928203230275509)
    iso = clipped(_tree(), max_norm=pg).noise_stddev_for(noise_multiplier=2.0,
                                                          allocation="isotropic")
    assert iso == pytest.approx(2.0 * math.sqrt(40.0))
    with pytest.raises(ConfigurationError):
        c.noise_stddev_for(noise_multiplier=-1.0)
    with pytest.raises(ConfigurationError):
        c.noise_stddev_for(noise_multiplier=1.0, allocation="greedy")
    with pytest.raises(ValueError):  # ConfigurationError is a ValueError
        c.noise_stddev_for(noise_multiplier=-1.0)


@pytest.mark.parametrize("factor", [2.0, -0.5, 3])
def test_scalar_rescaling(factor):
    c = clipped(_tree(), max_norm=0.75)
    for out in (c * factor, factor * c):
        assert isinstance(out, ClippedPytree)
        assert out.max_norm == pytest.approx(abs(factor) * 0.75)
        assert torch.equal(out.pytree["w"], c.pytree["w"] * factor)
        assert torch.equal(out.pytree["b"], c.pytree["b"] * factor)
        assert out.pytree["meta"] == "keep"
    d = c / factor
    assert d.max_norm == pytest.approx(0.75 / abs(factor))
    assert torch.allclose(d.pytree["b"], c.pytree["b"] / factor)
    n = -c
    assert n.max_norm == 0.75 and torch.equal(n.pytree["b"], -c.pytree["b"])


def test_per_group_rescaling_and_products():
    pg = PerGroup({"w": "a", "b": "b"}, {"a": 1.0, "b": 2.0})
    out = clipped(_tree(), max_norm=pg) * -3.0
    assert dict(out.max_norm.values) == {"a": 3.0, "b": 6.0}
    sq = pg * pg
    assert dict(sq.values) == {"a": 1.0, "b": 4.0}
    assert dict((pg / 2.0).values) == {"a": 0.5, "b": 1.0}
    other = PerGroup({"w": "a"}, {"a": 1.0})
    with pytest.raises(ConfigurationError, match="identical group mappings"):
        pg * other


def test_noised_pytree_scales_its_stddev():
    n = noised(_tree(), max_norm=1.0, noise_stddev=0.25)
    out = n * -4.0
    assert isinstance(out, NoisedPytree)
    assert out.max_norm == 4.0 and out.noise_stddev == 1.0
    assert (n / 2.0).noise_stddev == 0.125
    assert noised(_tree(), max_norm=1.0, noise_stddev=None).__mul__(2.0).noise_stddev is None


@pytest.mark.parametrize("op", [
    lambda c: c + 1.0, lambda c: 1.0 + c, lambda c: c - 1.0, lambda c: 1.0 - c,
    lambda c: c + c, lambda c: c ** 2, lambda c: 2.0 / c,
    lambda c: c * torch.tensor(2.0), lambda c: c * True, lambda c: c / "2",
])
def test_unsafe_operations_raise(op):
    c = clipped(_tree(), max_norm=1.0)
    with pytest.raises(InputTypeError):
        op(c)
    with pytest.raises(TypeError):
        op(c)


def test_division_by_zero():
    with pytest.raises(ZeroDivisionError):
        clipped(_tree(), max_norm=1.0) / 0.0


def test_tensor_methods_keep_metadata():
    n = noised(_tree(), max_norm=0.5, noise_stddev=0.1)
    for out in (n.clone(), n.detach(), n.to(torch.float64)):
        assert isinstance(out, NoisedPytree)
        assert out.max_norm == 0.5 and out.noise_stddev == 0.1
        assert out.pytree["meta"] == "keep"
    assert n.to(torch.float64).pytree["w"].dtype == torch.float64


def test_empty_batch_uses_the_transformed_schema_and_dtype():
    # An empty batch returns zeros shaped by pre_clipping_transform, in
    # `dtype` (empty_clipped_grads_like, _helpers.py:95-122); no kernel runs.
    from opake_amd.clipping import clipped_grad

    def loss(p, x):
        return (p["w"] * x).sum()

    fn, st = clipped_grad(loss, clipping_norm=1.0, dtype=torch.float64,
                          pre_clipping_transform=lambda g: {"scaled": g["w"] * 2})
    res, _ = fn({"w": torch.ones(3)}, torch.zeros(0, 3), state=st)
    assert set(res.pytree) == {"scaled"}
    assert res.pytree["scaled"].dtype == torch.float64
    assert torch.equal(res.pytree["scaled"], torch.zeros(3, dtype=torch.float64))


def test_compute_dtype_must_be_floating_point():
    from opake_amd.clipping import clipped_fun

    fn, st = clipped_fun(lambda v: v, batch_argnums=0, clipping_norm=1.0,
                         compute_dtype=torch.int32)
    with pytest.raises(InputTypeError, match="compute_dtype"):
        fn({"x": torch.ones(2, 3)}, state=st)

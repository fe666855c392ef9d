"""CPU oracle of the DP clip -> sum -> noise step (TEST INFRASTRUCTURE ONLY).

This package restates the reference algorithm (JetBrains-Research/opake) on
the CPU so that tests can check the HIP path against it.  It is imported only
by ``tests/``, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg
of ``bench.py``; the product package ``opake_amd`` never imports, links or
executes anything here.

Modules and what pins each of them (see also the header of each module):

* ``clip_oracle``  - clipping numerics and the streaming clip-and-sum of
  ``packages/opake-engine/src/opake/api/engine/clipping/{_pytree,_streaming,
  _clipped_fun}.py``.  Pinned by the reference tests' closed forms
  (``tests/test_oracle_clip.py``) and by brute-force float64 checks.
* ``ghost_oracle`` - per-example gradients of linear layers / the config-1 MLP
  through ``torch.func.vmap(grad)`` (library behaviour), pinned by the
  closed form ``G_i^T A_i`` and by finite differences on tiny inputs.
* ``noise_oracle`` - ``key``/``fold_in`` (BLAKE2b-64) and the reference noise
  stream (CPU ``torch.Generator`` + ``torch.randn`` in flatten order), pinned by
  the reference RNG and noise tests' properties and statistics.
* ``dpc_oracle.c`` - Philox4x32-10 and the device-stream Box-Muller map,
  pinned by the Random123 known-answer vectors.
"""

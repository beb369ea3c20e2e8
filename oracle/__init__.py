"""CPU oracle for the SSD / decode / KDA scan path -- TEST INFRASTRUCTURE ONLY.

This package restates, in float64 numpy, the arithmetic of the reference
(Find-Vulnerabilities/Mamformer, ``mamformer 671b/``) for the hot path:

* ``oracle.ssd``  -- ``selective_scan`` (mamformer/layers/mamba2.py:70-130),
  ``Mamba2Block._recurrent_step`` (mamba2.py:407-458) and the Mamba-2 SSD
  convention mapped onto them by an exact reparameterisation (the "bridge").
* ``oracle.kda``  -- the KDA-Diff linear scans: the reference's normalised
  phi(x)=elu(x)+1 scan (mamformer/layers/kda_diff.py:67-89, 357-478, 564-605;
  mamformer/kernels/triton_ssd.py:121-181) and the decay-gated un-normalised
  recurrence that has no reference function (stated in closed form).
* ``oracle.baseline`` -- a torch-CPU restatement that keeps the reference's
  *cost structure* (materialised (b,L,d_inner,N) tensors and a per-timestep
  loop) so ``bench.py`` can time "the reference's CPU path".

Who may use it: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, and only as the *checker* (or the timed
CPU baseline).  The product package ``mamformer_amd`` never imports it; the
product path has no CPU fallback and fails loudly without its HIP library.

Every function here is pinned by a check that does not retype its formula
(closed forms, brute-force semiseparable / attention matrices, invariants such
as chunked == sequential, linearity, prefill+decode == prefill), see
``tests/test_oracle.py``.  The reference ships no numeric golden vectors for
this path (its tests check shapes, finiteness and self-determinism only:
tests/test_mamba2.py:17-84), so no function is pinned against reference data.
"""

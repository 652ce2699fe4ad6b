"""CPU oracle for brainstate's spiking-network step.

TEST INFRASTRUCTURE ONLY.  This package is a plain numpy restatement of the
reference algorithm (chaobrain/brainstate 0.5.4 plus the arithmetic of its
un-vendored dependencies brainevent and brainpy.state, restated from their call
sites).  It is imported only by ``tests/``, ``__graft_entry__.smoke()`` (as the
checker) and the ``cpu_baseline`` leg of ``bench.py``.  The product
(``brainstate_amd``) never imports it and fails loudly when its HIP library is
missing.

Modules
-------
bsmath    fp32 exp / exprel (Cody-Waite + Taylor), bit-identical op sequence to the
          device functions.  Pinned against float64 ``numpy.exp`` (<= 2 ulp).
conn      fixed-num / CSR connectivity exactly as brainstate/nn/_event_fixedprob.py:142-196.
event     spike compaction, event scatter / gather mat-vec, EventLinear.
neuron    exp-Euler (brainstate/nn/_exp_euler.py:226-249), LIF, COBA-LIF, HH steps.
network   whole E/I network loops (COBA-LIF, COBA-HH) in the per-step order of
          examples/105_COBA_HH_2007_braincell.py:76-82.

Parity status per function (what pins it) is listed in each module header.
Functions marked "parity unpinned" there have no reference test, golden vector or
closed form that fixes their bits; they are restatements from equations only.
"""

"""CPU oracle for the Pairformer pair-stack hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``opendde_amd`` imports this package;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or as the timed CPU baseline),
never as the thing measured or shipped.

``oracle.reference`` restates, in plain PyTorch CPU ops that run in whatever
floating dtype the inputs carry (float64 for pinning, float32 for the parity
tier), the reference's "torch" path for:

* triangle attention (starting / ending node) and its MHA core,
* the triangle multiplicative update (outgoing / incoming), standard and
  in-place (z-cache) forms,
* the pair / single Transition, AttentionPairBias, PairformerBlock and
  PairformerStack.

Each function cites the reference file:line it follows.  How each function is
pinned (float64 brute force, closed forms, invariants, library routines) is
listed in ``oracle.reference.PINNED_BY``; every function there has at least
one independent check in ``tests/test_oracle_*.py``.
"""

"""CPU oracle for the LVSA sparse-attention hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of the two
subsystems this repository implements on MI355X:

* ``oracle.lvsa_mask``   — the frame-granularity mask rules (anchor frames,
  rotated keyframe grid, adaptive / expanded sliding window) and the
  frame-level block CSR the reference hands to its block-sparse backend,
  plus the canonical token-block refinement of that mask.
* ``oracle.attention``   — fp32 masked scaled-dot-product attention over that
  mask (per-frame gather form and explicit-mask form), with log-sum-exp.

Who may use it: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, and there only as the checker or the
timed CPU baseline — never as part of the product path.  The product package
(``longvideosparseattention_amd``) must never import anything from here.

How it is pinned (each function's docstring names its reference lines):

* golden vectors written from the reference implementation in
  ``tests/golden/`` (window bounds, global sets and frame CSR over the
  BASELINE configurations and a random grid);
* the known answers held by the reference's own tests;
* closed forms and brute force (see ``tests/test_oracle_*.py``).
"""

"""TEST INFRASTRUCTURE ONLY -- the checker, never the product.

CPU restatement of the reference's Per-Slot EMA hot path.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
anything from this package, and only to check or to time the reference
algorithm beside the HIP path.  Nothing in ``mathbrain`` imports it; the
product fails loudly when its HIP library is missing instead of falling back
here.

Modules
-------
scan       EMA query scan and key-side boundary scan (C restatement in
           ``ema_oracle.c`` via ctypes, plus pure-Python closed forms for tiny
           cases).  Follows mathbrain/triton_ema_query.py:67-117 and
           mathbrain/triton_flash_ema.py:29-78.
attention  Dense flash-EMA attention (mathbrain/flash_ema_attention.py:19-85,
           generalised with a key-side c_base scatter and an out-of-place state
           update so autograd can differentiate it) and the sparse unique-slot
           form with the absent-slot softmax mass.
gating     Fused symmetric query gating (mathbrain/triton_fused_gating.py:
           179-197, CPU branch :187-195) and its closed-form backward
           (triton_fused_gating.py:61-119, :173-175).

Pinning status (every function is checked in tests/test_oracle_*.py):
  scan.query_scan          pinned: reference KATs + closed form + chunk invariance
  scan.boundary_states     pinned: closed form + dense-state consistency
  attention.dense          pinned: hand-derived KATs, zero-state and
                           constant-gate cases reduced to torch SDPA
  attention.sparse         pinned: equals attention.dense (dense == sparse +
                           absent mass) on random inputs
  attention backward       pinned: float64 gradcheck of the oracle forward and
                           the reference's closed-form gradient formulas
                           (triton_flash_ema.py:336-350, 446-465)
  gating.forward/backward  pinned: torch layer_norm/silu library routines,
                           W_pe=0 special case, float64 gradcheck
"""

"""CPU oracle of the SiQ-VL training hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker (or, for
the baseline, as the timed CPU restatement of the reference path).  The
product (``siq_vl_amd``) never imports it and has no CPU fallback.

Modules:
  attention   -- fp64 numpy varlen attention forward/backward (per-sequence
                 loop), restating the eager path of the reference's models.
  cross_entropy -- fp64 numpy linear cross-entropy forward/backward.
  labels      -- pure-Python restatement of the reference's label masking
                 and of the packing (flattening) collator contract.
  cpu_path    -- the reference's own CPU path (the same torch library calls
                 SDPA / F.cross_entropy the reference reaches), used as the
                 library cross-check and as the timed CPU baseline.

Parity pinning of every function is listed in each module's header.  The
reference repository ships no tests, golden vectors or fixtures for this
path (its arithmetic lives in transformers/torch), so the oracle is pinned
by closed forms, brute force, invariants and a library cross-check.
"""

"""CPU oracle for the MI355X sparse-MoE expert layer -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of seruva19/mirai's
routed expert layer (``CompressedGroupedExperts.run_direct_routed`` and the
helpers it calls). It exists to check the HIP product path and to time the
reference-style CPU baseline. Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the
checker; the product package ``mirai_amd`` never imports it and never falls
back to it.

Modules
  codec    NF4 (blocksize 64, bf16 absmax) and INT8 (per-row, bf16 scale)
           quantise / dequantise, plus bf16 rounding helpers (numpy).
  routing  softmax top-k routing and its renormalisation (numpy / torch).
  plan     the dispatch plan: stable argsort, bincount, cumsum (numpy).
  layer    the expert layer forward and backward in the reference op order
           (torch on CPU, bf16 tensors, fp32 combine).

Every function cites the reference file:line it follows. How each one is
pinned (golden vectors, closed forms, library routines, brute force) is
listed in the tests and in the repository's design notes.
"""

"""CPU oracle for the ATMA global-layer mixer -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU (fp32 / fp64), the reference
algorithm of the four hot-path operations the HIP library implements:

* Polar attention (materialised ``polar_reduce`` and the streaming form the
  kernels follow) -- ``oracle.polar``;
* the paged Polar decode (dense reduce over the gathered pages) -- ``oracle.polar``;
* the gated-delta memory: sequential definition, chunked UT/WY form, the FLA
  ``chunk_gated_delta_rule`` contract and the single-token decode step --
  ``oracle.gated_delta``;
* the paged KV write ``store_kvcache`` -- ``oracle.kvcache``;
* one global block (Polar + memory + MLP) for the CPU baseline -- ``oracle.block``;
* the inference fusions (``squared_relu_gate``, ``softcap_logits``,
  ``packed_causal_conv1d``) -- ``oracle.inference_ops``.

Every function cites the reference file:line it follows (paths relative to the
akbar2habibullah/atma repository root).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker / the timed CPU
baseline.  The product (``atma_amd``) never imports it and has no CPU fallback.

Pinning: each oracle function is pinned in ``tests/test_oracle_*.py`` by closed
forms, special cases that reduce to library routines (softmax attention,
triangular solves), invariants and brute-force sequential scans -- the reference
ships no golden tensors for this path.
"""

"""CPU restatement of the reference's per-layer attention hot path.

TEST INFRASTRUCTURE ONLY.  This package is the checker: it may be imported by
``tests/``, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of
``bench.py``, and by nothing else.  The product (the ``slo_attn`` host layer
and its HIP library) never imports, links or calls it.

Modules and the reference code each one restates:

* ``fp8``       -- E4M3FN codec (benchmarks/v0/probe_quant_support.py:24-56)
                   and the KV quantisation contract (docs/project_manual.md:527-537).
* ``kvstore``   -- slot-mapped KV write (nanovllm/layers/attention.py:10-40),
                   bf16 and quantised.
* ``attention`` -- dense causal bottom-right GQA attention in fp32
                   (benchmarks/v1_validation/reference.py:7-23), paged gather
                   (reference.py:60-62, benchmarks/v1_diagnostics/layer_replay.py:40-47),
                   varlen / decode oracles (reference.py:64-82) and the mixed
                   step's write-then-read ordering (nanovllm/layers/mixed_attention.py:29-57).
* ``metadata``  -- slot formula and per-row metadata (nanovllm/engine/batch_metadata.py:94-118,
                   mixed_model_runner.py:58-92, benchmarks/v1_diagnostics/layer_replay.py:32-37).

How each function is pinned (golden vectors, closed forms, brute force) is
listed in tests/test_oracle.py.
"""

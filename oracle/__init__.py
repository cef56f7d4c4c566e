"""CPU oracle for the continuous-batching attention path. TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithms of lean-vLLM's attention path so that the HIP kernels can
be checked against them. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import it, and only as the reference results to compare against or the timed CPU baseline -- never as the
product path. The product (``lean-vllm_amd/lvattn``) never imports anything from here.

Modules:
- ``pack``: ragged-batch packing (``lean_vllm/engine/model_runner.py:51-63,349-464``), a vectorised numpy
  restatement and a per-token loop restatement of the reference test oracle
  (``tests/test_model_runner.py:509-533``).
- ``store``: the paged-cache scatter (``lean_vllm/attention/torch_backend.py:34-60``).
- ``attention``: ``TorchAttention``'s gather/pad/mask/SDPA math in fp32 (``lean_vllm/attention/torch_backend.py``),
  the textbook dense oracle (``tests/test_attention_backends.py:93-116``), the log-sum-exp merge
  (``lean_vllm/attention/merge.py:8-15``) and absorbed MLA decode (``lean_vllm/layers/attention.py:319-335``).

Pinning (what checks each function beyond its own formula) is listed in each module's header and exercised by
``tests/test_oracle_*.py``. Every function here is pinned by at least one known answer, closed form, brute-force
loop or invariant; none is "parity unpinned".
"""

"""CPU oracle for the decode-step token sampler -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import anything under ``oracle/``, and only as the checker or the
timed CPU baseline.  The product path (``vllm_mps_amd``) never touches it.

* ``mis_oracle.c`` / ``oracle.py``: the contract restatement of
  ``model/sampler.py:18-60`` that the HIP kernels must match.
* ``faithful.py``: the literal reference algorithm re-stated with torch CPU
  ops (unstable sort, ``torch.multinomial``, one call per row), used as the
  CPU throughput baseline.
"""

"""CPU oracle for the sparse-MLA and flash-attention hot path.

TEST INFRASTRUCTURE ONLY. This package restates the reference's numerical
references on the CPU (NumPy / PyTorch-CPU FP32) so that the HIP kernels in
``ascendflow_amd`` can be checked against them. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and there only as the checker: the product path never calls it and
has no CPU fallback.

Modules:
- ``dtypes``            b16 storage codec (ties-to-even), restates
                        ``benchmarks/validation/dtypes.py:6-26``.
- ``sparse_reference``  TND/PA_BBND row selection, gather layout and FP32 sparse
                        MLA with per-head sinks, restates
                        ``benchmarks/attention/sparse_reference.py:15-181``.
- ``topk_reference``    top-k index selection over index scores under the
                        ``cmp_sparse_indices`` contract of
                        ``docs/operators/sparse-mla.md:41-51,79`` (the reference
                        has no indexer of its own).
- ``attention``         FA online-softmax oracle and the teaching-attention
                        reference, restates ``benchmarks/validation/attention.py:19-121``
                        and ``benchmarks/attention/run_simple.py:115-118``.
- ``cpu_reference``     vectorised FP32 PyTorch-CPU sparse MLA used as the timed
                        CPU baseline (restates ``sparse_reference.py:141-171``).

Every function is pinned by a known-answer or closed-form test under
``tests/test_oracle_*.py``; none is "parity unpinned".
"""

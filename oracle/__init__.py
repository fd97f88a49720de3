"""ORACLE: test infrastructure, not product code.

CPU restatements of the reference's paged-attention path, used only as the
checker by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py``.  Nothing in the product (the HIP library under
``flashengine.cpp_amd/``) imports, links or calls anything here.

Modules:
  aten_attention  torch-CPU restatement of the ATen reference attention
                  (src/portable_gpu_ops.cpp:18-44) plus natural-log LSE.
  rope_store      numpy restatement of rope / store / fused append, bit-exact
                  (src/cuda_kernels.cu:19-24, src/portable_gpu_ops.cpp:50-54).
  brute           float64 scalar-loop attention for tiny shapes; pins the
                  restatement independently of torch's kernels.
  step_metadata   restatement of CudaModel::prepare's metadata, graph_buckets
                  and the FIFO page allocator (src/cuda_model.cpp:131-142,
                  src/common.cpp:45-51, src/scheduler.cpp:5,31,35).
  norm_ops        numpy restatement of RMSNorm, the SiLU-gated product,
                  greedy acceptance and the fused q/k norm + rope + append
                  (src/cuda_kernels.cu:11-18,25, src/cuda_model.cpp:91-95).

Pinning (what each function is checked against) is listed in each module's
docstring and exercised by tests/test_oracle_*.py.
"""

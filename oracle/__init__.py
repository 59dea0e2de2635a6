"""CPU oracle for the Wayfinder causal top-K + sparse-attention path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product package (wayfinder-attention_amd/).

Two restatements live here:

* ``oracle.native``  -- ctypes binding of ``libwf_oracle.so`` (``wf_oracle.c``): the exact
  semantics the HIP kernels must reproduce bit-for-bit on indices (fp32 FMA-chain scores,
  lower-index tie rule, canonical slot order, reference pad indices) and within tolerance
  on outputs (double-accumulated softmax readout).
* ``oracle.torch_reference`` -- an op-by-op PyTorch-CPU restatement of the reference's own
  path (row-blocked bmm + mask + topk(sorted=False) + finalize; gather + softmax + sum),
  used as the CPU baseline and as an independent cross-check of index sets.
"""

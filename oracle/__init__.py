"""CPU oracle for the PECO per-layer attention hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/ and __graft_entry__.smoke(), which check the
GPU results against it, and by bench.py's cpu_baseline leg, which times it as the CPU
baseline. The product package (peco_amd) never imports it, and no GPU figure is measured on
it.

Two layers:
- ``oracle.canonical``: ctypes wrapper over ``peco_oracle.c``, the fixed-order
  fp32 restatement the HIP kernels must match bit for bit (k-means assign/update,
  stable sort, Base-Offset quantizer) plus a double-precision sparse attention.
- ``oracle.reference_path``: the reference's CPU torch path restated with the
  same torch operations (clustering.py CPU branches, selection, quantization,
  processor orchestration, block-sparse CPU attention). It is the CPU baseline
  that bench.py times, and the pin for the canonical layer.

Parity pins:
- tests/test_oracle.py: brute-force float64 argmin with near-tie certification;
  torch bmm/scatter_add_/argsort/elementwise ops as library routines; closed
  forms and special cases (constant residual, duplicate centroids, empty
  clusters, p=1, all-true map == SDPA, block-diagonal map == per-cluster SDPA,
  masked rows == 0); hand-written fixtures for the text partition.
- tests/test_oracle_layer.py: the end-to-end layer (reference_path.peco_layer)
  equals library SDPA with a separate padding segment when every pair is kept
  (with and without Base-Offset), and, for any selection, masked attention in
  original token order built from the labels and the cluster map alone.
- tests/test_processor_call.py: the processor prologue/epilogue restatement
  against identity projections and a quarter-turn rotation; the rotary
  embedding against complex multiplication.
Parity unpinned: the rotary embedding's agreement with diffusers' own
apply_rotary_emb (diffusers is not installed); only its published formula is
pinned.
"""

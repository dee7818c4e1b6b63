"""PECO per-layer attention hot path, MI355X-native (gfx950 HIP kernels behind a C-ABI).

Drop-in modules with the reference's names (Tom-HKUST/PECO ``peco`` package):
``processor`` (PecoConfig, InferenceContext, PecoAttention), ``clustering``,
``quantization``, ``clustering_cuda`` and ``attention_cuda``; ``model`` wires the
processor into a HunyuanVideo-style transformer.
"""

__version__ = "0.1.0"

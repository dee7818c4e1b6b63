"""The reference's import name for this package.

``from peco.processor import PecoConfig`` and ``from peco.model import install_attention,
reset_state`` (the calls of the reference's generate.py:63-64) resolve to the modules of
``peco_amd``: each ``peco.<name>`` below is the same module object as ``peco_amd.<name>``,
so state such as the loaded HIP library is shared between the two names.
"""
import importlib
import sys

_MODULES = ("processor", "clustering", "quantization", "clustering_cuda", "attention_cuda", "model")

for _name in _MODULES:
    _module = importlib.import_module(f"peco_amd.{_name}")
    sys.modules[f"{__name__}.{_name}"] = _module
    globals()[_name] = _module

del _name, _module

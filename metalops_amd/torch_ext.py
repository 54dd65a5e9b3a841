"""The PyTorch-ROCm extension binding (``_lib/torch_ext_build/mcq4_torch.so``).

It is the binding a metalcore maintainer registers in place of the Metal one:
``matmul_ggml_q4_0(X, W_blocks)`` with the signature, checks and stream
behaviour of ``matmul_ggml_q4_0_metal`` (native/core_mps.mm:5917-5975,
registered at :6938), calling ``mcq4_matmul_q4_0_f16`` of ``libmcq4.so``.
``__graft_entry__.build()`` compiles it with ``torch.utils.cpp_extension``; this
module only loads the built file (no compiler is needed at run time) and fails
loudly when it is missing.
"""
from __future__ import annotations

import importlib.machinery
import importlib.util
import os

from . import _lib  # loads libmcq4.so first: the extension links against its soname

EXT_NAME = "mcq4_torch"
EXT_PATH = os.path.join(os.path.dirname(_lib.LIB_PATH), "torch_ext_build", EXT_NAME + ".so")


def _load():
    if not os.path.exists(EXT_PATH):
        raise ImportError(f"metalops_amd: torch extension {EXT_PATH} is not built; "
                          "run `python -c 'import __graft_entry__ as g; g.build()'`")
    loader = importlib.machinery.ExtensionFileLoader(EXT_NAME, EXT_PATH)
    spec = importlib.util.spec_from_file_location(EXT_NAME, EXT_PATH, loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    return mod


backend = _load()
matmul_ggml_q4_0 = backend.matmul_ggml_q4_0

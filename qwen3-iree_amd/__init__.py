"""MI355X-native decode GEMV path of Qwen3-0.6B (gfx950).

Modules
  q8gemv   ctypes binding of libq8gemv (the C ABI in include/q8gemv.h): the six
           substituted decode dispatches plus a small device runtime.
  decode   the whole decode step (include/qwen3_decode.h): device weights,
           sessions with a KV cache, prompt ingestion, the generation loop, run.
  gguf     GGUF v2/v3 reader / writer and Qwen3-0.6B checkpoint ingestion into
           the device layout (no IREE).
  weights  Q8_0 quantisation / stacking (the reference's offline weight prep)
           and seeded synthetic inputs.
  build    hipcc / g++ recipe for lib/q8gemv_gfx950.hsaco, lib/decode_gfx950.hsaco
           and lib/libq8gemv.so.

The directory name is not a Python identifier; load it as a package with
load_package() below (or put this directory on sys.path and import the
modules directly).
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
PACKAGE_NAME = "qwen3_iree_amd"


def load_package():
    """Import this directory as the package `qwen3_iree_amd`."""
    if PACKAGE_NAME in sys.modules:
        return sys.modules[PACKAGE_NAME]
    spec = importlib.util.spec_from_file_location(
        PACKAGE_NAME, PACKAGE_DIR / "__init__.py", submodule_search_locations=[str(PACKAGE_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[PACKAGE_NAME] = mod
    spec.loader.exec_module(mod)
    return mod

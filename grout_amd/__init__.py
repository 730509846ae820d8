"""grout_amd -- MI355X-native (gfx950) attention hot path of grout.

Hand-written HIP kernels behind the C ABI in include/grout_attn.h
(grout_amd/libgrout_attn.so, built by `python -m grout_amd.build`).  This
package is the host-side mirror of the reference's attention operators:
``ops`` (one function per reference operator) and ``engine`` (KV caches,
StepGraph ops, decode-step HIP graph).
"""
from ._lib import GroutError, lib, LIB_PATH  # noqa: F401

__all__ = ["GroutError", "lib", "LIB_PATH", "ops", "engine"]


def __getattr__(name):
    if name in ("ops", "engine"):
        import importlib

        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(name)

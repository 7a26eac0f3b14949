"""rapidllm_amd -- MI355X (gfx950) decode backend for RapidLLM.

Hand-written HIP kernels behind a C ABI (include/rapidllm_hip.h), built in-tree
into rapidllm_amd/_lib/librapidllm_hip.so.  This package is the host-side mirror
of the reference's kernel/engine surface used by tests and bench.py.
"""
from . import hip  # noqa: F401

__all__ = ["hip"]

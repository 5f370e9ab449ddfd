"""MI355X-native (gfx950) decode hot path of threadcut.

Modules mirror the reference's: ``flash_decode`` (split-KV GQA decode),
``attention`` (the ``"threadcut"`` transformers attention), ``kv`` (RoPE
shift, suffix splice, GrowingLayer cache) and ``match`` (Split). The compute
runs in the HIP kernels of ``libthreadcut_hip.so`` (``threadcut_amd.build``).
"""
from .match import Split, lcp, split  # noqa: F401

__all__ = ["Split", "lcp", "split"]

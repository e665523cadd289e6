"""MI355X (gfx950) implementation of LeanSelect's prefill hot path.

Modules mirror the reference's call surface: ``selector`` (leanselect/selector.py),
``pages`` (leanselect/pages.py), ``ops`` (leanselect/ops) and ``infllm_v2`` (the
native-op names the model files import).  All computation runs in
``libleanselect_hip.so`` (built by ``leanselect_amd.build``).
"""
__version__ = "0.1.0"

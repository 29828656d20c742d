"""Exports of the reference outside the measured hot path that have no gfx950
implementation yet: the softmax comparison kernels and benchmark CLI
(reference kernels.py:534-562, 852-884, 1233-1325, 2832-3132).  They are importable so
that ``from smooth_attn import *`` keeps working, and raise when called."""
from __future__ import annotations


def _missing(name):
    def fn(*args, **kwargs):
        raise NotImplementedError(f"smooth_attn.{name} has no gfx950 implementation yet")

    fn.__name__ = name
    return fn


softmax_triton = _missing("softmax_triton")
softmax_triton_out = _missing("softmax_triton_out")
softmax_causal_triton = _missing("softmax_causal_triton")
softmax_causal_triton_out = _missing("softmax_causal_triton_out")
benchmark_rowwise_suite = _missing("benchmark_rowwise_suite")
benchmark_causal_suite = _missing("benchmark_causal_suite")
main = _missing("main")

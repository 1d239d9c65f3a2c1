"""nsosx: the MI355X (gfx950) hybrid-layer hot path of vitorGgC569/reimagined.

BitLinear ternary GEMV/GEMM, the packed ragged Mamba selective scan and top-k
MoE routing, as hand-written HIP kernels behind the C ABI of include/nsosx.h
(built into reimagined_amd/libnsosx.so by `python -m reimagined_amd.build`).
"""
from ._lib import LIB_PATH, NsosxError, header_symbols, lib  # noqa: F401

__all__ = ["LIB_PATH", "NsosxError", "header_symbols", "lib"]

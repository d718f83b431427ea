"""velox_amd — MI355X (gfx950) speculative-decoding verify path.

A from-scratch HIP implementation of the verify path of the reference's Metal
backend: int4 g64 GEMM at the k+1 verify rows, tree-masked paged attention,
fused acceptance (greedy / stochastic / tree), and the C++ spec-decode engine
around them.  `velox_amd.ops` mirrors the reference's operator API,
`velox_amd.engine` its PagedKvCache / PagedQwen3 / SpecEngine.
"""
from ._lib import BF16, F16, F32, VeloxError, lib  # noqa: F401

__version__ = lib.vx_version().decode()

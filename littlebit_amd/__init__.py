"""MI355X-native LittleBitLinear forward (HIP kernels for gfx950 behind a C ABI).

Public surface:
  * :class:`LittleBitLinear` -- drop-in for quantization/modules/littlebit.py
  * :func:`littlebit_linear` -- GPU form of the reference operator
    ``littlebit_cpu_ops::littlebit_linear``
  * :class:`LittleBitProjection` / :class:`LittleBitBranch` -- prepared fused
    forward of a projection's draft and residual branches
  * :class:`LittleBitProjectionGroup` -- projections sharing one input
    (q/k/v, gate/up) in the launches of one
  * :class:`LittleBitChain` -- calls reading each other's outputs at one row
    (o, gate/up, down, next q/k/v) in one launch per link boundary
  * :func:`binary_packer` / :func:`binary_unpacker` -- the reference word format
  * :func:`repack_signs_to_i2` -- the reference CPU runtime's 2-bit sign rows
  * :func:`set_deterministic` / :func:`deterministic` -- bit-for-bit repeatable
    decode-path calls (fixed-order split-K sums)
"""
from .binary_packer import binary_packer, binary_unpacker, repack_signs_to_i2, words_per_row
from .ops import (ChainLink, LittleBitBranch, LittleBitChain, LittleBitProjection, LittleBitProjectionGroup,
                  deterministic, littlebit_forward, littlebit_linear, set_deterministic)
from .modules import LittleBitLinear, sign_pm1

__all__ = [
    "LittleBitLinear",
    "LittleBitBranch",
    "LittleBitProjection",
    "LittleBitProjectionGroup",
    "LittleBitChain",
    "ChainLink",
    "littlebit_forward",
    "littlebit_linear",
    "binary_packer",
    "binary_unpacker",
    "repack_signs_to_i2",
    "words_per_row",
    "sign_pm1",
    "set_deterministic",
    "deterministic",
]

__version__ = "0.1.0"

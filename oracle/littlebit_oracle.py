"""CPU oracle for the LittleBitLinear forward and its sign packing.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``littlebit_amd``) may
import, call or link this module: only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg use it, and only as the checker.

It restates, in numpy (float64 for the arithmetic, exact integers for the
bits), the reference's algorithm for the hot path:

* ``sign_pm1``       -- quantization/functions/binary.py:6-10 (sign, 0 -> +1)
* ``pack_signs``     -- quantization/utils/binary_packer.py:5-51
* ``unpack_signs``   -- quantization/utils/binary_packer.py:54-97
* ``fuse_mid``       -- convert_hf_to_runtime.py:54-57 (mid = v1 * u2 in fp32)
* ``branch_forward`` -- quantization/modules/littlebit.py:114-121
* ``littlebit_forward`` -- quantization/modules/littlebit.py:95-112
  (main branch + optional residual branch + optional bias; the branches may
  have different ranks, which the reference module does not allow but its
  runtime layout does: convert_hf_to_runtime.py:66-84)
* ``rms_norm``, ``silu_mul`` -- the inputs the reference's CPU decode step
  feeds its projections: rms_norm_inline and silu_mul_inline,
  patches/littlebit_cpu_optimized.cpp:1370-1405 and 1410-1438

Every function here is pinned in ``tests/test_oracle.py`` by hand-derived
golden words, textbook special cases, a brute-force dense evaluation built
with independent bit arithmetic, torch float64, and algebraic invariants.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "sign_pm1",
    "pack_signs",
    "rms_norm",
    "silu_mul",
    "unpack_signs",
    "words_per_row",
    "fuse_mid",
    "branch_forward",
    "littlebit_forward",
    "rel_err",
]


def words_per_row(cols: int) -> int:
    """Number of 32-bit words holding ``cols`` signs (binary_packer.py:32)."""
    return (int(cols) + 31) // 32


def sign_pm1(a: np.ndarray) -> np.ndarray:
    """Sign with sign(0) = +1, as int8 in {-1, +1}.

    Follows quantization/functions/binary.py:6-10 (``x.sign()`` then
    ``y[y == 0] = 1``); the same rule is applied at pack time
    (quantization/modules/littlebit.py:316).
    """
    s = np.sign(np.asarray(a, dtype=np.float64))
    s[s == 0] = 1
    return s.astype(np.int8)


def pack_signs(signs: np.ndarray) -> np.ndarray:
    """Pack a {-1,+1} int8 matrix into int32 words, LSB first.

    Follows quantization/utils/binary_packer.py:5-51:
      * column ``32*w + j`` of a row goes to bit ``j`` of word ``w``;
      * bit = 1 encodes -1, bit = 0 encodes +1 (``(1 - s) // 2``, :43);
      * rows are padded to a multiple of 32 with +1, i.e. bit 0 (:36-39);
      * the word is the int32 sum of ``bit * 2**j``; 2**31 wraps to the sign
        bit, so the result is the two's-complement view of the bit pattern
        (:47-50).
    Raises TypeError for non-int8 input (:27-28).
    """
    signs = np.asarray(signs)
    if signs.dtype != np.int8:
        raise TypeError("Input tensor must be int8.")
    if signs.ndim != 2:
        raise ValueError("expected a 2-D matrix")
    rows, cols = signs.shape
    wpr = words_per_row(cols)
    padded = np.ones((rows, wpr * 32), dtype=np.int8)
    padded[:, :cols] = signs
    bits = ((1 - padded.astype(np.int64)) // 2).astype(np.uint64)
    bits = bits.reshape(rows, wpr, 32)
    weights = np.uint64(1) << np.arange(32, dtype=np.uint64)
    words = (bits * weights).sum(axis=2, dtype=np.uint64).astype(np.uint32)
    return words.view(np.int32).reshape(rows, wpr).copy()


def unpack_signs(packed: np.ndarray, shape) -> np.ndarray:
    """Inverse of :func:`pack_signs`, trimmed to ``shape[1]`` columns.

    Follows quantization/utils/binary_packer.py:54-97: bit ``j`` of word ``w``
    is column ``32*w + j``; bit 1 -> -1, bit 0 -> +1.  A packed tensor that is
    not 2-D with shape ``(rows, ceil(cols/32))`` raises ValueError (:96-97).
    """
    packed = np.asarray(packed)
    rows, cols = int(shape[0]), int(shape[1])
    wpr = words_per_row(cols)
    if packed.ndim != 2 or packed.shape != (rows, wpr):
        raise ValueError(
            "Unsupported packed tensor format. Expected 2D tensor with shape "
            f"(n_rows, words_per_row), got {packed.shape} with {packed.ndim} dimensions.")
    words = packed.astype(np.int64) & 0xFFFFFFFF
    shifts = np.arange(32, dtype=np.int64)
    bits = (words[:, :, None] >> shifts[None, None, :]) & 1
    bits = bits.reshape(rows, wpr * 32)[:, :cols]
    return (1 - 2 * bits).astype(np.int8)


def fuse_mid(v1: np.ndarray, u2: np.ndarray) -> np.ndarray:
    """Latent scale ``mid = v1.float() * u2.float()`` (convert_hf_to_runtime.py:54-57)."""
    return (np.asarray(v1, dtype=np.float32) * np.asarray(u2, dtype=np.float32)).astype(np.float32)


def branch_forward(x, v_packed, u_packed, g, l, h, K: int, R: int, N: int) -> np.ndarray:
    """One LittleBit branch in float64.

    quantization/modules/littlebit.py:114-121 computes
    ``((((x * v2) @ Vq.t()) * (v1 * u2)) @ Uq.t()) * u1`` with
    Vq = sign(V) [R, K], Uq = sign(U) [N, R]; here ``g = v2`` [K],
    ``l = v1*u2`` [R] and ``h = u1`` [N].  Vq and Uq come from the packed words.
    """
    x = np.asarray(x, dtype=np.float64).reshape(-1, K)
    V = unpack_signs(v_packed, (R, K)).astype(np.float64)
    U = unpack_signs(u_packed, (N, R)).astype(np.float64)
    g = np.asarray(g, dtype=np.float64).reshape(1, K)
    l = np.asarray(l, dtype=np.float64).reshape(1, R)
    h = np.asarray(h, dtype=np.float64).reshape(1, N)
    t = ((x * g) @ V.T) * l
    return (t @ U.T) * h


def littlebit_forward(x, branches, K: int, N: int, bias=None) -> np.ndarray:
    """Sum of the branches (main, then residual) plus bias.

    quantization/modules/littlebit.py:95-112: flatten the leading dims, main
    branch, ``y = y + res`` for the residual branch, ``y += bias``, reshape.
    ``branches`` is a sequence of dicts with keys v_sign, u_sign, g, l, h, R.
    """
    x = np.asarray(x, dtype=np.float64)
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    y = np.zeros((x2.shape[0], N), dtype=np.float64)
    for b in branches:
        y = y + branch_forward(x2, b["v_sign"], b["u_sign"], b["g"], b["l"], b["h"], K, int(b["R"]), N)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64).reshape(1, N)
    return y.reshape(*lead, N)


def rms_norm(x, w, eps: float) -> np.ndarray:
    """x / sqrt(mean(x^2) + eps) * w over the last axis (patch:1370-1405)."""
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * np.asarray(w, dtype=np.float64)


def silu_mul(gate, up) -> np.ndarray:
    """gate * sigmoid(gate) * up (patch:1410-1438)."""
    g = np.asarray(gate, dtype=np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(up, dtype=np.float64)


def rel_err(y, y_ref) -> float:
    """Parity metric: max|y - y_ref| / max|y_ref| (0 for empty outputs)."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    if y_ref.size == 0:
        return 0.0
    denom = float(np.max(np.abs(y_ref)))
    num = float(np.max(np.abs(y - y_ref)))
    if denom == 0.0:
        return num
    return num / denom

"""CPU oracle for the reference's 2-bit ("i2") sign layout.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``littlebit_amd``) may
import, call or link this module: only ``tests/`` use it, as the checker.

``repack_signs_to_i2`` restates repack_signs_to_i2_cpu,
patches/littlebit_cpu_optimized.cpp:712-764 (registered as
``littlebit_cpu_ops::repack_signs_to_i2`` at :2340, called at load time by
cpu_draft_model.py:247-250), in exact integer numpy:

* a row of ``n_cols`` signs (int32 words, bit ``c % 32`` of word ``c // 32``,
  bit 1 = -1; binary_packer.py:36-50) becomes ``ceil(n_cols / 4)`` bytes;
* each sign becomes a 2-bit value, 2 for +1 and 0 for -1 (:735-736);
* column ``c = 128 b + 32 g + p`` lands in byte ``32 b + p`` at bit shift
  ``6 - 2 g`` (:738-755);
* a column whose byte index is ``>= ceil(n_cols / 4)`` is dropped (:753), which
  happens in the last, partial block of 128 columns whenever
  ``n_cols % 128 != 0``; fields that no kept column fills stay 0 (the output
  starts as zeros, :724).

``i2_kept_columns`` names the columns the layout keeps, and ``decode_i2``
reads a layout back; the tests use both to pin the restatement by
invariants, beside hand-built bytes and the reference's own op.
"""
from __future__ import annotations

import numpy as np

__all__ = ["i2_bytes_per_row", "repack_signs_to_i2", "i2_kept_columns", "decode_i2"]


def i2_bytes_per_row(n_cols: int) -> int:
    """Bytes of an i2 row: ceil(n_cols / 4) (patch:722)."""
    return (int(n_cols) + 3) // 4


def _sign_bits(words: np.ndarray, n_cols: int) -> np.ndarray:
    """bits[r, c] = bit (c % 32) of word (c // 32) of row r, c < n_cols."""
    w = np.asarray(words).astype(np.int64) & 0xFFFFFFFF
    c = np.arange(n_cols)
    return ((w[:, c // 32] >> (c % 32)) & 1).astype(np.uint8)


def _byte_and_shift(n_cols: int):
    c = np.arange(n_cols)
    return 32 * (c // 128) + c % 32, 6 - 2 * ((c % 128) // 32)


def repack_signs_to_i2(words: np.ndarray, n_cols: int) -> np.ndarray:
    """uint8 [rows, ceil(n_cols/4)] exactly as repack_signs_to_i2_cpu writes it.

    ``words`` is int32 (or uint32) [rows, >= ceil(n_cols/32)]; the reference
    reads word ``c // 32`` of each row for every ``c < n_cols`` (:733-734).
    """
    words = np.asarray(words)
    if words.ndim != 2:
        raise ValueError("expected a 2-D matrix of words")
    n_cols = int(n_cols)
    rows = words.shape[0]
    nb = i2_bytes_per_row(n_cols)
    out = np.zeros((rows, nb), dtype=np.uint8)
    if rows == 0 or n_cols == 0:
        return out
    if words.shape[1] * 32 < n_cols:
        raise ValueError("fewer sign words than columns")
    val = (2 * (1 - _sign_bits(words, n_cols))).astype(np.uint8)   # +1 -> 2, -1 -> 0
    byte, shift = _byte_and_shift(n_cols)
    keep = byte < nb
    # within one shift (one group g) every kept column has its own byte
    for s in (6, 4, 2, 0):
        cols = np.nonzero(keep & (shift == s))[0]
        out[:, byte[cols]] |= (val[:, cols] << s).astype(np.uint8)
    return out


def i2_kept_columns(n_cols: int) -> np.ndarray:
    """Boolean [n_cols]: the columns whose 2-bit field the layout holds."""
    byte, _ = _byte_and_shift(int(n_cols))
    return byte < i2_bytes_per_row(n_cols)


def decode_i2(i2: np.ndarray, n_cols: int) -> np.ndarray:
    """int8 [rows, n_cols]: the field of each column read back (2 -> +1,
    0 -> -1); columns the layout dropped read 0."""
    i2 = np.asarray(i2, dtype=np.uint8)
    n_cols = int(n_cols)
    byte, shift = _byte_and_shift(n_cols)
    keep = byte < i2_bytes_per_row(n_cols)
    out = np.zeros((i2.shape[0], n_cols), dtype=np.int8)
    if n_cols == 0:
        return out
    fields = (i2[:, np.minimum(byte, max(i2.shape[1] - 1, 0))] >> shift) & 3
    out[:, keep] = (fields[:, keep].astype(np.int8) - 1)
    return out

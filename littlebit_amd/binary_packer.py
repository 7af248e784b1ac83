"""Sign packing with the reference's word format.

Mirrors quantization/utils/binary_packer.py (``binary_packer`` :5-51,
``binary_unpacker`` :54-97): column ``32*w + j`` of a row is bit ``j`` of
word ``w``; bit 1 means -1, bit 0 means +1; rows are padded with +1 (bit 0);
words are int32 (bit 31 is the sign bit).

Tensors on a GPU are packed and unpacked by the HIP kernels of the library;
CPU tensors (checkpoint load and save) by torch bit operations.

``repack_signs_to_i2`` writes the 2-bit layout of the reference's CPU runtime
(``littlebit_cpu_ops::repack_signs_to_i2``, patches/littlebit_cpu_optimized.cpp:
712-764) from the words, on the GPU.
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import _lib

__all__ = ["binary_packer", "binary_unpacker", "repack_signs_to_i2", "words_per_row"]


def words_per_row(cols: int) -> int:
    return (int(cols) + 31) // 32


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def binary_packer(tensor: torch.Tensor) -> torch.Tensor:
    """Pack an int8 {-1,+1} matrix [rows, cols] to int32 words [rows, ceil(cols/32)].

    Raises TypeError for a non-int8 input, like the reference (:27-28).
    Negative entries become bit 1 and all others bit 0, which equals the
    reference's ``(1 - t) // 2`` on {-1, +1}.
    """
    if tensor.dtype != torch.int8:
        raise TypeError("Input tensor must be int8.")
    if tensor.dim() != 2:
        raise ValueError(f"expected a 2-D tensor, got {tensor.dim()} dimensions")
    rows, cols = tensor.shape
    wpr = words_per_row(cols)
    if tensor.is_cuda:
        src = tensor.contiguous()
        out = torch.empty((rows, wpr), dtype=torch.int32, device=tensor.device)
        if rows and cols:
            lib = _lib.load()
            with torch.cuda.device(tensor.device):
                rc = lib.lbk_pack_signs(src.data_ptr(), rows, cols, out.data_ptr(),
                                        _stream_handle(tensor.device))
            _lib.check(rc, "binary_packer")
        return out
    pad = wpr * 32 - cols
    bits = (tensor < 0).to(torch.int64)
    if pad:
        bits = torch.cat([bits, torch.zeros((rows, pad), dtype=torch.int64)], dim=1)
    bits = bits.reshape(rows, wpr, 32)
    words = (bits << torch.arange(32, dtype=torch.int64)).sum(dim=2)
    words = torch.where(words >= 2**31, words - 2**32, words)
    return words.to(torch.int32).contiguous()


def binary_unpacker(packed_tensor: torch.Tensor, original_shape: Tuple[int, int]) -> torch.Tensor:
    """Unpack int32 words to an int8 {-1,+1} matrix of ``original_shape``.

    Raises ValueError when ``packed_tensor`` is not 2-D of shape
    (rows, ceil(cols/32)), like the reference (:96-97).
    """
    n_rows, n_cols = int(original_shape[0]), int(original_shape[1])
    wpr = words_per_row(n_cols)
    if packed_tensor.dim() != 2 or tuple(packed_tensor.shape) != (n_rows, wpr):
        raise ValueError(
            "Unsupported packed tensor format. Expected 2D tensor with shape "
            f"(n_rows, words_per_row), got {tuple(packed_tensor.shape)} with "
            f"{packed_tensor.dim()} dimensions.")
    if packed_tensor.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"packed words must be int32, got {packed_tensor.dtype}")
    if packed_tensor.is_cuda:
        src = packed_tensor.contiguous()
        out = torch.empty((n_rows, n_cols), dtype=torch.int8, device=packed_tensor.device)
        if n_rows and n_cols:
            lib = _lib.load()
            with torch.cuda.device(packed_tensor.device):
                rc = lib.lbk_unpack_signs(src.data_ptr(), n_rows, n_cols, out.data_ptr(),
                                          _stream_handle(packed_tensor.device))
            _lib.check(rc, "binary_unpacker")
        return out
    words = packed_tensor.to(torch.int64) & 0xFFFFFFFF
    bits = (words.unsqueeze(-1) >> torch.arange(32, dtype=torch.int64)) & 1
    bits = bits.reshape(n_rows, wpr * 32)[:, :n_cols]
    return (1 - 2 * bits).to(torch.int8)


def repack_signs_to_i2(packed_signs: torch.Tensor, n_cols: int) -> torch.Tensor:
    """Sign words [rows, words] -> uint8 [rows, ceil(n_cols/4)] in the
    reference runtime's 2-bit layout, byte for byte as
    ``littlebit_cpu_ops::repack_signs_to_i2`` (patch:712-764) writes it:
    column ``128 b + 32 g + p`` is the field at bit shift ``6 - 2 g`` of byte
    ``32 b + p``, 2 for +1 and 0 for -1; columns whose byte index reaches
    ``ceil(n_cols/4)`` are dropped as the reference drops them.

    The same checks as the reference (int32 words, :718) plus: the tensor is
    on a GPU, 2-D, and holds at least ``ceil(n_cols/32)`` words per row.
    """
    if not isinstance(packed_signs, torch.Tensor) or not packed_signs.is_cuda:
        raise RuntimeError("packed_signs must be a CUDA (HIP) tensor")
    if packed_signs.dtype != torch.int32:
        raise RuntimeError("packed_signs must be int32")
    if packed_signs.dim() != 2:
        raise RuntimeError(f"packed_signs must be 2-D, got {packed_signs.dim()} dimensions")
    n_cols = int(n_cols)
    if n_cols < 0:
        raise RuntimeError(f"n_cols must be >= 0, got {n_cols}")
    src = packed_signs.contiguous()
    rows, wpr = src.shape
    out = torch.empty((rows, (n_cols + 3) // 4), dtype=torch.uint8, device=src.device)
    lib = _lib.load()
    with torch.cuda.device(src.device):
        rc = lib.lbk_repack_signs_to_i2(src.data_ptr(), rows, wpr, n_cols, out.data_ptr(),
                                        _stream_handle(src.device))
    _lib.check(rc, "repack_signs_to_i2")
    return out

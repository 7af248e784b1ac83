"""CPU oracle for the draft step's Q4_0 lm_head and argmax.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``littlebit_amd``) may
import, call or link this module: only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg use it, and only as the checker.

It restates, in numpy, the reference's ``generate_token`` tail
(patches/littlebit_cpu_optimized.cpp:2254-2317): the lm_head weight is
quantised to Q4_0 (:2129-2149, ``quantize_lm_head_q4`` :2225-2251), the
final hidden state to Q8_0 (:2152-2165), each logit is the Q4_0 x Q8_0 block
dot product (:2168-2222, scalar form :2208-2219) and the token is the first
index of the largest logit (:2305-2314).

* ``fp16_bits``       -- fp32_to_fp16 (:2119-2127): truncating, subnormals
  flushed to zero, overflow to infinity (not IEEE rounding)
* ``fp16_value``      -- fp16_to_fp32 (:2101-2117): the exact IEEE half value
* ``quantize_q4_0``   -- quantize_row_fp32_to_q4_0, as (nibbles, scale bits)
* ``q4_0_reference_bytes`` -- the same as the reference's 18-byte blocks
* ``quantize_q8_0``   -- quantize_row_fp32_to_q8_0
* ``q4_q8_logits``    -- vec_dot_q4_0_q8_0 for every row (float64 sums of the
  exact per-block integer dots times the fp32 scale products)
* ``generate_token_head`` -- Q8_0 of the hidden state, logits, first argmax

Pinned in ``tests/test_oracle_q4.py``: hand-derived fp16 bit patterns
(including the cases where truncation and IEEE rounding differ), the
reference's own ``quantize_lm_head_q4`` bytes and ``generate_token`` tokens
(oracle/_ref, when built), and brute-force dequantised dot products.
"""
from __future__ import annotations

import numpy as np

__all__ = ["fp16_bits", "fp16_value", "quantize_q4_0", "q4_0_reference_bytes", "quantize_q8_0", "q4_q8_logits",
           "generate_token_head"]

QK = 32  # values per Q4_0 / Q8_0 block


def fp16_bits(x) -> np.ndarray:
    """fp32 -> fp16 bits by exponent rebias and mantissa truncation
    (patch:2119-2127): exponents below the fp16 range give a signed zero,
    above it a signed infinity."""
    v = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.int64)
    sign = (v >> 16) & 0x8000
    expo = ((v >> 23) & 0xFF) - 127 + 15
    mant = (v >> 13) & 0x3FF
    out = np.where(expo <= 0, sign, np.where(expo >= 31, sign | 0x7C00, sign | (np.clip(expo, 0, 31) << 10) | mant))
    return out.astype(np.uint16)


def fp16_value(bits) -> np.ndarray:
    """The float32 value of fp16 bits (exact; patch:2101-2117)."""
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def quantize_q4_0(w):
    """w [rows, cols] fp32, cols % 32 == 0 -> (qs uint8 [rows, cols/32, 16],
    d uint16 [rows, cols/32]).  Per block of 32: m = the first value of
    largest magnitude, d = m / -8, q = min(15, int(x / d + 8.5)) in fp32
    (x * (1/d), then + 8.5, each rounded); byte j holds q[j] in its low
    nibble and q[j + 16] in its high nibble (patch:2129-2149)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    assert cols % QK == 0
    blk = w.reshape(rows, cols // QK, QK)
    first = np.argmax(np.abs(blk), axis=-1)  # first index of the maximum
    m = np.take_along_axis(blk, first[..., None], axis=-1)[..., 0]
    d = (m / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0))
    inv = inv.astype(np.float32)
    t = (blk * inv[..., None]).astype(np.float32)
    t = (t + np.float32(8.5)).astype(np.float32)
    q = np.minimum(15, np.trunc(t).astype(np.int64)).astype(np.uint8)
    qs = (q[..., :QK // 2] | (q[..., QK // 2:] << 4)).astype(np.uint8)
    return qs, fp16_bits(d)


def q4_0_reference_bytes(qs, d) -> np.ndarray:
    """The reference's packed lm_head: per row, per block, the fp16 scale
    (2 bytes, little-endian) then the 16 nibble bytes (patch:2085-2090)."""
    rows, nb, _ = qs.shape
    out = np.empty((rows, nb, 18), np.uint8)
    out[..., 0] = (d & 0xFF).astype(np.uint8)
    out[..., 1] = (d >> 8).astype(np.uint8)
    out[..., 2:] = qs
    return out.reshape(-1)


def quantize_q8_0(x):
    """x [cols] fp32 -> (qs int8 [cols/32, 32], d uint16 [cols/32]):
    d = amax / 127 in fp32, q = round-half-away(x * (1/d)) (patch:2152-2165;
    the fp16 scale is stored, the fp32 1/d is what rounds)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, QK)
    amax = np.abs(x).max(axis=-1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0))
    v = (x * inv.astype(np.float32)[:, None]).astype(np.float32).astype(np.float64)
    q = np.where(v >= 0, np.floor(v + 0.5), np.ceil(v - 0.5)).astype(np.int8)
    return q, fp16_bits(d)


def q4_q8_logits(qs4, d4, q8, d8) -> np.ndarray:
    """Every row's sum over blocks of (fp16(d4) * fp16(d8) in fp32) times
    the exact integer sum_j (nibble_j - 8) * q8_j, in float64."""
    lo = (qs4 & 0x0F).astype(np.int64) - 8
    hi = (qs4 >> 4).astype(np.int64) - 8
    q8 = q8.astype(np.int64)
    sumi = (lo * q8[None, :, :QK // 2]).sum(-1) + (hi * q8[None, :, QK // 2:]).sum(-1)  # [rows, nb]
    scale = (fp16_value(d4) * fp16_value(d8)[None, :]).astype(np.float32)
    return (scale.astype(np.float64) * sumi).sum(-1)


def generate_token_head(hidden, qs4, d4):
    """(logits [rows] float64, token) for a final hidden state [cols]:
    Q8_0 of the hidden, the Q4_0 x Q8_0 logits, the first largest."""
    q8, d8 = quantize_q8_0(hidden)
    logits = q4_q8_logits(qs4, d4, q8, d8)
    return logits, int(np.argmax(logits))

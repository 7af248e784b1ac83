"""Pins of the Q4_0 lm_head oracle (oracle/lm_head_q4_oracle.py).

* fp16 bit patterns derived by hand, including the cases where the
  reference's truncating conversion differs from IEEE rounding;
* the reference's own ``quantize_lm_head_q4`` bytes and ``generate_token``
  tokens (oracle/_ref, built from the reference's C++; skipped without it);
* the logits against a brute-force dequantised dot product, and the block
  layout against a hand-built block.
"""
import numpy as np
import pytest
import torch

from oracle import build_ref
from oracle import lm_head_q4_oracle as Q

needs_ref = pytest.mark.skipif(not build_ref.OUT.exists(), reason="oracle/_ref not built")


def test_fp16_bits_hand_vectors():
    cases = [
        (1.0, 0x3C00), (-2.0, 0xC000), (0.5, 0x3800), (65504.0, 0x7BFF),
        (65536.0, 0x7C00),              # exponent 16 + 15 = 31: infinity
        (-1e6, 0xFC00),
        (1.0 + 2 ** -10 + 2 ** -11, 0x3C01),  # IEEE rounding (half, to even) gives 0x3C02
        (1.0 + 2 ** -10 + 2 ** -11 + 2 ** -12, 0x3C01),  # above half: IEEE gives 0x3C02
        (2.0 ** -14, 0x0400),           # smallest normal
        (2.0 ** -15, 0x0000),           # an IEEE subnormal, flushed to zero here
        (-(2.0 ** -20), 0x8000),
        (0.0, 0x0000), (-0.0, 0x8000),
        (1.0 / 3.0, 0x3555),
    ]
    x = np.array([c[0] for c in cases], np.float32)
    assert Q.fp16_bits(x).tolist() == [c[1] for c in cases]
    # the value side is exact IEEE half
    assert Q.fp16_value(np.array([0x3C01, 0x0400, 0xC000], np.uint16)).tolist() == [1.0 + 2 ** -10, 2 ** -14, -2.0]


def test_q4_block_layout_by_hand():
    """One block: m = -16 (first largest magnitude, before +16), d = 2,
    q = min(15, int(x / 2 + 8.5)); byte j = q[j] | q[j + 16] << 4."""
    x = np.zeros(32, np.float32)
    x[3], x[20] = -16.0, 16.0   # equal magnitude: the first (x[3]) sets d = -16 / -8 = 2
    x[0], x[16] = 3.0, -3.0     # 3/2 + 8.5 = 10 -> 10;  -1.5 + 8.5 = 7 -> 7
    x[1] = 2.999                # 1.4995 + 8.5 = 9.9995 -> 9 (truncation)
    qs, d = Q.quantize_q4_0(x[None])
    assert d.tolist() == [[0x4000]]  # 2.0
    q = np.full(32, 8)
    q[3], q[20], q[0], q[16], q[1] = 0, 15, 10, 7, 9  # -16/2+8.5 = 0.5 -> 0; 16/2 + 8.5 = 16.5 -> 15
    assert qs[0, 0].tolist() == [int(q[j] | (q[j + 16] << 4)) for j in range(16)]
    b = Q.q4_0_reference_bytes(qs, d)
    assert b[:2].tolist() == [0x00, 0x40] and b.size == 18


def test_zero_block_and_q8_rounding():
    qs, d = Q.quantize_q4_0(np.zeros((1, 32), np.float32))
    assert d.tolist() == [[0x8000]] and (qs == 0x88).all()  # d = 0 / -8 = -0; nibble 8 = value 0
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2], x[3] = 127.0, 0.5, -0.5, -1.5  # d = 1: half away from zero
    q8, d8 = Q.quantize_q8_0(x)
    assert d8.tolist() == [0x3C00]
    assert q8[0, :4].tolist() == [127, 1, -1, -2]


def test_logits_match_dequantised_brute_force():
    rng = np.random.Generator(np.random.PCG64(5))
    w = rng.standard_normal((37, 96)).astype(np.float32)
    h = rng.standard_normal(96).astype(np.float32)
    qs, d = Q.quantize_q4_0(w)
    q8, d8 = Q.quantize_q8_0(h)
    lo = (qs & 15).astype(np.float64) - 8
    hi = (qs >> 4).astype(np.float64) - 8
    wq = np.concatenate([lo, hi], axis=-1) * Q.fp16_value(d).astype(np.float64)[..., None]  # [37, 3, 32]
    hq = q8.astype(np.float64) * Q.fp16_value(d8).astype(np.float64)[:, None]
    brute = (wq * hq[None]).sum((1, 2))
    got = Q.q4_q8_logits(qs, d, q8, d8)
    assert np.allclose(got, brute, rtol=1e-6, atol=1e-6)
    # and both approximate the dense product
    assert np.abs(brute - w @ h).max() < 0.15 * np.abs(w @ h).max()


@needs_ref
@pytest.mark.parametrize("rows,cols,seed", [(64, 256, 1), (33, 4096, 2), (7, 32, 3)])
def test_q4_quantizer_bytes_equal_reference(rows, cols, seed):
    ops = build_ref.load()
    rng = np.random.Generator(np.random.PCG64(seed))
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    w[0, :32] = 0.0                        # all-zero block
    w[1, 5], w[1, 9] = 0.5, -0.5           # a magnitude tie
    w[2, 0] = 7e4                          # scale overflows fp16: infinity
    w[3, :32] = 1e-9                       # scale below fp16: zero
    ref = ops.quantize_lm_head_q4(torch.from_numpy(w)).numpy()
    qs, d = Q.quantize_q4_0(w)
    assert np.array_equal(Q.q4_0_reference_bytes(qs, d), ref)


@needs_ref
def test_generate_token_tail_equals_reference():
    """generate_token with no layers: embedding row -> final RMSNorm ->
    Q4_0 lm_head -> argmax.  The oracle, given the reference's own normed
    hidden (full_forward with no layers), picks the same token."""
    ops = build_ref.load()
    rng = np.random.Generator(np.random.PCG64(11))
    vocab, hidden = 500, 256
    emb = rng.standard_normal((vocab, hidden)).astype(np.float32)
    norm = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    head = (rng.standard_normal((vocab, hidden)) * 0.05).astype(np.float32)
    t = torch.from_numpy
    q4 = ops.quantize_lm_head_q4(t(head))
    qs, d = Q.quantize_q4_0(head)
    for tok in range(0, vocab, 17):
        args = (t(emb), t(norm), [], [], [])
        h = ops.full_forward(tok, *args, 0, hidden, 1, 1, 32, 16, 0, 1.0, 1e-6).numpy().reshape(-1)
        want = ops.generate_token(tok, *args, q4, vocab, 0, hidden, 1, 1, 32, 16, 0, 1.0, 1e-6)
        _, got = Q.generate_token_head(h, qs, d)
        assert got == want, tok

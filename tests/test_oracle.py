"""Pins of the CPU oracle (oracle/littlebit_oracle.py).

Each oracle function is checked against something that does not share its
code: hand-built golden words, a brute-force evaluation with Python integers
and math.fsum, closed forms, torch float64, and algebraic invariants chosen
so that a dropped scale, a swapped factor, a wrong bit order or a wrong sign
convention fails at least one of them.
"""
import json

import numpy as np
import pytest
import torch

from oracle import littlebit_oracle as O
from tests.conftest import GOLDEN


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def _rand_branch(rng, K, R, N):
    V = (1 - 2 * rng.integers(0, 2, size=(R, K))).astype(np.int8)
    U = (1 - 2 * rng.integers(0, 2, size=(N, R))).astype(np.int8)
    return {
        "V": V, "U": U,
        "v_sign": O.pack_signs(V), "u_sign": O.pack_signs(U),
        "g": np.abs(rng.standard_normal(K)) + 0.05,
        "l": np.abs(rng.standard_normal(R)) + 0.05,
        "h": np.abs(rng.standard_normal(N)) + 0.05,
        "R": R,
    }


# --------------------------------------------------------------------------- packing
PACK_CASES = json.loads((GOLDEN / "pack_vectors.json").read_text())


@pytest.mark.parametrize("case", PACK_CASES, ids=[c["name"] for c in PACK_CASES])
def test_pack_matches_golden_words(case):
    signs = np.array(case["signs"], dtype=np.int8)
    words = O.pack_signs(signs)
    assert words.dtype == np.int32
    assert words.tolist() == case["words"]


@pytest.mark.parametrize("case", PACK_CASES, ids=[c["name"] for c in PACK_CASES])
def test_unpack_inverts_golden_words(case):
    words = np.array(case["words"], dtype=np.int32)
    rows = len(case["signs"])
    out = O.unpack_signs(words, (rows, case["cols"]))
    assert out.dtype == np.int8
    assert out.tolist() == case["signs"]


def test_bit31_is_int32_min():
    s = np.ones((1, 32), dtype=np.int8)
    s[0, 31] = -1
    assert O.pack_signs(s)[0, 0] == np.iinfo(np.int32).min
    assert O.unpack_signs(np.array([[np.iinfo(np.int32).min]], dtype=np.int32), (1, 32))[0, 31] == -1


def test_pad_bits_are_zero_and_trimmed():
    s = -np.ones((2, 70), dtype=np.int8)
    w = O.pack_signs(s)
    assert w.shape == (2, 3)
    assert (w[:, 2].view(np.uint32) >> 6).tolist() == [0, 0]
    # set pad bits by hand: unpack must ignore them
    w2 = w.copy()
    w2[:, 2] = -1
    assert (O.unpack_signs(w2, (2, 70)) == s).all()


def test_pack_rejects_non_int8():
    with pytest.raises(TypeError):
        O.pack_signs(np.ones((1, 4), dtype=np.int32))


@pytest.mark.parametrize("bad", [(2, 2), (3, 3), (1, 2, 3)])
def test_unpack_rejects_wrong_shape(bad):
    with pytest.raises(ValueError):
        O.unpack_signs(np.zeros(bad, dtype=np.int32), (2, 70))


def test_pack_roundtrip_random():
    rng = _rng(3)
    for cols in (1, 31, 32, 33, 64, 205, 1843):
        s = (1 - 2 * rng.integers(0, 2, size=(5, cols))).astype(np.int8)
        assert (O.unpack_signs(O.pack_signs(s), s.shape) == s).all()


def test_sign_zero_is_plus_one():
    assert O.sign_pm1(np.array([-2.0, -0.0, 0.0, 1e-30, 3.0])).tolist() == [-1, 1, 1, 1, 1]


# --------------------------------------------------------------------------- forward
def test_forward_matches_bruteforce_fixture(forward_cases):
    for c in forward_cases:
        y = O.littlebit_forward(c["x"], c["branches"], c["K"], c["N"], bias=c["bias"])
        assert O.rel_err(y, c["y"]) < 1e-12, c["name"]


def test_forward_all_plus_closed_form():
    rng = _rng(5)
    K, R, N = 70, 13, 40
    x = rng.standard_normal((3, K))
    g, l, h = rng.random(K) + 0.1, rng.random(R) + 0.1, rng.random(N) + 0.1
    b = {"v_sign": np.zeros((R, 3), np.int32), "u_sign": np.zeros((N, 1), np.int32),
         "g": g, "l": l, "h": h, "R": R}
    y = O.littlebit_forward(x, [b], K, N)
    expect = h[None, :] * l.sum() * (x @ g)[:, None]
    np.testing.assert_allclose(y, expect, rtol=1e-12)


def test_forward_rank1_outer_product():
    rng = _rng(6)
    K, N = 45, 33
    b = _rand_branch(rng, K, 1, N)
    x = rng.standard_normal((2, K))
    y = O.littlebit_forward(x, [b], K, N)
    v = b["V"][0].astype(np.float64)
    u = b["U"][:, 0].astype(np.float64)
    s = (x * b["g"]) @ v * b["l"][0]
    np.testing.assert_allclose(y, s[:, None] * (u * b["h"])[None, :], rtol=1e-12)


def test_forward_matches_torch_float64():
    rng = _rng(7)
    K, R, N, M = 130, 47, 77, 4
    b = _rand_branch(rng, K, R, N)
    x = rng.standard_normal((M, K))
    y = O.littlebit_forward(x, [b], K, N)
    tx = torch.from_numpy(x)
    Vq = torch.from_numpy(b["V"]).double()
    Uq = torch.from_numpy(b["U"]).double()
    ref = ((((tx * torch.from_numpy(b["g"])) @ Vq.t()) * torch.from_numpy(b["l"])) @ Uq.t()) * torch.from_numpy(b["h"])
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-12, atol=1e-12)


def test_forward_linear_in_x_and_scales():
    rng = _rng(8)
    K, R, N = 64, 20, 50
    b = _rand_branch(rng, K, R, N)
    x1, x2 = rng.standard_normal((2, K)), rng.standard_normal((2, K))
    f = lambda x, br: O.littlebit_forward(x, [br], K, N)
    np.testing.assert_allclose(f(2.5 * x1 - x2, b), 2.5 * f(x1, b) - f(x2, b), rtol=1e-10, atol=1e-10)
    for key, n in (("g", K), ("l", R), ("h", N)):
        b2 = dict(b)
        b2[key] = b[key] * 3.0
        np.testing.assert_allclose(f(x1, b2), 3.0 * f(x1, b), rtol=1e-12)


def test_forward_residual_is_sum_of_branches():
    rng = _rng(9)
    K, N = 70, 45
    b0, b1 = _rand_branch(rng, K, 11, N), _rand_branch(rng, K, 37, N)
    x = rng.standard_normal((3, K))
    bias = rng.standard_normal(N)
    both = O.littlebit_forward(x, [b0, b1], K, N, bias=bias)
    parts = O.littlebit_forward(x, [b0], K, N) + O.littlebit_forward(x, [b1], K, N) + bias
    np.testing.assert_allclose(both, parts, rtol=1e-12, atol=1e-12)


def test_forward_single_bit_flip_delta():
    """Flipping V[r, k] changes y[n] by -2 * h[n] * U[n, r] * l[r] * V[r, k] * g[k] * x[k]."""
    rng = _rng(10)
    K, R, N = 40, 9, 21
    b = _rand_branch(rng, K, R, N)
    x = rng.standard_normal((1, K))
    y0 = O.littlebit_forward(x, [b], K, N)
    r, k = 4, 33
    V2 = b["V"].copy()
    V2[r, k] = -V2[r, k]
    b2 = dict(b, v_sign=O.pack_signs(V2))
    y1 = O.littlebit_forward(x, [b2], K, N)
    delta = -2.0 * b["h"] * b["U"][:, r] * b["l"][r] * b["V"][r, k] * b["g"][k] * x[0, k]
    np.testing.assert_allclose(y1[0] - y0[0], delta, rtol=1e-9, atol=1e-12)


def test_paired_sign_flip_is_invariant():
    """Negating V row r and U column r together leaves y unchanged."""
    rng = _rng(11)
    K, R, N = 50, 7, 19
    b = _rand_branch(rng, K, R, N)
    x = rng.standard_normal((2, K))
    V2, U2 = b["V"].copy(), b["U"].copy()
    V2[3] *= -1
    U2[:, 3] *= -1
    b2 = dict(b, v_sign=O.pack_signs(V2), u_sign=O.pack_signs(U2))
    np.testing.assert_allclose(O.littlebit_forward(x, [b2], K, N), O.littlebit_forward(x, [b], K, N),
                               rtol=1e-12, atol=1e-12)


def test_fuse_mid_is_exact_product_of_bf16():
    """mid = v1.float() * u2.float() (convert_hf_to_runtime.py:54-57); a product of
    two bf16 values is exact in fp32."""
    rng = _rng(12)
    v1 = torch.from_numpy(rng.standard_normal(300).astype(np.float32)).bfloat16()
    u2 = torch.from_numpy(rng.standard_normal(300).astype(np.float32)).bfloat16()
    mid = O.fuse_mid(v1.float().numpy(), u2.float().numpy())
    exact = v1.double().numpy() * u2.double().numpy()
    assert (mid.astype(np.float64) == exact).all()


def test_rel_err_definition():
    assert O.rel_err(np.array([1.0, 2.0]), np.array([1.0, 4.0])) == pytest.approx(0.5)
    assert O.rel_err(np.zeros((0, 3)), np.zeros((0, 3))) == 0.0


# --------------------------------------------------------------------------- fused inputs
def test_rms_norm_closed_forms():
    w = np.array([1.0, 2.0, -3.0, 0.5])
    # a constant row c: mean(x^2) = c^2, so the output is c / sqrt(c^2 + eps) * w
    for c in (2.0, -0.5):
        x = np.full((1, 4), c)
        np.testing.assert_allclose(O.rms_norm(x, w, 1e-6), c / np.sqrt(c * c + 1e-6) * w[None], rtol=1e-15)
    # eps = 0: scale invariant, unit RMS
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 64))
    np.testing.assert_allclose(O.rms_norm(7.5 * x, np.ones(64), 0.0), O.rms_norm(x, np.ones(64), 0.0), rtol=1e-12)
    np.testing.assert_allclose(np.sqrt((O.rms_norm(x, np.ones(64), 0.0) ** 2).mean(-1)), 1.0, rtol=1e-12)
    # torch's float64 RMSNorm agrees
    tx = torch.from_numpy(x)
    ref = torch.nn.functional.rms_norm(tx, (64,), torch.ones(64, dtype=torch.float64), eps=1e-5).numpy()
    np.testing.assert_allclose(O.rms_norm(x, np.ones(64), 1e-5), ref, rtol=1e-12)


def test_silu_mul_closed_forms():
    assert O.silu_mul(0.0, 5.0) == 0.0
    np.testing.assert_allclose(O.silu_mul(2.0, 3.0), 2.0 / (1.0 + np.exp(-2.0)) * 3.0, rtol=1e-15)
    np.testing.assert_allclose(O.silu_mul(40.0, 1.0), 40.0, rtol=1e-15)  # sigmoid -> 1
    assert abs(O.silu_mul(-40.0, 1.0)) < 1e-15
    g = np.linspace(-6, 6, 25)
    np.testing.assert_allclose(O.silu_mul(g, 1.0), torch.nn.functional.silu(torch.from_numpy(g)).numpy(), rtol=1e-12)

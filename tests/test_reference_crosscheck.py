"""The oracle against the reference's own C++ kernels (oracle/_ref, built from
/root/reference/patches/littlebit_cpu_optimized.cpp by oracle/build_ref.py).

littlebit_cpu_ops::littlebit_linear (patch:598-701) quantises x*v2 and the
latent vector to int8 per row (patch:669, :684), so it agrees with the exact
forward only to the int8 rounding error: max|dy|/max|y| of a few 1e-2.  The
bound 5e-2 still fails for a wrong bit order, sign convention or missing
scale, each of which gives errors of order 1.  Skipped when the reference
library is not built (no /root/reference)."""
import numpy as np
import pytest
import torch

from oracle import build_ref
from oracle import littlebit_oracle as O

pytestmark = pytest.mark.skipif(not build_ref.OUT.exists(), reason="oracle/_ref not built")


def _rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def _case(seed, M, K, N, R):
    rng = _rng(seed)
    V = (1 - 2 * rng.integers(0, 2, size=(R, K))).astype(np.int8)
    U = (1 - 2 * rng.integers(0, 2, size=(N, R))).astype(np.int8)
    b = {"v_sign": O.pack_signs(V), "u_sign": O.pack_signs(U),
         "g": (np.abs(rng.standard_normal(K)) + 0.05).astype(np.float32),
         "l": (np.abs(rng.standard_normal(R)) + 0.05).astype(np.float32),
         "h": (np.abs(rng.standard_normal(N)) + 0.05).astype(np.float32), "R": R}
    x = rng.standard_normal((M, K)).astype(np.float32)
    return x, b


def _ref_linear(ops, x, b, K, N):
    R = b["R"]
    t = torch.from_numpy
    return ops.littlebit_linear(t(x), t(b["g"]).reshape(1, K), t(b["v_sign"]), K, t(b["l"]).reshape(1, R),
                                t(b["u_sign"]), R, t(b["h"]).reshape(1, N)).numpy()


@pytest.mark.parametrize("M,K,N,R", [(1, 4096, 4096, 205), (2, 512, 300, 64), (3, 70, 45, 37), (1, 4096, 11008, 298)])
def test_oracle_matches_reference_cpu_kernel(M, K, N, R):
    ops = build_ref.load()
    x, b = _case(100 + M + R, M, K, N, R)
    err = O.rel_err(_ref_linear(ops, x, b, K, N), O.littlebit_forward(x, [b], K, N))
    assert err < 5e-2, err


def test_reference_rejects_bad_shapes_like_the_gpu_op():
    """The reference's TORCH_CHECKs (patch:607-634) raise RuntimeError; the
    GPU operator mirrors those messages."""
    ops = build_ref.load()
    x, b = _case(1, 1, 64, 32, 8)
    with pytest.raises(RuntimeError, match="v_cols"):
        t = torch.from_numpy
        ops.littlebit_linear(t(x), t(b["g"]).reshape(1, 64), t(b["v_sign"]), 65, t(b["l"]).reshape(1, 8),
                             t(b["u_sign"]), 8, t(b["h"]).reshape(1, 32))

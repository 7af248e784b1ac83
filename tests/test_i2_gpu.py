"""GPU i2 repack (``lbk_repack_signs_to_i2``) byte for byte against the
reference's ``repack_signs_to_i2`` (patches/littlebit_cpu_optimized.cpp:
712-764): against the oracle restatement (oracle/i2_oracle.py) everywhere,
and against the reference's own op (oracle/_ref, built from the patch) where
that library is present.

Shapes: U [N, ceil(R/32)] repacked over R columns and V [R, ceil(K/32)] over
K columns, for the ranks the Llama-2-7B draft and target use (205, 298, 1843,
2686) at K = 4096 and 11008, plus the tails of small and ragged shapes.
"""
import numpy as np
import pytest
import torch

from oracle import build_ref
from oracle import i2_oracle as I

pytestmark = pytest.mark.gpu


def _words(rng, rows, n, extra=0):
    w = rng.integers(0, 2**32, size=(rows, (n + 31) // 32 + extra), dtype=np.uint64).astype(np.uint32)
    if rows and w.shape[1]:
        w[0, 0] = 0x80000000       # bit 31 only
        w[-1, -1] = 0xFFFFFFFF     # pad bits set past n
    return w.view(np.int32)


def _gpu_repack(gpu, w, n):
    from littlebit_amd import repack_signs_to_i2
    out = repack_signs_to_i2(torch.from_numpy(np.ascontiguousarray(w)).to(gpu), n)
    torch.cuda.synchronize()
    return out.cpu().numpy()


_REF = build_ref.OUT.exists()


def _reference(w, n):
    ops = build_ref.load()
    return ops.repack_signs_to_i2(torch.from_numpy(np.ascontiguousarray(w)), n).numpy()


@pytest.mark.parametrize("which,rows,n", [
    ("U", 4096, 205), ("U", 11008, 298), ("U", 4096, 1843), ("U", 11008, 2686), ("U", 4096, 2686),
    ("V", 205, 4096), ("V", 298, 4096), ("V", 1843, 4096), ("V", 2686, 4096),
    ("V", 298, 11008), ("V", 2686, 11008),
])
def test_repack_llama_shapes(gpu, which, rows, n):
    rng = np.random.default_rng(rows * 31 + n)
    w = _words(rng, rows, n)
    out = _gpu_repack(gpu, w, n)
    want = I.repack_signs_to_i2(w, n)
    print(f"[i2] {which} rows={rows} n_cols={n} bytes={out.size}", flush=True)
    assert out.dtype == np.uint8 and out.shape == want.shape
    assert np.array_equal(out, want)
    if _REF:
        assert np.array_equal(out, _reference(w, n))


@pytest.mark.parametrize("rows,n,extra", [(1, 1, 0), (3, 4, 0), (2, 5, 0), (3, 70, 1), (2, 128, 0), (2, 129, 0),
                                          (5, 131, 2), (3, 132, 0), (7, 160, 0), (1, 255, 0), (2, 257, 3)])
def test_repack_tails_and_strides(gpu, rows, n, extra):
    rng = np.random.default_rng(7 * n + rows)
    w = _words(rng, rows, n, extra)
    out = _gpu_repack(gpu, w, n)
    assert np.array_equal(out, I.repack_signs_to_i2(w, n))
    if _REF:
        assert np.array_equal(out, _reference(w, n))


def test_repack_empty_and_errors(gpu):
    from littlebit_amd import repack_signs_to_i2
    z = torch.zeros((0, 3), dtype=torch.int32, device=gpu)
    assert tuple(repack_signs_to_i2(z, 70).shape) == (0, 18)
    z = torch.zeros((3, 1), dtype=torch.int32, device=gpu)
    assert tuple(repack_signs_to_i2(z, 0).shape) == (3, 0)
    with pytest.raises(RuntimeError, match="sign words"):
        repack_signs_to_i2(torch.zeros((2, 2), dtype=torch.int32, device=gpu), 65)
    with pytest.raises(RuntimeError, match="int32"):
        repack_signs_to_i2(torch.zeros((2, 2), dtype=torch.int64, device=gpu), 40)
    with pytest.raises(RuntimeError, match="CUDA"):
        repack_signs_to_i2(torch.zeros((2, 2), dtype=torch.int32), 40)

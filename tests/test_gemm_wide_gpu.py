"""Wide stage-2 tiles of the GEMM path (bf16 activations, enough blocks).

When a bf16 call's stage 2 has at least two blocks per CU in 256-column
tiles, each wave covers 64 x 128 outputs with one set of accumulators for
both branches: acc = S0, rescaled per column by h0 / h1 in fp32, then S1 is
added and y = h1 * acc (branch 1 dropped where |h1| is zero or denormal).
These shapes take that path; rows are checked against the float64 oracle on
a fixed sample (rows are independent), including the first and last m-tile,
with the column scales at their edges.
"""
import numpy as np
import pytest
import torch

from oracle import littlebit_oracle as O

pytestmark = pytest.mark.gpu

TOL_BF16_PREFILL = 5e-3


def _dev_branch(b, dev):
    from littlebit_amd import LittleBitBranch
    t = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a if dt is None else np.asarray(a, dt))).to(dev)  # noqa: E731
    return LittleBitBranch(v_sign=t(b["v_sign"]), u_sign=t(b["u_sign"]), v2=t(b["g"], np.float32),
                           mid=t(b["l"], np.float32), u1=t(b["h"], np.float32))


def _rows(M, seed):
    r = {0, 1, 63, 64, 127, 128, M // 2, M - 129, M - 128, M - 2, M - 1}
    r |= set(np.random.Generator(np.random.PCG64(seed)).choice(M, 21, replace=False).tolist())
    return np.array(sorted(r))


def test_wide_tiles_branch_scale_edges(gpu):
    """Columns with h1 = 0, h0 = 0, h1 denormal, h1 tiny and huge against h0,
    and mixed signs, across subtiles of both wave columns."""
    from littlebit_amd import LittleBitProjection
    from littlebit_amd.synthetic import make_branch
    M, K, N = 1024, 256, 16384  # 8 m-tiles x 64 wide column tiles = 512 blocks
    rng = np.random.Generator(np.random.PCG64(9100))
    brs = [make_branch(rng, K, R, N, direct_words=True).as_dict() for R in (40, 300)]
    h0 = np.asarray(brs[0]["h"], np.float32).copy()
    h1 = np.asarray(brs[1]["h"], np.float32).copy()
    h1[0:40] = 0.0
    h0[40:80] = 0.0
    h1[80:120] = np.float32(1e-38)            # denormal-adjacent: below the rescale threshold
    h1[120:160] = h0[120:160] * 1e-25         # h0 / h1 huge but finite
    h0[160:200] = h1[160:200] * 1e-25
    h1[200:240] = -h1[200:240]
    h0[300:400] = -3.0 * h0[300:400]
    h1[16000:16384] = 0.0                     # last tile
    brs[0]["h"], brs[1]["h"] = h0, h1
    proj = LittleBitProjection([_dev_branch(b, gpu) for b in brs])
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(gpu).to(torch.bfloat16)
    y = proj.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = _rows(M, 9101)
    xs = x.float().cpu().numpy()[rows]
    ref = O.littlebit_forward(xs, brs, K, N)
    yr = y.cpu().numpy()[rows]
    err = O.rel_err(yr, ref)
    print(f"[wide] edges rows={len(rows)} rel_err={err:.3e}", flush=True)
    assert err <= TOL_BF16_PREFILL
    for lo, hi in [(0, 40), (40, 80), (80, 120), (120, 160), (160, 200), (200, 240), (16000, 16384)]:
        e = O.rel_err(yr[:, lo:hi], ref[:, lo:hi])
        print(f"[wide] columns {lo}-{hi} rel_err={e:.3e}", flush=True)
        assert e <= TOL_BF16_PREFILL, (lo, hi, e)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_wide_tiles_group_bias_residual(gpu, out_dtype):
    """A group of two projections (columns of both in one grid), bias, and a
    residual that is the output itself (fp32) or separate (bf16 output)."""
    from littlebit_amd import LittleBitProjection, LittleBitProjectionGroup
    from littlebit_amd.synthetic import make_branch
    M, K, N = 1100, 512, 8192  # 9 m-tiles x (32 + 32) wide column tiles = 576 blocks; ragged last m-tile
    rng = np.random.Generator(np.random.PCG64(9200))
    host = [[make_branch(rng, K, R, N, direct_words=True).as_dict() for R in (37, 301)] for _ in range(2)]
    biases = [rng.standard_normal(N).astype(np.float32) for _ in range(2)]
    grp = LittleBitProjectionGroup([LittleBitProjection([_dev_branch(b, gpu) for b in brs],
                                                        torch.from_numpy(bb).to(gpu))
                                    for brs, bb in zip(host, biases)])
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(gpu).to(torch.bfloat16)
    res = [torch.from_numpy((rng.standard_normal((M, N)) * 2).astype(np.float32)).to(gpu) for _ in range(2)]
    if out_dtype == torch.float32:
        outs = [r.clone() for r in res]
        grp.forward(x, outs=outs, out_dtype=out_dtype, residuals=outs)
    else:
        outs = [torch.empty((M, N), dtype=out_dtype, device=gpu) for _ in range(2)]
        grp.forward(x, outs=outs, out_dtype=out_dtype, residuals=res)
    torch.cuda.synchronize()
    rows = _rows(M, 9201)
    xs = x.float().cpu().numpy()[rows]
    for i in range(2):
        ref = O.littlebit_forward(xs, host[i], K, N, bias=biases[i]) + res[i].cpu().numpy()[rows]
        err = O.rel_err(outs[i].float().cpu().numpy()[rows], ref)
        print(f"[wide] group proj {i} out={out_dtype} rel_err={err:.3e}", flush=True)
        assert err <= TOL_BF16_PREFILL


def test_wide_tiles_large_scale_ratio_with_large_inputs(gpu):
    """Columns with |h0 / h1| far beyond 2^40 (h1 = 1e-29, h0 = 1e3) on inputs
    of magnitude 1e6: rescaling acc by h0 / h1 would overflow fp32 there, so
    branch 1 is dropped (its term is below 2^-40 of branch 0's scale); columns
    with |h0 / h1| just under 2^40 keep the rescale.  Every output finite and
    within the bar against the oracle."""
    from littlebit_amd import LittleBitProjection
    from littlebit_amd.synthetic import make_branch
    M, K, N = 1024, 256, 16384
    rng = np.random.Generator(np.random.PCG64(9150))
    brs = [make_branch(rng, K, R, N, direct_words=True).as_dict() for R in (40, 300)]
    h0 = np.asarray(brs[0]["h"], np.float32).copy()
    h1 = np.asarray(brs[1]["h"], np.float32).copy()
    h1[0:64] = np.float32(1e-29)
    h0[0:64] = np.float32(1e3)
    h1[64:128] = h0[64:128] * np.float32(2.0 ** -39)   # ratio 2^39: rescaled
    h1[128:192] = -np.float32(1e-29)
    h0[128:192] = -np.float32(1e3)
    brs[0]["h"], brs[1]["h"] = h0, h1
    proj = LittleBitProjection([_dev_branch(b, gpu) for b in brs])
    x = torch.from_numpy((rng.standard_normal((M, K)) * 1e6).astype(np.float32)).to(gpu).to(torch.bfloat16)
    y = proj.forward(x, out_dtype=torch.float32)
    torch.cuda.synchronize()
    yc = y.cpu().numpy()
    assert np.isfinite(yc).all()
    rows = _rows(M, 9151)
    ref = O.littlebit_forward(x.float().cpu().numpy()[rows], brs, K, N)
    yr = yc[rows]
    for lo, hi in [(0, 64), (64, 128), (128, 192), (192, N)]:
        e = O.rel_err(yr[:, lo:hi], ref[:, lo:hi])
        print(f"[wide] large ratio columns {lo}-{hi} rel_err={e:.3e}", flush=True)
        assert e <= TOL_BF16_PREFILL, (lo, hi, e)

"""An output that shares memory with the input, where the rows run as row
chunks one launch pair after another (deterministic mode above 16 rows;
rows whose latent vectors do not fit one latent half at once).  bf16 x with
fp32 y at x's address: y's rows are twice as wide as x's, so a chunk's
output covers the input rows of the chunks after it.  The library runs the
chunks last to first, reading every input row before any output overlaps
it; the result is checked against the oracle on the input as it was."""
import numpy as np
import pytest
import torch

from oracle import littlebit_oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3


def _group(seed, K, specs, dev):
    from littlebit_amd import LittleBitBranch, LittleBitProjection, LittleBitProjectionGroup
    from littlebit_amd.synthetic import make_projection
    host, projs = [], []
    for i, (N, ranks) in enumerate(specs):
        _, brs = make_projection(seed + 13 * i, 1, K, N, ranks)
        host.append([b.as_dict() for b in brs])
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        projs.append(LittleBitProjection([LittleBitBranch(v_sign=t(b.v_sign), u_sign=t(b.u_sign), v2=t(b.g),
                                                          mid=t(b.l), u1=t(b.h)) for b in brs]))
    return host, LittleBitProjectionGroup(projs)


def _aliased_call(gpu, seed, M, K, specs):
    host, grp = _group(seed, K, specs, gpu)
    N0 = specs[0][0]
    buf = torch.empty(M * max(N0 * 4, K * 2), dtype=torch.uint8, device=gpu)
    x = buf[:M * K * 2].view(torch.bfloat16).view(M, K)
    g = torch.Generator(device="cpu").manual_seed(seed)
    x.copy_(torch.randn((M, K), generator=g).to(torch.bfloat16).to(gpu))
    xs = x.float().cpu().numpy()
    y0 = buf[:M * N0 * 4].view(torch.float32).view(M, N0)
    outs = [y0] + [torch.empty((M, N), device=gpu) for N, _ in specs[1:]]
    print(f"[alias] M={M} K={K} N={[n for n, _ in specs]} y0 at x's address", flush=True)
    grp.forward(x, outs=outs, out_dtype=torch.float32)
    torch.cuda.synchronize()
    for i, ((N, _), y) in enumerate(zip(specs, outs)):
        err = O.rel_err(y.cpu().numpy(), O.littlebit_forward(xs, host[i], K, N))
        print(f"[alias] projection {i}: rel_err={err:.3e}", flush=True)
        assert err <= TOL_F32, (M, i, err)


def test_aliased_output_deterministic_chunks(gpu):
    """Deterministic mode: 33 rows as 16 + 16 + 1 rows one after another."""
    from littlebit_amd import deterministic
    with deterministic():
        _aliased_call(gpu, 9300, 33, 4096, [(4096, [205, 1843])])


def test_aliased_output_chunks_whose_latents_do_not_fit(gpu):
    """48 rows of a target q/k/v group: 48 x 3 x (256 + 1920) latent floats
    exceed one latent half, so the chunks run one after another."""
    _aliased_call(gpu, 9400, 48, 4096, [(4096, [205, 1843]), (4096, [205, 1843]), (4096, [205, 1843])])

"""V's tiled copy (lbk_tile_v_signs, read by the decode path's latent
kernel when lbk_branch.v_sign_tiled is set): the copy against the documented
layout, and forwards that read it against forwards that read V as stored --
bit for bit in deterministic mode (the same products summed in the same
order), and against the oracle -- over ragged ranks and K (K % 128 != 0,
ceil(K/32) % 4 != 0, a partial last cell), every k-chunk width the planner
picks (M = 1, 5, 8, 16 and row chunks at 33), fused inputs and groups."""
import numpy as np
import pytest
import torch

from oracle import littlebit_oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3


def _tiled_np(v, R, K):
    """[ceil(R/16)][ceil(KW/4)][16][4] of v [R, KW], zero-padded."""
    KW = (K + 31) // 32
    R16, KW4 = (R + 15) // 16, (KW + 3) // 4
    pad = np.zeros((R16 * 16, KW4 * 4), dtype=np.int32)
    pad[:R, :KW] = v
    return pad.reshape(R16, 16, KW4, 4).transpose(0, 2, 1, 3).reshape(-1)


@pytest.mark.parametrize("R,K", [(1, 32), (16, 128), (37, 70), (205, 4096), (298, 11008), (1843, 4096), (45, 3000)])
def test_tile_v_layout(gpu, R, K):
    import littlebit_amd._lib as L
    lib = L.load()
    rng = np.random.default_rng(R * 7 + K)
    KW = (K + 31) // 32
    v = rng.integers(-2**31, 2**31, size=(R, KW), dtype=np.int64).astype(np.int32)
    n = lib.lbk_tiled_v_words(R, K)
    assert n == ((R + 15) // 16) * ((KW + 3) // 4) * 64
    out = torch.full((n,), -7, dtype=torch.int32, device=gpu)
    L.check(lib.lbk_tile_v_signs(torch.from_numpy(v).to(gpu).data_ptr(), R, K, out.data_ptr(),
                                 torch.cuda.current_stream(gpu).cuda_stream), "lbk_tile_v_signs")
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), _tiled_np(v, R, K))


def _pair(seed, K, specs, gpu, bias=False):
    """Two groups over the same device factors: V tiled and V as stored."""
    from littlebit_amd import LittleBitBranch, LittleBitProjection, LittleBitProjectionGroup
    from littlebit_amd.synthetic import make_projection
    host, pt, pu = [], [], []
    for i, (N, ranks) in enumerate(specs):
        _, brs = make_projection(seed + 11 * i, 1, K, N, ranks)
        host.append([b.as_dict() for b in brs])
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
        dev = [LittleBitBranch(v_sign=t(b.v_sign), u_sign=t(b.u_sign), v2=t(b.g), mid=t(b.l), u1=t(b.h))
               for b in brs]
        bb = torch.from_numpy(np.random.default_rng(seed + i).standard_normal(N).astype(np.float32)).to(gpu) \
            if bias else None
        pt.append(LittleBitProjection(dev, bb, tile_v=True))
        pu.append(LittleBitProjection(dev, bb, tile_v=False))
        assert len(pt[-1]._v_tiled) == len(brs) and not pu[-1]._v_tiled
    return host, LittleBitProjectionGroup(pt), LittleBitProjectionGroup(pu), [p.bias for p in pt]


@pytest.mark.parametrize("M", [1, 5, 8, 16, 33])
@pytest.mark.parametrize("K,specs", [
    (4096, [(4096, [205, 1843]), (1024, [205, 1843]), (1024, [205, 1843])]),   # target q/k/v group
    (11008, [(4096, [298, 2686])]),                                             # target down
    (3000, [(700, [45, 130])]),                                                 # ragged: KW = 94, a partial cell
    (70, [(96, [37])]),                                                         # K < 128
])
def test_tiled_forward_matches_stored_layout(gpu, M, K, specs):
    from littlebit_amd import deterministic
    host, gt, gu, biases = _pair(9500 + M + K, K, specs, gpu, bias=True)
    x = torch.from_numpy(np.random.default_rng(M * 31 + K).standard_normal((M, K)).astype(np.float32)).to(gpu)
    print(f"[tiled] M={M} K={K} N={[n for n, _ in specs]}", flush=True)
    with deterministic():
        yt = [y.cpu().numpy() for y in gt.forward(x)]
        yu = [y.cpu().numpy() for y in gu.forward(x)]
    for i, (a, b) in enumerate(zip(yt, yu)):
        assert np.array_equal(a, b), (M, K, i, O.rel_err(a, b))
    yt = [y.cpu().numpy() for y in gt.forward(x)]
    xs = x.cpu().numpy()
    for i, ((N, _), y) in enumerate(zip(specs, yt)):
        err = O.rel_err(y, O.littlebit_forward(xs, host[i], K, N, bias=biases[i].cpu().numpy()))
        print(f"[tiled] projection {i}: rel_err={err:.2e}", flush=True)
        assert err <= TOL_F32


def test_tiled_fused_inputs(gpu):
    """RMSNorm input on a group and SiLU * up with an in-place residual, 8 rows."""
    host, gt, gu, _ = _pair(9600, 4096, [(11008, [298, 2686]), (11008, [298, 2686])], gpu)
    g = torch.Generator(device="cpu").manual_seed(9601)
    x = torch.randn((8, 4096), generator=g).to(gpu)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to(gpu)
    a = gt.forward(x, rms_weight=w, rms_eps=1e-6)
    b = gu.forward(x, rms_weight=w, rms_eps=1e-6)
    xn = O.rms_norm(x.double().cpu().numpy(), w.double().cpu().numpy(), 1e-6)
    for i in range(2):
        assert O.rel_err(a[i].cpu().numpy(), b[i].cpu().numpy()) <= 1e-5
        assert O.rel_err(a[i].cpu().numpy(), O.littlebit_forward(xn, host[i], 4096, 11008)) <= TOL_F32
    hd, dt, du, _ = _pair(9700, 11008, [(4096, [298, 2686])], gpu)
    gate, up = a[0], a[1]
    res = torch.randn((8, 4096), generator=g).to(gpu)
    yt, yu = res.clone(), res.clone()
    dt.forward(gate, outs=[yt], x_up=up, residuals=[yt])
    du.forward(gate, outs=[yu], x_up=up, residuals=[yu])
    ref = O.littlebit_forward(O.silu_mul(gate.double().cpu().numpy(), up.double().cpu().numpy()), hd[0], 11008,
                              4096) + res.double().cpu().numpy()
    assert O.rel_err(yt.cpu().numpy(), yu.cpu().numpy()) <= 1e-5
    assert O.rel_err(yt.cpu().numpy(), ref) <= TOL_F32

"""lbk_group_forward_noalloc (the entry point that allocates nothing; its
workspace is the library's per-device scratch array) against
lbk_group_forward_ex with a caller workspace, through the C ABI, and both
against the oracle.  Calls follow each other on the one scratch with
different shapes, each later one smaller, so state a call leaves behind
(latent-buffer halves, sizes) must not leak into the next."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import littlebit_oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3


def _projections(seed, M, K, specs, dev):
    from littlebit_amd import LittleBitBranch, LittleBitProjection
    from littlebit_amd.synthetic import make_projection
    x = None
    host, projs = [], []
    for i, (N, ranks) in enumerate(specs):
        xi, brs = make_projection(seed + 17 * i, M, K, N, ranks)
        x = xi if x is None else x
        host.append([b.as_dict() for b in brs])
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        projs.append(LittleBitProjection([LittleBitBranch(v_sign=t(b.v_sign), u_sign=t(b.u_sign), v2=t(b.g),
                                                          mid=t(b.l), u1=t(b.h)) for b in brs]))
    return x, host, projs


def _array(projs, outs):
    import littlebit_amd._lib as L
    arr = (L.LbkProjection * len(projs))()
    for i, (p, o) in enumerate(zip(projs, outs)):
        arr[i].branches = ctypes.cast(p._arr, ctypes.POINTER(L.LbkBranch))
        arr[i].n_branches = len(p.branches)
        arr[i].out_features = p.out_features
        arr[i].bias = None
        arr[i].y = o.data_ptr()
        arr[i].residual = None
    return arr


def _both(gpu, M, K, specs, seed):
    """(noalloc outputs, workspace outputs, host factors, x) of one group call."""
    import littlebit_amd._lib as L
    lib = L.load()
    x, host, projs = _projections(seed, M, K, specs, gpu)
    tx = torch.from_numpy(x).to(gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    outs_a = [torch.full((M, N), float("nan"), device=gpu) for N, _ in specs]
    outs_b = [torch.full((M, N), float("nan"), device=gpu) for N, _ in specs]
    arr_a, arr_b = _array(projs, outs_a), _array(projs, outs_b)
    print(f"[noalloc] M={M} K={K} specs={specs}", flush=True)
    rc = lib.lbk_group_forward_noalloc(arr_a, len(projs), M, K, tx.data_ptr(), L.LBK_F32, None, L.LBK_F32, stream)
    L.check(rc, "lbk_group_forward_noalloc")
    need = lib.lbk_group_workspace_bytes(arr_b, len(projs), M, K)
    assert 0 < need <= L.LBK_NOALLOC_SCRATCH_BYTES
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    rc = lib.lbk_group_forward_ex(arr_b, len(projs), M, K, tx.data_ptr(), L.LBK_F32, None, L.LBK_F32,
                                  ws.data_ptr(), need, stream)
    L.check(rc, "lbk_group_forward_ex")
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs_a], [o.cpu().numpy() for o in outs_b], host, x


def test_noalloc_matches_workspace_entry_point(gpu):
    # decode path (M = 8, a target q/k/v group), GEMM path (M = 100), then
    # smaller calls on the same scratch: M = 3, then M = 1 with a smaller shape
    cases = [(8, 4096, [(4096, [205, 1843]), (1024, [205, 1843]), (1024, [205, 1843])], 7100),
             (100, 1000, [(300, [64, 130])], 7200),
             (3, 4096, [(11008, [298])], 7300),
             (1, 512, [(96, [45])], 7400)]
    for M, K, specs, seed in cases:
        ya, yb, host, x = _both(gpu, M, K, specs, seed)
        for i, ((N, _), a, b) in enumerate(zip(specs, ya, yb)):
            assert np.isfinite(a).all(), (M, i)
            same = O.rel_err(a, b)
            ref = O.rel_err(a, O.littlebit_forward(x, host[i], K, N))
            print(f"[noalloc] M={M} proj {i}: vs workspace entry {same:.2e}, vs oracle {ref:.2e}", flush=True)
            # k-chunk partial sums meet in fp32 atomics: equal up to their order
            assert same <= 1e-5, (M, i, same)
            assert ref <= TOL_F32, (M, i, ref)


def test_noalloc_rejects_shapes_beyond_its_scratch(gpu):
    """A call whose workspace exceeds the scratch fails with
    LBK_ERR_WORKSPACE before any launch, and the next call still works."""
    import littlebit_amd._lib as L
    lib = L.load()
    M, K, specs = 4096, 4096, [(4096, [205, 1843])]
    _, _, projs = _projections(7500, 1, K, specs, gpu)
    out = torch.empty((M, 4096), device=gpu)
    arr = _array(projs, [out])
    assert lib.lbk_group_workspace_bytes(arr, 1, M, K) > L.LBK_NOALLOC_SCRATCH_BYTES
    x = torch.zeros((M, K), device=gpu)
    rc = lib.lbk_group_forward_noalloc(arr, 1, M, K, x.data_ptr(), L.LBK_F32, None, L.LBK_F32,
                                       torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == L.LBK_ERR_WORKSPACE and "scratch" in L.last_error()
    ya, yb, host, xs = _both(gpu, 2, 512, [(96, [45, 7])], 7600)
    assert O.rel_err(ya[0], yb[0]) <= 1e-5
    assert O.rel_err(ya[0], O.littlebit_forward(xs, host[0], 512, 96)) <= TOL_F32


def test_noalloc_captured_and_replayed_between_eager_calls(gpu):
    """A noalloc call captured in a graph and replayed four times, with eager
    noalloc calls of another shape on the same scratch between the replays
    (the replays and the eager calls hand the latent buffer on to each
    other); every replay and every eager call against the oracle."""
    import littlebit_amd._lib as L
    lib = L.load()
    K, M, specs = 4096, 8, [(4096, [205, 1843])]
    x, host, projs = _projections(7700, M, K, specs, gpu)
    tx = torch.from_numpy(x).to(gpu)
    y = torch.zeros((M, 4096), device=gpu)
    arr = _array(projs, [y])
    ref = O.littlebit_forward(x, host[0], K, 4096)
    # the eager shape: one row of a draft gate/up-like projection
    xe, host_e, projs_e = _projections(7800, 1, K, [(11008, [298])], gpu)
    txe = torch.from_numpy(xe).to(gpu)
    ye = torch.zeros((1, 11008), device=gpu)
    arr_e = _array(projs_e, [ye])
    ref_e = O.littlebit_forward(xe, host_e[0], K, 11008)

    def eager():
        rc = lib.lbk_group_forward_noalloc(arr_e, 1, 1, K, txe.data_ptr(), L.LBK_F32, None, L.LBK_F32,
                                           torch.cuda.current_stream(gpu).cuda_stream)
        L.check(rc, "lbk_group_forward_noalloc (eager)")
        torch.cuda.synchronize()
        assert O.rel_err(ye.cpu().numpy(), ref_e) <= TOL_F32

    eager()  # the scratch is set up and cleared before the capture
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        # warm the call on the capture stream once, eagerly
        L.check(lib.lbk_group_forward_noalloc(arr, 1, M, K, tx.data_ptr(), L.LBK_F32, None, L.LBK_F32,
                                              side.cuda_stream), "lbk_group_forward_noalloc (warm)")
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()
    print("[noalloc] capturing M=8 target q shape", flush=True)
    with torch.cuda.graph(graph):
        rc = lib.lbk_group_forward_noalloc(arr, 1, M, K, tx.data_ptr(), L.LBK_F32, None, L.LBK_F32,
                                           torch.cuda.current_stream(gpu).cuda_stream)
    L.check(rc, "lbk_group_forward_noalloc (captured)")
    for rep in range(4):
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        err = O.rel_err(y.cpu().numpy(), ref)
        print(f"[noalloc] replay {rep}: rel_err={err:.2e}", flush=True)
        assert err <= TOL_F32, (rep, err)
        eager()

"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Bar: sign unpacking bit-exact; forward
max|y - y_ref| / max|y_ref| <= 1e-3 for fp32 outputs.  bf16 outputs add the
rounding of the output itself (relative 2**-9 per element), so their bar is
4e-3.  Inputs are the seeded generator's (numpy PCG64).
"""
import numpy as np
import pytest
import torch

from oracle import littlebit_oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3
TOL_BF16_OUT = 4e-3
TOL_BF16_PREFILL = 5e-3  # bf16 activations at M > 16: bf16 MFMA operands


def _dev_branch(b, dev):
    from littlebit_amd import LittleBitBranch
    return LittleBitBranch(
        v_sign=torch.from_numpy(np.ascontiguousarray(b["v_sign"])).to(dev),
        u_sign=torch.from_numpy(np.ascontiguousarray(b["u_sign"])).to(dev),
        v2=torch.from_numpy(np.asarray(b["g"], np.float32)).to(dev),
        mid=torch.from_numpy(np.asarray(b["l"], np.float32)).to(dev),
        u1=torch.from_numpy(np.asarray(b["h"], np.float32)).to(dev),
    )


def _run(dev, x, branches, bias=None, x_dtype=torch.float32, out_dtype=None):
    from littlebit_amd import LittleBitProjection
    proj = LittleBitProjection([_dev_branch(b, dev) for b in branches],
                               None if bias is None else torch.from_numpy(bias).to(dev))
    tx = torch.from_numpy(np.asarray(x, np.float32)).to(dev).to(x_dtype)
    y = proj.forward(tx, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), tx.float().cpu().numpy()


def _synthetic(seed, M, K, N, ranks):
    from littlebit_amd.synthetic import make_projection
    x, brs = make_projection(seed, M, K, N, ranks)
    return x, [b.as_dict() for b in brs]


def _check(y, x_used, branches, K, N, tol, bias=None, what=""):
    ref = O.littlebit_forward(x_used, branches, K, N, bias=bias)
    err = O.rel_err(y, ref)
    print(f"[parity] {what} rel_err={err:.3e}", flush=True)
    assert err <= tol, f"{what}: rel_err {err:.3e} > {tol}"
    return err


# --------------------------------------------------------------------------- sign unpack / pack
@pytest.mark.parametrize("rows,cols", [(1, 32), (5, 70), (205, 4096), (4096, 205), (7, 1843)])
def test_unpack_bit_exact(gpu, rows, cols):
    from littlebit_amd import binary_unpacker
    rng = np.random.Generator(np.random.PCG64(rows * 7919 + cols))
    wpr = (cols + 31) // 32
    words = rng.integers(0, 2**32, size=(rows, wpr), dtype=np.uint64).astype(np.uint32)
    words[0, 0] = 0x80000000  # bit 31 only
    if rows > 1:
        words[1, -1] = 0xFFFFFFFF  # pad bits set: must be ignored
    w32 = words.view(np.int32)
    out = binary_unpacker(torch.from_numpy(w32).to(gpu), (rows, cols)).cpu().numpy()
    assert (out == O.unpack_signs(w32, (rows, cols))).all()


@pytest.mark.parametrize("rows,cols", [(1, 32), (5, 70), (205, 4096), (11008, 298)])
def test_pack_bit_exact(gpu, rows, cols):
    from littlebit_amd import binary_packer
    rng = np.random.Generator(np.random.PCG64(rows + 31 * cols))
    s = (1 - 2 * rng.integers(0, 2, size=(rows, cols))).astype(np.int8)
    out = binary_packer(torch.from_numpy(s).to(gpu)).cpu().numpy()
    assert (out == O.pack_signs(s)).all()


# --------------------------------------------------------------------------- forward
def test_golden_fixtures(gpu, forward_cases):
    for c in forward_cases:
        y, _ = _run(gpu, c["x"], c["branches"], bias=c["bias"])
        err = O.rel_err(y, c["y"])
        print(f"[parity] fixture {c['name']} rel_err={err:.3e}", flush=True)
        assert err <= 1e-4, c["name"]  # 10x tighter than the 1e-3 bar


def test_config0_gemv(gpu):
    K = N = 4096
    x, brs = _synthetic(1000, 1, K, N, [205])
    y, xu = _run(gpu, x, brs)
    _check(y, xu, brs, K, N, TOL_F32, what="config0 M=1")


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_config1_draft_plus_residual(gpu, M):
    K = N = 4096
    x, brs = _synthetic(1001, M, K, N, [205, 1843])
    y, xu = _run(gpu, x, brs)
    _check(y, xu, brs, K, N, TOL_F32, what=f"config1 M={M}")


@pytest.mark.parametrize("name,K,N,ranks,M", [
    ("gate_up_verify", 4096, 11008, [298, 2686], 8),
    ("down_verify", 11008, 4096, [298, 2686], 8),
    ("down_draft", 11008, 4096, [298], 1),
    ("qkv_tree32", 4096, 4096, [205, 1843], 32),
])
def test_llama_shapes(gpu, name, K, N, ranks, M):
    x, brs = _synthetic(1003, M, K, N, ranks)
    y, xu = _run(gpu, x, brs)
    _check(y, xu, brs, K, N, TOL_F32, what=name)


@pytest.mark.parametrize("M,K,N,ranks", [(3, 70, 45, [37]), (5, 33, 31, [31, 1]), (9, 1000, 77, [64, 95]),
                                         (17, 96, 130, [3])])
def test_ragged_shapes(gpu, M, K, N, ranks):
    x, brs = _synthetic(77 + M, M, K, N, ranks)
    y, xu = _run(gpu, x, brs)
    _check(y, xu, brs, K, N, TOL_F32, what=f"ragged M={M} K={K} N={N} R={ranks}")


@pytest.mark.parametrize("M,K,N,ranks", [(1, 256, 300, [8192]), (1, 320, 200, [100, 7000]), (2, 256, 130, [6000]),
                                         (8, 128, 96, [4600]), (8, 200, 70, [300, 4200])])
def test_expand_staging_tail(gpu, M, K, N, ranks):
    """Rank slices with more staging tasks than the expand block has threads: at one row a rank of 7000-8192 is
    875-1024 chunks of 8 ranks in one slice (one-row calls are not sliced) against at most 768 threads, so the
    block stages the rest before it issues its sign words; at 2 and 8 rows whichever slices the planner picks."""
    x, brs = _synthetic(4242 + M + ranks[-1], M, K, N, ranks)
    y, xu = _run(gpu, x, brs)
    _check(y, xu, brs, K, N, TOL_F32, what=f"tail M={M} K={K} N={N} ranks={ranks}")


def test_bias(gpu):
    K, N = 300, 200
    x, brs = _synthetic(5, 4, K, N, [40, 70])
    bias = np.random.Generator(np.random.PCG64(5)).standard_normal(N).astype(np.float32)
    y, xu = _run(gpu, x, brs, bias=bias)
    _check(y, xu, brs, K, N, TOL_F32, bias=bias, what="bias")


def test_bf16_in_fp32_out(gpu):
    K = N = 4096
    x, brs = _synthetic(1004, 8, K, N, [205, 1843])
    y, xu = _run(gpu, x, brs, x_dtype=torch.bfloat16, out_dtype=torch.float32)
    _check(y, xu, brs, K, N, TOL_F32, what="bf16 in / fp32 out")


def test_bf16_in_bf16_out(gpu):
    K = N = 4096
    x, brs = _synthetic(1005, 64, K, N, [204, 1843])
    y, xu = _run(gpu, x, brs, x_dtype=torch.bfloat16, out_dtype=torch.bfloat16)
    _check(y, xu, brs, K, N, TOL_BF16_OUT, what="bf16 in / bf16 out M=64")


def test_prefill_shape_small(gpu):
    """bf16 activations at M > 16 take the bf16 GEMM path (a Llama-3-8B prefill shape, fewer tokens)."""
    K, N = 4096, 4096
    x, brs = _synthetic(1006, 256, K, N, [204, 1843])
    y, xu = _run(gpu, x, brs, x_dtype=torch.bfloat16, out_dtype=torch.float32)
    _check(y, xu, brs, K, N, TOL_BF16_PREFILL, what="bf16 M=256")


@pytest.mark.parametrize("M,K,N,ranks", [(512, 4096, 1024, [81, 737]), (130, 14336, 4096, [318]),
                                         (200, 4096, 14336, [318, 2867])])
def test_prefill_bf16_llama3_shapes(gpu, M, K, N, ranks):
    x, brs = _synthetic(1010 + M, M, K, N, ranks)
    y, xu = _run(gpu, x, brs, x_dtype=torch.bfloat16, out_dtype=torch.bfloat16)
    _check(y, xu, brs, K, N, TOL_BF16_PREFILL, what=f"bf16 M={M} K={K} N={N} R={ranks}")


@pytest.mark.parametrize("M,K,N,ranks,offset", [(129, 1000, 300, [130, 7], 0), (100, 4160, 520, [37, 300], 0),
                                                (96, 4096, 1024, [81, 737], 1), (70, 64, 33, [1, 64], 0)])
def test_gemm_path_bf16_input_forms(gpu, M, K, N, ranks, offset):
    """bf16 GEMM path, both forms of stage 1: rows of whole 64-k steps at a
    16-byte aligned address go to the MFMA as they are, with g in the sign
    operand; other K, or x at a misaligned address (a view `offset` elements
    into its buffer), take a g-scaled copy first."""
    from littlebit_amd import LittleBitProjection
    x, brs = _synthetic(1030 + M, M, K, N, ranks)
    proj = LittleBitProjection([_dev_branch(b, gpu) for b in brs])
    buf = torch.zeros(M * K + offset, dtype=torch.bfloat16, device=gpu)
    tx = buf[offset:].view(M, K)
    tx.copy_(torch.from_numpy(np.asarray(x, np.float32)).to(gpu))
    y = proj.forward(tx, out_dtype=torch.float32)
    torch.cuda.synchronize()
    _check(y.cpu().numpy(), tx.float().cpu().numpy(), brs, K, N, TOL_BF16_PREFILL,
           what=f"bf16 gemm M={M} K={K} N={N} R={ranks} offset={offset}")


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_gemm_expand_branch_scale_edges(gpu, x_dtype):
    """The GEMM path's stage 2 scales each branch's sums by its own row
    scale h before adding them: columns with h1 = 0, h0 = 0, h1 tiny against
    h0, h0 tiny against h1 and mixed signs, against the oracle (a form that
    folds the scales into one accumulator set must pass these too)."""
    M, K, N = 100, 512, 300
    x, brs = _synthetic(1040, M, K, N, [40, 300])
    h0 = np.asarray(brs[0]["h"], np.float32).copy()
    h1 = np.asarray(brs[1]["h"], np.float32).copy()
    h1[0:20] = 0.0
    h0[20:40] = 0.0
    h1[40:60] = h0[40:60] * 1e-25
    h0[60:80] = h1[60:80] * 1e-25
    h1[80:100] = -h1[80:100]
    h0[100:120] = -3.0 * h0[100:120]
    brs[0]["h"], brs[1]["h"] = h0, h1
    y, xu = _run(gpu, x, brs, x_dtype=x_dtype, out_dtype=torch.float32)
    tol = TOL_F32 if x_dtype == torch.float32 else TOL_BF16_PREFILL
    _check(y, xu, brs, K, N, tol, what=f"expand branch scale edges {x_dtype}")
    ref = O.littlebit_forward(xu, brs, K, N)
    for lo, hi in [(0, 20), (20, 40), (40, 60), (60, 80)]:
        err = O.rel_err(y[:, lo:hi], ref[:, lo:hi])
        print(f"[parity] columns {lo}-{hi} rel_err={err:.3e}", flush=True)
        assert err <= tol, (lo, hi, err)


def _min_workspace(lib, arr, n, M, K, x, x_dtype, ws, stream):
    """Smallest workspace the call accepts (a smaller one is refused before any launch)."""
    import littlebit_amd._lib as L
    lo, hi = 1, ws.numel()
    while lo < hi:
        mid = (lo + hi) // 2
        if lib.lbk_group_forward_ex(arr, n, M, K, x, x_dtype, None, L.LBK_F32, ws.data_ptr(), mid, stream) == 0:
            hi = mid
        else:
            lo = mid + 1
    return lo


@pytest.mark.parametrize("M,K,specs,x_dtype", [
    (100, 4096, [(4096, [204, 1843]), (1024, [81, 737])], torch.bfloat16),  # 4 parts per tile
    (2048, 4096, [(4096, [204, 1843])], torch.bfloat16),                    # 512 blocks, 8 XCD groups
    (300, 14336, [(4096, [318, 2867])], torch.bfloat16),
    (129, 4096, [(1024, [130, 7])], torch.float32),                         # hi/lo planes, scaled copy
])
def test_stream_k_matches_whole_tiles(gpu, M, K, specs, x_dtype):
    """Stage 1 of the GEMM path shares its (tile, k-step) iterations over
    resident blocks when whole tiles would leave CUs idle (stream-K, partial
    tiles summed by the part that completes them); given a workspace without
    room for the partial tiles the same call runs whole tiles.  The partial
    sums meet in another order, so the forms agree to fp32 rounding with fp32
    activations (T kept as hi/lo bf16 planes, ~2**-17), and to 1e-3 with bf16
    ones (T rounded to bf16: an ulp of fp32 can move a T element by 2**-8);
    twice in a row (the tile counters are left at zero), each form bit for
    bit the same both times (the completing part sums the parts in block
    order); both match the oracle."""
    import ctypes
    import littlebit_amd._lib as L
    from littlebit_amd import LittleBitProjection
    lib = L.load()
    rng = np.random.Generator(np.random.PCG64(7700 + M))
    from littlebit_amd.synthetic import make_branch
    host = [[make_branch(rng, K, R, N, direct_words=True) for R in ranks] for N, ranks in specs]
    projs = [LittleBitProjection([_dev_branch(b.as_dict(), gpu) for b in brs]) for brs in host]
    x = rng.standard_normal((M, K)).astype(np.float32)
    tx = torch.from_numpy(x).to(gpu).to(x_dtype)
    xu = tx.float().cpu().numpy()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    dt = L.LBK_BF16 if x_dtype == torch.bfloat16 else L.LBK_F32
    results = []
    for form in ("whole", "stream-k", "whole", "stream-k"):
        outs = [torch.full((M, N), float("nan"), device=gpu) for N, _ in specs]
        arr = (L.LbkProjection * len(projs))()
        for i, (p, o) in enumerate(zip(projs, outs)):
            arr[i].branches = ctypes.cast(p._arr, ctypes.POINTER(L.LbkBranch))
            arr[i].n_branches = len(p.branches)
            arr[i].out_features = p.out_features
            arr[i].bias = None
            arr[i].y = o.data_ptr()
            arr[i].residual = None
        full = lib.lbk_group_workspace_bytes(arr, len(projs), M, K)
        ws = torch.zeros(full, dtype=torch.uint8, device=gpu)
        n = full if form == "stream-k" else _min_workspace(lib, arr, len(projs), M, K, tx.data_ptr(), dt, ws, stream)
        print(f"[stream-k] M={M} K={K} {form}: workspace {n} of {full}", flush=True)
        L.check(lib.lbk_group_forward_ex(arr, len(projs), M, K, tx.data_ptr(), dt, None, L.LBK_F32, ws.data_ptr(), n,
                                         stream), "lbk_group_forward_ex")
        torch.cuda.synchronize()
        results.append([o.cpu().numpy() for o in outs])
    assert full > _min_workspace(lib, arr, len(projs), M, K, tx.data_ptr(), dt, ws, stream), "no stream-K form"
    for a, b in zip(results[0] + results[1], results[2] + results[3]):
        assert np.array_equal(a, b), "a GEMM-path form changed between two identical calls"
    agree = 1e-3 if x_dtype == torch.bfloat16 else 1e-5
    for r in results[1:]:
        for a, b in zip(results[0], r):
            err = O.rel_err(b, a)
            print(f"[stream-k] forms differ by {err:.2e}", flush=True)
            assert err <= agree
    tol = TOL_BF16_PREFILL if x_dtype == torch.bfloat16 else TOL_F32
    rows = np.unique(np.r_[0:min(M, 48), max(0, M - 48):M])  # rows are independent: a sample pins the call
    for (N, _), brs, y in zip(specs, host, results[1]):
        _check(y[rows], xu[rows], [b.as_dict() for b in brs], K, N, tol, what=f"stream-K M={M} K={K} N={N}")


@pytest.mark.parametrize("M,K,N,ranks", [(65, 4096, 4096, [205, 1843]), (96, 11008, 4096, [298, 2686]),
                                         (129, 1000, 300, [130]), (8, 4096, 4096, [4000, 4000])])
def test_gemm_path_fp32(gpu, M, K, N, ranks):
    """fp32 activations at M > 64 or with operands too large for the decode
    kernels' LDS at any chunk of rows: hi/lo-split GEMM path, fp32 tolerance."""
    x, brs = _synthetic(1020 + M, M, K, N, ranks)
    y, xu = _run(gpu, x, brs)
    _check(y, xu, brs, K, N, TOL_F32, what=f"fp32 gemm M={M} K={K} N={N} R={ranks}")


@pytest.mark.parametrize("M,K,N,ranks", [(32, 4096, 4096, [205, 1843]), (17, 4096, 11008, [298, 2686]),
                                         (64, 11008, 4096, [298, 2686]), (33, 70, 45, [37, 5]),
                                         (12, 4096, 11008, [298, 2686]), (41, 96, 130, [3])])
def test_chunked_rows_fp32(gpu, M, K, N, ranks):
    """17 <= M <= 64 (tree verify), and M <= 16 whose t does not fit the
    decode kernels' LDS at once: decode-path calls over chunks of 16 or 8
    rows, fp32 tolerance."""
    x, brs = _synthetic(1020 + M, M, K, N, ranks)
    y, xu = _run(gpu, x, brs)
    _check(y, xu, brs, K, N, TOL_F32, what=f"fp32 chunked M={M} K={K} N={N} R={ranks}")


def test_empty_batch(gpu):
    from littlebit_amd import LittleBitProjection
    _, brs = _synthetic(3, 1, 64, 48, [8])
    proj = LittleBitProjection([_dev_branch(b, gpu) for b in brs])
    y = proj.forward(torch.empty((0, 64), device=gpu))
    assert tuple(y.shape) == (0, 48)


def test_leading_dims_preserved(gpu):
    from littlebit_amd import LittleBitProjection
    K, N = 128, 96
    x, brs = _synthetic(4, 6, K, N, [16])
    proj = LittleBitProjection([_dev_branch(b, gpu) for b in brs])
    y = proj.forward(torch.from_numpy(x).to(gpu).reshape(2, 3, K))
    assert tuple(y.shape) == (2, 3, N)
    _check(y.reshape(6, N).cpu().numpy(), x, brs, K, N, TOL_F32, what="leading dims")


def test_repeatable(gpu):
    """Repeated calls agree to 1e-5: the k-chunk partial sums are added with
    atomics, so their order, and with it the last bits of t and the bf16
    hi/lo split of t (relative 2**-17), may change."""
    K = N = 4096
    x, brs = _synthetic(1007, 8, K, N, [205, 1843])
    y1, xu = _run(gpu, x, brs)
    for _ in range(3):
        y2, _ = _run(gpu, x, brs)
        assert O.rel_err(y2, y1) <= 1e-5
    _check(y2, xu, brs, K, N, TOL_F32, what="repeat")


def test_shape_changes_between_calls(gpu):
    """One workspace serves projections of different shapes in any order; the
    latent buffer it keeps zero between calls must stay zero."""
    cases = [(1, 4096, 4096, [205, 1843]), (8, 4096, 11008, [298, 2686]), (3, 70, 45, [37]),
             (16, 11008, 4096, [298]), (1, 4096, 4096, [205, 1843]), (300, 96, 64, [9])]
    for i, (M, K, N, ranks) in enumerate(cases * 2):
        x, brs = _synthetic(2000 + i, M, K, N, ranks)
        y, xu = _run(gpu, x, brs)
        _check(y, xu, brs, K, N, TOL_F32, what=f"interleaved #{i} M={M} K={K} N={N} R={ranks}")


def test_graph_replay_matches_eager(gpu):
    from littlebit_amd import LittleBitProjection
    K = N = 4096
    x, brs = _synthetic(1008, 4, K, N, [205, 1843])
    proj = LittleBitProjection([_dev_branch(b, gpu) for b in brs])
    tx = torch.from_numpy(x).to(gpu)
    eager = proj.forward(tx).clone()
    out = torch.empty_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        proj.forward(tx, out=out)  # sizes the per-stream workspace before capture
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        proj.forward(tx, out=out)
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        # split-K partial sums are added with atomics: equal up to their order
        assert O.rel_err(out.cpu().numpy(), eager.cpu().numpy()) <= 1e-5, f"replay {i}"
        tx.mul_(1.0)  # eager work between replays
        torch.cuda.synchronize()


# --------------------------------------------------------------------------- projection groups
def _run_group(dev, x, projs, x_dtype=torch.float32, out_dtype=None):
    """projs: list of (branches, bias or None); one lbk_group_forward call."""
    from littlebit_amd import LittleBitProjection, LittleBitProjectionGroup
    group = LittleBitProjectionGroup([
        LittleBitProjection([_dev_branch(b, dev) for b in brs], None if bias is None else torch.from_numpy(bias).to(dev))
        for brs, bias in projs])
    tx = torch.from_numpy(np.asarray(x, np.float32)).to(dev).to(x_dtype)
    ys = group.forward(tx, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return [y.float().cpu().numpy() for y in ys], tx.float().cpu().numpy()


def _group_case(seed, M, K, specs, bias=False):
    """specs: [(N, ranks)]; x shared, each projection its own seeded factors."""
    from littlebit_amd.synthetic import make_projection
    x = None
    projs = []
    for i, (N, ranks) in enumerate(specs):
        xi, brs = make_projection(seed + 17 * i, M, K, N, ranks)
        x = xi if x is None else x
        b = (np.random.Generator(np.random.PCG64(seed + i)).standard_normal(N).astype(np.float32)
             if bias else None)
        projs.append(([br.as_dict() for br in brs], b))
    return x, projs


@pytest.mark.parametrize("what,M,K,specs", [
    ("qkv draft", 1, 4096, [(4096, [205])] * 3),
    ("qkv target", 8, 4096, [(4096, [205, 1843])] * 3),
    ("gate/up target", 8, 4096, [(11008, [298, 2686])] * 2),
    ("gate/up draft", 1, 4096, [(11008, [298])] * 2),
    ("llama3 q/k/v gqa", 4, 4096, [(4096, [204, 1843]), (1024, [81, 737]), (1024, [81, 737])]),
    ("ragged four", 3, 70, [(45, [37]), (77, [64, 95]), (31, [31, 1]), (5, [3])]),
    ("tree M=16", 16, 4096, [(4096, [205, 1843])] * 3),
    ("general path M=20", 20, 4096, [(4096, [205]), (1024, [81, 9])]),
])
def test_group_matches_oracle(gpu, what, M, K, specs):
    x, projs = _group_case(3000 + M, M, K, specs)
    ys, xu = _run_group(gpu, x, projs)
    for i, ((brs, _), y) in enumerate(zip(projs, ys)):
        _check(y, xu, brs, K, specs[i][0], TOL_F32, what=f"{what} proj {i}")


def test_group_bias_bf16(gpu):
    K = 512
    specs = [(300, [45, 301]), (512, [64])]
    x, projs = _group_case(3100, 2, K, specs, bias=True)
    ys, xu = _run_group(gpu, x, projs, x_dtype=torch.bfloat16, out_dtype=torch.bfloat16)
    for i, ((brs, b), y) in enumerate(zip(projs, ys)):
        _check(y, xu, brs, K, specs[i][0], TOL_BF16_OUT, bias=b, what=f"bias bf16 proj {i}")


def test_group_equals_single_calls(gpu):
    """A group's outputs equal the projections' separate forwards."""
    from littlebit_amd import LittleBitProjection, LittleBitProjectionGroup
    K = 4096
    x, projs = _group_case(3200, 8, K, [(4096, [205, 1843]), (4096, [205]), (1024, [81])])
    ps = [LittleBitProjection([_dev_branch(b, gpu) for b in brs]) for brs, _ in projs]
    tx = torch.from_numpy(x).to(gpu)
    ys = LittleBitProjectionGroup(ps).forward(tx)
    for i, p in enumerate(ps):
        y1 = p.forward(tx)
        torch.cuda.synchronize()
        assert O.rel_err(ys[i].cpu().numpy(), y1.cpu().numpy()) <= 1e-5, f"proj {i}"


def test_group_graph_replay_interleaved(gpu):
    """Groups and single projections captured in one graph, replayed with
    eager work in between; every replay matches the eager outputs."""
    from littlebit_amd import LittleBitProjection, LittleBitProjectionGroup
    K = 4096
    x, projs = _group_case(3300, 1, K, [(4096, [205])] * 3)
    ps = [LittleBitProjection([_dev_branch(b, gpu) for b in brs]) for brs, _ in projs]
    grp = LittleBitProjectionGroup(ps)
    tx = torch.from_numpy(x).to(gpu)
    outs = [torch.empty((1, 4096), device=gpu) for _ in range(3)]
    single = torch.empty((1, 4096), device=gpu)

    def step():
        grp.forward(tx, outs=outs)
        ps[0].forward(outs[2], out=single)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    s.synchronize()
    eager = [o.clone() for o in outs] + [single.clone()]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    for rep in range(4):
        for o in outs + [single]:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs + [single], eager)):
            assert O.rel_err(o.cpu().numpy(), e.cpu().numpy()) <= 1e-5, f"replay {rep} output {i}"
        ps[1].forward(tx)  # eager call on another stream's workspace in between
        torch.cuda.synchronize()


# --------------------------------------------------------------------------- module / op boundary
def test_module_forward_matches_oracle(gpu):
    from littlebit_amd import LittleBitLinear
    K, N = 4096, 4096
    x, brs = _synthetic(1009, 8, K, N, [205, 1843])
    branches = [{"u_packed": torch.from_numpy(b["u_sign"]), "v_packed": torch.from_numpy(b["v_sign"]),
                 "u1": torch.from_numpy(b["h"]).reshape(1, N), "v2": torch.from_numpy(b["g"]).reshape(1, K),
                 "mid": torch.from_numpy(b["l"]).reshape(1, -1)} for b in brs]
    m = LittleBitLinear.from_packed(K, N, branches, device=gpu)
    y = m(torch.from_numpy(x).to(gpu).reshape(2, 4, K))
    assert tuple(y.shape) == (2, 4, N) and y.dtype == torch.float32
    _check(y.reshape(8, N).cpu().numpy(), x, brs, K, N, TOL_F32, what="LittleBitLinear module")


def test_op_littlebit_linear_matches_oracle(gpu):
    from littlebit_amd import littlebit_linear
    K, N, R = 4096, 4096, 205
    x, brs = _synthetic(1010, 2, K, N, [R])
    b = brs[0]
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    y = littlebit_linear(d(x), d(b["g"]).reshape(1, K), d(b["v_sign"]), K, d(b["l"]).reshape(1, R),
                         d(b["u_sign"]), R, d(b["h"]).reshape(1, N))
    _check(y.cpu().numpy(), x, brs, K, N, TOL_F32, what="littlebit_linear op")


def test_op_precondition_errors(gpu):
    from littlebit_amd import littlebit_linear
    K, N, R = 64, 32, 8
    x, brs = _synthetic(1011, 1, K, N, [R])
    b = brs[0]
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    args = [d(x), d(b["g"]).reshape(1, K), d(b["v_sign"]), K, d(b["l"]).reshape(1, R), d(b["u_sign"]), R,
            d(b["h"]).reshape(1, N)]
    bad_k = list(args)
    bad_k[3] = K + 1
    with pytest.raises(RuntimeError, match="v_cols"):
        littlebit_linear(*bad_k)
    bad_dtype = list(args)
    bad_dtype[2] = bad_dtype[2].to(torch.int64)
    with pytest.raises(RuntimeError, match="int32"):
        littlebit_linear(*bad_dtype)
    cpu_in = list(args)
    cpu_in[0] = cpu_in[0].cpu()
    with pytest.raises(RuntimeError, match="GPU"):
        littlebit_linear(*cpu_in)


# --------------------------------------------------------------------------- fused inputs / residual
def _fused_run(gpu, M, K, specs, mode, x_dtype=torch.float32, residual=False, seed=3400):
    from littlebit_amd import LittleBitProjection, LittleBitProjectionGroup
    x, projs = _group_case(seed + M, M, K, specs)
    rng = np.random.Generator(np.random.PCG64(seed))
    group = LittleBitProjectionGroup([LittleBitProjection([_dev_branch(b, gpu) for b in brs]) for brs, _ in projs])
    tx = torch.from_numpy(x).to(gpu).to(x_dtype)
    kw = {}
    if mode == "rms":
        w = (1 + 0.2 * rng.standard_normal(K)).astype(np.float32)
        kw = {"rms_weight": torch.from_numpy(w).to(gpu), "rms_eps": 1e-5}
        xin = O.rms_norm(tx.float().cpu().numpy(), w, 1e-5)
    else:
        u = rng.standard_normal((M, K)).astype(np.float32)
        tu = torch.from_numpy(u).to(gpu).to(x_dtype)
        kw = {"x_up": tu}
        xin = O.silu_mul(tx.float().cpu().numpy(), tu.float().cpu().numpy())
    outs = res_np = None
    if residual:
        res_np = [rng.standard_normal((M, N)).astype(np.float32) * 50 for N, _ in specs]
        outs = [torch.from_numpy(r).to(gpu) for r in res_np]
        kw["residuals"] = outs  # in place: y aliases the residual
    ys = group.forward(tx, outs=outs, out_dtype=torch.float32, **kw)
    torch.cuda.synchronize()
    tol = TOL_BF16_PREFILL if (x_dtype == torch.bfloat16 and M > 16) else TOL_F32
    for i, ((brs, _), y) in enumerate(zip(projs, ys)):
        ref = O.littlebit_forward(xin, brs, K, specs[i][0])
        if residual:
            ref = ref + res_np[i]
        err = O.rel_err(y.cpu().numpy(), ref)
        print(f"[fused] {mode} M={M} proj {i} rel_err={err:.2e}", flush=True)
        assert err <= tol, (mode, M, i, err)


@pytest.mark.parametrize("M", [1, 8, 16, 40])
def test_fused_rmsnorm_group(gpu, M):
    _fused_run(gpu, M, 4096, [(4096, [205, 1843]), (1024, [81])], "rms")


@pytest.mark.parametrize("M,x_dtype", [(1, torch.float32), (8, torch.float32), (40, torch.float32),
                                       (3, torch.bfloat16), (200, torch.bfloat16)])
def test_fused_silu_mul(gpu, M, x_dtype):
    _fused_run(gpu, M, 1000, [(300, [64, 130])], "silu", x_dtype=x_dtype)


@pytest.mark.parametrize("M", [1, 8, 33])
def test_residual_in_place(gpu, M):
    _fused_run(gpu, M, 512, [(512, [45, 301]), (96, [9])], "rms", residual=True)
    _fused_run(gpu, M, 1000, [(4096, [298])], "silu", residual=True)


# --------------------------------------------------------------------------- attention partials as input
@pytest.mark.parametrize("heads,kvh,hd,max_seq,pos,ranks,device_pos", [
    (32, 32, 128, 600, 513, [205], True), (32, 32, 128, 600, 513, [205, 1843], False),
    (16, 4, 64, 100, 15, [64], True), (16, 4, 64, 100, 16, [31, 97], True),
    (16, 16, 128, 2048, 1500, [300], True), (4, 2, 64, 40, 39, [16], False)])
def test_attention_merge_input(gpu, heads, kvh, hd, max_seq, pos, ranks, device_pos):
    """lbk_attention_decode without an output, then a projection reading its
    partials (LBK_INPUT_ATTN_MERGE) with a residual: the oracle's projection
    of the float64 attention output, plus the residual; a position past the
    cache leaves y = residual (the attention reads as zeros)."""
    import littlebit_amd._lib as L
    from littlebit_amd import LittleBitProjection
    from littlebit_amd.ops import AttentionPartials
    K, N = heads * hd, 384
    x_unused, brs = _synthetic(4100 + pos, 1, K, N, ranks)
    proj = LittleBitProjection([_dev_branch(b, gpu) for b in brs])
    g = torch.Generator(device="cpu").manual_seed(pos * 7 + heads)
    kc = torch.randn((kvh, max_seq, hd), generator=g).to(gpu)
    vc = torch.randn((kvh, max_seq, hd), generator=g).to(gpu)
    q = torch.randn((heads * hd,), generator=g).to(gpu)
    k = torch.randn((kvh * hd,), generator=g).to(gpu)
    v = torch.randn((kvh * hd,), generator=g).to(gpu)
    res = (torch.randn((1, N), generator=g) * 3).to(gpu)
    scale = hd ** -0.5
    K_ = kc.clone().double().cpu()
    V_ = vc.clone().double().cpu()
    K_[:, pos] = k.view(kvh, hd).double().cpu()
    V_[:, pos] = v.view(kvh, hd).double().cpu()
    rep = heads // kvh
    s = torch.einsum("grd,gtd->grt", q.view(kvh, rep, hd).double().cpu(), K_[:, :pos + 1]) * scale
    a_ref = torch.einsum("grt,gtd->grd", torch.softmax(s, dim=-1), V_[:, :pos + 1]).reshape(1, K).numpy()
    ref = O.littlebit_forward(a_ref, brs, K, N) + res.double().cpu().numpy()
    lib = L.load()
    part = torch.empty(lib.lbk_attention_partial_bytes(heads, max_seq, hd) // 4 + 4, device=gpu)
    for at in ([pos, max_seq] if device_pos else [pos]):
        pos_t = torch.tensor([at], dtype=torch.int64, device=gpu)
        print(f"[attn_merge] heads={heads} hd={hd} max_seq={max_seq} pos={at} ranks={ranks} dev={device_pos}",
              flush=True)
        rc = lib.lbk_attention_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), heads,
                                      kvh, hd, max_seq, pos_t.data_ptr() if device_pos else None,
                                      0 if device_pos else at, scale, part.data_ptr(), part.numel() * 4, None, None)
        L.check(rc, "lbk_attention_decode")
        y = res.clone()
        proj.forward(None, out=y, residual=y, attn=AttentionPartials(part, hd, max_seq, pos_t if device_pos else None,
                                                                     0 if device_pos else at))
        torch.cuda.synchronize()
        if at < max_seq:
            err = O.rel_err(y.cpu().numpy(), ref)
            print(f"[attn_merge] rel_err={err:.2e}", flush=True)
            assert err <= TOL_F32
            assert torch.equal(kc[:, at], k.view(kvh, hd))
        else:
            assert torch.equal(y, res)


def test_attention_merge_input_errors(gpu):
    import littlebit_amd._lib as L
    from littlebit_amd import LittleBitProjection
    from littlebit_amd.ops import AttentionPartials
    _, brs = _synthetic(11, 1, 512, 64, [16])
    proj = LittleBitProjection([_dev_branch(b, gpu) for b in brs])
    part = torch.zeros(1 << 16, device=gpu)
    with pytest.raises(RuntimeError, match="head_dim"):
        proj.forward(None, attn=AttentionPartials(part, 96, 64, None, 3))
    odd = LittleBitProjection([_dev_branch(b, gpu) for b in _synthetic(12, 1, 448, 64, [16])[1]])
    with pytest.raises(RuntimeError, match="heads"):  # K = 448 is no multiple of 128
        odd.forward(None, attn=AttentionPartials(part, 128, 64, None, 3))
    with pytest.raises(RuntimeError, match="aligned"):
        proj.forward(None, attn=AttentionPartials(part[1:], 64, 64, None, 3))

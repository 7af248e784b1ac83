"""The C ABI: the built library loads and exports every function that
include/*.h declares, with the binding's argument lists in step.  No GPU work
is issued: the error paths checked here return before any HIP call."""
import ctypes
import re

import pytest

from tests.conftest import ROOT

HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(lbk_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_entry_points():
    names = declared_functions()
    assert {"lbk_linear_forward", "lbk_littlebit_linear", "lbk_unpack_signs", "lbk_pack_signs",
            "lbk_abi_version", "lbk_last_error", "lbk_linear_workspace_bytes"} <= names


def test_library_exports_every_declared_symbol():
    import littlebit_amd._lib as L
    lib = L.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"


def test_binding_covers_header_exactly():
    import littlebit_amd._lib as L
    assert set(L.SIGNATURES) == declared_functions()


def test_abi_version_matches_header():
    import littlebit_amd._lib as L
    text = (ROOT / "include" / "littlebit_amd.h").read_text()
    ver = int(re.search(r"#define LBK_ABI_VERSION (\d+)", text).group(1))
    assert L.load().lbk_abi_version() == ver


def test_constants_match_header():
    import littlebit_amd._lib as L
    text = (ROOT / "include" / "littlebit_amd.h").read_text()
    for name in ("LBK_F32", "LBK_BF16", "LBK_OK"):
        assert int(re.search(rf"#define {name} (\d+)", text).group(1)) == getattr(L, name)
    for name in ("LBK_ERR_ARG", "LBK_ERR_DTYPE", "LBK_ERR_WORKSPACE", "LBK_ERR_HIP"):
        assert int(re.search(rf"#define {name} \((-\d+)\)", text).group(1)) == getattr(L, name)


def test_struct_layout():
    import littlebit_amd._lib as L
    assert ctypes.sizeof(L.LbkBranch) == 7 * 8
    assert L.LbkBranch.rank.offset == 40
    assert L.LbkBranch.v_sign_tiled.offset == 48


def _branch(rank=8):
    import littlebit_amd._lib as L
    b = (L.LbkBranch * 2)()
    for i in range(2):
        b[i].v_sign = b[i].u_sign = b[i].v2 = b[i].mid = b[i].u1 = 0x1000
        b[i].rank = rank
    return b


def test_validation_errors_without_gpu_work():
    import littlebit_amd._lib as L
    lib = L.load()
    br = _branch()
    fwd = lib.lbk_linear_forward
    # bad branch count
    assert fwd(br, 3, 1, 64, 64, 0x1000, L.LBK_F32, None, 0x1000, L.LBK_F32, 0x1000, 1 << 20, None) == L.LBK_ERR_ARG
    assert "n_branches" in L.last_error()
    # bad K
    assert fwd(br, 1, 1, 0, 64, 0x1000, L.LBK_F32, None, 0x1000, L.LBK_F32, 0x1000, 1 << 20, None) == L.LBK_ERR_ARG
    # bad dtype
    assert fwd(br, 1, 1, 64, 64, 0x1000, 7, None, 0x1000, L.LBK_F32, 0x1000, 1 << 20, None) == L.LBK_ERR_DTYPE
    # workspace too small
    assert fwd(br, 2, 4, 64, 64, 0x1000, L.LBK_F32, None, 0x1000, L.LBK_F32, 0x1000, 16, None) == L.LBK_ERR_WORKSPACE
    assert "workspace" in L.last_error()
    # null factor pointer
    br[0].u_sign = 0
    assert fwd(br, 1, 1, 64, 64, 0x1000, L.LBK_F32, None, 0x1000, L.LBK_F32, 0x1000, 1 << 20, None) == L.LBK_ERR_ARG
    # M == 0 is a no-op success
    br[0].u_sign = 0x1000
    assert fwd(br, 1, 0, 64, 64, None, L.LBK_F32, None, None, L.LBK_F32, None, 0, None) == L.LBK_OK


def test_workspace_query():
    import littlebit_amd._lib as L
    lib = L.load()
    br = _branch(rank=100)
    n1 = lib.lbk_linear_workspace_bytes(br, 1, 8, 4096, 4096)
    n2 = lib.lbk_linear_workspace_bytes(br, 2, 8, 4096, 4096)
    big = lib.lbk_linear_workspace_bytes(br, 2, 4096, 4096, 4096)
    assert 0 < n1 <= n2 < big
    assert lib.lbk_linear_workspace_bytes(br, 5, 8, 4096, 4096) == 0


def _group(n, rank=8, N=64):
    import littlebit_amd._lib as L
    brs = [_branch(rank) for _ in range(n)]
    arr = (L.LbkProjection * max(n, 1))()
    for i in range(n):
        arr[i].branches = ctypes.cast(brs[i], ctypes.POINTER(L.LbkBranch))
        arr[i].n_branches = 2
        arr[i].out_features = N
        arr[i].y = 0x1000
    return arr, brs


def test_group_struct_layout():
    import littlebit_amd._lib as L
    assert ctypes.sizeof(L.LbkProjection) == 48
    assert L.LbkProjection.out_features.offset == 16 and L.LbkProjection.y.offset == 32
    assert L.LbkProjection.residual.offset == 40
    assert ctypes.sizeof(L.LbkInput) == 56
    assert (L.LbkInput.rms_weight.offset, L.LbkInput.rms_eps.offset, L.LbkInput.x1.offset) == (8, 16, 24)
    assert (L.LbkInput.head_dim.offset, L.LbkInput.max_seq.offset, L.LbkInput.pos_device.offset,
            L.LbkInput.pos.offset) == (32, 36, 40, 48)


def test_input_kind_validation():
    import littlebit_amd._lib as L
    lib = L.load()
    arr, keep = _group(2)
    fx = lib.lbk_group_forward_ex
    bad = L.LbkInput(7, None, 0.0, None)
    assert fx(arr, 2, 1, 64, 0x1000, L.LBK_F32, ctypes.byref(bad), L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    assert "input kind" in L.last_error()
    rms = L.LbkInput(L.LBK_INPUT_RMSNORM, None, 1e-6, None)
    assert fx(arr, 2, 1, 64, 0x1000, L.LBK_F32, ctypes.byref(rms), L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    assert "rms_weight" in L.last_error()
    silu = L.LbkInput(L.LBK_INPUT_SILU_MUL, None, 0.0, None)
    assert fx(arr, 2, 1, 64, 0x1000, L.LBK_F32, ctypes.byref(silu), L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    assert "x1" in L.last_error()
    # attention partials: one row, fp32, K a multiple of head_dim 64 / 128, aligned
    att = L.LbkInput(L.LBK_INPUT_ATTN_MERGE, None, 0.0, None, 64, 128, None, 5)
    assert fx(arr, 2, 2, 64, 0x1000, L.LBK_F32, ctypes.byref(att), L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    assert "M == 1" in L.last_error()
    assert fx(arr, 2, 1, 64, 0x1000, L.LBK_BF16, ctypes.byref(att), L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_DTYPE
    assert fx(arr, 2, 1, 64, 0x1008, L.LBK_F32, ctypes.byref(att), L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    assert "aligned" in L.last_error()
    att.head_dim = 128
    assert fx(arr, 2, 1, 64, 0x1000, L.LBK_F32, ctypes.byref(att), L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    assert "heads * head_dim" in L.last_error()
    att.head_dim, att.max_seq = 64, 0
    assert fx(arr, 2, 1, 64, 0x1000, L.LBK_F32, ctypes.byref(att), L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    assert "max_seq" in L.last_error()


def test_group_validation_errors():
    import littlebit_amd._lib as L
    lib = L.load()
    arr, keep = _group(4)
    fwd = lib.lbk_group_forward
    assert fwd(arr, 0, 1, 64, 0x1000, L.LBK_F32, L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    assert "n_proj" in L.last_error()
    assert fwd(arr, 5, 1, 64, 0x1000, L.LBK_F32, L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    arr[2].y = None
    assert fwd(arr, 4, 1, 64, 0x1000, L.LBK_F32, L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    assert "projection 2" in L.last_error()
    arr[2].y = 0x1000
    arr[1].n_branches = 3
    assert fwd(arr, 4, 1, 64, 0x1000, L.LBK_F32, L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    assert "projection 1" in L.last_error()
    arr[1].n_branches = 2
    assert fwd(arr, 4, 1, 64, 0x1000, 9, L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_DTYPE
    assert fwd(arr, 4, 1, 64, 0x1000, L.LBK_F32, L.LBK_F32, 0x1000, 16, None) == L.LBK_ERR_WORKSPACE
    # total rank over the group is bounded
    big, keep2 = _group(3, rank=3000)
    assert fwd(big, 3, 1, 64, 0x1000, L.LBK_F32, L.LBK_F32, 0x1000, 1 << 24, None) == L.LBK_ERR_ARG
    assert "ranks" in L.last_error()
    assert fwd(arr, 4, 0, 64, None, L.LBK_F32, L.LBK_F32, None, 0, None) == L.LBK_OK


def test_group_workspace_query():
    import littlebit_amd._lib as L
    lib = L.load()
    arr, keep = _group(3, rank=205, N=4096)
    br = _branch(rank=205)
    one = lib.lbk_linear_workspace_bytes(br, 2, 8, 4096, 4096)
    grp = lib.lbk_group_workspace_bytes(arr, 3, 8, 4096)
    assert 0 < one <= grp
    # up to 64 rows: decode-path calls over chunks of rows, the same workspace
    assert lib.lbk_group_workspace_bytes(arr, 3, 33, 4096) == grp
    assert lib.lbk_group_workspace_bytes(arr, 3, 64, 4096) == grp
    assert lib.lbk_group_workspace_bytes(arr, 3, 65, 4096) > grp  # GEMM path: per-call planes
    assert lib.lbk_group_workspace_bytes(arr, 0, 8, 4096) == 0
    # M = 0 plans no tiles (the stream-K sizing once divided by its zero block count)
    assert lib.lbk_group_workspace_bytes(arr, 3, 0, 4096) > 0
    assert lib.lbk_linear_workspace_bytes(br, 2, 0, 4096, 4096) > 0


def test_deterministic_mode_switch_and_workspace():
    import littlebit_amd._lib as L
    lib = L.load()
    arr, keep = _group(1, rank=205, N=4096)
    prev = lib.lbk_set_deterministic(0)
    try:
        off = lib.lbk_group_workspace_bytes(arr, 1, 8, 4096)
        assert lib.lbk_set_deterministic(1) == 0
        assert lib.lbk_set_deterministic(1) == 1
        on = lib.lbk_group_workspace_bytes(arr, 1, 8, 4096)
        assert on > off  # the k-chunk partials
        assert lib.lbk_group_workspace_bytes(arr, 1, 1000, 4096) > 0
        assert lib.lbk_set_deterministic(0) == 1
        assert lib.lbk_group_workspace_bytes(arr, 1, 8, 4096) == off
    finally:
        lib.lbk_set_deterministic(prev)


def test_pack_unpack_argument_errors():
    import littlebit_amd._lib as L
    lib = L.load()
    assert lib.lbk_unpack_signs(None, -1, 4, None, None) == L.LBK_ERR_ARG
    assert lib.lbk_pack_signs(None, 2, -4, None, None) == L.LBK_ERR_ARG
    assert lib.lbk_unpack_signs(None, 0, 4, None, None) == L.LBK_OK  # empty: nothing to do
    assert lib.lbk_repack_signs_to_i2(None, 2, 2, -1, None, None) == L.LBK_ERR_ARG
    assert lib.lbk_repack_signs_to_i2(None, 2, 2, 65, None, None) == L.LBK_ERR_ARG  # 65 columns need 3 words
    assert "3 sign words" in L.last_error()
    assert lib.lbk_repack_signs_to_i2(None, 2, 3, 65, None, None) == L.LBK_ERR_ARG  # NULL pointers
    assert lib.lbk_repack_signs_to_i2(None, 0, 3, 65, None, None) == L.LBK_OK  # no rows
    assert lib.lbk_repack_signs_to_i2(None, 4, 0, 0, None, None) == L.LBK_OK  # no columns


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    import littlebit_amd._lib as L
    monkeypatch.setattr(L, "_lib", None)
    monkeypatch.setattr(L, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(L.LittleBitLibraryMissing):
        L.load()


def test_q4_head_argument_errors():
    import littlebit_amd._lib as L
    lib = L.load()
    assert lib.lbk_q4_0_quantize(0x1000, 2, 33, 0x1000, 0x1000, None) == L.LBK_ERR_ARG  # cols % 32
    assert lib.lbk_q4_0_quantize(0x1004, 2, 32, 0x1000, 0x1000, None) == L.LBK_ERR_ARG  # alignment
    assert "aligned" in L.last_error()
    assert lib.lbk_q4_0_quantize(None, 0, 32, None, None, None) == L.LBK_OK  # nothing to do
    assert lib.lbk_lm_head_q4_workspace_bytes(0, 4096) == 0
    need = lib.lbk_lm_head_q4_workspace_bytes(32000, 4096)
    assert need >= 500 * 8  # one argmax key per block of 64 rows
    fx = lib.lbk_lm_head_q4_argmax
    assert fx(0x1000, 0x1000, 100, 48, 0x1000, None, 0.0, None, 0x1000, 0x1000, 1 << 20, None) == L.LBK_ERR_ARG
    assert "multiple of 32" in L.last_error()
    assert fx(0x1000, 0x1000, 100, 32768, 0x1000, None, 0.0, None, 0x1000, 0x1000, 1 << 20, None) == L.LBK_ERR_ARG
    assert fx(0x1000, 0x1000, 0, 64, 0x1000, None, 0.0, None, 0x1000, 0x1000, 1 << 20, None) == L.LBK_ERR_ARG
    assert fx(0x1008, 0x1000, 100, 64, 0x1000, None, 0.0, None, 0x1000, 0x1000, 1 << 20, None) == L.LBK_ERR_ARG
    assert fx(0x1000, 0x1000, 100, 64, 0x1000, 0x1000, -1.0, None, 0x1000, 0x1000, 1 << 20, None) == L.LBK_ERR_ARG
    assert fx(0x1000, 0x1000, 32000, 4096, 0x1000, None, 0.0, None, 0x1000, 0x1000, 8, None) == L.LBK_ERR_WORKSPACE
    assert fx(0x1000, 0x1000, 100, 64, None, None, 0.0, None, 0x1000, 0x1000, 1 << 20, None) == L.LBK_ERR_ARG
    assert fx(0x1000, 0x1000, 100, 64, 0x1004, None, 0.0, None, 0x1000, 0x1000, 1 << 20, None) == L.LBK_ERR_ARG
    assert fx(0x1000, 0x1000, 100, 64, 0x1000, 0x1008, 0.0, None, 0x1000, 0x1000, 1 << 20, None) == L.LBK_ERR_ARG


def test_output_overlapping_later_chunks_is_refused():
    """Rows that run as row chunks one after another (48 rows of three
    target-shaped projections: their latent vectors do not fit at once): an
    output over the input rows of the next chunk (projection 0, one chunk
    down) is safe only last to first, one over the previous chunk's rows
    (projection 1, one chunk up) only first to last; with both in one call no
    order is safe and the call is refused before any launch."""
    import littlebit_amd._lib as L
    lib = L.load()
    K, N, M = 4096, 2048, 48          # fp32 y rows of N = bf16 x rows of K: 8 KiB each
    brs = [(L.LbkBranch * 2)() for _ in range(3)]
    for b in brs:
        for i, r in enumerate((205, 1843)):
            b[i].v_sign = b[i].u_sign = b[i].v2 = b[i].mid = b[i].u1 = 0x1000
            b[i].rank = r
    arr = (L.LbkProjection * 3)()
    X, row, chunk = 0x40000000, 2 * K, 16
    ys = [X + chunk * row, X - chunk * row, 0x80000000]
    for i in range(3):
        arr[i].branches = ctypes.cast(brs[i], ctypes.POINTER(L.LbkBranch))
        arr[i].n_branches = 2
        arr[i].out_features = N
        arr[i].y = ys[i]
    rc = lib.lbk_group_forward_ex(arr, 3, M, K, X, L.LBK_BF16, None, L.LBK_F32, 0x1000, 1 << 30, None)
    assert rc == L.LBK_ERR_ARG
    assert "overlaps input rows of other row chunks" in L.last_error()

"""Operator-level entry points of the HIP LittleBitLinear forward.

* :func:`littlebit_linear` keeps the schema and argument checks of the
  reference operator ``littlebit_cpu_ops::littlebit_linear``
  (patches/littlebit_cpu_optimized.cpp:2324-2329, checks at :607-634) but
  runs on a GPU and computes in fp32 (the reference quantises activations to
  int8 at both stages, patch:669 and :684).
* :class:`LittleBitBranch` / :class:`LittleBitProjection` hold one
  projection's device-resident packed factors and scales and run the fused
  forward (all branches + bias in one call) through ``lbk_linear_forward``.
* :class:`LittleBitProjectionGroup` runs up to four projections that read the
  same input (q/k/v, gate/up) in the launches of one, through
  ``lbk_group_forward`` -- the GPU form of the reference decode step's
  batched q/k/v and gate/up stages (patch:1697-1723, 1777-1798).
* :class:`LittleBitChain` runs calls that each read the one before's outputs
  (o, gate/up, down, next q/k/v) at one row in one launch per link boundary,
  through ``lbk_chain_forward`` (the reference's one-call layer, patch:1627-1833).

Everything here requires CUDA (HIP) tensors; there is no CPU path.
"""
from __future__ import annotations

import ctypes
import threading
from contextlib import contextmanager
from dataclasses import dataclass
from typing import Dict, Optional, Sequence, Tuple

import torch

from . import _lib

__all__ = [
    "LittleBitBranch",
    "LittleBitProjection",
    "LittleBitProjectionGroup",
    "ChainLink",
    "LittleBitChain",
    "littlebit_linear",
    "littlebit_forward",
    "workspace_for",
    "PrivateWorkspace",
    "private_workspace",
    "set_deterministic",
    "deterministic",
]

_DTYPE_CODES = {torch.float32: _lib.LBK_F32, torch.bfloat16: _lib.LBK_BF16}

# (device index, stream handle) -> uint8 workspace tensor
_workspaces: Dict[Tuple[int, int], torch.Tensor] = {}
# Workspaces a captured HIP graph baked in: a replay may use them at any
# time, so they stay allocated for the life of the process.  A workspace that
# no capture used is freed when it is outgrown or dropped.
_graph_held: list = []
_override = threading.local()


class PrivateWorkspace:
    """A workspace owned by one captured graph, outside the per-stream pool.

    The per-stream pool is keyed by stream handle; a graph replayed on
    another stream than the one it was captured on, while eager calls run on
    a stream that reuses the capture stream's handle, would share one
    workspace between concurrent calls.  Calls made inside
    ``with private_workspace(ws):`` use ``ws`` instead.  Size it with an eager
    run of the same calls before the capture (it cannot grow under capture).
    """

    def __init__(self):
        self.buffer: Optional[torch.Tensor] = None

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor:
        b = self.buffer
        if b is None or b.numel() < nbytes or b.device != device:
            _check(not torch.cuda.is_current_stream_capturing(),
                   "a private workspace must be sized by an eager run of the same calls before capture")
            self.buffer = b = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        return b


@contextmanager
def private_workspace(ws: PrivateWorkspace):
    """Run the calls of the block on ``ws`` (see :class:`PrivateWorkspace`)."""
    prev = getattr(_override, "ws", None)
    _override.ws = ws
    try:
        yield ws
    finally:
        _override.ws = prev


def set_deterministic(on: bool) -> bool:
    """Turn the library's deterministic mode on or off (process-wide) and
    return the previous setting.  With it on, decode-path calls (M <= 16, and
    row chunks up to 64) add their split-K partial sums in a fixed order (the
    last block of each row-block adds them), so outputs repeat bit for bit; the GEMM path
    always does.  Workspaces grow on demand, so later calls size theirs with
    the mode in force; a HIP graph captured in one mode replays that mode."""
    return bool(_lib.load().lbk_set_deterministic(1 if on else 0))


@contextmanager
def deterministic(on: bool = True):
    """Run the block with deterministic mode set to ``on``, restoring it after."""
    prev = set_deterministic(on)
    try:
        yield
    finally:
        set_deterministic(prev)


def _ws_key(device: torch.device, stream: int) -> Tuple[int, int]:
    return (device.index if device.index is not None else torch.cuda.current_device(), int(stream))


def workspace_for(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """Scratch buffer of the calls on (device, stream), grown on demand.

    It starts zeroed: the library keeps the state of its latent buffer at
    its head, which a zeroed buffer starts consistently and every complete
    call leaves consistent.  Inside ``private_workspace`` the block's own
    workspace is used instead.
    """
    priv = getattr(_override, "ws", None)
    if priv is not None:
        return priv.get(device, nbytes)
    key = _ws_key(device, stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    if torch.cuda.is_current_stream_capturing() and not any(w is ws for w in _graph_held):
        _graph_held.append(ws)
    return ws


def _call(rc: int, what: str, device: torch.device, stream: int) -> None:
    """Raise for a failed call.  After a launch failure the workspace's state
    may be left half updated (a latent stage ran, its expand stage did not),
    so the workspace is replaced by a fresh zeroed one for the next call."""
    if rc == _lib.LBK_ERR_HIP:
        priv = getattr(_override, "ws", None)
        if priv is not None:
            if priv.buffer is not None:
                _graph_held.append(priv.buffer)  # a capture may have baked it in
            priv.buffer = None
        else:
            _workspaces.pop(_ws_key(device, stream), None)
    _lib.check(rc, what)


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _require_cuda(t: torch.Tensor, name: str) -> None:
    _check(isinstance(t, torch.Tensor), f"{name} must be a tensor")
    _check(t.is_cuda, f"{name} must be a GPU tensor (the HIP path has no CPU fallback)")
    _check(t.is_contiguous(), f"{name} must be contiguous")


@dataclass
class LittleBitBranch:
    """One branch's device tensors, in the runtime-checkpoint naming.

    v_sign [R, ceil(K/32)] int32 (``v_sign_rt``), u_sign [N, ceil(R/32)] int32
    (``u_sign_rt``), v2 [K] fp32, mid [R] fp32 (= v1*u2), u1 [N] fp32
    (convert_hf_to_runtime.py:46-57).
    """

    v_sign: torch.Tensor
    u_sign: torch.Tensor
    v2: torch.Tensor
    mid: torch.Tensor
    u1: torch.Tensor

    @property
    def rank(self) -> int:
        return int(self.v_sign.shape[0])

    @property
    def in_features(self) -> int:
        return int(self.v2.numel())

    @property
    def out_features(self) -> int:
        return int(self.u1.numel())

    def validate(self, K: int, N: int, name: str = "branch") -> None:
        R = self.rank
        for t, nm in ((self.v_sign, "v_sign"), (self.u_sign, "u_sign"), (self.v2, "v2"),
                      (self.mid, "mid"), (self.u1, "u1")):
            _require_cuda(t, f"{name}.{nm}")
        _check(self.v_sign.dtype == torch.int32, f"{name}.v_sign must be int32")
        _check(self.u_sign.dtype == torch.int32, f"{name}.u_sign must be int32")
        for t, nm in ((self.v2, "v2"), (self.mid, "mid"), (self.u1, "u1")):
            _check(t.dtype == torch.float32, f"{name}.{nm} must be float32")
        _check(self.v_sign.dim() == 2 and self.v_sign.shape[1] == (K + 31) // 32,
               f"{name}.v_sign must have shape [R, ceil(K/32)] = [{R}, {(K + 31) // 32}], got {tuple(self.v_sign.shape)}")
        _check(self.u_sign.dim() == 2 and tuple(self.u_sign.shape) == (N, (R + 31) // 32),
               f"{name}.u_sign must have shape [N, ceil(R/32)] = [{N}, {(R + 31) // 32}], got {tuple(self.u_sign.shape)}")
        _check(self.v2.numel() == K, f"{name}.v2 must have K={K} elements")
        _check(self.mid.numel() == R, f"{name}.mid must have R={R} elements")
        _check(self.u1.numel() == N, f"{name}.u1 must have N={N} elements")
        dev = self.v_sign.device
        for t in (self.u_sign, self.v2, self.mid, self.u1):
            _check(t.device == dev, f"{name}: all tensors must be on one device")


@dataclass
class AttentionPartials:
    """The per-chunk partials of one token's attention, as
    ``lbk_attention_decode`` leaves them when called without an output
    (fp32 [heads][ceil(max_seq / 16)][head_dim + 4]).  A projection given
    them as its input merges the attention output while it stages it."""
    partials: torch.Tensor
    head_dim: int
    max_seq: int
    pos: Optional[torch.Tensor] = None  # int64 [1] on the device (graph replay)
    pos_host: int = 0                   # the position when ``pos`` is None


class LittleBitProjection:
    """A projection's branches (draft, optional residual) and optional bias,
    prepared once so that each forward is one C call."""

    def __init__(self, branches: Sequence[LittleBitBranch], bias: Optional[torch.Tensor] = None,
                 tile_v: bool = True):
        """``tile_v`` (default) keeps a tiled copy of each branch's V words
        (``lbk_tile_v_signs``) that the decode path (M <= 64) reads with whole
        128-byte lines per load; the stored words serve every other path."""
        _check(1 <= len(branches) <= 2, "a projection has one or two branches")
        self.branches = list(branches)
        self.in_features = self.branches[0].in_features
        self.out_features = self.branches[0].out_features
        for i, b in enumerate(self.branches):
            b.validate(self.in_features, self.out_features, f"branch{i}")
        self.device = self.branches[0].v_sign.device
        if bias is not None:
            _require_cuda(bias, "bias")
            _check(bias.dtype == torch.float32 and bias.numel() == self.out_features,
                   "bias must be float32 with out_features elements")
            _check(bias.device == self.device, "bias must be on the factors' device")
        self.bias = bias
        arr = (_lib.LbkBranch * len(self.branches))()
        for i, b in enumerate(self.branches):
            arr[i].v_sign = b.v_sign.data_ptr()
            arr[i].u_sign = b.u_sign.data_ptr()
            arr[i].v2 = b.v2.data_ptr()
            arr[i].mid = b.mid.data_ptr()
            arr[i].u1 = b.u1.data_ptr()
            arr[i].rank = b.rank
        # the tiled copies, made once here (not under graph capture, where the
        # projection keeps reading V as stored)
        self._v_tiled = []
        if tile_v and not torch.cuda.is_current_stream_capturing():
            lib = _lib.load()
            stream = torch.cuda.current_stream(self.device)
            for i, b in enumerate(self.branches):
                vt = torch.empty(int(lib.lbk_tiled_v_words(b.rank, self.in_features)), dtype=torch.int32,
                                 device=self.device)
                with torch.cuda.device(self.device):
                    rc = lib.lbk_tile_v_signs(b.v_sign.data_ptr(), b.rank, self.in_features, vt.data_ptr(),
                                              stream.cuda_stream)
                _lib.check(rc, "lbk_tile_v_signs")
                arr[i].v_sign_tiled = vt.data_ptr()
                self._v_tiled.append(vt)
            stream.synchronize()  # the copies are complete before any stream uses them
        self._arr = arr
        self._group = None

    @property
    def ranks(self) -> Tuple[int, ...]:
        return tuple(b.rank for b in self.branches)

    def workspace_bytes(self, M: int) -> int:
        lib = _lib.load()
        n = lib.lbk_linear_workspace_bytes(self._arr, len(self.branches), int(M), self.in_features,
                                           self.out_features)
        if n == 0 and M > 0:
            _lib.check(_lib.LBK_ERR_ARG, "lbk_linear_workspace_bytes")
        return int(n)

    def forward(self, x: Optional[torch.Tensor], out: Optional[torch.Tensor] = None,
                out_dtype: Optional[torch.dtype] = None, *, rms_weight: Optional[torch.Tensor] = None,
                rms_eps: float = 1e-6, x_up: Optional[torch.Tensor] = None,
                residual: Optional[torch.Tensor] = None,
                attn: Optional[AttentionPartials] = None) -> torch.Tensor:
        """y[..., N] = sum of branches (+ bias) for x[..., K] (fp32 or bf16);
        the fusions of :meth:`LittleBitProjectionGroup.forward`."""
        if rms_weight is not None or x_up is not None or residual is not None or attn is not None:
            if self._group is None:
                self._group = LittleBitProjectionGroup([self])
            return self._group.forward(x, None if out is None else [out], out_dtype, rms_weight=rms_weight,
                                       rms_eps=rms_eps, x_up=x_up, residuals=[residual], attn=attn)[0]
        _check(isinstance(x, torch.Tensor) and x.is_cuda, "input must be a GPU tensor")
        _check(x.device == self.device, "input must be on the factors' device")
        _check(x.dtype in _DTYPE_CODES, f"input dtype {x.dtype} unsupported (float32 or bfloat16)")
        _check(x.shape[-1] == self.in_features,
               f"input last dimension {x.shape[-1]} != in_features {self.in_features}")
        lead = tuple(x.shape[:-1])
        x2 = x.reshape(-1, self.in_features)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        M = x2.shape[0]
        odt = out_dtype or x.dtype
        _check(odt in _DTYPE_CODES, f"output dtype {odt} unsupported")
        if out is None:
            out = torch.empty((*lead, self.out_features), dtype=odt, device=x.device)
        else:
            _check(out.is_cuda and out.is_contiguous() and out.dtype == odt
                   and out.numel() == M * self.out_features, "out has the wrong shape, dtype or layout")
        if M == 0:
            return out
        lib = _lib.load()
        stream = torch.cuda.current_stream(x.device).cuda_stream
        need = self.workspace_bytes(M)
        ws = workspace_for(x.device, stream, need)
        rc = lib.lbk_linear_forward(
            self._arr, len(self.branches), M, self.in_features, self.out_features,
            x2.data_ptr(), _DTYPE_CODES[x.dtype],
            self.bias.data_ptr() if self.bias is not None else None,
            out.data_ptr(), _DTYPE_CODES[odt], ws.data_ptr(), ws.numel(), stream)
        _call(rc, "lbk_linear_forward", x.device, stream)
        return out

    __call__ = forward


class LittleBitProjectionGroup:
    """Projections that read the same input, run together.

    ``forward(x)`` returns ``[p.forward(x) for p in projections]`` (same
    values, to the MFMA path's run-to-run tolerance) from two launches in
    total instead of two per projection."""

    def __init__(self, projections: Sequence[LittleBitProjection]):
        _check(1 <= len(projections) <= _lib.LBK_MAX_GROUP,
               f"a group has 1 to {_lib.LBK_MAX_GROUP} projections, got {len(projections)}")
        self.projections = list(projections)
        self.in_features = self.projections[0].in_features
        self.device = self.projections[0].device
        for i, p in enumerate(self.projections):
            _check(p.in_features == self.in_features, f"projection {i}: in_features differs within the group")
            _check(p.device == self.device, f"projection {i}: all projections must be on one device")
        arr = (_lib.LbkProjection * len(self.projections))()
        for i, p in enumerate(self.projections):
            arr[i].branches = ctypes.cast(p._arr, ctypes.POINTER(_lib.LbkBranch))
            arr[i].n_branches = len(p.branches)
            arr[i].out_features = p.out_features
            arr[i].bias = p.bias.data_ptr() if p.bias is not None else None
        self._arr = arr

    def workspace_bytes(self, M: int) -> int:
        lib = _lib.load()
        n = lib.lbk_group_workspace_bytes(self._arr, len(self.projections), int(M), self.in_features)
        if n == 0 and M > 0:
            _lib.check(_lib.LBK_ERR_ARG, "lbk_group_workspace_bytes")
        return int(n)

    def forward(self, x: Optional[torch.Tensor], outs: Optional[Sequence[torch.Tensor]] = None,
                out_dtype: Optional[torch.dtype] = None, *, rms_weight: Optional[torch.Tensor] = None,
                rms_eps: float = 1e-6, x_up: Optional[torch.Tensor] = None,
                residuals: Optional[Sequence[Optional[torch.Tensor]]] = None,
                attn: Optional[AttentionPartials] = None) -> list:
        """Outputs of every projection for input x [..., K].

        Fusions (the reference decode step's inline operations,
        patch:1370-1438 and the residual adds at :1738-1750):
          ``rms_weight``  the projections read RMSNorm(x) * rms_weight;
          ``x_up``        they read SiLU(x) * x_up (x the gate output);
          ``residuals``   per projection an fp32 [..., N] tensor added to its
                          output; it may be the output tensor itself;
          ``attn``        (x None, one row) they read the attention output
                          merged from ``attn``'s partials (patch:1441-1510
                          feeding o_proj), outputs [1, N].
        """
        if attn is not None:
            _check(x is None and rms_weight is None and x_up is None, "attn replaces x and the other input fusions")
            part = attn.partials
            _require_cuda(part, "attn.partials")
            _check(part.dtype == torch.float32 and part.is_contiguous() and part.device == self.device,
                   "attn.partials must be a contiguous float32 tensor on the factors' device")
            if attn.pos is not None:
                _require_cuda(attn.pos, "attn.pos")
                _check(attn.pos.dtype == torch.int64, "attn.pos must be int64")
            odt = out_dtype or torch.float32
            x = part
            x2 = part
            M = 1
            lead = (1,)
            inp = _lib.LbkInput(_lib.LBK_INPUT_ATTN_MERGE, None, 0.0, None, int(attn.head_dim), int(attn.max_seq),
                                None if attn.pos is None else attn.pos.data_ptr(), int(attn.pos_host))
            return self._launch(x2, M, lead, odt, outs, inp, residuals)
        _check(isinstance(x, torch.Tensor) and x.is_cuda, "input must be a GPU tensor")
        _check(x.device == self.device, "input must be on the factors' device")
        _check(x.dtype in _DTYPE_CODES, f"input dtype {x.dtype} unsupported (float32 or bfloat16)")
        _check(x.shape[-1] == self.in_features,
               f"input last dimension {x.shape[-1]} != in_features {self.in_features}")
        _check(rms_weight is None or x_up is None, "rms_weight and x_up exclude each other")
        lead = tuple(x.shape[:-1])
        x2 = x.reshape(-1, self.in_features)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        M = x2.shape[0]
        odt = out_dtype or x.dtype
        inp = None
        if rms_weight is not None:
            _require_cuda(rms_weight, "rms_weight")
            _check(rms_weight.dtype == torch.float32 and rms_weight.numel() == self.in_features,
                   "rms_weight must be float32 with in_features elements")
            inp = _lib.LbkInput(_lib.LBK_INPUT_RMSNORM, rms_weight.data_ptr(), float(rms_eps), None)
        elif x_up is not None:
            _require_cuda(x_up, "x_up")
            _check(x_up.dtype == x.dtype and x_up.numel() == x.numel(), "x_up must match x in dtype and size")
            inp = _lib.LbkInput(_lib.LBK_INPUT_SILU_MUL, None, 0.0, x_up.data_ptr())
        return self._launch(x2, M, lead, odt, outs, inp, residuals)

    def _launch(self, x2, M, lead, odt, outs, inp, residuals) -> list:
        _check(odt in _DTYPE_CODES, f"output dtype {odt} unsupported")
        if outs is None:
            outs = [torch.empty((*lead, p.out_features), dtype=odt, device=x2.device) for p in self.projections]
        else:
            _check(len(outs) == len(self.projections), "one output per projection")
            for o, p in zip(outs, self.projections):
                _check(o.is_cuda and o.is_contiguous() and o.dtype == odt and o.numel() == M * p.out_features,
                       "an output has the wrong shape, dtype or layout")
        if M == 0:
            return list(outs)
        keep = []
        for i, o in enumerate(outs):
            self._arr[i].y = o.data_ptr()
            r = None if residuals is None else residuals[i]
            if r is not None:
                _require_cuda(r, f"residuals[{i}]")
                _check(r.dtype == torch.float32 and r.numel() == o.numel(), "a residual must be float32 like its output")
                keep.append(r)
            self._arr[i].residual = None if r is None else r.data_ptr()
        lib = _lib.load()
        stream = torch.cuda.current_stream(x2.device).cuda_stream
        ws = workspace_for(x2.device, stream, self.workspace_bytes(M))
        rc = lib.lbk_group_forward_ex(self._arr, len(self.projections), M, self.in_features, x2.data_ptr(),
                                      _DTYPE_CODES[x2.dtype], ctypes.byref(inp) if inp is not None else None,
                                      _DTYPE_CODES[odt], ws.data_ptr(), ws.numel(), stream)
        _call(rc, "lbk_group_forward_ex", x2.device, stream)
        return list(outs)

    __call__ = forward


class ChainLink:
    """One call of a :class:`LittleBitChain`: projections that read one input
    (a :class:`LittleBitProjection`, a :class:`LittleBitProjectionGroup` or a
    list of projections), their fp32 output tensors [1, N] and optional fp32
    residuals (each may be its output tensor itself: x += projection(...)).

    How the link reads its input -- for the first link the chain's x, for
    the others the outputs of the link before:
      ``rms_weight``  RMSNorm(input) * rms_weight (the link before has one projection);
      ``silu_mul``    SiLU(gate) * up of the link before's two projections
                      (the first link gets x_up at :meth:`LittleBitChain.forward`);
      neither         the input itself (the link before has one projection).
    """

    def __init__(self, projections, outs: Sequence[torch.Tensor], *,
                 residuals: Optional[Sequence[Optional[torch.Tensor]]] = None,
                 rms_weight: Optional[torch.Tensor] = None, rms_eps: float = 1e-6, silu_mul: bool = False):
        if isinstance(projections, LittleBitProjection):
            projections = [projections]
        elif isinstance(projections, LittleBitProjectionGroup):
            projections = projections.projections
        self.projections = list(projections)
        _check(1 <= len(self.projections) <= _lib.LBK_MAX_GROUP,
               f"a link has 1 to {_lib.LBK_MAX_GROUP} projections, got {len(self.projections)}")
        _check(not (rms_weight is not None and silu_mul), "rms_weight and silu_mul exclude each other")
        self.in_features = self.projections[0].in_features
        for i, p in enumerate(self.projections):
            _check(p.in_features == self.in_features, f"projection {i}: in_features differs within the link")
        _check(len(outs) == len(self.projections), "one output per projection")
        for o, p in zip(outs, self.projections):
            _require_cuda(o, "out")
            _check(o.dtype == torch.float32 and o.is_contiguous() and o.numel() == p.out_features,
                   "an output must be a contiguous float32 tensor with out_features elements (one row)")
        self.outs = list(outs)
        self.residuals = list(residuals) if residuals is not None else [None] * len(self.projections)
        _check(len(self.residuals) == len(self.projections), "one residual (or None) per projection")
        for r, p in zip(self.residuals, self.projections):
            if r is not None:
                _require_cuda(r, "residual")
                _check(r.dtype == torch.float32 and r.numel() == p.out_features,
                       "a residual must be float32 with out_features elements")
        if rms_weight is not None:
            _require_cuda(rms_weight, "rms_weight")
            _check(rms_weight.dtype == torch.float32 and rms_weight.numel() == self.in_features,
                   "rms_weight must be float32 with in_features elements")
        self.rms_weight = rms_weight
        self.rms_eps = float(rms_eps)
        self.silu_mul = bool(silu_mul)


class LittleBitChain:
    """Calls in sequence at one row, each reading the outputs of the one
    before (``lbk_chain_forward``): o, gate/up, down and the next layer's
    q/k/v of a decode step.  Same results as running the links one by one
    with :meth:`LittleBitProjectionGroup.forward`; n links take n + 1
    launches instead of 2 n (the kernel between two links expands the first
    link's rows and adds their part of the next link's latent vector).  The
    reference runs a decoder layer's projections in one call
    (patches/littlebit_cpu_optimized.cpp:1627-1833).  The output and residual
    tensors are fixed when the chain is made, so it can be captured in a HIP
    graph."""

    def __init__(self, links: Sequence[ChainLink]):
        _check(1 <= len(links) <= _lib.LBK_MAX_CHAIN, f"a chain has 1 to {_lib.LBK_MAX_CHAIN} links")
        self.links = list(links)
        self.device = self.links[0].projections[0].device
        self._keep = []
        arr = (_lib.LbkChainLink * len(self.links))()
        for j, lk in enumerate(self.links):
            projs = (_lib.LbkProjection * len(lk.projections))()
            for i, p in enumerate(lk.projections):
                _check(p.device == self.device, "all projections of a chain must be on one device")
                projs[i].branches = ctypes.cast(p._arr, ctypes.POINTER(_lib.LbkBranch))
                projs[i].n_branches = len(p.branches)
                projs[i].out_features = p.out_features
                projs[i].bias = p.bias.data_ptr() if p.bias is not None else None
                projs[i].y = lk.outs[i].data_ptr()
                projs[i].residual = None if lk.residuals[i] is None else lk.residuals[i].data_ptr()
            if lk.rms_weight is not None:
                inp = _lib.LbkInput(_lib.LBK_INPUT_RMSNORM, lk.rms_weight.data_ptr(), lk.rms_eps, None)
            elif lk.silu_mul:
                inp = _lib.LbkInput(_lib.LBK_INPUT_SILU_MUL, None, 0.0, None)
            else:
                inp = _lib.LbkInput(_lib.LBK_INPUT_PLAIN, None, 0.0, None)
            self._keep += [projs, inp, lk.projections]
            arr[j].projs = ctypes.cast(projs, ctypes.POINTER(_lib.LbkProjection))
            arr[j].n_proj = len(lk.projections)
            arr[j].in_features = lk.in_features
            arr[j].input = ctypes.pointer(inp)
        self._arr = arr
        self._inp0 = self._keep[1]
        lib = _lib.load()
        n = lib.lbk_chain_workspace_bytes(arr, len(self.links))
        if n == 0:
            _lib.check(_lib.LBK_ERR_ARG, "lbk_chain_workspace_bytes")
        self._ws_bytes = int(n)

    def fused(self, x: Optional[torch.Tensor] = None, attn: Optional[AttentionPartials] = None) -> bool:
        """Whether the links run joined (n + 1 launches) for this input."""
        ptr = self._set_input(x, attn, None)
        rc = _lib.load().lbk_chain_fused(self._arr, len(self.links), ptr)
        if rc < 0:
            _lib.check(rc, "lbk_chain_fused")
        return rc == 1

    def _set_input(self, x, attn, x_up):
        lk = self.links[0]
        inp = self._inp0
        if attn is not None:
            _check(x is None and x_up is None and lk.rms_weight is None and not lk.silu_mul,
                   "attn replaces x and the first link's other input fusions")
            part = attn.partials
            _require_cuda(part, "attn.partials")
            _check(part.dtype == torch.float32 and part.is_contiguous() and part.device == self.device,
                   "attn.partials must be a contiguous float32 tensor on the chain's device")
            inp.kind = _lib.LBK_INPUT_ATTN_MERGE
            inp.head_dim = int(attn.head_dim)
            inp.max_seq = int(attn.max_seq)
            inp.pos_device = None if attn.pos is None else attn.pos.data_ptr()
            inp.pos = int(attn.pos_host)
            return part.data_ptr()
        _check(isinstance(x, torch.Tensor) and x.is_cuda and x.device == self.device, "x must be a GPU tensor on the chain's device")
        _check(x.dtype == torch.float32 and x.is_contiguous() and x.numel() == lk.in_features,
               "x must be a contiguous float32 tensor with the first link's in_features elements (one row)")
        if lk.rms_weight is not None:
            inp.kind = _lib.LBK_INPUT_RMSNORM
        elif lk.silu_mul:
            _check(isinstance(x_up, torch.Tensor) and x_up.is_cuda and x_up.dtype == torch.float32
                   and x_up.is_contiguous() and x_up.numel() == x.numel(), "the first link's SiLU * up needs x_up like x")
            inp.kind = _lib.LBK_INPUT_SILU_MUL
            inp.x1 = x_up.data_ptr()
        else:
            inp.kind = _lib.LBK_INPUT_PLAIN
        return x.data_ptr()

    def forward(self, x: Optional[torch.Tensor] = None, *, attn: Optional[AttentionPartials] = None,
                x_up: Optional[torch.Tensor] = None) -> None:
        """Run the chain on x [1, K] fp32 (or the attention partials ``attn``);
        the results are in the links' output tensors."""
        ptr = self._set_input(x, attn, x_up)
        lib = _lib.load()
        stream = torch.cuda.current_stream(self.device).cuda_stream
        ws = workspace_for(self.device, stream, self._ws_bytes)
        rc = lib.lbk_chain_forward(self._arr, len(self.links), ptr, ws.data_ptr(), ws.numel(), stream)
        _call(rc, "lbk_chain_forward", self.device, stream)

    __call__ = forward


def littlebit_forward(x: torch.Tensor, branches: Sequence[LittleBitBranch],
                      bias: Optional[torch.Tensor] = None,
                      out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """One-shot fused forward (prepares a :class:`LittleBitProjection`)."""
    return LittleBitProjection(branches, bias).forward(x, out_dtype=out_dtype)


def littlebit_linear(input: torch.Tensor, v2: torch.Tensor, v_sign: torch.Tensor, v_cols: int,
                     mid: torch.Tensor, u_sign: torch.Tensor, u_cols: int,
                     u1: torch.Tensor) -> torch.Tensor:
    """GPU counterpart of ``torch.ops.littlebit_cpu_ops.littlebit_linear``.

    Same arguments and the same precondition checks (patch:607-634, raised as
    RuntimeError), output fp32 [M, N]; computed in fp32 without the
    reference's int8 activation quantisation.
    """
    for t, nm in ((input, "input"), (v2, "v2"), (mid, "mid"), (u1, "u1")):
        _require_cuda(t, nm)
        _check(t.dtype == torch.float32, f"{nm} must be float32")
    for t, nm in ((v_sign, "v_sign"), (u_sign, "u_sign")):
        _require_cuda(t, nm)
        _check(t.dtype == torch.int32, f"{nm} must be int32")
    _check(input.dim() == 2, "input must have shape [M, K]")
    _check(v2.dim() == 2 and v2.size(0) == 1, "v2 must have shape [1, K]")
    _check(mid.dim() == 2 and mid.size(0) == 1, "mid must have shape [1, R]")
    _check(u1.dim() == 2 and u1.size(0) == 1, "u1 must have shape [1, N]")
    _check(input.size(1) == v_cols, "input K must match v_cols")
    _check(v2.size(1) == v_cols, "v2 second dimension must match v_cols")
    _check(v_sign.dim() == 2, "v_sign must have shape [R, ceil(K/32)]")
    _check(u_sign.dim() == 2, "u_sign must have shape [N, ceil(R/32)]")
    _check(v_sign.size(0) == mid.size(1), "mid rank must match v_sign rows")
    _check(u_sign.size(0) == u1.size(1), "u1 out_features must match u_sign rows")
    _check(mid.size(1) == u_cols, "mid rank must match u_cols")
    _check(v_sign.size(1) == (v_cols + 31) // 32, "v_sign second dimension must equal ceil(v_cols / 32)")
    _check(u_sign.size(1) == (u_cols + 31) // 32, "u_sign second dimension must equal ceil(u_cols / 32)")
    dev = input.device
    for t in (v2, v_sign, mid, u_sign, u1):
        _check(t.device == dev, "all tensors must be on one device")
    M = input.size(0)
    N = u_sign.size(0)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    if M == 0:
        return out
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    br = (_lib.LbkBranch * 1)()
    br[0].v_sign = v_sign.data_ptr()
    br[0].u_sign = u_sign.data_ptr()
    br[0].v2 = v2.data_ptr()
    br[0].mid = mid.data_ptr()
    br[0].u1 = u1.data_ptr()
    br[0].rank = int(u_cols)
    need = lib.lbk_linear_workspace_bytes(br, 1, M, int(v_cols), N)
    if need == 0:
        _lib.check(_lib.LBK_ERR_ARG, "littlebit_linear")
    ws = workspace_for(dev, stream, int(need))
    rc = lib.lbk_littlebit_linear(input.data_ptr(), M, v2.data_ptr(), v_sign.data_ptr(), int(v_cols),
                                  mid.data_ptr(), u_sign.data_ptr(), int(u_cols), u1.data_ptr(), N,
                                  out.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    _call(rc, "littlebit_linear", dev, stream)
    return out

"""Drop-in ``LittleBitLinear`` whose binarised forward runs the HIP kernels.

Mirrors quantization/modules/littlebit.py:
  * construction by class swap + ``__quant_convert__`` (:9-48) with the same
    split-dim / effective-bit bookkeeping (:50-93) and buffers
    ``_eff_bit_target``, ``_split_dim_final``, ``_eff_bit_actual`` (:41-43);
  * parameter names U, V, u1, u2, v1, v2 (+ ``_R``) (:154-168);
  * ``state_dict`` in the packed format ``{U,V,U_R,V_R}_packed`` (int32) and
    ``*_shape`` (int64) (:307-345);
  * ``forward`` = main branch + residual branch + bias (:95-112).

Differences, all on purpose:
  * In binarised mode the signs stay packed (one bit each) on the GPU; the
    reference unpacks them to +-1 in the activation dtype
    (quantization/utils/quant_util.py:247-251).
  * The residual branch may have its own rank (``residual_split_dim``); the
    reference module forces the same rank on both (:161-168) while its runtime
    layout allows any (convert_hf_to_runtime.py:66-84).
  * ``forward`` needs GPU tensors; there is no CPU path.
  * Training-time initialisation (SVD, :175-305) is not provided.
"""
from __future__ import annotations

from typing import Dict, Optional

import torch
import torch.nn as nn

from .binary_packer import binary_packer, words_per_row
from .ops import LittleBitBranch, LittleBitProjection

__all__ = ["LittleBitLinear", "sign_pm1"]


def sign_pm1(x: torch.Tensor) -> torch.Tensor:
    """sign(x) with sign(0) = +1 (quantization/functions/binary.py:6-10), as int8."""
    s = torch.sign(x)
    s = torch.where(s == 0, torch.ones_like(s), s)
    return s.to(torch.int8)


_BRANCH_SUFFIX = {"main": "", "residual": "_R"}


class LittleBitLinear(nn.Linear):
    # ------------------------------------------------------------------
    # construction (littlebit.py:9-93)
    # ------------------------------------------------------------------
    def __quant_convert__(
        self,
        do_train: bool = False,
        quant_func=None,
        *,
        split_dim: int = 1024,
        eff_bit: Optional[float] = None,
        residual: bool = False,
        ratio_factor: float = 1.0,
        min_split_dim: int = 8,
        residual_split_dim: Optional[int] = None,
        **kwargs,
    ):
        if do_train:
            raise NotImplementedError("training-time initialisation is not part of this package")
        self.do_train = False
        self.quant_func = quant_func
        self.residual = residual
        self._binarized = False

        a, b = self.in_features, self.out_features
        split_float = self._estimate_split_dim(a, b, eff_bit, residual)
        if split_float:
            split_float *= ratio_factor
        final_split = self._finalize_split_dim(split_float, split_dim, min_split_dim)
        self.split_dim = final_split
        self.split_dim_R = int(residual_split_dim) if residual_split_dim else final_split

        eff_actual = self._compute_eff_bits(a, b, final_split, residual)
        self.register_buffer("_eff_bit_target", torch.tensor(-1.0 if eff_bit is None else float(eff_bit)))
        self.register_buffer("_split_dim_final", torch.tensor(final_split))
        self.register_buffer("_eff_bit_actual", torch.tensor(eff_actual))
        self._initialize_empty_parameters()
        self._proj: Optional[LittleBitProjection] = None

    @staticmethod
    def _bits_per_weight(a: int, b: int, rank: int, residual: bool) -> float:
        """What a rank-``rank`` factorisation of an a x b weight costs per weight
        (the accounting of littlebit.py:83-93): per branch, one sign per entry
        of U and V plus 16 bits per latent entry (rank * (a + b + 16)), and
        16 bits per input and output scale (16 * (a + b)); the residual form
        holds two branches."""
        if a * b == 0:
            return float("inf")
        branches = 2 if residual else 1
        return branches * (rank * (a + b + 16) + 16 * (a + b)) / (a * b)

    @staticmethod
    def _estimate_split_dim(a, b, eff_bit_target, residual) -> Optional[float]:
        """The (fractional) rank at which _bits_per_weight meets
        ``eff_bit_target``, solved from its linear form (littlebit.py:50-63);
        None without a target or for an empty weight."""
        if eff_bit_target is None or a * b == 0:
            return None
        branches = 2 if residual else 1
        per_rank = branches * (a + b + 16)
        fixed = branches * 16 * (a + b)
        return (a * b * eff_bit_target - fixed) / per_rank if per_rank else None

    @staticmethod
    def _finalize_split_dim(split_float, split_default, min_split_dim) -> int:
        """The estimate (the default without one), truncated to an integer and
        rounded down to a multiple of 8; zero or anything below
        ``min_split_dim`` gives ``min_split_dim`` (littlebit.py:65-81)."""
        raw = split_default if split_float is None else split_float
        rank = 8 * (int(raw or 0) // 8)
        return max(rank or min_split_dim, min_split_dim)

    @staticmethod
    def _compute_eff_bits(a: int, b: int, s: int, residual: bool) -> float:
        """Bits per weight of the rank-s factorisation (littlebit.py:83-93)."""
        return LittleBitLinear._bits_per_weight(a, b, s, residual)

    def _initialize_empty_parameters(self):
        """Meta-device placeholders with the reference names (littlebit.py:144-173)."""
        def param(*shape):
            return nn.Parameter(torch.empty(*shape, device="meta", dtype=torch.bfloat16), requires_grad=False)

        self.U = param(self.out_features, self.split_dim)
        self.V = param(self.split_dim, self.in_features)
        self.u1 = param(1, self.out_features)
        self.u2 = param(1, self.split_dim)
        self.v1 = param(1, self.split_dim)
        self.v2 = param(1, self.in_features)
        if self.residual:
            self.U_R = param(self.out_features, self.split_dim_R)
            self.V_R = param(self.split_dim_R, self.in_features)
            self.u1_R = param(1, self.out_features)
            self.u2_R = param(1, self.split_dim_R)
            self.v1_R = param(1, self.split_dim_R)
            self.v2_R = param(1, self.in_features)
        if "weight" in self._parameters:
            del self._parameters["weight"]
        self.register_parameter("weight", None)

    # ------------------------------------------------------------------
    # packed storage
    # ------------------------------------------------------------------
    def _branches(self):
        return ("main", "residual") if self.residual else ("main",)

    def set_packed_branch(self, branch: str, u_packed: torch.Tensor, v_packed: torch.Tensor,
                          u1: torch.Tensor, v2: torch.Tensor, *, v1: Optional[torch.Tensor] = None,
                          u2: Optional[torch.Tensor] = None, mid: Optional[torch.Tensor] = None,
                          rank: Optional[int] = None) -> None:
        """Install one branch from packed words and scales.

        Either (v1, u2) -- the HF packed checkpoint -- or ``mid`` -- the runtime
        checkpoint -- gives the latent scale; mid = v1.float() * u2.float()
        exactly as convert_hf_to_runtime.py:54-57.
        """
        sfx = _BRANCH_SUFFIX[branch]
        if branch == "residual" and not self.residual:
            raise RuntimeError("module was converted without a residual branch")
        R = int(rank) if rank is not None else int(v_packed.shape[0])
        if tuple(v_packed.shape) != (R, words_per_row(self.in_features)):
            raise RuntimeError(f"V packed shape {tuple(v_packed.shape)} != ({R}, {words_per_row(self.in_features)})")
        if tuple(u_packed.shape) != (self.out_features, words_per_row(R)):
            raise RuntimeError(f"U packed shape {tuple(u_packed.shape)} != ({self.out_features}, {words_per_row(R)})")
        if mid is None:
            if v1 is None or u2 is None:
                raise RuntimeError("need mid or (v1, u2)")
            mid = v1.to(torch.float32) * u2.to(torch.float32)
            setattr(self, "v1" + sfx, nn.Parameter(v1.detach().clone(), requires_grad=False))
            setattr(self, "u2" + sfx, nn.Parameter(u2.detach().clone(), requires_grad=False))
        else:
            # runtime layout: only the fused latent scale exists
            for nm in ("v1" + sfx, "u2" + sfx):
                if nm in self._parameters:
                    del self._parameters[nm]
        if branch == "main":
            # the rank comes from the tensors, as in quant_util.py:259-297
            self.split_dim = R
            self._split_dim_final = torch.tensor(R)
            self._eff_bit_actual = torch.tensor(
                self._compute_eff_bits(self.in_features, self.out_features, R, self.residual))
        else:
            self.split_dim_R = R
        setattr(self, "u1" + sfx, nn.Parameter(u1.detach().clone(), requires_grad=False))
        setattr(self, "v2" + sfx, nn.Parameter(v2.detach().clone(), requires_grad=False))
        # the dense factors are replaced by their packed words
        for nm in ("U" + sfx, "V" + sfx):
            if nm in self._parameters:
                del self._parameters[nm]
        self.register_buffer("U" + sfx + "_packed", u_packed.detach().to(torch.int32).contiguous())
        self.register_buffer("V" + sfx + "_packed", v_packed.detach().to(torch.int32).contiguous())
        self.register_buffer("mid" + sfx, mid.detach().to(torch.float32).reshape(1, R).contiguous())
        self._binarized = True
        self._proj = None

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        """Accept the packed HF keys (littlebit.py:315-318), the runtime keys
        (convert_hf_to_runtime.py:46-84) or dense U/V, then let nn.Module load
        the remaining parameters and buffers."""
        consumed = set()
        installed = set()  # parameter / buffer names this call set from the state dict itself
        for branch in self._branches():
            sfx = _BRANCH_SUFFIX[branch]
            rsfx = "_r" if branch == "residual" else ""
            hf_u, hf_v = prefix + "U" + sfx + "_packed", prefix + "V" + sfx + "_packed"
            rt_u, rt_v = prefix + f"u_sign{rsfx}_rt", prefix + f"v_sign{rsfx}_rt"
            # the latent scale: v1 and u2 (the HF format), else mid (the
            # runtime format, or this module's own state_dict after a runtime load)
            v1, u2 = state_dict.get(prefix + "v1" + sfx), state_dict.get(prefix + "u2" + sfx)
            mid = state_dict.get(prefix + "mid" + sfx)
            if v1 is None or u2 is None:
                v1 = u2 = None
            if hf_u in state_dict and hf_v in state_dict:
                shape_v = state_dict.get(prefix + "V" + sfx + "_shape")
                if v1 is None and mid is None:
                    raise KeyError(f"{prefix}{'v1' + sfx}: packed branch {branch!r} has neither (v1, u2) nor mid")
                self.set_packed_branch(
                    branch, state_dict[hf_u], state_dict[hf_v], state_dict[prefix + "u1" + sfx],
                    state_dict[prefix + "v2" + sfx], v1=v1, u2=u2, mid=None if v1 is not None else mid,
                    rank=int(shape_v[0]) if shape_v is not None else None)
                consumed.update({hf_u, hf_v, prefix + "U" + sfx + "_shape", prefix + "V" + sfx + "_shape"})
            elif rt_u in state_dict and rt_v in state_dict:
                shape_v = state_dict.get(rt_v + "_shape")
                self.set_packed_branch(
                    branch, state_dict[rt_u], state_dict[rt_v], state_dict[prefix + "u1" + rsfx],
                    state_dict[prefix + "v2" + rsfx], mid=state_dict[prefix + "mid" + rsfx],
                    rank=int(shape_v[0]) if shape_v is not None else None)
                consumed.update({rt_u, rt_v, rt_u + "_shape", rt_v + "_shape", prefix + "u1" + rsfx,
                                 prefix + "v2" + rsfx, prefix + "mid" + rsfx})
                installed.update({"u1" + sfx, "v2" + sfx})
            elif prefix + "U" + sfx in state_dict and prefix + "V" + sfx in state_dict:
                self.set_packed_branch(
                    branch, binary_packer(sign_pm1(state_dict[prefix + "U" + sfx].detach().cpu())),
                    binary_packer(sign_pm1(state_dict[prefix + "V" + sfx].detach().cpu())),
                    state_dict[prefix + "u1" + sfx], state_dict[prefix + "v2" + sfx],
                    v1=state_dict[prefix + "v1" + sfx], u2=state_dict[prefix + "u2" + sfx])
                consumed.update({prefix + "U" + sfx, prefix + "V" + sfx})
            else:
                continue
            installed.update({"U" + sfx + "_packed", "V" + sfx + "_packed", "mid" + sfx})
            consumed.add(prefix + "mid" + sfx)
        rest = {k: v for k, v in state_dict.items() if k not in consumed}
        super()._load_from_state_dict(rest, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)
        # buffers installed above from keys consumed here are not missing, nor
        # is the split-dim bookkeeping, which the runtime layout drops
        # (convert_hf_to_runtime.py:86-93) and set_packed_branch recomputes
        for nm in installed | {"_eff_bit_target", "_split_dim_final", "_eff_bit_actual"}:
            while prefix + nm in missing_keys:
                missing_keys.remove(prefix + nm)
        self._proj = None

    def state_dict(self, *args, **kwargs):
        """Packed format: ``{U,V}[_R]_packed`` int32 + ``*_shape`` int64 (littlebit.py:307-345)."""
        prefix = kwargs.get("prefix", "")
        state = super().state_dict(*args, **kwargs)
        for k in [k for k in state if k[len(prefix):].startswith(("U", "V"))]:
            del state[k]
        # The latent scale goes out as v1 and u2, as the reference saves it;
        # a branch loaded from the runtime layout has only mid = v1 * u2,
        # which then goes out instead (and loads back through the same key).
        for branch in self._branches():
            sfx = _BRANCH_SUFFIX[branch]
            if "v1" + sfx in self._parameters and "u2" + sfx in self._parameters:
                state.pop(prefix + "mid" + sfx, None)
        for k, v in self.pack_weights().items():
            state[prefix + k] = v
        return state

    def pack_weights(self) -> Dict[str, torch.Tensor]:
        out = {}
        for branch in self._branches():
            sfx = _BRANCH_SUFFIX[branch]
            R = self.split_dim if branch == "main" else self.split_dim_R
            if getattr(self, "U" + sfx + "_packed", None) is not None:
                u = getattr(self, "U" + sfx + "_packed")
                v = getattr(self, "V" + sfx + "_packed")
            else:
                u = binary_packer(sign_pm1(getattr(self, "U" + sfx).data.cpu()))
                v = binary_packer(sign_pm1(getattr(self, "V" + sfx).data.cpu()))
            out["U" + sfx + "_packed"] = u
            out["U" + sfx + "_shape"] = torch.tensor([self.out_features, R], dtype=torch.long)
            out["V" + sfx + "_packed"] = v
            out["V" + sfx + "_shape"] = torch.tensor([R, self.in_features], dtype=torch.long)
        return out

    # ------------------------------------------------------------------
    # forward (littlebit.py:95-121)
    # ------------------------------------------------------------------
    def _projection(self) -> LittleBitProjection:
        if self._proj is not None and self._proj.device == self.U_packed.device:
            return self._proj
        branches = []
        for branch in self._branches():
            sfx = _BRANCH_SUFFIX[branch]
            u = getattr(self, "U" + sfx + "_packed", None)
            if u is None:
                raise RuntimeError(f"branch {branch!r} has no packed weights; load a packed state dict first")
            branches.append(LittleBitBranch(
                v_sign=getattr(self, "V" + sfx + "_packed").contiguous(),
                u_sign=u.contiguous(),
                v2=getattr(self, "v2" + sfx).detach().to(torch.float32).reshape(-1).contiguous(),
                mid=getattr(self, "mid" + sfx).detach().to(torch.float32).reshape(-1).contiguous(),
                u1=getattr(self, "u1" + sfx).detach().to(torch.float32).reshape(-1).contiguous(),
            ))
        bias = self.bias.detach().to(torch.float32).contiguous() if self.bias is not None else None
        self._proj = LittleBitProjection(branches, bias)
        return self._proj

    def _apply(self, fn, *args, **kwargs):
        self._proj = None
        return super()._apply(fn, *args, **kwargs)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self._binarized:
            raise RuntimeError("LittleBitLinear.forward needs packed (binarised) weights")
        return self._projection().forward(x, out_dtype=x.dtype)

    # ------------------------------------------------------------------
    @property
    def eff_bit_target(self):
        v = self._eff_bit_target.item()
        return None if v < 0 else v

    @property
    def eff_bit_actual(self):
        return self._eff_bit_actual.item()

    @property
    def total_bit_usage(self):
        return self.eff_bit_actual * self.in_features * self.out_features

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, split_dim={self.split_dim}, residual={self.residual}"
                + (f", split_dim_R={self.split_dim_R}" if self.residual else "")
                + f", binarized={self._binarized}")

    @classmethod
    def from_packed(cls, in_features: int, out_features: int, branches, bias: Optional[torch.Tensor] = None,
                    device=None) -> "LittleBitLinear":
        """Build a binarised module from per-branch dicts with keys
        u_packed, v_packed, u1, v2 and either mid or (v1, u2)."""
        m = nn.Linear(in_features, out_features, bias=bias is not None, device="meta")
        m.__class__ = cls
        ranks = [int(b["v_packed"].shape[0]) for b in branches]
        m.__quant_convert__(False, None, split_dim=ranks[0], residual=len(branches) > 1,
                            residual_split_dim=ranks[1] if len(branches) > 1 else None)
        for name, b in zip(("main", "residual"), branches):
            m.set_packed_branch(name, b["u_packed"], b["v_packed"], b["u1"], b["v2"], v1=b.get("v1"),
                                u2=b.get("u2"), mid=b.get("mid"))
        if bias is not None:
            m.bias = nn.Parameter(bias.detach().clone(), requires_grad=False)
        if device is not None:
            m.to(device)
        return m

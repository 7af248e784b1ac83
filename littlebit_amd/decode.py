"""GPU decode and verify steps of a LittleBit Llama-style model.

The call sites of the LittleBitLinear forward in the reference are its CPU
runtime's draft and target models:

* ``CPUDraftModel`` (cpu_draft_model.py:141-593): one LittleBit model with a
  persistent KV cache, ``prefill`` / ``generate_draft_tokens`` with the draft
  positions rolled back after each call;
* ``CPUTargetModel`` (cpu_target_model.py:371-556): two LittleBit models (the
  draft checkpoint and the residual checkpoint, ``_LBModelUnit``
  :137-364) whose final hidden states are summed before one lm_head;
  ``forward(input_ids)`` reuses the KV caches over the common prefix with the
  previous call and returns zero logits for the cached rows.

:class:`GPUDraftModel` and :class:`GPUTargetModel` keep those APIs and cache
semantics on one GPU.  :class:`LittleBitDecoder` is the model unit.  Its
layer is the reference runtime's (``full_forward_cpu``, patches/
littlebit_cpu_optimized.cpp:1522-1840, batch form :1846-2079):

    h = RMSNorm(x; ln1);  q, k, v = LB(h)
    a = attention(q, K[0..pos], V[0..pos])      (GQA, no rotary embedding)
    x = x + LB_o(a);  h = RMSNorm(x; ln2)
    x = x + LB_down(SiLU(LB_gate(h)) * LB_up(h))

with ``RMSNorm(x) = x / sqrt(mean(x^2) + eps) * w`` (patch:1370-1405), the
KV cache of each layer [kv_heads, max_seq, head_dim] fp32 (patch:1441-1456),
scores scaled by ``attn_scale`` and a plain softmax (patch:1474-1489).  All
projections run through the HIP LittleBitLinear kernels; q/k/v and gate/up
are one group call each (the reference batches their U-stages the same way,
patch:1697-1723 and 1777-1798).  Norms, attention, SiLU and the lm_head are
plain PyTorch on the GPU.

The reference's model config and loader come from the un-vendored
``lb_kernels`` package (DummyLlama3Config, load_dummy_llama3_model_from_state);
:class:`DecoderConfig` takes the fields of the ``dummy_llama3_config.json``
that convert_hf_to_runtime.py:193-213 writes, and ``attn_scale`` is
``head_dim ** -0.5``.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from .ops import LittleBitProjection, LittleBitProjectionGroup, PrivateWorkspace, private_workspace
from .runtime import load_runtime_checkpoint, runtime_projections

__all__ = ["DecoderConfig", "LittleBitDecoder", "GPUDraftModel", "GPUTargetModel", "rms_norm"]

_PROJ_ATTN = ("q_proj", "k_proj", "v_proj", "o_proj")
_PROJ_MLP = ("gate_proj", "up_proj", "down_proj")


@dataclass
class DecoderConfig:
    """Fields of dummy_llama3_config.json (convert_hf_to_runtime.py:193-213)."""

    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    vocab_size: int
    rms_norm_eps: float = 1e-6
    name: str = "llama"

    @classmethod
    def from_dict(cls, d: Dict) -> "DecoderConfig":
        # like cpu_draft_model.py:166-172: keys that are not model fields are dropped
        keys = cls.__dataclass_fields__.keys()
        return cls(**{k: v for k, v in d.items() if k in keys})

    @classmethod
    def from_file(cls, path) -> "DecoderConfig":
        return cls.from_dict(json.loads(Path(path).read_text()))

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def kv_repeat(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    @property
    def attn_scale(self) -> float:
        return self.head_dim ** -0.5


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """x / sqrt(mean(x^2) + eps) * w over the last dim (patch:1370-1405)."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


class LittleBitDecoder:
    """One LittleBit transformer on the GPU with its KV cache.

    ``state`` is a runtime-layout state dict (:func:`~littlebit_amd.runtime.
    convert_state_dict` keys).  ``residual`` selects the projections'
    in-module residual branches (``_r`` keys): None uses them where present,
    False ignores them.  ``fuse`` (default) runs the RMSNorms, SiLU * up and
    the residual adds inside the LittleBitLinear calls, as the reference's
    C++ step does inline; ``fuse=False`` runs them as separate PyTorch ops.
    """

    def __init__(self, state: Dict[str, torch.Tensor], config: DecoderConfig, device="cuda",
                 max_seq_len: int = 4096, residual: Optional[bool] = None, fuse: bool = True):
        dev = torch.device(device)
        self.fuse = bool(fuse)
        if dev.type != "cuda":
            raise RuntimeError("LittleBitDecoder runs on a GPU (the HIP kernels have no CPU path)")
        self.config = config
        self.device = dev
        self.max_seq_len = int(max_seq_len)
        projs = runtime_projections(state, dev, residual=residual)

        def f32(key):
            if key not in state:
                raise KeyError(f"runtime state has no {key}")
            return state[key].to(dev, torch.float32).reshape(-1).contiguous()

        self.layers = []
        for i in range(config.num_hidden_layers):
            p = f"model.layers.{i}"
            get = lambda n, sub: projs[f"{p}.{sub}.{n}"]  # noqa: E731
            q, k, v, o = (get(n, "self_attn") for n in _PROJ_ATTN)
            gate, up, down = (get(n, "mlp") for n in _PROJ_MLP)
            self.layers.append({
                "ln1": f32(f"{p}.input_layernorm.weight"),
                "ln2": f32(f"{p}.post_attention_layernorm.weight"),
                "qkv": LittleBitProjectionGroup([q, k, v]),
                "o": o,
                "gate_up": LittleBitProjectionGroup([gate, up]),
                "down": down,
            })
        self.final_norm = f32("model.norm.weight")
        c = config
        shape = (c.num_hidden_layers, c.num_key_value_heads, self.max_seq_len, c.head_dim)
        self.k_cache = torch.zeros(shape, dtype=torch.float32, device=dev)
        self.v_cache = torch.zeros(shape, dtype=torch.float32, device=dev)
        self.cache_pos = 0
        # one-token steps and batches of up to 64 tokens use the HIP attention
        # (head_dim 64 or 128)
        self._hip_attn = self.fuse and c.head_dim in (64, 128)
        if self._hip_attn:
            from . import _lib
            nbytes = _lib.load().lbk_attention_partial_bytes(c.num_attention_heads, self.max_seq_len, c.head_dim)
            self._attn_part = torch.empty(max(int(nbytes) // 4, 1), dtype=torch.float32, device=dev)
        self._batch_part = None  # partials of the batched attention, grown as needed
        self._chains = None  # one-token steps: each layer's o .. next q/k/v as one LittleBitChain

    def reset(self):
        """Forget the cached positions (the reference's _LBModelUnit.reset)."""
        self.cache_pos = 0

    # ------------------------------------------------------------------ core
    def _attention(self, li: int, q, k, v, start: int, length: Optional[int], pos_t: Optional[torch.Tensor],
                   tree_mask: Optional[torch.Tensor]):
        """q [N, heads*hd], k/v [N, kv*hd] at positions start..start+N-1.

        ``length`` (eager) attends over cache[:length]; with ``pos_t`` (a
        device scalar, graph-capturable, N == 1) over the whole cache with
        positions > pos masked.  ``tree_mask`` [N, N] bool restricts the new
        tokens to their tree ancestors (all earlier positions stay visible).
        """
        c = self.config
        N = q.shape[0]
        kvh, hd, rep = c.num_key_value_heads, c.head_dim, c.kv_repeat
        kc, vc = self.k_cache[li], self.v_cache[li]
        if N == 1 and tree_mask is None and self._hip_attn:
            return self._attention_hip(q, k, v, kc, vc, start, pos_t)
        if 1 < N <= 64 and pos_t is None and self._hip_attn and length == start + N:
            return self._attention_batch_hip(q, k, v, kc, vc, start, tree_mask)
        k3 = k.view(N, kvh, hd).transpose(0, 1)
        v3 = v.view(N, kvh, hd).transpose(0, 1)
        if pos_t is None:
            kc[:, start:start + N] = k3
            vc[:, start:start + N] = v3
            S = length
            keys, vals = kc[:, :S], vc[:, :S]
        else:
            kc.index_copy_(1, pos_t, k3)
            vc.index_copy_(1, pos_t, v3)
            S = self.max_seq_len
            keys, vals = kc, vc
        qg = q.view(N, kvh, rep, hd).permute(1, 2, 0, 3).reshape(kvh, rep * N, hd)
        scores = torch.matmul(qg, keys.transpose(1, 2)) * c.attn_scale  # [kvh, rep*N, S]
        if pos_t is not None:
            allowed = (torch.arange(S, device=q.device) <= pos_t).view(1, 1, S)
            scores = scores.masked_fill(~allowed, float("-inf"))
        elif N > 1 or tree_mask is not None:
            j = torch.arange(S, device=q.device).view(1, S)
            i = torch.arange(N, device=q.device).view(N, 1)
            allowed = j <= (start + i)  # causal
            if tree_mask is not None:
                new = j >= start
                tm = torch.zeros((N, S), dtype=torch.bool, device=q.device)
                tm[:, start:start + N] = tree_mask.to(torch.bool)
                allowed = torch.where(new, tm, allowed)
            allowed = allowed.view(1, 1, N, S).expand(kvh, rep, N, S).reshape(kvh, rep * N, S)
            scores = scores.masked_fill(~allowed, float("-inf"))
        probs = torch.softmax(scores, dim=-1)
        out = torch.matmul(probs, vals)  # [kvh, rep*N, hd]
        return out.view(kvh, rep, N, hd).permute(2, 0, 1, 3).reshape(N, kvh * rep * hd)

    def _attention_hip(self, q, k, v, kc, vc, start: int, pos_t: Optional[torch.Tensor]):
        from . import _lib
        c = self.config
        out = torch.empty((1, c.num_attention_heads * c.head_dim), dtype=torch.float32, device=q.device)
        q, k, v = (t.to(torch.float32).contiguous() for t in (q, k, v))
        rc = _lib.load().lbk_attention_decode(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), c.num_attention_heads,
            c.num_key_value_heads, c.head_dim, self.max_seq_len, None if pos_t is None else pos_t.data_ptr(),
            int(start), float(c.attn_scale), self._attn_part.data_ptr(), self._attn_part.numel() * 4, out.data_ptr(),
            torch.cuda.current_stream(q.device).cuda_stream)
        _lib.check(rc, "lbk_attention_decode")
        return out

    def _attention_partials(self, li: int, q, k, v, start: int, pos_t: Optional[torch.Tensor]):
        """One token's attention stopped at its per-chunk partials, for the
        o projection to merge (``lbk_attention_decode`` without an output)."""
        from . import _lib
        from .ops import AttentionPartials
        c = self.config
        q, k, v = (t.to(torch.float32).contiguous() for t in (q, k, v))
        rc = _lib.load().lbk_attention_decode(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), self.k_cache[li].data_ptr(), self.v_cache[li].data_ptr(),
            c.num_attention_heads, c.num_key_value_heads, c.head_dim, self.max_seq_len,
            None if pos_t is None else pos_t.data_ptr(), int(start), float(c.attn_scale), self._attn_part.data_ptr(),
            self._attn_part.numel() * 4, None, torch.cuda.current_stream(q.device).cuda_stream)
        _lib.check(rc, "lbk_attention_decode")
        return AttentionPartials(self._attn_part, c.head_dim, self.max_seq_len, pos_t, int(start))

    def _attention_batch_hip(self, q, k, v, kc, vc, start: int, tree_mask: Optional[torch.Tensor],
                             pos_t: Optional[torch.Tensor] = None):
        """N new tokens in one launch pair (causal or ``tree_mask``); with
        ``pos_t`` the start is read on the device (graph-capturable)."""
        from . import _lib
        c = self.config
        N = q.shape[0]
        lib = _lib.load()
        grid_start = self.max_seq_len - N if pos_t is not None else int(start)
        need = int(lib.lbk_attention_batch_partial_bytes(c.num_attention_heads, N, grid_start, c.head_dim))
        if self._batch_part is None or self._batch_part.numel() * 4 < need:
            self._batch_part = torch.empty(max(need // 4, 1), dtype=torch.float32, device=q.device)
        out = torch.empty((N, c.num_attention_heads * c.head_dim), dtype=torch.float32, device=q.device)
        q, k, v = (t.to(torch.float32).contiguous() for t in (q, k, v))
        tm = None
        if tree_mask is not None:  # forward_hidden converts it once for all layers
            tm = tree_mask.to(device=q.device, dtype=torch.uint8).contiguous()
        rc = lib.lbk_attention_batch(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), N, c.num_attention_heads,
            c.num_key_value_heads, c.head_dim, self.max_seq_len, None if pos_t is None else pos_t.data_ptr(),
            int(start), None if tm is None else tm.data_ptr(),
            float(c.attn_scale), self._batch_part.data_ptr(), self._batch_part.numel() * 4, out.data_ptr(),
            torch.cuda.current_stream(q.device).cuda_stream)
        _lib.check(rc, "lbk_attention_batch")
        return out

    def forward_hidden(self, x: torch.Tensor, start: int, length: Optional[int] = None,
                       pos_t: Optional[torch.Tensor] = None,
                       tree_mask: Optional[torch.Tensor] = None, final_norm: bool = True) -> torch.Tensor:
        """x [N, hidden] fp32 at positions start.. -> final-norm hidden [N, hidden]
        (``final_norm=False``: the residual stream before the final RMSNorm,
        for a consumer that applies it, such as :class:`Q4LMHead`)."""
        eps = self.config.rms_norm_eps
        if length is None and pos_t is None:
            length = start + x.shape[0]
        if not self.fuse:
            for li, L in enumerate(self.layers):
                h = rms_norm(x, L["ln1"], eps)
                q, k, v = L["qkv"].forward(h)
                a = self._attention(li, q, k, v, start, length, pos_t, tree_mask)
                x = x + L["o"].forward(a)
                h = rms_norm(x, L["ln2"], eps)
                g, u = L["gate_up"].forward(h)
                x = x + L["down"].forward(F.silu(g) * u)
            return rms_norm(x, self.final_norm, eps) if final_norm else x
        # the norms, SiLU * up and the residual adds run inside the projection
        # calls; x (a private copy) is updated in place by o and down
        merge = x.shape[0] == 1 and tree_mask is None and self._hip_attn
        if merge:
            return self._forward_one_chained(x, start, pos_t, final_norm)
        x = x.to(torch.float32).clone()
        if tree_mask is not None and self._hip_attn:
            # the batched attention kernel reads the mask as bytes: convert it
            # once here rather than in every layer (a copy launch per layer)
            tree_mask = tree_mask.to(device=x.device, dtype=torch.uint8).contiguous()
        for li, L in enumerate(self.layers):
            q, k, v = L["qkv"].forward(x, rms_weight=L["ln1"], rms_eps=eps)
            if merge:  # o reads the attention's per-chunk partials and merges them itself
                L["o"].forward(None, out=x, residual=x, attn=self._attention_partials(li, q, k, v, start, pos_t))
            else:
                a = self._attention(li, q, k, v, start, length, pos_t, tree_mask)
                L["o"].forward(a, out=x, residual=x)
            g, u = L["gate_up"].forward(x, rms_weight=L["ln2"], rms_eps=eps)
            L["down"].forward(g, out=x, residual=x, x_up=u)
        return rms_norm(x, self.final_norm, eps) if final_norm else x

    def _chain_buffers(self):
        """Persistent one-row buffers and, per layer, the chain o -> gate/up ->
        down -> next layer's q/k/v (the last layer's ends at down), made once:
        the chains are bound to these buffers."""
        if self._chains is not None:
            return
        from .ops import ChainLink, LittleBitChain
        c, dev = self.config, self.device
        z = lambda n: torch.zeros((1, n), dtype=torch.float32, device=dev)  # noqa: E731
        L0 = self.layers[0]
        self._cx = z(c.hidden_size)
        self._cq, self._ck, self._cv = (z(p.out_features) for p in L0["qkv"].projections)
        self._cg, self._cu = (z(p.out_features) for p in L0["gate_up"].projections)
        eps = c.rms_norm_eps
        chains = []
        for li, L in enumerate(self.layers):
            links = [ChainLink(L["o"], [self._cx], residuals=[self._cx]),
                     ChainLink(L["gate_up"], [self._cg, self._cu], rms_weight=L["ln2"], rms_eps=eps),
                     ChainLink(L["down"], [self._cx], residuals=[self._cx], silu_mul=True)]
            if li + 1 < len(self.layers):
                nx = self.layers[li + 1]
                links.append(ChainLink(nx["qkv"], [self._cq, self._ck, self._cv], rms_weight=nx["ln1"], rms_eps=eps))
            chains.append(LittleBitChain(links))
        self._chains = chains

    def _forward_one_chained(self, x: torch.Tensor, start: int, pos_t: Optional[torch.Tensor],
                             final_norm: bool) -> torch.Tensor:
        """One token: layer 0's q/k/v, then per layer the attention (stopped at
        its partials) and one chain from o through the next layer's q/k/v,
        which runs the layer's calls in one launch per call boundary
        (lbk_chain_forward; the reference's full_forward runs a layer as one
        call, patches/littlebit_cpu_optimized.cpp:1627-1833)."""
        self._chain_buffers()
        eps = self.config.rms_norm_eps
        self._cx.copy_(x.reshape(1, -1))
        L0 = self.layers[0]
        L0["qkv"].forward(self._cx, outs=[self._cq, self._ck, self._cv], rms_weight=L0["ln1"], rms_eps=eps)
        for li, chain in enumerate(self._chains):
            chain.forward(attn=self._attention_partials(li, self._cq, self._ck, self._cv, start, pos_t))
        return rms_norm(self._cx, self.final_norm, eps) if final_norm else self._cx.clone()

    def forward_batch(self, token_ids: Sequence[int], embed_tokens: torch.Tensor,
                      tree_mask: Optional[torch.Tensor] = None, final_norm: bool = True) -> torch.Tensor:
        """N tokens at positions cache_pos.. (causal, or ``tree_mask``);
        advances cache_pos by N.  Returns final-norm hidden [N, hidden]
        (the reference's _LBModelUnit.forward_batch, cpu_target_model.py:325-368)."""
        n = len(token_ids)
        if n == 0:
            return torch.empty((0, self.config.hidden_size), device=self.device)
        if self.cache_pos + n > self.max_seq_len:
            raise RuntimeError(f"KV cache full: {self.cache_pos} + {n} > max_seq_len {self.max_seq_len}")
        ids = torch.as_tensor(list(token_ids), dtype=torch.long, device=self.device)
        x = embed_tokens.index_select(0, ids).to(torch.float32)
        out = self.forward_hidden(x, self.cache_pos, tree_mask=tree_mask, final_norm=final_norm)
        self.cache_pos += n
        return out

    def forward_token(self, token_id: int, embed_tokens: torch.Tensor, final_norm: bool = True) -> torch.Tensor:
        """One token; returns final-norm hidden [1, hidden] (cpu_target_model.py:240-323)."""
        return self.forward_batch([token_id], embed_tokens, final_norm=final_norm)


def _embed_and_head(state: Dict[str, torch.Tensor], dev, embed_tokens, lm_head_weight, base_model_id, dtype):
    """Embedding and lm_head: given tensors, else the runtime state's own
    ``model.embed_tokens.weight`` / ``lm_head.weight``, else the base model
    (cpu_draft_model.py:181-197), read from local files only."""
    if embed_tokens is None and "model.embed_tokens.weight" in state:
        embed_tokens = state["model.embed_tokens.weight"]
    if lm_head_weight is None and "lm_head.weight" in state:
        lm_head_weight = state["lm_head.weight"]
    if embed_tokens is None or lm_head_weight is None:
        if base_model_id is None:
            raise ValueError("embed_tokens / lm_head_weight not given and not in the runtime state; "
                             "pass them or a locally available base_model_id")
        from transformers import AutoModelForCausalLM
        base = AutoModelForCausalLM.from_pretrained(base_model_id, torch_dtype=torch.float32, device_map="cpu",
                                                    low_cpu_mem_usage=True, local_files_only=True)
        if embed_tokens is None:
            embed_tokens = base.model.embed_tokens.weight.data
        if lm_head_weight is None:
            lm_head_weight = base.lm_head.weight.data
        del base
    return (embed_tokens.to(dev, torch.float32).contiguous(),
            lm_head_weight.to(dev, dtype).contiguous())


def _load_state(runtime_path, state, config):
    if state is None:
        if runtime_path is None:
            raise ValueError("give runtime_path or state")
        state, _ = load_runtime_checkpoint(runtime_path, device="cpu")
    if config is None:
        if runtime_path is None:
            raise ValueError("give config with an in-memory state")
        config = DecoderConfig.from_file(Path(runtime_path) / "dummy_llama3_config.json")
    elif isinstance(config, dict):
        config = DecoderConfig.from_dict(config)
    return state, config


class GPUDraftModel:
    """GPU counterpart of CPUDraftModel (cpu_draft_model.py:141-593).

    ``generate_draft_tokens`` returns the same structures (lists of [1, 1]
    token tensors and [1, 1, vocab] probabilities) and leaves the cache at
    the prompt boundary: the last prompt token's KV stays committed, the
    draft positions are rolled back (:586-591).  With ``use_graph`` the
    one-token step (embedding, all layers, final norm, lm_head, argmax) is a
    HIP graph that feeds its argmax back as the next input, so greedy drafts
    run without host round trips; attention then spans the whole cache with
    later positions masked, so size ``max_seq_len`` to the context.

    ``lm_head="q4"`` (the default) is the reference's C++ draft path
    (generate_token, cpu_draft_model.py:485-563): the lm_head quantised to
    Q4_0, the hidden state to Q8_0, the token their argmax, the returned
    probabilities one-hot at it, whatever ``greedy`` and ``temperature`` say.
    ``lm_head="dense"`` is its Python fallback (:565-584): ``F.linear`` in
    ``torch_dtype``, softmax probabilities, greedy or sampled tokens.
    """

    def __init__(self, runtime_path: Optional[str] = None, base_model_id: Optional[str] = None,
                 torch_dtype=torch.float32, *, state: Optional[Dict[str, torch.Tensor]] = None,
                 config=None, embed_tokens: Optional[torch.Tensor] = None,
                 lm_head_weight: Optional[torch.Tensor] = None, device="cuda", max_seq_len: int = 4096,
                 use_graph: bool = True, lm_head: str = "q4"):
        if lm_head not in ("q4", "dense"):
            raise ValueError(f"lm_head must be 'q4' or 'dense', got {lm_head!r}")
        state, config = _load_state(runtime_path, state, config)
        dev = torch.device(device)
        self.config = config
        self.device = dev
        self.max_seq_len = int(max_seq_len)
        self.lm_head_mode = lm_head
        self.unit = LittleBitDecoder(state, config, dev, max_seq_len, residual=False)
        q4 = lm_head == "q4"
        self.embed_tokens, head = _embed_and_head(state, dev, embed_tokens, lm_head_weight, base_model_id,
                                                  torch.float32 if q4 else torch_dtype)
        self._vocab_size = int(head.shape[0])
        self._q4 = None
        self.lm_head_weight = None
        if q4:
            from .lm_head import Q4LMHead
            self._q4 = Q4LMHead(head)  # quantised from the fp32 weight, which is then dropped
            del head
        else:
            self.lm_head_weight = head
        self._cache_pos = 0
        self._cached_seq_len = 0
        self._last_hidden = None
        self._prompt_hidden = None
        self.use_graph = bool(use_graph)
        self._graph = None

    # ------------------------------------------------------------------ internals
    def reset(self):
        self._cache_pos = 0
        self._cached_seq_len = 0
        self._last_hidden = None
        self._prompt_hidden = None  # final hidden of the last cached prompt token

    def _lm_head(self, hidden: torch.Tensor) -> torch.Tensor:
        return F.linear(hidden.to(self.lm_head_weight.dtype), self.lm_head_weight).to(torch.float32)

    def _head_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        """Logits [1, vocab] fp32 of a final hidden state as this model holds
        it (before the final norm with the Q4_0 head, after it with dense)."""
        if self._q4 is None:
            return self._lm_head(hidden)
        logits = torch.empty((1, self._vocab_size), dtype=torch.float32, device=self.device)
        self._q4.argmax(hidden, self.unit.final_norm, self.config.rms_norm_eps, logits=logits)
        return logits

    def _q4_token(self, hidden: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Token of a pre-norm hidden state: final RMSNorm, Q8_0, Q4_0 logits,
        argmax (generate_token's tail, patch:2276-2314), on the device."""
        return self._q4.argmax(hidden, self.unit.final_norm, self.config.rms_norm_eps, out=out)

    @torch.no_grad()
    def _forward_token(self, token_id: int) -> torch.Tensor:
        """One token at _cache_pos (committed); returns final hidden [1, hidden]
        (before the final norm with the Q4_0 head, which applies it)."""
        self.unit.cache_pos = self._cache_pos
        h = self.unit.forward_token(token_id, self.embed_tokens, final_norm=self._q4 is None)
        self._cache_pos += 1
        self._last_hidden = h
        return h

    def _build_graph(self):
        dev = self.device
        self._tok = torch.zeros(1, dtype=torch.long, device=dev)
        self._pos = torch.zeros(1, dtype=torch.long, device=dev)
        if self._q4 is None:
            self._out_tok = torch.zeros(1, dtype=torch.long, device=dev)
            self._out_logits = torch.zeros((1, self._vocab_size), dtype=torch.float32, device=dev)
        stream = torch.cuda.Stream(device=dev)

        def step():
            x = self.embed_tokens.index_select(0, self._tok)
            if self._q4 is not None:  # norm, Q4_0 head and argmax in two launches; the token is the next input
                h = self.unit.forward_hidden(x, 0, pos_t=self._pos, final_norm=False)
                self._q4_token(h, out=self._tok)
            else:
                h = self.unit.forward_hidden(x, 0, pos_t=self._pos)
                logits = self._lm_head(h)
                self._out_logits.copy_(logits)
                nxt = torch.argmax(logits, dim=-1)
                self._out_tok.copy_(nxt)
                self._tok.copy_(nxt)
            self._pos.add_(1)

        # The warm run really executes: it writes KV at _pos, so it runs at
        # the first uncommitted position (the draft positions are scratch).
        if self._cache_pos >= self.max_seq_len:
            raise RuntimeError("KV cache full")
        self._pos.fill_(self._cache_pos)
        stream.wait_stream(torch.cuda.current_stream(dev))
        # the graph's calls run on a workspace of its own: replays may run on
        # any stream, concurrently with eager calls on the pooled workspaces
        self._graph_ws = PrivateWorkspace()
        with private_workspace(self._graph_ws):
            with torch.cuda.stream(stream):
                step()  # warm: sizes the graph's workspace before capture
            stream.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                step()
        torch.cuda.synchronize(dev)
        self._graph = g

    # ------------------------------------------------------------------ API
    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor):
        """Cache the prompt's KV; only positions not yet cached are computed
        (cpu_draft_model.py:437-461).  A prompt that repeats the cached one
        is not recomputed (the reference's Python path resets then, its C++
        path does not); a shorter prompt resets the cache."""
        seq_len = int(input_ids.shape[1])
        if self._cached_seq_len > 0 and seq_len >= self._cached_seq_len and self._prompt_hidden is not None:
            start = self._cached_seq_len  # extends (or repeats) the cached prompt
        else:
            self.reset()
            start = 0
        ids = input_ids[0, start:seq_len].tolist()
        if ids:
            self.unit.cache_pos = start
            h = self.unit.forward_batch(ids, self.embed_tokens, final_norm=self._q4 is None)
            self._prompt_hidden = h[-1:].contiguous()
        self._last_hidden = self._prompt_hidden
        self._cache_pos = seq_len
        self._cached_seq_len = seq_len

    @torch.no_grad()
    def generate_draft_tokens(self, input_ids: torch.Tensor, attention_mask=None, draft_length: int = 5,
                              temperature: float = 1.0, greedy: bool = True):
        """K draft tokens after ``input_ids`` (cpu_draft_model.py:463-593)."""
        seq_len = int(input_ids.shape[1])
        if self._cached_seq_len > seq_len:
            self.reset()
        self.prefill(input_ids)
        cache_pos_before_draft = self._cache_pos
        tokens: List[torch.Tensor] = []
        probs: List[torch.Tensor] = []
        if draft_length > 0 and self._q4 is not None:
            # generate_token per draft position: argmax of the Q4_0 logits,
            # one-hot probabilities (cpu_draft_model.py:526-563)
            if self._cache_pos + draft_length > self.max_seq_len:
                raise RuntimeError("KV cache full")
            first = self._q4_token(self._last_hidden)
            outs = [first.clone()]
            if draft_length > 1 and self.use_graph:
                if self._graph is None:
                    self._build_graph()
                self._tok.copy_(first)
                self._pos.fill_(self._cache_pos)
                for _ in range(draft_length - 1):
                    self._graph.replay()
                    outs.append(self._tok.clone())
                toks = torch.cat(outs).cpu().tolist()
            else:
                toks = [int(first.item())]
                for _ in range(draft_length - 1):
                    toks.append(int(self._q4_token(self._forward_token(toks[-1])).item()))
            for t in toks:
                tokens.append(torch.tensor([[t]], dtype=torch.long))
                p = torch.zeros(1, self._vocab_size)
                p[0, t] = 1.0
                probs.append(p.unsqueeze(0))
        elif draft_length > 0 and greedy and self.use_graph:
            if self._cache_pos + draft_length > self.max_seq_len:
                raise RuntimeError("KV cache full")
            if self._graph is None:
                self._build_graph()
            # the prompt's last hidden gives the first token; each replay then
            # embeds that token, runs the layers at _pos and predicts the next
            logits = self._lm_head(self._last_hidden)
            first = torch.argmax(logits, dim=-1)
            outs_t, outs_l = [first.clone()], [logits]
            self._tok.copy_(first)
            self._pos.fill_(self._cache_pos)
            for _ in range(draft_length - 1):
                self._graph.replay()
                outs_t.append(self._out_tok.clone())
                outs_l.append(self._out_logits.clone())
            toks = torch.stack(outs_t).view(-1).cpu().tolist()
            for t, lg in zip(toks, outs_l):
                tokens.append(torch.tensor([[t]], dtype=torch.long))
                probs.append(F.softmax(lg / max(temperature, 1e-8), dim=-1).unsqueeze(0))
        else:
            last_hidden = self._last_hidden
            for k in range(draft_length):
                logits = self._lm_head(last_hidden)
                p = F.softmax(logits / max(temperature, 1e-8), dim=-1)
                if greedy:
                    nxt = torch.argmax(logits, dim=-1, keepdim=True)
                else:
                    nxt = torch.multinomial(p, num_samples=1)
                tokens.append(nxt.cpu())
                probs.append(p.unsqueeze(0))
                if k + 1 < draft_length:
                    last_hidden = self._forward_token(int(nxt.item()))
        self._cache_pos = cache_pos_before_draft
        self._cached_seq_len = seq_len
        self._last_hidden = self._prompt_hidden
        return tokens, probs


class GPUTargetModel:
    """GPU counterpart of CPUTargetModel (cpu_target_model.py:371-556).

    Two model units -- the draft checkpoint and the residual checkpoint --
    whose final hidden states are summed before one lm_head.  With
    ``residual_runtime_path=None`` (or ``residual_state=None``) a single unit
    uses the projections' in-module residual branches instead (the 1.0-BPW
    target as draft + residual factors per projection).
    """

    def __init__(self, draft_runtime_path: Optional[str] = None, residual_runtime_path: Optional[str] = None,
                 base_model_id: Optional[str] = None, torch_dtype=torch.float32, *,
                 draft_state: Optional[Dict[str, torch.Tensor]] = None,
                 residual_state: Optional[Dict[str, torch.Tensor]] = None, config=None,
                 embed_tokens: Optional[torch.Tensor] = None, lm_head_weight: Optional[torch.Tensor] = None,
                 device="cuda", max_seq_len: int = 4096):
        draft_state, config = _load_state(draft_runtime_path, draft_state, config)
        dev = torch.device(device)
        self.config = config
        self.device = dev
        two_units = residual_runtime_path is not None or residual_state is not None
        if two_units:
            residual_state, _ = _load_state(residual_runtime_path, residual_state, config)
            self.draft_unit = LittleBitDecoder(draft_state, config, dev, max_seq_len, residual=False)
            self.residual_unit = LittleBitDecoder(residual_state, config, dev, max_seq_len, residual=False)
            self.units = [self.draft_unit, self.residual_unit]
        else:
            self.draft_unit = LittleBitDecoder(draft_state, config, dev, max_seq_len, residual=None)
            self.residual_unit = None
            self.units = [self.draft_unit]
        self.embed_tokens, self.lm_head_weight = _embed_and_head(draft_state, dev, embed_tokens, lm_head_weight,
                                                                 base_model_id, torch_dtype)
        self._vocab_size = int(self.lm_head_weight.shape[0])
        self._cached_tokens: Optional[List[int]] = None

    def reset_cache(self):
        for u in self.units:
            u.reset()
        self._cached_tokens = None

    def _logits(self, ids: List[int], tree_mask=None) -> torch.Tensor:
        hidden = None
        for u in self.units:
            h = u.forward_batch(ids, self.embed_tokens, tree_mask=tree_mask)
            hidden = h if hidden is None else hidden + h
        return F.linear(hidden.to(self.lm_head_weight.dtype), self.lm_head_weight).to(torch.float32)

    def _common_prefix(self, ids: List[int]) -> int:
        common = 0
        if self._cached_tokens is not None:
            for a, b in zip(ids, self._cached_tokens):
                if a != b:
                    break
                common += 1
        return common

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, attention_mask=None) -> torch.Tensor:
        """(1, seq_len, vocab) logits; rows of the reused prefix are zero
        (cpu_target_model.py:467-556).  attention_mask is ignored, as there."""
        ids = input_ids[0].tolist()
        seq_len = len(ids)
        common = self._common_prefix(ids)
        for u in self.units:
            u.cache_pos = common
        n_new = seq_len - common
        out = torch.zeros((1, seq_len, self._vocab_size), dtype=torch.float32, device=self.device)
        if n_new > 0:
            out[0, common:] = self._logits(ids[common:])
        self._cached_tokens = ids
        return out

    @torch.no_grad()
    def forward_tree(self, prefix_ids: torch.Tensor, tree_tokens: Sequence[int],
                     tree_mask: torch.Tensor) -> torch.Tensor:
        """Logits [T, vocab] of a token tree whose root (node 0) is the last
        prefix token: ``tree_tokens`` [T] and ``tree_mask`` [T, T] (the
        ancestor mask of :func:`littlebit_amd.tree.generate_tree_buffers`).
        Row 0 predicts the first tree level.  The prefix is cached as in
        :meth:`forward`; the nodes' positions are dropped afterwards."""
        ids = prefix_ids[0].tolist()
        P = len(ids)
        tree_tokens = [int(t) for t in tree_tokens]
        if P < 1 or tree_tokens[0] != ids[-1]:
            raise ValueError("the tree root must be the last prefix token")
        common = min(self._common_prefix(ids), P - 1)
        for u in self.units:
            u.cache_pos = common
            if P - 1 > common:
                u.forward_batch(ids[common:P - 1], self.embed_tokens)
        logits = self._logits(tree_tokens, tree_mask=tree_mask)
        for u in self.units:
            u.cache_pos = P  # the root's KV (the last prefix token) stays
        self._cached_tokens = ids
        return logits

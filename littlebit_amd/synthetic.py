"""Seeded synthetic LittleBit projections for the benchmark configurations.

Distributions: x ~ N(0, 1); signs Bernoulli(0.5) -> +-1, packed along the
reduction dimension with the reference rule (LSB first, bit 1 == -1, pad 0);
scales g, l, h = |N(0, 1)| + 0.05.  Generator: numpy PCG64 with
seed = 1000 + config index.  Draw order per branch: V signs, U signs, g, l, h
(x is drawn first by the caller).

``direct_words=True`` draws the packed words themselves (uniform 32-bit words
with the pad bits cleared), which is the same distribution and is what the
benchmark uses for multi-hundred-MB models.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

__all__ = [
    "HostBranch",
    "pack_signs_np",
    "random_words",
    "make_branch",
    "make_projection",
    "config_seed",
    "LLAMA2_7B",
    "llama_projection_shapes",
    "synthetic_runtime_state",
]


def config_seed(index: int) -> int:
    return 1000 + int(index)


def pack_signs_np(signs: np.ndarray) -> np.ndarray:
    """int8 {-1,+1} [rows, cols] -> int32 words [rows, ceil(cols/32)] (LSB first, bit 1 == -1)."""
    rows, cols = signs.shape
    wpr = (cols + 31) // 32
    bits = np.zeros((rows, wpr * 32), dtype=np.uint8)
    bits[:, :cols] = signs < 0
    packed = np.packbits(bits, axis=1, bitorder="little")  # bytes, LSB first
    return np.ascontiguousarray(packed).view("<u4").view(np.int32).reshape(rows, wpr)


def random_words(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """Uniform packed sign words with pad bits (columns >= cols) cleared."""
    wpr = (cols + 31) // 32
    w = rng.integers(0, 2**32, size=(rows, wpr), dtype=np.uint32)
    tail = cols - 32 * (wpr - 1)
    if tail < 32:
        w[:, -1] &= np.uint32((1 << tail) - 1)
    return w.view(np.int32)


@dataclass
class HostBranch:
    v_sign: np.ndarray  # int32 [R, ceil(K/32)]
    u_sign: np.ndarray  # int32 [N, ceil(R/32)]
    g: np.ndarray       # fp32 [K]   (v2)
    l: np.ndarray       # fp32 [R]   (mid)
    h: np.ndarray       # fp32 [N]   (u1)
    R: int

    def as_dict(self) -> Dict:
        return {"v_sign": self.v_sign, "u_sign": self.u_sign, "g": self.g, "l": self.l,
                "h": self.h, "R": self.R}

    @property
    def nbytes(self) -> int:
        return int(self.v_sign.nbytes + self.u_sign.nbytes + self.g.nbytes + self.l.nbytes + self.h.nbytes)


def _scales(rng: np.random.Generator, n: int) -> np.ndarray:
    return (np.abs(rng.standard_normal(n)) + 0.05).astype(np.float32)


def make_branch(rng: np.random.Generator, K: int, R: int, N: int, direct_words: bool = False) -> HostBranch:
    if direct_words:
        v = random_words(rng, R, K)
        u = random_words(rng, N, R)
    else:
        v = pack_signs_np((1 - 2 * rng.integers(0, 2, size=(R, K))).astype(np.int8))
        u = pack_signs_np((1 - 2 * rng.integers(0, 2, size=(N, R))).astype(np.int8))
    g = _scales(rng, K)
    l = _scales(rng, R)
    h = _scales(rng, N)
    return HostBranch(v, u, g, l, h, int(R))


def make_projection(seed: int, M: int, K: int, N: int, ranks: List[int],
                    x_dtype=np.float32, direct_words: bool = False):
    """x [M, K] then one branch per rank, from one PCG64 stream."""
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_normal((M, K)).astype(np.float32).astype(x_dtype)
    branches = [make_branch(rng, K, R, N, direct_words) for R in ranks]
    return x, branches


# Llama-2-7B shapes and the 0.1-BPW ranks of the draft, plus
# the residual ranks that make the ~1.0-BPW target.
LLAMA2_7B = {
    "hidden": 4096,
    "intermediate": 11008,
    "layers": 32,
    "heads": 32,
    "kv_heads": 32,
    "vocab": 32000,
    "draft_rank": {"attn": 205, "mlp": 298},
    "residual_rank": {"attn": 1843, "mlp": 2686},
}


def llama_projection_shapes(cfg: Optional[Dict] = None, residual: bool = False):
    """[(name, K, N, ranks)] for the 7 projections of one decoder layer."""
    cfg = cfg or LLAMA2_7B
    H, I = cfg["hidden"], cfg["intermediate"]
    ra, rm = cfg["draft_rank"]["attn"], cfg["draft_rank"]["mlp"]
    qa, qm = cfg["residual_rank"]["attn"], cfg["residual_rank"]["mlp"]
    kv = H * cfg["kv_heads"] // cfg["heads"]
    out = []
    for name, K, N, r, rr in (
        ("q_proj", H, H, ra, qa),
        ("k_proj", H, kv, ra, qa),
        ("v_proj", H, kv, ra, qa),
        ("o_proj", H, H, ra, qa),
        ("gate_proj", H, I, rm, qm),
        ("up_proj", H, I, rm, qm),
        ("down_proj", I, H, rm, qm),
    ):
        out.append((name, K, N, [r, rr] if residual else [r]))
    return out


def synthetic_runtime_state(config, draft_ranks: Dict[str, int], residual_ranks: Optional[Dict[str, int]] = None,
                            seed: int = 0, device="cpu", normalized: bool = False, embed: bool = True):
    """A runtime-layout state dict (convert_hf_to_runtime.py key names) of a
    random LittleBit Llama model: packed sign words, scales |N(0,1)| + 0.05,
    norm weights 1 + 0.1 N(0,1), and (``embed``) ``model.embed_tokens.weight``
    and ``lm_head.weight`` ~ N(0, 1).

    ``draft_ranks`` / ``residual_ranks`` map "attn" / "mlp" to ranks;
    ``residual_ranks`` adds in-module residual branches (``_r`` keys).
    ``normalized`` divides g by sqrt(K) and l by sqrt(R) so that every
    projection maps unit-RMS inputs to O(1) outputs (keeps attention scores
    moderate for numerical comparisons); the benchmark leaves it off.
    """
    import torch

    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(int(seed))
    c = config
    kv = c.num_key_value_heads * c.head_dim
    shapes = {"self_attn.q_proj": (c.hidden_size, c.hidden_size, "attn"),
              "self_attn.k_proj": (c.hidden_size, kv, "attn"),
              "self_attn.v_proj": (c.hidden_size, kv, "attn"),
              "self_attn.o_proj": (c.hidden_size, c.hidden_size, "attn"),
              "mlp.gate_proj": (c.hidden_size, c.intermediate_size, "mlp"),
              "mlp.up_proj": (c.hidden_size, c.intermediate_size, "mlp"),
              "mlp.down_proj": (c.intermediate_size, c.hidden_size, "mlp")}

    def words(rows, cols):
        wpr = (cols + 31) // 32
        w = torch.randint(-2**31, 2**31, (rows, wpr), generator=gen, dtype=torch.int64, device=dev)
        tail = cols - 32 * (wpr - 1)
        if tail < 32:
            w[:, -1] &= (1 << tail) - 1
        return w.to(torch.int32)

    def scales(n, div=1.0):
        return ((torch.randn(n, generator=gen, device=dev).abs() + 0.05) / div).reshape(1, n)

    state = {}
    for i in range(c.num_hidden_layers):
        for name, (K, N, kind) in shapes.items():
            p = f"model.layers.{i}.{name}"
            for tag, sfx, ranks in (("", "", draft_ranks), ("_r", "_r", residual_ranks)):
                if ranks is None:
                    continue
                R = int(ranks[kind])
                state[f"{p}.v_sign{tag}_rt"] = words(R, K)
                state[f"{p}.v_sign{tag}_rt_shape"] = torch.tensor([R, K], dtype=torch.int64)
                state[f"{p}.u_sign{tag}_rt"] = words(N, R)
                state[f"{p}.u_sign{tag}_rt_shape"] = torch.tensor([N, R], dtype=torch.int64)
                state[f"{p}.v2{sfx}"] = scales(K, K ** 0.5 if normalized else 1.0)
                state[f"{p}.mid{sfx}"] = scales(R, R ** 0.5 if normalized else 1.0)
                state[f"{p}.u1{sfx}"] = scales(N)
        for nm in ("input_layernorm", "post_attention_layernorm"):
            state[f"model.layers.{i}.{nm}.weight"] = 1 + 0.1 * torch.randn(c.hidden_size, generator=gen, device=dev)
    state["model.norm.weight"] = 1 + 0.1 * torch.randn(c.hidden_size, generator=gen, device=dev)
    if embed:
        state["model.embed_tokens.weight"] = torch.randn((c.vocab_size, c.hidden_size), generator=gen, device=dev)
        state["lm_head.weight"] = torch.randn((c.vocab_size, c.hidden_size), generator=gen, device=dev)
    return state

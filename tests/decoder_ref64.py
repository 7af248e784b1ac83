"""A float64 reference decoder in torch, for checks at the full Llama-2-7B
size where the numpy oracle decoder (``test_decode_gpu.ref_hidden``) would
take minutes: the same layer (full_forward_cpu,
patches/littlebit_cpu_optimized.cpp:1522-1840: RMSNorm, q/k/v, GQA attention
without rotary embedding, o + residual, RMSNorm, SiLU(gate) * up, down +
residual, final RMSNorm) and the same projection formula as
``oracle.littlebit_oracle.littlebit_forward`` (littlebit.py:114-121), in
float64 on any torch device.  Sign words are unpacked with torch bit
operations (bit c % 32 of word c // 32, bit 1 = -1), not with the library.

Test infrastructure only; pinned against the numpy oracle decoder by
tests/test_decoder_ref64.py.
"""
from __future__ import annotations

import torch


def unpack_pm1(words: torch.Tensor, cols: int) -> torch.Tensor:
    """int32 words [rows, ceil(cols/32)] -> float64 +-1 [rows, cols]."""
    w = words.to(torch.int64) & 0xFFFFFFFF
    sh = torch.arange(32, device=words.device, dtype=torch.int64)
    bits = ((w.unsqueeze(-1) >> sh) & 1).reshape(words.shape[0], -1)[:, :cols]
    return (1 - 2 * bits).to(torch.float64)


def _branches(state, p, residual, dev):
    out = []
    for tag, sfx in (("", ""), ("_r", "_r")):
        if f"{p}.u_sign{tag}_rt" not in state or (tag and not residual):
            continue
        out.append(tuple(state[k].to(dev) for k in (f"{p}.v_sign{tag}_rt", f"{p}.u_sign{tag}_rt", f"{p}.v2{sfx}",
                                                   f"{p}.mid{sfx}", f"{p}.u1{sfx}")))
    return out


def linear64(x: torch.Tensor, branches, K: int, N: int) -> torch.Tensor:
    """sum_b h_b * (U_b . (l_b * (V_b^T . (g_b * x)))) in float64; x [n, K]."""
    y = torch.zeros((x.shape[0], N), dtype=torch.float64, device=x.device)
    for v, u, g, l, h in branches:
        R = v.shape[0]
        t = ((x * g.reshape(1, K).double()) @ unpack_pm1(v, K).T) * l.reshape(1, R).double()
        y += (t @ unpack_pm1(u, R).T) * h.reshape(1, N).double()
    return y


def ref_hidden64(state, cfg, ids, residual: bool, device="cpu") -> torch.Tensor:
    """Final-norm hidden [n, H] (float64, on ``device``) of tokens ids from an
    empty cache, causal."""
    dev = torch.device(device)
    H, eps = cfg.hidden_size, cfg.rms_norm_eps
    kvh, hd, rep = cfg.num_key_value_heads, cfg.head_dim, cfg.kv_repeat

    def norm(x, key):
        w = state[key].to(dev).double().reshape(1, -1)
        return x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps) * w

    def lin(x, p, K, N):
        return linear64(x, _branches(state, p, residual, dev), K, N)

    ids_t = torch.as_tensor(list(ids), dtype=torch.long, device=dev)
    x = state["model.embed_tokens.weight"].to(dev).index_select(0, ids_t).double()
    n = len(ids)
    mask = torch.tril(torch.ones((n, n), dtype=torch.bool, device=dev))
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}"
        h = norm(x, f"{p}.input_layernorm.weight")
        q = lin(h, f"{p}.self_attn.q_proj", H, H).reshape(n, kvh, rep, hd)
        k = lin(h, f"{p}.self_attn.k_proj", H, kvh * hd).reshape(n, kvh, hd)
        v = lin(h, f"{p}.self_attn.v_proj", H, kvh * hd).reshape(n, kvh, hd)
        # scores [kvh, rep, n_q, n_k]
        s = torch.matmul(q.permute(1, 2, 0, 3), k.permute(1, 2, 0).unsqueeze(1).contiguous()) * cfg.attn_scale
        s = s.masked_fill(~mask, float("-inf"))
        s = torch.softmax(s, dim=-1)
        a = torch.matmul(s, v.permute(1, 0, 2).unsqueeze(1).contiguous())  # [kvh, rep, n, hd]
        a = a.permute(2, 0, 1, 3).reshape(n, H)
        x = x + lin(a, f"{p}.self_attn.o_proj", H, H)
        h = norm(x, f"{p}.post_attention_layernorm.weight")
        I = cfg.intermediate_size
        g = lin(h, f"{p}.mlp.gate_proj", H, I)
        u = lin(h, f"{p}.mlp.up_proj", H, I)
        x = x + lin(g / (1 + torch.exp(-g)) * u, f"{p}.mlp.down_proj", I, H)
    return norm(x, "model.norm.weight")

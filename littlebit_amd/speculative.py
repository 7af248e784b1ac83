"""Speculative decoding loops over the GPU draft and target models.

Same control flow and statistics as the reference's
``speculative_decode`` (speculative_decoding.py:240-398: draft K tokens,
verify them in one target forward, accept the longest agreeing prefix,
take the target's token at the first disagreement or a bonus token when all
K agree) and ``speculative_decode_tree`` (:454-617, greedy: verify a token
tree in one forward with the ancestor mask and accept the longest agreeing
root-to-leaf path).  With greedy decoding the output equals the target's
own greedy continuation, which the tests check.
"""
from __future__ import annotations

import time
from typing import Dict, Optional

import torch
import torch.nn.functional as F

from .tree import evaluate_posterior_greedy, generate_draft_tree

__all__ = ["speculative_decode", "speculative_decode_tree", "autoregressive_decode"]


@torch.no_grad()
def speculative_decode(draft_model, target_model, input_ids: torch.Tensor, attention_mask=None,
                       max_new_tokens: int = 256, draft_length: int = 5, temperature: float = 1.0,
                       greedy: bool = True, eos_token_id: int = 2, generator: Optional[torch.Generator] = None):
    input_ids = input_ids.cpu()
    generated = []
    total_draft = total_accepted = steps = 0
    current = input_ids
    t0 = time.time()
    while len(generated) < max_new_tokens:
        steps += 1
        k = min(draft_length, max_new_tokens - len(generated))
        d_tokens, d_probs = draft_model.generate_draft_tokens(current, None, draft_length=k,
                                                              temperature=temperature, greedy=greedy)
        d_ids = torch.cat(d_tokens, dim=1).cpu()
        verify = torch.cat([current, d_ids], dim=1)
        logits = target_model.forward(verify)  # (1, seq + k, vocab)
        seq_len = current.shape[1]
        accepted = 0
        stop = False
        for i in range(k):
            lg = logits[:, seq_len - 1 + i, :]
            tok = int(d_ids[0, i])
            if greedy:
                tgt = int(torch.argmax(lg, dim=-1))
                if tgt == tok:
                    accepted += 1
                    generated.append(tok)
                    if tok == eos_token_id:
                        stop = True
                        break
                else:
                    generated.append(tgt)
                    stop = tgt == eos_token_id
                    break
            else:
                p_t = F.softmax(lg / max(temperature, 1e-8), dim=-1)
                p_d = d_probs[i][0].to(p_t.device)
                ratio = float(p_t[0, tok]) / max(float(p_d[0, tok]), 1e-10)
                if float(torch.rand(1, generator=generator)) < min(1.0, ratio):
                    accepted += 1
                    generated.append(tok)
                    if tok == eos_token_id:
                        stop = True
                        break
                else:
                    res = torch.clamp(p_t - p_d, min=0)
                    res = res / (res.sum() + 1e-10)
                    tok2 = int(torch.multinomial(res.cpu(), 1, generator=generator))
                    generated.append(tok2)
                    stop = tok2 == eos_token_id
                    break
        if not stop and accepted == k and len(generated) < max_new_tokens:
            lg = logits[:, seq_len + k - 1, :]
            if greedy:
                generated.append(int(torch.argmax(lg, dim=-1)))
            else:
                p = F.softmax(lg / max(temperature, 1e-8), dim=-1).cpu()
                generated.append(int(torch.multinomial(p, 1, generator=generator)))
        total_draft += k
        total_accepted += accepted
        current = torch.cat([input_ids, torch.tensor([generated], dtype=torch.long)], dim=1)
        if generated[-1] == eos_token_id:
            break
    elapsed = time.time() - t0
    stats = _stats(generated, total_draft, total_accepted, steps, elapsed)
    stats["draft_length_k"] = draft_length
    return torch.cat([input_ids, torch.tensor([generated], dtype=torch.long)], dim=1), stats


@torch.no_grad()
def speculative_decode_tree(draft_model, target_model, input_ids: torch.Tensor, attention_mask=None,
                            max_new_tokens: int = 256, tree_buffers: Dict = None, top_k: int = 10,
                            eos_token_id: int = 2):
    """Greedy tree decoding: one draft tree and one target forward per step."""
    input_ids = input_ids.cpu()
    retrieve = tree_buffers["retrieve_indices"].cpu()
    mask = tree_buffers["tree_attn_mask"][0, 0]
    tree_len = tree_buffers["tree_len"]
    generated = []
    total_draft = total_accepted = steps = 0
    current = input_ids
    t0 = time.time()
    while len(generated) < max_new_tokens:
        steps += 1
        cand = generate_draft_tree(draft_model, current, tree_buffers, top_k=top_k)  # (1, T)
        logits = target_model.forward_tree(current, cand[0].tolist(), mask).cpu()    # (T, V)
        padded_c = torch.cat([cand, torch.full((1, 1), -1, dtype=torch.long)], dim=1)
        cart_c = padded_c[0, retrieve]
        padded_l = torch.cat([logits, torch.zeros((1, logits.shape[-1]))], dim=0)
        cart_l = padded_l[retrieve]
        best, acc, nxt = evaluate_posterior_greedy(cart_l, cart_c)
        stop = False
        for t in cart_c[best, 1:acc + 1].tolist():
            if len(generated) >= max_new_tokens:
                break
            generated.append(int(t))
            if t == eos_token_id:
                stop = True
                break
        if not stop and len(generated) < max_new_tokens:
            generated.append(int(torch.argmax(nxt)))
        total_draft += tree_len - 1
        total_accepted += acc
        current = torch.cat([input_ids, torch.tensor([generated], dtype=torch.long)], dim=1)
        if generated[-1] == eos_token_id:
            break
    elapsed = time.time() - t0
    stats = _stats(generated, total_draft, total_accepted, steps, elapsed)
    stats.update({"decode_mode": "tree", "tree_size": tree_len})
    return torch.cat([input_ids, torch.tensor([generated], dtype=torch.long)], dim=1), stats


@torch.no_grad()
def autoregressive_decode(target_model, input_ids: torch.Tensor, max_new_tokens: int, eos_token_id: int = 2):
    """The target's own greedy continuation, one token per forward."""
    ids = input_ids.cpu()
    for _ in range(max_new_tokens):
        logits = target_model.forward(ids)
        tok = int(torch.argmax(logits[0, -1]))
        ids = torch.cat([ids, torch.tensor([[tok]], dtype=torch.long)], dim=1)
        if tok == eos_token_id:
            break
    return ids


def _stats(generated, total_draft, total_accepted, steps, elapsed):
    return {
        "total_tokens_generated": len(generated),
        "total_draft_tokens": total_draft,
        "total_accepted_tokens": total_accepted,
        "num_steps": steps,
        "mean_acceptance_length": total_accepted / max(steps, 1),
        "acceptance_rate": total_accepted / max(total_draft, 1),
        "tokens_per_second": len(generated) / max(elapsed, 1e-6),
        "elapsed_seconds": elapsed,
    }

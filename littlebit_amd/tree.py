"""Token trees for tree-verified speculative decoding.

Same structures and semantics as the reference's tree_utils.py (adapted
there from EAGLE):

* a tree is a list of paths ("tree choices"): path ``[a, b]`` is the b-th
  ranked child of the a-th ranked child of the root;
* :func:`generate_tree_buffers` (tree_utils.py:72-175) sorts the paths by
  (depth, path), numbers the nodes 1.. after the root 0 and returns the
  ancestor mask ``tree_attn_mask`` (1, 1, T, T), ``tree_position_ids``
  (depth of each node), ``retrieve_indices`` (one row per leaf: the node
  indices from the root to the leaf, padded with -1, rows sorted) and
  ``tree_len``, ``depth_counts``, ``sorted_tree_choices``;
* :func:`build_tree_attention_mask` (:501-552) the additive mask of a
  prefix followed by the tree;
* :func:`evaluate_posterior_greedy` (:182-214) the longest candidate path
  that agrees with the target's argmax.

The reference ships fixed presets of 9, 25 and 35 nodes; the verify
benchmark uses a 32-node tree of depth 5 with at most 4 children per node, which
:func:`ranked_tree_choices` builds by a rule: the ``n`` most likely paths
when the k-th ranked child is accepted with probability ``weights[k]``.
"""
from __future__ import annotations

import heapq
from typing import Dict, List, Sequence, Tuple

import torch
import torch.nn.functional as F

__all__ = [
    "ranked_tree_choices",
    "config3_tree_choices",
    "generate_tree_buffers",
    "build_tree_attention_mask",
    "evaluate_posterior_greedy",
    "generate_draft_tree",
]


def ranked_tree_choices(n_nodes: int, max_depth: int, max_branch: int,
                        weights: Sequence[float] = (0.6, 0.2, 0.1, 0.05)) -> List[List[int]]:
    """The ``n_nodes`` paths of highest prob(path) = prod weights[k_i]
    (depth <= max_depth, child rank < max_branch).  The set is closed under
    prefixes and under lower sibling ranks because weights are < 1 and
    decreasing."""
    w = list(weights)[:max_branch]
    if any(not (0 < a < 1) for a in w) or any(w[i] <= w[i + 1] for i in range(len(w) - 1)):
        raise ValueError("weights must be decreasing and in (0, 1)")
    heap: List[Tuple[float, Tuple[int, ...]]] = [(-w[k], (k,)) for k in range(len(w))]
    heapq.heapify(heap)
    out: List[List[int]] = []
    while heap and len(out) < n_nodes:
        negp, path = heapq.heappop(heap)
        out.append(list(path))
        if len(path) < max_depth:
            for k in range(len(w)):
                heapq.heappush(heap, (negp * w[k], path + (k,)))
    return out


def config3_tree_choices() -> List[List[int]]:
    """32 nodes, depth 5, at most 4 children per node (the verify benchmark's tree)."""
    return ranked_tree_choices(32, 5, 4, weights=(0.72, 0.16, 0.07, 0.03))


def generate_tree_buffers(tree_choices: List[List[int]], device="cuda") -> Dict:
    """Node numbering, ancestor mask, depths and leaf paths of a tree."""
    paths = sorted((tuple(p) for p in tree_choices), key=lambda p: (len(p), p))
    index = {p: i + 1 for i, p in enumerate(paths)}  # root is node 0
    for p in paths:
        for d in range(1, len(p)):
            if p[:d] not in index:
                raise ValueError(f"tree path {list(p)} lacks its prefix {list(p[:d])}")
    T = len(paths) + 1
    mask = torch.eye(T)
    mask[:, 0] = 1
    depth = torch.zeros(T, dtype=torch.long)
    for p, i in index.items():
        depth[i] = len(p)
        for d in range(1, len(p)):
            mask[i, index[p[:d]]] = 1
    depth_counts: List[int] = []
    for p in paths:
        while len(depth_counts) < len(p):
            depth_counts.append(0)
        depth_counts[len(p) - 1] += 1
    prefixes = {p[:d] for p in paths for d in range(1, len(p))}
    leaves = [p for p in paths if p not in prefixes]
    width = max(len(p) for p in leaves) + 1
    rows = []
    for p in leaves:
        row = [0] + [index[p[:d]] for d in range(1, len(p) + 1)]
        rows.append(row + [-1] * (width - len(row)))
    big = T + 5
    rows.sort(key=lambda r: [x if x >= 0 else big for x in r])
    bufs = {
        "tree_attn_mask": mask.view(1, 1, T, T),
        "tree_position_ids": depth,
        "retrieve_indices": torch.tensor(rows, dtype=torch.long),
        "sorted_tree_choices": [list(p) for p in paths],
        "tree_len": T,
        "depth_counts": depth_counts,
    }
    return {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in bufs.items()}


def build_tree_attention_mask(prefix_len: int, tree_attn_mask: torch.Tensor, device=None,
                              dtype=torch.bfloat16) -> torch.Tensor:
    """Additive mask (1, 1, P+T, P+T): causal over the prefix, every tree
    node sees the whole prefix and its ancestors, the prefix sees no node."""
    device = device if device is not None else tree_attn_mask.device
    T = tree_attn_mask.shape[-1]
    total = prefix_len + T
    neg = torch.finfo(dtype).min
    allowed = torch.zeros((total, total), dtype=torch.bool, device=device)
    allowed[:prefix_len, :prefix_len] = torch.ones((prefix_len, prefix_len), dtype=torch.bool,
                                                   device=device).tril()
    allowed[prefix_len:, :prefix_len] = True
    allowed[prefix_len:, prefix_len:] = tree_attn_mask[0, 0].to(device).bool()
    out = torch.zeros((total, total), dtype=dtype, device=device).masked_fill(~allowed, neg)
    return out.view(1, 1, total, total)


def evaluate_posterior_greedy(logits: torch.Tensor, candidates: torch.Tensor):
    """(best candidate, accepted length, logits for the bonus token).

    logits (C, L, V) of the target along each candidate path, candidates
    (C, L) token ids (column 0 the root); token i+1 is accepted when it is
    the argmax of logits[:, i] and all earlier ones were."""
    match = (candidates[:, 1:].to(logits.device) == torch.argmax(logits[:, :-1], dim=-1)).int()
    lengths = torch.cumprod(match, dim=1).sum(dim=1)
    accept = int(lengths.max().item())
    best = torch.argmax(lengths) if accept > 0 else torch.tensor(0, device=lengths.device)
    best = best.to(torch.long)
    return best, accept, logits[best, accept]


@torch.no_grad()
def generate_draft_tree(draft, input_ids: torch.Tensor, tree_buffers: Dict, top_k: int = 10) -> torch.Tensor:
    """Tokens of every tree node (1, T) from a GPUDraftModel: the root is the
    last prompt token, the k-th child of a node is the draft's k-th most
    likely token after the node's path (tree_utils.py:314-494), ranked by the
    draft's own head (the Q4_0 logits when it uses the Q4_0 head)."""
    paths = [tuple(p) for p in tree_buffers["sorted_tree_choices"]]
    need = {p[:d] for p in paths for d in range(1, len(p))}
    draft.prefill(input_ids)
    prefix = int(input_ids.shape[1])
    root_logits = draft._head_logits(draft._last_hidden)
    k_max = max(max(p) for p in paths) + 1
    if k_max > top_k:
        raise ValueError(f"tree needs top_k >= {k_max}")
    children = {(): torch.topk(root_logits[0], k_max).indices.tolist()}
    tokens = {}
    for p in paths:
        tokens[p] = children[p[:-1]][p[-1]]
        if p in need:
            ids = [tokens[p[:d]] for d in range(1, len(p) + 1)]
            draft.unit.cache_pos = prefix
            h = draft.unit.forward_batch(ids, draft.embed_tokens, final_norm=draft._q4 is None)
            children[p] = torch.topk(draft._head_logits(h[-1:].contiguous())[0], k_max).indices.tolist()
    draft.unit.cache_pos = prefix
    out = [int(input_ids[0, -1])] + [tokens[p] for p in paths]
    return torch.tensor([out], dtype=torch.long)

"""Tree buffers, masks and greedy posterior (CPU).

Pinned by a hand-derived small case and by invariants that fix the
semantics of tree_utils.py:72-214, 501-552: the mask is the ancestor-or-self
relation, position ids are depths, retrieve rows are the root-to-leaf paths
of every leaf exactly once.
"""
import itertools

import pytest
import torch

from littlebit_amd.tree import (build_tree_attention_mask, config3_tree_choices, evaluate_posterior_greedy,
                                generate_tree_buffers, ranked_tree_choices)


def test_small_tree_by_hand():
    # paths sorted by (depth, path): [0] -> 1, [1] -> 2, [0, 0] -> 3
    b = generate_tree_buffers([[0, 0], [1], [0]], device="cpu")
    assert b["tree_len"] == 4
    assert b["sorted_tree_choices"] == [[0], [1], [0, 0]]
    expect = torch.tensor([[1, 0, 0, 0], [1, 1, 0, 0], [1, 0, 1, 0], [1, 1, 0, 1]], dtype=torch.float32)
    assert torch.equal(b["tree_attn_mask"][0, 0], expect)
    assert b["tree_position_ids"].tolist() == [0, 1, 1, 2]
    assert b["retrieve_indices"].tolist() == [[0, 1, 3], [0, 2, -1]]
    assert b["depth_counts"] == [2, 1]


def test_missing_prefix_rejected():
    with pytest.raises(ValueError):
        generate_tree_buffers([[0], [1, 0]], device="cpu")


@pytest.mark.parametrize("choices", [config3_tree_choices(), ranked_tree_choices(25, 5, 4),
                                     ranked_tree_choices(9, 4, 3), [[0]]])
def test_buffer_invariants(choices):
    b = generate_tree_buffers(choices, device="cpu")
    paths = [tuple(p) for p in b["sorted_tree_choices"]]
    node = {(): 0}
    node.update({p: i + 1 for i, p in enumerate(paths)})
    T = b["tree_len"]
    mask = b["tree_attn_mask"][0, 0]
    for p, i in node.items():
        anc = {node[p[:d]] for d in range(len(p) + 1)}
        assert set(torch.nonzero(mask[i]).view(-1).tolist()) == anc
        assert int(b["tree_position_ids"][i]) == len(p)
    leaves = [p for p in paths if not any(q[:len(p)] == p and len(q) > len(p) for q in paths)]
    rows = b["retrieve_indices"].tolist()
    assert len(rows) == len(leaves)
    got = set()
    for r in rows:
        r = [x for x in r if x >= 0]
        assert r[0] == 0
        inv = {v: k for k, v in node.items()}
        ps = [inv[x] for x in r]
        for a, c in zip(ps, ps[1:]):
            assert c[:-1] == a  # each step is a child of the previous
        got.add(ps[-1])
    assert got == set(leaves)
    key = [[x if x >= 0 else T + 5 for x in r] for r in rows]
    assert key == sorted(key)


def test_config3_tree_shape():
    t = config3_tree_choices()
    assert len(t) == 32
    assert max(len(p) for p in t) == 5
    kids = {}
    for p in t:
        kids.setdefault(tuple(p[:-1]), []).append(p[-1])
    assert max(len(v) for v in kids.values()) <= 4
    for v in kids.values():  # ranks 0..n-1 present
        assert sorted(v) == list(range(len(v)))


def test_ranked_choices_closed():
    t = [tuple(p) for p in ranked_tree_choices(40, 6, 3)]
    s = set(t)
    for p in t:
        assert all(p[:d] in s for d in range(1, len(p)))
        if p[-1] > 0:
            assert p[:-1] + (p[-1] - 1,) in s


def test_attention_mask_blocks():
    b = generate_tree_buffers([[0], [1], [0, 0]], device="cpu")
    m = build_tree_attention_mask(3, b["tree_attn_mask"], device="cpu", dtype=torch.float32)
    ok = m[0, 0] == 0
    P, T = 3, 4
    assert torch.equal(ok[:P, :P], torch.ones(P, P, dtype=torch.bool).tril())
    assert not ok[:P, P:].any()
    assert ok[P:, :P].all()
    assert torch.equal(ok[P:, P:], b["tree_attn_mask"][0, 0].bool())
    assert (m[0, 0][~ok] == torch.finfo(torch.float32).min).all()


def test_evaluate_posterior_greedy():
    V = 7
    cand = torch.tensor([[5, 1, 2, 3], [5, 1, 4, 6], [5, 0, 2, 2]])
    logits = torch.zeros(3, 4, V)
    # target argmax along each path: path 1 agrees on 2 tokens (1, 4), then says 0 != 6
    for c, seq in enumerate([[1, 0, 0, 0], [1, 4, 0, 3], [1, 0, 0, 0]]):
        for i, t in enumerate(seq):
            logits[c, i, t] = 1.0
    best, acc, nxt = evaluate_posterior_greedy(logits, cand)
    assert int(best) == 1 and acc == 2
    assert torch.equal(nxt, logits[1, 2])
    best, acc, nxt = evaluate_posterior_greedy(torch.zeros(3, 4, V), cand + 1)  # nothing agrees
    assert acc == 0 and int(best) == 0

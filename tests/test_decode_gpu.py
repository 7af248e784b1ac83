"""GPU decode/verify steps (the call sites of the forward) against a float64
reference decoder built on the oracle, and the speculative loops against
the target's own greedy decoding.

The reference decoder restates the layer of full_forward_cpu
(patches/littlebit_cpu_optimized.cpp:1522-1840): RMSNorm, q/k/v, GQA
attention without rotary embedding over the cache, o + residual, RMSNorm,
SiLU(gate) * up, down + residual, final RMSNorm; its projections are
oracle.littlebit_forward on the same packed words.
"""
import numpy as np
import pytest
import torch

from oracle import littlebit_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _cfg(hd=32):
    """4 query / 2 KV heads of hd dims: hd 32 runs the decoder's torch
    attention, hd 64 its HIP attention (one-token steps with the merge in the
    o projection, batches with lbk_attention_batch)."""
    from littlebit_amd.decode import DecoderConfig
    return DecoderConfig(hidden_size=4 * hd, intermediate_size=320, num_hidden_layers=2, num_attention_heads=4,
                         num_key_value_heads=2, vocab_size=384, rms_norm_eps=1e-6)


def _state(seed, residual=True, draft=(16, 24), res=(40, 56), hd=32):
    from littlebit_amd.synthetic import synthetic_runtime_state
    return synthetic_runtime_state(_cfg(hd), {"attn": draft[0], "mlp": draft[1]},
                                   {"attn": res[0], "mlp": res[1]} if residual else None,
                                   seed=seed, normalized=True)


def _np(t):
    return t.detach().cpu().double().numpy()


def _branches(state, p, residual):
    out = []
    for tag, sfx in (("", ""), ("_r", "_r")):
        if f"{p}.u_sign{tag}_rt" not in state or (tag and not residual):
            continue
        v = state[f"{p}.v_sign{tag}_rt"].numpy()
        out.append({"v_sign": v, "u_sign": state[f"{p}.u_sign{tag}_rt"].numpy(),
                    "g": _np(state[f"{p}.v2{sfx}"]).reshape(-1), "l": _np(state[f"{p}.mid{sfx}"]).reshape(-1),
                    "h": _np(state[f"{p}.u1{sfx}"]).reshape(-1), "R": v.shape[0]})
    return out


def ref_hidden(state, cfg, ids, residual):
    """Final-norm hidden [N, H] of tokens ids[0..N) from an empty cache."""
    H, eps = cfg.hidden_size, cfg.rms_norm_eps
    kvh, hd, rep = cfg.num_key_value_heads, cfg.head_dim, cfg.kv_repeat

    def norm(x, w):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w

    def lin(x, p, K, N):
        return O.littlebit_forward(x, _branches(state, p, residual), K, N)

    x = _np(state["model.embed_tokens.weight"])[ids]
    n = len(ids)
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}"
        h = norm(x, _np(state[f"{p}.input_layernorm.weight"]))
        q = lin(h, f"{p}.self_attn.q_proj", H, H).reshape(n, kvh, rep, hd)
        k = lin(h, f"{p}.self_attn.k_proj", H, kvh * hd).reshape(n, kvh, hd)
        v = lin(h, f"{p}.self_attn.v_proj", H, kvh * hd).reshape(n, kvh, hd)
        s = np.einsum("tgrd,sgd->grts", q, k) * cfg.attn_scale
        s = np.where(np.tril(np.ones((n, n), bool))[None, None], s, -np.inf)
        s = np.exp(s - s.max(-1, keepdims=True))
        s /= s.sum(-1, keepdims=True)
        a = np.einsum("grts,sgd->tgrd", s, v).reshape(n, H)
        x = x + lin(a, f"{p}.self_attn.o_proj", H, H)
        h = norm(x, _np(state[f"{p}.post_attention_layernorm.weight"]))
        I = cfg.intermediate_size
        g = lin(h, f"{p}.mlp.gate_proj", H, I)
        u = lin(h, f"{p}.mlp.up_proj", H, I)
        x = x + lin(g / (1 + np.exp(-g)) * u, f"{p}.mlp.down_proj", I, H)
    return norm(x, _np(state["model.norm.weight"]))


@pytest.mark.parametrize("residual,fuse", [(False, True), (True, True), (True, False)])
@pytest.mark.parametrize("hd", [32, 64])
def test_decoder_matches_float64_reference(gpu, hd, residual, fuse):
    from littlebit_amd.decode import LittleBitDecoder
    cfg = _cfg(hd)
    st = _state(11, hd=hd)
    dec = LittleBitDecoder(st, cfg, gpu, max_seq_len=64, residual=None if residual else False, fuse=fuse)
    ids = [3, 17, 250, 9, 101, 42, 7]
    h = dec.forward_batch(ids, st["model.embed_tokens.weight"].to(gpu))
    err = O.rel_err(h.cpu().numpy(), ref_hidden(st, cfg, ids, residual))
    print(f"[decode] residual={residual} rel_err={err:.2e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("heads,kvh,hd,max_seq,pos", [(4, 2, 128, 64, 0), (4, 2, 128, 64, 37), (8, 8, 64, 400, 300),
                                                      (32, 8, 128, 700, 513), (2, 1, 64, 256, 255)])
@pytest.mark.parametrize("device_pos", [False, True])
def test_attention_decode_kernel(gpu, heads, kvh, hd, max_seq, pos, device_pos):
    """lbk_attention_decode against torch: softmax(scale q.K) V over 0..pos,
    the new k/v used at pos and stored into the cache.  Two calls share one
    scratch, the second at an earlier position (fewer chunks)."""
    import littlebit_amd._lib as L
    lib = L.load()
    need = lib.lbk_attention_partial_bytes(heads, max_seq, hd)
    part = torch.empty(need // 4 + 1, device=gpu)
    for call, at in enumerate((pos, pos // 2)):
        g = torch.Generator(device="cpu").manual_seed(at + heads + 17 * call)
        kc = torch.randn((kvh, max_seq, hd), generator=g).to(gpu)
        vc = torch.randn((kvh, max_seq, hd), generator=g).to(gpu)
        q = torch.randn((heads * hd,), generator=g).to(gpu)
        k = torch.randn((kvh * hd,), generator=g).to(gpu)
        v = torch.randn((kvh * hd,), generator=g).to(gpu)
        scale = hd ** -0.5
        K = kc.clone()
        V = vc.clone()
        K[:, at] = k.view(kvh, hd)
        V[:, at] = v.view(kvh, hd)
        rep = heads // kvh
        qg = q.view(kvh, rep, hd).double().cpu()
        s = torch.einsum("grd,gtd->grt", qg, K[:, :at + 1].double().cpu()) * scale
        ref = torch.einsum("grt,gtd->grd", torch.softmax(s, dim=-1), V[:, :at + 1].double().cpu()).reshape(-1)
        out = torch.full((heads * hd,), float("nan"), device=gpu)
        pos_t = torch.tensor([at], dtype=torch.int64, device=gpu)
        print(f"[attention_decode] heads={heads} kvh={kvh} hd={hd} max_seq={max_seq} pos={at} dev={device_pos}",
              flush=True)
        rc = lib.lbk_attention_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), heads,
                                      kvh, hd, max_seq, pos_t.data_ptr() if device_pos else None,
                                      0 if device_pos else at, scale, part.data_ptr(), part.numel() * 4,
                                      out.data_ptr(), None)
        L.check(rc, "lbk_attention_decode")
        torch.cuda.synchronize()
        assert O.rel_err(out.cpu().numpy(), ref.numpy()) <= 1e-5
        assert torch.equal(kc[:, at], k.view(kvh, hd)) and torch.equal(vc[:, at], v.view(kvh, hd))
        assert torch.equal(kc[:, :at], K[:, :at])  # nothing else changed


@pytest.mark.parametrize("hd,pos", [(128, 0), (128, 37), (64, 100)])
def test_attention_decode_ignores_rows_past_the_length(gpu, hd, pos):
    """Cache rows past the new position may hold anything (here NaN and
    Inf): the kernel reads whole chunks before it knows the position, and
    those rows must not reach the output or the partials' merge."""
    import littlebit_amd._lib as L
    lib = L.load()
    heads, kvh, max_seq = 4, 2, 160
    need = lib.lbk_attention_partial_bytes(heads, max_seq, hd)
    part = torch.empty(need // 4 + 1, device=gpu)
    g = torch.Generator(device="cpu").manual_seed(pos + hd)
    kc = torch.randn((kvh, max_seq, hd), generator=g)
    vc = torch.randn((kvh, max_seq, hd), generator=g)
    kc[:, pos + 1:] = float("nan")
    vc[:, pos + 1::2] = float("inf")
    vc[:, pos + 2::2] = float("nan")
    q = torch.randn((heads * hd,), generator=g)
    k = torch.randn((kvh * hd,), generator=g)
    v = torch.randn((kvh * hd,), generator=g)
    scale = hd ** -0.5
    K, V = kc[:, :pos + 1].clone().double(), vc[:, :pos + 1].clone().double()
    K[:, pos] = k.view(kvh, hd).double()
    V[:, pos] = v.view(kvh, hd).double()
    qg = q.view(kvh, heads // kvh, hd).double()
    ref = torch.matmul(torch.softmax(torch.matmul(qg, K.transpose(1, 2).contiguous()) * scale, dim=-1), V).reshape(-1)
    kc, vc, q, k, v = (t.to(gpu) for t in (kc, vc, q, k, v))
    for out in (torch.full((heads * hd,), float("nan"), device=gpu), None):
        rc = lib.lbk_attention_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), heads,
                                      kvh, hd, max_seq, None, pos, scale, part.data_ptr(), part.numel() * 4,
                                      None if out is None else out.data_ptr(), None)
        L.check(rc, "lbk_attention_decode")
        torch.cuda.synchronize()
        if out is not None:
            got = out.cpu().double()
        else:  # the partials, merged on the host (chunks 0 .. pos // 16)
            P = part[: heads * (-(-max_seq // 16)) * (hd + 4)].view(heads, -1, hd + 4)[:, : pos // 16 + 1].cpu().double()
            w = torch.exp(P[..., hd] - P[..., hd].max(dim=1, keepdim=True).values)
            got = ((w[..., None] * P[..., :hd]).sum(1) / (w * P[..., hd + 1]).sum(1)[:, None]).reshape(-1)
        assert torch.isfinite(got).all()
        assert O.rel_err(got.numpy(), ref.numpy()) <= 1e-5


def test_attention_decode_rejects_bad_args(gpu):
    import littlebit_amd._lib as L
    lib = L.load()
    x = torch.zeros(1024, device=gpu)
    p = x.data_ptr()
    assert lib.lbk_attention_decode(p, p, p, p, p, 6, 4, 128, 64, None, 0, 1.0, p, 4096, p, None) == L.LBK_ERR_ARG
    assert lib.lbk_attention_decode(p, p, p, p, p, 4, 4, 96, 64, None, 0, 1.0, p, 4096, p, None) == L.LBK_ERR_ARG
    assert lib.lbk_attention_decode(p, p, p, p, p, 4, 4, 64, 64, None, 64, 1.0, p, 4096, p, None) == L.LBK_ERR_ARG
    assert lib.lbk_attention_decode(p, p, p, p, p, 4, 4, 64, 300, None, 0, 1.0, p, 16, p, None) == L.LBK_ERR_WORKSPACE


@pytest.mark.parametrize("n,heads,kvh,hd,max_seq,start,tree", [
    (2, 4, 4, 64, 64, 0, False), (8, 32, 32, 128, 1100, 1024, False), (16, 8, 2, 128, 200, 100, False),
    (17, 8, 8, 64, 80, 37, True), (33, 32, 32, 128, 1100, 1024, True), (64, 4, 1, 128, 600, 500, False),
    (5, 4, 2, 64, 16, 3, True), (40, 2, 2, 64, 40, 0, False)])
def test_attention_batch_kernel(gpu, n, heads, kvh, hd, max_seq, start, tree):
    """lbk_attention_batch against float64: token i at start + i attends to
    every cached position and the new tokens j <= i (or its tree-mask row),
    the new k/v stored into the cache."""
    import littlebit_amd._lib as L
    g = torch.Generator(device="cpu").manual_seed(n * 131 + start)
    kc = torch.randn((kvh, max_seq, hd), generator=g).to(gpu)
    vc = torch.randn((kvh, max_seq, hd), generator=g).to(gpu)
    q = torch.randn((n, heads * hd), generator=g).to(gpu)
    k = torch.randn((n, kvh * hd), generator=g).to(gpu)
    v = torch.randn((n, kvh * hd), generator=g).to(gpu)
    if tree:
        mask = torch.rand((n, n), generator=g) < 0.5
        mask |= torch.eye(n, dtype=torch.bool)
    else:
        mask = torch.tril(torch.ones((n, n), dtype=torch.bool))
    scale = hd ** -0.5
    K = torch.cat([kc[:, :start].double().cpu(), k.view(n, kvh, hd).transpose(0, 1).double().cpu()], dim=1)
    V = torch.cat([vc[:, :start].double().cpu(), v.view(n, kvh, hd).transpose(0, 1).double().cpu()], dim=1)
    rep = heads // kvh
    allowed = torch.cat([torch.ones((n, start), dtype=torch.bool), mask], dim=1)  # [n, start + n]
    qd = q.view(n, kvh, rep, hd).double().cpu()
    s = torch.einsum("ngrd,gtd->ngrt", qd, K) * scale
    s = s.masked_fill(~allowed.view(n, 1, 1, start + n), float("-inf"))
    ref = torch.einsum("ngrt,gtd->ngrd", torch.softmax(s, dim=-1), V).reshape(n, heads * hd)
    lib = L.load()
    part = torch.empty(lib.lbk_attention_batch_partial_bytes(heads, n, start, hd) // 4 + 1, device=gpu)
    out = torch.full((n, heads * hd), float("nan"), device=gpu)
    tm = mask.to(torch.uint8).to(gpu) if tree else None
    old_k = kc.clone()
    print(f"[attention_batch] n={n} heads={heads} kvh={kvh} hd={hd} start={start} tree={tree}", flush=True)
    rc = lib.lbk_attention_batch(q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), n, heads,
                                 kvh, hd, max_seq, None, start, None if tm is None else tm.data_ptr(), scale, part.data_ptr(),
                                 part.numel() * 4, out.data_ptr(), None)
    L.check(rc, "lbk_attention_batch")
    torch.cuda.synchronize()
    err = O.rel_err(out.cpu().numpy(), ref.numpy())
    print(f"[attention_batch] rel_err={err:.2e}", flush=True)
    assert err <= 1e-5
    assert torch.equal(kc[:, start:start + n], k.view(n, kvh, hd).transpose(0, 1))
    assert torch.equal(vc[:, start:start + n], v.view(n, kvh, hd).transpose(0, 1))
    assert torch.equal(kc[:, :start], old_k[:, :start]) and torch.equal(kc[:, start + n:], old_k[:, start + n:])


@pytest.mark.parametrize("n,tree", [(1, False), (8, False), (5, True)])
def test_attention_batch_device_start(gpu, n, tree):
    """A start read from device memory (the host value ignored) gives the
    host-start result and cache; a start whose positions leave the cache
    stores nothing and yields zeros."""
    import littlebit_amd._lib as L
    heads, kvh, hd, max_seq, start = 8, 2, 128, 300, 211
    g = torch.Generator(device="cpu").manual_seed(7 + n)
    kc0 = torch.randn((kvh, max_seq, hd), generator=g).to(gpu)
    vc0 = torch.randn((kvh, max_seq, hd), generator=g).to(gpu)
    q, k, v = (torch.randn((n, w * hd), generator=g).to(gpu) for w in (heads, kvh, kvh))
    tm = (torch.rand((n, n), generator=g) < 0.5) | torch.eye(n, dtype=torch.bool)
    tm = tm.to(torch.uint8).to(gpu) if tree else None
    lib = L.load()
    part = torch.empty(lib.lbk_attention_batch_partial_bytes(heads, n, max_seq - n, hd) // 4 + 1, device=gpu)

    def run(dev_start, host_start):
        kc, vc = kc0.clone(), vc0.clone()
        out = torch.full((n, heads * hd), float("nan"), device=gpu)
        ds = None if dev_start is None else torch.tensor([dev_start], dtype=torch.int64, device=gpu)
        print(f"[attention_batch_dev] n={n} tree={tree} dev={dev_start} host={host_start}", flush=True)
        rc = lib.lbk_attention_batch(q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), n,
                                     heads, kvh, hd, max_seq, None if ds is None else ds.data_ptr(), host_start,
                                     None if tm is None else tm.data_ptr(), hd ** -0.5, part.data_ptr(),
                                     part.numel() * 4, out.data_ptr(), None)
        L.check(rc, "lbk_attention_batch")
        torch.cuda.synchronize()
        return out, kc, vc

    ref, kr, vr = run(None, start)
    out, kd, vd = run(start, 0)
    assert O.rel_err(out.cpu().numpy(), ref.cpu().numpy()) <= 1e-6
    assert torch.equal(kd, kr) and torch.equal(vd, vr)
    out, kd, vd = run(max_seq - n + 1, 0)  # last position past the cache
    assert torch.equal(out, torch.zeros_like(out))
    assert torch.equal(kd, kc0) and torch.equal(vd, vc0)


def test_attention_batch_rejects_bad_args(gpu):
    import littlebit_amd._lib as L
    lib = L.load()
    x = torch.zeros(1 << 16, device=gpu)
    p = x.data_ptr()
    big = x.numel() * 4
    assert lib.lbk_attention_batch(p, p, p, p, p, 65, 4, 4, 64, 128, None, 0, None, 1.0, p, big, p, None) == L.LBK_ERR_ARG
    assert lib.lbk_attention_batch(p, p, p, p, p, 8, 6, 4, 64, 128, None, 0, None, 1.0, p, big, p, None) == L.LBK_ERR_ARG
    assert lib.lbk_attention_batch(p, p, p, p, p, 8, 4, 4, 96, 128, None, 0, None, 1.0, p, big, p, None) == L.LBK_ERR_ARG
    assert lib.lbk_attention_batch(p, p, p, p, p, 8, 4, 4, 64, 128, None, 121, None, 1.0, p, big, p, None) == L.LBK_ERR_ARG
    assert lib.lbk_attention_batch(p + 4, p, p, p, p, 8, 4, 4, 64, 128, None, 0, None, 1.0, p, big, p, None) == L.LBK_ERR_ARG
    assert lib.lbk_attention_batch(p, p, p, p, p, 8, 4, 4, 64, 128, None, 0, None, 1.0, p, 16, p, None) == L.LBK_ERR_WORKSPACE


@pytest.mark.parametrize("hd", [32, 64])
def test_batch_equals_token_by_token(gpu, hd):
    from littlebit_amd.decode import LittleBitDecoder
    cfg = _cfg(hd)
    st = _state(12, hd=hd)
    emb = st["model.embed_tokens.weight"].to(gpu)
    ids = [5, 6, 7, 8, 300, 2]
    a = LittleBitDecoder(st, cfg, gpu, max_seq_len=32)
    b = LittleBitDecoder(st, cfg, gpu, max_seq_len=32)
    hb = a.forward_batch(ids, emb)
    ht = torch.cat([b.forward_token(t, emb) for t in ids])
    err = O.rel_err(hb.cpu().numpy(), ht.cpu().numpy())
    print(f"[batch_vs_tokens] hd={hd} rel_err={err:.2e}", flush=True)
    # fp32 summation orders differ (batched MFMA attention and row tiles
    # against one-token steps); a mask or position mistake would be O(1)
    assert err <= 1e-4
    assert a.cache_pos == b.cache_pos == len(ids)


def _same_tokens_or_tie(st, cfg, gpu, head, prompt, ta, tb, what):
    """Two draft sequences for one prompt must agree token for token, except
    that they may part where the two candidates tie: the graph step's
    attention sums over the whole cache with later positions masked, the
    eager step's over the filled positions only, and the Q8_0 quantisation
    of the hidden state (Q4_0 head) can turn that rounding difference into
    a different argmax when the two largest logits are within it.  At the
    first difference the eager logits of the common prefix must hold both
    tokens within 1e-3 of the largest logit's magnitude."""
    from littlebit_amd.decode import GPUDraftModel
    ta, tb = [int(t) for t in ta], [int(t) for t in tb]
    if ta == tb:
        return
    k = next(i for i, (a, b) in enumerate(zip(ta, tb)) if a != b)
    m = GPUDraftModel(state=st, config=cfg, device=gpu, max_seq_len=48, use_graph=False, lm_head=head)
    m.prefill(torch.cat([prompt, torch.tensor([ta[:k]], dtype=prompt.dtype)], dim=1))
    lg = m._head_logits(m._prompt_hidden if m._prompt_hidden is not None else m._last_hidden)[0]
    gap = float((lg[ta[k]] - lg[tb[k]]).abs())
    scale = float(lg.abs().max())
    print(f"[draft] {what}: tokens part at {k} ({ta[k]} vs {tb[k]}), logit gap {gap:.3e} of {scale:.2f}", flush=True)
    assert gap <= 1e-3 * scale, f"{what}: {ta} vs {tb} part at {k} with logit gap {gap} (not a tie)"


@pytest.mark.parametrize("hd", [32, 64])
@pytest.mark.parametrize("head", ["q4", "dense"])
def test_draft_graph_equals_eager_and_rolls_back(gpu, hd, head):
    from littlebit_amd.decode import GPUDraftModel
    cfg = _cfg(hd)
    st = _state(13, residual=False, hd=hd)
    g = GPUDraftModel(state=st, config=cfg, device=gpu, max_seq_len=48, use_graph=True, lm_head=head)
    e = GPUDraftModel(state=st, config=cfg, device=gpu, max_seq_len=48, use_graph=False, lm_head=head)
    prompt = torch.tensor([[1, 44, 90, 200, 3]])
    for rnd in range(3):
        tg, pg = g.generate_draft_tokens(prompt, draft_length=6)
        te, pe = e.generate_draft_tokens(prompt, draft_length=6)
        _same_tokens_or_tie(st, cfg, gpu, head, prompt, tg, te, f"round {rnd}")
        k = next((i for i, (a, b) in enumerate(zip(tg, te)) if int(a) != int(b)), len(tg))
        for a, b in zip(pg[:k + 1], pe[:k + 1]):  # the same prefix: the same distribution
            assert a.shape == (1, 1, cfg.vocab_size)
            if head == "dense":
                assert float((a - b).abs().max()) <= 1e-4
        assert g._cache_pos == prompt.shape[1] and g._cached_seq_len == prompt.shape[1]
        # next prompt = accepted drafts + one more token: only the new part is computed
        prompt = torch.cat([prompt, torch.tensor([[int(tg[0]), int(tg[1]), 77]])], dim=1)
    # a fresh model on the final prompt drafts the same tokens
    f = GPUDraftModel(state=st, config=cfg, device=gpu, max_seq_len=48, use_graph=False, lm_head=head)
    _same_tokens_or_tie(st, cfg, gpu, head, prompt, f.generate_draft_tokens(prompt, draft_length=4)[0],
                        g.generate_draft_tokens(prompt, draft_length=4)[0], "fresh model")


@pytest.mark.parametrize("hd", [32, 64])
def test_target_prefix_reuse_and_zero_rows(gpu, hd):
    from littlebit_amd.decode import GPUTargetModel
    cfg = _cfg(hd)
    d, r = _state(14, residual=False, hd=hd), _state(15, residual=False, hd=hd)
    t = GPUTargetModel(draft_state=d, residual_state=r, config=cfg, device=gpu, max_seq_len=64)
    fresh = GPUTargetModel(draft_state=d, residual_state=r, config=cfg, device=gpu, max_seq_len=64)
    a = torch.tensor([[4, 8, 15, 16, 23]])
    b = torch.tensor([[4, 8, 15, 99, 42, 7]])  # shares 3 tokens
    t.forward(a)
    lb = t.forward(b)
    assert float(lb[0, :3].abs().max()) == 0.0
    full = fresh.forward(b)
    assert O.rel_err(lb[0, 3:].cpu().numpy(), full[0, 3:].cpu().numpy()) <= 1e-5
    # hidden sum of two units = logits through one lm_head (cpu_target_model.py:520-527)
    # both units embed with the draft checkpoint's table, as with the shared base model
    r_shared = {**r, "model.embed_tokens.weight": d["model.embed_tokens.weight"]}
    h = ref_hidden(d, cfg, b[0].tolist(), False) + ref_hidden(r_shared, cfg, b[0].tolist(), False)
    W = d["lm_head.weight"].double().numpy()
    assert O.rel_err(full[0].cpu().numpy(), h @ W.T) <= TOL


@pytest.mark.parametrize("hd", [32, 64])
def test_single_unit_target_uses_residual_branches(gpu, hd):
    from littlebit_amd.decode import GPUTargetModel
    cfg = _cfg(hd)
    st = _state(16, residual=True, hd=hd)
    t = GPUTargetModel(draft_state=st, config=cfg, device=gpu, max_seq_len=64)
    ids = [1, 2, 3, 4]
    lg = t.forward(torch.tensor([ids]))
    ref = ref_hidden(st, cfg, ids, True) @ st["lm_head.weight"].double().numpy().T
    assert O.rel_err(lg[0].cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("hd", [32, 64])
def test_forward_tree_chain_equals_sequence(gpu, hd):
    """A tree that is one chain verifies like the plain sequence."""
    from littlebit_amd.decode import GPUTargetModel
    from littlebit_amd.tree import generate_tree_buffers
    cfg = _cfg(hd)
    st = _state(17, hd=hd)
    t1 = GPUTargetModel(draft_state=st, config=cfg, device=gpu, max_seq_len=64)
    t2 = GPUTargetModel(draft_state=st, config=cfg, device=gpu, max_seq_len=64)
    prefix = [9, 8, 7, 6]
    chain = [31, 32, 33]
    bufs = generate_tree_buffers([[0], [0, 0], [0, 0, 0]], device=gpu)
    lt = t1.forward_tree(torch.tensor([prefix]), [prefix[-1]] + chain, bufs["tree_attn_mask"][0, 0])
    ls = t2.forward(torch.tensor([prefix + chain]))
    assert O.rel_err(lt.cpu().numpy(), ls[0, len(prefix) - 1:].cpu().numpy()) <= 1e-5
    assert t1.draft_unit.cache_pos == len(prefix)


@pytest.mark.parametrize("hd", [32, 64])
def test_speculative_greedy_equals_autoregressive(gpu, hd):
    from littlebit_amd.decode import GPUDraftModel, GPUTargetModel
    from littlebit_amd.speculative import autoregressive_decode, speculative_decode
    cfg = _cfg(hd)
    d, r = _state(18, residual=False, hd=hd), _state(19, residual=False, hd=hd)
    draft = GPUDraftModel(state=d, config=cfg, device=gpu, max_seq_len=96)
    target = GPUTargetModel(draft_state=d, residual_state=r, config=cfg, device=gpu, max_seq_len=96)
    ref_t = GPUTargetModel(draft_state=d, residual_state=r, config=cfg, device=gpu, max_seq_len=96)
    prompt = torch.tensor([[10, 20, 30, 40]])
    out, stats = speculative_decode(draft, target, prompt, max_new_tokens=24, draft_length=5, eos_token_id=-1)
    ref = autoregressive_decode(ref_t, prompt, 24, eos_token_id=-1)
    print(f"[spec] accepted {stats['total_accepted_tokens']}/{stats['total_draft_tokens']}", flush=True)
    assert out.tolist() == ref.tolist()
    assert stats["total_tokens_generated"] == 24


@pytest.mark.parametrize("hd", [32, 64])
def test_speculative_tree_equals_autoregressive(gpu, hd):
    from littlebit_amd.decode import GPUDraftModel, GPUTargetModel
    from littlebit_amd.speculative import autoregressive_decode, speculative_decode_tree
    from littlebit_amd.tree import generate_tree_buffers, ranked_tree_choices
    cfg = _cfg(hd)
    d, r = _state(20, residual=False, hd=hd), _state(21, residual=False, hd=hd)
    draft = GPUDraftModel(state=d, config=cfg, device=gpu, max_seq_len=128, use_graph=False)
    target = GPUTargetModel(draft_state=d, residual_state=r, config=cfg, device=gpu, max_seq_len=128)
    ref_t = GPUTargetModel(draft_state=d, residual_state=r, config=cfg, device=gpu, max_seq_len=128)
    bufs = generate_tree_buffers(ranked_tree_choices(12, 4, 3), device=gpu)
    prompt = torch.tensor([[3, 1, 4, 1, 5]])
    out, stats = speculative_decode_tree(draft, target, prompt, max_new_tokens=16, tree_buffers=bufs, top_k=4,
                                         eos_token_id=-1)
    ref = autoregressive_decode(ref_t, prompt, 16, eos_token_id=-1)
    assert out.tolist() == ref.tolist()


@pytest.mark.parametrize("hd", [32, 64])
def test_q4_draft_tokens_follow_generate_token(gpu, hd):
    """The Q4_0 draft path (the reference's generate_token): each draft
    token is the Q4_0 x Q8_0 argmax of the previous position's final hidden
    state (oracle on the float64 reference decoder's hidden), and the
    probabilities are one-hot at it (cpu_draft_model.py:541-563)."""
    from littlebit_amd.decode import GPUDraftModel
    from oracle import lm_head_q4_oracle as Q
    cfg = _cfg(hd)
    st = _state(23, residual=False, hd=hd)
    m = GPUDraftModel(state=st, config=cfg, device=gpu, max_seq_len=48, lm_head="q4")
    prompt = [5, 9, 100, 7]
    toks, probs = m.generate_draft_tokens(torch.tensor([prompt]), draft_length=4)
    toks = [int(t) for t in toks]
    qs, d = Q.quantize_q4_0(st["lm_head.weight"].float().numpy())
    seq = list(prompt)
    for t, p in zip(toks, probs):
        assert p.shape == (1, 1, cfg.vocab_size) and float(p[0, 0, t]) == 1.0 and float(p.sum()) == 1.0
        h = ref_hidden(st, cfg, seq, False)[-1].astype(np.float32)
        logits, _ = Q.generate_token_head(h, qs, d)
        assert logits[t] >= logits.max() - 2e-3 * np.abs(logits).max(), (seq, t)
        seq.append(t)

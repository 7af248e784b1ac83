"""lbk_chain_forward (LittleBitChain): calls that each read the one before's
outputs at one row -- o, gate/up, down and the next layer's q/k/v of a
decode step -- joined into one kernel per link boundary.  Every link's
outputs are checked against the float64 oracle composed the same way
(residual adds, RMSNorm, SiLU * up) and against the same links run one by
one through lbk_group_forward_ex."""
import numpy as np
import pytest
import torch

from oracle import littlebit_oracle as O

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3
EPS = 1e-5


def _proj(seed, K, N, ranks, dev, bias=False):
    from littlebit_amd import LittleBitBranch, LittleBitProjection
    from littlebit_amd.synthetic import make_projection
    _, brs = make_projection(seed, 1, K, N, ranks)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    b = None
    if bias:
        b = np.random.Generator(np.random.PCG64(seed + 5)).standard_normal(N).astype(np.float32)
    p = LittleBitProjection([LittleBitBranch(v_sign=t(x.v_sign), u_sign=t(x.u_sign), v2=t(x.g), mid=t(x.l),
                                             u1=t(x.h)) for x in brs], bias=None if b is None else t(b))
    return p, [x.as_dict() for x in brs], b


class Layer:
    """One decoder layer's linears (o; gate, up; down) and the next layer's
    q, k, v, with RMSNorm weights, at hidden H and intermediate I."""

    def __init__(self, seed, dev, H, I, kv, ra, rm, bias=False):
        self.H, self.I, self.kv = H, I, kv
        specs = {"o": (H, H, ra), "gate": (H, I, rm), "up": (H, I, rm), "down": (I, H, rm),
                 "q": (H, H, ra), "k": (H, kv, ra), "v": (H, kv, ra)}
        self.p, self.h, self.b = {}, {}, {}
        for i, (name, (K, N, ranks)) in enumerate(specs.items()):
            self.p[name], self.h[name], self.b[name] = _proj(seed + 31 * i, K, N, ranks, dev,
                                                             bias=bias and name in ("o", "up", "k"))
        rng = np.random.Generator(np.random.PCG64(seed + 999))
        self.ln2 = (rng.random(H) + 0.5).astype(np.float32)
        self.ln1 = (rng.random(H) + 0.5).astype(np.float32)
        self.tln2 = torch.from_numpy(self.ln2).to(dev)
        self.tln1 = torch.from_numpy(self.ln1).to(dev)

    def oracle(self, a, x):
        """(x after o, gate, up, x after down, q, k, v) in float64."""
        f = lambda n, inp: O.littlebit_forward(inp, self.h[n], inp.shape[-1], self.p[n].out_features,  # noqa: E731
                                               bias=self.b[n])
        x1 = x + f("o", a)
        h = O.rms_norm(x1, self.ln2, EPS)
        g, u = f("gate", h), f("up", h)
        x2 = x1 + f("down", O.silu_mul(g, u))
        h = O.rms_norm(x2, self.ln1, EPS)
        return x1, g, u, x2, f("q", h), f("k", h), f("v", h)

    def chain(self, x, g, u, q, k, v):
        from littlebit_amd import ChainLink, LittleBitChain, LittleBitProjectionGroup
        return LittleBitChain([
            ChainLink(self.p["o"], [x], residuals=[x]),
            ChainLink(LittleBitProjectionGroup([self.p["gate"], self.p["up"]]), [g, u], rms_weight=self.tln2,
                      rms_eps=EPS),
            ChainLink(self.p["down"], [x], residuals=[x], silu_mul=True),
            ChainLink(LittleBitProjectionGroup([self.p["q"], self.p["k"], self.p["v"]]), [q, k, v],
                      rms_weight=self.tln1, rms_eps=EPS),
        ])

    def buffers(self, dev):
        z = lambda n: torch.full((1, n), float("nan"), device=dev)  # noqa: E731
        return z(self.H), z(self.I), z(self.I), z(self.H), z(self.kv), z(self.kv)

    def one_by_one(self, a, x, g, u, q, k, v):
        from littlebit_amd import LittleBitProjectionGroup
        self.p["o"].forward(a, out=x, residual=x)
        LittleBitProjectionGroup([self.p["gate"], self.p["up"]]).forward(x, outs=[g, u], rms_weight=self.tln2,
                                                                        rms_eps=EPS)
        self.p["down"].forward(g, out=x, residual=x, x_up=u)
        LittleBitProjectionGroup([self.p["q"], self.p["k"], self.p["v"]]).forward(x, outs=[q, k, v],
                                                                                 rms_weight=self.tln1, rms_eps=EPS)


def _inputs(seed, H, dev):
    rng = np.random.Generator(np.random.PCG64(seed))
    a = rng.standard_normal((1, H)).astype(np.float32)
    x0 = rng.standard_normal((1, H)).astype(np.float32)
    return a, x0


def _check_layer(L, dev, seed, expect_fused=True):
    a, x0 = _inputs(seed, L.H, dev)
    ref = L.oracle(a.astype(np.float64), x0.astype(np.float64))
    x, g, u, q, k, v = L.buffers(dev)
    x.copy_(torch.from_numpy(x0))
    ta = torch.from_numpy(a).to(dev)
    chain = L.chain(x, g, u, q, k, v)
    assert chain.fused(ta) == expect_fused
    chain.forward(ta)
    torch.cuda.synchronize()
    got = [x, g, u, q, k, v]
    names = ["x after down", "gate", "up", "q", "k", "v"]
    want = [ref[3], ref[1], ref[2], ref[4], ref[5], ref[6]]
    # the same links one by one
    xs, gs, us, qs, ks, vs = L.buffers(dev)
    xs.copy_(torch.from_numpy(x0))
    L.one_by_one(ta, xs, gs, us, qs, ks, vs)
    torch.cuda.synchronize()
    for name, t, w, s in zip(names, got, want, [xs, gs, us, qs, ks, vs]):
        y = t.cpu().numpy()
        assert np.isfinite(y).all(), name
        err = O.rel_err(y, w)
        same = O.rel_err(y, s.cpu().numpy())
        print(f"[chain] {name}: vs oracle {err:.2e}, vs one by one {same:.2e}", flush=True)
        assert err <= TOL_F32, (name, err)
        # both within ~1e-5 of the oracle, their fp32 sums in different orders
        assert same <= 5e-5, (name, same)
    return chain, (x, g, u, q, k, v), (ta, x0), want


def test_chain_draft_layer(gpu):
    """Llama-2-7B draft shapes (rank 205 / 298): o -> gate/up -> down -> q/k/v."""
    print("[chain] draft layer, hidden 4096", flush=True)
    L = Layer(8100, gpu, 4096, 11008, 4096, [205], [298])
    _check_layer(L, gpu, 8101)


def test_chain_two_branches_ragged(gpu):
    """Draft + residual branches, biases, output counts that are not
    multiples of a block's rows (1000 = 7 * 128 + 104; 40 for k and v)."""
    print("[chain] two branches, hidden 512, intermediate 1000", flush=True)
    L = Layer(8200, gpu, 512, 1000, 40, [45, 300], [64, 300], bias=True)
    _check_layer(L, gpu, 8201)


def test_chain_regions_between_calls(gpu):
    """Chains of different lengths and shapes, a group call between them and
    a repeat of the first chain on one workspace: the latent regions the
    chains leave behind must not leak into the next chain."""
    from littlebit_amd import ChainLink, LittleBitChain
    print("[chain] regions between calls", flush=True)
    A = Layer(8300, gpu, 512, 1000, 40, [45, 300], [64, 300])
    B = Layer(8400, gpu, 256, 768, 256, [33], [70])
    chain_a, bufs_a, (ta, x0), want_a = _check_layer(A, gpu, 8301)
    # a two-link chain of B (o -> gate/up) and a one-by-one call between
    a, xb0 = _inputs(8401, B.H, gpu)
    refb = B.oracle(a.astype(np.float64), xb0.astype(np.float64))
    xb, gb, ub, _, _, _ = B.buffers(gpu)
    xb.copy_(torch.from_numpy(xb0))
    from littlebit_amd import LittleBitProjectionGroup
    two = LittleBitChain([ChainLink(B.p["o"], [xb], residuals=[xb]),
                          ChainLink(LittleBitProjectionGroup([B.p["gate"], B.p["up"]]), [gb, ub],
                                    rms_weight=B.tln2, rms_eps=EPS)])
    assert two.fused(torch.from_numpy(a).to(gpu))
    q_alone = torch.empty((1, B.H), device=gpu)
    B.p["q"].forward(torch.from_numpy(xb0).to(gpu), out=q_alone)
    two.forward(torch.from_numpy(a).to(gpu))
    torch.cuda.synchronize()
    for name, t, w in [("x after o", xb, refb[0]), ("gate", gb, refb[1]), ("up", ub, refb[2])]:
        err = O.rel_err(t.cpu().numpy(), w)
        print(f"[chain] B {name}: vs oracle {err:.2e}", flush=True)
        assert err <= TOL_F32, (name, err)
    want_q = O.littlebit_forward(xb0.astype(np.float64), B.h["q"], B.H, B.H)
    assert O.rel_err(q_alone.cpu().numpy(), want_q) <= TOL_F32
    # the first chain again, from the same inputs
    x = bufs_a[0]
    x.copy_(torch.from_numpy(x0))
    for t in bufs_a[1:]:
        t.fill_(float("nan"))
    chain_a.forward(ta)
    torch.cuda.synchronize()
    for t, w in zip(bufs_a, want_a):
        err = O.rel_err(t.cpu().numpy(), w)
        assert err <= TOL_F32, err


def test_chain_graph_replays(gpu):
    """A captured chain replayed several times, with eager work between the
    replays, against the eager result each time."""
    print("[chain] graph replays", flush=True)
    L = Layer(8500, gpu, 512, 1000, 40, [45, 300], [64, 300])
    a, x0 = _inputs(8501, L.H, gpu)
    ref = L.oracle(a.astype(np.float64), x0.astype(np.float64))
    want = [ref[3], ref[1], ref[2], ref[4], ref[5], ref[6]]
    x, g, u, q, k, v = L.buffers(gpu)
    ta = torch.from_numpy(a).to(gpu)
    chain = L.chain(x, g, u, q, k, v)
    x.copy_(torch.from_numpy(x0))
    chain.forward(ta)
    torch.cuda.synchronize()
    eager = [t.clone() for t in (x, g, u, q, k, v)]
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    x.copy_(torch.from_numpy(x0))
    with torch.cuda.stream(stream):
        chain.forward(ta)  # warm on this stream
    stream.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        chain.forward(ta)
    for rep in range(4):
        x.copy_(torch.from_numpy(x0))
        for t in (g, u, q, k, v):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for t, e, w in zip((x, g, u, q, k, v), eager, want):
            y = t.cpu().numpy()
            d = O.rel_err(y, e.cpu().numpy())
            assert d <= 5e-5, (rep, d)  # fp32 atomics in another order
            assert O.rel_err(y, w) <= TOL_F32, rep
        # eager calls on the default stream's workspace between replays
        L.p["q"].forward(ta)
    torch.cuda.synchronize()


def test_chain_deterministic_runs_unjoined(gpu):
    """Under deterministic mode the links run as separate calls: the same
    results, bit for bit from run to run."""
    from littlebit_amd import deterministic
    print("[chain] deterministic mode", flush=True)
    L = Layer(8600, gpu, 512, 1000, 40, [45, 300], [64, 300])
    with deterministic(True):
        chain, bufs, (ta, x0), want = _check_layer(L, gpu, 8601, expect_fused=False)
        first = [t.clone() for t in bufs]
        bufs[0].copy_(torch.from_numpy(x0))
        chain.forward(ta)
        torch.cuda.synchronize()
        for t, f in zip(bufs, first):
            assert torch.equal(t, f)


def test_chain_invalid_links(gpu):
    """A link whose input does not match the link before is refused."""
    import littlebit_amd._lib as L
    from littlebit_amd import ChainLink, LittleBitChain
    Ly = Layer(8700, gpu, 256, 768, 256, [33], [70])
    x, g, u, q, k, v = Ly.buffers(gpu)
    with pytest.raises(Exception):
        # down reads SiLU * up of a link with one projection
        LittleBitChain([ChainLink(Ly.p["o"], [x]), ChainLink(Ly.p["down"], [x], silu_mul=True)]).forward(
            torch.zeros((1, 256), device=gpu))
    with pytest.raises(Exception):
        # gate/up (K = 256) after down (N = 256) is fine; o (K = 256) after gate (N = 768) is not
        LittleBitChain([ChainLink(Ly.p["gate"], [g]), ChainLink(Ly.p["o"], [x])]).forward(
            torch.zeros((1, 256), device=gpu))
    assert "link 1" in L.load().lbk_last_error().decode()


def test_chain_eight_links(gpu):
    """The longest chain (LBK_MAX_CHAIN links): every latent region in use,
    the last link's region the last one, links of every input kind (plain,
    RMSNorm, two projections then SiLU * up), two-branch and ragged ranks, a
    bias and an output that is also its own residual; against the float64
    oracle and the same links one by one, on two calls in a row (the regions
    a chain leaves behind must not leak into the next call)."""
    from littlebit_amd import ChainLink, LittleBitChain, LittleBitProjectionGroup
    specs = [  # name, K, N, ranks, bias
        ("a", 512, 640, [40], False), ("b", 640, 512, [24, 56], False), ("c", 512, 768, [64], False),
        ("d", 768, 384, [33], False), ("g", 384, 1000, [48], False), ("u", 384, 1000, [48], True),
        ("e", 1000, 384, [30, 70], False), ("f", 384, 512, [20], False), ("h", 512, 256, [36, 12], True)]
    P, H, B = {}, {}, {}
    for i, (nm, K, N, ranks, bias) in enumerate(specs):
        P[nm], H[nm], B[nm] = _proj(9100 + 17 * i, K, N, ranks, gpu, bias=bias)
    rng = np.random.Generator(np.random.PCG64(9199))
    w_c = (rng.random(512) + 0.5).astype(np.float32)
    w_g = (rng.random(384) + 0.5).astype(np.float32)
    w_h = (rng.random(512) + 0.5).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(gpu)  # noqa: E731
    tw_c, tw_g, tw_h = t(w_c), t(w_g), t(w_h)
    nan = lambda n: torch.full((1, n), float("nan"), device=gpu)  # noqa: E731

    def f(nm, inp):
        return O.littlebit_forward(inp, H[nm], inp.shape[-1], P[nm].out_features, bias=B[nm])

    def oracle(x, d0):
        ya = f("a", x)
        yb = f("b", ya)
        yc = f("c", O.rms_norm(yb, w_c, EPS))
        yd = f("d", yc)
        hg = O.rms_norm(yd, w_g, EPS)
        yg, yu = f("g", hg), f("u", hg)
        ye = d0 + f("e", O.silu_mul(yg, yu))   # e adds into its residual buffer
        yf = f("f", ye)
        yh = f("h", O.rms_norm(yf, w_h, EPS))
        return [ya, yb, yc, yd, yg, yu, ye, yf, yh]

    def buffers():
        return [nan(640), nan(512), nan(768), nan(384), nan(1000), nan(1000), nan(384), nan(512), nan(256)]

    def links(o):
        ya, yb, yc, yd, yg, yu, ye, yf, yh = o
        return [ChainLink(P["a"], [ya]), ChainLink(P["b"], [yb]),
                ChainLink(P["c"], [yc], rms_weight=tw_c, rms_eps=EPS), ChainLink(P["d"], [yd]),
                ChainLink(LittleBitProjectionGroup([P["g"], P["u"]]), [yg, yu], rms_weight=tw_g, rms_eps=EPS),
                ChainLink(P["e"], [ye], residuals=[ye], silu_mul=True), ChainLink(P["f"], [yf]),
                ChainLink(P["h"], [yh], rms_weight=tw_h, rms_eps=EPS)]

    import littlebit_amd._lib as L
    assert L.LBK_MAX_CHAIN == 8
    out = buffers()
    chain = LittleBitChain(links(out))
    for call in range(2):
        x = rng.standard_normal((1, 512)).astype(np.float32)
        d0 = rng.standard_normal((1, 384)).astype(np.float32)
        tx = t(x)
        assert chain.fused(tx)
        out[6].copy_(t(d0))
        chain.forward(tx)
        # one by one
        s = buffers()
        P["a"].forward(tx, out=s[0])
        P["b"].forward(s[0], out=s[1])
        P["c"].forward(s[1], out=s[2], rms_weight=tw_c, rms_eps=EPS)
        P["d"].forward(s[2], out=s[3])
        LittleBitProjectionGroup([P["g"], P["u"]]).forward(s[3], outs=[s[4], s[5]], rms_weight=tw_g, rms_eps=EPS)
        s[6].copy_(t(d0))
        P["e"].forward(s[4], out=s[6], residual=s[6], x_up=s[5])
        P["f"].forward(s[6], out=s[7])
        P["h"].forward(s[7], out=s[8], rms_weight=tw_h, rms_eps=EPS)
        torch.cuda.synchronize()
        want = oracle(x.astype(np.float64), d0.astype(np.float64))
        for i, (got, one, w) in enumerate(zip(out, s, want)):
            y = got.cpu().numpy()
            assert np.isfinite(y).all(), (call, i)
            err, same = O.rel_err(y, w), O.rel_err(y, one.cpu().numpy())
            print(f"[chain8] call {call} link output {i}: vs oracle {err:.2e}, vs one by one {same:.2e}", flush=True)
            assert err <= TOL_F32, (call, i, err)
            assert same <= 5e-5, (call, i, same)


def test_chain_first_link_input_kinds(gpu):
    """Chains whose first link reads RMSNorm(x) * w (gate/up -> down) or
    SiLU(gate) * up of the caller's tensors (down -> q/k/v), against the
    oracle and the same calls one by one."""
    from littlebit_amd import ChainLink, LittleBitChain, LittleBitProjectionGroup
    Ly = Layer(9700, gpu, 512, 1000, 256, [40, 90], [64])
    rng = np.random.Generator(np.random.PCG64(9701))
    x = rng.standard_normal((1, 512)).astype(np.float32)
    gt = rng.standard_normal((1, 1000)).astype(np.float32)
    ut = rng.standard_normal((1, 1000)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(gpu)  # noqa: E731
    f = lambda n, inp: O.littlebit_forward(inp, Ly.h[n], inp.shape[-1], Ly.p[n].out_features,  # noqa: E731
                                           bias=Ly.b[n])
    gu = LittleBitProjectionGroup([Ly.p["gate"], Ly.p["up"]])
    qkv = LittleBitProjectionGroup([Ly.p["q"], Ly.p["k"], Ly.p["v"]])
    nan = lambda n: torch.full((1, n), float("nan"), device=gpu)  # noqa: E731

    # RMSNorm first: gate/up of RMSNorm(x) * ln2, then down of SiLU(gate) * up
    g, u, d = nan(1000), nan(1000), nan(512)
    chain = LittleBitChain([ChainLink(gu, [g, u], rms_weight=Ly.tln2, rms_eps=EPS),
                            ChainLink(Ly.p["down"], [d], silu_mul=True)])
    tx = t(x)
    assert chain.fused(tx)
    chain.forward(tx)
    g1, u1, d1 = nan(1000), nan(1000), nan(512)
    gu.forward(tx, outs=[g1, u1], rms_weight=Ly.tln2, rms_eps=EPS)
    Ly.p["down"].forward(g1, out=d1, x_up=u1)
    torch.cuda.synchronize()
    h = O.rms_norm(x.astype(np.float64), Ly.ln2, EPS)
    wg, wu = f("gate", h), f("up", h)
    wd = f("down", O.silu_mul(wg, wu))
    for name, got, one, want in (("gate", g, g1, wg), ("up", u, u1, wu), ("down", d, d1, wd)):
        y = got.cpu().numpy()
        err, same = O.rel_err(y, want), O.rel_err(y, one.cpu().numpy())
        print(f"[chain-first] rmsnorm {name}: vs oracle {err:.2e}, vs one by one {same:.2e}", flush=True)
        assert np.isfinite(y).all() and err <= TOL_F32 and same <= 5e-5, (name, err, same)

    # SiLU * up first: down of SiLU(gt) * ut, then q/k/v of RMSNorm(down) * ln1
    d, q, k, v = nan(512), nan(512), nan(256), nan(256)
    chain = LittleBitChain([ChainLink(Ly.p["down"], [d], silu_mul=True),
                            ChainLink(qkv, [q, k, v], rms_weight=Ly.tln1, rms_eps=EPS)])
    tg, tu = t(gt), t(ut)
    chain.forward(tg, x_up=tu)
    d1, q1, k1, v1 = nan(512), nan(512), nan(256), nan(256)
    Ly.p["down"].forward(tg, out=d1, x_up=tu)
    qkv.forward(d1, outs=[q1, k1, v1], rms_weight=Ly.tln1, rms_eps=EPS)
    torch.cuda.synchronize()
    wd = f("down", O.silu_mul(gt.astype(np.float64), ut.astype(np.float64)))
    h = O.rms_norm(wd, Ly.ln1, EPS)
    for name, got, one, want in (("down", d, d1, wd), ("q", q, q1, f("q", h)), ("k", k, k1, f("k", h)),
                                 ("v", v, v1, f("v", h))):
        y = got.cpu().numpy()
        err, same = O.rel_err(y, want), O.rel_err(y, one.cpu().numpy())
        print(f"[chain-first] silu {name}: vs oracle {err:.2e}, vs one by one {same:.2e}", flush=True)
        assert np.isfinite(y).all() and err <= TOL_F32 and same <= 5e-5, (name, err, same)

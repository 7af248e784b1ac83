"""Benchmark of the LittleBitLinear forward on one MI355X.

Workload: the Llama-2-7B-shaped 0.1-BPW draft decode
step -- the 7 projections of each of 32 decoder layers at batch 1 (q, k, v, o
4096->4096 rank 205; gate, up 4096->11008 rank 298; down 11008->4096 rank
298), fp32 activations, random packed signs and |N(0,1)|+0.05 scales, with
the decode step's data flow (ChainStep): q/k/v of RMSNorm(x), o of a fixed
stand-in for the attention output added to x, gate/up of RMSNorm(x), down of
SiLU(gate) * up added to x.  One step = the 224 forwards captured as one HIP
graph; each layer's o, gate/up, down and the next layer's q/k/v run as one
LittleBitChain (lbk_chain_forward: 5 launches per layer, each kernel between
two calls expanding one call's rows and adding their part of the next call's
latent vector).  The same step with each call on its own (8 launches per
layer) and the previous workload (224 calls with independent inputs) are
reported beside it.

value = algorithmic bytes of a step / time of a step, with the weights cold:
the step rotates over enough weight replicas that the working set exceeds
the 256 MB Infinity Cache.  The warm figure (one replica) is reported too.

roofline = the dominant unit of the step, one layer's chain (its 5 kernels,
7 projections), timed with HIP events around the step's graphs (32 layer
chains each); bytes from sign words + scales + x read once + y written once
per projection.  cpu_baseline = the reference AVX2 kernel littlebit_linear
(oracle/_ref, built from the reference source) on the host cores, over a
bounded number of whole steps.

python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "µs/layer + achieved GB/s (LittleBitLinear GEMV); draft tok/s, Llama-2-7B 0.1BPW"
HBM_PEAK_GBS = 8000.0
# HBM bytes per call of a call kind's kernel pair (latent + expand), from two
# rocprofv3 --pmc passes over `--only <kind>` graphs: FETCH_SIZE x 2.0 +
# WRITE_SIZE x 1.0, the factors a 256 MiB device copy reads (FETCH_SIZE counts
# half the bytes moved).  Commands and figures in
# profiles/littlebit_decode_calls.md; a kind without a measurement reports null.
MEASURED_TRAFFIC = {"qkv": 1_229_984, "o": 616_288, "gate/up": 1_811_040, "down": 1_128_064}
# the same for the target's calls at M = 8 (profiles/littlebit_verify_m8_target.md)
MEASURED_TRAFFIC_M8 = {"qkv": 11_636_122, "o": 5_105_971, "gate/up": 17_666_765, "down": 9_626_419}
# the same for one layer's chain (latent_mfma_kernel + 3 chain_mfma_kernel +
# expand_mfma_kernel) of the chained draft step (profiles/littlebit_decode_chain.md)
MEASURED_TRAFFIC_CHAIN = 4_604_313
MALL_BYTES = 256 << 20


def proj_bytes(M, K, N, ranks, sx=4, sy=4):
    """Algorithmic bytes of one forward: every branch's sign words and scales,
    x read once and y written once (the latent vector stays on chip)."""
    b = 0
    for R in ranks:
        b += R * math.ceil(K / 32) * 4 + N * math.ceil(R / 32) * 4 + 4 * (K + R + N)
    return b + M * K * sx + M * N * sy


def draft_layer_shapes():
    from littlebit_amd.synthetic import llama_projection_shapes
    return llama_projection_shapes(residual=False)


def make_device_branch(gen, K, R, N, dev):
    import torch
    from littlebit_amd import LittleBitBranch

    def words(rows, cols):
        wpr = (cols + 31) // 32
        w = torch.randint(-2**31, 2**31, (rows, wpr), generator=gen, dtype=torch.int64, device="cpu")
        tail = cols - 32 * (wpr - 1)
        if tail < 32:
            w[:, -1] &= (1 << tail) - 1
        return w.to(torch.int32).to(dev)

    def scales(n):
        return (torch.randn(n, generator=gen).abs() + 0.05).to(dev)

    return LittleBitBranch(v_sign=words(R, K), u_sign=words(N, R), v2=scales(K), mid=scales(R), u1=scales(N))


# One decoder layer's linears as launches: projections reading the same input
# run as one group call (q/k/v, gate/up), the others alone.
LAYER_CALLS = [("qkv", ("q_proj", "k_proj", "v_proj")), ("o", ("o_proj",)),
               ("gate/up", ("gate_proj", "up_proj")), ("down", ("down_proj",))]


class Call:
    """One launch pair: a projection or a group of projections with a shared
    input, its input x [1, K] and outputs."""

    def __init__(self, gen, dev, names, grouped=True, M=1, residual=False):
        import torch
        from littlebit_amd import LittleBitProjection, LittleBitProjectionGroup
        from littlebit_amd.synthetic import llama_projection_shapes
        shapes = {s[0]: s for s in llama_projection_shapes(residual=residual)}
        self.names = names
        self.projs = []
        for nm in names:
            _, K, N, ranks = shapes[nm]
            self.projs.append(LittleBitProjection([make_device_branch(gen, K, R, N, dev) for R in ranks]))
        self.K = self.projs[0].in_features
        self.x = torch.randn((M, self.K), generator=gen).to(dev)
        self.outs = [torch.empty((M, p.out_features), device=dev) for p in self.projs]
        self.group = LittleBitProjectionGroup(self.projs) if grouped and len(self.projs) > 1 else None
        self.bytes = sum(proj_bytes(M, p.in_features, p.out_features, p.ranks) for p in self.projs)
        self.weight_bytes = sum(proj_bytes(M, p.in_features, p.out_features, p.ranks)
                                - 4 * M * (p.in_features + p.out_features) for p in self.projs)

    def run(self):
        if self.group is not None:
            self.group.forward(self.x, outs=self.outs)
        else:
            for p, o in zip(self.projs, self.outs):
                p.forward(self.x, out=o)


class DraftStep:
    """One replica of a step's 224 projections (32 layers x 7) as calls."""

    def __init__(self, gen, dev, layers, grouped=True, M=1, residual=False):
        self.calls = [Call(gen, dev, names, grouped, M, residual) for _ in range(layers) for _, names in LAYER_CALLS]

    @property
    def bytes(self):
        return sum(c.bytes for c in self.calls)

    @property
    def weight_bytes(self):
        return sum(c.weight_bytes for c in self.calls)

    def run(self):
        for c in self.calls:
            c.run()


class ChainStep:
    """One replica of a draft step's 224 projections with a decode step's
    data flow: q/k/v of RMSNorm(x); o of a fixed stand-in for the attention
    output, added to x (the residual stream); gate/up of RMSNorm(x); down of
    SiLU(gate) * up, added to x; then the next layer's q/k/v.  ``joined``
    runs each layer's o, gate/up, down and the next layer's q/k/v as one
    LittleBitChain (n + 1 launches for n links: 5 per layer); otherwise the
    same calls one by one (8 per layer).  Every step starts from the same x0
    (layer 0's o adds into x from x0), so replays repeat exactly."""

    def __init__(self, gen, dev, layers, joined=True):
        import torch
        from littlebit_amd import ChainLink, LittleBitChain, LittleBitProjection, LittleBitProjectionGroup
        from littlebit_amd.synthetic import llama_projection_shapes
        shapes = {s[0]: s for s in llama_projection_shapes(residual=False)}
        H, I = shapes["gate_proj"][1], shapes["gate_proj"][2]
        kv = shapes["k_proj"][2]
        self.joined = joined
        self.bytes = self.weight_bytes = 0
        self.layers = []
        for _ in range(layers):
            lp = {}
            for nm, (_, K, N, ranks) in shapes.items():
                lp[nm] = LittleBitProjection([make_device_branch(gen, K, R, N, dev) for R in ranks])
                self.bytes += proj_bytes(1, K, N, ranks)
                self.weight_bytes += proj_bytes(1, K, N, ranks) - 4 * (K + N)
            lp["ln1"] = (torch.rand(H, generator=gen) + 0.5).to(dev)
            lp["ln2"] = (torch.rand(H, generator=gen) + 0.5).to(dev)
            lp["qkv"] = LittleBitProjectionGroup([lp["q_proj"], lp["k_proj"], lp["v_proj"]])
            lp["gu"] = LittleBitProjectionGroup([lp["gate_proj"], lp["up_proj"]])
            self.layers.append(lp)
        self.x0 = torch.randn((1, H), generator=gen).to(dev)
        self.a = torch.randn((1, H), generator=gen).to(dev)
        self.x = torch.empty((1, H), device=dev)
        self.q, self.k, self.v = (torch.empty((1, n), device=dev) for n in (H, kv, kv))
        self.g, self.u = (torch.empty((1, I), device=dev) for _ in range(2))
        self.chains = []
        if joined:
            for li, lp in enumerate(self.layers):
                links = [ChainLink(lp["o_proj"], [self.x], residuals=[self.x0 if li == 0 else self.x]),
                         ChainLink(lp["gu"], [self.g, self.u], rms_weight=lp["ln2"]),
                         ChainLink(lp["down_proj"], [self.x], residuals=[self.x], silu_mul=True)]
                if li + 1 < len(self.layers):
                    nx = self.layers[li + 1]
                    links.append(ChainLink(nx["qkv"], [self.q, self.k, self.v], rms_weight=nx["ln1"]))
                self.chains.append(LittleBitChain(links))
        # whether every chain runs joined (not in deterministic mode)
        self.all_joined = joined and all(c.fused(self.a) for c in self.chains)

    def run(self):
        L0 = self.layers[0]
        L0["qkv"].forward(self.x0, outs=[self.q, self.k, self.v], rms_weight=L0["ln1"])
        if self.joined:
            for c in self.chains:
                c.forward(self.a)
            return
        for li, lp in enumerate(self.layers):
            lp["o_proj"].forward(self.a, out=self.x, residual=self.x0 if li == 0 else self.x)
            lp["gu"].forward(self.x, outs=[self.g, self.u], rms_weight=lp["ln2"])
            lp["down_proj"].forward(self.g, out=self.x, residual=self.x, x_up=self.u)
            if li + 1 < len(self.layers):
                nx = self.layers[li + 1]
                nx["qkv"].forward(self.x, outs=[self.q, self.k, self.v], rms_weight=nx["ln1"])


def chain_step_bench(gen, dev, stream, layers, steps, warmup, forms=(True, False)):
    """The decode step's 224 projections with their data flow, joined into
    chains and one by one, cold (replicas rotated) and warm."""
    out = {}
    for joined in forms:
        first = ChainStep(gen, dev, layers, joined)
        replicas = max(2, math.ceil(2 * MALL_BYTES / first.weight_bytes))
        reps = [first] + [ChainStep(gen, dev, layers, joined) for _ in range(replicas - 1)]
        graphs = [capture(r.run, stream) for r in reps]
        cold = time_graphs(graphs, steps, warmup, stream)
        warm = time_graphs(graphs[:1], steps, warmup, stream)
        key = "joined" if joined else "one_by_one"
        out[key] = {"ms_per_step": round(cold, 4), "warm_ms_per_step": round(warm, 4),
                    "value": round(first.bytes / (cold * 1e-3) / 1e9, 3), "bytes_per_step": first.bytes,
                    "replicas": replicas}
        del graphs, reps, first
    return out


def capture(fn, stream):
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        fn()  # warm: sizes this stream's workspace outside the capture
    stream.synchronize()
    with torch.cuda.graph(g, stream=stream):
        fn()
    return g


def time_graphs(graphs, steps, warmup, stream):
    import torch
    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for i in range(steps):
            graphs[i % len(graphs)].replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms per step


def call_duration_us(gen, dev, names, stream, count=32, steps=100, warmup=10):
    """Duration of one call (its latent + expand kernels and the gap between
    them) in a HIP graph of `count` back-to-back calls of one kind with
    distinct weights, from HIP events on the launch stream around the
    graph replays.  Returns (call, microseconds)."""
    calls = [Call(gen, dev, names) for _ in range(count)]
    g = capture(lambda: [c.run() for c in calls], stream)
    ms = time_graphs([g], steps, warmup, stream)
    return calls[0], ms * 1000.0 / count


def small_configs_bench(gen, dev, stream, count=32, steps=100, warmup=10):
    """BASELINE configs 0 and 1: one 4096 -> 4096 projection, draft branch R =
    205 alone (M = 1) and with the residual branch R = 1843 (M = 1, 2, 4, 8),
    fp32 in and out; microseconds per call in a graph of `count` calls with
    distinct weights (70 MB: the Infinity Cache holds them), and GB/s on the
    algorithmic bytes of BASELINE's formula."""
    import torch
    from littlebit_amd import LittleBitProjection
    K = N = 4096
    out = {}
    for name, ranks, M in [("config0", [205], 1)] + [(f"config1_m{m}", [205, 1843], m) for m in (1, 2, 4, 8)]:
        projs = [LittleBitProjection([make_device_branch(gen, K, R, N, dev) for R in ranks]) for _ in range(count)]
        x = torch.randn((M, K), generator=gen).to(dev)
        ys = [torch.empty((M, N), device=dev) for _ in range(count)]
        g = capture(lambda: [p.forward(x, out=y) for p, y in zip(projs, ys)], stream)
        us = time_graphs([g], steps, warmup, stream) * 1000.0 / count
        nbytes = sum(R * (-(-K // 32)) * 4 + N * (-(-R // 32)) * 4 + 4 * (K + R + N) for R in ranks) + 4 * M * K + 4 * M * N
        out[name] = {"M": M, "ranks": ranks, "us_per_call": round(us, 3), "bytes": nbytes,
                     "gbs": round(nbytes / us / 1e3, 2)}
        del projs, ys, g
    return out


def copy_ceiling(dev, stream, nbytes=512 << 20, reps=20):
    """Measured device-to-device copy bandwidth (torch copy_ of 512 MiB fp32,
    bytes read + written counted): the practical HBM ceiling beside the
    8 TB/s spec peak."""
    import torch
    src = torch.ones(nbytes // 4, device=dev)
    dst = torch.empty_like(src)
    with torch.cuda.stream(stream):
        for _ in range(3):
            dst.copy_(src)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            dst.copy_(src)
        b.record(stream)
    torch.cuda.synchronize()
    sec = a.elapsed_time(b) * 1e-3
    del src, dst
    torch.cuda.empty_cache()
    return {"gbs": round(2 * nbytes * reps / sec / 1e9, 1), "bytes_per_copy": 2 * nbytes,
            "method": f"torch copy_ of {nbytes >> 20} MiB fp32 device to device, read + written bytes, {reps} reps"}


def launch_floor_us(dev, stream, count=32, steps=100, warmup=10):
    """Duration of the smallest decode-path call (K = N = 256, rank 8, M = 1:
    the same latent + expand kernels with almost no work) in a graph of
    `count` back-to-back calls: the per-call floor of the two launches."""
    import torch
    from littlebit_amd import LittleBitProjection
    gen = torch.Generator().manual_seed(11)
    projs = [LittleBitProjection([make_device_branch(gen, 256, 8, 256, dev)]) for _ in range(count)]
    x = torch.randn((1, 256), generator=gen).to(dev)
    outs = [torch.empty((1, 256), device=dev) for _ in range(count)]
    g = capture(lambda: [p.forward(x, out=o) for p, o in zip(projs, outs)], stream)
    return time_graphs([g], steps, warmup, stream) * 1000.0 / count


# Llama-3-8B-shaped prefill, draft 0.1 BPW + residual 0.9 BPW
# per projection (ranks floor(bpw*K*N/(K+N))), M = 2048 bf16 tokens.
PREFILL_M = 2048
PREFILL_LAYER = [("qkv", [(4096, 4096, [204, 1843]), (4096, 1024, [81, 737]), (4096, 1024, [81, 737])]),
                 ("o", [(4096, 4096, [204, 1843])]),
                 ("gate/up", [(4096, 14336, [318, 2867]), (4096, 14336, [318, 2867])]),
                 ("down", [(14336, 4096, [318, 2867])])]
MFMA_BF16_PEAK_TFLOPS = 2500.0


def proj_flops(M, K, N, ranks):
    return sum(2 * M * (R * K + N * R) for R in ranks)


def _up(a, b):
    return -(-a // b) * b


def proj_mfma_flops(M, K, N, ranks):
    """Flops the GEMM path's MFMAs execute for one projection, tile padding
    included: stage 1 runs 128-row x 128-latent-row tiles over K in 64-k
    steps, stage 2 128 x 128 output tiles over each branch's sign words in
    64-k steps (two words).  Per kernel this is SQ_INSTS_VALU_MFMA_MOPS_BF16
    x 512 exactly (profiles/littlebit_prefill_llama3.md)."""
    Mp, Np, Kp = _up(M, 128), _up(N, 128), _up(K, 64)
    return sum(2 * Mp * _up(R, 128) * Kp + 2 * Mp * Np * 64 * _up(-(-R // 32), 2) // 2 for R in ranks)


class PrefillLayer:
    """One decoder layer's linears at M tokens (bf16 in, bf16 out), as calls."""

    def __init__(self, gen, dev, M):
        import torch
        from littlebit_amd import LittleBitProjection, LittleBitProjectionGroup
        self.calls = []
        self.flops = 0
        self.mfma_flops = 0
        for kind, shapes in PREFILL_LAYER:
            projs = [LittleBitProjection([make_device_branch(gen, K, R, N, dev) for R in ranks])
                     for K, N, ranks in shapes]
            K = shapes[0][0]
            x = torch.randn((M, K), generator=gen).to(torch.bfloat16).to(dev)
            outs = [torch.empty((M, N), dtype=torch.bfloat16, device=dev) for _, N, _ in shapes]
            self.calls.append((kind, LittleBitProjectionGroup(projs), x, outs))
            self.flops += sum(proj_flops(M, K, N, ranks) for K, N, ranks in shapes)
            self.mfma_flops += sum(proj_mfma_flops(M, K, N, ranks) for K, N, ranks in shapes)

    def run(self, only=None):
        for kind, grp, x, outs in self.calls:
            if only is None or kind == only:
                grp.forward(x, outs=outs)


def lm_head_bench(dev, stream, steps=100, warmup=10, copies=4):
    """The draft step's Q4_0 lm_head + argmax (Llama-2-7B: 32000 x 4096) on
    its own: ``copies`` quantised weights rotated so that each call reads
    its planes from HBM (4 x 74 MB > the 256 MB Infinity Cache)."""
    import torch
    from littlebit_amd.lm_head import Q4LMHead
    g = torch.Generator(device="cpu").manual_seed(3)
    V, H = 32000, 4096
    heads = []
    for _ in range(copies):
        w = torch.randn((V, H), generator=g).to(dev)
        heads.append(Q4LMHead(w))
        del w
    x = torch.randn(H, generator=g).to(dev)
    nw = torch.ones(H, device=dev)
    tok = torch.zeros(1, dtype=torch.int64, device=dev)
    with torch.cuda.stream(stream):
        for i in range(warmup):
            heads[i % copies].argmax(x, nw, 1e-6, out=tok)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(steps):
            heads[i % copies].argmax(x, nw, 1e-6, out=tok)
        b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1000.0 / steps
    nbytes = heads[0].nbytes + 4 * H * 2
    return {"workload": f"Q4_0 lm_head + argmax, vocab {V} x hidden {H}, final RMSNorm fused, {copies} weight "
                        "copies rotated (cold)", "us_per_call": round(us, 2), "bytes_per_call": nbytes,
            "gbs": round(nbytes / us / 1000.0, 1), "launches": 2}


def prefill_library_reference(dev, stream, steps=20, warmup=3):
    """The same layer as plain bf16 GEMMs through the vendor library (torch.matmul -> hipBLASLt), a reference point
    for the hand-written kernels and not a path of this library: weights already dense bf16 (no sign expansion),
    stage 1 = x[M, K] @ [V_b]^T over the group's branches concatenated, stage 2 = T_b @ [U_0 | U_1]^T per
    projection, both weights stored [N, K] (the layout the library ran fastest in at these shapes), 2 copies of the
    layer rotated, one graph per call kind."""
    import torch
    g = torch.Generator().manual_seed(7)
    rnd = lambda *s: torch.randn(s, generator=g).to(torch.bfloat16).to(dev)  # noqa: E731
    per_kind, total_ms = {}, 0.0
    for kind, shapes in PREFILL_LAYER:
        K = shapes[0][0]
        rs = sum(sum(ranks) for _, _, ranks in shapes)
        copies = []
        for _ in range(2):
            x = rnd(PREFILL_M, K)
            w1 = rnd(rs, K)
            w2 = [(rnd(PREFILL_M, sum(ranks)), rnd(N, sum(ranks))) for _, N, ranks in shapes]
            copies.append((x, w1, w2))

        def run(c):
            x, w1, w2 = c
            torch.matmul(x, w1.t())
            for t, w in w2:
                torch.matmul(t, w.t())
        graphs = [capture(lambda c=c: run(c), stream) for c in copies]
        ms = time_graphs(graphs, steps, warmup, stream)
        per_kind[kind] = round(ms * 1000.0, 2)
        total_ms += ms
        del graphs, copies
    flops = sum(proj_flops(PREFILL_M, K, N, ranks) for _, shapes in PREFILL_LAYER for K, N, ranks in shapes)
    return {"what": "plain bf16 GEMMs of the same shapes through torch.matmul (hipBLASLt) on dense bf16 weights: "
                    "a reference point, not this library's path", "ms_per_layer": round(total_ms, 4),
            "tflops": round(flops / (total_ms * 1e-3) / 1e12, 1), "us_per_call": per_kind}


def prefill_bench(gen, dev, stream, steps=20, warmup=3, library_reference=True):
    """ms per layer and TFLOP/s of the config-4 linears (2 layers' weights rotated)."""
    layers = [PrefillLayer(gen, dev, PREFILL_M) for _ in range(2)]
    graphs = [capture(l.run, stream) for l in layers]
    ms = time_graphs(graphs, steps, warmup, stream)
    per_call = {}
    for kind, _ in PREFILL_LAYER:
        g = [capture(lambda l=l: l.run(kind), stream) for l in layers]
        per_call[kind] = round(time_graphs(g, steps, warmup, stream) * 1000.0, 2)
    tflops = layers[0].flops / (ms * 1e-3) / 1e12
    executed = layers[0].mfma_flops / (ms * 1e-3) / 1e12
    out = {"workload": "llama3-8b prefill linears, 1 layer (q/k/v, o, gate/up, down; draft + residual branches)",
           "M": PREFILL_M, "dtype": "bf16", "ms_per_layer": round(ms, 4),
           "ms_per_forward_32_layers": round(32 * ms, 3), "flops_per_layer": layers[0].flops,
           "tflops": round(tflops, 1), "mfma_peak_tflops": MFMA_BF16_PEAK_TFLOPS,
           "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
           "mfma_flops_executed_per_layer": layers[0].mfma_flops,
           "mfma_frac_executed": round(executed / MFMA_BF16_PEAK_TFLOPS, 4), "us_per_call": per_call}
    del graphs, layers
    if library_reference:
        out["library_reference"] = prefill_library_reference(dev, stream, steps, warmup)
    return out


def verify_linears_bench(gen, dev, stream, layers=32, M=8, steps=50, warmup=5, per_class=True):
    """The ~1.0-BPW target's verify linears: the 224 target projections (draft +
    residual branch each) at M = 8 (a verify of 8 draft tokens), grouped as in the draft step, one HIP graph per
    pass, weights cold (2 replicas of 0.9 GB rotated).  ``per_class``: each call kind's duration at M = 8 in a
    graph of 32 calls with distinct weights, and a roofline block for the longest one."""
    import torch
    reps = [DraftStep(gen, dev, layers, M=M, residual=True) for _ in range(2)]
    graphs = [capture(r.run, stream) for r in reps]
    ms = time_graphs(graphs, steps, warmup, stream)
    b = reps[0].bytes
    del graphs, reps
    gbs = b / (ms * 1e-3) / 1e9
    out = {"workload": f"llama2-7b 1.0-bpw target linears, {layers} layers x 7 projections at M={M} "
                       "(draft rank 205/298 + residual 1843/2686 per projection), fp32",
           "ms_per_pass": round(ms, 4), "us_per_layer": round(ms * 1000.0 / layers, 2),
           "bytes_per_pass": b, "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if not per_class:
        return out
    cls = {}
    for kind, names in LAYER_CALLS:
        calls = [Call(gen, dev, names, M=M, residual=True) for _ in range(32)]
        g = capture(lambda: [c.run() for c in calls], stream)
        us = time_graphs([g], steps, warmup, stream) * 1000.0 / 32
        cls[kind] = {"projections": "+".join(names), "us_per_call": round(us, 3), "bytes": calls[0].bytes,
                     "gbs": round(calls[0].bytes / us / 1e3, 2)}
        del calls, g
    dom = max(cls, key=lambda c: cls[c]["us_per_call"])
    d = cls[dom]
    out["per_class"] = cls
    out["roofline"] = {"bound": "hbm", "achieved": d["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": round(d["gbs"] / HBM_PEAK_GBS, 5), "traffic": MEASURED_TRAFFIC_M8.get(dom),
                       "traffic_source": "not measured in this run: calibrated rocprofv3 FETCH_SIZE + WRITE_SIZE of "
                                         "the same call kind at M = 8, profiles/littlebit_verify_m8_target.md",
                       "kernel": f"LittleBitLinear {dom} call at M = {M} ({d['projections']}, draft + residual "
                                 "branches): latent_mfma_kernel + expand_mfma_kernel",
                       "bytes_per_launch": d["bytes"], "us_per_launch": d["us_per_call"]}
    return out


def decode_bench(dev, draft_len=8, kv_draft=512, kv_target=1024, replays=32, target=True):
    """0.1-BPW draft tokens at KV length 512 and ~1.0-BPW target verification
    (8 tokens, and a 33-token tree) at KV length 1024 on whole Llama-2-7B-shaped
    models (random packed factors, |N|+0.05 scales; embedding and lm_head
    N(0,1)): linears, attention and the Q4_0 lm_head on the HIP kernels,
    norms inside the linear calls, one HIP graph per step."""
    import torch
    from littlebit_amd.decode import DecoderConfig, GPUDraftModel, GPUTargetModel
    from littlebit_amd.synthetic import LLAMA2_7B as C, synthetic_runtime_state
    from littlebit_amd.tree import config3_tree_choices, generate_tree_buffers
    cfg = DecoderConfig(hidden_size=C["hidden"], intermediate_size=C["intermediate"], num_hidden_layers=C["layers"],
                        num_attention_heads=C["heads"], num_key_value_heads=C["kv_heads"], vocab_size=C["vocab"])
    ev = lambda: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))  # noqa: E731
    out = {}
    gen = torch.Generator().manual_seed(5)
    # --- draft model (0.1 BPW), KV length 512 -------------------------------------
    st = synthetic_runtime_state(cfg, C["draft_rank"], None, seed=1, device=dev)
    prompt = torch.randint(0, cfg.vocab_size, (1, kv_draft), generator=gen)

    def measure_draft(head):
        draft = GPUDraftModel(state=st, config=cfg, device=dev, max_seq_len=kv_draft + replays + draft_len + 8,
                              torch_dtype=torch.bfloat16, lm_head=head)
        draft.generate_draft_tokens(prompt, draft_length=2)  # prefill + builds the graph
        torch.cuda.synchronize()
        draft._pos.fill_(kv_draft)
        for _ in range(3):
            draft._graph.replay()
        draft._pos.fill_(kv_draft)
        a, b = ev()
        a.record()
        for _ in range(replays):
            draft._graph.replay()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / replays
        a, b = ev()
        a.record()
        draft.generate_draft_tokens(prompt, draft_length=draft_len)
        b.record()
        torch.cuda.synchronize()
        gen_ms = a.elapsed_time(b)
        del draft
        torch.cuda.empty_cache()
        return ms, gen_ms

    ms_tok, gen_ms = measure_draft("q4")
    ms_dense, _ = measure_draft("dense")
    out["draft"] = {"workload": f"llama2-7b 0.1-bpw draft, one token at KV length {kv_draft}: embedding, 32 layers "
                                "(norms, attention, 7 LittleBitLinear forwards), final norm, Q4_0 lm_head (Q8_0 "
                                "activations) and argmax as the reference's generate_token; one HIP graph per token",
                    "ms_per_token": round(ms_tok, 4), "tok_per_s": round(1000.0 / ms_tok, 1),
                    f"generate_draft_tokens_k{draft_len}_ms": round(gen_ms, 3),
                    "dense_bf16_lm_head": {"ms_per_token": round(ms_dense, 4),
                                           "tok_per_s": round(1000.0 / ms_dense, 1)}}
    del st
    torch.cuda.empty_cache()
    if not target:
        return out
    # --- 1.0-BPW target (draft + residual branch per projection), KV length 1024
    st = synthetic_runtime_state(cfg, C["draft_rank"], C["residual_rank"], seed=2, device=dev)
    target = GPUTargetModel(draft_state=st, config=cfg, device=dev, max_seq_len=kv_target + 64,
                            torch_dtype=torch.bfloat16)
    prefix = torch.randint(0, cfg.vocab_size, (1, kv_target), generator=gen)
    target.forward(prefix)
    toks = torch.randint(0, cfg.vocab_size, (1, draft_len), generator=gen)

    import torch.nn.functional as F
    from littlebit_amd.synthetic import llama_projection_shapes
    unit, W = target.draft_unit, target.lm_head_weight
    stream = torch.cuda.Stream()
    bufs = generate_tree_buffers(config3_tree_choices(), device=dev)
    tree = [int(prefix[0, -1])] + torch.randint(0, cfg.vocab_size, (bufs["tree_len"] - 1,), generator=gen).tolist()
    x_v = target.embed_tokens.index_select(0, toks[0].to(dev))
    x_t = target.embed_tokens.index_select(0, torch.tensor(tree, device=dev))
    tmask = bufs["tree_attn_mask"][0, 0].bool()

    def vstep():  # the draft_len new tokens after the prefix, causal
        F.linear(unit.forward_hidden(x_v, kv_target).to(W.dtype), W)

    def tstep():  # root (last prefix token) + tree nodes, ancestor mask
        F.linear(unit.forward_hidden(x_t, kv_target - 1, tree_mask=tmask).to(W.dtype), W)

    ms_v = time_graphs([capture(vstep, stream)], 20, 3, stream)
    ms_t = time_graphs([capture(tstep, stream)], 20, 3, stream)
    vbytes = 32 * sum(proj_bytes(draft_len, K, N, ranks) for _, K, N, ranks in llama_projection_shapes(residual=True))
    out["verify"] = {"workload": f"llama2-7b 1.0-bpw target (draft + residual branch per projection) at KV length "
                                 f"{kv_target}: {draft_len} tokens in one forward, and a {bufs['tree_len'] - 1}-node "
                                 "tree (depth 5, branching <= 4) plus its root in one forward with the tree mask; "
                                 "each one HIP graph (32 layers, attention, norms, bf16 lm_head)",
                     f"verify_{draft_len}_ms": round(ms_v, 4), "tree_verify_ms": round(ms_t, 4),
                     f"linear_bytes_per_verify": vbytes,
                     f"round_ms_k{draft_len}": round(draft_len * ms_tok + ms_v, 3)}
    return out


def cpu_baseline(layers, budget_s=12.0):
    """The reference's CPU kernels (oracle/_ref, the reference patch compiled
    from its source) on this host, within a time budget of about 3 x budget_s:

    * value: ``littlebit_linear`` (int32-packed signs, int8 activations) over
      whole draft steps, the 224 linears of config 2, in GB/s of the same
      algorithmic bytes as the GPU value -- the reference's fastest linears
      on a many-core host (its i2 linears, timed through ``full_forward`` at
      position 0, run their first stage on one thread);
    * the same op on the 1.0-BPW target's verify linears at M = 8 (both
      branches of every projection; a sample of layers, scaled to 32);
    * ``generate_token``, the reference's fastest CPU draft token (i2 signs,
      attention at KV 512, Q4_0 lm_head; patch:2254-2317), 32 layers;
    * ``full_forward_batch`` of 8 tokens at KV 1024 for the two-unit target
      (draft model + residual model, patch:1846-2079), per layer, scaled to 32.

    Threads: all physical cores, but at most 16 (the CPU share of one GPU's
    jobs on the GPU box), and 4 as the reference's run scripts use
    (eval_speculative_matryoshka_cpu.sh:45)."""
    import torch
    try:
        from oracle import build_ref, ref_runtime as RR  # checker / baseline only
        ops = build_ref.load()
    except Exception as e:  # noqa: BLE001
        return {"value": None, "unit": "GB/s", "cores": 0, "kind": "reference",
                "sample": f"unavailable: {e}"}
    facts = RR.cpu_facts()
    phys = facts.get("physical_cores") or (os.cpu_count() or 1)
    threads = max(1, min(16, phys))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(7)

    def timed(fn, budget):
        fn()
        t0 = time.perf_counter()
        n = 0
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget or n >= 100000:
                return n, el

    # --- draft-step linears (value) --------------------------------------------
    step = []
    for _ in range(layers):
        for name, K, N, ranks in draft_layer_shapes():
            R = ranks[0]
            b = make_device_branch(gen, K, R, N, "cpu")
            x = torch.randn((1, K), generator=gen)
            step.append((K, N, R, x, b))
    step_bytes = sum(proj_bytes(1, K, N, [R]) for K, N, R, _, _ in step)

    def one_step():
        for K, N, R, x, b in step:
            ops.littlebit_linear(x, b.v2.reshape(1, K), b.v_sign, K, b.mid.reshape(1, R), b.u_sign, R,
                                 b.u1.reshape(1, N))

    steps, el = timed(one_step, budget_s * 0.5)
    ms_step = el / steps * 1000.0
    torch.set_num_threads(4)
    steps4, el4 = timed(one_step, budget_s * 0.25)
    torch.set_num_threads(threads)
    ms4 = el4 / steps4 * 1000.0
    del step

    # --- verify linears at M = 8: both branches of every target projection ------
    from littlebit_amd.synthetic import llama_projection_shapes
    vl = 4  # layers in the sample
    vstep = []
    for _ in range(vl):
        for name, K, N, ranks in llama_projection_shapes(residual=True):
            brs = [make_device_branch(gen, K, R, N, "cpu") for R in ranks]
            vstep.append((K, N, torch.randn((8, K), generator=gen), brs))
    vbytes = 32 * sum(proj_bytes(8, K, N, ranks) for _, K, N, ranks in llama_projection_shapes(residual=True))

    def verify_layers():
        for K, N, x, brs in vstep:
            y = None
            for b in brs:
                R = b.rank
                o = ops.littlebit_linear(x, b.v2.reshape(1, K), b.v_sign, K, b.mid.reshape(1, R), b.u_sign, R,
                                         b.u1.reshape(1, N))
                y = o if y is None else y + o

    nv, elv = timed(verify_layers, budget_s * 0.35)
    ms_verify = elv / nv * 1000.0 * 32 / vl
    del vstep

    # --- the reference's decode runtime ------------------------------------------
    H, I, V, HD = 4096, 11008, 32000, 128
    draft_layers, draft_dims = RR.build_layers(ops, H, I, H, {"attn": 205, "mlp": 298}, layers, seed=3)
    # the runtime's i2 linears: full_forward at position 0 (attention over one position)
    ff_s, ff_n = RR.time_full_forward(ops, draft_layers, draft_dims, layers, H, V, 32, HD, 0, 600, budget_s * 0.15)
    tok_s, tok_n = RR.time_generate_token(ops, draft_layers, draft_dims, layers, H, V, 32, HD, 512, 600,
                                          budget_s * 0.35)
    torch.set_num_threads(4)
    tok4_s, tok4_n = RR.time_generate_token(ops, draft_layers, draft_dims, layers, H, V, 32, HD, 512, 600,
                                            budget_s * 0.2)
    torch.set_num_threads(threads)
    ffb_d, nd = RR.time_full_forward_batch(ops, draft_layers, draft_dims, layers, H, V, 32, HD, 8, 1024, 1040,
                                           budget_s * 0.2)
    del draft_layers
    rl = 4
    res_layers, res_dims = RR.build_layers(ops, H, I, H, {"attn": 1843, "mlp": 2686}, rl, seed=4)
    ffb_r, nr = RR.time_full_forward_batch(ops, res_layers, res_dims, rl, H, V, 32, HD, 8, 1024, 1040,
                                           budget_s * 0.25)
    del res_layers
    verify_ms = (ffb_d + ffb_r * layers / rl) * 1000.0
    return {"value": round(step_bytes * steps / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "reference",
            "cpu": facts, "threads": threads,
            "thread_note": "all physical cores capped at 16, the CPU share of one GPU's jobs on the GPU box",
            "ms_per_step": round(ms_step, 3), "tok_per_s_linears": round(1000.0 / ms_step, 2),
            "threads_4": {"value": round(step_bytes * steps4 / el4 / 1e9, 3), "ms_per_step": round(ms4, 3),
                          "steps": steps4},
            "verify_linears_m8": {"ms_per_pass": round(ms_verify, 2), "gbs": round(vbytes / ms_verify / 1e6, 3),
                                  "sample": f"{vl} layers x 7 projections (draft + residual branch each, summed), "
                                            f"{nv} passes in {elv:.1f} s, scaled to 32 layers"},
            "draft_step_i2_full_forward": {
                "ms_per_step": round(ff_s * 1000.0, 3), "gbs": round(step_bytes / ff_s / 1e9, 3), "calls": ff_n,
                "workload": f"full_forward at position 0: the runtime's {layers} layers of i2 linears (patch:1320-1369; "
                            "their first stage runs on one thread) with RMSNorms, SiLU * up and residual adds, "
                            "attention over one position; GB/s on the draft step's algorithmic bytes"},
            "draft_token_generate_token": {
                "ms_per_token": round(tok_s * 1000.0, 3), "tok_per_s": round(1.0 / tok_s, 2), "tokens": tok_n,
                "threads_4": {"ms_per_token": round(tok4_s * 1000.0, 3), "tokens": tok4_n},
                "workload": f"{layers} layers, ranks 205/298, i2 signs, attention at KV 512, Q4_0 lm_head "
                            "32000 x 4096 and argmax"},
            "verify_8_full_forward_batch": {
                "ms_per_verify": round(verify_ms, 2),
                "workload": f"two-unit target: draft model ({layers} layers, ranks 205/298, {nd} calls) + residual "
                            f"model (ranks 1843/2686, {rl}-layer sample x {layers // rl}, {nr} calls), 8 tokens at "
                            "KV 1024, hidden states only"},
            "sample": (f"littlebit_cpu_ops::littlebit_linear (reference AVX2 kernel, int8 activations) over "
                       f"{steps} whole draft steps ({layers} layers x 7 projections, distinct weights, "
                       f"{step_bytes / 2**20:.0f} MiB per step) in {el:.1f} s; torch intra-op threads = {threads}; "
                       f"threads_4: the same with 4 threads, {steps4} steps in {el4:.1f} s")}


def stage_handoff(stages: int = 64):
    """One dependent stage as a kernel boundary (launches in a graph) and as
    a grid-wide handoff inside one launch (agent-scope stores, non-returning
    counter adds, polled counters; littlebit_amd/csrc/handoff_probe.hip), in
    us per stage.  Run as a child process (the probe is its own program)."""
    import subprocess
    from littlebit_amd.build import PROBE_PATH
    if not PROBE_PATH.exists():
        return {"error": f"{PROBE_PATH} not built (python -m littlebit_amd.build)"}
    proc = subprocess.run([str(PROBE_PATH), str(stages)], capture_output=True, text=True, timeout=120)
    if proc.returncode != 0:
        return {"error": f"handoff probe exited {proc.returncode}: {proc.stderr[-500:]}"}
    out = json.loads(proc.stdout.strip().splitlines()[-1])
    out["program"] = "littlebit_amd/csrc/handoff_probe.hip"
    return out


def mfma_issue():
    """What the GEMM path's mainloop can sustain: 32x32x16 bf16 MFMAs with V
    independent (or B-operand-rewriting) VALU instructions after each, and
    with A fragments read from LDS (littlebit_amd/csrc/mfma_issue_probe.hip),
    at two and three waves per SIMD, and the mainloop's skeleton with and
    without its A-tile loads.  Run as a child process."""
    import subprocess
    from littlebit_amd.build import ISSUE_PROBE_PATH
    if not ISSUE_PROBE_PATH.exists():
        return {"error": f"{ISSUE_PROBE_PATH} not built (python -m littlebit_amd.build)"}
    proc = subprocess.run([str(ISSUE_PROBE_PATH)], capture_output=True, text=True, timeout=120)
    if proc.returncode != 0:
        return {"error": f"MFMA issue probe exited {proc.returncode}: {proc.stderr[-500:]}"}
    return {"program": "littlebit_amd/csrc/mfma_issue_probe.hip",
            "cases": [json.loads(l) for l in proc.stdout.strip().splitlines()]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-4 prefill measurement")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-2/3 whole-model decode measurement")
    ap.add_argument("--only", choices=["qkv", "o", "gate_up", "down", "prefill", "decode", "draft", "verify", "copy",
                                       "lm_head", "small", "handoff", "issue", "chain", "chain_joined"], default=None,
                    help="profiling aid: replay only this call kind (32 per graph) and print its timing")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build uses no collectives); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    # the handoff probe is its own program: it runs as a child process before
    # this process touches the GPU (a process that has initialised the GPU
    # starts no other program)
    handoff = None if args.only not in (None, "handoff") else stage_handoff()
    if args.only == "handoff":
        print(json.dumps(handoff))
        return
    if args.only == "issue":
        print(json.dumps(mfma_issue()))
        return

    import torch
    import littlebit_amd._lib as L
    L.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()

    gen = torch.Generator().manual_seed(1002)
    kinds = dict(LAYER_CALLS)
    if args.only == "prefill":
        print(json.dumps(prefill_bench(gen, dev, stream, args.steps, args.warmup)))
        return
    if args.only == "lm_head":
        print(json.dumps(lm_head_bench(dev, stream, args.steps, args.warmup)))
        return

    if args.only == "small":
        print(json.dumps(small_configs_bench(gen, dev, stream, steps=args.steps, warmup=args.warmup)))
        return
    if args.only == "copy":
        # calibration for the HBM byte counters: a plain device copy of known size
        n = 64 << 20  # floats: 256 MiB read + 256 MiB written per copy
        src = torch.randn(n, device=dev)
        dst = torch.empty_like(src)
        for _ in range(max(args.steps, 1)):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"only": "copy", "bytes_read_per_copy": 4 * n, "bytes_written_per_copy": 4 * n,
                          "copies": max(args.steps, 1)}))
        return
    if args.only in ("decode", "draft"):
        print(json.dumps(decode_bench(dev, target=args.only == "decode")))
        return
    if args.only in ("chain", "chain_joined"):
        forms = (True,) if args.only == "chain_joined" else (True, False)
        print(json.dumps(chain_step_bench(gen, dev, stream, args.layers, args.steps, args.warmup, forms)))
        return
    if args.only == "verify":
        print(json.dumps(verify_linears_bench(gen, dev, stream, args.layers, steps=args.steps, warmup=args.warmup)))
        return
    if args.only:
        names = kinds[args.only.replace("gate_up", "gate/up")]
        call, us = call_duration_us(gen, dev, names, stream, args.layers, args.steps, args.warmup)
        print(json.dumps({"only": args.only, "projections": list(names), "us_per_call_in_graph": round(us, 3),
                          "bytes_per_call": call.bytes, "gbs": round(call.bytes / us / 1e3, 2)}))
        return
    first = ChainStep(gen, dev, args.layers, joined=True)
    assert first.all_joined, "the chained draft step runs its chains joined"
    step_bytes, weight_bytes = first.bytes, first.weight_bytes
    replicas = max(2, math.ceil(2 * MALL_BYTES / weight_bytes))
    steps_list = [first] + [ChainStep(gen, dev, args.layers, joined=True) for _ in range(replicas - 1)]
    graphs = [capture(s.run, stream) for s in steps_list]
    ms_cold = time_graphs(graphs, args.steps, args.warmup, stream)
    ms_warm = time_graphs(graphs[:1], args.steps, args.warmup, stream)
    del graphs, steps_list, first

    def step_ms(make, det=False):
        import littlebit_amd as lb
        with lb.deterministic(det):
            reps = [make() for _ in range(replicas)]
            gs = [capture(r.run, stream) for r in reps]
            ms = time_graphs(gs, args.steps, args.warmup, stream)
        del gs, reps
        return ms
    # the same step with each call on its own (two launches per call)
    ms_one = step_ms(lambda: ChainStep(gen, dev, args.layers, joined=False))
    # in deterministic mode the chains run as separate calls, with fixed-order split-K sums
    ms_det = step_ms(lambda: ChainStep(gen, dev, args.layers, joined=True), det=True)
    # the previous workload: 224 calls with independent inputs, grouped, and every projection alone
    ms_indep = step_ms(lambda: DraftStep(gen, dev, args.layers))
    ms_single = step_ms(lambda: DraftStep(gen, dev, args.layers, grouped=False))

    # per call kind (each call alone): duration in a graph of back-to-back calls of that kind
    cls_stats = {}
    for kind, names in LAYER_CALLS:
        call, us = call_duration_us(gen, dev, names, stream)
        cls_stats[kind] = {"projections": "+".join(names), "us_per_call": round(us, 3), "bytes": call.bytes,
                           "gbs": call.bytes / us / 1e3, "traffic": MEASURED_TRAFFIC.get(kind)}
    ceiling = copy_ceiling(dev, stream)
    floor_us = launch_floor_us(dev, stream)
    # the dominant unit of the step: one layer's chain (7 projections, 5
    # kernels: o's latent stage, three joined kernels, q/k/v's expand stage),
    # the step's HIP-event time per layer
    layer_bytes = step_bytes / args.layers
    layer_us = ms_cold * 1000.0 / args.layers
    layer_gbs = layer_bytes / layer_us / 1e3
    roofline = {"bound": "hbm", "achieved": round(layer_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(layer_gbs / HBM_PEAK_GBS, 5), "traffic": MEASURED_TRAFFIC_CHAIN,
                "traffic_source": "not measured in this run: calibrated rocprofv3 FETCH_SIZE + WRITE_SIZE of one "
                                  "layer's chain kernels, profiles/littlebit_decode_chain.md",
                "copy_ceiling_gbs": ceiling["gbs"], "frac_of_copy_ceiling": round(layer_gbs / ceiling["gbs"], 5),
                "kernel": "one layer's LittleBitChain o -> gate/up -> down -> next q/k/v: latent_mfma_kernel + "
                          "3 x chain_mfma_kernel + expand_mfma_kernel",
                "bytes_per_launch": round(layer_bytes), "us_per_launch": round(layer_us, 3)}

    small = small_configs_bench(gen, dev, stream)
    verify_lin = verify_linears_bench(gen, dev, stream, args.layers)
    verify_lin["frac_of_copy_ceiling"] = round(verify_lin["gbs"] / ceiling["gbs"], 4)
    prefill = None if args.no_prefill else prefill_bench(gen, dev, stream)
    decode = None if args.no_decode else decode_bench(dev)
    cpu = None if args.no_cpu else cpu_baseline(args.layers, args.cpu_budget)
    value = step_bytes / (ms_cold * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_cold, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "llama2-7b-draft-0.1bpw-decode-step (224 LittleBitLinear forwards, M=1, the decode "
                               "step's data flow: RMSNorm, SiLU * up and residual adds fused)",
                   "launches": "5 per layer: o -> gate/up -> down -> next q/k/v as one LittleBitChain "
                               "(2 for layer 0's q/k/v)",
                   "layers": args.layers, "hidden": 4096, "intermediate": 11008,
                   "ranks": {"attn": 205, "mlp": 298}, "batch": 1, "activations": "fp32",
                   "bytes_per_step": step_bytes, "weight_bytes_per_step": weight_bytes,
                   "cache": f"cold: {replicas} weight replicas rotated ({replicas * weight_bytes / 2**20:.0f} MiB "
                            f"> 256 MiB Infinity Cache)", "graph": "one HIP graph per step"},
        "us_per_layer": round(ms_cold * 1000.0 / args.layers, 3),
        "tok_per_s_linears": round(1000.0 / ms_cold, 2),
        "warm": {"ms_per_step": round(ms_warm, 4), "value": round(step_bytes / (ms_warm * 1e-3) / 1e9, 3),
                 "us_per_layer": round(ms_warm * 1000.0 / args.layers, 3)},
        "one_by_one": {"ms_per_step": round(ms_one, 4), "value": round(step_bytes / (ms_one * 1e-3) / 1e9, 3),
                       "launches": "8 per layer: the same calls each on its own (q/k/v and gate/up as group "
                                   "calls), cold"},
        "independent_calls": {"ms_per_step": round(ms_indep, 4),
                              "value": round(step_bytes / (ms_indep * 1e-3) / 1e9, 3),
                              "launches": "8 per layer: 224 calls with independent plain inputs (q/k/v and "
                                          "gate/up grouped), cold"},
        "ungrouped": {"ms_per_step": round(ms_single, 4), "value": round(step_bytes / (ms_single * 1e-3) / 1e9, 3),
                      "launches": "14 per layer (independent calls, each projection alone), cold"},
        "deterministic": {"ms_per_step": round(ms_det, 4), "value": round(step_bytes / (ms_det * 1e-3) / 1e9, 3),
                          "note": "lbk_set_deterministic(1): the chains run as separate calls, split-K partials "
                                  "summed in chunk order, bit-for-bit repeatable; cold"},
        "per_class": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                      for k, v in cls_stats.items()},
        "roofline": roofline,
        "ceilings": {"hbm_peak_gbs": HBM_PEAK_GBS, "copy": ceiling,
                     "value_frac_of_copy_ceiling": round(value / ceiling["gbs"], 5),
                     "launch_floor_us_per_call": round(floor_us, 3),
                     "launch_floor_ms_per_step": round(floor_us * len(LAYER_CALLS) * args.layers / 1000.0, 4),
                     "launch_floor_note": "smallest decode-path call (K = N = 256, rank 8, M = 1): the latent + "
                                          "expand launches with almost no work, in a graph of 32 calls; a step "
                                          f"of calls each on its own is {len(LAYER_CALLS) * args.layers} such "
                                          "calls, the chained step 5/8 as many launches",
                     "stage_handoff": handoff},
        "configs_0_1": small,
        "verify_linears": verify_lin,
        "prefill": prefill,
        "decode": decode,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()

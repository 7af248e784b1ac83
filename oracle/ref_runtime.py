"""The reference's own CPU decode runtime, driven on synthetic weights.

TEST / BASELINE INFRASTRUCTURE ONLY.  Nothing in the product (``littlebit_amd``)
may import this module: only ``tests/`` and ``bench.py``'s ``cpu_baseline``
leg use it, to time the reference's fastest CPU paths on the host beside the
GPU figures.  It needs ``oracle/_ref`` (the reference patch compiled in place
by ``oracle/build_ref.py``).

The argument lists follow the reference's call sites:

* ``layer_tensors`` / ``layer_dims`` as ``CPUDraftModel`` builds them for
  ``full_forward`` (cpu_draft_model.py:225-264): per layer the two RMSNorm
  weights, then per projection (q, k, v, o, gate, up, down) ``v2``, the
  ``repack_signs_to_i2`` V words, ``mid``, the i2 U words and ``u1``
  (patch:1307-1317); dims ``[v_cols, rank, u_cols, out_features]``;
* KV caches ``[kv_heads, max_seq, head_dim]`` fp32 per layer and tensor
  (patch:1451-1456, 1726-1727);
* ``generate_token`` (patch:2254-2317) adds the Q4_0 lm_head of
  ``quantize_lm_head_q4`` and the argmax; ``full_forward_batch``
  (patch:1846-2079) verifies N tokens, token-serial in its linears.

The reference ops compute with int8 activations and 2-bit signs whose tails
are inexact when a rank is not a multiple of 128 (patch:749-758, 855-869);
they are timed here, not checked.  ``littlebit_linear_i2`` (patch:873-967) is
not used: its scratch is ``thread_local`` and resized on the calling thread
only, while its ``at::parallel_for`` lambdas name that scratch, so a worker
thread reads its own empty vectors (null data) and the process faults whenever
the U stage runs in parallel (any out_features > 256 with more than one
thread).  ``full_forward`` passes caller-owned buffers to its linears
(``lb_linear_i2_inline``, patch:1320-1369) and runs.
"""
from __future__ import annotations

import time
from typing import Dict, List, Sequence, Tuple

import numpy as np

PROJ = ("q", "k", "v", "o", "gate", "up", "down")


def _words(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    wpr = (cols + 31) // 32
    w = rng.integers(0, 2**32, size=(rows, wpr), dtype=np.uint32)
    tail = cols - 32 * (wpr - 1)
    if tail < 32:
        w[:, -1] &= np.uint32((1 << tail) - 1)
    return w.view(np.int32)


def _scales(rng: np.random.Generator, n: int) -> np.ndarray:
    return (np.abs(rng.standard_normal(n)) + 0.05).astype(np.float32)


def build_layers(ops, hidden: int, inter: int, kv_dim: int, ranks: Dict[str, int], n_layers: int,
                 seed: int = 0) -> Tuple[List, List[int]]:
    """(layer_tensors, layer_dims) of ``n_layers`` random LittleBit layers
    with ranks {"attn": r, "mlp": r}, as CPUDraftModel passes them."""
    import torch

    rng = np.random.Generator(np.random.PCG64(seed))
    shapes = {"q": (hidden, hidden, "attn"), "k": (hidden, kv_dim, "attn"), "v": (hidden, kv_dim, "attn"),
              "o": (hidden, hidden, "attn"), "gate": (hidden, inter, "mlp"), "up": (hidden, inter, "mlp"),
              "down": (inter, hidden, "mlp")}
    tensors: List = []
    dims: List[int] = []
    for _ in range(n_layers):
        tensors.append(torch.from_numpy((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)))
        tensors.append(torch.from_numpy((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)))
        for p in PROJ:
            K, N, kind = shapes[p]
            R = int(ranks[kind])
            v = torch.from_numpy(_words(rng, R, K))
            u = torch.from_numpy(_words(rng, N, R))
            tensors += [torch.from_numpy(_scales(rng, K)), ops.repack_signs_to_i2(v, K).contiguous(),
                        torch.from_numpy(_scales(rng, R)), ops.repack_signs_to_i2(u, R).contiguous(),
                        torch.from_numpy(_scales(rng, N))]
            dims += [K, R, R, N]
    return tensors, dims


def kv_caches(n_layers: int, kv_heads: int, max_seq: int, head_dim: int) -> List:
    import torch
    return [torch.zeros((kv_heads, max_seq, head_dim), dtype=torch.float32) for _ in range(2 * n_layers)]


def time_generate_token(ops, layers, dims, n_layers: int, hidden: int, vocab: int, kv_heads: int, head_dim: int,
                        start: int, max_seq: int, budget_s: float, seed: int = 1) -> Tuple[float, int]:
    """Seconds per token of ``generate_token`` (all layers, Q4_0 head,
    argmax) at positions start, start + 1, ... within a time budget; returns
    (seconds per token, tokens timed)."""
    import torch

    rng = np.random.Generator(np.random.PCG64(seed))
    emb = torch.from_numpy(rng.standard_normal((vocab, hidden)).astype(np.float32))
    norm = torch.from_numpy((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32))
    head = ops.quantize_lm_head_q4(torch.from_numpy(rng.standard_normal((vocab, hidden)).astype(np.float32)))
    kv = kv_caches(n_layers, kv_heads, max_seq, head_dim)
    scale = head_dim ** -0.5
    tok, pos = 1, start

    def step():
        nonlocal tok, pos
        tok = int(ops.generate_token(tok, emb, norm, layers, kv, dims, head, vocab, n_layers, hidden, kv_heads,
                                     (hidden // head_dim) // kv_heads, head_dim, max_seq, pos, scale, 1e-6))
        pos = start + (pos + 1 - start) % (max_seq - start)

    step()  # warm
    t0, n = time.perf_counter(), 0
    while True:
        step()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 10000:
            return el / n, n


def time_full_forward(ops, layers, dims, n_layers: int, hidden: int, vocab: int, kv_heads: int, head_dim: int,
                      position: int, max_seq: int, budget_s: float, seed: int = 1) -> Tuple[float, int]:
    """Seconds per call of ``full_forward`` (embedding, all layers, final
    norm; no lm_head) for one token at a fixed ``position``, within a time
    budget; returns (seconds per call, calls timed).  At position 0 the
    attention covers one position, so the call is the layers' i2 linears
    (patch:1320-1369) plus the RMSNorms, SiLU * up and residual adds."""
    import torch

    rng = np.random.Generator(np.random.PCG64(seed))
    emb = torch.from_numpy(rng.standard_normal((vocab, hidden)).astype(np.float32))
    norm = torch.from_numpy((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32))
    kv = kv_caches(n_layers, kv_heads, max_seq, head_dim)
    scale = head_dim ** -0.5

    def step():
        ops.full_forward(1, emb, norm, layers, kv, dims, n_layers, hidden, kv_heads,
                         (hidden // head_dim) // kv_heads, head_dim, max_seq, position, scale, 1e-6)

    step()  # warm
    t0, n = time.perf_counter(), 0
    while True:
        step()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 10000:
            return el / n, n


def time_full_forward_batch(ops, layers, dims, n_layers: int, hidden: int, vocab: int, kv_heads: int,
                            head_dim: int, n_tokens: int, start: int, max_seq: int, budget_s: float,
                            seed: int = 2) -> Tuple[float, int]:
    """Seconds per call of ``full_forward_batch`` on ``n_tokens`` tokens at
    positions start .. start + n_tokens - 1 (the reference's verify)."""
    import torch

    rng = np.random.Generator(np.random.PCG64(seed))
    emb = torch.from_numpy(rng.standard_normal((vocab, hidden)).astype(np.float32))
    norm = torch.from_numpy((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32))
    kv = kv_caches(n_layers, kv_heads, max_seq, head_dim)
    ids = torch.from_numpy(rng.integers(0, vocab, n_tokens).astype(np.int64))
    scale = head_dim ** -0.5

    def call():
        ops.full_forward_batch(ids, emb, norm, layers, kv, dims, n_layers, hidden, kv_heads,
                               (hidden // head_dim) // kv_heads, head_dim, max_seq, start, scale, 1e-6)

    call()
    t0, n = time.perf_counter(), 0
    while True:
        call()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 10000:
            return el / n, n


def cpu_facts() -> Dict:
    """CPU model and core counts of this host, from lscpu (and the thread
    share a GPU box gives one GPU's jobs)."""
    import os
    import subprocess

    out = {"model": None, "sockets": None, "cores_per_socket": None, "physical_cores": None,
           "logical_cpus": os.cpu_count()}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except Exception:  # noqa: BLE001
        return out
    kv = {}
    for line in txt.splitlines():
        if ":" in line:
            k, v = line.split(":", 1)
            kv[k.strip()] = v.strip()
    out["model"] = kv.get("Model name")
    try:
        out["sockets"] = int(kv.get("Socket(s)", "0"))
        out["cores_per_socket"] = int(kv.get("Core(s) per socket", "0"))
        out["physical_cores"] = out["sockets"] * out["cores_per_socket"]
    except ValueError:
        pass
    return out

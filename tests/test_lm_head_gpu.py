"""GPU Q4_0 lm_head (lbk_q4_0_quantize, lbk_lm_head_q4_argmax) against the
oracle (oracle/lm_head_q4_oracle.py, pinned to the reference's
quantize_lm_head_q4 bytes and generate_token tokens in test_oracle_q4.py).

Bar: the quantised planes bit-exact; logits within 1e-5 of max|logit| (fp32
sums of exact integer block dots in another order); the token the first
index whose oracle logit is the maximum, up to that tolerance.  With the
final RMSNorm fused, the hidden state differs from the float64 norm in its
last bits, which can move a Q8_0 value by one step: logits within 2e-3.
"""
import numpy as np
import pytest
import torch

from oracle import lm_head_q4_oracle as Q
from oracle import littlebit_oracle as O

pytestmark = pytest.mark.gpu


def _weights(seed, vocab, hidden):
    rng = np.random.Generator(np.random.PCG64(seed))
    w = (rng.standard_normal((vocab, hidden)) * 0.05).astype(np.float32)
    w[0, :32] = 0.0
    if vocab > 3:
        w[1, 5], w[1, 9] = 0.5, -0.5
        w[2, :32] = 1e-9
    return rng, w


def _head(gpu, w):
    from littlebit_amd.lm_head import Q4LMHead
    return Q4LMHead(torch.from_numpy(w).to(gpu))


@pytest.mark.parametrize("vocab,hidden", [(37, 96), (1000, 4096), (77, 32), (300, 5120), (64, 16384)])
def test_q4_quantizer_bit_exact(gpu, vocab, hidden):
    _, w = _weights(vocab + hidden, vocab, hidden)
    print(f"[q4_quantize] vocab={vocab} hidden={hidden}", flush=True)
    head = _head(gpu, w)
    torch.cuda.synchronize()
    qs, d = Q.quantize_q4_0(w)
    assert np.array_equal(head.qs.cpu().numpy(), qs.reshape(vocab, hidden // 2))
    assert np.array_equal(head.d.cpu().numpy().view(np.uint16), d)


@pytest.mark.parametrize("vocab,hidden", [(1000, 4096), (77, 32), (300, 5120), (513, 8192), (64, 16384),
                                          (32000, 4096)])
def test_q4_logits_and_token(gpu, vocab, hidden):
    rng, w = _weights(7 * vocab + hidden, vocab, hidden)
    x = rng.standard_normal(hidden).astype(np.float32)
    head = _head(gpu, w)
    logits = torch.empty(vocab, device=gpu)
    print(f"[q4_head] vocab={vocab} hidden={hidden}", flush=True)
    tok = head.argmax(torch.from_numpy(x).to(gpu), logits=logits)
    torch.cuda.synchronize()
    qs, d = Q.quantize_q4_0(w)
    ref, _ = Q.generate_token_head(x, qs, d)
    got = logits.cpu().numpy()
    err = O.rel_err(got, ref)
    print(f"[q4_head] rel_err={err:.2e}", flush=True)
    assert err <= 1e-5
    t = int(tok.item())
    scale = np.abs(ref).max()
    assert ref[t] >= ref.max() - 1e-5 * scale


def test_q4_first_maximum_wins(gpu):
    """Equal rows: the first of them is the token (patch:2307-2313)."""
    rng, w = _weights(3, 200, 256)
    x = rng.standard_normal(256).astype(np.float32)
    top = int(np.argmax(w @ x))
    w[150] = w[top] * 1.5
    w[40] = w[150]
    w[170] = w[150]
    head = _head(gpu, w)
    assert int(head.argmax(torch.from_numpy(x).to(gpu)).item()) == 40


def test_q4_fused_final_norm(gpu):
    from littlebit_amd.lm_head import Q4LMHead
    rng, w = _weights(9, 4000, 4096)
    x = (rng.standard_normal(4096) * 3).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    head = Q4LMHead(torch.from_numpy(w).to(gpu))
    logits = torch.empty(4000, device=gpu)
    tok = head.argmax(torch.from_numpy(x).to(gpu), torch.from_numpy(nw).to(gpu), 1e-5, logits=logits)
    torch.cuda.synchronize()
    xn = O.rms_norm(x, nw, 1e-5).astype(np.float32)
    qs, d = Q.quantize_q4_0(w)
    ref, _ = Q.generate_token_head(xn, qs, d)
    err = O.rel_err(logits.cpu().numpy(), ref)
    print(f"[q4_head_norm] rel_err={err:.2e}", flush=True)
    assert err <= 2e-3
    t = int(tok.item())
    assert ref[t] >= ref.max() - 2e-3 * np.abs(ref).max()


def test_q4_head_in_graph_replays(gpu):
    """Captured: each replay reads the token the previous one wrote (a
    feedback chain like the draft step's) and matches eager calls."""
    rng, w = _weights(21, 500, 128)
    E = rng.standard_normal((500, 128)).astype(np.float32)
    head = _head(gpu, w)
    emb = torch.from_numpy(E).to(gpu)
    tok = torch.zeros(1, dtype=torch.int64, device=gpu)
    s = torch.cuda.Stream(device=gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        head.argmax(emb.index_select(0, tok).view(-1), out=tok)  # warm
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        head.argmax(emb.index_select(0, tok).view(-1), out=tok)
    torch.cuda.synchronize()
    for start in (3, 77):
        tok.fill_(start)
        eager = [start]
        for _ in range(6):
            eager.append(int(head.argmax(emb[eager[-1]].contiguous()).item()))
        tok.fill_(start)
        seen = [start]
        for _ in range(6):
            g.replay()
            torch.cuda.synchronize()
            seen.append(int(tok.item()))
        assert seen == eager

"""The decoders at the full Llama-2-7B shape that bench.py's `decode` block
times (hidden 4096, 32 layers, 32 heads, MLP 11008, vocab 32000): one draft
token of the 0.1-BPW draft (ranks 205 / 298; the one-token step, attention
partials merged in the o projection) and one 8-token verify of the 1.0-BPW
target (draft + residual ranks 1843 / 2686 per projection: the M = 8 calls
of config 3), each after a 4-token prompt, against the float64 reference
decoder (tests/decoder_ref64.py, pinned to the oracle decoder) on the same
synthetic runtime state.  Bar: max|dh| / max|h| <= 1e-3 over every hidden
row of the step (cpu_draft_model.py:463-593, cpu_target_model.py:467-556).
"""
import pytest
import torch

from oracle import littlebit_oracle as O
from tests.decoder_ref64 import ref_hidden64

pytestmark = pytest.mark.gpu

TOL = 1e-3
PROMPT = [11, 2047, 31999, 5]


def _cfg():
    from littlebit_amd.decode import DecoderConfig
    from littlebit_amd.synthetic import LLAMA2_7B as C
    return DecoderConfig(hidden_size=C["hidden"], intermediate_size=C["intermediate"],
                         num_hidden_layers=C["layers"], num_attention_heads=C["heads"],
                         num_key_value_heads=C["kv_heads"], vocab_size=C["vocab"], rms_norm_eps=1e-6)


def _state(gpu, residual, seed):
    from littlebit_amd.synthetic import LLAMA2_7B as C, synthetic_runtime_state
    return synthetic_runtime_state(_cfg(), C["draft_rank"], C["residual_rank"] if residual else None, seed=seed,
                                   device=gpu, normalized=True)


def test_fullsize_draft_token(gpu):
    from littlebit_amd.decode import LittleBitDecoder
    cfg = _cfg()
    st = _state(gpu, False, 4242)
    dec = LittleBitDecoder(st, cfg, gpu, max_seq_len=64, residual=False)
    emb = st["model.embed_tokens.weight"]
    dec.forward_batch(PROMPT, emb)
    nxt = 20000
    print(f"[fullsize] draft: hidden {cfg.hidden_size}, {cfg.num_hidden_layers} layers, one token after "
          f"{len(PROMPT)}", flush=True)
    h = dec.forward_token(nxt, emb)
    torch.cuda.synchronize()
    ref = ref_hidden64(st, cfg, PROMPT + [nxt], residual=False, device=gpu)[-1:]
    err = O.rel_err(h.double().cpu().numpy(), ref.cpu().numpy())
    print(f"[fullsize] draft token rel_err={err:.3e}", flush=True)
    assert err <= TOL


def test_fullsize_target_verify_8(gpu):
    from littlebit_amd.decode import LittleBitDecoder
    cfg = _cfg()
    st = _state(gpu, True, 4343)
    dec = LittleBitDecoder(st, cfg, gpu, max_seq_len=64, residual=None)
    emb = st["model.embed_tokens.weight"]
    dec.forward_batch(PROMPT, emb)
    verify = [7, 123, 31000, 4096, 1, 17, 29999, 256]
    print(f"[fullsize] target: verify of {len(verify)} tokens after {len(PROMPT)}", flush=True)
    h = dec.forward_batch(verify, emb)
    torch.cuda.synchronize()
    ref = ref_hidden64(st, cfg, PROMPT + verify, residual=True, device=gpu)[len(PROMPT):]
    err = O.rel_err(h.double().cpu().numpy(), ref.cpu().numpy())
    print(f"[fullsize] target verify rel_err={err:.3e}", flush=True)
    assert err <= TOL

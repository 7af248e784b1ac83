"""The torch float64 reference decoder (tests/decoder_ref64.py) against the
numpy oracle decoder (test_decode_gpu.ref_hidden, built on
oracle.littlebit_oracle) on the CPU, for the small shapes the oracle
finishes in seconds: with and without residual branches, GQA with one and
two query heads per KV head, sequences of 1 and 7 tokens."""
import numpy as np
import pytest

from oracle import littlebit_oracle as O
from tests.decoder_ref64 import ref_hidden64, unpack_pm1
from test_decode_gpu import ref_hidden


def _cfg(hidden, heads, kvh, inter=96, layers=2):
    from littlebit_amd.decode import DecoderConfig
    return DecoderConfig(hidden_size=hidden, intermediate_size=inter, num_hidden_layers=layers,
                         num_attention_heads=heads, num_key_value_heads=kvh, vocab_size=200, rms_norm_eps=1e-6)


def test_unpack_matches_oracle():
    import torch
    rng = np.random.default_rng(5)
    w = rng.integers(-2**31, 2**31, size=(7, 3), dtype=np.int64).astype(np.int32)
    got = unpack_pm1(torch.from_numpy(w), 70).numpy()
    assert np.array_equal(got, O.unpack_signs(w, (7, 70)).astype(np.float64))


@pytest.mark.parametrize("hidden,heads,kvh,residual,ids", [
    (64, 4, 2, False, [5]), (64, 4, 2, True, [3, 17, 150, 9, 101, 42, 7]), (96, 3, 3, True, [1, 2, 3, 4])])
def test_torch_fp64_decoder_equals_oracle_decoder(hidden, heads, kvh, residual, ids):
    from littlebit_amd.synthetic import synthetic_runtime_state
    cfg = _cfg(hidden, heads, kvh)
    st = synthetic_runtime_state(cfg, {"attn": 12, "mlp": 20}, {"attn": 33, "mlp": 45} if residual else None,
                                 seed=hidden + len(ids), normalized=True)
    a = ref_hidden64(st, cfg, ids, residual).numpy()
    b = ref_hidden(st, cfg, ids, residual)
    assert a.shape == b.shape
    assert O.rel_err(a, b) <= 1e-12

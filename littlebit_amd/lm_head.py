"""Q4_0 lm_head with argmax: the GPU form of the reference's
``quantize_lm_head_q4`` + ``generate_token`` tail
(patches/littlebit_cpu_optimized.cpp:2225-2317), which its CPU draft model
uses whenever the C++ ops are present (cpu_draft_model.py:270-286, 485-563).

The weight is quantised once on the GPU to the reference's Q4_0 values (bit
for bit), held as a nibble plane [vocab, hidden/2] and an fp16-bit scale
plane [vocab, hidden/32]; each call quantises the final hidden state to
Q8_0, takes every row's Q4_0 x Q8_0 dot product and writes the first index of
the largest logit to a device int64 -- two launches, no host round trip, so
a captured draft step can feed the token straight back as its next input.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .ops import _check, _require_cuda


class Q4LMHead:
    """``weight`` [vocab, hidden] (any float dtype; quantised from its fp32
    values, as the reference quantises ``lm_head_weight.float()``), hidden a
    multiple of 32 and at most 16384."""

    def __init__(self, weight: torch.Tensor):
        _check(isinstance(weight, torch.Tensor) and weight.dim() == 2, "weight must be a 2-D tensor")
        _check(weight.is_cuda, "weight must be a GPU tensor (the HIP path has no CPU fallback)")
        vocab, hidden = (int(s) for s in weight.shape)
        _check(hidden % 32 == 0 and 32 <= hidden <= 16384, "hidden must be a multiple of 32 in [32, 16384]")
        dev = weight.device
        w = weight.detach().to(torch.float32).contiguous()
        self.vocab, self.hidden, self.device = vocab, hidden, dev
        self.qs = torch.empty((vocab, hidden // 2), dtype=torch.uint8, device=dev)
        self.d = torch.empty((vocab, hidden // 32), dtype=torch.int16, device=dev)  # fp16 bit patterns
        lib = _lib.load()
        stream = torch.cuda.current_stream(dev).cuda_stream
        _lib.check(lib.lbk_q4_0_quantize(w.data_ptr(), vocab, hidden, self.qs.data_ptr(), self.d.data_ptr(), stream),
                   "lbk_q4_0_quantize")
        nbytes = int(lib.lbk_lm_head_q4_workspace_bytes(vocab, hidden))
        self._ws = torch.empty(max(nbytes // 8, 1), dtype=torch.int64, device=dev)

    @property
    def nbytes(self) -> int:
        """HBM bytes one call reads from the weight planes."""
        return self.qs.numel() + 2 * self.d.numel()

    def argmax(self, x: torch.Tensor, norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6, *,
               out: Optional[torch.Tensor] = None, logits: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Token (int64 [1] on the device) for the final hidden state ``x``
        ([hidden] or [1, hidden], fp32): RMSNorm(x) * norm_weight first when
        ``norm_weight`` is given.  ``out`` receives the token (e.g. a captured
        graph's input slot); ``logits`` [vocab] fp32, when given, the logits."""
        _require_cuda(x, "x")
        _check(x.dtype == torch.float32 and x.numel() == self.hidden and x.device == self.device,
               "x must be float32 with hidden elements on the weight's device")
        if norm_weight is not None:
            _require_cuda(norm_weight, "norm_weight")
            _check(norm_weight.dtype == torch.float32 and norm_weight.numel() == self.hidden,
                   "norm_weight must be float32 with hidden elements")
        if out is None:
            out = torch.empty(1, dtype=torch.int64, device=self.device)
        _check(out.is_cuda and out.dtype == torch.int64 and out.numel() >= 1, "out must be a GPU int64 tensor")
        if logits is not None:
            _require_cuda(logits, "logits")
            _check(logits.dtype == torch.float32 and logits.numel() == self.vocab, "logits must be float32 [vocab]")
        lib = _lib.load()
        stream = torch.cuda.current_stream(self.device).cuda_stream
        rc = lib.lbk_lm_head_q4_argmax(
            self.qs.data_ptr(), self.d.data_ptr(), self.vocab, self.hidden, x.data_ptr(),
            None if norm_weight is None else norm_weight.data_ptr(), float(eps),
            None if logits is None else logits.data_ptr(), out.data_ptr(), self._ws.data_ptr(),
            self._ws.numel() * 8, stream)
        _lib.check(rc, "lbk_lm_head_q4_argmax")
        return out

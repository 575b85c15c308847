"""Token sampling on the device (reference src/llm/decoder.rs:878-1020).

``sample_logits`` applies the repetition penalty and draws one token from a
device logits vector without reading it back: greedy when the temperature is
not finite or <= 0 or top_k == 1, else top-k (ties to the lower index),
temperature softmax, nucleus cut at top_p and one draw.  The reference's draw
comes from an unseeded generator; here draw number ``counter`` of ``seed`` uses
u = ``sample_uniform(seed, counter)``, so a seed fixes the sequence.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import torch

from . import _lib
from .quantization import _on_gpu, _ptr, _stream, _target


def sample_uniform(seed: int, counter: int) -> float:
    """The uniform in [0, 1) of draw ``counter`` under ``seed``."""
    return float(_lib.lib().tb_sample_uniform(int(seed) & (2 ** 64 - 1),
                                               int(counter) & (2 ** 64 - 1)))


def sample_logits(logits: torch.Tensor, temperature: float = 0.7, top_k: int = 40,
                  top_p: float = 1.0, repetition_penalty: float = 1.0,
                  recent_tokens: Optional[Sequence[int]] = None, seed: int = 0,
                  counter: int = 0, return_u: bool = False):
    """One token from ``logits`` (vocab,) on the GPU; the caller's tensor is not
    modified (the penalty works on a copy)."""
    dev = _target(logits)
    lg = _on_gpu(logits.reshape(-1), torch.float32, dev)
    rec = list(recent_tokens or [])
    rt = None
    if repetition_penalty > 1.0 and rec:
        lg = lg.clone() if lg.data_ptr() == logits.data_ptr() else lg
        rt = torch.tensor(rec, dtype=torch.int64, device=dev)
    tok, u = C.c_int64(), C.c_float()
    _lib.call("tb_sample_logits", _ptr(lg), lg.numel(), float(temperature), int(top_k),
              float(top_p), float(repetition_penalty), _ptr(rt), 0 if rt is None else rt.numel(),
              int(seed) & (2 ** 64 - 1), int(counter) & (2 ** 64 - 1), C.byref(tok), C.byref(u),
              _stream(dev))
    return (int(tok.value), float(u.value)) if return_u else int(tok.value)

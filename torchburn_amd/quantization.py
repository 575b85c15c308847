"""Quantized linear ops on MI355X, with the reference's Python API.

Mirrors python/torchburn/quantization.py of the reference: the same function
names, argument order, defaults, weight layouts and output shapes, so callers
of ``torchburn.w4a32_grouped_linear`` / ``QuantizedLinear`` switch by import.
Compute runs in libtbhip.so (gfx950 HIP kernels) on the tensors' GPU; CPU
tensors are moved to the current GPU for the call and the result is returned
on the caller's device.  There is no CPU compute path.
"""
from __future__ import annotations

import gc
from typing import Any, List, Optional, Tuple

import torch
import torch.nn as nn

from . import _lib
from ._lib import UnsupportedOpError


def _gpu() -> torch.device:
    if not torch.cuda.is_available():
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} torchburn_amd needs a ROCm GPU (no CPU fallback)")
    return torch.device("cuda", torch.cuda.current_device())


def _on_gpu(t: Optional[torch.Tensor], dtype: torch.dtype, dev: torch.device):
    if t is None:
        return None
    if t.dtype != dtype:
        t = t.to(dtype)
    if t.device != dev:
        t = t.to(dev)
    return t.contiguous()


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _target(x: torch.Tensor) -> torch.device:
    return x.device if x.is_cuda else _gpu()


def _flattened_rows(shape: torch.Size) -> int:
    rows = 1
    for d in shape[:-1]:
        rows *= int(d)
    return rows


# --------------------------------------------------------------------------
# Quantizers (reference python/torchburn/quantization.py:30-118 and
# src/quantization/fused_ops.rs:554-589).  Formulas kept identical so that the
# packed bytes are the reference's.
# --------------------------------------------------------------------------

def quantize_weight_int4_grouped(
    weight: torch.Tensor,
    group_size: int = 64,
    chunk_size: int = 1024,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(N, K) float -> (packed uint8 (N, (K+1)//2), scales float32 (N, K//group_size)).

    Per group: s = max(amax / 7, 1e-8); q = clamp(round_half_even(w / s), -8, 7);
    byte j = (q[2j] + 8) | (q[2j+1] + 8) << 4  (reference quantization.py:53-118).
    Rows are processed in chunks of ``chunk_size`` to bound peak memory.
    """
    if weight.ndim != 2:
        raise ValueError(
            "Expected 2D weight matrix for quantize_weight_int4_grouped, got "
            f"{weight.ndim}D tensor of shape {tuple(weight.shape)}")
    n, k = weight.shape
    if k % group_size != 0:
        raise ValueError(
            f"Weight dimension K={k} must be divisible by group_size={group_size}. "
            f"Consider padding the weight tensor along dim 1 to a multiple of {group_size}.")
    ng = k // group_size
    dev = weight.device
    packed = torch.empty((n, (k + 1) // 2), dtype=torch.uint8, device=dev)
    scales = torch.empty((n, ng), dtype=torch.float32, device=dev)
    for r0 in range(0, n, chunk_size):
        r1 = min(r0 + chunk_size, n)
        wg = weight[r0:r1].detach().to(torch.float32).view(r1 - r0, ng, group_size)
        s = torch.clamp(wg.abs().amax(dim=-1, keepdim=True) / 7.0, min=1e-8)
        q = torch.clamp(torch.round(wg / s), -8, 7).to(torch.int8).view(r1 - r0, k)
        u = (q + 8).to(torch.uint8)
        packed[r0:r1] = (u[:, 0::2] & 0x0F) | ((u[:, 1::2] & 0x0F) << 4)
        scales[r0:r1] = s.view(r1 - r0, ng)
    return packed, scales


def quantize_weight_int8(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(N, K) float -> (int8 (N, K), float32 scales (N,)).

    s = amax / 127 (1 when amax == 0); q = clamp(round_half_away(w * (1/s)), -127, 127)
    (reference src/quantization/fused_ops.rs:554-589).
    """
    if w.ndim != 2:
        raise ValueError(f"Expected 2D weight, got {w.shape}")
    wf = w.detach().to(torch.float32)
    amax = wf.abs().amax(dim=1)
    s = torch.where(amax > 0, amax / 127.0, torch.ones_like(amax))
    v = wf * (1.0 / s)[:, None]
    q = torch.clamp(torch.sign(v) * torch.floor(v.abs() + 0.5), -127, 127).to(torch.int8)
    return q, s


# --------------------------------------------------------------------------
# Linear ops (reference quantization.py:193-269 -> src/ffi/quantization_ffi.rs)
# --------------------------------------------------------------------------

def w4a32_grouped_linear(
    x: torch.Tensor,
    w_packed: torch.Tensor,
    scales: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    group_size: int = 64,
) -> torch.Tensor:
    """out[..., N] = grouped-INT4 linear of x[..., K] (reference quantization.py:245-269)."""
    dev = _target(x)
    k = x.shape[-1]
    x2 = _on_gpu(x.reshape(-1, k), torch.float32, dev)
    m = x2.shape[0]
    w = _on_gpu(w_packed, torch.uint8, dev)
    s = _on_gpu(scales, torch.float32, dev)
    b = _on_gpu(bias, torch.float32, dev)
    if w.ndim != 2:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} w4a32_grouped_linear requires 2D packed weight matrix")
    n = w.shape[0]
    if w.shape[1] != (k + 1) // 2:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} w4a32_grouped_linear dimension mismatch: x K={k}, "
            f"w packed K={w.shape[1]} (expected {(k + 1) // 2})")
    ng = (k + group_size - 1) // group_size
    if s.ndim != 2 or tuple(s.shape) != (n, ng):
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} w4a32_grouped_linear scales mismatch: expected "
            f"[{n}, {ng}], got {list(s.shape)}")
    if b is not None and b.numel() != n:
        raise UnsupportedOpError(f"{_lib.UNSUPPORTED_MARKER} bias must have {n} elements")
    out = torch.empty((m, n), dtype=torch.float32, device=dev)
    _lib.call("tb_w4a32_grouped_linear", _ptr(x2), _ptr(w), _ptr(s), _ptr(b), _ptr(out),
              m, n, k, group_size, _stream(dev))
    return out.reshape(*x.shape[:-1], n).to(x.device)


def w4a32_grouped_linear_residual(
    x: torch.Tensor,
    w_packed: torch.Tensor,
    scales: torch.Tensor,
    residual: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    group_size: int = 64,
) -> torch.Tensor:
    """residual + w4a32_grouped_linear(x): the projection with its residual-add epilogue."""
    dev = _target(x)
    k = x.shape[-1]
    x2 = _on_gpu(x.reshape(-1, k), torch.float32, dev)
    m = x2.shape[0]
    w = _on_gpu(w_packed, torch.uint8, dev)
    s = _on_gpu(scales, torch.float32, dev)
    b = _on_gpu(bias, torch.float32, dev)
    n = w.shape[0]
    r = _on_gpu(residual.reshape(m, n), torch.float32, dev)
    out = torch.empty((m, n), dtype=torch.float32, device=dev)
    _lib.call("tb_w4a32_grouped_linear_residual", _ptr(x2), _ptr(w), _ptr(s), _ptr(b), _ptr(r),
              _ptr(out), m, n, k, group_size, _stream(dev))
    return out.reshape(*x.shape[:-1], n).to(x.device)


def fused_swiglu_mlp_w4a32(
    x: torch.Tensor,
    gate_w: torch.Tensor, gate_s: torch.Tensor, gate_b: Optional[torch.Tensor],
    up_w: torch.Tensor, up_s: torch.Tensor, up_b: Optional[torch.Tensor],
    down_w: torch.Tensor, down_s: torch.Tensor, down_b: Optional[torch.Tensor],
    group_size: int = 64,
    residual: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """down(silu(gate(x)) * up(x)) [+ residual] (reference fused_ops.rs:138-424)."""
    dev = _target(x)
    k = x.shape[-1]
    x2 = _on_gpu(x.reshape(-1, k), torch.float32, dev)
    m = x2.shape[0]
    gw, uw, dw = (_on_gpu(t, torch.uint8, dev) for t in (gate_w, up_w, down_w))
    gs, us, ds = (_on_gpu(t, torch.float32, dev) for t in (gate_s, up_s, down_s))
    gb, ub, db = (_on_gpu(t, torch.float32, dev) for t in (gate_b, up_b, down_b))
    inter, n_out = gw.shape[0], dw.shape[0]
    for name, w_, rows, kk in (("gate", gw, inter, k), ("up", uw, inter, k),
                               ("down", dw, n_out, inter)):
        if w_.ndim != 2 or w_.shape[0] != rows or w_.shape[1] != (kk + 1) // 2:
            raise UnsupportedOpError(
                f"{_lib.UNSUPPORTED_MARKER} fused_swiglu_mlp_w4a32 {name} weight shape "
                f"{list(w_.shape)} does not match ({rows}, {(kk + 1) // 2})")
    r = None if residual is None else _on_gpu(residual.reshape(m, n_out), torch.float32, dev)
    out = torch.empty((m, n_out), dtype=torch.float32, device=dev)
    _lib.call("tb_fused_swiglu_mlp_w4a32", _ptr(x2), _ptr(gw), _ptr(gs), _ptr(gb), _ptr(uw),
              _ptr(us), _ptr(ub), _ptr(dw), _ptr(ds), _ptr(db), _ptr(r), _ptr(out),
              m, k, inter, n_out, group_size, _stream(dev))
    return out.reshape(*x.shape[:-1], n_out).to(x.device)


def w8a32_linear(
    x: torch.Tensor,
    w: torch.Tensor,
    scales: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """out = (x @ w.T) * scales + bias for int8 w (reference quantization.py:193-216)."""
    dev = _target(x)
    k = x.shape[-1]
    x2 = _on_gpu(x.reshape(-1, k), torch.float32, dev)
    m = x2.shape[0]
    wt = _on_gpu(w, torch.int8, dev)
    s = _on_gpu(scales, torch.float32, dev).reshape(-1)
    b = _on_gpu(bias, torch.float32, dev)
    if wt.ndim != 2 or wt.shape[1] != k:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} w8a32_linear dimension mismatch: x K={k}, "
            f"w {list(wt.shape)}")
    n = wt.shape[0]
    out = torch.empty((m, n), dtype=torch.float32, device=dev)
    _lib.call("tb_w8a32_linear", _ptr(x2), _ptr(wt), _ptr(s), s.numel(), _ptr(b), _ptr(out),
              m, n, k, _stream(dev))
    return out.reshape(*x.shape[:-1], n).to(x.device)


def fused_swiglu_mlp_w8a32(
    x: torch.Tensor,
    gate_w: torch.Tensor, gate_s: torch.Tensor, gate_b: Optional[torch.Tensor],
    up_w: torch.Tensor, up_s: torch.Tensor, up_b: Optional[torch.Tensor],
    down_w: torch.Tensor, down_s: torch.Tensor, down_b: Optional[torch.Tensor],
    residual: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """INT8 down(silu(gate(x)) * up(x)) [+ residual] (reference fused_ops.rs:8-133)."""
    dev = _target(x)
    k = x.shape[-1]
    x2 = _on_gpu(x.reshape(-1, k), torch.float32, dev)
    m = x2.shape[0]
    gw, uw, dw = (_on_gpu(t, torch.int8, dev) for t in (gate_w, up_w, down_w))
    gs, us, ds = (_on_gpu(t, torch.float32, dev).reshape(-1) for t in (gate_s, up_s, down_s))
    gb, ub, db = (_on_gpu(t, torch.float32, dev) for t in (gate_b, up_b, down_b))
    inter, n_out = gw.shape[0], dw.shape[0]
    r = None if residual is None else _on_gpu(residual.reshape(m, n_out), torch.float32, dev)
    out = torch.empty((m, n_out), dtype=torch.float32, device=dev)
    _lib.call("tb_fused_swiglu_mlp_w8a32", _ptr(x2), _ptr(gw), _ptr(gs), _ptr(gb), _ptr(uw),
              _ptr(us), _ptr(ub), _ptr(dw), _ptr(ds), _ptr(db), _ptr(r), _ptr(out),
              m, k, inter, n_out, _stream(dev))
    return out.reshape(*x.shape[:-1], n_out).to(x.device)


def fused_swiglu_mlp(x: torch.Tensor, gate: Any, up: Any, down: Any) -> torch.Tensor:
    """Fused SwiGLU MLP over three QuantizedLinear modules (reference quantization.py:299-355)."""
    if gate.bits == 8:
        return fused_swiglu_mlp_w8a32(
            x, gate.qweight, gate.scales, gate.bias, up.qweight, up.scales, up.bias,
            down.qweight, down.scales, down.bias)
    if gate.bits == 4:
        return fused_swiglu_mlp_w4a32(
            x, gate.qweight, gate.scales, gate.bias, up.qweight, up.scales, up.bias,
            down.qweight, down.scales, down.bias, gate.group_size)
    raise ValueError(f"Unsupported bits={gate.bits}")


# --------------------------------------------------------------------------
# QuantizedLinear (reference quantization.py:756-869)
# --------------------------------------------------------------------------

class QuantizedLinear(nn.Module):
    """Drop-in replacement for nn.Linear running the gfx950 quantized GEMV/GEMM."""

    qweight: torch.Tensor
    scales: torch.Tensor
    bias: Optional[torch.Tensor]

    def __init__(self, in_features: int, out_features: int, bias: bool = False, bits: int = 8,
                 group_size: int = 64, backend: str = "gpu"):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.bits = bits
        self.group_size = group_size
        self.backend = backend
        if bits == 8:
            self.register_buffer("qweight", torch.zeros((out_features, in_features),
                                                        dtype=torch.int8))
            self.register_buffer("scales", torch.ones(out_features, dtype=torch.float32))
        elif bits == 4:
            self.register_buffer("qweight", torch.zeros((out_features, (in_features + 1) // 2),
                                                        dtype=torch.uint8))
            ng = (in_features + group_size - 1) // group_size
            self.register_buffer("scales", torch.ones((out_features, ng), dtype=torch.float32))
        else:
            raise ValueError(f"Supported quantization bits are 8 and 4, got {bits}")
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.float32))
        else:
            self.register_parameter("bias", None)

    @classmethod
    def from_float(cls, linear: nn.Linear, bits: int = 8, group_size: int = 64,
                   backend: str = "gpu") -> "QuantizedLinear":
        has_bias = linear.bias is not None
        ql = cls(linear.in_features, linear.out_features, bias=has_bias, bits=bits,
                 group_size=group_size, backend=backend)
        with torch.no_grad():
            if bits == 8:
                qw, sc = quantize_weight_int8(linear.weight)
            else:
                qw, sc = quantize_weight_int4_grouped(linear.weight, group_size=group_size)
            ql.qweight.copy_(qw)
            ql.scales.copy_(sc)
            if has_bias and linear.bias is not None:
                ql.bias.copy_(linear.bias.float())
        return ql

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.bits == 8:
            return w8a32_linear(x, self.qweight, self.scales, self.bias)
        return w4a32_grouped_linear(x, self.qweight, self.scales, self.bias,
                                    group_size=self.group_size)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, bits={self.bits}, "
                f"group_size={self.group_size}, backend={self.backend}")


def quantize_model(model: nn.Module, bits: int = 8, group_size: int = 64,
                   exclude_modules: Optional[List[str]] = None,
                   backend: str = "gpu") -> nn.Module:
    """Replace every nn.Linear (except ``exclude_modules``, default ["lm_head"])."""
    exclude = set(exclude_modules if exclude_modules is not None else ["lm_head"])

    def _replace(module: nn.Module, prefix: str = ""):
        for name, child in list(module.named_children()):
            full = f"{prefix}.{name}" if prefix else name
            if isinstance(child, nn.Linear):
                if name in exclude or full in exclude:
                    continue
                setattr(module, name, QuantizedLinear.from_float(
                    child, bits=bits, group_size=group_size, backend=backend))
                del child
            else:
                _replace(child, full)

    _replace(model)
    gc.collect()
    return model

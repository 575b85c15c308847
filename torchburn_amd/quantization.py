"""Quantized linear ops on MI355X, with the reference's Python API.

Mirrors python/torchburn/quantization.py of the reference: the same function
names, argument order, defaults, weight layouts and output shapes, so callers
of ``torchburn.w4a32_grouped_linear`` / ``QuantizedLinear`` switch by import.
Compute runs in libtbhip.so (gfx950 HIP kernels) on the tensors' GPU; CPU
tensors are moved to the current GPU for the call and the result is returned
on the caller's device.  There is no CPU compute path.
"""
from __future__ import annotations

import ctypes as C
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
    Runs on the GPU (tb_quantize_weight_int4_grouped), ``chunk_size`` rows of a
    host tensor at a time; the result is on the weight's device.  Any group size
    that divides K, as the reference takes (the GEMVs read even group sizes).
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
    if k % 2 != 0:
        # the reference's low | high pairs (K + 1) // 2 low nibbles with
        # (K - 1) // 2 high ones, and torch raises on the mismatch
        raise RuntimeError(
            f"quantize_weight_int4_grouped: K={k} is odd: {(k + 1) // 2} low nibbles against "
            f"{(k - 1) // 2} high ones")
    dev = _target(weight)
    packed = torch.empty((n, (k + 1) // 2), dtype=torch.uint8, device=dev)
    scales = torch.empty((n, k // group_size), dtype=torch.float32, device=dev)
    step = n if weight.is_cuda else max(int(chunk_size), 1)
    for r0 in range(0, n, step):
        r1 = min(r0 + step, n)
        wc = _on_gpu(weight[r0:r1].detach(), torch.float32, dev)
        _lib.call("tb_quantize_weight_int4_grouped", _ptr(wc), _ptr(packed[r0:r1]),
                  _ptr(scales[r0:r1]), r1 - r0, k, group_size, _stream(dev))
    return packed.to(weight.device), scales.to(weight.device)


def quantize_weight_int4(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(N, K) float -> (packed uint8 (N, (K+1)//2), per-channel float32 scales (N,))
    on the GPU (tb_quantize_weight_int4): s = amax / 7 (1 when amax <= 1e-8),
    q = clamp(round_half_away(w * (1/s)), -8, 7) + 8, two per byte (reference
    python/torchburn/quantization.py:44-50 -> src/quantization/fused_ops.rs:592-639).
    The result is on w's device."""
    if w.ndim != 2:
        raise ValueError(f"Expected 2D weight, got {w.shape}")
    n, k = w.shape
    dev = _target(w)
    wc = _on_gpu(w.detach(), torch.float32, dev)
    q = torch.empty((n, (k + 1) // 2), dtype=torch.uint8, device=dev)
    s = torch.empty(n, dtype=torch.float32, device=dev)
    _lib.call("tb_quantize_weight_int4", _ptr(wc), _ptr(q), _ptr(s), n, k, _stream(dev))
    return q.to(w.device), s.to(w.device)


def pack_rows_w4a32_group64_v1_to_v2(w_packed: torch.Tensor, scales: torch.Tensor,
                                     k: int) -> torch.Tensor:
    """v1 nibbles (N, K/2) + f32 scales (N, K/64) -> v2 blocks (N, (K/64) * 34) uint8:
    per group 32 nibble bytes then the scale as little-endian binary16, rounded to
    nearest even (reference src/quantization/packed_v2.rs:114-143, 66-105)."""
    if k % 64 != 0:
        raise ValueError(f"K={k} must be divisible by 64 for the v2 layout")
    dev = _target(w_packed)
    w = _on_gpu(w_packed, torch.uint8, dev)
    s = _on_gpu(scales, torch.float32, dev)
    n = w.shape[0]
    if tuple(w.shape) != (n, k // 2) or s.numel() != n * (k // 64):
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} pack_rows_w4a32_group64_v1_to_v2: expected packed "
            f"({n}, {k // 2}) and {n * (k // 64)} scales, got {list(w.shape)} / {s.numel()}")
    out = torch.empty((n, (k // 64) * 34), dtype=torch.uint8, device=dev)
    _lib.call("tb_pack_rows_w4a32_group64_v1_to_v2", _ptr(w), _ptr(s), _ptr(out), n, k,
              _stream(dev))
    return out.to(w_packed.device)


def quantize_weight_int4_grouped_v2(
    weight: torch.Tensor,
    group_size: int = 64,
    chunk_size: int = 1024,
) -> torch.Tensor:
    """(N, K) float -> v2 blocks (N, (K/64) * 34) uint8 (reference
    python/torchburn/quantization.py:121-152): the v1 quantizer, then each group's
    nibbles and binary16 scale packed into one 34-byte block."""
    if weight.ndim != 2:
        raise ValueError(
            f"Expected 2D weight matrix for quantize_weight_int4_grouped_v2, got {weight.ndim}D")
    n, k = weight.shape
    if k % group_size != 0:
        raise ValueError(f"K={k} must be divisible by group_size={group_size}")
    if group_size != 64:
        raise ValueError(f"the v2 layout is defined for group_size=64, got {group_size}")
    packed, scales = quantize_weight_int4_grouped(weight, group_size, chunk_size)
    return pack_rows_w4a32_group64_v1_to_v2(packed, scales, k).to(weight.device)


def dequantize_int4_grouped_v2(blocked: torch.Tensor, group_size: int = 64) -> torch.Tensor:
    """Inverse of quantize_weight_int4_grouped_v2: f32 (N, K) with (nib - 8) * f16 scale
    (reference python/torchburn/quantization.py:155-169)."""
    if group_size != 64:
        raise ValueError(f"the v2 layout is defined for group_size=64, got {group_size}")
    dev = _target(blocked)
    b = _on_gpu(blocked, torch.uint8, dev)
    n, cols = b.shape
    if cols % 34 != 0:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} v2 rows must be whole 34-byte blocks, got {cols} bytes")
    k = (cols // 34) * 64
    out = torch.empty((n, k), dtype=torch.float32, device=dev)
    _lib.call("tb_dequantize_int4_grouped_v2", _ptr(b), _ptr(out), n, k, _stream(dev))
    return out.to(blocked.device)


def release_stream_workspace(stream=None) -> None:
    """Frees the library's scratch for `stream` (default: the current torch
    stream) on the current device: for streams created per request.  Waits for
    the device; graphs captured on that stream must not be replayed afterwards.
    No reference counterpart (the reference allocates per call)."""
    s = stream if stream is not None else torch.cuda.current_stream()
    _lib.check(_lib.lib().tb_release_stream_workspace(C.c_void_p(s.cuda_stream)))


def set_vnni_semantics(enabled: bool) -> bool:
    """Selects the reference's AVX-512 VNNI-tier arithmetic for group-64 INT4
    projections: activations quantized per row to bytes (s_x = max|x| / 127,
    round-half-even) before the contraction (src/quantization/gemv.rs:1353-1473).
    Off by default (the exact W4A32 result of the other tiers).  Returns the
    previous setting."""
    return bool(_lib.lib().tb_set_vnni_semantics(1 if enabled else 0))


def quantize_weight_int8(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(N, K) float -> (int8 (N, K), float32 scales (N,)) on the GPU
    (tb_quantize_weight_int8): s = amax / 127 (1 when amax <= 1e-8);
    q = clamp(round_half_away(w * (1/s)), -127, 127) (reference
    src/quantization/fused_ops.rs:554-589).  The result is on w's device."""
    if w.ndim != 2:
        raise ValueError(f"Expected 2D weight, got {w.shape}")
    n, k = w.shape
    dev = _target(w)
    wc = _on_gpu(w.detach(), torch.float32, dev)
    q = torch.empty((n, k), dtype=torch.int8, device=dev)
    s = torch.empty(n, dtype=torch.float32, device=dev)
    _lib.call("tb_quantize_weight_int8", _ptr(wc), _ptr(q), _ptr(s), n, k, _stream(dev))
    return q.to(w.device), s.to(w.device)


def unpack_rows_w4a32_group64_v2_to_v1(blocked: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """v2 blocks (N, (K/64) * 34) -> (v1 nibbles (N, K/2), f32 scales (N, K/64)): the
    reference loader's cache migration (python/torchburn/llm/loader.py:540-561),
    on the device.  The result is on the blocks' device."""
    dev = _target(blocked)
    b = _on_gpu(blocked, torch.uint8, dev)
    n, cols = b.shape
    if cols % 34 != 0:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} v2 rows must be whole 34-byte blocks, got {cols} bytes")
    k = (cols // 34) * 64
    w = torch.empty((n, k // 2), dtype=torch.uint8, device=dev)
    s = torch.empty((n, k // 64), dtype=torch.float32, device=dev)
    _lib.call("tb_unpack_rows_w4a32_group64_v2_to_v1", _ptr(b), _ptr(w), _ptr(s), n, k,
              _stream(dev))
    return w.to(blocked.device), s.to(blocked.device)


# --------------------------------------------------------------------------
# Linear ops (reference quantization.py:193-269 -> src/ffi/quantization_ffi.rs)
# --------------------------------------------------------------------------

def w4a32_linear(
    x: torch.Tensor,
    w_packed: torch.Tensor,
    scales: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Per-channel INT4 linear: out[..., N] = (x @ unpack(w).T) * scales + bias
    (reference quantization.py:219-243 -> gemv.rs:1066-1182); scales of N
    elements or one per-tensor scalar."""
    if x.dim() < 1:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} w4a32_linear requires x with at least 1 dimension")
    dev = _target(x)
    k = x.shape[-1]
    x2 = _on_gpu(x.reshape(-1, k), torch.float32, dev)
    m = x2.shape[0]
    w = _on_gpu(w_packed, torch.uint8, dev)
    s = _on_gpu(scales, torch.float32, dev).reshape(-1)
    b = _on_gpu(bias, torch.float32, dev)
    if w.ndim != 2:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} w4a32_linear requires 2D packed weight matrix")
    n = w.shape[0]
    if w.shape[1] != (k + 1) // 2:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} w4a32_linear dimension mismatch: x K={k}, "
            f"w packed K={w.shape[1]} (expected {(k + 1) // 2})")
    if s.numel() not in (1, n):
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} w4a32_linear scales must have 1 or {n} elements, "
            f"got {s.numel()}")
    if b is not None and b.numel() != n:
        raise UnsupportedOpError(f"{_lib.UNSUPPORTED_MARKER} bias must have {n} elements")
    out = torch.empty((m, n), dtype=torch.float32, device=dev)
    _lib.call("tb_w4a32_linear", _ptr(x2), _ptr(w), _ptr(s), s.numel(), _ptr(b), _ptr(out),
              m, n, k, _stream(dev))
    return out.reshape(*x.shape[:-1], n).to(x.device)


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


def w4a32_grouped_linear_v2(
    x: torch.Tensor,
    blocked: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    group_size: int = 64,
) -> torch.Tensor:
    """out[..., N] = x[..., K] @ dequant(blocked)^T + bias over v2 blocks
    (reference quantization.py:172-190 -> packed_v2.rs:489-553)."""
    if x.dim() < 1:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} w4a32_grouped_linear_v2 requires x with at least 1 dimension")
    dev = _target(x)
    k = x.shape[-1]
    x2 = _on_gpu(x.reshape(-1, k), torch.float32, dev)
    m = x2.shape[0]
    w = _on_gpu(blocked, torch.uint8, dev)
    b = _on_gpu(bias, torch.float32, dev)
    if w.ndim != 2:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} w4a32_grouped_linear_v2 requires 2D blocked weight matrix")
    n = w.shape[0]
    expected = (k // group_size) * 34
    if w.shape[1] != expected:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} w4a32_grouped_linear_v2 dimension mismatch: K={k} "
            f"group={group_size} needs {expected} blocked bytes per row, got {w.shape[1]}")
    if b is not None and b.numel() != n:
        raise UnsupportedOpError(f"{_lib.UNSUPPORTED_MARKER} bias must have {n} elements")
    out = torch.empty((m, n), dtype=torch.float32, device=dev)
    _lib.call("tb_w4a32_grouped_linear_v2", _ptr(x2), _ptr(w), _ptr(b), _ptr(out), m, n, k,
              group_size, _stream(dev))
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
    op = "fused_swiglu_mlp_w4a32"
    _check_w4(op, "gate", gw, gs, gb, inter, k, group_size)
    _check_w4(op, "up", uw, us, ub, inter, k, group_size)
    _check_w4(op, "down", dw, ds, db, n_out, inter, group_size)
    r = None if residual is None else _on_gpu(residual.reshape(m, n_out), torch.float32, dev)
    out = torch.empty((m, n_out), dtype=torch.float32, device=dev)
    _lib.call("tb_fused_swiglu_mlp_w4a32", _ptr(x2), _ptr(gw), _ptr(gs), _ptr(gb), _ptr(uw),
              _ptr(us), _ptr(ub), _ptr(dw), _ptr(ds), _ptr(db), _ptr(r), _ptr(out),
              m, k, inter, n_out, group_size, _stream(dev))
    return out.reshape(*x.shape[:-1], n_out).to(x.device)


def fused_swiglu_mlp_batched_w4a32(
    x: torch.Tensor,
    gate_w: torch.Tensor, gate_s: torch.Tensor, gate_b: Optional[torch.Tensor],
    up_w: torch.Tensor, up_s: torch.Tensor, up_b: Optional[torch.Tensor],
    down_w: torch.Tensor, down_s: torch.Tensor, down_b: Optional[torch.Tensor],
    group_size: int = 64,
) -> torch.Tensor:
    """Prefill SwiGLU MLP over x (batch, T, K) -> (batch, T, N_down)
    (reference quantization_ffi.rs:511-570 -> fused_ops.rs:1267-1319: gate GEMM,
    up GEMM, silu(g) * u, down GEMM; one row delegates to the per-token path).
    Both cases go through tb_fused_swiglu_mlp_w4a32, which runs rows >= 5 as the
    FP32-MFMA GEMM pair and fewer as GEMV passes."""
    if x.dim() < 1:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} fused_swiglu_mlp_batched_w4a32: x needs >= 1 dim")
    return fused_swiglu_mlp_w4a32(x, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s,
                                  down_b, group_size)


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
    _check_w8("w8a32_linear", "w", wt, s, b, n, k)
    out = torch.empty((m, n), dtype=torch.float32, device=dev)
    _lib.call("tb_w8a32_linear", _ptr(x2), _ptr(wt), _ptr(s), s.numel(), _ptr(b), _ptr(out),
              m, n, k, _stream(dev))
    return out.reshape(*x.shape[:-1], n).to(x.device)


def _check_w4(op: str, name: str, w: torch.Tensor, s: torch.Tensor, b: Optional[torch.Tensor],
              n: int, k: int, gs: int) -> None:
    """Grouped INT4 projection operands: packed w (n, ceil(k/2)), scales of
    n * ceil(k/gs) elements, bias of n elements or None (the reference's checks,
    src/quantization/packed_v2.rs:565-596)."""
    if w.ndim != 2 or tuple(w.shape) != (n, (k + 1) // 2):
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} {op} {name} weight shape {list(w.shape)} does not "
            f"match ({n}, {(k + 1) // 2})")
    ng = (k + gs - 1) // gs
    if s.numel() != n * ng:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} {op} {name} scales must be [{n}, {ng}], got "
            f"{list(s.shape)}")
    if b is not None and b.numel() != n:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} {op} {name} bias must have {n} elements, got {b.numel()}")


def _check_w8(op: str, name: str, w: torch.Tensor, s: torch.Tensor, b: Optional[torch.Tensor],
              n: int, k: int) -> None:
    """INT8 projection operands: w (n, k); 1 (per-tensor) or n (per-row) scales;
    bias of n elements or None (the reference's gemv_w8a32 s_len rule,
    src/quantization/fused_ops.rs:80-97)."""
    if w.ndim != 2 or tuple(w.shape) != (n, k):
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} {op} {name} weight shape {list(w.shape)} does not "
            f"match ({n}, {k})")
    if s.numel() not in (1, n):
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} {op} {name} scales must have 1 or {n} elements, "
            f"got {s.numel()}")
    if b is not None and b.numel() != n:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} {op} {name} bias must have {n} elements, got {b.numel()}")


def fused_swiglu_mlp_w8a32(
    x: torch.Tensor,
    gate_w: torch.Tensor, gate_s: torch.Tensor, gate_b: Optional[torch.Tensor],
    up_w: torch.Tensor, up_s: torch.Tensor, up_b: Optional[torch.Tensor],
    down_w: torch.Tensor, down_s: torch.Tensor, down_b: Optional[torch.Tensor],
    residual: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """INT8 down(silu(gate(x)) * up(x)) [+ residual] (reference fused_ops.rs:8-133).
    Each projection's scales are per row or one per-tensor scalar; biases are
    optional."""
    dev = _target(x)
    k = x.shape[-1]
    x2 = _on_gpu(x.reshape(-1, k), torch.float32, dev)
    m = x2.shape[0]
    gw, uw, dw = (_on_gpu(t, torch.int8, dev) for t in (gate_w, up_w, down_w))
    gs, us, ds = (_on_gpu(t, torch.float32, dev).reshape(-1) for t in (gate_s, up_s, down_s))
    gb, ub, db = (_on_gpu(t, torch.float32, dev) for t in (gate_b, up_b, down_b))
    inter, n_out = gw.shape[0], dw.shape[0]
    op = "fused_swiglu_mlp_w8a32"
    _check_w8(op, "gate", gw, gs, gb, inter, k)
    _check_w8(op, "up", uw, us, ub, inter, k)
    _check_w8(op, "down", dw, ds, db, n_out, inter)
    r = None if residual is None else _on_gpu(residual.reshape(m, n_out), torch.float32, dev)
    out = torch.empty((m, n_out), dtype=torch.float32, device=dev)
    _lib.call("tb_fused_swiglu_mlp_w8a32", _ptr(x2), _ptr(gw), _ptr(gs), gs.numel(), _ptr(gb),
              _ptr(uw), _ptr(us), us.numel(), _ptr(ub), _ptr(dw), _ptr(ds), ds.numel(), _ptr(db),
              _ptr(r), _ptr(out), m, k, inter, n_out, _stream(dev))
    return out.reshape(*x.shape[:-1], n_out).to(x.device)


def fused_swiglu_mlp_batched(x: torch.Tensor, gate: Any, up: Any, down: Any) -> torch.Tensor:
    """Prefill SwiGLU MLP over three QuantizedLinear modules (reference
    quantization.py:358-405, called at python/torchburn/llm/model.py:359): INT4
    runs fused_swiglu_mlp_batched_w4a32 (all T rows as one FP32-MFMA GEMM pair
    from 5 rows), INT8 the per-token fused_swiglu_mlp."""
    if gate.bits != 4:
        return fused_swiglu_mlp(x, gate, up, down)
    return fused_swiglu_mlp_batched_w4a32(
        x, gate.qweight, gate.scales, gate.bias, up.qweight, up.scales, up.bias, down.qweight,
        down.scales, down.bias, gate.group_size)


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
# Per-layer decode steps (reference quantization.py:408-572; native
# fused_ops.rs:718-1062, fused_transformer.rs:16-376)
# --------------------------------------------------------------------------

def _cache_on_gpu(c: torch.Tensor, dev: torch.device, name: str, num_kv_heads: int,
                  head_dim: int):
    """The cache as a contiguous f32 device tensor (the caller's own tensor when
    it already is one) and its max_seq (the length of dim -2: [.., Hkv, max, hd]).
    The kernels write k / v at `offset` of every KV head, so the shape is checked
    against num_kv_heads and head_dim here (the reference's slices are
    bounds-checked, fused_ops.rs:981-994)."""
    if c.ndim < 3 or int(c.shape[-3]) != num_kv_heads or int(c.shape[-1]) != head_dim:
        raise UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} {name} must be [..., num_kv_heads={num_kv_heads}, "
            f"max_seq, head_dim={head_dim}], got {list(c.shape)}")
    g = c if (c.device == dev and c.dtype == torch.float32 and c.is_contiguous()) else \
        c.detach().to(device=dev, dtype=torch.float32).contiguous()
    return g, int(c.shape[-2])


def _write_back(dst: torch.Tensor, src: torch.Tensor) -> None:
    """In-place semantics of the reference (its caches / x are mutated): copy the
    GPU result into the caller's tensor when it is not that tensor."""
    if src.data_ptr() != dst.data_ptr():
        with torch.no_grad():
            dst.copy_(src.reshape(dst.shape))


def _attention_step(bits: int, x, qkv_w, qkv_s, qkv_b, o_w, o_s, o_b, k_cache, v_cache, cos, sin,
                    offset: int, num_heads: int, num_kv_heads: int, head_dim: int,
                    group_size: int) -> torch.Tensor:
    name = f"fused_attention_step_w{bits}a32"
    if x.ndim < 1:
        raise UnsupportedOpError(f"{_lib.UNSUPPORTED_MARKER} {name} requires x with at least 1 dim")
    dev = _target(x)
    h = x.shape[-1]
    x1 = _on_gpu(x.reshape(-1, h)[0], torch.float32, dev)   # the reference reads the first row
    wdt = torch.uint8 if bits == 4 else torch.int8
    qw, ow = _on_gpu(qkv_w, wdt, dev), _on_gpu(o_w, wdt, dev)
    qs, os_ = _on_gpu(qkv_s, torch.float32, dev), _on_gpu(o_s, torch.float32, dev)
    qb, ob = _on_gpu(qkv_b, torch.float32, dev), _on_gpu(o_b, torch.float32, dev)
    kc, max_seq = _cache_on_gpu(k_cache, dev, "k_cache", num_kv_heads, head_dim)
    vc, _ = _cache_on_gpu(v_cache, dev, "v_cache", num_kv_heads, head_dim)
    if tuple(vc.shape[-3:]) != tuple(kc.shape[-3:]):
        raise UnsupportedOpError(f"{_lib.UNSUPPORTED_MARKER} {name}: k / v caches differ in shape")
    cs = _on_gpu(cos.reshape(-1), torch.float32, dev)
    sn = _on_gpu(sin.reshape(-1), torch.float32, dev)
    nq = (num_heads + 2 * num_kv_heads) * head_dim
    qd = num_heads * head_dim
    if bits == 4:
        _check_w4(name, "qkv", qw, qs, qb, nq, h, group_size)
        _check_w4(name, "o", ow, os_, ob, h, qd, group_size)
    else:
        _check_w8(name, "qkv", qw, qs.reshape(-1), qb, nq, h)
        _check_w8(name, "o", ow, os_.reshape(-1), ob, h, qd)
    if cs.numel() < head_dim or sn.numel() < head_dim:
        raise UnsupportedOpError(f"{_lib.UNSUPPORTED_MARKER} {name}: cos / sin need head_dim values")
    out = torch.empty(h, dtype=torch.float32, device=dev)
    if bits == 4:
        _lib.call("tb_fused_attention_step_w4a32", _ptr(x1), _ptr(qw), _ptr(qs), _ptr(qb),
                  _ptr(ow), _ptr(os_), _ptr(ob), _ptr(kc), _ptr(vc), _ptr(cs), _ptr(sn),
                  _ptr(out), h, offset, max_seq, num_heads, num_kv_heads, head_dim, group_size,
                  _stream(dev))
    else:
        qs, os_ = qs.reshape(-1), os_.reshape(-1)
        _lib.call("tb_fused_attention_step_w8a32", _ptr(x1), _ptr(qw), _ptr(qs), qs.numel(),
                  _ptr(qb), _ptr(ow), _ptr(os_), os_.numel(), _ptr(ob), _ptr(kc), _ptr(vc),
                  _ptr(cs), _ptr(sn), _ptr(out), h, offset, max_seq, num_heads, num_kv_heads,
                  head_dim, _stream(dev))
    _write_back(k_cache, kc)
    _write_back(v_cache, vc)
    return out.reshape(1, h).to(x.device)


def fused_attention_step_w4a32(x, qkv_w, qkv_s, qkv_b, o_w, o_s, o_b, k_cache, v_cache, cos,
                               sin, offset: int, num_heads: int, num_kv_heads: int,
                               head_dim: int, group_size: int) -> torch.Tensor:
    """One attention decode step on INT4 projections (reference
    fused_ops.rs:891-1062): QKV + bias, RoPE with this position's cos / sin row,
    k / v written into the caches at `offset` (in place), GQA attention over
    0..offset, O projection + bias.  Returns [1, hidden]."""
    return _attention_step(4, x, qkv_w, qkv_s, qkv_b, o_w, o_s, o_b, k_cache, v_cache, cos, sin,
                           offset, num_heads, num_kv_heads, head_dim, group_size)


def fused_attention_step_w8a32(x, qkv_w, qkv_s, qkv_b, o_w, o_s, o_b, k_cache, v_cache, cos,
                               sin, offset: int, num_heads: int, num_kv_heads: int,
                               head_dim: int) -> torch.Tensor:
    """fused_attention_step_w4a32 with INT8 per-channel projections (reference
    fused_ops.rs:718-888)."""
    return _attention_step(8, x, qkv_w, qkv_s, qkv_b, o_w, o_s, o_b, k_cache, v_cache, cos, sin,
                           offset, num_heads, num_kv_heads, head_dim, 32)


def fused_transformer_layer_step_w4a32(x, input_norm_w, qkv_w, qkv_s, qkv_b, o_w, o_s, o_b,
                                       post_norm_w, gate_w, gate_s, gate_b, up_w, up_s, up_b,
                                       down_w, down_s, down_b, k_cache, v_cache, cos, sin,
                                       offset: int, num_heads: int, num_kv_heads: int,
                                       head_dim: int, group_size: int, eps: float = 1e-6) -> None:
    """One decoder layer in place on x [.., hidden] (reference
    fused_transformer.rs:16-376): x += attention(RMSNorm(x)); x += MLP(RMSNorm(x))."""
    name = "fused_transformer_layer_step_w4a32"
    if x.ndim < 1:
        raise UnsupportedOpError(f"{_lib.UNSUPPORTED_MARKER} {name} requires x with at least 1 dim")
    dev = _target(x)
    h = x.shape[-1]
    xg = x if (x.device == dev and x.dtype == torch.float32 and x.is_contiguous()) else \
        x.detach().to(device=dev, dtype=torch.float32).contiguous()
    g = lambda t, dt=torch.float32: _on_gpu(t, dt, dev)
    qw, ow, gw, uw, dw = (g(t, torch.uint8) for t in (qkv_w, o_w, gate_w, up_w, down_w))
    qs, os_, gs, us, ds = (g(t) for t in (qkv_s, o_s, gate_s, up_s, down_s))
    qb, ob, gb, ub, db = (g(t) for t in (qkv_b, o_b, gate_b, up_b, down_b))
    inw, pnw = g(input_norm_w), g(post_norm_w)
    kc, max_seq = _cache_on_gpu(k_cache, dev, "k_cache", num_kv_heads, head_dim)
    vc, _ = _cache_on_gpu(v_cache, dev, "v_cache", num_kv_heads, head_dim)
    if tuple(vc.shape[-3:]) != tuple(kc.shape[-3:]):
        raise UnsupportedOpError(f"{_lib.UNSUPPORTED_MARKER} {name}: k / v caches differ in shape")
    cs, sn = g(cos.reshape(-1)), g(sin.reshape(-1))
    if cs.numel() < head_dim or sn.numel() < head_dim:
        raise UnsupportedOpError(f"{_lib.UNSUPPORTED_MARKER} {name}: cos / sin need head_dim values")
    inter = gw.shape[0]
    nq, qd = (num_heads + 2 * num_kv_heads) * head_dim, num_heads * head_dim
    _check_w4(name, "qkv", qw, qs, qb, nq, h, group_size)
    _check_w4(name, "o", ow, os_, ob, h, qd, group_size)
    _check_w4(name, "gate", gw, gs, gb, inter, h, group_size)
    _check_w4(name, "up", uw, us, ub, inter, h, group_size)
    _check_w4(name, "down", dw, ds, db, h, inter, group_size)
    if inw.numel() != h or pnw.numel() != h:
        raise UnsupportedOpError(f"{_lib.UNSUPPORTED_MARKER} {name}: norm weights need {h} values")
    _lib.call("tb_fused_transformer_layer_step_w4a32", _ptr(xg), _ptr(inw), _ptr(qw), _ptr(qs),
              _ptr(qb), _ptr(ow), _ptr(os_), _ptr(ob), _ptr(pnw), _ptr(gw), _ptr(gs), _ptr(gb),
              _ptr(uw), _ptr(us), _ptr(ub), _ptr(dw), _ptr(ds), _ptr(db), _ptr(kc), _ptr(vc),
              _ptr(cs), _ptr(sn), h, inter, offset, max_seq, num_heads, num_kv_heads, head_dim,
              group_size, float(eps), _stream(dev))
    _write_back(k_cache, kc)
    _write_back(v_cache, vc)
    _write_back(x, xg)


def fused_attention_step(x: torch.Tensor, qkv: Any, o_proj: Any, k_cache: torch.Tensor,
                         v_cache: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, offset: int,
                         num_heads: int, num_kv_heads: int, head_dim: int) -> torch.Tensor:
    """Attention decode step over QuantizedLinear modules (reference quantization.py:408-485);
    returns x's shape."""
    if qkv.bits == 8:
        out = fused_attention_step_w8a32(x, qkv.qweight, qkv.scales, qkv.bias, o_proj.qweight,
                                         o_proj.scales, o_proj.bias, k_cache, v_cache, cos, sin,
                                         offset, num_heads, num_kv_heads, head_dim)
    elif qkv.bits == 4:
        out = fused_attention_step_w4a32(x, qkv.qweight, qkv.scales, qkv.bias, o_proj.qweight,
                                         o_proj.scales, o_proj.bias, k_cache, v_cache, cos, sin,
                                         offset, num_heads, num_kv_heads, head_dim,
                                         qkv.group_size)
    else:
        raise ValueError(f"Unsupported bits={qkv.bits}")
    return out.reshape(x.shape)


def fused_transformer_layer_step(x: torch.Tensor, layer: Any, k_cache: torch.Tensor,
                                 v_cache: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                                 offset: int, num_heads: int, num_kv_heads: int, head_dim: int,
                                 eps: float = 1e-6) -> torch.Tensor:
    """One decoder block over a layer of QuantizedLinear modules (reference
    quantization.py:488-572): x is updated in place and returned."""
    at, mlp = layer.self_attn, layer.mlp
    qkv, o, gt, up, dn = at.qkv_proj, at.o_proj, mlp.gate_proj, mlp.up_proj, mlp.down_proj
    fused_transformer_layer_step_w4a32(
        x, layer.input_layernorm.weight, qkv.qweight, qkv.scales, qkv.bias, o.qweight, o.scales,
        o.bias, layer.post_attention_layernorm.weight, gt.qweight, gt.scales, gt.bias, up.qweight,
        up.scales, up.bias, dn.qweight, dn.scales, dn.bias, k_cache, v_cache, cos, sin, offset,
        num_heads, num_kv_heads, head_dim, qkv.group_size, eps)
    return x


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

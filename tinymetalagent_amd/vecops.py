"""torch-tensor wrappers of the decode-layer vector operations (the te_hip_*
device entry points of libtinyengine.so): quantized matvec over GGUF-format
weights, RMSNorm, SwiGLU, residual add and argmax.

Weights are byte tensors holding the GGUF tensor data (rows back to back, the
block formats of reference c/src/ops.c:15-21); every call enqueues on the
current (or given) stream and raises TinyEngineError on a non-OK status.
"""
from __future__ import annotations

import torch

from .attention import _ptr, _stream
from .runtime import check, load_library

GGML_F32, GGML_Q4_0, GGML_Q8_0 = 0, 2, 8
_BLOCK_BYTES = {GGML_Q4_0: 18, GGML_Q8_0: 34}


def row_bytes(ggml_type: int, cols: int) -> int:
    if ggml_type == GGML_F32:
        return cols * 4
    return cols // 32 * _BLOCK_BYTES[ggml_type]


def matvec(weights: torch.Tensor, ggml_type: int, x: torch.Tensor, rows: int, *, out=None, stream=None):
    """out[r] = sum_c W[r][c] * x[c] for the [rows][len(x)] GGUF tensor in `weights` (uint8, on the GPU)."""
    cols = x.numel()
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise TypeError("x must be a contiguous float32 tensor")
    if weights.dtype != torch.uint8 or weights.numel() < rows * row_bytes(ggml_type, cols):
        raise ValueError("weights must be a uint8 tensor holding rows x row_bytes bytes")
    if out is None:
        out = torch.empty(rows, dtype=torch.float32, device=x.device)
    check(load_library().te_hip_matvec_f32(_ptr(weights), ggml_type, _ptr(x), cols, rows, _ptr(out),
                                           _stream(stream)))
    return out


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, epsilon: float, *, out=None, stream=None):
    """RMSNorm of each row of x ([rows, len] or [len]) with one weight vector."""
    rows, n = (1, x.numel()) if x.dim() == 1 else (x.numel() // x.shape[-1], x.shape[-1])
    if out is None:
        out = torch.empty_like(x)
    check(load_library().te_hip_rmsnorm_f32(_ptr(x), _ptr(weight), rows, n, epsilon, _ptr(out), _stream(stream)))
    return out


def swiglu(gate: torch.Tensor, up: torch.Tensor, *, out=None, stream=None):
    if out is None:
        out = torch.empty_like(gate)
    check(load_library().te_hip_swiglu_f32(_ptr(gate), _ptr(up), gate.numel(), _ptr(out), _stream(stream)))
    return out


def add(lhs: torch.Tensor, rhs: torch.Tensor, *, out=None, stream=None):
    if out is None:
        out = torch.empty_like(lhs)
    check(load_library().te_hip_add_f32(_ptr(lhs), _ptr(rhs), lhs.numel(), _ptr(out), _stream(stream)))
    return out


def argmax(values: torch.Tensor, *, out=None, stream=None) -> torch.Tensor:
    """Index of the first maximum, as a one-element int32 tensor on the device."""
    if out is None:
        out = torch.empty(1, dtype=torch.int32, device=values.device)
    check(load_library().te_hip_argmax_f32(_ptr(values), values.numel(), _ptr(out), _stream(stream)))
    return out

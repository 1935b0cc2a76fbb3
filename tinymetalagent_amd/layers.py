"""torch-tensor wrapper of te_hip_decode_all_layers_f16: one decode token through
every layer of a Qwen2 model (and optionally the final norm, lm_head and argmax),
the HIP twin of the reference's te_metal_decode_all_layers_f32
(c/src/metal_backend.h:239-276).

`mapping` is a uint8 device tensor holding the model's tensor bytes; `offsets`
maps "q", "k", "v", "output", "gate", "up", "down" to per-layer byte offsets into
it.  Everything else is a device tensor; the call is asynchronous on the current
(or given) stream and raises TinyEngineError on a non-OK status.
"""
from __future__ import annotations

import ctypes

import torch

from .attention import _ptr, _stream
from .runtime import check, load_library

_NAMES = ("q", "k", "v", "output", "gate", "up", "down")


def workspace_bytes(position: int, hidden: int, kv: int, heads: int, kv_heads: int, head_dim: int, ffn: int,
                    vocab: int = 0) -> int:
    return int(load_library().te_hip_decode_all_layers_workspace_bytes(position, hidden, kv, heads, kv_heads,
                                                                       head_dim, ffn, vocab))


def workspace(position: int, hidden: int, kv: int, heads: int, kv_heads: int, head_dim: int, ffn: int,
              vocab: int = 0, device="cuda") -> torch.Tensor:
    return torch.empty(workspace_bytes(position, hidden, kv, heads, kv_heads, head_dim, ffn, vocab),
                       dtype=torch.uint8, device=device)


def decode_all_layers(mapping: torch.Tensor, offsets: dict, layers: int, ggml_type: int, hidden_in: torch.Tensor,
                      attn_norm: torch.Tensor, ffn_norm: torch.Tensor, q_bias: torch.Tensor, k_bias: torch.Tensor,
                      v_bias: torch.Tensor, rope_cos: torch.Tensor, rope_sin: torch.Tensor,
                      key_cache: torch.Tensor, value_cache: torch.Tensor, position: int, context_tokens: int,
                      heads: int, kv_heads: int, head_dim: int, ffn: int, epsilon: float, *, out=None,
                      head=None, output_norm=None, vocab: int = 0, token_out=None, ws=None, stream=None):
    """Returns `out` (the final hidden state); with head = (offset, ggml_type),
    also writes the greedy next token to `token_out` (int32 device tensor, made
    when not given) and returns (out, token_out)."""
    hidden = heads * head_dim
    kv = kv_heads * head_dim
    arrays = [(ctypes.c_uint64 * layers)(*[int(o) for o in offsets[n]]) for n in _NAMES]
    if out is None:
        out = torch.empty_like(hidden_in)
    want_token = head is not None
    if want_token and token_out is None:
        token_out = torch.empty(1, dtype=torch.int32, device=hidden_in.device)
    if ws is None:
        ws = workspace(position, hidden, kv, heads, kv_heads, head_dim, ffn, vocab if want_token else 0,
                       hidden_in.device)
    head_off, head_type = head if want_token else (0, 0)
    check(load_library().te_hip_decode_all_layers_f16(
        _ptr(mapping), mapping.numel(), *[ctypes.cast(a, ctypes.POINTER(ctypes.c_uint64)) for a in arrays],
        layers, ggml_type, _ptr(hidden_in), _ptr(attn_norm), _ptr(ffn_norm), _ptr(q_bias), _ptr(k_bias),
        _ptr(v_bias), _ptr(rope_cos), _ptr(rope_sin), _ptr(key_cache), _ptr(value_cache), position,
        context_tokens, hidden, kv, heads, kv_heads, head_dim, ffn, epsilon, _ptr(out), head_off, head_type,
        _ptr(output_norm) if want_token else None, vocab if want_token else 0,
        _ptr(token_out) if want_token else None, _ptr(ws), ws.numel(), _stream(stream)))
    return (out, token_out) if want_token else out


def prefill_workspace(batch: int, hidden: int, kv: int, ffn: int, device="cuda") -> torch.Tensor:
    n = int(load_library().te_hip_prefill_all_layers_workspace_bytes(batch, hidden, kv, ffn))
    return torch.empty(n, dtype=torch.uint8, device=device)


def prefill_all_layers(mapping: torch.Tensor, offsets: dict, layers: int, ggml_type: int, hidden_in: torch.Tensor,
                       attn_norm: torch.Tensor, ffn_norm: torch.Tensor, q_bias: torch.Tensor, k_bias: torch.Tensor,
                       v_bias: torch.Tensor, rope_cos: torch.Tensor, rope_sin: torch.Tensor,
                       key_cache: torch.Tensor, value_cache: torch.Tensor, value_t: torch.Tensor,
                       base_position: int, context_tokens: int, heads: int, kv_heads: int, head_dim: int, ffn: int,
                       epsilon: float, *, out=None, ws=None, stream=None) -> torch.Tensor:
    """te_hip_prefill_all_layers_f16: hidden_in [batch, hidden] at positions
    base_position .. base_position + batch - 1 through every layer; returns the
    final hidden states [batch, hidden] and appends every layer's k / v (and
    V^T) for those positions."""
    batch = hidden_in.shape[0]
    hidden = heads * head_dim
    kv = kv_heads * head_dim
    arrays = [(ctypes.c_uint64 * layers)(*[int(o) for o in offsets[n]]) for n in _NAMES]
    if out is None:
        out = torch.empty_like(hidden_in)
    if ws is None:
        ws = prefill_workspace(batch, hidden, kv, ffn, hidden_in.device)
    check(load_library().te_hip_prefill_all_layers_f16(
        _ptr(mapping), mapping.numel(), *[ctypes.cast(a, ctypes.POINTER(ctypes.c_uint64)) for a in arrays],
        layers, ggml_type, _ptr(hidden_in), _ptr(attn_norm), _ptr(ffn_norm), _ptr(q_bias), _ptr(k_bias),
        _ptr(v_bias), _ptr(rope_cos), _ptr(rope_sin), _ptr(key_cache), _ptr(value_cache), _ptr(value_t),
        base_position, batch, context_tokens, hidden, kv, heads, kv_heads, head_dim, ffn, epsilon, _ptr(out),
        _ptr(ws), ws.numel(), _stream(stream)))
    return out

"""Device-level attention step on torch tensors (HBM-resident inputs).

Thin wrappers over the te_hip_* C-ABI entry points of libtinyengine.so.  torch
only provides device memory and the current HIP stream; every arithmetic step
runs in the library's hand-written gfx950 kernels.  Tensors must be contiguous,
on the GPU, with the dtypes and layouts of include/te_hip_backend.h:

    q, out        float32  [seqs, layers, tokens, heads, head_dim]
    k, v          float32  [seqs, layers, tokens, kv_heads, head_dim]
    key/value     float16  [seqs, layers, context_tokens, kv_heads, head_dim]
    rope cos/sin  float32  [context_tokens, head_dim // 2]

A missing library or GPU raises TinyEngineError; nothing falls back to the CPU.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from .runtime import TE_HIP_MAX_SEQS, TinyEngineError, check, load_library


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise TinyEngineError("invalid argument: tensor is not on the GPU")
    if not t.is_contiguous():
        raise TinyEngineError("invalid argument: tensor is not contiguous")
    return t.data_ptr()


def _dtype(t: torch.Tensor | None, dtype: torch.dtype, name: str) -> None:
    if t is not None and t.dtype != dtype:
        raise TinyEngineError(f"invalid argument: {name} must be {dtype}, got {t.dtype}")


def _stream(stream: torch.cuda.Stream | None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _positions(positions: Sequence[int] | None):
    if positions is None:
        return None
    if len(positions) > TE_HIP_MAX_SEQS:
        raise TinyEngineError("unsupported")
    arr = (ctypes.c_size_t * len(positions))(*[int(p) for p in positions])
    return arr


def rope_table(context_tokens: int, head_dim: int, theta: float, device="cuda"):
    """Device cos/sin tables built with the reference formula (host libm)."""
    cos = torch.empty((context_tokens, head_dim // 2), dtype=torch.float32, device=device)
    sin = torch.empty_like(cos)
    check(load_library().te_hip_rope_table_f32(_ptr(cos), _ptr(sin), context_tokens, head_dim,
                                               ctypes.c_float(theta)))
    return cos, sin


def rope_kv_append(q, k, v, rope_cos, rope_sin, key_cache, value_cache, *, base_position: int = 0,
                   base_positions: Sequence[int] | None = None, q_bias=None, k_bias=None, v_bias=None,
                   q_half: torch.Tensor | None = None, stream=None) -> None:
    """In place: bias + RoPE on q/k (and bias on v), fp16 append of k/v to the cache."""
    seqs, layers, tokens, heads, head_dim = q.shape
    kv_heads = k.shape[3]
    ctx = key_cache.shape[2]
    for t, dt, n in ((q, torch.float32, "q"), (k, torch.float32, "k"), (v, torch.float32, "v"),
                     (key_cache, torch.float16, "key_cache"), (value_cache, torch.float16, "value_cache"),
                     (q_half, torch.float16, "q_half"), (rope_cos, torch.float32, "rope_cos"),
                     (rope_sin, torch.float32, "rope_sin")):
        _dtype(t, dt, n)
    bp = _positions(base_positions)
    check(load_library().te_hip_rope_kv_append_f16(
        _ptr(q), _ptr(k), _ptr(v), _ptr(q_bias), _ptr(k_bias), _ptr(v_bias), _ptr(rope_cos), _ptr(rope_sin),
        _ptr(key_cache), _ptr(value_cache), _ptr(q_half), seqs, layers, tokens, bp, base_position, ctx, heads,
        kv_heads, head_dim, _stream(stream)))


def decode_workspace(seqs: int, layers: int, heads: int, kv_heads: int, head_dim: int, *, position: int = 0,
                     positions: Sequence[int] | None = None, device="cuda") -> torch.Tensor:
    """Workspace for attention_decode with exactly these positions."""
    n = load_library().te_hip_attention_decode_workspace_bytes(_positions(positions), position, seqs, layers, heads,
                                                                kv_heads, head_dim)
    if n == 0:
        raise TinyEngineError("invalid argument")
    return torch.empty(n, dtype=torch.uint8, device=device)


def attention_decode(query, key_cache, value_cache, *, position: int = 0, positions: Sequence[int] | None = None,
                     out: torch.Tensor | None = None, workspace: torch.Tensor | None = None, stream=None,
                     stage: str = "both") -> torch.Tensor:
    """Split-K GQA decode: query [seqs, layers, heads, d] (or with a tokens=1 axis).

    stage: "both" (split-K + combine), "splitk" or "combine" -- the last two let
    a caller time the split-K kernel alone (the workspace must be given).
    """
    q = query if query.dim() == 4 else query.reshape(query.shape[0], query.shape[1], query.shape[-2],
                                                     query.shape[-1])
    seqs, layers, heads, head_dim = q.shape
    ctx, kv_heads = key_cache.shape[2], key_cache.shape[3]
    _dtype(q, torch.float32, "query")
    _dtype(key_cache, torch.float16, "key_cache")
    _dtype(value_cache, torch.float16, "value_cache")
    if out is None:
        out = torch.empty_like(q)
    pp = _positions(positions)
    lib = load_library()
    ws_ptr = _ptr(workspace)
    ws_bytes = workspace.numel() if workspace is not None else 0
    s = _stream(stream)
    if stage == "both":
        check(lib.te_hip_attention_decode_f16(_ptr(q), _ptr(key_cache), _ptr(value_cache), pp, position, seqs,
                                              layers, ctx, heads, kv_heads, head_dim, _ptr(out), ws_ptr, ws_bytes,
                                              s))
    elif stage == "splitk":
        check(lib.te_hip_attention_decode_splitk_f16(_ptr(q), _ptr(key_cache), _ptr(value_cache), pp, position,
                                                     seqs, layers, ctx, heads, kv_heads, head_dim, ws_ptr,
                                                     ws_bytes, s))
    elif stage == "combine":
        check(lib.te_hip_attention_decode_combine(pp, position, seqs, layers, heads, kv_heads, head_dim, _ptr(out),
                                                  ws_ptr, ws_bytes, s))
    else:
        raise ValueError(stage)
    return out


def decode_step(query, k_new, v_new, rope_cos, rope_sin, key_cache, value_cache, *, position: int = 0,
                positions: Sequence[int] | None = None, q_bias=None, k_bias=None, v_bias=None,
                out: torch.Tensor | None = None, workspace: torch.Tensor | None = None, stream=None,
                stage: str = "both") -> torch.Tensor:
    """Fused decode step: bias + RoPE + fp16 append of the new token and split-K
    attention, one split-K launch + the combine.  query/k_new/v_new are read only.

    stage: "both", or "splitk" for the fused split-K launch alone (partials into
    the workspace; attention_decode(..., stage="combine") finishes the step)."""
    q = query if query.dim() == 4 else query.reshape(query.shape[0], query.shape[1], query.shape[-2],
                                                     query.shape[-1])
    seqs, layers, heads, head_dim = q.shape
    ctx, kv_heads = key_cache.shape[2], key_cache.shape[3]
    for t, dt, n in ((q, torch.float32, "query"), (k_new, torch.float32, "k_new"), (v_new, torch.float32, "v_new"),
                     (key_cache, torch.float16, "key_cache"), (value_cache, torch.float16, "value_cache")):
        _dtype(t, dt, n)
    if out is None:
        out = torch.empty_like(q)
    if workspace is None:
        workspace = decode_workspace(seqs, layers, heads, kv_heads, head_dim, position=position, positions=positions,
                                     device=q.device)
    lib = load_library()
    args = (_ptr(q), _ptr(k_new), _ptr(v_new), _ptr(q_bias), _ptr(k_bias), _ptr(v_bias), _ptr(rope_cos),
            _ptr(rope_sin), _ptr(key_cache), _ptr(value_cache), _positions(positions), position, seqs, layers, ctx,
            heads, kv_heads, head_dim)
    if stage == "both":
        check(lib.te_hip_attention_decode_step_f16(*args, _ptr(out), _ptr(workspace), workspace.numel(),
                                                   _stream(stream)))
    elif stage == "splitk":
        check(lib.te_hip_attention_decode_step_splitk_f16(*args, _ptr(workspace), workspace.numel(),
                                                          _stream(stream)))
    else:
        raise ValueError(stage)
    return out


def decode_step_noalloc(query, k_new, v_new, rope_cos, rope_sin, key_cache, value_cache, *, position: int = 0,
                        positions: Sequence[int] | None = None, q_bias=None, k_bias=None, v_bias=None,
                        out: torch.Tensor, stream=None) -> torch.Tensor:
    """decode_step through te_hip_attention_decode_step_noalloc_f16: the split-K
    partials live in the library's per-GPU device array, so the call allocates
    nothing (`out` is required).  Calls that overlap on one GPU race."""
    q = query if query.dim() == 4 else query.reshape(query.shape[0], query.shape[1], query.shape[-2],
                                                     query.shape[-1])
    seqs, layers, heads, head_dim = q.shape
    ctx, kv_heads = key_cache.shape[2], key_cache.shape[3]
    for t, dt, n in ((q, torch.float32, "query"), (k_new, torch.float32, "k_new"), (v_new, torch.float32, "v_new"),
                     (key_cache, torch.float16, "key_cache"), (value_cache, torch.float16, "value_cache"),
                     (out, torch.float32, "out")):
        _dtype(t, dt, n)
    check(load_library().te_hip_attention_decode_step_noalloc_f16(
        _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(q_bias), _ptr(k_bias), _ptr(v_bias), _ptr(rope_cos), _ptr(rope_sin),
        _ptr(key_cache), _ptr(value_cache), _positions(positions), position, seqs, layers, ctx, heads, kv_heads,
        head_dim, _ptr(out), _stream(stream)))
    return out


def attention_prefill(q_half, key_cache, value_cache, *, base_position: int = 0, out: torch.Tensor | None = None,
                      stream=None) -> torch.Tensor:
    """Causal prefill: q_half fp16 [seqs, layers, tokens, heads, d] -> out fp32, same shape."""
    seqs, layers, tokens, heads, head_dim = q_half.shape
    ctx, kv_heads = key_cache.shape[2], key_cache.shape[3]
    _dtype(q_half, torch.float16, "q_half")
    _dtype(key_cache, torch.float16, "key_cache")
    _dtype(value_cache, torch.float16, "value_cache")
    if out is None:
        out = torch.empty(q_half.shape, dtype=torch.float32, device=q_half.device)
    check(load_library().te_hip_attention_prefill_f16(_ptr(q_half), _ptr(key_cache), _ptr(value_cache), seqs,
                                                      layers, tokens, base_position, ctx, heads, kv_heads, head_dim,
                                                      _ptr(out), _stream(stream)))
    return out


def value_t_buffer(seqs: int, layers: int, context_tokens: int, kv_heads: int, head_dim: int,
                   device="cuda") -> torch.Tensor:
    """A zeroed V^T buffer [seqs, layers, kv_heads, head_dim, ctx_pad] (fp16) for
    the *_vt prefill entry points; ctx_pad = context_tokens rounded up to 64."""
    n = load_library().te_hip_value_t_bytes(seqs, layers, context_tokens, kv_heads, head_dim)
    if n == 0:
        raise TinyEngineError("invalid argument")
    pad = n // (2 * seqs * layers * kv_heads * head_dim)
    return torch.zeros((seqs, layers, kv_heads, head_dim, pad), dtype=torch.float16, device=device)


def value_transpose(value_cache, value_t, *, first_position: int = 0, count: int | None = None,
                    stream=None) -> torch.Tensor:
    """te_hip_value_transpose_f16: V^T of positions [first, first + count) of
    every (seq, layer, kv head) into value_t (zeros up to the next multiple of 8)."""
    seqs, layers, ctx, kv_heads, head_dim = value_cache.shape
    _dtype(value_cache, torch.float16, "value_cache")
    _dtype(value_t, torch.float16, "value_t")
    if count is None:
        count = ctx - first_position
    check(load_library().te_hip_value_transpose_f16(_ptr(value_cache), _ptr(value_t), seqs, layers, first_position,
                                                    count, ctx, kv_heads, head_dim, _stream(stream)))
    return value_t


def prefill_vt_workspace(seqs: int, layers: int, tokens: int, heads: int, kv_heads: int, head_dim: int, *,
                         base_position: int = 0, context_tokens: int, device="cuda") -> torch.Tensor | None:
    """Key-split partials for the *_vt prefill entry points (None: no split)."""
    n = load_library().te_hip_attention_prefill_vt_workspace_bytes(seqs, layers, tokens, base_position,
                                                                   context_tokens, heads, kv_heads, head_dim)
    return None if n == 0 else torch.empty(n, dtype=torch.uint8, device=device)


def attention_prefill_vt(q_half, key_cache, value_t, *, base_position: int = 0, out: torch.Tensor | None = None,
                         workspace: torch.Tensor | None = None, context_tokens: int | None = None,
                         stream=None) -> torch.Tensor:
    """Causal prefill over the K cache and V^T; `workspace` (prefill_vt_workspace)
    lets the launch split keys, None runs one split."""
    seqs, layers, tokens, heads, head_dim = q_half.shape
    ctx, kv_heads = key_cache.shape[2], key_cache.shape[3]
    _dtype(q_half, torch.float16, "q_half")
    _dtype(key_cache, torch.float16, "key_cache")
    _dtype(value_t, torch.float16, "value_t")
    if out is None:
        out = torch.empty(q_half.shape, dtype=torch.float32, device=q_half.device)
    nbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(load_library().te_hip_attention_prefill_vt_f16(
        _ptr(q_half), _ptr(key_cache), _ptr(value_t), seqs, layers, tokens, base_position, ctx, heads, kv_heads,
        head_dim, _ptr(out), _ptr(workspace), nbytes, _stream(stream)))
    return out


def prefill_step_vt(query, k_new, v_new, rope_cos, rope_sin, key_cache, value_cache, value_t, *,
                    base_position: int = 0, q_bias=None, k_bias=None, v_bias=None, out: torch.Tensor | None = None,
                    workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Fused prefill step keeping V^T: bias + RoPE + fp16 append of the chunk's
    k / v (into key_cache, value_cache and value_t), then the causal attention
    over the K cache and V^T.  query / k_new / v_new are read only."""
    seqs, layers, tokens, heads, head_dim = query.shape
    ctx, kv_heads = key_cache.shape[2], key_cache.shape[3]
    for t, dt, n in ((query, torch.float32, "query"), (k_new, torch.float32, "k_new"),
                     (v_new, torch.float32, "v_new"), (key_cache, torch.float16, "key_cache"),
                     (value_cache, torch.float16, "value_cache"), (value_t, torch.float16, "value_t")):
        _dtype(t, dt, n)
    if out is None:
        out = torch.empty(query.shape, dtype=torch.float32, device=query.device)
    nbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(load_library().te_hip_attention_prefill_step_vt_f16(
        _ptr(query), _ptr(k_new), _ptr(v_new), _ptr(q_bias), _ptr(k_bias), _ptr(v_bias), _ptr(rope_cos),
        _ptr(rope_sin), _ptr(key_cache), _ptr(value_cache), _ptr(value_t), seqs, layers, tokens, base_position, ctx,
        heads, kv_heads, head_dim, _ptr(out), _ptr(workspace), nbytes, _stream(stream)))
    return out


def prefill_workspace(seqs: int, layers: int, tokens: int, heads: int, kv_heads: int, head_dim: int, *,
                      base_position: int = 0, context_tokens: int, device="cuda") -> torch.Tensor | None:
    """Workspace for attention_prefill_split: the key-split partials (none when
    the launch does not split) plus a V^T of the whole prefix, which the split
    entry rebuilds on every call -- so it is never None.  Chunked prefill over
    a long cache should keep a V^T buffer and use the *_vt entries instead."""
    n = load_library().te_hip_attention_prefill_workspace_bytes(seqs, layers, tokens, base_position, context_tokens,
                                                                heads, kv_heads, head_dim)
    if n == 0:
        raise TinyEngineError("invalid argument")
    return torch.empty(n, dtype=torch.uint8, device=device)


def attention_prefill_split(q_half, key_cache, value_cache, *, base_position: int = 0, out: torch.Tensor | None = None,
                            workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """attention_prefill with the key-split launch (partials in `workspace`, then a merge)."""
    seqs, layers, tokens, heads, head_dim = q_half.shape
    ctx, kv_heads = key_cache.shape[2], key_cache.shape[3]
    _dtype(q_half, torch.float16, "q_half")
    _dtype(key_cache, torch.float16, "key_cache")
    _dtype(value_cache, torch.float16, "value_cache")
    if out is None:
        out = torch.empty(q_half.shape, dtype=torch.float32, device=q_half.device)
    if workspace is None:
        workspace = prefill_workspace(seqs, layers, tokens, heads, kv_heads, head_dim, base_position=base_position,
                                      context_tokens=ctx, device=q_half.device)
    nbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(load_library().te_hip_attention_prefill_split_f16(
        _ptr(q_half), _ptr(key_cache), _ptr(value_cache), seqs, layers, tokens, base_position, ctx, heads, kv_heads,
        head_dim, _ptr(out), _ptr(workspace), nbytes, _stream(stream)))
    return out


def prefill_step(query, k_new, v_new, rope_cos, rope_sin, key_cache, value_cache, *, base_position: int = 0,
                 q_bias=None, k_bias=None, v_bias=None, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Fused prefill step: bias + RoPE + fp16 append of the chunk's k/v, then causal
    attention with bias + RoPE of q applied on load.  query fp32 [seqs, layers,
    tokens, heads, d]; query/k_new/v_new are read only; out fp32, same shape."""
    seqs, layers, tokens, heads, head_dim = query.shape
    ctx, kv_heads = key_cache.shape[2], key_cache.shape[3]
    for t, dt, n in ((query, torch.float32, "query"), (k_new, torch.float32, "k_new"), (v_new, torch.float32, "v_new"),
                     (key_cache, torch.float16, "key_cache"), (value_cache, torch.float16, "value_cache"),
                     (rope_cos, torch.float32, "rope_cos"), (rope_sin, torch.float32, "rope_sin")):
        _dtype(t, dt, n)
    if out is None:
        out = torch.empty(query.shape, dtype=torch.float32, device=query.device)
    check(load_library().te_hip_attention_prefill_step_f16(
        _ptr(query), _ptr(k_new), _ptr(v_new), _ptr(q_bias), _ptr(k_bias), _ptr(v_bias), _ptr(rope_cos),
        _ptr(rope_sin), _ptr(key_cache), _ptr(value_cache), seqs, layers, tokens, base_position, ctx, heads,
        kv_heads, head_dim, _ptr(out), _stream(stream)))
    return out

"""TEST INFRASTRUCTURE ONLY: ctypes access to the CPU parity checker.

`oracle/_build/liboracle.so` is this repository's C restatement of the
reference attention step (te_oracle.c); `oracle/_ref/libte_ref_ops.so` is the
reference's own c/src/ops.c compiled from the read-only reference tree (built
only where that tree exists).  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import this package; the product library never
does.

All wrappers take and return numpy arrays (float32 / uint16 fp16 bits).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "_build" / "liboracle.so"
REF_LIB = HERE / "_ref" / "libte_ref_ops.so"
REFERENCE_TREE = Path(os.environ.get("TE_REFERENCE_TREE", "/root/reference"))

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_szp = ctypes.POINTER(ctypes.c_size_t)
_sz = ctypes.c_size_t

_oracle = None
_ref = None


def build(with_reference: bool | None = None) -> None:
    """Compile the oracle (and the reference ops.c when its tree is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    if with_reference is None:
        with_reference = (REFERENCE_TREE / "c" / "src" / "ops.c").is_file()
    if with_reference:
        subprocess.run(["make", "-s", "-C", str(HERE), "ref", f"REFERENCE={REFERENCE_TREE}"], check=True)


def _p(a: np.ndarray, ptype):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ptype)


def lib() -> ctypes.CDLL:
    global _oracle
    if _oracle is None:
        if not ORACLE_LIB.is_file():
            # Never compiled on demand: a test process may already hold the
            # GPU, and the GPU box only runs what was built beforehand.
            raise RuntimeError(f"{ORACLE_LIB} is missing: build it first (__graft_entry__.build() or "
                               f"`make -C {HERE}`)")
        l = ctypes.CDLL(str(ORACLE_LIB))
        l.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        l.orc_f16_to_f32.restype = ctypes.c_float
        l.orc_f32_to_f16_rne.argtypes = [ctypes.c_float]
        l.orc_f32_to_f16_rne.restype = ctypes.c_uint16
        l.orc_f16_to_f32_array.argtypes = [_u16p, _f32p, _sz]
        l.orc_f32_to_f16_array.argtypes = [_f32p, _u16p, _sz]
        l.orc_rope_f32.argtypes = [_f32p, _sz, _sz, _sz, ctypes.c_float]
        l.orc_rope_table.argtypes = [_f32p, _f32p, _sz, _sz, ctypes.c_float]
        l.orc_rope_cached.argtypes = [_f32p, _sz, _sz, _f32p, _f32p, _sz]
        l.orc_attention_decode_f32.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _f32p]
        l.orc_rope_kv_append_f16.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                             _u16p, _u16p, _sz, _sz, _sz, _szp, _sz, _sz, _sz, _sz, _sz]
        l.orc_attention_decode_f16kv.argtypes = [_f32p, _u16p, _u16p, _szp, _sz, _sz, _sz, _sz, _sz, _sz,
                                                 _sz, _f32p]
        l.orc_attention_prefill.argtypes = [_f32p, _u16p, _u16p, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz,
                                            _sz, _f32p]
        _bind_vector_ops(l, "orc_")
        l.orc_ggml_row_bytes.argtypes = [ctypes.c_uint32, _sz]
        l.orc_ggml_row_bytes.restype = _sz
        l.orc_dequantize_row_f32.argtypes = [_u8p, ctypes.c_uint32, _sz, _sz, _f32p]
        l.orc_matvec_f32.argtypes = [_u8p, ctypes.c_uint32, _f32p, _sz, _sz, _f32p]
        _oracle = l
    return _oracle


def ref_lib() -> ctypes.CDLL | None:
    """The compiled reference ops.c, or None when it was not built here."""
    global _ref
    if _ref is None and REF_LIB.is_file():
        l = ctypes.CDLL(str(REF_LIB))
        l.te_rope_f32.argtypes = [_f32p, _sz, _sz, _sz, ctypes.c_float]
        l.te_rope_f32.restype = ctypes.c_int
        l.te_attention_decode_f32.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _f32p]
        l.te_attention_decode_f32.restype = ctypes.c_int
        _bind_vector_ops(l, "te_")
        _ref = l
    return _ref


def _bind_vector_ops(l: ctypes.CDLL, prefix: str) -> None:
    for name, args in (("rmsnorm_f32", [_f32p, _f32p, _sz, ctypes.c_float, _f32p]),
                       ("swiglu_f32", [_f32p, _f32p, _sz, _f32p]),
                       ("add_f32", [_f32p, _f32p, _sz, _f32p]),
                       ("argmax_f32", [_f32p, _sz, _u32p])):
        fn = getattr(l, prefix + name)
        fn.argtypes = args
        fn.restype = ctypes.c_int


def _check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"oracle {what} returned status {status}")


# ---- fp16 -------------------------------------------------------------------

def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(_p(bits, _u16p), _p(out, _f32p), bits.size)
    return out


def f32_to_f16(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(values.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(_p(values, _f32p), _p(out, _u16p), values.size)
    return out


# ---- RoPE -------------------------------------------------------------------

def rope_f32(values: np.ndarray, heads: int, head_dim: int, position: int, theta: float, *, use_ref=False):
    """Returns a rotated copy; raises on a non-OK status."""
    v = np.array(values, dtype=np.float32, copy=True, order="C")
    fn = ref_lib().te_rope_f32 if use_ref else lib().orc_rope_f32
    _check(fn(_p(v, _f32p), heads, head_dim, position, ctypes.c_float(theta)), "rope_f32")
    return v


def rope_status(values, heads, head_dim, position, theta, *, use_ref=False) -> int:
    v = None if values is None else np.array(values, dtype=np.float32, copy=True, order="C")
    fn = ref_lib().te_rope_f32 if use_ref else lib().orc_rope_f32
    return fn(_p(v, _f32p) if v is not None else None, heads, head_dim, position, ctypes.c_float(theta))


def rope_table(context_tokens: int, head_dim: int, theta: float):
    cos = np.empty((context_tokens, head_dim // 2), dtype=np.float32)
    sin = np.empty_like(cos)
    _check(lib().orc_rope_table(_p(cos, _f32p), _p(sin, _f32p), context_tokens, head_dim,
                                ctypes.c_float(theta)), "rope_table")
    return cos, sin


def rope_cached(values, heads, head_dim, cos, sin, position):
    v = np.array(values, dtype=np.float32, copy=True, order="C")
    _check(lib().orc_rope_cached(_p(v, _f32p), heads, head_dim, _p(cos, _f32p), _p(sin, _f32p), position),
           "rope_cached")
    return v


# ---- attention --------------------------------------------------------------

def attention_decode_f32(query, key_cache, value_cache, position, heads, kv_heads, head_dim, *, use_ref=False):
    q = np.ascontiguousarray(query, dtype=np.float32)
    k = np.ascontiguousarray(key_cache, dtype=np.float32)
    v = np.ascontiguousarray(value_cache, dtype=np.float32)
    out = np.zeros(heads * head_dim, dtype=np.float32)
    fn = ref_lib().te_attention_decode_f32 if use_ref else lib().orc_attention_decode_f32
    _check(fn(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), position, heads, kv_heads, head_dim, _p(out, _f32p)),
           "attention_decode_f32")
    return out


def rope_kv_append_f16(q, k, v, q_bias, k_bias, v_bias, cos, sin, key_cache, value_cache, seqs, layers, tokens,
                       base_positions, base_position, context_tokens, heads, kv_heads, head_dim):
    """In-place on q, k, v, key_cache, value_cache (numpy arrays)."""
    bp = None
    if base_positions is not None:
        bp = np.ascontiguousarray(base_positions, dtype=np.uintp)
    _check(lib().orc_rope_kv_append_f16(
        _p(q, _f32p), _p(k, _f32p), _p(v, _f32p), _p(q_bias, _f32p), _p(k_bias, _f32p), _p(v_bias, _f32p),
        _p(cos, _f32p), _p(sin, _f32p), _p(key_cache, _u16p), _p(value_cache, _u16p), seqs, layers, tokens,
        _p(bp, _szp) if bp is not None else None, base_position, context_tokens, heads, kv_heads, head_dim),
        "rope_kv_append_f16")


def attention_decode_f16kv(query, key_cache, value_cache, positions, position, seqs, layers, context_tokens,
                           heads, kv_heads, head_dim):
    q = np.ascontiguousarray(query, dtype=np.float32)
    out = np.zeros(seqs * layers * heads * head_dim, dtype=np.float32)
    pp = None if positions is None else np.ascontiguousarray(positions, dtype=np.uintp)
    _check(lib().orc_attention_decode_f16kv(
        _p(q, _f32p), _p(key_cache, _u16p), _p(value_cache, _u16p), _p(pp, _szp) if pp is not None else None,
        position, seqs, layers, context_tokens, heads, kv_heads, head_dim, _p(out, _f32p)),
        "attention_decode_f16kv")
    return out.reshape(seqs, layers, heads, head_dim)


def attention_prefill(query, key_cache, value_cache, tokens, base_position, context_tokens, heads, kv_heads,
                      head_dim, row_begin=0, row_end=None, row_step=1):
    """query fp32 [tokens][heads][d]; caches fp16 bits [ctx][kv][d] for one (seq, layer).
    Rows outside the sample are NaN in the result."""
    q = np.ascontiguousarray(query, dtype=np.float32)
    out = np.full(tokens * heads * head_dim, np.nan, dtype=np.float32)
    if row_end is None:
        row_end = tokens
    _check(lib().orc_attention_prefill(
        _p(q, _f32p), _p(np.ascontiguousarray(key_cache), _u16p), _p(np.ascontiguousarray(value_cache), _u16p),
        tokens, base_position, context_tokens, heads, kv_heads, head_dim, row_begin, row_end, row_step,
        _p(out, _f32p)), "attention_prefill")
    return out.reshape(tokens, heads, head_dim)


# ---- decode-layer vector operations ------------------------------------------

def _vec_lib(use_ref: bool):
    return (ref_lib(), "te_") if use_ref else (lib(), "orc_")


def rmsnorm_f32(x, weight, epsilon, *, use_ref=False):
    l, pre = _vec_lib(use_ref)
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(weight, dtype=np.float32)
    out = np.empty_like(x)
    _check(getattr(l, pre + "rmsnorm_f32")(_p(x, _f32p), _p(w, _f32p), x.size, ctypes.c_float(epsilon),
                                          _p(out, _f32p)), "rmsnorm_f32")
    return out


def swiglu_f32(gate, up, *, use_ref=False):
    l, pre = _vec_lib(use_ref)
    g = np.ascontiguousarray(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    out = np.empty_like(g)
    _check(getattr(l, pre + "swiglu_f32")(_p(g, _f32p), _p(u, _f32p), g.size, _p(out, _f32p)), "swiglu_f32")
    return out


def add_f32(lhs, rhs, *, use_ref=False):
    l, pre = _vec_lib(use_ref)
    a = np.ascontiguousarray(lhs, dtype=np.float32)
    b = np.ascontiguousarray(rhs, dtype=np.float32)
    out = np.empty_like(a)
    _check(getattr(l, pre + "add_f32")(_p(a, _f32p), _p(b, _f32p), a.size, _p(out, _f32p)), "add_f32")
    return out


def argmax_f32(values, *, use_ref=False) -> int:
    l, pre = _vec_lib(use_ref)
    v = np.ascontiguousarray(values, dtype=np.float32)
    idx = ctypes.c_uint32(0)
    _check(getattr(l, pre + "argmax_f32")(_p(v, _f32p), v.size, ctypes.byref(idx)), "argmax_f32")
    return int(idx.value)


GGML_F32, GGML_Q4_0, GGML_Q8_0 = 0, 2, 8


def ggml_row_bytes(ggml_type: int, cols: int) -> int:
    return int(lib().orc_ggml_row_bytes(ggml_type, cols))


def dequantize_rows(data, ggml_type: int, cols: int, rows: int) -> np.ndarray:
    """All rows of a tensor as fp32 [rows][cols]."""
    d = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty((rows, cols), dtype=np.float32)
    for r in range(rows):
        _check(lib().orc_dequantize_row_f32(_p(d, _u8p), ggml_type, cols, r, _p(out[r], _f32p)), "dequantize_row")
    return out


def matvec_f32(data, ggml_type: int, x, cols: int, rows: int) -> np.ndarray:
    d = np.ascontiguousarray(data, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(rows, dtype=np.float32)
    _check(lib().orc_matvec_f32(_p(d, _u8p), ggml_type, _p(x, _f32p), cols, rows, _p(out, _f32p)), "matvec_f32")
    return out


# ---- one decode token through every layer -----------------------------------

def decode_all_layers(mapping, offsets, layers, ggml_type, hidden_in, attn_norm, ffn_norm, q_bias, k_bias, v_bias,
                      cos, sin, key_cache, value_cache, position, context_tokens, hidden, kv, heads, kv_heads,
                      head_dim, ffn, epsilon, head=None, output_norm=None, vocab=0):
    """The reference's per-token layer loop (qwen.c:907-1087, te_qwen_forward_token)
    composed from this package's restated functions, on the HIP path's fp16 cache:
    per layer rmsnorm -> q/k/v matvec -> bias + RoPE + fp16 append
    (rope_kv_append_f16) -> decode attention (attention_decode_f16kv) -> Wo +
    residual -> rmsnorm -> gate/up -> SwiGLU -> Wd + residual; then, with
    `head` = (offset, type), the greedy projection rmsnorm(output_norm) -> head
    matvec -> argmax (qwen.c:1337-1375).  `mapping` is the model bytes (uint8),
    `offsets` a dict of per-layer byte offsets (q, k, v, output, gate, up, down);
    key_cache / value_cache are fp16 bits [layers][context][kv] and are updated
    in place.  Returns (hidden, token or None, logits or None)."""
    mp = np.ascontiguousarray(mapping, dtype=np.uint8)

    def w(off, rows, cols, t=ggml_type):
        n = rows * ggml_row_bytes(t, cols)
        return mp[off:off + n]

    x = np.array(hidden_in, dtype=np.float32, copy=True)
    for l in range(layers):
        norm = rmsnorm_f32(x, attn_norm[l], epsilon)
        q = matvec_f32(w(offsets["q"][l], hidden, hidden), ggml_type, norm, hidden, hidden)
        k = matvec_f32(w(offsets["k"][l], kv, hidden), ggml_type, norm, hidden, kv)
        v = matvec_f32(w(offsets["v"][l], kv, hidden), ggml_type, norm, hidden, kv)
        kc = key_cache[l]
        vc = value_cache[l]
        rope_kv_append_f16(q, k, v, np.ascontiguousarray(q_bias[l]), np.ascontiguousarray(k_bias[l]),
                           np.ascontiguousarray(v_bias[l]), cos, sin, kc, vc, 1, 1, 1, None, position,
                           context_tokens, heads, kv_heads, head_dim)
        attn = attention_decode_f16kv(q, kc, vc, None, position, 1, 1, context_tokens, heads, kv_heads,
                                      head_dim).reshape(-1)
        proj = matvec_f32(w(offsets["output"][l], hidden, hidden), ggml_type, attn, hidden, hidden)
        x = add_f32(x, proj)
        norm = rmsnorm_f32(x, ffn_norm[l], epsilon)
        gate = matvec_f32(w(offsets["gate"][l], ffn, hidden), ggml_type, norm, hidden, ffn)
        up = matvec_f32(w(offsets["up"][l], ffn, hidden), ggml_type, norm, hidden, ffn)
        proj = matvec_f32(w(offsets["down"][l], hidden, ffn), ggml_type, swiglu_f32(gate, up), ffn, hidden)
        x = add_f32(x, proj)
    if head is None:
        return x, None, None
    head_off, head_type = head
    norm = rmsnorm_f32(x, output_norm, epsilon)
    logits = matvec_f32(w(head_off, vocab, hidden, head_type), head_type, norm, hidden, vocab)
    return x, argmax_f32(logits), logits

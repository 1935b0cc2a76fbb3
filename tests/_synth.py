"""Seeded synthetic inputs shared by the golden-vector script and the tests.

Every tensor is drawn from numpy's PCG64 generator keyed by (seed, tag), so a
test can regenerate exactly the inputs a fixture was made from; fixtures also
store a SHA-256 of the regenerated inputs, checked before any comparison.
fp16 tensors are IEEE round-to-nearest-even of the fp32 draw (numpy's cast,
pinned to the oracle's own RNE in tests/test_oracle.py).
"""
from __future__ import annotations

import hashlib
import zlib

import numpy as np

SEED = 42  # reference c/Makefile:33 ORACLE_SEED


def rng(seed: int, tag: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(tag.encode())])


def normal(seed: int, tag: str, shape, scale: float = 1.0) -> np.ndarray:
    x = rng(seed, tag).standard_normal(size=shape, dtype=np.float64) * scale
    return x.astype(np.float32)


def to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def digest(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def outlier_keys(seed: int, tag: str, shape, channels: int = 3, spike: float = 20.0) -> np.ndarray:
    """K ~ N(0,1) plus +-`spike` on a fixed set of `channels` channels per KV head
    (random sign per element), the config-5 stress pattern.  shape = [..., kv, d]."""
    k = normal(seed, tag, shape)
    d = shape[-1]
    kv = shape[-2]
    r = rng(seed, tag + "/outliers")
    for h in range(kv):
        ch = r.choice(d, size=channels, replace=False)
        signs = r.choice(np.array([-1.0, 1.0], dtype=np.float32), size=shape[:-2] + (channels,))
        k[..., h, ch] += spike * signs
    return k


def ggml_tensor(seed: int, tag: str, ggml_type: int, rows: int, cols: int, scale: float = 0.02) -> np.ndarray:
    """Random GGUF tensor bytes [rows * row_bytes] in the block formats of the
    reference matvec (ops.c:15-21): F32 = 0 (plain floats), Q4_0 = 2 (f16 scale +
    16 bytes of 4-bit codes), Q8_0 = 8 (f16 scale + 32 int8 codes).  Scales are
    positive and negative fp16 values around `scale`; codes are uniform."""
    r = rng(seed, tag)
    if ggml_type == 0:
        return (r.standard_normal((rows, cols)) * scale).astype(np.float32).reshape(-1).view(np.uint8).copy()
    blocks = rows * (cols // 32)
    d = (r.standard_normal(blocks) * scale).astype(np.float16).view(np.uint16)
    if ggml_type == 2:
        codes = r.integers(0, 256, size=(blocks, 16), dtype=np.uint8)
        out = np.empty((blocks, 18), dtype=np.uint8)
    elif ggml_type == 8:
        codes = r.integers(0, 256, size=(blocks, 32), dtype=np.uint8)
        out = np.empty((blocks, 34), dtype=np.uint8)
    else:
        raise ValueError(ggml_type)
    out[:, 0] = d & 0xFF
    out[:, 1] = d >> 8
    out[:, 2:] = codes
    return out.reshape(-1)


def synthetic_model(seed: int, ggml_type: int, layers: int, heads: int, kv_heads: int, head_dim: int, ffn: int,
                    vocab: int, context_tokens: int, position: int, head_type: int | None = None,
                    misalign: int = 0) -> dict:
    """A random Qwen2-shaped decode state: the tensor bytes of every layer's
    seven projections and of the head packed into one `mapping` (each tensor
    32-byte aligned as GGUF data, plus `misalign` bytes), per-layer norm weights
    and biases, the input hidden state, and fp16 KV caches [layers][context][kv]
    holding random history at positions below `position` (zeros above).
    Block scales keep every projection's output near unit variance."""
    hidden, kv = heads * head_dim, kv_heads * head_dim
    head_type = ggml_type if head_type is None else head_type
    code_std = {0: 1.0, 2: 4.6, 8: 74.0}

    def tensor(tag, t, rows, cols):
        return ggml_tensor(seed, tag, t, rows, cols, scale=1.0 / (code_std[t] * np.sqrt(cols)))

    parts, offsets, cursor = [], {n: [] for n in ("q", "k", "v", "output", "gate", "up", "down")}, 0

    def place(data):
        nonlocal cursor
        pad = (-cursor) % 32 + misalign
        parts.append(np.zeros(pad, np.uint8))
        cursor += pad
        off = cursor
        parts.append(data)
        cursor += data.size
        return off

    shapes = {"q": (hidden, hidden), "k": (kv, hidden), "v": (kv, hidden), "output": (hidden, hidden),
              "gate": (ffn, hidden), "up": (ffn, hidden), "down": (hidden, ffn)}
    for l in range(layers):
        for n, (rows, cols) in shapes.items():
            offsets[n].append(place(tensor(f"w{n}{l}", ggml_type, rows, cols)))
    head_off = place(tensor("head", head_type, vocab, hidden))
    parts.append(np.zeros(64, np.uint8))
    kc = np.zeros((layers, context_tokens, kv), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :position] = to_f16_bits(normal(seed, "kh", (layers, position, kv)))
    vc[:, :position] = to_f16_bits(normal(seed, "vh", (layers, position, kv)))
    return {
        "mapping": np.concatenate(parts), "offsets": offsets, "head": (head_off, head_type),
        "attn_norm": normal(seed, "an", (layers, hidden), 0.1) + 1.0,
        "ffn_norm": normal(seed, "fn", (layers, hidden), 0.1) + 1.0,
        "output_norm": normal(seed, "on", (hidden,), 0.1) + 1.0,
        "q_bias": normal(seed, "qb", (layers, hidden), 0.1), "k_bias": normal(seed, "kb", (layers, kv), 0.1),
        "v_bias": normal(seed, "vb", (layers, kv), 0.1), "hidden_in": normal(seed, "x", (hidden,)),
        "key_cache": kc, "value_cache": vc, "hidden": hidden, "kv": kv,
    }

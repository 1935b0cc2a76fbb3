"""GGUF files for the tests, written at test time (no network, no model
downloads), the way the reference's C tests write theirs (c/tests/kernel_ops.c:
163-215).

`GGUFWriter` emits GGUF v2/v3: header, metadata (any value type, arrays
included), the tensor table and the data section at the file's alignment.
`kernel_ops_fixture` writes the reference test's own file byte for byte;
`qwen2_model` writes a small random Qwen2 model with a byte-level BPE
vocabulary, for generation tests.
"""
from __future__ import annotations

import struct

import numpy as np

import _synth as S

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, value) -> bytes:
    if vtype == STR:
        return _str(value)
    if vtype == ARR:
        etype, items = value
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, v) for v in items)
    return struct.pack(_FMT[vtype], value)


class GGUFWriter:
    def __init__(self, version: int = 3, alignment: int = 32):
        self.version = version
        self.alignment = alignment
        self.kvs: list[bytes] = []
        self.tensors: list[tuple] = []
        self.blobs: list[tuple[int, bytes]] = []
        self.cursor = 0

    def kv(self, key, vtype: int, value) -> "GGUFWriter":
        self.kvs.append(_str(key) + struct.pack("<I", vtype) + _value(vtype, value))
        return self

    def raw_kv(self, data: bytes) -> "GGUFWriter":
        self.kvs.append(data)
        return self

    def tensor(self, name, dims, ggml_type: int, data=b"", offset: int | None = None,
               align: int | None = None) -> int:
        """Adds a tensor; `offset` (relative to the data section) defaults to the
        next multiple of `align` (the file alignment) after the previous data."""
        a = self.alignment if align is None else align
        if offset is None:
            offset = (self.cursor + a - 1) // a * a
        self.tensors.append((name, tuple(dims), ggml_type, offset))
        data = data.tobytes() if isinstance(data, np.ndarray) else bytes(data)
        if data:
            self.blobs.append((offset, bytes(data)))
            self.cursor = max(self.cursor, offset + len(data))
        return offset

    def header(self) -> bytes:
        out = [struct.pack("<IIQQ", 0x46554747, self.version, len(self.tensors), len(self.kvs))]
        out += self.kvs
        for name, dims, t, off in self.tensors:
            out.append(_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
                       + struct.pack("<IQ", t, off))
        return b"".join(out)

    def tobytes(self) -> bytes:
        head = self.header()
        pad = (-len(head)) % self.alignment
        data = bytearray(self.cursor)
        for off, blob in self.blobs:
            data[off:off + len(blob)] = blob
        return head + b"\0" * pad + bytes(data)

    def write(self, path) -> str:
        with open(path, "wb") as f:
            f.write(self.tobytes())
        return str(path)


# ---- the reference test's file (kernel_ops.c:163-215) -------------------------

def _q4_row(scale_bits: int, kind: int) -> bytes:
    codes = bytes((i | ((15 - i) << 4)) if kind == 0 else 0x88 for i in range(16))
    return struct.pack("<H", scale_bits) + codes


def _q8_row(scale_bits: int, kind: int) -> bytes:
    return struct.pack("<H", scale_bits) + bytes(((i - 16) & 0xFF) if kind == 0 else 1 for i in range(32))


def kernel_ops_fixture(path) -> str:
    """The GGUF the reference's kernel_ops.c writes: a 32-wide qwen2 stub, a
    three-token tokenizer ("a", "b", "ab", merge "a b"), Q4_0 token_embd at
    data offset 0, Q8_0 output.weight at 54 (2-byte aligned) and the F32
    output_norm at 156."""
    w = GGUFWriter(3, 32)
    w.kv("general.name", STR, "tiny-c-kernel-test").kv("general.architecture", STR, "qwen2")
    w.kv("qwen2.embedding_length", U32, 32).kv("qwen2.block_count", U32, 1)
    w.kv("qwen2.feed_forward_length", U32, 64).kv("qwen2.attention.head_count", U32, 1)
    w.kv("qwen2.attention.head_count_kv", U32, 1).kv("qwen2.attention.layer_norm_rms_epsilon", F32, 1e-6)
    w.kv("tokenizer.ggml.model", STR, "gpt2").kv("tokenizer.ggml.pre", STR, "qwen2")
    w.kv("tokenizer.ggml.tokens", ARR, (STR, ["a", "b", "ab"]))
    w.kv("tokenizer.ggml.token_type", ARR, (I32, [1, 1, 1]))
    w.kv("tokenizer.ggml.merges", ARR, (STR, ["a b"]))
    w.kv("tokenizer.ggml.bos_token_id", U32, 0).kv("tokenizer.ggml.eos_token_id", U32, 1)
    w.kv("tokenizer.ggml.padding_token_id", U32, 0).kv("tokenizer.ggml.add_bos_token", BOOL, 0)
    q4 = _q4_row(0x3C00, 0) + _q4_row(0x3800, 1) + _q4_row(0x3800, 1)
    q8 = _q8_row(0x3400, 0) + _q8_row(0x3C00, 1) + _q8_row(0x3C00, 1)
    norm = np.array([1.0 + i / 32.0 for i in range(32)], np.float32).tobytes()
    w.tensor("token_embd.weight", (32, 3), 2, q4, offset=0)
    w.tensor("output.weight", (32, 3), 8, q8, offset=54)
    w.tensor("output_norm.weight", (32,), 0, norm, offset=156)
    return w.write(path)


# ---- a small random Qwen2 model -------------------------------------------------

def gpt2_byte_symbols() -> list[str]:
    """The 256 byte symbols of byte-level BPE, in byte order: printable bytes
    stand for themselves, the others map to U+0100 onwards."""
    keep = [b for b in range(256) if 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255]
    out, extra = [], 0
    for b in range(256):
        if b in keep:
            out.append(chr(b))
        else:
            out.append(chr(256 + extra))
            extra += 1
    return out


SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]


def bpe_vocab(seed: int, n_merges: int) -> tuple[list[str], list[str]]:
    """A byte-level vocabulary (256 byte symbols), `n_merges` merges learned
    greedily from a random English-like corpus, and their merged tokens."""
    syms = gpt2_byte_symbols()
    r = S.rng(seed, "corpus")
    words = ["the", "hello", "world", "token", "engine", "model", "qwen", "attention", "cache", "gpu", " a", " is",
             "ing", "tion", "er", " th", "\n", "  ", "{\"", "\":", "json", "def ", "return"]
    corpus = "".join(words[i] for i in r.integers(0, len(words), 4000))
    seq = [syms[b] for b in corpus.encode()]
    merges, tokens = [], []
    for _ in range(n_merges):
        counts: dict[tuple[str, str], int] = {}
        for a, b in zip(seq, seq[1:]):
            counts[(a, b)] = counts.get((a, b), 0) + 1
        if not counts:
            break
        (a, b), _n = max(counts.items(), key=lambda kv: (kv[1], kv[0]))
        merges.append(f"{a} {b}")
        tokens.append(a + b)
        out, i = [], 0
        while i < len(seq):
            if i + 1 < len(seq) and seq[i] == a and seq[i + 1] == b:
                out.append(a + b)
                i += 2
            else:
                out.append(seq[i])
                i += 1
        seq = out
    return syms + tokens, merges


def qwen2_model(path, seed: int = 5, ggml_type: int = 2, layers: int = 2, heads: int = 4, kv_heads: int = 2,
                head_dim: int = 64, ffn: int = 256, n_merges: int = 60, head_type: int | None = None,
                tied_head: bool = False, embd_type: int | None = None, alignment: int = 32) -> dict:
    """A random Qwen2 GGUF: `layers` blocks of Q4_0 / Q8_0 projections with F32
    norms and biases, a byte-level BPE tokenizer (256 byte symbols, merges,
    then the three chat specials; eos = <|im_end|>, padding = <|endoftext|>),
    token_embd and (unless tied) output.weight.  Returns the path and the
    arrays the oracle needs."""
    hidden, kv = heads * head_dim, kv_heads * head_dim
    tokens, merges = bpe_vocab(seed, n_merges)
    tokens = tokens + SPECIALS
    vocab = len(tokens)
    types = [1] * (vocab - len(SPECIALS)) + [3] * len(SPECIALS)
    head_type = ggml_type if head_type is None else head_type
    embd_type = ggml_type if embd_type is None else embd_type
    code_std = {0: 1.0, 2: 4.6, 8: 74.0}

    def weights(tag, t, rows, cols):
        return S.ggml_tensor(seed, tag, t, rows, cols, scale=1.0 / (code_std[t] * np.sqrt(cols)))

    w = GGUFWriter(3, alignment)
    w.kv("general.name", STR, "synthetic-qwen2").kv("general.architecture", STR, "qwen2")
    if alignment != 32:
        w.kv("general.alignment", U32, alignment)
    w.kv("qwen2.context_length", U32, 4096).kv("qwen2.embedding_length", U32, hidden)
    w.kv("qwen2.block_count", U32, layers).kv("qwen2.feed_forward_length", U32, ffn)
    w.kv("qwen2.attention.head_count", U32, heads).kv("qwen2.attention.head_count_kv", U32, kv_heads)
    w.kv("qwen2.attention.layer_norm_rms_epsilon", F32, 1e-6).kv("qwen2.rope.freq_base", F32, 1e6)
    w.kv("tokenizer.ggml.model", STR, "gpt2").kv("tokenizer.ggml.pre", STR, "qwen2")
    w.kv("tokenizer.ggml.tokens", ARR, (STR, tokens)).kv("tokenizer.ggml.token_type", ARR, (I32, types))
    w.kv("tokenizer.ggml.merges", ARR, (STR, merges))
    w.kv("tokenizer.ggml.eos_token_id", U32, vocab - 1).kv("tokenizer.ggml.padding_token_id", U32, vocab - 3)
    w.kv("tokenizer.ggml.bos_token_id", U32, vocab - 3).kv("tokenizer.ggml.add_bos_token", BOOL, 0)
    arrays = {"attn_norm": [], "ffn_norm": [], "q_bias": [], "k_bias": [], "v_bias": []}
    shapes = {"attn_q": (hidden, hidden), "attn_k": (kv, hidden), "attn_v": (kv, hidden),
              "attn_output": (hidden, hidden), "ffn_gate": (ffn, hidden), "ffn_up": (ffn, hidden),
              "ffn_down": (hidden, ffn)}
    offsets = {n: [] for n in ("q", "k", "v", "output", "gate", "up", "down")}
    short = dict(zip(shapes, offsets))
    data_start = None
    for l in range(layers):
        for n, (rows, cols) in shapes.items():
            off = w.tensor(f"blk.{l}.{n}.weight", (cols, rows), ggml_type, weights(f"{n}{l}", ggml_type, rows, cols))
            offsets[short[n]].append(off)
        f32 = {"attn_norm": S.normal(seed, f"an{l}", (hidden,), 0.1) + 1.0,
               "ffn_norm": S.normal(seed, f"fn{l}", (hidden,), 0.1) + 1.0,
               "q_bias": S.normal(seed, f"qb{l}", (hidden,), 0.1), "k_bias": S.normal(seed, f"kb{l}", (kv,), 0.1),
               "v_bias": S.normal(seed, f"vb{l}", (kv,), 0.1)}
        names = {"attn_norm": "attn_norm.weight", "ffn_norm": "ffn_norm.weight", "q_bias": "attn_q.bias",
                 "k_bias": "attn_k.bias", "v_bias": "attn_v.bias"}
        for k, a in f32.items():
            w.tensor(f"blk.{l}.{names[k]}", a.shape, 0, a.astype(np.float32).tobytes())
            arrays[k].append(a)
    out_norm = S.normal(seed, "on", (hidden,), 0.1) + 1.0
    w.tensor("output_norm.weight", (hidden,), 0, out_norm.astype(np.float32).tobytes())
    embd_off = w.tensor("token_embd.weight", (hidden, vocab), embd_type,
                        S.ggml_tensor(seed, "embd", embd_type, vocab, hidden, scale=1.0 / code_std[embd_type]))
    head = (embd_off, embd_type)
    if not tied_head:
        head = (w.tensor("output.weight", (hidden, vocab), head_type, weights("head", head_type, vocab, hidden)),
                head_type)
    w.write(path)
    data_start = len(w.header()) + (-len(w.header())) % alignment
    blob = np.fromfile(path, dtype=np.uint8)[data_start:]
    return {"path": str(path), "tokens": tokens, "merges": merges, "types": types, "vocab": vocab,
            "hidden": hidden, "kv": kv, "heads": heads, "kv_heads": kv_heads, "head_dim": head_dim, "ffn": ffn,
            "layers": layers, "ggml_type": ggml_type, "data": blob, "offsets": offsets, "head": head,
            "embd": (embd_off, embd_type), "output_norm": out_norm.astype(np.float32),
            **{k: np.stack(v).astype(np.float32) for k, v in arrays.items()}}

"""TEST INFRASTRUCTURE ONLY: CPU restatement of the reference's tokenizer,
chat template, sampler and generation loop, the checker for te_model.hip.
Only tests/ import it.

- tokenize / detokenize: c/src/tokenizer.c:84-205 (byte-level BPE over the
  GPT-2 byte alphabet :387-417, the lowest-rank leftmost merge :645-700,
  special tokens longest-first at '<' :615-643); the special-token rule of the
  loader, gguf.c:593-596.
- chat_prompt: tokenizer.c:52-82.
- xorshift_uniform / sample: c/src/qwen.c:1170-1250 (xorshift64*, top-k
  with the reference's replacement order, temperature softmax in fp64,
  `r <= acc` choice).  xorshift_uniform is pinned to the reference's own
  te_qwen_rng_uniform, evaluated statement by statement from its source text
  (tests/test_model_cpu.py::test_rng_matches_reference_source); sample is
  pinned by what fixes it (top-k 1 and a vanishing temperature are argmax,
  the candidates are the k largest logits, draw frequencies follow the
  tempered softmax); the temperature is a float32, as the reference holds it.
- generate: c/src/qwen.c:261-400 (prompt, then tokens until eos / padding /
  max_tokens), each token through oracle.decode_all_layers (qwen.c:907-1087)
  on an fp16 KV cache.

RefTokenizer wraps the reference's own gguf.c loader and tokenizer.c
(oracle/_ref, built where the reference tree is present) for checking this
restatement and the product's tokenizer on the same GGUF file.
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np

from . import HERE

REF_TOK_LIB = HERE / "_ref" / "libte_ref_tok.so"


def byte_symbols() -> list[str]:
    """GPT-2 byte alphabet (tokenizer.c:387-417): bytes 33-126, 161-172 and
    174-255 are themselves; the other 68 bytes map to U+0100.. in byte order."""
    out, extra = [], 0
    for b in range(256):
        if 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255:
            out.append(chr(b))
        else:
            out.append(chr(256 + extra))
            extra += 1
    return out


_SYM = byte_symbols()
_BYTE = {ord(s): b for b, s in enumerate(_SYM)}


class Tokenizer:
    """The tokenizer state of a model: token texts (str), types, merges."""

    def __init__(self, tokens: list[str], types: list[int] | None, merges: list[str]):
        self.tokens = [t.encode() for t in tokens]
        self.types = list(types) if types is not None else [0] * len(tokens)
        self.special = [ty != 1 or t.startswith(b"<|") for t, ty in zip(self.tokens, self.types)]
        self.to_id = {}
        for i, t in enumerate(self.tokens):
            self.to_id[t] = i  # last wins
        self.rank = {}
        for i, m in enumerate(merges):
            self.rank[m.encode()] = i

    def _special_at(self, text: bytes, pos: int):
        if text[pos:pos + 1] != b"<":
            return None
        best = None
        for i, t in enumerate(self.tokens):
            if self.special[i] and t and (best is None or len(t) > len(self.tokens[best])) and text.startswith(t, pos):
                best = i
        return best

    def _bpe(self, seg: bytes) -> list[int]:
        syms = [_SYM[b].encode() for b in seg]
        while len(syms) > 1:
            best, at = None, 0
            for i in range(len(syms) - 1):
                r = self.rank.get(syms[i] + b" " + syms[i + 1])
                if r is not None and (best is None or r < best):
                    best, at = r, i
            if best is None:
                break
            syms[at:at + 2] = [syms[at] + syms[at + 1]]
        out = []
        for s in syms:
            if s not in self.to_id:
                raise KeyError(s)
            out.append(self.to_id[s])
        return out

    def tokenize(self, text: bytes, parse_special: bool = True) -> list[int]:
        text = text.split(b"\0", 1)[0]
        out, pos, n = [], 0, len(text)
        while pos < n:
            if parse_special:
                sid = self._special_at(text, pos)
                if sid is not None:
                    out.append(sid)
                    pos += len(self.tokens[sid])
                    continue
            end = n
            if parse_special:
                for scan in range(pos + 1, n):
                    if self._special_at(text, scan) is not None:
                        end = scan
                        break
            out += self._bpe(text[pos:end])
            pos = end
        return out

    def detokenize(self, ids, skip_special: bool = True) -> bytes:
        out = bytearray()
        for i in ids:
            if skip_special and self.special[i]:
                continue
            for ch in self.tokens[i].decode("utf-8", errors="surrogatepass"):
                cp = ord(ch)
                if cp in _BYTE:
                    out.append(_BYTE[cp])
                else:
                    out += ch.encode("utf-8", errors="surrogatepass")
        return bytes(out)


def chat_prompt(prompt: str) -> str:
    return "<|im_start|>user\n" + prompt + "<|im_end|>\n<|im_start|>assistant\n"


_MASK = (1 << 64) - 1


def xorshift_uniform(state: int) -> tuple[float, int]:
    """xorshift64* (qwen.c:1170-1178): the next state and (x * M) >> 11 / 2^53."""
    x = state
    x ^= x >> 12
    x ^= (x << 25) & _MASK
    x ^= x >> 27
    r = (x * 0x2545F4914F6CDD1D) & _MASK
    return (r >> 11) / 9007199254740992.0, x


def top_k(logits: np.ndarray, k: int) -> tuple[list[float], list[int]]:
    """The candidate list in the reference's order (qwen.c:1198-1225): the
    first k logits, then each larger one replacing the current minimum (the
    first minimum on a tie)."""
    vals, idx = [], []
    min_pos = 0
    for i, v in enumerate(logits.tolist()):
        if len(vals) < k:
            vals.append(v)
            idx.append(i)
            if len(vals) == k:
                min_pos = min(range(k), key=lambda j: (vals[j], j))
        elif v > vals[min_pos]:
            vals[min_pos] = v
            idx[min_pos] = i
            min_pos = min(range(k), key=lambda j: (vals[j], j))
    return vals, idx


def sample(logits: np.ndarray, temperature: float, k: int, state: int) -> tuple[int, int, dict]:
    """Top-k temperature sampling (qwen.c:1182-1250).  Returns the token, the
    next RNG state and the draw (probabilities in candidate order, r) so that
    a test can see how close the draw came to a boundary."""
    k = 1 if k == 0 else min(k, 1024, logits.size)
    vals, idx = top_k(np.asarray(logits, np.float32), k)
    mx = max(vals)
    # the reference holds the temperature as a float (qwen.c:42) and widens
    # it after a float comparison (qwen.c:1229)
    t32 = np.float32(temperature)
    t = float(t32) if t32 > np.float32(1e-6) else 1e-6
    p = [math.exp((float(v) - float(mx)) / t) for v in vals]
    s = 0.0
    for e in p:
        s += e
    u, state = xorshift_uniform(state)
    r = u * s
    cum, acc = [], 0.0
    for e in p:
        acc += e
        cum.append(acc)
    choice = next((j for j, c in enumerate(cum) if r <= c), len(p) - 1)
    return idx[choice], state, {"probs": p, "cum": cum, "r": r, "idx": idx}


def generate(model: dict, prompt_ids: list[int], max_tokens: int, *, eos: int, pad: int, context_tokens: int,
             temperature: float = 0.0, top_k_n: int = 40, seed: int = 0x9E3779B97F4A7C15, forced=None,
             rope_theta: float = 1e6, epsilon: float = 1e-6):
    """The reference generation loop on the oracle's decode composition.

    `model` is the dict of tests/_gguf.qwen2_model.  With `forced` (token ids
    produced by the implementation under test) each step's logits are taken
    after feeding the forced tokens (teacher forcing), so the caller can
    check every step's choice against that step's logits.  Returns (tokens the
    oracle chose, per-step logits, per-step draws)."""
    from . import decode_all_layers, dequantize_rows, rope_table
    L, H, KV, d = model["layers"], model["heads"], model["kv_heads"], model["head_dim"]
    hidden, kv, ffn, vocab = model["hidden"], model["kv"], model["ffn"], model["vocab"]
    data = model["data"]
    embd_off, embd_type = model["embd"]
    from . import ggml_row_bytes
    erow = ggml_row_bytes(embd_type, hidden)
    cos, sin = rope_table(context_tokens, d, rope_theta)
    kc = np.zeros((L, context_tokens, kv), np.uint16)
    vc = np.zeros_like(kc)

    def step(tok, pos):
        x = dequantize_rows(data[embd_off + tok * erow: embd_off + (tok + 1) * erow], embd_type, hidden, 1)[0]
        h, t, logits = decode_all_layers(data, model["offsets"], L, model["ggml_type"], x, model["attn_norm"],
                                         model["ffn_norm"], model["q_bias"], model["k_bias"], model["v_bias"], cos,
                                         sin, kc, vc, pos, context_tokens, hidden, kv, H, KV, d, ffn, epsilon,
                                         head=model["head"], output_norm=model["output_norm"], vocab=vocab)
        return logits

    logits = None
    for i, tok in enumerate(prompt_ids):
        logits = step(tok, i)
    chosen, all_logits, draws = [], [], []
    state = seed
    pos = len(prompt_ids)
    for g in range(max_tokens):
        all_logits.append(logits)
        if temperature > 0.0:
            nxt, state, draw = sample(logits, temperature, top_k_n, state)
        else:
            nxt, draw = int(np.argmax(logits)), None
        draws.append(draw)
        chosen.append(nxt)
        use = forced[g] if forced is not None and g < len(forced) else nxt
        if use in (eos, pad) or g + 1 == max_tokens:
            break
        logits = step(use, pos)
        pos += 1
    return chosen, all_logits, draws


class RefTokenizer:
    """The reference's tokenizer.c over a GGUF file loaded by the reference's
    gguf.c (te_model_parse_gguf).  The library keeps gguf.c's one reference to
    the Metal backend unresolved, so it is loaded with lazy binding; a model is
    never released (gguf.c's release path is that reference)."""

    def __init__(self, path):
        lib = ctypes.CDLL(str(REF_TOK_LIB), mode=os.RTLD_LAZY | os.RTLD_LOCAL)
        lib.ref_tok_load.restype = ctypes.c_void_p
        lib.ref_tok_load.argtypes = [ctypes.c_char_p]
        lib.te_model_tokenize.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int,
                                          ctypes.POINTER(ctypes.c_uint32), ctypes.c_size_t,
                                          ctypes.POINTER(ctypes.c_size_t)]
        lib.te_model_detokenize.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32), ctypes.c_size_t,
                                            ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t,
                                            ctypes.POINTER(ctypes.c_size_t)]
        self._lib = lib
        self._h = lib.ref_tok_load(str(path).encode())
        assert self._h, f"the reference's gguf.c rejected {path}"

    def tokenize(self, text: bytes, parse_special: bool = True):
        cap = len(text) + 16
        out = (ctypes.c_uint32 * cap)()
        n = ctypes.c_size_t()
        st = self._lib.te_model_tokenize(self._h, text, int(parse_special), out, cap, ctypes.byref(n))
        return st, list(out[:n.value]) if st == 0 else None

    def detokenize(self, ids, skip_special: bool = True):
        arr = (ctypes.c_uint32 * max(len(ids), 1))(*ids)
        cap = 16 * len(ids) + 16
        buf = ctypes.create_string_buffer(cap)
        n = ctypes.c_size_t()
        st = self._lib.te_model_detokenize(self._h, arr, len(ids), int(skip_special), buf, cap, ctypes.byref(n))
        return st, buf.raw[:n.value] if st == 0 else None


def ref_tokenizer_available() -> bool:
    return REF_TOK_LIB.is_file()

"""GGUF loading, model / tensor / tokenizer info and the tokenizer of
libtinyengine.so (te_model.hip), on the CPU: none of these calls touch the
GPU.

- The reference's own test file and expectations (c/tests/kernel_ops.c:163-215,
  :256-290): info fields, tokenize("ab") -> [2], detokenize, the F32 read.
- Loader statuses as the reference's parser returns them (c/src/gguf.c:
  221-369, tinyengine.c:270-305).
- Tokenizer parity on random text: this build against the oracle's
  restatement (oracle/text.py), the reference's own tokenizer.c (oracle/_ref,
  where it was built) and an independent byte-level BPE (the `tokenizers`
  library with no pre-tokenizer split, which is what the reference does).
- The sampler restatement against what fixes it: top_k 1 and a vanishing
  temperature are argmax, the candidates are the k largest logits, and the
  empirical draw frequencies follow the tempered softmax.
"""
import os
import random
import struct

import numpy as np
import pytest

import _gguf as G
from oracle import text as OT
from tinymetalagent_amd import runtime as R
from tinymetalagent_amd.model import Model, RuntimeOptions, format_qwen_chat_prompt


@pytest.fixture(scope="module")
def fixture_model(tmp_path_factory):
    path = G.kernel_ops_fixture(tmp_path_factory.mktemp("gguf") / "kernel-test.gguf")
    with Model(path) as m:
        yield m


@pytest.fixture(scope="module")
def qwen_file(tmp_path_factory):
    return G.qwen2_model(tmp_path_factory.mktemp("gguf") / "qwen.gguf", seed=5, n_merges=80)


def test_kernel_ops_fixture_info(fixture_model):
    m = fixture_model
    info = m.info()
    assert info.embedding_length == 32 and info.vocab_size == 3
    assert info.architecture == "qwen2" and info.name == "tiny-c-kernel-test"
    assert info.gguf_version == 3 and info.metadata_kv_count == 17 and info.tensor_count == 3
    assert info.head_dim == 32 and info.block_count == 1 and info.feed_forward_length == 64
    assert info.rope_freq_base == 1e6  # the qwen2 default (gguf.c:427-430)
    assert info.parameter_count == 32 * 3 * 2 + 32
    assert info.tensor_data_bytes == 54 + 102 + 128
    assert info.tensor_data_offset % 32 == 0
    assert info.quant_tensor_counts[1] == 1 and info.quant_tensor_counts[4] == 1 and info.quant_tensor_counts[8] == 1
    tok = m.tokenizer_info()
    assert (tok.model, tok.pre) == ("gpt2", "qwen2")
    assert (tok.token_count, tok.token_type_count, tok.merge_count) == (3, 3, 1)
    assert (tok.eos_token_id, tok.padding_token_id, tok.add_bos_token) == (1, 0, False)
    t = m.tensor_info("token_embd.weight")
    assert t.dims == (32, 3) and t.ggml_type == 2 and t.bytes == 54 and t.relative_offset == 0
    o = m.tensor_info("output.weight")
    assert o.relative_offset == 54 and o.absolute_offset == info.tensor_data_offset + 54 and o.quant == 8


def test_kernel_ops_fixture_tokenizer_and_f32(fixture_model):
    m = fixture_model
    assert m.tokenize("ab") == [2]
    assert m.detokenize([2]) == "ab"
    norm = m.read_f32_tensor("output_norm.weight")
    assert len(norm) == 32 and norm[0] == 1.0 and norm[31] == 1.96875


def test_chat_prompt_format():
    assert format_qwen_chat_prompt("hi") == OT.chat_prompt("hi")
    lib = R.load_library()
    import ctypes
    n = ctypes.c_size_t()
    buf = ctypes.create_string_buffer(64)
    req = len(OT.chat_prompt("hi").encode())
    assert lib.te_format_qwen_chat_prompt(b"hi", buf, req, ctypes.byref(n)) == 1 and n.value == req  # no room for NUL
    assert lib.te_format_qwen_chat_prompt(b"hi", None, 0, ctypes.byref(n)) == 1 and n.value == req
    assert lib.te_format_qwen_chat_prompt(b"hi", buf, req + 1, ctypes.byref(n)) == 0


def _status(path, options=None):
    import ctypes
    lib = R.load_library()
    h = ctypes.c_void_p()
    opts = (options or RuntimeOptions())._to_c()
    st = lib.te_model_load_gguf(str(path).encode(), ctypes.byref(opts), ctypes.byref(h))
    if st == 0:
        lib.te_model_free(h)
    return st


def _base_writer(**over):
    w = G.GGUFWriter(over.pop("version", 3), over.pop("alignment", 32))
    w.kv("general.architecture", G.STR, over.pop("arch", "qwen2"))
    for k, v in (("embedding_length", 32), ("block_count", 1), ("feed_forward_length", 64),
                 ("attention.head_count", 1)):
        w.kv(f"qwen2.{k}", G.U32, v)
    w.kv("qwen2.attention.layer_norm_rms_epsilon", G.F32, 1e-6)
    w.kv("tokenizer.ggml.tokens", G.ARR, (G.STR, ["a", "b", "ab"]))
    w.tensor("token_embd.weight", (32, 3), 2, bytes(54))
    return w


def test_loader_statuses(tmp_path):
    ok = _base_writer().write(tmp_path / "ok.gguf")
    assert _status(ok) == 0
    assert _status(tmp_path / "missing.gguf") == R.TE_STATUS_IO_ERROR
    raw = open(ok, "rb").read()
    cases = {
        "magic": (b"GGUX" + raw[4:], R.TE_STATUS_UNSUPPORTED),
        "v1": (raw[:4] + struct.pack("<I", 1) + raw[8:], R.TE_STATUS_UNSUPPORTED),
        "v4": (raw[:4] + struct.pack("<I", 4) + raw[8:], R.TE_STATUS_UNSUPPORTED),
        "header": (raw[:20], R.TE_STATUS_RUNTIME_ERROR),
        "metadata": (raw[:60], R.TE_STATUS_RUNTIME_ERROR),
        "count": (raw[:8] + struct.pack("<Q", (1 << 20) + 1) + raw[16:], R.TE_STATUS_UNSUPPORTED),
        "data": (raw[:-10], R.TE_STATUS_RUNTIME_ERROR),  # the tensor runs past the end
    }
    for name, (data, want) in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        assert _status(p) == want, name
    empty = tmp_path / "empty.gguf"
    empty.write_bytes(b"")
    assert _status(empty) == R.TE_STATUS_IO_ERROR
    # options that make no kernel plan (tinyengine.c:290-295)
    import ctypes
    lib = R.load_library()
    opts = RuntimeOptions()._to_c()
    opts.abi_version = 2
    h = ctypes.c_void_p()
    assert lib.te_model_load_gguf(str(ok).encode(), ctypes.byref(opts), ctypes.byref(h)) == R.TE_STATUS_UNSUPPORTED
    assert lib.te_model_load_gguf(None, None, ctypes.byref(h)) == R.TE_STATUS_INVALID_ARGUMENT


def test_loader_metadata_rules(tmp_path):
    def st(w):
        return _status(w.write(tmp_path / "x.gguf"))

    # no architecture -> unsupported; bad alignment -> unsupported; missing sizes -> unsupported
    w = G.GGUFWriter()
    w.kv("qwen2.embedding_length", G.U32, 32)
    assert st(w) == R.TE_STATUS_UNSUPPORTED
    assert st(_base_writer().kv("general.alignment", G.U32, 24)) == R.TE_STATUS_UNSUPPORTED
    assert st(_base_writer().kv("general.alignment", G.U32, 0)) == R.TE_STATUS_UNSUPPORTED
    w = G.GGUFWriter()
    w.kv("general.architecture", G.STR, "qwen2").kv("qwen2.embedding_length", G.U32, 32)
    assert st(w) == R.TE_STATUS_UNSUPPORTED
    # nested arrays are skipped; nesting deeper than 8 and unknown value types are not
    nested = (G.ARR, [(G.U8, [1, 2]), (G.U8, [])])
    assert st(_base_writer().kv("x.nested", G.ARR, nested)) == 0
    deep = (G.U32, [7])
    for _ in range(9):
        deep = (G.ARR, [deep])
    assert st(_base_writer().kv("x.deep", G.ARR, deep)) == R.TE_STATUS_UNSUPPORTED
    assert st(_base_writer().raw_kv(G._str("x.bad") + struct.pack("<I", 13))) == R.TE_STATUS_UNSUPPORTED
    # tokenizer arrays: tokens must be strings, types int32 of the same length
    w = _base_writer()
    w.kvs[-1] = G._str("tokenizer.ggml.tokens") + struct.pack("<I", G.ARR) + G._value(G.ARR, (G.U32, [1, 2, 3]))
    assert st(w) == R.TE_STATUS_UNSUPPORTED
    assert st(_base_writer().kv("tokenizer.ggml.token_type", G.ARR, (G.I32, [1, 1]))) == R.TE_STATUS_UNSUPPORTED
    assert st(_base_writer().kv("tokenizer.ggml.token_type", G.ARR, (G.U32, [1, 1, 1]))) == R.TE_STATUS_UNSUPPORTED
    assert st(_base_writer().kv("tokenizer.ggml.merges", G.ARR, (G.I32, [1]))) == R.TE_STATUS_UNSUPPORTED
    # integer keys read from u32 / u64 / i32 / i64 only; the head count divides the width
    w = _base_writer()
    w.kv("qwen2.attention.head_count_kv", G.I64, 1)
    path = w.write(tmp_path / "i64.gguf")
    with Model(path) as m:
        assert m.info().attention_head_count_kv == 1 and m.info().vocab_size == 3
    w = G.GGUFWriter()
    w.kv("general.architecture", G.STR, "qwen2").kv("qwen2.embedding_length", G.U32, 32)
    w.kv("qwen2.block_count", G.U16, 1)  # u16: not read -> block_count 0 -> unsupported
    w.kv("qwen2.feed_forward_length", G.U32, 64).kv("qwen2.attention.head_count", G.U32, 1)
    w.kv("qwen2.attention.layer_norm_rms_epsilon", G.F32, 1e-6)
    w.tensor("token_embd.weight", (32, 3), 2, bytes(54))
    assert st(w) == R.TE_STATUS_UNSUPPORTED
    assert st(_base_writer().kv("qwen2.attention.head_count", G.U32, 5)) == 0  # first key wins
    w = _base_writer()
    w.kvs = [k for k in w.kvs if b"head_count" not in k]
    w.kv("qwen2.attention.head_count", G.U32, 5)
    assert st(w) == R.TE_STATUS_UNSUPPORTED  # 32 % 5 != 0


def test_model_entry_point_statuses(fixture_model):
    import ctypes
    m, lib = fixture_model, R.load_library()
    h = m.handle
    n = ctypes.c_size_t()
    buf = (ctypes.c_float * 64)()
    with pytest.raises(R.TinyEngineError, match="invalid argument"):
        m.tensor_info("nope")
    assert lib.te_model_read_f32_tensor(h, b"token_embd.weight", buf, 64, ctypes.byref(n)) == 1  # not F32
    assert lib.te_model_read_f32_tensor(h, b"output_norm.weight", buf, 31, ctypes.byref(n)) == 1 and n.value == 32
    assert lib.te_model_read_f32_tensor(h, b"output_norm.weight", buf, 32, None) == 1
    # argument and shape checks come before any GPU use
    assert lib.te_model_dequantize_row_f32(h, b"token_embd.weight", 3, buf, 64, ctypes.byref(n)) == 1
    assert lib.te_model_dequantize_row_f32(h, b"output_norm.weight", 0, buf, 64, ctypes.byref(n)) == 3  # rank 1
    assert lib.te_model_dequantize_row_f32(h, b"token_embd.weight", 0, buf, 31, ctypes.byref(n)) == 1
    assert n.value == 32
    assert lib.te_model_matvec_f32(h, b"output.weight", buf, 31, buf, 3, ctypes.byref(n)) == 1
    assert lib.te_model_matvec_f32(h, b"output.weight", buf, 32, buf, 2, ctypes.byref(n)) == 1 and n.value == 3
    assert lib.te_model_matvec_f32(h, b"nope", buf, 32, buf, 3, ctypes.byref(n)) == 1
    assert lib.te_model_matvec_f32(h, b"output_norm.weight", buf, 32, buf, 3, ctypes.byref(n)) == 3
    ids = (ctypes.c_uint32 * 2)(2, 7)
    out = ctypes.create_string_buffer(16)
    assert lib.te_model_detokenize(h, ids, 2, 1, out, 16, ctypes.byref(n)) == 1  # id 7 out of range
    assert lib.te_model_detokenize(h, ids, 1, 1, out, 2, ctypes.byref(n)) == 1 and n.value == 2  # no room for NUL
    toks = (ctypes.c_uint32 * 1)()
    assert lib.te_model_tokenize(h, b"abab", 1, toks, 1, ctypes.byref(n)) == 1 and n.value == 2
    assert lib.te_model_tokenize(h, b"c", 1, toks, 1, ctypes.byref(n)) == R.TE_STATUS_RUNTIME_ERROR  # no token


def _texts(seed, n, specials=True):
    r = random.Random(seed)
    pieces = ["the", "hel", "lo", " wor", "ld", "tion", "é", "中", "\n", " ", "{", "\"", "ing", "x", "q", "  ",
              "attention", "🙂", "\t", "json", "def "]
    if specials:
        pieces += ["<|im_start|>", "<|im_end|>", "<|endoftext|>", "<|im_", "<", "<|"]
    out = []
    for _ in range(n):
        s = "".join(r.choice(pieces) for _ in range(r.randint(0, 24)))
        out.append(s.encode())
    for _ in range(n // 4):  # raw bytes, not UTF-8
        out.append(bytes(r.randint(1, 255) for _ in range(r.randint(1, 16))))
    return out


def test_tokenizer_parity_random_text(qwen_file):
    q = qwen_file
    orc = OT.Tokenizer(q["tokens"], q["types"], q["merges"])
    ref = OT.RefTokenizer(q["path"]) if OT.ref_tokenizer_available() else None
    with Model(q["path"]) as m:
        for text in _texts(11, 200):
            for special in (True, False):
                got = m.tokenize(text, special)
                assert got == orc.tokenize(text, special), text
                if ref is not None:
                    st, want = ref.tokenize(text, special)
                    assert st == 0 and got == want, text
                for skip in (True, False):
                    back = m.detokenize_bytes(got, skip)
                    assert back == orc.detokenize(got, skip)
                    if ref is not None:
                        assert ref.detokenize(got, skip) == (0, back)
                if not special or b"<|" not in text:
                    assert m.detokenize_bytes(got, False) == text  # every byte has a token: exact round trip


def test_oracle_bpe_matches_independent_bpe(qwen_file):
    """The oracle's merge loop against HuggingFace `tokenizers` byte-level BPE
    (no regex pre-split, no added prefix space) on the same vocabulary."""
    tokenizers = pytest.importorskip("tokenizers")
    q = qwen_file
    vocab = {t: i for i, t in enumerate(q["tokens"][:-3])}
    tk = tokenizers.Tokenizer(tokenizers.models.BPE(vocab=vocab, merges=[tuple(m.split(" ")) for m in q["merges"]]))
    tk.pre_tokenizer = tokenizers.pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)
    orc = OT.Tokenizer(q["tokens"], q["types"], q["merges"])
    for text in _texts(12, 300, specials=False):
        s = text.decode("utf-8", errors="ignore")
        if s:
            assert tk.encode(s).ids == orc.tokenize(s.encode(), False), s


def test_tokenizer_duplicates_and_specials(tmp_path):
    """Repeated token texts and merges keep their last id / rank (tokenizer.c:
    294-318); special tokens match longest-first, only at '<'."""
    syms = OT.byte_symbols()
    tokens = syms + ["ab", "ab", "<|a|>", "<|a|>x", "<|b"]
    types = [1] * (len(syms) + 2) + [3, 3, 1]
    merges = ["a b", "x y", "a b"]
    w = _base_writer()
    w.kvs = [k for k in w.kvs if b"tokenizer" not in k]
    w.kv("tokenizer.ggml.tokens", G.ARR, (G.STR, tokens)).kv("tokenizer.ggml.token_type", G.ARR, (G.I32, types))
    w.kv("tokenizer.ggml.merges", G.ARR, (G.STR, merges))
    path = w.write(tmp_path / "dup.gguf")
    orc = OT.Tokenizer(tokens, types, merges)
    ref = OT.RefTokenizer(path) if OT.ref_tokenizer_available() else None
    with Model(path) as m:
        assert m.tokenize("ab") == [257] == orc.tokenize(b"ab")
        assert m.tokenize("<|a|>xab<|b") == orc.tokenize(b"<|a|>xab<|b")
        assert m.tokenize("<|a|>xab<|b")[0] == 259  # the longer special
        assert m.tokenize("<|a|>x", False) == orc.tokenize(b"<|a|>x", False)
        assert m.detokenize([259, 257]) == "ab"  # specials skipped ("<|b" is special by its prefix)
        if ref is not None:  # the reference's loader and tokenizer on the same file
            for text, special in ((b"ab", True), (b"<|a|>xab<|b", True), (b"<|a|>x", False)):
                assert ref.tokenize(text, special) == (0, m.tokenize(text, special))
            assert ref.detokenize([259, 257], True) == (0, b"ab")


def test_sampler_restatement_pins():
    r = np.random.default_rng(3)
    for trial in range(20):
        logits = r.standard_normal(500).astype(np.float32) * 3
        logits[r.integers(0, 500, 5)] = logits.max()  # ties at the top
        vals, idx = OT.top_k(logits, 40)
        assert sorted(idx) == sorted(np.argsort(-logits, kind="stable")[:40].tolist()) or \
            sorted(vals) == sorted(np.sort(logits)[-40:].tolist())
        tok, _, _ = OT.sample(logits, 0.7, 1, 12345 + trial)
        assert tok == int(np.argmax(logits))  # top_k 1: the first maximum
        tok, _, _ = OT.sample(logits, 1e-9, 40, 999 + trial)
        assert logits[tok] == logits.max()
    # draw frequencies follow softmax(top-k / T)
    logits = np.array([2.0, 1.0, 0.5, 0.0, -1.0, -5.0], np.float32)
    state, counts = 0x9E3779B97F4A7C15, np.zeros(6)
    for _ in range(20000):
        tok, state, _ = OT.sample(logits, 0.8, 4, state)
        counts[tok] += 1
    p = np.exp((logits[:4] - logits.max()) / 0.8)
    p /= p.sum()
    assert counts[4:].sum() == 0
    assert np.all(np.abs(counts[:4] / 20000 - p) < 0.015)
    # the generator's draws are uniform on [0, 1)
    u, state = [], 1
    for _ in range(20000):
        v, state = OT.xorshift_uniform(state)
        u.append(v)
    u = np.array(u)
    assert 0.0 <= u.min() and u.max() < 1.0 and abs(u.mean() - 0.5) < 0.01 and abs(u.var() - 1 / 12) < 0.003


def test_loader_survives_corrupted_files(tmp_path, qwen_file):
    """Truncations, byte flips and oversized counts / lengths anywhere in the
    header and metadata: every load returns a status (OK or an error), never
    crashes; a model that loads still tokenizes and reports info."""
    import ctypes
    lib = R.load_library()
    good = open(G.kernel_ops_fixture(tmp_path / "k.gguf"), "rb").read()
    big = open(qwen_file["path"], "rb").read()[:200000]
    r = random.Random(9)
    opts = RuntimeOptions()._to_c()
    seen = set()
    for trial in range(600):
        src = good if trial % 2 == 0 else big
        data = bytearray(src)
        kind = trial % 4
        if kind == 0:
            data = data[:r.randint(0, len(data))]
        elif kind == 1:
            for _ in range(r.randint(1, 8)):
                data[r.randrange(0, min(len(data), 4096))] = r.randrange(256)
        elif kind == 2:  # a huge u64 (count / length / dimension / offset) somewhere in the header
            at = r.randrange(8, min(len(data), 4096) - 8)
            data[at:at + 8] = struct.pack("<Q", r.choice([2 ** 63, 2 ** 64 - 1, 2 ** 32, 2 ** 40 + 7]))
        else:
            at = r.randrange(8, min(len(data), 4096) - 4)
            data[at:at + 4] = struct.pack("<I", r.choice([9, 12, 13, 255, 2 ** 31]))
        p = tmp_path / "fuzz.gguf"
        p.write_bytes(bytes(data))
        h = ctypes.c_void_p()
        st = lib.te_model_load_gguf(str(p).encode(), ctypes.byref(opts), ctypes.byref(h))
        seen.add(st)
        assert st in (0, 2, 3, 4, 5)
        if st == 0:
            m = Model.__new__(Model)
            m._lib, m._model, m._options = lib, h, RuntimeOptions()
            m.info()
            m.tokenizer_info()
            try:
                m.tokenize("ab <|im_start|> x")
                m.detokenize_bytes(list(range(min(3, m.tokenizer_info().token_count))))
            except R.TinyEngineError:
                pass
            m.close()
        else:
            assert not h.value
    assert 0 in seen and len(seen) >= 3


def test_rng_matches_reference_source():
    """Pins the oracle's xorshift64* (the sampler's generator) to the
    reference's own te_qwen_rng_uniform (c/src/qwen.c:1170-1178), read as text
    where the reference tree is present: each statement of that function is
    evaluated over 64-bit integers by a small interpreter that accepts only the
    statement forms it contains (shift-xor, the state store, the multiply and
    the final scaling), and the result must equal oracle.text.xorshift_uniform
    for many states.  A wrong shift, direction, order or constant in the
    oracle fails; a change of the reference's function fails loudly."""
    import re
    from pathlib import Path

    src_path = Path("/root/reference/c/src/qwen.c")
    if not src_path.is_file():
        pytest.skip("reference tree not present")
    src = src_path.read_text()
    m = re.search(r"static double te_qwen_rng_uniform\(te_qwen_state \*state\) \{(.*?)\n\}", src, re.S)
    assert m, "te_qwen_rng_uniform not found"
    body = re.sub(r"/\*.*?\*/", "", m.group(1), flags=re.S)
    stmts = [s.strip() for s in body.split(";") if s.strip()]
    mask = (1 << 64) - 1

    def run(state):
        env = {}
        for s in stmts:
            if re.fullmatch(r"uint64_t x = state->rng_state", s):
                env["x"] = state
            elif mm := re.fullmatch(r"x \^= x (>>|<<) (\d+)", s):
                n = int(mm.group(2))
                env["x"] ^= (env["x"] >> n) if mm.group(1) == ">>" else ((env["x"] << n) & mask)
            elif re.fullmatch(r"state->rng_state = x", s):
                env["state"] = env["x"]
            elif mm := re.fullmatch(r"const uint64_t r = x \* (0x[0-9A-Fa-f]+)ULL", s):
                env["r"] = (env["x"] * int(mm.group(1), 16)) & mask
            elif mm := re.fullmatch(r"return \(double\)\(r >> (\d+)\) / ([0-9.]+)", s):
                return (env["r"] >> int(mm.group(1))) / float(mm.group(2)), env["state"]
            else:
                raise AssertionError(f"unexpected statement in the reference's generator: {s!r}")
        raise AssertionError("no return")

    r = random.Random(3)
    states = [0x9E3779B97F4A7C15, 1, 2, mask] + [r.getrandbits(64) | 1 for _ in range(200)]
    for st in states:
        want_u, want_s = run(st)
        got_u, got_s = OT.xorshift_uniform(st)
        assert (got_u, got_s) == (want_u, want_s), hex(st)
    # a chain of draws from the reference default seed
    st = 0x9E3779B97F4A7C15
    for _ in range(1000):
        want_u, want_s = run(st)
        got_u, got_s = OT.xorshift_uniform(st)
        assert got_u == want_u and got_s == want_s
        st = got_s

"""GPU parity of the model-level entry points and of generation
(te_model.hip): te_model_dequantize_row_f32 and te_model_matvec_f32 on GGUF
tensors, and te_generate / te_generate_raw through the HIP decode path.

- The reference's own expectations on its test file (c/tests/kernel_ops.c:
  291-326): exact dequantized rows and exact matvec results.
- Matvec on tensors at any byte alignment and F32 rows of any width (an
  aligned, zero-padded copy) against the fp64 product, with the GEMV bound.
- Generation against the oracle's restatement of the reference loop
  (qwen.c:261-400) on a random Qwen2 GGUF.  The oracle is fed the tokens the
  GPU chose (teacher forcing) and checks each step: greedy -- the chosen
  token's oracle logit within `tol` of the oracle's maximum, and equal to the
  oracle's argmax when the top two differ by more than `tol`; sampled (same
  seed, top-k, temperature) -- equal to the oracle's draw whenever the draw
  lies farther than the logit tolerance can move it from every boundary of
  the cumulative distribution.  `tol` is the attention bar (2e-3 of the
  largest logit magnitude), carried to the logits.
"""
import ctypes

import numpy as np
import pytest

import _gguf as G
from oracle import text as OT

pytestmark = pytest.mark.gpu

from tinymetalagent_amd import runtime as R  # noqa: E402
from tinymetalagent_amd.model import Model, RuntimeOptions  # noqa: E402


@pytest.fixture(scope="module")
def fixture_path(tmp_path_factory):
    return G.kernel_ops_fixture(tmp_path_factory.mktemp("gguf") / "kernel-test.gguf")


def test_kernel_ops_fixture_dequantize_and_matvec(fixture_path):
    with Model(fixture_path) as m:
        row = m.dequantize_row("token_embd.weight", 0)
        assert row[:16] == [float(i - 8) for i in range(16)]
        assert row[16:] == [float(7 - i) for i in range(16)]
        assert m.dequantize_row("token_embd.weight", 1) == [0.0] * 32
        assert m.dequantize_row("output.weight", 0) == [(i - 16) * 0.25 for i in range(32)]
        assert m.dequantize_row("output.weight", 2) == [1.0] * 32
        ones = [1.0] * 32
        assert m.matvec("token_embd.weight", ones) == [-16.0, 0.0, 0.0]
        assert m.matvec("output.weight", ones) == [-4.0, 32.0, 32.0]  # a 2-byte aligned Q8_0 tensor


def _bound(w, x):
    w64, x64 = w.astype(np.float64), x.astype(np.float64)
    exact = w64 @ x64
    bound = 2.0 ** -19 * (np.abs(w64) @ np.abs(x64))
    if w.shape[1] % 32 == 0:
        block_max = np.repeat(np.abs(x64).reshape(-1, 32).max(1), 32)
        bound += 2.0 ** -21 * (np.abs(w64) @ block_max) + 2.0 ** -126 * np.abs(w64).sum(1)
    return exact, bound + 1e-30


@pytest.mark.parametrize("ggml_type,cols,rows,offset", [
    (2, 256, 300, 3), (8, 128, 257, 2), (2, 4096, 40, 0), (8, 96, 33, 1),
    (0, 37, 50, 0), (0, 64, 20, 4), (0, 7, 3, 1)])
def test_model_matvec_any_alignment(oracle_mod, tmp_path, ggml_type, cols, rows, offset):
    import _synth as S
    data = S.ggml_tensor(9, f"mv{ggml_type}{cols}", ggml_type, rows, cols, scale=0.05)
    w = G.GGUFWriter(3, 1)
    w.kv("general.architecture", G.STR, "qwen2").kv("general.alignment", G.U32, 1)
    for k, v in (("embedding_length", 32), ("block_count", 1), ("feed_forward_length", 64),
                 ("attention.head_count", 1)):
        w.kv(f"qwen2.{k}", G.U32, v)
    w.kv("qwen2.attention.layer_norm_rms_epsilon", G.F32, 1e-6)
    w.tensor("pad", (offset or 1,), 0, b"", offset=0)
    w.tensor("t.weight", (cols, rows), ggml_type, data, offset=offset)
    w.tensor("token_embd.weight", (32, 3), 0, np.zeros(96, np.float32), offset=offset + data.size)
    path = w.write(tmp_path / "mv.gguf")
    x = S.normal(9, "x", (cols,))
    with Model(path) as m:
        assert m.tensor_info("t.weight").absolute_offset % 16 == (m.info().tensor_data_offset + offset) % 16
        got = np.array(m.matvec("t.weight", x.tolist()), np.float64)
        wf = oracle_mod.dequantize_rows(data, ggml_type, cols, rows)
        exact, bound = _bound(wf, x)
        assert np.all(np.abs(got - exact) <= bound)
        for r in (0, rows - 1):
            assert np.array_equal(np.array(m.dequantize_row("t.weight", r), np.float32), wf[r])


def _gpu_generate(path, prompt, max_tokens, raw=True, ctx=256, monkeypatch=None, env=None):
    for k, v in (env or {}).items():
        monkeypatch.setenv(k, v)
    ids, pieces = [], []
    with Model(path, RuntimeOptions(context_tokens=ctx)) as m:
        fn = m.generate_raw if raw else m.generate
        text = fn(prompt, max_tokens, on_token=lambda s, i: (ids.append(i), pieces.append(s)))
    return ids, text


def _prompt_ids(q, text):
    return OT.Tokenizer(q["tokens"], q["types"], q["merges"]).tokenize(text.encode(), True)


def _check_greedy(q, prompt_ids, got, ctx):
    chosen, logits, _ = OT.generate(q, prompt_ids, len(got), eos=-1, pad=-1, context_tokens=ctx, forced=got)
    exact = 0
    for i, (g, lg) in enumerate(zip(got, logits)):
        tol = 2e-3 * float(np.abs(lg).max())
        top2 = np.sort(lg)[-2:]
        assert lg[g] >= top2[1] - tol, (i, g, chosen[i])
        if top2[1] - top2[0] > tol:
            assert g == chosen[i], i
            exact += 1
    return exact


@pytest.fixture(scope="module")
def q4_model(tmp_path_factory):
    return G.qwen2_model(tmp_path_factory.mktemp("gguf") / "q4.gguf", seed=5, ggml_type=2, layers=2, heads=4,
                         kv_heads=2, head_dim=64, ffn=256, n_merges=80)


@pytest.mark.parametrize("path_env", [
    {},
    {"TINYENGINE_DECODE_ALL_LAYERS": "0"},
    {"TINYENGINE_FUSED_DECODE_LAYER": "0"},
    {"TINYENGINE_PREFILL_ALL_LAYERS": "0"},
    {"TINYENGINE_PREFILL_ALL_LAYERS": "0", "TINYENGINE_FUSED_PREFILL_LAYER": "0"},
], ids=["fused", "decode-per-layer", "decode-op-by-op", "prefill-per-layer", "prefill-token-by-token"])
def test_generate_raw_greedy_vs_oracle(q4_model, monkeypatch, path_env):
    """Greedy generation against the oracle's loop on every path the
    reference's switches select (qwen.c:1392, :1484, :1646, :1799): the fused
    all-layers flows, one fused layer per launch sequence, the layer as
    separate operations, and the prompt token by token."""
    q = q4_model
    prompt = "<|im_start|>user\nhello world, the engine<|im_end|>\n<|im_start|>assistant\n"
    got, text = _gpu_generate(q["path"], prompt, 24, monkeypatch=monkeypatch,
                              env={"TINYENGINE_TEMPERATURE": "0", "TINYENGINE_IGNORE_EOS": "1", **path_env})
    assert len(got) == 24
    pids = _prompt_ids(q, prompt)
    exact = _check_greedy(q, pids, got, 256)
    print(f"greedy: {exact}/24 steps decided beyond the tolerance, all equal")
    orc = OT.Tokenizer(q["tokens"], q["types"], q["merges"])
    # each callback piece is one token's bytes, decoded by the binding on its own
    assert text == "".join(orc.detokenize([i]).decode(errors="replace") for i in got)


def test_generate_chat_template_q8_tied_f32_embedding(tmp_path, monkeypatch):
    """te_generate (chat template), Q8_0 layers, head_dim 128, F32 token
    embeddings used as the head (no output.weight)."""
    q = G.qwen2_model(tmp_path / "q8.gguf", seed=7, ggml_type=8, layers=2, heads=2, kv_heads=1, head_dim=128,
                      ffn=384, n_merges=40, tied_head=True, embd_type=0)
    got, _ = _gpu_generate(q["path"], "the cache", 12, raw=False, ctx=128, monkeypatch=monkeypatch,
                           env={"TINYENGINE_TEMPERATURE": "0", "TINYENGINE_IGNORE_EOS": "1"})
    assert len(got) == 12
    _check_greedy(q, _prompt_ids(q, OT.chat_prompt("the cache")), got, 128)


def test_generate_sampled_vs_oracle(q4_model, monkeypatch):
    """Temperature sampling (the reference default T = 0.3, top-k 40, a fixed
    seed).  Every GPU token must be one of the oracle's top-k candidates
    (within tol); the tokens equal the oracle's draws at >= 90 % of the steps.
    Exact equality at every step is not a valid bar: a logit difference far
    below tol can reorder the reference's candidate list (its replacement
    scan compares logits) or move a boundary of the cumulative distribution
    past the draw.  With top_k 1 the sampled path must give the greedy
    path's tokens exactly (same GEMV head, argmax on the host)."""
    q = q4_model
    prompt = "qwen model attention"
    temperature, k, seed, n = 0.3, 40, 1234, 64
    got, _ = _gpu_generate(q["path"], prompt, n, monkeypatch=monkeypatch,
                           env={"TINYENGINE_TEMPERATURE": str(temperature), "TINYENGINE_TOP_K": str(k),
                                "TINYENGINE_SEED": str(seed), "TINYENGINE_IGNORE_EOS": "1"})
    assert len(got) == n
    chosen, logits, _ = OT.generate(q, _prompt_ids(q, prompt), n, eos=-1, pad=-1, context_tokens=256,
                                    temperature=temperature, top_k_n=k, seed=seed, forced=got)
    for i, (g, lg) in enumerate(zip(got, logits)):
        tol = 2e-3 * float(np.abs(lg).max())
        assert lg[g] >= np.sort(lg)[-k] - tol, i  # a top-k candidate
    same = sum(int(g == c) for g, c in zip(got, chosen))
    print(f"sampled: {same}/{n} draws equal to the oracle's")
    assert same >= 0.9 * n
    top1, _ = _gpu_generate(q["path"], prompt, 24, monkeypatch=monkeypatch,
                            env={"TINYENGINE_TEMPERATURE": "0.8", "TINYENGINE_TOP_K": "1"})
    greedy, _ = _gpu_generate(q["path"], prompt, 24, monkeypatch=monkeypatch, env={"TINYENGINE_TEMPERATURE": "0"})
    assert top1 == greedy


def test_generate_statuses_and_stub(q4_model, fixture_path, monkeypatch):
    q = q4_model
    lib = R.load_library()
    monkeypatch.setenv("TINYENGINE_TEMPERATURE", "0")
    with Model(q["path"], RuntimeOptions(context_tokens=16)) as m:
        with pytest.raises(R.TinyEngineError, match="unsupported"):  # prompt + max_tokens > context
            m.generate_raw("hello world, the engine", 16)
        with pytest.raises(R.TinyEngineError, match="invalid argument"):
            m.generate_raw("", 4)
        assert m.generate_raw("hello", 0) == ""
        monkeypatch.setenv("TINYENGINE_GENERATION", "stub")
        seen = []
        assert m.generate("anything", 3, on_token=lambda s, i: seen.append(i)) == "Mi chiamo"
        assert seen == [41887, 521, 34214]
        monkeypatch.delenv("TINYENGINE_GENERATION")
    with Model(fixture_path) as m:  # no layers: the norm weights are missing
        with pytest.raises(R.TinyEngineError, match="invalid argument"):
            m.generate_raw("ab", 2)
    # one context, two generations: the second starts again from position 0
    with Model(q["path"], RuntimeOptions(context_tokens=64)) as m:
        ctx = ctypes.c_void_p()
        opts = RuntimeOptions(context_tokens=64)._to_c()
        R.check(lib.te_context_create(m.handle, ctypes.byref(opts), ctypes.byref(ctx)))
        runs = []
        for _ in range(2):
            ids = []
            cb = R._TOKEN_CALLBACK(lambda s, i, u: ids.append(i))
            monkeypatch.setenv("TINYENGINE_IGNORE_EOS", "1")
            R.check(lib.te_generate_raw(ctx, b"the world", 10, cb, None))
            runs.append(ids)
        lib.te_context_free(ctx)
        assert runs[0] == runs[1] and len(runs[0]) == 10


def test_generate_stops_at_eos(q4_model, monkeypatch):
    """Without TINYENGINE_IGNORE_EOS the loop ends before emitting eos or the
    padding token (qwen.c:374-377, :2488-2498): the emitted ids never hold them."""
    q = q4_model
    monkeypatch.delenv("TINYENGINE_IGNORE_EOS", raising=False)
    for seed in ("3", "4", "5"):
        got, _ = _gpu_generate(q["path"], "json def", 40, monkeypatch=monkeypatch,
                               env={"TINYENGINE_TEMPERATURE": "1.5", "TINYENGINE_SEED": seed,
                                    "TINYENGINE_TOP_K": "400"})
        assert q["vocab"] - 1 not in got and q["vocab"] - 3 not in got


def test_session_kv_reuse_matches_fresh_context(q4_model, monkeypatch):
    """A second call on the same context reuses the K / V of the tokens it
    shares with the first call's sequence; its tokens equal a fresh context's
    and those of the same context with reuse off (TINYENGINE_KV_REUSE=0)."""
    q = q4_model
    monkeypatch.setenv("TINYENGINE_TEMPERATURE", "0")
    monkeypatch.setenv("TINYENGINE_IGNORE_EOS", "1")
    # one numeric path for every token: the batched prefill rounds activations
    # differently from the decode path, so a mix of the two agrees only to tolerance
    monkeypatch.setenv("TINYENGINE_BATCH_PREFILL", "0")
    turn1 = "<|im_start|>user\nhello world<|im_end|>\n<|im_start|>assistant\n"
    with Model(q["path"], RuntimeOptions(context_tokens=256)) as m:
        runs = {}
        for mode in ("reuse", "off"):
            monkeypatch.setenv("TINYENGINE_KV_REUSE", "1" if mode == "reuse" else "0")
            with m.session() as s:
                ids1 = []
                reply = s.generate_raw(turn1, 16, on_token=lambda t, i: ids1.append(i))
                turn2 = turn1 + reply + "<|im_end|>\n<|im_start|>user\nthe engine<|im_end|>\n"
                ids2 = []
                s.generate_raw(turn2, 16, on_token=lambda t, i: ids2.append(i))
                ids3 = []
                s.generate_raw(turn1, 16, on_token=lambda t, i: ids3.append(i))  # a shorter prompt again
            runs[mode] = (ids1, ids2, ids3)
        fresh = []
        m.generate_raw(turn2, 16, on_token=lambda t, i: fresh.append(i))
    assert runs["reuse"] == runs["off"]
    assert runs["reuse"][1] == fresh and runs["reuse"][2] == runs["reuse"][0]


@pytest.mark.parametrize("batch", ["1", "0"])
def test_long_prompt_batched_and_token_by_token_vs_oracle(q4_model, monkeypatch, batch):
    """A 600-token prompt: two chunks of batched prefill (512 rows, then 88 from
    base position 512), or one token at a time; greedy tokens against the
    oracle's loop, teacher-forced."""
    q = q4_model
    import random
    rnd = random.Random(4)
    words = ["hello", " world", " the", " engine", " cache", "\n", " json", "{", "}", " qwen", " gpu"]
    prompt = "".join(rnd.choice(words) for _ in range(800))
    pids = _prompt_ids(q, prompt)
    assert len(pids) > 600
    pids = pids[:600]
    orc = OT.Tokenizer(q["tokens"], q["types"], q["merges"])
    prompt = orc.detokenize(pids, False).decode()
    assert _prompt_ids(q, prompt) == pids
    got, _ = _gpu_generate(q["path"], prompt, 12, ctx=1024, monkeypatch=monkeypatch,
                           env={"TINYENGINE_TEMPERATURE": "0", "TINYENGINE_IGNORE_EOS": "1",
                                "TINYENGINE_BATCH_PREFILL": batch})
    assert len(got) == 12
    exact = _check_greedy(q, pids, got, 1024)
    print(f"600-token prompt, batch {batch}: {exact}/12 steps decided beyond the tolerance, all equal")


def test_two_threads_two_contexts_one_model(q4_model, monkeypatch):
    """Two threads generate at once on two contexts of one freshly loaded
    model (the first GPU use, the file upload, races between them); each gets
    the tokens a lone call gets."""
    import threading
    q = q4_model
    monkeypatch.setenv("TINYENGINE_TEMPERATURE", "0")
    monkeypatch.setenv("TINYENGINE_IGNORE_EOS", "1")
    prompts = ["hello world, the engine", "json def return the cache"]
    with Model(q["path"], RuntimeOptions(context_tokens=128)) as m:
        alone = []
        for p in prompts:
            ids = []
            m.generate_raw(p, 16, on_token=lambda t, i, ids=ids: ids.append(i))
            alone.append(ids)
    with Model(q["path"], RuntimeOptions(context_tokens=128)) as m:
        got = [[], []]
        errors = []

        def run(k):
            try:
                for _ in range(3):
                    ids = []
                    m.generate_raw(prompts[k], 16, on_token=lambda t, i: ids.append(i))
                    got[k].append(ids)
            except Exception as e:  # pragma: no cover
                errors.append(e)

        threads = [threading.Thread(target=run, args=(k,)) for k in range(2)]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=120)
        assert not errors
        for k in range(2):
            assert got[k] == [alone[k]] * 3


def test_context_boundary(q4_model, monkeypatch):
    """prompt + max_tokens == context_tokens runs (the last token lands on the
    last slot); one more is UNSUPPORTED (qwen.c:446-450)."""
    q = q4_model
    monkeypatch.setenv("TINYENGINE_TEMPERATURE", "0")
    monkeypatch.setenv("TINYENGINE_IGNORE_EOS", "1")
    prompt = "hello world, the engine"
    n = len(_prompt_ids(q, prompt))
    with Model(q["path"], RuntimeOptions(context_tokens=n + 8)) as m:
        ids = []
        m.generate_raw(prompt, 8, on_token=lambda t, i: ids.append(i))
        assert len(ids) == 8
        with pytest.raises(R.TinyEngineError, match="unsupported"):
            m.generate_raw(prompt, 9)


def test_session_reuse_with_batched_prefill_vs_oracle(q4_model, monkeypatch):
    """Second turn on one context with batched prefill: the cached prefix
    (prompt from the batched path, the reply from the decode path) plus a
    batched suffix from its base position; greedy tokens against the oracle's
    loop over the whole second-turn prompt, teacher-forced."""
    q = q4_model
    monkeypatch.setenv("TINYENGINE_TEMPERATURE", "0")
    monkeypatch.setenv("TINYENGINE_IGNORE_EOS", "1")
    monkeypatch.delenv("TINYENGINE_BATCH_PREFILL", raising=False)
    orc = OT.Tokenizer(q["tokens"], q["types"], q["merges"])
    turn1 = "<|im_start|>user\nhello world<|im_end|>\n<|im_start|>assistant\n"
    with Model(q["path"], RuntimeOptions(context_tokens=256)) as m, m.session() as s:
        ids1 = []
        s.generate_raw(turn1, 16, on_token=lambda t, i: ids1.append(i))
        reply = orc.detokenize(ids1, False).decode(errors="replace")
        turn2 = turn1 + reply + "<|im_end|>\n<|im_start|>user\nthe engine json<|im_end|>\n"
        got = []
        s.generate_raw(turn2, 12, on_token=lambda t, i: got.append(i))
    assert len(got) == 12
    exact = _check_greedy(q, _prompt_ids(q, turn2), got, 256)
    print(f"second turn with reuse: {exact}/12 steps decided beyond the tolerance, all equal")


@pytest.mark.parametrize("path_env", [{}, {"TINYENGINE_FUSED_DECODE_LAYER": "0"}], ids=["fused", "op-by-op"])
def test_profile_line(q4_model, monkeypatch, capfd, path_env):
    """TINYENGINE_PROFILE=1 prints one line per generate call on stderr in the
    reference's format (qwen.c:2262-2304: the same keys in the same order),
    followed by this build's buckets; call counts follow the launches: one
    per layer and matrix for the prompt chunk and for every forwarded token,
    one head projection per next token."""
    import re

    q = q4_model
    prompt = "qwen model attention"
    n = 6
    got, _ = _gpu_generate(q["path"], prompt, n, monkeypatch=monkeypatch,
                           env={"TINYENGINE_TEMPERATURE": "0", "TINYENGINE_IGNORE_EOS": "1",
                                "TINYENGINE_PROFILE": "1", **path_env})
    assert len(got) == n
    err = capfd.readouterr().err
    lines = [ln for ln in err.splitlines() if ln.startswith("tinyengine_profile:")]
    assert len(lines) == 1, err
    line = lines[0]
    print(line)
    ref_keys = ("total_ms tokenize_ms init_ms embed_ms matvec_ms q k v o gate up down lm_head other").split()
    keys = re.findall(r" (\w+)=", line)
    assert tuple(keys[:len(ref_keys)]) == tuple(ref_keys)
    f = dict(re.findall(r" (\w+)=([\d.]+(?:/\d+)?)", line))
    ms = {k: float(v.split("/")[0]) for k, v in f.items()}
    calls = {k: int(v.split("/")[1]) for k, v in f.items() if "/" in v}
    layers = 2
    forwards = n - 1  # the last emitted token is not run
    for key in ("q", "k", "v", "o", "gate", "up", "down"):
        assert calls[key] == layers * (1 + forwards), (key, calls[key])
        assert ms[key] > 0.0
    assert calls["lm_head"] == n
    assert calls["attention"] >= layers * (1 + forwards)
    buckets = sum(ms[k] for k in ("q", "k", "v", "o", "gate", "up", "down", "lm_head", "other"))
    assert abs(buckets - ms["matvec_ms"]) <= 0.02 * len(ref_keys)
    assert ms["total_ms"] >= ms["prefill_ms"] + ms["decode_ms"]
    assert int(f["prompt_tokens"]) == len(_prompt_ids(q, prompt)) and int(f["generated_tokens"]) == n

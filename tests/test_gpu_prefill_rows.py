"""The rows kernel of the causal prefill (prefill_rows_f16_kernel in
te_prefill.hip: one workgroup per 32 query rows of one head, the row group's
64-key blocks split round-robin over its 8 waves, the waves' softmax states
merged once through LDS).  The library takes it for launches with one split
over at most 256 keys (base + tokens <= 256); TE_HIP_PREFILL_ROWS=1 forces
it, =0 keeps the tile kernel.

Every row is checked against the oracle (row t = the reference decode at
position base + t, qwen.c:810-824), at shapes with several blocks per wave
(the lazy reference raised inside a wave), ragged row groups, a chunk after a
cached prefix, head_dim 64, several (seq, layer) units in one launch, and
through the fused step (bias + RoPE on the query load); and against the tile
kernel on the same inputs."""
import math

import numpy as np
import pytest

import _synth as S

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tinymetalagent_amd import attention as A  # noqa: E402

TOL = 2e-3  # max-abs error bar for attention outputs (north_star)


def f16_dev(bits_u16):
    return torch.from_numpy(np.ascontiguousarray(bits_u16)).view(torch.float16).to("cuda")


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def _run(monkeypatch, kernel, q16, kc, vc, base):
    if kernel is None:
        monkeypatch.delenv("TE_HIP_PREFILL_ROWS", raising=False)
    else:
        monkeypatch.setenv("TE_HIP_PREFILL_ROWS", kernel)
    out = A.attention_prefill(f16_dev(q16), f16_dev(kc), f16_dev(vc), base_position=base)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("seqs,layers,h,kv,d,tokens,base", [
    (1, 1, 16, 2, 128, 512, 0),      # BASELINE config 3 (3B) at L=512: one block per wave
    (1, 1, 16, 2, 128, 1000, 0),     # 16 blocks: two per wave
    (1, 1, 16, 2, 128, 100, 700),    # chunk after a prefix: 13 blocks, ragged last group
    (1, 1, 16, 2, 128, 33, 0),       # one full group and a one-row group
    (1, 1, 8, 1, 128, 31, 5),        # one partial group, one KV head
    (1, 1, 14, 2, 64, 77, 0),        # head_dim 64
    (2, 3, 12, 2, 128, 129, 40),     # six (seq, layer) units
    (1, 1, 28, 4, 128, 1, 2000),     # one row over 32 blocks: four per wave
])
def test_rows_kernel_vs_oracle(oracle_mod, monkeypatch, seqs, layers, h, kv, d, tokens, base):
    ctx = base + tokens + 5
    tag = f"rows{seqs}{layers}{h}{kv}{d}{tokens}{base}"
    kc = S.to_f16_bits(S.normal(61, tag + "k", (seqs, layers, ctx, kv, d)))
    vc = S.to_f16_bits(S.normal(61, tag + "v", (seqs, layers, ctx, kv, d)))
    q16 = S.to_f16_bits(S.normal(61, tag + "q", (seqs, layers, tokens, h, d)))
    rows = _run(monkeypatch, "1", q16, kc, vc, base).cpu().numpy()
    tile = _run(monkeypatch, "0", q16, kc, vc, base).cpu().numpy()
    assert np.isfinite(rows).all()
    worst = 0.0
    for s_ in range(seqs):
        for l_ in range(layers):
            want = oracle_mod.attention_prefill(S.f16_bits_to_f32(q16[s_, l_]).reshape(tokens, h, d),
                                                kc[s_, l_].copy(), vc[s_, l_].copy(), tokens, base, ctx, h, kv, d)
            worst = max(worst, float(np.abs(rows[s_, l_] - want.reshape(tokens, h, d)).max()))
    drift = float(np.abs(rows - tile).max())
    print(f"rows kernel {seqs}x{layers} H{h} KV{kv} d{d} L{tokens} base{base}: max abs err {worst:.3e}, "
          f"vs tile kernel {drift:.3e}")
    assert worst <= TOL
    assert drift <= TOL


@pytest.mark.parametrize("tokens,base,rows_default", [(256, 0, True), (100, 156, True), (257, 0, False),
                                                      (512, 0, False), (100, 420, False)])
def test_rows_kernel_is_the_default_up_to_256_keys(monkeypatch, tokens, base, rows_default):
    """The default choice: the rows kernel exactly when base + tokens <= 256
    (its output bits equal the forced rows kernel's there, the forced tile
    kernel's otherwise)."""
    h, kv, d = 16, 2, 128
    ctx = base + tokens
    tag = f"rowsdef{tokens}{base}"
    kc = S.to_f16_bits(S.normal(62, tag + "k", (1, 1, ctx, kv, d)))
    vc = S.to_f16_bits(S.normal(62, tag + "v", (1, 1, ctx, kv, d)))
    q16 = S.to_f16_bits(S.normal(62, tag + "q", (1, 1, tokens, h, d)))
    auto = _run(monkeypatch, None, q16, kc, vc, base)
    rows = _run(monkeypatch, "1", q16, kc, vc, base)
    tile = _run(monkeypatch, "0", q16, kc, vc, base)
    assert not torch.equal(rows, tile)  # the two kernels round differently on these inputs
    assert torch.equal(auto, rows if rows_default else tile)


@pytest.mark.parametrize("tokens,base,rows_default", [(512, 0, True), (300, 213, False), (300, 212, True)])
def test_rows_kernel_is_the_fused_step_default_up_to_512_keys(monkeypatch, tokens, base, rows_default):
    """The fused step (fp32 queries, bias and RoPE on load) takes the rows
    kernel by default up to base + tokens <= 512 keys: its output bits equal
    the forced rows kernel's there, the forced tile kernel's past it."""
    h, kv, d = 16, 2, 128
    ctx = base + tokens
    g = torch.Generator(device="cuda").manual_seed(tokens + base)
    q = torch.randn((1, 1, tokens, h, d), generator=g, device="cuda") / math.sqrt(d)
    k = torch.randn((1, 1, tokens, kv, d), generator=g, device="cuda")
    v = torch.randn((1, 1, tokens, kv, d), generator=g, device="cuda")
    kc0 = torch.randn((1, 1, ctx, kv, d), generator=g, device="cuda").half()
    vc0 = torch.randn((1, 1, ctx, kv, d), generator=g, device="cuda").half()
    cos, sin = A.rope_table(ctx, d, 1e6)

    def step(mode):
        if mode is None:
            monkeypatch.delenv("TE_HIP_PREFILL_ROWS", raising=False)
        else:
            monkeypatch.setenv("TE_HIP_PREFILL_ROWS", mode)
        kc, vc = kc0.clone(), vc0.clone()
        vt = A.value_t_buffer(1, 1, ctx, kv, d)
        A.value_transpose(vc, vt, first_position=0, count=base)
        out = A.prefill_step_vt(q, k, v, cos, sin, kc, vc, vt, base_position=base)
        torch.cuda.synchronize()
        return out

    auto, rows, tile = step(None), step("1"), step("0")
    assert not torch.equal(rows, tile)  # the two kernels round differently on these inputs
    assert torch.equal(auto, rows if rows_default else tile)


@pytest.mark.parametrize("seqs,layers,h,kv,d,tokens,base,bias", [
    (1, 1, 16, 2, 128, 512, 0, True),
    (2, 2, 14, 2, 64, 130, 37, True),
    (1, 2, 12, 2, 128, 200, 500, False),   # 11 blocks: forced rows kernel, two blocks on some waves
])
def test_rows_kernel_fused_step_vs_oracle(oracle_mod, monkeypatch, seqs, layers, h, kv, d, tokens, base, bias):
    """The fused V^T step (bias + RoPE + fp16 append + V^T rows, then the
    attention applying the query's bias and rotation on load) through the
    rows kernel: caches bit-exact against the oracle's append, the output bits
    equal to the attention-only launch on the fp16 queries the unfused path
    stores, every row within the bar of the oracle."""
    monkeypatch.setenv("TE_HIP_PREFILL_ROWS", "1")
    ctx = base + tokens + 3
    tag = f"rowsstep{h}{kv}{d}{tokens}{base}"
    q = S.normal(63, tag + "q", (seqs, layers, tokens, h, d), 1 / math.sqrt(d))
    k = S.normal(63, tag + "k", (seqs, layers, tokens, kv, d))
    v = S.normal(63, tag + "v", (seqs, layers, tokens, kv, d))
    qb = S.normal(63, tag + "qb", (layers, h * d), 0.1) if bias else None
    kb = S.normal(63, tag + "kb", (layers, kv * d), 0.1) if bias else None
    vb = S.normal(63, tag + "vb", (layers, kv * d), 0.1) if bias else None
    kc0 = S.to_f16_bits(S.normal(63, tag + "kc", (seqs, layers, ctx, kv, d)))
    vc0 = S.to_f16_bits(S.normal(63, tag + "vc", (seqs, layers, ctx, kv, d)))
    cos, sin = oracle_mod.rope_table(ctx, d, 1e6)
    q_o, k_o, v_o, kc_o, vc_o = q.copy(), k.copy(), v.copy(), kc0.copy(), vc0.copy()
    oracle_mod.rope_kv_append_f16(q_o, k_o, v_o, qb, kb, vb, cos, sin, kc_o, vc_o, seqs, layers, tokens, None, base,
                                  ctx, h, kv, d)
    q_half = S.to_f16_bits(q_o)
    dcos, dsin = A.rope_table(ctx, d, 1e6)
    kc, vc = f16_dev(kc0), f16_dev(vc0)
    vt = A.value_t_buffer(seqs, layers, ctx, kv, d)
    A.value_transpose(vc, vt)
    out = A.prefill_step_vt(to_dev(q), to_dev(k), to_dev(v), dcos, dsin, kc, vc, vt, base_position=base,
                            q_bias=to_dev(qb) if bias else None, k_bias=to_dev(kb) if bias else None,
                            v_bias=to_dev(vb) if bias else None)
    torch.cuda.synchronize()
    assert np.array_equal(kc.cpu().view(torch.int16).numpy().view(np.uint16), kc_o)
    assert np.array_equal(vc.cpu().view(torch.int16).numpy().view(np.uint16), vc_o)
    ref = A.attention_prefill_vt(f16_dev(q_half), kc, vt, base_position=base)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    got = out.cpu().numpy()
    worst = 0.0
    for s_ in range(seqs):
        for l_ in range(layers):
            want = oracle_mod.attention_prefill(S.f16_bits_to_f32(q_half[s_, l_]).reshape(tokens, h, d),
                                                kc_o[s_, l_].copy(), vc_o[s_, l_].copy(), tokens, base, ctx, h, kv, d)
            worst = max(worst, float(np.abs(got[s_, l_] - want.reshape(tokens, h, d)).max()))
    print(f"rows kernel fused step H{h} KV{kv} d{d} L{tokens} base{base} x{seqs * layers}: max abs err {worst:.3e}")
    assert worst <= TOL

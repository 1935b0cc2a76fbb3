"""GPU parity tests: the HIP kernels (through the C-ABI of libtinyengine.so)
against the CPU oracle, the reference's golden vectors and known-answer tests.

Bars: bit-exact for RoPE'd values, cache slot indexing,
fp16 cache contents and positions; max-abs error <= 2e-3 for attention outputs
(fp32 softmax and accumulation).  Shapes: the BASELINE configs, reduced where
the single-threaded oracle must finish in seconds, plus full-size checks
through size-independent properties (sampled rows/layers against the oracle,
constant-V, prefill row t == decode at base+t).
"""
import math

import numpy as np
import pytest

import _synth as S
import cases as C

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tinymetalagent_amd import attention as A  # noqa: E402
from tinymetalagent_amd import runtime as R  # noqa: E402

TOL = 2e-3  # max-abs error bar for attention outputs (north_star)
DEV = "cuda"


def bits32(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def to_dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.to(DEV)


def f16_dev(bits_u16):
    return torch.from_numpy(np.ascontiguousarray(bits_u16).view(np.int16)).to(DEV).view(torch.float16)


def f16_host_bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def maxabs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


# ------------------------------------------------------------------ device ---

def test_hip_path_is_live():
    assert R.hip_available(), "libtinyengine.so found no gfx950 device"
    name, cus = R.device_info()
    assert "gfx950" in name and cus >= 1
    print(f"device: {name}, {cus} CUs, library {R.library_path()}")


# -------------------------------------------------------------- public ABI ---

def test_rope_f32_public_matches_reference_bits(golden):
    data, meta = golden
    for name, heads, d, pos, theta in C.ROPE_CASES:
        x = C.rope_input(name, heads, d)
        got = R.rope_f32(x, heads, d, pos, theta)
        assert np.array_equal(bits32(got), bits32(data[f"rope/{name}"])), name


def test_rope_table_device_matches_reference_bits(golden):
    data, meta = golden
    positions = meta["rope_rows"]["positions"]
    for d in (64, 128):
        cos, sin = A.rope_table(max(positions) + 1, d, 1e6)
        cos, sin = cos.cpu().numpy(), sin.cpu().numpy()
        rows = data[f"rope_rows/d{d}"]
        for i, p in enumerate(positions):
            assert np.array_equal(bits32(cos[p]), bits32(rows[i, : d // 2])), (d, p)
            assert np.array_equal(bits32(sin[p]), bits32(rows[i, d // 2:])), (d, p)


def test_attention_decode_f32_public_kat():
    # reference c/tests/kernel_ops.c:341-356
    out = R.attention_decode_f32(np.array([1, 0, 0, 1], np.float32), np.array([1, 0, 0, 1], np.float32),
                                 np.array([10, 20, 30, 40], np.float32), 1, 2, 1, 2)
    sc = 1 / math.sqrt(2)
    hi = math.exp(sc)
    wh, wl = hi / (hi + 1), 1 / (hi + 1)
    want = [wh * 10 + wl * 30, wh * 20 + wl * 40, wl * 10 + wh * 30, wl * 20 + wh * 40]
    np.testing.assert_allclose(out, want, atol=1e-5, rtol=0)


def test_attention_decode_f32_public_golden(golden):
    data, meta = golden
    for case in C.DECODE_CASES:
        q, kb, vb = C.decode_inputs(case)
        assert S.digest(q, kb, vb) == meta["decode"][case["name"]]["input_sha256"]
        got = R.attention_decode_f32(q, S.f16_bits_to_f32(kb), S.f16_bits_to_f32(vb), case["pos"], case["heads"],
                                     case["kv"], case["d"])
        err = maxabs(got, data[f"decode/{case['name']}"])
        print(f"te_attention_decode_f32 {case['name']}: max abs err {err:.3e}")
        assert err <= 5e-5, case["name"]


def _kat_inputs(k_cols, kscale, vscale):
    # formulas of reference c/tests/kernel_ops.c:522-741
    q = np.array([[(q + 1) * ((d % 7) + 1) * 0.0078125 for d in range(64)] for q in range(8)], np.float32)
    kt = np.array([[((d % 5) + 1) * (k + 2) * kscale for k in range(k_cols)] for d in range(64)], np.float32)
    v = np.array([[(k + 3) * ((d % 11) + 1) * vscale for d in range(64)] for k in range(k_cols)], np.float32)
    return q, kt, v


def _kat_expected(q, kt, v, q_base=None):
    s = q.astype(np.float32) @ kt.astype(np.float32) / np.float32(8.0)
    if q_base is not None:
        for r in range(8):
            s[r, q_base + r + 1:] = -np.inf
    w = np.exp(s - s.max(1, keepdims=True))
    return (w / w.sum(1, keepdims=True)) @ v


def test_mma_twins_reference_kats():
    q, kt, _ = _kat_inputs(8, 0.015625, 0)
    got = R.attention_qk_mma_f32(q, kt, 8, 8, 64).reshape(8, 8)
    np.testing.assert_allclose(got, q @ kt, atol=1e-4, rtol=0)
    q, kt, v = _kat_inputs(8, 0.015625, 0.00390625)
    got = R.attention_tile_mma_f32(q, kt, v, 8, 8, 64).reshape(8, 64)
    np.testing.assert_allclose(got, _kat_expected(q, kt, v), atol=1e-4, rtol=0)
    q, kt, v = _kat_inputs(24, 0.00390625, 0.001953125)
    got = R.attention_stream_mma_f32(q, kt, v, 8, 24, 64).reshape(8, 64)
    np.testing.assert_allclose(got, _kat_expected(q, kt, v), atol=1e-4, rtol=0)
    got = R.attention_causal_mma_f32(q, kt, v, 8, 24, 64, 8).reshape(8, 64)
    np.testing.assert_allclose(got, _kat_expected(q, kt, v, q_base=8), atol=1e-4, rtol=0)


# ---------------------------------------------------------- RoPE + append ---

def test_rope_kv_append_bit_exact(oracle_mod):
    seqs, layers, tokens, ctx, h, kv, d = 3, 2, 5, 48, 16, 2, 128
    bases = [0, 17, 43]
    q = S.normal(20, "gq", (seqs, layers, tokens, h, d))
    k = S.normal(20, "gk", (seqs, layers, tokens, kv, d))
    v = S.normal(20, "gv", (seqs, layers, tokens, kv, d))
    qb = S.normal(20, "gqb", (layers, h * d), 0.1)
    kb = S.normal(20, "gkb", (layers, kv * d), 0.1)
    vb = S.normal(20, "gvb", (layers, kv * d), 0.1)
    cos, sin = oracle_mod.rope_table(ctx, d, 1e6)
    sentinel = np.full((seqs, layers, ctx, kv, d), 0x7E01, np.uint16)
    # oracle
    q_o, k_o, v_o = q.copy(), k.copy(), v.copy()
    kc_o, vc_o = sentinel.copy(), sentinel.copy()
    oracle_mod.rope_kv_append_f16(q_o, k_o, v_o, qb, kb, vb, cos, sin, kc_o, vc_o, seqs, layers, tokens, bases, 0,
                                  ctx, h, kv, d)
    # GPU
    tq, tk, tv = to_dev(q), to_dev(k), to_dev(v)
    dcos, dsin = A.rope_table(ctx, d, 1e6)
    kc, vc = f16_dev(sentinel), f16_dev(sentinel)
    qh = torch.empty(q.shape, dtype=torch.float16, device=DEV)
    A.rope_kv_append(tq, tk, tv, dcos, dsin, kc, vc, base_positions=bases, q_bias=to_dev(qb), k_bias=to_dev(kb),
                     v_bias=to_dev(vb), q_half=qh)
    torch.cuda.synchronize()
    assert np.array_equal(bits32(tq.cpu().numpy()), bits32(q_o))
    assert np.array_equal(bits32(tk.cpu().numpy()), bits32(k_o))
    assert np.array_equal(bits32(tv.cpu().numpy()), bits32(v_o))
    assert np.array_equal(f16_host_bits(kc), kc_o)
    assert np.array_equal(f16_host_bits(vc), vc_o)
    assert np.array_equal(f16_host_bits(qh), S.to_f16_bits(q_o))


def test_rope_kv_append_no_bias_decode_all_layers(oracle_mod):
    seqs, layers, ctx, h, kv, d = 1, 36, 9000, 16, 2, 128
    pos = 8192
    q = S.normal(21, "dq", (seqs, layers, 1, h, d), 1 / math.sqrt(d))
    k = S.normal(21, "dk", (seqs, layers, 1, kv, d))
    v = S.normal(21, "dv", (seqs, layers, 1, kv, d))
    cos, sin = oracle_mod.rope_table(ctx, d, 1e6)
    kc_o = np.zeros((seqs, layers, ctx, kv, d), np.uint16)
    vc_o = kc_o.copy()
    q_o, k_o, v_o = q.copy(), k.copy(), v.copy()
    oracle_mod.rope_kv_append_f16(q_o, k_o, v_o, None, None, None, cos, sin, kc_o, vc_o, seqs, layers, 1, None, pos,
                                  ctx, h, kv, d)
    tq, tk, tv = to_dev(q), to_dev(k), to_dev(v)
    dcos, dsin = A.rope_table(ctx, d, 1e6)
    kc = torch.zeros((seqs, layers, ctx, kv, d), dtype=torch.float16, device=DEV)
    vc = torch.zeros_like(kc)
    A.rope_kv_append(tq, tk, tv, dcos, dsin, kc, vc, base_position=pos)
    torch.cuda.synchronize()
    assert np.array_equal(bits32(tq.cpu().numpy()), bits32(q_o))
    assert np.array_equal(f16_host_bits(kc[:, :, pos]), kc_o[:, :, pos])
    assert np.array_equal(f16_host_bits(vc[:, :, pos]), vc_o[:, :, pos])
    assert int(torch.count_nonzero(kc[:, :, :pos])) == 0 and int(torch.count_nonzero(kc[:, :, pos + 1:])) == 0


# ------------------------------------------------------------------ decode ---

def _decode_gpu(q, kc_bits, vc_bits, positions, seqs, layers, ctx, h, kv, d):
    tq = to_dev(q.reshape(seqs, layers, h, d))
    kc = f16_dev(kc_bits.reshape(seqs, layers, ctx, kv, d))
    vc = f16_dev(vc_bits.reshape(seqs, layers, ctx, kv, d))
    out = A.attention_decode(tq, kc, vc, positions=positions)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_decode_f16_golden(golden):
    data, meta = golden
    for case in C.DECODE_CASES:
        q, kb, vb = C.decode_inputs(case)
        assert S.digest(q, kb, vb) == meta["decode"][case["name"]]["input_sha256"]
        n = case["pos"] + 1
        ctx = n + 5  # cache capacity beyond the attended range
        kc = np.zeros((ctx, case["kv"], case["d"]), np.uint16)
        vc = np.zeros_like(kc)
        kc[:n] = kb.reshape(n, case["kv"], case["d"])
        vc[:n] = vb.reshape(n, case["kv"], case["d"])
        kc[n:] = 0x7C00  # +inf past the end: must never be read
        vc[n:] = 0x7E00  # NaN past the end
        got = _decode_gpu(q, kc, vc, [case["pos"]], 1, 1, ctx, case["heads"], case["kv"], case["d"])
        err = maxabs(got.reshape(-1), data[f"decode/{case['name']}"])
        print(f"decode_f16 {case['name']}: max abs err {err:.3e}")
        assert err <= TOL, case["name"]


@pytest.mark.parametrize("shape", [
    # heads, kv, d, layers, positions (per sequence)
    (14, 2, 64, 1, [0, 1, 31, 32, 127, 128, 129, 255, 256, 512, 1000]),
    (16, 2, 128, 3, [2047]),
    (28, 4, 128, 2, "ragged8"),
    (12, 2, 128, 1, [4096]),
    (16, 16, 128, 1, [300]),
    (8, 1, 64, 2, [5000, 3]),
    (16, 1, 128, 1, [777]),  # a 16-head group: every MFMA column is a real head
])
def test_decode_f16_vs_oracle(oracle_mod, shape):
    h, kv, d, layers, positions = shape
    if positions == "ragged8":
        positions = [int(x) for x in S.rng(S.SEED, "ragged").integers(1, 3000, size=8)]
    outliers = h == 12
    seqs = len(positions)
    ctx = max(positions) + 3
    tag = f"dec{h}{kv}{d}{layers}{seqs}"
    q = S.normal(22, tag + "q", (seqs, layers, h, d), 1 / math.sqrt(d))
    shape_kv = (seqs, layers, ctx, kv, d)
    kf = S.outlier_keys(22, tag + "k", shape_kv) if outliers else S.normal(22, tag + "k", shape_kv)
    kc = S.to_f16_bits(kf)
    vc = S.to_f16_bits(S.normal(22, tag + "v", shape_kv))
    want = oracle_mod.attention_decode_f16kv(q, kc, vc, positions, 0, seqs, layers, ctx, h, kv, d)
    got = _decode_gpu(q, kc, vc, positions, seqs, layers, ctx, h, kv, d)
    err = maxabs(got, want)
    print(f"decode_f16 {shape[:4]} positions={positions}: max abs err {err:.3e}")
    assert err <= TOL


def test_decode_sharp_softmax(oracle_mod):
    # large-magnitude queries: near one-hot attention stresses P rounding
    h, kv, d, ctx = 16, 2, 128, 1500
    q = S.normal(23, "sq", (1, 1, h, d), 1.5)
    kc = S.to_f16_bits(S.normal(23, "sk", (1, 1, ctx, kv, d)))
    vc = S.to_f16_bits(S.normal(23, "sv", (1, 1, ctx, kv, d)))
    want = oracle_mod.attention_decode_f16kv(q, kc, vc, [ctx - 1], 0, 1, 1, ctx, h, kv, d)
    got = _decode_gpu(q, kc, vc, [ctx - 1], 1, 1, ctx, h, kv, d)
    err = maxabs(got, want)
    print(f"decode_f16 sharp softmax: max abs err {err:.3e}")
    assert err <= TOL


def test_decode_config1_step(oracle_mod):
    """BASELINE config 1 end to end: RoPE + fp16 append of 512 cached tokens,
    then one decode step at position 512 (append + attention)."""
    h, kv, d, theta, pos = 14, 2, 64, 1e6, 512
    ctx = pos + 1
    scale = 1 / math.sqrt(d)
    qs = S.normal(24, "c1q", (1, 1, pos + 1, h, d), scale)
    ks = S.normal(24, "c1k", (1, 1, pos + 1, kv, d), scale)
    vs = S.normal(24, "c1v", (1, 1, pos + 1, kv, d), scale)
    cos, sin = oracle_mod.rope_table(ctx, d, theta)
    kc_o = np.zeros((1, 1, ctx, kv, d), np.uint16)
    vc_o = kc_o.copy()
    q_o, k_o, v_o = qs.copy(), ks.copy(), vs.copy()
    oracle_mod.rope_kv_append_f16(q_o, k_o, v_o, None, None, None, cos, sin, kc_o, vc_o, 1, 1, pos + 1, None, 0, ctx,
                                  h, kv, d)
    want = oracle_mod.attention_decode_f16kv(q_o[:, :, pos].copy(), kc_o, vc_o, None, pos, 1, 1, ctx, h, kv, d)

    dcos, dsin = A.rope_table(ctx, d, theta)
    kc = torch.zeros((1, 1, ctx, kv, d), dtype=torch.float16, device=DEV)
    vc = torch.zeros_like(kc)
    tq, tk, tv = to_dev(qs[:, :, :pos].copy()), to_dev(ks[:, :, :pos].copy()), to_dev(vs[:, :, :pos].copy())
    A.rope_kv_append(tq, tk, tv, dcos, dsin, kc, vc, base_position=0)          # cached prefix 0..511
    sq, sk, sv = to_dev(qs[:, :, pos:].copy()), to_dev(ks[:, :, pos:].copy()), to_dev(vs[:, :, pos:].copy())
    A.rope_kv_append(sq, sk, sv, dcos, dsin, kc, vc, base_position=pos)        # the decode token
    out = A.attention_decode(sq, kc, vc, position=pos)
    torch.cuda.synchronize()
    assert np.array_equal(f16_host_bits(kc), kc_o) and np.array_equal(f16_host_bits(vc), vc_o)
    err = maxabs(out.cpu().numpy().reshape(-1), want.reshape(-1))
    print(f"config-1 decode step: max abs err {err:.3e}")
    assert err <= TOL


def test_decode_full_size_3b_8k_sampled_layers(oracle_mod):
    """BASELINE config 2 at 8K, all 36 layers on the GPU; layers 0, 17, 35 against the oracle."""
    h, kv, d, layers, pos = 16, 2, 128, 36, 8192
    ctx = pos + 1
    g = torch.Generator(device=DEV).manual_seed(S.SEED)
    kc = torch.randn((1, layers, ctx, kv, d), generator=g, device=DEV).half()
    vc = torch.randn((1, layers, ctx, kv, d), generator=g, device=DEV).half()
    q = torch.randn((1, layers, h, d), generator=g, device=DEV) / math.sqrt(d)
    out = A.attention_decode(q, kc, vc, position=pos).cpu().numpy()
    for layer in (0, 17, 35):
        want = oracle_mod.attention_decode_f16kv(q[:, layer].cpu().numpy().copy(), f16_host_bits(kc[:, layer]),
                                                 f16_host_bits(vc[:, layer]), None, pos, 1, 1, ctx, h, kv, d)
        err = maxabs(out[:, layer], want)
        print(f"3B 8K layer {layer}: max abs err {err:.3e}")
        assert err <= TOL


def test_decode_constant_values_32k():
    """Size-independent property at 32K: V constant over positions -> output == that constant."""
    h, kv, d, layers, pos = 16, 2, 128, 2, 32767
    ctx = pos + 1
    g = torch.Generator(device=DEV).manual_seed(7)
    kc = torch.randn((1, layers, ctx, kv, d), generator=g, device=DEV).half()
    row = torch.randn((1, layers, 1, kv, d), generator=g, device=DEV).half()
    vc = row.expand(1, layers, ctx, kv, d).contiguous()
    q = torch.randn((1, layers, h, d), generator=g, device=DEV)
    out = A.attention_decode(q, kc, vc, position=pos)
    want = row[:, :, 0].float().repeat_interleave(h // kv, dim=2)
    err = float((out - want).abs().max())
    print(f"constant-V 32K: max abs err {err:.3e}")
    assert err <= 1e-4


def test_decode_step_full_size_1p5b_128k_outliers(oracle_mod):
    """BASELINE config 5 decode at full size: 1.5B shape, position 131072, K with
    +-20 spikes on 3 fixed channels per KV head; the fused step (RoPE + append +
    split-K) on 2 layers, layer 1 against the oracle, appended slots bit-exact."""
    h, kv, d, layers, pos = 12, 2, 128, 2, 131072
    ctx = pos + 1
    g = torch.Generator(device=DEV).manual_seed(11)
    kc = torch.randn((1, layers, ctx, kv, d), generator=g, device=DEV)
    gen = torch.Generator().manual_seed(7)
    for hk in range(kv):
        ch = torch.randperm(d, generator=gen)[:3].to(DEV)
        sign = torch.randint(0, 2, (1, layers, ctx, 3), generator=g, device=DEV) * 2 - 1
        kc[:, :, :, hk, ch] += 20.0 * sign
    kc = kc.half()
    vc = torch.randn((1, layers, ctx, kv, d), generator=g, device=DEV).half()
    q = torch.randn((1, layers, 1, h, d), generator=g, device=DEV) / math.sqrt(d)
    k = torch.randn((1, layers, 1, kv, d), generator=g, device=DEV)
    v = torch.randn((1, layers, 1, kv, d), generator=g, device=DEV)
    cos, sin = A.rope_table(ctx, d, 1e6)
    out = A.decode_step(q, k, v, cos, sin, kc, vc, position=pos)
    torch.cuda.synchronize()
    # oracle: RoPE + append of the new token into a host copy of layer 1, then decode
    hcos, hsin = oracle_mod.rope_table(ctx, d, 1e6)
    kc1, vc1 = f16_host_bits(kc[:, 1:2]).copy(), f16_host_bits(vc[:, 1:2]).copy()
    q1, k1, v1 = (t[:, 1:2].cpu().numpy().copy() for t in (q, k, v))
    kslot, vslot = kc1[0, 0, pos].copy(), vc1[0, 0, pos].copy()
    oracle_mod.rope_kv_append_f16(q1, k1, v1, None, None, None, hcos, hsin, kc1, vc1, 1, 1, 1, None, pos, ctx, h, kv, d)
    assert np.array_equal(kslot, kc1[0, 0, pos]) and np.array_equal(vslot, vc1[0, 0, pos])  # GPU wrote the same slot
    want = oracle_mod.attention_decode_f16kv(q1[:, :, 0].copy(), kc1, vc1, None, pos, 1, 1, ctx, h, kv, d)
    err = maxabs(out[:, 1].cpu().numpy(), want)
    print(f"1.5B 128K outlier keys, fused step, layer 1: max abs err {err:.3e}")
    assert err <= TOL


def test_prefill_chunk_after_128k_cache(oracle_mod):
    """BASELINE config 5 (B): a 256-token prefill chunk at base 131072 over the
    cached prefix; sampled rows t against the oracle decode at base + t."""
    h, kv, d, tokens, base = 12, 2, 128, 256, 131072
    ctx = base + tokens
    g = torch.Generator(device=DEV).manual_seed(12)
    kc = torch.randn((1, 1, ctx, kv, d), generator=g, device=DEV).half()
    vc = torch.randn((1, 1, ctx, kv, d), generator=g, device=DEV).half()
    qh = torch.randn((1, 1, tokens, h, d), generator=g, device=DEV).half()
    out = A.attention_prefill(qh, kc, vc, base_position=base).cpu().numpy().reshape(tokens, h, d)
    kb, vb = f16_host_bits(kc), f16_host_bits(vc)
    qf = qh.float().cpu().numpy().reshape(tokens, h, d)
    for t in (0, 129, tokens - 1):
        want = oracle_mod.attention_decode_f16kv(qf[t].reshape(1, 1, h, d).copy(), kb, vb, None, base + t, 1, 1, ctx,
                                                 h, kv, d)
        err = maxabs(out[t], want.reshape(h, d))
        print(f"prefill chunk after 128K, row {t}: max abs err {err:.3e}")
        assert err <= TOL


# ----------------------------------------------------------------- prefill ---

def _prefill_case(oracle_mod, h, kv, d, tokens, base, seed):
    ctx = base + tokens
    tag = f"pf{h}{kv}{d}{tokens}{base}"
    # cached prefix (base positions) + the chunk's own K/V, all fp16 in the cache
    kc = S.to_f16_bits(S.normal(seed, tag + "k", (1, 1, ctx, kv, d)))
    vc = S.to_f16_bits(S.normal(seed, tag + "v", (1, 1, ctx, kv, d)))
    q32 = S.normal(seed, tag + "q", (1, 1, tokens, h, d))
    q16 = S.to_f16_bits(q32)
    want = oracle_mod.attention_prefill(S.f16_bits_to_f32(q16).reshape(tokens, h, d), kc[0, 0], vc[0, 0], tokens,
                                        base, ctx, h, kv, d)
    out = A.attention_prefill(f16_dev(q16), f16_dev(kc), f16_dev(vc), base_position=base)
    torch.cuda.synchronize()
    return out.cpu().numpy().reshape(tokens, h, d), want


@pytest.mark.parametrize("kernel", ["auto", "tile", "rows"])
@pytest.mark.parametrize("h,kv,d,tokens,base", [
    (16, 2, 128, 300, 0),
    (16, 2, 128, 130, 200),
    (16, 2, 128, 1, 0),
    (16, 2, 128, 64, 0),
    (16, 2, 128, 512, 0),      # BASELINE config 3 (3B) at L=512
    (14, 2, 64, 200, 37),
    (28, 4, 128, 257, 0),
    (12, 2, 128, 129, 1000),
])
def test_prefill_vs_oracle(oracle_mod, monkeypatch, kernel, h, kv, d, tokens, base):
    """Every row against the oracle, with the library's kernel choice and with
    each kernel forced (TE_HIP_PREFILL_ROWS: the tile kernel, 128-row tiles
    over a step loop; the rows kernel, 32-row groups with their keys split over
    the waves)."""
    if kernel != "auto":
        monkeypatch.setenv("TE_HIP_PREFILL_ROWS", "1" if kernel == "rows" else "0")
    got, want = _prefill_case(oracle_mod, h, kv, d, tokens, base, 25)
    err = maxabs(got, want)
    print(f"prefill ({kernel}) H{h} KV{kv} d{d} L{tokens} base{base}: max abs err {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("seqs,layers,h,kv,d,tokens,base", [
    (1, 1, 16, 2, 128, 300, 0),      # 3 tiles: the lone middle tile and a pair, several splits
    (1, 1, 16, 2, 128, 130, 200),    # chunk after a cached prefix
    (1, 1, 16, 2, 128, 1, 0),        # one row
    (1, 1, 14, 2, 64, 200, 37),      # head_dim 64
    (2, 3, 12, 2, 128, 129, 1000),   # several (seq, layer) units, long prefix
    (1, 1, 16, 2, 128, 512, 0),      # BASELINE config 3 at L=512
    (1, 1, 16, 2, 128, 2048, 0),     # BASELINE config 3 at L=2048
])
def test_prefill_split_vs_oracle(oracle_mod, seqs, layers, h, kv, d, tokens, base):
    """Key-split prefill (partials in a workspace, then the merge launch)
    against the oracle for every row; the split count is the library's own
    choice for the shape on this device and is printed.  Also the plain
    kernel on the same inputs, and the workspace query."""
    ctx = base + tokens + 3
    tag = f"pfs{seqs}{layers}{h}{d}{tokens}{base}"
    kc = S.to_f16_bits(S.normal(41, tag + "k", (seqs, layers, ctx, kv, d)))
    vc = S.to_f16_bits(S.normal(41, tag + "v", (seqs, layers, ctx, kv, d)))
    q16 = S.to_f16_bits(S.normal(41, tag + "q", (seqs, layers, tokens, h, d)))
    lib = R.load_library()
    nbytes = lib.te_hip_attention_prefill_workspace_bytes(seqs, layers, tokens, base, ctx, h, kv, d)
    part = nbytes - lib.te_hip_value_t_bytes(seqs, layers, ctx, kv, d)
    splits = part // (seqs * layers * tokens * h * (d + 2) * 4) if part else 1
    assert part == 0 or part == splits * seqs * layers * tokens * h * (d + 2) * 4
    qd, kd, vd = f16_dev(q16), f16_dev(kc), f16_dev(vc)
    got = A.attention_prefill_split(qd, kd, vd, base_position=base).cpu().numpy()
    plain = A.attention_prefill(qd, kd, vd, base_position=base).cpu().numpy()
    worst = 0.0
    for s_ in range(seqs):
        for l_ in range(layers):
            want = oracle_mod.attention_prefill(S.f16_bits_to_f32(q16[s_, l_]).reshape(tokens, h, d),
                                                kc[s_, l_].copy(), vc[s_, l_].copy(), tokens, base, ctx, h, kv, d)
            worst = max(worst, maxabs(got[s_, l_], want.reshape(tokens, h, d)))
    drift = float(np.abs(got - plain).max())
    print(f"split prefill {seqs}x{layers} H{h} d{d} L{tokens} base{base}: {splits} splits, "
          f"max abs err {worst:.3e}, vs plain kernel {drift:.3e}")
    assert worst <= TOL
    assert drift <= TOL
    with pytest.raises(R.TinyEngineError):
        A.attention_prefill_split(qd, kd, vd, base_position=base,
                                  workspace=torch.empty(nbytes - 4, dtype=torch.uint8, device=DEV))


def test_prefill_several_sequences_and_layers(oracle_mod):
    """seqs x layers (seq, layer) units in one launch, each with its own data,
    chunk at base 50: every row of every unit against the oracle."""
    seqs, layers, h, kv, d, tokens, base = 2, 3, 16, 2, 128, 200, 50
    ctx = base + tokens + 7
    tag = "pfsl"
    kc = S.to_f16_bits(S.normal(27, tag + "k", (seqs, layers, ctx, kv, d)))
    vc = S.to_f16_bits(S.normal(27, tag + "v", (seqs, layers, ctx, kv, d)))
    q16 = S.to_f16_bits(S.normal(27, tag + "q", (seqs, layers, tokens, h, d)))
    out = A.attention_prefill(f16_dev(q16), f16_dev(kc), f16_dev(vc), base_position=base)
    got = out.cpu().numpy()
    worst = 0.0
    for s_ in range(seqs):
        for l_ in range(layers):
            want = oracle_mod.attention_prefill(S.f16_bits_to_f32(q16[s_, l_]).reshape(tokens, h, d),
                                                kc[s_, l_].copy(), vc[s_, l_].copy(), tokens, base, ctx, h, kv, d)
            worst = max(worst, maxabs(got[s_, l_], want.reshape(tokens, h, d)))
    print(f"prefill {seqs} seqs x {layers} layers, base {base}: max abs err {worst:.3e}")
    assert worst <= TOL


@pytest.mark.parametrize("seqs,layers,h,kv,d,tokens,base,bias", [
    (1, 1, 16, 2, 128, 300, 0, True),
    (2, 2, 14, 2, 64, 130, 37, True),
    (1, 2, 12, 2, 128, 200, 500, False),
])
def test_prefill_step_fused_vs_oracle(oracle_mod, monkeypatch, seqs, layers, h, kv, d, tokens, base, bias):
    """te_hip_attention_prefill_step_f16 == rope_kv_append (with q_half) +
    prefill, per the oracle: cache slots bit-exact, outputs within the bar,
    query/k/v untouched.  The unfused launch it is compared with bit for bit
    is forced to the kernel the fused step chooses (the rows kernel up to 512
    keys for fp32 queries, 256 for fp16 ones)."""
    ctx = base + tokens + 3
    tag = f"pfs{h}{kv}{d}{tokens}{base}"
    q = S.normal(28, tag + "q", (seqs, layers, tokens, h, d), 1 / math.sqrt(d))
    k = S.normal(28, tag + "k", (seqs, layers, tokens, kv, d))
    v = S.normal(28, tag + "v", (seqs, layers, tokens, kv, d))
    qb = S.normal(28, tag + "qb", (layers, h * d), 0.1) if bias else None
    kb = S.normal(28, tag + "kb", (layers, kv * d), 0.1) if bias else None
    vb = S.normal(28, tag + "vb", (layers, kv * d), 0.1) if bias else None
    kc0 = S.to_f16_bits(S.normal(28, tag + "kc", (seqs, layers, ctx, kv, d)))  # cached prefix (positions < base)
    vc0 = S.to_f16_bits(S.normal(28, tag + "vc", (seqs, layers, ctx, kv, d)))
    cos, sin = oracle_mod.rope_table(ctx, d, 1e6)
    q_o, k_o, v_o, kc_o, vc_o = q.copy(), k.copy(), v.copy(), kc0.copy(), vc0.copy()
    oracle_mod.rope_kv_append_f16(q_o, k_o, v_o, qb, kb, vb, cos, sin, kc_o, vc_o, seqs, layers, tokens, None, base,
                                  ctx, h, kv, d)
    q_half = S.to_f16_bits(q_o)  # the fp16 operand the unfused path stores
    tq, tk, tv = to_dev(q), to_dev(k), to_dev(v)
    dcos, dsin = A.rope_table(ctx, d, 1e6)
    kc, vc = f16_dev(kc0), f16_dev(vc0)
    out = A.prefill_step(tq, tk, tv, dcos, dsin, kc, vc, base_position=base,
                         q_bias=to_dev(qb) if bias else None, k_bias=to_dev(kb) if bias else None,
                         v_bias=to_dev(vb) if bias else None)
    torch.cuda.synchronize()
    assert np.array_equal(f16_host_bits(kc), kc_o) and np.array_equal(f16_host_bits(vc), vc_o)
    assert np.array_equal(tq.cpu().numpy(), q) and np.array_equal(tk.cpu().numpy(), k)
    assert np.array_equal(tv.cpu().numpy(), v)
    # same output bits as the unfused kernel on the stored fp16 queries
    monkeypatch.setenv("TE_HIP_PREFILL_ROWS", "1" if base + tokens <= 512 else "0")
    ref = A.attention_prefill(f16_dev(q_half), kc, vc, base_position=base)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    got = out.cpu().numpy()
    worst = 0.0
    for s_ in range(seqs):
        for l_ in range(layers):
            want = oracle_mod.attention_prefill(S.f16_bits_to_f32(q_half[s_, l_]).reshape(tokens, h, d),
                                                kc_o[s_, l_].copy(), vc_o[s_, l_].copy(), tokens, base, ctx, h, kv, d)
            worst = max(worst, maxabs(got[s_, l_], want.reshape(tokens, h, d)))
    print(f"fused prefill step H{h} KV{kv} d{d} L{tokens} base{base} x{seqs * layers}: max abs err {worst:.3e}")
    assert worst <= TOL


def test_prefill_full_size_4k_rows(oracle_mod):
    """BASELINE config 3 at L=4096 (fp16 Q/K/V ~ N(0,1), RoPE at 0..L-1, causal):
    strided rows against the oracle, plus row t == the decode kernel at position t."""
    h, kv, d, L, theta = 16, 2, 128, 4096, 1e6
    g = torch.Generator(device=DEV).manual_seed(S.SEED)
    q = torch.randn((1, 1, L, h, d), generator=g, device=DEV).half().float()
    k = torch.randn((1, 1, L, kv, d), generator=g, device=DEV).half().float()
    v = torch.randn((1, 1, L, kv, d), generator=g, device=DEV).half().float()
    dcos, dsin = A.rope_table(L, d, theta)
    kc = torch.zeros((1, 1, L, kv, d), dtype=torch.float16, device=DEV)
    vc = torch.zeros_like(kc)
    qh = torch.empty((1, 1, L, h, d), dtype=torch.float16, device=DEV)
    A.rope_kv_append(q, k, v, dcos, dsin, kc, vc, base_position=0, q_half=qh)
    out = A.attention_prefill(qh, kc, vc, base_position=0)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(L, h, d)
    rows = list(range(0, L, 257)) + [L - 1]
    want = oracle_mod.attention_prefill(q.cpu().numpy().reshape(L, h, d), f16_host_bits(kc[0, 0]),
                                        f16_host_bits(vc[0, 0]), L, 0, L, h, kv, d, 0, L, 257)
    want[L - 1] = oracle_mod.attention_prefill(q.cpu().numpy().reshape(L, h, d), f16_host_bits(kc[0, 0]),
                                               f16_host_bits(vc[0, 0]), L, 0, L, h, kv, d, L - 1, L, 1)[L - 1]
    err = max(maxabs(got[r], want[r]) for r in rows)
    print(f"prefill 3B L=4096 sampled rows: max abs err vs oracle (fp32 q) {err:.3e}")
    assert err <= TOL
    # Every row t of prefill == decode at position t (the split-K decode
    # kernel, pinned to the oracle to ~1e-7): with the same fp16 queries (the
    # prefill kernel's own error) and with the fp32 queries before their fp16
    # rounding (what a caller of the fp16-query entry point sees).
    worst_same = worst_fp32 = 0.0
    dec = torch.empty((1, 1, h, d), dtype=torch.float32, device=DEV)
    dec32 = torch.empty_like(dec)
    q16f = qh.float()
    for t in range(L):
        A.attention_decode(q16f[:, :, t].contiguous(), kc, vc, position=t, out=dec)
        A.attention_decode(q[:, :, t].contiguous(), kc, vc, position=t, out=dec32)
        worst_same = max(worst_same, float((dec[0, 0] - out[0, 0, t]).abs().max()))
        worst_fp32 = max(worst_fp32, float((dec32[0, 0] - out[0, 0, t]).abs().max()))
    print(f"prefill 3B L=4096, all {L} rows x {h} heads vs the decode kernel: max abs err {worst_same:.3e} "
          f"(same fp16 q), {worst_fp32:.3e} (fp32 q)")
    assert worst_same <= 1e-3 and worst_fp32 <= TOL


# ------------------------------------------------------------- fused step ---

@pytest.mark.parametrize("h,kv,d,layers,positions,bias", [
    (16, 2, 128, 2, [0, 63, 64, 1000], True),
    (14, 2, 64, 3, [512], False),
    (28, 4, 128, 1, [4095, 17, 2048], True),
])
def test_decode_step_fused_vs_oracle(oracle_mod, h, kv, d, layers, positions, bias):
    """te_hip_attention_decode_step_f16 == rope_kv_append + decode, per the oracle:
    cache slots bit-exact, outputs within the bar, inputs left untouched."""
    seqs = len(positions)
    ctx = max(positions) + 2
    tag = f"step{h}{kv}{d}{layers}{seqs}"
    q = S.normal(26, tag + "q", (seqs, layers, 1, h, d), 1 / math.sqrt(d))
    k = S.normal(26, tag + "k", (seqs, layers, 1, kv, d))
    v = S.normal(26, tag + "v", (seqs, layers, 1, kv, d))
    qb = S.normal(26, tag + "qb", (layers, h * d), 0.1) if bias else None
    kb = S.normal(26, tag + "kb", (layers, kv * d), 0.1) if bias else None
    vb = S.normal(26, tag + "vb", (layers, kv * d), 0.1) if bias else None
    kc0 = S.to_f16_bits(S.normal(26, tag + "kc", (seqs, layers, ctx, kv, d)))
    vc0 = S.to_f16_bits(S.normal(26, tag + "vc", (seqs, layers, ctx, kv, d)))
    cos, sin = oracle_mod.rope_table(ctx, d, 1e6)
    # oracle: append then decode
    q_o, k_o, v_o, kc_o, vc_o = q.copy(), k.copy(), v.copy(), kc0.copy(), vc0.copy()
    oracle_mod.rope_kv_append_f16(q_o, k_o, v_o, qb, kb, vb, cos, sin, kc_o, vc_o, seqs, layers, 1, positions, 0, ctx,
                                  h, kv, d)
    want = oracle_mod.attention_decode_f16kv(q_o[:, :, 0].copy(), kc_o, vc_o, positions, 0, seqs, layers, ctx, h, kv, d)
    # GPU fused step
    tq, tk, tv = to_dev(q), to_dev(k), to_dev(v)
    dcos, dsin = A.rope_table(ctx, d, 1e6)
    kc, vc = f16_dev(kc0), f16_dev(vc0)
    out = A.decode_step(tq, tk, tv, dcos, dsin, kc, vc, positions=positions,
                        q_bias=to_dev(qb) if bias else None, k_bias=to_dev(kb) if bias else None,
                        v_bias=to_dev(vb) if bias else None)
    torch.cuda.synchronize()
    assert np.array_equal(f16_host_bits(kc), kc_o) and np.array_equal(f16_host_bits(vc), vc_o)
    assert np.array_equal(tq.cpu().numpy(), q) and np.array_equal(tk.cpu().numpy(), k)
    err = maxabs(out.cpu().numpy(), want)
    print(f"fused decode step H{h} KV{kv} d{d} layers{layers} positions={positions}: max abs err {err:.3e}")
    assert err <= TOL
    # the fused split-K launch alone, repeated (idempotent append), then the
    # combine: the same output bits and the same cache
    ws = A.decode_workspace(seqs, layers, h, kv, d, positions=positions)
    out2 = torch.empty_like(out)
    for _ in range(2):
        A.decode_step(tq, tk, tv, dcos, dsin, kc, vc, positions=positions,
                      q_bias=to_dev(qb) if bias else None, k_bias=to_dev(kb) if bias else None,
                      v_bias=to_dev(vb) if bias else None, workspace=ws, stage="splitk")
    A.attention_decode(tq, kc, vc, positions=positions, out=out2, workspace=ws, stage="combine")
    torch.cuda.synchronize()
    assert torch.equal(out2, out)
    assert np.array_equal(f16_host_bits(kc), kc_o) and np.array_equal(f16_host_bits(vc), vc_o)


# ------------------------------------------------------------ HIP graphs ---

def test_decode_step_graph_replay():
    """The per-layer fused decode step captured in one HIP graph: every replay
    (with eager work and synchronisation between replays) reproduces the eager
    launches bit for bit, and the appended cache slots stay identical."""
    h, kv, d, layers, pos = 16, 2, 128, 4, 777
    ctx = pos + 1
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn((1, layers, 1, h, d), generator=g, device="cuda") / math.sqrt(d)
    k = torch.randn((1, layers, 1, kv, d), generator=g, device="cuda")
    v = torch.randn((1, layers, 1, kv, d), generator=g, device="cuda")
    kc = torch.randn((1, layers, ctx, kv, d), generator=g, device="cuda").half()
    vc = torch.randn((1, layers, ctx, kv, d), generator=g, device="cuda").half()
    cos, sin = A.rope_table(ctx, d, 1e6)
    ws = A.decode_workspace(1, 1, h, kv, d, position=pos)
    out = torch.empty((1, layers, h, d), dtype=torch.float32, device="cuda")

    def run():
        for l in range(layers):
            A.decode_step(q[:, l:l + 1], k[:, l:l + 1], v[:, l:l + 1], cos, sin, kc[:, l:l + 1], vc[:, l:l + 1],
                          position=pos, out=out[:, l:l + 1], workspace=ws)

    run()
    torch.cuda.synchronize()
    eager = out.clone()
    kc_eager, vc_eager = kc.clone(), vc.clone()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for rep in range(4):
        out.fill_(float(rep + 1))       # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager launches"
        assert torch.equal(kc, kc_eager) and torch.equal(vc, vc_eager)
    print(f"graph of {2 * layers} launches: 4 replays identical to eager")


def test_calibration_kernel_runs():
    """The measurement-only MFMA loop behind bench.py's ceilings launches and
    writes every output element (the buffer starts as NaN)."""
    lib = R.load_library()
    blocks, iters = 4, 3
    out = torch.full((blocks * 512,), float("nan"), dtype=torch.float32, device="cuda")
    R.check(lib.te_hip_calibrate_mfma_f16(blocks, iters, out.data_ptr(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()


# ----------------------------------------------------- V^T prefill paths ---

@pytest.mark.parametrize("seqs,layers,ctx,kv,d,first,count", [
    (1, 1, 300, 2, 128, 0, 300),     # whole cache, ctx not a multiple of 8 or 64
    (2, 3, 130, 4, 64, 5, 100),      # unaligned range, zero tail 105..111
    (1, 2, 1000, 2, 128, 937, 61),   # tail range ending at the cache end
    (1, 1, 64, 2, 128, 10, 0),       # nothing to do
])
def test_value_transpose_bits(seqs, layers, ctx, kv, d, first, count):
    """te_hip_value_transpose_f16: V^T[.., i, p] = V[.., p, .., i] bit for bit over
    [first, first + count), 0 from there to the next multiple of 8, every
    other position untouched."""
    g = torch.Generator(device=DEV).manual_seed(ctx + first)
    vc = torch.randn((seqs, layers, ctx, kv, d), generator=g, device=DEV).half()
    vt = A.value_t_buffer(seqs, layers, ctx, kv, d)
    pad = vt.shape[-1]
    assert pad % 64 == 0 and pad >= ctx
    vt.fill_(7.0)
    A.value_transpose(vc, vt, first_position=first, count=count)
    torch.cuda.synchronize()
    want = torch.full_like(vt, 7.0)
    end = first + count
    want[..., first:end] = vc.permute(0, 1, 3, 4, 2)[..., first:end]
    if count:
        want[..., end:min((end + 7) // 8 * 8, pad)] = 0.0
    assert torch.equal(vt.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("seqs,layers,h,kv,d,tokens,base", [
    (1, 1, 16, 2, 128, 300, 0),      # 3 tiles: the lone middle tile and a pair
    (1, 1, 16, 2, 128, 130, 200),    # chunk after a cached prefix
    (1, 1, 16, 2, 128, 1, 0),        # one row
    (1, 1, 14, 2, 64, 200, 37),      # head_dim 64, unaligned base
    (2, 3, 12, 2, 128, 129, 1000),   # several (seq, layer) units, long prefix
    (1, 1, 28, 4, 128, 257, 3),      # 7B grouping
])
def test_prefill_vt_vs_oracle(oracle_mod, seqs, layers, h, kv, d, tokens, base):
    """te_hip_attention_prefill_vt_f16 over V^T from te_hip_value_transpose_f16,
    with one split and with the library's key split, against the oracle for
    every row; one split is bit-identical to the plain-cache entry point."""
    ctx = base + tokens + 5
    tag = f"pvt{seqs}{layers}{h}{d}{tokens}{base}"
    kc = S.to_f16_bits(S.normal(43, tag + "k", (seqs, layers, ctx, kv, d)))
    vc = S.to_f16_bits(S.normal(43, tag + "v", (seqs, layers, ctx, kv, d)))
    q16 = S.to_f16_bits(S.normal(43, tag + "q", (seqs, layers, tokens, h, d)))
    qd, kd, vd = f16_dev(q16), f16_dev(kc), f16_dev(vc)
    vt = A.value_t_buffer(seqs, layers, ctx, kv, d)
    A.value_transpose(vd, vt, first_position=0, count=base + tokens)
    ws = A.prefill_vt_workspace(seqs, layers, tokens, h, kv, d, base_position=base, context_tokens=ctx)
    one = A.attention_prefill_vt(qd, kd, vt, base_position=base).cpu().numpy()
    split = A.attention_prefill_vt(qd, kd, vt, base_position=base, workspace=ws).cpu().numpy()
    plain = A.attention_prefill(qd, kd, vd, base_position=base).cpu().numpy()
    assert np.array_equal(one, plain)
    worst = 0.0
    for s_ in range(seqs):
        for l_ in range(layers):
            want = oracle_mod.attention_prefill(S.f16_bits_to_f32(q16[s_, l_]).reshape(tokens, h, d),
                                                kc[s_, l_].copy(), vc[s_, l_].copy(), tokens, base, ctx, h, kv, d)
            want = want.reshape(tokens, h, d)
            worst = max(worst, maxabs(one[s_, l_], want), maxabs(split[s_, l_], want))
    nsplit = 1 if ws is None else ws.numel() // (seqs * layers * tokens * h * (d + 2) * 4)
    print(f"prefill V^T {seqs}x{layers} H{h} KV{kv} d{d} L{tokens} base{base} ({nsplit} splits): "
          f"max abs err {worst:.3e}")
    assert worst <= TOL


@pytest.mark.parametrize("seqs,layers,h,kv,d,tokens,base,bias", [
    (1, 1, 16, 2, 128, 300, 0, True),
    (2, 2, 14, 2, 64, 130, 37, True),
    (1, 2, 12, 2, 128, 200, 500, False),
])
def test_prefill_step_vt_matches_plain_step(seqs, layers, h, kv, d, tokens, base, bias):
    """te_hip_attention_prefill_step_vt_f16 (caller V^T, key split) against
    te_hip_attention_prefill_step_f16 (library V^T, one split): the same cache
    bits, V^T equal to the transposed value cache over positions
    0 .. base + tokens - 1, and the same output (bit for bit without a split,
    within the bar with one)."""
    ctx = base + tokens + 3
    g = torch.Generator(device=DEV).manual_seed(tokens + base)
    q = torch.randn((seqs, layers, tokens, h, d), generator=g, device=DEV) / math.sqrt(d)
    k = torch.randn((seqs, layers, tokens, kv, d), generator=g, device=DEV)
    v = torch.randn((seqs, layers, tokens, kv, d), generator=g, device=DEV)
    qb = torch.randn((layers, h * d), generator=g, device=DEV) * 0.1 if bias else None
    kb = torch.randn((layers, kv * d), generator=g, device=DEV) * 0.1 if bias else None
    vb = torch.randn((layers, kv * d), generator=g, device=DEV) * 0.1 if bias else None
    kc0 = torch.randn((seqs, layers, ctx, kv, d), generator=g, device=DEV).half()
    vc0 = torch.randn((seqs, layers, ctx, kv, d), generator=g, device=DEV).half()
    cos, sin = A.rope_table(ctx, d, 1e6)
    kc1, vc1 = kc0.clone(), vc0.clone()
    ref = A.prefill_step(q, k, v, cos, sin, kc1, vc1, base_position=base, q_bias=qb, k_bias=kb, v_bias=vb)
    kc2, vc2 = kc0.clone(), vc0.clone()
    vt = A.value_t_buffer(seqs, layers, ctx, kv, d)
    A.value_transpose(vc2, vt, first_position=0, count=base)  # the cached prefix
    one = A.prefill_step_vt(q, k, v, cos, sin, kc2, vc2, vt, base_position=base, q_bias=qb, k_bias=kb, v_bias=vb)
    torch.cuda.synchronize()
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16))
    n = base + tokens
    assert torch.equal(vt[..., :n].view(torch.int16), vc2.permute(0, 1, 3, 4, 2)[..., :n].view(torch.int16))
    assert torch.equal(one, ref)
    ws = A.prefill_vt_workspace(seqs, layers, tokens, h, kv, d, base_position=base, context_tokens=ctx)
    kc3, vc3 = kc0.clone(), vc0.clone()
    vt3 = A.value_t_buffer(seqs, layers, ctx, kv, d)
    A.value_transpose(vc3, vt3, first_position=0, count=base)
    split = A.prefill_step_vt(q, k, v, cos, sin, kc3, vc3, vt3, base_position=base, q_bias=qb, k_bias=kb,
                              v_bias=vb, workspace=ws)
    torch.cuda.synchronize()
    err = float((split - ref).abs().max())
    print(f"fused step V^T H{h} d{d} L{tokens} base{base}: split vs one split {err:.3e}")
    assert err <= TOL


def _off16(t):
    """A contiguous copy of t whose data pointer is one element past 16-byte alignment."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    view = buf[1:].view(t.shape)
    view.copy_(t)
    assert view.data_ptr() % 16 != 0
    return view


def test_prefill_step_vt_misaligned_kv_rows():
    """k_new / v_new one float off 16-byte alignment: the fused V^T step takes
    the element-wise append and the chunk's transpose instead of the 16-byte
    kernel, with the same cache, V^T and output bits as aligned rows.  A query,
    cache, V^T or output off alignment is refused (UNSUPPORTED), as is a
    misaligned value cache in te_hip_value_transpose_f16."""
    seqs, layers, h, kv, d, tokens, base = 1, 2, 16, 2, 128, 200, 37
    ctx = base + tokens + 3
    g = torch.Generator(device=DEV).manual_seed(11)
    q = torch.randn((seqs, layers, tokens, h, d), generator=g, device=DEV) / math.sqrt(d)
    k = torch.randn((seqs, layers, tokens, kv, d), generator=g, device=DEV)
    v = torch.randn((seqs, layers, tokens, kv, d), generator=g, device=DEV)
    qb = torch.randn((layers, h * d), generator=g, device=DEV) * 0.1
    kb = torch.randn((layers, kv * d), generator=g, device=DEV) * 0.1
    vb = torch.randn((layers, kv * d), generator=g, device=DEV) * 0.1
    kc0 = torch.randn((seqs, layers, ctx, kv, d), generator=g, device=DEV).half()
    vc0 = torch.randn((seqs, layers, ctx, kv, d), generator=g, device=DEV).half()
    cos, sin = A.rope_table(ctx, d, 1e6)

    def run(kk, vv):
        kc, vc = kc0.clone(), vc0.clone()
        vt = A.value_t_buffer(seqs, layers, ctx, kv, d)
        A.value_transpose(vc, vt, first_position=0, count=base)
        out = A.prefill_step_vt(q, kk, vv, cos, sin, kc, vc, vt, base_position=base, q_bias=qb, k_bias=kb,
                                v_bias=vb)
        torch.cuda.synchronize()
        return kc, vc, vt, out

    ref = run(k, v)
    got = run(_off16(k), _off16(v))
    for x, y in zip(ref[:3], got[:3]):
        assert torch.equal(x.view(torch.int16), y.view(torch.int16))
    assert torch.equal(ref[3], got[3])

    kc, vc = kc0.clone(), vc0.clone()
    vt = A.value_t_buffer(seqs, layers, ctx, kv, d)
    with pytest.raises(R.TinyEngineError, match="unsupported"):
        A.prefill_step_vt(_off16(q), k, v, cos, sin, kc, vc, vt, base_position=base)
    with pytest.raises(R.TinyEngineError, match="unsupported"):
        A.prefill_step_vt(q, k, v, cos, sin, kc, vc, vt, base_position=base, out=_off16(torch.empty_like(q)))
    qh = q.half()
    with pytest.raises(R.TinyEngineError, match="unsupported"):
        A.attention_prefill_vt(qh, _off16(kc), vt, base_position=base)
    with pytest.raises(R.TinyEngineError, match="unsupported"):
        A.attention_prefill(_off16(qh), kc, vc, base_position=base)
    with pytest.raises(R.TinyEngineError, match="unsupported"):
        A.value_transpose(_off16(vc), vt, first_position=0, count=base)


@pytest.mark.parametrize("tokens,base", [(300, 0), (130, 203), (1, 5)])
def test_prefill_vt_ignores_positions_past_rounded_end(oracle_mod, tokens, base):
    """V^T positions at and past base + tokens rounded up to 8 are never read
    as values.  V^T is filled with fp16 NaN (0x7E00) before the writers run
    (te_hip_value_transpose_f16 and the fused step write the positions up to
    the end and zeros up to the next multiple of 8); the outputs, with one
    split and with the key split, are finite, match the oracle and equal the
    outputs over a zero-filled V^T."""
    h, kv, d = 16, 2, 128
    end = base + tokens
    ctx = end + 40
    tag = f"nanvt{tokens}{base}"
    kc = S.to_f16_bits(S.normal(47, tag + "k", (1, 1, ctx, kv, d)))
    vc = S.to_f16_bits(S.normal(47, tag + "v", (1, 1, ctx, kv, d)))
    q16 = S.to_f16_bits(S.normal(47, tag + "q", (1, 1, tokens, h, d)))
    qd, kd, vd = f16_dev(q16), f16_dev(kc), f16_dev(vc)
    vt_nan = A.value_t_buffer(1, 1, ctx, kv, d)
    vt_nan.view(torch.int16).fill_(0x7E00)
    A.value_transpose(vd, vt_nan, first_position=0, count=end)
    end8 = (end + 7) // 8 * 8
    assert torch.isnan(vt_nan[..., end8:]).all() and not torch.isnan(vt_nan[..., :end8]).any()
    vt_zero = A.value_t_buffer(1, 1, ctx, kv, d)
    A.value_transpose(vd, vt_zero, first_position=0, count=end)
    ws = A.prefill_vt_workspace(1, 1, tokens, h, kv, d, base_position=base, context_tokens=ctx)
    want = oracle_mod.attention_prefill(S.f16_bits_to_f32(q16[0, 0]).reshape(tokens, h, d), kc[0, 0].copy(),
                                        vc[0, 0].copy(), tokens, base, ctx, h, kv, d).reshape(tokens, h, d)
    one = A.attention_prefill_vt(qd, kd, vt_nan, base_position=base)
    split = A.attention_prefill_vt(qd, kd, vt_nan, base_position=base, workspace=ws)
    zero = A.attention_prefill_vt(qd, kd, vt_zero, base_position=base)
    torch.cuda.synchronize()
    assert torch.isfinite(one).all() and torch.isfinite(split).all()
    assert torch.equal(one, zero)
    err = max(maxabs(one.cpu().numpy()[0, 0], want), maxabs(split.cpu().numpy()[0, 0], want))

    # the fused step over a NaN-filled V^T holding only the cached prefix
    g = torch.Generator(device=DEV).manual_seed(tokens + base)
    qf = torch.randn((1, 1, tokens, h, d), generator=g, device=DEV) / math.sqrt(d)
    kf = torch.randn((1, 1, tokens, kv, d), generator=g, device=DEV)
    vf = torch.randn((1, 1, tokens, kv, d), generator=g, device=DEV)
    cos, sin = A.rope_table(ctx, d, 1e6)
    outs = []
    for fill, work in ((0x7E00, None), (0x7E00, ws), (0, None)):
        kc2, vc2 = kd.clone(), vd.clone()
        vt2 = A.value_t_buffer(1, 1, ctx, kv, d)
        vt2.view(torch.int16).fill_(fill)
        A.value_transpose(vc2, vt2, first_position=0, count=base)
        outs.append(A.prefill_step_vt(qf, kf, vf, cos, sin, kc2, vc2, vt2, base_position=base, workspace=work))
    torch.cuda.synchronize()
    assert all(torch.isfinite(o).all() for o in outs)
    assert torch.equal(outs[0], outs[2])
    err_step = float((outs[1] - outs[2]).abs().max())
    print(f"NaN past the rounded V^T end, L{tokens} base{base}: max abs err {err:.3e} (oracle), "
          f"fused step split vs one split {err_step:.3e}")
    assert err <= TOL and err_step <= TOL


@pytest.mark.parametrize("kernel,tokens,base", [("tile", 300, 20), ("rows", 300, 20), ("rows", 300, 700)])
@pytest.mark.parametrize("growth", [0.0, 0.02, 0.1, 0.2])
def test_prefill_rising_scores_rescale(oracle_mod, monkeypatch, growth, kernel, tokens, base):
    """Scores that keep rising along the keys (key p scaled by 1 + growth * p /
    16, q = k direction shared), so later blocks exceed an earlier reference by
    far more than 2^16 in the weights: the exact rescale path must run, with
    and without a key split, and every row must still match the oracle.  Each
    kernel forced: the tile kernel, and the rows kernel with one block per
    wave (320 keys: the waves' references differ and only the merge rescales)
    and with two (1,000 keys: a wave's second block raises its reference)."""
    monkeypatch.setenv("TE_HIP_PREFILL_ROWS", "1" if kernel == "rows" else "0")
    h, kv, d = 4, 1, 128
    ctx = base + tokens
    g = np.random.default_rng(5)
    dirn = g.standard_normal(d).astype(np.float32)
    dirn /= np.linalg.norm(dirn)
    k = (g.standard_normal((ctx, kv, d)) * 0.3 + dirn * 8.0).astype(np.float32)
    k *= (1.0 + growth * np.arange(ctx, dtype=np.float32) / 16.0)[:, None, None]
    v = g.standard_normal((ctx, kv, d)).astype(np.float32)
    q = (g.standard_normal((tokens, h, d)) * 0.3 + dirn * 8.0).astype(np.float32)
    kc, vc, q16 = S.to_f16_bits(k), S.to_f16_bits(v), S.to_f16_bits(q)
    want = oracle_mod.attention_prefill(S.f16_bits_to_f32(q16), kc, vc, tokens, base, ctx, h, kv, d)
    qd = f16_dev(q16.reshape(1, 1, tokens, h, d))
    kd = f16_dev(kc.reshape(1, 1, ctx, kv, d))
    vd = f16_dev(vc.reshape(1, 1, ctx, kv, d))
    vt = A.value_t_buffer(1, 1, ctx, kv, d)
    A.value_transpose(vd, vt)
    ws = A.prefill_vt_workspace(1, 1, tokens, h, kv, d, base_position=base, context_tokens=ctx)
    one = A.attention_prefill_vt(qd, kd, vt, base_position=base).cpu().numpy().reshape(tokens, h, d)
    split = A.attention_prefill_vt(qd, kd, vt, base_position=base, workspace=ws).cpu().numpy().reshape(tokens, h, d)
    assert np.isfinite(one).all() and np.isfinite(split).all()
    err = max(maxabs(one, want), maxabs(split, want))
    print(f"prefill rising scores ({kernel}, L{tokens} base{base}, growth {growth}): max abs err {err:.3e}")
    assert err <= TOL

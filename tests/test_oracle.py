"""Pins the CPU oracle (oracle/te_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something other than its own formula:
the reference's known-answer tests (c/tests/kernel_ops.c:330-356), golden
vectors written by the reference's own compiled ops.c (tests/golden), the
compiled reference directly when it was built here (oracle/_ref), fp64 brute
force, exhaustive fp16 enumeration and closed-form invariants.
"""
import math

import numpy as np
import pytest

import _synth as S
import cases as C

F32 = np.float32


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- fp16 ------

def test_f16_to_f32_exhaustive(oracle_mod):
    b = np.arange(65536, dtype=np.uint16)
    got = oracle_mod.f16_to_f32(b)
    want = b.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])


def test_f32_to_f16_roundtrip_exhaustive(oracle_mod):
    b = np.arange(65536, dtype=np.uint16)
    f = oracle_mod.f16_to_f32(b)
    back = oracle_mod.f32_to_f16(f)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], b[~nan])
    assert np.all((back[nan] & 0x7C00) == 0x7C00) and np.all((back[nan] & 0x3FF) != 0)


def test_f32_to_f16_ties_to_even(oracle_mod):
    # midpoints between consecutive finite fp16 values are exact in fp32
    b = np.arange(0, 0x7BFF, dtype=np.uint16)
    lo = b.view(np.float16).astype(np.float64)
    hi = (b + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    assert np.array_equal(mid.astype(np.float64), (lo + hi) / 2)
    got = oracle_mod.f32_to_f16(mid)
    want = np.where(b % 2 == 0, b, b + 1).astype(np.uint16)
    assert np.array_equal(got, want)
    got_neg = oracle_mod.f32_to_f16(-mid)
    assert np.array_equal(got_neg, want | 0x8000)


def test_f32_to_f16_edges(oracle_mod):
    cases = {
        65504.0: 0x7BFF, 65519.996: 0x7BFF, 65520.0: 0x7C00, 1e9: 0x7C00, float("inf"): 0x7C00,
        2.0 ** -24: 0x0001, 2.0 ** -25: 0x0000, 2.0 ** -25 * 1.0000001: 0x0001, 3 * 2.0 ** -25: 0x0002,
        2.0 ** -14: 0x0400, 0.0: 0x0000, 1.0: 0x3C00, 2.0 ** -26: 0x0000,
    }
    for x, want in cases.items():
        assert int(oracle_mod.f32_to_f16(np.array([x], F32))[0]) == want, x
        assert int(oracle_mod.f32_to_f16(np.array([-x], F32))[0]) == want | 0x8000, -x


def test_f32_to_f16_random_vs_numpy(oracle_mod):
    r = np.random.default_rng(7)
    x = r.integers(0, 2 ** 32, size=1 << 22, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[np.isfinite(x)]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle_mod.f32_to_f16(x), want)


# ---------------------------------------------------------------- RoPE ------

def test_rope_reference_kat(oracle_mod):
    # reference c/tests/kernel_ops.c:330-339
    v = oracle_mod.rope_f32(np.array([1, 2, 3, 4], F32), 1, 4, 1, 10000.0)
    s0, c0, s1, c1 = math.sin(1.0), math.cos(1.0), math.sin(0.01), math.cos(0.01)
    assert abs(v[0] - (1 * c0 - 3 * s0)) <= 1e-6
    assert abs(v[2] - (3 * c0 + 1 * s0)) <= 1e-6
    assert abs(v[1] - (2 * c1 - 4 * s1)) <= 1e-6
    assert abs(v[3] - (4 * c1 + 2 * s1)) <= 1e-6


def test_rope_golden(oracle_mod, golden):
    data, meta = golden
    for name, heads, d, pos, theta in C.ROPE_CASES:
        x = C.rope_input(name, heads, d)
        assert S.digest(x) == meta["rope"][name]["input_sha256"]
        got = oracle_mod.rope_f32(x, heads, d, pos, theta)
        assert np.array_equal(bits(got), bits(data[f"rope/{name}"])), name


def test_rope_table_golden_rows(oracle_mod, golden):
    data, meta = golden
    positions = meta["rope_rows"]["positions"]
    for d in (64, 128):
        cos, sin = oracle_mod.rope_table(max(positions) + 1, d, 1e6)
        rows = data[f"rope_rows/d{d}"]
        for i, p in enumerate(positions):
            assert np.array_equal(bits(cos[p]), bits(rows[i, : d // 2])), (d, p)
            assert np.array_equal(bits(sin[p]), bits(rows[i, d // 2:])), (d, p)


def test_rope_cached_equals_rope(oracle_mod):
    cos, sin = oracle_mod.rope_table(9000, 128, 1e6)
    for p in (0, 1, 777, 8191, 8999):
        x = S.normal(1, f"rc{p}", (16 * 128,))
        a = oracle_mod.rope_f32(x, 16, 128, p, 1e6)
        b = oracle_mod.rope_cached(x, 16, 128, cos, sin, p)
        assert np.array_equal(bits(a), bits(b)), p


def test_rope_closed_forms(oracle_mod):
    x = S.normal(2, "cf", (12 * 128,))
    assert np.array_equal(bits(oracle_mod.rope_f32(x, 12, 128, 0, 1e6)), bits(x))  # position 0: identity
    y = oracle_mod.rope_f32(x, 12, 128, 4321, 1e6).reshape(12, 2, 64).astype(np.float64)
    xx = x.reshape(12, 2, 64).astype(np.float64)
    np.testing.assert_allclose((y ** 2).sum(1), (xx ** 2).sum(1), rtol=1e-5, atol=1e-6)  # pair norms
    # a plausible mistake -- rotating the adjacent (interleaved) pair instead of (i, i+d/2) -- breaks the KAT
    v = np.array([1, 2, 3, 4], np.float64)
    wrong0 = v[0] * math.cos(1.0) - v[1] * math.sin(1.0)
    assert abs(oracle_mod.rope_f32(v.astype(F32), 1, 4, 1, 1e4)[0] - wrong0) > 1e-2


def test_rope_argument_checks(oracle_mod):
    x = np.ones(8, F32)
    assert oracle_mod.rope_status(None, 1, 8, 0, 1e6) == 1
    assert oracle_mod.rope_status(x, 0, 8, 0, 1e6) == 1
    assert oracle_mod.rope_status(x, 1, 0, 0, 1e6) == 1
    assert oracle_mod.rope_status(x, 1, 7, 0, 1e6) == 1
    assert oracle_mod.rope_status(x, 1, 8, 0, 0.0) == 1
    assert oracle_mod.rope_status(x, 1, 8, 0, -1.0) == 1


@pytest.mark.skipif(not __import__("oracle").REF_LIB.is_file(), reason="reference ops.c not built here")
def test_rope_vs_compiled_reference(oracle_mod):
    r = np.random.default_rng(3)
    for _ in range(20):
        d = int(r.choice([2, 4, 64, 128, 256]))
        heads = int(r.integers(1, 20))
        pos = int(r.integers(0, 200000))
        theta = float(r.choice([1e4, 1e6, 5e5]))
        x = S.normal(3, f"ref{pos}", (heads * d,))
        a = oracle_mod.rope_f32(x, heads, d, pos, theta)
        b = oracle_mod.rope_f32(x, heads, d, pos, theta, use_ref=True)
        assert np.array_equal(bits(a), bits(b))
    for args in ((np.ones(8, F32), 1, 7, 0, 1e6), (np.ones(8, F32), 1, 8, 0, 0.0)):
        assert oracle_mod.rope_status(*args) == oracle_mod.rope_status(*args, use_ref=True)


# ---------------------------------------------------------- attention -------

def brute_force_decode(q, k, v, pos, heads, kv_heads, d):
    """fp64 attention from the definition, independent of loop order."""
    q = q.reshape(heads, d).astype(np.float64)
    k = k.reshape(-1, kv_heads, d)[: pos + 1].astype(np.float64)
    v = v.reshape(-1, kv_heads, d)[: pos + 1].astype(np.float64)
    group = heads // kv_heads
    out = np.empty((heads, d))
    for h in range(heads):
        s = k[:, h // group, :] @ q[h] / math.sqrt(d)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ v[:, h // group, :]
    return out.reshape(-1)


def test_decode_reference_kat(oracle_mod):
    # reference c/tests/kernel_ops.c:341-356
    out = oracle_mod.attention_decode_f32(np.array([1, 0, 0, 1], F32), np.array([1, 0, 0, 1], F32),
                                          np.array([10, 20, 30, 40], F32), 1, 2, 1, 2)
    sc = 1 / math.sqrt(2)
    hi, lo = math.exp(sc), 1.0
    wh, wl = hi / (hi + lo), lo / (hi + lo)
    want = [wh * 10 + wl * 30, wh * 20 + wl * 40, wl * 10 + wh * 30, wl * 20 + wh * 40]
    np.testing.assert_allclose(out, want, atol=1e-5, rtol=0)


def test_decode_golden(oracle_mod, golden):
    data, meta = golden
    for case in C.DECODE_CASES:
        q, kb, vb = C.decode_inputs(case)
        assert S.digest(q, kb, vb) == meta["decode"][case["name"]]["input_sha256"], case["name"]
        got = oracle_mod.attention_decode_f32(q, S.f16_bits_to_f32(kb), S.f16_bits_to_f32(vb), case["pos"],
                                              case["heads"], case["kv"], case["d"])
        assert np.array_equal(bits(got), bits(data[f"decode/{case['name']}"])), case["name"]


def test_decode_brute_force(oracle_mod):
    for (h, kv, d, pos) in ((2, 1, 2, 1), (4, 2, 8, 5), (14, 2, 64, 40), (12, 2, 128, 17), (7, 7, 16, 9)):
        q = S.normal(5, f"bf{h}{pos}", (h * d,), 0.3)
        k = S.normal(5, f"bfk{h}{pos}", ((pos + 1) * kv * d,))
        v = S.normal(5, f"bfv{h}{pos}", ((pos + 1) * kv * d,))
        got = oracle_mod.attention_decode_f32(q, k, v, pos, h, kv, d)
        np.testing.assert_allclose(got, brute_force_decode(q, k, v, pos, h, kv, d), atol=1e-5, rtol=1e-5)


def test_decode_invariants(oracle_mod):
    h, kv, d = 16, 2, 128
    q = S.normal(6, "inv_q", (h * d,))
    k = S.normal(6, "inv_k", (300 * kv * d,))
    v = S.normal(6, "inv_v", (300 * kv * d,))
    # one key -> V[0] exactly
    out = oracle_mod.attention_decode_f32(q, k, v, 0, h, kv, d).reshape(h, d)
    for hh in range(h):
        assert np.array_equal(bits(out[hh]), bits(v.reshape(-1, kv, d)[0, hh // 8]))
    # constant V along positions -> that constant
    vc = np.tile(S.normal(6, "inv_vc", (1, kv, d)), (300, 1, 1)).reshape(-1)
    out = oracle_mod.attention_decode_f32(q, k, vc, 299, h, kv, d).reshape(h, d)
    for hh in range(h):
        np.testing.assert_allclose(out[hh], vc.reshape(-1, kv, d)[0, hh // 8], atol=1e-5)
    # heads of one group with equal queries give equal outputs
    qe = q.reshape(h, d).copy()
    qe[1:8] = qe[0]
    out = oracle_mod.attention_decode_f32(qe.reshape(-1), k, v, 299, h, kv, d).reshape(h, d)
    for hh in range(1, 8):
        assert np.array_equal(bits(out[hh]), bits(out[0]))


def test_decode_argument_checks(oracle_mod):
    lib = oracle_mod.lib()
    a = np.ones(64, F32)
    p = a.ctypes.data_as(__import__("ctypes").POINTER(__import__("ctypes").c_float))
    assert lib.orc_attention_decode_f32(p, p, p, 0, 3, 2, 4, p) == 1   # heads % kv_heads
    assert lib.orc_attention_decode_f32(None, p, p, 0, 2, 1, 4, p) == 1
    assert lib.orc_attention_decode_f32(p, p, p, 0, 0, 1, 4, p) == 1
    assert lib.orc_attention_decode_f32(p, p, p, 2 ** 64 - 1, 2, 1, 4, p) == 3  # position == SIZE_MAX


@pytest.mark.skipif(not __import__("oracle").REF_LIB.is_file(), reason="reference ops.c not built here")
def test_decode_vs_compiled_reference(oracle_mod):
    for (h, kv, d, pos) in ((14, 2, 64, 1030), (16, 2, 128, 64), (28, 4, 128, 513), (12, 2, 128, 2000)):
        q = S.normal(8, f"r{h}{pos}", (h * d,), 0.2)
        k = S.f16_bits_to_f32(S.to_f16_bits(S.normal(8, f"rk{h}{pos}", ((pos + 1) * kv * d,))))
        v = S.f16_bits_to_f32(S.to_f16_bits(S.normal(8, f"rv{h}{pos}", ((pos + 1) * kv * d,))))
        a = oracle_mod.attention_decode_f32(q, k, v, pos, h, kv, d)
        b = oracle_mod.attention_decode_f32(q, k, v, pos, h, kv, d, use_ref=True)
        assert np.array_equal(bits(a), bits(b))


# ------------------------------------------------ append / compositions -----

def test_append_slot_formula(oracle_mod):
    """Position-tagged values land at (((s*L + layer)*ctx + pos)*kv + h)*d + i."""
    seqs, layers, tokens, ctx, h, kv, d = 3, 2, 4, 40, 4, 2, 8
    bases = [0, 17, 36]
    q = np.zeros((seqs, layers, tokens, h, d), F32)
    k = np.zeros((seqs, layers, tokens, kv, d), F32)
    v = np.zeros((seqs, layers, tokens, kv, d), F32)
    for s in range(seqs):
        for layer in range(layers):
            for b in range(tokens):
                for kh in range(kv):
                    v[s, layer, b, kh] = (((s * layers + layer) * tokens + b) * kv + kh) * d + np.arange(d)
    cos, sin = oracle_mod.rope_table(ctx, d, 1e6)
    kc = np.full((seqs, layers, ctx, kv, d), 0xFFFF, np.uint16)
    vc = kc.copy()
    oracle_mod.rope_kv_append_f16(q, k, v, None, None, None, cos, sin, kc, vc, seqs, layers, tokens, bases, 0,
                                  ctx, h, kv, d)
    got = S.f16_bits_to_f32(vc)
    for s in range(seqs):
        for layer in range(layers):
            for p in range(ctx):
                b = p - bases[s]
                if 0 <= b < tokens:
                    assert np.array_equal(got[s, layer, p], v[s, layer, b])
                else:
                    assert np.all(vc[s, layer, p] == 0xFFFF)


def test_append_rotation_matches_rope_cached(oracle_mod):
    seqs, layers, tokens, ctx, h, kv, d = 1, 2, 5, 64, 16, 2, 128
    q = S.normal(9, "aq", (seqs, layers, tokens, h, d))
    k = S.normal(9, "ak", (seqs, layers, tokens, kv, d))
    v = S.normal(9, "av", (seqs, layers, tokens, kv, d))
    qb = S.normal(9, "aqb", (layers, h * d), 0.1)
    kb = S.normal(9, "akb", (layers, kv * d), 0.1)
    vb = S.normal(9, "avb", (layers, kv * d), 0.1)
    cos, sin = oracle_mod.rope_table(ctx, d, 1e6)
    kc = np.zeros((seqs, layers, ctx, kv, d), np.uint16)
    vc = np.zeros_like(kc)
    q2, k2, v2 = q.copy(), k.copy(), v.copy()
    oracle_mod.rope_kv_append_f16(q2, k2, v2, qb, kb, vb, cos, sin, kc, vc, seqs, layers, tokens, None, 30, ctx,
                                  h, kv, d)
    for layer in range(layers):
        for b in range(tokens):
            want_q = oracle_mod.rope_cached((q[0, layer, b].reshape(-1) + qb[layer]), h, d, cos, sin, 30 + b)
            want_k = oracle_mod.rope_cached((k[0, layer, b].reshape(-1) + kb[layer]), kv, d, cos, sin, 30 + b)
            assert np.array_equal(bits(q2[0, layer, b].reshape(-1)), bits(want_q))
            assert np.array_equal(kc[0, layer, 30 + b].reshape(-1), S.to_f16_bits(want_k))
            assert np.array_equal(vc[0, layer, 30 + b].reshape(-1), S.to_f16_bits(v[0, layer, b].reshape(-1) + vb[layer]))


def test_prefill_rows_equal_decode_and_brute_force(oracle_mod):
    tokens, base, h, kv, d = 9, 5, 4, 2, 16
    ctx = base + tokens
    q = S.normal(10, "pq", (tokens, h, d), 0.5)
    kcb = S.to_f16_bits(S.normal(10, "pk", (ctx, kv, d)))
    vcb = S.to_f16_bits(S.normal(10, "pv", (ctx, kv, d)))
    out = oracle_mod.attention_prefill(q, kcb, vcb, tokens, base, ctx, h, kv, d)
    kf, vf = S.f16_bits_to_f32(kcb), S.f16_bits_to_f32(vcb)
    for t in range(tokens):
        dec = oracle_mod.attention_decode_f32(q[t].reshape(-1), kf, vf, base + t, h, kv, d)
        assert np.array_equal(bits(out[t].reshape(-1)), bits(dec))
        np.testing.assert_allclose(out[t].reshape(-1), brute_force_decode(q[t], kf, vf, base + t, h, kv, d),
                                   atol=1e-5)
    # strided sample leaves the other rows untouched (NaN)
    part = oracle_mod.attention_prefill(q, kcb, vcb, tokens, base, ctx, h, kv, d, 1, tokens, 3)
    assert np.all(np.isnan(part[0])) and not np.any(np.isnan(part[1])) and np.all(np.isnan(part[2]))


def test_decode_f16kv_indexing(oracle_mod):
    seqs, layers, ctx, h, kv, d = 2, 3, 50, 8, 2, 64
    positions = [49, 7]
    q = S.normal(11, "iq", (seqs, layers, h, d))
    kc = S.to_f16_bits(S.normal(11, "ik", (seqs, layers, ctx, kv, d)))
    vc = S.to_f16_bits(S.normal(11, "iv", (seqs, layers, ctx, kv, d)))
    out = oracle_mod.attention_decode_f16kv(q, kc, vc, positions, 0, seqs, layers, ctx, h, kv, d)
    for s in range(seqs):
        for layer in range(layers):
            want = oracle_mod.attention_decode_f32(q[s, layer].reshape(-1), S.f16_bits_to_f32(kc[s, layer]),
                                                   S.f16_bits_to_f32(vc[s, layer]), positions[s], h, kv, d)
            assert np.array_equal(bits(out[s, layer].reshape(-1)), bits(want))


# ------------------------------------------------- decode-layer vector ops ---

def _vec_inputs(n, seed=60):
    x = S.normal(seed, f"vec{n}x", (n,))
    y = S.normal(seed, f"vec{n}y", (n,), 3.0)
    return x, y


@pytest.mark.parametrize("n", [1, 7, 896, 2048, 11008])
def test_vector_ops_match_compiled_reference(oracle_mod, n):
    """orc_rmsnorm/swiglu/add/argmax bit-identical to the reference's own
    compiled ops.c te_* functions on the same inputs."""
    if oracle_mod.ref_lib() is None:
        pytest.skip("reference ops.c not built here")
    x, y = _vec_inputs(n)
    w = S.normal(61, f"vec{n}w", (n,), 0.5) + 1.0
    for eps in (1e-6, 1e-5):
        assert np.array_equal(oracle_mod.rmsnorm_f32(x, w, eps), oracle_mod.rmsnorm_f32(x, w, eps, use_ref=True))
    assert np.array_equal(oracle_mod.swiglu_f32(y, x), oracle_mod.swiglu_f32(y, x, use_ref=True))
    assert np.array_equal(oracle_mod.add_f32(x, y), oracle_mod.add_f32(x, y, use_ref=True))
    assert oracle_mod.argmax_f32(y) == oracle_mod.argmax_f32(y, use_ref=True)


def test_vector_ops_closed_forms(oracle_mod):
    # RMSNorm of a constant vector c with unit weights is c / sqrt(c^2 + eps) per element
    x = np.full(64, 3.0, np.float32)
    got = oracle_mod.rmsnorm_f32(x, np.ones(64, np.float32), 1e-6)
    assert np.allclose(got, 3.0 / np.sqrt(9.0 + 1e-6), rtol=1e-6)
    # silu(0) = 0, silu(g) -> g for large g, silu(g) -> 0 for very negative g
    g = np.array([0.0, 30.0, -30.0], np.float32)
    assert np.allclose(oracle_mod.swiglu_f32(g, np.ones(3, np.float32)), [0.0, 30.0, 0.0], atol=1e-9)
    # argmax: first of equal maxima; NaN never taken; all -inf -> 0; -FLT_MAX -> 0
    assert oracle_mod.argmax_f32(np.array([1, 5, 5, 2], np.float32)) == 1
    assert oracle_mod.argmax_f32(np.array([np.nan, 1, np.nan, 3], np.float32)) == 3
    assert oracle_mod.argmax_f32(np.full(5, -np.inf, np.float32)) == 0
    assert oracle_mod.argmax_f32(np.array([np.finfo(np.float32).min] * 3, np.float32)) == 0
    assert oracle_mod.argmax_f32(np.array([-np.inf, np.finfo(np.float32).min, -1e38], np.float32)) == 2


@pytest.mark.parametrize("ggml_type", [2, 8])
def test_dequantize_every_code(oracle_mod, ggml_type):
    """Each 4-bit / 8-bit code at each position of a block dequantizes to
    (code - 8) * d (Q4_0: low nibble = element j, high nibble = element j+16) or
    int8(code) * d (Q8_0), for d = 0.5, -3.25 and an fp16 subnormal."""
    for dbits in (0x3800, 0xC280, 0x0001):
        d = float(np.uint16(dbits).view(np.float16))
        if ggml_type == 2:
            codes = np.arange(256, dtype=np.uint8)[:, None].repeat(16, 1)  # one block per byte value
            blk = np.empty((256, 18), np.uint8)
            want = np.empty((256, 32), np.float32)
            want[:, :16] = ((codes & 0x0F).astype(np.float32) - 8.0) * np.float32(d)
            want[:, 16:] = ((codes >> 4).astype(np.float32) - 8.0) * np.float32(d)
        else:
            codes = np.arange(256, dtype=np.uint8)[:, None].repeat(32, 1)
            blk = np.empty((256, 34), np.uint8)
            want = codes.view(np.int8).astype(np.float32) * np.float32(d)
        blk[:, 0] = dbits & 0xFF
        blk[:, 1] = dbits >> 8
        blk[:, 2:] = codes
        got = oracle_mod.dequantize_rows(blk.reshape(-1), ggml_type, 32, 256)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("ggml_type,rows,cols", [(0, 5, 64), (2, 7, 96), (8, 6, 128), (2, 3, 2048), (8, 2, 11008)])
def test_matvec_vs_fp64(oracle_mod, ggml_type, rows, cols):
    """orc_matvec_f32 against an fp64 dot of the dequantized rows: within the
    sequential fp32 error bound cols * 2^-24 * sum |w x| (plus one ulp)."""
    data = S.ggml_tensor(62, f"mv{ggml_type}{rows}{cols}", ggml_type, rows, cols)
    x = S.normal(62, f"mvx{cols}", (cols,))
    got = oracle_mod.matvec_f32(data, ggml_type, x, cols, rows)
    w = oracle_mod.dequantize_rows(data, ggml_type, cols, rows).astype(np.float64)
    exact = w @ x.astype(np.float64)
    bound = cols * 2.0 ** -24 * (np.abs(w) @ np.abs(x.astype(np.float64))) + np.abs(exact) * 2.0 ** -23
    assert np.all(np.abs(got - exact) <= bound)
    assert oracle_mod.ggml_row_bytes(ggml_type, cols) * rows == data.size


def test_decode_all_layers_composition_fp64(oracle_mod):
    """The oracle's per-token layer loop against an fp64 numpy forward pass of the
    same Qwen2 decode step (pre-norm attention block with q/k/v biases and
    half-split RoPE, GQA over the fp16 cache, SwiGLU MLP, residuals, final norm,
    head, argmax).  A misplaced residual, norm weight, bias or gate/up swap
    moves the result far past the fp32-vs-fp64 agreement asserted here."""
    import _synth as S
    layers, heads, kv_heads, d, ffn, vocab, ctx, pos = 2, 4, 2, 64, 128, 60, 8, 5
    m = S.synthetic_model(83, 8, layers, heads, kv_heads, d, ffn, vocab, ctx, pos)
    hidden, kv, eps = m["hidden"], m["kv"], 1e-6
    cos, sin = oracle_mod.rope_table(ctx, d, 1.0e6)
    kc, vc = m["key_cache"].copy(), m["value_cache"].copy()
    got_h, got_tok, got_logits = oracle_mod.decode_all_layers(
        m["mapping"], m["offsets"], layers, 8, m["hidden_in"], m["attn_norm"], m["ffn_norm"], m["q_bias"],
        m["k_bias"], m["v_bias"], cos, sin, kc, vc, pos, ctx, hidden, kv, heads, kv_heads, d, ffn, eps,
        head=m["head"], output_norm=m["output_norm"], vocab=vocab)

    mp = m["mapping"]

    def W(name, l, rows, cols):
        off = m["offsets"][name][l] if l is not None else m["head"][0]
        n = rows * oracle_mod.ggml_row_bytes(8, cols)
        return oracle_mod.dequantize_rows(mp[off:off + n], 8, cols, rows).astype(np.float64)

    def norm(x, w):
        return x / np.sqrt(np.mean(x * x) + eps) * w

    def rope(x, nh):
        x = x.reshape(nh, d).copy()
        c, s = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
        a, b = x[:, :d // 2].copy(), x[:, d // 2:].copy()
        x[:, :d // 2], x[:, d // 2:] = a * c - b * s, b * c + a * s
        return x.reshape(-1)

    x = m["hidden_in"].astype(np.float64)
    kref = m["key_cache"].view(np.float16).astype(np.float64)
    vref = m["value_cache"].view(np.float16).astype(np.float64)
    for l in range(layers):
        n = norm(x, m["attn_norm"][l])
        q = rope(W("q", l, hidden, hidden) @ n + m["q_bias"][l], heads)
        k = rope(W("k", l, kv, hidden) @ n + m["k_bias"][l], kv_heads)
        v = W("v", l, kv, hidden) @ n + m["v_bias"][l]
        kref[l, pos] = k.astype(np.float16).astype(np.float64)
        vref[l, pos] = v.astype(np.float16).astype(np.float64)
        attn = np.empty(hidden)
        for h in range(heads):
            g = h // (heads // kv_heads)
            ks = kref[l, :pos + 1, g * d:(g + 1) * d]
            sc = ks @ q[h * d:(h + 1) * d] / np.sqrt(d)
            p = np.exp(sc - sc.max())
            attn[h * d:(h + 1) * d] = (p / p.sum()) @ vref[l, :pos + 1, g * d:(g + 1) * d]
        x = x + W("output", l, hidden, hidden) @ attn
        n = norm(x, m["ffn_norm"][l])
        gate, up = W("gate", l, ffn, hidden) @ n, W("up", l, ffn, hidden) @ n
        x = x + W("down", l, hidden, ffn) @ (gate / (1.0 + np.exp(-gate)) * up)
    logits = W("head", None, vocab, hidden) @ norm(x, m["output_norm"])
    assert np.allclose(got_h, x, rtol=0, atol=2e-4 * np.abs(x).max())
    assert np.allclose(got_logits, logits, rtol=0, atol=2e-4 * np.abs(logits).max())
    assert got_tok == int(np.argmax(logits))
    # the slot written into the cache is k / v rounded to fp16 once (within one fp16 step of fp64's)
    for got, want in ((kc, kref), (vc, vref)):
        g = got[:, pos].view(np.float16).astype(np.float64)
        assert np.all(np.abs(g - want[:, pos]) <= 2.0 ** -10 * np.abs(want[:, pos]) + 2.0 ** -24)

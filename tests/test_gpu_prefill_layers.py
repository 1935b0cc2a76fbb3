"""GPU parity of te_hip_prefill_all_layers_f16 (a chunk of prompt tokens
through every layer, the twin of te_metal_prefill_all_layers_f32) against the
oracle's composition of the reference's per-token layer loop (qwen.c:907-1087):
row t of the chunk is one decode token at position base + t over the cache the
earlier rows appended (qwen.c:774-824), so the oracle runs decode_all_layers
token by token on a copy of the same fp16 cache.

Bars: the final hidden state of every row within 4e-3 of the oracle's largest
magnitude (the batched GEMM rounds each activation row to 15 bits per 32-value
block, the per-token matvec to 22 bits, and both carry the attention bar
through the layers); the appended k / v of every layer within a few fp16 steps
plus that carried error; the cache outside the chunk bit-exact; V^T equal to
the transposed value cache over positions 0 .. base + batch - 1.
"""
import ctypes

import numpy as np
import pytest

import _synth as S

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tinymetalagent_amd import attention as A  # noqa: E402
from tinymetalagent_amd import layers as LY  # noqa: E402
from tinymetalagent_amd import runtime as R  # noqa: E402

DEV = "cuda"


def _dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(DEV)
    return torch.from_numpy(a).to(DEV)


def _run(oracle_mod, ggml_type, layers, heads, kv_heads, head_dim, ffn, ctx, base, batch, *, per_layer=False):
    m = S.synthetic_model(91, ggml_type, layers, heads, kv_heads, head_dim, ffn, 64, ctx, base)
    hidden, kv = m["hidden"], m["kv"]
    cos, sin = oracle_mod.rope_table(ctx, head_dim, 1.0e6)
    eps = 1e-6
    x_in = S.normal(91, "rows", (batch, hidden))
    # oracle: the rows one token at a time, each appending to the cache the next reads
    kc_o, vc_o = m["key_cache"].copy(), m["value_cache"].copy()
    want = np.stack([oracle_mod.decode_all_layers(
        m["mapping"], m["offsets"], layers, ggml_type, x_in[t], m["attn_norm"], m["ffn_norm"], m["q_bias"],
        m["k_bias"], m["v_bias"], cos, sin, kc_o, vc_o, base + t, ctx, hidden, kv, heads, kv_heads, head_dim, ffn,
        eps)[0] for t in range(batch)])
    kc, vc = _dev(m["key_cache"]), _dev(m["value_cache"])
    kc16 = kc.view(torch.float16).reshape(1, layers, ctx, kv_heads, head_dim)
    vc16 = vc.view(torch.float16).reshape(1, layers, ctx, kv_heads, head_dim)
    vt = A.value_t_buffer(1, layers, ctx, kv_heads, head_dim)
    A.value_transpose(vc16, vt, first_position=0, count=base)
    args = (_dev(m["mapping"]), m["offsets"], layers, ggml_type)
    x = _dev(x_in)
    norms = (_dev(m["attn_norm"]), _dev(m["ffn_norm"]), _dev(m["q_bias"]), _dev(m["k_bias"]), _dev(m["v_bias"]),
             _dev(cos), _dev(sin))
    if not per_layer:
        got = LY.prefill_all_layers(*args, x, *norms, kc, vc, vt, base, ctx, heads, kv_heads, head_dim, ffn, eps)
    else:
        lib = R.load_library()
        ws = LY.prefill_workspace(batch, hidden, kv, ffn)
        got = x.clone()
        an, fn, qb, kb, vb, dcos, dsin = norms
        ctx_kv = ctx * kv
        vtl = vt[0]
        for l in range(layers):
            o = [int(m["offsets"][n][l]) for n in ("q", "k", "v", "output", "gate", "up", "down")]
            R.check(lib.te_hip_prefill_layer_f16(
                args[0].data_ptr(), args[0].numel(), *o, ggml_type, got.data_ptr(), an[l].data_ptr(),
                fn[l].data_ptr(), qb[l].data_ptr(), kb[l].data_ptr(), vb[l].data_ptr(), dcos.data_ptr(),
                dsin.data_ptr(), kc.data_ptr() + 2 * l * ctx_kv, vc.data_ptr() + 2 * l * ctx_kv,
                vtl[l].data_ptr(), base, batch, ctx, hidden, kv, heads, kv_heads, head_dim, ffn, eps,
                got.data_ptr(), ws.data_ptr(), ws.numel(), None))
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    tol = 4e-3 * float(np.abs(want).max())
    err = float(np.abs(got - want).max())
    print(f"prefill layers type {ggml_type} L{layers} base {base} batch {batch}: max err {err:.3g} (tol {tol:.3g})")
    assert err <= tol
    got_kc = kc.cpu().numpy().view(np.uint16)
    got_vc = vc.cpu().numpy().view(np.uint16)
    chunk = slice(base, base + batch)
    outside = np.ones(ctx, bool)
    outside[chunk] = False
    assert np.array_equal(got_kc[:, outside], kc_o[:, outside])
    assert np.array_equal(got_vc[:, outside], vc_o[:, outside])
    for g, w in ((got_kc, kc_o), (got_vc, vc_o)):
        gf = g[:, chunk].view(np.float16).astype(np.float32)
        wf = w[:, chunk].view(np.float16).astype(np.float32)
        bound = 4 * 2.0 ** -10 * np.abs(wf) + 4e-3 * np.abs(wf).max() + 2.0 ** -20
        assert np.all(np.abs(gf - wf) <= bound)
    n = base + batch
    vt_want = vc16.permute(0, 1, 3, 4, 2)[..., :n]
    assert torch.equal(vt[..., :n].view(torch.int16), vt_want.contiguous().view(torch.int16))
    return got


@pytest.mark.parametrize("ggml_type", [2, 8])
def test_prefill_all_layers_vs_oracle(oracle_mod, ggml_type):
    _run(oracle_mod, ggml_type, layers=3, heads=4, kv_heads=2, head_dim=64, ffn=512, ctx=96, base=0, batch=40)


def test_prefill_all_layers_after_cached_prefix_head_dim_128(oracle_mod):
    """A chunk at base 37 after a cached prefix, head_dim 128, 7:1 grouping."""
    _run(oracle_mod, 2, layers=2, heads=14, kv_heads=2, head_dim=128, ffn=1024, ctx=80, base=37, batch=21)


@pytest.mark.parametrize("ggml_type", [2, 8])
def test_prefill_paired_gate_up_gemm(oracle_mod, ggml_type, monkeypatch):
    """Gate and up as one GEMM launch whose epilogue writes the SwiGLU digits
    (TE_HIP_GEMM_GLU=1 takes it at this small grid; the library takes it by
    itself once the grid covers the GPU): the oracle's bar."""
    monkeypatch.setenv("TE_HIP_GEMM_GLU", "1")
    _run(oracle_mod, ggml_type, layers=2, heads=14, kv_heads=2, head_dim=128, ffn=1024, ctx=80, base=5, batch=70)


@pytest.mark.parametrize("ggml_type", [2, 8])
def test_prefill_paired_gate_up_gemm_bits(ggml_type, monkeypatch):
    """At a chunk whose two-GEMM path splits no K range (512 rows, ffn 8192:
    1024 output tiles), the paired launch gives the same output bits as the
    two GEMMs plus the SwiGLU digits kernel: the same products, summed in the
    same order, and the same digits.  The same holds for the next layer's
    RMSNorm digits formed inside down's split-K sums against the separate
    sums and digits launches (TE_HIP_GEMM_REDUCE_RMS=0)."""
    layers, heads, kv_heads, head_dim, ffn, batch, base = 2, 4, 2, 64, 8192, 512, 3
    ctx = base + batch
    m = S.synthetic_model(93, ggml_type, layers, heads, kv_heads, head_dim, ffn, 64, ctx, base)
    hidden = m["hidden"]
    cos, sin = A.rope_table(ctx, head_dim, 1.0e6)
    x_in = _dev(S.normal(93, "rows", (batch, hidden)))
    outs = []
    for mode, fused in (("1", "1"), ("0", "1"), ("1", "0")):
        monkeypatch.setenv("TE_HIP_GEMM_GLU", mode)
        monkeypatch.setenv("TE_HIP_GEMM_REDUCE_RMS", fused)
        kc, vc = _dev(m["key_cache"]), _dev(m["value_cache"])
        vt = A.value_t_buffer(1, layers, ctx, kv_heads, head_dim)
        A.value_transpose(vc.view(torch.float16).reshape(1, layers, ctx, kv_heads, head_dim), vt,
                          first_position=0, count=base)
        got = LY.prefill_all_layers(_dev(m["mapping"]), m["offsets"], layers, ggml_type, x_in.clone(),
                                    _dev(m["attn_norm"]), _dev(m["ffn_norm"]), _dev(m["q_bias"]), _dev(m["k_bias"]),
                                    _dev(m["v_bias"]), cos.contiguous(), sin.contiguous(), kc, vc, vt, base, ctx,
                                    heads, kv_heads, head_dim, ffn, 1e-6)
        torch.cuda.synchronize()
        outs.append(got.cpu().numpy())
    print(f"type {ggml_type}: paired vs two GEMMs max |diff| {np.abs(outs[0] - outs[1]).max():.3g}, "
          f"fused vs separate RMSNorm digits {np.abs(outs[0] - outs[2]).max():.3g}")
    assert np.isfinite(outs[0]).all() and np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


@pytest.mark.parametrize("batch,base", [(300, 300), (512, 0), (70, 5)])
def test_prefill_attention_digits_in_kernel_bits(batch, base, monkeypatch):
    """The attention kernel's own digits of its output rows (the default)
    against fp32 rows and the separate digits launch (TE_HIP_PREFILL_DIGITS=0):
    the same output bits.  300 rows after 300 cached positions take the
    128-row tile kernel (600 keys; a ragged last tile), 512 after 0 and 70
    after 5 the rows kernel (the fused step's choice up to 512 keys)."""
    layers, heads, kv_heads, head_dim, ffn = 2, 4, 2, 128, 512
    ctx = base + batch
    m = S.synthetic_model(94, 2, layers, heads, kv_heads, head_dim, ffn, 64, ctx, base)
    hidden = m["hidden"]
    cos, sin = A.rope_table(ctx, head_dim, 1.0e6)
    x_in = _dev(S.normal(94, "rows", (batch, hidden)))
    outs = []
    for mode in ("1", "0"):
        monkeypatch.setenv("TE_HIP_PREFILL_DIGITS", mode)
        kc, vc = _dev(m["key_cache"]), _dev(m["value_cache"])
        vt = A.value_t_buffer(1, layers, ctx, kv_heads, head_dim)
        A.value_transpose(vc.view(torch.float16).reshape(1, layers, ctx, kv_heads, head_dim), vt,
                          first_position=0, count=base)
        got = LY.prefill_all_layers(_dev(m["mapping"]), m["offsets"], layers, 2, x_in.clone(),
                                    _dev(m["attn_norm"]), _dev(m["ffn_norm"]), _dev(m["q_bias"]), _dev(m["k_bias"]),
                                    _dev(m["v_bias"]), cos.contiguous(), sin.contiguous(), kc, vc, vt, base, ctx,
                                    heads, kv_heads, head_dim, ffn, 1e-6)
        torch.cuda.synchronize()
        outs.append((got.cpu().numpy(), kc.cpu().numpy()))
    print(f"rows {batch} after {base}: in-kernel vs separate digits max |diff| "
          f"{np.abs(outs[0][0] - outs[1][0]).max():.3g}")
    assert np.isfinite(outs[0][0]).all()
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


def test_prefill_layer_by_layer(oracle_mod):
    """te_hip_prefill_layer_f16 once per layer: the same result as the all-layers flow."""
    _run(oracle_mod, 8, layers=2, heads=4, kv_heads=2, head_dim=64, ffn=256, ctx=48, base=5, batch=17,
         per_layer=True)


def test_prefill_all_layers_argument_checks():
    lib = R.load_library()
    m = S.synthetic_model(92, 2, 1, 4, 2, 64, 256, 64, 16, 0)
    mp = _dev(m["mapping"])
    f = torch.zeros(1 << 16, device=DEV)
    ws = torch.zeros(1 << 22, dtype=torch.uint8, device=DEV)
    offs = [(ctypes.c_uint64 * 1)(m["offsets"][n][0]) for n in ("q", "k", "v", "output", "gate", "up", "down")]
    p = f.data_ptr()

    def call(mapping_len=mp.numel(), layers=1, ggml_type=2, base=0, batch=4, ctx=16, hidden=256, kv=128, heads=4,
             kv_heads=2, head_dim=64, ffn=256, eps=1e-6, workspace=ws.data_ptr(), ws_bytes=ws.numel(), vt=p):
        return lib.te_hip_prefill_all_layers_f16(
            mp.data_ptr(), mapping_len, *[ctypes.cast(o, ctypes.POINTER(ctypes.c_uint64)) for o in offs],
            layers, ggml_type, p, p, p, p, p, p, p, p, p, p, vt, base, batch, ctx, hidden, kv, heads, kv_heads,
            head_dim, ffn, eps, p, workspace, ws_bytes, None)

    assert lib.te_hip_prefill_all_layers_workspace_bytes(4, 256, 128, 256) <= ws.numel()
    assert call(layers=0) == 1
    assert call(base=13) == 1                      # chunk past the cache
    assert call(eps=0.0) == 1
    assert call(mapping_len=1000) == 1             # tensors past the mapping
    assert call(ws_bytes=100) == 1
    assert call(vt=None) == 1
    assert call(hidden=192) == 3                   # hidden != heads * head_dim
    assert call(ggml_type=0) == 3                  # F32: not on the batched GEMM
    assert call(head_dim=32, hidden=128, kv=64) == 3


def test_prefill_stage_profile_lines(oracle_mod, monkeypatch, capfd):
    """TINYENGINE_METAL_PREFILL_STAGE_PROFILE (the reference's switch): one
    stderr line per stage and layer in the reference's format, the same result
    as without it (the stages are only synchronised)."""
    layers = 2
    want = _run(oracle_mod, 2, layers=layers, heads=4, kv_heads=2, head_dim=64, ffn=512, ctx=96, base=0, batch=40)
    capfd.readouterr()
    monkeypatch.setenv("TINYENGINE_METAL_PREFILL_STAGE_PROFILE", "1")
    got = _run(oracle_mod, 2, layers=layers, heads=4, kv_heads=2, head_dim=64, ffn=512, ctx=96, base=0, batch=40)
    err = capfd.readouterr().err
    assert np.array_equal(got, want)
    lines = [ln for ln in err.splitlines() if ln.startswith("tinyengine_metal_stage_profile: ")]
    stages = {}
    for ln in lines:
        kv = dict(f.split("=", 1) for f in ln.split(": ", 1)[1].split())
        assert kv["scope"] == "prefill_all_layers"
        assert float(kv["gpu_ms"]) >= 0.0 and float(kv["cpu_ms"]) >= 0.0
        stages.setdefault(int(kv["layer"]), []).append(kv["stage"])
    assert sorted(stages) == list(range(layers))
    assert stages[0][0] == "attn_norm_digits" and "attn_norm_digits" not in stages[1]
    for l in range(layers):
        assert "qkv_proj" in stages[l] and "qkv_bias_rope_flash_attention_mma_vt" in stages[l]
        assert stages[l][-1] == ("down_proj_add_attn_norm_digits" if l + 1 < layers else "down_proj_add")

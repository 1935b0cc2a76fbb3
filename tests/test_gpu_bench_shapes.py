"""GPU parity at the exact shapes bench.py times (4 and
5(B)), through the same entry points and workspaces: the full device work runs,
and sampled (sequence, layer) pairs or rows are checked against the oracle,
the appended cache slots bit for bit.

Bar: max-abs error <= 2e-3 for attention outputs,
bit-exact for the fp16 cache slots.
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tinymetalagent_amd import attention as A  # noqa: E402
from tinymetalagent_amd import runtime as R  # noqa: E402

TOL = 2e-3
DEV = "cuda"
THETA = 1e6


def f16_host_bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def maxabs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def _fused_step_pairs(oracle_mod, *, h, kv, d, layers, positions, pairs, seed):
    """One fused decode step (te_hip_attention_decode_step_f16) over every
    sequence and layer with the workspace bench.py uses; each sampled (seq,
    layer) pair is replayed on the host: RoPE + fp16 append of its token into
    a copy of its cache slice, then the oracle decode at its position."""
    seqs = len(positions)
    ctx = max(positions) + 1
    g = torch.Generator(device=DEV).manual_seed(seed)
    kc = torch.randn((seqs, layers, ctx, kv, d), generator=g, device=DEV).half()
    vc = torch.randn((seqs, layers, ctx, kv, d), generator=g, device=DEV).half()
    q = torch.randn((seqs, layers, 1, h, d), generator=g, device=DEV) / math.sqrt(d)
    k = torch.randn((seqs, layers, 1, kv, d), generator=g, device=DEV)
    v = torch.randn((seqs, layers, 1, kv, d), generator=g, device=DEV)
    # host copies of the sampled slices before the step appends into them
    before = {(s, l): (f16_host_bits(kc[s, l]).copy(), f16_host_bits(vc[s, l]).copy()) for s, l in pairs}
    cos, sin = A.rope_table(ctx, d, THETA)
    ws = A.decode_workspace(seqs, layers, h, kv, d, positions=positions)
    out = torch.empty((seqs, layers, h, d), dtype=torch.float32, device=DEV)
    A.decode_step(q, k, v, cos, sin, kc, vc, positions=positions, out=out, workspace=ws)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    hcos, hsin = oracle_mod.rope_table(ctx, d, THETA)
    worst = 0.0
    for s, l in pairs:
        pos = positions[s]
        kc1, vc1 = (b.reshape(1, 1, ctx, kv, d) for b in before[(s, l)])
        q1, k1, v1 = (t[s:s + 1, l:l + 1].cpu().numpy().copy() for t in (q, k, v))
        oracle_mod.rope_kv_append_f16(q1, k1, v1, None, None, None, hcos, hsin, kc1, vc1, 1, 1, 1, None, pos, ctx,
                                      h, kv, d)
        # the GPU wrote the same bits into the same slot and nothing else
        assert np.array_equal(f16_host_bits(kc[s, l]), kc1[0, 0]), (s, l)
        assert np.array_equal(f16_host_bits(vc[s, l]), vc1[0, 0]), (s, l)
        want = oracle_mod.attention_decode_f16kv(q1[:, :, 0].copy(), kc1, vc1, None, pos, 1, 1, ctx, h, kv, d)
        err = maxabs(got[s, l], want[0, 0])
        print(f"  seq {s} (position {pos}) layer {l}: max abs err {err:.3e}")
        worst = max(worst, err)
    return worst


def test_decode_step_headline_geometry(oracle_mod):
    """BASELINE config 2 as the headline times it: 3B (16 heads, 2 KV heads,
    d 128), 36 layers, append at position 8192 (13 split-K chunks per head on
    256 CUs); layers 0, 17 and 35 against the oracle."""
    err = _fused_step_pairs(oracle_mod, h=16, kv=2, d=128, layers=36, positions=[8192],
                            pairs=[(0, 0), (0, 17), (0, 35)], seed=42)
    print(f"3B fused step, 36 layers at 8192: max abs err {err:.3e}")
    assert err <= TOL


def test_decode_step_config4_ragged_full(oracle_mod):
    """BASELINE config 4 at full size: 7B (28 heads, 4 KV heads, d 128), 28
    layers, eight sequences at the positions bench.py draws in [1K, 16K]; one
    fused step over all of them, six (seq, layer) pairs against the oracle,
    covering the shortest and the longest sequence."""
    g = torch.Generator().manual_seed(42)
    positions = [int(x) for x in torch.randint(1024, 16385, (8,), generator=g)]
    short, long_ = int(np.argmin(positions)), int(np.argmax(positions))
    pairs = [(short, 0), (long_, 27), (0, 13), (3, 5), (5, 21), (7, 9)]
    err = _fused_step_pairs(oracle_mod, h=28, kv=4, d=128, layers=28, positions=positions, pairs=pairs, seed=7)
    print(f"7B ragged x8 {positions}, 28 layers: max abs err {err:.3e}")
    assert err <= TOL


def _chunk_after_128k(tokens=2048, base=131072, seed=12):
    h, kv, d = 12, 2, 128
    ctx = base + tokens
    g = torch.Generator(device=DEV).manual_seed(seed)
    kc = torch.randn((1, 1, ctx, kv, d), generator=g, device=DEV).half()
    vc = torch.randn((1, 1, ctx, kv, d), generator=g, device=DEV).half()
    qh = torch.randn((1, 1, tokens, h, d), generator=g, device=DEV).half()
    return h, kv, d, ctx, kc, vc, qh


ROWS_128K = (0, 1, 127, 128, 1029, 2047)


def _check_rows(oracle_mod, got, qh, kc, vc, base, ctx, h, kv, d, what):
    tokens = qh.shape[2]
    got = got.reshape(tokens, h, d)
    qf = qh.float().cpu().numpy().reshape(tokens, h, d)
    kb, vb = f16_host_bits(kc[0, 0]), f16_host_bits(vc[0, 0])
    worst = 0.0
    for t in ROWS_128K:
        want = oracle_mod.attention_prefill(qf, kb, vb, tokens, base, ctx, h, kv, d, t, t + 1)
        worst = max(worst, maxabs(got[t], want[t]))
    print(f"{what}: rows {ROWS_128K}: max abs err {worst:.3e}")
    return worst


def test_prefill_split_2048_after_128k(oracle_mod):
    """BASELINE config 5 (B) as bench.py times it: a 2048-row 1.5B chunk at base
    131072 through te_hip_attention_prefill_split_f16 with the library's own
    split count (8 on a 256-CU device), sampled rows against the oracle."""
    base = 131072
    h, kv, d, ctx, kc, vc, qh = _chunk_after_128k(base=base)
    tokens = qh.shape[2]
    lib = R.load_library()
    nbytes = lib.te_hip_attention_prefill_workspace_bytes(1, 1, tokens, base, ctx, h, kv, d)
    part = nbytes - lib.te_hip_value_t_bytes(1, 1, ctx, kv, d)
    splits = part // (tokens * h * (d + 2) * 4)
    assert splits * tokens * h * (d + 2) * 4 == part
    _, cus = R.device_info()
    print(f"library split count: {splits} ({cus} CUs)")
    if cus == 256:
        assert splits == 8
    got = A.attention_prefill_split(qh, kc, vc, base_position=base).cpu().numpy()
    assert _check_rows(oracle_mod, got, qh, kc, vc, base, ctx, h, kv, d, "split entry, 2048 rows after 128K") <= TOL


def test_prefill_vt_split_2048_after_128k(oracle_mod):
    """The same chunk through te_hip_attention_prefill_vt_f16 (V^T resident,
    key split from te_hip_attention_prefill_vt_workspace_bytes, as bench.py's
    split figures run it): sampled rows against the oracle, and the one-split
    launch within the bar of the split one."""
    base = 131072
    h, kv, d, ctx, kc, vc, qh = _chunk_after_128k(base=base, seed=13)
    tokens = qh.shape[2]
    vt = A.value_t_buffer(1, 1, ctx, kv, d)
    A.value_transpose(vc, vt)
    ws = A.prefill_vt_workspace(1, 1, tokens, h, kv, d, base_position=base, context_tokens=ctx)
    assert ws is not None
    nsplit = ws.numel() // (tokens * h * (d + 2) * 4)
    got = A.attention_prefill_vt(qh, kc, vt, base_position=base, workspace=ws).cpu().numpy()
    assert _check_rows(oracle_mod, got, qh, kc, vc, base, ctx, h, kv, d,
                       f"V^T entry, {nsplit} splits, 2048 rows after 128K") <= TOL
    one = A.attention_prefill_vt(qh, kc, vt, base_position=base).cpu().numpy()
    assert maxabs(one, got) <= TOL


def test_prefill_step_vt_config3_full(oracle_mod):
    """BASELINE config 3 as bench.py's whole-step figure runs it: 3B, L=4096
    from position 0, te_hip_attention_prefill_step_vt_f16 (RoPE + fp16 append
    + V^T of the chunk + attention) into empty caches; the caches equal the
    separate RoPE/append launch bit for bit, V^T equals the transposed value
    cache, and sampled rows match the oracle."""
    h, kv, d, L = 16, 2, 128, 4096
    g = torch.Generator(device=DEV).manual_seed(43)
    q = torch.randn((1, 1, L, h, d), generator=g, device=DEV).half().float()
    k = torch.randn((1, 1, L, kv, d), generator=g, device=DEV).half().float()
    v = torch.randn((1, 1, L, kv, d), generator=g, device=DEV).half().float()
    cos, sin = A.rope_table(L, d, THETA)
    kc = torch.zeros((1, 1, L, kv, d), dtype=torch.float16, device=DEV)
    vc = torch.zeros_like(kc)
    vt = A.value_t_buffer(1, 1, L, kv, d)
    ws = A.prefill_vt_workspace(1, 1, L, h, kv, d, base_position=0, context_tokens=L)
    out = A.prefill_step_vt(q, k, v, cos, sin, kc, vc, vt, base_position=0, workspace=ws)
    # the unfused launch on copies: same cache bits
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    qh = torch.empty((1, 1, L, h, d), dtype=torch.float16, device=DEV)
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    A.rope_kv_append(q2, k2, v2, cos, sin, kc2, vc2, base_position=0, q_half=qh)
    torch.cuda.synchronize()
    assert torch.equal(kc.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), vc2.view(torch.int16))
    assert torch.equal(vt[..., :L].view(torch.int16), vc.permute(0, 1, 3, 4, 2).view(torch.int16))
    assert not torch.equal(q, q2)  # the unfused launch rotated its q in place; the step left q alone
    got = out.cpu().numpy().reshape(L, h, d)
    qf = q2.cpu().numpy().reshape(L, h, d)  # rotated fp32 q, as the oracle takes it
    kb, vb = f16_host_bits(kc[0, 0]), f16_host_bits(vc[0, 0])
    worst = 0.0
    for t in (0, 1, 63, 64, 1000, 2047, 4000, 4095):
        want = oracle_mod.attention_prefill(qf, kb, vb, L, 0, L, h, kv, d, t, t + 1)
        worst = max(worst, maxabs(got[t], want[t]))
    print(f"fused V^T step 3B L=4096: max abs err {worst:.3e}")
    assert worst <= TOL

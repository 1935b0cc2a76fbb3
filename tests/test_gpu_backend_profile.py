"""TINYENGINE_METAL_PROFILE, the reference's backend call profile
(metal_backend_runtime.mm.inc:132-244): with the switch set, a process that
runs the layer flows prints at exit one line per bucket it used, in the
reference's format, with the calls it made -- a single-layer twin counts as
one decode_layer / prefill_layer call, not also as an all-layers call -- and
without the switch it prints none.  The flows run in a child process, since
the lines come at its exit.  The child also checks the decode single-layer
twin against the all-layers flow over the same layers (bit-identical: the
same launches in the same order)."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
TESTS = ROOT / "tests"

CHILD = r"""
import sys
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import torch
import oracle
oracle.lib()
import _synth as S
import test_gpu_decode_layers as DL
import test_gpu_prefill_layers as PL
from tinymetalagent_amd import layers as LY
from tinymetalagent_amd import runtime as R

if sys.argv[3] == "short":
    DL._run(oracle, 2, layers=2, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=100, ctx=32, position=11,
            head=False)
    raise SystemExit(0)
PL._run(oracle, 2, layers=2, heads=4, kv_heads=2, head_dim=64, ffn=512, ctx=96, base=0, batch=40)
PL._run(oracle, 2, layers=2, heads=4, kv_heads=2, head_dim=64, ffn=512, ctx=96, base=0, batch=40, per_layer=True)
DL._run(oracle, 2, layers=2, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=100, ctx=32, position=11, head=True)
DL._run(oracle, 2, layers=2, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=100, ctx=32, position=11, head=False)

# one decode token layer by layer through te_hip_decode_layer_f16, against the
# all-layers flow on a copy of the same caches
layers, heads, kv_heads, d, ffn, ctx, pos = 2, 4, 2, 64, 512, 32, 11
m = S.synthetic_model(81, 2, layers, heads, kv_heads, d, ffn, 100, ctx, pos)
hidden, kv = m["hidden"], m["kv"]
cos, sin = oracle.rope_table(ctx, d, 1.0e6)
dev = lambda a: DL._dev(a)
mp, an, fn = dev(m["mapping"]), dev(m["attn_norm"]), dev(m["ffn_norm"])
qb, kb, vb, dc, ds = dev(m["q_bias"]), dev(m["k_bias"]), dev(m["v_bias"]), dev(cos), dev(sin)
x = dev(m["hidden_in"])
kc1, vc1 = dev(m["key_cache"]), dev(m["value_cache"])
kc2, vc2 = kc1.clone(), vc1.clone()
want = LY.decode_all_layers(mp, m["offsets"], layers, 2, x, an, fn, qb, kb, vb, dc, ds, kc1, vc1, pos, ctx,
                            heads, kv_heads, d, ffn, 1e-6)
lib = R.load_library()
ws = LY.workspace(pos, hidden, kv, heads, kv_heads, d, ffn)
got = x.clone()
for l in range(layers):
    o = [int(m["offsets"][n][l]) for n in ("q", "k", "v", "output", "gate", "up", "down")]
    R.check(lib.te_hip_decode_layer_f16(
        mp.data_ptr(), mp.numel(), *o, 2, got.data_ptr(), an[l].data_ptr(), fn[l].data_ptr(), qb[l].data_ptr(),
        kb[l].data_ptr(), vb[l].data_ptr(), dc.data_ptr(), ds.data_ptr(), kc2.data_ptr() + 2 * l * ctx * kv,
        vc2.data_ptr() + 2 * l * ctx * kv, pos, ctx, hidden, kv, heads, kv_heads, d, ffn, 1e-6, got.data_ptr(),
        ws.data_ptr(), ws.numel(), None))
torch.cuda.synchronize()
assert torch.equal(got, want), "decode layer twin differs from the all-layers flow"
assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1), "decode layer twin caches differ"
print("child done", flush=True)
"""


def _child(mode, profile):
    env = dict(os.environ)
    env.pop("TINYENGINE_METAL_PROFILE", None)
    if profile:
        env["TINYENGINE_METAL_PROFILE"] = "1"
    p = subprocess.run([sys.executable, "-c", CHILD, str(ROOT), str(TESTS), mode], env=env, capture_output=True,
                       text=True, timeout=600)
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-4000:]
    lines = [ln for ln in p.stderr.splitlines() if ln.startswith("tinyengine_metal_profile: ")]
    return p.stdout, lines


def test_backend_profile_buckets_at_exit():
    out, lines = _child("full", True)
    assert "child done" in out
    buckets = {}
    for ln in lines:
        kv = dict(f.split("=", 1) for f in ln.split(": ", 1)[1].split())
        assert list(kv) == ["name", "calls", "cpu_ms", "gpu_ms", "avg_cpu_ms", "avg_gpu_ms"]
        calls = int(kv["calls"])
        cpu, gpu = float(kv["cpu_ms"]), float(kv["gpu_ms"])
        assert calls > 0 and cpu > 0.0 and gpu > 0.0
        assert abs(float(kv["avg_cpu_ms"]) - cpu / calls) <= 1e-3
        assert abs(float(kv["avg_gpu_ms"]) - gpu / calls) <= 1e-3
        # a call's GPU time lies inside its host wall time (3 decimals printed)
        assert gpu <= cpu + 1e-3 * calls + 0.01
        buckets[kv["name"]] = calls
    assert buckets == {"prefill_all_layers": 1, "prefill_layer": 2, "decode_project": 1, "decode_all_layers": 2,
                       "decode_layer": 2}, buckets


def test_backend_profile_off_prints_nothing():
    _, lines = _child("short", False)
    assert lines == []

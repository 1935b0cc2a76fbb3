"""te_hip_attention_decode_step_noalloc_f16 (the decode step whose split-K
partials live in the library's static per-GPU array) against
te_hip_attention_decode_step_f16 with a caller workspace: the output and the
appended cache slots must be bit-identical, on two calls in a row, the second
smaller than the first (the array keeps the first call's partials)."""
import ctypes

import pytest

torch = pytest.importorskip("torch")

from tinymetalagent_amd import attention as A  # noqa: E402
from tinymetalagent_amd import runtime as R  # noqa: E402

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(seed, seqs, layers, ctx, heads, kv, d):
    g = torch.Generator().manual_seed(seed)
    t = {
        "query": torch.randn(seqs, layers, heads, d, generator=g) / d ** 0.5,
        "k_new": torch.randn(seqs, layers, kv, d, generator=g),
        "v_new": torch.randn(seqs, layers, kv, d, generator=g),
        "q_bias": torch.randn(layers, heads * d, generator=g) * 0.1,
        "k_bias": torch.randn(layers, kv * d, generator=g) * 0.1,
        "v_bias": torch.randn(layers, kv * d, generator=g) * 0.1,
        "key_cache": torch.randn(seqs, layers, ctx, kv, d, generator=g).half(),
        "value_cache": torch.randn(seqs, layers, ctx, kv, d, generator=g).half(),
    }
    return {k: v.to(DEV) for k, v in t.items()}


def _both(case, positions, position):
    seqs, layers, ctx, heads, kv, d = case
    print(f"noalloc case seqs={seqs} layers={layers} ctx={ctx} heads={heads} kv={kv} d={d} "
          f"positions={positions} position={position}", flush=True)
    t = _inputs(7 + ctx, *case)
    cos, sin = A.rope_table(ctx, d, 1e6)
    kw = dict(position=position, positions=positions, q_bias=t["q_bias"], k_bias=t["k_bias"], v_bias=t["v_bias"])
    kc1, vc1 = t["key_cache"].clone(), t["value_cache"].clone()
    ref = A.decode_step(t["query"], t["k_new"], t["v_new"], cos, sin, kc1, vc1, **kw)
    kc2, vc2 = t["key_cache"].clone(), t["value_cache"].clone()
    out = torch.full_like(ref, float("nan"))
    A.decode_step_noalloc(t["query"], t["k_new"], t["v_new"], cos, sin, kc2, vc2, out=out, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16))
    assert not torch.equal(kc2, t["key_cache"])  # the new token was appended


def test_noalloc_decode_step_matches_workspace_entry_point():
    if not R.hip_available():
        pytest.fail("libtinyengine.so sees no gfx950 device")
    # the headline shape first (3B, 36 layers, position 8191), then a smaller ragged call
    _both((1, 36, 8192, 16, 2, 128), None, 8191)
    _both((2, 2, 1024, 14, 2, 64), [700, 90], 0)


def test_noalloc_decode_step_rejects_partials_beyond_the_array():
    lib = R.load_library()
    seqs, layers, heads, kv, d, ctx = 64, 28, 28, 4, 128, 1
    chunk, chunks = ctypes.c_size_t(), ctypes.c_size_t()
    R.check(lib.te_hip_attention_decode_chunking(None, 0, seqs, layers, kv, 0, ctypes.byref(chunk),
                                                 ctypes.byref(chunks)))
    assert seqs * layers * heads * chunks.value * (d + 2) * 4 > 16 << 20
    small = torch.zeros(seqs * layers * ctx * kv * d, dtype=torch.float16, device=DEV)
    f32 = torch.zeros(seqs * layers * heads * d, device=DEV)
    p, h = f32.data_ptr(), small.data_ptr()
    st = lib.te_hip_attention_decode_step_noalloc_f16(p, p, p, None, None, None, p, p, h, h, None, 0, seqs, layers,
                                                      ctx, heads, kv, d, p, None)
    assert st == R.TE_STATUS_UNSUPPORTED

"""Golden-vector cases: input builders shared by make_golden.py and the tests.

Each decode case rebuilds its inputs from the seed: raw N(0,1) draws, RoPE of
K at every cache position and of q at the query position (via the oracle's
te_rope_f32 restatement, itself pinned bit-exact to the reference), fp16 RNE
of the cache.  The fixture stores the SHA-256 of the rebuilt inputs next to
the reference output, so a test first proves it rebuilt the very inputs the
reference saw.
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

import _synth as S  # noqa: E402

ROPE_CASES = [
    # (name, heads, head_dim, position, theta)
    ("kat_d4_theta1e4_pos1", 1, 4, 1, 10000.0),
    ("q_0p5b_pos0", 14, 64, 0, 1e6),
    ("q_0p5b_pos512", 14, 64, 512, 1e6),
    ("q_3b_pos8192", 16, 128, 8192, 1e6),
    ("k_3b_pos32768", 2, 128, 32768, 1e6),
    ("q_1p5b_pos131072", 12, 128, 131072, 1e6),
    ("q_7b_pos16383", 28, 128, 16383, 1e6),
]

ROPE_ROW_POSITIONS = [0, 1, 2, 511, 512, 4095, 4096, 8192, 32768, 131072, 147455]

DECODE_CASES = [
    # name, heads, kv_heads, head_dim, position, q_scale, kv_scale, rope_cache, outliers
    dict(name="cfg1_0p5b_pos512", heads=14, kv=2, d=64, pos=512, q_scale=1 / 8, kv_scale=1 / 8, rope=True),
    dict(name="cfg2_3b_pos1100", heads=16, kv=2, d=128, pos=1100, q_scale=1 / math.sqrt(128), kv_scale=1.0,
         rope=False),
    dict(name="cfg5_1p5b_pos300_outliers", heads=12, kv=2, d=128, pos=300, q_scale=1 / math.sqrt(128),
         kv_scale=1.0, rope=False, outliers=True),
    dict(name="cfg4_7b_pos200", heads=28, kv=4, d=128, pos=200, q_scale=1 / math.sqrt(128), kv_scale=1.0,
         rope=False),
    dict(name="pos0_single_key", heads=16, kv=2, d=128, pos=0, q_scale=1 / math.sqrt(128), kv_scale=1.0,
         rope=False),
    dict(name="pos1023_stack_scores", heads=14, kv=2, d=64, pos=1023, q_scale=1 / 8, kv_scale=1 / 8, rope=True),
    dict(name="pos1024_heap_scores", heads=14, kv=2, d=64, pos=1024, q_scale=1 / 8, kv_scale=1 / 8, rope=True),
    dict(name="sharp_softmax_3b", heads=16, kv=2, d=128, pos=777, q_scale=1.0, kv_scale=1.0, rope=False),
]


def rope_input(name: str, heads: int, head_dim: int) -> np.ndarray:
    if name.startswith("kat_"):
        return np.array([1.0, 2.0, 3.0, 4.0], dtype=np.float32)
    return S.normal(S.SEED, "rope/" + name, (heads * head_dim,))


def decode_inputs(case: dict, use_ref: bool = False):
    """Returns (q fp32 [H*d], key_bits u16 [(pos+1)*kv*d], value_bits u16 [...]).

    use_ref=True rotates with the compiled reference te_rope_f32 (make_golden.py);
    the tests rebuild with the oracle's restatement and must hit the same digest."""
    import oracle

    h, kv, d, pos = case["heads"], case["kv"], case["d"], case["pos"]
    n = pos + 1
    tag = "decode/" + case["name"]
    q = S.normal(S.SEED, tag + "/q", (h * d,), case["q_scale"])
    if case.get("outliers"):
        k = S.outlier_keys(S.SEED, tag + "/k", (n, kv, d)) * np.float32(case["kv_scale"])
    else:
        k = S.normal(S.SEED, tag + "/k", (n, kv, d), case["kv_scale"])
    v = S.normal(S.SEED, tag + "/v", (n, kv, d), case["kv_scale"])
    if case["rope"]:
        for p in range(n):
            k[p] = oracle.rope_f32(k[p].reshape(-1), kv, d, p, 1e6, use_ref=use_ref).reshape(kv, d)
        q = oracle.rope_f32(q, h, d, pos, 1e6, use_ref=use_ref)
    kb = S.to_f16_bits(k).reshape(-1)
    vb = S.to_f16_bits(v).reshape(-1)
    return q.astype(np.float32), kb, vb

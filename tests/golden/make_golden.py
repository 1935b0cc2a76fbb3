"""Write tests/golden/golden.npz + golden.json from the REFERENCE's own C code.

Runs the reference te_rope_f32 / te_attention_decode_f32 (c/src/ops.c,
compiled from the read-only reference tree into oracle/_ref by
oracle/Makefile `ref`) on the inputs of cases.py and stores their outputs.
Inputs are not stored (they are rebuilt from the seed); their SHA-256 is.

    make -C oracle all ref && python tests/golden/make_golden.py

Only needs to run where the reference tree exists; the fixtures it writes are
committed and travel with the tests.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))

import cases as C  # noqa: E402
import _synth as S  # noqa: E402
import oracle  # noqa: E402


def main() -> None:
    oracle.build(with_reference=True)
    if oracle.ref_lib() is None:
        raise SystemExit("oracle/_ref/libte_ref_ops.so missing: the reference tree is required")
    arrays: dict[str, np.ndarray] = {}
    meta: dict = {"seed": S.SEED, "source": "reference c/src/ops.c te_rope_f32 / te_attention_decode_f32",
                  "rope": {}, "rope_rows": {}, "decode": {}}

    for name, heads, d, pos, theta in C.ROPE_CASES:
        x = C.rope_input(name, heads, d)
        out = oracle.rope_f32(x, heads, d, pos, theta, use_ref=True)
        arrays[f"rope/{name}"] = out
        meta["rope"][name] = dict(heads=heads, head_dim=d, position=pos, theta=theta, input_sha256=S.digest(x))

    # cos/sin table rows, read back through the reference rotation itself:
    # rotating a = 1, b = 0 yields a' = cos, b' = sin exactly.
    for d in (64, 128):
        unit = np.concatenate([np.ones(d // 2, np.float32), np.zeros(d // 2, np.float32)])
        rows = np.stack([oracle.rope_f32(unit, 1, d, p, 1e6, use_ref=True) for p in C.ROPE_ROW_POSITIONS])
        arrays[f"rope_rows/d{d}"] = rows
    meta["rope_rows"] = dict(positions=C.ROPE_ROW_POSITIONS, theta=1e6, layout="[row][cos(d/2) | sin(d/2)]")

    for case in C.DECODE_CASES:
        q, kb, vb = C.decode_inputs(case, use_ref=True)
        kf = S.f16_bits_to_f32(kb)
        vf = S.f16_bits_to_f32(vb)
        out = oracle.attention_decode_f32(q, kf, vf, case["pos"], case["heads"], case["kv"], case["d"], use_ref=True)
        arrays[f"decode/{case['name']}"] = out
        meta["decode"][case["name"]] = dict(case, input_sha256=S.digest(q, kb, vb))

    np.savez_compressed(HERE / "golden.npz", **arrays)
    (HERE / "golden.json").write_text(json.dumps(meta, indent=1, sort_keys=True) + "\n")
    total = sum(a.nbytes for a in arrays.values())
    print(f"wrote {len(arrays)} arrays ({total} bytes) to {HERE / 'golden.npz'}")


if __name__ == "__main__":
    main()

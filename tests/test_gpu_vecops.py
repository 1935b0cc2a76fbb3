"""GPU parity of the decode-layer vector operations (te_hip_matvec_f32,
te_hip_rmsnorm_f32, te_hip_swiglu_f32, te_hip_add_f32, te_hip_argmax_f32 and
the public te_rmsnorm_f32 / te_swiglu_f32 / te_add_f32 / te_argmax_f32)
against the CPU oracle, which matches the reference's compiled ops.c.

Bars: add and argmax bit-exact; RMSNorm and SwiGLU within 2 ulps relative
(fp64 sum of squares in a different order; the device expf); matvec within
2^-19 of the sum of the absolute values of its terms (fp32 accumulation in a
different order, with the block scale factored out), checked against an fp64
dot of the dequantized rows.
"""
import numpy as np
import pytest

import _synth as S

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tinymetalagent_amd import runtime as R  # noqa: E402
from tinymetalagent_amd import vecops as V  # noqa: E402

DEV = "cuda"


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _matvec_bound(oracle_mod, data, ggml_type, x, cols, rows):
    """2^-19 x sum over the row's blocks of |d| * sum_j (u_j + offset) |x_j| --
    the magnitudes the kernel's factored form accumulates."""
    w = oracle_mod.dequantize_rows(data, ggml_type, cols, rows).astype(np.float64)
    exact = w @ x.astype(np.float64)
    if ggml_type == V.GGML_F32:
        mag = np.abs(w) @ np.abs(x.astype(np.float64))
    else:
        blocks = data.reshape(rows, cols // 32, -1)
        d = np.abs(blocks[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64))
        off = 8.0 if ggml_type == V.GGML_Q4_0 else 128.0
        ax = np.abs(x.astype(np.float64)).reshape(cols // 32, 32)
        # u_j <= 15 (Q4_0) or 255 (Q8_0): bound |u_j| + offset by 2 * offset
        mag = (d * (2 * off + off) * ax.sum(1)[None, :]).sum(1)
    return exact, 2.0 ** -19 * mag + 1e-30


@pytest.mark.parametrize("ggml_type,rows,cols", [
    (V.GGML_Q4_0, 1, 32), (V.GGML_Q4_0, 7, 96), (V.GGML_Q4_0, 2048, 2048), (V.GGML_Q4_0, 256, 11008),
    (V.GGML_Q4_0, 16387, 256),                         # four rows per wave, ragged last wave
    (V.GGML_Q8_0, 3, 64), (V.GGML_Q8_0, 8195, 160),    # two rows per wave, ragged
    (V.GGML_Q8_0, 512, 2048), (V.GGML_F32, 5, 4), (V.GGML_F32, 300, 2052), (V.GGML_F32, 9000, 64),
])
def test_matvec_vs_oracle(oracle_mod, ggml_type, rows, cols):
    data = S.ggml_tensor(70, f"gmv{ggml_type}{rows}{cols}", ggml_type, rows, cols)
    x = S.normal(70, f"gmvx{cols}", (cols,))
    got = V.matvec(_dev(data), ggml_type, _dev(x), rows).cpu().numpy()
    exact, bound = _matvec_bound(oracle_mod, data, ggml_type, x, cols, rows)
    err = np.abs(got.astype(np.float64) - exact)
    print(f"matvec type {ggml_type} {rows}x{cols}: max err / bound {float((err / bound).max()):.3f}")
    assert np.all(err <= bound)
    orc = oracle_mod.matvec_f32(data, ggml_type, x, cols, rows)
    assert np.all(np.abs(got.astype(np.float64) - orc) <= 2 * bound)


def test_matvec_unaligned_row_starts(oracle_mod):
    """Blocks 2 bytes past a dword boundary and a tensor ending 2 bytes past one
    (odd block count per row): every row of a Q4_0 [33][3*32] tensor."""
    rows, cols = 33, 96
    data = S.ggml_tensor(71, "gmvodd", V.GGML_Q4_0, rows, cols)
    x = S.normal(71, "gmvoddx", (cols,))
    buf = torch.zeros(data.size + 2, dtype=torch.uint8, device=DEV)
    buf[: data.size] = _dev(data)
    got = V.matvec(buf, V.GGML_Q4_0, _dev(x), rows).cpu().numpy()
    exact, bound = _matvec_bound(oracle_mod, data, V.GGML_Q4_0, x, cols, rows)
    assert np.all(np.abs(got - exact) <= bound)


def test_matvec_argument_checks():
    lib = R.load_library()
    w = torch.zeros(64, dtype=torch.uint8, device=DEV)
    x = torch.zeros(32, device=DEV)
    y = torch.zeros(2, device=DEV)
    assert lib.te_hip_matvec_f32(w.data_ptr(), 2, x.data_ptr(), 30, 2, y.data_ptr(), None) == 3  # cols % 32
    assert lib.te_hip_matvec_f32(w.data_ptr(), 12, x.data_ptr(), 32, 2, y.data_ptr(), None) == 3  # Q4_K: not here
    assert lib.te_hip_matvec_f32(None, 2, x.data_ptr(), 32, 2, y.data_ptr(), None) == 1


@pytest.mark.parametrize("rows,n", [(1, 1), (1, 896), (4, 2048), (3, 11008)])
def test_rmsnorm_vs_oracle(oracle_mod, rows, n):
    x = S.normal(72, f"rn{rows}{n}", (rows, n), 2.0)
    w = S.normal(72, f"rnw{n}", (n,), 0.3) + 1.0
    got = V.rmsnorm(_dev(x), _dev(w), 1e-6).cpu().numpy()
    want = np.stack([oracle_mod.rmsnorm_f32(x[r], w, 1e-6) for r in range(rows)])
    np.testing.assert_allclose(got, want, rtol=2.4e-7, atol=0)
    pub = R.rmsnorm_f32(x[0], w, 1e-6)
    np.testing.assert_allclose(pub, want[0], rtol=2.4e-7, atol=0)


@pytest.mark.parametrize("n", [1, 5000, 11008])
def test_swiglu_add_vs_oracle(oracle_mod, n):
    g = S.normal(73, f"sg{n}", (n,), 4.0)
    u = S.normal(73, f"su{n}", (n,))
    got = V.swiglu(_dev(g), _dev(u)).cpu().numpy()
    want = oracle_mod.swiglu_f32(g, u)
    np.testing.assert_allclose(got, want, rtol=2.4e-7, atol=1e-37)
    np.testing.assert_allclose(R.swiglu_f32(g, u), want, rtol=2.4e-7, atol=1e-37)
    assert np.array_equal(V.add(_dev(g), _dev(u)).cpu().numpy(), oracle_mod.add_f32(g, u))
    assert np.array_equal(R.add_f32(g, u), oracle_mod.add_f32(g, u))


def test_argmax_vs_oracle(oracle_mod):
    fmin = np.finfo(np.float32).min
    cases = [np.array([1, 5, 5, 2], np.float32), np.array([np.nan, 1, np.nan, 3], np.float32),
             np.full(7, -np.inf, np.float32), np.array([fmin] * 3, np.float32),
             np.array([-np.inf, fmin, -1e38], np.float32), np.array([2.0], np.float32)]
    big = S.normal(74, "am", (151936,))
    big[[17, 151000, 99999]] = 9.0  # equal maxima far apart: the first wins
    cases.append(big)
    tied = np.zeros(4097, np.float32)
    cases.append(tied)
    for v in cases:
        want = oracle_mod.argmax_f32(v)
        assert int(V.argmax(_dev(v)).item()) == want
        assert R.argmax_f32(v) == want

"""GPU parity of the decode-layer vector operations (te_hip_matvec_f32,
te_hip_rmsnorm_f32, te_hip_swiglu_f32, te_hip_add_f32, te_hip_argmax_f32 and
the public te_rmsnorm_f32 / te_swiglu_f32 / te_add_f32 / te_argmax_f32)
against the CPU oracle, which matches the reference's compiled ops.c.

Bars: add and argmax bit-exact; RMSNorm and SwiGLU within 2 ulps relative
(fp64 sum of squares in a different order; the device expf).  Matvec, checked
against an fp64 dot of the dequantized rows: F32 within 2^-19 of sum |w x|
(fp32 accumulation in a different order); Q4_0 / Q8_0 within 2^-19 sum |w x|
+ 2^-21 sum_blocks max|x_block| sum_block |w| (+ 2^-126 sum |w|) -- the
kernel rounds each 32-value block of x to 22-bit integers relative to the
block's largest magnitude (error <= 2^-22 of it per value; at most 2^-127
for blocks below 2^-104) and sums the products exactly.
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
    """(exact fp64 product, bound): fp32 rounding 2^-19 sum |w x|, plus for the
    quantized types the rounding of x to 22 bits of its block maximum."""
    w = oracle_mod.dequantize_rows(data, ggml_type, cols, rows).astype(np.float64)
    ax = np.abs(x.astype(np.float64))
    exact = w @ x.astype(np.float64)
    bound = 2.0 ** -19 * (np.abs(w) @ ax)
    if ggml_type != V.GGML_F32:
        block_max = np.repeat(ax.reshape(cols // 32, 32).max(1), 32)
        # blocks below 2^-104 are scaled by at most 2^126: absolute error 2^-127 per value
        bound += 2.0 ** -21 * (np.abs(w) @ block_max) + 2.0 ** -126 * np.abs(w).sum(1)
    return exact, bound + 1e-30


@pytest.mark.parametrize("ggml_type,rows,cols", [
    (V.GGML_Q4_0, 1, 32), (V.GGML_Q4_0, 7, 96), (V.GGML_Q4_0, 2048, 2048), (V.GGML_Q4_0, 256, 11008),
    (V.GGML_Q4_0, 16387, 256),                         # one row per lane group, ragged last wave
    (V.GGML_Q8_0, 3, 64), (V.GGML_Q8_0, 8195, 160),    # ragged
    (V.GGML_Q4_0, 40003, 256), (V.GGML_Q8_0, 60001, 256),  # two rows per lane group, ragged last tile
    (V.GGML_Q8_0, 512, 2048), (V.GGML_F32, 5, 4), (V.GGML_F32, 300, 2052), (V.GGML_F32, 9000, 64),
    (V.GGML_Q4_0, 200003, 128),                        # several row tiles per wave, ragged last tile
    (V.GGML_Q8_0, 1000, 2560),                         # two pair steps per tile, the second partial
    (V.GGML_Q4_0, 64, 18944), (V.GGML_Q8_0, 40, 18944),  # staged input above 64 KB of LDS
    (V.GGML_Q8_0, 600, 11008),                         # 11.4 KB row tiles (the largest streamed tile)
    (V.GGML_Q4_0, 151936, 256),                        # four-row tiles of the 16-lane groups, many per wave
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


@pytest.mark.parametrize("ggml_type", [V.GGML_Q4_0, V.GGML_Q8_0])
def test_matvec_input_ranges(oracle_mod, ggml_type):
    """Blocks of x spanning 40 binades, an all-zero block, a block below 2^-104
    (scale clamped), a block near 1e30 and exact powers of two: the bound
    holds in every row."""
    rows, cols = 300, 2048
    rng = np.random.default_rng(75)
    x = S.normal(75, "gmvr", (cols,))
    x[0:32] *= np.exp2(rng.uniform(-30, 10, 32)).astype(np.float32)
    x[32:64] = 0.0
    x[64:96] *= np.float32(1e-33)
    x[96:128] *= np.float32(1e30)
    x[128:160] = np.exp2(rng.integers(-20, 20, 32)).astype(np.float32) * rng.choice([-1, 1], 32)
    x[160] = np.float32(2.0 ** 21)
    data = S.ggml_tensor(75, f"gmvr{ggml_type}", ggml_type, rows, cols)
    got = V.matvec(_dev(data), ggml_type, _dev(x), rows).cpu().numpy()
    exact, bound = _matvec_bound(oracle_mod, data, ggml_type, x, cols, rows)
    err = np.abs(got.astype(np.float64) - exact)
    print(f"ranges type {ggml_type}: max err / bound {float((err / bound).max()):.3f}")
    assert np.all(err <= bound)
    # each block alone (x zero elsewhere): the per-block bound, not the row's largest block, holds
    for b in range(6):
        xb = np.zeros_like(x)
        xb[32 * b:32 * b + 32] = x[32 * b:32 * b + 32]
        got = V.matvec(_dev(data), ggml_type, _dev(xb), rows).cpu().numpy()
        exact, bound = _matvec_bound(oracle_mod, data, ggml_type, xb, cols, rows)
        assert np.all(np.abs(got.astype(np.float64) - exact) <= bound), b


def test_matvec_nonfinite_input(oracle_mod):
    """A NaN or inf input value makes every row non-finite, as in the reference
    (the reference gives +-inf or NaN per row; the block kernel gives NaN)."""
    rows, cols = 64, 2048
    for ggml_type in (V.GGML_Q4_0, V.GGML_Q8_0):
        data = S.ggml_tensor(76, f"gmvnf{ggml_type}", ggml_type, rows, cols)
        for bad in (np.nan, np.inf):
            x = S.normal(76, "gmvnfx", (cols,))
            x[1000] = bad
            got = V.matvec(_dev(data), ggml_type, _dev(x), rows).cpu().numpy()
            orc = oracle_mod.matvec_f32(data, ggml_type, x, cols, rows)
            assert not np.isfinite(got).any() and not np.isfinite(orc).any()


@pytest.mark.parametrize("ggml_type,rows,cols,shift", [
    (V.GGML_Q4_0, 300, 2048, 4), (V.GGML_Q8_0, 300, 2048, 8),  # weights 4 / 8 bytes past 16: strided kernel
    (V.GGML_Q4_0, 7, 128, 0),                                 # 7 x 72 bytes, not a multiple of 16: strided
    (V.GGML_Q8_0, 200, 18944, 0),                             # 20 KB rows: past the streamed tile
])
def test_matvec_strided_pair_kernel(oracle_mod, ggml_type, rows, cols, shift):
    """Even block counts that the streamed kernel declines, at a dword-aligned
    tensor start: the strided pair kernel's results."""
    data = S.ggml_tensor(77, f"gmvs{ggml_type}{rows}{cols}", ggml_type, rows, cols)
    x = S.normal(77, f"gmvsx{cols}", (cols,))
    buf = torch.zeros(data.size + 16, dtype=torch.uint8, device=DEV)
    buf[shift:shift + data.size] = _dev(data)
    got = V.matvec(buf[shift:], ggml_type, _dev(x), rows).cpu().numpy()
    exact, bound = _matvec_bound(oracle_mod, data, ggml_type, x, cols, rows)
    assert np.all(np.abs(got.astype(np.float64) - exact) <= bound)


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

"""GPU parity of te_hip_gemm_q_f32 (the batched-prefill projections): every
row of the product against the fp64 product of the oracle's pre-op output
and dequantized weights.

Bound per output: 2^-14 sum_blocks max|x_block| sum_block |w| (the
activations' 15-bit block rounding) + (blocks + 2) 2^-24 sum |w x| (fp32
accumulation per block) + 2^-21 sum |w x| (the pre-op's last bits: RMSNorm and
SwiGLU within 2 ulps of the oracle's).
"""
import ctypes

import numpy as np
import pytest

import _synth as S

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from tinymetalagent_amd import runtime as R  # noqa: E402

DEV = "cuda"


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _run(oracle_mod, ggml_type, rows, n, k, pre=0, resid=False, seed=3, scale=1.0, split_bytes=0, clip=None,
         w_scale=0.05):
    lib = R.load_library()
    w = S.ggml_tensor(seed, f"gw{ggml_type}{n}{k}", ggml_type, n, k, scale=w_scale)
    x = S.normal(seed, "gx", (rows, k))
    if clip is not None:
        x = np.clip(x, -clip, clip)
    x = (x.astype(np.float64) * scale).astype(np.float32)
    x2 = S.normal(seed, "gx2", (rows, k))
    nw = S.normal(seed, "gnw", (k,), 0.1) + 1.0
    r = S.normal(seed, "gr", (rows, n))
    if pre == 1:
        xp = np.stack([oracle_mod.rmsnorm_f32(x[i], nw, 1e-6) for i in range(rows)])
    elif pre == 2:
        xp = np.stack([oracle_mod.swiglu_f32(x[i], x2[i]) for i in range(rows)])
    else:
        xp = x
    wf = oracle_mod.dequantize_rows(w, ggml_type, k, n).astype(np.float64)
    exact = xp.astype(np.float64) @ wf.T
    if resid:
        exact += r
    ax = np.abs(xp.astype(np.float64))
    bmax = np.repeat(ax.reshape(rows, k // 32, 32).max(2), 32, axis=1)
    awx = ax @ np.abs(wf).T
    bound = 2.0 ** -14 * (bmax @ np.abs(wf).T) + ((k // 32 + 2) * 2.0 ** -24 + 2.0 ** -21) * awx + 1e-30
    if resid:
        bound += 2.0 ** -24 * (np.abs(r) + awx)
    dw, dx, dx2, dn, dr = _dev(w), _dev(x), _dev(x2), _dev(nw), _dev(r)
    out = torch.empty(rows, n, device=DEV)
    act = torch.empty(lib.te_hip_gemm_act_bytes(rows, k), dtype=torch.uint8, device=DEV)
    part = torch.empty(max(split_bytes, 4), dtype=torch.uint8, device=DEV)
    R.check(lib.te_hip_gemm_q_f32(dw.data_ptr(), ggml_type, dx.data_ptr(), dx2.data_ptr(), dn.data_ptr(), 1e-6, pre,
                                  rows, n, k, out.data_ptr(), dr.data_ptr() if resid else None, act.data_ptr(),
                                  part.data_ptr() if split_bytes else None, split_bytes, None))
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    ratio = float((np.abs(got - exact) / bound).max())
    print(f"gemm type {ggml_type} {rows}x{n}x{k} pre {pre}: max err / bound {ratio:.3f}")
    assert np.all(np.abs(got - exact) <= bound)
    return got


@pytest.mark.parametrize("ggml_type,rows,n,k", [
    (2, 1, 64, 64), (2, 7, 100, 96), (8, 64, 64, 2048), (2, 130, 257, 256), (8, 65, 33, 512), (2, 256, 512, 2048),
    # Q8_0 stages a weight chunk of 8 blocks in two halves: one partial chunk
    # (no second half staged ahead), and a full chunk then a partial one
    (8, 7, 100, 96), (8, 130, 257, 288)])
def test_gemm_vs_fp64(oracle_mod, ggml_type, rows, n, k):
    _run(oracle_mod, ggml_type, rows, n, k)


@pytest.mark.parametrize("ggml_type,rows,n,k,resid", [
    (2, 256, 2048, 11008 // 32 * 32, True), (8, 100, 256, 2048, False), (2, 33, 96, 512, True)])
def test_gemm_split_k(oracle_mod, ggml_type, rows, n, k, resid):
    """Small output grids split K over up to 8 parts (partial sums, then a
    fixed-order reduction); same bound, and the same result on a second call."""
    a = _run(oracle_mod, ggml_type, rows, n, k, resid=resid, split_bytes=8 * rows * n * 4)
    b = _run(oracle_mod, ggml_type, rows, n, k, resid=resid, split_bytes=8 * rows * n * 4)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("pre", [1, 2])
def test_gemm_pre_ops_and_residual(oracle_mod, pre):
    _run(oracle_mod, 2, 70, 96, 1024, pre=pre, resid=True)
    _run(oracle_mod, 8, 33, 64, 11008 // 32 * 32, pre=pre)


def test_gemm_input_ranges(oracle_mod):
    """Rows of very different magnitude (1e-30 .. 1e30) and zero rows."""
    lib = R.load_library()
    for scale in (1e-30, 1e-3, 1e30):
        _run(oracle_mod, 2, 40, 64, 256, scale=scale)
    # finite blocks whose largest magnitude is in (3e38, FLT_MAX] take the finite
    # scale 2^114 (small weights keep every block sum inside fp32)
    got = _run(oracle_mod, 2, 2, 40, 64, scale=3.3e38, clip=1.0, w_scale=1e-3)
    assert np.isfinite(got).all()


def test_gemm_argument_checks():
    lib = R.load_library()
    f = torch.zeros(4096, device=DEV)
    p = f.data_ptr()
    assert lib.te_hip_gemm_q_f32(None, 2, p, p, p, 1e-6, 0, 4, 4, 64, p, None, p, None, 0, None) == 1
    assert lib.te_hip_gemm_q_f32(p, 2, p, p, None, 1e-6, 1, 4, 4, 64, p, None, p, None, 0, None) == 1  # no weight
    assert lib.te_hip_gemm_q_f32(p, 2, p, None, None, 1e-6, 2, 4, 4, 64, p, None, p, None, 0, None) == 1  # no up
    assert lib.te_hip_gemm_q_f32(p, 12, p, p, p, 1e-6, 0, 4, 4, 64, p, None, p, None, 0, None) == 3  # Q4_K
    assert lib.te_hip_gemm_q_f32(p, 2, p, p, p, 1e-6, 0, 4, 4, 48, p, None, p, None, 0, None) == 3  # k % 32
    assert lib.te_hip_gemm_q_f32(p + 1, 2, p, p, p, 1e-6, 0, 4, 4, 64, p, None, p, None, 0, None) == 3  # odd

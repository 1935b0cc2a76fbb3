"""GPU parity of te_hip_sample_top_k_f32 (device candidate search, host scan
and draw) against the oracle's restatement of the reference sampler
(qwen.c:1182-1250, pinned by test_model_cpu.py): for the same logits, top-k,
temperature and RNG state, the same token and the same next state, bit for
bit.  The cases cover what decides which logits reach the host: ties, every
logit entering the list (increasing logits), almost none entering
(decreasing), vocabularies shorter than a block or than k, k at 1 and at the
1024 cap, a NaN logit (the host then scans every logit) and infinities."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from oracle import text as OT  # noqa: E402
from tinymetalagent_amd import runtime as R  # noqa: E402


def _device_sample(logits, k, temperature, state):
    lib = R.load_library()
    x = torch.from_numpy(np.ascontiguousarray(logits, np.float32)).cuda()
    ws = torch.empty(lib.te_hip_sample_workspace_bytes(x.numel()), dtype=torch.uint8, device="cuda")
    rng = ctypes.c_uint64(state)
    tok = ctypes.c_uint32(0xFFFFFFFF)
    R.check(lib.te_hip_sample_top_k_f32(x.data_ptr(), x.numel(), k, temperature, ctypes.byref(rng),
                                        ctypes.byref(tok), ws.data_ptr(), ws.numel(), None))
    return tok.value, rng.value


def _check(logits, k, temperature, state, what):
    got_tok, got_state = _device_sample(logits, k, temperature, state)
    want_tok, want_state, _ = OT.sample(np.asarray(logits, np.float32), temperature, k, state)
    print(f"{what}: token {got_tok} (oracle {want_tok})")
    assert (got_tok, got_state) == (want_tok, want_state), what


VOCAB = 151936


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_sample_normal_logits(seed):
    rng = np.random.default_rng(seed)
    logits = rng.normal(0.0, 3.0, VOCAB).astype(np.float32)
    for draw in range(6):
        _check(logits, 40, 0.3, 0x9E3779B97F4A7C15 + 977 * draw + seed, f"normal seed {seed} draw {draw}")
    _check(logits, 40, 1.5, 12345 + seed, "T 1.5")


def test_sample_ties_and_orders():
    rng = np.random.default_rng(7)
    ties = np.round(rng.normal(0.0, 2.0, VOCAB) * 2.0) / 2.0  # values on a 0.5 grid: many equal logits
    _check(ties, 40, 0.3, 99, "ties")
    _check(ties, 1000, 0.8, 98, "ties, k 1000")
    inc = np.linspace(-8.0, 8.0, VOCAB)  # every logit enters the list
    _check(inc, 40, 0.3, 97, "increasing")
    dec = inc[::-1].copy()  # only the fill enters
    _check(dec, 40, 0.3, 96, "decreasing")
    late = rng.normal(0.0, 1.0, VOCAB)
    late[-5:] += 30.0  # the winners in the last, partial block
    _check(late, 40, 0.3, 95, "late winners")


def test_sample_few_distinct_values():
    """Four distinct logit values over the whole vocabulary: every replacement
    meets ties, so the list's minimum slot (the first slot of the smallest
    value) decides which slot each new logit takes, and the draw walks the
    slots in that order."""
    rng = np.random.default_rng(13)
    few = np.floor(rng.uniform(0.0, 4.0, VOCAB)).astype(np.float32)
    for k, state in ((40, 31), (300, 32), (1024, 33)):
        _check(few, k, 0.7, state, f"four values, k {k}")
    signed_zeros = np.where(rng.uniform(size=20000) < 0.5, -0.0, 0.0).astype(np.float32)
    signed_zeros[[5, 777, 19000]] = [1.0, 2.0, 1.0]
    _check(signed_zeros, 40, 0.3, 34, "signed zeros")


def test_sample_small_and_edge_cases():
    rng = np.random.default_rng(11)
    _check(rng.normal(size=700), 40, 0.3, 5, "vocab 700")
    _check(rng.normal(size=25), 40, 0.3, 6, "vocab below k")
    _check(rng.normal(size=3000), 1, 0.3, 7, "k 1")
    _check(rng.normal(size=3000), 0, 0.3, 8, "k 0 (means 1)")
    _check(rng.normal(size=5000), 1024, 0.3, 9, "k 1024")
    _check(rng.normal(size=VOCAB), 4000, 0.3, 10, "k above the cap")
    inf = rng.normal(size=20000)
    inf[[3, 15000]] = [np.inf, -np.inf]
    _check(inf, 40, 0.3, 11, "infinities")
    nan = rng.normal(size=20000)
    nan[[17, 12345]] = np.nan
    _check(nan, 40, 0.3, 12, "NaN logits")
    _check(np.zeros(9000), 40, 0.3, 13, "all equal")


def test_sample_argument_checks():
    lib = R.load_library()
    rng = ctypes.c_uint64(1)
    tok = ctypes.c_uint32(0)
    x = torch.zeros(100, device="cuda")
    ws = torch.empty(lib.te_hip_sample_workspace_bytes(100), dtype=torch.uint8, device="cuda")
    bad = lib.te_hip_sample_top_k_f32(x.data_ptr(), 100, 40, 0.3, ctypes.byref(rng), ctypes.byref(tok),
                                      ws.data_ptr(), ws.numel() - 1, None)
    assert bad == 1  # INVALID_ARGUMENT: workspace too small
    assert lib.te_hip_sample_top_k_f32(None, 100, 40, 0.3, ctypes.byref(rng), ctypes.byref(tok), ws.data_ptr(),
                                       ws.numel(), None) == 1
    assert lib.te_hip_sample_workspace_bytes(0) == 0

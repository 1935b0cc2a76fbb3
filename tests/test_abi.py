"""CPU checks of the C-ABI boundary: the library loads, exports every symbol the
headers declare and every symbol the reference ctypes binding binds, and
honours the reference's status conventions on argument errors (no compute
calls: these run without a GPU)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]

# python/tinyengine/runtime.py:271-378 of the reference binds these 22 symbols.
REFERENCE_BINDING_SYMBOLS = [
    "te_strerror", "te_detect_arch", "te_get_capabilities", "te_make_kernel_plan",
    "te_kernel_plan_supports_quant", "te_kernel_plan_optimizes_quant", "te_kernel_plan_supports_op",
    "te_model_load_gguf", "te_model_get_info", "te_model_get_tokenizer_info", "te_model_get_tensor_info",
    "te_format_qwen_chat_prompt", "te_model_tokenize", "te_model_detokenize", "te_model_read_f32_tensor",
    "te_model_dequantize_row_f32", "te_model_matvec_f32", "te_model_free", "te_context_create",
    "te_context_free", "te_generate", "te_generate_raw",
]


@pytest.fixture(scope="module")
def lib():
    from tinymetalagent_amd import runtime

    return runtime.load_library()


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        for m in re.finditer(r"TE_API\s+[^;(]*?\b(te_\w+)\s*\(", text, re.S):
            names.add(m.group(1))
    return sorted(names)


def test_every_header_symbol_is_exported(lib):
    names = declared_symbols()
    assert len(names) >= 45
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_reference_binding_symbols_resolve(lib):
    for n in REFERENCE_BINDING_SYMBOLS:
        assert hasattr(lib, n), n


def test_status_strings(lib):
    want = {0: "ok", 1: "invalid argument", 2: "I/O error", 3: "unsupported", 4: "out of memory",
            5: "runtime error", 99: "unknown error"}
    for k, v in want.items():
        assert lib.te_strerror(k).decode() == v


def test_defaults_and_capabilities():
    from tinymetalagent_amd import runtime

    lib = runtime.load_library()
    opts = lib.te_default_options()
    assert (opts.abi_version, opts.context_tokens, opts.batch_tokens) == (3, 512, 128)
    caps = runtime.capabilities()
    assert caps.abi_version == 3 and caps.backend_name == "hip-gfx950"
    for op in (runtime.TE_OP_ROPE, runtime.TE_OP_CAUSAL_ATTENTION, runtime.TE_OP_KV_CACHE):
        assert caps.vector_op_mask >> op & 1
    plan = runtime._KernelPlan()
    o = runtime._RuntimeOptions(abi_version=3, context_tokens=8192)
    runtime.check(lib.te_make_kernel_plan(ctypes.byref(o), ctypes.byref(plan)))
    assert lib.te_kernel_plan_supports_op(ctypes.byref(plan), runtime.TE_OP_CAUSAL_ATTENTION) == 1
    for op in (0, 4, 7, 8, 9):  # matvec, RMSNorm, SwiGLU, residual add, argmax
        assert lib.te_kernel_plan_supports_op(ctypes.byref(plan), op) == 1
    for op in (3, 10, 12):  # decode token, sampling, tokenize
        assert lib.te_kernel_plan_supports_op(ctypes.byref(plan), op) == 1
    assert lib.te_kernel_plan_supports_op(ctypes.byref(plan), 1) == 0  # matmul: not in this build
    for quant, want in ((1, 1), (2, 1), (4, 1), (8, 1), (5, 0), (11, 0)):  # F32 F16 Q4_0 Q8_0 | Q4_1 Q4_K
        assert lib.te_kernel_plan_supports_quant(ctypes.byref(plan), quant) == want
    assert plan.max_context_tokens == 8192
    o.abi_version = 2
    assert lib.te_make_kernel_plan(ctypes.byref(o), ctypes.byref(plan)) == runtime.TE_STATUS_UNSUPPORTED


# Reference c/src/tinyengine.c:36-83 (te_quant_name) and :85-118 (te_vector_op_name),
# in enum order (c/include/tinyengine.h:46-87); out-of-range values print the default.
REFERENCE_QUANT_NAMES = [
    "UNKNOWN", "F32", "F16", "BF16", "GGUF_Q4_0", "GGUF_Q4_1", "GGUF_Q5_0", "GGUF_Q5_1", "GGUF_Q8_0",
    "GGUF_Q2_K", "GGUF_Q3_K", "GGUF_Q4_K", "GGUF_Q5_K", "GGUF_Q6_K", "GGUF_Q8_K", "GGUF_IQ2_XXS",
    "GGUF_IQ2_XS", "GGUF_IQ3_XXS", "GGUF_IQ3_S", "GGUF_IQ4_NL", "GGUF_IQ4_XS", "MXFP4",
]
REFERENCE_OP_NAMES = [
    "matvec", "matmul", "batched-prefill", "decode-token", "rmsnorm", "rope", "causal-attention",
    "swiglu", "residual-add", "argmax", "sampling", "kv-cache", "tokenize",
]


def test_quant_and_op_names_match_reference(lib):
    lib.te_quant_name.restype = ctypes.c_char_p
    lib.te_quant_name.argtypes = [ctypes.c_int]
    lib.te_vector_op_name.restype = ctypes.c_char_p
    lib.te_vector_op_name.argtypes = [ctypes.c_int]
    assert [lib.te_quant_name(i).decode() for i in range(22)] == REFERENCE_QUANT_NAMES
    for bad in (22, 99, -1):  # TE_QUANT_COUNT and out of range: the reference's default
        assert lib.te_quant_name(bad).decode() == "UNKNOWN"
    assert [lib.te_vector_op_name(i).decode() for i in range(13)] == REFERENCE_OP_NAMES
    for bad in (13, 99, -1):
        assert lib.te_vector_op_name(bad).decode() == "unknown"


def test_kernel_plan_defaults_match_reference(lib):
    """Reference tinyengine.c:201-235: NULL options mean te_default_options(),
    ABI version 0 is accepted, a NULL plan is an invalid argument."""
    from tinymetalagent_amd import runtime

    plan = runtime._KernelPlan()
    assert lib.te_make_kernel_plan(None, ctypes.byref(plan)) == runtime.TE_STATUS_OK
    assert plan.abi_version == 3 and plan.max_context_tokens == 512  # the default options' context
    o = runtime._RuntimeOptions(abi_version=0, context_tokens=4096)
    assert lib.te_make_kernel_plan(ctypes.byref(o), ctypes.byref(plan)) == runtime.TE_STATUS_OK
    assert plan.abi_version == 3 and plan.max_context_tokens == 4096
    assert lib.te_make_kernel_plan(ctypes.byref(o), None) == runtime.TE_STATUS_INVALID_ARGUMENT
    # te_compile_kernels (reference :237-246): the plan is required, the options are not
    assert lib.te_compile_kernels(None, None) == runtime.TE_STATUS_INVALID_ARGUMENT
    bad = runtime._KernelPlan()
    ctypes.memmove(ctypes.byref(bad), ctypes.byref(plan), ctypes.sizeof(plan))
    bad.abi_version = 2
    assert lib.te_compile_kernels(None, ctypes.byref(bad)) == runtime.TE_STATUS_UNSUPPORTED


def test_public_attention_argument_checks(lib):
    f = np.ones(64, np.float32)
    p = f.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    # te_rope_f32: reference ops.c:302-304
    assert lib.te_rope_f32(None, 1, 8, 0, ctypes.c_float(1e6)) == 1
    assert lib.te_rope_f32(p, 0, 8, 0, ctypes.c_float(1e6)) == 1
    assert lib.te_rope_f32(p, 1, 7, 0, ctypes.c_float(1e6)) == 1
    assert lib.te_rope_f32(p, 1, 8, 0, ctypes.c_float(0.0)) == 1
    # te_attention_decode_f32: reference ops.c:333-339
    assert lib.te_attention_decode_f32(p, p, p, 0, 3, 2, 4, p) == 1
    assert lib.te_attention_decode_f32(None, p, p, 0, 2, 1, 4, p) == 1
    assert lib.te_attention_decode_f32(p, p, p, 2 ** 64 - 1, 2, 1, 4, p) == 3


def test_public_vector_op_argument_checks(lib):
    """The reference checks of ops.c:272-433 before any device work."""
    f = np.ones(8, np.float32)
    p = f.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    idx = ctypes.c_uint32(0)
    assert lib.te_rmsnorm_f32(None, p, 8, ctypes.c_float(1e-6), p) == 1
    assert lib.te_rmsnorm_f32(p, p, 0, ctypes.c_float(1e-6), p) == 1
    assert lib.te_rmsnorm_f32(p, p, 8, ctypes.c_float(0.0), p) == 1  # epsilon <= 0
    assert lib.te_swiglu_f32(p, None, 8, p) == 1
    assert lib.te_add_f32(p, p, 0, p) == 1
    assert lib.te_argmax_f32(p, 0, ctypes.byref(idx)) == 1
    assert lib.te_argmax_f32(p, 8, None) == 1
    buf = ctypes.c_void_p(0x1000)  # never dereferenced: every call fails its checks first
    assert lib.te_hip_matvec_f32(buf, 2, buf, 48, 4, buf, None) == 3  # cols not a multiple of 32
    assert lib.te_hip_matvec_f32(buf, 14, buf, 64, 4, buf, None) == 3  # Q8_K: not here
    assert lib.te_hip_matvec_f32(buf, 0, buf, 6, 4, buf, None) == 3  # F32 cols % 4
    assert lib.te_hip_matvec_f32(buf, 2, buf, 64, 0, buf, None) == 1
    assert lib.te_hip_rmsnorm_f32(buf, buf, 1, 8, ctypes.c_float(-1.0), buf, None) == 1
    assert lib.te_hip_argmax_f32(buf, 0, buf, None) == 1


def test_backend_guard_conventions(lib):
    """NULL first argument -> INVALID_ARGUMENT or UNSUPPORTED; unsupported shape -> UNSUPPORTED
    (the convention of reference c/tests/generate_metal_guard_tests.py:68-79)."""
    from tinymetalagent_amd import runtime

    buf = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails its checks first
    ws = ctypes.c_void_p(0x2000)
    ok = (runtime.TE_STATUS_INVALID_ARGUMENT, runtime.TE_STATUS_UNSUPPORTED)
    assert lib.te_hip_rope_kv_append_f16(None, buf, buf, None, None, None, buf, buf, buf, buf, None,
                                         1, 1, 1, None, 0, 8, 2, 1, 4, None) in ok
    assert lib.te_hip_rope_kv_append_f16(buf, buf, buf, None, None, None, buf, buf, buf, buf, None,
                                         1, 1, 1, None, 0, 8, 2, 1, 3, None) == 1  # odd head_dim
    assert lib.te_hip_rope_kv_append_f16(buf, buf, buf, None, None, None, buf, buf, buf, buf, None,
                                         1, 1, 4, None, 6, 8, 2, 1, 4, None) == 1  # positions past the cache
    assert lib.te_hip_attention_decode_splitk_f16(None, buf, buf, None, 0, 1, 1, 8, 2, 1, 128, ws, 1 << 20,
                                                  None) in ok
    assert lib.te_hip_attention_decode_splitk_f16(buf, buf, buf, None, 0, 1, 1, 8, 2, 1, 96, ws, 1 << 20,
                                                  None) == 3  # head_dim 96
    assert lib.te_hip_attention_decode_splitk_f16(buf, buf, buf, None, 0, 1, 1, 8, 34, 2, 128, ws, 1 << 20,
                                                  None) == 3  # group of 17 heads
    assert lib.te_hip_attention_decode_splitk_f16(buf, buf, buf, None, 8, 1, 1, 8, 2, 1, 128, ws, 1 << 20,
                                                  None) == 1  # position >= context
    assert lib.te_hip_attention_decode_splitk_f16(buf, buf, buf, None, 0, 1, 1, 8, 2, 1, 128, ws, 16,
                                                  None) == 1  # workspace too small
    for fn in (lib.te_hip_attention_decode_step_f16, lib.te_hip_attention_decode_step_splitk_f16):
        tail = (buf, ws, 1 << 20, None) if fn is lib.te_hip_attention_decode_step_f16 else (ws, 1 << 20, None)
        assert fn(buf, None, buf, None, None, None, buf, buf, buf, buf, None, 0, 1, 1, 8, 2, 1, 128,
                  *tail) == 1  # no k_new
        assert fn(buf, buf, buf, None, None, None, buf, buf, buf, buf, None, 0, 1, 1, 8, 2, 1, 96,
                  *tail) == 3  # head_dim 96
        assert fn(buf, buf, buf, None, None, None, buf, buf, buf, buf, None, 8, 1, 1, 8, 2, 1, 128,
                  *tail) == 1  # position >= context
    assert lib.te_hip_attention_prefill_f16(None, buf, buf, 1, 1, 4, 0, 8, 2, 1, 128, buf, None) in ok
    assert lib.te_hip_attention_prefill_f16(buf, buf, buf, 1, 1, 4, 6, 8, 2, 1, 128, buf, None) == 1
    assert lib.te_hip_attention_prefill_f16(buf, buf, buf, 1, 1, 4, 0, 8, 2, 1, 80, buf, None) == 3
    assert lib.te_hip_attention_prefill_workspace_bytes(1, 1, 4, 6, 8, 2, 1, 128) == 0  # chunk past the cache
    assert lib.te_hip_attention_prefill_workspace_bytes(1, 1, 4, 0, 8, 2, 1, 80) == 0  # head_dim 80
    need = lib.te_hip_attention_prefill_workspace_bytes(1, 1, 300, 0, 300, 16, 2, 128)
    vt = lib.te_hip_value_t_bytes(1, 1, 300, 2, 128)
    assert vt == 2 * 128 * 320 * 2  # [kv][head_dim][ctx rounded up to 64] fp16
    part = lib.te_hip_attention_prefill_vt_workspace_bytes(1, 1, 300, 0, 300, 16, 2, 128)
    assert need == part + vt
    assert part % (300 * 16 * 130 * 4) == 0  # splits x rows x heads x (head_dim + 2) floats
    split = lib.te_hip_attention_prefill_split_f16
    assert split(None, buf, buf, 1, 1, 4, 0, 8, 2, 1, 128, buf, None, 0, None) in ok
    assert split(buf, buf, buf, 1, 1, 4, 0, 8, 2, 1, 80, buf, None, 0, None) == 3  # head_dim 80
    assert split(buf, buf, buf, 1, 1, 300, 0, 300, 16, 2, 128, buf, None, 0, None) == 1  # workspace missing
    assert split(buf, buf, buf, 1, 1, 300, 0, 300, 16, 2, 128, buf, ws, need - 1, None) == 1  # too small
    vt_attn = lib.te_hip_attention_prefill_vt_f16
    assert vt_attn(None, buf, buf, 1, 1, 4, 0, 8, 2, 1, 128, buf, None, 0, None) in ok
    assert vt_attn(buf, buf, buf, 1, 1, 4, 6, 8, 2, 1, 128, buf, None, 0, None) == 1  # chunk past the cache
    assert vt_attn(buf, buf, buf, 1, 1, 4, 0, 8, 2, 1, 80, buf, None, 0, None) == 3  # head_dim 80
    if part:
        assert vt_attn(buf, buf, buf, 1, 1, 300, 0, 300, 16, 2, 128, buf, ws, part - 1, None) == 1  # too small
    tr = lib.te_hip_value_transpose_f16
    assert tr(None, buf, 1, 1, 0, 4, 8, 2, 128, None) == 1
    assert tr(buf, buf, 1, 1, 6, 4, 8, 2, 128, None) == 1  # range past the cache
    assert tr(buf, buf, 1, 1, 0, 4, 8, 2, 96, None) == 3  # head_dim 96
    assert tr(buf, buf, 1, 1, 3, 0, 8, 2, 128, None) == 0  # nothing to do
    step_vt = lib.te_hip_attention_prefill_step_vt_f16
    assert step_vt(buf, buf, buf, None, None, None, buf, buf, buf, buf, None, 1, 1, 4, 0, 8, 2, 1, 128,
                   buf, None, 0, None) == 1  # no V^T buffer
    assert step_vt(buf, buf, buf, None, None, None, buf, buf, buf, buf, buf, 1, 1, 4, 0, 8, 2, 1, 80,
                   buf, None, 0, None) == 3  # head_dim 80
    step = lib.te_hip_attention_prefill_step_f16
    assert step(buf, None, buf, None, None, None, buf, buf, buf, buf, 1, 1, 4, 0, 8, 2, 1, 128,
                buf, None) == 1  # no k_new
    assert step(buf, buf, buf, None, None, None, None, buf, buf, buf, 1, 1, 4, 0, 8, 2, 1, 128,
                buf, None) == 1  # no rope table
    assert step(buf, buf, buf, None, None, None, buf, buf, buf, buf, 1, 1, 4, 6, 8, 2, 1, 128,
                buf, None) == 1  # chunk past the cache
    assert step(buf, buf, buf, None, None, None, buf, buf, buf, buf, 1, 1, 4, 0, 8, 2, 1, 80,
                buf, None) == 3  # head_dim 80
    assert step(buf, buf, buf, None, None, None, buf, buf, buf, buf, 65, 1, 4, 0, 8, 2, 1, 128,
                buf, None) == 3  # more than 64 sequences
    assert lib.te_hip_calibrate_mfma_f16(0, 10, buf, None) == 1  # no workgroups
    assert lib.te_hip_calibrate_mfma_f16(1, 0, buf, None) == 1  # no iterations
    assert lib.te_hip_calibrate_mfma_f16(1, 10, None, None) == 1  # no output
    q = np.ones(8 * 64, np.float32).ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    assert lib.te_hip_attention_qk_mma_f32(None, q, 8, 8, 64, q) in ok
    assert lib.te_hip_attention_qk_mma_f32(q, q, 4, 8, 64, q) == 3
    assert lib.te_hip_attention_stream_mma_f32(q, q, q, 8, 12, 64, q) == 3
    assert lib.te_hip_attention_causal_mma_f32(q, q, q, 8, 24, 64, 25, q) == 3


def test_workspace_query(lib):
    n = lib.te_hip_attention_decode_workspace_bytes(None, 8192, 1, 36, 16, 2, 128)
    assert n > 0
    assert lib.te_hip_attention_decode_workspace_bytes(None, 8192, 0, 36, 16, 2, 128) == 0
    pos = (ctypes.c_size_t * 3)(100, 5000, 7)
    assert lib.te_hip_attention_decode_workspace_bytes(pos, 0, 3, 2, 28, 4, 128) > 0


def _chunking(lib, position, layers, kv_heads, fp32=0, positions=None):
    chunk, chunks = ctypes.c_size_t(), ctypes.c_size_t()
    seqs = 1 if positions is None else len(positions)
    arr = None if positions is None else (ctypes.c_size_t * seqs)(*positions)
    st = lib.te_hip_attention_decode_chunking(arr, ctypes.c_size_t(position), seqs, layers, kv_heads, fp32,
                                              ctypes.byref(chunk), ctypes.byref(chunks))
    assert st == 0
    return chunk.value, chunks.value


def test_decode_workspace_sized_at_the_last_position_serves_every_earlier_one(lib):
    """A caller sizes the decode workspace once, at context_tokens - 1 (the
    engine's context does), then decodes every position below it.  The launch
    needs seqs*layers*heads*chunks(p)*(head_dim+2)*4 bytes, and the chunk
    count is not monotone in p, so the size query must bound every p below."""
    lib.te_hip_attention_decode_workspace_bytes.restype = ctypes.c_size_t
    for layers, heads, kv, ctx in ((1, 16, 2, 131072), (1, 28, 4, 32768), (36, 16, 2, 32768),
                                   (28, 12, 2, 131072), (1, 14, 2, 4096)):
        have = lib.te_hip_attention_decode_workspace_bytes(None, ctypes.c_size_t(ctx - 1), 1, layers, heads, kv, 128)
        step = 1 if ctx <= 32768 else 7
        worst = 0
        for p in range(0, ctx, step):
            chunk, chunks = _chunking(lib, p, layers, kv)
            assert chunk % 32 == 0 and chunks * chunk >= p + 1 and (chunks - 1) * chunk < p + 1
            worst = max(worst, layers * heads * chunks * (128 + 2) * 4)
        assert worst <= have, (layers, heads, kv, ctx, worst, have)
    # the case that failed before: 1 layer, 2 KV heads, position 28608 against ctx 32768
    _, c_small = _chunking(lib, 28608, 1, 2)
    _, c_last = _chunking(lib, 32767, 1, 2)
    assert c_small > c_last
    have = lib.te_hip_attention_decode_workspace_bytes(None, ctypes.c_size_t(32767), 1, 1, 16, 2, 128)
    assert 16 * c_small * 130 * 4 <= have
    # ragged batches: sized at the largest position
    positions = [3924, 1976, 11519, 12470, 1263, 4276, 3298, 9268]
    _, chunks = _chunking(lib, 0, 28, 4, positions=positions)
    arr = (ctypes.c_size_t * 8)(*positions)
    assert 8 * 28 * 28 * chunks * 130 * 4 <= lib.te_hip_attention_decode_workspace_bytes(arr, 0, 8, 28, 28, 4, 128)


def test_fp32_decode_chunking_fits_the_combine_at_any_position(lib):
    """te_attention_decode_f32 accepts positions up to 2^30; its chunks must
    stay within the 4096 per-chunk weights the combine kernel keeps in LDS."""
    for p in [0, 1, 511, 512, 4096 * 512 - 1, 4096 * 512, 4096 * 512 + 1, 3_000_000, 2 ** 24 + 5,
              2 ** 30 - 1, 2 ** 30]:
        chunk, chunks = _chunking(lib, p, 1, 1, fp32=1)
        assert chunk % 512 == 0 and (chunk // 512) & (chunk // 512 - 1) == 0
        assert chunks <= 4096 and chunks * chunk >= p + 1 and (chunks - 1) * chunk < p + 1
    assert _chunking(lib, 4096 * 512 - 1, 1, 1, fp32=1) == (512, 4096)
    assert _chunking(lib, 4096 * 512, 1, 1, fp32=1) == (1024, 2049)


def test_model_and_generate_argument_statuses():
    """Missing file -> IO_ERROR (tinyengine.c:278-280), the "unsupported"
    text the agent layer matches, NULL handles -> INVALID_ARGUMENT."""
    from tinymetalagent_amd import runtime

    lib = runtime.load_library()
    model = ctypes.c_void_p()
    status = lib.te_model_load_gguf(b"/nonexistent.gguf", None, ctypes.byref(model))
    assert status == runtime.TE_STATUS_IO_ERROR and model.value is None
    with pytest.raises(runtime.TinyEngineError, match="^unsupported$"):
        runtime.check(runtime.TE_STATUS_UNSUPPORTED)
    assert lib.te_context_create(None, None, ctypes.byref(model)) == 1
    cb = runtime._TOKEN_CALLBACK(lambda *a: None)
    assert lib.te_generate(None, b"hi", 4, cb, None) == 1
    assert lib.te_generate_raw(None, b"hi", 4, cb, None) == 1
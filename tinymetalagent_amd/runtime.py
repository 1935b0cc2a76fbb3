"""ctypes binding over libtinyengine.so (this build).

Mirrors the reference binding python/tinyengine/runtime.py: the same library
search order (TINYENGINE_LIBRARY, then ./c/build, then next to the package --
runtime.py:244-258), the same struct layouts (runtime.py:18-129), the same
error convention (non-zero status -> TinyEngineError(te_strerror(status)),
runtime.py:381-384).  On top of the reference's symbols it binds the
attention-step entry points of include/tinyengine.h and the te_hip_* backend
slot of include/te_hip_backend.h.

There is no CPU fallback anywhere in this module: if the library or the GPU
is missing, calls raise.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

TE_ABI_VERSION = 3
TE_QUANT_COUNT = 22
TE_HIP_MAX_SEQS = 64

TE_STATUS_OK = 0
TE_STATUS_INVALID_ARGUMENT = 1
TE_STATUS_IO_ERROR = 2
TE_STATUS_UNSUPPORTED = 3
TE_STATUS_OUT_OF_MEMORY = 4
TE_STATUS_RUNTIME_ERROR = 5

TE_OP_ROPE = 5
TE_OP_CAUSAL_ATTENTION = 6
TE_OP_KV_CACHE = 11


class TinyEngineError(RuntimeError):
    """Raised with te_strerror(status) for any non-OK status."""

    def __init__(self, message: str, status: int | None = None):
        super().__init__(message)
        self.status = status


class _ArchInfo(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int),
        ("name", ctypes.c_char * 64),
        ("cpu_cores", ctypes.c_uint32),
        ("gpu_cores", ctypes.c_uint32),
        ("unified_memory_bytes", ctypes.c_uint64),
        ("recommended_max_context", ctypes.c_uint32),
    ]


class _RuntimeOptions(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("target_arch", ctypes.c_int),
        ("context_tokens", ctypes.c_uint32),
        ("batch_tokens", ctypes.c_uint32),
        ("memory_limit_bytes", ctypes.c_uint64),
        ("kernel_cache_dir", ctypes.c_char_p),
        ("flags", ctypes.c_uint32),
    ]


class _Capabilities(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("known_quant_mask", ctypes.c_uint64 * 2),
        ("optimized_quant_mask", ctypes.c_uint64 * 2),
        ("vector_op_mask", ctypes.c_uint64),
        ("optimization_flags", ctypes.c_uint32),
        ("preferred_alignment_bytes", ctypes.c_uint32),
        ("backend_name", ctypes.c_char * 32),
        ("notes", ctypes.c_char * 160),
    ]


class _KernelPlan(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("target_arch", ctypes.c_int),
        ("quant_mask", ctypes.c_uint64 * 2),
        ("optimized_quant_mask", ctypes.c_uint64 * 2),
        ("vector_op_mask", ctypes.c_uint64),
        ("optimization_flags", ctypes.c_uint32),
        ("q4_prefill_batch_tile", ctypes.c_uint32),
        ("q4_decode_row_tile", ctypes.c_uint32),
        ("q8_lm_head_row_tile", ctypes.c_uint32),
        ("dot_threads", ctypes.c_uint32),
        ("preferred_alignment_bytes", ctypes.c_uint32),
        ("max_context_tokens", ctypes.c_uint32),
        ("memory_budget_bytes", ctypes.c_uint64),
        ("metal_function_suffix", ctypes.c_char * 32),
    ]


_TOKEN_CALLBACK = ctypes.CFUNCTYPE(None, ctypes.c_char_p, ctypes.c_uint32, ctypes.c_void_p)

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_f32p = ctypes.POINTER(ctypes.c_float)
_szp = ctypes.POINTER(ctypes.c_size_t)
_int = ctypes.c_int


def _candidate_libraries() -> list[Path]:
    env = os.environ.get("TINYENGINE_LIBRARY")
    here = Path(__file__).resolve()
    candidates: list[Path] = []
    if env:
        candidates.append(Path(env))
    candidates.extend([
        Path.cwd() / "c" / "build" / "libtinyengine.so",
        here.parents[1] / "c" / "build" / "libtinyengine.so",
        here.parent / "libtinyengine.so",
    ])
    return candidates


_LIB: ctypes.CDLL | None = None


def library_path() -> Path:
    for cand in _candidate_libraries():
        if cand.is_file():
            return cand
    searched = "\n".join(str(p) for p in _candidate_libraries())
    raise TinyEngineError(f"Could not find libtinyengine. Searched:\n{searched}")


def load_library() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        lib = ctypes.CDLL(str(library_path()))
        _configure_library(lib)
        _LIB = lib
    return _LIB


def _sig(lib, name, argtypes, restype=_int):
    fn = getattr(lib, name)
    fn.argtypes = argtypes
    fn.restype = restype


def _configure_library(lib: ctypes.CDLL) -> None:
    # Reference binding symbols (python/tinyengine/runtime.py:271-378).
    _sig(lib, "te_strerror", [_int], ctypes.c_char_p)
    _sig(lib, "te_version", [], ctypes.c_char_p)
    _sig(lib, "te_detect_arch", [ctypes.POINTER(_ArchInfo)])
    _sig(lib, "te_get_capabilities", [ctypes.POINTER(_Capabilities)])
    _sig(lib, "te_make_kernel_plan", [ctypes.POINTER(_RuntimeOptions), ctypes.POINTER(_KernelPlan)])
    _sig(lib, "te_kernel_plan_supports_quant", [ctypes.POINTER(_KernelPlan), _int])
    _sig(lib, "te_kernel_plan_optimizes_quant", [ctypes.POINTER(_KernelPlan), _int])
    _sig(lib, "te_kernel_plan_supports_op", [ctypes.POINTER(_KernelPlan), _int])
    _sig(lib, "te_model_load_gguf", [ctypes.c_char_p, ctypes.POINTER(_RuntimeOptions), ctypes.POINTER(_vp)])
    _sig(lib, "te_context_create", [_vp, ctypes.POINTER(_RuntimeOptions), ctypes.POINTER(_vp)])
    _sig(lib, "te_context_free", [_vp], None)
    _sig(lib, "te_generate", [_vp, ctypes.c_char_p, ctypes.c_uint32, _TOKEN_CALLBACK, _vp])
    _sig(lib, "te_generate_raw", [_vp, ctypes.c_char_p, ctypes.c_uint32, _TOKEN_CALLBACK, _vp])
    _sig(lib, "te_default_options", [], _RuntimeOptions)
    _sig(lib, "te_model_get_info", [_vp, _vp])
    _sig(lib, "te_model_get_tokenizer_info", [_vp, _vp])
    _sig(lib, "te_model_get_tensor_info", [_vp, ctypes.c_char_p, _vp])
    _sig(lib, "te_format_qwen_chat_prompt", [ctypes.c_char_p, ctypes.c_char_p, _sz, _szp])
    _sig(lib, "te_model_tokenize", [_vp, ctypes.c_char_p, _int, ctypes.POINTER(ctypes.c_uint32), _sz, _szp])
    _sig(lib, "te_model_detokenize",
         [_vp, ctypes.POINTER(ctypes.c_uint32), _sz, _int, ctypes.c_char_p, _sz, _szp])
    _sig(lib, "te_model_read_f32_tensor", [_vp, ctypes.c_char_p, _f32p, _sz, _szp])
    _sig(lib, "te_model_dequantize_row_f32", [_vp, ctypes.c_char_p, ctypes.c_uint64, _f32p, _sz, _szp])
    _sig(lib, "te_model_matvec_f32", [_vp, ctypes.c_char_p, _f32p, _sz, _f32p, _sz, _szp])
    _sig(lib, "te_model_free", [_vp], None)
    # Attention step, public (include/tinyengine.h).
    _sig(lib, "te_rope_f32", [_f32p, _sz, _sz, _sz, ctypes.c_float])
    _sig(lib, "te_attention_decode_f32", [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _f32p])
    _sig(lib, "te_rmsnorm_f32", [_f32p, _f32p, _sz, ctypes.c_float, _f32p])
    _sig(lib, "te_swiglu_f32", [_f32p, _f32p, _sz, _f32p])
    _sig(lib, "te_add_f32", [_f32p, _f32p, _sz, _f32p])
    _sig(lib, "te_argmax_f32", [_f32p, _sz, ctypes.POINTER(ctypes.c_uint32)])
    # HIP backend slot (include/te_hip_backend.h).
    _sig(lib, "te_hip_available", [], _int)
    _sig(lib, "te_hip_device_info", [ctypes.c_char_p, _sz, ctypes.POINTER(ctypes.c_uint32)])
    _sig(lib, "te_hip_rope_table_f32", [_vp, _vp, _sz, _sz, ctypes.c_float])
    _sig(lib, "te_hip_rope_kv_append_f16",
         [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _szp, _sz, _sz, _sz, _sz, _sz, _vp])
    _sig(lib, "te_hip_attention_decode_workspace_bytes", [_szp, _sz, _sz, _sz, _sz, _sz, _sz], _sz)
    _sig(lib, "te_hip_attention_decode_f16",
         [_vp, _vp, _vp, _szp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _sz, _vp])
    _sig(lib, "te_hip_attention_decode_splitk_f16",
         [_vp, _vp, _vp, _szp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _sz, _vp])
    _sig(lib, "te_hip_attention_decode_combine", [_szp, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _sz, _vp])
    _sig(lib, "te_hip_attention_decode_step_f16",
         [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _szp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _sz,
          _vp])
    _sig(lib, "te_hip_attention_decode_step_splitk_f16",
         [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _szp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _sz, _vp])
    _sig(lib, "te_hip_attention_decode_step_noalloc_f16",
         [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _szp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _vp])
    _sig(lib, "te_hip_attention_decode_chunking", [_szp, _sz, _sz, _sz, _sz, _int, _szp, _szp])
    _sig(lib, "te_hip_attention_prefill_f16", [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _vp])
    _sig(lib, "te_hip_value_t_bytes", [_sz] * 5, _sz)
    _sig(lib, "te_hip_value_transpose_f16", [_vp, _vp] + [_sz] * 7 + [_vp])
    _sig(lib, "te_hip_attention_prefill_vt_workspace_bytes", [_sz] * 8, _sz)
    _sig(lib, "te_hip_attention_prefill_vt_f16",
         [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _sz, _vp])
    _sig(lib, "te_hip_attention_prefill_step_vt_f16",
         [_vp] * 11 + [_sz] * 8 + [_vp, _vp, _sz, _vp])
    _sig(lib, "te_hip_attention_prefill_workspace_bytes", [_sz] * 8, _sz)
    _sig(lib, "te_hip_attention_prefill_split_f16",
         [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _sz, _vp])
    _sig(lib, "te_hip_attention_prefill_step_f16",
         [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _vp])
    _sig(lib, "te_hip_attention_qk_mma_f32", [_f32p, _f32p, _sz, _sz, _sz, _f32p])
    _sig(lib, "te_hip_attention_tile_mma_f32", [_f32p, _f32p, _f32p, _sz, _sz, _sz, _f32p])
    _sig(lib, "te_hip_attention_stream_mma_f32", [_f32p, _f32p, _f32p, _sz, _sz, _sz, _f32p])
    _sig(lib, "te_hip_attention_causal_mma_f32", [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _f32p])
    _sig(lib, "te_hip_calibrate_mfma_f16", [_sz, _sz, _vp, _vp])
    _sig(lib, "te_hip_matvec_f32", [_vp, ctypes.c_uint32, _vp, _sz, _sz, _vp, _vp])
    _sig(lib, "te_hip_rmsnorm_f32", [_vp, _vp, _sz, _sz, ctypes.c_float, _vp, _vp])
    _sig(lib, "te_hip_swiglu_f32", [_vp, _vp, _sz, _vp, _vp])
    _sig(lib, "te_hip_add_f32", [_vp, _vp, _sz, _vp, _vp])
    _sig(lib, "te_hip_argmax_f32", [_vp, _sz, _vp, _vp])
    _sig(lib, "te_hip_sample_workspace_bytes", [_sz], _sz)
    _sig(lib, "te_hip_sample_top_k_f32", [_vp, _sz, ctypes.c_uint32, ctypes.c_float,
                                          ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint32), _vp,
                                          _sz, _vp])
    _u64p = ctypes.POINTER(ctypes.c_uint64)
    _sig(lib, "te_hip_gemm_act_bytes", [_sz, _sz], _sz)
    _sig(lib, "te_hip_gemm_q_f32", [_vp, ctypes.c_uint32, _vp, _vp, _vp, ctypes.c_float, _int, _sz, _sz, _sz, _vp,
                                    _vp, _vp, _vp, _sz, _vp])
    _sig(lib, "te_hip_prefill_all_layers_workspace_bytes", [_sz] * 4, _sz)
    _sig(lib, "te_hip_prefill_all_layers_f16",
         [_vp, _sz] + [_u64p] * 7 + [_sz, ctypes.c_uint32] + [_vp] * 11 + [_sz] * 9
         + [ctypes.c_float, _vp, _vp, _sz, _vp])
    _sig(lib, "te_hip_prefill_layer_f16",
         [_vp, _sz] + [ctypes.c_uint64] * 7 + [ctypes.c_uint32] + [_vp] * 11 + [_sz] * 9
         + [ctypes.c_float, _vp, _vp, _sz, _vp])
    _sig(lib, "te_hip_decode_layer_f16",
         [_vp, _sz] + [ctypes.c_uint64] * 7 + [ctypes.c_uint32] + [_vp] * 10 + [_sz] * 8
         + [ctypes.c_float, _vp, _vp, _sz, _vp])
    _sig(lib, "te_hip_decode_all_layers_workspace_bytes", [_sz] * 8, _sz)
    _sig(lib, "te_hip_decode_all_layers_f16",
         [_vp, _sz] + [_u64p] * 7 + [_sz, ctypes.c_uint32] + [_vp] * 10 + [_sz] * 8
         + [ctypes.c_float, _vp, ctypes.c_uint64, ctypes.c_uint32, _vp, _sz, _vp, _vp, _sz, _vp])


def strerror(status: int) -> str:
    return load_library().te_strerror(status).decode()


def check(status: int) -> None:
    """Reference runtime.py:381-384: raise TinyEngineError(te_strerror(status))."""
    if status != TE_STATUS_OK:
        raise TinyEngineError(strerror(status), status)


# ---- reference-binding style helpers -----------------------------------------

@dataclass(frozen=True)
class ArchInfo:
    kind: int
    name: str
    cpu_cores: int
    gpu_cores: int
    recommended_max_context: int


@dataclass(frozen=True)
class Capabilities:
    abi_version: int
    vector_op_mask: int
    optimization_flags: int
    preferred_alignment_bytes: int
    backend_name: str
    notes: str


def detect_arch() -> ArchInfo:
    lib = load_library()
    raw = _ArchInfo()
    check(lib.te_detect_arch(ctypes.byref(raw)))
    return ArchInfo(raw.kind, raw.name.decode(), raw.cpu_cores, raw.gpu_cores, raw.recommended_max_context)


def capabilities() -> Capabilities:
    lib = load_library()
    raw = _Capabilities()
    check(lib.te_get_capabilities(ctypes.byref(raw)))
    return Capabilities(raw.abi_version, raw.vector_op_mask, raw.optimization_flags,
                        raw.preferred_alignment_bytes, raw.backend_name.decode(), raw.notes.decode())


def hip_available() -> bool:
    return bool(load_library().te_hip_available())


def device_info() -> tuple[str, int]:
    lib = load_library()
    name = ctypes.create_string_buffer(128)
    cus = ctypes.c_uint32()
    check(lib.te_hip_device_info(name, 128, ctypes.byref(cus)))
    return name.value.decode(), cus.value


# ---- public attention-step functions (host numpy arrays) ----------------------

def _f32(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f32p)


def rope_f32(values: np.ndarray, heads: int, head_dim: int, position: int, theta: float) -> np.ndarray:
    """te_rope_f32 on the GPU; returns the rotated copy of `values`."""
    out = np.array(values, dtype=np.float32, copy=True, order="C")
    check(load_library().te_rope_f32(_f32(out), heads, head_dim, position, ctypes.c_float(theta)))
    return out


def attention_decode_f32(query: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray, position: int,
                         heads: int, kv_heads: int, head_dim: int) -> np.ndarray:
    """te_attention_decode_f32 on the GPU (fp32 cache [position+1][kv_heads][head_dim])."""
    q = np.ascontiguousarray(query, dtype=np.float32)
    k = np.ascontiguousarray(key_cache, dtype=np.float32)
    v = np.ascontiguousarray(value_cache, dtype=np.float32)
    out = np.zeros(heads * head_dim, dtype=np.float32)
    check(load_library().te_attention_decode_f32(_f32(q), _f32(k), _f32(v), position, heads, kv_heads, head_dim,
                                                 _f32(out)))
    return out


def rmsnorm_f32(x: np.ndarray, weight: np.ndarray, epsilon: float) -> np.ndarray:
    """Public te_rmsnorm_f32 (host arrays, runs on the GPU)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(weight, dtype=np.float32)
    out = np.empty_like(x)
    check(load_library().te_rmsnorm_f32(_f32(x), _f32(w), x.size, ctypes.c_float(epsilon), _f32(out)))
    return out


def swiglu_f32(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    out = np.empty_like(g)
    check(load_library().te_swiglu_f32(_f32(g), _f32(u), g.size, _f32(out)))
    return out


def add_f32(lhs: np.ndarray, rhs: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(lhs, dtype=np.float32)
    b = np.ascontiguousarray(rhs, dtype=np.float32)
    out = np.empty_like(a)
    check(load_library().te_add_f32(_f32(a), _f32(b), a.size, _f32(out)))
    return out


def argmax_f32(values: np.ndarray) -> int:
    v = np.ascontiguousarray(values, dtype=np.float32)
    idx = ctypes.c_uint32(0)
    check(load_library().te_argmax_f32(_f32(v), v.size, ctypes.byref(idx)))
    return int(idx.value)


def _mma(name: str, *args) -> None:
    check(getattr(load_library(), name)(*args))


def attention_qk_mma_f32(query, key_t, q_rows, k_cols, head_dim):
    out = np.zeros(q_rows * k_cols, dtype=np.float32)
    _mma("te_hip_attention_qk_mma_f32", _f32(np.ascontiguousarray(query, np.float32)),
         _f32(np.ascontiguousarray(key_t, np.float32)), q_rows, k_cols, head_dim, _f32(out))
    return out


def attention_tile_mma_f32(query, key_t, value, q_rows, k_cols, head_dim):
    out = np.zeros(q_rows * head_dim, dtype=np.float32)
    _mma("te_hip_attention_tile_mma_f32", _f32(np.ascontiguousarray(query, np.float32)),
         _f32(np.ascontiguousarray(key_t, np.float32)), _f32(np.ascontiguousarray(value, np.float32)),
         q_rows, k_cols, head_dim, _f32(out))
    return out


def attention_stream_mma_f32(query, key_t, value, q_rows, k_cols, head_dim):
    out = np.zeros(q_rows * head_dim, dtype=np.float32)
    _mma("te_hip_attention_stream_mma_f32", _f32(np.ascontiguousarray(query, np.float32)),
         _f32(np.ascontiguousarray(key_t, np.float32)), _f32(np.ascontiguousarray(value, np.float32)),
         q_rows, k_cols, head_dim, _f32(out))
    return out


def attention_causal_mma_f32(query, key_t, value, q_rows, k_cols, head_dim, q_base):
    out = np.zeros(q_rows * head_dim, dtype=np.float32)
    _mma("te_hip_attention_causal_mma_f32", _f32(np.ascontiguousarray(query, np.float32)),
         _f32(np.ascontiguousarray(key_t, np.float32)), _f32(np.ascontiguousarray(value, np.float32)),
         q_rows, k_cols, head_dim, q_base, _f32(out))
    return out

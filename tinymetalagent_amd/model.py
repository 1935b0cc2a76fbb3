"""GGUF models, the tokenizer and generation over libtinyengine.so: the
`Model` class and `format_qwen_chat_prompt` of the reference binding
(python/tinyengine/runtime.py:133-243 for the info types, :438-693 for the
calls), with the same struct layouts (tinyengine.h:100-198), retry-on-short-
buffer behaviour and errors (TinyEngineError(te_strerror(status))).

Loading, tensor info and the tokenizer are host code; dequantize_row, matvec
and generate run on the GPU and raise where none is present.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Callable, Optional

from .runtime import (TE_ABI_VERSION, TE_QUANT_COUNT, TE_STATUS_INVALID_ARGUMENT, TinyEngineError, _RuntimeOptions,
                      _TOKEN_CALLBACK, check, load_library)


class _ModelInfo(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("gguf_version", ctypes.c_uint32),
        ("metadata_kv_count", ctypes.c_uint64),
        ("tensor_count", ctypes.c_uint64),
        ("tensor_data_offset", ctypes.c_uint64),
        ("tensor_data_bytes", ctypes.c_uint64),
        ("parameter_count", ctypes.c_uint64),
        ("file_size_bytes", ctypes.c_uint64),
        ("name", ctypes.c_char * 128),
        ("architecture", ctypes.c_char * 32),
        ("context_length", ctypes.c_uint32),
        ("embedding_length", ctypes.c_uint32),
        ("block_count", ctypes.c_uint32),
        ("feed_forward_length", ctypes.c_uint32),
        ("attention_head_count", ctypes.c_uint32),
        ("attention_head_count_kv", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("vocab_size", ctypes.c_uint32),
        ("rms_norm_epsilon", ctypes.c_float),
        ("rope_freq_base", ctypes.c_float),
        ("quant_tensor_counts", ctypes.c_uint64 * TE_QUANT_COUNT),
        ("reserved", ctypes.c_uint32 * 16),
    ]


class _TensorInfo(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("quant", ctypes.c_int),
        ("ggml_type", ctypes.c_uint32),
        ("n_dims", ctypes.c_uint32),
        ("dims", ctypes.c_uint64 * 4),
        ("elements", ctypes.c_uint64),
        ("bytes", ctypes.c_uint64),
        ("relative_offset", ctypes.c_uint64),
        ("absolute_offset", ctypes.c_uint64),
        ("name", ctypes.c_char * 128),
        ("reserved", ctypes.c_uint32 * 16),
    ]


class _TokenizerInfo(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_uint32),
        ("model", ctypes.c_char * 32),
        ("pre", ctypes.c_char * 32),
        ("token_count", ctypes.c_uint64),
        ("token_type_count", ctypes.c_uint64),
        ("merge_count", ctypes.c_uint64),
        ("bos_token_id", ctypes.c_uint32),
        ("eos_token_id", ctypes.c_uint32),
        ("padding_token_id", ctypes.c_uint32),
        ("add_bos_token", ctypes.c_int),
        ("reserved", ctypes.c_uint32 * 16),
    ]


def _text(raw: bytes) -> str:
    return raw.split(b"\0", 1)[0].decode(errors="replace")


@dataclass(frozen=True)
class RuntimeOptions:
    target_arch: int = 0
    context_tokens: int = 512
    batch_tokens: int = 128
    memory_limit_bytes: int = 0
    kernel_cache_dir: Optional[str] = None
    flags: int = 0

    def _to_c(self) -> _RuntimeOptions:
        raw = _RuntimeOptions()
        raw.abi_version = TE_ABI_VERSION
        raw.target_arch = self.target_arch
        raw.context_tokens = self.context_tokens
        raw.batch_tokens = self.batch_tokens
        raw.memory_limit_bytes = self.memory_limit_bytes
        raw.kernel_cache_dir = self.kernel_cache_dir.encode() if self.kernel_cache_dir else None
        raw.flags = self.flags
        return raw


@dataclass(frozen=True)
class ModelInfo:
    gguf_version: int
    metadata_kv_count: int
    tensor_count: int
    tensor_data_offset: int
    tensor_data_bytes: int
    parameter_count: int
    file_size_bytes: int
    name: str
    architecture: str
    context_length: int
    embedding_length: int
    block_count: int
    feed_forward_length: int
    attention_head_count: int
    attention_head_count_kv: int
    head_dim: int
    vocab_size: int
    rms_norm_epsilon: float
    rope_freq_base: float
    quant_tensor_counts: tuple


@dataclass(frozen=True)
class TensorInfo:
    name: str
    quant: int
    ggml_type: int
    dims: tuple
    elements: int
    bytes: int
    relative_offset: int
    absolute_offset: int


@dataclass(frozen=True)
class TokenizerInfo:
    model: str
    pre: str
    token_count: int
    token_type_count: int
    merge_count: int
    bos_token_id: int
    eos_token_id: int
    padding_token_id: int
    add_bos_token: bool


def format_qwen_chat_prompt(prompt: str) -> str:
    lib = load_library()
    data = prompt.encode()
    capacity = len(data) + 64
    while True:
        out = ctypes.create_string_buffer(capacity)
        written = ctypes.c_size_t()
        status = lib.te_format_qwen_chat_prompt(data, out, capacity, ctypes.byref(written))
        if status == 0:
            return out.value.decode()
        if status == TE_STATUS_INVALID_ARGUMENT and written.value + 1 > capacity:
            capacity = written.value + 1
            continue
        check(status)


class Model:
    """A loaded GGUF file (te_model_load_gguf)."""

    def __init__(self, gguf_path, options: RuntimeOptions = RuntimeOptions()):
        self._lib = load_library()
        self._options = options
        raw = options._to_c()
        self._model = ctypes.c_void_p()
        check(self._lib.te_model_load_gguf(os.fsencode(gguf_path), ctypes.byref(raw), ctypes.byref(self._model)))

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._model

    def info(self) -> ModelInfo:
        r = _ModelInfo()
        check(self._lib.te_model_get_info(self._model, ctypes.byref(r)))
        return ModelInfo(r.gguf_version, r.metadata_kv_count, r.tensor_count, r.tensor_data_offset,
                         r.tensor_data_bytes, r.parameter_count, r.file_size_bytes, _text(r.name),
                         _text(r.architecture), r.context_length, r.embedding_length, r.block_count,
                         r.feed_forward_length, r.attention_head_count, r.attention_head_count_kv, r.head_dim,
                         r.vocab_size, float(r.rms_norm_epsilon), float(r.rope_freq_base),
                         tuple(r.quant_tensor_counts))

    def tensor_info(self, name: str) -> TensorInfo:
        r = _TensorInfo()
        check(self._lib.te_model_get_tensor_info(self._model, name.encode(), ctypes.byref(r)))
        return TensorInfo(_text(r.name), r.quant, r.ggml_type, tuple(r.dims[:r.n_dims]), r.elements, r.bytes,
                          r.relative_offset, r.absolute_offset)

    def tokenizer_info(self) -> TokenizerInfo:
        r = _TokenizerInfo()
        check(self._lib.te_model_get_tokenizer_info(self._model, ctypes.byref(r)))
        return TokenizerInfo(_text(r.model), _text(r.pre), r.token_count, r.token_type_count, r.merge_count,
                             r.bos_token_id, r.eos_token_id, r.padding_token_id, bool(r.add_bos_token))

    def tokenize(self, text, parse_special: bool = True) -> list[int]:
        data = text.encode() if isinstance(text, str) else bytes(text)
        capacity = max(len(data) + 16, 16)
        while True:
            out = (ctypes.c_uint32 * capacity)()
            written = ctypes.c_size_t()
            status = self._lib.te_model_tokenize(self._model, data, int(parse_special), out, capacity,
                                                 ctypes.byref(written))
            if status == 0:
                return list(out[:written.value])
            if status == TE_STATUS_INVALID_ARGUMENT and written.value > capacity:
                capacity = written.value
                continue
            check(status)

    def detokenize_bytes(self, tokens, skip_special: bool = True) -> bytes:
        ids = (ctypes.c_uint32 * max(len(tokens), 1))(*tokens)
        capacity = max(len(tokens) * 16 + 16, 16)
        while True:
            out = ctypes.create_string_buffer(capacity)
            written = ctypes.c_size_t()
            status = self._lib.te_model_detokenize(self._model, ids, len(tokens), int(skip_special), out, capacity,
                                                   ctypes.byref(written))
            if status == 0:
                return out.raw[:written.value]
            if status == TE_STATUS_INVALID_ARGUMENT and written.value + 1 > capacity:
                capacity = written.value + 1
                continue
            check(status)

    def detokenize(self, tokens, skip_special: bool = True) -> str:
        return self.detokenize_bytes(tokens, skip_special).decode()

    def read_f32_tensor(self, name: str) -> list[float]:
        info = self.tensor_info(name)
        values = (ctypes.c_float * max(info.elements, 1))()
        written = ctypes.c_size_t()
        check(self._lib.te_model_read_f32_tensor(self._model, name.encode(), values, info.elements,
                                                 ctypes.byref(written)))
        return list(values[:written.value])

    def dequantize_row(self, name: str, row_index: int) -> list[float]:
        info = self.tensor_info(name)
        if len(info.dims) != 2:
            raise TinyEngineError(f"{name} is not rank-2")
        cols = info.dims[0]
        values = (ctypes.c_float * cols)()
        written = ctypes.c_size_t()
        check(self._lib.te_model_dequantize_row_f32(self._model, name.encode(), row_index, values, cols,
                                                    ctypes.byref(written)))
        return list(values[:written.value])

    def matvec(self, name: str, input_values) -> list[float]:
        info = self.tensor_info(name)
        if len(info.dims) != 2:
            raise TinyEngineError(f"{name} is not rank-2")
        x = (ctypes.c_float * max(len(input_values), 1))(*input_values)
        rows = info.dims[1]
        out = (ctypes.c_float * rows)()
        written = ctypes.c_size_t()
        check(self._lib.te_model_matvec_f32(self._model, name.encode(), x, len(input_values), out, rows,
                                            ctypes.byref(written)))
        return list(out[:written.value])

    def generate(self, prompt: str, max_tokens: int = 16,
                 on_token: Optional[Callable[[str, int], None]] = None) -> str:
        return self._run_generate(self._lib.te_generate, prompt, max_tokens, on_token)

    def generate_raw(self, prompt: str, max_tokens: int = 256,
                     on_token: Optional[Callable[[str, int], None]] = None) -> str:
        """The prompt verbatim (special tokens parsed), no chat template."""
        return self._run_generate(self._lib.te_generate_raw, prompt, max_tokens, on_token)

    def _run_generate(self, fn, prompt: str, max_tokens: int, on_token) -> str:
        raw = self._options._to_c()
        context = ctypes.c_void_p()
        check(self._lib.te_context_create(self._model, ctypes.byref(raw), ctypes.byref(context)))
        chunks: list[str] = []

        def callback(text: bytes, token_id: int, _userdata) -> None:
            chunk = text.decode(errors="replace")
            chunks.append(chunk)
            if on_token is not None:
                on_token(chunk, token_id)

        c_callback = _TOKEN_CALLBACK(callback)
        try:
            check(fn(context, prompt.encode(), max_tokens, c_callback, None))
        finally:
            self._lib.te_context_free(context)
        return "".join(chunks)

    def session(self) -> "Session":
        """A context kept across calls: each call reuses the K / V of the
        leading tokens it shares with the previous call's sequence."""
        return Session(self)

    def close(self) -> None:
        if getattr(self, "_model", None):
            self._lib.te_model_free(self._model)
            self._model = None

    def __enter__(self) -> "Model":
        return self

    def __exit__(self, *_exc) -> None:
        self.close()

    def __del__(self) -> None:
        self.close()


class Session:
    """One te_context over a Model, kept open between generate calls (this
    build's addition: the reference binding makes a context per call)."""

    def __init__(self, model: Model):
        self._model = model
        self._lib = model._lib
        raw = model._options._to_c()
        self._ctx = ctypes.c_void_p()
        check(self._lib.te_context_create(model.handle, ctypes.byref(raw), ctypes.byref(self._ctx)))

    def _run(self, fn, prompt: str, max_tokens: int, on_token) -> str:
        chunks: list[str] = []

        def callback(text: bytes, token_id: int, _userdata) -> None:
            chunk = text.decode(errors="replace")
            chunks.append(chunk)
            if on_token is not None:
                on_token(chunk, token_id)

        c_callback = _TOKEN_CALLBACK(callback)
        check(fn(self._ctx, prompt.encode(), max_tokens, c_callback, None))
        return "".join(chunks)

    def generate(self, prompt: str, max_tokens: int = 16, on_token=None) -> str:
        return self._run(self._lib.te_generate, prompt, max_tokens, on_token)

    def generate_raw(self, prompt: str, max_tokens: int = 256, on_token=None) -> str:
        return self._run(self._lib.te_generate_raw, prompt, max_tokens, on_token)

    def close(self) -> None:
        if getattr(self, "_ctx", None):
            self._lib.te_context_free(self._ctx)
            self._ctx = None

    def __enter__(self) -> "Session":
        return self

    def __exit__(self, *_exc) -> None:
        self.close()

    def __del__(self) -> None:
        self.close()

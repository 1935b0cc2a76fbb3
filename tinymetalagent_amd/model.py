"""GGUF models, the tokenizer and generation over libtinyengine.so.

The public surface is the reference binding's (python/tinyengine/runtime.py:
133-243 for the info types, :438-693 for the calls): the same class and
method names and signatures, the same struct layouts (tinyengine.h:100-198),
and errors raised as TinyEngineError(te_strerror(status)).  Every call that
fills a caller buffer goes through one grow-and-retry helper (_sized_call),
and generation runs through a context object that owns the te_context and the
callback (_Context).

Loading, tensor info and the tokenizer are host code; dequantize_row, matvec
and generate run on the GPU and raise where none is present.
"""
from __future__ import annotations

import ctypes
import dataclasses
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


class _Handle:
    """Owner of one library handle: close() releases it once; usable as a
    context manager, and released at garbage collection."""

    _handle_attr = "_handle"

    def _release(self, handle) -> None:  # pragma: no cover - overridden
        raise NotImplementedError

    def close(self) -> None:
        handle = self.__dict__.get(self._handle_attr)
        if handle:
            self.__dict__[self._handle_attr] = None
            self._release(handle)

    def __enter__(self):
        return self

    def __exit__(self, *_exc) -> None:
        self.close()

    def __del__(self) -> None:
        self.close()


def _sized_call(call, alloc, capacity: int, slack: int):
    """Run call(buffer, capacity, written) into alloc(capacity).  The library
    reports a short buffer as INVALID_ARGUMENT with `written` set to the
    length the result needs; `slack` extra elements hold a terminator.  The
    buffer then grows to fit and the call runs again.  Returns (buffer,
    written)."""
    written = ctypes.c_size_t()
    while True:
        buffer = alloc(capacity)
        status = call(buffer, capacity, ctypes.byref(written))
        needed = written.value + slack
        if status == TE_STATUS_INVALID_ARGUMENT and needed > capacity:
            capacity = needed
            continue
        check(status)
        return buffer, written.value


def format_qwen_chat_prompt(prompt: str) -> str:
    lib = load_library()
    data = prompt.encode()
    buffer, n = _sized_call(lambda buf, cap, w: lib.te_format_qwen_chat_prompt(data, buf, cap, w),
                            ctypes.create_string_buffer, len(data) + 128, 1)
    return buffer.raw[:n].decode()


class _TextSink:
    """Collects the text te_generate* hands to its callback and forwards each
    piece to an optional Python callable; owns the ctypes callback object for
    the duration of one call."""

    def __init__(self, on_token: Optional[Callable[[str, int], None]]):
        self.pieces: list[str] = []
        self._on_token = on_token
        self.c_callback = _TOKEN_CALLBACK(self._receive)

    def _receive(self, text: bytes, token_id: int, _userdata) -> None:
        piece = (text or b"").decode("utf-8", "replace")
        self.pieces.append(piece)
        if self._on_token is not None:
            self._on_token(piece, token_id)

    def text(self) -> str:
        return "".join(self.pieces)


class _Context(_Handle):
    """One te_context: generation state (the KV cache in HBM) of a model."""

    def __init__(self, model: "Model"):
        self._lib = model._lib
        handle = ctypes.c_void_p()
        options = model._options._to_c()
        check(self._lib.te_context_create(model.handle, ctypes.byref(options), ctypes.byref(handle)))
        self._handle = handle

    def _release(self, handle) -> None:
        self._lib.te_context_free(handle)

    def run(self, raw: bool, prompt: str, max_tokens: int, on_token) -> str:
        fn = self._lib.te_generate_raw if raw else self._lib.te_generate
        sink = _TextSink(on_token)
        check(fn(self._handle, prompt.encode(), max_tokens, sink.c_callback, None))
        return sink.text()


class Model(_Handle):
    """A loaded GGUF file (te_model_load_gguf)."""

    _handle_attr = "_model"

    def __init__(self, gguf_path, options: RuntimeOptions = RuntimeOptions()):
        self._lib = load_library()
        self._options = options
        self._model = None
        handle = ctypes.c_void_p()
        raw = options._to_c()
        check(self._lib.te_model_load_gguf(os.fsencode(gguf_path), ctypes.byref(raw), ctypes.byref(handle)))
        self._model = handle

    def _release(self, handle) -> None:
        self._lib.te_model_free(handle)

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._model

    def _query(self, fn, struct_type, *args):
        out = struct_type()
        check(fn(self._model, *args, ctypes.byref(out)))
        return out

    def info(self) -> ModelInfo:
        r = self._query(self._lib.te_model_get_info, _ModelInfo)
        fields = {f.name: getattr(r, f.name) for f in dataclasses.fields(ModelInfo)}
        fields.update(name=_text(r.name), architecture=_text(r.architecture),
                      rms_norm_epsilon=float(r.rms_norm_epsilon), rope_freq_base=float(r.rope_freq_base),
                      quant_tensor_counts=tuple(r.quant_tensor_counts))
        return ModelInfo(**fields)

    def tensor_info(self, name: str) -> TensorInfo:
        r = self._query(self._lib.te_model_get_tensor_info, _TensorInfo, name.encode())
        fields = {f.name: getattr(r, f.name) for f in dataclasses.fields(TensorInfo) if f.name not in ("name", "dims")}
        return TensorInfo(name=_text(r.name), dims=tuple(r.dims[:r.n_dims]), **fields)

    def tokenizer_info(self) -> TokenizerInfo:
        r = self._query(self._lib.te_model_get_tokenizer_info, _TokenizerInfo)
        fields = {f.name: getattr(r, f.name) for f in dataclasses.fields(TokenizerInfo)}
        fields.update(model=_text(r.model), pre=_text(r.pre), add_bos_token=bool(r.add_bos_token))
        return TokenizerInfo(**fields)

    def tokenize(self, text, parse_special: bool = True) -> list[int]:
        data = text.encode() if isinstance(text, str) else bytes(text)
        # byte-level BPE: at most one token per byte, plus a BOS token
        buffer, n = _sized_call(
            lambda buf, cap, w: self._lib.te_model_tokenize(self._model, data, int(parse_special), buf, cap, w),
            lambda cap: (ctypes.c_uint32 * cap)(), len(data) + 2, 0)
        return list(buffer[:n])

    def detokenize_bytes(self, tokens, skip_special: bool = True) -> bytes:
        ids = list(tokens)
        arr = (ctypes.c_uint32 * max(len(ids), 1))(*ids)
        buffer, n = _sized_call(
            lambda buf, cap, w: self._lib.te_model_detokenize(self._model, arr, len(ids), int(skip_special), buf,
                                                              cap, w),
            ctypes.create_string_buffer, 8 * len(ids) + 64, 1)
        return buffer.raw[:n]

    def detokenize(self, tokens, skip_special: bool = True) -> str:
        return self.detokenize_bytes(tokens, skip_special).decode()

    def read_f32_tensor(self, name: str) -> list[float]:
        count = self.tensor_info(name).elements
        buffer, n = _sized_call(
            lambda buf, cap, w: self._lib.te_model_read_f32_tensor(self._model, name.encode(), buf, cap, w),
            lambda cap: (ctypes.c_float * max(cap, 1))(), count, 0)
        return list(buffer[:n])

    def _matrix_dims(self, name: str) -> tuple[int, int]:
        dims = self.tensor_info(name).dims
        if len(dims) != 2:
            raise TinyEngineError(f"tensor {name!r} has {len(dims)} dimensions; this call takes a matrix")
        return dims[0], dims[1]

    def dequantize_row(self, name: str, row_index: int) -> list[float]:
        cols, _rows = self._matrix_dims(name)
        buffer, n = _sized_call(
            lambda buf, cap, w: self._lib.te_model_dequantize_row_f32(self._model, name.encode(), row_index, buf,
                                                                      cap, w),
            lambda cap: (ctypes.c_float * max(cap, 1))(), cols, 0)
        return list(buffer[:n])

    def matvec(self, name: str, input_values) -> list[float]:
        _cols, rows = self._matrix_dims(name)
        values = list(input_values)
        x = (ctypes.c_float * max(len(values), 1))(*values)
        buffer, n = _sized_call(
            lambda buf, cap, w: self._lib.te_model_matvec_f32(self._model, name.encode(), x, len(values), buf,
                                                              cap, w),
            lambda cap: (ctypes.c_float * max(cap, 1))(), rows, 0)
        return list(buffer[:n])

    def generate(self, prompt: str, max_tokens: int = 16,
                 on_token: Optional[Callable[[str, int], None]] = None) -> str:
        """Chat-templated generation in a fresh context."""
        with _Context(self) as ctx:
            return ctx.run(False, prompt, max_tokens, on_token)

    def generate_raw(self, prompt: str, max_tokens: int = 256,
                     on_token: Optional[Callable[[str, int], None]] = None) -> str:
        """The prompt verbatim (special tokens parsed), no chat template."""
        with _Context(self) as ctx:
            return ctx.run(True, prompt, max_tokens, on_token)

    def session(self) -> "Session":
        """A context kept across calls: each call reuses the K / V of the
        leading tokens it shares with the previous call's sequence."""
        return Session(self)


class Session(_Handle):
    """One te_context over a Model, kept open between generate calls (this
    build's addition: the reference binding makes a context per call)."""

    _handle_attr = "_context"

    def __init__(self, model: Model):
        self._model = model
        self._context = _Context(model)

    def _release(self, context: _Context) -> None:
        context.close()

    def generate(self, prompt: str, max_tokens: int = 16, on_token=None) -> str:
        return self._context.run(False, prompt, max_tokens, on_token)

    def generate_raw(self, prompt: str, max_tokens: int = 256, on_token=None) -> str:
        return self._context.run(True, prompt, max_tokens, on_token)

"""Python host mirror of the OrionServe-RS hot-path interface over liborion_hip.so.

The reference binds a device through Rust traits (crates/orion-core/src/traits.rs):
``Backend`` (:159-183), ``ForwardBatch`` (:193-261), ``ForwardOutput`` (:271-290) and
``LanguageModel`` (:297-309).  This module restates those types in Python on top of
the C ABI declared in include/orion_hip.h, so tests and benchmarks read like the
reference's own.  It loads the in-tree HIP library and fails loudly when it is
missing: there is no CPU fallback here.
"""
from __future__ import annotations

import array
import ctypes as C
import os
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborion_hip.so")

OK = 0
ERR_INTERNAL = 1
ERR_BACKEND = 2

# DType, traits.rs:21-29
F32, F16, BF16, I8, I4 = 0, 1, 2, 3, 4

# Weight ids (include/orion_hip.h)
W_EMBED, W_FINAL_NORM, W_LM_HEAD = 0, 1, 2
W_INPUT_NORM, W_Q, W_K, W_V, W_O = 3, 4, 5, 6, 7
W_Q_BIAS, W_K_BIAS, W_V_BIAS, W_POST_NORM = 8, 9, 10, 11
W_GATE, W_UP, W_DOWN = 12, 13, 14

# Every symbol include/orion_hip.h declares.
EXPORTED = [
    "orion_hip_last_error", "orion_hip_last_error_stage", "orion_hip_device_count",
    "orion_hip_device_open", "orion_hip_device_close", "orion_hip_device_name",
    "orion_hip_mem_info", "orion_hip_synchronize", "orion_hip_supports_dtype",
    "orion_hip_alloc", "orion_hip_free", "orion_hip_memcpy_h2d", "orion_hip_memcpy_d2h",
    "orion_hip_memcpy_d2d", "orion_hip_memset", "orion_hip_timer_start", "orion_hip_timer_stop",
    "orion_hip_kernel_timing", "orion_hip_kernel_timing_read",
    "orion_hip_kernel_timing_samples",
    "orion_hip_model_create", "orion_hip_model_destroy", "orion_hip_model_upload_weight",
    "orion_hip_model_init_synthetic", "orion_hip_synthetic_value",
    "orion_hip_checkpoint_open", "orion_hip_checkpoint_close", "orion_hip_checkpoint_num_tensors",
    "orion_hip_checkpoint_tensor_info", "orion_hip_checkpoint_read_f32",
    "orion_hip_model_load_checkpoint", "orion_hip_sample", "orion_hip_model_sample",
    "orion_hip_model_download_weight", "orion_hip_model_forward", "orion_hip_model_kv_read",
    "orion_hip_model_kv_write", "orion_hip_model_kv_arena", "orion_hip_model_kv_layout", "orion_hip_decode_plan_create",
    "orion_hip_decode_plan_destroy", "orion_hip_decode_plan_info",
    "orion_hip_decode_plan_packed", "orion_hip_paged_attention_decode",
    "orion_hip_paged_attention_prefill", "orion_hip_rope_and_cache", "orion_hip_rmsnorm",
    "orion_hip_gemm", "orion_hip_gemm_noalloc", "orion_hip_silu_mul", "orion_hip_argmax",
]


class EngineError(Exception):
    """Mirror of orion_core::EngineError (crates/orion-core/src/error.rs)."""


class InternalError(EngineError):
    """EngineError::Internal: an invariant or index violation (error.rs:125-130)."""


class BackendError(EngineError):
    """EngineError::Backend {backend: "hip", stage, reason} (error.rs:118-124)."""

    def __init__(self, stage: str, reason: str):
        super().__init__(f"backend `hip` failed during {stage}: {reason}")
        self.stage = stage
        self.reason = reason


class SamplingParams(C.Structure):
    """orion_core::SamplingParams (orion-core/src/sampling.rs:22-70), the fields
    the sampler reads; defaults as SamplingParams::default (:55-70)."""

    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float),
                ("repetition_penalty", C.c_float)]

    def __init__(self, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0):
        super().__init__(temperature, top_k, top_p, repetition_penalty)


class ModelDesc(C.Structure):
    _fields_ = [
        ("num_layers", C.c_int32), ("hidden_size", C.c_int32),
        ("num_attention_heads", C.c_int32), ("num_kv_heads", C.c_int32),
        ("head_dim", C.c_int32), ("intermediate_size", C.c_int32),
        ("vocab_size", C.c_int32), ("max_position_embeddings", C.c_int32),
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float),
        ("has_qkv_bias", C.c_int32), ("tied_lm_head", C.c_int32),
        ("num_blocks", C.c_int32), ("block_size", C.c_int32), ("kv_dtype", C.c_int32),
    ]


class BatchDesc(C.Structure):
    _fields_ = [
        ("num_tokens", C.c_int64), ("num_seqs", C.c_int64),
        ("tokens", C.c_void_p), ("positions", C.c_void_p),
        ("slot_token_counts", C.c_void_p), ("context_lens", C.c_void_p),
        ("block_table_offsets", C.c_void_p), ("block_table_ids", C.c_void_p),
        ("has_prefill", C.c_int32),
    ]


class KvLayout(C.Structure):
    _fields_ = [
        ("num_layers", C.c_int64), ("num_blocks", C.c_int64), ("block_size", C.c_int64),
        ("num_kv_heads", C.c_int64), ("head_dim", C.c_int64), ("dtype", C.c_int32),
        ("head_major", C.c_int32),
    ]


_lib = None


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Loads liborion_hip.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python orionserve-rs_amd/build.py` "
            "(or __graft_entry__.build()). There is no CPU fallback.")
    lib = C.CDLL(path)
    vp, i32, i64, u32, u64, f32, sz = (C.c_void_p, C.c_int32, C.c_int64, C.c_uint32,
                                       C.c_uint64, C.c_float, C.c_size_t)
    P = C.POINTER
    sig = {
        "orion_hip_last_error": ([], C.c_char_p),
        "orion_hip_last_error_stage": ([], C.c_char_p),
        "orion_hip_device_count": ([P(C.c_int)], C.c_int),
        "orion_hip_device_open": ([C.c_int, P(vp)], C.c_int),
        "orion_hip_device_close": ([vp], None),
        "orion_hip_device_name": ([vp, C.c_char_p, sz], C.c_int),
        "orion_hip_mem_info": ([vp, P(u64), P(u64)], C.c_int),
        "orion_hip_synchronize": ([vp], C.c_int),
        "orion_hip_supports_dtype": ([vp, C.c_int], C.c_int),
        "orion_hip_alloc": ([vp, sz, P(vp)], C.c_int),
        "orion_hip_free": ([vp, vp], C.c_int),
        "orion_hip_memcpy_h2d": ([vp, vp, vp, sz], C.c_int),
        "orion_hip_memcpy_d2h": ([vp, vp, vp, sz], C.c_int),
        "orion_hip_memcpy_d2d": ([vp, vp, vp, sz], C.c_int),
        "orion_hip_memset": ([vp, vp, C.c_int, sz], C.c_int),
        "orion_hip_timer_start": ([vp], C.c_int),
        "orion_hip_timer_stop": ([vp, P(f32)], C.c_int),
        "orion_hip_kernel_timing": ([vp, C.c_int], C.c_int),
        "orion_hip_kernel_timing_read": ([vp, C.c_int, P(C.c_double), P(i64)], C.c_int),
        "orion_hip_kernel_timing_samples": ([vp, C.c_int, vp, i64, P(i64)], C.c_int),
        "orion_hip_model_create": ([vp, P(ModelDesc), P(vp)], C.c_int),
        "orion_hip_model_destroy": ([vp], None),
        "orion_hip_model_upload_weight": ([vp, C.c_int, C.c_int, vp, C.c_int, sz], C.c_int),
        "orion_hip_model_init_synthetic": ([vp, u64, f32], C.c_int),
        "orion_hip_synthetic_value": ([u64, C.c_int, C.c_int, u64, f32], f32),
        "orion_hip_checkpoint_open": ([C.c_char_p, P(vp)], C.c_int),
        "orion_hip_checkpoint_close": ([vp], None),
        "orion_hip_checkpoint_num_tensors": ([vp, P(i64)], C.c_int),
        "orion_hip_checkpoint_tensor_info": ([vp, i64, C.c_char_p, sz, P(i32), P(i32), P(i64)],
                                             C.c_int),
        "orion_hip_checkpoint_read_f32": ([vp, C.c_char_p, vp, sz], C.c_int),
        "orion_hip_model_load_checkpoint": ([vp, vp], C.c_int),
        "orion_hip_sample": ([vp, vp, i64, i64, P(SamplingParams), vp, vp, vp, vp], C.c_int),
        "orion_hip_model_sample": ([vp, P(SamplingParams), vp, vp, vp, vp], C.c_int),
        "orion_hip_model_download_weight": ([vp, C.c_int, C.c_int, vp, sz], C.c_int),
        "orion_hip_model_forward": ([vp, P(BatchDesc), vp, vp], C.c_int),
        "orion_hip_model_kv_read": ([vp, i64, u32, i64, i64, C.c_int, vp], C.c_int),
        "orion_hip_model_kv_write": ([vp, i64, u32, i64, i64, C.c_int, vp, i64], C.c_int),
        "orion_hip_model_kv_arena": ([vp, P(vp), P(sz)], C.c_int),
        "orion_hip_model_kv_layout": ([vp, P(KvLayout)], C.c_int),
        "orion_hip_decode_plan_create": ([vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, P(vp)],
                                         C.c_int),
        "orion_hip_decode_plan_destroy": ([vp], None),
        "orion_hip_decode_plan_info": ([vp, P(i64), P(i64), P(i64)], C.c_int),
        "orion_hip_decode_plan_packed": ([vp, P(i64), P(i64)], C.c_int),
        "orion_hip_paged_attention_decode": (
            [vp, P(KvLayout), vp, i64, vp, i64, i64, vp, vp, vp, vp, vp, vp], C.c_int),
        "orion_hip_paged_attention_prefill": (
            [vp, P(KvLayout), vp, i64, vp, i64, i64, vp, vp, vp, vp, vp, i64, i64, C.c_int32, vp],
            C.c_int),
        "orion_hip_rope_and_cache": (
            [vp, P(KvLayout), vp, i64, i64, i64, vp, i64, vp, vp, i64, vp, i64, vp, vp, vp, vp,
             vp, vp], C.c_int),
        "orion_hip_rmsnorm": ([vp, vp, vp, i64, i64, f32, vp], C.c_int),
        "orion_hip_gemm": ([vp, vp, vp, vp, i64, i64, i64, C.c_int, vp], C.c_int),
        "orion_hip_gemm_noalloc": ([vp, vp, vp, vp, i64, i64, i64, C.c_int, vp], C.c_int),
        "orion_hip_silu_mul": ([vp, vp, vp, i64], C.c_int),
        "orion_hip_argmax": ([vp, vp, i64, i64, vp], C.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def _check(rc: int) -> None:
    if rc == OK:
        return
    lib = load_library()
    msg = (lib.orion_hip_last_error() or b"").decode()
    stage = (lib.orion_hip_last_error_stage() or b"").decode()
    if rc == ERR_INTERNAL:
        raise InternalError(msg)
    raise BackendError(stage, msg)


def _ptr(a: Optional[np.ndarray]) -> Optional[int]:
    return None if a is None else a.ctypes.data


def device_count() -> int:
    lib = load_library()
    n = C.c_int(0)
    _check(lib.orion_hip_device_count(C.byref(n)))
    return n.value


class DeviceBuffer:
    """A device allocation owned by a HipBackend."""

    def __init__(self, backend: "HipBackend", nbytes: int):
        self.backend = backend
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _check(backend.lib.orion_hip_alloc(backend.handle, max(self.nbytes, 1), C.byref(p)))
        self.ptr = p.value

    def upload(self, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        _check(self.backend.lib.orion_hip_memcpy_h2d(self.backend.handle, self.ptr,
                                                     arr.ctypes.data, arr.nbytes))
        return self

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        _check(self.backend.lib.orion_hip_memcpy_d2h(self.backend.handle, out.ctypes.data,
                                                     self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            _check(self.backend.lib.orion_hip_free(self.backend.handle, self.ptr))
            self.ptr = None


class HipBackend:
    """`Backend` (traits.rs:159-183) for one MI355X; mirrors CpuBackend
    (crates/orion-models/src/backend.rs:11-55) and the planned CudaBackend
    (crates/orion-cuda/src/lib.rs:104-179)."""

    def __init__(self, ordinal: int = 0):
        self.lib = load_library()
        h = C.c_void_p()
        _check(self.lib.orion_hip_device_open(ordinal, C.byref(h)))
        self.handle = h.value
        self.ordinal = ordinal
        self._bufs: List[DeviceBuffer] = []

    # --- Backend ---
    def name(self) -> str:
        return "hip"

    def device(self) -> str:
        return f"cuda:{self.ordinal}"  # Device::Cuda(ordinal), traits.rs:61-65

    def device_name(self) -> str:
        buf = C.create_string_buffer(256)
        _check(self.lib.orion_hip_device_name(self.handle, buf, 256))
        return buf.value.decode()

    def _mem(self):
        t, f = C.c_uint64(), C.c_uint64()
        _check(self.lib.orion_hip_mem_info(self.handle, C.byref(t), C.byref(f)))
        return t.value, f.value

    def total_memory(self) -> int:
        return self._mem()[0]

    def available_memory(self) -> int:
        return self._mem()[1]

    def synchronize(self) -> None:
        _check(self.lib.orion_hip_synchronize(self.handle))

    def supports_dtype(self, dtype: int) -> bool:
        return bool(self.lib.orion_hip_supports_dtype(self.handle, dtype))

    # --- buffers / timing ---
    def alloc(self, nbytes: int) -> DeviceBuffer:
        b = DeviceBuffer(self, nbytes)
        self._bufs.append(b)
        return b

    def to_device(self, arr: np.ndarray) -> DeviceBuffer:
        arr = np.ascontiguousarray(arr)
        return self.alloc(arr.nbytes).upload(arr)

    def memcpy_d2d(self, dst: int, src: int, nbytes: int) -> None:
        _check(self.lib.orion_hip_memcpy_d2d(self.handle, dst, src, nbytes))

    def timer_start(self) -> None:
        _check(self.lib.orion_hip_timer_start(self.handle))

    def timer_stop(self) -> float:
        ms = C.c_float()
        _check(self.lib.orion_hip_timer_stop(self.handle, C.byref(ms)))
        return ms.value

    # Kernel indices for kernel_timing_read.
    K_DECODE_SPLIT, K_DECODE_MERGE, K_PREFILL, K_GEMM = 0, 1, 2, 3

    def kernel_timing(self, enable: bool) -> None:
        """Start (and reset) or stop per-kernel event timing of the attention ops."""
        _check(self.lib.orion_hip_kernel_timing(self.handle, 1 if enable else 0))

    def kernel_timing_read(self, kernel: int):
        """(total milliseconds, launches) recorded for `kernel` since enabling."""
        ms, n = C.c_double(), C.c_int64()
        _check(self.lib.orion_hip_kernel_timing_read(self.handle, kernel, C.byref(ms),
                                                     C.byref(n)))
        return ms.value, n.value

    def kernel_timing_samples(self, kernel: int) -> np.ndarray:
        """Per-launch milliseconds recorded for `kernel` since enabling, in launch order."""
        n = C.c_int64()
        _check(self.lib.orion_hip_kernel_timing_samples(self.handle, kernel, None, 0,
                                                        C.byref(n)))
        out = np.zeros(n.value, np.float32)
        _check(self.lib.orion_hip_kernel_timing_samples(self.handle, kernel, _ptr(out), n.value,
                                                        C.byref(n)))
        return out

    def close(self) -> None:
        if self.handle:
            for b in self._bufs:
                b.free()
            self._bufs.clear()
            self.lib.orion_hip_device_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


# ---------------------------------------------------------------------------
# Batch / output types (traits.rs:193-290)
# ---------------------------------------------------------------------------


@dataclass
class ForwardBatch:
    """Ragged batch (traits.rs:193-210)."""

    tokens: List[int]
    positions: List[int]
    sequence_ids: List[int]
    slot_token_counts: List[int]
    context_lens: List[int]
    block_tables: List[List[int]]
    has_prefill: bool = False

    def num_sequences(self) -> int:
        return len(self.sequence_ids)

    def num_tokens(self) -> int:
        return len(self.tokens)

    def is_empty(self) -> bool:
        return len(self.tokens) == 0

    def validate(self) -> None:
        """traits.rs:232-261."""
        n = len(self.sequence_ids)
        if (len(self.slot_token_counts) != n or len(self.context_lens) != n
                or len(self.block_tables) != n):
            raise InternalError(
                f"ForwardBatch arrays disagree: {n} sequence ids, "
                f"{len(self.slot_token_counts)} token counts, {len(self.context_lens)} "
                f"context lens, {len(self.block_tables)} block tables")
        if len(self.positions) != len(self.tokens):
            raise InternalError(f"ForwardBatch has {len(self.tokens)} tokens but "
                                f"{len(self.positions)} positions")
        s = sum(self.slot_token_counts)
        if s != len(self.tokens):
            raise InternalError(f"ForwardBatch slot token counts sum to {s} but there are "
                                f"{len(self.tokens)} tokens")

    def prepare(self) -> "ForwardBatch":
        """Validates and flattens the batch once, for a caller that runs the
        same batch repeatedly: forward() then reuses the arrays instead of
        rebuilding them from the Python lists (about a millisecond for 34 k
        block-table entries).  A caller that edits the lists afterwards calls
        prepare() again.  The library validates the flattened batch on every
        forward either way."""
        self.validate()
        self._prepared = self.to_csr()
        return self

    def advance_decode(self, next_tokens: Sequence[int]) -> "ForwardBatch":
        """The next step of a prepared decode batch (one row per sequence, no
        prefill): sequence i's token becomes next_tokens[i], and its position
        and context length advance by one, in the lists and in the prepared
        arrays alike (no re-flattening of the block tables).  The tables are
        kept as they are; each must already hold a block for the new position,
        which the library checks on forward as for any batch."""
        prepared = getattr(self, "_prepared", None)
        if prepared is None or self.has_prefill or any(c != 1 for c in self.slot_token_counts):
            raise InternalError("advance_decode needs a prepared decode batch "
                                "(one row per sequence)")
        if len(next_tokens) != len(self.tokens):
            raise InternalError(f"advance_decode got {len(next_tokens)} tokens for "
                                f"{len(self.tokens)} sequences")
        tokens, positions, _, ctx, _, _ = prepared
        tokens[:] = array.array("I", next_tokens)  # (raises on out-of-range ids)
        positions += 1
        ctx += 1
        self.tokens = list(next_tokens)
        self.positions = [p + 1 for p in self.positions]
        self.context_lens = [c + 1 for c in self.context_lens]
        return self

    def to_csr(self):
        """Flattened arrays in the layout of orion_hip_batch.  Built with
        array.array (straight from Python ints; an out-of-range value raises
        OverflowError as numpy's conversion does), which keeps the per-step
        host cost of a 32-sequence decode batch in the tens of microseconds."""
        def arr(code, values):
            return np.frombuffer(array.array(code, values), dtype=np.dtype(code))
        tokens = arr("I", self.tokens)
        positions = arr("I", self.positions)
        counts = arr("q", self.slot_token_counts)
        ctx = arr("q", self.context_lens)
        flat = array.array("I")
        offs = array.array("q", [0])
        for t in self.block_tables:
            flat.extend(t)
            offs.append(len(flat))
        ids = np.frombuffer(flat, dtype=np.uint32) if len(flat) else np.zeros(1, dtype=np.uint32)
        return tokens, positions, counts, ctx, np.frombuffer(offs, dtype=np.int64), ids


@dataclass
class ForwardOutput:
    """Last-row logits per sequence (traits.rs:271-290)."""

    logits: np.ndarray  # [num_sequences, vocab] f32
    vocab_size: int
    sequence_ids: List[int]
    argmax: Optional[np.ndarray] = None

    def row(self, i: int) -> Optional[np.ndarray]:
        if i < 0 or i >= self.logits.shape[0]:
            return None
        return self.logits[i]

    def num_sequences(self) -> int:
        return len(self.sequence_ids)


@dataclass
class ModelMetadata:
    """traits.rs:95-123 (the fields the hot path uses)."""

    hidden_size: int
    num_layers: int
    num_attention_heads: int
    num_kv_heads: int
    head_dim: int
    vocab_size: int
    intermediate_size: int
    max_position_embeddings: int = 2048
    rope_theta: float = 10000.0
    rms_norm_eps: float = 1e-5
    architecture: str = "llama"
    name: str = "model"
    tied_lm_head: bool = False

    def has_qkv_bias(self) -> bool:  # config.rs:134-139
        return self.architecture == "qwen2"


def _model_error(e: InternalError):
    """The reference's ModelError variant for a checkpoint failure, from the
    kind the library's message starts with."""
    import hf_config as hc

    msg = str(e)
    for prefix, cls in (("path not found", hc.PathNotFound), ("missing file", hc.MissingFile),
                        ("malformed", hc.Malformed), ("tensor not found", hc.TensorNotFound),
                        ("shape mismatch", hc.ShapeMismatch),
                        ("unsupported dtype", hc.UnsupportedDtype)):
        if msg.startswith(prefix):
            return cls(msg)
    return e


class Checkpoint:
    """CheckpointLoader (crates/orion-models/src/loader.rs:102-236) over the
    library's memory-mapped safetensors reader; host-side, needs no GPU."""

    def __init__(self, directory: str):
        lib = load_library()
        h = C.c_void_p()
        try:
            _check(lib.orion_hip_checkpoint_open(os.fsencode(directory), C.byref(h)))
        except InternalError as e:
            raise _model_error(e) from None
        self.handle = h.value
        self._lib = lib

    def __len__(self) -> int:
        n = C.c_int64()
        _check(self._lib.orion_hip_checkpoint_num_tensors(self.handle, C.byref(n)))
        return n.value

    def info(self, index: int):
        """(name, dtype code or -1, shape) of tensor `index` in name order."""
        buf = C.create_string_buffer(1024)
        dt, nd = C.c_int32(), C.c_int32()
        shape = (C.c_int64 * 8)()
        _check(self._lib.orion_hip_checkpoint_tensor_info(self.handle, index, buf, 1024,
                                                          C.byref(dt), C.byref(nd), shape))
        return buf.value.decode(), dt.value, [shape[i] for i in range(nd.value)]

    def names(self) -> List[str]:
        return [self.info(i)[0] for i in range(len(self))]

    def contains(self, name: str) -> bool:
        return name in self.names()

    def tensor(self, name: str):
        """(f32 values, shape), CheckpointLoader::tensor (loader.rs:188-202)."""
        for i in range(len(self)):
            n, dt, shape = self.info(i)
            if n == name:
                out = np.empty(int(np.prod(shape, dtype=np.int64)), dtype=np.float32)
                try:
                    _check(self._lib.orion_hip_checkpoint_read_f32(
                        self.handle, name.encode(), out.ctypes.data, out.size))
                except InternalError as e:
                    raise _model_error(e) from None
                return out, shape
        import hf_config as hc
        raise hc.TensorNotFound(f"tensor not found: {name}")

    def close(self) -> None:
        if self.handle:
            self._lib.orion_hip_checkpoint_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class HipTransformerModel:
    """`LanguageModel` (traits.rs:297-309) over the reference's TransformerModel
    (transformer.rs:137-443), executing on one MI355X."""

    def __init__(self, meta: ModelMetadata, num_blocks: int, block_size: int,
                 backend: HipBackend, kv_dtype: int = BF16):
        self.meta = meta
        self._backend = backend
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.kv_dtype = kv_dtype
        d = ModelDesc(meta.num_layers, meta.hidden_size, meta.num_attention_heads,
                      meta.num_kv_heads, meta.head_dim, meta.intermediate_size, meta.vocab_size,
                      meta.max_position_embeddings, meta.rms_norm_eps, meta.rope_theta,
                      int(meta.has_qkv_bias()), int(meta.tied_lm_head), num_blocks, block_size,
                      kv_dtype)
        h = C.c_void_p()
        _check(backend.lib.orion_hip_model_create(backend.handle, C.byref(d), C.byref(h)))
        self.handle = h.value

    @classmethod
    def from_directory(cls, directory: str, num_blocks: int, block_size: int,
                       backend: HipBackend, kv_dtype: int = BF16) -> "HipTransformerModel":
        """TransformerModel::from_directory (transformer.rs:180-204): config.json
        through HfConfig, then every weight straight from the safetensors
        mapping to the device in the file's dtype."""
        import hf_config as hc

        cfg = hc.HfConfig.load(directory)
        name = os.path.basename(os.path.normpath(directory)) or "model"
        meta = cfg.to_metadata(name)
        with Checkpoint(directory) as ck:
            model = cls(meta, num_blocks, block_size, backend, kv_dtype)
            try:
                model.load_checkpoint(ck)
            except BaseException:
                model.close()
                raise
        return model

    def load_checkpoint(self, ck: Checkpoint) -> None:
        """ModelWeights::load (transformer.rs:62-120) from an open checkpoint."""
        try:
            _check(self._backend.lib.orion_hip_model_load_checkpoint(self.handle, ck.handle))
        except InternalError as e:
            raise _model_error(e) from None

    def metadata(self) -> ModelMetadata:
        return self.meta

    def backend(self) -> HipBackend:
        return self._backend

    def upload_weight(self, which: int, layer: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data)
        if data.dtype == np.float32:
            dt = F32
        elif data.dtype == np.uint16:
            dt = BF16  # raw bf16 bits
        elif data.dtype == np.float16:
            dt = F16
        else:
            raise TypeError(f"unsupported weight dtype {data.dtype}")
        _check(self._backend.lib.orion_hip_model_upload_weight(
            self.handle, which, layer, data.ctypes.data, dt, data.size))

    def download_weight(self, which: int, layer: int, count: int) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        _check(self._backend.lib.orion_hip_model_download_weight(
            self.handle, which, layer, out.ctypes.data, count))
        return out

    def init_synthetic(self, seed: int, std: float = 0.02) -> None:
        _check(self._backend.lib.orion_hip_model_init_synthetic(self.handle, seed, std))

    def forward(self, batch: ForwardBatch, want_logits: bool = True,
                want_argmax: bool = False) -> ForwardOutput:
        """LanguageModel::forward (transformer.rs:359-442)."""
        prepared = getattr(batch, "_prepared", None)
        if prepared is None:
            batch.validate()
        S = batch.num_sequences()
        V = self.meta.vocab_size
        if batch.is_empty():
            return ForwardOutput(np.zeros((0, V), np.float32), V, [])
        tokens, positions, counts, ctx, offs, ids = prepared or batch.to_csr()
        bd = BatchDesc(len(tokens), S, tokens.ctypes.data, positions.ctypes.data,
                       counts.ctypes.data, ctx.ctypes.data, offs.ctypes.data, ids.ctypes.data,
                       int(batch.has_prefill))
        logits = np.empty((S, V), dtype=np.float32) if want_logits else None
        am = np.empty(S, dtype=np.int64) if want_argmax else None
        _check(self._backend.lib.orion_hip_model_forward(self.handle, C.byref(bd), _ptr(logits),
                                                         _ptr(am)))
        return ForwardOutput(logits if logits is not None else np.zeros((S, 0), np.float32), V,
                             list(batch.sequence_ids), am)

    def sample(self, params, previous, uniforms) -> List[int]:
        """Samples one token per sequence of the last forward from its logits,
        which stay on the device (runtime/src/sampling.rs DefaultSampler)."""
        par, offs, toks, uni, out = _sampling_args(params, previous, uniforms)
        _check(self._backend.lib.orion_hip_model_sample(self.handle, par, offs.ctypes.data,
                                                        toks.ctypes.data, uni.ctypes.data,
                                                        out.ctypes.data))
        return out[:len(params)].tolist()

    def kv_read(self, layer: int, block: int, slot: int, head: int, is_value: bool) -> np.ndarray:
        out = np.empty(self.meta.head_dim, dtype=np.float32)
        _check(self._backend.lib.orion_hip_model_kv_read(self.handle, layer, block, slot, head,
                                                         int(is_value), out.ctypes.data))
        return out

    def kv_write(self, layer: int, block: int, slot: int, head: int, is_value: bool,
                 vec: Sequence[float]) -> None:
        v = np.ascontiguousarray(vec, dtype=np.float32)
        _check(self._backend.lib.orion_hip_model_kv_write(self.handle, layer, block, slot, head,
                                                          int(is_value), v.ctypes.data, v.size))

    def kv_arena(self):
        p, n = C.c_void_p(), C.c_size_t()
        _check(self._backend.lib.orion_hip_model_kv_arena(self.handle, C.byref(p), C.byref(n)))
        return p.value, n.value

    def kv_layout(self) -> "KvLayout":
        lay = KvLayout()
        _check(self._backend.lib.orion_hip_model_kv_layout(self.handle, C.byref(lay)))
        return lay

    def close(self) -> None:
        if self.handle:
            self._backend.lib.orion_hip_model_destroy(self.handle)
            self.handle = None


def _sampling_args(params, previous, uniforms):
    rows = len(params)
    if len(previous) != rows or len(uniforms) != rows:
        raise ValueError("one params, previous-token list and uniform per row")
    par = (SamplingParams * max(rows, 1))(*params)
    offs = np.zeros(rows + 1, np.int64)
    offs[1:] = np.cumsum([len(p) for p in previous])
    toks = (np.concatenate([np.asarray(p, np.uint32) for p in previous])
            if rows and offs[-1] else np.zeros(1, np.uint32))
    uni = np.ascontiguousarray(uniforms, dtype=np.float32)
    out = np.empty(max(rows, 1), np.int32)
    return par, offs, toks, uni, out


def sample(be: HipBackend, logits_ptr: int, rows: int, vocab: int, params, previous, uniforms):
    """Sampler::sample on the device for each row of device logits (filtered in
    place); `uniforms` are the draws' r values.  Returns the tokens."""
    par, offs, toks, uni, out = _sampling_args(params, previous, uniforms)
    _check(be.lib.orion_hip_sample(be.handle, logits_ptr, rows, vocab, par, offs.ctypes.data,
                                   toks.ctypes.data, uni.ctypes.data, out.ctypes.data))
    return out[:rows].tolist()


def synthetic_value(seed: int, which: int, layer: int, index: int, std: float = 0.02) -> float:
    return load_library().orion_hip_synthetic_value(seed, which, layer, index, std)


# ---------------------------------------------------------------------------
# Op-level entry points (device buffers)
# ---------------------------------------------------------------------------


def kv_layout(num_layers, num_blocks, block_size, num_kv_heads, head_dim, dtype,
              head_major=False) -> KvLayout:
    """Arena geometry; head_major selects the [kv_head][k|v][slot][dim] block order
    instead of the reference [k|v][slot][kv_head][dim]."""
    return KvLayout(num_layers, num_blocks, block_size, num_kv_heads, head_dim, dtype,
                    1 if head_major else 0)


class DecodePlan:
    """orion_hip_decode_plan: the longest-first (row, chunk) work list for one
    batch of decode rows, built from the rows' positions (host copy)."""

    def __init__(self, be: HipBackend, positions, row_seq, bt_offsets, bt_ids, num_q_heads: int,
                 num_kv_heads: int, head_dim: int, block_size: int):
        pos = np.ascontiguousarray(positions, dtype=np.uint32)
        rs = np.ascontiguousarray(row_seq, dtype=np.int32)
        bo = np.ascontiguousarray(bt_offsets, dtype=np.int64)
        bi = np.ascontiguousarray(bt_ids, dtype=np.uint32)
        h = C.c_void_p()
        _check(be.lib.orion_hip_decode_plan_create(be.handle, pos.ctypes.data, rs.ctypes.data,
                                                   bo.ctypes.data, bi.ctypes.data, pos.size,
                                                   num_q_heads, num_kv_heads, head_dim,
                                                   block_size, C.byref(h)))
        self.be = be
        self.handle = h.value

    def info(self):
        c, n, m = C.c_int64(), C.c_int64(), C.c_int64()
        _check(self.be.lib.orion_hip_decode_plan_info(self.handle, C.byref(c), C.byref(n),
                                                      C.byref(m)))
        p, r = C.c_int64(), C.c_int64()
        _check(self.be.lib.orion_hip_decode_plan_packed(self.handle, C.byref(p), C.byref(r)))
        return {"chunk": c.value, "num_work": n.value, "max_splits": m.value,
                "packed_items": p.value, "rows_per_pack": r.value}

    def close(self) -> None:
        if self.handle:
            self.be.lib.orion_hip_decode_plan_destroy(self.handle)
            self.handle = None


def paged_attention_decode(be: HipBackend, kv: KvLayout, arena_ptr: int, layer: int, q_ptr: int,
                           num_rows: int, num_q_heads: int, pos_ptr: int, row_seq_ptr: int,
                           bt_off_ptr: int, bt_ids_ptr: int, plan: DecodePlan,
                           out_ptr: int) -> None:
    _check(be.lib.orion_hip_paged_attention_decode(
        be.handle, C.byref(kv), arena_ptr, layer, q_ptr, num_rows, num_q_heads, pos_ptr,
        row_seq_ptr, bt_off_ptr, bt_ids_ptr, plan.handle, out_ptr))


def paged_attention_prefill(be: HipBackend, kv: KvLayout, arena_ptr: int, layer: int, q_ptr: int,
                            num_q_heads: int, num_seqs: int, row_start_ptr: int,
                            row_count_ptr: int, first_pos_ptr: int, bt_off_ptr: int,
                            bt_ids_ptr: int, max_rows: int, max_position: int,
                            out_ptr: int, hilo=False) -> None:
    """hilo: False / True (bf16 / hi+lo Q and P), or the C mode 0..3
    (2: hi/lo Q only, 3: hi/lo P only)."""
    mode = int(hilo) if not isinstance(hilo, bool) else (1 if hilo else 0)
    _check(be.lib.orion_hip_paged_attention_prefill(
        be.handle, C.byref(kv), arena_ptr, layer, q_ptr, num_q_heads, num_seqs, row_start_ptr,
        row_count_ptr, first_pos_ptr, bt_off_ptr, bt_ids_ptr, max_rows, max_position,
        mode, out_ptr))


def rope_and_cache(be: HipBackend, kv: KvLayout, arena_ptr: int, layer: int, num_rows: int,
                   num_q_heads: int, q_in: int, q_stride: int, q_out: int, k: int, k_stride: int,
                   v: int, v_stride: int, pos: int, row_seq: int, bt_off: int, bt_ids: int,
                   cos: int, sin: int) -> None:
    _check(be.lib.orion_hip_rope_and_cache(be.handle, C.byref(kv), arena_ptr, layer, num_rows,
                                           num_q_heads, q_in, q_stride, q_out, k, k_stride, v,
                                           v_stride, pos, row_seq, bt_off, bt_ids, cos, sin))


def rmsnorm(be: HipBackend, x: int, w: int, rows: int, cols: int, eps: float, out: int) -> None:
    _check(be.lib.orion_hip_rmsnorm(be.handle, x, w, rows, cols, eps, out))


GEMM_STORE, GEMM_ACCUMULATE, GEMM_SWIGLU = 0, 1, 2


def gemm(be: HipBackend, x: int, w: int, bias: Optional[int], M: int, N: int, K: int,
         accumulate, out: int) -> None:
    """orion_hip_gemm; `accumulate` is a bool (store / accumulate) or one of
    GEMM_STORE, GEMM_ACCUMULATE, GEMM_SWIGLU."""
    _check(be.lib.orion_hip_gemm(be.handle, x, w, bias, M, N, K, int(accumulate), out))


def silu_mul(be: HipBackend, gate: int, up: int, count: int) -> None:
    _check(be.lib.orion_hip_silu_mul(be.handle, gate, up, count))


def argmax(be: HipBackend, logits: int, rows: int, cols: int, out: int) -> None:
    _check(be.lib.orion_hip_argmax(be.handle, logits, rows, cols, out))


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (as the device does)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)

"""CPU oracle for the OrionServe-RS hot path.  TEST INFRASTRUCTURE ONLY.

ctypes wrapper over liborion_oracle.so, the C++ restatement of the reference CPU
backend (crates/orion-models/src/{tensor,attention,transformer}.rs, see
oracle/orion_oracle.cpp for per-function citations).  Only tests/, the smoke
check in __graft_entry__.py and bench.py's cpu_baseline leg use it, and only as
the checker / CPU baseline — never as the product path.

Pinning status (what checks each function besides its own restatement):
  locate, KvStore offsets/read/write ... reference KATs + brute force enumeration
  linear, rms_norm, silu, swiglu ......... reference KATs + float64 numpy
  softmax_inplace ........................ reference KATs + float64 numpy
  RopeTable / apply_rope ................. reference KATs (identity, rotate-half
                                           pairing, norm, relative position) + float64
  paged_attention ........................ reference KATs + torch SDPA on de-paged K/V
  model forward .......................... reference fixture model invariants +
                                           float64 numpy restatement of the forward
  argmax, validate ....................... reference KATs
  DefaultSampler (sample) ................ reference KATs (sampling.rs:296-552) + an
                                           independent float64 numpy restatement on
                                           small rows (tests/test_oracle_sampling.py)
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import List, Optional, Sequence, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborion_oracle.so")

W_EMBED, W_FINAL_NORM, W_LM_HEAD = 0, 1, 2
W_INPUT_NORM, W_Q, W_K, W_V, W_O = 3, 4, 5, 6, 7
W_Q_BIAS, W_K_BIAS, W_V_BIAS, W_POST_NORM = 8, 9, 10, 11
W_GATE, W_UP, W_DOWN = 12, 13, 14


class OracleError(Exception):
    """EngineError::Internal raised by the oracle."""


def build() -> str:
    """Compiles the oracle with its Makefile (gcc, -ffp-contract=off, OpenMP)."""
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liborion_oracle.so"], check=True)
    return LIB_PATH


class OracleModelDesc(C.Structure):
    _fields_ = [
        ("num_layers", C.c_int32), ("hidden", C.c_int32), ("num_q_heads", C.c_int32),
        ("num_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("ffn", C.c_int32),
        ("vocab", C.c_int32), ("max_positions", C.c_int32), ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float), ("has_qkv_bias", C.c_int32), ("tied_lm_head", C.c_int32),
        ("num_blocks", C.c_int32), ("block_size", C.c_int32),
    ]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = C.CDLL(LIB_PATH)
    vp, i64, f32, u32 = C.c_void_p, C.c_int64, C.c_float, C.c_uint32
    sig = {
        "oracle_last_error": ([], C.c_char_p),
        "oracle_num_threads": ([], C.c_int),
        "oracle_set_num_threads": ([C.c_int], None),
        "oracle_linear": ([vp, i64, i64, vp, i64, i64, vp, i64, vp], C.c_int),
        "oracle_rms_norm": ([vp, i64, i64, vp, i64, f32], C.c_int),
        "oracle_silu": ([f32], f32),
        "oracle_swiglu": ([vp, i64, i64, vp, i64, i64], C.c_int),
        "oracle_softmax_inplace": ([vp, i64], None),
        "oracle_rope_table": ([i64, i64, f32, vp, vp], C.c_int),
        "oracle_apply_rope": ([vp, i64, vp, vp, i64], C.c_int),
        "oracle_locate": ([vp, i64, i64, i64, C.POINTER(u32), C.POINTER(i64)], C.c_int),
        "oracle_kv_len": ([i64] * 5, i64),
        "oracle_kv_offset": ([i64] * 5 + [i64, u32, C.c_int, i64, i64], i64),
        "oracle_kv_write": ([vp] + [i64] * 6 + [u32, i64, i64, C.c_int, vp, i64], C.c_int),
        "oracle_kv_read": ([vp] + [i64] * 6 + [u32, i64, i64, C.c_int, vp], C.c_int),
        "oracle_paged_attention": ([vp, i64, i64, i64, i64, i64, vp, i64, vp, i64, i64, i64,
                                    i64, i64, i64, i64, i64, vp, i64], C.c_int),
        "oracle_paged_attention_rows": ([vp, i64, i64, i64, i64, i64, i64, i64, i64, vp, vp,
                                         vp, vp, vp, vp], C.c_int),
        "oracle_argmax": ([vp, i64], i64),
        "oracle_sample": ([vp, i64, vp, i64, f32, i64, f32, f32, f32, C.POINTER(f32)], i64),
        "oracle_validate": ([vp, vp, i64, f32, f32, C.POINTER(f32), C.POINTER(f32),
                             C.POINTER(i64)], i64),
        "oracle_model_create": ([C.POINTER(OracleModelDesc)], vp),
        "oracle_model_destroy": ([vp], None),
        "oracle_model_kv": ([vp, C.POINTER(i64)], C.POINTER(C.c_float)),
        "oracle_model_set_weight": ([vp, C.c_int, C.c_int, vp, i64], C.c_int),
        "oracle_model_forward": ([vp, i64, i64, vp, vp, vp, vp, vp, vp, vp], C.c_int),
        "oracle_model_set_kv_bf16": ([vp, C.c_int], None),
        "oracle_synthetic_fill": ([C.c_uint64, C.c_int, C.c_int, f32, i64, vp], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != 0:
        raise OracleError(lib().oracle_last_error().decode())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def synthetic_weight(seed: int, which: int, layer: int, count: int, std: float = 0.02):
    """The HIP library's synthetic weight values (a test input generator restated in
    the oracle, not a reference function): f32, bf16-exact, logical row-major order."""
    out = np.empty(count, np.float32)
    lib().oracle_synthetic_fill(seed, which, layer, std, count, out.ctypes.data)
    return out


def set_num_threads(n: int) -> None:
    lib().oracle_set_num_threads(n)


def num_threads() -> int:
    return lib().oracle_num_threads()


# ---------------------------------------------------------------------------
# tensor.rs
# ---------------------------------------------------------------------------


def linear(x: np.ndarray, weight: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    """tensor.rs:96-130.  x [n, k], weight [out, in] -> [n, out]."""
    x = _f32(x)
    w = _f32(weight)
    n, k = x.shape
    o, i = w.shape
    b = None if bias is None else _f32(bias)
    out = np.empty((n, o), dtype=np.float32)
    _check(lib().oracle_linear(x.ctypes.data, n, k, w.ctypes.data, o, i,
                               None if b is None else b.ctypes.data,
                               0 if b is None else b.size, out.ctypes.data))
    return out


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """tensor.rs:143-163 (returns a normalised copy)."""
    x = _f32(x).copy()
    w = _f32(weight)
    rows, cols = x.shape
    _check(lib().oracle_rms_norm(x.ctypes.data, rows, cols, w.ctypes.data, w.size, eps))
    return x


def silu(x: float) -> float:
    """tensor.rs:167-169."""
    return lib().oracle_silu(x)


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """tensor.rs:175-189 (returns a new array)."""
    g = _f32(gate).copy()
    u = _f32(up)
    g2 = g.reshape(g.shape[0] if g.ndim > 1 else 1, -1)
    u2 = u.reshape(u.shape[0] if u.ndim > 1 else 1, -1)
    _check(lib().oracle_swiglu(g2.ctypes.data, g2.shape[0], g2.shape[1], u2.ctypes.data,
                               u2.shape[0], u2.shape[1]))
    return g2.reshape(g.shape)


def softmax_inplace(x: np.ndarray) -> np.ndarray:
    """tensor.rs:192-209 (returns the softmaxed copy)."""
    x = _f32(x).copy()
    lib().oracle_softmax_inplace(x.ctypes.data, x.size)
    return x


class RopeTable:
    """tensor.rs:218-274."""

    def __init__(self, head_dim: int, max_positions: int, theta: float):
        self.head_dim = head_dim
        self.max_positions = max_positions
        half = head_dim // 2
        self.cos = np.empty((max_positions, max(half, 0)), dtype=np.float32)
        self.sin = np.empty((max_positions, max(half, 0)), dtype=np.float32)
        _check(lib().oracle_rope_table(head_dim, max_positions, theta, self.cos.ctypes.data,
                                       self.sin.ctypes.data))

    def at(self, pos: int) -> Optional[Tuple[np.ndarray, np.ndarray]]:
        if pos >= self.max_positions:
            return None
        return self.cos[pos], self.sin[pos]


def apply_rope(vec: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """tensor.rs:283-298 (returns the rotated copy)."""
    v = _f32(vec).copy()
    c, s = _f32(cos), _f32(sin)
    if c.size != s.size:
        raise OracleError("cos/sin size mismatch")
    _check(lib().oracle_apply_rope(v.ctypes.data, v.size, c.ctypes.data, s.ctypes.data, c.size))
    return v


# ---------------------------------------------------------------------------
# attention.rs
# ---------------------------------------------------------------------------


def locate(block_table: Sequence[int], position: int, block_size: int):
    """attention.rs:182-186 -> (block, slot) or None."""
    t = np.ascontiguousarray(block_table, dtype=np.uint32)
    b, s = C.c_uint32(), C.c_int64()
    ok = lib().oracle_locate(t.ctypes.data if t.size else None, t.size, position, block_size,
                             C.byref(b), C.byref(s))
    return (b.value, s.value) if ok else None


class KvStore:
    """attention.rs:34-176: flat arena [layer][block][k|v][slot][head][dim] (f32)."""

    def __init__(self, num_layers, num_blocks, block_size, num_kv_heads, head_dim):
        self.dims = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        self.data = np.zeros(lib().oracle_kv_len(*self.dims), dtype=np.float32)

    def __len__(self):
        return self.data.size

    def block_size(self):
        return self.dims[2]

    def num_blocks(self):
        return self.dims[1]

    def offset(self, layer, block, is_value, slot, head) -> int:
        return lib().oracle_kv_offset(*self.dims, layer, block, int(is_value), slot, head)

    def write(self, layer, block, slot, head, is_value, vector) -> None:
        v = _f32(vector)
        _check(lib().oracle_kv_write(self.data.ctypes.data, *self.dims, layer, block, slot, head,
                                     int(is_value), v.ctypes.data, v.size))

    def read(self, layer, block, slot, head, is_value) -> np.ndarray:
        out = np.empty(self.dims[4], dtype=np.float32)
        _check(lib().oracle_kv_read(self.data.ctypes.data, *self.dims, layer, block, slot, head,
                                    int(is_value), out.ctypes.data))
        return out


def paged_attention(store: KvStore, query, block_table, context_len, query_position, layer,
                    num_query_heads, num_kv_heads, head_dim, block_size) -> np.ndarray:
    """attention.rs:219-295 for one query row (AttentionArgs fields as keywords)."""
    q = _f32(query)
    t = np.ascontiguousarray(block_table, dtype=np.uint32)
    out = np.empty(q.size, dtype=np.float32)
    _check(lib().oracle_paged_attention(
        store.data.ctypes.data, *store.dims[:3], store.dims[3], store.dims[4], q.ctypes.data,
        q.size, t.ctypes.data if t.size else None, t.size, context_len, query_position, layer,
        num_query_heads, num_kv_heads, head_dim, block_size, out.ctypes.data, out.size))
    return out


def paged_attention_rows(arena: np.ndarray, dims, layer, hq, q, positions, row_seq, bt_offsets,
                         bt_ids) -> np.ndarray:
    """Per-row paged_attention over many rows (OpenMP over (row, head))."""
    q = _f32(q)
    rows = q.shape[0]
    out = np.empty((rows, hq * dims[4]), dtype=np.float32)
    pos = np.ascontiguousarray(positions, dtype=np.uint32)
    rs = np.ascontiguousarray(row_seq, dtype=np.int32)
    bo = np.ascontiguousarray(bt_offsets, dtype=np.int64)
    bi = np.ascontiguousarray(bt_ids, dtype=np.uint32)
    arena = np.ascontiguousarray(arena, dtype=np.float32)
    _check(lib().oracle_paged_attention_rows(arena.ctypes.data, *dims, layer, hq, rows,
                                             q.ctypes.data, pos.ctypes.data, rs.ctypes.data,
                                             bo.ctypes.data, bi.ctypes.data, out.ctypes.data))
    return out


def argmax(logits) -> Optional[int]:
    """runtime/src/sampling.rs:196-207."""
    x = _f32(logits)
    r = lib().oracle_argmax(x.ctypes.data, x.size)
    return None if r < 0 else r


def sample(logits, previous=(), temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0,
           r=0.5):
    """DefaultSampler::sample (runtime/src/sampling.rs:266-293) with the draw's
    uniform `r` given.  Returns (token or None, filtered logits, margin of r
    to the nearest cumulative boundary)."""
    x = _f32(logits).copy()
    prev = np.ascontiguousarray(previous, dtype=np.uint32)
    m = C.c_float()
    t = lib().oracle_sample(x.ctypes.data, x.size, prev.ctypes.data if prev.size else None,
                            prev.size, temperature, top_k, top_p, repetition_penalty, r,
                            C.byref(m))
    return (None if t < 0 else int(t)), x, m.value


class Tolerance:
    """orion-cuda/src/lib.rs:188-224."""

    def __init__(self, abs_: float, rel: float):
        self.abs = abs_
        self.rel = rel


Tolerance.F32 = Tolerance(1e-5, 1e-5)
Tolerance.F16 = Tolerance(1e-2, 1e-2)


def validate(expected, actual, tol: Tolerance):
    """orion-cuda/src/lib.rs:269-317 -> (mismatches, max_abs, max_rel, worst_index)."""
    e, a = _f32(expected).ravel(), _f32(actual).ravel()
    if e.size != a.size:
        raise OracleError(f"validation shape mismatch: {e.size} vs {a.size}")
    ma, mr, wi = C.c_float(), C.c_float(), C.c_int64()
    mm = lib().oracle_validate(e.ctypes.data, a.ctypes.data, e.size, tol.abs, tol.rel,
                               C.byref(ma), C.byref(mr), C.byref(wi))
    return mm, ma.value, mr.value, (None if wi.value < 0 else wi.value)


# ---------------------------------------------------------------------------
# transformer.rs
# ---------------------------------------------------------------------------


class OracleTransformer:
    """TransformerModel (transformer.rs:137-443) with an f32 KV arena (the
    reference's), or with every K/V element rounded to bf16 when written
    (kv_bf16=True: the KV dtype of the bf16 benchmark configurations)."""

    def __init__(self, num_layers, hidden, num_q_heads, num_kv_heads, head_dim, ffn, vocab,
                 max_positions, rms_norm_eps, rope_theta, has_qkv_bias, tied_lm_head, num_blocks,
                 block_size, kv_bf16=False):
        self.desc = OracleModelDesc(num_layers, hidden, num_q_heads, num_kv_heads, head_dim, ffn,
                                    vocab, max_positions, rms_norm_eps, rope_theta,
                                    int(has_qkv_bias), int(tied_lm_head), num_blocks, block_size)
        self.h = lib().oracle_model_create(C.byref(self.desc))
        if not self.h:
            raise OracleError(lib().oracle_last_error().decode())
        lib().oracle_model_set_kv_bf16(self.h, int(kv_bf16))

    def set_weight(self, which, layer, data) -> None:
        d = _f32(data).ravel()
        _check(lib().oracle_model_set_weight(self.h, which, layer, d.ctypes.data, d.size))

    def kv(self) -> np.ndarray:
        n = C.c_int64()
        p = lib().oracle_model_kv(self.h, C.byref(n))
        return np.ctypeslib.as_array(p, shape=(n.value,))

    def forward(self, tokens, positions, slot_token_counts, context_lens,
                block_tables: List[Sequence[int]]) -> np.ndarray:
        """transformer.rs:359-442 -> logits [S, vocab]."""
        tok = np.ascontiguousarray(tokens, dtype=np.uint32)
        pos = np.ascontiguousarray(positions, dtype=np.uint32)
        cnt = np.ascontiguousarray(slot_token_counts, dtype=np.int64)
        ctx = np.ascontiguousarray(context_lens, dtype=np.int64)
        offs = np.zeros(len(block_tables) + 1, dtype=np.int64)
        if block_tables:
            offs[1:] = np.cumsum([len(t) for t in block_tables])
        ids = (np.concatenate([np.asarray(t, dtype=np.uint32) for t in block_tables])
               if offs[-1] > 0 else np.zeros(1, dtype=np.uint32))
        S = len(slot_token_counts)
        logits = np.empty((S, self.desc.vocab), dtype=np.float32)
        _check(lib().oracle_model_forward(self.h, tok.size, S, tok.ctypes.data, pos.ctypes.data,
                                          cnt.ctypes.data, ctx.ctypes.data, offs.ctypes.data,
                                          ids.ctypes.data, logits.ctypes.data))
        return logits

    def close(self):
        if self.h:
            lib().oracle_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

"""numpy front end of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Loads ``oracle/_build/libjv_oracle.so`` (built by ``oracle/Makefile``): a plain-C restatement of
the reference's GGML block decode (crates/jevons-formats/src/quant.rs), type table
(crates/jevons-formats/src/gguf.rs:107-145), f64 product (crates/jevons-gemma4-diffusion/src/
gpu/tests.rs:445-451) and greedy argmax (crates/jevons-core/src/model.rs:207-219).

Only tests/, the smoke check and bench.py's CPU-baseline leg import this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libjv_oracle.so")

F32, F16, Q5_0, Q8_0, Q4K, Q6K = 0, 1, 6, 8, 12, 14
TYPE_NAMES = {F32: "F32", F16: "F16", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4K: "Q4K", Q6K: "Q6K"}

_lib = None


def build() -> None:
    """Compiles the oracle with its Makefile (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P, S, U32, U64 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_uint64
        L.jvo_type_block.argtypes = [U32, C.POINTER(U32), C.POINTER(U32)]
        L.jvo_f16_to_f32.argtypes = [C.c_uint16]
        L.jvo_f16_to_f32.restype = C.c_float
        L.jvo_f32_to_f16.argtypes = [C.c_float]
        L.jvo_f32_to_f16.restype = C.c_uint16
        L.jvo_bf16_to_f32.argtypes = [C.c_uint16]
        L.jvo_bf16_to_f32.restype = C.c_float
        L.jvo_f32_to_bf16.argtypes = [C.c_float]
        L.jvo_f32_to_bf16.restype = C.c_uint16
        L.jvo_q4k_scale_min.argtypes = [C.c_int, P, P, P]
        L.jvo_dequantize.argtypes = [U32, P, S, P, S]
        L.jvo_packed_words.argtypes = [U32] + [C.POINTER(S)] * 4
        L.jvo_pack.argtypes = [U32, P, S, P, P, P, P]
        L.jvo_matmul_f64.argtypes = [P, S, S, P, S, P]
        L.jvo_greedy.argtypes = [P, S, C.POINTER(C.c_int32), C.POINTER(C.c_double)]
        L.jvo_rng_next.argtypes = [C.POINTER(U64)]
        L.jvo_rng_next.restype = C.c_float
        L.jvo_recipe_q8_0.argtypes = [C.POINTER(U64), S, P]
        L.jvo_recipe_q6k.argtypes = [C.POINTER(U64), S, P]
        L.jvo_recipe_h16_vec.argtypes = [C.POINTER(U64), S, C.c_float, P]
        L.jvo_cpu_dequant_matmul.argtypes = [U32, P, S, S, P, S, P, P, C.c_int, C.c_int]
        L.jvo_group_routes.argtypes = [P, S, S, S, P, P, P]
        L.jvo_group_routes.restype = C.c_int
        L.jvo_omp_max_threads.restype = C.c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def type_block(type_id: int):
    e, b = C.c_uint32(), C.c_uint32()
    if not lib().jvo_type_block(type_id, C.byref(e), C.byref(b)):
        return None
    return (e.value, b.value)


def f16_to_f32(h: int) -> float:
    return lib().jvo_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().jvo_f32_to_f16(f)


def q4k_scale_min(j: int, q: bytes):
    buf = np.frombuffer(bytes(q), dtype=np.uint8).copy()
    s, m = C.c_uint8(), C.c_uint8()
    lib().jvo_q4k_scale_min(j, _ptr(buf), C.addressof(s), C.addressof(m))
    return (s.value, m.value)


class OracleError(Exception):
    pass


DEQUANT_ERRORS = {1: "unsupported tensor type", 2: "dequantization size mismatch"}
PACK_ERRORS = {1: "unsupported tensor type", 2: "tensor is not a whole number of blocks",
               3: "has no GPU block layout"}


def dequantize(type_id: int, raw: np.ndarray, nout: int | None = None) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    tb = type_block(type_id)
    if nout is None:
        nout = 0 if tb is None else raw.size // tb[1] * tb[0]
    out = np.empty(max(nout, 1), dtype=np.float32)
    st = lib().jvo_dequantize(type_id, _ptr(raw), raw.size, _ptr(out), nout)
    if st:
        raise OracleError(DEQUANT_ERRORS[st])
    return out[:nout]


def packed_words(type_id: int):
    v = [C.c_size_t() for _ in range(4)]
    lib().jvo_packed_words(type_id, *[C.byref(x) for x in v])
    return tuple(x.value for x in v)


def pack(type_id: int, raw: np.ndarray):
    """The reference's structure-of-arrays repack: returns (q, h, s, d) arrays."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    tb = type_block(type_id)
    blocks = 0 if tb is None else raw.size // tb[1]
    wq, wh, ws, wd = packed_words(type_id)
    q = np.zeros(max(blocks * wq, 1), np.uint32)
    h = np.zeros(max(blocks * wh, 1), np.uint32)
    s = np.zeros(max(blocks * ws, 1), np.uint32)
    d = np.zeros(max(blocks * wd, 1), np.float32)
    st = lib().jvo_pack(type_id, _ptr(raw), raw.size, _ptr(q), _ptr(h), _ptr(s), _ptr(d))
    if st:
        raise OracleError(PACK_ERRORS[st])
    return q[: blocks * wq], h[: blocks * wh], s[: blocks * ws], d[: blocks * wd]


def matmul_f64(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """out[r, c] = sum_k f64(x[r, k]) * f64(w[c, k])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = x.shape
    n, k2 = w.shape
    assert k == k2
    out = np.empty((m, n), dtype=np.float64)
    lib().jvo_matmul_f64(_ptr(x), m, k, _ptr(w), n, _ptr(out))
    return out


def greedy(row: np.ndarray):
    row = np.ascontiguousarray(row, dtype=np.float32).reshape(-1)
    idx, prob = C.c_int32(), C.c_double()
    buf = row if row.size else np.zeros(1, np.float32)
    if lib().jvo_greedy(_ptr(buf), row.size, C.byref(idx), C.byref(prob)):
        raise OracleError("invalid logits")
    return idx.value, prob.value


def group_routes(ids: np.ndarray, experts: int, bm: int):
    """ops::group (crates/jevons-gemma4-diffusion/src/gpu/ops.rs:522-587): (sorted, offsets,
    jobs) with jobs[0] = job count and (expert, start) pairs after it."""
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    a = ids.size
    max_jobs = (a + bm - 1) // bm + experts
    sorted_ = np.zeros(max(a, 1), np.uint32)
    offsets = np.zeros(experts + 1, np.uint32)
    jobs = np.zeros(1 + 2 * max_jobs, np.uint32)
    buf = ids if a else np.zeros(1, np.uint32)
    lib().jvo_group_routes(_ptr(buf), a, experts, bm, _ptr(sorted_), _ptr(offsets), _ptr(jobs))
    return sorted_[:offsets[experts]], offsets, jobs


def grouped_product_f64(x: np.ndarray, w: np.ndarray, ids: np.ndarray, in_div: int, n: int):
    """Reference of the grouped products: output row a = x[a // in_div] . W[ids[a] n : +n]^T in
    f64 (the check of gpu/tests.rs:379-386), w the decoded [experts n, k] weights."""
    ids = np.asarray(ids)
    out = np.empty((ids.size, n), np.float64)
    for a, e in enumerate(ids):
        out[a] = matmul_f64(x[a // in_div][None, :], w[int(e) * n:(int(e) + 1) * n])[0]
    return out


def softcap(v, cap: float):
    """Final-logit soft capping cap tanh(v / cap) in f64 (gpu/ops.rs:750-758)."""
    return cap * np.tanh(np.asarray(v, np.float64) / cap)


def pick_logits_f64(x: np.ndarray, table: np.ndarray, pairs: np.ndarray, cap: float) -> np.ndarray:
    """pick_logits (gpu/ops.rs:589-634) in f64: softcap(x[row] . E[token]) per (row, token) pair,
    table the decoded [tokens, d] rows."""
    pairs = np.asarray(pairs).reshape(-1, 2)
    dots = np.array([x[r].astype(np.float64) @ table[t].astype(np.float64) for r, t in pairs])
    return softcap(dots, cap)


class Rng:
    """xorshift64 fixture generator of crates/jevons-gemma4-diffusion/src/gpu/tests.rs:11-23."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed)

    def next(self) -> float:
        return lib().jvo_rng_next(C.byref(self.state))

    def recipe_q8_0(self, blocks: int) -> np.ndarray:
        out = np.empty(blocks * 34, np.uint8)
        lib().jvo_recipe_q8_0(C.byref(self.state), blocks, _ptr(out))
        return out

    def recipe_q6k(self, blocks: int) -> np.ndarray:
        out = np.empty(blocks * 210, np.uint8)
        lib().jvo_recipe_q6k(C.byref(self.state), blocks, _ptr(out))
        return out

    def h16_vec(self, n: int, scale: float = 1.0) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().jvo_recipe_h16_vec(C.byref(self.state), n, scale, _ptr(out))
        return out


def cpu_dequant_matmul(type_id: int, raw: np.ndarray, n: int, k: int, x: np.ndarray,
                       threads: int = 0, wdec: np.ndarray | None = None,
                       decode: bool = True) -> np.ndarray:
    """The CPU baseline: decode to f32 then f32-accumulate x . W^T (OpenMP)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.shape[0]
    out = np.empty((m, n), np.float32)
    if wdec is None:
        wdec = np.empty(n * k, np.float32)
    st = lib().jvo_cpu_dequant_matmul(type_id, _ptr(raw), n, k, _ptr(x), m, _ptr(out),
                                      _ptr(wdec), 1 if decode else 0, threads)
    if st:
        raise OracleError(DEQUANT_ERRORS.get(st, "error"))
    return out


def omp_max_threads() -> int:
    return lib().jvo_omp_max_threads()


def normalized_error(got: np.ndarray, want: np.ndarray) -> float:
    """max_i |got - want| / max_j |want| (gpu/tests.rs:37-47; scale floored at 1e-6)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    scale = max(1e-6, float(np.max(np.abs(want))) if want.size else 0.0)
    return float(np.max(np.abs(got - want))) / scale if want.size else 0.0

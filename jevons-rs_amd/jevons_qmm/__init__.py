"""Python front end of the gfx950 quantized GGML products (ctypes over the C ABI).

Mirrors crates/jevons-kernels/src/gemm.rs (QMatrix, Plan, SplitScratch, matmul, matmul_plan,
matvec, matmul_split, matmul_tiled), crates/jevons-kernels/src/lib.rs (Gpu) and
crates/jevons-burn/src/kernels.rs (f16_matmul / f16_linear). Device memory is torch tensors on
the GPU; every product is queued on torch's current stream.

The library must be built (``python jevons-rs_amd/build.py``); nothing here has a CPU path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(os.path.dirname(HERE), "lib")
LIB_PATH = os.path.join(LIB_DIR, "libjevons_qmm.so")
HSACO_PATH = os.path.join(LIB_DIR, "jevons_qmm.hsaco")

# GGML tensor type ids (gguf.rs:120-131)
F32, F16, Q5_0, Q8_0, Q4K, Q6K = 0, 1, 6, 8, 12, 14
# kernel formats (gemm.rs:25-30)
FMT_Q4K, FMT_Q6K, FMT_Q5_0, FMT_Q8_0, FMT_F16 = 0, 1, 2, 3, 4
ACT_F16, ACT_BF16, ACT_F32 = 0, 1, 2
OUT_F32, OUT_BF16 = 0, 1
# Largest row count of the small-row product (gemm.rs:1019)
GEMV_ROWS = 16

STATUS = {0: "ok", 1: "invalid", 2: "unsupported", 3: "hip", 4: "no kernels", 5: "no memory"}


class JvError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status
        self.message = message


class jv_groups(C.Structure):
    _fields_ = [("ids", C.c_void_p), ("offsets", C.c_void_p), ("jobs", C.c_void_p),
                ("max_jobs", C.c_size_t), ("in_div", C.c_uint32), ("rows", C.c_size_t)]


class jv_plan(C.Structure):
    _fields_ = [("bm", C.c_uint32), ("bn", C.c_uint32), ("splits", C.c_uint32)]


class jv_device_info(C.Structure):
    _fields_ = [("device", C.c_int), ("compute_units", C.c_int), ("wave_size", C.c_int),
                ("lds_bytes", C.c_size_t), ("total_memory", C.c_size_t), ("arch", C.c_char * 64)]


_lib = None


def lib() -> C.CDLL:
    """Loads libjevons_qmm.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(f"{LIB_PATH} is missing: run python jevons-rs_amd/build.py")
    L = C.CDLL(LIB_PATH)
    P, S, U32, I = C.c_void_p, C.c_size_t, C.c_uint32, C.c_int
    PP = C.POINTER(C.c_void_p)
    sigs = {
        "jv_type_block": (I, [U32, C.POINTER(U32), C.POINTER(U32)]),
        "jv_open": (I, [I, PP]),
        "jv_close": (None, [P]),
        "jv_device_info_get": (I, [P, C.POINTER(jv_device_info)]),
        "jv_sync": (I, [P]),
        "jv_qmatrix_upload": (I, [P, U32, S, S, S, P, S, PP]),
        "jv_qmatrix_upload_device": (I, [P, U32, S, S, S, P, S, PP]),
        "jv_qmatrix_from_packed": (I, [P, U32, S, S, S, P, S, P, S, P, S, P, S, PP]),
        "jv_qmatrix_f16_view": (I, [P, S, S, P, S, PP]),
        "jv_qmatrix_free": (None, [P]),
        "jv_qmatrix_bytes": (S, [P]),
        "jv_qmatrix_shape": (I, [P, C.POINTER(U32), C.POINTER(S), C.POINTER(S), C.POINTER(S)]),
        "jv_plan_heuristic": (jv_plan, [P, S, I, S]),
        "jv_plan_auto": (jv_plan, [P, S, I]),
        "jv_plan_valid": (I, [P, S, jv_plan]),
        "jv_scratch_new": (I, [P, PP]),
        "jv_scratch_free": (None, [P]),
        "jv_matmul": (I, [P, P, I, S, S, P, P, I, S, P, P]),
        "jv_matmul_noalloc": (I, [P, P, I, S, S, P, P, I, S, P]),
        "jv_matmul_plan": (I, [P, P, I, S, S, P, P, I, S, P, jv_plan, P]),
        "jv_matvec": (I, [P, P, I, S, S, P, P, I, S, P]),
        "jv_matmul_split": (I, [P, P, I, S, S, P, P, I, S, U32, U32, U32, P, P]),
        "jv_f16_matmul": (I, [P, P, S, S, P, S, P, P]),
        "jv_argmax_rows": (I, [P, P, S, S, P, P, P]),
        "jv_matmul_argmax": (I, [P, P, I, S, S, P, P, S, C.c_float, P, P, P]),
        "jv_dequant_rows_f32": (I, [P, P, S, S, P, P]),
        "jv_dequant_rows_f16": (I, [P, P, S, S, P, P]),
        "jv_group_routes": (I, [P, P, S, S, U32, P, P, P, S, P]),
        "jv_matmul_grouped": (I, [P, P, I, S, P, C.POINTER(jv_groups), P, I, S, U32, U32, U32, P, P]),
        "jv_matvec_grouped": (I, [P, P, I, S, P, C.POINTER(jv_groups), P, I, S, U32, P]),
        "jv_softcap_logits": (I, [P, P, S, C.c_float, P]),
        "jv_pick_logits": (I, [P, P, I, S, P, P, S, P, S, C.c_float, P]),
        "jv_tune_bucket": (S, [S]),
        "jv_tune_buckets": (S, [S, S, C.POINTER(S), S]),
        "jv_tune_pick": (I, [C.POINTER(C.c_double), C.POINTER(U32), S, U32]),
        "jv_tuner_new": (I, [P, C.c_char_p, PP]),
        "jv_tuner_open_table": (I, [C.c_char_p, C.c_char_p, PP]),
        "jv_tuner_free": (None, [P]),
        "jv_tuner_profile": (C.c_char_p, [P]),
        "jv_tuner_entries": (S, [P]),
        "jv_tuner_lookup_dense": (I, [P, U32, S, S, S, I, C.POINTER(jv_plan)]),
        "jv_tuner_insert_dense": (None, [P, U32, S, S, S, I, jv_plan]),
        "jv_tuner_insert_grouped": (None, [P, U32, S, S, S, S, U32, U32]),
        "jv_tuner_dense": (jv_plan, [P, P, S, I]),
        "jv_tuner_grouped": (I, [P, P, S, C.POINTER(U32), C.POINTER(U32)]),
        "jv_tuner_tune_dense": (I, [P, C.POINTER(P), S, S, I, P, I, S, P, S, P, C.POINTER(I)]),
        "jv_tuner_tune_grouped": (I, [P, C.POINTER(P), S, S, S, P, I, S, P, S, P, S, P, P, P, S, P,
                                      C.POINTER(I)]),
        "jv_tuner_save": (I, [P]),
        "jv_gguf_open": (I, [C.c_char_p, PP]),
        "jv_gguf_close": (None, [P]),
        "jv_gguf_tensor_count": (S, [P]),
        "jv_gguf_tensor_info": (I, [P, S, C.POINTER(C.c_char_p), C.POINTER(U32), C.POINTER(U32),
                                    C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
        "jv_gguf_find": (I, [P, C.c_char_p, C.POINTER(S)]),
        "jv_gguf_u64": (I, [P, C.c_char_p, C.POINTER(C.c_uint64)]),
        "jv_gguf_f32": (I, [P, C.c_char_p, C.POINTER(C.c_float)]),
        "jv_gguf_str": (I, [P, C.c_char_p, C.POINTER(C.c_char_p)]),
        "jv_gguf_read": (I, [P, S, C.c_uint64, C.c_uint64, P]),
        "jv_gguf_upload": (I, [P, P, C.c_char_p, PP]),
        "jv_last_error": (C.c_char_p, []),
    }
    for name, (res, args) in sigs.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _check(status: int) -> None:
    if status != 0:
        raise JvError(status, lib().jv_last_error().decode())


def type_block(type_id: int):
    e, b = C.c_uint32(), C.c_uint32()
    st = lib().jv_type_block(type_id, C.byref(e), C.byref(b))
    return None if st else (e.value, b.value)


def _stream(stream=None):
    import torch

    s = torch.cuda.current_stream() if stream is None else stream
    return C.c_void_p(s.cuda_stream)


def _act(t) -> int:
    import torch

    return {torch.float16: ACT_F16, torch.bfloat16: ACT_BF16, torch.float32: ACT_F32}[t.dtype]


def _out(t) -> int:
    import torch

    return {torch.float32: OUT_F32, torch.bfloat16: OUT_BF16}[t.dtype]


def _dev(t) -> C.c_void_p:
    assert t.is_cuda and t.is_contiguous(), "device buffers must be contiguous GPU tensors"
    return C.c_void_p(t.data_ptr())


class Gpu:
    """The device client (crates/jevons-kernels/src/lib.rs Gpu)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _check(lib().jv_open(device, C.byref(h)))
        self.handle = h
        info = jv_device_info()
        _check(lib().jv_device_info_get(h, C.byref(info)))
        self.info = info
        self.device = device

    def sync(self) -> None:
        _check(lib().jv_sync(self.handle))

    def close(self) -> None:
        if self.handle:
            lib().jv_close(self.handle)
            self.handle = None


class QMatrix:
    """Quantized weights [experts * n, k] resident on the device (gemm.rs:817-953)."""

    def __init__(self, handle: C.c_void_p, owner=None):
        self.handle = handle
        self._owner = owner  # keeps a borrowed buffer alive
        fmt, n, k, e = C.c_uint32(), C.c_size_t(), C.c_size_t(), C.c_size_t()
        _check(lib().jv_qmatrix_shape(handle, C.byref(fmt), C.byref(n), C.byref(k), C.byref(e)))
        self.fmt, self.n, self.k, self.experts = fmt.value, n.value, k.value, e.value

    @staticmethod
    def upload(gpu: Gpu, kind: int, n: int, k: int, experts: int, raw) -> "QMatrix":
        raw = np.ascontiguousarray(np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray)) else raw,
                                   dtype=np.uint8).reshape(-1)
        h = C.c_void_p()
        _check(lib().jv_qmatrix_upload(gpu.handle, kind, n, k, experts,
                                       C.c_void_p(raw.ctypes.data if raw.size else 0), raw.size, C.byref(h)))
        return QMatrix(h)

    @staticmethod
    def upload_device(gpu: Gpu, kind: int, n: int, k: int, experts: int, raw_dev) -> "QMatrix":
        h = C.c_void_p()
        _check(lib().jv_qmatrix_upload_device(gpu.handle, kind, n, k, experts, _dev(raw_dev),
                                              raw_dev.numel() * raw_dev.element_size(), C.byref(h)))
        return QMatrix(h)

    @staticmethod
    def from_packed(gpu: Gpu, kind: int, n: int, k: int, experts: int, q, h, s, d) -> "QMatrix":
        arrs = [np.ascontiguousarray(a, dtype=t) for a, t in
                ((q, np.uint32), (h, np.uint32), (s, np.uint32), (d, np.float32))]
        ptrs = [C.c_void_p(a.ctypes.data if a.size else 0) for a in arrs]
        out = C.c_void_p()
        _check(lib().jv_qmatrix_from_packed(gpu.handle, kind, n, k, experts,
                                            ptrs[0], arrs[0].size, ptrs[1], arrs[1].size,
                                            ptrs[2], arrs[2].size, ptrs[3], arrs[3].size, C.byref(out)))
        return QMatrix(out)

    @staticmethod
    def f16_view(gpu: Gpu, n: int, k: int, weight) -> "QMatrix":
        """Views a row-major float16 GPU tensor [n, k] without copying it."""
        h = C.c_void_p()
        _check(lib().jv_qmatrix_f16_view(gpu.handle, n, k, _dev(weight), weight.numel() // 2, C.byref(h)))
        return QMatrix(h, owner=weight)

    def bytes(self) -> int:
        return lib().jv_qmatrix_bytes(self.handle)

    def free(self) -> None:
        if self.handle:
            lib().jv_qmatrix_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Plan:
    """Launch configuration (gemm.rs:973-1016). bm == 0 selects the small-row kernel."""

    ROW_TILES = (32, 64, 128)
    COL_TILES = (64, 128)
    GFX950_COL_TILES = (64, 128, 256)
    # gfx950 Q4_K tile: Plan(256, 128, 1)
    GFX950_Q4K_TILE = (256, 128)

    def __init__(self, bm: int, bn: int, splits: int):
        self.bm, self.bn, self.splits = bm, bn, splits

    def c(self) -> jv_plan:
        return jv_plan(self.bm, self.bn, self.splits)

    @staticmethod
    def _from(p: jv_plan) -> "Plan":
        return Plan(p.bm, p.bn, p.splits)

    @staticmethod
    def heuristic(w: QMatrix, m: int, row_invariant: bool, groups_target: int) -> "Plan":
        return Plan._from(lib().jv_plan_heuristic(w.handle, m, int(row_invariant), groups_target))

    @staticmethod
    def auto(w: QMatrix, m: int, row_invariant: bool = False) -> "Plan":
        return Plan._from(lib().jv_plan_auto(w.handle, m, int(row_invariant)))

    def valid_for(self, w: QMatrix, m: int) -> bool:
        return bool(lib().jv_plan_valid(w.handle, m, self.c()))

    def __eq__(self, o):
        return isinstance(o, Plan) and (self.bm, self.bn, self.splits) == (o.bm, o.bn, o.splits)

    def __repr__(self):
        return f"Plan {{ bm: {self.bm}, bn: {self.bn}, splits: {self.splits} }}"


class SplitScratch:
    """Split-K partial sums and argmax partials, grown on demand (gemm.rs:1041-1065)."""

    def __init__(self, gpu: Gpu):
        h = C.c_void_p()
        _check(lib().jv_scratch_new(gpu.handle, C.byref(h)))
        self.handle = h

    def free(self) -> None:
        if self.handle:
            lib().jv_scratch_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _sh(s):
    return s.handle if s is not None else None


def matmul(gpu: Gpu, x, m: int, w: QMatrix, out, scratch: SplitScratch | None = None, stream=None):
    """out[m, n] = x[m, k] . W^T with this library's gfx950 plan (gemm.rs:1069-1088)."""
    _check(lib().jv_matmul(gpu.handle, _dev(x), _act(x), x.numel(), m, w.handle, _dev(out),
                           _out(out), out.numel(), _sh(scratch), _stream(stream)))


def matmul_noalloc(gpu: Gpu, x, m: int, w: QMatrix, out, stream=None):
    """matmul's product staged through the library's fixed device array instead of allocated
    buffers (no counterpart in the reference; for callers that cannot allocate)."""
    _check(lib().jv_matmul_noalloc(gpu.handle, _dev(x), _act(x), x.numel(), m, w.handle, _dev(out),
                                   _out(out), out.numel(), _stream(stream)))


NOALLOC_SCRATCH_BYTES = 32 << 20  # JV_NOALLOC_SCRATCH_BYTES


def matmul_plan(gpu: Gpu, x, m: int, w: QMatrix, out, scratch: SplitScratch | None, plan: Plan,
                stream=None):
    """Product with an explicit plan (gemm.rs:1093-1119)."""
    _check(lib().jv_matmul_plan(gpu.handle, _dev(x), _act(x), x.numel(), m, w.handle, _dev(out),
                                _out(out), out.numel(), _sh(scratch), plan.c(), _stream(stream)))


def matvec(gpu: Gpu, x, m: int, w: QMatrix, out, stream=None):
    """Small-row product, m <= 16 (gemm.rs:1136-1168)."""
    _check(lib().jv_matvec(gpu.handle, _dev(x), _act(x), x.numel(), m, w.handle, _dev(out),
                           _out(out), out.numel(), _stream(stream)))


def matmul_split(gpu: Gpu, x, m: int, w: QMatrix, out, bm: int, bn: int, splits: int,
                 scratch: SplitScratch | None, stream=None):
    """Tiled product with split-K (gemm.rs:1206-1257)."""
    _check(lib().jv_matmul_split(gpu.handle, _dev(x), _act(x), x.numel(), m, w.handle, _dev(out),
                                 _out(out), out.numel(), bm, bn, splits, _sh(scratch), _stream(stream)))


def matmul_tiled(gpu: Gpu, x, m: int, w: QMatrix, out, bm: int, bn: int, stream=None):
    """matmul_split without split-K (gemm.rs:1122-1133)."""
    matmul_split(gpu, x, m, w, out, bm, bn, 1, None, stream)


def f16_matmul(gpu: Gpu, x, weight, stream=None):
    """Burn's GemmOps::f16_matmul (crates/jevons-burn/src/kernels.rs:52-97): float16 x [m, k]
    times float16 weight [n, k]^T into a new float32 [m, n]."""
    import torch

    x = x.contiguous()
    weight = weight.contiguous()
    assert x.dtype == torch.float16 and weight.dtype == torch.float16, "f16 matmul needs FP16 operands"
    m, k = x.shape
    n = weight.shape[0]
    assert weight.shape[1] == k, "f16 matmul needs dense row-major [M, K] x [N, K]"
    out = torch.empty((m, n), dtype=torch.float32, device=x.device)
    _check(lib().jv_f16_matmul(gpu.handle, _dev(x), m, k, _dev(weight), n, _dev(out), _stream(stream)))
    return out


F16_ROW_LIMIT = 16384.0


def f16_linear(gpu: Gpu, x, weight):
    """x @ weight^T in f32 with x cast to FP16 (kernels.rs:109-114)."""
    import torch

    return f16_matmul(gpu, x.to(torch.float16), weight)


def f16_linear_scaled(gpu: Gpu, x, weight):
    """f16_linear with rows above F16_ROW_LIMIT divided down first and multiplied back
    (kernels.rs:120-130)."""
    import torch

    x = x.to(torch.float32)
    scale = (x.abs().amax(dim=1, keepdim=True) / F16_ROW_LIMIT).clamp_min(1.0)
    return f16_linear(gpu, x / scale, weight) * scale


class Groups:
    """Expert grouping produced on the device (Groups, gemm.rs:955-966): `ids` (sorted assignment
    ids), `offsets` [experts + 1] and `jobs` are device uint32 tensors (int32 storage)."""

    def __init__(self, ids, offsets, jobs, max_jobs: int, in_div: int, rows: int):
        self.ids, self.offsets, self.jobs = ids, offsets, jobs
        self.max_jobs, self.in_div, self.rows = max_jobs, in_div, rows

    def c(self) -> jv_groups:
        return jv_groups(_dev(self.ids), _dev(self.offsets), _dev(self.jobs), self.max_jobs,
                         self.in_div, self.rows)


def group_routes(gpu: Gpu, ids, experts: int, bm: int, in_div: int = 1, stream=None,
                 into: "Groups | None" = None) -> Groups:
    """ops::group_routes (crates/jevons-gemma4-diffusion/src/gpu/ops.rs:1100-1130): groups the
    routed assignments `ids` (device int32 expert per assignment) by expert for row tiles of bm.
    `into`: the Groups of an earlier call with the same sizes, whose buffers are written again
    (no allocation, e.g. under graph capture)."""
    import torch

    a = ids.numel()
    max_jobs = (a + bm - 1) // bm + experts
    if into is not None:
        sorted_, offsets, jobs = into.ids, into.offsets, into.jobs
        if sorted_.numel() != max(a, 1) or offsets.numel() != experts + 1 or jobs.numel() != 1 + 2 * max_jobs:
            raise ValueError("group_routes: `into` was made for other sizes")
    else:
        sorted_ = torch.zeros(max(a, 1), dtype=torch.int32, device=ids.device)
        offsets = torch.zeros(experts + 1, dtype=torch.int32, device=ids.device)
        jobs = torch.zeros(1 + 2 * max_jobs, dtype=torch.int32, device=ids.device)
    _check(lib().jv_group_routes(gpu.handle, _dev(ids), a, experts, bm, _dev(sorted_), _dev(offsets),
                                 _dev(jobs), jobs.numel(), _stream(stream)))
    return Groups(sorted_, offsets, jobs, max_jobs, in_div, a)


def matmul_grouped(gpu: Gpu, x, w: QMatrix, g: Groups, out, bm: int, bn: int, splits: int,
                   scratch: SplitScratch | None, stream=None):
    """Expert-grouped product (matmul_grouped, gemm.rs:1274-1321)."""
    gc = g.c()
    _check(lib().jv_matmul_grouped(gpu.handle, _dev(x), _act(x), x.numel(), w.handle, C.byref(gc),
                                   _dev(out), _out(out), out.numel(), bm, bn, splits, _sh(scratch),
                                   _stream(stream)))


def matvec_grouped(gpu: Gpu, x, w: QMatrix, g: Groups, out, mr: int, stream=None):
    """Expert-grouped small-row product (matvec_grouped, gemm.rs:1171-1203)."""
    gc = g.c()
    _check(lib().jv_matvec_grouped(gpu.handle, _dev(x), _act(x), x.numel(), w.handle, C.byref(gc),
                                   _dev(out), _out(out), out.numel(), mr, _stream(stream)))


def tune_bucket(m: int) -> int:
    """Row bucket (bucket, tune.rs:73-76)."""
    return lib().jv_tune_bucket(m)


def tune_buckets(lo: int, hi: int) -> list[int]:
    """Buckets tuned for row counts up to hi (buckets, tune.rs:489-497)."""
    n = lib().jv_tune_buckets(lo, hi, None, 0)
    out = (C.c_size_t * max(n, 1))()
    lib().jv_tune_buckets(lo, hi, out, n)
    return list(out[:n])


def tune_pick(times, ids, baseline: int) -> int | None:
    """Index of the chosen candidate (pick, tune.rs:556-566), None for no candidates."""
    n = len(times)
    t = (C.c_double * max(n, 1))(*times)
    i = (C.c_uint32 * max(n, 1))(*ids)
    r = lib().jv_tune_pick(t, i, n, baseline)
    return None if r < 0 else r


class Tuner:
    """Launch-plan tuner and its table (Tuner, crates/jevons-gemma4-diffusion/src/gpu/tune.rs)."""

    def __init__(self, handle):
        self.handle = handle

    @staticmethod
    def new(gpu: "Gpu", path: str | None) -> "Tuner":
        h = C.c_void_p()
        _check(lib().jv_tuner_new(gpu.handle, path.encode() if path else None, C.byref(h)))
        return Tuner(h)

    @staticmethod
    def open_table(profile: str, path: str | None) -> "Tuner":
        h = C.c_void_p()
        _check(lib().jv_tuner_open_table(profile.encode(), path.encode() if path else None, C.byref(h)))
        return Tuner(h)

    def __del__(self):
        if getattr(self, "handle", None):
            lib().jv_tuner_free(self.handle)
            self.handle = None

    @property
    def profile(self) -> str:
        return lib().jv_tuner_profile(self.handle).decode()

    def entries(self) -> int:
        return lib().jv_tuner_entries(self.handle)

    def lookup_dense(self, fmt: int, n: int, k: int, m: int, row_invariant: bool):
        p = jv_plan()
        if lib().jv_tuner_lookup_dense(self.handle, fmt, n, k, m, int(row_invariant), C.byref(p)):
            return Plan(p.bm, p.bn, p.splits)
        return None

    def insert_dense(self, fmt, n, k, bucket, row_invariant, plan: "Plan"):
        lib().jv_tuner_insert_dense(self.handle, fmt, n, k, bucket, int(row_invariant), plan.c())

    def insert_grouped(self, fmt, n, k, experts, bucket, bm, bn):
        lib().jv_tuner_insert_grouped(self.handle, fmt, n, k, experts, bucket, bm, bn)

    def dense(self, w: "QMatrix", m: int, row_invariant: bool) -> "Plan":
        p = lib().jv_tuner_dense(self.handle, w.handle, m, int(row_invariant))
        return Plan(p.bm, p.bn, p.splits)

    def grouped(self, w: "QMatrix", rows: int):
        bm, bn = C.c_uint32(), C.c_uint32()
        _check(lib().jv_tuner_grouped(self.handle, w.handle, rows, C.byref(bm), C.byref(bn)))
        return bm.value, bn.value

    def tune_dense(self, ws, m: int, row_invariant: bool, x, out, scratch) -> bool:
        arr = (C.c_void_p * len(ws))(*[w.handle for w in ws])
        added = C.c_int()
        _check(lib().jv_tuner_tune_dense(self.handle, arr, len(ws), m, int(row_invariant), _dev(x), _act(x),
                                         x.numel(), _dev(out), out.numel(), _sh(scratch), C.byref(added)))
        return bool(added.value)

    def tune_grouped(self, ws, rows: int, top_k: int, x, out, route_ids, sorted_, offsets, jobs, scratch) -> bool:
        arr = (C.c_void_p * len(ws))(*[w.handle for w in ws])
        added = C.c_int()
        _check(lib().jv_tuner_tune_grouped(self.handle, arr, len(ws), rows, top_k, _dev(x), _act(x), x.numel(),
                                           _dev(out), out.numel(), _dev(route_ids), route_ids.numel(),
                                           _dev(sorted_), _dev(offsets), _dev(jobs), jobs.numel(), _sh(scratch),
                                           C.byref(added)))
        return bool(added.value)

    def save(self) -> None:
        _check(lib().jv_tuner_save(self.handle))


class Gguf:
    """GGUF v2/v3 file (Gguf, crates/jevons-formats/src/gguf.rs:163-372)."""

    def __init__(self, path: str):
        self.handle = None
        h = C.c_void_p()
        _check(lib().jv_gguf_open(path.encode(), C.byref(h)))
        self.handle = h

    def __del__(self):
        if getattr(self, "handle", None):
            lib().jv_gguf_close(self.handle)
            self.handle = None

    def tensors(self) -> dict:
        """name -> (ggml_type, dims, absolute offset, bytes)."""
        out = {}
        for i in range(lib().jv_gguf_tensor_count(self.handle)):
            name, t, nd = C.c_char_p(), C.c_uint32(), C.c_uint32()
            dims, off, nb = (C.c_uint64 * 4)(), C.c_uint64(), C.c_uint64()
            _check(lib().jv_gguf_tensor_info(self.handle, i, C.byref(name), C.byref(t), C.byref(nd), dims,
                                             C.byref(off), C.byref(nb)))
            out[name.value.decode()] = (t.value, list(dims[:nd.value]), off.value, nb.value)
        return out

    def u64(self, key: str) -> int:
        v = C.c_uint64()
        _check(lib().jv_gguf_u64(self.handle, key.encode(), C.byref(v)))
        return v.value

    def f32(self, key: str) -> float:
        v = C.c_float()
        _check(lib().jv_gguf_f32(self.handle, key.encode(), C.byref(v)))
        return v.value

    def str(self, key: str) -> str:
        v = C.c_char_p()
        _check(lib().jv_gguf_str(self.handle, key.encode(), C.byref(v)))
        return v.value.decode()

    def read(self, name: str, start: int = 0, length: int | None = None):
        import numpy as np

        idx = C.c_size_t()
        _check(lib().jv_gguf_find(self.handle, name.encode(), C.byref(idx)))
        if length is None:
            length = self.tensors()[name][3] - start
        buf = np.empty(max(length, 1), np.uint8)
        _check(lib().jv_gguf_read(self.handle, idx.value, start, length, buf.ctypes.data))
        return buf[:length]

    def upload(self, gpu: Gpu, name: str) -> "QMatrix":
        h = C.c_void_p()
        _check(lib().jv_gguf_upload(gpu.handle, self.handle, name.encode(), C.byref(h)))
        return QMatrix(h)


def softcap_logits(gpu: Gpu, x, cap: float, stream=None) -> None:
    """In-place x = cap tanh(x / cap) (softcap_logits, gpu/ops.rs:1159-1168)."""
    _check(lib().jv_softcap_logits(gpu.handle, _dev(x), x.numel(), cap, _stream(stream)))


def pick_logits(gpu: Gpu, x, table: QMatrix, pairs, cap: float, stream=None):
    """Candidate logits cap tanh(x[row] . E[token] / cap) for device int32 (row, token) pairs
    [count, 2] (pick, gpu/ops.rs:1133-1157)."""
    import torch

    count = pairs.numel() // 2
    out = torch.empty(count, dtype=torch.float32, device=x.device)
    _check(lib().jv_pick_logits(gpu.handle, _dev(x), _act(x), x.numel(), table.handle, _dev(pairs),
                                count, _dev(out), out.numel(), cap, _stream(stream)))
    return out


def argmax_rows(gpu: Gpu, logits, scratch: SplitScratch, stream=None):
    """Per-row argmax of float32 logits [rows, n] with greedy's rule (first max wins;
    a non-finite row gives -1) (crates/jevons-core/src/model.rs:207-219)."""
    import torch

    rows, n = logits.shape
    idx = torch.empty(rows, dtype=torch.int32, device=logits.device)
    _check(lib().jv_argmax_rows(gpu.handle, _dev(logits), rows, n, _dev(idx), scratch.handle,
                                _stream(stream)))
    return idx


def matmul_argmax(gpu: Gpu, x, m: int, w: QMatrix, out, cap: float, scratch: SplitScratch, stream=None):
    """The vocabulary projection's logits into float32 `out` [m, n], soft-capped when cap > 0,
    and greedy's argmax of every row (crates/jevons-gemma4-diffusion/src/model.rs:1192-1204, then
    crates/jevons-core/src/model.rs:207-219 per row): the int32 indices, -1 for a row holding a
    non-finite value."""
    import torch

    idx = torch.empty(m, dtype=torch.int32, device=out.device)
    _check(lib().jv_matmul_argmax(gpu.handle, _dev(x), _act(x), x.numel(), m, w.handle, _dev(out),
                                  out.numel(), cap, _dev(idx), scratch.handle, _stream(stream)))
    return idx


def dequant_rows(gpu: Gpu, w: QMatrix, row0: int, rows: int, f16: bool = False, stream=None):
    """The products' device decoder applied to rows [row0, row0 + rows): FP32 weights equal to
    quant::dequantize, or the FP16 tile values the MFMA consumes."""
    import torch

    out = torch.empty((rows, w.k), dtype=torch.float16 if f16 else torch.float32, device="cuda")
    fn = lib().jv_dequant_rows_f16 if f16 else lib().jv_dequant_rows_f32
    _check(fn(gpu.handle, w.handle, row0, rows, _dev(out), _stream(stream)))
    return out


def header_symbols(header: str | None = None) -> list[str]:
    """Function names declared in include/jevons_qmm.h."""
    import re

    if header is None:
        header = os.path.join(os.path.dirname(os.path.dirname(HERE)), "include", "jevons_qmm.h")
    text = open(header).read()
    return sorted(set(re.findall(r"\b(jv_[a-z0-9_]+)\s*\(", text)))

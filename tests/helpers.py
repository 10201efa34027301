"""Shared test helpers: device tensors from numpy, the reference's error metric."""
import numpy as np
import torch

import oracle as O
from jevons_qmm import synth


def bf16_tensor(x32: np.ndarray):
    """float32 numpy -> (device bfloat16 tensor, the exact float32 values it holds)."""
    bits = synth.to_bf16(x32)
    t = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).cuda()
    return t, synth.bf16_to_f32(bits).reshape(x32.shape)


def f16_tensor(x32: np.ndarray):
    h = x32.astype(np.float16)
    return torch.from_numpy(h.copy()).cuda(), h.astype(np.float32)


def f32_tensor(x32: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(x32, dtype=np.float32)).cuda(), x32.astype(np.float32)


def activations(act: str, x32: np.ndarray):
    return {"bf16": bf16_tensor, "f16": f16_tensor, "f32": f32_tensor}[act](x32)


def err(got, want) -> float:
    """max |got - want| / max |want| (crates/jevons-gemma4-diffusion/src/gpu/tests.rs:37-47)."""
    return O.normalized_error(got, want)


def oracle_product(type_id: int, raw: np.ndarray, n: int, k: int, x32: np.ndarray) -> np.ndarray:
    w = O.dequantize(type_id, raw).reshape(n, k)
    return O.matmul_f64(x32, w)


def say(*a):
    print(*a, flush=True)


def write_gguf(path: str, metadata: dict, tensors: list, version: int = 3, alignment: int | None = None,
               corrupt: str | None = None) -> None:
    """A GGUF v2/v3 file (the layout gguf.rs:234-321 reads): metadata values given as
    (type id, value) pairs, tensors as (name, dims, ggml type id, raw bytes). `corrupt` plants one
    format error for the rejection tests."""
    import struct

    def s(v: str) -> bytes:
        b = v.encode()
        return struct.pack("<Q", len(b)) + b

    def val(kind, v):
        fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}
        if kind == 8:
            return s(v)
        if kind == 9:
            inner, items = v
            return struct.pack("<IQ", inner, len(items)) + b"".join(val(inner, x) for x in items)
        return struct.pack(fmt[kind], v)

    meta = dict(metadata)
    if alignment is not None:
        meta["general.alignment"] = (4, alignment)
    align = alignment or 32
    head = bytearray(b"GGUF" if corrupt != "magic" else b"GGUX")
    head += struct.pack("<IQQ", version, len(tensors), len(meta) + (1 if corrupt == "dup_key" else 0))
    items = list(meta.items()) + ([next(iter(meta.items()))] if corrupt == "dup_key" else [])
    for k, (kind, v) in items:
        head += s(k) + struct.pack("<I", kind) + val(kind, v)
    offsets, off = [], 0
    for name, dims, ttype, raw in tensors:
        offsets.append(off)
        off = (off + len(raw) + align - 1) // align * align
    for (name, dims, ttype, raw), o in zip(tensors, offsets):
        o2 = o + (8 if corrupt == "misaligned" else 0)
        head += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ttype, o2)
    data_start = (len(head) + align - 1) // align * align
    out = bytes(head) + bytes(data_start - len(head))
    for (name, dims, ttype, raw), o in zip(tensors, offsets):
        out += bytes(data_start + o - len(out)) + bytes(raw)
    if corrupt == "truncate":
        out = out[:-16]
    with open(path, "wb") as f:
        f.write(out)

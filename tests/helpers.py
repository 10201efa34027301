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

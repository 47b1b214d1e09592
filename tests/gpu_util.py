"""Helpers for the GPU parity tests: numpy <-> device tensors, raw device reads."""
import numpy as np
import pytest
import torch

from oracle import oracle as O


def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def dev(a: np.ndarray, bf16: bool = False):
    """numpy -> cuda tensor; uint16 arrays become bfloat16 tensors (same bits)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    if a.dtype == np.uint32:
        return torch.from_numpy(a.view(np.int32)).cuda()
    return torch.from_numpy(a).cuda()


def host(t, dtype=None) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    a = t.cpu().numpy()
    return a.view(dtype) if dtype is not None else a


def empty_bf16(*shape):
    return torch.zeros(*shape, dtype=torch.bfloat16, device="cuda")


def read_device(ptr: int, nbytes: int, dtype) -> np.ndarray:
    torch.cuda.synchronize()
    from oracle.layer_ref import read_device as rd
    return rd(ptr, nbytes, dtype)


def rand_bf16(rng, shape, sigma=1.0):
    return O.f32_to_bf16(rng.standard_normal(shape).astype(np.float32) * np.float32(sigma))


def qweights(rng, rows, K, gs, sigma=0.02):
    w = rand_bf16(rng, (rows, K), sigma)
    return O.affine_quantize(w, gs)


_hip = None


def write_device(ptr: int, a: np.ndarray):
    """Copy a host array into raw device memory (a pointer the library owns)."""
    import ctypes as C
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    a = np.ascontiguousarray(a)
    torch.cuda.synchronize()
    assert _hip.hipMemcpy(C.c_void_p(ptr), a.ctypes.data, a.nbytes, 1) == 0  # host -> device

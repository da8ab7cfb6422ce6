"""Helpers for the GPU parity tests: numpy <-> device tensors and C-ABI calls."""
import ctypes
import os

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "muon_sr_amd", "libmuon_sr_amd.so")


def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    # A GPU box without the built library is a failure, not a skip.
    assert os.path.exists(LIB_PATH), f"{LIB_PATH} not built (run __graft_entry__.build())"
    from muon_sr_amd import _lib
    return _lib.lib()


DEV = "cuda:0"


def u16_to_dev(a):
    """numpy uint16 (bf16 bits) -> device bf16 tensor."""
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16).copy())
    return t.view(torch.bfloat16).to(DEV)


def dev_to_u16(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).copy()


def np_to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a).copy()).to(DEV)


def stream():
    return torch.cuda.current_stream().cuda_stream


def ptr(t):
    return None if t is None else t.data_ptr()


def check(lib, rc, what=""):
    if rc != 0:
        raise AssertionError(f"{what} rc={rc}: {lib.msr_last_error().decode()}")


def ptr_array(ptrs, ctype=ctypes.c_void_p):
    return (ctype * len(ptrs))(*ptrs)


def rel_fro(x, ref):
    x = x.double().flatten()
    ref = ref.double().flatten()
    return (torch.linalg.norm(x - ref) / torch.linalg.norm(ref)).item()

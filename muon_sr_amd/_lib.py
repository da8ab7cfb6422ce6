"""ctypes binding of libmuon_sr_amd.so (declared in include/muon_sr_amd.h).

There is no CPU fallback: every optimizer step goes through this library, and
loading fails with an error when the library has not been built.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmuon_sr_amd.so")

NOISE_TRITON = 0
NOISE_PHILOX8 = 1
NOISE_INJECT = 2
_NOISE_NAMES = {"triton": NOISE_TRITON, "philox8": NOISE_PHILOX8}

_P = ctypes.c_void_p
_I64, _I32, _U32, _F = ctypes.c_int64, ctypes.c_int32, ctypes.c_uint32, ctypes.c_float
_SIZE_P = ctypes.POINTER(ctypes.c_size_t)


class AccumItem(ctypes.Structure):
    """msr_accum_item (include/muon_sr_amd.h)."""
    _fields_ = [("acc", ctypes.c_void_p), ("grad", ctypes.c_void_p), ("n", ctypes.c_int64),
                ("seed", ctypes.c_uint32), ("flags", ctypes.c_int32)]


ACCUM_ZERO_INIT = 1
ACCUM_GRAD_F32 = 2


class MuonGroup(ctypes.Structure):
    """msr_muon_group (include/muon_sr_amd.h)."""
    _fields_ = [("grads", ctypes.c_void_p), ("buf", ctypes.c_void_p), ("params", ctypes.c_void_p),
                ("apply_seeds", ctypes.c_void_p), ("first", ctypes.c_int64), ("batch", ctypes.c_int64),
                ("rows", ctypes.c_int64), ("cols", ctypes.c_int64), ("prepare_seed", ctypes.c_uint32),
                ("grads_f32", ctypes.c_int32), ("scale", ctypes.c_float)]

# name -> (restype, argtypes); mirrors include/muon_sr_amd.h
SIGNATURES = {
    "msr_version": (ctypes.c_int, []),
    "msr_last_error": (ctypes.c_char_p, []),
    "msr_sr_accum": (ctypes.c_int, [_P, _P, _I32, _I64, _U32, _I32, _I32, _P, _P]),
    "msr_sr_accum_multi": (ctypes.c_int, [ctypes.POINTER(AccumItem), _I32, _I32, _P]),
    "msr_adamw_bf16_step": (ctypes.c_int, [_P, _P, _P, _P, _I64, _F, _F, _F, _F, _F, _F, _F, _U32, _I32, _P, _P]),
    "msr_centralize_workspace_bytes": (ctypes.c_int, [_I64, _I64, _SIZE_P]),
    "msr_centralize_bf16": (ctypes.c_int, [_P, _P, _I64, _I64, _F, _P, ctypes.c_size_t, _P]),
    "msr_centralize_bf16_noalloc": (ctypes.c_int, [_P, _P, _I64, _I64, _F, _P]),
    "msr_adamw8bit_step": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32,
                                          _F, _F, _F, _F, _F, _F, _F, _U32, _I32, _P, _P]),
    "msr_muon_prepare": (ctypes.c_int, [_P, _I32, _P, _P, _I64, _I32, _F, _I32, _U32, _I32, _P, _P]),
    "msr_muon_apply": (ctypes.c_int, [_P, _P, _I64, _I32, _F, _F, _F, _P, _I32, _P, _P]),
    "msr_ns_workspace_bytes": (ctypes.c_int, [_I64, _I64, _I64, _SIZE_P]),
    "msr_newton_schulz": (ctypes.c_int, [_P, _P, _I64, _I64, _I64, _I32, _F, _F, _F, _P, ctypes.c_size_t, _P]),
    "msr_muon_ns_apply": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _I64, _I32, _F, _F, _F, _F, _F, _F, _I32, _P,
                                         _P, ctypes.c_size_t, _P]),
    "msr_muon_fused_step": (ctypes.c_int, [_P, _I32, _P, _I64, _I64, _I64, _I64, _F, _I32, _U32, _I32, _F, _F, _F,
                                           _P, _P, _P, _F, _F, _F, _I32, _P, _P, _P, ctypes.c_size_t, _P]),
    "msr_muon_fused_steps": (ctypes.c_int, [ctypes.POINTER(MuonGroup), _I32, _F, _I32, _I32, _F, _F, _F, _F, _F, _I32,
                                            _P, ctypes.c_size_t, _P]),
    "msr_noise_fill": (ctypes.c_int, [_P, _I64, _I64, _U32, _U32, _I32, _P]),
    "msr_stream_probe8": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _P]),
    "msr_quantize": (ctypes.c_int, [_P, _P, _I64, _P, _I32, _P, _P]),
    "msr_quant_table_bytes": (ctypes.c_size_t, []),
    "msr_quant_table_build": (ctypes.c_int, [_P, _P, _P, ctypes.c_size_t]),
    "msr_quant_table_check": (ctypes.c_int, [_P, _P, _P, _U32, _U32, _P, _I32, _P]),
    "msr_fastmath_check": (ctypes.c_int, [_I32, _U32, _U32, _P, _I32, _P]),
    "msr_gemm_nt": (ctypes.c_int, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                   _I64, _I64, _I64, _I64, _F, _F, _F, _P]),
    "msr_gemm_nn": (ctypes.c_int, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                   _I64, _I64, _I64, _I64, _F, _F, _F, _P]),
    "msr_linear_wgrad_sr_accum": (ctypes.c_int, [_P, _P, _I64, _P, _I64, _I64, _I64, _I64, _U32, _I32, _I32, _P, _P]),
}

_lib = None
_lock = threading.Lock()


class MuonSRLibraryError(RuntimeError):
    pass


def lib():
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise MuonSRLibraryError(
                        f"{LIB_PATH} is missing: build it with `python -m muon_sr_amd._build` "
                        "(muon_sr_amd has no CPU fallback)")
                L = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(L, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().msr_last_error()
        raise MuonSRLibraryError(f"{what} failed with code {rc}: {msg.decode() if msg else ''}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor):
    """The current HIP stream of t's device, as the raw handle the library takes.
    torch's raw-stream query returns the same handle as current_stream().cuda_stream
    in a twentieth of the host time (it builds no Stream object), which matters on
    the per-hook accumulation path."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr_array(ptrs, ctype=ctypes.c_void_p):
    arr = (ctype * len(ptrs))(*ptrs)
    return arr


# ---------------------------------------------------------------------------
# Stochastic-rounding noise source
# ---------------------------------------------------------------------------

_noise_mode = _NOISE_NAMES.get(os.environ.get("MUON_SR_AMD_NOISE", "philox8").lower(), NOISE_PHILOX8)


def set_sr_noise(mode: str) -> None:
    """Select the stochastic-rounding noise stream used by every optimizer.

    ``"philox8"`` (default): one Philox4x32-10 call per 8 consecutive elements.
    ``"triton"``: word 0 of Philox4x32-10 per element, keyed exactly like the
    reference's ``tl.randint(seed, offset)``, i.e. the reference's noise bits.
    Both are counter-based: the noise is a pure function of (seed, offset), so
    every data-parallel replica applies the same rounding.
    """
    global _noise_mode
    if mode not in _NOISE_NAMES:
        raise ValueError(f"unknown SR noise mode {mode!r}; choose from {sorted(_NOISE_NAMES)}")
    _noise_mode = _NOISE_NAMES[mode]


def get_sr_noise() -> str:
    return {v: k for k, v in _NOISE_NAMES.items()}[_noise_mode]


def noise_mode() -> int:
    return _noise_mode


def require_gpu(t: torch.Tensor, what: str, exc=ValueError) -> None:
    if not t.is_cuda:
        raise exc(f"{what} requires tensors on a ROCm GPU (got device {t.device})")

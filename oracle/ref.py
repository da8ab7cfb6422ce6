"""ctypes bindings to ``oracle.c`` plus numpy/torch restatements.

Test infrastructure only (see the package docstring).  Arrays are numpy; bf16
values travel as ``np.uint16`` bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle.so")

NOISE_TRITON = 0
NOISE_PHILOX8 = 1
NOISE_INJECT = 2

__all__ = [
    "NOISE_TRITON", "NOISE_PHILOX8", "NOISE_INJECT",
    "build", "lib", "philox", "seed_key", "noise16",
    "bf16_to_f32", "f32_to_bf16_rne", "f32_to_bf16_trunc",
    "create_dynamic_map", "quantize", "deterministic_seed",
    "sr_accum", "adamw_bf16", "adamw8bit", "muon_prepare", "muon_apply",
    "adamw_bias_corrections", "ns_fp32", "ns_bf16_torch", "ns_scalar_map", "NS_COEFFS", "NoiseSpec",
    "NS_CHUNK_NUMEL", "ns_scale", "muon_batch_step", "muon_param_step",
]


def build() -> str:
    """Compile ``liboracle.so`` with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


_lib = None


class _Noise(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int32), ("key_lo", ctypes.c_uint32),
                ("key_hi", ctypes.c_uint32), ("inject", ctypes.c_void_p)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        P = ctypes.c_void_p
        I64, I32, U32, F = ctypes.c_int64, ctypes.c_int32, ctypes.c_uint32, ctypes.c_float
        NP = ctypes.POINTER(_Noise)
        L.orc_philox4x32_10.argtypes = [P, P, P]
        L.orc_seed_key.argtypes = [U32, U32, P]
        L.orc_noise16_batch.argtypes = [NP, P, I64, P]
        L.orc_bf16_rne_batch.argtypes = [P, I64, P]
        L.orc_quantize.argtypes = [P, I64, P, I32, P]
        L.orc_sr_accum.argtypes = [P, P, I32, I64, NP]
        L.orc_adamw_bf16.argtypes = [P, P, P, P, I64, F, F, F, F, F, F, F, NP, NP, NP]
        L.orc_adamw8bit.argtypes = [P, P, P, P, P, P, P, P, P, P, I64, I32, I32,
                                    F, F, F, F, F, F, F, NP, NP, NP]
        L.orc_muon_prepare.argtypes = [P, I32, P, P, P, I64, F, I32, NP]
        L.orc_muon_apply.argtypes = [P, P, I64, F, F, F, NP]
        L.orc_num_threads.restype = I32
        L.orc_num_threads.argtypes = []
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------------------
# RNG
# ---------------------------------------------------------------------------

def philox(ctr, key):
    """Philox4x32-10 of a 4-word counter and 2-word key (triton/language/random.py:12-41)."""
    c = np.asarray(ctr, dtype=np.uint32).copy()
    k = np.asarray(key, dtype=np.uint32).copy()
    out = np.zeros(4, dtype=np.uint32)
    lib().orc_philox4x32_10(_ptr(c), _ptr(k), _ptr(out))
    return out


def seed_key(seed: int, k: int = 0):
    """Philox key words of Triton's ``SEED + k`` stream (i32/u32 typing of the seed)."""
    key = np.zeros(2, dtype=np.uint32)
    lib().orc_seed_key(seed & 0xFFFFFFFF, k & 0xFFFFFFFF, _ptr(key))
    return int(key[0]), int(key[1])


class NoiseSpec:
    """One SR stream: mode plus the seed (and salt k for ``SEED + k``) or injected noise."""

    def __init__(self, mode: int, seed: int = 0, k: int = 0, inject=None):
        self.mode = mode
        self.inject = None if inject is None else np.ascontiguousarray(inject, dtype=np.uint16)
        lo, hi = seed_key(seed, k)
        self.struct = _Noise(mode, lo, hi, None if self.inject is None else self.inject.ctypes.data)

    def ref(self):
        return ctypes.byref(self.struct)


def noise16(mode: int, seed: int, offsets, k: int = 0):
    offs = np.ascontiguousarray(offsets, dtype=np.int64)
    out = np.zeros(offs.shape, dtype=np.uint16)
    ns = NoiseSpec(mode, seed, k)
    lib().orc_noise16_batch(ns.ref(), _ptr(offs), offs.size, _ptr(out))
    return out


# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------

def bf16_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_rne(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.shape, dtype=np.uint16)
    lib().orc_bf16_rne_batch(_ptr(x), x.size, _ptr(out))
    return out


def f32_to_bf16_trunc(x):
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


# ---------------------------------------------------------------------------
# Codebook, quantizer, seeds
# ---------------------------------------------------------------------------

def create_dynamic_map(signed: bool = True) -> np.ndarray:
    """bitsandbytes dynamic (signed) / unsigned-dynamic 256-entry codebook.

    Restates muon_sr/triton_adamw_8bit.py:14-24: for each decade i=0..6, the
    midpoints of ``torch.linspace(0.1, 1, 2**i + 1)`` (signed) or
    ``2**(i+1) + 1`` points (unsigned) in fp32, scaled by 10**(i-6) in fp32,
    mirrored for the signed map, plus 0 and 1, sorted.  ``torch.linspace`` is
    the library routine the reference calls, so it is called here as well.
    """
    import torch
    vals = []
    for i in range(7):
        pts = torch.linspace(0.1, 1, 2 ** (i if signed else i + 1) + 1, dtype=torch.float32)
        mids = (pts[:-1] + pts[1:]) / 2
        scale = 10 ** (-6 + i)
        vals.extend((scale * mids).tolist())
        if signed:
            vals.extend((-scale * mids).tolist())
    return np.array(sorted(vals + [0.0, 1.0]), dtype=np.float32)


def quantize(x, Q, signed: bool) -> np.ndarray:
    """Reference quantizer search (muon_sr/triton_adamw_8bit.py:27-53)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    Q = np.ascontiguousarray(Q, dtype=np.float32)
    out = np.zeros(x.shape, dtype=np.uint8)
    lib().orc_quantize(_ptr(x), x.size, _ptr(Q), int(bool(signed)), _ptr(out))
    return out


def deterministic_seed(step: int, param_idx: int, salt: int = 0) -> int:
    """muon_sr/triton_muon_sr.py:83-85 and muon_sr/triton_adamw.py:97."""
    return (step * 2654435761 ^ param_idx * 1234567891 ^ salt) & 0xFFFFFFFF


def adamw_bias_corrections(beta1: float, beta2: float, step: int):
    """Python-double bias corrections of muon_sr/triton_adamw.py:88-89."""
    return 1.0 - beta1 ** step, (1.0 - beta2 ** step) ** 0.5


# ---------------------------------------------------------------------------
# Kernels (all return new arrays; inputs are not modified)
# ---------------------------------------------------------------------------

def _f(x):
    return float(np.float32(x))


def sr_accum(acc, grad, noise: NoiseSpec):
    acc = np.array(acc, dtype=np.uint16, copy=True)
    g = np.ascontiguousarray(grad)
    is_f32 = int(g.dtype == np.float32)
    if not is_f32:
        g = g.astype(np.uint16, copy=False)
    lib().orc_sr_accum(_ptr(acc), _ptr(g), is_f32, acc.size, noise.ref())
    return acc


def adamw_bf16(p, g, ema, ema_sq, lr, beta1, beta2, eps, weight_decay, bc, bc_sqrt,
               n_ema: NoiseSpec, n_ema_sq: NoiseSpec, n_p: NoiseSpec):
    p = np.array(p, dtype=np.uint16, copy=True)
    ema = np.array(ema, dtype=np.uint16, copy=True)
    ema_sq = np.array(ema_sq, dtype=np.uint16, copy=True)
    g = np.ascontiguousarray(g, dtype=np.uint16)
    lib().orc_adamw_bf16(_ptr(p), _ptr(g), _ptr(ema), _ptr(ema_sq), p.size,
                         _f(lr), _f(beta1), _f(beta2), _f(eps), _f(weight_decay), _f(bc), _f(bc_sqrt),
                         n_ema.ref(), n_ema_sq.ref(), n_p.ref())
    return p, ema, ema_sq


def adamw8bit(p, g, state1, state2, absmax1, absmax2, q1, q2, block, quantized,
              lr, b1, b2, eps, wd, bc1, bc2, n_p: NoiseSpec, n_m: NoiseSpec = None, n_v: NoiseSpec = None):
    """One step of muon_sr/triton_adamw_8bit.py:56-99 on one flat parameter."""
    p = np.array(p, dtype=np.uint16, copy=True)
    g = np.ascontiguousarray(g, dtype=np.uint16)
    n = p.size
    dummy = NoiseSpec(NOISE_TRITON, 0)
    if quantized:
        s1 = np.array(state1, dtype=np.uint8, copy=True)
        s2 = np.array(state2, dtype=np.uint8, copy=True)
        a1 = np.array(absmax1, dtype=np.float32, copy=True)
        a2 = np.array(absmax2, dtype=np.float32, copy=True)
        lib().orc_adamw8bit(_ptr(p), _ptr(g), _ptr(s1), _ptr(s2), _ptr(a1), _ptr(a2),
                            _ptr(np.ascontiguousarray(q1, np.float32)), _ptr(np.ascontiguousarray(q2, np.float32)),
                            None, None, n, int(block), 1,
                            _f(lr), _f(b1), _f(b2), _f(eps), _f(wd), _f(bc1), _f(bc2),
                            n_p.ref(), dummy.ref(), dummy.ref())
        return p, s1, s2, a1, a2
    s1 = np.array(state1, dtype=np.uint16, copy=True)
    s2 = np.array(state2, dtype=np.uint16, copy=True)
    lib().orc_adamw8bit(_ptr(p), _ptr(g), None, None, None, None, None, None,
                        _ptr(s1), _ptr(s2), n, int(block), 0,
                        _f(lr), _f(b1), _f(b2), _f(eps), _f(wd), _f(bc1), _f(bc2),
                        n_p.ref(), n_m.ref(), n_v.ref())
    return p, s1, s2


def muon_prepare(g, buf, beta, nesterov, noise: NoiseSpec):
    """Returns (new_buf_bf16, update_f32, update_bf16_rne).  ``g``: bf16 bits (uint16) or
    float32 (read as fp32, as the reference's kernel reads an fp32 gradient)."""
    f32 = np.asarray(g).dtype == np.float32
    g = np.ascontiguousarray(g, dtype=np.float32 if f32 else np.uint16)
    buf = np.array(buf, dtype=np.uint16, copy=True)
    out32 = np.zeros(buf.shape, dtype=np.float32)
    out16 = np.zeros(buf.shape, dtype=np.uint16)
    lib().orc_muon_prepare(_ptr(g), int(f32), _ptr(buf), _ptr(out32), _ptr(out16), buf.size,
                           _f(beta), int(bool(nesterov)), noise.ref())
    return buf, out32, out16


def muon_apply(p, upd, lr, weight_decay, scale, noise: NoiseSpec):
    p = np.array(p, dtype=np.uint16, copy=True)
    upd = np.ascontiguousarray(upd, dtype=np.uint16)
    lib().orc_muon_apply(_ptr(p), _ptr(upd), p.size, _f(lr), _f(weight_decay), _f(scale), noise.ref())
    return p


# ---------------------------------------------------------------------------
# Muon step composition (seeds, stacking, chunking, scale)
# ---------------------------------------------------------------------------

NS_CHUNK_NUMEL = 1 << 28


def ns_scale(shape) -> float:
    """muon_sr/triton_muon_sr.py:101-102."""
    return max(1.0, shape[-2] / shape[-1]) ** 0.5


def _pre_ns(u32, u16, rounding):
    # rounding "rne": the compiled kernel's fp32->bf16 store; "trunc": what the
    # Triton interpreter (which wrote the golden trajectories) stores instead
    return u16 if rounding == "rne" else f32_to_bf16_trunc(u32)


def muon_batch_step(params, grads, bufs, step, lr, weight_decay, beta, nesterov, ns, mode, rounding="rne"):
    """One batch_ns Muon step with every gradient present (muon_sr/triton_muon_sr.py:123-168).

    params, grads: lists of uint16 (bf16 bits) arrays shaped like the parameters,
    in parameter-group order; bufs: dict shape -> uint16 momentum stack
    [count, *shape], rows in first-occurrence order (muon_sr/muon_sr.py:112-146);
    ns: callable mapping a uint16 stack [k, *shape] to its Newton-Schulz output.
    Shape groups are visited in first-occurrence order (shape_idx); prepare runs
    over the whole stack with seed (step, shape_idx, salt 0); NS runs per chunk
    of at most NS_CHUNK_NUMEL elements; apply runs per matrix with seed
    (step, shape_idx * 10000 + i, salt 1).  Returns (new params, new bufs).
    """
    groups = {}
    for i, p in enumerate(params):
        groups.setdefault(tuple(p.shape), []).append(i)
    new_p = [np.array(p, copy=True) for p in params]
    new_b = {}
    for shape_idx, (shape, idxs) in enumerate(groups.items()):
        g = np.concatenate([np.ascontiguousarray(grads[i]).ravel() for i in idxs])
        buf, u32, u16 = muon_prepare(g, np.ascontiguousarray(bufs[shape]).ravel(), beta, nesterov,
                                     NoiseSpec(mode, deterministic_seed(step, shape_idx, 0)))
        new_b[shape] = buf.reshape(len(idxs), *shape)
        work = _pre_ns(u32, u16, rounding).reshape(len(idxs), *shape)
        numel = int(np.prod(shape))
        k = max(1, NS_CHUNK_NUMEL // numel)
        for start in range(0, len(idxs), k):
            X = ns(work[start:start + k])
            for j in range(X.shape[0]):
                i = start + j
                seed = deterministic_seed(step, shape_idx * 10000 + i, 1)
                new_p[idxs[i]] = muon_apply(params[idxs[i]].ravel(), X[j].ravel(), lr, weight_decay, ns_scale(shape),
                                            NoiseSpec(mode, seed)).reshape(shape)
    return new_p, new_b


def muon_param_step(p, g, buf, step, param_idx, lr, weight_decay, beta, nesterov, ns, mode, rounding="rne"):
    """One per-parameter Muon step (muon_sr/triton_muon_sr.py:88-120): prepare with
    seed (step, param_idx, salt 0), NS, apply with seed (step, param_idx, salt 1).
    Returns (new p, new buf)."""
    shape = p.shape
    nbuf, u32, u16 = muon_prepare(np.ascontiguousarray(g).ravel(), np.ascontiguousarray(buf).ravel(), beta, nesterov,
                                  NoiseSpec(mode, deterministic_seed(step, param_idx, 0)))
    X = ns(_pre_ns(u32, u16, rounding).reshape(shape))
    newp = muon_apply(p.ravel(), np.ascontiguousarray(X).ravel(), lr, weight_decay, ns_scale(shape),
                      NoiseSpec(mode, deterministic_seed(step, param_idx, 1)))
    return newp.reshape(shape), nbuf.reshape(shape)


# ---------------------------------------------------------------------------
# Newton-Schulz
# ---------------------------------------------------------------------------

NS_COEFFS = (3.4445, -4.7750, 2.0315)


def ns_fp32(G, steps: int = 5, dtype=None):
    """fp32 restatement of muon_sr/muon_sr.py:82-98 (same iteration, fp32 throughout).

    ``G`` is a torch tensor ``[..., rows, cols]``; returns fp32 (or ``dtype``, e.g.
    float64 for large matrices on a GPU) of the same shape.
    """
    import torch
    a, b, c = NS_COEFFS
    X = G.to(torch.float32 if dtype is None else dtype)
    transposed = X.size(-2) > X.size(-1)
    if transposed:
        X = X.mT
    X = X / (X.norm(dim=(-2, -1), keepdim=True) + 1e-7)
    for _ in range(steps):
        A = X @ X.mT
        B = b * A + c * (A @ A)
        X = a * X + B @ X
    if transposed:
        X = X.mT
    return X.contiguous()


def ns_bf16_torch(G, steps: int = 5):
    """The reference's bf16 op sequence (muon_sr/muon_sr.py:82-98) on CPU torch."""
    import torch
    a, b, c = NS_COEFFS
    X = G.to(torch.bfloat16)
    transposed = X.size(-2) > X.size(-1)
    if transposed:
        X = X.mT.contiguous()   # (a transposed bf16 right operand of a batched product is avoided on GPUs)
    X = X / (X.norm(dim=(-2, -1), keepdim=True) + 1e-7)
    for _ in range(steps):
        A = X @ X.mT.contiguous()
        B = b * A + c * (A @ A)
        X = a * X + B @ X
    if transposed:
        X = X.mT
    return X.contiguous()


def ns_scalar_map(sigma, steps: int = 5):
    """Closed form of NS on singular values: with G = U diag(s) V^T, the iteration
    maps s/||s||_2 through x -> a x + b x^3 + c x^5 ``steps`` times (float64)."""
    a, b, c = NS_COEFFS
    x = np.asarray(sigma, dtype=np.float64)
    x = x / (np.sqrt(np.sum(x * x)) + 1e-7)
    for _ in range(steps):
        x = a * x + b * x ** 3 + c * x ** 5
    return x

"""Gradient centralization of TritonAdamW on the device (muon_sr/triton_adamw.py:179-187).

The reference computes g' = bf16(g32 - g32.mean(dims 1..) * c) with torch ops.
The fused kernel's fp32 row sums have their own (fixed) order, so g' is held to
within 1 bf16 ulp of both the reference's op sequence (torch fp32 on the CPU)
and a float64 evaluation, and equal to them for at least 99.9% of elements.
The AdamW step that consumes g' is bit-exact against the oracle.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from _gpu import DEV, check, dev_to_u16, need_gpu, stream

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return need_gpu()


def ulps(a, b):
    a = a.astype(np.int64)
    b = b.astype(np.int64)
    sa = np.where(a & 0x8000, -(a & 0x7fff), a & 0x7fff)
    sb = np.where(b & 0x8000, -(b & 0x7fff), b & 0x7fff)
    return np.abs(sa - sb)


def reference_ops(g_bf16_cpu, c):
    """The reference's op sequence (muon_sr/triton_adamw.py:180-186) on CPU torch."""
    g = g_bf16_cpu.to(torch.float32)
    g.sub_(g.mean(dim=tuple(range(1, g.dim())), keepdim=True).mul_(c))
    return g.to(torch.bfloat16)


def fp64_centralized(g_bf16_cpu, c):
    g = g_bf16_cpu.double()
    rows = g.shape[0] if g.dim() >= 2 else 1
    g2 = g.reshape(rows, -1)
    out = g2 - g2.mean(dim=1, keepdim=True) * c
    return out.reshape(g.shape).float().to(torch.bfloat16)


@pytest.mark.parametrize("shape", [(64, 300), (3, 40000), (4096,), (33, 16, 5), (1,), (7, 8), (2, 16384)])
@pytest.mark.parametrize("c", [1.0, 0.37])
def test_centralize_matches_reference_ops(L, shape, c):
    from muon_sr_amd.adamw import centralize
    gen = torch.Generator().manual_seed(sum(shape) + int(c * 100))
    g = torch.randn(shape, generator=gen) * 1e-3
    g = g + torch.randn(shape[:1] + (1,) * (len(shape) - 1), generator=gen) * 5e-4   # non-zero row means
    g = g.to(torch.bfloat16)
    out = dev_to_u16(centralize(g.to(DEV), c)).reshape(-1)
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)  # noqa: E731
    for ref in (bits(reference_ops(g, c)), bits(fp64_centralized(g, c))):
        d = ulps(out, ref)
        assert d.max() <= 1, (shape, int(d.max()))
        assert (d == 0).mean() >= 0.999, (shape, float((d == 0).mean()))


def test_centralize_in_place_and_deterministic(L):
    g = (torch.randn(17, 20000, device=DEV) * 1e-3).to(torch.bfloat16)
    nbytes = ctypes.c_size_t()
    check(L, L.msr_centralize_workspace_bytes(17, 20000, ctypes.byref(nbytes)))
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=DEV)
    outs = []
    for _ in range(2):
        o = torch.empty_like(g)
        check(L, L.msr_centralize_bf16(g.data_ptr(), o.data_ptr(), 17, 20000, 0.5, ws.data_ptr(), ws.numel(), stream()))
        outs.append(dev_to_u16(o))
    h = g.clone()
    check(L, L.msr_centralize_bf16(h.data_ptr(), h.data_ptr(), 17, 20000, 0.5, ws.data_ptr(), ws.numel(), stream()))
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[0], dev_to_u16(h))
    # a workspace that is too small is refused
    assert L.msr_centralize_bf16(g.data_ptr(), h.data_ptr(), 17, 20000, 0.5, ws.data_ptr(), 8, stream()) != 0


def test_triton_adamw_centralization_step(L):
    """TritonAdamW(centralization=c): the step consumes the centralized gradient
    exactly as the oracle's AdamW does (reference noise stream, bit-exact)."""
    import muon_sr_amd
    from muon_sr_amd import TritonAdamW
    from muon_sr_amd.adamw import centralize
    old = muon_sr_amd.get_sr_noise()
    muon_sr_amd.set_sr_noise("triton")
    try:
        gen = torch.Generator().manual_seed(5)
        shapes = [(48, 40), (40,)]
        ps = [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.02).to(torch.bfloat16).to(DEV)) for s in shapes]
        opt = TritonAdamW(ps, lr=1e-3, betas=(0.9, 0.99), eps=1e-8, weight_decay=0.01, centralization=0.5)
        ema = [np.zeros(p.numel(), np.uint16) for p in ps]
        ema_sq = [np.zeros(p.numel(), np.uint16) for p in ps]
        pn = [dev_to_u16(p).reshape(-1) for p in ps]
        for step in (1, 2):
            grads = [(torch.randn(s, generator=gen) * 1e-3 + 2e-4).to(torch.bfloat16).to(DEV) for s in shapes]
            gc = [dev_to_u16(centralize(g, 0.5)).reshape(-1) for g in grads]
            for p, g in zip(ps, grads):
                p.grad = g
            opt.step()
            bc, bcs = O.adamw_bias_corrections(0.9, 0.99, step)
            for i, p in enumerate(ps):
                seed = O.deterministic_seed(step, i)
                pn[i], ema[i], ema_sq[i] = O.adamw_bf16(
                    pn[i], gc[i], ema[i], ema_sq[i], 1e-3, 0.9, 0.99, 1e-8, 0.01, bc, bcs,
                    O.NoiseSpec(O.NOISE_TRITON, seed, 0), O.NoiseSpec(O.NOISE_TRITON, seed, 1),
                    O.NoiseSpec(O.NOISE_TRITON, seed, 2))
                assert np.array_equal(dev_to_u16(p).reshape(-1), pn[i]), (step, i)
                assert np.array_equal(dev_to_u16(opt.state[p]["ema"]).reshape(-1), ema[i]), (step, i)
                assert np.array_equal(dev_to_u16(opt.state[p]["ema_squared"]).reshape(-1), ema_sq[i]), (step, i)
    finally:
        muon_sr_amd.set_sr_noise(old)

"""SR accumulation fused with the weight-gradient GEMM (msr_linear_wgrad_sr_accum, SRLinear).

The fused kernel must equal, bit for bit, the library's unfused path on the
same inputs: the bf16 weight gradient from the diagnostic GEMM (same
accumulation order), then msr_sr_accum with the same seed and noise mode
(the reference's _grad_accum_kernel, muon_sr/triton_adamw.py:206-229, as
pinned in test_gpu_kernels.py).  The GEMM part is held to torch fp32
products, and SRLinear to nn.Linear with TritonSRAccumulator hooks.
"""
import random

import pytest
import torch

import oracle as O
from _gpu import DEV, check, need_gpu, stream

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return need_gpu()


def _inputs(T, fin, fout, seed, pad=0):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    x = (torch.randn(T, fin + pad, device=DEV, generator=gen)).to(torch.bfloat16)
    dy = (torch.randn(T, fout + pad, device=DEV, generator=gen) * 1e-2).to(torch.bfloat16)
    acc = (torch.randn(fout, fin, device=DEV, generator=gen) * 0.1).to(torch.bfloat16)
    return x, dy, acc


def _gemm_dw(L, x, dy, T, fin, fout):
    """bf16 dW = dy^T x through the diagnostic NT GEMM on transposed copies."""
    P = dy[:, :fout].t().contiguous()
    Q = x[:, :fin].t().contiguous()
    dw = torch.empty(fout, fin, device=DEV, dtype=torch.bfloat16)
    check(L, L.msr_gemm_nt(P.data_ptr(), T, fout * T, Q.data_ptr(), T, fin * T, None, fin, fout * fin, dw.data_ptr(),
                           fin, fout * fin, fout, fin, T, 1, 1.0, 0.0, 0.0, stream()), "gemm")
    return dw


@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8, O.NOISE_INJECT])
@pytest.mark.parametrize("zero_init", [0, 1])
def test_fused_equals_gemm_then_accumulate(L, mode, zero_init):
    T, fin, fout, pad = 384, 512, 768, 8
    x, dy, acc = _inputs(T, fin, fout, 3 + mode + 7 * zero_init, pad)
    inj = torch.randint(0, 1 << 16, (fout * fin,), device=DEV, dtype=torch.int32).to(torch.int16)
    inj_p = inj.data_ptr() if mode == O.NOISE_INJECT else None
    seed = 0x9E3779B1 + mode
    a1 = acc.clone()
    check(L, L.msr_linear_wgrad_sr_accum(a1.data_ptr(), x.data_ptr(), fin + pad, dy.data_ptr(), fout + pad, T, fin,
                                         fout, seed, zero_init, mode, inj_p, stream()), "fused")
    dw = _gemm_dw(L, x, dy, T, fin, fout)
    a2 = acc.clone()
    check(L, L.msr_sr_accum(a2.data_ptr(), dw.data_ptr(), 0, fout * fin, seed, zero_init, mode, inj_p, stream()),
          "sr_accum")
    assert torch.equal(a1, a2)


def test_fused_wgrad_vs_torch_fp32(L):
    """From a zero buffer with zero noise the result is bf16(dW) itself."""
    T, fin, fout = 512, 768, 256
    x, dy, _ = _inputs(T, fin, fout, 11)
    acc = torch.empty(fout, fin, device=DEV, dtype=torch.bfloat16)
    inj = torch.zeros(fout * fin, device=DEV, dtype=torch.int16)
    check(L, L.msr_linear_wgrad_sr_accum(acc.data_ptr(), x.data_ptr(), fin, dy.data_ptr(), fout, T, fin, fout, 1, 1,
                                         O.NOISE_INJECT, inj.data_ptr(), stream()), "fused")
    ref = dy.float().t() @ x.float()
    err = (acc.float() - ref).abs()
    tol = 2.0 ** -8 * ref.abs() + 1e-5 * ref.abs().max()
    assert bool((err <= tol).all()), float((err - tol).max())


def test_fused_rejects_what_it_cannot_take(L):
    a = torch.zeros(256, 256, device=DEV, dtype=torch.bfloat16)
    x = torch.zeros(256, 256, device=DEV, dtype=torch.bfloat16)
    assert L.msr_linear_wgrad_sr_accum(a.data_ptr(), x.data_ptr(), 256, x.data_ptr(), 256, 100, 256, 256, 0, 0,
                                       O.NOISE_TRITON, None, stream()) == 1001          # tokens % 128
    assert L.msr_linear_wgrad_sr_accum(a.data_ptr(), a.data_ptr(), 256, x.data_ptr(), 256, 256, 256, 256, 0, 0,
                                       O.NOISE_TRITON, None, stream()) == 1005          # acc is x


def _model(cls, fin, fout, seed):
    torch.manual_seed(seed)
    m = cls(fin, fout, bias=True).to(DEV).to(torch.bfloat16)
    return m


@pytest.mark.parametrize("fin,fout,T", [(512, 768, 384), (300, 256, 128)])
def test_sr_linear_matches_hook_accumulation(L, fin, fout, T):
    """SRLinear + hooks against nn.Linear + hooks over two micro-batches (reference
    noise stream, same seeds).  The weight gradients come from different GEMMs
    (torch's and this library's), so the accumulators agree to a bf16 step per
    micro-batch; SRLinear leaves weight.grad unset.  (300 features take the
    unfused fallback.)"""
    import muon_sr_amd
    from muon_sr_amd import SRLinear, TritonSRAccumulator
    old = muon_sr_amd.get_sr_noise()
    muon_sr_amd.set_sr_noise("triton")
    try:
        ref, fused = _model(torch.nn.Linear, fin, fout, 5), _model(SRLinear, fin, fout, 5)
        assert torch.equal(ref.weight, fused.weight)
        h = TritonSRAccumulator.assign_hooks(ref) + TritonSRAccumulator.assign_hooks(fused)
        gen = torch.Generator(device=DEV)
        gen.manual_seed(17)
        for mb in range(2):
            x = torch.randn(2, T // 2, fin, device=DEV, generator=gen).to(torch.bfloat16)
            w = torch.randn(2, T // 2, fout, device=DEV, generator=gen).to(torch.bfloat16)
            outs = []
            for m in (ref, fused):
                xi = x.clone().requires_grad_(True)
                random.seed(100 + mb)
                (m(xi).float() * w.float()).sum().backward()
                outs.append(xi.grad)
            torch.testing.assert_close(outs[0].float(), outs[1].float(), rtol=2 ** -7, atol=1e-6)
            assert fused.weight.grad is None
        for h_ in h:
            h_.remove()
        a_ref, a_fused = ref.weight.acc_grad.float(), fused.weight.acc_grad.float()
        d = (a_ref - a_fused).abs()   # at most one bf16 step per micro-batch
        assert bool((d <= 2.0 ** -6 * a_ref.abs() + 1e-6).all()), float(d.max())
        torch.testing.assert_close(ref.bias.acc_grad.float(), fused.bias.acc_grad.float(), rtol=2 ** -6, atol=1e-6)
    finally:
        muon_sr_amd.set_sr_noise(old)


def test_sr_linear_edge_cases(L):
    """No bias, an input without grad, a non-contiguous 3-D input, and an fp32 layer
    (which returns dW to autograd, so the hook or .grad sees it as for nn.Linear)."""
    from muon_sr_amd import SRLinear, TritonSRAccumulator
    torch.manual_seed(3)
    m = SRLinear(256, 512, bias=False).to(DEV).to(torch.bfloat16)
    h = TritonSRAccumulator.assign_hooks(m)
    x = torch.randn(256, 4, 256, device=DEV).to(torch.bfloat16).transpose(0, 1)   # [4, 256, 256], non-contiguous
    m(x).float().sum().backward()
    assert m.weight.grad is None and m.weight.acc_grad.shape == (512, 256)
    dy = torch.ones(4 * 256, 512, device=DEV, dtype=torch.bfloat16)
    ref = (dy.float().t() @ x.reshape(-1, 256).float())
    torch.testing.assert_close(m.weight.acc_grad.float(), ref, rtol=2 ** -7, atol=1e-3)
    for h_ in h:
        h_.remove()
    f = SRLinear(256, 256).to(DEV)                       # fp32: unfused, dW returned to autograd
    xf = torch.randn(128, 256, device=DEV, requires_grad=True)
    f(xf).sum().backward()
    assert f.weight.grad is not None and not hasattr(f.weight, "acc_grad")
    torch.testing.assert_close(f.weight.grad, torch.ones(128, 256, device=DEV).t() @ xf.detach(), rtol=1e-5, atol=1e-4)
    assert xf.grad is not None and f.bias.grad is not None


def test_sr_linear_falls_back_on_unaddressable_operands(L):
    """A misaligned activation view fails the fused kernel's 16-byte alignment: the
    predicate sends it to the unfused path (dW returned to autograd) instead of letting
    msr_linear_wgrad_sr_accum raise inside backward."""
    from muon_sr_amd import SRLinear
    from muon_sr_amd.linear import linear_wgrad_sr_accum
    w = torch.zeros(256, 256, device=DEV, dtype=torch.bfloat16)
    buf = torch.randn(128 * 256 + 1, device=DEV).to(torch.bfloat16)
    x2 = buf[1:].view(128, 256)                      # 2-byte misaligned
    dy2 = torch.randn(128, 256, device=DEV).to(torch.bfloat16)
    assert not linear_wgrad_sr_accum(w, x2, dy2) and not hasattr(w, "acc_grad")
    m = SRLinear(256, 256, bias=False).to(DEV).to(torch.bfloat16)
    x = buf[1:].view(128, 256).requires_grad_(False)
    m(x).float().sum().backward()
    assert m.weight.grad is not None and not hasattr(m.weight, "acc_grad")
    torch.testing.assert_close(m.weight.grad.float(), torch.ones(256, 128, device=DEV) @ x.float(), rtol=2 ** -7,
                               atol=1e-3)

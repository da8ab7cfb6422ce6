"""BASELINE.json's configs 1 and 3 run through the HIP path at their own workloads,
against the C oracle, and the momentum noise offsets of config 5's largest stacks.

* Config 1: TritonMuonSRWithAuxAdam on 4 x 256^2 Muon matrices plus AdamW on
  2 x 256 and 512 x 256, 10 steps, with batch_ns on and off
  (muon_sr/triton_muon_sr.py:258-373).  The oracle composes the reference's
  kernels, seeds and stacking (it reproduces the reference's own trajectories
  bit for bit on the CPU); this library's Newton-Schulz output is substituted
  into it, so every parameter, momentum and AdamW moment must be bit-exact.
* Config 3: TritonSRAccumulator over the 217 tensors of a 24-layer d=2048,
  ffn=5632 transformer (1,298,759,680 elements), 3 micro-batches in the
  reference's noise stream, one launch per hook (the reference's behaviour,
  muon_sr/triton_adamw.py:252-265) and queued, against orc_sr_accum.
* Noise offsets: the reference numbers a momentum stack's noise by the element
  offset cut to int32 (muon_sr/triton_muon_sr.py:44); config 5's 64-matrix
  gate/up stack (3.76e9 elements) starts chunks at 2.1e9 and 3.2e9.  The fused
  step's `first` moves only that counter, so small matrices reach it.
"""
import ctypes
import random

import numpy as np
import pytest
import torch

import oracle as O
from _gpu import DEV, check, dev_to_u16, need_gpu, ptr_array, stream, u16_to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return need_gpu()


@pytest.fixture
def noise():
    import muon_sr_amd
    old = muon_sr_amd.get_sr_noise()
    yield muon_sr_amd.set_sr_noise
    muon_sr_amd.set_sr_noise(old)


def _gpu_ns(U):
    from muon_sr_amd.muon import newton_schulz
    return dev_to_u16(newton_schulz(u16_to_dev(U.ravel()).view(U.shape))).reshape(U.shape)


# ---------------------------------------------------------------------------
# Config 1
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("batch_ns", [True, False])
@pytest.mark.parametrize("mode_name", ["triton", "philox8"])
def test_config1_hybrid_vs_oracle(L, noise, batch_ns, mode_name):
    """Config 1's parameter set and schedule (Muon lr 0.02, momentum 0.95, nesterov,
    5 NS steps, wd 0.01; AdamW lr 3e-4, betas 0.9/0.95, eps 1e-10, wd 0.01; params
    ~N(0, 0.02), grads ~N(0, 1e-3) per step), 10 steps of TritonMuonSRWithAuxAdam.
    batch_ns: one stacked momentum per shape, the global step, seeds of shape group 0
    (muon_sr/triton_muon_sr.py:128-177, 315-337).  Without: per-parameter steps with
    index i in the group (:338-350).  AdamW: seed index group offset + i (:351-371)."""
    from muon_sr_amd import TritonMuonSRWithAuxAdam
    noise(mode_name)
    mode = O.NOISE_TRITON if mode_name == "triton" else O.NOISE_PHILOX8
    gen = torch.Generator().manual_seed(1)

    def bf(shape, std):
        return (torch.randn(shape, generator=gen) * std).to(torch.bfloat16)

    shapes = [(256, 256)] * 4 + [(256,), (256,), (512, 256)]
    p0 = [bf(s, 0.02) for s in shapes]
    ps = [torch.nn.Parameter(x.to(DEV)) for x in p0]
    lr, wd, beta, alr, betas, eps, awd = 0.02, 0.01, 0.95, 3e-4, (0.9, 0.95), 1e-10, 0.01
    opt = TritonMuonSRWithAuxAdam([
        dict(params=ps[:4], use_muon=True, lr=lr, momentum=beta, nesterov=True, ns_steps=5, weight_decay=wd),
        dict(params=ps[4:], use_muon=False, lr=alr, betas=betas, eps=eps, weight_decay=awd)], batch_ns=batch_ns)

    def bits(t):
        return t.view(torch.int16).numpy().view(np.uint16).copy()

    P = [bits(x) for x in p0]
    bufs = {(256, 256): np.zeros((4, 256, 256), np.uint16)} if batch_ns else [np.zeros(s, np.uint16)
                                                                             for s in shapes[:4]]
    adam = {i: dict(e=np.zeros(int(np.prod(shapes[i])), np.uint16), s=np.zeros(int(np.prod(shapes[i])), np.uint16))
            for i in range(4, 7)}
    b1, b2 = betas
    for step in range(1, 11):
        G = [bf(s, 1e-3) for s in shapes]
        for p, g in zip(ps, G):
            p.grad = g.to(DEV)
        opt.step()
        G = [bits(g) for g in G]
        if batch_ns:
            newP, bufs = O.muon_batch_step(P[:4], G[:4], bufs, step, lr, wd, beta, True, _gpu_ns, mode)
            P[:4] = newP
            exp_bufs = list(bufs[(256, 256)])
        else:
            for j in range(4):
                P[j], bufs[j] = O.muon_param_step(P[j], G[j], bufs[j], step, j, lr, wd, beta, True, _gpu_ns, mode)
            exp_bufs = bufs
        bc, bcs = O.adamw_bias_corrections(b1, b2, step)
        for i in range(4, 7):
            seed = O.deterministic_seed(step, i)
            st = adam[i]
            newp, st["e"], st["s"] = O.adamw_bf16(P[i].ravel(), G[i].ravel(), st["e"], st["s"], alr, b1, b2, eps, awd,
                                                  bc, bcs, O.NoiseSpec(mode, seed, 0), O.NoiseSpec(mode, seed, 1),
                                                  O.NoiseSpec(mode, seed, 2))
            P[i] = newp.reshape(shapes[i])
        for i, p in enumerate(ps):
            assert np.array_equal(dev_to_u16(p.data).ravel(), P[i].ravel()), (step, i)
        for j in range(4):
            assert opt.state[ps[j]]["step"] == step
            assert np.array_equal(dev_to_u16(opt.state[ps[j]]["momentum_buffer"]).ravel(),
                                  np.asarray(exp_bufs[j]).ravel()), (step, j)
        for i in range(4, 7):
            st = opt.state[ps[i]]
            assert st["step"] == step
            assert np.array_equal(dev_to_u16(st["ema"]).ravel(), adam[i]["e"]), (step, i)
            assert np.array_equal(dev_to_u16(st["ema_squared"]).ravel(), adam[i]["s"]), (step, i)
    if batch_ns:
        assert opt._global_step == 10


@pytest.mark.parametrize("mode_name", ["triton", "philox8"])
def test_two_muon_groups_global_step_vs_oracle(L, noise, mode_name):
    """Two batch_ns Muon groups with their own hyperparameters around an AdamW group.  The
    reference advances the global step once per Muon group (muon_sr/triton_muon_sr.py:319-329),
    so at step k the first group draws its seeds with global step 2k - 1 and the second with
    2k; AdamW seeds use the group offset (:351-371).  After 3 steps the state goes through
    state_dict() into a new optimizer, whose global step is restored as the largest per-param
    step (:13-15), and 2 more steps continue the same sequence."""
    from muon_sr_amd import TritonMuonSRWithAuxAdam
    noise(mode_name)
    mode = O.NOISE_TRITON if mode_name == "triton" else O.NOISE_PHILOX8
    gen = torch.Generator().manual_seed(7)

    def bf(shape, std):
        return (torch.randn(shape, generator=gen) * std).to(torch.bfloat16)

    def bits(t):
        return t.view(torch.int16).numpy().view(np.uint16).copy()

    sa = [(256, 256), (256, 512), (256, 256)]       # Muon group A
    sb = [(256,), (128, 64)]                        # AdamW group
    sc = [(256, 256), (512, 256)]                   # Muon group C
    shapes = sa + sb + sc
    p0 = [bf(x, 0.02) for x in shapes]
    ps = [torch.nn.Parameter(x.to(DEV)) for x in p0]
    hA = dict(lr=0.02, momentum=0.95, nesterov=True, weight_decay=0.01)
    hC = dict(lr=0.01, momentum=0.9, nesterov=False, weight_decay=0.0)
    alr, betas, eps, awd = 3e-4, (0.9, 0.95), 1e-10, 0.01

    def make():
        return TritonMuonSRWithAuxAdam([
            dict(params=ps[0:3], use_muon=True, ns_steps=5, **hA),
            dict(params=ps[3:5], use_muon=False, lr=alr, betas=betas, eps=eps, weight_decay=awd),
            dict(params=ps[5:7], use_muon=True, ns_steps=5, **hC)], batch_ns=True)

    opt = make()
    P = [bits(x) for x in p0]
    bufA = {sh: np.zeros((sa.count(sh), *sh), np.uint16) for sh in dict.fromkeys(sa)}
    bufC = {sh: np.zeros((sc.count(sh), *sh), np.uint16) for sh in dict.fromkeys(sc)}
    adam = {i: dict(e=np.zeros(int(np.prod(shapes[i])), np.uint16), s=np.zeros(int(np.prod(shapes[i])), np.uint16))
            for i in (3, 4)}
    b1, b2 = betas
    for k in range(1, 6):
        if k == 4:   # resume from a checkpoint of step 3
            sd = opt.state_dict()
            opt = make()
            opt.load_state_dict(sd)
        G = [bf(x, 1e-3) for x in shapes]
        for p, g in zip(ps, G):
            p.grad = g.to(DEV)
        opt.step()
        G = [bits(g) for g in G]
        P[0:3], bufA = O.muon_batch_step(P[0:3], G[0:3], bufA, 2 * k - 1, hA["lr"], hA["weight_decay"],
                                         hA["momentum"], hA["nesterov"], _gpu_ns, mode)
        P[5:7], bufC = O.muon_batch_step(P[5:7], G[5:7], bufC, 2 * k, hC["lr"], hC["weight_decay"],
                                         hC["momentum"], hC["nesterov"], _gpu_ns, mode)
        bc, bcs = O.adamw_bias_corrections(b1, b2, k)
        for i in (3, 4):
            seed = O.deterministic_seed(k, i)
            st = adam[i]
            newp, st["e"], st["s"] = O.adamw_bf16(P[i].ravel(), G[i].ravel(), st["e"], st["s"], alr, b1, b2, eps, awd,
                                                  bc, bcs, O.NoiseSpec(mode, seed, 0), O.NoiseSpec(mode, seed, 1),
                                                  O.NoiseSpec(mode, seed, 2))
            P[i] = newp.reshape(shapes[i])
        for i, p in enumerate(ps):
            assert np.array_equal(dev_to_u16(p.data).ravel(), P[i].ravel()), (k, i)
        for j, (bufs, idx) in enumerate(((bufA, range(0, 3)), (bufC, range(5, 7)))):
            seen = {}
            for i in idx:
                sh = shapes[i]
                r = seen.get(sh, 0)
                seen[sh] = r + 1
                assert opt.state[ps[i]]["step"] == 2 * k - 1 + j, (k, i)
                assert np.array_equal(dev_to_u16(opt.state[ps[i]]["momentum_buffer"]).ravel(),
                                      np.asarray(bufs[sh][r]).ravel()), (k, i)
        for i in (3, 4):
            assert opt.state[ps[i]]["step"] == k
            assert np.array_equal(dev_to_u16(opt.state[ps[i]]["ema"]).ravel(), adam[i]["e"]), (k, i)
        assert opt._global_step == 2 * k


@pytest.mark.parametrize("batch_ns", [True, False])
@pytest.mark.parametrize("mode_name", ["triton", "philox8"])
def test_muon_params_of_more_than_two_dims_vs_oracle(L, noise, batch_ns, mode_name):
    """Muon parameters of 3 and 4 dimensions (stacks of matrices, conv-like weights) beside
    2-D ones: the reference's Newton-Schulz treats the last two dimensions as the matrix and
    the leading ones as a batch, normalizes each matrix on its own, transposes by the last two
    dimensions (muon_sr/muon_sr.py:82-98) and scales by shape[-2] / shape[-1]
    (muon_sr/triton_muon_sr.py:101-102).  TritonMuonSR, 3 steps, per parameter and batch_ns,
    bit-exact against the oracle with this library's Newton-Schulz substituted."""
    from muon_sr_amd import TritonMuonSR
    noise(mode_name)
    mode = O.NOISE_TRITON if mode_name == "triton" else O.NOISE_PHILOX8
    gen = torch.Generator().manual_seed(11)

    def bf(shape, std):
        return (torch.randn(shape, generator=gen) * std).to(torch.bfloat16)

    def bits(t):
        return t.view(torch.int16).numpy().view(np.uint16).copy()

    shapes = [(3, 64, 96), (2, 4, 48, 32), (3, 64, 96), (64, 96)]
    p0 = [bf(x, 0.02) for x in shapes]
    ps = [torch.nn.Parameter(x.to(DEV)) for x in p0]
    lr, wd, beta = 0.02, 0.01, 0.95
    opt = TritonMuonSR(ps, lr=lr, weight_decay=wd, momentum=beta, nesterov=True, batch_ns=batch_ns)
    P = [bits(x) for x in p0]
    if batch_ns:
        bufs = {sh: np.zeros((shapes.count(sh), *sh), np.uint16) for sh in dict.fromkeys(shapes)}
    else:
        bufs = [np.zeros(sh, np.uint16) for sh in shapes]
    for step in range(1, 4):
        G = [bf(x, 1e-3) for x in shapes]
        for p, g in zip(ps, G):
            p.grad = g.to(DEV)
        opt.step()
        G = [bits(g) for g in G]
        if batch_ns:
            P, bufs = O.muon_batch_step(P, G, bufs, step, lr, wd, beta, True, _gpu_ns, mode)
        else:
            for j in range(len(shapes)):
                P[j], bufs[j] = O.muon_param_step(P[j], G[j], bufs[j], step, j, lr, wd, beta, True, _gpu_ns, mode)
        for i, p in enumerate(ps):
            assert np.array_equal(dev_to_u16(p.data).ravel(), np.asarray(P[i]).ravel()), (step, i)
        seen = {}
        for i, p in enumerate(ps):
            if batch_ns:
                r = seen.get(shapes[i], 0)
                seen[shapes[i]] = r + 1
                exp = bufs[shapes[i]][r]
            else:
                exp = bufs[i]
            assert np.array_equal(dev_to_u16(opt.state[p]["momentum_buffer"]).ravel(), np.asarray(exp).ravel()), (step, i)


# ---------------------------------------------------------------------------
# Config 3
# ---------------------------------------------------------------------------

def config3_shapes():
    """Per layer q, k, v, o 2048 x 2048, gate, up 5632 x 2048, down 2048 x 5632 and two
    2048 norms; 24 layers, then the 32000 x 2048 embedding (217 tensors)."""
    shapes = []
    for _ in range(24):
        shapes += [(2048, 2048)] * 4 + [(5632, 2048)] * 2 + [(2048, 5632)] + [(2048,)] * 2
    shapes.append((32000, 2048))
    return shapes


def test_config3_sr_accumulation_vs_oracle(L, noise):
    """Three micro-batches over config 3's 217 tensors (grads ~N(0, 1e-4), bf16), hooks
    fired in backward order, reference noise stream (one Philox word 0 per element,
    seed random.getrandbits(32) per hook call, muon_sr/triton_adamw.py:206-229,
    252-265).  One launch per hook: p.acc_grad holds the running sum after every
    micro-batch.  Queued (TritonSRAccumulator.deferred()): the same sums after the
    flush.  Both bit-exact against orc_sr_accum; reassign_grad_buffer hands the sums
    over as p.grad."""
    from muon_sr_amd import TritonSRAccumulator
    noise("triton")
    shapes = config3_shapes()
    assert len(shapes) == 217 and sum(int(np.prod(s)) for s in shapes) == 1298759680
    model = torch.nn.Module()
    model.ps = torch.nn.ParameterList([torch.nn.Parameter(torch.zeros(s, dtype=torch.bfloat16, device=DEV))
                                       for s in shapes])
    params = list(model.ps)
    order = list(range(len(params)))[::-1]          # the backward pass reaches the last layer first
    micro = 3

    def grad(mb, t):
        g = torch.Generator(device=DEV)
        g.manual_seed(1000 * mb + t)
        return (torch.randn(shapes[t], device=DEV, generator=g) * 1e-4).to(torch.bfloat16)

    # the oracle: one getrandbits(32) per hook call, in call order
    rs = random.Random(31337)
    exp = [None] * len(params)
    expected = []                                   # per micro-batch: the running sums (host)
    for mb in range(micro):
        for t in order:
            seed = rs.getrandbits(32)
            g = dev_to_u16(grad(mb, t)).ravel()
            prev = exp[t] if exp[t] is not None else np.zeros_like(g)
            exp[t] = O.sr_accum(prev, g, O.NoiseSpec(O.NOISE_TRITON, seed))
        expected.append(list(exp))                  # sr_accum returns new arrays
    print(f"config 3: oracle done ({sum(e.size for e in exp)} elements x {micro})", flush=True)

    hooks = TritonSRAccumulator.assign_hooks(model)
    try:
        for queued in (False, True):
            random.seed(31337)
            for mb in range(micro):
                ctx = TritonSRAccumulator.deferred() if queued else _nullcontext()
                with ctx:
                    for t in order:
                        params[t].grad = grad(mb, t)
                        TritonSRAccumulator._accum_hook(params[t])
                        assert params[t].grad is None
                torch.cuda.synchronize()
                for t in range(len(params)):
                    assert np.array_equal(dev_to_u16(params[t].acc_grad).ravel(), expected[mb][t]), (queued, mb, t)
            TritonSRAccumulator.reassign_grad_buffer(model)
            for t, p in enumerate(params):
                assert not hasattr(p, "acc_grad")
                assert np.array_equal(dev_to_u16(p.grad).ravel(), exp[t]), (queued, t)
                p.grad = None
            print(f"config 3: {'queued' if queued else 'one launch per hook'} bit-exact", flush=True)
    finally:
        for h in hooks:
            h.remove()


class _nullcontext:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


# ---------------------------------------------------------------------------
# Momentum noise offsets at and beyond 2^31 and 2^32
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,cols,start", [(64, 128, 1 << 31), (64, 128, 1 << 32), (61, 99, 1 << 31),
                                             (61, 99, 3 << 30), (128, 64, (1 << 32) + (1 << 31))])
@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8])
@pytest.mark.parametrize("fused_apply", [True, False])
def test_fused_step_noise_offsets_beyond_int32(L, rows, cols, start, mode, fused_apply):
    """A chunk whose rows sit at stack index `first`, with first * rows * cols just below
    `start`, so that its three matrices' momentum noise offsets cross `start` (2^31,
    3 * 2^30, 2^32, 2^32 + 2^31).  The new momentum must equal the oracle's prepare
    with the noise of those offsets (the reference's stream keeps their low 32 bits,
    muon_sr/triton_muon_sr.py:44); the Newton-Schulz output and, with the fused
    apply, the parameters (whose noise offsets start at 0 in every matrix) follow."""
    from muon_sr_amd.muon import newton_schulz, NS_COEFFS
    a, b, c = NS_COEFFS
    numel = rows * cols
    batch = 3
    first = start // numel - 1                 # row `first` starts below `start`, row first+1 crosses or starts at it
    off0 = first * numel
    assert off0 < start <= off0 + batch * numel
    gen = torch.Generator(device=DEV)
    gen.manual_seed(rows + cols + mode + (start >> 20))
    grads = [(torch.randn(rows, cols, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16) for _ in range(batch)]
    buf0 = (torch.randn(batch, rows, cols, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16)
    params0 = (torch.randn(batch, rows, cols, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    beta, pseed, lr, wd, scale = 0.95, 0x6C8E9CF5, 0.02, 0.01, max(1.0, rows / cols) ** 0.5
    seeds = [(0x9E3779B9 * (i + 5)) & 0xFFFFFFFF for i in range(batch)]
    # the oracle, with the noise of stack offsets off0 .. off0 + batch*numel injected
    nz = O.noise16(mode, pseed, off0 + np.arange(batch * numel, dtype=np.int64))
    g_host = np.concatenate([dev_to_u16(g).ravel() for g in grads])
    nbuf, _, u16 = O.muon_prepare(g_host, dev_to_u16(buf0).ravel(), beta, True,
                                  O.NoiseSpec(O.NOISE_INJECT, inject=nz))
    X = newton_schulz(u16_to_dev(u16).view(batch, rows, cols))
    # the fused call: buf points at row `first` of a stack whose earlier rows are not touched
    buf = buf0.clone()
    prm = params0.clone()
    nb = ctypes.c_size_t(0)
    check(L, L.msr_ns_workspace_bytes(batch, rows, cols, ctypes.byref(nb)), "ws")
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    out = None if fused_apply else torch.empty(batch, rows, cols, dtype=torch.bfloat16, device=DEV)
    seeds_c = ptr_array(seeds, ctypes.c_uint32)
    check(L, L.msr_muon_fused_step(ptr_array([g.data_ptr() for g in grads]), 0, buf.data_ptr(), first, batch, rows,
                                   cols, beta, 1, pseed, 5, a, b, c, None if fused_apply else out.data_ptr(),
                                   ptr_array([prm[i].data_ptr() for i in range(batch)]) if fused_apply else None,
                                   seeds_c if fused_apply else None, lr, wd, scale, mode, None, None,
                                   ws.data_ptr(), nb.value, stream()), "msr_muon_fused_step")
    torch.cuda.synchronize()
    assert np.array_equal(dev_to_u16(buf).ravel(), nbuf)
    if fused_apply:
        Xh = dev_to_u16(X)
        for i in range(batch):
            exp = O.muon_apply(dev_to_u16(params0[i]).ravel(), Xh[i].ravel(), lr, wd, scale, O.NoiseSpec(mode, seeds[i]))
            assert np.array_equal(dev_to_u16(prm[i]).ravel(), exp), i
    else:
        assert torch.equal(out.view(torch.int16), X.view(torch.int16))

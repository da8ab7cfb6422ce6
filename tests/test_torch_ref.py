"""The torch restatement of the reference's pure-PyTorch optimizers (the host-core
baseline) against trajectories written by the reference's own classes
(tests/golden/torch_path.npz, from tests/golden/make_torch_golden.py).

Bit-exact: the restatement draws its stochastic-rounding noise from torch's
global generator in the reference's order, and each step is run under the same
``torch.manual_seed`` as the recorded one.
"""
import numpy as np
import pytest
import torch

from oracle import torch_ref as T


def noise_seed(case, step):
    return 9000 + 100 * case + step


def bf(u):
    return torch.from_numpy(np.asarray(u, np.uint16).view(np.int16).copy()).view(torch.bfloat16)


def bits(t):
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16)


def load_params(z, tag, count, shapes):
    return [torch.nn.Parameter(bf(z[f"{tag}/p0/{i}"]).reshape(shapes[i])) for i in range(count)]


@pytest.mark.parametrize("case", [0, 1, 2])
def test_hybrid_trajectory_bit_exact(golden, case):
    z = golden("torch_path")
    tag = f"hybrid{case}"
    muon_shapes = [tuple(s) for s in z["meta/muon_shapes"]]
    shapes = muon_shapes + [(16,), (16,), (20, 12)]
    ps = load_params(z, tag, len(shapes), shapes)
    nm = len(muon_shapes)
    opt = T.TorchMuonSRWithAuxAdam([
        dict(params=ps[:nm], use_muon=True, lr=0.02, momentum=0.95, nesterov=bool(z[f"{tag}/nesterov"]), ns_steps=5,
             weight_decay=0.01),
        dict(params=ps[nm:], use_muon=False, lr=3e-4, betas=(0.9, 0.95), eps=1e-10, weight_decay=0.01),
    ], batch_ns=bool(z[f"{tag}/batch_ns"]))
    for step in range(1, int(z["meta/steps"]) + 1):
        for i, p in enumerate(ps):
            g = z[f"{tag}/g{step}/{i}"]
            p.grad = None if g.size == 0 else bf(g).reshape(shapes[i])
        torch.manual_seed(noise_seed(case, step))
        opt.step()
        for i, p in enumerate(ps):
            assert np.array_equal(bits(p), z[f"{tag}/p{step}/{i}"]), (step, i)
            st = opt.state.get(p, {})
            if f"{tag}/buf{step}/{i}" in z:
                assert np.array_equal(bits(st["momentum_buffer"]), z[f"{tag}/buf{step}/{i}"]), (step, i)
            if f"{tag}/ema{step}/{i}" in z:
                assert np.array_equal(bits(st["ema"]), z[f"{tag}/ema{step}/{i}"]), (step, i)
                assert np.array_equal(bits(st["ema_squared"]), z[f"{tag}/emasq{step}/{i}"]), (step, i)


def test_muonsr_trajectory_bit_exact(golden):
    z = golden("torch_path")
    tag, case = "muonsr3", 3
    shapes = [(16, 32), (40, 16)]
    ps = load_params(z, tag, 2, shapes)
    opt = T.TorchMuonSR(ps, lr=0.02, momentum=0.9, nesterov=True, ns_steps=3)
    for step in (1, 2):
        for i, p in enumerate(ps):
            p.grad = bf(z[f"{tag}/g{step}/{i}"]).reshape(shapes[i])
        torch.manual_seed(noise_seed(case, step))
        opt.step()
        for i, p in enumerate(ps):
            assert np.array_equal(bits(p), z[f"{tag}/p{step}/{i}"]), (step, i)
            assert np.array_equal(bits(opt.state[p]["momentum_buffer"]), z[f"{tag}/buf{step}/{i}"]), (step, i)


def test_accumulator_bit_exact(golden):
    z = golden("torch_path")
    tag, case = "accum4", 4
    model = torch.nn.Linear(16, 24, bias=True).to(torch.bfloat16)
    params = list(model.parameters())
    torch.manual_seed(noise_seed(case, 0))
    for mb in range(4):
        for i, p in enumerate(params):
            p.grad = bf(z[f"{tag}/g{mb}/{i}"]).reshape(p.shape)
            T.accumulate(p)
    T.reassign_grad_buffer(model)
    for i, p in enumerate(params):
        assert np.array_equal(bits(p.grad), z[f"{tag}/acc/{i}"]), i


def test_seed_slip_is_detected(golden):
    """A restatement that draws its noise under another seed fails the pin."""
    z = golden("torch_path")
    tag, case = "muonsr3", 3
    shapes = [(16, 32), (40, 16)]
    ps = load_params(z, tag, 2, shapes)
    opt = T.TorchMuonSR(ps, lr=0.02, momentum=0.9, nesterov=True, ns_steps=3)
    for i, p in enumerate(ps):
        p.grad = bf(z[f"{tag}/g1/{i}"]).reshape(shapes[i])
    torch.manual_seed(noise_seed(case, 1) + 1)
    opt.step()
    assert not np.array_equal(bits(ps[0]), z[f"{tag}/p1/0"])


# ---------------------------------------------------------------------------
# torch transcription of the 8-bit step against the C oracle (itself pinned by
# the reference's vectors in tests/test_oracle.py)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,block", [(4096 + 77, 256), (1000, 64), (300, 2048)])
def test_adamw8bit_torch_equals_oracle(n, block):
    import oracle as O
    rng = np.random.default_rng(n + block)
    nb = (n + block - 1) // block
    q1, q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
    p = O.f32_to_bf16_rne((rng.standard_normal(n) * 0.02).astype(np.float32))
    s1, s2 = np.full(n, 127, np.uint8), np.zeros(n, np.uint8)
    a1, a2 = np.zeros(nb, np.float32), np.zeros(nb, np.float32)
    tp, ts1, ts2 = bf(p), torch.from_numpy(s1.copy()), torch.from_numpy(s2.copy())
    ta1, ta2 = torch.from_numpy(a1.copy()), torch.from_numpy(a2.copy())
    tq1, tq2 = torch.from_numpy(q1), torch.from_numpy(q2)
    for step in range(1, 5):
        gf = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        if step == 3:
            gf[5] = np.inf
            gf[17] = np.nan
            gf[block:2 * block] = 0.0 if n > 2 * block else gf[block:2 * block]
        g = O.f32_to_bf16_rne(gf)
        noise = rng.integers(0, 1 << 16, n).astype(np.uint16)
        hyper = (3e-4, 0.9, 0.95, 1e-10, 0.01, 1 - 0.9 ** step, 1 - 0.95 ** step)
        p, s1, s2, a1, a2 = O.adamw8bit(p, g, s1, s2, a1, a2, q1, q2, block, True, *hyper,
                                        O.NoiseSpec(O.NOISE_INJECT, 0, 0, noise))
        T.adamw8bit_step(tp, bf(g), ts1, ts2, ta1, ta2, tq1, tq2, block, *hyper,
                         torch.from_numpy(noise.astype(np.int32)))
        assert np.array_equal(bits(tp), p), step
        assert np.array_equal(ts1.numpy(), s1) and np.array_equal(ts2.numpy(), s2), step
        assert np.array_equal(ta1.numpy(), a1) and np.array_equal(ta2.numpy(), a2), step


@pytest.mark.parametrize("signed", [True, False])
def test_quantize_search_torch_equals_oracle(signed):
    import oracle as O
    Q = O.create_dynamic_map(signed)
    rng = np.random.default_rng(7)
    lo = -1.0 if signed else 0.0
    x = np.concatenate([rng.uniform(lo, 1.0, 200000).astype(np.float32), Q,
                        ((Q[1:] + Q[:-1]) * np.float32(0.5)).astype(np.float32),
                        np.nextafter(Q, np.float32(2)), np.nextafter(Q, np.float32(-2))]).astype(np.float32)
    x = np.clip(x, lo, 1.0).astype(np.float32)
    got = T.quantize_search(torch.from_numpy(x), torch.from_numpy(Q), signed).numpy()
    assert np.array_equal(got, O.quantize(x, Q, signed))

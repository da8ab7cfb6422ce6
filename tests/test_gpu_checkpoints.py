"""Checkpoints written by the reference's own classes load into this library's classes.

`tests/golden/checkpoints.pt` holds, for four optimizers, the reference's `state_dict()`
after two steps, the parameters at that point, the gradients of a third step and the
reference's parameters, states and state_dict layout after that third step (written by
`tests/golden/make_golden.py` under Triton's interpreter; loaded here with
`torch.load(weights_only=True)`). Each test builds this library's optimizer on the
checkpointed parameters, loads the reference's state_dict, takes the third step in the
reference's noise stream and checks it against what the reference did:

* `TritonAdamW` (one group with centralization, a parameter with one step fewer) and
  `TritonAdamW8bit` (8-bit codes with a ragged last block, a bf16-moment tensor below
  `min_8bit_size`, an `optim_bits=16` group): parameters and every state tensor bit-exact
  (muon_sr/triton_adamw.py:117-203, muon_sr/triton_adamw_8bit.py:152-241);
* `TritonMuonSR(batch_ns=True)` and `TritonMuonSRWithAuxAdam(batch_ns=True)`: momentum
  buffers and AdamW states bit-exact against the reference, Muon parameters bit-exact
  against the oracle's step composition with this library's Newton-Schulz substituted
  (the reference's own bf16 NS is not reproducible bit for bit). The momentum seeds use
  the global step, so these pin its restore from the per-parameter steps
  (muon_sr/triton_muon_sr.py:13-15, 218-226; muon_sr/muon_sr.py:112-158).

Then this library's `state_dict()` after the step has the reference's layout: the same
state keys, dtypes and shapes per parameter and the same param groups.
"""
import os

import numpy as np
import pytest
import torch

import oracle as O
from _gpu import DEV, dev_to_u16, need_gpu, u16_to_dev

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "checkpoints.pt")


@pytest.fixture(scope="module")
def L():
    return need_gpu()


@pytest.fixture(scope="module")
def ckpt():
    return torch.load(GOLDEN, weights_only=True)


@pytest.fixture
def triton_noise():
    import muon_sr_amd
    old = muon_sr_amd.get_sr_noise()
    muon_sr_amd.set_sr_noise("triton")
    yield
    muon_sr_amd.set_sr_noise(old)


def _u16(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def _params(rec):
    return [torch.nn.Parameter(p.to(DEV)) for p in rec["p_ckpt"]]


def _step(opt, ps, rec):
    for p, g in zip(ps, rec["grads_next"]):
        p.grad = None if g is None else g.to(DEV)
    opt.step()
    torch.cuda.synchronize()


def _same_tensor(a, b):
    assert a.dtype == b.dtype and tuple(a.shape) == tuple(b.shape), (a.dtype, b.dtype, a.shape, b.shape)
    a, b = a.detach().cpu(), b.detach().cpu()
    if a.dtype == torch.bfloat16:
        return np.array_equal(_u16(a), _u16(b))
    return torch.equal(a, b)


def _structure(sd):
    st = {int(i): {k: ((str(v.dtype), tuple(v.shape)) if torch.is_tensor(v) else v) for k, v in d.items()}
          for i, d in sd["state"].items()}
    return {"state": st, "param_groups": [dict(g) for g in sd["param_groups"]]}


def _check_layout(opt, rec):
    ours = _structure(opt.state_dict())
    ref = rec["structure_next"]
    assert ours["state"] == ref["state"]
    assert ours["param_groups"] == ref["param_groups"]


def _check_states(opt, ps, rec, keys):
    for j, p in enumerate(ps):
        assert _same_tensor(p.data, rec["p_next"][j]), ("param", j)
        if j not in rec["state_next"]:
            assert p not in opt.state or not opt.state[p]
            continue
        st, ref = opt.state[p], rec["state_next"][j]
        assert st["step"] == ref["step"], ("step", j)
        for k in keys:
            if k in ref:
                assert _same_tensor(st[k], ref[k]), (k, j)


def _gpu_ns(U):
    from muon_sr_amd.muon import newton_schulz
    return dev_to_u16(newton_schulz(u16_to_dev(U.ravel()).view(U.shape))).reshape(U.shape)


# Relative Frobenius distance allowed between this library's and the reference's Muon step
# deltas: the reference's bf16 Newton-Schulz differs from this library's by 2-3 % on such
# inputs, and a small difference before stochastic rounding flips whole-ulp rounding
# decisions although the noise bits are the same (the trajectory tests measure 3.8-4.5e-2).
MUON_DELTA_TOL = 6e-2


def _check_muon_batch(opt, ps, rec, idx, lr, wd):
    """Muon parameters idx: momentum against the reference, parameters against the oracle's
    composition of the same step with this library's NS (seeds at the restored global step),
    and the step itself against the reference's next parameters within MUON_DELTA_TOL."""
    sd = rec["state_dict"]
    params = [_u16(rec["p_ckpt"][j]).reshape(tuple(rec["p_ckpt"][j].shape)) for j in idx]
    grads = [_u16(rec["grads_next"][j]).reshape(params[i].shape) for i, j in enumerate(idx)]
    bufs = {}
    for j in idx:
        shape = tuple(rec["p_ckpt"][j].shape)
        bufs.setdefault(shape, []).append(_u16(sd["state"][j]["momentum_buffer"]).reshape(shape))
    bufs = {s: np.stack(b) for s, b in bufs.items()}
    step = max(sd["state"][j]["step"] for j in idx) + 1
    new_p, _ = O.muon_batch_step(params, grads, bufs, step, lr, wd, 0.95, True, _gpu_ns, O.NOISE_TRITON)
    for i, j in enumerate(idx):
        st = opt.state[ps[j]]
        assert st["step"] == rec["state_next"][j]["step"] == step, ("step", j)
        assert _same_tensor(st["momentum_buffer"], rec["state_next"][j]["momentum_buffer"]), ("momentum", j)
        assert np.array_equal(dev_to_u16(ps[j].data).ravel(), new_p[i].ravel()), ("param", j)
        before = torch.from_numpy(np.ascontiguousarray(params[i]).view(np.int16).copy()).view(torch.bfloat16).double()
        ref_next = rec["p_next"][j].detach().cpu().double().reshape(before.shape)
        d_ours = ps[j].data.detach().cpu().double().reshape(before.shape) - before
        d_ref = ref_next - before
        e = (torch.linalg.norm(d_ours - d_ref) / torch.linalg.norm(d_ref)).item()
        print(f"param {j}: step delta vs the reference's, relative Frobenius {e:.3e}")
        assert e < MUON_DELTA_TOL, ("step delta", j, e)


def test_reference_checkpoint_triton_adamw(L, ckpt, triton_noise):
    from muon_sr_amd import TritonAdamW
    rec = ckpt["adamw"]
    ps = _params(rec)
    opt = TritonAdamW([{"params": ps[:2]}, {"params": ps[2:], "lr": 2e-3, "weight_decay": 0.1,
                                             "centralization": 0.5}],
                      lr=1e-3, betas=(0.9, 0.95), eps=1e-8)
    opt.load_state_dict(rec["state_dict"])
    _step(opt, ps, rec)
    _check_states(opt, ps, rec, ("ema", "ema_squared"))
    _check_layout(opt, rec)


def test_reference_checkpoint_adamw8bit(L, ckpt, triton_noise):
    from muon_sr_amd import TritonAdamW8bit
    rec = ckpt["adamw8bit"]
    ps = _params(rec)
    opt = TritonAdamW8bit([{"params": ps[:2]}, {"params": ps[2:], "optim_bits": 16}],
                          lr=3e-4, betas=(0.9, 0.95), eps=1e-10, weight_decay=0.01)
    opt.load_state_dict(rec["state_dict"])
    for p in ps:   # the reference's loader keeps uint8 codes and fp32 scales (:207-241)
        st = opt.state[p]
        assert st["state1"].device == p.device
        if st["optim_bits"] == 8:
            assert st["state1"].dtype == torch.uint8 and st["absmax1"].dtype == torch.float32
    _step(opt, ps, rec)
    _check_states(opt, ps, rec, ("state1", "state2", "absmax1", "absmax2", "qmap1", "qmap2"))
    _check_layout(opt, rec)


def test_reference_checkpoint_muon_batch(L, ckpt, triton_noise):
    from muon_sr_amd import TritonMuonSR
    rec = ckpt["muon_batch"]
    ps = _params(rec)
    opt = TritonMuonSR(ps, lr=0.02, weight_decay=0.01, batch_ns=True)
    opt.load_state_dict(rec["state_dict"])
    _step(opt, ps, rec)
    _check_muon_batch(opt, ps, rec, [0, 1, 2, 3], 0.02, 0.01)
    _check_layout(opt, rec)


def test_reference_checkpoint_hybrid_batch(L, ckpt, triton_noise):
    from muon_sr_amd import TritonMuonSRWithAuxAdam
    rec = ckpt["hybrid_batch"]
    ps = _params(rec)
    opt = TritonMuonSRWithAuxAdam(
        [{"params": ps[:3], "use_muon": True, "weight_decay": 0.01},
         {"params": ps[3:], "use_muon": False, "lr": 3e-4, "betas": (0.9, 0.95), "eps": 1e-10,
          "weight_decay": 0.01}],
        batch_ns=True)
    opt.load_state_dict(rec["state_dict"])
    _step(opt, ps, rec)
    _check_muon_batch(opt, ps, rec, [0, 1, 2], 0.02, 0.01)
    for j in (3, 4):
        assert _same_tensor(ps[j].data, rec["p_next"][j]), ("param", j)
        for k in ("ema", "ema_squared"):
            assert _same_tensor(opt.state[ps[j]][k], rec["state_next"][j][k]), (k, j)
    _check_layout(opt, rec)

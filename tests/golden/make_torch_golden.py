"""Write golden trajectories of the reference's pure-PyTorch optimizers.

Run in the development container only (the GPU box has no reference checkout):

    python tests/golden/make_torch_golden.py [/path/to/reference]

It imports bab2min/muon_sr 0.1.2 and steps its CPU classes ``MuonSR``,
``MuonSRWithAuxAdam`` and ``SRAccumulator`` (muon_sr/muon_sr.py) on small seeded
bf16 tensors.  Their stochastic rounding draws its noise from torch's global
generator, so every step is preceded by ``torch.manual_seed(noise_seed(step))``;
parameters and gradients come from a separate ``torch.Generator``.  Only the
results are committed (``torch_path.npz`` beside this file).
"""
from __future__ import annotations

import os
import sys

# importing the reference must not write bytecode into its (read-only) checkout
sys.dont_write_bytecode = True

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
sys.path.insert(0, REF)

from muon_sr import muon_sr as rp  # noqa: E402

MUON_SHAPES = [(16, 24), (16, 24), (32, 16), (16, 24), (24, 24)]
ADAM_SHAPES = [(16,), (16,), (20, 12)]
STEPS = 3
MISSING = {(1, 1), (2, 4)}       # (step, muon index) whose gradient is None at that step


def noise_seed(case: int, step: int) -> int:
    return 9000 + 100 * case + step


def u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def make_params(gen, shapes, std):
    return [torch.nn.Parameter((torch.randn(s, generator=gen) * std).to(torch.bfloat16)) for s in shapes]


def hybrid_case(case: int, batch_ns: bool, nesterov: bool, out: dict):
    gen = torch.Generator().manual_seed(100 + case)
    muon = make_params(gen, MUON_SHAPES, 0.02)
    adam = make_params(gen, ADAM_SHAPES, 0.02)
    opt = rp.MuonSRWithAuxAdam([
        dict(params=muon, use_muon=True, lr=0.02, momentum=0.95, nesterov=nesterov, ns_steps=5, weight_decay=0.01),
        dict(params=adam, use_muon=False, lr=3e-4, betas=(0.9, 0.95), eps=1e-10, weight_decay=0.01),
    ], batch_ns=batch_ns)
    tag = f"hybrid{case}"
    out[f"{tag}/batch_ns"] = np.int32(batch_ns)
    out[f"{tag}/nesterov"] = np.int32(nesterov)
    for i, p in enumerate(muon + adam):
        out[f"{tag}/p0/{i}"] = u16(p)
    for step in range(1, STEPS + 1):
        for i, p in enumerate(muon + adam):
            missing = i < len(muon) and (step, i) in MISSING
            g = None if missing else (torch.randn(p.shape, generator=gen) * 1e-3).to(torch.bfloat16)
            p.grad = g
            out[f"{tag}/g{step}/{i}"] = np.zeros(0, np.uint16) if g is None else u16(g)
        torch.manual_seed(noise_seed(case, step))
        opt.step()
        for i, p in enumerate(muon + adam):
            out[f"{tag}/p{step}/{i}"] = u16(p)
            st = opt.state[p]
            if "momentum_buffer" in st:
                out[f"{tag}/buf{step}/{i}"] = u16(st["momentum_buffer"])
            if "ema" in st:
                out[f"{tag}/ema{step}/{i}"] = u16(st["ema"])
                out[f"{tag}/emasq{step}/{i}"] = u16(st["ema_squared"])


def muonsr_case(case: int, out: dict):
    """MuonSR (single group, per-matrix path, no weight decay)."""
    gen = torch.Generator().manual_seed(100 + case)
    ps = make_params(gen, [(16, 32), (40, 16)], 0.02)
    opt = rp.MuonSR(ps, lr=0.02, momentum=0.9, nesterov=True, ns_steps=3)
    tag = f"muonsr{case}"
    for i, p in enumerate(ps):
        out[f"{tag}/p0/{i}"] = u16(p)
    for step in range(1, 3):
        for i, p in enumerate(ps):
            p.grad = (torch.randn(p.shape, generator=gen) * 1e-3).to(torch.bfloat16)
            out[f"{tag}/g{step}/{i}"] = u16(p.grad)
        torch.manual_seed(noise_seed(case, step))
        opt.step()
        for i, p in enumerate(ps):
            out[f"{tag}/p{step}/{i}"] = u16(p)
            out[f"{tag}/buf{step}/{i}"] = u16(opt.state[p]["momentum_buffer"])


def accum_case(case: int, out: dict):
    gen = torch.Generator().manual_seed(100 + case)
    model = torch.nn.Linear(16, 24, bias=True).to(torch.bfloat16)
    params = [p for _, p in model.named_parameters()]
    tag = f"accum{case}"
    torch.manual_seed(noise_seed(case, 0))
    for mb in range(4):
        for i, p in enumerate(params):
            g = (torch.randn(p.shape, generator=gen) * 1e-4).to(torch.bfloat16)
            out[f"{tag}/g{mb}/{i}"] = u16(g)
            p.grad = g
            rp.SRAccumulator.stochastic_grad_accum(p)
    rp.SRAccumulator.reassign_grad_buffer(model)
    for i, p in enumerate(params):
        out[f"{tag}/acc/{i}"] = u16(p.grad)


def main():
    out = {}
    hybrid_case(0, batch_ns=True, nesterov=True, out=out)
    hybrid_case(1, batch_ns=False, nesterov=True, out=out)
    hybrid_case(2, batch_ns=True, nesterov=False, out=out)
    muonsr_case(3, out)
    accum_case(4, out)
    out["meta/muon_shapes"] = np.array(MUON_SHAPES, np.int32)
    out["meta/steps"] = np.int32(STEPS)
    out["meta/missing"] = np.array(sorted(MISSING), np.int32)
    path = os.path.join(HERE, "torch_path.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()

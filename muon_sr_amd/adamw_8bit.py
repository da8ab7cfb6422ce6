"""bitsandbytes-style blockwise 8-bit AdamW with BF16 weight stochastic rounding.

Drop-in for ``muon_sr.triton_adamw_8bit.TritonAdamW8bit`` (bab2min/muon_sr
0.1.2, muon_sr/triton_adamw_8bit.py:102-241): same constructor, param-group
keys, validation errors, state format (``format_version=2``) and seeds.  The
step runs one fused gfx950 kernel per tensor (libmuon_sr_amd.so).
"""
from __future__ import annotations

import math
import weakref

import torch
from torch.optim import Optimizer

from . import _lib


def create_dynamic_map(signed: bool = True) -> torch.Tensor:
    """The 256-entry dynamic (signed) or unsigned-dynamic codebook.

    For each decade i = 0..6 the fp32 midpoints of ``linspace(0.1, 1, 2**i + 1)``
    (signed) or ``linspace(0.1, 1, 2**(i+1) + 1)`` (unsigned), scaled by
    10**(i-6) (and negated as well for the signed map), plus 0 and 1, sorted
    (muon_sr/triton_adamw_8bit.py:14-24).
    """
    vals = []
    for i in range(7):
        pts = torch.linspace(0.1, 1, 2 ** (i if signed else i + 1) + 1, dtype=torch.float32)
        mids = (pts[:-1] + pts[1:]) / 2
        scale = 10 ** (-6 + i)
        vals.extend((scale * mids).tolist())
        if signed:
            vals.extend((-scale * mids).tolist())
    return torch.tensor(sorted(vals + [0.0, 1.0]), dtype=torch.float32)


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


# Quantizer tables: built once per process on the host from the standard
# codebooks, copied once per device; used only for states whose codebooks are
# bit-identical to the standard ones (checked once per codebook tensor).
_std_maps = None
_host_table = None
_dev_tables = {}
_map_verdict = {}  # id(qmap1) -> (weakref(qmap1), weakref(qmap2), bool)


def _standard_maps():
    global _std_maps
    if _std_maps is None:
        _std_maps = (create_dynamic_map(True), create_dynamic_map(False))
    return _std_maps


def quant_table(state):
    """Device pointer of the quantizer table for this state's codebooks, or None."""
    global _host_table
    q1, q2 = state["qmap1"], state["qmap2"]
    verdict = _map_verdict.get(id(q1))
    if verdict is None or verdict[0]() is not q1 or verdict[1]() is not q2:
        s1, s2 = _standard_maps()
        ok = torch.equal(q1.detach().cpu(), s1) and torch.equal(q2.detach().cpu(), s2)
        verdict = (weakref.ref(q1), weakref.ref(q2), ok)
        _map_verdict[id(q1)] = verdict
    if not verdict[2]:
        return None
    dev = q1.device
    t = _dev_tables.get(dev)
    if t is None:
        if _host_table is None:
            L = _lib.lib()
            nbytes = L.msr_quant_table_bytes()
            buf = torch.zeros(nbytes, dtype=torch.uint8)
            s1, s2 = _standard_maps()
            _lib.check(L.msr_quant_table_build(s1.data_ptr(), s2.data_ptr(), buf.data_ptr(), nbytes),
                       "msr_quant_table_build")
            _host_table = buf
        t = _host_table.to(dev)
        _dev_tables[dev] = t
    return t.data_ptr()


def adamw8bit_launch(p, g, state, lr, beta1, beta2, eps, weight_decay, seed):
    """One fused 8-bit (or bf16-moment) step of one tensor with state from ``init_8bit_state``."""
    n = state["step"]
    quant = state["optim_bits"] == 8
    get = lambda k: state[k].data_ptr() if k in state else None  # noqa: E731
    qt = quant_table(state) if quant else None
    rc = _lib.lib().msr_adamw8bit_step(
        p.data_ptr(), g.data_ptr(), state["state1"].data_ptr(), state["state2"].data_ptr(),
        get("absmax1"), get("absmax2"), get("qmap1"), get("qmap2"), qt, p.numel(), state["block_size"], int(quant),
        lr, beta1, beta2, eps, weight_decay, 1 - beta1 ** n, 1 - beta2 ** n, seed,
        _lib.noise_mode(), None, _lib.stream_of(p))
    _lib.check(rc, "msr_adamw8bit_step")


def init_8bit_state(p, block_size, optim_bits, min_8bit_size, maps):
    """State of one tensor (muon_sr/triton_adamw_8bit.py:152-165)."""
    bits = 16 if p.numel() < min_8bit_size else optim_bits
    state = dict(step=0, format_version=2, block_size=block_size, optim_bits=bits)
    dtype = torch.uint8 if bits == 8 else torch.bfloat16
    state.update(state1=torch.zeros_like(p, dtype=dtype, memory_format=torch.contiguous_format),
                 state2=torch.zeros_like(p, dtype=dtype, memory_format=torch.contiguous_format))
    if bits == 8:
        if p.device not in maps:
            maps[p.device] = (create_dynamic_map(True).to(p.device), create_dynamic_map(False).to(p.device))
        state["qmap1"], state["qmap2"] = maps[p.device]
        blocks = _cdiv(p.numel(), block_size)
        state["absmax1"] = torch.zeros(blocks, device=p.device, dtype=torch.float32)
        state["absmax2"] = torch.zeros_like(state["absmax1"])
        state["state1"].fill_(127)  # the signed codebook's exact zero
    return state


_QUANT_KEYS = ("state1", "state2", "qmap1", "qmap2", "absmax1", "absmax2")


def split_8bit_state(state_dict, param_groups, is_8bit_group):
    """Take the 8-bit states of a checkpoint out of torch's Optimizer.load_state_dict,
    which would cast every floating-point state tensor to the parameter's dtype
    (fp32 block scales and codebooks to bf16).

    ``is_8bit_group(saved_group)`` selects the groups whose states use the
    TritonAdamW8bit format.  Their states are checked against format_version 2
    and the group's block size and bits (the errors of
    muon_sr/triton_adamw_8bit.py:219-236).  Returns (the state dict without those
    tensors, restore), where ``restore(optimizer.state)`` puts copies back on each
    parameter's device after torch has loaded the rest."""
    groups = state_dict["param_groups"]
    mapping = dict(zip([i for g in groups for i in g["params"]], [p for g in param_groups for p in g["params"]]))
    restored = {}
    for group in groups:
        if not is_8bit_group(group):
            continue
        for ident in group["params"]:
            state = state_dict["state"].get(ident, {})
            if not state:
                continue
            p = mapping[ident]
            bits = 16 if p.numel() < group["min_8bit_size"] else group["optim_bits"]
            if (state.get("format_version") != 2 or state.get("block_size") != group["block_size"]
                    or state.get("optim_bits") != bits):
                raise ValueError("Incompatible state format/quantization configuration")
            specs = {key: (p.shape, torch.uint8 if bits == 8 else torch.bfloat16) for key in ("state1", "state2")}
            if bits == 8:
                specs.update({key: ((256,), torch.float32) for key in ("qmap1", "qmap2")})
                specs.update({key: ((_cdiv(p.numel(), group["block_size"]),), torch.float32)
                              for key in ("absmax1", "absmax2")})
            restored[ident] = {}
            for key, (shape, dtype) in specs.items():
                value = state[key]
                if value.dtype != dtype or tuple(value.shape) != tuple(shape):
                    raise ValueError(f"Invalid checkpoint state: {key}")
                restored[ident][key] = value.to(device=p.device, dtype=dtype).clone(
                    memory_format=torch.contiguous_format)
    stripped = dict(state_dict, state={i: ({k: v for k, v in st.items() if k not in _QUANT_KEYS}
                                           if i in restored else st)
                                       for i, st in state_dict["state"].items()})

    def restore(opt_state):
        for ident, values in restored.items():
            opt_state[mapping[ident]].update(values)
    return stripped, restore


def step_seed(step: int, param_index: int) -> int:
    """muon_sr/triton_adamw_8bit.py:197."""
    return (step * 2654435761 ^ param_index * 1234567891) & 0xFFFFFFFF


class TritonAdamW8bit(Optimizer):
    """Dynamic-codebook 8-bit moments, BF16-SR fallback, BF16 weight SR.

    Default blocks contain 256 elements. Tensors below min_8bit_size=4096 use
    BF16 moments with SR. Set group optim_bits=16 to exclude embeddings/other
    tensors; for_model() creates these groups automatically.
    GPU, dense contiguous tensors only. No CPU offload, AMSGrad, or clipping.
    """

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
                 weight_decay=0., block_size=256, min_8bit_size=4096, optim_bits=8):
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay,
                                      block_size=block_size, min_8bit_size=min_8bit_size,
                                      optim_bits=optim_bits))
        self._maps = {}
        for group in self.param_groups:
            self._validate_group(group)

    @classmethod
    def for_model(cls, model, min_8bit_size=4096, **kwargs):
        """Keep embeddings (including tied heads) and small tensors on 16-bit states
        (muon_sr/triton_adamw_8bit.py:119-136)."""
        if "optim_bits" in kwargs:
            raise ValueError("for_model selects optim_bits per group")
        embeddings = {id(p) for mod in model.modules() if isinstance(mod, torch.nn.Embedding)
                      for p in mod.parameters()}
        groups = {8: [], 16: []}
        for p in model.parameters():
            if p.requires_grad:
                bits = 16 if id(p) in embeddings or p.numel() < min_8bit_size else 8
                groups[bits].append(p)
        return cls([dict(params=params, optim_bits=bits) for bits, params in groups.items() if params],
                   min_8bit_size=min_8bit_size, **kwargs)

    @staticmethod
    def _validate_group(g):
        """muon_sr/triton_adamw_8bit.py:138-150."""
        for key in ("lr", "eps", "weight_decay"):
            v = g[key]
            if not isinstance(v, (int, float)) or not math.isfinite(v) or v < 0:
                raise ValueError(f"{key} must be a finite nonnegative scalar")
        if g["eps"] == 0 or len(g["betas"]) != 2 or any(not 0 <= b < 1 for b in g["betas"]):
            raise ValueError("eps must be positive and betas must be in [0,1)")
        block = g["block_size"]
        if not isinstance(block, int) or block < 32 or block > 4096 or block & (block - 1):
            raise ValueError("block_size must be a power of two between 32 and 4096")
        if g["optim_bits"] not in (8, 16) or not isinstance(g["min_8bit_size"], int) or g["min_8bit_size"] < 0:
            raise ValueError("optim_bits must be 8/16; min_8bit_size must be nonnegative")

    def _init_state(self, p, group):
        return init_8bit_state(p, group["block_size"], group["optim_bits"], group["min_8bit_size"], self._maps)

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        index = 0
        for group in self.param_groups:
            self._validate_group(group)
            b1, b2 = group["betas"]
            for p in group["params"]:
                param_index = index
                index += 1
                if p.grad is None:
                    continue
                if p.dtype != torch.bfloat16 or not p.is_cuda:
                    raise ValueError("TritonAdamW8bit requires CUDA BF16 parameters")
                g = p.grad
                if g.is_sparse or not p.is_contiguous() or not g.is_contiguous():
                    raise ValueError("Parameters/gradients must be contiguous and dense")
                if not p.numel():
                    continue
                state = self.state[p]
                if not state:
                    state.update(self._init_state(p, group))
                expected_bits = 16 if p.numel() < group["min_8bit_size"] else group["optim_bits"]
                if state["block_size"] != group["block_size"] or state["optim_bits"] != expected_bits:
                    raise ValueError("Cannot change quantization configuration after state initialization")
                state["step"] += 1
                seed = step_seed(state["step"], param_index)
                adamw8bit_launch(p, g, state, group["lr"], b1, b2, group["eps"], group["weight_decay"], seed)
        return loss

    def load_state_dict(self, state_dict):
        """Restore uint8 codes and fp32 scales without torch's cast to the
        parameter dtype (muon_sr/triton_adamw_8bit.py:207-241)."""
        groups = state_dict["param_groups"]
        if len(groups) != len(self.param_groups) or any(
                len(a["params"]) != len(b["params"]) for a, b in zip(groups, self.param_groups)):
            raise ValueError("Checkpoint parameter groups do not match optimizer")
        for group in groups:
            self._validate_group(group)
        stripped, restore = split_8bit_state(state_dict, self.param_groups, lambda group: True)
        super().load_state_dict(stripped)
        restore(self.state)

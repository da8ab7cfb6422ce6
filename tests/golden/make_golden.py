"""Write golden input/output vectors from the reference's own kernels.

Run in the development container only (the GPU box has no reference checkout):

    python tests/golden/make_golden.py [/path/to/reference] [--only name,name]

It imports bab2min/muon_sr 0.1.2 with ``TRITON_INTERPRET=1`` so that its Triton
kernels execute on CPU tensors through Triton's interpreter (numpy, IEEE fp32,
no contraction).  Only the results are committed (``*.npz`` beside this file).

Argument typing: a compiled Triton launch types a Python float argument as an
fp32 scalar and an int in [2^31, 2^63) as i64 (``triton.runtime.jit.mangle_type``
returns 'fp32' / 'i64'); the interpreter instead keeps floats as Python doubles,
so pure-scalar subexpressions such as ``1 - B1`` would be folded in double.
``_compiled_arg_typing`` below marshals float and large-int arguments the way
the compiled launcher types them, so the vectors follow the compiled kernel's
scalar arithmetic.  The reference's kernel code runs unmodified.

Interpreter caveat: its fp32->bf16 cast truncates where the compiled kernel
rounds to nearest even.  Stochastic-rounding stores are unaffected (their low 16
bits are already zero); the one RNE store on the path, ``_muon_prepare_kernel``'s
update (muon_sr/triton_muon_sr.py:50), is captured unrounded by passing an fp32
output buffer, and the composed Muon trajectories below record the interpreter's
truncating behaviour explicitly (``prepare_rounding = "trunc"``).
"""
from __future__ import annotations

import copy
import os
import sys

# importing the reference must not write bytecode into its (read-only) checkout
sys.dont_write_bytecode = True

os.environ["TRITON_INTERPRET"] = "1"

import numpy as np  # noqa: E402
import torch  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 and not sys.argv[1].startswith("--") else "/root/reference"
sys.path.insert(0, REF)

import triton  # noqa: E402
import triton.language as tl  # noqa: E402
import muon_sr  # noqa: E402
from muon_sr import triton_adamw_8bit as r8  # noqa: E402
from muon_sr import triton_adamw as ra  # noqa: E402
from muon_sr import triton_muon_sr as rm  # noqa: E402
from muon_sr import muon_sr as rp  # noqa: E402
import triton.runtime.interpreter as _interp  # noqa: E402

_interp_cvt = _interp._implicit_cvt


def _compiled_arg_typing(arg):
    if isinstance(arg, float):
        assert triton.runtime.jit.mangle_type(arg) == "fp32"
        return tl.tensor(_interp.TensorHandle(np.array([arg], np.float32), tl.float32), tl.float32)
    if isinstance(arg, int) and not isinstance(arg, bool) and 2**31 <= arg < 2**63:
        assert triton.runtime.jit.mangle_type(arg) == "i64"
        return tl.tensor(_interp.TensorHandle(np.array([arg], np.int64), tl.int64), tl.int64)
    return _interp_cvt(arg)


_interp._implicit_cvt = _compiled_arg_typing


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def bf(t_np_u16: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(t_np_u16.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)


def randn_bf16(gen, n, std):
    return (torch.randn(n, generator=gen, dtype=torch.float32) * std).to(torch.bfloat16)


# ---------------------------------------------------------------------------
# 1. codebooks and the quantizer
# ---------------------------------------------------------------------------

@triton.jit
def _quantize_probe(X, OUT, N, Q, SIGNED: tl.constexpr, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    mask = offs < N
    x = tl.load(X + offs, mask, other=0.)
    tl.store(OUT + offs, r8._quantize(x, Q, SIGNED), mask)


def quantizer_inputs(Q: np.ndarray, signed: bool, rng) -> np.ndarray:
    Q = Q.astype(np.float32)
    mids = ((Q[1:] + Q[:-1]) * np.float32(0.5)).astype(np.float32)
    pts = np.concatenate([Q, mids])
    near = [pts, np.nextafter(pts, np.float32(np.inf)), np.nextafter(pts, np.float32(-np.inf))]
    for k in (2, 3):
        up, dn = pts.copy(), pts.copy()
        for _ in range(k):
            up = np.nextafter(up, np.float32(np.inf))
            dn = np.nextafter(dn, np.float32(-np.inf))
        near += [up, dn]
    lo = -1.0 if signed else 0.0
    uni = rng.uniform(lo, 1.0, 6000).astype(np.float32)
    mags = (10.0 ** rng.uniform(-9, 0, 6000)).astype(np.float32)
    if signed:
        mags *= rng.choice(np.array([-1, 1], np.float32), 6000)
    special = np.array([0.0, -0.0, 1.0, -1.0, 1e-45, -1e-45, 1e-38, -1e-38, 5e-8, -5e-8], np.float32)
    x = np.concatenate(near + [uni, mags, special]).astype(np.float32)
    x = x[(x >= lo) & (x <= 1.0) | (x == 0)]
    if not signed:
        x = x[~np.signbit(x) | (x == 0)]
    return np.ascontiguousarray(x)


def gen_quantize(rng):
    q1 = r8.create_dynamic_map(True)
    q2 = r8.create_dynamic_map(False)
    out = {"qmap1": q1.numpy(), "qmap2": q2.numpy()}
    for name, Q, signed in (("signed", q1, True), ("unsigned", q2, False)):
        x = quantizer_inputs(Q.numpy(), signed, rng)
        codes = torch.zeros(x.size, dtype=torch.uint8)
        xt = torch.from_numpy(x)
        BLOCK = 1024
        _quantize_probe[(triton.cdiv(x.size, BLOCK),)](xt, codes, x.size, Q, SIGNED=signed, BLOCK=BLOCK)
        out[f"x_{name}"] = x
        out[f"code_{name}"] = codes.numpy()
    np.savez_compressed(os.path.join(HERE, "quantize.npz"), **out)


# ---------------------------------------------------------------------------
# 2. 8-bit AdamW kernel (both variants)
# ---------------------------------------------------------------------------

def gen_adamw8bit():
    gen = torch.Generator().manual_seed(1234)
    q1 = r8.create_dynamic_map(True)
    q2 = r8.create_dynamic_map(False)
    cases = {}
    # (name, n, block, quantized, steps, lr, betas, eps, wd, seed_base)
    specs = [
        ("q256", 1000, 256, True, 4, 3e-4, (0.9, 0.95), 1e-10, 0.01, None),
        ("q32", 100, 32, True, 3, 1e-3, (0.9, 0.999), 1e-8, 0.0, None),
        ("q128_bigseed", 300, 128, True, 2, 2e-3, (0.8, 0.99), 1e-6, 0.1, 0xFFFFFFF0),
        ("b16", 333, 256, False, 3, 3e-4, (0.9, 0.95), 1e-10, 0.01, None),
        ("b16_wrap", 200, 64, False, 2, 1e-3, (0.9, 0.999), 1e-8, 0.05, 0x7FFFFFFE),
        ("b16_i64wrap", 150, 32, False, 2, 1e-3, (0.9, 0.999), 1e-8, 0.05, 0xFFFFFFFD),
    ]
    for name, n, block, quantized, steps, lr, (b1, b2), eps, wd, seed_base in specs:
        p = randn_bf16(gen, n, 0.02)
        blocks = triton.cdiv(n, block)
        if quantized:
            s1 = torch.full((n,), 127, dtype=torch.uint8)
            s2 = torch.zeros(n, dtype=torch.uint8)
            a1 = torch.zeros(blocks, dtype=torch.float32)
            a2 = torch.zeros(blocks, dtype=torch.float32)
        else:
            s1 = torch.zeros(n, dtype=torch.bfloat16)
            s2 = torch.zeros(n, dtype=torch.bfloat16)
            a1 = p
            a2 = p
        rec = {"n": n, "block": block, "quantized": int(quantized), "lr": lr, "b1": b1, "b2": b2,
               "eps": eps, "wd": wd, "steps": steps, "p0": u16(p)}
        if quantized:
            rec["s1_0"], rec["s2_0"] = s1.numpy().copy(), s2.numpy().copy()
            rec["a1_0"], rec["a2_0"] = a1.numpy().copy(), a2.numpy().copy()
        else:
            rec["s1_0"], rec["s2_0"] = u16(s1), u16(s2)
        for step in range(1, steps + 1):
            g = randn_bf16(gen, n, 1e-3)
            if step == 1 and n >= 2 * block:
                g[block:2 * block] = 0.0  # an all-zero block: absmax 0 on the first step
            if step == 2:
                g[5] = float("nan")
                g[7] = float("inf")
                g[n - 1] = float("-inf")
            seed = seed_base + step if seed_base is not None else (step * 2654435761 ^ 3 * 1234567891) & 0xFFFFFFFF
            rec[f"g_{step}"] = u16(g)
            rec[f"seed_{step}"] = seed
            r8._adamw_8bit_kernel[(blocks,)](
                p, g, s1, s2, a1, a2, q1 if quantized else p, q2 if quantized else p, n,
                lr, b1, b2, eps, wd, 1 - b1 ** step, 1 - b2 ** step, seed,
                BLOCK=block, QUANTIZED=quantized)
            rec[f"p_{step}"] = u16(p)
            if quantized:
                rec[f"s1_{step}"], rec[f"s2_{step}"] = s1.numpy().copy(), s2.numpy().copy()
                rec[f"a1_{step}"], rec[f"a2_{step}"] = a1.numpy().copy(), a2.numpy().copy()
            else:
                rec[f"s1_{step}"], rec[f"s2_{step}"] = u16(s1), u16(s2)
        for k, v in rec.items():
            cases[f"{name}/{k}"] = np.asarray(v)
    np.savez_compressed(os.path.join(HERE, "adamw8bit.npz"), **cases)


# ---------------------------------------------------------------------------
# 3. bf16-moment AdamW, SR accumulate, Muon prepare/apply kernels
# ---------------------------------------------------------------------------

def gen_elementwise():
    gen = torch.Generator().manual_seed(99)
    out = {}
    # _adamw_kernel: seeds chosen to cover i32, the i32 wrap of seed+1/seed+2, and u32
    n = 3000
    for tag, seed in (("s_small", 12345), ("s_wrap", 0x7FFFFFFF), ("s_wrap2", 0x7FFFFFFE), ("s_u32", 0xDEADBEEF),
                      ("s_i64wrap", 0xFFFFFFFF)):
        p = randn_bf16(gen, n, 0.02)
        g = randn_bf16(gen, n, 1e-3)
        e = randn_bf16(gen, n, 1e-4)
        s = (randn_bf16(gen, n, 1e-4).float() ** 2).to(torch.bfloat16)
        out[f"adamw/{tag}/in_p"], out[f"adamw/{tag}/in_g"] = u16(p), u16(g)
        out[f"adamw/{tag}/in_e"], out[f"adamw/{tag}/in_s"] = u16(e), u16(s)
        step, lr, b1, b2, eps, wd = 3, 1e-3, 0.9, 0.999, 1e-8, 0.01
        bc, bcs = 1.0 - b1 ** step, (1.0 - b2 ** step) ** 0.5
        ra._adamw_kernel[(triton.cdiv(n, 1024),)](p, g, e, s, lr, b1, b2, eps, wd, bc, bcs, n, seed, BLOCK_SIZE=1024)
        out[f"adamw/{tag}/seed"] = np.asarray(seed)
        out[f"adamw/{tag}/hyper"] = np.asarray([lr, b1, b2, eps, wd, bc, bcs])
        out[f"adamw/{tag}/out_p"], out[f"adamw/{tag}/out_e"], out[f"adamw/{tag}/out_s"] = u16(p), u16(e), u16(s)

    # _grad_accum_kernel: bf16 and fp32 gradients
    n = 2500
    acc = randn_bf16(gen, n, 1e-3)
    g = randn_bf16(gen, n, 1e-4)
    g32 = torch.randn(n, generator=gen) * 1e-4
    out["accum/in_acc"], out["accum/in_g"], out["accum/in_g32"] = u16(acc), u16(g), g32.numpy()
    a1 = acc.clone()
    ra._grad_accum_kernel[(triton.cdiv(n, 1024),)](a1, g, n, 777, BLOCK_SIZE=1024)
    a2 = acc.clone()
    ra._grad_accum_kernel[(triton.cdiv(n, 1024),)](a2, g32, n, 0x9E3779B9, BLOCK_SIZE=1024)
    out["accum/out_bf16g"], out["accum/out_f32g"] = u16(a1), u16(a2)

    # _muon_prepare_kernel with an fp32 output (captures the update before its RNE cast)
    n = 2000
    for nest in (True, False):
        g = randn_bf16(gen, n, 1e-3)
        buf = randn_bf16(gen, n, 1e-3)
        upd = torch.zeros(n, dtype=torch.float32)
        out[f"prepare/{int(nest)}/in_g"], out[f"prepare/{int(nest)}/in_buf"] = u16(g), u16(buf)
        seed = rm._deterministic_seed(7, 2, salt=0)
        rm._muon_prepare_kernel[(triton.cdiv(n, 1024),)](g, buf, upd, 0.95, nest, n, seed, BLOCK_SIZE=1024)
        out[f"prepare/{int(nest)}/seed"] = np.asarray(seed)
        out[f"prepare/{int(nest)}/out_buf"], out[f"prepare/{int(nest)}/out_upd_f32"] = u16(buf), upd.numpy()

    # _muon_apply_kernel
    p = randn_bf16(gen, n, 0.02)
    u = randn_bf16(gen, n, 0.05)
    out["apply/in_p"], out["apply/in_u"] = u16(p), u16(u)
    seed = rm._deterministic_seed(5, 20003, salt=1)
    scale = max(1.0, 5632 / 2048) ** 0.5
    rm._muon_apply_kernel[(triton.cdiv(n, 1024),)](p, u, 0.02, 0.01, scale, n, seed, BLOCK_SIZE=1024)
    out["apply/seed"], out["apply/scale"] = np.asarray(seed), np.asarray(scale)
    out["apply/out_p"] = u16(p)
    np.savez_compressed(os.path.join(HERE, "elementwise.npz"), **out)


# ---------------------------------------------------------------------------
# 4. Newton-Schulz (torch CPU bf16) and composed optimizer trajectories
# ---------------------------------------------------------------------------

def gen_ns_and_trajectories():
    gen = torch.Generator().manual_seed(2024)
    out = {}
    for i, shape in enumerate([(64, 128), (128, 64), (3, 32, 48), (96, 96)]):
        G = (torch.randn(*shape, generator=gen) * 1e-3).to(torch.bfloat16)
        X = rp._newton_schulz(G, steps=5, out_dtype=None)
        out[f"ns/{i}/in"] = u16(G)
        out[f"ns/{i}/shape"] = np.asarray(shape)
        out[f"ns/{i}/out"] = u16(X)

    # TritonAdamW on two groups (seeds use group_offset + i, muon_sr/triton_adamw.py:153-201)
    ps = [randn_bf16(gen, 300, 0.02).view(10, 30).clone(), randn_bf16(gen, 64, 0.02).clone(),
          randn_bf16(gen, 128, 0.02).clone()]
    ps = [torch.nn.Parameter(p) for p in ps]
    for j, p in enumerate(ps):
        out[f"traj_adamw/p{j}_0"] = u16(p.data)
    opt = ra.TritonAdamW([{"params": ps[:2]}, {"params": ps[2:], "lr": 2e-3, "weight_decay": 0.1}],
                         lr=1e-3, betas=(0.9, 0.95), eps=1e-8)
    for step in range(1, 4):
        for j, p in enumerate(ps):
            p.grad = randn_bf16(gen, p.numel(), 1e-3).view(p.shape)
            if step == 2 and j == 1:
                p.grad = None
            out[f"traj_adamw/g{j}_{step}"] = u16(p.grad) if p.grad is not None else np.zeros(0, np.uint16)
        opt.step()
        for j, p in enumerate(ps):
            out[f"traj_adamw/p{j}_{step}"] = u16(p.data)
            out[f"traj_adamw/e{j}_{step}"] = u16(opt.state[p]["ema"])
            out[f"traj_adamw/s{j}_{step}"] = u16(opt.state[p]["ema_squared"])

    # TritonMuonSR batch_ns=True and the hybrid with batch_ns=False (prepare rounding: interpreter truncation)
    for tag, make in (("muon_batch", lambda ps: rm.TritonMuonSR(ps, lr=0.02, weight_decay=0.01, batch_ns=True)),
                      ("hybrid_nobatch", lambda ps: rm.TritonMuonSRWithAuxAdam(
                          [{"params": ps[:3], "use_muon": True, "weight_decay": 0.01},
                           {"params": ps[3:], "use_muon": False, "lr": 3e-4, "betas": (0.9, 0.95), "eps": 1e-10}],
                          batch_ns=False))):
        shapes = [(32, 48), (48, 32), (32, 48), (40,), (8, 8)] if tag == "hybrid_nobatch" else [(32, 48), (48, 32), (32, 48)]
        ps = [torch.nn.Parameter((torch.randn(*s, generator=gen) * 0.02).to(torch.bfloat16)) for s in shapes]
        for j, p in enumerate(ps):
            out[f"{tag}/p{j}_0"] = u16(p.data)
            out[f"{tag}/shape{j}"] = np.asarray(p.shape)
        opt = make(ps)
        for step in range(1, 3):
            for j, p in enumerate(ps):
                p.grad = (torch.randn(*p.shape, generator=gen) * 1e-3).to(torch.bfloat16)
                out[f"{tag}/g{j}_{step}"] = u16(p.grad)
            opt.step()
            for j, p in enumerate(ps):
                out[f"{tag}/p{j}_{step}"] = u16(p.data)
                st = opt.state[p]
                if "momentum_buffer" in st:
                    out[f"{tag}/buf{j}_{step}"] = u16(st["momentum_buffer"])
                else:
                    out[f"{tag}/e{j}_{step}"] = u16(st["ema"])
                    out[f"{tag}/s{j}_{step}"] = u16(st["ema_squared"])
    out["prepare_rounding"] = np.asarray("trunc")
    np.savez_compressed(os.path.join(HERE, "ns_traj.npz"), **out)


# ---------------------------------------------------------------------------
# 5. Checkpoints written by the reference's classes
# ---------------------------------------------------------------------------

def _structure(sd):
    """Keys, dtypes and shapes of a state_dict, and its param groups (plain data)."""
    st = {int(i): {k: ((str(v.dtype), tuple(v.shape)) if torch.is_tensor(v) else v) for k, v in d.items()}
          for i, d in sd["state"].items()}
    return {"state": st, "param_groups": [dict(g) for g in sd["param_groups"]]}


def _case(opt, ps, gen, steps_before, grad_std, missing=()):
    """Run steps_before steps, record the state_dict and parameters, then one more step and its results."""
    rec = {"p0": [p.detach().clone() for p in ps]}
    for step in range(1, steps_before + 2):
        grads = []
        for j, p in enumerate(ps):
            g = (torch.randn(*p.shape, generator=gen) * grad_std).to(torch.bfloat16)
            p.grad = None if (step, j) in missing else g
            grads.append(None if p.grad is None else g.clone())
        if step == steps_before + 1:
            # the checkpoint: torch.save of the reference's own state_dict() (views of the
            # batch_ns stacks are saved with their storage, as a user's torch.save would)
            rec["state_dict"] = copy.deepcopy(opt.state_dict())   # its entries are live objects
            rec["p_ckpt"] = [p.detach().clone() for p in ps]
            rec["grads_next"] = grads
        opt.step()
    rec["p_next"] = [p.detach().clone() for p in ps]
    rec["state_next"] = {j: {k: (v.clone() if torch.is_tensor(v) else v) for k, v in opt.state[p].items()}
                         for j, p in enumerate(ps) if p in opt.state}
    rec["structure_next"] = _structure(opt.state_dict())
    return rec


def _adamw8bit_reference_steps(opt, ps, gen, steps):
    """TritonAdamW8bit.step (muon_sr/triton_adamw_8bit.py:169-204) refuses CPU tensors, so the
    interpreter cannot run it; this calls the class's own _init_state and kernel with the
    step's seed and bias corrections, in the step's parameter order, for `steps` steps."""
    for _ in range(steps):
        index = 0
        for group in opt.param_groups:
            opt._validate_group(group)
            b1, b2 = group["betas"]
            for p in group["params"]:
                param_index = index
                index += 1
                g = p.grad
                if g is None:
                    continue
                state = opt.state[p]
                if not state:
                    state.update(opt._init_state(p, group))
                state["step"] += 1
                n = state["step"]
                seed = (n * 2654435761 ^ param_index * 1234567891) & 0xFFFFFFFF
                r8._adamw_8bit_kernel[(triton.cdiv(p.numel(), group["block_size"]),)](
                    p, g, state["state1"], state["state2"],
                    state.get("absmax1", p), state.get("absmax2", p),
                    state.get("qmap1", p), state.get("qmap2", p), p.numel(),
                    group["lr"], b1, b2, group["eps"], group["weight_decay"],
                    1 - b1 ** n, 1 - b2 ** n, seed, BLOCK=group["block_size"],
                    QUANTIZED=state["optim_bits"] == 8)


class _StepAs8bit:
    """Gives _case an optimizer whose step() runs _adamw8bit_reference_steps once."""
    def __init__(self, opt, ps, gen):
        self.opt, self.ps = opt, ps
        self.state = opt.state

    def step(self):
        _adamw8bit_reference_steps(self.opt, self.ps, None, 1)

    def state_dict(self):
        return self.opt.state_dict()


def gen_checkpoints():
    gen = torch.Generator().manual_seed(4242)
    cases = {}

    def params(shapes, std=0.02):
        return [torch.nn.Parameter((torch.randn(*s, generator=gen) * std).to(torch.bfloat16)) for s in shapes]

    # TritonMuonSR(batch_ns=True): stacks of two shapes plus a single one; the global step is
    # restored from the per-parameter steps on load (muon_sr/triton_muon_sr.py:13-15, 218-226)
    ps = params([(32, 48), (48, 32), (32, 48), (16, 16)])
    opt = rm.TritonMuonSR(ps, lr=0.02, weight_decay=0.01, batch_ns=True)
    cases["muon_batch"] = _case(opt, ps, gen, 2, 1e-3)
    # TritonAdamW: two groups (the second with centralization), a missing gradient in step 1
    ps = params([(10, 30), (64,), (8, 16)])
    opt = ra.TritonAdamW([{"params": ps[:2]}, {"params": ps[2:], "lr": 2e-3, "weight_decay": 0.1,
                                                 "centralization": 0.5}],
                         lr=1e-3, betas=(0.9, 0.95), eps=1e-8)
    cases["adamw"] = _case(opt, ps, gen, 2, 1e-3, missing={(1, 1)})
    # TritonMuonSRWithAuxAdam(batch_ns=True): Muon group and AdamW group
    ps = params([(32, 48), (48, 32), (32, 48), (40,), (8, 8)])
    opt = rm.TritonMuonSRWithAuxAdam(
        [{"params": ps[:3], "use_muon": True, "weight_decay": 0.01},
         {"params": ps[3:], "use_muon": False, "lr": 3e-4, "betas": (0.9, 0.95), "eps": 1e-10,
          "weight_decay": 0.01}],
        batch_ns=True)
    cases["hybrid_batch"] = _case(opt, ps, gen, 2, 1e-3)
    # TritonAdamW8bit: an 8-bit tensor with a ragged last block, a tensor below min_8bit_size
    # (bf16 moments) and an optim_bits=16 group
    ps = params([(40, 260), (30, 40), (8, 64)])
    opt = r8.TritonAdamW8bit([{"params": ps[:2]}, {"params": ps[2:], "optim_bits": 16}],
                             lr=3e-4, betas=(0.9, 0.95), eps=1e-10, weight_decay=0.01)
    cases["adamw8bit"] = _case(_StepAs8bit(opt, ps, gen), ps, gen, 2, 1e-3)
    torch.save(cases, os.path.join(HERE, "checkpoints.pt"))


if __name__ == "__main__":
    only = sys.argv[sys.argv.index("--only") + 1].split(",") if "--only" in sys.argv else None
    print("reference version", muon_sr.__version__)
    for name, fn in (("quantize", lambda: gen_quantize(np.random.default_rng(7))), ("adamw8bit", gen_adamw8bit),
                     ("elementwise", gen_elementwise), ("ns_traj", gen_ns_and_trajectories),
                     ("checkpoints", gen_checkpoints)):
        if only is None or name in only:
            fn()
            print(name, "done")

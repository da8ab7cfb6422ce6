"""Small-GPT convergence replication of the reference's `examples.py` (variants 4-8) on one GPU.

The reference trains a byte-level GPT (8 layers, d_model 384, 6 heads, vocab 16384, sequence
128) for 500 optimizer steps of batch 32 with 4 micro-batches, from identical weights and
identical batches, with a cosine learning-rate schedule, and reports the final loss, the mean
of the last 50 steps, the wall time and the peak memory of each variant
(examples.py:209-327; its results: README.md:140-163). This script runs the same experiment
with this library:

  4  MuonSRWithAuxAdam + SRAccumulator: the reference's pure-PyTorch SR path, as restated in
     oracle/torch_ref.py (a checker of this test suite; here run on the GPU's tensors)
  5  TritonMuonSRWithAuxAdam + TritonSRAccumulator
  6  TritonMuonSRWithAuxAdam, no accumulator (bf16 gradients summed by autograd)
  7  TritonMuonSRWithAuxAdam(batch_ns=True) + TritonSRAccumulator
  8  TritonMuonSRWithAuxAdam(batch_ns=True), no accumulator

plus two baselines written out below, the same Muon/AdamW update in plain torch:

  fp32    fp32 parameters and optimizer (the role of the reference's variant 1)
  bf16rn  bf16 parameters and optimizer with round-to-nearest (the role of its variant 3)

The reference's variants 1-3 use Keller Jordan's `muon` package, which is not installed here.
Attention is computed in fp32 in every variant (the reference's runs in the model dtype).

Usage (GPU; the corpus defaults to the first 20 MB of this image's Python sources):

    python tests/convergence/small_gpt.py [--corpus FILE] [--steps 500] [--variants 4,5,6,7,8,fp32,bf16rn]
                                          [--json out.json]
"""
from __future__ import annotations

import argparse
import copy
import glob
import json
import math
import os
import sys
import time

import torch
import torch.nn as nn
import torch.nn.functional as F

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

VOCAB, D_MODEL, HEADS, LAYERS, MAX_T = 16384, 384, 6, 8, 256
BATCH, SEQ, ACCUM = 32, 128, 4


# ---------------------------------------------------------------------------
# model: pre-norm GPT with learned positions (examples.py:31-82)
# ---------------------------------------------------------------------------

class Attention(nn.Module):
    def __init__(self, d, heads):
        super().__init__()
        self.heads = heads
        self.qkv = nn.Linear(d, 3 * d, bias=False)
        self.proj = nn.Linear(d, d, bias=False)

    def forward(self, x):
        b, t, d = x.shape
        q, k, v = self.qkv(x).view(b, t, 3, self.heads, d // self.heads).permute(2, 0, 3, 1, 4)
        # attention in fp32: batched bf16 products with transposed operands (which the
        # attention math path and the backward of batched products form) are avoided on these GPUs
        y = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True).to(x.dtype)
        return self.proj(y.transpose(1, 2).reshape(b, t, d))


class Block(nn.Module):
    def __init__(self, d, heads):
        super().__init__()
        self.ln1, self.ln2 = nn.LayerNorm(d), nn.LayerNorm(d)
        self.attn = Attention(d, heads)
        self.mlp = nn.Sequential(nn.Linear(d, 4 * d, bias=False), nn.GELU(), nn.Linear(4 * d, d, bias=False))

    def forward(self, x):
        x = x + self.attn(self.ln1(x))
        return x + self.mlp(self.ln2(x))


class SmallGPT(nn.Module):
    def __init__(self):
        super().__init__()
        self.embed = nn.Embedding(VOCAB, D_MODEL)
        self.pos_embed = nn.Embedding(MAX_T, D_MODEL)
        self.blocks = nn.ModuleList([Block(D_MODEL, HEADS) for _ in range(LAYERS)])
        self.ln_f = nn.LayerNorm(D_MODEL)
        self.head = nn.Linear(D_MODEL, VOCAB, bias=False)

    def forward(self, idx):
        x = self.embed(idx) + self.pos_embed(torch.arange(idx.size(1), device=idx.device))
        for blk in self.blocks:
            x = blk(x)
        return self.head(self.ln_f(x))


def param_groups(model):
    """Matrices of the blocks go to Muon; embeddings, head, norms to AdamW (examples.py:137-150)."""
    muon, adam = [], []
    for name, p in model.named_parameters():
        aux = any(k in name for k in ("embed", "head", "ln", "bias"))
        (muon if p.ndim >= 2 and not aux else adam).append(p)
    return [dict(params=muon, lr=0.02, momentum=0.95, weight_decay=0.01, use_muon=True),
            dict(params=adam, lr=3e-4, betas=(0.9, 0.95), eps=1e-10, weight_decay=0.1, use_muon=False)]


# ---------------------------------------------------------------------------
# data (examples.py:89-130): bytes, tiled to >= 2 MB, batches pre-sampled from a seed
# ---------------------------------------------------------------------------

def load_corpus(path=None, limit=20 << 20):
    if path:
        with open(path, "rb") as f:
            raw = f.read()
    else:
        parts, total = [], 0
        for fn in sorted(glob.glob("/usr/lib/python3*/**/*.py", recursive=True)):
            with open(fn, "rb") as f:
                b = f.read()
            parts.append(b)
            total += len(b)
            if total >= limit:
                break
        raw = b"".join(parts)[:limit]
    data = torch.frombuffer(bytearray(raw), dtype=torch.uint8).long()
    if data.numel() < (2 << 20):
        data = data.repeat(-(-(2 << 20) // data.numel()))
    return data


def batches(data, steps, seed, device):
    gen = torch.Generator().manual_seed(seed)
    starts = torch.randint(0, data.numel() - SEQ - 1, (steps * ACCUM, BATCH), generator=gen)
    idx = starts.unsqueeze(-1) + torch.arange(SEQ)
    return data[idx].to(device), data[idx + 1].to(device)


# ---------------------------------------------------------------------------
# baselines: Muon + AdamW in plain torch, in the parameters' dtype (round to nearest)
# ---------------------------------------------------------------------------

def _ns5(G, steps=5):
    a, b, c = 3.4445, -4.7750, 2.0315
    X = G.to(torch.bfloat16)
    tall = X.size(-2) > X.size(-1)
    if tall:
        X = X.mT.contiguous()
    X = X / (X.norm() + 1e-7)
    for _ in range(steps):
        A = X @ X.mT.contiguous()
        X = a * X + (b * A + c * (A @ A)) @ X
    return X.mT if tall else X


class PlainMuonAdam(torch.optim.Optimizer):
    """Muon (momentum, nesterov, bf16 Newton-Schulz, scale sqrt(max(1, rows/cols)),
    decoupled weight decay) and AdamW, with states in the parameter dtype and every store
    rounded to nearest."""

    def __init__(self, groups):
        super().__init__(groups, {})

    @torch.no_grad()
    def step(self):
        for g in self.param_groups:
            for p in g["params"]:
                if p.grad is None:
                    continue
                st = self.state[p]
                if g["use_muon"]:
                    buf = st.setdefault("momentum_buffer", torch.zeros_like(p))
                    buf.lerp_(p.grad, 1 - g["momentum"])
                    u = p.grad.lerp(buf, g["momentum"])
                    u = _ns5(u).to(p.dtype) * max(1, p.size(-2) / p.size(-1)) ** 0.5
                    p.mul_(1 - g["lr"] * g["weight_decay"]).add_(u, alpha=-g["lr"])
                else:
                    st["step"] = st.get("step", 0) + 1
                    m = st.setdefault("exp_avg", torch.zeros_like(p))
                    v = st.setdefault("exp_avg_sq", torch.zeros_like(p))
                    b1, b2 = g["betas"]
                    m.lerp_(p.grad, 1 - b1)
                    v.mul_(b2).addcmul_(p.grad, p.grad, value=1 - b2)
                    m_hat = m / (1 - b1 ** st["step"])
                    v_hat = v / (1 - b2 ** st["step"])
                    p.mul_(1 - g["lr"] * g["weight_decay"]).addcdiv_(m_hat, v_hat.sqrt() + g["eps"], value=-g["lr"])


# ---------------------------------------------------------------------------
# variants
# ---------------------------------------------------------------------------

class TorchSRAccumulator:
    """The reference's SRAccumulator hooks (muon_sr/muon_sr.py:29-70) on the restated accumulate."""

    @staticmethod
    def assign_hooks(model):
        from oracle import torch_ref
        return [p.register_post_accumulate_grad_hook(torch_ref.accumulate) for p in model.parameters()
                if p.requires_grad]

    @staticmethod
    def reassign_grad_buffer(model):
        from oracle import torch_ref
        torch_ref.reassign_grad_buffer(model)


def make_variant(name, model):
    from muon_sr_amd import TritonMuonSRWithAuxAdam, TritonSRAccumulator
    if name == "4":
        from oracle.torch_ref import TorchMuonSRWithAuxAdam
        return TorchMuonSRWithAuxAdam(param_groups(model)), TorchSRAccumulator
    if name in ("5", "6", "7", "8"):
        opt = TritonMuonSRWithAuxAdam(param_groups(model), batch_ns=name in ("7", "8"))
        return opt, TritonSRAccumulator if name in ("5", "7") else None
    if name in ("fp32", "bf16rn"):
        return PlainMuonAdam(param_groups(model)), None
    raise ValueError(name)


LABELS = {
    "fp32": "fp32 Muon (plain torch)",
    "bf16rn": "pure bf16 Muon, round-to-nearest (plain torch)",
    "4": "MuonSRWithAuxAdam + SRAccumulator (torch restatement)",
    "5": "TritonMuonSRWithAuxAdam + TritonSRAccumulator",
    "6": "TritonMuonSRWithAuxAdam, no accumulator",
    "7": "TritonMuonSRWithAuxAdam(batch_ns=True) + TritonSRAccumulator",
    "8": "TritonMuonSRWithAuxAdam(batch_ns=True), no accumulator",
}


def train(name, base, xs, ys, steps, log_every, keep=False):
    """Trains a copy of `base` with variant `name`; with `keep`, the result also holds the
    trained model and its optimizer (key "trained")."""
    model = copy.deepcopy(base)
    if name == "fp32":
        model = model.float()
    opt, acc = make_variant(name, model)
    hooks = acc.assign_hooks(model) if acc is not None else []
    base_lr = [g["lr"] for g in opt.param_groups]
    losses = []
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    t0 = time.perf_counter()
    for step in range(steps):
        total = 0.0
        for micro in range(ACCUM):
            i = step * ACCUM + micro
            logits = model(xs[i])
            loss = F.cross_entropy(logits.reshape(-1, logits.size(-1)), ys[i].reshape(-1))
            (loss / ACCUM).backward()
            total += loss.item() / ACCUM
        if acc is not None:
            acc.reassign_grad_buffer(model)
        opt.step()
        for p in model.parameters():
            p.grad = None
        # cosine annealing to 0 over the run (what CosineAnnealingLR(T_max=steps) computes)
        for g, lr0 in zip(opt.param_groups, base_lr):
            g["lr"] = lr0 * (1 + math.cos(math.pi * (step + 1) / steps)) / 2
        losses.append(total)
        if (step + 1) % log_every == 0:
            print(f"  [{name}] step {step + 1}/{steps} loss {sum(losses[-log_every:]) / log_every:.4f}", flush=True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    peak = torch.cuda.max_memory_allocated() / 2 ** 20
    for h in hooks:
        h.remove()
    out = {"variant": name, "label": LABELS[name], "final_loss": losses[-1],
           "mean_last_50": sum(losses[-50:]) / min(50, len(losses)), "time_s": elapsed, "peak_mb": peak,
           "losses": losses}
    if keep:
        out["trained"] = (model, opt)
    else:
        del model, opt
        torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--corpus", default=None)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--variants", default="fp32,bf16rn,4,5,6,7,8")
    ap.add_argument("--log-every", type=int, default=50)
    ap.add_argument("--json", default=None)
    args = ap.parse_args()
    dev = "cuda"
    torch.manual_seed(42)
    data = load_corpus(args.corpus)
    print(f"corpus: {data.numel():,} bytes", flush=True)
    xs, ys = batches(data, args.steps, 42, dev)
    base = SmallGPT().to(device=dev, dtype=torch.bfloat16)
    print(f"parameters: {sum(p.numel() for p in base.parameters()):,}", flush=True)
    results = []
    for name in args.variants.split(","):
        print(f"=== {name}: {LABELS[name]}", flush=True)
        results.append(train(name, base, xs, ys, args.steps, args.log_every))
    ref = next((r for r in results if r["variant"] == "fp32"), None)
    print(f"\n{'variant':<8} {'final':>8} {'last50':>8} {'vs fp32':>8} {'time s':>7} {'peak MB':>8}")
    for r in results:
        d = r["final_loss"] - ref["final_loss"] if ref else float("nan")
        print(f"{r['variant']:<8} {r['final_loss']:8.4f} {r['mean_last_50']:8.4f} {d:+8.4f} {r['time_s']:7.1f} "
              f"{r['peak_mb']:8.0f}  {r['label']}")
    if args.json:
        with open(args.json, "w") as f:
            json.dump({"steps": args.steps, "corpus_bytes": data.numel(), "results": results}, f)


if __name__ == "__main__":
    main()

"""Benchmark of the muon_sr optimizer-step hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--configs adamw8bit,probe8,sr_accum,ns,centralize,wgrad,full]
                    [--noise philox8|triton] [--no-cpu-baseline] [--copy-calibration]

Prints ONE JSON line.  ``value`` is the headline workload (BASELINE.json
configs[1]): one fused 8-bit blockwise AdamW step on a flat bf16 parameter of
2^28 elements, in GB/s of algorithmic traffic (10.0625 B/element: read p, g,
m, v and write p, m, v, plus 16 B of absmax per 256-element block).  The other
configs of BASELINE.json are measured in the same run and reported under
``configs``: SR gradient accumulation (config 3), the Muon Newton-Schulz step
(config 4, TFLOP/s) and the full Llama-3-8B-shaped hybrid step (config 5, ms).

Inputs are synthetic, seeded, and resident in HBM before the timed region.
Kernel durations come from HIP events recorded on the stream the kernels run
on; whole-step times from a synchronised wall clock around exactly K steps.
"""
from __future__ import annotations

import argparse
import json
import statistics
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0       # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA, TFLOP/s
N8 = 1 << 28
B8_PER_ELEM = 10.0 + 16.0 / 256  # 10.0625


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def sync():
    import torch
    torch.cuda.synchronize()


class LaunchTimer:
    """HIP events recorded on the launch stream immediately before and after
    every call of the named C-ABI entry points, so each pair brackets that
    launch (and not the Python work of the optimizer step around it)."""

    def __init__(self, *names):
        from muon_sr_amd import _lib
        self.names = set(names)
        self.real = _lib.lib()
        self.pairs = []
        self.on = False
        timer = self

        class Proxy:
            def __getattr__(self, attr):
                fn = getattr(timer.real, attr)
                if attr not in timer.names:
                    return fn

                def timed(*args):
                    import torch
                    if not timer.on:
                        return fn(*args)
                    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    s.record()
                    rc = fn(*args)
                    e.record()
                    timer.pairs.append((s, e))
                    return rc
                return timed

        self.proxy = Proxy()

    def __enter__(self):
        from muon_sr_amd import _lib
        self._saved = _lib._lib
        _lib._lib = self.proxy
        return self

    def __exit__(self, *exc):
        from muon_sr_amd import _lib
        _lib._lib = self._saved

    def mean_ms(self):
        return self.total_ms() / max(1, len(self.pairs))

    def median_ms(self):
        ts = sorted(s.elapsed_time(e) for s, e in self.pairs)
        return ts[len(ts) // 2] if ts else 0.0

    def total_ms(self):
        return sum(s.elapsed_time(e) for s, e in self.pairs)


# ---------------------------------------------------------------------------
# config 2: 8-bit AdamW on one flat bf16 parameter of 2^28 elements
# ---------------------------------------------------------------------------

def bench_adamw8bit(steps, warmup, n=N8):
    import torch
    from muon_sr_amd import TritonAdamW8bit
    dev = "cuda:0"
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    p = torch.nn.Parameter((torch.randn(n, device=dev, generator=gen) * 0.02).to(torch.bfloat16))
    opt = TritonAdamW8bit([p], lr=3e-4, betas=(0.9, 0.95), eps=1e-10, weight_decay=0.01)
    # Seeded gradients generated before any timing, in a pool of 4 buffers used in
    # turn: consecutive steps see different data, and, as in training, where each
    # step rewrites the same .grad storage, the step reads gradient memory the GPU
    # has mapped before (a fresh 512 MiB buffer per step would time page-table walks).
    grads = []
    for s in range(4):
        gen.manual_seed(1000 + s)
        grads.append((torch.randn(n, device=dev, generator=gen) * 1e-3).to(torch.bfloat16))
    it = 0
    for _ in range(10 + warmup):   # build the uint8 codes and block scales; clocks settle
        p.grad = grads[it % 4]; it += 1
        opt.step()
    sync()
    with LaunchTimer("msr_adamw8bit_step") as lt:
        t0 = time.perf_counter()
        lt.on = True
        for _ in range(steps):
            p.grad = grads[it % 4]; it += 1
            opt.step()
        lt.on = False
        sync()
        wall = (time.perf_counter() - t0) * 1e3 / steps
    kms = lt.median_ms()      # the median launch of the timed steps
    nbytes = B8_PER_ELEM * n
    st = opt.state[p]
    assert st["optim_bits"] == 8 and st["state1"].dtype == torch.uint8
    out = dict(ms_per_step=wall, kernel_ms=kms, kernel_ms_mean=lt.mean_ms(), gbps=nbytes / (wall * 1e6),
               kernel_gbps=nbytes / (kms * 1e6), bytes_per_step=nbytes)
    del grads, opt, p
    torch.cuda.empty_cache()
    return out


def bench_stream8_probe(n=N8, reps=10):
    """The 8-bit step's memory accesses with the arithmetic taken out (msr_stream_probe8: the
    same pair walk, loads and stores, one integer operation per word), swept over occupancy
    (k work-groups of 4 waves per CU, set by each work-group's LDS) and grid (1 or 2 rounds of
    the resident work-groups).  The best rate is the memory system's ceiling for this access
    pattern on this GPU, measured in the same run as the step."""
    import torch
    from muon_sr_amd import _lib
    L = _lib.lib()
    dev = "cuda:0"
    p = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    g = torch.ones(n, dtype=torch.bfloat16, device=dev)
    m = torch.zeros(n, dtype=torch.uint8, device=dev)
    v = torch.zeros(n, dtype=torch.uint8, device=dev)
    a1 = torch.zeros(n // 256, dtype=torch.float32, device=dev)
    a2 = torch.zeros(n // 256, dtype=torch.float32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    lds_per_cu = 160 << 10
    nbytes = B8_PER_ELEM * n
    rows = []
    for k in (2, 3, 4, 6, 8):                       # work-groups (of 4 waves) per CU
        lds = min(64 << 10, lds_per_cu // k - (1 << 10))
        for rounds in (1, 2):
            grid = 256 * k * rounds

            def run():
                _lib.check(L.msr_stream_probe8(p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr(), a1.data_ptr(),
                                               a2.data_ptr(), n, grid, lds, s), "msr_stream_probe8")
            for _ in range(3):
                run()
            evs = []
            for _ in range(reps):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                run()
                e1.record()
                evs.append((e0, e1))
            sync()
            ms = statistics.median(x.elapsed_time(y) for x, y in evs)
            rows.append(dict(waves_per_cu=4 * k, grid=grid, ms=round(ms, 4), gbps=round(nbytes / (ms * 1e6), 1)))
    best = max(rows, key=lambda r: r["gbps"])
    del p, g, m, v, a1, a2
    torch.cuda.empty_cache()
    return dict(bytes_per_launch=nbytes, best_gbps=best["gbps"], best=best, sweep=rows)


def host_cpu():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline_adamw8bit(budget_s=8.0):
    """The oracle's C restatement (OpenMP over blocks) on a bounded sample of config 2."""
    import numpy as np
    import oracle as O
    n = 1 << 24
    rng = np.random.default_rng(0)
    p = O.f32_to_bf16_rne((rng.standard_normal(n) * 0.02).astype(np.float32))
    q1, q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
    s1 = np.full(n, 127, np.uint8)
    s2 = np.zeros(n, np.uint8)
    a1 = np.zeros(n // 256, np.float32)
    a2 = np.zeros(n // 256, np.float32)
    g = O.f32_to_bf16_rne((rng.standard_normal(n) * 1e-3).astype(np.float32))
    steps, t = 0, 0.0
    while t < budget_s:
        step = steps + 1
        t0 = time.perf_counter()
        p, s1, s2, a1, a2 = O.adamw8bit(p, g, s1, s2, a1, a2, q1, q2, 256, True, 3e-4, 0.9, 0.95, 1e-10, 0.01,
                                        1 - 0.9 ** step, 1 - 0.95 ** step,
                                        O.NoiseSpec(O.NOISE_PHILOX8, step * 2654435761 & 0xFFFFFFFF))
        t += time.perf_counter() - t0
        steps += 1
    gbps = B8_PER_ELEM * n * steps / t / 1e9
    threads = int(O.lib().orc_num_threads())
    return dict(value=round(gbps, 4), unit="GB/s", cores=threads, host_cpus=os.cpu_count(), kind="port",
                sample=f"{steps} steps of the C oracle (restatement of muon_sr/triton_adamw_8bit.py:56-89, "
                       f"OpenMP over blocks) on 2^24 of the 2^28 elements (same per-element work), {t:.1f} s, "
                       f"{threads} threads of {host_cpu()}")


def host_threads():
    """Threads for the host-core baselines: every CPU the process sees
    (os.cpu_count()), capped by the job's CPU share when the environment states
    one (OMP_NUM_THREADS; a GPU box of this pool gives a one-GPU job 16 threads)."""
    n = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS")
    if share and share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return n


def cpu_baselines_torch(budget_s=6.0):
    """The torch restatement of the reference's pure-PyTorch optimizers
    (oracle/torch_ref.py) timed on the host cores, per config.  Config 1 runs
    whole; the others run a bounded sample and are scaled to the config:
    config 2 by elements (2^22 of 2^28), config 3 by elements (one layer's
    tensors), configs 4 and 5 by Newton-Schulz flops of one 2048x2048 Muon
    matrix step plus the 8-bit AdamW group by bytes (extrapolated)."""
    import numpy as np
    import torch
    import oracle as O
    from oracle import torch_ref as T
    torch.set_num_threads(host_threads())
    threads = torch.get_num_threads()
    out = {"cores": threads, "host_cpus": os.cpu_count(), "kind": "port", "host": host_cpu()}
    gen = torch.Generator().manual_seed(1)

    def bf(shape, std):
        return (torch.randn(shape, generator=gen) * std).to(torch.bfloat16)

    # config 1: MuonSRWithAuxAdam, 4x256^2 Muon + 2x256 + 512x256 AdamW, 10 steps
    muon = [torch.nn.Parameter(bf((256, 256), 0.02)) for _ in range(4)]
    adam = [torch.nn.Parameter(bf((256,), 0.02)) for _ in range(2)] + [torch.nn.Parameter(bf((512, 256), 0.02))]
    opt = T.TorchMuonSRWithAuxAdam([dict(params=muon, use_muon=True, lr=0.02, momentum=0.95, nesterov=True,
                                         ns_steps=5, weight_decay=0.01),
                                    dict(params=adam, use_muon=False, lr=3e-4, betas=(0.9, 0.95), eps=1e-10,
                                         weight_decay=0.01)], batch_ns=True)
    t0 = time.perf_counter()
    for _ in range(10):
        for p in muon + adam:
            p.grad = bf(p.shape, 1e-3)
        opt.step()
    out["cpu_plumbing_ms_per_step"] = round((time.perf_counter() - t0) * 1e3 / 10, 3)

    # config 2 (torch transcription of the 8-bit math, noise from torch.randint)
    n = 1 << 22
    q1, q2 = torch.from_numpy(O.create_dynamic_map(True)), torch.from_numpy(O.create_dynamic_map(False))
    p, g = bf(n, 0.02), bf(n, 1e-3)
    s1, s2 = torch.full((n,), 127, dtype=torch.uint8), torch.zeros(n, dtype=torch.uint8)
    a1, a2 = torch.zeros(n // 256), torch.zeros(n // 256)
    steps, t = 0, 0.0
    while t < budget_s / 2 or steps < 2:
        steps += 1
        t0 = time.perf_counter()
        noise = torch.randint(0, 1 << 16, (n,), dtype=torch.int32)
        T.adamw8bit_step(p, g, s1, s2, a1, a2, q1, q2, 256, 3e-4, 0.9, 0.95, 1e-10, 0.01,
                         1 - 0.9 ** steps, 1 - 0.95 ** steps, noise)
        t += time.perf_counter() - t0
    a8_gbps = B8_PER_ELEM * n * steps / t / 1e9
    out["adamw8bit_torch_gbps"] = round(a8_gbps, 4)

    # config 3: SR accumulation of one layer's 9 tensors (the second micro-batch onwards)
    layer = llama_small_shapes()[:9]
    ps = [torch.nn.Parameter(torch.zeros(s, dtype=torch.bfloat16)) for s in layer]
    grads = [bf(s, 1e-4) for s in layer]
    for p_, g_ in zip(ps, grads):
        p_.grad = g_
        T.accumulate(p_)
    el = sum(p_.numel() for p_ in ps)
    t0 = time.perf_counter()
    for p_, g_ in zip(ps, grads):
        p_.grad = g_
        T.accumulate(p_)
    acc_s = time.perf_counter() - t0
    total_el = sum(int(np.prod(s)) for s in llama_small_shapes())
    out["sr_accum_ms_per_microbatch_extrapolated"] = round(acc_s * total_el / el * 1e3, 1)
    out["sr_accum_gbps"] = round(6.0 * el / acc_s / 1e9, 4)
    del ps, grads

    # configs 4 and 5: one 2048x2048 Muon matrix step, scaled by NS flops
    w = torch.nn.Parameter(bf((2048, 2048), 0.02))
    buf = torch.zeros(2048, 2048, dtype=torch.bfloat16)
    w.grad = bf((2048, 2048), 1e-3)
    T.muon_matrix_step(w, w.grad, buf, 0.95, True, 5, 0.02, 0.01)   # warm-up (library set-up)
    t0 = time.perf_counter()
    for _ in range(2):
        T.muon_matrix_step(w, w.grad, buf, 0.95, True, 5, 0.02, 0.01)
    mt = (time.perf_counter() - t0) / 2
    rate = ns_flops([(2048, 2048)]) / mt
    out["muon_2048_matrix_step_s"] = round(mt, 3)
    out["ns_gflops"] = round(rate / 1e9, 2)
    out["muon_ns_16L_d2048_ms_extrapolated"] = round(ns_flops(config4_shapes()) / rate * 1e3, 1)
    adam_bytes = B8_PER_ELEM * 1050939392
    out["hybrid_llama3_8b_ms_extrapolated"] = round((ns_flops(llama8b_muon_shapes()) / rate
                                                     + adam_bytes / (a8_gbps * 1e9)) * 1e3, 1)
    out["sample"] = ("config 1 whole (10 steps); config 2: 2^22 elements; config 3: one layer (9 tensors) scaled "
                     "by elements; configs 4/5: one 2048x2048 Muon step scaled by NS flops, plus the 8-bit "
                     "AdamW group at the torch transcription's GB/s (extrapolated)")
    return out


# ---------------------------------------------------------------------------
# config 3: SR gradient accumulation, 24-layer d=2048 ffn=5632 parameter set
# ---------------------------------------------------------------------------

def llama_small_shapes():
    shapes = []
    for _ in range(24):
        shapes += [(2048, 2048)] * 4 + [(5632, 2048)] * 2 + [(2048, 5632)] + [(2048,)] * 2
    shapes.append((32000, 2048))
    return shapes


def bench_sr_accum(micro=16):
    """Config 3.  The hooks of one micro-batch are queued (as inside a backward
    pass) and launched together; the timed region is that launch, with the
    gradients and accumulators resident in HBM.  The one-launch-per-hook path
    (hooks called outside a backward pass) is timed beside it."""
    import torch
    from muon_sr_amd import TritonSRAccumulator
    dev = "cuda:0"
    shapes = llama_small_shapes()
    params = [torch.nn.Parameter(torch.empty(s, device=dev, dtype=torch.bfloat16)) for s in shapes]
    numel = sum(p.numel() for p in params)
    gen = torch.Generator(device=dev)
    gsets = []
    for k in range(2):              # two seeded gradient sets, alternated across micro-batches
        gen.manual_seed(300 + k)
        gsets.append([(torch.randn(p.shape, device=dev, generator=gen) * 1e-4).to(torch.bfloat16) for p in params])

    class Holder(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.ps = torch.nn.ParameterList(params)

    model = Holder()
    TritonSRAccumulator.max_deferred_bytes = 1 << 40   # one launch per micro-batch
    host_s = []   # host time of the hook loop, one launch per hook

    def micro_batch(gs, evs=None, deferred=True):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        if deferred:
            with TritonSRAccumulator.deferred():
                for p, g in zip(params, gs):
                    p.grad = g
                    TritonSRAccumulator._accum_hook(p)
                s.record()
            e.record()
        else:
            s.record()
            h0 = time.perf_counter()
            for p, g in zip(params, gs):
                p.grad = g
                TritonSRAccumulator._accum_hook(p)
            host_s.append(time.perf_counter() - h0)
            e.record()
        if evs is not None:
            evs.append((s, e))

    for mb in range(micro):    # warm-up pass
        micro_batch(gsets[mb % 2])
    TritonSRAccumulator.reassign_grad_buffer(model)
    for p in params:
        p.grad = None
    sync()
    t0 = time.perf_counter()
    evs = []
    for mb in range(micro):
        micro_batch(gsets[mb % 2], evs)
    TritonSRAccumulator.reassign_grad_buffer(model)
    sync()
    wall = (time.perf_counter() - t0) * 1e3
    ms = [s.elapsed_time(e) for s, e in evs]
    steady = sum(ms[1:]) / (micro - 1)
    # one launch per hook, for comparison
    for p in params:
        p.grad = None
    evs1 = []
    for mb in range(4):
        micro_batch(gsets[mb % 2], evs1, deferred=False)
    TritonSRAccumulator.reassign_grad_buffer(model)
    sync()
    per_tensor = sum(s.elapsed_time(e) for s, e in evs1[1:]) / 3
    # host time per hook (the Python hook, the ctypes call and the launch), micro-batches 2-4
    host_us = sum(host_s[1:]) / len(host_s[1:]) / len(params) * 1e6
    out = dict(tensors=len(params), elements=numel, micro_batches=micro, total_ms=wall,
               first_microbatch_ms=ms[0], accumulate_ms=steady,
               accumulate_gbps=6.0 * numel / (steady * 1e6), first_gbps=4.0 * numel / (ms[0] * 1e6),
               per_tensor_launch_ms=per_tensor, per_tensor_launch_gbps=6.0 * numel / (per_tensor * 1e6),
               host_us_per_hook=host_us)
    del gsets, params, model
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------
# config 4: Muon step with batch_ns on 16 layers of d=2048 / ffn=5632 matrices
# ---------------------------------------------------------------------------

def ns_flops(shapes, steps=5):
    f = 0
    for s in shapes:
        m, n = min(s), max(s)
        f += steps * (4 * m * m * n + 2 * m ** 3)
    return f


def ns_exec_flops(shapes, steps=5, tile=256):
    """Flops the MFMAs execute (the textbook count less the tiles the symmetric products
    skip, on the 256-padded matrices): per iteration A = X X^T and B' = c A A + b A + a I
    compute the upper triangle of 256-tiles only, X' = B' X every tile.  (The diagonal
    residual term of X' adds 16 MFMAs per wave in the diagonal block, not counted.)"""
    f = 0
    for s in shapes:
        m, n = min(s), max(s)
        mp, np_ = -(-m // tile) * tile, -(-n // tile) * tile
        t, tn = mp // tile, np_ // tile
        tri = t * (t + 1) // 2
        f += steps * 2 * tile * tile * (tri * np_ + tri * mp + t * tn * mp)
    return f


def bench_muon(shapes, steps_timed, warmup, label):
    import torch
    from muon_sr_amd import TritonMuonSR
    dev = "cuda:0"
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    params = [torch.nn.Parameter((torch.randn(s, device=dev, generator=gen) * 0.02).to(torch.bfloat16))
              for s in shapes]
    gen.manual_seed(5)
    grads = [(torch.randn(s, device=dev, generator=gen) * 1e-3).to(torch.bfloat16) for s in shapes]
    opt = TritonMuonSR(params, lr=0.02, weight_decay=0.01, momentum=0.95, nesterov=True, ns_steps=5, batch_ns=True)
    for p, g in zip(params, grads):
        p.grad = g
    for _ in range(warmup):
        opt.step()
    sync()
    # The step's device time beside its wall time: events on the caller's stream right
    # before and after each step (the calls on the side stream join that stream before
    # the step returns; with the steps enqueued back to back, the device runs step k + 1
    # right after step k and the events bracket its own work).  Per chunk the library
    # call makes the momentum step in the Newton-Schulz prologue, the 5 iterations and
    # the parameter update in the last product's store.
    evs = []
    t0 = time.perf_counter()
    for _ in range(steps_timed):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        opt.step()
        e1.record()
        evs.append((e0, e1))
    sync()
    ms = (time.perf_counter() - t0) * 1e3 / steps_timed
    ns_ms = sum(x.elapsed_time(y) for x, y in evs) / steps_timed
    fl, fx = ns_flops(shapes), ns_exec_flops(shapes)
    # executed: the flops the MFMAs run over the step's device time; step_executed: the
    # same flops over the whole step's wall time (host work included)
    out = dict(matrices=len(shapes), ns_tflop=fl / 1e12, ms_per_step=ms, tflops=fl / (ms * 1e9),
               fused_calls_ms=ns_ms, fused_calls_tflops=fl / (ns_ms * 1e9), executed_tflop=fx / 1e12,
               executed_tflops=fx / (ns_ms * 1e9), step_executed_tflops=fx / (ms * 1e9))
    del opt, params, grads
    torch.cuda.empty_cache()
    out.update(bench_ns_alone(shapes))
    return out


def bench_ns_alone(shapes, reps=3):
    """Newton-Schulz alone (msr_newton_schulz, 5 iterations, bf16 in and out) over the same
    matrices, one call per shape group and chunk as the optimizer makes them: the step's
    Newton-Schulz without the momentum step and the parameter update.  Inputs resident in
    HBM; one workspace serves the calls in turn (one stream)."""
    import ctypes
    import torch
    from muon_sr_amd import _lib
    from muon_sr_amd.muon import NS_BATCH_NUMEL, NS_COEFFS
    L = _lib.lib()
    dev = "cuda:0"
    gen = torch.Generator(device=dev)
    gen.manual_seed(6)
    counts = {}
    for s in shapes:
        counts[s] = counts.get(s, 0) + 1
    calls, ws_bytes = [], 0
    for (r, c), k in counts.items():
        chunk = max(1, NS_BATCH_NUMEL // (r * c))
        for b0 in range(0, k, chunk):
            b = min(chunk, k - b0)
            x = (torch.randn(b, r, c, device=dev, generator=gen) * 1e-3).to(torch.bfloat16)
            nb = ctypes.c_size_t(0)
            _lib.check(L.msr_ns_workspace_bytes(b, r, c, ctypes.byref(nb)), "msr_ns_workspace_bytes")
            ws_bytes = max(ws_bytes, nb.value)
            calls.append((x, torch.empty_like(x), b, r, c))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    a, b_, c_ = NS_COEFFS

    def one_pass():
        for x, y, b, r, c in calls:
            _lib.check(L.msr_newton_schulz(x.data_ptr(), y.data_ptr(), b, r, c, 5, a, b_, c_, ws.data_ptr(), ws_bytes,
                                           stream), "msr_newton_schulz")
    one_pass()
    sync()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        one_pass()
    e1.record()
    sync()
    ms = e0.elapsed_time(e1) / reps
    fl, n_calls = ns_flops(shapes), len(calls)
    del calls, ws
    torch.cuda.empty_cache()
    return dict(ns_alone_ms=ms, ns_alone_tflops=fl / (ms * 1e9), ns_alone_calls=n_calls)


def bench_gemm_nt(reps=10):
    """The NS GEMM kernel on its own (diagnostic, not a default config): msr_gemm_nt, a batch of 64
    products 2048 x 2048 x 2048 (both operands K-contiguous, 4096 tiles of 256 x 256)."""
    import torch
    from muon_sr_amd import _lib
    L = _lib.lib()
    M = N = K = 2048
    batch = 64
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(10)
    P = torch.randn(batch, M, K, device="cuda:0", generator=gen).to(torch.bfloat16)
    Q = torch.randn(batch, N, K, device="cuda:0", generator=gen).to(torch.bfloat16)
    D = torch.empty(batch, M, N, device="cuda:0", dtype=torch.bfloat16)
    s = torch.cuda.current_stream().cuda_stream

    def run():
        _lib.check(L.msr_gemm_nt(P.data_ptr(), K, M * K, Q.data_ptr(), K, N * K, None, 0, 0, D.data_ptr(), N, M * N,
                                 M, N, K, batch, 1.0, 0.0, 0.0, s), "msr_gemm_nt")
    for _ in range(3):
        run()
    evs = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        run()
        e1.record()
        evs.append((e0, e1))
    sync()
    ms = statistics.median(a.elapsed_time(b) for a, b in evs)
    fl = 2.0 * M * N * K * batch
    del P, Q, D
    torch.cuda.empty_cache()
    return dict(batch=batch, m=M, n=N, k=K, ms=ms, tflops=fl / (ms * 1e9))


def config4_shapes():
    return [(2048, 2048)] * 64 + [(5632, 2048)] * 32 + [(2048, 5632)] * 16


# ---------------------------------------------------------------------------
# config 5: full hybrid step on Llama-3-8B shapes (Muon + 8-bit AdamW groups)
# ---------------------------------------------------------------------------

def llama8b_muon_shapes():
    d, ffn, kv = 4096, 14336, 1024
    return [(d, d), (kv, d), (kv, d), (d, d), (ffn, d), (ffn, d), (d, ffn)] * 32


def bench_full(steps_timed, warmup):
    import torch
    from muon_sr_amd import TritonMuonSRWithAuxAdam
    dev = "cuda:0"
    gen = torch.Generator(device=dev)
    gen.manual_seed(8)
    mk = lambda s: torch.nn.Parameter((torch.randn(s, device=dev, generator=gen) * 0.02).to(torch.bfloat16))  # noqa
    d, ffn, kv, vocab = 4096, 14336, 1024, 128256
    muon, adam = [], []
    embed = mk((vocab, d))
    adam.append(embed)
    for _ in range(32):
        muon += [mk((d, d)), mk((kv, d)), mk((kv, d)), mk((d, d)), mk((ffn, d)), mk((ffn, d)), mk((d, ffn))]
        adam += [mk((d,)), mk((d,))]
    adam += [mk((d,)), mk((vocab, d))]
    opt = TritonMuonSRWithAuxAdam([
        dict(params=muon, use_muon=True, lr=0.02, weight_decay=0.01),
        dict(params=adam, use_muon=False, lr=3e-4, betas=(0.9, 0.95), eps=1e-10, weight_decay=0.01, optim_bits=8),
    ], batch_ns=True)
    gen.manual_seed(9)
    for p in muon + adam:
        p.grad = (torch.randn(p.shape, device=dev, generator=gen) * 1e-3).to(torch.bfloat16)
    for _ in range(warmup):
        opt.step()
    sync()
    t0 = time.perf_counter()
    for _ in range(steps_timed):
        opt.step()
    sync()
    ms = (time.perf_counter() - t0) * 1e3 / steps_timed
    fl, fx = ns_flops([tuple(p.shape) for p in muon]), ns_exec_flops([tuple(p.shape) for p in muon])
    # over the whole hybrid step's wall time (the 8-bit AdamW group and host work included)
    out = dict(muon_matrices=len(muon), adamw_tensors=len(adam), ns_tflop=fl / 1e12, ms_per_step=ms,
               ns_tflops_effective=fl / (ms * 1e9), executed_tflop=fx / 1e12, step_executed_tflops=fx / (ms * 1e9))
    shapes = [tuple(p.shape) for p in muon]
    del opt, muon, adam
    torch.cuda.empty_cache()
    out.update(bench_ns_alone(shapes))
    return out


def bench_centralize(reps=10):
    """TritonAdamW's gradient centralization on a Llama-3-8B embedding-sized bf16
    gradient (128256 x 4096): this library's fused kernels against the
    reference's torch op sequence (muon_sr/triton_adamw.py:180-186) on the same
    GPU.  Algorithmic traffic 6 B/element (read g twice, write g')."""
    import torch
    from muon_sr_amd.adamw import centralize
    dev = "cuda:0"
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    g = (torch.randn(128256, 4096, device=dev, generator=gen) * 1e-3).to(torch.bfloat16)

    def ref_ops():
        x = g.to(torch.float32)
        x.sub_(x.mean(dim=tuple(range(1, x.dim())), keepdim=True).mul_(0.5))
        return x.to(torch.bfloat16)

    def timed(fn):
        for _ in range(2):
            fn()
        sync()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        sync()
        return s.elapsed_time(e) / reps

    ms = timed(lambda: centralize(g, 0.5))
    ref_ms = timed(ref_ops)
    n = g.numel()
    out = dict(elements=n, ms=ms, gbps=6.0 * n / (ms * 1e6), reference_torch_ops_ms=ref_ms,
               speedup_vs_reference_ops=ref_ms / ms)
    del g
    torch.cuda.empty_cache()
    return out


def bench_wgrad(reps=5, tokens=8192):
    """Weight gradients of one Llama-3-8B decoder layer (q, k, v, o, gate, up,
    down) over `tokens` tokens, accumulated into bf16 buffers with SR: this
    library's fused kernel (msr_linear_wgrad_sr_accum: dW never written)
    against what the reference's hook does after autograd, a torch bf16 GEMM
    writing dW then the accumulation (msr_sr_accum).  Flops 2 * tokens * in *
    out per weight."""
    import random
    import torch
    from muon_sr_amd import _lib
    from muon_sr_amd.linear import linear_wgrad_sr_accum
    dev = "cuda:0"
    gen = torch.Generator(device=dev)
    gen.manual_seed(12)
    d, kv, ffn = 4096, 1024, 14336
    shapes = [(d, d), (kv, d), (kv, d), (d, d), (ffn, d), (ffn, d), (d, ffn)]   # (out, in)
    xs = {fin: (torch.randn(tokens, fin, device=dev, generator=gen)).to(torch.bfloat16) for fin in (d, ffn)}
    dys = {fout: (torch.randn(tokens, fout, device=dev, generator=gen) * 1e-3).to(torch.bfloat16)
           for fout in (d, kv, ffn)}
    ws = [torch.nn.Parameter(torch.zeros(o, i, device=dev, dtype=torch.bfloat16)) for o, i in shapes]
    accs = [torch.zeros(o, i, device=dev, dtype=torch.bfloat16) for o, i in shapes]
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream

    def fused():
        for w, (o, i) in zip(ws, shapes):
            assert linear_wgrad_sr_accum(w, xs[i], dys[o], seed=random.getrandbits(32))

    def unfused():
        for acc, (o, i) in zip(accs, shapes):
            dw = dys[o].t() @ xs[i]
            _lib.check(L.msr_sr_accum(acc.data_ptr(), dw.data_ptr(), 0, dw.numel(), random.getrandbits(32), 0,
                                      _lib.noise_mode(), None, stream), "msr_sr_accum")

    def timed(fn):
        fn()
        sync()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        sync()
        return s.elapsed_time(e) / reps

    ms, ref_ms = timed(fused), timed(unfused)
    fl = sum(2.0 * tokens * o * i for o, i in shapes)
    out = dict(tokens=tokens, weights=len(shapes), tflop=fl / 1e12, fused_ms=ms, fused_tflops=fl / (ms * 1e9),
               torch_gemm_then_accum_ms=ref_ms, speedup=ref_ms / ms)
    del xs, dys, ws, accs
    torch.cuda.empty_cache()
    return out


def device_copy_gbps(reps=20):
    """A reference streaming rate measured in the same run: a 2 GiB -> 2 GiB device copy
    (torch copy_, i.e. the runtime's device-to-device copy), median of `reps` launches."""
    import torch
    n = 1 << 29
    a = torch.ones(n, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    evs = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        b.copy_(a)
        e1.record()
        evs.append((e0, e1))
    sync()
    ms = statistics.median(x.elapsed_time(y) for x, y in evs)
    del a, b
    torch.cuda.empty_cache()
    return 2.0 * 4 * n / (ms * 1e6)


def copy_calibration():
    """A plain device copy of known size (2^28 fp32: 1 GiB read + 1 GiB written per
    launch).  Profiled with FETCH_SIZE / WRITE_SIZE, it gives the factor that turns
    those counters into bytes on this GPU."""
    import torch
    n = 1 << 28
    a = torch.ones(n, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    sync()
    print(json.dumps({"copy_calibration_bytes_read": n * 4, "copy_calibration_bytes_written": n * 4,
                      "launches": 3}), flush=True)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "adamw8bit_2e28_hbm_traffic.txt")


def measured_traffic():
    """HBM bytes per launch of the 8-bit kernel from the committed counter summary
    (FETCH_SIZE and WRITE_SIZE passes, scaled by the copy calibration), or None."""
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("hbm_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


COUNTERS_FILE = os.path.join(ROOT, "profiles", "adamw8bit_2e28_counters.md")


def measured_valu_issue():
    """Fraction of the 8-bit kernel's time that its VALU instructions take to issue, from the
    committed counter summary (SQ_INSTS_VALU per pair x 4 cycles / SIMDs / clock, against
    the dispatch's duration in the same counter run), or None."""
    try:
        for line in open(COUNTERS_FILE):
            if line.startswith("valu_issue_fraction:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="adamw8bit,probe8,sr_accum,ns,centralize,wgrad,full")
    ap.add_argument("--noise", default="philox8", choices=["philox8", "triton"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run the plain copy used to calibrate the HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU: every box has one MI355X and the optimizer step "
                                   "has no multi-GPU path here; run with --gpus 1"}))
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration()
        return
    import torch
    import muon_sr_amd
    muon_sr_amd.set_sr_noise(args.noise)
    torch.backends.cuda.matmul.allow_tf32 = False
    todo = set(args.configs.split(","))
    log(f"device: {torch.cuda.get_device_name(0)}  noise: {args.noise}")

    r8 = bench_adamw8bit(args.steps, args.warmup)
    log(f"adamw8bit: {r8}")
    copy_gbps = device_copy_gbps()
    log(f"device copy 2 GiB -> 2 GiB: {copy_gbps:.0f} GB/s")
    configs = {"adamw8bit_2^28": {k: round(v, 4) for k, v in r8.items()}}
    probe = None
    if "probe8" in todo:
        probe = bench_stream8_probe()
        log(f"8-bit access pattern without the arithmetic: best {probe['best']}")
        configs["stream8_probe_2^28"] = probe
    other = "triton" if args.noise == "philox8" else "philox8"
    if "adamw8bit" in todo:   # the same step with the other noise stream (triton: the reference's bits)
        muon_sr_amd.set_sr_noise(other)
        r = bench_adamw8bit(max(5, args.steps // 2), 2)
        muon_sr_amd.set_sr_noise(args.noise)
        log(f"adamw8bit ({other} noise): {r}")
        configs[f"adamw8bit_2^28_{other}_noise"] = {k: round(v, 4) for k, v in r.items()}
    if "sr_accum" in todo:
        r = bench_sr_accum()
        log(f"sr_accum: {r}")
        configs["sr_accum_24L_d2048"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
        muon_sr_amd.set_sr_noise(other)
        r = bench_sr_accum(micro=6)
        muon_sr_amd.set_sr_noise(args.noise)
        log(f"sr_accum ({other} noise): {r}")
        configs[f"sr_accum_24L_d2048_{other}_noise"] = {k: round(v, 4) if isinstance(v, float) else v
                                                        for k, v in r.items()}
    if "ns" in todo:
        r = bench_muon(config4_shapes(), steps_timed=5, warmup=2, label="config4")
        log(f"muon config4: {r}")
        configs["muon_ns_16L_d2048"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
    if "gemm" in todo:
        r = bench_gemm_nt()
        log(f"gemm_nt: {r}")
        configs["gemm_nt_64x2048^3"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
    if "centralize" in todo:
        r = bench_centralize()
        log(f"centralize: {r}")
        configs["centralize_embed_128256x4096"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
    if "wgrad" in todo:
        r = bench_wgrad()
        log(f"wgrad: {r}")
        configs["wgrad_sr_accum_llama3_8b_layer"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
    if "full" in todo:
        r = bench_full(steps_timed=5, warmup=2)
        log(f"full hybrid: {r}")
        configs["hybrid_llama3_8b"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_adamw8bit()
        log(f"cpu baseline (C oracle, 8-bit): {cpu}")
        tb = cpu_baselines_torch()
        log(f"cpu baseline (torch restatement): {tb}")
        configs["cpu_torch_restatement"] = tb
    kernel_gbps = r8["kernel_gbps"]
    line = {
        "metric": "8-bit AdamW step GB/s (% HBM peak); Muon NS bf16 TFLOP/s; full step ms",
        "value": round(r8["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r8["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 arithmetic (bf16 params/grads, u8 moment codes)",
        "data": "synthetic (seeded normal params/grads, resident in HBM)",
        "config": {"workload": "8-bit blockwise AdamW step, one flat bf16 parameter of 2^28 elements "
                               "(BASELINE.json configs[1])",
                   "elements": N8, "block_size": 256, "lr": 3e-4, "betas": [0.9, 0.95], "eps": 1e-10,
                   "weight_decay": 0.01, "sr_noise": args.noise, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(kernel_gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(kernel_gbps / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(),
                     "traffic_source": "profiles/adamw8bit_2e28_hbm_traffic.txt: rocprofv3 --pmc FETCH_SIZE and "
                                       "WRITE_SIZE runs of this kernel, scaled by a copy calibration (committed "
                                       "counter run, not measured in this run)",
                     "kernel": "adamw8bit_fast_kernel", "kernel_ms": round(r8["kernel_ms"], 4),
                     "kernel_ms_stat": "median of the timed launches (HIP events on the launch stream)",
                     "bytes_per_launch": r8["bytes_per_step"],
                     # context, not the peak: the runtime's own device copy (half reads, half writes),
                     # measured in this run
                     "device_copy_gbps_this_run": round(copy_gbps, 1),
                     # what binds the kernel below the HBM peak: the issue time of its VALU instructions
                     "valu_issue_frac_of_kernel_time": measured_valu_issue(),
                     "valu_issue_source": "profiles/adamw8bit_2e28_counters.md: rocprofv3 --pmc SQ_INSTS_VALU, "
                                          "GRBM_GUI_ACTIVE runs of this kernel (committed counter run, not "
                                          "measured in this run)"},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    if probe is not None:
        # the same accesses without the arithmetic, best over occupancy and grid, this run
        line["roofline"]["pattern_ceiling_gbps"] = probe["best_gbps"]
        line["roofline"]["frac_of_pattern_ceiling"] = round(kernel_gbps / probe["best_gbps"], 4)
    k_other = f"adamw8bit_2^28_{other}_noise"
    if k_other in configs:   # the same kernel with the other noise stream
        line["roofline"][f"frac_{other}_noise"] = round(configs[k_other]["kernel_gbps"] / HBM_PEAK_GBPS, 4)
    # config 3, SR accumulation (HBM-bound, 6 B per element and micro-batch): queued hooks
    # (one launch per up to 80 tensors) and one launch per hook, in both noise streams
    sr = {}
    for key, tag in (("sr_accum_24L_d2048", args.noise), (f"sr_accum_24L_d2048_{other}_noise", other)):
        if key in configs:
            c = configs[key]
            sr[tag] = {"queued_gbps": c["accumulate_gbps"], "queued_frac": round(c["accumulate_gbps"] / HBM_PEAK_GBPS, 4),
                       "per_hook_gbps": c["per_tensor_launch_gbps"],
                       "per_hook_frac": round(c["per_tensor_launch_gbps"] / HBM_PEAK_GBPS, 4),
                       "host_us_per_hook": c["host_us_per_hook"]}
    if sr:
        line["roofline_sr_accum"] = {"bound": "hbm", "peak": HBM_PEAK_GBPS, "unit": "GB/s", "noise": sr}
    if "muon_ns_16L_d2048" in configs:
        line["ns_tflops"] = configs["muon_ns_16L_d2048"]["tflops"]
        line["ns_frac_of_bf16_peak"] = round(configs["muon_ns_16L_d2048"]["tflops"] / BF16_PEAK_TFLOPS, 4)
        line["fused_calls_frac_of_bf16_peak"] = round(configs["muon_ns_16L_d2048"]["fused_calls_tflops"] / BF16_PEAK_TFLOPS,
                                                   4)
        # what the matrix cores execute (the symmetric products skip their lower 256-tiles),
        # over the fused calls' launch time
        line["ns_executed_frac_of_bf16_peak"] = round(configs["muon_ns_16L_d2048"]["executed_tflops"] / BF16_PEAK_TFLOPS,
                                                   4)
        # Newton-Schulz alone on the same matrices (no momentum step, no parameter update)
        line["ns_alone_frac_of_bf16_peak"] = round(configs["muon_ns_16L_d2048"]["ns_alone_tflops"] / BF16_PEAK_TFLOPS,
                                                4)
    if "hybrid_llama3_8b" in configs:
        line["full_step_ms"] = configs["hybrid_llama3_8b"]["ms_per_step"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

"""msr_muon_fused_steps: the whole Muon step of several shape groups in one call.

Each group's matrices share the Newton-Schulz product launches with the other
groups' (every group's shape is group 0's or its transpose).  The call must equal,
bit for bit, one msr_muon_fused_step per group with the same arguments (that entry
point is pinned to prepare + Newton-Schulz + apply and, through them, to the
oracle): momentum rows and parameters.  Argument errors are checked on the CPU
(tests/test_abi.py).
"""
import ctypes

import pytest
import torch

import oracle as O
from _gpu import DEV, check, need_gpu, ptr_array, stream
from muon_sr_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return need_gpu()


@pytest.fixture
def noise():
    """Select the SR noise stream for one test and restore it afterwards."""
    import muon_sr_amd
    old = muon_sr_amd.get_sr_noise()
    yield muon_sr_amd.set_sr_noise
    muon_sr_amd.set_sr_noise(old)


def _bits(t):
    return t.detach().contiguous().view(torch.int16)


class _Group:
    """k matrices of rows x cols: gradients, a momentum stack of first + k rows (the
    call's rows start at `first`), parameters, seeds."""

    def __init__(self, gen, k, rows, cols, first, f32, seed0):
        self.k, self.rows, self.cols, self.first = k, rows, cols, first
        g = [torch.randn(rows, cols, device=DEV, generator=gen) * 1e-3 for _ in range(k)]
        self.grads = g if f32 else [x.to(torch.bfloat16) for x in g]
        self.f32 = int(f32)
        self.stack0 = (torch.randn(first + k, rows, cols, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16)
        self.params0 = (torch.randn(k, rows, cols, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
        self.pseed = (0x2545F491 + 977 * seed0) & 0xFFFFFFFF
        self.seeds = [(0x9E3779B9 * (i + 3 + seed0)) & 0xFFFFFFFF for i in range(k)]
        self.scale = max(1.0, rows / cols) ** 0.5
        self.reset()

    def reset(self):
        self.stack = self.stack0.clone()
        self.params = self.params0.clone()


def _ws(L, batch, rows, cols):
    nb = ctypes.c_size_t(0)
    check(L, L.msr_ns_workspace_bytes(batch, rows, cols, ctypes.byref(nb)), "workspace")
    return torch.empty(nb.value, dtype=torch.uint8, device=DEV), nb.value


def _per_group(L, groups, mode, beta, nest, lr, wd):
    from muon_sr_amd.muon import NS_COEFFS
    a, b, c = NS_COEFFS
    for gr in groups:
        ws, nb = _ws(L, gr.k, gr.rows, gr.cols)
        check(L, L.msr_muon_fused_step(ptr_array([x.data_ptr() for x in gr.grads]), gr.f32,
                                       gr.stack[gr.first].data_ptr(), gr.first, gr.k, gr.rows, gr.cols, beta, int(nest),
                                       gr.pseed, 5, a, b, c, None,
                                       ptr_array([gr.params[i].data_ptr() for i in range(gr.k)]),
                                       ptr_array(gr.seeds, ctypes.c_uint32), lr, wd, gr.scale, mode, None, None,
                                       ws.data_ptr(), nb, stream()), "msr_muon_fused_step")


def _grouped(L, groups, mode, beta, nest, lr, wd):
    from muon_sr_amd.muon import NS_COEFFS
    a, b, c = NS_COEFFS
    ws, nb = _ws(L, sum(gr.k for gr in groups), groups[0].rows, groups[0].cols)
    keep = []   # the host tables, alive until the call returns
    arr = (_lib.MuonGroup * len(groups))()
    for i, gr in enumerate(groups):
        gt = ptr_array([x.data_ptr() for x in gr.grads])
        pt = ptr_array([gr.params[j].data_ptr() for j in range(gr.k)])
        st = ptr_array(gr.seeds, ctypes.c_uint32)
        keep += [gt, pt, st]
        arr[i] = _lib.MuonGroup(ctypes.addressof(gt), gr.stack[gr.first].data_ptr(), ctypes.addressof(pt),
                                ctypes.addressof(st), gr.first, gr.k, gr.rows, gr.cols, gr.pseed, gr.f32, gr.scale)
    return L.msr_muon_fused_steps(arr, len(groups), beta, int(nest), 5, a, b, c, lr, wd, mode, ws.data_ptr(), nb,
                                  stream())


# (k, rows, cols, first, f32) per group
CASES = {
    "wide+tall": [(3, 256, 512, 0, False), (2, 512, 256, 0, False)],
    "tall+wide ragged, offsets, fp32": [(2, 320, 200, 1, True), (1, 200, 320, 2, False), (2, 320, 200, 0, False)],
    "one group": [(4, 384, 640, 0, False)],
    # more tiles than work-groups: the products draw tiles from the workspace counters
    "many tiles": [(5, 2048, 5632, 0, False), (3, 5632, 2048, 0, False)],
    # more matrices than one prologue launch (96) and one apply launch (128) take
    "many matrices": [(130, 256, 320, 0, False), (40, 320, 256, 3, False)],
}


@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8])
@pytest.mark.parametrize("case", list(CASES))
def test_fused_steps_equal_one_call_per_group(L, case, mode):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(len(case) * 31 + mode)
    groups = [_Group(gen, k, r, c, f, f32, i) for i, (k, r, c, f, f32) in enumerate(CASES[case])]
    nest = case != "one group"
    beta, lr, wd = 0.95, 0.02, 0.01
    _per_group(L, groups, mode, beta, nest, lr, wd)
    torch.cuda.synchronize()
    ref = [(gr.stack.clone(), gr.params.clone()) for gr in groups]
    for gr in groups:
        gr.reset()
    check(L, _grouped(L, groups, mode, beta, nest, lr, wd), "msr_muon_fused_steps")
    torch.cuda.synchronize()
    for i, (gr, (st, pr)) in enumerate(zip(groups, ref)):
        assert torch.equal(_bits(gr.stack), _bits(st)), (case, i, "momentum")
        assert torch.equal(_bits(gr.params), _bits(pr)), (case, i, "params")
        assert not torch.equal(_bits(gr.params), _bits(gr.params0)), (case, i, "no update")


@pytest.mark.parametrize("mode_name", ["triton", "philox8"])
def test_batch_step_merged_equals_chunked(L, noise, mode_name, monkeypatch):
    """TritonMuonSR(batch_ns=True) with a pair of transposed shape groups: the step that
    takes both groups in one call (msr_muon_fused_steps) equals, bit for bit, the step
    with a chunk limit so small that each group runs alone in chunks of two matrices."""
    from muon_sr_amd import TritonMuonSR
    from muon_sr_amd import muon as M
    noise(mode_name)
    shapes = [(256, 512), (512, 256), (256, 512), (384, 384), (512, 256), (256, 512)]
    gen = torch.Generator(device=DEV)
    gen.manual_seed(17)
    p0 = [(torch.randn(s, device=DEV, generator=gen) * 0.02).to(torch.bfloat16) for s in shapes]
    grads = [[(torch.randn(s, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16) for s in shapes]
             for _ in range(2)]
    calls = []
    real = M._fused_steps
    monkeypatch.setattr(M, "_fused_steps", lambda *a, **k: (calls.append(1), real(*a, **k)))

    def run(chunk):
        monkeypatch.setattr(M, "NS_BATCH_NUMEL", chunk)
        ps = [torch.nn.Parameter(x.clone()) for x in p0]
        opt = TritonMuonSR(ps, lr=0.02, weight_decay=0.01, batch_ns=True)
        for step in range(2):
            for p, g in zip(ps, grads[step]):
                p.grad = g
            opt.step()
        torch.cuda.synchronize()
        return [p.detach().clone() for p in ps], [opt.state[p]["momentum_buffer"].clone() for p in ps]

    merged = run(1 << 30)
    assert len(calls) == 2, "one merged call per step expected"
    chunked = run(2 * 256 * 512)
    assert len(calls) == 2, "the small chunk limit must not merge"
    for i in range(len(shapes)):
        assert torch.equal(_bits(merged[0][i]), _bits(chunked[0][i])), ("param", i)
        assert torch.equal(_bits(merged[1][i]), _bits(chunked[1][i])), ("momentum", i)


@pytest.mark.parametrize("mode_name", ["triton", "philox8"])
def test_batch_step_two_streams_equals_one(L, noise, mode_name, monkeypatch):
    """The fused calls of a batch_ns step alternate between the caller's stream and a side
    stream; three steps with several calls each (a transposed pair, a square group and a
    group cut into chunks) equal, bit for bit, the same steps on one stream, and the
    caller's stream sees the results without a device-wide synchronisation."""
    from muon_sr_amd import TritonMuonSR
    from muon_sr_amd import muon as M
    noise(mode_name)
    shapes = [(256, 512), (512, 256), (384, 384), (256, 512), (128, 640), (128, 640), (128, 640)]
    gen = torch.Generator(device=DEV)
    gen.manual_seed(23)
    p0 = [(torch.randn(s, device=DEV, generator=gen) * 0.02).to(torch.bfloat16) for s in shapes]
    grads = [[(torch.randn(s, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16) for s in shapes]
             for _ in range(3)]
    monkeypatch.setattr(M, "NS_BATCH_NUMEL", 2 * 128 * 640 + 1000)   # the 128 x 640 group runs in 2 chunks
    n_calls = []
    real = M._run_calls
    monkeypatch.setattr(M, "_run_calls", lambda calls, dev: (n_calls.append(len(calls)), real(calls, dev)))
    assert sum(p.numel() for p in p0) <= M.TWO_STREAMS_MAX_NUMEL

    def run(two):
        monkeypatch.setattr(M, "TWO_STREAMS", two)
        ps = [torch.nn.Parameter(x.clone()) for x in p0]
        opt = TritonMuonSR(ps, lr=0.02, weight_decay=0.01, batch_ns=True)
        for step in range(3):
            for p, g in zip(ps, grads[step]):
                p.grad = g.clone()
            opt.step()
            for p in ps:
                p.grad = None   # gradients freed while the side stream may still run
        # read on the caller's stream: ordered after the side stream by the step's join
        out = [p.detach().clone() for p in ps], [opt.state[p]["momentum_buffer"].clone() for p in ps]
        torch.cuda.synchronize()
        return out

    one = run(False)
    two = run(True)
    assert n_calls and min(n_calls) >= 3, n_calls
    for i in range(len(shapes)):
        assert torch.equal(_bits(one[0][i]), _bits(two[0][i])), ("param", i)
        assert torch.equal(_bits(one[1][i]), _bits(two[1][i])), ("momentum", i)

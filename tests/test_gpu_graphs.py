"""The optimizer-step entry points under HIP graph capture.

Nothing in the library allocates, frees, clears memory or synchronizes inside an
entry point (workspaces are the caller's), so a caller can capture a step into a
graph and replay it.  Each test captures one call, replays the graph three times with
eager work and synchronizations between the replays, and checks every replay against
the same call run eagerly on a copy of the same state, bit for bit.
"""
import ctypes

import pytest
import torch

import oracle as O
from _gpu import DEV, check, need_gpu, ptr_array

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return need_gpu()


def _bits(t):
    return t.detach().contiguous().view(torch.uint8)


def _same(xs, ys):
    return all(torch.equal(_bits(x), _bits(y)) for x, y in zip(xs, ys))


def _eager_work():
    x = torch.randn(1 << 20, device=DEV)
    (x * 2.0 + 1.0).sum()
    torch.cuda.synchronize()


def _replay_vs_eager(call, state, replays=3):
    """call(tensors, stream) runs one step in place on `tensors`.  Returns after
    checking `replays` graph replays against as many eager calls."""
    eager = [t.clone() for t in state]
    graphed = [t.clone() for t in state]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # a first eager call on a side stream, as torch recommends before capture
        warm = [t.clone() for t in state]
        call(warm, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(graphed, torch.cuda.current_stream().cuda_stream)
    for r in range(replays):
        g.replay()
        _eager_work()
        call(eager, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert _same(graphed, eager), r


@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8])
def test_adamw8bit_step_in_hip_graph(L, mode):
    from muon_sr_amd.adamw_8bit import create_dynamic_map
    n, block = (1 << 20) + 300, 256
    gen = torch.Generator(device=DEV)
    gen.manual_seed(21 + mode)
    p = (torch.randn(n, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    g = (torch.randn(n, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16)
    s1 = torch.full((n,), 127, dtype=torch.uint8, device=DEV)
    s2 = torch.zeros(n, dtype=torch.uint8, device=DEV)
    nb = (n + block - 1) // block
    a1 = torch.zeros(nb, device=DEV)
    a2 = torch.zeros(nb, device=DEV)
    q1, q2 = create_dynamic_map(True).to(DEV), create_dynamic_map(False).to(DEV)

    def call(t, stream):
        pp, ss1, ss2, aa1, aa2 = t
        check(L, L.msr_adamw8bit_step(pp.data_ptr(), g.data_ptr(), ss1.data_ptr(), ss2.data_ptr(), aa1.data_ptr(),
                                      aa2.data_ptr(), q1.data_ptr(), q2.data_ptr(), None, n, block, 1, 3e-4, 0.9,
                                      0.95, 1e-10, 0.01, 0.1, 0.05, 1234567, mode, None, stream), "adamw8bit")
    _replay_vs_eager(call, [p, s1, s2, a1, a2])


@pytest.mark.parametrize("k,rows,cols", [(3, 512, 768), (3, 768, 512), (8, 2048, 5632)])
def test_muon_fused_step_in_hip_graph(L, k, rows, cols):
    """Momentum step, Newton-Schulz and the parameter update (msr_muon_fused_step) of
    a chunk of k matrices, wide and tall.  8 x 2048 x 5632 gives the products more
    tiles than work-groups, so their work-groups draw tiles from the counters in the
    workspace (whole matrices per XCD for A and B', tiles spread for X')."""
    from muon_sr_amd.muon import NS_COEFFS
    gen = torch.Generator(device=DEV)
    gen.manual_seed(rows + cols)
    grads = [(torch.randn(rows, cols, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16) for _ in range(k)]
    buf = (torch.randn(k, rows, cols, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16)
    params = (torch.randn(k, rows, cols, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    nbytes = ctypes.c_size_t(0)
    check(L, L.msr_ns_workspace_bytes(k, rows, cols, ctypes.byref(nbytes)), "workspace")
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=DEV)
    a, b, c = NS_COEFFS
    gtab = ptr_array([t.data_ptr() for t in grads])
    seeds = ptr_array([11 * (i + 1) for i in range(k)], ctypes.c_uint32)
    scale = max(1.0, rows / cols) ** 0.5

    def call(t, stream):
        bb, pp = t
        ptab = ptr_array([pp[i].data_ptr() for i in range(k)])
        check(L, L.msr_muon_fused_step(gtab, 0, bb.data_ptr(), 0, k, rows, cols, 0.95, 1, 777, 5, a, b, c, None, ptab,
                                       seeds, 0.02, 0.01, scale, O.NOISE_PHILOX8, None, None, ws.data_ptr(),
                                       nbytes.value, stream), "fused step")
    _replay_vs_eager(call, [buf, params])


def test_muon_fused_steps_in_hip_graph(L):
    """msr_muon_fused_steps of a wide and a tall shape group (3 x 2048 x 5632 and 5 x 5632 x
    2048: more tiles than work-groups, so the products draw tiles from the workspace
    counters) captured and replayed."""
    from muon_sr_amd import _lib
    from muon_sr_amd.muon import NS_COEFFS
    shapes = [(3, 2048, 5632), (5, 5632, 2048)]
    gen = torch.Generator(device=DEV)
    gen.manual_seed(29)
    grads = [[(torch.randn(r, c, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16) for _ in range(k)]
             for k, r, c in shapes]
    bufs = [(torch.randn(k, r, c, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16) for k, r, c in shapes]
    params = [(torch.randn(k, r, c, device=DEV, generator=gen) * 0.02).to(torch.bfloat16) for k, r, c in shapes]
    nbytes = ctypes.c_size_t(0)
    check(L, L.msr_ns_workspace_bytes(8, 2048, 5632, ctypes.byref(nbytes)), "workspace")
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=DEV)
    a, b, c = NS_COEFFS
    gtabs = [ptr_array([g.data_ptr() for g in gs]) for gs in grads]
    stabs = [ptr_array([7 * (i + 1) + 100 * j for i in range(k)], ctypes.c_uint32) for j, (k, _, _) in enumerate(shapes)]

    def call(t, stream):
        keep = []
        arr = (_lib.MuonGroup * 2)()
        for j, (k, r, cc) in enumerate(shapes):
            bb, pp = t[j], t[2 + j]
            ptab = ptr_array([pp[i].data_ptr() for i in range(k)])
            keep.append(ptab)
            arr[j] = _lib.MuonGroup(ctypes.addressof(gtabs[j]), bb.data_ptr(), ctypes.addressof(ptab),
                                    ctypes.addressof(stabs[j]), 0, k, r, cc, 1234 + j, 0, max(1.0, r / cc) ** 0.5)
        check(L, L.msr_muon_fused_steps(arr, 2, 0.95, 1, 5, a, b, c, 0.02, 0.01, O.NOISE_PHILOX8, ws.data_ptr(),
                                        nbytes.value, stream), "fused steps")
    _replay_vs_eager(call, bufs + params)

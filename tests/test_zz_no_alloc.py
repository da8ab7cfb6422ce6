"""msr_centralize_bf16_noalloc: the allocation-free variant of msr_centralize_bf16
(its workspace is a static device array of the library).  No counterpart in the
reference; checked against the workspace entry point, bit for bit, on two calls in
a row (the second smaller, so it reads scratch the first call left behind), in
place and out of place, one and several chunks per row."""
import ctypes

import pytest
import torch

from _gpu import DEV, check, need_gpu, stream

pytestmark = pytest.mark.gpu

MSR_ERR_WORKSPACE = 1004
SCRATCH_BYTES = 4 << 20


@pytest.fixture(scope="module")
def L():
    return need_gpu()


def with_workspace(L, g, alpha, out):
    rows, cols = g.shape
    nb = ctypes.c_size_t(0)
    check(L, L.msr_centralize_workspace_bytes(rows, cols, ctypes.byref(nb)), "workspace bytes")
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    check(L, L.msr_centralize_bf16(g.data_ptr(), out.data_ptr(), rows, cols, alpha, ws.data_ptr(), nb.value,
                                   stream()), "msr_centralize_bf16")


@pytest.mark.parametrize("in_place", [False, True])
def test_noalloc_equals_workspace_entry(L, in_place):
    gen = torch.Generator(device=DEV)
    gen.manual_seed(3 + in_place)
    # (rows, cols): 3 chunks per row, then a smaller call with 2 chunks; then one chunk
    # per row at many rows, then fewer rows
    for rows, cols, alpha in [(700, 40000, 1.0), (300, 20000, 0.37), (100000, 4096, 0.5), (5000, 1000, 1.0)]:
        g = (torch.randn(rows, cols, device=DEV, generator=gen) * 1e-3
             + torch.randn(rows, 1, device=DEV, generator=gen) * 5e-4).to(torch.bfloat16)
        ref = torch.empty_like(g)
        with_workspace(L, g, alpha, ref)
        out = g.clone() if in_place else torch.empty_like(g)
        src = out if in_place else g
        check(L, L.msr_centralize_bf16_noalloc(src.data_ptr(), out.data_ptr(), rows, cols, alpha, stream()),
              "msr_centralize_bf16_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (rows, cols)


def test_noalloc_rejects_sizes_beyond_scratch(L):
    g = torch.zeros(8, device=DEV, dtype=torch.bfloat16)
    rows = SCRATCH_BYTES // 8 + 1           # partials + means: 8 bytes per row at one chunk per row
    rc = L.msr_centralize_bf16_noalloc(g.data_ptr(), g.data_ptr(), rows, 8, 1.0, stream())
    assert rc == MSR_ERR_WORKSPACE and b"scratch" in L.msr_last_error()
    torch.cuda.synchronize()

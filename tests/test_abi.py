"""CPU checks of the C ABI: the library loads and exports every declared symbol.

No kernel is launched (no GPU here); argument validation paths that return
before any HIP call are exercised.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "muon_sr_amd.h")
LIB = os.path.join(ROOT, "muon_sr_amd", "libmuon_sr_amd.so")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char \*)\s*(msr_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built; run __graft_entry__.build()")
    from muon_sr_amd import _lib
    return _lib.lib()


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("msr_sr_accum", "msr_adamw8bit_step", "msr_adamw_bf16_step", "msr_muon_prepare", "msr_muon_apply",
              "msr_newton_schulz", "msr_ns_workspace_bytes", "msr_last_error", "msr_version"):
        assert s in syms


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(LIB)
    for s in declared_symbols():
        assert hasattr(raw, s), s


def test_python_signatures_cover_header(lib):
    from muon_sr_amd import _lib
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_argument_validation_without_gpu(lib):
    assert lib.msr_version() >= 100
    # bad block size / negative sizes / bad noise mode are rejected before any HIP call
    rc = lib.msr_adamw8bit_step(1, 1, 1, 1, 1, 1, 1, 1, None, 100, 48, 1, 1e-3, 0.9, 0.99, 1e-8, 0.0, 0.1, 0.01, 0,
                                1, None, None)
    assert rc == 1001 and b"block" in lib.msr_last_error()
    assert lib.msr_sr_accum(None, None, 0, -1, 0, 0, 1, None, None) == 1001
    # the allocation-free centralization refuses sizes beyond its static scratch before any HIP call
    assert lib.msr_centralize_bf16_noalloc(1, 1, 1 << 20, 8, 1.0, None) == 1004
    assert b"scratch" in lib.msr_last_error()
    assert lib.msr_sr_accum(1, 1, 0, 10, 0, 0, 7, None, None) == 1001
    assert lib.msr_sr_accum(1, 1, 0, 10, 0, 0, 2, None, None) == 1001   # INJECT without a buffer
    from muon_sr_amd import _lib
    bad = (_lib.AccumItem * 1)(_lib.AccumItem(1, 1, 10, 0, 8))
    assert lib.msr_sr_accum_multi(bad, 1, 1, None) == 1001          # unknown flag
    ok = (_lib.AccumItem * 1)(_lib.AccumItem(1, 1, 10, 0, 0))
    assert lib.msr_sr_accum_multi(ok, 1, 2, None) == 1001           # INJECT is not offered
    size = ctypes.c_size_t(0)
    assert lib.msr_ns_workspace_bytes(2, 100, 60, ctypes.byref(size)) == 0
    # two 256x256-padded iterates (ping-pong) + A + B, bf16, plus partial sums, per matrix
    assert size.value >= 2 * (2 * 256 * 256 * 2 + 2 * 256 * 256 * 2)
    assert lib.msr_newton_schulz(1, 1, 1, 300, 300, 5, 1.0, 1.0, 1.0, 1, 16, None) == 1004
    assert lib.msr_gemm_nt(1, 64, 0, 1, 64, 0, None, 0, 0, 1, 256, 0, 255, 256, 64, 1, 1.0, 0.0, 0.0, None) == 1001
    # K must be a multiple of 128 (the K loop runs two 64-wide slabs per iteration)
    assert lib.msr_gemm_nt(1, 64, 0, 1, 64, 0, None, 0, 0, 1, 256, 0, 256, 256, 64, 1, 1.0, 0.0, 0.0, None) == 1001
    assert lib.msr_gemm_nn(1, 64, 0, 1, 64, 0, None, 0, 0, 1, 256, 0, 256, 256, 64, 1, 1.0, 0.0, 0.0, None) == 1001
    # fused weight-gradient accumulation: features multiples of 256, tokens of 128, known noise mode
    assert lib.msr_linear_wgrad_sr_accum(1, 1, 256, 1, 256, 100, 256, 256, 0, 0, 0, None, None) == 1001
    assert lib.msr_linear_wgrad_sr_accum(1, 1, 300, 1, 256, 128, 300, 256, 0, 0, 0, None, None) == 1001
    assert lib.msr_linear_wgrad_sr_accum(1, 1, 256, 1, 256, 128, 256, 256, 0, 0, 7, None, None) == 1001
    assert lib.msr_linear_wgrad_sr_accum(1, 1, 256, 1, 256, 128, 256, 256, 0, 0, 2, None, None) == 1001


def test_overlapping_operands_are_rejected(lib):
    """Operands that share memory without being the same buffer would race; every
    entry point refuses them (MSR_ERR_OVERLAP) before any HIP call."""
    from muon_sr_amd import _lib
    OVERLAP = 1005
    A, B, C, D = 0x100000, 0x200000, 0x300000, 0x400000
    # acc and grad: half a buffer apart
    assert lib.msr_sr_accum(A, A + 64, 0, 100, 0, 0, 1, None, None) == OVERLAP
    # an fp32 gradient in place of its bf16 accumulator: same start, different extent
    assert lib.msr_sr_accum(A, A, 1, 100, 0, 0, 1, None, None) == OVERLAP
    items = (_lib.AccumItem * 2)(_lib.AccumItem(A, B, 100, 0, 0), _lib.AccumItem(A + 100, C, 100, 0, 0))
    assert lib.msr_sr_accum_multi(items, 2, 1, None) == OVERLAP
    assert lib.msr_adamw_bf16_step(A, B, C, C + 2, 64, 1e-3, 0.9, 0.99, 1e-8, 0.0, 0.1, 0.1, 0, 1, None, None) == OVERLAP
    # 8-bit: the code buffer runs into the block scales
    assert lib.msr_adamw8bit_step(A, B, C, D, C + 32, D + 4096, 1, 1, None, 1024, 256, 1, 1e-3, 0.9, 0.99, 1e-8,
                                  0.0, 0.1, 0.01, 0, 1, None, None) == OVERLAP
    grads = _lib.ptr_array([A, A + 128])
    assert lib.msr_muon_prepare(grads, 0, B, B + 64, 64, 2, 0.95, 1, 0, 1, None, None) == OVERLAP
    params = _lib.ptr_array([A, A + 64])
    seeds = _lib.ptr_array([1, 2], ctypes.c_uint32)
    assert lib.msr_muon_apply(params, B, 64, 2, 0.02, 0.0, 1.0, seeds, 1, None, None) == OVERLAP
    nb = ctypes.c_size_t()
    assert lib.msr_centralize_workspace_bytes(4, 100, ctypes.byref(nb)) == 0
    assert lib.msr_centralize_bf16(A, A + 2, 4, 100, 0.5, C, nb.value, None) == OVERLAP
    assert lib.msr_centralize_bf16(A, B, 4, 100, 0.5, A + 8, nb.value, None) == OVERLAP
    assert lib.msr_ns_workspace_bytes(2, 256, 256, ctypes.byref(nb)) == 0
    assert lib.msr_newton_schulz(A, B, 2, 256, 256, 5, 3.4445, -4.775, 2.0315, A + 1024, nb.value, None) == OVERLAP
    assert b"overlap" in lib.msr_last_error()


def test_fused_steps_validation_without_gpu(lib):
    """msr_muon_fused_steps rejects, before any HIP call, groups of different
    Newton-Schulz shapes, injected noise, a short workspace and operands shared
    across groups (fake device addresses: nothing is dereferenced)."""
    from muon_sr_amd import _lib
    keep = []

    def group(base, k, rows, cols, params=None):
        n = rows * cols
        grads = (ctypes.c_void_p * k)(*[base + 2 * n * i for i in range(k)])
        prm = (ctypes.c_void_p * k)(*(params or [base + (1 << 32) + 2 * n * i for i in range(k)]))
        seeds = (ctypes.c_uint32 * k)(*range(k))
        keep.extend([grads, prm, seeds])
        return _lib.MuonGroup(ctypes.addressof(grads), base + (2 << 32), ctypes.addressof(prm), ctypes.addressof(seeds),
                              0, k, rows, cols, 7, 0, 1.0)

    def call(groups, mode=1, ws_bytes=1 << 40, steps=5):
        arr = (_lib.MuonGroup * len(groups))(*groups)
        return lib.msr_muon_fused_steps(arr, len(groups), 0.95, 1, steps, 3.4, -4.7, 2.0, 0.02, 0.01, mode,
                                        1 << 46, ws_bytes, None)

    g0 = group(1 << 36, 2, 256, 512)
    g1 = group(1 << 37, 1, 512, 256)
    assert call([g0, group(1 << 38, 1, 512, 384)]) == 1001
    assert b"same shape up to transposition" in lib.msr_last_error()
    assert call([g0, g1], mode=2) == 1001          # injected noise: msr_muon_fused_step only
    assert call([g0, g1], steps=0) == 1001
    assert lib.msr_muon_fused_steps(None, 0, 0.95, 1, 5, 3.4, -4.7, 2.0, 0.02, 0.01, 1, 1 << 46, 1 << 40, None) == 1001
    nb = ctypes.c_size_t(0)
    assert lib.msr_ns_workspace_bytes(3, 256, 512, ctypes.byref(nb)) == 0
    assert call([g0, g1], ws_bytes=nb.value - 1) == 1004
    # a parameter of group 1 that is also one of group 0's
    g2 = group(1 << 38, 1, 512, 256, params=[(1 << 36) + (1 << 32)])
    assert call([g0, g2], ws_bytes=nb.value) == 1005
    assert b"overlaps another operand" in lib.msr_last_error()
    # a gradient of group 1 inside group 0's momentum
    g3 = group((1 << 36) + (2 << 32), 1, 512, 256)
    g3.buf = (1 << 39) + (2 << 32)
    assert call([g0, g3], ws_bytes=nb.value) == 1005
    assert b"overlaps a momentum" in lib.msr_last_error()


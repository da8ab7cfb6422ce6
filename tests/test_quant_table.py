"""CPU checks of the host-built quantizer table (no GPU needed).

The table (msr_quant_table_build, host code of the library) is decoded here and
evaluated with a numpy restatement of the device lookup, then compared with the
oracle's reference quantizer search on dense samples of [-1, 1]: every codebook
value and rounding midpoint +-3 ulps, every table threshold +-2 ulps, and 2^22
random floats.  The exhaustive comparison over all 2^31 floats runs on the GPU.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "muon_sr_amd", "libmuon_sr_amd.so")


@pytest.fixture(scope="module")
def table():
    if not os.path.exists(LIB):
        pytest.fail("library not built")
    from muon_sr_amd import _lib
    L = _lib.lib()
    nbytes = L.msr_quant_table_bytes()
    buf = np.zeros(nbytes, np.uint8)
    q1, q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
    assert L.msr_quant_table_build(q1.ctypes.data, q2.ctypes.data, buf.ctypes.data, nbytes) == 0
    words = buf.view(np.uint32)
    n_bkt = int(words[0])
    oct_ = words[4:4 + 1024].copy()
    bkt = words[4 + 1024:4 + 1024 + 2 * n_bkt].reshape(-1, 2).copy()
    return n_bkt, oct_, bkt


def lookup(x, oct_, bkt, signed):
    """numpy restatement of quantize_lookup (the device/host table read)."""
    x = np.asarray(x, np.float32)
    u = x.view(np.uint32)
    o = oct_[(0 if signed else 512) + (u >> 23)]
    b = (o >> 8) + ((u & np.uint32(0x7FFFFF)) >> (o & 31))
    en = bkt[b]
    return ((en[:, 1] >> np.where((u & np.uint32(0x7FFFFFFF)) >= en[:, 0], 8, 0)) & 0xFF).astype(np.uint8)


def test_table_size(table):
    n_bkt, oct_, bkt = table
    assert 128 * 3 <= n_bkt <= 2048


def probe_points(Q, rng, thresholds):
    mids = ((Q[1:] + Q[:-1]) * np.float32(0.5)).astype(np.float32)
    pts = np.concatenate([Q, mids, thresholds])
    out = [pts]
    up, dn = pts.copy(), pts.copy()
    for _ in range(3):
        up = np.nextafter(up, np.float32(2))
        dn = np.nextafter(dn, np.float32(-2))
        out += [up, dn]
    out.append(rng.uniform(-1, 1, 1 << 22).astype(np.float32))
    out.append((10.0 ** rng.uniform(-40, 0, 1 << 20)).astype(np.float32))
    x = np.concatenate(out).astype(np.float32)
    return x[np.abs(x) <= 1]


@pytest.mark.parametrize("signed", [True, False])
def test_table_matches_search(table, signed):
    n_bkt, oct_, bkt = table
    Q = O.create_dynamic_map(signed)
    thr = bkt[:, 0][bkt[:, 0] <= 0x3F800000].astype(np.uint32).view(np.float32)
    x = probe_points(Q, np.random.default_rng(1 + signed), thr)
    nans = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0xFFFFFFFF], np.uint32).view(np.float32)
    if signed:
        x = np.concatenate([x, -x, nans, np.array([-0.0, 0.0], np.float32)])
    else:
        x = np.concatenate([np.abs(x), nans, np.array([0.0], np.float32)])
    got = lookup(x, oct_, bkt, signed)
    ref = O.quantize(x, Q, signed)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, (x[bad[:5]], got[bad[:5]], ref[bad[:5]])

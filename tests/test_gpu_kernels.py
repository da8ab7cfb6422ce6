"""GPU parity tests: each kernel through the C ABI against the CPU oracle.

Bar: bit-exact for every stochastic-rounding kernel (same noise bits: injected,
the reference's Philox word-0 stream, or this library's Philox8 stream, all of
which the oracle also produces), bit-exact quantizer codes and block scales;
Newton-Schulz within 1e-2 relative Frobenius of an fp32 emulation of the same
bf16-storage op.
"""
import numpy as np
import pytest
import torch

import oracle as O
from _gpu import DEV, check, dev_to_u16, need_gpu, np_to_dev, ptr, ptr_array, rel_fro, stream, u16_to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    return need_gpu()


def rng_bf16(rng, n, std):
    return O.f32_to_bf16_rne((rng.standard_normal(n) * std).astype(np.float32))


def unaligned(t):
    """A view of t starting one element in (breaks 16-byte alignment)."""
    big = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    v = big[1:]
    v.copy_(t.flatten())
    return v


# ---------------------------------------------------------------------------
# RNG
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8])
def test_noise_streams_match_oracle(L, mode):
    n = 4096
    for seed, k in [(12345, 0), (0x7FFFFFFF, 1), (0x7FFFFFFE, 2), (0xFFFFFFFF, 2), (0xDEADBEEF, 0)]:
        for off0 in (0, 2**31 - 100, 2**32 - 50, 2**40 + 8):
            out = torch.empty(n, dtype=torch.int16, device=DEV)
            check(L, L.msr_noise_fill(out.data_ptr(), n, off0, seed, k, mode, stream()), "noise_fill")
            got = out.cpu().numpy().view(np.uint16)
            exp = O.noise16(mode, seed, np.arange(off0, off0 + n, dtype=np.int64), k)
            assert np.array_equal(got, exp), (mode, seed, k, off0)


# ---------------------------------------------------------------------------
# (c) SR accumulate
# ---------------------------------------------------------------------------

def test_sr_accum_reference_vectors(L, golden):
    z = golden("elementwise")
    acc = u16_to_dev(z["accum/in_acc"])
    g = u16_to_dev(z["accum/in_g"])
    check(L, L.msr_sr_accum(acc.data_ptr(), g.data_ptr(), 0, acc.numel(), 777, 0, O.NOISE_TRITON, None, stream()))
    assert np.array_equal(dev_to_u16(acc), z["accum/out_bf16g"])
    acc = u16_to_dev(z["accum/in_acc"])
    g32 = np_to_dev(z["accum/in_g32"])
    check(L, L.msr_sr_accum(acc.data_ptr(), g32.data_ptr(), 1, acc.numel(), 0x9E3779B9, 0, O.NOISE_TRITON, None,
                            stream()))
    assert np.array_equal(dev_to_u16(acc), z["accum/out_f32g"])


@pytest.mark.parametrize("n", [1, 7, 8, 1000, 4099, 65536 + 13])
@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8, O.NOISE_INJECT])
def test_sr_accum_vs_oracle(L, n, mode):
    rng = np.random.default_rng(n * 7 + mode)
    acc0 = rng_bf16(rng, n, 1e-3)
    g16 = rng_bf16(rng, n, 1e-4)
    g32 = (rng.standard_normal(n) * 1e-4).astype(np.float32)
    inj = rng.integers(0, 65536, n).astype(np.uint16)
    seed = int(rng.integers(0, 2**32))
    spec = O.NoiseSpec(mode, seed, 0, inj if mode == O.NOISE_INJECT else None)
    inj_d = np_to_dev(inj.view(np.int16)) if mode == O.NOISE_INJECT else None
    for gname, gnp in (("bf16", g16), ("f32", g32)):
        for zero in (0, 1):
            for misalign in (False, True):
                acc = u16_to_dev(acc0)
                g = u16_to_dev(gnp) if gname == "bf16" else np_to_dev(gnp)
                if misalign:
                    acc, g = unaligned(acc), unaligned(g)
                check(L, L.msr_sr_accum(acc.data_ptr(), g.data_ptr(), int(gname == "f32"), n, seed, zero, mode,
                                        ptr(inj_d), stream()))
                start = np.zeros(n, np.uint16) if zero else acc0
                exp = O.sr_accum(start, gnp, spec)
                assert np.array_equal(dev_to_u16(acc), exp), (gname, zero, misalign)


@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8])
def test_sr_accum_multi_equals_single_launches(L, mode):
    """One multi-tensor launch (200 items: more than one launch's worth, ragged
    sizes, unaligned views, fp32 grads, zero-init) equals one msr_sr_accum per
    item, bit for bit."""
    from muon_sr_amd import _lib
    rng = np.random.default_rng(5 + mode)
    sizes = [0, 1, 7, 8, 9, 1000, 100003, 4096, 333] + list(rng.integers(1, 20000, 191))
    items, singles, accs_m, accs_s, keep = [], [], [], [], []
    for i, n in enumerate(sizes):
        n = int(n)
        f32 = i % 5 == 3
        zero = i % 7 == 2
        acc0 = rng_bf16(rng, n, 1e-3)
        am, as_ = u16_to_dev(acc0), u16_to_dev(acc0)
        if i % 4 == 1:   # unaligned accumulators
            am, as_ = unaligned(am), unaligned(as_)
        if f32:
            g = np_to_dev((rng.standard_normal(n) * 1e-3).astype(np.float32))
        else:
            g = u16_to_dev(rng_bf16(rng, n, 1e-3))
            if i % 6 == 5:
                g = unaligned(g)
        seed = int(rng.integers(0, 2**32))
        flags = (_lib.ACCUM_ZERO_INIT if zero else 0) | (_lib.ACCUM_GRAD_F32 if f32 else 0)
        items.append(_lib.AccumItem(am.data_ptr(), g.data_ptr(), n, seed, flags))
        singles.append((as_, g, f32, n, seed, zero))
        accs_m.append(am)
        accs_s.append(as_)
        keep.append(g)
    arr = (_lib.AccumItem * len(items))(*items)
    check(L, L.msr_sr_accum_multi(arr, len(items), mode, stream()), "multi")
    for as_, g, f32, n, seed, zero in singles:
        check(L, L.msr_sr_accum(as_.data_ptr(), g.data_ptr(), int(f32), n, seed, int(zero), mode, None, stream()))
    for i, (am, as_) in enumerate(zip(accs_m, accs_s)):
        assert np.array_equal(dev_to_u16(am), dev_to_u16(as_)), (i, sizes[i])


# ---------------------------------------------------------------------------
# BF16-moment AdamW
# ---------------------------------------------------------------------------

def test_adamw_bf16_reference_vectors(L, golden):
    z = golden("elementwise")
    for tag in ("s_small", "s_wrap", "s_wrap2", "s_u32", "s_i64wrap"):
        k = lambda s: z[f"adamw/{tag}/{s}"]  # noqa: E731
        lr, b1, b2, eps, wd, bc, bcs = (float(v) for v in k("hyper"))
        p, g, e, s = (u16_to_dev(k(x)) for x in ("in_p", "in_g", "in_e", "in_s"))
        check(L, L.msr_adamw_bf16_step(p.data_ptr(), g.data_ptr(), e.data_ptr(), s.data_ptr(), p.numel(),
                                       lr, b1, b2, eps, wd, bc, bcs, int(k("seed")), O.NOISE_TRITON, None, stream()))
        assert np.array_equal(dev_to_u16(p), k("out_p")), tag
        assert np.array_equal(dev_to_u16(e), k("out_e")), tag
        assert np.array_equal(dev_to_u16(s), k("out_s")), tag


@pytest.mark.parametrize("mode", [O.NOISE_PHILOX8, O.NOISE_INJECT, O.NOISE_TRITON])
@pytest.mark.parametrize("misalign", [False, True])
def test_adamw_bf16_vs_oracle(L, mode, misalign):
    rng = np.random.default_rng(11 + mode)
    n = 5003
    p0, g0, e0 = rng_bf16(rng, n, 0.02), rng_bf16(rng, n, 1e-3), rng_bf16(rng, n, 1e-4)
    s0 = O.f32_to_bf16_rne((rng.standard_normal(n) * 1e-4).astype(np.float32) ** 2)
    inj = rng.integers(0, 65536, 3 * n).astype(np.uint16)
    seed = 0x7FFFFFFE
    lr, b1, b2, eps, wd = 1e-3, 0.9, 0.999, 1e-8, 0.01
    bc, bcs = O.adamw_bias_corrections(b1, b2, 7)
    specs = [O.NoiseSpec(mode, seed, k, inj[k * n:(k + 1) * n] if mode == O.NOISE_INJECT else None) for k in range(3)]
    ep, ee, es = O.adamw_bf16(p0, g0, e0, s0, lr, b1, b2, eps, wd, bc, bcs, specs[0], specs[1], specs[2])
    p, g, e, s = (u16_to_dev(x) for x in (p0, g0, e0, s0))
    if misalign:
        p, g, e, s = (unaligned(x) for x in (p, g, e, s))
    inj_d = np_to_dev(inj.view(np.int16)) if mode == O.NOISE_INJECT else None
    check(L, L.msr_adamw_bf16_step(p.data_ptr(), g.data_ptr(), e.data_ptr(), s.data_ptr(), n, lr, b1, b2, eps, wd,
                                   bc, bcs, seed, mode, ptr(inj_d), stream()))
    assert np.array_equal(dev_to_u16(p), ep)
    assert np.array_equal(dev_to_u16(e), ee)
    assert np.array_equal(dev_to_u16(s), es)


# ---------------------------------------------------------------------------
# (a) 8-bit AdamW
# ---------------------------------------------------------------------------

_QT = {}


def qtable_dev(L):
    """Device copy of the quantizer table of the standard codebooks."""
    if "t" not in _QT:
        nbytes = L.msr_quant_table_bytes()
        buf = np.zeros(nbytes, np.uint8)
        q1, q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
        check(L, L.msr_quant_table_build(q1.ctypes.data, q2.ctypes.data, buf.ctypes.data, nbytes), "table build")
        _QT["t"] = np_to_dev(buf)
    return _QT["t"]


def _adam8_call(L, p, g, s1, s2, a1, a2, q1, q2, n, block, quant, hyper, seed, mode, inj=None, qt=None):
    lr, b1, b2, eps, wd, bc1, bc2 = hyper
    check(L, L.msr_adamw8bit_step(p.data_ptr(), g.data_ptr(), s1.data_ptr(), s2.data_ptr(), ptr(a1), ptr(a2),
                                  ptr(q1), ptr(q2), ptr(qt), n, block, int(quant), lr, b1, b2, eps, wd, bc1, bc2,
                                  seed, mode, ptr(inj), stream()), "adamw8bit")


@pytest.mark.parametrize("use_table", [False, True])
def test_adamw8bit_reference_vectors(L, golden, use_table):
    z = golden("adamw8bit")
    qt = qtable_dev(L) if use_table else None
    q1 = np_to_dev(O.create_dynamic_map(True))
    q2 = np_to_dev(O.create_dynamic_map(False))
    names = sorted({k.split("/")[0] for k in z.files})
    for name in names:
        k = lambda s: z[f"{name}/{s}"]  # noqa: E731
        quant = bool(k("quantized"))
        n, block = int(k("n")), int(k("block"))
        lr, b1, b2, eps, wd = (float(k(x)) for x in ("lr", "b1", "b2", "eps", "wd"))
        p = u16_to_dev(k("p0"))
        if quant:
            s1, s2 = np_to_dev(k("s1_0")), np_to_dev(k("s2_0"))
            a1, a2 = np_to_dev(k("a1_0")), np_to_dev(k("a2_0"))
        else:
            s1, s2 = u16_to_dev(k("s1_0")), u16_to_dev(k("s2_0"))
            a1 = a2 = None
        for step in range(1, int(k("steps")) + 1):
            g = u16_to_dev(k(f"g_{step}"))
            hyper = (lr, b1, b2, eps, wd, 1 - b1 ** step, 1 - b2 ** step)
            _adam8_call(L, p, g, s1, s2, a1, a2, q1 if quant else None, q2 if quant else None, n, block, quant,
                        hyper, int(k(f"seed_{step}")), O.NOISE_TRITON, qt=qt if quant else None)
            assert np.array_equal(dev_to_u16(p), k(f"p_{step}")), (name, step)
            if quant:
                assert np.array_equal(s1.cpu().numpy(), k(f"s1_{step}")), (name, step)
                assert np.array_equal(s2.cpu().numpy(), k(f"s2_{step}")), (name, step)
                assert np.array_equal(a1.cpu().numpy().view(np.uint32), k(f"a1_{step}").view(np.uint32)), (name, step)
                assert np.array_equal(a2.cpu().numpy().view(np.uint32), k(f"a2_{step}").view(np.uint32)), (name, step)
            else:
                assert np.array_equal(dev_to_u16(s1), k(f"s1_{step}")), (name, step)
                assert np.array_equal(dev_to_u16(s2), k(f"s2_{step}")), (name, step)


@pytest.mark.parametrize("block", [32, 64, 128, 256, 512, 1024, 2048, 4096])
@pytest.mark.parametrize("mode", [O.NOISE_PHILOX8, O.NOISE_INJECT])
@pytest.mark.parametrize("use_table", [True, False])
def test_adamw8bit_blocks_vs_oracle(L, block, mode, use_table):
    rng = np.random.default_rng(block + mode)
    n = 5 * block + 77
    nb = (n + block - 1) // block
    Q1, Q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
    q1, q2 = np_to_dev(Q1), np_to_dev(Q2)
    p0 = rng_bf16(rng, n, 0.02)
    s1 = np.full(n, 127, np.uint8)
    s2 = np.zeros(n, np.uint8)
    a1 = np.zeros(nb, np.float32)
    a2 = np.zeros(nb, np.float32)
    pd, s1d, s2d, a1d, a2d = u16_to_dev(p0), np_to_dev(s1), np_to_dev(s2), np_to_dev(a1), np_to_dev(a2)
    pe = p0
    lr, b1, b2, eps, wd = 3e-4, 0.9, 0.95, 1e-10, 0.01
    for step in range(1, 4):
        g0 = rng_bf16(rng, n, 1e-3)
        if step == 1:
            g0[block:2 * block] = 0          # all-zero block
        if step == 2:
            g0[[3, n - 1]] = [0x7FC0, 0xFF80]  # NaN, -inf
        inj = rng.integers(0, 65536, 3 * n).astype(np.uint16)
        seed = int(rng.integers(0, 2**32))
        hyper = (lr, b1, b2, eps, wd, 1 - b1 ** step, 1 - b2 ** step)
        spec = O.NoiseSpec(mode, seed, 0, inj[:n] if mode == O.NOISE_INJECT else None)
        pe, s1, s2, a1, a2 = O.adamw8bit(pe, g0, s1, s2, a1, a2, Q1, Q2, block, True, *hyper, spec)
        inj_d = np_to_dev(inj.view(np.int16)) if mode == O.NOISE_INJECT else None
        _adam8_call(L, pd, u16_to_dev(g0), s1d, s2d, a1d, a2d, q1, q2, n, block, True, hyper, seed, mode, inj_d,
                    qt=qtable_dev(L) if use_table else None)
        assert np.array_equal(dev_to_u16(pd), pe), step
        assert np.array_equal(s1d.cpu().numpy(), s1), step
        assert np.array_equal(s2d.cpu().numpy(), s2), step
        assert np.array_equal(a1d.cpu().numpy().view(np.uint32), a1.view(np.uint32)), step
        assert np.array_equal(a2d.cpu().numpy().view(np.uint32), a2.view(np.uint32)), step


@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8])
def test_adamw8bit_unaligned_and_bf16_branch(L, mode):
    rng = np.random.default_rng(5)
    n, block = 3000, 256
    Q1, Q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
    p0, g0 = rng_bf16(rng, n, 0.02), rng_bf16(rng, n, 1e-3)
    nb = (n + block - 1) // block
    hyper = (1e-3, 0.9, 0.999, 1e-8, 0.1, 0.1, 0.001)
    seed = 0x7FFFFFFF
    # quantized state, parameter and gradient views not 16-byte aligned
    pe, e1, e2, ea1, ea2 = O.adamw8bit(p0, g0, np.full(n, 127, np.uint8), np.zeros(n, np.uint8),
                                       np.zeros(nb, np.float32), np.zeros(nb, np.float32), Q1, Q2, block, True,
                                       *hyper, O.NoiseSpec(mode, seed))
    p, g = unaligned(u16_to_dev(p0)), unaligned(u16_to_dev(g0))
    s1, s2 = np_to_dev(np.full(n, 127, np.uint8)), np_to_dev(np.zeros(n, np.uint8))
    a1, a2 = np_to_dev(np.zeros(nb, np.float32)), np_to_dev(np.zeros(nb, np.float32))
    _adam8_call(L, p, g, s1, s2, a1, a2, np_to_dev(Q1), np_to_dev(Q2), n, block, True, hyper, seed, mode,
                qt=qtable_dev(L))
    assert np.array_equal(dev_to_u16(p), pe)
    assert np.array_equal(s1.cpu().numpy(), e1) and np.array_equal(s2.cpu().numpy(), e2)
    # bf16-moment branch (seed streams SEED, SEED+1 (wraps the i32 seed), SEED+2)
    m0, v0 = rng_bf16(rng, n, 1e-4), O.f32_to_bf16_rne((rng.standard_normal(n) * 1e-4).astype(np.float32) ** 2)
    pe, me, ve = O.adamw8bit(p0, g0, m0, v0, None, None, None, None, block, False, *hyper,
                             O.NoiseSpec(mode, seed), O.NoiseSpec(mode, seed, 1), O.NoiseSpec(mode, seed, 2))
    p, g, m, v = (u16_to_dev(x) for x in (p0, g0, m0, v0))
    _adam8_call(L, p, g, m, v, None, None, None, None, n, block, False, hyper, seed, mode)
    assert np.array_equal(dev_to_u16(p), pe)
    assert np.array_equal(dev_to_u16(m), me)
    assert np.array_equal(dev_to_u16(v), ve)


def test_quantizer_device_vs_oracle(L, golden):
    z = golden("quantize")
    rng = np.random.default_rng(9)
    for signed in (True, False):
        Q = O.create_dynamic_map(signed)
        name = "signed" if signed else "unsigned"
        lo = -1.0 if signed else 0.0
        x = np.concatenate([z[f"x_{name}"], rng.uniform(lo, 1, 1 << 20).astype(np.float32),
                            (10.0 ** rng.uniform(-12, 0, 1 << 20)).astype(np.float32)
                            * (rng.choice([-1, 1], 1 << 20) if signed else 1)]).astype(np.float32)
        xd = np_to_dev(x)
        expect = O.quantize(x, Q, signed)
        for qt in (None, qtable_dev(L)):
            out = torch.empty(x.size, dtype=torch.uint8, device=DEV)
            check(L, L.msr_quantize(xd.data_ptr(), out.data_ptr(), x.size, np_to_dev(Q).data_ptr(), int(signed),
                                    ptr(qt), stream()))
            got = out.cpu().numpy()
            assert np.array_equal(got[:z[f"x_{name}"].size], z[f"code_{name}"])
            assert np.array_equal(got, expect)


def test_quant_table_exhaustive(L):
    """The table equals the reference search for every float in [-1, 1], both maps."""
    q1 = np_to_dev(O.create_dynamic_map(True))
    q2 = np_to_dev(O.create_dynamic_map(False))
    qt = qtable_dev(L)
    nblk = 4096
    counts = torch.zeros(nblk, dtype=torch.int32, device=DEV)
    check(L, L.msr_quant_table_check(qt.data_ptr(), q1.data_ptr(), q2.data_ptr(), 0, 0x3F800000, counts.data_ptr(),
                                     nblk, stream()), "table check")
    assert int(counts.sum().item()) == 0


SQRT_HI = 0x5E800000                     # bits(2^62)
RCP_LO, RCP_HI = 0x21800000, 0x3FFFFFFF  # bits(2^-60), bits(2) - 1
UPD_HI = 0x4F7FFFFF                      # bits(2^32) - 1


@pytest.mark.parametrize("kind,lo,hi", [
    (0, 0, SQRT_HI),                       # sqrt: every float in [0, 2^62]
    (1, RCP_LO, UPD_HI),                   # reciprocal: every float in [2^-60, 2^32)
    (2, 0x3F800000, RCP_HI),               # quotient: every d in [1, 2), 16 m each
    (2, RCP_LO, RCP_LO + (1 << 23) - 1),   # ... every d in [2^-60, 2^-59)
    (2, 0x30000000, 0x307FFFFF),           # ... every d in [2^-31, 2^-30)
    (3, 0, 0xFFFFFFFF),                    # hardware bf16 rounding: every fp32 bit pattern
    (4, 0x3F800000, RCP_HI),               # update quotient: every d in [1, 2), 16 n each
    (4, RCP_LO, RCP_LO + (1 << 23) - 1),   # ... every d in [2^-60, 2^-59)
    (4, 0x4F000000, UPD_HI),               # ... every d in [2^31, 2^32)
    (4, 0x30000000, 0x307FFFFF),           # ... every d in [2^-31, 2^-30)
])
def test_fastmath_exhaustive(L, kind, lo, hi):
    """The fast 8-bit kernel's sqrt, reciprocal and quotients equal the IEEE operations
    on their whole input ranges (the quotients on hashed samples of numerators), and
    the hardware fp32->bf16 conversion of the GEMM epilogues equals the bit-level
    round-to-nearest-even on every fp32 bit pattern."""
    nblk = 4096
    counts = torch.zeros(nblk, dtype=torch.int32, device=DEV)
    check(L, L.msr_fastmath_check(kind, lo, hi, counts.data_ptr(), nblk, stream()), "fastmath check")
    assert int(counts.sum().item()) == 0


@pytest.mark.parametrize("mode", [O.NOISE_PHILOX8, O.NOISE_TRITON, O.NOISE_INJECT])
def test_adamw8bit_fast_kernel_vs_oracle(L, mode):
    """Block 256, standard codebooks, aligned: full block pairs run through the fast kernel,
    whose waves switch to the exact branch for pairs with non-finite gradients or extreme
    moments; the odd last full block and the ragged tail run through the general kernel.
    Bit-exact against the oracle (parameters, codes, block scales) over four steps."""
    rng = np.random.default_rng(100 + mode)
    block = 256
    n = (1 << 19) + 3 * block + 77          # 2051 full blocks (odd) + a ragged tail
    nb = (n + block - 1) // block
    Q1, Q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
    q1, q2, qt = np_to_dev(Q1), np_to_dev(Q2), qtable_dev(L)
    p0 = rng_bf16(rng, n, 0.02)
    s1, s2 = np.full(n, 127, np.uint8), np.zeros(n, np.uint8)
    a1, a2 = np.zeros(nb, np.float32), np.zeros(nb, np.float32)
    pair = lambda i: slice(512 * i, 512 * (i + 1))  # noqa: E731
    # pair 25: negative codes with zero block scales dequantize to -0, so -0 gradients give
    # m' = -0 and the update's numerator -0 against parameters -0 (fast branch)
    s1[pair(25)] = 0
    p0[512 * 25:512 * 25 + 8] = 0x8000
    pd, s1d, s2d, a1d, a2d = u16_to_dev(p0), np_to_dev(s1), np_to_dev(s2), np_to_dev(a1), np_to_dev(a2)
    pe = p0
    lr, b1, b2, eps, wd = 3e-4, 0.9, 0.95, 1e-10, 0.01
    for step in range(1, 5):
        g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        if step == 1:
            g[pair(3)][100] = np.nan            # non-finite gradient: exact branch
            g[pair(7)] *= 3e21                  # v' above 2^62: exact branch
            g[pair(11)] *= 1e-22                # block scales below 2^-60: exact branch
            g[pair(13)] = 0.0                   # all-zero pair: fast branch, divisor 1
            g[pair(21)][9] = 1e-33              # one update numerator below 2^-90: exact branch
            g[pair(25)][:8] = -0.0
        if step == 2:
            g[pair(5)][7] = -np.inf
            g[pair(17)][:256] *= 1e-30          # one tiny block next to a normal one
        if step == 3:
            g[pair(19)] *= 1e4                  # block scales in [2, ...): exact branch
        g0 = O.f32_to_bf16_rne(g)
        inj = rng.integers(0, 65536, 3 * n).astype(np.uint16)
        seed = int(rng.integers(0, 2**32))
        hyper = (lr, b1, b2, eps, wd, 1 - b1 ** step, 1 - b2 ** step)
        spec = O.NoiseSpec(mode, seed, 0, inj[:n] if mode == O.NOISE_INJECT else None)
        pe, s1, s2, a1, a2 = O.adamw8bit(pe, g0, s1, s2, a1, a2, Q1, Q2, block, True, *hyper, spec)
        inj_d = np_to_dev(inj.view(np.int16)) if mode == O.NOISE_INJECT else None
        _adam8_call(L, pd, u16_to_dev(g0), s1d, s2d, a1d, a2d, q1, q2, n, block, True, hyper, seed, mode, inj_d,
                    qt=qt)
        got = dev_to_u16(pd)
        same = (got == pe) | (np.isnan(O.bf16_to_f32(got)) & np.isnan(O.bf16_to_f32(pe)))
        assert same.all(), (step, np.flatnonzero(~same)[:10])
        assert np.array_equal(s1d.cpu().numpy(), s1), step
        assert np.array_equal(s2d.cpu().numpy(), s2), step
        assert np.array_equal(a1d.cpu().numpy().view(np.uint32), a1.view(np.uint32)), step
        assert np.array_equal(a2d.cpu().numpy().view(np.uint32), a2.view(np.uint32)), step


@pytest.mark.parametrize("lr,eps", [(3e-4, 0.0), (1e21, 1e-10), (1.6e21, 1e-10), (3e21, 1e-10)])
def test_adamw8bit_launch_and_branch_conditions(L, lr, eps):
    """eps = 0 puts the update's divisor outside the fast kernel's range (sqrt(v') + eps
    may be 0 or tiny), so the launcher runs the general kernel on a tensor the fast one
    would otherwise take (zero-gradient elements give 0/0 in the update).  Learning rates
    of 1e21 to 3e21 put the update's numerators step_c * m' around 2^60, where the fast
    kernel's waves send the pairs above it to the exact branch (none of the first step's
    blocks at 1e21, 58 of 258 at 1.6e21, all at 3e21).  Bit-exact against the oracle in
    every case."""
    rng = np.random.default_rng(23)
    block, n = 256, (1 << 16) + 512
    nb = n // block
    Q1, Q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
    q1, q2, qt = np_to_dev(Q1), np_to_dev(Q2), qtable_dev(L)
    p0 = rng_bf16(rng, n, 0.02)
    s1, s2 = np.full(n, 127, np.uint8), np.zeros(n, np.uint8)
    a1, a2 = np.zeros(nb, np.float32), np.zeros(nb, np.float32)
    pd, s1d, s2d, a1d, a2d = u16_to_dev(p0), np_to_dev(s1), np_to_dev(s2), np_to_dev(a1), np_to_dev(a2)
    pe = p0
    for step in (1, 2):
        g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        g[1000:1100] = 0.0
        g0 = O.f32_to_bf16_rne(g)
        hyper = (lr, 0.9, 0.95, eps, 0.01, 1 - 0.9 ** step, 1 - 0.95 ** step)
        seed = 77 + step
        pe, s1, s2, a1, a2 = O.adamw8bit(pe, g0, s1, s2, a1, a2, Q1, Q2, block, True, *hyper,
                                         O.NoiseSpec(O.NOISE_PHILOX8, seed))
        _adam8_call(L, pd, u16_to_dev(g0), s1d, s2d, a1d, a2d, q1, q2, n, block, True, hyper, seed,
                    O.NOISE_PHILOX8, None, qt=qt)
        got = dev_to_u16(pd)
        same = (got == pe) | (np.isnan(O.bf16_to_f32(got)) & np.isnan(O.bf16_to_f32(pe)))
        assert same.all(), (step, np.flatnonzero(~same)[:10])
        assert np.array_equal(s1d.cpu().numpy(), s1) and np.array_equal(s2d.cpu().numpy(), s2), step
        assert np.array_equal(a1d.cpu().numpy().view(np.uint32), a1.view(np.uint32)), step
        assert np.array_equal(a2d.cpu().numpy().view(np.uint32), a2.view(np.uint32)), step


def test_adamw8bit_extreme_moments(L):
    """Huge gradients (v overflows to inf), denormal-scale moments and -0: the
    exact-quotient and table paths against the oracle."""
    Q1, Q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
    n, block = 2048, 256
    nb = n // block
    rng = np.random.default_rng(17)
    g = rng.standard_normal(n).astype(np.float32)
    g[:256] *= 1e-30                 # tiny moments: quotients near the subnormal range
    g[256:512] *= 3e19               # (1-b2) g^2 overflows to inf in some lanes
    g[512:520] = -0.0
    g[520:524] = [1e-38, -1e-38, 1e-45, -1e-45]
    g0 = O.f32_to_bf16_rne(g)
    p0 = O.f32_to_bf16_rne((rng.standard_normal(n) * 0.02).astype(np.float32))
    hyper = (1e-3, 0.9, 0.999, 1e-8, 0.0, 0.1, 0.001)
    for qt in (None, qtable_dev(L)):
        pe, e1, e2, ea1, ea2 = O.adamw8bit(p0, g0, np.full(n, 127, np.uint8), np.zeros(n, np.uint8),
                                           np.zeros(nb, np.float32), np.zeros(nb, np.float32), Q1, Q2, block, True,
                                           *hyper, O.NoiseSpec(O.NOISE_TRITON, 99))
        p, gd = u16_to_dev(p0), u16_to_dev(g0)
        s1, s2 = np_to_dev(np.full(n, 127, np.uint8)), np_to_dev(np.zeros(n, np.uint8))
        a1, a2 = np_to_dev(np.zeros(nb, np.float32)), np_to_dev(np.zeros(nb, np.float32))
        _adam8_call(L, p, gd, s1, s2, a1, a2, np_to_dev(Q1), np_to_dev(Q2), n, block, True, hyper, 99,
                    O.NOISE_TRITON, qt=qt)
        assert np.array_equal(s1.cpu().numpy(), e1), "m codes"
        assert np.array_equal(s2.cpu().numpy(), e2), "v codes"
        assert np.array_equal(a1.cpu().numpy().view(np.uint32), ea1.view(np.uint32))
        assert np.array_equal(a2.cpu().numpy().view(np.uint32), ea2.view(np.uint32))
        got = dev_to_u16(p)
        same = (got == pe) | (np.isnan(O.bf16_to_f32(got)) & np.isnan(O.bf16_to_f32(pe)))
        assert same.all()


# ---------------------------------------------------------------------------
# (b) Muon prepare / apply
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("nest", [1, 0])
def test_muon_prepare_reference_vectors(L, golden, nest):
    z = golden("elementwise")
    k = lambda s: z[f"prepare/{nest}/{s}"]  # noqa: E731
    g, buf = u16_to_dev(k("in_g")), u16_to_dev(k("in_buf"))
    out = torch.empty_like(buf)
    tbl = ptr_array([g.data_ptr()])
    check(L, L.msr_muon_prepare(tbl, 0, buf.data_ptr(), out.data_ptr(), g.numel(), 1, 0.95, nest, int(k("seed")),
                                O.NOISE_TRITON, None, stream()))
    assert np.array_equal(dev_to_u16(buf), k("out_buf"))
    rne = torch.from_numpy(k("out_upd_f32")).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(dev_to_u16(out), rne)


@pytest.mark.parametrize("rows,cols", [(33, 65), (64, 128)])
@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8, O.NOISE_INJECT])
def test_muon_prepare_stack_vs_oracle(L, rows, cols, mode):
    rng = np.random.default_rng(rows + mode)
    count, numel = 5, rows * cols
    grads = [rng_bf16(rng, numel, 1e-3) for _ in range(count)]
    buf0 = rng_bf16(rng, count * numel, 1e-3)
    inj = rng.integers(0, 65536, count * numel).astype(np.uint16)
    seed = 0xFFFFFFF0
    spec = O.NoiseSpec(mode, seed, 0, inj if mode == O.NOISE_INJECT else None)
    eb, _, eu = O.muon_prepare(np.concatenate(grads), buf0, 0.95, True, spec)
    gd = [u16_to_dev(g) for g in grads]
    buf = u16_to_dev(buf0)
    out = torch.empty_like(buf)
    inj_d = np_to_dev(inj.view(np.int16)) if mode == O.NOISE_INJECT else None
    check(L, L.msr_muon_prepare(ptr_array([t.data_ptr() for t in gd]), 0, buf.data_ptr(), out.data_ptr(), numel,
                                count, 0.95, 1, seed, mode, ptr(inj_d), stream()))
    assert np.array_equal(dev_to_u16(buf), eb)
    assert np.array_equal(dev_to_u16(out), eu)


@pytest.mark.parametrize("numel,offset", [(4096, 0), (1000 + 3, 0), (4096, 1)])
@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8])
def test_muon_prepare_fp32_grads_vs_oracle(L, numel, offset, mode):
    """fp32 gradients are read as fp32 (the reference's per-parameter path), 16-byte
    and element-wise loads (offset 1 misaligns the gradient)."""
    rng = np.random.default_rng(numel + mode)
    count = 3
    grads = [(rng.standard_normal(numel) * 1e-3).astype(np.float32) for _ in range(count)]
    buf0 = rng_bf16(rng, count * numel, 1e-3)
    seed = 12345
    eb, _, eu = O.muon_prepare(np.concatenate(grads), buf0, 0.95, True, O.NoiseSpec(mode, seed))
    gd = []
    for g in grads:
        t = torch.zeros(numel + offset, dtype=torch.float32, device=DEV)
        t[offset:] = torch.from_numpy(g).to(DEV)
        gd.append(t)
    buf = u16_to_dev(buf0)
    out = torch.empty_like(buf)
    check(L, L.msr_muon_prepare(ptr_array([t[offset:].data_ptr() for t in gd]), 1, buf.data_ptr(), out.data_ptr(),
                                numel, count, 0.95, 1, seed, mode, None, stream()))
    assert np.array_equal(dev_to_u16(buf), eb)
    assert np.array_equal(dev_to_u16(out), eu)


def test_muon_apply_reference_vectors(L, golden):
    z = golden("elementwise")
    p, u = u16_to_dev(z["apply/in_p"]), u16_to_dev(z["apply/in_u"])
    seeds = ptr_array([int(z["apply/seed"])], __import__("ctypes").c_uint32)
    check(L, L.msr_muon_apply(ptr_array([p.data_ptr()]), u.data_ptr(), p.numel(), 1, 0.02, 0.01,
                              float(z["apply/scale"]), seeds, O.NOISE_TRITON, None, stream()))
    assert np.array_equal(dev_to_u16(p), z["apply/out_p"])


@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8, O.NOISE_INJECT])
def test_muon_apply_multi_vs_oracle(L, mode):
    import ctypes
    rng = np.random.default_rng(3 + mode)
    count, numel = 4, 37 * 41
    ps = [rng_bf16(rng, numel, 0.02) for _ in range(count)]
    upd = rng_bf16(rng, count * numel, 0.05)
    seeds = [int(s) for s in rng.integers(0, 2**32, count)]
    inj = rng.integers(0, 65536, count * numel).astype(np.uint16)
    pd = [u16_to_dev(p) for p in ps]
    ud = u16_to_dev(upd)
    inj_d = np_to_dev(inj.view(np.int16)) if mode == O.NOISE_INJECT else None
    check(L, L.msr_muon_apply(ptr_array([t.data_ptr() for t in pd]), ud.data_ptr(), numel, count, 0.02, 0.01, 1.6583,
                              ptr_array(seeds, ctypes.c_uint32), mode, ptr(inj_d), stream()))
    for i in range(count):
        spec = O.NoiseSpec(mode, seeds[i], 0, inj[i * numel:(i + 1) * numel] if mode == O.NOISE_INJECT else None)
        exp = O.muon_apply(ps[i], upd[i * numel:(i + 1) * numel], 0.02, 0.01, 1.6583, spec)
        assert np.array_equal(dev_to_u16(pd[i]), exp), i


# ---------------------------------------------------------------------------
# (b) MFMA GEMM and Newton-Schulz
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M,N,K,batch,alpha,beta,diag", [(256, 256, 128, 1, 1.0, 0.0, 0.0),
                                                         (512, 768, 384, 2, 0.5, -1.25, 3.4445),
                                                         (256, 512, 1024, 3, 2.0315, -4.775, 0.0)])
def test_gemm_nt_vs_torch_fp32(L, M, N, K, batch, alpha, beta, diag):
    torch.manual_seed(M + N + K)
    P = torch.randn(batch, M, K, device=DEV).to(torch.bfloat16)
    Q = torch.randn(batch, N, K, device=DEV).to(torch.bfloat16)
    C = torch.randn(batch, M, N, device=DEV).to(torch.bfloat16)
    D = torch.empty(batch, M, N, device=DEV, dtype=torch.bfloat16)
    check(L, L.msr_gemm_nt(P.data_ptr(), K, M * K, Q.data_ptr(), K, N * K, C.data_ptr(), N, M * N, D.data_ptr(), N,
                           M * N, M, N, K, batch, alpha, beta, diag, stream()), "gemm")
    ref = alpha * torch.matmul(P.float(), Q.float().transpose(1, 2).contiguous()) + beta * C.float()
    ref = ref + diag * torch.eye(M, N, device=DEV)
    err = (D.float() - ref).abs()
    tol = 2.0 ** -8 * ref.abs() + 1e-5 * ref.abs().max()
    assert bool((err <= tol).all()), float((err - tol).max())


@pytest.mark.parametrize("M,N,K,batch,alpha,beta,pad", [(256, 256, 128, 1, 1.0, 0.0, 0), (512, 768, 384, 2, 0.5, -1.25, 8),
                                                        (256, 512, 1024, 3, 1.0, 3.4445, 0), (768, 256, 256, 9, 1.0, 0.0, 16)])
def test_gemm_nn_vs_torch_fp32(L, M, N, K, batch, alpha, beta, pad):
    """K-major Q (the X' = B X + a X product of Newton-Schulz): transposing LDS reads."""
    torch.manual_seed(M + 3 * N + K)
    ldq = N + pad
    P = torch.randn(batch, M, K, device=DEV).to(torch.bfloat16)
    Qs = torch.randn(batch, K, ldq, device=DEV).to(torch.bfloat16)
    C = torch.randn(batch, M, N, device=DEV).to(torch.bfloat16)
    D = torch.empty(batch, M, N, device=DEV, dtype=torch.bfloat16)
    check(L, L.msr_gemm_nn(P.data_ptr(), K, M * K, Qs.data_ptr(), ldq, K * ldq, C.data_ptr(), N, M * N, D.data_ptr(),
                           N, M * N, M, N, K, batch, alpha, beta, 0.0, stream()), "gemm nn")
    ref = alpha * torch.matmul(P.float(), Qs[:, :, :N].float().contiguous()) + beta * C.float()
    err = (D.float() - ref).abs()
    tol = 2.0 ** -8 * ref.abs() + 1e-5 * ref.abs().max()
    assert bool((err <= tol).all()), float((err - tol).max())


@pytest.mark.parametrize("M,N,K,batch,with_c", [
    (512, 1024, 256, 48, False),    # 8 tiles per matrix, 384 tiles: work-groups take 1-2 tiles each
    (512, 1024, 256, 48, True),     # the same with C (stores bounded per element)
    (2048, 2304, 128, 8, False),    # 72 tiles per matrix (tile ranges spread over the XCDs), 576 tiles
    (2048, 2048, 128, 136, False),  # 8704 tiles: more than 32 per CU, one tile per work-group
])
def test_gemm_tiles_per_work_group(L, M, N, K, batch, with_c):
    """Launches whose work-groups walk several tiles (one work-group per CU, the next
    tile's first slab loaded during the epilogue), and one long enough to run a tile
    per work-group: every product equals the same product launched alone, bit for bit,
    and torch's fp32 product within bf16 rounding."""
    torch.manual_seed(M + N + K + batch)
    P = torch.randn(batch, M, K, device=DEV).to(torch.bfloat16)
    Q = torch.randn(batch, N, K, device=DEV).to(torch.bfloat16)
    C = torch.randn(batch, M, N, device=DEV).to(torch.bfloat16) if with_c else None
    beta = -1.25 if with_c else 0.0
    D = torch.empty(batch, M, N, device=DEV, dtype=torch.bfloat16)

    def gemm(b0, nb, out):
        cp = C[b0].data_ptr() if with_c else None
        check(L, L.msr_gemm_nt(P[b0].data_ptr(), K, M * K, Q[b0].data_ptr(), K, N * K, cp, N, M * N, out.data_ptr(),
                               N, M * N, M, N, K, nb, 1.0, beta, 0.0, stream()), "gemm")
    gemm(0, batch, D)
    one = torch.empty(1, M, N, device=DEV, dtype=torch.bfloat16)
    for b in sorted({0, 1, batch // 2, batch - 1}):
        gemm(b, 1, one)
        assert torch.equal(one[0].view(torch.int16), D[b].view(torch.int16)), b
        ref = torch.matmul(P[b].float(), Q[b].float().t().contiguous())
        if with_c:
            ref = ref + beta * C[b].float()
        err = (D[b].float() - ref).abs()
        tol = 2.0 ** -8 * ref.abs() + 1e-5 * ref.abs().max()
        assert bool((err <= tol).all()), (b, float((err - tol).max()))


def test_gemm_nn_equals_nt_on_transposed_operand(L):
    """The NN product with Q equals the NT product with Q^T bit for bit: same fp32
    accumulation order and the same MFMA operand layout, only the LDS path differs."""
    torch.manual_seed(11)
    M, N, K, batch = 512, 768, 512, 2
    P = torch.randn(batch, M, K, device=DEV).to(torch.bfloat16)
    Q = torch.randn(batch, K, N, device=DEV).to(torch.bfloat16)
    QT = Q.transpose(1, 2).contiguous()
    C = torch.randn(batch, M, N, device=DEV).to(torch.bfloat16)
    D1 = torch.empty(batch, M, N, device=DEV, dtype=torch.bfloat16)
    D2 = torch.empty_like(D1)
    check(L, L.msr_gemm_nn(P.data_ptr(), K, M * K, Q.data_ptr(), N, K * N, C.data_ptr(), N, M * N, D1.data_ptr(), N,
                           M * N, M, N, K, batch, 1.0, 3.4445, 0.0, stream()), "gemm nn")
    check(L, L.msr_gemm_nt(P.data_ptr(), K, M * K, QT.data_ptr(), K, N * K, C.data_ptr(), N, M * N, D2.data_ptr(), N,
                           M * N, M, N, K, batch, 1.0, 3.4445, 0.0, stream()), "gemm nt")
    assert torch.equal(D1, D2)


# Newton-Schulz tolerance against the exact iteration (O.ns_fp32: the same quintic in
# fp32 throughout, pinned by its closed form on singular values): 1e-2 relative
# Frobenius, the contract's bound.  Measured 0.46-0.83e-2 on Gaussian inputs; the
# reference's own bf16 op sequence (O.ns_bf16_torch) is 1.7-4.8e-2 from it.
NS_TOL = 1e-2


def ns_emul_step(X, first, a, b, c):
    """One iteration of this library's Newton-Schulz in float64 from a bf16 iterate X
    (wide orientation, [batch, m, n]), with its bf16 roundings:
      first: x0 = X 2^-e (e = exponent of ||X||_F), s = 2^e / (||X||_F + 1e-7), else s = 1;
      A  = bf16(s^2 x0 x0^T),            rho = diag(s^2 x0 x0^T) - diag(A);
      B' = c A A + b A + a I + diag(rho (b + 2 c diag(A))),   B = bf16(B'),  r = diag(B') - diag(B);
      X' = bf16(s (B x0 + bf16(r) * x0)).
    Returns X' (float64 holding bf16 values)."""
    rb = lambda t: t.to(torch.bfloat16).double()  # noqa: E731
    x0 = X.double()
    if first:
        nrm = x0.float().pow(2).sum(dim=(-2, -1)).sqrt()          # fp32 sum of squares, as the device
        e = torch.frexp(nrm).exponent
        x0 = torch.ldexp(x0, -e.double()[:, None, None])
        s = (torch.ldexp(torch.ones_like(nrm.double()), e.double()) / (nrm.double() + 1e-7))[:, None, None]
    else:
        s = torch.ones(X.size(0), 1, 1, dtype=torch.float64, device=X.device)
    Af = (s * s) * (x0 @ x0.mT)
    A = rb(Af)
    rho = torch.diagonal(Af, dim1=-2, dim2=-1) - torch.diagonal(A, dim1=-2, dim2=-1)
    dA = torch.diagonal(A, dim1=-2, dim2=-1)
    Bf = c * (A @ A) + b * A + torch.diag_embed(a + rho * (b + 2 * c * dA))
    B = rb(Bf)
    r = torch.diagonal(Bf, dim1=-2, dim2=-1) - torch.diagonal(B, dim1=-2, dim2=-1)
    return rb(s * (B @ x0 + rb(r)[..., None] * x0))


def bf16_ulps(x, ref):
    """|x - ref| in units of the bf16 spacing at ref (both hold bf16 values)."""
    ref = ref.double()
    sp = torch.ldexp(torch.ones_like(ref), torch.frexp(ref).exponent - 8)
    sp = torch.where(ref == 0, torch.full_like(ref, 2.0 ** -133), sp)
    return (x.double() - ref).abs() / sp


@pytest.mark.parametrize("rows,cols,batch", [(1024, 1536, 2), (1536, 1024, 2), (100, 60, 3), (320, 192, 2)])
def test_newton_schulz_iterations_vs_emulation(L, rows, cols, batch):
    """Every iteration of msr_newton_schulz against a float64 emulation of it started from
    the device's previous iterate (NS with steps = k returns X_k): the prescaled first
    products, the upper-tile storage of A and B' read back transposed (4 x 4 tiles of A at
    1024 x 1536 run every K range of the mixed-layout loop), the diagonal residuals and the
    transposed store of tall outputs.  The device sums in fp32 in its own order, so a few
    elements round the other way: those few, within 2 bf16 ulps except where a result is
    far below the matrix's typical magnitude (its ulp is then below the fp32 error of the
    sum), and the whole within 5e-4 relative Frobenius.  A wrong residual, alpha or tile
    read moves the result by 1e-3 or more."""
    from muon_sr_amd.muon import newton_schulz, NS_COEFFS
    a, b, c = NS_COEFFS
    torch.manual_seed(rows + cols)
    G = (torch.randn(batch, rows, cols, device=DEV) * 1e-3).to(torch.bfloat16)
    tall = rows > cols
    wide = lambda t: t.mT if tall else t  # noqa: E731
    prev = G
    for k in range(3):
        Xk1 = newton_schulz(G, steps=k + 1)
        emu = ns_emul_step(wide(prev), k == 0, a, b, c)
        u = bf16_ulps(wide(Xk1), emu)
        frac = (u > 0).double().mean().item()
        rel = rel_fro(wide(Xk1), emu)
        big = emu.abs() >= 0.25 * emu.pow(2).mean().sqrt()
        print(f"NS {rows}x{cols} iteration {k + 1}: max {u.max().item():.0f} ulp ({u[big].max().item():.0f} "
              f"on typical elements), {frac:.2e} of elements differ, rel {rel:.2e}")
        assert u[big].max().item() <= 2, (k, u[big].max().item())
        assert frac <= 5e-3, (k, frac)
        assert rel <= 5e-4, (k, rel)
        prev = Xk1


@pytest.mark.parametrize("shape", [(256, 256), (3, 128, 320), (2, 320, 128), (1024, 256), (256, 1024),
                                   (100, 60), (61, 99), (2, 512, 1536), (64, 64), (37, 1000)])
def test_newton_schulz_vs_fp32(L, shape):
    """Within NS_TOL of the exact iteration, and closer to it than the reference's own
    bf16 op sequence is."""
    from muon_sr_amd.muon import newton_schulz
    torch.manual_seed(sum(shape))
    G = (torch.randn(*shape) * 1e-3).to(torch.bfloat16)
    out = newton_schulz(G.to(DEV)).cpu().float()
    exact = O.ns_fp32(G.double()).double()
    ref16 = O.ns_bf16_torch(G).float()
    e_exact, e_ref, e_vs_ref = rel_fro(out, exact), rel_fro(ref16, exact), rel_fro(out, ref16)
    print(f"NS {shape}: vs exact NS {e_exact:.2e}; reference bf16 NS vs exact {e_ref:.2e}, vs ours {e_vs_ref:.2e}")
    assert e_exact < NS_TOL
    assert e_exact < e_ref


@pytest.mark.parametrize("shape,offset", [((2, 192, 320), 0), ((3, 61, 99), 0), ((2, 320, 128), 0),
                                          ((2, 192, 320), 1), ((1, 1024, 4096), 0)])
def test_ns_normalize_exact(L, shape, offset):
    """steps=0 returns the reference's bf16 normalisation bf16(G / d), d =
    bf16(bf16(||G||_F) + 1e-7) (muon_sr/muon_sr.py:93), for the 16-byte and the
    element-wise prologue (offset 1 makes the input pointer unaligned)."""
    from muon_sr_amd.muon import newton_schulz
    torch.manual_seed(7)
    n = int(np.prod(shape))
    flat = (torch.randn(n + offset) * 3e-3).to(torch.bfloat16)
    G = flat[offset:].view(shape)
    Gd = flat.to(DEV)[offset:].view(shape)
    X0 = newton_schulz(Gd, steps=0).cpu()
    g64 = G.double()
    nrm = g64.pow(2).sum(dim=(-2, -1), keepdim=True).sqrt()
    nb = nrm.float().to(torch.bfloat16).double()
    # the device sums in fp32 in its own order: keep clear of bf16 rounding ties of the norm
    ulp = torch.ldexp(torch.ones_like(nb), torch.frexp(nb).exponent - 8)   # bf16 spacing at nb
    mid = (nrm - nb).abs() - ulp / 2
    assert bool((mid.abs() > 1e-4 * nb).all()), "input too close to a bf16 rounding boundary of the norm"
    d = (nb.float() + 1e-7).to(torch.bfloat16).float()
    exp = (G.float() / d).to(torch.bfloat16)
    assert torch.equal(X0.view(torch.int16), exp.view(torch.int16))


def test_newton_schulz_batch_invariant_and_steps0(L):
    from muon_sr_amd.muon import newton_schulz
    torch.manual_seed(0)
    G = (torch.randn(4, 192, 320, device=DEV) * 1e-2).to(torch.bfloat16)
    full = newton_schulz(G)
    for i in range(4):
        one = newton_schulz(G[i:i + 1].clone())
        assert torch.equal(full[i:i + 1], one), i
    X0 = newton_schulz(G, steps=0).float()
    nrm = G.float().norm(dim=(-2, -1), keepdim=True).to(torch.bfloat16).float()
    exp = (G.float() / (nrm + 1e-7).to(torch.bfloat16).float()).to(torch.bfloat16).float()
    assert rel_fro(X0, exp) < 1e-2


@pytest.mark.parametrize("batch,rows,cols", [(300, 200, 300), (300, 300, 200)])
def test_newton_schulz_many_tiles_batch_invariant(L, batch, rows, cols):
    """Hundreds of padded matrices: the products' work-groups each walk several tiles and
    the last product's stores are bounded (partial tiles), wide and tall (transposed
    store).  Every matrix equals its own Newton-Schulz, bit for bit."""
    from muon_sr_amd.muon import newton_schulz
    gen = torch.Generator(device=DEV)
    gen.manual_seed(batch + rows)
    G = (torch.randn(batch, rows, cols, device=DEV, generator=gen) * 1e-2).to(torch.bfloat16)
    full = newton_schulz(G)
    for i in (0, 1, batch // 2, batch - 1):
        assert torch.equal(full[i:i + 1], newton_schulz(G[i:i + 1].clone())), i


@pytest.mark.parametrize("batch,rows,cols", [(3, 256, 512), (2, 640, 256), (3, 100, 60), (130, 256, 256), (2, 61, 99),
                                             (150, 300, 700), (150, 700, 300)])
@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8, O.NOISE_INJECT])
def test_muon_ns_apply_equals_ns_then_apply(L, batch, rows, cols, mode):
    """msr_muon_ns_apply (the apply done by the last Newton-Schulz product's store) equals
    msr_newton_schulz followed by msr_muon_apply bit for bit: wide, tall and padded shapes,
    columns that are no multiple of 8 (element-wise stores and noise), more than 128
    matrices (several apply launches), launches whose work-groups walk several tiles and
    misaligned parameters."""
    import ctypes
    from muon_sr_amd.muon import newton_schulz, NS_COEFFS
    a, b, c = NS_COEFFS
    gen = torch.Generator(device=DEV)
    gen.manual_seed(batch * rows + cols + mode)
    U = (torch.randn(batch, rows, cols, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16)
    numel = rows * cols
    misalign = (batch % 2 == 1)
    store = torch.randn(batch * (numel + 8), device=DEV, generator=gen).mul(0.02).to(torch.bfloat16)
    # parameter i at element offset i*(numel+8) (+1 for odd i when misaligned)
    offs = [i * (numel + 8) + (1 if misalign and i % 2 else 0) for i in range(batch)]
    p_ref = [store[o:o + numel].clone() for o in offs]
    seeds = [(0x9E3779B9 * (i + 1)) & 0xFFFFFFFF for i in range(batch)]
    inj = torch.randint(0, 65536, (batch * numel,), device=DEV, generator=gen, dtype=torch.int32).to(torch.int16) \
        if mode == O.NOISE_INJECT else None
    lr, wd, scale = 0.02, 0.01, max(1.0, rows / cols) ** 0.5
    X = newton_schulz(U)
    pref_stack = torch.stack(p_ref)
    seeds_c = ptr_array(seeds, ctypes.c_uint32)
    check(L, L.msr_muon_apply(ptr_array([t.data_ptr() for t in pref_stack]), X.data_ptr(), numel, batch, lr, wd, scale,
                              seeds_c, mode, ptr(inj), stream()), "msr_muon_apply")
    nb = ctypes.c_size_t(0)
    check(L, L.msr_ns_workspace_bytes(batch, rows, cols, ctypes.byref(nb)), "ws")
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    params = [store[o:o + numel] for o in offs]
    before = store.clone()
    check(L, L.msr_muon_ns_apply(U.data_ptr(), ptr_array([t.data_ptr() for t in params]), seeds_c, batch, rows, cols, 5,
                                 a, b, c, lr, wd, scale, mode, ptr(inj), ws.data_ptr(), nb.value, stream()),
          "msr_muon_ns_apply")
    for i in range(batch):
        assert torch.equal(params[i].view(torch.int16), pref_stack[i].view(torch.int16)), i
    # memory between and around the parameters is untouched
    mask = torch.ones(store.numel(), dtype=torch.bool, device=DEV)
    for o in offs:
        mask[o:o + numel] = False
    assert torch.equal(store[mask].view(torch.int16), before[mask].view(torch.int16))


@pytest.mark.parametrize("batch,rows,cols,first,f32,nest", [
    (3, 256, 512, 0, False, True), (2, 640, 256, 1, False, True), (3, 100, 60, 2, False, True),
    (130, 64, 128, 0, False, True), (2, 61, 99, 0, True, False), (1, 96, 96, 0, True, True),
    (4, 72, 40, 3, False, False)])
@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8, O.NOISE_INJECT])
@pytest.mark.parametrize("fused_apply", [True, False])
def test_muon_fused_step_equals_separate_calls(L, batch, rows, cols, first, f32, nest, mode, fused_apply):
    """msr_muon_fused_step (the momentum step made inside the Newton-Schulz prologue, and
    the apply in the last product's store or, with `out`, the NS output) equals
    msr_muon_prepare over the momentum stack, then msr_newton_schulz, then msr_muon_apply,
    bit for bit: momentum rows, parameters or NS output.  Wide, tall, padded and
    non-multiple-of-8 shapes, a chunk that starts inside its stack (`first`: the noise
    offsets continue the stack's), fp32 gradients, nesterov off, more matrices than one
    prologue and one apply launch take (96, 128), all three noise streams."""
    import ctypes
    from muon_sr_amd.muon import newton_schulz, NS_COEFFS
    a, b, c = NS_COEFFS
    gen = torch.Generator(device=DEV)
    gen.manual_seed(batch * rows + cols + 7 * mode + first)
    numel = rows * cols
    total = first + batch                      # the momentum stack holds `total` matrices
    grads = [(torch.randn(rows, cols, device=DEV, generator=gen) * 1e-3) for _ in range(batch)]
    grads = [g if f32 else g.to(torch.bfloat16) for g in grads]
    stack0 = (torch.randn(total, rows, cols, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16)
    params0 = (torch.randn(batch, rows, cols, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    inj_p = torch.randint(0, 65536, (total * numel,), device=DEV, generator=gen, dtype=torch.int32).to(torch.int16) \
        if mode == O.NOISE_INJECT else None
    inj_a = torch.randint(0, 65536, (batch * numel,), device=DEV, generator=gen, dtype=torch.int32).to(torch.int16) \
        if mode == O.NOISE_INJECT else None
    beta, pseed = 0.95, 0x2545F491
    seeds = [(0x9E3779B9 * (i + 3)) & 0xFFFFFFFF for i in range(batch)]
    lr, wd, scale = 0.02, 0.01, max(1.0, rows / cols) ** 0.5
    # separate calls: prepare over rows first.. of the stack (noise offsets from the stack's start)
    stack_ref = stack0.clone()
    work = torch.empty(batch, rows, cols, dtype=torch.bfloat16, device=DEV)
    gtab = ptr_array([g.data_ptr() for g in grads])
    # msr_muon_prepare numbers its noise from its own first row: seed and offsets of rows first..
    # are those of the whole stack only when first == 0, so the reference runs it over the whole
    # stack with the chunk's gradients in rows first.. and zeros before
    if first:
        pad = [torch.zeros(rows, cols, dtype=grads[0].dtype, device=DEV) for _ in range(first)]
        full = pad + grads
        work_full = torch.empty(total, rows, cols, dtype=torch.bfloat16, device=DEV)
        check(L, L.msr_muon_prepare(ptr_array([g.data_ptr() for g in full]), int(f32), stack_ref.data_ptr(),
                                    work_full.data_ptr(), numel, total, beta, int(nest), pseed, mode, ptr(inj_p),
                                    stream()), "msr_muon_prepare")
        work = work_full[first:].contiguous()
        stack_ref[:first] = stack0[:first]
    else:
        check(L, L.msr_muon_prepare(gtab, int(f32), stack_ref.data_ptr(), work.data_ptr(), numel, batch, beta,
                                    int(nest), pseed, mode, ptr(inj_p), stream()), "msr_muon_prepare")
    X = newton_schulz(work)
    p_ref = params0.clone()
    seeds_c = ptr_array(seeds, ctypes.c_uint32)
    check(L, L.msr_muon_apply(ptr_array([p_ref[i].data_ptr() for i in range(batch)]), X.data_ptr(), numel, batch, lr, wd,
                              scale, seeds_c, mode, ptr(inj_a), stream()), "msr_muon_apply")
    # the fused call
    stack = stack0.clone()
    prm = params0.clone()
    nb = ctypes.c_size_t(0)
    check(L, L.msr_ns_workspace_bytes(batch, rows, cols, ctypes.byref(nb)), "ws")
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    out = None if fused_apply else torch.empty(batch, rows, cols, dtype=torch.bfloat16, device=DEV)
    check(L, L.msr_muon_fused_step(gtab, int(f32), stack[first].data_ptr(), first, batch, rows, cols, beta, int(nest),
                                   pseed, 5, a, b, c, None if fused_apply else out.data_ptr(),
                                   ptr_array([prm[i].data_ptr() for i in range(batch)]) if fused_apply else None,
                                   seeds_c if fused_apply else None, lr, wd, scale, mode, ptr(inj_p),
                                   ptr(inj_a) if fused_apply else None, ws.data_ptr(), nb.value, stream()),
          "msr_muon_fused_step")
    torch.cuda.synchronize()
    assert torch.equal(stack.view(torch.int16), stack_ref.view(torch.int16))   # rows before `first` untouched
    if fused_apply:
        assert torch.equal(prm.view(torch.int16), p_ref.view(torch.int16))
    else:
        assert torch.equal(out.view(torch.int16), X.view(torch.int16))
        assert torch.equal(prm.view(torch.int16), params0.view(torch.int16))


@pytest.mark.parametrize("steps", [1, 2, 3])
@pytest.mark.parametrize("rows,cols", [(256, 512), (512, 256)])
@pytest.mark.parametrize("mode", [O.NOISE_TRITON, O.NOISE_PHILOX8])
def test_muon_fused_step_few_iterations(L, steps, rows, cols, mode):
    """ns_steps below the default: with one iteration the first X' product both takes the
    normalisation factor s (the prologue leaves X0 unscaled) and applies the update in its
    store.  msr_muon_fused_step equals msr_muon_prepare + msr_newton_schulz(steps) +
    msr_muon_apply bit for bit, wide and tall (muon_sr/triton_muon_sr.py:18-80; ns_steps is a
    param-group key, muon_sr/triton_muon_sr.py:198-200)."""
    import ctypes
    from muon_sr_amd.muon import newton_schulz, NS_COEFFS
    a, b, c = NS_COEFFS
    gen = torch.Generator(device=DEV)
    gen.manual_seed(31 * steps + rows + mode)
    batch, numel = 3, rows * cols
    grads = [(torch.randn(rows, cols, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16) for _ in range(batch)]
    stack0 = (torch.randn(batch, rows, cols, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16)
    params0 = (torch.randn(batch, rows, cols, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    beta, pseed = 0.95, 0x1B873593
    seeds = [(0x85EBCA6B * (i + 5)) & 0xFFFFFFFF for i in range(batch)]
    lr, wd, scale = 0.02, 0.01, max(1.0, rows / cols) ** 0.5
    gtab = ptr_array([g.data_ptr() for g in grads])
    seeds_c = ptr_array(seeds, ctypes.c_uint32)
    stack_ref = stack0.clone()
    work = torch.empty(batch, rows, cols, dtype=torch.bfloat16, device=DEV)
    check(L, L.msr_muon_prepare(gtab, 0, stack_ref.data_ptr(), work.data_ptr(), numel, batch, beta, 1, pseed, mode,
                                None, stream()), "msr_muon_prepare")
    X = newton_schulz(work, steps=steps)
    p_ref = params0.clone()
    check(L, L.msr_muon_apply(ptr_array([p_ref[i].data_ptr() for i in range(batch)]), X.data_ptr(), numel, batch, lr, wd,
                              scale, seeds_c, mode, None, stream()), "msr_muon_apply")
    stack, prm = stack0.clone(), params0.clone()
    nb = ctypes.c_size_t(0)
    check(L, L.msr_ns_workspace_bytes(batch, rows, cols, ctypes.byref(nb)), "ws")
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    check(L, L.msr_muon_fused_step(gtab, 0, stack.data_ptr(), 0, batch, rows, cols, beta, 1, pseed, steps, a, b, c, None,
                                   ptr_array([prm[i].data_ptr() for i in range(batch)]), seeds_c, lr, wd, scale, mode,
                                   None, None, ws.data_ptr(), nb.value, stream()), "msr_muon_fused_step")
    torch.cuda.synchronize()
    assert torch.equal(stack.view(torch.int16), stack_ref.view(torch.int16))
    assert torch.equal(prm.view(torch.int16), p_ref.view(torch.int16))
    assert not torch.equal(prm.view(torch.int16), params0.view(torch.int16))


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (2048, 2048),
                                       (5632, 2048), (2048, 5632)])
def test_muon_fused_step_at_config_shapes(L, rows, cols):
    """At the Llama-3-8B (config 5) and config-4 shapes, two matrices of a chunk that starts at
    row 1 of its momentum stack: msr_muon_fused_step with the apply in the last product's store,
    as the classes run it for wide and tall matrices alike (tall ones store that product
    transposed), equals msr_muon_prepare + msr_newton_schulz + msr_muon_apply bit for bit
    (momentum and parameters), in the reference's noise stream.  Tall shapes also take the NS
    output (`out`) followed by one msr_muon_apply launch, which must give the same bits."""
    import ctypes
    from muon_sr_amd.muon import newton_schulz, NS_COEFFS
    a, b, c = NS_COEFFS
    gen = torch.Generator(device=DEV)
    gen.manual_seed(rows + cols)
    batch, first, total = 2, 1, 3
    numel = rows * cols
    mode = O.NOISE_TRITON
    grads = [(torch.randn(rows, cols, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16) for _ in range(batch)]
    stack0 = (torch.randn(total, rows, cols, device=DEV, generator=gen) * 1e-3).to(torch.bfloat16)
    params0 = (torch.randn(batch, rows, cols, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    beta, pseed, lr, wd, scale = 0.95, 0x1234567, 0.02, 0.01, max(1.0, rows / cols) ** 0.5
    seeds = [(0x85EBCA6B * (i + 1)) & 0xFFFFFFFF for i in range(batch)]
    seeds_c = ptr_array(seeds, ctypes.c_uint32)
    # separate calls over the whole stack (row 0 gets a zero gradient and is restored)
    full = [torch.zeros(rows, cols, dtype=torch.bfloat16, device=DEV)] + grads
    stack_ref = stack0.clone()
    work = torch.empty(total, rows, cols, dtype=torch.bfloat16, device=DEV)
    check(L, L.msr_muon_prepare(ptr_array([g.data_ptr() for g in full]), 0, stack_ref.data_ptr(), work.data_ptr(),
                                numel, total, beta, 1, pseed, mode, None, stream()), "msr_muon_prepare")
    stack_ref[0] = stack0[0]
    X = newton_schulz(work[first:])
    p_ref = params0.clone()
    check(L, L.msr_muon_apply(ptr_array([p_ref[i].data_ptr() for i in range(batch)]), X.data_ptr(), numel, batch, lr,
                              wd, scale, seeds_c, mode, None, stream()), "msr_muon_apply")
    del work
    nb = ctypes.c_size_t(0)
    check(L, L.msr_ns_workspace_bytes(batch, rows, cols, ctypes.byref(nb)), "ws")
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    gtab = ptr_array([g.data_ptr() for g in grads])
    # the fused call as the classes make it: the update applied in the last product's store
    stack, prm = stack0.clone(), params0.clone()
    ptab = ptr_array([prm[i].data_ptr() for i in range(batch)])
    check(L, L.msr_muon_fused_step(gtab, 0, stack[first].data_ptr(), first, batch, rows, cols, beta, 1, pseed, 5,
                                   a, b, c, None, ptab, seeds_c, lr, wd, scale, mode, None, None,
                                   ws.data_ptr(), nb.value, stream()), "msr_muon_fused_step")
    torch.cuda.synchronize()
    assert torch.equal(stack.view(torch.int16), stack_ref.view(torch.int16))
    assert torch.equal(prm.view(torch.int16), p_ref.view(torch.int16))
    if rows > cols:
        # the same step with the NS output written, then one apply launch
        stack, prm = stack0.clone(), params0.clone()
        out = torch.empty(batch, rows, cols, dtype=torch.bfloat16, device=DEV)
        ptab = ptr_array([prm[i].data_ptr() for i in range(batch)])
        check(L, L.msr_muon_fused_step(gtab, 0, stack[first].data_ptr(), first, batch, rows, cols, beta, 1, pseed,
                                       5, a, b, c, out.data_ptr(), None, None, lr, wd, scale, mode, None, None,
                                       ws.data_ptr(), nb.value, stream()), "msr_muon_fused_step")
        check(L, L.msr_muon_apply(ptab, out.data_ptr(), numel, batch, lr, wd, scale, seeds_c, mode, None, stream()),
              "msr_muon_apply")
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), X.view(torch.int16))
        assert torch.equal(stack.view(torch.int16), stack_ref.view(torch.int16))
        assert torch.equal(prm.view(torch.int16), p_ref.view(torch.int16))


@pytest.mark.parametrize("shape", [(2, 128, 256), (2, 256, 96)])
@pytest.mark.parametrize("e", [-40, -20, -17, -16, -4, 0, 16, 17, 40])
def test_newton_schulz_prologue_scales(L, shape, e):
    """The prologue keeps X0 = u when the exponent e of ||u||_F has |e| <= 16 and rescales
    it by 2^-e beyond (products of unscaled tiny or huge values would leave fp32's normal
    range).  For ||u||_F around 2^e, e from -40 to 40 on both sides of the switch, the output
    stays within the Newton-Schulz bound of the exact iteration of the same input (with its
    1e-7, which dominates the smallest norms)."""
    from muon_sr_amd.muon import newton_schulz
    g = torch.Generator().manual_seed(11)
    G = torch.randn(*shape, generator=g)
    G = G / G[0].norm()
    u = (G * 2.0 ** e).to(torch.bfloat16)
    X = newton_schulz(u.to(DEV)).float().cpu()
    ref = O.ns_fp32(u)
    assert torch.isfinite(X).all()
    assert rel_fro(X, ref) < 1e-2, rel_fro(X, ref)

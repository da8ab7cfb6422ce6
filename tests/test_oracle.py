"""Pins for the CPU oracle (no GPU needed).

Each oracle function is checked against (a) the golden vectors written from the
reference's own kernels (tests/golden/make_golden.py), (b) published
known-answer vectors, and/or (c) closed forms and brute force, chosen so that a
dropped term, a wrong sign/index or a transposed operand fails.
"""
import numpy as np
import pytest
import torch

import oracle as O
import oracle.ref  # noqa: F401  (module whose seed function the slip test swaps)


def bf(u16):
    return torch.from_numpy(np.asarray(u16, np.uint16).view(np.int16).copy()).view(torch.bfloat16)


# ---------------------------------------------------------------------------
# Philox and seeds
# ---------------------------------------------------------------------------

# Random123 known-answer vectors for Philox4x32-10 (kat_vectors of the Random123
# distribution): counter, key -> output.
PHILOX_KAT = [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]


@pytest.mark.parametrize("ctr,key,expect", PHILOX_KAT)
def test_philox_kat(ctr, key, expect):
    assert [int(v) for v in O.philox(ctr, key)] == expect


def test_seed_key_typing():
    # i32 seeds: no high word unless seed + k wraps past 2^31 - 1
    assert O.seed_key(5, 2) == (7, 0)
    assert O.seed_key(0x7FFFFFFF, 0) == (0x7FFFFFFF, 0)
    assert O.seed_key(0x7FFFFFFF, 1) == (0x80000000, 0xFFFFFFFF)
    assert O.seed_key(0x7FFFFFFE, 2) == (0x80000000, 0xFFFFFFFF)
    assert O.seed_key(0x7FFFFFFE, 1) == (0x7FFFFFFF, 0)
    # seeds >= 2^31 are i64 arguments: no wrap at 2^32, the carry lands in the high word
    assert O.seed_key(0x80000000, 1) == (0x80000001, 0)
    assert O.seed_key(0xFFFFFFFE, 1) == (0xFFFFFFFF, 0)
    assert O.seed_key(0xFFFFFFFF, 1) == (0, 1)
    assert O.seed_key(0xFFFFFFFE, 2) == (0, 1)


def test_noise_modes_are_philox_words():
    offs = np.array([0, 1, 7, 8, 12345, 2**31 - 1, 2**31, 2**32 + 5, 2**40 + 3], np.int64)
    tri = O.noise16(O.NOISE_TRITON, 0xABCDEF, offs)
    for o, v in zip(offs, tri):
        w = O.philox([int(o) & 0xFFFFFFFF, 0, 0, 0], [0xABCDEF, 0])
        assert v == w[0] & 0xFFFF
    p8 = O.noise16(O.NOISE_PHILOX8, 0xABCDEF, offs)
    for o, v in zip(offs, p8):
        o = int(o)
        w = O.philox([(o >> 3) & 0xFFFFFFFF, (o >> 35) & 0xFFFFFFFF, 0, 0], [0xABCDEF, 0])
        lane = o & 7
        assert v == (int(w[lane >> 1]) >> (16 * (lane & 1))) & 0xFFFF


def test_deterministic_seed():
    # muon_sr/triton_muon_sr.py:83-85 evaluated by hand for two cases
    assert O.deterministic_seed(1, 0, 0) == 2654435761
    assert O.deterministic_seed(3, 2, 1) == ((3 * 2654435761) ^ (2 * 1234567891) ^ 1) & 0xFFFFFFFF


# ---------------------------------------------------------------------------
# Stochastic rounding (brute force over every noise value)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("x", [1.0 + 2**-10, -3.14159, 1e-30, 65504.7, 2.5e-3])
def test_sr_exhaustive_noise(x):
    x = np.float32(x)
    noise = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    acc = np.zeros(65536, np.uint16)
    g = np.full(65536, x, np.float32)
    out = O.sr_accum(acc, g, O.NoiseSpec(O.NOISE_INJECT, inject=noise))
    bits = int(np.float32(x).view(np.uint32))
    lo, trunc = bits & 0xFFFF, bits >> 16
    up = (trunc + 1) & 0xFFFF
    assert set(np.unique(out).tolist()) <= {trunc, up}
    assert int((out == up).sum()) == lo          # P(up) = low16 / 2^16 exactly
    assert int((out == trunc).sum()) == 65536 - lo


def test_sr_exact_when_representable_and_unbiased():
    rng = np.random.default_rng(0)
    g = O.f32_to_bf16_rne(rng.standard_normal(4096).astype(np.float32))
    out = O.sr_accum(np.zeros(4096, np.uint16), g, O.NoiseSpec(O.NOISE_PHILOX8, 123))
    zero_sum = (O.bf16_to_f32(g) + np.float32(0)).astype(np.float32)
    assert np.array_equal(O.bf16_to_f32(out), zero_sum)
    # unbiasedness over 10^4 draws of one value, within 3 sigma
    x = np.float32(1.0 + 0.3 * 2**-7)
    draws = 10000
    outs = O.sr_accum(np.zeros(draws, np.uint16), np.full(draws, x, np.float32),
                      O.NoiseSpec(O.NOISE_PHILOX8, 77))
    vals = O.bf16_to_f32(outs).astype(np.float64)
    ulp = 2.0 ** -7
    p = 0.3
    sigma = ulp * np.sqrt(p * (1 - p) / draws)
    assert abs(vals.mean() - float(x)) < 3 * sigma


# ---------------------------------------------------------------------------
# Codebook and quantizer
# ---------------------------------------------------------------------------

def test_codebooks_match_reference(golden):
    q = golden("quantize")
    q1, q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
    assert np.array_equal(q1.view(np.uint32), q["qmap1"].view(np.uint32))
    assert np.array_equal(q2.view(np.uint32), q["qmap2"].view(np.uint32))
    for Q in (q1, q2):
        assert Q.shape == (256,) and np.all(np.diff(Q) > 0) and Q[255] == 1.0
    assert q1[127] == 0.0 and q2[0] == 0.0
    assert np.array_equal(q1[:127], -q1[128:255][::-1])     # signed map is symmetric
    assert q1[0] == np.float32(-0.99296875) or abs(q1[0] + 0.99297) < 1e-5


@pytest.mark.parametrize("signed", [True, False])
def test_quantizer_matches_reference(golden, signed):
    q = golden("quantize")
    name = "signed" if signed else "unsigned"
    Q = q["qmap1"] if signed else q["qmap2"]
    got = O.quantize(q[f"x_{name}"], Q, signed)
    assert np.array_equal(got, q[f"code_{name}"])


@pytest.mark.parametrize("signed", [True, False])
def test_quantizer_is_nearest_code(signed):
    # Property: the code is a nearest codebook entry (ties and the signed
    # tiny-negative fix excepted), so a wrong index or compare direction fails.
    Q = O.create_dynamic_map(signed)
    rng = np.random.default_rng(3)
    x = rng.uniform(-1 if signed else 0, 1, 200000).astype(np.float32)
    codes = O.quantize(x, Q, signed).astype(np.int64)
    d_got = np.abs(Q[codes].astype(np.float64) - x)
    d_best = np.min(np.abs(Q[None, :].astype(np.float64) - x[:20000, None]), axis=1)
    assert np.all(d_got[:20000] <= d_best + 1e-7)
    if signed:
        neg = x < 0
        assert np.all(Q[codes[neg]] < 0)          # sign is preserved for negatives


# ---------------------------------------------------------------------------
# Kernels vs golden vectors
# ---------------------------------------------------------------------------

def _cases(z):
    return sorted({k.split("/")[0] for k in z.files})


def test_adamw8bit_matches_reference(golden):
    z = golden("adamw8bit")
    q1, q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
    for name in _cases(z):
        g = lambda k: z[f"{name}/{k}"]  # noqa: E731
        quant = bool(g("quantized"))
        block = int(g("block"))
        lr, b1, b2, eps, wd = (float(g(k)) for k in ("lr", "b1", "b2", "eps", "wd"))
        p, s1, s2 = g("p0"), g("s1_0"), g("s2_0")
        a1, a2 = (g("a1_0"), g("a2_0")) if quant else (None, None)
        for step in range(1, int(g("steps")) + 1):
            seed = int(g(f"seed_{step}"))
            bc1, bc2 = 1 - b1 ** step, 1 - b2 ** step
            gr = g(f"g_{step}")
            if quant:
                p, s1, s2, a1, a2 = O.adamw8bit(p, gr, s1, s2, a1, a2, q1, q2, block, True,
                                                lr, b1, b2, eps, wd, bc1, bc2,
                                                O.NoiseSpec(O.NOISE_TRITON, seed))
                assert np.array_equal(a1.view(np.uint32), g(f"a1_{step}").view(np.uint32)), (name, step)
                assert np.array_equal(a2.view(np.uint32), g(f"a2_{step}").view(np.uint32)), (name, step)
            else:
                p, s1, s2 = O.adamw8bit(p, gr, s1, s2, None, None, None, None, block, False,
                                        lr, b1, b2, eps, wd, bc1, bc2,
                                        O.NoiseSpec(O.NOISE_TRITON, seed),
                                        O.NoiseSpec(O.NOISE_TRITON, seed, 1),
                                        O.NoiseSpec(O.NOISE_TRITON, seed, 2))
            assert np.array_equal(p, g(f"p_{step}")), (name, step)
            assert np.array_equal(s1, g(f"s1_{step}")), (name, step)
            assert np.array_equal(s2, g(f"s2_{step}")), (name, step)


def test_adamw8bit_special_cases():
    q1, q2 = O.create_dynamic_map(True), O.create_dynamic_map(False)
    n, block = 512, 256
    rng = np.random.default_rng(1)
    p = O.f32_to_bf16_rne(rng.standard_normal(n).astype(np.float32) * 0.02)
    g = np.zeros(n, np.uint16)
    s1 = np.full(n, 127, np.uint8)
    s2 = np.zeros(n, np.uint8)
    a = np.zeros(2, np.float32)
    lr, wd = 1e-3, 0.1
    # zero gradient and zero state: p <- SR(p * (1 - lr*wd)); moments stay zero, absmax 0
    zero_noise = O.NoiseSpec(O.NOISE_INJECT, inject=np.zeros(n, np.uint16))
    p1, t1, t2, a1, a2 = O.adamw8bit(p, g, s1, s2, a, a, q1, q2, block, True, lr, 0.9, 0.95, 1e-8, wd,
                                     0.1, 0.05, zero_noise)
    expect = O.f32_to_bf16_trunc(O.bf16_to_f32(p) * (np.float32(1) - np.float32(lr) * np.float32(wd)))
    assert np.array_equal(p1, expect)
    assert np.all(t1 == 127) and np.all(t2 == 0) and np.all(a1 == 0) and np.all(a2 == 0)
    # non-finite gradients: weight unchanged, both moments decode to zero
    g2 = O.f32_to_bf16_rne(rng.standard_normal(n).astype(np.float32) * 1e-3)
    g2[[3, 300]] = [0x7FC0, 0xFF80]
    p2, u1, u2, b1_, b2_ = O.adamw8bit(p, g2, s1, s2, a, a, q1, q2, block, True, lr, 0.9, 0.95, 1e-8, wd,
                                       0.1, 0.05, zero_noise)
    assert p2[3] == p[3] and p2[300] == p[300]
    assert q1[u1[3]] == 0 and q2[u2[3]] == 0 and q1[u1[300]] == 0 and q2[u2[300]] == 0
    # first step: m = (1-b1) g, so the element with the largest finite |g| of a block
    # normalises to +-1 and codes to the map's end (Q1[255] = 1, Q1[0] = -0.99297; no -1 entry)
    gf = O.bf16_to_f32(g2[:256]).copy()
    gf[~np.isfinite(gf)] = 0
    i = int(np.argmax(np.abs(gf)))
    assert u1[i] == (255 if gf[i] > 0 else 0)
    assert u2[i] == 255


def test_adamw_bf16_matches_reference(golden):
    z = golden("elementwise")
    for tag in ("s_small", "s_wrap", "s_wrap2", "s_u32", "s_i64wrap"):
        k = lambda s: z[f"adamw/{tag}/{s}"]  # noqa: E731
        lr, b1, b2, eps, wd, bc, bcs = (float(v) for v in k("hyper"))
        seed = int(k("seed"))
        p, e, s = O.adamw_bf16(k("in_p"), k("in_g"), k("in_e"), k("in_s"), lr, b1, b2, eps, wd, bc, bcs,
                               O.NoiseSpec(O.NOISE_TRITON, seed), O.NoiseSpec(O.NOISE_TRITON, seed, 1),
                               O.NoiseSpec(O.NOISE_TRITON, seed, 2))
        assert np.array_equal(p, k("out_p")), tag
        assert np.array_equal(e, k("out_e")), tag
        assert np.array_equal(s, k("out_s")), tag


def test_sr_accum_matches_reference(golden):
    z = golden("elementwise")
    a1 = O.sr_accum(z["accum/in_acc"], z["accum/in_g"], O.NoiseSpec(O.NOISE_TRITON, 777))
    assert np.array_equal(a1, z["accum/out_bf16g"])
    a2 = O.sr_accum(z["accum/in_acc"], z["accum/in_g32"], O.NoiseSpec(O.NOISE_TRITON, 0x9E3779B9))
    assert np.array_equal(a2, z["accum/out_f32g"])


@pytest.mark.parametrize("nest", [1, 0])
def test_muon_prepare_matches_reference(golden, nest):
    z = golden("elementwise")
    k = lambda s: z[f"prepare/{nest}/{s}"]  # noqa: E731
    buf, u32, u16 = O.muon_prepare(k("in_g"), k("in_buf"), 0.95, bool(nest),
                                   O.NoiseSpec(O.NOISE_TRITON, int(k("seed"))))
    assert np.array_equal(buf, k("out_buf"))
    assert np.array_equal(u32.view(np.uint32), k("out_upd_f32").view(np.uint32))
    # the bf16 output is the RNE cast of the fp32 update (torch's CPU cast is RNE)
    rne = torch.from_numpy(k("out_upd_f32")).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(u16, rne)


def test_muon_prepare_fp32_gradient(golden):
    """The fp32-gradient path (the reference's per-parameter launch reads the gradient in
    its own dtype, muon_sr/triton_muon_sr.py:34): fp32 gradients holding bf16 values give
    the reference vectors' results exactly, and other fp32 values are not rounded to bf16
    first (an update computed from the bf16-rounded gradient differs)."""
    z = golden("elementwise")
    k = lambda s: z[f"prepare/1/{s}"]  # noqa: E731
    g32 = (k("in_g").astype(np.uint32) << 16).view(np.float32)
    spec = O.NoiseSpec(O.NOISE_TRITON, int(k("seed")))
    buf, u32, _ = O.muon_prepare(g32, k("in_buf"), 0.95, True, spec)
    assert np.array_equal(buf, k("out_buf"))
    assert np.array_equal(u32.view(np.uint32), k("out_upd_f32").view(np.uint32))
    rng = np.random.default_rng(0)
    g = (rng.standard_normal(4096) * 1e-3).astype(np.float32)
    b0 = O.f32_to_bf16_rne((rng.standard_normal(4096) * 1e-3).astype(np.float32))
    _, u_f32, _ = O.muon_prepare(g, b0, 0.95, True, spec)
    _, u_b16, _ = O.muon_prepare(O.f32_to_bf16_rne(g), b0, 0.95, True, spec)
    assert (u_f32 != u_b16).mean() > 0.9


def test_muon_apply_matches_reference(golden):
    z = golden("elementwise")
    out = O.muon_apply(z["apply/in_p"], z["apply/in_u"], 0.02, 0.01, float(z["apply/scale"]),
                       O.NoiseSpec(O.NOISE_TRITON, int(z["apply/seed"])))
    assert np.array_equal(out, z["apply/out_p"])


def test_rne_matches_torch():
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, 1e-40], np.float32)]).astype(np.float32)
    ours = O.f32_to_bf16_rne(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


# ---------------------------------------------------------------------------
# Newton-Schulz
# ---------------------------------------------------------------------------

def test_ns_bf16_matches_reference_golden(golden):
    z = golden("ns_traj")
    for i in range(4):
        shape = tuple(int(s) for s in z[f"ns/{i}/shape"])
        G = bf(z[f"ns/{i}/in"]).view(shape)
        ref = bf(z[f"ns/{i}/out"]).view(shape).float()
        got = O.ns_bf16_torch(G).float()
        rel = (torch.linalg.norm((got - ref).flatten()) / torch.linalg.norm(ref.flatten())).item()
        assert rel < 1e-2, (shape, rel)   # bit-identical here; tolerance covers other CPUs' bf16 GEMMs


def test_ns_fp32_closed_form():
    # G = U diag(s) V^T  =>  NS(G) = U diag(f^5(s / ||s||)) V^T  (quintic map on singular values)
    torch.manual_seed(0)
    for m, n in ((24, 40), (40, 24)):
        k = min(m, n)
        U, _ = torch.linalg.qr(torch.randn(m, k, dtype=torch.float64))
        V, _ = torch.linalg.qr(torch.randn(n, k, dtype=torch.float64))
        s = torch.linspace(0.05, 1.0, k, dtype=torch.float64)
        G = (U * s) @ V.T
        out = O.ns_fp32(G.float()).double()
        exp = (U * torch.from_numpy(O.ns_scalar_map(s.numpy()))) @ V.T
        assert (torch.linalg.norm(out - exp) / torch.linalg.norm(exp)).item() < 1e-5


# ---------------------------------------------------------------------------
# Muon step composition (seeds, stacking, NS, scale) against the reference's
# own two-step trajectories
# ---------------------------------------------------------------------------

def _ref_ns_bits(U):
    """The reference's bf16 Newton-Schulz (reproduced bit-exactly on CPU by
    O.ns_bf16_torch, see test_ns_bf16_matches_reference_golden) on bf16 bits."""
    X = O.ns_bf16_torch(bf(U).view(U.shape))
    return X.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("tag", ["muon_batch", "hybrid_nobatch"])
def test_muon_composition_matches_reference_trajectory(golden, tag):
    z = golden("ns_traj")
    assert str(z["prepare_rounding"]) == "trunc"
    nmuon = 3
    shapes = [tuple(int(s) for s in z[f"{tag}/shape{j}"]) for j in range(nmuon)]
    params = [z[f"{tag}/p{j}_0"].reshape(shapes[j]) for j in range(nmuon)]
    if tag == "muon_batch":
        bufs = {}
        for s in shapes:
            bufs.setdefault(s, 0)
            bufs[s] += 1
        bufs = {s: np.zeros((c, *s), np.uint16) for s, c in bufs.items()}
    else:
        bufs = [np.zeros(s, np.uint16) for s in shapes]
    for step in (1, 2):
        grads = [z[f"{tag}/g{j}_{step}"].reshape(shapes[j]) for j in range(nmuon)]
        if tag == "muon_batch":
            params, bufs = O.muon_batch_step(params, grads, bufs, step, 0.02, 0.01, 0.95, True, _ref_ns_bits,
                                             O.NOISE_TRITON, rounding="trunc")
            rows = {}
            got_bufs = []
            for s in shapes:
                got_bufs.append(bufs[s][rows.get(s, 0)])
                rows[s] = rows.get(s, 0) + 1
        else:
            out = [O.muon_param_step(params[j], grads[j], bufs[j], step, j, 0.02, 0.01, 0.95, True, _ref_ns_bits,
                                     O.NOISE_TRITON, rounding="trunc") for j in range(nmuon)]
            params = [o[0] for o in out]
            bufs = got_bufs = [o[1] for o in out]
        for j in range(nmuon):
            assert np.array_equal(got_bufs[j].ravel(), z[f"{tag}/buf{j}_{step}"].ravel()), (tag, step, j)
            assert np.array_equal(params[j].ravel(), z[f"{tag}/p{j}_{step}"].ravel()), (tag, step, j)


def test_muon_composition_detects_seed_slip(golden):
    """The trajectory pins the apply seeds: a composition that indexes the
    apply seed by the shape group instead of the matrix fails it."""
    z = golden("ns_traj")
    tag = "muon_batch"
    shapes = [tuple(int(s) for s in z[f"{tag}/shape{j}"]) for j in range(3)]
    params = [z[f"{tag}/p{j}_0"].reshape(shapes[j]) for j in range(3)]
    grads = [z[f"{tag}/g{j}_1"].reshape(shapes[j]) for j in range(3)]
    bufs = {(32, 48): np.zeros((2, 32, 48), np.uint16), (48, 32): np.zeros((1, 48, 32), np.uint16)}
    real = O.ref.deterministic_seed
    try:
        O.ref.deterministic_seed = lambda step, idx, salt=0: real(step, idx // 10000 if salt else idx, salt)
        slipped, _ = O.ref.muon_batch_step(params, grads, bufs, 1, 0.02, 0.01, 0.95, True, _ref_ns_bits,
                                           O.NOISE_TRITON, rounding="trunc")
    finally:
        O.ref.deterministic_seed = real
    assert not np.array_equal(slipped[2].ravel(), z[f"{tag}/p2_1"].ravel())

"""Weight path on the GPU: the model kernels against numpy, and a whole
model.wpk model (full geometry: 42 layers, vocabulary 130560, random weights
shared between even and odd layers) through mc_model_load / mc_prefill /
mc_decode_one / mc_batch_step against the forward oracle
(oracle/model_ref.py).

Tolerances: projections, norms and SwiGLU round to bf16 once, so the kernels
are held to one bf16 ulp of the fp64 result; the 42-layer forward compares
logits by relative L2 (< 2e-2) and cosine (> 0.999), and the greedy tokens
where the oracle's top-2 margin leaves no doubt. Batched steps must equal solo
decodes bit for bit (same kernels per row), and graph replay must equal eager.
"""
import ctypes as C
import os

import numpy as np
import pytest

import wpk_util as W
from _util import from_dev, to_dev

pytestmark = pytest.mark.gpu


def P(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def stream():
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg._native.lib()


@pytest.fixture(scope="module")
def rt(pkg, dev):
    import importlib
    return importlib.import_module("minicpm5-5080fast_amd.runtime")


def rnd_bf16(orc, rng, shape, scale=1.0):
    return orc.f32_to_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))


def within_ulp(orc, got_bits, ref, ulps=1.0, frac=0.999):
    got = orc.bf16_to_f32(got_bits).astype(np.float64)
    err = np.abs(got - ref)
    ok = err <= ulps * orc.bf16_ulp(ref) + 1e-30
    return ok.mean() >= frac and np.all(err <= 2 * ulps * orc.bf16_ulp(ref) + 1e-6), \
        (ok.mean(), err.max())


@pytest.mark.parametrize("M,N,K", [(1, 2048, 2048), (1, 2560, 2048), (3, 1000, 6144),
                                   (8, 2048, 2048), (5, 777, 6144), (1, 12288, 2048)])
def test_gemv(lib, orc, dev, M, N, K):
    import torch
    rng = np.random.default_rng(M * 1000 + N + K)
    w = rnd_bf16(orc, rng, (N, K), K ** -0.5)
    x = rnd_bf16(orc, rng, (M, K + 8))  # row stride K + 8
    y = torch.full((M, N + 3), -1, dtype=torch.int16, device=dev)
    dw, dx = to_dev(w, dev), to_dev(x, dev)
    assert lib.mc_model_gemv(P(dw), P(dx), K + 8, P(y), N + 3, M, N, K, stream()) == 0
    torch.cuda.synchronize()
    got = from_dev(y).reshape(M, N + 3)
    ref = orc.bf16_to_f32(x[:, :K]).astype(np.float64) @ orc.bf16_to_f32(w).astype(np.float64).T
    ok, st = within_ulp(orc, got[:, :N], ref)
    assert ok, st
    assert np.all(got[:, N:] == np.uint16(0xFFFF))  # past N untouched


@pytest.mark.parametrize("M,N,K,swi", [(9, 2560, 2048, 0), (16, 2048, 6144, 0),
                                      (17, 2560, 2048, 0), (32, 2048, 2048, 0),
                                      (25, 2048, 6144, 0), (32, 12288, 2048, 0),
                                      (12, 6144, 2048, 1), (20, 6144, 2048, 1),
                                      (32, 160, 2048, 1), (31, 96, 2048, 1)])
def test_gemm_rows(lib, orc, dev, M, N, K, swi):
    """Row GEMM of 9..32 rows (mc_model_gemm_rows) against a float64
    product: plain, within 1 bf16 ulp for 99.9% of outputs (2 for all); with
    the SwiGLU epilogue, the gate and up projections rounded to bf16 and then
    the SwiGLU, within 2 ulps for 98%. Row strides past the matrices and the
    output columns past N stay untouched."""
    import torch
    from oracle import model_ref as R
    rng = np.random.default_rng(M * 131 + N + K + swi)
    rows = 2 * N if swi else N
    w = rnd_bf16(orc, rng, (rows, K), K ** -0.5)
    x = rnd_bf16(orc, rng, (M, K + 16))  # row stride K + 16
    y = torch.full((M, N + 4), -1, dtype=torch.int16, device=dev)
    assert lib.mc_model_gemm_rows(P(to_dev(w, dev)), P(to_dev(x, dev)), K + 16, P(y), N + 4, M,
                                  N, K, swi, stream()) == 0
    torch.cuda.synchronize()
    got = from_dev(y).reshape(M, N + 4)
    prod = orc.bf16_to_f32(x[:, :K]).astype(np.float64) @ orc.bf16_to_f32(w).astype(np.float64).T
    if swi:
        gu = R.bf16(prod)
        ref = R.silu_mul(gu[:, :N], gu[:, N:]).astype(np.float64)
        ok, st = within_ulp(orc, got[:, :N], ref, ulps=2.0, frac=0.98)
    else:
        ok, st = within_ulp(orc, got[:, :N], prod)
    assert ok, st
    assert np.all(got[:, N:] == np.uint16(0xFFFF))


def test_gemm_rows_rejects_bad_shapes(lib, dev):
    """Row counts outside 9..32, N not a multiple of 16, K other than 2048 or
    6144 (2048 with the SwiGLU epilogue), swiglu other than 0/1 and short
    strides are MC_E_INVALID_ARGUMENT, with nothing launched."""
    import torch
    buf = torch.zeros(1 << 20, dtype=torch.int16, device=dev)
    p = P(buf)
    for M, N, K, ldx, ldy, swi in [(8, 2048, 2048, 2048, 2048, 0), (33, 2048, 2048, 2048, 2048, 0),
                                   (32, 2050, 2048, 2048, 2050, 0), (32, 2048, 4096, 4096, 2048, 0),
                                   (32, 2048, 2048, 2040, 2048, 0), (32, 2048, 2048, 2048, 2000, 0),
                                   (32, 2048, 6144, 6144, 2048, 1), (32, 2048, 2048, 2048, 2048, 2)]:
        assert lib.mc_model_gemm_rows(p, p, ldx, p, ldy, M, N, K, swi, stream()) == 1, (M, N, K)


@pytest.mark.parametrize("M,add,N", [(1, False, 2560), (1, True, 2560), (4, True, 12288),
                                     (8, True, 1000)])
def test_gemv_resnorm(lib, orc, dev, M, add, N):
    import torch
    from oracle import model_ref as R
    rng = np.random.default_rng(M + N)
    w = rnd_bf16(orc, rng, (N, 2048), 2048 ** -0.5)
    res = rnd_bf16(orc, rng, (M, 2048), 2.0)
    dlt = rnd_bf16(orc, rng, (M, 2048), 0.5)
    g = orc.f32_to_bf16(1 + 0.1 * rng.standard_normal(2048, dtype=np.float32))
    dres, ddl, dg, dw = (to_dev(a, dev) for a in (res, dlt, g, w))
    rout = torch.zeros(M * 2048, dtype=torch.int16, device=dev)
    y = torch.zeros(M * N, dtype=torch.int16, device=dev)
    assert lib.mc_model_gemv_resnorm(P(dw), P(dres), P(ddl) if add else None, P(dg),
                                     P(rout) if add else None, 2048, P(y), N, M, N,
                                     C.c_float(1e-6), stream()) == 0
    torch.cuda.synchronize()
    r = orc.bf16_to_f32(res) + (orc.bf16_to_f32(dlt) if add else 0)
    r = R.bf16(r)
    if add:
        assert np.array_equal(from_dev(rout).reshape(M, 2048), orc.f32_to_bf16(r))
    x = R.rmsnorm(r, orc.bf16_to_f32(g))
    ref = x.astype(np.float64) @ orc.bf16_to_f32(w).astype(np.float64).T
    ok, st = within_ulp(orc, from_dev(y).reshape(M, N), ref, ulps=2.0, frac=0.99)
    assert ok, st


@pytest.mark.parametrize("form", ["plain", "plain6144", "resnorm", "resnorm_swiglu"])
def test_gemv_rows_independent_of_row_count(lib, orc, dev, form):
    """Every row of an M-row GEMV (M = 1..8, the batch steps) equals the
    1-row GEMV of that row bit for bit: the lane sums of all rows (and of the
    gate and up rows) go through one reduce-scatter whose addition tree does
    not depend on M. This is what keeps batched decode steps equal to solo
    decodes."""
    import torch
    rng = np.random.default_rng(11)
    K = 6144 if form == "plain6144" else 2048
    N = 640  # 16-column multiple but not of the grid: ragged wave coverage
    rows = 2 * N if form == "resnorm_swiglu" else N
    w = to_dev(rnd_bf16(orc, rng, (rows, K), K ** -0.5), dev)
    x = to_dev(rnd_bf16(orc, rng, (8, K), 2.0), dev).view(-1)
    add = to_dev(rnd_bf16(orc, rng, (8, K), 0.5), dev).view(-1)
    g = to_dev(orc.f32_to_bf16(1 + 0.1 * rng.standard_normal(K, dtype=np.float32)), dev)

    def run(M, xr, ar):
        y = torch.zeros(M * N, dtype=torch.int16, device=dev)
        if form.startswith("plain"):
            st = lib.mc_model_gemv(P(w), P(xr), K, P(y), N, M, N, K, stream())
        elif form == "resnorm":
            st = lib.mc_model_gemv_resnorm(P(w), P(xr), P(ar), P(g), None, K, P(y), N, M, N,
                                           C.c_float(1e-6), stream())
        else:
            st = lib.mc_model_gemv_resnorm_swiglu(P(w), P(xr), P(ar), P(g), None, K, P(y), N, M,
                                                  N, C.c_float(1e-6), stream())
        assert st == 0
        torch.cuda.synchronize()
        return from_dev(y).reshape(M, N)

    solo = [run(1, x[m * K:], add[m * K:]) for m in range(8)]
    for M in range(2, 9):
        got = run(M, x, add)
        for m in range(M):
            assert np.array_equal(got[m], solo[m][0]), (form, M, m)


@pytest.mark.parametrize("M,K", [(1, 6144), (2, 6144), (3, 2048)])
def test_gemv_swiglu(lib, orc, dev, M, K):
    import torch
    from oracle import model_ref as R
    rng = np.random.default_rng(M + K)
    N = 2048
    w = rnd_bf16(orc, rng, (N, K), K ** -0.5)
    gu = rnd_bf16(orc, rng, (M, 2 * K), 2.0)
    y = torch.zeros(M * N, dtype=torch.int16, device=dev)
    assert lib.mc_model_gemv_swiglu(P(to_dev(w, dev)), P(to_dev(gu, dev)), 2 * K, P(y), N, M, N,
                                    K, stream()) == 0
    torch.cuda.synchronize()
    g = orc.bf16_to_f32(gu)
    x = R.silu_mul(g[:, :K], g[:, K:])
    ref = x.astype(np.float64) @ orc.bf16_to_f32(w).astype(np.float64).T
    ok, st = within_ulp(orc, from_dev(y).reshape(M, N), ref, ulps=2.0, frac=0.99)
    assert ok, st


@pytest.mark.parametrize("M,I", [(1, 6144), (3, 6144), (8, 500)])
def test_gemv_resnorm_swiglu(lib, orc, dev, M, I):
    """gate_up projection with the norm prologue and the SwiGLU epilogue ==
    the same projection rounded to bf16, then the SwiGLU."""
    import torch
    from oracle import model_ref as R
    rng = np.random.default_rng(M * 7 + I)
    w = rnd_bf16(orc, rng, (2 * I, 2048), 2048 ** -0.5)
    res = rnd_bf16(orc, rng, (M, 2048), 2.0)
    dlt = rnd_bf16(orc, rng, (M, 2048), 0.5)
    g = orc.f32_to_bf16(1 + 0.1 * rng.standard_normal(2048, dtype=np.float32))
    rout = torch.zeros(M * 2048, dtype=torch.int16, device=dev)
    y = torch.zeros(M * I, dtype=torch.int16, device=dev)
    assert lib.mc_model_gemv_resnorm_swiglu(P(to_dev(w, dev)), P(to_dev(res, dev)),
                                            P(to_dev(dlt, dev)), P(to_dev(g, dev)), P(rout), 2048,
                                            P(y), I, M, I, C.c_float(1e-6), stream()) == 0
    torch.cuda.synchronize()
    r = R.bf16(orc.bf16_to_f32(res) + orc.bf16_to_f32(dlt))
    assert np.array_equal(from_dev(rout).reshape(M, 2048), orc.f32_to_bf16(r))
    x = R.rmsnorm(r, orc.bf16_to_f32(g))
    gu = R.bf16(x.astype(np.float64) @ orc.bf16_to_f32(w).astype(np.float64).T)
    ref = R.silu_mul(gu[:, :I], gu[:, I:]).astype(np.float64)
    ok, st = within_ulp(orc, from_dev(y).reshape(M, I), ref, ulps=2.0, frac=0.98)
    assert ok, st


def test_residual_rounding_specials(lib, orc, dev):
    """The residual add rounds bf16 + bf16 in fp32 to bf16 with the oracle's
    rule, bit for bit, on the cases a rounding shortcut would get wrong: exact
    ties (both directions), carries into the exponent, overflow to infinity,
    subnormals, signed zeros and infinities; a NaN operand gives a NaN of its
    sign (the payload an fp32 add propagates is the platform's choice). Rows
    go through the RMSNorm kernel and the fused GEMV prologue for one and for
    several activation rows."""
    import torch
    f = np.float32
    one_ulp = f(2.0 ** -7)
    pairs = [(1.0, 2.0 ** -8), (1.0 + 2.0 ** -7, 2.0 ** -8), (-1.0, -(2.0 ** -8)),
             (1.9921875, 2.0 ** -8), (3.3e38, 3.3e38), (-3.3e38, -3.3e38),
             (1e-39, 1e-39), (-1e-40, 1e-40), (0.0, -0.0), (-0.0, -0.0),
             (np.inf, 1.0), (-np.inf, 1.0), (1.0, one_ulp)]
    res_f = np.array([p[0] for p in pairs], dtype=f)
    add_f = np.array([p[1] for p in pairs], dtype=f)
    res_b, add_b = orc.f32_to_bf16(res_f), orc.f32_to_bf16(add_f)
    nan_bits = np.array([0x7FA5, 0xFF81, 0x7FC3], dtype=np.uint16)  # signalling, negative, quiet
    res_b = np.concatenate([res_b, nan_bits, np.full(3, 0x3F80, np.uint16)])
    add_b = np.concatenate([add_b, np.full(3, 0x3F80, np.uint16), nan_bits])
    n = len(res_b)
    rng = np.random.default_rng(5)
    row_r = rnd_bf16(orc, rng, (2048,), 2.0)
    row_a = rnd_bf16(orc, rng, (2048,), 0.5)
    row_r[:n], row_a[:n] = res_b, add_b
    with np.errstate(over="ignore", invalid="ignore"):
        want = orc.f32_to_bf16(orc.bf16_to_f32(row_r) + orc.bf16_to_f32(row_a))
    g = orc.f32_to_bf16(np.ones(2048, dtype=f))
    for M in (1, 3, 8):
        res = np.tile(row_r, (M, 1))
        dlt = np.tile(row_a, (M, 1))
        # the norm kernel (in place)
        dres, out = to_dev(res, dev), torch.zeros(M * 2048, dtype=torch.int16, device=dev)
        assert lib.mc_model_rmsnorm_rows(P(dres), P(to_dev(dlt, dev)), P(to_dev(g, dev)), P(out),
                                         M, 2048, C.c_float(1e-6), stream()) == 0
        # the GEMV prologue
        rout = torch.zeros(M * 2048, dtype=torch.int16, device=dev)
        w = torch.zeros(64 * 2048, dtype=torch.int16, device=dev)
        y = torch.zeros(M * 64, dtype=torch.int16, device=dev)
        assert lib.mc_model_gemv_resnorm(P(w), P(to_dev(res, dev)), P(to_dev(dlt, dev)),
                                         P(to_dev(g, dev)), P(rout), 2048, P(y), 64, M, 64,
                                         C.c_float(1e-6), stream()) == 0
        torch.cuda.synchronize()
        nan = np.zeros(2048, dtype=bool)
        nan[n - 6:n] = True
        for got in (from_dev(dres), from_dev(rout)):
            got = got.reshape(M, 2048).view(np.uint16)
            for m in range(M):
                assert np.array_equal(got[m][~nan], want[~nan]), \
                    (M, m, [(hex(a), hex(b)) for a, b in zip(got[m][:n], want[:n])])
                gn, wn = got[m][nan], want[nan]
                assert np.all((gn & 0x7F80) == 0x7F80) and np.all(gn & 0x7F), [hex(v) for v in gn]
                assert np.array_equal(gn & 0x8000, wn & 0x8000), [hex(v) for v in gn]


def test_norm_swiglu_embedding_rows(lib, orc, dev):
    import torch
    from oracle import model_ref as R
    rng = np.random.default_rng(11)
    rows = 37
    res = rnd_bf16(orc, rng, (rows, 2048), 3.0)
    dlt = rnd_bf16(orc, rng, (rows, 2048))
    g = orc.f32_to_bf16(1 + 0.1 * rng.standard_normal(2048, dtype=np.float32))
    dres, out = to_dev(res, dev), torch.zeros(rows * 2048, dtype=torch.int16, device=dev)
    assert lib.mc_model_rmsnorm_rows(P(dres), P(to_dev(dlt, dev)), P(to_dev(g, dev)), P(out), rows,
                                     2048, C.c_float(1e-6), stream()) == 0
    torch.cuda.synchronize()
    r = R.bf16(orc.bf16_to_f32(res) + orc.bf16_to_f32(dlt))
    assert np.array_equal(from_dev(dres).reshape(rows, 2048), orc.f32_to_bf16(r))
    ref = R.rmsnorm(r, orc.bf16_to_f32(g)).astype(np.float64)
    got = orc.bf16_to_f32(from_dev(out)).reshape(rows, 2048)
    assert np.mean(got == ref) > 0.99 and np.all(np.abs(got - ref) <= orc.bf16_ulp(ref) + 1e-30)
    # SwiGLU rows
    src = rnd_bf16(orc, rng, (rows, 2 * 6144), 3.0)
    sw = torch.zeros(rows * 6144, dtype=torch.int16, device=dev)
    assert lib.mc_model_swiglu_rows(P(to_dev(src, dev)), P(sw), rows, 6144, stream()) == 0
    torch.cuda.synchronize()
    s = orc.bf16_to_f32(src)
    ref = R.silu_mul(s[:, :6144], s[:, 6144:])
    got = orc.bf16_to_f32(from_dev(sw)).reshape(rows, 6144)
    assert np.mean(got == ref) > 0.99 and np.all(np.abs(got - ref) <= orc.bf16_ulp(ref) + 1e-30)
    # embedding (direct ids and per-slot token pointers): exact rows
    table = rnd_bf16(orc, rng, (500, 2048))
    ids = np.array([5, 0, 499, 5, 17], dtype=np.int32)
    dt = to_dev(table, dev)
    e1 = torch.zeros(5 * 2048, dtype=torch.int16, device=dev)
    assert lib.mc_model_embedding_gather(P(dt), P(to_dev(ids, dev)), None, P(e1), 2048, 5,
                                         stream()) == 0
    toks = [torch.tensor([int(i)], dtype=torch.int32, device=dev) for i in ids]
    tab = torch.tensor([t.data_ptr() for t in toks], dtype=torch.int64, device=dev)
    e2 = torch.zeros(5 * 2048, dtype=torch.int16, device=dev)
    assert lib.mc_model_embedding_gather(P(dt), None, P(tab), P(e2), 2048, 5, stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(e1).reshape(5, 2048), table[ids])
    assert np.array_equal(from_dev(e2).reshape(5, 2048), table[ids])


def test_argmax(lib, orc, dev):
    import torch
    rng = np.random.default_rng(13)
    n = 130560
    lg = rnd_bf16(orc, rng, (3, n))
    lg[1, 70000] = lg[1, 1234] = orc.f32_to_bf16(np.float32([100.0]))[0]  # tie: lowest index
    lg[2, n - 1] = orc.f32_to_bf16(np.float32([50.0]))[0]
    dlg = to_dev(lg, dev)
    sv = torch.zeros(3 * 64, dtype=torch.float32, device=dev)
    si = torch.zeros(3 * 64, dtype=torch.int32, device=dev)
    for staged in (False, True):
        out = torch.full((3,), -1, dtype=torch.int32, device=dev)
        assert lib.mc_model_argmax_bf16(P(dlg), n, 3, P(out), None, P(sv) if staged else None,
                                        P(si) if staged else None, stream()) == 0
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert got[0] == int(np.argmax(orc.bf16_to_f32(lg[0])))
        assert got[1] == 1234 and got[2] == n - 1
    # ties across slices: the lowest index wins
    lg2 = np.zeros((1, n), dtype=np.uint16)
    lg2[0, [n - 5, 3000, 70000]] = orc.f32_to_bf16(np.float32([7.0]))[0]
    out = torch.full((1,), -1, dtype=torch.int32, device=dev)
    assert lib.mc_model_argmax_bf16(P(to_dev(lg2, dev)), n, 1, P(out), None, P(sv), P(si),
                                    stream()) == 0
    torch.cuda.synchronize()
    assert int(out.cpu()[0]) == 3000
    # NaN never wins a comparison; an all-NaN row reports index 0
    lg3 = rnd_bf16(orc, rng, (2, n))
    lg3[0, ::7] = 0x7FC0
    lg3[0, 99999] = orc.f32_to_bf16(np.float32([60.0]))[0]
    lg3[1, :] = 0xFFC1
    out = torch.full((2,), -1, dtype=torch.int32, device=dev)
    for staged in (False, True):
        assert lib.mc_model_argmax_bf16(P(to_dev(lg3, dev)), n, 2, P(out), None,
                                        P(sv) if staged else None, P(si) if staged else None,
                                        stream()) == 0
        torch.cuda.synchronize()
        assert out.cpu().tolist() == [99999, 0], staged


# ---------------- FP8 projections ----------------

def fp8_ref(orc, x, q, scale):
    """float64 reference of bf16(scale * sum e4m3(q) x)."""
    from oracle import model_ref as R
    return (np.asarray(x, np.float64) @ R.e4m3_to_f32(q).astype(np.float64).T) * scale


def rnd_codes(rng, shape, specials=True):
    """Random e4m3 codes; with specials, some 0x7F / 0xFF codes (+-480) and
    subnormals."""
    q = rng.integers(0, 256, size=shape, dtype=np.uint8)
    if not specials:
        q[(q & 0x7F) == 0x7F] ^= 0x01
    return q


def test_fp8_decode_every_code(lib, orc, dev):
    """Every e4m3 code through the kernel: W row n holds code n at column k0
    (zeros elsewhere), x is one-hot at k0 and the scale 1, so y[n] is the
    code's value, which bf16 holds exactly; the codes 0x7F / 0xFF are
    +-480 (kernels.h:120-148) and the other rows, without such codes, take
    the hardware conversion."""
    import torch
    from oracle import model_ref as R
    want = orc.f32_to_bf16(R.e4m3_to_f32(np.arange(256, dtype=np.uint8)))
    want[0x80] = 0  # -0 * 1 summed into an accumulator that starts at +0
    for K, k0 in ((2048, 0), (2048, 1037), (6144, 6143)):
        w = np.zeros((256, K), dtype=np.uint8)
        w[:, k0] = np.arange(256, dtype=np.uint8)
        x = np.zeros(K, dtype=np.uint16)
        x[k0] = 0x3F80  # 1.0
        y = torch.zeros(256, dtype=torch.int16, device=dev)
        assert lib.mc_model_gemv_fp8(P(to_dev(w, dev)), P(to_dev(np.ones(256, np.float32), dev)),
                                     P(to_dev(x, dev)), P(y), 256, K, stream()) == 0
        torch.cuda.synchronize()
        got = from_dev(y).view(np.uint16)
        assert np.array_equal(got, want), (K, k0, [(i, hex(a), hex(b)) for i, (a, b) in
                                                   enumerate(zip(got, want)) if a != b][:8])


@pytest.mark.parametrize("N,K,specials", [(2560, 2048, False), (2048, 6144, True),
                                          (1000, 2048, True), (130560, 2048, False)])
def test_gemv_fp8(lib, orc, dev, N, K, specials):
    import torch
    rng = np.random.default_rng(N + K)
    q = rnd_codes(rng, (N, K), specials)
    scale = (rng.random(N, dtype=np.float32) * 1e-3 + 1e-4).astype(np.float32)
    x = rnd_bf16(orc, rng, (K,), 1.0)
    y = torch.zeros(N, dtype=torch.int16, device=dev)
    assert lib.mc_model_gemv_fp8(P(to_dev(q, dev)), P(to_dev(scale, dev)), P(to_dev(x, dev)),
                                 P(y), N, K, stream()) == 0
    torch.cuda.synchronize()
    ref = fp8_ref(orc, orc.bf16_to_f32(x)[None], q, scale)[0]
    ok, st = within_ulp(orc, from_dev(y), ref, ulps=2.0, frac=0.99)
    assert ok, st


@pytest.mark.parametrize("add", [False, True])
def test_gemv_fp8_prologues(lib, orc, dev, add):
    """Norm prologue (residual written bit-exactly), norm prologue with the
    SwiGLU epilogue (== the projection rounded to bf16, then the SwiGLU), and
    the SwiGLU prologue, against float64 references."""
    import torch
    from oracle import model_ref as R
    rng = np.random.default_rng(77 + add)
    res = rnd_bf16(orc, rng, (2048,), 2.0)
    dlt = rnd_bf16(orc, rng, (2048,), 0.5)
    g = orc.f32_to_bf16(1 + 0.1 * rng.standard_normal(2048, dtype=np.float32))
    r = R.bf16(orc.bf16_to_f32(res) + (orc.bf16_to_f32(dlt) if add else 0))
    x = R.rmsnorm(r[None], orc.bf16_to_f32(g))
    d_res, d_dlt, d_g = to_dev(res, dev), to_dev(dlt, dev), to_dev(g, dev)
    # norm prologue
    N = 2560
    q = rnd_codes(rng, (N, 2048), True)
    sc = (rng.random(N, dtype=np.float32) * 1e-3 + 1e-4).astype(np.float32)
    rout = torch.zeros(2048, dtype=torch.int16, device=dev)
    y = torch.zeros(N, dtype=torch.int16, device=dev)
    assert lib.mc_model_gemv_fp8_resnorm(P(to_dev(q, dev)), P(to_dev(sc, dev)), P(d_res),
                                         P(d_dlt) if add else None, P(d_g),
                                         P(rout) if add else None, P(y), N, C.c_float(1e-6),
                                         stream()) == 0
    torch.cuda.synchronize()
    if add:
        assert np.array_equal(from_dev(rout), orc.f32_to_bf16(r))
    ok, st = within_ulp(orc, from_dev(y), fp8_ref(orc, x, q, sc)[0], ulps=2.0, frac=0.99)
    assert ok, st
    # norm prologue + SwiGLU epilogue
    I = 1536
    q2 = rnd_codes(rng, (2 * I, 2048), False)
    sc2 = (rng.random(2 * I, dtype=np.float32) * 1e-3 + 1e-4).astype(np.float32)
    y2 = torch.zeros(I, dtype=torch.int16, device=dev)
    assert lib.mc_model_gemv_fp8_resnorm_swiglu(P(to_dev(q2, dev)), P(to_dev(sc2, dev)),
                                                P(d_res), P(d_dlt) if add else None, P(d_g),
                                                None, P(y2), I, C.c_float(1e-6), stream()) == 0
    torch.cuda.synchronize()
    gu = R.bf16(fp8_ref(orc, x, q2, sc2)[0])
    ref = R.silu_mul(gu[:I], gu[I:]).astype(np.float64)
    ok, st = within_ulp(orc, from_dev(y2), ref, ulps=2.0, frac=0.98)
    assert ok, st
    # SwiGLU prologue (the down projection's input), K = 6144
    gate_up = rnd_bf16(orc, rng, (2 * 6144,), 2.0)
    q3 = rnd_codes(rng, (2048, 6144), True)
    sc3 = (rng.random(2048, dtype=np.float32) * 1e-3 + 1e-4).astype(np.float32)
    y3 = torch.zeros(2048, dtype=torch.int16, device=dev)
    assert lib.mc_model_gemv_fp8_swiglu(P(to_dev(q3, dev)), P(to_dev(sc3, dev)),
                                        P(to_dev(gate_up, dev)), P(y3), 2048, 6144,
                                        stream()) == 0
    torch.cuda.synchronize()
    gg = orc.bf16_to_f32(gate_up)
    xs = R.silu_mul(gg[:6144], gg[6144:])
    ok, st = within_ulp(orc, from_dev(y3), fp8_ref(orc, xs[None], q3, sc3)[0], ulps=2.0,
                        frac=0.99)
    assert ok, st


# ---------------- whole model through the mc_* ABI ----------------

@pytest.fixture(scope="module")
def model_dir(tmp_path_factory, orc):
    """A full-geometry model.wpk with random weights (two layer sets)."""
    d = tmp_path_factory.mktemp("wpk")
    secs = W.model_sections(2)
    blobs = W.random_blobs(1234, 2, scale=1.0)
    W.write_wpk(os.path.join(d, "model.wpk"), secs, blobs)
    return str(d), W.weights_f32(secs, blobs)


def compare_logits(got, ref):
    d = got.astype(np.float64) - ref.astype(np.float64)
    rel = np.linalg.norm(d) / np.linalg.norm(ref)
    cos = float(got @ ref / (np.linalg.norm(got) * np.linalg.norm(ref)))
    return rel, cos


def clear_winner(logits):
    top = np.sort(logits)[-2:]
    return top[1] - top[0] > 0.05 * np.std(logits)


def test_model_prefill_decode_vs_oracle(rt, orc, model_dir):
    from oracle import model_ref as R
    path, w = model_dir
    m = rt.Model(path, rt.model_options(max_context_tokens=4096, max_sessions=2))
    s = rt.Session(m)
    ref = R.ModelRef(w, 42)
    prompt = [1, 500, 130559, 77, 9, 12345, 3, 3, 42]
    s.prefill(prompt)
    ref.forward(prompt)
    rel, cos = compare_logits(s.last_logits(), ref.last_logits)
    print("prefill logits rel", rel, "cos", cos)
    assert rel < 2e-2 and cos > 0.999
    cfg = rt.gen_config(max_new_tokens=16)
    for step in range(4):
        tok = s.decode_one(cfg)
        want = ref.next_token
        if clear_winner(ref.last_logits):
            assert tok == want, (step, tok, want)
        ref.next_token = tok  # both continue from the GPU's token
        ref.decode()
        rel, cos = compare_logits(s.last_logits(), ref.last_logits)
        print("decode", step, "token", tok, "rel", rel, "cos", cos)
        assert rel < 2e-2 and cos > 0.999
    info = s.info()
    assert info["seq_len"] == len(prompt) + 4
    seq = s.seq(len(prompt) + 4)
    assert seq[:len(prompt)] == prompt
    s.close()
    m.close()


_DUMP_CHILD = r"""
import importlib, json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
rt = importlib.import_module("minicpm5-5080fast_amd.runtime")
m = rt.Model(sys.argv[2], rt.model_options(max_context_tokens=4096, max_sessions=1,
                                           enable_cuda_graph=1))
s = rt.Session(m)
s.prefill(json.loads(sys.argv[4]))
lg = [s.last_logits()]
cfg = rt.gen_config(max_new_tokens=16)
toks = []
for _ in range(4):
    toks.append(s.decode_one(cfg))
    lg.append(s.last_logits())
np.save(sys.argv[3] + "/child_logits.npy", np.stack(lg))
print(json.dumps(toks))
s.close()
m.close()
"""


@pytest.mark.parametrize("prompt", [[1, 500, 130559, 77, 9, 12345, 3, 3, 42],
                                    [1, 500, 130559, 77, 9]])
def test_model_debug_dump_files(rt, orc, model_dir, tmp_path, prompt):
    """The reference's debug dump (debug_dump.h:1-12; MC_DEBUG_DUMP_DIR and
    MC_DEBUG_DUMP_STEPS, read once, so a child process runs the session):
    forwards 0..N-1 (the prefill, then each decode) write step{t}.logits /
    final_hidden / token, the prefill also layer{i}.hidden_in / attn_out /
    mlp_out (last row, bf16 widened to fp32). The files equal the session's
    own logits and tokens, and the layer rows and final rows match the
    oracle's within the logits tolerance. Decode steps that dump run
    eagerly under a graph-enabled model. A 9-token prompt runs the GEMM
    prefill, a 5-token one the row-GEMV prefill."""
    import json
    import subprocess
    import sys
    from oracle import model_ref as R
    path, w = model_dir
    d = tmp_path / "dump"
    d.mkdir()
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, MC_DEBUG_DUMP_DIR=str(d), MC_DEBUG_DUMP_STEPS="3")
    r = subprocess.run([sys.executable, "-c", _DUMP_CHILD, root, path, str(d),
                        json.dumps(prompt)], env=env, capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    toks = json.loads(r.stdout.strip().splitlines()[-1])
    lg = np.load(d / "child_logits.npy")
    rd = lambda name, dt=np.float32: np.fromfile(d / name, dtype=dt)
    for t in range(3):  # forward 0 = the prefill, 1 and 2 = the first decodes
        assert np.array_equal(rd(f"step{t}.logits.f32"), lg[t]), t
        assert int(rd(f"step{t}.token", np.int32)[0]) == toks[t], t
    assert not (d / "step3.logits.f32").exists() and not (d / "step3.token").exists()

    def close(got, want, what):
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert got.shape == want.shape and rel < 2e-2, (what, rel)

    ref = R.ModelRef(w, 42)
    ref.capture = {}
    ref.forward(prompt)
    for l in range(42):
        for k in ("hidden_in", "attn_out", "mlp_out"):
            close(rd(f"layer{l}.{k}.f32"), ref.capture[f"layer{l}.{k}"], (l, k))
    close(rd("step0.final_hidden.f32"), ref.capture["final_hidden"], "step0")
    ref.capture = {}
    ref.next_token = toks[0]  # continue from the GPU's token
    ref.decode()
    close(rd("step1.final_hidden.f32"), ref.capture["final_hidden"], "step1")


_GEMM_CHILD = r"""
import importlib, json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
rt = importlib.import_module("minicpm5-5080fast_amd.runtime")
m = rt.Model(sys.argv[2], rt.model_options(max_context_tokens=8448, max_sessions=1))
s = rt.Session(m)
out = []
for n in json.loads(sys.argv[4]):
    for _ in range(2):  # twice: the second run must repeat the first bitwise
        s.reset()
        s.prefill([(i * 7919) % 130560 for i in range(n)])
        out.append(s.last_logits())
np.save(sys.argv[3], np.stack(out))
s.close()
m.close()
"""


def test_model_tuned_gemm_solutions_match_default(rt, model_dir, tmp_path):
    """The prefill projections' tuned rocBLAS solutions (prefill_gemm_table.h)
    against rocBLAS's default heuristic (MC_PREFILL_GEMM_DEFAULT=1, read once,
    so in a child process): the last-row logits of prefills whose row counts
    select tuned rows (300 rows: the 256-row gate_up row; 6200 rows: the
    6144-row gate_up row; 8448 rows, one full chunk: gate_up and down) agree
    to the logits tolerance (only the GEMMs' summation order differs), and
    each prefill repeated on the same session gives bitwise the same logits."""
    import json
    import subprocess
    import sys
    path, _ = model_dir
    sizes = [300, 6200, 8448]
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = {}
    for tag, extra in (("tuned", {}), ("default", {"MC_PREFILL_GEMM_DEFAULT": "1"})):
        env = {k: v for k, v in os.environ.items() if k != "MC_PREFILL_GEMM_DEFAULT"}
        env.update(extra)
        f = str(tmp_path / f"{tag}.npy")
        r = subprocess.run([sys.executable, "-c", _GEMM_CHILD, root, path, f, json.dumps(sizes)],
                           env=env, capture_output=True, text=True, timeout=600)
        assert r.returncode == 0, r.stderr[-3000:]
        out[tag] = np.load(f)
    for tag in out:  # deterministic GEMM solutions: a repeated prefill is bitwise equal
        for i, n in enumerate(sizes):
            assert np.array_equal(out[tag][2 * i], out[tag][2 * i + 1]), (tag, n)
    for i, n in enumerate(sizes):
        rel, cos = compare_logits(out["tuned"][2 * i], out["default"][2 * i])
        print("rows", n, "rel", rel, "cos", cos)
        assert rel < 2e-2 and cos > 0.999, n


_ROWS_CHILD = r"""
import importlib, json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
rt = importlib.import_module("minicpm5-5080fast_amd.runtime")
m = rt.Model(sys.argv[2], rt.model_options(max_context_tokens=4096, max_sessions=1))
s = rt.Session(m)
out = []
for p in json.loads(sys.argv[4]):
    s.reset()
    s.prefill(p)
    out.append(s.last_logits())
np.save(sys.argv[3], np.stack(out))
s.close()
m.close()
"""


def test_model_short_prefill_rows_path(rt, orc, model_dir, tmp_path):
    """Prefill chunks of 2..8 tokens run their projections as M-row GEMVs
    (forward_prefill_rows), chunks of 9..32 tokens through the row GEMM
    (mc_model_gemm_rows), and a 48-token chunk through hipBLASLt (the library
    path of 33..1023 rows). Their last-row logits match the oracle's forward,
    the greedy continuation matches the oracle's decode, and they agree with
    the library GEMM path (MC_PREFILL_ROWS_GEMV_OFF=1, read once, so in a
    child process) to the logits tolerance. The child imports no torch and so
    runs /opt/rocm's rocBLAS / hipBLASLt, where this process runs PyTorch's;
    the 48-token chunk differs between the two only in rounding. A prompt
    prefilled as a 20-token
    call (row GEMM) and a 5-token call (row GEMVs) gives the same logits on
    two sessions and matches the oracle."""
    import json
    import subprocess
    import sys
    from oracle import model_ref as R
    path, w = model_dir
    prompts = [[7, 130000], [1, 500, 130559, 77, 9], [11 * i + 3 for i in range(8)],
               [(13 * i + 5) % 130560 for i in range(13)], [17 * i for i in range(16)],
               [(29 * i + 1) % 130560 for i in range(25)], [(7 * i) % 997 for i in range(32)],
               [(41 * i + 9) % 130560 for i in range(48)]]
    m = rt.Model(path, rt.model_options(max_context_tokens=4096, max_sessions=2))
    s = rt.Session(m)
    got = []
    cfg = rt.gen_config(max_new_tokens=8)
    for p in prompts:
        s.reset()
        s.prefill(p)
        got.append(s.last_logits())
        ref = R.ModelRef(w, 42)
        ref.forward(p)
        rel, cos = compare_logits(got[-1], ref.last_logits)
        print(len(p), "rows: oracle rel", rel, "cos", cos)
        assert rel < 2e-2 and cos > 0.999, (len(p), rel, cos)
        for step in range(2):
            tok = s.decode_one(cfg)
            if clear_winner(ref.last_logits):
                assert tok == ref.next_token, (len(p), step, tok, ref.next_token)
            ref.next_token = tok
            ref.decode()
            rel, cos = compare_logits(s.last_logits(), ref.last_logits)
            assert rel < 2e-2 and cos > 0.999, (len(p), step, rel, cos)
    s.close()
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    f = str(tmp_path / "gemm.npy")
    env = dict(os.environ, MC_PREFILL_ROWS_GEMV_OFF="1")
    r = subprocess.run([sys.executable, "-c", _ROWS_CHILD, root, path, f, json.dumps(prompts)],
                       env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    gemm = np.load(f)
    for i, p in enumerate(prompts):
        rel, cos = compare_logits(got[i], gemm[i])
        print(len(p), "rows: GEMM path rel", rel, "cos", cos)
        assert rel < 2e-2 and cos > 0.999, (len(p), rel, cos)
    # a 5-token call after a 20-token one continues the same session state
    a, b = rt.Session(m), rt.Session(m)
    long_p = [(i * 7919 + 1) % 130560 for i in range(25)]
    a.prefill(long_p[:20])
    a.prefill(long_p[20:])
    b.prefill(long_p[:20])
    b.prefill(long_p[20:])
    assert np.array_equal(a.last_logits(), b.last_logits())
    ref = R.ModelRef(w, 42)
    ref.forward(long_p[:20])
    ref.forward(long_p[20:])
    rel, cos = compare_logits(a.last_logits(), ref.last_logits)
    assert rel < 2e-2 and cos > 0.999, (rel, cos)
    a.close()
    b.close()
    m.close()


def test_model_seed_residual_hook(rt, model_dir, tmp_path):
    """mc_debug_seed_residual (debug_dump.cpp:159-199): without weights
    MC_E_UNSUPPORTED; with weights the row count is checked and a seeded
    session's next prefill is the same as an unseeded one's (its embedding
    gather starts the forward)."""
    empty = tmp_path / "nowpk"
    empty.mkdir()
    m0 = rt.Model(str(empty), rt.model_options(max_context_tokens=2048, max_sessions=1))
    s0 = rt.Session(m0)
    with pytest.raises(rt.McError) as e:
        s0.seed_residual(np.zeros((1, 2048), dtype=np.uint16))
    assert e.value.status == 7  # MC_E_UNSUPPORTED
    s0.close()
    m0.close()
    path, _ = model_dir
    m = rt.Model(path, rt.model_options(max_context_tokens=4096, max_sessions=2))
    a, b = rt.Session(m), rt.Session(m)
    with pytest.raises(rt.McError):
        a.seed_residual(np.zeros((0, 2048), dtype=np.uint16))
    rows = np.full((3, 2048), 0x3F80, dtype=np.uint16)
    a.seed_residual(rows)
    prompt = [7, 8, 9, 10]
    a.prefill(prompt)
    b.prefill(prompt)
    assert np.array_equal(a.last_logits(), b.last_logits())
    a.close()
    b.close()
    m.close()


def test_model_graph_equals_eager_and_batch_equals_solo(rt, model_dir):
    """Greedy tokens and logits: graph replay == eager, and a batch step of two
    sessions == their solo decodes (bitwise)."""
    path, _ = model_dir
    prompts = [[5, 6, 7, 8, 9, 10, 11], [200, 300, 400]]
    cfg = rt.gen_config(max_new_tokens=16)
    runs = {}
    for graphs in (0, 1):
        m = rt.Model(path, rt.model_options(max_context_tokens=4096, max_sessions=2,
                                            enable_cuda_graph=graphs))
        toks, lg = [], []
        for p in prompts:
            s = rt.Session(m)
            s.prefill(p)
            t = [s.decode_one(cfg) for _ in range(3)]
            toks.append(t)
            lg.append(s.last_logits())
            s.close()
        runs[graphs] = (toks, lg)
        # batch: both prompts in one group
        ss = [rt.Session(m) for _ in prompts]
        for s, p in zip(ss, prompts):
            s.prefill(p)
        g = rt.BatchGroup(m, 2, 4096)
        slots = [g.add(s) for s in ss]
        bt = [g.step(slots, [cfg, cfg]) for _ in range(3)]
        assert [list(x) for x in zip(*bt)] == toks, (bt, toks)
        for i, sl in enumerate(slots):
            assert np.array_equal(g.last_logits(sl), lg[i])
        g.close()
        for s in ss:
            s.close()
        m.close()
    assert runs[0][0] == runs[1][0]
    for a, b in zip(runs[0][1], runs[1][1]):
        assert np.array_equal(a, b)


def test_model_chunked_prefill_equals_split_calls(rt, model_dir):
    """A 9000-token prompt is prefilled in chunks of 8448 + 552 tokens
    (prefill_executor.cpp:27,104-146): the logits, the next token and the
    following decode equal those of two mc_prefill calls of the same
    lengths, bit for bit, and a one-token decode continues from position
    9000 in both."""
    path, _ = model_dir
    m = rt.Model(path, rt.model_options(max_context_tokens=16384, max_sessions=2))
    prompt = [(i * 7919 + 11) % 130560 for i in range(9000)]
    a, b = rt.Session(m), rt.Session(m)
    a.prefill(prompt)
    b.prefill(prompt[:8448])
    b.prefill(prompt[8448:])
    assert np.array_equal(a.last_logits(), b.last_logits())
    cfg = rt.gen_config(max_new_tokens=8)
    ta, tb = a.decode_one(cfg), b.decode_one(cfg)
    assert ta == tb
    assert np.array_equal(a.last_logits(), b.last_logits())
    assert a.info()["seq_len"] == b.info()["seq_len"] == 9001
    a.close()
    b.close()
    m.close()


def test_model_prefill_allocates_nothing_after_create(rt, model_dir):
    """The session's rocBLAS handle works in a workspace carved from the
    session arena at create (sized by rocBLAS's own query), so prefills of
    any length, decodes and resets leave the device's free memory unchanged
    (memory_arena.h:1-8: no allocation after steady state)."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]

    def free_bytes():
        f, t = C.c_size_t(), C.c_size_t()
        assert hip.hipMemGetInfo(C.byref(f), C.byref(t)) == 0
        return f.value

    path, _ = model_dir
    m = rt.Model(path, rt.model_options(max_context_tokens=16384, max_sessions=2))
    s = rt.Session(m)
    before = free_bytes()
    cfg = rt.gen_config(max_new_tokens=64)
    for n in (1, 7, 100, 333, 2048, 4097, 8448):
        s.reset()
        s.prefill([(i * 31 + n) % 130560 for i in range(n)])
        s.decode_one(cfg)
        assert free_bytes() == before, n
    s.reset()
    s.prefill([(i * 17) % 130560 for i in range(9000)])  # two chunks: 8448 + 552
    assert free_bytes() == before
    s.close()
    m.close()


@pytest.fixture(scope="module")
def model_dir8(tmp_path_factory):
    """model.wpk (bf16, as model_dir) plus model_fp8.wpk: e4m3 codes of
    normal samples and row scales for the two layer sets and the lm_head
    (the oracle runs the same codes, so they need not quantize the bf16
    weights; codes are cut from the fp32 bits — exponent rebiased, mantissa
    truncated to 3 bits — which is fast and gives weights shaped like real
    quantized ones)."""
    d = tmp_path_factory.mktemp("wpk8")
    secs = W.model_sections(2)
    blobs = W.random_blobs(1234, 2, scale=1.0)
    W.write_wpk(os.path.join(d, "model.wpk"), secs, blobs)
    rng = np.random.default_rng(88)
    q8 = {}
    for key, (n, k) in [(f"{nm}.{s}", shape) for s in range(2) for nm, shape in
                        (("qkv", (W.QKV, W.HIDDEN)), ("o", (W.HIDDEN, W.HIDDEN)),
                         ("gate_up", (2 * W.INTER, W.HIDDEN)), ("down", (W.HIDDEN, W.INTER)))] + \
            [("table", (W.VOCAB, W.HIDDEN))]:
        v = rng.standard_normal((n, k), dtype=np.float32) * np.float32(64.0)
        u = v.view(np.uint32)
        e = ((u >> 23) & 0xFF).astype(np.int32) - 120  # e4m3 exponent field
        mag = np.where(e < 1, 0, np.minimum((e << 3) | ((u >> 20) & 7), 0x7E))
        codes = (mag | ((u >> 24) & 0x80)).astype(np.uint8)
        # rows of rms ~ 1/sqrt(K), the bf16 weights' scale
        scale = np.full(n, 1.0 / (64.0 * np.sqrt(k)), dtype=np.float32)
        scale *= (1 + 0.2 * rng.random(n)).astype(np.float32)
        q8[key] = (codes, scale)
    secs8 = W.fp8_sections(2, lm_head=True)
    W.write_fp8_wpk(os.path.join(d, "model_fp8.wpk"), secs8, q8)
    return str(d), W.weights_f32(secs, blobs), W.fp8_weights(secs8, q8)


def test_model_fp8_decode_vs_oracle(rt, orc, model_dir8):
    """precision MC_FP8 (the dual copy): the prefill runs the bf16 weights, each
    decode the e4m3 projections and lm_head; logits and tokens against the
    oracle in FP8 mode; graph replay == eager; batch steps keep the bf16
    weights and equal a BF16 model's bit for bit."""
    from oracle import model_ref as R
    path, w, q8 = model_dir8
    prompt = [7, 70000, 3, 130000, 12, 99]
    cfg = rt.gen_config(max_new_tokens=16)
    ref = R.ModelRef(w, 42, fp8=q8)
    ref.forward(prompt)
    logits = {}
    for graphs in (0, 1):
        m = rt.Model(path, rt.model_options(max_context_tokens=4096, max_sessions=2,
                                            enable_cuda_graph=graphs, precision=2))
        s = rt.Session(m)
        s.prefill(prompt)
        if graphs == 0:
            rel, cos = compare_logits(s.last_logits(), ref.last_logits)
            assert rel < 2e-2 and cos > 0.999, (rel, cos)
        lg = []
        for step in range(3):
            tok = s.decode_one(cfg)
            if graphs == 0:
                if clear_winner(ref.last_logits):
                    assert tok == ref.next_token, (step, tok, ref.next_token)
                ref.next_token = tok
                ref.decode()
                rel, cos = compare_logits(s.last_logits(), ref.last_logits)
                print("fp8 decode", step, "rel", rel, "cos", cos)
                assert rel < 2e-2 and cos > 0.999, (step, rel, cos)
            lg.append(s.last_logits())
        logits[graphs] = lg
        s.close()
        m.close()
    for a, b in zip(logits[0], logits[1]):
        assert np.array_equal(a, b)
    # batch steps: bf16 weights in both precisions
    toks = {}
    for prec in (0, 2):
        m = rt.Model(path, rt.model_options(max_context_tokens=4096, max_sessions=2,
                                            precision=prec))
        ss = [rt.Session(m) for _ in range(2)]
        for s_, p_ in zip(ss, (prompt, prompt[:3])):
            s_.prefill(p_)
        g = rt.BatchGroup(m, 2, 4096)
        slots = [g.add(s_) for s_ in ss]
        toks[prec] = [g.step(slots, [cfg, cfg]) for _ in range(2)]
        g.close()
        for s_ in ss:
            s_.close()
        m.close()
    assert toks[0] == toks[2]


def test_model_one_token_chunk_is_a_decode_forward(rt, orc, model_dir8):
    """A prefill chunk of one token is a T = 1 forward, which the reference
    runs through its decode path (forward.cpp:117-130,252-282,444-456): in
    FP8 mode that means the e4m3 projections and lm_head. A one-token prompt
    matches the oracle in FP8 mode (and not the bf16 oracle as closely); a
    prompt whose last chunk is one token (8449 = 8448 + 1) gives the same
    logits and tokens as two prefill calls of 8448 and 1 tokens, and its last
    chunk used the FP8 weights (the logits differ from a bf16 model's)."""
    from oracle import model_ref as R
    path, w, q8 = model_dir8
    m = rt.Model(path, rt.model_options(max_context_tokens=16384, max_sessions=2,
                                        precision=2))
    s = rt.Session(m)
    ref = R.ModelRef(w, 42, fp8=q8)
    s.prefill([4242])
    ref.forward([4242])
    rel, cos = compare_logits(s.last_logits(), ref.last_logits)
    assert rel < 2e-2 and cos > 0.999, (rel, cos)
    ref_bf16 = R.ModelRef(w, 42)
    ref_bf16.forward([4242])
    rel16, _ = compare_logits(s.last_logits(), ref_bf16.last_logits)
    assert rel16 > 2 * rel, (rel16, rel)  # the FP8 weights were used
    s.close()
    prompt = [(i * 7919 + 5) % 130560 for i in range(8449)]
    a, b = rt.Session(m), rt.Session(m)
    a.prefill(prompt)
    b.prefill(prompt[:8448])
    b.prefill(prompt[8448:])
    cfg = rt.gen_config(max_new_tokens=8)
    fp8_logits = a.last_logits()
    assert np.array_equal(fp8_logits, b.last_logits())
    assert a.decode_one(cfg) == b.decode_one(cfg)
    assert np.array_equal(a.last_logits(), b.last_logits())
    for s_ in (a, b):
        s_.close()
    m.close()
    # precision bf16: the same prompt's last (one-token) chunk runs bf16 GEMVs,
    # so its logits differ from the FP8 run's (before the T = 1 routing both
    # ran the bf16 GEMMs and were equal)
    m = rt.Model(path, rt.model_options(max_context_tokens=16384, max_sessions=1))
    a = rt.Session(m)
    a.prefill(prompt)
    assert not np.array_equal(a.last_logits(), fp8_logits)
    a.close()
    m.close()


def test_model_fp8_lm_head_off(rt, model_dir8, monkeypatch):
    """MC_FP8_LMHEAD_OFF set at load (weight_loader.cpp:549-560): the decode
    lm_head stays bf16 while the layer projections run e4m3; logits against
    the oracle in that configuration."""
    from oracle import model_ref as R
    path, w, q8 = model_dir8
    monkeypatch.setenv("MC_FP8_LMHEAD_OFF", "1")
    m = rt.Model(path, rt.model_options(max_context_tokens=2048, max_sessions=1, precision=2))
    monkeypatch.delenv("MC_FP8_LMHEAD_OFF")
    ref = R.ModelRef(w, 42, fp8={k: v for k, v in q8.items() if k != "lm_head"})
    s = rt.Session(m)
    prompt = [11, 22, 33]
    s.prefill(prompt)
    ref.forward(prompt)
    tok = s.decode_one(rt.gen_config(max_new_tokens=4))
    ref.next_token = tok
    ref.decode()
    rel, cos = compare_logits(s.last_logits(), ref.last_logits)
    assert rel < 2e-2 and cos > 0.999, (rel, cos)
    s.close()
    m.close()


def test_model_fp8_needs_both_packages(rt, model_dir8, tmp_path):
    import shutil
    path, _, _ = model_dir8
    only_bf16 = tmp_path / "bf16"
    only_bf16.mkdir()
    os.symlink(os.path.join(path, "model.wpk"), only_bf16 / "model.wpk")
    with pytest.raises(rt.McError) as e:
        rt.Model(str(only_bf16), rt.model_options(precision=2))
    assert e.value.status == 4 and "model_fp8.wpk" in str(e.value)
    empty = tmp_path / "empty"
    empty.mkdir()
    with pytest.raises(rt.McError) as e:
        rt.Model(str(empty), rt.model_options(precision=2))
    assert e.value.status == 4 and "model_fp8.wpk" in str(e.value)  # abi_smoke.cpp:118-127
    # a bf16 load ignores model_fp8.wpk
    m = rt.Model(path, rt.model_options(precision=0))
    m.close()


def test_model_rejects_sampling_and_bad_package(rt, model_dir, tmp_path):
    path, _ = model_dir
    m = rt.Model(path, rt.model_options(max_context_tokens=1024, max_sessions=1))
    s = rt.Session(m)
    s.prefill([1, 2, 3])
    with pytest.raises(rt.McError) as e:
        s.decode_one(rt.gen_config(temperature=0.8, top_k=40))
    assert e.value.status == 7
    assert s.decode_one(rt.gen_config()) >= 0  # greedy still fine
    s.close()
    m.close()
    bad = tmp_path / "bad"
    bad.mkdir()
    (bad / "model.wpk").write_bytes(b"MKP0" + b"\x00" * 60)
    with pytest.raises(rt.McError) as e:
        rt.Model(str(bad), rt.model_options())
    assert e.value.status == 4

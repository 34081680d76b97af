"""Pins the oracle's restatement of the reference's assembly M = 1 backward
routines, scan1d_backward_m1_shared_bc_asm and _simple_asm
(cpu/scan1d_backward_m1_shared_bc.asm, _simple.asm; declared at
include/scan.h:103-104). No assembler is available, so the routines cannot
be run; the restatement is held by:
  * the reference's own unit test of those routines
    (tests/unit/test_scan1d_backward_asm.c): its inputs, drawn from glibc's
    rand() after srand(42) in the test's order, and its criterion (every
    output within 1e-4 of the C function scan1d_backward_m1_shared_bc, run
    here compiled from the reference's sources, or its bit-exact oracle
    restatement where those are absent);
  * the Taylor decay they use without A_diag: closed forms, a float64
    evaluation of the polynomial, agreement with exp near zero, and the
    routine with A_diag = NULL equal bit for bit to the routine given those
    polynomial values as A_diag;
  * the edge sizes the routines clear (L = 0: dA, dB, dC; D = 0: ddelta).
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from kmtest import rng_for

# tests/unit/test_scan1d_backward_asm.c:164-177, in its order.
REF_ASM_CASES = [("simple", 8, 4), ("simple", 32, 16), ("simple", 64, 32),
                 ("avx2", 8, 4), ("avx2", 32, 16), ("avx2", 16, 17), ("avx2", 64, 32)]
REF_EPS = 1e-4   # tests/unit/test_scan1d_backward_asm.c:18


def _glibc_rand_inputs():
    """The inputs of every case of the reference test, from glibc rand()
    after srand(42) (test_scan1d_backward_asm.c:162), each case drawing x,
    A, B, C, delta, dy in that order (:104-109) as lo + (hi - lo) *
    ((float)rand() / RAND_MAX) in fp32 (:48-51)."""
    libc = ctypes.CDLL("libc.so.6")
    libc.rand.restype = ctypes.c_int
    libc.srand(42)
    rmax = np.float32(2147483647)            # RAND_MAX, rounded to float as in the test

    def fill(n, lo, hi):
        r = np.array([libc.rand() for _ in range(n)], np.float64).astype(np.float32) / rmax
        return (np.float32(lo) + (np.float32(hi) - np.float32(lo)) * r).astype(np.float32)

    cases = []
    for kind, L, D in REF_ASM_CASES:
        x = fill(L * D, -1.0, 1.0).reshape(L, D)
        A = fill(D, -0.5, -0.01)
        B = fill(D, -0.3, 0.3)
        Cm = fill(D, -0.2, 0.2)
        dt = fill(L, 0.01, 0.1)
        dy = fill(L * D, -1.0, 1.0).reshape(L, D)
        cases.append((kind, x, A, B, Cm, dt, dy))
    return cases


def _forward_h(x, A, B, dt, h0=None):
    # forward_m1_shared of the reference test (:27-45): h_t = e h + (dt B) x.
    L, D = x.shape
    h = np.zeros((L, D), np.float32)
    s = np.zeros(D, np.float32) if h0 is None else h0.astype(np.float32)
    for t in range(L):
        e = np.exp(np.float32(dt[t]) * A).astype(np.float32)
        s = (e * s + (np.float32(dt[t]) * B) * x[t]).astype(np.float32)
        h[t] = s
    return h


@pytest.mark.parametrize("i", range(len(REF_ASM_CASES)))
def test_asm_restatement_meets_the_reference_unit_test(i):
    kind, x, A, B, Cm, dt, dy = _glibc_rand_inputs()[i]
    h = _forward_h(x, A, B, dt)
    A_diag = np.exp(dt[:, None] * A[None, :]).astype(np.float32)     # :116-119
    want = O.scan1d_backward_m1_shared_bc(x, A, B, Cm, dt, h, dy, A_diag=A_diag)
    if O.REF_AVAILABLE:
        ref = O.scan1d_backward_m1_shared_bc(x, A, B, Cm, dt, h, dy, A_diag=A_diag,
                                             lib=O._load_ref())
        for a, b in zip(want, ref):
            np.testing.assert_array_equal(a, b)
    got = O.scan1d_backward_m1_shared_bc_asm(x, A, B, Cm, dt, h, dy, A_diag=A_diag,
                                             simple=(kind == "simple"))
    for name, g, w in zip(("dx", "dA", "dB", "dC", "ddelta"), got, want):
        assert np.abs(g - w).max() <= REF_EPS, (kind, name)


def test_taylor_decay_closed_forms():
    for simple in (False, True):
        assert O.m1_asm_taylor(np.float32(0.0), simple) == 1.0
        # 1 - 1 + 1/2 - 1/6 = 1/3 and 1 - 2 + 2 - 8/6 = -1/3: a dropped or
        # mis-scaled term moves these by at least 1/6.
        assert abs(O.m1_asm_taylor(np.float32(-1.0), simple) - 1 / 3) < 2e-7
        assert abs(O.m1_asm_taylor(np.float32(-2.0), simple) + 1 / 3) < 5e-7
        assert abs(O.m1_asm_taylor(np.float32(1.0), simple) - 8 / 3) < 1e-6


def test_taylor_decay_against_float64_polynomial_and_exp():
    g = rng_for("m1asm-taylor")
    xs = np.concatenate([g.uniform(-4, 0.5, 2000), -g.uniform(0, 1e-3, 200)]).astype(np.float32)
    x64 = xs.astype(np.float64)
    poly = 1 + x64 + x64 ** 2 / 2 + x64 ** 3 / 6
    scale = 1 + np.abs(x64) + x64 ** 2 / 2 + np.abs(x64) ** 3 / 6
    for simple in (False, True):
        v = O.m1_asm_taylor(xs, simple).astype(np.float64)
        assert (np.abs(v - poly) <= 4 * np.finfo(np.float32).eps * scale).all()
        small = np.abs(x64) <= 1e-3
        assert (np.abs(v[small] - np.exp(x64[small])) <= 2 * np.finfo(np.float32).eps).all()
    # It is not exp away from zero.
    assert abs(O.m1_asm_taylor(np.float32(-1.0)) - np.exp(-1.0)) > 0.03


@pytest.mark.parametrize("simple", [False, True])
@pytest.mark.parametrize("L,D,use_h0", [(9, 5, False), (16, 17, True), (40, 64, False)])
def test_null_adiag_is_the_taylor_decay(simple, L, D, use_h0):
    g = rng_for("m1asm-null", L, D, use_h0)
    x = g.uniform(-1, 1, (L, D)).astype(np.float32)
    A = g.uniform(-1.5, -0.05, D).astype(np.float32)
    B = g.uniform(-0.5, 0.5, D).astype(np.float32)
    Cm = g.uniform(-0.5, 0.5, D).astype(np.float32)
    dt = g.uniform(0.05, 0.8, L).astype(np.float32)
    dy = g.standard_normal((L, D)).astype(np.float32)
    h0 = g.uniform(-1, 1, D).astype(np.float32) if use_h0 else None
    h = _forward_h(x, A, B, dt, h0)
    got = O.scan1d_backward_m1_shared_bc_asm(x, A, B, Cm, dt, h, dy, h0=h0, simple=simple)
    diag = O.m1_asm_taylor(dt[:, None] * A[None, :], simple)
    want = O.scan1d_backward_m1_shared_bc_asm(x, A, B, Cm, dt, h, dy, A_diag=diag, h0=h0,
                                              simple=simple)
    for a, b in zip(got, want):
        np.testing.assert_array_equal(a, b)
    # Against the C function with exp decays the polynomial changes results
    # at these step sizes (|delta*A| up to 1.2).
    c = O.scan1d_backward_m1_shared_bc(x, A, B, Cm, dt, h, dy, h0=h0)
    assert np.abs(got[1] - c[1]).max() > 1e-3 * np.abs(c[1]).max()


def test_avx2_and_scalar_routines_share_all_but_the_ddelta_order():
    L, D = 20, 37
    g = rng_for("m1asm-forms", L, D)
    x = g.uniform(-1, 1, (L, D)).astype(np.float32)
    A = g.uniform(-1, -0.05, D).astype(np.float32)
    B = g.uniform(-0.5, 0.5, D).astype(np.float32)
    Cm = g.uniform(-0.5, 0.5, D).astype(np.float32)
    dt = g.uniform(0.05, 0.5, L).astype(np.float32)
    dy = g.standard_normal((L, D)).astype(np.float32)
    h = _forward_h(x, A, B, dt)
    diag = np.exp(dt[:, None] * A[None, :]).astype(np.float32)
    a = O.scan1d_backward_m1_shared_bc_asm(x, A, B, Cm, dt, h, dy, A_diag=diag)
    s = O.scan1d_backward_m1_shared_bc_asm(x, A, B, Cm, dt, h, dy, A_diag=diag, simple=True)
    for i in range(4):
        np.testing.assert_array_equal(a[i], s[i])
    np.testing.assert_allclose(a[4], s[4], rtol=1e-5, atol=1e-6)
    # The eight-lane order is a real difference for ddelta somewhere.
    assert not np.array_equal(a[4], s[4])


@pytest.mark.parametrize("simple", [False, True])
def test_edge_sizes_clear_the_other_outputs(simple):
    D = 6
    p = O.ScanBackwardSharedParams()
    dA, dB, dC = (np.full(D, 7.0, np.float32) for _ in range(3))
    p.dA, p.dB, p.dC = O.P(dA), O.P(dB), O.P(dC)
    p.L, p.D = 0, D
    O.orc.orc_scan1d_backward_m1_shared_bc_asm(ctypes.byref(p), int(simple))
    assert not dA.any() and not dB.any() and not dC.any()
    L = 5
    q = O.ScanBackwardSharedParams()
    dd = np.full(L, 7.0, np.float32)
    delta = np.ones(L, np.float32)
    q.delta, q.ddelta, q.L, q.D = O.P(delta), O.P(dd), L, 0
    dx = np.zeros(1, np.float32)
    q.dx = O.P(dx)
    for n in ("dA", "dB", "dC"):
        setattr(q, n, O.P(np.zeros(1, np.float32)))
    O.orc.orc_scan1d_backward_m1_shared_bc_asm(ctypes.byref(q), int(simple))
    assert not dd.any()

"""Pins the CPU oracle (oracle/kmoracle.c) before it is trusted as the
checker of the HIP kernels.

Each oracle function is checked against what fixes it independently:
  * the reference's own C compiled in place (oracle/_ref/libkmref.so), bit
    for bit where the arithmetic order is the same;
  * the C restatements held inside the reference's unit tests
    (tests/unit/test_scan1d.c:33-68, tests/unit/test_scan1d_backward.c:28-60);
  * the known answers of the reference tests (tests/unit/test_scan_nd.c,
    test_wavefront_nd.c, test_convnd_full.c);
  * closed forms, invariants and fp64 brute force on tiny inputs, chosen so a
    dropped term, a wrong sign/index or a transposed operand fails.
The committed fixtures in tests/golden/ carry the compiled-reference outputs
to machines where /root/reference is absent.
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from kmtest import rng_for, rel_err

ROOT = Path(__file__).resolve().parent.parent
needs_ref = pytest.mark.skipif(not O.REF_AVAILABLE, reason="oracle/_ref not built (reference tree absent)")


def uniform(g, shape, lo, hi):
    return (lo + (hi - lo) * g.random(shape)).astype(np.float32)


# ----------------------------------------------------------------------------
# Scan1D forward
# ----------------------------------------------------------------------------
REF_SCAN1D_SHAPES = [(4, 8, 1), (16, 16, 1), (64, 32, 1), (32, 24, 1), (4, 8, 2), (16, 16, 2),
                     (128, 48, 16), (37, 5, 3)]


def _ref_test_inputs(L, D, M, seed):
    # Distributions of tests/unit/test_scan1d.c:119-124.
    g = rng_for("ref-test-scan1d", L, D, M, seed)
    x = uniform(g, (L, D), -1, 1)
    A = uniform(g, (D, M), -1, -0.01)
    B = uniform(g, (L, D, M), -0.5, 0.5)
    Cm = uniform(g, (L, D, M), -0.5, 0.5)
    dt = uniform(g, (L, D), 0.01, 0.5)
    return x, A, B, Cm, dt


@needs_ref
@pytest.mark.parametrize("L,D,M", REF_SCAN1D_SHAPES)
def test_scan1d_bit_exact_vs_reference_test_restatements(L, D, M):
    x, A, B, Cm, dt = _ref_test_inputs(L, D, M, 0)
    y, h = O.scan1d(x, A, B, Cm, dt, np.zeros((D, M), np.float32))
    for hook in ("kmr_test_scan1d_ref", "kmr_test_scan1d_backward_forward_ref"):
        yr = np.zeros((L, D), np.float32)
        hr = np.zeros((L, D, M), np.float32)
        getattr(O.ref, hook)(O.P(x), O.P(A), O.P(B), O.P(Cm), O.P(dt), O.P(hr), O.P(yr), L, D, M)
        np.testing.assert_array_equal(y, yr, err_msg=hook)
        np.testing.assert_array_equal(h, hr[-1], err_msg=hook)


def test_scan1d_zero_input():
    # tests/unit/test_scan1d.c:177-200: x = 0, B = 0 -> y = 0, h = 0.
    L, D, M = 4, 8, 1
    y, h = O.scan1d(np.zeros((L, D)), np.full((D, M), -0.5), np.zeros((L, D, M)),
                    np.ones((L, D, M)), np.full((L, D), 0.1), np.zeros((D, M)))
    assert np.abs(y).sum() == 0 and np.abs(h).sum() == 0


def test_scan1d_closed_form_constant_inputs():
    # a = exp(dt*A), b = B*dt*x constant: h_t = a^(t+1) h0 + b (1 - a^(t+1)) / (1 - a).
    L, D, M = 50, 3, 2
    A = np.array([[-0.3, -1.1], [-0.05, -2.0], [-0.7, -0.01]], np.float32)
    dt, xv, bv, cv = 0.4, 0.8, 0.6, 1.5
    h0 = np.array([[0.2, -0.1], [1.0, 0.0], [-0.5, 0.3]], np.float32)
    y, h = O.scan1d(np.full((L, D), xv), A, np.full((L, D, M), bv), np.full((L, D, M), cv),
                    np.full((L, D), dt), h0)
    a = np.exp(np.float64(dt) * A.astype(np.float64))
    b = bv * dt * xv
    t = np.arange(1, L + 1, dtype=np.float64)[:, None, None]
    ht = a ** t * h0 + b * (1 - a ** t) / (1 - a)
    assert rel_err(h, ht[-1]) < 2e-5
    assert rel_err(y, cv * ht.sum(axis=2)) < 2e-5


def test_scan1d_fp64_bruteforce():
    g = rng_for("bf64", 0)
    L, D, M = 23, 4, 5
    x, A, B, Cm, dt = _ref_test_inputs(L, D, M, 3)
    h0 = uniform(g, (D, M), -1, 1)
    y, h = O.scan1d(x, A, B, Cm, dt, h0)
    hs = h0.astype(np.float64)
    ys = np.zeros((L, D))
    for t in range(L):
        hs = np.exp(dt[t][:, None].astype(np.float64) * A) * hs + \
            B[t].astype(np.float64) * dt[t][:, None] * x[t][:, None]
        ys[t] = (Cm[t] * hs).sum(axis=1)
    assert rel_err(y, ys) < 1e-5
    assert rel_err(h, hs) < 1e-5


def test_scan1d_clamp_saturates_like_minss_maxss():
    # Growing state (A = 0 so a = 1, b > 0): the reference clamps to +1000
    # after every step (cpu/scan1d.asm:136-140), so h saturates at exactly 1000
    # and y = C * 1000 from then on; a negative drive saturates at -1000.
    L, D, M = 40, 2, 1
    x = np.full((L, D), 1.0, np.float32)
    x[:, 1] = -1.0
    B = np.full((L, D, M), 100.0, np.float32)
    y, h = O.scan1d(x, np.zeros((D, M)), B, np.ones((L, D, M)), np.full((L, D), 1.0),
                    np.zeros((D, M)))
    assert h[0, 0] == 1000.0 and h[1, 0] == -1000.0
    assert y[9, 0] == 1000.0 and y[-1, 1] == -1000.0
    assert y[8, 0] == 900.0


def test_scan1d_batched_equals_per_batch_and_threads():
    Bsz, L, D, N = 3, 33, 10, 4
    g = rng_for("batched", 0)
    x = g.standard_normal((Bsz, L, D)).astype(np.float32)
    dt = uniform(g, (Bsz, L, D), 0.01, 0.5)
    A = uniform(g, (D, N), -1, -0.01)
    Bm = g.standard_normal((Bsz, L, N)).astype(np.float32)
    Cm = g.standard_normal((Bsz, L, N)).astype(np.float32)
    h0 = g.standard_normal((Bsz, D, N)).astype(np.float32)
    y, h, hh = O.scan1d_batched(x, dt, A, Bm, Cm, h0=h0, hist=True)
    y4, h4, hh4 = O.scan1d_batched(x, dt, A, Bm, Cm, h0=h0, hist=True, nthreads=4)
    np.testing.assert_array_equal(y, y4)
    np.testing.assert_array_equal(hh, hh4)
    for b in range(Bsz):
        Bb = np.broadcast_to(Bm[b][:, None, :], (L, D, N))
        Cb = np.broadcast_to(Cm[b][:, None, :], (L, D, N))
        yb, hb = O.scan1d(x[b], A, Bb, Cb, dt[b], h0[b])
        np.testing.assert_array_equal(y[b], yb)
        np.testing.assert_array_equal(h[b], hb)
        np.testing.assert_array_equal(hh[b, -1], hb)


# ----------------------------------------------------------------------------
# Scan1D backward
# ----------------------------------------------------------------------------
@needs_ref
@pytest.mark.parametrize("L,D,M,use_h0", [(4, 8, 1, False), (8, 16, 1, True), (4, 8, 2, False),
                                          (8, 16, 2, True), (16, 12, 16, True)])
def test_scan1d_backward_bit_exact_vs_reference(L, D, M, use_h0):
    x, A, B, Cm, dt = _ref_test_inputs(L, D, M, 1)
    g = rng_for("bwd", L, D, M)
    h0 = uniform(g, (D, M), -1, 1) if use_h0 else None
    dy = uniform(g, (L, D), -1, 1)
    _, _, hh = O.scan1d_batched(x[None], dt[None], A, B[None], Cm[None],
                                h0=None if h0 is None else h0[None],
                                bc_strides=(L * D * M, D * M, M), clamp=False, hist=True)
    h = hh[0]
    got = O.scan1d_backward(x, A, B, Cm, dt, h, dy, h0=h0)
    want = O.scan1d_backward(x, A, B, Cm, dt, h, dy, h0=h0, lib=O.ref)
    for gv, wv, name in zip(got, want, ("dx", "dA", "dB", "dC", "ddelta")):
        np.testing.assert_array_equal(gv, wv, err_msg=name)


@needs_ref
@pytest.mark.parametrize("L,D,with_diag", [(6, 5, False), (6, 16, True), (7, 19, True), (5, 4, True)])
def test_scan1d_backward_m1_shared_bit_exact_vs_reference(L, D, with_diag):
    g = rng_for("m1shared", L, D)
    x = uniform(g, (L, D), -1, 1)
    A = uniform(g, (D,), -1, -0.01)
    B = uniform(g, (D,), -0.5, 0.5)
    Cm = uniform(g, (D,), -0.5, 0.5)
    dt = uniform(g, (L,), 0.01, 0.5)
    h = uniform(g, (L, D), -1, 1)
    dy = uniform(g, (L, D), -1, 1)
    h0 = uniform(g, (D,), -1, 1)
    A_diag = np.exp(dt[:, None] * A[None, :]).astype(np.float32) if with_diag else None
    got = O.scan1d_backward_m1_shared_bc(x, A, B, Cm, dt, h, dy, A_diag=A_diag, h0=h0)
    want = O.scan1d_backward_m1_shared_bc(x, A, B, Cm, dt, h, dy, A_diag=A_diag, h0=h0, lib=O.ref)
    for gv, wv, name in zip(got, want, ("dx", "dA", "dB", "dC", "ddelta")):
        np.testing.assert_array_equal(gv, wv, err_msg=name)


def _loss(x, A, B, Cm, dt, dy):
    y, _, _ = O.scan1d_batched(x[None], dt[None], A, B[None], Cm[None],
                               bc_strides=(B.size, B.shape[1] * B.shape[2], B.shape[2]), clamp=False)
    return float((y[0].astype(np.float64) * dy).sum())


def test_scan1d_backward_finite_differences():
    # Central differences in the spirit of tests/unit/test_scan1d_backward.c:98-121,
    # with a random upstream gradient so every output contributes.
    L, D, M = 6, 3, 2
    x, A, B, Cm, dt = _ref_test_inputs(L, D, M, 7)
    dy = uniform(rng_for("fd"), (L, D), -1, 1)
    _, _, hh = O.scan1d_batched(x[None], dt[None], A, B[None], Cm[None],
                                bc_strides=(L * D * M, D * M, M), clamp=False, hist=True)
    grads = O.scan1d_backward(x, A, B, Cm, dt, hh[0], dy)
    eps = 1e-2
    for arr, grad in ((x, grads[0]), (A, grads[1]), (B, grads[2]), (Cm, grads[3]), (dt, grads[4])):
        flat = arr.reshape(-1)
        for i in range(0, flat.size, max(1, flat.size // 7)):
            orig = flat[i]
            flat[i] = orig + eps
            lp = _loss(x, A, B, Cm, dt, dy)
            flat[i] = orig - eps
            lm = _loss(x, A, B, Cm, dt, dy)
            flat[i] = orig
            num = (lp - lm) / (2 * eps)
            assert abs(num - grad.reshape(-1)[i]) < 2e-3 * max(1.0, abs(num)), (arr.shape, i)


@needs_ref
def test_reference_backward_unit_test_passes():
    exe = ROOT / "oracle" / "_ref" / "test_scan1d_backward"
    if not exe.exists():
        pytest.skip("reference test binary not built")
    out = subprocess.run([str(exe)], capture_output=True, text=True, env={"OMP_NUM_THREADS": "1"})
    assert out.returncode == 0, out.stdout[-2000:]


def test_batched_backward_equals_per_batch_generic():
    Bsz, L, D, N = 2, 9, 5, 3
    g = rng_for("bb", 0)
    x = g.standard_normal((Bsz, L, D)).astype(np.float32)
    dt = uniform(g, (Bsz, L, D), 0.01, 0.5)
    A = uniform(g, (D, N), -1, -0.01)
    Bm = g.standard_normal((Bsz, L, N)).astype(np.float32)
    Cm = g.standard_normal((Bsz, L, N)).astype(np.float32)
    h0 = g.standard_normal((Bsz, D, N)).astype(np.float32)
    dy = g.standard_normal((Bsz, L, D)).astype(np.float32)
    _, _, hh = O.scan1d_batched(x, dt, A, Bm, Cm, h0=h0, clamp=False, hist=True)
    dx, ddt, dA, dB, dC = O.scan1d_batched_backward(x, dt, A, Bm, Cm, dy, hh, h0=h0, nthreads=3)
    dA_sum = np.zeros((D, N))
    for b in range(Bsz):
        Bb = np.ascontiguousarray(np.broadcast_to(Bm[b][:, None, :], (L, D, N)))
        Cb = np.ascontiguousarray(np.broadcast_to(Cm[b][:, None, :], (L, D, N)))
        rx, rA, rB, rC, rdt = O.scan1d_backward(x[b], A, Bb, Cb, dt[b], hh[b], dy[b], h0=h0[b])
        np.testing.assert_array_equal(dx[b], rx)
        np.testing.assert_array_equal(ddt[b], rdt)
        assert rel_err(dB[b], rB.astype(np.float64).sum(axis=1)) < 1e-5
        assert rel_err(dC[b], rC.astype(np.float64).sum(axis=1)) < 1e-5
        dA_sum += rA
    assert rel_err(dA, dA_sum) < 1e-5


# ----------------------------------------------------------------------------
# Scan2D / ScanND
# ----------------------------------------------------------------------------
def test_scannd_known_answer_2d():
    # tests/unit/test_scan_nd.c:41-88: 2x2, A = (ln2, ln3), delta = 1 -> y = {1, 4, 3, 18}.
    dims = (2, 2)
    A = np.array([np.log(2.0), np.log(3.0)], np.float32).reshape(2, 1, 1)
    ones = np.ones((4, 1), np.float32)
    y, _ = O.scannd_ref(dims, ones, A, ones[:, :, None], ones[:, :, None], np.ones((2, 4, 1)))
    np.testing.assert_allclose(y[:, 0], [1, 4, 3, 18], atol=1e-5)
    y2, _ = O.scannd(dims, ones, A, ones[:, :, None], ones[:, :, None], np.ones((2, 4, 1)))
    np.testing.assert_allclose(y2[:, 0], [1, 4, 3, 18], atol=1e-5)


def test_scannd_known_answer_3d_lattice_paths():
    # tests/unit/test_scan_nd.c:90-141: 2x2x2, A = 0 -> {1,2,2,5,2,5,5,16}.
    dims = (2, 2, 2)
    ones = np.ones((8, 1), np.float32)
    y, _ = O.scannd_ref(dims, ones, np.zeros((3, 1, 1)), ones[:, :, None], ones[:, :, None],
                        np.ones((3, 8, 1)))
    np.testing.assert_allclose(y[:, 0], [1, 2, 2, 5, 2, 5, 5, 16], atol=1e-5)


def _nd_inputs(dims, D, M, seed):
    g = rng_for("nd", dims, D, M, seed)
    nd, Pn = len(dims), int(np.prod(dims))
    x = g.standard_normal((Pn, D)).astype(np.float32)
    A = uniform(g, (nd, D, M), -1.0, -0.05)
    B = (g.standard_normal((Pn, D, M)) * 0.25).astype(np.float32)
    Cm = (g.standard_normal((Pn, D, M)) * 0.25).astype(np.float32)
    dt = uniform(g, (nd, Pn, D), 0.05, 1.0)
    return x, A, B, Cm, dt


ND_CASES = [((9,), 3, 2), ((7, 5), 3, 4), ((3, 4, 5), 2, 3), ((2, 3, 2, 3), 2, 2), ((6, 6), 4, 16)]


@needs_ref
@pytest.mark.parametrize("dims,D,M", ND_CASES)
def test_scannd_ref_bit_exact_vs_reference(dims, D, M):
    args = _nd_inputs(dims, D, M, 0)
    y, h = O.scannd_ref(dims, *args, nthreads=4)
    yr, hr = O.scannd_ref(dims, *args, use_ref=True)      # reference run single-threaded
    np.testing.assert_array_equal(y, yr)
    np.testing.assert_array_equal(h, hr)


@pytest.mark.parametrize("dims,D,M", [((7, 5), 3, 4), ((6, 6), 4, 16), ((1, 9), 2, 2)])
def test_scan2d_agrees_with_scannd_ref(dims, D, M):
    # scan2d (asm order) and scannd_ref differ only in association of
    # dt_bar*B*x and the decay sum (cpu/scan2d.asm against src/scan_nd.c).
    x, A, B, Cm, dt = _nd_inputs(dims, D, M, 1)
    Pn = int(np.prod(dims))
    y2, h2 = O.scan2d(x, A[0], A[1], B, Cm, dt[0], dt[1], *dims)
    yr, hr = O.scannd_ref(dims, x, A, B, Cm, dt)
    # Both fields cancel (B and C take both signs); bound the difference by
    # the same recurrence run on absolute values, which has no cancellation:
    # |h2 - hr| <= eps * h_abs and |y2 - yr| <= eps * sum_m |C| h_abs.
    _, h_abs = O.scannd_ref(dims, np.abs(x), A, np.abs(B), np.abs(Cm), dt)
    y_abs = (np.abs(Cm).astype(np.float64) * h_abs).sum(axis=2)
    assert np.all(np.abs(h2.astype(np.float64) - hr) <= 1e-5 * h_abs + 1e-30)
    assert np.all(np.abs(y2.astype(np.float64) - yr) <= 1e-5 * y_abs + 1e-30)
    yd, hd = O.scannd(dims, x, A, B, Cm, dt)
    np.testing.assert_array_equal(yd, y2)
    assert Pn == h2.shape[0]


def test_scannd_fp64_bruteforce_and_zero_decay():
    dims, D, M = (3, 4, 2), 2, 3
    x, A, B, Cm, dt = _nd_inputs(dims, D, M, 2)
    y, h = O.scannd_ref(dims, x, A, B, Cm, dt)
    Pn = int(np.prod(dims))
    hs = np.zeros((Pn, D, M))
    strides = (8, 2, 1)
    for off in range(Pn):                   # row-major order respects causality
        idx = (off // 8, (off // 2) % 4, off % 2)
        dtb = dt[:, off, :].astype(np.float64).sum(axis=0) / 3
        v = dtb[:, None] * B[off] * x[off][:, None]
        for a in range(3):
            if idx[a] > 0:
                v = v + np.exp(dt[a, off][:, None].astype(np.float64) * A[a]) * hs[off - strides[a]]
        hs[off] = v
    assert rel_err(h, hs) < 1e-5
    assert rel_err(y, (Cm * hs).sum(axis=2)) < 1e-5
    # Decay 0 (A = -inf): pointwise dt_bar * B * x.
    y0, h0 = O.scannd_ref(dims, x, np.full_like(A, -np.inf), B, Cm, dt)
    dtb = dt.astype(np.float64).sum(axis=0) / 3
    assert rel_err(h0, dtb[:, :, None] * B * x[:, :, None]) < 1e-6


def test_scannd_1d_reduces_to_scan1d():
    L, D, M = 17, 3, 4
    x, A, B, Cm, dt = _nd_inputs((L,), D, M, 3)
    y, h = O.scannd_ref((L,), x, A, B, Cm, dt)
    y1, h1 = O.scan1d(x, A[0], B, Cm, dt[0], np.zeros((D, M)))
    # Association of dt*B*x differs; bound by the cancellation-free recurrence.
    _, h_abs = O.scannd_ref((L,), np.abs(x), A, np.abs(B), np.abs(Cm), dt)
    y_abs = (np.abs(Cm).astype(np.float64) * h_abs).sum(axis=2)
    assert np.all(np.abs(h[-1].astype(np.float64) - h1) <= 1e-6 * h_abs[-1])
    assert np.all(np.abs(y.astype(np.float64) - y1) <= 1e-6 * y_abs)


# ----------------------------------------------------------------------------
# ConvND
# ----------------------------------------------------------------------------
CONV_CASES = [((11,), 3, 4, True), ((6, 7), 5, 3, True), ((4, 5, 3), 2, 3, False),
              ((5, 4), 2, 1, True), ((3, 3, 2, 2), 2, 2, True)]


@needs_ref
@pytest.mark.parametrize("dims,D,K,bias", CONV_CASES)
def test_convnd_bit_exact_vs_reference(dims, D, K, bias):
    g = rng_for("conv", dims, D, K)
    Pn, KV = int(np.prod(dims)), K ** len(dims)
    inp = g.standard_normal((Pn, D)).astype(np.float32)
    ker = g.standard_normal((KV, D)).astype(np.float32)
    b = g.standard_normal(D).astype(np.float32) if bias else None
    out = O.convnd_forward(dims, inp, ker, b, nthreads=3)
    np.testing.assert_array_equal(out, O.convnd_forward(dims, inp, ker, b, use_ref=True))
    dy = g.standard_normal((Pn, D)).astype(np.float32)
    got = O.convnd_backward(dims, inp, ker, dy, with_bias=bias)
    want = O.convnd_backward(dims, inp, ker, dy, with_bias=bias, use_ref=True)
    for gv, wv in zip(got, want):
        if wv is None:
            assert gv is None
        else:
            np.testing.assert_array_equal(gv, wv)


def test_convnd_known_answer_2d():
    # tests/unit/test_convnd_full.c:14-20 (values hold for the causal convnd):
    # input {1,2,3,4}, kernel {1,2,3,4}, bias 0.5, K=2 -> {4.5, 11.5, 14.5, 30.5}.
    out = O.convnd_forward((2, 2), np.arange(1, 5, dtype=np.float32)[:, None],
                           np.arange(1, 5, dtype=np.float32)[:, None], np.array([0.5], np.float32))
    np.testing.assert_allclose(out[:, 0], [4.5, 11.5, 14.5, 30.5], atol=1e-6)


def test_convnd_known_answer_1d_constants():
    # tests/unit/test_conv1d_final.c:233-295: input 2, kernel 3, bias 1, K=2 -> {7, 13, 13}.
    out = O.convnd_forward((3,), np.full((3, 1), 2.0), np.full((2, 1), 3.0), np.array([1.0]))
    np.testing.assert_allclose(out[:, 0], [7, 13, 13], atol=1e-6)


def test_convnd_impulse_returns_flipped_kernel_and_separable_factorisation():
    K, D = 3, 2
    dims = (6, 5)
    g = rng_for("imp")
    k0 = g.standard_normal((K, D)).astype(np.float32)
    k1 = g.standard_normal((K, D)).astype(np.float32)
    full = (k0[:, None, :] * k1[None, :, :]).reshape(K * K, D)
    inp = np.zeros((30, D), np.float32)
    inp[0] = 1.0
    out = O.convnd_forward(dims, inp, full, None).reshape(6, 5, D)
    for i in range(K):
        for j in range(K):
            np.testing.assert_allclose(out[i, j], full[(K - 1 - i) * K + (K - 1 - j)], rtol=1e-6)
    assert np.all(out[K:, :] == 0) and np.all(out[:, K:] == 0)
    # Separable kernel == causal 1D pass along axis 1 then along axis 0.
    x = g.standard_normal((30, D)).astype(np.float32)
    full_out = O.convnd_forward(dims, x, full, None)
    t = np.zeros((6, 5, D))
    xx = x.reshape(6, 5, D).astype(np.float64)
    for j in range(5):
        for k in range(K):
            if j - (K - 1 - k) >= 0:
                t[:, j] += xx[:, j - (K - 1 - k)] * k1[k]
    s = np.zeros_like(t)
    for i in range(6):
        for k in range(K):
            if i - (K - 1 - k) >= 0:
                s[i] += t[i - (K - 1 - k)] * k0[k]
    assert rel_err(full_out, s.reshape(30, D)) < 1e-5


# ----------------------------------------------------------------------------
# Wavefront plan
# ----------------------------------------------------------------------------
def _plan_sizes(dims):
    starts, offs, mls = O.plan_tables(dims)
    return np.diff(starts), offs, mls


def test_wavefront_level_size_known_answers():
    # tests/unit/test_wavefront_nd.c:104-156.
    sizes, _, _ = _plan_sizes((3, 4))
    assert list(sizes) == [1, 2, 3, 3, 2, 1]
    sizes, _, _ = _plan_sizes((2, 3, 2))
    assert list(sizes) == [1, 3, 4, 3, 1]
    dd = O.longs((2, 3, 2))
    assert O.orc.orc_wavefront_row_major_offset(dd, O.longs((1, 2, 1)), 3) == 11


def test_plan_closed_form_2d_and_invariants():
    d1, d2 = 13, 7
    sizes, offs, mls = _plan_sizes((d1, d2))
    for k, s in enumerate(sizes):
        assert s == min(k, d1 - 1) - max(0, k - d2 + 1) + 1
    assert sorted(offs) == list(range(d1 * d2)) and mls == 7


@needs_ref
@pytest.mark.parametrize("dims", [(1,), (5,), (3, 4), (2, 3, 2), (4, 1, 3), (2, 2, 2, 3), (16, 16),
                                  (5, 3, 2, 2, 2)])
def test_plan_bit_exact_vs_reference(dims):
    mine = O.plan_tables(dims)
    theirs = O.plan_tables(dims, use_ref=True)
    np.testing.assert_array_equal(mine[0], theirs[0])
    np.testing.assert_array_equal(mine[1], theirs[1])
    assert mine[2] == theirs[2]


def mamba3_params(D, N, R, seed=0):
    g = rng_for("mamba3", D, N, R, seed)
    s = np.float32(1.0 / np.sqrt(D))
    return {"W_in": (g.standard_normal((R, D)) * s).astype(np.float32),
            "W_out": (g.standard_normal((D, R)) * 0.3).astype(np.float32),
            "A_log": -g.uniform(0.2, 2.0, N).astype(np.float32),
            "W_B": (g.standard_normal((N * R, D)) * s).astype(np.float32),
            "W_C": (g.standard_normal((N * R, D)) * s).astype(np.float32),
            "delta_proj": (g.standard_normal((1, D)) * s).astype(np.float32),
            "lambda_proj": (g.standard_normal((1, D)) * s).astype(np.float32),
            "b_B": (g.standard_normal(N * R) * 0.1).astype(np.float32),
            "b_C": (g.standard_normal(N * R) * 0.1).astype(np.float32),
            "theta": g.uniform(0, 2 * np.pi / N, max(N // 2, 1)).astype(np.float32)}


@needs_ref
@pytest.mark.parametrize("D,N,L,R,batch", [(24, 8, 37, 2, 3), (16, 16, 64, 1, 2), (10, 7, 20, 1, 1),
                                           (33, 4, 9, 3, 2), (8, 1, 5, 1, 1)])
def test_mamba3_forward_bit_exact_vs_reference(D, N, L, R, batch):
    # src/mamba_block.c:471-501 compiled in place; same parameters written
    # into a block made by the reference's mamba_block_create.
    p = mamba3_params(D, N, R)
    x = rng_for("m3x", D, N, L).standard_normal((batch, L, D)).astype(np.float32)
    got = O.mamba3_forward(p, x, dt_min=0.01, dt_max=0.5)
    want = O.mamba3_forward(p, x, dt_min=0.01, dt_max=0.5, use_ref=True)
    np.testing.assert_array_equal(got, want)


@needs_ref
@pytest.mark.parametrize("V,D,N,L,layers,R,tying", [(37, 12, 6, 9, 2, 1, 0), (50, 16, 8, 20, 3, 2, 1),
                                                    (10, 8, 4, 7, 1, 1, 0)])
def test_kmamba_forward_bit_exact_vs_reference(V, D, N, L, layers, R, tying):
    # src/kmamba.c:344-372 compiled in place, the reference initialising the
    # model (kmamba_init); the oracle composes the embedding rows, its
    # Mamba-3 blocks and its gemm_f32 on the same parameters. The reference
    # runs on one OpenMP thread: its gemm_f32 updates a row of C from
    # several threads at once (kernels/gemm_f32.c:22-29).
    import ctypes as C
    m = O.ref.kmamba_create(C.byref(O.kmamba_config(V, D, N, L, layers, R=R, weight_tying=tying)))
    assert m and O.ref.kmamba_init(m, 3) == 0
    toks = rng_for("kmtok", V, L).integers(0, V + 5, L).astype(np.uint32)   # a few past the vocabulary
    assert (toks >= V).any() or L < 10
    want = np.zeros((L, V), np.float32)
    gomp = C.CDLL("libgomp.so.1")
    prev = gomp.omp_get_max_threads()
    gomp.omp_set_num_threads(1)
    try:
        assert O.ref.kmamba_forward(m, toks.ctypes.data, want.ctypes.data) == 0
    finally:
        gomp.omp_set_num_threads(prev)
    emb, head, blocks = O.model_params(m)
    got = O.kmamba_forward(emb, head, blocks, toks)
    O.ref.kmamba_free(m)
    np.testing.assert_array_equal(got, want)
    assert np.abs(want).max() > 0


def test_gemm_f32_matches_float64():
    # The restated gemm_f32 against float64 products (k-ordered fp32 sums
    # carry at most K roundings of the partial sums).
    g = rng_for("gemmf32")
    A = g.standard_normal((13, 40)).astype(np.float32)
    B = g.standard_normal((40, 29)).astype(np.float32)
    got = O.gemm_f32(A, B)
    want = A.astype(np.float64) @ B.astype(np.float64)
    scale = np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)
    assert np.max(np.abs(got - want) / scale) < 40 * 2.0 ** -24
    # one nonzero term per element: exact
    np.testing.assert_array_equal(O.gemm_f32(np.eye(5, dtype=np.float32), B[:5]), B[:5])


def test_mamba3_forward_closed_forms():
    # With B = C = 0 (zero weights and biases) the state stays zero and the
    # block is the identity (the residual); with theta = 0, lambda = 1 and a
    # single constant input the state follows h_t = a h_{t-1} + dt*Bu.
    D, N, L = 6, 4, 12
    p = mamba3_params(D, N, 1)
    for k in ("W_B", "W_C", "b_B", "b_C"):
        p[k] = np.zeros_like(p[k])
    x = rng_for("m3cf").standard_normal((2, L, D)).astype(np.float32)
    np.testing.assert_array_equal(O.mamba3_forward(p, x), x)
    # constant drive, no rotation: compare with the float64 recurrence
    p = mamba3_params(D, N, 1, seed=1)
    p["theta"][:] = 0
    x1 = np.tile(rng_for("m3c").standard_normal(D).astype(np.float32), (1, L, 1))
    out = O.mamba3_forward(p, x1, dt_min=1e-4, dt_max=10.0).astype(np.float64)
    xt = x1[0, 0].astype(np.float64)
    z = p["W_in"].astype(np.float64) @ xt
    u = z / (1 + np.exp(-z))
    dt = np.log1p(np.exp(p["delta_proj"].astype(np.float64) @ xt))[0]
    lam = 1 / (1 + np.exp(-(p["lambda_proj"].astype(np.float64) @ xt)[0]))
    Bt = p["W_B"].astype(np.float64) @ xt + p["b_B"]
    Ct = p["W_C"].astype(np.float64) @ xt + p["b_C"]
    bu = Bt * u[0]
    alpha = np.exp(dt * p["A_log"].astype(np.float64))
    h = np.zeros(N)
    for t in range(L):
        h = alpha * h + (1 - lam) * dt * alpha * (bu if t > 0 else 0) + lam * dt * bu
        y = Ct @ h
        want = xt + p["W_out"][:, 0] * y
        np.testing.assert_allclose(out[0, t], want, rtol=2e-5, atol=2e-6)


# ---------------------------------------------------------------------------
# ScanND adjoint (no reference function: pinned by float64 finite
# differences and by its 1D case, which is the reference's scan1d_backward)
# ---------------------------------------------------------------------------
def _scannd_f64(dims, x, A, B, Cm, delta):
    """Brute-force float64 forward of scannd_ref (src/scan_nd.c:74-192,
    non-lambda branch) for tiny grids: y [P, D]."""
    nd = len(dims)
    Pn = int(np.prod(dims))
    strides = [int(np.prod(dims[a + 1:])) for a in range(nd)]
    h = np.zeros(B.shape)
    y = np.zeros(x.shape)
    for q in range(Pn):
        idx = [(q // strides[a]) % dims[a] for a in range(nd)]
        dtb = delta[:, q, :].sum(0) / nd                      # [D]
        hq = (dtb * x[q])[:, None] * B[q]
        for a in range(nd):
            if idx[a] > 0:
                hq = hq + np.exp(delta[a, q][:, None] * A[a]) * h[q - strides[a]]
        h[q] = hq
        y[q] = (Cm[q] * hq).sum(-1)
    return y


def _nd_case(dims, D, M, seed):
    g = rng_for("ndadj", dims, D, M, seed)
    Pn, nd = int(np.prod(dims)), len(dims)
    return dict(x=g.standard_normal((Pn, D)), A=-g.uniform(0.2, 1.5, (nd, D, M)),
                B=g.standard_normal((Pn, D, M)) * 0.5, Cm=g.standard_normal((Pn, D, M)) * 0.5,
                delta=g.uniform(0.05, 0.6, (nd, Pn, D)), dy=g.standard_normal((Pn, D)))


@pytest.mark.parametrize("dims,D,M", [((5,), 2, 3), ((3, 4), 2, 3), ((2, 3, 2), 1, 2), ((2, 2, 2, 2), 1, 1)])
def test_scannd_backward_vs_finite_differences(dims, D, M):
    # Central differences of L = sum dy . y on the float64 forward; the
    # oracle runs in fp32 on the same (fp32-representable) inputs.
    c = {k: v.astype(np.float32).astype(np.float64) for k, v in _nd_case(dims, D, M, 0).items()}
    y32, h32 = O.scannd_ref(dims, c["x"], c["A"], c["B"], c["Cm"], c["delta"])
    got = O.scannd_backward(dims, c["x"], c["A"], c["B"], c["Cm"], c["delta"], h32, c["dy"])
    names = {"x": "dx", "A": "dA", "B": "dB", "Cm": "dC", "delta": "ddelta"}

    def loss(**kw):
        args = {k: kw.get(k, c[k]) for k in ("x", "A", "B", "Cm", "delta")}
        return float((c["dy"] * _scannd_f64(dims, **args)).sum())
    for name, gname in names.items():
        base = c[name]
        fd = np.zeros_like(base)
        eps = 1e-6
        for i in np.ndindex(base.shape):
            up, dn = base.copy(), base.copy()
            up[i] += eps
            dn[i] -= eps
            fd[i] = (loss(**{name: up}) - loss(**{name: dn})) / (2 * eps)
        err = np.abs(got[gname] - fd).max() / max(np.abs(fd).max(), 1e-12)
        assert err < 2e-5, f"{gname}: max error {err:.2e} relative to max |grad|"


@needs_ref
@pytest.mark.parametrize("L,D,M", [(9, 3, 4), (40, 8, 16)])
def test_scannd_backward_1d_equals_reference_scan1d_backward(L, D, M):
    # With ndims = 1, dtbar = delta and the ScanND recurrence is Scan1D's
    # without the clamp, so the adjoint is cpu/scan1d_backward.c:248-295
    # (h0 = 0; B, C per channel [L, D, M], the layout both use).
    c = _nd_case((L,), D, M, 1)
    c = {k: v.astype(np.float32) for k, v in c.items()}
    y, h = O.scannd_ref((L,), c["x"], c["A"], c["B"], c["Cm"], c["delta"])
    got = O.scannd_backward((L,), c["x"], c["A"], c["B"], c["Cm"], c["delta"], h, c["dy"])
    dx, dA, dB, dC, dd = O.scan1d_backward(c["x"], c["A"][0], c["B"], c["Cm"], c["delta"][0], h,
                                           c["dy"], lib=O.ref)
    for name, want, have in (("dx", dx, got["dx"]), ("dA", dA, got["dA"][0]), ("dB", dB, got["dB"]),
                             ("dC", dC, got["dC"]), ("ddelta", dd, got["ddelta"][0])):
        scale = max(np.abs(want).max(), 1e-30)
        assert np.abs(have - want).max() / scale < 1e-5, name

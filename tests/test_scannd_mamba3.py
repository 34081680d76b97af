"""ScanND Mamba-3 (lambda) branch: src/scan_nd.c:59-210.

The reference's branch keeps its rotated states in a [D, M] buffer that it
indexes by point (src/scan_nd.c:63, :166, :200-205): out-of-bounds and, with
theta NULL, uninitialised reads, so the compiled reference cannot serve as an
oracle here. The restatement in oracle/kmoracle.c follows the evident intent
(rotated states kept per point). Its CPU pins below use only closed forms and
invariants that a plausible mistake breaks:
  * lambda = 1 reduces the branch to the lambda-free recurrence with A
    clamped to -1e-5 (bit-exact): catches a swapped lambda / (1 - lambda), a
    wrong dt_bar factor, a missing clamp;
  * theta = 0 equals theta = NULL (bit-exact): the rotation is applied to the
    pair as a rotation, not to one channel only;
  * an odd last channel is never rotated (bit-exact);
  * y(2x) = 2 y(x) (bit-exact): every term is proportional to x;
  * a sink point's readout is affine in its own lambda;
  * a two-point chain with theta = pi/2 against a hand-derived closed form in
    float64 (rotation direction, predecessor B*x, the clamp).
The GPU tests compare every entry point with the restatement.
"""
import ctypes as C
import math

import numpy as np
import pytest

import oracle as O
from kmtest import TOL_F32, assert_close, rng_for


def m3_inputs(dims, D, M, seed, lam_lo=0.0, lam_hi=1.0, a_hi=0.2):
    g = rng_for("nd-m3", dims, D, M, seed)
    nd, P = len(dims), int(np.prod(dims))
    x = g.standard_normal((P, D)).astype(np.float32)
    # Some A above the branch's -1e-5 clamp (decay ~1), some below.
    A = g.uniform(-1.0, a_hi, (nd, D, M)).astype(np.float32)
    B = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    Cm = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    dt = g.uniform(0.05, 1.0, (nd, P, D)).astype(np.float32)
    theta = g.uniform(-math.pi, math.pi, (max(D // 2, 1),)).astype(np.float32)
    lam = g.uniform(lam_lo, lam_hi, (P,)).astype(np.float32)
    return x, A, B, Cm, dt, theta, lam


PIN_SHAPES = [((5, 4), 4, 3), ((3, 4, 2), 5, 2), ((9,), 3, 4), ((2, 3, 2, 2), 2, 2)]


@pytest.mark.parametrize("dims,D,M", PIN_SHAPES)
def test_lambda_one_is_the_clamped_lambda_free_recurrence(dims, D, M):
    x, A, B, Cm, dt, _, _ = m3_inputs(dims, D, M, 1)
    lam = np.ones(int(np.prod(dims)), np.float32)
    y1, h1 = O.scannd_ref(dims, x, A, B, Cm, dt, lam=lam)
    Ac = np.minimum(A, np.float32(-1e-5)).astype(np.float32)
    y0, h0 = O.scannd_ref(dims, x, Ac, B, Cm, dt)
    np.testing.assert_array_equal(h1, h0)
    np.testing.assert_array_equal(y1, y0)


@pytest.mark.parametrize("dims,D,M", PIN_SHAPES)
def test_theta_zero_is_no_rotation_and_odd_channel_unrotated(dims, D, M):
    x, A, B, Cm, dt, theta, lam = m3_inputs(dims, D, M, 2)
    yn, hn = O.scannd_ref(dims, x, A, B, Cm, dt, lam=lam)
    yz, hz = O.scannd_ref(dims, x, A, B, Cm, dt, lam=lam, theta=np.zeros_like(theta))
    np.testing.assert_array_equal(hz, hn)
    np.testing.assert_array_equal(yz, yn)
    yt, ht = O.scannd_ref(dims, x, A, B, Cm, dt, lam=lam, theta=theta)
    if D % 2 == 1:
        np.testing.assert_array_equal(ht[:, D - 1], hn[:, D - 1])
        np.testing.assert_array_equal(yt[:, D - 1], yn[:, D - 1])
    if int(np.prod(dims)) > 1 and D >= 2:
        assert not np.array_equal(ht[:, :2], hn[:, :2])   # the rotation reaches successors


@pytest.mark.parametrize("dims,D,M", PIN_SHAPES)
def test_outputs_are_linear_in_x(dims, D, M):
    x, A, B, Cm, dt, theta, lam = m3_inputs(dims, D, M, 3)
    y1, h1 = O.scannd_ref(dims, x, A, B, Cm, dt, lam=lam, theta=theta)
    y2, h2 = O.scannd_ref(dims, 2 * x, A, B, Cm, dt, lam=lam, theta=theta)
    np.testing.assert_array_equal(h2, 2 * h1)
    np.testing.assert_array_equal(y2, 2 * y1)


def test_sink_readout_is_affine_in_its_lambda():
    dims, D, M = (4, 3), 4, 3
    x, A, B, Cm, dt, theta, lam = m3_inputs(dims, D, M, 4)
    ys = []
    for v in (0.0, 1.0, 0.25):
        lm = lam.copy()
        lm[-1] = v                                   # the last point has no successor
        y, h = O.scannd_ref(dims, x, A, B, Cm, dt, lam=lm, theta=theta)
        ys.append(y[-1].astype(np.float64))
    np.testing.assert_allclose(ys[2], 0.75 * ys[0] + 0.25 * ys[1], rtol=1e-5, atol=1e-6)


def test_two_point_chain_rotation_closed_form():
    # dims (2,), D = 2, M = 1, theta = pi/2: point 0 has no predecessor,
    # h0[c] = B0[c] x0[c] (lam0 dt0[c]); its rotated states are
    # (cos h0[0] - sin h0[1], sin h0[0] + cos h0[1]); point 1 adds
    # B0 x0 ((1 - lam1) dt1 alpha) + B1 x1 (lam1 dt1) + alpha hrot0, with
    # alpha = exp(dt1 min(A, -1e-5)).
    x = np.array([[0.7, -1.3], [0.4, 2.1]], np.float32)
    A = np.array([[[-0.6], [0.3]]], np.float32)          # channel 1 hits the clamp
    B = np.array([[[0.9], [-0.5]], [[1.2], [0.8]]], np.float32)
    Cm = np.array([[[1.0], [1.0]], [[0.5], [-2.0]]], np.float32)
    dt = np.array([[[0.3, 0.8], [0.6, 0.2]]], np.float32)
    theta = np.array([math.pi / 2], np.float32)
    lam = np.array([0.35, 0.6], np.float32)
    y, h = O.scannd_ref((2,), x, A, B, Cm, dt, lam=lam, theta=theta)
    f = np.float64
    h0 = [f(B[0, c, 0]) * f(x[0, c]) * (f(lam[0]) * f(dt[0, 0, c])) for c in range(2)]
    th = f(theta[0])
    rot = [math.cos(th) * h0[0] - math.sin(th) * h0[1], math.sin(th) * h0[0] + math.cos(th) * h0[1]]
    h1 = []
    for c in range(2):
        alpha = math.exp(f(dt[0, 1, c]) * min(f(A[0, c, 0]), -1e-5))
        bpa = f(B[0, c, 0]) * f(x[0, c])
        h1.append(bpa * ((1 - f(lam[1])) * f(dt[0, 1, c]) * alpha)
                  + f(B[1, c, 0]) * f(x[1, c]) * (f(lam[1]) * f(dt[0, 1, c])) + alpha * rot[c])
    np.testing.assert_allclose(h[0, :, 0], h0, rtol=1e-6)
    np.testing.assert_allclose(h[1, :, 0], h1, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(y[1], [0.5 * h1[0], -2.0 * h1[1]], rtol=1e-5, atol=1e-7)


def test_backward_rejects_the_lambda_branch():
    dims, D, M = (3, 3), 2, 2
    x, A, B, Cm, dt, theta, lam = m3_inputs(dims, D, M, 5)
    P = int(np.prod(dims))
    h = np.zeros((P, D, M), np.float32)
    y = np.zeros((P, D), np.float32)
    p, _keep = O._nd_params(dims, x, A, B, Cm, dt, h, y, theta, lam)
    outs = [np.zeros_like(a) for a in (x, dt, A, B, Cm)]
    rc = O.orc.orc_scannd_backward(C.byref(p), O.P(np.zeros_like(y)), *[O.P(o) for o in outs])
    assert rc == -1


# ---------------------------------------------------------------------------
# GPU parity (every entry point) against the restatement.
# ---------------------------------------------------------------------------
# (dims, D, M, upper end of A): decays of ~1 (A above the clamp) only where
# the grid has few wavefront levels; over many levels they make the states
# grow combinatorially with rotation-mixed cancellation, an ill-conditioned
# sum whose fp32 result depends on the summation order.
GPU_CASES = [((7, 5), 4, 3, 0.2), ((16, 12), 5, 4, 0.2), ((6, 5, 4), 3, 8, 0.2),
             ((1, 9), 2, 16, 0.2), ((11,), 6, 4, 0.2), ((3, 4, 2, 3), 4, 2, 0.2),
             ((20, 24), 64, 16, -0.05), ((24, 16, 12), 8, 16, -0.05)]


@pytest.mark.gpu
@pytest.mark.parametrize("dims,D,M,a_hi", GPU_CASES)
@pytest.mark.parametrize("with_theta", [True, False])
def test_device_entry_points_vs_oracle(dims, D, M, a_hi, with_theta):
    import kmamba as K
    import torch
    x, A, B, Cm, dt, theta, lam = m3_inputs(dims, D, M, 6, a_hi=a_hi)
    th = theta if with_theta else None
    yr, hr = O.scannd_ref(dims, x, A, B, Cm, dt, lam=lam, theta=th, nthreads=8, fast=True)
    ya, ha = O.scannd_ref(dims, np.abs(x), A, np.abs(B), np.abs(Cm), dt, lam=lam,
                          theta=None if th is None else np.zeros_like(th), nthreads=8, fast=True)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    P = int(np.prod(dims))
    for entry in ("km", "om"):
        h = torch.zeros((P, D, M), device="cuda")
        y = torch.zeros((P, D), device="cuda")
        ts = [T(a) for a in (x, A, B, Cm, dt)]
        tth = None if th is None else T(th)
        tl = T(lam)
        if entry == "km":
            K.scannd_fwd(dims, *ts, h, y, theta=tth, lam=tl)
            torch.cuda.synchronize()
        else:
            p, keep = K.scannd_params(dims, *ts, h, y, tth, tl)
            assert K.om_scannd_forward(C.byref(p)) == 0, K.km_last_error()
        # kappa: magnitudes without cancellation (rotation by 0 keeps them so).
        assert_close(y.cpu().numpy(), yr, TOL_F32, f"{entry} y", np.abs(ya) + np.abs(yr))
        assert_close(h.cpu().numpy(), hr, TOL_F32, f"{entry} h", np.abs(ha) + np.abs(hr))


@pytest.mark.gpu
def test_host_pointer_entry_points_and_dispatch_semantics():
    import kmamba as K
    for dims, D, M in (((6, 5), 4, 3), ((4, 3, 5), 3, 4)):
        x, A, B, Cm, dt, theta, lam = m3_inputs(dims, D, M, 7)
        P = int(np.prod(dims))
        yr, hr = O.scannd_ref(dims, x, A, B, Cm, dt, lam=lam, theta=theta)
        ya, ha = O.scannd_ref(dims, np.abs(x), A, np.abs(B), np.abs(Cm), dt, lam=lam,
                              theta=np.zeros_like(theta))
        for fn in ("ref", "plan", "dispatch"):
            h = np.zeros((P, D, M), np.float32)
            y = np.zeros((P, D), np.float32)
            p, keep = K.scannd_params(dims, x, A, B, Cm, dt, h, y, theta, lam)
            if fn == "ref":
                rc = K.scannd_ref(C.byref(p))
            elif fn == "plan":
                plan = K.km_wavefront_plan_create(K.longs(dims), len(dims))
                rc = K.scannd_ref_with_plan(C.byref(p), plan)
                K.km_wavefront_plan_free(plan)
            else:
                rc = K.scannd(C.byref(p))
            assert rc == 0, (fn, K.km_last_error())
            if fn == "dispatch" and len(dims) == 2:
                # The reference dispatcher's rank-2 path (scan2d) has no
                # Mamba-3 operands: the lambda-free scan2d result.
                y2, h2 = O.scannd_ref(dims, x, A, B, Cm, dt)
                yk, hk = O.scannd_ref(dims, np.abs(x), A, np.abs(B), np.abs(Cm), dt)
                assert_close(y, y2, TOL_F32, "dispatch 2D y", yk)
                continue
            assert_close(y, yr, TOL_F32, f"{fn} y", np.abs(ya) + np.abs(yr))
            assert_close(h, hr, TOL_F32, f"{fn} h", np.abs(ha) + np.abs(hr))


@pytest.mark.gpu
def test_noalloc_rejects_the_lambda_branch():
    import kmamba as K
    import torch
    dims, D, M = (8, 8), 4, 16
    x, A, B, Cm, dt, theta, lam = m3_inputs(dims, D, M, 8)
    P = int(np.prod(dims))
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    h = torch.zeros((P, D, M), device="cuda")
    y = torch.zeros((P, D), device="cuda")
    p, keep = K.scannd_params(dims, T(x), T(A), T(B), T(Cm), T(dt), h, y, None, T(lam))
    assert K.km_scannd_fwd_noalloc_c(C.byref(p), None) == -1
    assert "lambda" in K.km_last_error()

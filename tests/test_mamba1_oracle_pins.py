"""Pins of the configs[4] Mamba-1 block oracle (tests/kmtest.py
mamba1_block_ref) and of the reference activations it uses (CPU only).

The reference has no Mamba-1 block function; configs[4] composes reference
pieces: the projections (kernels/gemm_f32.c:13-31), the causal ConvND in 1D
(src/convnd.c:83-126), SiLU / softplus (include/kmamba_kernels.h:35-49,
kernels/activations_f32.c:7-29) and the Scan1D recurrence
(cpu/scan1d.asm:53-169). What is pinned here:

* the activations, bit-exact against the compiled reference's silu_f32 /
  softplus_f32 (oracle/_ref), plus their closed forms;
* the composition, against an independent float64 loop implementation
  written from the published Mamba-1 block (Gu & Dao 2023, "Mamba:
  Linear-Time Sequence Modeling with Selective State Spaces", Algorithm 2
  and Figure 3: in_proj -> (x, z); x -> causal depthwise conv1d -> SiLU ->
  selective SSM with Abar = exp(delta A), Bbar = delta B, delta =
  softplus(dt_proj(x_proj(u)[:R]) + dt_bias); y = (SSM(u) + D u) * SiLU(z);
  out_proj), and against closed forms that a composition mistake breaks:
  an impulse conv kernel, delta -> 0 through dt_bias -> -inf, a zero z half
  of W_in (an x/z swap shows), the conv orientation, and the D skip inside
  the gate.
"""
import math

import numpy as np
import pytest

import oracle as O
from kmtest import mamba1_block_ref, rng_for, silu_ref, softplus_ref

needs_ref = pytest.mark.skipif(not O.REF_AVAILABLE, reason="oracle/_ref not built (reference tree absent)")


def _activation_inputs():
    g = rng_for("act-pins")
    special = np.array([0.0, -0.0, 1.0, -1.0, 1e-30, -1e-30, 1e-45, 20.0, -20.0, 80.0, -80.0,
                        88.0, 88.7, 88.8, 89.0, -88.7, -89.0, -103.0, -104.0, 100.0, -100.0,
                        1e4, -1e4, np.finfo(np.float32).max, -np.finfo(np.float32).max],
                       dtype=np.float32)
    return np.concatenate([special, g.standard_normal(20000).astype(np.float32) * 6,
                           g.uniform(-120, 120, 20000).astype(np.float32)])


@needs_ref
def test_activations_bit_exact_vs_compiled_reference():
    v = _activation_inputs()
    for name, fn in (("silu", O.silu), ("softplus", O.softplus)):
        ours, theirs = fn(v), fn(v, use_ref=True)
        same = (ours.view(np.uint32) == theirs.view(np.uint32)) | (np.isnan(ours) & np.isnan(theirs))
        assert same.all(), f"{name}: {np.count_nonzero(~same)} values differ from the reference"
    # The block oracle's helpers are the pinned restatement.
    assert np.array_equal(silu_ref(v), O.silu(v), equal_nan=True)
    assert np.array_equal(softplus_ref(v), O.softplus(v), equal_nan=True)


def test_activations_closed_forms():
    v = _activation_inputs()
    v = v[np.abs(v) < 80]
    d = v.astype(np.float64)
    silu64 = d / (1.0 + np.exp(-d))
    soft64 = np.log1p(np.exp(d))
    # A few fp32 roundings (exp, add, div / log) against float64.
    assert np.max(np.abs(O.silu(v) - silu64) / np.maximum(np.abs(silu64), 1e-30)) < 1e-6
    # logf(1 + e^x) is accurate to a few ulp of max(1, result): for x << 0 the
    # sum 1 + e^x rounds to 1 first, so the error there is absolute.
    assert np.max(np.abs(O.softplus(v) - soft64) / np.maximum(soft64, 1.0)) < 3e-7
    assert O.silu(np.float32([0.0]))[0] == 0.0
    assert O.softplus(np.float32([0.0]))[0] == np.float32(math.log(2.0))
    # No overflow guard in the reference: softplus(89) is +inf, and far below
    # zero 1 + e^x rounds to 1, so softplus is exactly 0.
    assert np.isinf(O.softplus(np.float32([89.0]))[0])
    assert O.softplus(np.float32([-100.0]))[0] == 0.0
    assert O.silu(np.float32([100.0]))[0] == np.float32(100.0)


# ---------------------------------------------------------------------------
# Composition
# ---------------------------------------------------------------------------
def _weights(dim, di, N, K, R, seed=0, std=0.3):
    g = rng_for("m1pin", dim, di, N, K, R, seed)
    return {
        "W_in": (g.standard_normal((2 * di, dim)) * std).astype(np.float32),
        "conv_w": (g.standard_normal((K, di)) * 0.5).astype(np.float32),
        "conv_b": (g.standard_normal(di) * 0.1).astype(np.float32),
        "W_x": (g.standard_normal((R + 2 * N, di)) * std).astype(np.float32),
        "W_dt": (g.standard_normal((di, R)) * std).astype(np.float32),
        "dt_bias": (g.standard_normal(di) * 0.5 - 1.0).astype(np.float32),
        "A": -g.uniform(0.5, 3.0, (di, N)).astype(np.float32),
        "Dskip": g.uniform(0.5, 1.5, di).astype(np.float32),
        "W_out": (g.standard_normal((dim, di)) * std).astype(np.float32),
    }


def mamba1_fp64_loops(x, w):
    """Mamba-1 block forward in float64 with explicit loops, written from the
    published algorithm (Gu & Dao 2023, Algorithm 2 and Figure 3), not from
    the oracle: per batch element b and step t,
      xi_t = W_in[:di] x_t;  z_t = W_in[di:] x_t
      c_t[j] = conv_b[j] + sum_{k<K, t-(K-1)+k >= 0} conv_w[k, j] xi_{t-(K-1)+k}[j]
      u_t = SiLU(c_t)
      [dt_low | B_t | C_t] = W_x u_t
      delta_t = softplus(W_dt dt_low + dt_bias)
      h_t[j, n] = exp(delta_t[j] A[j, n]) h_{t-1}[j, n] + delta_t[j] B_t[n] u_t[j]
      y_t[j] = (sum_n C_t[n] h_t[j, n] + D[j] u_t[j]) SiLU(z_t[j])
      out_t = W_out y_t."""
    f = {k: np.asarray(v, np.float64) for k, v in w.items()}
    x = np.asarray(x, np.float64)
    Bsz, L, dim = x.shape
    di = f["W_in"].shape[0] // 2
    K = f["conv_w"].shape[0]
    N = f["A"].shape[1]
    R = f["W_dt"].shape[1]

    def silu(v):
        return v / (1.0 + math.exp(-v))

    def softplus(v):
        return math.log1p(math.exp(v)) if v < 30 else v + math.log1p(math.exp(-v))

    out = np.zeros((Bsz, L, dim))
    for b in range(Bsz):
        xi = np.zeros((L, di))
        z = np.zeros((L, di))
        for t in range(L):
            for j in range(di):
                xi[t, j] = sum(f["W_in"][j, i] * x[b, t, i] for i in range(dim))
                z[t, j] = sum(f["W_in"][di + j, i] * x[b, t, i] for i in range(dim))
        h = np.zeros((di, N))
        for t in range(L):
            u = np.zeros(di)
            for j in range(di):
                c = f["conv_b"][j]
                for k in range(K):
                    s = t - (K - 1) + k
                    if s >= 0:
                        c += f["conv_w"][k, j] * xi[s, j]
                u[j] = silu(c)
            proj = [sum(f["W_x"][r, j] * u[j] for j in range(di)) for r in range(R + 2 * N)]
            dt_low, Bt, Ct = proj[:R], proj[R:R + N], proj[R + N:]
            y = np.zeros(di)
            for j in range(di):
                delta = softplus(sum(f["W_dt"][j, r] * dt_low[r] for r in range(R)) + f["dt_bias"][j])
                acc = 0.0
                for n in range(N):
                    h[j, n] = math.exp(delta * f["A"][j, n]) * h[j, n] + delta * Bt[n] * u[j]
                    acc += Ct[n] * h[j, n]
                y[j] = (acc + f["Dskip"][j] * u[j]) * silu(z[t, j])
            for o in range(dim):
                out[b, t, o] = sum(f["W_out"][o, j] * y[j] for j in range(di))
    return out


@pytest.mark.parametrize("Bsz,L,dim,di,N,K,R", [(2, 9, 6, 5, 4, 4, 2), (1, 12, 4, 7, 3, 2, 3),
                                                (2, 6, 5, 4, 2, 3, 1)])
def test_block_oracle_vs_fp64_published_algorithm(Bsz, L, dim, di, N, K, R):
    w = _weights(dim, di, N, K, R)
    x = rng_for("m1x", Bsz, L, dim).standard_normal((Bsz, L, dim)).astype(np.float32)
    got = mamba1_block_ref(x, w, clamp=False).astype(np.float64)
    want = mamba1_fp64_loops(x, w)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < 2e-6, err
    # A plausible mistake fails it: dt_bias after the softplus instead of inside.
    bad = dict(w)
    bad["dt_bias"] = w["dt_bias"] + np.float32(0.25)
    assert np.abs(mamba1_block_ref(x, bad, clamp=False) - want).max() / np.abs(want).max() > 1e-3


def test_impulse_conv_kernel_is_identity():
    dim, di, N, K, R = 6, 5, 4, 4, 2
    w = _weights(dim, di, N, K, R, seed=1)
    w["conv_w"] = np.zeros((K, di), np.float32)
    w["conv_w"][K - 1] = 1.0          # the current step's tap
    w["conv_b"] = np.zeros(di, np.float32)
    x = rng_for("m1imp").standard_normal((2, 8, dim)).astype(np.float32)
    _, p = mamba1_block_ref(x, w, parts=True)
    assert np.array_equal(p["u"], silu_ref(p["xi"]))


def test_conv_orientation_first_tap_is_oldest_step():
    dim, di, N, K, R = 6, 5, 4, 4, 2
    w = _weights(dim, di, N, K, R, seed=2)
    w["conv_w"] = np.zeros((K, di), np.float32)
    w["conv_w"][0] = 1.0              # tap k = 0 reads step t - (K - 1)
    x = rng_for("m1ori").standard_normal((2, 9, dim)).astype(np.float32)
    _, p = mamba1_block_ref(x, w, parts=True)
    shifted = p["xi"][:, :-(K - 1)] + w["conv_b"]
    assert np.array_equal(p["u"][:, K - 1:], silu_ref(shifted.astype(np.float32)))
    assert np.array_equal(p["u"][:, :K - 1], np.broadcast_to(silu_ref(w["conv_b"]), p["u"][:, :K - 1].shape))


def test_dt_bias_to_minus_infinity_removes_the_scan():
    # softplus(v - 200) is exactly 0 in fp32, so delta = 0, h stays 0 and the
    # block reduces to out = W_out ((D u) SiLU(z)).
    dim, di, N, K, R = 6, 5, 4, 4, 2
    w = _weights(dim, di, N, K, R, seed=3)
    w["dt_bias"] = np.full(di, -200.0, np.float32)
    x = rng_for("m1dt").standard_normal((2, 7, dim)).astype(np.float32)
    out, p = mamba1_block_ref(x, w, parts=True)
    assert not p["delta"].any()
    assert not p["scan"].any()
    y = (w["Dskip"] * p["u"]) * silu_ref(p["z"])
    assert np.array_equal(p["y"], y.astype(np.float32))
    np.testing.assert_allclose(out, y @ w["W_out"].T, rtol=1e-6, atol=1e-7)


def test_zero_z_half_zeroes_the_output_and_exposes_a_swap():
    # With the z half of W_in zero, SiLU(z) = 0 gates everything to 0; with
    # the x half zero instead, the output is not 0 (u = SiLU(conv_b) != 0).
    dim, di, N, K, R = 6, 5, 4, 4, 2
    x = rng_for("m1z").standard_normal((2, 7, dim)).astype(np.float32)
    w = _weights(dim, di, N, K, R, seed=4)
    w["W_in"][di:] = 0.0
    assert not mamba1_block_ref(x, w).any()
    w = _weights(dim, di, N, K, R, seed=4)
    w["W_in"][:di] = 0.0
    out, p = mamba1_block_ref(x, w, parts=True)
    assert np.abs(out).max() > 1e-3
    assert np.array_equal(p["u"], np.broadcast_to(silu_ref(w["conv_b"]), p["u"].shape))


def test_skip_term_sits_inside_the_gate():
    # y = (scan + D u) SiLU(z): doubling D adds exactly D u SiLU(z) once more.
    dim, di, N, K, R = 6, 5, 4, 4, 2
    w = _weights(dim, di, N, K, R, seed=5)
    x = rng_for("m1d").standard_normal((1, 8, dim)).astype(np.float32)
    _, p1 = mamba1_block_ref(x, w, parts=True)
    w2 = dict(w)
    w2["Dskip"] = 2 * w["Dskip"]
    _, p2 = mamba1_block_ref(x, w2, parts=True)
    extra = (w["Dskip"].astype(np.float64) * p1["u"]) * silu_ref(p1["z"])
    np.testing.assert_allclose(p2["y"] - p1["y"], extra, rtol=1e-5, atol=1e-6)

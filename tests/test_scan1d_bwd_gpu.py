"""GPU parity of the Scan1D backward (libkmamba, gfx950) against the CPU
oracle's restatement of cpu/scan1d_backward.c on identical seeded inputs.

Metric: condition-scaled max relative error (tests/kmtest.py), kappa from
scan1d_bwd_kappa (the backward on absolute values). Tolerances 1e-4 (fp32
I/O) and 2e-2 (bf16 I/O against the fp32 oracle of the unrounded inputs).
"""
import ctypes as C

import numpy as np
import pytest

import kmamba as K
import oracle as O
from kmtest import (TOL_BF16, TOL_F32, assert_close, bf16_round, rng_for, scan1d_bwd_kappa,
                    scan1d_inputs)

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"
NAMES = ("dx", "ddelta", "dA", "dB", "dC")


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    torch.zeros(1, device=DEV)
    assert K.kmamba_cuda_available() == 1, K.km_last_error()


def T(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


def oracle_bwd(x, dt, A, Bm, Cm, dy, *, h0=None, bc_strides=None, clamp=True):
    _, _, hh = O.scan1d_batched(x, dt, A, Bm, Cm, h0=h0, bc_strides=bc_strides, clamp=clamp,
                                hist=True, nthreads=8, fast=True)
    out = O.scan1d_batched_backward(x, dt, A, Bm, Cm, dy, hh, h0=h0, bc_strides=bc_strides,
                                    nthreads=8, fast=True)
    return out, hh


def run_bwd(x, dt, A, Bm, Cm, dy, *, mode, h0=None, hist=None, bc_strides=None, clamp=True,
            bf16=False, workspace=False):
    """mode: 'hist' (states given), 'ckpt' (forward checkpoints from
    km_scan1d_fwd), 'recompute' (the library recomputes them)."""
    io = torch.bfloat16 if bf16 else torch.float32
    tx, tdt, tB, tC, tdy = T(x, io), T(dt, io), T(Bm, io), T(Cm, io), T(dy, io)
    tA = T(A)
    th0 = None if h0 is None else T(h0)
    Bsz, L, D = x.shape
    N = A.shape[1]
    dx, ddt = torch.empty_like(tx), torch.empty_like(tx)
    dA = torch.empty((D, N), device=DEV)
    dB, dC = torch.full_like(tB, float("nan")), torch.full_like(tC, float("nan"))
    kw = dict(h0=th0, bc_strides=bc_strides, clamp=clamp)
    if mode == "hist":
        kw["h_hist"] = T(hist)
    elif mode == "ckpt":
        nck = (L + K.KM_SCAN1D_CKPT_STEPS - 1) // K.KM_SCAN1D_CKPT_STEPS
        ck = torch.full((Bsz, nck, D, N), float("nan"), device=DEV)
        K.scan1d_fwd(tx, tdt, tA, tB, tC, None, h0=th0, h_ckpt=ck, bc_strides=bc_strides,
                     clamp=clamp)
        kw["h_ckpt"] = ck
    if workspace:
        args = K.scan1d_bwd_args(tx, tdt, tA, tB, tC, tdy, dx, ddt, dA, dB, dC, **kw)
        nbytes = K.km_scan1d_bwd_workspace_bytes(C.byref(args))
        kw["workspace"] = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=DEV)
    K.scan1d_bwd(tx, tdt, tA, tB, tC, tdy, dx, ddt, dA, dB, dC, **kw)
    torch.cuda.synchronize()
    return tuple(t.float().cpu().numpy() for t in (dx, ddt, dA, dB, dC))


def check_all(got, ref, kap, tol, tag):
    errs = {}
    for n, g, r, k in zip(NAMES, got, ref, kap):
        errs[n] = assert_close(g, r, tol, f"{tag} {n}", k)
    return errs


def dy_for(Bsz, L, D, seed=5):
    return rng_for("dy", Bsz, L, D, seed).standard_normal((Bsz, L, D), dtype=np.float32)


@pytest.mark.parametrize("mode", ["hist", "ckpt", "recompute"])
@pytest.mark.parametrize("Bsz,L,D,N", [(2, 200, 48, 16), (1, 64, 16, 16), (2, 130, 64, 8),
                                       (1, 77, 100, 4), (2, 65, 64, 2), (1, 300, 65, 1),
                                       (2, 50, 40, 3), (3, 1, 32, 16), (1, 129, 33, 16),
                                       (2, 31, 17, 16), (1, 96, 200, 16)])
def test_shared_bc_vs_oracle(Bsz, L, D, N, mode):
    # L = 1 and 31 give one partial super-chunk; D = 17, 33 and 200 leave
    # the last channel group partly filled.
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=11)
    dy = dy_for(Bsz, L, D)
    ref, hh = oracle_bwd(x, dt, A, Bm, Cm, dy)
    got = run_bwd(x, dt, A, Bm, Cm, dy, mode=mode, hist=hh)
    kap = scan1d_bwd_kappa(x, dt, A, Bm, Cm, dy)
    check_all(got, ref, kap, TOL_F32, f"shared {mode}")


@pytest.mark.parametrize("mode", ["hist", "recompute"])
@pytest.mark.parametrize("Bsz,L,D,N", [(2, 150, 40, 16), (1, 70, 64, 8), (2, 33, 17, 1)])
def test_per_channel_bc_generic_A_and_h0(Bsz, L, D, N, mode):
    x, dt, A, _, _ = scan1d_inputs(Bsz, L, D, N, seed=12)
    g = rng_for("pc", Bsz, L, D, N)
    A = (A * g.uniform(0.1, 1.0, size=A.shape)).astype(np.float32)
    Bm = (g.standard_normal((Bsz, L, D, N)) * 0.25).astype(np.float32)
    Cm = (g.standard_normal((Bsz, L, D, N)) * 0.25).astype(np.float32)
    h0 = g.standard_normal((Bsz, D, N)).astype(np.float32)
    strides = (L * D * N, D * N, N)
    dy = dy_for(Bsz, L, D)
    ref, hh = oracle_bwd(x, dt, A, Bm, Cm, dy, h0=h0, bc_strides=strides)
    got = run_bwd(x, dt, A, Bm, Cm, dy, mode=mode, hist=hh, h0=h0, bc_strides=strides)
    kap = scan1d_bwd_kappa(x, dt, A, Bm, Cm, dy, h0=h0, bc_strides=strides)
    check_all(got, ref, kap, TOL_F32, f"per-channel {mode}")


def test_caller_workspace_matches_library_workspace():
    x, dt, A, Bm, Cm = scan1d_inputs(2, 300, 64, 16, seed=13)
    dy = dy_for(2, 300, 64)
    a = run_bwd(x, dt, A, Bm, Cm, dy, mode="recompute")
    b = run_bwd(x, dt, A, Bm, Cm, dy, mode="recompute", workspace=True)
    for n, u, v in zip(NAMES, a, b):
        scale = np.abs(u).max() + 1e-30
        assert np.abs(u - v).max() <= 1e-5 * scale, n


def test_recompute_follows_forward_clamp():
    # States leave [-1000, 1000]: checkpoints and recomputation must follow
    # the per-step clamp of the forward, as the saved history does.
    Bsz, L, D, N = 2, 200, 32, 16
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=14)
    Bm = Bm * 800.0
    A = A * 0.01
    dy = dy_for(Bsz, L, D)
    ref, hh = oracle_bwd(x, dt, A, Bm, Cm, dy)
    assert np.abs(hh).max() == 1000.0
    kap = scan1d_bwd_kappa(x, dt, A, Bm, Cm, dy)
    for mode in ("hist", "ckpt", "recompute"):
        got = run_bwd(x, dt, A, Bm, Cm, dy, mode=mode, hist=hh)
        check_all(got, ref, kap, TOL_F32, f"clamped {mode}")


@pytest.mark.parametrize("N", [16, 8])
def test_recompute_clamp_in_a_few_steps_generic_A(N):
    # Generic (not S4D-real) decays, and states that leave [-1000, 1000] only
    # around steps 150-155 of 300: the recomputation from checkpoints must
    # follow the clamp there and nowhere else, for every output of the
    # channel groups it touches.
    Bsz, L, D = 2, 300, 40
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=21)
    g = rng_for("clamp-local", N)
    A = (A * g.uniform(0.001, 0.01, size=A.shape)).astype(np.float32)
    Bm = Bm.copy()
    Bm[:, 150:156] *= 4000.0
    dy = dy_for(Bsz, L, D)
    ref, hh = oracle_bwd(x, dt, A, Bm, Cm, dy)
    assert np.abs(hh).max() == 1000.0
    assert np.abs(hh[:, :140]).max() < 1000.0
    kap = scan1d_bwd_kappa(x, dt, A, Bm, Cm, dy)
    for mode in ("ckpt", "recompute"):
        got = run_bwd(x, dt, A, Bm, Cm, dy, mode=mode, hist=hh)
        check_all(got, ref, kap, TOL_F32, f"locally clamped {mode}")


def test_bf16_io_against_fp32_oracle():
    x, dt, A, Bm, Cm = scan1d_inputs(2, 256, 64, 16, seed=15)
    dy = dy_for(2, 256, 64)
    ref, _ = oracle_bwd(x, dt, A, Bm, Cm, dy)
    got = run_bwd(x, dt, A, Bm, Cm, dy, mode="recompute", bf16=True)
    kap = scan1d_bwd_kappa(x, dt, A, Bm, Cm, dy)
    check_all(got, ref, kap, TOL_BF16, "bf16")
    # Against the oracle on the bf16-rounded inputs, with bf16-rounded outputs.
    xr, dtr, Br, Cr, dyr = (bf16_round(v) for v in (x, dt, Bm, Cm, dy))
    ref_r, _ = oracle_bwd(xr, dtr, A, Br, Cr, dyr)
    for n, g, r, k in zip(NAMES, got, ref_r, kap):
        rr = r if n == "dA" else bf16_round(r)
        assert_close(g, rr, 1e-2, f"bf16 rounded-input {n}", k)


def _ref_api_inputs(L, D, M, seed=0):
    g = rng_for("bwdapi", L, D, M, seed)
    x = g.uniform(-1, 1, (L, D)).astype(np.float32)
    A = g.uniform(-1, -0.01, (D, M)).astype(np.float32)
    B = g.uniform(-0.5, 0.5, (L, D, M)).astype(np.float32)
    Cm = g.uniform(-0.5, 0.5, (L, D, M)).astype(np.float32)
    dt = g.uniform(0.01, 0.5, (L, D)).astype(np.float32)
    dy = g.standard_normal((L, D)).astype(np.float32)
    h0 = g.uniform(-1, 1, (D, M)).astype(np.float32)
    return x, A, B, Cm, dt, dy, h0


def _api_kappa(x, A, B, Cm, dt, dy, h0):
    L, D, M = B.shape
    k = scan1d_bwd_kappa(x[None], dt[None], A, B[None], Cm[None], dy[None],
                         h0=None if h0 is None else h0[None], bc_strides=(L * D * M, D * M, M))
    return k[0][0], k[1][0], k[2], k[3][0], k[4][0]


@pytest.mark.parametrize("L,D,M,use_h0", [(4, 8, 1, False), (16, 16, 2, True), (64, 32, 16, True),
                                          (130, 48, 16, False), (40, 20, 5, True)])
def test_scan1d_backward_host_pointer_api(L, D, M, use_h0):
    x, A, B, Cm, dt, dy, h0 = _ref_api_inputs(L, D, M)
    h0 = h0 if use_h0 else None
    # Forward history as the reference harness produces it (running state).
    _, _, hh = O.scan1d_batched(x[None], dt[None], A, B[None], Cm[None],
                                h0=None if h0 is None else h0[None],
                                bc_strides=(L * D * M, D * M, M), hist=True)
    h = hh[0]
    rdx, rdA, rdB, rdC, rdd = O.scan1d_backward(x, A, B, Cm, dt, h, dy, h0=h0)
    out = dict(dx=np.full((L, D), np.nan, np.float32), dA=np.full((D, M), np.nan, np.float32),
               dB=np.full((L, D, M), np.nan, np.float32), dC=np.full((L, D, M), np.nan, np.float32),
               ddelta=np.full((L, D), np.nan, np.float32))
    p = K.ScanBackwardParams(K.ptr(x), K.ptr(A), K.ptr(B), K.ptr(Cm), K.ptr(dt), K.ptr(h0),
                             K.ptr(h), K.ptr(dy), K.ptr(out["dx"]), K.ptr(out["dA"]),
                             K.ptr(out["dB"]), K.ptr(out["dC"]), K.ptr(out["ddelta"]), L, D, M)
    K.scan1d_backward(C.byref(p))
    assert K.km_last_error() == ""
    kdx, kdd, kdA, kdB, kdC = _api_kappa(x, A, B, Cm, dt, dy, h0)
    assert_close(out["dx"], rdx, TOL_F32, "dx", kdx)
    assert_close(out["ddelta"], rdd, TOL_F32, "ddelta", kdd)
    assert_close(out["dA"], rdA, TOL_F32, "dA", kdA)
    assert_close(out["dB"], rdB, TOL_F32, "dB", kdB)
    assert_close(out["dC"], rdC, TOL_F32, "dC", kdC)


def test_om_scan1d_backward_device_api():
    L, D, M = 150, 40, 16
    x, A, B, Cm, dt, dy, _ = _ref_api_inputs(L, D, M, seed=1)
    _, _, hh = O.scan1d_batched(x[None], dt[None], A, B[None], Cm[None],
                                bc_strides=(L * D * M, D * M, M), hist=True)
    h = hh[0]
    rdx, rdA, rdB, rdC, rdd = O.scan1d_backward(x, A, B, Cm, dt, h, dy)
    tx, tA, tB, tC, tdt, th, tdy = map(T, (x, A, B, Cm, dt, h, dy))
    dx, ddt = torch.empty((L, D), device=DEV), torch.empty((L, D), device=DEV)
    dA = torch.empty((D, M), device=DEV)
    dB, dC = torch.empty((L, D, M), device=DEV), torch.empty((L, D, M), device=DEV)
    for fn in (K.om_scan1d_backward, K.mamba_scan1d_cuda_backward):
        fn(K.ptr(tdy), K.ptr(tx), K.ptr(tA), K.ptr(tB), K.ptr(tC), K.ptr(tdt), K.ptr(th), K.ptr(dx),
           K.ptr(dA), K.ptr(dB), K.ptr(dC), K.ptr(ddt), L, D, M)
        assert K.km_last_error() == ""
        kdx, kdd, kdA, kdB, kdC = _api_kappa(x, A, B, Cm, dt, dy, None)
        assert_close(dx.cpu().numpy(), rdx, TOL_F32, "dx", kdx)
        assert_close(ddt.cpu().numpy(), rdd, TOL_F32, "ddelta", kdd)
        assert_close(dA.cpu().numpy(), rdA, TOL_F32, "dA", kdA)
        assert_close(dB.cpu().numpy(), rdB, TOL_F32, "dB", kdB)
        assert_close(dC.cpu().numpy(), rdC, TOL_F32, "dC", kdC)


@pytest.mark.parametrize("L,D,with_diag,use_h0", [(6, 5, False, False), (6, 16, True, True),
                                                 (70, 300, True, False), (33, 19, False, True)])
def test_m1_shared_bc_vs_oracle(L, D, with_diag, use_h0):
    g = rng_for("m1", L, D)
    x = g.uniform(-1, 1, (L, D)).astype(np.float32)
    A = g.uniform(-1, -0.05, D).astype(np.float32)
    B = g.uniform(-0.5, 0.5, D).astype(np.float32)
    Cm = g.uniform(-0.5, 0.5, D).astype(np.float32)
    dt = g.uniform(0.05, 0.5, L).astype(np.float32)
    dy = g.standard_normal((L, D)).astype(np.float32)
    h0 = g.uniform(-1, 1, D).astype(np.float32) if use_h0 else None
    # Forward history of the shared-B/C M=1 scan.
    e = np.exp(dt[:, None].astype(np.float64) * A[None, :])
    h = np.zeros((L, D))
    prev = np.zeros(D) if h0 is None else h0.astype(np.float64)
    for t in range(L):
        prev = e[t] * prev + B * dt[t] * x[t]
        h[t] = prev
    h = h.astype(np.float32)
    A_diag = np.exp(dt[:, None] * A[None, :]).astype(np.float32) if with_diag else None
    ref = O.scan1d_backward_m1_shared_bc(x, A, B, Cm, dt, h, dy, A_diag=A_diag, h0=h0)
    out = [np.full((L, D), np.nan, np.float32), np.full(D, np.nan, np.float32),
           np.full(D, np.nan, np.float32), np.full(D, np.nan, np.float32),
           np.full(L, np.nan, np.float32)]
    p = K.ScanBackwardSharedParams(K.ptr(x), K.ptr(A), K.ptr(A_diag), K.ptr(B), K.ptr(Cm),
                                   K.ptr(dt), K.ptr(h0), K.ptr(h), K.ptr(dy), *map(K.ptr, out), L, D)
    K.mamba_scan1d_backward_m1_shared_bc(C.byref(p))
    assert K.km_last_error() == ""
    # kappa: the same backward on absolute values (|ddelta| bound as in kmtest).
    ab = [np.abs(v) for v in (x, B, Cm, dy)]
    habs = np.zeros((L, D))
    prev = np.zeros(D) if h0 is None else np.abs(h0).astype(np.float64)
    for t in range(L):
        prev = e[t] * prev + ab[1] * dt[t] * ab[0][t]
        habs[t] = prev
    kap = O.scan1d_backward_m1_shared_bc(ab[0], A, ab[1], ab[2], dt, habs.astype(np.float32), ab[3],
                                         A_diag=A_diag, h0=None if h0 is None else np.abs(h0))
    t2 = (ab[0] * kap[0]).sum(axis=1) / dt
    kdd = np.maximum(2 * t2 - kap[4], 0)
    for n, gg, r, k in zip(("dx", "dA", "dB", "dC", "ddelta"), out, ref,
                           (kap[0], kap[1], kap[2], kap[3], kdd)):
        assert_close(gg, r, TOL_F32, f"m1 {n}", k)


def test_config1_full_size_sampled():
    # configs[1] backward (B=8, L=4096, D=1024, N=16, fp32) on the GPU, with
    # states recomputed from checkpoints. Checked against the oracle on a
    # sample of channels over every batch element (dx, ddelta, dA are exact
    # sub-problems per channel) and on batch element 0 in full (dB, dC sum
    # over all channels).
    Bsz, L, D, N = 8, 4096, 1024, 16
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=0, tag="config1")
    dy = dy_for(Bsz, L, D, seed=0)
    got = run_bwd(x, dt, A, Bm, Cm, dy, mode="ckpt")
    for gg in got:
        assert np.isfinite(gg).all()
    sel = np.sort(rng_for("bsel").choice(D, 32, replace=False))
    args = (x[:, :, sel], dt[:, :, sel], A[sel], Bm, Cm, dy[:, :, sel])
    ref, _ = oracle_bwd(*args)
    kap = scan1d_bwd_kappa(*args)
    assert_close(got[0][:, :, sel], ref[0], TOL_F32, "dx", kap[0])
    assert_close(got[1][:, :, sel], ref[1], TOL_F32, "ddelta", kap[1])
    assert_close(got[2][sel], ref[2], TOL_F32, "dA", kap[2])
    args0 = (x[:1], dt[:1], A, Bm[:1], Cm[:1], dy[:1])
    ref0, _ = oracle_bwd(*args0)
    kap0 = scan1d_bwd_kappa(*args0)
    assert_close(got[3][:1], ref0[3], TOL_F32, "dB[b=0]", kap0[3])
    assert_close(got[4][:1], ref0[4], TOL_F32, "dC[b=0]", kap0[4])


def test_config1_bf16_full_size_sampled():
    # configs[1] backward with bf16 I/O (x, delta, B, C, dy and dx, ddelta,
    # dB, dC bf16; A, dA and the states fp32) at full size, B=8 L=4096 D=1024
    # N=16, states from the forward's checkpoints. Against the fp32 oracle of
    # the unrounded inputs at the bf16 tolerance: dx, ddelta, dA on a sample
    # of channels over every batch element (exact sub-problems per channel),
    # dB, dC (sums over every channel) on batch elements 0 and 7 in full.
    Bsz, L, D, N = 8, 4096, 1024, 16
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=0, tag="config1")
    dy = dy_for(Bsz, L, D, seed=0)
    got = run_bwd(x, dt, A, Bm, Cm, dy, mode="ckpt", bf16=True)
    for gg in got:
        assert np.isfinite(gg).all()
    sel = np.sort(rng_for("bsel-bf16").choice(D, 24, replace=False))
    args = (x[:, :, sel], dt[:, :, sel], A[sel], Bm, Cm, dy[:, :, sel])
    ref, _ = oracle_bwd(*args)
    kap = scan1d_bwd_kappa(*args)
    assert_close(got[0][:, :, sel], ref[0], TOL_BF16, "bf16 dx", kap[0])
    assert_close(got[1][:, :, sel], ref[1], TOL_BF16, "bf16 ddelta", kap[1])
    assert_close(got[2][sel], ref[2], TOL_BF16, "bf16 dA", kap[2])
    for b in (0, Bsz - 1):
        argsb = (x[b:b + 1], dt[b:b + 1], A, Bm[b:b + 1], Cm[b:b + 1], dy[b:b + 1])
        refb, _ = oracle_bwd(*argsb)
        kapb = scan1d_bwd_kappa(*argsb)
        assert_close(got[3][b:b + 1], refb[3], TOL_BF16, f"bf16 dB[b={b}]", kapb[3])
        assert_close(got[4][b:b + 1], refb[4], TOL_BF16, f"bf16 dC[b={b}]", kapb[4])


@pytest.mark.parametrize("Bsz,L,D,N,layout", [(2, 300, 96, 16, "shared"), (2, 130, 64, 8, "shared"),
                                               (2, 77, 40, 3, "shared"), (1, 90, 48, 16, "channel"),
                                               (3, 65, 200, 5, "shared")])
def test_backward_bit_identical_across_runs(Bsz, L, D, N, layout):
    # dA (summed over batch and time) and the shared dB / dC (summed over
    # channels) are formed from per-workgroup partials in a fixed order: two
    # runs give the same bits. The per-channel layout covers dA alone.
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=21)
    dy = dy_for(Bsz, L, D, seed=21)
    kw = {}
    if layout == "channel":
        g = rng_for("bitid", Bsz, L, D, N)
        Bm = (g.standard_normal((Bsz, L, D, N)) * 0.25).astype(np.float32)
        Cm = (g.standard_normal((Bsz, L, D, N)) * 0.25).astype(np.float32)
        kw["bc_strides"] = (L * D * N, D * N, N)
    runs = [run_bwd(x, dt, A, Bm, Cm, dy, mode="recompute", **kw) for _ in range(2)]
    for n, a, b in zip(NAMES, runs[0], runs[1]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{n} differs between runs"


@pytest.mark.parametrize("wide", ["0", "1"])
@pytest.mark.parametrize("Bsz,L,D,N", [(2, 200, 48, 16), (1, 31, 17, 16), (2, 96, 200, 16),
                                       (3, 1, 32, 16), (1, 129, 33, 16)])
def test_shared_bc_n16_both_workgroup_widths(Bsz, L, D, N, wide, monkeypatch):
    # Shared B/C with N = 16 runs 8-wave workgroups on 16 channels, or, on
    # grids that give every CU one, 16-wave workgroups on 32
    # channels whose two halves add their dB / dC sums in LDS.
    # KM_SCAN1D_BWD_WIDE forces either: both match the oracle at these
    # sizes (D = 17, 33, 200 leave the second half of the last group partly
    # or wholly past D), in every mode, and repeat bit for bit.
    monkeypatch.setenv("KM_SCAN1D_BWD_WIDE", wide)
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=31)
    dy = dy_for(Bsz, L, D, seed=31)
    ref, hh = oracle_bwd(x, dt, A, Bm, Cm, dy)
    kap = scan1d_bwd_kappa(x, dt, A, Bm, Cm, dy)
    for mode in ("hist", "ckpt", "recompute"):
        got = run_bwd(x, dt, A, Bm, Cm, dy, mode=mode, hist=hh)
        check_all(got, ref, kap, TOL_F32, f"wide={wide} {mode}")
    again = run_bwd(x, dt, A, Bm, Cm, dy, mode="recompute")
    for n, a, b in zip(NAMES, got, again):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{n} differs between runs"


@pytest.mark.parametrize("wide", ["0", "1"])
def test_recompute_clamp_both_workgroup_widths(wide, monkeypatch):
    # The clamped re-run (states leaving [-1000, 1000]) with either
    # workgroup width: the halves' channel sums are flushed after the main
    # pass and after the re-run.
    monkeypatch.setenv("KM_SCAN1D_BWD_WIDE", wide)
    Bsz, L, D, N = 2, 200, 48, 16
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=14)
    Bm = Bm * 800.0
    A = A * 0.01
    dy = dy_for(Bsz, L, D)
    ref, hh = oracle_bwd(x, dt, A, Bm, Cm, dy)
    assert np.abs(hh).max() == 1000.0
    kap = scan1d_bwd_kappa(x, dt, A, Bm, Cm, dy)
    for mode in ("ckpt", "recompute"):
        got = run_bwd(x, dt, A, Bm, Cm, dy, mode=mode, hist=hh)
        check_all(got, ref, kap, TOL_F32, f"clamped wide={wide} {mode}")


def test_m1_shared_bc_ddelta_bit_identical_across_runs():
    # ddelta of the M = 1 entry point sums every channel's term per step:
    # per-workgroup partials added in workgroup order, identical run to run.
    L, D = 50, 700
    g = rng_for("m1bitid", L, D)
    x = g.standard_normal((L, D)).astype(np.float32)
    A = -g.uniform(0.1, 1.0, D).astype(np.float32)
    B = g.standard_normal(D).astype(np.float32)
    Cm = g.standard_normal(D).astype(np.float32)
    dt = g.uniform(0.01, 0.5, L).astype(np.float32)
    h = g.standard_normal((L, D)).astype(np.float32)
    dy = g.standard_normal((L, D)).astype(np.float32)
    outs = []
    for _ in range(2):
        dx, ddt = np.zeros((L, D), np.float32), np.zeros(L, np.float32)
        dA, dB, dC = (np.zeros(D, np.float32) for _ in range(3))
        p = K.ScanBackwardSharedParams(K.ptr(x), K.ptr(A), None, K.ptr(B), K.ptr(Cm), K.ptr(dt),
                                       None, K.ptr(h), K.ptr(dy), K.ptr(dx), K.ptr(dA), K.ptr(dB),
                                       K.ptr(dC), K.ptr(ddt), L, D)
        K.scan1d_backward_m1_shared_bc(C.byref(p))
        assert K.km_last_error() == ""
        outs.append(ddt)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("kind", ["avx2", "simple"])
@pytest.mark.parametrize("L,D,with_diag,use_h0,on_device",
                         [(6, 5, False, False, False), (16, 17, False, True, False),
                          (70, 300, True, False, True), (33, 1000, False, True, True)])
def test_m1_asm_entry_points_vs_oracle(kind, L, D, with_diag, use_h0, on_device):
    # scan1d_backward_m1_shared_bc_asm / _simple_asm: without A_diag the decay
    # is the routines' Taylor polynomial (checked against the oracle's
    # restatement of the assembly, which the CPU pins hold), with A_diag the
    # given decays. Host and device pointers.
    g = rng_for("m1asm", kind, L, D)
    x = g.uniform(-1, 1, (L, D)).astype(np.float32)
    A = g.uniform(-1.5, -0.05, D).astype(np.float32)
    B = g.uniform(-0.5, 0.5, D).astype(np.float32)
    Cm = g.uniform(-0.5, 0.5, D).astype(np.float32)
    dt = g.uniform(0.05, 0.8, L).astype(np.float32)
    dy = g.standard_normal((L, D)).astype(np.float32)
    h0 = g.uniform(-1, 1, D).astype(np.float32) if use_h0 else None
    e = np.exp(dt[:, None].astype(np.float64) * A[None, :])
    h = np.zeros((L, D))
    prev = np.zeros(D) if h0 is None else h0.astype(np.float64)
    for t in range(L):
        prev = e[t] * prev + B * dt[t] * x[t]
        h[t] = prev
    h = h.astype(np.float32)
    A_diag = np.exp(dt[:, None] * A[None, :]).astype(np.float32) if with_diag else None
    simple = kind == "simple"
    ref = O.scan1d_backward_m1_shared_bc_asm(x, A, B, Cm, dt, h, dy, A_diag=A_diag, h0=h0,
                                             simple=simple)
    fn = K.scan1d_backward_m1_shared_bc_simple_asm if simple else K.scan1d_backward_m1_shared_bc_asm
    ins = [x, A, A_diag, B, Cm, dt, h0, h, dy]
    outs = [np.full((L, D), np.nan, np.float32), np.full(D, np.nan, np.float32),
            np.full(D, np.nan, np.float32), np.full(D, np.nan, np.float32),
            np.full(L, np.nan, np.float32)]
    if on_device:
        dins = [None if a is None else torch.from_numpy(a).cuda() for a in ins]
        douts = [torch.from_numpy(a).cuda() for a in outs]
        p = K.ScanBackwardSharedParams(*(K.ptr(a) for a in dins), *(K.ptr(a) for a in douts), L, D)
        fn(C.byref(p))
        got = [a.cpu().numpy() for a in douts]
    else:
        p = K.ScanBackwardSharedParams(*(K.ptr(a) for a in ins), *(K.ptr(a) for a in outs), L, D)
        fn(C.byref(p))
        got = outs
    assert K.km_last_error() == ""
    ab = [np.abs(v) for v in (x, B, Cm, dy)]
    habs = np.zeros((L, D))
    prev = np.zeros(D) if h0 is None else np.abs(h0).astype(np.float64)
    for t in range(L):
        prev = e[t] * prev + ab[1] * dt[t] * ab[0][t]
        habs[t] = prev
    diag_abs = A_diag if with_diag else np.abs(O.m1_asm_taylor(dt[:, None] * A[None, :], simple))
    kap = O.scan1d_backward_m1_shared_bc_asm(ab[0], A, ab[1], ab[2], dt, habs.astype(np.float32),
                                             ab[3], A_diag=diag_abs,
                                             h0=None if h0 is None else np.abs(h0), simple=simple)
    t2 = (ab[0] * kap[0]).sum(axis=1) / dt
    kdd = np.maximum(2 * t2 - kap[4], 0)
    for n, gg, r, k in zip(("dx", "dA", "dB", "dC", "ddelta"), got, ref,
                           (kap[0], kap[1], kap[2], kap[3], kdd)):
        assert_close(gg, r, TOL_F32, f"m1 asm {kind} {n}", k)


@pytest.mark.parametrize("simple", [False, True])
def test_m1_asm_entry_points_edge_sizes_and_errors(simple):
    # L = 0 clears dA, dB, dC; D = 0 clears ddelta (as the routines do); a
    # missing output is an error that writes nothing.
    fn = K.scan1d_backward_m1_shared_bc_simple_asm if simple else K.scan1d_backward_m1_shared_bc_asm
    D, L = 7, 5
    dA, dB, dC = (np.full(D, 3.0, np.float32) for _ in range(3))
    p = K.ScanBackwardSharedParams()
    p.dA, p.dB, p.dC, p.L, p.D = K.ptr(dA), K.ptr(dB), K.ptr(dC), 0, D
    fn(C.byref(p))
    assert K.km_last_error() == ""
    assert not dA.any() and not dB.any() and not dC.any()
    dd = np.full(L, 3.0, np.float32)
    q = K.ScanBackwardSharedParams()
    q.ddelta, q.L, q.D = K.ptr(dd), L, 0
    fn(C.byref(q))
    assert K.km_last_error() == ""
    assert not dd.any()
    dd[:] = 3.0
    r = K.ScanBackwardSharedParams()
    r.L, r.D = L, D
    fn(C.byref(r))
    assert "invalid parameters" in K.km_last_error()

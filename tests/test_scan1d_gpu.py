"""GPU parity of the Scan1D forward kernels (libkmamba, gfx950) against the
CPU oracle on identical seeded inputs.

Tolerances: condition-scaled max relative error (tests/kmtest.py) <= 1e-4
for fp32 I/O and <= 2e-2 for bf16 I/O against the fp32 oracle of the
unrounded inputs; the 1e-3*rms floor metric is printed beside it.
"""
import ctypes as C

import numpy as np
import pytest

import kmamba as K
import oracle as O
from kmtest import (TOL_BF16, TOL_F32, assert_close, bf16_round, rel_err, rel_err_cond, rng_for,
                    scan1d_inputs, scan1d_kappa, silu_ref)

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    torch.zeros(1, device=DEV)
    assert K.kmamba_cuda_available() == 1, K.km_last_error()


def T(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


def run_km(x, dt, A, Bm, Cm, *, h0=None, hist=False, bc_strides=None, clamp=True, bf16=False,
           z=None, Dskip=None):
    Bsz, L, D = x.shape
    N = A.shape[1]
    io = torch.bfloat16 if bf16 else torch.float32
    tx, tdt, tB, tC = T(x, io), T(dt, io), T(Bm, io), T(Cm, io)
    tA = T(A)
    y = torch.empty((Bsz, L, D), device=DEV, dtype=io)
    th0 = None if h0 is None else T(h0)
    hf = torch.empty((Bsz, D, N), device=DEV)
    hh = torch.empty((Bsz, L, D, N), device=DEV) if hist else None
    tz = None if z is None else T(z, io)
    tD = None if Dskip is None else T(Dskip)
    K.scan1d_fwd(tx, tdt, tA, tB, tC, y, h0=th0, h_final=hf, h_hist=hh, bc_strides=bc_strides,
                 clamp=clamp, z=tz, Dskip=tD)
    torch.cuda.synchronize()
    return (y.float().cpu().numpy(), hf.cpu().numpy(), None if hh is None else hh.cpu().numpy())


def test_config0_fp32_parity():
    # Scan1D fwd fp32, B=1, L=128, D=384, N=16.
    x, dt, A, Bm, Cm = scan1d_inputs(1, 128, 384, 16, seed=0)
    yr, hr, _ = O.scan1d_batched(x, dt, A, Bm, Cm)
    assert np.abs(hr).max() < 1000          # clamp inactive on the config inputs
    y, hf, _ = run_km(x, dt, A, Bm, Cm)
    ky, kh, _ = scan1d_kappa(x, dt, A, Bm, Cm)
    e_y = assert_close(y, yr, TOL_F32, "y", ky)
    e_h = assert_close(hf, hr, TOL_F32, "h_final", kh)
    print(f"config0 fp32: cond rel err y {e_y:.2e} h {e_h:.2e}; floor metric y {rel_err(y, yr):.2e} "
          f"h {rel_err(hf, hr):.2e}")


SHAPES = [
    (2, 1, 32, 16), (1, 63, 33, 16), (3, 200, 70, 16), (2, 130, 64, 8), (1, 77, 100, 4),
    (2, 65, 64, 2), (1, 300, 65, 1), (2, 50, 40, 3), (1, 40, 20, 32), (1, 1000, 32, 16),
]


@pytest.mark.parametrize("Bsz,L,D,N", SHAPES)
@pytest.mark.parametrize("layout", ["shared", "per_channel"])
def test_shapes_layouts_h0_hist(Bsz, L, D, N, layout):
    x, dt, A, _, _ = scan1d_inputs(Bsz, L, D, N, seed=1)
    g = rng_for("shapes", Bsz, L, D, N)
    A = A * g.uniform(0.1, 1.0, size=A.shape).astype(np.float32)
    h0 = g.standard_normal((Bsz, D, N)).astype(np.float32)
    if layout == "shared":
        Bm = (g.standard_normal((Bsz, L, N)) * 0.25).astype(np.float32)
        Cm = (g.standard_normal((Bsz, L, N)) * 0.25).astype(np.float32)
        strides = (L * N, N, 0)
    else:
        Bm = (g.standard_normal((Bsz, L, D, N)) * 0.25).astype(np.float32)
        Cm = (g.standard_normal((Bsz, L, D, N)) * 0.25).astype(np.float32)
        strides = (L * D * N, D * N, N)
    yr, hr, hhr = O.scan1d_batched(x, dt, A, Bm, Cm, h0=h0, bc_strides=strides, hist=True)
    y, hf, hh = run_km(x, dt, A, Bm, Cm, h0=h0, hist=True, bc_strides=strides)
    ky, kh, khh = scan1d_kappa(x, dt, A, Bm, Cm, h0=h0, bc_strides=strides)
    assert_close(y, yr, TOL_F32, "y", ky)
    assert_close(hf, hr, TOL_F32, "h_final", kh)
    assert_close(hh, hhr, TOL_F32, "h_hist", khh)


def test_clamp_fallback_follows_per_step_clamp():
    # Large drive: states leave [-1000, 1000]; the kernel must reproduce the
    # reference's per-step clamp (cpu/scan1d.asm:136-140) exactly.
    Bsz, L, D, N = 2, 300, 64, 16
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=2)
    Bm = Bm * 800.0
    A = A * 0.01
    yr, hr, hhr = O.scan1d_batched(x, dt, A, Bm, Cm, hist=True)
    assert np.abs(hhr).max() == 1000.0
    y, hf, hh = run_km(x, dt, A, Bm, Cm, hist=True)
    ky, kh, khh = scan1d_kappa(x, dt, A, Bm, Cm)
    assert_close(y, yr, TOL_F32, "y", ky)
    assert_close(hf, hr, TOL_F32, "h_final", np.minimum(kh, 1000.0))
    assert np.abs(hh).max() == 1000.0
    # Without the clamp flag the states run free.
    y2, _, hh2 = run_km(x, dt, A, Bm, Cm, hist=True, clamp=False)
    yu, _, hhu = O.scan1d_batched(x, dt, A, Bm, Cm, hist=True, clamp=False)
    assert np.abs(hh2).max() > 1000.0
    assert_close(hh2, hhu, TOL_F32, "unclamped h", khh)


# Few (batch, 32-channel group) pairs and a long sequence with N = 16: the
# launcher splits the sequence into segments over workgroups (segment end
# states from a zero start, a fold over segments, a replay from the folded
# states); these shapes take the split under its cost model (4 to 64
# segments, 10 and 12 among them). D not a multiple of 32 leaves lanes
# without a channel; B > 1 exercises the [B*S, Ls, ...] view of the batch.
SPLIT = [(1, 1024, 64), (2, 1024, 40), (3, 1024, 100), (1, 4096, 32), (1, 640, 96), (2, 768, 200)]


@pytest.mark.parametrize("Bsz,L,D", SPLIT)
@pytest.mark.parametrize("layout", ["shared", "per_channel"])
def test_split_sequence_h0_hist(Bsz, L, D, layout):
    N = 16
    x, dt, A, _, _ = scan1d_inputs(Bsz, L, D, N, seed=11)
    g = rng_for("split", Bsz, L, D, N)
    h0 = g.standard_normal((Bsz, D, N)).astype(np.float32)
    if layout == "shared":
        Bm = (g.standard_normal((Bsz, L, N)) * 0.25).astype(np.float32)
        Cm = (g.standard_normal((Bsz, L, N)) * 0.25).astype(np.float32)
        strides = (L * N, N, 0)
    else:
        Bm = (g.standard_normal((Bsz, L, D, N)) * 0.25).astype(np.float32)
        Cm = (g.standard_normal((Bsz, L, D, N)) * 0.25).astype(np.float32)
        strides = (L * D * N, D * N, N)
    yr, hr, hhr = O.scan1d_batched(x, dt, A, Bm, Cm, h0=h0, bc_strides=strides, hist=True)
    ky, kh, khh = scan1d_kappa(x, dt, A, Bm, Cm, h0=h0, bc_strides=strides)
    # With and without the history store (different replay kernels).
    y, hf, hh = run_km(x, dt, A, Bm, Cm, h0=h0, hist=True, bc_strides=strides)
    assert_close(y, yr, TOL_F32, "y", ky)
    assert_close(hf, hr, TOL_F32, "h_final", kh)
    assert_close(hh, hhr, TOL_F32, "h_hist", khh)
    y2, hf2, _ = run_km(x, dt, A, Bm, Cm, h0=h0, bc_strides=strides)
    assert_close(y2, yr, TOL_F32, "y (no history)", ky)
    assert_close(hf2, hr, TOL_F32, "h_final (no history)", kh)


@pytest.mark.parametrize("Bsz,L,D", SPLIT[:3])
def test_split_sequence_bf16_gated(Bsz, L, D):
    N = 16
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=12)
    g = rng_for("split-gated", Bsz, L, D, N)
    z = (2.0 * g.standard_normal((Bsz, L, D))).astype(np.float32)
    Dsk = g.uniform(0.5, 1.5, D).astype(np.float32)
    xr, dtr, Br, Cr, zr = (bf16_round(a) for a in (x, dt, Bm, Cm, z))
    yr, hr, _ = O.scan1d_batched(xr, dtr, A, Br, Cr)
    ky, kh, _ = scan1d_kappa(xr, dtr, A, Br, Cr)
    sz = silu_ref(zr)
    ref, kap = (yr + Dsk * xr) * sz, (ky + np.abs(Dsk * xr)) * np.abs(sz)
    y, hf, _ = run_km(x, dt, A, Bm, Cm, bf16=True, z=z, Dskip=Dsk)
    assert rel_err_cond(y, bf16_round(ref), kap) < 1e-2
    assert_close(hf, hr, TOL_BF16, "h_final", kh)


def test_split_sequence_clamp_in_one_group_mid_sequence():
    # The drive leaves [-1000, 1000] only in steps 300..340 and only for the
    # first 32 channels (one channel group): that group's sequence is re-run
    # with the per-step clamp of cpu/scan1d.asm:136-140, the other group keeps
    # the split result, and both match the clamped reference.
    Bsz, L, D, N = 1, 1024, 64, 16
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=13)
    x[:, 300:340, :32] *= 4000.0
    yr, hr, hhr = O.scan1d_batched(x, dt, A, Bm, Cm, hist=True)
    assert np.abs(hhr[:, :, :32]).max() == 1000.0
    assert np.abs(hhr[:, :, 32:]).max() < 1000.0
    ky, kh, khh = scan1d_kappa(x, dt, A, Bm, Cm)
    for hist in (True, False):
        y, hf, hh = run_km(x, dt, A, Bm, Cm, hist=hist)
        assert_close(y, yr, TOL_F32, "y", ky)
        assert_close(hf, hr, TOL_F32, "h_final", np.minimum(kh, 1000.0))
        if hist:
            assert_close(hh, hhr, TOL_F32, "h_hist", np.minimum(khh, 1000.0))
    # Without the clamp the same drive runs free through the split path.
    yu, hu, _ = O.scan1d_batched(x, dt, A, Bm, Cm, clamp=False)
    y, hf, _ = run_km(x, dt, A, Bm, Cm, clamp=False)
    assert_close(y, yu, TOL_F32, "unclamped y", ky)
    assert_close(hf, hu, TOL_F32, "unclamped h_final", kh)


GATED = [(2, 1, 32, 16), (1, 63, 33, 16), (2, 131, 70, 16), (1, 77, 100, 8), (2, 65, 64, 4),
         (1, 200, 96, 2)]


@pytest.mark.parametrize("Bsz,L,D,N", GATED)
@pytest.mark.parametrize("bf16", [False, True], ids=["f32", "bf16"])
@pytest.mark.parametrize("parts", ["z+Dskip", "z", "Dskip"])
def test_gated_output(Bsz, L, D, N, bf16, parts):
    # y = (sum_n C*h + Dskip*x) * SiLU(z), the Mamba-1 output gating fused into
    # the store. Odd L leaves a step pair across the end of the sequence;
    # D not a multiple of 32 leaves lanes without a channel.
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=7)
    g = rng_for("gated", Bsz, L, D, N)
    z = (2.0 * g.standard_normal((Bsz, L, D))).astype(np.float32) if "z" in parts else None
    Dsk = g.uniform(0.5, 1.5, D).astype(np.float32) if "Dskip" in parts else None
    rnd = bf16_round if bf16 else (lambda a: a)
    xr, dtr, Br, Cr = rnd(x), rnd(dt), rnd(Bm), rnd(Cm)
    yr, hr, _ = O.scan1d_batched(xr, dtr, A, Br, Cr)
    ky, kh, _ = scan1d_kappa(xr, dtr, A, Br, Cr)
    ref, kap = yr.copy(), ky.copy()
    if Dsk is not None:
        ref = ref + Dsk * xr
        kap = kap + np.abs(Dsk * xr)
    if z is not None:
        sz = silu_ref(rnd(z))
        ref, kap = ref * sz, kap * np.abs(sz)
    y, hf, _ = run_km(x, dt, A, Bm, Cm, bf16=bf16, z=z, Dskip=Dsk)
    if bf16:
        assert rel_err_cond(y, bf16_round(ref), kap) < 1e-2
    else:
        assert_close(y, ref, TOL_F32, "gated y", kap)
    assert_close(hf, hr, TOL_BF16 if bf16 else TOL_F32, "h_final", kh)


def test_bf16_io_against_fp32_oracle():
    x, dt, A, Bm, Cm = scan1d_inputs(2, 512, 256, 16, seed=3)
    yr, hr, _ = O.scan1d_batched(x, dt, A, Bm, Cm)
    y, hf, _ = run_km(x, dt, A, Bm, Cm, bf16=True)
    ky, _, _ = scan1d_kappa(x, dt, A, Bm, Cm)
    e = assert_close(y, yr, TOL_BF16, "bf16 y", ky)
    # And tighter against the oracle run on the bf16-rounded inputs.
    yb, _, _ = O.scan1d_batched(*(bf16_round(a) for a in (x, dt)), A, bf16_round(Bm), bf16_round(Cm))
    assert rel_err_cond(y, bf16_round(yb), ky) < 1e-2
    print(f"bf16 y rel err vs fp32 oracle {e:.2e}")


def test_om_scan1d_forward_reference_api():
    # om_scan1d_forward: B, C, h are [L, D, M]; h receives the full history.
    L, D, M = 150, 40, 16
    x, A, B, Cm, dt = _api_inputs(L, D, M)
    yr, _, hhr = O.scan1d_batched(x[None], dt[None], A, B[None], Cm[None],
                                  bc_strides=(L * D * M, D * M, M), hist=True)
    tx, tA, tB, tC, tdt = map(T, (x, A, B, Cm, dt))
    y = torch.zeros((L, D), device=DEV)
    h = torch.zeros((L, D, M), device=DEV)
    K.om_scan1d_forward(K.ptr(tx), K.ptr(tA), K.ptr(tB), K.ptr(tC), K.ptr(tdt), K.ptr(y), K.ptr(h),
                        L, D, M)
    assert K.km_last_error() == ""
    ky, _, khh = scan1d_kappa(x[None], dt[None], A, B[None], Cm[None], bc_strides=(L * D * M, D * M, M))
    assert_close(y.cpu().numpy(), yr[0], TOL_F32, "y", ky[0])
    assert_close(h.cpu().numpy(), hhr[0], TOL_F32, "h history", khh[0])


def _api_inputs(L, D, M):
    g = rng_for("api", L, D, M)
    x = g.uniform(-1, 1, (L, D)).astype(np.float32)
    A = g.uniform(-1, -0.01, (D, M)).astype(np.float32)
    B = g.uniform(-0.5, 0.5, (L, D, M)).astype(np.float32)
    Cm = g.uniform(-0.5, 0.5, (L, D, M)).astype(np.float32)
    dt = g.uniform(0.01, 0.5, (L, D)).astype(np.float32)
    return x, A, B, Cm, dt


@pytest.mark.parametrize("L,D,M", [(4, 8, 1), (16, 16, 2), (64, 32, 1), (128, 48, 16),
                                   (2100, 1024, 16)])
def test_scan1d_host_pointer_api(L, D, M):
    # scan1d(ScanParams*) on host memory, running [D, M] state in/out. The
    # last shape's pageable buffers (x, y 8.6 MB; B, C 138 MB) go through the
    # library's pinned ring in several slot-sized pieces, the last ragged.
    x, A, B, Cm, dt = _api_inputs(L, D, M)
    h0 = rng_for("h0", L, D, M).uniform(-1, 1, (D, M)).astype(np.float32)
    yr, hr = O.scan1d(x, A, B, Cm, dt, h0)
    y = np.zeros((L, D), np.float32)
    h = h0.copy()
    p = K.ScanParams(K.ptr(x), K.ptr(A), K.ptr(B), K.ptr(Cm), K.ptr(dt), K.ptr(h), K.ptr(y), L, D, M)
    K.mamba_scan1d_forward(C.byref(p))
    assert K.km_last_error() == ""
    ky, kh, _ = scan1d_kappa(x[None], dt[None], A, B[None], Cm[None], h0=h0[None],
                             bc_strides=(L * D * M, D * M, M))
    assert_close(y, yr, TOL_F32, "y", ky[0])
    assert_close(h, hr, TOL_F32, "h", kh[0])


def test_scan1d_host_pointer_api_pinned_buffers():
    # The same entry point on page-locked host buffers (torch pin_memory):
    # those copy directly instead of through the library's pinned ring.
    L, D, M = 2100, 1024, 16
    x, A, B, Cm, dt = _api_inputs(L, D, M)
    h0 = rng_for("h0", L, D, M).uniform(-1, 1, (D, M)).astype(np.float32)
    yr, hr = O.scan1d(x, A, B, Cm, dt, h0)

    def pinned(a):
        t = torch.empty(a.shape, dtype=torch.float32, pin_memory=True)
        t.numpy()[...] = a
        return t

    px, pA, pB, pC, pdt, ph = (pinned(a) for a in (x, A, B, Cm, dt, h0))
    py = pinned(np.zeros((L, D), np.float32))
    p = K.ScanParams(*(t.data_ptr() for t in (px, pA, pB, pC, pdt, ph, py)), L, D, M)
    K.mamba_scan1d_forward(C.byref(p))
    assert K.km_last_error() == ""
    ky, kh, _ = scan1d_kappa(x[None], dt[None], A, B[None], Cm[None], h0=h0[None],
                             bc_strides=(L * D * M, D * M, M))
    assert_close(py.numpy(), yr, TOL_F32, "y", ky[0])
    assert_close(ph.numpy(), hr, TOL_F32, "h", kh[0])


def test_config1_full_size_sampled_parity():
    # configs[1] shape (B=8, L=4096, D=1024, N=16) on the GPU, checked against
    # the oracle on a sample of channels of the first and last batch element
    # (channels are independent, so the sample is an exact sub-problem).
    Bsz, L, D, N = 8, 4096, 1024, 16
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=0, tag="config1")
    y, hf, _ = run_km(x, dt, A, Bm, Cm)
    assert np.isfinite(y).all()
    sel = np.sort(rng_for("sel").choice(D, 48, replace=False))
    for b in (0, Bsz - 1):
        args = (x[b:b + 1][:, :, sel], dt[b:b + 1][:, :, sel], A[sel], Bm[b:b + 1], Cm[b:b + 1])
        yr, hr, _ = O.scan1d_batched(*args, nthreads=8, fast=True)
        ky, kh, _ = scan1d_kappa(*args)
        assert_close(y[b][:, sel], yr[0], TOL_F32, f"y[b={b}]", ky[0])
        assert_close(hf[b][sel], hr[0], TOL_F32, f"h[b={b}]", kh[0])


def test_config1_bf16_full_size_sampled_parity():
    # configs[1] with bf16 I/O (x, delta, B, C, y bf16; A and the state fp32)
    # at full size, B=8 L=4096 D=1024 N=16. Checked against the fp32 oracle of
    # the unrounded inputs at the bf16 tolerance on a sample of channels of
    # every batch element (channels are independent: an exact sub-problem).
    Bsz, L, D, N = 8, 4096, 1024, 16
    x, dt, A, Bm, Cm = scan1d_inputs(Bsz, L, D, N, seed=0, tag="config1")
    y, hf, _ = run_km(x, dt, A, Bm, Cm, bf16=True)
    assert np.isfinite(y).all() and np.isfinite(hf).all()
    sel = np.sort(rng_for("sel-bf16").choice(D, 24, replace=False))
    args = (x[:, :, sel], dt[:, :, sel], A[sel], Bm, Cm)
    yr, hr, _ = O.scan1d_batched(*args, nthreads=8, fast=True)
    ky, kh, _ = scan1d_kappa(*args)
    assert_close(y[:, :, sel], yr, TOL_BF16, "bf16 y", ky)
    assert_close(hf[:, sel], hr, TOL_BF16, "bf16 h_final", kh)

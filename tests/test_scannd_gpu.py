"""GPU parity of ScanND / Scan2D (libkmamba band kernels) against the oracle's
restatement of scannd_ref / scan2d on identical seeded inputs, through every
entry point of the reference API (om_scannd_forward, scannd_ref,
scannd_ref_with_plan, scannd, scan2d, mamba_scan2d_forward).

Tolerance: condition-scaled max relative error <= 1e-4 (tests/kmtest.py);
kappa is the same recurrence on |x|, |B|, |C| (positive decays).
"""
import ctypes as C

import numpy as np
import pytest

import kmamba as K
import oracle as O
from kmtest import TOL_F32, assert_close, rng_for

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available()
    torch.zeros(1, device=DEV)


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(DEV)


def nd_inputs(dims, D, M, seed, lo=-1.0, hi=-0.05):
    g = rng_for("nd-gpu", dims, D, M, seed)
    nd, P = len(dims), int(np.prod(dims))
    x = g.standard_normal((P, D)).astype(np.float32)
    A = g.uniform(lo, hi, (nd, D, M)).astype(np.float32)
    B = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    Cm = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    dt = g.uniform(0.05, 1.0, (nd, P, D)).astype(np.float32)
    return x, A, B, Cm, dt


def kappa(dims, x, A, B, Cm, dt):
    ya, ha = O.scannd_ref(dims, np.abs(x), A, np.abs(B), np.abs(Cm), dt, nthreads=8, fast=True)
    return ya, ha


def run_device(dims, x, A, B, Cm, dt, entry="km"):
    P = int(np.prod(dims))
    D, M = A.shape[1], A.shape[2]
    t = [T(a) for a in (x, A, B, Cm, dt)]
    h = torch.zeros((P, D, M), device=DEV)
    y = torch.zeros((P, D), device=DEV)
    if entry == "km":
        K.scannd_fwd(dims, t[0], t[1], t[2], t[3], t[4], h, y)
        torch.cuda.synchronize()
    else:
        p, keep = K.scannd_params(dims, t[0], t[1], t[2], t[3], t[4], h, y)
        fn = K.om_scannd_forward if entry == "om" else K.mamba_scannd_cuda_forward
        assert fn(C.byref(p)) == 0, K.km_last_error()
    return y.cpu().numpy(), h.cpu().numpy()


# Shapes on the tile kernels: 2D, 3D with the register ring (tiles of 4 rows
# along axis 1), 3D without it, 4D, ragged edges, several channel groups.
SCHED_CASES = [((64, 96), 64, 16), ((130, 70), 8, 8), ((9, 6, 11), 4, 16), ((7, 5, 10), 4, 16),
               ((5, 5, 5, 9), 4, 16), ((33, 65), 8, 16), ((40, 24, 24), 16, 16)]


@pytest.mark.parametrize("dims,D,M", SCHED_CASES)
def test_dataflow_and_band_schedules_agree(dims, D, M, monkeypatch):
    # The per-tile dataflow launch (on a device with 8 XCDs) and one launch
    # per tile band compute every state with the same arithmetic: h agrees
    # bit for bit, and so does y in 3+ dims, where both use the same tiles.
    # 2D uses rows of 4 points under the dataflow schedule and of 8 per band
    # launch, which changes the order of y's sum over the M states: y then
    # agrees with the oracle like the band schedule's.
    # Stable decays (configs[2]: a_k ~ U(0.05, 0.9/ndims), A = log a_k), so
    # every value stays finite on the larger grids.
    nd, P = len(dims), int(np.prod(dims))
    g = rng_for("nd-sched", dims, D, M)
    x = g.standard_normal((P, D)).astype(np.float32)
    A = np.log(g.uniform(0.05, 0.9 / nd, (nd, D, M))).astype(np.float32)
    B = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    Cm = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    dt = g.uniform(0.5, 1.0, (nd, P, D)).astype(np.float32)
    y1, h1 = run_device(dims, x, A, B, Cm, dt)
    monkeypatch.setenv("KM_SCANND_SCHED", "band")
    y2, h2 = run_device(dims, x, A, B, Cm, dt)
    assert np.isfinite(y1).all() and np.isfinite(h1).all()
    if nd > 2:
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    assert np.array_equal(h1.view(np.uint32), h2.view(np.uint32))
    yr, hr = O.scannd_ref(dims, x, A, B, Cm, dt, nthreads=8, fast=True)
    ya, ha = kappa(dims, x, A, B, Cm, dt)
    assert_close(y1, yr, TOL_F32, "y", ya)
    assert_close(y2, yr, TOL_F32, "y", ya)
    assert_close(h2, hr, TOL_F32, "h", ha)


PENCIL_CASES = [((9, 6, 11), 4, 16), ((7, 5, 10), 4, 16), ((40, 24, 24), 16, 16), ((13, 10, 17), 8, 8),
                ((5, 12, 9), 32, 4)]


@pytest.mark.parametrize("dims,D,M", PENCIL_CASES)
def test_pencil_and_tile_dataflow_agree(dims, D, M, monkeypatch):
    # Under the dataflow schedule 3D ring tiles run as pencils along axis 0
    # (flags per 4 planes, the axis-0 neighbour carried in registers) or,
    # with KM_SCANND_PENCIL=0, as separate tiles reading it back from h: the
    # same arithmetic, so h and y agree bit for bit. Covers partial last
    # sub-tiles (9, 7, 13, 5 planes), rows past a tile's edge and M < 16.
    x, A, B, Cm, dt = _stable_nd_inputs(dims, D, M, "nd-pencil")
    y1, h1 = run_device(dims, x, A, B, Cm, dt)
    monkeypatch.setenv("KM_SCANND_PENCIL", "0")
    y2, h2 = run_device(dims, x, A, B, Cm, dt)
    assert np.isfinite(y1).all() and np.isfinite(h1).all()
    assert np.array_equal(h1.view(np.uint32), h2.view(np.uint32))
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    yr, hr = O.scannd_ref(dims, x, A, B, Cm, dt, nthreads=8, fast=True)
    ya, ha = kappa(dims, x, A, B, Cm, dt)
    assert_close(y1, yr, TOL_F32, "y", ya)
    assert_close(h1, hr, TOL_F32, "h", ha)


def _stable_nd_inputs(dims, D, M, tag):
    nd, P = len(dims), int(np.prod(dims))
    g = rng_for(tag, dims, D, M)
    x = g.standard_normal((P, D)).astype(np.float32)
    A = np.log(g.uniform(0.05, 0.9 / nd, (nd, D, M))).astype(np.float32)
    B = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    Cm = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    dt = g.uniform(0.5, 1.0, (nd, P, D)).astype(np.float32)
    return x, A, B, Cm, dt


_BUDGET0 = r"""
import ctypes as C, sys
import numpy as np, torch
sys.path[:0] = [sys.argv[2], sys.argv[3]]
import kmamba as K
d = np.load(sys.argv[1])
dims = tuple(int(v) for v in d["dims"])
t = [torch.from_numpy(d[k]).cuda() for k in ("x", "A", "B", "C", "dt")]
P, D, M = int(np.prod(dims)), t[1].shape[1], t[1].shape[2]
out = {}
# Asynchronous entry point: every dataflow wait gives up at once.
h = torch.zeros((P, D, M), device="cuda"); y = torch.zeros((P, D), device="cuda")
K.scannd_fwd(dims, *t, h, y)
out["status_async"] = np.int64(K.scannd_status())
torch.cuda.synchronize()
out["y_async"] = y.cpu().numpy()
# The allocation-free entry point reports the same way.
h = torch.zeros((P, D, M), device="cuda"); y = torch.zeros((P, D), device="cuda")
K.scannd_fwd_noalloc(dims, *t, h, y)
out["status_noalloc"] = np.int64(K.scannd_status())
# Synchronous entry point: the same failure, then the band schedule.
h = torch.zeros((P, D, M), device="cuda"); y = torch.zeros((P, D), device="cuda")
p, keep = K.scannd_params(dims, *t, h, y)
rc = K.om_scannd_forward(C.byref(p))
out["status_sync"] = np.int64(K.scannd_status())
out["rc"] = np.int64(rc); out["y_sync"] = y.cpu().numpy(); out["h_sync"] = h.cpu().numpy()
np.savez(sys.argv[4], **out)
print("budget0 done", flush=True)
"""


def test_dataflow_wait_budget_exhausted_fails_loudly_and_sync_api_recovers(tmp_path):
    # KM_SCANND_FLOW_SPIN=0 (read once per process, so a child process) makes
    # every dataflow wait give up without polling; every kernel still exits
    # normally. The waves then write NaN into their tiles instead of
    # computing, so the asynchronous km_scannd_fwd returns NaN wherever a
    # tile had a predecessor (never a silently wrong value), and the
    # synchronous om_scannd_forward sees the status word and re-runs the
    # call on the band schedule: exact result.
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    dims, D, M = (9, 6, 11), 4, 16
    x, A, B, Cm, dt = _stable_nd_inputs(dims, D, M, "nd-budget0")
    src, dst = tmp_path / "in.npz", tmp_path / "out.npz"
    np.savez(src, dims=np.array(dims), x=x, A=A, B=B, C=Cm, dt=dt)
    env = dict(__import__("os").environ, KM_SCANND_FLOW_SPIN="0")
    r = subprocess.run([sys.executable, "-c", _BUDGET0, str(src), str(root / "k-mamba_amd"),
                        str(root / "oracle"), str(dst)], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    out = np.load(dst)
    yr, hr = O.scannd_ref(dims, x, A, B, Cm, dt, nthreads=8, fast=True)
    ya, ha = kappa(dims, x, A, B, Cm, dt)
    assert int(out["rc"]) == 0
    # km_scannd_status: the failed asynchronous calls report 1; the latest
    # launch of the synchronous call (its band re-run) is exact.
    assert int(out["status_async"]) == 1 and int(out["status_noalloc"]) == 1
    assert int(out["status_sync"]) == 0
    assert_close(out["y_sync"], yr, TOL_F32, "y after re-run", ya)
    assert_close(out["h_sync"], hr, TOL_F32, "h after re-run", ha)
    ya_ = out["y_async"].reshape(dims + (D,))
    assert np.isnan(ya_).any(), "a failed wait must not leave finite outputs behind"
    assert np.isfinite(ya_[0, 0, 0]).all()           # the first tile has no predecessor
    assert np.isnan(ya_[-1, -1, -1]).all()           # the last one depends on everything
    fin = np.isfinite(out["y_async"])
    np.testing.assert_allclose(out["y_async"][fin], yr[fin], rtol=0, atol=1e-4 * float(np.abs(ya).max()))


def test_dataflow_on_two_streams_concurrently():
    # Each (device, stream) pair has its own dataflow flags and counters:
    # launches on two streams back to back, with no synchronisation between
    # them, both match the oracle. km_release_stream then frees the two
    # streams' blocks.
    dims, D, M = (40, 24, 24), 16, 16
    P = int(np.prod(dims))
    sets = [_stable_nd_inputs(dims, D, M, f"nd-streams{i}") for i in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = []
    for arrs in sets:
        t = [T(a) for a in arrs]
        outs.append((t, torch.zeros((P, D, M), device=DEV), torch.zeros((P, D), device=DEV)))
    torch.cuda.synchronize()
    for rep in range(3):
        for (t, h, y), st in zip(outs, streams):
            K.scannd_fwd(dims, *t, h, y, stream=st)
    torch.cuda.synchronize()
    assert [K.scannd_status(st) for st in streams] == [0, 0]
    for arrs, (t, h, y) in zip(sets, outs):
        yr, hr = O.scannd_ref(dims, *arrs, nthreads=8, fast=True)
        ya, ha = kappa(dims, *arrs)
        assert_close(y.cpu().numpy(), yr, TOL_F32, "y", ya)
        assert_close(h.cpu().numpy(), hr, TOL_F32, "h", ha)
    held = K.km_device_bytes_held()
    freed = sum(K.km_release_stream(C.c_void_p(st.cuda_stream)) for st in streams)
    assert freed > 0 and K.km_device_bytes_held() == held - freed


def test_known_answers_all_entry_points():
    # tests/unit/test_scan_nd.c:41-141.
    for dims, A, want in (((2, 2), [np.log(2.0), np.log(3.0)], [1, 4, 3, 18]),
                          ((2, 2, 2), [0.0, 0.0, 0.0], [1, 2, 2, 5, 2, 5, 5, 16])):
        nd, P = len(dims), int(np.prod(dims))
        Aa = np.array(A, np.float32).reshape(nd, 1, 1)
        ones = np.ones((P, 1), np.float32)
        dt = np.ones((nd, P, 1), np.float32)
        for entry in ("km", "om", "mamba"):
            y, _ = run_device(dims, ones, Aa, ones[:, :, None], ones[:, :, None], dt, entry)
            np.testing.assert_allclose(y[:, 0], want, rtol=1e-5, err_msg=entry)
        # Host-pointer API: scannd_ref, scannd_ref_with_plan, scannd (dispatch).
        for fn in ("ref", "plan", "dispatch"):
            h = np.zeros((P, 1, 1), np.float32)
            y = np.zeros((P, 1), np.float32)
            B = np.ones((P, 1, 1), np.float32)
            p, keep = K.scannd_params(dims, ones, Aa, B, B, dt, h, y)
            if fn == "ref":
                rc = K.scannd_ref(C.byref(p))
            elif fn == "plan":
                plan = K.km_wavefront_plan_create(K.longs(dims), nd)
                rc = K.scannd_ref_with_plan(C.byref(p), plan)
                K.km_wavefront_plan_free(plan)
            else:
                rc = K.scannd(C.byref(p))
            assert rc == 0, (fn, K.km_last_error())
            np.testing.assert_allclose(y[:, 0], want, rtol=1e-5, err_msg=fn)


CASES = [((7, 5), 3, 4), ((40, 70), 4, 16), ((33, 65), 8, 16), ((1, 90), 4, 16), ((90, 1), 4, 16),
         ((5, 18, 20), 4, 16), ((3, 4, 5, 6), 4, 16), ((6, 7, 9), 3, 3), ((17, 33), 2, 32),
         ((100,), 4, 16), ((64, 64), 64, 1),
         # ragged tiles with a single row per plane and length-1 row axes
         # (the default 3D / 4D tiles are 4 per leading axis, 2D rows 6):
         ((7, 5, 10), 4, 16), ((5, 1, 9), 4, 16), ((10, 9, 13), 4, 16), ((5, 5, 5, 9), 4, 16),
         ((3, 1, 4, 5), 4, 16), ((13, 25), 4, 16), ((2, 1, 1, 6), 4, 16),
         # 3D tiles of 4 rows along axis 1 (previous plane kept in registers),
         # ragged along every axis:
         ((9, 6, 11), 4, 16), ((6, 4, 17), 8, 8)]


@pytest.mark.parametrize("dims,D,M", CASES)
def test_random_shapes_vs_oracle(dims, D, M):
    x, A, B, Cm, dt = nd_inputs(dims, D, M, 0)
    yr, hr = O.scannd_ref(dims, x, A, B, Cm, dt, nthreads=8, fast=True)
    y, h = run_device(dims, x, A, B, Cm, dt)
    ya, ha = kappa(dims, x, A, B, Cm, dt)
    assert_close(y, yr, TOL_F32, "y", ya)
    assert_close(h, hr, TOL_F32, "h", ha)


def test_plan_mismatch_rejected():
    dims = (4, 4)
    x, A, B, Cm, dt = nd_inputs(dims, 4, 16, 1)
    h = np.zeros_like(B)
    y = np.zeros_like(x)
    p, keep = K.scannd_params(dims, x, A, B, Cm, dt, h, y)
    plan = K.km_wavefront_plan_create(K.longs((4, 5)), 2)
    assert K.scannd_ref_with_plan(C.byref(p), plan) == -1
    K.km_wavefront_plan_free(plan)
    # theta without lambda changes nothing (the rotation belongs to the
    # Mamba-3 lambda branch, src/scan_nd.c:59-72).
    assert K.scannd_ref(C.byref(p)) == 0, K.km_last_error()
    y0, h0 = y.copy(), h.copy()
    theta = np.full((2,), 0.7, np.float32)
    p.theta = theta.ctypes.data
    assert K.scannd_ref(C.byref(p)) == 0, K.km_last_error()
    np.testing.assert_array_equal(y, y0)
    np.testing.assert_array_equal(h, h0)


@pytest.mark.parametrize("d1,d2,D,M", [(7, 5, 3, 4), (40, 33, 4, 16), (1, 1, 4, 16)])
def test_scan2d_host_api_vs_oracle_scan2d(d1, d2, D, M):
    x, A, B, Cm, dt = nd_inputs((d1, d2), D, M, 2)
    yr, hr = O.scan2d(x, A[0], A[1], B, Cm, dt[0], dt[1], d1, d2)
    h = np.zeros((d1 * d2, D, M), np.float32)
    y = np.zeros((d1 * d2, D), np.float32)
    arrs = [np.ascontiguousarray(a) for a in (x, A[0], A[1], B, Cm, dt[0], dt[1])]
    p = K.Scan2DParams(*[K.ptr(a) for a in arrs], K.ptr(h), K.ptr(y), d1, d2, D, M)
    K.mamba_scan2d_forward(C.byref(p))
    assert K.km_last_error() == ""
    ya, ha = kappa((d1, d2), x, A, B, Cm, dt)
    assert_close(y, yr, TOL_F32, "y", ya)
    assert_close(h, hr, TOL_F32, "h", ha)


def test_scannd_dispatch_1d_is_scan1d_with_running_state():
    # scannd() with ndims == 1 follows scan1d: h is a running [D, M] state
    # (src/scan_nd.c:266-281) and the +-1000 clamp applies.
    L, D, M = 50, 4, 16
    x, A, B, Cm, dt = nd_inputs((L,), D, M, 3)
    h0 = rng_for("h0nd").uniform(-1, 1, (D, M)).astype(np.float32)
    yr, hr = O.scannd((L,), x, A, B, Cm, dt, h=np.concatenate([h0[None], np.zeros((L - 1, D, M))]))
    h = np.zeros((L, D, M), np.float32)
    h[0] = h0
    y = np.zeros((L, D), np.float32)
    p, keep = K.scannd_params((L,), x, A, B, Cm, dt, h, y)
    assert K.scannd(C.byref(p)) == 0, K.km_last_error()
    np.testing.assert_allclose(y, yr, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(h[0], hr[0], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("dims,D,M", [((256, 256), 256, 16), ((64, 64, 64), 128, 16)])
def test_config2_full_size_sampled(dims, D, M):
    # configs[2] on the GPU; one channel of every channel group (64 (d, m)
    # lanes: 64 // M channels) checked elementwise against the oracle at
    # every point (channels are independent). Every group, and so every
    # wave's lane set and, on the 3D dataflow schedule, every XCD's queue
    # of groups, is compared. Inputs per BASELINE: delta = 1, decay
    # a_k ~ U(0.05, 0.9/ndims) as A = log(a_k), B, C ~ N(0, 1/16), x ~ N(0, 1).
    nd, P = len(dims), int(np.prod(dims))
    per = 64 // M
    g = rng_for("config2", dims)
    x = g.standard_normal((P, D), dtype=np.float32)
    A = np.log(g.uniform(0.05, 0.9 / nd, (nd, D, M))).astype(np.float32)
    B = (g.standard_normal((P, D, M), dtype=np.float32) * 0.25).astype(np.float32)
    Cm = (g.standard_normal((P, D, M), dtype=np.float32) * 0.25).astype(np.float32)
    dt = np.ones((nd, P, D), np.float32)
    y, h = run_device(dims, x, A, B, Cm, dt)
    assert np.isfinite(y).all()
    ngroups = D * M // 64
    sel = np.arange(ngroups) * per + g.integers(0, per, ngroups)
    assert len(np.unique(sel // per)) == ngroups
    args = (x[:, sel], A[:, sel], B[:, sel], Cm[:, sel], dt[:, :, sel])
    yr, hr = O.scannd_ref(dims, *args, nthreads=8, fast=True)
    ya, ha = kappa(dims, *args)
    assert_close(y[:, sel], yr, TOL_F32, "y", ya)
    assert_close(h[:, sel], hr, TOL_F32, "h", ha)


# ---------------------------------------------------------------------------
# ScanND backward (km_scannd_bwd; the oracle's adjoint is pinned in
# test_oracle_pins.py by float64 finite differences and by the reference's
# scan1d_backward in 1D). Metric: normwise per output, max |got - ref| /
# max |ref| <= 1e-4 (fp32; dA and ddelta are sums of signed terms).
# ---------------------------------------------------------------------------
BWD_CASES = [((50,), 8, 4), ((17, 23), 8, 16), ((64, 64), 32, 16), ((5, 6, 7), 4, 8),
             ((3, 2, 3, 2, 2), 2, 16),     # ndims * M = 80: the shuffle path needs no LDS
             ((16, 16, 16), 16, 16), ((3, 4, 2, 5), 3, 5), ((9, 11), 5, 32), ((256, 256), 16, 16),
             ((64, 64, 64), 8, 16),
             # The tiled paths (D*M a multiple of 64) on grids ragged in every
             # axis, with each lane-sum width of the gradient tiles.
             ((6, 13, 19), 4, 16), ((19, 70), 2, 32), ((10, 33), 8, 8), ((7, 9, 12), 16, 4),
             ((5, 130), 1, 64), ((9, 10, 11), 64, 1)]


def bwd_inputs(dims, D, M, seed):
    # Decays whose sum over the axes stays <= 0.9 (A = log U(0.05, 0.9/nd),
    # delta in [1, 2]), as the configs[2] inputs: the adjoint, like the
    # forward, sums over every lattice path and overflows fp32 on large grids
    # when that sum nears 1.
    x, A, B, Cm, dt = nd_inputs(dims, D, M, seed)
    g = rng_for("ndbwd", dims, D, M, seed)
    nd = len(dims)
    A = np.log(g.uniform(0.05, 0.9 / nd, A.shape)).astype(np.float32)
    dt = g.uniform(1.0, 2.0, dt.shape).astype(np.float32)
    dy = g.standard_normal((int(np.prod(dims)), D)).astype(np.float32)
    _, h = O.scannd_ref(dims, x, A, B, Cm, dt, nthreads=8, fast=True)
    return x, A, B, Cm, dt, h, dy


def run_bwd(dims, x, A, B, Cm, dt, h, dy):
    Pn, D = x.shape
    nd, _, M = A.shape
    out = {"dx": torch.full((Pn, D), float("nan"), device="cuda"),
           "ddelta": torch.full((nd, Pn, D), float("nan"), device="cuda"),
           "dA": torch.full((nd, D, M), float("nan"), device="cuda"),
           "dB": torch.full((Pn, D, M), float("nan"), device="cuda"),
           "dC": torch.full((Pn, D, M), float("nan"), device="cuda")}
    K.scannd_bwd(dims, T(x), T(A), T(B), T(Cm), T(dt), T(h), T(dy), out["dx"], out["ddelta"],
                 out["dA"], out["dB"], out["dC"])
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


@pytest.mark.parametrize("dims,D,M", BWD_CASES)
def test_backward_vs_oracle(dims, D, M):
    x, A, B, Cm, dt, h, dy = bwd_inputs(dims, D, M, 0)
    want = O.scannd_backward(dims, x, A, B, Cm, dt, h, dy, fast=True)
    got = run_bwd(dims, x, A, B, Cm, dt, h, dy)
    for k in want:
        assert np.isfinite(got[k]).all(), k
        err = np.abs(got[k] - want[k]).max() / max(np.abs(want[k]).max(), 1e-30)
        assert err <= 1e-4, f"{k}: normwise error {err:.2e}"


@pytest.mark.parametrize("dims,D,M", [((33, 65), 8, 16), ((64, 96), 4, 16), ((9, 6, 11), 4, 16),
                                      ((40, 24, 24), 16, 16), ((7, 13, 17), 8, 8)])
def test_backward_dataflow_and_band_schedules_agree(dims, D, M, monkeypatch):
    # The adjoint sweep on the dataflow schedule (one launch, tiles waiting
    # on their successors) and one launch per tile band compute every state
    # with the same arithmetic: every gradient agrees bit for bit, and the
    # band schedule matches the oracle.
    x, A, B, Cm, dt, h, dy = bwd_inputs(dims, D, M, 3)
    a = run_bwd(dims, x, A, B, Cm, dt, h, dy)
    monkeypatch.setenv("KM_SCANND_SCHED", "band")
    b = run_bwd(dims, x, A, B, Cm, dt, h, dy)
    for k in a:
        assert np.isfinite(a[k]).all(), k
        assert np.array_equal(a[k].view(np.uint32), b[k].view(np.uint32)), k
    want = O.scannd_backward(dims, x, A, B, Cm, dt, h, dy, fast=True)
    for k in want:
        err = np.abs(b[k] - want[k]).max() / max(np.abs(want[k]).max(), 1e-30)
        assert err <= 1e-4, f"{k}: normwise error {err:.2e}"


FUSED_CASES = [((43, 37), 128, 16), ((17, 70), 256, 8), ((9, 5), 512, 4), ((25, 30), 64, 32),
               ((64, 64), 128, 16),
               ((9, 10, 11), 128, 16), ((13, 6, 7), 256, 8), ((6, 9, 5), 64, 32), ((20, 16, 16), 128, 16),
               ((5, 4, 4), 128, 16)]


@pytest.mark.parametrize("dims,D,M", FUSED_CASES)
def test_backward_fused_2d_matches_two_pass(dims, D, M, monkeypatch):
    # Grids whose channel groups fill workgroups of four per XCD (D*M a
    # multiple of 2048) run the fused backward: the adjoint state and every
    # gradient in one dataflow launch (2D pencils of 4 columns through every
    # row in sub-tiles of 8 rows; 3D pencils of 4 x 4 columns through every
    # plane in sub-tiles of 2 planes), only the boundary states stored.
    # KM_SCANND_BWD_FUSED=0 runs the adjoint sweep, then the gradient pass:
    # the same arithmetic at every point, so dx, ddelta, dB and dC agree bit
    # for bit; dA adds its terms per pencil and agrees to rounding. Covers partial tiles, pencils and sub-tiles on every axis,
    # M = 4 to 32 (3D: 8 to 32).
    x, A, B, Cm, dt, h, dy = bwd_inputs(dims, D, M, 5)
    a = run_bwd(dims, x, A, B, Cm, dt, h, dy)
    monkeypatch.setenv("KM_SCANND_BWD_FUSED", "0")
    b = run_bwd(dims, x, A, B, Cm, dt, h, dy)
    for k in ("dx", "ddelta", "dB", "dC"):
        assert np.isfinite(a[k]).all(), k
        assert np.array_equal(a[k].view(np.uint32), b[k].view(np.uint32)), k
    np.testing.assert_allclose(a["dA"], b["dA"], rtol=1e-5, atol=1e-6 * float(np.abs(b["dA"]).max()))
    want = O.scannd_backward(dims, x, A, B, Cm, dt, h, dy, fast=True)
    for k in want:
        err = np.abs(a[k] - want[k]).max() / max(np.abs(want[k]).max(), 1e-30)
        assert err <= 1e-4, f"{k}: normwise error {err:.2e}"


_BWD_BUDGET0 = r"""
import sys
import numpy as np, torch
sys.path[:0] = [sys.argv[2], sys.argv[3]]
import kmamba as K
d = np.load(sys.argv[1])
dims = tuple(int(v) for v in d["dims"])
t = [torch.from_numpy(d[k]).cuda() for k in ("x", "A", "B", "C", "dt", "h", "dy")]
P, D = t[0].shape
nd, _, M = t[1].shape
outs = [torch.zeros(s, device="cuda") for s in ((P, D), (nd, P, D), (nd, D, M), (P, D, M), (P, D, M))]
K.scannd_bwd(dims, *t, *outs)
res = {"status": np.int64(K.scannd_status())}
for k, v in zip(("dx", "ddelta", "dA", "dB", "dC"), outs):
    res[k] = v.cpu().numpy()
np.savez(sys.argv[4], **res)
print("bwd budget0 done", flush=True)
"""


@pytest.mark.parametrize("dims,D,M", [((33, 65), 8, 16), ((9, 6, 11), 4, 16), ((43, 37), 128, 16),
                                      ((9, 10, 11), 128, 16)])
def test_backward_dataflow_wait_budget_exhausted_fails_loudly(dims, D, M, tmp_path):
    # KM_SCANND_FLOW_SPIN=0 (read once per process, so a child process):
    # every wait of the adjoint sweep gives up without polling, every kernel
    # still exits normally. A tile that had a successor writes NaN instead of
    # its states, so its gradients are NaN (never silently wrong), and
    # km_scannd_status reports the failed wait. The last tile, which has no
    # successor, is exact.
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    x, A, B, Cm, dt, h, dy = bwd_inputs(dims, D, M, 4)
    src, dst = tmp_path / "in.npz", tmp_path / "out.npz"
    np.savez(src, dims=np.array(dims), x=x, A=A, B=B, C=Cm, dt=dt, h=h, dy=dy)
    env = dict(__import__("os").environ, KM_SCANND_FLOW_SPIN="0")
    r = subprocess.run([sys.executable, "-c", _BWD_BUDGET0, str(src), str(root / "k-mamba_amd"),
                        str(root / "oracle"), str(dst)], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    out = np.load(dst)
    assert int(out["status"]) == 1
    # dB = g * mean(delta) * x carries the adjoint state g (dC = dy * h does not).
    dB = out["dB"].reshape(dims + (D, M))
    assert np.isnan(dB).any(), "a failed wait must not leave finite gradients behind"
    assert np.isnan(dB[(0,) * len(dims)]).all()      # the first point depends on every other
    assert np.isnan(out["dx"]).any()
    want = O.scannd_backward(dims, x, A, B, Cm, dt, h, dy, fast=True)
    last = (-1,) * len(dims)
    np.testing.assert_allclose(dB[last], want["dB"].reshape(dims + (D, M))[last], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dims,D,M", [((33, 40), 8, 16), ((24, 20), 128, 16), ((7, 9, 10), 128, 16)])
def test_backward_deterministic_and_workspace(dims, D, M):
    x, A, B, Cm, dt, h, dy = bwd_inputs(dims, D, M, 1)
    a = run_bwd(dims, x, A, B, Cm, dt, h, dy)
    b = run_bwd(dims, x, A, B, Cm, dt, h, dy)
    for k in a:
        assert np.array_equal(a[k].view(np.uint32), b[k].view(np.uint32)), k
    # An explicit workspace of the queried size gives the same result.
    nd = len(dims)
    args = K.KMScanNDBwd(K.longs(dims), nd, D, M)
    need = K.km_scannd_bwd_workspace_bytes(C.byref(args))
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    Pn = int(np.prod(dims))
    out = [torch.empty(s, device="cuda") for s in ((Pn, D), (nd, Pn, D), (nd, D, M), (Pn, D, M), (Pn, D, M))]
    K.scannd_bwd(dims, T(x), T(A), T(B), T(Cm), T(dt), T(h), T(dy), *out, workspace=ws)
    torch.cuda.synchronize()
    for k, t in zip(("dx", "ddelta", "dA", "dB", "dC"), out):
        assert np.array_equal(t.cpu().numpy().view(np.uint32), a[k].view(np.uint32)), k
    small = torch.empty(need - 256, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="workspace"):
        K.scannd_bwd(dims, T(x), T(A), T(B), T(Cm), T(dt), T(h), T(dy), *out, workspace=small)


def test_backward_rejects_invalid():
    dims, D, M = (4, 4), 2, 33                 # M not a power of two and ndims * M = 66 > 64
    args = K.KMScanNDBwd(K.longs(dims), 2, D, M)
    assert K.km_scannd_bwd_workspace_bytes(C.byref(args)) == 0
    assert "exceeds" in K.km_last_error()
    assert K.km_scannd_bwd_c(C.byref(args), None) == -1
    args = K.KMScanNDBwd(K.longs((4, 0)), 2, 2, 4)
    assert K.km_scannd_bwd_c(C.byref(args), None) == -1


@pytest.mark.parametrize("dims,D,M", [((256, 256), 256, 16), ((64, 64, 64), 128, 16)])
def test_backward_full_size_adjoint_identities(dims, D, M):
    # configs[2] sizes, checked through what the recurrence fixes at any
    # size: y is linear in x, in B and in C separately (h is linear in B x),
    # so sum dx.x = sum dB.B = sum dC.C = sum dy.y exactly in real
    # arithmetic. The forward's y and h come from km_scannd_fwd.
    nd = len(dims)
    Pn = int(np.prod(dims))
    g = torch.Generator(device="cuda").manual_seed(21)
    x = torch.randn((Pn, D), device="cuda", generator=g)
    A = torch.log(0.05 + (0.9 / nd - 0.05) * torch.rand((nd, D, M), device="cuda", generator=g))
    B = torch.randn((Pn, D, M), device="cuda", generator=g) * 0.25
    Cm = torch.randn((Pn, D, M), device="cuda", generator=g) * 0.25
    dt = 1.0 + torch.rand((nd, Pn, D), device="cuda", generator=g)
    h = torch.empty((Pn, D, M), device="cuda")
    y = torch.empty((Pn, D), device="cuda")
    K.scannd_fwd(dims, x, A, B, Cm, dt, h, y)
    dy = torch.randn((Pn, D), device="cuda", generator=g)
    dx, ddt = torch.empty_like(x), torch.empty_like(dt)
    dA, dB, dC = torch.empty_like(A), torch.empty_like(B), torch.empty_like(Cm)
    K.scannd_bwd(dims, x, A, B, Cm, dt, h, dy, dx, ddt, dA, dB, dC)
    torch.cuda.synchronize()
    ref = (dy.double() * y.double()).sum().item()
    scale = (dy.double().abs() * y.double().abs()).sum().item()
    for name, grad, val in (("dx", dx, x), ("dB", dB, B), ("dC", dC, Cm)):
        assert torch.isfinite(grad).all(), name
        got = (grad.double() * val.double()).sum().item()
        assert abs(got - ref) <= 1e-5 * scale, f"{name}: <grad, input> {got:.6e} vs <dy, y> {ref:.6e}"
    for t in (dA, ddt):
        assert torch.isfinite(t).all()

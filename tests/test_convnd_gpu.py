"""GPU parity of ConvND forward / backward (libkmamba, gfx950) against the
CPU oracle's restatement of src/convnd.c on identical seeded inputs.

Metric: condition-scaled max relative error (tests/kmtest.py) <= 1e-4 with
kappa = the same convolution on absolute values (no cancellation).
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
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    torch.zeros(1, device=DEV)
    assert K.kmamba_cuda_available() == 1, K.km_last_error()


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, torch.float32)


def conv_inputs(dims, D, Kk, seed=0, bias=True):
    g = rng_for("conv", dims, D, Kk, seed)
    Pn = int(np.prod(dims))
    KV = Kk ** len(dims)
    inp = g.standard_normal((Pn, D)).astype(np.float32)
    ker = (g.standard_normal((KV, D)) / np.sqrt(KV)).astype(np.float32)
    b = (g.standard_normal(D) * 0.1).astype(np.float32) if bias else None
    dy = g.standard_normal((Pn, D)).astype(np.float32)
    return inp, ker, b, dy


def fwd_kappa(dims, inp, ker, b):
    return O.convnd_forward(dims, np.abs(inp), np.abs(ker), None if b is None else np.abs(b),
                            nthreads=8, fast=True)


def bwd_kappa(dims, inp, ker, dy, with_bias):
    return O.convnd_backward(dims, np.abs(inp), np.abs(ker), np.abs(dy), with_bias=with_bias)


def gpu_fwd(dims, inp, ker, b):
    out = torch.full(inp.shape, float("nan"), device=DEV)
    K.convnd_fwd(dims, T(inp), T(ker), None if b is None else T(b), out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def gpu_bwd(dims, inp, ker, dy, with_bias):
    din = torch.full(inp.shape, float("nan"), device=DEV)
    dker = torch.full(ker.shape, float("nan"), device=DEV)
    db = torch.full((inp.shape[1],), float("nan"), device=DEV) if with_bias else None
    K.convnd_bwd(dims, T(inp), T(ker), T(dy), din, dker, db)
    torch.cuda.synchronize()
    return din.cpu().numpy(), dker.cpu().numpy(), None if db is None else db.cpu().numpy()


CASES = [((7,), 3, 2), ((9,), 70, 3), ((33,), 64, 4), ((5, 6), 5, 2), ((8, 9), 64, 3),
         ((70, 3), 130, 3), ((4, 5), 3, 4), ((3, 4, 5), 64, 3), ((5, 4, 3), 7, 2),
         ((2, 3, 2, 3), 5, 3), ((6, 7), 4, 5), ((1, 1, 4), 65, 3), ((9,), 2, 1),
         ((4, 7, 9), 70, 3), ((10, 11), 65, 4), ((3, 6, 70), 3, 2)]


@pytest.mark.parametrize("dims,D,Kk", CASES)
@pytest.mark.parametrize("bias", [True, False])
def test_forward_vs_oracle(dims, D, Kk, bias):
    inp, ker, b, _ = conv_inputs(dims, D, Kk, bias=bias)
    ref = O.convnd_forward(dims, inp, ker, b, nthreads=8, fast=True)
    got = gpu_fwd(dims, inp, ker, b)
    assert_close(got, ref, TOL_F32, "output", fwd_kappa(dims, inp, ker, b))


@pytest.mark.parametrize("dims,D,Kk", CASES)
@pytest.mark.parametrize("bias", [True, False])
def test_backward_vs_oracle(dims, D, Kk, bias):
    inp, ker, _, dy = conv_inputs(dims, D, Kk, seed=1)
    rdi, rdk, rdb = O.convnd_backward(dims, inp, ker, dy, with_bias=bias)
    gdi, gdk, gdb = gpu_bwd(dims, inp, ker, dy, bias)
    kdi, kdk, kdb = bwd_kappa(dims, inp, ker, dy, bias)
    assert_close(gdi, rdi, TOL_F32, "dinput", kdi)
    assert_close(gdk, rdk, TOL_F32, "dkernel", kdk)
    if bias:
        assert_close(gdb, rdb, TOL_F32, "dbias", kdb)


def test_known_answers():
    # tests/unit/test_convnd_full.c:14-20: 2x2, K=2 -> {4.5, 11.5, 14.5, 30.5};
    # tests/unit/test_conv1d_final.c:233-295: input 2, kernel 3, bias 1 -> {7, 13, 13}.
    got = gpu_fwd((2, 2), np.arange(1, 5, dtype=np.float32)[:, None],
                  np.arange(1, 5, dtype=np.float32)[:, None], np.array([0.5], np.float32))
    np.testing.assert_allclose(got[:, 0], [4.5, 11.5, 14.5, 30.5], atol=1e-6)
    got = gpu_fwd((3,), np.full((3, 1), 2.0, np.float32), np.full((2, 1), 3.0, np.float32),
                  np.array([1.0], np.float32))
    np.testing.assert_allclose(got[:, 0], [7, 13, 13], atol=1e-6)


def test_batched_equals_per_grid():
    dims, D, Kk, nb = (6, 7), 66, 3, 3
    parts = [conv_inputs(dims, D, Kk, seed=10 + i) for i in range(nb)]
    ker, b = parts[0][1], parts[0][2]
    inp = np.stack([p[0] for p in parts])
    dy = np.stack([p[3] for p in parts])
    out = torch.empty(inp.shape, device=DEV)
    K.convnd_fwd(dims, T(inp), T(ker), T(b), out, batch=nb)
    din = torch.empty(inp.shape, device=DEV)
    dker = torch.empty(ker.shape, device=DEV)
    db = torch.empty(D, device=DEV)
    K.convnd_bwd(dims, T(inp), T(ker), T(dy), din, dker, db, batch=nb)
    torch.cuda.synchronize()
    sk, sb, kk, kb = 0, 0, 0, 0
    for i in range(nb):
        ref = O.convnd_forward(dims, inp[i], ker, b)
        assert_close(out[i].cpu().numpy(), ref, TOL_F32, f"out[{i}]", fwd_kappa(dims, inp[i], ker, b))
        rdi, rdk, rdb = O.convnd_backward(dims, inp[i], ker, dy[i])
        kdi, kdk, kdb = bwd_kappa(dims, inp[i], ker, dy[i], True)
        assert_close(din[i].cpu().numpy(), rdi, TOL_F32, f"dinput[{i}]", kdi)
        sk, sb, kk, kb = sk + rdk, sb + rdb, kk + kdk, kb + kdb
    assert_close(dker.cpu().numpy(), sk, TOL_F32, "dkernel (sum over batch)", kk)
    assert_close(db.cpu().numpy(), sb, TOL_F32, "dbias (sum over batch)", kb)


def test_backward_many_tasks_deterministic():
    # 2 x (2048, 48) grids, D = 100 (two channel groups): 32-point strips, and
    # each dkernel workgroup sums two quads of line tasks into its slot. The
    # slots are added in a fixed order, so two runs agree bit for bit.
    dims, D, Kk, nb = (2048, 48), 100, 3, 2
    parts = [conv_inputs(dims, D, Kk, seed=20 + i) for i in range(nb)]
    ker = parts[0][1]
    inp = np.stack([p[0] for p in parts])
    dy = np.stack([p[3] for p in parts])
    runs = []
    for _ in range(2):
        din = torch.full(inp.shape, float("nan"), device=DEV)
        dker = torch.full(ker.shape, float("nan"), device=DEV)
        db = torch.full((D,), float("nan"), device=DEV)
        K.convnd_bwd(dims, T(inp), T(ker), T(dy), din, dker, db, batch=nb)
        torch.cuda.synchronize()
        runs.append((din.cpu().numpy(), dker.cpu().numpy(), db.cpu().numpy()))
    for a, b in zip(runs[0], runs[1]):
        assert np.array_equal(a, b)
    sk, sb, kk, kb = 0, 0, 0, 0
    for i in range(nb):
        rdi, rdk, rdb = O.convnd_backward(dims, inp[i], ker, dy[i])
        kdi, kdk, kdb = bwd_kappa(dims, inp[i], ker, dy[i], True)
        assert_close(runs[0][0][i], rdi, TOL_F32, f"dinput[{i}]", kdi)
        sk, sb, kk, kb = sk + rdk, sb + rdb, kk + kdk, kb + kdb
    assert_close(runs[0][1], sk, TOL_F32, "dkernel (sum over batch)", kk)
    assert_close(runs[0][2], sb, TOL_F32, "dbias (sum over batch)", kb)


def test_reference_entry_points_host_and_device():
    dims, D, Kk = (9, 10), 20, 3
    inp, ker, b, dy = conv_inputs(dims, D, Kk, seed=3)
    ref = O.convnd_forward(dims, inp, ker, b)
    rdi, rdk, rdb = O.convnd_backward(dims, inp, ker, dy)
    kf = fwd_kappa(dims, inp, ker, b)
    kdi, kdk, kdb = bwd_kappa(dims, inp, ker, dy, True)
    # host pointers through convnd(COMPLETE) and the *_wavefront entry points
    out = np.full_like(inp, np.nan)
    din, dker, db = np.full_like(inp, np.nan), np.full_like(ker, np.nan), np.full(D, np.nan, np.float32)
    p, _keep = K.convnd_params(dims, inp, ker, b, out, dy, din, dker, db, D=D, K=Kk)
    K.convnd(C.byref(p), K.CONVND_COMPLETE)
    assert K.km_last_error() == ""
    assert_close(out, ref, TOL_F32, "convnd out", kf)
    assert_close(din, rdi, TOL_F32, "convnd dinput", kdi)
    assert_close(dker, rdk, TOL_F32, "convnd dkernel", kdk)
    assert_close(db, rdb, TOL_F32, "convnd dbias", kdb)
    plan = K.km_wavefront_plan_create(K.longs(dims), len(dims))
    out2 = np.full_like(inp, np.nan)
    p2, _k2 = K.convnd_params(dims, inp, ker, b, out2, D=D, K=Kk)
    K.convnd_forward_wavefront(C.byref(p2), plan)
    assert_close(out2, ref, TOL_F32, "forward_wavefront", kf)
    din2, dker2 = np.full_like(inp, np.nan), np.full_like(ker, np.nan)
    p3, _k3 = K.convnd_params(dims, inp, ker, None, None, dy, din2, dker2, None, D=D, K=Kk)
    K.convnd_backward_wavefront(C.byref(p3), plan)
    assert_close(din2, rdi, TOL_F32, "backward_wavefront dinput", kdi)
    assert_close(dker2, rdk, TOL_F32, "backward_wavefront dkernel", kdk)
    # plan of other dims: refused, outputs untouched
    bad = K.km_wavefront_plan_create(K.longs((10, 9)), 2)
    out3 = np.full_like(inp, 7.0)
    p4, _k4 = K.convnd_params(dims, inp, ker, b, out3, D=D, K=Kk)
    K.convnd_forward_wavefront(C.byref(p4), bad)
    assert "plan" in K.km_last_error() and (out3 == 7.0).all()
    K.km_wavefront_plan_free(plan)
    K.km_wavefront_plan_free(bad)
    # device pointers through om_convnd_forward / om_convnd_backward
    tin, tker, tb, tdy = T(inp), T(ker), T(b), T(dy)
    tout, tdin = torch.empty_like(tin), torch.empty_like(tin)
    tdker, tdb = torch.empty_like(tker), torch.empty_like(tb)
    pd, _kd = K.convnd_params(dims, tin, tker, tb, tout, tdy, tdin, tdker, tdb, D=D, K=Kk)
    assert K.om_convnd_forward(C.byref(pd)) == 0
    assert K.om_convnd_backward(C.byref(pd)) == 0
    assert_close(tout.cpu().numpy(), ref, TOL_F32, "om out", kf)
    assert_close(tdin.cpu().numpy(), rdi, TOL_F32, "om dinput", kdi)
    assert_close(tdker.cpu().numpy(), rdk, TOL_F32, "om dkernel", kdk)
    assert_close(tdb.cpu().numpy(), rdb, TOL_F32, "om dbias", kdb)


def test_invalid_parameters_rejected():
    pbad, _k = K.convnd_params((4, 4), None, None, None, None, D=3, K=2)
    assert K.om_convnd_forward(C.byref(pbad)) == -1
    assert K.km_last_error() != ""
    assert K.convnd_kernel_volume(3, 3) == 27 and K.convnd_kernel_volume(0, 3) == 0


@pytest.mark.parametrize("dims", [(512, 512), (64, 64, 64)])
def test_config3_full_size(dims):
    # D=64, K=3, fp32, forward and backward at full size.
    D, Kk = 64, 3
    inp, ker, b, dy = conv_inputs(dims, D, Kk, seed=0)
    ref = O.convnd_forward(dims, inp, ker, b, nthreads=8, fast=True)
    got = gpu_fwd(dims, inp, ker, b)
    assert_close(got, ref, TOL_F32, "output", fwd_kappa(dims, inp, ker, b))
    rdi, rdk, rdb = O.convnd_backward(dims, inp, ker, dy)
    gdi, gdk, gdb = gpu_bwd(dims, inp, ker, dy, True)
    kdi, kdk, kdb = bwd_kappa(dims, inp, ker, dy, True)
    assert_close(gdi, rdi, TOL_F32, "dinput", kdi)
    assert_close(gdk, rdk, TOL_F32, "dkernel", kdk)
    assert_close(gdb, rdb, TOL_F32, "dbias", kdb)

"""km_scannd_fwd_noalloc (the allocation-free variant of km_scannd_fwd)
against km_scannd_fwd through the C ABI: the same kernels on the same
inputs, so the outputs must agree bit for bit. Two calls in a row, the
second on a smaller grid, exercise the reuse of the fixed device array
(counters and status cleared by a kernel at every launch, flags told apart
by the launch epoch, which the device advances). A captured HIP graph is
replayed on changed inputs; 1D grids, whose allocating path splits the
sequence over a workspace, run without one and allocate nothing."""
import ctypes as C
import subprocess
import sys
from pathlib import Path

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


def _inputs(dims, D, M, tag):
    nd, P = len(dims), int(np.prod(dims))
    g = rng_for(tag, dims, D, M)
    x = g.standard_normal((P, D)).astype(np.float32)
    A = np.log(g.uniform(0.05, 0.9 / nd, (nd, D, M))).astype(np.float32)
    B = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    Cm = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    dt = g.uniform(0.5, 1.0, (nd, P, D)).astype(np.float32)
    return x, A, B, Cm, dt


def _run(fn, dims, arrs):
    P = int(np.prod(dims))
    D, M = arrs[1].shape[1], arrs[1].shape[2]
    t = [torch.from_numpy(a).to(DEV) for a in arrs]
    h = torch.full((P, D, M), float("nan"), device=DEV)
    y = torch.full((P, D), float("nan"), device=DEV)
    p, keep = K.scannd_params(dims, *t, h, y)
    rc = fn(C.byref(p), None)
    assert rc == 0, K.km_last_error()
    torch.cuda.synchronize()
    return y.cpu().numpy(), h.cpu().numpy()


@pytest.mark.parametrize("shapes", [[((40, 24, 24), 16, 16), ((9, 6, 11), 4, 16)],
                                    [((12, 10, 9, 8), 4, 16), ((64, 48), 8, 8)]])
def test_noalloc_matches_allocating_entry_point(shapes):
    for dims, D, M in shapes:           # the second call is on a smaller grid
        arrs = _inputs(dims, D, M, "noalloc")
        y_na, h_na = _run(K.km_scannd_fwd_noalloc_c, dims, arrs)
        y_ref, h_ref = _run(K.km_scannd_fwd_c, dims, arrs)
        assert np.isfinite(y_na).all() and np.isfinite(h_na).all()
        assert np.array_equal(y_na.view(np.uint32), y_ref.view(np.uint32)), dims
        assert np.array_equal(h_na.view(np.uint32), h_ref.view(np.uint32)), dims
    # And the last (smaller) call against the oracle.
    yr, hr = O.scannd_ref(dims, *arrs, nthreads=8, fast=True)
    ya, ha = O.scannd_ref(dims, np.abs(arrs[0]), arrs[1], np.abs(arrs[2]), np.abs(arrs[3]), arrs[4],
                          nthreads=8, fast=True)
    assert_close(y_na, yr, TOL_F32, "y", ya)
    assert_close(h_na, hr, TOL_F32, "h", ha)


def test_noalloc_rejects_shapes_outside_the_tile_kernels():
    # D*M not a multiple of 64: the per-level schedule needs an allocated plan
    # buffer, so the allocation-free entry point refuses before launching.
    dims, D, M = (5, 6, 7), 3, 5
    arrs = _inputs(dims, D, M, "noalloc-reject")
    P = int(np.prod(dims))
    t = [torch.from_numpy(a).to(DEV) for a in arrs]
    h = torch.zeros((P, D, M), device=DEV)
    y = torch.zeros((P, D), device=DEV)
    p, keep = K.scannd_params(dims, *t, h, y)
    assert K.km_scannd_fwd_noalloc_c(C.byref(p), None) == -1
    assert "per-level" in K.km_last_error()


def test_noalloc_replays_from_a_captured_graph():
    # A 3D grid runs the dataflow schedule, whose flags are told apart by an
    # epoch. The call is captured once in a graph and replayed on changed x
    # and B: every replay must equal an eager km_scannd_fwd on the same
    # inputs (an epoch fixed at capture time would let replay 2 see replay
    # 1's flags and read predecessor states before they are written).
    dims, D, M = (40, 24, 24), 16, 16
    P = int(np.prod(dims))
    arrs = _inputs(dims, D, M, "noalloc-graph")
    t = [torch.from_numpy(a).to(DEV) for a in arrs]
    h = torch.zeros((P, D, M), device=DEV)
    y = torch.zeros((P, D), device=DEV)
    p, keep = K.scannd_params(dims, *t, h, y)
    assert K.km_scannd_fwd_noalloc_c(C.byref(p), None) == 0, K.km_last_error()   # set-up, eager
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        rc = K.km_scannd_fwd_noalloc_c(C.byref(p), C.c_void_p(side.cuda_stream))
    assert rc == 0, K.km_last_error()
    for rep in range(4):
        g = rng_for("noalloc-graph-replay", rep)
        xs = g.standard_normal((P, D)).astype(np.float32)
        Bs = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
        t[0].copy_(torch.from_numpy(xs))
        t[2].copy_(torch.from_numpy(Bs))
        h.fill_(float("nan"))
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        y_g, h_g = y.cpu().numpy(), h.cpu().numpy()
        assert K.scannd_status() == 0
        cur = (xs, arrs[1], Bs, arrs[3], arrs[4])
        y_e, h_e = _run(K.km_scannd_fwd_c, dims, cur)
        assert np.isfinite(y_g).all() and np.isfinite(h_g).all(), rep
        assert np.array_equal(y_g.view(np.uint32), y_e.view(np.uint32)), rep
        assert np.array_equal(h_g.view(np.uint32), h_e.view(np.uint32)), rep
    del graph
    torch.cuda.synchronize()


_ONE_D = r"""
import ctypes as C, sys
import numpy as np, torch
sys.path[:0] = [sys.argv[1]]
import kmamba as K
d = np.load(sys.argv[2])
def call(fn, dims, arrs):
    P = int(np.prod(dims)); D, M = arrs[1].shape[1], arrs[1].shape[2]
    t = [torch.from_numpy(a).cuda() for a in arrs]
    h = torch.full((P, D, M), float("nan"), device="cuda")
    y = torch.full((P, D), float("nan"), device="cuda")
    torch.cuda.synchronize()
    p, keep = K.scannd_params(dims, *t, h, y)
    held0, free0 = K.km_device_bytes_held(), torch.cuda.mem_get_info()[0]
    rc = fn(C.byref(p), None)
    assert rc == 0, K.km_last_error()
    torch.cuda.synchronize()
    held1, free1 = K.km_device_bytes_held(), torch.cuda.mem_get_info()[0]
    return y.cpu().numpy(), h.cpu().numpy(), held1 - held0, free0 - free1
small = [d["sx"], d["sA"], d["sB"], d["sC"], d["sdt"]]
big = [d["x"], d["A"], d["B"], d["C"], d["dt"]]
# Load both modules' code (Scan1D kernels: a 1D call; tile kernels: a 2D call).
call(K.km_scannd_fwd_noalloc_c, (64,), small)
call(K.km_scannd_fwd_noalloc_c, (8, 8), [small[0], small[1][:1].repeat(2, 0), small[2], small[3],
                                         small[4].repeat(2, 0)])
y, h, dheld, dfree = call(K.km_scannd_fwd_noalloc_c, (8192,), big)
print("noalloc 1D: library bytes +%d, device free -%d" % (dheld, dfree), flush=True)
ya, ha, dheld_a, _ = call(K.km_scannd_fwd_c, (8192,), big)
print("allocating 1D: library bytes +%d" % dheld_a, flush=True)
np.savez(sys.argv[3], y=y, h=h, ya=ya, ha=ha, dheld=dheld, dfree=dfree, dheld_a=dheld_a)
"""


def test_noalloc_1d_allocates_nothing(tmp_path):
    # dims (8192,), D 64, M 16: two channel groups and a long sequence, which
    # km_scannd_fwd splits over workgroups through a workspace block. The
    # allocation-free entry point must run it unsplit: in a fresh process
    # (the library holding no blocks yet) neither the library's held bytes
    # nor the device's free memory may change across the call, while the
    # allocating call on the same shape does take a block. Both agree with
    # the oracle.
    dims, D, M = (8192,), 64, 16
    root = Path(__file__).resolve().parent.parent
    x, A, B, Cm, dt = _inputs(dims, D, M, "noalloc-1d")
    sx, sA, sB, sC, sdt = _inputs((64,), D, M, "noalloc-1d-small")
    src, dst = tmp_path / "in.npz", tmp_path / "out.npz"
    np.savez(src, x=x, A=A, B=B, C=Cm, dt=dt, sx=sx, sA=sA, sB=sB, sC=sC, sdt=sdt)
    r = subprocess.run([sys.executable, "-c", _ONE_D, str(root / "k-mamba_amd"), str(src), str(dst)],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    out = np.load(dst)
    assert int(out["dheld"]) == 0, "the allocation-free call grew the library's blocks"
    assert int(out["dfree"]) == 0, "device free memory changed across the allocation-free call"
    assert int(out["dheld_a"]) > 0, "the allocating call was expected to split (take a block)"
    yr, hr = O.scannd_ref(dims, x, A, B, Cm, dt, nthreads=8, fast=True)
    ya, ha = O.scannd_ref(dims, np.abs(x), A, np.abs(B), np.abs(Cm), dt, nthreads=8, fast=True)
    assert_close(out["y"], yr, TOL_F32, "y noalloc", ya)
    assert_close(out["h"], hr, TOL_F32, "h noalloc", ha)
    assert_close(out["ya"], yr, TOL_F32, "y allocating", ya)
    assert_close(out["ha"], hr, TOL_F32, "h allocating", ha)

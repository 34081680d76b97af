"""km_scannd_fwd_noalloc (the allocation-free variant of km_scannd_fwd)
against km_scannd_fwd through the C ABI: the same kernels on the same
inputs, so the outputs must agree bit for bit. Two calls in a row, the
second on a smaller grid, exercise the reuse of the fixed device array
(counters and status cleared by a kernel at every launch, flags told apart
by the launch epoch)."""
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

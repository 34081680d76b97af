"""Empty-sequence cases (L = 0) of the Scan1D entry points.

The reference's scan1d (cpu/scan1d.asm:40-179) loops over no steps when
L = 0: the running state it was given is left as it is and y is not
written. scan1d_backward (cpu/scan1d_backward.c:199-205) zeroes its outputs
before a loop that then runs no step, so dA is zero. With no step the
sequence tensors may be empty (NULL) on the km_* API.
"""
import ctypes as C

import numpy as np
import pytest

import kmamba as K

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    torch.zeros(1, device=DEV)
    assert K.kmamba_cuda_available() == 1, K.km_last_error()


def _empty_inputs(Bsz, D, N, io):
    x = torch.empty((Bsz, 0, D), device=DEV, dtype=io)
    A = -torch.arange(1, N + 1, dtype=torch.float32, device=DEV).repeat(D, 1).contiguous()
    Bm = torch.empty((Bsz, 0, N), device=DEV, dtype=io)
    return x, torch.empty_like(x), A, Bm, torch.empty_like(Bm)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("with_h0", [False, True])
def test_fwd_empty_sequence_final_state_is_initial(with_h0, bf16):
    Bsz, D, N = 3, 40, 16
    x, dt, A, Bm, Cm = _empty_inputs(Bsz, D, N, torch.bfloat16 if bf16 else torch.float32)
    y = torch.empty_like(x)
    h0 = torch.randn((Bsz, D, N), device=DEV) if with_h0 else None
    hf = torch.full((Bsz, D, N), 7.0, device=DEV)
    K.scan1d_fwd(x, dt, A, Bm, Cm, y, h0=h0, h_final=hf)
    torch.cuda.synchronize()
    want = h0 if with_h0 else torch.zeros_like(hf)
    assert torch.equal(hf, want)


@pytest.mark.parametrize("bf16", [False, True])
def test_bwd_empty_sequence_zero_dA(bf16):
    Bsz, D, N = 2, 40, 16
    io = torch.bfloat16 if bf16 else torch.float32
    x, dt, A, Bm, Cm = _empty_inputs(Bsz, D, N, io)
    dy, dx, ddt = torch.empty_like(x), torch.empty_like(x), torch.empty_like(x)
    dB, dC = torch.empty_like(Bm), torch.empty_like(Bm)
    dA = torch.full((D, N), 5.0, device=DEV)
    K.scan1d_bwd(x, dt, A, Bm, Cm, dy, dx, ddt, dA, dB, dC)
    torch.cuda.synchronize()
    assert torch.count_nonzero(dA).item() == 0


def test_host_api_empty_sequence_leaves_state_and_y():
    L, D, M = 0, 24, 4
    g = np.random.default_rng(5)
    x = np.zeros((1, D), np.float32)          # one row of backing store, no step reads it
    A = -g.uniform(0.1, 1.0, (D, M)).astype(np.float32)
    B = np.zeros((1, D, M), np.float32)
    y = np.full((1, D), 3.0, np.float32)
    h0 = g.uniform(-1, 1, (D, M)).astype(np.float32)
    h = h0.copy()
    p = K.ScanParams(K.ptr(x), K.ptr(A), K.ptr(B), K.ptr(B), K.ptr(x), K.ptr(h), K.ptr(y), L, D, M)
    K.scan1d(C.byref(p))
    assert K.km_last_error() == ""
    assert np.array_equal(h, h0)
    assert np.all(y == 3.0)

"""The drop-in as existing C code uses it: a gcc-built C program
(tests/c/c_caller.c) links lib/libkmamba.so with no torch or Python in the
process and calls the reference host-pointer API (mamba_scan1d_forward on
host memory, running [D, M] state) and the model API (kmamba_create / init
/ forward / save / load). Its outputs must match the oracle."""
import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

import ctypes as C

import kmamba as K
import oracle as O
from kmtest import TOL_F32, assert_close, scan1d_kappa

pytestmark = pytest.mark.gpu
EXE = Path(__file__).resolve().parent / "c" / "c_caller"


def test_c_caller_scan1d_host_api(tmp_path):
    assert EXE.exists(), "tests/c/c_caller not built (build() builds it)"
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    env = dict(os.environ, KM_C_CALLER_IN=str(fin), KM_C_CALLER_OUT=str(fout))
    r = subprocess.run([str(EXE)], capture_output=True, text=True, env=env, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    L, D, M = 33, 40, 16
    raw = np.fromfile(fin, np.float32)
    sizes = [L * D, L * D, D * M, L * D * M, L * D * M, D * M]
    parts = np.split(raw, np.cumsum(sizes)[:-1])
    x, dt, A, B, Cm, h0 = (parts[0].reshape(L, D), parts[1].reshape(L, D), parts[2].reshape(D, M),
                          parts[3].reshape(L, D, M), parts[4].reshape(L, D, M), parts[5].reshape(D, M))
    out = np.fromfile(fout, np.float32)
    y, h = out[:L * D].reshape(L, D), out[L * D:].reshape(D, M)
    yr, hr = O.scan1d(x, A, B, Cm, dt, h0)
    ky, kh, _ = scan1d_kappa(x[None], dt[None], A, B[None], Cm[None], h0=h0[None],
                             bc_strides=(L * D * M, D * M, M))
    assert_close(y, yr, TOL_F32, "y", ky[0])
    assert_close(h, hr, TOL_F32, "h", kh[0])


def test_c_caller_model_api(tmp_path):
    # The C program's logits against the oracle's model forward on the
    # checkpoint it wrote (read back through kmamba_load).
    assert EXE.exists(), "tests/c/c_caller not built (build() builds it)"
    ckpt, fmodel = tmp_path / "m.kmamba", tmp_path / "model.bin"
    env = dict(os.environ, KM_C_CALLER_IN="/dev/null", KM_C_CALLER_OUT="/dev/null",
               KM_C_CALLER_CKPT=str(ckpt), KM_C_CALLER_MODEL=str(fmodel))
    r = subprocess.run([str(EXE)], capture_output=True, text=True, env=env, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "identical after reload: 1" in r.stdout
    raw = np.fromfile(fmodel, np.uint32)
    toks, logits = raw[:12], raw[12:].view(np.float32).reshape(12, 50)
    m = K.kmamba_load(str(ckpt).encode(), 0, None, 0.0, 0.0)
    assert m, K.km_last_error()
    emb, head, blocks = O.model_params(C.cast(m, C.POINTER(O.KMamba)))
    K.kmamba_free(m)
    want = O.kmamba_forward(emb, head, blocks, toks)
    x = np.zeros((1, 12, 16), np.float32)
    ok = toks < 50
    x[0, ok] = emb[toks[ok]]
    for p in blocks:
        x = O.mamba3_forward(p, x)
    kappa = np.abs(x[0]).astype(np.float64) @ np.abs(head).astype(np.float64)
    err = float(np.max(np.abs(logits.astype(np.float64) - want) / np.maximum(kappa, 1e-30)))
    assert err <= 1e-4, f"condition-scaled logits error {err:.3e}"

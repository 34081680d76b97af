"""The read-once tuning switches KM_SCAN1D_CFG, KM_SCANND_T2 and KM_SCANND_T3
change how the work is laid out on the GPU (B*u kept in registers or
recomputed; the ScanND tile shape), not the arithmetic of any output: a
child process with them set must return the same bits as this process
without them, and both match the oracle. KM_SCAN1D_SPLIT sets the segment
length of a split sequence (here 256 steps, not the cost model's choice);
the fold over segments rounds differently from an unsplit run, so that case
is checked against the oracle only.
"""
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import kmamba as K
import oracle as O
from kmtest import TOL_F32, assert_close, rng_for, scan1d_inputs, scan1d_kappa

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"
ROOT = Path(__file__).resolve().parent.parent

# Scan1D N = 16 (shared and per-channel B/C, no history: the layouts the
# switch covers) and ScanND 2D / 3D grids that run on tiles.
S1 = [(2, 600, 96, "shared"), (1, 333, 64, "per_channel")]
SPLIT = (2, 1024, 96, "shared")     # 256-step segments under KM_SCAN1D_SPLIT=256
ND = [((40, 36), 8, 16), ((12, 10, 9), 4, 16)]

_CHILD = r"""
import sys
import numpy as np, torch
sys.path[:0] = [sys.argv[2]]
import kmamba as K
d = np.load(sys.argv[1])
out = {}
for i in range(int(d["n1"])):
    x, dt, A, Bm, Cm = (torch.from_numpy(d[f"s{i}_{k}"]).cuda() for k in ("x", "dt", "A", "B", "C"))
    Bsz, L, D = x.shape
    y = torch.empty((Bsz, L, D), device="cuda"); hf = torch.empty((Bsz, D, A.shape[1]), device="cuda")
    K.scan1d_fwd(x, dt, A, Bm, Cm, y, h_final=hf, bc_strides=tuple(int(v) for v in d[f"s{i}_st"]))
    torch.cuda.synchronize()
    out[f"s{i}_y"] = y.cpu().numpy(); out[f"s{i}_h"] = hf.cpu().numpy()
for i in range(int(d["nn"])):
    dims = tuple(int(v) for v in d[f"n{i}_dims"])
    t = [torch.from_numpy(d[f"n{i}_{k}"]).cuda() for k in ("x", "A", "B", "C", "dt")]
    P, D, M = int(np.prod(dims)), t[1].shape[1], t[1].shape[2]
    h = torch.zeros((P, D, M), device="cuda"); y = torch.zeros((P, D), device="cuda")
    K.scannd_fwd(dims, *t, h, y)
    torch.cuda.synchronize()
    assert K.scannd_status() == 0
    out[f"n{i}_y"] = y.cpu().numpy(); out[f"n{i}_h"] = h.cpu().numpy()
x, dt, A, Bm, Cm = (torch.from_numpy(d[f"sp_{k}"]).cuda() for k in ("x", "dt", "A", "B", "C"))
Bsz, L, D = x.shape
y = torch.empty((Bsz, L, D), device="cuda"); hf = torch.empty((Bsz, D, A.shape[1]), device="cuda")
K.scan1d_fwd(x, dt, A, Bm, Cm, y, h_final=hf, bc_strides=tuple(int(v) for v in d["sp_st"]))
torch.cuda.synchronize()
out["split_y"] = y.cpu().numpy(); out["split_h"] = hf.cpu().numpy()
np.savez(sys.argv[3], **out)
print("knobs child done", flush=True)
"""


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    torch.zeros(1, device=DEV)
    assert K.kmamba_cuda_available() == 1, K.km_last_error()


def _s1_case(Bsz, L, D, layout):
    N = 16
    x, dt, A, _, _ = scan1d_inputs(Bsz, L, D, N, seed=7)
    g = rng_for("knobs-1d", Bsz, L, D, layout)
    # (batch, step, channel) strides of B / C: [B, L, N] shared, [B, L, D, N] per channel.
    shape, st = ((Bsz, L, N), (L * N, N, 0)) if layout == "shared" else \
        ((Bsz, L, D, N), (L * D * N, D * N, N))
    Bm = (g.standard_normal(shape) * 0.25).astype(np.float32)
    Cm = (g.standard_normal(shape) * 0.25).astype(np.float32)
    return x, dt, A, Bm, Cm, st


def _nd_case(dims, D, M):
    nd, P = len(dims), int(np.prod(dims))
    g = rng_for("knobs-nd", dims, D, M)
    x = g.standard_normal((P, D)).astype(np.float32)
    A = np.log(g.uniform(0.05, 0.9 / nd, (nd, D, M))).astype(np.float32)
    B = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    Cm = (g.standard_normal((P, D, M)) * 0.25).astype(np.float32)
    dt = g.uniform(0.5, 1.0, (nd, P, D)).astype(np.float32)
    return x, A, B, Cm, dt


def test_tuning_switches_give_identical_bits(tmp_path):
    arrays = {"n1": np.int64(len(S1)), "nn": np.int64(len(ND))}
    here = {}
    for i, case in enumerate(S1):
        x, dt, A, Bm, Cm, st = _s1_case(*case)
        arrays.update({f"s{i}_x": x, f"s{i}_dt": dt, f"s{i}_A": A, f"s{i}_B": Bm, f"s{i}_C": Cm,
                       f"s{i}_st": np.array(st)})
        tx, tdt, tA, tB, tC = (torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
                               for a in (x, dt, A, Bm, Cm))
        Bsz, L, D = x.shape
        y = torch.empty((Bsz, L, D), device=DEV)
        hf = torch.empty((Bsz, D, 16), device=DEV)
        K.scan1d_fwd(tx, tdt, tA, tB, tC, y, h_final=hf, bc_strides=st)
        torch.cuda.synchronize()
        here[f"s{i}_y"], here[f"s{i}_h"] = y.cpu().numpy(), hf.cpu().numpy()
        yr, hr = O.scan1d_batched(x, dt, A, Bm, Cm, bc_strides=st, nthreads=8, fast=True)[:2]
        ky, kh, _ = scan1d_kappa(x, dt, A, Bm, Cm, bc_strides=st)
        assert_close(here[f"s{i}_y"], yr, TOL_F32, f"scan1d {case} y", ky)
        assert_close(here[f"s{i}_h"], hr, TOL_F32, f"scan1d {case} h", kh)
    for i, (dims, D, M) in enumerate(ND):
        x, A, B, Cm, dt = _nd_case(dims, D, M)
        arrays.update({f"n{i}_dims": np.array(dims), f"n{i}_x": x, f"n{i}_A": A, f"n{i}_B": B,
                       f"n{i}_C": Cm, f"n{i}_dt": dt})
        t = [torch.from_numpy(a).to(DEV) for a in (x, A, B, Cm, dt)]
        P = int(np.prod(dims))
        h = torch.zeros((P, D, M), device=DEV)
        y = torch.zeros((P, D), device=DEV)
        K.scannd_fwd(dims, *t, h, y)
        torch.cuda.synchronize()
        here[f"n{i}_y"], here[f"n{i}_h"] = y.cpu().numpy(), h.cpu().numpy()
        yr, hr = O.scannd_ref(dims, x, A, B, Cm, dt, nthreads=8, fast=True)
        ya, ha = O.scannd_ref(dims, np.abs(x), A, np.abs(B), np.abs(Cm), dt, nthreads=8, fast=True)
        assert_close(here[f"n{i}_y"].reshape(yr.shape), yr, TOL_F32, f"scannd {dims} y", ya)
        assert_close(here[f"n{i}_h"].reshape(hr.shape), hr, TOL_F32, f"scannd {dims} h", ha)
    xs, dts, As, Bs, Cs, sts = _s1_case(*SPLIT)
    arrays.update({"sp_x": xs, "sp_dt": dts, "sp_A": As, "sp_B": Bs, "sp_C": Cs, "sp_st": np.array(sts)})
    src, dst = tmp_path / "in.npz", tmp_path / "out.npz"
    np.savez(src, **arrays)
    # Non-default values of each switch: B*u recomputed in the replay; 2D
    # tiles of 4 rows x 16 points (default 8 x 4), 3D tiles 2 x 2 x 4
    # (default 4 x 4 x 8); Scan1D sequences in 256-step segments.
    env = dict(os.environ, KM_SCAN1D_CFG="0", KM_SCANND_T2="16,4", KM_SCANND_T3="4,2",
               KM_SCAN1D_SPLIT="256")
    print("knobs child: KM_SCAN1D_CFG=0 KM_SCANND_T2=16,4 KM_SCANND_T3=4,2 KM_SCAN1D_SPLIT=256",
          flush=True)
    r = subprocess.run([sys.executable, "-c", _CHILD, str(src), str(ROOT / "k-mamba_amd"), str(dst)],
                       env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    there = np.load(dst)
    for k, v in here.items():
        assert np.array_equal(there[k], v, equal_nan=True), f"{k} differs under the tuning switches"
    yr, hr = O.scan1d_batched(xs, dts, As, Bs, Cs, bc_strides=sts, nthreads=8, fast=True)[:2]
    ky, kh, _ = scan1d_kappa(xs, dts, As, Bs, Cs, bc_strides=sts)
    assert_close(there["split_y"], yr, TOL_F32, "forced split y", ky)
    assert_close(there["split_h"], hr, TOL_F32, "forced split h", kh)

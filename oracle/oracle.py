"""ctypes binding of the CPU oracle (test infrastructure only).

Loads oracle/liboracle.so (the C restatement of the reference CPU path,
kmoracle.c). oracle/_ref/libkmref.so (the reference's own C compiled in
place, built only where the reference tree exists) is loaded lazily, on the
first access to `ref` or a use_ref=True call: only the CPU pin tests do that,
so GPU test processes never load the compiled reference. REF_AVAILABLE says
whether it was built, without loading it. Only the tests,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module;
the product never does.

All wrappers take and return numpy float32 / int64 arrays.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# KM_ORACLE_LIB names another build of the oracle (the sanitizer build,
# oracle/_san/liboracle.so); it then serves the timing entry points too.
ORACLE_SO = Path(os.environ.get("KM_ORACLE_LIB") or HERE / "liboracle.so")
ORACLE_FAST_SO = ORACLE_SO if os.environ.get("KM_ORACLE_LIB") else HERE / "liboracle_fast.so"
REF_SO = HERE / "_ref" / "libkmref.so"

if not ORACLE_SO.exists():
    raise ImportError(f"{ORACLE_SO} missing: run make -C oracle")

orc = C.CDLL(str(ORACLE_SO))
orc_fast = C.CDLL(str(ORACLE_FAST_SO)) if ORACLE_FAST_SO.exists() else orc
REF_AVAILABLE = REF_SO.exists()
_ref_lib = None
_REF_SIGS = []   # signature setters run when the compiled reference is loaded

vp = C.c_void_p
lp = C.POINTER(C.c_long)


def P(a):
    """Address of a numpy array (None -> NULL)."""
    return None if a is None else a.ctypes.data_as(vp)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def longs(vals):
    return (C.c_long * len(vals))(*[int(v) for v in vals])


class ScanParams(C.Structure):
    _fields_ = [(n, vp) for n in ("x", "A", "B", "C", "delta", "h", "y")] + \
               [(n, C.c_long) for n in ("L", "D", "M")]


class ScanBackwardParams(C.Structure):
    _fields_ = [(n, vp) for n in ("x", "A", "B", "C", "delta", "h0", "h", "dy",
                                  "dx", "dA", "dB", "dC", "ddelta")] + \
               [(n, C.c_long) for n in ("L", "D", "M")]


class ScanBackwardSharedParams(C.Structure):
    _fields_ = [(n, vp) for n in ("x", "A", "A_diag", "B", "C", "delta", "h0", "h", "dy",
                                  "dx", "dA", "dB", "dC", "ddelta")] + \
               [(n, C.c_long) for n in ("L", "D")]


class Scan2DParams(C.Structure):
    _fields_ = [(n, vp) for n in ("x", "A1", "A2", "B", "C", "delta1", "delta2", "h", "y")] + \
               [(n, C.c_long) for n in ("d1", "d2", "D", "M")]


class ScanNDParams(C.Structure):
    _fields_ = [("dims", lp), ("ndims", C.c_long), ("D", C.c_long), ("M", C.c_long)] + \
               [(n, vp) for n in ("x", "A", "B", "C", "delta", "h", "y", "theta", "lambda_")]


class ConvNDParams(C.Structure):
    _fields_ = [(n, vp) for n in ("input", "kernel", "bias", "output", "dy", "dinput",
                                  "dkernel", "dbias")] + \
               [("dims", lp), ("ndims", C.c_long), ("D", C.c_long), ("K", C.c_long)]


class Plan(C.Structure):
    _fields_ = [("dims", lp), ("ndims", C.c_long), ("total_points", C.c_long),
                ("max_level", C.c_long), ("max_level_size", C.c_long),
                ("level_starts", lp), ("level_offsets", lp)]


def _sig(lib, name, restype, argtypes):
    if lib is None:
        return None
    fn = getattr(lib, name)
    fn.restype = restype
    fn.argtypes = argtypes
    return fn


for _lib in {orc, orc_fast}:
    _sig(_lib, "orc_scan1d", None, [C.POINTER(ScanParams)])
    _sig(_lib, "orc_scan1d_batched", None, [vp] * 8 + [C.c_long] * 7 + [C.c_int, C.c_int])
    _sig(_lib, "orc_scan1d_backward", None, [C.POINTER(ScanBackwardParams)])
    _sig(_lib, "orc_scan1d_backward_m1_shared_bc", None, [C.POINTER(ScanBackwardSharedParams)])
    _sig(_lib, "orc_scan1d_backward_m1_shared_bc_asm", None,
         [C.POINTER(ScanBackwardSharedParams), C.c_int])
    _sig(_lib, "orc_m1_asm_taylor", C.c_float, [C.c_float, C.c_int])
    _sig(_lib, "orc_scan1d_batched_backward", None, [vp] * 13 + [C.c_long] * 7 + [C.c_int])
    _sig(_lib, "orc_scan2d", None, [C.POINTER(Scan2DParams)])
    _sig(_lib, "orc_scannd_ref", C.c_int, [C.POINTER(ScanNDParams), C.c_int])
    _sig(_lib, "orc_scannd", C.c_int, [C.POINTER(ScanNDParams), C.c_int])
    _sig(_lib, "orc_scannd_backward", C.c_int, [C.POINTER(ScanNDParams), vp, vp, vp, vp, vp, vp])
    _sig(_lib, "orc_convnd_forward", None, [C.POINTER(ConvNDParams), C.c_int])
    _sig(_lib, "orc_convnd_backward", None, [C.POINTER(ConvNDParams)])
    _sig(_lib, "orc_plan_create", C.POINTER(Plan), [lp, C.c_long])
    _sig(_lib, "orc_plan_free", None, [C.POINTER(Plan)])
    _sig(_lib, "orc_wavefront_level_size", C.c_long, [lp, C.c_long, C.c_long])
    _sig(_lib, "orc_wavefront_total_points", C.c_long, [lp, C.c_long])
    _sig(_lib, "orc_wavefront_max_level", C.c_long, [lp, C.c_long])
    _sig(_lib, "orc_wavefront_row_major_offset", C.c_long, [lp, lp, C.c_long])
    _sig(_lib, "orc_silu_f32", None, [vp, vp, C.c_long])
    _sig(_lib, "orc_softplus_f32", None, [vp, vp, C.c_long])

def _load_ref():
    """The compiled reference (oracle/_ref/libkmref.so), loaded on first use."""
    global _ref_lib
    if _ref_lib is not None:
        return _ref_lib
    if not REF_AVAILABLE:
        raise RuntimeError(f"{REF_SO} not built (the reference tree is absent)")
    ref = C.CDLL(str(REF_SO))
    _sig(ref, "scannd_ref", C.c_int, [C.POINTER(ScanNDParams)])
    _sig(ref, "convnd_forward_wavefront", None, [C.POINTER(ConvNDParams), C.POINTER(Plan)])
    _sig(ref, "convnd_backward_wavefront", None, [C.POINTER(ConvNDParams), C.POINTER(Plan)])
    _sig(ref, "scan1d_backward", None, [C.POINTER(ScanBackwardParams)])
    _sig(ref, "scan1d_backward_m1_shared_bc", None, [C.POINTER(ScanBackwardSharedParams)])
    _sig(ref, "km_wavefront_plan_create", C.POINTER(Plan), [lp, C.c_long])
    _sig(ref, "km_wavefront_plan_free", None, [C.POINTER(Plan)])
    _sig(ref, "wavefront_nd_level_size", C.c_long, [lp, C.c_long, C.c_long])
    _sig(ref, "kmr_test_scan1d_ref", None, [vp] * 7 + [C.c_long] * 3)
    _sig(ref, "kmr_test_scan1d_backward_forward_ref", None, [vp] * 7 + [C.c_long] * 3)
    _sig(ref, "silu_f32", None, [vp, vp, C.c_long])
    _sig(ref, "softplus_f32", None, [vp, vp, C.c_long])
    # The reference's scannd_ref shares one idx[] scratch array between the
    # OpenMP threads of its level loop (src/scan_nd.c:44 allocates it once,
    # every thread writes it at :89), so it races with more than one thread.
    # Its other loops are deterministic either way. Run the reference with a
    # single OpenMP thread; the oracle's own loops name num_threads explicitly.
    ref.omp_set_num_threads.argtypes = [C.c_int]
    ref.omp_set_num_threads(1)
    for setter in _REF_SIGS:
        setter(ref)
    _ref_lib = ref
    return ref


def __getattr__(name):
    # `oracle.ref` is the compiled reference, loaded on first access.
    if name == "ref":
        return _load_ref()
    raise AttributeError(f"module 'oracle' has no attribute {name!r}")


# ---------------------------------------------------------------------------
# Scan1D
# ---------------------------------------------------------------------------
def scan1d(x, A, B, Cm, delta, h):
    """Reference scan1d (asm semantics): x, delta [L, D]; A [D, M];
    B, C [L, D, M]; h [D, M] running state. Returns (y, h_final)."""
    x, A, B, Cm, delta = map(f32, (x, A, B, Cm, delta))
    h = f32(h).copy()
    L, D = x.shape
    M = A.shape[1]
    y = np.zeros((L, D), np.float32)
    p = ScanParams(P(x), P(A), P(B), P(Cm), P(delta), P(h), P(y), L, D, M)
    orc.orc_scan1d(C.byref(p))
    return y, h


def scan1d_batched(x, delta, A, Bm, Cm, *, h0=None, bc_strides=None, clamp=True,
                   hist=False, nthreads=1, fast=False):
    """Batched scan: x, delta [B, L, D]; A [D, N]; B/C shared [B, L, N] by
    default, or any buffer with strides bc_strides=(sb, st, sd).
    Returns (y, h_final, h_hist or None)."""
    x, delta, A, Bm, Cm = map(f32, (x, delta, A, Bm, Cm))
    Bsz, L, D = x.shape
    N = A.shape[1]
    if bc_strides is None:
        bc_strides = (L * N, N, 0)
    h = np.zeros((Bsz, D, N), np.float32) if h0 is None else f32(h0).copy()
    y = np.zeros((Bsz, L, D), np.float32)
    hh = np.zeros((Bsz, L, D, N), np.float32) if hist else None
    lib = orc_fast if fast else orc
    lib.orc_scan1d_batched(P(x), P(delta), P(A), P(Bm), P(Cm), P(y), P(h), P(hh),
                           Bsz, L, D, N, *bc_strides, int(clamp), int(nthreads))
    return y, h, hh


def scan1d_backward(x, A, B, Cm, delta, h, dy, h0=None, lib=None):
    """Generic backward (cpu/scan1d_backward.c:297-306). Returns
    (dx, dA, dB, dC, ddelta)."""
    lib = lib or orc
    x, A, B, Cm, delta, h, dy = map(f32, (x, A, B, Cm, delta, h, dy))
    L, D = x.shape
    M = A.shape[1]
    out = dict(dx=np.zeros((L, D), np.float32), dA=np.zeros((D, M), np.float32),
               dB=np.zeros((L, D, M), np.float32), dC=np.zeros((L, D, M), np.float32),
               ddelta=np.zeros((L, D), np.float32))
    h0 = None if h0 is None else f32(h0)
    p = ScanBackwardParams(P(x), P(A), P(B), P(Cm), P(delta), P(h0), P(h), P(dy),
                           P(out["dx"]), P(out["dA"]), P(out["dB"]), P(out["dC"]),
                           P(out["ddelta"]), L, D, M)
    if lib is orc:
        orc.orc_scan1d_backward(C.byref(p))
    else:
        lib.scan1d_backward(C.byref(p))
    return out["dx"], out["dA"], out["dB"], out["dC"], out["ddelta"]


def scan1d_backward_m1_shared_bc_asm(x, A, B, Cm, delta, h, dy, A_diag=None, h0=None,
                                     simple=False):
    """Restatement of the reference's scan1d_backward_m1_shared_bc_asm
    (simple=False) / _simple_asm (simple=True): returns dx, dA, dB, dC,
    ddelta. x, h, dy [L, D]; A, B, Cm [D]; delta [L]."""
    x, A, B, Cm, delta, h, dy = map(f32, (x, A, B, Cm, delta, h, dy))
    L, D = x.shape
    A_diag = None if A_diag is None else f32(A_diag)
    h0 = None if h0 is None else f32(h0)
    out = dict(dx=np.zeros((L, D), np.float32), dA=np.zeros(D, np.float32),
               dB=np.zeros(D, np.float32), dC=np.zeros(D, np.float32),
               ddelta=np.zeros(L, np.float32))
    p = ScanBackwardSharedParams(P(x), P(A), P(A_diag), P(B), P(Cm), P(delta), P(h0), P(h),
                                 P(dy), P(out["dx"]), P(out["dA"]), P(out["dB"]), P(out["dC"]),
                                 P(out["ddelta"]), L, D)
    orc.orc_scan1d_backward_m1_shared_bc_asm(C.byref(p), int(bool(simple)))
    return out["dx"], out["dA"], out["dB"], out["dC"], out["ddelta"]


def m1_asm_taylor(xs, simple=False):
    """The asm routines' Taylor decay of each fp32 value of xs."""
    xs = f32(np.asarray(xs))
    return np.array([orc.orc_m1_asm_taylor(float(v), int(bool(simple))) for v in xs.ravel()],
                    np.float32).reshape(xs.shape)


def scan1d_backward_m1_shared_bc(x, A, B, Cm, delta, h, dy, A_diag=None, h0=None, lib=None):
    lib = lib or orc
    x, A, B, Cm, delta, h, dy = map(f32, (x, A, B, Cm, delta, h, dy))
    L, D = x.shape
    A_diag = None if A_diag is None else f32(A_diag)
    h0 = None if h0 is None else f32(h0)
    out = dict(dx=np.zeros((L, D), np.float32), dA=np.zeros(D, np.float32),
               dB=np.zeros(D, np.float32), dC=np.zeros(D, np.float32),
               ddelta=np.zeros(L, np.float32))
    p = ScanBackwardSharedParams(P(x), P(A), P(A_diag), P(B), P(Cm), P(delta), P(h0), P(h),
                                 P(dy), P(out["dx"]), P(out["dA"]), P(out["dB"]), P(out["dC"]),
                                 P(out["ddelta"]), L, D)
    if lib is orc:
        orc.orc_scan1d_backward_m1_shared_bc(C.byref(p))
    else:
        lib.scan1d_backward_m1_shared_bc(C.byref(p))
    return out["dx"], out["dA"], out["dB"], out["dC"], out["ddelta"]


def scan1d_batched_backward(x, delta, A, Bm, Cm, dy, h_hist, *, h0=None, bc_strides=None,
                            nthreads=1, fast=False):
    """Adjoint of scan1d_batched (no clamp). Returns dx, ddelta [B, L, D],
    dA [D, N], dB, dC (shape of Bm: [B, L, N] when shared)."""
    x, delta, A, Bm, Cm, dy, h_hist = map(f32, (x, delta, A, Bm, Cm, dy, h_hist))
    Bsz, L, D = x.shape
    N = A.shape[1]
    if bc_strides is None:
        bc_strides = (L * N, N, 0)
    dx = np.zeros_like(x)
    ddt = np.zeros_like(x)
    dA = np.zeros((D, N), np.float32)
    dB = np.zeros_like(Bm)
    dC = np.zeros_like(Cm)
    h0 = None if h0 is None else f32(h0)
    lib = orc_fast if fast else orc
    lib.orc_scan1d_batched_backward(P(x), P(delta), P(A), P(Bm), P(Cm), P(dy), P(h0), P(h_hist),
                                    P(dx), P(ddt), P(dA), P(dB), P(dC),
                                    Bsz, L, D, N, *bc_strides, int(nthreads))
    return dx, ddt, dA, dB, dC


# ---------------------------------------------------------------------------
# Scan2D / ScanND
# ---------------------------------------------------------------------------
def scan2d(x, A1, A2, B, Cm, delta1, delta2, d1, d2):
    x, A1, A2, B, Cm, delta1, delta2 = map(f32, (x, A1, A2, B, Cm, delta1, delta2))
    D, M = A1.shape
    h = np.zeros((d1 * d2, D, M), np.float32)
    y = np.zeros((d1 * d2, D), np.float32)
    p = Scan2DParams(P(x), P(A1), P(A2), P(B), P(Cm), P(delta1), P(delta2), P(h), P(y),
                     d1, d2, D, M)
    orc.orc_scan2d(C.byref(p))
    return y, h


def _nd_params(dims, x, A, B, Cm, delta, h, y, theta=None, lam=None):
    dd = longs(dims)
    D, M = A.shape[1], A.shape[2]
    p = ScanNDParams(dd, len(dims), D, M, P(x), P(A), P(B), P(Cm), P(delta), P(h), P(y),
                     None if theta is None else P(theta), None if lam is None else P(lam))
    return p, dd


def scannd_ref(dims, x, A, B, Cm, delta, *, theta=None, lam=None, nthreads=1, use_ref=False,
               fast=False):
    """scannd_ref semantics: x [P, D]; A [nd, D, M]; B, C [P, D, M];
    delta [nd, P, D]; optional Mamba-3 theta [D/2] and lambda [P] (the
    restated lambda branch, see kmoracle.c). Returns (y, h)."""
    x, A, B, Cm, delta = map(f32, (x, A, B, Cm, delta))
    theta = None if theta is None else f32(theta)
    lam = None if lam is None else f32(lam)
    Pn = int(np.prod(dims))
    D, M = A.shape[1], A.shape[2]
    h = np.zeros((Pn, D, M), np.float32)
    y = np.zeros((Pn, D), np.float32)
    p, _keep = _nd_params(dims, x, A, B, Cm, delta, h, y, theta, lam)
    if use_ref:
        # The reference's lambda branch reads out of bounds (undefined output).
        if lam is not None:
            raise ValueError("the compiled reference's Mamba-3 branch is undefined; use the restatement")
        rc = _load_ref().scannd_ref(C.byref(p))
    else:
        rc = (orc_fast if fast else orc).orc_scannd_ref(C.byref(p), int(nthreads))
    if rc != 0:
        raise RuntimeError("scannd_ref failed")
    return y, h


def scannd_backward(dims, x, A, B, Cm, delta, h, dy, *, fast=False):
    """Adjoint of scannd_ref for L = sum dy . y (restated in kmoracle.c; the
    reference has no ScanND backward): h is the forward's states [P, D, M].
    Returns dict dx [P, D], ddelta [nd, P, D], dA [nd, D, M], dB, dC [P, D, M]."""
    x, A, B, Cm, delta, h, dy = map(f32, (x, A, B, Cm, delta, h, dy))
    Pn = int(np.prod(dims))
    nd, D, M = A.shape
    out = {"dx": np.zeros((Pn, D), np.float32), "ddelta": np.zeros((nd, Pn, D), np.float32),
           "dA": np.zeros((nd, D, M), np.float32), "dB": np.zeros((Pn, D, M), np.float32),
           "dC": np.zeros((Pn, D, M), np.float32)}
    y = np.zeros((Pn, D), np.float32)
    p, _keep = _nd_params(dims, x, A, B, Cm, delta, h, y)
    rc = (orc_fast if fast else orc).orc_scannd_backward(
        C.byref(p), P(dy), P(out["dx"]), P(out["ddelta"]), P(out["dA"]), P(out["dB"]), P(out["dC"]))
    if rc != 0:
        raise RuntimeError("orc_scannd_backward failed")
    return out


def scannd(dims, x, A, B, Cm, delta, h=None, *, nthreads=1):
    """CPU dispatch semantics of scannd (1D -> scan1d, 2D -> scan2d)."""
    x, A, B, Cm, delta = map(f32, (x, A, B, Cm, delta))
    Pn = int(np.prod(dims))
    D, M = A.shape[1], A.shape[2]
    if h is None:
        h = np.zeros((Pn, D, M), np.float32)
    h = f32(h).copy()
    y = np.zeros((Pn, D), np.float32)
    p, _keep = _nd_params(dims, x, A, B, Cm, delta, h, y)
    if orc.orc_scannd(C.byref(p), int(nthreads)) != 0:
        raise RuntimeError("scannd failed")
    return y, h


# ---------------------------------------------------------------------------
# ConvND
# ---------------------------------------------------------------------------
def convnd_forward(dims, inp, kernel, bias, *, nthreads=1, use_ref=False, fast=False):
    inp, kernel = f32(inp), f32(kernel)
    bias = None if bias is None else f32(bias)
    D = inp.shape[1]
    K = int(round(kernel.shape[0] ** (1.0 / len(dims))))
    out = np.zeros_like(inp)
    dd = longs(dims)
    p = ConvNDParams(P(inp), P(kernel), P(bias), P(out), None, None, None, None,
                     dd, len(dims), D, K)
    if use_ref:
        ref = _load_ref()
        plan = ref.km_wavefront_plan_create(dd, len(dims))
        ref.convnd_forward_wavefront(C.byref(p), plan)
        ref.km_wavefront_plan_free(plan)
    else:
        (orc_fast if fast else orc).orc_convnd_forward(C.byref(p), int(nthreads))
    return out


def convnd_backward(dims, inp, kernel, dy, *, with_bias=True, use_ref=False):
    inp, kernel, dy = f32(inp), f32(kernel), f32(dy)
    D = inp.shape[1]
    K = int(round(kernel.shape[0] ** (1.0 / len(dims))))
    dinp = np.zeros_like(inp)
    dker = np.zeros_like(kernel)
    dbias = np.zeros(D, np.float32) if with_bias else None
    dd = longs(dims)
    p = ConvNDParams(P(inp), P(kernel), None, None, P(dy), P(dinp), P(dker), P(dbias),
                     dd, len(dims), D, K)
    if use_ref:
        ref = _load_ref()
        plan = ref.km_wavefront_plan_create(dd, len(dims))
        ref.convnd_backward_wavefront(C.byref(p), plan)
        ref.km_wavefront_plan_free(plan)
    else:
        orc.orc_convnd_backward(C.byref(p))
    return dinp, dker, dbias


# ---------------------------------------------------------------------------
# Wavefront plan
# ---------------------------------------------------------------------------
def plan_tables(dims, use_ref=False):
    """(level_starts, level_offsets, max_level_size) as int64 arrays."""
    dd = longs(dims)
    lib = _load_ref() if use_ref else orc
    create = lib.km_wavefront_plan_create if use_ref else lib.orc_plan_create
    free = lib.km_wavefront_plan_free if use_ref else lib.orc_plan_free
    pl = create(dd, len(dims))
    if not pl:
        return None
    p = pl.contents
    starts = np.ctypeslib.as_array(p.level_starts, shape=(p.max_level + 2,)).copy()
    offs = np.ctypeslib.as_array(p.level_offsets, shape=(p.total_points,)).copy()
    mls = p.max_level_size
    free(pl)
    return starts, offs, mls


# ---------------------------------------------------------------------------
# Mamba-3 block forward
# ---------------------------------------------------------------------------
class MBMatrix(C.Structure):              # ref include/kmamba.h:17-24
    _fields_ = [("data", C.POINTER(C.c_float)), ("rows", C.c_size_t), ("cols", C.c_size_t)]


class MBConfig(C.Structure):              # ref include/kmamba.h:27-54
    _fields_ = [(n, C.c_size_t) for n in ("dim", "state_size", "seq_len", "mimo_rank")] + \
               [(n, C.c_float) for n in ("dt_scale", "dt_min", "dt_max")] + \
               [("use_fp16", C.c_int), ("use_bf16", C.c_int), ("loss_scale", C.c_float),
                ("spatial_ndims", C.c_long), ("spatial_dims", C.c_long * 8),
                ("use_convnd", C.c_int), ("convnd_K", C.c_long), ("convnd_ndims", C.c_long)]


class MambaBlock(C.Structure):            # ref include/kmamba.h:116-150
    _fields_ = [("config", MBConfig)] + \
               [(n, MBMatrix) for n in ("W_in", "W_out", "A_log", "W_B", "W_C", "delta_proj")] + \
               [(n, C.POINTER(C.c_float)) for n in ("b_B", "b_C", "theta")] + \
               [("lambda_proj", MBMatrix), ("wavefront_plan", vp)] + \
               [(n, C.POINTER(C.c_float)) for n in ("convnd_kernel", "convnd_bias", "hidden",
                                                   "delta", "scan_B", "scan_C", "scan_delta",
                                                   "scan_h")] + [("opt_state", vp)]


class OrcMamba3(C.Structure):
    _fields_ = [(n, vp) for n in ("W_in", "W_out", "A_log", "W_B", "W_C", "delta_proj",
                                  "lambda_proj", "b_B", "b_C", "theta")] + \
               [(n, C.c_long) for n in ("L", "D", "N", "R")] + \
               [(n, C.c_float) for n in ("dt_scale", "dt_min", "dt_max")]


MAMBA3_PARAMS = ("W_in", "W_out", "A_log", "W_B", "W_C", "delta_proj", "lambda_proj", "b_B", "b_C",
                 "theta")

_sig(orc, "orc_mamba3_forward", None, [C.POINTER(OrcMamba3), vp, vp, C.c_long])


@_REF_SIGS.append
def _ref_block_sigs(ref):
    _sig(ref, "mamba_block_create", C.POINTER(MambaBlock), [C.POINTER(MBConfig)])
    _sig(ref, "mamba_block_free", None, [C.POINTER(MambaBlock)])
    _sig(ref, "mamba_block_init", None, [C.POINTER(MambaBlock)])
    _sig(ref, "mamba_block_forward", None, [C.POINTER(MambaBlock), vp, vp, C.c_size_t])


# ---------------------------------------------------------------------------
# The stacked model: embedding, Mamba-3 blocks, head (src/kmamba.c)
# ---------------------------------------------------------------------------
class KMambaConfig(C.Structure):          # ref include/kmamba.h:159-183
    _fields_ = [(n, C.c_size_t) for n in ("vocab_size", "dim", "state_size", "seq_len",
                                          "n_layers", "mimo_rank")] + \
               [(n, C.c_float) for n in ("dt_scale", "dt_min", "dt_max")] + \
               [("spatial_ndims", C.c_long), ("spatial_dims", C.c_long * 8),
                ("use_convnd", C.c_int), ("convnd_K", C.c_long), ("convnd_ndims", C.c_long),
                ("weight_tying", C.c_int)]


class MBOptimConfig(C.Structure):         # ref include/kmamba_kernels.h:78-85
    _fields_ = [(n, C.c_float) for n in ("lr", "mu", "beta2", "eps", "clip_norm", "weight_decay")]


class KMamba(C.Structure):                # ref include/kmamba.h:185-223 (CPU build)
    _fields_ = [("cfg", KMambaConfig), ("embedding", C.POINTER(C.c_float)),
                ("head", C.POINTER(C.c_float)), ("layers", C.POINTER(C.POINTER(MambaBlock))),
                ("for_training", C.c_int), ("opt_blocks", MBOptimConfig),
                ("lr_embed_head", C.c_float), ("weight_decay", C.c_float)] + \
               [(n, C.POINTER(C.c_float)) for n in ("m_embedding", "v_embedding", "m_head",
                                                   "v_head")] + \
               [("step_embed_head", C.c_size_t), ("last_grad_norm", C.c_float),
                ("last_grad_over_clip", C.c_float), ("last_grad_would_clip", C.c_int)]


_sig(orc, "orc_gemm_f32", None, [vp, vp, vp, C.c_long, C.c_long, C.c_long])


@_REF_SIGS.append
def _ref_model_sigs(ref):
    _sig(ref, "kmamba_create", C.POINTER(KMamba), [C.POINTER(KMambaConfig)])
    _sig(ref, "kmamba_free", None, [C.POINTER(KMamba)])
    _sig(ref, "kmamba_init", C.c_int, [C.POINTER(KMamba), C.c_uint32])
    _sig(ref, "kmamba_forward", C.c_int, [C.POINTER(KMamba), vp, vp])
    _sig(ref, "kmamba_save", C.c_int, [C.POINTER(KMamba), C.c_char_p])
    _sig(ref, "kmamba_load", C.POINTER(KMamba), [C.c_char_p, C.c_int, vp, C.c_float, C.c_float])


def kmamba_config(vocab, dim, N, L, n_layers, R=1, dt_scale=0.1, dt_min=1e-3, dt_max=0.1,
                  weight_tying=0, cls=KMambaConfig):
    cfg = cls()
    cfg.vocab_size, cfg.dim, cfg.state_size, cfg.seq_len = vocab, dim, N, L
    cfg.n_layers, cfg.mimo_rank = n_layers, R
    cfg.dt_scale, cfg.dt_min, cfg.dt_max = dt_scale, dt_min, dt_max
    cfg.weight_tying = weight_tying
    return cfg


def model_params(m):
    """Copies of a KMamba's parameters: embedding [V, D], head [D, V] and one
    block_params dict per layer (works on any library's KMamba pointer)."""
    c = m.contents.cfg
    V, D = c.vocab_size, c.dim
    emb = np.ctypeslib.as_array(m.contents.embedding, shape=(V * D,)).reshape(V, D).copy()
    head = np.ctypeslib.as_array(m.contents.head, shape=(D * V,)).reshape(D, V).copy()
    layers = [block_params(C.cast(m.contents.layers[i], C.POINTER(MambaBlock)))
              for i in range(c.n_layers)]
    return emb, head, layers


def silu(v, *, use_ref=False):
    """The reference SiLU x / (1 + expf(-x)) (include/kmamba_kernels.h:35-37),
    elementwise in fp32: the oracle's restatement, or with use_ref the
    compiled reference's silu_f32 (kernels/activations_f32.c:7-11)."""
    v = f32(v)
    out = np.empty_like(v)
    fn = _load_ref().silu_f32 if use_ref else orc.orc_silu_f32
    fn(P(v), P(out), v.size)
    return out


def softplus(v, *, use_ref=False):
    """The reference softplus logf(1 + expf(x)) (include/kmamba_kernels.h:47-49),
    elementwise in fp32: the oracle's restatement, or with use_ref the
    compiled reference's softplus_f32 (kernels/activations_f32.c:25-29)."""
    v = f32(v)
    out = np.empty_like(v)
    fn = _load_ref().softplus_f32 if use_ref else orc.orc_softplus_f32
    fn(P(v), P(out), v.size)
    return out


def gemm_f32(A, B):
    """C = A . B in the reference gemm_f32's order (kernels/gemm_f32.c:13-31)."""
    A, B = f32(A), f32(B)
    M, K = A.shape
    N = B.shape[1]
    out = np.empty((M, N), np.float32)
    orc.orc_gemm_f32(P(A), P(B), P(out), M, K, N)
    return out


def kmamba_forward(emb, head, layers, tokens, *, dt_scale=0.1, dt_min=1e-3, dt_max=0.1):
    """The model forward of src/kmamba.c:344-372: embedding rows (ids past the
    vocabulary embed as zeros, :85-98), the blocks in order, then h . head."""
    emb, head = f32(emb), f32(head)
    V = emb.shape[0]
    tokens = np.asarray(tokens, dtype=np.int64)
    x = np.zeros((1, tokens.size, emb.shape[1]), np.float32)
    ok = tokens < V
    x[0, ok] = emb[tokens[ok]]
    for p in layers:
        x = mamba3_forward(p, x, dt_scale=dt_scale, dt_min=dt_min, dt_max=dt_max)
    return gemm_f32(x[0], head)


def mb_config(dim, N, L, R=1, dt_scale=0.1, dt_min=1e-3, dt_max=0.1):
    cfg = MBConfig()
    cfg.dim, cfg.state_size, cfg.seq_len, cfg.mimo_rank = dim, N, L, R
    cfg.dt_scale, cfg.dt_min, cfg.dt_max = dt_scale, dt_min, dt_max
    return cfg


def block_params(blk):
    """Copies of a MambaBlock's parameter arrays (numpy, fp32)."""
    b = blk.contents
    N, R = b.config.state_size, max(b.config.mimo_rank, 1)
    out = {}
    for name in ("W_in", "W_out", "A_log", "W_B", "W_C", "delta_proj", "lambda_proj"):
        m = getattr(b, name)
        out[name] = np.ctypeslib.as_array(m.data, shape=(m.rows * m.cols,)).reshape(m.rows, m.cols).copy()
    out["b_B"] = np.ctypeslib.as_array(b.b_B, shape=(N * R,)).copy()
    out["b_C"] = np.ctypeslib.as_array(b.b_C, shape=(N * R,)).copy()
    out["theta"] = np.ctypeslib.as_array(b.theta, shape=(max(N // 2, 1),)).copy()
    return out


def set_block_params(blk, params):
    """Writes parameter arrays into a MambaBlock's buffers."""
    b = blk.contents
    for name in ("W_in", "W_out", "A_log", "W_B", "W_C", "delta_proj", "lambda_proj"):
        m = getattr(b, name)
        dst = np.ctypeslib.as_array(m.data, shape=(m.rows * m.cols,))
        dst[:] = f32(params[name]).ravel()
    for name in ("b_B", "b_C", "theta"):
        src = f32(params[name]).ravel()
        np.ctypeslib.as_array(getattr(b, name), shape=(src.size,))[:] = src


def mamba3_forward(params, x, *, dt_scale=0.1, dt_min=1e-3, dt_max=0.1, use_ref=False):
    """Mamba-3 block forward (src/mamba_block.c:471-501): x [batch, L, D]."""
    x = f32(x)
    batch, L, D = x.shape
    N = params["A_log"].size
    R = params["W_in"].shape[0]
    out = np.zeros_like(x)
    if use_ref:
        ref = _load_ref()
        blk = ref.mamba_block_create(C.byref(mb_config(D, N, L, R, dt_scale, dt_min, dt_max)))
        if not blk:
            raise RuntimeError("reference mamba_block_create failed")
        set_block_params(blk, params)
        ref.mamba_block_forward(blk, P(out), P(x), batch)
        ref.mamba_block_free(blk)
        return out
    keep = {k: f32(v) for k, v in params.items()}
    p = OrcMamba3(*(P(keep[k]) for k in MAMBA3_PARAMS), L, D, N, R, dt_scale, dt_min, dt_max)
    orc.orc_mamba3_forward(C.byref(p), P(x), P(out), batch)
    return out

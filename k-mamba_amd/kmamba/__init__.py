"""Python mirror of libkmamba's C ABI (ctypes), used by the tests and bench.

The library is the product: hand-written HIP kernels for gfx950 behind the
reference k-mamba C API (include/*.h). This module only loads
lib/libkmamba.so, declares the C structures with the reference layouts and
offers thin helpers that pass torch device buffers to the C entry points.
Importing it fails loudly when the shared library has not been built: there is
no Python or CPU fallback for any kernel.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent          # k-mamba_amd/
# KMAMBA_LIB names another build of the library (same ABI) to load instead.
LIB_PATH = Path(os.environ.get("KMAMBA_LIB") or PKG_ROOT / "lib" / "libkmamba.so")
INCLUDE_DIR = PKG_ROOT.parent / "include"

if not LIB_PATH.exists():
    raise ImportError(
        f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()' "
        "or make -C k-mamba_amd)")

# Load torch's HIP runtime first when torch is present, so the process holds
# a single libamdhip64 shared by torch allocations and libkmamba kernels.
try:
    import torch  # noqa: F401
except ImportError:  # C-only use of the mirror (host-side functions)
    torch = None

lib = C.CDLL(str(LIB_PATH))

c_long_p = C.POINTER(C.c_long)
c_float_p = C.POINTER(C.c_float)

KM_F32 = 0
KM_BF16 = 1

KMAMBA_BACKEND_AUTO, KMAMBA_BACKEND_CPU, KMAMBA_BACKEND_GPU = 0, 1, 2
CONVND_FORWARD, CONVND_BACKWARD, CONVND_COMPLETE = 1, 2, 3


class ScanParams(C.Structure):            # include/scan.h (ref include/scan.h:45-56)
    _fields_ = [(n, C.c_void_p) for n in ("x", "A", "B", "C", "delta", "h", "y")] + \
               [(n, C.c_long) for n in ("L", "D", "M")]


class ScanBackwardParams(C.Structure):    # ref include/scan.h:61-78
    _fields_ = [(n, C.c_void_p) for n in ("x", "A", "B", "C", "delta", "h0", "h", "dy",
                                          "dx", "dA", "dB", "dC", "ddelta")] + \
               [(n, C.c_long) for n in ("L", "D", "M")]


class ScanBackwardSharedParams(C.Structure):   # ref include/scan.h:83-100
    _fields_ = [(n, C.c_void_p) for n in ("x", "A", "A_diag", "B", "C", "delta", "h0", "h", "dy",
                                          "dx", "dA", "dB", "dC", "ddelta")] + \
               [(n, C.c_long) for n in ("L", "D")]


class Scan2DParams(C.Structure):          # ref include/scan.h:117-131
    _fields_ = [(n, C.c_void_p) for n in ("x", "A1", "A2", "B", "C", "delta1", "delta2", "h", "y")] + \
               [(n, C.c_long) for n in ("d1", "d2", "D", "M")]


class ScanNDParams(C.Structure):          # ref include/scan_nd.h:40-55
    _fields_ = [("dims", c_long_p), ("ndims", C.c_long), ("D", C.c_long), ("M", C.c_long)] + \
               [(n, C.c_void_p) for n in ("x", "A", "B", "C", "delta", "h", "y", "theta", "lambda_")]


class ConvNDParams(C.Structure):          # ref include/convnd.h:10-23
    _fields_ = [(n, C.c_void_p) for n in ("input", "kernel", "bias", "output", "dy", "dinput",
                                          "dkernel", "dbias")] + \
               [("dims", c_long_p), ("ndims", C.c_long), ("D", C.c_long), ("K", C.c_long)]


class KMWavefrontPlan(C.Structure):       # ref include/wavefront_plan.h:27-35
    _fields_ = [("dims", c_long_p), ("ndims", C.c_long), ("total_points", C.c_long),
                ("max_level", C.c_long), ("max_level_size", C.c_long),
                ("level_starts", c_long_p), ("level_offsets", c_long_p)]


class KMScan1DFwd(C.Structure):           # include/kmamba_km.h
    _fields_ = [(n, C.c_void_p) for n in ("x", "delta", "A", "Bm", "Cm", "y", "h0",
                                          "h_final", "h_hist")] + \
               [(n, C.c_long) for n in ("B", "L", "D", "N", "bc_sb", "bc_st", "bc_sd")] + \
               [("dtype", C.c_int), ("clamp", C.c_int), ("h_ckpt", C.c_void_p), ("z", C.c_void_p),
                ("Dskip", C.c_void_p)]


class KMScan1DBwd(C.Structure):           # include/kmamba_km.h
    _fields_ = [(n, C.c_void_p) for n in ("x", "delta", "A", "Bm", "Cm", "dy", "h0", "h_hist",
                                          "h_ckpt", "dx", "ddelta", "dA", "dB", "dC")] + \
               [(n, C.c_long) for n in ("B", "L", "D", "N", "bc_sb", "bc_st", "bc_sd")] + \
               [("dtype", C.c_int), ("clamp", C.c_int), ("workspace", C.c_void_p),
                ("workspace_bytes", C.c_size_t)]


KM_SCAN1D_CKPT_STEPS = 32
KM_EPI_NONE, KM_EPI_SOFTPLUS, KM_EPI_SILU = 0, 1, 2


class KMGemm(C.Structure):                # include/kmamba_km.h
    _fields_ = [(n, C.c_void_p) for n in ("A", "B", "C", "bias")] + \
               [(n, C.c_long) for n in ("M", "N", "K", "lda", "ldb", "ldc")] + \
               [("c_dtype", C.c_int), ("epilogue", C.c_int)]


class KMMamba1Weights(C.Structure):       # include/kmamba_km.h
    _fields_ = [(n, C.c_long) for n in ("dim", "d_inner", "d_state", "d_conv", "dt_rank")] + \
               [(n, C.c_void_p) for n in ("W_in", "conv_w", "conv_b", "W_x", "W_dt", "dt_bias",
                                          "A", "Dskip", "W_out")] + [("clamp", C.c_int)]


class MBMatrix(C.Structure):              # include/kmamba.h (ref include/kmamba.h:17-24)
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
               [("lambda_proj", MBMatrix), ("wavefront_plan", C.c_void_p)] + \
               [(n, C.POINTER(C.c_float)) for n in ("convnd_kernel", "convnd_bias", "hidden",
                                                   "delta", "scan_B", "scan_C", "scan_delta",
                                                   "scan_h")] + [("opt_state", C.c_void_p)]


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


VisitFn = C.CFUNCTYPE(C.c_int, c_long_p, C.c_long, C.c_long, C.c_long, C.c_void_p)


def _decl(name, restype, argtypes):
    fn = getattr(lib, name)
    fn.restype = restype
    fn.argtypes = argtypes
    return fn


# --- host-side topology / plan (run on the CPU, no GPU needed) -------------
wavefront_nd_validate_dims = _decl("wavefront_nd_validate_dims", C.c_int, [c_long_p, C.c_long])
wavefront_nd_total_points = _decl("wavefront_nd_total_points", C.c_long, [c_long_p, C.c_long])
wavefront_nd_max_level = _decl("wavefront_nd_max_level", C.c_long, [c_long_p, C.c_long])
wavefront_nd_row_major_offset = _decl("wavefront_nd_row_major_offset", C.c_long,
                                      [c_long_p, c_long_p, C.c_long])
wavefront_nd_level_size = _decl("wavefront_nd_level_size", C.c_long, [c_long_p, C.c_long, C.c_long])
wavefront_nd_for_level = _decl("wavefront_nd_for_level", C.c_int,
                               [c_long_p, C.c_long, C.c_long, c_long_p, VisitFn, C.c_void_p])
wavefront_nd_for_each_level = _decl("wavefront_nd_for_each_level", C.c_int,
                                    [c_long_p, C.c_long, c_long_p, VisitFn, C.c_void_p])
km_wavefront_plan_create = _decl("km_wavefront_plan_create", C.POINTER(KMWavefrontPlan),
                                 [c_long_p, C.c_long])
km_wavefront_plan_free = _decl("km_wavefront_plan_free", None, [C.POINTER(KMWavefrontPlan)])
km_wavefront_plan_matches_dims = _decl("km_wavefront_plan_matches_dims", C.c_int,
                                       [C.POINTER(KMWavefrontPlan), c_long_p, C.c_long])
km_wavefront_plan_level_size = _decl("km_wavefront_plan_level_size", C.c_long,
                                     [C.POINTER(KMWavefrontPlan), C.c_long])
km_wavefront_plan_level_offsets = _decl("km_wavefront_plan_level_offsets", c_long_p,
                                        [C.POINTER(KMWavefrontPlan), C.c_long])
km_spatial_dims_product = _decl("km_spatial_dims_product", C.c_int,
                                [c_long_p, C.c_long, C.POINTER(C.c_size_t)])
km_make_row_major_strides = _decl("km_make_row_major_strides", C.c_int, [c_long_p, C.c_long, c_long_p])
km_unravel_index = _decl("km_unravel_index", None, [C.c_long, c_long_p, c_long_p, C.c_long, c_long_p])
km_ravel_index = _decl("km_ravel_index", C.c_long, [c_long_p, c_long_p, c_long_p, C.c_long])
km_power_long = _decl("km_power_long", C.c_long, [C.c_long, C.c_long])
km_normalize_spatial_topology = _decl("km_normalize_spatial_topology", C.c_int,
                                      [c_long_p, c_long_p, C.c_size_t, C.c_int, c_long_p, C.c_long])

# --- backend / errors --------------------------------------------------------
kmamba_cuda_available = _decl("kmamba_cuda_available", C.c_int, [])
kmamba_cuda_device_count = _decl("kmamba_cuda_device_count", C.c_int, [])
kmamba_cuda_current_device = _decl("kmamba_cuda_current_device", C.c_int, [])
kmamba_backend_init = _decl("kmamba_backend_init", None, [])
kmamba_backend_select = _decl("kmamba_backend_select", C.c_int, [])
km_last_error_c = _decl("km_last_error", C.c_char_p, [])
km_clear_error = _decl("km_clear_error", None, [])
km_version = _decl("km_version", C.c_char_p, [])
km_device_bytes_held = _decl("km_device_bytes_held", C.c_size_t, [])
km_release_stream = _decl("km_release_stream", C.c_size_t, [C.c_void_p])

# --- scans -------------------------------------------------------------------
scan1d = _decl("scan1d", None, [C.POINTER(ScanParams)])
mamba_scan1d_forward = _decl("mamba_scan1d_forward", None, [C.POINTER(ScanParams)])
om_scan1d_forward = _decl("om_scan1d_forward", None,
                          [C.c_void_p] * 7 + [C.c_int] * 3)
mamba_scan1d_cuda_forward = _decl("mamba_scan1d_cuda_forward", None,
                                  [C.c_void_p] * 7 + [C.c_int] * 3)
km_scan1d_fwd_c = _decl("km_scan1d_fwd", C.c_int, [C.POINTER(KMScan1DFwd), C.c_void_p])
scan1d_backward = _decl("scan1d_backward", None, [C.POINTER(ScanBackwardParams)])
mamba_scan1d_backward = _decl("mamba_scan1d_backward", None, [C.POINTER(ScanBackwardParams)])
scan1d_backward_m1_shared_bc = _decl("scan1d_backward_m1_shared_bc", None,
                                     [C.POINTER(ScanBackwardSharedParams)])
mamba_scan1d_backward_m1_shared_bc = _decl("mamba_scan1d_backward_m1_shared_bc", None,
                                           [C.POINTER(ScanBackwardSharedParams)])
scan1d_backward_m1_shared_bc_asm = _decl("scan1d_backward_m1_shared_bc_asm", None,
                                         [C.POINTER(ScanBackwardSharedParams)])
scan1d_backward_m1_shared_bc_simple_asm = _decl("scan1d_backward_m1_shared_bc_simple_asm", None,
                                                [C.POINTER(ScanBackwardSharedParams)])
om_scan1d_backward = _decl("om_scan1d_backward", None, [C.c_void_p] * 12 + [C.c_int] * 3)
mamba_scan1d_cuda_backward = _decl("mamba_scan1d_cuda_backward", None,
                                   [C.c_void_p] * 12 + [C.c_int] * 3)
km_scan1d_bwd_c = _decl("km_scan1d_bwd", C.c_int, [C.POINTER(KMScan1DBwd), C.c_void_p])
km_scan1d_bwd_workspace_bytes = _decl("km_scan1d_bwd_workspace_bytes", C.c_size_t,
                                      [C.POINTER(KMScan1DBwd)])


def km_last_error() -> str:
    return km_last_error_c().decode()


def longs(values):
    arr = (C.c_long * len(values))(*values)
    return arr


def ptr(t):
    """Device (or host numpy) buffer address for the C ABI; None -> NULL."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    if hasattr(t, "ctypes"):
        return t.ctypes.data
    raise TypeError(type(t))


def check(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"{what} failed: {km_last_error()}")


def stream_handle(stream=None):
    """hipStream_t of a torch stream (current stream when None)."""
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _need(t, name, *, shape=None, dtype=None, optional=False):
    """Checks a torch tensor argument before its address goes to the C ABI:
    contiguous, and of the given shape and dtype (the device is checked by
    _on_gpu once every argument passed these checks). Raises ValueError
    naming the argument otherwise (a wrong dtype or stride would make the
    kernel read or write past the tensor)."""
    import torch
    if t is None:
        if optional:
            return
        raise ValueError(f"{name} is required")
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch tensor")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _on_gpu(**tensors):
    """Every given (non-None) tensor must live on the GPU."""
    for name, t in tensors.items():
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"{name} must be a GPU tensor")


def _scan1d_io(x, A, Bm, Cm, bc_strides):
    """Validates the operands common to the Scan1D forward and backward and
    returns (B, L, D, N, io dtype, KMDtype, bc_strides)."""
    import torch
    _need(x, "x")
    if x.dim() != 3:
        raise ValueError(f"x must be [B, L, D], got shape {tuple(x.shape)}")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"x has dtype {x.dtype}; fp32 or bf16 expected")
    Bsz, L, D = x.shape
    _need(A, "A", dtype=torch.float32)
    if A.dim() != 2 or A.shape[0] != D:
        raise ValueError(f"A must be [D={D}, N], got shape {tuple(A.shape)}")
    N = A.shape[1]
    io = x.dtype
    if bc_strides is None:
        _need(Bm, "Bm", shape=(Bsz, L, N), dtype=io)
        _need(Cm, "Cm", shape=(Bsz, L, N), dtype=io)
        bc_strides = (L * N, N, 0)
    else:
        sb, st, sd = (int(v) for v in bc_strides)
        if min(sb, st, sd) < 0:
            raise ValueError("bc_strides must be non-negative")
        need = 0 if L == 0 else (Bsz - 1) * sb + (L - 1) * st + (D - 1) * sd + N
        for t, name in ((Bm, "Bm"), (Cm, "Cm")):
            _need(t, name, dtype=io)
            if t.numel() < need:
                raise ValueError(f"{name} holds {t.numel()} elements; bc_strides address {need}")
        if Bm.shape != Cm.shape:
            raise ValueError(f"Cm shape {tuple(Cm.shape)} differs from Bm {tuple(Bm.shape)}")
    return Bsz, L, D, N, io, (KM_BF16 if io == torch.bfloat16 else KM_F32), bc_strides


def scan1d_fwd_args(x, delta, A, Bm, Cm, y, *, h0=None, h_final=None, h_hist=None, h_ckpt=None,
                    bc_strides=None, clamp=True, z=None, Dskip=None):
    """KMScan1DFwd over torch device tensors.

    x, delta, y: [B, L, D] (one dtype: fp32 or bf16); A: [D, N] fp32;
    Bm/Cm: [B, L, N] shared over channels (default strides) or any layout
    described by bc_strides = (sb, st, sd) in elements with N contiguous;
    h0 / h_final [B, D, N], h_hist [B, L, D, N], h_ckpt [B, ceil(L/32), D, N]
    fp32; z [B, L, D] as x; Dskip [D] fp32. Every tensor must be contiguous
    and on the GPU (ValueError otherwise).
    """
    import torch
    Bsz, L, D, N, io, dt, bc_strides = _scan1d_io(x, A, Bm, Cm, bc_strides)
    _need(delta, "delta", shape=x.shape, dtype=io)
    _need(y, "y", shape=x.shape, dtype=io, optional=True)
    _need(z, "z", shape=x.shape, dtype=io, optional=True)
    _need(Dskip, "Dskip", shape=(D,), dtype=torch.float32, optional=True)
    _need(h0, "h0", shape=(Bsz, D, N), dtype=torch.float32, optional=True)
    _need(h_final, "h_final", shape=(Bsz, D, N), dtype=torch.float32, optional=True)
    _need(h_hist, "h_hist", shape=(Bsz, L, D, N), dtype=torch.float32, optional=True)
    nck = (L + KM_SCAN1D_CKPT_STEPS - 1) // KM_SCAN1D_CKPT_STEPS
    _need(h_ckpt, "h_ckpt", shape=(Bsz, nck, D, N), dtype=torch.float32, optional=True)
    _on_gpu(x=x, delta=delta, A=A, Bm=Bm, Cm=Cm, y=y, z=z, Dskip=Dskip, h0=h0, h_final=h_final,
            h_hist=h_hist, h_ckpt=h_ckpt)
    return KMScan1DFwd(ptr(x), ptr(delta), ptr(A), ptr(Bm), ptr(Cm), ptr(y), ptr(h0),
                       ptr(h_final), ptr(h_hist), Bsz, L, D, N, *bc_strides, dt, int(clamp),
                       ptr(h_ckpt), ptr(z), ptr(Dskip))


def scan1d_fwd(x, delta, A, Bm, Cm, y, *, stream=None, **kw):
    """km_scan1d_fwd on torch device tensors (arguments as scan1d_fwd_args)."""
    args = scan1d_fwd_args(x, delta, A, Bm, Cm, y, **kw)
    check(km_scan1d_fwd_c(C.byref(args), C.c_void_p(stream_handle(stream))), "km_scan1d_fwd")


def scan1d_bwd_args(x, delta, A, Bm, Cm, dy, dx, ddelta, dA, dB, dC, *, h0=None, h_hist=None,
                    h_ckpt=None, bc_strides=None, clamp=True, workspace=None):
    """KMScan1DBwd over torch device tensors (layouts as scan1d_fwd; dx,
    ddelta, dy as x; dA [D, N] fp32; dB, dC [B, L, N] when B/C are shared
    over channels, else the shape of Bm). Raises ValueError on a tensor of
    the wrong device, dtype, shape or layout."""
    import torch
    Bsz, L, D, N, io, dt, bc_strides = _scan1d_io(x, A, Bm, Cm, bc_strides)
    for t, name in ((delta, "delta"), (dy, "dy"), (dx, "dx"), (ddelta, "ddelta")):
        _need(t, name, shape=x.shape, dtype=io)
    _need(dA, "dA", shape=(D, N), dtype=torch.float32)
    gshape = (Bsz, L, N) if bc_strides[2] == 0 else tuple(Bm.shape)
    _need(dB, "dB", shape=gshape, dtype=io)
    _need(dC, "dC", shape=gshape, dtype=io)
    _need(h0, "h0", shape=(Bsz, D, N), dtype=torch.float32, optional=True)
    _need(h_hist, "h_hist", shape=(Bsz, L, D, N), dtype=torch.float32, optional=True)
    nck = (L + KM_SCAN1D_CKPT_STEPS - 1) // KM_SCAN1D_CKPT_STEPS
    _need(h_ckpt, "h_ckpt", shape=(Bsz, nck, D, N), dtype=torch.float32, optional=True)
    if workspace is not None:
        _need(workspace, "workspace")
    _on_gpu(x=x, delta=delta, A=A, Bm=Bm, Cm=Cm, dy=dy, dx=dx, ddelta=ddelta, dA=dA, dB=dB, dC=dC,
            h0=h0, h_hist=h_hist, h_ckpt=h_ckpt, workspace=workspace)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    return KMScan1DBwd(ptr(x), ptr(delta), ptr(A), ptr(Bm), ptr(Cm), ptr(dy), ptr(h0), ptr(h_hist),
                       ptr(h_ckpt), ptr(dx), ptr(ddelta), ptr(dA), ptr(dB), ptr(dC),
                       Bsz, L, D, N, *bc_strides, dt, int(clamp), ptr(workspace), ws_bytes)


def scan1d_bwd(x, delta, A, Bm, Cm, dy, dx, ddelta, dA, dB, dC, *, stream=None, **kw):
    """km_scan1d_bwd on torch device tensors."""
    args = scan1d_bwd_args(x, delta, A, Bm, Cm, dy, dx, ddelta, dA, dB, dC, **kw)
    check(km_scan1d_bwd_c(C.byref(args), C.c_void_p(stream_handle(stream))), "km_scan1d_bwd")


# --- ConvND -------------------------------------------------------------------
convnd_kernel_volume = _decl("convnd_kernel_volume", C.c_long, [C.c_long, C.c_long])
convnd_forward_wavefront = _decl("convnd_forward_wavefront", None,
                                 [C.POINTER(ConvNDParams), C.POINTER(KMWavefrontPlan)])
convnd_backward_wavefront = _decl("convnd_backward_wavefront", None,
                                  [C.POINTER(ConvNDParams), C.POINTER(KMWavefrontPlan)])
convnd = _decl("convnd", None, [C.POINTER(ConvNDParams), C.c_int])
om_convnd_forward = _decl("om_convnd_forward", C.c_int, [C.POINTER(ConvNDParams)])
om_convnd_backward = _decl("om_convnd_backward", C.c_int, [C.POINTER(ConvNDParams)])
km_convnd_fwd_c = _decl("km_convnd_fwd", C.c_int, [C.POINTER(ConvNDParams), C.c_long, C.c_void_p])
km_convnd_bwd_c = _decl("km_convnd_bwd", C.c_int, [C.POINTER(ConvNDParams), C.c_long, C.c_void_p])


def convnd_params(dims, inp=None, kernel=None, bias=None, output=None, dy=None, dinput=None,
                  dkernel=None, dbias=None, *, D, K):
    """ConvNDParams over buffers (torch device tensors or numpy arrays);
    returns (params, keepalive)."""
    dd = longs(dims)
    p = ConvNDParams(ptr(inp), ptr(kernel), ptr(bias), ptr(output), ptr(dy), ptr(dinput),
                     ptr(dkernel), ptr(dbias), dd, len(dims), D, K)
    return p, dd


def convnd_fwd(dims, inp, kernel, bias, output, *, batch=1, stream=None):
    """km_convnd_fwd: inp/output [batch, P, D] (or [P, D]); kernel [K^nd, D]."""
    D = inp.shape[-1]
    K = int(round(kernel.shape[0] ** (1.0 / len(dims))))
    p, _keep = convnd_params(dims, inp, kernel, bias, output, D=D, K=K)
    check(km_convnd_fwd_c(C.byref(p), batch, C.c_void_p(stream_handle(stream))), "km_convnd_fwd")


def convnd_bwd(dims, inp, kernel, dy, dinput, dkernel, dbias, *, batch=1, stream=None):
    D = inp.shape[-1]
    K = int(round(kernel.shape[0] ** (1.0 / len(dims))))
    p, _keep = convnd_params(dims, inp, kernel, None, None, dy, dinput, dkernel, dbias, D=D, K=K)
    check(km_convnd_bwd_c(C.byref(p), batch, C.c_void_p(stream_handle(stream))), "km_convnd_bwd")


# --- bf16 GEMM and the Mamba-1 block -------------------------------------------
km_gemm_bf16_c = _decl("km_gemm_bf16", C.c_int, [C.POINTER(KMGemm), C.c_void_p])
km_mamba1_block_workspace_bytes = _decl("km_mamba1_block_workspace_bytes", C.c_size_t,
                                        [C.POINTER(KMMamba1Weights), C.c_long, C.c_long])
km_mamba1_block_fwd_c = _decl("km_mamba1_block_fwd", C.c_int,
                              [C.POINTER(KMMamba1Weights), C.c_void_p, C.c_void_p, C.c_long,
                               C.c_long, C.c_void_p, C.c_size_t, C.c_void_p])


def gemm_bf16(A, B, Cout, *, bias=None, epilogue=KM_EPI_NONE, M=None, N=None, K=None, lda=None,
              ldb=None, ldc=None, stream=None):
    """km_gemm_bf16: Cout = epi(A . B^T + bias); A [M, K], B [N, K] bf16
    (row strides lda, ldb), Cout [M, N] fp32 or bf16 (row stride ldc)."""
    import torch
    M = A.shape[0] if M is None else M
    K = A.shape[1] if K is None else K
    N = B.shape[0] if N is None else N
    g = KMGemm(ptr(A), ptr(B), ptr(Cout), ptr(bias), M, N, K,
               A.stride(0) if lda is None else lda, B.stride(0) if ldb is None else ldb,
               Cout.stride(0) if ldc is None else ldc,
               KM_BF16 if Cout.dtype == torch.bfloat16 else KM_F32, epilogue)
    check(km_gemm_bf16_c(C.byref(g), C.c_void_p(stream_handle(stream))), "km_gemm_bf16")


def mamba1_weights(w, clamp=True):
    """KMMamba1Weights from a dict of torch device tensors (keys as the
    struct fields; conv_b and Dskip optional)."""
    di, dim = w["W_in"].shape[0] // 2, w["W_in"].shape[1]
    N = w["A"].shape[1]
    return KMMamba1Weights(dim, di, N, w["conv_w"].shape[0], w["W_dt"].shape[1],
                           ptr(w["W_in"]), ptr(w["conv_w"]), ptr(w.get("conv_b")), ptr(w["W_x"]),
                           ptr(w["W_dt"]), ptr(w["dt_bias"]), ptr(w["A"]), ptr(w.get("Dskip")),
                           ptr(w["W_out"]), int(clamp))


def mamba1_block_fwd(w, x, out, *, workspace=None, clamp=True, stream=None):
    """km_mamba1_block_fwd: x, out [B, L, dim] bf16."""
    Bsz, L, _ = x.shape
    ws = mamba1_weights(w, clamp)
    nb = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(km_mamba1_block_fwd_c(C.byref(ws), ptr(x), ptr(out), Bsz, L, ptr(workspace), nb,
                                C.c_void_p(stream_handle(stream))), "km_mamba1_block_fwd")


# --- Mamba-3 block -------------------------------------------------------------
mamba_block_create = _decl("mamba_block_create", C.POINTER(MambaBlock), [C.POINTER(MBConfig)])
mamba_block_free = _decl("mamba_block_free", None, [C.POINTER(MambaBlock)])
mamba_block_init = _decl("mamba_block_init", None, [C.POINTER(MambaBlock)])
mamba_block_forward = _decl("mamba_block_forward", None,
                            [C.POINTER(MambaBlock), C.c_void_p, C.c_void_p, C.c_size_t])


# --- The stacked model ----------------------------------------------------------
kmamba_create = _decl("kmamba_create", C.POINTER(KMamba), [C.POINTER(KMambaConfig)])
kmamba_free = _decl("kmamba_free", None, [C.POINTER(KMamba)])
kmamba_init = _decl("kmamba_init", C.c_int, [C.POINTER(KMamba), C.c_uint32])
kmamba_save = _decl("kmamba_save", C.c_int, [C.POINTER(KMamba), C.c_char_p])
kmamba_load = _decl("kmamba_load", C.POINTER(KMamba),
                    [C.c_char_p, C.c_int, C.POINTER(MBOptimConfig), C.c_float, C.c_float])
kmamba_forward = _decl("kmamba_forward", C.c_int, [C.POINTER(KMamba), C.c_void_p, C.c_void_p])


# --- ScanND / Scan2D ----------------------------------------------------------
scannd_validate = _decl("scannd_validate", C.c_int, [C.POINTER(ScanNDParams)])
scannd_ref = _decl("scannd_ref", C.c_int, [C.POINTER(ScanNDParams)])
scannd_ref_with_plan = _decl("scannd_ref_with_plan", C.c_int,
                             [C.POINTER(ScanNDParams), C.POINTER(KMWavefrontPlan)])
scannd = _decl("scannd", C.c_int, [C.POINTER(ScanNDParams)])
om_scannd_forward = _decl("om_scannd_forward", C.c_int, [C.POINTER(ScanNDParams)])
mamba_scannd_cuda_forward = _decl("mamba_scannd_cuda_forward", C.c_int, [C.POINTER(ScanNDParams)])
km_scannd_fwd_c = _decl("km_scannd_fwd", C.c_int, [C.POINTER(ScanNDParams), C.c_void_p])
km_scannd_fwd_noalloc_c = _decl("km_scannd_fwd_noalloc", C.c_int,
                                  [C.POINTER(ScanNDParams), C.c_void_p])
km_scannd_status_c = _decl("km_scannd_status", C.c_int, [C.c_void_p])
scan2d = _decl("scan2d", None, [C.POINTER(Scan2DParams)])
mamba_scan2d_forward = _decl("mamba_scan2d_forward", None, [C.POINTER(Scan2DParams)])


def scannd_params(dims, x, A, B, Cm, delta, h, y, theta=None, lam=None):
    """ScanNDParams over buffers (torch device tensors or numpy arrays), with
    the optional Mamba-3 theta [D/2] and lambda [P]. Returns (params,
    keepalive)."""
    dd = longs(dims)
    D, M = A.shape[-2], A.shape[-1]
    p = ScanNDParams(C.cast(dd, c_long_p), len(dims), D, M, ptr(x), ptr(A), ptr(B), ptr(Cm),
                     ptr(delta), ptr(h), ptr(y), None if theta is None else ptr(theta),
                     None if lam is None else ptr(lam))
    return p, dd


class KMScanNDBwd(C.Structure):           # include/kmamba_km.h (no reference counterpart)
    _fields_ = [("dims", c_long_p), ("ndims", C.c_long), ("D", C.c_long), ("M", C.c_long)] + \
               [(n, C.c_void_p) for n in ("x", "A", "B", "C", "delta", "h", "dy", "dx", "ddelta",
                                          "dA", "dB", "dC", "workspace")] + \
               [("workspace_bytes", C.c_size_t)]


km_scannd_bwd_workspace_bytes = _decl("km_scannd_bwd_workspace_bytes", C.c_size_t,
                                      [C.POINTER(KMScanNDBwd)])
km_scannd_bwd_c = _decl("km_scannd_bwd", C.c_int, [C.POINTER(KMScanNDBwd), C.c_void_p])


def scannd_bwd(dims, x, A, B, Cm, delta, h, dy, dx, ddelta, dA, dB, dC, *, workspace=None,
               stream=None):
    """km_scannd_bwd on torch device tensors (layouts as scannd_fwd)."""
    dd = longs(dims)
    nd, D, M = A.shape
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    args = KMScanNDBwd(dd, len(dims), D, M, ptr(x), ptr(A), ptr(B), ptr(Cm), ptr(delta), ptr(h),
                       ptr(dy), ptr(dx), ptr(ddelta), ptr(dA), ptr(dB), ptr(dC), ptr(workspace),
                       ws_bytes)
    check(km_scannd_bwd_c(C.byref(args), C.c_void_p(stream_handle(stream))), "km_scannd_bwd")


def scannd_fwd(dims, x, A, B, Cm, delta, h, y, stream=None, theta=None, lam=None):
    """km_scannd_fwd (scannd_ref semantics, the Mamba-3 branch when lam is
    given) on torch device tensors."""
    p, keep = scannd_params(dims, x, A, B, Cm, delta, h, y, theta, lam)
    check(km_scannd_fwd_c(C.byref(p), C.c_void_p(stream_handle(stream))), "km_scannd_fwd")
    return keep


def scannd_status(stream=None) -> int:
    """km_scannd_status: waits for the stream; 0 when the latest ScanND
    forward or backward on it is exact, 1 when a dataflow wait gave up (NaN
    tiles)."""
    rc = km_scannd_status_c(C.c_void_p(stream_handle(stream)))
    if rc < 0:
        raise RuntimeError(f"km_scannd_status: {km_last_error()}")
    return rc


def scannd_fwd_noalloc(dims, x, A, B, Cm, delta, h, y, stream=None, theta=None, lam=None):
    """km_scannd_fwd_noalloc: km_scannd_fwd with its dataflow state in the
    library's fixed device array (no allocation)."""
    p, keep = scannd_params(dims, x, A, B, Cm, delta, h, y, theta, lam)
    check(km_scannd_fwd_noalloc_c(C.byref(p), C.c_void_p(stream_handle(stream))),
          "km_scannd_fwd_noalloc")
    return keep

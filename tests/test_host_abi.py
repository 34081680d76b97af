"""CPU tests of libkmamba's host side: C-ABI exports, the wavefront plan /
enumeration / topology code (bit-exact against the compiled reference and the
oracle), and the behaviour of the compute entry points when no GPU is usable.
"""
import ctypes as C
import os
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import kmamba as K
import oracle as O

ROOT = Path(__file__).resolve().parent.parent
needs_ref = pytest.mark.skipif(not O.REF_AVAILABLE, reason="oracle/_ref not built (reference tree absent)")


def header_functions():
    """Names of every function (and extern object) declared in include/*.h."""
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        text = re.sub(r"^\s*#.*?(?<!\\)$", "", text, flags=re.M | re.S)
        text = re.sub(r"typedef\s+(struct|enum)\s*\{.*?\}\s*\w+\s*;", "", text, flags=re.S)
        text = re.sub(r"typedef[^;]*;", "", text)
        text = text.replace('extern "C" {', "").replace("}", " ")
        for stmt in text.split(";"):
            stmt = " ".join(stmt.split())
            if not stmt or "{" in stmt:
                continue
            m = re.match(r"^(?:extern\s+)?[\w\s\*]*?\b(\w+)\s*\(", stmt)
            if m:
                names.add(m.group(1))
            elif stmt.startswith("extern "):
                names.add(stmt.split()[-1].strip("*"))
    return sorted(names)


def test_headers_parse():
    names = header_functions()
    for must in ("scan1d", "om_scan1d_forward", "scannd", "km_wavefront_plan_create",
                 "convnd", "kmamba_backend_preference", "km_scan1d_fwd"):
        assert must in names, must


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", str(K.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [n for n in header_functions() if n not in exported]
    assert not missing, f"declared in include/*.h but not exported: {missing}"


# ---------------------------------------------------------------------------
# Plan / wavefront / topology
# ---------------------------------------------------------------------------
def product_plan(dims):
    dd = K.longs(dims)
    pl = K.km_wavefront_plan_create(dd, len(dims))
    if not pl:
        return None
    p = pl.contents
    starts = np.ctypeslib.as_array(p.level_starts, shape=(p.max_level + 2,)).copy()
    offs = np.ctypeslib.as_array(p.level_offsets, shape=(p.total_points,)).copy()
    meta = (p.ndims, p.total_points, p.max_level, p.max_level_size,
            list(np.ctypeslib.as_array(p.dims, shape=(p.ndims,))))
    assert K.km_wavefront_plan_matches_dims(pl, dd, len(dims)) == 1
    for lvl in (0, p.max_level // 2, p.max_level):
        size = K.km_wavefront_plan_level_size(pl, lvl)
        assert size == starts[lvl + 1] - starts[lvl]
        lo = K.km_wavefront_plan_level_offsets(pl, lvl)
        if size > 0:
            np.testing.assert_array_equal(np.ctypeslib.as_array(lo, shape=(size,)),
                                          offs[starts[lvl]:starts[lvl + 1]])
    assert K.km_wavefront_plan_level_size(pl, -1) == -1
    assert K.km_wavefront_plan_level_size(pl, p.max_level + 1) == -1
    assert not K.km_wavefront_plan_level_offsets(pl, p.max_level + 1)
    K.km_wavefront_plan_free(pl)
    return starts, offs, meta


PLAN_DIMS = [(1,), (7,), (3, 4), (2, 3, 2), (4, 1, 3), (2, 2, 2, 3), (16, 16), (5, 3, 2, 2, 2),
             (1, 1, 1), (3, 1, 4, 1, 5, 1, 2, 2)]


@pytest.mark.parametrize("dims", PLAN_DIMS)
def test_plan_matches_oracle(dims):
    starts, offs, meta = product_plan(dims)
    o_starts, o_offs, o_mls = O.plan_tables(dims)
    np.testing.assert_array_equal(starts, o_starts)
    np.testing.assert_array_equal(offs, o_offs)
    assert meta[3] == o_mls and meta[1] == int(np.prod(dims))


@needs_ref
@pytest.mark.parametrize("dims", PLAN_DIMS + [(256, 256), (64, 64, 64), (512, 512)])
def test_plan_bit_exact_vs_reference(dims):
    starts, offs, meta = product_plan(dims)
    r_starts, r_offs, r_mls = O.plan_tables(dims, use_ref=True)
    np.testing.assert_array_equal(starts, r_starts)
    np.testing.assert_array_equal(offs, r_offs)
    assert meta[3] == r_mls


def test_plan_config_shapes():
    # Plan shapes of the benchmark grids: 256^2 (Scan2D), 64^3 (ScanND 3D), 512^2 (ConvND 2D).
    for dims, maxl, mls in (((256, 256), 510, 256), ((64, 64, 64), 189, None), ((512, 512), 1022, 512)):
        starts, offs, meta = product_plan(dims)
        assert meta[2] == maxl
        if mls:
            assert meta[3] == mls
        assert starts[-1] == int(np.prod(dims))
    assert not K.km_wavefront_plan_create(K.longs((3, 0)), 2)
    assert not K.km_wavefront_plan_create(K.longs((3,)), 0)


def _visits(lib_fn, dims, level=None):
    seen = []

    @K.VisitFn
    def cb(idx, nd, lvl, ordinal, user):
        seen.append((tuple(idx[i] for i in range(nd)), lvl, ordinal))
        return 0

    dd = K.longs(dims)
    rc = lib_fn(dd, len(dims), level, None, cb, None) if level is not None else \
        lib_fn(dd, len(dims), None, cb, None)
    return rc, seen


@pytest.mark.parametrize("dims", [(3, 4), (2, 3, 2), (4, 1, 3), (5,), (2, 2, 3, 2)])
def test_for_each_level_order_and_coverage(dims):
    rc, seen = _visits(K.wavefront_nd_for_each_level, dims)
    assert rc == 0
    offs = [K.wavefront_nd_row_major_offset(K.longs(dims), K.longs(i), len(dims)) for i, _, _ in seen]
    assert sorted(offs) == list(range(int(np.prod(dims))))
    _, o_offs, _ = O.plan_tables(dims)
    assert offs == list(o_offs)                       # level order, ascending offsets in a level
    for i, lvl, _ in seen:
        assert sum(i) == lvl
    prev = None
    for _, lvl, ordinal in seen:                      # ordinals restart at each level
        assert ordinal == (0 if lvl != prev else last + 1)
        prev, last = lvl, ordinal


@needs_ref
@pytest.mark.parametrize("dims", [(3, 4), (2, 3, 2), (4, 1, 3), (2, 2, 3, 2), (6, 5, 4)])
def test_for_level_visits_equal_reference(dims):
    O.ref.wavefront_nd_for_level.restype = C.c_int
    O.ref.wavefront_nd_for_level.argtypes = [K.c_long_p, C.c_long, C.c_long, K.c_long_p, K.VisitFn,
                                             C.c_void_p]
    maxl = sum(d - 1 for d in dims)
    for lvl in range(maxl + 1):
        a = _visits(K.wavefront_nd_for_level, dims, lvl)
        b = _visits(O.ref.wavefront_nd_for_level, dims, lvl)
        assert a == b
        assert K.wavefront_nd_level_size(K.longs(dims), len(dims), lvl) == \
            O.ref.wavefront_nd_level_size(O.longs(dims), len(dims), lvl)


def test_for_level_early_stop_and_invalid():
    # tests/unit/test_wavefront_nd.c:212-248.
    count = [0]

    @K.VisitFn
    def stop_after_two(idx, nd, lvl, ordinal, user):
        count[0] += 1
        return 77 if count[0] >= 2 else 0

    assert K.wavefront_nd_for_level(K.longs((3, 4)), 2, 3, None, stop_after_two, None) == 77
    assert count[0] == 2
    bad = K.longs((3, 0))
    assert K.wavefront_nd_validate_dims(bad, 2) == 0
    assert K.wavefront_nd_total_points(bad, 2) == -1
    assert K.wavefront_nd_max_level(bad, 2) == -1
    assert K.wavefront_nd_for_each_level(bad, 2, None, stop_after_two, None) == -1
    assert K.wavefront_nd_level_size(K.longs((3, 4)), 2, 6) == -1
    assert K.wavefront_nd_row_major_offset(K.longs((2, 3, 2)), K.longs((1, 2, 1)), 3) == 11
    assert K.wavefront_nd_row_major_offset(K.longs((2, 3, 2)), K.longs((1, 3, 1)), 3) == -1
    big = K.longs((1 << 40, 1 << 40))
    assert K.wavefront_nd_total_points(big, 2) == -1          # overflow detected
    # Inclusion-exclusion: C(1502,2) - 3*C(502,2) points of [0,999]^3 sum to 1500.
    assert K.wavefront_nd_level_size(K.longs((1000, 1000, 1000)), 3, 1500) == \
        1502 * 1501 // 2 - 3 * (502 * 501 // 2)


def test_topology_helpers():
    dims = K.longs((2, 3, 4))
    st = (C.c_long * 3)()
    assert K.km_make_row_major_strides(dims, 3, st) == 1 and list(st) == [12, 4, 1]
    co = (C.c_long * 3)()
    K.km_unravel_index(17, dims, st, 3, co)
    assert list(co) == [1, 1, 1]
    assert K.km_ravel_index(co, dims, st, 3) == 17
    co[1] = 3
    assert K.km_ravel_index(co, dims, st, 3) == -1
    assert K.km_power_long(0, 0) == 0 and K.km_power_long(3, 4) == 81 and K.km_power_long(2, -1) == 0
    prod = C.c_size_t()
    assert K.km_spatial_dims_product(dims, 3, C.byref(prod)) == 1 and prod.value == 24
    nd = C.c_long(0)
    sd = (C.c_long * 8)()
    cn = C.c_long(0)
    assert K.km_normalize_spatial_topology(C.byref(nd), sd, 12, 1, C.byref(cn), 3) == 0
    assert nd.value == 1 and sd[0] == 12 and cn.value == 1
    nd2 = C.c_long(2)
    sd2 = (C.c_long * 8)(3, 5)
    assert K.km_normalize_spatial_topology(C.byref(nd2), sd2, 12, 0, None, 0) == -1


# ---------------------------------------------------------------------------
# Backend selection and behaviour without a GPU
# ---------------------------------------------------------------------------
def _run_py(code, env_extra):
    env = dict(os.environ, **env_extra)
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env,
                          cwd=str(ROOT), timeout=120)


def test_backend_env_parsing():
    code = ("import sys; sys.path[:0]=['k-mamba_amd']; import kmamba as K; "
            "K.kmamba_backend_init(); print(int(K.lib.kmamba_backend_preference if False else 0)); "
            "import ctypes; v=ctypes.c_int.in_dll(K.lib,'kmamba_backend_preference'); print(v.value)")
    for val, want in (("cpu", 1), ("GPU", 2), ("cuda", 2), ("auto", 0), ("weird", 0)):
        out = _run_py(code, {"KMAMBA_BACKEND": val})
        assert out.returncode == 0, out.stderr
        assert out.stdout.split()[-1] == str(want), (val, out.stdout)


def test_cpu_backend_request_fails_loudly():
    # With KMAMBA_BACKEND=cpu the library refuses to compute (no CPU path)
    # and leaves outputs untouched instead of producing something else.
    code = ("import sys, ctypes as C, numpy as np; sys.path[:0]=['k-mamba_amd']; import kmamba as K\n"
            "x=np.ones((4,3),np.float32); y=np.full((4,3),7,np.float32); A=-np.ones((3,2),np.float32)\n"
            "B=np.ones((4,3,2),np.float32); h=np.zeros((3,2),np.float32)\n"
            "p=K.ScanParams(K.ptr(x),K.ptr(A),K.ptr(B),K.ptr(B),K.ptr(x),K.ptr(h),K.ptr(y),4,3,2)\n"
            "K.scan1d(C.byref(p)); print(K.km_last_error()); print(float(y.sum()))")
    out = _run_py(code, {"KMAMBA_BACKEND": "cpu"})
    assert out.returncode == 0, out.stderr
    lines = out.stdout.strip().splitlines()
    assert "no CPU compute path" in lines[-2]
    assert lines[-1] == "84.0"


@pytest.mark.skipif(K.kmamba_cuda_available() == 1, reason="a GPU is present")
def test_no_gpu_reports_error():
    assert K.kmamba_cuda_device_count() == 0
    assert K.kmamba_backend_select() == K.KMAMBA_BACKEND_CPU
    args = K.KMScan1DFwd()
    args.B = args.L = args.D = args.N = 1
    args.x = args.delta = args.A = args.Bm = args.Cm = args.y = 1
    assert K.km_scan1d_fwd_c(C.byref(args), None) == -1
    assert "HIP device" in K.km_last_error()


# ---------------------------------------------------------------------------
# Mamba-3 block: create / init / free (host side, no GPU needed)
# ---------------------------------------------------------------------------
def _mb_cfg(lib_cfg_cls, dim=12, N=6, L=10, R=2):
    cfg = lib_cfg_cls()
    cfg.dim, cfg.state_size, cfg.seq_len, cfg.mimo_rank = dim, N, L, R
    cfg.dt_scale, cfg.dt_min, cfg.dt_max = 0.1, 1e-3, 0.1
    return cfg


def test_mamba_block_layout_matches_reference_header():
    # MBConfig / MambaBlock field offsets (ref include/kmamba.h:27-54, :116-150).
    assert C.sizeof(K.MBConfig) == C.sizeof(O.MBConfig) == 152
    assert C.sizeof(K.MambaBlock) == C.sizeof(O.MambaBlock)
    for name, _ in K.MambaBlock._fields_:
        assert getattr(K.MambaBlock, name).offset == getattr(O.MambaBlock, name).offset, name


@needs_ref
@pytest.mark.parametrize("dim,N,L,R", [(12, 6, 10, 2), (8, 16, 4, 1), (5, 3, 7, 0)])
def test_mamba_block_create_and_init_match_reference(dim, N, L, R):
    libc = C.CDLL(None)
    ours = K.mamba_block_create(C.byref(_mb_cfg(K.MBConfig, dim, N, L, R)))
    theirs = O.ref.mamba_block_create(C.byref(_mb_cfg(O.MBConfig, dim, N, L, R)))
    assert ours and theirs
    a, b = ours.contents, theirs.contents
    assert a.config.mimo_rank == b.config.mimo_rank == max(R, 1)
    assert a.config.spatial_ndims == b.config.spatial_ndims == 1
    assert a.config.spatial_dims[0] == b.config.spatial_dims[0] == L
    for name in ("W_in", "W_out", "A_log", "W_B", "W_C", "delta_proj", "lambda_proj"):
        ma, mb = getattr(a, name), getattr(b, name)
        assert (ma.rows, ma.cols) == (mb.rows, mb.cols), name
    # same rand() stream -> bit-identical initial parameters
    libc.srand(1234)
    K.mamba_block_init(ours)
    libc.srand(1234)
    O.ref.mamba_block_init(theirs)
    pa, pb = O.block_params(C.cast(ours, C.POINTER(O.MambaBlock))), O.block_params(theirs)
    for k in pa:
        np.testing.assert_array_equal(pa[k], pb[k], err_msg=k)
    K.mamba_block_free(ours)
    O.ref.mamba_block_free(theirs)


def test_mamba_block_create_rejects_bad_topology():
    cfg = _mb_cfg(K.MBConfig, L=10)
    cfg.spatial_ndims = 2
    cfg.spatial_dims[0], cfg.spatial_dims[1] = 3, 4          # 12 != seq_len
    assert not K.mamba_block_create(C.byref(cfg))
    assert "topology" in K.km_last_error()
    K.mamba_block_free(None)


# ---------------------------------------------------------------------------
# The stacked model: layout, create / init / save / load (host side)
# ---------------------------------------------------------------------------
REF_INC = Path("/root/reference/include")
MODEL_STRUCTS = ("KMambaConfig", "MBOptimConfig", "KMamba")


@pytest.mark.skipif(not (REF_INC / "kmamba.h").exists(), reason="reference headers absent")
def test_kmamba_layout_matches_reference_header(tmp_path):
    # Sizes and field offsets as gcc lays out the reference's own header
    # (include/kmamba.h:159-223, include/kmamba_kernels.h:78-85, CPU build).
    src = ['#include <stdio.h>', '#include <stddef.h>', '#include "kmamba.h"', 'int main(void) {']
    for cls in MODEL_STRUCTS:
        src.append(f'printf("{cls} %zu\\n", sizeof({cls}));')
        for name, _ in getattr(K, cls)._fields_:
            src.append(f'printf("{cls}.{name} %zu\\n", offsetof({cls}, {name}));')
    src.append("return 0; }")
    (tmp_path / "lay.c").write_text("\n".join(src) + "\n")
    subprocess.run(["gcc", "-w", f"-I{REF_INC}", f"-I{REF_INC.parent / 'cpu' / 'include'}",
                    str(tmp_path / "lay.c"), "-o", str(tmp_path / "lay")], check=True)
    got = dict(line.rsplit(" ", 1) for line in
               subprocess.run([str(tmp_path / "lay")], capture_output=True, text=True,
                              check=True).stdout.split("\n") if line)
    for cls in MODEL_STRUCTS:
        ct = getattr(K, cls)
        assert int(got[cls]) == C.sizeof(ct), cls
        for name, _ in ct._fields_:
            assert int(got[f"{cls}.{name}"]) == getattr(ct, name).offset, (cls, name)


def _model_arrays(m):
    return O.model_params(C.cast(m, C.POINTER(O.KMamba)))


def _assert_same_params(pa, pb):
    np.testing.assert_array_equal(pa[0], pb[0], err_msg="embedding")
    np.testing.assert_array_equal(pa[1], pb[1], err_msg="head")
    assert len(pa[2]) == len(pb[2])
    for la, lb in zip(pa[2], pb[2]):
        for k in la:
            np.testing.assert_array_equal(la[k], lb[k], err_msg=k)


@needs_ref
@pytest.mark.parametrize("tying,R", [(0, 1), (1, 2), (0, 0)])
def test_kmamba_checkpoint_matches_reference(tmp_path, tying, R):
    # Same seed -> the same parameters (the reference's rand() order,
    # src/kmamba.c:177-188) and byte-identical version-4 files
    # (src/kmamba.c:241-294); each library reads the other's file.
    args = (37, 12, 6, 9, 2)                       # vocab, dim, N, seq_len, layers
    ours = K.kmamba_create(C.byref(O.kmamba_config(*args, R=R, weight_tying=tying,
                                                   cls=K.KMambaConfig)))
    theirs = O.ref.kmamba_create(C.byref(O.kmamba_config(*args, R=R, weight_tying=tying)))
    assert ours and theirs
    assert bool(tying) == (C.addressof(ours.contents.head.contents)
                           == C.addressof(ours.contents.embedding.contents))
    assert K.kmamba_init(ours, 77) == 0 and O.ref.kmamba_init(theirs, 77) == 0
    _assert_same_params(_model_arrays(ours), O.model_params(theirs))
    fa, fb = tmp_path / "ours.kmamba", tmp_path / "theirs.kmamba"
    assert K.kmamba_save(ours, str(fa).encode()) == 0
    assert O.ref.kmamba_save(theirs, str(fb).encode()) == 0
    assert fa.read_bytes() == fb.read_bytes()
    la = K.kmamba_load(str(fb).encode(), 0, None, 0.0, 0.0)
    lb = O.ref.kmamba_load(str(fa).encode(), 0, None, 0.0, 0.0)
    assert la and lb
    assert la.contents.cfg.mimo_rank == lb.contents.cfg.mimo_rank == max(R, 1)
    assert la.contents.cfg.weight_tying == lb.contents.cfg.weight_tying == 0
    _assert_same_params(_model_arrays(la), O.model_params(lb))
    _assert_same_params(_model_arrays(la), _model_arrays(ours))
    for m in (ours, la):
        K.kmamba_free(m)
    for m in (theirs, lb):
        O.ref.kmamba_free(m)


def test_kmamba_create_and_load_errors(tmp_path):
    zero = O.kmamba_config(0, 8, 4, 6, 1, cls=K.KMambaConfig)
    assert not K.kmamba_create(C.byref(zero))
    assert "non-zero" in K.km_last_error()
    topo = O.kmamba_config(11, 8, 4, 6, 1, cls=K.KMambaConfig)
    topo.spatial_ndims = 2
    topo.spatial_dims[0], topo.spatial_dims[1] = 2, 2          # 4 != seq_len
    assert not K.kmamba_create(C.byref(topo))
    assert K.kmamba_init(None, 1) == -1
    K.kmamba_free(None)
    m = K.kmamba_create(C.byref(O.kmamba_config(11, 8, 4, 6, 2, R=2, cls=K.KMambaConfig)))
    assert m and K.kmamba_init(m, 5) == 0
    good = tmp_path / "m.kmamba"
    assert K.kmamba_save(m, str(good).encode()) == 0
    raw = good.read_bytes()
    assert raw[:8] == b"KMAMBA\0\0" and int.from_bytes(raw[8:12], "little") == 4
    assert not K.kmamba_load(str(tmp_path / "missing").encode(), 0, None, 0.0, 0.0)
    cases = {"magic": b"KMAMBX" + raw[6:], "version5": raw[:8] + (5).to_bytes(4, "little") + raw[12:],
             "truncated": raw[:-4], "header_only": raw[:80]}
    for name, data in cases.items():
        (tmp_path / name).write_bytes(data)
        assert not K.kmamba_load(str(tmp_path / name).encode(), 0, None, 0.0, 0.0), name
        assert K.km_last_error(), name
    # Below version 4 the header's rank is ignored: the file loads as
    # mimo_rank 1, reading rank-1 arrays and leaving the rest unread, as the
    # reference does (src/kmamba.c:313, no trailing-data check).
    v3 = tmp_path / "v3"
    v3.write_bytes(raw[:8] + (3).to_bytes(4, "little") + raw[12:])
    old = K.kmamba_load(str(v3).encode(), 0, None, 0.0, 0.0)
    assert old and old.contents.cfg.mimo_rank == 1
    K.kmamba_free(old)
    opt = K.MBOptimConfig()
    assert not K.kmamba_load(str(good).encode(), 1, C.byref(opt), 1e-3, 0.0)
    assert "training" in K.km_last_error()
    loaded = K.kmamba_load(str(good).encode(), 0, None, 0.0, 0.0)
    assert loaded
    _assert_same_params(_model_arrays(loaded), _model_arrays(m))
    K.kmamba_free(loaded)
    K.kmamba_free(m)


def test_scan1d_wrappers_reject_mismatched_tensors():
    # The Python mirror checks dtype, shape and layout before an address goes
    # to the C ABI (a bf16 y beside an fp32 x would make the kernel write past
    # y). These errors are raised before any device check, so they run here.
    torch = pytest.importorskip("torch")
    Bsz, L, D, N = 2, 8, 4, 8
    x = torch.zeros((Bsz, L, D))
    dt = torch.zeros((Bsz, L, D))
    A = torch.zeros((D, N))
    Bm = torch.zeros((Bsz, L, N))
    Cm = torch.zeros((Bsz, L, N))
    y = torch.zeros((Bsz, L, D))
    with pytest.raises(ValueError, match="y has dtype"):
        K.scan1d_fwd(x, dt, A, Bm, Cm, y.bfloat16())
    with pytest.raises(ValueError, match="delta has shape"):
        K.scan1d_fwd(x, dt[:, :4], A, Bm, Cm, y)
    with pytest.raises(ValueError, match="x must be contiguous"):
        K.scan1d_fwd(x.transpose(1, 2).contiguous().transpose(1, 2), dt, A, Bm, Cm, y)
    with pytest.raises(ValueError, match="Cm has shape"):
        K.scan1d_fwd(x, dt, A, Bm, Cm[:, :, :2], y)
    with pytest.raises(ValueError, match="A has dtype"):
        K.scan1d_fwd(x, dt, A.double(), Bm, Cm, y)
    with pytest.raises(ValueError, match="h_final has shape"):
        K.scan1d_fwd(x, dt, A, Bm, Cm, y, h_final=torch.zeros((Bsz, N, D)))
    with pytest.raises(ValueError, match="Bm holds"):
        K.scan1d_fwd(x, dt, A, Bm, Cm, y, bc_strides=(L * D * N, D * N, N))
    with pytest.raises(ValueError, match="must be a GPU tensor"):
        K.scan1d_fwd(x, dt, A, Bm, Cm, y)
    g = torch.zeros((Bsz, L, D))
    with pytest.raises(ValueError, match="dA has shape"):
        K.scan1d_bwd_args(x, dt, A, Bm, Cm, g, g, g, torch.zeros((N, D)), Bm, Cm)
    with pytest.raises(ValueError, match="dB has dtype"):
        K.scan1d_bwd_args(x, dt, A, Bm, Cm, g, g, g, torch.zeros((D, N)), Bm.bfloat16(), Cm)


@needs_ref
def test_topology_bit_exact_vs_reference():
    # Every topology helper against the compiled reference on random and
    # edge-case inputs: wrapping products, invalid ranks, zero/negative
    # extents, out-of-range coordinates, the implicit 1D topology.
    ref = O.ref
    lp = C.POINTER(C.c_long)
    for lib in (ref, K.lib):
        lib.km_power_long.restype = C.c_long
        lib.km_power_long.argtypes = [C.c_long, C.c_long]
        lib.km_make_row_major_strides.restype = C.c_int
        lib.km_make_row_major_strides.argtypes = [lp, C.c_long, lp]
        lib.km_ravel_index.restype = C.c_long
        lib.km_ravel_index.argtypes = [lp, lp, lp, C.c_long]
        lib.km_unravel_index.restype = None
        lib.km_unravel_index.argtypes = [C.c_long, lp, lp, C.c_long, lp]
        lib.km_spatial_dims_product.restype = C.c_int
        lib.km_spatial_dims_product.argtypes = [lp, C.c_long, C.POINTER(C.c_size_t)]
        lib.km_normalize_spatial_topology.restype = C.c_int
        lib.km_normalize_spatial_topology.argtypes = [lp, lp, C.c_size_t, C.c_int, lp, C.c_long]
    g = np.random.default_rng(11)
    for base in (-7, -2, -1, 0, 1, 2, 3, 10, 1 << 20, (1 << 62) + 3):
        for e in (-3, -1, 0, 1, 2, 5, 31, 63, 64, 65, 200):
            assert K.lib.km_power_long(base, e) == ref.km_power_long(base, e), (base, e)
    shapes = [(3,), (2, 3, 4), (1, 1, 1, 1), (7, 5), (1 << 20, 1 << 20, 1 << 20, 1 << 10),
              (2,) * 8, (2,) * 9, (4, 0, 2), (4, -1), ()]
    for dims in shapes:
        n = len(dims)
        dd = K.longs(dims) if n else (C.c_long * 1)()
        s1, s2 = (C.c_long * 9)(), (C.c_long * 9)()
        r1 = K.lib.km_make_row_major_strides(dd, n, s1)
        r2 = ref.km_make_row_major_strides(dd, n, s2)
        assert r1 == r2 and list(s1) == list(s2), dims
        p1, p2 = C.c_size_t(77), C.c_size_t(77)
        assert (K.lib.km_spatial_dims_product(dd, n, C.byref(p1)) ==
                ref.km_spatial_dims_product(dd, n, C.byref(p2))) and p1.value == p2.value, dims
        if r1 != 1:
            continue
        for _ in range(50):
            co = (C.c_long * 9)(*[int(g.integers(-1, d + 1)) for d in dims])
            assert K.lib.km_ravel_index(co, dd, s1, n) == ref.km_ravel_index(co, dd, s2, n)
            lin = int(g.integers(-2, 1 << 40))
            c1, c2 = (C.c_long * 9)(*([5] * 9)), (C.c_long * 9)(*([5] * 9))
            K.lib.km_unravel_index(lin, dd, s1, n, c1)
            ref.km_unravel_index(lin, dd, s2, n, c2)
            assert list(c1) == list(c2), (dims, lin)
    for nd0, dims, seq, conv, cnd in [(0, (), 12, 1, 0), (0, (), 12, 0, 0), (2, (3, 4), 12, 1, 0),
                                      (2, (3, 4), 12, 1, 3), (2, (3, 4), 13, 0, 0),
                                      (3, (2, 2, 3), 12, 1, 3), (1, (12,), 12, 1, -1),
                                      (9, (1,) * 9, 1, 0, 0), (0, (), 0, 0, 0)]:
        outs = []
        for lib in (K.lib, ref):
            nd = C.c_long(nd0)
            sd = (C.c_long * 8)(*([9] * 8))
            for i, v in enumerate(dims[:8]):
                sd[i] = v
            cn = C.c_long(cnd)
            rc = lib.km_normalize_spatial_topology(C.byref(nd), sd, seq, conv, C.byref(cn), 3)
            outs.append((rc, nd.value, list(sd), cn.value))
        assert outs[0] == outs[1], (nd0, dims, seq, conv, cnd, outs)

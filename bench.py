"""Benchmark of the k-mamba hot path on one MI355X.

Headline (BASELINE.json metric): Scan1D selective-scan forward, fp32, at
configs[1] (B=8, L=4096, D=1024, N=16, B/C shared over channels [B, L, N]):
output elements per second, with the dominant kernel's achieved HBM
bandwidth against the 8 TB/s peak. A "step" is one forward pass over one
batch of synthetic inputs already resident in HBM.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5]

Prints one JSON line. The CPU baseline (the oracle restatement of the
reference CPU path, timed on a bounded sample on this host) is reported
beside it; it is a baseline, not the target.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT / "k-mamba_amd", ROOT / "oracle", ROOT / "tests"):
    sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0
METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"]


def scan1d_alg_bytes(Bsz, L, D, N, s):
    """Algorithmic bytes of one Scan1D forward with shared B/C: x, delta, y
    [B,L,D] at s bytes; A [D,N] fp32; B, C [B,L,N] at s bytes; h_final
    [B,D,N] fp32."""
    return 3 * Bsz * L * D * s + D * N * 4 + 2 * Bsz * L * N * s + Bsz * D * N * 4


def scan1d_bwd_alg_bytes(Bsz, L, D, N, s):
    """Algorithmic bytes of one Scan1D backward with shared B/C: x, delta, dy
    read and dx, ddelta written [B,L,D] at s bytes; B, C read and dB, dC
    written [B,L,N] at s bytes; A read and dA written [D,N] fp32. Saved
    checkpoints and recomputation are overhead, not algorithmic bytes."""
    return 5 * Bsz * L * D * s + 4 * Bsz * L * N * s + 2 * D * N * 4


def bench_scan1d_bwd(torch, K, stream, Bsz, L, D, N, dtype, steps, warmup):
    """configs[1] backward: the forward writes 32-step state checkpoints (not
    timed here), the backward recomputes states from them; dy ~ N(0,1)."""
    x, dt, A, Bm, Cm = make_inputs(torch, Bsz, L, D, N, dtype, seed=3)
    g = torch.Generator(device="cuda").manual_seed(4)
    dy = torch.randn((Bsz, L, D), device="cuda", generator=g).to(x.dtype)
    nck = (L + K.KM_SCAN1D_CKPT_STEPS - 1) // K.KM_SCAN1D_CKPT_STEPS
    ck = torch.empty((Bsz, nck, D, N), device="cuda")
    y = torch.empty_like(x)
    dx, ddt = torch.empty_like(x), torch.empty_like(x)
    dA = torch.empty((D, N), device="cuda")
    dB, dC = torch.empty_like(Bm), torch.empty_like(Cm)
    fwd = lambda: K.scan1d_fwd(x, dt, A, Bm, Cm, y, h_ckpt=ck, stream=stream)  # noqa: E731
    bwd = lambda: K.scan1d_bwd(x, dt, A, Bm, Cm, dy, dx, ddt, dA, dB, dC,  # noqa: E731
                               h_ckpt=ck, stream=stream)
    fwd()
    per, _ = time_launches(torch, stream, bwd, steps, warmup)
    perf, _ = time_launches(torch, stream, fwd, steps, warmup)
    ms = sum(per) / len(per)
    msf = sum(perf) / len(perf)
    alg = scan1d_bwd_alg_bytes(Bsz, L, D, N, 2 if dtype == "bf16" else 4)
    return {"bwd_ms": round(ms, 4), "bwd_elems_per_s": Bsz * L * D / (ms * 1e-3),
            "bwd_alg_bytes": alg, "bwd_achieved_GBs": round(alg / (ms * 1e-3) / 1e9, 1),
            "bwd_frac_hbm": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "fwd_with_ckpt_ms": round(msf, 4),
            "fwd_plus_bwd_elems_per_s": Bsz * L * D / ((ms + msf) * 1e-3)}


def bench_scan1d_shape(torch, K, stream, Bsz, L, D, N, dtype, steps, warmup):
    """Scan1D forward at one shape (make_inputs' distributions, B/C shared
    over channels, y and h_final written), called through the C-ABI with a
    prebuilt argument struct so that small shapes time the GPU, not the
    Python wrapper."""
    import ctypes as C
    x, dt, A, Bm, Cm = make_inputs(torch, Bsz, L, D, N, dtype)
    y = torch.empty_like(x)
    hf = torch.empty((Bsz, D, N), device="cuda")
    args = K.scan1d_fwd_args(x, dt, A, Bm, Cm, y, h_final=hf)
    ref, st = C.byref(args), C.c_void_p(stream.cuda_stream)

    def fn():
        if K.km_scan1d_fwd_c(ref, st) != 0:
            raise RuntimeError(K.km_last_error())
    per, _ = time_launches(torch, stream, fn, steps, warmup)
    ms = sum(per) / len(per)
    alg = scan1d_alg_bytes(Bsz, L, D, N, 2 if dtype == "bf16" else 4)
    return {"ms": round(ms, 5), "elems_per_s": Bsz * L * D / (ms * 1e-3),
            "achieved_GBs": round(alg / (ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_convnd(torch, K, stream, dims, D, Kk, steps, warmup):
    """configs[3] workload: input ~ N(0,1) [P,D]; kernel ~ N(0, 1/K^nd)
    [K^nd,D]; bias ~ N(0, 0.01) [D]; causal zero padding, stride 1.
    Forward algorithmic bytes: input read + output written (P*D*4 each) +
    kernel + bias. Backward: input, dy read and dinput written (P*D*4
    each) + kernel read + dkernel, dbias written."""
    nd = len(dims)
    P = 1
    for v in dims:
        P *= v
    KV = Kk ** nd
    g = torch.Generator(device="cuda").manual_seed(21)
    inp = torch.randn((P, D), device="cuda", generator=g)
    ker = torch.randn((KV, D), device="cuda", generator=g) / KV ** 0.5
    bias = torch.randn((D,), device="cuda", generator=g) * 0.1
    out = torch.empty_like(inp)
    dy = torch.randn((P, D), device="cuda", generator=g)
    din, dker, db = torch.empty_like(inp), torch.empty_like(ker), torch.empty_like(bias)
    fwd = lambda: K.convnd_fwd(dims, inp, ker, bias, out, stream=stream)  # noqa: E731
    bwd = lambda: K.convnd_bwd(dims, inp, ker, dy, din, dker, db, stream=stream)  # noqa: E731
    per, _ = time_launches(torch, stream, fwd, steps, warmup)
    perb, _ = time_launches(torch, stream, bwd, steps, warmup)
    ms, msb = sum(per) / len(per), sum(perb) / len(perb)
    alg = 2 * P * D * 4 + KV * D * 4 + D * 4
    algb = 3 * P * D * 4 + 2 * KV * D * 4 + D * 4
    # The 134 MB working set fits the 256 MB last-level cache, so
    # back-to-back launches on the same buffers may read it from there:
    # also timed over 5 input / output sets (670 MB).
    sets = [(torch.randn((P, D), device="cuda", generator=g), torch.empty_like(inp)) for _ in range(5)]
    fns = [(lambda i_, o_: (lambda: K.convnd_fwd(dims, i_, ker, bias, o_, stream=stream)))(i_, o_)
           for i_, o_ in sets]
    perr, _ = time_rotating(torch, stream, fns, steps, warmup)
    msr = sum(perr) / len(perr)
    del sets, fns
    return {"fwd_ms": round(ms, 4), "fwd_elems_per_s": P * D / (ms * 1e-3), "fwd_alg_bytes": alg,
            "fwd_achieved_GBs": round(alg / (ms * 1e-3) / 1e9, 1),
            "fwd_frac_hbm": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "fwd_ms_rotating_5_sets": round(msr, 4),
            "fwd_frac_hbm_rotating": round(alg / (msr * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "bwd_ms": round(msb, 4), "bwd_alg_bytes": algb,
            "bwd_achieved_GBs": round(algb / (msb * 1e-3) / 1e9, 1),
            "bwd_frac_hbm": round(algb / (msb * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


MFMA_BF16_PEAK_TFLOPS = 2500.0


def bench_mamba1_block(torch, K, stream, steps, warmup, Bsz=8, L=2048, dim=1024, di=2048, N=16,
                       dconv=4, R=64):
    """Mamba-1 block forward, bf16 weights/activations, fp32
    state; weights ~ N(0, 0.02), A = -(1..N), x ~ N(0, 1). Reports tokens/s
    for the whole block and, for the in/out projections (the MFMA GEMMs),
    TFLOP/s against the 2.5 PFLOP/s dense bf16 peak."""
    g = torch.Generator(device="cuda").manual_seed(31)
    rn = lambda *s_, std=0.02: (torch.randn(s_, device="cuda", generator=g) * std)  # noqa: E731
    w = {"W_in": rn(2 * di, dim).to(torch.bfloat16), "conv_w": rn(dconv, di, std=0.5),
         "conv_b": rn(di, std=0.1), "W_x": rn(R + 2 * N, di).to(torch.bfloat16),
         "W_dt": rn(di, R).to(torch.bfloat16), "dt_bias": rn(di, std=0.5) - 2.0,
         "A": -torch.arange(1, N + 1, device="cuda", dtype=torch.float32).repeat(di, 1).contiguous(),
         "Dskip": torch.ones(di, device="cuda"), "W_out": rn(dim, di).to(torch.bfloat16)}
    x = torch.randn((Bsz, L, dim), device="cuda", generator=g).to(torch.bfloat16)
    out = torch.empty_like(x)
    ws = torch.empty(K.km_mamba1_block_workspace_bytes(K.C.byref(K.mamba1_weights(w)), Bsz, L),
                     dtype=torch.uint8, device="cuda")
    blk = lambda: K.mamba1_block_fwd(w, x, out, workspace=ws, stream=stream)  # noqa: E731
    per, _ = time_launches(torch, stream, blk, steps, warmup)
    ms = sum(per) / len(per)
    T = Bsz * L
    xi = torch.empty((T, di), device="cuda", dtype=torch.bfloat16)
    # The standalone out_proj runs on data shaped like the gated scan's
    # output: matrix-core throughput depends on the operand bits (zeros, as
    # an uninitialised buffer often holds, run ~25 % faster than real data).
    y = torch.randn((T, di), device="cuda", generator=g).to(torch.bfloat16)
    o = torch.empty((T, dim), device="cuda", dtype=torch.bfloat16)
    inp = lambda: K.gemm_bf16(x.view(T, dim), w["W_in"][:di], xi, stream=stream)  # noqa: E731
    outp = lambda: K.gemm_bf16(y, w["W_out"], o, stream=stream)  # noqa: E731
    pi, _ = time_launches(torch, stream, inp, steps, warmup)
    po, _ = time_launches(torch, stream, outp, steps, warmup)
    mi, mo = sum(pi) / len(pi), sum(po) / len(po)
    fi, fo = 2.0 * T * di * dim, 2.0 * T * dim * di
    return {"block_ms": round(ms, 4), "tokens_per_s": T / (ms * 1e-3),
            "projections": "every projection on km_gemm_bf16 (hand-written bf16 MFMA); the figures "
                           "below time the in_proj half and out_proj shapes alone",
            "in_proj_half_ms": round(mi, 4),
            "in_proj_TFLOPs": round(fi / (mi * 1e-3) / 1e12, 1),
            "in_proj_frac_mfma_peak": round(fi / (mi * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "out_proj_ms": round(mo, 4), "out_proj_TFLOPs": round(fo / (mo * 1e-3) / 1e12, 1),
            "out_proj_frac_mfma_peak": round(fo / (mo * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "config": {"B": Bsz, "L": L, "dim": dim, "d_inner": di, "d_state": N, "d_conv": dconv,
                       "dt_rank": R}}


def bench_scan1d_gated(torch, K, stream, steps, warmup, Bsz=8, L=2048, D=2048, N=16, R=64):
    """The block's gated Scan1D on its own (configs[4] shapes: bf16 x, delta,
    z [B, L, D], B/C read through the x_proj output's strides, Dskip), the
    same launch ungated, and each launch timed alone (two HIP events around
    it) after two in_proj-sized GEMMs, or after a 512 MB device copy that
    empties the last-level cache."""
    import ctypes as C
    g = torch.Generator(device="cuda").manual_seed(17)
    bf = torch.bfloat16
    x = torch.randn((Bsz, L, D), device="cuda", generator=g).to(bf)
    dt = torch.nn.functional.softplus(0.5 * torch.randn((Bsz, L, D), device="cuda", generator=g)
                                      - 2.0).to(bf)
    A = -torch.arange(1, N + 1, device="cuda", dtype=torch.float32).repeat(D, 1).contiguous()
    NX = R + 2 * N
    xd = (torch.randn((Bsz, L, NX), device="cuda", generator=g) * 0.3).to(bf).view(-1)
    Bm, Cm = xd.narrow(0, R, xd.numel() - R - N), xd.narrow(0, R + N, xd.numel() - R - N)
    z = torch.randn((Bsz, L, D), device="cuda", generator=g).to(bf)
    Ds = torch.ones(D, device="cuda")
    y = torch.empty_like(x)
    h = C.c_void_p(K.stream_handle(stream))
    gated = K.scan1d_fwd_args(x, dt, A, Bm, Cm, y, bc_strides=(L * NX, NX, 0), z=z, Dskip=Ds)
    plain = K.scan1d_fwd_args(x, dt, A, Bm, Cm, y, bc_strides=(L * NX, NX, 0))
    run = lambda a: K.check(K.km_scan1d_fwd_c(C.byref(a), h), "km_scan1d_fwd")  # noqa: E731
    _, wg = time_launches(torch, stream, lambda: run(gated), steps, warmup)
    _, wp = time_launches(torch, stream, lambda: run(plain), steps, warmup)
    T = Bsz * L
    a = torch.randn((T, 1024), device="cuda", generator=g).to(bf)
    wgt = (torch.randn((D, 1024), device="cuda", generator=g) * 0.02).to(bf)
    o = torch.empty((T, D), device="cuda", dtype=bf)
    big0 = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    big1 = torch.empty_like(big0)

    def after(prep, n):
        e = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(n)]
        for i in range(n + warmup):
            prep()
            if i >= warmup:
                e[i - warmup][0].record(stream)
            run(gated)
            if i >= warmup:
                e[i - warmup][1].record(stream)
        torch.cuda.synchronize()
        return sum(a.elapsed_time(b) for a, b in e) / n * 1000

    n = max(10, min(steps, 50))
    us_gemm = after(lambda: (K.gemm_bf16(a, wgt, o, stream=stream),
                             K.gemm_bf16(a, wgt, o, stream=stream)), n)
    us_copy = after(lambda: big1.copy_(big0), n)
    return {"gated_us": round(wg / steps * 1000, 1), "ungated_us": round(wp / steps * 1000, 1),
            "gated_after_two_gemms_us": round(us_gemm, 1),
            "gated_after_512MB_copy_us": round(us_copy, 1),
            "config": {"B": Bsz, "L": L, "D": D, "N": N, "bc_row": NX, "dtype": "bf16"}}


def bench_gemm_vs_library(torch, K, stream, steps, warmup):
    """The block's projection shapes (in_proj: 16384 x 4096 x 1024, one
    launch in the block with its x and z column halves routed to two
    buffers; its half 16384 x 2048 x 1024; out_proj: 16384 x 1024 x 2048) on
    km_gemm_bf16 and on torch.matmul (hipBLASLt on ROCm), same bf16 operands
    (N(0,1) activations, N(0, 0.02) weights: matrix-core throughput depends
    on the operand bits), bf16 out."""
    g = torch.Generator(device="cuda").manual_seed(11)
    out = {}
    for name, (M, N, Kd) in {"in_proj": (16384, 4096, 1024),
                             "in_proj_half": (16384, 2048, 1024),
                             "out_proj": (16384, 1024, 2048)}.items():
        A = torch.randn((M, Kd), device="cuda", generator=g).to(torch.bfloat16)
        B = (torch.randn((N, Kd), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        C = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
        Bt = B.t()
        pk, _ = time_launches(torch, stream, lambda: K.gemm_bf16(A, B, C, stream=stream), steps, warmup)
        pl, _ = time_launches(torch, stream, lambda: torch.matmul(A, Bt, out=C), steps, warmup)
        fl = 2.0 * M * N * Kd
        mk, ml = sum(pk) / len(pk), sum(pl) / len(pl)
        out[name] = {"M": M, "N": N, "K": Kd,
                     "km_ms": round(mk, 4), "km_TFLOPs": round(fl / (mk * 1e-3) / 1e12, 1),
                     "torch_matmul_ms": round(ml, 4),
                     "torch_matmul_TFLOPs": round(fl / (ml * 1e-3) / 1e12, 1)}
    return out


def bench_model(K, steps, warmup, V=32768, D=1024, N=16, L=2048, n_layers=4):
    """The stacked model's forward (kmamba_forward: embedding rows, n_layers
    Mamba-3 blocks, head product; host tokens in, host logits out, the
    head uploaded per call as its parameters are host-owned), wall clock per
    call. Reports the head product's fp32 FLOP rate bound as well."""
    import ctypes
    import numpy as np
    cfg = K.KMambaConfig()
    cfg.vocab_size, cfg.dim, cfg.state_size, cfg.seq_len, cfg.n_layers = V, D, N, L, n_layers
    cfg.mimo_rank, cfg.dt_scale, cfg.dt_min, cfg.dt_max = 1, 0.1, 1e-3, 0.1
    m = K.kmamba_create(ctypes.byref(cfg))
    if not m:
        raise RuntimeError(K.km_last_error())
    K.kmamba_init(m, 7)
    toks = np.random.default_rng(7).integers(0, V, L).astype(np.uint32)
    logits = np.empty((L, V), np.float32)
    fn = lambda: K.kmamba_forward(m, toks.ctypes.data, logits.ctypes.data)  # noqa: E731
    for _ in range(warmup):
        fn()
    t = time.perf_counter()
    for _ in range(steps):
        rc = fn()
    ms = (time.perf_counter() - t) * 1e3 / steps
    err = K.km_last_error() if rc else ""
    K.kmamba_free(m)
    if err:
        raise RuntimeError(err)
    return {"ms": round(ms, 3), "tokens_per_s": L / (ms * 1e-3),
            "head_GFLOP": round(2.0 * L * D * V / 1e9, 1),
            "host_bytes_per_call": {"head_up": 4 * D * V, "logits_down": 4 * L * V,
                                    "embedding_rows_up": 4 * L * D},
            "config": {"vocab": V, "dim": D, "state_size": N, "seq_len": L, "n_layers": n_layers,
                       "io": "host tokens and logits"}}


def scannd_alg_bytes(dims, D, M):
    """Algorithmic bytes of one ScanND forward: x [P,D], delta [nd,P,D],
    A [nd,D,M], B and C [P,D,M] read; h [P,D,M] and y [P,D] written (fp32)."""
    nd = len(dims)
    P = 1
    for v in dims:
        P *= v
    return 4 * (P * D + nd * P * D + nd * D * M + 2 * P * D * M + P * D * M + P * D)


def bench_mamba3(torch, K, steps, warmup, Bsz=8, L=2048, dim=1024, N=16, R=1):
    """The reference Mamba-3 block forward (mamba_block_forward: the API's
    synchronous call, input and output resident on the device, parameters
    from mamba_block_init), at the configs[4] width and sequence length. The
    call uploads the block's host-side parameters each time, as the
    reference layout keeps them on the host; wall clock per call."""
    import ctypes
    cfg = K.MBConfig()
    cfg.dim, cfg.state_size, cfg.seq_len, cfg.mimo_rank = dim, N, L, R
    cfg.dt_scale, cfg.dt_min, cfg.dt_max = 0.1, 1e-3, 0.1
    blk = K.mamba_block_create(ctypes.byref(cfg))
    ctypes.CDLL(None).srand(11)
    K.mamba_block_init(blk)
    g = torch.Generator(device="cuda").manual_seed(41)
    x = torch.randn((Bsz, L, dim), device="cuda", generator=g)
    out = torch.empty_like(x)
    fn = lambda: K.mamba_block_forward(blk, K.ptr(out), K.ptr(x), Bsz)  # noqa: E731
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t) * 1e3 / steps
    err = K.km_last_error()
    # The same call on host (pageable) arrays, as the reference's callers
    # pass them: 64 MB in and out per call over PCIe.
    import numpy as np
    xh = x.cpu().numpy()
    oh = np.empty_like(xh)
    fh = lambda: K.mamba_block_forward(blk, oh.ctypes.data, xh.ctypes.data, Bsz)  # noqa: E731
    for _ in range(max(1, warmup // 4)):
        fh()
    t = time.perf_counter()
    hsteps = max(1, steps // 4)
    for _ in range(hsteps):
        fh()
    host_ms = (time.perf_counter() - t) * 1e3 / hsteps
    err = err or K.km_last_error()
    K.mamba_block_free(blk)
    if err:
        raise RuntimeError(err)
    T = Bsz * L
    return {"ms": round(ms, 4), "tokens_per_s": T / (ms * 1e-3),
            "host_io_ms": round(host_ms, 4), "host_io_tokens_per_s": T / (host_ms * 1e-3),
            "host_io_bytes_per_call": 2 * xh.nbytes,
            "config": {"B": Bsz, "L": L, "dim": dim, "state_size": N, "mimo_rank": R,
                       "io": "device pointers (ms); host pageable arrays (host_io_ms)"}}


def bench_scannd(torch, K, stream, dims, D, M, steps, warmup):
    """configs[2] workload: x ~ N(0,1); delta = 1; A = log(U(0.05, 0.9/nd));
    B, C ~ N(0, 1/16); scannd_ref semantics (h and y written)."""
    nd = len(dims)
    P = 1
    for v in dims:
        P *= v
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn((P, D), device="cuda", generator=g)
    A = torch.log(0.05 + (0.9 / nd - 0.05) * torch.rand((nd, D, M), device="cuda", generator=g))
    B = torch.randn((P, D, M), device="cuda", generator=g) * 0.25
    Cm = torch.randn((P, D, M), device="cuda", generator=g) * 0.25
    dt = torch.ones((nd, P, D), device="cuda")
    h = torch.empty((P, D, M), device="cuda")
    y = torch.empty((P, D), device="cuda")
    fn = lambda: K.scannd_fwd(dims, x, A, B, Cm, dt, h, y, stream=stream)  # noqa: E731
    per, wall = time_launches(torch, stream, fn, steps, warmup)
    ms = wall / steps
    alg = scannd_alg_bytes(dims, D, M)
    return {"ms": round(ms, 4), "elems_per_s": P * D / (ms * 1e-3),
            "achieved_GBs": round(alg / (ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "alg_bytes": alg,
            "launches_per_step": "one dataflow launch (and its flag reset)"}


def scannd_bwd_alg_bytes(dims, D, M):
    """Algorithmic bytes of one ScanND backward: x, dy [P,D], delta [nd,P,D],
    A [nd,D,M], B, C, h [P,D,M] read; dx [P,D], ddelta [nd,P,D], dA
    [nd,D,M], dB, dC [P,D,M] written (fp32)."""
    nd = len(dims)
    P = 1
    for v in dims:
        P *= v
    reads = 2 * P * D + nd * P * D + nd * D * M + 3 * P * D * M
    writes = P * D + nd * P * D + nd * D * M + 2 * P * D * M
    return 4 * (reads + writes)


def bench_scannd_bwd(torch, K, stream, dims, D, M, steps, warmup):
    """The ScanND backward on the configs[2] grids and inputs (h from the
    forward, dy ~ N(0, 1)): on an 8-XCD device one dataflow launch on
    pencils forming the adjoint state and every gradient, then the two
    fixed-order dA sums (KM_SCANND_BWD_FUSED=0: the adjoint sweep, then the
    gradient pass). Wall time per backward over the timed launches."""
    nd = len(dims)
    P = 1
    for v in dims:
        P *= v
    g = torch.Generator(device="cuda").manual_seed(12)
    x = torch.randn((P, D), device="cuda", generator=g)
    A = torch.log(0.05 + (0.9 / nd - 0.05) * torch.rand((nd, D, M), device="cuda", generator=g))
    B = torch.randn((P, D, M), device="cuda", generator=g) * 0.25
    Cm = torch.randn((P, D, M), device="cuda", generator=g) * 0.25
    dt = torch.ones((nd, P, D), device="cuda")
    h = torch.empty((P, D, M), device="cuda")
    y = torch.empty((P, D), device="cuda")
    K.scannd_fwd(dims, x, A, B, Cm, dt, h, y, stream=stream)
    dy = torch.randn((P, D), device="cuda", generator=g)
    dx, ddt = torch.empty_like(x), torch.empty_like(dt)
    dA, dB, dC = torch.empty_like(A), torch.empty_like(B), torch.empty_like(Cm)
    fn = lambda: K.scannd_bwd(dims, x, A, B, Cm, dt, h, dy, dx, ddt, dA, dB, dC, stream=stream)  # noqa: E731
    per, wall = time_launches(torch, stream, fn, steps, warmup)
    ms = wall / steps
    alg = scannd_bwd_alg_bytes(dims, D, M)
    return {"ms": round(ms, 4), "elems_per_s": P * D / (ms * 1e-3),
            "achieved_GBs": round(alg / (ms * 1e-3) / 1e9, 1),
            "frac_hbm": round(alg / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "alg_bytes": alg,
            "launches": ("fused pencil launch + dA sums" if os.environ.get("KM_SCANND_BWD_FUSED") != "0"
                         else "adjoint sweep + gradient pass + dA sums")}


def make_inputs(torch, Bsz, L, D, N, dtype, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    dev = "cuda"
    x = torch.randn((Bsz, L, D), device=dev, generator=g)
    dt = torch.nn.functional.softplus(0.5 * torch.randn((Bsz, L, D), device=dev, generator=g) - 1.0)
    A = -torch.arange(1, N + 1, device=dev, dtype=torch.float32).repeat(D, 1).contiguous()
    Bm = torch.randn((Bsz, L, N), device=dev, generator=g) / N ** 0.5
    Cm = torch.randn((Bsz, L, N), device=dev, generator=g) / N ** 0.5
    cast = (lambda t: t.to(torch.bfloat16)) if dtype == "bf16" else (lambda t: t)
    return cast(x), cast(dt), A, cast(Bm), cast(Cm)


def time_launches(torch, stream, fn, steps, warmup):
    """Average duration (ms) of one call of fn, from two HIP events recorded
    on the launch stream around `steps` back-to-back calls (events between
    the calls would add their own gaps), as a per-call list, plus the wall
    time of the timed region."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        fn()
    t1.record(stream)
    torch.cuda.synchronize()
    wall = t0.elapsed_time(t1)
    return [wall / steps] * steps, wall


def time_rotating(torch, stream, fns, steps, warmup):
    """time_launches over a list of calls that each use their own buffer set
    (call i of the timed region runs fns[i % len(fns)]): with the sets
    together larger than the 256 MB last-level cache, no launch finds its
    operands left there by the previous one."""
    it = [0]

    def fn():
        fns[it[0] % len(fns)]()
        it[0] += 1
    return time_launches(torch, stream, fn, steps, warmup)


def bench_copy(torch, stream, steps, warmup):
    """A plain device copy of 1 GiB (fp32, torch's copy kernel): the HBM
    bandwidth a streaming kernel can reach on this box, read + write."""
    n = 1 << 28
    src = torch.ones(n, device="cuda")
    dst = torch.empty_like(src)
    per, _ = time_launches(torch, stream, lambda: dst.copy_(src), steps, warmup)
    ms = sum(per) / len(per)
    del src, dst
    return {"bytes_read": 4 * n, "bytes_written": 4 * n, "ms": round(ms, 4),
            "GBs_read_plus_write": round(8 * n / (ms * 1e-3) / 1e9, 1),
            "frac_of_8TBs": round(8 * n / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def host_info():
    """CPU model, glibc and thread settings of the host the CPU legs run on."""
    model = platform.processor() or platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu": model, "glibc": "-".join(platform.libc_ver()), "nproc": os.cpu_count(),
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}


def cpu_threads():
    """Threads of the all-cores legs: OMP_NUM_THREADS when set (the GPU
    boxes set it to the box's CPU share), else every core, at most 16."""
    try:
        n = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        n = 0
    return max(1, min(n if n > 0 else (os.cpu_count() or 1), 16))


def cpu_baseline_scan1d(x, dt, A, Bm, Cm, nthreads=1, budget_s=3.0):
    """Oracle restatement of the reference scan1d (cpu/scan1d.asm) on whole
    batch elements of the workload, repeated until the time budget is used: one
    thread (the asm is single-threaded), or nthreads over (batch, channel)
    as the reference's batch threading (src/kmamba.c:512-531). Returns
    (elems/s, batch elements done, seconds)."""
    import numpy as np
    import oracle as O
    Bsz, L, D = x.shape
    done, t_total, b = 0, 0.0, 0
    per = 1 if nthreads == 1 else Bsz
    while t_total < budget_s:            # whole batch elements, repeated up to the budget
        nb = min(per, Bsz - b % Bsz)
        i0 = b % Bsz
        xs, dts, Bs, Cs = (np.ascontiguousarray(a[i0:i0 + nb]) for a in (x, dt, Bm, Cm))
        t = time.perf_counter()
        O.scan1d_batched(xs, dts, A, Bs, Cs, nthreads=nthreads, fast=True)
        t_total += time.perf_counter() - t
        done += nb * L * D
        b += nb
    return done / t_total, b, t_total


def cpu_baseline_scan2d(nthreads, dims=(256, 256), D=256, M=16, dsample=16, budget_s=3.0):
    """The oracle's scannd_ref (src/scan_nd.c, OpenMP over the points of each
    wavefront level as src/scan_nd.c:86) on configs[2]'s 256x256 grid with
    dsample of the D channels (channels are independent, so this is an exact
    sub-problem; the state arrays of all 256 channels would take 3 GB of host
    memory), repeated until the time budget is used. Returns (y elems/s,
    seconds)."""
    import numpy as np
    import oracle as O
    g = np.random.default_rng(7)
    P, nd = int(np.prod(dims)), len(dims)
    x = g.standard_normal((P, dsample)).astype(np.float32)
    A = np.log(g.uniform(0.05, 0.9 / nd, (nd, dsample, M))).astype(np.float32)
    B = (g.standard_normal((P, dsample, M)) * 0.25).astype(np.float32)
    C = (g.standard_normal((P, dsample, M)) * 0.25).astype(np.float32)
    dt = np.ones((nd, P, dsample), np.float32)
    secs, runs = 0.0, 0
    while secs < budget_s:
        t = time.perf_counter()
        O.scannd_ref(dims, x, A, B, C, dt, nthreads=nthreads, fast=True)
        secs += time.perf_counter() - t
        runs += 1
    return runs * P * dsample / secs, secs


def cpu_baseline_convnd(nthreads, dims=(512, 512), D=64, K=3, budget_s=3.0):
    """The oracle's ConvND forward (src/convnd.c:58-126: the K^N stencil per
    point and channel, OpenMP over points as src/convnd.c:88) on configs[3]'s
    512x512 D=64 K=3 case, repeated until the time budget is used. Returns
    (output elems/s, seconds)."""
    import numpy as np
    import oracle as O
    g = np.random.default_rng(5)
    P = int(np.prod(dims))
    inp = g.standard_normal((P, D)).astype(np.float32)
    ker = (g.standard_normal((K ** len(dims), D)) / K).astype(np.float32)
    bias = (g.standard_normal(D) * 0.1).astype(np.float32)
    secs, runs = 0.0, 0
    while secs < budget_s:
        t = time.perf_counter()
        O.convnd_forward(dims, inp, ker, bias, nthreads=nthreads, fast=True)
        secs += time.perf_counter() - t
        runs += 1
    return runs * P * D / secs, secs


def cpu_baselines(x, dt, A, Bm, Cm):
    """The CPU legs (the oracle's optimised build; a reported baseline, not
    the target), timed on this host before the GPU work."""
    nt = cpu_threads()
    r1, nb1, s1 = cpu_baseline_scan1d(x, dt, A, Bm, Cm, nthreads=1)
    rn, nbn, sn = cpu_baseline_scan1d(x, dt, A, Bm, Cm, nthreads=nt)
    r2, s2 = cpu_baseline_scan2d(1)
    r2n, s2n = cpu_baseline_scan2d(nt)
    r3, s3 = cpu_baseline_convnd(1)
    r3n, s3n = cpu_baseline_convnd(nt)
    Bsz, L, D = x.shape
    return {"value": r1, "unit": "elems/s", "cores": 1, "kind": "port",
            "sample": f"{nb1} batch elements (of {Bsz}, cycled) of the headline workload (L={L}, D={D}, "
                      f"N={A.shape[1]}), the oracle's restatement of cpu/scan1d.asm, one thread as "
                      f"the asm, {s1:.1f} s",
            "all_cores": {"value": rn, "unit": "elems/s", "cores": nt,
                          "sample": f"{nbn} batch elements, OpenMP over (batch, channel), {sn:.1f} s"},
            "scan2d_256x256": {"value": r2, "unit": "elems/s", "cores": 1,
                               "all_cores_value": r2n, "all_cores": nt,
                               "sample": f"scannd_ref restatement, 16 of 256 channels (independent), "
                                         f"N=16; {s2:.1f} s on one thread, {s2n:.1f} s on {nt} "
                                         f"(OpenMP per wavefront level)"},
            "convnd_512x512": {"value": r3, "unit": "elems/s", "cores": 1,
                               "all_cores_value": r3n, "all_cores": nt,
                               "sample": f"ConvND forward restatement (src/convnd.c), 512x512 D=64 "
                                         f"K=3, whole grid; {s3:.1f} s on one thread, {s3n:.1f} s "
                                         f"on {nt} (OpenMP over points)"},
            "host": host_info()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    # The headline runs after every other reported workload, so its clocks
    # have settled; --only modes time the ramp unless the warm-up is long
    # (the GPU needs ~0.1 s of load after idle).
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", choices=["all", "scan1d", "scan1d_shapes", "scan1d_bwd", "scannd",
                                       "convnd", "block", "scan1d_gated", "mamba3", "gemm", "model",
                                       "scannd_bwd", "copy"],
                    default="all",
                    help="profiling modes: scan1d = the fp32 headline kernel only; scan1d_shapes = "
                         "the forward at each --shapes entry; copy = a plain 1 GiB device copy "
                         "(calibrates rocprof FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--shapes", nargs="+", default=["1,128,384"],
                    help="B,L,D[,dtype] entries for --only scan1d_shapes (N = 16; dtype f32 or bf16)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; multi-GPU sharding is design-only "
              "(the kernels shard over batch and channels with no exchange), so --gpus must be 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import kmamba as K

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    stream = torch.cuda.Stream()
    if args.only == "copy":
        n = 1 << 28
        with torch.cuda.stream(stream):
            src = torch.ones(n, device="cuda")
            dst = torch.empty_like(src)
            per, _ = time_launches(torch, stream, lambda: dst.copy_(src), args.steps, args.warmup)
        ms = sum(per) / len(per)
        print(json.dumps({"copy_bytes_read": 4 * n, "copy_bytes_written": 4 * n, "ms": ms,
                          "GBs_read_plus_write": 8 * n / (ms * 1e-3) / 1e9}))
        return
    if args.only == "scan1d_bwd":
        with torch.cuda.stream(stream):
            r = bench_scan1d_bwd(torch, K, stream, 8, 4096, 1024, 16, "f32", args.steps, args.warmup)
            rb = bench_scan1d_bwd(torch, K, stream, 8, 4096, 1024, 16, "bf16", args.steps,
                                  args.warmup)
        print(json.dumps({"scan1d_bwd_f32": r, "scan1d_bwd_bf16": rb}))
        return
    if args.only == "scan1d_gated":
        with torch.cuda.stream(stream):
            r = bench_scan1d_gated(torch, K, stream, args.steps, args.warmup)
        print(json.dumps({"scan1d_gated_block_shape": r}))
        return
    if args.only == "block":
        with torch.cuda.stream(stream):
            r = bench_mamba1_block(torch, K, stream, args.steps, args.warmup)
        print(json.dumps({"mamba1_block_configs4": r}))
        return
    if args.only == "scannd_bwd":
        with torch.cuda.stream(stream):
            r2 = bench_scannd_bwd(torch, K, stream, (256, 256), 256, 16, args.steps, min(args.warmup, 10))
            r3 = bench_scannd_bwd(torch, K, stream, (64, 64, 64), 128, 16, args.steps, min(args.warmup, 10))
        print(json.dumps({"scannd_bwd_2d_256x256_D256_M16": r2, "scannd_bwd_3d_64cubed_D128_M16": r3}))
        return
    if args.only == "model":
        print(json.dumps({"kmamba_forward": bench_model(K, args.steps, min(args.warmup, 3))}))
        return
    if args.only == "gemm":
        with torch.cuda.stream(stream):
            r = bench_gemm_vs_library(torch, K, stream, args.steps, min(args.warmup, 200))
        print(json.dumps({"gemm_bf16_vs_torch_matmul": r}))
        return
    if args.only == "mamba3":
        print(json.dumps({"mamba3_block_fwd": bench_mamba3(torch, K, args.steps, min(args.warmup, 20))}))
        return
    if args.only == "convnd":
        with torch.cuda.stream(stream):
            r2 = bench_convnd(torch, K, stream, (512, 512), 64, 3, args.steps, args.warmup)
            r3 = bench_convnd(torch, K, stream, (64, 64, 64), 64, 3, args.steps, args.warmup)
        print(json.dumps({"convnd_2d_512x512_D64_K3": r2, "convnd_3d_64cubed_D64_K3": r3}))
        return
    if args.only == "scan1d":
        Bsz, L, D, N = 8, 4096, 1024, 16
        with torch.cuda.stream(stream):
            x, dt, A, Bm, Cm = make_inputs(torch, Bsz, L, D, N, "f32")
            y = torch.empty_like(x)
            hf = torch.empty((Bsz, D, N), device="cuda")
            fn = lambda: K.scan1d_fwd(x, dt, A, Bm, Cm, y, h_final=hf, stream=stream)  # noqa: E731
            per, _ = time_launches(torch, stream, fn, args.steps, args.warmup)
        ms = sum(per) / len(per)
        print(json.dumps({"scan1d_f32_ms": ms, "GBs": scan1d_alg_bytes(Bsz, L, D, N, 4) / (ms * 1e-3) / 1e9}))
        return
    if args.only == "scan1d_shapes":
        out = {}
        with torch.cuda.stream(stream):
            for e in args.shapes:
                f = e.split(",")
                Bsz, L, D = (int(v) for v in f[:3])
                dtype = f[3] if len(f) > 3 else "f32"
                out[f"B{Bsz}_L{L}_D{D}_{dtype}"] = bench_scan1d_shape(torch, K, stream, Bsz, L, D, 16,
                                                                      dtype, args.steps, args.warmup)
        print(json.dumps(out))
        return
    if args.only == "scannd":
        with torch.cuda.stream(stream):
            r2 = bench_scannd(torch, K, stream, (256, 256), 256, 16, args.steps, args.warmup)
            r3 = bench_scannd(torch, K, stream, (64, 64, 64), 128, 16, args.steps, args.warmup)
        print(json.dumps({"scan2d_256x256_D256_M16": r2, "scan3d_64cubed_D128_M16": r3}))
        return
    # Order: the CPU legs first (the GPU idles), then every reported GPU
    # workload, then the headline's W warm-up and K timed steps, which thus
    # run on a GPU whose clocks have settled under load (~0.1 s of load
    # after idle; W = 5 alone would time the ramp).
    Bsz, L, D, N = 8, 4096, 1024, 16
    extra = {}
    with torch.cuda.stream(stream):
        x, dt, A, Bm, Cm = make_inputs(torch, Bsz, L, D, N, "f32")
    torch.cuda.synchronize()
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baselines(*(t.float().cpu().numpy() for t in (x, dt, A, Bm, Cm)))
    elems = Bsz * L * D
    alg = scan1d_alg_bytes(Bsz, L, D, N, 4)
    extra["kmamba_forward_f32"] = bench_model(K, 3, 1)
    with torch.cuda.stream(stream):
        # Untimed: ~0.2 s of forward launches so the reported workloads below
        # start on settled clocks.
        y = torch.empty_like(x)
        hf = torch.empty((Bsz, D, N), device="cuda")
        t_end = time.perf_counter() + 0.2
        while time.perf_counter() < t_end:
            for _ in range(50):
                K.scan1d_fwd(x, dt, A, Bm, Cm, y, h_final=hf, stream=stream)
            torch.cuda.synchronize()
        extra["scan1d_bwd_f32"] = bench_scan1d_bwd(torch, K, stream, Bsz, L, D, N, "f32",
                                                   max(5, args.steps // 2), 5)
        extra["scan1d_bwd_bf16"] = bench_scan1d_bwd(torch, K, stream, Bsz, L, D, N, "bf16",
                                                    max(5, args.steps // 2), 5)
        extra["scannd_2d_256x256_D256_M16_f32"] = bench_scannd(torch, K, stream, (256, 256), 256, 16,
                                                                max(5, args.steps // 2), 5)
        extra["convnd_2d_512x512_D64_K3_f32"] = bench_convnd(torch, K, stream, (512, 512), 64, 3,
                                                             max(5, args.steps // 2), 5)
        extra["convnd_3d_64cubed_D64_K3_f32"] = bench_convnd(torch, K, stream, (64, 64, 64), 64, 3,
                                                             max(5, args.steps // 2), 5)
        extra["mamba1_block_configs4_bf16"] = bench_mamba1_block(torch, K, stream,
                                                                  max(5, args.steps // 2), 5)
        extra["scannd_3d_64cubed_D128_M16_f32"] = bench_scannd(torch, K, stream, (64, 64, 64), 128, 16,
                                                                max(5, args.steps // 2), 5)
        extra["mamba3_block_fwd_f32"] = bench_mamba3(torch, K, max(5, args.steps // 10), 2)
        extra["scannd_bwd_2d_256x256_D256_M16_f32"] = bench_scannd_bwd(
            torch, K, stream, (256, 256), 256, 16, max(5, args.steps // 10), 2)
        extra["scannd_bwd_3d_64cubed_D128_M16_f32"] = bench_scannd_bwd(
            torch, K, stream, (64, 64, 64), 128, 16, max(5, args.steps // 10), 2)
        # configs[0] (the reference's CPU-runnable case: 12 workgroups, one
        # per (batch, 32-channel group)) and a few-pairs long sequence that
        # the launcher splits over 256 workgroups (8 segments of 1024 steps).
        extra["scan1d_fwd_configs0_B1_L128_D384_f32"] = bench_scan1d_shape(
            torch, K, stream, 1, 128, 384, 16, "f32", max(20, args.steps), 10)
        extra["scan1d_fwd_split_B1_L8192_D1024_f32"] = bench_scan1d_shape(
            torch, K, stream, 1, 8192, 1024, 16, "f32", max(20, args.steps), 10)

        # bf16 I/O forward (reported, not the headline). Its 204 MB working
        # set fits the 256 MB last-level cache: also timed over 3 input /
        # output sets (612 MB).
        bsets = []
        for sd in range(3):
            xb, dtb, Ab, Bb, Cb = make_inputs(torch, Bsz, L, D, N, "bf16", seed=sd)
            bsets.append((xb, dtb, Ab, Bb, Cb, torch.empty_like(xb)))
        xb, dtb, Ab, Bb, Cb, yb = bsets[0]
        fnb = lambda: K.scan1d_fwd(xb, dtb, Ab, Bb, Cb, yb, h_final=hf, stream=stream)  # noqa: E731
        perb, _ = time_launches(torch, stream, fnb, args.steps, 20)
        msb = sum(perb) / len(perb)
        fnsb = [(lambda t_: (lambda: K.scan1d_fwd(*t_[:5], t_[5], h_final=hf, stream=stream)))(t_)
                for t_ in bsets]
        perbr, _ = time_rotating(torch, stream, fnsb, args.steps, 20)
        msbr = sum(perbr) / len(perbr)
        algb = scan1d_alg_bytes(Bsz, L, D, N, 2)
        extra["scan1d_fwd_bf16"] = {"ms": round(msb, 4), "elems_per_s": elems / (msb * 1e-3),
                                    "state_updates_per_s": elems * N / (msb * 1e-3),
                                    "achieved_GBs": round(algb / (msb * 1e-3) / 1e9, 1),
                                    "frac_hbm": round(algb / (msb * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                    "ms_rotating_3_sets": round(msbr, 4),
                                    "frac_hbm_rotating": round(algb / (msbr * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del bsets, fnsb, xb, dtb, Bb, Cb, yb

        # fp32 headline workload over 2 input / output sets (815 MB): its
        # 407 MB working set already exceeds the last-level cache; the
        # rotating figure shows no cache-assisted gain in the headline.
        x2, dt2, A2, B2, C2 = make_inputs(torch, Bsz, L, D, N, "f32", seed=5)
        y2 = torch.empty_like(x2)
        fnsr = [lambda: K.scan1d_fwd(x, dt, A, Bm, Cm, y, h_final=hf, stream=stream),
                lambda: K.scan1d_fwd(x2, dt2, A2, B2, C2, y2, h_final=hf, stream=stream)]
        perr, _ = time_rotating(torch, stream, fnsr, args.steps, 20)
        msr = sum(perr) / len(perr)
        extra["scan1d_fwd_f32_rotating_2_sets"] = {
            "ms": round(msr, 4), "frac_hbm": round(alg / (msr * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del x2, dt2, B2, C2, y2, fnsr

        # Measured copy peak (1 GiB read + 1 GiB written), beside the 8 TB/s
        # nominal.
        extra["copy_1GiB"] = bench_copy(torch, stream, max(10, args.steps // 5), 5)

        # Generic decays: the same workload with A perturbed off the S4D-real
        # structure, which disables the power-chain path (one exp per state).
        Ag = A * (1.0 + 0.01 * torch.rand(A.shape, device="cuda", generator=torch.Generator(
            device="cuda").manual_seed(7)))
        fng = lambda: K.scan1d_fwd(x, dt, Ag, Bm, Cm, y, h_final=hf, stream=stream)  # noqa: E731
        perg, _ = time_launches(torch, stream, fng, args.steps, 20)
        msg = sum(perg) / len(perg)
        extra["scan1d_fwd_f32_generic_A"] = {
            "ms": round(msg, 4), "elems_per_s": elems / (msg * 1e-3),
            "achieved_GBs": round(alg / (msg * 1e-3) / 1e9, 1),
            "frac_hbm": round(alg / (msg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}

        # The headline: W warm-up steps, then exactly K timed steps.
        fn = lambda: K.scan1d_fwd(x, dt, A, Bm, Cm, y, h_final=hf, stream=stream)  # noqa: E731
        per, wall = time_launches(torch, stream, fn, args.steps, args.warmup)
        ms = sum(per) / len(per)
        ach = alg / (ms * 1e-3) / 1e9

    traffic = None
    tf = ROOT / "profiles" / "scan1d_fwd_c1_traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC,
        "value": elems / (ms * 1e-3),
        "unit": "elems/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "Scan1D selective-scan forward, configs[1]: B=8 L=4096 D=1024 N=16, "
                               "fp32, B/C shared over channels [B,L,N], A=-(1..N) (S4D-real; the "
                               "kernel detects A[d,n]=(n+1)A[d,0] and uses one exp per step plus a "
                               "power chain; the one-exp-per-state path is in extra)",
                   "B": Bsz, "L": L, "D": D, "N": N},
        "state_updates_per_s": elems * N / (ms * 1e-3),
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "measured_copy_GBs": extra["copy_1GiB"]["GBs_read_plus_write"],
                     "frac_of_measured_copy": round(ach / extra["copy_1GiB"]["GBs_read_plus_write"], 4),
                     "traffic_source": "profiles/scan1d_fwd_c1_traffic.json: rocprofv3 TCC read "
                                       "requests by size and write requests of this kernel (the same "
                                       "formulas read a 1 GiB copy exactly)",
                     "kernel": "km::scan1d_fwd_chunked (fp32, B/C shared over channels)",
                     "alg_bytes": alg,
                     "avg_launch_ms": round(ms, 5)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()

"""GPU parity of the Mamba-3 block forward (mamba_block_forward, the
reference src/mamba_block.c:471-501) against the oracle restatement, which
is bit-exact to the compiled reference (test_oracle_pins.py).

Metric: the block's contribution out - x (the residual is exact) compared
normwise: max |got - ref| / max |ref| <= 1e-4 (fp32).
"""
import ctypes as C

import numpy as np
import pytest

import kmamba as K
import oracle as O
from kmtest import rng_for
from test_oracle_pins import mamba3_params

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    torch.zeros(1, device="cuda")
    assert K.kmamba_cuda_available() == 1, K.km_last_error()


def make_block(D, N, L, R, params, dt_min=0.01, dt_max=0.5):
    cfg = K.MBConfig()
    cfg.dim, cfg.state_size, cfg.seq_len, cfg.mimo_rank = D, N, L, R
    cfg.dt_scale, cfg.dt_min, cfg.dt_max = 0.1, dt_min, dt_max
    blk = K.mamba_block_create(C.byref(cfg))
    assert blk, K.km_last_error()
    O.set_block_params(C.cast(blk, C.POINTER(O.MambaBlock)), params)
    return blk


def check(got, want, x, tol=1e-4):
    dg, dw = got - x, want - x
    err = np.abs(dg - dw).max() / max(np.abs(dw).max(), 1e-30)
    assert err <= tol, f"normwise error of out - x: {err:.3e}"
    return err


@pytest.mark.parametrize("D,N,L,R,batch", [(24, 8, 37, 2, 3), (16, 16, 64, 1, 2), (10, 7, 20, 1, 1),
                                           (33, 4, 9, 3, 2), (8, 1, 5, 1, 1), (64, 16, 300, 1, 4),
                                           # 101 controller rows: two row groups of 64
                                           (32, 16, 40, 3, 2)])
def test_forward_host_pointers_vs_oracle(D, N, L, R, batch):
    p = mamba3_params(D, N, R)
    x = rng_for("m3x", D, N, L).standard_normal((batch, L, D)).astype(np.float32)
    want = O.mamba3_forward(p, x, dt_min=0.01, dt_max=0.5)
    blk = make_block(D, N, L, R, p)
    out = np.full_like(x, np.nan)
    K.mamba_block_forward(blk, K.ptr(out), K.ptr(x), batch)
    assert K.km_last_error() == ""
    check(out, want, x)
    K.mamba_block_free(blk)


def test_forward_device_pointers_and_reference_init():
    # Parameters from mamba_block_init (the reference's rand() initialisation).
    D, N, L, R, batch = 128, 16, 512, 1, 2
    cfg = K.MBConfig()
    cfg.dim, cfg.state_size, cfg.seq_len, cfg.mimo_rank = D, N, L, R
    cfg.dt_scale, cfg.dt_min, cfg.dt_max = 0.1, 1e-3, 0.1
    blk = K.mamba_block_create(C.byref(cfg))
    C.CDLL(None).srand(7)
    K.mamba_block_init(blk)
    p = O.block_params(C.cast(blk, C.POINTER(O.MambaBlock)))
    x = rng_for("m3dev").standard_normal((batch, L, D)).astype(np.float32)
    want = O.mamba3_forward(p, x, dt_min=1e-3, dt_max=0.1)
    tx = torch.from_numpy(x).cuda()
    tout = torch.empty_like(tx)
    K.mamba_block_forward(blk, K.ptr(tout), K.ptr(tx), batch)
    assert K.km_last_error() == ""
    check(tout.cpu().numpy(), want, x)
    K.mamba_block_free(blk)


def test_forward_rejects_invalid():
    K.mamba_block_forward(None, None, None, 1)
    assert "invalid" in K.km_last_error()


def test_forward_larger_model_sampled():
    # dim 1024, N 16, L 2048 (the configs[4] sequence and width), batch 2.
    D, N, L, R, batch = 1024, 16, 2048, 1, 2
    p = mamba3_params(D, N, R, seed=3)
    x = rng_for("m3big").standard_normal((batch, L, D)).astype(np.float32)
    blk = make_block(D, N, L, R, p)
    out = np.empty_like(x)
    K.mamba_block_forward(blk, K.ptr(out), K.ptr(x), batch)
    assert K.km_last_error() == ""
    want = O.mamba3_forward(p, x[:1], dt_min=0.01, dt_max=0.5)
    check(out[:1], want, x[:1])
    K.mamba_block_free(blk)


# ---------------------------------------------------------------------------
# The stacked model (kmamba_forward, ref src/kmamba.c:344-372)
# ---------------------------------------------------------------------------
def model_forward(m, toks):
    c = m.contents.cfg
    logits = np.full((c.seq_len, c.vocab_size), np.nan, np.float32)
    assert K.kmamba_forward(m, toks.ctypes.data, logits.ctypes.data) == 0, K.km_last_error()
    return logits


@pytest.mark.parametrize("V,D,N,L,layers,R,tying", [
    (37, 12, 6, 9, 2, 1, 0),          # ragged everything, below one head tile
    (97, 64, 16, 130, 2, 1, 1),       # tied head, M spans three row tiles
    (300, 40, 8, 77, 3, 2, 0),        # MIMO rank 2, N spans five column tiles
    (4096, 256, 16, 512, 2, 1, 0),    # 16 K steps, 64 x 8 head tiles
])
def test_kmamba_forward_vs_oracle(V, D, N, L, layers, R, tying):
    # Logits against the oracle's model forward (bit-exact to the compiled
    # reference) on this model's own parameters. Metric: condition-scaled,
    # max |got - ref| / (|h| . |head|) <= 1e-4 with h the oracle's last
    # block output (the head's sums carry no cancellation in that scale).
    m = K.kmamba_create(C.byref(O.kmamba_config(V, D, N, L, layers, R=R, weight_tying=tying,
                                                cls=K.KMambaConfig)))
    assert m, K.km_last_error()
    assert K.kmamba_init(m, 11) == 0
    toks = rng_for("kmgpu", V, L).integers(0, V + 3, L).astype(np.uint32)
    got = model_forward(m, toks)
    emb, head, blocks = O.model_params(C.cast(m, C.POINTER(O.KMamba)))
    want = O.kmamba_forward(emb, head, blocks, toks)
    x = np.zeros((1, L, D), np.float32)
    ok = toks < V
    x[0, ok] = emb[toks[ok]]
    for p in blocks:
        x = O.mamba3_forward(p, x)
    kappa = np.abs(x[0]).astype(np.float64) @ np.abs(head).astype(np.float64)
    err = float(np.max(np.abs(got.astype(np.float64) - want) / np.maximum(kappa, 1e-30)))
    K.kmamba_free(m)
    assert np.isfinite(got).all()
    assert err <= 1e-4, f"condition-scaled logits error {err:.3e}"


def test_kmamba_forward_pipelined_copies_many_pieces():
    # A head (41 MB) and logits (96 MB) that span several slots of the pinned
    # ring, with ragged last pieces and download pieces (52 rows each) that
    # straddle the 256-row chunks of the head product. Logits against
    # float64 products of the oracle's last block output, condition-scaled
    # as above; a second, smaller model afterwards reuses the ring.
    V, D, N, L = 40000, 256, 16, 600
    m = K.kmamba_create(C.byref(O.kmamba_config(V, D, N, L, 2, cls=K.KMambaConfig)))
    assert m and K.kmamba_init(m, 5) == 0, K.km_last_error()
    toks = rng_for("kmpipe", V, L).integers(0, V + 2, L).astype(np.uint32)
    got = model_forward(m, toks)
    emb, head, blocks = O.model_params(C.cast(m, C.POINTER(O.KMamba)))
    x = np.zeros((1, L, D), np.float32)
    ok = toks < V
    x[0, ok] = emb[toks[ok]]
    for p in blocks:
        x = O.mamba3_forward(p, x)
    want = x[0].astype(np.float64) @ head.astype(np.float64)
    kappa = np.abs(x[0]).astype(np.float64) @ np.abs(head).astype(np.float64)
    err = float(np.max(np.abs(got - want) / np.maximum(kappa, 1e-30)))
    K.kmamba_free(m)
    assert np.isfinite(got).all()
    assert err <= 1e-4, f"condition-scaled logits error {err:.3e}"
    m2 = K.kmamba_create(C.byref(O.kmamba_config(97, 64, 16, 130, 2, cls=K.KMambaConfig)))
    assert m2 and K.kmamba_init(m2, 6) == 0
    t2 = rng_for("kmpipe2").integers(0, 97, 130).astype(np.uint32)
    got2 = model_forward(m2, t2)
    emb2, head2, blocks2 = O.model_params(C.cast(m2, C.POINTER(O.KMamba)))
    want2 = O.kmamba_forward(emb2, head2, blocks2, t2)
    K.kmamba_free(m2)
    np.testing.assert_allclose(got2, want2, rtol=0, atol=1e-4 * float(np.abs(want2).max()))


def test_kmamba_checkpoint_roundtrip_forward(tmp_path):
    # A saved and reloaded model (untied on load) gives the same logits.
    V, D, N, L = 200, 32, 8, 50
    m = K.kmamba_create(C.byref(O.kmamba_config(V, D, N, L, 2, weight_tying=1, cls=K.KMambaConfig)))
    assert m and K.kmamba_init(m, 4) == 0
    toks = rng_for("kmrt", V, L).integers(0, V, L).astype(np.uint32)
    a = model_forward(m, toks)
    path = str(tmp_path / "m.kmamba").encode()
    assert K.kmamba_save(m, path) == 0
    m2 = K.kmamba_load(path, 0, None, 0.0, 0.0)
    assert m2, K.km_last_error()
    assert m2.contents.cfg.weight_tying == 0
    b = model_forward(m2, toks)
    np.testing.assert_array_equal(a, b)
    # The blocks' hidden / scan_h are cleared by the forward (src/kmamba.c:351-354).
    blk = m2.contents.layers[0].contents
    assert not np.any(np.ctypeslib.as_array(blk.hidden, shape=(N,)))
    assert K.kmamba_forward(m2, None, a.ctypes.data) == -1
    assert "NULL" in K.km_last_error()
    K.kmamba_free(m)
    K.kmamba_free(m2)

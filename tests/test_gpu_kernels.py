"""GPU parity of the HIP kernels against the CPU oracle, through the C ABI.

Bit-exact for every output: the kernels follow the oracle's evaluation order
(integer-limb q4 dot products, fixed float fold orders, the shared exp).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, empty_bf16, host, need_gpu, qweights, rand_bf16  # noqa: E402


@pytest.fixture(scope="module")
def ctx():
    need_gpu()
    import mtpx
    c = mtpx.Context(0)
    yield c
    c.close()


def _print_case(**kw):
    print("case", kw, flush=True)


# ---------------------------------------------------------------------------- a1
@pytest.mark.parametrize("rows,K,gs", [(64, 2560, 64), (33, 640, 32), (8, 2048, 64)])
def test_quantize_bit_exact(ctx, rows, K, gs):
    _print_case(rows=rows, K=K, gs=gs)
    r = np.random.default_rng(rows + K)
    w = rand_bf16(r, (rows, K), 0.02)
    # edge groups: constant, zeros, a single outlier, all negative
    w[0, :gs] = O.f32_to_bf16(np.full(gs, 0.5, np.float32))
    w[1, :gs] = 0
    w[2, :gs] = O.f32_to_bf16(np.r_[np.zeros(gs - 1), -3.0].astype(np.float32))
    w[3, :gs] = O.f32_to_bf16(-np.abs(r.standard_normal(gs)).astype(np.float32))
    wq_o, s_o, b_o = O.affine_quantize(w, gs)
    wd = dev(w)
    wq = torch.zeros(rows, K // 8, dtype=torch.int32, device="cuda")
    s = empty_bf16(rows, K // gs)
    b = empty_bf16(rows, K // gs)
    ctx.affine_quantize(wd, gs, wq, s, b)
    ctx.synchronize()
    assert np.array_equal(host(wq).view(np.uint32), wq_o)
    assert np.array_equal(host(s), s_o)
    assert np.array_equal(host(b), b_o)


def test_randn_deterministic_and_normal(ctx):
    a = empty_bf16(1 << 20)
    b = empty_bf16(1 << 20)
    ctx.randn_bf16(a, 7, 3, 0.02)
    ctx.randn_bf16(b, 7, 3, 0.02)
    ctx.synchronize()
    ha, hb = host(a), host(b)
    assert np.array_equal(ha, hb)
    v = O.bf16_to_f32(ha).astype(np.float64)
    assert abs(v.mean()) < 1e-4 and abs(v.std() - 0.02) < 2e-4


# ---------------------------------------------------------------------------- a2-a4, a12
@pytest.mark.parametrize("N,K,gs,M", [
    (640, 2560, 64, 1), (1280, 2560, 32, 4), (2560, 640, 64, 6), (2048, 768, 64, 2),
    (768, 2048, 32, 1), (256, 6144, 64, 4), (100, 256, 32, 8), (13440, 2560, 64, 7), (37, 320, 32, 3),
    (300, 6144, 64, 8), (64, 96, 32, 5),
    # matrix-core path (2..4 tokens per launch, packed pairs): the model's dense shapes, ragged rows
    (16480, 2560, 64, 4), (2560, 6144, 64, 4), (1000, 2560, 64, 3), (2560, 6144, 32, 2), (4096, 2048, 64, 4),
    (520, 10240, 64, 4), (2560, 2560, 32, 5),
    # one token group, several tile groups per workgroup: ragged rows
    (66001, 2560, 64, 3), (65550, 2560, 32, 4),
    # two token groups in one launch (5..8 tokens): ragged rows, several tile groups per workgroup
    (16480, 2560, 64, 6), (1000, 2560, 64, 8), (66000, 2560, 64, 5), (4096, 2048, 64, 8), (13440, 2560, 32, 7),
    # one token group whose eight-wave tile groups just outnumber the CUs: ten-wave workgroups, ragged last tile
    # (one window, and two windows of four)
    (16470, 2560, 32, 4), (16470, 2560, 64, 6),
    # the dot-product kernel's equal windows past the CU count: five-wave workgroups (two windows of 2 and of 3
    # tokens, a ragged last workgroup); three tokens (2 + 1) keep four waves
    (2560, 6144, 64, 6), (2490, 6144, 64, 4), (2560, 6144, 64, 3), (2560, 6144, 32, 8),
])
def test_qmv_bit_exact(ctx, N, K, gs, M):
    _print_case(N=N, K=K, gs=gs, M=M)
    r = np.random.default_rng(N * 7 + K + M)
    wq, s, b = qweights(r, N, K, gs)
    x = rand_bf16(r, (M, K))
    y_o, yf_o = O.qmv(wq, s, b, gs, x)
    ds, db = dev(s), dev(b)
    for sb in (None, ctx.pack_sb(ds, db, K, gs)):  # checkpoint scale/bias rows, then the packed pairs
        y = empty_bf16(M, N)
        yf = torch.zeros(M, N, dtype=torch.float32, device="cuda")
        ctx.qmv(dev(wq), ds, db, gs, dev(x), y, yf, sb=sb)
        ctx.synchronize()
        assert np.array_equal(host(yf).view(np.uint32), yf_o.view(np.uint32))
        assert np.array_equal(host(y), y_o)


# more than 8 tokens: the batch GEMM (packed pairs, 1024 rows or more) at every chain depth it takes, ragged
# rows and token blocks; fewer rows (and checkpoint pairs): the windowed GEMV
@pytest.mark.parametrize("N,K,gs,M", [
    (2000, 2560, 64, 37), (1100, 6144, 64, 21), (1100, 10240, 64, 9), (2560, 2560, 32, 64), (1030, 2048, 64, 100),
    (1030, 512, 64, 33), (1030, 640, 32, 17), (1150, 6144, 32, 40), (330, 10240, 64, 9), (4, 10240, 64, 19),
])
def test_qmv_batch_gemm_bit_exact(ctx, N, K, gs, M):
    _print_case(N=N, K=K, gs=gs, M=M)
    r = np.random.default_rng(N * 11 + K + M)
    wq, s, b = qweights(r, N, K, gs)
    x = rand_bf16(r, (M, K))
    y_o, yf_o = O.qmv(wq, s, b, gs, x)
    ds, db = dev(s), dev(b)
    for sb in (None, ctx.pack_sb(ds, db, K, gs)):
        y = empty_bf16(M, N)
        yf = torch.zeros(M, N, dtype=torch.float32, device="cuda")
        ctx.qmv(dev(wq), ds, db, gs, dev(x), y, yf, sb=sb)
        ctx.synchronize()
        assert np.array_equal(host(yf).view(np.uint32), yf_o.view(np.uint32))
        assert np.array_equal(host(y), y_o)


@pytest.mark.parametrize("N,K", [(16480, 2560), (13440, 2560), (2560, 6144), (320, 10240)])
def test_qmv_batch_gemm_matches_windows(ctx, N, K):
    """A prefill batch of 256 tokens at the model's shapes: the GEMM's rows equal the windows of 8."""
    _print_case(N=N, K=K, M=256)
    r = np.random.default_rng(N + K)
    wq, s, b = qweights(r, N, K, 64)
    ds, db, dq = dev(s), dev(b), dev(wq)
    sb = ctx.pack_sb(ds, db, K, 64)
    x = dev(rand_bf16(r, (256, K)))
    y = empty_bf16(256, N)
    yf = torch.zeros(256, N, dtype=torch.float32, device="cuda")
    ctx.qmv(dq, ds, db, 64, x, y, yf, sb=sb)
    yw = torch.zeros(256, N, dtype=torch.float32, device="cuda")
    for w0 in range(0, 256, 8):
        ctx.qmv(dq, ds, db, 64, x[w0:w0 + 8], empty_bf16(8, N), yw[w0:w0 + 8], sb=sb)
    ctx.synchronize()
    assert torch.equal(yf.view(torch.int32), yw.view(torch.int32))


def test_qmv_repeat_is_bit_stable(ctx):
    r = np.random.default_rng(5)
    wq, s, b = qweights(r, 512, 2560, 64)
    x = dev(rand_bf16(r, (3, 2560)))
    outs = []
    for _ in range(3):
        y = empty_bf16(3, 512)
        ctx.qmv(dev(wq), dev(s), dev(b), 64, x, y)
        ctx.synchronize()
        outs.append(host(y))
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def test_qmv_rejects_bad_shapes(ctx):
    import mtpx
    r = np.random.default_rng(0)
    wq, s, b = qweights(r, 8, 256, 32)
    with pytest.raises(mtpx.MtpxError):
        ctx.qmv(dev(wq), dev(s), dev(b), 48, dev(rand_bf16(r, (1, 256))), empty_bf16(1, 8))
    with pytest.raises(mtpx.MtpxError):
        ctx.qmv(dev(wq), dev(s), dev(b), 32, dev(rand_bf16(r, (4097, 256))), empty_bf16(4097, 8))


# ---------------------------------------------------------------------------- rmsnorm / add
def test_rmsnorm_bit_exact(ctx):
    r = np.random.default_rng(11)
    x = rand_bf16(r, (5, 2560), 3.0)
    res = rand_bf16(r, (5, 2560), 1.0)
    w = O.f32_to_bf16((1 + 0.1 * r.standard_normal(2560)).astype(np.float32))
    y_o = O.rmsnorm(x, w, 1e-6)
    y = empty_bf16(5, 2560)
    ctx.rmsnorm(dev(x), dev(w), 1e-6, y)
    ctx.synchronize()
    assert np.array_equal(host(y), y_o)
    s_o = O.f32_to_bf16(O.bf16_to_f32(x) + O.bf16_to_f32(res))
    y2_o = O.rmsnorm(s_o, w, 1e-6)
    s = empty_bf16(5, 2560)
    ctx.rmsnorm(dev(x), dev(w), 1e-6, y, resid=dev(res), sum_out=s)
    ctx.synchronize()
    assert np.array_equal(host(s), s_o)
    assert np.array_equal(host(y), y2_o)

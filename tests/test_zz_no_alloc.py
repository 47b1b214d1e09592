"""The allocation-free MoE entry point (mtpx_moe_forward_noalloc) against mtpx_moe_forward through
the C ABI, bit-exact, on two calls in a row (the second with a smaller window, so stale scratch
from the first call is present), at the model's full MoE shape and at a small one; a window whose
workspace exceeds the scratch is refused."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

from gpu_util import dev, host, need_gpu, rand_bf16  # noqa: E402

FULL = dict(hidden=2560, experts=512, top_k=10, expert_width=640, heads=24, kv_heads=2, head_dim=256, rot_dims=64,
            index_dim=128, rope_theta=1e7, eps=1e-6, max_positions=64)
SMALL = dict(hidden=512, experts=16, top_k=4, expert_width=256, heads=8, kv_heads=2, head_dim=64, rot_dims=16,
             index_dim=32, rope_theta=1e7, eps=1e-6, max_positions=64)


def _run(ctx, fn, mw, x, K):
    M, H = x.shape
    y = torch.zeros(M, H, dtype=torch.bfloat16, device="cuda")
    idx = torch.full((M, K), -1, dtype=torch.int32, device="cuda")
    wts = torch.zeros(M, K, dtype=torch.float32, device="cuda")
    nu = torch.zeros(1, dtype=torch.int32, device="cuda")
    fn(mw, x, y, idx, wts, None, nu)
    ctx.synchronize()
    return host(y), host(idx), host(wts), int(host(nu)[0])


@pytest.mark.parametrize("cfg,gs", [(FULL, 64), (SMALL, 32)], ids=["full-gs64", "small-gs32"])
def test_noalloc_moe_matches_moe_forward(cfg, gs):
    need_gpu()
    import mtpx
    ctx = mtpx.Context(0)
    layer = mtpx.DecoderLayer(ctx, mtpx.LayerConfig(**dict(cfg, group_size=gs)), seed=71)
    mw = layer.weights().moe
    r = np.random.default_rng(72)
    for M in (8, 2):  # the second call is smaller: the scratch still holds the first call's data
        print("case noalloc", cfg["hidden"], gs, "M", M, flush=True)
        x = dev(rand_bf16(r, (M, cfg["hidden"])))
        want = _run(ctx, ctx.moe_forward, mw, x, cfg["top_k"])
        got = _run(ctx, ctx.moe_forward_noalloc, mw, x, cfg["top_k"])
        for a, b in zip(got[:3], want[:3]):
            assert np.array_equal(a, b)
        assert got[3] == want[3]
    layer.close()
    ctx.close()


def test_noalloc_refuses_windows_past_the_scratch():
    need_gpu()
    import mtpx
    from mtpx import MoEWeights
    ctx = mtpx.Context(0)
    H, E, K, F, gs = 4096, 16, 16, 4096, 64  # 8 tokens x 17 slots x (4096 + 4096) bf16 > 2 MiB
    z = torch.zeros(64, dtype=torch.int32, device="cuda")  # never read: the call is refused before any launch
    w = MoEWeights(H, E, K, F, gs)
    for name, _ in MoEWeights._fields_[5:]:
        setattr(w, name, None if name.endswith("_sb") else z.data_ptr())
    x = torch.zeros(8, H, dtype=torch.bfloat16, device="cuda")
    y = torch.zeros(8, H, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(mtpx.MtpxError, match="scratch"):
        ctx.moe_forward_noalloc(w, x, y)
    ctx.close()


def test_noalloc_scratch_belongs_to_one_context():
    """The device's scratch array serves one context at a time: a second context on the same GPU is
    refused (MTPX_ERR_STATE) while the first one lives, and gets it once the first is freed.  A
    refused call launches nothing; mtpx_last_moe_bytes does not count allocation-free calls."""
    need_gpu()
    import mtpx
    a, b = mtpx.Context(0), mtpx.Context(0)
    layer = mtpx.DecoderLayer(b, mtpx.LayerConfig(**dict(SMALL, group_size=32)), seed=73)  # outlives a
    mw = layer.weights().moe
    x = dev(rand_bf16(np.random.default_rng(74), (2, SMALL["hidden"])))
    print("case noalloc two contexts", flush=True)
    want = _run(a, a.moe_forward, mw, x, SMALL["top_k"])
    assert _run(a, a.moe_forward_noalloc, mw, x, SMALL["top_k"])[3] == want[3]
    with pytest.raises(mtpx.MtpxError, match="another context"):
        _run(b, b.moe_forward_noalloc, mw, x, SMALL["top_k"])
    with pytest.raises(mtpx.MtpxError, match="allocation-free"):
        a.last_moe_bytes()
    a.close()
    got = _run(b, b.moe_forward_noalloc, mw, x, SMALL["top_k"])
    for u, v in zip(got[:3], want[:3]):
        assert np.array_equal(u, v)
    layer.close()
    b.close()

"""GPU parity of one decoder layer (rmsnorm, qkv GEMV, prep + KV append, verify
attention + gate, o_proj, residual, rmsnorm, MoE, residual) against the oracle
composed layer by layer, bit-exact, across a prefill window, a verify window, a
rollback and the re-verify after it."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, empty_bf16, host, need_gpu, rand_bf16  # noqa: E402
from oracle.layer_ref import download, oracle_layer  # noqa: E402

CFG = dict(hidden=512, experts=16, top_k=4, expert_width=256, group_size=64, heads=8, kv_heads=2, head_dim=64,
           rot_dims=16, index_dim=32, rope_theta=1e7, eps=1e-6, max_positions=64)


def test_layer_windows_and_rollback_bit_exact():
    need_gpu()
    import mtpx
    ctx = mtpx.Context(0)
    cfg = CFG
    lc = mtpx.LayerConfig(**cfg)
    layer = mtpx.DecoderLayer(ctx, lc, seed=42)
    kv = mtpx.KVCache(ctx, cfg["kv_heads"], cfg["head_dim"], cfg["max_positions"])
    w = download(layer.weights(), cfg)
    HK, D, P, H = cfg["kv_heads"], cfg["head_dim"], cfg["max_positions"], cfg["hidden"]
    kc = np.zeros((HK, P, D), np.uint16)
    vc = np.zeros_like(kc)
    r = np.random.default_rng(1)
    steps = [("fwd", 8), ("fwd", 4), ("trim", 2), ("fwd", 3), ("fwd", 1)]
    pos = 0
    for kind, n in steps:
        print("case layer", kind, n, "pos", pos, flush=True)
        if kind == "trim":
            assert kv.trim(n) == n
            pos -= n
            continue
        x = rand_bf16(r, (n, H))
        want = oracle_layer(w, cfg, kc, vc, x, pos)
        y = empty_bf16(n, H)
        layer.forward(kv, dev(x), y)
        ctx.synchronize()
        pos += n
        assert kv.offset == pos
        got = host(y)
        assert np.array_equal(got, want), np.abs(O.bf16_to_f32(got) - O.bf16_to_f32(want)).max()
    layer.close()
    kv.close()
    ctx.close()

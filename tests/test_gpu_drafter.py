"""GPU parity of the drafter's rounds (mtpx_drafter) against the oracle head:
an observed target chunk flushed through the head in windows of at most eight
inputs (checked against one oracle pass over all of them), chained speculative
steps, finalize with one committed draft, the next round's flush, discard, the
round after the discard from the rolled-back cache, and the refused
out-of-sequence calls, all through the C ABI."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

from gpu_util import dev, empty_bf16, host, need_gpu, rand_bf16  # noqa: E402

LAYER = dict(hidden=256, experts=16, top_k=4, expert_width=128, group_size=32, heads=4, kv_heads=2, head_dim=64,
             rot_dims=16, index_dim=32, rope_theta=1e7, eps=1e-6, max_positions=64)
HC, LOWRANK, VOCAB = 4, 64, 1000


def test_drafter_rounds_bit_exact():
    need_gpu()
    import mtpx
    from oracle.head_ref import download_head, oracle_head
    ctx = mtpx.Context(0)
    hcfg = mtpx.HeadConfig(mtpx.LayerConfig(**LAYER), HC, LOWRANK, VOCAB, 500, 980)
    head = mtpx.MTPHead(ctx, hcfg, seed=5)
    cfg = dict(LAYER, hc=HC, lowrank=LOWRANK, vocab=VOCAB)
    ow = download_head(head.weights(), cfg)
    dr = mtpx.Drafter(ctx, head)
    H, W = LAYER["hidden"], HC * LAYER["hidden"]
    HK, D, P = LAYER["kv_heads"], LAYER["head_dim"], LAYER["max_positions"]
    kc = np.zeros((HK, P, D), np.uint16)
    vc = np.zeros_like(kc)
    r = np.random.default_rng(3)
    assert dr.bytes_per_token() == (2 * HK * D + LAYER["index_dim"]) * 2 + W * 2 + 4

    def out_bufs():
        return torch.full((1,), -1, dtype=torch.int32, device="cuda"), empty_bf16(1, W)

    # observe a 12-token target chunk: 11 transitions in the backlog, frontier = row 11
    toks = r.integers(0, VOCAB, 12).astype(np.int32)
    hid = rand_bf16(r, (12, W))
    dr.observe(dev(toks), dev(hid))
    info = dr.info()
    assert info["backlog_inputs"] == 11 and info["has_frontier"] == 1 and info["cache_offset"] == 0

    # round 1, step 1: flush (hid[t], toks[t+1]) for t < 11 plus the carry -> 12 head inputs (windows 8 + 4)
    carry_t = np.array([7], np.int32)
    carry_h = rand_bf16(r, (1, W))
    print("case drafter flush 12", flush=True)
    d1, m1 = out_bufs()
    dr.step(dev(carry_t), dev(carry_h), d1, m1)
    ids = np.concatenate([toks[1:], carry_t])
    mult = np.concatenate([hid[:11], carry_h])
    want_mn, _, want_d = oracle_head(ow, cfg, kc, vc, ids, mult, 0)
    assert int(host(d1)[0]) == want_d
    assert np.array_equal(host(m1), want_mn[-1:])
    info = dr.info()
    assert info["cache_offset"] == 12 and info["round_valid_offset"] == 12 and info["round_in_flight"] == 1

    # step 2: the previous draft and multi fed back (speculative)
    print("case drafter chain", flush=True)
    d2, m2 = out_bufs()
    dr.step(d1, m1, d2, m2)
    want_mn2, _, want_d2 = oracle_head(ow, cfg, kc, vc, np.array([want_d], np.int32), want_mn[-1:], 12)
    assert int(host(d2)[0]) == want_d2
    assert np.array_equal(host(m2), want_mn2)
    assert dr.info()["staged_inputs"] == 1

    # finalize: 2 confirmed inputs, 1 committed draft with the target's multi at its position
    tgt_h = rand_bf16(r, (1, W))
    dr.finalize(2, dev(np.array([want_d], np.int32)), dev(tgt_h))
    info = dr.info()
    assert info["cache_offset"] == 12 and info["backlog_inputs"] == 1 and info["round_in_flight"] == 0
    assert info["committed_inputs"] == 13

    # round 2: flush (committed draft, carry), one speculative step, then discard
    carry2_t = np.array([42], np.int32)
    carry2_h = rand_bf16(r, (1, W))
    ids2 = np.array([want_d, 42], np.int32)
    mult2 = np.concatenate([tgt_h, carry2_h])
    want_mn3, _, want_d3 = oracle_head(ow, cfg, kc, vc, ids2, mult2, 12)
    print("case drafter round 2", flush=True)
    d3, m3 = out_bufs()
    dr.step(dev(carry2_t), dev(carry2_h), d3, m3)
    assert int(host(d3)[0]) == want_d3
    assert np.array_equal(host(m3), want_mn3[-1:])
    d4, m4 = out_bufs()
    dr.step(d3, m3, d4, m4)
    assert dr.info()["cache_offset"] == 15
    dr.discard()
    info = dr.info()
    assert info["cache_offset"] == 12 and info["backlog_inputs"] == 2 and info["round_in_flight"] == 0
    # round 3 after the discard: the restored transitions plus the new carry, from the rolled-back cache
    carry3_t = np.array([43], np.int32)
    carry3_h = rand_bf16(r, (1, W))
    ids3 = np.array([want_d, 42, 43], np.int32)
    mult3 = np.concatenate([tgt_h, carry2_h, carry3_h])
    want_mn5, _, want_d5 = oracle_head(ow, cfg, kc, vc, ids3, mult3, 12)
    print("case drafter round 3", flush=True)
    d5, m5 = out_bufs()
    dr.step(dev(carry3_t), dev(carry3_h), d5, m5)
    assert int(host(d5)[0]) == want_d5
    assert np.array_equal(host(m5), want_mn5[-1:])
    # out-of-sequence calls are refused with the state unchanged
    with pytest.raises(mtpx.MtpxError):
        dr.observe(dev(toks[:2]), dev(hid[:2]))  # during a round
    with pytest.raises(mtpx.MtpxError):
        dr.finalize(3)  # confirmed prefix beyond the round
    dr.finalize(1)
    info = dr.info()
    assert info["cache_offset"] == 15 and info["backlog_inputs"] == 0 and info["committed_inputs"] == 15
    dr.release()
    with pytest.raises(mtpx.MtpxError):
        dr.step(dev(carry_t), dev(carry_h), *out_bufs())
    dr.close()
    head.close()
    ctx.close()

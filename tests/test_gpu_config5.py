"""BASELINE config 5 at full shape through the C ABI: the random-init 48-layer gs64 target (36 GDN +
12 attention layers, hyper-connection mixers, 512-expert top-10 + shared MoE, vocab 248320) with the
PLE block on layer 1 (its full 320,001,446-row table resident) and the full-dims MTP head (the
98,584-row shortlist).

* A 1024-token random prompt goes through mtpx_session_prefill (two batches of 512 positions).
* The serial decode's next tokens are checked against the oracle's 48-layer verify chain started
  from the committed state the prefill left, read back from the device (KV caches, GDN conv and
  recurrent states, the PLE block's conv rows and context).  The prefill itself equals the windowed
  verify path (tests/test_gpu_prefill.py) and the windowed verify equals the oracle at this shape
  (tests/test_gpu_fullshape.py).
* Every draft depth 1..5 with the forcing hook at p = 0.7 decodes 64 tokens in a fresh session and
  emits exactly the serial sequence; each round accepts exactly the run of forced positions after
  its carry (the forcing mask read back through the hook), capped at the depth.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, need_gpu, read_device  # noqa: E402

FULL = dict(hidden=2560, experts=512, top_k=10, expert_width=640, heads=24, kv_heads=2, head_dim=256, rot_dims=64,
            index_dim=128, rope_theta=1e7, eps=1e-6)
LINEAR = dict(key_heads=16, value_heads=48, conv_kernel=4, full_attention_interval=4, hc=4, lowrank=320, vocab=248320)
PROMPT, GEN, P = 1024, 64, 1152
RATE, FSEED = 0.7, 0x5EED0009


@pytest.fixture(scope="module")
def model():
    need_gpu()
    import mtpx
    ctx = mtpx.Context(0)
    lc = dict(FULL, group_size=64, max_positions=P)
    tc = mtpx.TargetConfig(mtpx.LayerConfig(**lc), LINEAR["key_heads"], LINEAR["value_heads"], LINEAR["conv_kernel"],
                           48, LINEAR["full_attention_interval"], LINEAR["hc"], LINEAR["lowrank"], LINEAR["vocab"])
    tc.ple_layer = 1
    tc.ple = mtpx.PLEConfig(hidden=2560, hc=4, embed_dim=2560, ngram_size=3, heads_per_ngram=8, conv_kernel=4,
                            group_size=64, row_group_size=32, eos=248044, vocab_base=20_000_000, token_vocab=248320,
                            eps=FULL["eps"])
    print("case config5: building the 48-layer target and the head", flush=True)
    t = mtpx.Target(ctx, tc, seed=0x5EED0004)
    head = mtpx.MTPHead(ctx, mtpx.HeadConfig(mtpx.LayerConfig(**lc), LINEAR["hc"], LINEAR["lowrank"],
                                             LINEAR["vocab"], 98304, 248044), seed=0x5EED0007)
    prompt = np.random.default_rng(0x5EED0005).integers(0, LINEAR["vocab"], PROMPT).astype(np.int32)
    cfg = dict(lc, **LINEAR, num_layers=48, ple_layer=1)
    yield ctx, t, head, prompt, cfg
    head.close()
    t.close()
    ctx.close()


def _read_state(st, kinds, cfg):
    """The committed state of a target state on the host, in the oracle's layout."""
    HK, D, hc, H = cfg["kv_heads"], cfg["head_dim"], cfg["hc"], cfg["hidden"]
    out = dict(kc={}, vc={}, conv={}, ssm={})
    for i, kind in enumerate(kinds):
        if kind == 1:
            kp, vp, tmax = st.kv(i).buffers()
            out["kc"][i] = read_device(kp, HK * tmax * D * 2, np.uint16).reshape(HK, tmax, D).copy()
            out["vc"][i] = read_device(vp, HK * tmax * D * 2, np.uint16).reshape(HK, tmax, D).copy()
        else:
            g = O.gdn_geom(cfg["key_heads"], cfg["value_heads"], cfg["conv_kernel"])
            conv = torch.zeros(g.kc - 1, g.conv_dim, dtype=torch.bfloat16, device="cuda")
            ssm = torch.zeros(g.hv, 128, 128, dtype=torch.float32, device="cuda")
            st.gdn(i).store(conv, ssm)
            torch.cuda.synchronize()
            out["conv"][i] = conv.view(torch.int16).cpu().numpy().view(np.uint16)
            out["ssm"][i] = ssm.cpu().numpy()
    conv = torch.zeros(9, hc * H, dtype=torch.bfloat16, device="cuda")
    context = torch.zeros(2, dtype=torch.int32, device="cuda")
    st.ple().store(conv, context)
    torch.cuda.synchronize()
    out["ple"] = (conv.view(torch.int16).cpu().numpy().view(np.uint16), context.cpu().numpy())
    return out


@pytest.fixture(scope="module")
def serial(model):
    """The serial greedy sequence (prefill, then depth-0 rounds) and the state the prefill left."""
    import mtpx
    ctx, t, head, prompt, cfg = model
    s = mtpx.Session(ctx, t, head)
    print("case config5: prefill of", PROMPT, "tokens", flush=True)
    toks = [s.prefill(dev(prompt))]
    kinds = [t.layer_weights(i).kind for i in range(48)]
    state = _read_state(s.state(), kinds, cfg)
    assert s.offset() == PROMPT
    while len(toks) < GEN:
        toks += s.round(0)
    print("case config5: serial tokens", toks[:8], flush=True)
    s.close()
    return toks, state


@pytest.mark.timeout(900)
def test_serial_decode_matches_oracle_after_prompt(model, serial):
    """Two serial steps after the prompt through the oracle's 48-layer verify, from the prefill's state."""
    from oracle.target_ref import download_target, oracle_commit, oracle_verify
    ctx, t, head, prompt, cfg = model
    toks, state = serial
    ow = download_target(t, cfg, lazy=True)
    pos = PROMPT
    for step in range(2):
        print("case config5: oracle serial step", step, "pos", pos, flush=True)
        lg, _, _, win = oracle_verify(ow, cfg, state, np.array([toks[step]], np.int32), pos)
        assert int(O.argmax_rows(O.bf16_to_f32(lg))[0]) == toks[step + 1], step
        oracle_commit(ow, cfg, state, win, 1)
        pos += 1


@pytest.mark.timeout(600)
@pytest.mark.parametrize("k", [1, 2, 3, 4, 5])
def test_speculative_depths_emit_the_serial_sequence(model, serial, k):
    import mtpx
    ctx, t, head, prompt, cfg = model
    ref = serial[0]
    teacher = np.zeros(P, np.int32)
    teacher[:PROMPT] = prompt
    teacher[PROMPT:PROMPT + GEN] = ref
    # the forcing mask of every position, read back through the hook on a scratch token
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    mark = dev(np.full(P, -5, np.int32))
    mask = []
    for pos in range(PROMPT, PROMPT + GEN + 8):
        tok.fill_(0)
        ctx.force_draft(tok, mark, pos, RATE, FSEED)
        mask.append(int(tok.cpu()[0]) == -5)
    s = mtpx.Session(ctx, t, head)
    s.set_force(dev(teacher), RATE, FSEED)
    toks = [s.prefill(dev(prompt))]
    off, accepted = PROMPT, []
    while len(toks) < GEN:
        depth = min(k, GEN - len(toks) - 1)
        got = s.round(depth)
        n = len(got) - 1
        run = 0
        while run < depth and mask[off + 1 + run - PROMPT]:
            run += 1
        assert n == run, (off, n, run)
        accepted.append(n)
        toks += got
        off += n + 1
    print("case config5 depth", k, "rounds", len(accepted), "accepted", sum(accepted), flush=True)
    assert toks[:GEN] == ref
    assert s.offset() == PROMPT + len(toks) - 1
    assert sum(accepted) > 0
    s.close()

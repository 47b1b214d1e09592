"""GPU tests of the device-resident speculative round (mtpx_session_* / mtpx_round) through the
C ABI: the prefill's first token and the serial decode (k = 0) against the oracle's verify
forward; speculative decode at draft depths 1..4, with the forcing hook at rate 0.7 (drafts
replaced by the serial sequence's tokens) and without it, emits exactly the serial greedy
sequence (the accept/rollback invariant: speculative decode changes speed, never tokens);
the accepted counts follow the forcing mask; the drafter keeps every committed transition at
mixed depths; the sampled round (temperature > 0) against the oracle's speculative sampling;
refused calls."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

from gpu_util import dev, host, need_gpu  # noqa: E402

LAYER = dict(hidden=256, experts=16, top_k=4, expert_width=128, group_size=32, heads=4, kv_heads=2, head_dim=64,
             rot_dims=16, index_dim=32, rope_theta=1e7, eps=1e-6, max_positions=96)
TARGET = dict(key_heads=1, value_heads=2, conv_kernel=4, num_layers=5, full_attention_interval=4, hc=4, lowrank=64,
              vocab=1000)
PROMPT, GEN = 21, 40


@pytest.fixture(scope="module")
def model():
    need_gpu()
    import mtpx
    ctx = mtpx.Context(0)
    tc = mtpx.TargetConfig(mtpx.LayerConfig(**LAYER), *[TARGET[k] for k in (
        "key_heads", "value_heads", "conv_kernel", "num_layers", "full_attention_interval", "hc", "lowrank",
        "vocab")])
    tc.ple_layer = 1
    tc.ple = mtpx.PLEConfig(hidden=LAYER["hidden"], hc=TARGET["hc"], embed_dim=256, ngram_size=3, heads_per_ngram=2,
                            conv_kernel=4, group_size=LAYER["group_size"], row_group_size=32, eos=7, vocab_base=300,
                            token_vocab=TARGET["vocab"], eps=LAYER["eps"])
    t = mtpx.Target(ctx, tc, seed=31)
    head = mtpx.MTPHead(ctx, mtpx.HeadConfig(mtpx.LayerConfig(**LAYER), TARGET["hc"], TARGET["lowrank"],
                                             TARGET["vocab"], 500, 980), seed=32)
    prompt = np.random.default_rng(33).integers(0, TARGET["vocab"], PROMPT).astype(np.int32)
    yield ctx, t, head, prompt
    head.close()
    t.close()
    ctx.close()


def serial(model):
    import mtpx
    ctx, t, head, prompt = model
    s = mtpx.Session(ctx, t, head)
    toks = [s.prefill(dev(prompt))]
    while len(toks) < GEN:
        toks += s.round(0)
    assert s.offset() == PROMPT + GEN - 1
    s.close()
    return toks


def test_serial_decode_matches_oracle(model):
    from oracle.target_ref import download_target, oracle_commit, oracle_verify
    ctx, t, head, prompt = model
    toks = serial(model)
    cfg = dict(LAYER, **TARGET, ple_layer=1)
    ow = download_target(t, cfg)
    HK, D, P, hc, H = LAYER["kv_heads"], LAYER["head_dim"], LAYER["max_positions"], TARGET["hc"], LAYER["hidden"]
    st = dict(kc={}, vc={}, conv={}, ssm={}, ple=(np.zeros((9, hc * H), np.uint16), np.array([7, 7], np.int32)))
    for i, L in enumerate(ow["layers"]):
        if L["kind"] == 1:
            st["kc"][i], st["vc"][i] = np.zeros((HK, P, D), np.uint16), np.zeros((HK, P, D), np.uint16)
        else:
            g = L["gdn"]["geom"]
            st["conv"][i], st["ssm"][i] = np.zeros((g.kc - 1, g.conv_dim), np.uint16), np.zeros((g.hv, 128, 128),
                                                                                                 np.float32)
    pos = 0
    for off in range(0, PROMPT, 8):
        ids = prompt[off:off + 8]
        lg, _, _, win = oracle_verify(ow, cfg, st, ids, pos)
        oracle_commit(ow, cfg, st, win, len(ids))
        pos += len(ids)
    want = [int(np.argmax(O.bf16_to_f32(lg[-1])))]
    for step in range(5):
        print("case round serial oracle step", step, flush=True)
        lg, _, _, win = oracle_verify(ow, cfg, st, np.array([want[-1]], np.int32), pos)
        oracle_commit(ow, cfg, st, win, 1)
        pos += 1
        want.append(int(np.argmax(O.bf16_to_f32(lg[0]))))
    assert toks[:6] == want


@pytest.mark.parametrize("k", [1, 2, 3, 4])
@pytest.mark.parametrize("rate", [0.7, 0.0])
def test_speculative_equals_serial(model, k, rate):
    import mtpx
    ctx, t, head, prompt = model
    ref = serial(model)
    teacher = np.zeros(LAYER["max_positions"], np.int32)
    teacher[:PROMPT] = prompt
    teacher[PROMPT:PROMPT + GEN] = ref
    td = dev(teacher)
    s = mtpx.Session(ctx, t, head)
    s.set_force(td, rate, 0x5EED)
    toks = [s.prefill(dev(prompt))]
    accepted = []
    while len(toks) < GEN:
        depth = min(k, GEN - len(toks) - 1)
        got = s.round(depth)
        accepted.append(len(got) - 1)
        toks += got
    print("case round k", k, "rate", rate, "accepted", accepted, flush=True)
    assert toks[:GEN] == ref
    assert s.offset() == PROMPT + len(toks) - 1
    if rate > 0:
        assert sum(accepted) > 0
    s.close()


def test_mixed_depths_keep_every_transition(model):
    """Every committed position t > 0 gives the drafter one trusted transition (multi[t-1],
    token[t]), whatever depth produced it: after each round the drafter holds offset - 1 of them
    (in its head cache or its backlog).  A serial step right after a drafted round (no frontier)
    must first pair the carry's stream with the carry token; the sequence also checks that the
    tokens stay the serial ones."""
    import mtpx
    ctx, t, head, prompt = model
    ref = serial(model)
    teacher = np.zeros(LAYER["max_positions"], np.int32)
    teacher[:PROMPT] = prompt
    teacher[PROMPT:PROMPT + GEN] = ref
    s = mtpx.Session(ctx, t, head)
    s.set_force(dev(teacher), 0.7, 0x5EED)
    toks = [s.prefill(dev(prompt))]
    assert s.drafter_info()["committed_inputs"] == s.offset() - 1
    for k in [2, 0, 0, 3, 0, 1, 0, 2, 2, 0]:
        toks += s.round(k)
        info = s.drafter_info()
        print("case round mixed k", k, "offset", s.offset(), "committed", info["committed_inputs"], flush=True)
        assert info["round_in_flight"] == 0
        assert info["committed_inputs"] == s.offset() - 1, (k, info)
    n = len(toks)
    assert toks == ref[:n]
    s.close()


@pytest.mark.parametrize("k,T", [(0, 0.7), (2, 0.7), (3, 0.2), (2, 1e-4)])
def test_sampled_round_matches_oracle(model, k, T):
    """mtpx_round_sampled against its parts.  Forcing at rate 1 makes every draft the teacher's
    token, so each round's verify inputs are known: a second target state verifies the same tokens
    (bit-equal logits) and the oracle's speculative sampling with one-hot drafts (key = seed,
    counter offset = the committed position) decides n and the token; the round must emit exactly
    drafts[:n] + [token].  At a temperature near 0 every row whose maximum is unique gives its
    argmax, so the emitted tokens are the greedy ones there."""
    import mtpx
    ctx, t, head, prompt = model
    ref = serial(model)
    teacher = np.zeros(LAYER["max_positions"], np.int32)
    teacher[:PROMPT] = prompt
    teacher[PROMPT:PROMPT + GEN] = ref
    seed = 0x5A3
    s = mtpx.Session(ctx, t, head)
    s.set_force(dev(teacher), 1.0, 11)
    ts = mtpx.TargetState(ctx, t)
    carry = s.prefill(dev(prompt))
    t.prefill(ts, dev(prompt))
    off, emitted, accepted, unique_rows = PROMPT, 1, [], 0
    V = TARGET["vocab"]
    while emitted < GEN:
        depth = min(k, GEN - emitted - 1)
        got = s.round(depth, T, seed)
        drafts = teacher[off + 1:off + 1 + depth].copy()
        ids = np.array([carry] + list(drafts), np.int32)
        lg = torch.zeros(depth + 1, V, dtype=torch.bfloat16, device="cuda")
        t.verify(ts, dev(ids), logits=lg)
        lf = O.bf16_to_f32(host(lg))
        want = O.accept_sample(lf, None, drafts, T, seed, off, off)
        n = int(want[0])
        assert got == list(drafts[:n]) + [int(want[1])], (off, got, want)
        if T < 1e-3:
            for i, tok in enumerate(got):
                row = lf[i]
                if np.sum(row == row.max()) == 1:
                    unique_rows += 1
                    assert tok == int(np.argmax(row)), (off, i)
        ts.commit(n + 1)
        accepted.append(n)
        carry = got[-1]
        off += n + 1
        emitted += n + 1
    print("case sampled round k", k, "T", T, "accepted", accepted, flush=True)
    assert s.offset() == off
    if T < 1e-3:
        assert unique_rows >= GEN // 2
        assert sum(accepted) > 0
    s.close()
    ts.close()


def test_forcing_mask_decides_acceptance(model):
    """With the teacher equal to the serial sequence every forced draft is accepted: the accepted
    count of a round is the run of forced positions after the carry (capped at k)."""
    import mtpx
    ctx, t, head, prompt = model
    ref = serial(model)
    teacher = np.zeros(LAYER["max_positions"], np.int32)
    teacher[PROMPT:PROMPT + GEN] = ref
    seed, rate, k = 99, 0.7, 3
    # the mask of each position, read back through the hook on a scratch token
    mask = []
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    mark = dev(np.full(LAYER["max_positions"], -5, np.int32))
    for pos in range(LAYER["max_positions"]):
        tok.fill_(0)
        ctx.force_draft(tok, mark, pos, rate, seed)
        mask.append(int(tok.cpu()[0]) == -5)
    assert 0.4 < np.mean(mask) < 0.95
    s = mtpx.Session(ctx, t, head)
    s.set_force(dev(teacher), rate, seed)
    s.prefill(dev(prompt))
    off = PROMPT
    for _ in range(6):
        got = s.round(k)
        n = len(got) - 1
        run = 0
        while run < k and mask[off + 1 + run]:
            run += 1
        assert n == run, (off, n, run)
        off += n + 1
    s.close()


def test_round_refusals(model):
    import mtpx
    ctx, t, head, prompt = model
    s = mtpx.Session(ctx, t, head)
    with pytest.raises(mtpx.MtpxError):
        s.round(1)  # no prefill
    s.prefill(dev(prompt))
    with pytest.raises(mtpx.MtpxError):
        s.round(7)  # deeper than the drafter's maximum
    with pytest.raises(mtpx.MtpxError):
        s.prefill(dev(prompt))  # already holds a context
    s.reset()
    assert s.offset() == 0
    s.close()
    ns = mtpx.Session(ctx, t)  # serial only
    ns.prefill(dev(prompt))
    with pytest.raises(mtpx.MtpxError):
        ns.round(1)
    ns.round(0)
    ns.close()


def test_host_ids_refused_before_any_launch(model):
    """Token ids in plain host memory are refused by the session prefill, the target verify and the
    target prefill (a kernel reading them would fault the GPU).  Each call also carries an argument
    refused later but still before any launch (past the indexer budget of 2048 positions, wider than
    a verify window of 8, past the cache), so none of them launches whichever check refuses it; the
    message says which did.  The refusals change nothing: the session then prefills and decodes."""
    import mtpx
    ctx, t, head, prompt = model
    s = mtpx.Session(ctx, t, head)
    with pytest.raises(mtpx.MtpxError, match="ids are not memory the device can read"):
        s.prefill(torch.zeros(2048 + 1, dtype=torch.int32))
    st = mtpx.TargetState(ctx, t)
    with pytest.raises(mtpx.MtpxError, match="ids: not memory the device can read"):
        t.verify(st, torch.zeros(9, dtype=torch.int32))
    with pytest.raises(mtpx.MtpxError, match="ids: not memory the device can read"):
        t.prefill(st, torch.zeros(LAYER["max_positions"] + 1, dtype=torch.int32))
    st.close()
    first = s.prefill(dev(prompt))
    assert 0 <= first < TARGET["vocab"]
    assert len(s.round(1)) >= 1
    s.close()


def test_failed_prefill_breaks_the_session_until_reset(model):
    """A prompt longer than the caches fails in its last windows after earlier windows were
    committed: the session refuses further calls until reset, then works again."""
    import mtpx
    ctx, t, head, prompt = model
    P = LAYER["max_positions"]
    long_prompt = np.random.default_rng(34).integers(0, TARGET["vocab"], P + 4).astype(np.int32)
    s = mtpx.Session(ctx, t, head)
    with pytest.raises(mtpx.MtpxError):
        s.prefill(dev(long_prompt))
    with pytest.raises(mtpx.MtpxError, match="reset"):
        s.round(1)
    s.reset()
    first = s.prefill(dev(prompt))
    assert [first] + s.round(0) == serial(model)[:2]
    s.close()


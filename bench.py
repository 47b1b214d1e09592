"""Benchmark of single-stream MTP speculative decode on one MI355X.

Default workload: BASELINE config 5 -- the full-depth random-init 125B-A6B model (48 layers: 36
gated-deltanet + 12 attention, each with hyper-connection mixers and a 512-expert top-10 + shared
MoE; hidden 2560, vocab 248320, affine 4-bit gs64, all weights resident in HBM; layer 1 carries the
PLE n-gram block with its full 320,001,446-row table, 32 GB, --no-ple leaves it out) with the MTP
head.  A 1024-token random prompt goes through mtpx_session_prefill (the target prefill in batches of
512 positions, bit-equal to verifying and committing windows of 8; the drafter observes it), then
1024 tokens are generated greedily through mtpx_round (the device-resident round: k drafter
steps, a verify of the carry and the k drafts, the on-device greedy accept read back once, target
commit, drafter finalize).  First a serial greedy decode (k = 0) of the same 1024 tokens gives the
reference sequence; random-init drafts would never match the target, so acceptance is forced at
p = 0.7 by the drafter's forcing hook: each drafted position takes the reference sequence's token
with probability p (a seeded Philox draw per position).  The accept kernel's own count drives the
commit, and every depth must emit exactly the serial sequence.  Depths 1..5 are swept; value =
realized tokens/s of the best depth over all rounds of its 1024-token generation; the serial decode,
per-depth medians and accepted lengths, the draft step's time and a gs32 line (the checkpoint's
~113 GB format, at the best depth) are reported beside it.

Before the decode the same run measures BASELINE config 4 (a verify of 4 tokens after the prompt,
--steps timed steps; reported under "verify") and the per-kernel HIP event timings of that verify.
`roofline` is the routed-expert gate|up+SwiGLU kernel (the largest HBM stream of the step):
algorithmic bytes of its average launch (distinct experts of every layer read back from the
device) / its average duration from HIP events recorded on the launch stream.  `cpu_baseline`
times the CPU oracle on a bounded sample of the same round (1 thread and all host threads, the
oracle's exact arithmetic and MLX's CPU bf16-accumulating quantized matmul), scaled as its
`sample` field states.  `--no-e2e` reports the config-4 verify as the value; `--workload layer`
runs config 3 (one full-shape decoder layer, plain residuals, 4 tokens over 1024 cached
positions); `--workload prefill` times the prompt's prefill alone.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "mlxfast-qwen38-125b-a6b-engine_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "single-stream decode tok/s w/ MTP spec decode; MoE qGEMV HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0


def full_layer_cfg(gs: int, max_positions: int) -> dict:
    # dims: fixtures/qwen3_8_125b_a6b_config.json (text_config)
    return dict(hidden=2560, experts=512, top_k=10, expert_width=640, group_size=gs, heads=24, kv_heads=2,
                head_dim=256, rot_dims=64, index_dim=128, rope_theta=1e7, eps=1e-6, max_positions=max_positions)


def qbytes(N: int, K: int, gs: int) -> int:
    """Algorithmic bytes of one affine-4-bit matrix: nibbles + bf16 scale + bf16 bias."""
    return N * K // 2 + 4 * N * K // gs


def traffic_record(gs: int, M: int, T0: int, workload: str):
    """HBM bytes per launch of the gate|up kernel for this workload, as measured by the
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes summarised in profiles/ (None when absent)."""
    path = os.path.join(ROOT, "profiles", "moe_gate_up_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        rec = json.load(f)
    key = f"{workload}_gs{gs}_M{M}_T{T0}"
    return rec.get(key)


def cpu_baseline(layer, ctx, kv, cfg, M, seconds=15.0, max_steps=40):
    """Time the oracle's composition of the same layer step on the host (1 thread)."""
    import numpy as np

    from oracle import oracle as O
    from oracle.layer_ref import download, oracle_layer, read_device

    import torch

    torch.cuda.synchronize()
    w = download(layer.weights(), cfg)
    kp, vp, tmax = kv.buffers()
    HK, D = cfg["kv_heads"], cfg["head_dim"]
    kc = read_device(kp, HK * tmax * D * 2, np.uint16).reshape(HK, tmax, D)
    vc = read_device(vp, HK * tmax * D * 2, np.uint16).reshape(HK, tmax, D)
    r = np.random.default_rng(7)
    x = O.f32_to_bf16(r.standard_normal((M, cfg["hidden"])).astype(np.float32))
    pos0 = kv.offset
    n = 0
    t0 = time.perf_counter()
    while n < max_steps and (n == 0 or time.perf_counter() - t0 < seconds):
        oracle_layer(w, cfg, kc, vc, x, pos0)
        n += 1
    dt = time.perf_counter() - t0
    return dict(value=M * n / dt, unit="tok/s", cores=1, kind="port",
                sample=f"{n} verify steps (M={M}) of the same full-shape layer through the C oracle, "
                       f"single thread, {dt:.1f} s")


def target_cfgs(gs: int, max_positions: int, layers: int):
    lc = full_layer_cfg(gs, max_positions)
    # linear-attention dims, hyper-connections and vocabulary: fixtures/qwen3_8_125b_a6b_config.json
    tc = dict(key_heads=16, value_heads=48, conv_kernel=4, num_layers=layers, full_attention_interval=4, hc=4,
              lowrank=320, vocab=248320)
    # the PLE n-gram block on layer index 1 (ple_layer_ids [2] is 1-based): ngram_size 3, 8 heads per
    # n-gram, ple_embed_dim 2560, conv kernel 4, table rows 4-bit gs32, eos 248044, base 20,000,000
    tc["ple_layer"] = 1 if layers > 1 else -1
    tc["ple"] = dict(hidden=lc["hidden"], hc=4, embed_dim=2560, ngram_size=3, heads_per_ngram=8, conv_kernel=4,
                     group_size=gs, row_group_size=32, eos=248044, vocab_base=20_000_000, token_vocab=248320,
                     eps=lc["eps"])
    return lc, tc


def target_config(mtpx, lc, tc):
    cfg = mtpx.TargetConfig(mtpx.LayerConfig(**lc), *[tc[k] for k in (
        "key_heads", "value_heads", "conv_kernel", "num_layers", "full_attention_interval", "hc", "lowrank",
        "vocab")])
    cfg.ple_layer = tc["ple_layer"]
    cfg.ple = mtpx.PLEConfig(**tc["ple"])
    return cfg


def synthetic_prefix(mtpx, ctx, state, lc, tc, kinds, T0):
    """Random committed state in place of a prompt (--prefix synthetic, for counter runs that need
    the verify alone): attention K/V rows, GDN conv rows and recurrent states, the PLE block's
    conv rows and token context."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(0x5EED0005)
    for i, kind in enumerate(kinds):
        if kind == 1:
            kp, vp, tmax = state.kv(i).buffers()
            n_kv = lc["kv_heads"] * tmax * lc["head_dim"]
            for ptr, tensor in ((kp, 2 * i + 1), (vp, 2 * i + 2)):
                mtpx.check(ctx.lib.mtpx_randn_bf16(ctx.h, C.c_void_p(ptr), n_kv, 0x5EED0006, tensor, 1.0),
                           "randn kv")
        else:
            conv = torch.randn(tc["conv_kernel"] - 1, (2 * tc["key_heads"] + tc["value_heads"]) * 128,
                               device="cuda", generator=g).to(torch.bfloat16)
            ssm = torch.randn(tc["value_heads"], 128, 128, device="cuda", generator=g) * 0.05
            state.gdn(i).load(conv, ssm)
            torch.cuda.synchronize()
    if tc["ple_layer"] >= 0:
        pc = tc["ple"]
        conv = torch.randn((pc["conv_kernel"] - 1) * pc["ngram_size"], pc["hc"] * pc["hidden"], device="cuda",
                           generator=g).to(torch.bfloat16)
        context = torch.randint(0, tc["vocab"], (pc["ngram_size"] - 1,), device="cuda", generator=g,
                                dtype=torch.int32)
        state.ple().load(conv, context)
        torch.cuda.synchronize()
    state.set_offset(T0)


def _mlx_cpu_patch(O):
    """Swap the oracle's q4 GEMV and MoE block for MLX's CPU quantized matmul (_qmm_t with bf16
    accumulation, O.qmm_t_bf16) for the mlx_cpu timing mode; returns the undo function."""
    import numpy as np

    qmv0, moe0 = O.qmv, O.moe_block

    def qmv(wq, s_, b_, gs, x):
        return O.qmm_t_bf16(wq, s_, b_, gs, x), None

    def moe_block(w, x, H, E, K, F, gs):
        x = np.asarray(x, np.uint16).reshape(-1, H)
        idx, wk = O.topk_softmax(O.router_gemv(w["router"], O.bf16_to_f32(x)), K)
        ng, ngF = H // gs, F // gs
        y = np.zeros((x.shape[0], H), np.float32)
        for m in range(x.shape[0]):
            def ffn(gw, gsc, gb, uw, usc, ub, dw, dsc, db):
                g = O.bf16_to_f32(O.qmm_t_bf16(gw, gsc, gb, gs, x[m]))
                u = O.bf16_to_f32(O.qmm_t_bf16(uw, usc, ub, gs, x[m]))
                a = O.f32_to_bf16(g / (1 + np.exp(-g)) * u)
                return O.bf16_to_f32(O.qmm_t_bf16(dw, dsc, db, gs, a))[0]
            for k, e in enumerate(idx[m]):
                rows = slice(e * F, (e + 1) * F)
                hrows = slice(e * H, (e + 1) * H)
                y[m] += wk[m, k] * ffn(w["gate_w"][rows], w["gate_s"][rows], w["gate_b"][rows], w["up_w"][rows],
                                       w["up_s"][rows], w["up_b"][rows], w["down_w"][hrows], w["down_s"][hrows],
                                       w["down_b"][hrows])
            gl = float(O.router_gemv(w["shared_gate"], O.bf16_to_f32(x[m]))[0, 0])
            y[m] += ffn(w["sh_gate_w"], w["sh_gate_s"], w["sh_gate_b"], w["sh_up_w"], w["sh_up_s"], w["sh_up_b"],
                        w["sh_down_w"], w["sh_down_s"], w["sh_down_b"]) / (1 + np.exp(-gl))
        return dict(y=O.f32_to_bf16(y), idx=idx)

    O.qmv, O.moe_block = qmv, moe_block

    def undo():
        O.qmv, O.moe_block = qmv0, moe0
    return undo


def cpu_layer_times(target, lc, tc, widths, kinds, T0, runs=(("port", 1, 6.0),)):
    """The oracle on a bounded sample of the target step: per verify width M, the first GDN layer and
    the first attention layer (each with its mixers and MoE, attention over T0 random cached positions),
    16384 of the lm_head rows and the PLE block (the row gather from the first 65536 table rows, whose
    cost does not depend on the table's size).  runs: (mode, threads, seconds) -- mode "port": the
    oracle's exact int24 arithmetic; "mlx_cpu": its q4 GEMVs and MoE replaced by MLX's CPU _qmm_t (bf16
    accumulation); threads: OpenMP threads of the row-parallel loops; at least one iteration per width.
    -> ({(mode, threads): {M: (t_gdn, t_attn, t_head_rows, t_ple)}}, rows, {(mode, threads): iterations})."""
    import numpy as np

    from oracle import oracle as O
    from oracle.head_ref import _mix
    from oracle.layer_ref import download, download_moe, moe_y, oracle_attn, read_device
    from oracle.target_ref import _q, download_gdn, download_hc

    import torch

    torch.cuda.synchronize()
    cfg = dict(lc, **tc)
    H, gs, hc, LW, eps = lc["hidden"], lc["group_size"], tc["hc"], tc["lowrank"], lc["eps"]
    E, K, F = lc["experts"], lc["top_k"], lc["expert_width"]
    gi, ai = kinds.index(0), kinds.index(1)
    lw_g, lw_a = target.layer_weights(gi), target.layer_weights(ai)
    Lg = dict(hc=download_hc(lw_g.attn_hc, H, hc, LW, gs), mhc=download_hc(lw_g.mlp_hc, H, hc, LW, gs),
              gdn=download_gdn(lw_g.gdn, H, tc["key_heads"], tc["value_heads"], tc["conv_kernel"], gs),
              moe=download_moe(lw_g.attn.moe, cfg, lazy=True))
    La = dict(hc=download_hc(lw_a.attn_hc, H, hc, LW, gs), mhc=download_hc(lw_a.mlp_hc, H, hc, LW, gs),
              attn=download(lw_a.attn, cfg, lazy=True))
    La["moe"] = La["attn"]["moe"]
    HK, D, P = lc["kv_heads"], lc["head_dim"], lc["max_positions"]
    r = np.random.default_rng(9)
    kc = np.zeros((HK, P, D), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :T0] = O.f32_to_bf16(r.standard_normal((HK, T0, D)).astype(np.float32))
    vc[:, :T0] = O.f32_to_bf16(r.standard_normal((HK, T0, D)).astype(np.float32))
    g = Lg["gdn"]["geom"]
    conv = O.f32_to_bf16(r.standard_normal((g.kc - 1, g.conv_dim)).astype(np.float32))
    ssm = (r.standard_normal((g.hv, 128, 128)) * 0.05).astype(np.float32)
    rows = 16384
    head = _q(target.weights().lm_head, rows, H, gs)  # the first `rows` rows of lm_head
    ple = None
    if tc["ple_layer"] >= 0:
        pc, pw = tc["ple"], target.layer_weights(tc["ple_layer"]).ple
        W, Ed, nh = hc * H, pc["embed_dim"], 2 * pc["heads_per_ngram"]
        rd, nt = Ed // nh, 65536
        table = (read_device(pw.table.w, nt * rd // 2, np.uint32).reshape(nt, rd // 8),
                 read_device(pw.table.s, nt * rd // 16, np.uint16).reshape(nt, rd // 32),
                 read_device(pw.table.b, nt * rd // 16, np.uint16).reshape(nt, rd // 32))
        vocab = np.array(O.primes_above(nt // nh - 300, nh), np.int64)
        ple = dict(key_proj=_q(pw.key_proj, W, Ed, gs), value_proj=_q(pw.value_proj, H, Ed, gs),
                   norm_key=read_device(pw.norm_key, 2 * W, np.uint16),
                   norm_query=read_device(pw.norm_query, 2 * W, np.uint16),
                   norm_conv=read_device(pw.norm_conv, 2 * W, np.uint16),
                   conv_w=read_device(pw.conv_w, 2 * W * pc["conv_kernel"], np.uint16).reshape(W, -1), table=table,
                   mult=np.array(list(pw.table.multiplier)[:3], np.int64), vocab=vocab,
                   offs=np.concatenate([[0], np.cumsum(vocab)[:-1]]).astype(np.int64))
        ple_conv = O.f32_to_bf16(r.standard_normal(((pc["conv_kernel"] - 1) * pc["ngram_size"], W)).astype(np.float32))

    def layer_step(L, gdn, sW):
        s_, n = O.hc_norm(sW, None, None, L["hc"]["scale"], hc, eps)
        x, j = _mix(L["hc"], n, hc, gs)
        if gdn:
            d = L["gdn"]
            proj, _ = O.qmv(*d["in_proj"], gs, x)
            o = O.gdn_core(d["geom"], proj, conv, ssm, d["conv_w"], d["nea"], d["dtb"], d["nw"], eps)
            ao, _ = O.qmv(*d["out_proj"], gs, o["gated"])
        else:
            ao = oracle_attn(L["attn"], cfg, kc, vc, x, T0)
        s2, n = O.hc_norm(s_, ao, j, L["mhc"]["scale"], hc, eps)
        x, j = _mix(L["mhc"], n, hc, gs)
        moe_y(L["moe"], x, H, E, K, F, gs)

    inputs = {}
    for M in widths:
        sW = O.f32_to_bf16(r.standard_normal((M, hc * H)).astype(np.float32))
        xh = O.f32_to_bf16(r.standard_normal((M, H)).astype(np.float32))
        ids = r.integers(0, tc["vocab"], M).astype(np.int32)
        O.set_threads(cpu_threads_all())
        layer_step(Lg, True, sW)  # fetches the routed experts of these inputs (not timed)
        layer_step(La, False, sW)
        inputs[M] = (sW, xh, ids)
    all_times, all_iters = {}, {}
    for mode, threads, seconds in runs:
        O.set_threads(threads)
        undo = _mlx_cpu_patch(O) if mode == "mlx_cpu" else (lambda: None)
        times, iters = {}, {}
        try:
            for M in widths:
                sW, xh, ids = inputs[M]
                samples = []
                t0 = time.perf_counter()
                while not samples or time.perf_counter() - t0 < seconds / len(widths):
                    a = time.perf_counter()
                    layer_step(Lg, True, sW)
                    b = time.perf_counter()
                    layer_step(La, False, sW)
                    c = time.perf_counter()
                    O.qmv(*head, gs, xh)
                    d = time.perf_counter()
                    if ple is not None:
                        O.ple_forward(ple, dict(tc["ple"]), sW, ids, ple_conv,
                                      ids[:2] if M >= 2 else np.r_[ids, ids])
                    e = time.perf_counter()
                    samples.append((b - a, c - b, d - c, e - d))
                # median of each part over the iterations that fit the bound (at least one)
                times[M], iters[M] = tuple(float(v) for v in np.median(np.array(samples), axis=0)), len(samples)
        finally:
            undo()
        all_times[(mode, threads)], all_iters[(mode, threads)] = times, iters
        log(f"cpu sample {mode} x{threads}: {times}")
    O.set_threads(cpu_threads_all())
    return all_times, rows, all_iters


def _cpu_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return os.cpu_count(), len(os.sched_getaffinity(0)), model


def cpu_threads_all():
    return int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))


def cpu_baseline_full(target, lc, tc, M, kinds, T0):
    """CPU baseline of the verify step (config 4): the sampled oracle layers scaled to the stack, on all
    host threads (port mode)."""
    th = cpu_threads_all()
    all_times, rows, all_iters = cpu_layer_times(target, lc, tc, [M], kinds, T0, runs=(("port", th, 6.0),))
    tg, ta, thr, tp = all_times[("port", th)][M]
    n_gdn, n_attn = kinds.count(0), kinds.count(1)
    step_s = n_gdn * tg + n_attn * ta + thr * tc["vocab"] / rows + tp
    return dict(value=M / step_s, unit="tok/s", cores=th, kind="port",
                sample=f"{all_iters[('port', th)][M]} x (one GDN layer {tg:.3f} s, one attention layer {ta:.3f} s, "
                       f"{rows} of {tc['vocab']} lm_head rows {thr:.3f} s, the PLE block {tp:.3f} s) of the verify "
                       f"step (M={M}) through the C oracle on {th} threads, scaled to {n_gdn} GDN + {n_attn} "
                       f"attention layers and the whole lm_head: {step_s:.2f} s per step")


def cpu_baseline_e2e(target, lc, tc, kinds, k, tokens_per_round, shortlist_rows, T0):
    """CPU baseline of MTP speculative decode at draft depth k, one round = k draft steps + a verify of
    k+1 tokens; a draft step = one attention layer with its mixers and MoE at one token + the shortlist
    GEMV (lm_head rows scaled); the verify = the sampled GDN and attention layers scaled to the stack +
    lm_head + PLE.  Timed in the oracle's int24 arithmetic (port) and with MLX's CPU _qmm_t (bf16
    accumulation, mlx_cpu), each on 1 thread (MLX runs one op at a time on its stream worker) and on all
    host threads; the headline entry is the fastest.  Time-bounded: about 4 s per (mode, threads), split
    over the two widths, each part the median of the iterations that fit (at least one, after one
    untimed call that fetches the routed experts); the iteration counts are reported."""
    n_gdn, n_attn = kinds.count(0), kinds.count(1)
    ncpu, nav, model = _cpu_info()
    th = cpu_threads_all()
    runs = (("port", 1, 4.0), ("port", th, 4.0), ("mlx_cpu", 1, 4.0), ("mlx_cpu", th, 4.0))
    t0 = time.perf_counter()
    all_times, rows, all_iters = cpu_layer_times(target, lc, tc, sorted({1, k + 1}), kinds, T0, runs=runs)
    entries = []
    for mode, threads, _ in runs:
        times = all_times[(mode, threads)]
        tg, ta, thr, tp = times[k + 1]
        verify_s = n_gdn * tg + n_attn * ta + thr * tc["vocab"] / rows + tp
        _, ta1, th1, _ = times[1]
        draft_s = ta1 + th1 * shortlist_rows / rows
        round_s = k * draft_s + verify_s
        entries.append(dict(mode=mode, threads=threads, tok_s=round(tokens_per_round / round_s, 4),
                            round_s=round(round_s, 3), verify_s=round(verify_s, 3), draft_s=round(draft_s, 4),
                            iterations={str(m): v for m, v in all_iters[(mode, threads)].items()}))
    best = max(entries, key=lambda e: e["tok_s"])
    return dict(value=best["tok_s"], unit="tok/s", cores=best["threads"], kind="port",
                sample=f"draft depth {k}, {tokens_per_round:.3f} tokens per round (the GPU run's realized rate): "
                       f"one round = {k} draft steps (an attention layer with mixers and MoE at one token + "
                       f"{shortlist_rows} shortlist rows) + a verify of {k + 1} tokens ({n_gdn} GDN + {n_attn} "
                       f"attention layers scaled from one of each, lm_head from 16384 rows, PLE); mode "
                       f"{best['mode']} on {best['threads']} threads; host: {model}, {ncpu} CPUs "
                       f"({nav} available to this process); {time.perf_counter() - t0:.0f} s of sampling, "
                       f"time-bounded (about 4 s per mode), each part the median of the iterations that fit",
                modes=entries, cpu_model=model, nproc=ncpu)


MAXPOS = 2048 + 16  # the indexer budget (2048 positions) plus one verify window


def build_model(mtpx, ctx, args, gs, with_head=True):
    """The random-init target (and MTP head) at group size gs, weights generated on the device."""
    lc, tc = target_cfgs(gs, MAXPOS, args.layers)
    if args.no_ple:
        tc["ple_layer"] = -1
    t0 = time.perf_counter()
    target = mtpx.Target(ctx, target_config(mtpx, lc, tc), seed=0x5EED0004)
    head = mtpx.MTPHead(ctx, mtpx.HeadConfig(mtpx.LayerConfig(**lc), tc["hc"], tc["lowrank"], tc["vocab"], 98304,
                                             248044), seed=0x5EED0007) if with_head else None
    import torch
    torch.cuda.synchronize()
    log(f"gs{gs} model ({args.layers} layers, PLE layer {tc['ple_layer']}) initialised in "
        f"{time.perf_counter() - t0:.1f} s")
    return target, head, lc, tc


def log(msg):
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def prompt_ids(args, vocab):
    import torch
    g = torch.Generator().manual_seed(0x5EED0005)
    return torch.randint(0, vocab, (args.prompt,), generator=g, dtype=torch.int32).cuda()


def generate(session, first, k, gen):
    """Rounds of depth k (the depth shrinks at the end so exactly `gen` tokens are emitted,
    counting the prefill's first token).  -> (tokens, per-round seconds, accepted per round)."""
    toks, times, acc = [first], [], []
    while len(toks) < gen:
        d = min(k, gen - len(toks) - 1)
        t0 = time.perf_counter()
        got = session.round(d)
        times.append(time.perf_counter() - t0)
        acc.append(len(got) - 1)
        toks += got
    return toks[:gen], times, acc


def verify_measure(args, ctx, target, state, lc, tc, kinds, first, M, steps, warmup, profile):
    """Config 4: a verify of M tokens (the carry + M-1 ids) over the committed prompt; the window
    is left open and discarded by the next verify."""
    import torch
    V, W = tc["vocab"], tc["hc"] * lc["hidden"]
    g = torch.Generator().manual_seed(0x5EED0006 + M)
    ids = torch.randint(0, V, (M,), generator=g, dtype=torch.int32)
    ids[0] = first
    ids = ids.cuda()
    logits = torch.empty(M, V, dtype=torch.bfloat16, device="cuda")
    multi = torch.empty(M, W, dtype=torch.bfloat16, device="cuda")
    for _ in range(warmup):
        target.verify(state, ids, logits, multi)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        target.verify(state, ids, logits, multi)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    stats = None
    if profile:
        ctx.profile(True)
        ctx.profile_reset()
        for _ in range(steps):
            target.verify(state, ids, logits, multi)
        stats = ctx.profile_stats()
        ctx.profile(False)
    return ms, stats


def step_bytes_of(lc, tc, kinds, uniq, M, T0, gs):
    """Algorithmic HBM bytes of one verify of M tokens after T0 positions."""
    H, V, hc = lc["hidden"], tc["vocab"], tc["hc"]
    F, E = lc["expert_width"], lc["experts"]
    moe_bytes = sum((u + 1) * (2 * qbytes(F, H, gs) + qbytes(H, F, gs)) + 2 * E * H + 2 * H for u in uniq)
    hd = lc["heads"] * lc["head_dim"]
    qkv_rows = 2 * hd + 2 * lc["kv_heads"] * lc["head_dim"] + lc["index_dim"]
    cd = (2 * tc["key_heads"] + tc["value_heads"]) * 128
    pw = cd + tc["value_heads"] * 128 + 2 * tc["value_heads"]
    W, LW = hc * H, tc["lowrank"]
    mixer = qbytes(LW, W, gs) + qbytes(W, LW, gs)
    n_attn, n_gdn = kinds.count(1), kinds.count(0)
    attn_bytes = n_attn * (qbytes(qkv_rows, H, gs) + qbytes(H, hd, gs) + 2 * 2 * lc["kv_heads"] * (T0 + M) *
                           lc["head_dim"])
    gdn_bytes = n_gdn * (qbytes(pw, H, gs) + qbytes(H, tc["value_heads"] * 128, gs) +
                         2 * 4 * tc["value_heads"] * 128 * 128)
    hc_bytes = len(kinds) * 2 * (mixer + qbytes(hc, W, gs)) + mixer
    ple_bytes = 0
    if tc["ple_layer"] >= 0:  # key and value projections + 16 table rows of 100 bytes per token
        pc = tc["ple"]
        ple_bytes = qbytes(W, pc["embed_dim"], gs) + qbytes(H, pc["embed_dim"], gs) + M * 16 * 100
    total = moe_bytes + attn_bytes + gdn_bytes + hc_bytes + ple_bytes + qbytes(V, H, gs) + M * qbytes(1, H, gs)
    return total, moe_bytes


def serial_token_bytes(lc, tc, gs):
    """Active weight bytes of one serial decode token (3.823 GB at gs64): every dense matrix, the
    router, top-k + shared experts, the PLE projections, lm_head; caches excluded."""
    H, hc, W, LW = lc["hidden"], tc["hc"], tc["hc"] * lc["hidden"], tc["lowrank"]
    F, E, K = lc["expert_width"], lc["experts"], lc["top_k"]
    n = tc["num_layers"]
    n_attn = n // tc["full_attention_interval"]
    hd = lc["heads"] * lc["head_dim"]
    qkv_rows = 2 * hd + 2 * lc["kv_heads"] * lc["head_dim"] + lc["index_dim"]
    cd = (2 * tc["key_heads"] + tc["value_heads"]) * 128
    pw = cd + tc["value_heads"] * 128 + 2 * tc["value_heads"]
    mixer = qbytes(LW, W, gs) + qbytes(W, LW, gs)
    b = n * ((K + 1) * (2 * qbytes(F, H, gs) + qbytes(H, F, gs)) + 2 * E * H + 2 * H)
    b += n_attn * (qbytes(qkv_rows, H, gs) + qbytes(H, hd, gs))
    b += (n - n_attn) * (qbytes(pw, H, gs) + qbytes(H, tc["value_heads"] * 128, gs))
    b += n * 2 * (mixer + qbytes(hc, W, gs)) + mixer + qbytes(tc["vocab"], H, gs)
    if tc["ple_layer"] >= 0:
        b += qbytes(W, tc["ple"]["embed_dim"], gs) + qbytes(H, tc["ple"]["embed_dim"], gs)
    return b


FORCE_SEED = 0x5EED0009


def forcing_mask(ctx, prompt, gen, p, seed):
    """The forcing hook's decision at every position up to prompt + gen + 8, read back through the hook
    itself (a scratch token per position, one readback): True where the draft takes the teacher's token."""
    import numpy as np
    import torch
    n = prompt + gen + 8
    mark = torch.full((n,), -5, dtype=torch.int32, device="cuda")
    tok = torch.zeros(n, dtype=torch.int32, device="cuda")
    for pos in range(prompt, n):
        ctx.force_draft(tok[pos:pos + 1], mark, pos, p, seed)
    return tok.cpu().numpy() == -5


def rounds_from_mask(mask, prompt, gen, k):
    """Rounds of depth k that emit gen tokens (the prefill's first one included) when exactly the
    forced drafts are accepted: each round accepts the run of forced positions after its carry."""
    off, emitted, rounds = prompt, 1, 0
    while emitted < gen:
        d = min(k, gen - emitted - 1)
        n = 0
        while n < d and mask[off + 1 + n]:
            n += 1
        emitted, off, rounds = emitted + n + 1, off + n + 1, rounds + 1
    return rounds


def headline_runs(args, mtpx, ctx, target, head, prompt, teacher, ref, k):
    """The headline: W warmup and then exactly K timed config-5 decodes at depth k (a step = one decode of
    gen - 1 tokens after the prompt), each in its own session prefilled beforehand (untimed), the K
    timed decodes back to back between two device synchronisations; every decode must emit the serial
    sequence.  -> (seconds of the K decodes, per-decode seconds, rounds per decode)."""
    import numpy as np
    import torch
    W, K = args.warmup, args.steps
    sessions = []
    for _ in range(W + K):
        s = mtpx.Session(ctx, target, head)
        first = s.prefill(prompt)
        s.set_force(teacher, args.accept_rate, FORCE_SEED)
        sessions.append((s, first))
    for s, first in sessions[:W]:
        toks, _, _ = generate(s, first, k, args.gen)
        assert toks == ref, "warmup decode emitted another sequence than the serial decode"
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    per, rounds, outs = [], [], []
    for s, first in sessions[W:]:
        a = time.perf_counter()
        toks, times, _ = generate(s, first, k, args.gen)
        per.append(time.perf_counter() - a)
        rounds.append(len(times))
        outs.append(toks)
    torch.cuda.synchronize()
    total = time.perf_counter() - t0
    for s, _ in sessions:
        s.close()
    if any(o != ref for o in outs):
        raise SystemExit("a timed decode emitted another sequence than the serial decode")
    return total, per, rounds


def decode_sweep(args, mtpx, ctx, target, head, lc, tc, depths, gs):
    """Config 5 at group size gs: the prompt, a serial greedy decode of --gen tokens (the teacher of the
    forcing hook and the reference sequence), then speculative decode at each depth with forced acceptance
    at rate p; every depth must emit the serial sequence exactly."""
    import numpy as np
    import torch

    V = tc["vocab"]
    prompt = prompt_ids(args, V)
    sess = mtpx.Session(ctx, target, head)
    t0 = time.perf_counter()
    first = sess.prefill(prompt)
    prefill_s = time.perf_counter() - t0
    log(f"gs{gs} prefill of {args.prompt} tokens: {prefill_s * 1e3:.1f} ms")
    ref, st, _ = generate(sess, first, 0, args.gen)
    serial = dict(tok_s=round((args.gen - 1) / sum(st), 2), ms_per_token_median=round(1e3 * float(np.median(st)), 3),
                  tokens=args.gen - 1)
    log(f"gs{gs} serial decode: {serial}")
    teacher = torch.zeros(MAXPOS, dtype=torch.int32)
    teacher[:args.prompt] = prompt.cpu()
    teacher[args.prompt:args.prompt + args.gen] = torch.tensor(ref, dtype=torch.int32)
    teacher = teacher.cuda()
    p = args.accept_rate
    mask = forcing_mask(ctx, args.prompt, args.gen, p, FORCE_SEED)
    drafted = mask[args.prompt + 1:args.prompt + args.gen]
    forcing = dict(rate=p, realized_rate=round(float(np.mean(drafted)), 4), positions=int(drafted.size),
                   note="share of the generated positions whose draft the seeded mask forces to the serial token")
    log(f"gs{gs} forcing mask: {forcing}")
    res = {}
    warm = []  # the prompt again for every depth: prefill times after the first (warm workspace)
    for k in depths:
        sess.reset()
        t1 = time.perf_counter()
        f2 = sess.prefill(prompt)
        warm.append(time.perf_counter() - t1)
        sess.set_force(teacher, p, FORCE_SEED)
        toks, times, acc = generate(sess, f2, k, args.gen)
        same = toks == ref
        full = [t for t, a in zip(times, acc)]
        r = dict(tok_s=round((args.gen - 1) / sum(times), 2), rounds=len(times),
                 ms_per_round_median=round(1e3 * float(np.median(full)), 3),
                 ms_per_round_mean=round(1e3 * sum(times) / len(times), 3),
                 mean_accepted=round(float(np.mean(acc)), 3),
                 tokens_per_round=round((args.gen - 1) / len(times), 3),
                 expected_tokens_per_round=round(sum(p ** i for i in range(k + 1)), 4),
                 tokens_per_round_from_mask=round((args.gen - 1) / rounds_from_mask(mask, args.prompt, args.gen, k), 3),
                 greedy_identical_to_serial=bool(same))
        log(f"gs{gs} depth {k}: {r}")
        if not same:
            raise SystemExit(f"speculative decode at depth {k} emitted another sequence than the serial decode")
        res[k] = r
    sess.set_force(None, 0.0, 0)
    prefill = dict(first_ms=round(prefill_s * 1e3, 1), warm_ms_median=round(1e3 * float(np.median(warm)), 1))
    prefill["tok_s"] = round(args.prompt / (prefill["warm_ms_median"] / 1e3), 1)
    log(f"gs{gs} prefill: {prefill}")
    return sess, first, prompt, serial, res, prefill, dict(teacher=teacher, ref=ref, forcing=forcing)


def run_full(args, out):
    import numpy as np
    import torch

    import mtpx

    gs = args.group_size
    ctx = mtpx.Context(0)
    target, head, lc, tc = build_model(mtpx, ctx, args, gs, with_head=args.prefix == "prompt")
    kinds = [target.layer_weights(i).kind for i in range(args.layers)]
    n_attn, n_gdn = kinds.count(1), kinds.count(0)

    # ---- config 4: verify of M tokens after the real 1024-token prompt
    prompt = prompt_ids(args, tc["vocab"])
    if args.prefix == "synthetic":  # the target state alone (no head, no session)
        sess = st = mtpx.TargetState(ctx, target)
        synthetic_prefix(mtpx, ctx, st, lc, tc, kinds, args.prompt)
        first, T0 = int(prompt[-1]), args.prompt
    else:
        sess = mtpx.Session(ctx, target, head)
        first = sess.prefill(prompt)
        T0 = sess.offset()
        st = sess.state()
    M = args.verify_width
    ms_per_step, stats = verify_measure(args, ctx, target, st, lc, tc, kinds, first, M, args.steps, args.warmup, True)
    uniq = st.moe_unique(args.layers)
    widths = {}
    for w in range(1, 7):
        widths[w] = round(verify_measure(args, ctx, target, st, lc, tc, kinds, first, w, 10, 2, False)[0], 4)
    log(f"verify of {M} tokens: {ms_per_step:.3f} ms; by width {widths}")
    sess.close()
    H, F = lc["hidden"], lc["expert_width"]
    gu_bytes = [(u + 1) * 2 * qbytes(F, H, gs) for u in uniq]
    step_bytes, moe_bytes = step_bytes_of(lc, tc, kinds, uniq, M, T0, gs)
    kernels = {k: dict(launches=n, avg_us=round(1e3 * ms / n, 3)) for k, (n, ms) in stats.items()}
    gu_s = stats["moe_gate_up"][1] / stats["moe_gate_up"][0] / 1e3
    gu_avg = sum(gu_bytes) / len(gu_bytes)
    achieved = gu_avg / gu_s / 1e9
    verify = {
        "what": f"BASELINE config 4: full-depth verify forward ({args.layers} layers: {n_gdn} GDN + {n_attn} "
                f"attention) of {M} tokens after the {T0}-token random prompt (processed by the target "
                f"prefill); value = verified positions/s; {args.steps} timed steps after "
                f"{args.warmup} warmup",
        "value": round(M / (ms_per_step / 1e3), 2), "unit": "positions/s", "ms_per_step": round(ms_per_step, 4),
        "ms_by_width": widths,
        "step_bytes": step_bytes, "step_GBps": round(step_bytes / (ms_per_step / 1e3) / 1e9, 1),
        "decode_roofline_frac": round(step_bytes / (ms_per_step / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        "moe": {"distinct_experts_per_layer": uniq, "bytes_per_step": moe_bytes},
        "kernels": kernels,
    }
    out["roofline"] = {
        "bound": "hbm",
        "kernel": f"moe_gate_up (routed + shared gate|up GEMV + SwiGLU) in the config-4 verify (M={M}), "
                  f"average launch over all layers",
        "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
        "algorithmic_bytes": round(gu_avg), "avg_us": round(gu_s * 1e6, 3),
    }
    tr = traffic_record(gs, M, 1024, "full")
    if tr is not None:
        out["roofline"]["traffic"] = tr["gate_up_bytes_per_launch"]
        out["roofline"]["traffic_source"] = tr["source"]
    if args.copy_calibration:
        copy_calibration()
    base_cfg = {"prompt_tokens": args.prompt, "layers": args.layers, "group_size": gs, "parallelism": "none (1 GPU)",
                "ple_layer": tc["ple_layer"]}
    ple_note = ("the PLE n-gram block on layer 1 with the full 320,001,446-row table resident"
                if tc["ple_layer"] >= 0 else "the PLE block of layer 1 left out (--no-ple)")
    if args.no_e2e:
        out.update({
            "value": verify["value"], "unit": "tok/s", "ms_per_step": verify["ms_per_step"],
            "config": dict(base_cfg, workload=verify["what"] + " (" + ple_note + ")", verify_width=M),
            "verify": verify,
        })
        if not args.no_cpu_baseline:
            out["cpu_baseline"] = cpu_baseline_full(target, lc, tc, M, kinds, T0)
        return out

    # ---- config 5: 1024-token prompt + 1024 generated tokens, depths swept, forced acceptance at p
    sess, first, prompt, serial, sweep, prefill, dd = decode_sweep(args, mtpx, ctx, target, head, lc, tc, args.depths,
                                                                   gs)
    best = max(sweep, key=lambda d: sweep[d]["tok_s"])
    fin = sweep[best]
    sess.close()
    hl_s, hl_per, hl_rounds = headline_runs(args, mtpx, ctx, target, head, prompt, dd["teacher"], dd["ref"], best)
    hl = dict(tok_s=round(args.steps * (args.gen - 1) / hl_s, 2), steps=args.steps, warmup=args.warmup,
              seconds=round(hl_s, 3), ms_per_decode_mean=round(1e3 * hl_s / args.steps, 2),
              tok_s_per_decode_min=round((args.gen - 1) / max(hl_per), 2),
              tok_s_per_decode_max=round((args.gen - 1) / min(hl_per), 2), rounds_per_decode=sorted(set(hl_rounds)))
    log(f"gs{gs} headline at depth {best}: {hl}")
    tok_bytes = serial_token_bytes(lc, tc, gs)
    draft_ms = {k: round((r["ms_per_round_median"] - widths[k + 1]) / k, 4) for k, r in sweep.items() if k + 1 in widths}
    gs32 = None
    if args.gs32_line and gs != 32:
        target.close()
        head.close()
        torch.cuda.synchronize()
        t32, h32, lc32, tc32 = build_model(mtpx, ctx, args, 32)
        s32, _, _, serial32, sw32, pf32, _ = decode_sweep(args, mtpx, ctx, t32, h32, lc32, tc32, [best], 32)
        r32 = sw32[best]
        b32 = serial_token_bytes(lc32, tc32, 32)
        gs32 = dict(r32, draft_depth=best, serial_tok_s=serial32["tok_s"], prefill=pf32,
                    bytes_per_serial_token=b32,
                    roofline_frac=round(r32["tok_s"] * b32 / 1e9 / HBM_PEAK_GBS, 4))
        s32.close()
        t32.close()
        h32.close()
        target = None
    out.update({
        "value": hl["tok_s"],
        "ms_per_step": hl["ms_per_decode_mean"],
        "steps": args.steps,
        "warmup": args.warmup,
        "config": dict(base_cfg, workload=(
            f"BASELINE config 5: single-stream MTP speculative decode on the full-depth random-init 125B-A6B "
            f"target ({args.layers} layers: {n_gdn} GDN + {n_attn} attention, hyper-connection mixers, 512-expert "
            f"top-10 + shared MoE, hidden 2560, vocab 248320, gs{gs}, weights resident in HBM) with the MTP head "
            f"(attention + MoE, 98584-row shortlist; {ple_note}). A {args.prompt}-token random prompt is processed "
            f"(the target prefill, observed by the drafter), then {args.gen} tokens are generated greedily in rounds (k "
            f"drafter steps, a verify of k+1 tokens, the on-device greedy accept read back once, target commit, "
            f"drafter finalize). Acceptance is forced at p={args.accept_rate}: each drafted position takes the "
            f"serial greedy sequence's token with probability p (seeded per position); every depth emits "
            f"exactly the serial sequence. Draft depth {best} = the best of {list(args.depths)} in a sweep of "
            f"one decode per depth. A step = one decode of the {args.gen - 1} round-generated tokens at that "
            f"depth ({fin['rounds']} rounds) in a session whose prompt was prefilled beforehand (untimed); "
            f"{args.warmup} warmup decodes, then {args.steps} timed decodes back to back between two device "
            f"synchronisations; value = {args.steps} x {args.gen - 1} tokens / their seconds; ms_per_step = "
            f"mean decode"),
            draft_depth=best, accept_rate=args.accept_rate, generated_tokens=args.gen,
            mean_accepted=fin["mean_accepted"], tokens_per_round=fin["tokens_per_round"],
            expected_tokens_per_round=fin["expected_tokens_per_round"],
            ms_per_round_median=fin["ms_per_round_median"], rounds_per_decode=fin["rounds"]),
        "decode": {
            "headline": hl,
            "forcing": dd["forcing"],
            "depth_sweep": {str(d): r for d, r in sweep.items()},
            "serial_decode": serial,
            "prefill": prefill,
            "draft_step_ms_by_depth": draft_ms,
            "bytes_per_serial_token": tok_bytes,
            "roofline_frac": round(hl["tok_s"] * tok_bytes / 1e9 / HBM_PEAK_GBS, 4),
            "gs32": gs32,
        },
        "verify": verify,
    })
    if not args.no_cpu_baseline and target is not None:
        out["cpu_baseline"] = cpu_baseline_e2e(target, lc, tc, kinds, best, fin["tokens_per_round"], 98304 + 276,
                                               T0)
    elif not args.no_cpu_baseline:
        t2, h2, lc2, tc2 = build_model(mtpx, ctx, args, gs)
        out["cpu_baseline"] = cpu_baseline_e2e(t2, lc2, tc2, kinds, best, fin["tokens_per_round"], 98304 + 276, T0)
        t2.close()
        h2.close()
    return out


def copy_calibration():
    import torch
    a = torch.empty(128 << 20, dtype=torch.int16, device="cuda").fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()


def run_layer(args, out):
    import torch

    import mtpx

    M, T0, gs = args.verify_width, args.cached, args.group_size
    cfg = full_layer_cfg(gs, T0 + 64)
    ctx = mtpx.Context(0)
    layer = mtpx.DecoderLayer(ctx, mtpx.LayerConfig(**cfg), seed=0x5EED0003)
    kv = mtpx.KVCache(ctx, cfg["kv_heads"], cfg["head_dim"], cfg["max_positions"])
    kp, vp, tmax = kv.buffers()
    n_kv = cfg["kv_heads"] * tmax * cfg["head_dim"]
    for ptr, tensor in ((kp, 1), (vp, 2)):
        mtpx.check(ctx.lib.mtpx_randn_bf16(ctx.h, C.c_void_p(ptr), n_kv, 0x5EED0004, tensor, 1.0), "randn kv")
    kv.offset = T0
    g = torch.Generator(device="cuda").manual_seed(0x5EED0005)
    x = torch.randn(M, cfg["hidden"], device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty_like(x)

    def step():
        layer.forward(kv, x, y)
        kv.trim(M)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps

    # per-kernel durations: the same steps with events around every launch
    ctx.profile(True)
    ctx.profile_reset()
    for _ in range(args.steps):
        step()
    stats = ctx.profile_stats()
    ctx.profile(False)
    moe_bytes, n_unique = ctx.last_moe_bytes()

    H, F, E = cfg["hidden"], cfg["expert_width"], cfg["experts"]
    gate_up_bytes = (n_unique + 1) * 2 * qbytes(F, H, gs)
    down_bytes = (n_unique + 1) * qbytes(H, F, gs)
    kernels = {k: dict(launches=n, avg_us=round(1e3 * ms / n, 3)) for k, (n, ms) in stats.items()}
    gu_s = stats["moe_gate_up"][1] / stats["moe_gate_up"][0] / 1e3
    dn_s = stats["moe_down"][1] / stats["moe_down"][0] / 1e3
    moe_s = sum(stats[k][1] / stats[k][0] for k in ("moe_router_route", "moe_gate_up", "moe_down", "moe_combine")) / 1e3
    achieved = gate_up_bytes / gu_s / 1e9
    qkv_rows = cfg["heads"] * cfg["head_dim"] * 2 + 2 * cfg["kv_heads"] * cfg["head_dim"] + cfg["index_dim"]
    attn_bytes = qbytes(qkv_rows, H, gs) + qbytes(H, cfg["heads"] * cfg["head_dim"], gs)
    step_bytes = moe_bytes + attn_bytes + 2 * 2 * cfg["kv_heads"] * (T0 + M) * cfg["head_dim"]
    out.update({
        "value": round(M / (ms_per_step / 1e3), 2),
        "ms_per_step": round(ms_per_step, 4),
        "config": {
            "workload": f"BASELINE config 3: one full-shape 125B-A6B decoder layer (attention + MoE, "
                        f"hidden 2560, 512 experts top-10 + shared, width 640, 24/2 heads x 256, gs{gs}); "
                        f"verify window of {M} tokens over {T0} cached positions; value = verified tokens/s "
                        f"through this one layer (not full-model decode tok/s)",
            "verify_width": M, "cached_positions": T0, "group_size": gs, "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "moe_gate_up (routed + shared gate|up GEMV + SwiGLU)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "algorithmic_bytes": gate_up_bytes,
            "avg_us": round(gu_s * 1e6, 3),
        },
        "moe": {
            "distinct_experts": n_unique,
            "bytes": moe_bytes,
            "block_GBps": round(moe_bytes / moe_s / 1e9, 1),
            "down_GBps": round(down_bytes / dn_s / 1e9, 1),
        },
        "step_GBps": round(step_bytes / (ms_per_step / 1e3) / 1e9, 1),
        "kernels": kernels,
    })
    tr = traffic_record(gs, M, T0, "layer")
    if tr is not None:
        out["roofline"]["traffic"] = tr["gate_up_bytes_per_launch"]
        out["roofline"]["traffic_source"] = tr["source"]
    if args.copy_calibration:
        copy_calibration()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(layer, ctx, kv, cfg, M)
    return out


def run_prefill(args, out):
    """The prompt of configs 4 and 5 through mtpx_session_prefill (the target prefill in batches,
    the drafter observing it): --warmup untimed and --steps timed prefills of a fresh session."""
    import numpy as np
    import torch

    import mtpx

    gs = args.group_size
    ctx = mtpx.Context(0)
    target, head, lc, tc = build_model(mtpx, ctx, args, gs, with_head=True)
    prompt = prompt_ids(args, tc["vocab"])
    sess = mtpx.Session(ctx, target, head)
    times, first = [], None
    for i in range(args.warmup + args.steps):
        sess.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        f = sess.prefill(prompt)  # synchronises once (the first token's readback)
        dt = time.perf_counter() - t0
        if first is None:
            first = f
        if f != first:
            raise SystemExit("prefill gave another first token on a repeat")
        if i >= args.warmup:
            times.append(dt)
        log(f"prefill {i}: {dt * 1e3:.1f} ms")
    ms = 1e3 * float(np.median(times))
    out.update({
        "metric": "prefill tok/s (the configs' 1024-token prompt, target + drafter observation)",
        "value": round(args.prompt / (ms / 1e3), 1), "unit": "tok/s", "ms_per_step": round(ms, 2),
        "config": {"workload": f"mtpx_session_prefill of a {args.prompt}-token random prompt on the full-depth "
                               f"random-init 125B-A6B target (gs{gs}, {args.layers} layers, PLE layer "
                               f"{tc['ple_layer']}) with the MTP head; value = prompt tokens / median wall time",
                   "prompt_tokens": args.prompt, "layers": args.layers, "group_size": gs,
                   "parallelism": "none (1 GPU)"},
        "first_token": int(first),
    })
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=("full", "layer", "prefill"), default="full")
    ap.add_argument("--depths", type=int, nargs="+", default=[1, 2, 3, 4, 5], help="draft depths of the decode sweep")
    ap.add_argument("--prompt", type=int, default=1024, help="prompt tokens (config 4 and 5)")
    ap.add_argument("--gen", type=int, default=1024, help="generated tokens per decode run (config 5)")
    ap.add_argument("--prefix", choices=("prompt", "synthetic"), default="prompt",
                    help="config 4's committed state: the prompt through the verify path, or random caches "
                         "(counter runs of the verify alone; implies --no-e2e)")
    ap.add_argument("--no-gs32", dest="gs32_line", action="store_false",
                    help="skip the gs32 (checkpoint format) decode line at the best depth")
    ap.add_argument("--accept-rate", type=float, default=0.7)
    ap.add_argument("--layers", type=int, default=48, help="depth of the full workload")
    ap.add_argument("--verify-width", type=int, default=4)
    ap.add_argument("--cached", type=int, default=1024)
    ap.add_argument("--group-size", type=int, default=64)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ple", action="store_true", help="leave the PLE block (and its 32 GB table) out")
    ap.add_argument("--no-e2e", action="store_true", help="report the config-4 verify as the value (no decode rounds)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the timed steps, copy 256 MiB once (the reference kernel for HBM byte counters)")
    args = ap.parse_args()
    if args.prefix == "synthetic":
        args.no_e2e = True
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not implemented)"}))
        return 2
    out = {
        "metric": METRIC, "value": None, "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q4 weights x bf16 activations, exact int24 dot, f32 combine",
        "data": "synthetic (seeded random-init weights, seeded random prompt token ids)",
    }
    if args.workload == "full":
        out = run_full(args, out)
    elif args.workload == "prefill":
        out = run_prefill(args, out)
    else:
        out = run_layer(args, out)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Oracle-side composition of the target's verify forward -- TEST INFRASTRUCTURE ONLY.

Used by tests/test_gpu_target.py: downloads a target's device weights and runs
the verify forward through the CPU oracle in the order of
Runner/FastModel/TrackFastModel.swift:1165-1265 (fastStreams: hyper-connection
inject + norm, mixer, GDN or attention, inject + norm, mixer, MoE per layer;
the final mixer) and :1330-1333 (lm_head on the mixed row), with the window
commit of :726-731 as a replay of the committed positions.  On the PLE layer
(:1188-1200) the first inject-norm's stream goes through the PLE block
(oracle.ple_forward) and is normed again.

Parity unpinned: the layer wiring follows those files by reading only; every
piece it calls is pinned on its own (tests/test_oracle_*.py).
"""
import numpy as np

from oracle import oracle as O
from oracle.head_ref import _mix, embed
from oracle.layer_ref import LazyQ4, download, download_moe, moe_y, oracle_attn, read_device


def _bf(ptr, n):
    return read_device(ptr, 2 * n, np.uint16)


def _q(q4, rows, K, gs):
    return (read_device(q4.w, rows * K // 2, np.uint32).reshape(rows, K // 8),
            _bf(q4.s, rows * K // gs).reshape(rows, K // gs), _bf(q4.b, rows * K // gs).reshape(rows, K // gs))


def download_hc(m, H, hc, LW, gs):
    W = hc * H
    return dict(scale=_bf(m.norm_scale, W), down=_q(m.down, LW, W, gs), up=_q(m.up, W, LW, gs),
                inject=_q(m.inject, hc, W, gs) if m.inject.w else None)


def download_gdn(w, H, hk, hv, kc, gs):
    g = O.gdn_geom(hk, hv, kc)
    return dict(in_proj=_q(w.in_proj, g.proj_w, H, gs), out_proj=_q(w.out_proj, H, hv * 128, gs),
                conv_w=_bf(w.conv_w, g.conv_dim * g.kc).reshape(g.conv_dim, g.kc),
                nea=read_device(w.neg_exp_alog, 4 * hv, np.float32), dtb=_bf(w.dt_bias, hv), nw=_bf(w.norm_w, 128),
                geom=g)


def ple_cfg_dict(pc):
    """The oracle's PLE config dict from an mtpx.PLEConfig."""
    return dict(hidden=pc.hidden, hc=pc.hc, embed_dim=pc.embed_dim, ngram_size=pc.ngram_size,
                heads_per_ngram=pc.heads_per_ngram, conv_kernel=pc.conv_kernel, group_size=pc.group_size,
                row_group_size=pc.row_group_size, eos=pc.eos, eps=pc.eps)


def download_ple(pw, pc, lazy=False):
    """Device weights of a PLE block (mtpx.PLEWeights) for oracle.ple_forward.  lazy: table rows
    are copied from the device only as a window's n-gram ids select them (ple_fetch)."""
    H, W, E, gs, rgs = pc.hidden, pc.hc * pc.hidden, pc.embed_dim, pc.group_size, pc.row_group_size
    nh = (pc.ngram_size - 1) * pc.heads_per_ngram
    rd = E // nh
    t = pw.table
    rows = t.rows
    lazy_table = None
    if lazy:
        lazy_table = LazyQ4(t.w, t.s, t.b, rows, rd, rgs)
        table = lazy_table.arrays
    else:
        table = (read_device(t.w, rows * rd // 2, np.uint32).reshape(rows, rd // 8),
                 _bf(t.s, rows * rd // rgs).reshape(rows, rd // rgs),
                 _bf(t.b, rows * rd // rgs).reshape(rows, rd // rgs))
    return dict(_lazy_table=lazy_table, key_proj=_q(pw.key_proj, W, E, gs), value_proj=_q(pw.value_proj, H, E, gs),
                norm_key=_bf(pw.norm_key, W), norm_query=_bf(pw.norm_query, W), norm_conv=_bf(pw.norm_conv, W),
                conv_w=_bf(pw.conv_w, W * pc.conv_kernel).reshape(W, pc.conv_kernel), table=table,
                mult=np.array(list(t.multiplier)[:pc.ngram_size], np.int64),
                vocab=np.array(list(t.vocab)[:nh], np.int64), offs=np.array(list(t.offset)[:nh], np.int64))


def ple_fetch(Lp, pc, ids, context):
    """Copy the table rows a window's n-gram ids select (a lazily downloaded table)."""
    lt = Lp.get("_lazy_table")
    if lt is None:
        return
    hist = np.concatenate([np.asarray(context, np.int32), np.asarray(ids, np.int32)])
    rid = O.ngram_row_ids(hist, len(context), pc["ngram_size"], pc["heads_per_ngram"], Lp["mult"], Lp["vocab"],
                          Lp["offs"], lt.have.size, pc["eos"])
    lt.fetch(np.concatenate([rid.reshape(-1), [0]]))


def download_target(t, cfg, lazy=False):
    """cfg: dict with the layer config keys plus key_heads, value_heads, conv_kernel,
    num_layers, full_attention_interval, hc, lowrank, vocab.  lazy: embedding rows, routed
    experts and n-gram table rows are copied from the device only as the oracle uses them."""
    H, gs, hc, LW, V = cfg["hidden"], cfg["group_size"], cfg["hc"], cfg["lowrank"], cfg["vocab"]
    tw = t.weights()
    emb = LazyQ4(tw.embed.w, tw.embed.s, tw.embed.b, V, H, gs) if lazy else _q(tw.embed, V, H, gs)
    w = dict(embed=emb, lm_head=_q(tw.lm_head, V, H, gs),
             final_hc=download_hc(tw.final_hc, H, hc, LW, gs), layers=[])
    for i in range(cfg["num_layers"]):
        lw = t.layer_weights(i)
        L = dict(kind=lw.kind, attn_hc=download_hc(lw.attn_hc, H, hc, LW, gs),
                 mlp_hc=download_hc(lw.mlp_hc, H, hc, LW, gs))
        if lw.kind == 1:
            L["attn"] = download(lw.attn, cfg, lazy)
            L["moe"] = L["attn"]["moe"]
        else:
            L["gdn"] = download_gdn(lw.gdn, H, cfg["key_heads"], cfg["value_heads"], cfg["conv_kernel"], gs)
            L["moe"] = download_moe(lw.attn.moe, cfg, lazy)
        if i == cfg.get("ple_layer", -1):
            L["ple"] = download_ple(lw.ple, t.cfg.ple, lazy)
            L["ple_cfg"] = ple_cfg_dict(t.cfg.ple)
        w["layers"].append(L)
    return w


def _gdn(L, proj, conv, ssm, eps):
    d = L["gdn"]
    return O.gdn_core(d["geom"], proj, conv, ssm, d["conv_w"], d["nea"], d["dtb"], d["nw"], eps)


def oracle_verify(w, cfg, state, ids, pos0):
    """state: dict(kc={layer: [HK, P, D]}, vc=..., conv={layer: ...}, ssm={layer: ...},
    ple=(conv rows, context) of the PLE layer) of the committed caches (kc/vc receive the
    window's rows in place).
    -> (logits [S, V], multi [S, hc*H], mixed [S, H], window) where window feeds oracle_commit."""
    H, gs, hc, eps = cfg["hidden"], cfg["group_size"], cfg["hc"], cfg["eps"]
    e = embed(w["embed"], gs, ids)
    resid, out, inj, tile = e, None, None, True
    window = {}
    for i, L in enumerate(w["layers"]):
        sA, n = O.hc_norm(resid, out, inj, L["attn_hc"]["scale"], hc, eps, tile=tile)
        if "ple" in L:
            conv, context = state["ple"]
            ple_fetch(L["ple"], L["ple_cfg"], ids, context)
            res = O.ple_forward(L["ple"], L["ple_cfg"], sA, ids, conv, context)
            window["ple"] = (i, res)
            sA, n = O.hc_norm(res["sum"], None, None, L["attn_hc"]["scale"], hc, eps)
        x, jA = _mix(L["attn_hc"], n, hc, gs)
        if L["kind"] == 0:
            proj, _ = O.qmv(*L["gdn"]["in_proj"], gs, x)
            r = _gdn(L, proj, state["conv"][i], state["ssm"][i], eps)
            window[i] = proj
            ao, _ = O.qmv(*L["gdn"]["out_proj"], gs, r["gated"])
        else:
            ao = oracle_attn(L["attn"], cfg, state["kc"][i], state["vc"][i], x, pos0)
        sM, n = O.hc_norm(sA, ao, jA, L["mlp_hc"]["scale"], hc, eps)
        x, jM = _mix(L["mlp_hc"], n, hc, gs)
        mo = moe_y(L["moe"], x, H, cfg["experts"], cfg["top_k"], cfg["expert_width"], gs)
        resid, out, inj, tile = sM, mo, jM, False
    multi, n = O.hc_norm(resid, out, inj, w["final_hc"]["scale"], hc, eps)
    mixed, _ = _mix(w["final_hc"], n, hc, gs)
    logits, _ = O.qmv(*w["lm_head"], gs, mixed)
    return logits, multi, mixed, window


def oracle_commit(w, cfg, state, window, n):
    """Advance the GDN (and PLE) states of `state` by the first n positions of a verify window."""
    for i, proj in window.items():
        if i == "ple":
            li, res = proj
            pc = w["layers"][li]["ple_cfg"]
            nb = (pc["conv_kernel"] - 1) * pc["ngram_size"]
            state["ple"] = O.ple_advance(res, n, nb, max(1, pc["ngram_size"] - 1))
            continue
        if n == 0:
            continue
        r = _gdn(w["layers"][i], proj[:n], state["conv"][i], state["ssm"][i], cfg["eps"])
        state["conv"][i], state["ssm"][i] = r["conv_state"], r["ssm"]

"""Oracle-side composition of one MTP head draft step -- TEST INFRASTRUCTURE ONLY.

Used by tests/test_gpu_head.py: downloads a head's device weights and runs the
same draft step through the CPU oracle, in the order of
Runner/FastModel/TrackFastHead.swift:101-153 (the fast head forward) and
Runner/Qwen4ExpMTP.swift:101-130 (the module wiring), with the drafter's
shortlist argmax (Runner/Qwen4ExpMTPDrafter.swift:122-153).

Parity unpinned: the wiring of oracle_head (which stream feeds which norm,
mixer and sublayer) follows those files by reading only; no reference output
exists to check it against.  Every piece it calls is pinned on its own
(tests/test_oracle_pin.py, tests/test_oracle_head_pin.py).
"""
import numpy as np

from oracle import oracle as O
from oracle.layer_ref import LazyQ4, download, moe_y, oracle_attn, read_device


def embed(e, gs, ids):
    """Embedding rows of ids; e is a q4 triple or a LazyQ4 (rows fetched first)."""
    if isinstance(e, LazyQ4):
        e.fetch(ids)
        e = e.arrays
    return O.embed_rows(*e, gs, ids)


def download_head(hw, hcfg, lazy=False):
    """hcfg: dict with the layer config keys plus hc, lowrank, vocab.  lazy: embedding rows
    and routed experts are copied from the device only as the oracle uses them."""
    H, gs, hc, LW = hcfg["hidden"], hcfg["group_size"], hcfg["hc"], hcfg["lowrank"]
    W = hc * H

    def bf(ptr, n):
        return read_device(ptr, 2 * n, np.uint16)

    def q(q4, rows, K):
        return (read_device(q4.w, rows * K // 2, np.uint32).reshape(rows, K // 8),
                bf(q4.s, rows * K // gs).reshape(rows, K // gs), bf(q4.b, rows * K // gs).reshape(rows, K // gs))

    emb = (LazyQ4(hw.embed.w, hw.embed.s, hw.embed.b, hcfg["vocab"], H, gs) if lazy
           else q(hw.embed, hcfg["vocab"], H))
    w = dict(layer=download(hw.layer, hcfg, lazy), embed=emb,
             pre_norm_embedding=bf(hw.pre_norm_embedding, H), pre_norm_hidden=bf(hw.pre_norm_hidden, W),
             fc_embedding=q(hw.fc_embedding, H, H), fc_hidden=q(hw.fc_hidden, H, H))
    for name in ("attn_hc", "mlp_hc", "final_hc"):
        m = getattr(hw, name)
        w[name] = dict(scale=bf(m.norm_scale, W), down=q(m.down, LW, W), up=q(m.up, W, LW),
                       inject=q(m.inject, hc, W) if m.inject.w else None)
    ns = hw.shortlist_rows
    w["shortlist"] = q(hw.shortlist, ns, H)
    w["shortlist_ids"] = read_device(hw.shortlist_ids, 4 * ns, np.int32)
    return w


def _mix(m, normed, hc, gs):
    lo, _ = O.qmv(*m["down"], gs, normed)
    inj = O.qmv(*m["inject"], gs, normed)[0] if m["inject"] is not None else None
    act = O.silu_rows(lo)
    wm, _ = O.qmv(*m["up"], gs, act)
    return O.hc_mix(wm, normed, inj, hc)


def oracle_head(w, hcfg, kc, vc, ids, multi, pos0):
    """-> (multi_next [S, hc*H], sample [S, H], draft id of the last row)."""
    H, gs, hc, eps = hcfg["hidden"], hcfg["group_size"], hcfg["hc"], hcfg["eps"]
    S = len(ids)
    e = embed(w["embed"], gs, ids)
    _, en = O.hc_norm(e, None, None, w["pre_norm_embedding"], 1, eps)
    emb, _ = O.qmv(*w["fc_embedding"], gs, en)
    _, mn = O.hc_norm(multi, None, None, w["pre_norm_hidden"], 1, eps)
    hs, _ = O.qmv(*w["fc_hidden"], gs, mn.reshape(S * hc, H))
    hs = hs.reshape(S, hc * H)
    st0, n0 = O.hc_norm(hs, emb, None, w["attn_hc"]["scale"], hc, eps)
    x, j = _mix(w["attn_hc"], n0, hc, gs)
    ao = oracle_attn(w["layer"], hcfg, kc, vc, x, pos0)
    st1, n1 = O.hc_norm(st0, ao, j, w["mlp_hc"]["scale"], hc, eps)
    x, j = _mix(w["mlp_hc"], n1, hc, gs)
    m = moe_y(w["layer"]["moe"], x, H, hcfg["experts"], hcfg["top_k"], hcfg["expert_width"], gs)
    multi_next, n2 = O.hc_norm(st1, m, j, w["final_hc"]["scale"], hc, eps)
    sample, _ = _mix(w["final_hc"], n2, hc, gs)
    logits, _ = O.qmv(*w["shortlist"], gs, sample[S - 1:S])
    draft = O.shortlist_argmax(logits, w["shortlist_ids"])
    return multi_next, sample, draft

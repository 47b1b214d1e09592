"""CPU-side checks of the C ABI: the library loads and exports every entry point
that include/mtpx.h declares (no compute call is made without a GPU)."""
import ctypes as C
import os

import pytest

from mtpx import _lib


def test_header_symbols_exported():
    L = C.CDLL(_lib.LIB_PATH)
    syms = _lib.header_symbols()
    assert len(syms) >= 25
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_binding_covers_header():
    assert set(_lib.header_symbols()) == set(_lib._SIGS)


def test_version_and_error_string():
    L = _lib.lib()
    assert L.mtpx_version().decode().startswith("mtpx")
    assert isinstance(L.mtpx_last_error(), bytes)


def test_struct_sizes_match_header_layout():
    # offsets of the pointer block after five ints (padded to 8)
    assert C.sizeof(_lib.MoEWeights) == 24 + 30 * 8
    assert _lib.LayerWeights.moe.offset == 12 * 8


def test_struct_layouts_match_c_compiler(tmp_path):
    """sizeof/offsetof of every ABI struct as gcc lays out include/mtpx.h, against ctypes."""
    import shutil
    import subprocess
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    inc = os.path.dirname(_lib.HEADER)
    checks = {
        "mtpx_moe_weights": (_lib.MoEWeights, ["router", "gate_w", "sh_down_b", "gate_sb", "sh_down_sb"]),
        "mtpx_layer_config": (_lib.LayerConfig, ["rope_theta", "max_positions"]),
        "mtpx_layer_weights": (_lib.LayerWeights, ["rope_sin", "moe", "qkv_rows", "qkv_sb", "o_sb"]),
        "mtpx_q4": (_lib.Q4, ["s", "b", "sb"]),
        "mtpx_hc_weights": (_lib.HCWeights, ["down", "inject", "up"]),
        "mtpx_head_config": (_lib.HeadConfig, ["hc", "lowrank", "vocab", "shortlist_low", "shortlist_special_from"]),
        "mtpx_drafter_info": (_lib.DrafterInfo, ["round_base_offset", "round_in_flight", "released"]),
        "mtpx_head_weights": (_lib.HeadWeights, ["pre_norm_hidden", "attn_hc", "final_hc", "layer", "shortlist",
                                                 "shortlist_ids", "shortlist_rows"]),
        "mtpx_gdn_config": (_lib.GDNConfig, ["value_heads", "group_size", "eps"]),
        "mtpx_gdn_weights": (_lib.GDNWeights, ["conv_w", "neg_exp_alog", "norm_w", "out_proj"]),
        "mtpx_target_config": (_lib.TargetConfig, ["key_heads", "num_layers", "lowrank", "vocab"]),
        "mtpx_target_layer_weights": (_lib.TargetLayerWeights, ["attn", "gdn", "attn_hc", "mlp_hc"]),
        "mtpx_target_weights": (_lib.TargetWeights, ["final_hc", "lm_head"]),
        "mtpx_force_params": (_lib.ForceParams, ["teacher_len", "rate", "seed"]),
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "mtpx.h"', "int main(void) {"]
    for name, (_, fields) in checks.items():
        lines.append(f'printf("{name} %zu\\n", sizeof({name}));')
        for f in fields:
            lines.append(f'printf("{name}.{f} %zu\\n", offsetof({name}, {f}));')
    lines.append("return 0; }")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-I", inc, str(src), "-o", str(exe)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], check=True, capture_output=True,
                                                  text=True).stdout.splitlines())
    for name, (cls, fields) in checks.items():
        assert int(got[name]) == C.sizeof(cls), name
        for f in fields:
            assert int(got[f"{name}.{f}"]) == getattr(cls, f).offset, f"{name}.{f}"

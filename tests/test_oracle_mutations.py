"""Plants plausible wiring slips in copies of the oracle (on the CPU) and
checks that the composition pins (test_oracle_layer_pins.py) catch each one.

Every mutant is oracle.c with one textual change, built into a temporary
library and loaded through MYL_ORACLE_LIB by a pytest subprocess that runs
the pins; the unchanged source built the same way must pass them.  A
mutant that passes means the pins leave that slip open.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
ORACLE = ROOT / "oracle"

# name -> [(text in oracle.c, replacement)]; model.rs lines the slip contradicts
MUTANTS = {
    # model.rs:576-581: the o_proj accumulation scale is the coarser (min) one
    "acc_attn_max": [("acc_attn[i] = L->res_in_frac[i] < L->res_mid_frac[i] ?",
                      "acc_attn[i] = L->res_in_frac[i] > L->res_mid_frac[i] ?")],
    # model.rs:612-617
    "acc_mlp_max": [("acc_mlp[i] = L->res_mid_frac[i] < out_res_frac[i] ?",
                     "acc_mlp[i] = L->res_mid_frac[i] > out_res_frac[i] ?")],
    # model.rs:543-545: score_shift = q_frac + k_frac + 15 - score_frac_bits
    "score_shift_plus1": [("+ sc->k_frac + 15u;", "+ sc->k_frac + 16u;")],
    "score_shift_minus1": [("+ sc->k_frac + 15u;", "+ sc->k_frac + 14u;")],
    # model.rs:500-503: V is cached unrotated
    "v_rotated": [("memcpy(kv_at(m->vcache, s, l, h, pos), vf + h * hd, hd * 2);",
                   "or_rotate_half_split_i16(vf + h * hd, hd, cr, sr, MYL_TV_ROPE_FRAC_BITS, "
                   "kv_at(m->vcache, s, l, h, pos));")],
    # model.rs:449-451 then :475-477: the K bias comes before RoPE
    "k_bias_after_rope": [
        ("        or_add_bias_i16(kf, L->bk, L->bk_s, kvN, sc->k_frac);\n", ""),
        ("or_rotate_half_split_i16(kf + h * hd, hd, cr, sr, MYL_TV_ROPE_FRAC_BITS, kv_at(m->kcache, s, l, h, pos));",
         "or_rotate_half_split_i16(kf + h * hd, hd, cr, sr, MYL_TV_ROPE_FRAC_BITS, kv_at(m->kcache, s, l, h, pos));"
         " if (s->attention_bias) or_add_bias_i16(kv_at(m->kcache, s, l, h, pos), L->bk + h * hd, L->bk_s + h * hd,"
         " hd, sc->k_frac);")],
    # model.rs:452-454: the V bias
    "v_bias_dropped": [("        or_add_bias_i16(vf, L->bv, L->bv_s, kvN, sc->v_frac);\n", "")],
    # model.rs:563-567: attention output rescaled v_frac -> attn_out_frac
    "attn_out_not_rescaled": [("if (sc->attn_out_frac != sc->v_frac)", "if (0)")],
    # model.rs:588-593: residual read at res_in, written at res_mid
    "resid1_reads_mid": [("or_rescale_i64(hidden[i], L->res_in_frac[i], acc_attn[i])",
                          "or_rescale_i64(hidden[i], L->res_mid_frac[i], acc_attn[i])")],
    "resid1_writes_in": [("or_rescale_i64(sum, acc_attn[i], L->res_mid_frac[i])",
                          "or_rescale_i64(sum, acc_attn[i], L->res_in_frac[i])")],
    # model.rs:666-671: the residual moved onto the accumulation scale first
    "resid2_not_moved": [("int64_t r = or_rescale_i64(resid[i], L->res_mid_frac[i], acc_mlp[i]);",
                          "int64_t r = resid[i];")],
    # model.rs:508-511: head h reads KV head h / group
    "gqa_modulo": [("uint32_t kvh = (uint32_t)h / group;", "uint32_t kvh = (uint32_t)h % s->kv_heads;")],
    # model.rs:469-473: RoPE row pos % n_pos
    "rope_row_clamped": [("idx = pos % n_pos;", "idx = pos < n_pos ? pos : n_pos - 1;")],
    # model.rs:339-356: a layer writes at the next layer's input scale
    "layer_out_at_own_scale": [("? m->layers[l + 1].res_in_frac :", "? m->layers[l].res_in_frac :")],
    # model.rs:241-248: the embedding lands on the first layer's input scale
    "embed_at_final_scale": [("const uint8_t* first = m->layers[0].res_in_frac;",
                              "const uint8_t* first = m->final_res_frac;")],
    # model.rs:293-295: LM head shift = row shift + final_norm_frac
    "head_without_norm_frac": [("(uint8_t)(sh + m->final_norm_frac)", "(uint8_t)(sh)")],
}


def _build(name: str, edits, tmp: Path) -> Path:
    src = (ORACLE / "oracle.c").read_text()
    for old, new in edits:
        assert src.count(old) == 1, f"{name}: the text to replace must occur exactly once: {old!r}"
        src = src.replace(old, new)
    c = tmp / f"{name}.c"
    c.write_text(src)
    so = tmp / f"lib{name}.so"
    # -I the oracle directory: oracle.c's "oracle.h" and "../include/..." resolve there
    subprocess.run(["gcc", "-O2", "-march=x86-64-v3", "-fPIC", "-fopenmp", "-std=gnu11", "-shared",
                    "-I", str(ORACLE), "-o", str(so), str(c)], check=True, capture_output=True)
    return so


def _run_pins(so: Path) -> subprocess.CompletedProcess:
    env = dict(os.environ, MYL_ORACLE_LIB=str(so))
    return subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                           str(ROOT / "tests" / "test_oracle_layer_pins.py")], cwd=ROOT, env=env,
                          capture_output=True, text=True, timeout=600)


def test_pins_catch_every_planted_slip(tmp_path):
    jobs = {"unchanged": []}
    jobs.update(MUTANTS)
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        libs = dict(zip(jobs, ex.map(lambda kv: _build(kv[0], kv[1], tmp_path), jobs.items())))
        runs = dict(zip(libs, ex.map(_run_pins, libs.values())))
    control = runs.pop("unchanged")
    assert control.returncode == 0, "the pins fail on the unchanged oracle:\n" + control.stdout[-3000:]
    survivors = [name for name, r in runs.items() if r.returncode == 0]
    assert not survivors, f"slips the pins do not catch: {survivors}"
    for name, r in runs.items():
        assert "failed" in r.stdout, f"{name}: the pins did not fail cleanly:\n{r.stdout[-2000:]}{r.stderr[-2000:]}"

"""GPU parity of models built from the reference's artifact format and from
tensor uploads (include/myl_hip.h section 5) against the oracle.

The oracle's synthetic model supplies the tensors in the reference layout
(IntegerModel fields, runtime/src/model.rs); an artifact written from them is
loaded through myl_model_load_artifact and must reproduce the oracle's
forward pass bit for bit.  Downloads, exports, the untied int8 head, uniform
manifest shifts and the refusal paths are covered as well."""
from __future__ import annotations

import json

import numpy as np
import pytest

from conftest import case

pytestmark = pytest.mark.gpu

FRAC_FIELDS = ("norm_attn_frac", "q_frac", "k_frac", "v_frac", "attn_out_frac", "norm_mlp_frac", "gate_frac",
               "up_frac", "down_in_frac")


def tiny(hd=64, lm16=0, bias=1, kv_heads=2, layers=2, max_pos=256, seed=21):
    heads = 4 if kv_heads <= 2 else 8
    return dict(seed=seed, vocab=1000, hidden=heads * hd, layers=layers, heads=heads, kv_heads=kv_heads, head_dim=hd,
                inter=320, max_pos=max_pos, lm_head_int16=lm16, attention_bias=bias)


def dims_of(spec, tie=1):
    d = {k: spec[k] for k in ("vocab", "hidden", "layers", "heads", "kv_heads", "head_dim", "inter",
                              "lm_head_int16", "attention_bias")}
    d.update(max_context=spec["max_pos"], tie_word_embeddings=tie)
    return d


def oracle_parts(om, spec):
    """The oracle model's tensors by HF name, its LayerScales and final scales."""
    H, I, V = spec["hidden"], spec["inter"], spec["vocab"]
    nq, nkv = spec["heads"] * spec["head_dim"], spec["kv_heads"] * spec["head_dim"]
    u8 = np.uint8
    t = {"model.embed_tokens.weight": (om.tensor("emb").reshape(V, H), om.tensor("emb_shifts", 0, u8)),
         "model.norm.weight": (om.tensor("final_gamma"), om.tensor("final_gamma_shifts", 0, u8))}
    if spec["lm_head_int16"]:
        t["lm_head.weight"] = (om.tensor("lm16", 0, np.int16).reshape(V, H), om.tensor("lm16_shifts", 0, u8))
    layers = []
    for l in range(spec["layers"]):
        p = f"model.layers.{l}."
        T = lambda n, dt=np.int8: om.tensor(n, l, dt)
        t[p + "input_layernorm.weight"] = (T("in_gamma"), T("in_gamma_shifts", u8))
        t[p + "post_attention_layernorm.weight"] = (T("post_gamma"), T("post_gamma_shifts", u8))
        for w, s, rows, cols, nm in (("wq", "sq", nq, H, "self_attn.q_proj"), ("wk", "sk", nkv, H, "self_attn.k_proj"),
                                     ("wv", "sv", nkv, H, "self_attn.v_proj"), ("wo", "so", H, nq, "self_attn.o_proj"),
                                     ("wg", "sg", I, H, "mlp.gate_proj"), ("wu", "su", I, H, "mlp.up_proj"),
                                     ("wd", "sd", H, I, "mlp.down_proj")):
            t[p + nm + ".weight"] = (T(w).reshape(rows, cols), T(s, u8))
        if spec["attention_bias"]:
            for b, nm in (("bq", "q_proj"), ("bk", "k_proj"), ("bv", "v_proj")):
                t[p + f"self_attn.{nm}.bias"] = (T(b, np.int16), T(b + "_s", u8))
        fr = T("layer_fracs", u8)
        layers.append((dict(zip(FRAC_FIELDS, map(int, fr))), T("res_in_frac", u8), T("res_mid_frac", u8)))
    final = (int(om.tensor("final_norm_frac", 0, u8)[0]), om.tensor("final_res_frac", 0, u8))
    return t, layers, final


def oracle_model(spec, luts):
    from oracle.binding import OracleModel
    return OracleModel(spec, luts, threads=16)


def fill(gm, tensors, layers, final):
    for name, (data, shifts) in tensors.items():
        gm.upload_tensor(name, data, shifts)
    for l, (fr, ri, rm) in enumerate(layers):
        gm.set_layer_scales(l, fr, ri, rm)
    gm.set_final_scales(*final)
    gm.finalize()


def same_forward(gm, om, spec, n=40, seed=0):
    toks = np.random.default_rng(seed).integers(0, spec["vocab"], n)
    gm.reset()
    om.reset()
    for pos, tok in enumerate(toks):
        assert np.array_equal(gm.forward_token(int(tok), pos), om.forward_token(int(tok), pos)), pos
    for l in range(spec["layers"]):
        for h in range(spec["kv_heads"]):
            gk, gv = gm.read_kv(l, h, n)
            ok, ov = om.read_kv(l, h, n)
            assert np.array_equal(gk, ok) and np.array_equal(gv, ov), (l, h)


@pytest.mark.parametrize("hd,lm16,bias,kvh", [(64, 0, 1, 2), (128, 1, 1, 2), (64, 1, 0, 1)])
def test_artifact_from_oracle_tensors_loads_and_matches(backend, tmp_path, hd, lm16, bias, kvh):
    from myelith_amd.artifact import Artifact, write_artifact
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    spec = tiny(hd, lm16, bias, kvh)
    case(f"artifact from oracle tensors {spec}")
    luts = LutSet.for_head_dim(hd)
    om = oracle_model(spec, luts)
    tensors, layers, final = oracle_parts(om, spec)
    write_artifact(tmp_path, dims_of(spec), tensors, layers, final, luts)
    with Artifact(tmp_path) as a:
        a.verify()
        gm = IntegerModel.from_artifact(backend, a)
    same_forward(gm, om, spec)
    # every tensor reads back in the reference layout
    for name, (data, shifts) in tensors.items():
        got, gs = gm.download_tensor(name, data.shape, 16 if data.dtype == np.int16 else 8)
        assert np.array_equal(got, data) and np.array_equal(gs, shifts), name
    gm.close()


def test_uploads_match_the_synthetic_model_and_export_round_trips(backend, tmp_path):
    from myelith_amd.artifact import export_model
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel, dekodieren_mit_digest
    spec = tiny(128, 1, 1, 2, layers=3)
    case("upload path vs synthetic; export -> load")
    luts = LutSet.for_head_dim(128)
    om = oracle_model(spec, luts)
    tensors, layers, final = oracle_parts(om, spec)
    up = IntegerModel.create(backend, dims_of(spec), spec["max_pos"], luts)
    with pytest.raises(ValueError, match="not finalized"):
        up.forward_token(1, 0)
    fill(up, tensors, layers, final)
    syn = IntegerModel(backend, spec, luts)
    toks = np.random.default_rng(1).integers(0, spec["vocab"], 24)
    out_up, dig_up = dekodieren_mit_digest(up, toks[:8], 16)
    out_syn, dig_syn = dekodieren_mit_digest(syn, toks[:8], 16)
    assert out_up == out_syn and dig_up == dig_syn
    export_model(syn, tmp_path / "exp")
    back = IntegerModel.from_artifact(backend, tmp_path / "exp")
    for l in range(spec["layers"]):
        f0, ri0, rm0 = syn.layer_scales(l)
        f1, ri1, rm1 = back.layer_scales(l)
        assert f0 == f1 and np.array_equal(ri0, ri1) and np.array_equal(rm0, rm1)
    out_b, dig_b = dekodieren_mit_digest(back, toks[:8], 16)
    assert out_b == out_syn and dig_b == dig_syn
    # greedy decode on the device (graph replay) agrees as well
    syn.reset()
    back.reset()
    syn.prefill(toks[:8])
    back.prefill(toks[:8])
    a, _ = syn.decode_greedy(int(toks[8]), 8, 12)
    b, _ = back.decode_greedy(int(toks[8]), 8, 12)
    assert np.array_equal(a, b)
    for m in (up, syn, back):
        m.close()


def test_untied_int8_head(backend):
    """tie_word_embeddings = false without an int16 head: logits come from
    lm_head.weight, the token embedding from model.embed_tokens.weight
    (model.rs:297-307, loader.rs:730-735)."""
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    spec = tiny(64, 0, 1, 2)
    case("untied int8 head")
    luts = LutSet.for_head_dim(64)
    om = oracle_model(spec, luts)
    tensors, layers, final = oracle_parts(om, spec)
    rng = np.random.default_rng(5)
    V, H = spec["vocab"], spec["hidden"]
    w2 = rng.integers(-127, 128, (V, H)).astype(np.int8)
    s2 = rng.integers(8, 12, V).astype(np.uint8)
    untied = IntegerModel.create(backend, dims_of(spec, tie=0), spec["max_pos"], luts)
    fill(untied, dict(tensors, **{"lm_head.weight": (w2, s2)}), layers, final)
    tied = IntegerModel.create(backend, dims_of(spec, tie=1), spec["max_pos"], luts)
    fill(tied, dict(tensors, **{"model.embed_tokens.weight": (w2, s2)}), layers, final)
    for tok in (0, 7, 999):
        assert np.array_equal(untied.embed_token(tok), om.embed_token(tok))
    for s in range(4):
        h = rng.integers(-20000, 20000, H).astype(np.int16)
        assert np.array_equal(untied.head_logits(h), tied.head_logits(h))
    # finalize names a missing head
    bare = IntegerModel.create(backend, dims_of(spec, tie=0), spec["max_pos"], luts)
    with pytest.raises(ValueError, match="lm_head.weight"):
        fill(bare, tensors, layers, final)
    for m in (untied, tied, bare):
        m.close()


def test_uniform_manifest_shift_and_refusals(backend, tmp_path):
    """A manifest entry without shifts_file carries one shift for every row
    (loader.rs:476-484); a tampered tensor file refuses the load; uploads of
    the wrong shape or name are refused."""
    from myelith_amd.artifact import write_artifact
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    spec = tiny(64, 0, 1, 2)
    case("uniform manifest shift; refusals")
    luts = LutSet.for_head_dim(64)
    om = oracle_model(spec, luts)
    tensors, layers, final = oracle_parts(om, spec)
    name = "model.layers.1.self_attn.o_proj.weight"
    w, s = tensors[name]
    tensors[name] = (w, np.full_like(s, 7))
    ref = IntegerModel.create(backend, dims_of(spec), spec["max_pos"], luts)
    fill(ref, tensors, layers, final)
    d = tmp_path / "uni"
    write_artifact(d, dims_of(spec), tensors, layers, final, luts)
    man = json.loads((d / "weights_manifest.json").read_text())
    e = man["model_layers_1_self_attn_o_proj_weight"]
    e.pop("shifts_file")
    e.pop("shifts_hash")
    e["shift"] = 7
    (d / "weights_manifest.json").write_text(json.dumps(man))
    theta = json.loads((d / "theta_v.json").read_text())
    import hashlib
    theta["weights_hash"] = hashlib.sha256((d / "weights_manifest.json").read_bytes()).hexdigest()
    (d / "theta_v.json").write_text(json.dumps(theta))
    uni = IntegerModel.from_artifact(backend, d)
    toks = [3, 500, 999, 0, 42]
    for pos, t in enumerate(toks):
        assert np.array_equal(uni.forward_token(t, pos), ref.forward_token(t, pos))
    # a flipped byte in one tensor file: the load fails, no model is returned
    f = d / "model_layers_0_mlp_up_proj_weight.bin"
    raw = bytearray(f.read_bytes())
    raw[100] ^= 1
    f.write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="SHA-256"):
        IntegerModel.from_artifact(backend, d)
    with pytest.raises(ValueError, match="shape"):
        ref.upload_tensor("model.norm.weight", np.zeros(spec["hidden"] + 16, np.int8), np.zeros(spec["hidden"] + 16))
    with pytest.raises(ValueError, match="unknown tensor"):
        ref.upload_tensor("model.layers.9.mlp.up_proj.weight", np.zeros((320, 256), np.int8), np.zeros(320))
    for m in (ref, uni):
        m.close()

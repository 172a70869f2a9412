"""The artifact reader of libmyl_hip.so on the CPU (no GPU): the checks of
INTEGER_LLM/runtime/src/loader.rs (load_weights / load_luts / load_scales /
load_model_dims / ThetaV / build_model) on fixtures shaped like the
reference's own loader tests (loader.rs:855-1998), SHA-256 known answers, and
the reference's shipped Qwen2.5-0.5B scale pack where it is present."""
from __future__ import annotations

import hashlib
import json
import os
import shutil
from pathlib import Path

import numpy as np
import pytest

from myelith_amd.artifact import THETA_V_VERSION, Artifact, sha256_hex, write_artifact

SCALE_PACK = Path("/root/reference/INTEGER_LLM/scale_packs/qwen2.5-0.5b")


def sha(b: bytes) -> str:
    return hashlib.sha256(b).hexdigest()


# ---- SHA-256 -----------------------------------------------------------------

def test_sha256_known_vectors():
    # FIPS 180-4 / loader.rs:889-900
    assert sha256_hex(b"abc") == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert sha256_hex(b"") == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"
    # two-block message of FIPS 180-4 appendix B.2
    assert sha256_hex(b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq") == \
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"


def test_sha256_matches_hashlib_across_block_boundaries():
    rng = np.random.default_rng(7)
    for n in list(range(0, 140)) + [1000, 4095, 4096, 65537, 1 << 20]:
        b = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert sha256_hex(b) == sha(b), n


# ---- a fixture built the way the reference's loader tests build theirs -------
# (loader.rs:1355-1488 write_full_fixture: 1 layer, hidden 4, 2 heads, 1 KV
# head, head_dim 2, inter 4, vocab 3; int8 data (i % 7), uniform shift 0 and
# no shifts file; int16 biases (i % 11) - 5 with shifts i % 3; short LUTs)

SCALES_1L = {
    "model.layers.0.input_layernorm": (4, 10.0),
    "model.layers.0.self_attn.q_proj": (5, 20.0),
    "model.layers.0.self_attn.k_proj": (5, 20.0),
    "model.layers.0.self_attn.v_proj": (5, 20.0),
    "model.layers.0.self_attn": (6, 15.0),
    "model.layers.0.post_attention_layernorm": (3, 40.0),
    "model.layers.0.mlp.gate_proj": (4, 30.0),
    "model.layers.0.mlp.up_proj": (3, 60.0),
    "model.layers.0.mlp.down_proj.input": (0, 100.0),
    "model.layers.0.input_layernorm.input": (12, 0.06),
    "model.layers.0.post_attention_layernorm.input": (5, 25.0),
    "model.norm": (2, 120.0),
    "model.norm.input": (4, 80.0),
}


def write_theta_v(d: Path, version: str = THETA_V_VERSION) -> None:
    h = {k: sha((d / f).read_bytes()) for k, f in (("weights_hash", "weights_manifest.json"),
                                                     ("scales_hash", "scales.json"), ("luts_hash", "luts.json"))}
    (d / "theta_v.json").write_text(json.dumps({"version": version, **h}))


def write_full_fixture(d: Path, tie: bool = True, bias: bool = True, int16_head: bool = False) -> None:
    hidden, heads, kv, hd, inter, vocab = 4, 2, 1, 2, 4, 3
    d.mkdir(parents=True, exist_ok=True)
    (d / "model_config.json").write_text(json.dumps({
        "family": "qwen2.5", "variant": "test", "num_layers": 1, "hidden_size": hidden, "intermediate_size": inter,
        "num_heads": heads, "num_kv_heads": kv, "head_dim": hd, "vocab_size": vocab, "max_context": 8,
        "tie_word_embeddings": tie, "attention_bias": bias}))
    (d / "scales.json").write_text(json.dumps(
        {k: {"shift": s, "scale": 2.0 ** -s, "absmax_observed": a} for k, (s, a) in SCALES_1L.items()}))
    manifest = {}

    def put(name, shape):
        n = int(np.prod(shape))
        data = bytes(i % 7 for i in range(n))
        key = name.replace(".", "_")
        (d / f"{key}.bin").write_bytes(data)
        manifest[key] = {"original_name": name, "file": f"{key}.bin", "shape": list(shape), "scale": 1.0,
                         "shift": 0, "dtype": "int8", "hash": sha(data)}

    put("model.embed_tokens.weight", [vocab, hidden])
    put("model.norm.weight", [hidden])
    if not tie:
        put("lm_head.weight", [vocab, hidden])
    for sfx, shape in (("input_layernorm.weight", [hidden]), ("post_attention_layernorm.weight", [hidden]),
                       ("self_attn.q_proj.weight", [heads * hd, hidden]), ("self_attn.k_proj.weight", [kv * hd, hidden]),
                       ("self_attn.v_proj.weight", [kv * hd, hidden]), ("self_attn.o_proj.weight", [hidden, heads * hd]),
                       ("mlp.gate_proj.weight", [inter, hidden]), ("mlp.up_proj.weight", [inter, hidden]),
                       ("mlp.down_proj.weight", [hidden, inter])):
        put("model.layers.0." + sfx, shape)

    def put16(name, key, shape, vals, shifts):
        data = np.asarray(vals, "<i2").tobytes()
        (d / f"{key}.bin").write_bytes(data)
        (d / f"{key}_shifts.bin").write_bytes(bytes(shifts))
        manifest[key] = {"original_name": name, "file": f"{key}.bin", "shape": shape, "scale": -1.0, "shift": -1,
                         "dtype": "int16", "hash": sha(data), "shifts_file": f"{key}_shifts.bin",
                         "shifts_hash": sha(bytes(shifts))}

    if bias:
        for p, n in (("q_proj", heads * hd), ("k_proj", kv * hd), ("v_proj", kv * hd)):
            name = f"model.layers.0.self_attn.{p}.bias"
            put16(name, name.replace(".", "_"), [n], [(i % 11) - 5 for i in range(n)], [i % 3 for i in range(n)])
    if int16_head:
        put16("lm_head.weight", "lm_head", [vocab, hidden], [i - 6 for i in range(vocab * hidden)], [5] * vocab)
    (d / "weights_manifest.json").write_text(json.dumps(manifest))
    luts = {}
    for name, vals in (("cos", [256, 0, -256, 0]), ("sin", [0, 256, 0, -256]), ("exp", [256, 128, 64]),
                       ("silu", [-10, 0, 10, 20]), ("rsqrt", [256, 181, 148])):
        raw = np.asarray(vals, "<i2").tobytes()
        (d / f"{name}.lut.bin").write_bytes(raw)
        luts[name] = {"file": f"{name}.lut.bin", "hash": sha(raw), "length": len(vals), "dtype": "int16"}
    (d / "luts.json").write_text(json.dumps(luts))
    write_theta_v(d)


def edit_json(d: Path, fname: str, fn, rehash: bool = True) -> None:
    obj = json.loads((d / fname).read_text())
    fn(obj)
    (d / fname).write_text(json.dumps(obj))
    if rehash:
        write_theta_v(d)


def open_err(d: Path) -> str:
    with pytest.raises(ValueError) as e:
        Artifact(d)
    return str(e.value)


def test_load_model_end_to_end_tied_embeddings(tmp_path):
    write_full_fixture(tmp_path, tie=True, bias=True)
    with Artifact(tmp_path) as a:
        d = a.dims
        assert (d["layers"], d["heads"], d["kv_heads"], d["head_dim"], d["hidden"], d["vocab"], d["inter"]) == \
            (1, 2, 1, 2, 4, 3, 4)
        assert d["tie_word_embeddings"] == 1 and d["attention_bias"] == 1 and d["lm_head_int16"] == 0
        assert d["max_context"] == 8
        f, ri, rm = a.layer_scales(0)
        assert f == dict(norm_attn_frac=4, q_frac=5, k_frac=5, v_frac=5, attn_out_frac=6, norm_mlp_frac=3,
                         gate_frac=4, up_frac=3, down_in_frac=0)
        # scalar residual shifts broadcast per channel (loader.rs:228-235)
        assert ri.tolist() == [12] * 4 and rm.tolist() == [5] * 4
        nf, fr = a.final_scales()
        assert nf == 2 and fr.tolist() == [4] * 4
        assert a.lut("cos").tolist() == [256, 0, -256, 0]
        assert a.lut("rsqrt").tolist() == [256, 181, 148]
        a.verify()


def test_load_model_end_to_end_untied_and_without_bias(tmp_path):
    write_full_fixture(tmp_path / "u", tie=False, bias=True)
    with Artifact(tmp_path / "u") as a:
        assert a.dims["tie_word_embeddings"] == 0
    write_full_fixture(tmp_path / "n", tie=True, bias=False)
    with Artifact(tmp_path / "n") as a:
        assert a.dims["attention_bias"] == 0


def test_load_model_with_int16_lm_head(tmp_path):
    write_full_fixture(tmp_path, tie=True, int16_head=True)
    with Artifact(tmp_path) as a:
        assert a.dims["lm_head_int16"] == 1
        a.verify()


def test_per_channel_shifts_read_real_array(tmp_path):
    write_full_fixture(tmp_path)
    edit_json(tmp_path, "scales.json", lambda s: s["model.layers.0.input_layernorm.input"].update(shifts=[11, 12, 13, 14]))
    with Artifact(tmp_path) as a:
        assert a.layer_scales(0)[1].tolist() == [11, 12, 13, 14]


def test_rejections(tmp_path):
    def fresh(name, **kw):
        d = tmp_path / name
        write_full_fixture(d, **kw)
        return d

    # tensor content hash: checked by verify (and by the device load)
    d = fresh("badhash")
    (d / "model_norm_weight.bin").write_bytes(b"\x09\x09\x09\x09")
    with Artifact(d) as a:
        with pytest.raises(ValueError, match="SHA-256"):
            a.verify()
    # shifts file hash
    d = fresh("badshifthash")
    (d / "model_layers_0_self_attn_q_proj_bias_shifts.bin").write_bytes(bytes([2, 2, 2, 2]))
    with Artifact(d) as a:
        with pytest.raises(ValueError, match="shifts file"):
            a.verify()
    # file size against the shape
    d = fresh("badsize")
    (d / "model_norm_weight.bin").write_bytes(b"\x01\x02\x03")
    assert "bytes" in open_err(d)
    # missing manifests
    for f in ("weights_manifest.json", "scales.json", "luts.json", "model_config.json", "theta_v.json"):
        d = fresh("no_" + f.split(".")[0])
        (d / f).unlink()
        assert f in open_err(d)
    # int16 only for the LM head and biases; int16 needs a shifts file
    d = fresh("i16")
    edit_json(d, "weights_manifest.json", lambda m: m["model_norm_weight"].update(dtype="int16"))
    assert "int16 is allowed only" in open_err(d)
    d = fresh("i16noshift")
    edit_json(d, "weights_manifest.json", lambda m: m["model_layers_0_self_attn_q_proj_bias"].pop("shifts_file"))
    assert "without shifts_file" in open_err(d)
    d = fresh("dtype")
    edit_json(d, "weights_manifest.json", lambda m: m["model_norm_weight"].update(dtype="float32"))
    assert "unsupported dtype" in open_err(d)
    d = fresh("shiftrange")
    edit_json(d, "weights_manifest.json", lambda m: m["model_norm_weight"].update(shift=256))
    assert "outside 0..=255" in open_err(d)
    # LUTs
    d = fresh("luthash")
    (d / "exp.lut.bin").write_bytes(np.asarray([256, 128, 63], "<i2").tobytes())
    assert "SHA-256" in open_err(d)
    d = fresh("lutsize")
    edit_json(d, "luts.json", lambda m: m["exp"].update(length=4))
    assert "bytes" in open_err(d)
    d = fresh("lutdtype")
    edit_json(d, "luts.json", lambda m: m["exp"].update(dtype="int8"))
    assert "unsupported dtype" in open_err(d)
    # scales
    d = fresh("pow2")
    edit_json(d, "scales.json", lambda s: s["model.norm"].update(scale=0.3))
    assert "power of two" in open_err(d)
    d = fresh("scalerange")
    edit_json(d, "scales.json", lambda s: s["model.norm"].update(shift=300, scale=2.0 ** -300))
    assert "outside 0..=255" in open_err(d)
    d = fresh("pclen")
    edit_json(d, "scales.json", lambda s: s["model.norm.input"].update(shifts=[1, 2, 3]))
    assert "per-channel shifts, expected 4" in open_err(d)
    d = fresh("noscale")
    edit_json(d, "scales.json", lambda s: s.pop("model.layers.0.mlp.up_proj"))
    assert "missing calibrated activation scale" in open_err(d) and "up_proj" in open_err(d)
    # model_config.json
    d = fresh("hidden")
    edit_json(d, "model_config.json", lambda c: c.update(hidden_size=6), rehash=False)
    assert "hidden_size" in open_err(d)
    d = fresh("gqa")
    edit_json(d, "model_config.json", lambda c: c.update(num_kv_heads=3, num_heads=2), rehash=False)
    assert "multiple of num_kv_heads" in open_err(d)
    d = fresh("nobias_field")
    edit_json(d, "model_config.json", lambda c: c.pop("attention_bias"), rehash=False)
    assert "attention_bias" in open_err(d)
    d = fresh("zero")
    edit_json(d, "model_config.json", lambda c: c.update(vocab_size=0), rehash=False)
    assert "> 0" in open_err(d)
    # theta_v: version and manifest hashes
    d = fresh("version")
    write_theta_v(d, version="0.16.9")
    assert "theta_v version" in open_err(d)
    d = fresh("tamper")
    edit_json(d, "weights_manifest.json", lambda m: m["model_norm_weight"].update(scale=2.0), rehash=False)
    assert "weights hash mismatch" in open_err(d)
    d = fresh("tamper_scales")
    edit_json(d, "scales.json", lambda s: s["model.norm"].update(absmax_observed=1.0), rehash=False)
    assert "scales hash mismatch" in open_err(d)
    # build_model requirements
    d = fresh("noweight")
    edit_json(d, "weights_manifest.json", lambda m: m.pop("model_layers_0_mlp_down_proj_weight"))
    assert "missing weight" in open_err(d) and "down_proj" in open_err(d)
    d = fresh("nolmhead", tie=False)
    edit_json(d, "weights_manifest.json", lambda m: m.pop("lm_head_weight"))
    assert "lm_head.weight" in open_err(d)
    d = fresh("nobias")
    edit_json(d, "weights_manifest.json", lambda m: m.pop("model_layers_0_self_attn_k_proj_bias"))
    assert "int16 bias" in open_err(d)
    d = fresh("biaslen")

    def longer(m):
        e = m["model_layers_0_self_attn_v_proj_bias"]
        data = np.zeros(3, "<i2").tobytes()
        (d / e["file"]).write_bytes(data)
        (d / e["shifts_file"]).write_bytes(bytes(3))
        e.update(shape=[3], hash=sha(data), shifts_hash=sha(bytes(3)))
    edit_json(d, "weights_manifest.json", longer)
    assert "bias length" in open_err(d)
    d = fresh("lmshape", int16_head=True)

    def short(m):
        e = m["lm_head"]
        data = np.zeros(8, "<i2").tobytes()
        (d / e["file"]).write_bytes(data)
        (d / e["shifts_file"]).write_bytes(bytes(2))
        e.update(shape=[2, 4], hash=sha(data), shifts_hash=sha(bytes(2)))
    edit_json(d, "weights_manifest.json", short)
    assert "LM head shape" in open_err(d)
    d = fresh("wshape")
    edit_json(d, "weights_manifest.json", lambda m: m["model_layers_0_mlp_gate_proj_weight"].update(shape=[2, 8]))
    assert "does not match the model dimensions" in open_err(d)
    d = fresh("nolut")
    edit_json(d, "luts.json", lambda m: m.pop("silu"))
    assert "missing lookup table" in open_err(d) and "silu" in open_err(d)
    d = fresh("badjson")
    (d / "model_config.json").write_text('{"family": "qwen2.5",')
    assert "invalid model_config.json" in open_err(d)


def test_json_reader_accepts_escapes_and_unicode(tmp_path):
    write_full_fixture(tmp_path)
    # non-ASCII text is written as \\u escapes (and a surrogate pair) by json.dumps
    edit_json(tmp_path, "model_config.json", lambda c: c.update(variant="tëst \U0001F600 \"q\" \\ /"),
              rehash=False)
    with Artifact(tmp_path) as a:
        assert a.dims["hidden"] == 4
    (tmp_path / "model_config.json").write_text(
        (tmp_path / "model_config.json").read_text().replace(", ", ",\n\t ").replace(": ", " :  "))
    with Artifact(tmp_path) as a:
        assert a.dims["hidden"] == 4


def test_writer_output_is_a_valid_artifact(tmp_path):
    """write_artifact's directory passes every check of the reader, with the
    manifest conventions of the reference (keys, int16 lm_head key, sentinels)."""
    from myelith_amd.luts import LutSet
    rng = np.random.default_rng(3)
    dims = dict(vocab=40, hidden=16, layers=2, heads=2, kv_heads=1, head_dim=8, inter=32, max_context=64,
                tie_word_embeddings=1, attention_bias=1, lm_head_int16=1)
    from myelith_amd.artifact import model_tensors
    tensors = {}
    for name, shape, bits in model_tensors(dims):
        dt = np.int16 if bits == 16 else np.int8
        lo, hi = (-300, 300) if bits == 16 else (-127, 128)
        tensors[name] = (rng.integers(lo, hi, shape).astype(dt), rng.integers(0, 12, shape[0]).astype(np.uint8))
    ls = [(dict(norm_attn_frac=10, q_frac=9, k_frac=8, v_frac=10, attn_out_frac=11, norm_mlp_frac=10, gate_frac=10,
                up_frac=11, down_in_frac=12), rng.integers(6, 12, 16).astype(np.uint8),
           rng.integers(6, 12, 16).astype(np.uint8)) for _ in range(2)]
    fs = (9, rng.integers(6, 12, 16).astype(np.uint8))
    luts = LutSet.for_head_dim(64)
    write_artifact(tmp_path, dims, tensors, ls, fs, luts)
    man = json.loads((tmp_path / "weights_manifest.json").read_text())
    assert "lm_head" in man and man["lm_head"]["dtype"] == "int16" and man["lm_head"]["original_name"] == "lm_head.weight"
    assert man["model_layers_1_mlp_up_proj_weight"]["shape"] == [32, 16]
    with Artifact(tmp_path) as a:
        a.verify()
        assert a.dims["lm_head_int16"] == 1 and a.dims["vocab"] == 40
        for l in range(2):
            f, ri, rm = a.layer_scales(l)
            assert f == ls[l][0] and np.array_equal(ri, ls[l][1]) and np.array_equal(rm, ls[l][2])
        nf, fr = a.final_scales()
        assert nf == 9 and np.array_equal(fr, fs[1])
        for n in ("cos", "sin", "exp", "silu", "rsqrt"):
            assert np.array_equal(a.lut(n), getattr(luts, n))


@pytest.mark.skipif(not SCALE_PACK.is_dir(), reason="the reference's scale pack is not on this machine")
def test_reference_scale_pack_qwen25_05b(tmp_path):
    """The shipped scales.json / luts.json / theta_v.json of the 0.5B scale
    pack: the reader accepts them with their recorded manifest hashes (SHA-256
    of the file bytes), finds all 24 layers' scales with per-channel residual
    shifts of length 896, and its LUT tables equal this library's generator.
    Weight files are sparse stand-ins of the right sizes (content hashes are
    not checked at open)."""
    for f in ("scales.json", "luts.json", "cos.lut.bin", "sin.lut.bin", "exp.lut.bin", "silu.lut.bin",
              "rsqrt.lut.bin"):
        shutil.copy(SCALE_PACK / f, tmp_path / f)
    theta = json.loads((SCALE_PACK / "theta_v.json").read_text())
    dims = dict(vocab=151936, hidden=896, layers=24, heads=14, kv_heads=2, head_dim=64, inter=4864)
    (tmp_path / "model_config.json").write_text(json.dumps({
        "family": "qwen2.5", "variant": "0.5b", "num_layers": 24, "hidden_size": 896, "intermediate_size": 4864,
        "num_heads": 14, "num_kv_heads": 2, "head_dim": 64, "vocab_size": 151936, "max_context": 2304,
        "tie_word_embeddings": True, "attention_bias": True}))
    from myelith_amd.artifact import model_tensors
    man = {}
    for name, shape, bits in model_tensors(dict(dims, tie_word_embeddings=1, attention_bias=1, lm_head_int16=0)):
        key = name.replace(".", "_")
        with open(tmp_path / f"{key}.bin", "wb") as fh:
            fh.truncate(int(np.prod(shape)) * bits // 8)
        (tmp_path / f"{key}_shifts.bin").write_bytes(bytes(shape[0]))
        man[key] = {"original_name": name, "file": f"{key}.bin", "shape": list(shape), "scale": -1.0, "shift": -1,
                    "dtype": "int16" if bits == 16 else "int8", "hash": "0" * 64, "shifts_file": f"{key}_shifts.bin"}
    (tmp_path / "weights_manifest.json").write_text(json.dumps(man))
    theta["weights_hash"] = sha((tmp_path / "weights_manifest.json").read_bytes())
    (tmp_path / "theta_v.json").write_text(json.dumps(theta))
    assert theta["version"] == THETA_V_VERSION
    scales = json.loads((SCALE_PACK / "scales.json").read_text())
    from myelith_amd.artifact import LAYER_SCALE_KEYS, RES_IN_KEY, RES_MID_KEY
    from myelith_amd.luts import LutSet
    with Artifact(tmp_path) as a:
        for l in range(24):
            f, ri, rm = a.layer_scales(l)
            p = f"model.layers.{l}."
            assert f == {k: scales[p + v]["shift"] for k, v in LAYER_SCALE_KEYS.items()}
            assert ri.tolist() == scales[p + RES_IN_KEY]["shifts"]
            assert rm.tolist() == scales[p + RES_MID_KEY]["shifts"]
        nf, fr = a.final_scales()
        assert nf == scales["model.norm"]["shift"] and fr.tolist() == scales["model.norm.input"]["shifts"]
        mine = LutSet.for_head_dim(64)
        for n in ("cos", "sin", "exp", "silu", "rsqrt"):
            assert np.array_equal(a.lut(n), getattr(mine, n)), n

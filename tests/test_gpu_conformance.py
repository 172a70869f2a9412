"""Conformance runs on the GPU: the reference's forward op vectors through the
Backend-trait entry points, and layer / e2e vectors in the reference's format
(golden_generate.rs) exchanged between the oracle and the device model in both
directions, as golden_model.rs replays them."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from conftest import case

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_reference_op_vectors(backend):
    from myelith_amd.conformance import FORWARD_OPS, run_op
    ops = json.loads((GOLDEN / "op_vectors.json").read_text())
    case("op vectors")
    for name in FORWARD_OPS:
        r = run_op(backend, ops[name], name)
        assert r.passed is True, (name, r.detail)


def oracle_vectors(om, spec, out: Path, prompts: dict, max_new_tokens=3):
    """Layer and e2e vectors computed by the oracle, written like golden_generate.rs."""
    from myelith_amd.conformance import THETA_V_SPEC_SHA256, layer_input, tensor_json
    from myelith_amd.model import dekodieren_mit_digest
    th = "sha256:" + THETA_V_SPEC_SHA256
    (out / "layer").mkdir(parents=True)
    (out / "e2e").mkdir(parents=True)
    for l in range(spec["layers"]):
        h = layer_input(l, spec["hidden"])
        om.reset()
        y = om.run_layers(h, 0, l, l + 1)
        gv = {"name": f"transformer_layer_{l}", "level": "layer", "theta_v_hash": th,
              "metadata": {"layer_idx": l, "seq_len": 1},
              "inputs": {"hidden": tensor_json(h, "int16"), "position": tensor_json([0], "int32")},
              "outputs": {"hidden_out": tensor_json(y, "int16")}}
        (out / "layer" / f"layer_{l:02d}.golden.json").write_text(json.dumps(gv))
    for name, ids in prompts.items():
        # greedy (as golden_generate.rs:128-150 writes them) and sampled with a seed
        for suffix, greedy, seed in (("", True, 42), ("_sampled", False, 7)):
            toks, dig = dekodieren_mit_digest(om, ids, max_new_tokens, seed=seed, greedy=greedy)
            gv = {"name": f"e2e_prompt_{name}{suffix}", "level": "e2e", "theta_v_hash": th,
                  "metadata": {"max_new_tokens": max_new_tokens, "greedy": greedy, "seed": seed,
                               "logits_sha256": dig},
                  "inputs": {"prompt_tokens": tensor_json(ids, "int32")},
                  "outputs": {"tokens": tensor_json(toks, "int32")}}
            (out / "e2e" / f"e2e_{name}{suffix}.golden.json").write_text(json.dumps(gv))


def reference_prompts():
    idx = json.loads((GOLDEN / "model_vector_index.json").read_text())
    return {v["source"].rsplit("e2e_", 1)[1].split(".")[0]: v["tensors"]["inputs.prompt_tokens"]["data"]
            for v in idx.values() if v["level"] == "e2e"}


@pytest.mark.parametrize("shape", ["tiny", "qwen2.5-0.5b"])
def test_oracle_vectors_replay_on_the_device(backend, tmp_path, shape):
    from myelith_amd.conformance import run_batch
    from myelith_amd.luts import LutSet
    from myelith_amd.model import QWEN25_05B, IntegerModel, make_spec
    from oracle.binding import OracleModel
    if shape == "tiny":
        spec = dict(seed=31, vocab=1000, hidden=256, layers=3, heads=4, kv_heads=2, head_dim=64, inter=320,
                    max_pos=64, lm_head_int16=1, attention_bias=1)
        prompts = {"a": [5, 900, 17], "b": [999]}
    else:
        spec = make_spec(QWEN25_05B, seed=1234, max_pos=64)
        prompts = reference_prompts()  # the token ids of the shipped e2e vectors
    case(f"conformance replay {shape}")
    luts = LutSet.for_head_dim(spec["head_dim"])
    om = OracleModel(spec, luts, threads=16)
    oracle_vectors(om, spec, tmp_path, prompts)
    gm = IntegerModel(backend, spec, luts)
    res = run_batch(gm, tmp_path)
    assert len(res) == spec["layers"] + 2 * len(prompts)
    assert all(r.passed for r in res), [(r.name, r.detail) for r in res if not r.passed]
    # a vector whose payload was edited is refused before it is run
    p = tmp_path / "layer" / "layer_00.golden.json"
    gv = json.loads(p.read_text())
    gv["outputs"]["hidden_out"]["data"][3] += 1
    p.write_text(json.dumps(gv))
    bad = run_batch(gm, tmp_path)[0]
    assert bad.passed is False and "hash" in bad.detail
    gm.close()


def test_device_vectors_replay_on_the_oracle(backend, tmp_path):
    from myelith_amd.conformance import generate_vectors, run_batch
    from myelith_amd.luts import LutSet
    from myelith_amd.model import IntegerModel
    from oracle.binding import OracleModel
    spec = dict(seed=32, vocab=1000, hidden=512, layers=2, heads=4, kv_heads=2, head_dim=128, inter=320,
                max_pos=64, lm_head_int16=0, attention_bias=1)
    case("device-generated vectors on the oracle")
    luts = LutSet.for_head_dim(128)
    gm = IntegerModel(backend, spec, luts)
    root = generate_vectors(gm, tmp_path, {"x": [1, 2, 3, 4], "y": [777]})
    gv = json.loads((root / "layer" / "layer_01.golden.json").read_text())
    assert len(gv["metadata"]["residual_in_frac"]) == 512 and len(gv["metadata"]["out_residual_frac"]) == 512
    om = OracleModel(spec, luts, threads=16)
    res = run_batch(om, root)
    assert len(res) == 4 and all(r.passed for r in res), [(r.name, r.detail) for r in res]
    gm.close()

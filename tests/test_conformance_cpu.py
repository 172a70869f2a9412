"""The conformance runner's vector handling on the CPU: the tensor-hash
contract of golden_runner.rs:48-87, the seeded layer inputs of
golden_generate.rs:40-53 against every layer vector the reference ships
(tests/golden/model_vector_index.json), and refusals."""
from __future__ import annotations

import copy
import json
from pathlib import Path

import numpy as np

from myelith_amd.conformance import (BACKWARD_OPS, THETA_V_SPEC_SHA256, hash_mismatches, layer_input, run_op,
                                     tensor_hash, tensor_json)

GOLDEN = Path(__file__).resolve().parent / "golden"


def index():
    return json.loads((GOLDEN / "model_vector_index.json").read_text())


def test_layer_inputs_reproduce_the_reference_vectors():
    idx = index()
    layers = sorted((v for v in idx.values() if v["level"] == "layer"), key=lambda v: v["metadata"]["layer_idx"])
    assert len(layers) == 24
    for v in layers:
        l = v["metadata"]["layer_idx"]
        t = v["tensors"]["inputs.hidden"]
        h = layer_input(l, t["shape"][0])
        assert tensor_hash(h, "int16") == t["hash"], l
        assert v["tensors"]["inputs.position"]["data"] == [0]
        assert tensor_hash([0], "int32") == v["tensors"]["inputs.position"]["hash"]


def test_tensor_hash_contract_on_the_reference_vectors():
    idx = index()
    n = 0
    for v in idx.values():
        assert v["theta_v_hash"] == "sha256:" + THETA_V_SPEC_SHA256
        for t in v["tensors"].values():
            if "data" in t:
                assert tensor_hash(t["data"], t["dtype"]) == t["hash"]
                n += 1
    assert n >= 30
    ops = json.loads((GOLDEN / "op_vectors.json").read_text())
    for name, gv in ops.items():
        assert hash_mismatches(gv) == [], name
    # i8/i16/i32 packing keeps the low bits (`v as iN`)
    assert tensor_hash([-1, 255], "int8") == tensor_hash([255, -1], "int8")
    assert tensor_hash([70000], "int16") == tensor_hash([70000 - 65536], "int16")
    assert tensor_hash([1.5], "float32") is None
    e = tensor_json(np.array([3, -4], np.int16), "int16")
    assert e == {"dtype": "int16", "shape": [2], "hash": tensor_hash([3, -4], "int16"), "data": [3, -4]}


def test_tampered_vectors_and_backward_ops_are_refused():
    ops = json.loads((GOLDEN / "op_vectors.json").read_text())
    gv = copy.deepcopy(ops["softmax_basic"])
    gv["outputs"]["probs"]["data"][0] += 1
    assert hash_mismatches(gv)
    r = run_op(None, gv, "softmax_basic")
    assert r.passed is False and "hash" in r.detail
    for name in BACKWARD_OPS:
        r = run_op(None, {"name": name, "metadata": {}, "inputs": {}, "outputs": {}})
        assert r.passed is None
    assert run_op(None, {"name": "nope", "metadata": {}, "inputs": {}, "outputs": {}}).passed is False

"""Writes the reference's own golden data for this path as small fixtures.

Run once in a container that has the reference tree at /root/reference:

    python tests/golden/extract_reference_fixtures.py

It copies DATA only (inputs, expected outputs, hashes), never source:
  - the three forward op conformance vectors
    INTEGER_LLM/conformance/vectors/op/{linear_w8a16_identity,rmsnorm_basic,softmax_basic}.golden.json
    -> tests/golden/op_vectors.json (tensor data + metadata + declared SHA-256);
  - the LUT hashes of both scale packs
    INTEGER_LLM/scale_packs/qwen2.5-{0.5b,7b}/luts.json -> tests/golden/lut_hashes.json;
  - the layer and e2e conformance vectors of Qwen2.5-0.5B without their bulk
    data: each vector's name, level, metadata scalars, declared tensor hashes,
    and the small integer arrays (position, prompt and generated token ids)
    INTEGER_LLM/conformance/vectors/{layer,e2e}/*.golden.json
    -> tests/golden/model_vector_index.json.  The hidden-state payloads need
    the calibrated 0.5B weights to mean anything; their hashes pin the seeded
    layer-input generator.

The GPU machines never see /root/reference; the tests read only these files.
"""
from __future__ import annotations

import json
from pathlib import Path

REF = Path("/root/reference/INTEGER_LLM")
OUT = Path(__file__).resolve().parent

OP_VECTORS = ("linear_w8a16_identity", "rmsnorm_basic", "softmax_basic")


def main() -> None:
    ops = {}
    for name in OP_VECTORS:
        src = REF / "conformance" / "vectors" / "op" / f"{name}.golden.json"
        gv = json.loads(src.read_text())
        ops[name] = {
            "source": f"INTEGER_LLM/conformance/vectors/op/{name}.golden.json",
            "inputs": gv["inputs"],
            "outputs": gv["outputs"],
            "metadata": gv["metadata"],
            "theta_v_hash": gv["theta_v_hash"],
        }
    (OUT / "op_vectors.json").write_text(json.dumps(ops, indent=1, sort_keys=True) + "\n")

    hashes = {}
    for pack in ("qwen2.5-0.5b", "qwen2.5-7b"):
        meta = json.loads((REF / "scale_packs" / pack / "luts.json").read_text())
        hashes[pack] = {k: {"sha256": v["hash"], "length": v["length"]} for k, v in meta.items()}
    (OUT / "lut_hashes.json").write_text(json.dumps(hashes, indent=1, sort_keys=True) + "\n")
    index = {}
    for level in ("layer", "e2e"):
        for src in sorted((REF / "conformance" / "vectors" / level).glob("*.golden.json")):
            gv = json.loads(src.read_text())
            meta = {k: v for k, v in gv["metadata"].items() if not isinstance(v, list)}
            tensors = {}
            for side in ("inputs", "outputs"):
                for name, t in gv[side].items():
                    e = {"dtype": t["dtype"], "shape": t.get("shape"), "hash": t["hash"]}
                    if len(t["data"]) <= 64:
                        e["data"] = t["data"]
                    tensors[f"{side}.{name}"] = e
            index[gv["name"]] = {"source": f"INTEGER_LLM/conformance/vectors/{level}/{src.name}", "level": gv["level"],
                                 "theta_v_hash": gv["theta_v_hash"], "metadata": meta, "tensors": tensors}
    (OUT / "model_vector_index.json").write_text(json.dumps(index, indent=1, sort_keys=True) + "\n")
    print("wrote", OUT / "op_vectors.json", OUT / "lut_hashes.json", "and", OUT / "model_vector_index.json")


if __name__ == "__main__":
    main()

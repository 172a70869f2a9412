"""Writes the reference's own golden data for this path as small fixtures.

Run once in a container that has the reference tree at /root/reference:

    python tests/golden/extract_reference_fixtures.py

It copies DATA only (inputs, expected outputs, hashes), never source:
  - the three forward op conformance vectors
    INTEGER_LLM/conformance/vectors/op/{linear_w8a16_identity,rmsnorm_basic,softmax_basic}.golden.json
    -> tests/golden/op_vectors.json (tensor data + metadata + declared SHA-256);
  - the LUT hashes of both scale packs
    INTEGER_LLM/scale_packs/qwen2.5-{0.5b,7b}/luts.json -> tests/golden/lut_hashes.json.

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
    print("wrote", OUT / "op_vectors.json", "and", OUT / "lut_hashes.json")


if __name__ == "__main__":
    main()

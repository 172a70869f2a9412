"""Conformance runner: the reference's golden vectors replayed on this backend.

    python -m myelith_amd.conformance op <golden.json>...
    python -m myelith_amd.conformance model <artifact_dir> <golden.json | --batch vectors_dir>
    python -m myelith_amd.conformance generate <artifact_dir> <out_dir>

`op` follows INTEGER_LLM/kernels/src/bin/golden_runner.rs: the vector's
tensor hashes are checked first (SHA-256 over the little-endian packed
payload, golden_runner.rs:48-87), then the forward op named by the vector runs
through the Backend-trait entry points of libmyl_hip.so and must reproduce
the outputs bit for bit.  `model` follows runtime/src/bin/golden_model.rs:
layer vectors run one layer on a fresh KV cache (:183-215), e2e vectors run
generation (greedy, or sampled with the vector's seed) and compare the tokens
and the logits digest of generate.rs:98-137 (:210-268); --batch walks layer/
then e2e/ in file order
(:120-160).  `generate` writes layer and e2e vectors of a model the way
runtime/src/bin/golden_generate.rs does (seeded layer inputs, :40-95), with
prompt token ids given directly (tokenisation is not part of this backend).

Exit status: 0 all passed, 1 a failure, 2 refused (a vector this backend does
not run, e.g. the backward-pass op vectors).
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import sys
from dataclasses import dataclass
from pathlib import Path

import numpy as np

# theta_v_hash of vectors generated under theta_v 0.17.0: "sha256:" + SHA-256
# of that version's spec.json (golden_generate.rs:27, loader.rs:17-19).
THETA_V_SPEC_SHA256 = "2857db731e25dcf3018b1633c2954309658b00dcacd4b48810e0adf5a0e84609"

_PACK = {"int8": "<i1", "int16": "<i2", "int32": "<i4"}
FORWARD_OPS = ("rmsnorm_basic", "linear_w8a16_identity", "softmax_basic")
BACKWARD_OPS = ("backward_linear", "backward_softmax", "backward_rope")


@dataclass
class Result:
    name: str
    passed: bool | None  # None: refused (not run by this backend)
    detail: str = ""


def tensor_hash(data, dtype: str) -> str | None:
    """SHA-256 over the little-endian packed payload; None for dtypes the
    vector format does not pack (golden_runner.rs:48-68)."""
    if dtype not in _PACK:
        return None
    a = np.asarray(data, dtype=np.int64)
    width = {"int8": 8, "int16": 16, "int32": 32}[dtype]
    # `v as iN` of Rust: keep the low bits
    a = ((a + (1 << (width - 1))) % (1 << width)) - (1 << (width - 1))
    return hashlib.sha256(a.astype(_PACK[dtype]).tobytes()).hexdigest()


def tensor_json(data, dtype: str) -> dict:
    """A tensor entry of the vector format (golden_generate.rs:197-227)."""
    a = np.asarray(data).reshape(-1)
    return {"dtype": dtype, "shape": [int(a.size)], "hash": tensor_hash(a, dtype), "data": [int(v) for v in a]}


def hash_mismatches(gv: dict) -> list[str]:
    out = []
    for side in ("inputs", "outputs"):
        for name, t in gv.get(side, {}).items():
            h = tensor_hash(t["data"], t["dtype"])
            if h is not None and h != t["hash"]:
                out.append(f"{side[:-1]} '{name}': declared {t['hash']}, computed {h}")
    return out


def _u8(v) -> np.ndarray:
    return np.asarray(v, dtype=np.int64).astype(np.uint8)


def run_op(backend, gv: dict, name: str | None = None) -> Result:
    """One op vector (golden_runner.rs:89-258, forward ops)."""
    name = name or gv["name"]
    bad = hash_mismatches(gv)
    if bad:
        return Result(name, False, "vector hash check failed: " + "; ".join(bad))
    md, inp, outp = gv["metadata"], gv["inputs"], gv["outputs"]
    if name == "rmsnorm_basic":
        x = np.asarray(inp["x"]["data"], np.int64).astype(np.int16)
        gamma = np.asarray(inp["gamma"]["data"], np.int64).astype(np.int8)
        xs = _u8(md["x_shifts"]) if "x_shifts" in md else np.zeros(x.size, np.uint8)
        gs = _u8(md["gamma_shifts"]) if "gamma_shifts" in md else np.full(gamma.size, md["gamma_shift"], np.uint8)
        got = backend.rmsnorm(x, xs, gamma, gs, np.asarray(md["rsqrt_lut"], np.int64).astype(np.int16),
                              md["lut_input_shift"], md["lut_output_frac"], md["inv_n_q20"], md["out_frac"])
        want = np.asarray(outp["y"]["data"], np.int64).astype(np.int16)
    elif name == "linear_w8a16_identity":
        rows = md["W"]
        k = len(rows[0])
        W = np.asarray(rows, np.int64).astype(np.int8).reshape(-1)
        x = np.asarray(inp["x"]["data"], np.int64).astype(np.int16)
        ws = _u8(md["w_shifts"]) if "w_shifts" in md else np.full(len(rows), md["weight_frac"], np.uint8)
        got = backend.linear_w8a16(x, W, k, len(rows), ws, md["act_frac"], md["out_frac"])
        want = np.asarray(outp["y"]["data"], np.int64).astype(np.int16)
    elif name == "softmax_basic":
        z = np.asarray(inp["logits"]["data"], np.int64).astype(np.int32)
        if "exp_lut" in md:
            lut = np.asarray(md["exp_lut"], np.int64).astype(np.int16)
        else:  # the runner's default table (golden_runner.rs:232-239)
            lut = np.asarray([round(math.exp(-i / 256.0) * 256.0) for i in range(128)], np.int16)
        got = backend.softmax(z, lut, md["lut_shift"], md["frac_bits"])
        want = np.asarray(outp["probs"]["data"], np.int64).astype(np.int32)
    elif name in BACKWARD_OPS:
        return Result(name, None, "the backward pass is not part of this backend (forward path only)")
    else:
        return Result(name, False, "unknown golden vector")
    if not np.array_equal(got, want):
        return Result(name, False, f"expected {want.tolist()}, got {np.asarray(got).tolist()}")
    return Result(name, True)


def validate_layer(model, gv: dict) -> Result:
    """golden_model.rs:183-215: one layer at position 0 on a fresh cache."""
    layer = int(gv["metadata"]["layer_idx"])
    hidden = np.asarray(gv["inputs"]["hidden"]["data"], np.int64).astype(np.int16)
    model.reset()
    out = model.run_layers(hidden, 0, layer, layer + 1)
    want = np.asarray(gv["outputs"]["hidden_out"]["data"], np.int64).astype(np.int16)
    if out.size != want.size:
        return Result(gv["name"], False, f"length {out.size} vs {want.size}")
    bad = np.flatnonzero(out != want)
    if bad.size:
        first = [(int(i), int(out[i]), int(want[i])) for i in bad[:5]]
        return Result(gv["name"], False, f"{bad.size} mismatches in layer {layer} (first: {first})")
    return Result(gv["name"], True)


def validate_e2e(model, gv: dict) -> Result:
    """golden_model.rs:210-268: the generated tokens and the logits digest,
    greedy or sampled with the vector's seed (defaults true and 42 as there)."""
    from .model import dekodieren_mit_digest
    md = gv["metadata"]
    greedy = bool(md.get("greedy", True))
    seed = int(md.get("seed", 42))
    prompt = [int(t) for t in gv["inputs"]["prompt_tokens"]["data"]]
    toks, digest = dekodieren_mit_digest(model, prompt, int(md["max_new_tokens"]), seed=seed, greedy=greedy)
    want = [int(t) for t in gv["outputs"]["tokens"]["data"]]
    if toks != want:
        return Result(gv["name"], False, f"token mismatch: generated {toks}, expected {want}")
    exp = md.get("logits_sha256")
    if not isinstance(exp, str):
        return Result(gv["name"], False, "the vector carries no metadata.logits_sha256 and checks tokens only")
    if digest != exp:
        return Result(gv["name"], False, f"logits digest {digest}, expected {exp} (tokens agree)")
    return Result(gv["name"], True)


def validate(model, gv: dict) -> Result:
    bad = hash_mismatches(gv)
    if bad:
        return Result(gv["name"], False, "vector hash check failed: " + "; ".join(bad))
    if gv["level"] == "layer":
        return validate_layer(model, gv)
    if gv["level"] == "e2e":
        return validate_e2e(model, gv)
    return Result(gv["name"], False, f"unknown level {gv['level']}")


def run_batch(model, vectors_dir) -> list[Result]:
    out = []
    for level in ("layer", "e2e"):
        d = Path(vectors_dir) / level
        if d.is_dir():
            for p in sorted(d.glob("*.golden.json")):
                out.append(validate(model, json.loads(p.read_text())))
    return out


def layer_input(layer_idx: int, hidden: int) -> np.ndarray:
    """The seeded hidden state of a layer vector (golden_generate.rs:44-53):
    splitmix64 from seed layer * 0x9E3779B97F4A7C15 + 1, each value the
    wrapping i16 sum of bits 63..48 and 47..32 of one output."""
    M = (1 << 64) - 1
    state = (layer_idx * 0x9E3779B97F4A7C15 + 1) & M
    out = np.zeros(hidden, np.int16)
    for i in range(hidden):
        state = (state + 0x9E3779B97F4A7C15) & M
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        z ^= z >> 31
        v = ((z >> 48) & 0xFFFF) + ((z >> 32) & 0xFFFF)
        out[i] = np.int16(np.uint16(v & 0xFFFF).view(np.int16))
    return out


def generate_vectors(model, out_dir, prompts: dict, max_new_tokens: int = 3, seed: int = 42) -> Path:
    """Layer vectors for every layer and e2e vectors for `prompts`
    ({name: token ids}) in the reference's format (golden_generate.rs)."""
    from .model import dekodieren_mit_digest
    root = Path(out_dir) / "vectors"
    (root / "layer").mkdir(parents=True, exist_ok=True)
    (root / "e2e").mkdir(parents=True, exist_ok=True)
    th = "sha256:" + THETA_V_SPEC_SHA256
    L = model.num_layers
    for l in range(L):
        h = layer_input(l, model.hidden_size)
        model.reset()
        out = model.run_layers(h, 0, l, l + 1)
        fr, ri, _ = model.layer_scales(l)
        out_frac = model.layer_scales(l + 1)[1] if l + 1 < L else model.final_scales()[1]
        gv = {"name": f"transformer_layer_{l}", "level": "layer", "theta_v_hash": th,
              "metadata": {"layer_idx": l, "seq_len": 1, "residual_in_frac": [int(x) for x in ri],
                           "out_residual_frac": [int(x) for x in out_frac]},
              "inputs": {"hidden": tensor_json(h, "int16"), "position": tensor_json([0], "int32")},
              "outputs": {"hidden_out": tensor_json(out, "int16")}}
        (root / "layer" / f"layer_{l:02d}.golden.json").write_text(json.dumps(gv))
    for name, ids in prompts.items():
        toks, digest = dekodieren_mit_digest(model, [int(t) for t in ids], max_new_tokens)
        gv = {"name": f"e2e_prompt_{name}", "level": "e2e", "theta_v_hash": th,
              "metadata": {"max_new_tokens": max_new_tokens, "greedy": True, "seed": seed, "logits_sha256": digest},
              "inputs": {"prompt_tokens": tensor_json(ids, "int32")},
              "outputs": {"tokens": tensor_json(toks, "int32")}}
        (root / "e2e" / f"e2e_{name}.golden.json").write_text(json.dumps(gv))
    return root


def _report(results: list[Result]) -> int:
    for r in results:
        tag = "PASS" if r.passed else ("REFUSED" if r.passed is None else "FAIL")
        print(f"{tag}: {r.name}" + (f"  ({r.detail})" if r.detail else ""))
    n_pass = sum(1 for r in results if r.passed)
    print(f"\n{n_pass} of {len(results)} passed")
    if any(r.passed is False for r in results):
        return 1
    if any(r.passed is None for r in results):
        return 2
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m myelith_amd.conformance")
    sub = ap.add_subparsers(dest="cmd", required=True)
    p_op = sub.add_parser("op")
    p_op.add_argument("vectors", nargs="+")
    p_model = sub.add_parser("model")
    p_model.add_argument("artifact")
    p_model.add_argument("vector", nargs="?")
    p_model.add_argument("--batch")
    p_model.add_argument("--max-pos", type=int, default=0)
    p_gen = sub.add_parser("generate")
    p_gen.add_argument("artifact")
    p_gen.add_argument("out")
    p_gen.add_argument("--prompt", action="append", default=[], help="name=id,id,... (token ids)")
    p_gen.add_argument("--max-new-tokens", type=int, default=3)
    args = ap.parse_args(argv)

    from .backend import RocmBackend
    backend = RocmBackend(0)
    if args.cmd == "op":
        return _report([run_op(backend, json.loads(Path(v).read_text())) for v in args.vectors])
    from .model import IntegerModel
    model = IntegerModel.from_artifact(backend, args.artifact, args.max_pos)
    if args.cmd == "model":
        if args.batch:
            return _report(run_batch(model, args.batch))
        if not args.vector:
            ap.error("model: a vector file or --batch <dir>")
        return _report([validate(model, json.loads(Path(args.vector).read_text()))])
    prompts = {}
    for spec in args.prompt or ["hello=9707"]:
        name, ids = spec.split("=", 1)
        prompts[name] = [int(t) for t in ids.split(",")]
    root = generate_vectors(model, args.out, prompts, args.max_new_tokens)
    print(f"wrote {root}")
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Artifact directories in the reference's model format.

An artifact (INTEGER_LLM/runtime/src/loader.rs:322-600) is a directory with
  theta_v.json           version + SHA-256 of the three manifests (loader.rs:33-87)
  model_config.json      ModelDims (loader.rs:240-304)
  weights_manifest.json  one entry per tensor: original_name, file, shape,
                         scale, shift, dtype, hash, shifts_file, shifts_hash
                         (loader.rs:89-107); raw little-endian data files
  scales.json            activation scales: shift, scale = 2^-shift,
                         absmax_observed, per-channel `shifts` for the three
                         residual segments (loader.rs:196-236)
  luts.json              the five int16 tables and their *.lut.bin files
                         (loader.rs:172-178, 496-545)

Reading is the library's (libmyl_hip.so: myl_artifact_open / myl_model_load_artifact,
with every check of load_model); `Artifact` wraps it.  `write_artifact` writes
the same format from host arrays, and `export_model` writes a device model's
tensors, so a synthetic model here can be loaded by the reference's loader on a
machine that builds it.
"""
from __future__ import annotations

import ctypes as C
import json
import os
from pathlib import Path

import numpy as np

from ._lib import LayerFracs, ModelDims, lib

THETA_V_VERSION = "0.17.0"  # MYL_TV_VERSION (include/myl_theta_v.h)
LUT_NAMES = ("cos", "exp", "rsqrt", "silu", "sin")

# LayerScales field -> scales.json module suffix (loader.rs:784-797).
LAYER_SCALE_KEYS = {
    "norm_attn_frac": "input_layernorm",
    "q_frac": "self_attn.q_proj",
    "k_frac": "self_attn.k_proj",
    "v_frac": "self_attn.v_proj",
    "attn_out_frac": "self_attn",
    "norm_mlp_frac": "post_attention_layernorm",
    "gate_frac": "mlp.gate_proj",
    "up_frac": "mlp.up_proj",
    "down_in_frac": "mlp.down_proj.input",
}
RES_IN_KEY = "input_layernorm.input"            # per-channel residual segment entering layer l
RES_MID_KEY = "post_attention_layernorm.input"  # after the attention residual


def sha256_hex(data: bytes) -> str:
    """SHA-256 as lowercase hex (loader.rs:600-605), computed by the library."""
    out = C.create_string_buffer(65)
    buf = C.create_string_buffer(bytes(data), len(data)) if data else None
    rc = lib().myl_sha256_hex(buf, len(data), out)
    if rc != 0:
        raise ValueError("sha256")
    return out.value.decode()


class Artifact:
    """An opened and checked artifact directory (myl_artifact_open)."""

    def __init__(self, path):
        self.path = Path(path)
        h = C.c_void_p()
        err = C.create_string_buffer(1024)
        rc = lib().myl_artifact_open(str(self.path).encode(), C.byref(h), err, len(err))
        if rc != 0:
            raise ValueError(f"artifact {self.path}: {err.value.decode()}")
        self._h = h
        d = ModelDims()
        lib().myl_artifact_dims(self._h, C.byref(d))
        self.dims = {k: int(getattr(d, k)) for k, _ in ModelDims._fields_}

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().myl_artifact_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int, what: str) -> None:
        if rc != 0:
            raise ValueError(f"{what}: {lib().myl_artifact_last_error(self._h).decode()}")

    def verify(self) -> None:
        """Hashes every tensor and shifts file of the manifest (loader.rs:364-399)."""
        self._check(lib().myl_artifact_verify(self._h), "verify")

    def lut(self, name: str) -> np.ndarray:
        n = C.c_size_t()
        self._check(lib().myl_artifact_lut(self._h, name.encode(), None, 0, C.byref(n)), f"lut {name}")
        out = np.zeros(n.value, np.int16)
        self._check(lib().myl_artifact_lut(self._h, name.encode(), out.ctypes.data, out.size, C.byref(n)),
                    f"lut {name}")
        return out

    def layer_scales(self, layer: int):
        f = LayerFracs()
        H = self.dims["hidden"]
        ri = np.zeros(H, np.uint8)
        rm = np.zeros(H, np.uint8)
        self._check(lib().myl_artifact_layer_scales(self._h, layer, C.byref(f), ri.ctypes.data, rm.ctypes.data),
                    "layer_scales")
        return {k: int(getattr(f, k)) for k, _ in LayerFracs._fields_}, ri, rm

    def final_scales(self):
        nf = C.c_uint8()
        fr = np.zeros(self.dims["hidden"], np.uint8)
        self._check(lib().myl_artifact_final_scales(self._h, C.byref(nf), fr.ctypes.data), "final_scales")
        return int(nf.value), fr


def model_tensors(dims: dict) -> list[tuple[str, tuple, int]]:
    """(HF name, shape, bits) of every tensor an IntegerModel of `dims` reads
    (loader.rs:728-812)."""
    H, I, V = dims["hidden"], dims["inter"], dims["vocab"]
    nq, nkv = dims["heads"] * dims["head_dim"], dims["kv_heads"] * dims["head_dim"]
    out = [("model.embed_tokens.weight", (V, H), 8), ("model.norm.weight", (H,), 8)]
    if dims.get("lm_head_int16"):
        out.append(("lm_head.weight", (V, H), 16))
    elif not dims.get("tie_word_embeddings", 1):
        out.append(("lm_head.weight", (V, H), 8))
    for l in range(dims["layers"]):
        p = f"model.layers.{l}."
        out += [(p + "input_layernorm.weight", (H,), 8), (p + "post_attention_layernorm.weight", (H,), 8),
                (p + "self_attn.q_proj.weight", (nq, H), 8), (p + "self_attn.k_proj.weight", (nkv, H), 8),
                (p + "self_attn.v_proj.weight", (nkv, H), 8), (p + "self_attn.o_proj.weight", (H, nq), 8),
                (p + "mlp.gate_proj.weight", (I, H), 8), (p + "mlp.up_proj.weight", (I, H), 8),
                (p + "mlp.down_proj.weight", (H, I), 8)]
        if dims.get("attention_bias"):
            out += [(p + "self_attn.q_proj.bias", (nq,), 16), (p + "self_attn.k_proj.bias", (nkv,), 16),
                    (p + "self_attn.v_proj.bias", (nkv,), 16)]
    return out


def _scale_entry(shift: int, shifts=None) -> dict:
    e = {"absmax_observed": 32767.0 * 2.0 ** -shift, "scale": 2.0 ** -shift, "shift": int(shift)}
    if shifts is not None:
        e["shifts"] = [int(x) for x in shifts]
    return e


def _write(path: Path, data: bytes) -> str:
    path.write_bytes(data)
    return sha256_hex(data)


def write_artifact(path, dims: dict, tensors: dict, layer_scales: list, final_scales: tuple, luts,
                   family: str = "qwen2.5", variant: str = "synthetic") -> Path:
    """Writes an artifact directory.

    tensors       {HF name: (array int8 or int16, per-row u8 shifts)}; an int16
                  lm_head.weight is stored under the manifest key "lm_head"
                  (loader.rs:331-339), every other key is the name with dots
                  replaced by underscores (loader.rs:163-170)
    layer_scales  per layer (LayerScales dict, res_in [H], res_mid [H])
    final_scales  (model.norm frac, model.norm.input [H])
    luts          an object with rsqrt/silu/exp/cos/sin int16 arrays
    """
    out = Path(path)
    out.mkdir(parents=True, exist_ok=True)
    manifest = {}
    for name, (data, shifts) in tensors.items():
        a = np.ascontiguousarray(data)
        bits = 16 if a.dtype == np.int16 else 8
        key = "lm_head" if (name == "lm_head.weight" and bits == 16) else name.replace(".", "_")
        raw = a.astype("<i2" if bits == 16 else np.int8, copy=False).tobytes()
        sh = np.ascontiguousarray(shifts, dtype=np.uint8)
        assert sh.size == a.shape[0], name
        manifest[key] = {
            "original_name": name, "file": key + ".bin", "shape": [int(x) for x in a.shape],
            "scale": -1.0, "shift": -1, "dtype": "int16" if bits == 16 else "int8",
            "hash": _write(out / (key + ".bin"), raw),
            "shifts_file": key + "_shifts.bin", "shifts_hash": _write(out / (key + "_shifts.bin"), sh.tobytes()),
        }
    scales = {}
    for l, (fr, res_in, res_mid) in enumerate(layer_scales):
        p = f"model.layers.{l}."
        for field, sfx in LAYER_SCALE_KEYS.items():
            scales[p + sfx] = _scale_entry(fr[field])
        scales[p + RES_IN_KEY] = _scale_entry(int(np.min(res_in)), res_in)
        scales[p + RES_MID_KEY] = _scale_entry(int(np.min(res_mid)), res_mid)
    nf, final_res = final_scales
    scales["model.norm"] = _scale_entry(nf)
    scales["model.norm.input"] = _scale_entry(int(np.min(final_res)), final_res)
    lut_manifest = {}
    for n in LUT_NAMES:
        t = np.ascontiguousarray(getattr(luts, n), dtype="<i2")
        lut_manifest[n] = {"dtype": "int16", "file": f"{n}.lut.bin", "hash": _write(out / f"{n}.lut.bin", t.tobytes()),
                           "length": int(t.size)}
    config = {"family": family, "variant": variant, "num_layers": dims["layers"], "hidden_size": dims["hidden"],
              "intermediate_size": dims["inter"], "num_heads": dims["heads"], "num_kv_heads": dims["kv_heads"],
              "head_dim": dims["head_dim"], "vocab_size": dims["vocab"],
              "max_context": int(dims.get("max_context") or dims.get("max_pos") or 0),
              "tie_word_embeddings": bool(dims.get("tie_word_embeddings", 1)),
              "attention_bias": bool(dims.get("attention_bias", 1))}
    (out / "model_config.json").write_text(json.dumps(config, sort_keys=True))
    hashes = {}
    for fname, obj in (("weights_manifest.json", manifest), ("scales.json", scales), ("luts.json", lut_manifest)):
        hashes[fname] = _write(out / fname, json.dumps(obj, sort_keys=True).encode())
    theta = {"version": THETA_V_VERSION, "weights_hash": hashes["weights_manifest.json"],
             "scales_hash": hashes["scales.json"], "luts_hash": hashes["luts.json"]}
    (out / "theta_v.json").write_text(json.dumps(theta, sort_keys=True))
    return out


def export_model(model, path, family: str = "qwen2.5", variant: str = "synthetic") -> Path:
    """Writes a device IntegerModel (myelith_amd.model) as an artifact."""
    dims = dict(model.spec)
    dims.setdefault("tie_word_embeddings", int(model.tied))
    dims["max_context"] = dims.get("max_context") or dims["max_pos"]
    tensors = {}
    for name, shape, bits in model_tensors(dims):
        tensors[name] = model.download_tensor(name, shape, bits)
    layer_scales = [model.layer_scales(l) for l in range(dims["layers"])]
    return write_artifact(path, dims, tensors, layer_scales, model.final_scales(), model.luts, family, variant)


def load_model(backend, path, max_pos: int = 0):
    """load_model (loader.rs:611-636) onto the device."""
    from .model import IntegerModel
    return IntegerModel.from_artifact(backend, os.fspath(path), max_pos)

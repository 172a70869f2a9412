"""IntegerModel on the GPU: the host mirror of INTEGER_LLM/runtime/src/model.rs.

`IntegerModel` wraps a device-resident model of libmyl_hip.so (weights in HBM,
KV cache in HBM) and keeps the reference's method names: forward_token
(model.rs:229-311), embed_token (:323-331), run_layers (:339-356),
head_logits (:360-399), greedy_next (:780-782).  `dekodieren_mit_digest`
reproduces runtime/src/generate.rs:98-137 (the SHA-256 logits digest that is
the parity contract between machines).

Models are the seeded synthetic models of include/myl_synth.h: real
checkpoints are not available where this runs.
"""
from __future__ import annotations

import ctypes as C
import hashlib

import numpy as np

from ._lib import LayerFracs, Luts, ModelDims, SynthSpec, lib
from .backend import RocmBackend
from .luts import LutSet

# Architectures of the benchmark workloads (the Qwen2.5-0.5B and Qwen2.5-7B layouts).
QWEN25_05B = dict(vocab=151936, hidden=896, layers=24, heads=14, kv_heads=2, head_dim=64, inter=4864,
                  lm_head_int16=0, attention_bias=1)
QWEN25_7B = dict(vocab=152064, hidden=3584, layers=28, heads=28, kv_heads=4, head_dim=128, inter=18944,
                 lm_head_int16=1, attention_bias=1)


def make_spec(arch: dict, seed: int, max_pos: int, **over) -> dict:
    spec = dict(arch)
    spec.update(seed=seed, max_pos=max_pos)
    spec.update(over)
    return spec


def luts_struct(luts: LutSet) -> tuple[Luts, tuple]:
    arrs = tuple(np.ascontiguousarray(a, dtype=np.int16) for a in (luts.rsqrt, luts.silu, luts.exp, luts.cos, luts.sin))
    s = Luts(arrs[0].ctypes.data, arrs[0].size, arrs[1].ctypes.data, arrs[1].size, arrs[2].ctypes.data, arrs[2].size,
             arrs[3].ctypes.data, arrs[4].ctypes.data, arrs[3].size)
    return s, arrs


class IntegerModel:
    """model.rs:120-163, device-resident."""

    def __init__(self, backend: RocmBackend, spec: dict, luts: LutSet | None = None, _handle=None):
        """The seeded synthetic model of `spec` (include/myl_synth.h); the
        classmethods `create` and `from_artifact` build the other kinds."""
        self.backend = backend
        self.spec = dict(spec)
        self.luts = luts or LutSet.for_head_dim(spec["head_dim"])
        if _handle is None:
            cspec = SynthSpec(**{k: int(spec[k]) for k, _ in SynthSpec._fields_})
            cl, keep = luts_struct(self.luts)
            _handle = C.c_void_p()
            backend.check(lib().myl_model_create_synthetic(backend.handle, C.byref(cspec), C.byref(cl),
                                                           C.byref(_handle)), "model_create_synthetic")
        self._h = _handle
        backend.adopt(self)
        self.vocab_size = spec["vocab"]
        self.hidden_size = spec["hidden"]
        self.num_layers = spec["layers"]
        self.num_kv_heads = spec["kv_heads"]
        self.head_dim = spec["head_dim"]
        self.tied = bool(spec.get("tie_word_embeddings", True))

    @classmethod
    def create(cls, backend: RocmBackend, dims: dict, max_pos: int, luts: LutSet | None = None) -> "IntegerModel":
        """An empty model of `dims` (ModelDims keys of _lib.ModelDims) to be
        filled by upload_tensor / set_*_scales and sealed by finalize()."""
        luts = luts or LutSet.for_head_dim(dims["head_dim"])
        cd = ModelDims(**{k: int(dims.get(k, 0)) for k, _ in ModelDims._fields_})
        cl, keep = luts_struct(luts)
        h = C.c_void_p()
        backend.check(lib().myl_model_create(backend.handle, C.byref(cd), max_pos, C.byref(cl), C.byref(h)),
                      "model_create")
        spec = {k: int(getattr(cd, k)) for k, _ in ModelDims._fields_}
        spec["max_pos"] = max_pos or spec["max_context"]
        return cls(backend, spec, luts, _handle=h)

    @classmethod
    def from_artifact(cls, backend: RocmBackend, artifact, max_pos: int = 0) -> "IntegerModel":
        """load_model (loader.rs:611-636): the model of an artifact directory
        (a path or an opened myelith_amd.artifact.Artifact) streamed to HBM."""
        from .artifact import Artifact
        art = artifact if isinstance(artifact, Artifact) else Artifact(artifact)
        try:
            h = C.c_void_p()
            backend.check(lib().myl_model_load_artifact(backend.handle, art.handle, max_pos, C.byref(h)),
                          "model_load_artifact")
            spec = dict(art.dims)
            spec["max_pos"] = max_pos or spec["max_context"]
            luts = LutSet.from_tables(spec["head_dim"], **{n: art.lut(n) for n in ("rsqrt", "silu", "exp", "cos", "sin")})
            return cls(backend, spec, luts, _handle=h)
        finally:
            if art is not artifact:
                art.close()

    # ---- tensors and scales in the reference layout ----

    def upload_tensor(self, name: str, data, shifts) -> None:
        """One tensor by its HF name (include/myl_hip.h, myl_model_upload_tensor);
        int16 data selects the 16-bit form (the int16 LM head, biases)."""
        a = np.ascontiguousarray(data)
        bits = 16 if a.dtype == np.int16 else 8
        if bits == 8:
            a = a.astype(np.int8, copy=False)
        sh = np.ascontiguousarray(shifts, dtype=np.uint8)
        shape = (C.c_uint64 * a.ndim)(*a.shape)
        self._check(lib().myl_model_upload_tensor(self._h, name.encode(), a.ctypes.data, bits, shape, a.ndim,
                                                  sh.ctypes.data, sh.size), f"upload {name}")

    def download_tensor(self, name: str, shape, bits: int = 8):
        """The tensor `name` in the reference layout and its per-row shifts."""
        a = np.zeros(shape, np.int16 if bits == 16 else np.int8)
        sh = np.zeros(a.shape[0], np.uint8)
        self._check(lib().myl_model_download_tensor(self._h, name.encode(), bits, a.ctypes.data, a.nbytes,
                                                    sh.ctypes.data, sh.size), f"download {name}")
        return a, sh

    def set_layer_scales(self, layer: int, fracs: dict, res_in, res_mid) -> None:
        f = LayerFracs(**{k: int(fracs[k]) for k, _ in LayerFracs._fields_})
        ri = np.ascontiguousarray(res_in, dtype=np.uint8)
        rm = np.ascontiguousarray(res_mid, dtype=np.uint8)
        assert ri.size == self.hidden_size and rm.size == self.hidden_size
        self._check(lib().myl_model_set_layer_scales(self._h, layer, C.byref(f), ri.ctypes.data, rm.ctypes.data),
                    "set_layer_scales")

    def set_final_scales(self, final_norm_frac: int, final_res) -> None:
        fr = np.ascontiguousarray(final_res, dtype=np.uint8)
        assert fr.size == self.hidden_size
        self._check(lib().myl_model_set_final_scales(self._h, final_norm_frac, fr.ctypes.data), "set_final_scales")

    def layer_scales(self, layer: int):
        f = LayerFracs()
        ri = np.zeros(self.hidden_size, np.uint8)
        rm = np.zeros(self.hidden_size, np.uint8)
        self._check(lib().myl_model_get_layer_scales(self._h, layer, C.byref(f), ri.ctypes.data, rm.ctypes.data),
                    "layer_scales")
        return {k: int(getattr(f, k)) for k, _ in LayerFracs._fields_}, ri, rm

    def final_scales(self):
        nf = C.c_uint8()
        fr = np.zeros(self.hidden_size, np.uint8)
        self._check(lib().myl_model_get_final_scales(self._h, C.byref(nf), fr.ctypes.data), "final_scales")
        return int(nf.value), fr

    def finalize(self) -> None:
        self._check(lib().myl_model_finalize(self._h), "finalize")

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().myl_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        self.backend.check(rc, what)

    def reset(self) -> None:
        """A fresh KV cache (KVCache::new, kv_cache.rs:14-16)."""
        self._check(lib().myl_model_reset(self._h), "reset")

    def forward_token(self, token_id: int, pos: int, want_logits: bool = True):
        logits = np.zeros(self.vocab_size, np.int32) if want_logits else None
        am = C.c_int64()
        self._check(lib().myl_model_forward_token(self._h, token_id, pos,
                                                  None if logits is None else logits.ctypes.data, C.byref(am)),
                    "forward_token")
        self.last_argmax = am.value
        return logits

    def decode_greedy(self, token: int, pos: int, n_steps: int, want_logits: bool = False):
        """n_steps forward passes, each feeding its argmax to the next on the device."""
        toks = np.zeros(n_steps, np.int64)
        logits = np.zeros((n_steps, self.vocab_size), np.int32) if want_logits else None
        self._check(lib().myl_model_decode_greedy(self._h, token, pos, n_steps, toks.ctypes.data,
                                                  None if logits is None else logits.ctypes.data), "decode_greedy")
        return toks, logits

    def prefill(self, token_ids, pos0: int = 0, want_logits: bool = True):
        """The prompt loop of generate.rs:28-32 in one call; returns the last logits."""
        toks = np.ascontiguousarray(token_ids, dtype=np.uint32)
        logits = np.zeros(self.vocab_size, np.int32) if want_logits else None
        self._check(lib().myl_model_prefill(self._h, toks.ctypes.data, toks.size, pos0,
                                            None if logits is None else logits.ctypes.data), "prefill")
        return logits

    def set_graphs(self, enable: bool) -> None:
        self._check(lib().myl_model_set_graphs(self._h, int(enable)), "set_graphs")

    KERNEL_CLASSES = ("embed", "rmsnorm", "qkv", "attention", "o_proj", "gate_up", "down", "lm_head")

    def set_kernel_repeat(self, kclass: str, times: int) -> None:
        """Launches the kernel class `times` times per layer and decode step
        (a measurement hook; only "gate_up": each repeat streams the next
        layers' weights into scratch rows, so every output is unchanged).  The
        next greedy decode recaptures its step graph."""
        self._check(lib().myl_model_set_kernel_repeat(self._h, self.KERNEL_CLASSES.index(kclass), int(times)),
                    "set_kernel_repeat")

    def timing(self, enable: bool):
        """Starts (True) or stops (False) per-kernel-class HIP event timing.
        Stopping returns {class: (total_ms, launches)}."""
        ms = np.zeros(8, np.float64)
        n = np.zeros(8, np.uint64)
        self._check(lib().myl_model_timing(self._h, int(enable), ms.ctypes.data, n.ctypes.data), "timing")
        if enable:
            return None
        return {k: (float(ms[i]), int(n[i])) for i, k in enumerate(self.KERNEL_CLASSES)}

    def embed_token(self, token_id: int) -> np.ndarray:
        h = np.zeros(self.hidden_size, np.int16)
        self._check(lib().myl_model_embed_token(self._h, token_id, h.ctypes.data), "embed_token")
        return h

    def run_layers(self, hidden, pos: int, layer_start: int, layer_end: int) -> np.ndarray:
        h = np.ascontiguousarray(hidden, dtype=np.int16).copy()
        self._check(lib().myl_model_run_layers(self._h, h.ctypes.data, pos, layer_start, layer_end), "run_layers")
        return h

    def head_logits(self, hidden) -> np.ndarray:
        h = np.ascontiguousarray(hidden, dtype=np.int16)
        out = np.zeros(self.vocab_size, np.int32)
        self._check(lib().myl_model_head_logits(self._h, h.ctypes.data, out.ctypes.data), "head_logits")
        return out

    def read_kv(self, layer: int, kv_head: int, n_pos: int):
        k = np.zeros((n_pos, self.head_dim), np.int16)
        v = np.zeros((n_pos, self.head_dim), np.int16)
        self._check(lib().myl_model_read_kv(self._h, layer, kv_head, n_pos, k.ctypes.data, v.ctypes.data), "read_kv")
        return k, v

    def read_tensor(self, name: str, layer: int, nbytes: int, dtype=np.int8) -> np.ndarray:
        buf = np.zeros(nbytes, np.uint8)
        self._check(lib().myl_model_read_tensor(self._h, name.encode(), layer, buf.ctypes.data, nbytes), "read_tensor")
        return buf.view(dtype)

    # ---- batched forward (many sequences, each with its own KV cache) ----

    def batch_begin(self, n_seqs: int) -> None:
        """KV caches for n_seqs sequences, all empty."""
        self._check(lib().myl_model_batch_begin(self._h, n_seqs), "batch_begin")
        self.n_seqs = n_seqs

    def forward_batch(self, seq, pos, tokens, want_logits: bool = True):
        """Rows (seq[r], pos[r], tokens[r]); row r equals forward_token(tokens[r], pos[r])
        on sequence seq[r].  Returns (logits [R x vocab] or None, argmax [R])."""
        s = np.ascontiguousarray(seq, dtype=np.uint32)
        p = np.ascontiguousarray(pos, dtype=np.uint32)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        R = s.size
        assert p.size == R and t.size == R
        logits = np.zeros((R, self.vocab_size), np.int32) if want_logits else None
        am = np.zeros(R, np.int64)
        self._check(lib().myl_model_forward_batch(self._h, R, s.ctypes.data, p.ctypes.data, t.ctypes.data,
                                                  None if logits is None else logits.ctypes.data, am.ctypes.data),
                    "forward_batch")
        return logits, am

    def batch_logits_dev(self, rows: int):
        """The last batch's logits as a torch view on the device (no copy)."""
        import torch
        ptr = C.c_void_p()
        self._check(lib().myl_model_batch_logits_dev(self._h, C.byref(ptr)), "batch_logits_dev")
        return _device_view_i32(ptr.value, rows, self.vocab_size)

    def batch_decode_greedy(self, seq, pos, tokens, n_steps: int):
        """Lock-step greedy decode of len(seq) sequences; returns [n_steps x rows] argmax tokens."""
        s = np.ascontiguousarray(seq, dtype=np.uint32)
        p = np.ascontiguousarray(pos, dtype=np.uint32)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.zeros((n_steps, s.size), np.int64)
        self._check(lib().myl_model_batch_decode_greedy(self._h, s.size, s.ctypes.data, p.ctypes.data, t.ctypes.data,
                                                        n_steps, out.ctypes.data), "batch_decode_greedy")
        return out

    def batch_read_kv(self, seq: int, layer: int, kv_head: int, n_pos: int):
        k = np.zeros((n_pos, self.head_dim), np.int16)
        v = np.zeros((n_pos, self.head_dim), np.int16)
        self._check(lib().myl_model_batch_read_kv(self._h, seq, layer, kv_head, n_pos, k.ctypes.data, v.ctypes.data),
                    "batch_read_kv")
        return k, v

    @staticmethod
    def greedy_next(logits) -> int:
        """argmax_int (sampling.rs:8-18): the first maximum wins."""
        return int(np.argmax(np.asarray(logits)))

    def sample_next(self, logits, state: int):
        """sample_integer_cdf (sampling.rs:27-46) on the GPU: (token, new_state)."""
        return self.backend.sample_integer_cdf(logits, state)


def _device_view_i32(ptr: int, rows: int, cols: int):
    """A torch int32 tensor over device memory owned by the library."""
    import torch

    class _Arr:
        __cuda_array_interface__ = {"shape": (rows, cols), "typestr": "<i4", "data": (ptr, False), "version": 3,
                                    "strides": None}
    return torch.as_tensor(_Arr(), device="cuda")


def dekodieren_mit_digest(model, token_ids, max_new_tokens: int, seed: int = 0, greedy: bool = True):
    """generate.rs:98-137: prefill the prompt, then for each decode step hash
    all logits as i32 LE followed by the chosen token as u32 LE.  The token is
    the first maximum (greedy_next, model.rs:780-782) or, with greedy False,
    model.sample_next(logits, state) (model.rs:785-787), the state starting at
    seed and carried from step to step.

    Works with any object exposing forward_token(token, pos), reset() and,
    for sampling, sample_next(logits, state)."""
    model.reset()
    pos = 0
    logits = None
    for tid in token_ids:
        logits = model.forward_token(int(tid), pos)
        pos += 1
    h = hashlib.sha256()
    out = []
    state = int(seed) & (2**64 - 1)
    for _ in range(max_new_tokens):
        h.update(np.ascontiguousarray(logits, dtype="<i4").tobytes())
        if greedy:
            nxt = int(np.argmax(logits))
        else:
            nxt, state = model.sample_next(logits, state)
        h.update(np.uint32(nxt).astype("<u4").tobytes())
        out.append(nxt)
        logits = model.forward_token(nxt, pos)
        pos += 1
    return out, h.hexdigest()

"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker that the HIP path is compared against.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    """Compiles liboracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    """The oracle library; MYL_ORACLE_LIB names another build of oracle.c
    (the mutation test runs the pins against deliberately broken copies)."""
    global _lib
    if _lib is None:
        path = os.environ.get("MYL_ORACLE_LIB")
        if not path:
            if not LIB_PATH.exists():
                build()
            path = str(LIB_PATH)
        _lib = C.CDLL(path)
        _declare(_lib)
    return _lib


P = C.c_void_p
u8, i8, i16, i32, i64, u32, u64, sz = (C.c_uint8, C.c_int8, C.c_int16, C.c_int32, C.c_int64,
                                        C.c_uint32, C.c_uint64, C.c_size_t)


class SynthSpec(C.Structure):
    _fields_ = [("seed", u64), ("vocab", u32), ("hidden", u32), ("layers", u32), ("heads", u32),
                ("kv_heads", u32), ("head_dim", u32), ("inter", u32), ("max_pos", u32),
                ("lm_head_int16", i32), ("attention_bias", i32)]


class MoeSpec(C.Structure):
    _fields_ = [("seed", u64), ("hidden", u32), ("n_experts", u32), ("inter", u32), ("top_k", u32),
                ("shared_inter", u32)]


class Luts(C.Structure):
    _fields_ = [("rsqrt", P), ("rsqrt_len", sz), ("silu", P), ("silu_len", sz), ("exp", P),
                ("exp_len", sz), ("cos", P), ("sin", P), ("rope_len", sz)]


def _declare(L) -> None:
    sigs = {
        "or_clamp_i8": (i8, [i32]), "or_clamp_i16": (i16, [i32]),
        "or_clamp_i16_from_i64": (i16, [i64]), "or_clamp_i32": (i32, [i64]),
        "or_rshift_round": (i32, [i32, u8]), "or_rshift_round_i64": (i64, [i64, u8]),
        "or_rshift_round_i128": (None, [i64, u64, u32, C.POINTER(i64), C.POINTER(u64)]),
        "or_rescale": (i32, [i32, u8, u8]), "or_rescale_i64": (i64, [i64, u8, u8]),
        "or_inv_sqrt_q15": (i64, [sz]), "or_isqrt_round": (u64, [u64]),
        "or_dot_i8_i16": (i64, [P, P, sz]),
        "or_linear_w8a16": (C.c_int, [P, P, sz, P, sz, u8, u8, P]),
        "or_linear_w8a16_pc": (C.c_int, [P, P, sz, P, sz, u8, P, P]),
        "or_add_bias_i16": (C.c_int, [P, P, P, sz, u8]),
        "or_linear_w8a16_batch": (C.c_int, [P, sz, P, sz, sz, P, u8, u8, P, P]),
        "or_linear_w8a16_mult": (C.c_int, [P, sz, P, sz, sz, P, P, P]),
        "or_requant_shift": (C.c_int, [P, sz, sz, P, u8, u8, P]),
        "or_requant_mult": (C.c_int, [P, sz, sz, P, P, P]),
        "or_inv_n_q20": (i64, [sz]),
        "or_rmsnorm_i16": (C.c_int, [P, P, P, P, sz, P, sz, u8, u8, i64, u8, P]),
        "or_rotate_half_split_i16": (C.c_int, [P, sz, P, P, u8, P]),
        "or_apply_rope_i16": (C.c_int, [P, P, sz, sz, P, P, sz, P, u8, P, P]),
        "or_exp_lut_lookup": (i32, [i32, P, sz, u8, i32]),
        "or_softmax_int": (C.c_int, [P, sz, P, sz, u8, u8, P]),
        "or_dot_int": (i64, [P, P, sz]),
        "or_attention_int": (C.c_int, [P, P, P, P, sz, sz, sz, i64, u8, P, sz, u8, u8, P]),
        "or_lut_lookup": (i16, [i16, P, sz, u8, i16]),
        "or_mlp_int": (C.c_int, [P, P, P, P, sz, sz, P, P, P, P, sz, u8, u8, u8, u8, u8, i16, u8, P, P]),
        "or_argmax_int": (i64, [P, sz]),
        "or_splitmix64": (None, [u64, C.POINTER(u64), C.POINTER(u64)]),
        "or_sample_integer_cdf": (None, [P, sz, u64, C.POINTER(i64), C.POINTER(u64)]),
        "or_log2_q16": (None, [u64, C.POINTER(i32), C.POINTER(u32)]),
        "or_ln_q16": (i64, [u64]),
        "or_logsoftmax_at": (i64, [P, sz, P, sz, i64]),
        "or_model_create_synthetic": (P, [C.POINTER(SynthSpec), C.POINTER(Luts)]),
        "or_moe_create_synthetic": (P, [C.POINTER(MoeSpec), P, C.POINTER(Luts)]),
        "or_moe_destroy": (None, [P]),
        "or_moe_synth_input": (None, [P, u32, P]),
        "or_moe_route": (C.c_int, [P, P, u32, P, P, P, P, P]),
        "or_moe_token": (C.c_int, [P, P, P, P, P]),
        "or_moe_expert": (C.c_int, [P, P, u32, P]),
        "or_moe_router_logits": (None, [P, P, P]),
        "or_model_destroy": (None, [P]), "or_model_reset": (None, [P]),
        "or_set_threads": (None, [C.c_int]), "or_set_simd": (None, [C.c_int]),
        "or_model_forward_token": (C.c_int, [P, u32, u32, P]),
        "or_model_embed_token": (C.c_int, [P, u32, P]),
        "or_model_run_layers": (C.c_int, [P, P, u32, u32, u32]),
        "or_model_head_logits": (C.c_int, [P, P, P]),
        "or_model_read_kv": (C.c_int, [P, u32, u32, u32, P, P]),
        "or_model_write_kv": (C.c_int, [P, u32, u32, u32, P, P]),
        "or_model_set_cached": (C.c_int, [P, u32]),
        "or_model_tensor": (P, [P, C.c_char_p, u32, C.POINTER(sz)]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _arr(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=dtype)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (status {rc})")


# ---- scalar helpers ---------------------------------------------------------
def rshift_round(v: int, s: int) -> int: return lib().or_rshift_round(v, s)
def rshift_round_i64(v: int, s: int) -> int: return lib().or_rshift_round_i64(v, s)
def rescale(v: int, a: int, b: int) -> int: return lib().or_rescale(v, a, b)
def rescale_i64(v: int, a: int, b: int) -> int: return lib().or_rescale_i64(v, a, b)
def inv_sqrt_q15(hd: int) -> int: return lib().or_inv_sqrt_q15(hd)
def isqrt_round(n: int) -> int: return lib().or_isqrt_round(n)
def inv_n_q20(n: int) -> int: return lib().or_inv_n_q20(n)


def rshift_round_i128(v: int, s: int) -> int:
    v &= (1 << 128) - 1
    hi, lo = v >> 64, v & ((1 << 64) - 1)
    if hi >= 1 << 63:
        hi -= 1 << 64
    oh, ol = i64(), u64()
    lib().or_rshift_round_i128(hi, lo, s, C.byref(oh), C.byref(ol))
    r = (oh.value << 64) | ol.value
    return r - (1 << 128) if r >= 1 << 127 else r


def splitmix64(state: int) -> tuple[int, int]:
    ns, out = u64(), u64()
    lib().or_splitmix64(state, C.byref(ns), C.byref(out))
    return ns.value, out.value


# ---- vector ops -------------------------------------------------------------
def linear_w8a16(x, W, in_features, w_shifts, act_frac, out_frac) -> np.ndarray:
    x, W, ws = _arr(x, np.int16), _arr(W, np.int8), _arr(w_shifts, np.uint8)
    out = np.zeros(len(ws), np.int16)
    _check(lib().or_linear_w8a16(ptr(x), ptr(W), in_features, ptr(ws), len(ws), act_frac, out_frac, ptr(out)),
           "linear_w8a16")
    return out


def linear_w8a16_pc(x, W, in_features, w_shifts, act_frac, out_frac) -> np.ndarray:
    x, W, ws, of = _arr(x, np.int16), _arr(W, np.int8), _arr(w_shifts, np.uint8), _arr(out_frac, np.uint8)
    out = np.zeros(len(ws), np.int16)
    _check(lib().or_linear_w8a16_pc(ptr(x), ptr(W), in_features, ptr(ws), len(ws), act_frac, ptr(of), ptr(out)),
           "linear_w8a16_pc")
    return out


def linear_batch(x, W, w_shifts, act_frac, out_frac=0, out_frac_pc=None) -> np.ndarray:
    x, W, ws = _arr(x, np.int16), _arr(W, np.int8), _arr(w_shifts, np.uint8)
    M, K = x.shape
    N = W.shape[0]
    of = None if out_frac_pc is None else _arr(out_frac_pc, np.uint8)
    out = np.zeros((M, N), np.int16)
    _check(lib().or_linear_w8a16_batch(ptr(x), M, ptr(W), N, K, ptr(ws), act_frac, out_frac, ptr(of), ptr(out)),
           "linear_w8a16_batch")
    return out


def linear_mult(x, W, mult, shift) -> np.ndarray:
    x, W = _arr(x, np.int16), _arr(W, np.int8)
    mult, shift = _arr(mult, np.int32), _arr(shift, np.uint8)
    M, K = x.shape
    N = W.shape[0]
    out = np.zeros((M, N), np.int16)
    _check(lib().or_linear_w8a16_mult(ptr(x), M, ptr(W), N, K, ptr(mult), ptr(shift), ptr(out)), "linear_mult")
    return out


def requant_shift(acc, w_shifts, act_frac, out_frac) -> np.ndarray:
    """linear_w8a16's requant (linear.rs:61-68) of exact sums acc [M x N]."""
    acc, ws = _arr(acc, np.int64), _arr(w_shifts, np.uint8)
    M, N = acc.shape
    out = np.zeros((M, N), np.int16)
    _check(lib().or_requant_shift(ptr(acc), M, N, ptr(ws), act_frac, out_frac, ptr(out)), "requant_shift")
    return out


def requant_mult(acc, mult, shift) -> np.ndarray:
    """The multiplier requant of exact sums acc [M x N]."""
    acc, mult, shift = _arr(acc, np.int64), _arr(mult, np.int32), _arr(shift, np.uint8)
    M, N = acc.shape
    out = np.zeros((M, N), np.int16)
    _check(lib().or_requant_mult(ptr(acc), M, N, ptr(mult), ptr(shift), ptr(out)), "requant_mult")
    return out


def add_bias_i16(out, bias, bias_shifts, out_frac) -> np.ndarray:
    o = _arr(out, np.int16).copy()
    b, bs = _arr(bias, np.int16), _arr(bias_shifts, np.uint8)
    _check(lib().or_add_bias_i16(ptr(o), ptr(b), ptr(bs), len(o), out_frac), "add_bias_i16")
    return o


def rmsnorm_i16(x, x_shifts, gamma, gamma_shifts, rsqrt_lut, lut_input_shift, lut_output_frac, inv_n, out_frac):
    x, xs = _arr(x, np.int16), _arr(x_shifts, np.uint8)
    g, gs, lut = _arr(gamma, np.int8), _arr(gamma_shifts, np.uint8), _arr(rsqrt_lut, np.int16)
    out = np.zeros(len(x), np.int16)
    _check(lib().or_rmsnorm_i16(ptr(x), ptr(xs), ptr(g), ptr(gs), len(x), ptr(lut), len(lut), lut_input_shift,
                                lut_output_frac, inv_n, out_frac, ptr(out)), "rmsnorm_i16")
    return out


def rotate_half_split_i16(vec, cos_row, sin_row, frac_bits) -> np.ndarray:
    v, c, s = _arr(vec, np.int16), _arr(cos_row, np.int16), _arr(sin_row, np.int16)
    out = np.zeros(len(v), np.int16)
    lib().or_rotate_half_split_i16(ptr(v), len(v), ptr(c), ptr(s), frac_bits, ptr(out))
    return out


def apply_rope_i16(q, k, cos_lut, sin_lut, positions, frac_bits):
    q, k = _arr(q, np.int16), _arr(k, np.int16)
    c, s, p = _arr(cos_lut, np.int16), _arr(sin_lut, np.int16), _arr(positions, np.uint64)
    n, hd = q.shape
    qo, ko = np.zeros_like(q), np.zeros_like(k)
    _check(lib().or_apply_rope_i16(ptr(q), ptr(k), n, hd, ptr(c), ptr(s), len(c), ptr(p), frac_bits, ptr(qo), ptr(ko)),
           "apply_rope_i16")
    return qo, ko


def softmax_int(logits, exp_lut, lut_shift, frac_bits) -> np.ndarray:
    lg, lut = _arr(logits, np.int32), _arr(exp_lut, np.int16)
    out = np.zeros(len(lg), np.int32)
    _check(lib().or_softmax_int(ptr(lg), len(lg), ptr(lut), len(lut), lut_shift, frac_bits, ptr(out)), "softmax_int")
    return out


def attention_int(q, k, v, score_mult, score_shift, exp_lut, lut_shift, prob_frac_bits, mask=None):
    q, k, v = _arr(q, np.int16), _arr(k, np.int16), _arr(v, np.int16)
    lut = _arr(exp_lut, np.int16)
    ql, hd = q.shape
    kl = k.shape[0]
    mk = None if mask is None else _arr(mask, np.uint8)
    out = np.zeros((ql, hd), np.int16)
    _check(lib().or_attention_int(ptr(q), ptr(k), ptr(v), ptr(mk), ql, kl, hd, score_mult, score_shift, ptr(lut),
                                  len(lut), lut_shift, prob_frac_bits, ptr(out)), "attention_int")
    return out


def lut_lookup(x, lut, shift, offset) -> int:
    lut = _arr(lut, np.int16)
    return lib().or_lut_lookup(x, ptr(lut), len(lut), shift, offset)


def mlp_int(x, W_gate, W_up, W_down, hidden, inter, gs, us, ds, silu, in_frac, gate_frac, up_frac,
            down_in_frac, silu_in_frac, silu_off, silu_out_frac, out_frac) -> np.ndarray:
    x, Wg, Wu, Wd = _arr(x, np.int16), _arr(W_gate, np.int8), _arr(W_up, np.int8), _arr(W_down, np.int8)
    gs, us, ds = _arr(gs, np.uint8), _arr(us, np.uint8), _arr(ds, np.uint8)
    silu, of = _arr(silu, np.int16), _arr(out_frac, np.uint8)
    out = np.zeros(hidden, np.int16)
    _check(lib().or_mlp_int(ptr(x), ptr(Wg), ptr(Wu), ptr(Wd), hidden, inter, ptr(gs), ptr(us), ptr(ds), ptr(silu),
                            len(silu), in_frac, gate_frac, up_frac, down_in_frac, silu_in_frac, silu_off,
                            silu_out_frac, ptr(of), ptr(out)), "mlp_int")
    return out


def argmax_int(v) -> int:
    a = _arr(v, np.int32)
    return lib().or_argmax_int(ptr(a), len(a))


def sample_integer_cdf(v, state: int) -> tuple[int, int]:
    """sampling.rs:27-46: (token, new_state)."""
    a = _arr(v, np.int32)
    tok, ns = i64(), u64()
    lib().or_sample_integer_cdf(ptr(a), len(a), int(state) & (2**64 - 1), C.byref(tok), C.byref(ns))
    return int(tok.value), int(ns.value)


# ---- integer log-softmax (build-defined) ---------------------------------------
def log2_q16(S: int) -> tuple[int, int]:
    e, f = i32(), u32()
    lib().or_log2_q16(S, C.byref(e), C.byref(f))
    return e.value, f.value


def ln_q16(S: int) -> int:
    return lib().or_ln_q16(S)


def logsoftmax_at(z, exp_lut, target: int) -> int:
    a = _arr(z, np.int32)
    lut = _arr(exp_lut, np.int16)
    return lib().or_logsoftmax_at(ptr(a), len(a), ptr(lut), len(lut), target)


# ---- model -------------------------------------------------------------------
def make_luts_struct(luts) -> tuple[Luts, tuple]:
    arrs = tuple(np.ascontiguousarray(a, dtype=np.int16) for a in (luts.rsqrt, luts.silu, luts.exp, luts.cos, luts.sin))
    s = Luts(ptr(arrs[0]), len(arrs[0]), ptr(arrs[1]), len(arrs[1]), ptr(arrs[2]), len(arrs[2]),
             ptr(arrs[3]), ptr(arrs[4]), len(arrs[3]))
    return s, arrs


class OracleModel:
    """The reference IntegerModel (model.rs:120-163) on a seeded synthetic spec."""

    def __init__(self, spec: dict, luts, threads: int = 1):
        self.spec = dict(spec)
        self._cspec = SynthSpec(**{k: spec[k] for k, _ in SynthSpec._fields_})
        self._luts, self._keep = make_luts_struct(luts)
        lib().or_set_threads(threads)
        self._h = lib().or_model_create_synthetic(C.byref(self._cspec), C.byref(self._luts))
        if not self._h:
            raise ValueError("oracle model creation failed (bad spec or out of memory)")

    def close(self) -> None:
        if self._h:
            lib().or_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self) -> None:
        lib().or_model_reset(self._h)

    def forward_token(self, token: int, pos: int, want_logits: bool = True):
        logits = np.zeros(self.spec["vocab"], np.int32) if want_logits else None
        _check(lib().or_model_forward_token(self._h, token, pos, ptr(logits)), "forward_token")
        return logits

    @staticmethod
    def sample_next(logits, state: int):
        """IntegerModel::sample_next (model.rs:785-787)."""
        return sample_integer_cdf(logits, state)

    def embed_token(self, token: int) -> np.ndarray:
        h = np.zeros(self.spec["hidden"], np.int16)
        _check(lib().or_model_embed_token(self._h, token, ptr(h)), "embed_token")
        return h

    def run_layers(self, hidden, pos: int, layer_start: int, layer_end: int) -> np.ndarray:
        h = _arr(hidden, np.int16).copy()
        _check(lib().or_model_run_layers(self._h, ptr(h), pos, layer_start, layer_end), "run_layers")
        return h

    def head_logits(self, hidden) -> np.ndarray:
        h = _arr(hidden, np.int16)
        out = np.zeros(self.spec["vocab"], np.int32)
        _check(lib().or_model_head_logits(self._h, ptr(h), ptr(out)), "head_logits")
        return out

    def read_kv(self, layer: int, kv_head: int, n_pos: int):
        hd = self.spec["head_dim"]
        k = np.zeros((n_pos, hd), np.int16)
        v = np.zeros((n_pos, hd), np.int16)
        _check(lib().or_model_read_kv(self._h, layer, kv_head, n_pos, ptr(k), ptr(v)), "read_kv")
        return k, v

    def write_kv(self, layer: int, kv_head: int, k, v) -> None:
        """Overwrites cache positions [0, len(k)) of (layer, kv_head)."""
        k, v = _arr(k, np.int16), _arr(v, np.int16)
        assert k.shape == v.shape and k.shape[1] == self.spec["head_dim"]
        _check(lib().or_model_write_kv(self._h, layer, kv_head, k.shape[0], ptr(k), ptr(v)), "write_kv")

    def set_cached(self, n_pos: int) -> None:
        """The cached length: the next forward_token may run at any position <= n_pos."""
        _check(lib().or_model_set_cached(self._h, n_pos), "set_cached")

    def tensor(self, name: str, layer: int = 0, dtype=np.int8) -> np.ndarray:
        """A copy of one of the model's tensors (or_model_tensor names)."""
        return self.tensor_view(name, layer, dtype).copy()

    def tensor_view(self, name: str, layer: int = 0, dtype=np.int8) -> np.ndarray:
        """The model's own memory for tensor `name`: writes change the model
        (tests build special-case layers this way).  "layer_fracs" is the
        nine bytes norm_attn, q, k, v, attn_out, norm_mlp, gate, up, down_in."""
        n = sz()
        p = lib().or_model_tensor(self._h, name.encode(), layer, C.byref(n))
        if not p:
            raise KeyError(name)
        buf = (C.c_char * n.value).from_address(p)
        return np.frombuffer(buf, dtype=dtype)


class OracleMoe:
    """The build-defined integer MoE layer (include/myl_hip.h section 4) on the CPU."""

    def __init__(self, spec: dict, bias, luts, threads: int = 1):
        self.spec = dict(spec)
        self._cspec = MoeSpec(**{k: int(spec[k]) for k, _ in MoeSpec._fields_})
        self._luts, self._keep = make_luts_struct(luts)
        self.bias = _arr(bias, np.int32)
        lib().or_set_threads(threads)
        self._h = lib().or_moe_create_synthetic(C.byref(self._cspec), ptr(self.bias), C.byref(self._luts))
        if not self._h:
            raise ValueError("oracle MoE creation failed")

    def close(self) -> None:
        if self._h:
            lib().or_moe_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synth_input(self, n_tokens: int) -> np.ndarray:
        x = np.zeros((n_tokens, self.spec["hidden"]), np.int16)
        lib().or_moe_synth_input(self._h, n_tokens, ptr(x))
        return x

    def route(self, x) -> dict:
        x = _arr(x, np.int16)
        T = x.shape[0]
        K, E = self.spec["top_k"], self.spec["n_experts"]
        ids = np.zeros((T, K), np.int32)
        gates = np.zeros((T, K), np.int32)
        counts = np.zeros(E, np.int32)
        offsets = np.zeros(E + 1, np.int32)
        lst = np.zeros(T * K, np.int32)
        _check(lib().or_moe_route(self._h, ptr(x), T, ptr(ids), ptr(gates), ptr(counts), ptr(offsets), ptr(lst)),
               "moe_route")
        return dict(ids=ids, gates=gates, counts=counts, offsets=offsets, list_tok=lst)

    def token(self, xt, ids_t, gates_t) -> np.ndarray:
        out = np.zeros(self.spec["hidden"], np.int16)
        _check(lib().or_moe_token(self._h, ptr(_arr(xt, np.int16)), ptr(_arr(ids_t, np.int32)),
                                  ptr(_arr(gates_t, np.int32)), ptr(out)), "moe_token")
        return out

    def expert(self, xt, expert: int) -> np.ndarray:
        out = np.zeros(self.spec["hidden"], np.int16)
        _check(lib().or_moe_expert(self._h, ptr(_arr(xt, np.int16)), expert, ptr(out)), "moe_expert")
        return out

    def router_logits(self, xt) -> np.ndarray:
        z = np.zeros(self.spec["n_experts"], np.int32)
        lib().or_moe_router_logits(self._h, ptr(_arr(xt, np.int16)), ptr(z))
        return z


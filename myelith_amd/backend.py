"""RocmBackend: the host-side mirror of the reference's `Backend` trait.

Mirrors INTEGER_LLM/kernels/src/backends/rocm.rs (RocmBackend::init, name,
hardware_family, feature_tag, gcn_arch) and the trait methods of
INTEGER_LLM/kernels/src/backend.rs:23-127, plus the free functions that
runtime/src/model.rs calls directly (linear_w8a16_pc, add_bias_i16,
argmax_int).  Every method calls libmyl_hip.so; arguments keep the reference's
names, order and meaning.  Shape errors raise ValueError where the reference
panics.

The `*_dev` methods take torch tensors already on the GPU and run on torch's
current stream (plumbing only: the arithmetic is in the HIP kernels).
"""
from __future__ import annotations

import ctypes as C
import weakref

import numpy as np

from ._lib import MYL_E_INVALID, lib


class MylError(RuntimeError):
    pass


def _a(x, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x), dtype=dtype)


def _p(a):
    return None if a is None else a.ctypes.data


class RocmBackend:
    """One HIP context on one device (rocm.rs:41-60)."""

    def __init__(self, device_id: int = 0):
        h = C.c_void_p()
        rc = lib().myl_init(device_id, C.byref(h))
        if rc != 0:
            raise MylError(f"RocmBackend::init({device_id}) failed with status {rc}")
        self._h = h
        self._device_id = device_id
        # models and MoE layers on this context: closed before it is destroyed,
        # whatever order the interpreter finalises them in
        self._owned = weakref.WeakSet()
        arch = C.create_string_buffer(128)
        cus = C.c_int()
        hbm = C.c_uint64()
        lib().myl_device_info(self._h, arch, 128, C.byref(cus), C.byref(hbm))
        self._arch = arch.value.decode()
        self.cu_count = cus.value
        self.hbm_bytes = hbm.value

    # ---- identity (rocm.rs:62-82) -------------------------------------------
    def device_id(self) -> int:
        return self._device_id

    def gcn_arch(self) -> str:
        return self._arch

    @staticmethod
    def name() -> str:
        return lib().myl_backend_name().decode()

    @staticmethod
    def hardware_family() -> str:
        return lib().myl_hardware_family().decode()

    @staticmethod
    def feature_tag() -> str:
        return lib().myl_feature_tag().decode()

    # ---- plumbing -------------------------------------------------------------
    @property
    def handle(self):
        return self._h

    def adopt(self, obj) -> None:
        """Registers an object holding device state of this context; close()
        closes it first."""
        self._owned.add(obj)

    def close(self) -> None:
        if self._h:
            for obj in list(self._owned):
                obj.close()
            lib().myl_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, rc: int, what: str) -> None:
        if rc != 0:
            msg = lib().myl_last_error(self._h).decode()
            if rc == MYL_E_INVALID:
                raise ValueError(f"{what}: {msg}")
            raise MylError(f"{what} failed ({rc}): {msg}")

    def synchronize(self) -> None:
        self.check(lib().myl_synchronize(self._h), "synchronize")

    def read_probe_dev(self, buf, out) -> None:
        """One pass of 16-byte nontemporal loads over the device tensor buf (a
        measurement of the achievable read rate; out: a device int32 word)."""
        self.check(lib().myl_read_probe(self._h, buf.data_ptr(), buf.numel() * buf.element_size(), out.data_ptr()),
                   "read_probe")

    def use_torch_stream(self) -> None:
        """Launch on torch's current HIP stream (so torch events time our kernels)."""
        import torch
        self.check(lib().myl_set_stream(self._h, C.c_void_p(torch.cuda.current_stream().cuda_stream)), "set_stream")

    # ---- Backend trait (backend.rs:39-126), host slices ----------------------------
    def linear_w8a16(self, x, W, in_features: int, out_features: int, w_shifts, act_frac: int, out_frac: int):
        x, W, ws = _a(x, np.int16), _a(W, np.int8), _a(w_shifts, np.uint8)
        if W.size != in_features * out_features or ws.size != out_features or x.size < in_features:
            raise ValueError("linear_w8a16: W does not hold out_features rows of in_features (linear.rs:51-58)")
        out = np.zeros(out_features, np.int16)
        self.check(lib().myl_linear_w8a16(self._h, _p(x), _p(W), _p(out), in_features, out_features, _p(ws),
                                          act_frac, out_frac), "linear_w8a16")
        return out

    def linear_w8a16_pc(self, x, W, in_features: int, w_shifts, act_frac: int, out_frac):
        x, W, ws, of = _a(x, np.int16), _a(W, np.int8), _a(w_shifts, np.uint8), _a(out_frac, np.uint8)
        n = ws.size
        if W.size != in_features * n or of.size != n or x.size < in_features:
            raise ValueError("linear_w8a16_pc: shape mismatch (linear.rs:95-107)")
        out = np.zeros(n, np.int16)
        self.check(lib().myl_linear_w8a16_pc(self._h, _p(x), _p(W), _p(out), in_features, n, _p(ws), act_frac,
                                             _p(of)), "linear_w8a16_pc")
        return out

    def add_bias_i16(self, out, bias, bias_shifts, out_frac: int):
        o, b, bs = _a(out, np.int16).copy(), _a(bias, np.int16), _a(bias_shifts, np.uint8)
        if o.size != b.size or b.size != bs.size:
            raise ValueError("add_bias_i16: out, bias and shifts must have the same length (linear.rs:133-140)")
        self.check(lib().myl_add_bias_i16(self._h, _p(o), _p(b), _p(bs), o.size, out_frac), "add_bias_i16")
        return o

    def rmsnorm(self, x, x_shifts, gamma, gamma_shifts, rsqrt_lut, lut_input_shift: int, lut_output_frac: int,
                inv_n_q20: int, out_frac: int):
        x, xs, g, gs = _a(x, np.int16), _a(x_shifts, np.uint8), _a(gamma, np.int8), _a(gamma_shifts, np.uint8)
        lut = _a(rsqrt_lut, np.int16)
        n = x.size
        if not (g.size == n and gs.size == n and xs.size == n):
            raise ValueError("rmsnorm: x, gamma, gamma_shifts and x_shifts must match (rmsnorm.rs:73-75)")
        out = np.zeros(n, np.int16)
        self.check(lib().myl_rmsnorm(self._h, _p(x), _p(xs), _p(g), _p(gs), n, _p(lut), lut.size, lut_input_shift,
                                     lut_output_frac, inv_n_q20, _p(out), out_frac), "rmsnorm")
        return out

    def softmax(self, logits, exp_lut, lut_shift: int, frac_bits: int):
        z, lut = _a(logits, np.int32), _a(exp_lut, np.int16)
        out = np.zeros(z.size, np.int32)
        self.check(lib().myl_softmax(self._h, _p(z), _p(out), z.size, _p(lut), lut.size, lut_shift, frac_bits),
                   "softmax")
        return out

    def attention(self, q, k, v, mask, score_mult: int, score_shift: int, exp_lut, lut_shift: int,
                  prob_frac: int):
        q, k, v = _a(q, np.int16), _a(k, np.int16), _a(v, np.int16)
        if q.ndim != 2 or k.shape != v.shape or k.shape[1] != q.shape[1]:
            raise ValueError("attention: q [q_len x hd], k and v [kv_len x hd] (attention.rs:53-56)")
        ql, hd = q.shape
        kl = k.shape[0]
        mk = None if mask is None else _a(mask, np.uint8)
        if mk is not None and mk.shape != (ql, kl):
            raise ValueError("attention: mask must be [q_len x kv_len]")
        lut = _a(exp_lut, np.int16)
        out = np.zeros((ql, hd), np.int16)
        self.check(lib().myl_attention(self._h, _p(q), _p(k), _p(v), _p(out), ql, kl, hd, _p(mk), score_mult,
                                       score_shift, _p(lut), lut.size, lut_shift, prob_frac), "attention")
        return out

    def rope(self, q, k, cos_lut, sin_lut, positions, frac_bits: int):
        q, k = _a(q, np.int16).copy(), _a(k, np.int16).copy()
        c, s, p = _a(cos_lut, np.int16), _a(sin_lut, np.int16), _a(positions, np.uint64)
        n, hd = q.shape
        if k.shape != q.shape or p.size != n:
            raise ValueError("rope: q, k and positions must agree")
        self.check(lib().myl_rope(self._h, _p(q), _p(k), n, hd, _p(c), _p(s), c.size, _p(p), frac_bits), "rope")
        return q, k

    def mlp(self, x, W_gate, W_up, W_down, gate_w_shifts, up_w_shifts, down_w_shifts, silu_lut, in_frac: int,
            gate_out_frac: int, up_out_frac: int, down_in_frac: int, silu_in_frac: int, silu_lut_offset: int,
            silu_out_frac: int, out_frac):
        x = _a(x, np.int16)
        hidden = x.size
        Wg, Wu, Wd = _a(W_gate, np.int8), _a(W_up, np.int8), _a(W_down, np.int8)
        inter = Wg.size // hidden  # rocm.rs:183-186
        gs, us, ds = _a(gate_w_shifts, np.uint8), _a(up_w_shifts, np.uint8), _a(down_w_shifts, np.uint8)
        silu, of = _a(silu_lut, np.int16), _a(out_frac, np.uint8)
        if Wg.size != inter * hidden or Wu.size != Wg.size or Wd.size != Wg.size or gs.size != inter \
                or us.size != inter or ds.size != hidden or of.size != hidden:
            raise ValueError("mlp: weight and shift shapes do not agree (mlp.rs:28-74)")
        out = np.zeros(hidden, np.int16)
        self.check(lib().myl_mlp(self._h, _p(x), _p(Wg), _p(Wu), _p(Wd), _p(out), hidden, inter, _p(gs), _p(us),
                                 _p(ds), _p(silu), silu.size, in_frac, gate_out_frac, up_out_frac, down_in_frac,
                                 silu_in_frac, silu_lut_offset, silu_out_frac, _p(of)), "mlp")
        return out

    def argmax_int(self, values) -> int:
        v = _a(values, np.int32)
        out = C.c_int64()
        self.check(lib().myl_argmax_int(self._h, _p(v), v.size, C.byref(out)), "argmax_int")
        return out.value

    def sample_integer_cdf(self, logits, state: int):
        """sampling.rs:27-46 on the GPU: (token, new_state)."""
        v = _a(logits, np.int32)
        tok, ns = C.c_int64(), C.c_uint64()
        self.check(lib().myl_sample_integer_cdf(self._h, _p(v), v.size, int(state) & (2**64 - 1), C.byref(tok),
                                                C.byref(ns)), "sample_integer_cdf")
        return int(tok.value), int(ns.value)

    # ---- device forms (torch tensors on the GPU) ------------------------------
    def linear_w8a16_dev(self, x, W, w_shifts, act_frac: int, out_frac: int = 0, out_frac_pc=None, out=None):
        import torch
        M, K = x.shape
        N = W.shape[0]
        if out is None:
            out = torch.empty((M, N), dtype=torch.int16, device=x.device)
        self.check(lib().myl_linear_w8a16_dev(self._h, x.data_ptr(), M, x.stride(0), W.data_ptr(), N, K,
                                              w_shifts.data_ptr(), act_frac, out_frac,
                                              None if out_frac_pc is None else out_frac_pc.data_ptr(),
                                              out.data_ptr(), out.stride(0)), "linear_w8a16_dev")
        return out

    def linear_w8a16_dev_noalloc(self, x, W, w_shifts, act_frac: int, out_frac: int = 0, out_frac_pc=None, out=None):
        """linear_w8a16_dev without device allocation: `out` must be given
        (the library allocates nothing; include/myl_hip.h states the limit)."""
        M, K = x.shape
        N = W.shape[0]
        assert out is not None and tuple(out.shape) == (M, N), "out [M x N] is the caller's"
        self.check(lib().myl_linear_w8a16_dev_noalloc(self._h, x.data_ptr(), M, x.stride(0), W.data_ptr(), N, K,
                                                      w_shifts.data_ptr(), act_frac, out_frac,
                                                      None if out_frac_pc is None else out_frac_pc.data_ptr(),
                                                      out.data_ptr(), out.stride(0)), "linear_w8a16_dev_noalloc")
        return out

    def linear_w8a16_mult_dev(self, x, W, mult, shift, out=None):
        import torch
        M, K = x.shape
        N = W.shape[0]
        if out is None:
            out = torch.empty((M, N), dtype=torch.int16, device=x.device)
        self.check(lib().myl_linear_w8a16_mult_dev(self._h, x.data_ptr(), M, x.stride(0), W.data_ptr(), N, K,
                                                   mult.data_ptr(), shift.data_ptr(), out.data_ptr(), out.stride(0)),
                   "linear_w8a16_mult_dev")
        return out

    def logits_dev(self, x, W, row_shifts, norm_frac: int, logit_frac: int, out=None):
        import torch
        M, K = x.shape
        N = W.shape[0]
        bits = 16 if W.dtype == torch.int16 else 8
        if out is None:
            out = torch.empty((M, N), dtype=torch.int32, device=x.device)
        self.check(lib().myl_logits_dev(self._h, x.data_ptr(), M, x.stride(0), W.data_ptr(), bits, N, K,
                                        row_shifts.data_ptr(), norm_frac, logit_frac, out.data_ptr(), out.stride(0)),
                   "logits_dev")
        return out

    def dot_i8_i16_dev(self, x, W, out=None):
        import torch
        M, K = x.shape
        N = W.shape[0]
        if out is None:
            out = torch.empty((M, N), dtype=torch.int64, device=x.device)
        self.check(lib().myl_dot_i8_i16_dev(self._h, x.data_ptr(), M, x.stride(0), W.data_ptr(), N, K,
                                            out.data_ptr(), out.stride(0)), "dot_i8_i16_dev")
        return out

    def rmsnorm_dev(self, x, x_shifts, gamma, gamma_shifts, rsqrt_lut, lut_input_shift, lut_output_frac, inv_n_q20,
                    out_frac, out=None):
        import torch
        M, n = x.shape
        if out is None:
            out = torch.empty_like(x)
        self.check(lib().myl_rmsnorm_dev(self._h, x.data_ptr(), M, x.stride(0), x_shifts.data_ptr(), gamma.data_ptr(),
                                         gamma_shifts.data_ptr(), n, rsqrt_lut.data_ptr(), rsqrt_lut.numel(),
                                         lut_input_shift, lut_output_frac, inv_n_q20, out_frac, out.data_ptr(),
                                         out.stride(0)), "rmsnorm_dev")
        return out

    def softmax_dev(self, z, exp_lut, lut_shift, frac_bits, out=None):
        import torch
        M, n = z.shape
        if out is None:
            out = torch.empty_like(z)
        self.check(lib().myl_softmax_dev(self._h, z.data_ptr(), M, n, z.stride(0), exp_lut.data_ptr(), exp_lut.numel(),
                                         lut_shift, frac_bits, out.data_ptr(), out.stride(0)), "softmax_dev")
        return out

    def argmax_dev(self, v, out=None):
        import torch
        M, n = v.shape
        if out is None:
            out = torch.empty(M, dtype=torch.int64, device=v.device)
        self.check(lib().myl_argmax_dev(self._h, v.data_ptr(), M, n, v.stride(0), out.data_ptr()), "argmax_dev")
        return out

    def sample_dev(self, z, states, tokens=None, new_states=None):
        """Rows of sample_integer_cdf (sampling.rs:27-46): z int32 [M x n],
        states uint64 [M] (torch int64 tensors hold the bits)."""
        import torch
        M, n = z.shape
        if tokens is None:
            tokens = torch.empty(M, dtype=torch.int64, device=z.device)
        if new_states is None:
            new_states = torch.empty(M, dtype=torch.int64, device=z.device)
        self.check(lib().myl_sample_dev(self._h, z.data_ptr(), M, n, z.stride(0), states.data_ptr(), tokens.data_ptr(),
                                        new_states.data_ptr()), "sample_dev")
        return tokens, new_states

    def logsoftmax_dev(self, z, exp_lut, targets, out=None):
        """Integer log-softmax at targets[m] per row, Q16 int64 (build-defined;
        the reference's perplexity probe uses f64, perplexity_probe.rs:55-67)."""
        import torch
        M, n = z.shape
        lut = exp_lut if isinstance(exp_lut, torch.Tensor) else torch.from_numpy(
            np.ascontiguousarray(exp_lut, dtype=np.int16)).to(z.device)
        t = targets if isinstance(targets, torch.Tensor) else torch.as_tensor(
            np.asarray(targets, dtype=np.int64), device=z.device)
        if out is None:
            out = torch.empty(M, dtype=torch.int64, device=z.device)
        self.check(lib().myl_logsoftmax_dev(self._h, z.data_ptr(), M, n, z.stride(0), lut.data_ptr(), lut.numel(),
                                            t.data_ptr(), out.data_ptr()), "logsoftmax_dev")
        return out

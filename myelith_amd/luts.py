"""Lookup tables of the theta_v 0.17.0 numeric contract.

These are the closed forms of INTEGER_LLM/calibrate/src/luts.py:32-150,
evaluated in double precision and rounded half-to-even (Python's ``round``),
exactly as the reference's offline generator does.  The tables are built once
at model construction; nothing here runs on the integer hot path.

The SHA-256 of each table's int16 little-endian bytes is what the reference's
scale packs record (INTEGER_LLM/scale_packs/qwen2.5-*/luts.json), so a table
produced here can be checked byte for byte against the shipped ones.
"""
from __future__ import annotations

import hashlib
import math

import numpy as np

# theta_v/spec.json "nonlinear" section (see also include/myl_theta_v.h).
RSQRT_INPUT_RANGE_MAX = 32767
RSQRT_INPUT_SHIFT = 8
RSQRT_OUTPUT_FRAC = 8
SILU_INPUT_MIN, SILU_INPUT_MAX = -8192, 8191
SILU_INPUT_FRAC = 6
SILU_OUTPUT_FRAC = 8
EXP_LUT_RANGE = 16384
EXP_INPUT_FRAC = 8
EXP_LUT_FRAC = 14
ROPE_MAX_SEQ_LEN = 2048
ROPE_FRAC = 8
ROPE_THETA = 1000000.0


def rsqrt_lut(max_input: int = RSQRT_INPUT_RANGE_MAX, input_shift: int = RSQRT_INPUT_SHIFT,
              frac_bits: int = RSQRT_OUTPUT_FRAC) -> np.ndarray:
    """luts.py:32-49: lut[x] = round(2^frac / sqrt(x / 2^input_shift)), lut[0] = 2^frac."""
    scale = 1 << frac_bits
    out = [scale]
    for x in range(1, max_input + 1):
        real = x / (1 << input_shift)
        out.append(int(round(1.0 / math.sqrt(real) * scale)))
    return np.asarray(out, dtype=np.int16)


def silu_lut(input_min: int = SILU_INPUT_MIN, input_max: int = SILU_INPUT_MAX,
             input_frac: int = SILU_INPUT_FRAC, output_frac: int = SILU_OUTPUT_FRAC) -> np.ndarray:
    """luts.py:52-68: lut[x - input_min] = round(silu(x / 2^in) * 2^out)."""
    in_scale = 1 << input_frac
    out_scale = 1 << output_frac
    out = []
    for x in range(input_min, input_max + 1):
        xf = x / in_scale
        out.append(int(round(xf * (1.0 / (1.0 + math.exp(-xf))) * out_scale)))
    return np.asarray(out, dtype=np.int16)


def exp_lut(exp_range: int = EXP_LUT_RANGE, input_frac: int = EXP_INPUT_FRAC,
            output_frac: int = EXP_LUT_FRAC) -> np.ndarray:
    """luts.py:101-118: lut[i] = round(exp(-i / 2^in) * 2^out), i in [0, range]."""
    in_scale = 1 << input_frac
    out_scale = 1 << output_frac
    return np.asarray([int(round(math.exp(-(i / in_scale)) * out_scale)) for i in range(exp_range + 1)],
                      dtype=np.int16)


def rope_luts(head_dim: int, max_seq_len: int = ROPE_MAX_SEQ_LEN, rope_theta: float = ROPE_THETA,
              frac_bits: int = ROPE_FRAC) -> tuple[np.ndarray, np.ndarray]:
    """luts.py:121-150: flat [max_seq_len x head_dim/2]; theta_j = theta^-(j/half).

    Returns (cos, sin)."""
    scale = 1 << frac_bits
    half = head_dim // 2
    cos_l, sin_l = [], []
    thetas = [1.0 / (rope_theta ** (j / half)) for j in range(half)]
    for p in range(max_seq_len):
        for j in range(half):
            angle = p * thetas[j]
            cos_l.append(int(round(math.cos(angle) * scale)))
            sin_l.append(int(round(math.sin(angle) * scale)))
    return np.asarray(cos_l, dtype=np.int16), np.asarray(sin_l, dtype=np.int16)


def sha256_i16(table: np.ndarray) -> str:
    """SHA-256 over the table's int16 little-endian bytes (the .lut.bin layout)."""
    return hashlib.sha256(np.ascontiguousarray(table, dtype="<i2").tobytes()).hexdigest()


class LutSet:
    """The five tables a model consumes (loader.rs:509, model.rs:149-155)."""

    _cache: dict[int, "LutSet"] = {}

    def __init__(self, head_dim: int):
        self.head_dim = head_dim
        self.rsqrt = rsqrt_lut()
        self.silu = silu_lut()
        self.exp = exp_lut()
        self.cos, self.sin = rope_luts(head_dim)

    @classmethod
    def from_tables(cls, head_dim: int, rsqrt, silu, exp, cos, sin) -> "LutSet":
        """A set holding given tables (an artifact's luts.json)."""
        self = cls.__new__(cls)
        self.head_dim = head_dim
        for name, t in (("rsqrt", rsqrt), ("silu", silu), ("exp", exp), ("cos", cos), ("sin", sin)):
            setattr(self, name, np.ascontiguousarray(t, dtype=np.int16))
        return self

    @classmethod
    def for_head_dim(cls, head_dim: int) -> "LutSet":
        if head_dim not in cls._cache:
            cls._cache[head_dim] = cls(head_dim)
        return cls._cache[head_dim]

    def hashes(self) -> dict[str, str]:
        return {name: sha256_i16(getattr(self, name)) for name in ("cos", "exp", "rsqrt", "silu", "sin")}

// rows_epi.h -- epilogues of the row-batched products (batched forward, MoE):
// each maps the exact sum of weight row n and activation row m to the
// reference's requantized output (see gemm_dispatch.h for the interface).
#pragma once

#include "fixed.h"
#include "wave.h"
#include "../../include/myl_theta_v.h"

namespace myl {

template <class D>
struct EpiApply {
    template <int R, int MT>
    __device__ inline void apply(int row0, int N, int M, int lane, const int64_t (&tot)[R][MT]) const {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (lane == r * MT + m && row0 + r < N && m < M)
                    static_cast<const D*>(this)->one(row0 + r, m, tot[r][m]);
    }
};

// q/k/v rows (pair-ordered within each head): requant to the segment's frac,
// then the bias (linear.rs:132-145).
struct EpiQKVRows : EpiApply<EpiQKVRows> {
    const uint8_t* shifts;
    const int16_t* bias;      // or null
    const uint8_t* bias_sh;
    uint8_t act_frac, q_frac, k_frac, v_frac;
    int nq, nkv;
    int16_t* out; int ldo;
    EpiQKVRows offset_m(int m0) const { EpiQKVRows e = *this; e.out += (size_t)m0 * ldo; return e; }
    // the requantised projection (+ bias) of output n, not stored
    __device__ inline int16_t value(int n, int64_t acc) const { return value_with(val_ops(n), n, acc); }
    // the same in two steps: the row's operands, fetched ahead of the sum
    struct ValOps { uint8_t sh, bs; int16_t b; };
    __device__ inline ValOps val_ops(int n) const {
        return ValOps{shifts[n], bias ? bias_sh[n] : (uint8_t)0, bias ? bias[n] : (int16_t)0};
    }
    __device__ inline int16_t value_with(const ValOps& o, int n, int64_t acc) const {
        const uint8_t frac = n < nq ? q_frac : (n < nq + nkv ? k_frac : v_frac);
        int16_t v = clamp_i16_i64(rescale64(acc, (uint8_t)(o.sh + act_frac), frac));
        if (bias) v = clamp_i16_i64((int64_t)v + (int64_t)rescale32((int32_t)o.b, o.bs, frac));
        return v;
    }
    __device__ inline void one(int n, int m, int64_t acc) const { out[(size_t)m * ldo + n] = value(n, acc); }
};

// o_proj / down_proj with the residual add (model.rs:576-593, 612-671):
// o = clamp(rescale(acc, w_shift + act, acc_frac)), h = rescale(res, res_frac,
// acc_frac), out = clamp(rescale(h + o, acc_frac, out_frac)).
struct EpiResidRows : EpiApply<EpiResidRows> {
    const uint8_t* shifts;
    uint8_t act_frac;
    const uint8_t* acc_frac;
    const uint8_t* res_frac;
    const uint8_t* out_frac;
    const int16_t* res; int ldr;
    int16_t* out; int ldo;
    EpiResidRows offset_m(int m0) const {
        EpiResidRows e = *this;
        e.res += (size_t)m0 * ldr;
        e.out += (size_t)m0 * ldo;
        return e;
    }
    // the output element, also stored
    __device__ inline int16_t value(int n, int m, int64_t acc) const {
        const int16_t y = value_of(acc, fin_ops(n, m));
        out[(size_t)m * ldo + n] = y;
        return y;
    }
    // The same in two steps, so a caller can issue every operand load of
    // several elements before any store (a store may alias the operands, so
    // the compiler would otherwise keep each element's loads behind the
    // previous element's stores: one memory round trip per element).
    struct FinOps { uint8_t af, sh, rf, of; int16_t r; };
    __device__ inline FinOps fin_ops(int n, int m) const {
        return FinOps{acc_frac[n], shifts[n], res_frac[n], out_frac[n], res[(size_t)m * ldr + n]};
    }
    __device__ inline int16_t value_of(int64_t acc, const FinOps& o) const {
        const int16_t v = clamp_i16_i64(rescale64(acc, (uint8_t)(o.sh + act_frac), o.af));
        const int64_t h = rescale64((int64_t)o.r, o.rf, o.af);
        return clamp_i16_i64(rescale64(wadd64(h, (int64_t)v), o.af, o.of));
    }
    __device__ inline void one(int n, int m, int64_t acc) const { (void)value(n, m, acc); }
};

// gate (even rows) and up (odd rows) requantized to their own fracs (mlp.rs:46-53).
struct EpiGURows : EpiApply<EpiGURows> {
    const uint8_t* shifts;
    uint8_t act_frac, gate_frac, up_frac;
    int16_t* out; int ldo;
    EpiGURows offset_m(int m0) const { EpiGURows e = *this; e.out += (size_t)m0 * ldo; return e; }
    __device__ inline void one(int n, int m, int64_t acc) const {
        const uint8_t frac = (n & 1) ? up_frac : gate_frac;
        out[(size_t)m * ldo + n] = clamp_i16_i64(rescale64(acc, (uint8_t)(shifts[n] + act_frac), frac));
    }
};

// mlp.rs:55-65 for one element: h = clamp(rescale(silu(g) * u, 8 + up_frac,
// down_in_frac)), silu(g) from the LUT over g in the LUT's input domain.
__device__ inline int32_t silu_mul(int16_t g, int16_t u, const int16_t* __restrict__ silu, uint32_t silu_len,
                                   uint8_t gate_frac, uint8_t up_frac, uint8_t down_in_frac) {
    const int32_t g_dom = rescale32((int32_t)g, gate_frac, MYL_TV_SILU_IN_FRAC);
    const int16_t act = lut_lookup_i16((int16_t)g_dom, silu, silu_len, (int16_t)MYL_TV_SILU_LUT_OFFSET);
    const int64_t prod = (int64_t)act * (int64_t)u;
    return clamp_i16_i64(rescale64(prod, (uint8_t)(MYL_TV_SILU_OUT_FRAC + up_frac), down_in_frac));
}

// The gate/up product fused with the SiLU gate and the byte-plane split of
// its output (mm2_staged_kernel): weight rows 2i (gate) and 2i+1 (up) are
// requantized to their own fracs, staged, and each 8-element chunk of
// h = silu(g) * u leaves as one 8-byte hi row piece (planes[2m][i0..]) and one
// lo' piece (planes[2m+1][i0..]) of the down product's operand [2M x I]
// (I % 8 == 0).
struct EpiGUSiluPlanes {
    const uint8_t* shifts;
    uint8_t act_frac, gate_frac, up_frac, down_in_frac;
    const int16_t* silu; uint32_t silu_len;
    int8_t* planes; int I;
    __device__ inline int16_t stage(int n, int64_t acc) const { return stage_with(op(n), n, acc); }
    // the same in two steps: the row's operand, fetched ahead of the sum
    using Op = uint8_t;
    __device__ inline Op op(int n) const { return shifts[n]; }
    __device__ inline int16_t stage_with(Op sh, int n, int64_t acc) const {
        return clamp_i16_i64(rescale64(acc, (uint8_t)(sh + act_frac), (n & 1) ? up_frac : gate_frac));
    }
    __device__ inline void emit(int m, int i0, const uint4& a, const uint4& b) const {
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};  // (g, u) pairs
        uint32_t hi[2] = {0, 0}, lo[2] = {0, 0};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int32_t h = silu_mul((int16_t)(w[k] & 0xFFFFu), (int16_t)(w[k] >> 16), silu, silu_len, gate_frac,
                                       up_frac, down_in_frac);
            hi[k >> 2] |= ((uint32_t)(h >> 8) & 0xFFu) << (8 * (k & 3));
            lo[k >> 2] |= ((uint32_t)((h & 255) - 128) & 0xFFu) << (8 * (k & 3));
        }
        *reinterpret_cast<uint2*>(planes + (size_t)(2 * m) * I + i0) = make_uint2(hi[0], hi[1]);
        *reinterpret_cast<uint2*>(planes + (size_t)(2 * m + 1) * I + i0) = make_uint2(lo[0], lo[1]);
    }
};

}  // namespace myl

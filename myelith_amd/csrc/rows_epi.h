// rows_epi.h -- epilogues of the row-batched products (batched forward, MoE):
// each maps the exact sum of weight row n and activation row m to the
// reference's requantized output (see gemm_dispatch.h for the interface).
#pragma once

#include "fixed.h"

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
    __device__ inline void one(int n, int m, int64_t acc) const {
        const uint8_t frac = n < nq ? q_frac : (n < nq + nkv ? k_frac : v_frac);
        int16_t v = clamp_i16_i64(rescale64(acc, (uint8_t)(shifts[n] + act_frac), frac));
        if (bias) v = clamp_i16_i64((int64_t)v + (int64_t)rescale32((int32_t)bias[n], bias_sh[n], frac));
        out[(size_t)m * ldo + n] = v;
    }
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
    __device__ inline void one(int n, int m, int64_t acc) const {
        const uint8_t af = acc_frac[n];
        const int16_t o = clamp_i16_i64(rescale64(acc, (uint8_t)(shifts[n] + act_frac), af));
        const int64_t h = rescale64((int64_t)res[(size_t)m * ldr + n], res_frac[n], af);
        out[(size_t)m * ldo + n] = clamp_i16_i64(rescale64(wadd64(h, (int64_t)o), af, out_frac[n]));
    }
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

}  // namespace myl

// rows_attn.h -- integer attention of batched rows on the int8 matrix cores
// (attention.rs:42-90 with softmax.rs:12-64, one sequence's KV cache per row).
//
// Rows of one sequence form a tile; a tile's G query heads per KV head are
// stacked into at most 128 query vectors (qv = row * G + head), so one block
// reads each K/V position once for all of them.  Both products run as plain
// int8 MFMAs on byte planes: an int16 x = 256*hi + lo' + 128 (hi = x >> 8,
// lo' = (x & 255) - 128), and for two such operands
//   sum_d a_d b_d = 65536*sum(ah bh) + 256*sum(ah bl' + al' bh) + sum(al' bl')
//                   + 128*sum_d a_d + 128*sum_d b_d - 16384*D
// (D terms; exact for any int16 values).  The three plane sums fit int32:
// |hi|, |lo'| <= 128, so each is at most 2^15 per term, over D <= 256 terms.
//
//   rows_qk_kernel   s_j = (i32)RNE(q . k_j * mult, shift) for j <= pos, written
//                    to scores[row][head][j]                  (attention.rs:66-67)
//   rows_probs_kernel (batch.hip) per (row, head): max, wrapping exp-LUT sum
//                    S, then p_j = RNE(e_j 2^14 / S) (or the uniform split when
//                    S = 0, softmax.rs:42-63) as int16 into probs[row][head][j];
//                    p in [0, 2^14] (a non-negative exp table whose sums do not
//                    wrap) so p >> 8 <= 64
//   rows_pv_kernel   sum_j p_j v_j exactly as int64 per 256-position range,
//                    written to part[range][row][q dim].  The range's P planes
//                    and transposed V planes are built in LDS in one phase
//                    (every load in flight at once), then the products run over
//                    its 32-position steps
//   rows_attn_out    sums the ranges, RNE by 14, clamps (attention.rs:84-86),
//                    then the attn_out rescale (model.rs:563-567)
// Each kernel's grid is (tiles, KV heads, 256-position ranges); a block whose
// range starts past every position of its tile returns at once.
#pragma once

#include "gemm_mfma.h"
#include "qk_planes.h"
#include "gemv.h"
#include "ops.h"
#include "wave.h"

namespace myl {

constexpr int kAttnTileRows = 32;  // rows a tile can list
constexpr int kAttnQV = 128;       // query vectors per tile (G x rows)
constexpr int kAttnRange = 256;    // positions per block
constexpr int kAttnThreads = 512;

struct AttnTile {
    int32_t seq, n;
    int32_t row[kAttnTileRows];
};

// LDS bytes of rows_qk_kernel: Q planes for MT*32 vectors and K planes for
// `sub` positions, MT*32 + sub <= 192 rows of (HD + 16) bytes, two planes
// (55 KB at HD 128: two blocks per CU).
template <int HD>
constexpr size_t attn_qk_lds() { return (size_t)2 * 192 * (HD + 16); }

// LDS bytes of rows_pv_kernel: P planes for QVM vectors, each a row of the
// range's positions (+16 bytes of padding), and V planes for HD dimensions,
// each a row of one pass's positions (a range in one pass for QVM = 128, in
// two passes of 128 positions for QVM = 32: 60 KB, two blocks per CU).
constexpr int attn_pv_passes(int QVM) { return QVM == kAttnQV ? 1 : 2; }
template <int HD, int QVM = kAttnQV>
constexpr size_t attn_pv_lds() {
    return (size_t)2 * QVM * (kAttnRange + 16) + (size_t)2 * HD * (kAttnRange / attn_pv_passes(QVM) + 16);
}


// Sum over the CH lanes (CH = 16 or 8, aligned rows of a wave) holding one vector.
template <int CH>
__device__ inline int32_t chunk_row_sum(int32_t v) {
    return CH == 16 ? row_sum16_i32(v) : row_sum8_i32(v);
}

// Positions per K pass: (query tiles) x (position tiles) stays at 4-8 wave tasks.
__device__ inline int attn_sub(int MT) { return MT <= 2 ? 128 : 64; }

// Row, head and position of each query vector of the block's tile.
struct AttnQv {
    int32_t row[kAttnQV], head[kAttnQV], pos[kAttnQV];
};

__device__ inline int attn_setup(const AttnTile* __restrict__ tiles, const int32_t* __restrict__ rows, int rows_cap,
                                 int G, int g, AttnQv& qv, int* s_pmax, int& QV) {
    const AttnTile* T = tiles + blockIdx.x;
    const int n = T->n;
    QV = n * G;
    const int tid = threadIdx.x;
    if (tid < QV) {
        int i = 0, h = tid;  // tid / G and tid % G without a divide (QV <= 128)
        while (h >= G) {
            h -= G;
            ++i;
        }
        const int r = T->row[i];
        qv.row[tid] = r;
        qv.head[tid] = g * G + h;
        qv.pos[tid] = rows[rows_cap + r];
    }
    if (tid == 0) {
        int pm = 0;
        for (int i = 0; i < n; ++i) pm = max(pm, rows[rows_cap + T->row[i]]);
        *s_pmax = pm;
    }
    __syncthreads();
    return T->seq;
}

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void rows_qk_kernel(
    const AttnTile* __restrict__ tiles, const int32_t* __restrict__ rows, int rows_cap, const int16_t* __restrict__ Q,
    int nq, const int16_t* __restrict__ kc, size_t seq_stride, int max_pos, int G, int64_t mult, uint8_t shift,
    int32_t* __restrict__ scores, int heads, int lcap) {
    constexpr int S = HD + 16;  // LDS row stride of a plane
    extern __shared__ __align__(16) int8_t lds[];
    __shared__ AttnQv qv;
    __shared__ int32_t q_sum[kAttnQV];
    __shared__ int32_t k_sum[256];
    __shared__ int s_pmax;
    const int g = blockIdx.y, j0 = blockIdx.z * kAttnRange;
    int QV;
    const int seq = attn_setup(tiles, rows, rows_cap, G, g, qv, &s_pmax, QV);
    const int pmax = s_pmax;
    if (j0 > pmax) return;
    const int jend = min(j0 + kAttnRange, pmax + 1);
    const int MT = (QV + 31) / 32, sub = attn_sub(MT), NT = sub / 32;
    const int nt_log = sub == 128 ? 2 : 1;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int8_t* qh = lds;
    int8_t* ql = qh + MT * 32 * S;
    int8_t* kh = ql + MT * 32 * S;
    int8_t* kl = kh + sub * S;
    constexpr int CH = HD / 8;  // 16-byte chunks per vector (a power of two)
    constexpr int CH_LOG = HD == 128 ? 4 : 3;
    // Whole CH-lane rows are active together (the bounds are multiples of
    // 64 lanes), so the row sums see every chunk of a vector.  Each staging
    // pass issues all of a thread's loads before using any.
    constexpr int kQit = kAttnQV * CH / kAttnThreads;   // Q chunks per thread
    constexpr int kKit = 128 * CH / kAttnThreads;       // K chunks per thread (sub <= 128)
    {
        uint4 qx[kQit];
#pragma unroll
        for (int i = 0; i < kQit; ++i) {
            const int t = tid + i * kAttnThreads;
            const int v = t >> CH_LOG, c = t & (CH - 1);
            qx[i] = v < QV ? *reinterpret_cast<const uint4*>(Q + (size_t)qv.row[v] * nq + (size_t)qv.head[v] * HD + c * 8)
                           : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < kQit; ++i) {
            const int t = tid + i * kAttnThreads;
            if (t >= MT * 32 * CH) break;  // wave-uniform
            const int v = t >> CH_LOG, c = t & (CH - 1);
            uint2 h, l;
            split_planes8(qx[i], h, l);
            *reinterpret_cast<uint2*>(qh + v * S + c * 8) = h;
            *reinterpret_cast<uint2*>(ql + v * S + c * 8) = l;
            const int32_t sv = chunk_row_sum<CH>(sum8_i16(qx[i]));
            if (c == 0 && v < QV) q_sum[v] = sv;
        }
    }
    const int16_t* kg = kc + (size_t)seq * seq_stride + (size_t)g * max_pos * HD;
    for (int js = j0; js < jend; js += sub) {
        uint4 kx[kKit];
#pragma unroll
        for (int i = 0; i < kKit; ++i) {
            const int t = tid + i * kAttnThreads;
            const int j = js + (t >> CH_LOG), c = t & (CH - 1);
            kx[i] = t < sub * CH && j < max_pos ? *reinterpret_cast<const uint4*>(kg + (size_t)j * HD + c * 8)
                                                : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < kKit; ++i) {
            const int t = tid + i * kAttnThreads;
            if (t >= sub * CH) break;  // wave-uniform
            const int p = t >> CH_LOG, c = t & (CH - 1);
            uint2 h, l;
            split_planes8(kx[i], h, l);
            *reinterpret_cast<uint2*>(kh + p * S + c * 8) = h;
            *reinterpret_cast<uint2*>(kl + p * S + c * 8) = l;
            const int32_t sk = chunk_row_sum<CH>(sum8_i16(kx[i]));
            if (c == 0) k_sum[p] = sk;
        }
        __syncthreads();
        for (int task = wave; task < MT * NT; task += kAttnThreads / 64) {
            const int mt = task >> nt_log, nt = task & (NT - 1);
            v16i32_t hh, mid, ll;
#pragma unroll
            for (int r = 0; r < 16; ++r) hh[r] = mid[r] = ll[r] = 0;
            const int ar = mt * 32 + (lane & 31), br = nt * 32 + (lane & 31);
#pragma unroll
            for (int ks = 0; ks < HD / 32; ++ks) {
                const int off = ks * 32 + 16 * (lane >> 5);
                const v4i32_t ah = *reinterpret_cast<const v4i32_t*>(qh + ar * S + off);
                const v4i32_t al = *reinterpret_cast<const v4i32_t*>(ql + ar * S + off);
                const v4i32_t bh = *reinterpret_cast<const v4i32_t*>(kh + br * S + off);
                const v4i32_t bl = *reinterpret_cast<const v4i32_t*>(kl + br * S + off);
                hh = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, bh, hh, 0, 0, 0);
                mid = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, bl, mid, 0, 0, 0);
                mid = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, bh, mid, 0, 0, 0);
                ll = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, bl, ll, 0, 0, 0);
            }
            // lane: position column br; registers r: vectors 8*(r/4) + 4*(lane/32) + r%4
            const int j = js + br;
            const int64_t kterm = 128 * (int64_t)k_sum[br] - 16384 * (int64_t)HD;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int v = mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (v < QV && j <= qv.pos[v]) {
                    const int64_t dot = 65536 * (int64_t)hh[r] + 256 * (int64_t)mid[r] + (int64_t)ll[r] +
                                        128 * (int64_t)q_sum[v] + kterm;
                    scores[((size_t)qv.row[v] * heads + qv.head[v]) * lcap + j] =
                        (int32_t)rshift_round64(wmul64(dot, mult), shift);
                }
            }
        }
        __syncthreads();  // the next pass overwrites the K planes
    }
}

template <int HD, bool LOOP, int QVM = kAttnQV>
__global__ __launch_bounds__(kAttnThreads) void rows_pv_kernel(
    const AttnTile* __restrict__ tiles, const int32_t* __restrict__ rows, int rows_cap,
    const int16_t* __restrict__ probs /* [row][head][lcap] */, int heads, int lcap, const int16_t* __restrict__ vc,
    size_t seq_stride, int max_pos, int G, int64_t* __restrict__ part, size_t part_stride, int nq,
    uint8_t v_frac, uint8_t out_frac, int16_t* __restrict__ A, int8_t* __restrict__ planes) {
    static_assert(QVM == kAttnQV || QVM == 32, "tile widths");
    constexpr int RS = kAttnRange + 16;  // LDS row stride of a P plane: the range's positions of one vector
    constexpr int VP = attn_pv_passes(QVM);
    constexpr int PW = kAttnRange / VP;   // positions per V pass
    constexpr int RSV = PW + 16;          // LDS row stride of a V plane: one pass's positions of a dimension
    constexpr int SLOTS = PW / 16;        // 16-byte position chunks per V row (the swizzle's range)
    constexpr int NT = HD / 32;
    constexpr int CH = HD / 8, CH_LOG = HD == 128 ? 4 : 3;
    extern __shared__ __align__(16) int8_t lds[];
    int8_t* ph = lds;
    int8_t* pl = ph + QVM * RS;
    int8_t* vh = pl + QVM * RS;
    int8_t* vl = vh + HD * RSV;
    __shared__ AttnQv qv;
    __shared__ int32_t p_sum[QVM], v_sum[HD];
    __shared__ int s_pmax;
    const int g = blockIdx.y;
    int QV;
    const int seq = attn_setup(tiles, rows, rows_cap, G, g, qv, &s_pmax, QV);
    const int pmax = s_pmax;
    // one range (blockIdx.z), or every range of the tile in turn (LOOP)
    const int r_first = LOOP ? 0 : (int)blockIdx.z;
    const int r_last = LOOP ? pmax / kAttnRange : (int)blockIdx.z;
    if (r_first * kAttnRange > pmax || QV > QVM) return;  // the launcher picks QVM >= every tile's QV
    const int MT = (QV + 31) / 32;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ntask = MT * NT;
    // exact P.V sums of the block's (vector, dimension) outputs over its ranges
    int64_t tot[2][16];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r) tot[a][r] = 0;
    for (int range = r_first; range <= r_last; ++range) {
        const int j0 = range * kAttnRange;
        const int nk = (min(j0 + kAttnRange, pmax + 1) - j0 + 31) / 32;  // 32-position steps
        if (tid < HD) v_sum[tid] = 0;
        __syncthreads();
        // Every probability load of the wave and every V load of the thread is
        // issued before any of them is used (one memory latency instead of one
        // per vector and per item).
        constexpr int kVpw = QVM / (kAttnThreads / 64);               // vectors per wave
        constexpr int kGroups = PW / 4;                                // 4-position groups per V pass
        constexpr int kVit = (CH * kGroups + kAttnThreads - 1) / kAttnThreads;  // V items per thread
        const int q4 = lane, jb = j0 + 4 * q4;
        uint2 pv4[kVpw];
#pragma unroll
        for (int i = 0; i < kVpw; ++i) {
            const int v = wave + i * (kAttnThreads / 64);
            pv4[i] = make_uint2(0, 0);
            if (q4 < 8 * nk && v < QV && jb <= qv.pos[v])
                pv4[i] = *reinterpret_cast<const uint2*>(probs + ((size_t)qv.row[v] * heads + qv.head[v]) * lcap + jb);
        }
        const int16_t* vg = vc + (size_t)seq * seq_stride + (size_t)g * max_pos * HD;
        uint4 vw[kVit][4];
        // V of pass vp: item t = (8-dimension chunk c, 4-position group vq4)
        auto load_v = [&](int vp) {
#pragma unroll
            for (int i = 0; i < kVit; ++i) {
                const int t = tid + i * kAttnThreads;
                const int c = t & (CH - 1), vq4 = t >> CH_LOG;
                const bool ok = t < CH * kGroups && vp * kGroups + vq4 < 8 * nk;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int j = j0 + vp * PW + 4 * vq4 + k;
                    vw[i][k] = ok && j < max_pos ? *reinterpret_cast<const uint4*>(vg + (size_t)j * HD + c * 8)
                                                 : make_uint4(0, 0, 0, 0);
                }
            }
        };
        load_v(0);
        // P planes [vector][position]: a wave per vector, its lanes over the
        // range's 4-position groups (8 * nk <= 64 of them)
#pragma unroll
        for (int i = 0; i < kVpw; ++i) {
            const int v = wave + i * (kAttnThreads / 64);
            if (v >= MT * 32) break;  // wave-uniform
            uint32_t hw = 0, lw = 0x80808080u;  // p = 0: hi 0, lo' -128
            int32_t ps = 0;
            if (q4 < 8 * nk && v < QV && jb <= qv.pos[v]) {
                const int pos = qv.pos[v];
                const uint32_t pw[2] = {pv4[i].x, pv4[i].y};
                lw = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    // positions past the row's own are not its probabilities
                    const int32_t p =
                        jb + k <= pos ? (int32_t)(int16_t)((k & 1) ? (pw[k >> 1] >> 16) : (pw[k >> 1] & 0xFFFFu)) : 0;
                    ps += p;
                    hw |= ((uint32_t)(p >> 8) & 0xFFu) << (8 * k);
                    lw |= ((uint32_t)((p & 255) - 128) & 0xFFu) << (8 * k);
                }
            }
            if (q4 < 8 * nk) {
                *reinterpret_cast<uint32_t*>(ph + v * RS + 4 * q4) = hw;
                *reinterpret_cast<uint32_t*>(pl + v * RS + 4 * q4) = lw;
            }
            ps = wave_sum_i32(ps);
            if (lane == 0) p_sum[v] = ps;
        }
        // wave tasks: (query tile, dimension tile) pairs, at most two per wave
        v16i32_t acc[2][3];
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 3; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[a][b][r] = 0;
#pragma unroll
        for (int vp = 0; vp < VP; ++vp) {
            if (vp > 0) {
                __syncthreads();  // the previous pass's V planes are consumed
                load_v(vp);
            }
            // V planes transposed to [dimension][position]: 8 dimensions x 4
            // positions per item; 16-byte position chunk (vq4 >> 2) at slot
            // chunk ^ ((d >> 3) % SLOTS), so rows eight apart do not share banks
#pragma unroll
            for (int i = 0; i < kVit; ++i) {
                const int t = tid + i * kAttnThreads;
                const int c = t & (CH - 1), vq4 = t >> CH_LOG;
                if (t >= CH * kGroups || vp * kGroups + vq4 >= 8 * nk) continue;
                const uint4 (&w)[4] = vw[i];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    uint32_t hw = 0, lw = 0;
                    int32_t vs = 0;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint32_t word =
                            (e >> 1) == 0 ? w[k].x : ((e >> 1) == 1 ? w[k].y : ((e >> 1) == 2 ? w[k].z : w[k].w));
                        const int32_t x = (int16_t)((e & 1) ? (word >> 16) : (word & 0xFFFFu));
                        vs += x;
                        hw |= ((uint32_t)(x >> 8) & 0xFFu) << (8 * k);
                        lw |= ((uint32_t)((x & 255) - 128) & 0xFFu) << (8 * k);
                    }
                    const int d = c * 8 + e;
                    const int off = (((vq4 >> 2) ^ (c & (SLOTS - 1))) << 4) + 4 * (vq4 & 3);
                    *reinterpret_cast<uint32_t*>(vh + d * RSV + off) = hw;
                    *reinterpret_cast<uint32_t*>(vl + d * RSV + off) = lw;
                    atomicAdd(&v_sum[d], vs);
                }
            }
            __syncthreads();
            const int k0 = vp * (PW / 32), k1 = min(nk, k0 + PW / 32);  // this pass's 32-position steps
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                const int task = wave + a * (kAttnThreads / 64);
                if (task >= ntask) continue;
                const int mt = task / NT, nt = task - mt * NT;
                const int8_t* ah_row = ph + (mt * 32 + (lane & 31)) * RS + 16 * (lane >> 5);
                const int8_t* al_row = pl + (mt * 32 + (lane & 31)) * RS + 16 * (lane >> 5);
                const int dr = nt * 32 + (lane & 31);
                const int8_t* bh_row = vh + dr * RSV;
                const int8_t* bl_row = vl + dr * RSV;
                const int sw = (dr >> 3) & (SLOTS - 1);
                for (int kk = k0; kk < k1; ++kk) {
                    const int slot = ((2 * (kk - k0) + (lane >> 5)) ^ sw) << 4;
                    const v4i32_t ah = *reinterpret_cast<const v4i32_t*>(ah_row + 32 * kk);
                    const v4i32_t al = *reinterpret_cast<const v4i32_t*>(al_row + 32 * kk);
                    const v4i32_t bh = *reinterpret_cast<const v4i32_t*>(bh_row + slot);
                    const v4i32_t bl = *reinterpret_cast<const v4i32_t*>(bl_row + slot);
                    acc[a][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, bh, acc[a][0], 0, 0, 0);
                    acc[a][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, bl, acc[a][1], 0, 0, 0);
                    acc[a][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, bh, acc[a][1], 0, 0, 0);
                    acc[a][2] = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, bl, acc[a][2], 0, 0, 0);
                }
            }
        }
        const int64_t cterm = 16384 * 32 * (int64_t)nk;
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            const int task = wave + a * (kAttnThreads / 64);
            if (task >= ntask) continue;
            const int mt = task / NT, nt = task - mt * NT;
            const int d = nt * 32 + (lane & 31);
            const int64_t dterm = 128 * (int64_t)v_sum[d] - cterm;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int v = mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                tot[a][r] = wadd64(tot[a][r], 65536 * (int64_t)acc[a][0][r] + 256 * (int64_t)acc[a][1][r] +
                                                  (int64_t)acc[a][2][r] + 128 * (int64_t)p_sum[v] + dterm);
            }
        }
        __syncthreads();  // the next range overwrites the planes, p_sum and v_sum
    }
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        const int task = wave + a * (kAttnThreads / 64);
        if (task >= ntask) continue;
        const int mt = task / NT, nt = task - mt * NT;
        const int d = nt * 32 + (lane & 31);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int v = mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (v >= QV) continue;
            const size_t o = (size_t)qv.row[v] * nq + (size_t)qv.head[v] * HD + d;
            if (!LOOP) {
                part[(size_t)r_first * part_stride + o] = tot[a][r];
                continue;
            }
            // attention.rs:84-86 then model.rs:563-567 (as rows_attn_out_kernel)
            const int16_t vv = clamp_i16_i64(rshift_round64(tot[a][r], MYL_TV_PROB_FRAC_BITS));
            const int16_t av = clamp_i16(rescale32((int32_t)vv, v_frac, out_frac));
            if (planes) {
                const size_t ro = (size_t)qv.row[v] * 2 * nq + (size_t)qv.head[v] * HD + d;
                planes[ro] = (int8_t)(av >> 8);
                planes[ro + nq] = (int8_t)((av & 255) - 128);
            } else {
                A[o] = av;
            }
        }
    }
}

// attention.rs:84-86 then model.rs:563-567: the ranges' exact sums, one
// rounding, the attn_out rescale; into A, or as byte planes when planes is
// given.  Grid (ceil(nq / 256), R); nranges is the range count of the P.V
// launch (every range slot it names lies in part).  The partials of all
// nranges slots are loaded together, without waiting for the row's length,
// which then selects the ranges the row's P.V blocks wrote.
__global__ __launch_bounds__(256) void rows_attn_out_kernel(const int64_t* __restrict__ part, size_t part_stride,
                                                            const int32_t* __restrict__ rows, int rows_cap, int nq,
                                                            int nranges, uint8_t v_frac, uint8_t out_frac,
                                                            int16_t* __restrict__ A, int8_t* __restrict__ planes) {
    constexpr int kBatch = 16;  // range slots loaded before the first add
    const int r = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= nq) return;
    const int nr = rows[rows_cap + r] / kAttnRange + 1;
    const int64_t* pr = part + (size_t)r * nq + i;
    int64_t s = 0;
    for (int c0 = 0; c0 < nranges; c0 += kBatch) {
        int64_t v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) v[k] = c0 + k < nranges ? pr[(size_t)(c0 + k) * part_stride] : 0;
#pragma unroll
        for (int k = 0; k < kBatch; ++k) s = wadd64(s, c0 + k < nr ? v[k] : 0);
    }
    const int16_t v = clamp_i16_i64(rshift_round64(s, MYL_TV_PROB_FRAC_BITS));
    const int16_t a = clamp_i16(rescale32((int32_t)v, v_frac, out_frac));
    if (planes) {  // byte planes [2R x nq] for the o_proj product
        planes[(size_t)(2 * r) * nq + i] = (int8_t)(a >> 8);
        planes[(size_t)(2 * r + 1) * nq + i] = (int8_t)((a & 255) - 128);
    } else {
        A[(size_t)r * nq + i] = a;
    }
}

}  // namespace myl

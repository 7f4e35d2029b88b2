// int4 affine (group 64) expert kernels for gfx950.
//
// Weight layout (reference state layout, metal_q4_decode_v4.py:161-169): codes u32 [E, N, K/8] with
// nibble i of word j = element 8j+i, scales / biases bf16 [E, N, K/64]; w = s*q + b.
//
// Dot products run on v_dot2_f32_bf16: a 16-byte chunk of 32 codes is decoded to bf16 pairs holding
// 128+q (exact), dotted with bf16 activation pairs, and the offset is folded into the bias:
//   sum_k (s q_k + b) x_k = s * sum_k (128 + q_k) x_k + (b - 128 s) * sum_k x_k      (per 32-chunk)
// Products of bf16 pairs are exact in fp32; accumulation is fp32.
//
// The GLU output h is kept at fp32 precision as two bf16 planes, h = hi + lo (hi = bf16(h), lo = bf16(h - hi),
// |h - hi - lo| <= 2^-18 |h|), so the down projection runs on v_dot2_f32_bf16 twice per pair instead of
// losing 2^-9 of h to a bf16 store.
//
// Per-slot path (T == 1, and the stock-style per-slot gather at T > 1; reference metal_q4_decode_v4.py):
//   q4_gate_up_slots: one wave per RW rows of one slot; lanes stride over 16-byte chunks of the rows,
//                     gate and up rows of the same index are read together so SwiGLU runs in-wave.
//   q4_down_slots:    LPR lanes per down row, 4 waves split the slots of a token and reduce in LDS
//                     straight into y (no partial buffer, no combine launch).
// Grouped path (T > 1; reference metal_q4_tiles_v2.py): one block per (active expert, row block) reads
//   the expert's rows once and applies them to up to NB of its slots per pass; down writes weighted fp32
//   partials per slot and q4_combine sums the k slots of each token.
#include "moe_common.h"
#include "moe_internal.h"

namespace moe {

constexpr int GU_WAVES = 4;
constexpr int DN_WAVES = 4;

// ------------------------------------------------------------------------------------------ helpers
__device__ __forceinline__ float q4_fold(float acc, float s, float b, float dot, float xsum) {
    // acc + s*dot + (b - 128 s) * xsum
    const float beff = __builtin_fmaf(-MOE_Q4_OFFSET, s, b);
    return __builtin_fmaf(s, dot, __builtin_fmaf(beff, xsum, acc));
}

// store h as hi/lo bf16 planes
__device__ __forceinline__ void store_h(uint16_t* hhi, uint16_t* hlo, size_t i, float v) {
    const uint16_t hi = f32_to_bf16(v);
    hhi[i] = hi;
    hlo[i] = f32_to_bf16(v - bf16_to_f32(hi));
}

// one 32-element chunk of h (both planes) against decoded codes: returns sum (128+q) h, and sum h in *hs
__device__ __forceinline__ float dot_h32(const uint32_t qp[16], const uint16_t* hhi, const uint16_t* hlo, float* hs) {
    uint32_t hw[16], hp[16];
    load_x32(hhi, hw);
    pair_x32(hw, hp);
    float s = sum_x32(hw);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc = dot2_bf16(qp[i], hp[i], acc);
    load_x32(hlo, hw);
    pair_x32(hw, hp);
    s += sum_x32(hw);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc = dot2_bf16(qp[i], hp[i], acc);
    *hs = s;
    return acc;
}

// output store in the caller's dtype (bf16 or fp32)
__device__ __forceinline__ void store_y(void* y, size_t i, float v, int y32) {
    if (y32) reinterpret_cast<float*>(y)[i] = v;
    else reinterpret_cast<uint16_t*>(y)[i] = f32_to_bf16(v);
}
__device__ __forceinline__ float load_y(const void* y, size_t i, int y32) {
    return y32 ? reinterpret_cast<const float*>(y)[i] : bf16_to_f32(reinterpret_cast<const uint16_t*>(y)[i]);
}

__device__ __forceinline__ void decode_q4x32(uint4 w, uint32_t qp[16]) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) qp[4 * j + i] = q4pair_bf16(ws[j], i);
}

__device__ __forceinline__ float dot_pairs16(const uint32_t qp[16], const uint32_t xp[16]) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc = dot2_bf16(qp[i], xp[i], acc);
    return acc;
}

// ------------------------------------------------------------------------------ per-slot gate / up
// grid (ceil(F / (GU_WAVES*RW)), T*k), block 64*GU_WAVES. h planes [T*k, F].
template <int RW, int ACT>
__global__ void __launch_bounds__(64 * GU_WAVES)
q4_gate_up_slots(const uint16_t* __restrict__ x, const uint32_t* __restrict__ gq, const uint16_t* __restrict__ gs,
                 const uint16_t* __restrict__ gb, const uint32_t* __restrict__ uq, const uint16_t* __restrict__ us,
                 const uint16_t* __restrict__ ub, const float* __restrict__ bg, const float* __restrict__ bu,
                 const int32_t* __restrict__ idx, int k, int d, int F, int E, uint16_t* __restrict__ hhi,
                 uint16_t* __restrict__ hlo) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int slot = blockIdx.y;
    const int row0 = (blockIdx.x * GU_WAVES + wave) * RW;
    if (row0 >= F) return;
    const int e = idx[slot];
    const bool valid = (unsigned)e < (unsigned)E;
    const int t = slot / k;
    const int nchunk = d >> 5, ngrp = d >> 6, wpr = d >> 3;
    float ag[RW], au[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) ag[r] = au[r] = 0.f;
    if (valid) {
        const uint16_t* xr = x + (size_t)t * d;
        for (int c = lane; c < nchunk; c += 64) {
            uint4 wg[RW], wu[RW];
            float sg[RW], zg[RW], su[RW], zu[RW];
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const int n = min(row0 + r, F - 1);
                const size_t row = (size_t)e * F + n;
                wg[r] = reinterpret_cast<const uint4*>(gq + row * wpr)[c];
                wu[r] = reinterpret_cast<const uint4*>(uq + row * wpr)[c];
                sg[r] = bf16_to_f32(gs[row * ngrp + (c >> 1)]);
                zg[r] = bf16_to_f32(gb[row * ngrp + (c >> 1)]);
                su[r] = bf16_to_f32(us[row * ngrp + (c >> 1)]);
                zu[r] = bf16_to_f32(ub[row * ngrp + (c >> 1)]);
            }
            uint32_t xw[16], xp[16];
            load_x32(xr + c * 32, xw);
            pair_x32(xw, xp);
            const float xs = sum_x32(xw);
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                ag[r] = q4_fold(ag[r], sg[r], zg[r], dot_q4x32(wg[r], xp), xs);
                au[r] = q4_fold(au[r], su[r], zu[r], dot_q4x32(wu[r], xp), xs);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        ag[r] = wave_sum(ag[r]);
        au[r] = wave_sum(au[r]);
    }
    if (lane < RW) {
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int r = 0; r < RW; ++r)
            if (r == lane) { g = ag[r]; u = au[r]; }
        const int n = row0 + lane;
        if (n < F) {
            float hv = 0.f;
            if (valid) {
                if (bg) g += bg[(size_t)e * F + n];
                if (bu) u += bu[(size_t)e * F + n];
                hv = glu<ACT>(g, u);
            }
            store_h(hhi, hlo, (size_t)slot * F + n, hv);
        }
    }
}

// ------------------------------------------------------------------------------------ per-slot down
// grid (ceil(D / RPW), T), block 64*DN_WAVES; RPW = 64 / LPR rows per block, the 4 waves split the k slots.
// y [T, D] (or [T*k, D] unweighted when nored), fp32 when y32 else bf16; resid has y's dtype.
template <int LPR>
__global__ void __launch_bounds__(64 * DN_WAVES)
q4_down_slots(const uint16_t* __restrict__ hhi, const uint16_t* __restrict__ hlo, const uint32_t* __restrict__ dq,
              const uint16_t* __restrict__ ds, const uint16_t* __restrict__ db, const float* __restrict__ bd,
              const int32_t* __restrict__ idx, const float* __restrict__ wts, int k, int D, int F, int E, int nored,
              int y32, const void* __restrict__ resid, void* __restrict__ y) {
    constexpr int RPW = 64 / LPR;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = blockIdx.y;
    const int rsub = lane / LPR, psub = lane % LPR;
    const int n = blockIdx.x * RPW + rsub;
    const bool row_ok = n < D;
    const int nn = row_ok ? n : D - 1;
    const int cpr = F >> 5, ngrp = F >> 6, wpr = F >> 3;
    float yacc = 0.f;
    for (int j = wave; j < k; j += DN_WAVES) {
        const int slot = t * k + j;
        const int e = idx[slot];
        if ((unsigned)e >= (unsigned)E) {
            if (nored && psub == 0 && row_ok) store_y(y, (size_t)slot * D + n, 0.f, y32);
            continue;
        }
        const size_t row = (size_t)e * D + nn;
        const uint4* wrow = reinterpret_cast<const uint4*>(dq + row * wpr);
        const size_t hoff = (size_t)slot * F;
        float acc = 0.f;
        for (int p0 = psub; p0 < cpr; p0 += 4 * LPR) {
            uint4 wv[4];
            float s[4], z[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = min(p0 + i * LPR, cpr - 1);
                wv[i] = wrow[p];
                s[i] = bf16_to_f32(ds[row * ngrp + (p >> 1)]);
                z[i] = bf16_to_f32(db[row * ngrp + (p >> 1)]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = p0 + i * LPR;
                if (p < cpr) {
                    uint32_t qp[16];
                    decode_q4x32(wv[i], qp);
                    float hs;
                    const float dd = dot_h32(qp, hhi + hoff + p * 32, hlo + hoff + p * 32, &hs);
                    acc = q4_fold(acc, s[i], z[i], dd, hs);
                }
            }
        }
        acc = group_sum<LPR>(acc);
        if (bd) acc += bd[(size_t)e * D + nn];
        if (nored) {
            if (psub == 0 && row_ok) store_y(y, (size_t)slot * D + n, acc, y32);
        } else {
            yacc = __builtin_fmaf(wts[slot], acc, yacc);
        }
    }
    if (nored) return;
    __shared__ float red[DN_WAVES][RPW];
    if (psub == 0) red[wave][rsub] = yacc;
    __syncthreads();
    if (wave == 0 && lane < RPW) {
        const int n2 = blockIdx.x * RPW + lane;
        if (n2 < D) {
            float v = red[0][lane];
#pragma unroll
            for (int w = 1; w < DN_WAVES; ++w) v += red[w][lane];
            const size_t o = (size_t)t * D + n2;
            if (resid) v += load_y(resid, o, y32);
            store_y(y, o, v, y32);
        }
    }
}

// ------------------------------------------------------------------------------- grouped gate / up
// grid (ceil(F / (GU_WAVES*RW)), max_active), block 64*GU_WAVES. Block (rb, a) handles rows of expert
// active[a] for all of its slots, NB slots per pass: each weight chunk is decoded once per pass.
template <int RW, int NB, int ACT>
__global__ void __launch_bounds__(64 * GU_WAVES)
q4_gate_up_grouped(const uint16_t* __restrict__ x, const uint32_t* __restrict__ gq, const uint16_t* __restrict__ gs,
                   const uint16_t* __restrict__ gb, const uint32_t* __restrict__ uq, const uint16_t* __restrict__ us,
                   const uint16_t* __restrict__ ub, const float* __restrict__ bg, const float* __restrict__ bu,
                   const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
                   const int32_t* __restrict__ sorted, const int32_t* __restrict__ active,
                   const int32_t* __restrict__ meta, int k, int d, int F, uint16_t* __restrict__ hhi,
                   uint16_t* __restrict__ hlo) {
    const int a = blockIdx.y;
    if (a >= meta[0]) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * GU_WAVES + wave) * RW;
    if (row0 >= F) return;
    const int e = active[a];
    const int beg = offsets[e], cnt = counts[e];
    const int nchunk = d >> 5, ngrp = d >> 6, wpr = d >> 3;
    for (int tb = 0; tb < cnt; tb += NB) {
        const int nb = min(NB, cnt - tb);
        int slot[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) slot[i] = sorted[beg + tb + min(i, nb - 1)];
        float ag[RW][NB], au[RW][NB];
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int i = 0; i < NB; ++i) ag[r][i] = au[r][i] = 0.f;
        for (int c = lane; c < nchunk; c += 64) {
            uint4 wg[RW], wu[RW];
            float sg[RW], zg[RW], su[RW], zu[RW];
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const int n = min(row0 + r, F - 1);
                const size_t row = (size_t)e * F + n;
                wg[r] = reinterpret_cast<const uint4*>(gq + row * wpr)[c];
                wu[r] = reinterpret_cast<const uint4*>(uq + row * wpr)[c];
                sg[r] = bf16_to_f32(gs[row * ngrp + (c >> 1)]);
                zg[r] = bf16_to_f32(gb[row * ngrp + (c >> 1)]);
                su[r] = bf16_to_f32(us[row * ngrp + (c >> 1)]);
                zu[r] = bf16_to_f32(ub[row * ngrp + (c >> 1)]);
            }
            uint32_t xp[NB][16];
            float xs[NB];
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                uint32_t xw[16];
                load_x32(x + (size_t)(slot[i] / k) * d + c * 32, xw);
                pair_x32(xw, xp[i]);
                xs[i] = sum_x32(xw);
            }
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                uint32_t qg[16], qu[16];
                decode_q4x32(wg[r], qg);
                decode_q4x32(wu[r], qu);
#pragma unroll
                for (int i = 0; i < NB; ++i) {
                    ag[r][i] = q4_fold(ag[r][i], sg[r], zg[r], dot_pairs16(qg, xp[i]), xs[i]);
                    au[r][i] = q4_fold(au[r][i], su[r], zu[r], dot_pairs16(qu, xp[i]), xs[i]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                ag[r][i] = wave_sum(ag[r][i]);
                au[r][i] = wave_sum(au[r][i]);
            }
        // lane (r*NB + i) writes row r of slot i
        if (lane < RW * NB) {
            float g = 0.f, u = 0.f;
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int i = 0; i < NB; ++i)
                    if (r * NB + i == lane) { g = ag[r][i]; u = au[r][i]; }
            const int r = lane / NB, i = lane % NB;
            const int n = row0 + r;
            if (n < F && i < nb) {
                if (bg) g += bg[(size_t)e * F + n];
                if (bu) u += bu[(size_t)e * F + n];
                int s_i = 0;
#pragma unroll
                for (int q = 0; q < NB; ++q)
                    if (q == i) s_i = slot[q];
                store_h(hhi, hlo, (size_t)s_i * F + n, glu<ACT>(g, u));
            }
        }
    }
}

// ------------------------------------------------------------------------------------ grouped down
// grid (ceil(D / (DN_WAVES*RPW)), max_active), block 64*DN_WAVES; each wave owns RPW rows of the block.
// yp [T*k, D] fp32: yp[slot] = wts[slot] * (W_d h[slot] + bd).
template <int LPR, int NB>
__global__ void __launch_bounds__(64 * DN_WAVES)
q4_down_grouped(const uint16_t* __restrict__ hhi, const uint16_t* __restrict__ hlo, const uint32_t* __restrict__ dq,
                const uint16_t* __restrict__ ds, const uint16_t* __restrict__ db, const float* __restrict__ bd,
                const float* __restrict__ wts, const int32_t* __restrict__ counts,
                const int32_t* __restrict__ offsets, const int32_t* __restrict__ sorted,
                const int32_t* __restrict__ active, const int32_t* __restrict__ meta, int D, int F,
                float* __restrict__ yp) {
    constexpr int RPW = 64 / LPR;
    const int a = blockIdx.y;
    if (a >= meta[0]) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rsub = lane / LPR, psub = lane % LPR;
    const int n = (blockIdx.x * DN_WAVES + wave) * RPW + rsub;
    const bool row_ok = n < D;
    const int nn = row_ok ? n : D - 1;
    const int e = active[a];
    const int beg = offsets[e], cnt = counts[e];
    const int cpr = F >> 5, ngrp = F >> 6, wpr = F >> 3;
    const size_t row = (size_t)e * D + nn;
    const uint4* wrow = reinterpret_cast<const uint4*>(dq + row * wpr);
    const float bias_n = bd ? bd[row] : 0.f;
    for (int tb = 0; tb < cnt; tb += NB) {
        const int nb = min(NB, cnt - tb);
        int slot[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) slot[i] = sorted[beg + tb + min(i, nb - 1)];
        float acc[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) acc[i] = 0.f;
        for (int p0 = psub; p0 < cpr; p0 += 2 * LPR) {
            uint4 wv[2];
            float s[2], z[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int p = min(p0 + q * LPR, cpr - 1);
                wv[q] = wrow[p];
                s[q] = bf16_to_f32(ds[row * ngrp + (p >> 1)]);
                z[q] = bf16_to_f32(db[row * ngrp + (p >> 1)]);
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int p = p0 + q * LPR;
                if (p < cpr) {
                    uint32_t qp[16];
                    decode_q4x32(wv[q], qp);
#pragma unroll
                    for (int i = 0; i < NB; ++i) {
                        float hs;
                        const size_t ho = (size_t)slot[i] * F + p * 32;
                        const float dd = dot_h32(qp, hhi + ho, hlo + ho, &hs);
                        acc[i] = q4_fold(acc[i], s[q], z[q], dd, hs);
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) acc[i] = group_sum<LPR>(acc[i]);
        if (psub == 0 && row_ok) {
#pragma unroll
            for (int i = 0; i < NB; ++i)
                if (i < nb) yp[(size_t)slot[i] * D + n] = wts[slot[i]] * (acc[i] + bias_n);
        }
    }
}

// ------------------------------------------------------------------------------------------ combine
// y[t, n] = residual[t, n] + sum_j yp[t*k + j, n], 4 outputs per thread (D % 4 == 0); y, resid bf16 or fp32.
__global__ void __launch_bounds__(256)
moe_combine(const float* __restrict__ yp, const void* __restrict__ resid, void* __restrict__ y, int T, int k, int D,
            int y32) {
    const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t total4 = (size_t)T * D / 4;
    if (i4 >= total4) return;
    const size_t i = i4 * 4;
    const int t = (int)(i / D), n = (int)(i % D);
    float4 acc = reinterpret_cast<const float4*>(yp + ((size_t)t * k) * D + n)[0];
    for (int j = 1; j < k; ++j) {
        const float4 v = reinterpret_cast<const float4*>(yp + ((size_t)t * k + j) * D + n)[0];
        acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    if (y32) {
        if (resid) {
            const float4 r = reinterpret_cast<const float4*>(resid)[i4];
            acc.x += r.x; acc.y += r.y; acc.z += r.z; acc.w += r.w;
        }
        reinterpret_cast<float4*>(y)[i4] = acc;
        return;
    }
    if (resid) {
        const uint2 r = reinterpret_cast<const uint2*>(resid)[i4];
        acc.x += bf16lo(r.x); acc.y += bf16hi(r.x); acc.z += bf16lo(r.y); acc.w += bf16hi(r.y);
    }
    uint2 o;
    o.x = (uint32_t)f32_to_bf16(acc.x) | ((uint32_t)f32_to_bf16(acc.y) << 16);
    o.y = (uint32_t)f32_to_bf16(acc.z) | ((uint32_t)f32_to_bf16(acc.w) << 16);
    reinterpret_cast<uint2*>(y)[i4] = o;
}

// ------------------------------------------------------------------------------------ host side
static int pick_lpr(int cpr) {
    // lanes per down row: smallest power of two >= cpr / 3 (about three 16-byte chunks per lane), in [4, 64]
    int l = 4;
    while (l < 64 && l * 3 < cpr) l *= 2;
    return l;
}

template <int ACT>
static void launch_gu_slots(const ExpertsArgs& a, int RW, dim3 grid) {
    const moe_experts_t* w = a.w;
    auto* x = (const uint16_t*)a.x;
    auto* gq = (const uint32_t*)w->gate.codes;
    auto* gs = (const uint16_t*)w->gate.scales;
    auto* gb = (const uint16_t*)w->gate.biases;
    auto* uq = (const uint32_t*)w->up.codes;
    auto* us = (const uint16_t*)w->up.scales;
    auto* ub = (const uint16_t*)w->up.biases;
    if (RW == 4)
        q4_gate_up_slots<4, ACT><<<grid, 64 * GU_WAVES, 0, a.st>>>(x, gq, gs, gb, uq, us, ub, w->gate.bias,
                                                                  w->up.bias, a.idx, a.k, w->d, w->F, w->E, a.hhi,
                                                                  a.hlo);
    else
        q4_gate_up_slots<2, ACT><<<grid, 64 * GU_WAVES, 0, a.st>>>(x, gq, gs, gb, uq, us, ub, w->gate.bias,
                                                                  w->up.bias, a.idx, a.k, w->d, w->F, w->E, a.hhi,
                                                                  a.hlo);
}

int run_int4_slots(const ExpertsArgs& a) {
    const moe_experts_t* w = a.w;
    const int d = w->d, F = w->F, E = w->E;
    const int nslots = a.T * a.k;
    // gate/up: RW rows per wave; fewer rows per wave when the launch would be short of waves
    const int RW = ((long)nslots * F / 4 >= 1024) ? 4 : 2;
    if (a.stages & 1) {
        dim3 g1((F + GU_WAVES * RW - 1) / (GU_WAVES * RW), nslots);
        if (a.act == 0) launch_gu_slots<0>(a, RW, g1);
        else if (a.act == 1) launch_gu_slots<1>(a, RW, g1);
        else launch_gu_slots<2>(a, RW, g1);
        if (hipGetLastError() != hipSuccess) return MOE_ERR_LAUNCH;
    }
    if (!(a.stages & 2)) return 0;

    const int lpr = pick_lpr(F >> 5);
    const int rpw = 64 / lpr;
    dim3 g2((d + rpw - 1) / rpw, a.T);
    auto* dq = (const uint32_t*)w->down.codes;
    auto* ds = (const uint16_t*)w->down.scales;
    auto* db = (const uint16_t*)w->down.biases;
#define MOE_DN(L)                                                                                              \
    q4_down_slots<L><<<g2, 64 * DN_WAVES, 0, a.st>>>(a.hhi, a.hlo, dq, ds, db, w->down.bias, a.idx, a.wts, a.k, \
                                                      d, F, E, a.nored, a.y32, a.residual, a.y)
    switch (lpr) {
        case 4: MOE_DN(4); break;
        case 8: MOE_DN(8); break;
        case 16: MOE_DN(16); break;
        case 32: MOE_DN(32); break;
        default: MOE_DN(64); break;
    }
#undef MOE_DN
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

template <int ACT>
static void launch_gu_grouped(const ExpertsArgs& a, dim3 grid) {
    const moe_experts_t* w = a.w;
    constexpr int RW = 2, NB = 4;
    q4_gate_up_grouped<RW, NB, ACT><<<grid, 64 * GU_WAVES, 0, a.st>>>(
        (const uint16_t*)a.x, (const uint32_t*)w->gate.codes, (const uint16_t*)w->gate.scales,
        (const uint16_t*)w->gate.biases, (const uint32_t*)w->up.codes, (const uint16_t*)w->up.scales,
        (const uint16_t*)w->up.biases, w->gate.bias, w->up.bias, a.grp.counts, a.grp.offsets, a.grp.sorted,
        a.grp.active, a.grp.meta, a.k, w->d, w->F, a.hhi, a.hlo);
}

int run_int4_grouped(const ExpertsArgs& a) {
    const moe_experts_t* w = a.w;
    const int d = w->d, F = w->F, E = w->E;
    const int nslots = a.T * a.k;
    const int max_active = nslots < E ? nslots : E;
    if (a.stages & 1) {
        int rc = launch_group(a.idx, nslots, E, a.grp.counts, a.grp.offsets, a.grp.sorted, a.grp.active, a.grp.meta,
                              a.st);
        if (rc) return rc;
        constexpr int RW = 2;
        dim3 g1((F + GU_WAVES * RW - 1) / (GU_WAVES * RW), max_active);
        if (a.act == 0) launch_gu_grouped<0>(a, g1);
        else if (a.act == 1) launch_gu_grouped<1>(a, g1);
        else launch_gu_grouped<2>(a, g1);
        if (hipGetLastError() != hipSuccess) return MOE_ERR_LAUNCH;
    }
    if (!(a.stages & 2)) return 0;

    const int lpr = pick_lpr(F >> 5);
    const int rpw = 64 / lpr;
    dim3 g2((d + DN_WAVES * rpw - 1) / (DN_WAVES * rpw), max_active);
    auto* dq = (const uint32_t*)w->down.codes;
    auto* ds = (const uint16_t*)w->down.scales;
    auto* db = (const uint16_t*)w->down.biases;
#define MOE_DNG(L)                                                                                                \
    q4_down_grouped<L, 4><<<g2, 64 * DN_WAVES, 0, a.st>>>(a.hhi, a.hlo, dq, ds, db, w->down.bias, a.wts,         \
                                                           a.grp.counts, a.grp.offsets, a.grp.sorted, a.grp.active, \
                                                           a.grp.meta, d, F, a.yp)
    switch (lpr) {
        case 4: MOE_DNG(4); break;
        case 8: MOE_DNG(8); break;
        case 16: MOE_DNG(16); break;
        case 32: MOE_DNG(32); break;
        default: MOE_DNG(64); break;
    }
#undef MOE_DNG
    if (hipGetLastError() != hipSuccess) return MOE_ERR_LAUNCH;
    return launch_combine(a.yp, a.residual, a.y, a.T, a.k, d, a.y32, a.st);
}

int launch_combine(const float* yp, const void* residual, void* y, int T, int k, int d, int y32, hipStream_t st) {
    const size_t total4 = (size_t)T * d / 4;
    if (total4 == 0) return 0;
    dim3 grid((unsigned)((total4 + 255) / 256));
    moe_combine<<<grid, 256, 0, st>>>(yp, residual, y, T, k, d, y32);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

}  // namespace moe

// Expert kernels for gfx950 (MI355X): int4 affine g64 and MXFP4, SwiGLU / GeGLU / gpt-oss clamped GLU.
//
// Packed rows. Every weight row of K inputs is one record in HBM (moe_row_bytes): K/2 bytes of 4-bit
// codes (word j holds inputs 8j..8j+7, low nibble first, as the reference's state words,
// metal_q4_decode_v4.py:57-64), then the row's group metadata, padded to 16 bytes:
//   int4 g64: K/64 words (scale bf16 | bias bf16 << 16), w = scale*q + bias
//   MXFP4:    K/32 E8M0 bytes, w = e2m1(q) * 2^(s-127)  (reference metal_mxfp4_moe.py:1-41)
// A lane reads a 16-byte chunk (32 inputs) with one dwordx4 load and its metadata with one more load
// from the same record, so a row streams from one DRAM page.
//
// Arithmetic. A chunk is decoded to 16 bf16 pairs and dotted with bf16 activation pairs on
// v_dot2_f32_bf16 (exact products, fp32 accumulation):
//   int4:  pairs hold 128 + q (exact: the ulp of 128 in bf16 is 1), and per 32-chunk
//          sum_k (s q_k + b) x_k = s * sum_k (128 + q_k) x_k + (b - 128 s) * sum_k x_k
//   MXFP4: pairs hold e2m1(q) from two v_perm_b32 byte lookups, and the chunk's dot is scaled by
//          2^(s-127) in fp32 (one E8M0 group = one chunk).
// Pairs are (input 8j+i, input 8j+i+4): the activation side is paired the same way (pair_x32). The MXFP4
// per-slot rows (k_gate_up_rows, k_down_rows) take the converts' natural pairs (2i, 2i+1) instead, against x
// and h in natural order: no v_perm per code word and no pairing of x (FmtMxfp4::ROWS_NAT).
//
// The GLU output h (gate/up -> down) is kept at ~16 significant bits as two bf16 planes h = hi + lo,
// stored pre-paired (element n of a chunk at (n & ~7) | (n & 3) << 1 | (n >> 2) & 1), so the down
// projection loads ready-made pairs (MXFP4 rows: natural order; with the gpt-oss GLU one fp16 plane, h_is_f16).
//
// Kernels:
//   k_gate_up_slots / k_down_slots   per-slot GEMV (any T; the stock-style per-slot gather at T > 1)
//   k_combine                        y = residual + sum over a token's slots of wts * (yp + b_down); the
//                                    combine step of the grouped expert tiles (moe_tiles.hip)
#include "moe_common.h"
#include "moe_formats.h"
#include "moe_internal.h"

namespace moe {

// ============================================================================ activation planes
// fp16 and fp32 activations enter the expert kernels as NX bf16 planes whose sum is the value exactly: each plane
// takes the next 8 significant bits by truncation (plane = the top 16 bits of the remainder's fp32 pattern;
// the remainder after it is exact in fp32), so fp16 (11 bits) needs 2 planes and fp32 (24 bits) 3. inf and NaN
// go whole into plane 0 (NaN quieted), the other planes 0. The kernels run one product per plane against the
// same decoded weights and sum them in fp32, so every input bit reaches the accumulator.
// planes [NX][n] bf16, plane = n elements apart; one thread per 8 elements (n % 8 == 0).
template <int XDT>
__global__ void __launch_bounds__(256) k_x_planes(const void* __restrict__ x, uint16_t* __restrict__ planes,
                                                  size_t n8, size_t plane) {
    constexpr int NX = XDT == MOE_DTYPE_F16 ? 2 : 3;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    float v[8];
    if (XDT == MOE_DTYPE_F16) {
        const uint4 r = reinterpret_cast<const uint4*>(x)[i];
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v[2 * q] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[q] & 0xFFFFu));
            v[2 * q + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[q] >> 16));
        }
    } else {
        const float4 a = reinterpret_cast<const float4*>(x)[2 * i], b = reinterpret_cast<const float4*>(x)[2 * i + 1];
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    }
    uint32_t bits[8][NX];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float r = v[e];
        const bool fin = __builtin_isfinite(r);
#pragma unroll
        for (int p = 0; p < NX; ++p) {
            const uint32_t top = __float_as_uint(r) & 0xFFFF0000u;
            bits[e][p] = fin ? top >> 16 : (p == 0 ? (uint32_t)f32_to_bf16(r) : 0u);
            r = fin ? r - __uint_as_float(top) : 0.f;
        }
    }
    uint32_t out[NX][4];
#pragma unroll
    for (int p = 0; p < NX; ++p)
#pragma unroll
        for (int q = 0; q < 4; ++q) out[p][q] = bits[2 * q][p] | (bits[2 * q + 1][p] << 16);
#pragma unroll
    for (int p = 0; p < NX; ++p)
        reinterpret_cast<uint4*>(planes + p * plane)[i] = make_uint4(out[p][0], out[p][1], out[p][2], out[p][3]);
}



// ============================================================================ per-slot gate / up, balanced
// Work item q = slot * F + f: gate row f and up row f of expert idx[slot]. Wave gw = 4 * blockIdx.x + wave
// takes items gw*R .. gw*R + R - 1; R divides F, so they are R consecutive row pairs of one slot, and every
// wave (and every block) carries the same bytes. Lane l covers the 16-byte chunks l, l + 64, ... of a row,
// NCH of them per pass. Order of memory operations: the expert id (scalar load), the x chunks of the first
// pass (L2), then every weight chunk and metadata word of the pass, all before the first use; the math then
// runs in load order, so it overlaps with the loads still arriving. h is written as the two pre-paired bf16
// planes hi/lo (store_h).
// HX activation planes (bf16 x: 1; fp16 / fp32 x: k_x_planes' 2 or 3 planes, xplane elements apart): every plane
// is dotted with the same decoded chunk and the products add in fp32.
// One wave: gate and up rows f0 .. f0 + R - 1 of slot s's expert; lanes 48..63 write h.
// Routed (RJM > 0: RJM = ceil(E / 64) logits per lane): the expert is round s % k of the router tail over token
// s / k's logits, which the wave selects itself (topk_rank_id: that round alone, no earlier rounds); the wave with
// s % k == 0 and f0 == 0 also runs the whole tail (topk_core) once its weight loads are in flight, and writes the
// token's idx / wts for the down kernel and the caller.
struct RouteArgs {
    const float* logits;   // [T, E] fp32, or null: the expert ids come from idx
    int norm;
    float scale;
    int32_t* idx;          // outputs when routed
    float* wts;
};
template <class FMT, int R, int NCH, int HX, int RJM>
__device__ __forceinline__ void gate_up_rows_wave(const uint16_t* __restrict__ x, size_t xplane,
                                                  const uint8_t* __restrict__ G, const uint8_t* __restrict__ U,
                                                  const float* __restrict__ bg, const float* __restrict__ bu,
                                                  const int32_t* __restrict__ idx, int k, int d, int F, int E,
                                                  int act, uint16_t* __restrict__ hhi, uint16_t* __restrict__ hlo,
                                                  int s, int f0, int lane, const RouteArgs& rt = RouteArgs{}) {
    static_assert(R <= 16, "results live in lanes 48..63");
    const int nchunk = d >> 5;
    const uint16_t* xr = x + (size_t)(s / k) * d;
    int ch[NCH];
    bool cv[NCH];
    uint32_t xw[HX][NCH][16];
    auto load_x = [&](int c0) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            ch[c] = c0 + 64 * c + lane;
            cv[c] = ch[c] < nchunk;
            ch[c] = cv[c] ? ch[c] : nchunk - 1;
#pragma unroll
            for (int h = 0; h < HX; ++h) load_x32(xr + h * xplane + 32 * ch[c], xw[h][c]);
        }
    };
    load_x(0);   // x does not depend on the expert: its first loads go out before the expert id or router tail
    int e;
    constexpr int LJ = RJM > 0 ? RJM : 1;
    float lv[LJ];   // routed: the token's logits, logit j * 64 + lane in lv[j]
    const int tok = s / k;
    const bool writer = RJM > 0 && s - tok * k == 0 && f0 == 0;
    if constexpr (RJM > 0) {
        const float* lrow = rt.logits + (size_t)tok * E;
#pragma unroll
        for (int j = 0; j < LJ; ++j) lv[j] = j * 64 + lane < E ? lrow[j * 64 + lane] : -INFINITY;
        e = __builtin_amdgcn_readfirstlane((int)topk_rank_id<LJ>(lv, E, s - tok * k));
    } else {
        e = idx[s];   // wave-uniform: a scalar load
    }
    const size_t rb = rbytes(FMT::FMT, d);
    float ag[R], au[R];
#pragma unroll
    for (int r = 0; r < R; ++r) ag[r] = au[r] = 0.f;
    const bool valid = (unsigned)e < (unsigned)E;
    const int ee = valid ? e : 0;
    const uint8_t* gb0 = G + ((size_t)ee * F + f0) * rb;
    const uint8_t* ub0 = U + ((size_t)ee * F + f0) * rb;
    const int rl = lane - 48;
    float bgl = 0.f, bul = 0.f;
    for (int c0 = 0; c0 < nchunk; c0 += 64 * NCH) {
        if (c0) load_x(c0);
        uint4 wg[R][NCH], wu[R][NCH];
        uint32_t mg[R][NCH], mu[R][NCH];
        // 32-bit byte offsets from the wave-uniform row bases (R <= 16 rows of one record each)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const uint32_t ro = (uint32_t)(r * rb);
                wg[r][c] = *reinterpret_cast<const uint4*>(gb0 + (ro + 16u * (uint32_t)ch[c]));
                mg[r][c] = FMT::meta_at(gb0, ro + FMT::meta_off(d, ch[c]));
                wu[r][c] = *reinterpret_cast<const uint4*>(ub0 + (ro + 16u * (uint32_t)ch[c]));
                mu[r][c] = FMT::meta_at(ub0, ro + FMT::meta_off(d, ch[c]));
            }
        __builtin_amdgcn_sched_barrier(0);   // every load of the pass is in flight before any use
        // the lane that writes row f0 + (lane - 48) fetches its additive biases (gpt-oss) once the first pass's
        // weight loads are out: their pointers' kernel-argument load and its wait stay off the weights' path
        if (c0 == 0 && valid && rl >= 0 && rl < R) {
            if (bg) bgl = bg[(size_t)e * F + f0 + rl];
            if (bu) bul = bu[(size_t)e * F + f0 + rl];
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (RJM > 0) {
            // the token's whole tail, for idx / wts, while the weights arrive (it reads only registers)
            if (writer && c0 == 0) {
                uint32_t id;
                float w;
                topk_core<LJ>(lv, E, k, rt.norm, rt.scale, k, &id, &w);
                if (lane < k) {
                    rt.idx[(size_t)tok * k + lane] = (int32_t)id;
                    rt.wts[(size_t)tok * k + lane] = w;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        uint32_t xp[HX][NCH][16];
        float xs[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            xs[c] = 0.f;
#pragma unroll
            for (int h = 0; h < HX; ++h) {
                if constexpr (FMT::ROWS_NAT) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) xp[h][c][i] = xw[h][c][i];
                } else {
                    pair_x32(xw[h][c], xp[h][c]);
                }
                xs[c] = FMT::XSUM ? sum_x32(xw[h][c]) + xs[c] : 0.f;
            }
        }
        auto dotx = [&](const uint32_t (&qp)[16], int c) __attribute__((always_inline)) {
            float dd = 0.f;
#pragma unroll
            for (int h = 0; h < HX; ++h) dd = dot16(qp, xp[h][c], dd);
            return dd;
        };
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                uint32_t qp[16];
                FMT::decode_rows(wg[r][c], qp);
                const float dg = FMT::fold(0.f, mg[r][c], dotx(qp, c), xs[c]);
                FMT::decode_rows(wu[r][c], qp);
                const float du = FMT::fold(0.f, mu[r][c], dotx(qp, c), xs[c]);
                ag[r] += cv[c] ? dg : 0.f;
                au[r] += cv[c] ? du : 0.f;
            }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        ag[r] = sum_lanes<64>(ag[r]);
        au[r] = sum_lanes<64>(au[r]);
    }
    if (rl >= 0 && rl < R) {   // lanes 48..63 hold the sums
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int q = 0; q < R; ++q)
            if (q == rl) { g = ag[q]; u = au[q]; }
        const float hv = valid ? glu_act(act, g + bgl, u + bul) : 0.f;
        if (h_is_f16(FMT::FMT, act)) store_h16(hhi, (size_t)s * F, f0 + rl, hv, FMT::ROWS_NAT);
        else store_h(hhi, hlo, (size_t)s * F, f0 + rl, hv, FMT::ROWS_NAT);
    }
}

// Argument order: what the prologue needs before the first weight load (x, G, U, idx, k, d, F, Q, E) sits in the
// first 64 bytes of the kernel arguments, so the wave's scalar loads of them are one scalar-cache line.
template <class FMT, int R, int NCH, int HX, int RJM>
__global__ void __launch_bounds__(256)
k_gate_up_rows(const uint16_t* __restrict__ x, const uint8_t* __restrict__ G, const uint8_t* __restrict__ U,
               const int32_t* __restrict__ idx, int k, int d, int F, int Q, int E, int act, size_t xplane,
               const float* __restrict__ bg, const float* __restrict__ bu, uint16_t* __restrict__ hhi,
               uint16_t* __restrict__ hlo, RouteArgs rt) {
    // routed: every pointer argument is read into SGPRs at entry (one scalar-cache fill and one wait). Left to the
    // compiler, some of these loads sink past the rank search, and their wait (which covers every scalar load then
    // in flight) lands between the search and the first weight load. Not in the plain instance: an asm statement
    // before the expert id's load turns that scalar load into a vector load with a full wait.
    if constexpr (RJM > 0)
        asm volatile("" ::"s"(x), "s"(G), "s"(U), "s"(bg), "s"(bu), "s"(hhi), "s"(hlo), "s"(rt.logits), "s"(rt.idx),
                     "s"(rt.wts));
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int q0 = (blockIdx.x * 4 + wave) * R;
    if (q0 >= Q) return;
    const int s = q0 / F, f0 = q0 - s * F;
    gate_up_rows_wave<FMT, R, NCH, HX, RJM>(x, xplane, G, U, bg, bu, idx, k, d, F, E, act, hhi, hlo, s, f0, lane, rt);
}

// ============================================================================ per-slot down, h staged in LDS
#ifndef MOE_DN_PF_MAX
#define MOE_DN_PF_MAX 6   // h words per thread loaded ahead of the weights (k_down_rows)
#endif
// grid (ceil(D / RB), T), block 64 * NW (NW waves); every block computes RB = NW * RR rows of y[t] over all
// k slots of token t. Lane l of a wave: chunk phase p = l % L, slot j = l / L (64 / L >= k slot lanes, L a
// power of two), so one wave covers every (slot, chunk) pair of its RR rows, and the k-reduction is an
// in-wave DPP sum. A lane handles chunks p, p + L, ..., p + (NC-1) L of rows n .. n + RR - 1 and reuses
// each h chunk for the RR rows. The pre-paired h planes of the k slots are copied once per block into LDS
// (coalesced: consecutive lanes load consecutive 16-byte words), with each chunk's sum (the int4 fold needs it)
// in a ninth 16-byte word: a chunk record is 144 bytes, so the records of 16 consecutive chunks start on 16
// distinct 16-byte bank groups (144 = 9 x 16, 9 odd) and the math's ds_read_b128 of 16 lanes on consecutive
// chunks is free of bank conflicts (a 128-byte record puts every second chunk on the same 4 banks: an 8-way
// conflict). Order of memory operations: the lane's expert id and routing weight, the first staged h words
// (L2), every weight chunk and metadata word of the lane (branch-free: chunk indices past the row are clamped
// into it and masked out of the math), the LDS staging, then the math in load order.
// H16 (h_is_f16: MXFP4 with the gpt-oss GLU): h is one fp16 plane in hhi; a record is its 64 bytes plus one
// 16-byte pad word (80 = 5 x 16, 5 odd: the same bank spread), the codes decode to fp16 and the dots run on
// v_dot2_f32_f16, one per pair instead of two.
template <class FMT, int NC, int RR, int NW, bool H16 = false>
__global__ void __launch_bounds__(64 * NW)
k_down_rows(const uint16_t* __restrict__ hhi, const uint16_t* __restrict__ hlo, const uint8_t* __restrict__ Dw,
            const float* __restrict__ bd, const int32_t* __restrict__ idx, const float* __restrict__ wts, int k,
            int D, int F, int E, int lgL, int nored, int ydt, const void* __restrict__ resid,
            void* __restrict__ y) {
    static_assert(!H16 || !FMT::XSUM, "fp16 h: no chunk sums (MXFP4)");
    constexpr int SL = sum_lane<64>();
    constexpr int RB = NW * RR;
    constexpr int REC = H16 ? 5 : 9;   // 16-byte words per staged chunk record
    extern __shared__ uint4 s_dyn[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int t = blockIdx.y;
    const int L = 1 << lgL;
    const int p = lane & (L - 1), j = lane >> lgL;
    const int cpr = F >> 5;
    const int nch = k * cpr;   // chunks of h to stage
    uint4* s_h = s_dyn;   // [nch][REC]: hi pairs x4, lo pairs x4, {chunk sum, pad}; H16: fp16 pairs x4, pad
    // ---- expert id and routing weight of this lane's slot
    const bool jv = j < k;
    const int slot = t * k + (jv ? j : k - 1);
    const int e = idx[slot];
    const float wraw = wts[slot];
    // the id's load goes out first: the weight addresses wait on it, and the memory counter drains in issue order,
    // so an h load issued ahead of it would be waited for as well
    __builtin_amdgcn_sched_barrier(0);
    // ---- first staged words of this thread (L2): 16-byte word u of the token's hi and lo planes, u = thread +
    // m * block size, consecutive lanes on consecutive words (word u is quarter u & 3 of chunk u >> 2). The
    // token's k F / 8 words number at most 256 NC (k <= 64 / L slots of cpr <= NC L chunks, 4 words each), so
    // ceil(4 NC / NW) words per thread take them all in the first round trip (up to MOE_DN_PF_MAX)
    constexpr int PF = (4 * NC + NW - 1) / NW < MOE_DN_PF_MAX ? (4 * NC + NW - 1) / NW : MOE_DN_PF_MAX;
    const size_t hbase = (size_t)t * k * F;
    const uint4* h4 = reinterpret_cast<const uint4*>(hhi + hbase);
    const uint4* l4 = reinterpret_cast<const uint4*>(hlo + hbase);
    const int nu = nch * 4;
    uint4 hv[2 * PF];
#pragma unroll
    for (int m = 0; m < PF; ++m) {
        const int u = min((int)threadIdx.x + m * 64 * NW, nu - 1);
        hv[2 * m] = h4[u];
        if constexpr (!H16) hv[2 * m + 1] = l4[u];
    }
    // ---- weights of this lane
    const bool ev = jv && (unsigned)e < (unsigned)E;
    const int ee = ev ? e : 0;
    const size_t rb = rbytes(FMT::FMT, F);
    // row blocks XCD by XCD: blocks b = c (mod 8) run on one XCD, and XCD slot c takes a contiguous range of the
    // nb = ceil(D / RB) row blocks, so the cache line two neighbouring blocks' records share (a record is not a
    // whole number of lines) is fetched into one L2
    int rbk;
    {
        const int nb = (D + RB - 1) / RB, q8 = nb >> 3, r8 = nb & 7, c = (int)(blockIdx.x & 7u), m = (int)(blockIdx.x >> 3);
        rbk = (c < r8 ? c * (q8 + 1) : r8 * (q8 + 1) + (c - r8) * q8) + m;
    }
    const int n0 = rbk * RB + wave * RR;
    // the residual of the wave's output rows (added by the storing lane at the end), loaded with the first
    // loads so that no memory round trip follows the reduction
    uint32_t rres[RR];
#pragma unroll
    for (int i = 0; i < RR; ++i) rres[i] = resid ? load_y_bits(resid, (size_t)t * D + min(n0 + i, D - 1), ydt) : 0u;
    const uint8_t* rows[RR];
#pragma unroll
    for (int i = 0; i < RR; ++i) rows[i] = Dw + ((size_t)ee * D + min(n0 + i, D - 1)) * rb;
    float bdv[RR];
#pragma unroll
    for (int i = 0; i < RR; ++i) bdv[i] = (bd && ev && p == 0) ? bd[(size_t)e * D + min(n0 + i, D - 1)] : 0.f;
    uint4 wv[NC][RR];
    uint32_t mv[NC][RR];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int chk = min(p + c * L, cpr - 1);
#pragma unroll
        for (int i = 0; i < RR; ++i) {
            wv[c][i] = *reinterpret_cast<const uint4*>(rows[i] + 16 * chk);
            mv[c][i] = FMT::meta(rows[i], F, chk);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // ---- stage h: the prefetched words, then any further ones (only when k * F > 32 * PF * block size). The
    // four lanes of a chunk are consecutive lanes of one wave and always active together (nu and the block size
    // are multiples of 4), so the chunk sum (int4 fold) is a quad reduction.
    auto put = [&](int u, const uint4& a, const uint4& b) __attribute__((always_inline)) {
        uint4* r = s_h + (size_t)(u >> 2) * REC;
        r[u & 3] = a;
        if constexpr (!H16) r[4 + (u & 3)] = b;
        if (FMT::XSUM) {
            float sm = 0.f;
            sm = dot2_bf16(a.x, 0x3f803f80u, sm);
            sm = dot2_bf16(a.y, 0x3f803f80u, sm);
            sm = dot2_bf16(a.z, 0x3f803f80u, sm);
            sm = dot2_bf16(a.w, 0x3f803f80u, sm);
            sm = dot2_bf16(b.x, 0x3f803f80u, sm);
            sm = dot2_bf16(b.y, 0x3f803f80u, sm);
            sm = dot2_bf16(b.z, 0x3f803f80u, sm);
            sm = dot2_bf16(b.w, 0x3f803f80u, sm);
            sm += __shfl_xor(sm, 1, 64);
            sm += __shfl_xor(sm, 2, 64);
            if ((u & 3) == 0) reinterpret_cast<float*>(r + 8)[0] = sm;
        }
    };
#pragma unroll
    for (int m = 0; m < PF; ++m) {
        const int u = (int)threadIdx.x + m * 64 * NW;
        if (u < nu) put(u, hv[2 * m], hv[2 * m + 1]);
    }
    for (int u = (int)threadIdx.x + PF * 64 * NW; u < nu; u += 64 * NW) {
        if constexpr (H16) put(u, h4[u], uint4{});
        else put(u, h4[u], l4[u]);
    }
    __syncthreads();
    // ---- math
    float acc[RR];
#pragma unroll
    for (int i = 0; i < RR; ++i) acc[i] = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int chk = p + c * L;
        const bool cv = ev && chk < cpr;
        const size_t hc = (size_t)(jv ? j : 0) * cpr + min(chk, cpr - 1);
        uint32_t wh[16], wl[16];
        words16(&s_h[hc * REC], wh);
        if constexpr (!H16) words16(&s_h[hc * REC + 4], wl);
        const float hs = FMT::XSUM ? reinterpret_cast<const float*>(s_h + hc * REC + 8)[0] : 0.f;
#pragma unroll
        for (int i = 0; i < RR; ++i) {
            uint32_t qp[16];
            float dd;
            if constexpr (H16) {
                FMT::decode_rows_f16(wv[c][i], qp);
                dd = dot16_f16(qp, wh, 0.f);
            } else {
                FMT::decode_rows(wv[c][i], qp);
                dd = dot16(qp, wl, dot16(qp, wh, 0.f));
            }
            const float v = FMT::fold(0.f, mv[c][i], dd, hs);
            acc[i] += cv ? v : 0.f;
        }
    }
    if constexpr (H16) {
#pragma unroll
        for (int i = 0; i < RR; ++i) acc[i] *= 1.0f / MOE_H16_SCALE;   // a power of two: exact
    }
    if (nored) {
#pragma unroll
        for (int i = 0; i < RR; ++i) {
            const int n = n0 + i;
            float v = acc[i] + bdv[i];
            // sum over the L lanes of the slot: xor butterfly within the group
            for (int s2 = 1; s2 < L; s2 <<= 1) v += __shfl_xor(v, s2, 64);
            if (p == 0 && jv && n < D) store_y(y, (size_t)slot * D + n, v, ydt);
        }
        return;
    }
    const float wj = ev ? wraw : 0.f;
#pragma unroll
    for (int i = 0; i < RR; ++i) {
        const int n = n0 + i;
        const float v = sum_lanes<64>((acc[i] + bdv[i]) * wj);
        if (lane == SL && n < D) store_y(y, (size_t)t * D + n, resid ? v + y_bits_f32(rres[i], ydt) : v, ydt);
    }
}

// ============================================================================ per-slot gate / up
// grid (ceil(F / (4*NR)), T*k), block 256: wave w of block (bx, slot) computes gate and up rows
// row0 .. row0+NR-1 of expert idx[slot]; the 64 lanes stride over the 16-byte chunks of the rows.
template <class FMT, int ACT, int NR, int HX>
__global__ void __launch_bounds__(256)
k_gate_up_slots(const uint16_t* __restrict__ x, size_t xplane, const uint8_t* __restrict__ G, const uint8_t* __restrict__ U,
                const float* __restrict__ bg, const float* __restrict__ bu, const int32_t* __restrict__ idx, int k,
                int d, int F, int E, uint16_t* __restrict__ hhi, uint16_t* __restrict__ hlo) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int slot = blockIdx.y;
    const int row0 = (blockIdx.x * 4 + wave) * NR;
    if (row0 >= F) return;
    const int e = idx[slot];
    const bool valid = (unsigned)e < (unsigned)E;
    const size_t rb = rbytes(FMT::FMT, d);
    const int nchunk = d >> 5;
    float ag[NR], au[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) ag[r] = au[r] = 0.f;
    if (valid) {
        const uint16_t* xr = x + (size_t)(slot / k) * d;
        const uint8_t* gb0 = G + ((size_t)e * F + row0) * rb;
        const uint8_t* ub0 = U + ((size_t)e * F + row0) * rb;
        for (int c0 = 0; c0 < nchunk; c0 += 64) {
            const bool cv = c0 + lane < nchunk;
            const int c = cv ? c0 + lane : nchunk - 1;
            uint4 wg[NR], wu[NR];
            uint32_t mg[NR], mu[NR], xw[HX][16];
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const size_t ro = (size_t)min(r, F - 1 - row0) * rb;
                wg[r] = *reinterpret_cast<const uint4*>(gb0 + ro + 16 * c);
                wu[r] = *reinterpret_cast<const uint4*>(ub0 + ro + 16 * c);
                mg[r] = FMT::meta(gb0 + ro, d, c);
                mu[r] = FMT::meta(ub0 + ro, d, c);
            }
#pragma unroll
            for (int h = 0; h < HX; ++h) load_x32(xr + h * xplane + 32 * c, xw[h]);
            __builtin_amdgcn_sched_barrier(0);   // every load above is in flight before any use
            uint32_t xp[HX][16];
            float xs = 0.f;
#pragma unroll
            for (int h = 0; h < HX; ++h) {
                pair_x32(xw[h], xp[h]);
                xs = FMT::XSUM ? sum_x32(xw[h]) + xs : 0.f;
            }
            auto dotx = [&](const uint32_t (&qp)[16]) __attribute__((always_inline)) {
                float dd = 0.f;
#pragma unroll
                for (int h = 0; h < HX; ++h) dd = dot16(qp, xp[h], dd);
                return dd;
            };
            if (cv) {
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    uint32_t qp[16];
                    FMT::decode(wg[r], qp);
                    ag[r] = FMT::fold(ag[r], mg[r], dotx(qp), xs);
                    FMT::decode(wu[r], qp);
                    au[r] = FMT::fold(au[r], mu[r], dotx(qp), xs);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        ag[r] = sum_lanes<64>(ag[r]);
        au[r] = sum_lanes<64>(au[r]);
    }
    const int r = lane - 48;   // lanes 48..63 hold the sums
    if (r >= 0 && r < NR && row0 + r < F) {
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int q = 0; q < NR; ++q)
            if (q == r) { g = ag[q]; u = au[q]; }
        float hv = 0.f;
        if (valid) {
            if (bg) g += bg[(size_t)e * F + row0 + r];
            if (bu) u += bu[(size_t)e * F + row0 + r];
            hv = glu<ACT>(g, u);
        }
        store_h(hhi, hlo, (size_t)slot * F, row0 + r, hv);
    }
}

// ============================================================================ per-slot down
// grid (ceil(D / RPW), T), block 64*NW (NW = min(k, 8) waves): wave j handles slot t*k + j (and j + NW, ...)
// for RPW = 64/LPR rows (LPR lanes per row, NC chunks per lane: NC*LPR >= F/32). All of a slot's loads
// (weight chunks, metadata, pre-paired h) are issued before any use; the waves reduce their slots in LDS
// into y[t] (or write unweighted per-slot rows, nored).
template <class FMT, int LPR, int NC>
__global__ void __launch_bounds__(512)
k_down_slots(const uint16_t* __restrict__ hhi, const uint16_t* __restrict__ hlo, const uint8_t* __restrict__ Dw,
             const float* __restrict__ bd, const int32_t* __restrict__ idx, const float* __restrict__ wts, int k, int D,
             int F, int E, int nored, int ydt, const void* __restrict__ resid, void* __restrict__ y) {
    constexpr int RPW = 64 / LPR;
    constexpr int SL = sum_lane<LPR>();
    __shared__ float red[8][RPW];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nw = blockDim.x >> 6;
    const int t = blockIdx.y;
    const int rsub = lane / LPR, psub = lane % LPR;
    const int n = blockIdx.x * RPW + rsub;
    const bool row_ok = n < D;
    const int nn = row_ok ? n : D - 1;
    const size_t rb = rbytes(FMT::FMT, F);
    const int cpr = F >> 5;
    // the residual of the output row wave 0's lane stores at the end, loaded before the slots' loads
    const int nr = blockIdx.x * RPW + lane;
    const uint32_t rres = resid && !nored && wave == 0 && lane < RPW && nr < D ? load_y_bits(resid, (size_t)t * D + nr, ydt) : 0u;
    float yacc = 0.f;
    for (int j = wave; j < k; j += nw) {
        const int slot = t * k + j;
        const int e = idx[slot];
        if ((unsigned)e >= (unsigned)E) {
            if (nored && psub == SL && row_ok) store_y(y, (size_t)slot * D + n, 0.f, ydt);
            continue;
        }
        const uint8_t* rowp = Dw + ((size_t)e * D + nn) * rb;
        const uint4* hh = reinterpret_cast<const uint4*>(hhi + (size_t)slot * F);
        const uint4* hl = reinterpret_cast<const uint4*>(hlo + (size_t)slot * F);
        constexpr int NG = NC < 4 ? NC : 4;   // chunks whose loads are in flight together
        float acc = 0.f;
#pragma unroll
        for (int g0 = 0; g0 < NC; g0 += NG) {
            uint4 wv[NG], vh[NG][4], vl[NG][4];
            uint32_t m[NG];
#pragma unroll
            for (int i = 0; i < NG; ++i) {
                const int p = min(psub + (g0 + i) * LPR, cpr - 1);
                wv[i] = *reinterpret_cast<const uint4*>(rowp + 16 * p);
                m[i] = FMT::meta(rowp, F, p);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    vh[i][q] = hh[4 * p + q];
                    vl[i][q] = hl[4 * p + q];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < NG; ++i) {
                if (psub + (g0 + i) * LPR < cpr) {
                    uint32_t qp[16], wh[16], wl[16];
                    FMT::decode(wv[i], qp);
                    words16(vh[i], wh);
                    words16(vl[i], wl);
                    const float dt = dot16(qp, wl, dot16(qp, wh, 0.f));
                    const float hs = FMT::XSUM ? sum16(wl, sum16(wh, 0.f)) : 0.f;
                    acc = FMT::fold(acc, m[i], dt, hs);
                }
            }
        }
        acc = sum_lanes<LPR>(acc);
        if (bd) acc += bd[(size_t)e * D + nn];
        if (nored) {
            if (psub == SL && row_ok) store_y(y, (size_t)slot * D + n, acc, ydt);
        } else {
            yacc = __builtin_fmaf(wts[slot], acc, yacc);
        }
    }
    if (nored) return;
    if (psub == SL) red[wave][rsub] = yacc;
    __syncthreads();
    if (wave == 0 && lane < RPW) {
        const int n2 = blockIdx.x * RPW + lane;
        if (n2 < D) {
            float v = red[0][lane];
            for (int w = 1; w < nw; ++w) v += red[w][lane];
            store_y(y, (size_t)t * D + n2, resid ? v + y_bits_f32(rres, ydt) : v, ydt);
        }
    }
}

// ============================================================================ combine
// y[t, n] = residual[t, n] + sum_j wts[t, j] * (yp[t*k + j, n] (+ yp2[t*k + j, n], a second K part) +
// bd[idx[t, j], n]); slots whose id is outside
// [0, E) add nothing. 4 outputs per thread (D % 4 == 0). The slots are taken KC at a time (KC: k rounded up to a
// power of two, at most 8): their ids and weights first, then every yp row (and bias row) load of the KC at once
// (rows of skipped slots are read too, then discarded by a select, so no load waits on an id), then the sums in slot
// order.
template <int KC>
__global__ void __launch_bounds__(256)
k_combine(const float* __restrict__ yp, int nplanes, size_t plane, const int32_t* __restrict__ idx,
          const float* __restrict__ wts,
          const float* __restrict__ bd, int E, const void* __restrict__ resid, void* __restrict__ y, int T, int k,
          int D, int ydt) {
    // every pointer argument is read into SGPRs at entry (one scalar-cache fill, one wait); the kernel has no
    // scalar loads from memory, which an asm statement ahead of them would turn into vector loads
    asm volatile("" ::"s"(yp), "s"(idx), "s"(wts), "s"(bd), "s"(resid), "s"(y));
    const size_t i4 = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t total4 = (size_t)T * D / 4;
    if (i4 >= total4) return;
    const size_t i = i4 * 4;
    const int t = (int)(i / D), n = (int)(i % D);
    // the residual first, as raw bits: its load goes out with the slots' loads (one memory round trip for the
    // kernel) and is converted at the end (a conversion here would wait for it, and for nothing else in flight)
    uint4 rraw = make_uint4(0u, 0u, 0u, 0u);
    if (resid) {
        if (ydt == MOE_DTYPE_F32) {
            rraw = reinterpret_cast<const uint4*>(resid)[i4];
        } else {
            const uint2 r = reinterpret_cast<const uint2*>(resid)[i4];
            rraw.x = r.x;
            rraw.y = r.y;
        }
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j0 = 0; j0 < k; j0 += KC) {
        int e[KC];
        float w[KC];
        float4 v[KC], b[KC];
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const int slot = t * k + (j0 + j < k ? j0 + j : k - 1);
            e[j] = idx[slot];
            w[j] = wts[slot];
            v[j] = reinterpret_cast<const float4*>(yp + (size_t)slot * D + n)[0];
        }
        for (int pl = 1; pl < nplanes; ++pl) {   // K parts of a split down projection
#pragma unroll
            for (int j = 0; j < KC; ++j) {
                const int slot = t * k + (j0 + j < k ? j0 + j : k - 1);
                const float4 u = reinterpret_cast<const float4*>(yp + pl * plane + (size_t)slot * D + n)[0];
                v[j].x += u.x;
                v[j].y += u.y;
                v[j].z += u.z;
                v[j].w += u.w;
            }
        }
        if (bd) {
#pragma unroll
            for (int j = 0; j < KC; ++j) {
                const int ee = (unsigned)e[j] < (unsigned)E ? e[j] : 0;
                b[j] = reinterpret_cast<const float4*>(bd + (size_t)ee * D + n)[0];
            }
        }
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const bool ok = j0 + j < k && (unsigned)e[j] < (unsigned)E;
            float4 u = v[j];
            if (bd) {
                u.x += b[j].x;
                u.y += b[j].y;
                u.z += b[j].z;
                u.w += b[j].w;
            }
            acc.x = ok ? __builtin_fmaf(w[j], u.x, acc.x) : acc.x;
            acc.y = ok ? __builtin_fmaf(w[j], u.y, acc.y) : acc.y;
            acc.z = ok ? __builtin_fmaf(w[j], u.z, acc.z) : acc.z;
            acc.w = ok ? __builtin_fmaf(w[j], u.w, acc.w) : acc.w;
        }
    }
    if (resid) {
        float4 rv;
        if (ydt == MOE_DTYPE_F32) {
            rv = make_float4(__uint_as_float(rraw.x), __uint_as_float(rraw.y), __uint_as_float(rraw.z),
                             __uint_as_float(rraw.w));
        } else if (ydt == MOE_DTYPE_F16) {
            rv = make_float4(y_bits_f32(rraw.x & 0xFFFFu, ydt), y_bits_f32(rraw.x >> 16, ydt),
                             y_bits_f32(rraw.y & 0xFFFFu, ydt), y_bits_f32(rraw.y >> 16, ydt));
        } else {
            rv = make_float4(bf16lo(rraw.x), bf16hi(rraw.x), bf16lo(rraw.y), bf16hi(rraw.y));
        }
        acc.x += rv.x;
        acc.y += rv.y;
        acc.z += rv.z;
        acc.w += rv.w;
    }
    if (ydt == MOE_DTYPE_F32) {
        reinterpret_cast<float4*>(y)[i4] = acc;
        return;
    }
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    if (ydt == MOE_DTYPE_F16) {
        reinterpret_cast<h4*>(y)[i4] = h4{(_Float16)acc.x, (_Float16)acc.y, (_Float16)acc.z, (_Float16)acc.w};
        return;
    }
    uint2 o;
    o.x = (uint32_t)f32_to_bf16(acc.x) | ((uint32_t)f32_to_bf16(acc.y) << 16);
    o.y = (uint32_t)f32_to_bf16(acc.z) | ((uint32_t)f32_to_bf16(acc.w) << 16);
    reinterpret_cast<uint2*>(y)[i4] = o;
}

// ============================================================================ host side
namespace {

struct ProjPtrs {
    const uint8_t *G, *U, *Dn;
};
ProjPtrs ptrs(const moe_experts_t* w) {
    return {(const uint8_t*)w->gate.rows, (const uint8_t*)w->up.rows, (const uint8_t*)w->down.rows};
}

template <class FMT, int ACT>
void launch_gu_slots(const ExpertsArgs& a, int NR) {
    const moe_experts_t* w = a.w;
    const ProjPtrs P = ptrs(w);
    const int nslots = a.T * a.k;
    if (a.nx > 1) NR = 1;   // planes of fp16 / fp32 activations: one row pair per wave
    dim3 grid((w->F + 4 * NR - 1) / (4 * NR), nslots);
#define MOE_GUS(R, H)                                                                                           \
    k_gate_up_slots<FMT, ACT, R, H><<<grid, 256, 0, a.st>>>(a.xb, a.xplane, P.G, P.U, w->gate.bias, w->up.bias,  \
                                                             a.idx, a.k, w->d, w->F, w->E, a.hhi, a.hlo)
    if (a.nx == 3) MOE_GUS(1, 3);
    else if (a.nx == 2) MOE_GUS(1, 2);
    else if (NR == 4) MOE_GUS(4, 1);
    else if (NR == 2) MOE_GUS(2, 1);
    else MOE_GUS(1, 1);
#undef MOE_GUS
}

// lanes per down row and chunks per lane for the per-slot down kernel: LPR a power of two in [4, 64] with
// LPR * NC >= F/32, NC <= 4 (F up to 8192); longer rows use LPR = 64 and several passes (NC = 8).
template <class FMT>
void launch_dn_slots(const ExpertsArgs& a) {
    const moe_experts_t* w = a.w;
    const ProjPtrs P = ptrs(w);
    const int cpr = w->F >> 5;
    int lpr = 4;
    while (lpr < 64 && lpr * 3 < cpr) lpr *= 2;
    const int nc = (cpr + lpr - 1) / lpr;
    const int rpw = 64 / lpr;
    const int nw = a.k < 8 ? a.k : 8;
    dim3 grid((w->d + rpw - 1) / rpw, a.T);
#define MOE_DNS(L, C)                                                                                           \
    k_down_slots<FMT, L, C><<<grid, 64 * nw, 0, a.st>>>(a.hhi, a.hlo, P.Dn, w->down.bias, a.idx, a.wts, a.k,      \
                                                         w->d, w->F, w->E, a.nored, a.ydt, a.residual, a.y)
    if (lpr == 4) MOE_DNS(4, 3);
    else if (lpr == 8) MOE_DNS(8, 3);
    else if (lpr == 16) MOE_DNS(16, 3);
    else if (lpr == 32) MOE_DNS(32, 3);
    else if (nc <= 4) MOE_DNS(64, 4);
    else MOE_DNS(64, 8);   // F <= 16384 (checked by the API)
#undef MOE_DNS
}

// ---------------------------------------------------------------- balanced per-slot kernels
#ifndef MOE_GU_MIN_WAVES
#define MOE_GU_MIN_WAVES 2048   // gate/up: fewest waves a launch should have before rows per wave grow
#endif
// gate/up: R row pairs per wave (R divides F), as many as keeps >= 2048 waves in flight (2 blocks per CU on
// 256 CUs); NCH chunks per lane per pass (2 when a row has more than 64 chunks).
template <class FMT, int NCH>
int launch_gu_rows_n(const ExpertsArgs& a, int R) {
    const moe_experts_t* w = a.w;
    const ProjPtrs P = ptrs(w);
    const int Q = a.T * a.k * w->F;
    if (a.route_logits && a.nx > 1) return MOE_ERR_DTYPE;   // the routed gate/up reads bf16 x (one plane)
    if (a.nx > 1) R = w->F % 2 == 0 && Q / 2 >= MOE_GU_MIN_WAVES ? 2 : 1;   // fp16 / fp32 planes: R <= 2
    const int grid = (Q / R + 3) / 4;
    RouteArgs rt{a.route_logits, a.route_norm, a.route_scale, const_cast<int32_t*>(a.idx), const_cast<float*>(a.wts)};
#define MOE_GUR_J(RR, H, J)                                                                                       \
    k_gate_up_rows<FMT, RR, NCH, H, J><<<grid, 256, 0, a.st>>>(a.xb, P.G, P.U, a.idx, a.k, w->d, w->F, Q, w->E, a.act, \
                                                              a.xplane, w->gate.bias, w->up.bias, a.hhi, a.hlo, rt)
// routed: the tail's logits per lane at compile time (E <= 64 J); the layer call routes bf16 x only (H == 1)
#define MOE_GUR(RR, H)                                                                                           \
    do {                                                                                                         \
        if (!rt.logits || H != 1) MOE_GUR_J(RR, H, 0);                                                           \
        else if (w->E <= 64) MOE_GUR_J(RR, 1, 1);                                                                \
        else if (w->E <= 128) MOE_GUR_J(RR, 1, 2);                                                               \
        else if (w->E <= 256) MOE_GUR_J(RR, 1, 4);                                                               \
        else MOE_GUR_J(RR, 1, TOPK_MAX_J);                                                                       \
    } while (0)
    if (a.nx > 1) {
        if (a.nx == 3) {
            if (R == 2) MOE_GUR(2, 3);
            else MOE_GUR(1, 3);
        } else {
            if (R == 2) MOE_GUR(2, 2);
            else MOE_GUR(1, 2);
        }
        return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
    }
    switch (R) {
        case 8: MOE_GUR(8, 1); break;
        case 6: MOE_GUR(6, 1); break;
        case 4: MOE_GUR(4, 1); break;
        case 3: MOE_GUR(3, 1); break;
        case 2: MOE_GUR(2, 1); break;
        default: MOE_GUR(1, 1); break;
    }
#undef MOE_GUR
#undef MOE_GUR_J
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

#ifndef MOE_GU_RMAX
#define MOE_GU_RMAX 8
#endif
int pick_rows_per_wave(int Q, int F, int rmax) {
    const int cand[6] = {8, 6, 4, 3, 2, 1};
    for (int r : cand)
        if (r <= rmax && r <= MOE_GU_RMAX && F % r == 0 && Q / r >= MOE_GU_MIN_WAVES) return r;
    return 1;
}

template <class FMT>
int launch_gu_rows(const ExpertsArgs& a) {
    const int Q = a.T * a.k * a.w->F;
    if ((a.w->d >> 5) <= 64) return launch_gu_rows_n<FMT, 1>(a, pick_rows_per_wave(Q, a.w->F, 8));
    // two chunks per lane: at most 3 row pairs (gpt-oss T=1: 960 blocks of 3 pairs per wave ran 19.1 us per
    // layer against 19.5 for 720 blocks of 4)
    return launch_gu_rows_n<FMT, 2>(a, pick_rows_per_wave(Q, a.w->F, 3));
}

// down: L = 64 / KP lanes per row (KP = the power of two >= k), NCM >= cpr / L chunks per lane, RR rows per
// lane. Returns 1 when the shape does not fit (k > 64, or k * F too large for LDS): the caller falls back.
constexpr int DR_LDS_MAX = 150 * 1024;

int down_rows_lds(int k, int F) { return k * (F >> 5) * 144; }   // 144-byte chunk records

#ifndef MOE_DN_NW
#define MOE_DN_NW 4   // waves per down block
#endif
#ifndef MOE_DN_RR2_NC
#define MOE_DN_RR2_NC 2   // two rows per lane while NC <= this (at NC = 3, Qwen3: twice the blocks, 4.95 -> 4.68 us)
#endif
template <class FMT, int NC, int RR, bool H16>
int launch_dn_rows_kh(const ExpertsArgs& a, int lgL) {
    constexpr int NW = MOE_DN_NW;
    const moe_experts_t* w = a.w;
    const ProjPtrs P = ptrs(w);
    auto kern = k_down_rows<FMT, NC, RR, NW, H16>;
    const int lds = H16 ? a.k * (w->F >> 5) * 80 : down_rows_lds(a.k, w->F);
    // above 64 KB of LDS the kernel needs the attribute on the device it runs on: set on every such launch (a host
    // call, no stream work) rather than remembered, so no state is kept and every device gets it
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, DR_LDS_MAX) != hipSuccess)
        return MOE_ERR_LAUNCH;
    dim3 grid((w->d + NW * RR - 1) / (NW * RR), a.T);
    kern<<<grid, 64 * NW, lds, a.st>>>(a.hhi, a.hlo, P.Dn, w->down.bias, a.idx, a.wts, a.k, w->d, w->F, w->E, lgL,
                                   a.nored, a.ydt, a.residual, a.y);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}
// h as the gate/up stage wrote it (h_is_f16: one fp16 plane)
template <class FMT, int NC, int RR>
int launch_dn_rows_k(const ExpertsArgs& a, int lgL) {
    if constexpr (FMT::FMT == MOE_FMT_MXFP4)
        if (h_is_f16(FMT::FMT, a.act)) return launch_dn_rows_kh<FMT, NC, RR, true>(a, lgL);
    return launch_dn_rows_kh<FMT, NC, RR, false>(a, lgL);
}

// lanes per down row L = 64 / KP (KP = the power of two >= k); chunks per lane NC >= cpr / L, from a fixed
// menu; two rows per lane while NC <= MOE_DN_RR2_NC
int down_rows_plan(int k, int F, int* lgL) {
    if (k > 32 || k < 1) return 0;
    int kp = 1;
    while (kp < k) kp *= 2;
    const int L = 64 / kp;
    *lgL = 0;
    while ((1 << *lgL) < L) ++*lgL;
    const int need = ((F >> 5) + L - 1) / L;
    const int menu[8] = {1, 2, 3, 4, 6, 8, 12, 16};
    for (int nc : menu)
        if (nc >= need) return down_rows_lds(k, F) <= DR_LDS_MAX ? nc : 0;
    return 0;
}

bool down_rows_fits(int k, int F) {
    int lgL;
    return down_rows_plan(k, F, &lgL) != 0;
}

template <class FMT>
int launch_dn_rows(const ExpertsArgs& a) {
    int lgL = 0;
    switch (down_rows_plan(a.k, a.w->F, &lgL)) {
        case 1: return launch_dn_rows_k<FMT, 1, (1 <= MOE_DN_RR2_NC ? 2 : 1)>(a, lgL);
        case 2: return launch_dn_rows_k<FMT, 2, (2 <= MOE_DN_RR2_NC ? 2 : 1)>(a, lgL);
        case 3: return launch_dn_rows_k<FMT, 3, (3 <= MOE_DN_RR2_NC ? 2 : 1)>(a, lgL);
        case 4: return launch_dn_rows_k<FMT, 4, (4 <= MOE_DN_RR2_NC ? 2 : 1)>(a, lgL);
        case 6: return launch_dn_rows_k<FMT, 6, (6 <= MOE_DN_RR2_NC ? 2 : 1)>(a, lgL);
        case 8: return launch_dn_rows_k<FMT, 8, (8 <= MOE_DN_RR2_NC ? 2 : 1)>(a, lgL);
        case 12: return launch_dn_rows_k<FMT, 12, 1>(a, lgL);
        case 16: return launch_dn_rows_k<FMT, 16, 1>(a, lgL);
        default: return MOE_ERR_ARG;
    }
}

template <class FMT>
int run_slots_fmt(const ExpertsArgs& a) {
    const int nslots = a.T * a.k;
    if (down_rows_fits(a.k, a.w->F)) {
        if (a.stages & 1) {
            const int rc = launch_gu_rows<FMT>(a);
            if (rc) return rc;
        }
        if (a.stages & 2) return launch_dn_rows<FMT>(a);
        return 0;
    }
    if (a.stages & 1) {
        // fewer rows per wave when the launch would be short of waves
        const long waves4 = (long)nslots * a.w->F / 16;
        const int NR = waves4 >= 1024 ? 4 : ((long)nslots * a.w->F / 8 >= 1024 ? 2 : 1);
        if (a.act == 0) launch_gu_slots<FMT, 0>(a, NR);
        else if (a.act == 1) launch_gu_slots<FMT, 1>(a, NR);
        else launch_gu_slots<FMT, 2>(a, NR);
        if (hipGetLastError() != hipSuccess) return MOE_ERR_LAUNCH;
    }
    if (a.stages & 2) {
        launch_dn_slots<FMT>(a);
        if (hipGetLastError() != hipSuccess) return MOE_ERR_LAUNCH;
    }
    return 0;
}

}  // namespace

bool slots_route_in_gate_up(int k, int F) { return down_rows_fits(k, F); }

int run_experts_slots(const ExpertsArgs& a) {
    return a.w->fmt == MOE_FMT_INT4_G64 ? run_slots_fmt<FmtInt4>(a) : run_slots_fmt<FmtMxfp4>(a);
}

int launch_x_planes(const void* x, int xdt, int T, int d, uint16_t* planes, hipStream_t st) {
    const size_t n = (size_t)T * d, n8 = n / 8;
    if (n8 == 0) return 0;
    dim3 grid((unsigned)((n8 + 255) / 256));
    if (xdt == MOE_DTYPE_F16) k_x_planes<MOE_DTYPE_F16><<<grid, 256, 0, st>>>(x, planes, n8, n);
    else k_x_planes<MOE_DTYPE_F32><<<grid, 256, 0, st>>>(x, planes, n8, n);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

int launch_combine(const float* yp, int nplanes, size_t plane, const int32_t* idx, const float* wts, const float* bd, int E,
                   const void* residual, void* y, int T, int k, int d, int ydt, hipStream_t st) {
    const size_t total4 = (size_t)T * d / 4;
    if (total4 == 0) return 0;
    dim3 grid((unsigned)((total4 + 255) / 256));
    if (k <= 1) k_combine<1><<<grid, 256, 0, st>>>(yp, nplanes, plane, idx, wts, bd, E, residual, y, T, k, d, ydt);
    else if (k <= 2) k_combine<2><<<grid, 256, 0, st>>>(yp, nplanes, plane, idx, wts, bd, E, residual, y, T, k, d, ydt);
    else if (k <= 4) k_combine<4><<<grid, 256, 0, st>>>(yp, nplanes, plane, idx, wts, bd, E, residual, y, T, k, d, ydt);
    else k_combine<8><<<grid, 256, 0, st>>>(yp, nplanes, plane, idx, wts, bd, E, residual, y, T, k, d, ydt);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

}  // namespace moe

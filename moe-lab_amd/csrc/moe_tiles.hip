// Grouped expert tiles for T > 1 on bf16 MFMA (gfx950 v_mfma_f32_16x16x32_bf16): the expert-tile grouped
// GEMM of the reference's T > 1 path (metal_q4_tiles_v2.py:160-360 gate/up and down tiles, one MMA tile per
// 8 rows x 8 slots there), re-cut for 64-wide waves and MFMA.
//
// A block owns one active expert and TL_ROWS = 64 weight rows (16 per wave). For gate/up the same wave owns
// gate row r and up row r, so the GLU is applied in registers; for down it owns 16 rows of W_down. The
// expert's slots (stable, ascending slot id: the grouping of moe_group) are taken 16 * NT at a time; each
// pass streams the block's rows in K slices of TL_KC chunks (128 inputs) through LDS:
//   A (codes): each thread loads one 16-byte chunk of one row and scatters its 4 words so that lane (r, g)
//              later reads word g of the slice's 4 chunks with one ds_read_b128 (g = lane / 16 is the MFMA
//              K group of 8 inputs, r = lane % 16 the row);
//   metadata:  int4 (scale, bias - 128 scale) per 64-group, MXFP4 2^(s-127) per 32-group, as fp32;
//   B (activations of the pass's tokens): 16-byte pieces of 8 inputs, reordered (0,4,1,5,2,6,3,7) like the
//              decoded codes; tokens past the expert's count and inputs past K are zero.
// The next slice's global loads are issued before the current slice's MFMAs (register double buffer).
//
// Arithmetic (exact operands, fp32 accumulation; the reference's raw-code MMA with per-group fp32 fix-up,
// metal_q4_tiles_v2.py:242-263): codes decode to bf16 128 + q (int4) or e2m1(q) (MXFP4), exactly; per scale
// group the MFMA sums P = sum (128 + q) x over the group and, for int4, XS = sum x from one more MFMA with an
// all-ones A operand; then acc += s * P + (b - 128 s) * XS (int4) or acc += 2^(s-127) * P (MXFP4).
// The GLU output h is stored as two bf16 planes h = hi + lo (about 16 significant bits; the reference keeps
// it in x.dtype); the down projection runs one MFMA per plane into the same accumulator. The down output is
// yp[slot] = wts[slot] * (W_down h + b_down) in fp32, summed over the k slots of a token by k_combine.
#include "moe_common.h"
#include "moe_formats.h"
#include "moe_internal.h"

namespace moe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int TL_ROWS = 64;   // weight rows per block
constexpr int TL_KC = 4;      // chunks (32 inputs) per K slice
constexpr int TL_APAD = 20;   // words per staged row: [g 0..3][chunk 0..3] + 4 words of padding
constexpr int TL_BPAD = 17;   // 16-byte pieces per staged token: 16 + 1 of padding

struct TileArgs {
    const uint16_t* actv;  // gate/up: x [T, K]; down: h [T*k, K] (bf16; the hi plane of h = hi + lo)
    const uint16_t* actv2; // down: the lo plane of h
    int act_div;           // activation row of slot p: p / act_div (k for gate/up, 1 for down)
    const uint8_t* W0;     // gate (or down) row records [E, N, rb]
    const uint8_t* W1;     // up row records (gate/up only)
    const float* b0;       // additive row biases [E, N] (gpt-oss) or null
    const float* b1;
    const int32_t *counts, *offsets, *sorted, *active, *meta;
    const float* wts;      // routing weight per slot (down)
    int K, N, E, act;      // act: GLU kind (gate/up)
    uint16_t* hout;        // gate/up: h = hi + lo as two bf16 planes [T*k, N]
    uint16_t* hout2;
    float* yp;             // down: [T*k, N] fp32
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = {a, b, c, d};
    return __builtin_bit_cast(bf16x8, v);
}

// (x0..x7) as 4 bf16 words -> the decoded-code order: words (x0,x4), (x1,x5), (x2,x6), (x3,x7)
__device__ __forceinline__ uint4 pair8(uint4 v) {
    uint4 o;
    o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);   // (x0, x4)
    o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);   // (x1, x5)
    o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);   // (x2, x6)
    o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);   // (x3, x7)
    return o;
}

// NPROJ = 2: gate/up (+ GLU, h out as hi/lo planes); NPROJ = 1: down (activation h = hi + lo: HL = 2 planes)
template <class FMT, int NPROJ, int NT>
__global__ void __launch_bounds__(256)
k_tile(TileArgs a) {
    constexpr int NTOK = 16 * NT;
    constexpr bool INT4 = FMT::XSUM;
    constexpr int HL = NPROJ == 2 ? 1 : 2;   // activation planes
    __shared__ uint32_t sA[NPROJ][TL_ROWS][TL_APAD];
    __shared__ float4 sM[NPROJ][TL_ROWS];   // int4: (s0, c0, s1, c1) of the slice's 2 groups; MXFP4: 4 scales
    __shared__ uint4 sB[HL][NTOK][TL_BPAD];

    if ((int)blockIdx.y >= a.meta[0]) return;   // block-uniform: fewer active experts than the grid allows
    const int e = a.active[blockIdx.y];
    const int n = a.counts[e], beg = a.offsets[e];
    const int row0 = blockIdx.x * TL_ROWS;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;   // MFMA row / column and K group
    const int K = a.K, N = a.N;
    const int cpr = K >> 5;
    const int nslice = (cpr + TL_KC - 1) / TL_KC;
    const size_t rb = rbytes(FMT::FMT, K);
    const uint8_t* Wp[2] = {a.W0 + ((size_t)e * N + row0) * rb, NPROJ == 2 ? a.W1 + ((size_t)e * N + row0) * rb : nullptr};

    // staging assignment of this thread
    const int arow = tid >> 2, achunk = tid & 3;   // A: one chunk of one row per projection
    const int mrow = (tid & 127) >> 1, mgi = tid & 1, mproj = tid >> 7;   // int4 metadata word
    const uint32_t ones = 0x3F803F80u;
    const bf16x8 ONES = as_bf16x8(ones, ones, ones, ones);

    for (int tok0 = 0; tok0 < n; tok0 += NTOK) {
        // activation rows of this pass's tokens (staging: piece i of this thread is token (tid + 256 i) / 16)
        size_t brow[NT];
        bool bval[NT];
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const int tk = (tid + 256 * i) >> 4;
            bval[i] = tok0 + tk < n;
            const int slot = a.sorted[beg + min(tok0 + tk, n - 1)];
            brow[i] = (size_t)(slot / a.act_div) * K;
        }
        f32x4 acc[NPROJ][NT];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[p][t] = f32x4{0.f, 0.f, 0.f, 0.f};

        uint4 ra[NPROJ], rbv[HL][NT];
        uint32_t rm = 0;
        auto load_slice = [&](int s) {
            const int c = s * TL_KC + achunk;
#pragma unroll
            for (int p = 0; p < NPROJ; ++p)
                if (c < cpr) ra[p] = *reinterpret_cast<const uint4*>(Wp[p] + (size_t)arow * rb + 16 * c);
            if (INT4) {
                const int grp = 2 * s + mgi;
                if (mproj < NPROJ && grp < (K >> 6))
                    rm = *reinterpret_cast<const uint32_t*>(Wp[mproj] + (size_t)mrow * rb + (K >> 1) + 4 * grp);
            } else {
                if (tid < NPROJ * TL_ROWS) {
                    const int pr = tid / TL_ROWS, rw = tid % TL_ROWS;
                    rm = *reinterpret_cast<const uint32_t*>(Wp[pr] + (size_t)rw * rb + (K >> 1) + 4 * s);
                }
            }
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                const int q = (tid + 256 * i) & 15;
                const int k0 = s * 128 + 8 * q;
#pragma unroll
                for (int hl = 0; hl < HL; ++hl) {
                    rbv[hl][i] = make_uint4(0u, 0u, 0u, 0u);
                    if (bval[i] && k0 < K)
                        rbv[hl][i] = *reinterpret_cast<const uint4*>((hl ? a.actv2 : a.actv) + brow[i] + k0);
                }
            }
        };
        load_slice(0);
        for (int s = 0; s < nslice; ++s) {
            __syncthreads();   // the previous slice's readers are done with the LDS
            {
                const int c = s * TL_KC + achunk;
#pragma unroll
                for (int p = 0; p < NPROJ; ++p) {
                    const uint4 v = c < cpr ? ra[p] : make_uint4(0u, 0u, 0u, 0u);
                    sA[p][arow][0 * 4 + achunk] = v.x;
                    sA[p][arow][1 * 4 + achunk] = v.y;
                    sA[p][arow][2 * 4 + achunk] = v.z;
                    sA[p][arow][3 * 4 + achunk] = v.w;
                }
                if (INT4) {
                    if (mproj < NPROJ) {
                        const bool ok = 2 * s + mgi < (K >> 6);
                        const float sc = ok ? bf16lo(rm) : 0.f, bi = ok ? bf16hi(rm) : 0.f;
                        float* m = reinterpret_cast<float*>(&sM[mproj][mrow]);
                        m[2 * mgi] = sc;
                        m[2 * mgi + 1] = __builtin_fmaf(-128.f, sc, bi);
                    }
                } else if (tid < NPROJ * TL_ROWS) {
                    const int pr = tid / TL_ROWS, rw = tid % TL_ROWS;
                    float4 m;
                    // E8M0 byte s -> the fp32 with bits s << 23: 2^(s-127) for s = 1..254, 0 for s = 0;
                    // groups past K read the zero padding of the record or the next row's codes, so they
                    // are zeroed here (their activations are zero as well)
                    const int g0 = 4 * s;
                    m.x = g0 + 0 < cpr ? __uint_as_float((rm & 0xFFu) << 23) : 0.f;
                    m.y = g0 + 1 < cpr ? __uint_as_float(((rm >> 8) & 0xFFu) << 23) : 0.f;
                    m.z = g0 + 2 < cpr ? __uint_as_float(((rm >> 16) & 0xFFu) << 23) : 0.f;
                    m.w = g0 + 3 < cpr ? __uint_as_float((rm >> 24) << 23) : 0.f;
                    sM[pr][rw] = m;
                }
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    const int tk = (tid + 256 * i) >> 4, q = (tid + 256 * i) & 15;
#pragma unroll
                    for (int hl = 0; hl < HL; ++hl) sB[hl][tk][q] = pair8(rbv[hl][i]);
                }
            }
            __syncthreads();
            if (s + 1 < nslice) load_slice(s + 1);   // in flight during this slice's math

            // ---- math: this wave's 16 rows, every token tile of the pass
            uint4 aw[NPROJ];
            float4 mr[NPROJ][4];
#pragma unroll
            for (int p = 0; p < NPROJ; ++p) {
                aw[p] = *reinterpret_cast<const uint4*>(&sA[p][16 * wave + lr][4 * lg]);
#pragma unroll
                for (int v = 0; v < 4; ++v) mr[p][v] = sM[p][16 * wave + 4 * lg + v];
            }
            uint32_t awv[NPROJ][4];
#pragma unroll
            for (int p = 0; p < NPROJ; ++p) {
                awv[p][0] = aw[p].x;
                awv[p][1] = aw[p].y;
                awv[p][2] = aw[p].z;
                awv[p][3] = aw[p].w;
            }
            constexpr int CPG = INT4 ? 2 : 1;   // chunks per scale group
#pragma unroll
            for (int gi = 0; gi < TL_KC / CPG; ++gi) {
                bf16x8 A[NPROJ][CPG];
#pragma unroll
                for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                    for (int cc = 0; cc < CPG; ++cc) {
                        uint32_t q[4];
                        FMT::decode_word(awv[p][gi * CPG + cc], q);
                        A[p][cc] = as_bf16x8(q[0], q[1], q[2], q[3]);
                    }
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    bf16x8 B[HL][CPG];
#pragma unroll
                    for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                        for (int cc = 0; cc < CPG; ++cc) {
                            const uint4 bv = sB[hl][16 * t + lr][4 * (gi * CPG + cc) + lg];
                            B[hl][cc] = as_bf16x8(bv.x, bv.y, bv.z, bv.w);
                        }
                    f32x4 xs = f32x4{0.f, 0.f, 0.f, 0.f};
                    if (INT4) {
#pragma unroll
                        for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                            for (int cc = 0; cc < CPG; ++cc)
                                xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ONES, B[hl][cc], xs, 0, 0, 0);
                    }
#pragma unroll
                    for (int p = 0; p < NPROJ; ++p) {
                        f32x4 P = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                            for (int cc = 0; cc < CPG; ++cc)
                                P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[p][cc], B[hl][cc], P, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            const float4 m = mr[p][v];
                            if (INT4) {
                                const float sc = gi == 0 ? m.x : m.z, cb = gi == 0 ? m.y : m.w;
                                acc[p][t][v] = __builtin_fmaf(sc, P[v], __builtin_fmaf(cb, xs[v], acc[p][t][v]));
                            } else {
                                const float sc = gi == 0 ? m.x : (gi == 1 ? m.y : (gi == 2 ? m.z : m.w));
                                acc[p][t][v] = __builtin_fmaf(sc, P[v], acc[p][t][v]);
                            }
                        }
                    }
                }
            }
        }
        // ---- epilogue: lane holds rows 16 wave + 4 lg + v (v = 0..3) of token column lr of each tile
        const int rbase = row0 + 16 * wave + 4 * lg;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int j = tok0 + 16 * t + lr;
            if (j >= n) continue;
            const int slot = a.sorted[beg + j];
            if (NPROJ == 2) {
                uint32_t phi[2], plo[2];
#pragma unroll
                for (int v = 0; v < 4; v += 2) {
                    uint32_t hi2 = 0, lo2 = 0;
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        float g = acc[0][t][v + u], up = acc[NPROJ - 1][t][v + u];
                        if (a.b0) g += a.b0[(size_t)e * N + rbase + v + u];
                        if (a.b1) up += a.b1[(size_t)e * N + rbase + v + u];
                        const float hv = glu_act(a.act, g, up);
                        const uint16_t hi = f32_to_bf16(hv);
                        hi2 |= (uint32_t)hi << (16 * u);
                        lo2 |= (uint32_t)f32_to_bf16(hv - bf16_to_f32(hi)) << (16 * u);
                    }
                    phi[v / 2] = hi2;
                    plo[v / 2] = lo2;
                }
                *reinterpret_cast<uint2*>(a.hout + (size_t)slot * N + rbase) = make_uint2(phi[0], phi[1]);
                *reinterpret_cast<uint2*>(a.hout2 + (size_t)slot * N + rbase) = make_uint2(plo[0], plo[1]);
            } else {
                const float w = a.wts[slot];
                float4 o;
                float* ov = reinterpret_cast<float*>(&o);
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float y = acc[0][t][v];
                    if (a.b0) y += a.b0[(size_t)e * N + rbase + v];
                    ov[v] = w * y;
                }
                *reinterpret_cast<float4*>(a.yp + (size_t)slot * N + rbase) = o;
            }
        }
    }
}

// ------------------------------------------------------------------------------------ host side
namespace {

int tokens_per_pass_tiles(int T, int k, int E) {
    const int avg = (T * k + E - 1) / E;   // expected slots per active expert (uniform routing)
    return avg <= 16 ? 1 : (avg <= 32 ? 2 : (avg <= 64 ? 4 : 8));
}

template <class FMT, int NPROJ>
int launch_tile(const TileArgs& t, int nt, int max_active, hipStream_t st) {
    dim3 grid(t.N / TL_ROWS, max_active);
    switch (nt) {
        case 1: k_tile<FMT, NPROJ, 1><<<grid, 256, 0, st>>>(t); break;
        case 2: k_tile<FMT, NPROJ, 2><<<grid, 256, 0, st>>>(t); break;
        case 4: k_tile<FMT, NPROJ, 4><<<grid, 256, 0, st>>>(t); break;
        default: k_tile<FMT, NPROJ, 8><<<grid, 256, 0, st>>>(t); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

template <class FMT>
int run_tiles_fmt(const ExpertsArgs& a) {
    const moe_experts_t* w = a.w;
    const int nslots = a.T * a.k;
    const int max_active = nslots < w->E ? nslots : w->E;
    const int nt = tokens_per_pass_tiles(a.T, a.k, w->E);
    TileArgs t{};
    t.counts = a.grp.counts;
    t.offsets = a.grp.offsets;
    t.sorted = a.grp.sorted;
    t.active = a.grp.active;
    t.meta = a.grp.meta;
    t.E = w->E;
    t.act = a.act;
    if (a.stages & 1) {
        int rc = launch_group(a.idx, nslots, w->E, a.grp.counts, a.grp.offsets, a.grp.sorted, a.grp.active,
                              a.grp.meta, a.st);
        if (rc) return rc;
        TileArgs g = t;
        g.actv = (const uint16_t*)a.x;
        g.act_div = a.k;
        g.K = w->d;
        g.N = w->F;
        g.W0 = (const uint8_t*)w->gate.rows;
        g.W1 = (const uint8_t*)w->up.rows;
        g.b0 = w->gate.bias;
        g.b1 = w->up.bias;
        g.hout = a.hhi;
        g.hout2 = a.hlo;
        rc = launch_tile<FMT, 2>(g, nt, max_active, a.st);
        if (rc) return rc;
    }
    if (a.stages & 2) {
        TileArgs d = t;
        d.actv = a.hhi;
        d.actv2 = a.hlo;
        d.act_div = 1;
        d.K = w->F;
        d.N = w->d;
        d.W0 = (const uint8_t*)w->down.rows;
        d.b0 = w->down.bias;
        d.wts = a.wts;
        d.yp = a.yp;
        int rc = launch_tile<FMT, 1>(d, nt, max_active, a.st);
        if (rc) return rc;
        return launch_combine(a.yp, a.residual, a.y, a.T, a.k, w->d, a.y32, a.st);
    }
    return 0;
}

}  // namespace

int run_experts_tiles(const ExpertsArgs& a) {
    return a.w->fmt == MOE_FMT_INT4_G64 ? run_tiles_fmt<FmtInt4>(a) : run_tiles_fmt<FmtMxfp4>(a);
}

}  // namespace moe

// Grouped expert tiles for T > 1 on bf16 MFMA (gfx950 v_mfma_f32_16x16x32_bf16): the expert-tile grouped
// GEMM of the reference's T > 1 path (metal_q4_tiles_v2.py:160-360 gate/up and down tiles, one MMA tile per
// 8 rows x 8 slots there), re-cut for 64-wide waves and MFMA.
//
// A block owns one active expert and TL_ROWS = 64 weight rows (16 per wave). For gate/up the same wave owns
// gate row r and up row r, so the GLU is applied in registers; for down it owns 16 rows of W_down. The
// expert's slots (stable, ascending slot id: the grouping of moe_group) are taken 16 * NT at a time, pass z
// of an expert by the block with blockIdx.z = z mod gridDim.z (so a popular expert spreads over blocks); each
// pass streams the block's rows in K slices of TL_KC chunks (256 inputs) through LDS:
//   A (codes): each thread loads 16-byte chunks of the rows and scatters their 4 words so that lane (r, g)
//              later reads word g of the slice's chunks with ds_read_b128 (g = lane / 16 is the MFMA K group
//              of 8 inputs, r = lane % 16 the row);
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
// yp[slot] = W_down h in fp32; k_combine adds b_down, applies the routing weights and sums a token's slots.
#include "moe_common.h"
#include "moe_formats.h"
#include "moe_internal.h"

#include <math.h>

namespace moe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int TL_ROWS = 64;   // weight rows per block
constexpr int TL_KC = 8;      // chunks (32 inputs) per K slice
constexpr int TL_APAD = 4 * TL_KC + 4;   // words per staged row: [g 0..3][chunk 0..KC-1] + 4 words of padding
constexpr int TL_BPAD = 4 * TL_KC + 1;   // 16-byte pieces per staged token (8 inputs each) + 1 of padding
constexpr int TL_GMAX = TL_KC;           // scale groups per slice at most (MXFP4: one per chunk)

struct TileArgs {
    const uint16_t* actv;  // gate/up: x [T, K]; down: h [T*k, K] (bf16; the hi plane of h = hi + lo)
    const uint16_t* actv2; // down: the lo plane of h
    int act_div;           // activation row of slot p: p / act_div (k for gate/up, 1 for down)
    const uint8_t* W0;     // gate (or down) row records [E, N, rb]
    const uint8_t* W1;     // up row records (gate/up only)
    const float* b0;       // additive row biases [E, N] (gpt-oss) or null
    const float* b1;
    const int32_t *counts, *offsets, *sorted, *active, *meta;
    int K, N, E, act;      // act: GLU kind (gate/up)
    int rpb;               // row tiles per block (k_tile_run)
    int kslots;            // k (slots per token)
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

// workgroup barrier after this wave's LDS writes have completed, without a memory fence (a fence would also
// wait for every global load in flight); the "memory" clobber keeps the compiler from moving LDS accesses across
#define MOE_BARRIER_LDS() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

// NPROJ = 2: gate/up (+ GLU, h out as hi/lo planes); NPROJ = 1: down (activation h = hi + lo: HL = 2 planes)
#ifndef MOE_TILE_MINB
#define MOE_TILE_MINB 1   // blocks per CU the register allocation must allow
#endif
template <class FMT, int NPROJ, int NT>
__global__ void __launch_bounds__(256, MOE_TILE_MINB)
k_tile(TileArgs a) {
    constexpr int NTOK = 16 * NT;
    constexpr bool INT4 = FMT::XSUM;
    constexpr int HL = NPROJ == 2 ? 1 : 2;   // activation planes
    __shared__ uint32_t sA[NPROJ][TL_ROWS][TL_APAD];
    __shared__ float sM[NPROJ][TL_ROWS][TL_GMAX];   // int4: (s, b - 128 s) of the slice's 4 groups; MXFP4: 8 scales
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

    // staging assignment of this thread: A chunks (arow, achunk + 4 j), j = 0, 1, of every projection;
    // int4 metadata: word mgi of row mrow of projection mproj (4 groups per slice); MXFP4: 8 bytes of row
    const int arow = tid >> 2, achunk = tid & 3;
    const int mrow = (tid & 127) >> 1, mgi = tid & 1, mproj = tid >> 7;
    const uint32_t ones = 0x3F803F80u;
    const bf16x8 ONES = as_bf16x8(ones, ones, ones, ones);

    for (int tok0 = NTOK * blockIdx.z; tok0 < n; tok0 += NTOK * gridDim.z) {
        // activation rows of this pass's tokens (staging: piece i of this thread is token (tid + 256 i) / 16)
        constexpr int BPT0 = NT * TL_KC / 4;   // activation pieces (8 inputs) per thread per plane per slice
        size_t brow[BPT0];
        bool bval[BPT0];
#pragma unroll
        for (int i = 0; i < BPT0; ++i) {
            const int tk = (tid + 256 * i) / (4 * TL_KC);
            bval[i] = tok0 + tk < n;
            const int slot = a.sorted[beg + min(tok0 + tk, n - 1)];
            brow[i] = (size_t)(slot / a.act_div) * K;
        }
        f32x4 acc[NPROJ][NT];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[p][t] = f32x4{0.f, 0.f, 0.f, 0.f};

        constexpr int BPT = BPT0;
        uint4 ra[NPROJ][2], rbv[HL][BPT];
        uint2 rm = make_uint2(0u, 0u);
        auto load_slice = [&](int s) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int c = s * TL_KC + achunk + 4 * j;
#pragma unroll
                for (int p = 0; p < NPROJ; ++p)
                    if (c < cpr) ra[p][j] = *reinterpret_cast<const uint4*>(Wp[p] + (size_t)arow * rb + 16 * c);
            }
            if (INT4) {   // groups 4s + 2 mgi, 4s + 2 mgi + 1: one 8-byte load
                const int grp = 4 * s + 2 * mgi;
                if (mproj < NPROJ && grp < (K >> 6))
                    rm = *reinterpret_cast<const uint2*>(Wp[mproj] + (size_t)mrow * rb + (K >> 1) + 4 * grp);
            } else {   // E8M0 bytes 8s .. 8s + 7 (past the last group: record padding or the next record)
                if (tid < NPROJ * TL_ROWS) {
                    const int pr = tid / TL_ROWS, rw = tid % TL_ROWS;
                    const uint8_t* mp = Wp[pr] + (size_t)rw * rb + (K >> 1) + 8 * s;
                    rm.x = *reinterpret_cast<const uint32_t*>(mp);
                    if (8 * s + 4 < cpr) rm.y = *reinterpret_cast<const uint32_t*>(mp + 4);
                }
            }
#pragma unroll
            for (int i = 0; i < BPT; ++i) {
                const int q = (tid + 256 * i) % (4 * TL_KC);
                const int k0 = s * (32 * TL_KC) + 8 * q;
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
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int cl = achunk + 4 * j, c = s * TL_KC + cl;
#pragma unroll
                    for (int p = 0; p < NPROJ; ++p) {
                        const uint4 v = c < cpr ? ra[p][j] : make_uint4(0u, 0u, 0u, 0u);
                        sA[p][arow][0 * TL_KC + cl] = v.x;
                        sA[p][arow][1 * TL_KC + cl] = v.y;
                        sA[p][arow][2 * TL_KC + cl] = v.z;
                        sA[p][arow][3 * TL_KC + cl] = v.w;
                    }
                }
                if (INT4) {
                    if (mproj < NPROJ) {
                        const int grp = 4 * s + 2 * mgi;
                        const uint32_t w2[2] = {rm.x, rm.y};
#pragma unroll
                        for (int u = 0; u < 2; ++u) {
                            const bool ok = grp + u < (K >> 6);
                            const float sc = ok ? bf16lo(w2[u]) : 0.f, bi = ok ? bf16hi(w2[u]) : 0.f;
                            sM[mproj][mrow][2 * (2 * mgi + u)] = sc;
                            sM[mproj][mrow][2 * (2 * mgi + u) + 1] = __builtin_fmaf(-128.f, sc, bi);
                        }
                    }
                } else if (tid < NPROJ * TL_ROWS) {
                    const int pr = tid / TL_ROWS, rw = tid % TL_ROWS;
                    // E8M0 byte s -> the fp32 with bits s << 23: 2^(s-127) for s = 1..254, 0 for s = 0; groups
                    // past K (record padding or the next record's bytes) are zeroed, as are their activations
                    const uint32_t w2[2] = {rm.x, rm.y};
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const uint32_t b = (w2[u >> 2] >> (8 * (u & 3))) & 0xFFu;
                        sM[pr][rw][u] = 8 * s + u < cpr ? __uint_as_float(b << 23) : 0.f;
                    }
                }
#pragma unroll
                for (int i = 0; i < BPT; ++i) {
                    const int tk = (tid + 256 * i) / (4 * TL_KC), q = (tid + 256 * i) % (4 * TL_KC);
#pragma unroll
                    for (int hl = 0; hl < HL; ++hl) sB[hl][tk][q] = pair8(rbv[hl][i]);
                }
            }
            __syncthreads();
            if (s + 1 < nslice) load_slice(s + 1);   // in flight during this slice's math

            // ---- math: this wave's 16 rows, every token tile of the pass
            uint32_t awv[NPROJ][TL_KC];
#pragma unroll
            for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                for (int q = 0; q < TL_KC / 4; ++q) {
                    const uint4 aw = *reinterpret_cast<const uint4*>(&sA[p][16 * wave + lr][TL_KC * lg + 4 * q]);
                    awv[p][4 * q] = aw.x;
                    awv[p][4 * q + 1] = aw.y;
                    awv[p][4 * q + 2] = aw.z;
                    awv[p][4 * q + 3] = aw.w;
                }
            constexpr int CPG = INT4 ? 2 : 1;   // chunks per scale group
#pragma unroll
            for (int gi = 0; gi < TL_KC / CPG; ++gi) {
                // this group's metadata for the lane's 4 output rows: (s, b - 128 s) or the MXFP4 scale
                float ms[NPROJ][4], mc[NPROJ][4];
#pragma unroll
                for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float* m = &sM[p][16 * wave + 4 * lg + v][0];
                        if (INT4) {
                            const float2 m2 = *reinterpret_cast<const float2*>(m + 2 * gi);
                            ms[p][v] = m2.x;
                            mc[p][v] = m2.y;
                        } else {
                            ms[p][v] = m[gi];
                            mc[p][v] = 0.f;
                        }
                    }
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
                            const uint4 bv = sB[hl][16 * t + lr][4 * (gi * CPG + cc) + lg];   // piece = 4 chunk + g
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
                            if (INT4)
                                acc[p][t][v] = __builtin_fmaf(ms[p][v], P[v], __builtin_fmaf(mc[p][v], xs[v], acc[p][t][v]));
                            else
                                acc[p][t][v] = __builtin_fmaf(ms[p][v], P[v], acc[p][t][v]);
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
                *reinterpret_cast<float4*>(a.yp + (size_t)slot * N + rbase) =
                    make_float4(acc[0][t][0], acc[0][t][1], acc[0][t][2], acc[0][t][3]);
            }
        }
    }
}

// ============================================================================ DMA-ring tiles (NT <= 2)
// The same tile arithmetic with every operand brought into LDS by direct global->LDS DMA
// (global_load_lds_dwordx4: 16 bytes per lane, written at M0 + 16 * lane) into a ring of DR_NS stages, so
// DR_NS - 1 slices per block are in flight without holding registers. The stage buffers are distinct
// __shared__ objects indexed at compile time (the ring is unrolled), and blocks sync with a bare s_barrier,
// so the waits on the DMA are the explicit per-stage vmcnt waits below, not a full drain.
// Stage layouts (a K slice = DR_KC chunks = 256 inputs):
//   A [proj][row 0..63][pos 0..7] 16-byte chunks, pos = chunk ^ (row & 7) (bank spread for the reads of
//     lane (r, g): word g of chunk c of row r);
//   M int4: [proj][row] 16 bytes = the slice's 4 (scale | bias) words; MXFP4: [proj][word 0..1][row] 4 bytes;
//   B [plane][token 0..NTOK-1][pos 0..31] 16-byte pieces of 8 inputs, pos = piece ^ (token & 7); the
//     activations are already in the decoded-code order (x copied by k_pair8_rows, h written so).
// Chunks past K are clamped onto the row's last chunk and masked to zero on the A side; tokens past the
// expert's count are clamped onto its last token and their output columns dropped.
constexpr int DR_KC = 8;
constexpr int DR_NS = 3;

#define MOE_LDSP(p) ((__attribute__((address_space(3))) void*)(p))
// workgroup barrier without a memory fence (a fence would drain every outstanding DMA); the "memory" clobber
// keeps the compiler from moving LDS accesses across it
#define MOE_BARRIER() asm volatile("s_barrier" ::: "memory")
#define MOE_VMWAIT(N) __builtin_amdgcn_s_waitcnt(((N) & 0xF) | (((N) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

template <class FMT, int NPROJ, int NT>
struct DrStage {
    static constexpr int NTOK = 16 * NT;
    static constexpr int HL = NPROJ == 2 ? 1 : 2;
    static constexpr int MBYTES = FMT::XSUM ? 16 : 8;
    uint4 A[NPROJ][TL_ROWS][DR_KC];
    uint32_t M[NPROJ][TL_ROWS * MBYTES / 4];
    uint4 B[HL][NTOK][4 * DR_KC];
};

template <class FMT, int NPROJ, int NT>
__device__ __forceinline__ void dr_issue(DrStage<FMT, NPROJ, NT>& S, int s, const uint8_t* const Wp[2], size_t rb,
                                         int K, int cpr, const size_t* brow, const uint16_t* act0,
                                         const uint16_t* act1, int wave, int lane, int npair) {
    using St = DrStage<FMT, NPROJ, NT>;
    // A: 8 instructions per projection, 8 rows x 8 chunks each; wave w takes instructions w, w + 4
#pragma unroll
    for (int p = 0; p < NPROJ; ++p)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int i = wave + 4 * j;
            const int row = 8 * i + (lane >> 3), pos = lane & 7;
            const int gc = min(s * DR_KC + (pos ^ (row & 7)), cpr - 1);
            __builtin_amdgcn_global_load_lds((const void*)(Wp[p] + (size_t)row * rb + 16 * gc),
                                             MOE_LDSP(&S.A[p][8 * i][0]), 16, 0, 0);
        }
    // M
    if (FMT::XSUM) {
        if (wave < NPROJ) {   // the slice's 4 group words of row `lane` (record padding covers a short last slice)
            __builtin_amdgcn_global_load_lds((const void*)(Wp[wave] + (size_t)lane * rb + (K >> 1) + 16 * s),
                                             MOE_LDSP(&S.M[wave][0]), 16, 0, 0);
        }
    } else {
        if (wave < 2 * NPROJ) {   // E8M0 bytes 8s .. 8s+3 (word 0) and 8s+4 .. 8s+7 (word 1)
            const int p = wave >> 1, wj = wave & 1;
            const int byte0 = 8 * s + 4 * ((8 * s + 4 < cpr) ? wj : 0);
            __builtin_amdgcn_global_load_lds((const void*)(Wp[p] + (size_t)lane * rb + (K >> 1) + byte0),
                                             MOE_LDSP(&S.M[p][wj * TL_ROWS]), 4, 0, 0);
        }
    }
    // B: 2 tokens x 32 pieces per instruction; wave w takes instructions w, w + 4, ... below npair (the token
    // pairs the pass has: columns past the expert's count are never read into the math's kept outputs)
    constexpr int NBI = St::NTOK / 2;
#pragma unroll
    for (int hl = 0; hl < St::HL; ++hl)
#pragma unroll
        for (int j = 0; j < NBI / 4; ++j) {
            const int i = wave + 4 * j;
            if (i >= npair) continue;   // wave-uniform
            const int tk = 2 * i + (lane >> 5), pos = lane & 31;
            const int piece = pos ^ (tk & 7);
            const int k0 = min(s * (32 * DR_KC) + 8 * piece, K - 8);
            __builtin_amdgcn_global_load_lds((const void*)((hl ? act1 : act0) + brow[j] + k0),
                                             MOE_LDSP(&S.B[hl][2 * i][0]), 16, 0, 0);
        }
}

// DMA instructions a wave issues per stage: 2 per projection for A, one for the metadata on the waves that
// fetch it, and one per activation plane for each of its token-pair instructions below npair
template <class FMT, int NPROJ, int NT>
__device__ __forceinline__ int dr_wave_issues(int wave, int npair) {
    constexpr int NBI = 16 * NT / 2;
    int b = 0;
#pragma unroll
    for (int j = 0; j < NBI / 4; ++j) b += (wave + 4 * j < npair) ? 1 : 0;
    const bool meta = FMT::XSUM ? wave < NPROJ : wave < 2 * NPROJ;
    return 2 * NPROJ + (meta ? 1 : 0) + (NPROJ == 2 ? 1 : 2) * b;
}
// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 15]
__device__ __forceinline__ void vm_wait_n(int n) {
    switch (n) {
        case 0: MOE_VMWAIT(0); break;
        case 1: MOE_VMWAIT(1); break;
        case 2: MOE_VMWAIT(2); break;
        case 3: MOE_VMWAIT(3); break;
        case 4: MOE_VMWAIT(4); break;
        case 5: MOE_VMWAIT(5); break;
        case 6: MOE_VMWAIT(6); break;
        case 7: MOE_VMWAIT(7); break;
        case 8: MOE_VMWAIT(8); break;
        case 9: MOE_VMWAIT(9); break;
        case 10: MOE_VMWAIT(10); break;
        case 11: MOE_VMWAIT(11); break;
        case 12: MOE_VMWAIT(12); break;
        case 13: MOE_VMWAIT(13); break;
        case 14: MOE_VMWAIT(14); break;
        default: MOE_VMWAIT(15); break;
    }
}


// Transposed MFMA for the DMA tiles: the activations are the 16 x 32 operand (16 tokens), the decoded codes the
// 32 x 16 one (16 weight rows), so lane (lr, lg) ends with tokens 4 lg + v (v = 0..3) of weight row lr: one
// metadata word per group and projection per lane, and xs (sum of a token's inputs over the group) comes
// from the same MFMA with an all-ones weight operand.
template <class FMT, int NPROJ, int NT>
__device__ __forceinline__ void dr_math(const DrStage<FMT, NPROJ, NT>& S, int s, int cpr, int K, int wave, int lr,
                                        int lg, f32x4 (&acc)[NPROJ][NT]) {
    constexpr bool INT4 = FMT::XSUM;
    constexpr int HL = NPROJ == 2 ? 1 : 2;
    constexpr int CPG = INT4 ? 2 : 1;
    const uint32_t ones = 0x3F803F80u;
    const bf16x8 ONES = as_bf16x8(ones, ones, ones, ones);
    const int R = 16 * wave + lr;   // this lane's weight row inside the tile
    uint32_t awv[NPROJ][DR_KC];
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) {
        const uint32_t* rowp = reinterpret_cast<const uint32_t*>(&S.A[p][R][0]);
#pragma unroll
        for (int c = 0; c < DR_KC; ++c) awv[p][c] = rowp[4 * (c ^ (R & 7)) + lg];
    }
    // metadata of row R: int4 4 group words, MXFP4 8 E8M0 bytes
    uint32_t mw[NPROJ][INT4 ? 4 : 2];
#pragma unroll
    for (int p = 0; p < NPROJ; ++p) {
        if (INT4) {
            const uint4 m4 = *reinterpret_cast<const uint4*>(&S.M[p][4 * R]);
            mw[p][0] = m4.x;
            mw[p][1] = m4.y;
            mw[p][2] = m4.z;
            mw[p][3] = m4.w;
        } else {
            mw[p][0] = S.M[p][R];
            mw[p][INT4 ? 0 : 1] = S.M[p][TL_ROWS + R];
        }
    }
    const int nvalid = cpr - s * DR_KC;   // chunks of this slice inside the row (>= DR_KC: all)
#pragma unroll
    for (int gi = 0; gi < DR_KC / CPG; ++gi) {
        float ms[NPROJ], mc[NPROJ];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p) {
            if (INT4) {
                const uint32_t m = mw[p][gi];
                const bool ok = 4 * s + gi < (K >> 6);
                const float sc = ok ? bf16lo(m) : 0.f;
                ms[p] = sc;
                mc[p] = ok ? __builtin_fmaf(-128.f, sc, bf16hi(m)) : 0.f;
            } else {
                const uint32_t b = (mw[p][gi >> 2] >> (8 * (gi & 3))) & 0xFFu;
                ms[p] = gi < nvalid ? __uint_as_float(b << 23) : 0.f;
                mc[p] = 0.f;
            }
        }
        bf16x8 W[NPROJ][CPG];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p)
#pragma unroll
            for (int cc = 0; cc < CPG; ++cc) {
                uint32_t q[4];
                FMT::decode_word(awv[p][gi * CPG + cc], q);
                if (gi * CPG + cc >= nvalid) q[0] = q[1] = q[2] = q[3] = 0u;   // chunk past K
                W[p][cc] = as_bf16x8(q[0], q[1], q[2], q[3]);
            }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int tk = 16 * t + lr;
            bf16x8 X[HL][CPG];
#pragma unroll
            for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                for (int cc = 0; cc < CPG; ++cc) {
                    const int piece = 4 * (gi * CPG + cc) + lg;
                    const uint4 bv = S.B[hl][tk][piece ^ (tk & 7)];
                    X[hl][cc] = as_bf16x8(bv.x, bv.y, bv.z, bv.w);
                }
            f32x4 xs = f32x4{0.f, 0.f, 0.f, 0.f};
            if (INT4) {
#pragma unroll
                for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                    for (int cc = 0; cc < CPG; ++cc)
                        xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(X[hl][cc], ONES, xs, 0, 0, 0);
            }
#pragma unroll
            for (int p = 0; p < NPROJ; ++p) {
                f32x4 P = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                    for (int cc = 0; cc < CPG; ++cc)
                        P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(X[hl][cc], W[p][cc], P, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (INT4)
                        acc[p][t][v] = __builtin_fmaf(ms[p], P[v], __builtin_fmaf(mc[p], xs[v], acc[p][t][v]));
                    else
                        acc[p][t][v] = __builtin_fmaf(ms[p], P[v], acc[p][t][v]);
                }
            }
        }
    }
}

// position of element i (0..7) of an 8-input group in the decoded-code order (0,4,1,5,2,6,3,7)
__device__ __forceinline__ int code_pos8(int i) { return i < 4 ? 2 * i : 2 * (i - 4) + 1; }

// One block: one active expert (blockIdx.y), token pass blockIdx.z, and the row tiles
// blockIdx.x * RPB .. + RPB - 1 of that expert (RPB = a.rpb). The ring runs across the block's tiles, so
// the next tile's first slices are in flight while the current tile finishes. A tile's output is computed
// in registers at its last slice and stored at the next step, after that step's wait and barrier (stores
// issued after a stage's DMA would be counted ahead of it by the next vmcnt wait).
template <class FMT, int NPROJ, int NT>
__global__ void __launch_bounds__(256)
k_tile_run(TileArgs a) {
    using St = DrStage<FMT, NPROJ, NT>;
    constexpr int NTOK = St::NTOK;
    constexpr int NBI = NTOK / 2;
    __shared__ St S0, S1, S2;

    if ((int)blockIdx.y >= a.meta[0]) return;
    const int e = a.active[blockIdx.y];
    const int n = a.counts[e], beg = a.offsets[e];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const int K = a.K, N = a.N;
    const int cpr = K >> 5;
    const int nslice = (cpr + DR_KC - 1) / DR_KC;
    const size_t rb = rbytes(FMT::FMT, K);
    const int RT = N / TL_ROWS;
    const int rt0 = blockIdx.x * a.rpb;
    const int ntile = min(a.rpb, RT - rt0);
    if (ntile <= 0) return;
    const int U = ntile * nslice;
    const uint8_t* const W0e = a.W0 + (size_t)e * N * rb;
    const uint8_t* const W1e = (NPROJ == 2 ? a.W1 : a.W0) + (size_t)e * N * rb;

    for (int tok0 = NTOK * blockIdx.z; tok0 < n; tok0 += NTOK * gridDim.z) {
        const int npair = (min(NTOK, n - tok0) + 1) >> 1;   // token pairs of this pass
        const int WI = dr_wave_issues<FMT, NPROJ, NT>(wave, npair);   // this wave's DMA count per stage (<= 15)
        // activation rows of the B instructions this lane issues, and the output slot of each token column
        size_t brow[NBI / 4 > 0 ? NBI / 4 : 1];
#pragma unroll
        for (int j = 0; j < NBI / 4; ++j) {
            const int tk = 2 * (wave + 4 * j) + (lane >> 5);
            brow[j] = (size_t)(a.sorted[beg + min(tok0 + tk, n - 1)] / a.act_div) * K;
        }
        int oslot[NT][4];   // output slot of token 16 t + 4 lg + v (-1: past the expert's count)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int j = tok0 + 16 * t + 4 * lg + v;
                oslot[t][v] = j < n ? a.sorted[beg + j] : -1;
            }
        f32x4 acc[NPROJ][NT];
        float pbias[NPROJ];   // gate/up additive biases of this lane's row of the current tile
        // pending output of the last finished tile, per token: gate/up (hi | lo << 16); down fp32
        uint32_t pend[NT][4];
        int pend_row = -1;   // output row of the pending tile for this lane (-1: nothing pending)

        auto flush = [&]() {
            if (pend_row < 0) return;
            // h is written in the decoded-code order inside each 8-input group: row r -> 8 (r / 8) + pos8(r % 8)
            const int hpos = (pend_row & ~7) + code_pos8(pend_row & 7);
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (oslot[t][v] < 0) continue;
                    if (NPROJ == 2) {
                        a.hout[(size_t)oslot[t][v] * N + hpos] = (uint16_t)(pend[t][v] & 0xFFFFu);
                        a.hout2[(size_t)oslot[t][v] * N + hpos] = (uint16_t)(pend[t][v] >> 16);
                    } else {
                        a.yp[(size_t)oslot[t][v] * N + pend_row] = __uint_as_float(pend[t][v]);
                    }
                }
            pend_row = -1;
        };
        auto issue = [&](auto& S, int u) {
            const int q = u / nslice, si = u - q * nslice;
            const size_t roff = (size_t)(rt0 + q) * TL_ROWS * rb;
            const uint8_t* const Wp[2] = {W0e + roff, W1e + roff};
            dr_issue(S, si, Wp, rb, K, cpr, brow, a.actv, a.actv2, wave, lane, npair);
        };
        auto compute = [&](const auto& S, int u) {
            const int q = u / nslice, si = u - q * nslice;
            if (si == 0) {
#pragma unroll
                for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                    for (int t = 0; t < NT; ++t) acc[p][t] = f32x4{0.f, 0.f, 0.f, 0.f};
                // loaded here, ahead of the tile's later stages, so waiting for them at the tile's end
                // never waits for a stage that is not needed yet
                const int row = (rt0 + q) * TL_ROWS + 16 * wave + lr;
                pbias[0] = (NPROJ == 2 && a.b0) ? a.b0[(size_t)e * N + row] : 0.f;
                pbias[NPROJ - 1] = (NPROJ == 2 && a.b1) ? a.b1[(size_t)e * N + row] : 0.f;
            }
            dr_math(S, si, cpr, K, wave, lr, lg, acc);
            if (si == nslice - 1) {   // tile done: its output into registers, stored at the next step
                const int rbase = (rt0 + q) * TL_ROWS + 16 * wave + lr;   // this lane's output row
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        if (NPROJ == 2) {
                            const float g = acc[0][t][v] + pbias[0], up = acc[NPROJ - 1][t][v] + pbias[NPROJ - 1];
                            const float hv = glu_act(a.act, g, up);
                            const uint16_t hi = f32_to_bf16(hv);
                            pend[t][v] = (uint32_t)hi | ((uint32_t)f32_to_bf16(hv - bf16_to_f32(hi)) << 16);
                        } else {
                            pend[t][v] = __float_as_uint(acc[0][t][v]);
                        }
                    }
                pend_row = rbase;
            }
        };

        MOE_BARRIER();   // every wave is done reading the ring from the previous pass
        issue(S0, 0);
        if (U > 1) issue(S1, 1);
        for (int u = 0; u < U; u += DR_NS) {
#define MOE_DR_STEP(CUR, NXT, OFF)                                         \
    if (u + OFF < U) {                                                     \
        vm_wait_n(u + OFF + 1 >= U ? 0 : WI);                              \
        MOE_BARRIER();                                                     \
        flush();                                                           \
        if (u + OFF + 2 < U) issue(NXT, u + OFF + 2);                      \
        compute(CUR, u + OFF);                                             \
    }
            MOE_DR_STEP(S0, S2, 0)
            MOE_DR_STEP(S1, S0, 1)
            MOE_DR_STEP(S2, S1, 2)
#undef MOE_DR_STEP
        }
        flush();
    }
}

// x [T, d] -> the same rows with each 8-input group in the decoded-code order (for the DMA tiles' B side)
__global__ void __launch_bounds__(256)
k_pair8_rows(const uint4* __restrict__ x, uint4* __restrict__ xp, size_t npieces) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < npieces) xp[i] = pair8(x[i]);
}

// ------------------------------------------------------------------------------------ host side
namespace {

int tokens_per_pass_tiles(int T, int k, int E) {
    const int avg = (T * k + E - 1) / E;   // expected slots per active expert (uniform routing)
    return avg <= 16 ? 1 : (avg <= 32 ? 2 : (avg <= 64 ? 4 : 8));
}

template <class FMT, int NPROJ>
int launch_tile(const TileArgs& t, int nt, int max_active, int T, hipStream_t st) {
    // token passes spread over blockIdx.z: an expert has at most T slots when a token's k ids are distinct
    const int zp = (T + 16 * nt - 1) / (16 * nt);
    dim3 grid(t.N / TL_ROWS, max_active, zp < 1 ? 1 : (zp > 16 ? 16 : zp));
    switch (nt) {
        case 1: k_tile<FMT, NPROJ, 1><<<grid, 256, 0, st>>>(t); break;
        case 2: k_tile<FMT, NPROJ, 2><<<grid, 256, 0, st>>>(t); break;
        case 4: k_tile<FMT, NPROJ, 4><<<grid, 256, 0, st>>>(t); break;
        default: k_tile<FMT, NPROJ, 8><<<grid, 256, 0, st>>>(t); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

#ifndef MOE_TILE_BLOCKS
#define MOE_TILE_BLOCKS 512   // blocks the DMA tile launch aims at (2 per CU); tiles per block follow from it
#endif
template <class FMT, int NPROJ>
int launch_tile_dma(TileArgs t, int nt, int max_active, int T, hipStream_t st) {
    const int zp0 = (T + 16 * nt - 1) / (16 * nt);
    const int zp = zp0 < 1 ? 1 : (zp0 > 16 ? 16 : zp0);
    const int RT = t.N / TL_ROWS;
    // row tiles per block so that the busy blocks come near MOE_TILE_BLOCKS when routing is uniform (E(1 -
    // (1 - k/E)^T) experts active); capped at 2 so skewed routing, with few experts, still fills the device
    const double kE = (double)t.kslots / (double)t.E;
    double act = t.E * (1.0 - pow(1.0 - (kE < 1.0 ? kE : 1.0), (double)T));
    if (act > max_active) act = max_active;
    int rpb = (int)((act * RT + MOE_TILE_BLOCKS - 1) / MOE_TILE_BLOCKS);
    rpb = rpb < 1 ? 1 : (rpb > 2 ? 2 : rpb);
    if (rpb > RT) rpb = RT;
    t.rpb = rpb;
    dim3 grid((RT + rpb - 1) / rpb, max_active, zp);
    if (nt == 1) k_tile_run<FMT, NPROJ, 1><<<grid, 256, 0, st>>>(t);
    else k_tile_run<FMT, NPROJ, 2><<<grid, 256, 0, st>>>(t);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

#ifndef MOE_TILE_DMA_NT
#define MOE_TILE_DMA_NT 0   // token tiles per pass up to which the DMA-ring kernels run (0: never; measured
                            // slower than the register-staged tiles at the Qwen3 T = 16..64 shapes)
#endif

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
    t.kslots = a.k;
    if (a.stages & 1) {
        int rc = launch_group(a.idx, nslots, w->E, a.grp.counts, a.grp.offsets, a.grp.sorted, a.grp.active,
                              a.grp.meta, a.st);
        if (rc) return rc;
        TileArgs g = t;
        g.actv = (const uint16_t*)a.x;
        if (nt <= MOE_TILE_DMA_NT) {   // the DMA tiles read x in the decoded-code order
            const size_t np = (size_t)a.T * w->d / 8;
            k_pair8_rows<<<(unsigned)((np + 255) / 256), 256, 0, a.st>>>((const uint4*)a.x, (uint4*)a.xperm, np);
            g.actv = a.xperm;
        }
        g.act_div = a.k;
        g.K = w->d;
        g.N = w->F;
        g.W0 = (const uint8_t*)w->gate.rows;
        g.W1 = (const uint8_t*)w->up.rows;
        g.b0 = w->gate.bias;
        g.b1 = w->up.bias;
        g.hout = a.hhi;
        g.hout2 = a.hlo;
        rc = nt <= MOE_TILE_DMA_NT ? launch_tile_dma<FMT, 2>(g, nt, max_active, a.T, a.st)
                                   : launch_tile<FMT, 2>(g, nt, max_active, a.T, a.st);
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
        d.yp = a.yp;
        int rc = nt <= MOE_TILE_DMA_NT ? launch_tile_dma<FMT, 1>(d, nt, max_active, a.T, a.st)
                                       : launch_tile<FMT, 1>(d, nt, max_active, a.T, a.st);
        if (rc) return rc;
        return launch_combine(a.yp, a.idx, a.wts, w->down.bias, w->E, a.residual, a.y, a.T, a.k, w->d, a.y32, a.st);
    }
    return 0;
}

}  // namespace

int run_experts_tiles(const ExpertsArgs& a) {
    return a.w->fmt == MOE_FMT_INT4_G64 ? run_tiles_fmt<FmtInt4>(a) : run_tiles_fmt<FmtMxfp4>(a);
}

}  // namespace moe

// Grouped expert tiles for T > 1 on bf16 MFMA (gfx950 v_mfma_f32_16x16x32_bf16): the expert-tile grouped
// GEMM of the reference's T > 1 path (metal_q4_tiles_v2.py:160-360 gate/up and down tiles, one MMA tile per
// 8 rows x 8 slots there), re-cut for 64-wide waves and MFMA. Two kernels, by weight layout:
//   k_wave_tile  tile-major weights (moe_tiles_pack): one wave per 16 * RT rows and 16 tokens, no LDS, every
//                weight load a contiguous 1 KB burst (the fast path; layout and method described below);
//   k_tile       row records only: a block per 64 rows, K slices staged through LDS (described here).
// Arithmetic, both (exact operands, fp32 accumulation; the reference's raw-code MMA with per-group fp32 fix-up,
// metal_q4_tiles_v2.py:242-263): codes decode to bf16 128 + q (int4) or e2m1(q) (MXFP4), exactly; per scale
// group the MFMA sums P = sum (128 + q) x over the group and, for int4, XS = sum x from one more MFMA with an
// all-ones operand; then acc += s * P + (b - 128 s) * XS (int4) or acc += 2^(s-127) * P (MXFP4).
// The GLU output h is stored as two bf16 planes h = hi + lo (about 16 significant bits; the reference keeps
// it in x.dtype); the down projection runs one MFMA per plane into the same accumulator. The down output is
// yp[slot] = W_down h in fp32; k_combine adds b_down, applies the routing weights and sums a token's slots.
//
// k_tile: a block owns one active expert and TL_ROWS = 64 weight rows (16 per wave). For gate/up the same wave
// owns gate row r and up row r, so the GLU is applied in registers; for down it owns 16 rows of W_down. The
// expert's slots (stable, ascending slot id: the grouping of moe_group) are taken 16 * NT at a time, pass z
// of an expert by the block with blockIdx.z = z mod gridDim.z (so a popular expert spreads over blocks); each
// pass streams the block's rows in K slices of TL_KC chunks (256 inputs) through LDS:
//   A (codes): each thread loads 16-byte chunks of the rows and scatters their 4 words so that lane (r, g)
//              later reads word g of the slice's chunks (g = lane / 16 is the MFMA K group of 8 inputs,
//              r = lane % 16 the row);
//   metadata:  int4 (scale, bias - 128 scale) per 64-group, MXFP4 2^(s-127) per 32-group, as fp32;
//   B (activations of the pass's tokens): 16-byte pieces of 8 inputs, reordered (0,4,1,5,2,6,3,7) like the
//              decoded codes; tokens past the expert's count and inputs past K are zero.
// The next slice's global loads are issued before the current slice's MFMAs (register double buffer).
#include "moe_common.h"
#include "moe_formats.h"
#include "moe_group.h"
#include "moe_internal.h"
#include "moe_mxterms.h"

#include <math.h>
#include <stdlib.h>

#include <type_traits>

namespace moe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2x __attribute__((ext_vector_type(2)));

// Power-of-two exponent e with which the int4 dense tiles store a row (x16: a token's x; h16: a slot's 32-row chunk
// of h) of largest magnitude amax as fp16 v 2^-e: 0 while 2^-8 <= amax < 2^15 (fp16's subnormal rounding, 2^-25,
// then stays below 2^-17 of the row's largest), else floor(log2 amax) - 14, which puts the largest at [2^14, 2^15)
// (large rows: no overflow; small rows: no flush to zero), clamped to [-127, 127]. An all-zero row gives
// H16_ZERO_EXP, which never wins a slot's maximum (its values are 0 under any scaling); NaN gives 0.
constexpr int H16_ZERO_EXP = -128;
__device__ __forceinline__ int h16_exponent(float amax) {
    if (amax == 0.f) return H16_ZERO_EXP;
    if (!(amax < 32768.f && amax >= 0.00390625f)) {
        if (amax != amax) return 0;
        const int e = (int)((__float_as_uint(amax) >> 23) & 0xFFu) - 141;
        return e < -127 ? -127 : (e > 127 ? 127 : e);
    }
    return 0;
}
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int TL_ROWS = 64;   // weight rows per block
constexpr int TL_KC = 8;      // chunks (32 inputs) per K slice
constexpr int TL_APAD = 4 * TL_KC + 4;   // words per staged row: [g 0..3][chunk 0..KC-1] + 4 words of padding
constexpr int TL_BPAD = 4 * TL_KC + 1;   // 16-byte pieces per staged token (8 inputs each) + 1 of padding
constexpr int TL_GMAX = TL_KC;           // scale groups per slice at most (MXFP4: one per chunk)


// Byte of record-term position of input k (0..127) of a slice: the code order of the tile records within each
// word (inputs 8 i + (0 2 4 6 1 3 5 7)), then the A operand's lane order (bytes 32 g .. 32 g + 15: logical inputs
// 16 g .. 16 g + 15, bytes 32 g + 16 .. 32 g + 31: 64 + 16 g .. 64 + 16 g + 15)
__device__ __forceinline__ int mx_pos(int k) {
    const int e = k & 7;
    const int l = (k & ~7) | ((e >> 1) + 4 * (e & 1));
    return 32 * ((l & 63) >> 4) + 16 * (l >> 6) + (l & 15);
}

// One token's h on the 32 rows of a wave's block b of slice s (lane lr of its lane group: rows 16 rt + lr of
// the block, values h0 (rt 0) and h1 (rt 1)) -> the NTERM term bytes and scale bytes of that block in the token's
// record rec (the layout k_mx_terms writes). The 16 lanes of the group take part in the max reductions; only
// `write` lanes store. pad: also the zero blocks 2, 3 of a slice that ends at input 64 (K % 128 == 64).
template <int NTERM>
__device__ __forceinline__ void mx_h_block(float h0, float h1, bool write, uint8_t* rec, int b, int lr, bool pad) {
    const int p0 = mx_pos(32 * b + lr), p1 = mx_pos(32 * b + 16 + lr);
#pragma unroll
    for (int t = 0; t < NTERM; ++t) {
        float am = fmaxf(fabsf(h0), fabsf(h1));
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
        int e = am > 0.f ? (int)((__float_as_uint(am) >> 23) & 0xFFu) - 127 - 7 : -127;
        e = e < -127 ? -127 : (e > 127 ? 127 : e);
        const float inv = __builtin_ldexpf(1.f, -e);
        const uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(h0 * inv, h1 * inv, 0, false);
        h0 -= __builtin_ldexpf(__builtin_amdgcn_cvt_f32_fp8((int)w, 0), e);
        h1 -= __builtin_ldexpf(__builtin_amdgcn_cvt_f32_fp8((int)w, 1), e);
        if (write) {
            rec[128 * t + p0] = (uint8_t)(w & 0xFFu);
            rec[128 * t + p1] = (uint8_t)((w >> 8) & 0xFFu);
            if (lr == 0) rec[128 * NTERM + 4 * t + b] = (uint8_t)(e + 127);
        }
    }
    if (pad && write && lr < 2 * NTERM) {   // blocks 2 and 3: lane lr zeroes term lr >> 1's block 2 + (lr & 1)
        const int t = lr >> 1, bz = 2 + (lr & 1);
        uint8_t* z = rec + 128 * t + 64 * (bz & 1) + 16 * (bz >> 1);
        *reinterpret_cast<uint4*>(z) = uint4{0u, 0u, 0u, 0u};
        *reinterpret_cast<uint4*>(z + 32) = uint4{0u, 0u, 0u, 0u};
        rec[128 * NTERM + 4 * t + bz] = 127;
    }
}

// Field order: what the tile kernels' prologues read (the in-kernel grouping's ids, the weight and activation
// bases, the shapes, the pass lists) fills the first two 64-byte scalar-cache lines, so the prologue's scalar loads
// miss once instead of once per line; epilogue-only fields follow.
struct TileArgs {
    const int32_t* gidx;   // wave tiles: when set, each workgroup finds its pass from these raw ids (gn = T k of them)
    const uint8_t* W0;     // gate (or down) row records [E, N, rb]
    const uint8_t* W1;     // up row records (gate/up only)
    const uint16_t* actv;  // gate/up: x [T, K] (bf16 plane 0); down: h [T*k, K] (bf16; the hi plane of h = hi + lo)
    const uint16_t* actv2; // down: the lo plane of h
    size_t act_plane;      // gate/up with fp16 / fp32 x: elements between x's bf16 planes (k_x_planes)
    int gn, gfirst;        // instead of the grouping kernel's pass list (gfirst: expert-major first passes)
    int K, N;
    int E, act_div;        // act_div: activation row of slot p is p / act_div (k for gate/up, 1 for down)
    int nidx;              // 2 (first pass list) or 3 (second)
    int act;               // GLU kind (gate/up)
    const int32_t* meta;
    const int32_t* items;  // wave and dense tiles: pass list (expert, pass, passes), meta[nidx] passes
    const int32_t *counts, *offsets, *sorted;
    // gate/up wave tiles grouping in-kernel: the workgroup (0, emit_y) (the grid's last row, set by the launch) also
    // writes the grouping and the pass lists of these ids (as the grouping launch would) for the down stage;
    // emit_grp.counts null: none
    int emit_y;
    // down wave tiles from the emitted pass list: with at least this many live waves (passes x row blocks) a wave
    // keeps one slice in flight instead of D (0: always D)
    int shallow_min;
    GroupBufs emit_grp;
    int emit_P, emit_P2;
    const int32_t* active;
    const float* b0;       // additive row biases [E, N] (gpt-oss) or null
    const float* b1;
    int rpb;               // row tiles per block (k_tile_run)
    int kslots;            // k (slots per token)
    uint16_t* hout;        // gate/up: h = hi + lo as two bf16 planes [T*k, N]
    uint16_t* hout2;
    float* yp;             // down: [T*k, N] fp32 (dense tiles split over K: ksplit such planes, plane floats apart)
    int ksplit;
    size_t plane;
    size_t eslot_off;      // dense int4 down: per-slot exponents (int32 [slots]) at this byte offset from the exponent bytes
    const int32_t* xexp;   // dense int4 gate/up: per-token exponents of x16 (actv) [T]
    uint8_t* hterm;        // block-scaled MXFP4 gate/up: h leaves as 3-term records [T*k][ceil(N/128)] (no planes)
};

// In-kernel grouping, one wave: pass y of the wave tiles' pass list (passes of P slots; an expert's slots in
// ascending slot id, the grouping kernel's order within each expert) from the raw ids idx[0 .. n)
// (n <= 64 * GW_MAXJ). With first = 1 the list is expert-major: pass y < E is the first pass (ranks 0 .. P-1) of
// expert y, found from the ids alone (a ballot per 64 ids); passes E, E + 1, ... are the further passes (q >= 1)
// expert by expert. With first = 0 every pass is in the second, compact part (passes expert by expert from y = 0).
// The compact part takes an LDS histogram (sCnt [E]) and a wave scan of the per-expert pass counts.
// Returns false when pass y is empty (expert without slots, or past the last pass); else e, the pass's first
// rank tok0 within the expert, the expert's slot count cnt, and sSlot[0 .. min(P, cnt - tok0)) the pass's slots.
// Slots whose id is outside [0, E) join no pass. Called by whole one-wave workgroups.
constexpr int GW_MAXJ = 16;
__device__ __forceinline__ bool wave_find_pass(const int32_t* __restrict__ idx, int n, int E, int P, int first,
                                               int y, int* sCnt, int* sSlot, int& e, int& tok0, int& cnt) {
    const int lane = threadIdx.x & 63;
    int id[GW_MAXJ];
#pragma unroll
    for (int j = 0; j < GW_MAXJ; ++j) {
        const int p = lane + 64 * j;
        id[j] = p < n ? idx[p] : -1;
    }
    if (first && y < E) {
        e = y;
        tok0 = 0;
    } else {
        const int w = first ? y - E : y;
        for (int i = lane; i < E; i += 64) sCnt[i] = 0;
        __syncthreads();   // one-wave workgroup: orders the LDS accesses
#pragma unroll
        for (int j = 0; j < GW_MAXJ; ++j)
            if ((unsigned)id[j] < (unsigned)E) atomicAdd(&sCnt[id[j]], 1);
        __syncthreads();
        int run = 0;
        bool found = false;
        for (int base = 0; base < E && !found; base += 64) {
            const int ee = base + lane;
            const int c = ee < E ? sCnt[ee] : 0;
            const int np = c > 0 ? (c - 1) / P + 1 - first : 0;   // the expert's passes in this part
            const int inc = wave_incl_scan(np);
            const int excl = run + inc - np;
            const uint64_t hit = __ballot(np > 0 && excl <= w && w < excl + np);
            if (hit) {   // wave-uniform results: scalar registers for the tile bases
                const int src = __builtin_ctzll(hit);
                e = __builtin_amdgcn_readlane(ee, src);
                tok0 = (first + w - __builtin_amdgcn_readlane(excl, src)) * P;
                found = true;
            }
            run += __builtin_amdgcn_readlane(inc, 63);
        }
        if (!found) return false;
    }
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    int seen = 0;
#pragma unroll
    for (int j = 0; j < GW_MAXJ; ++j) {
        const bool m = id[j] == e;
        const uint64_t mask = __ballot(m);
        const int rank = seen + __popcll(mask & lt);
        if (m && rank >= tok0 && rank < tok0 + P) sSlot[rank - tok0] = lane + 64 * j;
        seen += __popcll(mask);
    }
    cnt = __builtin_amdgcn_readfirstlane(seen);
    if (tok0 >= cnt) return false;
    __syncthreads();
    return true;
}

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
template <class FMT, int NPROJ, int NT, int HX = 1>
__global__ void __launch_bounds__(256, MOE_TILE_MINB)
k_tile(TileArgs a) {
    constexpr int NTOK = 16 * NT;
    constexpr bool INT4 = FMT::XSUM;
    constexpr int HL = NPROJ == 2 ? HX : 2;   // activation planes: x's (1, or 2-3 for fp16 / fp32 x), h = hi + lo
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
                        rbv[hl][i] = *reinterpret_cast<const uint4*>(
                            (NPROJ == 2 ? a.actv + hl * a.act_plane : (hl ? a.actv2 : a.actv)) + brow[i] + k0);
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
            constexpr int CPG = INT4 ? 2 : 1;   // chunks per scale group
#pragma unroll
            for (int gi = 0; gi < TL_KC / CPG; ++gi) {
                __builtin_amdgcn_sched_barrier(0);
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
                        FMT::decode_word(sA[p][16 * wave + lr][TL_KC * lg + gi * CPG + cc], q);
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

// ============================================================================ wave tiles (tile-major weights)
// The grouped path's weights in the tile-major layout of moe_tiles_pack (include/moe_mi355x.h): for every
// expert, 16-row tile and slice of 128 inputs, one contiguous record holding the 16 rows' codes already in
// the MFMA operand order, then their group metadata. A wave's load of one slice of one tile is one 1 KB
// contiguous burst (16 B per lane, lane order); HBM streams such bursts near its peak, where loads that
// stride across row records (16 rows x 64 B per instruction) do not.
//
// Each 64-lane wave is a workgroup of its own and owns 16 * RT rows (of gate and up, or of down) for 16 * NT
// tokens of one expert; there is no LDS and no barrier. The product is computed token-major,
// D[token, row] = X[token, :] . W[row, :], on v_mfma_f32_16x16x32_bf16 with the activations as the A operand
// (lane (m, g) = token m, 8 inputs) and the decoded codes as the B operand (lane (r, g) = row r, 8 codes), so
// an output lane holds 4 tokens of ONE row and needs that row's group metadata only.
// A slice is 4 MFMA steps j; lane (r, g) holds the 4 code words it supplies, word j for step j, which are the
// row's words (w = 16 s + ...)
//     int4 g64:  j = 0, 1: 2 g + j        j = 2, 3: 8 + 2 g + (j - 2)     (steps 0,1 group 2s; 2,3 group 2s+1)
//     MXFP4 g32: 4 j + g                                                  (step j = group 4 s + j)
// and the A lane of token m loads the 8 activations of the same word (the piece with its index). The records
// store each word's nibbles interleaved (elements 0,2,4,6,1,3,5,7), so the 7-op decode yields its codes in
// natural order and x and h are read as they lie in memory.
// Every global load of slice s is issued D slices ahead into a register ring, in one fixed order, so the
// in-order vmcnt wait for slice s leaves the D - 1 slices behind it in flight.
// Tokens past the expert's count load the count's last token again (same addresses: no extra traffic); their
// D rows are dropped (a row of D depends on the same row of X only). Inputs past K (the last slice when
// K % 128 == 64) have zero codes and zero metadata in the record, and their activation loads are clamped into
// the row, so they add 0.
template <class FMT>
__host__ __device__ constexpr int tile_slice_bytes() {
    return FMT::XSUM ? TILE_SLICE_INT4 : TILE_SLICE_MXFP4;
}

// H16O (int4 gate/up before a dense down): h leaves as fp16 h16 = h 2^-e with e per (slot, 32-row chunk), the
// layout the dense down reads after k_h16_fix, instead of the two bf16 planes.
// MXT > 0 (MXFP4, bf16 x): the activations are fp8 term records (k_mx_terms, MXT terms) and the products run on
// the block-scaled MFMA (the weights undecoded, as in k_mxd)
template <class FMT, int NPROJ, int NT, int RT, int D, bool H16O = false, int HX = 1, int MXT = 0>
__global__ void __launch_bounds__(64) k_wave_tile(TileArgs a) {
    static_assert(!H16O || (NPROJ == 2 && RT % 2 == 0), "h16 output: gate/up, whole 32-row chunks per wave");
    static_assert(MXT == 0 || (!FMT::XSUM && HX == 1 && !H16O), "block-scaled: MXFP4, one activation source");
    constexpr bool INT4 = FMT::XSUM;
    constexpr int HL = NPROJ == 2 ? HX : 2;   // activation planes: x's (1, or 2-3 for fp16 / fp32 x), h = hi + lo
    constexpr int SB = tile_slice_bytes<FMT>();
    // in-kernel grouping from raw ids (a.gidx): the gate/up stage, and the block-scaled down that groups for itself;
    // the other downs always read a pass list (the launch rejects a.gidx for them)
    constexpr bool GIDX = NPROJ == 2 || MXT > 0;
    __shared__ int sCnt[GIDX ? 1024 : 1];       // in-kernel grouping: counts per expert (E <= 1024)
    __shared__ int sSlot[GIDX ? 16 * NT : 1];   // and the pass's slots
    int e, tok0, n, beg = 0;
    bool shallow = false;   // see TileArgs::shallow_min
    if constexpr (NPROJ == 2 && MXT == 0) {
        // the lists for the down stage, by the workgroup of the last row (usually past the live passes), first: its
        // own pass may be empty (not in the block-scaled variants: it would cost them occupancy)
        __shared__ int sGrp[NPROJ == 2 ? 2 * 1024 + 4 * 16 : 1];
        if (a.emit_grp.counts && blockIdx.x == 0 && (int)blockIdx.y == a.emit_y) {
            const int32_t* ids = a.gidx;
            group_block([&](int p) { return ids[p]; }, a.gn, a.E, a.emit_grp, a.emit_P, a.emit_P2, sGrp, 0);
        }
    }
    // slot of the lane's activation row (A side: token tok0 + 16 t + lr), read in each branch from its own memory:
    // a load through a pointer chosen between LDS and global memory is a flat load, which the compiler waits for
    // with a full vmcnt(0), ahead of the first weight loads
    int slotA[NT];
    if (GIDX && a.gidx) {
        if (!wave_find_pass(a.gidx, a.gn, a.E, 16 * NT, a.gfirst, (int)blockIdx.y, sCnt, sSlot, e, tok0, n))
            return;
        e = __builtin_amdgcn_readfirstlane(e);
        tok0 = __builtin_amdgcn_readfirstlane(tok0);
        const __attribute__((address_space(3))) int* ls = (const __attribute__((address_space(3))) int*)sSlot;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int m = tok0 + 16 * t + (int)(threadIdx.x & 15);
            slotA[t] = ls[(m < n ? m : n - 1) - tok0];
        }
    } else {
        // the row's list entry is read with the pass count, in one round trip: the list has room for the grid's
        // rows (max_passes of the launch's pass size), so the entry exists for rows past the live passes too, which
        // return before using it; the exit test reads both, so neither load waits for the other, and keeps a bad
        // entry's id off the weight addresses
        const int npass = a.meta[a.nidx];
        const int e_l = a.items[3 * blockIdx.y], p_l = a.items[3 * blockIdx.y + 1];
        const bool past = (int)blockIdx.y >= npass, bad = ((unsigned)e_l >= (unsigned)a.E) | (p_l < 0);
        if (past | bad) return;   // one pass of the work list per workgroup row
        shallow = a.shallow_min > 0 && npass * (a.N / (16 * RT)) >= a.shallow_min;
        e = e_l;
        tok0 = p_l * 16 * NT;
        n = a.counts[e];
        beg = a.offsets[e];
        const __attribute__((address_space(1))) int* gs = (const __attribute__((address_space(1))) int*)a.sorted;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int m = tok0 + 16 * t + (int)(threadIdx.x & 15);
            slotA[t] = gs[beg + (m < n ? m : n - 1)];
        }
    }
    const int lane = threadIdx.x, lr = lane & 15, lg = lane >> 4;
    const int K = a.K, N = a.N;
    const int nsl = (K + 127) >> 7;
    const int lastp = (K >> 3) - 1;   // last activation piece of a row
    const int r0 = blockIdx.x * 16 * RT;
    // wave-uniform tile bases (tile r0 / 16 + rt of expert e); lane offsets stay 32-bit
    const uint8_t* tb[NPROJ][RT];
#pragma unroll
    for (int p = 0; p < NPROJ; ++p)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            tb[p][rt] = (p ? a.W1 : a.W0) + ((size_t)e * (N >> 4) + (r0 >> 4) + rt) * (size_t)nsl * SB;
    const uint32_t ones = 0x3F803F80u;
    const bf16x8 ONES = as_bf16x8(ones, ones, ones, ones);

    {
        // byte offset of the lane's activation row (A side: token tok0 + 16 t + lr)
        uint32_t xo[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) xo[t] = (uint32_t)(slotA[t] / a.act_div) * (uint32_t)K * 2u;
        f32x4 acc[NPROJ][RT][NT];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[p][rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (MXT > 0) {
            typedef int v8i __attribute__((ext_vector_type(8)));
            constexpr int REC = mx_rec<MXT>();
            const uint8_t* xrec = reinterpret_cast<const uint8_t*>(a.actv);
            uint32_t ro[NT];   // byte offset of the lane's token's records
#pragma unroll
            for (int t = 0; t < NT; ++t) ro[t] = (uint32_t)(slotA[t] / a.act_div) * (uint32_t)nsl * (uint32_t)REC;
            // register ring: code words, E8M0 words, the lane's 32 bytes of each term and the terms' scale words
            uint4 rq[D][NPROJ][RT];
            uint32_t rm[D][NPROJ][RT];
            uint4 ra[D][MXT][NT][2];
            uint32_t rs[D][MXT][NT];
            auto issue = [&](int s, uint4 (&q)[NPROJ][RT], uint32_t (&m)[NPROJ][RT], uint4 (&x)[MXT][NT][2],
                             uint32_t (&xs)[MXT][NT]) {
#pragma unroll
                for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const uint8_t* sl = tb[p][rt] + (uint32_t)s * (uint32_t)SB;
                        q[p][rt] = *reinterpret_cast<const uint4*>(sl + 16 * lane);
                        m[p][rt] = *reinterpret_cast<const uint32_t*>(sl + 1024 + 4 * lr);
                    }
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int tm = 0; tm < MXT; ++tm) {
                        const uint8_t* r = xrec + (ro[t] + (uint32_t)s * (uint32_t)REC);
                        x[tm][t][0] = *reinterpret_cast<const uint4*>(r + 128 * tm + 32 * lg);
                        x[tm][t][1] = *reinterpret_cast<const uint4*>(r + 128 * tm + 32 * lg + 16);
                        xs[tm][t] = *reinterpret_cast<const uint32_t*>(r + 128 * MXT + 4 * tm);
                    }
            };
            auto compute = [&](bool live, const uint4 (&q)[NPROJ][RT], const uint32_t (&m)[NPROJ][RT],
                               const uint4 (&x)[MXT][NT][2], const uint32_t (&xs)[MXT][NT]) {
                if (!live) return;   // wave-uniform: slices past the last (the ring's rounding)
                v8i B[NPROJ][RT];
                int sb[NPROJ][RT];
#pragma unroll
                for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        // lane group g: words (g, 4 + g, 8 + g, 12 + g) -> (4 g .. 4 g + 3), i.e. block g
                        const uint4 v = q[p][rt];
                        const auto s0 = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
                        const auto s1 = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
                        const auto t0 = __builtin_amdgcn_permlane16_swap(s0[0], s1[0], false, false);
                        const auto t1 = __builtin_amdgcn_permlane16_swap(s0[1], s1[1], false, false);
                        B[p][rt] = v8i{(int)t0[0], (int)t0[1], (int)t1[0], (int)t1[1], 0, 0, 0, 0};
                        sb[p][rt] = (int)(m[p][rt] >> (8 * lg));
                    }
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int tm = 0; tm < MXT; ++tm) {
                        const uint4 a0 = x[tm][t][0], a1 = x[tm][t][1];
                        const v8i A = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
                        const int sa = (int)(xs[tm][t] >> (8 * lg));
#pragma unroll
                        for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                            for (int rt = 0; rt < RT; ++rt)
                                acc[p][rt][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                                    A, B[p][rt], acc[p][rt][t], 0, 4, 0, sa, 0, sb[p][rt]);
                    }
            };
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < D; ++i) {
                issue(i < nsl ? i : nsl - 1, rq[i], rm[i], ra[i], rs[i]);
                __builtin_amdgcn_sched_barrier(0);
            }
            for (int s0 = 0; s0 < nsl; s0 += D) {
#pragma unroll
                for (int i = 0; i < D; ++i) {
                    compute(s0 + i < nsl, rq[i], rm[i], ra[i], rs[i]);
                    __builtin_amdgcn_sched_barrier(0);
                    const int sn = s0 + i + D;
                    issue(sn < nsl ? sn : nsl - 1, rq[i], rm[i], ra[i], rs[i]);
                }
            }
        } else {
        const uint8_t* xbase[HL];
#pragma unroll
        for (int hl = 0; hl < HL; ++hl)
            xbase[hl] = reinterpret_cast<const uint8_t*>(NPROJ == 2 ? a.actv + hl * a.act_plane : (hl ? a.actv2 : a.actv));
        // register ring: code words, metadata, activation pieces of D slices
        uint4 rq[D][NPROJ][RT];
        uint2 rm[D][NPROJ][RT];
        uint4 rx[D][HL][NT][4];
        auto issue = [&](int s, uint4 (&q)[NPROJ][RT], uint2 (&m)[NPROJ][RT], uint4 (&x)[HL][NT][4]) {
#pragma unroll
            for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const uint8_t* sl = tb[p][rt] + (uint32_t)s * (uint32_t)SB;
                    q[p][rt] = *reinterpret_cast<const uint4*>(sl + 16 * lane);
                    if (INT4) m[p][rt] = *reinterpret_cast<const uint2*>(sl + 1024 + 8 * lr);
                    else m[p][rt].x = *reinterpret_cast<const uint32_t*>(sl + 1024 + 4 * lr);
                }
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        int piece = INT4 ? 16 * s + 8 * (j >> 1) + 2 * lg + (j & 1) : 16 * s + 4 * j + lg;
                        piece = piece < lastp ? piece : lastp;
                        x[hl][t][j] = *reinterpret_cast<const uint4*>(xbase[hl] + (xo[t] + 16u * piece));
                    }
        };
        auto compute = [&](bool live, const uint4 (&q)[NPROJ][RT], const uint2 (&m)[NPROJ][RT],
                           const uint4 (&x)[HL][NT][4]) {
            bf16x8 X[HL][NT][4];
#pragma unroll
            for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint4 v = x[hl][t][j];
                        X[hl][t][j] = as_bf16x8(v.x, v.y, v.z, v.w);
                    }
            f32x4 xs[NT][2];   // int4: sum of the activations over each of the slice's two groups
            if (INT4) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int G = 0; G < 2; ++G) {
                        xs[t][G] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                            for (int u = 0; u < 2; ++u)
                                xs[t][G] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(X[hl][t][2 * G + u], ONES, xs[t][G], 0, 0, 0);
                    }
            }
            if constexpr (INT4) {
                // software-pipelined over the (projection, row tile) items: the products of item i + 1 are issued
                // before item i's group sums are folded into acc, so the fold does not wait on the MFMAs it reads
                // (folding each item right after its own products stalled on them: ~10 us of a Qwen3 T=32 layer).
                // Each acc element still takes its groups in the same order, so the sums are unchanged.
                constexpr int NI = NPROJ * RT;
                f32x4 Pr[2][2][NT];   // [item parity][group][token tile]
                auto products = [&](int i, f32x4 (&P)[2][NT]) __attribute__((always_inline)) {
                    const int p = i / RT, rt = i % RT;
                    const uint32_t w4[4] = {q[p][rt].x, q[p][rt].y, q[p][rt].z, q[p][rt].w};
                    bf16x8 B[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        uint32_t c4[4];
                        FMT::decode_word(w4[j], c4);
                        B[j] = as_bf16x8(c4[0], c4[1], c4[2], c4[3]);
                    }
#pragma unroll
                    for (int G = 0; G < 2; ++G)
#pragma unroll
                        for (int t = 0; t < NT; ++t) {
                            P[G][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                                for (int u = 0; u < 2; ++u)
                                    P[G][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(X[hl][t][2 * G + u], B[2 * G + u],
                                                                                      P[G][t], 0, 0, 0);
                        }
                };
                auto fold = [&](int i, const f32x4 (&P)[2][NT]) __attribute__((always_inline)) {
                    const int p = i / RT, rt = i % RT;
#pragma unroll
                    for (int G = 0; G < 2; ++G) {
                        const uint32_t mw = live ? (G ? m[p][rt].y : m[p][rt].x) : 0u;
                        const float sc = bf16lo(mw), cb = __builtin_fmaf(-128.f, sc, bf16hi(mw));
#pragma unroll
                        for (int t = 0; t < NT; ++t)
#pragma unroll
                            for (int v = 0; v < 4; ++v)
                                acc[p][rt][t][v] = __builtin_fmaf(sc, P[G][t][v], __builtin_fmaf(cb, xs[t][G][v], acc[p][rt][t][v]));
                    }
                };
                products(0, Pr[0]);
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    if (i + 1 < NI) products(i + 1, Pr[(i + 1) & 1]);
                    fold(i, Pr[i & 1]);
                }
            } else {
#pragma unroll
            for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const uint32_t w4[4] = {q[p][rt].x, q[p][rt].y, q[p][rt].z, q[p][rt].w};
                    bf16x8 B[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        uint32_t c4[4];
                        FMT::decode_word(w4[j], c4);
                        B[j] = as_bf16x8(c4[0], c4[1], c4[2], c4[3]);
                    }
                    {
                        const uint32_t mw = live ? m[p][rt].x : 0u;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const float sc = __uint_as_float(((mw >> (8 * j)) & 0xFFu) << 23);
#pragma unroll
                            for (int t = 0; t < NT; ++t) {
                                f32x4 P = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                                for (int hl = 0; hl < HL; ++hl)
                                    P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(X[hl][t][j], B[j], P, 0, 0, 0);
#pragma unroll
                                for (int v = 0; v < 4; ++v) acc[p][rt][t][v] = __builtin_fmaf(sc, P[v], acc[p][rt][t][v]);
                            }
                        }
                    }
                }
            }
        };
        // int4: the records hold each row's scales and biases times 2^-E (E per row, moe_tiles_pack), so the
        // sums come back by 2^E in the epilogue. Only the epilogue reads the lane's exponents: they are loaded after
        // the ring's first slices, which then do not wait for them
        int rex[NPROJ][RT];
        auto load_rex = [&]() __attribute__((always_inline)) {
#pragma unroll
            for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    rex[p][rt] = INT4 ? tile_row_exps(p ? a.W1 : a.W0, a.E, N, K)[(size_t)e * N + r0 + 16 * rt + lr] : 0;
        };
        __builtin_amdgcn_sched_barrier(0);
        if (NPROJ == 1 && D > 1 && shallow) {
            // many live waves: one slice in flight per wave. The launch's waves already request more than the
            // memory system drains in a latency, and a deeper ring only lengthens its queues: Qwen3 down stage
            // 24.6 -> 23.9, 27.7 -> 26.2, 31.2 -> 29.5 us at T = 16, 32, 64 uniform, while the Zipf(1.1) routings,
            // with a few hundred live waves, keep the ring they need (a threshold of 1536 misses T = 16, 2560 all)
            issue(0, rq[0], rm[0], rx[0]);
            load_rex();
            for (int s = 0; s < nsl; ++s) {
                compute(true, rq[0], rm[0], rx[0]);
                __builtin_amdgcn_sched_barrier(0);
                if (s + 1 < nsl) issue(s + 1, rq[0], rm[0], rx[0]);
            }
        } else {
        // ring: slices s0 .. s0 + D - 1 in flight at the top of each step. The walk is rounded up to a multiple
        // of D: slices past the last re-load the last one (cache hits) and fold with scale 0, so the loop body
        // has no branch. Issued slice by slice in the steady state's order, so the vmcnt waits at the loop top
        // are the same on entry and on the back edge.
#pragma unroll
        for (int i = 0; i < D; ++i) {
            issue(i < nsl ? i : nsl - 1, rq[i], rm[i], rx[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
        load_rex();
        for (int s0 = 0; s0 < nsl; s0 += D) {
#pragma unroll
            for (int i = 0; i < D; ++i) {
                compute(s0 + i < nsl, rq[i], rm[i], rx[i]);
                // keep the slot's re-load below its last reads, so each slot stays in one register set
                __builtin_amdgcn_sched_barrier(0);
                const int sn = s0 + i + D;
                issue(sn < nsl ? sn : nsl - 1, rq[i], rm[i], rx[i]);
            }
        }
        }
        if constexpr (INT4) {
#pragma unroll
            for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[p][rt][t][v] = __builtin_ldexpf(acc[p][rt][t][v], rex[p][rt]);
        }
        }   // MXT == 0
        // ---- epilogue: lane holds row r0 + 16 rt + lr of tokens tok0 + 16 t + 4 lg + v
        if constexpr (MXT > 0 && NPROJ == 2) {   // h as the down's 3-term records: this wave's 32 rows = one block
            static_assert(RT == 2, "one 32-row block of h per wave");
            if (a.hterm) {
                const int nslN = (N + 127) >> 7, bk = (r0 & 127) >> 5;
                const bool pad = (N & 127) == 64 && (r0 >> 7) == nslN - 1 && bk == 1;
#pragma unroll
                for (int t = 0; t < NT; ++t)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int j = 4 * lg + v;
                        const int slot = __shfl(slotA[t], j, 64);   // lane j (any lane group) holds token j's slot
                        float hv[RT];
#pragma unroll
                        for (int rt = 0; rt < RT; ++rt) {
                            const int r = r0 + 16 * rt + lr;
                            float g = acc[0][rt][t][v], up = acc[1][rt][t][v];
                            if (a.b0) g += a.b0[(size_t)e * N + r];
                            if (a.b1) up += a.b1[(size_t)e * N + r];
                            hv[rt] = glu_act(a.act, g, up);
                        }
                        mx_h_block<3>(hv[0], hv[1], tok0 + 16 * t + j < n,
                                      a.hterm + ((size_t)slot * nslN + (r0 >> 7)) * mx_rec<3>(), bk, lr, pad);
                    }
                return;
            }
        }
        if constexpr (H16O) {
            int8_t* hexp_out = reinterpret_cast<int8_t*>(a.hout2);
            const int nch = N >> 5;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int j = 4 * lg + v;
                    const int slot = __shfl(slotA[t], j, 64);   // lane j (any lane group) holds token j's slot
                    float hv[RT];
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const int r = r0 + 16 * rt + lr;
                        float g = acc[0][rt][t][v], up = acc[1][rt][t][v];
                        if (a.b0) g += a.b0[(size_t)e * N + r];
                        if (a.b1) up += a.b1[(size_t)e * N + r];
                        hv[rt] = glu_act(a.act, g, up);
                    }
                    int ex[RT / 2];
#pragma unroll
                    for (int c = 0; c < RT / 2; ++c) {   // 32-row chunk c: row tiles 2c, 2c + 1
                        float am = fmaxf(fabsf(hv[2 * c]), fabsf(hv[2 * c + 1]));
#pragma unroll
                        for (int o = 1; o < 16; o <<= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
                        ex[c] = h16_exponent(am);
                    }
                    if (tok0 + 16 * t + j >= n) continue;
#pragma unroll
                    for (int c = 0; c < RT / 2; ++c)
                        if (lr == 0) hexp_out[(size_t)slot * nch + (r0 >> 5) + c] = (int8_t)ex[c];
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const _Float16 h16 = (_Float16)__builtin_ldexpf(hv[rt], -ex[rt >> 1]);
                        a.hout[(size_t)slot * N + r0 + 16 * rt + lr] = __builtin_bit_cast(uint16_t, h16);
                    }
                }
            return;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int j = 4 * lg + v;
                const int slot = __shfl(slotA[t], j, 64);   // lane j (any lane group) holds token j's slot
                if (tok0 + 16 * t + j >= n) continue;
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const int r = r0 + 16 * rt + lr;
                    if (NPROJ == 2) {
                        float g = acc[0][rt][t][v], up = acc[NPROJ - 1][rt][t][v];
                        if (a.b0) g += a.b0[(size_t)e * N + r];
                        if (a.b1) up += a.b1[(size_t)e * N + r];
                        const float hv = glu_act(a.act, g, up);
                        const uint16_t hi = f32_to_bf16(hv);
                        const size_t o = (size_t)slot * N + r;
                        a.hout[o] = hi;
                        a.hout2[o] = f32_to_bf16(hv - bf16_to_f32(hi));
                    } else {
                        a.yp[(size_t)slot * N + r] = acc[0][rt][t][v];
                    }
                }
            }
    }
}

// ============================================================================ dense tiles (many tokens per expert)
// Where an expert's token count makes the contraction dense (tens to hundreds of tokens per expert: prefill, the
// shared experts), each block keeps its weight tiles for a pass of 64 tokens and multiplies them on MFMA
// against activations staged once per block in LDS. k_dense: a block of 4 waves owns BN rows of one expert (gate
// and up: 128 rows of each, the GLU applied in registers; down: 256 rows) and one pass of the work list (up to
// 16 * NT tokens of it); each wave covers all the pass's tokens for its 64 rows. (8-wave blocks of 128 tokens,
// sharing each weight tile between two token halves, measured slower: one barrier domain per CU instead of two
// independent blocks.) Per K slice of 128 inputs:
//   activations: the pass's token rows, brought into LDS by global_load_lds_dwordx4 (16 bytes per lane, 4 token
//     rows of 256 bytes per instruction); piece p (8 inputs) of token m lies at position p ^ (m & 15) of the
//     token's row, so the MFMA operand reads (16 tokens x one piece) hit distinct banks. Two buffers (distinct
//     objects, so the compiler's LDS-DMA tracking sees that a read of one does not wait for the DMA into the
//     other): slice s + 1 is in flight while slice s is multiplied; one vmcnt(0) + barrier per slice.
//   weights: each wave streams its own 16-row tiles from the tile-major records (1 KB code burst + metadata per
//     tile and slice) into registers one slice ahead and decodes them exactly (int4: bf16 128 + q; MXFP4:
//     e2m1(q)), in natural order (the records interleave each word's nibbles for that).
//   product: token-major like the wave tiles, D[token, row] on v_mfma_f32_16x16x32_bf16 (activations A, codes
//     B) with the same per-group fp32 fold: per scale group P = sum code * x, int4 XS = sum x (one MFMA with an
//     all-ones operand per token tile), acc += s P + (b - 128 s) XS, or acc += 2^(e-127) P.
// Rounding the dequantised weights to bf16 instead would put up to ~2% of RMS of error on the outputs, and h
// kept in one bf16 plane (the reference keeps h in x.dtype) ~1%; the exact operands and h as two bf16 planes
// h = hi + lo (natural order, the wave tiles' layout) keep the error to fp32 accumulation. Down runs one MFMA
// per plane into the same accumulator and writes yp[slot] in fp32 for k_combine.
#define MOE_LDSP(p) ((__attribute__((address_space(3))) void*)(p))
// s_waitcnt vmcnt(0) with the other counters left alone (gfx9 encoding)
#define MOE_VMWAIT0() __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8))
// workgroup barrier without a memory fence; the "memory" clobber keeps LDS accesses on their side of it
#define MOE_BARRIER() asm volatile("s_barrier" ::: "memory")

// Dense tile shapes (measured at the Mixtral T=512 shape). int4 down (operands decoded to fp16 with the scale
// applied, no fold): 32 rows per wave; dense_nt's 128-token passes (each decoded operand feeding 8 MFMAs, 64
// accumulators, 2 waves per SIMD) measured 234 -> 214 us in the kernel alone against 64-token passes, but the call
// runs 64-token passes (make_plan's dn_nt): 4 waves per SIMD and no K split, faster per layer. int4 gate/up keeps
// 64-token passes with 32 rows of each
// projection per wave: with 128 tokens and 16 rows each, every activation slice staged in LDS serves half as many
// rows (K = d is long, the L2 -> LDS traffic doubles) and the kernel slowed 440 -> 509 us. MXFP4 (raw codes on
// bf16 MFMA, fp32 fold per group): 64-token passes, 32 / 64 rows per wave.
// The dense tiles' passes of one expert split its ceil(n / 16) token tiles evenly: pass p of np takes tiles
// [p T / np, (p + 1) T / np), at most ceil(T / np) <= BM / 16 of them. Passes that share a weight tile then do
// the same MFMA work and stream the tile side by side on one XCD (a short tail pass would run ahead of its
// partner, and the partner's weight reads would miss the L2).
__device__ __forceinline__ void pass_tokens(int n, int np, int p, int& tok0, int& nlive) {
    const int nt = (n + 15) >> 4;
    const int t0 = p * nt / np, t1 = (p + 1) * nt / np;
    tok0 = 16 * t0;
    nlive = (16 * t1 < n ? 16 * t1 : n) - tok0;
}

template <class FMT, int NPROJ>
__host__ __device__ constexpr int dense_nt() { return FMT::XSUM && NPROJ == 1 ? 8 : 4; }
template <class FMT, int NPROJ>
__host__ __device__ constexpr int dense_rt() { return FMT::XSUM ? 2 : 4 / NPROJ; }
template <class FMT, int NPROJ>
__host__ __device__ constexpr int dense_bn() { return 4 * 16 * dense_rt<FMT, NPROJ>(); }

template <class FMT, int NPROJ, int NT>
__global__ void __launch_bounds__(256, 2) k_dense(TileArgs a) {
    constexpr bool INT4 = FMT::XSUM;
    constexpr int SPG = INT4 ? 2 : 1;     // MFMA steps (32 inputs) per scale group
    constexpr int RT = dense_rt<FMT, NPROJ>();   // 16-row tiles per projection per wave
    constexpr int BM = 16 * NT;           // tokens per pass
    constexpr int BN = dense_bn<FMT, NPROJ>();   // rows per block (per projection)
    constexpr int SB = tile_slice_bytes<FMT>();
    // int4 (F16): activations travel as fp16 with power-of-two exponents (x16 per token; h16 per slot) and the
    // codes are dequantised to fp16 in registers; MXFP4 keeps the exact raw-code path on bf16 MFMA with its
    // per-group fold (its E8M0 scales do not fit fp16), h = hi + lo
    constexpr bool F16 = INT4;
    constexpr bool H16 = INT4;
    constexpr int HL = (NPROJ == 2 || H16) ? 1 : 2;   // activation planes: x, x16, h16, or h = hi + lo
    constexpr int NDMA = BM / 16;         // DMA instructions per wave per slice and plane (4 token rows each)
    __shared__ __attribute__((aligned(1024))) uint8_t sX0[HL * BM * 256];
    __shared__ __attribute__((aligned(1024))) uint8_t sX1[HL * BM * 256];
    __shared__ int sSlot[BM];

    // Work items (pass list x row blocks x K parts), ordered expert by expert, within an expert row block by row
    // block with the expert's passes adjacent, K part fastest. The launch hands workgroups to the 8 XCDs round
    // robin (workgroup b to XCD (b + c) mod 8, c fixed per launch), so XCD slot b & 7 takes the contiguous
    // eighth of the live items, in order: each XCD's L2 then holds the activations of few experts, and the
    // passes that share a weight tile run side by side on one XCD (their second reads hit its L2). The grid is
    // a multiple of 8 covering the largest possible item count.
    const int nrb = (a.N + BN - 1) / BN;
    const int nitems = a.meta[a.nidx] * nrb * a.ksplit;
    const int chunk = (nitems + 7) >> 3;
    const int rank = (int)(blockIdx.x >> 3);
    const int item = (int)(blockIdx.x & 7u) * chunk + rank;
    if (rank >= chunk || item >= nitems) return;
    const int ks = item % a.ksplit;               // K part (down only), the fastest index
    const int bid = item / a.ksplit;
    const int wq = bid / nrb;                      // some pass of the current expert
    const int e = a.items[3 * wq], np = a.items[3 * wq + 2];
    const int w0 = wq - a.items[3 * wq + 1];       // the expert's first pass
    const int local = bid - w0 * nrb;
    const int rb = local / np;
    const int n = a.counts[e], beg = a.offsets[e];
    int tok0, nlive;
    pass_tokens(n, np, local - rb * np, tok0, nlive);
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = a.K, N = a.N;
    const int nsl = (K + 127) >> 7;
    const int per = (nsl + a.ksplit - 1) / a.ksplit;
    const int sb0 = ks * per;                                // this block's slices: sb0 .. sb0 + scnt - 1
    const int scnt = nsl - sb0 < per ? nsl - sb0 : per;   // >= 1 (the host splits only when it is)
    const int lastp = (K >> 3) - 1;       // last 8-input piece of an activation row
    const int r0 = rb * BN + wave * 16 * RT;
    const bool wvalid = r0 < N;           // N % (16 RT) == 0: a wave's rows are all in range or all out
    const uint8_t* tb[NPROJ][RT];
#pragma unroll
    for (int p = 0; p < NPROJ; ++p)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            tb[p][rt] = (p ? a.W1 : a.W0) +
                        ((size_t)e * (N >> 4) + (wvalid ? (r0 >> 4) + rt : 0)) * (size_t)nsl * SB;
    const uint8_t* xb[HL];
    xb[0] = reinterpret_cast<const uint8_t*>(a.actv);
    if (HL == 2) xb[HL - 1] = reinterpret_cast<const uint8_t*>(a.actv2);
    // the DMA lanes: instruction i of this wave writes token rows 4 (wave + 4 i) + (lane >> 4), position lane & 15
    const int psw = (lane & 15) ^ ((4 * wave + (lane >> 4)) & 15);   // piece loaded by this lane
    const uint32_t ones = 0x3F803F80u;
    const bf16x8 ONES = as_bf16x8(ones, ones, ones, ones);

    {
        const int ntiles = (nlive + 15) >> 4;
        if (tid < BM) sSlot[tid] = a.sorted[beg + (tok0 + tid < n ? tok0 + tid : n - 1)];
        __syncthreads();
        uint32_t xrow[NDMA];
#pragma unroll
        for (int i = 0; i < NDMA; ++i)
            xrow[i] = (uint32_t)(sSlot[4 * (wave + 4 * i) + (lane >> 4)] / a.act_div) * (uint32_t)K * 2u;
        auto dma = [&](int s, uint8_t* buf) __attribute__((always_inline)) {
            int piece = 16 * s + psw;
            piece = piece < lastp ? piece : lastp;   // inputs past K meet zero codes and zero metadata
#pragma unroll
            for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                for (int i = 0; i < NDMA; ++i) {
                    // 32-bit offset from the uniform base (kept opaque so no 64-bit address is held per row)
                    uint32_t o = xrow[i];
                    asm volatile("" : "+v"(o));
                    __builtin_amdgcn_global_load_lds((const void*)(xb[hl] + (o + 16u * (uint32_t)piece)),
                                                     MOE_LDSP(buf + (hl * BM + 4 * (wave + 4 * i)) * 256), 16, 0, 0);
                }
        };
        uint4 rq[2][NPROJ][RT];
        uint2 rm[2][NPROJ][RT];
        // F16: entry h of lane j holds the exponent E of token 64 h + j of the pass: its activation row is x 2^-E
        // (x16, k_x16) or h 2^-E (h16, k_h16_fix)
        constexpr int NE = (BM + 63) / 64;   // lane j of entry h: token 64 h + j
        int eslot[NE];
#pragma unroll
        for (int h = 0; h < NE; ++h) {
            eslot[h] = 0;
            const int j = 64 * h + lane;
            if (F16 && j < BM) {
                if (NPROJ == 1)
                    eslot[h] = reinterpret_cast<const int32_t*>(reinterpret_cast<const uint8_t*>(a.actv2) + a.eslot_off)[sSlot[j]];
                else
                    eslot[h] = a.xexp[sSlot[j] / a.act_div];
            }
        }
        auto wissue = [&](int s, uint4 (&q)[NPROJ][RT], uint2 (&m)[NPROJ][RT]) __attribute__((always_inline)) {
#pragma unroll
            for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const uint8_t* sl = tb[p][rt] + (uint32_t)s * (uint32_t)SB;
                    q[p][rt] = *reinterpret_cast<const uint4*>(sl + 16 * lane);
                    if (INT4) m[p][rt] = *reinterpret_cast<const uint2*>(sl + 1024 + 8 * lr);
                    else m[p][rt].x = *reinterpret_cast<const uint32_t*>(sl + 1024 + 4 * lr);
                }
        };
        f32x4 acc[NPROJ][RT][NT];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[p][rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
        // F16 (int4): the B operands of projection p, row tile rt, scale group G, as fp16 w' = (s q + b) 2^-16 in
        // one rounding: each code pair (q_k, q_{k+4}) is masked into bits 4-7 of two fp16 halves with exponent 0,
        // which makes them the exact subnormals q 2^-20 (one shift and one mask), and one v_pk_fma_f16 takes
        // q 2^-20 (16 s) + b 2^-16. The records' row scaling keeps |s|, |b| below 2^11, so 16 s < 2^15 fits fp16 and
        // |w'| < 2^-1: a weight stays a normal fp16 number down to 2^-13 of that bound, and below it rounds to fp16's
        // subnormal step 2^-24 (2^-19 of the row's largest |s|, |b| in w' units). The epilogue adds 16 to the row
        // exponent. 11 VALU per code word. (Codes left in bits 0-3 as q 2^-24 save two shifts, 9 VALU, but bound
        // |w'| by 2^-5 and so put weights 2^9 below the row's largest into the subnormal range: one group per row at
        // 64x the others' scale and small x on it then reached 8e-3 of the output RMS in a numpy emulation, 4e-2 at
        // 256x, against 5e-7 and 1.4e-3 for this decode.)
        constexpr int DEC_EXP = 16;
        auto decode_f16 = [&](int G, int p, int rt, const uint4 (&q)[NPROJ][RT], const uint2 (&m)[NPROJ][RT],
                              f16x8 (&B)[NPROJ][RT][2]) __attribute__((always_inline)) {
            const uint32_t mw = G ? m[p][rt].y : m[p][rt].x;
            const _Float16 s16 = (_Float16)(bf16lo(mw) * 16.0f), b16 = (_Float16)(bf16hi(mw) * 0x1p-16f);
            const h2x s2 = {s16, s16}, b2 = {b16, b16};
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int j = 2 * G + u;
                const uint32_t w = j == 0 ? q[p][rt].x : (j == 1 ? q[p][rt].y : (j == 2 ? q[p][rt].z : q[p][rt].w));
                const uint32_t c4[4] = {(w << 4) & 0x00F000F0u, w & 0x00F000F0u, (w >> 4) & 0x00F000F0u,
                                        (w >> 8) & 0x00F000F0u};
                h2x v[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = __builtin_elementwise_fma(__builtin_bit_cast(h2x, c4[c]), s2, b2);
                B[p][rt][u] = f16x8{v[0][0], v[0][1], v[1][0], v[1][1], v[2][0], v[2][1], v[3][0], v[3][1]};
            }
        };
        // one slice as 2 NT steps f = G NT + t (scale group G, token tile t): group G's MFMAs (f16 x f16, fp32
        // accumulate, straight into acc) for token tile t; after each of group 0's steps, group 1's (projection,
        // row tile) pairs t * NPROJ * RT / NT ... are decoded, so that VALU work issues while MFMAs run. The A
        // operands of step f + 2 are read from LDS while step f's MFMAs run, across the group boundary (three
        // register sets; one step's MFMAs alone do not cover the LDS latency when a wave has only 2 row tiles), so
        // a slice waits for LDS reads once, before its first step.
        auto slice_f16 = [&](auto full, const uint8_t* xs, const uint4 (&q)[NPROJ][RT], const uint2 (&m)[NPROJ][RT])
                             __attribute__((always_inline)) {
            static_assert(NPROJ * RT % NT == 0 || NT % (NPROJ * RT) == 0, "decode pairs spread evenly over the token tiles");
            // pairs decoded after each token tile (PPT >= 1), or one pair after every TPP-th token tile
            constexpr int PPT = NPROJ * RT >= NT ? NPROJ * RT / NT : 1;
            constexpr int TPP = NPROJ * RT >= NT ? 1 : NT / (NPROJ * RT);
            constexpr int NS = 2 * NT;
            f16x8 B0[NPROJ][RT][2], B1[NPROJ][RT][2];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < NPROJ * RT; ++i) decode_f16(0, i / RT, i % RT, q, m, B0);
            __builtin_amdgcn_sched_barrier(0);
            auto live = [&](int f) __attribute__((always_inline)) { return decltype(full)::value || f % NT < ntiles; };
            auto load_a = [&](int f, f16x8 (&A)[2]) __attribute__((always_inline)) {
                const int G = f / NT, t = f % NT;
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int j = 2 * G + u;
                    const int wi = j < 2 ? 2 * lg + j : 8 + 2 * lg + (j - 2);
                    A[u] = __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(xs + (16 * t + lr) * 256 + 16 * (wi ^ lr)));
                }
            };
            f16x8 Ab[3][2];
            if (live(0)) load_a(0, Ab[0]);
            if (live(1)) load_a(1, Ab[1]);
#pragma unroll
            for (int f = 0; f < NS; ++f) {
                const int G = f / NT, t = f % NT;
                if (f + 2 < NS && live(f + 2)) load_a(f + 2, Ab[(f + 2) % 3]);
                __builtin_amdgcn_sched_barrier(0);
                if (live(f)) {   // wave-uniform
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                            for (int rt = 0; rt < RT; ++rt)
                                acc[p][rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                    Ab[f % 3][u], G ? B1[p][rt][u] : B0[p][rt][u], acc[p][rt][t], 0, 0, 0);
                }
                if (G == 0 && t % TPP == TPP - 1) {
#pragma unroll
                    for (int i = (t / TPP) * PPT; i < (t / TPP + 1) * PPT; ++i) decode_f16(1, i / RT, i % RT, q, m, B1);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        // one slice, scale group by scale group; lane (m, g) of MFMA step j supplies word wi(j, g) of its row
        // (the record order). FULL: every token tile of the pass is live (no branch inside the slice)
        auto compute = [&](auto full, const uint8_t* xs, const uint4 (&q)[NPROJ][RT], const uint2 (&m)[NPROJ][RT],
                           int) __attribute__((always_inline)) {
            if constexpr (F16) {
                slice_f16(full, xs, q, m);
                return;
            }
#pragma unroll
            for (int G = 0; G < 4 / SPG; ++G) {
                __builtin_amdgcn_sched_barrier(0);   // one group at a time: bounds the live operands
                bf16x8 B[NPROJ][RT][SPG];
                float ms[NPROJ][RT], mc[NPROJ][RT];
#pragma unroll
                for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
                        for (int u = 0; u < SPG; ++u) {
                            const int j = SPG * G + u;
                            const uint32_t w = j == 0 ? q[p][rt].x : (j == 1 ? q[p][rt].y : (j == 2 ? q[p][rt].z : q[p][rt].w));
                            uint32_t c4[4];
                            FMT::decode_word(w, c4);
                            B[p][rt][u] = as_bf16x8(c4[0], c4[1], c4[2], c4[3]);
                        }
                        if (INT4) {
                            const uint32_t mw = G ? m[p][rt].y : m[p][rt].x;
                            ms[p][rt] = bf16lo(mw);
                            mc[p][rt] = __builtin_fmaf(-128.f, ms[p][rt], bf16hi(mw));
                        } else {
                            ms[p][rt] = __uint_as_float(((m[p][rt].x >> (8 * G)) & 0xFFu) << 23);
                            mc[p][rt] = 0.f;
                        }
                    }
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    if (decltype(full)::value || t < ntiles) {   // wave-uniform
                        bf16x8 A[HL][SPG];
#pragma unroll
                        for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                            for (int u = 0; u < SPG; ++u) {
                                const int j = SPG * G + u;
                                const int wi = INT4 ? (j < 2 ? 2 * lg + j : 8 + 2 * lg + (j - 2)) : 4 * j + lg;
                                const uint4 av = *reinterpret_cast<const uint4*>(
                                    xs + (hl * BM + 16 * t + lr) * 256 + 16 * (wi ^ lr));
                                A[hl][u] = as_bf16x8(av.x, av.y, av.z, av.w);
                            }
                        f32x4 xsum = f32x4{0.f, 0.f, 0.f, 0.f};
                        if (INT4) {
#pragma unroll
                            for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                                for (int u = 0; u < SPG; ++u)
                                    xsum = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[hl][u], ONES, xsum, 0, 0, 0);
                        }
#pragma unroll
                        for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                            for (int rt = 0; rt < RT; ++rt) {
                                f32x4 P = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                                for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                                    for (int u = 0; u < SPG; ++u)
                                        P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[hl][u], B[p][rt][u], P, 0, 0, 0);
#pragma unroll
                                for (int v = 0; v < 4; ++v) {
                                    if (INT4)
                                        acc[p][rt][t][v] = __builtin_fmaf(ms[p][rt], P[v],
                                                                          __builtin_fmaf(mc[p][rt], xsum[v], acc[p][rt][t][v]));
                                    else
                                        acc[p][rt][t][v] = __builtin_fmaf(ms[p][rt], P[v], acc[p][rt][t][v]);
                                }
                            }
                    }
                }
            }
        };
        // int4: row exponents of the lane's rows (the records hold s 2^-E, b 2^-E; the epilogue scales by 2^E)
        int rex[NPROJ][RT];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
                rex[p][rt] = INT4 && wvalid ? tile_row_exps(p ? a.W1 : a.W0, a.E, N, K)[(size_t)e * N + r0 + 16 * rt + lr] + DEC_EXP : 0;
        // slice s sits in buffer / ring slot s & 1; slice s + 1 is fetched during slice s (the last slice fetches
        // itself again into the idle slot: no branch around the loads)
        auto run = [&](auto full) __attribute__((always_inline)) {
            dma(sb0, sX0);
            wissue(sb0, rq[0], rm[0]);
            MOE_VMWAIT0();
            MOE_BARRIER();
            int j = 0;
            for (; j + 2 <= scnt; j += 2) {
                wissue(sb0 + j + 1, rq[1], rm[1]);
                dma(sb0 + j + 1, sX1);
                compute(full, sX0, rq[0], rm[0], j);
                MOE_VMWAIT0();
                MOE_BARRIER();
                const int jn = sb0 + (j + 2 < scnt ? j + 2 : j + 1);
                wissue(jn, rq[0], rm[0]);
                dma(jn, sX0);
                compute(full, sX1, rq[1], rm[1], j + 1);
                MOE_VMWAIT0();
                MOE_BARRIER();
            }
            if (j < scnt) compute(full, sX0, rq[0], rm[0], j);   // odd count: the last slice is in slot 0
        };
        if (ntiles == NT) run(std::true_type{});
        else run(std::false_type{});

        // ---- epilogue: lane holds row r0 + 16 rt + lr of tokens tok0 + 16 t + 4 lg + v
        if constexpr (H16 && NPROJ == 2) {
            // h of the wave's 32 rows as fp16 h16 = h 2^-e, e per token: 0 while |h| < 2^15 on those rows, else
            // the power of two that brings their largest |h| below 2^15 (so fp16 never overflows); e goes to the
            // exponent bytes [slot, F / 32] (one 32-row chunk per wave)
            static_assert(RT == 2, "one 32-row chunk per wave");
            float hv[NT][4][RT];
            int xe[NT][4];   // x16 = x 2^-E per token: the sums are scaled back before the GLU
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int v = 0; v < 4; ++v) xe[t][v] = __shfl(eslot[(16 * t) >> 6], (16 * t + 4 * lg + v) & 63, 64);
            int8_t* hexp_out = reinterpret_cast<int8_t*>(a.hout2);
            const int nch = N >> 5;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float am = 0.f;
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const int r = r0 + 16 * rt + lr;
                        float g = __builtin_ldexpf(acc[0][rt][t][v], xe[t][v] + rex[0][rt]);
                        float up = __builtin_ldexpf(acc[1][rt][t][v], xe[t][v] + rex[1][rt]);
                        if (wvalid && a.b0) g += a.b0[(size_t)e * N + r];
                        if (wvalid && a.b1) up += a.b1[(size_t)e * N + r];
                        hv[t][v][rt] = wvalid ? glu_act(a.act, g, up) : 0.f;
                        am = fmaxf(am, fabsf(hv[t][v][rt]));
                    }
#pragma unroll
                    for (int o = 1; o < 16; o <<= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
                    const int ex = h16_exponent(am);
                    const int jt = 16 * t + 4 * lg + v;
                    if (jt >= nlive || !wvalid) continue;
                    const int slot = sSlot[jt];
                    if (lr == 0) hexp_out[(size_t)slot * nch + (r0 >> 5)] = (int8_t)ex;
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const _Float16 h16 = (_Float16)__builtin_ldexpf(hv[t][v][rt], -ex);
                        a.hout[(size_t)slot * N + r0 + 16 * rt + lr] = __builtin_bit_cast(uint16_t, h16);
                    }
                }
        } else {
            int es[NT][4];   // H16 down: the exponent of each of the lane's tokens (all lanes take part in the shuffle)
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int v = 0; v < 4; ++v) es[t][v] = H16 ? __shfl(eslot[(16 * t) >> 6], (16 * t + 4 * lg + v) & 63, 64) : 0;
            if (wvalid)
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int jt = 16 * t + 4 * lg + v;
                    if (jt >= nlive) continue;
                    const int slot = sSlot[jt];
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const int r = r0 + 16 * rt + lr;
                        if (NPROJ == 2) {
                            float g = acc[0][rt][t][v], up = acc[NPROJ - 1][rt][t][v];
                            if (a.b0) g += a.b0[(size_t)e * N + r];
                            if (a.b1) up += a.b1[(size_t)e * N + r];
                            const float hv = glu_act(a.act, g, up);
                            const uint16_t hi = f32_to_bf16(hv);
                            a.hout[(size_t)slot * N + r] = hi;
                            a.hout2[(size_t)slot * N + r] = f32_to_bf16(hv - bf16_to_f32(hi));
                        } else if (H16) {
                            a.yp[ks * a.plane + (size_t)slot * N + r] = __builtin_ldexpf(acc[0][rt][t][v], es[t][v] + rex[0][rt]);
                        } else {
                            a.yp[ks * a.plane + (size_t)slot * N + r] = acc[0][rt][t][v];
                        }
                    }
                }
        }
    }
}

// ============================================================================ MXFP4 dense tiles on the block-scaled MFMA
// gfx950's v_mfma_scale_f32_16x16x128_f8f6f4 multiplies fp8 (E4M3) A by fp4 (E2M1) B over 128 inputs, each
// operand's 32-input blocks (lane group g of the B operand: block g) times its own E8M0 power of two. The weights
// go in undecoded and unfolded from the tile-major records: lane (r, g) loads its 16 bytes of the slice record
// (row r's code words g, 4 + g, 8 + g, 12 + g), a 4 x 4 transpose across the lane groups (two v_permlane32_swap,
// two v_permlane16_swap) leaves it words 4 g .. 4 g + 3 = block g, and byte g of row r's E8M0 word is its scale.
// The words keep the records' nibble order (e0 e2 e4 e6 e1 e3 e5 e7); the activation terms are written in that
// order instead. The activations enter as a sum of fp8 terms, each with an E8M0 byte per (token, 32 inputs): term t of a block
// has scale 2^e, e = floor(log2 max |r|) - 7 (|r / 2^e| < 256, inside E4M3's range), q = E4M3(r / 2^e) and
// r -= q 2^e (exact). Two terms hold a bf16 x exactly for every input within ~2^12 of its 32-block's largest
// magnitude (4 significant bits each); smaller inputs fall into E4M3's subnormal range in both terms and keep an
// absolute error below the second term's step, 2^-20 of the block's largest. Three terms hold h = hi + lo to ~12
// bits. Measured on this part, the instruction's own accumulation keeps ~2e-5 of the outputs' RMS (two to four terms
// give the same result), against the 1e-2 RMS gate.

// x rows (bf16) -> their fp8 term records (mx_terms_block, moe_mxterms.h): one thread per 32-input block
template <int NTERM>
__global__ void __launch_bounds__(256) k_mx_terms(const uint16_t* __restrict__ src, int rows, int K,
                                                 uint8_t* __restrict__ out) {
    mx_terms_block<NTERM>(src, rows, K, out, (long)blockIdx.x * 256 + threadIdx.x);
}

// k_mxd: blocks of 4 waves own BN = 64 RT rows of one expert (per projection) and one pass of up to 64 of its slots
// (the dense tiles' work list, XCD-chunked the same way); each wave covers the pass's 4 token tiles for its RT row
// tiles. Per 128-input slice: the pass's activation records (64 x REC bytes) come into LDS by
// global_load_lds_dwordx4 (records of 17 or 25 16-byte pieces, an odd count, so the 16 lanes of a token tile read
// 16 distinct bank groups), double-buffered; each wave loads its row tiles' slice records (1 KB of codes + the
// E8M0 words) one slice ahead; NTERM x 4 x NPROJ x RT MFMAs per slice.
#ifndef MOE_MXD_RT_DN
#define MOE_MXD_RT_DN 4
#endif
#ifndef MOE_MXD_MINB_GU
#define MOE_MXD_MINB_GU 2
#endif
#ifndef MOE_MXD_MINB_DN
#define MOE_MXD_MINB_DN 2
#endif
template <int NPROJ>
__host__ __device__ constexpr int mxd_rt() { return NPROJ == 2 ? 2 : MOE_MXD_RT_DN; }

template <int NPROJ, int NTERM>
__global__ void __launch_bounds__(256, NPROJ == 2 ? MOE_MXD_MINB_GU : MOE_MXD_MINB_DN) k_mxd(TileArgs a) {
    constexpr int NT = 4, BM = 64;
    constexpr int RT = mxd_rt<NPROJ>();
    constexpr int BN = 64 * RT;
    constexpr int REC = mx_rec<NTERM>();
    constexpr int NPC = REC / 16;                     // 16-byte pieces per record
    constexpr int NCH = (BM * NPC + 63) / 64;         // 64-piece DMA chunks per slice
    constexpr int NDMA = (NCH + 3) / 4;               // DMA instructions per wave per slice (the last partial)
    typedef int v8i __attribute__((ext_vector_type(8)));
    __shared__ __attribute__((aligned(1024))) uint8_t sX0[NCH * 1024];
    __shared__ __attribute__((aligned(1024))) uint8_t sX1[NCH * 1024];
    __shared__ int sSlot[BM];

    const int nrb = (a.N + BN - 1) / BN;
    const int nitems = a.meta[a.nidx] * nrb;
    const int chunk = (nitems + 7) >> 3;
    const int rank = (int)(blockIdx.x >> 3);
    const int item = (int)(blockIdx.x & 7u) * chunk + rank;
    if (rank >= chunk || item >= nitems) return;
    const int wq = item / nrb;
    const int e = a.items[3 * wq], np = a.items[3 * wq + 2];
    const int w0 = wq - a.items[3 * wq + 1];
    const int local = item - w0 * nrb;
    const int rb = local / np;
    const int n = a.counts[e], beg = a.offsets[e];
    int tok0, nlive;
    pass_tokens(n, np, local - rb * np, tok0, nlive);
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = a.K, N = a.N;
    const int nsl = (K + 127) >> 7;
    const int r0 = rb * BN + wave * 16 * RT;
    const bool wvalid = r0 < N;                        // N % (16 RT) == 0
    constexpr int SB = TILE_SLICE_MXFP4;
    const uint8_t* tb[NPROJ][RT];
#pragma unroll
    for (int p = 0; p < NPROJ; ++p)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            tb[p][rt] = (p ? a.W1 : a.W0) + ((size_t)e * (N >> 4) + (wvalid ? (r0 >> 4) + rt : 0)) * (size_t)nsl * SB;
    const uint8_t* recs = reinterpret_cast<const uint8_t*>(a.actv);

    const int ntiles = (nlive + 15) >> 4;
    if (tid < BM) sSlot[tid] = a.sorted[beg + (tok0 + tid < n ? tok0 + tid : n - 1)];
    __syncthreads();
    // DMA lanes: chunk c = 4 i + wave of the slice's BM * NPC pieces; piece q = 64 c + lane -> record of token
    // q / NPC, piece q % NPC (pieces past the last record re-read the last piece into the buffer's tail)
    uint32_t xoff[NDMA];
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
        int q = 64 * (4 * i + wave) + lane;
        q = q < BM * NPC ? q : BM * NPC - 1;
        const int tok = q / NPC, pc = q - tok * NPC;
        xoff[i] = ((uint32_t)(sSlot[tok] / a.act_div) * (uint32_t)nsl) * (uint32_t)REC + 16u * (uint32_t)pc;
    }
    auto dma = [&](int s, uint8_t* buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NDMA; ++i)
            if (4 * i + wave < NCH) {   // wave-uniform
                uint32_t o = xoff[i] + (uint32_t)s * (uint32_t)REC;
                asm volatile("" : "+v"(o));
                __builtin_amdgcn_global_load_lds((const void*)(recs + o), MOE_LDSP(buf + (4 * i + wave) * 1024), 16, 0, 0);
            }
    };
    // weights of slice s: the lane's 16 bytes of each row tile's record and its row's E8M0 word (words and groups
    // past K are zero in the records: zero codes, scale 2^-127)
    auto wissue = [&](int s, uint4 (&q)[NPROJ][RT], uint32_t (&m)[NPROJ][RT]) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < NPROJ; ++p)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const uint8_t* sl = tb[p][rt] + (uint32_t)s * (uint32_t)SB;
                q[p][rt] = *reinterpret_cast<const uint4*>(sl + 16 * lane);
                m[p][rt] = *reinterpret_cast<const uint32_t*>(sl + 1024 + 4 * lr);
            }
    };
    // lane group g: words (g, 4 + g, 8 + g, 12 + g) -> (4 g, 4 g + 1, 4 g + 2, 4 g + 3)
    auto transpose = [](const uint4& v) __attribute__((always_inline)) {
        const auto s0 = __builtin_amdgcn_permlane32_swap(v.x, v.z, false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(v.y, v.w, false, false);
        const auto t0 = __builtin_amdgcn_permlane16_swap(s0[0], s1[0], false, false);
        const auto t1 = __builtin_amdgcn_permlane16_swap(s0[1], s1[1], false, false);
        return uint4{t0[0], t0[1], t1[0], t1[1]};
    };
    f32x4 acc[NPROJ][RT][NT];
#pragma unroll
    for (int p = 0; p < NPROJ; ++p)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[p][rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // token tile by token tile (live tiles only): the tile's NTERM A operands from LDS, then its MFMAs
    auto compute = [&](const uint8_t* xs, const uint4 (&q)[NPROJ][RT], const uint32_t (&m)[NPROJ][RT])
                       __attribute__((always_inline)) {
        v8i B[NPROJ][RT];
        int sb[NPROJ][RT];
#pragma unroll
        for (int p = 0; p < NPROJ; ++p)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const uint4 w = transpose(q[p][rt]);
                B[p][rt] = v8i{(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
                sb[p][rt] = (int)(m[p][rt] >> (8 * lg));
            }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t < ntiles) {   // wave-uniform
                const uint8_t* ra = xs + (16 * t + lr) * REC;
                v8i A[NTERM];
                int sa[NTERM];
#pragma unroll
                for (int tm = 0; tm < NTERM; ++tm) {
                    const uint4 a0 = *reinterpret_cast<const uint4*>(ra + 128 * tm + 32 * lg);
                    const uint4 a1 = *reinterpret_cast<const uint4*>(ra + 128 * tm + 32 * lg + 16);
                    A[tm] = v8i{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
                    sa[tm] = ra[128 * NTERM + 4 * tm + lg];
                }
#pragma unroll
                for (int tm = 0; tm < NTERM; ++tm)
#pragma unroll
                    for (int p = 0; p < NPROJ; ++p)
#pragma unroll
                        for (int rt = 0; rt < RT; ++rt)
                            acc[p][rt][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                                A[tm], B[p][rt], acc[p][rt][t], 0, 4, 0, sa[tm], 0, sb[p][rt]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    uint4 rq[2][NPROJ][RT];
    uint32_t rm[2][NPROJ][RT];
    // slice s in buffer / register set s & 1; slice s + 1 is fetched while slice s is multiplied (the last slice
    // fetches itself again into the idle set: no branch around the loads)
    dma(0, sX0);
    wissue(0, rq[0], rm[0]);
    MOE_VMWAIT0();
    MOE_BARRIER();
    int j = 0;
    for (; j + 2 <= nsl; j += 2) {
        wissue(j + 1, rq[1], rm[1]);
        dma(j + 1, sX1);
        compute(sX0, rq[0], rm[0]);
        MOE_VMWAIT0();
        MOE_BARRIER();
        const int jn = j + 2 < nsl ? j + 2 : j + 1;
        wissue(jn, rq[0], rm[0]);
        dma(jn, sX0);
        compute(sX1, rq[1], rm[1]);
        MOE_VMWAIT0();
        MOE_BARRIER();
    }
    if (j < nsl) compute(sX0, rq[0], rm[0]);   // odd count: the last slice is in buffer 0

    // ---- epilogue: lane holds row r0 + 16 rt + lr of tokens tok0 + 16 t + 4 lg + v
    if (!wvalid) return;
    if constexpr (NPROJ == 2) {   // h as the down's 3-term records: this wave's 32 rows = one block
        static_assert(RT == 2, "one 32-row block of h per wave");
        const int nslN = (N + 127) >> 7, bk = (r0 & 127) >> 5;
        const bool pad = (N & 127) == 64 && (r0 >> 7) == nslN - 1 && bk == 1;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int jt = 16 * t + 4 * lg + v;
                const int slot = sSlot[jt];
                float hv[RT];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const int r = r0 + 16 * rt + lr;
                    float g = acc[0][rt][t][v], up = acc[1][rt][t][v];
                    if (a.b0) g += a.b0[(size_t)e * N + r];
                    if (a.b1) up += a.b1[(size_t)e * N + r];
                    hv[rt] = glu_act(a.act, g, up);
                }
                mx_h_block<3>(hv[0], hv[1], jt < nlive, a.hterm + ((size_t)slot * nslN + (r0 >> 7)) * mx_rec<3>(), bk,
                              lr, pad);
            }
        return;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int jt = 16 * t + 4 * lg + v;
            if (jt >= nlive) continue;
            const int slot = sSlot[jt];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) a.yp[(size_t)slot * N + r0 + 16 * rt + lr] = acc[0][rt][t][v];
        }
}

template <int NPROJ, int NTERM>
int launch_mxd(const TileArgs& t, int nslots, hipStream_t st) {
    constexpr int BN = 64 * mxd_rt<NPROJ>();
    if (t.N % (16 * mxd_rt<NPROJ>())) return MOE_ERR_ARG;
    const long nblk = ((long)((t.N + BN - 1) / BN) * max_passes(nslots, t.E, 64) + 7) / 8 * 8;
    if (nblk > 0x7FFFFFF8L) return MOE_ERR_ARG;
    k_mxd<NPROJ, NTERM><<<dim3((unsigned)nblk), 256, 0, st>>>(t);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

template <int NTERM>
int launch_mx_terms(const uint16_t* src, int rows, int K, uint8_t* out, hipStream_t st) {
    const long n = (long)rows * 4 * ((K + 127) >> 7);
    if (n <= 0 || (n + 255) / 256 > 0x7FFFFFFFL) return MOE_ERR_ARG;
    k_mx_terms<NTERM><<<dim3((unsigned)((n + 255) / 256)), 256, 0, st>>>(src, rows, K, out);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

// Dense int4, before gate/up: x [T, d] (bf16 or fp16) -> x16 = x 2^-E fp16, one block per token, E = h16_exponent of
// the row's largest |x| (bf16 and fp16 to fp16 are then exact except far below the row's largest, where fp16's
// subnormal range rounds); E per token for the gate/up epilogue.
// 8 activations of x (bf16, fp16 or fp32) starting at element 8c of row `row`, as fp32
template <int XDT>
__device__ __forceinline__ void load_x8(const void* row, int c, float v[8]) {
    if (XDT == MOE_DTYPE_F32) {
        const float4 a = reinterpret_cast<const float4*>(row)[2 * c], b = reinterpret_cast<const float4*>(row)[2 * c + 1];
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
        return;
    }
    const uint4 r = reinterpret_cast<const uint4*>(row)[c];
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (XDT == MOE_DTYPE_F16) {
            v[2 * q] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[q] & 0xFFFFu));
            v[2 * q + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[q] >> 16));
        } else {
            v[2 * q] = bf16lo(w[q]);
            v[2 * q + 1] = bf16hi(w[q]);
        }
    }
}

template <int XDT>
__global__ void __launch_bounds__(256) k_x16(const void* __restrict__ x, uint16_t* __restrict__ x16,
                                             int32_t* __restrict__ xexp, int d) {
    __shared__ float sM[4];
    const int t = blockIdx.x, tid = threadIdx.x;
    const void* row = reinterpret_cast<const uint8_t*>(x) + (size_t)t * d * (XDT == MOE_DTYPE_F32 ? 4 : 2);
    uint4* out = reinterpret_cast<uint4*>(x16 + (size_t)t * d);
    const int nch = d >> 3;   // 8-element chunks; d <= 2048 * 8 for one round of 8 per thread
    constexpr int CPT = 8;
    float am = 0.f;
    for (int c0 = 0; c0 < nch; c0 += 256 * CPT) {
        float v[CPT][8];
#pragma unroll
        for (int i = 0; i < CPT; ++i)
            if (c0 + i * 256 + tid < nch) load_x8<XDT>(row, c0 + i * 256 + tid, v[i]);
#pragma unroll
        for (int i = 0; i < CPT; ++i)
            if (c0 + i * 256 + tid < nch) {
#pragma unroll
                for (int q = 0; q < 8; ++q) am = fmaxf(am, fabsf(v[i][q]));
            }
    }
    for (int o = 32; o; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
    if ((tid & 63) == 0) sM[tid >> 6] = am;
    __syncthreads();
    const float amax = fmaxf(fmaxf(sM[0], sM[1]), fmaxf(sM[2], sM[3]));
    const int E = h16_exponent(amax);
    if (tid == 0) xexp[t] = E;
    for (int c = tid; c < nch; c += 256) {   // the row again (cache hits)
        float v[8];
        load_x8<XDT>(row, c, v);
        uint32_t o4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const _Float16 lo = (_Float16)__builtin_ldexpf(v[2 * q], -E), hi = (_Float16)__builtin_ldexpf(v[2 * q + 1], -E);
            o4[q] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
        }
        out[c] = make_uint4(o4[0], o4[1], o4[2], o4[3]);
    }
}

// int4 grouped path, between gate/up and a dense down: one block per slot. The gate/up wrote h16 = h 2^-e with e
// per (slot, 32-row chunk) (h16_exponent); this brings the slot's row to one exponent E = max e (chunks with a
// smaller e are scaled by 2^(e - E): exact unless a value falls into fp16's subnormal range, where it is rounded:
// it is then below 2^-24 of the slot's largest) and writes E for the down projection's epilogue. All-zero chunks
// (H16_ZERO_EXP) take no part. A slot whose chunks share one exponent (the usual case: all 0) costs two exponent
// loads per thread.
__global__ void __launch_bounds__(256) k_h16_fix(const int8_t* __restrict__ hexp, uint16_t* __restrict__ h16,
                                                 int32_t* __restrict__ eslot, int F) {
    __shared__ int sE[512];   // F <= 16384: at most 512 chunks of 32
    __shared__ int sMax[4], sMin[4];
    const int slot = blockIdx.x, tid = threadIdx.x, nch = F >> 5;
    const int8_t* er = hexp + (size_t)slot * nch;
    const int e0 = tid < nch ? er[tid] : H16_ZERO_EXP, e1 = tid + 256 < nch ? er[tid + 256] : H16_ZERO_EXP;
    sE[tid] = e0;
    sE[tid + 256] = e1;
    int m = e0 > e1 ? e0 : e1;
    const int n0 = e0 == H16_ZERO_EXP ? 127 : e0, n1 = e1 == H16_ZERO_EXP ? 127 : e1;
    int mn = n0 < n1 ? n0 : n1;
    for (int o = 32; o; o >>= 1) {
        const int other = __shfl_xor(m, o, 64), omn = __shfl_xor(mn, o, 64);
        m = other > m ? other : m;
        mn = omn < mn ? omn : mn;
    }
    if ((tid & 63) == 0) {
        sMax[tid >> 6] = m;
        sMin[tid >> 6] = mn;
    }
    __syncthreads();
    int E = sMax[0];
    mn = sMin[0];
    for (int w = 1; w < 4; ++w) {
        E = sMax[w] > E ? sMax[w] : E;
        mn = sMin[w] < mn ? sMin[w] : mn;
    }
    if (tid == 0) eslot[slot] = E == H16_ZERO_EXP ? 0 : E;
    if (mn >= E) return;   // block-uniform: every chunk with a non-zero value is at E already (or none has one)
    // 16-byte pieces (8 values; 4 per chunk) of the row: every load first, then the rewrites
    constexpr int CPT = 8;   // pieces per thread per round (F <= 16384: 2048 pieces, one round)
    uint4* row = reinterpret_cast<uint4*>(h16 + (size_t)slot * F);
    const int np = F >> 3;
    for (int c0 = 0; c0 < np; c0 += 256 * CPT) {
        uint4 v[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = c0 + i * 256 + tid;
            if (c < np) v[i] = row[c];
        }
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = c0 + i * 256 + tid;
            if (c >= np) continue;
            const int ec = sE[c >> 2];
            if (ec == E || ec == H16_ZERO_EXP) continue;
            const int d = ec - E;
            uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t out = 0;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float f = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[q] >> (16 * h)));
                    out |= (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)__builtin_ldexpf(f, d)) << (16 * h);
                }
                w[q] = out;
            }
            row[c] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

// nibbles (e0 .. e7) of a word -> (e0, e2, e4, e6, e1, e3, e5, e7): the decode pairs nibbles i and i + 4, which
// then hold the adjacent elements (2i, 2i + 1)
__device__ __forceinline__ uint32_t interleave_nibbles(uint32_t w) {
    auto squeeze = [](uint32_t b) {   // low nibbles of the 4 bytes -> 16 bits
        return (b & 0xFu) | ((b >> 4) & 0xF0u) | ((b >> 8) & 0xF00u) | ((b >> 12) & 0xF000u);
    };
    return squeeze(w & 0x0F0F0F0Fu) | (squeeze((w >> 4) & 0x0F0F0F0Fu) << 16);
}

// int4 tile copies, before k_pack_tiles: the row exponent (int4_row_exponent) of each of the E * N rows, from the
// row's largest |scale| or |bias| over all its groups, into the exponent bytes after the records. One lane per row.
__global__ void __launch_bounds__(256) k_row_exp(const uint8_t* __restrict__ rows, int8_t* __restrict__ rexp,
                                                 int nrows, int K) {
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= nrows) return;
    const uint32_t* m = reinterpret_cast<const uint32_t*>(rows + (size_t)r * rbytes(MOE_FMT_INT4_G64, K) + (K >> 1));
    uint32_t amax = 0;   // bf16 magnitude bits: ordered as the magnitudes (NaN above inf)
    for (int g = 0; g < (K >> 6); ++g) {
        const uint32_t w = m[g], lo = w & 0x7FFFu, hi = (w >> 16) & 0x7FFFu;
        amax = lo > amax ? lo : amax;
        amax = hi > amax ? hi : amax;
    }
    rexp[r] = (int8_t)int4_row_exponent(amax);
}

// bf16 pair word (low, high) -> both halves times 2^-e, rounded to bf16 (exact for normal results)
__device__ __forceinline__ uint32_t scale_bf16_pair(uint32_t w, int e) {
    return (uint32_t)f32_to_bf16(__builtin_ldexpf(bf16lo(w), -e)) |
           ((uint32_t)f32_to_bf16(__builtin_ldexpf(bf16hi(w), -e)) << 16);
}

// rows [E, N, rbytes] -> tiles [E, N/16, ceil(K/128), slice record]; grid (slices, N/16, E), 64 lanes.
// int4: the metadata words go in as (s 2^-E, b 2^-E) with E the row's exponent (k_row_exp, run first)
template <class FMT>
__global__ void __launch_bounds__(64) k_pack_tiles(const uint8_t* __restrict__ rows, uint8_t* __restrict__ tiles,
                                                   int N, int K) {
    constexpr int SB = tile_slice_bytes<FMT>();
    const int s = blockIdx.x, tile = blockIdx.y, e = blockIdx.z;
    const int lane = threadIdx.x, r = lane & 15, g = lane >> 4;
    const int nsl = gridDim.x;
    const size_t rb = rbytes(FMT::FMT, K);
    const uint8_t* row = rows + ((size_t)e * N + 16 * tile + r) * rb;
    const uint32_t* words = reinterpret_cast<const uint32_t*>(row);
    uint8_t* rec = tiles + (((size_t)e * (N >> 4) + tile) * nsl + s) * SB;
    const int nw = K >> 3;   // code words of a row
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int wi = FMT::XSUM ? 16 * s + 8 * (j >> 1) + 2 * g + (j & 1) : 16 * s + 4 * j + g;
        w[j] = interleave_nibbles(wi < nw ? words[wi] : 0u);
    }
    *reinterpret_cast<uint4*>(rec + 16 * lane) = make_uint4(w[0], w[1], w[2], w[3]);
    if (g == 0) {
        if (FMT::XSUM) {   // group words 2s, 2s + 1, scaled by the row's exponent
            const int ng = K >> 6;
            const uint32_t* mw = reinterpret_cast<const uint32_t*>(row + (K >> 1));
            const int er = tile_row_exps(tiles, gridDim.z, N, K)[(size_t)e * N + 16 * tile + r];
            const uint32_t m0 = 2 * s < ng ? scale_bf16_pair(mw[2 * s], er) : 0u;
            const uint32_t m1 = 2 * s + 1 < ng ? scale_bf16_pair(mw[2 * s + 1], er) : 0u;
            *reinterpret_cast<uint2*>(rec + 1024 + 8 * r) = make_uint2(m0, m1);
        } else {           // E8M0 bytes of groups 4s .. 4s + 3
            const int ng = K >> 5;
            const uint8_t* mb = row + (K >> 1);
            uint32_t m = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (4 * s + j < ng) m |= (uint32_t)mb[4 * s + j] << (8 * j);
            *reinterpret_cast<uint32_t*>(rec + 1024 + 4 * r) = m;
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
int launch_tile(const TileArgs& t, int nt, int max_active, int T, hipStream_t st, int hx = 1) {
    // token passes spread over blockIdx.z: an expert has at most T slots when a token's k ids are distinct
    if (NPROJ == 2 && hx > 1) nt = 1;   // fp16 / fp32 x planes: one 16-token tile per pass (LDS)
    const int zp = (T + 16 * nt - 1) / (16 * nt);
    dim3 grid(t.N / TL_ROWS, max_active, zp < 1 ? 1 : (zp > 16 ? 16 : zp));
    if constexpr (NPROJ == 2) {
        if (hx > 1) {
            if (hx == 3) k_tile<FMT, 2, 1, 3><<<grid, 256, 0, st>>>(t);
            else k_tile<FMT, 2, 1, 2><<<grid, 256, 0, st>>>(t);
            return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
        }
    }
    switch (nt) {
        case 1: k_tile<FMT, NPROJ, 1><<<grid, 256, 0, st>>>(t); break;
        case 2: k_tile<FMT, NPROJ, 2><<<grid, 256, 0, st>>>(t); break;
        case 4: k_tile<FMT, NPROJ, 4><<<grid, 256, 0, st>>>(t); break;
        default: k_tile<FMT, NPROJ, 8><<<grid, 256, 0, st>>>(t); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

// Wave-tile shape (measured on MI355X at the Qwen3 T = 16..64 shapes): more rows per wave share each activation
// load across more weight bursts, more slices in flight hide more latency; both cost registers (occupancy).
#ifndef MOE_WAVE_D_GU
#define MOE_WAVE_D_GU 2    // slices (128 inputs) in flight per wave, gate/up
#endif
#ifndef MOE_WAVE_D_DN
#define MOE_WAVE_D_DN 2    // slices in flight per wave, down (its activations are two planes)
#endif
#ifndef MOE_WAVE_RT_GU
#define MOE_WAVE_RT_GU 2   // 16-row tiles per wave, gate/up (F % 32 == 0: F % 64 == 0 is required)
#endif
#ifndef MOE_WAVE_RT_DN_WIDE
#define MOE_WAVE_RT_DN_WIDE 8   // 16-row tiles per wave, down, when d % 128 == 0 (fewer activation loads per row)
#endif
#ifndef MOE_WAVE_RT_DN_MID
#define MOE_WAVE_RT_DN_MID 6    // next choice when d % 96 == 0 (gpt-oss, d = 2880); 0 = none
#endif
#ifndef MOE_WAVE_WIDE_MIN_WAVES
#define MOE_WAVE_WIDE_MIN_WAVES 1024   // the wide down only when its grid still has this many waves (4 per CU):
#endif                                 // a few shared experts' down (DSv2, 272 waves) ran 8% slower with it
#ifndef MOE_WAVE_RT_DN
#define MOE_WAVE_RT_DN 4   // 16-row tiles per wave, down (d % 64 == 0)
#endif
#ifndef MOE_WAVE_DN_SHALLOW
#define MOE_WAVE_DN_SHALLOW 1024   // live down waves from which a wave keeps one slice in flight (TileArgs::shallow_min)
#endif
template <class FMT, int NPROJ, int RT, int D, bool H16O = false>
int launch_wave_tile(const TileArgs& targs, int nt, int nslots, hipStream_t st, int hx = 1, int mxt = 0) {
    if (targs.N % (16 * RT)) return MOE_ERR_ARG;
    if (NPROJ == 1 && !mxt && targs.gidx) return MOE_ERR_ARG;   // these downs read a pass list (no in-kernel grouping)
    // in-kernel grouping, expert-major: E first passes and at most ceil(n / P) further ones (an expert with c
    // slots has ceil(c / P) - 1 <= (c - 1) / P of them)
    dim3 grid(targs.N / (16 * RT), targs.gidx && targs.gfirst ? targs.E + (nslots + 16 * nt - 1) / (16 * nt)
                                                           : max_passes(nslots, targs.E, 16 * nt));
    if (grid.y > 65535) return MOE_ERR_ARG;
    TileArgs t = targs;
    t.emit_y = (int)grid.y - 1;
    if constexpr (!FMT::XSUM && !H16O) {   // MXFP4 on the block-scaled MFMA: x 2 terms, h 3
        if (mxt) {
            constexpr int MT = NPROJ == 2 ? 2 : 3;
            if (hx != 1 || mxt != MT) return MOE_ERR_ARG;
            if (nt == 1) k_wave_tile<FMT, NPROJ, 1, RT, D, false, 1, MT><<<grid, 64, 0, st>>>(t);
            else k_wave_tile<FMT, NPROJ, 2, RT, D, false, 1, MT><<<grid, 64, 0, st>>>(t);
            return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
        }
    }
    if (mxt) return MOE_ERR_ARG;
    if constexpr (NPROJ == 2) {
        if (hx > 1) {   // fp16 / fp32 x planes: one 16-token tile per pass (the host passes nt = 1)
            if (nt != 1) return MOE_ERR_ARG;
            if (hx == 3) k_wave_tile<FMT, 2, 1, RT, D, H16O, 3><<<grid, 64, 0, st>>>(t);
            else k_wave_tile<FMT, 2, 1, RT, D, H16O, 2><<<grid, 64, 0, st>>>(t);
            return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
        }
    }
    if (nt == 1) k_wave_tile<FMT, NPROJ, 1, RT, D, H16O><<<grid, 64, 0, st>>>(t);
    else k_wave_tile<FMT, NPROJ, 2, RT, D, H16O><<<grid, 64, 0, st>>>(t);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

// Environment knobs, read per call (tuning and tests): MOE_DENSE = 0 turns the dense tiles off (the LDS-staged
// row tiles take the calls with more than 32 tokens per expert), 1 uses them for every such call, unset chooses
// by grid size; MOE_WAVE_NT = 1 or 2 forces the wave tiles' token tiles per pass.

// K parts of the dense down projection: 2 when the row blocks x passes would leave the chip under-filled (the
// combine adds the parts' planes); gate/up is never split (the GLU needs whole sums)
int dense_ksplit(int N, int K, int nslots, int E, int BN, int P) {
    const long blocks = (long)((N + BN - 1) / BN) * max_passes(nslots, E, P);
    const int nsl = (K + 127) / 128;
    int ks = env_int("MOE_DENSE_KSPLIT", 0);
    if (ks < 1 || ks > 4) ks = blocks < 4L * 256 && nsl >= 8 ? 2 : 1;
    // parts of ceil(nsl / ks) slices: as many as are non-empty (an empty part would read past the records)
    const int per = (nsl + ks - 1) / ks;
    return (nsl + per - 1) / per;
}

template <class FMT, int NPROJ, int NT = dense_nt<FMT, NPROJ>()>
int launch_dense(TileArgs t, int nslots, hipStream_t st) {
    constexpr int BN = dense_bn<FMT, NPROJ>();
    if (t.N % (16 * dense_rt<FMT, NPROJ>())) return MOE_ERR_ARG;   // whole row tiles per wave
    if (NPROJ == 2) t.ksplit = 1;
    // rounded up to a multiple of 8: every XCD slot then has a workgroup for each of its ceil(items / 8) items
    const long nblk = ((long)((t.N + BN - 1) / BN) * max_passes(nslots, t.E, 16 * NT) * t.ksplit + 7) / 8 * 8;
    if (nblk > 0x7FFFFFF8L) return MOE_ERR_ARG;
    k_dense<FMT, NPROJ, NT><<<dim3((unsigned)nblk), 256, 0, st>>>(t);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}


#ifndef MOE_DENSE_MIN_BLOCKS
#define MOE_DENSE_MIN_BLOCKS 256   // dense gate/up blocks below which the wave tiles fill the chip better
#endif

// The kernels a grouped call runs, from (w, T, k, x dtype) and the tuning environment only, so separately launched
// stages (and the router, which writes the pass lists in moe_layer_run) agree on the layout of h and the passes.
// Tile-major weights present: wave tiles for few tokens per expert, dense tiles for many (unless their grid would fill
// only part of the chip, e.g. a few shared experts: then the wave tiles, 32-token passes). int4 takes the dense down
// from fewer tokens per expert than the dense gate/up (the down's wave tiles read two h planes per token while the
// dense down shares its 64 tokens' h16 across a block): mid loads run the wave gate/up (h out as h16) and the dense
// down, on two pass lists.
struct Plan {
    bool tiled, dense_gu, dense_dn, mxd, wave_gu, wave_dn, mxw, h16, two_lists, ingroup;
    int nt, dn_nt, P_gu, P_dn;
};

template <class FMT>
Plan make_plan(const moe_experts_t* w, int T, int k, int x_dtype) {
    Plan p{};
    const int nslots = T * k;
    const int avg = (nslots + w->E - 1) / w->E;   // expected slots per active expert (uniform routing)
    const int nx = x_dtype == MOE_DTYPE_BF16 ? 1 : (x_dtype == MOE_DTYPE_F16 ? 2 : 3);
    constexpr bool INT4 = FmtInt4::FMT == FMT::FMT;
    p.tiled = w->gate.tiles && w->up.tiles && w->down.tiles;
    const int dmode = env_int("MOE_DENSE", -1);
    constexpr int DP_GU = 16 * dense_nt<FMT, 2>(), DP_DN = 16 * dense_nt<FMT, 1>();
    constexpr int BN_GU = dense_bn<FMT, 2>(), BN_DN = dense_bn<FMT, 1>();
    const long dblocks = (long)((w->F + BN_GU - 1) / BN_GU) * max_passes(nslots, w->E, DP_GU);
    const long dn_blocks = (long)((w->d + BN_DN - 1) / BN_DN) * max_passes(nslots, w->E, DP_DN);
    const int min_avg = env_int("MOE_DENSE_MIN_AVG", 32);
    const int dn_min_avg = env_int("MOE_DENSE_DN_MIN_AVG", 16);
    // activations as planes (fp16 / fp32 x): the dense gate/up takes only what it reads exactly, int4 with fp16 x
    // (x16); fp32 x and MXFP4 keep the exact-operand wave / row tiles, one 16-token tile per pass (nt = 1: the
    // planes' activation registers)
    const bool dense_gu_x = INT4 ? x_dtype != MOE_DTYPE_F32 : nx == 1;
    p.dense_gu = dense_gu_x && p.tiled && avg > min_avg &&
                 (dmode == 1 || (dmode < 0 && dblocks >= MOE_DENSE_MIN_BLOCKS));
    p.dense_dn = p.dense_gu || (INT4 && p.tiled && dmode != 0 && avg > dn_min_avg &&
                                (dmode == 1 || dn_blocks >= MOE_DENSE_MIN_BLOCKS));
    // MXFP4 with bf16 x on the dense tiles: the block-scaled MFMA kernels instead (MOE_MXMFMA=0: the bf16-MFMA
    // dense tiles). x's terms go to the x-planes region, h's terms to the yp planes the split down would use; both
    // must fit there, with 32-bit record offsets
    const size_t mx_xb = (size_t)T * ((w->d + 127) / 128) * mx_rec<2>();
    const size_t mx_hb = (size_t)nslots * ((w->F + 127) / 128) * mx_rec<3>();
    const bool mx_fit = !INT4 && nx == 1 && env_int("MOE_MXMFMA", 1) && mx_xb <= (size_t)6 * T * w->d &&
                        mx_hb <= (size_t)12 * nslots * w->d && mx_hb < (1ull << 32);
    p.mxd = mx_fit && p.dense_gu && w->F % (16 * mxd_rt<2>()) == 0 && w->d % (16 * mxd_rt<1>()) == 0;
    p.wave_gu = p.tiled && !p.dense_gu && (avg <= min_avg || dmode != 0);
    p.wave_dn = p.tiled && !p.dense_dn && (avg <= min_avg || dmode != 0);
    // the wave tiles of MXFP4 with bf16 x on the block-scaled MFMA too (terms as for the dense kernels)
    p.mxw = mx_fit && p.wave_gu && p.wave_dn;
    p.h16 = INT4 && p.dense_dn;   // h leaves the gate/up as h16 with per-32-row exponents
    const int wnt = env_int("MOE_WAVE_NT", 0);
    p.nt = nx > 1 ? 1
         : (p.wave_gu || p.wave_dn) ? (wnt == 1 || wnt == 2 ? wnt : (avg <= 16 ? 1 : 2))
                                    : tokens_per_pass_tiles(T, k, w->E);
    // pass lists: 16 nt tokens per pass for the wave tiles, DP_GU / 16 dn_nt for the dense tiles; a second list
    // when the two stages take different kernels
    // the int4 dense down's pass: 64 tokens (MOE_DENSE_DN_NT = 2, 4, 8 token tiles for A/B runs). Against 128-token
    // passes (each decoded weight tile feeding 8 token tiles, 64 accumulators, 2 waves per SIMD) the 64-token pass
    // runs 4 waves per SIMD (128 VGPRs) and, with twice the items, no K split: DeepSeek-V2-Lite T=256 (31 slots per
    // expert, where a 128-token pass decodes its tiles for 2 live token tiles) 166-168 -> 148-149 us per layer,
    // Mixtral T=512 655-672 -> 638-650 us (32-token passes: 147-153 and 682-696 us)
    const int dnt = env_int("MOE_DENSE_DN_NT", 0);
    p.dn_nt = !INT4 ? dense_nt<FMT, 1>() : (dnt == 2 || dnt == 4 || dnt == 8) ? dnt : 4;
    p.P_gu = p.dense_gu ? DP_GU : 16 * p.nt;
    p.P_dn = p.dense_dn ? 16 * p.dn_nt : 16 * p.nt;
    p.two_lists = p.P_gu != p.P_dn;
    // both stages on the wave tiles with few slots: each workgroup can find its pass from the raw ids itself (an LDS
    // histogram and a wave scan, the grouping launch's order), so the call needs no grouping launch
    p.ingroup = p.wave_gu && p.wave_dn && nslots <= 64 * GW_MAXJ && w->E <= 1024 && env_int("MOE_INGROUP", 1);
    return p;
}

template <class FMT>
int run_tiles_fmt(const ExpertsArgs& a) {
    const moe_experts_t* w = a.w;
    const int nslots = a.T * a.k;
    const int max_active = nslots < w->E ? nslots : w->E;
    TileArgs t{};
    t.ksplit = 1;
    t.counts = a.grp.counts;
    t.offsets = a.grp.offsets;
    t.sorted = a.grp.sorted;
    t.active = a.grp.active;
    t.meta = a.grp.meta;
    t.E = w->E;
    t.act = a.act;
    t.kslots = a.k;
    constexpr bool INT4 = FmtInt4::FMT == FMT::FMT;
    constexpr int BN_DN = dense_bn<FMT, 1>();
    const Plan pl = make_plan<FMT>(w, a.T, a.k, a.x_dtype);
    const bool dense_gu = pl.dense_gu, dense_dn = pl.dense_dn, mxd = pl.mxd && a.xterm, wave_gu = pl.wave_gu,
               wave_dn = pl.wave_dn, mxw = pl.mxw && a.xterm, h16 = pl.h16, two_lists = pl.two_lists;
    const int nt = pl.nt, P_gu = pl.P_gu, P_dn = pl.P_dn;
    if ((pl.mxd || pl.mxw) && !a.xterm) return MOE_ERR_ARG;
    t.items = a.grp.items;
    t.nidx = 2;
    // in-kernel grouping in the gate/up unless the router already wrote the grouping and pass lists; one gate/up
    // workgroup then also writes the lists, and the down stage reads them
    const bool ingroup = pl.ingroup && !a.pregrouped;
    const bool emit = ingroup && !mxw;   // the block-scaled gate/up wave tiles do not write lists: their down groups too
    if (ingroup) {
        t.gidx = a.idx;
        t.gn = nslots;
        // the compact pass list by default: its live passes come first in dispatch order whatever the skew. The
        // expert-major list (MOE_INGROUP_FIRST=1) spares most workgroups the histogram and scan; measured at
        // Qwen3 T=32 it gains ~1.3 us/layer with uniform routing but loses ~6 with Zipf routing, where the hot
        // experts' further passes sit behind ~100 empty rows
        t.gfirst = env_int("MOE_INGROUP_FIRST", 0) ? 1 : 0;
    }
    if (h16) {
        // the second h plane holds the exponent bytes [slots, F/32], then the slot exponents int32 [slots]
        t.eslot_off = ((size_t)nslots * (w->F / 32) + 255) / 256 * 256;
        if (t.eslot_off + (size_t)nslots * 4 > (size_t)nslots * w->F * 2) return MOE_ERR_ARG;
    }
    if (a.stages & 1) {
        int rc = ingroup || a.pregrouped
                     ? 0
                     : launch_group(a.idx, nslots, w->E, a.grp.counts, a.grp.offsets, a.grp.sorted, a.grp.active,
                                       a.grp.meta, a.st, P_gu, a.grp.items, two_lists ? P_dn : 0,
                                       two_lists ? a.grp.items2 : nullptr);
        if (rc) return rc;
        TileArgs g = t;
        if (emit) {
            g.emit_grp = a.grp;
            g.emit_grp.items2 = two_lists ? a.grp.items2 : nullptr;
            g.emit_P = P_gu;
            g.emit_P2 = two_lists ? P_dn : 0;
        }
        g.actv = a.xb;
        g.act_plane = a.xplane;
        g.act_div = a.k;
        g.K = w->d;
        g.N = w->F;
        g.W0 = (const uint8_t*)w->gate.rows;
        g.W1 = (const uint8_t*)w->up.rows;
        g.b0 = w->gate.bias;
        g.b1 = w->up.bias;
        g.hout = a.hhi;
        g.hout2 = a.hlo;
        if (wave_gu || dense_gu) {
            g.W0 = (const uint8_t*)w->gate.tiles;
            g.W1 = (const uint8_t*)w->up.tiles;
        }
        if (mxd || mxw) g.hterm = reinterpret_cast<uint8_t*>(a.yp + (size_t)nslots * w->d);   // h's records
        if (mxd) {
            g.W0 = (const uint8_t*)w->gate.tiles;
            g.W1 = (const uint8_t*)w->up.tiles;
            if (!a.xterm_ready) rc = launch_mx_terms<2>(a.xb, a.T, w->d, a.xterm, a.st);
            g.actv = reinterpret_cast<const uint16_t*>(a.xterm);
            if (!rc) rc = launch_mxd<2, 2>(g, nslots, a.st);
            if (rc) return rc;
        } else if (dense_gu && INT4) {
            if (a.x_dtype == MOE_DTYPE_F16) k_x16<MOE_DTYPE_F16><<<a.T, 256, 0, a.st>>>(a.x, a.x16, a.xexp, w->d);
            else k_x16<MOE_DTYPE_BF16><<<a.T, 256, 0, a.st>>>(a.x, a.x16, a.xexp, w->d);
            rc = hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
            if (rc) return rc;
            g.actv = a.x16;
            g.xexp = a.xexp;
        }
        if (mxw) {
            if (!a.xterm_ready) rc = launch_mx_terms<2>(a.xb, a.T, w->d, a.xterm, a.st);
            g.actv = reinterpret_cast<const uint16_t*>(a.xterm);
            if (!rc) rc = launch_wave_tile<FMT, 2, MOE_WAVE_RT_GU, MOE_WAVE_D_GU>(g, nt, nslots, a.st, 1, 2);
        } else if (mxd) rc = 0;
        else if (dense_gu) rc = launch_dense<FMT, 2>(g, nslots, a.st);
        else if (wave_gu && h16)
            rc = launch_wave_tile<FMT, 2, MOE_WAVE_RT_GU, MOE_WAVE_D_GU, INT4>(g, nt, nslots, a.st, a.nx);
        else if (wave_gu) rc = launch_wave_tile<FMT, 2, MOE_WAVE_RT_GU, MOE_WAVE_D_GU>(g, nt, nslots, a.st, a.nx);
        else rc = launch_tile<FMT, 2>(g, nt, max_active, a.T, a.st, a.nx);
        if (!rc && h16) {
            k_h16_fix<<<nslots, 256, 0, a.st>>>((const int8_t*)a.hlo, a.hhi,
                                              (int32_t*)((uint8_t*)a.hlo + t.eslot_off), w->F);
            rc = hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
        }
        if (rc) return rc;
    }
    if (a.stages & 2) {
        TileArgs d = t;
        if (!ingroup || emit) d.gidx = nullptr;   // the pass lists: from the grouping launch, the router or the gate/up
        d.actv = a.hhi;
        d.actv2 = a.hlo;
        d.act_div = 1;
        d.K = w->F;
        d.N = w->d;
        d.W0 = (const uint8_t*)w->down.rows;
        d.yp = a.yp;
        d.ksplit = dense_dn && !mxd ? dense_ksplit(d.N, d.K, nslots, w->E, BN_DN, P_dn) : 1;
        d.plane = (size_t)nslots * d.N;
        if (two_lists) {
            d.items = a.grp.items2;
            d.nidx = 3;
        }
        if (wave_dn || dense_dn) d.W0 = (const uint8_t*)w->down.tiles;
        d.shallow_min = env_int("MOE_WAVE_DN_SHALLOW", MOE_WAVE_DN_SHALLOW);
        // more row tiles per down wave (fewer activation loads per weight row) where d allows and the grid
        // keeps enough waves
        auto wide_dn = [&](int rt) {
            return rt > 0 && w->d % (16 * rt) == 0 &&
                   (long)(w->d / (16 * rt)) * max_passes(nslots, w->E, 16 * nt) >= MOE_WAVE_WIDE_MIN_WAVES;
        };
        int rc = 0;
        // block-scaled: h's 3-term records, written by the gate/up epilogue into the yp planes after the first
        if (mxw || mxd) d.actv = reinterpret_cast<const uint16_t*>(a.yp + d.plane);
        const int mxt = mxw ? 3 : 0;
        if (mxd) {
            d.W0 = (const uint8_t*)w->down.tiles;
            rc = launch_mxd<1, 3>(d, nslots, a.st);
        } else if (dense_dn) {
            if constexpr (INT4) {
                if (pl.dn_nt == 2) rc = launch_dense<FMT, 1, 2>(d, nslots, a.st);
                else if (pl.dn_nt == 4) rc = launch_dense<FMT, 1, 4>(d, nslots, a.st);
                else rc = launch_dense<FMT, 1>(d, nslots, a.st);
            } else {
                rc = launch_dense<FMT, 1>(d, nslots, a.st);
            }
        }
        else if (wave_dn && wide_dn(MOE_WAVE_RT_DN_WIDE))
            rc = launch_wave_tile<FMT, 1, MOE_WAVE_RT_DN_WIDE, MOE_WAVE_D_DN>(d, nt, nslots, a.st, 1, mxt);
        else if (MOE_WAVE_RT_DN_MID && wave_dn && wide_dn(MOE_WAVE_RT_DN_MID))
            rc = launch_wave_tile<FMT, 1, (MOE_WAVE_RT_DN_MID ? MOE_WAVE_RT_DN_MID : 2), MOE_WAVE_D_DN>(d, nt, nslots, a.st, 1, mxt);
        else if (wave_dn) rc = launch_wave_tile<FMT, 1, MOE_WAVE_RT_DN, MOE_WAVE_D_DN>(d, nt, nslots, a.st, 1, mxt);
        else rc = launch_tile<FMT, 1>(d, nt, max_active, a.T, a.st);
        if (rc) return rc;
        return launch_combine(a.yp, d.ksplit, d.plane, a.idx, a.wts, w->down.bias, w->E,
                              a.residual, a.y, a.T, a.k, w->d, a.ydt, a.st);
    }
    return 0;
}

}  // namespace

int run_experts_tiles(const ExpertsArgs& a) {
    return a.w->fmt == MOE_FMT_INT4_G64 ? run_tiles_fmt<FmtInt4>(a) : run_tiles_fmt<FmtMxfp4>(a);
}

TilePasses tile_passes(const moe_experts_t* w, int T, int k, int x_dtype) {
    const Plan p = w->fmt == MOE_FMT_INT4_G64 ? make_plan<FmtInt4>(w, T, k, x_dtype) : make_plan<FmtMxfp4>(w, T, k, x_dtype);
    return TilePasses{p.P_gu, p.two_lists ? p.P_dn : 0, p.ingroup ? 1 : 0, p.mxd || p.mxw ? 1 : 0};
}

int launch_pack_tiles(int fmt, int E, int N, int K, const void* rows, void* tiles, hipStream_t st) {
    dim3 grid((K + 127) / 128, N / 16, E);
    if (fmt == MOE_FMT_INT4_G64) {
        const int nrows = E * N;
        k_row_exp<<<(nrows + 255) / 256, 256, 0, st>>>(
            (const uint8_t*)rows, (int8_t*)tile_row_exps((const uint8_t*)tiles, E, N, K), nrows, K);
        if (hipGetLastError() != hipSuccess) return MOE_ERR_LAUNCH;
        k_pack_tiles<FmtInt4><<<grid, 64, 0, st>>>((const uint8_t*)rows, (uint8_t*)tiles, N, K);
    } else
        k_pack_tiles<FmtMxfp4><<<grid, 64, 0, st>>>((const uint8_t*)rows, (uint8_t*)tiles, N, K);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

}  // namespace moe

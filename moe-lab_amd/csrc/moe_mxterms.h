// x rows (bf16) -> fp8 term records for gfx950's block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4): the
// layout the block-scaled MXFP4 tiles read their activations in. Written by k_mx_terms, or by the router's
// finishing launch when a layer call feeds those tiles.
#pragma once
#include "moe_common.h"

namespace moe {

// block-scaled MXFP4 tiles: bytes of one (activation row, 128-input slice) record of NTERM fp8 terms + scales
template <int NTERM>
__host__ __device__ constexpr int mx_rec() { return 16 * (8 * NTERM + 1); }

// x rows (bf16) -> per (row, 128-input slice) records of REC = 16 (8 NTERM + 1) bytes: NTERM x 128 bytes of terms
// at mx_pos (the records' code order, then the A operand's lane order), then the E8M0 byte of term t, block b at
// 128 NTERM + 4 t + b. Inputs past K (K % 128 == 64) are zero codes with scale byte 127. This writes block i of
// the rows' 4 ceil(K / 128) blocks each (nothing for i past them). h's records come from the gate/up epilogues
// (mx_h_block).
template <int NTERM>
__device__ __forceinline__ void mx_terms_block(const uint16_t* __restrict__ src, int rows, int K,
                                               uint8_t* __restrict__ out, long i) {
    constexpr int REC = mx_rec<NTERM>();
    const int nsl = (K + 127) >> 7, nb = 4 * nsl;
    if (i >= (long)rows * nb) return;
    const int row = (int)(i / nb), blk = (int)(i - (long)row * nb);
    const int s = blk >> 2, b = blk & 3;
    uint8_t* rec = out + ((size_t)row * nsl + s) * REC;
    float r[32];
    if (32 * blk < K) {
        const uint4* p = reinterpret_cast<const uint4*>(src + (size_t)row * K + 32 * blk);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 v = p[q];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                r[8 * q + 2 * u] = bf16lo(w[u]);
                r[8 * q + 2 * u + 1] = bf16hi(w[u]);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 32; ++j) r[j] = 0.f;
    }
#pragma unroll
    for (int t = 0; t < NTERM; ++t) {
        float am = 0.f;
#pragma unroll
        for (int j = 0; j < 32; ++j) am = fmaxf(am, fabsf(r[j]));
        int e = am > 0.f ? (int)((__float_as_uint(am) >> 23) & 0xFFu) - 127 - 7 : -127;
        e = e < -127 ? -127 : (e > 127 ? 127 : e);
        const float inv = __builtin_ldexpf(1.f, -e);
        // byte j of the block's 32 = input 8 (j / 8) + (0 2 4 6 1 3 5 7)[j % 8]: the order of the codes in the tile
        // records' words (nibbles e0 e2 e4 e6 e1 e3 e5 e7)
        uint32_t qw[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i0 = 8 * (j >> 1) + (j & 1);
            uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(r[i0] * inv, r[i0 + 2] * inv, 0, false);
            w = __builtin_amdgcn_cvt_pk_fp8_f32(r[i0 + 4] * inv, r[i0 + 6] * inv, (int)w, true);
            qw[j] = w;
            r[i0] -= __builtin_ldexpf(__builtin_amdgcn_cvt_f32_fp8((int)w, 0), e);
            r[i0 + 2] -= __builtin_ldexpf(__builtin_amdgcn_cvt_f32_fp8((int)w, 1), e);
            r[i0 + 4] -= __builtin_ldexpf(__builtin_amdgcn_cvt_f32_fp8((int)w, 2), e);
            r[i0 + 6] -= __builtin_ldexpf(__builtin_amdgcn_cvt_f32_fp8((int)w, 3), e);
        }
        uint8_t* tq = rec + 128 * t + 64 * (b & 1) + 16 * (b >> 1);
        *reinterpret_cast<uint4*>(tq) = uint4{qw[0], qw[1], qw[2], qw[3]};        // code words 0, 1 of the block
        *reinterpret_cast<uint4*>(tq + 32) = uint4{qw[4], qw[5], qw[6], qw[7]};   // code words 2, 3
        rec[128 * NTERM + 4 * t + b] = (uint8_t)(32 * blk < K ? e + 127 : 127);
    }
}

}  // namespace moe

// Packed weight formats of the gfx950 MoE kernels: how a 16-byte chunk (32 inputs) of a row record is
// decoded to bf16 pairs and how its group metadata folds into the fp32 accumulator.
//
// A row record of K inputs: K/2 code bytes (8 nibbles per 32-bit word, low nibble first, as the reference's
// state words, metal_q4_decode_v4.py:57-64), then the group metadata, zero-padded to 16 bytes:
//   int4 g64: K/64 words (scale bf16 | bias bf16 << 16), w = scale*q + bias
//   MXFP4:    K/32 E8M0 bytes, w = e2m1(q) * 2^(s-127)  (reference metal_mxfp4_moe.py:1-41)
// Decoded pairs hold the elements (8j+i, 8j+i+4) of word j (i = 0..3), so the activation side is paired the
// same way (pair_x32), and an 8-element group handed to MFMA is in the order (0,4,1,5,2,6,3,7).
#pragma once
#include "moe_common.h"
#include "moe_mi355x.h"

namespace moe {

// bytes of one packed row record of K inputs (include/moe_mi355x.h: moe_row_bytes)
__host__ __device__ __forceinline__ size_t rbytes(int fmt, int K) {
    const size_t meta = fmt == MOE_FMT_INT4_G64 ? (size_t)K / 16 : (size_t)K / 32;
    return ((size_t)K / 2 + meta + 15) & ~(size_t)15;
}

// tile-major slice records (include/moe_mi355x.h: moe_tile_bytes): 16 rows x 128 inputs of codes + metadata
constexpr int TILE_SLICE_INT4 = 1024 + 16 * 8;
constexpr int TILE_SLICE_MXFP4 = 1024 + 16 * 4;
// one expert's slice records
__host__ __device__ __forceinline__ size_t tile_rec_bytes(int fmt, int N, int K) {
    const size_t sb = fmt == MOE_FMT_INT4_G64 ? TILE_SLICE_INT4 : TILE_SLICE_MXFP4;
    return (size_t)(N / 16) * (size_t)((K + 127) / 128) * sb;
}
// per expert: its records, plus (int4) one row-exponent byte per row; the exponent bytes of all E experts follow
// the records of all E experts
__host__ __device__ __forceinline__ size_t tile_bytes(int fmt, int N, int K) {
    return tile_rec_bytes(fmt, N, K) + (fmt == MOE_FMT_INT4_G64 ? (size_t)N : 0);
}
// int4 tile copies: the row exponents int8 [E, N] of projection base `tiles` (E experts)
__host__ __device__ __forceinline__ const int8_t* tile_row_exps(const uint8_t* tiles, int E, int N, int K) {
    return reinterpret_cast<const int8_t*>(tiles + (size_t)E * tile_rec_bytes(MOE_FMT_INT4_G64, N, K));
}
// Row exponent of an int4 row from amax, the largest bf16 magnitude bits (sign cleared) over the row's scales and
// biases: the records hold s 2^-E and b 2^-E (exact in bf16), which puts the row's largest at [2^10, 2^11) whatever
// the row's absolute scale. The dense tiles dequantise to fp16 w' = (s q + b) 2^-E 2^-16, below 2^-1 in magnitude:
// weights down to 2^-13 of that bound are normal fp16 numbers, smaller ones round to fp16's subnormal step 2^-24
// (2^-19 of the row's largest |s|, |b| in the same units), so a row's within-row dynamic range, not its absolute
// scale, is what limits their precision. E = (biased exponent of amax) - 127 - 10, clamped to [-120, 120] (bf16
// subnormals: -120); 0 for an all-zero row or one holding an inf or NaN.
__host__ __device__ __forceinline__ int int4_row_exponent(uint32_t amax) {
    const int ef = (int)(amax >> 7);
    if (amax == 0 || ef >= 0xFF) return 0;
    const int e = ef - 137;
    return e < -120 ? -120 : (e > 120 ? 120 : e);
}

// ============================================================================ packed row formats
struct FmtInt4 {
    static constexpr int FMT = MOE_FMT_INT4_G64;
    static constexpr bool XSUM = true;   // the fold needs sum(x) over each chunk
    __device__ static __forceinline__ uint32_t meta(const uint8_t* row, int K, int c) {
        return *reinterpret_cast<const uint32_t*>(row + (K >> 1) + 4 * (c >> 1));
    }
    // byte offset of chunk c's metadata word inside its row, and the load at a 32-bit offset from a wave-uniform
    // base (the base in SGPRs, the offset in one VGPR: no 64-bit address arithmetic per load)
    __device__ static __forceinline__ uint32_t meta_off(int K, int c) { return (uint32_t)(K >> 1) + 4u * (uint32_t)(c >> 1); }
    __device__ static __forceinline__ uint32_t meta_at(const uint8_t* base, uint32_t off) {
        return *reinterpret_cast<const uint32_t*>(base + off);
    }
    // 7 VALU ops per word: t holds nibbles 0, 2, 4, 6 and u nibbles 1, 3, 5, 7 in the low halves of its
    // bytes; each v_perm_b32 picks two of those bytes and puts the bf16 exponent byte 0x43 above each.
    __device__ static __forceinline__ void decode_word(uint32_t w, uint32_t q[4]) {
        const uint32_t t = w & 0x0F0F0F0Fu, u = (w >> 4) & 0x0F0F0F0Fu;
        q[0] = __builtin_amdgcn_perm(0x43434343u, t, 0x04020400u);   // (q0, q4)
        q[1] = __builtin_amdgcn_perm(0x43434343u, u, 0x04020400u);   // (q1, q5)
        q[2] = __builtin_amdgcn_perm(0x43434343u, t, 0x04030401u);   // (q2, q6)
        q[3] = __builtin_amdgcn_perm(0x43434343u, u, 0x04030401u);   // (q3, q7)
    }
    __device__ static __forceinline__ void decode(uint4 w, uint32_t qp[16]) {
        decode_word(w.x, qp);
        decode_word(w.y, qp + 4);
        decode_word(w.z, qp + 8);
        decode_word(w.w, qp + 12);
    }
    // per-slot GEMV rows: the same (n, n + 4) pairs (one shift and mask per two codes), x and h paired to match
    static constexpr bool ROWS_NAT = false;
    __device__ static __forceinline__ void decode_rows(uint4 w, uint32_t qp[16]) { decode(w, qp); }
    __device__ static __forceinline__ float fold(float acc, uint32_t m, float dot, float xsum) {
        const float s = bf16lo(m), b = bf16hi(m);
        return __builtin_fmaf(s, dot, __builtin_fmaf(__builtin_fmaf(-128.f, s, b), xsum, acc));
    }
};

struct FmtMxfp4 {
    static constexpr int FMT = MOE_FMT_MXFP4;
    static constexpr bool XSUM = false;
    __device__ static __forceinline__ uint32_t meta(const uint8_t* row, int K, int c) { return row[(K >> 1) + c]; }
    __device__ static __forceinline__ uint32_t meta_off(int K, int c) { return (uint32_t)(K >> 1) + (uint32_t)c; }
    __device__ static __forceinline__ uint32_t meta_at(const uint8_t* base, uint32_t off) { return base[off]; }
    // gfx950's v_cvt_scalef32_pk_bf16_fp4 turns the two E2M1 codes of one byte (low nibble first) into two bf16
    // (scale 1: exact), giving (e0, e1), (e2, e3), (e4, e5), (e6, e7); one v_perm_b32 per pair word regroups them
    // into the (n, n + 4) pairs the activations are laid out in. 8 VALU per code word, bit-identical to a
    // table decode of {0, .5, 1, 1.5, 2, 3, 4, 6} x sign for every byte value.
    __device__ static __forceinline__ void decode_word(uint32_t v, uint32_t q[4]) {
        const uint32_t p0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 0));
        const uint32_t p1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 1));
        const uint32_t p2 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 2));
        const uint32_t p3 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 3));
        q[0] = __builtin_amdgcn_perm(p2, p0, 0x05040100u);   // (e0, e4)
        q[1] = __builtin_amdgcn_perm(p2, p0, 0x07060302u);   // (e1, e5)
        q[2] = __builtin_amdgcn_perm(p3, p1, 0x05040100u);   // (e2, e6)
        q[3] = __builtin_amdgcn_perm(p3, p1, 0x07060302u);   // (e3, e7)
    }
    __device__ static __forceinline__ void decode(uint4 w, uint32_t qp[16]) {
        decode_word(w.x, qp);
        decode_word(w.y, qp + 4);
        decode_word(w.z, qp + 8);
        decode_word(w.w, qp + 12);
    }
    // Per-slot GEMV rows (k_gate_up_rows, k_down_rows): the codes in natural pairs (e_2b, e_2b+1) of each byte, as
    // the convert yields them (4 VALU per code word, no v_perm), against x and h in natural order too
    static constexpr bool ROWS_NAT = true;
    __device__ static __forceinline__ void decode_rows(uint4 w, uint32_t qp[16]) {
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qp[4 * i + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[i], 1.0f, 0));
            qp[4 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[i], 1.0f, 1));
            qp[4 * i + 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[i], 1.0f, 2));
            qp[4 * i + 3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[i], 1.0f, 3));
        }
    }
    // the same as fp16 (v_cvt_scalef32_pk_f16_fp4, scale 1: every e2m1 value is exact in fp16), for the per-slot
    // down when h is one fp16 plane
    __device__ static __forceinline__ void decode_rows_f16(uint4 w, uint32_t qp[16]) {
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qp[4 * i + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], 1.0f, 0));
            qp[4 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], 1.0f, 1));
            qp[4 * i + 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], 1.0f, 2));
            qp[4 * i + 3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wd[i], 1.0f, 3));
        }
    }
    __device__ static __forceinline__ float fold(float acc, uint32_t m, float dot, float) {
        return __builtin_fmaf(__uint_as_float(m << 23), dot, acc);
    }
};

}  // namespace moe

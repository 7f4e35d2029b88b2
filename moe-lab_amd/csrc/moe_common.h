// Shared device helpers for the gfx950 MoE kernels (wave64, CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

#include "moe_mi355x.h"

#define MOE_WAVE 64

typedef __bf16 moe_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 moe_f16x2 __attribute__((ext_vector_type(2)));

namespace moe {

// ------------------------------------------------------------------------------------ bf16 / fp32
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// a.x*b.x + a.y*b.y + c with bf16 pairs packed in 32-bit words (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(moe_bf16x2, a), __builtin_bit_cast(moe_bf16x2, b), c,
                                           false);
}

// Two 4-bit codes of one word -> a bf16 pair holding (128 + q_i, 128 + q_{i+4}): the code lands in the
// low mantissa bits of 128.0 (bf16 0x4300), whose ulp is exactly 1. Nibble i sits at bits 4i..4i+3 and
// nibble i+4 at bits 16+4i.., so one shift + mask + or decodes two weights.
__device__ __forceinline__ uint32_t q4pair_bf16(uint32_t word, int i) {
    return ((word >> (4 * i)) & 0x000F000Fu) | 0x43004300u;
}
#define MOE_Q4_OFFSET 128.0f

// Activation pairs matching q4pair_bf16's element order: for word j of a 32-element chunk the pair for
// nibble i is (x[8j+i], x[8j+i+4]). xw are the 16 words holding 32 consecutive bf16 (low half = even).
__device__ __forceinline__ void pair_x32(const uint32_t xw[16], uint32_t xp[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t a = xw[4 * j + 0], b = xw[4 * j + 1], c = xw[4 * j + 2], d = xw[4 * j + 3];
        xp[4 * j + 0] = (a & 0xffffu) | (c << 16);          // (x0, x4)
        xp[4 * j + 1] = (a >> 16) | (c & 0xffff0000u);      // (x1, x5)
        xp[4 * j + 2] = (b & 0xffffu) | (d << 16);          // (x2, x6)
        xp[4 * j + 3] = (b >> 16) | (d & 0xffff0000u);      // (x3, x7)
    }
}

// sum over 32 bf16 held as 16 words (any pairing)
__device__ __forceinline__ float sum_x32(const uint32_t xw[16]) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s = dot2_bf16(xw[i], 0x3f803f80u, s);
    return s;
}

// sum_k (128 + q_k) * x_k over one 16-byte chunk of 32 codes against paired activations
__device__ __forceinline__ float dot_q4x32(uint4 w, const uint32_t xp[16]) {
    float acc = 0.f;
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = dot2_bf16(q4pair_bf16(ws[j], i), xp[4 * j + i], acc);
    return acc;
}

__device__ __forceinline__ void load_x32(const uint16_t* p, uint32_t xw[16]) {
    const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint4 v = q[i];
        xw[4 * i + 0] = v.x;
        xw[4 * i + 1] = v.y;
        xw[4 * i + 2] = v.z;
        xw[4 * i + 3] = v.w;
    }
}

// ------------------------------------------------------------------------------------ DPP reductions
// v + (v moved across lanes by a DPP pattern); lanes the pattern does not write add 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                     0xF, false));
}
// Sum over aligned groups of G lanes (G = 1..64, power of two) with DPP moves only (no LDS crossbar):
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror, row_bcast15, row_bcast31.
// G <= 16: every lane of the group holds the sum. G == 32: lanes 16..31 of each 32-lane group do.
// G == 64: lanes 48..63 do. sum_lane<G>() names one lane offset inside the group that holds it.
template <int G>
__device__ __forceinline__ float sum_lanes(float v) {
    if (G >= 2) v = dpp_add<0xB1>(v);
    if (G >= 4) v = dpp_add<0x4E>(v);
    if (G >= 8) v = dpp_add<0x141>(v);
    if (G >= 16) v = dpp_add<0x140>(v);
    if (G >= 32) v = dpp_add<0x142, 0xA>(v);
    if (G >= 64) v = dpp_add<0x143, 0xC>(v);
    return v;
}
// Inclusive prefix sum over the 64 lanes: row_shr steps inside each row of 16 lanes, then the row totals
// (lanes 15, 31, 47) read as scalars and added to the rows after them.
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);   // row_shr:8
    const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31),
              r2 = __builtin_amdgcn_readlane(v, 47);
    const int row = (threadIdx.x & 63) >> 4;
    return v + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}
template <int G>
__host__ __device__ constexpr int sum_lane() { return G <= 16 ? 0 : (G == 32 ? 16 : 48); }

// Wave-wide max (fp32) / min (u32) with the same DPP pattern; every lane gets the result (read from lane 63).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_max(float v) {
    const float o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, -INFINITY),
                                                                         __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                         0xF, false));
    return fmaxf(v, o);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_min(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp((int)0xFFFFFFFFu, (int)v, CTRL, ROW_MASK, 0xF, false);
    return o < v ? o : v;
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = dpp_max<0xB1>(v);
    v = dpp_max<0x4E>(v);
    v = dpp_max<0x141>(v);
    v = dpp_max<0x140>(v);
    v = dpp_max<0x142, 0xA>(v);
    v = dpp_max<0x143, 0xC>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ uint32_t wave_min_dpp(uint32_t v) {
    v = dpp_min<0xB1>(v);
    v = dpp_min<0x4E>(v);
    v = dpp_min<0x141>(v);
    v = dpp_min<0x140>(v);
    v = dpp_min<0x142, 0xA>(v);
    v = dpp_min<0x143, 0xC>(v);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
// u32 max with the same DPP pattern; 0 (the max's identity) fills lanes a row mask leaves out, so each step can be
// one v_max_u32 with a DPP source operand
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_umax(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xF, false);
    return o > v ? o : v;
}
__device__ __forceinline__ uint32_t wave_umax_dpp(uint32_t v) {
    v = dpp_umax<0xB1>(v);
    v = dpp_umax<0x4E>(v);
    v = dpp_umax<0x141>(v);
    v = dpp_umax<0x140>(v);
    v = dpp_umax<0x142, 0xA>(v);
    v = dpp_umax<0x143, 0xC>(v);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = sum_lanes<64>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Cross-workgroup data on MI355X: the XCDs' L2 caches are not coherent with each other, and agent-scope
// release/acquire fences write back / invalidate a whole L2. Data handed between workgroups of one launch
// therefore goes through agent-scope atomic stores and loads (coherent at device level on their own), and a
// producer waits for its stores (s_waitcnt vmcnt(0): gfx9 counts stores in vmcnt) before it counts itself
// done with an agent-scope atomic add.
__device__ __forceinline__ void store_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int load_agent(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_agent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }

// ------------------------------------------------------------------------------------ wave reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) v += __shfl_xor(v, s, MOE_WAVE);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) v = fmaxf(v, __shfl_xor(v, s, MOE_WAVE));
    return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        uint32_t o = __shfl_xor(v, s, MOE_WAVE);
        v = o < v ? o : v;
    }
    return v;
}
// sum within aligned groups of G lanes (G a power of two <= 64); every lane of the group gets the sum
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int s = G / 2; s >= 1; s >>= 1) v += __shfl_xor(v, s, MOE_WAVE);
    return v;
}

// ------------------------------------------------------------------------------------ activations
// act 0: SiLU(g) * u; 1: tanh-GELU(g) * u; 2: gpt-oss clamped SwiGLU, g = min(g, 7), u = clip(u, -7, 7),
// g * sigmoid(1.702 g) * (u + 1).
template <int ACT>
__device__ __forceinline__ float glu(float g, float u) {
    if (ACT == 0) return g / (1.f + expf(-g)) * u;
    if (ACT == 1) return 0.5f * g * (1.f + tanhf(0.7978845608028654f * (g + 0.044715f * g * g * g))) * u;
    g = fminf(g, 7.f);
    u = fminf(fmaxf(u, -7.f), 7.f);
    return g / (1.f + expf(-1.702f * g)) * (u + 1.f);
}

__device__ __forceinline__ float glu_act(int act, float g, float u) {
    return act == 0 ? glu<0>(g, u) : (act == 1 ? glu<1>(g, u) : glu<2>(g, u));
}

// ------------------------------------------------------------------------------------ GEMV pieces (T = 1 kernels)
__device__ __forceinline__ float dot16(const uint32_t qp[16], const uint32_t xp[16], float acc) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc = dot2_bf16(qp[i], xp[i], acc);
    return acc;
}
__device__ __forceinline__ void words16(const uint4 v[4], uint32_t w[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w[4 * i + 0] = v[i].x;
        w[4 * i + 1] = v[i].y;
        w[4 * i + 2] = v[i].z;
        w[4 * i + 3] = v[i].w;
    }
}
__device__ __forceinline__ float sum16(const uint32_t w[16], float acc) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc = dot2_bf16(w[i], 0x3f803f80u, acc);
    return acc;
}

// h element n -> position inside its chunk so that 16-byte loads yield (n, n+4) pairs
__device__ __forceinline__ int paired_pos(int n) { return (n & ~7) | ((n & 3) << 1) | ((n >> 2) & 1); }
// nat: element n at position n (the MXFP4 per-slot rows, FmtMxfp4::ROWS_NAT), else pre-paired
__device__ __forceinline__ void store_h(uint16_t* hhi, uint16_t* hlo, size_t base, int n, float v, bool nat = false) {
    const uint16_t hi = f32_to_bf16(v);
    const size_t i = base + (nat ? n : paired_pos(n));
    hhi[i] = hi;
    hlo[i] = f32_to_bf16(v - bf16_to_f32(hi));
}

// The per-slot GEMV path (k_gate_up_rows -> k_down_rows) keeps h as one fp16 plane (in hhi, same pairing) when
// its value is bounded above: MXFP4 weights with the gpt-oss GLU, whose clamps (g <= 7, |u| <= 7) give
// |h| <= 7 * 1 * 8 = 56. The plane holds h 2^8 (<= 14336 < 65504), so h keeps fp16's 11 significant bits down to
// |h| = 2^-22 and an absolute step of 2^-32 below that (the hi + lo bf16 planes: ~16 bits at any magnitude), with
// half the bytes; the e2m1 codes decode to fp16 exactly and the down scales its sums back by 2^-8.
__host__ __device__ constexpr bool h_is_f16(int fmt, int act) { return fmt == MOE_FMT_MXFP4 && act == MOE_ACT_GPTOSS; }
#define MOE_H16_SCALE 256.0f
__device__ __forceinline__ void store_h16(uint16_t* h16, size_t base, int n, float v, bool nat) {
    h16[base + (nat ? n : paired_pos(n))] = __builtin_bit_cast(uint16_t, (_Float16)(v * MOE_H16_SCALE));
}
// a.x*b.x + a.y*b.y + c with fp16 pairs packed in 32-bit words (v_dot2_f32_f16)
__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(moe_f16x2, a), __builtin_bit_cast(moe_f16x2, b), c, false);
}
__device__ __forceinline__ float dot16_f16(const uint32_t qp[16], const uint32_t hp[16], float acc) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc = dot2_f16(qp[i], hp[i], acc);
    return acc;
}

// outputs and residuals: ydt = MOE_DTYPE_BF16, MOE_DTYPE_F16 or MOE_DTYPE_F32 (round to nearest even)
__device__ __forceinline__ void store_y(void* y, size_t i, float v, int ydt) {
    if (ydt == MOE_DTYPE_F32) reinterpret_cast<float*>(y)[i] = v;
    else if (ydt == MOE_DTYPE_F16) reinterpret_cast<_Float16*>(y)[i] = (_Float16)v;
    else reinterpret_cast<uint16_t*>(y)[i] = f32_to_bf16(v);
}
__device__ __forceinline__ float load_y(const void* y, size_t i, int ydt) {
    if (ydt == MOE_DTYPE_F32) return reinterpret_cast<const float*>(y)[i];
    if (ydt == MOE_DTYPE_F16) return (float)reinterpret_cast<const _Float16*>(y)[i];
    return bf16_to_f32(reinterpret_cast<const uint16_t*>(y)[i]);
}
// the same value in two steps: the raw bits (a load with no use, so no wait on it follows), then the conversion
// where the value is needed (a conversion inside the dtype branch would make the load's wait immediate, and the
// in-order memory counter would then also wait for every load issued before it)
__device__ __forceinline__ uint32_t load_y_bits(const void* y, size_t i, int ydt) {
    if (ydt == MOE_DTYPE_F32) return reinterpret_cast<const uint32_t*>(y)[i];
    return reinterpret_cast<const uint16_t*>(y)[i];
}
__device__ __forceinline__ float y_bits_f32(uint32_t b, int ydt) {
    if (ydt == MOE_DTYPE_F32) return __uint_as_float(b);
    if (ydt == MOE_DTYPE_F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
    return bf16_to_f32((uint16_t)b);
}

// ------------------------------------------------------------------------------------ router tail
constexpr int TOPK_MAX_J = 16;    // E <= 64 * 16 = 1024

// One wave: router tail for one token (reference moelab/router.py:15-66). `lg(e)` yields logit e as fp32. Lane r < k
// ends with round r's expert id (*id) and routing weight (*w): NaN counts as -inf, k rounds of arg-max with the lowest
// id winning ties, fewer than k finite logits -> the lowest unused ids with weight 0; norm: softmax over the top-k
// logits, !norm: full-softmax probabilities; weights times scale. rounds <= k stops after that many rounds (a caller
// that needs only round r passes r + 1; the weights are then not computed). JM >= ceil(E / 64) logits per lane
// (logit j * 64 + lane in v[j]). The rounds run on order-preserving u32 keys of the logits (a larger logit has a
// larger key; -0 keys as +0, since the two compare equal; a chosen logit's key becomes 0, below every logit's): a
// round is one DPP max over the lanes' largest keys (one v_max_u32 per step), then the lowest id holding it from one
// ballot per j (the lowest j with a lane at the maximum, then the lowest such lane).
__device__ __forceinline__ uint32_t logit_key(float f) {
    const uint32_t b = __float_as_uint(f == 0.f ? 0.f : f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_logit(uint32_t key) {
    return __uint_as_float((key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key);
}
template <int JM>
__device__ __forceinline__ void topk_core(float (&v)[JM], int E, int k, int norm, float scale, int rounds, uint32_t* id,
                                          float* w) {
    const int lane = threadIdx.x & 63;
    uint32_t key[JM];
#pragma unroll
    for (int j = 0; j < JM; ++j) {
        if (__builtin_isnan(v[j]) || j * 64 + lane >= E) v[j] = -INFINITY;
        key[j] = logit_key(v[j]);
    }
    const uint32_t KNEG = 0x007FFFFFu;   // logit_key(-inf): keys at or below it are no candidates
    const bool weights = rounds >= k;
    float m0 = -INFINITY;
#pragma unroll
    for (int j = 0; j < JM; ++j) m0 = fmaxf(m0, v[j]);
    if (weights) m0 = wave_max_dpp(m0);
    float den = 0.f;
    if (weights && !norm) {
#pragma unroll
        for (int j = 0; j < JM; ++j) den += (v[j] == -INFINITY) ? 0.f : expf(v[j] - m0);
        den = wave_sum_dpp(den);
    }
    float myv = -INFINITY;   // lane r < k holds round r's value and id
    uint32_t myi = 0;
    float top0 = -INFINITY;
    for (int r = 0; r < rounds; ++r) {
        uint32_t b = key[0];
#pragma unroll
        for (int j = 1; j < JM; ++j) b = key[j] > b ? key[j] : b;
        const uint32_t mk = wave_umax_dpp(b);
        uint32_t sel;
        float m;
        if (mk > KNEG) {   // wave-uniform: a finite (or +inf) logit is left
            sel = 0xFFFFFFFFu;
#pragma unroll
            for (int j = 0; j < JM; ++j) {
                const uint64_t hit = __ballot(key[j] == mk);
                if (sel == 0xFFFFFFFFu && hit) sel = (uint32_t)(j * 64 + __builtin_ctzll(hit));
            }
            m = key_logit(mk);
            if ((int)(sel & 63u) == lane) {
#pragma unroll
                for (int j = 0; j < JM; ++j)
                    if (j == (int)(sel >> 6)) key[j] = 0u;
            }
        } else {   // no finite candidate left: lowest id not chosen yet, weight 0
            sel = 0;
            while (__ballot(lane < r && myi == sel) != 0ull) ++sel;
            m = -INFINITY;
        }
        if (r == 0) top0 = m;
        if (lane == r) { myv = m; myi = sel; }
    }
    *id = myi;
    *w = 0.f;
    if (!weights) return;
    float s;
    if (norm) s = wave_sum_dpp(lane < k ? expf(myv - top0) : 0.f);
    else s = den;
    const float off = norm ? top0 : m0;
    *w = expf(myv - off) / s * scale;
}
// One wave, one rank: the expert id of round q of topk_core's tail on the same logits (q < k), without the q earlier
// rounds. Among the finite logits (nfin of them), round q's logit is the one of key Kq, the largest key with more than
// q keys at or above it, found bit by bit from the top (32 steps of one ballot and popcount per j); round q takes the
// (q - #keys above Kq)-th lowest id holding Kq. Past the finite logits (q >= nfin) round q takes the (q - nfin)-th
// lowest id below E whose logit is not finite, as topk_core's fallback does. Wave-uniform result.
template <int JM>
__device__ __forceinline__ uint32_t topk_rank_id(float (&v)[JM], int E, int q) {
    const int lane = threadIdx.x & 63;
    const uint32_t KNEG = 0x007FFFFFu;   // logit_key(-inf)
    uint32_t key[JM];
    int nfin = 0;
#pragma unroll
    for (int j = 0; j < JM; ++j) {
        const bool in = j * 64 + lane < E;
        key[j] = in && !__builtin_isnan(v[j]) ? logit_key(v[j]) : KNEG;
        nfin += __builtin_popcountll(__ballot(key[j] > KNEG));
    }
    uint64_t pick[JM];   // the candidates of rank q's kind, in ascending id (j-major)
    int skip;
    if (q < nfin) {
        uint32_t K = 0;
        for (int bit = 31; bit >= 0; --bit) {
            const uint32_t c = K | (1u << bit);
            int n = 0;
#pragma unroll
            for (int j = 0; j < JM; ++j) n += __builtin_popcountll(__ballot(key[j] >= c));
            K = n > q ? c : K;
        }
        int gt = 0;
#pragma unroll
        for (int j = 0; j < JM; ++j) {
            gt += __builtin_popcountll(__ballot(key[j] > K));
            pick[j] = __ballot(key[j] == K);
        }
        skip = q - gt;
    } else {
#pragma unroll
        for (int j = 0; j < JM; ++j) pick[j] = __ballot(key[j] <= KNEG && j * 64 + lane < E);
        skip = q - nfin;
    }
    uint32_t sel = 0;
    bool found = false;
#pragma unroll
    for (int j = 0; j < JM; ++j) {
        uint64_t m = pick[j];
        const int c = __builtin_popcountll(m);
        if (!found && skip < c) {
            for (int i = 0; i < skip; ++i) m &= m - 1;
            sel = (uint32_t)(j * 64 + __builtin_ctzll(m));
            found = true;
        } else if (!found) {
            skip -= c;
        }
    }
    return sel;
}

// topk_core on logits read through lg(e) (logit j * 64 + lane into v[j]; e >= E is not read)
template <int JM, typename F>
__device__ __forceinline__ void topk_lanes(F lg, int E, int k, int norm, float scale, int rounds, uint32_t* id,
                                           float* w) {
    const int lane = threadIdx.x & 63;
    float v[JM];
#pragma unroll
    for (int j = 0; j < JM; ++j) {
        const int e = j * 64 + lane;
        v[j] = e < E ? lg(e) : -INFINITY;
    }
    topk_core<JM>(v, E, k, norm, scale, rounds, id, w);
}
template <typename F>
__device__ __forceinline__ void wave_topk_lanes(F lg, int E, int k, int norm, float scale, int rounds, uint32_t* id,
                                                float* w) {
    if (E <= 64) topk_lanes<1>(lg, E, k, norm, scale, rounds, id, w);
    else if (E <= 128) topk_lanes<2>(lg, E, k, norm, scale, rounds, id, w);
    else if (E <= 256) topk_lanes<4>(lg, E, k, norm, scale, rounds, id, w);
    else topk_lanes<TOPK_MAX_J>(lg, E, k, norm, scale, rounds, id, w);
}

// topk_rank_id on logits read through lg(e)
template <typename F>
__device__ __forceinline__ uint32_t wave_rank_id(F lg, int E, int q) {
    auto run = [&](auto jm) __attribute__((always_inline)) {
        constexpr int JM = decltype(jm)::value;
        const int lane = threadIdx.x & 63;
        float v[JM];
#pragma unroll
        for (int j = 0; j < JM; ++j) {
            const int e = j * 64 + lane;
            v[j] = e < E ? lg(e) : -INFINITY;
        }
        return topk_rank_id<JM>(v, E, q);
    };
    if (E <= 64) return run(std::integral_constant<int, 1>{});
    if (E <= 128) return run(std::integral_constant<int, 2>{});
    if (E <= 256) return run(std::integral_constant<int, 4>{});
    return run(std::integral_constant<int, TOPK_MAX_J>{});
}

// One wave: router tail for one token, written to idx[k], wts[k].
template <typename F>
__device__ void wave_topk(F lg, int E, int k, int norm, float scale, int32_t* idx, float* wts) {
    uint32_t id;
    float w;
    wave_topk_lanes(lg, E, k, norm, scale, k, &id, &w);
    const int lane = threadIdx.x & 63;
    if (lane < k) {
        idx[lane] = (int32_t)id;
        wts[lane] = w;
    }
}

}  // namespace moe

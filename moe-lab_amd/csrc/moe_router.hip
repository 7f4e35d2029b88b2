// Router and slot grouping kernels for gfx950.
//
// router_logits: logits[t, e] = x[t] . Wr[e] (+ b[e]) in fp32, one wave per EPW experts x TPW tokens. route_finish,
// the next launch: the router tail (top-k, softmax) of one token per wave and, when the call asks for the grouping,
// the sort of all T*k slots by expert (group_block) in its last workgroup to finish. At T = 1 the layer call skips
// route_finish: the gate/up waves rank the token's logits themselves (moe_experts.hip).
// The logit reduction order is fixed, so a CPU restatement reproduces every logit bit for bit and top-k ids
// match exactly: lane l takes the 8-element chunks l, l+64, ... in order with fused multiply-adds in
// element order, starting from +0; the 64 lane partials a[0..63] are combined by the DPP tree of
// sum_lanes<64>: quads Q[q] = (a[4q] + a[4q+1]) + (a[4q+2] + a[4q+3]), half-rows H[h] = Q[2h] + Q[2h+1],
// rows R[r] = H[2r] + H[2r+1], total = (R[3] + R[2]) + (R[1] + R[0]); the bias is added last.
//
// Router tail semantics follow reference moelab/router.py:1-66: NaN counts as -inf, k rounds of arg-max
// with the lowest expert id winning ties, fewer than k finite logits -> lowest unused ids with weight 0,
// norm: softmax over the top-k logits, !norm: full-softmax probabilities; weights times `scale`.
//
// Grouping (group_block, run by the router's last block or by the group_slots launch): stable grouping of the
// T*k slots by expert (reference metal_q4_tiles_v2.py:362-373 lists a tile's slots in ascending slot id; closed
// form = stable argsort, reference triton_fused_moe.py:56-70), offsets from a wave prefix sum of the counts.
#include "moe_common.h"
#include "moe_group.h"
#include "moe_internal.h"
#include "moe_mxterms.h"

namespace moe {

constexpr int ROUTER_WAVES = 4;   // waves per block
constexpr int ROUTER_TPW = 4;     // tokens per wave for T > 1 (the Wr row chunk is reused across them)


template <typename LT>
__device__ __forceinline__ float to_f32(LT v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return bf16_to_f32(v); }
template <>
__device__ __forceinline__ float to_f32<_Float16>(_Float16 v) { return (float)v; }

constexpr int ROUTER_MAXC = 4;   // 16-byte chunks per lane held in registers per pass (2048 inputs)

// Logits: grid (ceil(rows / (ROUTER_WAVES * EPW)), ceil(T / TPW)), block 64 * ROUTER_WAVES; rows = a.lstride (the E
// router rows, plus the shared experts' gate row when a.gate is given). Each wave computes EPW rows for TPW tokens
// (the Wr chunk it loads serves all TPW tokens), so the E*d router bytes spread over many CUs.
template <int TPW, int EPW>
__global__ void __launch_bounds__(64 * ROUTER_WAVES) router_logits(RouterArgs a) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int rows = a.lstride;
    const int e0 = (blockIdx.x * ROUTER_WAVES + wave) * EPW;
    const int t0 = blockIdx.y * TPW;
    const int nt = min(TPW, a.T - t0);
    const int d = a.d;
    const int nchunk = d >> 3;
    if (a.arrive && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *a.arrive = 0;
    if (e0 >= rows) return;
    const uint16_t* wrow[EPW];   // row e < E of Wr, row E the gate
#pragma unroll
    for (int q = 0; q < EPW; ++q) {
        const int e = min(e0 + q, rows - 1);
        wrow[q] = e < a.E ? a.wr + (size_t)e * d : a.gate;
    }
    float acc[EPW][TPW];
#pragma unroll
    for (int q = 0; q < EPW; ++q)
#pragma unroll
        for (int i = 0; i < TPW; ++i) acc[q][i] = 0.f;
    for (int c0 = 0; c0 < nchunk; c0 += 64 * ROUTER_MAXC) {
        // all loads of this pass first (chunks c0 + lane + 64m), then the fma chains in chunk order
        uint4 w[EPW][ROUTER_MAXC], xv[TPW][ROUTER_MAXC];
#pragma unroll
        for (int m = 0; m < ROUTER_MAXC; ++m) {
            const int c = min(c0 + lane + 64 * m, nchunk - 1);
#pragma unroll
            for (int q = 0; q < EPW; ++q) w[q][m] = reinterpret_cast<const uint4*>(wrow[q])[c];
#pragma unroll
            for (int i = 0; i < TPW; ++i)
                xv[i][m] = reinterpret_cast<const uint4*>(a.x + (size_t)(t0 + min(i, nt - 1)) * d)[c];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < ROUTER_MAXC; ++m) {
            if (c0 + lane + 64 * m < nchunk) {
#pragma unroll
                for (int q = 0; q < EPW; ++q) {
                    const uint32_t ww[4] = {w[q][m].x, w[q][m].y, w[q][m].z, w[q][m].w};
#pragma unroll
                    for (int i = 0; i < TPW; ++i) {
                        const uint32_t xx[4] = {xv[i][m].x, xv[i][m].y, xv[i][m].z, xv[i][m].w};
                        float s = acc[q][i];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            s = __builtin_fmaf(bf16lo(xx[r]), bf16lo(ww[r]), s);
                            s = __builtin_fmaf(bf16hi(xx[r]), bf16hi(ww[r]), s);
                        }
                        acc[q][i] = s;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < EPW; ++q)
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            float s = sum_lanes<64>(acc[q][i]);   // lanes 48..63 hold the total
            const int e = e0 + q;
            if (lane == 63 && i < nt && e < rows) {
                if (a.bias && e < a.E) s = s + a.bias[e];
                a.logits[(size_t)(t0 + i) * rows + e] = s;
            }
        }
}

// The rest of the router, on the logits of the previous launch (its kernel boundary makes them visible): one wave per
// token, FIN_TOK tokens per workgroup of FIN_WAVES waves, so the tails (a chain of DPP reductions, VALU-issue bound)
// run one wave per SIMD on ceil(T / FIN_TOK) CUs, and the grouping has all FIN_WAVES waves of the last workgroup.
// A wave runs its token's tail, writes idx / wts and, with shared experts, the merged slot list (the S shared experts
// last, weight sigmoid(gate logit) or 1). With a.grp.counts the slots are then grouped (group_block: the counts'
// offsets from a wave prefix sum) and the pass lists written by the last workgroup to finish: the ids pass from the
// other workgroups by agent-scope stores and loads, and the arrival counter is a.grp.meta[0], zeroed by the logits
// launch and overwritten by the grouping's own meta[0]. a.mw: the ids and the per-wave count arrays fit the LDS;
// otherwise wave 0 places every slot.
constexpr int FIN_WAVES = 16;   // waves per workgroup: all of them group the slots in the last workgroup
constexpr int FIN_TOK = 4;      // tokens per workgroup: waves 0..3, one per SIMD, run the tails
template <int JM>
__global__ void __launch_bounds__(64 * FIN_WAVES) route_finish(RouterArgs a) {
    extern __shared__ int32_t sm[];   // grouping: cnt[FIN_WAVES][E + S], ids[T (k + S)] (mw); else cnt, cursor
    __shared__ int s_last;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int k = a.k, ws = a.k + a.S, Eg = a.E + a.S;
    const bool grouping = a.grp.counts != nullptr;
    const int nwg = (a.T + FIN_TOK - 1) / FIN_TOK;   // the grid (from T, not gridDim: no hidden-argument load)
    const bool single = nwg == 1;
    int32_t* ids = a.S ? a.sidx : a.idx;   // the list the grouping reads
    const int t = blockIdx.x * FIN_TOK + wave;
    if (wave < FIN_TOK && t < a.T) {
        const float* lrow = a.logits + (size_t)t * a.lstride;
        float v[JM];
#pragma unroll
        for (int j = 0; j < JM; ++j) v[j] = j * 64 + lane < a.E ? lrow[j * 64 + lane] : -INFINITY;
        const float gl = a.gate ? lrow[a.E] : 0.f;
        uint32_t id;
        float w;
        topk_core<JM>(v, a.E, k, a.norm, a.scale, k, &id, &w);
        int32_t sid = (int32_t)id;
        if (a.S && lane >= k) sid = a.E + lane - k;
        if (lane < k) {
            if (a.S) a.idx[(size_t)t * k + lane] = sid;
            a.wts[(size_t)t * k + lane] = w;
        }
        if (lane < ws) {
            if (a.S) a.swts[(size_t)t * ws + lane] = lane < k ? w : (a.gate ? 1.f / (1.f + expf(-gl)) : 1.f);
            if (grouping && !single) store_agent(&ids[(size_t)t * ws + lane], sid);
            else ids[(size_t)t * ws + lane] = sid;
        }
    }
    if (a.xterm) {
        // x's 2-term fp8 records for the block-scaled MXFP4 tiles (what k_mx_terms writes), for this workgroup's
        // tokens: one thread per 32-input block, numbered from wave FIN_TOK on, so that the waves that ran the
        // tails take blocks only when there are more blocks than the other waves' threads
        const int nsl = (a.d + 127) >> 7, t0 = blockIdx.x * FIN_TOK;
        const int rows = a.T - t0 < FIN_TOK ? a.T - t0 : FIN_TOK;
        const int i0 = ((int)threadIdx.x + 64 * (FIN_WAVES - FIN_TOK)) % (64 * FIN_WAVES);
        for (int i = i0; i < rows * 4 * nsl; i += 64 * FIN_WAVES)
            mx_terms_block<2>(a.x + (size_t)t0 * a.d, rows, a.d, a.xterm + (size_t)t0 * nsl * mx_rec<2>(), i);
    }
    if (!grouping) return;
    const int n = a.T * ws;
    if (single) {   // this workgroup wrote every id (the barrier orders its stores before the loads)
        __syncthreads();
        group_block([&](int p) { return ids[p]; }, n, Eg, a.grp, a.P, a.P2, sm, a.mw);
        return;
    }
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(&a.grp.meta[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (old == nwg - 1);
    }
    __syncthreads();
    if (!s_last) return;
    group_block([&](int p) { return load_agent(ids + p); }, n, Eg, a.grp, a.P, a.P2, sm, a.mw);
}

// Router tail on given logits [T, E] (fp32, bf16 or fp16): one wave per token.
template <typename LT>
__global__ void __launch_bounds__(256)
topk_kernel(const LT* __restrict__ logits, int T, int E, int lstride, int k, int norm, float scale,
            int32_t* __restrict__ idx, float* __restrict__ wts) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    const LT* lrow = logits + (size_t)t * lstride;
    wave_topk([&](int ee) { return to_f32<LT>(lrow[ee]); }, E, k, norm, scale, idx + (size_t)t * k,
              wts + (size_t)t * k);
}

// Stable slot grouping by expert in a launch of its own (group_block): one block.
__global__ void __launch_bounds__(1024)
group_slots(const int32_t* __restrict__ idx, int n, int E, GroupBufs o, int P, int P2, int mw) {
    extern __shared__ int32_t sm[];
    group_block([&](int p) { return idx[p]; }, n, E, o, P, P2, sm, mw);
}

// shared experts: token t's slot list is its k routed slots (copied from ridx / rwts [T, k]; none when k = 0)
// followed by S shared slots, expert E0 + s with weight g_t = sigmoid(x_t . gate) or 1, written as idx / wts
// [T, k + S] (k + S <= 64). One wave per token: lane l dots the 8-element chunks l, l + 64, ... in element
// order, the lane sums are added as the DPP tree of sum_lanes<64>, lanes 48..63 hold the total.
__global__ void __launch_bounds__(256)
shared_route(const void* __restrict__ x, int xdt, const uint16_t* __restrict__ gate, int T, int d, int S, int k,
             int E0, const int32_t* __restrict__ ridx, const float* __restrict__ rwts, int32_t* __restrict__ idx,
             float* __restrict__ wts) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + wave;
    if (t >= T) return;
    float g = 1.f;
    if (gate) {
        float acc = 0.f;
        for (int c = lane; c < (d >> 3); c += 64) {
            float xv[8];   // x of any of the three dtypes, as fp32 (exact)
            if (xdt == MOE_DTYPE_F32) {
                const float4* xr = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + (size_t)t * d);
                const float4 a = xr[2 * c], b = xr[2 * c + 1];
                xv[0] = a.x, xv[1] = a.y, xv[2] = a.z, xv[3] = a.w, xv[4] = b.x, xv[5] = b.y, xv[6] = b.z, xv[7] = b.w;
            } else {
                const uint4 r = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + (size_t)t * d)[c];
                const uint32_t xw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    xv[2 * i] = xdt == MOE_DTYPE_F16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)(xw[i] & 0xFFFFu))
                                                     : bf16lo(xw[i]);
                    xv[2 * i + 1] = xdt == MOE_DTYPE_F16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)(xw[i] >> 16))
                                                         : bf16hi(xw[i]);
                }
            }
            const uint4 gv = *reinterpret_cast<const uint4*>(gate + 8 * c);
            const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc = __builtin_fmaf(xv[2 * i], bf16lo(gw[i]), acc);
                acc = __builtin_fmaf(xv[2 * i + 1], bf16hi(gw[i]), acc);
            }
        }
        acc = sum_lanes<64>(acc);
        acc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 63));
        g = 1.f / (1.f + expf(-acc));
    }
    const int w = k + S;
    if (lane < k) {   // routed ids outside [0, E0) join no group (E0 .. E0 + S - 1 are the shared experts)
        const int id = ridx[(size_t)t * k + lane];
        idx[(size_t)t * w + lane] = (unsigned)id < (unsigned)E0 ? id : -1;
        wts[(size_t)t * w + lane] = rwts[(size_t)t * k + lane];
    } else if (lane < w) {
        idx[(size_t)t * w + lane] = E0 + lane - k;
        wts[(size_t)t * w + lane] = g;
    }
}

// ------------------------------------------------------------------------------------ host launchers
// route_finish's grouping LDS (every workgroup of the launch reserves it; only the last uses it): the ids and the
// per-wave count arrays up to FIN_LDS, else the counts and cursors only, with wave 0 placing every slot.
constexpr size_t FIN_LDS = 32 * 1024;

// logits (T > 1: ROUTER_TPW tokens per wave share each loaded Wr chunk; T == 1: one expert per wave, fewer larger
// waves or one wave per workgroup spread over E CUs measured no faster)
int launch_route_logits(const RouterArgs& a, hipStream_t st) {
    const dim3 grid((a.lstride + ROUTER_WAVES - 1) / ROUTER_WAVES, a.T == 1 ? 1 : (a.T + ROUTER_TPW - 1) / ROUTER_TPW);
    if (a.T == 1) router_logits<1, 1><<<grid, 64 * ROUTER_WAVES, 0, st>>>(a);
    else router_logits<ROUTER_TPW, 1><<<grid, 64 * ROUTER_WAVES, 0, st>>>(a);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

int launch_route(RouterArgs a, bool tail, hipStream_t st) {
    const int nwg = (a.T + FIN_TOK - 1) / FIN_TOK;
    a.arrive = tail && a.grp.counts && nwg > 1 ? a.grp.meta : nullptr;
    if (a.grp.counts && ((a.grp.items && (a.P < 1 || (a.P & (a.P - 1)))) ||
                         (a.grp.items2 && (a.P2 < 1 || (a.P2 & (a.P2 - 1))))))
        return MOE_ERR_ARG;   // pass sizes are powers of two
    int rc = launch_route_logits(a, st);
    if (rc || !tail) return rc;
    size_t lds = 0;
    if (a.grp.counts) {
        const int n = a.T * (a.k + a.S), Eg = a.E + a.S;
        a.mw = (size_t)group_lds_ints(n, Eg, FIN_WAVES, 1) * 4 <= FIN_LDS;
        lds = (size_t)group_lds_ints(n, Eg, FIN_WAVES, a.mw) * 4;
    }
    const dim3 grid(nwg);
    if (a.E <= 64) route_finish<1><<<grid, 64 * FIN_WAVES, lds, st>>>(a);
    else if (a.E <= 128) route_finish<2><<<grid, 64 * FIN_WAVES, lds, st>>>(a);
    else if (a.E <= 256) route_finish<4><<<grid, 64 * FIN_WAVES, lds, st>>>(a);
    else route_finish<TOPK_MAX_J><<<grid, 64 * FIN_WAVES, lds, st>>>(a);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

int launch_router(const uint16_t* x, const uint16_t* wr, const float* bias, int T, int d, int E, int k, int norm,
                  float scale, float* logits, int32_t* idx, float* wts, hipStream_t st) {
    RouterArgs a{};
    a.x = x, a.wr = wr, a.bias = bias, a.T = T, a.d = d, a.E = E, a.k = k, a.norm = norm, a.scale = scale;
    a.logits = logits, a.lstride = E, a.idx = idx, a.wts = wts;
    return launch_route(a, true, st);
}

int launch_router_logits(const uint16_t* x, const uint16_t* wr, const float* bias, int T, int d, int E, float* logits,
                         hipStream_t st) {
    RouterArgs a{};
    a.x = x, a.wr = wr, a.bias = bias, a.T = T, a.d = d, a.E = E, a.k = 1, a.norm = 1, a.scale = 1.f;
    a.logits = logits, a.lstride = E;
    return launch_route_logits(a, st);
}

int launch_topk(const void* logits, int dtype, int T, int E, int k, int norm, float scale, int32_t* idx, float* wts,
                hipStream_t st, int lstride) {
    dim3 grid((T + 3) / 4);
    if (lstride < E) lstride = E;
    if (dtype == MOE_DTYPE_F32)
        topk_kernel<float><<<grid, 256, 0, st>>>((const float*)logits, T, E, lstride, k, norm, scale, idx, wts);
    else if (dtype == MOE_DTYPE_BF16)
        topk_kernel<uint16_t><<<grid, 256, 0, st>>>((const uint16_t*)logits, T, E, lstride, k, norm, scale, idx, wts);
    else if (dtype == MOE_DTYPE_F16)
        topk_kernel<_Float16><<<grid, 256, 0, st>>>((const _Float16*)logits, T, E, lstride, k, norm, scale, idx, wts);
    else
        return MOE_ERR_DTYPE;
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

int launch_shared_route(const void* x, int xdt, const uint16_t* gate, int T, int d, int S, int32_t* idx, float* wts,
                        hipStream_t st, int k, int E0, const int32_t* ridx, const float* rwts) {
    if (T <= 0) return 0;
    if (k < 0 || S < 0 || k + S > 64 || (k > 0 && (!ridx || !rwts))) return MOE_ERR_ARG;
    shared_route<<<(T + 3) / 4, 256, 0, st>>>(x, xdt, gate, T, d, S, k, E0, ridx, rwts, idx, wts);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

int launch_group(const int32_t* idx, int n, int E, int32_t* counts, int32_t* offsets, int32_t* sorted,
                 int32_t* active, int32_t* meta, hipStream_t st, int P, int32_t* items, int P2, int32_t* items2) {
    if ((items && (P < 1 || (P & (P - 1)))) || (items2 && (P2 < 1 || (P2 & (P2 - 1))))) return MOE_ERR_ARG;
    // one block: 16 waves (1024 threads) each placing a sixteenth of the slots from 1024 slots, else 4 waves; the
    // per-wave counts and the ids in LDS (at most 64 KB), else wave 0 places all of them
    int nw = n >= 1024 ? 16 : 4;
    if ((size_t)group_lds_ints(n, E, nw, 1) * 4 > 64 * 1024) nw = 4;
    const int mw = (size_t)group_lds_ints(n, E, nw, 1) * 4 <= 64 * 1024 ? 1 : 0;
    const GroupBufs o{counts, offsets, sorted, active, meta, items, items2};
    group_slots<<<1, 64 * nw, (size_t)group_lds_ints(n, E, nw, mw) * 4, st>>>(idx, n, E, o, P, P2, mw);
    return hipGetLastError() == hipSuccess ? 0 : MOE_ERR_LAUNCH;
}

}  // namespace moe

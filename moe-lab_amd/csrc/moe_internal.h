// Internal launcher interface shared by the kernel translation units and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "moe_mi355x.h"

namespace moe {

// grouping scratch inside an experts workspace
struct GroupBufs {
    int32_t* counts;
    int32_t* offsets;
    int32_t* sorted;
    int32_t* active;
    int32_t* meta;    // [4]: active experts, bad ids, passes of the work list, passes of the second list
    int32_t* items;   // pass list, room for max_passes(n, E, 16) (expert, pass, passes) triples
    int32_t* items2;  // second pass list (dense down after wave gate/up), room for max_passes(n, E, 64)
};

// One router launch (moe_router.hip): the logits, then (tail) the top-k tail per token, the merged slot lists with
// shared experts, and the slot grouping.
// Field order: the logits launch's prologue reads the first 64-byte scalar-cache line only; the tail launch's
// (route_finish) reads the first two, then the grouping buffers in the third.
struct RouterArgs {
    const uint16_t* x;     // [T, d] bf16
    const uint16_t* wr;    // [E, d] bf16
    const uint16_t* gate;  // [d] bf16 or null: one more logit row (index E), the shared experts' gate
    float* logits;         // [T, lstride]
    int32_t* arrive;       // set by launch_route: the finishing workgroups' arrival counter, zeroed by the logits
    int T, d, E;
    int lstride;           // E, or E + 1 with the gate row
    const float* bias;     // [E] or null
    int k, norm;
    float scale;
    int S;                 // shared experts appended to every token's slots (0: none)
    int32_t* idx;          // [T, k] routed ids
    float* wts;            // [T, k] routed weights
    int32_t* sidx;         // S > 0: [T, k + S] the k routed ids, then E .. E + S - 1
    float* swts;           // S > 0: [T, k + S] the routed weights, then sigmoid(gate logit) or 1
    int mw;                // set by launch_route
    int P;                 // pass size of grp.items (unused when null)
    GroupBufs grp;         // grp.counts null: no grouping; else the grouping of the slots (sidx when S > 0, else idx)
    int P2;                // pass size of grp.items2
    uint8_t* xterm;        // or null: route_finish also writes x's 2-term fp8 records here (the block-scaled MXFP4
                           // tiles' activations, as k_mx_terms would), so the experts call launches no k_mx_terms
};
// The router's launches: the logits over many workgroups, then (tail) route_finish: the tails, the merged lists and the
// grouping (grp.counts) and pass lists. tail = false: logits only.
int launch_route(RouterArgs a, bool tail, hipStream_t st);
int launch_router(const uint16_t* x, const uint16_t* wr, const float* bias, int T, int d, int E, int k, int norm,
                  float scale, float* logits, int32_t* idx, float* wts, hipStream_t st);
// logits only (x . wr^T + bias in the router's fixed order), no tail
int launch_router_logits(const uint16_t* x, const uint16_t* wr, const float* bias, int T, int d, int E, float* logits,
                         hipStream_t st);
// lstride: elements between logit rows (0: E)
int launch_topk(const void* logits, int dtype, int T, int E, int k, int norm, float scale, int32_t* idx, float* wts,
                hipStream_t st, int lstride = 0);
// with items: also the grouped kernels' pass list for passes of P slots (items [3 * max_passes(n, E, P)], meta[2])
int launch_group(const int32_t* idx, int n, int E, int32_t* counts, int32_t* offsets, int32_t* sorted,
                 int32_t* active, int32_t* meta, hipStream_t st, int P = 0, int32_t* items = nullptr, int P2 = 0,
                 int32_t* items2 = nullptr);
// tuning and test knobs from the environment, read per call
inline int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v ? atoi(v) : dflt;
}
// upper bound of the pass count: sum over experts of ceil(count / P) <= n / P + (experts with a count)
inline int max_passes(int n, int E, int P) { return (n + P - 1) / P + (n < E ? n : E); }
int launch_shared_route(const void* x, int xdt, const uint16_t* gate, int T, int d, int S, int32_t* idx, float* wts,
                        hipStream_t st, int k = 0, int E0 = 0, const int32_t* ridx = nullptr, const float* rwts = nullptr);

// The grouped path's pass sizes for a call (the same choice run_experts_tiles makes): P the gate/up list's, P2 the
// down list's when it differs (else 0); ingroup: the wave tiles group the slots in-kernel (no list needed).
struct TilePasses {
    int P, P2, ingroup;
    int mx;   // the call runs the block-scaled MXFP4 tiles, which read x as 2-term fp8 records (xterm)
};
TilePasses tile_passes(const moe_experts_t* w, int T, int k, int x_dtype);

struct ExpertsArgs {
    const moe_experts_t* w;
    const void* x;
    int x_dtype;
    const int32_t* idx;
    const float* wts;
    int T, k, act, nored;
    const uint16_t* xb;   // x as bf16 planes: x itself (bf16, nx = 1) or k_x_planes' planes of fp16 / fp32 x
    int nx;               // 1, 2 (fp16) or 3 (fp32)
    size_t xplane;        // elements between planes (T * d)
    void* y;              // [T, d] (or [T*k, d] when nored), of dtype ydt
    int ydt;              // MOE_DTYPE_BF16, MOE_DTYPE_F16 or MOE_DTYPE_F32
    const void* residual; // same dtype as y, or NULL
    uint16_t* hhi;        // GLU output h = hi + lo, two bf16 planes [T*k, F] (per-slot rows path with h_is_f16: one fp16 plane in hhi)
    uint16_t* hlo;
    float* yp;      // 4 x [T*k, d] fp32 scratch (grouped path; the further planes for a K-split down projection)
    uint16_t* x16;  // grouped path, dense int4: x as fp16 [T, d] with a power-of-two exponent per token
    int32_t* xexp;  // [T]
    uint8_t* xterm; // grouped path, MXFP4 block-scaled MFMA: x's fp8 term records (the x-planes region when x is bf16)
    GroupBufs grp;  // grouped path
    int pregrouped; // grouped path: grp already holds the grouping and pass lists of idx (written by the router)
    int xterm_ready; // grouped path: xterm already holds x's term records (written by the router)
    int stages;     // bit 0: grouping + gate/up (writes h), bit 1: down + combine (reads h)
    // moe_layer_run at T == 1: the gate/up waves take their experts from the top-k of these router logits [T, E] (and
    // write idx / wts, which the down kernel reads); null: idx / wts are inputs
    const float* route_logits;
    int route_norm;
    float route_scale;
    hipStream_t st;
};

// expert kernels, both formats (moe_experts.hip)
int run_experts_slots(const ExpertsArgs& a);
// whether the per-slot gate/up takes its experts from router logits (ExpertsArgs::route_logits) at this (k, F)
bool slots_route_in_gate_up(int k, int F);
// grouped expert tiles on MFMA (moe_tiles.hip): grouping, gate/up + GLU, down, combine
int run_experts_tiles(const ExpertsArgs& a);
// rows -> tile-major records (moe_tiles.hip; layout in include/moe_mi355x.h)
int launch_pack_tiles(int fmt, int E, int N, int K, const void* rows, void* tiles, hipStream_t st);
// combine (moe_experts.hip): y[t] = residual[t] + sum_j wts[t*k + j] * (sum over the nplanes planes of yp[t*k + j]
// + bd[idx[t*k + j]])
int launch_combine(const float* yp, int nplanes, size_t plane, const int32_t* idx, const float* wts, const float* bd, int E,
                   const void* residual, void* y, int T, int k, int d, int ydt, hipStream_t st);
// guard probe (moe_probe.hip): XOR-fold a stream of 16-byte loads over nbytes into sink[MOE_PROBE_SINK]
int launch_probe_read(const void* src, size_t nbytes, uint32_t* sink, hipStream_t st);
// fp16 / fp32 activations x [T, d] -> bf16 planes [2 or 3][T, d] whose sum is x exactly (moe_experts.hip)
int launch_x_planes(const void* x, int xdt, int T, int d, uint16_t* planes, hipStream_t st);

}  // namespace moe

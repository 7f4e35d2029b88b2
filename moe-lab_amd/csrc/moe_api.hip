// C ABI of libmoe_mi355x.so (declarations and contract in include/moe_mi355x.h).
// Validates arguments before any launch, carves the caller's workspace and dispatches to the kernels.
#include <stdint.h>

#include <mutex>

#include "moe_formats.h"
#include "moe_internal.h"

// Workspace of moe_experts_run_static: a file-scope device array, one copy per GPU the library runs on (held until
// the process ends). Host code never passes its name to a kernel or a copy: the name is a host-side stand-in, and
// the array's device address on each GPU comes from hipGetSymbolAddress (static_scratch below).
static __device__ __align__(256) uint8_t scratch[MOE_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// the device address of `scratch` on the device the stream belongs to (the current device for the null stream),
// looked up on the first call there with that device current, then kept: the library's one table of mutable state
int static_scratch(hipStream_t st, void** out) {
    int dev = -1;
    if (st ? hipStreamGetDevice(st, &dev) != hipSuccess : hipGetDevice(&dev) != hipSuccess) return MOE_ERR_LAUNCH;
    if (dev < 0 || dev >= kMaxDevices) return MOE_ERR_ARG;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess) return MOE_ERR_LAUNCH;
        if (cur != dev && hipSetDevice(dev) != hipSuccess) return MOE_ERR_LAUNCH;
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev && hipSetDevice(cur) != hipSuccess) return MOE_ERR_LAUNCH;
        if (e != hipSuccess || !p) return MOE_ERR_LAUNCH;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MOE_OK;
}

constexpr size_t kAlign = 256;
inline size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int resolve_path(int path, int T) {
    if (path == MOE_PATH_AUTO) return T == 1 ? MOE_PATH_SLOTS : MOE_PATH_GROUPED;
    return path;
}

struct Layout {
    size_t h, xp, yp, x16, xexp, counts, offsets, sorted, active, meta, items, items2, total;
};

Layout layout(const moe_experts_t* w, int T, int k, int path) {
    Layout L{};
    const size_t nslots = (size_t)T * k;
    size_t off = 0;
    L.h = off;
    off += align_up(nslots * (size_t)w->F * 2) * 2;   // hi and lo planes
    L.xp = off;                                       // fp16 / fp32 x as up to 3 bf16 planes
    off += align_up((size_t)3 * T * w->d * 2);
    if (resolve_path(path, T) == MOE_PATH_GROUPED) {
        L.yp = off;
        off += align_up(nslots * (size_t)w->d * 4 * 4);   // four planes: the dense down projection may split K
        L.x16 = off;
        off += align_up((size_t)T * w->d * 2);
        L.xexp = off;
        off += align_up((size_t)T * 4);
        L.counts = off;
        off += align_up((size_t)w->E * 4);
        L.offsets = off;
        off += align_up((size_t)(w->E + 1) * 4);
        L.sorted = off;
        off += align_up(nslots * 4);
        L.active = off;
        off += align_up((size_t)w->E * 4);
        L.meta = off;
        off += align_up(4 * 4);
        L.items = off;
        off += align_up((size_t)moe::max_passes((int)nslots, w->E, 16) * 12);
        L.items2 = off;   // the dense down's list when the gate/up runs the wave tiles (64-token passes)
        off += align_up((size_t)moe::max_passes((int)nslots, w->E, 64) * 12);
    }
    L.total = off;
    return L;
}

int check_proj(const moe_proj_t& p) {
    if (!p.rows) return MOE_ERR_ARG;
    if (!aligned16(p.rows) || (p.tiles && !aligned16(p.tiles))) return MOE_ERR_ALIGN;
    return MOE_OK;
}

int check_experts(const moe_experts_t* w) {
    if (!w) return MOE_ERR_ARG;
    if (w->fmt != MOE_FMT_INT4_G64 && w->fmt != MOE_FMT_MXFP4) return MOE_ERR_DTYPE;
    if (w->E < 1 || w->d < 1 || w->F < 1) return MOE_ERR_ARG;
    const int g = w->fmt == MOE_FMT_INT4_G64 ? 64 : 32;
    if (w->d % 64 || w->F % 64 || w->d % g || w->F % g || w->F > 16384) return MOE_ERR_ARG;
    int rc;
    if ((rc = check_proj(w->gate)) || (rc = check_proj(w->up)) || (rc = check_proj(w->down))) return rc;
    return MOE_OK;
}

}  // namespace

extern "C" {

const char* moe_version(void) { return "moe_mi355x 0.3 (gfx950, wave64)"; }

int moe_probe_read(const void* src, size_t nbytes, uint32_t* sink, void* stream) {
    if (!src || !sink || nbytes < 16 || nbytes % 16) return MOE_ERR_ARG;
    if (!aligned16(src)) return MOE_ERR_ALIGN;
    return moe::launch_probe_read(src, nbytes, sink, (hipStream_t)stream);
}

size_t moe_row_bytes(int fmt, int K) {
    if (K < 64 || K % 64) return 0;
    if (fmt == MOE_FMT_INT4_G64) return ((size_t)K / 2 + (size_t)K / 16 + 15) & ~(size_t)15;
    if (fmt == MOE_FMT_MXFP4) return ((size_t)K / 2 + (size_t)K / 32 + 15) & ~(size_t)15;
    return 0;
}

size_t moe_tile_bytes(int fmt, int N, int K) {
    if ((fmt != MOE_FMT_INT4_G64 && fmt != MOE_FMT_MXFP4) || N < 16 || N % 16 || K < 64 || K % 64) return 0;
    return moe::tile_bytes(fmt, N, K);
}

int moe_tiles_pack(int fmt, int E, int N, int K, const void* rows, void* tiles, void* stream) {
    if (fmt != MOE_FMT_INT4_G64 && fmt != MOE_FMT_MXFP4) return MOE_ERR_DTYPE;
    if (E < 1 || N < 16 || N % 16 || K < 64 || K % 64 || N > 65535 * 16 || E > 65535 || (long)E * N > 0x7FFFFFFFL)
        return MOE_ERR_ARG;
    if (!rows || !tiles) return MOE_ERR_ARG;
    if (!aligned16(rows) || !aligned16(tiles)) return MOE_ERR_ALIGN;
    return moe::launch_pack_tiles(fmt, E, N, K, rows, tiles, (hipStream_t)stream);
}

// the router keeps no counters (its launches hand data over at kernel boundaries only): one int32, never read
int moe_router_counter_count(int T) { return T < 0 ? 0 : 1; }

int moe_router(const void* x, const void* wr, const float* bias, int T, int d, int E, int k, int norm, float scale,
               float* logits, int32_t* idx, float* wts, int32_t* counters, void* stream) {
    if (T < 0 || d < 8 || d % 8 || E < 1 || E > 1024 || k < 1 || k > E || k > 32) return MOE_ERR_ARG;
    if (T == 0) return MOE_OK;
    (void)counters;   // kept for ABI compatibility: the router hands data over at kernel boundaries only
    if (!x || !wr || !logits || !idx || !wts) return MOE_ERR_ARG;
    if (!aligned16(x) || !aligned16(wr)) return MOE_ERR_ALIGN;
    return moe::launch_router((const uint16_t*)x, (const uint16_t*)wr, bias, T, d, E, k, norm, scale, logits, idx, wts,
                              (hipStream_t)stream);
}

int moe_router_group(const void* x, const void* wr, const float* bias, int T, int d, int E, int k, int norm,
                     float scale, float* logits, int32_t* idx, float* wts, int32_t* counts, int32_t* offsets,
                     int32_t* sorted, int32_t* active, int32_t* meta, void* stream) {
    if (T < 0 || d < 8 || d % 8 || E < 1 || E > 1024 || k < 1 || k > E || k > 32) return MOE_ERR_ARG;
    if (T == 0) return MOE_OK;
    if (!x || !wr || !logits || !idx || !wts || !counts || !offsets || !sorted || !active || !meta) return MOE_ERR_ARG;
    if (!aligned16(x) || !aligned16(wr)) return MOE_ERR_ALIGN;
    moe::RouterArgs a{};
    a.x = (const uint16_t*)x, a.wr = (const uint16_t*)wr, a.bias = bias, a.T = T, a.d = d, a.E = E, a.k = k;
    a.norm = norm, a.scale = scale, a.logits = logits, a.lstride = E, a.idx = idx, a.wts = wts;
    a.grp = moe::GroupBufs{counts, offsets, sorted, active, meta, nullptr, nullptr};
    return moe::launch_route(a, true, (hipStream_t)stream);
}

int moe_topk(const void* logits, int dtype, int T, int E, int k, int norm, float scale, int32_t* idx, float* wts,
             void* stream) {
    if (T < 0 || E < 1 || E > 1024 || k < 1 || k > E || k > 32) return MOE_ERR_ARG;
    if (T == 0) return MOE_OK;
    if (!logits || !idx || !wts) return MOE_ERR_ARG;
    return moe::launch_topk(logits, dtype, T, E, k, norm, scale, idx, wts, (hipStream_t)stream);
}

int moe_group(const int32_t* idx, int n, int E, int32_t* counts, int32_t* offsets, int32_t* sorted, int32_t* active,
              int32_t* meta, void* stream) {
    if (n < 0 || E < 1 || E > 8192) return MOE_ERR_ARG;
    if (!counts || !offsets || !active || !meta || (n > 0 && (!idx || !sorted))) return MOE_ERR_ARG;
    return moe::launch_group(idx, n, E, counts, offsets, sorted, active, meta, (hipStream_t)stream);
}

size_t moe_experts_workspace_bytes(const moe_experts_t* w, int T, int k, int path) {
    if (!w || T < 0 || k < 1) return 0;
    return layout(w, T, k, path).total;
}

size_t moe_shared_experts_workspace_bytes(const moe_experts_t* ws, int T) {
    if (!ws || T < 0 || ws->E < 1) return 0;
    const size_t n = (size_t)T * ws->E;
    return layout(ws, T, ws->E, MOE_PATH_AUTO).total + 2 * align_up(n * 4);
}

int moe_shared_experts_run(const moe_experts_t* ws, const void* x, int x_dtype, int T, int act, const void* gate,
                           void* y, int y_dtype, const void* residual, void* workspace, size_t workspace_bytes,
                           void* stream) {
    int rc = check_experts(ws);
    if (rc) return rc;
    if (ws->E > 32 || T < 0) return MOE_ERR_ARG;
    if (T == 0) return MOE_OK;
    if (!x || !y || !workspace) return x && y ? MOE_ERR_WORKSPACE : MOE_ERR_ARG;
    if (x_dtype < MOE_DTYPE_BF16 || x_dtype > MOE_DTYPE_F32) return MOE_ERR_DTYPE;
    if (!aligned16(x) || (gate && !aligned16(gate)) || !aligned16(workspace)) return MOE_ERR_ALIGN;
    const size_t base = layout(ws, T, ws->E, MOE_PATH_AUTO).total;
    if (workspace_bytes < moe_shared_experts_workspace_bytes(ws, T)) return MOE_ERR_WORKSPACE;
    const size_t n = (size_t)T * ws->E;
    int32_t* idx = (int32_t*)((char*)workspace + base);
    float* wts = (float*)((char*)workspace + base + align_up(n * 4));
    rc = moe::launch_shared_route(x, x_dtype, (const uint16_t*)gate, T, ws->d, ws->E, idx, wts, (hipStream_t)stream);
    if (rc) return rc;
    return moe_experts_run_stages(ws, x, x_dtype, idx, wts, T, ws->E, act, MOE_PATH_AUTO, 0, y, y_dtype, residual,
                                  workspace, base, MOE_STAGE_ALL, stream);
}

size_t moe_experts_shared_workspace_bytes(const moe_experts_t* w, int S, int T, int k, int path) {
    if (!w || T < 0 || k < 1 || S < 1 || k + S > 64) return 0;
    const size_t n = (size_t)T * (k + S);
    return layout(w, T, k + S, path).total + 2 * align_up(n * 4);
}

// routed + shared in one call: the slot lists [T, k + S] (routed ids outside [0, E - S) become -1, so they join no
// group as in moe_experts_run), then the expert call on them
int moe_experts_run_shared(const moe_experts_t* w, int S, const void* x, int x_dtype, const int32_t* idx,
                           const float* wts, int T, int k, int act, int path, const void* gate, void* y, int y_dtype,
                           const void* residual, void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_experts(w);
    if (rc) return rc;
    if (S < 1 || k < 1 || k + S > 64 || S >= w->E || T < 0 || path < MOE_PATH_AUTO || path > MOE_PATH_GROUPED)
        return MOE_ERR_ARG;
    if (T == 0) return MOE_OK;
    if (!x || !y || !idx || !wts) return MOE_ERR_ARG;
    if (!workspace) return MOE_ERR_WORKSPACE;
    if (x_dtype < MOE_DTYPE_BF16 || x_dtype > MOE_DTYPE_F32) return MOE_ERR_DTYPE;
    if (!aligned16(x) || (gate && !aligned16(gate)) || !aligned16(workspace)) return MOE_ERR_ALIGN;
    if (workspace_bytes < moe_experts_shared_workspace_bytes(w, S, T, k, path)) return MOE_ERR_WORKSPACE;
    const size_t base = layout(w, T, k + S, path).total;
    const size_t n = (size_t)T * (k + S);
    int32_t* idx2 = (int32_t*)((char*)workspace + base);
    float* wts2 = (float*)((char*)workspace + base + align_up(n * 4));
    rc = moe::launch_shared_route(x, x_dtype, (const uint16_t*)gate, T, w->d, S, idx2, wts2, (hipStream_t)stream, k,
                                  w->E - S, idx, wts);
    if (rc) return rc;
    return moe_experts_run_stages(w, x, x_dtype, idx2, wts2, T, k + S, act, path, 0, y, y_dtype, residual, workspace,
                                  base, MOE_STAGE_ALL, stream);
}

int moe_experts_run(const moe_experts_t* w, const void* x, int x_dtype, const int32_t* idx, const float* wts, int T,
                    int k, int act, int path, int nored, void* y, int y_dtype, const void* residual, void* workspace,
                    size_t workspace_bytes, void* stream) {
    return moe_experts_run_stages(w, x, x_dtype, idx, wts, T, k, act, path, nored, y, y_dtype, residual, workspace,
                                  workspace_bytes, MOE_STAGE_ALL, stream);
}

int moe_experts_run_static(const moe_experts_t* w, const void* x, int x_dtype, const int32_t* idx, const float* wts,
                           int T, int k, int act, int path, int nored, void* y, int y_dtype, const void* residual,
                           void* stream) {
    void* ws = nullptr;
    int rc = static_scratch((hipStream_t)stream, &ws);   // first call on a device: the lookup; then a table read
    if (rc) return rc;
    if (T == 0) return MOE_OK;
    if (!w || T < 0 || k < 1) return MOE_ERR_ARG;
    if (moe_experts_workspace_bytes(w, T, k, path) > MOE_STATIC_SCRATCH_BYTES) return MOE_ERR_WORKSPACE;
    return moe_experts_run_stages(w, x, x_dtype, idx, wts, T, k, act, path, nored, y, y_dtype, residual, ws,
                                  MOE_STATIC_SCRATCH_BYTES, MOE_STAGE_ALL, stream);
}

namespace {
int experts_call(const moe_experts_t* w, const void* x, int x_dtype, const int32_t* idx, const float* wts, int T, int k,
                 int act, int path, int nored, void* y, int y_dtype, const void* residual, void* workspace,
                 size_t workspace_bytes, int stages, void* stream, const float* route_logits, int route_norm,
                 float route_scale, int pregrouped = 0, int xterm_ready = 0);
int layer_call(const moe_experts_t* w, int S, const void* x, int x_dtype, const void* wr, const float* wr_bias,
               const void* gate, int T, int k, int norm, float scale, int act, int32_t* idx, float* wts, void* y,
               int y_dtype, const void* residual, void* workspace, size_t workspace_bytes, void* stream);
}  // namespace

size_t moe_layer_workspace_bytes(const moe_experts_t* w, int T, int k) {
    if (!w || T < 0 || k < 1 || w->E < 1) return 0;
    return layout(w, T, k, MOE_PATH_AUTO).total + align_up((size_t)T * w->E * 4);   // + the router logits
}

size_t moe_layer_shared_workspace_bytes(const moe_experts_t* w, int S, int T, int k) {
    if (!w || T < 0 || k < 1 || S < 1 || S >= w->E || k + S > 64) return 0;
    const size_t n = (size_t)T * (k + S);
    // the experts' workspace for k + S slots, the router logits with the gate row, the merged slot lists
    return layout(w, T, k + S, MOE_PATH_AUTO).total + align_up((size_t)T * (w->E - S + 1) * 4) + 2 * align_up(n * 4);
}

int moe_layer_run(const moe_experts_t* w, const void* x, int x_dtype, const void* wr, const float* wr_bias, int T,
                  int k, int norm, float scale, int act, int32_t* idx, float* wts, void* y, int y_dtype,
                  const void* residual, void* workspace, size_t workspace_bytes, void* stream) {
    return layer_call(w, 0, x, x_dtype, wr, wr_bias, nullptr, T, k, norm, scale, act, idx, wts, y, y_dtype, residual,
                      workspace, workspace_bytes, stream);
}

int moe_layer_run_shared(const moe_experts_t* w, int S, const void* x, int x_dtype, const void* wr,
                         const float* wr_bias, const void* gate, int T, int k, int norm, float scale, int act,
                         int32_t* idx, float* wts, void* y, int y_dtype, const void* residual, void* workspace,
                         size_t workspace_bytes, void* stream) {
    if (S < 1) return MOE_ERR_ARG;
    return layer_call(w, S, x, x_dtype, wr, wr_bias, gate, T, k, norm, scale, act, idx, wts, y, y_dtype, residual,
                      workspace, workspace_bytes, stream);
}

int moe_experts_run_stages(const moe_experts_t* w, const void* x, int x_dtype, const int32_t* idx, const float* wts,
                           int T, int k, int act, int path, int nored, void* y, int y_dtype, const void* residual,
                           void* workspace, size_t workspace_bytes, int stages, void* stream) {
    return experts_call(w, x, x_dtype, idx, wts, T, k, act, path, nored, y, y_dtype, residual, workspace,
                        workspace_bytes, stages, stream, nullptr, 1, 1.f);
}

}  // extern "C"

namespace {
int experts_call(const moe_experts_t* w, const void* x, int x_dtype, const int32_t* idx, const float* wts, int T, int k,
                 int act, int path, int nored, void* y, int y_dtype, const void* residual, void* workspace,
                 size_t workspace_bytes, int stages, void* stream, const float* route_logits, int route_norm,
                 float route_scale, int pregrouped, int xterm_ready) {
    if (stages < 1 || stages > MOE_STAGE_ALL) return MOE_ERR_ARG;
    int rc = check_experts(w);
    if (rc) return rc;
    if (T < 0 || k < 1 || act < 0 || act > 2 || path < 0 || path > 2) return MOE_ERR_ARG;
    if (x_dtype < MOE_DTYPE_BF16 || x_dtype > MOE_DTYPE_F32) return MOE_ERR_DTYPE;
    if (y_dtype < MOE_DTYPE_BF16 || y_dtype > MOE_DTYPE_F32) return MOE_ERR_DTYPE;
    const int rpath = resolve_path(path, T);
    if (nored && (rpath != MOE_PATH_SLOTS || residual)) return MOE_ERR_ARG;
    if (T == 0) return MOE_OK;
    if (!x || !idx || !wts || !y) return MOE_ERR_ARG;
    if (!aligned16(x) || !aligned16(y) || (residual && !aligned16(residual))) return MOE_ERR_ALIGN;
    const Layout L = layout(w, T, k, path);
    if (!workspace || workspace_bytes < L.total) return MOE_ERR_WORKSPACE;
    if (!aligned16(workspace)) return MOE_ERR_ALIGN;
    char* ws = (char*)workspace;
    moe::ExpertsArgs a{};
    a.w = w;
    a.x = x;
    a.x_dtype = x_dtype;
    a.idx = idx;
    a.wts = wts;
    a.T = T;
    a.k = k;
    a.act = act;
    a.nored = nored;
    a.y = y;
    a.ydt = y_dtype;
    if (x_dtype == MOE_DTYPE_BF16) {
        a.xb = (const uint16_t*)x;
        a.nx = 1;
    } else {   // fp16 / fp32: the gate/up stage reads x as 2 / 3 bf16 planes (exact)
        a.xb = (const uint16_t*)(ws + L.xp);
        a.nx = x_dtype == MOE_DTYPE_F16 ? 2 : 3;
        a.xplane = (size_t)T * w->d;
        if (stages & MOE_STAGE_GATE_UP) {
            const int rc2 = moe::launch_x_planes(x, x_dtype, T, w->d, (uint16_t*)(ws + L.xp), (hipStream_t)stream);
            if (rc2) return rc2;
        }
    }
    a.residual = residual;
    a.hhi = (uint16_t*)(ws + L.h);
    a.hlo = a.hhi + align_up((size_t)T * k * w->F * 2) / 2;
    a.st = (hipStream_t)stream;
    a.stages = stages;
    a.route_logits = route_logits;
    a.route_norm = route_norm;
    a.route_scale = route_scale;
    if (rpath == MOE_PATH_GROUPED) {
        a.yp = (float*)(ws + L.yp);
        a.x16 = (uint16_t*)(ws + L.x16);
        a.xexp = (int32_t*)(ws + L.xexp);
        a.xterm = x_dtype == MOE_DTYPE_BF16 ? (uint8_t*)(ws + L.xp) : nullptr;
        a.grp.counts = (int32_t*)(ws + L.counts);
        a.grp.offsets = (int32_t*)(ws + L.offsets);
        a.grp.sorted = (int32_t*)(ws + L.sorted);
        a.grp.active = (int32_t*)(ws + L.active);
        a.grp.meta = (int32_t*)(ws + L.meta);
        a.grp.items = (int32_t*)(ws + L.items);
        a.grp.items2 = (int32_t*)(ws + L.items2);
        a.pregrouped = pregrouped;
        a.xterm_ready = a.xterm ? xterm_ready : 0;
    }
    return rpath == MOE_PATH_GROUPED ? moe::run_experts_tiles(a) : moe::run_experts_slots(a);
}


// Router and experts of one layer (S > 0: w's last S experts are shared ones, appended to every token's slots).
// T == 1 (no shared experts, k and F the per-slot gate/up can route at): a logits-only router launch, the tail in the
// gate/up waves. Otherwise the router's two launches compute the logits and the tails and write the merged slot lists
// (S > 0); on the grouped path they also build the grouping and the pass lists the expert kernels read, unless the
// gate/up wave tiles group the slots in-kernel (a few slots per expert: one of their workgroups then writes the lists
// for the down stage, which measured ~4 us faster at Qwen3 T=32 than the router's last workgroup grouping them;
// MOE_LAYER_INGROUP=0 makes the router group them there too). No top-k or grouping launch of its own either way.
int layer_call(const moe_experts_t* w, int S, const void* x, int x_dtype, const void* wr, const float* wr_bias,
               const void* gate, int T, int k, int norm, float scale, int act, int32_t* idx, float* wts, void* y,
               int y_dtype, const void* residual, void* workspace, size_t workspace_bytes, void* stream) {
    int rc = check_experts(w);
    if (rc) return rc;
    const int Er = w->E - S;   // routed experts
    if (T < 0 || S < 0 || Er < 1 || k < 1 || k > Er || k > 32 || Er > 1024 || k + S > 64 || act < 0 || act > 2)
        return MOE_ERR_ARG;
    if (S == 0 && gate) return MOE_ERR_ARG;
    if (x_dtype != MOE_DTYPE_BF16) return MOE_ERR_DTYPE;   // the router GEMV reads bf16 x
    if (y_dtype < MOE_DTYPE_BF16 || y_dtype > MOE_DTYPE_F32) return MOE_ERR_DTYPE;
    if (T == 0) return MOE_OK;
    if (!x || !wr || !idx || !wts || !y) return MOE_ERR_ARG;
    if (!aligned16(x) || !aligned16(wr) || !aligned16(y) || (residual && !aligned16(residual)) ||
        (gate && !aligned16(gate)))
        return MOE_ERR_ALIGN;
    const size_t need = S ? moe_layer_shared_workspace_bytes(w, S, T, k) : moe_layer_workspace_bytes(w, T, k);
    if (!workspace || workspace_bytes < need) return MOE_ERR_WORKSPACE;
    if (!aligned16(workspace)) return MOE_ERR_ALIGN;
    const int ks = k + S;   // slots per token
    const Layout L = layout(w, T, ks, MOE_PATH_AUTO);
    char* ws = (char*)workspace;
    hipStream_t st = (hipStream_t)stream;
    moe::RouterArgs ra{};
    ra.x = (const uint16_t*)x, ra.wr = (const uint16_t*)wr, ra.bias = wr_bias, ra.gate = (const uint16_t*)gate;
    ra.T = T, ra.d = w->d, ra.E = Er, ra.k = k, ra.norm = norm, ra.scale = scale;
    ra.logits = (float*)(ws + L.total), ra.lstride = Er + (gate ? 1 : 0);
    ra.idx = idx, ra.wts = wts, ra.S = S;
    const int32_t* eidx = idx;   // the slot lists the experts read
    const float* ewts = wts;
    if (S) {
        ra.sidx = (int32_t*)(ws + L.total + align_up((size_t)T * (Er + 1) * 4));
        ra.swts = (float*)((char*)ra.sidx + align_up((size_t)T * ks * 4));
        eidx = ra.sidx, ewts = ra.swts;
    }
    if (T == 1 && S == 0 && moe::slots_route_in_gate_up(k, w->F)) {   // the gate/up waves run the tail themselves
        rc = moe::launch_route(ra, false, st);
        if (rc) return rc;
        return experts_call(w, x, x_dtype, idx, wts, T, k, act, MOE_PATH_AUTO, 0, y, y_dtype, residual, workspace,
                            L.total, MOE_STAGE_ALL, stream, ra.logits, norm, scale);
    }
    int pregrouped = 0, xterm_ready = 0;
    if (resolve_path(MOE_PATH_AUTO, T) == MOE_PATH_GROUPED) {
        const moe::TilePasses tp = moe::tile_passes(w, T, ks, x_dtype);
        if (tp.mx) {   // the block-scaled MXFP4 tiles: the finishing launch also writes x's term records
            ra.xterm = (uint8_t*)(ws + L.xp);
            xterm_ready = 1;
        }
        if (!(tp.ingroup && moe::env_int("MOE_LAYER_INGROUP", 1))) {
            ra.grp = moe::GroupBufs{(int32_t*)(ws + L.counts), (int32_t*)(ws + L.offsets), (int32_t*)(ws + L.sorted),
                                    (int32_t*)(ws + L.active), (int32_t*)(ws + L.meta), (int32_t*)(ws + L.items),
                                    tp.P2 ? (int32_t*)(ws + L.items2) : nullptr};
            ra.P = tp.P, ra.P2 = tp.P2;
            pregrouped = 1;
        }
    }
    rc = moe::launch_route(ra, true, st);
    if (rc) return rc;
    return experts_call(w, x, x_dtype, eidx, ewts, T, ks, act, MOE_PATH_AUTO, 0, y, y_dtype, residual, workspace,
                        L.total, MOE_STAGE_ALL, stream, nullptr, 1, 1.f, pregrouped, xterm_ready);
}

}  // namespace

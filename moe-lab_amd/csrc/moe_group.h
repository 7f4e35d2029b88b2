// Stable slot grouping by one workgroup (group_block): used by the router's finishing launch, the grouping launch
// and the gate/up wave tiles that group their slots in-kernel (one of their workgroups also writes the lists).
#pragma once
#include "moe_common.h"
#include "moe_internal.h"

namespace moe {

// Stable slot grouping by one block (blockDim.x a multiple of 64). ld(p) yields the expert id of slot p = t*k + j;
// ids outside [0, E) are left out of every group (they contribute nothing) and counted in meta[1].
// Outputs (o): counts[E], offsets[E+1], sorted[n] (valid part: offsets[E] entries), active[E] (first meta[0]
// entries: experts with count > 0, ascending), meta[0] = number of active experts, meta[1] = bad ids.
// With o.items (the grouped kernels' work list, pass size P, a power of two): items[3w .. 3w + 2] = (expert, pass
// index q within the expert (first token q * P), the expert's pass count) of pass w; the passes of each active expert
// in ascending order, expert by expert; meta[2] = number of passes. o.items2 (pass size P2), if given, is a second
// such list, meta[3] its number of passes (the wave tiles' and the dense tiles' lists when a call uses both).
// sm: dynamic LDS of group_lds_ints(n, E, NW, mw) ints. mw (the ids and one count array per wave fit there): the ids
// are read once into LDS, and each wave places one contiguous share of the slots with its own cursors (the expert's
// offset plus the counts of the shares before it), so the order stays ascending within every expert. Otherwise wave 0
// places all slots. The offsets come from a two-level prefix sum: chunk ch of 64 experts belongs to wave ch % NW,
// which scans it in-wave (DPP) and leaves its totals in LDS; after a barrier every wave adds the earlier chunks'
// totals to its own.
__host__ __device__ inline int group_lds_ints(int n, int E, int nw, int mw) {
    return (mw ? nw * E + n : 2 * E) + 4 * ((E + 63) / 64);
}

template <typename LD>
__device__ void group_block(LD ld, int n, int E, const GroupBufs& o, int P, int P2, int32_t* sm, int mw) {
    const int NT = (int)blockDim.x, NWT = NT >> 6;
    const int NW = mw ? NWT : 1;
    int32_t* cnt = sm;            // mw: cnt[NW][E], ids[n]; else cnt[E], cursor[E]; then the chunk totals
    int32_t* cur1 = sm + E;
    int32_t* sidx = sm + NW * E;
    int32_t* tot = sm + (mw ? NW * E + n : 2 * E);   // [nch][4]: slots, active experts, passes, passes of list 2
    __shared__ int32_t s_bad;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int nch = (E + 63) >> 6;
    const int lgP = o.items ? __builtin_ctz((unsigned)P) : 0, lgP2 = o.items2 ? __builtin_ctz((unsigned)P2) : 0;
    for (int i = tid; i < NW * E; i += NT) cnt[i] = 0;
    if (tid == 0) s_bad = 0;
    __syncthreads();
    const int q4 = (n + NW - 1) / NW;   // mw: wave w takes slots [w q4, (w + 1) q4)
    // ids are read GB per lane at a time (one memory round trip per batch, not one per id)
    constexpr int GB = 8;
    if (mw) {
        const int b0 = wave * q4, b1 = b0 + q4 < n ? b0 + q4 : n;
        for (int base = b0; base < b1; base += 64 * GB) {
            int ev[GB];
#pragma unroll
            for (int j = 0; j < GB; ++j) {
                const int p = base + 64 * j + lane;
                ev[j] = p < b1 ? ld(p) : 0;
            }
#pragma unroll
            for (int j = 0; j < GB; ++j) {
                const int p = base + 64 * j + lane;
                if (p < b1) {
                    sidx[p] = ev[j];
                    if (ev[j] >= 0 && ev[j] < E) atomicAdd(&cnt[wave * E + ev[j]], 1);
                    else atomicAdd(&s_bad, 1);
                }
            }
        }
    } else {
        for (int base = 0; base < n; base += NT * GB) {
            int ev[GB];
#pragma unroll
            for (int j = 0; j < GB; ++j) {
                const int p = base + NT * j + tid;
                ev[j] = p < n ? ld(p) : 0;
            }
#pragma unroll
            for (int j = 0; j < GB; ++j) {
                const int p = base + NT * j + tid;
                if (p < n) {
                    if (ev[j] >= 0 && ev[j] < E) atomicAdd(&cnt[ev[j]], 1);
                    else atomicAdd(&s_bad, 1);
                }
            }
        }
    }
    __syncthreads();
    // chunk ch's counts: expert e = 64 ch + lane, summed over the per-wave count arrays
    auto chunk = [&](int ch, int& c, int& np, int& np2) __attribute__((always_inline)) {
        const int e = 64 * ch + lane;
        c = 0;
        if (e < E)
            for (int w = 0; w < NW; ++w) c += cnt[w * E + e];
        np = o.items ? (c + P - 1) >> lgP : 0;      // passes of expert e
        np2 = o.items2 ? (c + P2 - 1) >> lgP2 : 0;  // in the second list
    };
    for (int ch = wave; ch < nch; ch += NWT) {   // level 1: each chunk's totals
        int c, np, np2;
        chunk(ch, c, np, np2);
        const int t0 = wave_incl_scan(c), t1 = wave_incl_scan(c > 0 ? 1 : 0);
        const int t2 = wave_incl_scan(np), t3 = wave_incl_scan(np2);
        if (lane == 63) {
            tot[4 * ch] = t0;
            tot[4 * ch + 1] = t1;
            tot[4 * ch + 2] = t2;
            tot[4 * ch + 3] = t3;
        }
    }
    __syncthreads();
    int all_act = 0;
    for (int ch = 0; ch < nch; ++ch) all_act += tot[4 * ch + 1];
    for (int ch = wave; ch < nch; ch += NWT) {   // level 2: the earlier chunks' totals, then this chunk's outputs
        int run = 0, run_act = 0, run_p = 0, run_p2 = 0;
        for (int c2 = 0; c2 < ch; ++c2) {
            run += tot[4 * c2];
            run_act += tot[4 * c2 + 1];
            run_p += tot[4 * c2 + 2];
            run_p2 += tot[4 * c2 + 3];
        }
        int c, np, np2;
        chunk(ch, c, np, np2);
        const int inc = wave_incl_scan(c), act = wave_incl_scan(c > 0 ? 1 : 0);
        const int incp = wave_incl_scan(np), incp2 = wave_incl_scan(np2);
        const int e = 64 * ch + lane;
        if (e < E) {
            const int excl = run + inc - c;
            o.offsets[e] = excl;
            o.counts[e] = c;
            if (mw) {   // per-wave cursors: the earlier waves' slots come first
                int cc = excl;
                for (int w = 0; w < NW; ++w) {
                    const int cw = cnt[w * E + e];
                    cnt[w * E + e] = cc;
                    cc += cw;
                }
            } else {
                cur1[e] = excl;
            }
            if (c > 0) o.active[run_act + act - 1] = e;
            const int w0 = run_p + incp - np;
            for (int q = 0; q < np; ++q) {
                o.items[3 * (w0 + q)] = e;
                o.items[3 * (w0 + q) + 1] = q;
                o.items[3 * (w0 + q) + 2] = np;
            }
            const int w2 = run_p2 + incp2 - np2;
            for (int q = 0; q < np2; ++q) {
                o.items2[3 * (w2 + q)] = e;
                o.items2[3 * (w2 + q) + 1] = q;
                o.items2[3 * (w2 + q) + 2] = np2;
            }
        }
        if (ch == nch - 1 && lane == 63) {
            o.offsets[E] = run + inc;
            o.meta[0] = run_act + act;
            o.meta[1] = s_bad;
            if (o.items) o.meta[2] = run_p + incp;
            if (o.items2) o.meta[3] = run_p2 + incp2;
        }
    }
    for (int i = all_act + tid; i < E; i += NT) o.active[i] = -1;
    __syncthreads();
    if (mw || tid < 64) {   // stable placement, 64 slots per step in ascending order
        int32_t* cursor = mw ? cnt + wave * E : cur1;
        const int b0 = mw ? wave * q4 : 0;
        const int b1 = mw ? (b0 + q4 < n ? b0 + q4 : n) : n;
        int nbits = 0;
        while ((1 << nbits) < E) ++nbits;
        const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        int ev[GB];
        for (int base = b0; base < b1; base += 64) {
            const int j = ((base - b0) >> 6) % GB;
            if (j == 0) {   // the next GB steps' ids
#pragma unroll
                for (int i = 0; i < GB; ++i) {
                    const int q = base + 64 * i + lane;
                    ev[i] = q < b1 ? (mw ? sidx[q] : ld(q)) : -1;
                }
            }
            const int p = base + lane;
            int e = -1;
#pragma unroll
            for (int i = 0; i < GB; ++i)
                if (i == j) e = ev[i];
            const bool ok = (e >= 0 && e < E);
            // lanes holding the same valid expert: match on every bit of e
            uint64_t peers = __ballot(ok);
            for (int b = 0; b < nbits; ++b) {
                const bool bit = ok && ((e >> b) & 1);
                const uint64_t m = __ballot(bit);
                peers &= bit ? m : ~m;
            }
            int pos = 0;
            if (ok) pos = cursor[e] + __popcll(peers & lt_mask);
            __builtin_amdgcn_wave_barrier();
            if (ok) {
                o.sorted[pos] = p;
                if ((peers & lt_mask) == 0ull) cursor[e] += __popcll(peers);   // lowest lane of the group
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
}

}  // namespace moe

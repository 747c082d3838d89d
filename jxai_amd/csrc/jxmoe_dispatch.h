// Top-k selection and the token -> expert dispatch tables for few-token
// routing, shared by the router kernels and the decode GEMVs that group their
// own work from the router logits.
#pragma once

#include "jxmoe_device.h"
#include "jxmoe_kernels.h"

namespace jx {

constexpr int MAX_E = 512;
constexpr int MAX_K = 32;

// Selection order of select_experts_cache_aware (src/tier.cpp:144-146):
// descending logit; exact ties are ordered by expert index (the reference's
// std::sort leaves them unspecified).  NaN ranks as -inf, so the order is
// total and every token selects exactly k experts.
__device__ __forceinline__ float rank_key(float l) { return l != l ? -__builtin_inff() : l; }
__device__ __forceinline__ int ranks_above(float lf, int f, float le, int e) {
    return (lf > le) || (lf == le && f < e);
}

// Top-k + softmax (select_experts_cache_aware, src/tier.cpp:144-188) and the
// dispatch for n <= ROUTE_SMALL_MAX_N tokens, by one block of NTH threads:
// lgs holds the [n][E] logits in LDS (reused for the histogram), shl the raw
// shared-gate logit of each token (null: no shared gate).
template <int NTH>
__device__ void topk_dispatch_small(const RouteArgs& a, const DispatchOut& o, float* lgs, const float* shl,
                                    int (*rank_sel)[MAX_K], int tid) {
    const int n = a.n, E = a.E, k = a.k;
    if (tid < n * MAX_K) rank_sel[tid / MAX_K][tid % MAX_K] = tid % MAX_K;  // valid default slots
    __syncthreads();
    for (int i = tid; i < n * E; i += NTH) {
        const int t = i / E, e = i % E;
        const float* lt = lgs + (size_t)t * E;
        const float le = rank_key(lt[e]);
        int rank = 0;
        for (int f = 0; f < E; ++f) rank += ranks_above(rank_key(lt[f]), f, le, e);
        if (rank < k) rank_sel[t][rank] = e;
    }
    __syncthreads();
    if (tid < n) {
        const int t = tid;
        const float* lt = lgs + (size_t)t * E;
        float p[MAX_K];
        float mx = lt[rank_sel[t][0]];
        for (int i = 1; i < k; ++i) mx = fmaxf(mx, lt[rank_sel[t][i]]);
        float sum = 0.0f;
        for (int i = 0; i < k; ++i) {
            p[i] = expf(lt[rank_sel[t][i]] - mx);
            sum += p[i];
        }
        const float inv = (sum > 0.0f) ? 1.0f / sum : 1.0f / (float)k;
        for (int i = 0; i < k; ++i) {
            a.ids[(size_t)t * k + i] = rank_sel[t][i];
            a.probs[(size_t)t * k + i] = p[i] * inv;
        }
        if (a.shscale) a.shscale[t] = shl ? 1.0f / (1.0f + expf(-shl[t])) : 1.0f;
    }
    __syncthreads();
    // ---- dispatch (stable counting sort over the n*k pairs); the serial part
    // keeps every value it re-reads in LDS (a global read-back would cost an
    // L2 round trip per expert)
    int* hist = reinterpret_cast<int*>(lgs);  // [E] counts, then [E] running offsets
    int* pos = hist + E;
    for (int e = tid; e < E; e += NTH) hist[e] = 0;
    __syncthreads();
    if (tid == 0) {
        const int nk = n * k;
        for (int f = 0; f < nk; ++f) hist[rank_sel[f / k][f % k]]++;
        int off = 0, na = 0, nt = 0;
        for (int e = 0; e < E; ++e) {
            const int c = hist[e];
            pos[e] = off;
            if (c > 0) {
                o.act[na] = e;
                // first pair of an active expert is its smallest flat index
                int f0 = 0;
                while (rank_sel[f0 / k][f0 % k] != e) ++f0;
                o.slots[na] = make_int4(e, off, c, f0 / k);
                ++na;
                for (int i = 0; i * MFMA_BN < c; ++i)
                    o.tiles[nt++] = make_int4(e, off + i * MFMA_BN, min(MFMA_BN, c - i * MFMA_BN), 0);
            }
            off += c;
        }
        o.offs[E] = off;
        *o.n_act = na;
        *o.n_tiles = nt;
        for (int s2 = na; s2 < E; ++s2) o.slots[s2] = make_int4(0, 0, 0, 0);
        for (int f = 0; f < nk; ++f) {
            const int e = rank_sel[f / k][f % k];
            const int p = pos[e]++;
            o.pair_tok[p] = f / k;
            o.pos_of[f] = p;
        }
    }
    __syncthreads();
    for (int e = tid; e < E; e += NTH) {  // counts and offsets, written in parallel
        o.counts[e] = hist[e];
        o.offs[e] = pos[e] - hist[e];
    }
}

// Group of decode slot `slot` for n <= ROUTE_SMALL_MAX_N tokens and
// E <= SMALL_GROUP_MAX_E experts, recomputed by one wave (all 64 lanes) from
// the router logits: the same (expert, first pair, pair count, first token)
// record that topk_dispatch_small stores in o.slots -- active experts in
// increasing id, pairs ordered by (expert, token).
__device__ __forceinline__ int4 small_group(const Groups& g, int slot) {
    const int lane = threadIdx.x & 63, E = g.n_experts, k = g.top_k;
    uint64_t m[ROUTE_SMALL_MAX_N];
#pragma unroll
    for (int t = 0; t < ROUTE_SMALL_MAX_N; ++t) {
        m[t] = 0;
        if (t < g.n_tok) {
            const float l = rank_key(lane < E ? g.logits[(size_t)t * E + lane] : 0.0f);
            int rank = 0;
            for (int f = 0; f < E; ++f)
                rank += ranks_above(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), f)), f, l, lane);
            m[t] = __ballot(lane < E && rank < k);
        }
    }
    uint64_t any = 0;
#pragma unroll
    for (int t = 0; t < ROUTE_SMALL_MAX_N; ++t) any |= m[t];
    for (int s = 0; s < slot && any; ++s) any &= any - 1;
    if (!any) return make_int4(0, 0, 0, 0);
    const int e = __builtin_ctzll(any);
    const uint64_t below = (1ull << e) - 1ull;
    int cnt = 0, p0 = 0, first = -1;
#pragma unroll
    for (int t = 0; t < ROUTE_SMALL_MAX_N; ++t) {
        const int hit = (int)((m[t] >> e) & 1ull);
        cnt += hit;
        p0 += __popcll(m[t] & below);
        if (hit && first < 0) first = t;
    }
    return make_int4(e, p0, cnt, first);
}

}  // namespace jx

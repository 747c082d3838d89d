// Top-k selection and the token -> expert dispatch tables for few-token
// routing, shared by the router kernels and the decode GEMVs that group their
// own work from the router logits.
#pragma once

#include "jxmoe_device.h"
#include "jxmoe_kernels.h"

namespace jx {

constexpr int MAX_E = 512;
constexpr int MAX_K = 32;

// Q8_0 of one 32-block held one value per lane of a half-wave
// (quantize_row_q8_0, src/quant.cpp:1029-1045): amax, d = amax/127 (IEEE
// division), id = 1/d, q = clamp(round-half-away(x*id)), stored scale =
// truncated fp16 of d, and the block sum of q (for the Q4_0 -8 offset and the
// K-quant min terms).  Returns the lane's q; sv = (stored scale, sum).
__device__ __forceinline__ int q8_block_vals(float v, float2& sv) {
    const float amax = wave_max32(__builtin_fabsf(v));
    const float dd = amax / 127.0f;
    const float id = (dd != 0.0f) ? 1.0f / dd : 0.0f;
    float r = round_away(v * id);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    const int q = (int)r;
    sv = make_float2(f16_to_f32(f32_to_f16_trunc(dd)), (float)wave_sum32i(q));
    return q;
}

// Chain-major rows: element 16 i + j of a row at j * S + i, so lane j of a
// vec_dot_f32 chain reads its operands four at a time.  In LDS the stride is
// padded to a multiple of 4 floats plus 4 against bank conflicts; the router
// copy in global memory (chain_rows) uses the bare multiple of 4, and each
// lane's run of steps then sits in a few L1 lines it revisits (measured
// faster than interleaving the 16 chains for contiguous group loads).
__host__ __device__ constexpr int rs_stride(int d) { return ((d / 16 + 3) & ~3) + 4; }
__host__ __device__ constexpr int chain_stride_of(int d) { return (d / 16 + 3) & ~3; }

// Lane j (0..15) of one router row's chain group against one token, both
// chain-major in LDS with stride S: vec_dot_f32's fp32 FMA chain over elements
// 16 i + j (src/quant.cpp:2756-2778).  c8: an F16 / BF16 router row, whose
// dots (src/quant.cpp:3015-3055) run 8 chains over 8-element steps, i.e.
// chain-major columns jc and jc + 8 interleaved step by step (lanes 8-15
// repeat lanes 0-7).  d % 16 == 0.
__device__ __forceinline__ float chain_dot_lds(const float* w, const float* x, int S, int d, int j, bool c8) {
    const int jc = c8 ? (j & 7) : j;
    const float* wr = w + jc * S;
    const float* xr = x + jc * S;
    const int m = d / 16, m4 = m & ~3;
    float acc = 0.0f;
    if (c8) {
        for (int i = 0; i < m4; i += 4) {
            const float4 p = *reinterpret_cast<const float4*>(wr + i);
            const float4 p8 = *reinterpret_cast<const float4*>(wr + 8 * S + i);
            const float4 q = *reinterpret_cast<const float4*>(xr + i);
            const float4 q8 = *reinterpret_cast<const float4*>(xr + 8 * S + i);
            acc = __builtin_fmaf(p.x, q.x, acc);
            acc = __builtin_fmaf(p8.x, q8.x, acc);
            acc = __builtin_fmaf(p.y, q.y, acc);
            acc = __builtin_fmaf(p8.y, q8.y, acc);
            acc = __builtin_fmaf(p.z, q.z, acc);
            acc = __builtin_fmaf(p8.z, q8.z, acc);
            acc = __builtin_fmaf(p.w, q.w, acc);
            acc = __builtin_fmaf(p8.w, q8.w, acc);
        }
        for (int i = m4; i < m; ++i) {
            acc = __builtin_fmaf(wr[i], xr[i], acc);
            acc = __builtin_fmaf(wr[8 * S + i], xr[8 * S + i], acc);
        }
    } else {
#pragma unroll 8
        for (int i = 0; i < m4; i += 4) {
            const float4 p = *reinterpret_cast<const float4*>(wr + i);
            const float4 q = *reinterpret_cast<const float4*>(xr + i);
            acc = __builtin_fmaf(p.x, q.x, acc);
            acc = __builtin_fmaf(p.y, q.y, acc);
            acc = __builtin_fmaf(p.z, q.z, acc);
            acc = __builtin_fmaf(p.w, q.w, acc);
        }
        for (int i = m4; i < m; ++i) acc = __builtin_fmaf(wr[i], xr[i], acc);
    }
    return acc;
}

// The end of a 16-lane router chain group: vec_dot_f32 (src/quant.cpp:2756-2778) adds lane j + 8
// (the reference's acc1) to lane j < 8 (acc0), then sums lanes 0..7 in order from zero; the F16 /
// BF16 dots (src/quant.cpp:3015-3055) have the 8 lanes only.
__device__ __forceinline__ float chain_sum(float acc, bool c8) {
    const float hi = __shfl_down(acc, 8, 16);
    const float v = c8 ? acc : acc + hi;
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) s += __shfl(v, q, 16);
    return s;
}

// Selection order of select_experts_cache_aware (src/tier.cpp:144-146):
// descending logit; exact ties are ordered by expert index (the reference's
// std::sort leaves them unspecified).  NaN ranks as -inf, so the order is
// total and every token selects exactly k experts.
__device__ __forceinline__ float rank_key(float l) { return l != l ? -__builtin_inff() : l; }
__device__ __forceinline__ int ranks_above(float lf, int f, float le, int e) {
    return (lf > le) || (lf == le && f < e);
}

// Rank of expert e among the E logits lt (LDS): the number ordered before it.
// Unrolled so the LDS loads issue back to back instead of one round trip each.
__device__ __forceinline__ int rank_of(const float* lt, int E, int e) {
    const float le = rank_key(lt[e]);
    int rank = 0;
#pragma unroll 16
    for (int f = 0; f < E; ++f) rank += ranks_above(rank_key(lt[f]), f, le, e);
    return rank;
}

// Softmax over the k selected logits lt[sel[0..k)] of one token
// (select_experts_cache_aware, src/tier.cpp:144-188), by the 32 lanes of a
// half-wave, lane i for selection i (every lane of the half calls it): the
// max (order-free, NaN ignored as fmaxf does), one exponential per lane, their
// sum in selection order as the reference adds them, the weights.
__device__ inline void softmax_selected(const float* lt, const int* sel, int k, int i, int* ids, float* probs) {
    const bool v = i < k;
    const float l = v ? lt[sel[i]] : -__builtin_inff();
    float mx = l;
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 32));
    const float p = expf(l - mx);
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < MAX_K; ++q) {
        const float pq = __shfl(p, q, 32);
        if (q < k) sum += pq;
    }
    const float inv = (sum > 0.0f) ? 1.0f / sum : 1.0f / (float)k;
    if (v) {
        ids[i] = sel[i];
        probs[i] = p * inv;
    }
}

// Selection key of (rank key k, expert e) as one unsigned 64-bit value:
// larger is selected first (logit descending, then index ascending); 0 is
// below every expert.  The float maps to an order-preserving integer, -0 as
// +0 so that equal logits compare equal and fall to the index.
__device__ __forceinline__ uint64_t sel_key(float k, int e) {
    uint32_t u = __float_as_uint(k + 0.0f);
    u ^= (u >> 31) ? 0xFFFFFFFFu : 0x80000000u;
    return ((uint64_t)u << 32) | (uint32_t)(0xFFFF - e);
}
__device__ __forceinline__ int sel_expert(uint64_t key) { return 0xFFFF - (int)(key & 0xFFFFu); }

// One step of a wave max over 64-bit keys through a DPP lane move: lanes
// outside the row mask (or without a source) keep their own value.
template <int CTRL, int RM>
__device__ __forceinline__ uint64_t max_dpp(uint64_t x) {
    const int lo = (int)(uint32_t)x, hi = (int)(uint32_t)(x >> 32);
    const uint32_t lo2 = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, RM, 0xF, false);
    const uint32_t hi2 = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, RM, 0xF, false);
    const uint64_t y = ((uint64_t)hi2 << 32) | lo2;
    return y > x ? y : x;
}

// Wave-uniform maximum of one key per lane, branch-free: quad swaps, half-row
// and row mirrors (every lane of a 16-lane row holds the row maximum), then
// row broadcasts 15 and 31 fold the rows into lane 63.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t x) {
    x = max_dpp<0xB1, 0xF>(x);   // quad_perm [1,0,3,2]
    x = max_dpp<0x4E, 0xF>(x);   // quad_perm [2,3,0,1]
    x = max_dpp<0x141, 0xF>(x);  // row_half_mirror
    x = max_dpp<0x140, 0xF>(x);  // row_mirror
    x = max_dpp<0x142, 0xA>(x);  // row_bcast:15 into rows 1 and 3
    x = max_dpp<0x143, 0xC>(x);  // row_bcast:31 into rows 2 and 3
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}

// Top-k + softmax of one token (select_experts_cache_aware,
// src/tier.cpp:144-188) by ONE wave (all 64 lanes), NC = ceil(E / 64) <=
// MAX_E / 64 expert chunks; lt: the token's E logits (global or LDS), shl:
// its raw shared-gate logit (null: no shared gate).  k rounds of the wave
// argmax (order: logit descending, index ascending, NaN as -inf) give the
// selection in rank order; the softmax folds the max and the sum in that
// order as the reference does.  Writes ids, probs (a.ids non-null) and the
// shared-gate scale (a.shscale non-null) of token t; returns the selection mask
// and, on lane r < k, the expert of rank r (and in *myprob its weight).
template <int NC>
__device__ __forceinline__ int topk_token_wave(const RouteArgs& a, const float* lt, size_t t, const float* shl,
                                               uint64_t (&msk)[NC], float* myprob = nullptr) {
    static_assert(NC * 64 <= MAX_E, "expert chunks");
    constexpr float NEG = -__builtin_inff();
    const int lane = threadIdx.x & 63, E = a.E, k = a.k;
    float raw[NC], key[NC];
    uint32_t cand = 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int e = 64 * c + lane;
        raw[c] = e < E ? lt[e] : 0.0f;
        key[c] = e < E ? rank_key(raw[c]) : NEG;
        cand |= e < E ? 1u << c : 0u;
        msk[c] = 0;
    }
    float myl = 0.0f, mx = 0.0f;
    int myid = 0;
    for (int r = 0; r < k; ++r) {
        uint64_t best = 0;
#pragma unroll
        for (int c = 0; c < NC; ++c) {  // the lane's best remaining candidate
            const uint64_t kc = ((cand >> c) & 1u) ? sel_key(key[c], 64 * c + lane) : 0ull;
            best = kc > best ? kc : best;
        }
        const int bi = sel_expert(wave_max_key(best));
        const int bc = bi >> 6, bl = bi & 63;
        float rv = raw[0];
#pragma unroll
        for (int c = 1; c < NC; ++c) rv = c == bc ? raw[c] : rv;
        const float l = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rv), bl));
        mx = r == 0 ? l : fmaxf(mx, l);
#pragma unroll
        for (int c = 0; c < NC; ++c) msk[c] |= c == bc ? 1ull << bl : 0ull;
        cand &= lane == bl ? ~(1u << bc) : ~0u;
        myl = lane == r ? l : myl;
        myid = lane == r ? bi : myid;
    }
    const float p = expf(myl - mx);
    float sum = 0.0f;
    for (int r = 0; r < k; ++r) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), r));
    const float inv = (sum > 0.0f) ? 1.0f / sum : 1.0f / (float)k;
    if (lane < k && a.ids) {
        a.ids[t * k + lane] = myid;
        a.probs[t * k + lane] = p * inv;
    }
    if (myprob) *myprob = p * inv;
    if (lane == 0 && a.shscale) a.shscale[t] = shl ? 1.0f / (1.0f + expf(-shl[t])) : 1.0f;
    return myid;
}

// Top-k + softmax and the dispatch tables for n <= ROUTE_SMALL_MAX_N tokens,
// by ONE wave (all 64 lanes; no barriers, no LDS).  lg: the [n][E] logits,
// shl: raw shared-gate logit per token (null: no shared gate).  The tables
// follow from the selection masks: an expert's pair offset and active index
// are popcounts of the masks below it, pairs ordered by (expert, token).
template <int NC>
__device__ void topk_dispatch_wave(const RouteArgs& a, const DispatchOut& o, const float* lg, const float* shl) {
    static_assert(ROUTE_SMALL_MAX_N <= 2 && NC * 64 <= MAX_E, "few-token tables");
    const int lane = threadIdx.x & 63, n = a.n, E = a.E, k = a.k;
    uint64_t msk[ROUTE_SMALL_MAX_N][NC];
    int sid[ROUTE_SMALL_MAX_N];  // lane r < k: the expert of rank r of each token
#pragma unroll
    for (int t = 0; t < ROUTE_SMALL_MAX_N; ++t) {
        sid[t] = 0;
#pragma unroll
        for (int c = 0; c < NC; ++c) msk[t][c] = 0;
        if (t < n) sid[t] = topk_token_wave<NC>(a, lg + (size_t)t * E, (size_t)t, shl, msk[t]);  // uniform
    }
    // ---- dispatch from the masks
    const uint64_t below = (1ull << lane) - 1ull;
    int na_all = 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        uint64_t any = 0;
#pragma unroll
        for (int t = 0; t < ROUTE_SMALL_MAX_N; ++t) any |= msk[t][c];
        na_all += __popcll(any);
    }
    int pbase = 0, abase = 0;  // pairs and active experts in the chunks before
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int e = 64 * c + lane;
        const int h0 = (int)((msk[0][c] >> lane) & 1ull);
        const int h1 = ROUTE_SMALL_MAX_N > 1 ? (int)((msk[ROUTE_SMALL_MAX_N - 1][c] >> lane) & 1ull) : 0;
        uint64_t any = 0;
        int pc = 0, pb = 0;
#pragma unroll
        for (int t = 0; t < ROUTE_SMALL_MAX_N; ++t) {
            any |= msk[t][c];
            pc += __popcll(msk[t][c]);
            pb += __popcll(msk[t][c] & below);
        }
        const int cnt = h0 + h1, off = pbase + pb, na = abase + __popcll(any & below);
        if (e < E) {
            o.counts[e] = cnt;
            o.offs[e] = off;
            if (cnt > 0) {
                o.act[na] = e;
                o.slots[na] = make_int4(e, off, cnt, h0 ? 0 : 1);
                o.tiles[na] = make_int4(e, off, cnt, 0);  // cnt <= 2 <= MFMA_BN: one tile each
            } else {
                o.slots[na_all + (e - na)] = make_int4(0, 0, 0, 0);  // inactive experts fill slots n_act..E-1
            }
        }
        pbase += pc;
        abase += __popcll(any);
    }
    if (lane == 0) {
        o.offs[E] = pbase;
        *o.n_act = na_all;
        *o.n_tiles = na_all;
    }
    // pair positions: lane r of token t holds pair f = t * k + r
#pragma unroll
    for (int t = 0; t < ROUTE_SMALL_MAX_N; ++t) {
        if (t >= n || lane >= k) continue;
        const int e = sid[t];
        const int ec = e >> 6;
        const uint64_t eb = (1ull << (e & 63)) - 1ull;
        int p = 0, first_token_has = 0;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
#pragma unroll
            for (int u = 0; u < ROUTE_SMALL_MAX_N; ++u) {
                const uint64_t m = msk[u][c];
                p += c < ec ? __popcll(m) : (c == ec ? __popcll(m & eb) : 0);
                if (u < t && c == ec) first_token_has += (int)((m >> (e & 63)) & 1ull);
            }
        }
        p += first_token_has;  // the earlier token's pair of the same expert comes first
        o.pair_tok[p] = t;
        o.pos_of[(size_t)t * k + lane] = p;
    }
}

// Selected experts of token t as bit masks (sel[0]: experts 0-63, sel[1]: 64-127),
// by one wave (all 64 lanes) from the router logits.  Up to 16 experts: each
// lane ranks its own expert against every logit (rank < k selects it).  More:
// k rounds of a wave maximum over selection keys (logit descending, index
// ascending; NaN ranks as -inf), each lane holding experts lane and 64 + lane
// -- the same set as the ranks give.
__device__ __forceinline__ void small_selected(const Groups& g, int t, uint64_t sel[2]) {
    const int lane = threadIdx.x & 63, E = g.n_experts, k = g.top_k;
    const float* lt = g.logits + (size_t)t * E;
    sel[0] = sel[1] = 0;
    if (E <= 16) {
        const float l = rank_key(lane < E ? lt[lane] : 0.0f);
        int rank = 0;
        for (int f = 0; f < E; ++f)
            rank += ranks_above(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), f)), f, l, lane);
        sel[0] = __ballot(lane < E && rank < k);
        return;
    }
    const float a = lane < E ? rank_key(lt[lane]) : 0.0f;
    const float b = 64 + lane < E ? rank_key(lt[64 + lane]) : 0.0f;
    bool ca = lane < E, cb = 64 + lane < E;  // still candidates
    for (int r = 0; r < k; ++r) {
        const uint64_t ka = ca ? sel_key(a, lane) : 0ull, kb = cb ? sel_key(b, 64 + lane) : 0ull;
        const int bi = sel_expert(wave_max_key(ka > kb ? ka : kb));
        sel[0] |= bi < 64 ? 1ull << (bi & 63) : 0ull;
        sel[1] |= bi >= 64 ? 1ull << (bi & 63) : 0ull;
        ca = ca && lane != bi;
        cb = cb && lane + 64 != bi;
    }
}

// Group of decode slot `slot` for n <= ROUTE_SMALL_MAX_N tokens and
// E <= SMALL_GROUP_MAX_E experts, recomputed by one wave (all 64 lanes) from
// the router logits: the same (expert, first pair, pair count, first token)
// record that topk_dispatch_wave stores in o.slots -- active experts in
// increasing id, pairs ordered by (expert, token).
__device__ __forceinline__ int4 small_group(const Groups& g, int slot) {
    uint64_t m[ROUTE_SMALL_MAX_N][2];
#pragma unroll
    for (int t = 0; t < ROUTE_SMALL_MAX_N; ++t) {
        m[t][0] = m[t][1] = 0;
        if (t < g.n_tok) small_selected(g, t, m[t]);
    }
    uint64_t any0 = 0, any1 = 0;
#pragma unroll
    for (int t = 0; t < ROUTE_SMALL_MAX_N; ++t) {
        any0 |= m[t][0];
        any1 |= m[t][1];
    }
    int s = slot, e;
    if (s < __popcll(any0)) {
        for (; s > 0; --s) any0 &= any0 - 1;
        e = __builtin_ctzll(any0);
    } else {
        s -= __popcll(any0);
        if (s >= __popcll(any1)) return make_int4(0, 0, 0, 0);
        for (; s > 0; --s) any1 &= any1 - 1;
        e = 64 + __builtin_ctzll(any1);
    }
    const uint64_t below0 = e < 64 ? (1ull << e) - 1ull : ~0ull;
    const uint64_t below1 = e < 64 ? 0ull : (1ull << (e - 64)) - 1ull;
    int cnt = 0, p0 = 0, first = -1;
#pragma unroll
    for (int t = 0; t < ROUTE_SMALL_MAX_N; ++t) {
        const int hit = (int)((m[t][e >> 6] >> (e & 63)) & 1ull);
        cnt += hit;
        p0 += __popcll(m[t][0] & below0) + __popcll(m[t][1] & below1);
        if (hit && first < 0) first = t;
    }
    return make_int4(e, p0, cnt, first);
}

}  // namespace jx

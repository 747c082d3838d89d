// Routing side of the MoE expert path: router GEMV + top-k softmax + Q8_0
// activation quantization (one fused kernel), token->expert dispatch, the
// weighted combine, and the one-time weight repack.
#include <algorithm>

#include "jxmoe_device.h"
#include "jxmoe_dispatch.h"
#include "jxmoe_kernels.h"

namespace jx {

// Q8_0 of one 32-block held one value per lane of a half-wave (q8_block_vals),
// stored to o8 when ok: the int8 quants and (scale, block sum of q).  Returns q.
__device__ __forceinline__ int quant_block(float v, int l32, bool ok, const ActQ8& o8, size_t row, int b,
                                           float2* scale_out = nullptr) {
    float2 sv;
    const int q = q8_block_vals(v, sv);
    if (ok) {
        o8.q[row * o8.K + b * 32 + l32] = (int8_t)q;
        if (l32 == 0) {
            o8.s[row * (o8.K / 32) + b] = sv;
            if (scale_out) *scale_out = sv;
        }
    }
    return q;
}

// Matrix-core form (ActH) of one activation row from its Q8_0 quants q[K] and
// (scale, sum) per 32-block, written by the NTH threads of one block.  One
// exponent per row: E = exponent(max block scale of the row) - 7, so every
// dx * q * 2^-E (exact in fp32: an 11-bit scale times |q| <= 127) is below
// 2^15 and splits into fp16 hi + lo exactly (a block whose scale is 2^21
// times smaller than the row's largest loses bits of lo in fp16's subnormal
// range: at most 2^-25 absolute, 2^-40 of the row's largest value).  The Q4_K
// min-term values dx * sum(q) are stored times 2^-E as well; pe holds 2^E
// for every half-unit of the row.
// Row exponent of the matrix-core form from the row's largest block scale M.
__device__ __forceinline__ int acth_exponent(float M) {
    return (M > 0.0f) ? (int)((__float_as_uint(M) >> 23) & 0xFF) - 127 - 7 : 0;
}

// Exact bf16 (hi, mid, lo) pieces of an fp32 value (truncation keeps each
// remainder exact) at xm[0], xm[8], xm[16].
__device__ __forceinline__ void store_pieces3(uint16_t* xm, float X) {
    const uint32_t bh = __float_as_uint(X) & 0xFFFF0000u;
    const float r1 = X - __uint_as_float(bh);
    const uint32_t bm = __float_as_uint(r1) & 0xFFFF0000u;
    const float r2 = r1 - __uint_as_float(bm);
    xm[0] = (uint16_t)(bh >> 16);
    xm[8] = (uint16_t)(bm >> 16);
    xm[16] = (uint16_t)(__float_as_uint(r2) >> 16);
}

// Unit of the block-unit form after block b of a row with block scales
// sc[0..]: the last nonzero scale at or before b, 1 if there is none.
__device__ __forceinline__ float block_unit(const float2* sc, int b) {
    for (; b >= 0; --b) {
        const float d = sc[b].x;
        if (d != 0.0f) return d;
    }
    return 1.0f;
}

// Elements 8c .. 8c+7 of one row (all in one 32-block): for the hi/lo form
// one 16-byte store each of hi and lo, plus the row's pe entry and the
// block's min-term pieces when the chunk opens them; for the block-unit form
// the chunk's 8 quants as fp16, plus the block's unit ratio and min-term
// pieces and the half-unit's unit when the chunk opens them.
// qq: the chunk's 8 quants, sb: its block's (scale, sum), sr: the row's
// (scale, sum) of every block.
__device__ __forceinline__ void acth_chunk_v(uint2 qq, float2 sb, const float2* sr, int K, const ActH& o, size_t row,
                                             int c, int E, bool lo) {
    const int KH = K / 128;
    const int i = 8 * c, b = i >> 5, hh = i >> 7;
    if (o.q16) {
        // a block whose fp16 scale is zero (an underflow leaves nonzero quants) contributes nothing:
        // its quants are written as zeros, since the block keeps the previous block's unit
        if (sb.x == 0.0f) qq = make_uint2(0u, 0u);
        uint32_t w[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t word = u < 2 ? qq.x : qq.y;
            const _Float16 h0 = (_Float16)(float)(int8_t)(word >> (16 * (u & 1)));
            const _Float16 h1 = (_Float16)(float)(int8_t)(word >> (16 * (u & 1) + 8));
            w[u] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        }
        *reinterpret_cast<uint4*>(o.q16 + row * (size_t)K + i) = make_uint4(w[0], w[1], w[2], w[3]);
        if ((i & 31) == 0) {
            const int KB = K / 32;
            o.rx[row * (size_t)KB + b] = (b > 0 && sb.x != 0.0f) ? block_unit(sr, b - 1) / sb.x : 1.0f;
            const float uref = block_unit(sr, min((b & ~7) + 3, KB - 1));
            store_pieces3(o.xu + row * (size_t)o.KU * 24 + (b / 8) * 24 + (b % 8), sb.x * sb.y / uref);
        }
        if ((i & 127) == 0) o.pu[row * (size_t)KH + hh] = block_unit(sr, 4 * hh + 3);
    }
    if (!o.hl) return;
    const float dn = __uint_as_float((uint32_t)(127 - E) << 23), up = __uint_as_float((uint32_t)(127 + E) << 23);
    const float s = sb.x * dn;  // exact: power-of-two scaling
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const uint32_t word = u < 2 ? qq.x : qq.y;
        const int q0 = (int)(int8_t)(word >> (16 * (u & 1))), q1 = (int)(int8_t)(word >> (16 * (u & 1) + 8));
        const float v0 = s * (float)q0, v1 = s * (float)q1;  // exact: 11-bit scale x |q| <= 127
        const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
        const _Float16 l0 = (_Float16)(v0 - (float)h0), l1 = (_Float16)(v1 - (float)h1);
        hw[u] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        lw[u] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
    }
    uint16_t* hl = o.hl + row * (size_t)KH * 256 + hh * 256 + (i & 127);
    *reinterpret_cast<uint4*>(hl) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    if (lo) *reinterpret_cast<uint4*>(hl + 128) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    if ((i & 127) == 0) o.pe[row * (size_t)KH + hh] = up;
    if ((i & 31) == 0)  // exact: 11-bit scale x |sum| < 2^12, times 2^-E
        store_pieces3(o.xm + row * (size_t)o.KU * 24 + (b / 8) * 24 + (b % 8), sb.x * sb.y * dn);
}

__device__ __forceinline__ void acth_chunk(const int8_t* q, const float2* sc, int K, const ActH& o, size_t row, int c,
                                           int E, bool lo) {
    acth_chunk_v(*reinterpret_cast<const uint2*>(q + 8 * c), sc[c >> 2], sc, K, o, row, c, E, lo);
}

// One row by one wave (all 64 lanes): the row exponent from a wave maximum of
// the block scales, then four chunks per lane per pass with every load issued
// before the first store.
__device__ void write_acth_row(const int8_t* q, const float2* sc, int K, const ActH& o, size_t row, int lane,
                               bool lo = true) {
    const int KB = K / 32;
    float M = 0.0f;
    for (int b = lane; b < KB; b += 64) M = fmaxf(M, sc[b].x);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    const int E = acth_exponent(M);
    constexpr int U = 4;
    const int nc = K / 8;
    for (int c0 = lane; c0 < nc; c0 += U * 64) {
        uint2 qq[U];
        float2 sb[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = min(c0 + u * 64, nc - 1);
            qq[u] = *reinterpret_cast<const uint2*>(q + 8 * c);
            sb[u] = sc[c >> 2];
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (c0 + u * 64 < nc) acth_chunk_v(qq[u], sb[u], sc, K, o, row, c0 + u * 64, E, lo);
    }
}

int chain_stride(int d) { return chain_stride_of(d); }

void chain_rows(const float* rows, int nrows, int d, float* out) {
    const int S = chain_stride_of(d);
    std::fill(out, out + (size_t)nrows * 16 * S, 0.0f);
    for (int r = 0; r < nrows; ++r)
        for (int e = 0; e < d; ++e) out[(size_t)r * 16 * S + (e & 15) * S + (e >> 4)] = rows[(size_t)r * d + e];
}

// Routing for many tokens.  A block takes T tokens (T <= RT_TMAX, fewer when
// d is large or n small) and a split of the router rows (RPB rows; a single
// split when the rows fit one block's 16 lane groups):
//  1. the block's token rows -> LDS, chain-major.
//  2. (row split 0) Q8_0 of x, one thread per 32-block (quantize_row_q8_0,
//     src/quant.cpp:1029-1045): amax, d = amax/127 (IEEE division), id = 1/d,
//     q = clamp(round-half-away(x*id)), stored scale = truncated fp16 of d; the
//     block sum of q rides along for the Q4_0 (-8 offset) and Q4_K (min)
//     terms.  With a matrix-core consumer the rows' ActH form follows.
//  3. Router logits in vec_dot_f32's exact fp32 order (src/quant.cpp:2756-2778):
//     16 lanes per router row, lane j runs the FMA chain over elements 16i+j
//     (lanes 0-7 are the reference's acc0, 8-15 its acc1), then acc0+acc1 and
//     the sequential sum of the 8 lanes (d % 32 == 0: no tails).  One router
//     load (four chain steps, chain-major copy) feeds every token of the block,
//     whose chains are independent.  The shared-expert gate vector
//     (transformer.cpp:2748-2751) is one more row.
//  4. Top-k by rank counting (descending logit, ties by index) and softmax over
//     the k selected logits (select_experts_cache_aware, src/tier.cpp:144-188):
//     in the block with a single row split, else in k_route_topk once every
//     split has written its logits.
#ifndef JX_RT_TMAX
#define JX_RT_TMAX 4
#endif
#ifndef JX_RT_LDS_KB
#define JX_RT_LDS_KB 80
#endif
#ifndef JX_RT_UNROLL
#define JX_RT_UNROLL 4
#endif
constexpr int RT_THREADS = 256;
constexpr int RT_GROUPS = RT_THREADS / 16;  // router rows in flight per block
constexpr int RT_UNROLL = JX_RT_UNROLL;     // router loads in flight per lane (four chain steps each)
constexpr int RT_TMAX = JX_RT_TMAX;
constexpr size_t RT_LDS_TARGET = JX_RT_LDS_KB * 1024;  // two blocks per CU

static size_t route_lds(int T, int d, int E) {
    return (size_t)T * 16 * rs_stride(d) * sizeof(float) + (size_t)T * d + (size_t)T * (d / 32) * sizeof(float2) +
           (size_t)T * E * sizeof(float);
}

struct RouteShape {
    int T, RS, RPB;
};

// Rows R = E (+1 shared gate): up to 16 rows one split (fused top-k), more in
// splits of 16.  Tokens per block: a fused Mixtral-sized router measured best
// at 2, split routers (61 and 128 rows, d 2048) at 4 (1, 2 and 6-8 slower);
// small batches take one token per block for parallelism.
static RouteShape route_shape(const RouteArgs& a) {
    const int R = a.E + (a.shgate ? 1 : 0);
    RouteShape r;
    r.RS = R <= RT_GROUPS ? 1 : (R + RT_GROUPS - 1) / RT_GROUPS;
    r.RPB = r.RS == 1 ? R : RT_GROUPS;
    int T = r.RS == 1 ? 2 : RT_TMAX;
    if (a.n < 64 * T) T = std::max(1, a.n / 64);
    while (T > 1 && route_lds(T, a.d, a.E) > RT_LDS_TARGET) --T;
    r.T = T;
    return r;
}

// rpb = 0: only steps 1-2 (the quantized and matrix-core forms of x), for k_route_rows.
template <int T>
__global__ void __launch_bounds__(RT_THREADS) k_route(RouteArgs a, int nsplit, int rpb) {
    extern __shared__ __align__(16) float lds[];
    __shared__ int sel[T][MAX_K];
    __shared__ float shl[T];
    __shared__ float rmax[T];
    const int d = a.d, E = a.E, S = rs_stride(d), RS = 16 * S, KB = d / 32;
    const int split = blockIdx.x % nsplit;
    const int t0 = (blockIdx.x / nsplit) * T, nt = min(T, a.n - t0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float* xs = lds;                                       // [T][16][S] chain-major rows
    int8_t* qs = reinterpret_cast<int8_t*>(xs + T * RS);   // [T][d] quants
    float2* ss = reinterpret_cast<float2*>(qs + T * d);    // [T][KB] (scale, sum)
    float* lg = reinterpret_cast<float*>(ss + T * KB);     // [T][E] logits
    // every selection slot holds a valid expert even if NaN logits break the ranking
    for (int i = tid; i < T * MAX_K; i += RT_THREADS) sel[i / MAX_K][i % MAX_K] = i % MAX_K;

    // -- 1. rows -> LDS, four loads in flight per thread before their stores
    {
        const int c4 = d / 4, tot = nt * c4;
        for (int i0 = 0; i0 < tot; i0 += 4 * RT_THREADS) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = min(i0 + u * RT_THREADS + tid, tot - 1);
                const int t = i / c4, c = i - t * c4;
                v[u] = *reinterpret_cast<const float4*>(a.x + (size_t)(t0 + t) * d + 4 * c);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = min(i0 + u * RT_THREADS + tid, tot - 1);  // clamped duplicates store the same values
                const int t = i / c4, c = i - t * c4;
                float* dst = xs + t * RS + 4 * (c & 3) * S + (c >> 2);  // elements 4c..4c+3: j = 4(c%4)+q, i = c/4
                dst[0] = v[u].x;
                dst[S] = v[u].y;
                dst[2 * S] = v[u].z;
                dst[3 * S] = v[u].w;
            }
        }
    }
    __syncthreads();

    if (split == 0) {  // block-uniform
        // -- 2. Q8_0 of x: one thread per 32-block (its max and integer sum are order-free)
        for (int i = tid; i < nt * KB; i += RT_THREADS) {
            const int t = i / KB, b = i - t * KB;
            const float* xr = xs + t * RS + 2 * b;  // element 32b + u at (u % 16) * S + 2b + u / 16
            float v[32];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const float2 p = *reinterpret_cast<const float2*>(xr + u * S);
                v[u] = p.x;
                v[16 + u] = p.y;
            }
            float amax = 0.0f;
#pragma unroll
            for (int u = 0; u < 32; ++u) amax = fmaxf(amax, __builtin_fabsf(v[u]));
            const float dd = amax / 127.0f;
            const float id = (dd != 0.0f) ? 1.0f / dd : 0.0f;
            int sum = 0;
            uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                float r = round_away(v[u] * id);
                r = fminf(fmaxf(r, -127.0f), 127.0f);
                const int q = (int)r;
                sum += q;
                w[u >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (u & 3));
            }
            const float2 sv = make_float2(f16_to_f32(f32_to_f16_trunc(dd)), (float)sum);
            const uint4 w0 = make_uint4(w[0], w[1], w[2], w[3]), w1 = make_uint4(w[4], w[5], w[6], w[7]);
            uint4* gq = reinterpret_cast<uint4*>(a.xq.q + (size_t)(t0 + t) * a.xq.K + 32 * b);
            gq[0] = w0;
            gq[1] = w1;
            a.xq.s[(size_t)(t0 + t) * KB + b] = sv;
            uint4* lq = reinterpret_cast<uint4*>(qs + t * d + 32 * b);
            lq[0] = w0;
            lq[1] = w1;
            ss[t * KB + b] = sv;
        }
        __syncthreads();
        if (a.xh.hl || a.xh.q16) {  // matrix-core forms (hi/lo: one exponent per row from its largest block scale)
            for (int t = wave; t < nt; t += RT_THREADS / 64) {
                float M = 0.0f;
                for (int b = lane; b < KB; b += 64) M = fmaxf(M, ss[t * KB + b].x);
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
                if (lane == 0) rmax[t] = M;
            }
            __syncthreads();
            const int cpr = d / 8;
            for (int c = tid; c < nt * cpr; c += RT_THREADS) {
                const int t = c / cpr;
                acth_chunk(qs + t * d, ss + t * KB, d, a.xh, (size_t)(t0 + t), c - t * cpr, acth_exponent(rmax[t]), true);
            }
        }
    }

    if (rpb == 0) return;  // block-uniform
    // -- 3. router chains of this split's rows, exact vec_dot_f32 order
    {
        const int grp = tid >> 4, j = tid & 15;
        const int R = E + (a.shgate ? 1 : 0);
        const int r1 = min(R, (split + 1) * rpb);
        const int m = d / 16, m4 = m & ~3, Sg = chain_stride_of(d);
        for (int r = split * rpb + grp; r < r1; r += RT_GROUPS) {
            // F16 / BF16 router rows: vec_dot_{f16,bf16}_f32's order (src/quant.cpp:3015-3055), one chain
            // per lane jc < 8 over elements 8 i + jc, i.e. chain-major columns jc and jc + 8 interleaved
            // step by step (lanes 8-15 repeat lanes 0-7); the shared gate row stays fp32
            const bool c8 = a.chain8 && r < E;
            const int jc = c8 ? (j & 7) : j;
            const float* wr = a.router_cm + (size_t)r * 16 * Sg + jc * Sg;
            // token rows of the chains: tokens past nt (last block) repeat the last one, results dropped,
            // so the loop has no branches and the router loads can run ahead
            const float* xr[T];
#pragma unroll
            for (int t = 0; t < T; ++t) xr[t] = xs + min(t, nt - 1) * RS + jc * S;
            float acc[T];
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] = 0.0f;
            if (c8) {
                const float* wr8 = wr + 8 * Sg;
                for (int i = 0; i < m4; i += 4) {
                    const float4 w4 = *reinterpret_cast<const float4*>(wr + i);
                    const float4 w8 = *reinterpret_cast<const float4*>(wr8 + i);
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        const float4 x4 = *reinterpret_cast<const float4*>(xr[t] + i);
                        const float4 x8 = *reinterpret_cast<const float4*>(xr[t] + 8 * S + i);
                        acc[t] = __builtin_fmaf(w4.x, x4.x, acc[t]);
                        acc[t] = __builtin_fmaf(w8.x, x8.x, acc[t]);
                        acc[t] = __builtin_fmaf(w4.y, x4.y, acc[t]);
                        acc[t] = __builtin_fmaf(w8.y, x8.y, acc[t]);
                        acc[t] = __builtin_fmaf(w4.z, x4.z, acc[t]);
                        acc[t] = __builtin_fmaf(w8.z, x8.z, acc[t]);
                        acc[t] = __builtin_fmaf(w4.w, x4.w, acc[t]);
                        acc[t] = __builtin_fmaf(w8.w, x8.w, acc[t]);
                    }
                }
                for (int i = m4; i < m; ++i) {
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        acc[t] = __builtin_fmaf(wr[i], xr[t][i], acc[t]);
                        acc[t] = __builtin_fmaf(wr8[i], xr[t][8 * S + i], acc[t]);
                    }
                }
            } else {
#pragma unroll RT_UNROLL
                for (int i = 0; i < m4; i += 4) {
                    const float4 w4 = *reinterpret_cast<const float4*>(wr + i);
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        const float4 x4 = *reinterpret_cast<const float4*>(xr[t] + i);
                        acc[t] = __builtin_fmaf(w4.x, x4.x, acc[t]);
                        acc[t] = __builtin_fmaf(w4.y, x4.y, acc[t]);
                        acc[t] = __builtin_fmaf(w4.z, x4.z, acc[t]);
                        acc[t] = __builtin_fmaf(w4.w, x4.w, acc[t]);
                    }
                }
                for (int i = m4; i < m; ++i) {
                    const float wv = wr[i];
#pragma unroll
                    for (int t = 0; t < T; ++t) acc[t] = __builtin_fmaf(wv, xr[t][i], acc[t]);
                }
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                if (t < nt) {
                    const float s = chain_sum(acc[t], c8);
                    if (j == 0) {
                        const size_t tok = (size_t)(t0 + t);
                        if (r < E) {
                            const float l = a.bias ? s + a.bias[r] : s;
                            if (nsplit == 1) lg[t * E + r] = l;
                            else a.logits[tok * E + r] = l;
                        } else if (nsplit == 1) {
                            shl[t] = s;
                        } else {
                            a.shscale[tok] = s;  // raw shared-gate logit; k_route_topk applies the sigmoid
                        }
                    }
                }
            }
        }
    }
    if (nsplit > 1) return;  // block-uniform
    __syncthreads();

    // -- 4. top-k by rank, softmax over the selected logits
    for (int i = tid; i < nt * E; i += RT_THREADS) {
        const int t = i / E, e = i - t * E;
        const float* lt = lg + t * E;
        const int rank = rank_of(lt, E, e);
        if (rank < a.k) sel[t][rank] = e;
        if (a.logits) a.logits[(size_t)(t0 + t) * E + e] = lt[e];
    }
    __syncthreads();
    static_assert(32 * T <= RT_THREADS, "one half-wave per token");
    if (tid < 32 * nt) {
        const int t = tid >> 5, i = tid & 31, k = a.k;
        const size_t o = (size_t)(t0 + t) * k;
        softmax_selected(lg + t * E, sel[t], k, i, a.ids + o, a.probs + o);
        if (i == 0 && a.shscale) a.shscale[t0 + t] = a.shgate ? 1.0f / (1.0f + expf(-shl[t])) : 1.0f;
    }
}

// Router logits for many tokens against a router of more than 16 rows with
// d <= 2048 (d / 64 in 8, 16, 24, 32): a block owns 16 rows and tpb tokens.  Lane j
// of a row's 16-lane group keeps its whole vec_dot_f32 chain of router values
// in registers (read once), and the tokens stream through LDS four at a time,
// chain-major, the next chunk's loads in flight while the current one is
// consumed.  Router traffic is one read per block instead of one per 4 tokens.
// Same chain order and reduction as k_route (src/quant.cpp:2756-2778).
#ifndef JX_RR_TPB
#define JX_RR_TPB 32
#endif
#ifndef JX_RR_TC
#define JX_RR_TC 4
#endif
constexpr int RR_TPB = JX_RR_TPB;  // tokens per block, at most (fewer keep small batches spread)
constexpr int RR_TC = JX_RR_TC;    // tokens per LDS chunk

template <int M4>  // d / 64 float4 chain steps per lane
__global__ void __launch_bounds__(RT_THREADS) k_route_rows(RouteArgs a, int nsplit, int tpb) {
    extern __shared__ __align__(16) float xs[];  // [2][RR_TC][16][S]
    constexpr int d = 64 * M4, C4 = d / 4, S = rs_stride(d), RS = 16 * S, Sg = chain_stride_of(d);
    constexpr int PER = (RR_TC * C4 + RT_THREADS - 1) / RT_THREADS;  // float4 per thread per chunk
    const int split = blockIdx.x % nsplit, t0 = (blockIdx.x / nsplit) * tpb;
    const int tend = min(a.n, t0 + tpb);
    const int tid = threadIdx.x, grp = tid >> 4, j = tid & 15;
    const int E = a.E, R = E + (a.shgate ? 1 : 0);
    const int r = split * RT_GROUPS + grp;
    const bool live = r < R;
    float4 w[M4];
    {
        const float* wr = a.router_cm + (size_t)min(r, R - 1) * 16 * Sg + j * Sg;
#pragma unroll
        for (int i = 0; i < M4; ++i) w[i] = *reinterpret_cast<const float4*>(wr + 4 * i);
    }
    // chunk staging: RR_TC tokens x d floats; float4 c of token t holds chains 4(c%4)..4(c%4)+3 at step c/4
    float4 v[PER];
    auto issue = [&](int c0) {
        const int last = min(RR_TC, tend - c0) * C4 - 1;
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = min(u * RT_THREADS + tid, last);
            v[u] = *reinterpret_cast<const float4*>(a.x + (size_t)c0 * d + 4 * i);
        }
    };
    auto store = [&](int c0, float* buf) {
        const int last = min(RR_TC, tend - c0) * C4 - 1;
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = min(u * RT_THREADS + tid, last);  // clamped duplicates store the same values
            const int t = i / C4, c = i % C4;
            float* dst = buf + t * RS + 4 * (c & 3) * S + (c >> 2);
            dst[0] = v[u].x;
            dst[S] = v[u].y;
            dst[2 * S] = v[u].z;
            dst[3 * S] = v[u].w;
        }
    };
    issue(t0);
    store(t0, xs);
    int buf = 0;
    for (int c0 = t0; c0 < tend; c0 += RR_TC) {
        const int nt = min(RR_TC, tend - c0);
        if (c0 + RR_TC < tend) issue(c0 + RR_TC);  // block-uniform
        __syncthreads();  // chunk c0 staged; the other buffer's readers are done
        const float* xb = xs + buf * RR_TC * RS;
        if (live) {
            const float* xr[RR_TC];
#pragma unroll
            for (int t = 0; t < RR_TC; ++t) xr[t] = xb + min(t, nt - 1) * RS + j * S;
            float acc[RR_TC];
#pragma unroll
            for (int t = 0; t < RR_TC; ++t) acc[t] = 0.0f;
#pragma unroll
            for (int i = 0; i < M4; ++i) {
#pragma unroll
                for (int t = 0; t < RR_TC; ++t) {
                    const float4 x4 = *reinterpret_cast<const float4*>(xr[t] + 4 * i);
                    acc[t] = __builtin_fmaf(w[i].x, x4.x, acc[t]);
                    acc[t] = __builtin_fmaf(w[i].y, x4.y, acc[t]);
                    acc[t] = __builtin_fmaf(w[i].z, x4.z, acc[t]);
                    acc[t] = __builtin_fmaf(w[i].w, x4.w, acc[t]);
                }
            }
            float sums[RR_TC];
#pragma unroll
            for (int t = 0; t < RR_TC; ++t) {
                const float hi = __shfl_down(acc[t], 8, 16);
                const float vv = acc[t] + hi;  // acc0[j] + acc1[j] for j < 8
                float sum = 0.0f;
#pragma unroll
                for (int q = 0; q < 8; ++q) sum += __shfl(vv, q, 16);
                sums[t] = sum;
            }
#pragma unroll
            for (int t = 0; t < RR_TC; ++t) {
                const float sum = sums[t];
                if (j == 0 && t < nt) {
                    const size_t tok = (size_t)(c0 + t);
                    if (r < E) a.logits[tok * E + r] = a.bias ? sum + a.bias[r] : sum;
                    else a.shscale[tok] = sum;  // raw shared-gate logit; k_route_topk applies the sigmoid
                }
            }
        }
        if (c0 + RR_TC < tend) store(c0 + RR_TC, xs + (buf ^ 1) * RR_TC * RS);
        buf ^= 1;
    }
}

// Top-k and softmax once every split has written its logits (raw shared-gate
// logits in shscale): one wave per token, four tokens per block.
template <int NC>
__global__ void __launch_bounds__(256) k_route_topk(RouteArgs a) {
    const size_t t = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= (size_t)a.n) return;  // wave-uniform
    uint64_t msk[NC];
    (void)topk_token_wave<NC>(a, a.logits + t * a.E, t, a.shgate ? a.shscale : nullptr, msk);
}

static void launch_route_topk(const RouteArgs& a, hipStream_t st) {
    const dim3 grid((a.n + 3) / 4);
    const int nc = (a.E + 63) / 64;
    if (nc <= 1) hipLaunchKernelGGL(k_route_topk<1>, grid, dim3(256), 0, st, a);
    else if (nc <= 2) hipLaunchKernelGGL(k_route_topk<2>, grid, dim3(256), 0, st, a);
    else if (nc <= 4) hipLaunchKernelGGL(k_route_topk<4>, grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(k_route_topk<MAX_E / 64>, grid, dim3(256), 0, st, a);
}

static bool route_rows_fits(const RouteArgs& a) {
    const int R = a.E + (a.shgate ? 1 : 0);
    const int m4 = a.d / 64;
// below ~512 tokens the split k_route (one token per block, router from L2) measured faster
#ifndef JX_RR_MIN_N
#define JX_RR_MIN_N 512
#endif
    // (F16 / BF16 routers: two chain columns per lane would not fit the register-resident rows)
    return R > RT_GROUPS && a.d % 64 == 0 && (m4 == 8 || m4 == 16 || m4 == 24 || m4 == 32) && a.n >= JX_RR_MIN_N &&
           !a.chain8;
}

void launch_route(const RouteArgs& a, hipStream_t st) {
    if (route_rows_fits(a)) {
        // quantized / matrix-core forms of x, then the logits with register-resident router rows, then top-k
        const int T = a.n >= 256 ? 4 : 1;
        const size_t lq = route_lds(T, a.d, a.E);
        auto q = T == 4 ? k_route<4> : k_route<1>;
        if (lq > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(q), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)lq);
        hipLaunchKernelGGL(q, dim3((a.n + T - 1) / T), dim3(RT_THREADS), lq, st, a, 1, 0);
        const int R = a.E + (a.shgate ? 1 : 0), RS = (R + RT_GROUPS - 1) / RT_GROUPS;
        const size_t lr = (size_t)2 * RR_TC * 16 * rs_stride(a.d) * sizeof(float);
        // tokens per block: about 512 blocks in all, in whole LDS chunks, at most RR_TPB
        const int tpb = std::min(RR_TPB, std::max(RR_TC, ((a.n * RS + 511) / 512 + RR_TC - 1) / RR_TC * RR_TC));
        const dim3 grid(RS * ((a.n + tpb - 1) / tpb));
        auto go = [&](auto kern) {
            if (lr > 65536)
                (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lr);
            hipLaunchKernelGGL(kern, grid, dim3(RT_THREADS), lr, st, a, RS, tpb);
        };
        switch (a.d / 64) {
            case 8: go(k_route_rows<8>); break;
            case 16: go(k_route_rows<16>); break;
            case 24: go(k_route_rows<24>); break;
            default: go(k_route_rows<32>); break;
        }
        launch_route_topk(a, st);
        return;
    }
    RouteShape r = route_shape(a);
    r.T = r.T >= 4 ? 4 : r.T >= 2 ? 2 : 1;  // instantiated token counts
    const size_t lds = route_lds(r.T, a.d, a.E);
    const int tb = (a.n + r.T - 1) / r.T;
    auto go = [&](auto kern) {
        if (lds > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)lds);
        hipLaunchKernelGGL(kern, dim3(tb * r.RS), dim3(RT_THREADS), lds, st, a, r.RS, r.RPB);
    };
    switch (r.T) {
        case 4: go(k_route<4>); break;
        case 2: go(k_route<2>); break;
        default: go(k_route<1>); break;
    }
    if (r.RS > 1) launch_route_topk(a, st);
}

// Matrix-core form of Q8_0 activations already in global memory, one wave per row.
__global__ void __launch_bounds__(256) k_q8_to_acth(ActQ8 in, int rows, ActH out, int lo) {
    const size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= (size_t)rows) return;  // wave-uniform
    write_acth_row(in.q + row * in.K, in.s + row * (in.K / 32), in.K, out, row, threadIdx.x & 63, lo != 0);
}

__device__ __forceinline__ uint32_t comp4(const uint4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// The hi-only form (the down GEMM's operand, no block-unit form) of Q8_0 rows, one wave per row:
// every quant and scale load of the row is in flight before the first conversion (16 quants per lane
// and chunk, NC chunks per lane), and the row exponent comes from the scales already loaded.  The
// values are those of acth_chunk_v: fp16(dx * 2^-E * q), 2^E per half-unit, the min-term pieces of
// dx * sum(q) * 2^-E.
template <int NC>
__global__ void __launch_bounds__(256) k_q8_to_acth_hi(ActQ8 in, int rows, ActH o) {
    const size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= (size_t)rows) return;  // wave-uniform
    const int lane = threadIdx.x & 63, K = in.K, n16 = K / 16, KH = K / 128;
    const int8_t* q = in.q + row * K;
    const float2* sc = in.s + row * (K / 32);
    uint4 qv[NC];
    float2 sv[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = min(lane + 64 * c, n16 - 1);  // clamped duplicates are loaded, not stored
        qv[c] = ld16(q + 16 * i);
        sv[c] = sc[i >> 1];
    }
    float M = 0.0f;  // chunks 2b and 2b + 1 carry block b's scale, so this covers every block
#pragma unroll
    for (int c = 0; c < NC; ++c) M = fmaxf(M, sv[c].x);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    const int E = acth_exponent(M);
    const float dn = __uint_as_float((uint32_t)(127 - E) << 23), up = __uint_as_float((uint32_t)(127 + E) << 23);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int i = lane + 64 * c;
        if (i >= n16) break;
        const int e = 16 * i, b = e >> 5, hh = e >> 7;
        const float s = sv[c].x * dn;  // exact: power-of-two scaling
        uint32_t hw[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t word = comp4(qv[c], u >> 1);
            const int q0 = (int)(int8_t)(word >> (16 * (u & 1))), q1 = (int)(int8_t)(word >> (16 * (u & 1) + 8));
            const _Float16 h0 = (_Float16)(s * (float)q0), h1 = (_Float16)(s * (float)q1);  // products exact
            hw[u] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        }
        uint4* hl = reinterpret_cast<uint4*>(o.hl + row * (size_t)KH * 256 + hh * 256 + (e & 127));
        hl[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        hl[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
        if ((e & 127) == 0) o.pe[row * (size_t)KH + hh] = up;
        if ((e & 31) == 0)  // exact: 11-bit scale x |sum| < 2^12, times 2^-E
            store_pieces3(o.xm + row * (size_t)o.KU * 24 + (b / 8) * 24 + (b % 8), sv[c].x * sv[c].y * dn);
    }
}

void launch_q8_to_acth(const ActQ8& in, int rows, ActH out, hipStream_t st, bool lo) {
    const int nc = (in.K / 16 + 63) / 64;
    if (!lo && !out.q16 && in.K % 128 == 0 && nc <= 16) {
        const dim3 grid((rows + 3) / 4);
        if (nc <= 1) hipLaunchKernelGGL(k_q8_to_acth_hi<1>, grid, dim3(256), 0, st, in, rows, out);
        else if (nc <= 2) hipLaunchKernelGGL(k_q8_to_acth_hi<2>, grid, dim3(256), 0, st, in, rows, out);
        else if (nc <= 4) hipLaunchKernelGGL(k_q8_to_acth_hi<4>, grid, dim3(256), 0, st, in, rows, out);
        else if (nc <= 8) hipLaunchKernelGGL(k_q8_to_acth_hi<8>, grid, dim3(256), 0, st, in, rows, out);
        else hipLaunchKernelGGL(k_q8_to_acth_hi<16>, grid, dim3(256), 0, st, in, rows, out);
        return;
    }
    hipLaunchKernelGGL(k_q8_to_acth, dim3((rows + 3) / 4), dim3(256), 0, st, in, rows, out, lo ? 1 : 0);
}

// Matrix-core form (fp16 hi only) of fp32 activation rows h [rows][ld], out.K
// a multiple of 128 (K-quants: 256, zero padding past the real columns) -- the
// reference's fp32-activation products (vec_dot_quant_f32, src/quant.cpp:3269-3305)
// for a down projection without a Q8_0 form (Q5_0, or a K-quant whose K is not
// a multiple of 256).  One block per
// row: E = exponent(max |h|) - 14 so every h * 2^-E is below 2^15; hi =
// fp16(h * 2^-E) (relative error <= 2^-12 per value, as the Q8_0 down operand);
// the min-term value of each 32-block is its fp32 sum times 2^-E, split into
// three exact bf16 pieces.
__global__ void __launch_bounds__(256) k_f32_to_acth(const float* h, int ld, ActH o) {
    __shared__ float wmax[4];
    const size_t row = blockIdx.x;
    const int tid = threadIdx.x, K = o.K, KH = K / 128;
    const float* hr = h + row * (size_t)ld;
    float M = 0.0f;
    for (int i = tid; i < K / 4; i += 256) {
        const float4 v = *reinterpret_cast<const float4*>(hr + 4 * i);
        M = fmaxf(M, fmaxf(fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)), fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w))));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
    if ((tid & 63) == 0) wmax[tid >> 6] = M;
    __syncthreads();
    M = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const int E = (M > 0.0f) ? (int)((__float_as_uint(M) >> 23) & 0xFF) - 127 - 14 : 0;
    const float dn = __uint_as_float((uint32_t)(127 - E) << 23), up = __uint_as_float((uint32_t)(127 + E) << 23);
    // eight consecutive values per thread; the four threads of a 32-block are consecutive lanes
    for (int c = tid; c < K / 8; c += 256) {
        const int i = 8 * c, b = i >> 5, hh = i >> 7;
        const float4 v0 = *reinterpret_cast<const float4*>(hr + i), v1 = *reinterpret_cast<const float4*>(hr + i + 4);
        const float f[8] = {v0.x * dn, v0.y * dn, v0.z * dn, v0.w * dn, v1.x * dn, v1.y * dn, v1.z * dn, v1.w * dn};
        uint32_t hw[4];
        float sum = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const _Float16 h0 = (_Float16)f[2 * u], h1 = (_Float16)f[2 * u + 1];
            hw[u] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            sum += f[2 * u] + f[2 * u + 1];
        }
        uint16_t* hl = o.hl + row * (size_t)KH * 256 + hh * 256 + (i & 127);
        *reinterpret_cast<uint4*>(hl) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        if ((i & 127) == 0) o.pe[row * (size_t)KH + hh] = up;
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        if ((i & 31) == 0) {
            const uint32_t bh = __float_as_uint(sum) & 0xFFFF0000u;
            const float r1 = sum - __uint_as_float(bh);
            const uint32_t bm = __float_as_uint(r1) & 0xFFFF0000u;
            const float r2 = r1 - __uint_as_float(bm);
            uint16_t* xm = o.xm + row * (size_t)o.KU * 24 + (b / 8) * 24 + (b % 8);
            xm[0] = (uint16_t)(bh >> 16);
            xm[8] = (uint16_t)(bm >> 16);
            xm[16] = (uint16_t)(__float_as_uint(r2) >> 16);
        }
    }
}

void launch_f32_to_acth(const float* h, int ld, int rows, ActH out, hipStream_t st) {
    hipLaunchKernelGGL(k_f32_to_acth, dim3(rows), dim3(256), 0, st, h, ld, out);
}

// ---------------------------------------------------------------- few tokens
// Decode routing: a one-block-per-token kernel would serialise every router
// row behind one CU's load latency.  Here block r owns router row r (expert r,
// or the shared-expert gate vector as row E): it stages that row and the n
// tokens in LDS with all loads in flight, then 16 lanes per token run the
// vec_dot_f32 chains from LDS.  Blocks also split the Q8_0 quantization of x.
// A second one-block launch ranks, normalises and dispatches: with
// n*k <= 2*32 pairs the counting sort is a short serial loop.
constexpr int RS_THREADS = 256;
constexpr int RS_LDS_BYTES = 64 * 1024;

static size_t rs_lds(int n, int d) { return (size_t)(1 + n) * 16 * rs_stride(d) * sizeof(float); }

bool route_small_fits(int n, int d, int E) {
    return n >= 1 && n <= ROUTE_SMALL_MAX_N && E <= MAX_E && d % 32 == 0 && rs_lds(n, d) <= RS_LDS_BYTES;
}

__global__ void __launch_bounds__(RS_THREADS)
k_route_small(RouteArgs a) {
    extern __shared__ float lds[];  // (1 + n) chain-major rows: router row r, then the n tokens
    const int r = blockIdx.x, tid = threadIdx.x;
    if (r == 0)  // the folded combine's output starts at zero (CombineOut)
        for (int i = tid; i < a.zero_count; i += RS_THREADS) a.zero_out[i] = 0.0f;
    const int d = a.d, n = a.n, E = a.E, S = rs_stride(d), RS = 16 * S;
    const float* w = r < E ? a.router + (size_t)r * d : a.shgate;
    {  // router row + token rows -> LDS: every load in flight before the first store
        constexpr int PER = (ROUTE_SMALL_MAX_N + 1) * 8192 / 4 / RS_THREADS;  // float4 slots: d <= 8192
        const int c4 = d / 4, tot = (1 + n) * c4;
        float4 v[PER];
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = tid + q * RS_THREADS;
            if (i >= tot) break;
            const int row = i / c4, c = i - row * c4;
            const float* src = row == 0 ? w + 4 * c : a.x + (size_t)(row - 1) * d + 4 * c;
            v[q] = *reinterpret_cast<const float4*>(src);
        }
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = tid + q * RS_THREADS;
            if (i >= tot) break;
            const int row = i / c4, c = i - row * c4;
            float* dst = lds + row * RS + 4 * (c & 3) * S + (c >> 2);  // elements 4c..4c+3: j = 4(c%4)+q, i = c/4
            dst[0] = v[q].x;
            dst[S] = v[q].y;
            dst[2 * S] = v[q].z;
            dst[3 * S] = v[q].w;
        }
    }
    __syncthreads();
    const int wave = tid >> 6, lane = tid & 63;
    if (wave == 0) {
        // router row r for every token: vec_dot_f32 order (src/quant.cpp:2756-2778): lane j of
        // token group t runs the FMA chain over elements 16 i + j (lanes 0-7 the reference's acc0,
        // 8-15 its acc1), then acc0 + acc1 and the sequential sum of the 8 lanes (d % 16 == 0: no
        // tails)
        const int t = lane >> 4, j = lane & 15;
        if (t < n) {
            // F16 / BF16 router rows: columns jc and jc + 8 interleaved (as k_route); the shared gate fp32
            const bool c8 = a.chain8 && r < E;
            const float s = chain_sum(chain_dot_lds(lds, lds + (1 + t) * RS, S, d, j, c8), c8);
            if (j == 0) {
                if (r < E) a.logits[(size_t)t * E + r] = a.bias ? s + a.bias[r] : s;
                else a.shscale[t] = s;  // raw shared-gate logit; the top-k step applies the sigmoid
            }
        }
    } else {
        // this block's share of the Q8_0 blocks of x, one per half-wave of waves 1..
        const int nb = d / 32, tot = n * nb;
        const int per = (tot + gridDim.x - 1) / gridDim.x;
        const int b0 = r * per, b1 = min(tot, b0 + per);
        const int half = lane >> 5, l32 = lane & 31;
        constexpr int QW = RS_THREADS / 64 - 1;
        for (int bb = b0 + (wave - 1) * 2; bb < b1; bb += QW * 2) {
            const int b = bb + half;  // token-major: b = t*nb + block
            const bool ok = b < b1;
            const int t = ok ? b / nb : 0, q = ok ? (b % nb) * 32 + l32 : 0;
            const float xv = lds[(1 + t) * RS + (q & 15) * S + (q >> 4)];
            quant_block(xv, l32, ok, a.xq, (size_t)t, ok ? b % nb : 0);
        }
    }
}

// Second launch of the few-token router: top-k and dispatch tables from the
// logits of k_route_small (raw shared-gate logits in shscale), one wave.
template <int NC>
__global__ void __launch_bounds__(64) k_topk_small(RouteArgs a, DispatchOut o) {
    topk_dispatch_wave<NC>(a, o, a.logits, a.shgate ? a.shscale : nullptr);
}

// The whole few-token routing in one block when the router fits in LDS
// (Mixtral-sized routers: 8 x 4096 fp32 = 128 KB): stage router + tokens with
// every load in flight, Q8_0 of x, the vec_dot_f32 chains (16 lanes each, as
// in k_route), then top-k, softmax and dispatch.  One launch instead of two,
// one HBM round trip.
constexpr int R1_THREADS = 1024;
constexpr int R1_PER = 10;  // float4 staging slots per thread
constexpr size_t R1_LDS_BYTES = (size_t)R1_THREADS * R1_PER * 16;

static size_t route_one_lds(int n, int d, int E, bool shgate) {
    return ((size_t)(E + (shgate ? 1 : 0) + n) * d + (size_t)std::max(n, 2) * E) * sizeof(float);
}

bool route_one_fits(int n, int d, int E, bool shgate) {
    return n >= 1 && n <= ROUTE_SMALL_MAX_N && E <= 64 && d % 16 == 0 &&
           (size_t)(E + (shgate ? 1 : 0) + n) * d * sizeof(float) <= R1_LDS_BYTES &&
           route_one_lds(n, d, E, shgate) <= 160 * 1024;
}

__global__ void __launch_bounds__(R1_THREADS) k_route_one(RouteArgs a, DispatchOut o) {
    extern __shared__ float lds[];  // [rows][d] router (+ shared gate), [n][d] tokens, [n][E] logits
    __shared__ float shl[ROUTE_SMALL_MAX_N];
    const int tid = threadIdx.x;
    const int d = a.d, n = a.n, E = a.E, rows = E + (a.shgate ? 1 : 0);
    for (int i = tid; i < a.zero_count; i += R1_THREADS) a.zero_out[i] = 0.0f;  // folded combine (CombineOut)
    float* xs = lds + (size_t)rows * d;
    float* lgs = xs + (size_t)n * d;
    {
        const int c4 = d / 4, tot = (rows + n) * c4;  // route_one_fits: tot <= R1_THREADS * R1_PER
        float4 v[R1_PER];
#pragma unroll
        for (int q = 0; q < R1_PER; ++q) {
            const int i = min(tid + q * R1_THREADS, tot - 1);
            const int row = i / c4, c = i - row * c4;
            const float* src = row < E ? a.router + (size_t)row * d : (row < rows ? a.shgate : a.x + (size_t)(row - rows) * d);
            v[q] = *reinterpret_cast<const float4*>(src + 4 * c);
        }
#pragma unroll
        for (int q = 0; q < R1_PER; ++q) {
            const int i = min(tid + q * R1_THREADS, tot - 1);
            *reinterpret_cast<float4*>(lds + 4 * i) = v[q];
        }
    }
    __syncthreads();
    // the first CW waves run the (token, router row) chains, the others quantize x
    const int chains = n * rows, CW = min(R1_THREADS / 64 - 1, (chains + 3) / 4);
    if ((tid >> 6) >= CW) {  // Q8_0 of x, one 32-block per half-wave
        const int nb = d / 32, lane = tid & 63, half = lane >> 5, l32 = lane & 31;
        for (int b = ((tid >> 6) - CW) * 2 + half; b < n * nb; b += (R1_THREADS / 64 - CW) * 2)
            quant_block(xs[(size_t)b * 32 + l32], l32, true, a.xq, (size_t)(b / nb), b % nb);
    }
    // chains, 16 lanes each, vec_dot_f32 order (d % 16 == 0: no tails)
    for (int c = tid >> 4; c < chains && (tid >> 6) < CW; c += CW * 4) {
        const int t = c / rows, r = c % rows, j = tid & 15;
        const float* w = lds + (size_t)r * d;
        const float* xt = xs + (size_t)t * d;
        // F16 / BF16 router rows: 8 chains over 8-element steps (lanes 8-15 repeat lanes 0-7)
        const bool c8 = a.chain8 && r < E;
        float acc = 0.0f;
        if (c8) {
            const int jc = j & 7;
#pragma unroll 32
            for (int i = 0; i < d; i += 8) acc = __builtin_fmaf(w[i + jc], xt[i + jc], acc);
        } else {
#pragma unroll 32
            for (int i = 0; i < d; i += 16) acc = __builtin_fmaf(w[i + j], xt[i + j], acc);
        }
        const float s = chain_sum(acc, c8);
        if (j == 0) {
            if (r < E) {
                const float l = a.bias ? s + a.bias[r] : s;
                lgs[t * E + r] = l;
                a.logits[(size_t)t * E + r] = l;
            } else {
                shl[t] = s;
            }
        }
    }
    __syncthreads();
    if (tid < 64) topk_dispatch_wave<1>(a, o, lgs, a.shgate ? shl : nullptr);
}

void launch_route_logits(const RouteArgs& a, hipStream_t st) {
    const int rows = a.E + (a.shgate ? 1 : 0);
    hipLaunchKernelGGL(k_route_small, dim3(rows), dim3(RS_THREADS), rs_lds(a.n, a.d), st, a);
}

void launch_route_small(const RouteArgs& a, const DispatchOut& o, hipStream_t st) {
    const int rows = a.E + (a.shgate ? 1 : 0);
    if (route_one_fits(a.n, a.d, a.E, a.shgate != nullptr)) {
        const size_t lds = route_one_lds(a.n, a.d, a.E, a.shgate != nullptr);
        // dynamic LDS above 64 KB needs the kernel's opt-in; without it, the two-launch path
        const bool ok = lds <= 65536 || hipFuncSetAttribute(reinterpret_cast<const void*>(k_route_one),
                                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                                            (int)lds) == hipSuccess;
        if (ok) {
            hipLaunchKernelGGL(k_route_one, dim3(1), dim3(R1_THREADS), lds, st, a, o);
            return;
        }
        (void)hipGetLastError();  // clear the refused opt-in
    }
    hipLaunchKernelGGL(k_route_small, dim3(rows), dim3(RS_THREADS), rs_lds(a.n, a.d), st, a);
    const int nc = (a.E + 63) / 64;
    if (nc <= 1) hipLaunchKernelGGL(k_topk_small<1>, dim3(1), dim3(64), 0, st, a, o);
    else if (nc <= 2) hipLaunchKernelGGL(k_topk_small<2>, dim3(1), dim3(64), 0, st, a, o);
    else if (nc <= 4) hipLaunchKernelGGL(k_topk_small<4>, dim3(1), dim3(64), 0, st, a, o);
    else hipLaunchKernelGGL(k_topk_small<MAX_E / 64>, dim3(1), dim3(64), 0, st, a, o);
}

// One block per expert.  Every block builds the full per-expert histogram in
// LDS (no global atomics, nothing to clear between calls), derives its pair
// offset, MFMA tile offset and active-list slot, then writes the positions of
// its (token, slot) pairs in flat order -- a stable counting sort, so tokens
// keep their order inside each expert.
//  - histogram: four ids per thread per 16-byte load; up to 16 experts by
//    wave ballots (LDS atomics on so few bins would serialize), else LDS atomics;
//  - positions: rounds of up to 4 x DP_U x 256 ids, each wave a contiguous quarter:
//    one pass records the matches as a 64-bit mask per lane (4 ids x DP_U loads),
//    one barrier exchanges the wave totals, and the writes follow the masks
//    in flat order (lane prefixes from three ballots of the per-lane count).
constexpr int DISPATCH_THREADS = 256;
constexpr int DP_U = 16;  // 16-byte id loads per lane per round, at most

__device__ __forceinline__ int4 load_ids4(const int* ids, int f, int nk) {
    if (f + 3 < nk) return *reinterpret_cast<const int4*>(ids + f);  // ids 16-byte aligned, f % 4 == 0
    return make_int4(f < nk ? ids[f] : -1, f + 1 < nk ? ids[f + 1] : -1, f + 2 < nk ? ids[f + 2] : -1, -1);
}

__global__ void __launch_bounds__(DISPATCH_THREADS)
k_dispatch(const int* ids, int nk, int E, int top_k, DispatchOut o, int cold_max) {
    extern __shared__ int hist[];
    __shared__ int red[3][DISPATCH_THREADS / 64];
    __shared__ int wtot[2][DISPATCH_THREADS / 64];
    const int e = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int NW = DISPATCH_THREADS / 64;
    for (int i = tid; i < E; i += DISPATCH_THREADS) hist[i] = 0;
    __syncthreads();
    if (E <= 16) {
        // per-thread 8-bit counters (experts 0-7 in lo, 8-15 in hi), flushed before any can reach 256
        uint64_t lo = 0, hi = 0;
        int since = 0;
        auto flush = [&]() {
            for (int x = 0; x < E; ++x) {  // wave-uniform
                int c = (int)(((x < 8 ? lo : hi) >> (8 * (x & 7))) & 255u);
#pragma unroll
                for (int m = 32; m >= 1; m >>= 1) c += __shfl_xor(c, m, 64);
                if (lane == 0) atomicAdd(&hist[x], c);
            }
            lo = hi = 0;
        };
        auto count = [&](int id) {
            const uint64_t one = 1ull << (8 * (id & 7));
            lo += id >= 0 && id < 8 ? one : 0ull;
            hi += id >= 8 ? one : 0ull;
        };
        for (int base = wave * 256; base < nk; base += DISPATCH_THREADS * 4) {  // wave-uniform
            const int4 v = load_ids4(ids, base + 4 * lane, nk);
            count(v.x);
            count(v.y);
            count(v.z);
            count(v.w);
            if (++since == 63) {  // 63 * 4 = 252 per counter at most
                flush();
                since = 0;
            }
        }
        flush();
    } else {
        for (int f = 4 * tid; f < nk; f += 4 * DISPATCH_THREADS) {
            const int4 v = load_ids4(ids, f, nk);
            atomicAdd(&hist[v.x], 1);
            if (v.y >= 0) atomicAdd(&hist[v.y], 1);
            if (v.z >= 0) atomicAdd(&hist[v.z], 1);
            if (v.w >= 0) atomicAdd(&hist[v.w], 1);
        }
    }
    __syncthreads();
    // pair offset, tile offset and active index of expert e: sums over the experts before it (the tile
    // list holds the experts of at least cold_max pairs only, when cold_max > 0: the others take the GEMVs)
    int off = 0, toff = 0, na = 0;
    for (int i = tid; i < e; i += DISPATCH_THREADS) {
        const int c = hist[i];
        off += c;
        toff += c >= cold_max ? (c + MFMA_BN - 1) / MFMA_BN : 0;
        na += c > 0;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        off += __shfl_xor(off, m, 64);
        toff += __shfl_xor(toff, m, 64);
        na += __shfl_xor(na, m, 64);
    }
    if (lane == 0) {
        red[0][wave] = off;
        red[1][wave] = toff;
        red[2][wave] = na;
    }
    __syncthreads();
    off = toff = na = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        off += red[0][w];
        toff += red[1][w];
        na += red[2][w];
    }
    const int cnt = hist[e];
    const int ntl = cnt >= cold_max ? (cnt + MFMA_BN - 1) / MFMA_BN : 0;  // this expert's tiles
    if (tid == 0) {
        o.counts[e] = cnt;
        o.offs[e] = off;
        if (cnt > 0) o.act[na] = e;
        else o.slots[E - 1 - (e - na)] = make_int4(0, 0, 0, 0);  // inactive experts fill slots n_act..E-1
        if (e == E - 1) {
            o.offs[E] = off + cnt;
            *o.n_act = na + (cnt > 0);
            *o.n_tiles = toff + ntl;
        }
    }
    for (int i = tid; i < ntl; i += DISPATCH_THREADS)
        o.tiles[toff + i] = make_int4(e, off + i * MFMA_BN, min(MFMA_BN, cnt - i * MFMA_BN), 0);
    if (cnt == 0) return;  // block-uniform
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    // loads per lane and round: up to DP_U, fewer when the pairs fit, so every wave takes a share
    const int U = min(DP_U, (nk + NW * 256 - 1) / (NW * 256));
    int run = off;
    for (int r0 = 0, par = 0; r0 < nk; r0 += NW * 256 * U, par ^= 1) {
        const int wbase = r0 + wave * 256 * U;
        uint64_t bits = 0;  // bit 4u + c: id wbase + 256u + 4 lane + c is expert e
#pragma unroll
        for (int u = 0; u < DP_U; ++u) {
            if (u < U) {  // uniform
                const int4 v = load_ids4(ids, wbase + 256 * u + 4 * lane, nk);
                const uint32_t m = (v.x == e) | (v.y == e) << 1 | (v.z == e) << 2 | (v.w == e) << 3;
                bits |= (uint64_t)m << (4 * u);
            }
        }
        int wt = __popcll(bits);
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) wt += __shfl_xor(wt, m, 64);
        if (lane == 0) wtot[par][wave] = wt;
        __syncthreads();  // wtot[par] complete; the previous round's readers of wtot[par ^ 1] are done
        int p = run, total = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            p += w < wave ? wtot[par][w] : 0;
            total += wtot[par][w];
        }
        for (int u = 0; u < U; ++u) {
            const uint32_t m = (uint32_t)(bits >> (4 * u)) & 15u;
            if (__ballot(m != 0) == 0) continue;  // wave-uniform
            const int c = __popc(m);
            const uint64_t b0 = __ballot(c & 1), b1 = __ballot(c & 2), b2 = __ballot(c & 4);
            int q = p + __popcll(b0 & lt_mask) + 2 * __popcll(b1 & lt_mask) + 4 * __popcll(b2 & lt_mask);
            const int f0 = wbase + 256 * u + 4 * lane;
            for (int x = 0; x < 4; ++x) {
                if ((m >> x) & 1u) {
                    const int f = f0 + x;
                    o.pair_tok[q] = f / top_k;
                    o.pos_of[f] = q;
                    if (q == off) o.slots[na] = make_int4(e, off, cnt, f / top_k);
                    ++q;
                }
            }
            p += __popcll(b0) + 2 * __popcll(b1) + 4 * __popcll(b2);
        }
        run += total;
    }
}

void launch_dispatch(const int* ids, int nk, int E, int top_k, const DispatchOut& o, hipStream_t st, int cold_max) {
    hipLaunchKernelGGL(k_dispatch, dim3(E), dim3(DISPATCH_THREADS), (size_t)E * sizeof(int), st, ids, nk, E, top_k, o,
                       cold_max);
}

// sum_i x[i] * x[i] over one row in vec_dot_f32's order (src/quant.cpp:2756-2778;
// d % 16 == 0): lane j < 16 of the calling wave runs the fma chain over the
// elements 16 i + j of the chain-major row xs (element 16 i + j at j * S + i),
// lanes 0-7 are the reference's acc0, 8-15 its acc1; then acc0 + acc1 and the
// sequential sum of the 8 lanes.  Every lane of the wave calls it; the result
// is valid in lanes 0-15.
__device__ __forceinline__ float row_sumsq_chain(const float* xs, int S, int m, int lane) {
    const int j = lane & 15;
    float acc = 0.0f;
    if (lane < 16)
        for (int i = 0; i < m; ++i) {
            const float v = xs[j * S + i];
            acc = __builtin_fmaf(v, v, acc);
        }
    const float hi = __shfl_down(acc, 8, 16);
    const float v = acc + hi;  // acc0[j] + acc1[j] for j < 8
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) s += __shfl(v, q, 16);
    return s;
}

// MoETransformerEngine::rms_norm (src/transformer.cpp:67-73) of `rows` rows of
// d floats, one block per row: ss = vec_dot_f32(x, x) in the reference's
// order, inv = 1 / sqrt(ss / d + eps) (IEEE division and square root), then
// out[i] = x[i] * inv * w[i] (w == null: weight 1).
__global__ void __launch_bounds__(256) k_rms_norm(const float* x, const float* w, int d, float eps, float* out) {
    extern __shared__ float xs[];  // chain-major row
    __shared__ float inv_s;
    const size_t row = blockIdx.x;
    const int tid = threadIdx.x, S = d / 16 + 1;  // odd stride: the 16 chains hit distinct banks
    const float* xr = x + row * (size_t)d;
    for (int e = tid; e < d; e += 256) xs[(e & 15) * S + (e >> 4)] = xr[e];
    __syncthreads();
    if (tid < 64) {
        const float ss = row_sumsq_chain(xs, S, d / 16, tid);
        if (tid == 0) inv_s = 1.0f / sqrtf(ss / (float)d + eps);
    }
    __syncthreads();
    const float inv = inv_s;
    float* orow = out + row * (size_t)d;
    for (int e = tid; e < d; e += 256) {
        const float v = xr[e] * inv;
        orow[e] = w ? v * w[e] : v;
    }
}

void launch_rms_norm(const float* x, const float* w, int rows, int d, float eps, float* out, hipStream_t st) {
    const size_t lds = (size_t)16 * (d / 16 + 1) * sizeof(float);
    if (lds > 65536)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_rms_norm), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)lds);
    hipLaunchKernelGGL(k_rms_norm, dim3((unsigned)rows), dim3(256), lds, st, x, w, d, eps, out);
}

// MoE combine (transformer.cpp:2728-2730 and 2752-2754): starting from 0, for
// each selected expert in descending-logit order acc = fma(p, y, acc), then
// acc = fma(shared_scale, y_shared, acc).
// Four consecutive features of one token per thread (d % 32 == 0), 16-byte loads and stores; the
// per-feature order is k_combine's contract (fma in selection order, then the shared expert).
template <int KU>  // slots whose loads go out together (the fma order stays the selection order)
__global__ void __launch_bounds__(256)
k_combine(int n, int d, int k, const float* probs, const int* pos_of, const float* y, const float* ysh,
          const float* shscale, const float* resid, float* out, const float* y2, int shparts) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;  // float4 index
    const int d4 = d / 4;
    if (idx >= (size_t)n * d4) return;
    const int t = (int)(idx / d4), i = 4 * (int)(idx % d4);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s0 = 0; s0 < k; s0 += KU) {
        int p[KU];
        float w[KU];
        float4 v[KU];
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const int s = min(s0 + u, k - 1);
            p[u] = pos_of[(size_t)t * k + s];
            w[u] = probs[(size_t)t * k + s];
        }
#pragma unroll
        for (int u = 0; u < KU; ++u) v[u] = *reinterpret_cast<const float4*>(y + (size_t)p[u] * d + i);
        if (y2) {  // the K-split down GEMM's second part
#pragma unroll
            for (int u = 0; u < KU; ++u) {
                const float4 b = *reinterpret_cast<const float4*>(y2 + (size_t)p[u] * d + i);
                v[u] = make_float4(v[u].x + b.x, v[u].y + b.y, v[u].z + b.z, v[u].w + b.w);
            }
        }
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            if (s0 + u < k) {
                acc.x = __builtin_fmaf(w[u], v[u].x, acc.x);
                acc.y = __builtin_fmaf(w[u], v[u].y, acc.y);
                acc.z = __builtin_fmaf(w[u], v[u].z, acc.z);
                acc.w = __builtin_fmaf(w[u], v[u].w, acc.w);
            }
        }
    }
    if (ysh) {
        const float w = shscale[t];
        float4 v = *reinterpret_cast<const float4*>(ysh + (size_t)t * d + i);
        for (int q = 1; q < shparts; ++q) {  // the K parts of a shared down, in part order
            const float4 b = *reinterpret_cast<const float4*>(ysh + ((size_t)q * n + t) * d + i);
            v = make_float4(v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w);
        }
        acc.x = __builtin_fmaf(w, v.x, acc.x);
        acc.y = __builtin_fmaf(w, v.y, acc.y);
        acc.z = __builtin_fmaf(w, v.z, acc.z);
        acc.w = __builtin_fmaf(w, v.w, acc.w);
    }
    if (resid) {  // the residual add after the block (transformer.cpp:2762-2764)
        const float4 r = *reinterpret_cast<const float4*>(resid + (size_t)t * d + i);
        acc = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
    }
    *reinterpret_cast<float4*>(out + (size_t)t * d + i) = acc;
}

// The combine of one token per block followed by post_ffw_norm
// (transformer.cpp:2758-2760: rms_norm of moe_accum in place) and the residual
// add (2762-2764): out = resid + rms_norm(acc, post_w).  acc as k_combine
// computes it, staged chain-major for the exact vec_dot_f32 order of the norm.
__global__ void __launch_bounds__(256)
k_combine_norm(int n, int d, int k, const float* probs, const int* pos_of, const float* y, const float* ysh,
               const float* shscale, const float* post_w, float eps, const float* resid, float* out, const float* y2,
               int shparts) {
    extern __shared__ float as[];  // chain-major acc row
    __shared__ float inv_s;
    const int t = blockIdx.x, tid = threadIdx.x, S = d / 16 + 1;
    for (int i = tid; i < d; i += 256) {
        float acc = 0.0f;
        for (int s = 0; s < k; ++s) {
            const float w = probs[(size_t)t * k + s];
            const size_t o = (size_t)pos_of[(size_t)t * k + s] * d + i;
            acc = __builtin_fmaf(w, y2 ? y[o] + y2[o] : y[o], acc);
        }
        if (ysh) {
            float v = ysh[(size_t)t * d + i];
            for (int q = 1; q < shparts; ++q) v += ysh[((size_t)q * n + t) * d + i];
            acc = __builtin_fmaf(shscale[t], v, acc);
        }
        as[(i & 15) * S + (i >> 4)] = acc;
    }
    __syncthreads();
    if (tid < 64) {
        const float ss = row_sumsq_chain(as, S, d / 16, tid);
        if (tid == 0) inv_s = 1.0f / sqrtf(ss / (float)d + eps);
    }
    __syncthreads();
    const float inv = inv_s;
    for (int i = tid; i < d; i += 256) {
        const float v = as[(i & 15) * S + (i >> 4)] * inv * post_w[i];
        out[(size_t)t * d + i] = resid ? resid[(size_t)t * d + i] + v : v;
    }
}

void launch_combine(int n, int d, int k, const float* probs, const int* pos_of, const float* y, const float* ysh,
                    const float* shscale, float* out, hipStream_t st, const float* resid, const float* post_w,
                    float eps, const float* y2, int shparts) {
    if (post_w) {
        const size_t lds = (size_t)16 * (d / 16 + 1) * sizeof(float);
        if (lds > 65536)
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(k_combine_norm),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        hipLaunchKernelGGL(k_combine_norm, dim3((unsigned)n), dim3(256), lds, st, n, d, k, probs, pos_of, y, ysh,
                           shscale, post_w, eps, resid, out, y2, shparts);
        return;
    }
    const size_t tot = (size_t)n * (d / 4);
    const dim3 grid((unsigned)((tot + 255) / 256));
    if (k <= 2)
        hipLaunchKernelGGL(k_combine<2>, grid, dim3(256), 0, st, n, d, k, probs, pos_of, y, ysh, shscale, resid, out,
                           y2, shparts);
    else if (k <= 4)
        hipLaunchKernelGGL(k_combine<4>, grid, dim3(256), 0, st, n, d, k, probs, pos_of, y, ysh, shscale, resid, out,
                           y2, shparts);
    else
        hipLaunchKernelGGL(k_combine<8>, grid, dim3(256), 0, st, n, d, k, probs, pos_of, y, ysh, shscale, resid, out,
                           y2, shparts);
}

// Q8_0 of `rows` rows of K fp32 values (quantize_row_q8_0, src/quant.cpp:1029-1045),
// one 32-block per half-wave.
__global__ void __launch_bounds__(256) k_quant_q8(const float* x, int rows, int K, ActQ8 out) {
    const int nb = K / 32;
    const size_t gid = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int half = (threadIdx.x >> 5) & 1, l32 = threadIdx.x & 31;
    const size_t blk = gid * 2 + half;
    const bool ok = blk < (size_t)rows * nb;
    quant_block(ok ? x[blk * 32 + l32] : 0.0f, l32, ok, out, blk / nb, (int)(blk % nb));
}

// dst[0 .. kpad) = x[0 .. n) followed by zeros: the zero-padded fp32 activation row the
// fp32-activation GEMV reads (written by a kernel, so a captured graph holds no memset node).
__global__ void __launch_bounds__(256) k_copy_pad(const float* x, int n, int kpad, float* dst) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const size_t row = blockIdx.y;
    if (i < kpad) dst[row * kpad + i] = i < n ? x[row * n + i] : 0.0f;
}

void launch_copy_pad(const float* x, int n, int kpad, float* dst, hipStream_t st, int rows) {
    hipLaunchKernelGGL(k_copy_pad, dim3((unsigned)((kpad + 255) / 256), (unsigned)rows), dim3(256), 0, st, x, n, kpad,
                       dst);
}

void launch_quantize_q8(const float* x, int rows, int K, ActQ8 out, hipStream_t st) {
    const size_t blocks = (size_t)rows * (K / 32);
    const size_t waves = (blocks + 1) / 2;
    hipLaunchKernelGGL(k_quant_q8, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, x, rows, K, out);
}

// One thread per (matrix, row, K-unit): scatter a GGUF block into the tile
// layout described in jxmoe_kernels.h.
__global__ void __launch_bounds__(256) k_repack(const uint8_t* raw, QMat m, uint8_t* qs, uint8_t* sc, uint8_t* ex) {
    const size_t units = (size_t)m.n_mats * m.rows * m.nkb;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= units) return;
    const int kb = (int)(idx % m.nkb);
    const size_t er = idx / m.nkb;  // e*rows + r
    const int r = (int)(er % m.rows);
    const int e = (int)(er / m.rows);
    const int rt = r / ROWS_PER_TILE, mm = r % ROWS_PER_TILE;
    const size_t tile = ((size_t)e * m.nrt + rt) * m.nkb + kb;
    if (m.type == T_Q4_0) {
        const uint8_t* src = raw + idx * 18;
        uint8_t* dq = qs + (tile * 32 + mm) * 16;
        for (int i = 0; i < 16; ++i) dq[i] = src[2 + i];
        sc[(tile * 32 + mm) * 2 + 0] = src[0];
        sc[(tile * 32 + mm) * 2 + 1] = src[1];
    } else if (m.type == T_Q8_0) {
        const uint8_t* src = raw + idx * 34;
        for (int h = 0; h < 2; ++h) {
            uint8_t* dq = qs + ((tile * 2 + h) * 32 + mm) * 16;
            for (int i = 0; i < 16; ++i) dq[i] = src[2 + 16 * h + i];
        }
        sc[(tile * 32 + mm) * 2 + 0] = src[0];
        sc[(tile * 32 + mm) * 2 + 1] = src[1];
    } else if (m.type == T_Q5_0) {  // block_q5_0: d, qh (u32), qs[16]
        const uint8_t* src = raw + idx * 22;
        uint8_t* dq = qs + (tile * 32 + mm) * 16;
        for (int i = 0; i < 16; ++i) dq[i] = src[6 + i];
        sc[(tile * 32 + mm) * 2 + 0] = src[0];
        sc[(tile * 32 + mm) * 2 + 1] = src[1];
        for (int i = 0; i < 4; ++i) ex[(tile * 32 + mm) * 4 + i] = src[2 + i];
    } else if (m.type == T_Q6_K) {  // block_q6_K: ql[128], qh[64], scales[16], d
        const uint8_t* src = raw + idx * 210;
        for (int n = 0; n < 2; ++n)
            for (int c = 0; c < 6; ++c) {
                const uint8_t* s = c < 4 ? src + 64 * n + 16 * c : src + 128 + 32 * n + 16 * (c - 4);
                uint8_t* dq = qs + (((tile * 2 + n) * 6 + c) * 32 + mm) * 16;
                for (int i = 0; i < 16; ++i) dq[i] = s[i];
            }
        for (int i = 0; i < 16; ++i) sc[(tile * 32 + mm) * 16 + i] = src[192 + i];
        ex[(tile * 32 + mm) * 2 + 0] = src[208];
        ex[(tile * 32 + mm) * 2 + 1] = src[209];
    } else {  // Q4_K (144 B: header, qs[128]) or Q5_K (176 B: header, qh[32], qs[128])
        const bool q5 = m.type == T_Q5_K;
        const uint8_t* src = raw + idx * (q5 ? 176 : 144);
        const uint8_t* sq = src + (q5 ? 48 : 16);
        uint8_t* dh = sc + (tile * 32 + mm) * 16;
        for (int i = 0; i < 16; ++i) dh[i] = src[i];
        for (int p = 0; p < 4; ++p)
            for (int h = 0; h < 2; ++h) {
                uint8_t* dq = qs + (((tile * 4 + p) * 2 + h) * 32 + mm) * 16;
                for (int i = 0; i < 16; ++i) dq[i] = sq[32 * p + 16 * h + i];
            }
        if (q5)
            for (int h = 0; h < 2; ++h)
                for (int i = 0; i < 16; ++i) ex[((tile * 2 + h) * 32 + mm) * 16 + i] = src[16 + 16 * h + i];
    }
}

void launch_repack(const uint8_t* raw, QMat m, uint8_t* qs, uint8_t* sc, uint8_t* ex, hipStream_t st) {
    const size_t units = (size_t)m.n_mats * m.rows * m.nkb;
    hipLaunchKernelGGL(k_repack, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, st, raw, m, qs, sc, ex);
}

}  // namespace jx

// Decode regime (few tokens per expert): bandwidth-bound dequant-GEMV.
//
// A block owns one 32-row tile of one active expert's matrix (or two: gate
// and up) and every token routed to that expert; its waves split K.  Lane
// (m = lane % 32, h = lane / 32) streams 16-byte chunks of row m -- the 32
// lanes of a half-wave read one contiguous 512-byte run of the tile layout --
// and multiplies them against the tokens' Q8_0 activations with
// v_dot4_i32_i8.  The next K-unit's chunks are loaded before the current one
// is consumed.  Integer block sums are exact; each is scaled once in fp32
// (weight scale x activation scale) as in the reference's vec_dot_*_q8_0
// kernels (src/quant.cpp:3307-3573); only the fp32 summation order differs.
#include "jxmoe_device.h"
#include "jxmoe_kernels.h"

namespace jx {

// ------------------------------------------------------------ weight chunks
// Q4_0 / Q8_0: unit = one 32-block.  Q4_0 lanes of half h take the blocks of
// parity h; Q8_0 lanes take half h of every block.  Q4_K: unit = one
// 256-element super-block, lanes take half h of each of its 4 sub-block pairs.
struct Raw32 {
    uint4 q;
    uint32_t d;  // fp16 bits of the block scale
};
struct RawQ4K {
    uint4 q[4];
    uint4 hd;  // d | dmin << 16, then the 12 scale bytes
};

template <int TYPE>
struct Fmt;

template <>
struct Fmt<T_Q4_0> {
    using Raw = Raw32;
    static constexpr bool PARITY = true;
    __device__ static Raw load(const QMat& W, int e, int rt, int u, int m, int h) {
        (void)h;
        const size_t t = ((size_t)rt * W.nkb + u) * 32 + m;
        Raw c;
        c.q = ld_stream16(W.qs + e * W.qs_es + t * 16);
        c.d = reinterpret_cast<const uint16_t*>(W.sc + e * W.sc_es)[t];
        return c;
    }
};

template <>
struct Fmt<T_Q8_0> {
    using Raw = Raw32;
    static constexpr bool PARITY = false;
    __device__ static Raw load(const QMat& W, int e, int rt, int u, int m, int h) {
        const size_t t = (size_t)rt * W.nkb + u;
        Raw c;
        c.q = ld_stream16(W.qs + e * W.qs_es + ((t * 2 + h) * 32 + m) * 16);
        c.d = reinterpret_cast<const uint16_t*>(W.sc + e * W.sc_es)[t * 32 + m];
        return c;
    }
};

template <>
struct Fmt<T_Q4_K> {
    using Raw = RawQ4K;
    static constexpr bool PARITY = false;
    __device__ static Raw load(const QMat& W, int e, int rt, int u, int m, int h) {
        const size_t t = (size_t)rt * W.nkb + u;
        const uint8_t* qb = W.qs + e * W.qs_es;
        Raw c;
#pragma unroll
        for (int p = 0; p < 4; ++p) c.q[p] = ld_stream16(qb + (((t * 4 + p) * 2 + h) * 32 + m) * 16);
        c.hd = ld_stream16(W.sc + e * W.sc_es + (t * 32 + m) * 16);
        return c;
    }
};

__device__ __forceinline__ uint32_t byte_of(const uint4& v, int i) {
    const uint32_t w = i < 4 ? v.y : (i < 8 ? v.z : v.w);
    return (w >> (8 * (i & 3))) & 0xFFu;
}

// (scale, min) of sub-block j from a Q4_K header held in registers
// (get_scale_min_k4, src/quant.cpp:1107-1115).
__device__ __forceinline__ void hd_scale_min(const uint4& hd, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = byte_of(hd, j) & 63;
        mn = byte_of(hd, j + 4) & 63;
    } else {
        sc = (byte_of(hd, j + 4) & 0x0F) | ((byte_of(hd, j - 4) >> 6) << 4);
        mn = (byte_of(hd, j + 4) >> 4) | ((byte_of(hd, j) >> 6) << 4);
    }
}

// Accumulate one K-unit of one weight row against up to TB activation rows
// (Q8_0 activations).
template <int TYPE, int TB>
__device__ __forceinline__ void unit_accum(const typename Fmt<TYPE>::Raw& c, const int8_t* const* arow,
                                           const float2* const* as, int u, int h, int nt, float* acc) {
    if constexpr (TYPE == T_Q4_0) {
        const float dw = f16_to_f32(c.d);
        const uint32_t q[4] = {c.q.x, c.q.y, c.q.z, c.q.w};
        int ql[4], qh[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ql[i] = (int)(q[i] & 0x0F0F0F0Fu);
            qh[i] = (int)((q[i] >> 4) & 0x0F0F0F0Fu);
        }
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            if (j < nt) {
                const uint4 a0 = ld16(arow[j] + u * 32);
                const uint4 a1 = ld16(arow[j] + u * 32 + 16);
                const float2 s = as[j][u];
                int isum = sdot4(ql[0], (int)a0.x, 0);
                isum = sdot4(ql[1], (int)a0.y, isum);
                isum = sdot4(ql[2], (int)a0.z, isum);
                isum = sdot4(ql[3], (int)a0.w, isum);
                isum = sdot4(qh[0], (int)a1.x, isum);
                isum = sdot4(qh[1], (int)a1.y, isum);
                isum = sdot4(qh[2], (int)a1.z, isum);
                isum = sdot4(qh[3], (int)a1.w, isum);
                isum -= 8 * (int)s.y;  // weights are nibble - 8
                acc[j] = __builtin_fmaf(dw * s.x, (float)isum, acc[j]);
            }
        }
    } else if constexpr (TYPE == T_Q8_0) {
        const float dw = f16_to_f32(c.d);
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            if (j < nt) {
                const uint4 a = ld16(arow[j] + u * 32 + 16 * h);
                const float2 s = as[j][u];
                int isum = sdot4((int)c.q.x, (int)a.x, 0);
                isum = sdot4((int)c.q.y, (int)a.y, isum);
                isum = sdot4((int)c.q.z, (int)a.z, isum);
                isum = sdot4((int)c.q.w, (int)a.w, isum);
                acc[j] = __builtin_fmaf(dw * s.x, (float)isum, acc[j]);
            }
        }
    } else {
        const float d = f16_to_f32(c.hd.x & 0xFFFFu), dmin = f16_to_f32(c.hd.x >> 16);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            int s0, m0, s1, m1;
            hd_scale_min(c.hd, 2 * p, s0, m0);
            hd_scale_min(c.hd, 2 * p + 1, s1, m1);
            const float fs0 = d * (float)s0, fm0 = dmin * (float)m0;
            const float fs1 = d * (float)s1, fm1 = dmin * (float)m1;
            const uint32_t q[4] = {c.q[p].x, c.q[p].y, c.q[p].z, c.q[p].w};
            int ql[4], qh[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ql[i] = (int)(q[i] & 0x0F0F0F0Fu);
                qh[i] = (int)((q[i] >> 4) & 0x0F0F0F0Fu);
            }
            const int b0 = u * 8 + 2 * p;
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                if (j < nt) {
                    const uint4 a = ld16(arow[j] + b0 * 32 + 16 * h);
                    const uint4 b = ld16(arow[j] + (b0 + 1) * 32 + 16 * h);
                    const float2 sa = as[j][b0], sb = as[j][b0 + 1];
                    int ia = sdot4(ql[0], (int)a.x, 0);
                    ia = sdot4(ql[1], (int)a.y, ia);
                    ia = sdot4(ql[2], (int)a.z, ia);
                    ia = sdot4(ql[3], (int)a.w, ia);
                    int ib = sdot4(qh[0], (int)b.x, 0);
                    ib = sdot4(qh[1], (int)b.y, ib);
                    ib = sdot4(qh[2], (int)b.z, ib);
                    ib = sdot4(qh[3], (int)b.w, ib);
                    float v = acc[j];
                    v = __builtin_fmaf(fs0 * sa.x, (float)ia, v);
                    v = __builtin_fmaf(fs1 * sb.x, (float)ib, v);
                    if (h == 0) {  // min term once per sub-block: sum(y) over all 32 elements
                        v = __builtin_fmaf(-(fm0 * sa.x), sa.y, v);
                        v = __builtin_fmaf(-(fm1 * sb.x), sb.y, v);
                    }
                    acc[j] = v;
                }
            }
        }
    }
}

// Q4_K against fp32 activations (the reference's vec_dot_q4_K_f32 fallback,
// src/quant.cpp:2910-3013, used when K % 256 != 0): rows of y are zero-padded
// to whole super-blocks, so the partial last super-block needs no masking.
template <int TB>
__device__ __forceinline__ void unit_accum_f32(const RawQ4K& c, const float* const* yrow, int u, int h, int nt,
                                               float* acc) {
    const float d = f16_to_f32(c.hd.x & 0xFFFFu), dmin = f16_to_f32(c.hd.x >> 16);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        int s0, m0, s1, m1;
        hd_scale_min(c.hd, 2 * p, s0, m0);
        hd_scale_min(c.hd, 2 * p + 1, s1, m1);
        const float fs0 = d * (float)s0, fm0 = dmin * (float)m0;
        const float fs1 = d * (float)s1, fm1 = dmin * (float)m1;
        const uint32_t q[4] = {c.q[p].x, c.q[p].y, c.q[p].z, c.q[p].w};
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            if (j < nt) {
                const float* ya = yrow[j] + u * 256 + 64 * p + 16 * h;
                const float* yb = ya + 32;
                float sa = 0.0f, sb = 0.0f, ta = 0.0f, tb = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 va = *reinterpret_cast<const float4*>(ya + 4 * i);
                    const float4 vb = *reinterpret_cast<const float4*>(yb + 4 * i);
                    const float fa[4] = {va.x, va.y, va.z, va.w};
                    const float fb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
                    for (int z = 0; z < 4; ++z) {
                        const uint32_t byte = (q[i] >> (8 * z)) & 0xFFu;
                        sa = __builtin_fmaf((float)(byte & 15u), fa[z], sa);
                        sb = __builtin_fmaf((float)(byte >> 4), fb[z], sb);
                        ta = ta + fa[z];
                        tb = tb + fb[z];
                    }
                }
                float v = acc[j];
                v = __builtin_fmaf(fs0, sa, v);
                v = __builtin_fmaf(-fm0, ta, v);
                v = __builtin_fmaf(fs1, sb, v);
                v = __builtin_fmaf(-fm1, tb, v);
                acc[j] = v;
            }
        }
    }
}

// K-units handled by lane (wave, h) of a WAVES-wave block: [lo, hi) by `step`.
template <int TYPE, int WAVES>
__device__ __forceinline__ void unit_range(int nkb, int wave, int h, int& lo, int& hi, int& step) {
    if (Fmt<TYPE>::PARITY) {
        const int npair = (nkb + 1) / 2;
        const int per = (npair + WAVES - 1) / WAVES;
        lo = 2 * (wave * per) + h;
        hi = min(nkb, 2 * ((wave + 1) * per));
        step = 2;
    } else {
        const int per = (nkb + WAVES - 1) / WAVES;
        lo = wave * per;
        hi = min(nkb, (wave + 1) * per);
        step = 1;
    }
}

__device__ __forceinline__ void group_of(const Groups& g, int slot, int& e, int& p0, int& cnt) {
    if (g.identity) {
        e = 0;
        p0 = 0;
        cnt = slot == 0 ? g.n_tok : 0;
    } else if (slot < *g.n_act) {
        e = g.act[slot];
        p0 = g.offs[e];
        cnt = g.counts[e];
    } else {
        e = 0;
        p0 = 0;
        cnt = 0;
    }
}

__device__ __forceinline__ int token_of(const Groups& g, int p) {
    return g.identity ? p : g.pair_tok[p];
}

// Q8_0 of one 32-row block of h held by lanes 0..31 (quantize_row_q8_0).
__device__ __forceinline__ void store_q8_block(float hv, int m, bool writer, ActQ8& hq, size_t row, int blk) {
    const float amax = wave_max32(__builtin_fabsf(hv));
    const float dd = amax / 127.0f;
    const float id = (dd != 0.0f) ? 1.0f / dd : 0.0f;
    float r = round_away(hv * id);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    const int q = (int)r;
    const int s = wave_sum32i(q);
    if (writer) {
        hq.q[row * hq.K + blk * 32 + m] = (int8_t)q;
        if (m == 0) hq.s[row * (hq.K / 32) + blk] = make_float2(f16_to_f32(f32_to_f16_trunc(dd)), (float)s);
    }
}

// Gate + up + SwiGLU (matmul_swiglu_quant_f32, src/quant.cpp:3970-4009) and
// the Q8_0 quantization of the result for the down projection
// (matmul_quant_f32's quantize_row_q8_0, 3908-3914).
template <int TYPE, int TB, int WAVES>
__global__ void __launch_bounds__(WAVES * 64)
k_gemv_gateup(QMat G, QMat U, ActQ8 xq, Groups grp, ActQ8 hq, float* hf, int hf_ld) {
    using F = Fmt<TYPE>;
    __shared__ float red[WAVES][TB][2][32];
    const int rt = blockIdx.x;
    int e, p0, cnt;
    group_of(grp, blockIdx.y, e, p0, cnt);
    if (cnt == 0) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 31, h = lane >> 5;
    const int K = xq.K, KB = K / 32;
    int lo, hi, step;
    unit_range<TYPE, WAVES>(G.nkb, wave, h, lo, hi, step);
    for (int tb0 = 0; tb0 < cnt; tb0 += TB) {
        const int nt = min(TB, cnt - tb0);
        const int8_t* arow[TB];
        const float2* as[TB];
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            const int tok = token_of(grp, p0 + tb0 + min(j, nt - 1));
            arow[j] = xq.q + (size_t)tok * K;
            as[j] = xq.s + (size_t)tok * KB;
        }
        float ag[TB], au[TB];
#pragma unroll
        for (int j = 0; j < TB; ++j) ag[j] = au[j] = 0.0f;
        if (lo < hi) {
            auto cg = F::load(G, e, rt, lo, m, h);
            auto cu = F::load(U, e, rt, lo, m, h);
            for (int u = lo; u < hi; u += step) {
                const int un = min(u + step, hi - 1);
                const auto ng = F::load(G, e, rt, un, m, h);
                const auto nu = F::load(U, e, rt, un, m, h);
                unit_accum<TYPE, TB>(cg, arow, as, u, h, nt, ag);
                unit_accum<TYPE, TB>(cu, arow, as, u, h, nt, au);
                cg = ng;
                cu = nu;
            }
        }
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            ag[j] += __shfl_xor(ag[j], 32, 64);
            au[j] += __shfl_xor(au[j], 32, 64);
            if (h == 0) {
                red[wave][j][0][m] = ag[j];
                red[wave][j][1][m] = au[j];
            }
        }
        __syncthreads();
        if (wave == 0) {
            for (int j = 0; j < nt; ++j) {
                float g = 0.0f, u = 0.0f;
#pragma unroll
                for (int w = 0; w < WAVES; ++w) {
                    g += red[w][j][0][m];
                    u += red[w][j][1][m];
                }
                const float hv = (g / (1.0f + expf(-g))) * u;
                const size_t row = (size_t)(p0 + tb0 + j);
                store_q8_block(hv, m, h == 0 && hq.q != nullptr, hq, row, rt);
                if (hf && h == 0) hf[row * (size_t)hf_ld + rt * 32 + m] = hv;
            }
        }
        __syncthreads();
    }
}

// Down projection into y[pair][rows].
template <int TYPE, int TB, int WAVES, bool F32ACT>
__global__ void __launch_bounds__(WAVES * 64)
k_gemv_down(QMat D, ActQ8 hq, const float* hf, int hf_ld, Groups grp, float* y) {
    using F = Fmt<TYPE>;
    __shared__ float red[WAVES][TB][32];
    const int rt = blockIdx.x;
    int e, p0, cnt;
    group_of(grp, blockIdx.y, e, p0, cnt);
    if (cnt == 0) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 31, h = lane >> 5;
    int lo, hi, step;
    unit_range<TYPE, WAVES>(D.nkb, wave, h, lo, hi, step);
    const int K = hq.K, KB = K / 32;
    for (int tb0 = 0; tb0 < cnt; tb0 += TB) {
        const int nt = min(TB, cnt - tb0);
        const int8_t* arow[TB];
        const float2* as[TB];
        const float* yrow[TB];
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            const size_t row = (size_t)(p0 + tb0 + min(j, nt - 1));
            arow[j] = F32ACT ? nullptr : hq.q + row * K;
            as[j] = F32ACT ? nullptr : hq.s + row * KB;
            yrow[j] = F32ACT ? hf + row * (size_t)hf_ld : nullptr;
        }
        float acc[TB];
#pragma unroll
        for (int j = 0; j < TB; ++j) acc[j] = 0.0f;
        if (lo < hi) {
            auto c = F::load(D, e, rt, lo, m, h);
            for (int u = lo; u < hi; u += step) {
                const auto nc = F::load(D, e, rt, min(u + step, hi - 1), m, h);
                if constexpr (F32ACT)
                    unit_accum_f32<TB>(c, yrow, u, h, nt, acc);
                else
                    unit_accum<TYPE, TB>(c, arow, as, u, h, nt, acc);
                c = nc;
            }
        }
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            acc[j] += __shfl_xor(acc[j], 32, 64);
            if (h == 0) red[wave][j][m] = acc[j];
        }
        __syncthreads();
        if (wave == 0 && h == 0) {
            for (int j = 0; j < nt; ++j) {
                float s = 0.0f;
#pragma unroll
                for (int w = 0; w < WAVES; ++w) s += red[w][j][m];
                y[(size_t)(p0 + tb0 + j) * D.rows + rt * 32 + m] = s;
            }
        }
        __syncthreads();
    }
}

constexpr int GATEUP_WAVES = 4;
constexpr int DOWN_WAVES = 8;

template <int TYPE>
static void gateup_t(const QMat& g, const QMat& u, const ActQ8& xq, const Groups& grp, int slots, int tb,
                     ActQ8 hq, float* hf, hipStream_t st) {
    dim3 grid(g.nrt, slots);
    const int hf_ld = ((g.rows + 255) / 256) * 256;
    if (tb <= 1)
        hipLaunchKernelGGL((k_gemv_gateup<TYPE, 1, GATEUP_WAVES>), grid, dim3(GATEUP_WAVES * 64), 0, st, g, u, xq,
                           grp, hq, hf, hf_ld);
    else
        hipLaunchKernelGGL((k_gemv_gateup<TYPE, 4, GATEUP_WAVES>), grid, dim3(GATEUP_WAVES * 64), 0, st, g, u, xq,
                           grp, hq, hf, hf_ld);
}

void launch_gemv_gateup(const QMat& g, const QMat& u, const ActQ8& xq, const Groups& grp, int slots, int tb,
                        ActQ8 hq, float* hf, hipStream_t st) {
    switch (g.type) {
        case T_Q4_0: gateup_t<T_Q4_0>(g, u, xq, grp, slots, tb, hq, hf, st); break;
        case T_Q8_0: gateup_t<T_Q8_0>(g, u, xq, grp, slots, tb, hq, hf, st); break;
        case T_Q4_K: gateup_t<T_Q4_K>(g, u, xq, grp, slots, tb, hq, hf, st); break;
        default: break;
    }
}

template <int TYPE, bool F32ACT>
static void down_t(const QMat& dn, const ActQ8& hq, const float* hf, int hf_ld, const Groups& grp, int slots,
                   int tb, float* y, hipStream_t st) {
    dim3 grid(dn.nrt, slots);
    if (tb <= 1)
        hipLaunchKernelGGL((k_gemv_down<TYPE, 1, DOWN_WAVES, F32ACT>), grid, dim3(DOWN_WAVES * 64), 0, st, dn, hq,
                           hf, hf_ld, grp, y);
    else
        hipLaunchKernelGGL((k_gemv_down<TYPE, 4, DOWN_WAVES, F32ACT>), grid, dim3(DOWN_WAVES * 64), 0, st, dn, hq,
                           hf, hf_ld, grp, y);
}

void launch_gemv_down(const QMat& dn, const ActQ8& hq, const float* hf, int hf_ld, const Groups& grp, int slots,
                      int tb, float* y, hipStream_t st) {
    if (hf) {
        down_t<T_Q4_K, true>(dn, hq, hf, hf_ld, grp, slots, tb, y, st);
        return;
    }
    switch (dn.type) {
        case T_Q4_0: down_t<T_Q4_0, false>(dn, hq, hf, hf_ld, grp, slots, tb, y, st); break;
        case T_Q8_0: down_t<T_Q8_0, false>(dn, hq, hf, hf_ld, grp, slots, tb, y, st); break;
        case T_Q4_K: down_t<T_Q4_K, false>(dn, hq, hf, hf_ld, grp, slots, tb, y, st); break;
        default: break;
    }
}

}  // namespace jx

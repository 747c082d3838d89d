// Decode regime (few tokens per expert): bandwidth-bound dequant-GEMV.
//
// A block owns one 32-row tile of one active expert's matrix (or two: gate
// and up) and every token routed to that expert; its 16 waves split K.  Lane
// (m = lane % 32, h = lane / 32) streams 16-byte chunks of row m -- the 32
// lanes of a half-wave read one contiguous 512-byte run of the tile layout --
// and multiplies them against the token's Q8_0 activations with v_dot4_i32_i8.
// Integer block sums are exact; each is scaled once in fp32 (weight scale x
// activation scale), as the reference's vec_dot_*_q8_0 kernels do
// (src/quant.cpp:3307-3573), only the fp32 summation order differs.
#include "jxmoe_device.h"
#include "jxmoe_kernels.h"

namespace jx {

constexpr int GEMV_WAVES = 16;
constexpr int GEMV_THREADS = GEMV_WAVES * 64;

// ------------------------------------------------------------ weight chunks
// Q4_0: unit = one 32-block; lane h takes blocks of parity h.
struct ChunkQ4_0 {
    uint4 q;
    float d;
};
// Q8_0: unit = one 32-block; lane h takes half h of it.
struct ChunkQ8_0 {
    uint4 q;
    float d;
};
// Q4_K: unit = one 256 super-block; lane h takes half h of each of the 4
// sub-block pairs.
struct ChunkQ4_K {
    uint4 q[4];
    float dsc[8];
    float dmn[8];
};

template <int TYPE>
struct Traits;

template <>
struct Traits<T_Q4_0> {
    using Chunk = ChunkQ4_0;
    static constexpr int UNIT = 32;  // elements per K-unit
    // lane h processes units u with u % 2 == h
    static constexpr bool SPLIT_BY_PARITY = true;
    __device__ static Chunk load(const QMat& W, int e, int rt, int u, int m, int h) {
        (void)h;
        Chunk c;
        const size_t t = ((size_t)rt * W.nkb + u) * 32 + m;
        c.q = ld_stream16(W.qs + e * W.qs_es + t * 16);
        c.d = f16_to_f32(reinterpret_cast<const uint16_t*>(W.sc + e * W.sc_es)[t]);
        return c;
    }
    // Q8_0 activations: isum over the block, minus 8 * (sum of activations)
    __device__ static float dot(const Chunk& c, const int8_t* arow, const float2* as, int u, int h, float acc) {
        (void)h;
        const uint4 a0 = ld16(arow + u * 32);
        const uint4 a1 = ld16(arow + u * 32 + 16);
        const float2 s = as[u];
        const uint32_t q[4] = {c.q.x, c.q.y, c.q.z, c.q.w};
        const uint32_t lo[4] = {a0.x, a0.y, a0.z, a0.w};
        const uint32_t hi[4] = {a1.x, a1.y, a1.z, a1.w};
        int isum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            isum = sdot4((int)(q[i] & 0x0F0F0F0Fu), (int)lo[i], isum);
            isum = sdot4((int)((q[i] >> 4) & 0x0F0F0F0Fu), (int)hi[i], isum);
        }
        isum -= 8 * (int)s.y;
        return __builtin_fmaf(c.d * s.x, (float)isum, acc);
    }
};

template <>
struct Traits<T_Q8_0> {
    using Chunk = ChunkQ8_0;
    static constexpr int UNIT = 32;
    static constexpr bool SPLIT_BY_PARITY = false;
    __device__ static Chunk load(const QMat& W, int e, int rt, int u, int m, int h) {
        Chunk c;
        const size_t t = (size_t)rt * W.nkb + u;
        c.q = ld_stream16(W.qs + e * W.qs_es + ((t * 2 + h) * 32 + m) * 16);
        c.d = f16_to_f32(reinterpret_cast<const uint16_t*>(W.sc + e * W.sc_es)[t * 32 + m]);
        return c;
    }
    __device__ static float dot(const Chunk& c, const int8_t* arow, const float2* as, int u, int h, float acc) {
        const uint4 a = ld16(arow + u * 32 + 16 * h);
        const float2 s = as[u];
        int isum = 0;
        isum = sdot4((int)c.q.x, (int)a.x, isum);
        isum = sdot4((int)c.q.y, (int)a.y, isum);
        isum = sdot4((int)c.q.z, (int)a.z, isum);
        isum = sdot4((int)c.q.w, (int)a.w, isum);
        return __builtin_fmaf(c.d * s.x, (float)isum, acc);
    }
};

template <>
struct Traits<T_Q4_K> {
    using Chunk = ChunkQ4_K;
    static constexpr int UNIT = 256;
    static constexpr bool SPLIT_BY_PARITY = false;
    __device__ static Chunk load(const QMat& W, int e, int rt, int u, int m, int h) {
        Chunk c;
        const size_t t = (size_t)rt * W.nkb + u;
        const uint8_t* qb = W.qs + e * W.qs_es;
#pragma unroll
        for (int p = 0; p < 4; ++p) c.q[p] = ld_stream16(qb + (((t * 4 + p) * 2 + h) * 32 + m) * 16);
        const uint4 hd = ld_stream16(W.sc + e * W.sc_es + (t * 32 + m) * 16);
        const float d = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
        const uint32_t sw[3] = {hd.y, hd.z, hd.w};
        const uint8_t* s = reinterpret_cast<const uint8_t*>(sw);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            int sc, mn;
            q4k_scale_min(j, s, sc, mn);
            c.dsc[j] = d * (float)sc;
            c.dmn[j] = dmin * (float)mn;
        }
        return c;
    }
    // Q8_0 activations (the reference's vec_dot_q4_K_q8_0): per sub-block,
    // d*sc*dx*sum(q*y) - dmin*m*dx*sum(y); the min term is added once per
    // sub-block (by the h == 0 lanes).
    __device__ static float dot(const Chunk& c, const int8_t* arow, const float2* as, int u, int h, float acc) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int b0 = u * 8 + 2 * p;
            const uint4 a = ld16(arow + b0 * 32 + 16 * h);
            const uint4 b = ld16(arow + (b0 + 1) * 32 + 16 * h);
            const float2 s0 = as[b0], s1 = as[b0 + 1];
            const uint32_t q[4] = {c.q[p].x, c.q[p].y, c.q[p].z, c.q[p].w};
            const uint32_t av[4] = {a.x, a.y, a.z, a.w};
            const uint32_t bv[4] = {b.x, b.y, b.z, b.w};
            int ia = 0, ib = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ia = sdot4((int)(q[i] & 0x0F0F0F0Fu), (int)av[i], ia);
                ib = sdot4((int)((q[i] >> 4) & 0x0F0F0F0Fu), (int)bv[i], ib);
            }
            acc = __builtin_fmaf(c.dsc[2 * p] * s0.x, (float)ia, acc);
            acc = __builtin_fmaf(c.dsc[2 * p + 1] * s1.x, (float)ib, acc);
            if (h == 0) {
                acc = __builtin_fmaf(-(c.dmn[2 * p] * s0.x), s0.y, acc);
                acc = __builtin_fmaf(-(c.dmn[2 * p + 1] * s1.x), s1.y, acc);
            }
        }
        return acc;
    }
    // fp32 activations (the reference's vec_dot_q4_K_f32 fallback when
    // K % 256 != 0): rows of y are zero-padded to whole super-blocks.
    __device__ static float dot_f32(const Chunk& c, const float* y, int u, int h, float acc) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const float* ya = y + u * 256 + 64 * p + 16 * h;
            const float* yb = ya + 32;
            const uint32_t q[4] = {c.q[p].x, c.q[p].y, c.q[p].z, c.q[p].w};
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
            acc = __builtin_fmaf(c.dsc[2 * p], sa, acc);
            acc = __builtin_fmaf(-c.dmn[2 * p], ta, acc);
            acc = __builtin_fmaf(c.dsc[2 * p + 1], sb, acc);
            acc = __builtin_fmaf(-c.dmn[2 * p + 1], tb, acc);
        }
        return acc;
    }
};

// K-units handled by lane (wave, h): [lo, hi) stepping by `step`.
template <int TYPE>
__device__ __forceinline__ void unit_range(int nkb, int wave, int h, int& lo, int& hi, int& step) {
    if (Traits<TYPE>::SPLIT_BY_PARITY) {
        const int npair = (nkb + 1) / 2;
        const int per = (npair + GEMV_WAVES - 1) / GEMV_WAVES;
        lo = 2 * (wave * per) + h;
        hi = min(nkb, 2 * ((wave + 1) * per));
        step = 2;
    } else {
        const int per = (nkb + GEMV_WAVES - 1) / GEMV_WAVES;
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
    return g.identity ? p : g.pair_f[p] / g.top_k;
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
template <int TYPE, int TB>
__global__ void __launch_bounds__(GEMV_THREADS)
k_gemv_gateup(QMat G, QMat U, ActQ8 xq, Groups grp, ActQ8 hq, float* hf, int hf_ld) {
    using Tr = Traits<TYPE>;
    __shared__ float red[GEMV_WAVES][TB][2][32];
    const int rt = blockIdx.x;
    int e, p0, cnt;
    group_of(grp, blockIdx.y, e, p0, cnt);
    if (cnt == 0) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 31, h = lane >> 5;
    const int K = xq.K, KB = K / 32;
    int lo, hi, step;
    unit_range<TYPE>(G.nkb, wave, h, lo, hi, step);
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
        for (int u = lo; u < hi; u += step) {
            const auto cg = Tr::load(G, e, rt, u, m, h);
            const auto cu = Tr::load(U, e, rt, u, m, h);
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                if (j < nt) {
                    ag[j] = Tr::dot(cg, arow[j], as[j], u, h, ag[j]);
                    au[j] = Tr::dot(cu, arow[j], as[j], u, h, au[j]);
                }
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
                for (int w = 0; w < GEMV_WAVES; ++w) {
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

// Down projection into y[slice][pair][rows].
template <int TYPE, int TB, bool F32ACT>
__global__ void __launch_bounds__(GEMV_THREADS)
k_gemv_down(QMat D, ActQ8 hq, const float* hf, int hf_ld, Groups grp, float* y, size_t y_slice, int ksplit) {
    using Tr = Traits<TYPE>;
    __shared__ float red[GEMV_WAVES][TB][32];
    const int rt = blockIdx.x;
    int e, p0, cnt;
    group_of(grp, blockIdx.y, e, p0, cnt);
    if (cnt == 0) return;
    const int slice = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 31, h = lane >> 5;
    // this slice's K-units
    const int per_sl = (D.nkb + ksplit - 1) / ksplit;
    const int u0 = slice * per_sl, u1 = min(D.nkb, u0 + per_sl);
    int lo, hi, step;
    unit_range<TYPE>(u1 - u0, wave, h, lo, hi, step);
    lo += u0;
    hi += u0;
    const int K = hq.K, KB = K / 32;
    for (int tb0 = 0; tb0 < cnt; tb0 += TB) {
        const int nt = min(TB, cnt - tb0);
        float acc[TB];
#pragma unroll
        for (int j = 0; j < TB; ++j) acc[j] = 0.0f;
        for (int u = lo; u < hi; u += step) {
            const auto c = Tr::load(D, e, rt, u, m, h);
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                if (j < nt) {
                    const size_t row = (size_t)(p0 + tb0 + j);
                    if constexpr (F32ACT) {
                        acc[j] = Traits<T_Q4_K>::dot_f32(c, hf + row * hf_ld, u, h, acc[j]);
                    } else {
                        acc[j] = Tr::dot(c, hq.q + row * K, hq.s + row * KB, u, h, acc[j]);
                    }
                }
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
                for (int w = 0; w < GEMV_WAVES; ++w) s += red[w][j][m];
                y[slice * y_slice + (size_t)(p0 + tb0 + j) * D.rows + rt * 32 + m] = s;
            }
        }
        __syncthreads();
    }
}

template <int TYPE>
static void gateup_t(const QMat& g, const QMat& u, const ActQ8& xq, const Groups& grp, int slots, int tb,
                     ActQ8 hq, float* hf, hipStream_t st) {
    dim3 grid(g.nrt, slots);
    const int hf_ld = ((g.rows + 255) / 256) * 256;
    if (tb <= 1)
        hipLaunchKernelGGL((k_gemv_gateup<TYPE, 1>), grid, dim3(GEMV_THREADS), 0, st, g, u, xq, grp, hq, hf, hf_ld);
    else
        hipLaunchKernelGGL((k_gemv_gateup<TYPE, 4>), grid, dim3(GEMV_THREADS), 0, st, g, u, xq, grp, hq, hf, hf_ld);
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
                   int tb, int ksplit, float* y, size_t y_slice, hipStream_t st) {
    dim3 grid(dn.nrt, slots, ksplit);
    if (tb <= 1)
        hipLaunchKernelGGL((k_gemv_down<TYPE, 1, F32ACT>), grid, dim3(GEMV_THREADS), 0, st, dn, hq, hf, hf_ld, grp,
                           y, y_slice, ksplit);
    else
        hipLaunchKernelGGL((k_gemv_down<TYPE, 4, F32ACT>), grid, dim3(GEMV_THREADS), 0, st, dn, hq, hf, hf_ld, grp,
                           y, y_slice, ksplit);
}

void launch_gemv_down(const QMat& dn, const ActQ8& hq, const float* hf, int hf_ld, const Groups& grp, int slots,
                      int tb, int ksplit, float* y, size_t y_slice, hipStream_t st) {
    if (hf) {
        down_t<T_Q4_K, true>(dn, hq, hf, hf_ld, grp, slots, tb, ksplit, y, y_slice, st);
        return;
    }
    switch (dn.type) {
        case T_Q4_0: down_t<T_Q4_0, false>(dn, hq, hf, hf_ld, grp, slots, tb, ksplit, y, y_slice, st); break;
        case T_Q8_0: down_t<T_Q8_0, false>(dn, hq, hf, hf_ld, grp, slots, tb, ksplit, y, y_slice, st); break;
        case T_Q4_K: down_t<T_Q4_K, false>(dn, hq, hf, hf_ld, grp, slots, tb, ksplit, y, y_slice, st); break;
        default: break;
    }
}

}  // namespace jx

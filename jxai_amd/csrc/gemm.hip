// Prefill regime (many tokens per expert): grouped GEMM on the int8 matrix
// cores.
//
// The dispatch kernel sorted (token, slot) pairs by expert and cut each
// expert's pairs into tiles of 32.  A block owns 128 weight rows (4 waves x
// one 32-row tile) of the tile's expert and those 32 pairs.  Per 32-element
// K-block a wave issues v_mfma_i32_32x32x32_i8 with the weight rows as A
// (Q4 nibbles unpacked to int8) and the pairs' Q8_0 activations as B; the
// exact i32 block sums are scaled in fp32 by (weight scale x activation
// scale) in the epilogue -- the arithmetic of the reference's
// vec_dot_*_q8_0 kernels (src/quant.cpp:3307-3573) with a different fp32
// summation order.
//
// Output layout of a 32x32 i32 tile: lane l, register r holds
// D[row = 8*(r/4) + 4*(l/32) + r%4][col = l%32].
#include "jxmoe_device.h"
#include "jxmoe_kernels.h"

namespace jx {

constexpr int MFMA_WAVES = 4;
constexpr int MFMA_THREADS = MFMA_WAVES * 64;

__device__ __forceinline__ uint32_t nib_minus8(uint32_t nib) {
    // bytes n in 0..15 -> int8 (n - 8), no borrow between bytes
    return ((nib | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

template <int TYPE>
__device__ __forceinline__ v4i load_a(const QMat& W, int e, int rt, int kb, int row, int g) {
    const uint8_t* qs = W.qs + e * W.qs_es;
    v4i a;
    if (TYPE == T_Q4_0) {
        const uint4 q = ld16(qs + (((size_t)rt * W.nkb + kb) * 32 + row) * 16);
        const int sh = g ? 4 : 0;
        a.x = (int)nib_minus8((q.x >> sh) & 0x0F0F0F0Fu);
        a.y = (int)nib_minus8((q.y >> sh) & 0x0F0F0F0Fu);
        a.z = (int)nib_minus8((q.z >> sh) & 0x0F0F0F0Fu);
        a.w = (int)nib_minus8((q.w >> sh) & 0x0F0F0F0Fu);
    } else if (TYPE == T_Q8_0) {
        const uint4 q = ld16(qs + ((((size_t)rt * W.nkb + kb) * 2 + g) * 32 + row) * 16);
        a.x = (int)q.x;
        a.y = (int)q.y;
        a.z = (int)q.z;
        a.w = (int)q.w;
    } else {  // Q4_K: kb = 8*sb + j, sub-block j = low nibbles (j even) / high (j odd) of pair j/2
        const int sb = kb >> 3, j = kb & 7;
        const uint4 q = ld16(qs + (((((size_t)rt * W.nkb + sb) * 4 + (j >> 1)) * 2 + g) * 32 + row) * 16);
        const int sh = (j & 1) ? 4 : 0;
        a.x = (int)((q.x >> sh) & 0x0F0F0F0Fu);
        a.y = (int)((q.y >> sh) & 0x0F0F0F0Fu);
        a.z = (int)((q.z >> sh) & 0x0F0F0F0Fu);
        a.w = (int)((q.w >> sh) & 0x0F0F0F0Fu);
    }
    return a;
}

// Row scales of the 16 rows a lane holds for K-block kb:
//   s[r] = weight scale, mn[r] = Q4_K min scale (0 otherwise).
template <int TYPE>
__device__ __forceinline__ void load_scales(const QMat& W, int e, int rt, int kb, int g, float s[16], float mn[16]) {
    if (TYPE == T_Q4_K) {
        const int sb = kb >> 3, j = kb & 7;
        const float2* kt = W.kt + e * W.kt_es + ((((size_t)rt * W.nkb + sb) * 8 + j) * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v0 = *reinterpret_cast<const float4*>(kt + 8 * q + 4 * g);
            const float4 v1 = *reinterpret_cast<const float4*>(kt + 8 * q + 4 * g + 2);
            s[4 * q + 0] = v0.x; mn[4 * q + 0] = v0.y;
            s[4 * q + 1] = v0.z; mn[4 * q + 1] = v0.w;
            s[4 * q + 2] = v1.x; mn[4 * q + 2] = v1.y;
            s[4 * q + 3] = v1.z; mn[4 * q + 3] = v1.w;
        }
    } else {
        const uint16_t* sc = reinterpret_cast<const uint16_t*>(W.sc + e * W.sc_es) + ((size_t)rt * W.nkb + kb) * 32;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint2 v = *reinterpret_cast<const uint2*>(sc + 8 * q + 4 * g);
            s[4 * q + 0] = f16_to_f32(v.x & 0xFFFFu);
            s[4 * q + 1] = f16_to_f32(v.x >> 16);
            s[4 * q + 2] = f16_to_f32(v.y & 0xFFFFu);
            s[4 * q + 3] = f16_to_f32(v.y >> 16);
            mn[4 * q + 0] = mn[4 * q + 1] = mn[4 * q + 2] = mn[4 * q + 3] = 0.0f;
        }
    }
}

template <int TYPE>
__device__ __forceinline__ void epilogue_block(const v16i& D, const float s[16], const float mn[16], float dx,
                                               float dxsum, float acc[16]) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        acc[r] = __builtin_fmaf(s[r] * dx, (float)D[r], acc[r]);
        if (TYPE == T_Q4_K) acc[r] = __builtin_fmaf(-mn[r], dxsum, acc[r]);
    }
}

__device__ __forceinline__ bool tile_of(const Groups& grp, int ty, int& e, int& p0, int& cnt) {
    if (grp.identity) {
        e = 0;
        p0 = ty * MFMA_BN;
        cnt = min(MFMA_BN, grp.n_tok - p0);
        return cnt > 0;
    }
    if (ty >= *grp.n_tiles) return false;
    const int4 t = grp.tiles[ty];
    e = t.x;
    p0 = t.y;
    cnt = t.z;
    return true;
}

__device__ __forceinline__ int tok_of(const Groups& g, int p) {
    return g.identity ? p : g.pair_f[p] / g.top_k;
}

template <int TYPE>
__global__ void __launch_bounds__(MFMA_THREADS)
k_mfma_gateup(QMat G, QMat U, ActQ8 xq, Groups grp, ActQ8 hq, float* hf, int hf_ld) {
    int e, p0, cnt;
    if (!tile_of(grp, blockIdx.y, e, p0, cnt)) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 31, g = lane >> 5;
    const int rt = blockIdx.x * MFMA_WAVES + wave;
    if (rt >= G.nrt) return;
    const bool valid = n < cnt;
    const int tok = tok_of(grp, p0 + (valid ? n : 0));
    const int K = xq.K, KB = K / 32;
    const int8_t* brow = xq.q + (size_t)tok * K;
    const float2* bs = xq.s + (size_t)tok * KB;
    float ag[16], au[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) ag[r] = au[r] = 0.0f;
    const v16i zero = {};
    for (int kb = 0; kb < KB; ++kb) {
        const v4i A_g = load_a<TYPE>(G, e, rt, kb, n, g);
        const v4i A_u = load_a<TYPE>(U, e, rt, kb, n, g);
        v4i B = {0, 0, 0, 0};
        float dx = 0.0f, dxs = 0.0f;
        if (valid) {
            const uint4 b = ld16(brow + kb * 32 + 16 * g);
            B.x = (int)b.x; B.y = (int)b.y; B.z = (int)b.z; B.w = (int)b.w;
            const float2 sv = bs[kb];
            dx = sv.x;
            dxs = sv.x * sv.y;
        }
        const v16i Dg = __builtin_amdgcn_mfma_i32_32x32x32_i8(A_g, B, zero, 0, 0, 0);
        const v16i Du = __builtin_amdgcn_mfma_i32_32x32x32_i8(A_u, B, zero, 0, 0, 0);
        float s[16], mn[16];
        load_scales<TYPE>(G, e, rt, kb, g, s, mn);
        epilogue_block<TYPE>(Dg, s, mn, dx, dxs, ag);
        load_scales<TYPE>(U, e, rt, kb, g, s, mn);
        epilogue_block<TYPE>(Du, s, mn, dx, dxs, au);
    }
    // SwiGLU and Q8_0 of each pair's 32-row block (rows split over lanes n, n+32)
    float hv[16];
    float amax = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        hv[r] = (ag[r] / (1.0f + expf(-ag[r]))) * au[r];
        amax = fmaxf(amax, __builtin_fabsf(hv[r]));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    const float dd = amax / 127.0f;
    const float id = (dd != 0.0f) ? 1.0f / dd : 0.0f;
    int qv[16];
    int qs = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        float rr = round_away(hv[r] * id);
        rr = fminf(fmaxf(rr, -127.0f), 127.0f);
        qv[r] = (int)rr;
        qs += qv[r];
    }
    qs += __shfl_xor(qs, 32, 64);
    if (!valid) return;
    const size_t prow = (size_t)(p0 + n);
    int8_t* dst = hq.q + prow * hq.K + rt * 32 + 4 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t w = (uint32_t)(qv[4 * q] & 0xFF) | ((uint32_t)(qv[4 * q + 1] & 0xFF) << 8) |
                           ((uint32_t)(qv[4 * q + 2] & 0xFF) << 16) | ((uint32_t)(qv[4 * q + 3] & 0xFF) << 24);
        *reinterpret_cast<uint32_t*>(dst + 8 * q) = w;
    }
    if (g == 0) hq.s[prow * (hq.K / 32) + rt] = make_float2(f16_to_f32(f32_to_f16_trunc(dd)), (float)qs);
    if (hf) {
        float* fd = hf + prow * (size_t)hf_ld + rt * 32 + 4 * g;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<float4*>(fd + 8 * q) = make_float4(hv[4 * q], hv[4 * q + 1], hv[4 * q + 2], hv[4 * q + 3]);
    }
}

template <int TYPE>
__global__ void __launch_bounds__(MFMA_THREADS)
k_mfma_down(QMat D, ActQ8 hq, Groups grp, float* y) {
    int e, p0, cnt;
    if (!tile_of(grp, blockIdx.y, e, p0, cnt)) return;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 31, g = lane >> 5;
    const int rt = blockIdx.x * MFMA_WAVES + wave;
    if (rt >= D.nrt) return;
    const bool valid = n < cnt;
    const size_t prow = (size_t)(p0 + (valid ? n : 0));
    const int K = hq.K, KB = K / 32;
    const int8_t* brow = hq.q + prow * K;
    const float2* bs = hq.s + prow * KB;
    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    const v16i zero = {};
    for (int kb = 0; kb < KB; ++kb) {
        const v4i A = load_a<TYPE>(D, e, rt, kb, n, g);
        v4i B = {0, 0, 0, 0};
        float dx = 0.0f, dxs = 0.0f;
        if (valid) {
            const uint4 b = ld16(brow + kb * 32 + 16 * g);
            B.x = (int)b.x; B.y = (int)b.y; B.z = (int)b.z; B.w = (int)b.w;
            const float2 sv = bs[kb];
            dx = sv.x;
            dxs = sv.x * sv.y;
        }
        const v16i Dm = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, zero, 0, 0, 0);
        float s[16], mn[16];
        load_scales<TYPE>(D, e, rt, kb, g, s, mn);
        epilogue_block<TYPE>(Dm, s, mn, dx, dxs, acc);
    }
    if (!valid) return;
    float* dst = y + prow * (size_t)D.rows + rt * 32 + 4 * g;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4*>(dst + 8 * q) = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
}

void launch_mfma_gateup(const QMat& g, const QMat& u, const ActQ8& xq, const Groups& grp, int tiles_ub, ActQ8 hq,
                        float* hf, hipStream_t st) {
    dim3 grid((g.nrt + MFMA_WAVES - 1) / MFMA_WAVES, tiles_ub);
    const int hf_ld = ((g.rows + 255) / 256) * 256;
    switch (g.type) {
        case T_Q4_0: hipLaunchKernelGGL(k_mfma_gateup<T_Q4_0>, grid, dim3(MFMA_THREADS), 0, st, g, u, xq, grp, hq, hf, hf_ld); break;
        case T_Q8_0: hipLaunchKernelGGL(k_mfma_gateup<T_Q8_0>, grid, dim3(MFMA_THREADS), 0, st, g, u, xq, grp, hq, hf, hf_ld); break;
        case T_Q4_K: hipLaunchKernelGGL(k_mfma_gateup<T_Q4_K>, grid, dim3(MFMA_THREADS), 0, st, g, u, xq, grp, hq, hf, hf_ld); break;
        default: break;
    }
}

void launch_mfma_down(const QMat& dn, const ActQ8& hq, const Groups& grp, int tiles_ub, float* y, hipStream_t st) {
    dim3 grid((dn.nrt + MFMA_WAVES - 1) / MFMA_WAVES, tiles_ub);
    switch (dn.type) {
        case T_Q4_0: hipLaunchKernelGGL(k_mfma_down<T_Q4_0>, grid, dim3(MFMA_THREADS), 0, st, dn, hq, grp, y); break;
        case T_Q8_0: hipLaunchKernelGGL(k_mfma_down<T_Q8_0>, grid, dim3(MFMA_THREADS), 0, st, dn, hq, grp, y); break;
        case T_Q4_K: hipLaunchKernelGGL(k_mfma_down<T_Q4_K>, grid, dim3(MFMA_THREADS), 0, st, dn, hq, grp, y); break;
        default: break;
    }
}

}  // namespace jx

// Prefill regime (many tokens per expert): grouped GEMM on the matrix cores.
//
// The reference's dots (vec_dot_{q4_0,q8_0,q4_K}_q8_0, src/quant.cpp:3307-3573)
// sum each 32-element block exactly and scale it by (weight scale x
// activation scale).  On int8 MFMA that costs a convert, a multiply and an
// fma per output per 32-K block on the VALU, which on gfx950 barely overlaps
// the matrix core.  This kernel moves the scaling into the fp16 matrix core
// with operands that fp16 holds exactly:
//   A (weights)      Q4_K: sc_j * q  (0..945)   Q4_0: q - 8   Q8_0: q
//   B (activations)  dx * q * 2^-E of the Q8_0 activations as an exact fp16
//                    hi/lo pair (an 11-bit scale times |q| <= 127 has <= 18
//                    significant bits; hi + lo carry 22), with one power of
//                    two 2^E per 128-element half-unit keeping it in range
// Every product is exact in fp32, so each block's sum equals the
// reference's integer block sum times (sc_j and) dx up to fp32 rounding of
// the accumulation.  What is left on the VALU:
//   Q4_K      acc += (d 2^E) * D  once per half-unit (D accumulates its 4
//             sub-blocks inside the MFMA), and the min term
//             -dmin * sum_j m_j * (dx_j * sum q_j) as three bf16 MFMAs on
//             exact 3-piece splits (bf16 keeps fp32's range) accumulating
//             straight into acc once per super-block;
//   Q4_0/Q8_0 acc += (d_b 2^E) * D_b  per 32-block.
// Only the fp32 summation order differs from the reference.
//
// Work split: a workgroup (8 waves) owns one tile of MFMA_BN = 128 (token,
// expert) pairs of one expert and a group of weight rows; each wave owns 32
// rows (one MFMA M-edge) x 128 pairs (4 MFMA N-edges).  Gate/up: waves 0-3
// take 128 gate rows, waves 4-7 the same 128 up rows; SwiGLU and the Q8_0
// quantization of h for the down projection run in the epilogue.  Down: 8
// waves x 32 rows.  Activations are staged per 128-K half-unit into LDS with
// direct global->LDS loads (double-buffered; 16-byte chunks XOR-swizzled by
// row so the B-operand reads are bank-conflict free, and every lane's read
// offsets are precomputed).  Each wave streams its own weight rows from HBM
// into registers one half-unit ahead and converts them in registers.
// Workgroups are numbered XCD-major so the ~32 resident on one XCD share a
// pair tile, whose activations then stay in that XCD's L2.
//
// MFMA operand layout (v_mfma_f32_32x32x16_f16): lane (n, g) = (lane % 32,
// lane / 32) holds A[row n][k = 8g + i] and B[k = 8g + i][col n], i < 8; the
// 32x32 result sits in lane l, register r at row 8*(r/4) + 4*(l/32) + r%4,
// column l % 32.  A 32-K block takes two K-halves m; in half m, lane g
// carries block elements 16g + 8m + i of both operands (the sum is
// order-free).
#include "jxmoe_device.h"
#include "jxmoe_kernels.h"

namespace jx {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int GW = 8;                 // waves per workgroup (two per SIMD)
constexpr int GT = GW * 64;
constexpr int NT = MFMA_BN / 32;      // MFMA N-edges per wave
constexpr int HB = 4;                 // 32-blocks per staged half-unit
constexpr int HROW = 2 * HB * 32 * 2; // staged bytes per activation row per half-unit (hi + lo)
constexpr int TILE_B = 32 * HROW;     // LDS bytes of one 32-pair MFMA N-edge

template <bool MIN>
struct Stage {
    uint8_t q[MFMA_BN * HROW];                // row r, 16-byte chunk c at chunk (c ^ (r & 31))
    float pe[MFMA_BN];                        // 2^E of each row's half-unit
    uint16_t xm[MIN ? 3 * MFMA_BN * 8 : 8];   // [piece][row][8 blocks] bf16 of dx * sum(q)
};

template <int TYPE>
struct GemmSmem {
    static constexpr bool MIN = TYPE == T_Q4_K;
    Stage<MIN> st[2];
    int src[MFMA_BN];                 // activation row (token or pair) of each staged row
    float wsc[GW][MIN ? 32 : HB * 32];  // per-wave weight scales: Q4_K d per row, else [block][row]
};

static_assert(sizeof(GemmSmem<T_Q4_K>) <= 160 * 1024 && sizeof(GemmSmem<T_Q4_0>) <= 160 * 1024, "LDS budget");
// the gate/up epilogue reuses the stage buffers for the up accumulators and the block scales of h
static_assert(sizeof(Stage<false>) * 2 >= (4 * NT * 16 * 64 + 4 * MFMA_BN) * sizeof(float), "exchange buffer");

typedef __attribute__((address_space(3))) void* lds_ptr;

// 64 lanes x 16 (4) bytes from per-lane global addresses into LDS at `base`
// (wave-uniform), lane i at base + 16 i (4 i).
__device__ __forceinline__ void dma16(const void* src, void* base) {
    __builtin_amdgcn_global_load_lds(src, (lds_ptr)base, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, void* base) {
    __builtin_amdgcn_global_load_lds(src, (lds_ptr)base, 4, 0, 0);
}

__device__ __forceinline__ h2v as_h2(uint32_t v) { return __builtin_bit_cast(h2v, v); }

// 8 bytes (w0, w1) of small unsigned integers v (after mask/flip) -> 8 fp16
// c1 * (1024 + v) + c0, exact: the perm builds fp16 bit patterns 0x64vv =
// 1024 + vv and one fused fp16 fma removes the bias.
__device__ __forceinline__ h8 cvt8(uint32_t w0, uint32_t w1, uint32_t mask, uint32_t flip, h2v c1, h2v c0) {
    const uint32_t a = (w0 & mask) ^ flip, b = (w1 & mask) ^ flip;
    const h2v x0 = as_h2(__builtin_amdgcn_perm(0x64646464u, a, 0x04010400u));
    const h2v x1 = as_h2(__builtin_amdgcn_perm(0x64646464u, a, 0x04030402u));
    const h2v x2 = as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x04010400u));
    const h2v x3 = as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x04030402u));
    const h2v y0 = __builtin_elementwise_fma(x0, c1, c0);
    const h2v y1 = __builtin_elementwise_fma(x1, c1, c0);
    const h2v y2 = __builtin_elementwise_fma(x2, c1, c0);
    const h2v y3 = __builtin_elementwise_fma(x3, c1, c0);
    return h8{y0.x, y0.y, y1.x, y1.y, y2.x, y2.y, y3.x, y3.y};
}

__device__ __forceinline__ h2v splat(float v) {
    const _Float16 h = (_Float16)v;
    return h2v{h, h};
}

__device__ __forceinline__ v16f mfma16(h8 a, h8 b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v16f mfma16b(b8 a, b8 b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Exact 3-piece bf16 split of an fp32 value with at most 24 significant bits
// (truncation keeps each remainder exact).
__device__ __forceinline__ void split3(float v, uint16_t& h, uint16_t& m, uint16_t& l) {
    const uint32_t bh = __float_as_uint(v) & 0xFFFF0000u;
    const float r1 = v - __uint_as_float(bh);
    const uint32_t bm = __float_as_uint(r1) & 0xFFFF0000u;
    const float r2 = r1 - __uint_as_float(bm);
    h = (uint16_t)(bh >> 16);
    m = (uint16_t)(bm >> 16);
    l = (uint16_t)(__float_as_uint(r2) >> 16);
}

// Exact fp16 hi/lo pair of dx * q (see the header comment).
__device__ __forceinline__ void split2h(float v, uint16_t& h, uint16_t& l) {
    const _Float16 a = (_Float16)v;
    const _Float16 b = (_Float16)(v - (float)a);
    h = __builtin_bit_cast(uint16_t, a);
    l = __builtin_bit_cast(uint16_t, b);
}

// ---------------------------------------------------------------- weights
// Raw weight bytes of one half-unit for lane (n, g) of row tile rt.
template <int TYPE>
struct WRaw;

template <>
struct WRaw<T_Q4_K> {
    uint4 q[2];   // pairs 2s, 2s+1 of super-block h/2 (s = h&1), half g: elements 16g..16g+15
                  // of sub-blocks 2p (low nibbles) and 2p+1 (high nibbles)
    uint4 hd;     // header of row n (d | dmin << 16, scales[12]); loaded with the even half
    __device__ void load(const QMat& W, int e, int rt, int h, int n, int g, int lane, int nb) {
        (void)lane;
        (void)nb;
        const size_t t = (size_t)rt * W.nkb + (h >> 1);
        const uint8_t* qb = W.qs + e * W.qs_es;
        const int p0 = 2 * (h & 1);
#pragma unroll
        for (int p = 0; p < 2; ++p) q[p] = ld16(qb + (((t * 4 + p0 + p) * 2 + g) * 32 + n) * 16);
        if (!(h & 1)) hd = ld16(W.sc + e * W.sc_es + (t * 32 + n) * 16);
    }
};

template <int TYPE>
struct WRaw {  // Q4_0 / Q8_0: 16 bytes per 32-block, block scales of the half-unit
    uint4 q[HB];
    uint32_t sc;  // fp16 scales of block (lane/16), rows 2*(lane%16) and +1
    __device__ void load(const QMat& W, int e, int rt, int h, int n, int g, int lane, int nb) {
        const uint8_t* qb = W.qs + e * W.qs_es;
#pragma unroll
        for (int j = 0; j < HB; ++j) {
            if (j < nb) {
                const size_t b = (size_t)rt * W.nkb + h * HB + j;
                q[j] = TYPE == T_Q4_0 ? ld16(qb + (b * 32 + n) * 16) : ld16(qb + ((b * 2 + g) * 32 + n) * 16);
            }
        }
        if ((lane >> 4) < nb)
            sc = *reinterpret_cast<const uint32_t*>(W.sc + e * W.sc_es + (((size_t)rt * W.nkb + h * HB) * 32 + 2 * lane) * 2);
    }
};

// (scale, min) j of a Q4_K header in registers (get_scale_min_k4,
// src/quant.cpp:1107-1115).
__device__ __forceinline__ void hdr_scale_min(const uint4& hd, int j, int& sc, int& mn) {
    const uint32_t s0 = hd.y, s1 = hd.z, s2 = hd.w;  // scales[0..3], [4..7], [8..11]
    const int sh = 8 * (j & 3);
    if (j < 4) {
        sc = (s0 >> sh) & 63;
        mn = (s1 >> sh) & 63;
    } else {
        const uint32_t b = (s2 >> sh) & 0xFF;
        sc = (b & 0x0F) | ((((s0 >> sh) >> 6) & 3) << 4);
        mn = (b >> 4) | ((((s1 >> sh) >> 6) & 3) << 4);
    }
}

// ---------------------------------------------------------------- tiles
__device__ __forceinline__ bool pair_tile(const Groups& grp, int ti, int& e, int& p0, int& cnt) {
    if (grp.identity) {
        e = 0;
        p0 = ti * MFMA_BN;
        cnt = min(MFMA_BN, grp.n_tok - p0);
        return cnt > 0;
    }
    if (ti >= *grp.n_tiles) return false;
    const int4 t = grp.tiles[ti];
    e = t.x;
    p0 = t.y;
    cnt = t.z;
    return true;
}

// Workgroup -> (pair tile, row group): XCD-major numbering (hardware deals
// workgroups round-robin over the 8 XCDs), row group fastest.
__device__ __forceinline__ void work_item(int L, int n_items, int R, int& ti, int& rg) {
    const int x = L & 7, s = L >> 3;
    const int q = n_items >> 3, rem = n_items & 7;
    const int i = x * q + min(x, rem) + s;
    ti = i / R;
    rg = i - ti * R;
}

// Q8_0 of one 32-row block of h per pair, held as 16 registers in each lane
// half (quantize_row_q8_0, src/quant.cpp:1029-1045).  Returns the stored
// (fp16-truncated, widened) scale; q[] gets the quants.
__device__ __forceinline__ float q8_block16(const float h[16], int q[16], int& qsum) {
    float amax = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) amax = fmaxf(amax, __builtin_fabsf(h[r]));
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    const float dd = amax / 127.0f;
    const float id = (dd != 0.0f) ? 1.0f / dd : 0.0f;
    int s = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        float v = round_away(h[r] * id);
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        q[r] = (int)v;
        s += q[r];
    }
    qsum = s + __shfl_xor(s, 32, 64);
    return f16_to_f32(f32_to_f16_trunc(dd));
}

// Exponent of a half-unit from its largest block scale M: |dx * q| * 2^-E < 2^15.
__device__ __forceinline__ int half_exp(float M) {
    return (M > 0.0f) ? (int)((__float_as_uint(M) >> 23) & 0xFF) - 127 - 7 : 0;
}

// Writes one pair's Q8_0 block of h (32 rows = K-block `blk` of the down
// projection) in the matrix-core activation format with half-unit exponent E;
// lane half g holds rows 8*(r/4) + 4g + r%4.
__device__ __forceinline__ void store_hq(const ActH& o, size_t p, int blk, int g, const int q[16], float dd, int qsum,
                                         int E) {
    uint16_t* row = o.hl + p * (size_t)o.KH * 256 + (blk / HB) * 256 + (blk % HB) * 32 + 4 * g;
    const float sc = dd * __uint_as_float((uint32_t)(127 - E) << 23);  // exact: power-of-two scaling
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
        uint16_t h[4], l[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) split2h(sc * (float)q[4 * ii + c], h[c], l[c]);
        *reinterpret_cast<uint2*>(row + 8 * ii) =
            make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
        *reinterpret_cast<uint2*>(row + 128 + 8 * ii) =
            make_uint2((uint32_t)l[0] | ((uint32_t)l[1] << 16), (uint32_t)l[2] | ((uint32_t)l[3] << 16));
    }
    if (g == 0) {
        uint16_t h, m, l;
        split3(dd * (float)qsum, h, m, l);  // exact product: 11-bit scale x |sum| < 2^12
        uint16_t* xm = o.xm + p * (size_t)o.KU * 24 + (blk / 8) * 24 + (blk % 8);
        xm[0] = h;
        xm[8] = m;
        xm[16] = l;
        if (blk % HB == 0) o.pe[p * (size_t)o.KH + blk / HB] = __uint_as_float((uint32_t)(127 + E) << 23);
    }
}

template <bool V>
struct Parity {
    static constexpr bool value = V;
};

template <int TYPE, bool GATEUP>
__global__ void __launch_bounds__(GT)
k_wgemm(QMat W0, QMat W1, ActH in, Groups grp, int R, int n_items, ActH hq, float* hf, int hf_ld, float* y) {
    constexpr bool MIN = TYPE == T_Q4_K;
    __shared__ GemmSmem<TYPE> sm;
    int ti, rg;
    work_item(blockIdx.x, n_items, R, ti, rg);
    int e, p0, cnt;
    if (!pair_tile(grp, ti, e, p0, cnt)) return;  // whole workgroup

    const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int mat = GATEUP ? (wave >> 2) : 0;
    const int rt = GATEUP ? rg * 4 + (wave & 3) : rg * GW + wave;
    const QMat& W = (GATEUP && mat) ? W1 : W0;
    const bool active = rt < W.nrt;  // wave-uniform; inactive waves still stage and sync

    if (tid < MFMA_BN) {  // activation row of each staged row: token (gate/up) or pair (down)
        const int p = p0 + min(tid, cnt - 1);
        sm.src[tid] = (GATEUP && !grp.identity) ? grp.pair_tok[p] : p;
    }
    __syncthreads();
    const int xrow = sm.src[64 * (wave & 1) + lane];

    // LDS byte offsets of this lane's B-operand chunks: (hi/lo, block j, K-half m)
    int boff[2 * HB * 2];
#pragma unroll
    for (int hl = 0; hl < 2; ++hl)
#pragma unroll
        for (int j = 0; j < HB; ++j)
#pragma unroll
            for (int m = 0; m < 2; ++m)
                boff[(hl * HB + j) * 2 + m] = n * HROW + (((16 * hl + 4 * j + 2 * g + m) ^ n) << 4);

    const int H = in.KH;
    const size_t ldq = (size_t)H * 256;
    const int KB = in.K / 32;

    auto stage = [&](int h) {
        Stage<MIN>& S = sm.st[h & 1];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int r = 2 * (wave * 8 + k) + g;
            const int c = n ^ (r & 31);
            dma16(in.hl + (size_t)sm.src[r] * ldq + h * 256 + c * 8, S.q + (wave * 8 + k) * 1024);
        }
        if constexpr (MIN) {
            if ((h & 1) && wave < 6)
                dma16(in.xm + (size_t)xrow * in.KU * 24 + (h >> 1) * 24 + (wave >> 1) * 8,
                      S.xm + (wave >> 1) * (MFMA_BN * 8) + 64 * (wave & 1) * 8);
        }
        if (wave >= 6) dma4(in.pe + (size_t)xrow * H + h, S.pe + 64 * (wave & 1));
    };

    v16f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v16f{};

    WRaw<TYPE> cur, nxt;
    uint4 hdr = make_uint4(0, 0, 0, 0);  // Q4_K header of the current super-block
    if (active) cur.load(W, e, rt, 0, n, g, lane, min(HB, KB));
    stage(0);

    auto half = [&](int h, auto parity) {
        constexpr bool ODD = decltype(parity)::value;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (h + 1 < H) {
            stage(h + 1);
            if (active) nxt.load(W, e, rt, h + 1, n, g, lane, min(HB, KB - (h + 1) * HB));
        }
        if (active) {
            const uint8_t* sq = sm.st[ODD].q;
            const float* pe = sm.st[ODD].pe;
            float* wsc = sm.wsc[wave];
            // B operands, one (block j, K-half m, hi/lo) group of 4 N-edges ahead of its MFMAs
            h8 bq[2][NT];
            auto loadB = [&](int G, int buf) {
                const int j = G >> 2, m = (G >> 1) & 1, hl = G & 1;
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    bq[buf][t] = *reinterpret_cast<const h8*>(sq + boff[(hl * HB + j) * 2 + m] + t * TILE_B);
            };
            if constexpr (TYPE == T_Q4_K) {
                if (!ODD) {
                    hdr = cur.hd;
                    if (g == 0) wsc[n] = f16_to_f32(hdr.x & 0xFFFFu);
                } else {
                    // min term, once per super-block: acc += sum_j (-dmin m_j) (dx_j sum q_j) on
                    // bf16 3-piece splits; six of the nine piece products (all above 2^-24
                    // relative) in three MFMAs, (MFMA, lane half) -> (A piece, B piece):
                    // (0,0) h.h (0,1) h.m (1,0) m.h (1,1) h.l (2,0) l.h (2,1) m.m
                    const float dmin = f16_to_f32(hdr.x >> 16);
                    b8 am[3];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        int sc, mn;
                        hdr_scale_min(hdr, j, sc, mn);
                        uint16_t vh, vm, vl;
                        split3(-dmin * (float)mn, vh, vm, vl);  // exact: 11-bit x 6-bit
                        am[0][j] = __builtin_bit_cast(__bf16, vh);
                        am[1][j] = __builtin_bit_cast(__bf16, g ? vh : vm);
                        am[2][j] = __builtin_bit_cast(__bf16, g ? vm : vl);
                    }
                    const uint16_t* xm = sm.st[1].xm;
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const int row = 32 * t + n;
                        const b8 b0 = *reinterpret_cast<const b8*>(xm + (g ? 1 : 0) * MFMA_BN * 8 + row * 8);
                        const b8 b1 = *reinterpret_cast<const b8*>(xm + (g ? 2 : 0) * MFMA_BN * 8 + row * 8);
                        acc[t] = mfma16b(am[0], b0, acc[t]);
                        acc[t] = mfma16b(am[1], b1, acc[t]);
                        acc[t] = mfma16b(am[2], b0, acc[t]);
                    }
                }
                v16f sb[NT];  // this half-unit's 4 sub-blocks, accumulated by the MFMAs
                h8 A[2];
                loadB(0, 0);
#pragma unroll
                for (int G = 0; G < 4 * HB; ++G) {
                    const int j = G >> 2, m = (G >> 1) & 1, hl = G & 1;
                    if (G + 1 < 4 * HB) loadB(G + 1, (G + 1) & 1);
                    if ((G & 3) == 0) {
                        int sc, mn;
                        hdr_scale_min(hdr, 4 * ODD + j, sc, mn);
                        const uint4 raw = cur.q[j >> 1];
                        const bool hi = j & 1;
                        const h2v c1 = splat(hi ? (float)sc * 0.0625f : (float)sc);
                        const h2v c0 = splat(hi ? -64.0f * (float)sc : -1024.0f * (float)sc);
                        const uint32_t mask = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
                        A[0] = cvt8(raw.x, raw.y, mask, 0u, c1, c0);
                        A[1] = cvt8(raw.z, raw.w, mask, 0u, c1, c0);
                    }
#pragma unroll
                    for (int t = 0; t < NT; ++t) sb[t] = mfma16(A[m], bq[G & 1][t], G == 0 ? v16f{} : sb[t]);
                }
                float dr[16];
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    const float4 v = *reinterpret_cast<const float4*>(wsc + 8 * ii + 4 * g);
                    dr[4 * ii] = v.x;
                    dr[4 * ii + 1] = v.y;
                    dr[4 * ii + 2] = v.z;
                    dr[4 * ii + 3] = v.w;
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const float p2 = pe[32 * t + n];
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[t][r] = __builtin_fmaf(dr[r] * p2, sb[t][r], acc[t][r]);
                }
            } else {
                const int nb = min(HB, KB - h * HB);
                if ((lane >> 4) < nb)
                    *reinterpret_cast<float2*>(wsc + 2 * lane) =
                        make_float2(f16_to_f32(cur.sc & 0xFFFFu), f16_to_f32(cur.sc >> 16));
                uint32_t mask, flip;
                h2v c1, c0;
                if (TYPE == T_Q8_0) {
                    mask = 0xFFFFFFFFu;
                    flip = 0x80808080u;
                    c1 = splat(1.0f);
                    c0 = splat(-1152.0f);
                } else {
                    mask = g ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
                    flip = 0u;
                    c1 = splat(g ? 0.0625f : 1.0f);
                    c0 = splat(g ? -72.0f : -1032.0f);
                }
                h8 A[2];
                v16f D[NT];
                loadB(0, 0);
#pragma unroll
                for (int G = 0; G < 4 * HB; ++G) {
                    const int j = G >> 2, m = (G >> 1) & 1;
                    if (j >= nb) break;
                    if (G + 1 < 4 * nb) loadB(G + 1, (G + 1) & 1);
                    if ((G & 3) == 0) {
                        const uint4 raw = cur.q[j];
                        A[0] = cvt8(raw.x, raw.y, mask, flip, c1, c0);
                        A[1] = cvt8(raw.z, raw.w, mask, flip, c1, c0);
                    }
#pragma unroll
                    for (int t = 0; t < NT; ++t) D[t] = mfma16(A[m], bq[G & 1][t], (G & 3) == 0 ? v16f{} : D[t]);
                    if ((G & 3) == 3) {
                        float dr[16];
#pragma unroll
                        for (int ii = 0; ii < 4; ++ii) {
                            const float4 v = *reinterpret_cast<const float4*>(wsc + j * 32 + 8 * ii + 4 * g);
                            dr[4 * ii] = v.x;
                            dr[4 * ii + 1] = v.y;
                            dr[4 * ii + 2] = v.z;
                            dr[4 * ii + 3] = v.w;
                        }
#pragma unroll
                        for (int t = 0; t < NT; ++t) {
                            const float p2 = pe[32 * t + n];
#pragma unroll
                            for (int r = 0; r < 16; ++r) acc[t][r] = __builtin_fmaf(dr[r] * p2, D[t][r], acc[t][r]);
                        }
                    }
                }
            }
        }
        cur = nxt;
    };

    for (int h = 0; h < H; h += 2) {
        half(h, Parity<false>{});
        if (h + 1 < H) half(h + 1, Parity<true>{});
    }

    // ------------------------------------------------------------ epilogue
    if constexpr (GATEUP) {
        __syncthreads();  // every wave is done with the stage buffers
        float* ex = reinterpret_cast<float*>(&sm.st[0]);
        float* dsh = ex + 4 * NT * 16 * 64;  // [4 row tiles][128 pairs] block scales of h
        if (mat == 1) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) ex[((((wave & 3) * NT + t) * 16) + r) * 64 + lane] = acc[t][r];
        }
        __syncthreads();
        const bool work = mat == 0 && active;
        if (work) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float gv = acc[t][r];
                    const float uv = ex[((((wave & 3) * NT + t) * 16) + r) * 64 + lane];
                    acc[t][r] = (gv / (1.0f + expf(-gv))) * uv;  // SwiGLU, h in place
                }
                const int pr = 32 * t + n;
                const size_t p = (size_t)(p0 + pr);
                if (hf && pr < cnt) {
                    float* fd = hf + p * (size_t)hf_ld + rt * 32 + 4 * g;
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii)
                        *reinterpret_cast<float4*>(fd + 8 * ii) =
                            make_float4(acc[t][4 * ii], acc[t][4 * ii + 1], acc[t][4 * ii + 2], acc[t][4 * ii + 3]);
                }
                if (hq.hl) {
                    int q[16], qsum;
                    float hv[16];
#pragma unroll
                    for (int r = 0; r < 16; ++r) hv[r] = acc[t][r];
                    const float dd = q8_block16(hv, q, qsum);
                    if (g == 0) dsh[(wave & 3) * MFMA_BN + pr] = dd;
                }
            }
        }
        if (!hq.hl) return;
        __syncthreads();  // block scales of the 4 row tiles (one half-unit of the down K) are in dsh
        if (!work) return;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int pr = 32 * t + n;
            float M = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                if (rg * 4 + w < W0.nrt) M = fmaxf(M, dsh[w * MFMA_BN + pr]);
            int q[16], qsum;
            float hv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) hv[r] = acc[t][r];
            const float dd = q8_block16(hv, q, qsum);
            if (pr < cnt) store_hq(hq, (size_t)(p0 + pr), rt, g, q, dd, qsum, half_exp(M));
        }
    } else {
        if (!active) return;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int pr = 32 * t + n;
            if (pr >= cnt) continue;
            float* dst = y + (size_t)(p0 + pr) * W0.rows + rt * 32 + 4 * g;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
                *reinterpret_cast<float4*>(dst + 8 * ii) =
                    make_float4(acc[t][4 * ii], acc[t][4 * ii + 1], acc[t][4 * ii + 2], acc[t][4 * ii + 3]);
        }
    }
}

template <int TYPE, bool GATEUP>
static void launch_t(const QMat& w0, const QMat& w1, const ActH& in, const Groups& grp, int tiles_ub, const ActH& hq,
                     float* hf, int hf_ld, float* y, hipStream_t st) {
    const int R = GATEUP ? (w0.nrt + 3) / 4 : (w0.nrt + GW - 1) / GW;
    const int n_items = R * tiles_ub;
    if (n_items <= 0) return;
    hipLaunchKernelGGL((k_wgemm<TYPE, GATEUP>), dim3(n_items), dim3(GT), 0, st, w0, w1, in, grp, R, n_items, hq, hf,
                       hf_ld, y);
}

void launch_mfma_gateup(const QMat& g, const QMat& u, const ActH& xin, const Groups& grp, int tiles_ub,
                        const ActH& hq, float* hf, hipStream_t st) {
    const int hf_ld = ((g.rows + 255) / 256) * 256;
    switch (g.type) {
        case T_Q4_0: launch_t<T_Q4_0, true>(g, u, xin, grp, tiles_ub, hq, hf, hf_ld, nullptr, st); break;
        case T_Q8_0: launch_t<T_Q8_0, true>(g, u, xin, grp, tiles_ub, hq, hf, hf_ld, nullptr, st); break;
        case T_Q4_K: launch_t<T_Q4_K, true>(g, u, xin, grp, tiles_ub, hq, hf, hf_ld, nullptr, st); break;
        default: break;
    }
}

void launch_mfma_down(const QMat& dn, const ActH& hin, const Groups& grp, int tiles_ub, float* y, hipStream_t st) {
    const ActH none{};
    switch (dn.type) {
        case T_Q4_0: launch_t<T_Q4_0, false>(dn, dn, hin, grp, tiles_ub, none, nullptr, 0, y, st); break;
        case T_Q8_0: launch_t<T_Q8_0, false>(dn, dn, hin, grp, tiles_ub, none, nullptr, 0, y, st); break;
        case T_Q4_K: launch_t<T_Q4_K, false>(dn, dn, hin, grp, tiles_ub, none, nullptr, 0, y, st); break;
        default: break;
    }
}

}  // namespace jx

// Prefill regime (many tokens per expert): grouped GEMM on the matrix cores.
//
// The reference's dots (vec_dot_{q4_0,q8_0,q4_K}_q8_0, src/quant.cpp:3307-3573)
// sum each 32-element block exactly in integers and scale it by
// (weight scale x activation scale).  Done with int8 MFMA that costs a
// convert, a multiply and an fma per output per 32-K block on the VALU,
// which on gfx950 barely overlaps the matrix core.  This kernel instead
// feeds the fp16 matrix core integer-valued operands that fp16 holds
// exactly:
//   A (weights)      Q4_K: sc_j * q  (0..945)   Q4_0: q - 8   Q8_0: q
//   B (activations)  the Q8_0 quants q (|q| <= 127) of x or of SwiGLU(h)
// fp16 x fp16 products are exact in fp32 and every block sum stays below
// 2^24, so each 32-K block result D is the reference's exact integer sum
// (times sc_j for Q4_K).  What remains per block is one fp32 scale:
//   Q4_K      acc_sb += dx_j * D_j   over the 8 sub-blocks of a super-block,
//             acc    += d * acc_sb   once per super-block, and the min term
//             -dmin * sum_j m_j * (dx_j * sum q_j) as three bf16 MFMAs on
//             exact 3-piece splits (bf16 keeps fp32's range) accumulating
//             straight into acc;
//   Q4_0/Q8_0 acc    += (d_b * dx_b) * D_b.
// Only the fp32 summation order differs from the reference.
//
// Work split: a workgroup (8 waves) owns one tile of MFMA_BN = 128 (token,
// expert) pairs of one expert and a group of weight rows; each wave owns 32
// rows (one MFMA M-edge) x 128 pairs (4 MFMA N-edges).  Gate/up: waves 0-3
// take 128 gate rows, waves 4-7 the same 128 up rows, and SwiGLU + the Q8_0
// quantization of h for the down projection run in the epilogue.  Down: 8
// waves x 32 rows.  Activations are staged per 256-K unit into LDS with
// direct global->LDS loads (double-buffered, 16-byte chunks XOR-swizzled by
// row so the B-operand reads are bank-conflict free); each wave streams its
// own weight rows from HBM into registers one unit ahead and converts them
// in registers.  Workgroups are numbered XCD-major so that the ~32 resident
// on one XCD share a pair tile (its activations stay in that XCD's L2).
//
// MFMA operand layout (v_mfma_f32_32x32x16_f16): lane (n, g) = (lane % 32,
// lane / 32) holds A[row n][k = 8g + i] and B[k = 8g + i][col n], i < 8; the
// 32x32 result sits in lane l, register r at row 8*(r/4) + 4*(l/32) + r%4,
// column l % 32.  A 32-K block is two MFMAs; lane g of MFMA m carries block
// elements 16g + 8m + i for both operands (the sum is order-free).
#include "jxmoe_device.h"
#include "jxmoe_kernels.h"

namespace jx {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int GW = 8;                 // waves per workgroup
constexpr int GT = GW * 64;
constexpr int NT = MFMA_BN / 32;      // MFMA N-edges per wave
constexpr int UB = 8;                 // 32-blocks per staged unit
constexpr int QROW = UB * 32 * 2;     // staged bytes per activation row per unit (512)

template <bool MIN>
struct Stage {
    uint8_t q[MFMA_BN * QROW];        // row r, 16-byte chunk c stored at chunk (c ^ (r & 31))
    float dx[MFMA_BN * UB];           // [row][block]
    uint16_t xm[MIN ? MFMA_BN * 32 : 8];  // [row][hi x8, mid x8, lo x8, pad x8] bf16 of dx * sum(q)
};

template <int TYPE>
struct GemmSmem {
    static constexpr bool MIN = TYPE == T_Q4_K;
    Stage<MIN> st[2];
    float wsc[GW][MIN ? 32 : UB * 32];  // per-wave weight scales of the unit: Q4_K d per row, else [block][row]
};

static_assert(sizeof(GemmSmem<T_Q4_K>) <= 160 * 1024 && sizeof(GemmSmem<T_Q4_0>) <= 160 * 1024, "LDS budget");
// the gate/up epilogue reuses the stage buffers for the up accumulators
static_assert(sizeof(Stage<false>) * 2 >= 4 * NT * 16 * 64 * sizeof(float), "exchange buffer");

typedef __attribute__((address_space(3))) void* lds_ptr;

// 64 lanes x 16 bytes from per-lane global addresses into 1 KB of LDS at
// `base` (wave-uniform), lane i at base + 16 i.
__device__ __forceinline__ void dma16(const void* src, void* base) {
    __builtin_amdgcn_global_load_lds(src, (lds_ptr)base, 16, 0, 0);
}

__device__ __forceinline__ h2v as_h2(uint32_t v) { return __builtin_bit_cast(h2v, v); }

// 8 bytes (w0, w1) of small unsigned integers v (after `mask`) -> 8 fp16
// c1 * (1024 + v) + c0, exact: the perm builds fp16 bit patterns 0x64vv
// = 1024 + vv and a single fused fp16 fma removes the bias.
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

__device__ __forceinline__ h8 lds_h8(const uint8_t* p) { return *reinterpret_cast<const h8*>(p); }

// B operand (8 fp16) of MFMA m for block j of staged row `row`, lane half g.
template <bool MIN>
__device__ __forceinline__ h8 load_b(const Stage<MIN>& S, int row, int j, int g, int m) {
    const int c = 4 * j + 2 * g + m;
    return lds_h8(S.q + row * QROW + ((c ^ (row & 31)) << 4));
}

// ---------------------------------------------------------------- weights
// Raw weight bytes of one unit for lane (n, g) of row tile rt.
template <int TYPE>
struct WRaw;

template <>
struct WRaw<T_Q4_K> {
    uint4 q[4];   // pair p, half g: elements 16g..16g+15 of sub-blocks 2p (low nibbles) and 2p+1 (high)
    uint4 hd;     // header of row n: d | dmin << 16, scales[12]
    __device__ void load(const QMat& W, int e, int rt, int u, int n, int g) {
        const size_t t = (size_t)rt * W.nkb + u;
        const uint8_t* qb = W.qs + e * W.qs_es;
#pragma unroll
        for (int p = 0; p < 4; ++p) q[p] = ld16(qb + (((t * 4 + p) * 2 + g) * 32 + n) * 16);
        hd = ld16(W.sc + e * W.sc_es + (t * 32 + n) * 16);
    }
};

template <int TYPE>
struct WRaw {  // Q4_0 / Q8_0: 16 bytes per 32-block, block scales of the unit
    uint4 q[UB];
    uint2 sc;     // fp16 scales of blocks (lane/8) of rows 4*(lane%8)..+3
    __device__ void load(const QMat& W, int e, int rt, int u, int n, int g, int lane, int nb) {
        const uint8_t* qb = W.qs + e * W.qs_es;
#pragma unroll
        for (int j = 0; j < UB; ++j) {
            if (j < nb) {
                const size_t b = (size_t)rt * W.nkb + u * UB + j;
                q[j] = TYPE == T_Q4_0 ? ld16(qb + (b * 32 + n) * 16) : ld16(qb + ((b * 2 + g) * 32 + n) * 16);
            }
        }
        if ((lane >> 3) < nb)
            sc = *reinterpret_cast<const uint2*>(W.sc + e * W.sc_es + (((size_t)rt * W.nkb + u * UB) * 32 + 4 * lane) * 2);
    }
};

// (scale, min) pair j of a Q4_K header in registers (get_scale_min_k4,
// src/quant.cpp:1107-1115).
__device__ __forceinline__ void hdr_scale_min(const uint4& hd, int j, int& sc, int& mn) {
    const uint32_t s0 = hd.y, s1 = hd.z, s2 = hd.w;  // scales[0..3], [4..7], [8..11]
    const int sh = 8 * (j & 3);
    if (j < 4) {
        sc = (s0 >> sh) & 63;
        mn = (s1 >> sh) & 63;
    } else {
        const uint32_t b = (s2 >> sh) & 0xFF;
        sc = (b & 0x0F) | (((s0 >> sh) >> 6 & 3) << 4);
        mn = (b >> 4) | (((s1 >> sh) >> 6 & 3) << 4);
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
// half (quantize_row_q8_0, src/quant.cpp:1029-1045): returns the truncated
// fp16 scale (widened) and writes the quants into q[].
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

// Writes one pair's Q8_0 block of h (32 rows = K-block `blk` of the down
// projection) in the MFMA activation format; lane half g holds rows
// 8*(r/4) + 4g + r%4.
__device__ __forceinline__ void store_hq(const ActH& o, size_t p, int blk, int g, const int q[16], float dd, int qsum) {
    uint16_t* dst = o.q16 + p * (size_t)o.KU * 256 + blk * 32 + 4 * g;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
        uint32_t w0, w1;
        {
            const _Float16 a = (_Float16)(float)q[4 * ii], b = (_Float16)(float)q[4 * ii + 1];
            const _Float16 c = (_Float16)(float)q[4 * ii + 2], d = (_Float16)(float)q[4 * ii + 3];
            w0 = (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
            w1 = (uint32_t)__builtin_bit_cast(uint16_t, c) | ((uint32_t)__builtin_bit_cast(uint16_t, d) << 16);
        }
        *reinterpret_cast<uint2*>(dst + 8 * ii) = make_uint2(w0, w1);
    }
    if (g == 0) {
        o.dx[p * (size_t)o.KU * UB + blk] = dd;
        uint16_t h, m, l;
        split3(dd * (float)qsum, h, m, l);  // exact product: 11-bit scale x |sum| < 2^12
        uint16_t* xm = o.xm + p * (size_t)o.KU * 32 + (blk / UB) * 32 + (blk % UB);
        xm[0] = h;
        xm[8] = m;
        xm[16] = l;
    }
}

template <int TYPE, bool GATEUP>
__global__ void __launch_bounds__(GT, 1)
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

    // source rows (tokens of x, or pairs of h) of the staged rows this lane loads
    int srow[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int r = 2 * (wave * 8 + k) + g;
        const int p = p0 + min(r, cnt - 1);
        srow[k] = (GATEUP && !grp.identity) ? grp.pair_f[p] / grp.top_k : p;
    }
    int drow, xrow;  // source rows of this lane's dx (waves 0-3) and min-term (all waves) staging
    {
        const int r = (wave & 3) * 32 + (lane >> 1);
        const int p = p0 + min(r, cnt - 1);
        drow = (GATEUP && !grp.identity) ? grp.pair_f[p] / grp.top_k : p;
        const int r2 = wave * 16 + (lane >> 2);
        const int p2 = p0 + min(r2, cnt - 1);
        xrow = (GATEUP && !grp.identity) ? grp.pair_f[p2] / grp.top_k : p2;
    }
    const size_t ldq = (size_t)in.KU * 256;
    const int KB = in.K / 32;
    const int U = in.KU;

    auto stage = [&](int u) {
        Stage<MIN>& S = sm.st[u & 1];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int r = 2 * (wave * 8 + k) + g;
            const int c = n ^ (r & 31);
            dma16(in.q16 + (size_t)srow[k] * ldq + u * 256 + c * 8, S.q + (wave * 8 + k) * 1024);
        }
        if (wave < 4) dma16(in.dx + (size_t)drow * U * UB + u * UB + (lane & 1) * 4, S.dx + wave * 256);
        if constexpr (MIN) dma16(in.xm + (size_t)xrow * U * 32 + u * 32 + (lane & 3) * 8, S.xm + wave * 512);
    };

    v16f acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = v16f{};

    WRaw<TYPE> cur, nxt;
    auto wload = [&](WRaw<TYPE>& w, int u) {
        if constexpr (TYPE == T_Q4_K) w.load(W, e, rt, u, n, g);
        else w.load(W, e, rt, u, n, g, lane, min(UB, KB - u * UB));
    };
    if (active) wload(cur, 0);
    stage(0);

    for (int u = 0; u < U; ++u) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (u + 1 < U) {
            stage(u + 1);
            if (active) wload(nxt, u + 1);
        }
        const Stage<MIN>& S = sm.st[u & 1];
        if (active) {
            float* wsc = sm.wsc[wave];
            if constexpr (TYPE == T_Q4_K) {
                // ---- Q4_K: one super-block
                const float d = f16_to_f32(cur.hd.x & 0xFFFFu), dmin = f16_to_f32(cur.hd.x >> 16);
                if (g == 0) wsc[n] = d;
                v16f sb[NT];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    int sc, mn;
                    hdr_scale_min(cur.hd, j, sc, mn);
                    const uint4 raw = cur.q[j >> 1];
                    const bool hi = j & 1;
                    const h2v c1 = splat(hi ? (float)sc * 0.0625f : (float)sc);
                    const h2v c0 = splat(hi ? -64.0f * (float)sc : -1024.0f * (float)sc);
                    const uint32_t mask = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
                    const h8 a0 = cvt8(raw.x, raw.y, mask, 0u, c1, c0);
                    const h8 a1 = cvt8(raw.z, raw.w, mask, 0u, c1, c0);
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const int row = 32 * t + n;
                        v16f D = mfma16(a0, load_b(S, row, j, g, 0), v16f{});
                        D = mfma16(a1, load_b(S, row, j, g, 1), D);
                        const float dxv = S.dx[row * UB + j];
                        if (j == 0) {
                            sb[t] = dxv * D;
                        } else {
#pragma unroll
                            for (int r = 0; r < 16; ++r) sb[t][r] = __builtin_fmaf(dxv, D[r], sb[t][r]);
                        }
                    }
                }
                // min term: acc += sum_j (-dmin m_j) (dx_j sum q_j) on bf16 3-piece splits.
                // Six of the nine piece products (all above 2^-24 relative) in three
                // MFMAs; (MFMA, lane half) -> (A piece, B piece):
                //   (0,0) h.h  (0,1) h.m  (1,0) m.h  (1,1) h.l  (2,0) l.h  (2,1) m.m
                b8 am[3];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    int sc, mn;
                    hdr_scale_min(cur.hd, j, sc, mn);
                    uint16_t vh, vm, vl;
                    split3(-dmin * (float)mn, vh, vm, vl);  // exact: 11-bit x 6-bit
                    am[0][j] = __builtin_bit_cast(__bf16, vh);
                    am[1][j] = __builtin_bit_cast(__bf16, g ? vh : vm);
                    am[2][j] = __builtin_bit_cast(__bf16, g ? vm : vl);
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
                    const int row = 32 * t + n;
                    const b8 b0 = *reinterpret_cast<const b8*>(S.xm + row * 32 + (g ? 8 : 0));
                    const b8 b1 = *reinterpret_cast<const b8*>(S.xm + row * 32 + (g ? 16 : 0));
                    acc[t] = mfma16b(am[0], b0, acc[t]);
                    acc[t] = mfma16b(am[1], b1, acc[t]);
                    acc[t] = mfma16b(am[2], b0, acc[t]);
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[t][r] = __builtin_fmaf(dr[r], sb[t][r], acc[t][r]);
                }
            } else {
                // ---- Q4_0 / Q8_0: up to 8 blocks, per-block weight scales via LDS
                const int nb = min(UB, KB - u * UB);
                if ((lane >> 3) < nb) {
                    float4 f;
                    f.x = f16_to_f32(cur.sc.x & 0xFFFFu);
                    f.y = f16_to_f32(cur.sc.x >> 16);
                    f.z = f16_to_f32(cur.sc.y & 0xFFFFu);
                    f.w = f16_to_f32(cur.sc.y >> 16);
                    *reinterpret_cast<float4*>(wsc + 4 * lane) = f;
                }
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
#pragma unroll
                for (int j = 0; j < UB; ++j) {
                    if (j < nb) {
                        const uint4 raw = cur.q[j];
                        const h8 a0 = cvt8(raw.x, raw.y, mask, flip, c1, c0);
                        const h8 a1 = cvt8(raw.z, raw.w, mask, flip, c1, c0);
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
                            const int row = 32 * t + n;
                            v16f D = mfma16(a0, load_b(S, row, j, g, 0), v16f{});
                            D = mfma16(a1, load_b(S, row, j, g, 1), D);
                            const float dxv = S.dx[row * UB + j];
#pragma unroll
                            for (int r = 0; r < 16; ++r) acc[t][r] = __builtin_fmaf(dr[r] * dxv, D[r], acc[t][r]);
                        }
                    }
                }
            }
        }
        cur = nxt;
    }

    // ------------------------------------------------------------ epilogue
    if constexpr (GATEUP) {
        __syncthreads();  // every wave is done with the stage buffers
        float* ex = reinterpret_cast<float*>(&sm.st[0]);
        if (mat == 1) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) ex[((((wave & 3) * NT + t) * 16) + r) * 64 + lane] = acc[t][r];
        }
        __syncthreads();
        if (mat == 1 || !active) return;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float h[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float gv = acc[t][r];
                const float uv = ex[((((wave & 3) * NT + t) * 16) + r) * 64 + lane];
                h[r] = (gv / (1.0f + expf(-gv))) * uv;
            }
            const int pr = 32 * t + n;  // pair row of the tile
            const bool valid = pr < cnt;
            const size_t p = (size_t)(p0 + pr);
            if (hq.q16) {
                int q[16], qsum;
                const float dd = q8_block16(h, q, qsum);
                if (valid) store_hq(hq, p, rt, g, q, dd, qsum);
            }
            if (hf && valid) {
                float* fd = hf + p * (size_t)hf_ld + rt * 32 + 4 * g;
#pragma unroll
                for (int ii = 0; ii < 4; ++ii)
                    *reinterpret_cast<float4*>(fd + 8 * ii) = make_float4(h[4 * ii], h[4 * ii + 1], h[4 * ii + 2], h[4 * ii + 3]);
            }
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

// Prefill regime (many tokens per expert): grouped GEMM on the matrix cores.
//
// The reference's dots (vec_dot_{q4_0,q8_0,q4_K}_q8_0, src/quant.cpp:3307-3573)
// sum each 32-element block exactly and scale it by (weight scale x
// activation scale).  Scaling every 32-K block on the VALU would cost more
// than the matrix core's own work, so the scales ride in fp16 MFMA operands
// that fp16 holds exactly:
//   A (weights)      Q4_K: sc_j * q  (0..945)   Q4_0: q - 8   Q8_0: q
//   B (activations)  Q4_K gate/up: the Q8_0 quants q (block-unit form); acc is
//                    kept in units of the current block's dx per pair and
//                    multiplied by u(b-1) / u(b) once per 32-block, so a block's
//                    exact integer MFMA sum lands in the block's own units.
//                    Otherwise: dx * q * 2^-E as an exact fp16 hi/lo pair (an
//                    11-bit scale times |q| <= 127 has <= 18 significant bits;
//                    hi + lo carry 22), two MFMAs per product (down: hi only)
// Every product is exact in fp32, so each block's sum equals the reference's
// integer block sum times (sc_j and) dx up to fp32 rounding of the
// accumulation (and of the block-unit ratios).  (The exactness matters: h = SiLU(g) * u is re-quantized to
// Q8_0 before the down projection, and a relative error of 2^-11 in g and u
// moves ~1.4% of h's quants by one step, ~2.6e-3 relative in the layer output.)
// What is left on the VALU: the accumulator is kept in units of the current
// weight scale d of its row (Q4_K: per 256-K super-block; Q4_0 / Q8_0: per
// 32-block; 1 where d is zero, the weight operand then zeroed) and rescaled
// by d_prev / d_cur when the period changes; the token's exponent 2^E (one
// per row) and the last unit are applied once at the end.  The Q4_K min term
// -dmin * sum_j m_j * (dx_j * sum q_j) is three bf16 MFMAs on exact 3-piece
// splits once per super-block, straight into acc.  Only the fp32 rounding of
// the accumulation differs from the reference.
//
// Work split: the dispatch tables cut each expert's pairs into tiles of
// MFMA_BN = 128 (token, expert) pairs; a workgroup owns a tile (down) or half
// of one (gate/up: 64 pairs) and a group of weight rows -- gate/up: 128 gate
// rows and the same 128 up rows (one half-unit of the down projection's K, so
// h's Q8_0 blocks are settled inside the workgroup); down: 128 rows.  A wave
// owns TM row tiles x TN pair tiles of 32 (MFMA 32x32 edges): every B operand
// read from LDS feeds TM MFMAs and every A operand converted in registers
// feeds TN.  Activations are staged per 128-K half-unit into LDS with direct
// global->LDS loads (double-buffered; 16-byte chunks XOR-swizzled by pair so
// the B reads are bank-conflict free).  Each wave streams its own weight rows
// from HBM into registers one half-unit ahead and converts them there.
// Workgroups are numbered XCD-major so the ~32 resident on one XCD share a
// pair tile, whose activations then stay in that XCD's L2.
//
// MFMA operand layout (v_mfma_f32_32x32x16_f16): lane (n, g) = (lane % 32,
// lane / 32) holds A[row n][k = 8g + i] and B[k = 8g + i][col n], i < 8; the
// 32x32 result sits in lane l, register r at row 8*(r/4) + 4*(l/32) + r%4,
// column l % 32.  A 32-K block takes two K-halves m; in half m, lane g
// carries block elements 16g + 8m + i of both operands (the sum is
// order-free).
#include <algorithm>

#include "jxmoe_device.h"
#include "jxmoe_kernels.h"

namespace jx {

typedef __bf16 b8 __attribute__((ext_vector_type(8)));

constexpr int HB = 4;  // 32-blocks per staged half-unit

// One staged half-unit of BN activation rows: HL = 2 stages fp16 hi and lo
// (256 bytes each per row), HL = 1 hi only (or the block-unit form's fp16
// quants).
template <int HL, int BN>
struct Stage {
    static constexpr int PB = 256 * HL;   // bytes per row
    static constexpr int CPP = PB / 16;   // 16-byte chunks per row
    uint8_t q[BN * PB];                   // row r, chunk c at chunk (c ^ (r % CPP))
    float pe[BN];                         // 2^E (block-unit form: the unit) of each row
    uint16_t xm[3 * BN * 8];              // Q4_K: [piece][row][8 sub-blocks] bf16 of dx * sum(q)
};

// Block-unit form: the unit ratios of each stage's blocks, [stage][block][row]
// (an empty base otherwise: every byte of LDS counts where two workgroups
// share a CU).
template <int BN, bool RX>
struct RxStage {
    float rx[2][HB * BN];
};
template <int BN>
struct RxStage<BN, false> {};

template <int HL, int BN, bool RX>
struct GemmSmem : RxStage<BN, RX> {
    Stage<HL, BN> st[2];
    int src[BN];  // activation row (token or pair) of each staged pair
};

typedef __attribute__((address_space(3))) void* lds_ptr;

// 64 lanes x 16 (4) bytes from per-lane global addresses into LDS at `base`
// (wave-uniform), lane i at base + 16 i (4 i).
__device__ __forceinline__ void dma16(const void* src, void* base) {
    __builtin_amdgcn_global_load_lds(src, (lds_ptr)base, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* src, void* base) {
    __builtin_amdgcn_global_load_lds(src, (lds_ptr)base, 4, 0, 0);
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

// Workgroup -> (pair tile, part of the tile, row group).  Numbering is
// XCD-major (hardware deals workgroups round-robin over the 8 XCDs, so XCD x
// runs a contiguous range of items), and within it bands of RC row groups
// sweep every pair tile: the ~64 workgroups resident on one XCD then cover
// about RC row groups x 64 / RC tile parts, and each weight row group and each
// staged activation tile is fetched into that XCD's L2 once for several
// workgroups.  RC = R: all row groups of a tile part before the next part.
__device__ __forceinline__ void work_item(int L, int n_items, int R, int S, int RC, int& ti, int& sub, int& rg) {
    const int x = L & 7, s = L >> 3;
    const int q = n_items >> 3, rem = n_items & 7;
    const int i = x * q + min(x, rem) + s;
    const int TS = n_items / R;             // tile parts
    const int band = i / (RC * TS);         // full bands hold RC * TS items; the last one fewer rows
    const int rows = min(RC, R - band * RC);
    const int j = i - band * RC * TS;
    const int ts = j / rows;
    rg = band * RC + (j - ts * rows);
    ti = ts / S;
    sub = ts - ti * S;
}

// ---------------------------------------------------------------- weights

// Raw weight bytes of one half-unit for lane (n, g) of one row tile: the lane
// reads row n.  off() is the lane's byte offset of its row in the tile layout
// (jxmoe_kernels.h), at() the half-unit's offset, the same for every lane.
template <int TYPE>
struct WRaw;

template <>
struct WRaw<T_Q4_K> {
    uint4 q[2];   // sub-block pairs 2s, 2s+1 of super-block h/2 (s = h&1), half g: elements
                  // 16g..16g+15 of sub-blocks 2p (low nibbles) and 2p+1 (high nibbles)
    uint32_t hd;  // d | dmin << 16 of row n's header; loaded with the even half
    uint4 mn[3];  // min-term pieces of row n (hi, mid, lo; QMat::mn); loaded with the odd half
    uint4 cs;     // the 8 sub-blocks' fp16 operand scales s1 of row n (QMat::mn); loaded with the even half
    __device__ static uint32_t qoff(const QMat& W, int rt, int n, int g) {
        return (uint32_t)((((size_t)rt * W.nkb * 8 + g) * 32 + n) * 16);
    }
    __device__ static uint32_t soff(const QMat& W, int rt, int n) {
        return (uint32_t)(((size_t)rt * W.nkb * 32 + n) * 16);
    }
    __device__ static uint32_t moff(const QMat& W, int rt, int n) {
        return (uint32_t)(((size_t)rt * W.nkb * (MN_SB / 16) + n) * 16);
    }
    // PAR: the parity of h (even half-units carry the header, odd ones the min pieces), so each of the
    // two alternating register sets holds only the fields its parity uses
    __device__ static uint32_t xoff(const QMat&, int, int, int) { return 0; }
    template <int PAR>
    __device__ void load(const uint8_t* qb, const uint8_t* sb, const uint8_t* mb, const uint8_t*, uint32_t qo,
                         uint32_t so, uint32_t mo, uint32_t, int h, int nb) {
        (void)nb;
        static_assert(PAR == 0 || PAR == 1, "parity");
        const uint8_t* qh = qb + (size_t)(h >> 1) * 4096 + PAR * 2048;
#pragma unroll
        for (int p = 0; p < 2; ++p) q[p] = ld16(qh + p * 1024 + qo);
        const uint8_t* mh = mb + (size_t)(h >> 1) * MN_SB + mo;
        if (PAR == 0) {
            hd = *reinterpret_cast<const uint32_t*>(sb + (size_t)(h >> 1) * 512 + so);
            cs = ld16(mh + MN_CS);
        } else {
#pragma unroll
            for (int c = 0; c < 3; ++c) mn[c] = ld16(mh + c * 512);
        }
    }
};

// Q5_K: the Q4_K fields plus the lane's chunk of fifth bits (qh bytes 16g..16g+15, bit j = sub-block j),
// loaded with every half-unit.
template <>
struct WRaw<T_Q5_K> : WRaw<T_Q4_K> {
    uint4 qh;
    __device__ static uint32_t xoff(const QMat& W, int rt, int n, int g) {
        return (uint32_t)((((size_t)rt * W.nkb * 2 + g) * 32 + n) * 16);
    }
    template <int PAR>
    __device__ void load(const uint8_t* qb, const uint8_t* sb, const uint8_t* mb, const uint8_t* xb, uint32_t qo,
                         uint32_t so, uint32_t mo, uint32_t xo, int h, int nb) {
        WRaw<T_Q4_K>::template load<PAR>(qb, sb, mb, xb, qo, so, mo, xo, h, nb);
        qh = ld16(xb + (size_t)(h >> 1) * 1024 + xo);
    }
};

// Q6_K: half-unit h is 128-element half h & 1 of super-block h / 2; lane (n, g) takes elements
// 16g..16g+15 of its four 32-blocks: ql chunks g and 2 + g and qh chunk 4 + g of that half; the 16
// int8 scales and d of row n come with the even half-unit.
template <>
struct WRaw<T_Q6_K> {
    uint4 q[3];
    uint4 sc;
    uint32_t d;
    __device__ static uint32_t qoff(const QMat& W, int rt, int n, int g) {
        return (uint32_t)((size_t)rt * W.nkb * 6144 + g * 512 + n * 16);
    }
    __device__ static uint32_t soff(const QMat& W, int rt, int n) {
        return (uint32_t)(((size_t)rt * W.nkb * 32 + n) * 16);
    }
    __device__ static uint32_t moff(const QMat&, int, int) { return 0; }
    __device__ static uint32_t xoff(const QMat& W, int rt, int n, int) {
        return (uint32_t)(((size_t)rt * W.nkb * 32 + n) * 2);
    }
    template <int PAR>
    __device__ void load(const uint8_t* qb, const uint8_t* sb, const uint8_t*, const uint8_t* xb, uint32_t qo,
                         uint32_t so, uint32_t, uint32_t xo, int h, int nb) {
        (void)nb;
        const uint8_t* base = qb + (size_t)(h >> 1) * 6144 + (h & 1) * 3072 + qo;
#pragma unroll
        for (int c = 0; c < 3; ++c) q[c] = ld16(base + c * 1024);
        if (PAR == 0) {
            sc = ld16(sb + (size_t)(h >> 1) * 512 + so);
            d = *reinterpret_cast<const uint16_t*>(xb + (size_t)(h >> 1) * 64 + xo);
        }
    }
};

template <int TYPE>
struct WRaw {  // Q4_0 / Q5_0 / Q8_0: 16 bytes per 32-block, row n's fp16 block scales (Q5_0: and fifth bits)
    static constexpr bool Q5 = TYPE == T_Q5_0;
    uint4 q[HB];
    uint32_t d[HB];
    uint32_t qh[Q5 ? HB : 1];
    __device__ static uint32_t qoff(const QMat& W, int rt, int n, int g) {
        return TYPE != T_Q8_0 ? (uint32_t)(((size_t)rt * W.nkb * 32 + n) * 16)
                              : (uint32_t)((((size_t)rt * W.nkb * 2 + g) * 32 + n) * 16);
    }
    __device__ static uint32_t soff(const QMat& W, int rt, int n) {
        return (uint32_t)(((size_t)rt * W.nkb * 32 + n) * 2);
    }
    __device__ static uint32_t moff(const QMat&, int, int) { return 0; }
    __device__ static uint32_t xoff(const QMat& W, int rt, int n, int) {
        return Q5 ? (uint32_t)(((size_t)rt * W.nkb * 32 + n) * 4) : 0u;
    }
    template <int PAR>
    __device__ void load(const uint8_t* qb, const uint8_t* sb, const uint8_t*, const uint8_t* xb, uint32_t qo,
                         uint32_t so, uint32_t, uint32_t xo, int h, int nb) {
        constexpr int QB = TYPE != T_Q8_0 ? 512 : 1024;  // bytes per 32-block of a row tile
#pragma unroll
        for (int j = 0; j < HB; ++j) {
            if (j < nb) {
                q[j] = ld16(qb + (size_t)(h * HB + j) * QB + qo);
                d[j] = *reinterpret_cast<const uint16_t*>(sb + (size_t)(h * HB + j) * 64 + so);
                if constexpr (Q5) qh[j] = *reinterpret_cast<const uint32_t*>(xb + (size_t)(h * HB + j) * 128 + xo);
            }
        }
    }
};


template <bool V>
struct Parity {
    static constexpr bool value = V;
};


// Wave arrangement of a workgroup owning BN pairs (a dispatch tile of
// MFMA_BN, or a part of one): NPG pair groups of TN pair tiles (32 pairs each)
// side by side, RW row slots.  Gate/up: row slot s takes row tile s of the
// gate matrix and the same tile of the up matrix (TM = 2: tile 0 gate, tile 1
// up), so SwiGLU needs no exchange.  Down: row slot s takes TM row tiles.
template <bool GATEUP, int GW, int TM, int TN, int BN>
struct Arr {
    static constexpr int NPG = BN / (32 * TN);
    static constexpr int RW = GW / NPG;
    static constexpr int WROWS = GATEUP ? RW : RW * TM;  // row tiles of each matrix per workgroup
    static_assert(NPG * TN * 32 == BN && NPG * RW == GW && MFMA_BN % BN == 0, "wave arrangement");
    static_assert(!GATEUP || TM == 2, "gate/up: a gate and an up tile per wave");
};

// The MFMAs take the activations as operand A and the weights as operand B,
// so in each 32x32 result lane (n, g) holds weight row n (its scales are the
// lane's own) and registers r span pairs 8*(r/4) + 4g + r%4.
template <int TYPE, bool GATEUP, int GW, int TM, int TN, int WPE, int BN>
__global__ void __launch_bounds__(GW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
k_wgemm(QMat W0, QMat W1, ActH in, Groups grp, int R, int n_items, int RC, ActQ8 hq, float* hf, int hf_ld,
        float* y, int KS, size_t ystride) {
    constexpr int NTH = GW * 64;
    // K-quants (Q4_K / Q5_K / Q6_K): acc is kept in units of the current super-block's d (per weight
    // row) and rescaled by d_prev / d_cur at each super-block (fp32 rounding ~2^-24 per step); Q4_K and
    // Q5_K carry the min term (Q4K below), Q6_K has none and signed sub-block scales per 16 of K
    constexpr bool Q4K = TYPE == T_Q4_K || TYPE == T_Q5_K;
    constexpr bool K6 = TYPE == T_Q6_K;
    constexpr bool SUPER = Q4K || K6;
    static_assert(!(K6 && GATEUP), "Q6_K gate/up runs on the GEMVs (its sc * q operand is not exact in fp16)");
    constexpr bool RESCALE = true;
    // Q4_K gate/up: block-unit activations -- the exact quants q as the operand and acc kept in units of
    // the current block's dx per pair, rescaled by u(b-1) / u(b) (one multiply per accumulator element
    // and 32-block) before the block's MFMAs; the weight scale d stays per super-block.  Q4_0 / Q8_0
    // gate/up (d per block as well): exact hi + lo activation operands.  (h is re-quantized after
    // SwiGLU, so gate/up products stay exact.)  Down: the hi half only (relative error <= 2^-12 per
    // activation, no re-quantization downstream).
    constexpr bool UNIT = Q4K && GATEUP;
    constexpr int HL = GATEUP && !UNIT ? 2 : 1;
    constexpr int GB = UNIT ? 256 : 512;  // global bytes per row and half-unit
    using St = Stage<HL, BN>;
    constexpr int PB = St::PB, CPP = St::CPP, PPI = 64 / CPP;  // row bytes, chunks, rows per DMA
    constexpr int PER = BN / PPI / GW;  // 1 KB staging loads per wave and half-unit
    static_assert(PER * PPI * GW == BN, "staging split");
    __shared__ GemmSmem<HL, BN, UNIT> sm;
    int ti, sub, rg;
    // the grid covers the tile upper bound; the items of the tiles that exist are spread over the XCDs
    // as if the grid were exact, and the rest exit (otherwise the XCDs whose ranges hold the missing
    // tiles would idle)
    int n_eff = n_items;
    if (!grp.identity) n_eff = min(n_items, R * *grp.n_tiles * (MFMA_BN / BN));
    // down over a long K: KS adjacent workgroups per item (on different XCDs), each a range of K writing
    // its own part of y
    const int kp = GATEUP ? 0 : (int)(blockIdx.x % KS), LB = GATEUP ? (int)blockIdx.x : (int)(blockIdx.x / KS);
    if ((LB >> 3) >= (n_eff >> 3) + ((LB & 7) < (n_eff & 7) ? 1 : 0)) return;
    work_item(LB, n_eff, R, MFMA_BN / BN, RC, ti, sub, rg);
    int e, p0, cnt;
    if (!pair_tile(grp, ti, e, p0, cnt)) return;  // whole workgroup
    p0 += sub * BN;  // this workgroup's part of the tile
    cnt -= sub * BN;
    if (cnt <= 0) return;
    cnt = min(cnt, BN);

    const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    using A_ = Arr<GATEUP, GW, TM, TN, BN>;
    const int pg = wave % A_::NPG, rw = wave / A_::NPG;  // pair group, row slot
    const int pbase = pg * TN * 32;                       // first pair of the wave within the tile
    // the wave's row tiles: gate/up tile rt0 of both matrices, or down tiles rt0 .. rt0 + TM - 1
    const int rt0 = GATEUP ? rg * A_::RW + rw : (rg * A_::RW + rw) * TM;
    const bool active = rt0 < W0.nrt;  // wave-uniform; inactive waves still stage and sync

    if (tid < BN) {  // activation row of each staged pair: token (gate/up) or pair (down)
        const int p = p0 + min(tid, cnt - 1);
        sm.src[tid] = (GATEUP && !grp.identity) ? grp.pair_tok[p] : p;
    }
    __syncthreads();

    const int H = in.KH;
    const int KB = in.K / 32;
    // this workgroup's half-units [h0, h1): whole super-blocks (an even count), the last part the rest
    const int HP = ((H + KS - 1) / KS + 1) & ~1, h0 = GATEUP ? 0 : kp * HP, h1 = GATEUP ? H : min(H, h0 + HP);
    // Source rows ascend within a tile (an expert's pairs are in token order; down rows are
    // consecutive pairs), so the workgroup's buffers are based at its first source row in 64 bits
    // and every per-lane offset is relative to it: below 2^32 whenever n_tok rows of the activation
    // forms are (jx_moe_forward refuses larger batches).
    const size_t src0 = (size_t)sm.src[0];
    // Staging: a DMA instruction moves PPI rows x PB bytes; lane l takes chunk l % CPP of row
    // PPI * slot + l / CPP, stored at chunk ((l % CPP) ^ (row % CPP)), so the operand reads of 16
    // lanes hit 16 distinct 16-byte bank groups.  The half-unit adds h * 512, a uniform term.
    uint32_t soff[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int r = PPI * (wave * PER + k) + lane / CPP;
        soff[k] = (uint32_t)(sm.src[r] - (int)src0) * (uint32_t)(H * GB) + (uint32_t)(((lane % CPP) ^ (r % CPP)) << 4);
    }
    const int sj = wave;  // pe / xm / rx: lane l of wave w < BN / 64 takes pair 64 * w + l
    const uint32_t srow = (uint32_t)(sm.src[64 * min(sj, BN / 64 - 1) + lane] - (int)src0);
    const uint32_t peoff = srow * (uint32_t)(H * 4);
    const uint32_t xoff = Q4K ? srow * (uint32_t)(in.KU * 48) : 0u;
    const uint32_t rxoff = UNIT ? srow * (uint32_t)(H * HB * 4) : 0u;
    const uint8_t* qsrc = reinterpret_cast<const uint8_t*>(UNIT ? in.q16 : in.hl) + src0 * (size_t)(H * GB);
    const uint8_t* pesrc = reinterpret_cast<const uint8_t*>(UNIT ? in.pu : in.pe) + src0 * (size_t)(H * 4);
    const uint8_t* xmsrc = reinterpret_cast<const uint8_t*>(UNIT ? in.xu : in.xm) + src0 * (size_t)(in.KU * 48);
    const uint8_t* rxsrc = UNIT ? reinterpret_cast<const uint8_t*>(in.rx) + src0 * (size_t)(H * HB * 4) : nullptr;
    auto stage = [&](int h) {
        St& S = sm.st[h & 1];
        const uint8_t* base = qsrc + (size_t)h * GB;
#pragma unroll
        for (int k = 0; k < PER; ++k) dma16(base + soff[k], S.q + (wave * PER + k) * 1024);
        if constexpr (Q4K) {
            if (h & 1) {  // min-term values of the super-block: piece pc of the lane's pair
                const uint8_t* xb = xmsrc + (size_t)(h >> 1) * 48;
                if (wave < BN / 64)
                    for (int pc = 0; pc < 3; ++pc) dma16(xb + xoff + pc * 16, S.xm + pc * (BN * 8) + 64 * sj * 8);
            }
        }
        if constexpr (UNIT) {  // unit ratios of the half-unit's blocks, [block][pair]
            if (wave < BN / 64) {
                const uint8_t* rb = rxsrc + (size_t)h * (HB * 4) + rxoff;
#pragma unroll
                for (int j = 0; j < HB; ++j) dma4(rb + 4 * j, sm.rx[h & 1] + j * BN + 64 * sj);
            }
        }
        if (wave < BN / 64) dma4(pesrc + (size_t)h * 4 + peoff, S.pe + 64 * sj);
    };

    // weights: uniform bases, per-lane offsets of the wave's row tiles (tiles past the matrix load
    // a valid one; their results are dropped)
    const uint8_t* qbase[TM];
    const uint8_t* sbase[TM];
    const uint8_t* mbase[TM];
    const uint8_t* xbase[TM];
    uint32_t qo[TM], so[TM], mo[TM], xo[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const QMat& W = (GATEUP && i == 1) ? W1 : W0;
        qbase[i] = W.qs + (size_t)e * W.qs_es;
        sbase[i] = W.sc + (size_t)e * W.sc_es;
        mbase[i] = Q4K ? W.mn + (size_t)e * W.mn_es : nullptr;
        xbase[i] = W.ex ? W.ex + (size_t)e * W.ex_es : nullptr;
        const int rt = min(GATEUP ? rt0 : rt0 + i, W.nrt - 1);
        qo[i] = WRaw<TYPE>::qoff(W, rt, n, g);
        so[i] = WRaw<TYPE>::soff(W, rt, n);
        mo[i] = WRaw<TYPE>::moff(W, rt, n);
        xo[i] = WRaw<TYPE>::xoff(W, rt, n, g);
    }

    // Q4_0 / Q5_0 / Q8_0 down: two accumulator sets, acc for even 32-blocks and acc2 for odd ones, each in
    // its own unit (down only: with gate/up's two weight tiles per wave the second set spills, 394 -> 702 us)
    constexpr bool DUAL = !SUPER && !GATEUP;
    constexpr int TM2 = DUAL ? TM : 1, TN2 = DUAL ? TN : 1;
    v16f acc[TM][TN], acc2[TM2][TN2];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t) acc[i][t] = v16f{};
#pragma unroll
    for (int i = 0; i < TM2; ++i)
#pragma unroll
        for (int t = 0; t < TN2; ++t) acc2[i][t] = v16f{};

    WRaw<TYPE> wa[TM], wb[TM];
    uint4 hdr[TM];  // the current super-block's sub-block scales: Q6_K's 16 int8, Q4_K / Q5_K's 8 fp16 s1
    float dl[TM];   // the unit acc is kept in for the lane's row: the current super-block's (Q4_K) or
                    // block's (Q4_0 / Q8_0) weight scale d, 1 where d is zero
    float dl2[TM2]; // the unit of acc2
    bool dz[TM];    // Q4_K: this super-block's d is zero (its sc * q terms vanish)
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        hdr[i] = make_uint4(0, 0, 0, 0);
        dl[i] = RESCALE ? 1.0f : 0.0f;
        dz[i] = false;
    }
#pragma unroll
    for (int i = 0; i < TM2; ++i) dl2[i] = 1.0f;
    if (active)
#pragma unroll
        for (int i = 0; i < TM; ++i)
            wa[i].template load<0>(qbase[i], sbase[i], mbase[i], xbase[i], qo[i], so[i], mo[i], xo[i], h0,
                                   min(HB, KB - h0 * HB));
    stage(h0);

    // LDS byte offset of this lane's A chunk (hi/lo hl, sub-block j of the half-unit, K-half m) in pair tile 0
    auto boff = [&](int hl, int j, int m) { return n * PB + (((16 * hl + 4 * j + 2 * g + m) ^ (n % CPP)) << 4); };

    auto half = [&](int h, auto parity, WRaw<TYPE>(&cur)[TM], WRaw<TYPE>(&nxt)[TM]) {
        constexpr bool ODD = decltype(parity)::value;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (h + 1 < h1) {
            stage(h + 1);
            if (active)
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    nxt[i].template load<ODD ? 0 : 1>(qbase[i], sbase[i], mbase[i], xbase[i], qo[i], so[i], mo[i],
                                                      xo[i], h + 1, min(HB, KB - (h + 1) * HB));
        }
        if (!active) return;
        const uint8_t* sa = sm.st[ODD].q + pg * TN * 32 * PB;
        if constexpr (SUPER) {
            if (!ODD) {
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    float d;
                    if constexpr (K6) {
                        hdr[i] = cur[i].sc;
                        d = f16_to_f32(cur[i].d & 0xFFFFu);
                    } else {
                        hdr[i] = cur[i].cs;  // the super-block's operand scales, for both halves
                        d = f16_to_f32(cur[i].hd & 0xFFFFu);
                    }
                    if constexpr (RESCALE) {
                        dz[i] = d == 0.0f;
                        const float u = dz[i] ? 1.0f : d;  // the unit the min table divides by
                        const float ratio = dl[i] * __builtin_amdgcn_rcpf(u);  // ~1 ulp
                        dl[i] = u;
#pragma unroll
                        for (int t = 0; t < TN; ++t)
#pragma unroll
                            for (int r = 0; r < 16; ++r) acc[i][t][r] *= ratio;
                    } else {
                        (void)d;
                    }
                }
            } else if constexpr (Q4K) {
                // min term, once per super-block: acc += sum_j (dx_j sum q_j) (-dmin m_j / unit) on bf16
                // 3-piece splits (the activation side in xm, the weight side from the min table); six of
                // the nine piece products (all above 2^-24 relative) in three MFMAs, (MFMA, lane half) ->
                // (activation piece, weight piece): (0,0) h.h (0,1) m.h (1,0) h.m (1,1) l.h (2,0) h.l (2,1) m.m.
                // The down projection drops the third (h.l and m.m, ~2^-16 relative each): its hi-only
                // activations already carry 2^-12, and nothing downstream re-quantizes.
                const uint16_t* xm = sm.st[1].xm + pbase * 8;
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const uint4 w1 = g ? cur[i].mn[0] : cur[i].mn[1], w2 = g ? cur[i].mn[1] : cur[i].mn[2];
                    const b8 wm[3] = {__builtin_bit_cast(b8, cur[i].mn[0]), __builtin_bit_cast(b8, w1),
                                      __builtin_bit_cast(b8, w2)};
#pragma unroll
                    for (int t = 0; t < TN; ++t) {
                        const int pr = 32 * t + n;
                        const b8 x0 = *reinterpret_cast<const b8*>(xm + (g ? 1 : 0) * BN * 8 + pr * 8);
                        const b8 x1 = *reinterpret_cast<const b8*>(xm + (g ? 2 : 0) * BN * 8 + pr * 8);
                        acc[i][t] = mfma16b(x0, wm[0], acc[i][t]);
                        acc[i][t] = mfma16b(x1, wm[1], acc[i][t]);
                        if constexpr (GATEUP) acc[i][t] = mfma16b(x0, wm[2], acc[i][t]);
                    }
                }
            }
            // 8 K-steps of 16 per half-unit (sub-block jj = st / 2, K-half m = st % 2), software
            // pipelined: while step st's 2 * TN * TM MFMAs run, the activation operands of step st + 1
            // are read from LDS and its weights converted (the schedule is pinned below)
            h8 av[2][TN][HL];
            h8 wv[2][TM];
            h2v c1[TM], c0[TM];
            auto read_av = [&](int st, h8(&dst)[TN][HL]) {
#pragma unroll
                for (int t = 0; t < TN; ++t)
#pragma unroll
                    for (int hl = 0; hl < HL; ++hl)
                        dst[t][hl] = *reinterpret_cast<const h8*>(sa + t * 32 * PB + boff(hl, st >> 1, st & 1));
            };
            auto convert = [&](int st, h8(&dst)[TM]) {
                const int jj = st >> 1, m = st & 1;
                if (m == 0) {
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        if constexpr (K6) {
                            // sc * (q6 - 32) from v = 4 q6: (1024 + v) * sc / 4 - 288 sc in one fp16 fma (both
                            // constants exact; the result rounds once, exact up to |sc * (q6 - 32)| <= 2048)
                            const int k = 8 * ODD + 2 * jj + g;
                            const uint32_t wsc = k < 4 ? hdr[i].x : (k < 8 ? hdr[i].y : (k < 12 ? hdr[i].z : hdr[i].w));
                            const float scf = RESCALE && dz[i] ? 0.0f : (float)(int8_t)(uint8_t)(wsc >> (8 * (k & 3)));
                            c1[i] = splat(scf * 0.25f);
                            c0[i] = splat(scf * -288.0f);
                        } else {
                            // sub-block J = 4 ODD + jj's scale s1 from the table built at upload (k_min_table;
                            // zero where d is zero) and s0 = -1024 s1 (exact)
                            const uint32_t w2 = ODD ? (jj < 2 ? hdr[i].z : hdr[i].w) : (jj < 2 ? hdr[i].x : hdr[i].y);
                            const _Float16 s1 = as_h2(w2)[jj & 1];
                            c1[i] = h2v{s1, s1};
                            const _Float16 s0 = s1 * (_Float16)-1024.0f;
                            c0[i] = h2v{s0, s0};
                        }
                    }
                }
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    if constexpr (K6) {
                        const uint4 lo = cur[i].q[jj & 1], hb = cur[i].q[2];
                        const int sh = (jj >> 1) * 4;
                        const uint32_t l0 = ((m ? lo.z : lo.x) >> sh) & 0x0F0F0F0Fu, l1 = ((m ? lo.w : lo.y) >> sh) & 0x0F0F0F0Fu;
                        const uint32_t h0 = ((m ? hb.z : hb.x) >> (2 * jj)) & 0x03030303u;
                        const uint32_t h1 = ((m ? hb.w : hb.y) >> (2 * jj)) & 0x03030303u;
                        dst[i] = cvt8((l0 << 2) | (h0 << 6), (l1 << 2) | (h1 << 6), 0xFFFFFFFFu, 0u, c1[i], c0[i]);
                    } else if constexpr (TYPE == T_Q5_K) {
                        const uint4 raw = cur[i].q[jj >> 1], qb = cur[i].qh;
                        const int sh = (jj & 1) * 4, J = 4 * ODD + jj;
                        const uint32_t w0 = (((m ? raw.z : raw.x) >> sh) & 0x0F0F0F0Fu) | ((((m ? qb.z : qb.x) >> J) & 0x01010101u) << 4);
                        const uint32_t w1 = (((m ? raw.w : raw.y) >> sh) & 0x0F0F0F0Fu) | ((((m ? qb.w : qb.y) >> J) & 0x01010101u) << 4);
                        dst[i] = cvt8(w0, w1, 0xFFFFFFFFu, 0u, c1[i], c0[i]);
                    } else {
                        const uint32_t mask = (jj & 1) ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
                        const uint4 raw = cur[i].q[jj >> 1];
                        dst[i] = m ? cvt8(raw.z, raw.w, mask, 0u, c1[i], c0[i]) : cvt8(raw.x, raw.y, mask, 0u, c1[i], c0[i]);
                    }
                }
            };
            // block-unit form: each pair tile's 16 unit ratios of a block (register r <-> pair
            // 8 (r / 4) + 4 g + r % 4), read from LDS one step ahead (measured faster than reading
            // the second pair tile's at the block's first step, which saves registers)
            float4 rxv[UNIT ? TN : 1][4];
            const float* rxs = nullptr;
            if constexpr (UNIT) rxs = sm.rx[ODD] + pbase + 4 * g;
            auto read_rx = [&](int jj) {
#pragma unroll
                for (int t = 0; t < TN; ++t)
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii)
                        rxv[t][ii] = *reinterpret_cast<const float4*>(rxs + jj * BN + 32 * t + 8 * ii);
            };
            auto read_rx1 = [&](int jj, int t) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii)
                    rxv[t][ii] = *reinterpret_cast<const float4*>(rxs + jj * BN + 32 * t + 8 * ii);
            };
            auto rescale = [&](int i, int t) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    acc[i][t][4 * ii] *= rxv[t][ii].x;
                    acc[i][t][4 * ii + 1] *= rxv[t][ii].y;
                    acc[i][t][4 * ii + 2] *= rxv[t][ii].z;
                    acc[i][t][4 * ii + 3] *= rxv[t][ii].w;
                }
            };
            read_av(0, av[0]);
            convert(0, wv[0]);
            if constexpr (UNIT) read_rx(0);
#pragma unroll
            for (int st = 0; st < 2 * HB; ++st) {
                const int b = st & 1;

                // the next step's LDS reads go out before this step's MFMAs (nothing crosses the
                // scheduling barriers), so their latency hides behind 2 * TN * TM MFMAs
                if (st + 1 < 2 * HB) read_av(st + 1, av[b ^ 1]);
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (UNIT && TN == 2 && TM == 2) {
                    // tiles k = (t, i) in order (0,0) (0,1) (1,0) (1,1); tile k's rescale into block jj's
                    // units must fall between its last MFMA of block jj - 1 and its first of block jj:
                    // pair tile 0's two go in block jj - 1's second step, after their own MFMAs there,
                    // and pair tile 1's two in block jj's first step, before theirs, so every step
                    // carries two rescales beside its four MFMAs (a half-unit's first block has its
                    // ratios staged only at its own first step and takes all four there)
                    const int jj = st >> 1;
                    if (b == 0) {
                        if (jj == 0) {
                            rescale(0, 0);
                            acc[0][0] = mfma16(av[b][0][0], wv[b][0], acc[0][0]);
                            rescale(1, 0);
                            acc[1][0] = mfma16(av[b][0][0], wv[b][1], acc[1][0]);
                        } else {
                            acc[0][0] = mfma16(av[b][0][0], wv[b][0], acc[0][0]);
                            acc[1][0] = mfma16(av[b][0][0], wv[b][1], acc[1][0]);
                        }
                        rescale(0, 1);
                        acc[0][1] = mfma16(av[b][1][0], wv[b][0], acc[0][1]);
                        rescale(1, 1);
                        acc[1][1] = mfma16(av[b][1][0], wv[b][1], acc[1][1]);
                        if (jj + 1 < HB) read_rx1(jj + 1, 0);
                        if (jj == 0) {
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                            }
                        } else {
                            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                            __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                            __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    } else {
                        acc[0][0] = mfma16(av[b][0][0], wv[b][0], acc[0][0]);
                        acc[1][0] = mfma16(av[b][0][0], wv[b][1], acc[1][0]);
                        acc[0][1] = mfma16(av[b][1][0], wv[b][0], acc[0][1]);
                        acc[1][1] = mfma16(av[b][1][0], wv[b][1], acc[1][1]);
                        if (jj + 1 < HB) {
                            rescale(0, 0);
                            rescale(1, 0);
                            read_rx1(jj + 1, 1);
                            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                            __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                            __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                } else if (UNIT && b == 0) {
                    // a block's first step: each tile moves into the block's units right before its
                    // MFMA, so the MFMAs of the tiles before it run while the multiplies issue
#pragma unroll
                    for (int t = 0; t < TN; ++t)
#pragma unroll
                        for (int i = 0; i < TM; ++i) {
#pragma unroll
                            for (int ii = 0; ii < 4; ++ii) {
                                acc[i][t][4 * ii] *= rxv[t][ii].x;
                                acc[i][t][4 * ii + 1] *= rxv[t][ii].y;
                                acc[i][t][4 * ii + 2] *= rxv[t][ii].z;
                                acc[i][t][4 * ii + 3] *= rxv[t][ii].w;
                            }
                            acc[i][t] = mfma16(av[b][t][0], wv[b][i], acc[i][t]);
                        }
#pragma unroll
                    for (int k = 0; k < TN * TM; ++k) {
                        __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);  // VALU: one tile's rescale
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA: its product
                    }
                    __builtin_amdgcn_sched_barrier(0);
                } else {
#pragma unroll
                    for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                        for (int t = 0; t < TN; ++t)
#pragma unroll
                            for (int i = 0; i < TM; ++i) acc[i][t] = mfma16(av[b][t][hl], wv[b][i], acc[i][t]);
                }
                if (UNIT && !(TN == 2 && TM == 2) && b == 1 && st + 1 < 2 * HB) read_rx((st + 1) >> 1);
                if (st + 1 < 2 * HB) {
                    convert(st + 1, wv[b ^ 1]);  // VALU work spread between the MFMAs
                    if (!UNIT || (b == 1 && !(TN == 2 && TM == 2)))
#pragma unroll
                        for (int k = 0; k < HL * TN * TM; ++k) {
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
                        }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            // per 32-block: the block's accumulator set (acc for even blocks, acc2 for odd) rescaled into
            // the block's weight scale d (unit 1 and a zeroed weight operand where d is zero), then the
            // block's MFMAs straight into it. With two sets, one set's rescale does not wait for MFMAs
            // still writing the other, and the MFMAs of one block overlap the rescale of the next.
            // operand bytes: Q8_0 q + 128, Q4_0 the lane's nibble half in place, Q5_0 its 5-bit quants
            // (nibble + fifth bit, built in q5w); then fp16 k1 * (1024 + byte) + k0 = the weight
            const uint32_t mask = TYPE == T_Q4_0 ? (g ? 0xF0F0F0F0u : 0x0F0F0F0Fu) : 0xFFFFFFFFu;
            const uint32_t flip = TYPE == T_Q8_0 ? 0x80808080u : 0u;
            const float k1 = TYPE == T_Q4_0 && g ? 0.0625f : 1.0f;
            const float k0 = TYPE == T_Q8_0 ? -1152.0f : (TYPE == T_Q5_0 ? -1040.0f : (g ? -72.0f : -1032.0f));
            // Q5_0: elements 16g + 8m + i are nibble half g of qs[8m + i] with fifth bit 16g + 8m + i
            // (dequantize_row_q5_0, src/quant.cpp:1585-1600)
            auto q5w = [&](const WRaw<TYPE>& w, int j, int m, uint32_t& w0, uint32_t& w1) {
                const uint4 raw = w.q[j];
                const uint32_t bits = (w.qh[TYPE == T_Q5_0 ? j : 0] >> (8 * (2 * g + m))) & 0xFFu;
                w0 = (((m ? raw.z : raw.x) >> (4 * g)) & 0x0F0F0F0Fu) | (spread4(bits) << 4);
                w1 = (((m ? raw.w : raw.y) >> (4 * g)) & 0x0F0F0F0Fu) | (spread4(bits >> 4) << 4);
            };
            auto block = [&](int j, auto& A, auto& D) {  // A: an accumulator set, D: its units
                h2v c1[TM], c0[TM];
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const float d = f16_to_f32(cur[i].d[j]);
                    const bool z = d == 0.0f;
                    const float u = z ? 1.0f : d;
                    const float ratio = D[i] * __builtin_amdgcn_rcpf(u);  // ~1 ulp; units only need consistency
                    D[i] = u;
#pragma unroll
                    for (int t = 0; t < TN; ++t)
#pragma unroll
                        for (int r = 0; r < 16; ++r) A[i][t][r] *= ratio;
                    c1[i] = splat(z ? 0.0f : k1);
                    c0[i] = splat(z ? 0.0f : k0);
                }
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    h8 wv[TM], av[TN][HL];
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        if constexpr (TYPE == T_Q5_0) {
                            uint32_t w0, w1;
                            q5w(cur[i], j, m, w0, w1);
                            wv[i] = cvt8(w0, w1, mask, flip, c1[i], c0[i]);
                        } else {
                            const uint4 raw = cur[i].q[j];
                            wv[i] = m ? cvt8(raw.z, raw.w, mask, flip, c1[i], c0[i])
                                      : cvt8(raw.x, raw.y, mask, flip, c1[i], c0[i]);
                        }
                    }
#pragma unroll
                    for (int t = 0; t < TN; ++t)
#pragma unroll
                        for (int hl = 0; hl < HL; ++hl)
                            av[t][hl] = *reinterpret_cast<const h8*>(sa + t * 32 * PB + boff(hl, j, m));
#pragma unroll
                    for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                        for (int t = 0; t < TN; ++t)
#pragma unroll
                            for (int i = 0; i < TM; ++i) A[i][t] = mfma16(av[t][hl], wv[i], A[i][t]);
                }
            };
            static_assert(HB % 2 == 0, "block pairs");
            if constexpr (DUAL) {  // K % 128 == 0: every half-unit holds HB full blocks
#pragma unroll
                for (int j = 0; j < HB; j += 2) {
                    block(j, acc, dl);
                    block(j + 1, acc2, dl2);
                }
            } else if constexpr (!Q4K) {
                // software pipelined as the Q4_K path: step st = (block st / 2, K-half st % 2); the next
                // step's LDS reads and weight conversion go out around this step's MFMAs. At a block's
                // first step each tile is rescaled into the block's unit right before its own hi MFMA,
                // so the MFMAs of the tiles before it run while the multiplies issue.
                h8 av[2][TN][HL];
                h8 wv[2][TM];
                h2v c1[TM], c0[TM];
                float ratio[TM];
                auto scales = [&](int j) {
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        const float d = f16_to_f32(cur[i].d[j]);
                        const bool z = d == 0.0f;
                        const float u = z ? 1.0f : d;
                        ratio[i] = dl[i] * __builtin_amdgcn_rcpf(u);  // ~1 ulp; units only need consistency
                        dl[i] = u;
                        c1[i] = splat(z ? 0.0f : k1);
                        c0[i] = splat(z ? 0.0f : k0);
                    }
                };
                auto read_av = [&](int st, h8(&dst)[TN][HL]) {
#pragma unroll
                    for (int t = 0; t < TN; ++t)
#pragma unroll
                        for (int hl = 0; hl < HL; ++hl)
                            dst[t][hl] = *reinterpret_cast<const h8*>(sa + t * 32 * PB + boff(hl, st >> 1, st & 1));
                };
                auto convert = [&](int st, h8(&dst)[TM]) {
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        const uint4 raw = cur[i].q[st >> 1];
                        dst[i] = (st & 1) ? cvt8(raw.z, raw.w, mask, flip, c1[i], c0[i])
                                          : cvt8(raw.x, raw.y, mask, flip, c1[i], c0[i]);
                    }
                };
                scales(0);
                read_av(0, av[0]);
                convert(0, wv[0]);
#pragma unroll
                for (int st = 0; st < 2 * HB; ++st) {
                    const int b = st & 1;
                    if (st + 1 < 2 * HB) read_av(st + 1, av[b ^ 1]);
                    __builtin_amdgcn_sched_barrier(0);
                    if ((st & 1) == 0) {
#pragma unroll
                        for (int t = 0; t < TN; ++t)
#pragma unroll
                            for (int i = 0; i < TM; ++i) {
#pragma unroll
                                for (int r = 0; r < 16; ++r) acc[i][t][r] *= ratio[i];
                                acc[i][t] = mfma16(av[b][t][0], wv[b][i], acc[i][t]);
                            }
#pragma unroll
                        for (int hl = 1; hl < HL; ++hl)
#pragma unroll
                            for (int t = 0; t < TN; ++t)
#pragma unroll
                                for (int i = 0; i < TM; ++i) acc[i][t] = mfma16(av[b][t][hl], wv[b][i], acc[i][t]);
#pragma unroll
                        for (int k = 0; k < TN * TM; ++k) {
                            __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);  // VALU: one tile's rescale
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA: its hi product
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    } else {
#pragma unroll
                        for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                            for (int t = 0; t < TN; ++t)
#pragma unroll
                                for (int i = 0; i < TM; ++i) acc[i][t] = mfma16(av[b][t][hl], wv[b][i], acc[i][t]);
                    }
                    if (st + 1 < 2 * HB) {
                        if (!((st + 1) & 1)) scales((st + 1) >> 1);  // the next block's unit and operand constants
                        convert(st + 1, wv[b ^ 1]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    };

    for (int h = h0; h < h1; h += 2) {
        half(h, Parity<false>{}, wa, wb);
        if (h + 1 < h1) half(h + 1, Parity<true>{}, wb, wa);
    }

    // ------------------------------------------------------------ epilogue
    if (active) {  // back to natural units: the row's unit (RESCALE) and the token's exponent
        const float* pe = sm.st[(h1 - 1) & 1].pe + pbase;
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const float4 v = *reinterpret_cast<const float4*>(pe + 32 * t + 8 * ii + 4 * g);
                const float pv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        if constexpr (!DUAL)
                            acc[i][t][4 * ii + c] *= pv[c] * dl[i];
                        else  // both sets, back to natural units
                            acc[i][t][4 * ii + c] = (acc[i][t][4 * ii + c] * dl[i] + acc2[i][t][4 * ii + c] * dl2[i]) * pv[c];
                    }
            }
    }
    if constexpr (GATEUP) {
        // h = SiLU(g) * u in registers, written transposed to LDS: [pair][row of the workgroup]
        constexpr int HLD = A_::RW * 32 + 4;              // h row stride (floats)
        float* hs = reinterpret_cast<float*>(&sm.st[0]);  // [128 pairs][HLD], over both stage buffers
        static_assert((size_t)BN * HLD * 4 <= 2 * sizeof(St), "epilogue buffer");
        __syncthreads();  // every wave is done with the stage buffers
        if (active) {
#pragma unroll
            for (int t = 0; t < TN; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float gv = acc[0][t][r], uv = acc[1][t][r];
                    const int pr = pbase + 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
                    hs[pr * HLD + rw * 32 + n] = gated(gv, uv, W0.act);  // SwiGLU / GELU
                }
        }
        __syncthreads();
        // Q8_0 of h (quantize_row_q8_0 over the down projection's K = these rows), one thread per
        // (pair, 32-row block = gate/up row tile)
        for (int it = tid; it < A_::RW * BN; it += NTH) {
            const int pr = it % BN, b = it / BN;
            const int blk = rg * A_::RW + b;
            if (pr >= cnt || blk >= W0.nrt) continue;
            const size_t p = (size_t)(p0 + pr);
            const float* hv = hs + pr * HLD + b * 32;
            float v[32];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const float4 f = *reinterpret_cast<const float4*>(hv + 4 * c);
                v[4 * c] = f.x;
                v[4 * c + 1] = f.y;
                v[4 * c + 2] = f.z;
                v[4 * c + 3] = f.w;
            }
            if (hf) {
                float* fd = hf + p * (size_t)hf_ld + blk * 32;
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    *reinterpret_cast<float4*>(fd + 4 * c) = make_float4(v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]);
            }
            if (!hq.q) continue;
            float amax = 0.0f;
#pragma unroll
            for (int c = 0; c < 32; ++c) amax = fmaxf(amax, __builtin_fabsf(v[c]));
            const float d = amax / 127.0f;
            const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
            int s = 0;
            uint32_t w[8];
#pragma unroll
            for (int c = 0; c < 32; ++c) {
                float r = round_away(v[c] * id);
                r = fminf(fmaxf(r, -127.0f), 127.0f);
                const int q = (int)r;
                s += q;
                if ((c & 3) == 0) w[c >> 2] = 0;
                w[c >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (c & 3));
            }
            uint4* qd = reinterpret_cast<uint4*>(hq.q + p * (size_t)hq.K + blk * 32);
            qd[0] = make_uint4(w[0], w[1], w[2], w[3]);
            qd[1] = make_uint4(w[4], w[5], w[6], w[7]);
            hq.s[p * (size_t)(hq.K / 32) + blk] = make_float2(f16_to_f32(f32_to_f16_trunc(d)), (float)s);
        }
    } else {
        if (!active) return;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int rt = rt0 + i;
            if (rt >= W0.nrt) continue;
#pragma unroll
            for (int t = 0; t < TN; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int pr = pbase + 32 * t + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (pr < cnt) y[(size_t)kp * ystride + (size_t)(p0 + pr) * W0.rows + rt * 32 + n] = acc[i][t][r];
                }
        }
    }
}

// Min-term table of a repacked Q4_K matrix, one thread per (expert, row tile,
// super-block, row): the bf16 pieces of -dmin * m_j / u (u = d, 1 where d is
// zero) for the 8 sub-blocks, in the unit the GEMM's accumulator uses for that
// super-block.  -dmin * m_j is exact in fp32 (11-bit x 6-bit); the division
// rounds once; the split is exact.
// Also the GEMM's A-operand scale of each sub-block J (fp16, exact): the weight fragment holds 1024 + v
// with v = q for Q5_K and Q4_K low nibbles, v = 16 q for Q4_K high nibbles, and s1 (1024 + v) - 1024 s1 =
// sc_J q in one fused fp16 fma, with s1 = sc_J (sc_J / 16 for high nibbles), zero where d is zero.
// Converting the 6-bit scales in the kernel cost ~90 VALU instructions per super-block and wave of the
// gate/up GEMM.
__global__ void __launch_bounds__(256) k_min_table(QMat m, uint8_t* mn) {
    const size_t n = (size_t)m.n_mats * m.nrt * m.nkb * 32;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n) return;
    const size_t t = idx / 32, row = idx % 32;  // t = (e * nrt + rt) * nkb + super-block
    const uint4 hd = ld16(m.sc + (t * 32 + row) * 16);
    const float d = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
    const float u = d == 0.0f ? 1.0f : d;
    uint32_t pw[3][4], cw[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        uint16_t p[3][2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            int sc, mv;
            hdr_scale_min(hd, j + k, sc, mv);
            split3((-dmin * (float)mv) / u, p[0][k], p[1][k], p[2][k]);
            const bool hi = m.type == T_Q4_K && ((j + k) & 1);
            const float sv = d == 0.0f ? 0.0f : (float)sc;
            const _Float16 s1 = (_Float16)(hi ? sv * 0.0625f : sv);
            if (k == 0) cw[j / 2] = __builtin_bit_cast(uint16_t, s1);
            else cw[j / 2] |= (uint32_t)__builtin_bit_cast(uint16_t, s1) << 16;
        }
#pragma unroll
        for (int c = 0; c < 3; ++c) pw[c][j / 2] = (uint32_t)p[c][0] | ((uint32_t)p[c][1] << 16);
    }
    uint8_t* base = mn + t * MN_SB + row * 16;
#pragma unroll
    for (int c = 0; c < 3; ++c)
        *reinterpret_cast<uint4*>(base + c * 512) = make_uint4(pw[c][0], pw[c][1], pw[c][2], pw[c][3]);
    *reinterpret_cast<uint4*>(base + MN_CS) = make_uint4(cw[0], cw[1], cw[2], cw[3]);
}

void launch_min_table(const QMat& m, uint8_t* mn, hipStream_t st) {
    const size_t n = (size_t)m.n_mats * m.nrt * m.nkb * 32;
    hipLaunchKernelGGL(k_min_table, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, m, mn);
}

// Workgroup shape: waves, row tiles and pair tiles per wave, pairs per
// workgroup (BN) and workgroups per CU (WGS; the registers are budgeted for
// WGS * GW / 4 waves per SIMD).  Gate/up stages 64 pairs (hi and lo, 72 KB of
// LDS) and the hi-only down GEMM 128 pairs (78 KB), so two workgroups share a
// CU and one's staging waits overlap the other's matrix-core work.
#ifndef JX_GEMM_GU_GW
#define JX_GEMM_GU_GW 4
#endif
#ifndef JX_GEMM_GU_TN
#define JX_GEMM_GU_TN 2
#endif
#ifndef JX_GEMM_GU_WGS
#define JX_GEMM_GU_WGS 2
#endif
#ifndef JX_GEMM_GU_BN
#define JX_GEMM_GU_BN 64
#endif
#ifndef JX_DOWN_GW
#define JX_DOWN_GW 4
#endif
#ifndef JX_DOWN_TM
#define JX_DOWN_TM 1
#endif
#ifndef JX_DOWN_TN
#define JX_DOWN_TN 4
#endif
#ifndef JX_DOWN_WGS
#define JX_DOWN_WGS 2
#endif
// Row groups per band of the workgroup order (0: all of them).  Gate/up: 8
// (with the XCD-balanced item mapping, Qwen3-shaped 2048 tokens 384 -> 354 us,
// the other shapes unchanged; 2 and 16 slower); down: 4 (2 and 8 slower).
#ifndef JX_GEMM_GU_RC
#define JX_GEMM_GU_RC 8
#endif
#ifndef JX_DOWN_RC
#define JX_DOWN_RC 4
#endif
template <int TYPE, bool GATEUP>
struct Shape {
    static constexpr int GW = GATEUP ? JX_GEMM_GU_GW : JX_DOWN_GW;
    static constexpr int TM = GATEUP ? 2 : JX_DOWN_TM;
    static constexpr int TN = GATEUP ? JX_GEMM_GU_TN : JX_DOWN_TN;
    static constexpr int WPE = (GATEUP ? JX_GEMM_GU_WGS : JX_DOWN_WGS) * GW / 4;
    static constexpr int BN = GATEUP ? JX_GEMM_GU_BN : MFMA_BN;
    static constexpr int RC = GATEUP ? JX_GEMM_GU_RC : JX_DOWN_RC;
};

// Down over fewer pairs per expert (batched decode, where fp32-activation downs have no GEMV form on the
// matrix cores, and prefill up to ~256 pairs per expert): 64-pair tile parts (partial tiles waste half
// as much) and two pair tiles per wave, 40 KB of LDS per workgroup, and as many workgroups per CU as the
// registers allow without spills: 3 (Q6_K: 4; Q5_0: 2, whose 3-wave build spills), so more weight loads
// are in flight.  Measured DeepSeek-V2-Lite-shaped, weights from HBM: Q4_K (fp32 activations) 32
// tokens 63.6 -> 49.1 us, 8 tokens 49.3 -> 30.1 us; Q5_0 at 32 tokens 71.6 -> 50.9 us (prefill:
// MFMA_DOWN_SMALL_MAX_PPE).
template <int TYPE>
struct ShapeSmallDown {
    static constexpr int WPE = TYPE == T_Q6_K ? 4 : TYPE == T_Q5_0 ? 2 : 3;
    static constexpr int GW = 4, TM = 1, TN = 2, BN = 64, RC = JX_DOWN_RC;
};

template <int TYPE, bool GATEUP, typename S = Shape<TYPE, GATEUP>>
static void launch_t(const QMat& w0, const QMat& w1, const ActH& in, const Groups& grp, int tiles_ub, const ActQ8& hq,
                     float* hf, int hf_ld, float* y, hipStream_t st, int KS = 1, size_t ystride = 0) {
    constexpr int rows_per_wg = Arr<GATEUP, S::GW, S::TM, S::TN, S::BN>::WROWS;  // row tiles of each matrix per workgroup
    const int R = (w0.nrt + rows_per_wg - 1) / rows_per_wg;
    const int n_items = R * tiles_ub * (MFMA_BN / S::BN);
    if (n_items <= 0) return;
    const int RC = S::RC > 0 ? std::min(S::RC, R) : R;
    const int grid = n_items * KS;
    hipLaunchKernelGGL((k_wgemm<TYPE, GATEUP, S::GW, S::TM, S::TN, S::WPE, S::BN>), dim3(grid), dim3(S::GW * 64), 0, st,
                       w0, w1, in, grp, R, n_items, RC, hq, hf, hf_ld, y, KS, ystride);
}

void launch_mfma_gateup(const QMat& g, const QMat& u, const ActH& xin, const Groups& grp, int tiles_ub,
                        const ActQ8& hq, float* hf, hipStream_t st) {
    const int hf_ld = ((g.rows + 255) / 256) * 256;
    // Q4_K reads the block-unit form, the others the hi/lo form (the caller allocates the forms its
    // matrices need; a missing one is a caller bug, and nothing is launched on null pointers)
    const bool unit = g.type == T_Q4_K || g.type == T_Q5_K;
    if (unit ? !(xin.q16 && xin.rx && xin.pu && xin.xu) : !(xin.hl && xin.pe)) return;
    switch (g.type) {
        case T_Q4_0: launch_t<T_Q4_0, true>(g, u, xin, grp, tiles_ub, hq, hf, hf_ld, nullptr, st); break;
        case T_Q8_0: launch_t<T_Q8_0, true>(g, u, xin, grp, tiles_ub, hq, hf, hf_ld, nullptr, st); break;
        case T_Q4_K: launch_t<T_Q4_K, true>(g, u, xin, grp, tiles_ub, hq, hf, hf_ld, nullptr, st); break;
        case T_Q5_K: launch_t<T_Q5_K, true>(g, u, xin, grp, tiles_ub, hq, hf, hf_ld, nullptr, st); break;
        default: break;  // Q5_0 / Q6_K gate/up: GEMV only (gemm_gateup_ok)
    }
}

bool gemm_gateup_ok(int type) { return type == T_Q4_0 || type == T_Q8_0 || type == T_Q4_K || type == T_Q5_K; }

int mfma_down_ksplit(int K) { return K >= MFMA_DOWN_KSPLIT_MIN_K ? 2 : 1; }

template <int TYPE>
static void down_t(const QMat& dn, const ActH& hin, const Groups& grp, int tiles_ub, float* y, hipStream_t st, int KS,
                   size_t ystride, bool small) {
    const ActQ8 none{};
    if (small) launch_t<TYPE, false, ShapeSmallDown<TYPE>>(dn, dn, hin, grp, tiles_ub, none, nullptr, 0, y, st, KS, ystride);
    else launch_t<TYPE, false>(dn, dn, hin, grp, tiles_ub, none, nullptr, 0, y, st, KS, ystride);
}

void launch_mfma_down(const QMat& dn, const ActH& hin, const Groups& grp, int tiles_ub, float* y, hipStream_t st,
                      int KS, size_t ystride, bool small) {
    switch (dn.type) {
        case T_Q4_0: down_t<T_Q4_0>(dn, hin, grp, tiles_ub, y, st, KS, ystride, small); break;
        case T_Q8_0: down_t<T_Q8_0>(dn, hin, grp, tiles_ub, y, st, KS, ystride, small); break;
        case T_Q4_K: down_t<T_Q4_K>(dn, hin, grp, tiles_ub, y, st, KS, ystride, small); break;
        case T_Q5_0: down_t<T_Q5_0>(dn, hin, grp, tiles_ub, y, st, KS, ystride, small); break;
        case T_Q5_K: down_t<T_Q5_K>(dn, hin, grp, tiles_ub, y, st, KS, ystride, small); break;
        case T_Q6_K: down_t<T_Q6_K>(dn, hin, grp, tiles_ub, y, st, KS, ystride, small); break;
        default: break;
    }
}

}  // namespace jx

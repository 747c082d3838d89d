// Kernel argument blocks and host-side launchers of the MoE expert path.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace jx {

// One projection (gate, up or down) of every expert, repacked in HBM into
// tiles of 32 rows so a wave's 32 lanes read 32 rows' 16-byte chunks of the
// same K-block as one contiguous 512-byte run:
//   Q4_0  qs  [e][rt][b][32 rows][16 B]           sc  [e][rt][b][32] fp16 d
//   Q8_0  qs  [e][rt][b][2 halves][32 rows][16 B]  sc  [e][rt][b][32] fp16 d
//   Q4_K  qs  [e][rt][sb][4 pairs][2 halves][32 rows][16 B]
//         sc  [e][rt][sb][32 rows][16 B]  = (d, dmin, scales[12]) headers
//   Q5_0  qs  [e][rt][b][32 rows][16 B]           sc  [e][rt][b][32] fp16 d
//         ex  [e][rt][b][32] u32 qh (fifth bits)
//   Q5_K  qs, sc as Q4_K;  ex [e][rt][sb][2 halves][32 rows][16 B] = qh bytes 16h..16h+15
//   Q6_K  qs  [e][rt][sb][2 halves n][6 chunks c][32 rows][16 B]: c < 4 = ql bytes 64n + 16c ..,
//             c = 4, 5 = qh bytes 32n + 16(c - 4) ..
//         sc  [e][rt][sb][32 rows][16 B] = the 16 int8 sub-block scales
//         ex  [e][rt][sb][32] fp16 d
// Byte totals of qs+sc(+ex) equal the GGUF tensor (18/34/144/22/176/210 B per block).
constexpr int MN_SB = 2048, MN_CS = 1536;  // QMat::mn bytes per (row tile, super-block); scales offset

struct QMat {
    int type = 0;
    int rows = 0;       // per expert, multiple of 32
    int cols = 0;       // K
    int nrt = 0;        // rows / 32
    int nkb = 0;        // K-units: 32-blocks (Q4_0/Q5_0/Q8_0) or 256-super-blocks (Q4_K/Q5_K/Q6_K)
    const uint8_t* qs = nullptr;
    const uint8_t* sc = nullptr;
    size_t qs_es = 0, sc_es = 0;  // per-expert strides (bytes)
    int n_mats = 0;     // experts held
    // Zeroed QMAT_PAD-byte tails of the qs / sc allocations: loads a kernel
    // issues for units it will not use read here (uniform instruction streams).
    const uint8_t* pad_qs = nullptr;
    const uint8_t* pad_sc = nullptr;
    // Third region of the five- and six-bit formats (Q5_0 / Q5_K high bits, Q6_K d), its
    // per-expert stride and zeroed pad; null for the others.
    const uint8_t* ex = nullptr;
    size_t ex_es = 0;
    const uint8_t* pad_ex = nullptr;
    // Q4_K / Q5_K table for the matrix-core GEMMs (launch_min_table; null for other types
    // and for matrices only the GEMVs read): per (expert, row tile, super-block) MN_SB
    // bytes, 3 x [32 rows][16 B] = the bf16 pieces (hi, mid, lo) of -dmin * m_j / u for
    // the 8 sub-blocks j, u = d (1 where d is zero), then at MN_CS [32 rows][16 B] = the
    // fp16 A-operand scales s1 of the 8 sub-blocks.
    const uint8_t* mn = nullptr;
    size_t mn_es = 0;  // per-expert stride (bytes)
    // Gated activation applied to this matrix's outputs when it is the gate of
    // a gate/up pair (ACT_SILU or ACT_GELU_TANH); unused otherwise.
    int act = 0;
    // Rows that exist when `rows` was padded to whole tiles with zero blocks (a
    // single matrix of any row count, jx_qmatrix_create); the single-token down
    // GEMV writes outputs for these only.  0: every row.
    int valid_rows = 0;
};
constexpr size_t QMAT_PAD = 8192;

// Q8_0 activations on the device: q [rows][K] int8, s [rows][K/32] = (fp16-truncated
// scale as fp32, sum of the 32 quants as fp32).
struct ActQ8 {
    int8_t* q = nullptr;
    float2* s = nullptr;
    int K = 0;
};

// Q8_0 activations in the form the matrix-core GEMMs consume (K % 128 == 0):
//   hl [rows][KH][256]   per 128-element half-unit: fp16 hi x128, then lo x128,
//                        of dx * q * 2^-E (an exact split of the dequantized
//                        value scaled into fp16 range)
//   pe [rows][KH]        2^E of each half-unit, one E per row (the GEMMs apply
//                        the last half-unit's): the exponent of the row's largest
//                        block scale - 7 for Q8_0 rows (x from the router kernels,
//                        h from k_q8_to_acth), so |dx * q| * 2^-E < 2^15; the
//                        exponent of max |h| - 14 for fp32 rows (k_f32_to_acth)
//   xm [rows][KU][3][8]  per 256-element unit: bf16 pieces (hi, mid, lo) of
//                        dx * sum(q) (fp32 rows: the block sum) times 2^-E for its
//                        8 blocks (Q4_K min term)
// and, for the Q4_K gate/up GEMM, the block-unit form (each form is written
// where its pointers are set):
//   q16 [rows][K]        the quants q as fp16 (exact)
//   rx [rows][K/32]      u(b-1) / u(b) per 32-block b, where the unit u(b) is the
//                        block's scale dx, the previous unit where dx is zero, and
//                        1 before the first nonzero scale (rx = 1 for block 0)
//   pu [rows][KH]        u of the last block of each half-unit
//   xu [rows][KU][3][8]  as xm, of dx * sum(q) / u(8s + 3) for super-block s
struct ActH {
    uint16_t* hl = nullptr;
    float* pe = nullptr;
    uint16_t* xm = nullptr;
    uint16_t* q16 = nullptr;
    float* rx = nullptr;
    float* pu = nullptr;
    uint16_t* xu = nullptr;
    int K = 0;
    int KH = 0;  // K / 128
    int KU = 0;  // ceil(K / 256)
};

// Token -> expert grouping produced by the dispatch kernel.
struct Groups {
    const int* counts = nullptr;  // [E]
    const int* offs = nullptr;    // [E+1]
    const int* act = nullptr;     // [E] active experts, increasing id
    const int* n_act = nullptr;   // [1]
    const int4* slots = nullptr;  // [E] per active-expert slot: (expert, first pair, pair count, first
                                  // pair's token); slots >= n_act hold a zero count
    const int* pair_tok = nullptr;  // [P] sorted pair -> token
    const int4* tiles = nullptr;  // [T] (expert, first pair, pair count, 0) MFMA tiles
    const int* n_tiles = nullptr; // [1]
    int top_k = 1;
    int identity = 0;             // shared expert: pair p is token p, one group of n_tok (chunk 0) or
    int chunk = 0;                // groups of `chunk` tokens, group s from token s * chunk
    int n_tok = 0;
    // Few-token decode (n_tok <= ROUTE_SMALL_MAX_N, n_experts <= SMALL_GROUP_MAX_E): when set,
    // each block derives its slot's group from the router logits [n_tok][n_experts] itself
    // instead of reading dispatch tables (small_group in jxmoe_dispatch.h).
    const float* logits = nullptr;
    int n_experts = 0;
    // > 0: the multi-token GEMVs take only the experts with fewer pairs than this (the GEMMs take the
    // others: launch_dispatch's cold_max)
    int cold_max = 0;
};
constexpr int SMALL_GROUP_MAX_E = 128;
constexpr int MAX_SLOTS_DEC = 16;  // routed slots (top_k) of the fused one-token step

constexpr int MFMA_BN = 128;  // pairs per matrix-core GEMM tile
// shared expert on the matrix cores from this many tokens (one dense expert fills few GEMM
// workgroups below that: 44 gate/up and 16 down workgroups for a 5632 x 2048 expert at 64 tokens).
// The 16-token matrix-core GEMV in one group per 16 tokens is faster up to 256 tokens for the formats
// it runs at 3 waves per SIMD (Qwen1.5-shaped, Q4_0: 64 tokens 233 -> 177 us per step), up to 64 for
// Q4_K / Q6_K (2 waves per SIMD; DeepSeek-V2-Lite-shaped).
constexpr int MFMA_MIN_SHARED_TOKENS = 256;
constexpr int MFMA_MIN_SHARED_TOKENS_KQ = 64;  // Q4_K / Q6_K shared experts

// The weighted combine folded into the down GEMV (few-token decode with at most two
// contributions per output element: top_k <= 2 and no shared expert): out [n][d] is
// zeroed by the first kernel of the forward and each down block adds p * y for its
// rows atomically.  Two adds onto an exact zero commute, so the result does not
// depend on their order.
struct CombineOut {
    float* out = nullptr;         // [n][d]; null: the down GEMV writes y[pair][d] instead
    const float* probs = nullptr; // [n][k] softmax weights in selection order
    const int* ids = nullptr;     // [n][k] selected experts
    int k = 0;
};

struct RouteArgs {
    const float* x;        // [n][d]
    int n, d, E, k;
    const float* router;   // [E][d] fp32 (F16 / BF16 routers converted exactly at upload)
    const float* bias;     // [E] or null
    const float* shgate;   // [d] or null
    ActQ8 xq;              // out: Q8_0 of x (int8 + (scale, sum))
    ActH xh;               // out: Q8_0 of x for the matrix-core GEMMs (forms with null pointers: not written)
    int* ids;              // [n][k]
    float* probs;          // [n][k]
    float* shscale;        // [n]
    float* logits;         // [n][E] or null
    const float* router_cm;  // the router rows, then the shared gate, chain-major (chain_rows)
    float* zero_out = nullptr;  // few-token routers: zero this many floats here first (the folded
    int zero_count = 0;         // combine's output; CombineOut)
    int chain8 = 0;             // router rows (not the shared gate) in the F16 / BF16 dot order
};

// Outputs of the token -> expert dispatch (the device side of Groups).
struct DispatchOut {
    int* counts;    // [E]
    int* offs;      // [E+1]
    int* act;       // [E]
    int* n_act;     // [1]
    int* pair_tok;  // [n*k]
    int* pos_of;    // [n*k] flat (token, slot) -> sorted pair
    int4* tiles;    // MFMA tiles
    int* n_tiles;   // [1]
    int4* slots;    // [E] see Groups::slots
};

// Dispatch tables written by block (0, 0) of the routed gate/up GEMV when its
// groups come from the logits (the few-token decode path), for the kernels
// after it and the caller's outputs.
struct SmallTail {
    RouteArgs a;      // n, E, k, logits, ids, probs, shscale (raw shared-gate logits on entry), shgate
    DispatchOut o;
    int on = 0;
};

void launch_route(const RouteArgs& a, hipStream_t st);
// Host side: nrows rows of d floats in the chain-major order launch_route reads
// (out holds nrows * 16 * chain_stride(d) floats).
int chain_stride(int d);
void chain_rows(const float* rows, int nrows, int d, float* out);
// With cold_max > 0 the tile table (and n_tiles) holds only the experts with at least cold_max pairs:
// the matrix-core GEMMs take those, the GEMVs the others (Groups::cold_max).
void launch_dispatch(const int* ids, int nk, int E, int top_k, const DispatchOut& o, hipStream_t st,
                     int cold_max = 0);

// A dense shared expert's blocks appended to a routed multi-token GEMV launch (k_gemv_mxt): its own
// matrices and outputs over groups of 16 tokens, so its few long-lived blocks run among the routed
// ones instead of beside them from a second stream.  Gate/up: g and u, h into hq (and fp32 hf when its
// down takes fp32 h).  Down: g is the shared down over the Q8_0 h in hq; its K is cut into `kparts`
// ranges of whole units, part p writing y + p * n * rows, which the combine adds in part order.
struct SharedPart {
    QMat g, u;
    Groups grp;           // identity groups of `chunk` = 16 tokens
    int slots = 0;        // token groups
    ActQ8 hq;
    float* hf = nullptr;
    int hf_ld = 0;
    float* y = nullptr;
    int kparts = 1;
    int blocks0 = 0;      // set by the launcher: the routed blocks ahead of the shared ones
};
// The K parts of a shared down of Ks columns appended to a routed down of K columns: as many as make
// a shared block's unit range no longer than a routed block's (at most SHARED_KPARTS_MAX).
constexpr int SHARED_KPARTS_MAX = 8;
int shared_down_kparts(int type, int K, int Ks);
// Whether a GEMV launch of nrt row tiles over `slots` groups at `tb` tokens per group takes the multi-tile
// matrix-core form (k_gemv_mxt) for this weight format, with Q8_0 activations.
bool gemv_mxt_takes(int type, bool gateup, int nrt, int slots, int tb);
// Whether a shared gate/up of snrt row tiles over sslots token groups joins that launch: the multi-tile
// form, and the routed and shared blocks together within one resident round of 2-wave blocks (past it
// the launch takes 4-wave blocks or a second round, which measured slower than the shared expert on
// its own stream: Qwen1.5-shaped 64 tokens 141 -> 144 us, DeepSeek-V2-Lite-shaped 32 tokens 132 -> 142 us).
bool gemv_gateup_joins(int type, int nrt, int slots, int tb, int snrt, int sslots);

// Decode regime: gate+up dequant-GEMV with SwiGLU and Q8_0 re-quantization.
// Output rows are sorted pairs (routed) or tokens (shared).  With xf, the
// fp32-activation dots over rows of xf_ld floats (zero-padded to whole K-units;
// one token or groups of 4) instead of the Q8_0 form xq.  With sh, the shared expert's blocks join the
// launch where it takes the multi-tile matrix-core form with the same weight format (returns whether
// they did; otherwise the caller launches the shared expert itself).
bool launch_gemv_gateup(const QMat& g, const QMat& u, const ActQ8& xq, const Groups& grp, int slots,
                        int tb, ActQ8 hq, float* hf, hipStream_t st, const SmallTail* tail = nullptr,
                        const float* xf = nullptr, int xf_ld = 0, SharedPart* sh = nullptr);
// Largest K the GEMVs accept for token groups of `tb` rows (gate/up or down,
// Q8_0 or fp32 activations).
int gemv_max_k(bool gateup, int tb, bool f32);
// Decode regime: down projection over Q8_0 (hq) or fp32 (hf) activations into y[pair][d].
// With sh, the shared down's blocks as for launch_gemv_gateup.
bool launch_gemv_down(const QMat& dn, const ActQ8& hq, const float* hf, int hf_ld, const Groups& grp,
                      int slots, int tb, float* y, hipStream_t st, const CombineOut& comb = CombineOut{},
                      SharedPart* sh = nullptr);
// Decode regime, fp32 h (no Q8_0 form): the down projection on fp16 matrix cores over h's hi form (hh,
// k_f32_to_acth), a few tokens per expert; built for Q4_K and Q5_0 where the staged tokens fit the LDS.
bool gemv_down_f16_fits(int type, int K);
void launch_gemv_down_f16(const QMat& dn, const ActH& hh, const Groups& grp, int slots, float* y, hipStream_t st);
// Prefill regime: matrix-core grouped GEMMs over the dispatch tile table.
// gate/up writes SwiGLU(h) as Q8_0 (hq.q != null; the down GEMM takes it after
// launch_q8_to_acth) and/or fp32 (hf != null).
void launch_mfma_gateup(const QMat& g, const QMat& u, const ActH& xin, const Groups& grp, int tiles_ub,
                        const ActQ8& hq, float* hf, hipStream_t st);
// KS > 1: the K range split over KS workgroups per item (whole super-blocks each), part q of the
// output at y + q * ystride (the combine adds the parts in order).  small: few pairs per expert (the
// 64-pair tile form at more workgroups per CU).
void launch_mfma_down(const QMat& dn, const ActH& hin, const Groups& grp, int tiles_ub, float* y, hipStream_t st,
                      int KS = 1, size_t ystride = 0, bool small = false);
// Down GEMM in the small form up to this many (token, slot) pairs per expert on average (measured:
// Mixtral-shaped 512 tokens, 128 per expert, 239 -> 202 us; Qwen3-shaped 2048 tokens with Zipf-skewed
// routing 143 -> 124 us; DeepSeek-V2-Lite-shaped 2048 tokens 130 -> 122 us; Mixtral-shaped 2048 tokens,
// 512 per expert, 566 us in the 128-pair form against 590 in the small one).
constexpr int MFMA_DOWN_SMALL_MAX_PPE = 256;
// K-split of the down GEMM for a K of K: two parts from MFMA_DOWN_KSPLIT_MIN_K on (twice the
// workgroups, finer rounds; measured Mixtral-shaped, K 14336: 2048 tokens 634 -> 575 us, 256 tokens
// 155 -> 133 us; at K 768 - 1408 the per-workgroup overhead makes it slower).
constexpr int MFMA_DOWN_KSPLIT_MIN_K = 8192;
int mfma_down_ksplit(int K);
// Weight types the matrix-core gate/up GEMM takes (Q5_0 has no Q8_0-activation form; Q6_K's sc * q
// operand is not exact in fp16, and gate/up products must be: h is re-quantized).
bool gemm_gateup_ok(int type);
// Fill m.mn (m.n_mats * m.nrt * m.nkb * MN_SB bytes) from a repacked Q4_K or Q5_K matrix.
void launch_min_table(const QMat& m, uint8_t* mn, hipStream_t st);

// acc[t] = sum_s p[t][s] * y[pos(t,s)] (+ shscale[t] * ysh[t]), fma in selection order (y2 != null:
// each y row is y[p] + y2[p], the K-split down GEMM's two parts added in that order);
// out[t] = acc[t], or resid[t] + acc[t] (resid != null), or with post_w:
// (resid[t] +) rms_norm(acc[t], post_w, eps) (post_ffw_norm, transformer.cpp:2758-2764).
void launch_combine(int n, int d, int k, const float* probs, const int* pos_of, const float* y, const float* ysh,
                    const float* shscale, float* out, hipStream_t st, const float* resid = nullptr,
                    const float* post_w = nullptr, float eps = 0.0f, const float* y2 = nullptr,
                    int shparts = 1);  // ysh in shparts K parts of n * d floats, added in part order
// MoETransformerEngine::rms_norm (transformer.cpp:67-73) of rows x d floats: out = x * inv * w.
void launch_rms_norm(const float* x, const float* w, int rows, int d, float eps, float* out, hipStream_t st);

// Decode routing for n <= ROUTE_SMALL_MAX_N tokens and E <= SMALL_GROUP_MAX_E
// experts without a dispatch launch: router logits and Q8_0 of x (one block
// per router row); the routed gate/up GEMV then groups from the logits and
// writes the tables (SmallTail).
void launch_route_logits(const RouteArgs& a, hipStream_t st);

// Routing for a few tokens (n <= ROUTE_SMALL_MAX_N), two launches: one block
// per router row (the row and the tokens staged in LDS) writes the logits and
// its share of the Q8_0 activations; then one block ranks, normalises and
// dispatches (replacing launch_dispatch).  The kernel boundary orders the two
// (no device-scope fences, which on a multi-XCD part write back and
// invalidate L2).
constexpr int ROUTE_SMALL_MAX_N = 2;
bool route_small_fits(int n, int d, int E);
void launch_route_small(const RouteArgs& a, const DispatchOut& o, hipStream_t st);

// One-token step in one launch (k_decode1): router rows, dispatch tables, gate/up + SwiGLU + Q8_0
// of h, down (+ the folded combine) as blocks of one grid that hand over through device-coherent
// words.  DecodeSync is the layer's device state, zeroed once at creation; the host counts the
// fused launches of the layer (epoch = 1, 2, ...) and passes the count.
struct DecodeSync {
    uint64_t tag[SMALL_GROUP_MAX_E];  // router row r: (epoch << 32) | bits of its logit
    uint32_t err;                     // nonzero: a bounded wait gave up
    uint32_t pad;
};

struct Decode1Args {
    QMat G, U, D;               // gate, up (d_ff x d), down (d x d_ff); Q8_0-activation formats
    const float* x;             // [d] the token (normalized when the step carries the residual)
    const float* router;        // [E][d] fp32 rows (F16 / BF16 widened exactly at upload)
    const float* bias;          // [E] or null
    int d = 0, E = 0, k = 0, chain8 = 0;
    ActQ8 xq;                   // out: Q8_0 of x (for the caller)
    ActQ8 hq;                   // [k][d_ff] Q8_0 of h, row = slot
    RouteArgs ra;               // logits, ids, probs, shscale of the caller (n = 1)
    DispatchOut o;              // the dispatch tables of the caller
    float* out = nullptr;       // folded combine: [d] zeroed here, p * y added by the down blocks
    float* y = nullptr;         // otherwise: [k][d] per slot, for launch_combine
    DecodeSync* sync = nullptr;
    uint32_t epoch = 0;         // this launch's number among the layer's fused launches (from 1)
    uint32_t htag = 0;          // 1 + epoch % 8191: the tag in the low 13 bits of h's stored scales
    int sh = 0;                 // a shared expert of the routed formats:
    QMat SG, SU, SD;            //   its gate, up (d_ff_shared x d) and down (d x d_ff_shared)
    const float* shgate = nullptr;  // [d] its fp32 gate row (sigmoid weight), or null (weight 1)
    ActQ8 hqs;                  //   [1][d_ff_shared] Q8_0 of its h
    float* ysh = nullptr;       //   [d] its output, for launch_combine
    uint64_t* hw = nullptr;     // k_decode_p: [k][d_ff / 4] words of h, (epoch << 32) | four Q8_0 quants
    uint64_t* hfw = nullptr;    // k_decode1 with fp32 h: [k][d_ff] words, (epoch << 32) | fp32 h
    int hf_ld = 0;              //   h's zero-padded length for the down (whole K-units)
    uint32_t* herr = nullptr;   // host-visible word set (system scope) when a bounded wait gives up
    uint32_t spin_limit = 0;    // polls before a wait gives up
    uint32_t giveup_test = 0;   // nonzero: every wait treats its words as not yet published (error-path test)
};
// Whether k_decode1 is built for this shape: E router rows (+ the shared-expert gate row) <=
// SMALL_GROUP_MAX_E, even k <= MAX_SLOTS_DEC, d % 32 == 0 and d <= 8192, d_ff and the shared d_ff
// (fs, 0: none) <= 16384, gate/up and down formats with Q8_0 activations (a shared expert: the same
// formats as the routed ones).
// With df32 the routed down takes fp32 h (its d_ff has no Q8_0 form for the down's format); sdtype is the
// shared down's format.
bool decode1_fits(int gtype, int dtype, int d, int f, int E, int k, int fs, bool shgate, int sdtype, bool df32);
// Whether the fused launch is the faster one for routed gate/up matrices of gate_nrt row tiles at
// top-k and a shared gate/up of sgate_nrt (0: none).
bool decode1_pays(int gate_nrt, int k, int sgate_nrt);
void launch_decode1(const Decode1Args& a, int gtype, int dtype, hipStream_t st, int sdtype, bool df32);
// The same step as one grid of one 1024-thread block per CU (k_decode_p): every block routes the
// token itself, streams an even share of the gate/up row tiles, then its down tiles once h's tagged
// scale words say the slot is complete; top-2 with the folded combine and no shared expert, for
// layers whose gate/up tiles outnumber the CUs (decode1_pays false).  Returns nonzero when the launch
// fails.
bool decodep_fits(int gtype, int dtype, int d, int f, int E, int k, bool shared, bool fold, int gate_nrt,
                  int down_nrt);
int launch_decode_p(const Decode1Args& a, int gtype, int dtype, hipStream_t st);

// Q8_0 of rows x K fp32 (row-major, K % 32 == 0).
void launch_quantize_q8(const float* x, int rows, int K, ActQ8 out, hipStream_t st);
// dst[r][0 .. kpad) = x[r][0 .. n) then zeros, for rows r (x rows of n floats).
void launch_copy_pad(const float* x, int n, int kpad, float* dst, hipStream_t st, int rows = 1);

// Matrix-core form of existing Q8_0 activations (int8 quants + (scale, sum)).
// lo = false writes only the fp16 hi halves (the down GEMM's operand).
void launch_q8_to_acth(const ActQ8& in, int rows, ActH out, hipStream_t st, bool lo = true);
// Matrix-core form (hi only) of fp32 activation rows [rows][ld] (out.K % 128 == 0, columns up to
// out.K zero-padded).
void launch_f32_to_acth(const float* h, int ld, int rows, ActH out, hipStream_t st);

// Repack a GGUF block matrix set [n_mats][rows][cols] (already on the device
// as raw bytes) into the QMat layout.
void launch_repack(const uint8_t* raw, QMat m, uint8_t* qs, uint8_t* sc, uint8_t* ex, hipStream_t st);

}  // namespace jx

// C-ABI runtime of the MoE expert path: device init, one-time upload and
// repack of a layer, workspace management, the forward pipeline
//   route -> dispatch -> {dequant-GEMV | matrix-core GEMM} x (gate/up, down) -> combine
// and the function-level drop-ins of the reference's math API.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/jxmoe.h"
#include "jxmoe_device.h"
#include "jxmoe_kernels.h"

namespace {

thread_local std::string g_err;
// The device jx_moe_init selected, for the whole process (layers and matrices
// keep their own device; entry points make it current on the calling thread).
std::atomic<int> g_device{-1};

// Scratch of jx_matmul_quant_f32_noalloc: the Q8_0 activations (block scales
// and sums, then the quants) or the zero-padded fp32 copy of one activation
// row of at most NOALLOC_MAX_COLS columns.  Each GPU the library runs on holds
// its own copy until the process ends.  In host code `scratch` names a
// host-side stand-in: kernels and copies take the device address that
// jx_moe_init resolves per device (g_scratch).
constexpr size_t NOALLOC_MAX_COLS = JX_NOALLOC_MAX_COLS;
constexpr size_t NOALLOC_SCRATCH_BYTES = NOALLOC_MAX_COLS * sizeof(float);  // >= the Q8_0 form's 1.25 B/col
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];
constexpr int MAX_DEVICES = 64;
std::atomic<void*> g_scratch[MAX_DEVICES];

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

// One-block-per-CU fused steps (k_decode_p) need every block of the launch resident at once, so two of
// them running at the same time on one GPU (different layers or streams of this process) could each
// hold CUs the other waits for.  The stream of the last such launch that may still be running (an
// asynchronous call's) is kept per device; a launch on another stream while it is set first
// synchronizes the device.  Launches on one stream, and synchronous calls, add nothing.
struct FusedOrder {
    std::mutex mu;
    hipStream_t pending[MAX_DEVICES] = {};
};
FusedOrder g_fused_order;

#define HIPCHK(expr)                                                                              \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess)                                                                     \
            return fail(e_ == hipErrorOutOfMemory ? JX_ERR_NOMEM : JX_ERR_HIP,                    \
                        std::string(#expr) + ": " + hipGetErrorString(e_));                       \
    } while (0)

// IEEE half / bfloat16 bits -> float, exact for every input (the reference's fp16_to_fp32 and
// bf16_to_fp32, src/quant.cpp:876-932; F16C's conversion keeps NaN payloads, as this does).
float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {  // subnormal: normalise
            int k = 0;
            while (!(m & 0x400u)) {
                m <<= 1;
                ++k;
            }
            bits = sign | ((uint32_t)(113 - k) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

float bf16_to_float(uint16_t b) {
    const uint32_t bits = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

bool expert_type_ok(int t) {
    return t == jx::T_Q4_0 || t == jx::T_Q5_0 || t == jx::T_Q8_0 || t == jx::T_Q4_K || t == jx::T_Q5_K ||
           t == jx::T_Q6_K;
}

// ggml_type_size / tensor_byte_size (include/common.h:154-195)
size_t row_bytes(int t, int64_t cols) {
    switch (t) {
        case jx::T_Q4_0: return (size_t)((cols + 31) / 32) * 18;
        case jx::T_Q5_0: return (size_t)((cols + 31) / 32) * 22;
        case jx::T_Q8_0: return (size_t)((cols + 31) / 32) * 34;
        case jx::T_Q4_K: return (size_t)((cols + 255) / 256) * 144;
        case jx::T_Q5_K: return (size_t)((cols + 255) / 256) * 176;
        case jx::T_Q6_K: return (size_t)((cols + 255) / 256) * 210;
        default: return 0;
    }
}

// supports_q8_activation (src/quant.cpp:3881-3893): Q5_0 always takes fp32 activations
bool q8_activation(int t, int64_t cols) {
    if (t == jx::T_Q4_0 || t == jx::T_Q8_0) return cols % 32 == 0;
    if (jx::is_kquant(t)) return cols % 256 == 0;
    return false;
}

struct DevMat {
    jx::QMat m;
    uint8_t* qs = nullptr;
    uint8_t* sc = nullptr;
    uint8_t* ex = nullptr;  // Q5_0 / Q5_K high bits, Q6_K d
    uint8_t* mn = nullptr;  // Q4_K / Q5_K min-term table (matrix-core GEMMs)
    void release() {
        for (uint8_t* p : {qs, sc, ex, mn})
            if (p) (void)hipFree(p);
        qs = sc = ex = mn = nullptr;
    }
};

// Upload n_mats [rows][cols] block matrices and repack them on the device;
// with `gemm`, Q4_K / Q5_K matrices also get the matrix-core GEMMs' min-term table.
int upload_matrix(int type, int n_mats, int rows, int cols, const void* host, DevMat& out, hipStream_t st,
                  bool gemm = false) {
    if (!expert_type_ok(type))
        return fail(JX_ERR_UNSUPPORTED, "expert weight type must be Q4_0, Q5_0, Q8_0, Q4_K, Q5_K or Q6_K");
    if (rows % jx::ROWS_PER_TILE != 0) return fail(JX_ERR_UNSUPPORTED, "matrix rows must be a multiple of 32");
    if (cols % 32 != 0) return fail(JX_ERR_UNSUPPORTED, "matrix cols must be a multiple of 32");
    jx::QMat& m = out.m;
    m.type = type;
    m.rows = rows;
    m.cols = cols;
    m.nrt = rows / jx::ROWS_PER_TILE;
    m.nkb = jx::is_kquant(type) ? (cols + 255) / 256 : cols / 32;
    m.n_mats = n_mats;
    const size_t units = (size_t)rows * m.nkb;
    // bytes per row and K-unit of each region (qs + sc + ex = the GGUF block)
    size_t qs_u = 0, sc_u = 0, ex_u = 0;
    switch (type) {
        case jx::T_Q4_0: qs_u = 16, sc_u = 2; break;
        case jx::T_Q5_0: qs_u = 16, sc_u = 2, ex_u = 4; break;
        case jx::T_Q8_0: qs_u = 32, sc_u = 2; break;
        case jx::T_Q4_K: qs_u = 128, sc_u = 16; break;
        case jx::T_Q5_K: qs_u = 128, sc_u = 16, ex_u = 32; break;
        default: qs_u = 192, sc_u = 16, ex_u = 2; break;  // Q6_K
    }
    m.qs_es = units * qs_u;
    m.sc_es = units * sc_u;
    m.ex_es = units * ex_u;
    // the GEMMs address one expert's matrix with 32-bit offsets (the GEMM table: 4x the headers)
    if (m.qs_es >= ((size_t)1 << 32) || m.sc_es * 4 >= ((size_t)1 << 32))
        return fail(JX_ERR_UNSUPPORTED, "one expert matrix exceeds 4 GiB");
    const size_t raw_bytes = (size_t)n_mats * rows * row_bytes(type, cols);
    uint8_t* raw = nullptr;
    HIPCHK(hipMalloc(&out.qs, m.qs_es * n_mats + jx::QMAT_PAD));
    HIPCHK(hipMalloc(&out.sc, m.sc_es * n_mats + jx::QMAT_PAD));
    HIPCHK(hipMemsetAsync(out.qs + m.qs_es * n_mats, 0, jx::QMAT_PAD, st));
    HIPCHK(hipMemsetAsync(out.sc + m.sc_es * n_mats, 0, jx::QMAT_PAD, st));
    m.pad_qs = out.qs + m.qs_es * n_mats;
    m.pad_sc = out.sc + m.sc_es * n_mats;
    if (ex_u) {
        HIPCHK(hipMalloc(&out.ex, m.ex_es * n_mats + jx::QMAT_PAD));
        HIPCHK(hipMemsetAsync(out.ex + m.ex_es * n_mats, 0, jx::QMAT_PAD, st));
        m.pad_ex = out.ex + m.ex_es * n_mats;
    }
    HIPCHK(hipMalloc(&raw, raw_bytes));
    hipError_t e = hipMemcpyAsync(raw, host, raw_bytes, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) {
        m.qs = out.qs;
        m.sc = out.sc;
        m.ex = out.ex;
        jx::launch_repack(raw, m, out.qs, out.sc, out.ex, st);
        e = hipGetLastError();
    }
    if (e == hipSuccess && gemm && (type == jx::T_Q4_K || type == jx::T_Q5_K)) {
        m.mn_es = (size_t)m.nrt * m.nkb * jx::MN_SB;
        e = hipMalloc(&out.mn, m.mn_es * n_mats);
        if (e == hipSuccess) {
            m.mn = out.mn;
            jx::launch_min_table(m, out.mn, st);
            e = hipGetLastError();
        }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    (void)hipFree(raw);
    if (e != hipSuccess) return fail(JX_ERR_HIP, std::string("weight upload: ") + hipGetErrorString(e));
    return JX_OK;
}

template <typename T>
int dalloc(T*& p, size_t n) {
    if (p) (void)hipFree(p);
    p = nullptr;
    if (n == 0) return JX_OK;
    HIPCHK(hipMalloc(&p, n * sizeof(T)));
    return JX_OK;
}

// Matrix-core activation buffers for `rows` rows of K: the hi/lo form, the
// block-unit form (the Q4_K gate/up input), or both.
struct DevActH {
    jx::ActH a;
    void release() {
        for (void* p : {(void*)a.hl, (void*)a.pe, (void*)a.xm, (void*)a.q16, (void*)a.rx, (void*)a.pu, (void*)a.xu})
            if (p) (void)hipFree(p);
        a = jx::ActH{};
    }
    int alloc(size_t rows, int K, bool hilo = true, bool unit = false) {
        release();
        a.K = K;
        a.KH = K / 128;
        a.KU = (K + 255) / 256;
        if (K % 128 != 0) return JX_OK;  // the matrix-core path is not used for this shape
        if (hilo) {
            HIPCHK(hipMalloc(&a.hl, rows * a.KH * 256 * sizeof(uint16_t)));
            HIPCHK(hipMalloc(&a.pe, rows * a.KH * sizeof(float)));
            HIPCHK(hipMalloc(&a.xm, rows * a.KU * 24 * sizeof(uint16_t)));
        }
        if (unit) {
            HIPCHK(hipMalloc(&a.q16, rows * (size_t)K * sizeof(uint16_t)));
            HIPCHK(hipMalloc(&a.rx, rows * (size_t)(K / 32) * sizeof(float)));
            HIPCHK(hipMalloc(&a.pu, rows * a.KH * sizeof(float)));
            HIPCHK(hipMalloc(&a.xu, rows * a.KU * 24 * sizeof(uint16_t)));
        }
        return JX_OK;
    }
};

struct Prof {
    bool on = false;
    std::vector<hipEvent_t> pool;
    size_t used = 0;
    std::vector<std::pair<std::string, size_t>> pending;  // name, event index (start; end = +1)
    std::map<std::string, std::pair<double, int64_t>> acc;
};

}  // namespace

struct jx_moe_layer {
    int device = 0;
    int E = 0, k = 0, d = 0, F = 0, Fs = 0;
    bool shared = false, down_f32 = false, sdown_f32 = false;
    // gate/up over fp32 activations (no Q8_0 form at d_model: Q5_0, or a K-quant with d_model % 256 != 0),
    // routed / shared; they read xf, x zero-padded to dpad columns
    bool gu_f32 = false, sgu_f32 = false;
    int dpad = 0;
    float* router = nullptr;
    float* ffn_norm = nullptr;   // [d] or null (weight 1)
    float* post_norm = nullptr;  // [d] or null (no post_ffw_norm)
    float eps = 1e-5f;
    float* xn = nullptr;         // workspace: rms_norm of the residual stream (JX_FWD_RESIDUAL)
    float* router_cm = nullptr;  // router rows + shared gate, chain-major
    float* bias = nullptr;
    float* shgate = nullptr;
    DevMat gate, up, down, sgate, sup, sdown;
    // workspace
    int cap = 0;
    float *x = nullptr, *out = nullptr, *probs = nullptr, *shscale = nullptr, *logits = nullptr;
    int *ids = nullptr, *counts = nullptr, *offs = nullptr, *act = nullptr, *n_act = nullptr, *pair_tok = nullptr,
        *pos_of = nullptr, *n_tiles = nullptr;
    int4* tiles = nullptr;
    int4* slots = nullptr;
    jx::ActQ8 xq, hq, hqs;
    DevActH xh, hh, hhs;  // matrix-core forms of x, h, shared h
    float *hf = nullptr, *hfs = nullptr, *y = nullptr, *ysh = nullptr, *xf = nullptr;
    size_t ystride = 0;  // floats per part of y (the K-split down GEMM's second part follows the first)
    int last_n = 0;
    Prof prof;
    hipStream_t own = nullptr;  // used when the caller passes the null stream
    // the shared expert runs on a second stream between a fork after routing and a join before the
    // routed down projection (it needs only the quantized x)
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    struct GraphKey {
        int n;
        const float* x;
        float* out;
        uint32_t flags;
        bool operator<(const GraphKey& o) const {
            if (n != o.n) return n < o.n;
            if (x != o.x) return x < o.x;
            if (out != o.out) return out < o.out;
            return flags < o.flags;
        }
    };
    struct Graph {
        hipGraphExec_t exec;
        uint64_t last;  // graph_clock at the last replay
    };
    static constexpr int GRAPH_MAX_N = 64;      // token counts replayed from graphs
    static constexpr size_t GRAPH_CACHE = 64;   // graphs kept (least recently used evicted)
    std::map<GraphKey, Graph> graphs;
    uint64_t graph_clock = 0;
    bool use_graphs = true;
    bool fold_combine = true;  // JX_NO_FOLD=1 keeps the separate combine launch (A/B measurement)
    bool chain8 = false;       // F16 / BF16 router: the 8-lane dot order
    // one-token steps in one launch (k_decode1): its device state, zeroed at creation, and the number
    // of such launches so far (JX_NO_FUSED=1 keeps the separate launches: A/B measurement)
    jx::DecodeSync* dsync = nullptr;
    uint64_t* hw = nullptr;  // k_decode_p's h: [k][d_ff / 4] words of (launch number << 32 | four quants)
    uint64_t* hfw = nullptr;  // k_decode1's fp32 h (fp32-activation downs): [k][d_ff] tagged words
    // pinned host word the fused launches set when a bounded wait between their blocks gives up (their
    // outputs are then invalid); read on the synchronous path, by jx_moe_layer_status and at the entry
    // of every forward, so asynchronous callers learn of it too
    uint32_t* herr = nullptr;
    uint32_t* herr_dev = nullptr;
    uint32_t spin_limit = 1u << 18;  // polls (each a device-coherent round trip) before a wait gives up
    hipStream_t last_st = nullptr;   // stream of the last forward (jx_moe_layer_status waits on it)
    uint32_t dec_epoch = 0;
    int shparts_cap = 1;  // K parts of the shared down's output the workspace holds (ysh)
    int cold_pairs = 0;   // experts under this many pairs take the GEMVs in the matrix-core regime (0: none)
    bool sh_ksplit = true;  // JX_SH_KSPLIT=0: the standalone shared down in one part (A/B measurement)
    bool fused_decode = true;
    bool force_fused = false;  // JX_FUSED=1: also where the separate launches measured faster
    int smfma_min = 0;         // shared expert's GEMM threshold (JX_SMFMA_MIN overrides it: A/B)
    bool dec_used = false;     // the last forward took the fused launch
    bool decp_used = false;    // ... in its one-block-per-CU form (k_decode_p)
    int decp_mode = -1;        // JX_DECP=0 / 1: never / always that form where it fits (A/B measurement)
};

struct jx_qmatrix {
    int device = 0;
    int type = 0, rows = 0, cols = 0;
    DevMat w;
    // workspace of the device-pointer drop-ins, allocated with the matrix: the Q8_0 form of
    // one activation row of `cols`, and its fp32 copy zero-padded to whole super-blocks
    jx::ActQ8 xq;
    float* xf = nullptr;
};

namespace {

// K of a down projection's matrix-core activation form: d_ff, or for fp32 h of a K-quant d_ff padded to
// whole super-blocks (the fp32 rows are stored padded that far).
int down_h_k(int type, int f, bool f32) { return f32 && jx::is_kquant(type) ? (f + 255) / 256 * 256 : f; }

int ensure_workspace(jx_moe_layer* L, int n) {
    if (n <= L->cap) return JX_OK;
    // captured graphs hold the old buffer addresses
    for (auto& kv : L->graphs) (void)hipGraphExecDestroy(kv.second.exec);
    L->graphs.clear();
    const int cap = std::max(n, L->cap * 2);
    const size_t nk = (size_t)cap * L->k;
    int r;
#define WS(ptr, count)                                 \
    if ((r = dalloc(ptr, (size_t)(count))) != JX_OK) { \
        L->cap = 0;                                    \
        return r;                                      \
    }
    WS(L->x, (size_t)cap * L->d);
    WS(L->xn, (size_t)cap * L->d);
    WS(L->out, (size_t)cap * L->d);
    WS(L->probs, nk);
    WS(L->ids, nk);
    WS(L->shscale, cap);
    WS(L->logits, (size_t)cap * L->E);
    WS(L->counts, L->E);
    WS(L->offs, L->E + 1);
    WS(L->act, L->E);
    WS(L->n_act, 1);
    WS(L->pair_tok, nk);
    WS(L->pos_of, nk);
    WS(L->n_tiles, 1);
    WS(L->tiles, nk / jx::MFMA_BN + std::min<size_t>(L->E, nk) + 1);
    WS(L->slots, L->E);
    // h's matrix-core form: K = d_ff, or for fp32 h of a K-quant d_ff padded to whole super-blocks
    const int hK = down_h_k(L->down.m.type, L->F, L->down_f32);
    const int hKs = L->shared ? down_h_k(L->sdown.m.type, L->Fs, L->sdown_f32) : 0;
    // x's forms for the gate/up GEMMs: block-unit for Q4_K / Q5_K, hi/lo for Q4_0 / Q8_0 (routed and shared)
    auto unit_t = [](int t) { return t == jx::T_Q4_K || t == jx::T_Q5_K; };
    auto hilo_t = [](int t) { return t == jx::T_Q4_0 || t == jx::T_Q8_0; };
    const bool xunit = unit_t(L->gate.m.type) || (L->shared && unit_t(L->sgate.m.type));
    const bool xhilo = hilo_t(L->gate.m.type) || (L->shared && hilo_t(L->sgate.m.type));
    if ((r = L->xh.alloc((size_t)cap, L->d, xhilo, xunit)) != JX_OK || (r = L->hh.alloc(nk, hK)) != JX_OK) {
        L->cap = 0;
        return r;
    }
    if (L->shared && (r = L->hhs.alloc((size_t)cap, hKs)) != JX_OK) {
        L->cap = 0;
        return r;
    }
    WS(L->xq.q, (size_t)cap * L->d);
    WS(L->xq.s, (size_t)cap * L->d / 32);
    L->xq.K = L->d;
    WS(L->hq.q, nk * L->F);
    WS(L->hq.s, nk * L->F / 32);
    // the fused one-token step polls the low bits of h's scale words for its launch's tag: start untagged
    HIPCHK(hipMemset(L->hq.s, 0, nk * L->F / 32 * sizeof(float2)));
    L->hq.K = L->F;
    // y: the routed down output per pair; a K-split down GEMM writes its second part ystride floats on
    L->ystride = nk * L->d;
    WS(L->y, (size_t)jx::mfma_down_ksplit(hK) * nk * L->d);
    if (L->gu_f32 || L->sgu_f32) {
        WS(L->xf, (size_t)cap * L->dpad);
        HIPCHK(hipMemset(L->xf, 0, (size_t)cap * L->dpad * sizeof(float)));
    }
    const size_t fpad = ((size_t)L->F + 255) / 256 * 256;
    if (L->down_f32) {
        WS(L->hf, nk * fpad);
        HIPCHK(hipMemset(L->hf, 0, nk * fpad * sizeof(float)));
    }
    if (L->shared) {
        WS(L->hqs.q, (size_t)cap * L->Fs);
        WS(L->hqs.s, (size_t)cap * L->Fs / 32);
        // the fused step's shared down tiles poll these scale words for the launch's tag, as for hq.s
        HIPCHK(hipMemset(L->hqs.s, 0, (size_t)cap * L->Fs / 32 * sizeof(float2)));
        L->hqs.K = L->Fs;
        // the shared down's output, in K parts where its blocks join the routed down launch
        L->shparts_cap = L->sdown.m.type == L->down.m.type ? jx::shared_down_kparts(L->down.m.type, L->F, L->Fs) : 1;
        WS(L->ysh, (size_t)L->shparts_cap * cap * L->d);
        const size_t fspad = ((size_t)L->Fs + 255) / 256 * 256;
        if (L->sdown_f32) {
            WS(L->hfs, (size_t)cap * fspad);
            HIPCHK(hipMemset(L->hfs, 0, (size_t)cap * fspad * sizeof(float)));
        }
    }
#undef WS
    L->cap = cap;
    return JX_OK;
}

void free_layer(jx_moe_layer* L) {
    (void)hipSetDevice(L->device);
    if (L->own) {  // its stream goes away: no later launch may compare against it
        std::lock_guard<std::mutex> lk(g_fused_order.mu);
        if (g_fused_order.pending[L->device] == L->own) {
            (void)hipStreamSynchronize(L->own);
            g_fused_order.pending[L->device] = nullptr;
        }
    }
    for (auto* m : {&L->gate, &L->up, &L->down, &L->sgate, &L->sup, &L->sdown}) m->release();
    void* ptrs[] = {L->router, L->router_cm, L->bias, L->shgate, L->ffn_norm, L->post_norm, L->xn, L->x, L->out, L->probs, L->shscale, L->logits, L->ids,
                    L->counts, L->offs, L->act, L->n_act, L->pair_tok, L->pos_of, L->n_tiles, L->tiles,
                    L->slots, L->xq.q, L->xq.s, L->hq.q, L->hq.s, L->hqs.q, L->hqs.s, L->hf, L->hfs, L->y, L->ysh,
                    L->xf, L->dsync, L->hw, L->hfw};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    if (L->herr) (void)hipHostFree(L->herr);
    L->xh.release();
    L->hh.release();
    L->hhs.release();
    for (auto ev : L->prof.pool) (void)hipEventDestroy(ev);
    for (auto& kv : L->graphs) (void)hipGraphExecDestroy(kv.second.exec);
    if (L->own) (void)hipStreamDestroy(L->own);
    if (L->side) (void)hipStreamDestroy(L->side);
    if (L->ev_fork) (void)hipEventDestroy(L->ev_fork);
    if (L->ev_join) (void)hipEventDestroy(L->ev_join);
    delete L;
}

// Profiling: bracket a launch with two pooled events on the forward's stream.
struct Launch {
    jx_moe_layer* L;
    const char* name;
    hipStream_t st;
    size_t idx = (size_t)-1;
    Launch(jx_moe_layer* L_, const char* n, hipStream_t s) : L(L_), name(n), st(s) {
        if (!L->prof.on) return;
        Prof& P = L->prof;
        while (P.pool.size() < P.used + 2) {
            hipEvent_t ev;
            if (hipEventCreate(&ev) != hipSuccess) return;
            P.pool.push_back(ev);
        }
        idx = P.used;
        P.used += 2;
        (void)hipEventRecord(P.pool[idx], st);
    }
    ~Launch() {
        if (idx == (size_t)-1) return;
        (void)hipEventRecord(L->prof.pool[idx + 1], st);
        L->prof.pending.emplace_back(name, idx);
    }
};

int resolve_profile(jx_moe_layer* L) {
    Prof& P = L->prof;
    for (auto& pe : P.pending) {
        HIPCHK(hipEventSynchronize(P.pool[pe.second + 1]));
        float ms = 0.0f;
        HIPCHK(hipEventElapsedTime(&ms, P.pool[pe.second], P.pool[pe.second + 1]));
        auto& a = P.acc[pe.first];
        a.first += ms;
        a.second += 1;
    }
    P.pending.clear();
    P.used = 0;
    return JX_OK;
}

// Regime: the matrix-core GEMMs once the average expert sees this many (token, slot) pairs.  The
// multi-token GEMV (int8 matrix cores, 16 tokens per weight pass) streams an expert's weights once
// per 16 tokens, the GEMM once per 64-pair tile computing the whole tile.  Forced-GEMV vs forced-GEMM
// sweeps on MI355X put the crossover at 3-4 pairs for the Q8_0 layer (Qwen3-shaped), ~11 for the
// small 4-bit experts (DeepSeek-V2-Lite-, Qwen1.5-shaped) and ~15 for large ones (Mixtral-shaped,
// 14336 x 4096 per matrix, whose GEMV streams near its best rate).
constexpr int MFMA_MIN_PAIRS_PER_EXPERT_Q4 = 12;
constexpr int MFMA_MIN_PAIRS_PER_EXPERT_Q4_LARGE = 16;
constexpr int MFMA_MIN_PAIRS_PER_EXPERT_Q8 = 4;
constexpr size_t LARGE_EXPERT_ELEMS = (size_t)1 << 25;  // d * d_ff per matrix
// The cold experts' GEMVs beside the GEMMs: layers of at least HYBRID_MIN_E experts, experts under
// COLD_PAIRS pairs (JX_COLD_PAIRS overrides it, 0 turns the split off: A/B measurement).  Measured on
// the Qwen3-shaped 2048-token step with Zipf routing (61 / 76 / 86 / 93 experts under 16 / 32 / 48 / 64
// pairs): 624 us without the split, 600 / 609 / 621 / 637 us with these thresholds.  The GEMMs are
// matrix-core bound on the head experts (the largest holds 1902 pairs), and the GEMV blocks share the
// CUs with them.
constexpr int HYBRID_MIN_E = 32;
constexpr int COLD_PAIRS = 16;

// Whether a call takes the fused one-token launch (k_decode1), apart from stream capture: one token in
// the GEMV regime, Q8_0 activations on both sides, a shared expert (if any) in the routed formats, a
// shape the kernel is built for, and one where it measured faster (or JX_FUSED=1).
// The one-block-per-CU form of the fused step (k_decode_p): top-2 with the folded combine, no shared
// expert, a shape it is built for, and gate/up tiles too many for k_decode1's one block per CU
// (decode1_pays false; measured Mixtral-shaped: 42.2 us per step against 46.3 us for the separate
// launches), unless JX_DECP says otherwise.
static bool decodep_ok(const jx_moe_layer* L, uint32_t flags) {
    if (L->decp_mode == 0 || L->shared || L->k != 2 || (flags & JX_FWD_RESIDUAL) || !L->fold_combine || L->down_f32)
        return false;  // (k_decode_p hands h over in its Q8_0 form only)
    if (!jx::decodep_fits(L->gate.m.type, L->down.m.type, L->d, L->F, L->E, L->k, false, true, L->gate.m.nrt,
                          L->down.m.nrt))
        return false;
    return L->decp_mode == 1 || !jx::decode1_pays(L->gate.m.nrt, L->k, 0);
}

bool decode1_wanted(const jx_moe_layer* L, int n, uint32_t flags) {
    if (n != 1 || !L->fused_decode || (flags & (JX_FWD_UNFUSED | JX_FWD_FORCE_MFMA))) return false;
    if (L->gu_f32 || L->up.m.type != L->gate.m.type || (L->down_f32 && !L->hfw)) return false;
    if (L->shared && (L->sgu_f32 || L->sdown_f32 || L->sgate.m.type != L->gate.m.type ||
                      L->sup.m.type != L->gate.m.type))
        return false;
    if (L->E > jx::SMALL_GROUP_MAX_E || !jx::route_small_fits(1, L->d, L->E)) return false;
    if (!jx::decode1_fits(L->gate.m.type, L->down.m.type, L->d, L->F, L->E, L->k, L->shared ? L->Fs : 0,
                          L->shgate != nullptr, L->shared ? L->sdown.m.type : L->down.m.type, L->down_f32))
        return false;
    if (decodep_ok(L, flags)) return true;
    return L->force_fused || jx::decode1_pays(L->gate.m.nrt, L->k, L->shared ? L->sgate.m.nrt : 0);
}

int run_forward(jx_moe_layer* L, const float* xdev, int n, float* outdev, hipStream_t st, uint32_t flags) {
    const int E = L->E, k = L->k, d = L->d;
    // the residual-stream form: x_norm = rms_norm(x, ffn_norm) feeds the router; x is added back in the combine
    const bool resid = flags & JX_FWD_RESIDUAL;
    const float* xres = xdev;
    if (resid) {
        Launch l(L, "rms_norm", st);
        jx::launch_rms_norm(xdev, L->ffn_norm, n, d, L->eps, L->xn, st);
        xdev = L->xn;
    }
    const int nk = n * k;
    const int min_ppe = L->gate.m.type == jx::T_Q8_0                 ? MFMA_MIN_PAIRS_PER_EXPERT_Q8
                        : (size_t)d * L->F >= LARGE_EXPERT_ELEMS ? MFMA_MIN_PAIRS_PER_EXPERT_Q4_LARGE
                                                                 : MFMA_MIN_PAIRS_PER_EXPERT_Q4;
    bool mfma = (size_t)nk >= (size_t)min_ppe * E;
    if (flags & JX_FWD_FORCE_GEMV) mfma = false;
    if (flags & JX_FWD_FORCE_MFMA) mfma = true;
    // The matrix-core GEMMs stage K in 128-element half-units; their Q4_K / Q5_K matrices carry the min
    // table.  Gate/up takes the GEMM only with a Q8_0 form of x and a type whose products stay exact
    // there (gemm_gateup_ok); otherwise it runs on the GEMVs (the multi-token form at prefill sizes)
    // and the down projection still decides for itself.
    auto ready = [](const DevMat& M) {
        return !(M.m.type == jx::T_Q4_K || M.m.type == jx::T_Q5_K) || M.m.mn != nullptr;
    };
    auto gu_gemm = [&](const DevMat& G, const DevMat& U, bool f32) {
        return !f32 && jx::gemm_gateup_ok(G.m.type) && d % 128 == 0 && ready(G) && ready(U);
    };
    auto dn_gemm = [&](const DevMat& D, int f, bool f32) { return down_h_k(D.m.type, f, f32) % 128 == 0 && ready(D); };
    const bool mfma_gu = mfma && gu_gemm(L->gate, L->up, L->gu_f32);
    const bool dn_shape = dn_gemm(L->down, L->F, L->down_f32);
    const bool smfma = L->shared && n >= L->smfma_min && !(flags & JX_FWD_FORCE_GEMV);
    const bool smfma_gu = smfma && gu_gemm(L->sgate, L->sup, L->sgu_f32);
    const bool smfma_dn = smfma && dn_gemm(L->sdown, L->Fs, L->sdown_f32);
    mfma = mfma && (mfma_gu || dn_shape);
    jx::RouteArgs ra{xdev, n, d, E, k, L->router, L->bias, L->shgate, L->xq,
                     (mfma_gu || smfma_gu) ? L->xh.a : jx::ActH{}, L->ids, L->probs, L->shscale, L->logits,
                     L->router_cm};
    ra.chain8 = L->chain8 ? 1 : 0;
    const jx::DispatchOut dout{L->counts, L->offs,   L->act,   L->n_act, L->pair_tok,
                               L->pos_of,  L->tiles, L->n_tiles, L->slots};
    // few-token decode: logits on one block per router row, grouping in the GEMVs
    const bool small_logits = !mfma && !smfma && n <= jx::ROUTE_SMALL_MAX_N && E <= jx::SMALL_GROUP_MAX_E &&
                              jx::route_small_fits(n, d, E);
    // GEMV form: one token; groups of 4 on the VALU (few tokens per expert); or 16 per weight pass on
    // the int8 matrix cores, which streams faster once experts see one token on average (Mixtral-sized
    // experts: 1.5; Q8_0, whose VALU form is slower: 0.5): measured on every configured shape
    // (Qwen1.5-shaped 16 / 32 tokens 127 / 164 -> 112 / 131 us, DeepSeek-V2-Lite-shaped 12 / 16 tokens
    // 127 / 137 -> 117 / 116 us against the VALU form; Mixtral-shaped 4 tokens 144 us VALU, 154 us MFMA)
    const bool q8w = L->gate.m.type == jx::T_Q8_0;
    const bool large = (size_t)d * L->F >= LARGE_EXPERT_ELEMS;
    auto gemv_tb = [&](int tokens_per_expert_x2) {  // twice the average tokens per expert
        return n == 1 ? 1 : (tokens_per_expert_x2 >= (q8w ? 1 : large ? 3 : 2) ? 16 : 4);
    };
    const int tb = gemv_tb(2 * nk / E);
    // fp32 h (no Q8_0 form at d_ff) takes the matrix-core down GEMM from 2 tokens on (every dispatch path
    // writes the MFMA tiles, the few-token one from the gate/up GEMV's tail block): the fp32 GEMV's
    // multi-token form re-streams the weights per group of 4 tokens in fp32
    const bool mfma_down = (mfma || (L->down_f32 && n >= 2)) && dn_shape;
    // The weighted combine folds into the down GEMV when the few-token routers run and every output
    // element receives at most two contributions (top_k <= 2, no shared expert; CombineOut).
    const bool fold = jx::route_small_fits(n, d, E) && k <= 2 && !L->shared && !mfma_down && tb <= 4 &&
                      !resid && L->fold_combine;
    if (fold) {
        ra.zero_out = outdev;
        ra.zero_count = n * d;
    }
    // one token, no shared expert: router, gate/up and down (and the folded combine) in one launch
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIPCHK(hipStreamIsCapturing(st, &cap));
    L->dec_used = small_logits && tb == 1 && cap == hipStreamCaptureStatusNone && decode1_wanted(L, n, flags);
    if (L->dec_used) {
        if (++L->dec_epoch == 0) {  // 2^32 launches: start the counts over
            HIPCHK(hipMemsetAsync(L->dsync, 0, sizeof(jx::DecodeSync), st));
            HIPCHK(hipMemsetAsync(L->hw, 0, (size_t)L->k * L->F / 4 * sizeof(uint64_t), st));
            if (L->hfw) HIPCHK(hipMemsetAsync(L->hfw, 0, (size_t)L->k * L->F * sizeof(uint64_t), st));
            L->dec_epoch = 1;
        }
        jx::Decode1Args a;
        a.G = L->gate.m;
        a.U = L->up.m;
        a.D = L->down.m;
        a.x = xdev;
        a.router = L->router;
        a.bias = L->bias;
        a.d = d;
        a.E = E;
        a.k = k;
        a.chain8 = L->chain8 ? 1 : 0;
        a.xq = L->xq;
        a.hq = L->hq;
        a.ra = ra;
        a.ra.zero_out = nullptr;
        a.ra.zero_count = 0;
        a.o = dout;
        a.out = fold ? outdev : nullptr;
        a.y = L->y;
        a.sync = L->dsync;
        a.epoch = L->dec_epoch;
        a.htag = 1u + L->dec_epoch % 8191u;  // never 0, the low bits of every untagged scale
        a.herr = L->herr_dev;
        a.hfw = L->hfw;
        a.hf_ld = (int)(((size_t)L->F + 255) / 256 * 256);
        a.giveup_test = (flags & JX_FWD_TEST_GIVEUP) ? 1u : 0u;
        a.spin_limit = a.giveup_test ? 64u : L->spin_limit;
        if (L->shared) {
            a.sh = 1;
            a.SG = L->sgate.m;
            a.SU = L->sup.m;
            a.SD = L->sdown.m;
            a.shgate = L->shgate;
            a.hqs = L->hqs;
            a.ysh = L->ysh;
        }
        L->decp_used = fold && decodep_ok(L, flags);
        if (L->decp_used) {
            a.hw = L->hw;
            {
                std::lock_guard<std::mutex> lk(g_fused_order.mu);
                hipStream_t& pending = g_fused_order.pending[L->device];
                if (pending && pending != st) HIPCHK(hipDeviceSynchronize());  // it may still be running
                pending = st;
            }
            Launch l(L, "decode_fused_cu", st);
            if (jx::launch_decode_p(a, L->gate.m.type, L->down.m.type, st) != 0)
                return fail(JX_ERR_HIP, "fused one-token step: launch failed");
        } else {
            Launch l(L, fold ? "decode_fused" : "decode_fused_y", st);
            jx::launch_decode1(a, L->gate.m.type, L->down.m.type, st, L->shared ? L->sdown.m.type : L->down.m.type,
                               L->down_f32);
        }
        if (!fold) {
            Launch l(L, "combine", st);
            jx::launch_combine(n, d, k, L->probs, L->pos_of, L->y, L->shared ? L->ysh : nullptr, L->shscale, outdev,
                               st, resid ? xres : nullptr, resid ? L->post_norm : nullptr, L->eps);
        }
        HIPCHK(hipGetLastError());
        return JX_OK;
    }
    if (small_logits) {
        Launch l(L, "route", st);
        jx::launch_route_logits(ra, st);
    } else if (jx::route_small_fits(n, d, E)) {
        {
            Launch l(L, "route_dispatch", st);
            jx::launch_route_small(ra, dout, st);
        }
        if (mfma_gu || smfma_gu) {
            Launch l(L, "to_matrix_form", st);
            jx::launch_q8_to_acth(L->xq, n, L->xh.a, st);
        }
    } else {
        Launch l(L, "route", st);
        jx::launch_route(ra, st);
    }
    // the dispatch tables (many-token path) follow the shared expert's fork: it needs only x's forms
    const bool dispatch_later = !small_logits && !jx::route_small_fits(n, d, E);
    jx::Groups grp;
    grp.counts = L->counts;
    grp.offs = L->offs;
    grp.act = L->act;
    grp.n_act = L->n_act;
    grp.slots = L->slots;
    grp.pair_tok = L->pair_tok;
    grp.tiles = L->tiles;
    grp.n_tiles = L->n_tiles;
    grp.top_k = k;
    grp.n_tok = n;
    const int slots = std::min(E, nk);
    const int tbs = n == 1 ? 1 : (n >= 3 ? 16 : 4);  // the shared expert sees every token
    const int tiles_ub = nk / jx::MFMA_BN + slots;
    const size_t fpad = ((size_t)L->F + 255) / 256 * 256;
    if (L->gu_f32 || L->sgu_f32) {  // fp32 x zero-padded for the fp32-activation gate/up
        Launch l(L, "x_pad", st);
        jx::launch_copy_pad(xdev, d, L->dpad, L->xf, st, n);
    }
    jx::Groups sg;  // the shared expert's groups: every token
    sg.identity = 1;
    sg.n_tok = n;
    sg.top_k = 1;
    // the GEMVs' 16-token form: one group per 16 tokens, so the dense expert's row tiles spread
    // over n / 16 times as many blocks as one group of all tokens (which each block streams pass
    // by pass)
    const int sslots = tbs == 16 ? (n + 15) / 16 : 1;
    if (tbs == 16) sg.chunk = 16;
    const size_t fspad = ((size_t)L->Fs + 255) / 256 * 256;
    const int st_ub = (n + jx::MFMA_BN - 1) / jx::MFMA_BN;
    // The shared expert's GEMV blocks join the routed multi-tile launches where both take that form in one
    // weight format and the gate/up blocks stay in one resident round (the down also needs Q8_0 h on both
    // sides): its few long-lived blocks then run among the routed ones instead of from a second stream
    // beside them, which costs far more than its bytes (measured without the shared expert:
    // Qwen1.5-shaped 64 tokens 148 -> 113 us per step, DeepSeek-V2-Lite-shaped 32 tokens 134 -> 111 us,
    // for ~20 and ~10 MB of its weights; joined: Qwen1.5-shaped 16 / 32 tokens 111.5 / 123.6 ->
    // 108.5 / 117.9 us).
    // Only both launches together: with the down left on the side stream the joined gate/up measured
    // slower (DeepSeek-V2-Lite-shaped, fp32 h: 16 / 32 tokens 112.4 / 130.1 -> 123.0 / 140.3 us).
    const bool sh_dn = L->shared && !smfma && tbs == 16 && tb == 16 && !mfma_down && !L->down_f32 && !L->sdown_f32 &&
                       L->sdown.m.type == L->down.m.type && L->shparts_cap > 1 &&
                       jx::gemv_mxt_takes(L->down.m.type, false, L->down.m.nrt, slots, tb);
    const bool sh_gu = sh_dn && !mfma_gu && !L->gu_f32 && !L->sgu_f32 && L->sgate.m.type == L->gate.m.type &&
                       L->sup.m.type == L->up.m.type &&
                       jx::gemv_gateup_joins(L->gate.m.type, L->gate.m.nrt, slots, tb, L->sgate.m.nrt, sslots);
    int shparts = 1;  // K parts of the shared down's output (the combine adds them)
    // A standalone shared down of at least 4 routed K's (Qwen1.5-shaped: 5632 against 1408) in K parts;
    // measured per step, weights from HBM: 48 / 64 tokens 133.6 / 138.8 -> 127.2 / 137.3 us.  Two parts
    // (DeepSeek-V2-Lite-shaped 2816 against 1408) measured slower: 32 tokens 132.5 -> 135.7 us.
    const bool sh_ksplit = L->shared && !smfma_dn && tbs == 16 && !L->sdown_f32 && L->shparts_cap >= 4 && L->sh_ksplit;
    auto shared_gateup = [&](hipStream_t ss) {
        if (smfma_gu) {
            Launch l(L, "shared_gateup_mfma", ss);
            jx::launch_mfma_gateup(L->sgate.m, L->sup.m, L->xh.a, sg, st_ub, L->sdown_f32 ? jx::ActQ8{} : L->hqs,
                                   L->sdown_f32 ? L->hfs : nullptr, ss);
        } else {
            Launch l(L, "shared_gateup_gemv", ss);
            jx::launch_gemv_gateup(L->sgate.m, L->sup.m, L->xq, sg, sslots, tbs, L->hqs, L->sdown_f32 ? L->hfs : nullptr, ss,
                                   nullptr, L->sgu_f32 ? L->xf : nullptr, L->dpad);
        }
    };
    auto shared_down = [&](hipStream_t ss) {
        if (smfma_dn) {
            Launch l(L, "shared_down", ss);
            if (L->sdown_f32)
                jx::launch_f32_to_acth(L->hfs, (int)fspad, n, L->hhs.a, ss);
            else
                jx::launch_q8_to_acth(L->hqs, n, L->hhs.a, ss, false);
            jx::launch_mfma_down(L->sdown.m, L->hhs.a, sg, st_ub, L->ysh, ss);
        } else if (sh_ksplit) {
            // the dense shared down's long K in parts, each block a routed block's share of units (the
            // combine adds the parts), so it is done before the routed gate/up that the routed down
            // waits on with it
            jx::SharedPart sp;
            sp.g = L->sdown.m;
            sp.grp = sg;
            sp.slots = sslots;
            sp.hq = L->hqs;
            sp.y = L->ysh;
            sp.kparts = L->shparts_cap;
            Launch l(L, "shared_down_kparts", ss);
            if (jx::launch_gemv_down(L->sdown.m, L->hqs, nullptr, 0, sg, 0, tbs, L->ysh, ss, jx::CombineOut{}, &sp))
                shparts = sp.kparts;
            else
                jx::launch_gemv_down(L->sdown.m, L->hqs, nullptr, 0, sg, sslots, tbs, L->ysh, ss);
        } else {
            Launch l(L, "shared_down", ss);
            jx::launch_gemv_down(L->sdown.m, L->hqs, L->sdown_f32 ? L->hfs : nullptr, (int)fspad, sg, sslots, tbs, L->ysh,
                                 ss);
        }
    };
    // otherwise the shared expert runs on the side stream, concurrent with the routed gate/up
    if (L->shared && !sh_gu) {
        HIPCHK(hipEventRecord(L->ev_fork, st));
        HIPCHK(hipStreamWaitEvent(L->side, L->ev_fork, 0));
        shared_gateup(L->side);
        shared_down(L->side);
        HIPCHK(hipEventRecord(L->ev_join, L->side));
    }
    // Skewed routing over many experts in the matrix-core regime: the experts with fewer than COLD_PAIRS
    // pairs take the multi-token GEMVs (weights streamed once per 16 tokens) on the side stream, beside
    // the GEMMs over the others, instead of a mostly empty GEMM tile each.  The dispatch keeps them out of
    // the tile table; the GEMV blocks of the others exit at once.
    const bool hybrid = mfma && mfma_gu && mfma_down && !L->shared && dispatch_later && E >= HYBRID_MIN_E &&
                        !L->gu_f32 && !L->down_f32 && !(flags & JX_FWD_FORCE_MFMA) &&
                        jx::mfma_down_ksplit(L->hh.a.K) == 1 && L->cold_pairs > 0;
    if (dispatch_later) {
        Launch l(L, "dispatch", st);
        jx::launch_dispatch(L->ids, nk, E, k, dout, st, hybrid ? L->cold_pairs : 0);
    }
    if (hybrid) {
        HIPCHK(hipEventRecord(L->ev_fork, st));
        HIPCHK(hipStreamWaitEvent(L->side, L->ev_fork, 0));
        jx::Groups cg = grp;
        cg.cold_max = L->cold_pairs;
        {
            Launch l(L, "gateup_gemv_cold", L->side);
            jx::launch_gemv_gateup(L->gate.m, L->up.m, L->xq, cg, slots, 16, L->hq, nullptr, L->side);
        }
        {
            Launch l(L, "down_gemv_cold", L->side);
            jx::launch_gemv_down(L->down.m, L->hq, nullptr, 0, cg, slots, 16, L->y, L->side);
        }
        HIPCHK(hipEventRecord(L->ev_join, L->side));
    }
    const float* gxf = L->gu_f32 ? L->xf : nullptr;
    if (mfma_gu) {
        Launch l(L, "gateup_mfma", st);
        jx::launch_mfma_gateup(L->gate.m, L->up.m, L->xh.a, grp, tiles_ub, L->down_f32 ? jx::ActQ8{} : L->hq,
                               L->down_f32 ? L->hf : nullptr, st);
    } else if (small_logits) {
        jx::Groups lg = grp;
        lg.logits = L->logits;
        lg.n_experts = E;
        jx::SmallTail tail;
        tail.a = ra;
        tail.o = dout;
        tail.on = 1;
        Launch l(L, "gateup_gemv", st);
        jx::launch_gemv_gateup(L->gate.m, L->up.m, L->xq, lg, slots, tb, L->hq, L->down_f32 ? L->hf : nullptr, st,
                               &tail, gxf, L->dpad);
    } else {
        jx::SharedPart spg;
        if (sh_gu) {
            spg.g = L->sgate.m;
            spg.u = L->sup.m;
            spg.grp = sg;
            spg.slots = sslots;
            spg.hq = L->hqs;
            spg.hf = L->sdown_f32 ? L->hfs : nullptr;
            spg.hf_ld = (int)fspad;
        }
        bool joined = false;
        {
            Launch l(L, sh_gu ? "gateup_gemv_shared" : "gateup_gemv", st);
            joined = jx::launch_gemv_gateup(L->gate.m, L->up.m, L->xq, grp, slots, tb, L->hq,
                                            L->down_f32 ? L->hf : nullptr, st, nullptr, gxf, L->dpad,
                                            sh_gu ? &spg : nullptr);
        }
        if (sh_gu && !joined) shared_gateup(st);  // (the launch took another form)
    }
    if (L->shared && !sh_gu) HIPCHK(hipStreamWaitEvent(st, L->ev_join, 0));

    int ks = 1;  // parts of the down GEMM's K (the combine adds them)
    if (mfma_down) {
        {
            Launch l(L, "h_to_matrix_form", st);
            if (L->down_f32)
                jx::launch_f32_to_acth(L->hf, (int)fpad, nk, L->hh.a, st);
            else
                jx::launch_q8_to_acth(L->hq, nk, L->hh.a, st, false);
        }
        // fp32 h at a few tokens per expert: the multi-token down on the fp16 matrix cores where built
        if (!mfma && L->down_f32 && jx::gemv_down_f16_fits(L->down.m.type, L->hh.a.K)) {
            Launch l(L, "down_gemv_f16", st);
            jx::launch_gemv_down_f16(L->down.m, L->hh.a, grp, slots, L->y, st);
        } else {
            Launch l(L, "down_mfma", st);
            ks = jx::mfma_down_ksplit(L->hh.a.K);
            jx::launch_mfma_down(L->down.m, L->hh.a, grp, tiles_ub, L->y, st, ks, L->ystride,
                                 nk <= jx::MFMA_DOWN_SMALL_MAX_PPE * E);
        }
    } else {
        jx::CombineOut comb;
        if (fold) {
            comb.out = outdev;
            comb.probs = L->probs;
            comb.ids = L->ids;
            comb.k = k;
        }
        jx::SharedPart spd;
        if (sh_gu) {
            spd.g = L->sdown.m;
            spd.grp = sg;
            spd.slots = sslots;
            spd.hq = L->hqs;
            spd.y = L->ysh;
            spd.kparts = std::min(L->shparts_cap, jx::shared_down_kparts(L->down.m.type, L->F, L->Fs));
        }
        bool joined = false;
        {
            Launch l(L, fold ? "down_gemv_combine" : (L->down_f32 ? "down_gemv_f32" : sh_gu ? "down_gemv_shared" : "down_gemv"),
                     st);
            joined = jx::launch_gemv_down(L->down.m, L->hq, L->down_f32 ? L->hf : nullptr, (int)fpad, grp, slots, tb, L->y,
                                          st, comb, sh_gu ? &spd : nullptr);
        }
        if (sh_gu && !joined) shared_down(st);  // (the launch took another form)
        if (joined) shparts = spd.kparts;
    }
    if (hybrid) HIPCHK(hipStreamWaitEvent(st, L->ev_join, 0));
    if (!fold) {
        Launch l(L, "combine", st);
        jx::launch_combine(n, d, k, L->probs, L->pos_of, L->y, L->shared ? L->ysh : nullptr, L->shscale, outdev, st,
                           resid ? xres : nullptr, resid ? L->post_norm : nullptr, L->eps,
                           ks > 1 ? L->y + L->ystride : nullptr, shparts);
    }
    HIPCHK(hipGetLastError());
    return JX_OK;
}

// The fp16 bits of a value that is an fp16 widened to fp32 (exact narrowing).
uint16_t narrow_f16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int e = (int)((u >> 23) & 0xFF) - 112;
    const uint32_t m = u & 0x7FFFFFu;
    if (e <= 0) return (e < -10) ? (uint16_t)sign : (uint16_t)(sign | ((m | 0x800000u) >> (uint32_t)(14 - e)));
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | (m >> 13));
}

// Q8_0 blocks (fp16 d, 32 int8) from a device ActQ8 of `rows` rows.
int download_q8_blocks(const jx::ActQ8& a, int rows, uint8_t* out) {
    const size_t k = (size_t)a.K, nb = (size_t)rows * (k / 32);
    std::vector<int8_t> q((size_t)rows * k);
    std::vector<float2> sc(nb);
    HIPCHK(hipMemcpy(q.data(), a.q, q.size(), hipMemcpyDeviceToHost));
    HIPCHK(hipMemcpy(sc.data(), a.s, nb * sizeof(float2), hipMemcpyDeviceToHost));
    for (size_t b = 0; b < nb; ++b) {
        const uint16_t h = narrow_f16(sc[b].x);
        std::memcpy(out + b * 34, &h, 2);
        std::memcpy(out + b * 34 + 2, q.data() + b * 32, 32);
    }
    return JX_OK;
}

// Scratch for the drop-ins (allocated per call; these are function-level
// entry points for parity checks and single-matrix callers, not the layer path).
struct Scratch {
    std::vector<void*> ptrs;
    ~Scratch() {
        for (void* p : ptrs) (void)hipFree(p);
    }
    template <typename T>
    T* get(size_t n) {
        void* p = nullptr;
        if (hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)) != hipSuccess) return nullptr;
        ptrs.push_back(p);
        return static_cast<T*>(p);
    }
};

}  // namespace

extern "C" {

const char* jx_moe_last_error(void) { return g_err.c_str(); }

int jx_moe_init(int32_t device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(JX_ERR_NODEVICE, "no HIP device");
    if (device < 0 || device >= n) return fail(JX_ERR_NODEVICE, "device index out of range");
    hipDeviceProp_t p;
    HIPCHK(hipGetDeviceProperties(&p, device));
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(JX_ERR_NODEVICE, std::string("device is ") + p.gcnArchName + ", this build targets gfx950");
    HIPCHK(hipSetDevice(device));
    if (device >= MAX_DEVICES) return fail(JX_ERR_NODEVICE, "device index beyond the library's table");
    if (!g_scratch[device].load()) {  // this device's copy of the static scratch, with the device current
        void* p = nullptr;
        HIPCHK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(JX_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
        g_scratch[device].store(p);
    }
    g_device = device;
    return JX_OK;
}

int jx_moe_layer_create(const jx_moe_layer_desc* D, jx_moe_layer** out) {
    if (!D || !out) return fail(JX_ERR_INVALID, "null argument");
    *out = nullptr;
    if (g_device < 0) return fail(JX_ERR_NODEVICE, "jx_moe_init has not been called");
    if (D->n_experts < 1 || D->n_experts > 512) return fail(JX_ERR_UNSUPPORTED, "n_experts must be 1..512");
    if (D->top_k < 1 || D->top_k > 32 || D->top_k > D->n_experts) return fail(JX_ERR_UNSUPPORTED, "top_k must be 1..min(32, E)");
    if (D->d_model < 32 || D->d_model % 32 != 0 || D->d_model > 8192)
        return fail(JX_ERR_UNSUPPORTED, "d_model must be a multiple of 32, at most 8192");
    if (D->d_ff < 32 || D->d_ff % 32 != 0) return fail(JX_ERR_UNSUPPORTED, "d_ff must be a multiple of 32");
    if (!D->router || !D->gate_exps || !D->up_exps || !D->down_exps) return fail(JX_ERR_INVALID, "missing tensor");
    if (D->router_type != JX_TYPE_F32 && D->router_type != JX_TYPE_F16 && D->router_type != JX_TYPE_BF16)
        return fail(JX_ERR_UNSUPPORTED, "router must be F32, F16 or BF16");
    if (D->activation != JX_ACT_SILU && D->activation != JX_ACT_GELU_TANH)
        return fail(JX_ERR_INVALID, "activation must be JX_ACT_SILU or JX_ACT_GELU_TANH");
    if (D->gate_type != D->up_type) return fail(JX_ERR_UNSUPPORTED, "gate and up must share a type");
    const bool has_sh = D->d_ff_shared > 0;
    for (int t : {D->gate_type, D->down_type, has_sh ? D->sh_gate_type : D->gate_type, has_sh ? D->sh_down_type : D->down_type})
        if (!expert_type_ok(t))
            return fail(JX_ERR_UNSUPPORTED, "expert weight type must be Q4_0, Q5_0, Q8_0, Q4_K, Q5_K or Q6_K");
    if (has_sh) {
        if (D->d_ff_shared % 32 != 0) return fail(JX_ERR_UNSUPPORTED, "d_ff_shared must be a multiple of 32");
        if (!D->sh_gate || !D->sh_up || !D->sh_down) return fail(JX_ERR_INVALID, "missing shared expert tensor");
        if (D->sh_gate_type != D->sh_up_type) return fail(JX_ERR_UNSUPPORTED, "shared gate and up must share a type");
    }
    {  // the GEMVs stage up to 4 token rows of activations in LDS: Q8_0 forms at K, fp32 rows padded
        // to whole super-blocks (K-quants) where the reference keeps fp32 activations
        auto act_k = [](int t, int f) { return q8_activation(t, f) || !jx::is_kquant(t) ? f : (f + 255) / 256 * 256; };
        auto fits = [&](bool gateup, int t, int f) {
            return act_k(t, f) <= jx::gemv_max_k(gateup, 4, !q8_activation(t, f));
        };
        if (!fits(true, D->gate_type, D->d_model) || !fits(false, D->down_type, D->d_ff) ||
            (has_sh && (!fits(true, D->sh_gate_type, D->d_model) || !fits(false, D->sh_down_type, D->d_ff_shared))))
            return fail(JX_ERR_UNSUPPORTED, "d_model / d_ff exceed the GEMVs' staged activation capacity");
    }
    auto* L = new jx_moe_layer();
    L->device = g_device;
    L->E = D->n_experts;
    L->k = D->top_k;
    L->d = D->d_model;
    L->F = D->d_ff;
    L->Fs = D->d_ff_shared;
    L->shared = D->d_ff_shared > 0;
    // rows >= 8 always holds here, so the reference uses Q8_0 activations exactly when
    // supports_q8_activation allows (matmul_quant_f32, 3908-3914; matmul_swiglu_quant_f32, 3985-3991,
    // whose Q8_0 x is used by the rows of types that support it)
    L->down_f32 = !q8_activation(D->down_type, D->d_ff);
    L->sdown_f32 = L->shared && !q8_activation(D->sh_down_type, D->d_ff_shared);
    L->gu_f32 = !q8_activation(D->gate_type, D->d_model);
    L->sgu_f32 = L->shared && !q8_activation(D->sh_gate_type, D->d_model);
    L->dpad = (D->d_model + 255) / 256 * 256;
    hipStream_t st = nullptr;
    int r = JX_OK;
    auto bail = [&](int code) {
        free_layer(L);
        return code;
    };
    if (hipSetDevice(L->device) != hipSuccess) return bail(fail(JX_ERR_HIP, "hipSetDevice"));
    const size_t E = L->E, d = L->d;
    // F16 / BF16 routers widen to fp32 exactly (fp16_to_fp32 / bf16_to_fp32, src/quant.cpp:876-932); the
    // router kernels then take their products in the F16 / BF16 dot order (RouteArgs::chain8)
    std::vector<float> router_f32(E * d);
    L->chain8 = D->router_type != JX_TYPE_F32;
    if (D->router_type == JX_TYPE_F32) {
        std::copy(static_cast<const float*>(D->router), static_cast<const float*>(D->router) + E * d, router_f32.begin());
    } else {
        const uint16_t* h = static_cast<const uint16_t*>(D->router);
        for (size_t i = 0; i < E * d; ++i)
            router_f32[i] = D->router_type == JX_TYPE_F16 ? half_to_float(h[i]) : bf16_to_float(h[i]);
    }
    if ((r = dalloc(L->router, E * d)) != JX_OK) return bail(r);
    if (hipMemcpy(L->router, router_f32.data(), E * d * 4, hipMemcpyHostToDevice) != hipSuccess)
        return bail(fail(JX_ERR_HIP, "router upload"));
    if (D->router_bias) {
        if ((r = dalloc(L->bias, E)) != JX_OK) return bail(r);
        if (hipMemcpy(L->bias, D->router_bias, E * 4, hipMemcpyHostToDevice) != hipSuccess)
            return bail(fail(JX_ERR_HIP, "router bias upload"));
    }
    if ((r = upload_matrix(D->gate_type, L->E, L->F, L->d, D->gate_exps, L->gate, st, true)) != JX_OK) return bail(r);
    L->gate.m.act = D->activation;
    if ((r = upload_matrix(D->up_type, L->E, L->F, L->d, D->up_exps, L->up, st, true)) != JX_OK) return bail(r);
    if ((r = upload_matrix(D->down_type, L->E, L->d, L->F, D->down_exps, L->down, st, true)) != JX_OK) return bail(r);
    if (L->shared) {
        if ((r = upload_matrix(D->sh_gate_type, 1, L->Fs, L->d, D->sh_gate, L->sgate, st, true)) != JX_OK) return bail(r);
        // The shared expert is always SwiGLU: src/transformer.cpp:2741-2745 calls matmul_swiglu_quant_f32
        // without hp_.use_gelu (default false, include/quant.h:361); GELU-tanh reaches only the routed
        // experts (2721-2724).
        L->sgate.m.act = jx::ACT_SILU;
        if ((r = upload_matrix(D->sh_up_type, 1, L->Fs, L->d, D->sh_up, L->sup, st, true)) != JX_OK) return bail(r);
        if ((r = upload_matrix(D->sh_down_type, 1, L->d, L->Fs, D->sh_down, L->sdown, st, true)) != JX_OK) return bail(r);
        if (D->sh_gate_inp) {
            if ((r = dalloc(L->shgate, d)) != JX_OK) return bail(r);
            if (hipMemcpy(L->shgate, D->sh_gate_inp, d * 4, hipMemcpyHostToDevice) != hipSuccess)
                return bail(fail(JX_ERR_HIP, "shared gate upload"));
        }
    }
    L->eps = D->rms_norm_eps;
    if (D->ffn_norm) {
        if ((r = dalloc(L->ffn_norm, d)) != JX_OK) return bail(r);
        if (hipMemcpy(L->ffn_norm, D->ffn_norm, d * 4, hipMemcpyHostToDevice) != hipSuccess)
            return bail(fail(JX_ERR_HIP, "ffn_norm upload"));
    }
    if (D->post_ffw_norm) {
        if ((r = dalloc(L->post_norm, d)) != JX_OK) return bail(r);
        if (hipMemcpy(L->post_norm, D->post_ffw_norm, d * 4, hipMemcpyHostToDevice) != hipSuccess)
            return bail(fail(JX_ERR_HIP, "post_ffw_norm upload"));
    }
    {  // chain-major router copy for the many-token router
        const int R = L->E + (L->shgate ? 1 : 0);
        std::vector<float> rows((size_t)R * d), cm((size_t)R * 16 * jx::chain_stride((int)d));
        std::copy(router_f32.begin(), router_f32.end(), rows.begin());
        if (L->shgate) std::copy(D->sh_gate_inp, D->sh_gate_inp + d, rows.begin() + E * d);
        jx::chain_rows(rows.data(), R, (int)d, cm.data());
        if ((r = dalloc(L->router_cm, cm.size())) != JX_OK) return bail(r);
        if (hipMemcpy(L->router_cm, cm.data(), cm.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            return bail(fail(JX_ERR_HIP, "router upload"));
    }
    if ((r = ensure_workspace(L, 1)) != JX_OK) return bail(r);
    if (hipStreamCreate(&L->own) != hipSuccess) return bail(fail(JX_ERR_HIP, "stream create"));
    // the side stream: the shared expert, or the cold experts' GEMVs beside the GEMMs
    if ((hipStreamCreate(&L->side) != hipSuccess ||
                      hipEventCreateWithFlags(&L->ev_fork, hipEventDisableTiming) != hipSuccess ||
                      hipEventCreateWithFlags(&L->ev_join, hipEventDisableTiming) != hipSuccess))
        return bail(fail(JX_ERR_HIP, "shared-expert stream create"));
    // Graph replays pay where the forward forks the shared expert onto its second stream (the fork and
    // join become graph edges instead of event waits): measured per decode step with the host running
    // ahead, Qwen1.5-shaped 53.2 -> 41.6 us, DeepSeek-V2-Lite-shaped 50.1 -> 41.6 us.  Without a shared
    // expert direct launches are faster (Mixtral-shaped 49.5 -> 46.4 us, Qwen3-shaped 30.8 -> 26.0 us).
    // JX_NO_GRAPH=1 / JX_GRAPHS=1 force either way (A/B measurement).
    L->use_graphs = L->shared;
    if (const char* g = std::getenv("JX_NO_GRAPH")) L->use_graphs = L->use_graphs && std::strcmp(g, "0") == 0;
    if (const char* g = std::getenv("JX_GRAPHS")) L->use_graphs = std::strcmp(g, "0") != 0;
    if (const char* f = std::getenv("JX_NO_FOLD")) L->fold_combine = std::strcmp(f, "0") == 0;
    if (const char* f = std::getenv("JX_NO_FUSED")) L->fused_decode = std::strcmp(f, "0") == 0;
    if (const char* f = std::getenv("JX_FUSED")) L->force_fused = std::strcmp(f, "0") != 0;
    if (const char* f = std::getenv("JX_DECP")) L->decp_mode = std::strcmp(f, "0") != 0 ? 1 : 0;
    L->cold_pairs = COLD_PAIRS;
    if (const char* f = std::getenv("JX_SH_KSPLIT")) L->sh_ksplit = std::strcmp(f, "0") != 0;
    if (const char* f = std::getenv("JX_COLD_PAIRS")) L->cold_pairs = std::max(0, std::atoi(f));
    L->smfma_min = (L->shared && (L->sgate.m.type == jx::T_Q4_K || L->sgate.m.type == jx::T_Q6_K))
                       ? jx::MFMA_MIN_SHARED_TOKENS_KQ
                       : jx::MFMA_MIN_SHARED_TOKENS;
    if (const char* f = std::getenv("JX_SMFMA_MIN")) L->smfma_min = std::max(1, std::atoi(f));
    if ((r = dalloc(L->dsync, 1)) != JX_OK) return bail(r);
    if ((r = dalloc(L->hw, (size_t)L->k * L->F / 4)) != JX_OK) return bail(r);
    if (L->down_f32) {
        if ((r = dalloc(L->hfw, (size_t)L->k * L->F)) != JX_OK) return bail(r);
        if (hipMemset(L->hfw, 0, (size_t)L->k * L->F * sizeof(uint64_t)) != hipSuccess)
            return bail(fail(JX_ERR_HIP, "decode state"));
    }
    if (hipMemset(L->hw, 0, (size_t)L->k * L->F / 4 * sizeof(uint64_t)) != hipSuccess)
        return bail(fail(JX_ERR_HIP, "decode state"));
    if (hipMemset(L->dsync, 0, sizeof(jx::DecodeSync)) != hipSuccess) return bail(fail(JX_ERR_HIP, "decode state"));
    if (hipHostMalloc(reinterpret_cast<void**>(&L->herr), sizeof(uint32_t), hipHostMallocMapped | hipHostMallocCoherent) !=
            hipSuccess ||
        hipHostGetDevicePointer(reinterpret_cast<void**>(&L->herr_dev), L->herr, 0) != hipSuccess)
        return bail(fail(JX_ERR_HIP, "decode error word"));
    __atomic_store_n(L->herr, 0u, __ATOMIC_RELEASE);
    *out = L;
    return JX_OK;
}

void jx_moe_layer_destroy(jx_moe_layer* L) {
    if (L) free_layer(L);
}

namespace {
// A fused one-token launch of this layer gave up a wait between its blocks: its outputs were invalid.
// Clear the error words (the launch count keeps going, so no later launch can match a word that launch
// left) and report it.
int take_fused_error(jx_moe_layer* L) {
    if (!L->herr || __atomic_load_n(L->herr, __ATOMIC_ACQUIRE) == 0) return JX_OK;
    __atomic_store_n(L->herr, 0u, __ATOMIC_RELEASE);
    return fail(JX_ERR_HIP,
                "fused one-token step: a wait between its blocks timed out (another kernel held the GPU's CUs); "
                "the outputs of that step are invalid");
}
}  // namespace

int jx_moe_layer_status(jx_moe_layer* L, int32_t wait) {
    if (!L) return fail(JX_ERR_INVALID, "null layer");
    HIPCHK(hipSetDevice(L->device));
    if (wait) HIPCHK(hipStreamSynchronize(L->last_st ? L->last_st : L->own));
    return take_fused_error(L);
}

int jx_moe_forward(jx_moe_layer* L, const float* x, int32_t n_tok, float* out, int32_t* topk_ids, float* topk_w,
                   int32_t* expert_counts, void* stream, uint32_t flags) {
    if (!L || !x || !out) return fail(JX_ERR_INVALID, "null argument");
    if (n_tok < 1) return fail(JX_ERR_INVALID, "n_tok must be >= 1");
    if ((flags & JX_FWD_ASYNC) && !(flags & JX_FWD_DEVICE_PTRS))
        return fail(JX_ERR_INVALID, "JX_FWD_ASYNC needs JX_FWD_DEVICE_PTRS");
    if ((flags & JX_FWD_FORCE_GEMV) && (flags & JX_FWD_FORCE_MFMA))
        return fail(JX_ERR_INVALID, "conflicting regime flags");
    // (token, slot) pairs are int32 indices, and the matrix-core GEMMs address a tile's activation rows
    // with 32-bit offsets from its first row (n_tok rows of x's hi/lo form: 4 bytes per element)
    if ((int64_t)n_tok * L->k > INT_MAX / 2 || (int64_t)n_tok * L->d * 4 >= ((int64_t)1 << 32))
        return fail(JX_ERR_UNSUPPORTED, "n_tok too large for one call (split the batch)");
    HIPCHK(hipSetDevice(L->device));
    // a failure of an earlier fused step that the caller has not been told of (asynchronous calls)
    int r = take_fused_error(L);
    if (r != JX_OK) return r;
    if ((r = ensure_workspace(L, n_tok)) != JX_OK) return r;
    hipStream_t st = stream ? reinterpret_cast<hipStream_t>(stream) : L->own;
    L->last_st = st;
    const bool dev = flags & JX_FWD_DEVICE_PTRS;
    const size_t xd = (size_t)n_tok * L->d;
    const float* xin = x;
    float* outp = out;
    if (!dev) {
        HIPCHK(hipMemcpyAsync(L->x, x, xd * 4, hipMemcpyHostToDevice, st));
        xin = L->x;
        outp = L->out;
    }
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    HIPCHK(hipStreamIsCapturing(st, &cap));
    // Graphs pay off where launch overhead is a large share of the step: batches up to GRAPH_MAX_N
    // tokens (decode and batched decode).  Larger batches (prefill: milliseconds of GEMM, and a new
    // length per prompt) launch directly instead of capturing a graph for every length.
    // (the fused one-token launch is one kernel: nothing for a graph to save)
    if (L->use_graphs && !L->prof.on && cap == hipStreamCaptureStatusNone && n_tok <= jx_moe_layer::GRAPH_MAX_N &&
        !decode1_wanted(L, n_tok, flags)) {
        // the launch sequence depends only on (n, buffers, regime flags): replay a captured graph
        const jx_moe_layer::GraphKey key{n_tok, xin, outp,
                                         flags & (JX_FWD_FORCE_GEMV | JX_FWD_FORCE_MFMA | JX_FWD_RESIDUAL)};
        auto it = L->graphs.find(key);
        if (it == L->graphs.end()) {
            HIPCHK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            r = run_forward(L, xin, n_tok, outp, st, flags);
            hipGraph_t g = nullptr;
            const hipError_t e = hipStreamEndCapture(st, &g);
            if (r != JX_OK) {
                if (g) (void)hipGraphDestroy(g);
                return r;
            }
            if (e != hipSuccess) return fail(JX_ERR_HIP, std::string("graph capture: ") + hipGetErrorString(e));
            hipGraphExec_t ex = nullptr;
            const hipError_t ei = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (ei != hipSuccess) return fail(JX_ERR_HIP, std::string("graph instantiate: ") + hipGetErrorString(ei));
            if (L->graphs.size() >= jx_moe_layer::GRAPH_CACHE) {  // evict the least recently used
                auto lru = L->graphs.begin();
                for (auto g2 = L->graphs.begin(); g2 != L->graphs.end(); ++g2)
                    if (g2->second.last < lru->second.last) lru = g2;
                (void)hipGraphExecDestroy(lru->second.exec);
                L->graphs.erase(lru);
            }
            it = L->graphs.emplace(key, jx_moe_layer::Graph{ex, 0}).first;
        }
        it->second.last = ++L->graph_clock;
        HIPCHK(hipGraphLaunch(it->second.exec, st));
    } else if ((r = run_forward(L, xin, n_tok, outp, st, flags)) != JX_OK) {
        return r;
    }
    L->last_n = n_tok;
    const size_t nk = (size_t)n_tok * L->k;
    const hipMemcpyKind k2 = dev ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost;
    if (!dev) HIPCHK(hipMemcpyAsync(out, L->out, xd * 4, hipMemcpyDeviceToHost, st));
    if (topk_ids) HIPCHK(hipMemcpyAsync(topk_ids, L->ids, nk * 4, k2, st));
    if (topk_w) HIPCHK(hipMemcpyAsync(topk_w, L->probs, nk * 4, k2, st));
    if (expert_counts) HIPCHK(hipMemcpyAsync(expert_counts, L->counts, (size_t)L->E * 4, k2, st));
    if (!(flags & JX_FWD_ASYNC)) {
        HIPCHK(hipStreamSynchronize(st));
        if (L->prof.on && (r = resolve_profile(L)) != JX_OK) return r;
        if (L->decp_used) {  // this call's one-block-per-CU launch is done
            std::lock_guard<std::mutex> lk(g_fused_order.mu);
            if (g_fused_order.pending[L->device] == st) g_fused_order.pending[L->device] = nullptr;
        }
        if ((r = take_fused_error(L)) != JX_OK) return r;  // a bounded wait of a fused launch gave up
    }
    return JX_OK;
}

int jx_moe_last_logits(jx_moe_layer* L, float* logits_host, int32_t n_tok) {
    if (!L || !logits_host) return fail(JX_ERR_INVALID, "null argument");
    if (n_tok < 1 || n_tok > L->last_n) return fail(JX_ERR_INVALID, "n_tok exceeds the last forward");
    HIPCHK(hipSetDevice(L->device));
    HIPCHK(hipDeviceSynchronize());
    HIPCHK(hipMemcpy(logits_host, L->logits, (size_t)n_tok * L->E * 4, hipMemcpyDeviceToHost));
    return JX_OK;
}

int jx_moe_last_xq8(jx_moe_layer* L, void* blocks_host, int32_t n_tok) {
    if (!L || !blocks_host) return fail(JX_ERR_INVALID, "null argument");
    if (n_tok < 1 || n_tok > L->last_n) return fail(JX_ERR_INVALID, "n_tok exceeds the last forward");
    HIPCHK(hipSetDevice(L->device));
    HIPCHK(hipDeviceSynchronize());
    return download_q8_blocks(L->xq, n_tok, static_cast<uint8_t*>(blocks_host));
}

int jx_moe_profile(jx_moe_layer* L, int32_t enable) {
    if (!L) return fail(JX_ERR_INVALID, "null layer");
    L->prof.on = enable != 0;
    L->prof.acc.clear();
    L->prof.pending.clear();
    L->prof.used = 0;
    return JX_OK;
}

int jx_moe_profile_read(jx_moe_layer* L, char* names_buf, size_t names_len, double* ms, int64_t* launches,
                        int32_t max_entries, int32_t* n_entries) {
    if (!L || !names_buf || !ms || !launches || !n_entries) return fail(JX_ERR_INVALID, "null argument");
    HIPCHK(hipSetDevice(L->device));
    int r = resolve_profile(L);
    if (r != JX_OK) return r;
    std::string names;
    int i = 0;
    for (auto& kv : L->prof.acc) {
        if (i >= max_entries) break;
        names += kv.first + ";";
        ms[i] = kv.second.first;
        launches[i] = kv.second.second;
        ++i;
    }
    if (names.size() + 1 > names_len) return fail(JX_ERR_INVALID, "names buffer too small");
    std::memcpy(names_buf, names.c_str(), names.size() + 1);
    *n_entries = i;
    return JX_OK;
}

// ---- math-API drop-ins -----------------------------------------------------

int jx_qmatrix_create(int32_t type, int64_t rows, int64_t cols, const void* host, jx_qmatrix** out) {
    if (!host || !out) return fail(JX_ERR_INVALID, "null argument");
    *out = nullptr;
    if (g_device < 0) return fail(JX_ERR_NODEVICE, "jx_moe_init has not been called");
    if (rows < 1 || cols < 1 || rows > (1 << 24) || cols > (1 << 20)) return fail(JX_ERR_INVALID, "bad shape");
    HIPCHK(hipSetDevice(g_device));
    auto* m = new jx_qmatrix();
    m->device = g_device;
    m->type = type;
    m->rows = (int)rows;
    m->cols = (int)cols;
    // rows padded to whole 32-row tiles with zero blocks (their dots are zero and never written out)
    const int64_t rpad = (rows + jx::ROWS_PER_TILE - 1) / jx::ROWS_PER_TILE * jx::ROWS_PER_TILE;
    const size_t rb = row_bytes(type, cols);
    std::vector<uint8_t> padded;
    const void* src = host;
    if (rpad != rows && rb) {
        padded.assign((size_t)rpad * rb, 0);
        std::memcpy(padded.data(), host, (size_t)rows * rb);
        src = padded.data();
    }
    int r = upload_matrix(type, 1, (int)rpad, (int)cols, src, m->w, nullptr);
    m->w.m.valid_rows = (int)rows;
    const size_t kpad = ((size_t)cols + 255) / 256 * 256;
    if (r == JX_OK) r = dalloc(m->xq.q, kpad);
    if (r == JX_OK) r = dalloc(m->xq.s, kpad / 32);
    if (r == JX_OK) r = dalloc(m->xf, kpad);
    if (r != JX_OK) {
        jx_qmatrix_destroy(m);
        return r;
    }
    m->xq.K = (int)cols;
    *out = m;
    return JX_OK;
}

void jx_qmatrix_destroy(jx_qmatrix* m) {
    if (!m) return;
    (void)hipSetDevice(m->device);
    m->w.release();
    for (void* p : {(void*)m->xq.q, (void*)m->xq.s, (void*)m->xf})
        if (p) (void)hipFree(p);
    delete m;
}

// One matrix of the device-pointer drop-ins: out[r] = W[r] . x over the Q8_0 form xq (q8) or the
// zero-padded fp32 copy xf of the same activation row.
static int dev_gemv(jx_qmatrix* W, bool q8, const jx::ActQ8& xq, float* xf, float* out, hipStream_t st) {
    const size_t kpad = ((size_t)W->cols + 255) / 256 * 256;
    if (kpad > (size_t)jx::gemv_max_k(false, 1, !q8))
        return fail(JX_ERR_UNSUPPORTED, "cols exceeds the GEMV's staged activation capacity");
    jx::Groups g;
    g.identity = 1;
    g.n_tok = 1;
    if (q8) {
        jx::launch_gemv_down(W->w.m, xq, nullptr, 0, g, 1, 1, out, st);
    } else {
        jx::ActQ8 a;
        a.K = (int)kpad;
        jx::launch_gemv_down(W->w.m, a, xf, (int)kpad, g, 1, 1, out, st);
    }
    return JX_OK;
}

int jx_matmul_quant_f32_dev(jx_qmatrix* W, const float* x_dev, float* out_dev, void* stream) {
    if (!W || !x_dev || !out_dev) return fail(JX_ERR_INVALID, "null argument");
    HIPCHK(hipSetDevice(W->device));
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const bool q8 = W->rows >= 8 && q8_activation(W->type, W->cols);  // matmul_quant_f32, quant.cpp:3908
    const size_t kpad = ((size_t)W->cols + 255) / 256 * 256;
    if (q8)
        jx::launch_quantize_q8(x_dev, 1, W->cols, W->xq, st);
    else
        jx::launch_copy_pad(x_dev, W->cols, (int)kpad, W->xf, st);
    int r = dev_gemv(W, q8, W->xq, W->xf, out_dev, st);
    if (r != JX_OK) return r;
    HIPCHK(hipGetLastError());
    return JX_OK;
}

int jx_matmul_qkv_quant_f32_dev(jx_qmatrix* Wq, jx_qmatrix* Wk, jx_qmatrix* Wv, const float* x_dev, float* q_dev,
                                float* k_dev, float* v_dev, void* stream) {
    jx_qmatrix* Ws[3] = {Wq, Wk, Wv};
    float* outs[3] = {q_dev, k_dev, v_dev};
    jx_qmatrix* first = nullptr;
    int64_t total_rows = 0;
    for (int i = 0; i < 3; ++i) {
        if (!Ws[i]) continue;
        if (!outs[i]) return fail(JX_ERR_INVALID, "null output for a given matrix");
        if (!first) first = Ws[i];
        if (Ws[i]->cols != first->cols || Ws[i]->device != first->device)
            return fail(JX_ERR_INVALID, "q, k and v matrices must share cols and device");
        total_rows += Ws[i]->rows;
    }
    if (!first || !x_dev) return fail(JX_ERR_INVALID, "null argument");
    HIPCHK(hipSetDevice(first->device));
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int cols = first->cols;
    const size_t kpad = ((size_t)cols + 255) / 256 * 256;
    // x quantized once when the three matrices hold 8 rows or more (matmul_qkv_quant_f32,
    // quant.cpp:3940-3947); each row then takes the Q8_0 form where its type allows
    // (vec_dot_row_with_q8, 3841-3879), fp32 otherwise
    const bool quantized = total_rows >= 8 && cols % 32 == 0;
    bool need_f32 = false;
    for (int i = 0; i < 3; ++i)
        if (Ws[i] && !(quantized && q8_activation(Ws[i]->type, cols))) need_f32 = true;
    if (quantized) jx::launch_quantize_q8(x_dev, 1, cols, first->xq, st);
    if (need_f32) jx::launch_copy_pad(x_dev, cols, (int)kpad, first->xf, st);
    for (int i = 0; i < 3; ++i) {
        if (!Ws[i]) continue;
        const int r = dev_gemv(Ws[i], quantized && q8_activation(Ws[i]->type, cols), first->xq, first->xf, outs[i], st);
        if (r != JX_OK) return r;
    }
    HIPCHK(hipGetLastError());
    return JX_OK;
}

int jx_matmul_quant_f32(jx_qmatrix* W, const float* x, float* out) {
    if (!W || !x || !out) return fail(JX_ERR_INVALID, "null argument");
    HIPCHK(hipSetDevice(W->device));
    const int rows = W->rows, cols = W->cols;
    const bool q8 = rows >= 8 && q8_activation(W->type, cols);
    if (((size_t)cols + 255) / 256 * 256 > (size_t)jx::gemv_max_k(false, 1, !q8))
        return fail(JX_ERR_UNSUPPORTED, "cols exceeds the GEMV's staged activation capacity");
    Scratch s;
    const size_t kpad = ((size_t)cols + 255) / 256 * 256;
    float* xd = s.get<float>(kpad);
    float* yd = s.get<float>(rows);
    if (!xd || !yd) return fail(JX_ERR_NOMEM, "scratch allocation");
    HIPCHK(hipMemset(xd, 0, kpad * 4));
    HIPCHK(hipMemcpy(xd, x, (size_t)cols * 4, hipMemcpyHostToDevice));
    jx::Groups g;
    g.identity = 1;
    g.n_tok = 1;
    jx::ActQ8 a;
    if (q8) {
        a.q = s.get<int8_t>(cols);
        a.s = s.get<float2>(cols / 32);
        a.K = cols;
        if (!a.q || !a.s) return fail(JX_ERR_NOMEM, "scratch allocation");
        jx::launch_quantize_q8(xd, 1, cols, a, nullptr);
        jx::launch_gemv_down(W->w.m, a, nullptr, 0, g, 1, 1, yd, nullptr);
    } else {
        a.K = (int)kpad;
        jx::launch_gemv_down(W->w.m, a, xd, (int)kpad, g, 1, 1, yd, nullptr);
    }
    HIPCHK(hipGetLastError());
    HIPCHK(hipMemcpy(out, yd, (size_t)rows * 4, hipMemcpyDeviceToHost));
    return JX_OK;
}

int jx_matmul_quant_f32_noalloc(jx_qmatrix* W, const float* x_dev, float* out_dev, void* stream) {
    if (!W || !x_dev || !out_dev) return fail(JX_ERR_INVALID, "null argument");
    const int rows = W->rows, cols = W->cols;
    const bool q8 = rows >= 8 && q8_activation(W->type, cols);
    const size_t kpad = ((size_t)cols + 255) / 256 * 256;
    if (kpad > NOALLOC_MAX_COLS)
        return fail(JX_ERR_UNSUPPORTED, "cols exceed the no-allocation scratch (" + std::to_string(NOALLOC_MAX_COLS) +
                                            " columns)");
    if (kpad > (size_t)jx::gemv_max_k(false, 1, !q8))
        return fail(JX_ERR_UNSUPPORTED, "cols exceeds the GEMV's staged activation capacity");
    if (W->device < 0 || W->device >= MAX_DEVICES || !g_scratch[W->device].load())
        return fail(JX_ERR_NODEVICE, "jx_moe_init has not been called for the matrix's device");
    HIPCHK(hipSetDevice(W->device));
    uint8_t* sp = static_cast<uint8_t*>(g_scratch[W->device].load());
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    jx::Groups g;
    g.identity = 1;
    g.n_tok = 1;
    jx::ActQ8 a;
    if (q8) {  // every scale, sum and quant of the row is written before the GEMV reads it
        a.s = reinterpret_cast<float2*>(sp);
        a.q = reinterpret_cast<int8_t*>(sp + (size_t)cols / 32 * sizeof(float2));
        a.K = cols;
        jx::launch_quantize_q8(x_dev, 1, cols, a, st);
        jx::launch_gemv_down(W->w.m, a, nullptr, 0, g, 1, 1, out_dev, st);
    } else {  // fp32 activations zero-padded to whole super-blocks (the padding is rewritten every call)
        float* xf = reinterpret_cast<float*>(sp);
        jx::launch_copy_pad(x_dev, cols, (int)kpad, xf, st);
        a.K = (int)kpad;
        jx::launch_gemv_down(W->w.m, a, xf, (int)kpad, g, 1, 1, out_dev, st);
    }
    HIPCHK(hipGetLastError());
    return JX_OK;
}

int jx_matmul_swiglu_quant_f32(jx_qmatrix* Wg, jx_qmatrix* Wu, const float* x, float* out, int32_t use_gelu) {
    if (!Wg || !Wu || !x || !out) return fail(JX_ERR_INVALID, "null argument");
    if (Wg->rows != Wu->rows || Wg->cols != Wu->cols || Wg->type != Wu->type)
        return fail(JX_ERR_UNSUPPORTED, "gate and up must share shape and type");
    HIPCHK(hipSetDevice(Wg->device));
    const int rows = Wg->rows, cols = Wg->cols;
    // Q8_0 x iff exp_dim >= 8 and cols % 32 == 0 (quant.cpp:3985-3991), used by rows whose type allows it
    const bool q8 = rows >= 8 && cols % 32 == 0 && q8_activation(Wg->type, cols);
    const size_t kpad = ((size_t)cols + 255) / 256 * 256;
    if ((q8 ? (size_t)cols : kpad) > (size_t)jx::gemv_max_k(true, 1, !q8))
        return fail(JX_ERR_UNSUPPORTED, "cols exceeds the GEMV's staged activation capacity");
    Scratch s;
    float* xd = s.get<float>(kpad);
    const size_t fpad = ((size_t)rows + 255) / 256 * 256;
    float* hf = s.get<float>(fpad);
    jx::ActQ8 a, hq;
    a.q = s.get<int8_t>(cols);
    a.s = s.get<float2>(cols / 32);
    a.K = cols;
    if (!xd || !hf || !a.q || !a.s) return fail(JX_ERR_NOMEM, "scratch allocation");
    HIPCHK(hipMemset(xd, 0, kpad * 4));
    HIPCHK(hipMemcpy(xd, x, (size_t)cols * 4, hipMemcpyHostToDevice));
    if (q8) jx::launch_quantize_q8(xd, 1, cols, a, nullptr);
    jx::Groups g;
    g.identity = 1;
    g.n_tok = 1;
    hq.K = rows;  // q == nullptr: no Q8_0 output wanted
    jx::QMat gm = Wg->w.m;
    gm.act = use_gelu ? jx::ACT_GELU_TANH : jx::ACT_SILU;
    jx::launch_gemv_gateup(gm, Wu->w.m, a, g, 1, 1, hq, hf, nullptr, nullptr, q8 ? nullptr : xd, (int)kpad);
    HIPCHK(hipGetLastError());
    HIPCHK(hipMemcpy(out, hf, (size_t)rows * 4, hipMemcpyDeviceToHost));
    return JX_OK;
}

int jx_quantize_row_q8_0(const float* x, void* blocks, int64_t k) {
    if (!x || !blocks) return fail(JX_ERR_INVALID, "null argument");
    if (k < 32 || k % 32 != 0) return fail(JX_ERR_INVALID, "k must be a positive multiple of 32");
    if (g_device < 0) return fail(JX_ERR_NODEVICE, "jx_moe_init has not been called");
    HIPCHK(hipSetDevice(g_device));
    Scratch s;
    float* xd = s.get<float>(k);
    jx::ActQ8 a;
    a.q = s.get<int8_t>(k);
    a.s = s.get<float2>(k / 32);
    a.K = (int)k;
    if (!xd || !a.q || !a.s) return fail(JX_ERR_NOMEM, "scratch allocation");
    HIPCHK(hipMemcpy(xd, x, (size_t)k * 4, hipMemcpyHostToDevice));
    jx::launch_quantize_q8(xd, 1, (int)k, a, nullptr);
    HIPCHK(hipGetLastError());
    return download_q8_blocks(a, 1, static_cast<uint8_t*>(blocks));
}

int jx_dev_alloc(size_t bytes, void** ptr) {
    if (!ptr) return fail(JX_ERR_INVALID, "null argument");
    if (g_device >= 0) HIPCHK(hipSetDevice(g_device));
    HIPCHK(hipMalloc(ptr, bytes));
    return JX_OK;
}

int jx_dev_free(void* ptr) {
    HIPCHK(hipFree(ptr));
    return JX_OK;
}

int jx_memcpy_htod(void* dst, const void* src, size_t bytes) {
    HIPCHK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return JX_OK;
}

int jx_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    HIPCHK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return JX_OK;
}

int jx_device_synchronize(void) {
    HIPCHK(hipDeviceSynchronize());
    return JX_OK;
}

#ifndef JX_SOURCE_SHA
#define JX_SOURCE_SHA "unknown"
#endif
const char* jx_build_id(void) { return JX_SOURCE_SHA; }

}  // extern "C"

// Golden-vector driver around the reference engine's own arithmetic --
// TEST INFRASTRUCTURE ONLY.
//
// Compiled together with the reference's src/quant.cpp and src/tier.cpp, read
// in place from the reference tree (see oracle/Makefile), into
// oracle/_ref/libjxref.so.  It exposes the oracle's C API (jxr_* mirrors
// jxo_*) so the tests can compare the C restatement in moe_oracle.c with the
// reference build bit for bit, and so the benchmark can time the reference's
// CPU path on the GPU host.  No reference source is copied: the MoE-block
// sequence below replays src/transformer.cpp:2589-2757 by calling the
// reference's own functions.
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "gguf.h"
#include "quant.h"
#include "tier.h"

#include "moe_oracle.h"

using moe::GGMLType;

extern "C" {

void jxr_set_avx512(int32_t on) {
    // The reference caches MOE_AVX512 on its first dot call
    // (quant.cpp:3823-3839); call this before any other jxr_ function.
    setenv("MOE_AVX512", on ? "1" : "0", 1);
}

uint16_t jxr_fp32_to_fp16(float f) { return moe::fp32_to_fp16(f); }
float jxr_fp16_to_fp32(uint16_t h) { return moe::fp16_to_fp32(h); }
void jxr_quantize_row_q8_0(const float* x, uint8_t* y, int64_t k) { moe::quantize_row_q8_0(x, y, k); }
void jxr_dequantize_row(int32_t type, const uint8_t* w, float* y, int64_t k) {
    moe::dequantize_row(static_cast<GGMLType>(type), w, y, k);
}
float jxr_vec_dot_f32(const float* a, const float* b, int64_t k) { return moe::vec_dot_f32(a, b, k); }
float jxr_vec_dot_q4_K_f32(const uint8_t* w, const float* y, int64_t k) { return moe::vec_dot_q4_K_f32(w, y, k); }

// The AVX2 block dots are exported by quant.h; the AVX-512 ones are file-local
// and reached through the matmul dispatcher only.
float jxr_vec_dot_q8(int32_t type, const uint8_t* w, const uint8_t* xq8, int64_t k) {
    const auto* y = reinterpret_cast<const moe::block_q8_0*>(xq8);
    switch (type) {
        case JXO_Q4_0: return moe::vec_dot_q4_0_q8_0(w, y, k);
        case JXO_Q8_0: return moe::vec_dot_q8_0_q8_0(w, y, k);
        case JXO_Q4_K: return moe::vec_dot_q4_K_q8_0(w, y, k);
        case JXO_Q5_K: return moe::vec_dot_q5_K_q8_0(w, y, k);
        case JXO_Q6_K: return moe::vec_dot_q6_K_q8_0(w, y, k);
        default: return 0.0f;
    }
}

float jxr_vec_dot_quant_f32(int32_t type, const uint8_t* w, const float* y, int64_t k) {
    return moe::vec_dot_quant_f32(static_cast<GGMLType>(type), w, y, k);
}

void jxr_matmul_quant_f32(int32_t type, const uint8_t* W, const float* x, float* out, int64_t rows, int64_t cols) {
    moe::matmul_quant_f32(static_cast<GGMLType>(type), W, x, out, rows, cols);
}

void jxr_matmul_swiglu_quant_f32(int32_t gt, const uint8_t* Wg, int32_t ut, const uint8_t* Wu,
                                 const float* x, float* out, int64_t exp_dim, int64_t cols, int32_t use_gelu) {
    moe::matmul_swiglu_quant_f32(static_cast<GGMLType>(gt), Wg, static_cast<GGMLType>(ut), Wu,
                                 x, out, exp_dim, cols, use_gelu != 0);
}

void jxr_matmul_qkv_quant_f32(int32_t qt, const uint8_t* Wq, int64_t q_rows, float* q_out, int32_t kt,
                              const uint8_t* Wk, int64_t k_rows, float* k_out, int32_t vt, const uint8_t* Wv,
                              int64_t v_rows, float* v_out, const float* x, int64_t cols) {
    moe::matmul_qkv_quant_f32(static_cast<GGMLType>(qt), Wq, q_rows, q_out, static_cast<GGMLType>(kt), Wk, k_rows,
                              k_out, static_cast<GGMLType>(vt), Wv, v_rows, v_out, x, cols);
}

// select_experts_cache_aware with CACHE_ROUTE off (eps = 0, nothing resident).
int32_t jxr_select_experts(const float* logits, int32_t E, int32_t k, int32_t* ids, float* probs) {
    moe::LFRUTierManager tier;
    tier.init(1, static_cast<uint32_t>(E), 0, 0, 0.0f);
    auto sel = tier.select_experts_cache_aware(0, logits, static_cast<uint32_t>(E), static_cast<uint32_t>(k));
    for (size_t i = 0; i < sel.size(); ++i) {
        ids[i] = static_cast<int32_t>(sel[i].expert_idx);
        probs[i] = sel[i].prob;
    }
    return static_cast<int32_t>(sel.size());
}

// ModelFile::open on a GGUF file (src/gguf.cpp), for checking the library's
// parser: the tensor count, then per name its type, dims, absolute offset and
// byte size, and metadata through get_u32 / get_f32.
void* jxr_gguf_open(const char* path) {
    auto* mf = new moe::ModelFile();
    std::string err;
    if (!mf->open(path, err)) {
        delete mf;
        return nullptr;
    }
    return mf;
}
void jxr_gguf_close(void* mf) { delete static_cast<moe::ModelFile*>(mf); }
int64_t jxr_gguf_tensor_count(void* mf) { return (int64_t)static_cast<moe::ModelFile*>(mf)->tensor_names().size(); }
const char* jxr_gguf_tensor_name(void* mf, int64_t i) {
    return static_cast<moe::ModelFile*>(mf)->tensor_names()[(size_t)i].c_str();
}
int32_t jxr_gguf_tensor(void* mf, const char* name, int32_t* type, int32_t* n_dims, uint64_t* dims,
                        uint64_t* abs_offset, uint64_t* byte_size) {
    const auto* t = static_cast<moe::ModelFile*>(mf)->find_tensor(name);
    if (!t) return -1;
    *type = static_cast<int32_t>(t->type);
    *n_dims = static_cast<int32_t>(t->n_dims);
    for (int d = 0; d < 4; ++d) dims[d] = t->dims[d];
    *abs_offset = t->abs_file_offset;
    *byte_size = t->byte_size;
    return 0;
}
uint32_t jxr_gguf_get_u32(void* mf, const char* key, uint32_t def) {
    return static_cast<moe::ModelFile*>(mf)->get_u32(key, def);
}
float jxr_gguf_get_f32(void* mf, const char* key, float def) {
    return static_cast<moe::ModelFile*>(mf)->get_f32(key, def);
}

// The counters select_experts_cache_aware leaves in LFRUTierManager
// (tier.cpp:186-194) for n_tok tokens routed one forward_token at a time
// (step_tick first, transformer.cpp:2371), after ticks_before earlier steps,
// read back through snapshot_telemetry (tier.cpp:233-263): activations, LFRU
// score and last probability per (layer, expert), flat [n_layers][E].
int32_t jxr_tier_replay(const float* logits, int32_t n_tok, int32_t E, int32_t k, int32_t layer, int32_t n_layers,
                        int32_t ticks_before, uint32_t* activations, uint32_t* lfru_score, float* last_prob) {
    moe::LFRUTierManager tier;
    tier.init(static_cast<uint32_t>(n_layers), static_cast<uint32_t>(E), 0, 0, 0.0f);
    for (int32_t i = 0; i < ticks_before; ++i) tier.step_tick();
    for (int32_t t = 0; t < n_tok; ++t) {
        tier.step_tick();
        (void)tier.select_experts_cache_aware(static_cast<uint32_t>(layer), logits + static_cast<size_t>(t) * E,
                                              static_cast<uint32_t>(E), static_cast<uint32_t>(k));
    }
    const auto snap = tier.snapshot_telemetry();
    for (const auto& e : snap) {
        const size_t flat = static_cast<size_t>(e.layer) * static_cast<size_t>(E) + e.expert;
        activations[flat] = e.activations;
        lfru_score[flat] = e.lfru_score;
        last_prob[flat] = e.last_prob;
    }
    return static_cast<int32_t>(snap.size());
}

// MoETransformerEngine::rms_norm (transformer.cpp:67-73) is a member of the
// engine, whose translation unit needs the whole engine; its three steps around
// the reference's own vec_dot_f32, for the residual-stream form below.
static void ref_rms_norm(float* out, const float* x, const float* w, int64_t size, float eps) {
    const float ss = moe::vec_dot_f32(x, x, size);
    const float inv_rms = 1.0f / std::sqrt((ss / static_cast<float>(size)) + eps);
    for (int64_t i = 0; i < size; ++i) out[i] = x[i] * inv_rms * (w ? w[i] : 1.0f);
}

// The MoE block of forward_token (transformer.cpp:2589-2757) for the listed
// tokens: router GEMV, optional harness-side logit bias, top-k, routed experts
// in selection order, shared expert with optional sigmoid gate.
int32_t jxr_moe_forward(const jxo_moe_desc* L, const float* x, int32_t n_tok,
                        const int32_t* token_idx, int32_t n_sel,
                        float* out, int32_t* topk_ids, float* topk_w, float* logits_out) {
    const uint32_t E = static_cast<uint32_t>(L->n_experts);
    const uint32_t d = static_cast<uint32_t>(L->d_model);
    const uint32_t Fd = static_cast<uint32_t>(L->d_ff);
    const uint32_t k = static_cast<uint32_t>(L->top_k);
    const auto gt = static_cast<GGMLType>(L->gate_type);
    const auto ut = static_cast<GGMLType>(L->up_type);
    const auto dt = static_cast<GGMLType>(L->down_type);
    const size_t gsl = static_cast<size_t>(Fd) * moe::tensor_byte_size(gt, d);
    const size_t usl = static_cast<size_t>(Fd) * moe::tensor_byte_size(ut, d);
    const size_t dsl = static_cast<size_t>(d) * moe::tensor_byte_size(dt, Fd);

    moe::LFRUTierManager tier;
    tier.init(1, E, 0, 0, 0.0f);

    const uint32_t fmax = Fd > static_cast<uint32_t>(L->d_ff_shared) ? Fd : static_cast<uint32_t>(L->d_ff_shared);
    std::vector<float> logits(E), gate_buf(fmax), down_buf(d), moe_accum(d);
    const int32_t cnt = token_idx ? n_sel : n_tok;
    for (int32_t i = 0; i < cnt; ++i) {
        const int32_t t = token_idx ? token_idx[i] : i;
        if (t < 0 || t >= n_tok) return -2;
        const float* xt = x + static_cast<size_t>(t) * d;
        std::vector<float> xnorm(d);
        if (L->residual) ref_rms_norm(xnorm.data(), xt, L->ffn_norm, d, L->rms_eps);  // 2585-2587
        const float* xn = L->residual ? xnorm.data() : xt;

        std::fill(logits.begin(), logits.end(), 0.0f);
        moe::matmul_quant_f32(static_cast<GGMLType>(L->router_type), L->router, xn, logits.data(), E, d);
        if (L->router_bias)
            for (uint32_t e = 0; e < E; ++e) logits[e] = logits[e] + L->router_bias[e];
        auto selected = tier.select_experts_cache_aware(0, logits.data(), E, k);

        std::fill(moe_accum.begin(), moe_accum.end(), 0.0f);
        for (uint32_t s = 0; s < selected.size(); ++s) {
            const auto& sel = selected[s];
            const size_t e = sel.expert_idx;
            moe::matmul_swiglu_quant_f32(gt, L->gate + e * gsl, ut, L->up + e * usl,
                                         xn, gate_buf.data(), Fd, d, L->activation != 0);
            moe::matmul_quant_f32(dt, L->down + e * dsl, gate_buf.data(), down_buf.data(), d, Fd);
            for (uint32_t j = 0; j < d; ++j) moe_accum[j] += sel.prob * down_buf[j];
            topk_ids[static_cast<size_t>(i) * k + s] = static_cast<int32_t>(sel.expert_idx);
            topk_w[static_cast<size_t>(i) * k + s] = sel.prob;
        }
        if (L->d_ff_shared > 0 && L->sh_gate && L->sh_up && L->sh_down) {
            const uint32_t sh_dim = static_cast<uint32_t>(L->d_ff_shared);
            std::vector<float> sh_buf(sh_dim, 0.0f);
            moe::matmul_swiglu_quant_f32(static_cast<GGMLType>(L->sh_gate_type), L->sh_gate,
                                         static_cast<GGMLType>(L->sh_up_type), L->sh_up,
                                         xn, sh_buf.data(), sh_dim, d);  // use_gelu left at false, as 2741-2745
            moe::matmul_quant_f32(static_cast<GGMLType>(L->sh_down_type), L->sh_down,
                                  sh_buf.data(), down_buf.data(), d, sh_dim);
            float sh_scale = 1.0f;
            if (L->sh_gate_inp) {
                const float g_val = moe::vec_dot_quant_f32(GGMLType::F32, L->sh_gate_inp, xn, d);
                sh_scale = 1.0f / (1.0f + std::exp(-g_val));
            }
            for (uint32_t j = 0; j < d; ++j) moe_accum[j] += sh_scale * down_buf[j];
        }
        if (L->residual) {
            if (L->post_ffw_norm) ref_rms_norm(moe_accum.data(), moe_accum.data(), L->post_ffw_norm, d, L->rms_eps);
            for (uint32_t j = 0; j < d; ++j) moe_accum[j] = xt[j] + moe_accum[j];  // 2762-2764
        }
        std::memcpy(out + static_cast<size_t>(i) * d, moe_accum.data(), sizeof(float) * d);
        if (logits_out) std::memcpy(logits_out + static_cast<size_t>(i) * E, logits.data(), sizeof(float) * E);
    }
    return 0;
}

}  // extern "C"

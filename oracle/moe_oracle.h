/*
 * CPU oracle for the MoE expert path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference engine's CPU arithmetic for the MoE
 * block (router GEMV, top-k softmax, Q8_0 activation quantization, quantized
 * gate/up/down dots with SwiGLU, weighted combine, shared expert).  It exists
 * to check the HIP library: only the test-suite, the smoke check and the
 * benchmark's CPU-baseline leg may load it.  The product path never calls it.
 *
 * Every function names the reference file:line it restates.  fp32 operations
 * are issued in the reference's order (the AVX2 lane layout of its dot
 * kernels, or the AVX-512 layout when order == JXO_ORDER_AVX512) with explicit
 * fmaf(), so results are bit-identical to the reference build.
 */
#ifndef JX_MOE_ORACLE_H
#define JX_MOE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { JXO_F32 = 0, JXO_F16 = 1, JXO_Q4_0 = 2, JXO_Q5_0 = 6, JXO_Q8_0 = 8, JXO_Q4_K = 12, JXO_Q5_K = 13,
       JXO_Q6_K = 14, JXO_BF16 = 30 };
enum { JXO_ORDER_AVX2 = 0, JXO_ORDER_AVX512 = 1 };

typedef struct {
    int32_t n_experts, top_k, d_model, d_ff;
    int32_t gate_type, up_type, down_type;
    const void* router;        /* [E][d] of router_type (F32, F16 or BF16)   */
    const float* router_bias;  /* [E] fp32 added after the GEMV, or NULL     */
    const uint8_t* gate;       /* [E][d_ff] rows of d_model, block layout     */
    const uint8_t* up;
    const uint8_t* down;       /* [E][d_model] rows of d_ff                  */
    int32_t d_ff_shared;       /* 0 = no shared expert                       */
    int32_t sh_gate_type, sh_up_type, sh_down_type;
    const uint8_t* sh_gate;
    const uint8_t* sh_up;
    const uint8_t* sh_down;
    const float* sh_gate_inp;  /* [d] fp32 sigmoid gate, or NULL             */
    int32_t activation;        /* 0 SiLU, 1 GELU-tanh (the reference's use_gelu) */
    const float* ffn_norm;     /* [d] fp32 or NULL (weight 1)                */
    const float* post_ffw_norm;/* [d] fp32 or NULL (none)                    */
    float rms_eps;
    int32_t residual;          /* x is the residual stream: out = x + post(block(rms_norm(x))) */
    int32_t router_type;       /* JXO_F32, JXO_F16 or JXO_BF16                */
} jxo_moe_desc;

uint16_t jxo_fp32_to_fp16(float f);
float jxo_fp16_to_fp32(uint16_t h);
int64_t jxo_row_bytes(int32_t type, int64_t cols);
void jxo_quantize_row_q8_0(const float* x, uint8_t* blocks, int64_t k);
void jxo_dequantize_row(int32_t type, const uint8_t* w, float* y, int64_t k);
float jxo_vec_dot_f32(const float* a, const float* b, int64_t k);
void jxo_rms_norm(float* out, const float* x, const float* weight, int64_t size, float eps);
float jxo_vec_dot_q8(int32_t type, const uint8_t* w, const uint8_t* xq8, int64_t k, int32_t order);
float jxo_vec_dot_q4_K_f32(const uint8_t* w, const float* y, int64_t k);
/* vec_dot_f16_f32 / vec_dot_bf16_f32 (src/quant.cpp:3015-3055): w holds half / bfloat16 bits. */
float jxo_vec_dot_h16_f32(int32_t type, const uint16_t* w, const float* y, int64_t k);
/* vec_dot_quant_f32 (src/quant.cpp:3269-3305) for F32, F16, BF16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K. */
float jxo_vec_dot_quant_f32(int32_t type, const uint8_t* w, const float* y, int64_t k);
void jxo_matmul_quant_f32(int32_t type, const uint8_t* W, const float* x, float* out,
                          int64_t rows, int64_t cols, int32_t order);
void jxo_matmul_swiglu_quant_f32(int32_t gate_type, const uint8_t* Wg, int32_t up_type, const uint8_t* Wu,
                                 const float* x, float* out, int64_t exp_dim, int64_t cols, int32_t use_gelu,
                                 int32_t order);
void jxo_matmul_qkv_quant_f32(int32_t wq_type, const uint8_t* Wq, int64_t q_rows, float* q_out,
                              int32_t wk_type, const uint8_t* Wk, int64_t k_rows, float* k_out,
                              int32_t wv_type, const uint8_t* Wv, int64_t v_rows, float* v_out,
                              const float* x, int64_t cols, int32_t order);
int32_t jxo_select_experts(const float* logits, int32_t n_experts, int32_t top_k,
                           int32_t* ids, float* probs);
/* One MoE block over the tokens listed in token_idx (all n_tok when NULL). */
int32_t jxo_moe_forward(const jxo_moe_desc* L, const float* x, int32_t n_tok,
                        const int32_t* token_idx, int32_t n_sel,
                        float* out, int32_t* topk_ids, float* topk_w, float* logits,
                        int32_t order);
void jxo_route(const jxo_moe_desc* L, const float* x, int32_t n_tok,
               float* logits, int32_t* topk_ids, float* topk_w);
void jxo_set_threads(int32_t n);

#ifdef __cplusplus
}
#endif
#endif

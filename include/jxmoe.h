/*
 * jxmoe -- MI355X (gfx950) MoE expert path behind a plain C ABI.
 *
 * The reference engine runs its MoE block inline in
 * MoETransformerEngine::forward_token (src/transformer.cpp:2584-2764) on top
 * of the math API in include/quant.h and the router selection in
 * include/tier.h.  This header is the boundary that replaces that block:
 * plain pointers and sizes, integer status codes, a thread-local error
 * string, no C++ types or exceptions across it.
 *
 * Ownership: weights are copied (and repacked) into device memory once by
 * jx_moe_layer_create; caller buffers are only borrowed for the duration of a
 * call.  One caller at a time per layer handle (its workspace is reused).
 */
#ifndef JXMOE_H
#define JXMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  Every entry point returns one; JX_OK == 0. */
enum {
    JX_OK = 0,
    JX_ERR_INVALID = 1,      /* bad argument / shape                          */
    JX_ERR_UNSUPPORTED = 2,  /* tensor type or shape the path does not cover  */
    JX_ERR_HIP = 3,          /* a HIP runtime call failed                     */
    JX_ERR_NOMEM = 4,        /* device allocation failed                      */
    JX_ERR_NODEVICE = 5      /* no gfx950 device / init not done              */
};

/* GGML tensor type codes, as GGMLType in include/common.h:45-77.  Expert and
 * qmatrix weights take the six block formats below; activations are Q8_0 where
 * supports_q8_activation allows (src/quant.cpp:3881-3893: Q4_0 / Q8_0 with
 * cols % 32 == 0, Q4_K / Q5_K / Q6_K with cols % 256 == 0), fp32 otherwise
 * (Q5_0 always), as the reference's dots. */
enum { JX_TYPE_F32 = 0, JX_TYPE_F16 = 1, JX_TYPE_Q4_0 = 2, JX_TYPE_Q5_0 = 6, JX_TYPE_Q8_0 = 8, JX_TYPE_Q4_K = 12,
       JX_TYPE_Q5_K = 13, JX_TYPE_Q6_K = 14, JX_TYPE_BF16 = 30 };

/* Gated activation of the expert FFN (hp_.use_gelu, src/transformer.cpp:1995,
 * passed to matmul_swiglu_quant_f32 at 2724; src/quant.cpp:3999-4007). */
enum { JX_ACT_SILU = 0, JX_ACT_GELU_TANH = 1 };

/* jx_moe_forward flags */
enum {
    JX_FWD_DEVICE_PTRS = 1u << 0, /* x, out, ids, weights, counts on the device  */
    JX_FWD_ASYNC = 1u << 1,       /* return after enqueueing (device ptrs only)   */
    JX_FWD_FORCE_GEMV = 1u << 2,  /* force the decode (dequant-GEMV) regime       */
    JX_FWD_FORCE_MFMA = 1u << 3,  /* force the prefill (matrix-core GEMM) regime  */
    JX_FWD_RESIDUAL = 1u << 4,    /* x is the residual stream before ffn_norm: the
                                     whole FFN step of forward_token (see below)   */
    JX_FWD_UNFUSED = 1u << 5,     /* one-token steps as separate router, gate/up and
                                     down launches instead of the single fused
                                     launch (same results).  Use it when kernels
                                     of other streams or processes may hold the
                                     GPU's CUs during the step (see below)          */
    JX_FWD_TEST_GIVEUP = 1u << 6  /* test hook, no counterpart in the reference: a
                                     fused one-token step's waits between its
                                     blocks give up after a few polls (every kernel
                                     still ends normally), to exercise the error
                                     reporting below; its outputs are invalid       */
};

/* One MoE layer, as bound by bind_tensors (src/transformer.cpp:2142-2186).
 * Expert tensors are the packed GGUF ffn_{gate,up,down}_exps blocks:
 * [n_experts][rows][ceil(cols/blk) blocks], expert e at e * bytes / n_experts.
 * gate/up rows = d_ff, cols = d_model; down rows = d_model, cols = d_ff. */
typedef struct jx_moe_layer_desc {
    int32_t n_experts;     /* E        (hp_.n_experts)                          */
    int32_t top_k;         /* k        (hp_.n_experts_used)                     */
    int32_t d_model;       /* d        (hp_.dim)                                */
    int32_t d_ff;          /* F        (hp_.moe_expert_dim)                     */
    int32_t gate_type, up_type, down_type;  /* JX_TYPE_Q*; gate == up      */
    const void* router;    /* [E][d] blk.L.ffn_gate_inp.weight, of router_type  */
    const float* router_bias; /* [E] fp32 added to the logits, or NULL          */
    const void* gate_exps;
    const void* up_exps;
    const void* down_exps;
    int32_t d_ff_shared;   /* 0 = no shared expert (ffn_*_shexp)                */
    int32_t sh_gate_type, sh_up_type, sh_down_type;
    const void* sh_gate;
    const void* sh_up;
    const void* sh_down;
    const float* sh_gate_inp; /* [d] fp32 ffn_gate_inp_shexp, or NULL (scale 1) */
    int32_t activation;    /* JX_ACT_SILU or JX_ACT_GELU_TANH (hp_.use_gelu)     */
    int32_t router_type;   /* type of `router`: JX_TYPE_F32, JX_TYPE_F16 or
                              JX_TYPE_BF16 (the reference routes through
                              matmul_quant_f32(lw.router_gate->type, ...),
                              transformer.cpp:2591: vec_dot_f32 for F32,
                              vec_dot_{f16,bf16}_f32's 8-lane order for the
                              others, quant.cpp:3015-3055); other types:
                              JX_ERR_UNSUPPORTED */
    /* The steps either side of the block, used with JX_FWD_RESIDUAL
     * (src/transformer.cpp:2585-2587, 2758-2764): */
    const float* ffn_norm;      /* [d] fp32 blk.L.ffn_norm, or NULL (weight 1)       */
    const float* post_ffw_norm; /* [d] fp32 blk.L.post_ffw_norm, or NULL (none)      */
    float rms_norm_eps;         /* hp_.rms_norm_eps (<arch>.attention.layer_norm_rms_epsilon) */
} jx_moe_layer_desc;

typedef struct jx_moe_layer jx_moe_layer;

/* Select and initialise a device.  Replaces nothing in the reference (its
 * "GPU" init, VulkanComputeBackend::init, src/vulkan_backend.cpp:64-156,
 * computes nothing).  Fails with JX_ERR_NODEVICE unless the device is gfx950. */
int jx_moe_init(int32_t device);

/* Upload + repack one layer's router and expert weights (replaces the
 * per-expert residency of LFRUTierManager::get_resident/admit_expert,
 * src/tier.cpp:41-122, and PILOT streaming, src/pilot_io.cpp:182-212: every
 * expert stays resident in HBM). */
int jx_moe_layer_create(const jx_moe_layer_desc* desc, jx_moe_layer** out);
void jx_moe_layer_destroy(jx_moe_layer* layer);

/* The MoE block for n_tok tokens (replaces src/transformer.cpp:2589-2757 for
 * one token at a time; tokens are independent, so a batch is the per-token
 * block applied to each row):
 *   x           [n_tok][d] fp32 post-ffn_norm activations
 *   out         [n_tok][d] fp32 moe_accum (the residual add stays with the caller)
 *   topk_ids    [n_tok][k] int32 selected experts, descending logit   (or NULL)
 *   topk_w      [n_tok][k] fp32 softmax weights over the k             (or NULL)
 *   expert_counts [E] int32 tokens routed to each expert              (or NULL)
 *   stream      hipStream_t (NULL = default stream)
 * With CACHE_ROUTE off, ids/order/counts are those of
 * select_experts_cache_aware (src/tier.cpp:124-198); exact logit ties are
 * ordered by expert index.
 * With JX_FWD_RESIDUAL, x is the residual stream and the call is the whole
 * FFN step of forward_token (src/transformer.cpp:2585-2764):
 *   x_norm = rms_norm(x, ffn_norm, eps)       (2585-2587; weight 1 when NULL)
 *   acc    = the MoE block on x_norm          (2589-2757)
 *   acc    = rms_norm(acc, post_ffw_norm, eps) if the layer has one (2758-2760)
 *   out    = x + acc                          (2762-2764; out may alias x) */
int jx_moe_forward(jx_moe_layer* layer, const float* x, int32_t n_tok, float* out, int32_t* topk_ids,
                   float* topk_w, int32_t* expert_counts, void* stream, uint32_t flags);
/* One-token steps may run as one launch whose blocks hand data to one another
 * (router rows -> gate/up -> down), which needs the launch's blocks resident
 * together.  A kernel of another stream or process that holds CUs meanwhile
 * delays the step; past a bound (2^18 polls, about a second) a wait gives up
 * and that step's outputs are invalid.  The synchronous call then returns
 * JX_ERR_HIP.  For an asynchronous call (JX_FWD_ASYNC) the failure is reported
 * by jx_moe_layer_status, and by the layer's next jx_moe_forward, which then
 * returns JX_ERR_HIP without doing any work; later calls run normally.
 * JX_FWD_UNFUSED keeps the separate launches, which have no such window.
 *
 * jx_moe_layer_status: JX_OK, or JX_ERR_HIP if a fused step of this layer gave
 * up a wait since the last report (the report clears it).  wait != 0 first
 * synchronizes the stream of the layer's last forward.  No counterpart in the
 * reference (its MoE block runs synchronously on the CPU). */
int jx_moe_layer_status(jx_moe_layer* layer, int32_t wait);

/* Router logits of the last forward, [n_tok][E] fp32, copied to host memory
 * (the reference's router_logits vector, src/transformer.cpp:2589-2594). */
int jx_moe_last_logits(jx_moe_layer* layer, float* logits_host, int32_t n_tok);

/* Q8_0 blocks of the last forward's activations as the router kernels wrote
 * them, [n_tok][d_model / 32] blocks of 34 bytes (fp16 d, 32 int8) in host
 * memory: the x_q8 vector matmul_swiglu_quant_f32 builds with
 * quantize_row_q8_0 (src/quant.cpp:3984-3992, 1029-1045). */
int jx_moe_last_xq8(jx_moe_layer* layer, void* blocks_host, int32_t n_tok);

/* Per-kernel-class device time of the forwards run since profiling was
 * enabled, measured with HIP events on the forward's stream.  names is a
 * ';'-separated list written into names_buf. */
int jx_moe_profile(jx_moe_layer* layer, int32_t enable);
int jx_moe_profile_read(jx_moe_layer* layer, char* names_buf, size_t names_len, double* ms, int64_t* launches,
                        int32_t max_entries, int32_t* n_entries);

/* ---- math-API drop-ins over a persistent device matrix ------------------ */

/* A single quantized weight matrix [rows][cols] in GGUF block layout, uploaded
 * and repacked once (the device counterpart of a mapped TensorDescriptor). */
typedef struct jx_qmatrix jx_qmatrix;
int jx_qmatrix_create(int32_t type, int64_t rows, int64_t cols, const void* host_blocks, jx_qmatrix** out);
void jx_qmatrix_destroy(jx_qmatrix* m);

/* out[r] = W[r] . x  (matmul_quant_f32, include/quant.h:336-343;
 * src/quant.cpp:3895-3922): Q8_0 activations under the reference's rule
 * (rows >= 8 and supports_q8_activation), fp32 otherwise.  Host pointers. */
int jx_matmul_quant_f32(jx_qmatrix* W, const float* x, float* out);

/* jx_matmul_quant_f32 on device pointers that allocates nothing.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  x_dev [cols] and out_dev [rows] are device fp32; the
 * work is enqueued on `stream` (hipStream_t, NULL = default stream) and the
 * call returns without synchronizing.  The activation scratch (Q8_0 form or
 * zero-padded fp32 copy) is one static device buffer per GPU holding at most
 * JX_NOALLOC_MAX_COLS columns (cols rounded up to 256); wider matrices are
 * refused with JX_ERR_UNSUPPORTED.  Every call on a GPU shares that buffer:
 * calls that overlap on one GPU (other streams, other threads) race on it.
 * Needs jx_moe_init on the matrix's device. */
#define JX_NOALLOC_MAX_COLS 65536
int jx_matmul_quant_f32_noalloc(jx_qmatrix* W, const float* x_dev, float* out_dev, void* stream);

/* out[r] = act(Wg[r] . x) * (Wu[r] . x), act = SiLU or (use_gelu) GELU-tanh
 * (matmul_swiglu_quant_f32, include/quant.h:354-362; src/quant.cpp:3970-4009).
 * Host pointers. */
int jx_matmul_swiglu_quant_f32(jx_qmatrix* Wg, jx_qmatrix* Wu, const float* x, float* out, int32_t use_gelu);

/* Device-pointer forms of the dense projections, enqueued on `stream`
 * (hipStream_t; returns without synchronizing), no per-call allocation: each
 * matrix holds a workspace for one activation row, allocated by
 * jx_qmatrix_create, so calls on one matrix (or one q/k/v set, whose first
 * matrix's workspace is used) must not overlap.
 *   jx_matmul_quant_f32_dev:     matmul_quant_f32 (src/quant.cpp:3895-3922)
 *   jx_matmul_qkv_quant_f32_dev: matmul_qkv_quant_f32 (src/quant.cpp:3924-3968):
 *     x quantized once when the given matrices hold >= 8 rows together; any of
 *     Wq, Wk, Wv may be NULL; they share cols. */
int jx_matmul_quant_f32_dev(jx_qmatrix* W, const float* x_dev, float* out_dev, void* stream);
int jx_matmul_qkv_quant_f32_dev(jx_qmatrix* Wq, jx_qmatrix* Wk, jx_qmatrix* Wv, const float* x_dev, float* q_dev,
                                float* k_dev, float* v_dev, void* stream);

/* quantize_row_q8_0 (include/quant.h:112; src/quant.cpp:1029-1045) on the
 * device: x [k] fp32 -> k/32 blocks of 34 bytes (fp16 d + 32 int8).  Host pointers. */
int jx_quantize_row_q8_0(const float* x, void* blocks, int64_t k);

/* ---- GGUF model files (host only) ---------------------------------------- */

/* A GGUF v2/v3 file mapped read-only and parsed: header, metadata, tensor table
 * (ModelFile::open / parse_gguf, src/gguf.cpp:810-889), every read bounds-checked;
 * each tensor must lie inside the file.  Errors: jx_gguf_last_error(). */
typedef struct jx_gguf jx_gguf;
int jx_gguf_open(const char* path, jx_gguf** out);
void jx_gguf_close(jx_gguf* g);
int64_t jx_gguf_tensor_count(const jx_gguf* g);
/* index of a tensor by name (ModelFile::find_tensor, include/gguf.h:73), -1 if absent */
int64_t jx_gguf_find_tensor(const jx_gguf* g, const char* name);
/* name, GGML type, dims (4 entries, 1-padded), absolute file offset, whole-tensor
 * bytes (tensor_byte_size, include/common.h:191-195) and mapped bytes of tensor i
 * (TensorDescriptor, include/gguf.h:36-46); outputs may be NULL */
int jx_gguf_tensor_info(const jx_gguf* g, int64_t i, const char** name, int32_t* type, int32_t* n_dims, uint64_t* dims,
                        uint64_t* file_offset, uint64_t* nbytes, const void** data);
/* metadata as ModelFile::get_u32 / get_f32 / get_str read it (src/gguf.cpp:1629-1642):
 * `def` when the key is absent; get_str gives NULL for absent or non-string keys */
int jx_gguf_get_u32(const jx_gguf* g, const char* key, uint32_t def, uint32_t* out);
int jx_gguf_get_f32(const jx_gguf* g, const char* key, float def, float* out);
int jx_gguf_get_str(const jx_gguf* g, const char* key, const char** out);
/* The MoE tensors of layer `layer` bound as bind_tensors binds them
 * (src/transformer.cpp:1954-1972, 2116-2199): router blk.L.ffn_gate_inp, the
 * packed ffn_{gate,up,down}_exps (n_experts and d_ff from their dims, top_k from
 * <arch>.expert_used_count), the shared expert ffn_*_shexp with
 * ffn_gate_inp_shexp, GELU-tanh for the gemma family; a dense FFN
 * (ffn_{gate,up,down}.weight) binds as one expert at top-1.  The pointers point
 * into the mapping: valid until jx_gguf_close; pass the desc to
 * jx_moe_layer_create, which copies the bytes to HBM. */
int jx_gguf_moe_layer_desc(jx_gguf* g, int32_t layer, jx_moe_layer_desc* desc);
const char* jx_gguf_last_error(void);

/* ---- host telemetry (no device work) ------------------------------------- */

/* The counter side effects of select_experts_cache_aware (src/tier.cpp:186-194)
 * replayed from a batch the GPU routed: tokens in order, token t at step
 * first_step + t (step_tick runs once per token, src/transformer.cpp:2371),
 * and for each selection s of token t, in rank order, with e = topk_ids[t][s]:
 *   activation_counts[layer * n_experts + e] += 1
 *   last_step        [layer * n_experts + e]  = first_step + t
 *   last_prob        [layer * n_experts + e]  = topk_w[t][s]
 * The tables are the caller's (LFRUTierManager's activation_counts_,
 * last_step_, last_prob_), table_len entries each; entries past table_len are
 * skipped as the reference skips them. */
int jx_tier_record(uint32_t layer, uint32_t n_experts, const int32_t* topk_ids, const float* topk_w, int32_t n_tok,
                   int32_t top_k, uint32_t first_step, uint32_t* activation_counts, uint32_t* last_step,
                   float* last_prob, size_t table_len);

/* LFRU score of one expert as snapshot_telemetry reports it (src/tier.cpp:233-263
 * with compute_lfru_score, 32-34): activations * 256 + recency, recency =
 * 255 - (current_step - last_step), 0 when that age reaches 255 or the expert
 * never ran (last_step 0). */
uint32_t jx_tier_lfru_score(uint32_t activations, uint32_t last_step, uint32_t current_step);

/* ---- device buffers (plumbing for callers without their own allocator) -- */
int jx_dev_alloc(size_t bytes, void** ptr);
int jx_dev_free(void* ptr);
int jx_memcpy_htod(void* dst, const void* src, size_t bytes);
int jx_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int jx_device_synchronize(void);

/* Identity of the loaded build: the first 16 hex digits of the SHA-256 over
 * the library's sources and this header, fixed at compile time.  Measurements
 * recorded with one build carry it.  No counterpart in the reference. */
const char* jx_build_id(void);

/* Last error message of the calling thread ("" if none). */
const char* jx_moe_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* JXMOE_H */

// Host-side expert telemetry fed from the GPU routing (no device code).
//
// The reference keeps per-(layer, expert) counters inside LFRUTierManager and
// updates them as a side effect of select_experts_cache_aware
// (src/tier.cpp:186-194): for every selected expert, activation_counts_ += 1,
// last_step_ = the current step and last_prob_ = its softmax weight, where the
// step advances once per token (step_tick in forward_token,
// src/transformer.cpp:2371).  /experts (src/server.cpp:1233-1261) reports
// them through snapshot_telemetry (src/tier.cpp:233-263) with the LFRU score
// frequency * 256 + min(255, recency) (src/tier.cpp:32-34).  With the MoE
// block on the GPU the selection no longer runs on the host, so these entry
// points replay its side effects from the batch's topk_ids / topk_w.
#include <cstddef>
#include <cstdint>

#include "../../include/jxmoe.h"

extern "C" {

int jx_tier_record(uint32_t layer, uint32_t n_experts, const int32_t* topk_ids, const float* topk_w, int32_t n_tok,
                   int32_t top_k, uint32_t first_step, uint32_t* activation_counts, uint32_t* last_step,
                   float* last_prob, size_t table_len) {
    if (!topk_ids || !topk_w || !activation_counts || !last_step || !last_prob) return JX_ERR_INVALID;
    if (n_tok < 0 || top_k < 1 || n_experts == 0) return JX_ERR_INVALID;
    const size_t base = (size_t)layer * n_experts;
    // tokens in order (the reference routes them one forward_token at a time), selections in rank order
    for (int32_t t = 0; t < n_tok; ++t) {
        const uint32_t step = first_step + (uint32_t)t;
        for (int32_t s = 0; s < top_k; ++s) {
            const int32_t e = topk_ids[(size_t)t * top_k + s];
            if (e < 0 || (uint32_t)e >= n_experts) return JX_ERR_INVALID;
            const size_t flat = base + (uint32_t)e;
            if (flat >= table_len) continue;  // as the reference: rows past its table are not counted
            activation_counts[flat]++;
            last_step[flat] = step;
            last_prob[flat] = topk_w[(size_t)t * top_k + s];
        }
    }
    return JX_OK;
}

uint32_t jx_tier_lfru_score(uint32_t activations, uint32_t last_step, uint32_t current_step) {
    // snapshot_telemetry's recency: 255 - age, 0 once the age reaches 255 or the expert never ran
    const uint32_t age = (current_step >= last_step && last_step > 0) ? (current_step - last_step) : 255u;
    const uint32_t recency = age >= 255u ? 0u : 255u - age;
    return activations * 256u + (recency < 255u ? recency : 255u);
}

}  // extern "C"

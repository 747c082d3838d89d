"""Host-side expert telemetry fed from the GPU routing.

Mirrors the counters LFRUTierManager keeps (src/tier.cpp:186-194) and the
snapshot /experts serves (src/tier.cpp:233-263, src/server.cpp:1233-1261):
per (layer, expert) the activation count, the step of the last selection, its
softmax weight, and the LFRU score.  The reference updates them inside
select_experts_cache_aware, one token per forward_token with step_tick first
(src/transformer.cpp:2371); here the library's jx_tier_record replays those
side effects from a batch's topk_ids / topk_w.  Every expert is resident in
HBM, so each reports the VRAM tier, unpinned.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import check, lib


class ExpertTelemetry:
    def __init__(self, n_layers: int, n_experts: int):
        self.n_layers, self.n_experts = int(n_layers), int(n_experts)
        m = self.n_layers * self.n_experts
        self.activation_counts = np.zeros(m, np.uint32)
        self.last_step = np.zeros(m, np.uint32)
        self.last_prob = np.zeros(m, np.float32)
        self.current_step = 1  # LFRUTierManager::current_step_ starts at 1 (include/tier.h:113)

    def step_tick(self, n: int = 1) -> None:
        self.current_step += int(n)

    def record(self, layer: int, topk_ids: np.ndarray, topk_w: np.ndarray) -> None:
        """The selections of n tokens routed in one batch, as n forward_token steps of the reference:
        the step advances once per token (the first token at current_step + 1)."""
        ids = np.ascontiguousarray(topk_ids, np.int32)
        w = np.ascontiguousarray(topk_w, np.float32)
        n, k = ids.shape
        P = lambda a: C.c_void_p(a.ctypes.data)  # noqa: E731
        check(lib().jx_tier_record(layer, self.n_experts, P(ids), P(w), n, k, self.current_step + 1,
                                   P(self.activation_counts), P(self.last_step), P(self.last_prob),
                                   self.activation_counts.size), "jx_tier_record")
        self.current_step += n

    def snapshot(self) -> list[dict]:
        """The /experts entries: layer, expert, activations, lfru_score, tier, pinned, last_prob."""
        out = []
        for l in range(self.n_layers):
            for e in range(self.n_experts):
                f = l * self.n_experts + e
                act = int(self.activation_counts[f])
                out.append({"layer": l, "expert": e, "activations": act,
                            "lfru_score": int(lib().jx_tier_lfru_score(act, int(self.last_step[f]), self.current_step)),
                            "tier": "VRAM", "pinned": False, "last_prob": float(self.last_prob[f])})
        return out

"""MoE-layer benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Default workload: the Mixtral-8x7B-shaped Q4_K MoE layer (d_model 4096,
8 experts, top-2, d_ff 14336).  A step is one pass of the MoE block over one
batch of seeded synthetic activations already resident in HBM:
  * prefill: 2048 tokens (matrix-core regime)     -> `value` (tokens/s)
  * decode : 1 token (dequant-GEMV regime)         -> the `decode` object
Both lines report the roofline of their dominant kernel from HIP events
recorded around every launch (a second pass of the same steps).  The prefill
GEMMs run v_mfma_f32_32x32x16_f16 on exact integer-valued operands (Q4_K
gate/up: sc*q in A, the Q8_0 quants q in B, the accumulator rescaled per
32-block into the activation scale's units; Q4_0/Q8_0 gate/up: dx*q split into
exact fp16 hi + lo in B), so their roofline peak is the fp16 one; the fraction
of the int8 peak the north star names, and of the fp16 peak counting the
MFMAs actually issued, are reported beside it.  The reference's CPU
path (its own quant.cpp/tier.cpp built in oracle/_ref, AVX2 dot order) is
timed on a bounded sample of the same workload on the host cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from jxai_amd import formats as F  # noqa: E402
from jxai_amd import synth  # noqa: E402

METRIC = "MoE-layer tok/s (1 GPU); decode HBM GB/s % peak; prefill int8 MFMA % peak"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
FP16_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "mixtral_layer_traffic.json")


def measured_traffic(role, tokens):
    """HBM bytes per launch of the kernel timed as `role` (gateup_mfma, down_mfma, gateup_gemv,
    down_gemv) at `tokens` tokens from the rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE in
    KiB per dispatch, each scaled by what the counter reads for a plain device copy of known size),
    or None when no summary covers it."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    k = t.get("kernels", {}).get(f"{role}@{tokens}")
    if not k:
        return None
    return 1024.0 * (k["fetch_kib"] * t["fetch_scale"] + k["write_kib"] * t["write_scale"])


def copy_calibration():
    """A plain device copy of 256 MiB, three times: the reference reading for the TCC byte counters."""
    import torch
    nbytes = 256 << 20
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(f"[bench] copied {nbytes} bytes x3", file=sys.stderr, flush=True)


def issued_per_algorithmic(cfg):
    """Matrix-core flops the gate/up GEMM issues per algorithmic flop: Q4_K one fp16 MFMA per
    16 of K plus the min term's three per 256 of K (19 / 16); Q4_0 / Q8_0 hi and lo (2)."""
    return 19 / 16 if cfg.wtype == F.Q4_K else 2.0


def algorithmic(cfg, n, counts):
    """Bytes and int8 ops of one layer pass (distinct routed experts from this run's counts)."""
    t = cfg.wtype
    d, Fd, E = cfg.d_model, cfg.d_ff, cfg.n_experts
    distinct = int((np.asarray(counts) > 0).sum())
    gu_bytes = 2 * F.matrix_bytes(t, Fd, d)
    dn_bytes = F.matrix_bytes(t, d, Fd)
    nbytes = distinct * (gu_bytes + dn_bytes) + synth.shared_bytes(cfg)
    nbytes += E * d * 4 + (d * 4 if cfg.shared_gate else 0) + n * d * 4 * 2
    ops = 2 * n * cfg.top_k * 3 * d * Fd + 2 * n * 3 * d * cfg.d_ff_shared
    return dict(bytes=nbytes, ops=ops, distinct=distinct, gateup_bytes=distinct * gu_bytes,
                gateup_ops=2 * n * cfg.top_k * 2 * d * Fd, down_bytes=distinct * dn_bytes)


def run_gpu(L, cfg, n, steps, warmup, regime):
    from jxai_amd import moe
    x = synth.make_tokens(cfg, n)
    xb = moe.DeviceBuffer(x.nbytes).upload(x)
    ob = moe.DeviceBuffer(x.nbytes)
    _, ids, w, counts = L.forward(x, regime=regime)  # routing of this batch (host copy)
    for _ in range(warmup):
        L.forward_device(xb, n, ob, sync=False, regime=regime)
    moe.lib().jx_device_synchronize()
    # timed region: the production path (captured graph replays), no per-launch events
    t0 = time.perf_counter()
    for _ in range(steps):
        L.forward_device(xb, n, ob, sync=False, regime=regime)
    moe.lib().jx_device_synchronize()
    t1 = time.perf_counter()
    # kernel durations: the same steps again with HIP events around every launch
    L.profile(True)
    for _ in range(steps):
        L.forward_device(xb, n, ob, sync=False, regime=regime)
    moe.lib().jx_device_synchronize()
    prof = L.profile_read()
    L.profile(False)
    xb.free()
    ob.free()
    return (t1 - t0) / steps, prof, counts


def cpu_baseline(lw, cfg, n, budget_s=12.0, max_tokens=None):
    """Reference CPU path (oracle/_ref) or the C restatement on a bounded token sample."""
    from oracle import oracle as O
    kind = "reference" if O.available("reference") else "port"
    o = O.Oracle(kind, avx512=False)
    x = synth.make_tokens(cfg, n)
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    o.moe_forward(lw, x, np.array([0], np.int32))  # warm-up (page-in, thread pool)
    done, t0 = 0, time.perf_counter()
    limit = max_tokens or n
    while done < limit and time.perf_counter() - t0 < budget_s:
        m = min(8, limit - done)
        o.moe_forward(lw, x, np.arange(done, done + m, dtype=np.int32))
        done += m
    dt = time.perf_counter() - t0
    return {"value": done / dt, "unit": "tok/s", "cores": cores, "kind": kind,
            "sample": f"first {done} of the {n} tokens through the MoE block, per-token path "
                      f"(the reference has no batched MoE), {dt:.1f} s, OMP threads {cores}, AVX2 dot order"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="mixtral")
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    ap.add_argument("--decode-tokens", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy (scale for the rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (experts would shard by "
              "expert parallelism, see DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from jxai_amd import moe
    cfg = synth.CONFIGS[args.config]
    print(f"[bench] generating {cfg.describe}", file=sys.stderr, flush=True)
    lw = synth.make_layer(cfg)
    moe.init(0)
    L = moe.MoELayer.from_weights(lw)

    n = args.prefill_tokens
    print(f"[bench] prefill {n} tokens", file=sys.stderr, flush=True)
    s_pre, prof_pre, counts_pre = run_gpu(L, cfg, n, args.steps, args.warmup, "mfma")
    a_pre = algorithmic(cfg, n, counts_pre)
    gu_ms, gu_n = prof_pre.get("gateup_mfma", (0.0, 1))
    gu_avg = gu_ms / max(gu_n, 1) / 1e3
    gu_rate = a_pre["gateup_ops"] / gu_avg / 1e12
    pre_roof = {"bound": "mfma", "kernel": "k_wgemm<Q4_K, gate+up> (fp16 matrix-core grouped GEMM + SwiGLU)",
                "achieved": gu_rate, "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": gu_rate / FP16_PEAK_TFLOPS,
                "traffic": measured_traffic("gateup_mfma", n),
                "avg_launch_us": gu_avg * 1e6,
                "int8_peak_frac": gu_rate / INT8_PEAK_TOPS,
                "issued_fp16_frac": issued_per_algorithmic(cfg) * gu_rate / FP16_PEAK_TFLOPS,
                "layer_int8_frac": a_pre["ops"] / s_pre / 1e12 / INT8_PEAK_TOPS}

    nd = args.decode_tokens
    print(f"[bench] decode {nd} token(s)", file=sys.stderr, flush=True)
    s_dec, prof_dec, counts_dec = run_gpu(L, cfg, nd, max(args.steps * 10, 50), args.warmup * 4, "gemv")
    a_dec = algorithmic(cfg, nd, counts_dec)
    dg_ms, dg_n = prof_dec.get("gateup_gemv", (0.0, 1))
    dg_avg = dg_ms / max(dg_n, 1) / 1e3
    dec_roof = {"bound": "hbm", "kernel": "k_gemv_gateup<Q4_K> (gate+up dequant-GEMV + SwiGLU)",
                "achieved": a_dec["gateup_bytes"] / dg_avg / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": a_dec["gateup_bytes"] / dg_avg / 1e9 / HBM_PEAK_GBS,
                "traffic": measured_traffic("gateup_gemv", nd),
                "avg_launch_us": dg_avg * 1e6,
                "layer_hbm_frac": a_dec["bytes"] / s_dec / 1e9 / HBM_PEAK_GBS}

    cpu = None
    if not args.no_cpu:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(lw, cfg, n)

    line = {
        "metric": METRIC,
        "value": n / s_pre,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": s_pre * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA on exact integer operands, f32 accumulate (decode: int8 dot, i32)",
        "data": "synthetic: seeded SplitMix64 Q4_K weights and N(0,1) activations of the layer shape",
        "config": {"workload": f"{cfg.describe}, prefill {n} tokens", "d_model": cfg.d_model,
                   "n_experts": cfg.n_experts, "top_k": cfg.top_k, "d_ff": cfg.d_ff,
                   "weights": F.NAMES[cfg.wtype], "tokens": n},
        "roofline": pre_roof,
        "cpu_baseline": cpu,
        "kernels_ms_per_step": {k: v[0] / args.steps for k, v in prof_pre.items()},
        "decode": {"value": nd / s_dec, "unit": "tok/s", "tokens": nd, "ms_per_step": s_dec * 1e3,
                   "roofline": dec_roof,
                   "kernels_us_per_step": {k: v[0] * 1e3 / max(args.steps * 10, 50) for k, v in prof_dec.items()}},
    }
    print(json.dumps(line), flush=True)
    L.close()


if __name__ == "__main__":
    main()

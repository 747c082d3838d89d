"""MoE-layer benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME] [--no-configs] [--no-cpu]

A step is one pass of the MoE block over one batch of seeded synthetic
activations already resident in HBM (weights uploaded beforehand, outside the
timed region).  Headline workload: the Mixtral-8x7B-shaped Q4_K MoE layer
(d_model 4096, 8 experts, top-2, d_ff 14336):
  * prefill: 2048 tokens (matrix-core regime)     -> `value` (tokens/s)
  * decode : 1 token (dequant-GEMV regime)         -> the `decode` object, with
    successive steps on distinct copies of the layer (as a model's layers follow
    one another) so that each step reads its experts from HBM; `decode_resident`
    is the same step repeated on one layer (its experts stay in the 256 MB
    last-level cache)
and `configs`, every configured layer shape at its token counts (few-token
points cycled over copies of the layer likewise), each with the algorithmic
bytes and int8 ops of the pass and their roofline fractions.

Timing: K steps back to back between two device synchronizations give `value`
and `ms_per_step` (nothing else is enqueued in that region: a timing event costs
the GPU 3-5 us); a second pass with one HIP event after each step on the
forward's stream gives the per-step median and p10/p90.  Before timing,
the device-pointer asynchronous path (the one timed) is checked bit for bit
against the host-pointer path.  Kernel durations for the rooflines come from a
second pass with HIP events around every launch.  The prefill roofline is the
fraction of the dense int8 peak (the path's products are int8 x int8 block
sums); the GEMMs run v_mfma_f32_32x32x16_f16 on exact integer-valued operands,
so the fraction of the fp16 peak is reported beside it.
The reference's CPU path (its own quant.cpp/tier.cpp built in oracle/_ref,
AVX2 dot order) is timed on a bounded token sample on the host cores.
"""
from __future__ import annotations

import argparse
import ctypes as C
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
DECODE_WARMUP = 300  # untimed few-token steps before a timed region (about 15 ms of decode)
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
FP16_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "mixtral_layer_traffic.json")

# every configured point: (config, tokens)
POINTS = [("toy", 1), ("qwen15moe", 1), ("qwen15moe", 64), ("mixtral", 1), ("mixtral", 512), ("mixtral", 2048),
          ("qwen3moe", 2048), ("dsv2lite", 32),
          # the mixed-format layers of Q4_K_M files (Q6_K down; Q5_0 routed down, Q6_K shared down)
          ("mixtral_q6k", 1), ("mixtral_q6k", 2048), ("dsv2lite_q50", 1), ("dsv2lite_q50", 32), ("dsv2lite_q50", 2048)]


class Hip:
    """Streams and timing events of the HIP runtime the library itself loaded (ctypes)."""

    def __init__(self):
        self.lib = C.CDLL("libamdhip64.so")
        for fn in ("hipStreamCreate", "hipEventCreate"):
            getattr(self.lib, fn).argtypes = [C.POINTER(C.c_void_p)]
        self.lib.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.lib.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.lib.hipStreamSynchronize.argtypes = [C.c_void_p]
        self.lib.hipEventDestroy.argtypes = [C.c_void_p]
        s = C.c_void_p()
        self._ok(self.lib.hipStreamCreate(C.byref(s)), "hipStreamCreate")
        self.stream = s.value

    @staticmethod
    def _ok(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {rc}")

    def events(self, n):
        evs = []
        for _ in range(n):
            e = C.c_void_p()
            self._ok(self.lib.hipEventCreate(C.byref(e)), "hipEventCreate")
            evs.append(e.value)
        return evs

    def record(self, ev):
        self._ok(self.lib.hipEventRecord(ev, self.stream), "hipEventRecord")

    def sync(self):
        self._ok(self.lib.hipStreamSynchronize(self.stream), "hipStreamSynchronize")

    def elapsed_ms(self, a, b):
        ms = C.c_float()
        self._ok(self.lib.hipEventElapsedTime(C.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def free(self, evs):
        for e in evs:
            self.lib.hipEventDestroy(e)


def measured_traffic(role, tokens):
    """(bytes, note): memory bytes per launch of the kernel timed as `role` (gateup_mfma, down_mfma,
    decode_fused_cu, ...) at `tokens` tokens from the rocprofv3 --pmc summary (the L2's read and write
    requests to memory times their sizes, exact on a plain device copy of known size), or None with the
    reason when no summary of the loaded build covers it.  The summary carries the jx_build_id() of the
    library it measured; a summary of another build is refused."""
    from jxai_amd._lib import lib
    build = lib().jx_build_id().decode()
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None, "no traffic summary"
    if t.get("build_id") != build:
        return None, f"stale: the traffic summary measured build {t.get('build_id')}, this is build {build}"
    k = t.get("kernels", {}).get(f"{role}@{tokens}")
    if not k:
        return None, f"the traffic summary has no {role}@{tokens}"
    return k["read_bytes"] + k["write_bytes"], f"rocprofv3 --pmc TCC_EA0 requests x size, build {build}"


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
    dn_bytes = F.matrix_bytes(cfg.down_t, d, Fd)
    nbytes = distinct * (gu_bytes + dn_bytes) + synth.shared_bytes(cfg)
    nbytes += E * d * 4 + (d * 4 if cfg.shared_gate else 0) + n * d * 4 * 2
    ops = 2 * n * cfg.top_k * 3 * d * Fd + 2 * n * 3 * d * cfg.d_ff_shared
    sh_gu = 2 * F.matrix_bytes(t, cfg.d_ff_shared, d) if cfg.d_ff_shared else 0
    return dict(bytes=nbytes, ops=ops, distinct=distinct, gateup_bytes=distinct * gu_bytes,
                gateup_ops=2 * n * cfg.top_k * 2 * d * Fd, down_bytes=distinct * dn_bytes,
                shared_gateup_bytes=sh_gu)


def pct(a, q):
    return float(np.percentile(np.asarray(a), q))


def run_gpu(hip, Ls, cfg, n, steps, warmup, regime=None):
    """A bit-exact check of the timed path, warm-up, K timed steps, a pass with one timing event per
    step (the per-step distribution), then a profiled pass.  Ls: one layer, or several copies of it
    (the same weights uploaded to distinct HBM) that step i runs as Ls[i % len(Ls)], as a model's
    layers follow one another: each step then reads its experts from HBM, not from the 256 MB
    last-level cache that holds a single layer's few-token working set across steps."""
    from jxai_amd import moe
    Ls = Ls if isinstance(Ls, (list, tuple)) else [Ls]
    x = synth.make_tokens(cfg, n)
    xb = moe.DeviceBuffer(x.nbytes).upload(x)
    ob = moe.DeviceBuffer(x.nbytes)
    want, ids, w, counts = Ls[0].forward(x, regime=regime)  # host-pointer path; routing of this batch
    for L in Ls:
        L.forward_device(xb, n, ob, sync=False, regime=regime, stream=hip.stream)
        hip.sync()
        got = ob.download(np.empty_like(x))
        if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
            raise SystemExit(f"bench: the timed device path differs from the host path ({cfg.name}, n={n})")

    def steps_of(k, after=None):
        for i in range(k):
            Ls[i % len(Ls)].forward_device(xb, n, ob, sync=False, regime=regime, stream=hip.stream)
            if after:
                after(i)

    # warm-up right before the timed region (the check above leaves the GPU idle for a while)
    steps_of(warmup)
    hip.sync()
    moe.lib().jx_device_synchronize()
    # timed region: K steps of the production path back to back between two device synchronizations,
    # nothing else in the stream (a timing event costs the GPU 3-5 us, a tenth of a decode step)
    t0 = time.perf_counter()
    steps_of(steps)
    hip.sync()
    moe.lib().jx_device_synchronize()
    t1 = time.perf_counter()
    # per-step distribution: the same steps with one timing event after each (step i = e[i] - e[i-1];
    # each interval includes one event's cost)
    evs = hip.events(steps + 1)
    hip.record(evs[0])
    steps_of(steps, lambda i: hip.record(evs[i + 1]))
    hip.sync()
    step_ms = [hip.elapsed_ms(evs[i], evs[i + 1]) for i in range(steps)]
    hip.free(evs)
    # kernel durations: the same steps again with HIP events around every launch
    for L in Ls:
        L.profile(True)
    steps_of(steps)
    hip.sync()
    prof = {}
    for L in Ls:
        for k, (ms, cnt) in L.profile_read().items():
            a = prof.setdefault(k, [0.0, 0])
            a[0] += ms
            a[1] += cnt
        L.profile(False)
    prof = {k: tuple(v) for k, v in prof.items()}
    # each layer's fused one-token steps completed every wait (asynchronous calls report it here)
    for L in Ls:
        L.status(wait=True)
    xb.free()
    ob.free()
    return dict(wall_s=(t1 - t0) / steps, step_ms=step_ms, prof=prof, counts=counts, copies=len(Ls))


CYCLE_BYTES = 1.2e9  # the copies a few-token point cycles through hold at least this many step bytes
MAX_COPIES = 16


def copies_for(cfg, n):
    """Copies of the layer a few-token point cycles through so that the bytes its steps read (cycled)
    exceed the last-level cache several times over: 1 where one step already reads more than
    CYCLE_BYTES, and for prefill batches (512 tokens and more), as for the headline prefill line."""
    if n >= 512:
        return 1
    per_expert = 2 * F.matrix_bytes(cfg.wtype, cfg.d_ff, cfg.d_model) + F.matrix_bytes(cfg.down_t, cfg.d_model,
                                                                                         cfg.d_ff)
    step = min(cfg.n_experts, n * cfg.top_k) * per_expert + synth.shared_bytes(cfg)
    return int(min(MAX_COPIES, max(1, -(-CYCLE_BYTES // step))))


def layer_copies(moe, lw, count):
    return [moe.MoELayer.from_weights(lw) for _ in range(count)]


def step_stats(r):
    """Per-step distribution (one timing event per step, included) beside the timed region's mean."""
    s = r["step_ms"]
    return {"median": float(np.median(s)), "p10": pct(s, 10), "p90": pct(s, 90), "mean_wall": r["wall_s"] * 1e3,
            "note": "median/p10/p90 from a second pass with one hipEvent per step (its cost, 3-5 us, included); "
                    "mean_wall = the timed region (K steps back to back between synchronizations) / K"}


def point_line(cfg, n, r):
    """tok/s, algorithmic work and roofline fractions of one configured point."""
    a = algorithmic(cfg, n, r["counts"])
    t = r["wall_s"]
    return {"tokens": n, "tok_s": n / t, "step_ms": step_stats(r), "layer_copies_cycled": r["copies"],
            "bytes": a["bytes"], "int8_ops": a["ops"],
            "distinct_experts": a["distinct"], "hbm_frac": a["bytes"] / t / 1e9 / HBM_PEAK_GBS,
            "int8_frac": a["ops"] / t / 1e12 / INT8_PEAK_TOPS,
            "roofline_frac": max(a["bytes"] / (HBM_PEAK_GBS * 1e9), a["ops"] / (INT8_PEAK_TOPS * 1e12)) / t,
            "kernels_us": {k: v[0] * 1e3 / max(v[1], 1) for k, v in r["prof"].items()}}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(lw, cfg, n, sample=512, runs=3):
    """Reference CPU path (oracle/_ref) or the C restatement: one warm-up, then the median of `runs`
    timings of the same contiguous token sample (the reference has no batched MoE: per token)."""
    from oracle import oracle as O
    kind = "reference" if O.available("reference") else "port"
    o = O.Oracle(kind, avx512=False)
    x = synth.make_tokens(cfg, n)
    affinity = len(os.sched_getaffinity(0))
    threads = int(os.environ.get("OMP_NUM_THREADS", affinity))
    cores = min(threads, affinity)
    m = min(sample, n)
    sel = np.arange(m, dtype=np.int32)
    o.moe_forward(lw, x, np.array([0], np.int32))  # warm-up (page-in, thread pool)
    rates = []
    for _ in range(runs):
        t0 = time.perf_counter()
        o.moe_forward(lw, x, sel)
        rates.append(m / (time.perf_counter() - t0))
    scaled = "" if m == n else f", scaled: the first {m} of the {n} tokens"
    return {"value": float(np.median(rates)), "unit": "tok/s", "cores": cores, "kind": kind,
            "cpu_model": cpu_model(), "affinity_cpus": affinity, "runs_tok_s": rates,
            "sample": f"median of {runs} runs over tokens 0..{m - 1} of the {n}-token batch through the MoE "
                      f"block, per-token path{scaled}; AVX2 dot order, OpenMP threads {cores}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="mixtral")
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    ap.add_argument("--decode-tokens", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config object")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy (scale for the rocprofv3 byte counters)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: there is no multi-GPU path (the experts would shard by expert "
              "parallelism, whole experts per GPU); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    steps = max(args.steps, 1)

    from jxai_amd import moe
    cfg = synth.CONFIGS[args.config]
    print(f"[bench] generating {cfg.describe}", file=sys.stderr, flush=True)
    lw = synth.make_layer(cfg)
    moe.init(0)
    hip = Hip()
    L = moe.MoELayer.from_weights(lw)

    n = args.prefill_tokens
    print(f"[bench] prefill {n} tokens", file=sys.stderr, flush=True)
    r_pre = run_gpu(hip, L, cfg, n, steps, args.warmup, "mfma")
    s_pre = r_pre["wall_s"]
    a_pre = algorithmic(cfg, n, r_pre["counts"])
    gu_ms, gu_n = r_pre["prof"].get("gateup_mfma", (0.0, 1))
    gu_avg = gu_ms / max(gu_n, 1) / 1e3
    gu_rate = a_pre["gateup_ops"] / gu_avg / 1e12
    traffic, traffic_note = measured_traffic("gateup_mfma", n)
    # the fraction of the int8 peak (the path's arithmetic is int8 x int8 block sums); the GEMM issues
    # v_mfma_f32_32x32x16_f16 on exact integer-valued operands, so its fraction of the fp16 peak and of
    # the issued matrix-core work are reported beside it
    pre_roof = {"bound": "mfma", "kernel": "k_wgemm<Q4_K, gate+up> (fp16 matrix-core grouped GEMM + SwiGLU)",
                "achieved": gu_rate, "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                "ops": "algorithmic int8 ops (2 per multiply-accumulate, 2*n*k*2*d*F per launch) per second in "
                       "units of 1e12, against the dense int8 peak of 5.0 POP/s",
                "frac": gu_rate / INT8_PEAK_TOPS,
                "traffic": traffic, "traffic_note": traffic_note,
                "avg_launch_us": gu_avg * 1e6,
                "fp16_peak_frac": gu_rate / FP16_PEAK_TFLOPS,
                "issued_fp16_frac": issued_per_algorithmic(cfg) * gu_rate / FP16_PEAK_TFLOPS,
                "layer_int8_frac": a_pre["ops"] / s_pre / 1e12 / INT8_PEAK_TOPS}

    nd = args.decode_tokens
    dsteps = max(steps * 10, 50)
    dwarm = max(args.warmup * 4, DECODE_WARMUP)

    def decode_line(r, label):
        s_dec = r["wall_s"]
        a_dec = algorithmic(cfg, nd, r["counts"])
        # the dominant decode kernel: the one-launch step where the layer takes it (all of the layer's
        # bytes), else the gate/up GEMV (the gate and up matrices of the selected experts, and of the
        # shared expert where its blocks join the launch: gateup_gemv_shared)
        # (decode_fused_y: the one-launch step writing y for a separate combine, top-k above 2)
        fused = next((kk for kk in ("decode_fused_cu", "decode_fused", "decode_fused_y") if kk in r["prof"]), None)
        role = fused or ("gateup_gemv_shared" if "gateup_gemv_shared" in r["prof"] else "gateup_gemv")
        if role not in r["prof"]:
            raise RuntimeError(f"decode: no {role} launch among the profiled kernels {sorted(r['prof'])}")
        dg_ms, dg_n = r["prof"][role]
        dg_avg = dg_ms / max(dg_n, 1) / 1e3
        dbytes = (a_dec["bytes"] if fused else
                  a_dec["gateup_bytes"] + (a_dec["shared_gateup_bytes"] if role == "gateup_gemv_shared" else 0))
        dec_med = float(np.median(r["step_ms"])) / 1e3
        tr, tr_note = measured_traffic(role, nd)
        roof = {"bound": "hbm",
                "kernel": ("k_decode_p (the whole one-token step, one block per CU)" if fused == "decode_fused_cu"
                           else "k_decode1 (the whole one-token step)" if fused
                           else "k_gemv_mxt (routed and shared gate+up GEMV + SwiGLU, one launch)"
                           if role == "gateup_gemv_shared" else "k_gemv_gateup (gate+up dequant-GEMV + SwiGLU)"),
                "achieved": dbytes / dg_avg / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": dbytes / dg_avg / 1e9 / HBM_PEAK_GBS,
                "traffic": tr, "traffic_note": tr_note,
                "avg_launch_us": dg_avg * 1e6,
                "layer_hbm_frac": a_dec["bytes"] / s_dec / 1e9 / HBM_PEAK_GBS,
                "layer_hbm_frac_median_step": a_dec["bytes"] / dec_med / 1e9 / HBM_PEAK_GBS}
        return {"value": nd / s_dec, "unit": "tok/s", "tokens": nd, "ms_per_step": s_dec * 1e3,
                "layer_copies_cycled": r["copies"], "weights_from": label,
                "step_ms": step_stats(r), "roofline": roof,
                "kernels_us_per_step": {k: v[0] * 1e3 / dsteps for k, v in r["prof"].items()}}

    # decode as a model runs it: successive steps on distinct copies of the layer, so every step reads
    # its two experts from HBM (copies_for), then on one layer (its experts stay in the last-level cache)
    ncop = copies_for(cfg, nd)
    print(f"[bench] decode {nd} token(s), {ncop} copies of the layer in turn", file=sys.stderr, flush=True)
    extra = layer_copies(moe, lw, ncop - 1)
    r_cyc = run_gpu(hip, [L] + extra, cfg, nd, dsteps, dwarm, "gemv")
    for Lc in extra:
        Lc.close()
    del extra
    print(f"[bench] decode {nd} token(s), one layer", file=sys.stderr, flush=True)
    # the untimed warm-up runs DECODE_WARMUP steps: decode steps run ~5% slower over the first few
    # hundred after the prefill (clock and cache warm-up)
    r_res = run_gpu(hip, L, cfg, nd, dsteps, dwarm, "gemv")
    decode = decode_line(r_cyc, f"HBM: {ncop} copies of the layer, one per step in turn")
    decode_res = decode_line(r_res, "one layer: its two experts stay in the 256 MB last-level cache across steps")

    cpu = None
    if not args.no_cpu:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(lw, cfg, n)
    L.close()

    configs = None
    if not args.no_configs:
        configs = {}
        cur = None
        for name, tok in POINTS:
            if cur is None or cur[0] != name:
                if cur is not None:
                    for Lc in cur[3]:
                        Lc.close()
                c = synth.CONFIGS[name]
                print(f"[bench] configs: {c.describe}", file=sys.stderr, flush=True)
                lwc = synth.make_layer(c)
                cur = (name, c, lwc, [moe.MoELayer.from_weights(lwc)])
            _, c, lwc, Lcs = cur
            ncp = copies_for(c, tok)
            if len(Lcs) < ncp:
                Lcs.extend(layer_copies(moe, lwc, ncp - len(Lcs)))
            print(f"[bench] configs: {name} @ {tok} ({ncp} copies in turn)", file=sys.stderr, flush=True)
            reps = steps if tok >= 512 else max(steps * 5, 50)
            r = run_gpu(hip, Lcs[:ncp], c, tok, reps,
                        args.warmup if tok >= 512 else max(args.warmup, DECODE_WARMUP))
            configs[f"{name}@{tok}"] = point_line(c, tok, r)
        if cur is not None:
            for Lc in cur[3]:
                Lc.close()
    del lw

    line = {
        "metric": METRIC,
        "value": n / s_pre,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps,
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
        "step_ms": step_stats(r_pre),
        "timed_path_check": "device-pointer async path == host path, bit for bit (every measured point, every "
                            "layer copy); jx_moe_layer_status clean after every pass",
        "roofline": pre_roof,
        "cpu_baseline": cpu,
        "kernels_ms_per_step": {k: v[0] / steps for k, v in r_pre["prof"].items()},
        "decode": decode,
        "decode_resident": decode_res,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

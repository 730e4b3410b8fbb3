"""Benchmark of the MoE FFN block on one MI355X.

Default workload: Qwen3.6-35B-A3B-shape MoE layer (hidden 2048, 256 experts
top-8, shared expert, intermediate 512, 4-bit group-32 weights), batch-1
decode: every step is one token's full MoE block (router, 8 routed experts,
shared expert, combine) with a fresh activation, launched in sequence.
Inputs are resident in HBM before the timed region.  Prints one JSON line.

  python bench.py [--steps K] [--warmup W] [--workload decode|toy|stack|gguf]
                  [--cpu-sample-s S] [--no-cpu]

--workload gguf: one layer's routed expert projection in the reference's GGUF
format (256 experts x 2048 x 512 weights, --gguf-type q3_k|q4_k|q8_0)
dequantized to fp32 in HBM, the work src/layers/gguf_port_loader.mojo:217-236
repeats for every layer of every token.

--workload gguf-moe: batch-1 decode of one Qwen3.6-shape MoE layer read from a
GGUF file (Q8_0 router, 256 Q3_K experts and a Q3_K shared expert, written
to TMPDIR with random payloads): the MoE section of forward_port_block with
the experts kept in their GGUF blocks in HBM.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "disk-streaming-moe-engine_amd"))

METRIC = "MoE-layer decode µs/token + achieved HBM GB/s (4-bit, batch 1, 1 GPU)"
HBM_PEAK_GBPS = 8000.0
# HBM bytes per launch of the decode kernel from the rocprofv3 FETCH_SIZE and
# WRITE_SIZE runs (scaled by a copy-kernel calibration) recorded in this file
TRAFFIC_PROFILE = os.path.join("profiles", "k_moe_decode_qwen36_layer_decode.md")
GGUF_PROFILE = os.path.join("profiles", "k_dequant_gguf_q3k_expert_layer.md")
GGUF_MOE_PROFILE = os.path.join("profiles", "gguf_moe_q3k_layer_decode.md")


def f10_metrics(ref, cand):
    """The reference's F10 comparison of a candidate output against a
    reference output (tools/dismoen-tools/src/compare.rs:648-700): delta_max =
    max |c - r|, epsilon_rel = sqrt(sum (c - r)^2 / sum r^2), cos_theta =
    r.c / (|r| |c|), in float64; and the G-M3-1 gate of the MoE-layer
    comparison (compare.rs:1041-1043): delta_max <= 1e-3 and
    epsilon_rel <= 1e-4."""
    import numpy as np
    r = np.asarray(ref, dtype=np.float64).reshape(-1)
    c = np.asarray(cand, dtype=np.float64).reshape(-1)
    if r.size != c.size or r.size == 0 or not (np.isfinite(r).all() and np.isfinite(c).all()):
        return {"error": "size mismatch, empty or non-finite"}
    d = np.abs(c - r)
    sr, sc = float(np.sum(r * r)), float(np.sum(c * c))
    eps = float(np.sqrt(np.sum(d * d) / sr)) if sr > 0 else 0.0
    nrm = np.sqrt(sr) * np.sqrt(sc)
    cos = float(np.dot(r, c) / nrm) if nrm > 0 else 0.0
    dmax = float(d.max())
    return {"delta_max": dmax, "epsilon_rel": eps, "cos_theta": cos,
            "g_m3_1_pass": bool(dmax <= 1e-3 and eps <= 1e-4)}


def profiled_traffic(profile=TRAFFIC_PROFILE, key="traffic_bytes_per_launch"):
    try:
        with open(os.path.join(ROOT, profile)) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "toy", "stack", "batch", "prefill", "copy", "gguf",
                             "gguf-moe"],
                    help="batch: --batch tokens per call (ragged small-batch decode); "
                         "prefill: --tokens per call with Zipf-skewed routing; "
                         "copy: a plain device copy of --copy-mib MiB, the calibration "
                         "kernel for HBM byte counters")
    ap.add_argument("--batch", type=int, default=32, help="tokens per call, batch workload")
    ap.add_argument("--tokens", type=int, default=2048, help="tokens per call, prefill workload")
    ap.add_argument("--zipf-s", type=float, default=1.1, help="prefill router skew exponent")
    ap.add_argument("--activations", default="bf16", choices=["bf16", "fp32"],
                    help="batch / prefill inputs: bf16 values, or fp32 values that are not "
                         "(hi and lo bf16 parts on the matrix cores, lane-chain router)")
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--layers", type=int, default=40, help="stack workload depth")
    ap.add_argument("--stack-norm", default="ref", choices=["ref", "tree"],
                    help="stack workload: the RMSNorm's sum of squares in the reference's "
                         "element order (ref) or as a 256-partial tree (tree)")
    ap.add_argument("--gguf-type", default="q3_k", choices=["q3_k", "q4_k", "q8_0"])
    ap.add_argument("--gguf-tokens", type=int, default=1,
                    help="tokens per call, gguf-moe workload (> 1: the grouped form)")
    ap.add_argument("--cpu-sample-s", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=1)
    return ap.parse_args()


def cpu_info():
    """Host cores this process may use and the CPU model name."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count()
    return n, model


def cpu_baseline(L, x_tokens, budget_s):
    """The oracle (CPU restatement of the reference composition) on bounded
    token samples of the same layer, in the reference's four CPU modes:
    threads=1 (its verdict mode) and threads=min(K, cores) through the
    worker-pool partition of parallel_moe_experts (router and shared expert
    serial), each with per-use dequantization of the selected experts (the
    reference's quant_loader) and with every expert pre-dequantized to fp32
    (a compute-only bound).  value: threads=1, dequant-per-use."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    ncores, model = cpu_info()
    nthr = max(1, min(L.top_k, ncores))

    def timed(budget, pool=None, cache=None):
        n, t0 = 0, time.perf_counter()
        while n < len(x_tokens) and (time.perf_counter() - t0) < budget:
            O.moe_layer_q4(L, x_tokens[n:n + 1], 1, pool=pool, cache=cache)
            n += 1
        return (time.perf_counter() - t0) / n * 1e6, n

    per_use_1, n1 = timed(budget_s * 0.4)
    pool = O.Pool(nthr)
    try:
        per_use_k, nk = timed(budget_s * 0.2, pool=pool)
        t0 = time.perf_counter()
        cache = O.LayerCache(L, threads=ncores)
        build_s = time.perf_counter() - t0
        cached_1, nc1 = timed(budget_s * 0.2, cache=cache)
        cached_k, nck = timed(budget_s * 0.2, pool=pool, cache=cache)
        del cache
    finally:
        pool.close()
    return {"value": round(per_use_1, 1), "unit": "us/token", "cores": 1, "kind": "port",
            "sample": f"{n1} decode tokens of the same layer, dequant-per-use, threads=1",
            "nproc": ncores, "cpu_model": model,
            "variants": {
                "threads1_dequant_per_use": {"us_per_token": round(per_use_1, 1), "tokens": n1},
                f"threads{nthr}_dequant_per_use": {"us_per_token": round(per_use_k, 1),
                                                    "tokens": nk},
                "threads1_predequantized_fp32": {"us_per_token": round(cached_1, 1),
                                                 "tokens": nc1},
                f"threads{nthr}_predequantized_fp32": {"us_per_token": round(cached_k, 1),
                                                       "tokens": nck},
                "predequantize_build_s": round(build_s, 2),
                "predequantize_build_threads": ncores}}


MFMA_BF16_PEAK_TFLOPS = 2500.0


def grouped(a, blk, stream, dev):
    """Several tokens per call: routing, count/scan/scatter by expert, grouped
    expert GEMMs and the ordered combine.  batch: fresh tokens every step,
    HBM-bound, bytes = union of the step's experts + shared + router + x/y.
    prefill: a chunk of tokens per step with a Zipf(s) log-popularity router
    bias (folded into router column 0, activations' feature 0 = 1), reported
    as tokens/s and MFMA utilisation of the algorithmic FLOPs."""
    import numpy as np
    import torch

    from dismoen import synth
    cfg = synth.CONFIG_QWEN36
    L = synth.make_layer(**cfg, seed=a.seed)
    prefill = a.workload == "prefill"
    if prefill:
        L = synth.with_router_bias(L, synth.zipf_router_bias(L.num_experts, a.zipf_s, a.seed + 5))
    blk.upload_layer(0, L)
    H, E, K, I, Ish = L.hidden, L.num_experts, L.top_k, L.inter, L.inter_sh
    T = a.tokens if prefill else a.batch
    nbuf = (a.warmup + a.steps) if not prefill else min(a.warmup + a.steps, 8)
    rng = np.random.default_rng(a.seed + 2000)
    x_host = synth.make_activations(rng, (nbuf, T, H))
    if a.activations == "fp32":
        # a scale that is not a power of two gives most values nonzero lo parts
        x_host = (x_host * np.float32(1.0 + 2.0 ** -10)).astype(np.float32)
    if prefill:
        x_host = synth.bias_feature(x_host)
    x = torch.from_numpy(x_host).to(dev)
    y = torch.empty((nbuf, T, H), dtype=torch.float32, device=dev)
    ids = torch.empty((nbuf, T, K), dtype=torch.int32, device=dev)
    probs = torch.empty((nbuf, T, K), dtype=torch.float32, device=dev)
    shg = torch.empty((nbuf, T), dtype=torch.float32, device=dev)
    xp, yp, ip, pp, sp = (t.data_ptr() for t in (x, y, ids, probs, shg))

    def step(i):
        b = i % nbuf
        blk.forward_device(0, xp + b * T * H * 4, T, yp + b * T * H * 4, ip + b * T * K * 4,
                           pp + b * T * K * 4, sp + b * T * 4)

    for i in range(a.warmup):
        step(i)
    torch.cuda.synchronize()
    blk.sync()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(a.warmup, a.warmup + a.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    blk.sync()
    ms = e0.elapsed_time(e1) / a.steps
    ids_h = ids.cpu().numpy()
    used = [i % nbuf for i in range(a.warmup, a.warmup + a.steps)]
    unions = [len(np.unique(ids_h[b])) for b in used]
    u_mean = float(np.mean(unions))
    eb = synth.expert_bytes(H, I)
    counts = np.bincount(ids_h[used[-1]].reshape(-1), minlength=E)
    # parity spot check of a few tokens of the last step against the oracle
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    b = used[-1]
    smp = np.random.default_rng(7).choice(T, min(T, 4), replace=False)
    yo, ido, _, _ = O.moe_layer_q4(L, x_host[b][smp], len(smp))
    yg = y[b].cpu().numpy()[smp].astype(np.float64)
    rel = max(float(np.max(np.abs(yg[j] - yo[j])) / np.sqrt(np.mean(yo[j].astype(np.float64) ** 2)))
              for j in range(len(smp)))
    ids_ok = bool(np.array_equal(ids_h[b][smp], ido))
    us = ms * 1e3
    common = {"n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 6),
              "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
              "parity_sample": {"tokens": len(smp), "ids_bit_exact": ids_ok,
                                "max_abs_over_rms": rel, "f10": f10_metrics(yo, yg)}}
    if not prefill:
        nbytes = u_mean * eb + synth.expert_bytes(H, Ish) + 2 * E * H + 2 * H + T * H * 8
        gbps = nbytes / (ms * 1e-3) / 1e9
        out = {"metric": f"MoE-layer small-batch decode µs/token + achieved HBM GB/s "
                         f"(4-bit, batch {T}, 1 GPU)",
               "value": round(us / T, 3), "unit": "us/token", "higher_is_better": False,
               "us_per_step": round(us, 3), **common,
               "config": {"workload": f"qwen3.6-35b-a3b moe layer, batch-{T} decode",
                          "batch": T, "hidden": H, "experts": E, "top_k": K, "inter": I,
                          "group": 32, "bits": 4, "activations": a.activations},
               "expert_union_mean": round(u_mean, 2),
               "roofline": {"bound": "hbm",
                            "kernel": ("k_moe_tokens (one launch, each token's block on one XCD)"
                                       if 3 <= T <= 8 else
                                       "grouped path (router, build, gate/up, down, combine)"),
                            "achieved": round(gbps, 1),
                            "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                            "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                            "bytes_per_step": int(nbytes)}}
    else:
        flops = T * (K + 1) * 2 * 3 * H * I + 2 * T * E * H
        tflops = flops / (ms * 1e-3) / 1e12
        out = {"metric": "MoE-layer prefill tokens/s + MFMA utilisation (4-bit weights, bf16 "
                         "MFMA, 1 GPU)",
               "value": round(T / (ms * 1e-3), 1), "unit": "tokens/s", "higher_is_better": True,
               "us_per_step": round(us, 3), **common,
               "config": {"workload": f"qwen3.6-35b-a3b moe layer, {T}-token prefill chunk, "
                                      f"zipf(s={a.zipf_s}) router bias",
                          "tokens": T, "hidden": H, "experts": E, "top_k": K, "inter": I,
                          "group": 32, "bits": 4, "activations": a.activations},
               "experts_touched": int((counts > 0).sum()),
               "hottest_expert_tokens": int(counts.max()),
               "roofline": {"bound": "mfma", "kernel": "grouped path (router, build, gate/up, "
                            "down, combine)", "achieved": round(tflops, 2),
                            "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                            "flops_per_step": flops}}
    print(json.dumps(out))


GGUF_TYPES = {"q3_k": (11, 256, 114, 112), "q4_k": (12, 256, 144, 0), "q8_0": (8, 32, 34, 0)}


def gguf_layer(a, blk, stream, dev):
    """256 experts x 2048 x 512 weights of one GGUF type -> fp32, resident in HBM."""
    import numpy as np
    import torch

    from dismoen import gguf
    t, bs, bpb, d_off = GGUF_TYPES[a.gguf_type]
    E, H, I = 256, 2048, 512
    n = E * H * I
    nb = n // bs
    g = torch.Generator(device=dev).manual_seed(a.seed)
    raw = torch.randint(0, 256, (nb, bpb), dtype=torch.uint8, device=dev, generator=g)
    raw[:, d_off + 1] %= 0x7C  # finite fp16 super-scales
    out = torch.empty(n, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def launch():
        gguf.dequantize_device(t, raw.data_ptr(), nb * bpb, n, out.data_ptr(), blk)

    for _ in range(a.warmup):
        launch()
    blk.sync()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(a.steps):
        launch()
    e1.record(stream)
    torch.cuda.synchronize()
    blk.sync()
    ms = e0.elapsed_time(e1) / a.steps
    alg = nb * bpb + n * 4
    gbps = alg / (ms * 1e-3) / 1e9
    rec = {"metric": f"GGUF {a.gguf_type.upper()} expert-layer dequant µs + achieved HBM GB/s",
           "value": round(ms * 1e3, 2), "unit": "us/layer", "n_gpus": 1, "steps": a.steps,
           "warmup": a.warmup, "ms_per_step": round(ms, 6), "higher_is_better": False,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": f"gguf {a.gguf_type} dequant, 256 experts x 2048 x 512 "
                                  "weights to fp32", "weights": n, "payload_bytes": nb * bpb},
           "roofline": {"bound": "hbm", "kernel": f"k_dequant_gguf<{t}>", "achieved": round(gbps, 1),
                        "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                        "traffic": profiled_traffic(GGUF_PROFILE) if t == 11 else None,
                        "bytes_per_launch": alg}}
    if not a.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as orc
        host = raw[:max(1, nb // 32)].cpu().numpy()  # 8 of the 256 experts
        t0 = time.perf_counter()
        reps = 0
        while True:
            orc.dequant_gguf(t, host.ravel(), host.shape[0] * bs)
            reps += 1
            if time.perf_counter() - t0 > min(a.cpu_sample_s, 10.0):
                break
        per = (time.perf_counter() - t0) / reps * (nb / host.shape[0])
        rec["cpu_baseline"] = {"value": round(per * 1e6, 1), "unit": "us/layer", "cores": 1,
                               "kind": "port",
                               "sample": f"{host.shape[0]} blocks (8 experts) x {reps} passes, "
                                         "scaled to 256 experts"}
    print(json.dumps(rec))


def gguf_moe_tokens(a, blk, stream, dev, dims):
    """Calls of a.gguf_tokens tokens on the uploaded GGUF layer: the grouped
    form (tokens grouped by expert, each expert row read once per unit)."""
    import numpy as np
    import torch

    from dismoen import synth
    H, E, K, I, Ish = dims
    T, nb = a.gguf_tokens, 8
    xs = synth.make_activations(np.random.default_rng(a.seed), (nb, T, H))
    xd = torch.from_numpy(xs).to(dev)
    yd = torch.empty((nb, T, H), dtype=torch.float32, device=dev)
    idd = torch.empty((nb, T, K), dtype=torch.int32, device=dev)
    pd = torch.empty((nb, T, K), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def step(i):
        b = i % nb
        blk.forward_gguf_device(0, xd[b].data_ptr(), T, yd[b].data_ptr(), idd[b].data_ptr(),
                                pd[b].data_ptr())

    for i in range(a.warmup):
        step(i)
    blk.sync()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(a.steps):
        step(a.warmup + i)
    e1.record(stream)
    torch.cuda.synchronize()
    blk.sync()
    ms = e0.elapsed_time(e1) / a.steps
    ids = idd.cpu().numpy()
    uniq = float(np.mean([len(np.unique(ids[b])) for b in range(nb)]))
    blk_bytes = lambda n: n // 256 * 114  # Q3_K payload of n weights
    # router, the distinct routed experts and the shared one read once, x in, y out
    alg = E * H * 4 + H * 4 + (uniq + 1) * 3 * blk_bytes(I * H) + 2 * T * H * 4
    gbps = alg / (ms * 1e-3) / 1e9
    rec = {"metric": f"GGUF Q3_K MoE-layer µs/token + achieved HBM GB/s ({T} tokens per call)",
           "value": round(ms * 1e3 / T, 3), "unit": "us/token", "us_per_step": round(ms * 1e3, 3),
           "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 6),
           "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
           "data": "synthetic",
           "config": {"workload": f"qwen3.6-35b-a3b moe layer from gguf (256 q3_k experts + "
                                  f"q3_k shared), {T} tokens per call", "hidden": H,
                      "experts": E, "top_k": K, "inter": I, "inter_sh": Ish, "tokens": T},
           "roofline": {"bound": "hbm", "kernel": "grouped gguf path (router, select, grouping, "
                                                  "gate/up, down, combine)",
                        "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                        "bytes_per_step": int(alg), "distinct_experts": uniq},
           "cpu_baseline": None}
    print(json.dumps(rec), flush=True)


def gguf_moe(a, blk, stream, dev):
    """Batch-1 decode of a Qwen3.6-shape GGUF MoE layer (Q3_K experts)."""
    import tempfile

    import numpy as np
    import torch

    from dismoen import gguf, synth
    H, E, K, I, Ish = 2048, 256, 8, 512, 512
    path = os.path.join(tempfile.gettempdir(), f"dismoen_bench_gguf_{os.getpid()}.gguf")
    gguf.write_gguf(path, synth.make_gguf_moe_layer(H, E, I, Ish, seed=a.seed))
    try:
        with gguf.parse_gguf_index(path) as g:
            blk.upload_layer_gguf(0, (H, E, K, I, Ish), g)
            if a.gguf_tokens > 1:
                return gguf_moe_tokens(a, blk, stream, dev, (H, E, K, I, Ish))
            ntok = a.warmup + a.steps
            rng = np.random.default_rng(a.seed)
            xs = synth.make_activations(rng, (ntok, H))
            xd = torch.from_numpy(xs).to(dev)
            yd = torch.empty((ntok, H), dtype=torch.float32, device=dev)
            idd = torch.empty((ntok, K), dtype=torch.int32, device=dev)
            pd = torch.empty((ntok, K), dtype=torch.float32, device=dev)
            torch.cuda.synchronize()
            xp, yp, ip, pp = xd.data_ptr(), yd.data_ptr(), idd.data_ptr(), pd.data_ptr()
            for t in range(a.warmup):
                blk.forward_gguf_device(0, xp + t * H * 4, 1, yp + t * H * 4, ip + t * K * 4,
                                        pp + t * K * 4)
            blk.sync()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for t in range(a.warmup, ntok):
                blk.forward_gguf_device(0, xp + t * H * 4, 1, yp + t * H * 4, ip + t * K * 4,
                                        pp + t * K * 4)
            e1.record(stream)
            torch.cuda.synchronize()
            blk.sync()
            ms = e0.elapsed_time(e1) / a.steps
            blk_bytes = lambda n: n // 256 * 114  # Q3_K payload of n weights
            alg = (E * H * 4 + H * 4 + (K + 1) * 3 * blk_bytes(I * H) + 2 * H * 4)
            gbps = alg / (ms * 1e-3) / 1e9
            rec = {"metric": "GGUF Q3_K MoE-layer decode µs/token + achieved HBM GB/s (batch 1)",
                   "value": round(ms * 1e3, 3), "unit": "us/token", "n_gpus": 1,
                   "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 6),
                   "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
                   "dtype": "f32", "data": "synthetic",
                   "config": {"workload": "qwen3.6-35b-a3b moe layer from gguf (q8_0 router, "
                                          "256 q3_k experts + q3_k shared), batch-1 decode",
                              "hidden": H, "experts": E, "top_k": K, "inter": I,
                              "inter_sh": Ish, "tokens": a.steps},
                   "roofline": {"bound": "hbm", "kernel": "k_gguf_one (one launch per token)",
                                "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                                "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                                "traffic": profiled_traffic(GGUF_MOE_PROFILE,
                                                            "traffic_bytes_per_token"),
                                "traffic_source": GGUF_MOE_PROFILE, "bytes_per_token": alg}}
            if not a.no_cpu:
                sys.path.insert(0, os.path.join(ROOT, "oracle"))
                import oracle as orc
                x = xs[-1:]
                p = "blk.0."

                def deq(name):
                    t = g.tensors[g.tensor_map[p + name]]
                    return orc.dequant_gguf(t.dtype, g.read_raw(p + name), t.num_elements)

                # the reference dequantizes every expert of the layer per token
                # (gguf_port_loader.mojo:217-236): timed on 8 of them, scaled
                t0 = time.perf_counter()
                for e in range(8):
                    for nm in ("gate", "up", "down"):
                        deq(f"ffn_{nm}.{e}.weight")
                t_deq = (time.perf_counter() - t0) * E / 8
                t0 = time.perf_counter()
                ids, probs = orc.router_forward(x, deq("ffn_gate_exps.weight"), 1, H, E, K)
                routed = np.zeros((1, K * H), np.float32)
                for k in range(K):
                    e = int(ids[0, k])
                    routed[0, k * H:(k + 1) * H] = orc.swiglu_forward(
                        x[0], deq(f"ffn_gate.{e}.weight"), deq(f"ffn_up.{e}.weight"),
                        deq(f"ffn_down.{e}.weight"), 1, H, I)
                sh = orc.swiglu_forward(x, deq("ffn_shared_gate.weight"),
                                        deq("ffn_shared_up.weight"),
                                        deq("ffn_shared_down.weight"), 1, H, Ish)
                gt = orc.shared_gate_forward(x, deq("shared_gate.weight"), 1, H)
                ref = orc.moe_aggregate(None, routed, probs, sh, gt, 1, H, K)
                t_blk = time.perf_counter() - t0
                y = yd[-1].cpu().numpy()
                rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
                rec["parity_last_token"] = {
                    "ids_bit_exact": bool(np.array_equal(idd[-1].cpu().numpy(), ids[0])),
                    "max_abs_over_rms": float(np.max(np.abs(y - ref)) / rms),
                    "f10": f10_metrics(ref, y)}
                rec["cpu_baseline"] = {"value": round((t_deq + t_blk) * 1e6, 1),
                                       "unit": "us/token", "cores": 1, "kind": "port",
                                       "sample": "dequant of 8 of the 256 experts scaled to 256 "
                                                 "(the reference's per-token dequant) + one "
                                                 "token's block, threads=1"}
            print(json.dumps(rec))
    finally:
        os.unlink(path)


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)
    import numpy as np
    import torch

    from dismoen import MoEBlock, _lib, synth

    dev = torch.device("cuda:0")
    if a.workload == "copy":
        n = a.copy_mib * (1 << 20) // 4
        src = torch.randn(n, device=dev)
        dst = torch.empty_like(src)
        for _ in range(a.warmup):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(a.steps):
            torch.neg(src, out=dst)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / a.steps
        nbytes = 2 * n * 4
        print(json.dumps({"metric": "device copy GB/s (read+write)", "value": round(nbytes / ms / 1e6, 1),
                          "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
                          "ms_per_step": round(ms, 6), "higher_is_better": True,
                          "read_bytes": n * 4, "write_bytes": n * 4, "dtype": "f32",
                          "data": "synthetic", "config": {"workload": f"copy {a.copy_mib} MiB"}}))
        return
    blk = MoEBlock(0)
    # time on the library's own stream (the stream every launch goes to)
    stream = torch.cuda.ExternalStream(blk.stream(), device=dev)
    if a.workload == "gguf":
        gguf_layer(a, blk, stream, dev)
        blk.close()
        return
    if a.workload == "gguf-moe":
        gguf_moe(a, blk, stream, dev)
        blk.close()
        return

    if a.workload in ("decode", "toy"):
        cfg = synth.CONFIG_QWEN36 if a.workload == "decode" else synth.CONFIG_TOY
        L = synth.make_layer(**cfg, seed=a.seed)
        blk.upload_layer(0, L)
        H, K = L.hidden, L.top_k
        ntok = a.warmup + a.steps
        rng = np.random.default_rng(a.seed + 1000)
        x_host = synth.make_activations(rng, (ntok, H))
        x = torch.from_numpy(x_host).to(dev)
        y = torch.empty((ntok, H), dtype=torch.float32, device=dev)
        ids = torch.empty((ntok, K), dtype=torch.int32, device=dev)
        probs = torch.empty((ntok, K), dtype=torch.float32, device=dev)
        shg = torch.empty((ntok,), dtype=torch.float32, device=dev)
        xp, yp, ip, pp, sp = (t.data_ptr() for t in (x, y, ids, probs, shg))

        def step(t):
            blk.forward_device(0, xp + t * H * 4, 1, yp + t * H * 4, ip + t * K * 4,
                               pp + t * K * 4, sp + t * 4)

        for t in range(a.warmup):
            step(t)
        torch.cuda.synchronize()
        blk.sync()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        e0.record(stream)
        for t in range(a.warmup, ntok):
            step(t)
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - w0
        blk.sync()
        ms = e0.elapsed_time(e1) / a.steps
        bytes_tok = synth.algorithmic_bytes_per_token(H, L.num_experts, K, L.inter, L.inter_sh)
        us = ms * 1e3
        gbps = bytes_tok / (us * 1e-6) / 1e9
        # parity spot check of the last token against the oracle (outside timing)
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        t_last = ntok - 1
        yo, ido, po, _ = O.moe_layer_q4(L, x_host[t_last:t_last + 1], 1)
        ids_ok = bool(np.array_equal(ids[t_last].cpu().numpy(), ido[0]))
        yl = y[t_last].cpu().numpy().astype(np.float64)
        rel = float(np.max(np.abs(yl - yo[0])) / np.sqrt(np.mean(yo[0].astype(np.float64) ** 2)))
        f10 = f10_metrics(yo[0], yl)
        traffic = profiled_traffic() if a.workload == "decode" else None
        # the drop-in's host-pointer form, as a compiled caller makes it: x and
        # the outputs in the caller's own host arrays, one synchronous C call
        # per token (reported beside value, never as value); the same call
        # through forward_into (argument checks in Python) and forward_arrays
        # (new numpy outputs per call) is timed too
        nh = min(200, a.steps)
        hy = np.empty(H, np.float32)
        hids = np.empty(K, np.int32)
        hprobs = np.empty(K, np.float32)
        hshg = np.empty(1, np.float32)
        xrows = [np.ascontiguousarray(x_host[t]) for t in range(a.warmup + nh)]
        for t in range(min(5, a.warmup)):  # first calls size the staging block
            blk.forward_into(0, xrows[t], 1, hy, hids, hprobs, hshg)
        fwd, hctx, ebuf = blk._lib.dmh_moe_forward, blk._h, _lib.errbuf()
        outp = (hy.ctypes.data, hids.ctypes.data, hprobs.ctypes.data, hshg.ctypes.data)
        xps = [r.ctypes.data for r in xrows]
        t0 = time.perf_counter()
        for t in range(a.warmup, a.warmup + nh):
            rc = fwd(hctx, 0, xps[t], None, 1, *outp, 0, ebuf, 2048)
            if rc:
                raise RuntimeError(ebuf.value.decode(errors="replace"))
        host_us = (time.perf_counter() - t0) / nh * 1e6
        t0 = time.perf_counter()
        for t in range(a.warmup, a.warmup + nh):
            blk.forward_into(0, xrows[t], 1, hy, hids, hprobs, hshg)
        host_into_us = (time.perf_counter() - t0) / nh * 1e6
        t0 = time.perf_counter()
        for t in range(a.warmup, a.warmup + nh):
            blk.forward_arrays(0, x_host[t:t + 1], 1)
        host_arrays_us = (time.perf_counter() - t0) / nh * 1e6
        out = {
            "metric": METRIC, "value": round(us, 3), "unit": "us/token", "n_gpus": 1,
            "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 6),
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic",
            "config": {"workload": ("qwen3.6-35b-a3b moe layer, batch-1 decode"
                                    if a.workload == "decode" else "toy moe layer, batch-1 decode"),
                       "hidden": H, "experts": L.num_experts, "top_k": K, "inter": L.inter,
                       "inter_sh": L.inter_sh, "group": 32, "bits": 4, "tokens": a.steps},
            "achieved_gbps": round(gbps, 1),
            "roofline": {"bound": "hbm",
                         "kernel": "k_moe_decode_xs (XCD-sliced fused launch per token)",
                         "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
                         "traffic_source": TRAFFIC_PROFILE if traffic else None,
                         "bytes_per_token": bytes_tok},
            "parity_last_token": {"ids_bit_exact": ids_ok, "max_abs_over_rms": rel, "f10": f10},
            "host_pointer_us_per_token": round(host_us, 2),
            "host_pointer_forward_into_us_per_token": round(host_into_us, 2),
            "host_pointer_forward_arrays_us_per_token": round(host_arrays_us, 2),
            "wall_s": round(wall, 3),
        }
        if not a.no_cpu:
            out["cpu_baseline"] = cpu_baseline(L, x_host, a.cpu_sample_s)
        print(json.dumps(out))
    elif a.workload in ("batch", "prefill"):
        grouped(a, blk, stream, dev)
    else:  # stack
        cfg = synth.CONFIG_QWEN36
        nl = a.layers
        dims = (cfg["hidden"], cfg["num_experts"], cfg["top_k"], cfg["inter"], cfg["inter_sh"])
        for l in range(nl):
            W = synth.make_layer_device(**cfg, seed=a.seed * 1000 + l, device=dev)
            torch.cuda.synchronize()  # drawn on torch's stream, read on the library's
            blk.upload_layer_device(l, dims, {k: v.data_ptr() for k, v in W.items()})
            blk.sync()
            del W
        H, K = cfg["hidden"], cfg["top_k"]
        ntok = a.warmup + a.steps
        x_host = synth.make_activations(np.random.default_rng(a.seed + 7), (ntok, H))
        x = torch.from_numpy(x_host).to(dev)
        y = torch.empty((ntok, H), dtype=torch.float32, device=dev)
        xp, yp = x.data_ptr(), y.data_ptr()
        tree = a.stack_norm == "tree"
        for t in range(a.warmup):
            blk.forward_stack_device(xp + t * H * 4, 0, nl, 1, yp + t * H * 4, tree=tree)
        torch.cuda.synchronize()
        blk.sync()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for t in range(a.warmup, ntok):
            blk.forward_stack_device(xp + t * H * 4, 0, nl, 1, yp + t * H * 4, tree=tree)
        e1.record(stream)
        torch.cuda.synchronize()
        blk.sync()
        ms = e0.elapsed_time(e1) / a.steps
        bytes_tok = nl * synth.algorithmic_bytes_per_token(H, cfg["num_experts"], K,
                                                            cfg["inter"], cfg["inter_sh"])
        gbps = bytes_tok / (ms * 1e-3) / 1e9
        print(json.dumps({
            "metric": METRIC, "value": round(ms * 1e3, 3), "unit": "us/token", "n_gpus": 1,
            "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 6),
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic",
            "config": {"workload": f"{nl}-layer moe stack resident in HBM, batch-1 decode",
                       "layers": nl, "hidden": H, "tokens": a.steps,
                       "norm_order": "reference (sequential)" if not tree else "tree"},
            "roofline": {"bound": "hbm", "kernel": "moe stack", "achieved": round(gbps, 1),
                         "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                         "bytes_per_token": bytes_tok}}))
    blk.close()


if __name__ == "__main__":
    main()

"""Per-layer phase timeline of the fused decode kernel over a resident stack.

Runs the 40-layer Qwen3.6-shape stack of `bench.py --workload stack` (layers
drawn on the GPU, identity mixer + residual, the block-edge RMSNorm in the
reference's order or as a tree) through the tracing build of the library
(`make -C disk-streaming-moe-engine_amd trace` -> libdismoen_hip_trace.so,
the same sources compiled with DM_PHASE_TRACE), then reads the timestamps
workgroup 0..255 of each layer's launch stored at eight points of
k_moe_decode_xs and prints, per layer and as medians over the layers, the
time of each point from the layer's first workgroup start (median over the
workgroups, and the last workgroup).

    python3 disk-streaming-moe-engine_amd/phase_trace.py [--norm ref|tree|none] [--tokens N]

--norm none traces the single-layer decode instead (one layer, no norm,
dmh_moe_forward on device pointers, the bench's default workload).

    python3 disk-streaming-moe-engine_amd/phase_trace.py --batch T

traces the several-token launch of k_moe_tokens instead (T = 3 .. 8 tokens
per call, one layer, device pointers, the last call's workgroups that hold a
token): x staged, routing done, gate/up tasks done, h staged, down products
done, end.
"""
import argparse
import ctypes as C
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
TRACE_LIB = os.path.join(HERE, "libdismoen_hip_trace.so")
SLOTS, WGS, POINTS = 64, 256, 8   # kTraceSlots x 256 workgroups x kTracePoints
NAMES = {1: "norm sum done", 2: "x staged", 3: "routing done", 4: "h staged",
         5: "partial published", 6: "partials polled", 7: "end"}
CLOCK_MHZ = 100.0  # wall_clock64


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--norm", default="ref", choices=["ref", "tree", "none"])
    ap.add_argument("--tokens", type=int, default=20)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--batch", type=int, default=0,
                    help="trace the several-token launch with this many tokens per call")
    a = ap.parse_args()
    if not os.path.exists(TRACE_LIB):
        raise SystemExit(f"{TRACE_LIB} not built (make -C {HERE} trace)")
    if a.layers > SLOTS:
        raise SystemExit(f"at most {SLOTS} layers are traced")
    os.environ["DISMOEN_LIB"] = TRACE_LIB
    sys.path.insert(0, HERE)
    import torch
    from dismoen import MoEBlock, synth, _lib
    assert _lib.LIB_PATH == TRACE_LIB
    dev = torch.device("cuda:0")
    blk = MoEBlock(0)
    fetch = blk._lib.dmh_phase_trace_fetch
    fetch.argtypes = [C.c_void_p, C.c_size_t]
    fetch.restype = C.c_int
    cfg = synth.CONFIG_QWEN36
    if a.batch:
        return trace_batch(a, blk, fetch, cfg, dev)
    nl = 1 if a.norm == "none" else a.layers
    dims = (cfg["hidden"], cfg["num_experts"], cfg["top_k"], cfg["inter"], cfg["inter_sh"])
    for l in range(nl):
        W = synth.make_layer_device(**cfg, seed=1000 + l, device=dev)
        torch.cuda.synchronize()
        blk.upload_layer_device(l, dims, {k: v.data_ptr() for k, v in W.items()})
        blk.sync()
        del W
    H = cfg["hidden"]
    x = torch.from_numpy(synth.make_activations(np.random.default_rng(7), (a.tokens, H))).to(dev)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    if a.norm == "none":
        K = cfg["top_k"]
        ids = torch.empty((a.tokens, K), dtype=torch.int32, device=dev)
        pr = torch.empty((a.tokens, K), dtype=torch.float32, device=dev)
        sg = torch.empty((a.tokens,), dtype=torch.float32, device=dev)
        for t in range(a.tokens):
            blk.forward_device(0, x[t].data_ptr(), 1, y[t].data_ptr(), ids[t].data_ptr(),
                               pr[t].data_ptr(), sg[t].data_ptr())
    else:
        for t in range(a.tokens):  # the last token's launches leave their stamps
            blk.forward_stack_device(x[t].data_ptr(), 0, nl, 1, y[t].data_ptr(),
                                     tree=a.norm == "tree")
    blk.sync()
    buf = np.zeros(SLOTS * WGS * POINTS, np.uint64)
    rc = fetch(C.c_void_p(buf.ctypes.data), buf.nbytes)
    if rc != 0:
        raise SystemExit(f"dmh_phase_trace_fetch returned {rc}")
    tr = buf.reshape(SLOTS, WGS, POINTS)[:nl].astype(np.int64)
    base = tr[:, :, 0].min(axis=1)
    rows = []
    # points no launch stored (the norm's, without a norm) are left out
    names = {k: nm for k, nm in NAMES.items() if (tr[:, :, k] > 0).all()}
    for l in range(nl):
        r = {"layer": l, "start_spread_us": round(float((tr[l, :, 0].max() - base[l]) / CLOCK_MHZ), 2)}
        for k, nm in names.items():
            d = (tr[l, :, k] - base[l]) / CLOCK_MHZ
            r[nm] = [round(float(np.median(d)), 2), round(float(d.max()), 2)]
        if l + 1 < nl:
            r["layer_us"] = round(float((base[l + 1] - base[l]) / CLOCK_MHZ), 2)
        rows.append(r)
    print("norm", a.norm, "layers", nl, "token", a.tokens - 1)
    for r in rows:
        print(json.dumps(r))
    lay = [r["layer_us"] for r in rows if "layer_us" in r]
    if lay:
        print(f"median layer start-to-start us {np.median(lay):.2f}; first to last start "
              f"{(base[-1] - base[0]) / CLOCK_MHZ:.2f} us")
    for k, nm in names.items():
        med = np.median([r[nm][0] for r in rows])
        mx = np.median([r[nm][1] for r in rows])
        print(f"{nm:>18}: median {med:.2f} us (median over layers of the last workgroup {mx:.2f})")


BATCH_NAMES = {1: "x staged", 2: "routing done", 3: "gate/up tasks done", 4: "h staged",
               5: "down products done", 7: "end"}


def trace_batch(a, blk, fetch, cfg, dev):
    import torch
    from dismoen import synth
    T = a.batch
    W = synth.make_layer_device(**cfg, seed=1000, device=dev)
    torch.cuda.synchronize()
    dims = (cfg["hidden"], cfg["num_experts"], cfg["top_k"], cfg["inter"], cfg["inter_sh"])
    blk.upload_layer_device(0, dims, {k: v.data_ptr() for k, v in W.items()})
    blk.sync()
    del W
    H, K = cfg["hidden"], cfg["top_k"]
    x = torch.from_numpy(synth.make_activations(np.random.default_rng(7), (a.tokens, T, H))).to(dev)
    y = torch.empty_like(x)
    ids = torch.empty((a.tokens, T, K), dtype=torch.int32, device=dev)
    pr = torch.empty((a.tokens, T, K), dtype=torch.float32, device=dev)
    sg = torch.empty((a.tokens, T), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    for i in range(a.tokens):  # the last call's launch leaves its stamps
        blk.forward_device(0, x[i].data_ptr(), T, y[i].data_ptr(), ids[i].data_ptr(),
                           pr[i].data_ptr(), sg[i].data_ptr())
    blk.sync()
    buf = np.zeros(SLOTS * WGS * POINTS, np.uint64)
    rc = fetch(C.c_void_p(buf.ctypes.data), buf.nbytes)
    if rc != 0:
        raise SystemExit(f"dmh_phase_trace_fetch returned {rc}")
    tr = buf.reshape(SLOTS, WGS, POINTS)[0].astype(np.int64)
    tr = tr[tr[:, 7] > 0]  # the workgroups that held a token
    base = tr[:, 0].min()
    print(f"batch {T}, {len(tr)} workgroups with a token, call {a.tokens - 1}")
    for k, nm in BATCH_NAMES.items():
        d = (tr[:, k] - base) / CLOCK_MHZ
        print(f"{nm:>20}: median {np.median(d):.2f} us (last workgroup {d.max():.2f})")


if __name__ == "__main__":
    main()

"""Benchmark: apply + encode of one RL-like update of a 7B-shaped bf16 state dict on one MI355X.

A step is one encode_update (trainer side) plus one apply_update (worker side) of a synthetic update
with the given changed fraction, inputs already resident in HBM, bytes kept in device memory
(encode_update_device / apply_update on the uint8 tensor), checksum caches warm on both sides.
Two synthetic states A and B alternate (A->B, B->A, ...), so every step is a full, verified update
and the receiver ends each step equal to the sender's new state.

Prints one JSON line. `roofline` covers the dominant kernel, timed with HIP events on its stream
during the timed steps; `cpu_baseline` times the CPU oracle (a plain-C port of the reference's
algorithm, one thread) on a bounded sample of the same workload and scales it to the full update.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "crukx-sync_amd"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="qwen2.5-7b", help="qwen2.5-1.5b | qwen2.5-7b | qwen2.5-32b | small4")
    ap.add_argument("--rho", type=float, default=0.01)
    ap.add_argument("--p-one", type=float, default=0.87)
    ap.add_argument("--cpu-baseline-layers", type=int, default=2,
                    help="decoder layers in the CPU baseline sample (0 disables it)")
    ap.add_argument("--host-bytes", action=argparse.BooleanOptionalAction, default=True,
                    help="also time the bytes API (PCIe-inclusive; reported in detail, never in value)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run three 2 GiB device-to-device copies (reference for HBM traffic counters)")
    args = ap.parse_args()

    if args.calibrate_copy:
        import torch
        a = torch.ones(1 << 31, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read_per_copy": a.numel(), "bytes_written_per_copy": b.numel()}))
        return

    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the update codec has no multi-GPU path "
                                   "here (sharding is described in DESIGN.md); run with --gpus 1"}))
        sys.exit(2)

    import torch

    import crukx_sync
    from crukx_sync import _native, workloads

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    shapes = workloads.shapes_for(args.workload)
    N = workloads.numel(shapes)
    log(f"[bench] generating {args.workload}: {N:,} weights in {len(shapes)} tensors, rho={args.rho}")
    t0 = time.time()
    A = workloads.make_weights(shapes, seed=0, device=dev)
    B = workloads.make_step(A, 1, rho=args.rho, p_one=args.p_one, seed=0)
    recv = {k: v.clone() for k, v in A.items()}
    torch.cuda.synchronize()
    log(f"[bench] generated in {time.time() - t0:.1f}s; "
        f"{torch.cuda.memory_allocated() / 2**30:.1f} GiB allocated")
    states = [A, B]
    send_chk, recv_chk = {}, {}

    def step(i, timed=None):
        old, new = states[i % 2], states[(i + 1) % 2]
        torch.cuda.synchronize()
        t_a = time.perf_counter()
        upd = crukx_sync.encode_update_device(old, new, send_chk)
        torch.cuda.synchronize()
        t_b = time.perf_counter()
        stats = crukx_sync.apply_update(recv, upd, recv_chk)
        torch.cuda.synchronize()
        t_c = time.perf_counter()
        if timed is not None:
            timed.append((t_b - t_a, t_c - t_b, upd.numel(), stats.changed))
        return upd, stats

    # cold step (full checksums on both sides), then warm-up
    cold = []
    step(0, cold)
    log(f"[bench] cold step: encode {cold[0][0] * 1e3:.2f} ms, apply {cold[0][1] * 1e3:.2f} ms, "
        f"{cold[0][2]:,} bytes, {cold[0][3]:,} changes")
    for i in range(1, 1 + args.warmup):
        step(i)
    for k in recv:
        assert torch.equal(recv[k].view(torch.int16), states[(1 + args.warmup) % 2][k].view(torch.int16)), k
    log("[bench] warm-up done, receiver exact")

    _native.timing_reset()
    _native.timing(True)
    timed = []
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for i in range(1 + args.warmup, 1 + args.warmup + args.steps):
        step(i, timed)
    torch.cuda.synchronize()
    t_total = time.perf_counter() - t_start
    _native.timing(False)
    kern = _native.timing_read()
    last = states[(1 + args.warmup + args.steps) % 2]
    for k in recv:
        assert torch.equal(recv[k].view(torch.int16), last[k].view(torch.int16)), k
    assert send_chk == {k: v[0] for k, v in recv_chk.items()}
    log(f"[bench] {args.steps} timed steps exact; kernels: " +
        ", ".join(f"{n} {ms / max(c, 1):.3f}ms" for n, (c, ms) in sorted(kern.items(), key=lambda x: -x[1][1])[:8]))

    ms_step = t_total / args.steps * 1e3
    enc_ms = sum(t[0] for t in timed) / len(timed) * 1e3
    app_ms = sum(t[1] for t in timed) / len(timed) * 1e3
    upd_bytes = sum(t[2] for t in timed) / len(timed)
    changes = sum(t[3] for t in timed) / len(timed)

    # roofline of the dominant kernel: algorithmic HBM bytes per launch / average launch time
    alg_bytes = {"enc_rank": 4 * N, "apply_hist": 2 * N, "select": 2 * N}
    dom = max((k for k in kern if k in alg_bytes), key=lambda k: kern[k][1])
    calls, tot_ms = kern[dom]
    avg_ms = tot_ms / calls
    achieved = alg_bytes[dom] / (avg_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(args.workload, args.rho, dom),
                "avg_launch_ms": round(avg_ms, 4), "alg_bytes_per_launch": alg_bytes[dom]}
    copy_gbs, read_gbs = stream_ceilings(torch, dev)
    roofline["copy_gbs"] = round(copy_gbs, 1)  # measured ceilings: device-to-device copy (read + write bytes)
    roofline["read_gbs"] = round(read_gbs, 1)  # and a read-only reduction
    roofline["frac_of_copy"] = round(achieved / copy_gbs, 4)
    whole = (6 * N + upd_bytes + 2 * changes) / (ms_step * 1e-3) / 1e9  # encode 4N+P, apply 2N+P+2C

    detail = {"encode_ms": round(enc_ms, 3), "apply_ms": round(app_ms, 3),
              "cold_encode_ms": round(cold[0][0] * 1e3, 3), "cold_apply_ms": round(cold[0][1] * 1e3, 3),
              "update_bytes": int(upd_bytes), "changes": int(changes),
              "bytes_per_change": round(upd_bytes / max(changes, 1), 4),
              "whole_update_alg_gbs": round(whole, 1), "whole_update_frac": round(whole / HBM_PEAK_GBS, 4),
              "kernels_ms_per_step": {n: round(ms / args.steps, 4) for n, (c, ms) in sorted(kern.items())}}

    if args.host_bytes:
        hb = []
        for i in range(3):
            old, new = states[(1 + args.warmup + args.steps + i) % 2], states[(2 + args.warmup + args.steps + i) % 2]
            torch.cuda.synchronize()
            ta = time.perf_counter()
            data = crukx_sync.encode_update(old, new, send_chk)
            tb = time.perf_counter()
            crukx_sync.apply_update(recv, data, recv_chk)
            torch.cuda.synchronize()
            hb.append((tb - ta, time.perf_counter() - tb))
        detail["host_bytes_encode_ms"] = round(min(x[0] for x in hb) * 1e3, 3)
        detail["host_bytes_apply_ms"] = round(min(x[1] for x in hb) * 1e3, 3)

    cpu = None
    if args.cpu_baseline_layers > 0:
        cpu = cpu_baseline(args, shapes, states, N, log)

    out = {"metric": "apply+encode ms/update, 7B-shaped bf16, 1% changed; % of HBM peak",
           "value": round(ms_step, 3), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(ms_step, 3), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
           "dtype": "u16 bit patterns (bf16)", "data": "synthetic",
           "config": {"workload": f"{args.workload}-shaped bf16 state dict, {N} weights, rho={args.rho}, "
                                  f"p_one={args.p_one}, warm checksum caches, device-resident bytes",
                      "tensors": len(shapes), "weights": N, "rho": args.rho},
           "roofline": roofline, "cpu_baseline": cpu, "detail": detail}
    print(json.dumps(out), flush=True)


def stream_ceilings(torch, dev, nbytes=4 << 30, reps=5):
    """Best rates (GB/s) of a device-to-device copy of nbytes (read + write bytes) and of a sum over
    them (read only): achievable HBM ceilings to set beside the 8 TB/s peak."""
    a = torch.ones(nbytes // 8, dtype=torch.int64, device=dev)
    b = torch.empty_like(a)
    best_c = best_r = float("inf")
    for _ in range(reps):
        torch.cuda.synchronize()
        t = time.perf_counter()
        b.copy_(a)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        a.sum()
        torch.cuda.synchronize()
        best_c = min(best_c, t1 - t)
        best_r = min(best_r, time.perf_counter() - t1)
    del a, b
    return 2 * nbytes / best_c / 1e9, nbytes / best_r / 1e9


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def measured_traffic(workload, rho, kernel):
    """HBM bytes per launch of `kernel` (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, calibrated against a 2 GiB
    copy) as recorded by rocprofv3 for this workload in profiles/, or None when not recorded."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        rec = json.load(f)
    if rec.get("rho") != rho or kernel not in rec.get("kernels", {}):
        return None
    return rec["kernels"][kernel]["bytes"]


def cpu_baseline(args, shapes, states, N, log):
    """The oracle (one core) on the first decoder layers of the same workload, warm caches."""
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    layers = args.cpu_baseline_layers
    names = [n for n, _, _ in shapes if any(n.startswith(f"model.layers.{i}.") for i in range(layers))]
    if not names:  # small workloads: the whole state dict
        names = [n for n, _, _ in shapes]
    old = {n: states[0][n].cpu() for n in names}
    new = {n: states[1][n].cpu() for n in names}
    n_sample = sum(v.numel() for v in old.values())
    send = {n: oracle.checksum(v) for n, v in old.items()}
    recv_cache = dict(send)
    recv = {n: v.clone() for n, v in old.items()}
    t0 = time.perf_counter()
    data = oracle.encode_update(old, new, send)
    t1 = time.perf_counter()
    oracle.apply_update(recv, data, recv_cache)
    t2 = time.perf_counter()
    for n in names:
        assert torch.equal(recv[n].view(torch.int16), new[n].view(torch.int16)), n
    scale = N / n_sample
    ms = (t2 - t0) * scale * 1e3
    log(f"[bench] cpu oracle on {n_sample:,} weights: encode {t1 - t0:.2f}s apply {t2 - t1:.2f}s "
        f"-> {ms / 1e3:.1f}s per full update")
    return {"value": round(ms, 1), "unit": "ms", "cores": 1, "kind": "port",
            "sample": f"decoder layers 0..{layers - 1} of the same synthetic step ({n_sample} of {N} weights, "
                      f"warm checksum caches), encode + apply by the C oracle on one host core ({cpu_model()}), "
                      f"time scaled by {scale:.2f} to the full update",
            "sample_encode_s": round(t1 - t0, 3), "sample_apply_s": round(t2 - t1, 3)}


if __name__ == "__main__":
    main()

"""Benchmark: apply + encode of one RL-like update of a 7B-shaped bf16 state dict on one MI355X.

A step is one encode_update (trainer side) plus one apply_update (worker side) of a synthetic update
with the given changed fraction, inputs already resident in HBM, bytes kept in device memory
(encode_update_device / apply_update on the uint8 tensor), checksum caches warm on both sides.
Two synthetic states A and B alternate (A->B, B->A, ...), so every step is a full, verified update
and the receiver ends each step equal to the sender's new state.

Prints one JSON line.
- `value`: the timed steps, with per-launch event timing only around the dominant streaming kernel
  (`roofline` divides its algorithmic bytes by its average duration over those same steps).
- `detail.kernels_ms_per_step`: every kernel and host phase, from a separate instrumented pass.
- `detail.cold_*`: the process's first update (first allocations included); `detail.cold2_*`: an
  update with both checksum caches dropped and the allocator warm, i.e. full checksums on both sides
  (the median of three such steps, each after a warm step).
- `detail.configs`: the same measurement at other sizes and densities.
- `cpu_baseline`: a torch-CPU restatement of the reference's CPU path (oracle/torch_cpu.py, bytes
  checked against the reference's golden vectors by the tests) on the host's physical cores: `value` is
  one warm step of the whole update (encode and apply timed apart, bytes identical to the GPU's);
  beside it the 1.5B workload's seven chained steps, the small4 chain, and a layer sample also run by
  the single-threaded C oracle (the sample's bytes from the GPU, the restatement and the oracle must be
  identical).  `--cpu-baseline full` adds the 7B cold step; `sample` keeps only the sample and small4.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "crukx-sync_amd"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
STREAMING = ("enc_rank", "select", "apply_hist")  # kernels whose bytes are the workload's weights


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
    ap.add_argument("--profile-steps", type=int, default=5, help="steps of the instrumented pass (kernel table)")
    ap.add_argument("--configs", default="qwen2.5-7b:0.02,qwen2.5-1.5b:0.01",
                    help="workload:rho pairs also measured (in detail.configs); '' for none")
    ap.add_argument("--cpu-baseline-layers", type=int, default=2,
                    help="decoder layers in the CPU baseline sample (0 disables it)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="host threads of the CPU baseline (0: the physical cores this process may use, at most 16)")
    ap.add_argument("--cpu-baseline", choices=("sample", "standard", "full"), default="standard",
                    help="sample: the layer sample and the small4 chain only; standard: also one warm step of the "
                         "whole 7B update and the 1.5B workload's seven chained steps (about 2.5 minutes of host "
                         "time); full: also the 7B cold step")
    ap.add_argument("--cpu-cap-s", type=float, default=300.0,
                    help="wall-clock cap of each phase of a whole-update CPU step (past it the step is reported as "
                         "capped and the next phase is skipped)")
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
        print(json.dumps({"error": "bench.py measures one GPU: the update codec here has no multi-GPU path "
                                   "(it would shard by whole tensors); run with --gpus 1"}))
        sys.exit(2)

    import torch

    from crukx_sync import workloads

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    shapes = workloads.shapes_for(args.workload)
    N = workloads.numel(shapes)
    log(f"[bench] generating {args.workload}: {N:,} weights in {len(shapes)} tensors, rho={args.rho}")
    t0 = time.time()
    A = workloads.make_weights(shapes, seed=0, device=dev)
    B = workloads.make_step(A, 1, rho=args.rho, p_one=args.p_one, seed=0)
    torch.cuda.synchronize()
    log(f"[bench] generated in {time.time() - t0:.1f}s; {torch.cuda.memory_allocated() / 2**30:.1f} GiB allocated")

    run = Run(A, B, N)
    res = run.measure(args.steps, args.warmup, args.profile_steps, cold=True, host_bytes=args.host_bytes)
    log(f"[bench] {args.steps} timed steps: {res['ms_step']:.3f} ms/step (encode {res['encode_ms']:.3f}, "
        f"apply {res['apply_ms']:.3f}); top kernels: " +
        ", ".join(f"{n} {ms:.3f}" for n, ms in sorted(res["kernels"].items(), key=lambda x: -x[1])[:8]))

    dom, avg_ms = res["dominant"], res["dominant_ms"]
    alg = alg_bytes(dom, N, res["changes"])
    achieved = alg / (avg_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(args.workload, args.rho, dom),
                "avg_launch_ms": round(avg_ms, 4), "alg_bytes_per_launch": alg}
    copy_gbs, read_gbs = stream_ceilings(torch, dev)
    roofline["copy_gbs"] = round(copy_gbs, 1)  # measured ceilings: device-to-device copy (read + write bytes)
    roofline["read_gbs"] = round(read_gbs, 1)  # and a read-only reduction
    whole = (6 * N + res["update_bytes"] + 2 * res["changes"]) / (res["ms_step"] * 1e-3) / 1e9

    detail = {k: res[k] for k in ("encode_ms", "apply_ms", "cold_encode_ms", "cold_apply_ms", "cold2_encode_ms",
                                  "cold2_apply_ms", "update_bytes", "changes")}
    detail["bytes_per_change"] = round(res["update_bytes"] / max(res["changes"], 1), 4)
    detail["whole_update_alg_gbs"] = round(whole, 1)
    detail["whole_update_frac"] = round(whole / HBM_PEAK_GBS, 4)
    detail["streaming_kernels"] = {k: {"ms": round(v, 4), "frac": round(alg_bytes(k, N, res["changes"]) / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
                                   for k, v in res["kernels"].items() if k in STREAMING}
    detail["kernels_ms_per_step"] = {n: round(ms, 4) for n, ms in sorted(res["kernels"].items())}
    detail["cold_breakdown_ms"] = res["cold_breakdown"]
    detail["cold2_breakdown_ms"] = res["cold2_breakdown"]
    for k in ("host_bytes_encode_ms", "host_bytes_apply_ms", "reference_api_ms"):
        if k in res:
            detail[k] = res[k]

    cpu = None
    if args.cpu_baseline_layers > 0:
        cpu = cpu_baseline(args, shapes, A, B, N)

    configs = {}
    for spec in [s for s in args.configs.split(",") if s]:
        wl, rho = spec.split(":")
        configs[spec] = other_config(torch, dev, wl, float(rho), args, A if wl == args.workload else None)
    if configs:
        detail["configs"] = configs

    out = {"metric": "apply+encode ms/update, 7B-shaped bf16, 1% changed; % of HBM peak",
           "value": round(res["ms_step"], 3), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(res["ms_step"], 3), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
           "dtype": "u16 bit patterns (bf16)", "data": "synthetic",
           "config": {"workload": f"{args.workload}-shaped bf16 state dict, {N} weights, rho={args.rho}, "
                                  f"p_one={args.p_one}, warm checksum caches, device-resident bytes",
                      "tensors": len(shapes), "weights": N, "rho": args.rho},
           "roofline": roofline, "cpu_baseline": cpu, "detail": detail}
    print(json.dumps(out), flush=True)


def alg_bytes(kernel: str, n: int, changes: int) -> int:
    """Algorithmic HBM bytes of one launch of a streaming kernel: the weights it must read, and for the
    select pass (which writes the new bits of the slabs it streams in one window) 2 bytes per change."""
    return {"enc_rank": 4 * n, "select": 2 * n + 2 * changes, "apply_hist": 2 * n}[kernel]


class Run:
    """Alternating encode + apply steps between states A and B, both checksum caches kept."""

    def __init__(self, A, B, n):
        import torch
        self.torch = torch
        self.states = [A, B]
        self.n = n
        self.recv = {k: v.clone() for k, v in A.items()}
        self.send_chk, self.recv_chk = {}, {}
        self.i = 0

    def step(self):
        import crukx_sync
        torch = self.torch
        old, new = self.states[self.i % 2], self.states[(self.i + 1) % 2]
        torch.cuda.synchronize()
        t_a = time.perf_counter()
        upd = crukx_sync.encode_update_device(old, new, self.send_chk)
        torch.cuda.synchronize()
        t_b = time.perf_counter()
        stats = crukx_sync.apply_update(self.recv, upd, self.recv_chk)
        torch.cuda.synchronize()
        t_c = time.perf_counter()
        self.i += 1
        return t_b - t_a, t_c - t_b, upd.numel(), stats.changed

    def exact(self):
        cur = self.states[self.i % 2]
        for k in self.recv:
            assert self.torch.equal(self.recv[k].view(self.torch.int16), cur[k].view(self.torch.int16)), k
        assert self.send_chk == {k: v[0] for k, v in self.recv_chk.items()}

    def cold_step(self, instrumented):
        """One step with both checksum caches dropped (full checksums on both sides)."""
        from crukx_sync import _native
        self.send_chk.clear()
        self.recv_chk.clear()
        if instrumented:
            _native.timing_reset()
            _native.timing(True)
        r = self.step()
        if instrumented:
            _native.timing(False)
            kern = _native.timing_read()
            return r, {n: round(ms, 3) for n, (c, ms) in sorted(kern.items(), key=lambda x: -x[1][1])[:10]}
        return r, None

    def measure(self, steps, warmup, profile_steps, cold=False, host_bytes=False):
        from crukx_sync import _native
        torch = self.torch
        out = {}
        if cold:  # the process's first update, instrumented for its breakdown
            (e, a, _, _), out["cold_breakdown"] = self.cold_step(True)
            out["cold_encode_ms"], out["cold_apply_ms"] = round(e * 1e3, 3), round(a * 1e3, 3)
            log(f"[bench] cold step: encode {e * 1e3:.2f} ms, apply {a * 1e3:.2f} ms")
        for _ in range(warmup):
            self.step()
        self.exact()
        # caches dropped, allocator warm: three plain steps, each after a warm step (the median is
        # reported: single such steps varied by up to 1 ms), then one instrumented; then warm again
        e2, a2 = [], []
        for _ in range(3):
            self.step()
            (e, a, _, _), _ = self.cold_step(False)
            e2.append(e)
            a2.append(a)
        log("[bench] caches dropped, three steps: encode " + " ".join(f"{x * 1e3:.2f}" for x in e2) +
            " ms, apply " + " ".join(f"{x * 1e3:.2f}" for x in a2) + " ms")
        e, a = sorted(e2)[1], sorted(a2)[1]
        out["cold2_encode_ms"], out["cold2_apply_ms"] = round(e * 1e3, 3), round(a * 1e3, 3)
        _, out["cold2_breakdown"] = self.cold_step(True)
        for _ in range(max(warmup, 1)):
            self.step()
        self.exact()
        log(f"[bench] caches dropped: encode {out['cold2_encode_ms']:.2f} ms, apply {out['cold2_apply_ms']:.2f} ms")
        # instrumented pass: every kernel and host phase
        _native.timing_reset()
        _native.timing(True)
        for _ in range(profile_steps):
            self.step()
        _native.timing(False)
        kern = {n: ms / profile_steps for n, (c, ms) in _native.timing_read().items()}
        self.exact()
        out["kernels"] = kern
        dom = max((k for k in kern if k in STREAMING), key=lambda k: kern[k])
        # timed steps: events only around the dominant kernel
        _native.timing_reset()
        _native.timing(True, only=[dom])
        timed = []
        torch.cuda.synchronize()
        t_start = time.perf_counter()
        for _ in range(steps):
            timed.append(self.step())
        torch.cuda.synchronize()
        t_total = time.perf_counter() - t_start
        _native.timing(False)
        calls, ms = _native.timing_read()[dom]
        self.exact()
        out["dominant"], out["dominant_ms"] = dom, ms / calls
        out["ms_step"] = t_total / steps * 1e3
        out["encode_ms"] = round(sum(t[0] for t in timed) / steps * 1e3, 3)
        out["apply_ms"] = round(sum(t[1] for t in timed) / steps * 1e3, 3)
        out["update_bytes"] = int(sum(t[2] for t in timed) / steps)
        out["changes"] = int(sum(t[3] for t in timed) / steps)
        if host_bytes:  # the reference's bytes API: device -> pageable host bytes -> device
            import crukx_sync
            hb = []
            for _ in range(3):
                old, new = self.states[self.i % 2], self.states[(self.i + 1) % 2]
                torch.cuda.synchronize()
                ta = time.perf_counter()
                data = crukx_sync.encode_update(old, new, self.send_chk)
                tb = time.perf_counter()
                crukx_sync.apply_update(self.recv, data, self.recv_chk)
                torch.cuda.synchronize()
                hb.append((tb - ta, time.perf_counter() - tb))
                self.i += 1
            self.exact()
            out["host_bytes_encode_ms"] = round(min(x[0] for x in hb) * 1e3, 3)
            out["host_bytes_apply_ms"] = round(min(x[1] for x in hb) * 1e3, 3)
            # the reference's own step shape: bytes out of encode_update and into apply_update, the
            # checksum caches only (the receiver's exponent counts are not kept across updates)
            from crukx_sync import codec
            codec._COUNT_CACHE = False
            ref = []
            try:
                for _ in range(3):
                    old, new = self.states[self.i % 2], self.states[(self.i + 1) % 2]
                    torch.cuda.synchronize()
                    ta = time.perf_counter()
                    data = crukx_sync.encode_update(old, new, self.send_chk)
                    tb = time.perf_counter()
                    crukx_sync.apply_update(self.recv, data, self.recv_chk)
                    torch.cuda.synchronize()
                    ref.append((tb - ta, time.perf_counter() - tb))
                    self.i += 1
            finally:
                codec._COUNT_CACHE = True
            self.exact()
            e, a = sorted(x[0] for x in ref)[1], sorted(x[1] for x in ref)[1]
            out["reference_api_ms"] = {"encode": round(e * 1e3, 3), "apply": round(a * 1e3, 3),
                                       "step": round((e + a) * 1e3, 3),
                                       "shape": "encode_update -> bytes -> apply_update(bytes), checksum caches on "
                                                "both sides, no receiver exponent-count cache (median of 3)"}
            log(f"[bench] reference API shape (bytes, checksum caches only): encode {e * 1e3:.2f} ms, "
                f"apply {a * 1e3:.2f} ms")
        return out


def other_config(torch, dev, workload, rho, args, base=None):
    """The same measurement (no first-call step) on another workload or density."""
    from crukx_sync import workloads
    shapes = workloads.shapes_for(workload)
    n = workloads.numel(shapes)
    A = base if base is not None else workloads.make_weights(shapes, seed=0, device=dev)
    B = workloads.make_step(A, 1, rho=rho, p_one=args.p_one, seed=0)
    run = Run(A, B, n)
    res = run.measure(5, 2, 3)
    dom = res["dominant"]
    out = {"weights": n, "rho": rho, "ms_per_step": round(res["ms_step"], 3), "encode_ms": res["encode_ms"],
           "apply_ms": res["apply_ms"], "cold2_encode_ms": res["cold2_encode_ms"],
           "cold2_apply_ms": res["cold2_apply_ms"], "changes": res["changes"], "update_bytes": res["update_bytes"],
           "dominant": dom, "dominant_frac": round(alg_bytes(dom, n, res["changes"]) / (res["dominant_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
           "streaming_kernels": {k: {"ms": round(v, 4), "frac": round(alg_bytes(k, n, res["changes"]) / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
                                 for k, v in res["kernels"].items() if k in STREAMING},
           "kernels_ms_per_step": {k: round(v, 4) for k, v in sorted(res["kernels"].items()) if not k.startswith("host:")}}
    log(f"[bench] {workload} rho={rho}: {out['ms_per_step']:.3f} ms/step (encode {out['encode_ms']:.3f}, "
        f"apply {out['apply_ms']:.3f}); {dom} at {out['dominant_frac']:.3f} of peak")
    del run, A, B
    torch.cuda.empty_cache()
    return out


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


def cpu_info() -> dict:
    """The host's CPU as lscpu reports it, and the CPUs this process may run on."""
    import subprocess
    info = {"model": cpu_model()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {k.strip(): v.strip() for k, v in (l.split(":", 1) for l in out.splitlines() if ":" in l)}
        sockets, cores = int(kv.get("Socket(s)", 0)), int(kv.get("Core(s) per socket", 0))
        info.update({"model": kv.get("Model name", info["model"]), "sockets": sockets, "cores_per_socket": cores,
                     "threads_per_core": int(kv.get("Thread(s) per core", 0)), "logical_cpus": int(kv.get("CPU(s)", 0)),
                     "physical_cores": sockets * cores})
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    info["cpus_available"] = len(os.sched_getaffinity(0))
    return info


def cpu_threads(args) -> int:
    """Threads of the CPU baseline: the physical cores, within the CPUs this process may use and the
    16 host CPUs that go with one GPU here (--cpu-threads overrides)."""
    if args.cpu_threads:
        return args.cpu_threads
    info = cpu_info()
    cores = info.get("physical_cores") or info["cpus_available"]
    return max(1, min(cores, info["cpus_available"], 16))


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


def cpu_baseline(args, shapes, A, B, N):
    """The reference's CPU path (torch-CPU restatement) on the first decoder layers of the same update,
    one warm step (caches as on the GPU), timed on the host cores and scaled to the whole update.
    The sample is also encoded on the GPU and by the C oracle: all three byte strings must agree."""
    import torch

    import crukx_sync
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import torch_cpu

    threads = cpu_threads(args)
    torch.set_num_threads(threads)
    layers = args.cpu_baseline_layers
    names = [n for n, _, _ in shapes if any(n.startswith(f"model.layers.{i}.") for i in range(layers))]
    if not names:  # small workloads: the whole state dict
        names = [n for n, _, _ in shapes]
    old = {n: A[n].cpu() for n in names}
    new = {n: B[n].cpu() for n in names}
    n_sample = sum(v.numel() for v in old.values())
    cache = {n: oracle.checksum(v) for n, v in old.items()}  # warm caches, as in the GPU steps
    gpu = crukx_sync.encode_update({n: A[n] for n in names}, {n: B[n] for n in names}, dict(cache))
    t0 = time.perf_counter()
    data = torch_cpu.encode_update(old, new, dict(cache))
    t1 = time.perf_counter()
    recv = {n: v.clone() for n, v in old.items()}
    torch_cpu.apply_update(recv, data, dict(cache))
    t2 = time.perf_counter()
    for n in names:
        assert torch.equal(recv[n].view(torch.int16), new[n].view(torch.int16)), n
    t3 = time.perf_counter()
    ref = oracle.encode_update(old, new, dict(cache))
    t4 = time.perf_counter()
    oracle.apply_update({n: v.clone() for n, v in old.items()}, ref, dict(cache))
    t5 = time.perf_counter()
    assert data == ref == gpu, "the sample's bytes differ between the GPU, the torch restatement and the oracle"
    scale = N / n_sample
    ms = (t2 - t0) * scale * 1e3
    log(f"[bench] torch-cpu restatement on {n_sample:,} weights ({threads} threads): encode {t1 - t0:.2f}s "
        f"apply {t2 - t1:.2f}s -> {ms / 1e3:.1f}s per full update; C oracle (1 thread) encode {t4 - t3:.2f}s "
        f"apply {t5 - t4:.2f}s; {len(data):,} bytes identical on GPU, restatement and oracle")
    small4 = small4_chain(threads)
    value, sample = ms, (f"decoder layers 0..{layers - 1} of the same synthetic update ({n_sample} of {N} weights, "
                         f"warm checksum caches), one encode + one apply on {threads} threads of {cpu_model()}, "
                         f"time scaled by {scale:.2f} to the whole update")
    out = {"unit": "ms", "cores": threads, "kind": "port",
           "impl": "torch-CPU restatement of the reference's CPU path (oracle/torch_cpu.py): slab-wise stable "
                   "argsort ranking (small tensors in shared sorts), 256-step vectorised block decode, index_put_ "
                   "scatter",
           "host": cpu_info(), "cap_s": args.cpu_cap_s,
           "layers_sample": {"weights": n_sample, "encode_s": round(t1 - t0, 3), "apply_s": round(t2 - t1, 3),
                             "scaled_ms": round(ms, 1), "bytes_identical": True},
           "c_oracle_1_thread": {"sample_encode_s": round(t4 - t3, 3), "sample_apply_s": round(t5 - t4, 3),
                                 "value_ms": round((t5 - t3) * scale * 1e3, 1)},
           "small4_chain": small4}
    if args.cpu_baseline != "sample":
        warm = whole_update_step(args, threads, A, B, names=[n for n, _, _ in shapes])
        out["whole_update_warm"] = warm
        if not warm["capped"]:  # the whole update measured: no scaling
            value = (warm["encode_s"] + warm["apply_s"]) * 1e3
            sample = (f"the whole update: one warm step (checksum caches on both sides), encode and apply, on "
                      f"{threads} threads of {cpu_model()}; bytes identical to the GPU's")
        out["qwen2.5-1.5b_chain"] = cpu_chain(args, threads, "qwen2.5-1.5b", 7)
        if args.cpu_baseline == "full":
            out["qwen2.5-7b_cold"] = cpu_chain(args, threads, "qwen2.5-7b", 1)
    out["value"] = round(value, 1)
    out["sample"] = sample
    return out


def whole_update_step(args, threads, A, B, names):
    """One warm step of the restatement over the whole update the GPU steps run (every tensor, embed and
    lm_head included): both checksum caches hold the old state's checksums (computed on the GPU), encode
    and apply timed apart, each under the wall-clock cap; bytes compared with the GPU's, the receiver
    compared with the new state."""
    import torch

    import crukx_sync
    from crukx_sync import codec
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import torch_cpu

    t0 = time.perf_counter()
    old = {n: A[n].cpu() for n in names}
    new = {n: B[n].cpu() for n in names}
    cache = {n: codec.checksum(A[n]) for n in names}
    gpu = crukx_sync.encode_update(A, B, dict(cache))
    recv = {n: v.clone() for n, v in old.items()}
    log(f"[cpu] whole update on the host in {time.perf_counter() - t0:.1f}s; warm step on {threads} threads")
    ta = time.perf_counter()
    data = torch_cpu.encode_update(old, new, dict(cache))
    tb = time.perf_counter()
    assert data == gpu, "whole update: the restatement's bytes differ from the GPU's"
    row = {"weights": sum(v.numel() for v in old.values()), "tensors": len(names), "caches": True,
           "encode_s": round(tb - ta, 3), "bytes_identical": True, "capped": tb - ta > args.cpu_cap_s}
    log(f"[cpu] whole update, warm: encode {tb - ta:.2f}s, {len(data):,} bytes identical to the GPU's")
    if not row["capped"]:
        torch_cpu.apply_update(recv, data, dict(cache))
        tc = time.perf_counter()
        row["apply_s"] = round(tc - tb, 3)
        row["capped"] = tc - tb > args.cpu_cap_s
        for n in names:
            assert torch.equal(recv[n].view(torch.int16), new[n].view(torch.int16)), n
        log(f"[cpu] whole update, warm: apply {tc - tb:.2f}s; receiver equals the new state")
    return row


def cpu_chain(args, threads, workload, steps):
    """The restatement over `steps` chained steps of a whole workload (the first without caches, the
    rest with both checksum caches), encode and apply timed apart, each phase under the wall-clock cap
    (a phase past it ends the chain, reported as capped).  Every step's bytes are compared with the
    GPU's, and the receiver with the last state."""
    import torch

    import crukx_sync
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import torch_cpu
    from crukx_sync import workloads

    cap = args.cpu_cap_s
    shapes = workloads.shapes_for(workload)
    n = workloads.numel(shapes)
    t0 = time.perf_counter()
    prev_g = workloads.make_weights(shapes, seed=0, device="cuda")
    prev = {k: v.cpu() for k, v in prev_g.items()}
    recv = {k: v.clone() for k, v in prev.items()}
    log(f"[cpu] {workload}: {n:,} weights on the host in {time.perf_counter() - t0:.1f}s")
    send_c, recv_c, send_g = {}, {}, {}
    rows = []
    for k in range(1, steps + 1):
        cur_g = workloads.make_step(prev_g, k, rho=0.01, p_one=args.p_one, seed=0)
        cur = {kk: v.cpu() for kk, v in cur_g.items()}
        gpu = crukx_sync.encode_update(prev_g, cur_g, send_g)
        ta = time.perf_counter()
        data = torch_cpu.encode_update(prev, cur, send_c)
        tb = time.perf_counter()
        assert data == gpu, f"{workload} step {k}: the restatement's bytes differ from the GPU's"
        row = {"step": k, "caches": k > 1, "encode_s": round(tb - ta, 3), "bytes_identical": True,
               "capped": tb - ta > cap}
        log(f"[cpu] {workload} step {k}: encode {tb - ta:.2f}s, {len(data):,} bytes identical to the GPU's")
        rows.append(row)
        if row["capped"]:
            break
        torch_cpu.apply_update(recv, data, recv_c)
        tc = time.perf_counter()
        row["apply_s"] = round(tc - tb, 3)
        row["capped"] = tc - tb > cap
        log(f"[cpu] {workload} step {k} ({'warm' if k > 1 else 'cold'}): apply {tc - tb:.2f}s on {threads} threads")
        prev, prev_g = cur, cur_g
        if row["capped"]:
            break
    done = not any(r["capped"] for r in rows)
    if done:
        for kk in recv:
            assert torch.equal(recv[kk].view(torch.int16), prev[kk].view(torch.int16)), kk
    del prev, recv, prev_g
    torch.cuda.empty_cache()
    out = {"weights": n, "threads": threads, "steps": rows, "receiver_equal": done}
    warm = [r for r in rows if r["caches"] and not r["capped"]]
    if warm:
        med = sorted(r["encode_s"] + r["apply_s"] for r in warm)[len(warm) // 2]
        out["warm_median_ms"] = round(med * 1e3, 1)
        out["warm_mean_ms"] = round(sum(r["encode_s"] + r["apply_s"] for r in warm) / len(warm) * 1e3, 1)
    return out


def small4_chain(threads):
    """The reference's CPU plumbing case in full: four tensors (26,611,713 weights), three chained
    steps with both checksum caches, through the torch-CPU restatement on the host threads and through
    the GPU (bytes API); every step's bytes must be identical, and both receivers end equal to the
    last state."""
    import torch

    import crukx_sync
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import torch_cpu
    from crukx_sync import workloads

    states = [workloads.make_weights(workloads.small4_shapes(), seed=0, device="cuda")]
    for k in range(1, 4):
        states.append(workloads.make_step(states[-1], k, rho=0.01, p_one=0.87, seed=0))
    host = [{n: v.cpu() for n, v in st.items()} for st in states]
    send_g, recv_g, send_c, recv_c = {}, {}, {}, {}
    w_gpu = {n: v.clone() for n, v in states[0].items()}
    w_cpu = {n: v.clone() for n, v in host[0].items()}
    cpu_enc, cpu_app, gpu_step = [], [], []
    for k in range(1, 4):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        data = crukx_sync.encode_update(states[k - 1], states[k], send_g)
        crukx_sync.apply_update(w_gpu, data, recv_g)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ref = torch_cpu.encode_update(host[k - 1], host[k], send_c)
        t2 = time.perf_counter()
        torch_cpu.apply_update(w_cpu, ref, recv_c)
        t3 = time.perf_counter()
        assert ref == data, f"small4 step {k}: the restatement's bytes differ from the GPU's"
        gpu_step.append(t1 - t0)
        cpu_enc.append(t2 - t1)
        cpu_app.append(t3 - t2)
    for n in w_cpu:
        assert torch.equal(w_cpu[n].view(torch.int16), host[3][n].view(torch.int16)), n
        assert torch.equal(w_gpu[n].view(torch.int16), states[3][n].view(torch.int16)), n
    log(f"[bench] small4 chain (26,611,713 weights, 3 steps): torch-cpu restatement encode "
        + " ".join(f"{x:.3f}" for x in cpu_enc) + " s, apply " + " ".join(f"{x:.3f}" for x in cpu_app)
        + " s; GPU (bytes API) " + " ".join(f"{x * 1e3:.2f}" for x in gpu_step) + " ms per step; bytes identical")
    return {"weights": 26611713, "steps": 3, "threads": threads, "cpu_encode_s": [round(x, 4) for x in cpu_enc],
            "cpu_apply_s": [round(x, 4) for x in cpu_app], "gpu_bytes_api_step_ms": [round(x * 1e3, 3) for x in gpu_step],
            "bytes_identical": True}


if __name__ == "__main__":
    main()

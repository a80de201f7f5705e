"""Benchmark: deterministic causal flash attention fwd+bwd on one MI355X.

Workload: B=4, H=16, S=2048, D=128, causal,
bf16 Q/K/V after RoPE (theta 10000), bf16 upstream gradient dO ~ N(0, 1).
One step = one forward (O, LSE) and one backward (dQ, dK, dV) through the
library's C ABI, with every input already resident in HBM.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-verify]

The attention workloads run with the score cache (the forward stores the
scaled scores, the dK/dV kernel reads them instead of recomputing Q K^T; same
bytes) unless --no-score-cache is given.

Prints ONE JSON line.  ``value`` is the algorithmic TFLOP/s of fwd+bwd
(FlashAttention convention: 14*D FLOP per unmasked causal pair, whatever the
kernels recompute or cache).  ``roofline`` covers the dominant phase, timed live with HIP
events recorded on the stream the kernels are launched on; ``cpu_baseline``
times the CPU oracle (this project's C restatement of the contract) on the
host cores over a bounded sample of the same workload.  The GPU result is
checked byte for byte against the CPU oracle on sample heads before the line
is printed.
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix / packed-VALU peak


def committed_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (profiles/attn_c2_traffic.md), or None if absent."""
    path = ROOT / "profiles" / "attn_c2_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 4 and cells[0] == f"`{kernel}`":
            return int(cells[3])
    return None


def host_box() -> dict:
    """What the CPU baseline ran on: the host's logical CPU count, the CPUs this
    process may use, the CPU model string and OMP_NUM_THREADS."""
    model = None
    try:
        for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"nproc": os.cpu_count(), "usable_cpus": usable, "cpu_model": model,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_threads() -> tuple[int, str]:
    """Threads for the CPU oracle and the reason for the count.  A one-GPU box
    grants its job a 16-CPU share of the host (OMP_NUM_THREADS is set to it), so
    the baseline uses every CPU of that share, and no more than the process may
    run on."""
    box = host_box()
    usable = box["usable_cpus"] or 1
    omp = box["omp_num_threads"]
    share = int(omp) if omp and omp.isdigit() and int(omp) > 0 else 16
    n = max(1, min(usable, share))
    why = (f"{n} threads = the job's CPU share (OMP_NUM_THREADS={omp}, {usable} usable of {box['nproc']} "
           f"logical CPUs, {box['cpu_model']})")
    return n, why


def median_time(fn, runs: int = 3) -> tuple[float, list, object]:
    """Median wall time (s) of ``runs`` calls of fn, every time, and the last result."""
    times, res = [], None
    for _ in range(runs):
        c0 = time.perf_counter()
        res = fn()
        times.append(time.perf_counter() - c0)
    return sorted(times)[len(times) // 2], times, res


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # Default: about 0.1 s of warm-up for the attention and loss workloads (the
    # first milliseconds of work run below the sustained clock: 3 warm-up steps
    # read 5 % slower than 30), 3 steps for the layer and model workloads.
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline leg")
    ap.add_argument("--no-verify", action="store_true", help="skip the byte comparison against the oracle")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="before the steps, run one plain device-to-device copy of MIB MiB (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    ap.add_argument("--workload", choices=("attention", "int8pv", "layer", "loss", "model"), default="attention",
                    help="attention: BASELINE configuration 2 (the headline); int8pv: the same shape through "
                         "int8pv_causal_flash_attention (int8 P.V forward, binary32 backward); layer: "
                         "configuration 5, the decoder layer around the kernel (fwd+bwd of RMSNorm, projections, "
                         "RoPE, attention, SwiGLU); loss: the fused cross-entropy + z-loss fwd+bwd on the "
                         "OPEN-1B lm-head logits (N 8192 x V 128256 bf16); model: one training step (fwd, "
                         "fused loss, bwd) of the OPEN-1B proxy model, B4 x T2048 tokens")
    ap.add_argument("--no-score-cache", action="store_true",
                    help="attention workloads: recompute Q K^T in the backward instead of reading the forward's "
                         "score cache (same bytes, less memory)")
    ap.add_argument("--ac", choices=("none", "wrapper", "cached"), default="none",
                    help="--workload model: activation checkpointing of every block, as the reference applies it "
                         "(parallelize_llama3_repop.py:107-130): checkpoint_wrapper without (wrapper) or with "
                         "(cached) the attention-recording context_fn")
    ap.add_argument("--config", choices=("c1", "c2", "c3", "c4", "open1b"), default="c2",
                    help="attention workload: BASELINE configuration (c2 = the headline; c1 = fp32 forward only "
                         "B1 H4 S256 D64; c3 = B1 H16 S8192 D128 with Q, K x 3, also checks 5 repeats; c4 = H16 "
                         "S1024 D128 at --batch sequences); open1b = the OPEN-1B training attention (B4 H16 Hkv4 "
                         "D128, int8-PV forward, binary32 backward) at S 2048/4096 and window 0/512")
    ap.add_argument("--seq", type=int, default=0, help="--config open1b: only this S (2048 or 4096)")
    ap.add_argument("--window", type=int, default=None, help="--config open1b: only this window (0 or 512)")
    ap.add_argument("--batch", type=int, default=16, help="sequences for --config c4 (1, 2, 8 or 16)")
    ap.add_argument("--cpu-batches", type=int, default=4,
                    help="sequences (all heads each) in the CPU sample and the byte check; 4 = the whole batch")
    ap.add_argument("--cpu-runs", type=int, default=3, help="CPU baseline: median of this many timed runs")
    return ap.parse_args()


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py: --gpus {args.gpus} is not supported: this build measures one GPU's share "
            "(attention shards over (batch, head) with no exchange between GPUs).",
            file=sys.stderr,
        )
        return 2

    import numpy as np
    import torch

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    from open_transformers_amd import _lib, synthetic

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    pkg.require_backend(dev, pkg.build_info())
    if args.warmup is None:
        args.warmup = 3 if args.workload in ("layer", "model") else 50
    if args.workload == "layer":
        return bench_layer(args, torch, dev)
    if args.workload == "loss":
        return bench_loss(args, torch, dev)
    if args.workload == "model":
        return bench_model(args, torch, dev)

    if args.workload == "attention" and args.config == "open1b":
        return bench_open1b(args, torch, dev)
    if args.workload == "attention" and args.config != "c2":
        return bench_attention_config(args, torch, dev)

    int8pv = args.workload == "int8pv"
    cfg = synthetic.CONFIGS["c2"]
    B, H, Hkv, S, D = cfg["B"], cfg["H"], cfg["Hkv"], cfg["S"], cfg["D"]
    window = 0
    t0 = time.time()
    inp = synthetic.make_inputs(B, H, Hkv, S, D, dtype="bf16", seed=2024, rope_theta=cfg["rope_theta"])
    print(f"bench: inputs ready in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    t = {n: torch.from_numpy(inp[n]).to(torch.bfloat16).to(dev) for n in ("q", "k", "v", "do")}
    q, k, v, do = t["q"], t["k"], t["v"], t["do"]

    stream = torch.cuda.current_stream(dev)
    lib = _lib.load()
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws_bytes = int(lib.otx_attn_bwd_workspace_bytes(B, H, Hkv, S, D, window))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)  # the caching allocator returns 256-byte aligned blocks
    ws8_bytes = int(lib.otx_attn_fwd_int8pv_workspace_bytes(B, H, Hkv, S, D))
    ws8 = torch.empty(ws8_bytes, dtype=torch.uint8, device=dev) if int8pv else None
    use_sc = not args.no_score_cache
    sc_bytes = int(lib.otx_attn_score_cache_bytes(B, H, S, window))
    sc = torch.empty(sc_bytes // 4, dtype=torch.float32, device=dev) if use_sc else None
    sid = stream.cuda_stream
    BF16 = _lib.DTYPE_BF16

    if args.copy_probe > 0:
        # A plain device-to-device copy of known size: the reference reading for
        # the FETCH_SIZE / WRITE_SIZE counters of a kernel profile of this run.
        src = torch.empty(args.copy_probe << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # One step = forward + the three backward launches, each bracketed by events
    # on the launch stream: [fwd] [Dsum] [dK/dV] [dQ].
    names = ("fwd", "dsum", "dkdv", "dq")

    def step(ev):
        ev[0].record(stream)
        if int8pv and use_sc:
            _lib.check(lib.otx_attn_fwd_int8pv_sc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                                  lse.data_ptr(), sc.data_ptr(), sc_bytes, B, H, Hkv, S, D, window,
                                                  BF16, ws8.data_ptr(), ws8_bytes, 0, sid), "fwd int8pv")
        elif int8pv:
            _lib.check(lib.otx_attn_fwd_int8pv(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                               lse.data_ptr(), B, H, Hkv, S, D, window, BF16, ws8.data_ptr(),
                                               ws8_bytes, sid), "fwd int8pv")
        elif use_sc:
            _lib.check(lib.otx_attn_fwd_sc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                           sc.data_ptr(), sc_bytes, B, H, Hkv, S, D, window, BF16, 0, sid), "fwd")
        else:
            _lib.check(lib.otx_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                        B, H, Hkv, S, D, window, BF16, sid), "fwd")
        ev[1].record(stream)
        for i, mask in enumerate((1, 2, 4)):
            ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), do.data_ptr(),
                    dq.data_ptr(), dk.data_ptr(), dv.data_ptr())
            if use_sc:
                rc = lib.otx_attn_bwd_sc(*ptrs, sc.data_ptr(), sc_bytes, B, H, Hkv, S, D, window, BF16,
                                         ws.data_ptr(), ws_bytes, 0, mask, sid)
            else:
                rc = lib.otx_attn_bwd_stages(*ptrs, B, H, Hkv, S, D, window, BF16, ws.data_ptr(), ws_bytes, 0, mask,
                                             sid)
            _lib.check(rc, "bwd")
            ev[2 + i].record(stream)

    def events():
        return [torch.cuda.Event(enable_timing=True) for _ in range(5)]

    for _ in range(args.warmup):
        step(events())
    torch.cuda.synchronize()

    # Timed region: K steps.
    evs = [events() for _ in range(args.steps)]
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for s in range(args.steps):
        step(evs[s])
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    out = (o, lse, dq, dk, dv)

    kern_ms = {n: sum(e[i].elapsed_time(e[i + 1]) for e in evs) / args.steps for i, n in enumerate(names)}
    ms_per_step = wall * 1e3 / args.steps
    fwd_avg = kern_ms["fwd"]
    bwd_avg = kern_ms["dsum"] + kern_ms["dkdv"] + kern_ms["dq"]

    flops_all = synthetic.attention_flops(B, H, S, D, window, backward=True)
    tflops = flops_all / (ms_per_step * 1e-3) / 1e12

    # Byte comparison against the CPU oracle on sample heads (full S, full D).
    verified = None
    cpu = None
    o, lse, dq, dk, dv = (x.float().cpu().numpy() for x in out)
    if not args.no_verify or not args.no_cpu:
        from oracle import oracle as orc

        nb = max(1, min(args.cpu_batches, B))
        sl = {n: np.ascontiguousarray(a[0:nb]) for n, a in inp.items()}
        nthreads, why = cpu_threads()
        fwd_ref = orc.attn_fwd_int8pv if int8pv else orc.attn_fwd

        def cpu_step():
            ro, rlse = fwd_ref(sl["q"], sl["k"], sl["v"], window=window, out_bf16=True, nthreads=nthreads)
            return (ro, rlse) + orc.attn_bwd(sl["q"], sl["k"], sl["v"], ro, rlse, sl["do"], window=window,
                                             out_bf16=True, nthreads=nthreads)

        cpu_s, cpu_all, (ro, rlse, rdq, rdk, rdv) = median_time(cpu_step, args.cpu_runs)
        sample_flops = synthetic.attention_flops(nb, H, S, D, window, backward=True)
        cpu = {
            "value": round(sample_flops / cpu_s / 1e12, 6),
            "unit": "TFLOP/s",
            "cores": nthreads,
            "kind": "port",
            "sample": f"sequences 0..{nb - 1} (all {H} heads) of the same inputs, fwd+bwd; median of "
                      f"{len(cpu_all)} runs {cpu_s:.2f} s (all: {', '.join(f'{x:.2f}' for x in cpu_all)} s); {why}",
            "box": host_box(),
        }
        if not args.no_verify:
            pairs = (("o", o, ro), ("lse", lse, rlse), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv))
            verified = True
            for name, got, ref in pairs:
                g = np.ascontiguousarray(got[0:nb]).view(np.uint32)
                if not np.array_equal(g, ref.view(np.uint32)):
                    bad = int(np.count_nonzero(g != ref.view(np.uint32)))
                    print(f"bench: {name} differs from the CPU oracle in {bad} elements", file=sys.stderr)
                    verified = False

    # Dominant kernel for the roofline entry: algorithmic FLOPs of that launch
    # (FlashAttention split of the 14*D per causal pair: forward 4*D, dK/dV 8*D
    # = QK^T recompute + dP + dV + dK, dQ 2*D) over its event-timed duration.
    # With the score cache the dK/dV launch does no QK^T: 6*D per pair.
    pairs = synthetic.causal_pairs(B, H, S, window)
    kflops = {"fwd": 4 * D * pairs, "dkdv": (6 if use_sc else 8) * D * pairs, "dq": 2 * D * pairs, "dsum": 0}
    dom = max(("fwd", "dkdv", "dq"), key=lambda n: kern_ms[n])
    dom_kernel = {"fwd": "attn_fwd_bf16_kernel", "dkdv": "attn_dkdv_bf16_kernel", "dq": "attn_dq_kernel"}[dom]
    achieved = kflops[dom] / (kern_ms[dom] * 1e-3) / 1e12
    traffic = committed_traffic(dom_kernel)
    line = {
        "metric": ("attn int8-PV fwd + binary32 bwd TFLOP/s (bit-exact vs CPU contract oracle) at B4 H16 S2048 D128"
                   if int8pv else "attn fwd+bwd TFLOP/s (bit-exact vs CPU contract oracle) at B4 H16 S2048 D128"),
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32+i8" if int8pv else "f32",
        "data": "synthetic (Philox N(0,1), RoPE theta 10000, bf16 storage)",
        "config": {"workload": ("int8-PV causal attention fwd + straight-through bwd B4 H16 S2048 D128 bf16"
                                if int8pv else "causal attention fwd+bwd B4 H16 S2048 D128 bf16 (BASELINE config 2)"),
                   "B": B, "H": H, "Hkv": Hkv, "S": S, "D": D, "window": window,
                   "score_cache_bytes": sc_bytes if use_sc else 0},
        "bit_exact_vs_oracle": verified,
        "phase_ms": {"fwd": round(fwd_avg, 4), "bwd": round(bwd_avg, 4)},
        "kernel_ms": {n: round(x, 4) for n, x in kern_ms.items()},
        "roofline": {
            "bound": "mfma",
            "kernel": dom_kernel,
            "achieved": round(achieved, 3),
            "peak": FP32_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0 if verified in (None, True) else 3


def bench_attention_config(args, torch, dev) -> int:
    """BASELINE configurations 1, 3 and 4 through the C ABI (score cache on for bf16
    unless --no-score-cache): time the step, check every output byte of the
    first sequences against the CPU oracle and, for configuration 3, that five
    repeated steps give identical bytes."""
    import numpy as np

    from open_transformers_amd import _lib, synthetic

    name = args.config
    cfg = dict(synthetic.CONFIGS[name])
    if name == "c4":
        cfg["B"] = args.batch
    B, H, Hkv, S, D = cfg["B"], cfg["H"], cfg["Hkv"], cfg["S"], cfg["D"]
    fp32 = cfg["dtype"] == "f32"
    backward = name != "c1"  # configuration 1 is the forward only
    window = 0
    inp = synthetic.make_inputs(B, H, Hkv, S, D, dtype=cfg["dtype"], seed=2024, rope_theta=cfg["rope_theta"],
                                qk_scale=cfg["qk_scale"])
    tdt = torch.float32 if fp32 else torch.bfloat16
    t = {n: torch.from_numpy(inp[n]).to(tdt).to(dev) for n in ("q", "k", "v", "do")}
    q, k, v, do = t["q"], t["k"], t["v"], t["do"]
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    sid = stream.cuda_stream
    dt = _lib.DTYPE_F32 if fp32 else _lib.DTYPE_BF16
    o, lse = torch.empty_like(q), torch.empty((B, H, S), dtype=torch.float32, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws_bytes = int(lib.otx_attn_bwd_workspace_bytes(B, H, Hkv, S, D, window))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    use_sc = backward and not fp32 and not args.no_score_cache
    sc_bytes = int(lib.otx_attn_score_cache_bytes(B, H, S, window))
    sc = torch.empty(sc_bytes // 4, dtype=torch.float32, device=dev) if use_sc else None
    ptrs = lambda: (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), do.data_ptr(),
                    dq.data_ptr(), dk.data_ptr(), dv.data_ptr())

    def step():
        if use_sc:
            _lib.check(lib.otx_attn_fwd_sc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                           sc.data_ptr(), sc_bytes, B, H, Hkv, S, D, window, dt, 0, sid), "fwd")
            _lib.check(lib.otx_attn_bwd_sc(*ptrs(), sc.data_ptr(), sc_bytes, B, H, Hkv, S, D, window, dt,
                                           ws.data_ptr(), ws_bytes, 0, 7, sid), "bwd")
            return
        _lib.check(lib.otx_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                    B, H, Hkv, S, D, window, dt, sid), "fwd")
        if backward:
            _lib.check(lib.otx_attn_bwd(*ptrs(), B, H, Hkv, S, D, window, dt, ws.data_ptr(), ws_bytes, sid), "bwd")

    steps = args.steps * (50 if name == "c1" else 1)  # configuration 1 is a 10-microsecond launch
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    names = ("o", "lse", "dq", "dk", "dv") if backward else ("o", "lse")
    grab = lambda: {n: x.float().cpu().numpy() for n, x in zip(("o", "lse", "dq", "dk", "dv"), (o, lse, dq, dk, dv))
                    if n in names}
    got = grab()
    repeats_identical = None
    if name == "c3":  # five runs, byte-identical
        repeats_identical = True
        for _ in range(4):
            step()
            torch.cuda.synchronize()
            again = grab()
            repeats_identical &= all(np.array_equal(again[n].view(np.uint32), got[n].view(np.uint32)) for n in names)
    flops = synthetic.attention_flops(B, H, S, D, window, backward=backward)
    verified, cpu = None, None
    if not args.no_verify or not args.no_cpu:
        from oracle import oracle as orc

        nb = max(1, min(args.cpu_batches, B))
        sl = {n: np.ascontiguousarray(a[0:nb]) for n, a in inp.items()}
        nthreads, why = cpu_threads()

        def cpu_step():
            ro, rlse = orc.attn_fwd(sl["q"], sl["k"], sl["v"], window=window, out_bf16=not fp32, nthreads=nthreads)
            r = {"o": ro, "lse": rlse}
            if backward:
                r["dq"], r["dk"], r["dv"] = orc.attn_bwd(sl["q"], sl["k"], sl["v"], ro, rlse, sl["do"],
                                                         window=window, out_bf16=not fp32, nthreads=nthreads)
            return r

        cpu_s, cpu_all, ref = median_time(cpu_step, args.cpu_runs)
        cpu = {"value": round(synthetic.attention_flops(nb, H, S, D, window, backward=backward) / cpu_s / 1e12, 6),
               "unit": "TFLOP/s", "cores": nthreads, "kind": "port",
               "sample": f"sequences 0..{nb - 1} (all {H} heads) of the same inputs, "
                         f"{'fwd+bwd' if backward else 'fwd'}; median of {len(cpu_all)} runs {cpu_s:.2f} s "
                         f"(all: {', '.join(f'{x:.2f}' for x in cpu_all)} s); {why}",
               "box": host_box()}
        if not args.no_verify:
            verified = all(np.array_equal(np.ascontiguousarray(got[n][0:nb]).view(np.uint32),
                                          ref[n].view(np.uint32)) for n in names)
    what = {"c1": "causal attention fwd B1 H4 S256 D64 fp32 (BASELINE config 1)",
            "c3": "causal attention fwd+bwd B1 H16 S8192 D128 bf16, Q/K x 3 (BASELINE config 3)",
            "c4": f"causal attention fwd+bwd B{B} H16 S1024 D128 bf16 (BASELINE config 4)"}[name]
    line = {
        "metric": f"attn {'fwd+bwd' if backward else 'fwd'} TFLOP/s (bit-exact vs CPU contract oracle), {what}",
        "value": round(flops / (ms * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (Philox N(0,1)" + (", Q/K x 3" if name == "c3" else "") + ")",
        "config": {"workload": what, "B": B, "H": H, "Hkv": Hkv, "S": S, "D": D, "window": window,
                   "score_cache_bytes": sc_bytes if use_sc else 0},
        "bit_exact_vs_oracle": verified,
        "repeats_identical": repeats_identical,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0 if verified in (None, True) and repeats_identical in (None, True) else 3


def bench_open1b(args, torch, dev) -> int:
    """The OPEN-1B training attention (configs/model/llama3_1b_proxy_repop.yaml:
    16 x 128 query heads, 4 KV heads, window 512 on four of five layers,
    int8-PV forward; configs/train/1b_repop_v2.yaml: micro-batch 4 x T4096),
    at S 2048 and 4096, window 0 and 512.  One step = the int8-PV forward
    (with the score cache) and the binary32 straight-through backward, timed
    per launch with HIP events on the launch stream.  ``value`` is the
    FlashAttention-convention rate of the four cases together (4*D + 10*D per
    unmasked pair, the forward's P.V counted although it runs as int8
    operations); each case carries its own per-kernel rooflines."""
    import numpy as np

    from open_transformers_amd import _lib, synthetic

    B, H, Hkv, D = 4, 16, 4, 128
    cases = [(2048, 0), (2048, 512), (4096, 0), (4096, 512)]
    if args.seq:
        cases = [c for c in cases if c[0] == args.seq]
    if args.window is not None:
        cases = [c for c in cases if c[1] == args.window]
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    sid = stream.cuda_stream
    BF16 = _lib.DTYPE_BF16
    I8_PEAK_TOPS = 5000.0  # MI355X dense int8 matrix peak
    nthreads, why = cpu_threads()
    results, tot_flops, tot_ms, all_ok = [], 0.0, 0.0, True
    for S, window in cases:
        print(f"bench open1b: S={S} window={window}", file=sys.stderr, flush=True)
        inp = synthetic.make_inputs(B, H, Hkv, S, D, dtype="bf16", seed=2024, rope_theta=500000.0)
        t = {n: torch.from_numpy(inp[n]).to(torch.bfloat16).to(dev) for n in ("q", "k", "v", "do")}
        q, k, v, do = t["q"], t["k"], t["v"], t["do"]
        o, lse = torch.empty_like(q), torch.empty((B, H, S), dtype=torch.float32, device=dev)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        ws_bytes = int(lib.otx_attn_bwd_workspace_bytes(B, H, Hkv, S, D, window))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        ws8_bytes = int(lib.otx_attn_fwd_int8pv_workspace_bytes(B, H, Hkv, S, D))
        ws8 = torch.empty(ws8_bytes, dtype=torch.uint8, device=dev)
        sc_bytes = int(lib.otx_attn_score_cache_bytes(B, H, S, window))
        sc = torch.empty(sc_bytes // 4, dtype=torch.float32, device=dev)
        ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), do.data_ptr(),
                dq.data_ptr(), dk.data_ptr(), dv.data_ptr())

        def step(ev):
            ev[0].record(stream)
            _lib.check(lib.otx_attn_fwd_int8pv_sc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                                  lse.data_ptr(), sc.data_ptr(), sc_bytes, B, H, Hkv, S, D, window,
                                                  BF16, ws8.data_ptr(), ws8_bytes, 0, sid), "fwd int8pv")
            ev[1].record(stream)
            for i, mask in enumerate((1, 2, 4)):
                _lib.check(lib.otx_attn_bwd_sc(*ptrs, sc.data_ptr(), sc_bytes, B, H, Hkv, S, D, window, BF16,
                                               ws.data_ptr(), ws_bytes, 0, mask, sid), "bwd")
                ev[2 + i].record(stream)

        events = lambda: [torch.cuda.Event(enable_timing=True) for _ in range(5)]
        for _ in range(args.warmup):
            step(events())
        torch.cuda.synchronize()
        evs = [events() for _ in range(args.steps)]
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        for s in range(args.steps):
            step(evs[s])
        torch.cuda.synchronize()
        ms = (time.perf_counter() - w0) * 1e3 / args.steps
        names = ("fwd", "dsum", "dkdv", "dq")
        kern_ms = {n: sum(e[i].elapsed_time(e[i + 1]) for e in evs) / args.steps for i, n in enumerate(names)}
        pairs = synthetic.causal_pairs(B, H, S, window)
        flops = synthetic.attention_flops(B, H, S, D, window, backward=True)
        tot_flops += flops
        tot_ms += ms
        # Per-kernel floors: the forward's Q K^T chain on the binary32 matrix instruction (2*D per pair) plus its
        # int8 P.V (2*D int8 operations per pair); dK/dV 6*D (score cache: dP, dV, dK); dQ 2*D.
        floor_ms = {"fwd": (2 * D * pairs / (FP32_PEAK_TFLOPS * 1e12) + 2 * D * pairs / (I8_PEAK_TOPS * 1e12)) * 1e3,
                    "dkdv": 6 * D * pairs / (FP32_PEAK_TFLOPS * 1e12) * 1e3,
                    "dq": 2 * D * pairs / (FP32_PEAK_TFLOPS * 1e12) * 1e3}
        kflops = {"fwd": 2 * D * pairs, "dkdv": 6 * D * pairs, "dq": 2 * D * pairs}
        roof = {n: {"bound": "mfma", "achieved": round(kflops[n] / (kern_ms[n] * 1e-3) / 1e12, 3),
                    "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(floor_ms[n] / kern_ms[n], 4),
                    "floor_ms": round(floor_ms[n], 4)} for n in ("fwd", "dkdv", "dq")}
        roof["fwd"]["note"] = ("binary32 FLOP of Q K^T only (2*D per pair); frac = floor / time with the floor "
                               "= 2*D pairs at 157.3 TFLOP/s + 2*D pairs int8 operations at 5 POP/s")
        # Byte check of sequence 0 (all heads) against the CPU oracle: int8-PV forward, binary32 backward.
        ok, cpu = None, None
        if not args.no_verify:
            from oracle import oracle as orc

            sl = {n: np.ascontiguousarray(a[0:1]) for n, a in inp.items()}

            def cpu_step():
                ro, rlse = orc.attn_fwd_int8pv(sl["q"], sl["k"], sl["v"], window=window, out_bf16=True,
                                               nthreads=nthreads)
                return (ro, rlse) + orc.attn_bwd(sl["q"], sl["k"], sl["v"], ro, rlse, sl["do"], window=window,
                                                 out_bf16=True, nthreads=nthreads)

            runs = args.cpu_runs if (not args.no_cpu and (S, window) == (4096, 0)) else 1
            cpu_s, cpu_all, ref = median_time(cpu_step, runs)
            got = [x.float().cpu().numpy()[0:1] for x in (o, lse, dq, dk, dv)]
            ok = all(np.array_equal(np.ascontiguousarray(g).view(np.uint32), r.view(np.uint32))
                     for g, r in zip(got, ref))
            all_ok &= ok
            if runs > 1:
                cpu = {"value": round(synthetic.attention_flops(1, H, S, D, window) / cpu_s / 1e12, 6),
                       "unit": "TFLOP/s", "cores": nthreads, "kind": "port",
                       "sample": f"sequence 0 (all {H} heads) of this case, int8-PV fwd + binary32 bwd; median of "
                                 f"{len(cpu_all)} runs {cpu_s:.2f} s; {why}", "box": host_box()}
        results.append({"S": S, "window": window, "ms_per_step": round(ms, 4),
                        "tflops": round(flops / (ms * 1e-3) / 1e12, 3),
                        "kernel_ms": {n: round(x, 4) for n, x in kern_ms.items()}, "roofline": roof,
                        "bit_exact_vs_oracle": ok, "score_cache_bytes": sc_bytes, "cpu_baseline": cpu})
        del q, k, v, do, o, lse, dq, dk, dv, ws, ws8, sc, t
        torch.cuda.empty_cache()
    dom = max(results, key=lambda r: r["kernel_ms"]["dkdv"])
    line = {
        "metric": "OPEN-1B attention int8-PV fwd + binary32 bwd TFLOP/s (bit-exact vs CPU contract oracle), "
                  "B4 H16 Hkv4 D128, S 2048/4096 x window 0/512",
        "value": round(tot_flops / (tot_ms * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(tot_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32+i8",
        "data": "synthetic (Philox N(0,1), RoPE theta 500000, bf16 storage)",
        "config": {"workload": "OPEN-1B attention shape: int8-PV fwd (score cache) + binary32 bwd, B4 H16 Hkv4 D128",
                   "cases": [[S, w] for S, w in cases]},
        "bit_exact_vs_oracle": all_ok if not args.no_verify else None,
        "roofline": dict(dom["roofline"]["dkdv"], kernel="attn_dkdv_bf16_kernel",
                         case=f"S{dom['S']} window {dom['window']}", traffic=None),
        "cpu_baseline": next((r["cpu_baseline"] for r in results if r["cpu_baseline"]), None),
        "cases": results,
    }
    print(json.dumps(line), flush=True)
    return 0 if all_ok in (None, True) else 3


def bench_layer(args, torch, dev) -> int:
    """one decoder layer fwd+bwd, B4 S2048 d2048,
    16 x 128 heads, d_ff 5632, bf16 weights N(0, 0.02), inputs N(0, 1)."""
    import numpy as np

    from open_transformers_amd import synthetic
    from open_transformers_amd.nn.layer import DecoderLayer, rope_tables

    B, S, d, H, hd, dff = 4, 2048, 2048, 16, 128, 5632
    rng = np.random.default_rng(5)
    layer = DecoderLayer(d, H, H, hd, dff, device=dev)
    with torch.no_grad():
        for n, p in layer.named_parameters():
            if n.startswith("norm"):
                v = np.ones(tuple(p.shape), np.float32)
            else:
                v = (rng.standard_normal(tuple(p.shape)) * 0.02).astype(np.float32)
            p.copy_(torch.from_numpy(synthetic.round_to_bf16(v)).to(torch.bfloat16))

    def bf16_normal(shape):
        v = synthetic.round_to_bf16(rng.standard_normal(shape).astype(np.float32))
        return torch.from_numpy(v).to(torch.bfloat16).to(dev)

    x = bf16_normal((B, S, d)).requires_grad_()
    dy = bf16_normal((B, S, d))
    cos, sin = (t.to(dev) for t in rope_tables(S, hd, 10000.0))

    def step():
        for p in layer.parameters():
            p.grad = None
        x.grad = None
        layer(x, cos, sin).backward(dy)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    M = B * S
    gemm_fwd = 2 * M * (d * H * hd * 2 + d * H * hd * 2 + d * 2 * dff + dff * d)
    flops = 3 * gemm_fwd + synthetic.attention_flops(B, H, S, hd)
    line = {
        "metric": "decoder layer fwd+bwd TFLOP/s (bit-exact vs CPU contract oracle), BASELINE configuration 5",
        "value": round(flops / (ms * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (bf16 weights N(0,0.02), inputs N(0,1), RoPE theta 10000)",
        "config": {"workload": "decoder layer fwd+bwd B4 S2048 d2048 16x128 d_ff 5632 (BASELINE config 5)",
                   "flop_per_step": flops},
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_loss(args, torch, dev) -> int:
    """Fused CE + z-loss (coeff 1e-4) fwd+bwd over the OPEN-1B lm-head logits:
    N = 4 x 2048 rows, V = 128256, bf16, logits N(0, 4) and uniform labels
    generated on the device.  HBM-bound: the algorithmic traffic is one read of
    the logits in the forward and one read plus one write in the backward."""
    import numpy as np

    from open_transformers_amd import _lib

    N, V, coeff = 8192, 128256, 1e-4
    gen = torch.Generator(device=dev).manual_seed(2024)
    logits = (torch.randn(N, V, device=dev, generator=gen) * 2.0).to(torch.bfloat16)
    labels = torch.randint(0, V, (N,), device=dev, generator=gen)
    stats = torch.empty((5, N), dtype=torch.float32, device=dev)
    loss = torch.empty(2, dtype=torch.float32, device=dev)
    gloss = torch.ones(2, dtype=torch.float32, device=dev)
    grad = torch.empty_like(logits)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    sid = stream.cuda_stream
    BF16 = _lib.DTYPE_BF16

    def step(ev):
        ev[0].record(stream)
        _lib.check(lib.otx_ce_zloss_fwd(logits.data_ptr(), labels.data_ptr(), N, V, BF16, coeff, stats.data_ptr(),
                                        loss.data_ptr(), sid), "loss fwd")
        ev[1].record(stream)
        _lib.check(lib.otx_ce_zloss_bwd(logits.data_ptr(), labels.data_ptr(), stats.data_ptr(), gloss.data_ptr(), N, V,
                                        BF16, coeff, grad.data_ptr(), sid), "loss bwd")
        ev[2].record(stream)

    def events():
        return [torch.cuda.Event(enable_timing=True) for _ in range(3)]

    for _ in range(args.warmup):
        step(events())
    torch.cuda.synchronize()
    evs = [events() for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step(evs[s])
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    fwd_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    bwd_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
    nbytes = N * V * 2
    step_bytes = 3 * nbytes
    bwd_gbs = 2 * nbytes / (bwd_ms * 1e-3) / 1e9

    verified, cpu = None, None
    if not args.no_verify or not args.no_cpu:
        from oracle import oracle as orc

        nthreads, why = cpu_threads()
        rows = 2048
        x = logits[:rows].float().cpu().numpy()
        lab = labels[:rows].cpu().numpy()

        def cpu_step():
            _, _, st = orc.ce_zloss_fwd(x, lab, coeff, nthreads=nthreads)
            return st, orc.ce_zloss_bwd(x, lab, st, coeff, n_total=N, nthreads=nthreads)

        cpu_s, cpu_all, (st_r, g_r) = median_time(cpu_step, args.cpu_runs)
        cpu = {"value": round(3 * rows * V * 2 / cpu_s / 1e9, 4), "unit": "GB/s", "cores": nthreads, "kind": "port",
               "sample": f"rows 0..{rows - 1} of the same logits, fwd+bwd; median of {len(cpu_all)} runs "
                         f"{cpu_s:.2f} s (all: {', '.join(f'{x:.2f}' for x in cpu_all)} s); {why}",
               "box": host_box()}
        if not args.no_verify:
            st = stats[:, :rows].cpu().numpy()
            ok = np.array_equal(st.view(np.uint32), st_r.view(np.uint32))
            ok = ok and np.array_equal(grad[:rows].float().cpu().numpy().view(np.uint32), g_r.view(np.uint32))
            all_x = logits.float().cpu().numpy()
            ce_r, z_r, st_all = orc.ce_zloss_fwd(all_x, labels.cpu().numpy(), coeff, nthreads=nthreads)
            del all_x
            got = loss.cpu().numpy()
            ok = ok and np.array_equal(got.view(np.uint32), np.array([ce_r, z_r], np.float32).view(np.uint32))
            ok = ok and np.array_equal(stats.cpu().numpy().view(np.uint32), st_all.view(np.uint32))
            verified = bool(ok)
            if not ok:
                print("bench: loss differs from the CPU oracle", file=sys.stderr)
    line = {
        "metric": "fused CE + z-loss fwd+bwd GB/s (bit-exact vs CPU contract oracle) at N8192 V128256 bf16",
        "value": round(step_bytes / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (bf16 logits N(0, 4), uniform labels, device Philox)",
        "config": {"workload": "fused CE + z-loss fwd+bwd, OPEN-1B lm head N 8192 V 128256 bf16, coeff 1e-4",
                   "N": N, "V": V, "coeff": coeff, "bytes_per_step": step_bytes},
        "bit_exact_vs_oracle": verified,
        "phase_ms": {"fwd": round(fwd_ms, 4), "bwd": round(bwd_ms, 4)},
        "roofline": {"bound": "hbm", "kernel": "ce_bwd_kernel", "achieved": round(bwd_gbs, 1), "peak": 8000.0,
                     "unit": "GB/s", "frac": round(bwd_gbs / 8000.0, 4), "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0 if verified in (None, True) else 3


def bench_model(args, torch, dev) -> int:
    """One training step (forward, fused CE + z-loss, backward; no optimizer) of
    the OPEN-1B proxy (configs/model/llama3_1b_proxy_repop.yaml: 24 layers,
    d 2048, 16 x 128 heads, 4 KV heads, d_ff 5632, vocab 128256, q/k norm,
    int8-PV attention, window 512 with every 5th layer full causal, z-loss
    1e-4) at B4 x T2048, bf16 weights N(0, 0.02).  Two steps on the same
    batch must give identical loss and gradient bytes."""
    import numpy as np

    from open_transformers_amd.nn.model import Llama3

    B, T, coeff = 4, 2048, 1e-4
    model = Llama3(128256, 2048, 24, 16, 4, 128, 5632, rope_theta=500000.0, swa_window=512, swa_full_every=5,
                   qk_norm=True, attn_int8_pv=True, device=dev)
    gen = torch.Generator(device=dev).manual_seed(7)
    with torch.no_grad():
        for n, p in model.named_parameters():
            if "norm" in n:
                p.fill_(1.0)
            else:
                p.copy_((torch.randn(p.shape, device=dev, generator=gen) * 0.02).to(torch.bfloat16))
    ids = torch.randint(0, 128256, (B, T), device=dev, generator=gen)
    labels = torch.randint(0, 128256, (B, T), device=dev, generator=gen)
    params = list(model.parameters())
    if args.ac != "none":
        from torch.distributed.algorithms._checkpoint.checkpoint_wrapper import checkpoint_wrapper

        from open_transformers_amd.nn.flash_attention import attention_checkpoint_contexts

        kw = {"context_fn": attention_checkpoint_contexts} if args.ac == "cached" else {}
        for i, blk in enumerate(list(model.blocks)):
            model.blocks[i] = checkpoint_wrapper(blk, preserve_rng_state=False, **kw)

    def step():
        for p in params:
            p.grad = None
        ce, z = model.loss(ids, labels, coeff)
        (ce + z).backward()
        return ce, z

    def digest():
        h = torch.zeros((), dtype=torch.int64, device=dev)
        for p in params:
            h = h * 1000003 + p.grad.view(torch.int16).to(torch.int64).sum()
        return int(h.item())

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ce, z = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    first = (ce.detach().float().cpu().numpy().tobytes(), z.detach().float().cpu().numpy().tobytes(), digest())
    ce2, z2 = step()
    torch.cuda.synchronize()
    again = (ce2.detach().float().cpu().numpy().tobytes(), z2.detach().float().cpu().numpy().tobytes(), digest())
    n_params = sum(p.numel() for p in params)
    line = {
        "metric": "OPEN-1B proxy training step tokens/s (fwd + fused loss + bwd, no optimizer), one MI355X",
        "value": round(B * T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32+i8",
        "data": "synthetic (bf16 weights N(0,0.02), uniform token ids and labels, device Philox)",
        "config": {"workload": "OPEN-1B proxy (24 layers, d2048, 16x128 heads, 4 KV heads, d_ff 5632, vocab 128256, "
                               "qk_norm, int8-PV, window 512 / full every 5th) B4 T2048",
                   "activation_checkpointing": args.ac,
                   "params": n_params, "loss": float(np.frombuffer(first[0], np.float32)[0])},
        "repeat_bytes_identical": first == again,
    }
    print(json.dumps(line), flush=True)
    return 0 if first == again else 3


if __name__ == "__main__":
    sys.exit(main())

"""Benchmark of the paged-attention path on one MI355X.

A step is one attention layer of one engine tick: the fused q/k RMSNorm +
RoPE + KV append of the step's tokens, then paged attention over the page
table. The headline workload is batched decode (batch 32, contexts uniform
in [256, 4096], 262,144-token pool); consecutive steps use different layers
of an 8-layer pool, as the 36 layers of a forward pass do, so the 256 MB
MALL cannot serve the K/V bytes. value = algorithmic bytes of a step
(every K/V row of every context once + q/out rows + appended rows) divided
by the measured step time, in GB/s. The K timed steps are captured as one
HIP graph and replayed (a serving engine replays its captured forward pass
the same way); the eager time of the same steps, with the host's launch
work between kernels, is reported beside it.

The JSON line also carries the other four workloads (GPU timing only), the
roofline of the dominant kernel (decode attention; its average duration is
measured with HIP events on the launch stream over the timed steps) and a
CPU baseline: the oracle's decode attention timed on the host, one thread,
on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hayate-exp_amd"))

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
METRIC = "decode attn HBM GB/s & prefill attn TFLOP/s (% of MI355X peak), Qwen3-4B"
EPS = 1e-6


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def step_fn(w, batch, layer, decode_only):
    """One step: the fused q/k norm + RoPE + append of the step's tokens,
    then attention. A batch of decode tokens runs both in one launch
    (decode_layer) plus the merge; other batches run the append launch and
    attend_layer."""
    if decode_only:
        return batch.decode_layer(layer, w.q, w.k, w.v, w.q_norm_w, w.k_norm_w, EPS, w.cos,
                                  w.sin)[1]
    q_rot = batch.norm_rope_write_layer(layer, w.q, w.k, w.v, w.q_norm_w, w.k_norm_w, EPS,
                                        w.cos, w.sin)
    return batch.attend_layer(q_rot, layer)


DECODE_KERNELS = ("hy_paged_decode", "hy_paged_decode_append")


def time_workload(name, steps, warmup, layers, split=0):
    """Times `steps` steps; returns a dict of measurements."""
    from hayate_amd.workloads import make_workload

    w = make_workload(name, device="cuda", num_layers=layers, tokens_per_split=split)
    batch = w.begin()
    decode_only = all(ql == 1 for ql in w.q_lens)
    stream = torch.cuda.current_stream()
    plan = batch.plan(w.q.shape[1])
    for i in range(warmup):
        step_fn(w, batch, i % layers, decode_only)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    # events bracketing the attention kernels, created before the timed region
    timed = DECODE_KERNELS + ("hy_paged_prefill",)
    pool = {n: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                for _ in range(steps)] for n in timed}
    used = {n: 0 for n in timed}

    def hook(kname, after):
        if kname in pool:
            pair = pool[kname][used[kname]]
            pair[1 if after else 0].record(stream)
            if after:
                used[kname] += 1

    batch.launch_hook = hook
    t0 = time.perf_counter()
    for i in range(steps):
        layer = i % layers
        ev[i][0].record(stream)
        step_fn(w, batch, layer, decode_only)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    batch.launch_hook = None
    step_events_ms = float(np.mean([a.elapsed_time(b) for a, b in ev]))
    step_ms = (t1 - t0) * 1e3 / steps
    kernel_ms = {n: float(np.mean([a.elapsed_time(b) for a, b in pool[n][: used[n]]]))
                 for n in timed if used[n]}
    dec_kernel = next((n for n in DECODE_KERNELS if n in kernel_ms), None)
    out = {
        "workload": w.spec.description,
        "ms_per_step": step_ms,
        "step_events_ms": step_events_ms,
        "decode_bytes": w.decode_bytes(),
        "decode_kernel_bytes": w.decode_bytes(include_append=decode_only),
        "prefill_flops": w.prefill_flops(),
        "n_decode_items": plan.n_decode,
        "n_prefill_items": plan.n_prefill,
        "kernel_ms": kernel_ms,
        "decode_kernel": dec_kernel,
    }
    if out["decode_bytes"]:
        out["decode_GBps_step"] = out["decode_bytes"] / (step_ms * 1e-3) / 1e9
        if dec_kernel and not out["prefill_flops"]:
            out["decode_GBps_kernel"] = (out["decode_kernel_bytes"]
                                         / (kernel_ms[dec_kernel] * 1e-3) / 1e9)
    if out["prefill_flops"]:
        out["prefill_TFLOPs_events"] = out["prefill_flops"] / (step_events_ms * 1e-3) / 1e12
        if "hy_paged_prefill" in kernel_ms and not out["decode_bytes"]:
            out["prefill_TFLOPs_kernel"] = (out["prefill_flops"]
                                            / (kernel_ms["hy_paged_prefill"] * 1e-3) / 1e12)
    out.update(time_graphs(w, batch, steps, layers, decode_only))
    if out["decode_bytes"]:
        out["decode_GBps_graph"] = out["decode_bytes"] / (out["ms_per_step_graph"] * 1e-3) / 1e9
    if out["prefill_flops"]:
        out["prefill_TFLOPs_graph"] = (out["prefill_flops"]
                                       / (out["ms_per_step_graph"] * 1e-3) / 1e12)
    del w, batch
    torch.cuda.empty_cache()
    return out


def time_graphs(w, batch, steps, layers, decode_only):
    """The same K steps captured as one HIP graph (a serving engine captures
    its forward pass over the layer stack the same way) and replayed: the
    step time without the host's per-launch work between kernels. One
    untimed replay first; then one timed replay of exactly K steps."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for layer in range(layers):
            step_fn(w, batch, layer, decode_only)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            step_fn(w, batch, i % layers, decode_only)
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    del g
    return {"ms_per_step_graph": (t1 - t0) * 1e3 / steps}


def cpu_baseline(budget_s=10.0):
    """Oracle decode attention on the host, 1 thread, over the batch-32
    decode workload: whole passes over its 32 requests until about
    `budget_s` seconds of work are done."""
    from threadpoolctl import threadpool_limits

    from hayate_amd.workloads import make_workload
    from oracle import paged_ref as R

    w = make_workload("decode_b32", device="cuda", num_layers=1)
    pk = R.torch_bf16_to_bits(w.manager.k_cache[0, 0])
    pv = R.torch_bf16_to_bits(w.manager.v_cache[0, 0])
    q = R.torch_bf16_to_bits(w.q)
    del w.manager
    torch.cuda.empty_cache()
    done_bytes = 0
    passes = 0
    torch.set_num_threads(1)
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < budget_s:
            R.paged_attention(q, pk, pv, w.page_lists, w.cache_lens, w.q_lens, 128,
                              dtype=np.float32)
            done_bytes += w.decode_bytes()
            passes += 1
        dt = time.perf_counter() - t0
    return {
        "value": round(done_bytes / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"oracle float32 paged decode attention, {passes} passes over the 32 requests "
                  f"of the batch-32 decode workload ({dt:.1f} s, one thread)",
    }


def traffic_from_profile(name):
    """HBM bytes per launch of the dominant kernel, read from the committed
    rocprofv3 --pmc summary profiles/<name>.md (FETCH_SIZE + WRITE_SIZE,
    each calibrated against a plain 1 GiB copy), or None."""
    path = os.path.join(ROOT, "profiles", f"{name}.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("hbm_bytes_per_launch ="):
                return int(line.split("=", 1)[1])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--split", type=int, default=0, help="decode tokens per split (0 = auto)")
    ap.add_argument("--only", default="", help="comma-separated workloads (default: all)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the paged-attention path runs on one "
              "MI355X; multi-GPU runs are not part of this build.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        sys.exit(1)

    from hayate_amd.workloads import ORDER

    # the headline workload first: its per-launch event timing is not
    # perturbed by the other workloads' launches
    names = ["decode_b32"] + [n for n in ORDER
                              if n != "decode_b32" and (not args.only or n in args.only.split(","))]
    results = {}
    for name in names:
        log(f"[bench] {name}")
        results[name] = time_workload(name, args.steps, args.warmup, args.layers, args.split)
        log(f"[bench] {name}: {json.dumps(results[name])}")

    head = results["decode_b32"]
    line = {
        "metric": METRIC,
        "value": round(head["decode_GBps_graph"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step_graph"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "decode_b32: batched paged decode, batch 32, contexts U[256, 4096], "
                        "262,144-token pool, 128-token pages, 32 q / 8 kv heads, head_dim 128; "
                        f"step = qk-norm+rope+append fused into decode attention (one launch) "
                        f"+ merge, {args.layers} layers rotated; the K timed steps replay as one "
                        "HIP graph",
            "ms_per_step_eager": round(head["ms_per_step"], 5),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"decode_kernel<4, fused append> ({head['decode_kernel']})",
            "achieved": round(head["decode_GBps_kernel"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(head["decode_GBps_kernel"] / HBM_PEAK_GBS, 4),
            "kernel_us": round(head["kernel_ms"][head["decode_kernel"]] * 1e3, 2),
            "algorithmic_bytes": head["decode_kernel_bytes"],
            "traffic": traffic_from_profile("decode_kernel_decode_b32"),
        },
    }
    if not args.no_cpu:
        log("[bench] cpu baseline")
        line["cpu_baseline"] = cpu_baseline()
    line["configs"] = {
        n: {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
        for n, r in results.items()
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

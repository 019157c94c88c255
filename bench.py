"""Benchmark of one Fast-AttnRes read (forward + backward) on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]

A "step" is one read: ``out = attnres(values, query)`` followed by
``torch.autograd.grad(out, (values, query), dO)``, the public path with the
gfx950 HIP kernels behind it.  Inputs are synthetic (seeded) and resident in
HBM before the timed region starts.  The default workload is the headline
configuration: packed BF16 values [S=25, B=8, T=2048, D=2048] (N=16384
tokens), R=2048, per-source std U[0.5, 4], 1% of channels x8, query
N(0,1)/sqrt(R), dO N(0,1).

Printed: ONE JSON line (rank 0).  ``value`` is the achieved algorithmic HBM
bandwidth of the whole read in TB/s (bytes below / measured time per read);
``ms_per_step`` is the time per read.  Algorithmic bytes per read:

    forward  = S*N*D*2 (values read) + N*D*2 (output write)
    backward = S*N*D*2 (values read) + N*D*2 (dO read) + S*N*D*2 (dvalues write)

``roofline`` describes the dominant launch, the backward op (the fused
backward kernel and the two kernels of the deterministic dq reduction),
timed with HIP events recorded on the stream the kernels run on; its
``traffic`` is the HBM bytes per launch measured with rocprofv3 counters
(profiles/attnres_<config>_hbm_traffic.json).  ``cpu_baseline`` times the CPU
FP32 oracle (test infrastructure under ``oracle/``) on the host over a
bounded sample of the same inputs.

``--copy-probe`` runs only a plain device copy of known size, used to scale
the hardware FETCH_SIZE / WRITE_SIZE counters when profiling.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _path in (ROOT, ROOT / "fast-attnres_amd"):
    if str(_path) not in sys.path:
        sys.path.insert(0, str(_path))

HBM_PEAK_TBS = 8.0  # MI355X HBM3E peak, TB/s

# name -> (sources, tokens as (batch, seq), width, rank)
CONFIGS = {
    "c2": dict(sources=25, batch=(8, 2048), width=2048, rank=2048,
               name="standard-full-read S=25 N=16384 D=2048 R=2048 packed"),
    "c3": dict(sources=16, batch=(16384,), width=4096, rank=1024,
               name="sliced-lowrank-read S=16 N=16384 D=4096 R=1024 packed"),
}


def read_bytes(sources: int, tokens: int, width: int) -> tuple[int, int]:
    """Algorithmic HBM bytes of one read: (forward, backward)."""
    row = tokens * width * 2
    return sources * row + row, sources * row + row + sources * row


def make_inputs(cfg: dict, device, seed: int = 0):
    import torch

    generator = torch.Generator(device=device).manual_seed(seed)
    sources, width, rank = cfg["sources"], cfg["width"], cfg["rank"]
    shape = (sources, *cfg["batch"], width)
    std = torch.rand(sources, generator=generator, device=device) * 3.5 + 0.5
    channel_scale = torch.ones(width, device=device)
    outliers = torch.randperm(width, generator=generator, device=device)[: max(1, width // 100)]
    channel_scale[outliers] = 8.0
    values = torch.empty(shape, device=device, dtype=torch.bfloat16)
    for s in range(sources):  # per source keeps the FP32 temporary small
        noise = torch.randn(shape[1:], generator=generator, device=device)
        values[s] = (noise * std[s] * channel_scale).to(torch.bfloat16)
    query = (torch.randn(rank, generator=generator, device=device) / math.sqrt(rank)).to(torch.bfloat16)
    grad_out = torch.randn(shape[1:], generator=generator, device=device).to(torch.bfloat16)
    return values, query, grad_out


def measured_traffic(config: str, key: str) -> int | None:
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    counters (calibrated against a device copy of known size), as recorded in
    profiles/attnres_<config>_hbm_traffic.json; None when not measured."""
    path = ROOT / "profiles" / f"attnres_{config}_hbm_traffic.json"
    if not path.is_file():
        return None
    return int(json.loads(path.read_text()).get(key)) or None


def copy_probe(gib: float = 1.0, reps: int = 5) -> None:
    """A plain device-to-device copy of known size (for counter scaling)."""
    import torch

    elems = int(gib * 2**30) // 2
    src = torch.randn(elems, device="cuda").to(torch.bfloat16)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": elems * 2, "copy_probe_bytes_written": elems * 2,
                      "reps": reps}), flush=True)


def cpu_baseline(values, query, grad_out, budget_s: float, chunk: int) -> dict:
    """Time the CPU FP32 oracle (forward + backward) over token chunks of the
    same inputs until ``budget_s`` seconds of oracle time have been spent;
    scale to one full read.  Tokens are independent, so chunking changes no
    result (dq is a sum over tokens)."""
    import torch

    from oracle.oracle import oracle_with_grads

    cores = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(cores)
    sources, width = values.shape[0], values.shape[-1]
    flat = values.reshape(sources, -1, width)
    upstream = grad_out.reshape(-1, width)
    tokens = flat.shape[1]
    query_cpu = query.cpu()
    # one untimed warm-up chunk (thread pool, allocator)
    oracle_with_grads(flat[:, :256].cpu(), query_cpu, upstream[:256].cpu())
    done, spent = 0, 0.0
    while done < tokens and spent < budget_s:
        stop = min(tokens, done + chunk)
        v, g = flat[:, done:stop].cpu(), upstream[done:stop].cpu()
        start = time.perf_counter()
        oracle_with_grads(v, query_cpu, g)
        spent += time.perf_counter() - start
        done = stop
    seconds_per_read = spent * tokens / done
    fwd, bwd = read_bytes(sources, tokens, width)
    return {
        "value": round((fwd + bwd) / seconds_per_read / 1e12, 6),
        "unit": "TB/s",
        "us_per_read": round(seconds_per_read * 1e6, 1),
        "cores": cores,
        "kind": "port",
        "sample": (f"CPU FP32 eager oracle (oracle/oracle.py, torch {torch.__version__}), "
                   f"forward+backward over {done} of {tokens} tokens of the same inputs in "
                   f"chunks of {chunk}, {spent:.1f} s, scaled to one full read"),
    }


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--config", choices=sorted(CONFIGS), default="c2")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU oracle time")
    parser.add_argument("--copy-probe", action="store_true")
    args = parser.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the read shards over tokens with no "
              "communication except the dq gradient all-reduce, and this build runs on "
              "a single MI355X (--gpus 1).", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    if args.copy_probe:
        copy_probe()
        return 0

    from attnres import _native, attnres

    _native.load()  # fail loudly if the HIP library is missing
    cfg = CONFIGS[args.config]
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    values, query, grad_out = make_inputs(cfg, device)
    values.requires_grad_(True)
    query.requires_grad_(True)
    sources, width = cfg["sources"], cfg["width"]
    tokens = math.prod(cfg["batch"])
    fwd_bytes, bwd_bytes = read_bytes(sources, tokens, width)

    def step(events=None):
        if events is not None:
            events[0].record()
        out = attnres(values, query)
        if events is not None:
            events[1].record()
        grads = torch.autograd.grad(out, (values, query), grad_out)
        if events is not None:
            events[2].record()
        return out, grads

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(args.steps):
        step(events[i])
    stop.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    fwd_ms = [e[0].elapsed_time(e[1]) for e in events]
    bwd_ms = [e[1].elapsed_time(e[2]) for e in events]

    ms_per_step = total_ms / args.steps
    fwd_avg = statistics.fmean(fwd_ms)
    bwd_avg = statistics.fmean(bwd_ms)
    value = (fwd_bytes + bwd_bytes) / (ms_per_step * 1e-3) / 1e12
    bwd_tbs = bwd_bytes / (bwd_avg * 1e-3) / 1e12
    fwd_tbs = fwd_bytes / (fwd_avg * 1e-3) / 1e12

    record = {
        "metric": "fwd+bwd us/read and achieved HBM TB/s (% peak), S=25 D=2048 N=16K tokens",
        "value": round(value, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_read": round(ms_per_step * 1e3, 2),
        "pct_of_peak": round(100 * value / HBM_PEAK_TBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "storage_dtype": "bf16",
        "data": "synthetic (seeded; per-source std U[0.5,4], 1% channels x8)",
        "config": {"workload": cfg["name"], "sources": sources, "tokens": tokens,
                   "width": width, "rank": cfg["rank"], "layout": "packed",
                   "bytes_per_read": fwd_bytes + bwd_bytes},
        "forward": {"us": round(fwd_avg * 1e3, 2), "bytes": fwd_bytes, "TB/s": round(fwd_tbs, 4),
                    "pct_of_peak": round(100 * fwd_tbs / HBM_PEAK_TBS, 2)},
        "backward": {"us": round(bwd_avg * 1e3, 2), "bytes": bwd_bytes, "TB/s": round(bwd_tbs, 4),
                     "pct_of_peak": round(100 * bwd_tbs / HBM_PEAK_TBS, 2)},
        "roofline": {"bound": "hbm",
                     "kernel": "backward op: attnres_bwd_kernel + attnres_dq_slices_kernel + "
                               "attnres_dq_finalize_kernel",
                     "achieved": round(bwd_tbs * 1e3, 1), "peak": HBM_PEAK_TBS * 1e3,
                     "unit": "GB/s", "frac": round(bwd_tbs / HBM_PEAK_TBS, 4),
                     "traffic": measured_traffic(args.config, "backward_bytes")},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        record["cpu_baseline"] = cpu_baseline(values.detach(), query.detach(), grad_out,
                                              args.cpu_budget, chunk=2048)
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""GRBeam end-to-end benchmark on one MI355X.

Workload (the reference's headline configuration): a Qwen3.5-0.8B-shaped
hybrid model (24 layers [3x Gated DeltaNet, 1x gated attention] x 6, hidden
1024, vocabulary 248320, tied embeddings) with random bf16 weights, batch 32,
prompts of 1024 uniform-random token ids, beam 256, 3 output tokens over the
full vocabulary.  One step is one ``grbeam_search`` call on the batch with the
reference's timing protocol (src/kadllm benchmarks/grbeam.py:266-330): output
token 1 from prefill, two decode calls, selection, synchronisation and the
copy of the tokens to the host are all inside the timed region; every step's
output is validated to hold 256 distinct fixed-depth sequences per request.

Printed: one JSON line with requests/s (= batch * steps / elapsed), the
roofline of the dominant kernel (the bf16 MFMA GEMM: algorithmic flops of all
GEMM launches in the timed steps divided by their summed durations from HIP
events recorded on the launch stream) and the CPU baseline (the oracle
restatement of the reference torch path on this host, one request).
"""

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "requests/s at B32/prefix1024/beam256/3 tok; per-kernel HBM GB/s & MFMA util"
H800_REQ_S = 36.08          # reference README, 1x H800, same workload
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA


def validate_output(tokens, batch, width, depth):
    """Each request holds `width` distinct fixed-depth sequences (grbeam.py:32-41)."""
    if len(tokens) != batch or any(
        len(beams) != width or any(len(s) != depth for s in beams)
        or len({tuple(s) for s in beams}) != width
        for beams in tokens
    ):
        raise ValueError("search did not return the requested distinct fixed-depth beams")


class GemmTimer:
    """Records a HIP event pair around every GEMM launch (torch's current stream,
    the stream the GEMM is launched on).  The events are created before the
    timed region (`reserve`), so that the timed loop only records them."""

    def __init__(self):
        self.events = []
        self.pool = []

    def reserve(self, n):
        self.pool.extend(torch.cuda.Event(enable_timing=True) for _ in range(2 * n))

    def __call__(self, launch, flops, nbytes):
        if len(self.pool) >= 2:
            e1, e0 = self.pool.pop(), self.pool.pop()
        else:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        launch()
        e1.record()
        self.events.append((e0, e1, flops, nbytes))

    def summary(self):
        torch.cuda.synchronize()
        ms = sum(e0.elapsed_time(e1) for e0, e1, _, _ in self.events)
        flops = sum(f for _, _, f, _ in self.events)
        nbytes = sum(b for _, _, _, b in self.events)
        return ms, flops, nbytes, len(self.events)


# HBM bytes per GEMM launch of this workload: rocprofv3 FETCH_SIZE and
# WRITE_SIZE over the GEMM dispatches of one search, each scaled by its reading
# for a 1 GiB device copy (reads x2.0, writes x1.0), divided by the launch
# count.  Re-measured with the command in profiles/gemm_hbm_traffic_b32_p1024_w256.md.
GEMM_TRAFFIC_BYTES_PER_LAUNCH = 386.2e6


def cpu_baseline(cfg, sd_cpu, prefix, beam, depth, threads):
    """Oracle search on the host for one request of the workload; returns requests/s."""
    from oracle import grbeam_ref
    from oracle.qwen35_ref import Qwen35Oracle

    torch.set_num_threads(threads)
    oracle = Qwen35Oracle(cfg, sd_cpu)

    class _Adapter:
        def prefill(self, ids):
            return oracle.prefill(ids)

        def decode(self, history, state):
            return oracle.decode(history, state)

    ids = torch.randint(0, cfg.vocab_size, (1, prefix), generator=torch.Generator().manual_seed(1))
    t0 = time.perf_counter()
    with torch.no_grad():
        tokens, _, _, _ = grbeam_ref.grbeam_search(_Adapter(), ids, [beam] * depth)
    tokens.tolist()
    dt = time.perf_counter() - t0
    return 1.0 / dt, dt


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--prefix", type=int, default=1024)
    ap.add_argument("--beam", type=int, default=256)
    ap.add_argument("--depth", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--prompts", choices=("uniform", "pattern"), default="uniform",
                    help="uniform: uniform-random prompt ids (default); pattern: the reference "
                         "runner's prompts, token i of request r = 10 + (i + 17 r) % 100")
    ap.add_argument("--workload", choices=("grbeam", "conditional_sid"), default="grbeam",
                    help="grbeam: the headline full-vocabulary search (default); "
                         "conditional_sid: B8, prefix 4096, coarse widths [32, 32] over the full "
                         "vocabulary, then 16 children per coarse beam for 2 tokens with "
                         "candidates restricted to a seeded 8192-id subset")
    a = ap.parse_args()
    if a.workload == "conditional_sid":
        return conditional_sid(a)
    if a.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for {a.gpus}); "
              "requests shard across GPUs with no exchange, see the design notes", file=sys.stderr)
        sys.exit(2)

    from kadllm_amd import grbeam_search, layers
    from kadllm_amd.adapters import Qwen35GRBeamAdapter, native_model
    from kadllm_amd.config import qwen35_08b_config
    from kadllm_amd.weights import random_state_dict

    dev = torch.device("cuda:0")
    cfg = qwen35_08b_config()
    sd = random_state_dict(cfg, seed=0, dtype=torch.bfloat16, device=dev)
    model, head = native_model(cfg, sd)
    adapter = Qwen35GRBeamAdapter(model, head)
    if a.prompts == "pattern":   # benchmarks/grbeam.py:254-257
        r = torch.arange(a.batch)[:, None]
        ids = (10 + (torch.arange(a.prefix)[None, :] + 17 * r) % 100).to(dev)
    else:
        ids = torch.randint(0, cfg.vocab_size, (a.batch, a.prefix),
                            generator=torch.Generator().manual_seed(0)).to(dev)
    widths = [a.beam] * a.depth

    def run():
        return grbeam_search(adapter, ids, widths).tokens.tolist()

    for _ in range(a.warmup):
        validate_output(run(), a.batch, a.beam, a.depth)
    torch.cuda.synchronize()

    timer = GemmTimer()
    timer.reserve(128 * a.steps * a.depth)   # GEMM launches: about 115 per level
    layers.set_launch_timer(timer)
    times, outputs = [], []
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for _ in range(a.steps):
        t0 = time.perf_counter()
        outputs.append(run())
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    layers.set_launch_timer(None)
    for out in outputs:
        validate_output(out, a.batch, a.beam, a.depth)
    gemm_ms, gemm_flops, gemm_bytes, n_gemm = timer.summary()
    achieved = gemm_flops / (gemm_ms * 1e-3) / 1e12  # TFLOP/s
    value = a.batch * a.steps / elapsed

    cpu = None
    if not a.no_cpu_baseline:
        sd_cpu = {k: v.cpu() for k, v in sd.items()}
        threads = min(a.cpu_threads, os.cpu_count() or 1)
        rps, dt = cpu_baseline(cfg, sd_cpu, a.prefix, a.beam, a.depth, threads)
        cpu = {"value": round(rps, 6), "unit": "requests/s", "cores": threads, "kind": "port",
               "sample": f"1 request (prefix {a.prefix}, beam {a.beam}, {a.depth} tokens, full "
                         f"vocabulary) through the oracle restatement of the reference torch "
                         f"path, bf16 weights, {dt:.1f} s"}

    workload_default = (a.batch, a.prefix, a.beam, a.depth) == (32, 1024, 256, 3)
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "requests/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(1000 * elapsed / a.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / H800_REQ_S, 3) if workload_default else None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, " + (
            "uniform-random prompt ids)" if a.prompts == "uniform"
            else "prompt ids 10 + (i + 17 r) % 100 as in the reference runner)"),
        "config": {"workload": f"grbeam_e2e qwen3.5-0.8B-shaped B{a.batch} P{a.prefix} "
                               f"W{a.beam} depth{a.depth} full-vocab",
                   "batch": a.batch, "prefix": a.prefix, "beam": a.beam, "depth": a.depth,
                   "vocab": cfg.vocab_size, "layers": cfg.num_hidden_layers},
        "roofline": {"kernel": "bf16 MFMA GEMM (all launches)", "bound": "mfma",
                     "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": GEMM_TRAFFIC_BYTES_PER_LAUNCH if workload_default else None,
                     "algorithmic_bytes_per_launch": round(gemm_bytes / n_gemm),
                     "launches_per_step": n_gemm // a.steps,
                     "gemm_ms_per_step": round(gemm_ms / a.steps, 3)},
        "cpu_baseline": cpu,
        "step_ms": [round(1000 * t, 2) for t in times],
    }
    print(json.dumps(line), flush=True)


def conditional_sid(a):
    """Two-level conditional semantic-ID search (no reference runner exists for it;
    vs_baseline is null).  One step is one conditional_search call on the batch,
    tokens copied to the host, inside the timed region."""
    if a.gpus != 1:
        print("bench.py runs on one GPU", file=sys.stderr)
        sys.exit(2)
    from kadllm_amd import conditional_search
    from kadllm_amd.adapters import Qwen35GRBeamAdapter, native_model
    from kadllm_amd.config import qwen35_08b_config
    from kadllm_amd.weights import random_state_dict

    B, P, coarse, fine, n_sub = 8, 4096, [32, 32], [16, 16], 8192
    dev = torch.device("cuda:0")
    cfg = qwen35_08b_config()
    sd = random_state_dict(cfg, seed=0, dtype=torch.bfloat16, device=dev)
    adapter = Qwen35GRBeamAdapter(*native_model(cfg, sd))
    ids = torch.randint(0, cfg.vocab_size, (B, P), generator=torch.Generator().manual_seed(0)).to(dev)
    sub = torch.zeros(cfg.vocab_size, dtype=torch.bool)
    sub[torch.randperm(cfg.vocab_size, generator=torch.Generator().manual_seed(0))[:n_sub]] = True
    sub = sub.to(dev)
    everything = torch.ones(cfg.vocab_size, dtype=torch.bool, device=dev)

    def allowed(history, logits):
        return sub if history.shape[2] >= len(coarse) else everything

    def run():
        res = conditional_search(adapter, ids, coarse, fine, allowed=allowed)
        return res.tokens.tolist()

    width = coarse[-1] * fine[-1]
    for _ in range(a.warmup):
        validate_output(run(), B, width, len(coarse) + len(fine))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    outs = [run() for _ in range(a.steps)]
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    for out in outs:
        validate_output(out, B, width, len(coarse) + len(fine))
    value = B * a.steps / elapsed
    print(json.dumps({
        "metric": "requests/s, two-level conditional SID search",
        "value": round(value, 3), "unit": "requests/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(1000 * elapsed / a.steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights, uniform-random prompt ids, seeded 8192-id subset)",
        "config": {"workload": f"conditional_sid qwen3.5-0.8B-shaped B{B} P{P} coarse{coarse} "
                               f"fine{fine}x{coarse[-1]} subset{n_sub}",
                   "batch": B, "prefix": P, "coarse_widths": coarse, "fine_widths": fine},
        "roofline": None, "cpu_baseline": None}), flush=True)


if __name__ == "__main__":
    main()

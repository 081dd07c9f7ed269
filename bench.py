"""GRBeam benchmarks on one MI355X.

Default workload (the reference's headline configuration): a
Qwen3.5-0.8B-shaped hybrid model (24 layers [3x Gated DeltaNet, 1x gated
attention] x 6, hidden 1024, vocabulary 248320, tied embeddings) with random
bf16 weights, batch 32, prompts of 1024 uniform-random token ids, beam 256,
3 output tokens over the full vocabulary.  One step is one ``grbeam_search``
call on the batch with the reference's timing protocol (src/kadllm
benchmarks/grbeam.py:266-330): output token 1 from prefill, two decode calls,
selection, synchronisation and the copy of the tokens to the host are all
inside the timed region; every step's output is validated to hold 256
distinct fixed-depth sequences per request.

Printed: one JSON line with requests/s (= batch * steps / elapsed), the
roofline of the dominant kernel (the bf16 MFMA GEMM), a per-kernel table
("kernels": launches, time, achieved GB/s or TFLOP/s and roofline fraction
per kernel class, from HIP events around every launch in extra untimed
steps), per-step host / enqueue / device times (device: from the step's start
to its last kernel), memory peaks, and the CPU
baseline (the oracle restatement of the reference torch path on this host's
cores, one request, timed twice).

Other modes:
  --protocol reference   3 processes x (3 warmups + 5 timed calls), latency
                         mean with a 95% CI over process means and the sampled
                         device-memory peak (README.md:116,119)
  --workload ops_gdn     isolated GDN suffix replay and conv4 (configuration 2)
  --workload ops_attention  isolated prefix-shared attention, T = 1, 2, 3
                         (configuration 3)
  --workload ops_gemm    every GEMM shape of the headline search alone, beside
                         torch.matmul (hipBLASLt) on the same operands
  --workload conditional_sid  two-level SID search (configuration 5)
  --workload sid_study   the setting of the reference's two-level SID study
                         (4,096-token SID head, beam 256, prefill + one suffix
                         decode, P512/1024 x B8/32; README.md:139-148)
  --workload hbm_copy    a 1 GiB device copy: measured streaming bandwidth and
                         the calibration of rocprofv3's FETCH/WRITE_SIZE
  --workload hbm_probe   the library's streaming probe over 4 GiB (copy, read,
                         write), which the default run also measures and
                         reports every HBM-bound kernel against
  --depth 7 --batch 4    the reference's 7-token runs (README.md:125)
"""

import argparse
import gc
import json
import math
import os
import platform
import statistics
import subprocess
import sys
import threading
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "requests/s at B32/prefix1024/beam256/3 tok; per-kernel HBM GB/s & MFMA util"
H800_REQ_S = 36.08          # reference README, 1x H800, same workload
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
T975 = {1: 12.706, 2: 4.303, 3: 3.182, 4: 2.776, 5: 2.571, 6: 2.447, 7: 2.365, 9: 2.262}

# HBM bytes per plain GEMM call of the default workload: rocprofv3 FETCH_SIZE
# and WRITE_SIZE over the GEMM dispatches of one search (the fused conv
# projection apart), each scaled by its reading for a 1 GiB device copy (reads
# x2.0, writes x1.0), divided by the number of GEMM calls (328; a call that
# splits its last round launches two kernels).  Re-measured with the commands
# in profiles/hbm_traffic_and_busy_b32_p1024_w256.md.
GEMM_TRAFFIC_BYTES_PER_LAUNCH = 326.0e6


def repeat_stability(outputs, first):
    """Whether any timed call's tokens differ from the last warm-up call's, and
    each call's mean per-request overlap of the beam sets with it
    (benchmarks/grbeam.py:331-340)."""
    differ = any(out != first for out in outputs)
    overlap = [round(statistics.mean(
        len({tuple(x) for x in left} & {tuple(x) for x in right}) / len(right)
        for left, right in zip(out, first)), 6) for out in outputs]
    return {"repeat_tokens_differ": differ, "repeat_beam_set_overlap": overlap}


def provenance(cfg, sd, ids):
    """SHA-256 of the model configuration, of the weights (in state-dict key
    order, raw bytes) and of the prompt ids (benchmarks/grbeam.py:24-29,159-160)."""
    import dataclasses
    import hashlib

    conf = json.dumps(dataclasses.asdict(cfg), sort_keys=True, default=str).encode()
    w = hashlib.sha256()
    for k in sorted(sd):
        w.update(k.encode())
        w.update(sd[k].detach().contiguous().cpu().view(torch.uint8).numpy().tobytes())
    p = hashlib.sha256(ids.cpu().contiguous().numpy().tobytes())
    return {"config_sha256": hashlib.sha256(conf).hexdigest(), "weights_sha256": w.hexdigest(),
            "prompt_ids_sha256": p.hexdigest()}


def validate_output(tokens, batch, width, depth):
    """Each request holds `width` distinct fixed-depth sequences (grbeam.py:32-41)."""
    if len(tokens) != batch or any(
        len(beams) != width or any(len(s) != depth for s in beams)
        or len({tuple(s) for s in beams}) != width
        for beams in tokens
    ):
        raise ValueError("search did not return the requested distinct fixed-depth beams")


# ---------------------------------------------------------------------------
# per-kernel accounting: algorithmic HBM bytes and flops of each C-ABI call,
# from its arguments (each input and output counted once)

def _es(code):
    return 4 if code == 2 else 2


def kernel_work(name, a):
    """(kernel class, bound, algorithmic bytes, algorithmic flops) of one call."""
    if name == "kad_gemm_bf16":
        M, N, K, epi = a[8], a[9], a[10], a[11]
        n_out = N // 2 if epi == 2 else N
        return "gemm", "mfma", 2 * (M * K + N * K + M * n_out + (M * n_out if a[6] else 0)), \
            2 * M * N * K
    if name in ("kad_gdn_suffix_replay", "kad_gdn_recurrent"):
        if name == "kad_gdn_suffix_replay":
            B, W, T, H, HV, K, V = a[15:22]
            BW, sdt = B * W, a[12]
        else:
            BW, T, H, HV, K, V = a[17:23]
            B, sdt = BW // max(a[13], 1), a[12]
        es = _es(a[5])
        nbytes = BW * T * (2 * H * K + 2 * HV * V) * es + B * HV * K * V * _es(sdt) \
            + BW * T * HV * 6
        label = "gdn_replay" if name == "kad_gdn_suffix_replay" else "gdn_recurrent"
        return label, "hbm", nbytes, BW * HV * 2 * T * 2 * K * V
    if name == "kad_gemm_bf16_conv":
        # the prefill's GDN input projection with the depthwise conv in its
        # epilogue (a class of its own: its time includes the conv's VALU
        # work): A, W and the output once (the conv's inputs stay on chip),
        # the conv state
        M, N, K, Cc, L = a[6], a[7], a[8], a[9], a[11]
        return "gemm_conv", "mfma", 2 * (M * K + N * K + M * N) + (M // L) * Cc * 4 * 2, \
            2 * M * N * K
    if name == "kad_gdn_suffix_replay_conv_gated_parents":
        # the last level's mixer: the earlier token's pre-conv rows read in
        # place from the parents' cache, the new token's rows and gate rows,
        # the state and the gates in, each beam's normed last-token row out
        B, W, T, H, HV, K, V = a[25:32]
        BW, C = B * W, 2 * H * K + HV * V
        nbytes = BW * T * C * 2 + BW * HV * V * 2 * 2 + B * HV * K * V * _es(a[18]) \
            + BW * T * HV * 6 + B * C * 3 * 2 + C * 4 * 2
        return "gdn_replay", "hbm", nbytes, BW * HV * 2 * T * 2 * K * V + 8 * BW * C * T
    if name in ("kad_gdn_suffix_replay_conv", "kad_gdn_suffix_replay_conv_gated"):
        # pre-conv q|k|v rows in, replay output out (the conv output stays on
        # chip); gated: the gate rows of the normed tokens in, normed rows out
        gated = name.endswith("_gated")
        B, W, T, H, HV, K, V = a[22:29] if gated else a[17:24]
        BW, C = B * W, 2 * H * K + HV * V
        t_out = (1 if a[19] else T) if gated else T
        nbytes = BW * T * C * 2 + BW * t_out * HV * V * 2 * (2 if gated else 1) \
            + B * HV * K * V * _es(a[14]) + BW * T * HV * 6 + B * C * 3 * 2 + C * 4 * 2
        return "gdn_replay", "hbm", nbytes, BW * HV * 2 * T * 2 * K * V + 8 * BW * C * T
    if name == "kad_causal_conv_suffix":
        B, W, C, T, dt = a[16], a[17], a[18], a[19], a[20]
        return "conv_suffix", "hbm", (2 * B * W * C * T + B * C * 3 + C * 4) * _es(dt), \
            8 * B * W * C * T
    if name in ("kad_prefix_attention_decode_ex", "kad_prefix_attention_decode"):
        if name.endswith("_ex"):
            B, W, Tq, Tk, H, HK, L, D = a[26:34]
        else:
            B, W, Tq, H, HK, L, D = a[26:33]
            Tk = Tq
        rows = B * W * Tq * H
        nbytes = 2 * (3 * rows * D + 2 * B * L * HK * D + 2 * B * W * Tk * HK * D)
        return "attention_decode", "mfma", nbytes, 4 * rows * (L + Tk) * D
    if name == "kad_attention_prefill":
        B, L, H, HK, D = a[17:22]
        return "attention_prefill", "mfma", 2 * (3 * B * L * H * D + 2 * B * L * HK * D), \
            4 * B * H * D * L * (L + 1) // 2
    if name == "kad_gdn_chunk":
        N, T, H, HV, K, V = a[19:25]
        return "gdn_chunk", "hbm", N * T * (2 * H * K + 2 * HV * V) * 2 + N * HV * K * V * 4, \
            None
    if name == "kad_gdn_chunk_gated":
        # the chunk rule plus the gate rows it reads for the fused norm
        N, T, H, HV, K, V = a[19:25]
        return "gdn_chunk", "hbm", N * T * (2 * H * K + 3 * HV * V) * 2 + N * HV * K * V * 4, \
            None
    if name == "kad_causal_conv_prefill":
        B, L, C = a[6], a[7], a[8]
        return "conv_prefill", "hbm", 2 * B * L * C * 2 + B * C * 4 * 2 + C * 8, None
    if name == "kad_beam_row_select":
        rows, V, K = a[6], a[8], a[9]
        return "row_select", "hbm", rows * V * _es(a[1]) + rows * K * 8, None
    if name == "kad_beam_merge_select":
        return "merge_select", "hbm", a[2] * a[3] * 8, None
    if name == "kad_gather_beam_rows":
        return "gather_rows", "hbm", 2 * a[9] * a[10] * a[6] * a[7], None
    if name == "kad_rmsnorm":
        return "rowwise", "hbm", 4 * a[6] * a[7], None
    if name == "kad_rmsnorm_gated":
        return "rowwise", "hbm", 6 * a[7] * a[8] * a[9], None
    if name in ("kad_qk_norm_rope", "kad_scatter_heads"):
        rows, heads, D = (a[10], a[3], a[11]) if name == "kad_qk_norm_rope" else (a[9], a[2], a[3])
        return "rowwise", "hbm", 4 * rows * heads * D, None
    if name == "kad_embedding":
        return "rowwise", "hbm", 4 * a[3] * a[4], None
    if name == "kad_gdn_gates":
        return "rowwise", "hbm", 10 * a[8] * a[9], None
    if name == "kad_cache_prefetch":
        return "prefetch", "hbm", (a[1] // 16 + a[3] // 16) * 16, None
    return "other", "hbm", None, None


class KernelProfiler:
    """C-ABI call hook: a HIP event pair around every launch, on the stream the
    launch goes to (torch's current stream), grouped by kernel class."""

    def __init__(self):
        self.records = []

    def __call__(self, name, args, launch):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        launch()
        e1.record()
        self.records.append((kernel_work(name, args), e0, e1))

    def table(self, steps):
        torch.cuda.synchronize()
        agg = {}
        for (label, bound, nbytes, flops), e0, e1 in self.records:
            r = agg.setdefault(label, dict(bound=bound, launches=0, ms=0.0, bytes=0, flops=0,
                                           have_bytes=True, have_flops=True))
            r["launches"] += 1
            r["ms"] += e0.elapsed_time(e1)
            r["have_bytes"] &= nbytes is not None
            r["have_flops"] &= flops is not None
            r["bytes"] += nbytes or 0
            r["flops"] += flops or 0
        out = {}
        for label, r in sorted(agg.items(), key=lambda kv: -kv[1]["ms"]):
            sec = r["ms"] * 1e-3
            e = {"bound": r["bound"], "launches_per_step": r["launches"] // steps,
                 "ms_per_step": round(r["ms"] / steps, 3),
                 "avg_us": round(1000 * r["ms"] / r["launches"], 2)}
            if r["have_bytes"] and sec > 0:
                e["GB/s"] = round(r["bytes"] / sec / 1e9, 1)
                e["hbm_frac"] = round(e["GB/s"] / PEAK_HBM_GBS, 4)
            if r["have_flops"] and sec > 0 and r["flops"]:
                e["TFLOP/s"] = round(r["flops"] / sec / 1e12, 2)
                e["mfma_frac"] = round(e["TFLOP/s"] / PEAK_BF16_TFLOPS, 4)
            e["frac"] = e.get("mfma_frac" if r["bound"] == "mfma" else "hbm_frac")
            e["bytes_per_launch"] = r["bytes"] // r["launches"] if r["have_bytes"] else None
            e["flops_per_launch"] = r["flops"] // r["launches"] if r["have_flops"] else None
            out[label] = e
        return out


class DeviceMemorySampler:
    """Whole-device memory in use (total - free), sampled every 100 ms in a
    thread, as the reference samples nvidia-smi (benchmarks/grbeam.py:125-141)."""

    def __init__(self, interval=0.1):
        self.interval, self.peak = interval, 0
        self._stop = threading.Event()
        self._thread = threading.Thread(target=self._run, daemon=True)

    def _run(self):
        while not self._stop.is_set():
            free, total = torch.cuda.mem_get_info()
            self.peak = max(self.peak, total - free)
            self._stop.wait(self.interval)

    def __enter__(self):
        self._thread.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._thread.join(timeout=3)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def host_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline_search(cfg, sd_cpu, prefix, beam, depth, repeats):
    """Oracle search on the host, one request of the workload, `repeats` times,
    on every core this process may use; returns (requests/s, seconds list)."""
    from oracle import grbeam_ref
    from oracle.qwen35_ref import Qwen35Oracle

    torch.set_num_threads(host_cores())
    oracle = Qwen35Oracle(cfg, sd_cpu)

    class _Adapter:
        def prefill(self, ids):
            return oracle.prefill(ids)

        def decode(self, history, state):
            return oracle.decode(history, state)

    ids = torch.randint(0, cfg.vocab_size, (1, prefix), generator=torch.Generator().manual_seed(1))
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        with torch.no_grad():
            tokens, _, _, _ = grbeam_ref.grbeam_search(_Adapter(), ids, [beam] * depth)
        tokens.tolist()
        times.append(time.perf_counter() - t0)
    return 1.0 / statistics.mean(times), times


def build_model(dev):
    from kadllm_amd.adapters import Qwen35GRBeamAdapter, native_model
    from kadllm_amd.config import qwen35_08b_config
    from kadllm_amd.weights import random_state_dict

    cfg = qwen35_08b_config()
    sd = random_state_dict(cfg, seed=0, dtype=torch.bfloat16, device=dev)
    return cfg, sd, Qwen35GRBeamAdapter(*native_model(cfg, sd))


# ---------------------------------------------------------------------------
def grbeam(a):
    from kadllm_amd import _lib, grbeam_search

    dev = torch.device("cuda:0")
    cfg, sd, adapter = build_model(dev)
    if a.prompts == "pattern":   # benchmarks/grbeam.py:254-257
        r = torch.arange(a.batch)[:, None]
        ids = (10 + (torch.arange(a.prefix)[None, :] + 17 * r) % 100).to(dev)
    else:
        ids = torch.randint(0, cfg.vocab_size, (a.batch, a.prefix),
                            generator=torch.Generator().manual_seed(0)).to(dev)
    widths = [a.beam] * a.depth
    enqueue = []

    def run(done=None):
        t0 = time.perf_counter()
        res = grbeam_search(adapter, ids, widths)
        enqueue.append(time.perf_counter() - t0)   # the host has issued every launch
        if done is not None:
            done.record()                          # after the search's last kernel
        return res.tokens.tolist()

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(a.steps)]
    first = None
    with DeviceMemorySampler() as mem:
        for _ in range(a.warmup):
            first = run()
            validate_output(first, a.batch, a.beam, a.depth)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        # The tokens' host copy (.tolist(), inside the timed region as in the
        # reference) builds ~33k Python objects, which periodically triggers a
        # full garbage collection over the whole interpreter heap (~35 ms).
        # As a serving process would, move the long-lived start-up objects
        # out of the collector's reach; new garbage is still collected.
        if not a.no_gc_freeze:
            gc.collect()
            gc.freeze()
        enqueue.clear()
        times, outputs = [], []
        torch.cuda.synchronize()
        t_start = time.perf_counter()
        for e0, e1 in ev:
            t0 = time.perf_counter()
            e0.record()
            outputs.append(run(e1))
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t_start
    gpu_ms = [e0.elapsed_time(e1) for e0, e1 in ev]
    for out in outputs:
        validate_output(out, a.batch, a.beam, a.depth)
    stability = repeat_stability(outputs, first if first is not None else outputs[0])
    memory = {"device_peak_gib": round(mem.peak / 2**30, 2),
              "torch_peak_allocated_gib": round(torch.cuda.max_memory_allocated() / 2**30, 2),
              "torch_peak_reserved_gib": round(torch.cuda.max_memory_reserved() / 2**30, 2)}
    value = a.batch * a.steps / elapsed

    kernels, roofline = None, None
    if a.profile_steps:
        prof = KernelProfiler()
        _lib.set_call_hook(prof)
        try:
            for _ in range(a.profile_steps):
                validate_output(run(), a.batch, a.beam, a.depth)
        finally:
            _lib.set_call_hook(None)
        kernels = prof.table(a.profile_steps)
        g = kernels.get("gemm")
        default = (a.batch, a.prefix, a.beam, a.depth) == (32, 1024, 256, 3)
        if g:
            roofline = {"kernel": "bf16 MFMA GEMM (all launches)", "bound": "mfma",
                        "achieved": g["TFLOP/s"], "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": g["mfma_frac"],
                        "traffic": GEMM_TRAFFIC_BYTES_PER_LAUNCH if default else None,
                        "algorithmic_bytes_per_launch": g["bytes_per_launch"],
                        "launches_per_step": g["launches_per_step"],
                        "gemm_ms_per_step": g["ms_per_step"]}

    probe = None
    if not a.no_probe:
        probe = hbm_probe_rates(4 << 30, 10)
        add_probe_fractions(kernels, probe)

    cpu = None
    if not a.no_cpu_baseline:
        sd_cpu = {k: v.cpu() for k, v in sd.items()}
        rps, secs = cpu_baseline_search(cfg, sd_cpu, a.prefix, a.beam, a.depth, a.cpu_repeats)
        cpu = {"value": round(rps, 6), "unit": "requests/s", "cores": host_cores(),
               "kind": "port", "cpu_model": cpu_model(),
               "sample": f"1 request (prefix {a.prefix}, beam {a.beam}, {a.depth} tokens, full "
                         f"vocabulary) through the oracle restatement of the reference torch "
                         f"path, bf16 weights, timed {len(secs)} times: "
                         + ", ".join(f"{s:.1f}" for s in secs) + " s"}

    default = (a.batch, a.prefix, a.beam, a.depth) == (32, 1024, 256, 3)
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
        "vs_baseline": round(value / H800_REQ_S, 3) if default else None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, " + (
            "uniform-random prompt ids)" if a.prompts == "uniform"
            else "prompt ids 10 + (i + 17 r) % 100 as in the reference runner)"),
        "config": {"workload": f"grbeam_e2e qwen3.5-0.8B-shaped B{a.batch} P{a.prefix} "
                               f"W{a.beam} depth{a.depth} full-vocab",
                   "batch": a.batch, "prefix": a.prefix, "beam": a.beam, "depth": a.depth,
                   "vocab": cfg.vocab_size, "layers": cfg.num_hidden_layers},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "hbm_probe": probe,
        "memory": memory,
        **stability,
        "provenance": provenance(cfg, sd, ids) if not a.no_provenance else None,
        "step_ms": [round(1000 * t, 2) for t in times],
        "step_gpu_ms": [round(t, 2) for t in gpu_ms],
        "step_enqueue_ms": [round(1000 * t, 2) for t in enqueue[:a.steps]],
    }
    print(json.dumps(line), flush=True)
    if stability["repeat_tokens_differ"]:
        raise SystemExit("the timed searches did not all return the warm-up's tokens")
    return line


def reference_protocol(a):
    """3 processes x (3 warmups + 5 timed calls): latency mean with a 95% CI
    over the process means, requests/s = batch / mean latency, and the sampled
    whole-device memory peak (README.md:116,119; benchmarks/grbeam.py:315-363)."""
    child = [sys.executable, os.path.abspath(__file__), "--steps", str(a.steps),
             "--warmup", str(a.warmup), "--batch", str(a.batch), "--prefix", str(a.prefix),
             "--beam", str(a.beam), "--depth", str(a.depth), "--prompts", a.prompts,
             "--no-cpu-baseline", "--profile-steps", "0", "--no-provenance", "--no-probe"]
    means, peaks, lines = [], [], []
    for p in range(a.processes):
        res = subprocess.run(child, capture_output=True, text=True, timeout=900)
        if res.returncode != 0:
            sys.stderr.write(res.stderr)
            raise SystemExit(f"process {p} failed with {res.returncode}")
        line = json.loads(res.stdout.strip().splitlines()[-1])
        lines.append(line)
        means.append(statistics.mean(line["step_ms"]))
        peaks.append(line["memory"]["device_peak_gib"])
        print(f"process {p}: mean {means[-1]:.2f} ms over {len(line['step_ms'])} calls",
              file=sys.stderr, flush=True)
    n = len(means)
    mean = statistics.mean(means)
    ci = T975.get(n - 1, 1.96) * statistics.stdev(means) / math.sqrt(n) if n > 1 else None
    value = a.batch / (mean / 1000)
    default = (a.batch, a.prefix, a.beam, a.depth) == (32, 1024, 256, 3)
    out = dict(lines[0])
    out.update({
        "value": round(value, 3), "steps": a.steps * n, "warmup": a.warmup,
        "ms_per_step": round(mean, 3),
        "vs_baseline": round(value / H800_REQ_S, 3) if default else None,
        "protocol": {"processes": n, "warmups_per_process": a.warmup,
                     "timed_calls_per_process": a.steps, "latency_ms": round(mean, 3),
                     "ci95_ms": round(ci, 3) if ci is not None else None,
                     "process_mean_ms": [round(m, 3) for m in means],
                     "device_peak_gib": max(peaks)},
        "step_ms": [t for line in lines for t in line["step_ms"]],
        "step_gpu_ms": [t for line in lines for t in line["step_gpu_ms"]],
    })
    out.pop("kernels", None)
    print(json.dumps(out), flush=True)


# ---------------------------------------------------------------------------
def _time_calls(fn, iters):
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters * 1e-3   # seconds per call


def _rel_check(actual, expected, name, rtol=1e-2, atol_frac=3e-3):
    a_, e_ = actual.detach().double().cpu(), expected.detach().double().cpu()
    bad = (a_ - e_).abs() > rtol * e_.abs() + atol_frac * e_.abs().max()
    if bool(bad.any()):
        raise SystemExit(f"{name}: {int(bad.sum())} elements outside tolerance")
    return ((a_ - e_).norm() / e_.norm()).item()


def _op_line(metric, value, unit, config, roofline, cpu, extra):
    line = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": extra.pop("iters"),
            "warmup": 3, "ms_per_step": extra.pop("ms"), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) inputs, as the workload describes)",
            "config": config, "roofline": roofline, "cpu_baseline": cpu}
    line.update(extra)
    print(json.dumps(line), flush=True)


def ops_gdn(a):
    """Configuration 2: GDN suffix replay (S [32,16,128,128] fp32 ~ N(0, 0.02^2),
    q/k/v [8192,3,16,128] bf16 ~ N(0,1), g = -softplus(N(0,1)), beta =
    sigmoid(N(0,1)), 256 beams per request) and the width-4 conv over the same
    beams (state [32,6144,3], x [8192,6144,3], w ~ U(-1/2,1/2)), each checked
    against the oracle on 2 requests and timed over repeated calls; the prefix
    tensors are compared bit for bit before and after."""
    import torch.nn.functional as F

    from kadllm_amd import ops
    from oracle import ops_ref

    dev = torch.device("cuda:0")
    B, W, T, H, HV, K, V, C = 32, 256, 3, 16, 16, 128, 128, 6144
    BW = B * W
    g = torch.Generator(device=dev).manual_seed(0)
    S = torch.randn(B, HV, K, V, generator=g, device=dev) * 0.02
    q = torch.randn(BW, T, H, K, generator=g, device=dev).bfloat16()
    k = torch.randn(BW, T, H, K, generator=g, device=dev).bfloat16()
    v = torch.randn(BW, T, HV, V, generator=g, device=dev).bfloat16()
    gate = -F.softplus(torch.randn(BW, T, HV, generator=g, device=dev))
    beta = torch.sigmoid(torch.randn(BW, T, HV, generator=g, device=dev)).bfloat16()
    S0 = S.clone()
    out = ops.gated_delta(q, k, v, gate, beta, S, beam_width=W)
    rows = torch.cat((torch.arange(0, W), torch.arange((B - 1) * W, B * W)))
    ref = ops_ref.gated_delta(*(t[rows].cpu() for t in (q, k, v, gate, beta)),
                              S[[0, B - 1]].cpu(), beam_width=W)
    err = _rel_check(out[rows], ref, "gdn replay")
    sec = _time_calls(lambda: ops.gated_delta(q, k, v, gate, beta, S, beam_width=W), a.op_iters)
    if not torch.equal(S, S0):
        raise SystemExit("gdn replay wrote the prefix state")
    nbytes = BW * T * (2 * H * K + 2 * HV * V) * 2 + B * HV * K * V * 4 + BW * T * HV * 6
    flops = BW * HV * 2 * T * 2 * K * V
    cpu = None
    if not a.no_cpu_baseline:
        torch.set_num_threads(host_cores())
        args1 = [t[:W].cpu() for t in (q, k, v, gate, beta)] + [S[:1].cpu()]
        t0 = time.perf_counter()
        ops_ref.gated_delta(*args1, beam_width=W)
        dt = time.perf_counter() - t0
        cpu = {"value": round(nbytes / B / dt / 1e9, 3), "unit": "GB/s", "cores": host_cores(),
               "kind": "port", "cpu_model": cpu_model(),
               "sample": f"1 of the 32 requests (256 beams) through the oracle's per-request "
                         f"fp32 recurrence, {dt:.2f} s"}
    gbs = nbytes / sec / 1e9
    _op_line("GDN suffix replay, configuration 2: achieved HBM GB/s", round(gbs, 1), "GB/s",
             {"workload": "gdn_replay B32 W256 T3 H16 HV16 K128 V128 (bf16 q/k/v, fp32 S)"},
             {"kernel": "gdn_replay_kernel<128,128,bf16,3>", "bound": "hbm",
              "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
              "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
              "algorithmic_bytes_per_launch": nbytes,
              "mfma_tflops": round(flops / sec / 1e12, 2),
              "mfma_frac": round(flops / sec / 1e12 / PEAK_BF16_TFLOPS, 4)},
             cpu, {"iters": a.op_iters, "ms": round(sec * 1e3, 4), "us_per_call": round(sec * 1e6, 2),
                   "rel_l2_vs_oracle": err})

    # conv4 over the same beams, the reference runner's [BW, C, T] layout and
    # the model's token-major rows
    xs = torch.randn(BW, C, T, generator=g, device=dev).bfloat16()
    st = torch.randn(B, C, 3, generator=g, device=dev).bfloat16()
    w = (torch.rand(C, 4, generator=g, device=dev) - 0.5).bfloat16()
    st0 = st.clone()
    nbytes = (2 * BW * C * T + B * C * 3 + C * 4) * 2
    for layout in ("reference [BW, C, T]", "token-major [BW, T, C]"):
        x = xs if layout.startswith("reference") else xs.transpose(1, 2).contiguous().transpose(1, 2)
        y = ops.causal_conv1d(x, st, w, beam_width=W)
        ref = ops_ref.causal_conv1d(x[rows].cpu(), st[[0, B - 1]].cpu(), w.cpu(), beam_width=W)
        err = _rel_check(y[rows], ref, "conv", rtol=1.6e-2, atol_frac=1e-3)
        sec = _time_calls(lambda: ops.causal_conv1d(x, st, w, beam_width=W), a.op_iters)
        if not torch.equal(st, st0):
            raise SystemExit("conv wrote the prefix state")
        cpu = None
        if not a.no_cpu_baseline:
            x1 = x[:W].cpu()
            t0 = time.perf_counter()
            ops_ref.causal_conv1d(x1, st[:1].cpu(), w.cpu(), beam_width=W)
            dt = time.perf_counter() - t0
            cpu = {"value": round(nbytes / B / dt / 1e9, 3), "unit": "GB/s",
                   "cores": host_cores(), "kind": "port", "cpu_model": cpu_model(),
                   "sample": f"1 of the 32 requests through the oracle's per-request conv1d, "
                             f"{dt:.3f} s"}
        gbs = nbytes / sec / 1e9
        _op_line(f"conv4 suffix, configuration 2, {layout}: achieved HBM GB/s", round(gbs, 1),
                 "GB/s", {"workload": f"conv4 B32 W256 C6144 T3 bf16, x {layout}"},
                 {"kernel": "conv_suffix", "bound": "hbm", "achieved": round(gbs, 1),
                  "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                  "traffic": None, "algorithmic_bytes_per_launch": nbytes},
                 cpu, {"iters": a.op_iters, "ms": round(sec * 1e3, 4),
                       "us_per_call": round(sec * 1e6, 2), "rel_l2_vs_oracle": err})


def ops_attention(a):
    """Configuration 3: prefix-shared gated GQA decode attention, 32 requests x
    256 beams, 8 q heads / 2 KV heads x 256, prefix 1024, suffix T = 1, 2, 3,
    output sigmoid gate; all inputs bf16 ~ N(0,1), scale 1/16.  Checked against
    the oracle on 2 requests, then timed."""
    from kadllm_amd import ops
    from oracle import ops_ref

    dev = torch.device("cuda:0")
    B, W, H, HK, L, D = 32, 256, 8, 2, 1024, 256
    BW = B * W
    g = torch.Generator(device=dev).manual_seed(0)
    pk = torch.randn(B, L, HK, D, generator=g, device=dev).bfloat16()
    pv = torch.randn(B, L, HK, D, generator=g, device=dev).bfloat16()
    pk0, pv0 = pk.clone(), pv.clone()
    rows = torch.cat((torch.arange(0, W), torch.arange((B - 1) * W, B * W)))
    for T in (1, 2, 3):
        q = torch.randn(BW, T, H, D, generator=g, device=dev).bfloat16()
        sk = torch.randn(BW, T, HK, D, generator=g, device=dev).bfloat16()
        sv = torch.randn(BW, T, HK, D, generator=g, device=dev).bfloat16()
        gate = torch.randn(BW, T, H * D, generator=g, device=dev).bfloat16()

        def call():
            return ops.prefix_attention(q, pk, pv, sk, sv, beam_width=W, scale=1 / 16, gate=gate)

        out = call()
        ref = ops_ref.prefix_attention(q[rows].cpu(), pk[[0, B - 1]].cpu(), pv[[0, B - 1]].cpu(),
                                       sk[rows].cpu(), sv[rows].cpu(), beam_width=W, scale=1 / 16)
        ref = (ref.float().reshape(2 * W, T, H * D)
               * torch.sigmoid(gate[rows].cpu().float()).bfloat16().float()).bfloat16()
        err = _rel_check(out[rows].reshape(2 * W, T, H * D), ref, "attention")
        sec = _time_calls(call, a.op_iters)
        if not (torch.equal(pk, pk0) and torch.equal(pv, pv0)):
            raise SystemExit("attention wrote the prefix K/V")
        flops = 4 * BW * T * H * (L + T) * D
        nbytes = 2 * (3 * BW * T * H * D + 2 * B * L * HK * D + 2 * BW * T * HK * D)
        tfs = flops / sec / 1e12
        cpu = None
        if not a.no_cpu_baseline:
            torch.set_num_threads(host_cores())
            t0 = time.perf_counter()
            ops_ref.prefix_attention(q[:W].cpu(), pk[:1].cpu(), pv[:1].cpu(), sk[:W].cpu(),
                                     sv[:W].cpu(), beam_width=W, scale=1 / 16)
            dt = time.perf_counter() - t0
            cpu = {"value": round(flops / B / dt / 1e12, 4), "unit": "TFLOP/s",
                   "cores": host_cores(), "kind": "port", "cpu_model": cpu_model(),
                   "sample": f"1 of the 32 requests through the oracle's fp32 folded-beam "
                             f"attention, {dt:.2f} s"}
        _op_line(f"prefix-shared gated GQA attention, configuration 3, T={T}: achieved TFLOP/s",
                 round(tfs, 2), "TFLOP/s",
                 {"workload": f"prefix_attention B32 W256 H8 HK2 D256 L1024 T{T} gated bf16"},
                 {"kernel": "attn3_kernel<false, 4>", "bound": "mfma", "achieved": round(tfs, 2),
                  "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                  "frac": round(tfs / PEAK_BF16_TFLOPS, 4), "traffic": None,
                  "algorithmic_flops_per_launch": flops, "algorithmic_bytes_per_launch": nbytes,
                  "hbm_GBps": round(nbytes / sec / 1e9, 1),
                  "hbm_frac": round(nbytes / sec / 1e9 / PEAK_HBM_GBS, 4)},
                 cpu, {"iters": a.op_iters, "ms": round(sec * 1e3, 4),
                       "us_per_call": round(sec * 1e6, 2), "rel_l2_vs_oracle": err})


# The GEMMs of one search at B32 / prefix 1024 / beam 256 / 3 tokens on the
# 0.8B model: (name, M, N, K, epilogue, dispatches per search).  Prefill runs
# every layer on 32 x 1024 rows (the last layer's attention output, o_proj and
# MLP only on the 32 last rows, which take the small-M kernel and are left
# out here), each of the two decode levels on 32 x 256.
GEMM_SHAPES = (
    ("prefill gdn in_proj", 32768, 8192, 1024, 0, 18),
    ("prefill attn qkv", 32768, 5120, 1024, 0, 5),
    ("prefill last attn layer kv", 32768, 1024, 1024, 0, 1),
    ("prefill mlp gate_up (SwiGLU)", 32768, 7168, 1024, 2, 23),
    ("prefill mixer out (residual)", 32768, 1024, 2048, 1, 23),
    ("prefill mlp down (residual)", 32768, 1024, 3584, 1, 23),
    ("decode gdn in_proj", 8192, 8192, 1024, 0, 36),
    ("decode attn qkv", 8192, 5120, 1024, 0, 12),
    ("decode mlp gate_up (SwiGLU)", 8192, 7168, 1024, 2, 48),
    ("decode mixer out (residual)", 8192, 1024, 2048, 1, 48),
    ("decode mlp down (residual)", 8192, 1024, 3584, 1, 48),
    ("decode lm head", 8192, 248320, 1024, 0, 2),
)


def ops_gemm(a):
    """The bf16 GEMM shapes of the headline search, one at a time: kad_gemm_bf16
    (automatic tile choice, fused epilogue), each tile configuration named by
    --gemm-configs through kad_gemm_bf16_tiled, and the same product through
    torch.matmul (hipBLASLt, no epilogue).  Inputs ~ N(0,1), weights ~ N(0,
    0.05^2); the automatic choice is checked against F.linear on 64 rows and
    every configuration against it bit for bit.  Timing: each form warmed,
    then 7 interleaved rounds (the order rotating per round) of --op-iters / 7
    back-to-back calls with HIP events, and each form's median; forms timed one
    after another show an order bias (the first form measured runs slowest)."""
    from torch.nn import functional as F

    from kadllm_amd import _lib, layers

    cfgs = [int(c) for c in a.gemm_configs.split(",") if c.strip()] if a.gemm_configs else []
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    rounds = 7
    per = max(a.op_iters // rounds, 3)
    total = {"auto": 0.0, "lib": 0.0, "flops": 0.0}
    total.update({c: 0.0 for c in cfgs})
    for name, M, N, K, epi, count in GEMM_SHAPES:
        x = torch.randn(M, K, generator=g, device=dev).bfloat16()
        w = (torch.randn(N, K, generator=g, device=dev) * 0.05).bfloat16()
        n_out = N // 2 if epi == layers.EPI_SWIGLU else N
        res = torch.randn(M, n_out, generator=g, device=dev).bfloat16()
        stream = _lib.stream_of(x)

        def form(cfg):
            out = res.clone()
            r = out if epi == layers.EPI_RESIDUAL else None

            def call():
                _lib.call("kad_gemm_bf16_tiled", _lib.ptr(x), K, _lib.ptr(w), K, _lib.ptr(out),
                          n_out, _lib.ptr(r), n_out if r is not None else 0, M, N, K, epi, cfg,
                          stream)
            return out, call

        out, auto = form(0)
        auto()
        torch.cuda.synchronize()
        first = out.clone()
        prod = F.linear(x[:64], w).float()
        if epi == layers.EPI_SWIGLU:
            gu = prod.bfloat16().float().view(64, N // 64, 2, 32)
            expect = (F.silu(gu[:, :, 0]).bfloat16().float() * gu[:, :, 1]).reshape(64, n_out)
        elif epi == layers.EPI_RESIDUAL:
            expect = res[:64].float() + prod.bfloat16().float()
        else:
            expect = prod
        _rel_check(first[:64].float(), expect, name, rtol=2e-2, atol_frac=1e-2)
        calls = {"auto": auto}
        for c in cfgs:
            o, f = form(c)
            try:
                f()
            except _lib.KadLibraryError:
                continue                      # the configuration does not take this shape
            torch.cuda.synchronize()
            if not torch.equal(o, first):
                raise SystemExit(f"{name}: tile configuration {c} differs from the automatic choice")
            calls[c] = f
        lib_out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        calls["lib"] = lambda: torch.matmul(x, w.t(), out=lib_out)
        for f in calls.values():
            for _ in range(3):
                f()
        samples = {k: [] for k in calls}
        keys = list(calls)
        for rd in range(rounds):
            for k in keys[rd % len(keys):] + keys[:rd % len(keys)]:
                samples[k].append(_time_calls(calls[k], per))
        med = {k: statistics.median(v) for k, v in samples.items()}
        flops = 2.0 * M * N * K
        nbytes = 2 * (M * K + N * K + M * n_out * (2 if epi == layers.EPI_RESIDUAL else 1))
        sec, lib_sec = med["auto"], med["lib"]
        tfs, lib_tfs = flops / sec / 1e12, flops / lib_sec / 1e12
        for k in med:
            if k in total:
                total[k] += count * med[k]
        total["flops"] += count * flops
        _op_line(f"bf16 GEMM {name}: achieved TFLOP/s", round(tfs, 1), "TFLOP/s",
                 {"workload": f"gemm M{M} N{N} K{K} epilogue {epi}"},
                 {"kernel": "gemm (automatic tile choice)", "bound": "mfma",
                  "achieved": round(tfs, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                  "frac": round(tfs / PEAK_BF16_TFLOPS, 4), "traffic": None,
                  "algorithmic_flops_per_launch": flops, "algorithmic_bytes_per_launch": nbytes},
                 None, {"iters": rounds * per, "ms": round(sec * 1e3, 4),
                        "us_per_call": round(sec * 1e6, 2), "dispatches_per_search": count,
                        "hipblaslt_us_per_call": round(lib_sec * 1e6, 2),
                        "hipblaslt_tflops": round(lib_tfs, 1),
                        "vs_hipblaslt": round(lib_sec / sec, 3),
                        "tile_config_us": {str(k): round(v * 1e6, 2) for k, v in med.items()
                                           if k not in ("auto", "lib")}})
        del x, w, res, lib_out, calls
        torch.cuda.empty_cache()
    tfs = total["flops"] / total["auto"] / 1e12
    _op_line("bf16 GEMMs of one headline search, dispatch-weighted: achieved TFLOP/s",
             round(tfs, 1), "TFLOP/s", {"workload": "gemm shapes of grbeam B32 P1024 W256 3 tokens"},
             {"kernel": "gemm (automatic tile choice)", "bound": "mfma", "achieved": round(tfs, 1),
              "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(tfs / PEAK_BF16_TFLOPS, 4),
              "traffic": None}, None,
             {"iters": rounds * per, "ms": round(total["auto"] * 1e3, 3),
              "hipblaslt_ms": round(total["lib"] * 1e3, 3),
              "hipblaslt_tflops": round(total["flops"] / total["lib"] / 1e12, 1),
              "tile_config_ms": {str(c): round(total[c] * 1e3, 3) for c in cfgs}})


# kernel classes whose algorithmic bytes are almost all reads (reported
# against the read probe); the others against the copy probe
READ_DOMINATED = {"row_select", "merge_select", "prefetch"}


def hbm_probe_rates(size=4 << 30, iters=10):
    """GB/s of the library's streaming probe (kad_hbm_probe) over `size`
    bytes: copy (read + write, counting both), read only, write only."""
    from kadllm_amd import _lib

    dev = torch.device("cuda:0")
    src = torch.empty(size, dtype=torch.uint8, device=dev).random_(0, 255)
    dst = torch.empty_like(src)
    stream = _lib.stream_of(src)
    rates = {}
    for mode, name, factor in ((0, "copy", 2), (1, "read", 1), (2, "write", 1)):
        def launch():
            _lib.call("kad_hbm_probe", _lib.ptr(src), _lib.ptr(dst), size, mode, stream)
        launch()
        sec = _time_calls(launch, iters)
        rates[name + "_GB/s"] = round(factor * size / sec / 1e9, 1)
    del src, dst
    torch.cuda.empty_cache()
    rates["bytes"] = size
    return rates


def add_probe_fractions(kernels, probe):
    """Each HBM-bound kernel class's GB/s as a fraction of the probe's (read
    probe for read-dominated classes, copy probe otherwise)."""
    for label, e in (kernels or {}).items():
        if e.get("GB/s") is None:
            continue
        ref = probe["read_GB/s"] if label in READ_DOMINATED else probe["copy_GB/s"]
        e["probe_frac"] = round(e["GB/s"] / ref, 4)
        e["probe"] = "read" if label in READ_DOMINATED else "copy"


def hbm_probe(a):
    """The library's own streaming kernel over 4 GiB (no profiler): the
    bandwidth this board gives a plain copy, read and write."""
    rates = hbm_probe_rates(4 << 30, a.op_iters)
    gbs = rates["copy_GB/s"]
    _op_line("HBM streaming probe 4 GiB: achieved GB/s (copy, read + write)", gbs, "GB/s",
             {"workload": "hbm_probe 4 GiB, 16-byte lanes, 8 workgroups per CU"},
             {"kernel": "hbm_probe_kernel", "bound": "hbm", "achieved": gbs,
              "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
              "traffic": None, "algorithmic_bytes_per_launch": 2 * rates["bytes"]}, None,
             {"iters": a.op_iters, "ms": round(2 * rates["bytes"] / gbs / 1e6, 4),
              "probe": rates})


def hbm_copy(a):
    """A 1 GiB device-to-device copy (torch's copy kernel), repeated: the
    bandwidth a plain streaming kernel reaches on this board, and the known
    byte count against which rocprofv3's FETCH_SIZE / WRITE_SIZE readings of
    the other kernels are scaled."""
    dev = torch.device("cuda:0")
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 255)
    dst = torch.empty_like(src)
    sec = _time_calls(lambda: dst.copy_(src), a.op_iters)
    gbs = 2 * n / sec / 1e9
    _op_line("device copy 1 GiB: achieved HBM GB/s (read + write)", round(gbs, 1), "GB/s",
             {"workload": "hbm_copy 1 GiB uint8"},
             {"kernel": "copy", "bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
              "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": 2 * n,
              "algorithmic_bytes_per_launch": 2 * n}, None,
             {"iters": a.op_iters, "ms": round(sec * 1e3, 4), "us_per_call": round(sec * 1e6, 2)})


def conditional_sid(a):
    """Two-level conditional semantic-ID search (no reference runner exists for it;
    vs_baseline is null).  One step is one conditional_search call on the batch,
    tokens copied to the host, inside the timed region."""
    from kadllm_amd import conditional_search

    B, P, coarse, fine, n_sub = 8, 4096, [32, 32], [16, 16], 8192
    dev = torch.device("cuda:0")
    cfg, _, adapter = build_model(dev)
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
    times, outs = [], []
    for _ in range(a.steps):
        t1 = time.perf_counter()
        outs.append(run())
        times.append(time.perf_counter() - t1)
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
        "roofline": None, "cpu_baseline": None,
        "step_ms": [round(1000 * t, 2) for t in times]}), flush=True)


# the reference's two-level conditional-SID study (README.md:139-148, RTX 4090,
# grouped prefix reuse): batch latency in ms by (prefix, batch)
SID_STUDY_4090_MS = {(512, 8): 89.2, (512, 32): 420.3, (1024, 8): 158.8, (1024, 32): 720.1}


def sid_study(a):
    """The setting of the reference's two-level conditional-SID study
    (README.md:139-148): a SID-only head of 4,096 token ids (each level picks
    from those 4,096 codes), beam 256, the first level from the prefill and the
    second from one suffix decode, at prefix 512 / 1024 x batch 8 / 32.  One
    step is one grbeam_search call with the tokens copied to the host, as in the
    headline protocol.  Latency is reported beside the reference's published
    RTX 4090 latencies (grouped column) as context: another GPU, and the
    reference's head and scoring details beyond this are unpublished."""
    from kadllm_amd import grbeam_search
    from kadllm_amd.adapters import Qwen35GRBeamAdapter, native_model
    from kadllm_amd.config import qwen35_08b_config
    from kadllm_amd.weights import random_state_dict

    dev = torch.device("cuda:0")
    cfg = qwen35_08b_config()
    sd = random_state_dict(cfg, seed=0, dtype=torch.bfloat16, device=dev)
    n_sid, beam = 4096, 256
    sid = torch.randperm(cfg.vocab_size, generator=torch.Generator().manual_seed(0))[:n_sid]
    adapter = Qwen35GRBeamAdapter(*native_model(cfg, sd), head_tokens=sid)
    rows = []
    for P in (512, 1024):
        for B in (8, 32):
            ids = torch.randint(0, cfg.vocab_size, (B, P),
                                generator=torch.Generator().manual_seed(P + B)).to(dev)

            def run():
                return grbeam_search(adapter, ids, [beam, beam]).tokens.tolist()

            for _ in range(a.warmup):
                validate_output(run(), B, beam, 2)
            torch.cuda.synchronize()
            if not a.no_gc_freeze:   # as in the headline run
                gc.collect()
                gc.freeze()
            times = []
            for _ in range(a.steps):
                t0 = time.perf_counter()
                out = run()
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t0)
                validate_output(out, B, beam, 2)
            mean = statistics.mean(times)
            ci = (T975.get(len(times) - 1, 1.96) * statistics.stdev(times) / math.sqrt(len(times))
                  if len(times) > 1 else None)
            ref = SID_STUDY_4090_MS[(P, B)]
            rows.append({"prefix": P, "batch": B, "latency_ms": round(1000 * mean, 3),
                         "ci95_ms": round(1000 * ci, 3) if ci is not None else None,
                         "requests_per_s": round(B / mean, 2),
                         "reference_4090_grouped_ms": ref,
                         "reference_4090_over_this": round(ref / (1000 * mean), 2)})
            print(f"sid study P{P} B{B}: {1000 * mean:.2f} ms per batch "
                  f"(RTX 4090 grouped: {ref} ms)", file=sys.stderr, flush=True)
    main_row = rows[-1]
    print(json.dumps({
        "metric": "batch latency, two-level conditional-SID study setting (P1024 B32 row)",
        "value": main_row["latency_ms"], "unit": "ms", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": main_row["latency_ms"], "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights, uniform-random prompt ids, seeded 4096-id "
                "SID-only head)",
        "config": {"workload": "sid_study qwen3.5-0.8B-shaped SID head 4096, beam 256, "
                               "prefill + one suffix decode, P512/1024 x B8/32"},
        "roofline": None, "cpu_baseline": None, "rows": rows}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--prefix", type=int, default=1024)
    ap.add_argument("--beam", type=int, default=256)
    ap.add_argument("--depth", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-repeats", type=int, default=2)
    ap.add_argument("--no-probe", action="store_true",
                    help="skip the 4 GiB HBM streaming probe after the timed steps")
    ap.add_argument("--no-provenance", action="store_true",
                    help="skip the SHA-256 of the configuration, weights and prompts")
    ap.add_argument("--no-gc-freeze", action="store_true",
                    help="leave the start-up heap to Python's full garbage collections")
    ap.add_argument("--profile-steps", type=int, default=2,
                    help="untimed steps after the timed ones with every launch timed")
    ap.add_argument("--prompts", choices=("uniform", "pattern"), default="uniform",
                    help="uniform: uniform-random prompt ids (default); pattern: the reference "
                         "runner's prompts, token i of request r = 10 + (i + 17 r) %% 100")
    ap.add_argument("--protocol", choices=("single", "reference"), default="single")
    ap.add_argument("--processes", type=int, default=3)
    ap.add_argument("--op-iters", type=int, default=50)
    ap.add_argument("--gemm-configs", default="",
                    help="ops_gemm: tile configurations to time beside the automatic choice, "
                         "e.g. 16,18,20,22")
    ap.add_argument("--workload",
                    choices=("grbeam", "conditional_sid", "ops_gdn", "ops_attention", "ops_gemm",
                             "hbm_copy", "hbm_probe", "sid_study"),
                    default="grbeam")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for {a.gpus}); "
              "requests shard across GPUs with no exchange, see the design notes", file=sys.stderr)
        sys.exit(2)
    if a.protocol == "reference":
        return reference_protocol(a)
    return {"grbeam": grbeam, "conditional_sid": conditional_sid, "ops_gdn": ops_gdn,
            "ops_attention": ops_attention, "ops_gemm": ops_gemm,
            "hbm_copy": hbm_copy, "hbm_probe": hbm_probe, "sid_study": sid_study}[a.workload](a)


if __name__ == "__main__":
    main()

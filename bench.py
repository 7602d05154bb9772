"""Benchmark of the decoder-layer hot path on one MI355X.

Workload: a Llama-2-7B-shaped pipeline stage of 8
decoder layers (hidden 4096, 32 heads x 128, FFN 11008, RoPE theta 1e4),
micro-batch 1, seq 4096, bf16 compute with fp32 master weights; one step =
forward through the 8 layers, backward, and the fused AdamW (lr 1e-4, betas
0.9 / 0.95, wd 0.1) applied to each layer's flat shard inside the backward
on the optimizer stream, as the reference's --optimizer_in_backwards path
does.  Inputs are synthetic (seeded N(0,1) activations and upstream grads,
N(0, 0.02) weights) and resident in HBM before the timed region.

value = decoder-layer fwd+bwd tokens/s = layers * B * S / (time per stage
step), the per-layer throughput the reference's profiler reports
(data/model_latencies.json).  The JSON line also carries the attention
kernels' TFLOP/s against the MFMA peak, the HBM-bound kernels' GB/s, and the
CPU oracle timed on a bounded sample.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

MFMA_BF16_PEAK_TFLOPS = 2516.6   # MI355X dense bf16 (256 CU x 4096 FLOP/clk x 2.4 GHz)
HBM_PEAK_GBS = 8000.0            # MI355X HBM3E
H100_FP16_LAYER_TOKS = 221_477   # data/model_latencies.json:7551, 7B layer seq 4096 fp16


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "hbm_traffic_cfg4.md")


def recorded_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (calibrated against a 1 GiB copy), or
    None when it has not been recorded."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                # "traffic_bytes_per_launch <kernel name, may contain spaces> <bytes>"
                head, _, rest = line.strip().partition(" ")
                name, _, value = rest.rpartition(" ")
                if head == "traffic_bytes_per_launch" and name == kernel and value.isdigit():
                    return int(value)
    except OSError:
        return None
    return None


def _events_time(fn, iters: int, warm: int = 2) -> float:
    """Average milliseconds per call of ``fn`` between HIP events recorded on
    torch's current stream (the stream every kernel here is launched on)."""
    for _ in range(warm):
        fn()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def build_stage(n_layers, dev, seed=3):
    from zorse_amd import llama_simple as L
    cfg = L.llama_config(hidden_size=4096, num_attention_heads=32, intermediate_size=11008,
                         rope_theta=1e4, max_position_embeddings=4096)
    g = torch.Generator().manual_seed(seed)
    layers = []
    for i in range(n_layers):
        with torch.device("meta"):
            layer = L.LlamaDecoderLayer(cfg, i, torch.bfloat16, param_dtype=torch.bfloat16)
        layer.flat_param = torch.nn.Parameter(
            torch.empty(layer.spec.numel, dtype=torch.bfloat16, device=dev))
        # N(0, 0.02) linear weights drawn on the device from a seeded generator
        gd = torch.Generator(device=dev).manual_seed(seed * 1000 + i)
        with torch.no_grad():
            layer.flat_param.normal_(0.0, 0.02, generator=gd)
            layer.param_view("ln1").fill_(1.0)
            layer.param_view("ln2").fill_(1.0)
        layers.append(layer)
    return cfg, layers, g


class KernelCases:
    """The hand-written kernels at the stage's shapes, each as a zero-argument
    launcher plus its algorithmic work per launch.  HBM-bound cases rotate
    through enough buffers that the working set exceeds the 256 MB Infinity
    Cache.  ``copy`` is a plain device copy of 1 GiB (read 1 GiB, write
    1 GiB), the calibration for the FETCH_SIZE / WRITE_SIZE counters."""

    NAMES = ("attn_fwd", "attn_bwd", "rmsnorm_fwd", "rmsnorm_bwd", "adamw", "adamw_t", "copy",
             "gemm_gu", "gemm_dgrad_gu", "gemm_wgrad_gu", "blas_gu", "blas_dgrad_gu",
             "blas_wgrad_gu", "rope", "lm_head", "lm_head_chunked", "lm_head_torch")

    # the last stage's LM head: the reference's default vocabulary
    # (models/llama_simple.py:559-561, vocab 49152)
    VOCAB = 49152

    def __init__(self, dev, spec, S):
        self.dev, self.spec, self.S = dev, spec, S

    def make(self, name):
        from zorse_amd import flops
        from zorse_amd import kernels as K
        dev, spec, S = self.dev, self.spec, self.S
        torch.manual_seed(0)
        B, H, d, h = 1, spec.heads, spec.head_dim, spec.hidden
        T = B * S
        if name in ("attn_fwd", "attn_bwd"):
            q = torch.randn(B, S, H, d, device=dev, dtype=torch.bfloat16)
            k = torch.randn(B, S, H, d, device=dev, dtype=torch.bfloat16)
            v = torch.randn(B, S, H, d, device=dev, dtype=torch.bfloat16)
            o, lse = K.attn_fwd(q, k, v)
            if name == "attn_fwd":
                return (lambda: K.attn_fwd(q, k, v, out=o)), flops.attn_fwd_flops(B, H, d, S, S)
            do = torch.randn_like(q)
            dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
            return ((lambda: K.attn_bwd(q, k, v, o, do, lse, dq=dq, dk=dk, dv=dv)),
                    flops.attn_bwd_flops(B, H, d, S, S))
        if name in ("rmsnorm_fwd", "rmsnorm_bwd"):
            nbuf = 8
            xs = [torch.randn(T, h, device=dev, dtype=torch.bfloat16) for _ in range(nbuf)]
            w = torch.ones(h, device=dev, dtype=torch.bfloat16)
            ys = [torch.empty_like(x) for x in xs]
            rs = [torch.empty(T, device=dev, dtype=torch.float32) for _ in xs]
            for i in range(nbuf):
                K.rmsnorm_fwd(xs[i], w, 1e-6, out=(ys[i], rs[i]))
            it = [0]
            if name == "rmsnorm_fwd":
                def run():
                    i = it[0] % nbuf
                    it[0] += 1
                    K.rmsnorm_fwd(xs[i], w, 1e-6, out=(ys[i], rs[i]))
                return run, flops.rmsnorm_fwd_bytes(T, h)
            ws = torch.empty(K.rmsnorm_bwd_workspace_elems(T, h), device=dev, dtype=torch.float32)
            dw = torch.empty(h, device=dev, dtype=torch.bfloat16)

            def run():
                i = it[0] % nbuf
                it[0] += 1
                K.rmsnorm_bwd(xs[(i + 1) % nbuf], xs[i], w, rs[i], dw=dw,
                              out=ys[(i + 2) % nbuf], workspace=ws)
            return run, flops.rmsnorm_bwd_bytes(T, h)
        if name == "adamw":
            n = spec.numel
            p = torch.randn(n, device=dev)
            m = torch.zeros(n, device=dev)
            vv = torch.zeros(n, device=dev)
            gr = torch.randn(n, device=dev, dtype=torch.bfloat16)
            lowp = torch.empty(n, device=dev, dtype=torch.bfloat16)
            step = [0]

            def run():
                step[0] += 1
                K.adamw_step(p, gr, m, vv, lr=1e-4, beta1=0.9, beta2=0.95, eps=1e-8,
                             weight_decay=0.1, step=step[0], lowp_out=lowp)
            return run, flops.adamw_bytes(n, 2, True)
        if name == "adamw_t":
            # zk_adamw_step_t's region kernel: one launch over the layer's four
            # projection matrices (each also written transposed) and the norms
            n, o, sp = spec.numel, spec.offsets(), spec
            p = torch.randn(n, device=dev)
            m = torch.zeros(n, device=dev)
            vv = torch.zeros(n, device=dev)
            gr = torch.randn(n, device=dev, dtype=torch.bfloat16)
            lowp = torch.empty(n, device=dev, dtype=torch.bfloat16)
            mats = [(o["q"][0], sp.q_dim + 2 * sp.kv_dim, sp.hidden),
                    (o["o"][0], sp.hidden, sp.q_dim), (o["gate"][0], 2 * sp.ffn, sp.hidden),
                    (o["down"][0], sp.hidden, sp.ffn)]
            regions = [(off, r, c, torch.empty(c, r, device=dev, dtype=torch.bfloat16))
                       for off, r, c in mats]
            tail = o["ln1"][0]
            regions.append((tail, 8, (n - tail) // 8, None))
            n_t = sum(r * c for _, r, c in mats)
            step = [0]

            def run():
                step[0] += 1
                K.adamw_step_t(p, gr, m, vv, lowp, regions, lr=1e-4, beta1=0.9, beta2=0.95,
                               eps=1e-8, weight_decay=0.1, step=step[0])
            return run, flops.adamw_bytes(n, 2, True) + 2 * n_t
        if name == "rope":
            # q and k rotated in place in the layer's q|k|v buffer (4 rotating
            # buffers, 1.2 GB: outside the Infinity Cache); bytes: q and k read
            # and written
            from zorse_amd.functional import rope_tables
            nbuf = 4
            bufs = [torch.randn(T, 3 * H * d, device=dev, dtype=torch.bfloat16)
                    for _ in range(nbuf)]
            cos, sin = rope_tables(S, d, spec.rope_theta, torch.bfloat16, dev)
            it = [0]

            def run():
                qkv = bufs[it[0] % nbuf]
                it[0] += 1
                K.rope_(qkv[:, :H * d].view(B, S, H, d), qkv[:, H * d:2 * H * d].view(B, S, H, d),
                        cos, sin)
            return run, 2 * 2 * T * H * d * 2
        if name in ("gemm_gu", "gemm_dgrad_gu", "gemm_wgrad_gu", "blas_gu", "blas_dgrad_gu",
                    "blas_wgrad_gu"):
            # the layer's largest projection GEMM, its three products on the
            # operands as the layer holds them: forward gate|up = n2 W_gu^T,
            # input gradient dn2 = dgu W_gu, weight gradient dgu^T n2.  gemm_*:
            # the hand-written zk_gemm the stage runs; blas_*: hipBLASLt through
            # torch.mm on the same operands, a reference point only
            F2 = 2 * spec.ffn
            hand = name.startswith("gemm_")
            a = torch.randn(T, h, device=dev, dtype=torch.bfloat16)
            w = 0.02 * torch.randn(F2, h, device=dev, dtype=torch.bfloat16)
            work = 2 * T * h * F2
            if name.endswith("_dgrad_gu"):
                dy = torch.randn(T, F2, device=dev, dtype=torch.bfloat16)
                y = torch.empty(T, h, device=dev, dtype=torch.bfloat16)
                if hand:
                    return (lambda: K.gemm(dy, w, b_kmajor=True, out=y)), work
                return (lambda: torch.mm(dy, w, out=y)), work
            if name.endswith("_wgrad_gu"):
                dy = torch.randn(T, F2, device=dev, dtype=torch.bfloat16)
                dw = torch.empty(F2, h, device=dev, dtype=torch.bfloat16)
                if hand:
                    return (lambda: K.gemm(dy, a, a_kmajor=True, b_kmajor=True, out=dw)), work
                return (lambda: torch.mm(dy.t(), a, out=dw)), work
            y = torch.empty(T, F2, device=dev, dtype=torch.bfloat16)
            if hand:
                return (lambda: K.gemm(a, w, out=y)), work
            return (lambda: torch.mm(a, w.t(), out=y)), work
        if name in ("lm_head", "lm_head_chunked", "lm_head_torch"):
            # LM head + cross-entropy fwd + bwd on [T, h] final hidden states:
            # lm_head the default chunking (here one chunk: 403 MB of logits,
            # kept for the backward), lm_head_chunked 8192-column chunks
            # (logits recomputed in the backward), lm_head_torch F.linear +
            # F.cross_entropy (hipBLASLt, [T, V] logits and their fp32
            # softmax) as a reference point.  Work: the three products, 6 T h V
            # (the chunked form runs a fourth, its recomputation)
            from zorse_amd.lm_head import lm_head_cross_entropy
            V = self.VOCAB
            x = torch.randn(T, h, device=dev, dtype=torch.bfloat16).requires_grad_(True)
            w = (0.02 * torch.randn(V, h, device=dev, dtype=torch.bfloat16)).requires_grad_(True)
            labels = torch.randint(0, V, (T,), device=dev)
            chunk = 8192 if name == "lm_head_chunked" else None

            def run():
                x.grad = None
                w.grad = None
                if name == "lm_head_torch":
                    loss = torch.nn.functional.cross_entropy(
                        torch.nn.functional.linear(x, w).float(), labels)
                else:
                    loss = lm_head_cross_entropy(x, w, labels, chunk=chunk)
                loss.backward()
            return run, 6 * T * h * V
        if name == "copy":
            src = torch.empty(1 << 28, device=dev, dtype=torch.float32).normal_()
            dst = torch.empty_like(src)
            return (lambda: dst.copy_(src)), 2 * src.numel() * 4
        raise ValueError(f"unknown kernel case {name!r}; one of {self.NAMES}")


def measure_kernels(dev, spec, S):
    """Live HIP-event timings of the hand-written kernels at the stage's
    shapes (see KernelCases), plus the layer's largest library GEMM as the
    reference point for the MFMA-bound ones."""
    cases = KernelCases(dev, spec, S)
    rows = {}
    spec_of = {
        "attn_fwd": ("attn_fwd_kernel<bf16,128,full>", "mfma", 20),
        "attn_bwd": ("zk_attn_bwd (attn_bwd_dq + attn_bwd_dkdv)", "mfma", 10),
        "rmsnorm_fwd": ("rmsnorm_fwd_vec<bf16,bf16,128,4>", "hbm", 32),
        "rmsnorm_bwd": ("rmsnorm_bwd_vec<bf16,bf16,256,2,2> + dw reduce", "hbm", 32),
        "adamw": ("adamw_elem<bf16,bf16,true>", "hbm", 10),
        "adamw_t": ("adamw_tile_t<bf16,bf16> (layer step with W^T copies)", "hbm", 10),
        "rope": ("rope_pos_kernel<bf16,128,half> (q and k of the q|k|v buffer)", "hbm", 20),
        "copy": ("device copy 1 GiB (HBM reference)", "hbm", 5),
        "gemm_gu": ("gemm_tiled_kernel<bf16,0,false,false> gate|up fwd 4096 x 22016 x 4096",
                    "mfma", 10),
        "gemm_dgrad_gu": ("gemm_tiled_kernel<bf16,0,false,true> gate|up input grad "
                          "4096 x 4096 x 22016", "mfma", 10),
        "gemm_wgrad_gu": ("gemm_tiled_kernel<bf16,0,true,true> gate|up weight grad "
                          "22016 x 4096 x 4096", "mfma", 10),
        "blas_gu": ("hipBLASLt gate|up fwd, same operands (reference point)", "mfma", 10),
        "blas_dgrad_gu": ("hipBLASLt gate|up input grad, same operands (reference point)",
                          "mfma", 10),
        "blas_wgrad_gu": ("hipBLASLt gate|up weight grad, same operands (reference point)",
                          "mfma", 10),
        "lm_head": ("LM head + CE fwd+bwd, 4096 x 4096 x 49152, default chunking: one chunk, "
                    "logits kept (zk_gemm + zk_ce_*_chunk)", "mfma", 8),
        "lm_head_chunked": ("LM head + CE fwd+bwd, 4096 x 4096 x 49152, 8192-column chunks "
                            "(logits recomputed)", "mfma", 8),
        "lm_head_torch": ("torch F.linear + F.cross_entropy fwd+bwd, same operands (reference "
                          "point)", "mfma", 8),
    }
    for name, (kname, bound, iters) in spec_of.items():
        run, work = cases.make(name)
        ms = _events_time(run, iters, warm=3)
        if bound == "mfma":
            ach, peak, unit = work / ms / 1e9, MFMA_BF16_PEAK_TFLOPS, "TFLOP/s"
        else:
            ach, peak, unit = work / ms / 1e6, HBM_PEAK_GBS, "GB/s"
        rows[name] = {"kernel": kname, "bound": bound, "achieved": round(ach, 1), "peak": peak,
                      "unit": unit, "frac": round(ach / peak, 4), "avg_ms": round(ms, 4),
                      "work_per_launch": work, "traffic": recorded_traffic(kname)}
        del run
        torch.cuda.empty_cache()
    return rows


def host_cpu() -> dict:
    """The host CPU as lscpu names it: model, sockets x cores x threads per
    core, and the CPUs this process may run on."""
    info = {}
    try:
        import subprocess
        out = subprocess.run(["lscpu"], stdout=subprocess.PIPE, stderr=subprocess.DEVNULL,
                             text=True, timeout=20).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return {"model": info.get("Model name"), "sockets": info.get("Socket(s)"),
            "cores_per_socket": info.get("Core(s) per socket"),
            "threads_per_core": info.get("Thread(s) per core"), "cpus": info.get("CPU(s)"),
            "usable_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity")
            else os.cpu_count()}


def cpu_threads() -> int:
    """Threads for the CPU baseline: the host's CPU count, capped by the CPU
    share the GPU box gives one GPU's job (OMP_NUM_THREADS, set to that share
    on the box; a larger count would oversubscribe the cores other jobs on
    the host hold)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    share = os.environ.get("OMP_NUM_THREADS")
    if share and share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return max(1, n or 1)


def cpu_baseline(spec, S, seed=3):
    """The CPU oracle (plain PyTorch, fp32) timed on one layer's fwd+bwd at the
    stage's shape -- a bounded sample (1 of the 8 layers) of the same
    workload, on the host's cores: one untimed iteration at the full shape
    (warm-up), then one timed iteration."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import decoder as O
    threads = cpu_threads()
    torch.set_num_threads(threads)
    shape = O.LayerShape(hidden=spec.hidden, heads=spec.heads, kv_heads=spec.kv_heads,
                         head_dim=spec.head_dim, ffn=spec.ffn, theta=spec.rope_theta)
    g = torch.Generator().manual_seed(seed)
    p = O.init_params(shape, g)
    x = torch.randn(1, S, spec.hidden, generator=g)
    dout = torch.randn(1, S, spec.hidden, generator=g)
    t0 = time.perf_counter()
    O.layer_fwd_bwd(x, p, shape, dout)       # warm-up at the full shape
    warm = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.layer_fwd_bwd(x, p, shape, dout)
    dt = time.perf_counter() - t0
    cpu = host_cpu()
    return {"value": round(S / dt, 1), "unit": "tokens/s", "cores": threads, "threads": threads,
            "kind": "port", "host_cpu": cpu,
            "sample": f"oracle (plain PyTorch fp32) fwd+bwd of 1 of the 8 layers at seq {S}: "
                      f"1 warm-up iteration at the full shape ({warm:.2f} s), then 1 timed "
                      f"iteration ({dt:.2f} s), torch.set_num_threads({threads}) on "
                      f"{cpu.get('model')} ({cpu.get('usable_cpus')} usable CPUs; threads "
                      f"capped at the job's CPU share)",
            "seconds": round(dt, 2)}


def summarize_stage(root: str, layers: int, steps: int, warmup: int) -> str:
    """Markdown summary of a rocprofv3 kernel trace of ``bench.py --steps
    <steps> --warmup <warmup> --layers <layers>`` (``root/bench_kernel_trace.csv``
    and ``root/bench_kernel_stats.csv``): kernel time per timed stage step by
    group over the window from the end of the warm-up's last ``adamw_elem``
    launch to the end of the last timed step's, the GPU's busy time in that
    window (overlapping kernels counted once), and the whole run's kernel
    table."""
    import collections
    import csv
    trace = sorted(csv.DictReader(open(os.path.join(root, "bench_kernel_trace.csv"))),
                   key=lambda r: int(r["Start_Timestamp"]))
    adam = [r for r in trace if "adamw_elem" in r["Kernel_Name"]]
    first, last = warmup * layers - 1, (warmup + steps) * layers - 1
    if warmup < 1 or len(adam) <= last:
        raise SystemExit(f"need >= 1 warm-up step and {last + 1} adamw_elem launches in the "
                         f"trace ({len(adam)} found)")
    t0, t1 = int(adam[first]["End_Timestamp"]), int(adam[last]["End_Timestamp"])
    win = [r for r in trace
           if int(r["Start_Timestamp"]) >= t0 and int(r["End_Timestamp"]) <= t1]
    groups = [("library GEMMs (hipBLASLt)", ("Cijk",)),
              ("hand-written GEMMs (zk_gemm / zk_gemm_swiglu)",
               ("gemm_tiled_kernel", "gemm_gen_kernel", "gemm_swiglu_kernel")),
              ("attention bwd: dq, dkdv", ("attn_bwd",)),
              ("AdamW (optimizer stream, overlapped)", ("adamw",)),
              ("attention fwd", ("attn_fwd",)),
              ("SwiGLU bwd", ("swiglu",)),
              ("transposes", ("transpose",)),
              ("RMSNorm fwd / bwd", ("rmsnorm",)), ("RoPE fwd / bwd", ("rope",)),
              ("device copies", ("copyBuffer",))]
    tot, other = collections.defaultdict(float), 0.0
    for r in win:
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6
        for name, pats in groups:
            if any(p in r["Kernel_Name"] for p in pats):
                tot[name] += d
                break
        else:
            other += d
    allk = sum(tot.values()) + other
    lines = ["| kernel group | ms per timed step | share of kernel time |", "|---|---|---|"]
    for name, _ in groups:
        lines.append(f"| {name} | {tot[name] / steps:.2f} | {100 * tot[name] / allk:.1f} % |")
    if other > 0:
        lines.append(f"| other | {other / steps:.2f} | {100 * other / allk:.1f} % |")
    # timeline shares: each instant of the window split evenly among the groups
    # running then, and the time each group runs with nothing beside it
    ev = []
    for r in win:
        g = next((name for name, pats in groups if any(p in r["Kernel_Name"] for p in pats)),
                 "other")
        ev += [(int(r["Start_Timestamp"]), 1, g), (int(r["End_Timestamp"]), -1, g)]
    ev.sort()
    active, share, alone, prev = collections.Counter(), collections.Counter(), \
        collections.Counter(), t0
    for t, d, g in ev:
        running = [k for k, c in active.items() if c]
        n = sum(active.values())
        for k in running:
            share[k] += (t - prev) * active[k] / n
        if n == 1:
            alone[running[0]] += t - prev
        active[g] += d
        prev = t
    lines += ["", "The same window as a timeline: each instant split evenly among the kernel groups "
                  "running then (the shares sum to the GPU's busy time), and the time each group "
                  "runs with nothing beside it:", "",
              "| kernel group | timeline share (ms per step) | running alone (ms per step) |",
              "|---|---|---|"]
    for name in [g for g, _ in groups] + (["other"] if other > 0 else []):
        lines.append(f"| {name} | {share[name] / steps / 1e6:.2f} | "
                     f"{alone[name] / steps / 1e6:.2f} |")
    iv = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in win)
    busy, (cs, ce) = 0, iv[0]
    for a, b in iv[1:]:
        if a > ce:
            busy += ce - cs
            cs, ce = a, b
        else:
            ce = max(ce, b)
    busy += ce - cs
    lines += ["", f"GPU busy over the {steps} timed steps: {busy / steps / 1e6:.2f} ms per step "
                  f"(window {(t1 - t0) / steps / 1e6:.2f} ms per step)."]
    staged = adam[first + 1:last + 1]
    avg_in = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in staged) / len(staged)
    lines.append(f"`adamw_elem` in the stage (beside the attention backward and GEMMs): "
                 f"{len(staged)} launches, {avg_in / 1e6:.3f} ms on average.")
    rest = adam[last + 1:]
    if rest:
        avg = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rest) / len(rest)
        lines.append(f"`adamw_elem` alone (bench.py's `adamw` case after the stage): "
                     f"{len(rest)} launches, {avg / 1e6:.3f} ms on average.  The kernel table "
                     f"below averages both groups together.")
    # the attention backward in the stage (beside the previous layer's AdamW
    # and the weight-gradient GEMMs) against bench.py's attn_bwd case after it
    after = trace[trace.index(adam[last]) + 1:]
    for kname in ("attn_bwd_dq", "attn_bwd_dkdv", "attn_fwd_kernel"):
        ins = [r for r in win if kname in r["Kernel_Name"]]
        out = [r for r in after if kname in r["Kernel_Name"]]
        if ins and out:
            avg_i = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in ins) / len(ins)
            avg_o = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in out) / len(out)
            lines.append(f"`{kname}` in the stage: {len(ins)} launches, {avg_i / 1e3:.1f} us on "
                         f"average; alone (bench.py's attention cases after the stage): "
                         f"{len(out)} launches, {avg_o / 1e3:.1f} us.")
    # the gemm_dgrad_gu case: the input-gradient form's launches after the
    # stage and before the gemm_wgrad_gu case's first (both-K-major) launch --
    # the LM head cases later in the run use the same form at other shapes
    tn = [i for i, r in enumerate(after)
          if "gemm_tiled_kernel" in r["Kernel_Name"] and "Lb1ELb1E" in r["Kernel_Name"]]
    nn = [r for r in after[:tn[0] if tn else len(after)]
          if "gemm_tiled_kernel" in r["Kernel_Name"] and "Lb0ELb1E" in r["Kernel_Name"]]
    if nn:
        avg = sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in nn) / len(nn)
        lines.append(f"`gemm_tiled_kernel<bf16,0,false,true>` in bench.py's `gemm_dgrad_gu` case "
                     f"after the stage (the `roofline` kernel; gate|up input gradient, 4096 x "
                     f"4096 x 22016): {len(nn)} launches, {avg / 1e6:.3f} ms on average.  In the "
                     f"stage the same kernel runs every input-gradient shape, so its table "
                     f"average below mixes them.")
    lines += ["", "All kernels of the run (rocprofv3 `bench_kernel_stats.csv`, top 30):", "",
              "| kernel | calls | total ms | avg us | % |", "|---|---|---|---|---|"]
    stats = list(csv.DictReader(open(os.path.join(root, "bench_kernel_stats.csv"))))
    for r in stats[:30]:
        lines.append(f"| `{r['Name'][:110]}` | {r['Calls']} | "
                     f"{float(r['TotalDurationNs']) / 1e6:.2f} | "
                     f"{float(r['AverageNs']) / 1e3:.1f} | {float(r['Percentage']):.2f} |")
    return "\n".join(lines) + "\n"


# kernel-case labels (as in the JSON line) and the rocprofv3 kernel names they cover
TRAFFIC_CASES = {
    "attn_fwd": ("attn_fwd_kernel<bf16,128,full>", ("attn_fwd_kernel",)),
    "attn_bwd": ("zk_attn_bwd (attn_bwd_dq + attn_bwd_dkdv)",
                 ("attn_bwd_dkdv", "attn_bwd_dq")),
    "rmsnorm_fwd": ("rmsnorm_fwd_vec<bf16,bf16,128,4>", ("rmsnorm_fwd_vec",)),
    "rmsnorm_bwd": ("rmsnorm_bwd_vec<bf16,bf16,256,2,2> + dw reduce",
                    ("rmsnorm_bwd_vec", "rmsnorm_dw_reduce")),
    "adamw": ("adamw_elem<bf16,bf16,true>", ("adamw_elem",)),
    "adamw_t": ("adamw_tile_t<bf16,bf16> (layer step with W^T copies)", ("adamw_tile_t",)),
    "gemm_dgrad_gu": ("gemm_tiled_kernel<bf16,0,false,true> gate|up input grad 4096 x 4096 x 22016",
                      ("gemm_tiled_kernel",)),
}


MFMA_COUNTERS = ("SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES",
                 "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "GRBM_GUI_ACTIVE")


def summarize_mfma(root: str) -> str:
    """Markdown summary of one rocprofv3 ``--pmc`` pass of MFMA_COUNTERS per
    MFMA-bound kernel case (``root/<case>/r_counter_collection.csv``):
    executed MFMA FLOPs (MOPS x 512), the clock the kernel ran at
    (GRBM_GUI_ACTIVE per XCC / duration), MFMA busy cycles per SIMD as a
    fraction of the kernel's active cycles (rocprof's MfmaUtil), and LDS bank
    conflicts per LDS access cycle."""
    import collections
    import csv
    simds, xccs = 1024, 8
    lines = ["| kernel | dispatches | avg duration (us) | clock (GHz) | MFMA FLOPs executed (GF) "
             "| MFMA busy / active cycles | LDS conflict cycles / access cycles |",
             "|---|---|---|---|---|---|---|"]
    for case in ("attn_fwd", "attn_bwd", "gemm_gu", "gemm_dgrad_gu", "gemm_wgrad_gu",
                 "blas_gu", "blas_dgrad_gu", "blas_wgrad_gu"):
        path = os.path.join(root, case, "r_counter_collection.csv")
        if not os.path.exists(path):
            continue
        disp, meta = collections.defaultdict(dict), {}
        for r in csv.DictReader(open(path)):
            d = int(r["Dispatch_Id"])
            disp[d][r["Counter_Name"]] = float(r["Counter_Value"])
            meta[d] = (r["Kernel_Name"], int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        groups = collections.defaultdict(list)
        for d, c in disp.items():
            name, dur = meta[d]
            if c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0) > 0:
                groups[name.split("(")[0][:60]].append((dur, c))
        for name, items in groups.items():
            n = len(items)
            dur = sum(t for t, _ in items) / n
            avg = {k: sum(c[k] for _, c in items) / n for k in MFMA_COUNTERS}
            cycles = avg["GRBM_GUI_ACTIVE"] / xccs
            busy = avg["SQ_VALU_MFMA_BUSY_CYCLES"] / simds
            lds = avg["SQ_LDS_IDX_ACTIVE"] - avg["SQ_LDS_BANK_CONFLICT"]
            conf = avg["SQ_LDS_BANK_CONFLICT"] / lds if lds > 0 else 0.0
            lines.append(f"| `{name}` ({case}) | {n} | {dur / 1e3:.1f} | {cycles / dur:.2f} "
                         f"| {avg['SQ_INSTS_VALU_MFMA_MOPS_BF16'] * 512 / 1e9:.1f} "
                         f"| {100 * busy / cycles:.1f} % | {conf:.3f} |")
    return "\n".join(lines) + "\n"


def summarize_traffic(root: str) -> str:
    """Markdown summary of rocprofv3 FETCH_SIZE / WRITE_SIZE runs of the kernel
    cases (``root/<case>_<COUNTER>/r_counter_collection.csv``), calibrated by
    the 1 GiB device copy of the ``copy`` case; the machine-readable lines are
    what ``recorded_traffic`` reads."""
    import csv
    from zorse_amd.layer import LayerSpec

    def per_dispatch(case, counter, names):
        vals = {}
        path = os.path.join(root, f"{case}_{counter}", "r_counter_collection.csv")
        for r in csv.DictReader(open(path)):
            if any(n in r["Kernel_Name"] for n in names):
                key = (r["Kernel_Name"], r["Dispatch_Id"])
                vals[key] = vals.get(key, 0.0) + float(r["Counter_Value"])
        by_kernel = {}
        for (k, _), v in vals.items():
            by_kernel.setdefault(k, []).append(v)
        # one launch of the case = one dispatch of each of its kernels (the mean)
        return sum(sum(v) / len(v) for v in by_kernel.values())

    copy_fetch = per_dispatch("copy", "FETCH_SIZE", ("copyBuffer",))
    copy_write = per_dispatch("copy", "WRITE_SIZE", ("copyBuffer",))
    gib_kib = float(1 << 20)
    f_fac, w_fac = gib_kib / copy_fetch, gib_kib / copy_write
    from zorse_amd import flops
    spec = LayerSpec(hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
    T, h, H, d = 4096, spec.hidden, spec.heads, spec.head_dim
    algo = {"attn_fwd": flops.attn_fwd_bytes(1, T, H, H, d),
            "attn_bwd": flops.attn_bwd_bytes(1, T, H, H, d),
            "rmsnorm_fwd": flops.rmsnorm_fwd_bytes(T, h),
            "rmsnorm_bwd": flops.rmsnorm_bwd_bytes(T, h),
            "adamw": flops.adamw_bytes(spec.numel, 2, True),
            "adamw_t": flops.adamw_bytes(spec.numel, 2, True)
            + 2 * (spec.numel - 2 * spec.hidden),
            # compulsory bytes of dX = dY W: dY [T, 2F] and W [2F, h] read, dX [T, h] written
            "gemm_dgrad_gu": 2 * (T * 2 * spec.ffn + 2 * spec.ffn * h + T * h)}
    lines = ["| kernel | FETCH_SIZE (MiB) | WRITE_SIZE (MiB) | HBM traffic (MB) | "
             "algorithmic bytes (MB) | traffic / algorithmic |", "|---|---|---|---|---|---|"]
    machine = []
    for case, (label, names) in TRAFFIC_CASES.items():
        fk = per_dispatch(case, "FETCH_SIZE", names)
        wk = per_dispatch(case, "WRITE_SIZE", names)
        traffic = (fk * f_fac + wk * w_fac) * 1024
        a = algo[case]
        lines.append(f"| `{label}` | {fk / 1024:.1f} | {wk / 1024:.1f} | {traffic / 1e6:.1f} | "
                     f"{a / 1e6:.1f} | {traffic / a:.3f} |")
        machine.append(f"traffic_bytes_per_launch {label} {int(round(traffic))}")
    head = (f"Calibration (case `copy`: 1 GiB read + 1 GiB written by one device copy): "
            f"HBM bytes = FETCH_SIZE x {f_fac:.3f} + WRITE_SIZE x {w_fac:.3f} (KiB per dispatch).")
    return "\n".join([head, ""] + lines + ["", "Machine-readable (read by bench.py for the "
                                                "`traffic` fields):", ""] + machine) + "\n"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--seq", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernel", choices=KernelCases.NAMES,
                    help="launch only this kernel case --steps times (for rocprofv3 --pmc)")
    ap.add_argument("--fused-mlp", choices=("on", "off"), default="on",
                    help="gate|up GEMM with the SwiGLU epilogue (zk_gemm_swiglu) in the stage")
    ap.add_argument("--summarize-mfma", metavar="DIR",
                    help="print the MFMA-counter summary of rocprofv3 runs under DIR and exit")
    ap.add_argument("--summarize-traffic", metavar="DIR",
                    help="print the HBM-traffic table from rocprofv3 --pmc runs of the kernel "
                         "cases under DIR and exit (no GPU needed)")
    ap.add_argument("--summarize-stage", metavar="DIR",
                    help="print the per-group kernel time of a rocprofv3 --kernel-trace --stats "
                         "run of this bench (DIR holds bench_kernel_trace.csv / "
                         "bench_kernel_stats.csv; pass that run's --steps / --warmup / "
                         "--layers) and exit (no GPU needed)")
    args = ap.parse_args()
    if args.summarize_stage:
        print(summarize_stage(args.summarize_stage, args.layers, args.steps, args.warmup), end="")
        return
    if args.summarize_mfma:
        print(summarize_mfma(args.summarize_mfma), end="")
        return
    if args.summarize_traffic:
        print(summarize_traffic(args.summarize_traffic), end="")
        return
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(collectives and sharding are out of scope); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    from zorse_amd import flops
    from zorse_amd import layer as _layer_mod
    from zorse_amd.stage import StageRunner

    _layer_mod.set_fused_gate_up(args.fused_mlp == "on")

    S, B = args.seq, 1
    if args.kernel:
        from zorse_amd.layer import LayerSpec
        spec = LayerSpec(hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
        run, work = KernelCases(dev, spec, S).make(args.kernel)
        ms = _events_time(run, args.steps, warm=args.warmup)
        print(json.dumps({"kernel": args.kernel, "launches": args.steps, "avg_ms": round(ms, 4),
                          "work_per_launch": work}), flush=True)
        return
    cfg, layers, g = build_stage(args.layers, dev)
    spec = layers[0].spec
    runner = StageRunner(layers, lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    x = torch.randn(B, S, spec.hidden, generator=g).to(torch.bfloat16).to(dev)
    dout = torch.randn(B, S, spec.hidden, generator=g).to(torch.bfloat16).to(dev)
    x.requires_grad_(False)

    for i in range(args.warmup):
        runner.step(x, dout)
        print(f"warmup step {i + 1}/{args.warmup} done", file=sys.stderr, flush=True)
    runner.wait_optimizer()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        runner.step(x, dout)
    runner.wait_optimizer()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = 1e3 * elapsed / args.steps
    print(f"timed {args.steps} steps: {ms_step:.2f} ms/step", file=sys.stderr, flush=True)
    layer_toks = args.layers * B * S / (ms_step / 1e3)
    layer_tflops = flops.layer_fwd_bwd_flops(spec, B, S) * args.layers / (ms_step / 1e3) / 1e12
    del runner, layers, x, dout
    torch.cuda.empty_cache()

    kern = measure_kernels(dev, spec, S)
    print("kernel timings done", file=sys.stderr, flush=True)
    cpu = None if args.no_cpu else cpu_baseline(spec, S)
    # the roofline line: the kernel with the largest share of the stage's
    # kernel time, the hand-written GEMM in its input-gradient form (the four
    # dY W products and the gate|up / q|k|v weight gradients on dY^T), at its
    # largest launch; the HBM-bound AdamW step beside it
    gm = kern["gemm_dgrad_gu"]
    a = kern["adamw"]
    af, ab = kern["attn_fwd"], kern["attn_bwd"]
    line = {
        "metric": "decoder-layer fwd+bwd tokens/s at 1 GPU; attention TFLOP/s vs MFMA peak",
        "value": round(layer_toks, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(layer_toks / H100_FP16_LAYER_TOKS, 3),
        "vs_baseline_ref": "H100-NVL fp16 7B layer seq 4096 mb 1, 221,477 tok/s/layer "
                           "(data/model_latencies.json:7551; other GPU and dtype, no AdamW)",
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations / grads, N(0,0.02) weights)",
        "config": {"workload": "llama2-7b-shaped pipeline stage fwd+bwd + per-layer AdamW in "
                               "backward (BASELINE configs[3])",
                   "layers": args.layers, "hidden": spec.hidden, "heads": spec.heads,
                   "head_dim": spec.head_dim, "ffn": spec.ffn, "micro_batch": B, "seq_len": S,
                   "global_batch": B, "parallelism": "none (1 GPU)",
                   "gate_up_swiglu": ("fused (zk_gemm_swiglu)" if _layer_mod._fused_gate_up
                                      else "zk_gemm + zk_swiglu_fwd"),
                   "projection_gemms": "hand-written zk_gemm (zorse_amd/csrc/gemm.hip) for all "
                                       "twelve products per layer, on untransposed operands",
                   "stage_tokens_per_s": round(B * S / (ms_step / 1e3), 1),
                   "layer_fwd_bwd_tflops": round(layer_tflops, 1)},
        "roofline": {"bound": gm["bound"], "achieved": gm["achieved"], "peak": gm["peak"],
                     "unit": gm["unit"], "frac": gm["frac"],
                     "traffic": gm["traffic"],
                     "kernel": gm["kernel"], "avg_ms": gm["avg_ms"],
                     "algorithmic_flops": gm["work_per_launch"],
                     "scope": "the kernel with the largest share of the stage's kernel time "
                              "(the hand-written GEMM's input-gradient form), at the stage's "
                              "largest launch of it: dX = dY W for gate|up, 2 x 4096 x 4096 x "
                              "22016 FLOPs"},
        "hbm_roofline": {"bound": a["bound"], "achieved": a["achieved"], "peak": a["peak"],
                         "unit": a["unit"], "frac": a["frac"],
                         "traffic": a["traffic"],
                         "kernel": a["kernel"], "avg_ms": a["avg_ms"],
                         "algorithmic_bytes": a["work_per_launch"],
                         "scope": "one launch over a layer's flat shard: the stage's whole "
                                  "optimizer step per layer; its 5.7 GB per launch is far "
                                  "larger than the Infinity Cache"},
        "attention_roofline": {
            "fwd": {"kernel": af["kernel"], "achieved": af["achieved"], "peak": af["peak"],
                    "unit": "TFLOP/s", "frac": af["frac"], "avg_ms": af["avg_ms"],
                    "traffic": af["traffic"]},
            "bwd": {"kernel": ab["kernel"], "achieved": ab["achieved"], "peak": ab["peak"],
                    "unit": "TFLOP/s", "frac": ab["frac"], "avg_ms": ab["avg_ms"],
                    "traffic": ab["traffic"]}},
        "kernels": kern,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

"""Layer profiler counterpart: times one decoder layer with the reference's
protocol and writes the result in the reference's latency-table format, so
the planner can plan for MI355X.

Protocol reproduced (utils/runtime_estimator.py:187-253, utils/profile.py:
96-130, bench/bench_layer.py, profile_models.sh:21):
  * a 1-layer model; the layer is fed the embedding of random token ids
    under ``torch.autocast(dtype)``, ``requires_grad`` set;
  * 15 forwards, each followed by a device synchronize and a 50 ms sleep,
    then ``grads = torch.rand(out.shape)`` and 15 ``out.backward(grads,
    retain_graph=True)``;
  * the time of one pass is the SUM OF GPU KERNEL DURATIONS (launch gaps and
    host time excluded) divided by the iteration count -- taken here from
    torch.profiler's device kernel events, which on ROCm come from the same
    kernel trace rocprofv3 reads;
  * micro-batch sizes 1..P, then a least-squares line per direction;
  * the optimizer step (fused Adam on the layer's parameters sliced to 1/N,
    ``grad = torch.rand``) timed over 50 steps for N = 1..8
    (utils/runtime_estimator.py:256-279).
Output entry (utils/runtime_estimator.py:388-414, read back by
utils/optimizer_utils.py:59-125):
    latencies[model][gpu][str(seq)][dtype] =
        [(slope_fwd, icpt_fwd), (slope_bwd, icpt_bwd), [fwd_ms...], [bwd_ms...]]
The GPU tables below add MI355X to the reference's GPU_MEMORY
(utils/runtime_estimator.py:22-38) and GPU_TFLOPs (utils/train_utils.py:
245-273), whose absence makes the planner's memory check raise
(zorse_optimizer/utils.py:52).
"""
from __future__ import annotations

import argparse
import json
import os
import time

import numpy as np
import torch

# GiB of device memory and dense matrix TFLOP/s (no sparsity) per GPU name
GPU_MEMORY = {"mi355x": 288.0}
GPU_TFLOPS = {
    "float32": {"mi355x": 157.3},
    "float16": {"mi355x": 2516.6},
    "bfloat16": {"mi355x": 2516.6},
}
DTYPE_NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


def clean_gpu_name(gpu_name: str) -> str:
    """utils/comm.py:70-88: lower-cased last word of the device name
    ("AMD Instinct MI355X" -> "mi355x")."""
    return gpu_name.lower().split(" ")[-1]


# architecture -> table name, for devices whose marketing name the runtime
# does not report (without the libdrm ids file it says "AMD Radeon Graphics")
ARCH_NAMES = {"gfx950": "mi355x"}


def gpu_name(device: int = 0) -> str:
    arch = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "").split(":")[0]
    if arch in ARCH_NAMES:
        return ARCH_NAMES[arch]
    return clean_gpu_name(torch.cuda.get_device_name(device))


def fit_line(y_values):
    """utils/profile.py:124-130: least-squares line through (1, y1), (2, y2)..."""
    x_values = np.arange(len(y_values)) + 1
    slope, intercept = np.polyfit(x_values, y_values, 1)
    return float(slope), float(intercept)


def _kernel_ms(fn, num_iterations: int, delay: float) -> float:
    """Sum of device kernel time over ``num_iterations`` calls of ``fn`` (each
    followed by a synchronize and ``delay`` seconds of sleep), divided by the
    iteration count (utils/profile.py:96-121)."""
    from torch.profiler import ProfilerActivity, profile
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        for _ in range(num_iterations):
            fn()
            torch.cuda.synchronize()
            if delay:
                time.sleep(delay)
    total_us = 0.0
    for ev in prof.events():
        if ev.device_type == torch.autograd.DeviceType.CUDA and ev.device_time_total > 0 \
                and not ev.name.startswith(("Memcpy", "Memset")):
            total_us += ev.device_time
    if total_us <= 0:
        raise RuntimeError("the profiler recorded no device kernels")
    return total_us / 1e3 / num_iterations


def get_compute_latency(layer, batch_size, seq_length, hidden, dtype, vocab_size=49152,
                        num_iterations=15, delay=0.05, seed=0):
    """(forward ms, backward ms) of ``layer`` for one micro-batch
    (utils/runtime_estimator.py:187-253)."""
    dev = next(layer.parameters()).device
    g = torch.Generator(device="cpu").manual_seed(seed + batch_size)
    ids = torch.randint(0, vocab_size, (batch_size, seq_length), generator=g)
    table = torch.randn(vocab_size, hidden, generator=g)
    emb = table[ids].to(dev).to(dtype).requires_grad_(True)
    out_box = []

    def fwd():
        with torch.autocast("cuda", dtype=dtype):
            o = layer(emb)
        out_box[:] = [o[0] if isinstance(o, tuple) else o]

    # the protocol sums kernel durations, which counts kernels that overlap
    # on two streams twice: the layer backward's weight-gradient GEMMs run in
    # order on the compute stream while it is measured
    from .layer import set_wgrad_stream
    prev = set_wgrad_stream(False)
    try:
        fwd_ms = _kernel_ms(fwd, num_iterations, delay)
        out = out_box[0]
        grads = torch.rand(out.shape, device=out.device, dtype=out.dtype)
        bwd_ms = _kernel_ms(lambda: out.backward(grads, retain_graph=True), num_iterations,
                            delay)
    finally:
        set_wgrad_stream(prev)
    return fwd_ms, bwd_ms


def get_optimizer_latency(layer, num_shards=1, num_iterations=50):
    """Fused Adam step on the layer's parameters sliced to their first
    1/num_shards rows, ``grad = torch.rand`` (utils/runtime_estimator.py:
    256-279)."""
    from .optim import FusedAdam
    params = []
    for p in layer.parameters():
        sl = torch.nn.Parameter(p.detach()[: max(1, p.shape[0] // num_shards)].clone().float())
        sl.grad = torch.rand_like(sl)
        params.append(sl)
    opt = FusedAdam(params)
    torch.cuda.synchronize()
    return _kernel_ms(opt.step, num_iterations, 0.0)


def profile_model(model_name, seq_length=4096, dtype=torch.bfloat16, profile_batches=4,
                  vocab_size=49152, num_iterations=15, delay=0.05, max_shards=8,
                  device="cuda"):
    """Profile the first layer of a 1-layer model; returns (entry, optimizer
    ms per shard count)."""
    from . import hf_models, llama_simple, mistral_simple
    name = model_name.lower()
    if name.startswith(("llama", "mistral")):   # the HF-factory routes
        model = hf_models.get_model(name, vocab_size=vocab_size, seq_length=seq_length, layers=1)
        layer = hf_models.get_layers(model)[0].to(device)
    else:
        mod = mistral_simple if name.startswith("deepspeedmistral") else llama_simple
        model = mod.get_model(model_name, vocab_size=vocab_size, seq_length=seq_length, layers=1)
        layer = model.layers[0].to(device)
    opt_ms = {n: get_optimizer_latency(layer, n) for n in range(1, max_shards + 1)}
    fwd, bwd = [], []
    for bs in range(1, profile_batches + 1):
        try:
            f, b = get_compute_latency(layer, bs, seq_length, model._hidden_size, dtype,
                                       vocab_size, num_iterations, delay)
        except torch.cuda.OutOfMemoryError as e:  # the reference skips OOM batch sizes
            print(f"skipping batch size {bs}: {e}")
            continue
        fwd.append(f)
        bwd.append(b)
    if len(fwd) < 2:
        raise RuntimeError("need at least two profiled batch sizes to fit a line")
    entry = [fit_line(fwd), fit_line(bwd), fwd, bwd]
    return entry, opt_ms


def update_latency_table(path, model_name, gpu, seq_length, dtype_name, entry):
    """Insert ``entry`` at latencies[model][gpu][str(seq)][dtype] of the JSON
    table at ``path`` (created if missing), as utils/runtime_estimator.py:
    392-414 does."""
    table = {}
    if os.path.exists(path):
        with open(path) as f:
            table = json.load(f)
    table.setdefault(model_name, {}).setdefault(gpu, {}).setdefault(str(seq_length), {})
    table[model_name][gpu][str(seq_length)][dtype_name] = [tuple(entry[0]), tuple(entry[1]),
                                                           list(entry[2]), list(entry[3])]
    with open(path, "w") as f:
        json.dump(table, f, ensure_ascii=False, indent=4, sort_keys=True)
    return table


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--model_name", default="deepspeedllama_7b")
    ap.add_argument("--seq_length", type=int, default=4096)
    ap.add_argument("--autocast_dtype", default="bfloat16", choices=["float32", "float16", "bfloat16"])
    ap.add_argument("--profile_batches", type=int, default=4)
    ap.add_argument("--vocab_size", type=int, default=49152)
    ap.add_argument("--out", default="model_latencies.json")
    args = ap.parse_args(argv)
    dtype = getattr(torch, args.autocast_dtype)
    entry, opt_ms = profile_model(args.model_name, args.seq_length, dtype, args.profile_batches,
                                  args.vocab_size)
    gpu = gpu_name()
    os.makedirs(os.path.dirname(os.path.abspath(args.out)), exist_ok=True)
    update_latency_table(args.out, args.model_name, gpu, args.seq_length, args.autocast_dtype, entry)
    print(json.dumps({"model": args.model_name, "gpu": gpu, "seq": args.seq_length,
                      "dtype": args.autocast_dtype, "fwd_ms": entry[2], "bwd_ms": entry[3],
                      "fit_fwd": entry[0], "fit_bwd": entry[1],
                      "optimizer_ms_per_shards": opt_ms}))


if __name__ == "__main__":
    main()

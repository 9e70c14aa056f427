"""Benchmark of the E8 HNLQ hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload ("C2"): 2^24 fp32 8-wide blocks ~ N(0,1)
(seeded), fixed beta = 1, q = 4, M = 2.  One step = the fused encode -> decode
pass over all blocks, writing packed level words (uint16 x 2 per block) and
the decoded fp32 blocks.  Inputs are resident in HBM before timing starts.

Prints one JSON line: whole-job Gblocks/s, the HBM roofline of the codec
kernel (HIP events on the launch stream) and the CPU oracle timed on a
bounded sample of the same workload on the host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
C2_BLOCKS = 1 << 24
C2_BYTES_PER_BLOCK = 32 + 4 + 32   # read x, write 2 u16 words, write decoded
METRIC = "E8 HNLQ encode+decode Gblocks/s & HBM GB/s; vLUT matmul tokens/s at 4096²"


def traffic_from_profile():
    """HBM bytes per launch measured by rocprofv3 PMC (profiles/), if recorded."""
    p = os.path.join(ROOT, "profiles", "hnlq_roundtrip_c2_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def cpu_baseline(x_sample: np.ndarray):
    """The C oracle (single thread) on a bounded slice of the same workload."""
    from oracle import oracle as O
    O.lib()
    t0 = time.perf_counter()
    codes = O.e8_encode(x_sample, 4, 2, 1.0)
    O.e8_decode(codes, 4, 2, 1.0)
    dt = time.perf_counter() - t0
    n = x_sample.shape[0]
    return {"value": n / dt / 1e9, "unit": "Gblocks/s", "cores": 1, "kind": "port",
            "sample": f"first {n} of the 2^24 C2 blocks (q4 M2 beta 1), C oracle enc+dec, "
                      f"{dt:.1f} s on one host core"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-sample", type=int, default=1 << 23,
                    help="blocks timed on the host CPU oracle (0 skips it)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        sys.exit("bench.py measures one GPU only: this build has no multi-GPU path "
                 "(run with --gpus 1)")

    import torch
    import coset_amd
    from coset_amd import _lib

    dev = _lib.require_gpu()
    n = C2_BLOCKS
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn((n, 8), device=dev, generator=g, dtype=torch.float32)
    packed = torch.empty((n, 2), dtype=torch.uint16, device=dev)
    out = torch.empty((n, 8), dtype=torch.float32, device=dev)

    def step():
        coset_amd.hnlq_roundtrip(x, 4, 2, 1.0, packed_out=packed, decoded_out=out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = e0.elapsed_time(e1)
    kernel_s = gpu_ms / 1e3 / args.steps
    ms_per_step = wall * 1e3 / args.steps

    # parity spot check of this very run (not timed)
    from oracle import oracle as O
    idx = torch.randint(0, n, (4096,), device=dev, generator=g)
    xs = x[idx].cpu().numpy()
    codes = O.e8_encode(xs, 4, 2, 1.0)
    ok = (np.array_equal(packed.cpu().numpy().astype(np.uint32)[idx.cpu().numpy()],
                         O.pack_words(codes, 4))
          and np.array_equal(out[idx].cpu().numpy(), O.e8_decode(codes, 4, 2, 1.0)))
    if not ok:
        sys.exit("parity spot check FAILED: GPU codes differ from the oracle")

    achieved = C2_BYTES_PER_BLOCK * n / kernel_s / 1e9
    cpu = None
    if args.cpu_sample > 0:
        cpu = cpu_baseline(x[: args.cpu_sample].cpu().numpy())
    value = n / (wall / args.steps) / 1e9
    rec = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "Gblocks/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) blocks, seed 2",
        "config": {"workload": "C2 bulk E8 HNLQ encode->decode", "blocks": n, "q": 4, "M": 2,
                   "beta": 1.0, "outputs": "packed u16 words + decoded fp32"},
        "hbm_gbs": round(achieved, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profile()},
        "kernel_us": round(kernel_s * 1e6, 2),
        "parity": "bit-exact vs oracle on 4096 sampled blocks",
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark of the BitSparse activation-compression path on one MI355X.

Headline (``value``): compress + decompress throughput of a 16384x16384 bf16
ReLU activation at 50% zeros (the shape its target
is quoted on), in algorithmic GB/s, inputs resident in HBM.  One step =
TensorBuffer reset + fused single-pass compress + full decompress.

Also reported on the same line:
  roofline      dominant kernel (compress), HIP-event timed on its stream
  kernels       per-kernel achieved GB/s for compress / decompress
  mlp           configs[1] GPT-2-small MLP fwd+bwd: compressed vs dense
                activation (step and backward ms, saved-activation bytes)
  cpu_baseline  the C oracle (single thread) on a bounded row sample of the
                same workload, same unit

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-mlp] [--skip-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "compress+decompress GB/s (% HBM peak); MLP fwd+bwd step ms; bytes saved"
HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def codec_bytes(M: int, N: int, nnz: int, vb_in: int = 2, vb: int = 2, vb_out: int = 2):
    """Algorithmic HBM bytes of one compress and one decompress launch."""
    T = ((M + 63) // 64) * ((N + 63) // 64)
    meta = M * N // 8 + 4 * (T + 1)
    return M * N * vb_in + meta + nnz * vb, meta + nnz * vb + M * N * vb_out


def make_activation(M: int, N: int, mu: float, device):
    import torch
    g = torch.Generator(device=device).manual_seed(0)
    return (torch.randn((M, N), device=device, generator=g) + mu).to(torch.bfloat16).relu_()


def bench_codec(M: int, N: int, mu: float, steps: int, warmup: int):
    import torch
    from bitsparse_amd import _lib
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.src.functions import dense_to_tilesparse
    from bitsparse_amd.src.hip_operators import unpack_batch_

    dev = torch.device("cuda", 0)
    x = make_activation(M, N, mu, dev)
    buf = TensorBuffer(2 * M * N, device=dev)
    out = torch.empty_like(x)
    gm, gn = (M + 63) // 64, (N + 63) // 64

    def step(ev=None):
        buf.reset_buffer()
        if ev is not None:
            ev[0].record()
        sp = dense_to_tilesparse(x, None, buf)
        if ev is not None:
            ev[1].record()
        unpack_batch_(sp, out, 0, gn, N, M, gm * gn)
        if ev is not None:
            ev[2].record()
        return sp

    for _ in range(warmup):
        sp = step()
    torch.cuda.synchronize()
    assert torch.equal(out, x), "round trip mismatch"
    nnz = int(sp.prefix[-1].item())
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    c_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / steps
    d_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / steps
    cb, db = codec_bytes(M, N, nnz)
    ws = _lib.workspace_for(dev)
    res = {
        "M": M, "N": N, "nnz": nnz, "sparsity": round(1 - nnz / (M * N), 4),
        "compress_ms": c_ms, "decompress_ms": d_ms,
        "compress_gbs": cb / (c_ms * 1e6), "decompress_gbs": db / (d_ms * 1e6),
        "roundtrip_gbs": (cb + db) / ((c_ms + d_ms) * 1e6),
        "compress_bytes": cb, "decompress_bytes": db,
        "step_ms_wall": wall * 1e3 / steps,
        "lookback_fallbacks": ws.fallback_count(),
        "stored_bytes": sp.vram_size(), "dense_bytes": 2 * M * N,
    }
    return res


def bench_mlp(steps: int, warmup: int):
    """8192 x 768 -> 3072 -> 768 bf16, W ~ N(0, 0.02), x, dY ~ N(0, 1)."""
    import torch
    from bitsparse_amd.bitsparse import TensorBuffer
    from bitsparse_amd.dense import DenseFFNRelu
    from bitsparse_amd.layers import FFNRelu

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(0)
    B, D, H = 8192, 768, 3072
    x = torch.randn((8, 1024, D), device=dev, generator=g).to(torch.bfloat16).requires_grad_()
    W1 = (0.02 * torch.randn((H, D), device=dev, generator=g)).to(torch.bfloat16).requires_grad_()
    W2 = (0.02 * torch.randn((D, H), device=dev, generator=g)).to(torch.bfloat16).requires_grad_()
    dY = torch.randn((8, 1024, D), device=dev, generator=g).to(torch.bfloat16)
    buf = TensorBuffer(2 * B * H, device=dev)

    def run(compressed: bool, ev=None):
        for p in (x, W1, W2):
            p.grad = None
        if ev is not None:
            ev[0].record()
        if compressed:
            buf.reset_buffer()
            y = FFNRelu.apply(x, W1, W2, sparse_data=buf)
        else:
            y = DenseFFNRelu.apply(x.reshape(-1, D), W1, W2).reshape(8, 1024, D)
        if ev is not None:
            ev[1].record()
        y.backward(dY)
        if ev is not None:
            ev[2].record()

    out = {}
    for mode in ("dense", "compressed"):
        comp = mode == "compressed"
        for _ in range(warmup):
            run(comp)
        torch.cuda.synchronize()
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
        for i in range(steps):
            run(comp, evs[i])
        torch.cuda.synchronize()
        out[mode] = {
            "step_ms": sum(e[0].elapsed_time(e[2]) for e in evs) / steps,
            "fwd_ms": sum(e[0].elapsed_time(e[1]) for e in evs) / steps,
            "bwd_ms": sum(e[1].elapsed_time(e[2]) for e in evs) / steps,
        }
    # saved activation bytes (reference BitsparseTensor.vram_size definition)
    from bitsparse_amd.src.functions import dense_to_tilesparse
    with torch.no_grad():
        h = (x.reshape(-1, D) @ W1.T).relu_()
        buf.reset_buffer()
        sp = dense_to_tilesparse(h, None, buf)
        stored = sp.vram_size()
    dense_bytes = 2 * B * H
    out["saved_activation_bytes"] = {"dense": dense_bytes, "compressed": stored,
                                     "saved": dense_bytes - stored,
                                     "ratio": round(stored / dense_bytes, 4)}
    out["bwd_ratio_compressed_over_dense"] = out["compressed"]["bwd_ms"] / out["dense"]["bwd_ms"]
    out["step_ratio_compressed_over_dense"] = out["compressed"]["step_ms"] / out["dense"]["step_ms"]
    return out


def cpu_baseline_codec(N: int, mu: float, budget_s: float = 12.0):
    """C oracle compress + decompress (one thread) on row blocks of the
    workload's distribution, repeated for about `budget_s` seconds."""
    import numpy as np
    import torch
    from oracle import oracle as O

    rows = 1024
    g = torch.Generator().manual_seed(0)
    x = (torch.randn((rows, N), generator=g) + mu).to(torch.bfloat16).relu_()
    xb = x.view(torch.int16).numpy().view(np.uint16)
    T = (rows // 64) * ((N + 63) // 64)
    bm = np.zeros(T * 512, np.uint8)
    pf = np.zeros(T + 1, np.uint32)
    cnt = np.zeros(T, np.int32)
    vals = np.zeros(rows * N, np.uint16)
    reps, t_c, t_d = 0, 0.0, 0.0
    nnz = 0
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < budget_s or reps < 2:
        a = time.perf_counter()
        nnz = O.compress_timed_call(xb, O.BF16, bm, pf, cnt, vals)
        b = time.perf_counter()
        out = O.decompress(vals, O.BF16, bm, pf, rows, N)
        c = time.perf_counter()
        t_c += b - a
        t_d += c - b
        reps += 1
    assert (out == xb).all()
    cb, db = codec_bytes(rows, N, nnz)
    return {"value": round((cb + db) * reps / ((t_c + t_d) * 1e9), 4), "unit": "GB/s",
            "cores": 1, "kind": "port",
            "sample": f"{rows}x{N} row block (seed 0), {reps} compress+decompress reps, "
                      f"C oracle -O2 single thread",
            "compress_gbs": round(cb * reps / (t_c * 1e9), 4),
            "decompress_gbs": round(db * reps / (t_d * 1e9), 4)}


def cpu_baseline_mlp(budget_s: float = 15.0):
    """Dense comparator MLP fwd+bwd in PyTorch on the host cores, bf16, on a
    1024-row slice of configs[1] (scaled x8 to the 8192-row step)."""
    import torch
    from bitsparse_amd.dense import DenseFFNRelu
    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(0)
    rows, D, H = 1024, 768, 3072
    x = torch.randn((rows, D), generator=g).to(torch.bfloat16).requires_grad_()
    W1 = (0.02 * torch.randn((H, D), generator=g)).to(torch.bfloat16).requires_grad_()
    W2 = (0.02 * torch.randn((D, H), generator=g)).to(torch.bfloat16).requires_grad_()
    dY = torch.randn((rows, D), generator=g).to(torch.bfloat16)
    times = []
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s or len(times) < 3:
        a = time.perf_counter()
        DenseFFNRelu.apply(x, W1, W2).backward(dY)
        times.append(time.perf_counter() - a)
        x.grad = W1.grad = W2.grad = None
    times.sort()
    med = times[len(times) // 2]
    return {"step_ms_full_batch_est": round(med * 1e3 * 8192 / rows, 2), "sample_rows": rows,
            "reps": len(times), "threads": torch.get_num_threads(), "dtype": "bf16"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sparsity-mu", type=float, default=0.0,
                    help="pre-activation mean (0 -> 50%% zeros)")
    ap.add_argument("--skip-mlp", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 1 GiB device copy (reference for rocprof byte counters)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures the single-GPU path only: the compressed activation never "
              "leaves its rank, so there is no multi-GPU figure to report (run with --gpus 1).",
              file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    from bitsparse_amd import _lib
    _lib.load()

    M = N = 16384
    log(f"codec: {M}x{N} bf16, mu={args.sparsity_mu}, steps={args.steps}, warmup={args.warmup}")
    codec = bench_codec(M, N, args.sparsity_mu, args.steps, args.warmup)
    log(f"codec done: {codec['roundtrip_gbs']:.1f} GB/s round trip")
    if args.calibrate_copy:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    mlp = None
    if not args.skip_mlp:
        log("mlp: configs[1] GPT-2-small block")
        mlp = bench_mlp(max(5, args.steps // 2), max(2, args.warmup // 2))
        log("mlp done")
    cpu = None
    cpu_mlp = None
    if not args.skip_cpu:
        log("cpu baseline: C oracle codec")
        cpu = cpu_baseline_codec(N, args.sparsity_mu)
        log("cpu baseline: dense MLP on host cores")
        if not args.skip_mlp:
            cpu_mlp = cpu_baseline_mlp()
            mlp["cpu_dense_mlp"] = cpu_mlp

    step_ms = codec["compress_ms"] + codec["decompress_ms"]
    # HBM bytes per compress launch from the committed rocprofv3 counter runs
    # (FETCH_SIZE / WRITE_SIZE, scaled by a 1 GiB copy in the same process);
    # only meaningful for the default workload
    traffic = None
    prof = os.path.join(ROOT, "profiles", "compress_decompress_16384x16384_bf16_s50.json")
    if args.sparsity_mu == 0.0 and os.path.exists(prof):
        with open(prof) as f:
            traffic = int(json.load(f)["compress"]["hbm_traffic_bytes"])
    result = {
        "metric": METRIC,
        "value": round(codec["roundtrip_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: relu(N(mu,1)) drawn on the GPU with seed 0",
        "config": {"workload": "configs[2] 16384x16384 bf16 ReLU activation round trip "
                               "(compress to bitmask+prefix+bf16 vals, decompress)",
                   "M": M, "N": N, "sparsity": codec["sparsity"], "value_storage": "bf16",
                   "pct_hbm_peak": round(100 * codec["roundtrip_gbs"] / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(codec["compress_gbs"], 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(codec["compress_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "kernel": "compress_kernel (fused single pass)",
                     "bytes_per_launch": codec["compress_bytes"],
                     "avg_launch_ms": round(codec["compress_ms"], 5)},
        "kernels": {"compress_gbs": round(codec["compress_gbs"], 2),
                    "decompress_gbs": round(codec["decompress_gbs"], 2),
                    "compress_ms": round(codec["compress_ms"], 5),
                    "decompress_ms": round(codec["decompress_ms"], 5),
                    "lookback_fallbacks": codec["lookback_fallbacks"]},
        "bytes_saved": {"dense": codec["dense_bytes"], "stored": codec["stored_bytes"],
                        "saved": codec["dense_bytes"] - codec["stored_bytes"]},
        "mlp": mlp,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

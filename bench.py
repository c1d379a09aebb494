"""Benchmark of the MI355X int4 LLM hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-e2e] [--skip-cpu] [--sweep-gemv]

Headline (the JSON line's `value`): BASELINE config 2, the int4 decode GEMV y = W x at N=5120,
K=3072 (fused qkv), group 128, fp16 x / fp16 y, fp32 accumulation, in achieved HBM GB/s. A step is
one GEMV launch over one weight copy; the timed region replays launches over 64 rotating weight
copies (520 MB, twice the 256 MB MALL) so every launch streams its weights from HBM. Launches are
replayed from a HIP graph so the host does not throttle them. Inputs are resident in HBM before
timing starts.

Extra fields: the other GEMV shapes of config 2, and (unless --skip-e2e) the batch-1 decode tokens/s
of the Llama-3.2-3B-shaped model (config 5) with its HBM roofline fraction.

`roofline` describes the dominant kernel (the GEMV): achieved = algorithmic bytes per launch /
average launch duration from HIP events around graph replays on the launch stream.
`cpu_baseline` times the reference-faithful CPU path (the oracle's QLinear: F.linear over a
per-call dequantized fp32 weight, llama_q4.py:72) on this host's cores, on a bounded sample.
"""

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "iree-adreno-genai-tuner_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
MALL_BYTES = 256 * 2 ** 20


def gemv_bytes(N, K, group, x_bytes=2, y_bytes=2):
    """Algorithmic bytes of one GEMV: packed weights + fp16 scales + x + y."""
    return N * K // 2 + N * (K // group) * 2 + K * x_bytes + N * y_bytes


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class GemvBench:
    """A GEMV problem resident in HBM with enough weight copies to defeat the MALL."""

    def __init__(self, dev, N, K, group=128, seed=0):
        import torch
        from q4llm import synth
        self.N, self.K, self.group = N, K, group
        qw, sc, x = synth.gemv_problem(N, K, group, seed)
        self.qw0 = torch.from_numpy(qw).to(dev)
        self.sc0 = torch.from_numpy(sc).to(dev)
        self.x = torch.from_numpy(x).to(dev)
        self.bytes = gemv_bytes(N, K, group)
        n_copies = max(64, -(-2 * MALL_BYTES // self.bytes))
        self.qws = [self.qw0.clone() for _ in range(n_copies)]
        self.scs = [self.sc0.clone() for _ in range(n_copies)]
        self.y = torch.empty(N, dtype=torch.float16, device=dev)

    def launch_all(self, cfg=-1, grid=0):
        from q4llm import ops
        for qw, sc in zip(self.qws, self.scs):
            ops.q4_gemv_cfg(qw, sc, self.x, self.group, self.y, cfg=cfg, grid=grid)

    def time(self, steps, warmup, cfg=-1, grid=0):
        """Returns (ms per launch, launches timed): graph of one pass over the copies, replayed."""
        import torch
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.launch_all(cfg, grid)  # eager warm-up (also loads the code object)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            self.launch_all(cfg, grid)
        per_replay = len(self.qws)
        reps_w = max(1, -(-warmup // per_replay))
        reps = max(1, -(-steps // per_replay))
        with torch.cuda.stream(s):
            for _ in range(reps_w):
                g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(reps):
                g.replay()
            e1.record(s)
            e1.synchronize()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (reps * per_replay), reps * per_replay

    def check(self):
        """Parity of the timed configuration against the fp64 CPU oracle (1e-2 x RMS)."""
        import torch
        from oracle import llama_q4_ref as R
        from q4llm import ops
        ops.q4_gemv(self.qw0, self.sc0, self.x, self.group, out=self.y)
        ref = R.dequantize_q4(self.qw0.cpu(), self.sc0.cpu(), self.group).double() @ self.x.cpu().double()
        err = (self.y.cpu().double() - ref).abs().max().item()
        rms = ref.pow(2).mean().sqrt().item()
        return err / rms


def graph_time(fn_list, steps, warmup):
    """Average ms per launch of a list of launch closures captured into one HIP graph and replayed."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in fn_list:
            f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for f in fn_list:
            f()
    n = len(fn_list)
    with torch.cuda.stream(s):
        for _ in range(max(1, -(-warmup // n))):
            g.replay()
        reps = max(1, -(-steps // n))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            g.replay()
        e1.record(s)
        e1.synchronize()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * n)


def probe_read(dev, nbytes, loads, copies=None):
    """Measured streaming-read bandwidth (gemm/roofline.py:51-70 analogue) over rotating buffers."""
    import torch
    from q4llm._lib import LIB
    copies = copies or max(4, -(-2 * MALL_BYTES // nbytes))
    bufs = [torch.empty(nbytes // 4, dtype=torch.int32, device=dev).fill_(i) for i in range(copies)]
    sink = torch.empty(1, dtype=torch.float32, device=dev)

    def mk(b):
        return lambda: LIB.call("q4_probe_read", b.data_ptr(), nbytes, sink.data_ptr(), loads,
                                torch.cuda.current_stream().cuda_stream)
    ms = graph_time([mk(b) for b in bufs], 512, 64)
    return ms * 1e3, nbytes / ms / 1e6


def probe_empty(grid, block=256):
    import torch
    from q4llm._lib import LIB

    def f():
        LIB.call("q4_probe_empty", grid, block, torch.cuda.current_stream().cuda_stream)
    return graph_time([f] * 64, 512, 64) * 1e3


def cpu_gemv_baseline(N, K, group, seconds=10.0):
    """Reference-faithful eager QLinear on the host: F.linear(x.float(), dequantize_q4(W)) per call."""
    import numpy as np
    import torch
    from oracle import llama_q4_ref as R
    from q4llm import synth
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    qw, sc, x = synth.gemv_problem(N, K, group)
    ql = R.QLinearRef(group=group, qweight=torch.from_numpy(qw), scales=torch.from_numpy(sc), cache=False)
    xf = torch.from_numpy(x.astype(np.float32)).reshape(1, K)
    ql(xf)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        ql(xf)
        n += 1
    dt = (time.perf_counter() - t0) / n
    # best case: pre-dequantized weight
    w = ql.weight()
    m, t1 = 0, time.perf_counter()
    while time.perf_counter() - t1 < min(3.0, seconds):
        torch.nn.functional.linear(xf, w)
        m += 1
    dt_best = (time.perf_counter() - t1) / m
    b = gemv_bytes(N, K, group)
    return dict(value=round(b / dt / 1e9, 3), unit="GB/s", cores=cores, kind="port",
                sample=f"{n} eager QLinear calls (per-call dequant + F.linear fp32) at N={N},K={K},G={group}, "
                       f"{n * dt:.1f} s; pre-dequantized F.linear best case {b / dt_best / 1e9:.2f} GB/s",
                ms_per_call=round(dt * 1e3, 3), best_case_gbs=round(b / dt_best / 1e9, 3))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=256)
    ap.add_argument("--skip-e2e", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--sweep-gemv", action="store_true", help="time every GEMV tile config (tuning)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {a.gpus} is not supported (this build runs on a "
              "single MI355X; multi-GPU sharding is design-only)", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("no ROCm GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    from q4llm._lib import LIB
    LIB.load()

    shapes = [(5120, 3072), (16384, 3072), (3072, 8192)]
    results = {}
    for (N, K) in shapes:
        gb = GemvBench(dev, N, K)
        rel = gb.check()
        if a.sweep_gemv:
            for cfg in range(LIB.raw("q4_gemv_num_configs")()):
                ms, _ = gb.time(512, 64, cfg=cfg)
                log(f"sweep N={N} K={K} cfg={cfg}: {ms * 1e3:.2f} us {gb.bytes / ms / 1e6:.0f} GB/s")
        steps = a.steps if (N, K) == shapes[0] else max(256, a.steps // 4)
        ms, n = gb.time(steps, a.warmup)
        results[(N, K)] = dict(us=ms * 1e3, gbs=gb.bytes / ms / 1e6, bytes=gb.bytes, err_rel_rms=rel, launches=n)
        log(f"gemv N={N} K={K}: {ms * 1e3:.3f} us/launch, {gb.bytes / ms / 1e6:.1f} GB/s, err/rms {rel:.2e}")
        del gb
        torch.cuda.empty_cache()

    probes = {}
    for nbytes in (8126464, 12998656, 25991168, 1 << 30):
        us, gbs = min(probe_read(dev, nbytes, L) for L in (1, 4))
        probes[f"read_{nbytes}B"] = {"us": round(us, 3), "GB/s": round(gbs, 1)}
        log(f"probe read {nbytes} B: {us:.3f} us {gbs:.1f} GB/s")
    for grid in (256, 1024):
        us = probe_empty(grid)
        probes[f"empty_g{grid}"] = {"us": round(us, 3)}
        log(f"probe empty grid {grid}: {us:.3f} us")
    torch.cuda.empty_cache()

    head = results[shapes[0]]
    out = {
        "metric": "int4 GEMV achieved HBM GB/s (% of peak) + batch-1 decode tokens/s, 3B-shape",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["launches"],
        "warmup": a.warmup,
        "ms_per_step": round(head["us"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights, fp16 x/y, fp32 accumulate",
        "data": "synthetic (seeded numpy: nibbles U[0,15], scales |N(0,0.01)| fp16, x N(0,1) fp16)",
        "config": {"workload": "int4 decode GEMV y=Wx, N=5120 (fused qkv), K=3072, group 128, batch 1",
                   "N": 5120, "K": 3072, "group": 128, "weight_copies_rotated": 64},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": head["bytes"], "avg_launch_us": round(head["us"], 4)},
        "gemv_shapes": {f"{N}x{K}": {"us": round(r["us"], 3), "GB/s": round(r["gbs"], 1),
                                      "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4),
                                      "err_over_rms": float(f"{r['err_rel_rms']:.3e}")}
                        for (N, K), r in results.items()},
        "measured_probes": probes,
    }
    if not a.skip_cpu:
        log("cpu baseline ...")
        out["cpu_baseline"] = cpu_gemv_baseline(5120, 3072, 128)
        out["gpu_over_cpu"] = round(out["value"] / out["cpu_baseline"]["value"], 1)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Benchmark of the MI355X int4 LLM hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-e2e] [--skip-cpu] [--skip-gemm]
                    [--skip-attn] [--skip-native] [--sweep-gemv]
    python bench.py --plain-launches attn|gemv|w4a16|gemm [...]   (untimed, for rocprofv3 --pmc passes)

Headline (the JSON line's `value`): BASELINE config 2, the int4 decode GEMV y = W x at N=5120,
K=3072 (fused qkv), group 128, fp16 x / fp16 y, fp32 accumulation, in achieved HBM GB/s. A step is
one GEMV launch over one weight copy. Launches rotate over >= 64 weight copies (>= 520 MB, twice the
256 MB MALL), so every launch streams its weights from HBM. The timed region is exactly K launches
(--steps), replayed from a HIP graph so the host does not throttle them and bracketed by HIP events on
the launch stream after a device synchronisation; it is repeated --reps times (>= 5) and the line
reports the median (`value`, `ms_per_step`) and the minimum, as the reference's harness does
(gemm/harness/vk_gemm_bench.c:426-448). When K is smaller than the rotation, the rest of the rotation
runs untimed between repetitions, so no timed launch finds its copy in the MALL. Inputs are resident
in HBM before timing.

Other legs (extra JSON fields): the other config-2 GEMV shapes; measured streaming-read and
empty-kernel probes (the measured roofline and the launch floor); the config-3 fp16 GEMM shapes in
TFLOP/s against the 2.5 PFLOP/s fp16 dense peak; config-4 decode attention in GB/s; and config 5,
batch-1 generation of the Llama-3.2-3B-shaped int4 model (512-token prompt in chunks of 256, 256
greedy tokens, buckets 256..4096) in tokens/s with its HBM roofline fraction.

`cpu_baseline` times the reference-faithful CPU path of the headline workload (the oracle's
QLinear: F.linear over a per-call dequantized fp32 weight, llama_q4.py:72) on this host's cores.
Every other leg carries its own CPU figure on the same host: the GEMM leg the fp32 host matmul that
is also its parity reference (gemm/shapes.py:62), the attention leg the oracle's attention block
(llama_q4.py:224-232), and the 3B leg the oracle's whole step with per-call dequant over a stated
number of decode steps.
"""

import argparse
import hashlib
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

# Profiled constants. Counters cannot be read inside a timed run, so these figures are carried here
# with their source files; tests/test_host_checks_cpu.py fails when a constant and its file disagree.
# HBM bytes per 5120x3072 launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes (each calibrated
# with a plain streaming read / fill of known size).
GEMV_TRAFFIC_BYTES_5120x3072 = 8_234_776
GEMV_TRAFFIC_SOURCE = "profiles/q4_gemv_5120x3072_traffic_pmc.md"
# Average duration of the 5120x3072 kernel in the rocprofv3 kernel trace (every dispatch isolated by
# the profiler, so an upper bound on back-to-back launches).
GEMV_ROCPROF_AVG_US = 3.670
GEMV_ROCPROF_SOURCE = "profiles/q4_gemv_5120x3072_kernel_stats.md"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(N, K, group, x_bytes=2, y_bytes=2):
    """Algorithmic bytes of one GEMV: packed weights + fp16 scales + x + y."""
    return N * K // 2 + N * (K // group) * 2 + K * x_bytes + N * y_bytes


STREAM_TIMING_MAX_STEPS = 256


def timed_steps(fn_list, steps, warmup, reps=7, mode=None):
    """Time exactly `steps` launches, `reps` times; launch i is fn_list[i % n] (a rotation over n
    buffers). Returns the ms per launch of each repetition.

    Before every repetition one untimed pass over the rotation runs, so each buffer's previous use
    is n - 1 launches back (the MALL holds none of them). The timed region is bracketed by HIP events
    on the launch stream, and all repetitions are queued before the host waits:
      * steps <= STREAM_TIMING_MAX_STEPS: the region is `steps` plain stream launches, queued behind a
        device-side wait (q4_probe_wait) long enough for the host to queue the whole region first;
        after queueing, the start event must still be pending, which proves no launch of the region
        waited for the host (else the repetition is re-queued with a longer wait);
      * larger `steps`, and any run under rocprofv3: the region is one replay of a HIP graph of the `steps` launches (its ~10 us
        of graph-launch cost is then under 0.5% of the region).
    `mode` ("stream" or "graph") forces one of the two (a profiled run always replays graphs)."""
    import torch
    from q4llm._lib import LIB
    n = len(fn_list)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in fn_list:
            f()
    torch.cuda.synchronize()

    def capture(idx):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in idx:
                fn_list[i % n]()
        return g

    rot = capture(range(n))
    # under a profiler dispatches serialize and the region cannot be queued ahead: graph replays only
    stream_mode = (steps <= STREAM_TIMING_MAX_STEPS if mode is None else mode == "stream") and not under_profiler()
    ga = None if stream_mode else capture(range(steps))
    out = []
    with torch.cuda.stream(s):
        for _ in range(max(1, -(-warmup // n))):
            rot.replay()
        torch.cuda.synchronize()
        if stream_mode:
            # host cost of queueing one launch, measured with the device busy
            LIB.call("q4_probe_wait", 20000, s.cuda_stream)
            t0 = time.perf_counter()
            for i in range(min(steps, n)):
                fn_list[i]()
            host_us = (time.perf_counter() - t0) * 1e6 / min(steps, n)
            torch.cuda.synchronize()
            wait_us = int(2 * steps * host_us + 500)
            events = []
            while len(out) < reps:
                LIB.call("q4_probe_wait", min(wait_us, 1000000), s.cuda_stream)
                rot.replay()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(s)
                for i in range(steps):
                    fn_list[i % n]()
                e1.record(s)
                queued_in_time = not e0.query()
                e1.synchronize()
                if queued_in_time:
                    out.append(e0.elapsed_time(e1) / steps)
                elif wait_us >= 1000000:
                    raise RuntimeError("timed region could not be queued ahead of the device")
                else:
                    wait_us *= 2
        else:
            events = []
            for _ in range(reps):
                rot.replay()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(s)
                ga.replay()
                e1.record(s)
                events.append((e0, e1))
            events[-1][1].synchronize()
            out = [e0.elapsed_time(e1) / steps for e0, e1 in events]
    torch.cuda.synchronize()
    del rot, ga
    return out


def stats_us(ms_list):
    """median / min / max in microseconds of per-launch times given in ms."""
    import statistics
    us = [m * 1e3 for m in ms_list]
    return {"median": round(statistics.median(us), 3), "min": round(min(us), 3), "max": round(max(us), 3),
            "reps": len(us)}


def under_profiler():
    """True inside rocprofv3 (its tool library is preloaded into this process and every child)."""
    return "librocprofiler-sdk" in os.environ.get("LD_PRELOAD", "") or bool(os.environ.get("ROCP_TOOL_LIBRARIES"))


def cpu_threads():
    import torch
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return cores


def cpu_time_ms(fn, reps=3, budget_s=10.0):
    """Median wall time of fn() in ms on the host (one untimed call first; fewer reps past the budget)."""
    import statistics
    fn()
    ts, t_all = [], time.perf_counter()
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
        if time.perf_counter() - t_all > budget_s:
            break
    return statistics.median(ts), len(ts)


# ------------------------------------------------------------------------------------------------
# config 2: int4 decode GEMV
# ------------------------------------------------------------------------------------------------


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

    def launches(self, cfg=-1):
        from q4llm import ops
        return [lambda q=q, s=s: ops.q4_gemv_cfg(q, s, self.x, self.group, self.y, cfg=cfg)
                for q, s in zip(self.qws, self.scs)]

    def time(self, steps, warmup, cfg=-1, reps=7):
        return timed_steps(self.launches(cfg), steps, warmup, reps)

    def check(self):
        """max|y - y_ref| / rms(y_ref) against the fp64 CPU oracle (bar: 1e-2)."""
        from oracle import llama_q4_ref as R
        from q4llm import ops
        ops.q4_gemv(self.qw0, self.sc0, self.x, self.group, out=self.y)
        ref = R.dequantize_q4(self.qw0.cpu(), self.sc0.cpu(), self.group).double() @ self.x.cpu().double()
        return (self.y.cpu().double() - ref).abs().max().item() / ref.pow(2).mean().sqrt().item()


def probe_read(dev, nbytes, loads):
    """Measured streaming-read time of `nbytes` over rotating buffers (gemm/roofline.py:51-70)."""
    import torch
    from q4llm._lib import LIB
    copies = max(4, -(-2 * MALL_BYTES // nbytes))
    bufs = [torch.empty(nbytes // 4, dtype=torch.int32, device=dev).fill_(i) for i in range(copies)]
    sink = torch.empty(1, dtype=torch.float32, device=dev)
    fns = [lambda b=b: LIB.call("q4_probe_read", b.data_ptr(), nbytes, sink.data_ptr(), loads,
                                torch.cuda.current_stream().cuda_stream) for b in bufs]
    ms = stats_us(timed_steps(fns, 512, 64, 5))["median"] / 1e3
    return ms * 1e3, nbytes / ms / 1e6


def probe_empty(grid, block=256, steps=512, mode=None):
    import torch
    from q4llm._lib import LIB
    fns = [lambda: LIB.call("q4_probe_empty", grid, block, torch.cuda.current_stream().cuda_stream)] * 64
    return stats_us(timed_steps(fns, steps, 64, 5, mode))["median"]


def cpu_gemv_baseline(N, K, group, seconds=10.0):
    """Reference-faithful eager QLinear on the host: F.linear(x.float(), dequantize_q4(W)) per call."""
    import numpy as np
    import torch
    from oracle import llama_q4_ref as R
    from q4llm import synth
    cores = cpu_threads()
    qw, sc, x = synth.gemv_problem(N, K, group)
    ql = R.QLinearRef(group=group, qweight=torch.from_numpy(qw), scales=torch.from_numpy(sc), cache=False)
    xf = torch.from_numpy(x.astype(np.float32)).reshape(1, K)
    ql(xf)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        ql(xf)
        n += 1
    dt = (time.perf_counter() - t0) / n
    w = ql.weight()
    m, t1 = 0, time.perf_counter()
    while time.perf_counter() - t1 < min(3.0, seconds):
        torch.nn.functional.linear(xf, w)
        m += 1
    dt_best = (time.perf_counter() - t1) / m
    b = gemv_bytes(N, K, group)
    return dict(value=round(b / dt / 1e9, 3), unit="GB/s", cores=cores, kind="port",
                sample=f"{n} eager QLinear calls (per-call dequant + fp32 F.linear) at N={N}, K={K}, "
                       f"group {group}: {n * dt:.1f} s; pre-dequantized F.linear best case "
                       f"{b / dt_best / 1e9:.2f} GB/s",
                ms_per_call=round(dt * 1e3, 3), best_case_gbs=round(b / dt_best / 1e9, 3))


# ------------------------------------------------------------------------------------------------
# config 3: fp16 GEMM; config 4: decode attention
# ------------------------------------------------------------------------------------------------

GEMM_SHAPES = [(256, 5120, 3072), (256, 16384, 3072), (256, 3072, 8192), (1024, 5120, 3072), (2048, 3072, 8192),
               (4096, 4096, 4096), (1, 3072, 3072)]


def vendor_gemm_us(A, B, Bs, reps=5):
    """Median / min us per launch of torch.matmul(A, B^T) (hipBLASLt on this image) over the same rotated
    B copies: plain stream launches bracketed by HIP events (no graph capture: library calls stay out
    of graphs here), the rotation run once untimed first."""
    import statistics
    import torch
    n = max(16, 2 * len(Bs))
    for b in Bs:
        torch.matmul(A, b.t())
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(n):
            torch.matmul(A, Bs[i % len(Bs)].t())
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3 / n)
    return round(statistics.median(ts), 3), round(min(ts), 3)


def bench_gemm(dev, shapes=GEMM_SHAPES, reps=5, vendor=False):
    """Config 3 through gemm_f16_nt_ws (the 256-row shapes split K over a workspace allocated once per
    shape, outside the timed region). Parity against the host fp32 matmul of the same fp16 inputs
    (gemm/shapes.py:62), whose wall time on this host's cores is the leg's CPU figure; error is
    max|C - ref| / rms(ref)."""
    import torch
    from q4llm import ops, synth
    cores = cpu_threads()
    out = {}
    for (M, N, K) in shapes:
        a, b = synth.gemm_problem(M, N, K, seed=0)
        A = torch.from_numpy(a).to(dev)
        B0 = torch.from_numpy(b).to(dev)
        nb = max(4, -(-2 * MALL_BYTES // (2 * N * K))) if M <= 256 else 2
        Bs = [B0.clone() for _ in range(nb)]
        C = torch.empty(M, N, dtype=torch.float16, device=dev)
        C.fill_(float("nan"))
        ws = torch.empty(max(ops.gemm_f16_nt_ws_bytes(M, N, K), 16), dtype=torch.uint8, device=dev)
        ops.gemm_f16_nt_ws(A, B0, out=C, workspace=ws)
        got = C.cpu().float()
        a32, b32 = torch.from_numpy(a).float(), torch.from_numpy(b).float()
        ref_box = {}

        def host_ref():
            ref_box["r"] = a32 @ b32.T

        cpu_ms, cpu_n = cpu_time_ms(host_ref, reps=3, budget_s=8.0)
        ref = ref_box["r"]
        err = (got - ref).abs().max().item() / ref.pow(2).mean().sqrt().item()
        del ref, ref_box, got
        fns = [lambda B=B: ops.gemm_f16_nt_ws(A, B, out=C, workspace=ws) for B in Bs]
        st = stats_us(timed_steps(fns, max(16, len(fns) * 2), len(fns), reps))
        ms = st["median"] / 1e3
        flops = 2.0 * M * N * K
        byts = 2.0 * (M * K + N * K + M * N)
        tf = flops / ms / 1e9
        attain = min(MFMA_F16_PEAK_TFLOPS, flops / byts * HBM_PEAK_GBS / 1e3)
        out[f"{M}x{N}x{K}"] = {"us": st["median"], "us_min": st["min"], "reps": st["reps"], "TFLOP/s": round(tf, 1),
                               "frac_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                               "attainable_TFLOP/s": round(attain, 1), "frac_attainable": round(tf / attain, 4),
                               "GB/s": round(byts / ms / 1e6, 1), "err_over_rms": float(f"{err:.3e}"),
                               "cpu_ms": round(cpu_ms, 3), "cpu_TFLOP/s": round(flops / cpu_ms / 1e9, 3),
                               "cpu_cores": cores, "cpu_reps": cpu_n}
        log(f"gemm {M}x{N}x{K}: {st['median']:.2f} us (min {st['min']:.2f}) {tf:.1f} TFLOP/s "
            f"({tf / attain:.1%} of attainable {attain:.0f}); host fp32 {cpu_ms:.2f} ms; err/rms {err:.2e}")
        if vendor and M > 1:
            v_med, v_min = vendor_gemm_us(A, B0, Bs)
            out[f"{M}x{N}x{K}"].update({"hipblaslt_us": v_med, "hipblaslt_us_min": v_min,
                                        "hipblaslt_TFLOP/s": round(flops / v_med / 1e6, 1)})
            log(f"  torch.matmul (hipBLASLt) {v_med:.2f} us (min {v_min:.2f}) {flops / v_med / 1e6:.1f} TFLOP/s")
        del A, B0, Bs, C, ws
        torch.cuda.empty_cache()
    return out


# The reference's tuned results on its Adreno target (gemm/runs/run2/final_table.json:2-97): GFLOP/s of
# the best schedule found ("tuned") and that device's attainable GFLOP/s ("roof") per problem, carried
# here (the reference tree is not present where the bench runs) so each row prints beside them.
REF_ADRENO_TUNED = {"S1": (173.1, 920.8), "S2": (107.2, 920.8), "S3": (127.4, 920.8), "S4": (69.5, 250.8),
                    "S5": (93.5, 920.8), "S6": (98.6, 490.3), "S7": (15.4, 15.8), "S8": (161.2, 920.8)}


def bench_ref_shapes(dev, reps=5):
    """The reference's eight GEMM problems S1-S8 (gemm/shapes.py:41-66) with its own data recipe and
    check (TOL 5e-3 of max|Cref| against the fp32 product of the fp16 inputs), timed on gemm_f16_nt_ws.
    The kernel is NT: problems stored in another layout (NN, TN, TT) run on their logical A [M, K] and
    B^T [N, K]; the one-time transposes that a caller holding such data would do are timed separately
    (`layout_prep_us`, torch transpose copies). Operands stay resident (B rotated over up to 64 copies),
    attainable = min(2.5 PFLOP/s, flops / compulsory bytes x 8 TB/s) as gemm/analyze.py:32-36."""
    import numpy as np
    import torch
    from q4llm import ops, synth
    out = {}
    for sid, name, M, N, K, lay in synth.REF_GEMM_SHAPES:
        a, b = synth.ref_gemm_problem(sid)
        cref = a.astype(np.float32) @ b.astype(np.float32)
        A = torch.from_numpy(a).to(dev)
        Bt0 = torch.from_numpy(np.ascontiguousarray(b.T)).to(dev)
        nb = min(64, max(2, -(-2 * MALL_BYTES // (2 * N * K))))
        Bts = [Bt0.clone() for _ in range(nb)]
        C = torch.empty(M, N, dtype=torch.float16, device=dev)
        ws = torch.empty(max(ops.gemm_f16_nt_ws_bytes(M, N, K), 16), dtype=torch.uint8, device=dev)
        ops.gemm_f16_nt_ws(A, Bt0, out=C, workspace=ws)
        err = float(np.abs(C.cpu().float().numpy() - cref).max() / np.abs(cref).max())
        fns = [lambda B=B: ops.gemm_f16_nt_ws(A, B, out=C, workspace=ws) for B in Bts]
        st = stats_us(timed_steps(fns, max(64, 2 * len(fns)), len(fns), reps))
        prep = None
        if lay != "NT":
            # the stored operands a caller would hold: A^T [K, M] for 'T' A, B [K, N] for 'N' B
            As = torch.from_numpy(np.ascontiguousarray(a.T) if lay[0] == "T" else a).to(dev)
            Bs = torch.from_numpy(b if lay[1] == "N" else np.ascontiguousarray(b.T)).to(dev)

            def prep_fn():
                if lay[0] == "T":
                    As.t().contiguous()
                if lay[1] == "N":
                    Bs.t().contiguous()
            prep = stats_us(timed_steps([prep_fn], 64, 8, reps))["median"]
        flops = 2.0 * M * N * K
        byts = 2.0 * (M * K + K * N + M * N)
        gf = flops / st["median"] / 1e3
        attain = min(MFMA_F16_PEAK_TFLOPS * 1e3, flops / byts * HBM_PEAK_GBS)
        ref_tuned, ref_roof = REF_ADRENO_TUNED[sid]
        out[sid] = {"name": name, "M": M, "N": N, "K": K, "layout": lay, "us": st["median"], "us_min": st["min"],
                    "GFLOP/s": round(gf, 1), "attainable_GFLOP/s": round(attain, 1),
                    "frac_attainable": round(gf / attain, 4), "err_over_max_ref": float(f"{err:.3e}"),
                    "within_ref_tol": err <= synth.REF_GEMM_TOL, "layout_prep_us": prep,
                    "ref_adreno_tuned_GFLOP/s": ref_tuned, "ref_adreno_frac_attainable": round(ref_tuned / ref_roof, 4)}
        log(f"ref {sid} {name} {M}x{N}x{K} {lay}: {st['median']:.2f} us {gf:.0f} GFLOP/s "
            f"({gf / attain:.1%} of attainable; Adreno tuned {ref_tuned} = {ref_tuned / ref_roof:.1%}); err {err:.1e}"
            + (f"; layout prep {prep:.2f} us" if prep is not None else ""))
        del A, Bt0, Bts, C, ws
        torch.cuda.empty_cache()
    return out


W4A16_SHAPES = [(256, 5120, 3072), (256, 3072, 3072), (256, 16384, 3072), (256, 3072, 8192)]


def bench_w4a16(dev, reps=5):
    """The 3B prefill projections of a 256-row chunk (qkv, o, gate/up, down; group 128) through the C-ABI
    q4_linear_ws on the reference weight layout: x split into fp16 planes, the GEMM (K split over the
    workspace where the rule takes one) and the partial reduce, all in the timed launch sequence, over
    rotated weight copies. Parity and the CPU figure: the reference QLinear on the host (per-call
    dequant + fp32 F.linear, llama_q4.py:72) over the same x and weights; error is max|y - ref| /
    rms(ref). The model's own step runs the same GEMM on the T16 copies with the partials added by the
    next kernel (profiles/decode_3b_step_kernel_stats.md)."""
    import torch
    from oracle import llama_q4_ref as R
    from q4llm import ops
    cores = cpu_threads()
    out = {}
    g = torch.Generator().manual_seed(0)
    for (M, N, K) in W4A16_SHAPES:
        w = torch.randn(N, K, generator=g) * 0.02
        qd, sd = ops.quantize_q4(w.to(dev), 128)
        qw, sc = R.quantize_q4(w, 128)  # the checker's copy: bit-identical to the GPU quantizer's
        assert torch.equal(qd.cpu(), qw) and torch.equal(sd.cpu().view(torch.int16), sc.view(torch.int16))
        x = torch.randn(M, K, generator=g)
        wbytes = N * K // 2 + N * (K // 128) * 2
        nb = max(4, -(-2 * MALL_BYTES // wbytes))
        copies = [(qd.clone(), sd.clone()) for _ in range(nb)]
        xd = x.to(dev)
        y = torch.empty(M, N, device=dev)
        ws = torch.empty(ops.q4_linear_ws_split_bytes(M, N, K, 128), dtype=torch.uint8, device=dev)
        ops.q4_linear_ws(xd, copies[0][0], copies[0][1], 128, out=y, workspace=ws)
        got = y.cpu()
        box = {}

        def host_ref():
            box["r"] = torch.nn.functional.linear(x, R.dequantize_q4(qw, sc, 128))

        cpu_ms, cpu_n = cpu_time_ms(host_ref, reps=3, budget_s=6.0)
        ref = box["r"]
        err = (got - ref).abs().max().item() / ref.pow(2).mean().sqrt().item()
        fns = [lambda q=q, s_=s_: ops.q4_linear_ws(xd, q, s_, 128, out=y, workspace=ws) for q, s_ in copies]
        st = stats_us(timed_steps(fns, max(16, 2 * len(fns)), len(fns), reps))
        flops = 2.0 * M * N * K
        tf = flops / st["median"] / 1e6
        byts = M * K * 4 + wbytes + M * N * 4
        attain = min(MFMA_F16_PEAK_TFLOPS, flops / byts * HBM_PEAK_GBS / 1e3)
        # issued: every k step runs two fp16 MFMAs (x split into hi + lo) for exact fp32 activations
        out[f"{M}x{N}x{K}"] = {"us": st["median"], "us_min": st["min"], "reps": st["reps"],
                               "TFLOP/s": round(tf, 1), "frac_mfma_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                               "issued_mfma_TFLOP/s": round(2 * tf, 1),
                               "frac_mfma_peak_issued": round(2 * tf / MFMA_F16_PEAK_TFLOPS, 4),
                               "attainable_TFLOP/s": round(attain, 1), "frac_attainable": round(tf / attain, 4),
                               "err_over_rms": float(f"{err:.3e}"),
                               "cpu_ms": round(cpu_ms, 3), "cpu_cores": cores, "cpu_reps": cpu_n}
        log(f"w4a16 {M}x{N}x{K}: {st['median']:.2f} us (min {st['min']:.2f}) {tf:.0f} TFLOP/s useful "
            f"({tf / MFMA_F16_PEAK_TFLOPS:.1%} of the fp16 peak, {2 * tf / MFMA_F16_PEAK_TFLOPS:.1%} issued); "
            f"host QLinear {cpu_ms:.1f} ms; err/rms {err:.2e}")
        del copies, xd, y, ws
        torch.cuda.empty_cache()
    return out


def bench_attn(dev, reps=5):
    """Config 4 (24/8 heads, hd 128, one query row at position valid - 1). CPU figure: the oracle's
    attention block (llama_q4.py:224-232) over the same caches on this host's cores."""
    import math
    import torch
    from oracle import llama_q4_ref as R
    from q4llm import ops, synth
    cores = cpu_threads()
    out = {}
    for L in (256, 512, 1024, 2048, 4096):
        q, k, v, valid = synth.attn_problem(L, seed=0)
        qd = torch.from_numpy(q).to(dev)
        kv_bytes = 2 * L * 8 * 128 * 2
        copies = max(8, -(-2 * MALL_BYTES // kv_bytes))
        ks = [torch.from_numpy(k).to(dev) for _ in range(copies)]
        vs = [torch.from_numpy(v).to(dev) for _ in range(copies)]
        start = torch.tensor([valid - 1], dtype=torch.int32, device=dev)
        ws = torch.empty(ops.attn_workspace_bytes(1, 24, 8, 128, L), dtype=torch.uint8, device=dev)
        o = torch.empty(1, 24 * 128, dtype=torch.float32, device=dev)
        fns = [lambda kk=kk, vv=vv: ops.attn_bucket(qd, kk, vv, L, start, 1 / math.sqrt(128), ws, o)
               for kk, vv in zip(ks, vs)]
        st = stats_us(timed_steps(fns, max(64, len(fns)), len(fns), reps))
        ms = st["median"] / 1e3
        qc, kc, vc = torch.from_numpy(q).reshape(1, 24, 128), torch.from_numpy(k), torch.from_numpy(v)
        allowed = torch.arange(L)[None, :] <= valid - 1
        cpu_ms, _ = cpu_time_ms(lambda: R.attention(qc, kc, vc, allowed, L, 1 / math.sqrt(128)), reps=5, budget_s=3.0)
        byts = 2 * valid * 8 * 128 * 2 + 24 * 128 * 4 * 2
        gbs = byts / ms / 1e6
        out[f"L{L}"] = {"valid": valid, "us": st["median"], "us_min": st["min"], "reps": st["reps"],
                        "GB/s_valid_rows": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                        "GB/s_bucket": round((2 * L * 8 * 128 * 2) / ms / 1e6, 1),
                        "cpu_us": round(cpu_ms * 1e3, 1), "cpu_cores": cores}
        log(f"attn L={L} valid={valid}: {st['median']:.2f} us (min {st['min']:.2f}), {gbs:.0f} GB/s over valid rows; "
            f"CPU oracle {cpu_ms * 1e3:.0f} us")
        del ks, vs
        torch.cuda.empty_cache()
    return out


# ------------------------------------------------------------------------------------------------
# config 5: Llama-3.2-3B-shaped batch-1 generation
# ------------------------------------------------------------------------------------------------

LAYER_BYTES_3B = 51_904_512     # wqkv + wo + wgu + wdown packed weights + fp16 scales, one layer
LM_HEAD_BYTES_3B = 203_157_504  # tied int4 embedding as the LM head
LAYER_PARAMS_3B = (5120 + 3072) * 3072 + 16384 * 3072 + 3072 * 8192  # weights per layer (qkv, o, gate/up, down)


def prefill_roofline_3b(n_prompt, chunk, n_layers=28, n_q=24, hd=128):
    """Useful flops per prompt token of the 3B prefill: 2 x the layer weights (the LM head runs on one row
    per chunk) plus the attention's QK^T and PV over each row's valid keys (4 n_q hd per key and layer),
    averaged over the prompt's causal rows; and the roofline rate min(fp16 MFMA peak / flops, HBM / bytes),
    bytes = one read of every layer weight per chunk spread over its rows."""
    avg_valid = (n_prompt + 1) / 2
    flops = 2.0 * n_layers * LAYER_PARAMS_3B + 4.0 * n_layers * n_q * hd * avg_valid
    bytes_per_tok = n_layers * LAYER_BYTES_3B / chunk
    rate = min(MFMA_F16_PEAK_TFLOPS * 1e12 / flops, HBM_PEAK_GBS * 1e9 / bytes_per_tok)
    return flops, rate


def cpu_decode_baseline(pc, host_tensors, token, pos=700, L=1024, max_steps=3, budget_s=20.0):
    """The reference's eager decode step on this host's cores: the oracle's LlamaQ4.step with every
    QLinear re-dequantizing its weight per call (llama_q4.py:72,199-239), over the same quantized
    weights as the GPU run, at the bucket and position the GPU decode uses. One step takes tens of
    seconds (each step dequantizes 1.66 GB of int4 weights), so at least one and at most `max_steps`
    steps are timed, stopping once `budget_s` has passed."""
    import torch
    from oracle import llama_q4_ref as R
    cores = cpu_threads()
    ref = R.LlamaQ4Ref.from_quantized(pc, host_tensors, cache=False)
    caches = ref.new_caches()
    tok = torch.tensor([[token]], dtype=torch.int32)
    ts = []
    for i in range(max_steps):
        if sum(ts) > budget_s:
            break
        t0 = time.perf_counter()
        nxt, _ = ref.step(tok, torch.tensor([pos + i], dtype=torch.int32), torch.tensor([0], dtype=torch.int32),
                          caches, L)
        ts.append(time.perf_counter() - t0)
        tok = nxt.reshape(1, 1)
    steps = len(ts)
    return {"decode_tok_s": round(steps / sum(ts), 4), "s_per_step": round(sum(ts) / steps, 3), "steps_timed": steps,
            "cores": cores, "kind": "port", "L": L,
            "sample": f"{steps} decode steps of the oracle LlamaQ4.step at L={L} from position {pos}, per-call "
                      "dequant of every int4 weight (eager QLinear.forward), same quantized weights"}


def bench_e2e(dev, n_new=256, native=True, cpu=True, reps=5, runs=5, native_runs=3):
    import statistics
    import torch
    from q4llm import llm_runner, synth
    from q4llm.llama_q4 import LlamaQ4
    t0 = time.time()
    sd = synth.PrefetchingWeights(synth.LLAMA32_3B, seed=0)
    model = LlamaQ4(None, group=synth.LLAMA32_3B_GROUP, max_ctx=4096, sd=sd, cfg=synth.LLAMA32_3B)
    sd.close()
    torch.cuda.synchronize()
    build_s = time.time() - t0
    log(f"e2e: 3B-shaped model built (synthetic weights, GPU quantization) in {build_s:.1f} s")
    prompt = synth.prompt_ids(512, synth.LLAMA32_3B["vocab_size"], seed=0)
    buckets = [256, 512, 1024, 2048, 4096]
    caches = model.new_caches()
    # `runs` whole generations (prefill + decode, each after the runner's own warm-up); the tok/s
    # figures are their medians, and every run must produce the same tokens
    results = [llm_runner.run(model, prompt, n_new, 256, buckets, caches=caches) for _ in range(runs)]
    res = results[-1]
    if any(r["tokens"] != res["tokens"] for r in results):
        raise RuntimeError("e2e: repeated generations produced different tokens")
    pf_runs = sorted(r["prefill_tok_s"] for r in results)
    dc_runs = sorted(r["decode_tok_s"] for r in results)
    # GPU-only time of one decode step at the bucket the run used: graph replays back to back, the
    # median and minimum over `reps` repetitions of 50 replays
    g = model.entry_point(1, 1024, caches)
    s = torch.cuda.current_stream()
    per = []
    for _ in range(reps):
        g.start.fill_(700)
        g.tokens.fill_(res["tokens"][-1])
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(50):
            g.replay()
        e1.record(s)
        e1.synchronize()
        per.append(e0.elapsed_time(e1) / 50)
    gpu_ms = statistics.median(per)
    n_layers = synth.LLAMA32_3B["num_hidden_layers"]
    w_bytes = n_layers * LAYER_BYTES_3B + LM_HEAD_BYTES_3B
    avg_valid = 512 + (n_new - 1) / 2 + 1
    kv_valid = n_layers * 2 * avg_valid * 8 * 128 * 2
    kv_bucket = n_layers * 2 * 1024 * 8 * 128 * 2
    tok_s = statistics.median(dc_runs)
    pf_tok_s = statistics.median(pf_runs)
    pf_flops, pf_roof = prefill_roofline_3b(len(prompt), 256)
    out = {
        "runs": runs, "decode_tok_s": round(tok_s, 2), "decode_tok_s_min_max": [dc_runs[0], dc_runs[-1]],
        "prefill_tok_s": round(pf_tok_s, 1), "prefill_tok_s_min_max": [pf_runs[0], pf_runs[-1]],
        "ttft_ms": statistics.median(r["ttft_ms"] for r in results),
        "decode_steps": res["decode_steps"], "gpu_ms_per_decode_step": round(gpu_ms, 4),
        "gpu_ms_per_decode_step_min": round(min(per), 4), "gpu_only_tok_s": round(1e3 / gpu_ms, 1),
        "bytes_per_step_valid_kv": int(w_bytes + kv_valid), "bytes_per_step_bucket_L1024": int(w_bytes + kv_bucket),
        "hbm_roofline_tok_s_L1024": round(HBM_PEAK_GBS * 1e9 / (w_bytes + kv_bucket), 1),
        "frac_hbm_roofline": round(tok_s * (w_bytes + kv_valid) / (HBM_PEAK_GBS * 1e9), 4),
        "frac_hbm_roofline_gpu_only": round((w_bytes + kv_valid) / (gpu_ms * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
        "prefill_flops_per_token": round(pf_flops), "prefill_roofline_tok_s": round(pf_roof, 1),
        "frac_prefill_roofline": round(pf_tok_s / pf_roof, 4),
        "tokens_sha1": hashlib.sha1(json.dumps(res["tokens"]).encode()).hexdigest(),
        "first_tokens": res["tokens"][:16], "model_build_s": round(build_s, 1),
        "buckets_used": sorted({L for L, _ in res["steps"]}),
    }
    log(f"e2e decode {tok_s:.1f} tok/s (GPU-only {1e3 / gpu_ms:.1f}), prefill {pf_tok_s:.0f} tok/s "
        f"(medians of {runs} runs)")
    host = None
    if cpu:
        host = {k: v.cpu() for k, v in model.packed_tensors().items()}
        pc = model.packed_config()
    if native and under_profiler():
        # the runner's HIP runtime crashes in the profiler's preloaded tool (observed under rocprofv3)
        log("e2e native runner: skipped under rocprofv3")
        out["native_runner"] = "skipped under a profiler"
        native = False
    if native:
        # the same generation through the native runner (lib/llm-runner) from the packed weights
        import tempfile
        from q4llm import sweep
        with tempfile.TemporaryDirectory() as td:
            wpath = pathlib.Path(td) / "llama32_3b_shape.q4w"
            model.save_packed(wpath)
            del model, caches, g
            torch.cuda.empty_cache()
            nats = [sweep.run_runner(wpath, prompt, n_new, 256, ",".join(map(str, buckets)), "bucketed")
                    for _ in range(native_runs)]
        match = all(n["tokens"] == res["tokens"] for n in nats)
        nat_dc = statistics.median(n["decode_tok_s"] for n in nats)
        nat_pf = statistics.median(n["prefill_tok_s"] for n in nats)
        out.update(native_runner_runs=native_runs, native_runner_decode_tok_s=nat_dc,
                   native_runner_prefill_tok_s=nat_pf,
                   native_runner_ttft_ms=statistics.median(n["ttft_ms"] for n in nats),
                   native_runner_tokens_match=match)
        log(f"e2e native runner: decode {nat_dc:.1f} tok/s, prefill {nat_pf:.0f} tok/s (medians of {native_runs} "
            f"runs), tokens match: {match}")
    else:
        del model, caches, g
        torch.cuda.empty_cache()
    if host is not None:
        log("e2e CPU baseline (oracle step, per-call dequant) ...")
        cb = cpu_decode_baseline(pc, host, res["tokens"][-1])
        del host
        cb["gpu_over_cpu"] = round(tok_s / cb["decode_tok_s"], 1)
        out["cpu_baseline"] = cb
        log(f"e2e CPU baseline: {cb['decode_tok_s']} tok/s on {cb['cores']} cores ({cb['s_per_step']} s per step)")
    return out, res["tokens"]


# ------------------------------------------------------------------------------------------------
# plain launches for hardware-counter passes
# ------------------------------------------------------------------------------------------------


def plain_launches(dev, what, Ls, shapes, iters, probe_bytes, vendor):
    """Plain stream launches of one leg's calls, a device synchronisation after each, then a streaming-
    read probe of a known byte count whose counter reading calibrates the pass. rocprofv3's counter
    mode (--pmc) samples every dispatch; this gives it a short, graph-free sequence of the launches the
    timed legs replay from graphs, each reading its operands from memory (rotating copies). One line
    per leg names the algorithmic bytes (or flops) per launch that the counters are compared with."""
    import math
    import torch
    from q4llm import ops, synth
    from q4llm._lib import LIB
    sync = torch.cuda.synchronize
    if what == "attn":
        for L in Ls:
            q, k, v, valid = synth.attn_problem(L, seed=0)
            qd = torch.from_numpy(q).to(dev)
            ks = [torch.from_numpy(k).to(dev) for _ in range(8)]
            vs = [torch.from_numpy(v).to(dev) for _ in range(8)]
            start = torch.tensor([valid - 1], dtype=torch.int32, device=dev)
            ws = torch.empty(ops.attn_workspace_bytes(1, 24, 8, 128, L), dtype=torch.uint8, device=dev)
            o = torch.empty(1, 24 * 128, dtype=torch.float32, device=dev)
            for i in range(iters):
                ops.attn_bucket(qd, ks[i % 8], vs[i % 8], L, start, 1 / math.sqrt(128), ws, o)
                sync()
            print(f"attn L={L} valid={valid} launches={iters}: K/V bytes of the valid rows {2 * valid * 8 * 128 * 2}, "
                  f"q + out {24 * 128 * 4 * 2}", flush=True)
            del ks, vs
    elif what == "gemv":
        N, K, group = 5120, 3072, 128
        qw, sc, x = synth.gemv_problem(N, K, group)
        qws = [torch.from_numpy(qw).to(dev) for _ in range(8)]
        scs = [torch.from_numpy(sc).to(dev) for _ in range(8)]
        xd = torch.from_numpy(x).to(dev)
        y = torch.empty(N, dtype=torch.float16, device=dev)
        for i in range(iters):
            ops.q4_gemv(qws[i % 8], scs[i % 8], xd, group, out=y)
            sync()
        print(f"gemv {N}x{K} launches={iters}: algorithmic bytes {gemv_bytes(N, K, group)}", flush=True)
    elif what == "w4a16":
        g = torch.Generator().manual_seed(0)
        for (M, N, K) in shapes or W4A16_SHAPES:
            qw, sc = ops.quantize_q4((torch.randn(N, K, generator=g) * 0.02).to(dev), 128)
            copies = [(qw.clone(), sc.clone()) for _ in range(8)]
            xd = torch.randn(M, K, generator=g).to(dev)
            y = torch.empty(M, N, device=dev)
            ws = torch.empty(ops.q4_linear_ws_split_bytes(M, N, K, 128), dtype=torch.uint8, device=dev)
            for i in range(iters):
                ops.q4_linear_ws(xd, copies[i % 8][0], copies[i % 8][1], 128, out=y, workspace=ws)
                sync()
            print(f"w4a16 {M}x{N}x{K} launches={iters}: useful flops {2 * M * N * K}", flush=True)
            del copies
    elif what == "gemm":
        for (M, N, K) in shapes or [(4096, 4096, 4096)]:
            a, b = synth.gemm_problem(M, N, K, seed=0)
            A = torch.from_numpy(a).to(dev)
            Bs = [torch.from_numpy(b).to(dev) for _ in range(2)]
            C = torch.empty(M, N, dtype=torch.float16, device=dev)
            ws = torch.empty(max(ops.gemm_f16_nt_ws_bytes(M, N, K), 16), dtype=torch.uint8, device=dev)
            for i in range(iters):
                ops.gemm_f16_nt_ws(A, Bs[i % 2], out=C, workspace=ws)
                sync()
            if vendor:
                for i in range(iters):
                    torch.matmul(A, Bs[i % 2].t())
                    sync()
            print(f"gemm {M}x{N}x{K} launches={iters}{' (+ torch.matmul)' if vendor else ''}: flops {2 * M * N * K}",
                  flush=True)
            del A, Bs, C, ws
    if probe_bytes:
        buf = torch.ones(probe_bytes // 4, dtype=torch.int32, device=dev)
        sink = torch.empty(1, dtype=torch.float32, device=dev)
        for _ in range(iters):
            LIB.call("q4_probe_read", buf.data_ptr(), probe_bytes, sink.data_ptr(), 1,
                     torch.cuda.current_stream().cuda_stream)
            sync()
        print(f"probe read_kernel<1> launches={iters}: bytes read {probe_bytes}", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048, help="timed launches per repetition of the headline GEMV")
    ap.add_argument("--warmup", type=int, default=256, help="untimed launches before timing")
    ap.add_argument("--reps", type=int, default=7, help="timed repetitions (median and min are reported; >= 5)")
    ap.add_argument("--skip-e2e", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true", help="leave out every CPU-baseline figure")
    ap.add_argument("--skip-gemm", action="store_true")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="also time torch.matmul (hipBLASLt) on the GEMM shapes, for comparison")
    ap.add_argument("--skip-attn", action="store_true")
    ap.add_argument("--skip-w4a16", action="store_true", help="leave out the prefill W4A16 GEMM leg")
    ap.add_argument("--skip-gemv", action="store_true",
                    help="leave out the GEMV and probe legs (profiling the other legs; the line then has no value)")
    ap.add_argument("--skip-native", action="store_true",
                    help="skip the native-runner e2e leg (also skipped by itself under rocprofv3)")
    ap.add_argument("--sweep-gemv", action="store_true", help="time every GEMV tile config (tuning)")
    ap.add_argument("--gemm-shapes", nargs="*", default=None, metavar="MxNxK",
                    help="run the GEMM leg on these shapes only (default: every config-3 shape)")
    ap.add_argument("--tokens-out", default=None, help="write the e2e generated token ids here")
    ap.add_argument("--plain-launches", choices=["attn", "gemv", "w4a16", "gemm"], default=None,
                    help="no timing: plain launches of one leg, a sync after each, for rocprofv3 --pmc passes")
    ap.add_argument("--plain-L", type=int, nargs="*", default=[1024, 4096], help="--plain-launches attn buckets")
    ap.add_argument("--plain-shapes", nargs="*", default=None, metavar="MxNxK",
                    help="--plain-launches w4a16 / gemm shapes (default: the W4A16 leg's shapes / 4096^3)")
    ap.add_argument("--plain-iters", type=int, default=40)
    ap.add_argument("--plain-vendor", action="store_true", help="--plain-launches gemm: also torch.matmul")
    ap.add_argument("--plain-probe", type=int, default=8126464,
                    help="bytes of the calibration read probe after the plain launches (0: none)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported: this build runs on a single "
              "MI355X and multi-GPU sharding is design-only", file=sys.stderr)
        return 2
    if a.steps < 1 or a.reps < 5:
        print("--steps must be >= 1 and --reps >= 5", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("no ROCm GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    from q4llm._lib import LIB
    LIB.load()
    if a.plain_launches:
        plain_launches(dev, a.plain_launches, a.plain_L,
                       None if a.plain_shapes is None else [tuple(int(v) for v in t.split("x")) for t in a.plain_shapes],
                       a.plain_iters, a.plain_probe, a.plain_vendor)
        return 0

    shapes = [(5120, 3072), (16384, 3072), (3072, 8192)]
    results = {}
    if a.skip_gemv:
        out = {"metric": "int4 GEMV achieved HBM GB/s (% of peak) + batch-1 decode tokens/s, 3B-shape", "value": None,
               "unit": "GB/s", "note": "--skip-gemv: profiling run of the other legs"}
        if not a.skip_gemm:
            out["gemm_f16"] = bench_gemm(dev, GEMM_SHAPES if a.gemm_shapes is None else
                                         [tuple(int(v) for v in t.split("x")) for t in a.gemm_shapes],
                                         vendor=a.vendor_gemm)
            if a.gemm_shapes is None:
                out["gemm_ref_shapes"] = bench_ref_shapes(dev)
        if not a.skip_attn:
            out["attn_decode"] = bench_attn(dev)
        if not a.skip_w4a16:
            out["w4a16_prefill"] = bench_w4a16(dev)
        if not a.skip_e2e:
            out["e2e_3b"] = bench_e2e(dev, native=not a.skip_native, cpu=not a.skip_cpu)[0]
        print(json.dumps(out), flush=True)
        return 0
    for (N, K) in shapes:
        gb = GemvBench(dev, N, K)
        rel = gb.check()
        if a.sweep_gemv:
            for cfg in range(LIB.raw("q4_gemv_num_configs")()):
                ms = stats_us(gb.time(512, 64, cfg=cfg, reps=5))["median"] / 1e3
                log(f"sweep N={N} K={K} cfg={cfg}: {ms * 1e3:.2f} us {gb.bytes / ms / 1e6:.0f} GB/s")
        steps = a.steps if (N, K) == shapes[0] else max(256, a.steps // 4)
        st = stats_us(gb.time(steps, a.warmup, reps=a.reps))
        us = st["median"]
        results[(N, K)] = dict(us=us, us_min=st["min"], us_max=st["max"], reps=st["reps"], gbs=gb.bytes / us / 1e3,
                               bytes=gb.bytes, err=rel, steps=steps, copies=len(gb.qws))
        if (N, K) == shapes[0]:
            # both launch modes beside the value, over long regions: plain stream launches (the mode
            # --steps <= 256 selects; 256 launches, the most the region queues ahead) and graph replays
            # (the mode the model's step runs in; 2048 launches)
            results[(N, K)]["modes"] = {
                "stream_256": stats_us(timed_steps(gb.launches(), STREAM_TIMING_MAX_STEPS, a.warmup, 5, "stream"))["median"],
                "graph_2048": stats_us(timed_steps(gb.launches(), 2048, a.warmup, 5, "graph"))["median"]}
        log(f"gemv N={N} K={K}: {us:.3f} us/launch (min {st['min']:.3f}, max {st['max']:.3f} over {st['reps']} reps "
            f"of {steps}), {gb.bytes / us / 1e3:.1f} GB/s, err/rms {rel:.2e}")
        del gb
        torch.cuda.empty_cache()

    probes = {}
    for nbytes in (8126464, 12998656, 25991168, 1 << 30):
        us, gbs = min(probe_read(dev, nbytes, L) for L in (1, 4))
        probes[f"read_{nbytes}B"] = {"us": round(us, 3), "GB/s": round(gbs, 1)}
        log(f"probe read {nbytes} B: {us:.3f} us {gbs:.1f} GB/s")
    probes["empty_kernel_us"] = round(probe_empty(256), 3)
    probes["empty_kernel_stream_us"] = round(probe_empty(256, steps=256, mode="stream"), 3)
    log(f"probe empty kernel: {probes['empty_kernel_us']} us per launch in graph replays, "
        f"{probes['empty_kernel_stream_us']} us as plain stream launches")
    torch.cuda.empty_cache()

    head = results[shapes[0]]
    floor = probes["read_8126464B"]["us"]
    out = {
        "metric": "int4 GEMV achieved HBM GB/s (% of peak) + batch-1 decode tokens/s, 3B-shape",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(head["us"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights, fp16 x/y, fp32 accumulate",
        "data": "synthetic (seeded numpy: nibbles U[0,15], group-128 scales |N(0,0.01)| fp16, x N(0,1) fp16)",
        "config": {"workload": "int4 decode GEMV y=Wx, N=5120 (fused qkv), K=3072, group 128, batch 1",
                   "N": 5120, "K": 3072, "group": 128, "weight_copies_rotated": head["copies"]},
        "timing": {"statistic": "median over repetitions of the timed region (value, ms_per_step)",
                   "reps": head["reps"], "steps_per_rep": head["steps"],
                   "launch_mode": "stream" if head["steps"] <= STREAM_TIMING_MAX_STEPS else "graph",
                   "us_per_step_median": head["us"],
                   "us_per_step_min": head["us_min"], "us_per_step_max": head["us_max"],
                   "us_per_launch_by_mode": head["modes"],
                   "note": "value is the launch mode this command's --steps selects (plain stream launches up to "
                           f"{STREAM_TIMING_MAX_STEPS} steps, one graph replay above); both modes over long regions "
                           "are reported beside it"},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4),
                     "frac_at_min": round(head["bytes"] / head["us_min"] / 1e3 / HBM_PEAK_GBS, 4),
                     "traffic": GEMV_TRAFFIC_BYTES_5120x3072,
                     "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated)",
                     "traffic_source": f"profiled constant, {GEMV_TRAFFIC_SOURCE}",
                     "algorithmic_bytes_per_launch": head["bytes"], "avg_launch_us": round(head["us"], 4),
                     "rocprof_profile": {"avg_kernel_us": GEMV_ROCPROF_AVG_US, "source": GEMV_ROCPROF_SOURCE,
                                         "frac_at_avg": round(head["bytes"] / GEMV_ROCPROF_AVG_US / 1e3 /
                                                              HBM_PEAK_GBS, 4),
                                         "note": "profiled constant: rocprofv3 kernel-trace average of "
                                                 "isolated dispatches, not this run"},
                     "measured_read_floor_us_same_bytes": floor,
                     "frac_of_measured_read_floor": round(floor / head["us"], 4)},
        "gemv_shapes": {f"{N}x{K}": {"us": round(r["us"], 3), "us_min": round(r["us_min"], 3),
                                      "GB/s": round(r["gbs"], 1), "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4),
                                      "err_over_rms": float(f"{r['err']:.3e}")} for (N, K), r in results.items()},
        "measured_probes": probes,
    }
    if not a.skip_gemm:
        shapes = ([tuple(int(v) for v in t.split("x")) for t in a.gemm_shapes] if a.gemm_shapes is not None
                  else GEMM_SHAPES)
        out["gemm_f16"] = bench_gemm(dev, shapes, vendor=a.vendor_gemm)
        if a.gemm_shapes is None:
            out["gemm_ref_shapes"] = bench_ref_shapes(dev)
    if not a.skip_attn:
        out["attn_decode"] = bench_attn(dev)
    if not a.skip_w4a16:
        out["w4a16_prefill"] = bench_w4a16(dev)
    if not a.skip_e2e:
        e2e, tokens = bench_e2e(dev, native=not a.skip_native, cpu=not a.skip_cpu)
        out["e2e_3b"] = e2e
        if a.tokens_out:
            pathlib.Path(a.tokens_out).write_text(json.dumps(tokens))
    if not a.skip_cpu:
        log("cpu baseline ...")
        out["cpu_baseline"] = cpu_gemv_baseline(5120, 3072, 128)
        out["gpu_over_cpu"] = round(out["value"] / out["cpu_baseline"]["value"], 1)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

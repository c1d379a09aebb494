"""Plain stream launches of one hot-path kernel family, for hardware-counter passes.

    python -m q4llm.kernel_runs attn --L 1024 4096 --iters 40
    python -m q4llm.kernel_runs gemv --iters 200

Each run ends with a streaming-read probe of --probe bytes (default 8,126,464), whose counter
reading against its known size calibrates the pass.

rocprofv3's counter mode (``--pmc``) serialises and samples every dispatch; this driver gives it a
short, graph-free sequence of the same launches bench.py times (config-4 decode attention over
rotating KV caches, the config-2 5120x3072 GEMV over rotating weight copies), synchronising after
each launch so every dispatch reads its operands from memory. It prints one line per leg with the
algorithmic bytes per launch, the figure the counters are compared against.
"""

import argparse
import math
import sys


def _attn(dev, Ls, iters):
    import torch
    from . import ops, synth
    for L in Ls:
        q, k, v, valid = synth.attn_problem(L, seed=0)
        qd = torch.from_numpy(q).to(dev)
        copies = 8
        ks = [torch.from_numpy(k).to(dev) for _ in range(copies)]
        vs = [torch.from_numpy(v).to(dev) for _ in range(copies)]
        start = torch.tensor([valid - 1], dtype=torch.int32, device=dev)
        ws = torch.empty(ops.attn_workspace_bytes(1, 24, 8, 128, L), dtype=torch.uint8, device=dev)
        o = torch.empty(1, 24 * 128, dtype=torch.float32, device=dev)
        for i in range(iters):
            ops.attn_bucket(qd, ks[i % copies], vs[i % copies], L, start, 1 / math.sqrt(128), ws, o)
            torch.cuda.synchronize()
        kv = 2 * valid * 8 * 128 * 2
        print(f"attn L={L} valid={valid} launches={iters}: K/V bytes of the valid rows {kv}, "
              f"q + out {24 * 128 * 4 * 2}", flush=True)


def _probe(dev, nbytes, iters):
    """Streaming-read probe of a known byte count: calibrates a counter pass run beside the legs."""
    import torch
    from ._lib import LIB
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    sink = torch.empty(1, dtype=torch.float32, device=dev)
    for _ in range(iters):
        LIB.call("q4_probe_read", buf.data_ptr(), nbytes, sink.data_ptr(), 1, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
    print(f"probe read_kernel<1> launches={iters}: bytes read {nbytes}", flush=True)


def _gemv(dev, iters):
    import torch
    from . import ops, synth
    N, K, group = 5120, 3072, 128
    qw, sc, x = synth.gemv_problem(N, K, group)
    copies = 8
    qws = [torch.from_numpy(qw).to(dev) for _ in range(copies)]
    scs = [torch.from_numpy(sc).to(dev) for _ in range(copies)]
    xd = torch.from_numpy(x).to(dev)
    y = torch.empty(N, dtype=torch.float16, device=dev)
    for i in range(iters):
        ops.q4_gemv(qws[i % copies], scs[i % copies], xd, group, out=y)
        torch.cuda.synchronize()
    b = N * K // 2 + N * (K // group) * 2 + 2 * K + 2 * N
    print(f"gemv {N}x{K} launches={iters}: algorithmic bytes {b}", flush=True)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("what", choices=["attn", "gemv"])
    ap.add_argument("--L", type=int, nargs="*", default=[1024, 4096])
    ap.add_argument("--iters", type=int, default=40)
    ap.add_argument("--probe", type=int, default=8126464, help="bytes of the calibration read probe (0: none)")
    a = ap.parse_args(argv)
    import torch
    if not torch.cuda.is_available():
        print("no ROCm GPU visible", file=sys.stderr)
        return 1
    from ._lib import LIB
    LIB.load()
    dev = torch.device("cuda:0")
    if a.what == "attn":
        _attn(dev, a.L, a.iters)
    else:
        _gemv(dev, a.iters)
    if a.probe:
        _probe(dev, a.probe, a.iters)
    return 0


if __name__ == "__main__":
    sys.exit(main())

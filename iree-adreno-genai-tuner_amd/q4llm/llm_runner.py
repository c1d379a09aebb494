"""Generation runner with the reference runner's scheduling contract (runner/llm_runner.c).

  python -m q4llm.llm_runner --synthetic tiny|3b [--seed 0] --prompt ids.txt --max_new_tokens 32
        --chunk 16 --buckets 64,128 [--schedule bucketed|max] [--stop_ids ...] [--warmup 1]
  python -m q4llm.llm_runner --model-dir <hf snapshot> --group 128 ...

Contract kept from llm_runner.c:
  * prefill in chunks of `chunk` tokens, the last chunk zero-padded, last = n - 1 of the chunk
    (:210-222); bucket = smallest compiled bucket >= start + chunk (:143-149, :215);
  * the first generated token comes from prefill; decode steps at pos = n_prompt, ... with bucket
    >= pos + 1 until max_new_tokens exist or a stop id appears (:229-245);
  * KV caches are allocated once, zeroed, owned by the runner and written in place (:301-315);
  * warm-up runs every entry point the schedule will use before timing (:175-203);
  * errors: empty prompt, prompt + new > max_ctx, no bucket >= need (:168-173, :216);
  * one JSON object with the same keys (:249-262).
Each (phase, bucket) entry point is a HIP graph captured once and replayed (LlamaQ4.entry_point).
"""

import argparse
import json
import pathlib
import sys
import time

import torch


class RunnerError(ValueError):
    pass


def pick_bucket(buckets, needed, use_max=False):
    """Smallest bucket >= needed (or the largest under schedule 'max'); -1 if none (llm_runner.c:143-149)."""
    if use_max:
        return buckets[-1]
    for b in buckets:
        if b >= needed:
            return b
    return -1


def plan(n_prompt, max_new, chunk, buckets, max_ctx, use_max=False):
    """Validate like llm_runner.c:168-173 and return the (prefill buckets, decode buckets) it uses."""
    if n_prompt == 0:
        raise RunnerError("empty prompt")
    total = n_prompt + max_new
    if total > max_ctx or ((n_prompt + chunk - 1) // chunk) * chunk > max_ctx:
        raise RunnerError(f"prompt {n_prompt} + new {max_new} exceeds max_ctx {max_ctx}")
    pre = [pick_bucket(buckets, s + chunk, use_max) for s in range(0, n_prompt, chunk)]
    if any(L < 0 for L in pre):
        raise RunnerError(f"no bucket >= {max(s + chunk for s in range(0, n_prompt, chunk))}")
    dec = [pick_bucket(buckets, pos + 1, use_max) for pos in range(n_prompt, total - 1)]
    return pre, dec


@torch.no_grad()
def run(model, prompt, max_new_tokens=32, chunk=128, buckets=(256, 512, 1024, 2048, 4096), schedule="bucketed",
        stop_ids=(), warmup=1, caches=None, sync_timing=True, decode_steps=8):
    """Generate with the llm_runner.c schedule; returns the runner's JSON report as a dict.

    decode_steps > 1: while `decode_steps` more tokens fit in max_new_tokens and in the current bucket,
    one graph replay runs that many decode steps (the model's multi-step entry point) and the host
    reads their tokens back at once; tokens after a stop id are dropped (their steps only wrote cache
    rows past the end of the sequence). The generated tokens are those of one step per replay."""
    buckets = sorted(buckets)
    use_max = schedule == "max"
    n_prompt = len(prompt)
    pre, dec = plan(n_prompt, max_new_tokens, chunk, buckets, model.max_ctx, use_max)
    caches = caches if caches is not None else model.new_caches()
    dev = model.device
    fns = {}

    def fn(Cn, L):
        if (Cn, L) not in fns:
            fns[(Cn, L)] = model.entry_point(Cn, L, caches)
        return fns[(Cn, L)]

    def dec_fn(L, k):
        if k == 1:
            return fn(1, L)
        if ("run", L, k) not in fns:
            fns[("run", L, k)] = model.entry_point(1, L, caches, steps=k)
        return fns[("run", L, k)]

    def run_len(pos, n_have):
        """decode steps of the next replay at position pos with n_have tokens generated"""
        if decode_steps <= 1 or n_have + decode_steps > max_new_tokens:
            return 1
        L = pick_bucket(buckets, pos + 1, use_max)
        return decode_steps if pick_bucket(buckets, pos + decode_steps, use_max) == L else 1

    # warm-up: every function the schedule uses; writes garbage KV at [0, C) that prefill overwrites
    t_warm = time.perf_counter()
    for _ in range(warmup):
        for L in sorted(set(pre)):
            fn(chunk, L)([0] * chunk, 0, 0)
        for L in sorted(set(dec)):
            fn(1, L)([0], 0, 0)
            if decode_steps > 1 and dec.count(L) >= decode_steps:
                dec_fn(L, decode_steps)  # built (captured), not run
    torch.cuda.synchronize(dev)
    t_warm = time.perf_counter() - t_warm

    chunks, steps, generated = [], [], []
    t0 = time.perf_counter()
    nxt = None
    for i, s in enumerate(range(0, n_prompt, chunk)):
        n = min(chunk, n_prompt - s)
        toks = list(prompt[s:s + n]) + [0] * (chunk - n)
        tc = time.perf_counter()
        nxt = int(fn(chunk, pre[i])(toks, s, n - 1).item())
        chunks.append([pre[i], (time.perf_counter() - tc) * 1e3])
    prefill_s = time.perf_counter() - t0
    generated.append(nxt)
    t1 = time.perf_counter()
    pos = n_prompt
    fed = {}  # decode graph -> (start, token) its device inputs hold after its last replay
    while len(generated) < max_new_tokens:
        if generated[-1] in stop_ids:
            break
        L = pick_bucket(buckets, pos + 1, use_max)
        if L < 0:
            break
        k = run_len(pos, len(generated))
        ts = time.perf_counter()
        g = dec_fn(L, k)
        if fed.get(id(g)) != (pos, generated[-1]):
            g.set_fed(pos, generated[-1])
        out = g.replay()
        toks = [int(out.item())] if k == 1 else out.tolist()
        if g.feeds_back:
            fed[id(g)] = (pos + k, toks[-1])
        ms = (time.perf_counter() - ts) * 1e3 / k
        for t in toks:
            steps.append([L, ms])
            generated.append(t)
            pos += 1
            if t in stop_ids:
                break
    decode_s = time.perf_counter() - t1
    n_steps = len(generated) - 1
    return {
        "schedule": schedule, "chunk": chunk, "prompt_tokens": n_prompt, "new_tokens": len(generated),
        "warmup_ms": round(t_warm * 1e3, 1), "prefill_ms": round(prefill_s * 1e3, 1),
        "prefill_tok_s": round(n_prompt / prefill_s, 2), "ttft_ms": round(prefill_s * 1e3, 1),
        "decode_ms": round(decode_s * 1e3, 1), "decode_steps": n_steps,
        "decode_tok_s": round(n_steps / decode_s, 2) if n_steps > 0 else 0.0,
        "chunks": [[L, round(ms, 1)] for L, ms in chunks], "steps": [[L, round(ms, 2)] for L, ms in steps],
        "tokens": generated,
    }


def parse_ints(s):
    out = []
    for tok in s.replace(",", " ").split():
        try:
            out.append(int(tok))
        except ValueError:
            continue
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    src = ap.add_mutually_exclusive_group(required=True)
    src.add_argument("--model-dir", type=pathlib.Path)
    src.add_argument("--synthetic", choices=["tiny", "3b"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--group", type=int, default=None)
    ap.add_argument("--prompt", required=True, help="file with whitespace-separated prompt token ids")
    ap.add_argument("--max_new_tokens", type=int, default=32)
    ap.add_argument("--chunk", type=int, default=128)
    ap.add_argument("--buckets", default="256,512,1024,2048,4096")
    ap.add_argument("--schedule", default="bucketed", choices=["bucketed", "max"])
    ap.add_argument("--n_layers", type=int, default=None)
    ap.add_argument("--max_ctx", type=int, default=None)
    ap.add_argument("--stop_ids", default="")
    ap.add_argument("--warmup", type=int, default=1)
    a = ap.parse_args(argv)
    from . import synth
    from .llama_q4 import LlamaQ4
    buckets = parse_ints(a.buckets)
    max_ctx = a.max_ctx or max(buckets)
    if a.synthetic:
        cfg = synth.TINY if a.synthetic == "tiny" else synth.LLAMA32_3B
        group = a.group or (synth.TINY_GROUP if a.synthetic == "tiny" else synth.LLAMA32_3B_GROUP)
        model = LlamaQ4(None, group=group, max_ctx=max_ctx, n_layers=a.n_layers, sd=synth.SyntheticWeights(cfg, a.seed),
                        cfg=cfg)
    else:
        model = LlamaQ4(a.model_dir, group=a.group or 32, max_ctx=max_ctx, n_layers=a.n_layers)
    prompt = parse_ints(pathlib.Path(a.prompt).read_text())
    try:
        res = run(model, prompt, a.max_new_tokens, a.chunk, buckets, a.schedule, set(parse_ints(a.stop_ids)), a.warmup)
    except RunnerError as e:
        print(f"error: {e}", file=sys.stderr)
        return 1
    print(json.dumps(res, separators=(",", ":")))
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Context-length sweep of batch-1 generation with the native runner, and its summary table.

    python -m q4llm.sweep run (--weights model.q4w | --synthetic tiny|3b) --out results.jsonl
           [--ctx 256 512 1024 2048 4096] [--new 64] [--schedule bucketed max] [--chunk 128]
           [--buckets 256,512,1024,2048,4096] [--kinds random] [--prompt-files ids.txt ...] [--tag run]
    python -m q4llm.sweep summarize results.jsonl [more.jsonl ...] [--json rows.json]

The counterpart of the reference's scripts/llm/bench.py:69-107 and summarize.py:13-38. For each
(prompt kind, context length) a prompt of ctx - new tokens is built, lib/llm-runner generates `new`
tokens under each schedule, and the runner's JSON line plus (kind, ctx, tag) is appended to the
output file; `summarize` prints per (tag, schedule, ctx) medians over the kinds with speedups
against the first (tag, schedule), as the reference does.

Prompts: the reference fills chat-templated prompts from three text corpora through the Llama-3
tokenizer. No tokenizer is available offline, so a kind here is either `random` (uniform ids from a
seeded PCG64 stream, seed = ctx) or an id file given with --prompt-files (the file's ids repeated
until long enough and cut to length, as build_prompt does with its corpus, bench.py:54-63).
Batch-1 step time does not depend on the token values.
"""

import argparse
import collections
import json
import pathlib
import statistics
import subprocess
import sys
import tempfile

import numpy as np

PKG = pathlib.Path(__file__).resolve().parent.parent
RUNNER = PKG / "lib" / "llm-runner"


def make_prompt(kind, n_tokens, vocab, files):
    if kind == "random":
        return np.random.default_rng(n_tokens).integers(0, vocab, n_tokens).tolist()
    ids = [int(v) for v in pathlib.Path(files[kind]).read_text().split()]
    if not ids:
        raise ValueError(f"prompt file {files[kind]} holds no ids")
    while len(ids) < n_tokens:
        ids = ids + ids
    return ids[:n_tokens]


def run_runner(weights, prompt, new, chunk, buckets, schedule, extra=()):
    with tempfile.NamedTemporaryFile("w", suffix=".txt", delete=False) as f:
        f.write(" ".join(map(str, prompt)))
        pf = f.name
    try:
        cmd = [str(RUNNER), f"--weights={weights}", f"--prompt={pf}", f"--max_new_tokens={new}", f"--chunk={chunk}",
               f"--buckets={buckets}", f"--schedule={schedule}", *extra]
        r = subprocess.run(cmd, capture_output=True, text=True)
    finally:
        pathlib.Path(pf).unlink(missing_ok=True)
    if r.returncode != 0:
        raise RuntimeError(f"llm-runner failed ({r.returncode}): {r.stderr.strip()[-800:]}")
    return json.loads(next(line for line in r.stdout.splitlines() if line.startswith("{")))


def synthetic_weights(name, max_ctx, path):
    """Build the synthetic BASELINE model (GPU quantization) and save it packed to `path`."""
    import torch
    from . import synth
    from .llama_q4 import LlamaQ4
    cfg, group = (synth.TINY, synth.TINY_GROUP) if name == "tiny" else (synth.LLAMA32_3B, synth.LLAMA32_3B_GROUP)
    sd = synth.PrefetchingWeights(cfg, seed=0) if name == "3b" else synth.SyntheticWeights(cfg, 0)
    model = LlamaQ4(None, group=group, max_ctx=max_ctx, sd=sd, cfg=cfg)
    if hasattr(sd, "close"):
        sd.close()
    model.save_packed(path)
    vocab = model.embed.vocab
    del model
    torch.cuda.empty_cache()
    return vocab


def cmd_run(a):
    from . import packed
    tmp = None
    if a.synthetic:
        tmp = tempfile.mkdtemp()
        weights = pathlib.Path(tmp) / f"{a.synthetic}.q4w"
        synthetic_weights(a.synthetic, max(int(b) for b in a.buckets.split(",")), weights)
    else:
        weights = pathlib.Path(a.weights)
    cfg, _ = packed.read_header(weights)
    files = {pathlib.Path(p).stem: p for p in (a.prompt_files or [])}
    kinds = list(a.kinds) + list(files)
    out = pathlib.Path(a.out)
    out.parent.mkdir(parents=True, exist_ok=True)
    try:
        for kind in kinds:
            for ctx in a.ctx:
                prompt = make_prompt(kind, ctx - a.new, cfg["vocab"], files)
                for sched in a.schedule:
                    res = run_runner(weights, prompt, a.new, a.chunk, a.buckets, sched)
                    res.update(kind=kind, ctx=ctx, tag=a.tag, weights=weights.name)
                    with open(out, "a") as f:
                        f.write(json.dumps(res) + "\n")
                    print(f"{kind:8s} ctx={ctx:5d} {sched:8s} prompt={res['prompt_tokens']:5d} prefill "
                          f"{res['prefill_tok_s']:9.1f} tok/s (TTFT {res['ttft_ms']:7.1f} ms)  decode "
                          f"{res['decode_tok_s']:7.1f} tok/s", flush=True)
    finally:
        if tmp:
            pathlib.Path(weights).unlink(missing_ok=True)
            pathlib.Path(tmp).rmdir()
    return 0


def summarize(records):
    """Rows of per (tag, schedule, ctx) medians over prompt kinds, in (tag, schedule, ctx) order."""
    groups = collections.defaultdict(list)
    for r in records:
        groups[(r["tag"], r["schedule"], r["ctx"])].append(r)
    rows = []
    for (tag, sched, ctx), rs in sorted(groups.items()):
        rows.append(dict(tag=tag, schedule=sched, ctx=ctx, n=len(rs),
                         prefill_tok_s=statistics.median(r["prefill_tok_s"] for r in rs),
                         ttft_s=statistics.median(r["ttft_ms"] for r in rs) / 1e3,
                         decode_tok_s=statistics.median(r["decode_tok_s"] for r in rs)))
    return rows


def table(rows):
    """Markdown table with speedups against the first (tag, schedule) at the same ctx."""
    if not rows:
        return ""
    first = (rows[0]["tag"], rows[0]["schedule"])
    base = {r["ctx"]: r for r in rows if (r["tag"], r["schedule"]) == first}
    lines = ["| config | ctx | prefill tok/s | TTFT s | decode tok/s | prefill x | decode x |",
             "|---|---|---|---|---|---|---|"]
    for r in rows:
        b = base.get(r["ctx"])
        sp = r["prefill_tok_s"] / b["prefill_tok_s"] if b else float("nan")
        sd = r["decode_tok_s"] / b["decode_tok_s"] if b and b["decode_tok_s"] else float("nan")
        lines.append(f"| {r['tag']}/{r['schedule']} | {r['ctx']} | {r['prefill_tok_s']:.1f} | {r['ttft_s']:.3f} | "
                     f"{r['decode_tok_s']:.1f} | {sp:.2f} | {sd:.2f} |")
    return "\n".join(lines)


def cmd_summarize(a):
    records = [json.loads(line) for f in a.files for line in pathlib.Path(f).read_text().splitlines() if line.strip()]
    rows = summarize(records)
    print(table(rows))
    if a.json:
        pathlib.Path(a.json).write_text(json.dumps(rows, indent=1))
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    src = r.add_mutually_exclusive_group(required=True)
    src.add_argument("--weights")
    src.add_argument("--synthetic", choices=["tiny", "3b"])
    r.add_argument("--out", required=True)
    r.add_argument("--ctx", type=int, nargs="+", default=[256, 512, 1024, 2048, 4096])
    r.add_argument("--new", type=int, default=64)
    r.add_argument("--schedule", nargs="+", default=["bucketed"], choices=["bucketed", "max"])
    r.add_argument("--chunk", type=int, default=128)
    r.add_argument("--buckets", default="256,512,1024,2048,4096")
    r.add_argument("--kinds", nargs="*", default=["random"])
    r.add_argument("--prompt-files", nargs="*", help="id files; each file's stem becomes a prompt kind")
    r.add_argument("--tag", default="run")
    s = sub.add_parser("summarize")
    s.add_argument("files", nargs="+")
    s.add_argument("--json")
    a = ap.parse_args(argv)
    return cmd_run(a) if a.cmd == "run" else cmd_summarize(a)


if __name__ == "__main__":
    sys.exit(main())

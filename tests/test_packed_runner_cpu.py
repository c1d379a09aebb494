"""CPU checks of the packed-weight format (q4llm/packed.py) and of the native runner's schedule
(lib/llm-runner --plan), which must equal llm_runner.c's (runner/llm_runner.c:143-173, 210-245) as
restated by the Python runner; these run without a GPU."""

import pathlib
import subprocess

import pytest
import torch

from q4llm import llm_runner, packed

ROOT = pathlib.Path(__file__).resolve().parent.parent
RUNNER = ROOT / "iree-adreno-genai-tuner_amd" / "lib" / "llm-runner"
CFG = dict(dim=256, n_layers=1, n_heads=4, n_kv=2, head_dim=64, inter=704, vocab=1024, group=32, max_ctx=128,
           eps=1e-5)


def test_packed_round_trip_bit_exact(tmp_path):
    g = torch.Generator().manual_seed(0)
    t = {
        "embed.qweight": torch.randint(-2 ** 31, 2 ** 31 - 1, (1024, 32), dtype=torch.int32, generator=g),
        "embed.scales": torch.randn(1024, 8, generator=g).half(),
        "ln_f": torch.randn(256, generator=g),
        "cos": torch.randn(128, 64, generator=g),
        "odd": torch.randn(3, 5, 7, generator=g),  # sizes that are not multiples of the alignment
    }
    p = tmp_path / "m.q4w"
    size = packed.write(p, CFG, t)
    assert size == p.stat().st_size
    cfg, meta = packed.read_header(p)
    assert cfg == CFG and list(meta) == list(t)
    offs = [meta[k][1] for k in t]
    assert all(o % packed.ALIGN == 0 for o in offs) and offs == sorted(offs)
    cfg2, t2 = packed.read(p)
    for k, v in t.items():
        assert t2[k].dtype == v.dtype and t2[k].shape == v.shape
        assert torch.equal(t2[k].view(torch.int8), v.contiguous().view(torch.int8)), k
    _, only = packed.read(p, names={"ln_f"})
    assert list(only) == ["ln_f"]


def test_packed_rejects_bad_files(tmp_path):
    bad = tmp_path / "bad.q4w"
    bad.write_bytes(b"not a packed file\n")
    with pytest.raises(packed.PackedFormatError):
        packed.read_header(bad)
    with pytest.raises(packed.PackedFormatError):
        packed.write(tmp_path / "x.q4w", {k: v for k, v in CFG.items() if k != "eps"}, {})
    with pytest.raises(packed.PackedFormatError):
        packed.write(tmp_path / "x.q4w", CFG, {"a b": torch.zeros(2)})
    p = tmp_path / "trunc.q4w"
    packed.write(p, CFG, {"w": torch.zeros(1000)})
    p.write_bytes(p.read_bytes()[:-2000])
    with pytest.raises(packed.PackedFormatError, match="past the end"):
        packed.read(p)


def _plan(tmp_path, prompt_len, *flags):
    ids = tmp_path / "ids.txt"
    ids.write_text(" ".join(str(i % 97) for i in range(prompt_len)))
    return subprocess.run([str(RUNNER), f"--prompt={ids}", "--plan", *flags], capture_output=True, text=True)


@pytest.mark.parametrize("n,new,chunk,buckets,max_ctx,schedule", [
    (16, 32, 16, [64, 128], 128, "bucketed"),
    (512, 256, 256, [256, 512, 1024, 2048, 4096], 4096, "bucketed"),
    (21, 10, 8, [16, 32, 64], 64, "bucketed"),
    (700, 40, 128, [256, 512, 1024, 2048, 4096], 4096, "max"),
    (1, 1, 4, [4, 8], 8, "bucketed"),
])
def test_native_plan_matches_runner_schedule(tmp_path, n, new, chunk, buckets, max_ctx, schedule):
    r = _plan(tmp_path, n, f"--max_new_tokens={new}", f"--chunk={chunk}", "--buckets=" + ",".join(map(str, buckets)),
              f"--max_ctx={max_ctx}", f"--schedule={schedule}")
    assert r.returncode == 0, r.stderr
    import json
    got = json.loads(r.stdout)
    pre, dec = llm_runner.plan(n, new, chunk, buckets, max_ctx, use_max=schedule == "max")
    assert got["prefill"] == pre and got["decode"] == dec


@pytest.mark.parametrize("n,flags,msg", [
    (0, ["--buckets=64,128"], "empty prompt"),
    (4000, ["--max_new_tokens=200", "--chunk=256", "--max_ctx=4096"], "exceeds max_ctx"),
    (300, ["--max_new_tokens=10", "--chunk=256", "--buckets=256", "--max_ctx=4096"], "no bucket"),
    (8, ["--schedule=greedy"], "--schedule"),
    (8, ["--buckets=128,64"], "ascending"),
    (8, ["--frobnicate=1"], "unknown flag"),
])
def test_native_runner_errors_exit_1(tmp_path, n, flags, msg):
    r = _plan(tmp_path, n, *flags)
    assert r.returncode == 1 and msg in r.stderr, (r.returncode, r.stderr)


def test_sweep_summary_medians_and_speedups():
    from q4llm import sweep
    recs = []
    for tag, sched, f in (("run", "bucketed", 1.0), ("run", "max", 0.5)):
        for ctx in (256, 512):
            for kind, k in (("a", 1.0), ("b", 3.0), ("c", 2.0)):
                recs.append(dict(tag=tag, schedule=sched, ctx=ctx, kind=kind, prefill_tok_s=1000 * k * f,
                                 ttft_ms=10 * k, decode_tok_s=100 * k * f))
    rows = sweep.summarize(recs)
    assert [(r["tag"], r["schedule"], r["ctx"]) for r in rows] == [
        ("run", "bucketed", 256), ("run", "bucketed", 512), ("run", "max", 256), ("run", "max", 512)]
    assert rows[0]["prefill_tok_s"] == 2000 and rows[0]["decode_tok_s"] == 200 and rows[0]["ttft_s"] == 0.02
    t = sweep.table(rows).splitlines()
    assert t[2].endswith("| 1.00 | 1.00 |") and t[4].endswith("| 0.50 | 0.50 |")


def test_sweep_prompts(tmp_path):
    from q4llm import sweep
    a = sweep.make_prompt("random", 300, 1024, {})
    assert a == sweep.make_prompt("random", 300, 1024, {}) and len(a) == 300 and max(a) < 1024
    f = tmp_path / "chat.txt"
    f.write_text("5 6 7")
    assert sweep.make_prompt("chat", 7, 1024, {"chat": f}) == [5, 6, 7, 5, 6, 7, 5]

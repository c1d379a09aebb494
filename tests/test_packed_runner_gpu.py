"""GPU checks of the packed-weight path and the native runner (lib/llm-runner): a model saved with
LlamaQ4.save_packed and loaded with LlamaQ4.from_packed, or run by the native runner, generates the
golden greedy tokens of BASELINE config 1 (tests/golden/tiny_tokens.json) and the Python runner's
tokens on a ragged prompt with stop ids (runner/llm_runner.c:143-262)."""

import json
import pathlib
import subprocess

import pytest
import torch

from q4llm import llm_runner, synth
from q4llm.llama_q4 import LlamaQ4

pytestmark = pytest.mark.gpu
ROOT = pathlib.Path(__file__).resolve().parent.parent
GOLD = ROOT / "tests" / "golden"
RUNNER = ROOT / "iree-adreno-genai-tuner_amd" / "lib" / "llm-runner"
VARIANT = "std0.2"


@pytest.fixture(scope="module")
def gold():
    return json.loads((GOLD / "tiny_tokens.json").read_text())[VARIANT]


@pytest.fixture(scope="module")
def packed_file(tmp_path_factory, gold, dev):
    sd = synth.SyntheticWeights(synth.TINY, gold["seed"], std=gold["std"])
    model = LlamaQ4(None, group=gold["group"], max_ctx=gold["max_ctx"], sd=sd, cfg=synth.TINY)
    p = tmp_path_factory.mktemp("packed") / "tiny.q4w"
    model.save_packed(p)
    return p, model


def run_native(weights, prompt, tmp_path, *flags):
    ids = tmp_path / "prompt.txt"
    ids.write_text(" ".join(map(str, prompt)))
    print(f"[native-runner] {weights.name} prompt={len(prompt)} {' '.join(flags)}", flush=True)
    r = subprocess.run([str(RUNNER), f"--weights={weights}", f"--prompt={ids}", *flags], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


def test_from_packed_is_bit_identical_and_generates_golden(packed_file, gold):
    p, model = packed_file
    loaded = LlamaQ4.from_packed(p)
    for k, v in model.packed_tensors().items():
        w = loaded.packed_tensors()[k]
        assert w.dtype == v.dtype and torch.equal(w.view(torch.int8), v.contiguous().view(torch.int8)), k
    res = llm_runner.run(loaded, gold["prompt"], gold["max_new_tokens"], gold["chunk"], gold["buckets"])
    assert res["tokens"] == gold["tokens"]


def test_native_runner_generates_golden(packed_file, gold, tmp_path):
    p, model = packed_file
    res = run_native(p, gold["prompt"], tmp_path, f"--max_new_tokens={gold['max_new_tokens']}",
                     f"--chunk={gold['chunk']}", "--buckets=" + ",".join(map(str, gold["buckets"])))
    assert res["tokens"] == gold["tokens"]
    py = llm_runner.run(model, gold["prompt"], gold["max_new_tokens"], gold["chunk"], gold["buckets"])
    assert list(res) == list(py)  # the same report keys, in the same order (llm_runner.c:249-262)
    assert res["decode_steps"] == gold["max_new_tokens"] - 1 and [L for L, _ in res["chunks"]] == [64]


def test_native_runner_ragged_prompt_stop_ids_and_max_schedule(packed_file, tmp_path):
    p, model = packed_file
    prompt = synth.prompt_ids(21, 1024, seed=3)
    py = llm_runner.run(model, prompt, 10, 8, [16, 32, 64])
    res = run_native(p, prompt, tmp_path, "--max_new_tokens=10", "--chunk=8", "--buckets=16,32,64")
    assert res["tokens"] == py["tokens"]
    assert [L for L, _ in res["chunks"]] == [16, 16, 32] and [L for L, _ in res["steps"]] == [L for L, _ in py["steps"]]
    stop = py["tokens"][3]
    res2 = run_native(p, prompt, tmp_path, "--max_new_tokens=10", "--chunk=8", "--buckets=16,32,64",
                      f"--stop_ids={stop}")
    assert res2["tokens"] == py["tokens"][: py["tokens"].index(stop) + 1]
    res3 = run_native(p, prompt, tmp_path, "--max_new_tokens=10", "--chunk=8", "--buckets=16,32,64",
                      "--schedule=max")
    assert res3["tokens"] == py["tokens"] and {L for L, _ in res3["steps"]} == {64}


def test_native_runner_no_warmup_keeps_live_kv(packed_file, tmp_path):
    """--warmup=0: each entry point (a prefill bucket switch 16 -> 32, a decode switch 32 -> 64) is
    first built while the caches hold the live sequence; its set-up launch must not write them."""
    p, model = packed_file
    prompt = synth.prompt_ids(21, 1024, seed=3)
    py = llm_runner.run(model, prompt, 20, 8, [16, 32, 64])
    res = run_native(p, prompt, tmp_path, "--max_new_tokens=20", "--chunk=8", "--buckets=16,32,64", "--warmup=0")
    assert {L for L, _ in res["steps"]} == {32, 64}
    assert res["tokens"] == py["tokens"]


def test_native_runner_multi_step_decode(packed_file, tmp_path):
    """--decode_steps: launches of 8 (or 5) self-feeding decode steps, single steps next to the bucket
    switches and the end, give the one-step runner's tokens; a stop id inside a launch ends the
    output at that token."""
    p, model = packed_file
    prompt = synth.prompt_ids(10, 1024, seed=8)
    flags = ("--max_new_tokens=60", "--chunk=8", "--buckets=16,32,64,128")
    one = run_native(p, prompt, tmp_path, *flags, "--decode_steps=1")
    py = llm_runner.run(model, prompt, 60, 8, [16, 32, 64, 128], decode_steps=1)
    assert one["tokens"] == py["tokens"]
    for k in (8, 5):
        assert run_native(p, prompt, tmp_path, *flags, f"--decode_steps={k}")["tokens"] == one["tokens"], k
    stop = one["tokens"][30]
    first = one["tokens"].index(stop)
    got = run_native(p, prompt, tmp_path, *flags, "--decode_steps=8", f"--stop_ids={stop}")
    assert got["tokens"] == one["tokens"][: first + 1]


def test_context_sweep_records(packed_file, tmp_path):
    """q4llm.sweep (scripts/llm/bench.py:69-107 contract): one record per (kind, ctx, schedule) with
    the runner's keys plus kind/ctx/tag, and the summary table over them."""
    from q4llm import sweep
    p, _ = packed_file
    out = tmp_path / "sweep.jsonl"
    assert sweep.main(["run", f"--weights={p}", f"--out={out}", "--ctx", "48", "96", "--new", "8", "--chunk", "16",
                       "--buckets", "64,128", "--schedule", "bucketed", "max", "--tag", "t"]) == 0
    recs = [json.loads(line) for line in out.read_text().splitlines()]
    assert [(r["ctx"], r["schedule"]) for r in recs] == [(48, "bucketed"), (48, "max"), (96, "bucketed"), (96, "max")]
    assert all(r["prompt_tokens"] == r["ctx"] - 8 and r["new_tokens"] == 8 for r in recs)
    assert {L for L, _ in recs[0]["steps"]} == {64} and {L for L, _ in recs[1]["steps"]} == {128}
    assert recs[0]["tokens"] == recs[1]["tokens"]  # the schedule changes buckets, not results
    rows = sweep.summarize(recs)
    assert len(rows) == 4 and "| t/bucketed | 48 |" in sweep.table(rows)

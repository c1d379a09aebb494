"""The Hugging Face checkpoint path (row f2, llama_q4.py:125-138,159-164): a synthetic tiny Llama
written as two safetensors shards plus config.json is loaded lazily by LlamaQ4(model_dir), quantized
on the GPU and run through the Python runner, the `--model-dir` CLI and, after save_packed, the
native runner. fp32 shards give the golden greedy tokens of BASELINE config 1 (tests/golden,
std-0.2 variant); bf16 shards (the dtype of real Llama-3.2 checkpoints) give the CPU oracle's
tokens on the same bf16 weights."""

import json
import pathlib
import subprocess
import sys

import pytest
import torch

from oracle import llama_q4_ref as R
from q4llm import llm_runner, synth
from q4llm.llama_q4 import LlamaQ4

pytestmark = pytest.mark.gpu
ROOT = pathlib.Path(__file__).resolve().parent.parent
GOLD = ROOT / "tests" / "golden"
RUNNER = ROOT / "iree-adreno-genai-tuner_amd" / "lib" / "llm-runner"


@pytest.fixture(scope="module")
def gold():
    return json.loads((GOLD / "tiny_tokens.json").read_text())["std0.2"]


def write_checkpoint(d: pathlib.Path, sd, cfg, dtype):
    """Two shards (layers split between them, as HF sharding does) and config.json."""
    from safetensors.torch import save_file
    d.mkdir(parents=True, exist_ok=True)
    names = list(sd.keys())
    half = len(names) // 2
    for i, part in enumerate((names[:half], names[half:])):
        save_file({k: sd[k].to(dtype).contiguous() for k in part},
                  str(d / f"model-{i + 1:05d}-of-00002.safetensors"), metadata={"format": "pt"})
    (d / "config.json").write_text(json.dumps(dict(cfg, model_type="llama", architectures=["LlamaForCausalLM"],
                                                   torch_dtype=str(dtype).replace("torch.", ""))))
    return d


@pytest.fixture(scope="module")
def ckpt_f32(tmp_path_factory, gold):
    sd = synth.SyntheticWeights(synth.TINY, gold["seed"], std=gold["std"])
    return write_checkpoint(tmp_path_factory.mktemp("hf_f32"), sd, synth.TINY, torch.float32)


def test_model_dir_loads_bit_exact_and_generates_golden(dev, gold, ckpt_f32):
    print(f"[checkpoint] {sorted(p.name for p in ckpt_f32.iterdir())}", flush=True)
    model = LlamaQ4(ckpt_f32, group=gold["group"], max_ctx=gold["max_ctx"])
    sd = synth.SyntheticWeights(synth.TINY, gold["seed"], std=gold["std"])
    from_sd = LlamaQ4(None, group=gold["group"], max_ctx=gold["max_ctx"], sd=sd, cfg=synth.TINY)
    a, b = model.packed_tensors(), from_sd.packed_tensors()
    assert a.keys() == b.keys()
    for k in a:
        assert torch.equal(a[k].contiguous().view(torch.int8), b[k].contiguous().view(torch.int8)), k
    res = llm_runner.run(model, gold["prompt"], gold["max_new_tokens"], gold["chunk"], gold["buckets"])
    assert res["tokens"] == gold["tokens"]


def test_model_dir_cli_and_native_runner(dev, gold, ckpt_f32, tmp_path):
    ids = tmp_path / "prompt.txt"
    ids.write_text(" ".join(map(str, gold["prompt"])))
    flags = [f"--prompt={ids}", f"--max_new_tokens={gold['max_new_tokens']}", f"--chunk={gold['chunk']}",
             "--buckets=" + ",".join(map(str, gold["buckets"])), f"--max_ctx={gold['max_ctx']}"]
    cmd = [sys.executable, "-m", "q4llm.llm_runner", f"--model-dir={ckpt_f32}", f"--group={gold['group']}", *flags]
    print("[cli] " + " ".join(cmd[1:]), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300,
                       cwd=str(ROOT / "iree-adreno-genai-tuner_amd"))
    assert r.returncode == 0, r.stderr
    assert json.loads(r.stdout)["tokens"] == gold["tokens"]
    # the model-dir model saved as a packed file and run by the native runner
    model = LlamaQ4(ckpt_f32, group=gold["group"], max_ctx=gold["max_ctx"])
    wpath = tmp_path / "tiny_from_hf.q4w"
    model.save_packed(wpath)
    print(f"[native-runner] {wpath.name}", flush=True)
    r = subprocess.run([str(RUNNER), f"--weights={wpath}", *flags], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert json.loads(r.stdout)["tokens"] == gold["tokens"]


def test_bf16_checkpoint_matches_oracle(dev, gold, tmp_path):
    """bf16 shards: Layer casts each tensor to fp32 on the device before quantizing, so the weights
    quantized are the bf16 values exactly; the oracle on the same bf16-rounded weights gives the
    same greedy tokens."""
    sd = synth.SyntheticWeights(synth.TINY, gold["seed"], std=gold["std"])
    d = write_checkpoint(tmp_path / "hf_bf16", sd, synth.TINY, torch.bfloat16)
    model = LlamaQ4(d, group=gold["group"], max_ctx=gold["max_ctx"])
    dense = {k: sd[k].to(torch.bfloat16).float() for k in sd.keys()}
    ref = R.LlamaQ4Ref(synth.TINY, dense, group=gold["group"], max_ctx=gold["max_ctx"],
                       rope=(model.cos.cpu(), model.sin.cpu()))
    assert torch.equal(model.embed.qweight.cpu(), ref.embed.qweight)
    want = R.generate(ref, gold["prompt"], gold["max_new_tokens"], gold["chunk"], gold["buckets"])
    res = llm_runner.run(model, gold["prompt"], gold["max_new_tokens"], gold["chunk"], gold["buckets"])
    assert res["tokens"] == want

"""CPU checks of host-side product code: RoPE tables (bit-identical to transformers, the source the
reference uses), and the runner's schedule validation (llm_runner.c:143-173)."""

import pytest
import torch

from q4llm import llm_runner, synth
from q4llm.rope import rope_tables

transformers = pytest.importorskip("transformers")

REF_TINY_ROPE = dict(hidden_size=256, num_attention_heads=8, num_key_value_heads=2, head_dim=32,
                     rope_theta=500000.0, max_position_embeddings=131072,
                     rope_scaling={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                   "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})


@pytest.mark.parametrize("cfg", [synth.TINY, synth.LLAMA32_3B, REF_TINY_ROPE], ids=["tiny", "3b", "ref_tiny_llama3"])
def test_rope_tables_bit_identical_to_transformers(cfg):
    from oracle.llama_q4_ref import rope_tables as hf_tables
    cos, sin = rope_tables(cfg, 4096)
    hc, hs = hf_tables(cfg, 4096)
    assert torch.equal(cos, hc) and torch.equal(sin, hs)


def test_pick_bucket_and_plan_errors():
    b = [256, 512, 1024, 2048, 4096]
    assert llm_runner.pick_bucket(b, 257) == 512
    assert llm_runner.pick_bucket(b, 5000) == -1
    assert llm_runner.pick_bucket(b, 1, use_max=True) == 4096
    pre, dec = llm_runner.plan(512, 256, 256, b, 4096)
    assert pre == [256, 512] and set(dec) == {1024} and len(dec) == 255
    with pytest.raises(llm_runner.RunnerError, match="empty prompt"):
        llm_runner.plan(0, 4, 16, b, 4096)
    with pytest.raises(llm_runner.RunnerError, match="exceeds max_ctx"):
        llm_runner.plan(4000, 200, 256, b, 4096)
    with pytest.raises(llm_runner.RunnerError, match="no bucket"):
        llm_runner.plan(300, 10, 256, [256], 4096)


def test_parse_ints_like_runner():
    assert llm_runner.parse_ints("1, 2,3\n 4 x 5") == [1, 2, 3, 4, 5]

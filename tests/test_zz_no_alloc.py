"""q4llm_step_noalloc (include/q4llm.h) through the C ABI: the step with its scratch in the library's
per-GPU device array gives the same next token, logits and KV caches as q4llm_step with a caller
workspace, bit for bit (same kernels), on two calls in a row, the second with a smaller input (a
16-token prefill chunk, then one decode token that reads the scratch the first call left behind);
a shape whose workspace exceeds the array is rejected with Q4_ERR_WORKSPACE."""

import ctypes as C

import pytest
import torch

from q4llm import synth
from q4llm._lib import LIB, ptr, stream_of
from q4llm.llama_q4 import LlamaQ4

pytestmark = pytest.mark.gpu
Q4_ERR_WORKSPACE = -5
SCRATCH_BYTES = 64 << 20


def i32(*v, dev):
    return torch.tensor(list(v), dtype=torch.int32, device=dev)


def test_step_noalloc_matches_step_on_two_calls(dev):
    sd = synth.SyntheticWeights(synth.TINY, 0, std=0.2)
    model = LlamaQ4(None, group=32, max_ctx=128, sd=sd, cfg=synth.TINY)
    desc = C.byref(model.descriptor())
    c_ref, c_na = model.new_caches(), model.new_caches()
    arr_ref, arr_na = model._cache_ptrs(c_ref), model._cache_ptrs(c_na)
    prompt = synth.prompt_ids(16, 1024, seed=5)
    V = model.embed.vocab
    s = stream_of(dev)
    calls = [(torch.tensor(prompt, dtype=torch.int32, device=dev), 0, 15, 64), (None, 16, 0, 64)]
    prev = None
    for i, (toks, start, last, L) in enumerate(calls):
        if toks is None:  # decode: feed the previous step's token
            toks = prev.clone()
        Cn = toks.numel()
        print(f"[no-alloc] call {i}: C={Cn} start={start} L={L}", flush=True)
        st, la = i32(start, dev=dev), i32(last, dev=dev)
        n_ref, l_ref = torch.empty(1, dtype=torch.int32, device=dev), torch.empty(V, device=dev)
        n_na, l_na = torch.full((1,), -1, dtype=torch.int32, device=dev), torch.full((V,), float("nan"), device=dev)
        ws = model.workspace(Cn, L)
        LIB.call("q4llm_step", desc, ptr(toks), Cn, ptr(st), ptr(la), arr_ref, L, ptr(n_ref), ptr(l_ref), ptr(ws),
                 ws.numel(), s)
        LIB.call("q4llm_step_noalloc", desc, ptr(toks), Cn, ptr(st), ptr(la), arr_na, L, ptr(n_na), ptr(l_na), s)
        torch.cuda.synchronize()
        assert int(n_na.item()) == int(n_ref.item())
        assert torch.equal(l_na, l_ref)
        for a, b in zip(c_na, c_ref):
            assert torch.equal(a, b)
        prev = n_ref


def test_step_noalloc_rejects_a_workspace_beyond_the_array(dev):
    cfg = dict(synth.TINY, vocab_size=SCRATCH_BYTES // 4 + 64, hidden_size=64, intermediate_size=64,
               num_attention_heads=1, num_key_value_heads=1, head_dim=64, num_hidden_layers=1)
    from q4llm.llama_q4 import _LayerC, _ModelC
    arr = (_LayerC * 1)(_LayerC(*([256] * 10)))
    m = _ModelC(64, 1, 1, 1, 64, 64, cfg["vocab_size"], 32, 128, 1e-5, 256, 256, 256, 256, 256,
                C.cast(arr, C.c_void_p))
    b = C.c_size_t(0)
    LIB.call("q4llm_step_workspace_bytes", C.byref(m), 1, 64, C.byref(b))
    assert b.value > SCRATCH_BYTES
    fake = torch.zeros(4, dtype=torch.int32, device=dev)
    caches = (C.c_void_p * 2)(fake.data_ptr(), fake.data_ptr())
    stv = LIB.raw("q4llm_step_noalloc")(C.byref(m), ptr(fake), 1, ptr(fake), ptr(fake), caches, 64, ptr(fake), None,
                                        stream_of(dev))
    assert stv == Q4_ERR_WORKSPACE

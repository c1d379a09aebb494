"""Host-side checks that need no GPU: the tensor wrappers reject wrong dtypes, shapes and layouts with
ValueError before any pointer reaches the library, and LazySafetensors (llama_q4.py:125-138) reads
tensors from sharded safetensors files exactly as they were written."""

import json

import pytest
import torch

from q4llm import ops, synth
from q4llm.llama_q4 import LazySafetensors


def w4(n=64, k=256, group=128):
    return torch.zeros(n, k // 8, dtype=torch.int32), torch.zeros(n, k // group, dtype=torch.float16)


@pytest.mark.parametrize("case", ["scales_f32", "scales_shape", "qweight_i64", "residual_1d_for_m2", "residual_f16",
                                  "out_shape", "x_f16", "x_k", "group"])
def test_q4_linear_rejects(case):
    qw, sc = w4()
    x = torch.zeros(2, 256)
    kw = dict(residual=None, out=None)
    group = 128
    if case == "scales_f32":
        sc = sc.float()
    elif case == "scales_shape":
        sc = torch.zeros(64, 4, dtype=torch.float16)
    elif case == "qweight_i64":
        qw = qw.long()
    elif case == "residual_1d_for_m2":
        kw["residual"] = torch.zeros(64)
    elif case == "residual_f16":
        kw["residual"] = torch.zeros(2, 64, dtype=torch.float16)
    elif case == "out_shape":
        kw["out"] = torch.zeros(1, 64)
    elif case == "x_f16":
        x = x.half()
    elif case == "x_k":
        x = torch.zeros(2, 128)
    elif case == "group":
        group = 96
    with pytest.raises(ValueError):
        ops.q4_linear(x, qw, sc, group, **kw)
    with pytest.raises(ValueError):
        ops.q4_linear_ws(x, qw, sc, group, **kw)


@pytest.mark.parametrize("case", ["scales_bf16", "residual_shape", "residual_with_f16_out", "x_len", "out_shape",
                                  "qweight_noncontig"])
def test_q4_gemv_rejects(case):
    qw, sc = w4()
    x = torch.zeros(256)
    kw = {}
    if case == "scales_bf16":
        sc = sc.to(torch.bfloat16)
    elif case == "residual_shape":
        kw["residual"] = torch.zeros(2, 64)
    elif case == "residual_with_f16_out":
        kw["residual"] = torch.zeros(64)
        kw["out"] = torch.zeros(64, dtype=torch.float16)
    elif case == "x_len":
        x = torch.zeros(255)
    elif case == "out_shape":
        kw["out"] = torch.zeros(63)
    elif case == "qweight_noncontig":
        qw = torch.zeros(32, 64, dtype=torch.int32).t()
    with pytest.raises(ValueError):
        ops.q4_gemv(qw, sc, x, 128, **kw)


def test_gemm_rejects_wrong_dtype_and_strided_rows():
    a = torch.zeros(4, 64, dtype=torch.float16)
    with pytest.raises(ValueError):
        ops.gemm_f16_nt(a.float(), torch.zeros(8, 64, dtype=torch.float16))
    with pytest.raises(ValueError):
        ops.gemm_f16_nt(a, torch.zeros(64, 8, dtype=torch.float16).t())
    with pytest.raises(ValueError):
        ops.gemm_f16_nt(a, torch.zeros(8, 64, dtype=torch.float16), out=torch.zeros(4, 8))


def test_valid_arguments_reach_the_device_check():
    """Well-formed CPU tensors pass every shape/dtype check and stop at the device check."""
    qw, sc = w4()
    with pytest.raises(ValueError, match="device"):
        ops.q4_linear(torch.zeros(2, 256), qw, sc, 128, residual=torch.zeros(2, 64))
    with pytest.raises(ValueError, match="device"):
        ops.q4_gemv(qw, sc, torch.zeros(256), 128, residual=torch.zeros(64))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lazy_safetensors_reads_two_shards(tmp_path, dtype):
    from safetensors.torch import save_file
    sd = synth.SyntheticWeights(synth.TINY, 0, std=0.2)
    names = list(sd.keys())
    half = len(names) // 2
    for i, part in enumerate((names[:half], names[half:])):
        save_file({k: sd[k].to(dtype) for k in part}, str(tmp_path / f"model-{i + 1:05d}-of-00002.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps(synth.TINY))
    lazy = LazySafetensors(tmp_path)
    assert len(lazy.handles) == 2 and set(lazy.where) == set(names)
    for k in (names[0], names[half - 1], names[half], names[-1]):
        assert k in lazy
        t = lazy[k]
        assert t.dtype == dtype and torch.equal(t, sd[k].to(dtype))
    assert "model.layers.99.mlp.up_proj.weight" not in lazy


def test_bench_profiled_constants_match_their_profiles():
    """bench.py carries two figures it cannot measure inside a timed run (the GEMV's counter-measured
    traffic and its rocprofv3 average); each must equal the figure in the profile file it names."""
    import pathlib
    import re
    import sys
    root = pathlib.Path(__file__).resolve().parent.parent
    sys.path.insert(0, str(root))
    import bench
    traffic = (root / bench.GEMV_TRAFFIC_SOURCE).read_text()
    assert f"{bench.GEMV_TRAFFIC_BYTES_5120x3072:,}" in traffic
    stats = (root / bench.GEMV_ROCPROF_SOURCE).read_text()
    row = next(line for line in stats.splitlines() if "N=5120, K=3072" in line and line.startswith("|"))
    avg = float(row.split("|")[3])
    assert avg == bench.GEMV_ROCPROF_AVG_US, (row, bench.GEMV_ROCPROF_AVG_US)
    for text in (stats, traffic):  # each names the committed command that produced it
        assert re.search(r"rocprofv3 .*bench\.py", text, re.S)

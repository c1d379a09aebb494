"""GPU parity of the matrix-core (int8 limb) decode GEMV used for fp32 activations.

The kernel turns each quantization group of x into exact integers (a power-of-two shift per group)
split into four signed bytes, and multiplies them with the raw nibbles on v_mfma_i32_16x16x64_i8.
The products are exact, so the result must sit within fp32 accumulation error of the fp64 oracle
(bar: 1e-5 x output RMS, the same bar as the fp32 model path), including for inputs the integer
conversion could get wrong: groups spanning many orders of magnitude, all-zero groups, exact
powers of two, a single non-zero element. The grid-stride variant (matrices taller than 65536 rows,
the tied LM head) and the short-matrix variant (8 used rows per block) are covered, and the result
is compared with the VALU kernel (the gemv_no_mx override) and checked to be deterministic."""


import numpy as np
import pytest
import torch

from oracle import llama_q4_ref as R
from q4llm import ops, synth

pytestmark = pytest.mark.gpu


def _problem(n, k, group, seed, x=None):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.02
    qw, sc = R.quantize_q4(w, group)
    if x is None:
        x = torch.randn(k, generator=g)
    ref = R.dequantize_q4(qw, sc, group).double() @ x.double()
    return qw, sc, x, ref


def _run(dev, qw, sc, x, group, no_mx=False):
    if no_mx:
        ops.debug_override("gemv_no_mx", 1)
    try:
        y = torch.full((qw.shape[0],), float("nan"), device=dev)
        ops.q4_gemv(qw.to(dev), sc.to(dev), x.to(dev), group, out=y)
        torch.cuda.synchronize()
        return y.cpu().double()
    finally:
        ops.debug_override("gemv_no_mx", None)


def _rel(y, ref):
    return (y - ref).abs().max().item() / ref.pow(2).mean().sqrt().item()


def _chunked_ref(qw, sc, x, group, rows=8192):
    out = []
    for r0 in range(0, qw.shape[0], rows):
        out.append(R.dequantize_q4(qw[r0:r0 + rows], sc[r0:r0 + rows], group).double() @ x.double())
    return torch.cat(out)


@pytest.mark.parametrize("n,k,group", [(65552, 3072, 128), (128256, 3072, 128)])
def test_mx_grid_stride_tall(dev, n, k, group):
    """Row counts past 65536 take the grid-stride variant (the 128256-row tied LM head); nibbles
    uniform in [0, 15], group scales |N(0, 0.01)| (the config-2 generator), x N(0, 1) fp32."""
    qw, sc, _ = synth.gemv_problem(n, k, group, seed=n)
    qw, sc = torch.from_numpy(qw), torch.from_numpy(sc)
    x = torch.randn(k, generator=torch.Generator().manual_seed(n))
    ref = _chunked_ref(qw, sc, x, group)
    y = _run(dev, qw, sc, x, group)
    assert torch.isfinite(y).all()
    assert _rel(y, ref) <= 1e-5


@pytest.mark.parametrize("n,k,group", [(3072, 3072, 128), (3072, 8192, 128), (200, 3072, 128), (24, 256, 32),
                                       (100, 704, 32), (4095, 512, 128)])
def test_mx_shapes_and_short_blocks(dev, n, k, group):
    qw, sc, x, ref = _problem(n, k, group, seed=n + k)
    assert _rel(_run(dev, qw, sc, x, group), ref) <= 1e-5


def _wide_range_x(k, group, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(k).astype(np.float32)
    ng = k // group
    for gi in range(ng):
        sl = slice(gi * group, (gi + 1) * group)
        kind = gi % 6
        if kind == 0:    # magnitudes from 1e-30 to 1e3 inside one group
            x[sl] *= (10.0 ** rng.uniform(-30, 3, group)).astype(np.float32)
        elif kind == 1:  # all zero
            x[sl] = 0.0
        elif kind == 2:  # exact powers of two, both signs
            x[sl] = np.sign(x[sl]) * 2.0 ** rng.integers(-20, 20, group)
        elif kind == 3:  # one non-zero element
            x[sl] = 0.0
            x[gi * group + 3] = -1234.5
        elif kind == 4:  # huge values
            x[sl] *= 1e20
        else:            # tiny values
            x[sl] *= 1e-25
    return torch.from_numpy(x)


@pytest.mark.parametrize("n,k,group", [(512, 3072, 128), (256, 256, 32), (384, 8192, 128)])
def test_mx_wide_dynamic_range(dev, n, k, group):
    """Per-group integer conversion: the error stays at fp32 level relative to each output's scale."""
    x = _wide_range_x(k, group, seed=k)
    qw, sc, _, _ = _problem(n, k, group, seed=k + 1)
    wd = R.dequantize_q4(qw, sc, group).double()
    ref = wd @ x.double()
    # fp32 accumulation bound: 2^-24-level error relative to sum_k |w x|
    bound = (wd.abs() @ x.double().abs()) * 1e-5
    y = _run(dev, qw, sc, x, group)
    assert torch.isfinite(y).all()
    assert ((y - ref).abs() <= bound + 1e-30).all()


def test_mx_matches_valu_kernel_and_is_deterministic(dev):
    qw, sc, x, ref = _problem(5120, 3072, 128, seed=11)
    a = _run(dev, qw, sc, x, 128)
    b = _run(dev, qw, sc, x, 128)
    assert torch.equal(a, b), "matrix-core GEMV is not deterministic"
    v = _run(dev, qw, sc, x, 128, no_mx=True)
    assert _rel(a, ref) <= 1e-5 and _rel(v, ref) <= 1e-5
    assert (a - v).abs().max().item() <= 2e-5 * ref.pow(2).mean().sqrt().item()

"""Packed-weight file: the quantized LlamaQ4 weights as they live in HBM, in one file.

This plays the part of the reference's IREE parameter archive (weights.irpa, written by
scripts/llm/export_llama.py:30-31 and read by the runner through --parameters): the int4 weights are
quantized once, saved in the exact device layout, and later loaded with plain copies by the Python
module (LlamaQ4.from_packed) or the native runner (lib/llm-runner --weights), with no quantization
pass and no checkpoint on hand.

Layout (all integers little-endian, offsets absolute from the start of the file):

    Q4LLM-PACKED 1
    config <key> <value>                          one line per model constant (ints; eps as %.9g)
    tensor <name> <dtype> <offset> <nbytes> <ndim> <d0> <d1> ...
    end
    <zero padding to `data_offset`> <tensor bytes, each 256-byte aligned>

dtype is one of i32, f16, f32. The header is ASCII text, so the file is self-describing and a C or
C++ loader needs nothing beyond sscanf. Tensor names:

    embed.qweight [vocab, dim/8] i32    embed.scales [vocab, dim/group] f16    ln_f [dim] f32
    cos [max_ctx, head_dim] f32         sin [max_ctx, head_dim] f32
    layers.<i>.{wqkv,wo,wgu,wdown}.{qweight,scales}   layers.<i>.ln_in [dim] f32   layers.<i>.ln_post
"""

import pathlib

import numpy as np
import torch

MAGIC = "Q4LLM-PACKED 1"
ALIGN = 256
CONFIG_KEYS = ("dim", "n_layers", "n_heads", "n_kv", "head_dim", "inter", "vocab", "group", "max_ctx")
_DT = {torch.int32: "i32", torch.float16: "f16", torch.float32: "f32"}
_NP = {"i32": np.int32, "f16": np.float16, "f32": np.float32}


class PackedFormatError(ValueError):
    pass


def _align(n: int, a: int = ALIGN) -> int:
    return (n + a - 1) // a * a


def write(path, config: dict, tensors: dict) -> int:
    """Write `tensors` (name -> torch tensor on any device) with the model `config` (CONFIG_KEYS plus
    'eps'); returns the file size in bytes. Tensors are written in insertion order."""
    missing = [k for k in CONFIG_KEYS + ("eps",) if k not in config]
    if missing:
        raise PackedFormatError(f"config lacks {missing}")
    lines = [MAGIC]
    lines += [f"config {k} {int(config[k])}" for k in CONFIG_KEYS]
    lines.append(f"config eps {float(config['eps']):.9g}")
    entries, off = [], 0
    for name, t in tensors.items():
        if t.dtype not in _DT:
            raise PackedFormatError(f"{name}: unsupported dtype {t.dtype}")
        if any(c.isspace() for c in name):
            raise PackedFormatError(f"tensor name {name!r} contains whitespace")
        nbytes = t.numel() * t.element_size()
        entries.append((name, t, off, nbytes))
        off = _align(off + nbytes)

    def header(data_offset):
        # offsets are fixed-width, so the header length does not depend on their values
        rows = [f"tensor {n} {_DT[t.dtype]} {data_offset + rel:016d} {nb} {t.dim()} " + " ".join(map(str, t.shape))
                for n, t, rel, nb in entries]
        return "\n".join(lines + rows + ["end", ""]).encode()

    data_offset = _align(len(header(0)), 4096)
    text = header(data_offset)
    path = pathlib.Path(path)
    with open(path, "wb") as f:
        f.write(text)
        f.write(b"\0" * (data_offset - len(text)))
        for name, t, rel, nb in entries:
            assert f.tell() == data_offset + rel, name
            f.write(t.detach().contiguous().cpu().numpy().tobytes())
            f.write(b"\0" * (_align(nb) - nb))
    return path.stat().st_size


def read_header(path):
    """Parse the header: (config dict, {name: (dtype, offset, nbytes, shape)})."""
    with open(path, "rb") as f:
        raw = f.read(1 << 20)
    end = raw.find(b"\nend\n")
    if not raw.startswith(MAGIC.encode() + b"\n") or end < 0:
        raise PackedFormatError(f"{path}: not a {MAGIC} file")
    cfg, tensors = {}, {}
    for line in raw[:end].decode().splitlines()[1:]:
        f = line.split()
        if f[0] == "config" and len(f) == 3:
            cfg[f[1]] = float(f[2]) if f[1] == "eps" else int(f[2])
        elif f[0] == "tensor" and len(f) >= 6:
            name, dt, off, nb, nd = f[1], f[2], int(f[3]), int(f[4]), int(f[5])
            shape = tuple(int(v) for v in f[6:6 + nd])
            if dt not in _NP or len(shape) != nd or int(np.prod(shape)) * np.dtype(_NP[dt]).itemsize != nb:
                raise PackedFormatError(f"{path}: bad tensor line {line!r}")
            tensors[name] = (dt, off, nb, shape)
        else:
            raise PackedFormatError(f"{path}: bad header line {line!r}")
    missing = [k for k in CONFIG_KEYS + ("eps",) if k not in cfg]
    if missing:
        raise PackedFormatError(f"{path}: config lacks {missing}")
    return cfg, tensors


def read(path, device=None, names=None):
    """Load tensors (all, or `names`) as torch tensors on `device` (CPU by default) via a read-only
    memory map of the file; returns (config, {name: tensor})."""
    cfg, meta = read_header(path)
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    out = {}
    for name, (dt, off, nb, shape) in meta.items():
        if names is not None and name not in names:
            continue
        if off + nb > mm.shape[0]:
            raise PackedFormatError(f"{path}: tensor {name} runs past the end of the file")
        arr = np.frombuffer(mm[off:off + nb], dtype=_NP[dt]).reshape(shape)
        t = torch.from_numpy(arr.copy())
        out[name] = t.to(device) if device is not None else t
    del mm
    return cfg, out

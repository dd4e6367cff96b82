"""The ``bf16x-v1`` on-disk format: a model's packed linears in one
safetensors file plus a meta JSON, loaded without re-quantization.

Mirrors pack_to_disk.py (same names, arguments, file layout and key names):

  <prefix>.safetensors   per packed linear <name>:
      <name>.sign / .mant / .delta   int32 word streams, each followed by one
                                     zero word (pack_to_disk.py:33-34, 67-69)
      <name>.emax                    uint8, one per 16 elements
      <name>.ovf_i / .ovf_v          int64 flat positions / int32 true deltas
                                     of the entries with delta > 7 only
                                     (the delta == 7 sentinel stays saturated,
                                     :62-64)
      <name>.bias                    bf16, when the linear has one (:79-84)
    file metadata {"format": "bf16x"} (:96)
  <prefix>.meta.json     {"kind": "bf16x-v1", "tensors": {name: {sign, mant,
                          delta, emax, ovf_i, ovf_v[, bias], out_f, in_f, N,
                          n_fix}}} (:14-17, 74-84)

Writing encodes with the C++ encoder (``bf16x_quantize``); loading reads the
file with safetensors (memory-mapped), checks every entry against the
shapes it claims, moves the streams to the GPU once and builds the device
overflow plan from the table.  ``Bf16xStreamLinear`` runs the exact fused
GEMV / GEMM (or, in mode "decode", the exact decode followed by F.linear,
the reference module's numerics, pack_to_disk.py:193-218).  The reference's
non-resident variant (pinned host streams copied per forward,
pack_to_disk.py:140-175) is the offload path for 24 GB cards and is not
built: it raises.
"""
from __future__ import annotations

import dataclasses
import gc
import json
import os
import time

import torch
from torch import nn

from . import ops
from .codec import Bf16xPlan, bf16x_quantize, build_plan_host, stream_words

KIND = "bf16x-v1"
_DEFAULT_SKIP = ("embed", "lm_head")
_STREAM_BITS = (("sign", 1), ("mant", 7), ("delta", 3))
_STREAM_FIELDS = (("sign", "sign_packed"), ("mant", "mant_packed"), ("delta", "delta_packed"))

__all__ = ["KIND", "LinearRecord", "pack_model_to_disk", "pack_linear", "load_meta", "Bf16xStreamLinear",
           "replace_linears_from_packed"]


@dataclasses.dataclass
class LinearRecord:
    """One packed linear as it goes to disk: the bf16x-v1 arrays in file
    order, the meta fields and the optional bias (bf16)."""
    name: str
    arrays: dict
    out_f: int
    in_f: int
    n_fix: int
    bias: torch.Tensor | None = None

    def meta(self, keys: dict) -> dict:
        m = dict(keys)
        m.update(out_f=self.out_f, in_f=self.in_f, N=self.out_f * self.in_f, n_fix=self.n_fix)
        return m


def _with_zero_word(words: torch.Tensor) -> torch.Tensor:
    """A stream with the format's trailing zero word."""
    out = torch.zeros(words.numel() + 1, dtype=words.dtype)
    out[:-1] = words
    return out


def pack_linear(w: torch.Tensor, sub: int = 16) -> dict:
    """One weight [out_f, in_f] -> the six on-disk arrays of bf16x-v1
    (CPU tensors) and its meta fields."""
    p = bf16x_quantize(w.detach().to(torch.bfloat16).cpu(), sub=sub)
    needed = p["delta_ovf_val"] > 7             # delta == 7 decodes exactly from the 3-bit code
    arrays = {key: _with_zero_word(p[field]) for key, field in _STREAM_FIELDS}
    arrays["emax"] = p["emax"]
    arrays["ovf_i"] = p["delta_ovf_idx"][needed].to(torch.int64).contiguous()
    arrays["ovf_v"] = p["delta_ovf_val"][needed].to(torch.int32).contiguous()
    out_f, in_f = int(p["out_f"]), int(p["in_f"])
    return {"arrays": arrays, "out_f": out_f, "in_f": in_f, "N": out_f * in_f, "n_fix": int(needed.sum())}


def _record(name: str, linear: nn.Linear, sub: int) -> LinearRecord:
    pk = pack_linear(linear.weight.data, sub=sub)
    bias = linear.bias.data.detach().to(torch.bfloat16).cpu().contiguous() if linear.bias is not None else None
    return LinearRecord(name, pk["arrays"], pk["out_f"], pk["in_f"], pk["n_fix"], bias)


def _packable(model: nn.Module, min_numel: int, skip) -> list:
    """(name, module) of the linears to pack, in module order."""
    return [(name, mod) for name, mod in model.named_modules()
            if isinstance(mod, nn.Linear) and mod.weight.numel() >= min_numel
            and not any(s in name for s in skip)]


class _BlobWriter:
    """Collects records into one safetensors dict and the meta table; the key
    of array k of linear n is "n.k"."""

    def __init__(self):
        self.tensors: dict = {}
        self.table: dict = {}
        self.nbytes = 0

    def _put(self, key: str, t: torch.Tensor) -> str:
        self.tensors[key] = t
        self.nbytes += t.numel() * t.element_size()
        return key

    def add(self, rec: LinearRecord):
        keys = {k: self._put(f"{rec.name}.{k}", t) for k, t in rec.arrays.items()}
        if rec.bias is not None:
            keys["bias"] = self._put(f"{rec.name}.bias", rec.bias)
        self.table[rec.name] = rec.meta(keys)

    def write(self, out_prefix: str) -> tuple:
        from safetensors.torch import save_file
        path = out_prefix + ".safetensors"
        save_file(self.tensors, path, metadata={"format": "bf16x"})
        with open(out_prefix + ".meta.json", "w") as f:
            json.dump({"kind": KIND, "tensors": self.table}, f)
        return path, os.path.getsize(path)


@torch.no_grad()
def pack_model_to_disk(model, out_prefix, min_numel=4096, sub=16, skip=_DEFAULT_SKIP, verbose=True):
    """Pack every nn.Linear (numel >= min_numel, name containing none of
    `skip`) into <out_prefix>.safetensors + <out_prefix>.meta.json; each
    original weight (and bias) is released as soon as it is packed, so the
    host holds at most one unpacked layer beside the packed ones
    (pack_to_disk.py:40-105).  Returns (n_packed, packed_bytes)."""
    writer = _BlobWriter()
    start = time.time()
    chosen = _packable(model, min_numel, skip)
    for i, (name, lin) in enumerate(chosen, 1):
        writer.add(_record(name, lin, sub))
        lin.weight.data = torch.empty(0)
        if lin.bias is not None:
            lin.bias.data = torch.empty(0)
        if verbose and i % 50 == 0:
            print(f"[bf16x-v1] packed {i}/{len(chosen)} linears ({writer.nbytes / 1e9:.2f} GB) "
                  f"after {time.time() - start:.0f} s", flush=True)
    path, size = writer.write(out_prefix)
    if verbose:
        print(f"[bf16x-v1] wrote {path}: {len(chosen)} linears, {size / 1e9:.2f} GB", flush=True)
    gc.collect()
    return len(chosen), writer.nbytes


def load_meta(out_prefix) -> dict:
    """The `tensors` table of <out_prefix>.meta.json (kind must be bf16x-v1)."""
    with open(out_prefix + ".meta.json") as f:
        meta = json.load(f)
    if meta.get("kind") != KIND:
        raise ValueError(f"{out_prefix}.meta.json: kind {meta.get('kind')!r}, expected {KIND!r}")
    return meta["tensors"]


def _check_entry(name: str, entry: dict, blob: dict):
    """The arrays of one linear agree with the shape its entry claims."""
    out_f, in_f = int(entry["out_f"]), int(entry["in_f"])
    n = out_f * in_f
    if int(entry.get("N", n)) != n or out_f <= 0 or in_f <= 0:
        raise ValueError(f"{name}: N={entry.get('N')} does not match out_f x in_f = {out_f}x{in_f}")
    for key, bits in _STREAM_BITS:
        t = blob[key]
        if t.dtype != torch.int32 or t.dim() != 1 or t.numel() < stream_words(n, bits):
            raise ValueError(f"{name}.{key}: int32 stream of >= {stream_words(n, bits)} words expected, "
                             f"got {t.dtype} {tuple(t.shape)}")
    e = blob["emax"]
    if e.dtype != torch.uint8 or e.numel() < (n + 15) // 16:
        raise ValueError(f"{name}.emax: uint8 [{(n + 15) // 16}] expected, got {e.dtype} {tuple(e.shape)}")
    oi, ov = blob.get("ovf_i"), blob.get("ovf_v")
    n_fix = int(entry.get("n_fix", 0))
    if n_fix:
        if oi is None or ov is None or oi.numel() != n_fix or ov.numel() != n_fix:
            raise ValueError(f"{name}: n_fix = {n_fix} but the table holds "
                             f"{None if oi is None else oi.numel()} / {None if ov is None else ov.numel()}")
        if int(oi.min()) < 0 or int(oi.max()) >= n or n > 2 ** 31 - 1:
            raise ValueError(f"{name}.ovf_i: positions outside [0, {n})")
        if bool((oi[1:] <= oi[:-1]).any()):
            raise ValueError(f"{name}.ovf_i: positions not strictly increasing")
        if int(ov.min()) <= 7 or int(ov.max()) > 255:
            raise ValueError(f"{name}.ovf_v: true deltas must be in (7, 255]")


class Bf16xStreamLinear(nn.Module):
    """Exact BF16X linear fed from a bf16x-v1 blob (pack_to_disk.py:108-218).

    mode "fused" (default): fused decode+GEMV for one token, the exact
    decode+GEMM dispatch otherwise; mode "decode": exact decode into a
    buffer shared per device, then F.linear (the reference module's two
    steps).  Both use the lossless weight.  Built from one meta entry and its
    arrays (checked first), with the streams moved to `device` once."""

    def __init__(self, entry: dict, blob: dict, device=None, name: str = "?"):
        super().__init__()
        _check_entry(name, entry, blob)
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.out_features, self.in_features = int(entry["out_f"]), int(entry["in_f"])
        self.N = self.out_features * self.in_features
        self.n_fix = int(entry.get("n_fix", 0))
        self.resident = True
        self.mode = "fused"
        self.gpu = {k: blob[k].contiguous().to(dev) for k in ("sign", "mant", "delta", "emax")}
        self.plan: Bf16xPlan = build_plan_host(self._host_dict(blob), device=dev)
        b = blob.get("bias")
        self.bias = b.to(dev, torch.bfloat16) if b is not None else None

    def _host_dict(self, blob: dict) -> dict:
        """The packed dict the plan builder reads: the file's table (entries
        with true delta > 7) in the dict's dtypes."""
        table = (blob["ovf_i"].to(torch.int32), blob["ovf_v"].to(torch.uint8)) if self.n_fix else \
            (torch.zeros(0, dtype=torch.int32), torch.zeros(0, dtype=torch.uint8))
        d = {field: blob[key] for key, field in _STREAM_FIELDS}
        d.update(emax=blob["emax"], delta_ovf_idx=table[0], delta_ovf_val=table[1], out_f=self.out_features,
                 in_f=self.in_features, sub=16)
        return d

    @classmethod
    def from_packed(cls, entry: dict, blob: dict, resident: bool = True, device=None, name: str = "?"):
        """The reference's constructor (pack_to_disk.py:108-140): only the
        resident variant exists here."""
        if not resident:
            raise NotImplementedError("the non-resident (pinned host, per-call copy) variant is not built: "
                                      "keep the streams resident on the GPU")
        return cls(entry, blob, device=device, name=name)

    def decoded_weight(self) -> torch.Tensor:
        g = self.gpu
        return ops.bf16x_decode(g["sign"], g["mant"], g["delta"], g["emax"], self.out_features, self.in_features,
                                plan=self.plan)

    def forward(self, x):
        if not x.is_cuda:
            raise ValueError("Bf16xStreamLinear runs on the GPU only: move the input to the module's device")
        g = self.gpu
        b = self.bias.to(x.dtype) if self.bias is not None else None
        if self.mode == "decode":
            from .nn import _shared_dec_buf
            w = ops.bf16x_decode(g["sign"], g["mant"], g["delta"], g["emax"], self.out_features, self.in_features,
                                 plan=self.plan, out=_shared_dec_buf(self.N, x.device)[: self.N])
            return torch.nn.functional.linear(x, w.view(self.out_features, self.in_features).to(x.dtype), b)
        if x.numel() == self.in_features:
            y = ops.bf16x_gemv(x, g["sign"], g["mant"], g["delta"], g["emax"], self.out_features,
                               self.in_features, plan=self.plan).view(*x.shape[:-1], self.out_features)
        else:
            y = ops.bf16x_gemm(x, g["sign"], g["mant"], g["delta"], g["emax"], self.out_features,
                               self.in_features, plan=self.plan)
        return y if b is None else y + b.to(y.dtype)


_ARRAY_KEYS = ("sign", "mant", "delta", "emax", "ovf_i", "ovf_v", "bias")


def _install(model: nn.Module, name: str, module: nn.Module):
    """Put `module` at the dotted path `name` of `model`."""
    parent_name, _, leaf = name.rpartition(".")
    setattr(model.get_submodule(parent_name) if parent_name else model, leaf, module)


@torch.no_grad()
def replace_linears_from_packed(model, out_prefix, resident_fn=None, keep_rest_bf16=True, verbose=True,
                                device=None):
    """Swap every packed nn.Linear of `model` for Bf16xStreamLinear
    (memory-mapped read, no re-quantization; pack_to_disk.py:221-265).
    resident_fn(name) -> bool selects GPU residency (only True is
    supported); other Linears become bf16 when keep_rest_bf16.  The model
    is moved to the GPU.  Returns the number replaced."""
    from safetensors import safe_open

    table = load_meta(out_prefix)
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    start = time.time()
    linears = [(name, mod) for name, mod in model.named_modules() if isinstance(mod, nn.Linear)]
    replaced = 0
    with safe_open(out_prefix + ".safetensors", framework="pt", device="cpu") as sf:
        for name, lin in linears:
            entry = table.get(name)
            if entry is None:
                if keep_rest_bf16:
                    lin.weight.data = lin.weight.data.to(torch.bfloat16)
                continue
            arrays = {k: sf.get_tensor(entry[k]) for k in _ARRAY_KEYS if entry.get(k)}
            resident = resident_fn(name) if resident_fn is not None else True
            _install(model, name, Bf16xStreamLinear.from_packed(entry, arrays, resident=resident, device=dev,
                                                                name=name))
            lin.weight.data = torch.empty(0)
            replaced += 1
    model.to(dev)
    if verbose:
        print(f"[bf16x-v1] loaded {replaced} linears from {out_prefix}.safetensors in "
              f"{time.time() - start:.1f} s, streams resident on {dev}", flush=True)
    return replaced

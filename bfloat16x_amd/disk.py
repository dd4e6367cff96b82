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

__all__ = ["KIND", "pack_model_to_disk", "pack_linear", "load_meta", "Bf16xStreamLinear",
           "replace_linears_from_packed"]


def _pad1(t: torch.Tensor) -> torch.Tensor:
    return torch.cat([t, torch.zeros(1, dtype=t.dtype)])


def pack_linear(w: torch.Tensor, sub: int = 16) -> dict:
    """One weight [out_f, in_f] -> the six on-disk arrays of bf16x-v1
    (CPU tensors) and its meta fields."""
    p = bf16x_quantize(w.detach().to(torch.bfloat16).cpu(), sub=sub)
    oi = p["delta_ovf_idx"].to(torch.int64)
    ov = p["delta_ovf_val"].to(torch.int64)
    keep = ov > 7
    oi, ov = oi[keep], ov[keep]
    arrays = {"sign": _pad1(p["sign_packed"]), "mant": _pad1(p["mant_packed"]),
              "delta": _pad1(p["delta_packed"]), "emax": p["emax"],
              "ovf_i": oi.contiguous(), "ovf_v": ov.to(torch.int32).contiguous()}
    out_f, in_f = int(p["out_f"]), int(p["in_f"])
    return {"arrays": arrays, "out_f": out_f, "in_f": in_f, "N": out_f * in_f, "n_fix": int(oi.numel())}


@torch.no_grad()
def pack_model_to_disk(model, out_prefix, min_numel=4096, sub=16, skip=_DEFAULT_SKIP, verbose=True):
    """Pack every nn.Linear (numel >= min_numel, name containing none of
    `skip`) into <out_prefix>.safetensors + <out_prefix>.meta.json; each
    original weight (and bias) is dropped once packed (pack_to_disk.py:40-105).
    Returns (n_packed, packed_bytes)."""
    from safetensors.torch import save_file

    blobs = {}
    meta = {"kind": KIND, "tensors": {}}
    total, n = 0, 0
    t0 = time.time()
    for name, mod in list(model.named_modules()):
        if not isinstance(mod, nn.Linear):
            continue
        if mod.weight.numel() < min_numel or any(s in name for s in skip):
            continue
        pk = pack_linear(mod.weight.data, sub=sub)
        m = {}
        for key, val in pk["arrays"].items():
            gk = f"{name}.{key}"
            blobs[gk] = val
            total += val.numel() * val.element_size()
            m[key] = gk
        m["out_f"], m["in_f"], m["N"], m["n_fix"] = pk["out_f"], pk["in_f"], pk["N"], pk["n_fix"]
        if mod.bias is not None:
            gk = f"{name}.bias"
            blobs[gk] = mod.bias.data.detach().to(torch.bfloat16).cpu().contiguous()
            total += blobs[gk].numel() * blobs[gk].element_size()
            m["bias"] = gk
            mod.bias.data = torch.empty(0)
        meta["tensors"][name] = m
        mod.weight.data = torch.empty(0)
        del pk
        n += 1
        if verbose and n % 50 == 0:
            print(f"  {n} packed, blob {total / 1e9:.1f}GB, {time.time() - t0:.0f}s", flush=True)
    pack_path, meta_path = out_prefix + ".safetensors", out_prefix + ".meta.json"
    save_file(blobs, pack_path, metadata={"format": "bf16x"})
    with open(meta_path, "w") as f:
        json.dump(meta, f)
    if verbose:
        print(f"  -> {pack_path} ({os.path.getsize(pack_path) / 1e9:.2f}GB, {n} linears)", flush=True)
    gc.collect()
    return n, total


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
    steps).  Both use the lossless weight."""

    def __init__(self):
        super().__init__()
        raise RuntimeError("use from_packed()")

    @classmethod
    def from_packed(cls, entry: dict, blob: dict, resident: bool = True, device=None, name: str = "?"):
        if not resident:
            raise NotImplementedError("the non-resident (pinned host, per-call copy) variant is not built: "
                                      "keep the streams resident on the GPU")
        _check_entry(name, entry, blob)
        obj = cls.__new__(cls)
        nn.Module.__init__(obj)
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        obj.out_features, obj.in_features = int(entry["out_f"]), int(entry["in_f"])
        obj.N = int(entry["N"])
        obj.n_fix = int(entry.get("n_fix", 0))
        obj.resident = True
        obj.mode = "fused"
        obj.gpu = {k: blob[k].contiguous().to(dev) for k in ("sign", "mant", "delta", "emax")}
        host = {"sign_packed": blob["sign"], "mant_packed": blob["mant"], "delta_packed": blob["delta"],
                "emax": blob["emax"], "out_f": obj.out_features, "in_f": obj.in_features, "sub": 16}
        if obj.n_fix:
            host["delta_ovf_idx"] = blob["ovf_i"].to(torch.int32)
            host["delta_ovf_val"] = blob["ovf_v"].to(torch.uint8)
        else:
            host["delta_ovf_idx"] = torch.zeros(0, dtype=torch.int32)
            host["delta_ovf_val"] = torch.zeros(0, dtype=torch.uint8)
        obj.plan: Bf16xPlan = build_plan_host(host, device=dev)
        b = blob.get("bias")
        obj.bias = b.to(dev, torch.bfloat16) if b is not None else None
        return obj

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


@torch.no_grad()
def replace_linears_from_packed(model, out_prefix, resident_fn=None, keep_rest_bf16=True, verbose=True,
                                device=None):
    """Swap every packed nn.Linear of `model` for Bf16xStreamLinear
    (memory-mapped read, no re-quantization; pack_to_disk.py:221-265).
    resident_fn(name) -> bool selects GPU residency (only True is
    supported); other Linears become bf16 when keep_rest_bf16.  The model
    is moved to the GPU.  Returns the number replaced."""
    from safetensors import safe_open

    meta = load_meta(out_prefix)
    n = 0
    t0 = time.time()
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    with safe_open(out_prefix + ".safetensors", framework="pt", device="cpu") as sf:
        for name, mod in list(model.named_modules()):
            if not isinstance(mod, nn.Linear):
                continue
            if name in meta:
                entry = meta[name]
                blob = {k: sf.get_tensor(entry[k]) for k in ("sign", "mant", "delta", "emax", "ovf_i", "ovf_v",
                                                              "bias") if entry.get(k)}
                res = resident_fn(name) if resident_fn else True
                new = Bf16xStreamLinear.from_packed(entry, blob, resident=res, device=dev, name=name)
                parent = model
                parts = name.split(".")
                for q in parts[:-1]:
                    parent = getattr(parent, q)
                setattr(parent, parts[-1], new)
                mod.weight.data = torch.empty(0)
                n += 1
                del blob
            elif keep_rest_bf16:
                mod.weight.data = mod.weight.data.to(torch.bfloat16)
    model.to(dev)
    if verbose:
        print(f"[bf16x] {n} linears from disk in {time.time() - t0:.1f}s (resident)", flush=True)
    return n

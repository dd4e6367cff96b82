"""CPU tests of the bf16x-v1 writer and loader checks (pack_to_disk.py):
file layout, key names, dtypes and padding as the reference writes them;
the streams byte-identical to the oracle encoder; the on-disk table decodes
(two-segment, as the reference module does) to the original bf16 bits; and
malformed entries rejected before any device work."""
import copy
import json

import numpy as np
import pytest
import torch
from torch import nn

from oracle import dict_codec as dc

from bfloat16x_amd import disk
from bfloat16x_amd.codec import stream_words


class Tiny(nn.Module):
    def __init__(self):
        super().__init__()
        g = torch.Generator().manual_seed(0)
        self.embed = nn.Embedding(100, 64)
        self.up = nn.Linear(64, 192)
        self.down = nn.Linear(192, 64, bias=False)
        self.small = nn.Linear(16, 16)
        self.lm_head = nn.Linear(64, 100, bias=False)
        for p in self.parameters():
            p.data = torch.randn(p.shape, generator=g) * 0.02
        with torch.no_grad():                         # outliers: entries with true delta > 7
            for w in (self.up.weight, self.down.weight):
                w.view(-1)[torch.randperm(w.numel(), generator=g)[: w.numel() // 50]] *= 300.0


@pytest.fixture(scope="module")
def packed(tmp_path_factory):
    model = Tiny()
    orig = copy.deepcopy(model)
    prefix = str(tmp_path_factory.mktemp("bf16x") / "tiny")
    n, total = disk.pack_model_to_disk(model, prefix, min_numel=4096, verbose=False)
    return model, orig, prefix, n, total


def test_layout_and_keys(packed):
    from safetensors import safe_open
    model, orig, prefix, n, total = packed
    assert n == 2
    meta = json.load(open(prefix + ".meta.json"))
    assert meta["kind"] == "bf16x-v1" and set(meta["tensors"]) == {"up", "down"}
    with safe_open(prefix + ".safetensors", framework="pt") as sf:
        assert sf.metadata() == {"format": "bf16x"}
        keys = set(sf.keys())
        assert keys == {f"{nm}.{k}" for nm in ("up", "down") for k in ("sign", "mant", "delta", "emax", "ovf_i",
                                                                     "ovf_v")} | {"up.bias"}
        nbytes = 0
        for nm, lin in (("up", orig.up), ("down", orig.down)):
            e = meta["tensors"][nm]
            N = lin.weight.numel()
            assert (e["out_f"], e["in_f"], e["N"]) == (lin.out_features, lin.in_features, N)
            for key, bits in (("sign", 1), ("mant", 7), ("delta", 3)):
                t = sf.get_tensor(e[key])
                assert t.dtype == torch.int32 and t.numel() == stream_words(N, bits) + 1 and int(t[-1]) == 0
            assert sf.get_tensor(e["emax"]).dtype == torch.uint8
            oi, ov = sf.get_tensor(e["ovf_i"]), sf.get_tensor(e["ovf_v"])
            assert oi.dtype == torch.int64 and ov.dtype == torch.int32
            assert e["n_fix"] == oi.numel() > 0 and bool((ov > 7).all()) and bool((oi[1:] > oi[:-1]).all())
            nbytes += sum(sf.get_tensor(e[k]).numel() * sf.get_tensor(e[k]).element_size()
                          for k in ("sign", "mant", "delta", "emax", "ovf_i", "ovf_v"))
        b = sf.get_tensor("up.bias")
        assert b.dtype == torch.bfloat16 and torch.equal(b, orig.up.bias.data.to(torch.bfloat16))
        nbytes += b.numel() * 2
    assert total == nbytes
    # originals dropped, others untouched
    assert model.up.weight.numel() == 0 and model.down.weight.numel() == 0 and model.up.bias.numel() == 0
    assert torch.equal(model.small.weight, orig.small.weight) and torch.equal(model.lm_head.weight,
                                                                              orig.lm_head.weight)


def test_streams_match_oracle_and_decode_exactly(packed):
    from safetensors import safe_open
    _, orig, prefix, _, _ = packed
    meta = disk.load_meta(prefix)
    with safe_open(prefix + ".safetensors", framework="pt") as sf:
        for nm, lin in (("up", orig.up), ("down", orig.down)):
            e = meta[nm]
            bits = lin.weight.data.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
            ref = dc.quantize(bits)
            got = {k: sf.get_tensor(e[k]).numpy() for k in ("sign", "mant", "delta", "emax", "ovf_i", "ovf_v")}
            assert np.array_equal(got["sign"][:-1], ref["sign_packed"])
            assert np.array_equal(got["mant"][:-1], ref["mant_packed"])
            assert np.array_equal(got["delta"][:-1], ref["delta_packed"])
            assert np.array_equal(got["emax"], ref["emax"])
            keep = ref["delta_ovf_val"] > 7
            assert np.array_equal(got["ovf_i"], ref["delta_ovf_idx"][keep].astype(np.int64))
            assert np.array_equal(got["ovf_v"], ref["delta_ovf_val"][keep].astype(np.int32))
            d = dict(sign_packed=got["sign"], mant_packed=got["mant"], delta_packed=got["delta"],
                     emax=got["emax"], delta_ovf_idx=got["ovf_i"], delta_ovf_val=got["ovf_v"],
                     out_f=e["out_f"], in_f=e["in_f"], sub=16)
            assert np.array_equal(dc.decode_two_segment(d), bits)


def _blob(prefix, name):
    from safetensors import safe_open
    e = disk.load_meta(prefix)[name]
    with safe_open(prefix + ".safetensors", framework="pt") as sf:
        return e, {k: sf.get_tensor(e[k]) for k in ("sign", "mant", "delta", "emax", "ovf_i", "ovf_v")}


def test_entry_checks_reject_malformed(packed):
    _, _, prefix, _, _ = packed
    e, b = _blob(prefix, "down")
    disk._check_entry("down", e, b)                       # well formed
    cases = [
        (dict(e, n_fix=e["n_fix"] + 1), b),
        (dict(e, N=e["N"] + 1), b),
        (e, dict(b, mant=b["mant"][:10])),
        (e, dict(b, sign=b["sign"].to(torch.int64))),
        (e, dict(b, emax=b["emax"][:3])),
        (e, dict(b, ovf_i=b["ovf_i"].flip(0))),
        (e, dict(b, ovf_v=torch.full_like(b["ovf_v"], 7))),
        (e, dict(b, ovf_i=b["ovf_i"] + e["N"])),
    ]
    for ee, bb in cases:
        with pytest.raises(ValueError):
            disk._check_entry("down", ee, bb)


def test_load_meta_rejects_other_kinds(tmp_path):
    p = str(tmp_path / "x")
    json.dump({"kind": "bf16x-v0", "tensors": {}}, open(p + ".meta.json", "w"))
    with pytest.raises(ValueError):
        disk.load_meta(p)


def test_non_resident_is_refused(packed):
    _, _, prefix, _, _ = packed
    e, b = _blob(prefix, "down")
    with pytest.raises(NotImplementedError):
        disk.Bf16xStreamLinear.from_packed(e, b, resident=False)

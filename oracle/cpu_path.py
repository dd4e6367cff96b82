"""The reference's CPU decode+matmul path, restated -- test/benchmark infrastructure only.

This is the timed CPU baseline: ``BF16XLinear`` of opqk_linear.py:327-404
run on host tensors.  It follows the reference algorithm step by step:

* ``_unpack`` -- opqk_linear.py:67-77: expand the covered words to one int64
  per bit (``(w >> arange(32)) & 1``), slice, regroup by ``b`` and sum the
  shifted bits;
* ``decode_tile`` -- opqk_linear.py:360-377: unpack the 7/3/1-bit fields of a
  tile of rows, substitute table deltas where the code is 7 via
  ``searchsorted`` over the whole table (:367-372), gather emax per 16
  elements (:373-374), exponent (emax - d) & 0xFF (:375), assemble the bits;
* ``forward`` -- opqk_linear.py:390-404: decode 1024-row tiles and
  ``torch.matmul(x, w_tile.t())`` each, concatenate, add the bias.

It is written here in torch on the CPU (the reference's own library), not
imported from the reference.
"""
from __future__ import annotations

import torch


def _unpack(words: torch.Tensor, bit_start: int, nbits: int, b: int) -> torch.Tensor:
    ws = bit_start // 32
    sk = bit_start % 32
    we = (bit_start + nbits + 31) // 32
    sw = words[ws:we].to(torch.int64)
    bits = (sw.unsqueeze(-1) >> torch.arange(32)) & 1
    bits = bits.reshape(-1)[sk:sk + nbits]
    return ((bits.reshape(-1, b) << torch.arange(b, dtype=torch.int64)).sum(-1)).to(torch.int32)


class CpuBf16xLinear:
    """Host-tensor BF16XLinear restatement (decode tiles + matmul)."""

    def __init__(self, packed: dict, tile: int = 1024, sub: int = 16, bias=None):
        self.out_f = int(packed["out_f"])
        self.in_f = int(packed["in_f"])
        self.tile = tile
        self.sub = sub
        self.bias = bias
        t = {}
        for k in ("emax", "sign_packed", "mant_packed", "delta_packed",
                  "delta_ovf_idx", "delta_ovf_val"):
            v = packed[k]
            t[k] = v if isinstance(v, torch.Tensor) else torch.from_numpy(v)
        self.emax = t["emax"]
        self.sign_packed = t["sign_packed"]
        self.mant_packed = t["mant_packed"]
        self.delta_packed = t["delta_packed"]
        self.ovf_idx = t["delta_ovf_idx"]
        self.ovf_val = t["delta_ovf_val"]

    def decode_tile(self, s: int, e: int) -> torch.Tensor:
        fs = s * self.in_f
        nv = (e - s) * self.in_f
        mant = _unpack(self.mant_packed, fs * 7, nv * 7, 7)
        d = _unpack(self.delta_packed, fs * 3, nv * 3, 3)
        sgn = _unpack(self.sign_packed, fs, nv, 1)
        ovf = d == 7
        if bool(ovf.any()) and self.ovf_idx.numel() > 0:
            pos = torch.arange(fs, fs + nv)
            loc = torch.searchsorted(self.ovf_idx.to(torch.int64), pos)
            loc = loc.clamp(max=self.ovf_idx.numel() - 1)
            d = torch.where(ovf, self.ovf_val.to(torch.int32)[loc], d)
        sub = torch.arange(fs, fs + nv) // self.sub
        emax = self.emax.to(torch.int32)[sub]
        expo = (emax - d) & 0xFF
        vbits = (sgn << 15) | (expo << 7) | (mant & 0x7F)
        return vbits.to(torch.int16).view(torch.bfloat16).reshape(e - s, self.in_f)

    def decode_to_bf16(self) -> torch.Tensor:
        return torch.cat([self.decode_tile(s, min(s + self.tile, self.out_f))
                          for s in range(0, self.out_f, self.tile)], dim=0)

    def forward(self, x: torch.Tensor, rows=None) -> torch.Tensor:
        """Decode+matmul over all rows, or only over the first ``rows`` rows
        (a bounded sample for timing)."""
        n_rows = self.out_f if rows is None else min(rows, self.out_f)
        xf = x.reshape(-1, self.in_f)
        outs = []
        for i in range(0, n_rows, self.tile):
            end = min(i + self.tile, n_rows)
            w_tile = self.decode_tile(i, end)
            outs.append(torch.matmul(xf, w_tile.t()))
            del w_tile
        out = torch.cat(outs, dim=-1).reshape(*x.shape[:-1], n_rows)
        if self.bias is not None and rows is None:
            out = out + self.bias
        return out

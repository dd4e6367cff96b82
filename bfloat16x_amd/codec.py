"""Packed-dict encoder and overflow plans.

``bf16x_quantize`` mirrors opqk_linear.py:291-324 (same name, arguments and
output dict, byte-identical fields) but runs the multi-threaded C++ encoder
of libbf16x_hip.so.

A ``Bf16xPlan`` is the device-resident form of the overflow table the HIP
kernels consume: the entries whose true delta exceeds 7, grouped per tile
(one row, or a 65536-column segment of a row), each entry 4 bytes
``(column << 16) | exact bf16 bits``.  It replaces the reference's per-row
CSR (bf16x_fused.py:165-182) and its per-call filtered H2D copy
(bf16x_triton_test.py:96-100).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib

SUB = 16
DICT_KEYS = ("emax", "sign_packed", "mant_packed", "delta_packed", "delta_ovf_idx", "delta_ovf_val")


def stream_words(n: int, bits: int) -> int:
    """Words of the reference packer for n values of `bits` bits (opqk_linear.py:53-64)."""
    return int(_lib.lib().bf16x_stream_words(int(n), int(bits)))


def _bf16_bits_host(w: torch.Tensor) -> torch.Tensor:
    b16 = w.detach().to(torch.bfloat16)          # round-to-nearest-even, as the reference (:298)
    return b16.reshape(-1).cpu().contiguous().view(torch.int16)


def _quantize_device(w: torch.Tensor) -> dict:
    """The device encoder (bf16x_encode): outputs on w's GPU."""
    out_f, in_f = (int(s) for s in w.shape)
    n = out_f * in_f
    dev = w.device
    bits = w.detach().to(torch.bfloat16).contiguous()
    if bits.data_ptr() % 16:
        bits = bits.clone()
    L = _lib.lib()
    i32 = dict(dtype=torch.int32, device=dev)
    sign = torch.empty(stream_words(n, 1), **i32)
    mant = torch.empty(stream_words(n, 7), **i32)
    delta = torch.empty(stream_words(n, 3), **i32)
    emax = torch.empty((n + SUB - 1) // SUB, dtype=torch.uint8, device=dev)
    ws = torch.empty((int(L.bf16x_encode_workspace(out_f, in_f)) + 15) // 16 * 4, **i32)
    n_ovf = torch.zeros(1, dtype=torch.int64, device=dev)
    cap = max(1, n // 8)
    stream = _lib.stream_of(dev)
    for _ in range(2):
        idx = torch.empty(cap, **i32)
        val = torch.empty(cap, dtype=torch.uint8, device=dev)
        st = L.bf16x_encode(bits.data_ptr(), out_f, in_f, SUB, sign.data_ptr(), sign.numel(), mant.data_ptr(),
                            mant.numel(), delta.data_ptr(), delta.numel(), emax.data_ptr(), emax.numel(),
                            idx.data_ptr(), val.data_ptr(), cap, n_ovf.data_ptr(), ws.data_ptr(),
                            ws.numel() * 4, stream)
        _lib.check(st, "bf16x_encode")
        k = int(n_ovf.item())
        if k <= cap:
            break
        cap = k
    return dict(emax=emax, sign_packed=sign, mant_packed=mant, delta_packed=delta,
                delta_ovf_idx=idx[:k].clone(), delta_ovf_val=val[:k].clone(),
                out_f=out_f, in_f=in_f, sub=SUB)


def bf16x_quantize(w: torch.Tensor, sub: int = SUB, n_threads: int = 0) -> dict:
    """bf16 weight [out_f, in_f] -> packed dict (opqk_linear.py:291).

    Keys: emax (uint8), sign_packed / mant_packed / delta_packed (int32 word
    streams), delta_ovf_idx (int32), delta_ovf_val (uint8), out_f, in_f, sub.
    A GPU weight is encoded on its GPU (sub = 16) and the dict's tensors stay
    there, as the reference's torch encoder does on a CUDA tensor; a CPU
    weight (or another sub) is encoded by the multi-threaded host encoder.
    Both give the same bytes.
    """
    if w.dim() != 2:
        raise ValueError("bf16x_quantize expects a 2-D weight [out_f, in_f]")
    if w.is_cuda and int(sub) == SUB and w.numel() <= 2 ** 31 - 1:
        return _quantize_device(w)
    out_f, in_f = (int(s) for s in w.shape)
    n = out_f * in_f
    bits = _bf16_bits_host(w)
    sign = torch.empty(stream_words(n, 1), dtype=torch.int32)
    mant = torch.empty(stream_words(n, 7), dtype=torch.int32)
    delta = torch.empty(stream_words(n, 3), dtype=torch.int32)
    emax = torch.empty((n + sub - 1) // sub, dtype=torch.uint8)
    cap = max(1, n // 16)
    for _ in range(2):
        idx = torch.empty(cap, dtype=torch.int32)
        val = torch.empty(cap, dtype=torch.uint8)
        n_ovf = ctypes.c_int64(0)
        st = _lib.lib().bf16x_encode_host(bits.data_ptr(), out_f, in_f, int(sub), sign.data_ptr(),
                                          mant.data_ptr(), delta.data_ptr(), emax.data_ptr(),
                                          idx.data_ptr(), val.data_ptr(), cap, ctypes.byref(n_ovf),
                                          int(n_threads))
        if st == _lib.ECAPACITY:
            cap = int(n_ovf.value)
            continue
        _lib.check(st, "bf16x_encode_host")
        break
    k = int(n_ovf.value)
    return dict(emax=emax, sign_packed=sign, mant_packed=mant, delta_packed=delta,
                delta_ovf_idx=idx[:k].clone(), delta_ovf_val=val[:k].clone(),
                out_f=out_f, in_f=in_f, sub=int(sub))


@dataclass
class Bf16xPlan:
    """Device overflow plan: tile_off uint32 [n_tiles+1], tile_ent uint32 [n_fix]
    ((column << 16) | exact bits), tile_sat uint8 [n_fix] (max(emax - 7, 0)).
    kp_off / kp_ent: the step-major regrouping used by the GEMM, built on the
    device on first use (see kplan()); cp_off / cp_ent: the chunk plan of the
    few-row GEMM (see cplan())."""
    tile_off: torch.Tensor
    tile_ent: torch.Tensor
    tile_sat: torch.Tensor
    n_fix: int
    out_f: int
    in_f: int
    kp_off: torch.Tensor | None = None
    kp_ent: torch.Tensor | None = None
    cp_off: torch.Tensor | None = None
    cp_ent: torch.Tensor | None = None

    @property
    def nbytes(self) -> int:
        n = self.tile_off.numel() * 4 + self.tile_ent.numel() * 4 + self.tile_sat.numel()
        if self.kp_off is not None:
            n += self.kp_off.numel() * 4 + self.kp_ent.numel() * 4
        if self.cp_off is not None:
            n += self.cp_off.numel() * 4 + self.cp_ent.numel() * 4
        return n

    def kplan(self):
        """(kp_off, kp_ent) on the plan's device, built once by bf16x_kplan_build."""
        if self.kp_off is None:
            dev = self.tile_off.device
            if not self.tile_off.is_cuda:
                raise ValueError("kplan(): the plan must live on the GPU")
            size = int(_lib.lib().bf16x_kplan_size(self.out_f, self.in_f))
            kp_off = torch.empty(max(size, 1), dtype=torch.int32, device=dev)
            kp_ent = torch.zeros(max(self.n_fix, 1), dtype=torch.int32, device=dev)
            st = _lib.lib().bf16x_kplan_build(self.tile_off.data_ptr(), self.tile_ent.data_ptr(), self.out_f,
                                              self.in_f, kp_off.data_ptr(), kp_ent.data_ptr(), _lib.stream_of(dev))
            _lib.check(st, "bf16x_kplan_build")
            self.kp_off, self.kp_ent = kp_off, kp_ent
        return self.kp_off, self.kp_ent

    def cplan(self):
        """(cp_off, cp_ent) on the plan's device, built once by
        bf16x_cplan_build: the entries regrouped by (256-column chunk, row)
        for the chunked few-row GEMM."""
        if self.cp_off is None:
            dev = self.tile_off.device
            if not self.tile_off.is_cuda:
                raise ValueError("cplan(): the plan must live on the GPU")
            size = int(_lib.lib().bf16x_cplan_size(self.out_f, self.in_f))
            if size < 0:
                raise _lib.Bf16xError(size, "bf16x_cplan_size")
            cp_off = torch.empty(size, dtype=torch.int32, device=dev)
            cp_ent = torch.zeros(self.n_fix + 1, dtype=torch.int32, device=dev)
            st = _lib.lib().bf16x_cplan_build(self.tile_off.data_ptr(), self.tile_ent.data_ptr(), self.out_f,
                                              self.in_f, cp_off.data_ptr(), cp_ent.data_ptr(), _lib.stream_of(dev))
            _lib.check(st, "bf16x_cplan_build")
            self.cp_off, self.cp_ent = cp_off, cp_ent
        return self.cp_off, self.cp_ent

    def to(self, device) -> "Bf16xPlan":
        return Bf16xPlan(self.tile_off.to(device), self.tile_ent.to(device), self.tile_sat.to(device),
                         self.n_fix, self.out_f, self.in_f)


def plan_tiles(out_f: int, in_f: int) -> int:
    return int(_lib.lib().bf16x_plan_tiles(int(out_f), int(in_f)))


def _host_i32(t) -> torch.Tensor:
    """Host, contiguous tensor view of a tensor or numpy array."""
    if not isinstance(t, torch.Tensor):
        t = torch.from_numpy(t)
    return t.detach().cpu().contiguous()


def build_plan_host(packed: dict, check: int = 1, device=None) -> Bf16xPlan:
    """Plan from a (host) packed dict with the C++ builder; moved to `device`."""
    out_f, in_f = int(packed["out_f"]), int(packed["in_f"])
    if int(packed.get("sub", SUB)) != SUB:
        raise _lib.Bf16xError(_lib.ESUB, "build_plan_host")
    sign = _host_i32(packed["sign_packed"])
    mant = _host_i32(packed["mant_packed"])
    delta = _host_i32(packed["delta_packed"])
    emax = _host_i32(packed["emax"])
    idx = _host_i32(packed["delta_ovf_idx"]).to(torch.int32)
    val = _host_i32(packed["delta_ovf_val"]).to(torch.uint8)
    n_tiles = plan_tiles(out_f, in_f)
    tile_off = torch.empty(n_tiles + 1, dtype=torch.int32)
    cap = int((val > 7).sum())
    tile_ent = torch.empty(max(cap, 1), dtype=torch.int32)
    tile_sat = torch.zeros(max(cap, 1), dtype=torch.uint8)
    n_fix = ctypes.c_int64(0)
    st = _lib.lib().bf16x_plan_host(idx.data_ptr(), val.data_ptr(), idx.numel(), sign.data_ptr(), sign.numel(),
                                    mant.data_ptr(), mant.numel(), delta.data_ptr(), delta.numel(),
                                    emax.data_ptr(), emax.numel(), out_f, in_f, int(check),
                                    tile_off.data_ptr(), tile_ent.data_ptr(), tile_sat.data_ptr(), cap,
                                    ctypes.byref(n_fix))
    _lib.check(st, "bf16x_plan_host")
    k = int(n_fix.value)
    plan = Bf16xPlan(tile_off, tile_ent[:max(k, 1)].clone(), tile_sat[:max(k, 1)].clone(), k, out_f, in_f)
    return plan.to(device) if device is not None else plan


def build_plan_from_csr(olk, old, oloff, sign, mant, emax, out_f: int, in_f: int) -> Bf16xPlan:
    """Plan from the reference's device CSR (bf16x_fused.py:165-179): the
    offsets are reused as tile offsets, entries are re-encoded on the GPU."""
    dev = sign.device
    for t, nm in ((olk, "olk"), (old, "old"), (oloff, "oloff")):
        if not isinstance(t, torch.Tensor) or not t.is_cuda or t.device != dev or t.dtype != torch.int32:
            raise ValueError(f"{nm} must be an int32 tensor on the streams' GPU ({dev})")
    if oloff.numel() != int(out_f) + 1 or old.numel() != olk.numel():
        raise ValueError("CSR shape: oloff needs out_f + 1 offsets and old one value per olk column")
    olk, old, oloff = olk.contiguous(), old.contiguous(), oloff.contiguous()
    n = int(olk.numel())
    ent = torch.zeros(max(n, 1), dtype=torch.int32, device=dev)
    sat = torch.zeros(max(n, 1), dtype=torch.uint8, device=dev)
    st = _lib.lib().bf16x_plan_from_csr(_lib.ptr(olk), _lib.ptr(old),
                                        oloff.data_ptr(), sign.data_ptr(), mant.data_ptr(), emax.data_ptr(),
                                        int(out_f), int(in_f), n, ent.data_ptr(), sat.data_ptr(),
                                        _lib.stream_of(dev))
    _lib.check(st, "bf16x_plan_from_csr")
    # the kernels read entries [off[r], off[r + 1]) of a row: offsets held in
    # [0, n] keep every read inside the entry arrays whatever the caller's CSR
    return Bf16xPlan(oloff.clamp(0, n), ent, sat, n, int(out_f), int(in_f))


def build_plan_device(ovf_idx, ovf_val, sign, mant, emax, out_f: int, in_f: int) -> Bf16xPlan:
    """Plan from the dict's table when the streams already live on the GPU
    (the call pattern of bf16x_decode_triton, bf16x_triton_test.py:80-108):
    filter val > 7, per-row offsets by binary search, entries re-encoded by
    the CSR kernel.  Runs once per table; callers cache the result."""
    dev = sign.device
    if in_f > 65536:
        raise _lib.Bf16xError(_lib.ESHAPE, "build_plan_device (in_f > 65536 needs the host builder)")
    idx = ovf_idx.to(dev, torch.int64)
    val = ovf_val.to(dev, torch.int32)
    keep = val > 7
    idx, val = idx[keep], val[keep]
    rows = torch.div(idx, in_f, rounding_mode="floor")
    cols = (idx - rows * in_f).to(torch.int32)
    bounds = torch.arange(out_f + 1, device=dev, dtype=torch.int64)
    oloff = torch.searchsorted(rows, bounds).to(torch.int32)
    return build_plan_from_csr(cols, val, oloff, sign, mant, emax, out_f, in_f)

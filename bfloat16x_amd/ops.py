"""Operator wrappers mirroring the reference's call surface.

bf16x_decode / bf16x_decode_triton  <- bf16x_triton_test.py:80-108
bf16x_fused_gemv                    <- bf16x_fused.py:114-127
bf16x_fused_gemm                    <- bf16x_gemm_fused.py:97-114

Every wrapper validates its tensors on the host, then calls one C-ABI entry
point of libbf16x_hip.so on torch's current stream.  There is no fallback:
a missing library or a CPU tensor raises.
"""
from __future__ import annotations

import collections

import torch

from . import _lib
from .codec import Bf16xPlan, build_plan_device, build_plan_from_csr, build_plan_host

_X_DTYPES = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float32: _lib.F32}


def _dev_tensor(t: torch.Tensor, name: str, dtypes) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the BF16X engine has no CPU path)")
    if t.dtype not in dtypes:
        raise TypeError(f"{name}: dtype {t.dtype} not in {dtypes}")
    return t.contiguous()


def _streams(sign, mant, delta, emax):
    s = _dev_tensor(sign, "sign", (torch.int32,))
    m = _dev_tensor(mant, "mant", (torch.int32,))
    d = _dev_tensor(delta, "delta", (torch.int32,))
    e = _dev_tensor(emax, "emax", (torch.uint8,))
    dev = s.device
    for t, nm in ((m, "mant"), (d, "delta"), (e, "emax")):
        if t.device != dev:
            raise ValueError(f"{nm} is on {t.device}, sign on {dev}")
    return s, m, d, e


def _on(t: torch.Tensor, dev: torch.device, name: str) -> torch.Tensor:
    """t, required to live on the streams' GPU (kernels get raw pointers)."""
    if not t.is_cuda or t.device != dev:
        raise ValueError(f"{name} is on {t.device}, the weight streams on {dev}")
    return t


def _out(out, n: int, dev: torch.device, name: str = "out") -> torch.Tensor:
    """A caller-supplied bf16 output: contiguous, on the streams' GPU, at least
    n elements (the kernels write n elements through its pointer)."""
    if not isinstance(out, torch.Tensor) or out.dtype != torch.bfloat16 or not out.is_contiguous() \
            or out.numel() < n:
        raise ValueError(f"{name} must be a contiguous bf16 tensor of at least {n} elements")
    return _on(out, dev, name)


def _plan_on(plan: Bf16xPlan | None, dev: torch.device, out_f: int, in_f: int) -> Bf16xPlan | None:
    """A plan for this weight's shape on the streams' GPU (the kernels index
    its offsets by row and column)."""
    if plan is not None:
        if (plan.out_f, plan.in_f) != (out_f, in_f):
            raise ValueError(f"plan is for a {plan.out_f}x{plan.in_f} weight, not {out_f}x{in_f}")
        for nm in ("tile_off", "tile_ent", "tile_sat"):
            _on(getattr(plan, nm), dev, f"plan.{nm}")
    return plan


class _PlanCache:
    """Plans keyed by the identity and version of the tensors they came from.
    Entries hold references to those tensors, so a key cannot be reused by a
    different allocation while cached."""

    def __init__(self, cap: int = 64):
        self.cap = cap
        self.d: "collections.OrderedDict" = collections.OrderedDict()

    @staticmethod
    def _key(ts, extra):
        return tuple((t.data_ptr(), t.numel(), t._version, str(t.device)) for t in ts) + tuple(extra)

    def get(self, ts, extra, make):
        k = self._key(ts, extra)
        hit = self.d.get(k)
        if hit is not None:
            self.d.move_to_end(k)
            return hit[0]
        plan = make()
        self.d[k] = (plan, tuple(ts))
        if len(self.d) > self.cap:
            self.d.popitem(last=False)
        return plan


_PLANS = _PlanCache()


def plan_for_table(sign, mant, emax, ovf_idx, ovf_val, out_f, in_f) -> Bf16xPlan:
    """Device plan for a dict table given as (ovf_idx, ovf_val), cached."""
    def make():
        if in_f <= 65536:
            return build_plan_device(ovf_idx, ovf_val, sign, mant, emax, out_f, in_f)
        packed = dict(sign_packed=sign, mant_packed=mant, emax=emax, delta_ovf_idx=ovf_idx,
                      delta_ovf_val=ovf_val, out_f=out_f, in_f=in_f, sub=16,
                      delta_packed=torch.zeros(0, dtype=torch.int32))
        return build_plan_host(packed, check=0, device=sign.device)
    return _PLANS.get((sign, mant, emax, ovf_idx, ovf_val), (out_f, in_f), make)


def plan_for_csr(olk, old, oloff, sign, mant, emax, out_f, in_f) -> Bf16xPlan:
    return _PLANS.get((olk, old, oloff, sign, mant, emax), (out_f, in_f, "csr"),
                      lambda: build_plan_from_csr(olk, old, oloff, sign, mant, emax, out_f, in_f))


def bf16x_decode(sign, mant, delta, emax, out_f, in_f, ovf_idx=None, ovf_val=None, sub=16, *,
                 plan: Bf16xPlan | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Decode a packed dict to bf16 [out_f, in_f] on the streams' GPU.

    Same signature as bf16x_decode_triton (bf16x_triton_test.py:80): without a
    table (ovf_idx/ovf_val None) the 3-bit codes are used as-is (the base
    decode); with a table (or `plan`) the decode is exact.  Unlike the
    reference, the table is turned into a device plan once and cached, so a
    repeated call performs no host sync and no copy."""
    s, m, d, e = _streams(sign, mant, delta, emax)
    out_f, in_f = int(out_f), int(in_f)
    if plan is None and ovf_idx is not None and ovf_val is not None and ovf_val.numel() > 0:
        plan = plan_for_table(s, m, e, ovf_idx, ovf_val, out_f, in_f)
    _plan_on(plan, s.device, out_f, in_f)
    mode = _lib.SATURATED if plan is None else _lib.EXACT
    if out is None:
        out = torch.empty(out_f, in_f, dtype=torch.bfloat16, device=s.device)
    else:
        _out(out, out_f * in_f, s.device)
    st = _lib.lib().bf16x_decode(s.data_ptr(), s.numel(), m.data_ptr(), m.numel(), d.data_ptr(), d.numel(),
                                 e.data_ptr(), e.numel(), _lib.ptr(plan.tile_off) if plan else None,
                                 _lib.ptr(plan.tile_ent) if plan else None, out_f, in_f, int(sub), mode,
                                 out.data_ptr(), _lib.stream_of(s.device))
    _lib.check(st, "bf16x_decode")
    return out


bf16x_decode_triton = bf16x_decode  # name of the reference entry point


def bf16x_gemv(x, sign, mant, delta, emax, out_f, in_f, plan: Bf16xPlan | None = None, sub=16,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """y[out_f] (bf16) = W . x with W decoded on the fly; exact with a plan,
    saturated without one."""
    s, m, d, e = _streams(sign, mant, delta, emax)
    xx = _dev_tensor(x, "x", tuple(_X_DTYPES)).reshape(-1)
    out_f, in_f = int(out_f), int(in_f)
    if xx.numel() != in_f:
        raise ValueError(f"x has {xx.numel()} elements, in_f = {in_f}")
    _on(xx, s.device, "x")
    _plan_on(plan, s.device, out_f, in_f)
    y = _out(out, out_f, s.device) if out is not None else torch.empty(out_f, dtype=torch.bfloat16, device=s.device)
    mode = _lib.SATURATED if plan is None else _lib.EXACT
    st = _lib.lib().bf16x_gemv(xx.data_ptr(), _X_DTYPES[xx.dtype], s.data_ptr(), s.numel(), m.data_ptr(),
                               m.numel(), d.data_ptr(), d.numel(), e.data_ptr(), e.numel(),
                               _lib.ptr(plan.tile_off) if plan else None, _lib.ptr(plan.tile_ent) if plan else None,
                               _lib.ptr(plan.tile_sat) if plan else None, out_f, in_f, int(sub), mode, y.data_ptr(),
                               _lib.stream_of(s.device))
    _lib.check(st, "bf16x_gemv")
    return y


def bf16x_gemv_swiglu(x, sign, mant, delta, emax, out_f, in_f, plan: Bf16xPlan | None = None,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """act[out_f // 2] (bf16) = silu(gate) * up of the GEMV W . x, W's rows in
    groups of 8 [gate 4b .. 4b+3, up 4b .. 4b+3] (include/bf16x_llama.h)."""
    s, m, d, e = _streams(sign, mant, delta, emax)
    xx = _dev_tensor(x, "x", (torch.bfloat16,)).reshape(-1)
    out_f, in_f = int(out_f), int(in_f)
    if xx.numel() != in_f:
        raise ValueError(f"x has {xx.numel()} elements, in_f = {in_f}")
    _on(xx, s.device, "x")
    _plan_on(plan, s.device, out_f, in_f)
    y = _out(out, out_f // 2, s.device) if out is not None else \
        torch.empty(out_f // 2, dtype=torch.bfloat16, device=s.device)
    mode = _lib.SATURATED if plan is None else _lib.EXACT
    st = _lib.lib().bf16x_gemv_swiglu(xx.data_ptr(), s.data_ptr(), s.numel(), m.data_ptr(), m.numel(), d.data_ptr(),
                                      d.numel(), e.data_ptr(), e.numel(),
                                      _lib.ptr(plan.tile_off) if plan else None,
                                      _lib.ptr(plan.tile_ent) if plan else None,
                                      _lib.ptr(plan.tile_sat) if plan else None, out_f, in_f, mode, y.data_ptr(),
                                      _lib.stream_of(s.device))
    _lib.check(st, "bf16x_gemv_swiglu")
    return y


def bf16x_gemv_norm(x, residual_in, norm_weight, residual_out, eps, sign, mant, delta, emax, out_f, in_f,
                    plan: Bf16xPlan | None = None, swiglu: bool = False,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """GEMV whose input is RMSNorm(x + residual_in) * norm_weight, computed in
    the kernel; x + residual_in is stored to residual_out (include/bf16x_llama.h).
    swiglu: the SwiGLU epilogue (out_f // 2 outputs)."""
    s, m, d, e = _streams(sign, mant, delta, emax)
    out_f, in_f = int(out_f), int(in_f)
    bf = (torch.bfloat16,)
    xx = _dev_tensor(x, "x", bf).reshape(-1)
    nw = _dev_tensor(norm_weight, "norm_weight", bf).reshape(-1)
    ri = _dev_tensor(residual_in, "residual_in", bf).reshape(-1) if residual_in is not None else None
    if residual_out is not None:
        _out(residual_out, in_f, s.device, "residual_out")
    for t, nm in ((xx, "x"), (nw, "norm_weight"), (ri, "residual_in")):
        if t is not None:
            _on(t, s.device, nm)
            if t.numel() != in_f:
                raise ValueError(f"{nm} has {t.numel()} elements, in_f = {in_f}")
    _plan_on(plan, s.device, out_f, in_f)
    n_out = out_f // 2 if swiglu else out_f
    y = _out(out, n_out, s.device) if out is not None else torch.empty(n_out, dtype=torch.bfloat16, device=s.device)
    mode = _lib.SATURATED if plan is None else _lib.EXACT
    st = _lib.lib().bf16x_gemv_norm(xx.data_ptr(), _lib.ptr(ri), nw.data_ptr(), _lib.ptr(residual_out), float(eps),
                                    s.data_ptr(), s.numel(), m.data_ptr(), m.numel(), d.data_ptr(), d.numel(),
                                    e.data_ptr(), e.numel(), _lib.ptr(plan.tile_off) if plan else None,
                                    _lib.ptr(plan.tile_ent) if plan else None,
                                    _lib.ptr(plan.tile_sat) if plan else None, out_f, in_f, mode,
                                    1 if swiglu else 0, y.data_ptr(), _lib.stream_of(s.device))
    _lib.check(st, "bf16x_gemv_norm")
    return y


def gemv_residual_slots(out_f, in_f) -> int:
    """Number of fp32 slots bf16x_gemv_residual writes for this shape."""
    n = int(_lib.lib().bf16x_gemv_residual_slots(int(out_f), int(in_f)))
    if n < 0:
        raise _lib.Bf16xError(_lib.ESHAPE, "bf16x_gemv_residual_slots")
    return n


def bf16x_gemv_residual(x, residual_in, residual_out, slots, sign, mant, delta, emax, out_f, in_f,
                        plan: Bf16xPlan | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """y = W . x, then h = bf16(y + residual_in) to residual_out and the sum of
    h^2 per workgroup to `slots` (fp32, gemv_residual_slots(out_f, in_f)
    entries), for a following bf16x_gemv_prenormed (include/bf16x_llama.h)."""
    s, m, d, e = _streams(sign, mant, delta, emax)
    out_f, in_f = int(out_f), int(in_f)
    xx = _on(_dev_tensor(x, "x", (torch.bfloat16,)).reshape(-1), s.device, "x")
    if xx.numel() != in_f:
        raise ValueError(f"x has {xx.numel()} elements, in_f = {in_f}")
    ri = _out(residual_in, out_f, s.device, "residual_in")
    ro = _out(residual_out, out_f, s.device, "residual_out")
    if not isinstance(slots, torch.Tensor) or slots.dtype != torch.float32 or not slots.is_contiguous():
        raise ValueError("slots must be a contiguous fp32 tensor")
    _on(slots, s.device, "slots")
    _plan_on(plan, s.device, out_f, in_f)
    y = _out(out, out_f, s.device) if out is not None else torch.empty(out_f, dtype=torch.bfloat16, device=s.device)
    mode = _lib.SATURATED if plan is None else _lib.EXACT
    st = _lib.lib().bf16x_gemv_residual(xx.data_ptr(), ri.data_ptr(), ro.data_ptr(), slots.data_ptr(), slots.numel(),
                                        s.data_ptr(), s.numel(), m.data_ptr(), m.numel(), d.data_ptr(), d.numel(),
                                        e.data_ptr(), e.numel(), _lib.ptr(plan.tile_off) if plan else None,
                                        _lib.ptr(plan.tile_ent) if plan else None,
                                        _lib.ptr(plan.tile_sat) if plan else None, out_f, in_f, mode, y.data_ptr(),
                                        _lib.stream_of(s.device))
    _lib.check(st, "bf16x_gemv_residual")
    return y


def bf16x_gemv_prenormed(h, norm_weight, eps, slots, n_slots, sign, mant, delta, emax, out_f, in_f,
                         plan: Bf16xPlan | None = None, swiglu: bool = False,
                         out: torch.Tensor | None = None) -> torch.Tensor:
    """GEMV of RMSNorm(h) * norm_weight with the sum of h^2 read from the
    first n_slots entries of `slots` (a bf16x_gemv_residual launch's);
    swiglu: the SwiGLU epilogue (out_f // 2 outputs)."""
    s, m, d, e = _streams(sign, mant, delta, emax)
    out_f, in_f = int(out_f), int(in_f)
    hh = _on(_dev_tensor(h, "h", (torch.bfloat16,)).reshape(-1), s.device, "h")
    nw = _on(_dev_tensor(norm_weight, "norm_weight", (torch.bfloat16,)).reshape(-1), s.device, "norm_weight")
    for t, nm in ((hh, "h"), (nw, "norm_weight")):
        if t.numel() != in_f:
            raise ValueError(f"{nm} has {t.numel()} elements, in_f = {in_f}")
    if not isinstance(slots, torch.Tensor) or slots.dtype != torch.float32 or not slots.is_contiguous() or \
            slots.numel() < int(n_slots):
        raise ValueError("slots must be a contiguous fp32 tensor of at least n_slots entries")
    _on(slots, s.device, "slots")
    _plan_on(plan, s.device, out_f, in_f)
    n_out = out_f // 2 if swiglu else out_f
    y = _out(out, n_out, s.device) if out is not None else torch.empty(n_out, dtype=torch.bfloat16, device=s.device)
    mode = _lib.SATURATED if plan is None else _lib.EXACT
    st = _lib.lib().bf16x_gemv_prenormed(hh.data_ptr(), nw.data_ptr(), float(eps), slots.data_ptr(), int(n_slots),
                                         s.data_ptr(), s.numel(), m.data_ptr(), m.numel(), d.data_ptr(), d.numel(),
                                         e.data_ptr(), e.numel(), _lib.ptr(plan.tile_off) if plan else None,
                                         _lib.ptr(plan.tile_ent) if plan else None,
                                         _lib.ptr(plan.tile_sat) if plan else None, out_f, in_f, mode,
                                         1 if swiglu else 0, y.data_ptr(), _lib.stream_of(s.device))
    _lib.check(st, "bf16x_gemv_prenormed")
    return y


def bf16x_fused_gemv(x, sign, mant, delta, emax, olk, old, oloff, out_f, in_f, group=16, r=4, bk=256,
                     num_warps=2, *, plan: Bf16xPlan | None = None) -> torch.Tensor:
    """Fused decode+GEMV with the reference's signature (bf16x_fused.py:114).

    olk/old/oloff is the reference's per-row CSR of entries with true delta
    > 7; it is converted once (cached) into a plan.  `r`, `bk`, `num_warps`
    are Triton tuning knobs with no meaning here and are ignored; `group`
    must be 16."""
    if group != 16:
        raise _lib.Bf16xError(_lib.ESUB, "bf16x_fused_gemv")
    if plan is None and oloff is not None:
        s, m, _, e = _streams(sign, mant, delta, emax)
        plan = plan_for_csr(olk, old, _dev_tensor(oloff, "oloff", (torch.int32,)), s, m, e, out_f, in_f)
    return bf16x_gemv(x, sign, mant, delta, emax, out_f, in_f, plan=plan)


# Activation rows up to which bf16x_gemm runs the row-streaming few-row
# kernel (bf16x_gemm_rows in the C ABI: weights of 2048 or 4096 columns).
GEMM_ROWS_MAX = 16
GEMM_ROWS_IN_F = (2048, 4096)
# Activation rows for which bf16x_gemm runs the chunked few-row kernel
# (bf16x_gemm_chunks: in_f % 256 == 0), for weights of at most
# GEMM_CHUNKS_MAX_IN_F columns, except above 32 rows when a CU has 16 rows or
# fewer (each CU then reads more x than weight).  Measured, exact, weights
# rotated through HBM, chunked against the 16x16x32 few-row kernel (us):
# 14336x4096 M = 24 / 32 / 48 / 64: 29.0 / 30.2 / 36.8 / 38.7 against 32.0 /
# 32.0 / 43.0 / 44.3; 4096x4096 M = 24 / 32: 16.4 / 17.5 against 19.9 / 19.6,
# M = 64: 22.6 against 20.8; 4096x14336 M = 32: 44.9 against 33.8.
GEMM_CHUNKS_MIN = 17
GEMM_CHUNKS_MAX = 64
GEMM_CHUNKS_MAX_IN_F = 8192


def _cus(dev) -> int:
    return torch.cuda.get_device_properties(dev).multi_processor_count


def _use_chunks(M: int, out_f: int, in_f: int, dev) -> bool:
    if not (GEMM_CHUNKS_MIN <= M <= GEMM_CHUNKS_MAX) or in_f % 256 or in_f > GEMM_CHUNKS_MAX_IN_F:
        return False
    return M <= 32 or -(-out_f // _cus(dev)) > 16
# One bf16 activation row goes to the GEMV (bf16x_gemv), which streams the
# weight faster than any GEMM kernel at one row (14336x4096: 19.4 against
# 24.2 us for the row-streaming GEMM).
GEMM_ONE_ROW_GEMV = True


def _gemm_launch(x2, s, m, d, e, out_f, in_f, plan, y, y_dtype, sub=16):
    mode = _lib.SATURATED if plan is None else _lib.EXACT
    L = _lib.lib()
    M = x2.shape[0]
    if M <= GEMM_ROWS_MAX and in_f in GEMM_ROWS_IN_F:
        st = L.bf16x_gemm_rows(x2.data_ptr(), _lib.BF16, M, s.data_ptr(), s.numel(), m.data_ptr(),
                               m.numel(), d.data_ptr(), d.numel(), e.data_ptr(), e.numel(),
                               _lib.ptr(plan.tile_off) if plan is not None else None,
                               _lib.ptr(plan.tile_ent) if plan is not None else None, out_f, in_f, int(sub),
                               mode, y.data_ptr(), y_dtype, _lib.stream_of(s.device))
        _lib.check(st, "bf16x_gemm_rows")
        return
    if _use_chunks(M, out_f, in_f, x2.device):
        cp_off, cp_ent = plan.cplan() if plan is not None else (None, None)
        st = L.bf16x_gemm_chunks(x2.data_ptr(), _lib.BF16, M, s.data_ptr(), s.numel(), m.data_ptr(),
                                 m.numel(), d.data_ptr(), d.numel(), e.data_ptr(), e.numel(), _lib.ptr(cp_off),
                                 _lib.ptr(cp_ent), out_f, in_f, int(sub), mode, y.data_ptr(), y_dtype,
                                 _lib.stream_of(s.device))
        _lib.check(st, "bf16x_gemm_chunks")
        return
    kp_off, kp_ent = plan.kplan() if plan is not None else (None, None)
    ws_bytes = int(L.bf16x_gemm_workspace(M, out_f, in_f))
    ws = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=x2.device) if ws_bytes else None
    st = L.bf16x_gemm(x2.data_ptr(), _lib.BF16, M, s.data_ptr(), s.numel(), m.data_ptr(),
                      m.numel(), d.data_ptr(), d.numel(), e.data_ptr(), e.numel(), _lib.ptr(kp_off),
                      _lib.ptr(kp_ent), out_f, in_f, int(sub), mode, y.data_ptr(), y_dtype,
                      _lib.ptr(ws), ws_bytes, _lib.stream_of(s.device))
    _lib.check(st, "bf16x_gemm")


# From this many activation rows on, bf16x_gemm decodes W once at HBM speed
# and runs the product as a plain library GEMM (hipBLASLt through
# F.linear): the decode is amortised over the rows and the library GEMM runs
# closer to the MFMA peak than the fused kernel, which decodes every W tile
# once per 256 activation rows (at 2048 rows, eight times).  Below it the
# fused kernel avoids writing and re-reading the decoded weight.  The switch
# depends on the weight's shape (GEMM_DECODE_MIN_ROWS for square weights,
# _TALL for more rows than columns, _WIDE for more columns than rows).
# Measured (exact, weights rotated through HBM, fused against decode +
# hipBLASLt, us): 4096x4096 M = 512 / 640 / 768: 42.4 / 53.9 / 54.7 against
# 54.0 / 53.9 / 52.3; 14336x4096 M = 512 / 640: 81.6 / 125.4 against
# 102.9 / 115.7; 28672x4096 M = 512 / 640: 165.9 / 234.3 against 179.2 /
# 218.8; 4096x14336 M = 1024 / 1536: 159.4 / 262.6 against 171.5 / 207.8.
GEMM_DECODE_MIN_ROWS = 704
GEMM_DECODE_MIN_ROWS_TALL = 640
GEMM_DECODE_MIN_ROWS_WIDE = 1536


def _decode_min_rows(out_f: int, in_f: int) -> int:
    if in_f > out_f:
        return GEMM_DECODE_MIN_ROWS_WIDE
    return GEMM_DECODE_MIN_ROWS_TALL if out_f > in_f else GEMM_DECODE_MIN_ROWS


def bf16x_gemm(x, sign, mant, delta, emax, out_f, in_f, plan: Bf16xPlan | None = None, sub=16,
               path: str = "auto") -> torch.Tensor:
    """y[..., out_f] = x[..., in_f] . W^T, in x's dtype.  Exact with a plan,
    saturated without one.

    path "fused": the fused decode+GEMM kernels (bf16x_gemm_rows up to
    GEMM_ROWS_MAX rows at in_f 2048 / 4096, bf16x_gemm_chunks from
    GEMM_CHUNKS_MIN to GEMM_CHUNKS_MAX rows (see _use_chunks), else
    bf16x_gemm in the C ABI; one bf16 row the fused GEMV, bf16x_gemv);
    bf16 activations run one bf16 MFMA pass, fp16/fp32 activations are split
    as x = hi + lo (two bf16 tensors, exact for fp16, 16 mantissa bits for
    fp32) accumulated over two passes in fp32.
    path "decode": W decoded into a temporary by the HIP decoder, then
    F.linear on the same device (fp32 for fp16/fp32 activations).
    path "auto": "decode" from GEMM_DECODE_MIN_ROWS rows on (_TALL / _WIDE for
    weights with more rows / columns) and for shapes the fused kernel does
    not take (in_f not a multiple of 64, or above 65536), "fused" otherwise."""
    if path not in ("auto", "fused", "decode"):
        raise ValueError(f"path must be auto, fused or decode, not {path!r}")
    s, m, d, e = _streams(sign, mant, delta, emax)
    out_f, in_f = int(out_f), int(in_f)
    xx = _on(_dev_tensor(x, "x", tuple(_X_DTYPES)), s.device, "x")
    if xx.shape[-1] != in_f:
        raise ValueError(f"x has last dimension {xx.shape[-1]}, in_f = {in_f}")
    _plan_on(plan, s.device, out_f, in_f)
    lead = xx.shape[:-1]
    x2 = xx.reshape(-1, in_f)
    if x2.shape[0] == 0:
        return torch.empty(*lead, out_f, dtype=xx.dtype, device=xx.device)
    fusable = in_f % 64 == 0 and in_f <= 65536
    if path == "fused" and not fusable:
        raise _lib.Bf16xError(_lib.ESHAPE, "bf16x_gemm (fused path needs in_f % 64 == 0 and in_f <= 65536)")
    if path == "decode" or (path == "auto" and (not fusable or x2.shape[0] >= _decode_min_rows(out_f, in_f))):
        w = bf16x_decode(s, m, d, e, out_f, in_f, sub=sub, plan=plan)
        if xx.dtype == torch.bfloat16:
            y = torch.nn.functional.linear(x2.contiguous(), w)
        else:
            y = torch.nn.functional.linear(x2.float(), w.float())
        return y.to(xx.dtype).reshape(*lead, out_f)
    if xx.dtype == torch.bfloat16 and x2.shape[0] == 1 and GEMM_ONE_ROW_GEMV:
        return bf16x_gemv(x2[0], s, m, d, e, out_f, in_f, plan=plan, sub=sub).reshape(*lead, out_f)
    if xx.dtype == torch.bfloat16:
        y = torch.empty(x2.shape[0], out_f, dtype=torch.bfloat16, device=xx.device)
        _gemm_launch(x2.contiguous(), s, m, d, e, out_f, in_f, plan, y, _lib.BF16, sub)
    else:
        xf = x2.float()
        hi = xf.to(torch.bfloat16)
        lo = (xf - hi.float()).to(torch.bfloat16)
        y = torch.empty(x2.shape[0], out_f, dtype=torch.float32, device=xx.device)
        y2 = torch.empty_like(y)
        _gemm_launch(hi.contiguous(), s, m, d, e, out_f, in_f, plan, y, _lib.F32, sub)
        _gemm_launch(lo.contiguous(), s, m, d, e, out_f, in_f, plan, y2, _lib.F32, sub)
        y = (y + y2).to(xx.dtype)
    return y.reshape(*lead, out_f)


def bf16x_fused_gemm(x, sign, mant, delta, emax, out_f, in_f, group=16, bn=128, bk=32, num_warps=8,
                     num_stages=1, *, plan: Bf16xPlan | None = None, path: str = "auto") -> torch.Tensor:
    """Fused decode+GEMM with the reference's signature (bf16x_gemm_fused.py:97).

    Without `plan` the weight is saturated exactly as the reference kernel
    decodes it (no overflow correction); with a plan it is exact.  Returns
    [M, out_f] in x's dtype for x of shape [*, in_f] (M = leading elements).
    `bn`, `bk`, `num_warps`, `num_stages` are Triton tuning knobs and are
    ignored; `group` must be 16."""
    if group != 16:
        raise _lib.Bf16xError(_lib.ESUB, "bf16x_fused_gemm")
    y = bf16x_gemm(x, sign, mant, delta, emax, out_f, in_f, plan=plan, path=path)
    return y.reshape(-1, int(out_f))

"""GPU tests of the Llama harness.

Kernels (include/bf16x_llama.h) against plain torch fp32 references of the
same ops on the same bf16 inputs; then a small stack end to end: prefill
logits against an fp32 CPU forward of the same weights, decode steps against
a prefill over the same tokens (KV cache and positions), the HIP-graph
decode against eager steps over several replays, and the BF16X-deployed
stack against the bf16 one on the same token path."""
import math

import numpy as np
import pytest
import torch

from bfloat16x_amd import llama
from oracle import dict_codec as dc
from tests.test_gpu_dict import DEV

pytestmark = pytest.mark.gpu

BF_ULP = 2.0 ** -7          # a bf16 ulp is at most 2^-7 of the value (7 stored mantissa bits)


@pytest.fixture(scope="module")
def bx():
    import bfloat16x_amd as m
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return m


def rnd(shape, seed, scale=1.0):
    return (torch.randn(shape, generator=torch.Generator().manual_seed(seed)) * scale).to(torch.bfloat16)


def bf(t):
    """fp32 -> bf16 -> fp32 (one round to nearest even)."""
    return t.to(torch.bfloat16).float()


def within_ulps(got, ref, ulps=1.0, floor=1e-30):
    got, ref = got.float().cpu(), ref.float().cpu()
    err = (got - ref).abs()
    bound = ulps * BF_ULP * ref.abs() + floor
    assert bool((err <= bound).all()), float((err - bound).max())


def norm_rel(y, r):
    y, r = np.asarray(y, np.float64).reshape(-1), np.asarray(r, np.float64).reshape(-1)
    return float(np.linalg.norm(y - r) / np.linalg.norm(r))


# --------------------------------------------------------------------------- kernels

@torch.no_grad()
@pytest.mark.parametrize("n,rows", [(4096, 3), (512, 5), (8192, 1), (1536, 2)])
def test_rmsnorm(bx, n, rows):
    x, r, w = rnd((rows, n), 1), rnd((rows, n), 2), rnd(n, 3)
    eps = 1e-5
    h = bf(x.float() + r.float())
    y = bf(h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps))
    ref = bf(y * w.float())
    res = r.to(DEV)
    out = torch.empty(rows, n, dtype=torch.bfloat16, device=DEV)
    llama.rmsnorm(x.to(DEV), w.to(DEV), out, res, flags=llama.NORM_ADD | llama.NORM_STORE, eps=eps)
    assert torch.equal(res.cpu(), h.to(torch.bfloat16))            # the residual add is exact RNE
    within_ulps(out, ref, 1.0)
    # plain norm, no residual
    y0 = bf(x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps))
    llama.rmsnorm(x.to(DEV), w.to(DEV), out, eps=eps)
    within_ulps(out, bf(y0 * w.float()), 1.0)


@torch.no_grad()
def test_rmsnorm_gather_store(bx):
    table, w = rnd((100, 512), 4), rnd(512, 5)
    ids = torch.tensor([7, 0, 99, 7, 42], dtype=torch.int64)
    res = torch.zeros(5, 512, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(5, 512, dtype=torch.bfloat16, device=DEV)
    llama.rmsnorm(table.to(DEV), w.to(DEV), out, res, row_idx=ids.to(DEV), flags=llama.NORM_STORE)
    h = table[ids].float()
    assert torch.equal(res.cpu(), table[ids])
    within_ulps(out, bf(bf(h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + 1e-5)) * w.float()), 1.0)


def rope_ref(x, cs, pos):
    """x [T, heads, 128] fp32, rotate-half at positions pos + t."""
    T = x.shape[0]
    c = cs[pos:pos + T, :, 0][:, None, :]
    s = cs[pos:pos + T, :, 1][:, None, :]
    a, b = x[..., :64], x[..., 64:]
    return torch.cat([a * c - b * s, b * c + a * s], dim=-1)


@torch.no_grad()
@pytest.mark.parametrize("T,pos", [(1, 0), (1, 37), (9, 5), (40, 0)])
def test_rope_kv(bx, T, pos):
    H, KV, L = 8, 2, 48
    qkv = rnd((T, (H + 2 * KV) * 128), 6)
    cs = llama.rope_table(L, 5e5, "cpu")
    kc = torch.zeros(KV, L, 128, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    q = torch.zeros(T, H * 128, dtype=torch.bfloat16, device=DEV)
    llama.rope_kv(qkv.to(DEV), torch.tensor([pos], dtype=torch.int32, device=DEV), cs.to(DEV), H, KV, q, kc, vc)
    x = qkv.float().view(T, H + 2 * KV, 128)
    qr = rope_ref(x[:, :H], cs, pos)
    kr = rope_ref(x[:, H:H + KV], cs, pos)
    within_ulps(q.view(T, H, 128), bf(qr), 1.0)
    within_ulps(kc[:, pos:pos + T].permute(1, 0, 2), bf(kr), 1.0)
    assert torch.equal(vc[:, pos:pos + T].permute(1, 0, 2).cpu(), qkv.view(T, H + 2 * KV, 128)[:, H + KV:])
    # nothing written outside [pos, pos + T)
    keep = torch.ones(L, dtype=torch.bool)
    keep[pos:pos + T] = False
    assert not kc[:, keep.to(DEV)].any() and not vc[:, keep.to(DEV)].any()


@torch.no_grad()
def test_rope_kv_positions_past_the_cache_are_dropped(bx):
    H, KV, L = 4, 2, 16
    qkv = rnd((4, (H + 2 * KV) * 128), 7)
    kc = torch.zeros(KV, L, 128, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    q = torch.zeros(4, H * 128, dtype=torch.bfloat16, device=DEV)
    llama.rope_kv(qkv.to(DEV), torch.tensor([14], dtype=torch.int32, device=DEV),
                  llama.rope_table(L, 5e5, DEV), H, KV, q, kc, vc)
    assert kc[:, 14:].abs().sum() > 0 and not kc[:, :14].any()          # positions 16, 17 not written


def attn_ref(q, kc, vc, pos, H, KV):
    """q [T, H, 128], caches [KV, L, 128] fp32; query t sees keys 0..pos+t."""
    T = q.shape[0]
    out = torch.empty(T, H, 128)
    for t in range(T):
        n = pos + t + 1
        for h in range(H):
            kvh = h // (H // KV)
            s = (kc[kvh, :n] @ q[t, h]) / math.sqrt(128)
            p = torch.softmax(s.double(), 0).float()
            out[t, h] = p @ vc[kvh, :n]
    return out


@torch.no_grad()
@pytest.mark.parametrize("T,pos,L", [(1, 0, 16), (1, 300, 640), (7, 10, 64), (3, 1021, 1024)])
def test_attention(bx, T, pos, L):
    H, KV = 8, 2
    q = rnd((T, H, 128), 8)
    kc, vc = rnd((KV, L, 128), 9), rnd((KV, L, 128), 10)
    out = torch.empty(T, H * 128, dtype=torch.bfloat16, device=DEV)
    llama.attention(q.to(DEV).view(T, H * 128), kc.to(DEV), vc.to(DEV),
                    torch.tensor([pos], dtype=torch.int32, device=DEV), H, KV, out)
    ref = attn_ref(q.float(), kc.float(), vc.float(), pos, H, KV)
    err = (out.float().cpu().view(T, H, 128) - ref).abs()
    # fp32 softmax and sums, one bf16 rounding of the output
    assert float((err - (BF_ULP * ref.abs() + 1e-4)).max()) <= 0, float(err.max())


def attn_ref_batched(q, kc, vc, pos, H, KV):
    """attn_ref with the causal mask as one masked matrix product per head
    (fp32 scores, fp64 softmax): q [T, H, 128], caches [KV, L, 128]."""
    T, L = q.shape[0], kc.shape[1]
    out = torch.zeros(T, H, 128)
    qpos = pos + torch.arange(T)
    keep = torch.arange(L)[None, :] <= qpos[:, None]                    # [T, L]
    for h in range(H):
        kvh = h // (H // KV)
        s = (q[:, h] @ kc[kvh].t()) / math.sqrt(128)                     # [T, L]
        s = s.double().masked_fill(~keep, float("-inf"))
        p = torch.softmax(s, 1).float()
        p = torch.nan_to_num(p)                                            # rows without keys
        out[:, h] = p @ vc[kvh]
    return out


@torch.no_grad()
@pytest.mark.parametrize("T,pos,L,H,KV", [(1, 0, 16, 8, 2), (7, 10, 64, 8, 2), (64, 0, 64, 8, 2),
                                          (100, 3, 128, 8, 2), (16, 0, 48, 4, 4), (65, 959, 1024, 8, 1),
                                          (512, 0, 640, 32, 8), (200, 300, 640, 32, 8)])
def test_attention_mfma(bx, tune, T, pos, L, H, KV):
    """The MFMA prefill kernel (forced with attn_mfma = 1, which the default
    dispatch takes from 16 query rows) against an fp32 reference with the
    causal mask, at full and ragged 64-row tiles, key counts that are not a
    multiple of the 32-key block, several GQA groupings and the prefill
    shape of the Llama harness; and against the scalar kernel."""
    tune(attn_mfma=1)
    q = rnd((T, H, 128), 21)
    kc, vc = rnd((KV, L, 128), 22), rnd((KV, L, 128), 23)
    p = torch.tensor([pos], dtype=torch.int32, device=DEV)
    out = torch.empty(T, H * 128, dtype=torch.bfloat16, device=DEV)
    llama.attention(q.to(DEV).view(T, H * 128), kc.to(DEV), vc.to(DEV), p, H, KV, out)
    ref = attn_ref_batched(q.float(), kc.float(), vc.float(), pos, H, KV)
    err = (out.float().cpu().view(T, H, 128) - ref).abs()
    # fp32 softmax and sums, one bf16 rounding of the output
    assert float((err - (BF_ULP * ref.abs() + 1e-4)).max()) <= 0, float(err.max())
    with bx.tuning(attn_mfma=0):
        out0 = torch.empty_like(out)
        llama.attention(q.to(DEV).view(T, H * 128), kc.to(DEV), vc.to(DEV), p, H, KV, out0)
    within_ulps(out, out0, 1.0, floor=1e-4)


@torch.no_grad()
@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("H,KV,pos,L", [(4, 4, 0, 16), (8, 4, 5, 64), (32, 8, 300, 640), (32, 8, 639, 640),
                                        (16, 2, 100, 640), (8, 1, 31, 48), (32, 8, 3000, 4096),
                                        (64, 8, 511, 1024), (32, 8, 1, 640), (32, 8, 199, 200),
                                        (32, 8, 767, 768), (64, 8, 700, 768), (8, 2, 400, 769), (32, 8, 257, 260)])
def test_attention_decode_matches_two_launch_path(bx, H, KV, pos, L, split, tune):
    """The fused one-token kernel against rope_kv + attention on the same
    inputs: the same cache rows and outputs (one bf16 rounding apart at
    most), and the fp32 reference.  Contexts up to 256 keys run the
    one-workgroup-per-KV-head kernel, up to 768 the one-workgroup-per-query-
    head kernel, unless the override attn_split = 1 selects the split kernel
    (which longer contexts always use)."""
    if split:
        tune(attn_split=1)
    assert llama.attention_decode_supported(H, KV, L)
    qkv = rnd((H + 2 * KV) * 128, 13)
    kc0, vc0 = rnd((KV, L, 128), 14), rnd((KV, L, 128), 15)
    cs = llama.rope_table(L, 5e5, DEV)
    p = torch.tensor([pos], dtype=torch.int32, device=DEV)
    kA, vA, kB, vB = kc0.to(DEV), vc0.to(DEV), kc0.to(DEV), vc0.to(DEV)
    q = torch.empty(H * 128, dtype=torch.bfloat16, device=DEV)
    outA = torch.empty(H * 128, dtype=torch.bfloat16, device=DEV)
    outB = torch.empty_like(outA)
    llama.rope_kv(qkv.to(DEV), p, cs, H, KV, q, kA, vA)
    llama.attention(q, kA, vA, p, H, KV, outA)
    ws = llama.attention_decode_workspace(H, KV, L, DEV)
    llama.attention_decode(qkv.to(DEV), p, cs, H, KV, kB, vB, outB, ws)
    assert not ws[:KV].any()                                        # the counters are left at zero
    assert torch.equal(vA, vB)
    within_ulps(kB, kA, 1.0)
    keep = torch.ones(L, dtype=torch.bool, device=DEV)
    keep[pos] = False
    assert torch.equal(kB[:, keep], kc0.to(DEV)[:, keep])           # only row `pos` written
    within_ulps(outB, outA, 1.0, floor=1e-4)         # summation order differs: near-zero outputs
    ref = attn_ref(q.float().cpu().view(1, H, 128), kA.float().cpu(), vA.float().cpu(), pos, H, KV)
    err = (outB.float().cpu().view(1, H, 128) - ref).abs()
    assert float((err - (BF_ULP * ref.abs() + 1e-4)).max()) <= 0, float(err.max())


@torch.no_grad()
@pytest.mark.parametrize("H,KV,in_f,L,mode,o_out_f", [(32, 8, 4096, 640, "exact", 4096),
                                                       (32, 8, 4096, 768, "saturated", 4100),
                                                       (32, 8, 4096, 300, "exact", 0), (16, 2, 3072, 300, "exact", 0),
                                                       (64, 8, 4096, 257, "exact", 0),
                                                       (8, 8, 2080, 512, "saturated", 0)])
def test_layer_front_matches_separate_launches(bx, H, KV, in_f, L, mode, o_out_f):
    """bf16x_layer_front_decode (the qkv GEMV, the decode attention and the
    o GEMV with the residual add in one launch, ordered by device counters)
    against bf16x_gemv_prenormed, bf16x_attention_decode and
    bf16x_gemv_residual in sequence: qkv, the attention output, both caches,
    the o output, the residual and its slots bit-identical, over consecutive
    calls at several positions that alternate between two counter buffers,
    each call clearing the other's (the timeout flag stays clear)."""
    import types
    from bfloat16x_amd import ops
    from tests.test_gpu_dict import bits_tensor, to_dev
    print("layer front", H, KV, in_f, L, mode, o_out_f, flush=True)
    out_f = (H + 2 * KV) * 128
    assert llama.layer_front_supported(H, KV, L, out_f, in_f)

    def module(of, seed):
        d = bx.bf16x_quantize(bits_tensor(dc.bench_weight_bits(of, in_f, seed=seed)))
        g = to_dev(d)
        plan = bx.build_plan_host(d, device=DEV) if mode == "exact" else None
        return types.SimpleNamespace(_sign=g["sign_packed"], _mant=g["mant_packed"], _delta=g["delta_packed"],
                                     _emax=g["emax"], _plan=plan, out_features=of, in_features=in_f)

    def streams(m):
        return m._sign, m._mant, m._delta, m._emax

    mq = module(out_f, in_f + L)
    mo = module(o_out_f, 7) if o_out_f else None
    w = (1.0 + 0.1 * rnd(in_f, 3).float()).to(torch.bfloat16).to(DEV)
    n_slots = 37
    kc0, vc0 = rnd((KV, L, 128), 14), rnd((KV, L, 128), 15)
    kA, vA, kB, vB = kc0.to(DEV), vc0.to(DEV), kc0.to(DEV), vc0.to(DEV)
    cs = llama.rope_table(L, 5e5, DEV)
    ws = llama.attention_decode_workspace(H, KV, L, DEV)
    sync = llama.layer_front_sync(DEV, 2)
    qA = torch.empty(out_f, dtype=torch.bfloat16, device=DEV)
    qB = torch.full_like(qA, float("nan"))
    oA = torch.empty(H * 128, dtype=torch.bfloat16, device=DEV)
    oB = torch.full_like(oA, float("nan"))
    if o_out_f:
        n_res = ops.gemv_residual_slots(o_out_f, in_f)
        res = rnd(o_out_f, 4).to(DEV)
        yA, yB = (torch.empty(o_out_f, dtype=torch.bfloat16, device=DEV) for _ in range(2))
        rA, rB = (torch.empty(o_out_f, dtype=torch.bfloat16, device=DEV) for _ in range(2))
        sA, sB = (torch.full((n_res + 2,), float("nan"), device=DEV) for _ in range(2))
    for call, pos in enumerate((L - 1, L // 2, 0, L // 2)):
        h = rnd(in_f, 20 + call).to(DEV)
        slots = (torch.rand(n_slots, generator=torch.Generator().manual_seed(call)) * in_f / n_slots).to(DEV)
        p = torch.tensor([pos], dtype=torch.int32, device=DEV)
        ops.bf16x_gemv_prenormed(h, w, 1e-5, slots, n_slots, *streams(mq), out_f, in_f, plan=mq._plan, out=qA)
        llama.attention_decode(qA, p, cs, H, KV, kA, vA, oA, ws)
        o = None
        if o_out_f:
            ops.bf16x_gemv_residual(oA, res, rA, sA, *streams(mo), o_out_f, in_f, plan=mo._plan, out=yA)
            o = (mo, res, rB, sB, yB)
        llama.layer_front_decode(h, w, 1e-5, slots, n_slots, mq, p, cs, H, KV, kB, vB, qB, oB, sync[call % 2],
                                 sync[1 - call % 2], o=o)
        torch.cuda.synchronize()
        assert not sync[1 - call % 2].any(), call                     # the other buffer cleared
        assert int(sync[call % 2][1024]) == 0, call                   # no wait ran out
        assert torch.equal(qB, qA), call
        assert torch.equal(oB, oA), call
        assert torch.equal(kB, kA) and torch.equal(vB, vA), call
        if o_out_f:
            assert torch.equal(yB, yA) and torch.equal(rB, rA), call
            assert torch.equal(sB[:n_res], sA[:n_res]) and torch.isnan(sB[n_res:]).all(), call


@torch.no_grad()
@pytest.mark.parametrize("pairs8", [False, True])
def test_silu_mul(bx, pairs8):
    T, F = 3, 1536
    gu = rnd((T, 2 * F), 11, 3.0)
    out = torch.empty(T, F, dtype=torch.bfloat16, device=DEV)
    src = gu[:, llama.pairs8_rows(F)].contiguous() if pairs8 else gu
    llama.silu_mul(src.to(DEV), out, F, pairs8=pairs8)
    g, u = gu[:, :F].float(), gu[:, F:].float()
    ref = bf(bf(g * torch.sigmoid(g)) * u)
    within_ulps(out, ref, 1.0)


@torch.no_grad()
@pytest.mark.parametrize("F,in_f,mode", [(1536, 512, "exact"), (14336, 4096, "exact"), (1024, 2048, "saturated"),
                                         (256, 64, "exact")])
def test_gemv_swiglu_matches_unfused(bx, F, in_f, mode):
    """The SwiGLU-epilogue GEMV equals the plain GEMV followed by silu_mul
    (bit for bit: same sums, same roundings) and the fp64 product."""
    from bfloat16x_amd import ops
    bits = dc.bench_weight_bits(2 * F, in_f, seed=12)
    w = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    wp = w[llama.pairs8_rows(F)].contiguous()
    d = bx.bf16x_quantize(wp.to(DEV))
    plan = bx.build_plan_host(d, device=DEV) if mode == "exact" else None
    x = rnd(in_f, 13).to(DEV)
    args = (d["sign_packed"], d["mant_packed"], d["delta_packed"], d["emax"], 2 * F, in_f)
    act = ops.bf16x_gemv_swiglu(x, *args, plan=plan)
    y = ops.bf16x_gemv(x, *args, plan=plan)
    ref = torch.empty(F, dtype=torch.bfloat16, device=DEV)
    llama.silu_mul(y, ref, F, pairs8=True)
    assert torch.equal(act, ref)
    if mode == "exact":
        # fp64 product through the same bf16 rounding chain (gate, up, silu,
        # product): within 3 ulps (the fp32 sums may round gate/up the other way)
        yw = torch.from_numpy(w.double().numpy() @ x.double().cpu().numpy())
        g, u = bf(yw[:F].float()), bf(yw[F:].float())
        ref64 = bf(bf(g * torch.sigmoid(g)) * u)
        within_ulps(act, ref64, 3.0, floor=1e-3 * float(ref64.abs().mean()))


@torch.no_grad()
@pytest.mark.parametrize("V", [3, 100, 1000, 1003, 128256, 140003])
def test_greedy(bx, V):
    """V < 256: most of the 32 workgroups have an empty range."""
    logits = rnd(V, 12)
    logits[V // 3] = 9.0
    logits[V - 1] = 9.0                                  # tie: the first index wins
    tok = torch.zeros(1, dtype=torch.int64, device=DEV)
    state = torch.tensor([50, 0], dtype=torch.int32, device=DEV)
    hist = torch.full((2,), -1, dtype=torch.int32, device=DEV)
    ws = llama.greedy_workspace(DEV)
    lg = logits.to(DEV)
    for _ in range(3):                                   # the third call is past the history: not written
        llama.greedy(lg, tok, state, hist, ws)
    assert int(tok) == V // 3 == int(torch.argmax(logits.float()))
    assert hist.tolist() == [V // 3, V // 3] and state.tolist() == [53, 3]
    assert int(ws[0]) == 0                               # the counter is back at zero


@torch.no_grad()
def test_greedy_two_streams(bx):
    """Two greedy launches in flight at once on two streams, each with its
    own workspace, give each its own argmax."""
    V = 128256
    la, lb = rnd(V, 21).to(DEV), rnd(V, 22).to(DEV)
    la[7], lb[V - 9] = 11.0, 11.0
    outs = []
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    args = []
    for lg in (la, lb):
        args.append((lg, torch.zeros(1, dtype=torch.int64, device=DEV), torch.zeros(2, dtype=torch.int32, device=DEV),
                     torch.zeros(200, dtype=torch.int32, device=DEV), llama.greedy_workspace(DEV)))
    torch.cuda.synchronize()
    for _ in range(100):
        with torch.cuda.stream(sa):
            llama.greedy(*args[0])
        with torch.cuda.stream(sb):
            llama.greedy(*args[1])
    torch.cuda.synchronize()
    assert args[0][3][:100].tolist() == [7] * 100
    assert args[1][3][:100].tolist() == [V - 9] * 100


@torch.no_grad()
@pytest.mark.parametrize("out_f,in_f,swiglu,res", [(6144, 4096, False, True), (28672, 4096, True, True),
                                                  (1024, 512, False, False), (3072, 512, True, True)])
def test_gemv_norm_matches_unfused(bx, out_f, in_f, swiglu, res):
    """RMSNorm folded into the GEMV's staging against the RMSNorm kernel
    followed by the plain (or SwiGLU) GEMV: the stored residual is bit-exact,
    the products agree to the north-star tolerance (the sum of squares is
    reduced in another order, so the scale may differ in its last bit)."""
    from bfloat16x_amd import ops
    from tests.test_gpu_dict import check_tol
    bits = dc.bench_weight_bits(out_f, in_f, seed=14)
    w = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    d = bx.bf16x_quantize(w.to(DEV))
    plan = bx.build_plan_host(d, device=DEV)
    args = (d["sign_packed"], d["mant_packed"], d["delta_packed"], d["emax"], out_f, in_f)
    x, r, nw = rnd(in_f, 15).to(DEV), rnd(in_f, 16).to(DEV), rnd(in_f, 17, 0.5).to(DEV)
    r_out = torch.empty(in_f, dtype=torch.bfloat16, device=DEV)
    y = ops.bf16x_gemv_norm(x, r if res else None, nw, r_out, 1e-5, *args, plan=plan, swiglu=swiglu)
    # unfused
    r2 = r.clone()
    normed = torch.empty(in_f, dtype=torch.bfloat16, device=DEV)
    if res:
        llama.rmsnorm(x, nw, normed, r2, flags=llama.NORM_ADD | llama.NORM_STORE)
        assert torch.equal(r_out, r2)
    else:
        llama.rmsnorm(x, nw, normed)
        assert torch.equal(r_out, x)
    y2 = ops.bf16x_gemv_swiglu(normed, *args, plan=plan) if swiglu else ops.bf16x_gemv(normed, *args, plan=plan)
    check_tol(y.float().cpu().numpy(), y2.double().cpu().numpy())


# --------------------------------------------------------------------------- the stack

SMALL = llama.LlamaConfig(n_layers=2, hidden=512, ffn=1536, n_heads=4, n_kv_heads=2, vocab=1000)


def rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def ref_forward(W, cfg, ids):
    """fp32 CPU forward of the same weights: logits of every position."""
    H, KV, T = cfg.n_heads, cfg.n_kv_heads, len(ids)
    cs = llama.rope_table(T, cfg.rope_theta, "cpu")
    x = W["embed"][ids]
    for lw in W["layers"]:
        h = rms(x, lw["attn_norm"], cfg.eps)
        qkv = (h @ lw["qkv"].T).view(T, H + 2 * KV, 128)
        q, k, v = rope_ref(qkv[:, :H], cs, 0), rope_ref(qkv[:, H:H + KV], cs, 0), qkv[:, H + KV:]
        a = attn_ref(q, k.permute(1, 0, 2), v.permute(1, 0, 2), 0, H, KV).reshape(T, -1)
        x = x + a @ lw["o"].T
        h = rms(x, lw["mlp_norm"], cfg.eps)
        gu = h @ lw["gate_up"].T
        g, u = gu[:, :cfg.ffn], gu[:, cfg.ffn:]
        x = x + (g * torch.sigmoid(g) * u) @ lw["down"].T
    return rms(x, W["norm"], cfg.eps) @ W["lm_head"].T


def host_weights(model):
    """fp32 CPU weights, gate_up back in the natural [gate; up] row order."""
    f = lambda t: t.detach().float().cpu()
    perm = llama.pairs8_rows(model.cfg.ffn)
    layers = []
    for l in model.layers:
        lw = {k: f(getattr(l, k).weight if k in ("qkv", "o", "gate_up", "down") else getattr(l, k))
              for k in ("attn_norm", "mlp_norm", "qkv", "o", "gate_up", "down")}
        nat = torch.empty_like(lw["gate_up"])
        nat[perm] = lw["gate_up"]
        lw["gate_up"] = nat
        layers.append(lw)
    return {"embed": f(model.embed), "norm": f(model.norm), "lm_head": f(model.lm_head.weight), "layers": layers}


@pytest.fixture(scope="module")
def small(bx):
    """(bf16 model, BF16X-deployed copy, host weights, prompt)."""
    m16 = llama.LlamaStack(SMALL, device=DEV, seed=3, std=0.05)
    W = host_weights(m16)
    mx = llama.LlamaStack(SMALL, device=DEV, seed=3, std=0.05)
    total, n_el = bx.deploy_bf16x_fused(mx, verbose=False)
    assert n_el == SMALL.linear_params() and isinstance(mx.layers[0].qkv, bx.Bf16xFused)
    ids = torch.randint(0, SMALL.vocab, (20,), generator=torch.Generator().manual_seed(0))
    return m16, mx, W, ids


@torch.no_grad()
@pytest.mark.parametrize("which", ["bf16", "bf16x"])
def test_prefill_logits_match_fp32_forward(small, which):
    m16, mx, W, ids = small
    r = llama.LlamaRunner(m16 if which == "bf16" else mx, max_len=64, max_new=8, max_prompt=32)
    r.prefill(ids.to(DEV))
    ref = ref_forward(W, SMALL, ids)[-1]
    assert norm_rel(r.logits.float().cpu().numpy(), ref.numpy()) < 2e-2
    assert int(r.token) == int(r.history[0]) and r.state.tolist() == [len(ids), 1]


@torch.no_grad()
def test_decode_steps_match_prefill_over_same_tokens(small):
    _, mx, _, ids = small
    r = llama.LlamaRunner(mx, max_len=64, max_new=8, max_prompt=32)
    toks = r.generate(ids.to(DEV), 6, graph=False)
    last = r.logits.float().cpu().numpy()
    full = torch.cat([ids, torch.tensor(toks[:-1])])              # the token path of the decode
    r2 = llama.LlamaRunner(mx, max_len=64, max_new=8, max_prompt=32)
    r2.prefill(full.to(DEV))
    assert norm_rel(last, r2.logits.float().cpu().numpy()) < 1e-2
    assert int(r2.history[0]) == toks[-1]


@torch.no_grad()
def test_norm_in_gemv_decode_matches_prefill(small):
    """The decode step with every RMSNorm folded into the following GEMV
    (norm_in_gemv) against a prefill over the same tokens, and against the
    unfused decode."""
    _, mx, _, ids = small
    r = llama.LlamaRunner(mx, max_len=64, max_new=8, max_prompt=32, norm_in_gemv=True)
    assert r.fused_norm
    toks = r.generate(ids.to(DEV), 6, graph=False)
    last = r.logits.float().cpu().numpy()
    r2 = llama.LlamaRunner(mx, max_len=64, max_new=8, max_prompt=32)
    r2.prefill(torch.cat([ids, torch.tensor(toks[:-1])]).to(DEV))
    assert norm_rel(last, r2.logits.float().cpu().numpy()) < 1e-2
    r3 = llama.LlamaRunner(mx, max_len=64, max_new=8, max_prompt=32)
    assert not r3.fused_norm
    r3.generate(ids.to(DEV), 6, graph=False)
    assert norm_rel(last, r3.logits.float().cpu().numpy()) < 1e-2


@torch.no_grad()
@pytest.mark.parametrize("out_f,in_f,dense", [(512, 1024, False), (1000, 6144, False), (384, 14336, False),
                                              (4100, 6144, True), (8192, 4096, False), (8200, 6144, True)])
def test_residual_and_prenormed_gemv(bx, out_f, in_f, dense):
    """bf16x_gemv_residual: y bit-identical to bf16x_gemv, residual_out =
    bf16(y + residual_in) bit for bit, the slots add up to sum(h^2).
    bf16x_gemv_prenormed with those slots: the GEMV of the RMSNorm of h within
    the GEMV tolerance (its sum of squares is added in another order than the
    standalone RMSNorm's, so the normalised input may differ by a rounding)."""
    from bfloat16x_amd import ops
    from oracle import dict_codec as dc
    from tests.test_gpu_dict import bits_tensor, check_tol, to_dev
    bits = dc.bench_weight_bits(out_f, in_f, seed=out_f + in_f)
    if dense:                  # 30 % tiny elements: every row has more entries than the read-ahead batches
        tiny = np.random.default_rng(5).random(bits.shape) < 0.3
        bits[tiny] = (bits[tiny] & 0x807F) | 0x0080
    d = bx.bf16x_quantize(bits_tensor(bits))
    g = to_dev(d)
    plan = bx.build_plan_host(d, device=DEV)
    streams = (g["sign_packed"], g["mant_packed"], g["delta_packed"], g["emax"])
    x = rnd(in_f, 1).to(DEV)
    res = rnd(out_f, 2).to(DEV)
    y = bx.bf16x_gemv(x, *streams, out_f, in_f, plan=plan)
    n = ops.gemv_residual_slots(out_f, in_f)
    slots = torch.full((n + 3,), float("nan"), dtype=torch.float32, device=DEV)
    ro = torch.empty(out_f, dtype=torch.bfloat16, device=DEV)
    yr = ops.bf16x_gemv_residual(x, res, ro, slots, *streams, out_f, in_f, plan=plan)
    assert torch.equal(yr, y)
    h = (y.float() + res.float()).to(torch.bfloat16)
    assert torch.equal(ro, h)
    ss = float((h.double() ** 2).sum())
    assert abs(float(slots[:n].double().sum()) - ss) <= 1e-5 * ss
    assert torch.isnan(slots[n:]).all()                           # only the launch's own slots are written
    # the next projection: RMSNorm(h) * w as its input
    if out_f <= 4096 and out_f % 32 == 0:
        nxt = dc.bench_weight_bits(256, out_f, seed=7)
        d2 = bx.bf16x_quantize(bits_tensor(nxt))
        g2 = to_dev(d2)
        p2 = bx.build_plan_host(d2, device=DEV)
        w = (1.0 + 0.1 * rnd(out_f, 3).float()).to(torch.bfloat16).to(DEV)
        normed = torch.empty(out_f, dtype=torch.bfloat16, device=DEV)
        llama.rmsnorm(h, w, normed, eps=1e-5)
        s2 = (g2["sign_packed"], g2["mant_packed"], g2["delta_packed"], g2["emax"])
        ref = bx.bf16x_gemv(normed, *s2, 256, out_f, plan=p2)
        got = ops.bf16x_gemv_prenormed(h, w, 1e-5, slots, n, *s2, 256, out_f, plan=p2)
        check_tol(got.float().cpu().numpy(), ref.float().cpu().numpy().astype(np.float64))


@torch.no_grad()
def test_residual_norm_decode_matches_prefill_and_unfused(small):
    """The default BF16X decode step (residual adds and RMSNorm statistics
    carried by the o / down GEMVs, bf16x_gemv_residual / _prenormed) against
    a prefill over the same tokens and against the decode with standalone
    RMSNorm launches."""
    _, mx, _, ids = small
    r = llama.LlamaRunner(mx, max_len=64, max_new=8, max_prompt=32)
    assert r.res_norm
    toks = r.generate(ids.to(DEV), 6, graph=False)
    last = r.logits.float().cpu().numpy()
    r2 = llama.LlamaRunner(mx, max_len=64, max_new=8, max_prompt=32)
    r2.prefill(torch.cat([ids, torch.tensor(toks[:-1])]).to(DEV))
    assert norm_rel(last, r2.logits.float().cpu().numpy()) < 1e-2
    r3 = llama.LlamaRunner(mx, max_len=64, max_new=8, max_prompt=32, residual_norm=False)
    assert not r3.res_norm and not r3.fused_norm
    r3.generate(ids.to(DEV), 6, graph=False)
    assert norm_rel(last, r3.logits.float().cpu().numpy()) < 1e-2


MID = llama.LlamaConfig(n_layers=3, hidden=4096, ffn=1024, n_heads=32, n_kv_heads=8, vocab=1000)


@torch.no_grad()
def test_layer_front_decode_step(bx):
    """A 3-layer stack of configuration-4 width with a 300-row cache: the
    decode step whose qkv GEMV, attention and o GEMV are one launch per layer
    (the default) gives the same tokens and bit-identical logits as the step
    with separate launches, eager and over HIP-graph replays."""
    mx = llama.LlamaStack(MID, device=DEV, seed=5, std=0.02)
    bx.deploy_bf16x_fused(mx, verbose=False)
    ids = torch.randint(0, MID.vocab, (40,), generator=torch.Generator().manual_seed(1)).to(DEV)
    ra = llama.LlamaRunner(mx, max_len=300, max_new=10, max_prompt=64)
    rb = llama.LlamaRunner(mx, max_len=300, max_new=10, max_prompt=64, layer_front=False)
    assert ra.front and not rb.front
    ta = ra.generate(ids, 10, graph=False)
    la = ra.logits.clone()
    tb = rb.generate(ids, 10, graph=False)
    assert ta == tb and torch.equal(la, rb.logits)
    ra.capture()
    for rep in range(3):
        torch.cuda.synchronize()
        assert ra.generate(ids, 10, graph=True) == ta, rep
        assert torch.equal(ra.logits, la), rep
        assert not ra.front_sync[:, 1024].any()
    # a timed-out wait (its flag, set here from the host) makes the runner raise
    # and clears the flag
    ra.front_sync[1, 1024] = 1
    with pytest.raises(RuntimeError, match="timed out"):
        ra.generate(ids, 10, graph=True)
    assert not ra.front_sync[:, 1024].any()
    assert ra.generate(ids, 10, graph=True) == ta


@torch.no_grad()
def test_graph_decode_matches_eager_over_replays(small):
    _, mx, _, ids = small
    r = llama.LlamaRunner(mx, max_len=64, max_new=12, max_prompt=32)
    eager = r.generate(ids.to(DEV), 12, graph=False)
    eager_logits = r.logits.clone()
    r.capture()
    for rep in range(3):                                          # eager work and syncs between the replays
        torch.cuda.synchronize()
        got = r.generate(ids.to(DEV), 12, graph=True)
        assert got == eager, (rep, got, eager)
        assert torch.equal(r.logits, eager_logits)


@torch.no_grad()
def test_bf16x_stack_tracks_bf16_stack(small):
    """Teacher-forced on the BF16X stack's own tokens, the bf16 stack's
    logits agree at every step (the weights are bit-identical; only the
    accumulation order of the products differs)."""
    m16, mx, _, ids = small
    rx = llama.LlamaRunner(mx, max_len=64, max_new=8, max_prompt=32)
    r16 = llama.LlamaRunner(m16, max_len=64, max_new=8, max_prompt=32)
    rx.prefill(ids.to(DEV))
    r16.prefill(ids.to(DEV))
    for k in range(7):
        assert norm_rel(rx.logits.float().cpu().numpy(), r16.logits.float().cpu().numpy()) < 1e-2, k
        r16.token.copy_(rx.token)
        rx.step()
        r16.step()

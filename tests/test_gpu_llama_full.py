"""Configuration 4 at full size (32 layers, hidden 4096, FFN 14336, 32/8 heads,
vocab 128256): the stack's logits in bf16 and in BF16X, each against an fp32
forward of the same weights over its own token path, computed on the GPU.

The BF16X weights are bit-identical to the bf16 ones (lossless), so both
stacks differ from the fp32 forward only through arithmetic: bf16 storage of
activations between kernels, and the accumulation order of each kernel
(hipBLASLt for the bf16 linears, the fused decode+GEMV / GEMM kernels for
BF16X).  The check is that BF16X adds no error of its own: its distance to
fp32 is within 10 % of the bf16 stack's, position by position on average.
Positions: the last token of three prefills (16, 40 and 256 tokens: the
few-row and the wave-specialised fused GEMMs) and seven greedy decode steps
after the 256-token prefill.  The greedy-agreement check of
the reference's harness (bench_fused_cpm5.py:96-100) compares the two stacks'
tokens; here each stack is also measured against fp32 directly.
"""
import math

import numpy as np
import pytest
import torch

from bfloat16x_amd import llama
from tests.test_gpu_dict import DEV

pytestmark = pytest.mark.gpu

PROMPT = 256
PREFILLS = (16, 40, 256)      # the 256-token prefill runs the wave-specialised GEMM
N_NEW = 8


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


@torch.no_grad()
def fp32_forward(m16, ids):
    """Logits [T, vocab] of every position of ids (int64 [T] on the GPU):
    the bf16 stack's weights upcast to fp32, every operation in fp32."""
    cfg = m16.cfg
    H, KV, D, T = cfg.n_heads, cfg.n_kv_heads, llama.HEAD_DIM, int(ids.numel())
    cs = llama.rope_table(T, cfg.rope_theta, ids.device)
    c, s = cs[:, None, :, 0], cs[:, None, :, 1]

    def rope(t):                                          # rotate-half, positions 0 .. T-1
        a, b = t[..., :64], t[..., 64:]
        return torch.cat([a * c - b * s, b * c + a * s], dim=-1)

    perm = llama.pairs8_rows(cfg.ffn).to(ids.device)     # gate_up rows are stored in PAIRS8 order
    mask = torch.full((T, T), float("-inf"), device=ids.device).triu(1)
    x = m16.embed[ids].float()
    for lay in m16.layers:
        h = _rms(x, lay.attn_norm.float(), cfg.eps)
        qkv = (h @ lay.qkv.weight.float().t()).view(T, H + 2 * KV, D)
        q = rope(qkv[:, :H]).permute(1, 0, 2).contiguous()                                    # [H, T, D]
        k = rope(qkv[:, H:H + KV]).repeat_interleave(H // KV, 1).permute(1, 2, 0).contiguous()  # [H, D, T]
        v = qkv[:, H + KV:].repeat_interleave(H // KV, 1).permute(1, 0, 2).contiguous()        # [H, T, D]
        p = torch.softmax(torch.matmul(q, k) / math.sqrt(D) + mask, dim=-1)
        a = torch.matmul(p, v).permute(1, 0, 2).reshape(T, H * D)
        x = x + a @ lay.o.weight.float().t()
        h = _rms(x, lay.mlp_norm.float(), cfg.eps)
        gu = torch.empty(T, 2 * cfg.ffn, device=ids.device)
        gu[:, perm] = h @ lay.gate_up.weight.float().t()  # natural [gate; up] order
        g, u = gu[:, :cfg.ffn], gu[:, cfg.ffn:]
        x = x + (g * torch.sigmoid(g) * u) @ lay.down.weight.float().t()
    return _rms(x, m16.norm.float(), cfg.eps) @ m16.lm_head.weight.float().t()


def norm_rel(y, r):
    return float(torch.linalg.vector_norm((y - r).double()) / torch.linalg.vector_norm(r.double()))


@torch.no_grad()
def stack_logits(m, ids):
    """Last-token logits of the prefills in PREFILLS, then of the decode steps
    after the full prompt; with the token path the decode took."""
    r = llama.LlamaRunner(m, max_len=PROMPT + N_NEW + 8, max_new=N_NEW, max_prompt=PROMPT)
    out = []
    for T in PREFILLS:
        r.prefill(ids[:T])
        out.append(r.logits.float().clone())
    dec = []
    for k in range(N_NEW - 1):
        r.step()
        dec.append(r.logits.float().clone())
    path = torch.cat([ids, r.history[:N_NEW - 1].to(torch.int64)])
    return out, dec, path


@torch.no_grad()
def test_config4_logits_track_fp32():
    import bfloat16x_amd as bx
    cfg = llama.LlamaConfig()
    print("config 4 stack: building bf16 and BF16X copies", flush=True)
    m16 = llama.LlamaStack(cfg, device=DEV, seed=0)
    mx = llama.LlamaStack(cfg, device=DEV, seed=0)
    bx.deploy_bf16x_fused(mx, verbose=False)
    ids = torch.randint(0, cfg.vocab, (PROMPT,), generator=torch.Generator().manual_seed(0)).to(DEV)
    errs, agree = {}, {}
    for tag, m in (("bf16", m16), ("bf16x", mx)):
        pre, dec, path = stack_logits(m, ids)
        ref = fp32_forward(m16, path)                 # the same weights, this stack's token path
        pos = [T - 1 for T in PREFILLS] + [PROMPT + k for k in range(N_NEW - 1)]
        got = pre + dec
        errs[tag] = [norm_rel(g, ref[p]) for g, p in zip(got, pos)]
        agree[tag] = sum(int(torch.argmax(g)) == int(torch.argmax(ref[p])) for g, p in zip(got, pos))
        print(f"{tag}: logits rel err vs fp32 per position {np.round(errs[tag], 5).tolist()}, "
              f"argmax agreement {agree[tag]}/{len(pos)}", flush=True)
    e16, ex = np.array(errs["bf16"]), np.array(errs["bf16x"])
    print(f"mean rel err: bf16 {e16.mean():.5f}, bf16x {ex.mean():.5f}, ratio {ex.mean() / e16.mean():.3f}",
          flush=True)
    assert ex.mean() <= 1.1 * e16.mean(), (e16.mean(), ex.mean())
    assert ex.max() <= 1.5 * e16.max(), (e16.max(), ex.max())
    assert agree["bf16x"] >= agree["bf16"] - 1

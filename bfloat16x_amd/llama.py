"""Llama-style decoder stack over BF16X linears: the caller of the hot path.

The reference's harness (bench_fused_cpm5.py:27-57) loads a Hugging Face
model, swaps its nn.Linears for Bf16xFused with deploy_bf16x_fused
(bf16x_fused.py:232-263), then runs a KV-cache greedy loop with one
`.item()` host sync per token.  Here the model is a seeded random-init
Llama-style stack (no checkpoint is available), its linears are swapped by
the same deploy_bf16x_fused (bfloat16x_amd.nn), and decoding runs on
device-resident state:

  * the next token, its position and the history live in device memory;
    the decode step reads them there, so one step is a fixed launch
    sequence captured once in a HIP graph (torch.cuda.CUDAGraph) and
    replayed per token with no host synchronisation;
  * the ops between the linears are the kernels of include/bf16x_llama.h:
    per layer RMSNorm(+residual), qkv GEMV, RoPE + KV append + attention
    (one launch per token), o GEMV, RMSNorm(+residual), gate_up GEMV,
    SwiGLU, down GEMV;
  * q/k/v and gate/up are single fused linears, so batch-1 decode runs 4
    GEMVs per layer; gate_up's rows are stored in groups of 8 [gate 4b ..
    4b+3, up 4b .. 4b+3] (pairs8_rows) so that the BF16X gate_up GEMV applies
    SwiGLU in its epilogue (bf16x_gemv_swiglu): 7 launches per layer;
  * by default a BF16X decode step runs 5 launches per layer: the o and down
    GEMVs add their output to the residual stream and leave per-workgroup
    sums of squares (bf16x_gemv_residual), and the qkv / gate_up GEMVs
    normalise their input from those sums (bf16x_gemv_prenormed), so no
    RMSNorm launch remains inside the stack (residual_norm; 3.15 against
    3.21 ms/token with the standalone RMSNorm launches).  norm_in_gemv, where
    every GEMV workgroup also recomputes the sum of squares itself, measured
    no faster and is off by default.

Shapes of the benchmark configuration (the defaults of LlamaConfig): 32
layers, hidden 4096, FFN 14336 (SwiGLU), 32 query / 8 KV heads, head_dim 128,
vocab 128256, RoPE theta 5e5, RMSNorm weights 1; all linear weights
N(0, 0.02) in bf16; embedding and lm_head bf16 N(0, 0.02), not compressed
(the reference's deploy skips "lm_head" and "embed").
"""
from __future__ import annotations

import dataclasses
import math

import torch
from torch import nn

from . import _lib, ops

__all__ = ["LlamaConfig", "LlamaStack", "LlamaRunner", "rope_table", "rmsnorm", "rope_kv", "attention", "pairs8_rows",
           "attention_decode", "attention_decode_supported", "attention_decode_workspace", "layer_front_decode",
           "layer_front_supported", "layer_front_sync", "layer_front_buffers", "silu_mul", "greedy", "greedy_workspace", "NORM_ADD", "NORM_STORE"]

NORM_ADD, NORM_STORE = 1, 2
HEAD_DIM = 128


@dataclasses.dataclass(frozen=True)
class LlamaConfig:
    n_layers: int = 32
    hidden: int = 4096
    ffn: int = 14336
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = HEAD_DIM
    vocab: int = 128256
    rope_theta: float = 5e5
    eps: float = 1e-5

    def __post_init__(self):
        if self.head_dim != HEAD_DIM:
            raise ValueError("head_dim must be 128")
        if self.n_heads % self.n_kv_heads or self.n_heads * self.head_dim != self.hidden:
            raise ValueError("n_heads * head_dim must equal hidden and n_kv_heads must divide n_heads")
        if self.hidden % 32 or self.ffn % 32 or self.vocab % 8 or self.hidden > 8192:
            raise ValueError("hidden, ffn must be multiples of 32 (hidden <= 8192), vocab of 8")

    @property
    def qkv_rows(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim

    def linear_shapes(self):
        """(name, out_f, in_f) of one layer's linears."""
        return [("qkv", self.qkv_rows, self.hidden), ("o", self.hidden, self.hidden),
                ("gate_up", 2 * self.ffn, self.hidden), ("down", self.hidden, self.ffn)]

    def linear_params(self) -> int:
        return self.n_layers * sum(o * i for _, o, i in self.linear_shapes())


# ---------------------------------------------------------------------------
# thin wrappers of include/bf16x_llama.h (shapes are checked here: the
# kernels trust the buffer sizes they are given)

def _stream(t: torch.Tensor):
    return _lib.stream_of(t.device)


def _need(cond: bool, what: str):
    if not cond:
        raise ValueError(what)


def _bf16_dev(t, name):
    _need(isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.bfloat16 and t.is_contiguous(),
          f"{name} must be a contiguous bf16 GPU tensor")


def rmsnorm(x, weight, out, residual=None, row_idx=None, flags=0, eps=1e-5):
    """out = RMSNorm(h) * weight with h = x (or x[row_idx], a gather) plus,
    with NORM_ADD, the residual; NORM_STORE writes h back to the residual."""
    n = weight.numel()
    for t, nm in ((x, "x"), (weight, "weight"), (out, "out")):
        _bf16_dev(t, nm)
    _need(x.numel() % n == 0, "x is not a whole number of rows")
    if row_idx is not None:
        _need(row_idx.is_cuda and row_idx.dtype == torch.int64 and row_idx.is_contiguous(), "row_idx: int64 GPU")
        rows = row_idx.numel()
    else:
        rows = x.numel() // n
    _need(out.numel() >= rows * n, "out too small")
    if flags:
        _bf16_dev(residual, "residual")
        _need(residual.numel() >= rows * n, "residual too small")
    st = _lib.lib().bf16x_rmsnorm(x.data_ptr(), _lib.ptr(row_idx), x.numel() // n,
                                  residual.data_ptr() if residual is not None else None, weight.data_ptr(),
                                  out.data_ptr(), rows, n, float(eps), int(flags), _stream(x))
    _lib.check(st, "bf16x_rmsnorm")


def _check_pos(pos):
    _need(pos.is_cuda and pos.dtype == torch.int32 and pos.numel() >= 1, "pos: int32 GPU tensor")


def rope_kv(qkv, pos, cos_sin, n_heads, n_kv_heads, q_out, k_cache, v_cache):
    """RoPE of the q/k heads of qkv [tokens, (H + 2 KV) * 128] at positions
    pos[0] + t; q to q_out, k and v appended to the [KV, max_len, 128]
    caches."""
    for t, nm in ((qkv, "qkv"), (q_out, "q_out"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _bf16_dev(t, nm)
    _check_pos(pos)
    row = (n_heads + 2 * n_kv_heads) * HEAD_DIM
    _need(qkv.numel() % row == 0, "qkv is not a whole number of tokens")
    tokens = qkv.numel() // row
    max_len = k_cache.numel() // (n_kv_heads * HEAD_DIM)
    _need(k_cache.numel() == max_len * n_kv_heads * HEAD_DIM and v_cache.numel() == k_cache.numel(), "cache shape")
    _need(q_out.numel() >= tokens * n_heads * HEAD_DIM, "q_out too small")
    _need(cos_sin.is_cuda and cos_sin.dtype == torch.float32 and cos_sin.numel() == max_len * HEAD_DIM,
          "cos_sin must be fp32 [max_len, 64, 2] on the GPU")
    st = _lib.lib().bf16x_rope_kv(qkv.data_ptr(), tokens, pos.data_ptr(), cos_sin.data_ptr(), n_heads, n_kv_heads,
                                  HEAD_DIM, max_len, q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                  _stream(qkv))
    _lib.check(st, "bf16x_rope_kv")


def attention(q, k_cache, v_cache, pos, n_heads, n_kv_heads, out, scale=None, tokens=None):
    """Causal GQA attention of `tokens` queries at positions pos[0] + t over
    the caches; out [tokens, n_heads * 128]."""
    for t, nm in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache"), (out, "out")):
        _bf16_dev(t, nm)
    _check_pos(pos)
    if tokens is None:
        tokens = q.numel() // (n_heads * HEAD_DIM)
    max_len = k_cache.numel() // (n_kv_heads * HEAD_DIM)
    _need(k_cache.numel() == max_len * n_kv_heads * HEAD_DIM and v_cache.numel() == k_cache.numel(), "cache shape")
    _need(q.numel() >= tokens * n_heads * HEAD_DIM and out.numel() >= tokens * n_heads * HEAD_DIM, "q/out size")
    scale = 1.0 / math.sqrt(HEAD_DIM) if scale is None else scale
    st = _lib.lib().bf16x_attention(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), pos.data_ptr(), tokens,
                                    n_heads, n_kv_heads, HEAD_DIM, max_len, float(scale), out.data_ptr(), _stream(q))
    _lib.check(st, "bf16x_attention")


def attention_decode_supported(n_heads, n_kv_heads, max_len) -> bool:
    return int(_lib.lib().bf16x_attention_decode_lds(n_heads, n_kv_heads, max_len)) >= 0


def attention_decode_workspace(n_heads, n_kv_heads, max_len, device) -> torch.Tensor:
    """Zeroed workspace of attention_decode (its counters must start at zero;
    every call leaves them zero)."""
    nbytes = int(_lib.lib().bf16x_attention_decode_workspace(n_heads, n_kv_heads, max_len))
    _need(nbytes > 0, "attention_decode does not support this shape")
    return torch.zeros(nbytes // 4 + 1, dtype=torch.int32, device=device)


def attention_decode(qkv, pos, cos_sin, n_heads, n_kv_heads, k_cache, v_cache, out, workspace, scale=None):
    """One decode token: rope_kv + attention (tokens = 1) in one launch.  Up to
    256 cache rows one workgroup per KV head takes all keys; longer caches
    split the keys over workgroups that combine through `workspace`
    (attention_decode_workspace)."""
    for t, nm in ((qkv, "qkv"), (k_cache, "k_cache"), (v_cache, "v_cache"), (out, "out")):
        _bf16_dev(t, nm)
    _check_pos(pos)
    _need(qkv.numel() == (n_heads + 2 * n_kv_heads) * HEAD_DIM, "qkv must hold one token")
    max_len = k_cache.numel() // (n_kv_heads * HEAD_DIM)
    _need(k_cache.numel() == max_len * n_kv_heads * HEAD_DIM and v_cache.numel() == k_cache.numel(), "cache shape")
    _need(out.numel() >= n_heads * HEAD_DIM, "out too small")
    _need(cos_sin.is_cuda and cos_sin.dtype == torch.float32 and cos_sin.numel() == max_len * HEAD_DIM,
          "cos_sin must be fp32 [max_len, 64, 2] on the GPU")
    _need(workspace.is_cuda and workspace.is_contiguous(), "workspace must be a contiguous GPU tensor")
    scale = 1.0 / math.sqrt(HEAD_DIM) if scale is None else scale
    st = _lib.lib().bf16x_attention_decode(qkv.data_ptr(), pos.data_ptr(), cos_sin.data_ptr(), n_heads, n_kv_heads,
                                           HEAD_DIM, max_len, float(scale), k_cache.data_ptr(), v_cache.data_ptr(),
                                           workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                                           out.data_ptr(), _stream(qkv))
    _lib.check(st, "bf16x_attention_decode")


def layer_front_supported(n_heads, n_kv_heads, max_len, out_f, in_f, cus=None) -> bool:
    """Shapes bf16x_layer_front_decode takes (the per-query-head attention,
    one wave per qkv row with two 64-atom steps).  cus: the device's compute
    units, when known: the waiting attention workgroups (one per query
    head) may hold at most half of them."""
    return (n_heads % 8 == 0 and n_heads <= 128 and n_heads % n_kv_heads == 0 and 256 < max_len <= 768
            and in_f % 32 == 0 and 2048 < in_f <= 4096 and out_f == (n_heads + 2 * n_kv_heads) * HEAD_DIM
            and (cus is None or 2 * n_heads <= cus))


def layer_front_sync(device, n: int = 1) -> torch.Tensor:
    """n zeroed counter buffers of layer_front_decode, one per row (word 1024
    of a row: the timeout flag)."""
    words = int(_lib.lib().bf16x_layer_front_sync_bytes()) // 4
    words = -(-words // 4) * 4                                   # rows 16-byte aligned
    return torch.zeros(n, words, dtype=torch.int32, device=device)


def layer_front_buffers(n_launches: int) -> list:
    """Counter buffer of each of the n_launches layer launches of a decode
    step (n_launches >= 2): launch k uses buffer c[k] and clears c[k - 1]
    (cyclically: the step repeats), so c[k] != c[k - 1] for every k,
    including c[0] != c[-1]; three buffers cover any count."""
    if n_launches < 2:
        raise ValueError("a decode step needs at least two layer launches (each clears its predecessor's counters)")
    return [k % 2 for k in range(n_launches - 1)] + [2]


def _dict_args(mod):
    plan = mod._plan
    return (mod._sign.data_ptr(), mod._sign.numel(), mod._mant.data_ptr(), mod._mant.numel(), mod._delta.data_ptr(),
            mod._delta.numel(), mod._emax.data_ptr(), mod._emax.numel(), _lib.ptr(plan.tile_off) if plan else None,
            _lib.ptr(plan.tile_ent) if plan else None, _lib.ptr(plan.tile_sat) if plan else None)


def layer_front_decode(h, norm_weight, eps, slots, n_slots, mod, pos, cos_sin, n_heads, n_kv_heads, k_cache,
                       v_cache, qkv_out, attn_out, sync, sync_clear=None, o=None, scale=None):
    """bf16x_gemv_prenormed(h, ...) of the qkv module `mod` into qkv_out, then
    attention_decode into attn_out and, with o = (o_mod, residual_in,
    residual_out, o_slots, o_y), bf16x_gemv_residual(attn_out, ...) of the o
    module, in one launch (bf16x_layer_front_decode).  `sync` must be zero;
    the launch zeroes `sync_clear` (the previous launch's buffer)."""
    for t, nm in ((h, "h"), (norm_weight, "norm_weight"), (qkv_out, "qkv_out"), (k_cache, "k_cache"),
                  (v_cache, "v_cache"), (attn_out, "attn_out")):
        _bf16_dev(t, nm)
    _check_pos(pos)
    out_f, in_f = mod.out_features, mod.in_features
    max_len = k_cache.numel() // (n_kv_heads * HEAD_DIM)
    _need(layer_front_supported(n_heads, n_kv_heads, max_len, out_f, in_f), "shape not supported")
    _need(h.numel() == in_f and norm_weight.numel() == in_f, "h / norm_weight must hold in_f values")
    _need(qkv_out.numel() == out_f and attn_out.numel() >= n_heads * HEAD_DIM, "qkv_out / attn_out size")
    _need(k_cache.numel() == max_len * n_kv_heads * HEAD_DIM and v_cache.numel() == k_cache.numel(), "cache shape")
    _need(cos_sin.is_cuda and cos_sin.dtype == torch.float32 and cos_sin.numel() == max_len * HEAD_DIM,
          "cos_sin must be fp32 [max_len, 64, 2] on the GPU")
    _need(slots.is_cuda and slots.dtype == torch.float32 and slots.numel() >= n_slots, "slots")
    nbytes = int(_lib.lib().bf16x_layer_front_sync_bytes())
    for t in (sync,) + ((sync_clear,) if sync_clear is not None else ()):
        _need(t.is_cuda and t.is_contiguous() and t.numel() * t.element_size() >= nbytes, "sync buffers")
    o_args = (None,) * 3 + (0,) + (None, 0) * 4 + (None,) * 3 + (0, None)
    if o is not None:
        o_mod, res_in, res_out, o_slots, o_y = o
        _need(o_mod.in_features == in_f, "o projection must take in_f inputs")
        for t, nm in ((res_in, "residual_in"), (res_out, "residual_out"), (o_y, "o_y")):
            _bf16_dev(t, nm)
            _need(t.numel() == o_mod.out_features, f"{nm} must hold o.out_features values")
        _need(o_slots.is_cuda and o_slots.dtype == torch.float32, "o_slots must be fp32 on the GPU")
        o_args = (res_in.data_ptr(), res_out.data_ptr(), o_slots.data_ptr(), o_slots.numel()) + \
            _dict_args(o_mod) + (o_mod.out_features, o_y.data_ptr())
    plan = mod._plan
    scale = 1.0 / math.sqrt(HEAD_DIM) if scale is None else scale
    st = _lib.lib().bf16x_layer_front_decode(
        h.data_ptr(), norm_weight.data_ptr(), float(eps), slots.data_ptr(), int(n_slots), *_dict_args(mod), out_f,
        in_f, _lib.EXACT if plan is not None else _lib.SATURATED, qkv_out.data_ptr(), pos.data_ptr(),
        cos_sin.data_ptr(), n_heads, n_kv_heads, HEAD_DIM, max_len, float(scale), k_cache.data_ptr(),
        v_cache.data_ptr(), attn_out.data_ptr(), *o_args, sync.data_ptr(),
        sync_clear.data_ptr() if sync_clear is not None else None, nbytes, _stream(h))
    _lib.check(st, "bf16x_layer_front_decode")


def pairs8_rows(ffn: int) -> torch.Tensor:
    """Natural row of each row of a PAIRS8 gate_up weight: groups of 8 rows
    [gate 4b .. 4b+3, up 4b .. 4b+3] from the natural [gate; up] order."""
    b = torch.arange(ffn // 4).repeat_interleave(8) * 4
    k = torch.arange(8).repeat(ffn // 4)
    return torch.where(k < 4, b + k, ffn + b + k - 4)


def silu_mul(gate_up, out, ffn, pairs8=False):
    """out[t] = silu(gate) * up of gate_up row t: natural [gate | up] columns,
    or (pairs8) groups of 8 [gate 4b .. 4b+3 | up 4b .. 4b+3]."""
    _bf16_dev(gate_up, "gate_up")
    _bf16_dev(out, "out")
    _need(gate_up.numel() % (2 * ffn) == 0, "gate_up is not a whole number of tokens")
    tokens = gate_up.numel() // (2 * ffn)
    _need(out.numel() >= tokens * ffn, "out too small")
    st = _lib.lib().bf16x_silu_mul(gate_up.data_ptr(), tokens, ffn, 1 if pairs8 else 0, out.data_ptr(),
                                   _stream(gate_up))
    _lib.check(st, "bf16x_silu_mul")


def greedy_workspace(device) -> torch.Tensor:
    """A zeroed workspace for greedy() (the launch's counter and partial
    results); every call puts the counter, word 0, back to zero."""
    n = int(_lib.lib().bf16x_greedy_workspace_bytes())
    return torch.zeros(-(-n // 16) * 4, dtype=torch.int32, device=device)


def greedy(logits, token, state, history, workspace):
    """token[0] = argmax(logits); history[state[1]] = token; state += 1.
    workspace: greedy_workspace(); calls that share one must not overlap."""
    _bf16_dev(logits, "logits")
    _need(token.is_cuda and token.dtype == torch.int64 and token.numel() >= 1, "token: int64 GPU")
    _need(state.is_cuda and state.dtype == torch.int32 and state.numel() >= 2, "state: int32[2] GPU")
    _need(history.is_cuda and history.dtype == torch.int32, "history: int32 GPU")
    _need(workspace.is_cuda and workspace.is_contiguous(), "workspace: greedy_workspace() on the GPU")
    st = _lib.lib().bf16x_greedy(logits.data_ptr(), logits.numel(), token.data_ptr(), state.data_ptr(),
                                 history.data_ptr(), history.numel(), workspace.data_ptr(),
                                 workspace.numel() * workspace.element_size(), _stream(logits))
    _lib.check(st, "bf16x_greedy")


def rope_table(max_len: int, theta: float, device) -> torch.Tensor:
    """fp32 [max_len, 64, 2] (cos, sin) of position x inverse frequency, the
    Hugging Face Llama construction: inv_freq = 1 / theta^(2i/128) and the
    angle product in fp32."""
    inv = 1.0 / (theta ** (torch.arange(0, HEAD_DIM, 2, dtype=torch.int64).float() / HEAD_DIM))
    ang = torch.outer(torch.arange(max_len, dtype=torch.float32), inv)
    return torch.stack([ang.cos(), ang.sin()], dim=-1).contiguous().to(device)


# ---------------------------------------------------------------------------
# the model

def _norm_gemv_ok(mod) -> bool:
    """A deployed BF16X linear the one-wave-per-row GEMV variants can run."""
    from .nn import Bf16xFused
    return (isinstance(mod, Bf16xFused) and mod.mode == "fused" and mod._bias is None
            and mod.in_features <= 4096)


def _swiglu_gemv_ok(mod) -> bool:
    """A deployed BF16X gate_up the SwiGLU-epilogue GEMV can run."""
    return _norm_gemv_ok(mod) and mod.out_features % 8 == 0


def _residual_gemv_ok(mod) -> bool:
    """A deployed BF16X o / down projection the residual-epilogue GEMV can run,
    with few enough slots (<= 1024) for bf16x_gemv_prenormed to read."""
    from .nn import Bf16xFused
    n = int(_lib.lib().bf16x_gemv_residual_slots(mod.out_features, mod.in_features)) \
        if isinstance(mod, Bf16xFused) else -1
    return isinstance(mod, Bf16xFused) and mod.mode == "fused" and mod._bias is None and 0 < n <= 1024


def _device(device):
    if device is None:
        if not torch.cuda.is_available():
            raise RuntimeError("the Llama harness runs on the GPU only")
        device = torch.device("cuda", torch.cuda.current_device())
    return torch.device(device)


def _linear(w: torch.Tensor) -> nn.Linear:
    lin = nn.Linear(w.shape[1], w.shape[0], bias=False, device="meta")
    lin.weight = nn.Parameter(w, requires_grad=False)
    return lin


class LlamaStack(nn.Module):
    """Random-init Llama-style decoder stack (bf16 nn.Linears until
    deploy_bf16x_fused replaces them).  Weights come from a device generator
    seeded per tensor, so the model does not depend on construction order."""

    def __init__(self, cfg: LlamaConfig = LlamaConfig(), device=None, seed: int = 0, std: float = 0.02):
        super().__init__()
        dev = _device(device)
        self.cfg = cfg
        g = torch.Generator(device=dev)

        def rnd(shape, k):
            g.manual_seed(seed * 1_000_003 + k)
            return (torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * std).to(torch.bfloat16)

        ones = lambda: nn.Parameter(torch.ones(cfg.hidden, dtype=torch.bfloat16, device=dev), requires_grad=False)
        self.embed = nn.Parameter(rnd((cfg.vocab, cfg.hidden), 1), requires_grad=False)
        self.layers = nn.ModuleList()
        perm = pairs8_rows(cfg.ffn).to(dev)
        for i in range(cfg.n_layers):
            lay = nn.Module()
            lay.attn_norm = ones()
            lay.mlp_norm = ones()
            for j, (name, o, n) in enumerate(cfg.linear_shapes()):
                w = rnd((o, n), 16 + 8 * i + j)
                if name == "gate_up":             # rows in PAIRS8 order (pairs8_rows)
                    w = w[perm].contiguous()
                setattr(lay, name, _linear(w))
            self.layers.append(lay)
        self.norm = ones()
        self.lm_head = _linear(rnd((cfg.vocab, cfg.hidden), 2))

    @property
    def device(self):
        return self.embed.device


class LlamaRunner:
    """Prefill + greedy decode over a LlamaStack whose linears are bf16
    nn.Linear or BF16X modules (anything mapping [.., in] -> [.., out]).

    Device state: `token` (int64 [1], the next input), `state` (int32 [2]:
    position of `token`, number of tokens in `history`), `history` (int32
    [max_new]).  prefill() fills the caches with the prompt and emits the
    first token; each decode step consumes `token`, appends one token to the
    history and advances the position."""

    def __init__(self, model: LlamaStack, max_len: int, max_new: int, max_prompt: int | None = None,
                 norm_in_gemv: bool = False, residual_norm: bool = True, layer_front: bool = True):
        cfg = model.cfg
        self.model, self.cfg = model, cfg
        dev = model.device
        if max_len > 16384:
            raise ValueError("max_len <= 16384 (attention scores are kept in LDS)")
        self.max_len, self.max_new = int(max_len), int(max_new)
        self.max_prompt = int(max_prompt if max_prompt is not None else max_len)
        T = max(self.max_prompt, 1)
        bf = dict(dtype=torch.bfloat16, device=dev)
        self.k_cache = torch.zeros(cfg.n_layers, cfg.n_kv_heads, self.max_len, HEAD_DIM, **bf)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.cos_sin = rope_table(self.max_len, cfg.rope_theta, dev)
        self.residual = torch.empty(T, cfg.hidden, **bf)
        self.normed = torch.empty(T, cfg.hidden, **bf)
        self.q = torch.empty(T, cfg.n_heads * HEAD_DIM, **bf)
        self.attn = torch.empty(T, cfg.n_heads * HEAD_DIM, **bf)
        self.act = torch.empty(T, cfg.ffn, **bf)
        self.token = torch.zeros(1, dtype=torch.int64, device=dev)
        self.state = torch.zeros(2, dtype=torch.int32, device=dev)
        self.history = torch.zeros(max(self.max_new, 1), dtype=torch.int32, device=dev)
        self.greedy_ws = greedy_workspace(dev)
        self.zero_pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.logits = None
        self.graph = None
        self._graph_logits = None
        # one-token steps fold RoPE + KV append into one attention launch per KV head
        self.fused_decode_attention = attention_decode_supported(cfg.n_heads, cfg.n_kv_heads, self.max_len)
        self.dec_ws = (attention_decode_workspace(cfg.n_heads, cfg.n_kv_heads, self.max_len, dev)
                       if self.fused_decode_attention else None)
        # norm_in_gemv: decode with the RMSNorms folded into the following GEMVs (bf16x_gemv_norm).  Off by
        # default: each of the ~900 workgroups of a GEMV recomputes the norm of the whole row before its
        # first weight row, which costs as much as the standalone RMSNorm launch it saves (measured: gate_up
        # 40.2 us vs 32.5 + 5.3 us, qkv 14.7 vs 15.3 us; 3.43 vs 3.37 ms/token)
        self.fused_norm = bool(norm_in_gemv) and self.fused_decode_attention and all(
            _norm_gemv_ok(lay.qkv) and _swiglu_gemv_ok(lay.gate_up) for lay in model.layers)
        # residual_norm (default, BF16X stacks): the o and down GEMVs add their output to the residual stream
        # and leave per-workgroup sums of squares (bf16x_gemv_residual); the next qkv / gate_up GEMV normalises
        # its input from them (bf16x_gemv_prenormed): no RMSNorm launch inside the stack, 5 launches per layer
        self.res_norm = (bool(residual_norm) and not self.fused_norm and self.fused_decode_attention and all(
            _norm_gemv_ok(lay.qkv) and _swiglu_gemv_ok(lay.gate_up) and _residual_gemv_ok(lay.o)
            and _residual_gemv_ok(lay.down) for lay in model.layers))
        self.res_a = torch.empty(cfg.hidden, **bf)
        self.res_b = torch.empty(cfg.hidden, **bf)
        self.qkv_buf = torch.empty(cfg.qkv_rows, **bf)
        if self.res_norm:
            lay0 = model.layers[0]
            self.n_slots_o = ops.gemv_residual_slots(lay0.o.out_features, lay0.o.in_features)
            self.n_slots_down = ops.gemv_residual_slots(lay0.down.out_features, lay0.down.in_features)
            self.slots = torch.zeros(max(self.n_slots_o, self.n_slots_down), dtype=torch.float32, device=dev)
            self.proj_out = torch.empty(cfg.hidden, **bf)     # o / down outputs (only h is used)
        # layer_front (default, residual_norm stacks of 3 layers or more): layers after the first run the qkv
        # GEMV, the decode attention and the o GEMV as one launch (bf16x_layer_front_decode).  Launch i (layer
        # i + 1) uses counter buffer c(i) and zeroes its predecessor's, so consecutive launches, cyclically over
        # the step (the graph repeats it), must differ: c = 0, 1, 0, 1, ..., and 2 for the last launch
        lay0 = model.layers[0]
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        self.front = bool(layer_front) and self.res_norm and cfg.n_layers >= 3 and layer_front_supported(
            cfg.n_heads, cfg.n_kv_heads, self.max_len, lay0.qkv.out_features, lay0.qkv.in_features, cus) and \
            lay0.o.in_features == lay0.qkv.in_features
        if self.front:
            self.front_sync = layer_front_sync(dev, 3)
            self.front_buf = layer_front_buffers(cfg.n_layers - 1)
        self._prompt_len = 0

    def _decode_fused(self, pos: torch.Tensor, ids: torch.Tensor):
        """One decode token with every RMSNorm after the first folded into the
        following GEMV's x staging (bf16x_gemv_norm) and SwiGLU into the
        gate_up GEMV: per layer qkv GEMV, attention, o GEMV, gate_up GEMV,
        down GEMV (5 launches).  The residual stream alternates between two
        one-row buffers (a GEMV stores x + residual to the other one)."""
        cfg, m = self.cfg, self.model
        H, KV = cfg.n_heads, cfg.n_kv_heads
        R = (self.res_a, self.res_b)
        cur = 0
        rmsnorm(m.embed, m.layers[0].attn_norm, self.normed, R[0], row_idx=ids, flags=NORM_STORE, eps=cfg.eps)
        prev = None
        for i, lay in enumerate(m.layers):
            q = lay.qkv
            if i == 0:
                qkv = q(self.normed[0])
            else:
                qkv = ops.bf16x_gemv_norm(prev, R[cur], lay.attn_norm, R[1 - cur], cfg.eps, q._sign, q._mant,
                                          q._delta, q._emax, q.out_features, q.in_features, plan=q._plan,
                                          out=self.qkv_buf)
                cur = 1 - cur
            attention_decode(qkv, pos, self.cos_sin, H, KV, self.k_cache[i], self.v_cache[i], self.attn, self.dec_ws)
            o = lay.o(self.attn[0])
            g = lay.gate_up
            ops.bf16x_gemv_norm(o, R[cur], lay.mlp_norm, R[1 - cur], cfg.eps, g._sign, g._mant, g._delta, g._emax,
                                g.out_features, g.in_features, plan=g._plan, swiglu=True, out=self.act[0])
            cur = 1 - cur
            prev = lay.down(self.act[0])
        return prev, R[cur]

    def _decode_resnorm(self, pos: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
        """One decode token with the residual adds and the RMSNorm statistics
        carried by the projections: per layer qkv GEMV (normalising its input
        from the previous down GEMV's sums of squares; the first layer takes
        the embedding's RMSNorm), attention, o GEMV (+ residual, sums of
        squares), gate_up GEMV (normalised input, SwiGLU), down GEMV (+
        residual, sums of squares); with layer_front the qkv GEMV, the
        attention and the o GEMV of every layer after the first are one
        launch.  Returns h after the last layer."""
        cfg, m = self.cfg, self.model
        H, KV = cfg.n_heads, cfg.n_kv_heads
        R = (self.res_a, self.res_b)
        cur = 0
        rmsnorm(m.embed, m.layers[0].attn_norm, self.normed, R[0], row_idx=ids, flags=NORM_STORE, eps=cfg.eps)
        for i, lay in enumerate(m.layers):
            q, o, g, d = lay.qkv, lay.o, lay.gate_up, lay.down
            if self.front and i > 0:
                fb = self.front_buf              # launch i - 1: its buffer, then its predecessor's (cyclic)
                layer_front_decode(R[cur], lay.attn_norm, cfg.eps, self.slots, self.n_slots_down, q, pos,
                                   self.cos_sin, H, KV, self.k_cache[i], self.v_cache[i], self.qkv_buf, self.attn[0],
                                   self.front_sync[fb[i - 1]], self.front_sync[fb[i - 2]],
                                   o=(o, R[cur], R[1 - cur], self.slots, self.proj_out))
            else:
                if i == 0:
                    qkv = q(self.normed[0])
                else:
                    qkv = ops.bf16x_gemv_prenormed(R[cur], lay.attn_norm, cfg.eps, self.slots, self.n_slots_down,
                                                   q._sign, q._mant, q._delta, q._emax, q.out_features, q.in_features,
                                                   plan=q._plan, out=self.qkv_buf)
                attention_decode(qkv, pos, self.cos_sin, H, KV, self.k_cache[i], self.v_cache[i], self.attn,
                                 self.dec_ws)
                ops.bf16x_gemv_residual(self.attn[0], R[cur], R[1 - cur], self.slots, o._sign, o._mant, o._delta,
                                        o._emax, o.out_features, o.in_features, plan=o._plan, out=self.proj_out)
            cur = 1 - cur
            ops.bf16x_gemv_prenormed(R[cur], lay.mlp_norm, cfg.eps, self.slots, self.n_slots_o, g._sign, g._mant,
                                     g._delta, g._emax, g.out_features, g.in_features, plan=g._plan, swiglu=True,
                                     out=self.act[0])
            ops.bf16x_gemv_residual(self.act[0], R[cur], R[1 - cur], self.slots, d._sign, d._mant, d._delta, d._emax,
                                    d.out_features, d.in_features, plan=d._plan, out=self.proj_out)
            cur = 1 - cur
        return R[cur]

    # one pass over the stack for `T` tokens starting at position pos[0]
    def _layers(self, T: int, pos: torch.Tensor, ids: torch.Tensor):
        cfg, m = self.cfg, self.model
        H, KV = cfg.n_heads, cfg.n_kv_heads
        one = T == 1

        def rows(buf):                    # decode feeds 1-D rows: the linears take the GEMV path
            return buf[0] if one else buf[:T]

        prev = None
        for i, lay in enumerate(m.layers):
            if i == 0:
                rmsnorm(m.embed, lay.attn_norm, self.normed, self.residual, row_idx=ids, flags=NORM_STORE,
                        eps=cfg.eps)
            else:
                rmsnorm(prev, lay.attn_norm, self.normed, self.residual, flags=NORM_ADD | NORM_STORE, eps=cfg.eps)
            qkv = lay.qkv(rows(self.normed))
            if one and self.fused_decode_attention:
                attention_decode(qkv, pos, self.cos_sin, H, KV, self.k_cache[i], self.v_cache[i], self.attn,
                                 self.dec_ws)
            else:
                rope_kv(qkv, pos, self.cos_sin, H, KV, self.q, self.k_cache[i], self.v_cache[i])
                attention(self.q, self.k_cache[i], self.v_cache[i], pos, H, KV, self.attn, tokens=T)
            o = lay.o(rows(self.attn))
            rmsnorm(o, lay.mlp_norm, self.normed, self.residual, flags=NORM_ADD | NORM_STORE, eps=cfg.eps)
            gu_mod = lay.gate_up
            if one and _swiglu_gemv_ok(gu_mod):
                # fused decode+GEMV with the SwiGLU epilogue: no gate_up round trip, one launch
                ops.bf16x_gemv_swiglu(self.normed[0], gu_mod._sign, gu_mod._mant, gu_mod._delta, gu_mod._emax,
                                      gu_mod.out_features, gu_mod.in_features, plan=gu_mod._plan, out=self.act[0])
            else:
                silu_mul(gu_mod(rows(self.normed)), self.act, cfg.ffn, pairs8=True)
            prev = lay.down(rows(self.act))
        return prev

    def _head(self, last_down: torch.Tensor, last_res: torch.Tensor):
        rmsnorm(last_down, self.model.norm, self.normed, last_res, flags=NORM_ADD, eps=self.cfg.eps)
        self.logits = self.model.lm_head(self.normed[0])
        greedy(self.logits, self.token, self.state, self.history, self.greedy_ws)

    @torch.no_grad()
    def prefill(self, ids: torch.Tensor) -> None:
        """Run the prompt (int64 token ids on the device), emit the first
        token: afterwards state = (len(ids), 1), history[0] = token."""
        T = int(ids.numel())
        if not (1 <= T <= self.max_prompt) or T + self.max_new > self.max_len:
            raise ValueError(f"prompt of {T} tokens: need 1 <= T <= {self.max_prompt} and T + max_new <= max_len")
        if ids.dtype != torch.int64 or not ids.is_cuda:
            raise ValueError("ids must be int64 on the GPU")
        ids = ids.reshape(-1).contiguous()
        self.state.copy_(torch.tensor([T - 1, 0], dtype=torch.int32))
        self._prompt_len = T
        down = self._layers(T, self.zero_pos, ids)
        self._head(down.reshape(T, -1)[T - 1], self.residual[T - 1])

    @torch.no_grad()
    def step(self) -> None:
        """One eager decode step."""
        if self.fused_norm:
            down, res = self._decode_fused(self.state, self.token)
            self._head(down, res)
            return
        if self.res_norm:
            h = self._decode_resnorm(self.state, self.token)
            rmsnorm(h, self.model.norm, self.normed, eps=self.cfg.eps)
            self.logits = self.model.lm_head(self.normed[0])
            greedy(self.logits, self.token, self.state, self.history, self.greedy_ws)
            return
        down = self._layers(1, self.state, self.token)
        self._head(down, self.residual[0])

    @torch.no_grad()
    def capture(self) -> None:
        """Capture one decode step in a HIP graph.  Warms up with an eager step
        first (library handles, plans); the warm-up advances the state, so
        run prefill() again before decoding."""
        s = torch.cuda.Stream(device=self.model.device)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        self.graph = g
        self._graph_logits = self.logits      # lives in the graph's pool, rewritten by every replay

    def decode(self, n_steps: int, graph: bool = True, check: bool = True) -> None:
        """n_steps decode steps, launched without a host sync between them.
        check: afterwards, wait for the stream and raise if a layer launch's
        bounded wait ran out (check_layer_launch); check=False leaves the
        steps queued and the check to the caller."""
        if graph and self.graph is None:
            raise RuntimeError("capture() first")
        for _ in range(int(n_steps)):
            if graph:
                self.graph.replay()
                self.logits = self._graph_logits
            else:
                self.step()
        if check:
            self.check_layer_launch()

    def check_layer_launch(self) -> None:
        """Raise RuntimeError if any layer launch since the last check ended a
        bounded wait by its time limit (word 1024 of its counter buffer, set by
        the kernel and never cleared by it: sticky across launches and graph
        replays).  The tokens and logits of those steps are then not valid.
        The flags are cleared before raising.  Waits for the stream."""
        if not self.front:
            return
        flags = self.front_sync[:, 1024]
        if bool((flags != 0).any()):
            flags.zero_()
            torch.cuda.current_stream().synchronize()
            raise RuntimeError("a layer launch (bf16x_layer_front_decode) timed out waiting for its producer "
                               "stage: the decode steps since the last check are invalid; build the runner with "
                               "layer_front=False to use the separate launches")

    def generate(self, ids: torch.Tensor, n_new: int, graph: bool = True) -> list:
        """Greedy decode of n_new tokens after the prompt; the token ids."""
        if not (1 <= n_new <= self.max_new):
            raise ValueError(f"n_new must be in [1, {self.max_new}]")
        self.prefill(ids)
        self.decode(n_new - 1, graph=graph)               # checks the layer launches' time-out flags
        return self.history[:n_new].tolist()

    def kv_bytes_per_step(self) -> int:
        """K and V bytes the attention of one decode step reads at the mean
        context length of a generation from the current prompt."""
        ctx = self._prompt_len + self.max_new / 2
        return int(2 * self.cfg.n_layers * self.cfg.n_kv_heads * ctx * HEAD_DIM * 2)

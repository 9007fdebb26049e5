"""A small pre-norm, decoder-only transformer in torch whose attention, norms and
linear layers can each run on the MI355X HIP kernels of :mod:`ferrite.kernels`
("pallas" route, the reference's name for its kernel route) or on plain torch
math ("xla" route).

Reference: src/ferrite/model/gpt.py. Same config fields, parameter tree, routing
rules and numerics:

- parameters live in f32 (``init_params(..., param_dtype=...)`` may keep them in
  bf16 instead); activations and linear layers run in ``cfg.dtype`` with f32
  accumulation;
- softmax statistics, RMS statistics, the LM-head logits and the loss are f32;
- the residual add that closes one sub-layer is fused into the norm that opens
  the next (gpt.py:130-142), so each sub-layer reads and writes the residual
  stream once;
- the LM head is tied to the token embedding (gpt.py:143).

Autograd provides the backward pass: each kernel wrapper carries the custom
backward of its reference custom_vjp.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Iterator

import torch
import torch.nn.functional as F

from ferrite import platform
from ferrite.kernels.flash_attention import (BlockSizes, flash_attention, flash_attention_qkv,
                                            flash_attention_qkv_supported, flash_attention_reference)
from ferrite.kernels.heads import merge_heads, split_heads
from ferrite.kernels.matmul import matmul, mlp_gelu
from ferrite.kernels.rmsnorm import rmsnorm, rmsnorm_reference

ROUTES = ("pallas", "xla")


@dataclasses.dataclass(frozen=True)
class GPTConfig:
    """Model shape and kernel routing (gpt.py:29-63)."""

    vocab_size: int = 256  # byte-level tokens
    seq_len: int = 256
    d_model: int = 512
    n_head: int = 4
    n_layer: int = 4
    d_ff: int = 2048
    attention: str = "pallas"  # "pallas" (HIP flash attention) | "xla" (torch f32 math)
    norm: str = "pallas"  # "pallas" (HIP add+RMSNorm) | "xla"
    linear: str = "xla"  # "xla" (torch/hipBLASLt) | "pallas" (HIP matmul)
    dtype: torch.dtype = torch.bfloat16
    eps: float = 1e-6
    # Loss of loss_fn (not a reference field): "pallas" = HIP cross-entropy fused with the
    # tied head's backward, "xla" = torch cross_entropy on the f32 logits.
    loss: str = "pallas"

    def __post_init__(self):
        for field in ("attention", "norm", "linear", "loss"):
            if getattr(self, field) not in ROUTES:
                raise ValueError(f"{field} must be one of {ROUTES}, got {getattr(self, field)!r}")

    @property
    def head_dim(self) -> int:
        assert self.d_model % self.n_head == 0
        return self.d_model // self.n_head

    def replace(self, **kw) -> "GPTConfig":
        return dataclasses.replace(self, **kw)

    def attention_blocks(self, seq_len: int | None = None) -> BlockSizes | None:
        """Block sizes for a sequence of ``seq_len``, or None when the kernel route does not
        take it (gpt.py:51-63): the sequence must be a multiple of 128, and the block is the
        largest multiple of 128 up to ``platform.default_tile()`` that divides it."""
        s = seq_len or self.seq_len
        if s % 128:
            return None
        t = min(platform.default_tile(), s)
        while s % t:
            t -= 128
        return BlockSizes(t, t, t, t)


# ---------------------------------------------------------------- parameters


def init_params(seed: int | torch.Generator, cfg: GPTConfig, *, device=None, param_dtype: torch.dtype = torch.float32) -> dict:
    """Parameter tree of gpt.py:66-88: N(0, 0.02) weights, GPT-2 scaled residual
    projections (std 0.02/sqrt(2L) for ``wo`` and ``w2``), unit norm gains.

    Drawn from a seeded CPU ``torch.Generator`` (JAX's PRNG streams are not
    reproduced), then moved to ``device`` in ``param_dtype``."""
    gen = seed if isinstance(seed, torch.Generator) else torch.Generator().manual_seed(int(seed))
    std = 0.02
    out_std = std / math.sqrt(2 * cfg.n_layer)
    d, f = cfg.d_model, cfg.d_ff

    def normal(shape, s):
        return (s * torch.randn(shape, generator=gen, dtype=torch.float32)).to(device=device, dtype=param_dtype)

    def ones(n):
        return torch.ones((n,), dtype=param_dtype, device=device)

    tok_emb = normal((cfg.vocab_size, d), std)
    pos_emb = normal((cfg.seq_len, d), std)
    layers = []
    for _ in range(cfg.n_layer):
        layers.append(
            {
                "ln1": ones(d),
                "wqkv": normal((d, 3 * d), std),
                "wo": normal((d, d), out_std),
                "ln2": ones(d),
                "w1": normal((d, f), std),
                "w2": normal((f, d), out_std),
            }
        )
    return {"tok_emb": tok_emb, "pos_emb": pos_emb, "layers": layers, "ln_f": ones(d)}


def named_leaves(tree, prefix: str = "") -> Iterator[tuple[str, torch.Tensor]]:
    """(path, tensor) pairs in sorted-key order, paths joined with '/' ("layers/0/wqkv").
    This is the leaf order and key format of the reference's checkpoint (train.py:167-170)."""
    if isinstance(tree, dict):
        for k in sorted(tree):
            yield from named_leaves(tree[k], f"{prefix}{k}/")
    elif isinstance(tree, (list, tuple)):
        for i, v in enumerate(tree):
            yield from named_leaves(v, f"{prefix}{i}/")
    else:
        yield prefix[:-1], tree


def leaves(tree) -> list[torch.Tensor]:
    return [t for _, t in named_leaves(tree)]


def unflatten(tree, flat: list):
    """A tree shaped like ``tree`` holding ``flat`` in ``named_leaves`` order."""
    it = iter(flat)

    def build(node):
        if isinstance(node, dict):
            return {k: build(node[k]) for k in sorted(node)}
        if isinstance(node, (list, tuple)):
            return [build(v) for v in node]
        return next(it)

    out = build(tree)
    if next(it, None) is not None:
        raise ValueError("more leaves than the tree holds")
    return out


def param_count(params) -> int:
    return sum(int(t.numel()) for t in leaves(params))


# ---------------------------------------------------------------- layers


def _linear(x, w, cfg: GPTConfig):
    """[..., in] @ [in, out] in cfg.dtype with f32 accumulation (gpt.py:95-104)."""
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1]).to(cfg.dtype)
    w = w.to(cfg.dtype)
    if cfg.linear == "pallas":
        y = matmul(x2, w)
    else:
        y = torch.matmul(x2, w)  # f32 accumulation, rounded to cfg.dtype
    return y.reshape(*lead, w.shape[1])


def _mlp(y, layer, cfg: GPTConfig):
    """gelu(y @ w1) @ w2 (gpt.py:141). The bf16 kernel route fuses the GELU and its derivative
    into the matmul kernels (mlp_gelu); otherwise two linears around torch's tanh GELU."""
    if cfg.linear == "pallas" and cfg.dtype == torch.bfloat16:
        return mlp_gelu(y.to(cfg.dtype), layer["w1"].to(cfg.dtype), layer["w2"].to(cfg.dtype))
    return _linear(F.gelu(_linear(y, layer["w1"], cfg), approximate="tanh"), layer["w2"], cfg)


def _norm(x, w, residual, cfg: GPTConfig):
    """RMSNorm, or fused add+RMSNorm returning (h, y) when ``residual`` is given (gpt.py:107-110)."""
    if cfg.norm == "pallas":
        return rmsnorm(x, w, residual=residual, eps=cfg.eps)
    return rmsnorm_reference(x, w, residual=residual, eps=cfg.eps)


def _attention(q, k, v, cfg: GPTConfig):
    """Causal attention on [B, H, S, hd] (gpt.py:113-121). Sequences the kernel route
    does not tile go to the f32 torch route, as the reference sends them to XLA."""
    blocks = cfg.attention_blocks(q.shape[2]) if cfg.attention == "pallas" else None
    if blocks is not None:
        return flash_attention(q, k, v, causal=True, block_sizes=blocks)
    return flash_attention_reference(q, k, v, causal=True)


def _attention_block(qkv, cfg: GPTConfig):
    """[B, S, 3d] projection -> [B, S, d] attention output (gpt.py:136-138). The kernel route
    reads the heads where the projection left them and writes the output token-major
    (flash_attention_qkv) when the shape allows; otherwise heads are split, attended and merged."""
    if (cfg.attention == "pallas" and cfg.attention_blocks(qkv.shape[1]) is not None
            and flash_attention_qkv_supported(qkv, cfg.n_head)):
        return flash_attention_qkv(qkv, cfg.n_head)
    q, k, v = _split_heads(qkv, cfg)  # [B, H, S, hd] each
    return _merge_heads(_attention(q, k, v, cfg), cfg)


def _split_heads(qkv, cfg: GPTConfig):
    """[B, S, 3d] -> q, k, v as dense [B, H, S, hd] (gpt.py:137). The kernel route moves them
    with the HIP layout kernel; the torch route permutes."""
    b, s, _ = qkv.shape
    if cfg.attention == "pallas":
        return split_heads(qkv, 3, cfg.n_head)
    return qkv.reshape(b, s, 3, cfg.n_head, cfg.head_dim).permute(2, 0, 3, 1, 4).unbind(0)


def _merge_heads(a, cfg: GPTConfig):
    """[B, H, S, hd] -> [B, S, d] (gpt.py:138)."""
    b, _, s, _ = a.shape
    if cfg.attention == "pallas":
        return merge_heads(a)
    return a.transpose(1, 2).reshape(b, s, cfg.d_model)


_MM_F32_OUT: dict[str, bool] = {}


def _dot_f32(a, b):
    """``a @ b`` with f32 accumulation and an unrounded f32 result, as
    ``jnp.dot(..., preferred_element_type=f32)``. On a GPU, bf16 operands go to the
    library GEMM with an f32 output (``torch.mm(..., out_dtype=f32)``) when torch has it;
    otherwise the operands are widened to f32 first, which computes the same sums."""
    if a.dtype == torch.float32 and b.dtype == torch.float32:
        return a @ b
    if a.is_cuda:
        key = str(a.dtype)
        if _MM_F32_OUT.get(key, True):
            try:
                out = torch.mm(a, b, out_dtype=torch.float32)
                _MM_F32_OUT[key] = True
                return out
            except (RuntimeError, TypeError):
                _MM_F32_OUT[key] = False
    return a.float() @ b.float()


class _TiedLogits(torch.autograd.Function):
    """f32 logits ``y @ E^T`` of the tied LM head (gpt.py:143). The backward rounds the f32
    cotangent to the operand dtype and runs two single-pass products with f32
    accumulation, which is what a DEFAULT-precision dot does with an f32 cotangent."""

    @staticmethod
    def forward(ctx, y2, emb):
        ctx.save_for_backward(y2, emb)
        return _dot_f32(y2, emb.t())

    @staticmethod
    def backward(ctx, g):
        y2, emb = ctx.saved_tensors
        gq = g.to(y2.dtype)
        dy = torch.mm(gq, emb)
        demb = torch.mm(gq.t(), y2)
        return dy, demb


class _TiedHeadLoss(torch.autograd.Function):
    """Mean cross-entropy of the tied head's f32 logits (gpt.py:143, :147-152) on the HIP
    loss kernels. The logits stay inside: the backward kernel turns them straight into
    the cotangent in the operand dtype, which then feeds the two head products."""

    @staticmethod
    def forward(ctx, y2, emb, targets):
        from ferrite.kernels.cross_entropy import cross_entropy_rows

        logits = _dot_f32(y2, emb.t())
        loss, lse = cross_entropy_rows(logits, targets)
        ctx.save_for_backward(y2, emb, logits, targets, lse)
        return loss.mean()

    @staticmethod
    def backward(ctx, dloss):
        from ferrite.kernels.cross_entropy import cross_entropy_grad

        y2, emb, logits, targets, lse = ctx.saved_tensors
        g = cross_entropy_grad(logits, targets, lse, dloss, 1.0 / logits.shape[0], y2.dtype)
        return torch.mm(g, emb), torch.mm(g.t(), y2), None


def _trunk(params, tokens, cfg: GPTConfig):
    """tokens [B, S] -> final normed hidden states [B*S, d] in cfg.dtype (gpt.py:124-142)."""
    b, s = tokens.shape
    if s > cfg.seq_len:
        raise ValueError(f"sequence {s} longer than cfg.seq_len={cfg.seq_len}")
    h = (params["tok_emb"][tokens] + params["pos_emb"][:s]).to(cfg.dtype)  # residual stream
    pending = None  # sub-layer output whose residual add is fused into the next norm
    for layer in params["layers"]:
        if pending is None:
            y = _norm(h, layer["ln1"], None, cfg)
        else:
            h, y = _norm(pending, layer["ln1"], h, cfg)
        qkv = _linear(y, layer["wqkv"], cfg)  # [B, S, 3 * d]: rows (q|k|v, head, hd)
        a = _linear(_attention_block(qkv, cfg), layer["wo"], cfg)  # [B, S, d] in, [B, S, d] out
        h, y2 = _norm(a, layer["ln2"], h, cfg)
        pending = _mlp(y2, layer, cfg)
    _, y = _norm(pending, params["ln_f"], h, cfg)
    return y.reshape(-1, cfg.d_model)


def forward(params, tokens, cfg: GPTConfig):
    """tokens [B, S] (int) -> logits [B, S, vocab] f32 (gpt.py:124-144)."""
    b, s = tokens.shape
    y = _trunk(params, tokens, cfg)
    logits = _TiedLogits.apply(y, params["tok_emb"].to(cfg.dtype))
    return logits.reshape(b, s, cfg.vocab_size)


def loss_fn(params, tokens, targets, cfg: GPTConfig):
    """Mean next-token cross-entropy in f32 (gpt.py:147-152)."""
    if cfg.loss == "pallas":
        y = _trunk(params, tokens, cfg)
        return _TiedHeadLoss.apply(y, params["tok_emb"].to(cfg.dtype), targets.reshape(-1).long())
    logits = forward(params, tokens, cfg)
    return F.cross_entropy(logits.reshape(-1, cfg.vocab_size), targets.reshape(-1).long())


def flops_per_token(cfg: GPTConfig, n_params_nonembed: int) -> dict:
    """Analytic forward FLOPs per token (training = 3x), split as in gpt.py:155-163.

    Dense: 2 FLOPs per parameter of the dense layers plus the tied LM head.
    Attention: QK^T and PV are 2*S*d each per token and layer, halved by causal skipping.
    """
    dense = 2 * (n_params_nonembed + cfg.vocab_size * cfg.d_model)
    attn = 4 * cfg.seq_len * cfg.d_model * cfg.n_layer * 0.5
    return {"dense": dense, "attention": attn, "total": dense + attn}

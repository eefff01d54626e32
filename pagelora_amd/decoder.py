"""Qwen3-shaped decoder around the paged-decode + LoRA hot path.

This is the caller of the kernels, shaped like the reference's graph-static
decode layer ``run_flashinfer_decode_layer_static_append_batch``
(model/flashinfer/layer_runner.py:340-396):

    rmsnorm -> packed q/k/v GEMM (+ no-merge LoRA delta, packed_ops.py:105-165)
    -> per-head q/k RMSNorm (projection.py:248-260) + RoPE (projection.py:155-190)
       + KV append into the page (layer_runner.py:399-412), one fused kernel
    -> paged decode attention (attention_backend.py:120-131)
    -> o_proj (+ LoRA, packed_ops.py:251-265 / linear.py:200-231) -> residual
    -> rmsnorm -> packed gate/up GEMM (+ LoRA, packed_ops.py:168-203) -> SiLU*up
    -> down_proj (+ LoRA) -> residual

Base GEMMs are plain library GEMMs (torch -> hipBLASLt); everything else --
norms (each residual add fused into the next norm), q/k-norm + RoPE + KV
append, attention, SiLU*up and the LoRA delta -- runs on the library's HIP
kernels.  Weights are random
(no checkpoints are available); shapes follow Qwen3-8B.

Prefill (``prefill``) is not on the decode path: it fills the paged KV pool
for the prompt with the same kernels except attention, which is plain torch
float32 math over the gathered pages, so decode starts from a real context.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import fused_ops
from .attention_backend import PagedDecodeAttention
from .kv_pool import PagedKVPool, Request
from .lora import lora_delta_, lora_linear


@dataclass(frozen=True)
class DecoderConfig:
    num_layers: int = 36
    hidden: int = 4096
    num_qo_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 12288
    vocab: int = 151936
    rope_theta: float = 1_000_000.0
    rms_eps: float = 1e-6
    qk_norm: bool = True
    lora_rank: int = 16
    lora_alpha: float = 32.0

    @property
    def q_dim(self) -> int:
        return self.num_qo_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.num_kv_heads * self.head_dim


QWEN3_8B = DecoderConfig()


class LayerWeights:
    """One decoder layer: packed base weights plus stacked LoRA adapters.

    Packed q/k/v and gate/up weights are the reference's packed layout
    (``_cached_packed_linear``, packed_ops.py:268-311).  LoRA A/B of each
    module are stacked over adapters: A [n, r, in], B [n, out, r].
    """

    def __init__(self, cfg: DecoderConfig, n_adapters: int, device, dtype, gen: torch.Generator) -> None:
        h, qd, kd, i, r = cfg.hidden, cfg.q_dim, cfg.kv_dim, cfg.intermediate, cfg.lora_rank

        def w(shape, std):
            return (torch.randn(shape, device=device, dtype=torch.float32, generator=gen) * std).to(dtype)

        self.input_norm = (1.0 + 0.1 * torch.randn(h, device=device, generator=gen)).to(dtype)
        self.post_norm = (1.0 + 0.1 * torch.randn(h, device=device, generator=gen)).to(dtype)
        self.q_norm = (1.0 + 0.1 * torch.randn(cfg.head_dim, device=device, generator=gen)).to(dtype)
        self.k_norm = (1.0 + 0.1 * torch.randn(cfg.head_dim, device=device, generator=gen)).to(dtype)
        self.w_qkv = w((qd + 2 * kd, h), 0.02)
        self.w_o = w((h, qd), 0.02)
        self.w_gate_up = w((2 * i, h), 0.02)
        self.w_down = w((h, i), 0.02)
        self.lora = {}
        for name, fin, fout in (("q", h, qd), ("k", h, kd), ("v", h, kd), ("o", qd, h),
                                ("gate", h, i), ("up", h, i), ("down", i, h)):
            self.lora[name] = (w((n_adapters, r, fin), fin ** -0.5), w((n_adapters, fout, r), 0.01))


class DecoderWeights:
    def __init__(self, cfg: DecoderConfig, *, n_adapters: int = 1, device="cuda", dtype=torch.bfloat16, seed: int = 0):
        gen = torch.Generator(device=device).manual_seed(seed)
        self.cfg = cfg
        self.dtype = dtype
        self.n_adapters = n_adapters
        self.embed = (torch.randn((cfg.vocab, cfg.hidden), device=device, generator=gen) * 0.02).to(dtype)
        self.final_norm = (1.0 + 0.1 * torch.randn(cfg.hidden, device=device, generator=gen)).to(dtype)
        self.lm_head = (torch.randn((cfg.vocab, cfg.hidden), device=device, generator=gen) * 0.02).to(dtype)
        self.layers = [LayerWeights(cfg, n_adapters, device, dtype, gen) for _ in range(cfg.num_layers)]
        self.lora_scale = cfg.lora_alpha / cfg.lora_rank  # linear.py:41, 71


# ------------------------------------------------------- decode (static) ---
class DecodeContext:
    """Graph-owned per-step buffers of a batch (cuda_graph.py:307-464 analogue)."""

    def __init__(self, batch: int, device) -> None:
        self.batch = batch
        self.tokens = torch.zeros(batch, dtype=torch.int64, device=device)
        self.positions = torch.zeros(batch, dtype=torch.int64, device=device)
        self.page_id = torch.zeros(batch, dtype=torch.int64, device=device)
        self.page_offset = torch.zeros(batch, dtype=torch.int64, device=device)
        self.adapter_ids = torch.zeros(batch, dtype=torch.int32, device=device)
        self.next_tokens = torch.zeros(batch, dtype=torch.int64, device=device)


# Projections with narrow outputs (q/k/v, o) run on the decode-sized linear
# kernel with the LoRA expand in its epilogue; the wide MLP projections keep
# the library GEMM plus the separate shrink/expand kernels, which is faster
# for them.  Longer inputs (prefill) always take the library GEMM.
FUSED_LINEAR_MAX_TOKENS = 16


def _qkv_projection(cfg: DecoderConfig, lw: LayerWeights, x, ids, scale: float) -> torch.Tensor:
    qd, kd = cfg.q_dim, cfg.kv_dim
    (Aq, Bq), (Ak, Bk), (Av, Bv) = lw.lora["q"], lw.lora["k"], lw.lora["v"]
    if x.shape[0] <= FUSED_LINEAR_MAX_TOKENS:
        return lora_linear(x, lw.w_qkv, [(Aq, Bq, 0, scale), (Ak, Bk, qd, scale), (Av, Bv, qd + kd, scale)], ids)
    qkv = F.linear(x, lw.w_qkv)
    lora_delta_(x, [(Aq, Bq, qkv[:, :qd], scale), (Ak, Bk, qkv[:, qd:qd + kd], scale),
                    (Av, Bv, qkv[:, qd + kd:], scale)], ids)
    return qkv


def _o_projection(lw: LayerWeights, attn, ids, scale: float) -> torch.Tensor:
    Ao, Bo = lw.lora["o"]
    if attn.shape[0] <= FUSED_LINEAR_MAX_TOKENS:
        return lora_linear(attn, lw.w_o, [(Ao, Bo, 0, scale)], ids)
    o = F.linear(attn, lw.w_o)
    lora_delta_(attn, [(Ao, Bo, o, scale)], ids)
    return o


def _mlp(cfg: DecoderConfig, lw: LayerWeights, x2, ids, scale: float) -> torch.Tensor:
    I = cfg.intermediate
    gu = F.linear(x2, lw.w_gate_up)
    (Ag, Bg), (Au, Bu) = lw.lora["gate"], lw.lora["up"]
    lora_delta_(x2, [(Ag, Bg, gu[:, :I], scale), (Au, Bu, gu[:, I:], scale)], ids)
    act = fused_ops.silu_mul(gu)
    d = F.linear(act, lw.w_down)
    Ad, Bd = lw.lora["down"]
    lora_delta_(act, [(Ad, Bd, d, scale)], ids)
    return d


def decode_layer_static(
    cfg: DecoderConfig,
    lw: LayerWeights,
    lora_scale: float,
    hidden: torch.Tensor,
    pending: torch.Tensor | None,
    layer_cache: torch.Tensor,
    backend: PagedDecodeAttention,
    ctx: DecodeContext,
) -> torch.Tensor:
    """One single-token decode layer for the whole batch; graph-capturable.

    ``hidden`` is the residual stream, updated in place; ``pending`` is the
    previous layer's MLP output, added to it by this layer's fused
    add+RMSNorm.  Returns this layer's MLP output (pending for the next).
    """
    B = hidden.shape[0]
    ids = ctx.adapter_ids
    if pending is None:
        x = fused_ops.rmsnorm(hidden, lw.input_norm, cfg.rms_eps)
    else:
        x = fused_ops.add_rmsnorm(hidden, pending, lw.input_norm, cfg.rms_eps)
    qkv = _qkv_projection(cfg, lw, x, ids, lora_scale)
    q = fused_ops.qk_norm_rope_append(
        qkv, lw.q_norm if cfg.qk_norm else None, lw.k_norm if cfg.qk_norm else None,
        ctx.positions, ctx.page_id, ctx.page_offset, layer_cache, num_qo_heads=cfg.num_qo_heads,
        num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim, page_size=backend.page_size,
        rope_theta=cfg.rope_theta, eps=cfg.rms_eps)
    attn = torch.empty_like(q)
    backend.run_decode_into(q, layer_cache, attn)
    attn = attn.view(B, cfg.q_dim)
    o = _o_projection(lw, attn, ids, lora_scale)
    x2 = fused_ops.add_rmsnorm(hidden, o, lw.post_norm, cfg.rms_eps)
    return _mlp(cfg, lw, x2, ids, lora_scale)


def decode_step_static(weights: DecoderWeights, pool: PagedKVPool, backend: PagedDecodeAttention,
                       ctx: DecodeContext) -> torch.Tensor:
    """embed -> layers -> final norm -> lm_head -> greedy argmax into ctx.next_tokens.

    Returns the logits [B, vocab] (graph-owned under capture).
    """
    cfg = weights.cfg
    hidden = F.embedding(ctx.tokens, weights.embed)
    pending = None
    for li, lw in enumerate(weights.layers):
        pending = decode_layer_static(cfg, lw, weights.lora_scale, hidden, pending, pool.layer_cache(li),
                                      backend, ctx)
    x = fused_ops.add_rmsnorm(hidden, pending, weights.final_norm, cfg.rms_eps)
    logits = F.linear(x, weights.lm_head)
    ctx.next_tokens.copy_(torch.argmax(logits, dim=-1))  # greedy, sampling.py:8-15
    return logits


# ------------------------------------------------------------- prefill ---
def prefill_backend(cfg: DecoderConfig, page_size: int, device) -> PagedDecodeAttention:
    """An attention backend for :func:`prefill` (the paged prefill kernel)."""
    return PagedDecodeAttention(device=device, workspace_mb=1, num_qo_heads=cfg.num_qo_heads,
                                num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim, page_size=page_size)


@torch.no_grad()
def prefill(weights: DecoderWeights, pool: PagedKVPool, request: Request, tokens: torch.Tensor,
            adapter: int = 0, chunk: int = 8192, backend: PagedDecodeAttention | None = None) -> torch.Tensor:
    """Run ``tokens`` (appended after ``request.length``) through the model,
    writing their K/V into the request's pages; returns the last hidden row's
    logits.  Pages for the tokens must already be reserved.

    The reference's segment prefill (generation.py:250-275, layer_runner.py:40-102):
    per chunk, one paged prefill plan (qo = the chunk, kv = prefix + chunk,
    causal) shared by all layers; per layer q/k-norm + RoPE + KV append into
    the pages, then causal paged attention over them.
    """
    cfg = weights.cfg
    ps = pool.page_size
    start = request.length - tokens.numel()
    assert start >= 0, "reserve pages for the prompt before prefill"
    host_pages = request.pages()
    pages = torch.tensor(host_pages, dtype=torch.int64, device=tokens.device)
    if backend is None:
        backend = prefill_backend(cfg, ps, tokens.device)
    s = weights.lora_scale
    last_logits = None
    for c0 in range(0, tokens.numel(), chunk):
        tok = tokens[c0:c0 + chunk]
        T = tok.numel()
        ctx_len = start + c0 + T
        n_pages = -(-ctx_len // ps)
        backend.plan_prefill(
            qo_indptr=torch.tensor([0, T], dtype=torch.int32),
            paged_kv_indptr=torch.tensor([0, n_pages], dtype=torch.int32),
            paged_kv_indices=torch.tensor(host_pages[:n_pages], dtype=torch.int32),
            paged_kv_last_page_len=torch.tensor([ctx_len - ps * (n_pages - 1)], dtype=torch.int32),
            causal=True,
        )
        pos = torch.arange(start + c0, ctx_len, device=tokens.device)
        page_of = pages[pos // ps]
        off_of = pos % ps
        hidden = F.embedding(tok, weights.embed)
        ids = torch.full((T,), adapter, dtype=torch.int32, device=tokens.device)
        attn = torch.empty((T, cfg.num_qo_heads, cfg.head_dim), dtype=hidden.dtype, device=tokens.device)
        pending = None
        for li, lw in enumerate(weights.layers):
            cache = pool.layer_cache(li)
            if pending is None:
                x = fused_ops.rmsnorm(hidden, lw.input_norm, cfg.rms_eps)
            else:
                x = fused_ops.add_rmsnorm(hidden, pending, lw.input_norm, cfg.rms_eps)
            qkv = _qkv_projection(cfg, lw, x, ids, s)
            q = fused_ops.qk_norm_rope_append(
                qkv, lw.q_norm if cfg.qk_norm else None, lw.k_norm if cfg.qk_norm else None, pos, page_of,
                off_of, cache, num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads,
                head_dim=cfg.head_dim, page_size=ps, rope_theta=cfg.rope_theta, eps=cfg.rms_eps)
            backend.run_prefill_into(q, cache, attn)
            o = _o_projection(lw, attn.view(T, cfg.q_dim), ids, s)
            x2 = fused_ops.add_rmsnorm(hidden, o, lw.post_norm, cfg.rms_eps)
            pending = _mlp(cfg, lw, x2, ids, s)
        x = fused_ops.add_rmsnorm(hidden, pending, weights.final_norm, cfg.rms_eps)
        last_logits = F.linear(x[-1:], weights.lm_head)
    return last_logits

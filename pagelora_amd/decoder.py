"""Qwen3-shaped decoder around the paged-decode + LoRA hot path.

This is the caller of the kernels, shaped like the reference's graph-static
decode layer ``run_flashinfer_decode_layer_static_append_batch``
(model/flashinfer/layer_runner.py:340-396), no-merge LoRA on all seven
modules (packed_ops.py:105-265, multilora/linear.py:200-231):

    [+ previous down_proj output, its LoRA delta] add+RMSNorm
    -> GEMM on [W_qkv; A_q; A_k; A_v]
    -> q/k/v LoRA up-projection + per-head q/k RMSNorm (projection.py:248-260)
       + RoPE (projection.py:155-190) + KV append (layer_runner.py:399-412)
       + paged decode attention (attention_backend.py:120-131), one kernel,
       then the split-KV merge
    -> GEMM on [W_o; A_o] -> o LoRA up-projection + residual add + RMSNorm
    -> GEMM on [W_gate_up; A_gate; A_up] -> LoRA up-projections + SiLU*up
    -> GEMM on [W_down; A_down] (its delta lands in the next layer's norm)

Seven kernels per decode layer at decode batch sizes: four GEMMs on the
shuffled weights, the attention kernel with the q/k/v epilogue folded in,
the merge and SiLU*up.  The RMSNorms run in the prologues of the q/k/v and
gate/up GEMMs; o_proj and down_proj add their output and LoRA delta into
the residual stream in their epilogues.  The q/k/v and gate/up LoRA shrink
rides in the base GEMM (the adapters' A rows stacked under W) and the
expand in the kernel that consumes the module output; o_proj's shrink runs
in the attention's merge and down_proj's in SiLU*up, so no separate LoRA
launches remain.  (With the fusion off, or past 16 rows: two add+RMSNorm
kernels and the o/down GEMMs with their A rows on side planes, nine.)  Prefill, and batches beyond
the decode GEMM's 64 rows, use the library GEMM (torch -> hipBLASLt);
prefill forms q and appends k/v in the separate q/k norm + RoPE + append
kernel.  Weights are random (no checkpoints are available); shapes follow
Qwen3-8B.

``prefill`` runs the same layer over a prompt segment with the paged
prefill attention kernel.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import _lib, fused_ops
from .attention_backend import PagedDecodeAttention
from .kv_pool import PagedKVPool, Request
from .linear import (LoraPartials, ShuffledWeight, SplitOutput, linear_shuffled, linear_shuffled_add,
                     linear_shuffled_norm, linear_shuffled_side, linear_shuffled_split, lora_a_rows)
from .lora import lora_linear


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


# Module names of the reference's adapters (HF leaf names of the wrapped
# nn.Linear, multilora/runtime.py:95-116) -> the decoder's short names.
MODULE_ALIASES = {"q_proj": "q", "k_proj": "k", "v_proj": "v", "o_proj": "o", "gate_proj": "gate",
                  "up_proj": "up", "down_proj": "down"}
MODULES = ("q", "k", "v", "o", "gate", "up", "down")


def projections(cfg: DecoderConfig):
    """(projection, in_features, ((module, out_features), ...)) in the packed
    order of the reference (q/k/v and gate/up share one input:
    packed_ops.py:105-203)."""
    h, qd, kd, i = cfg.hidden, cfg.q_dim, cfg.kv_dim, cfg.intermediate
    return (("qkv", h, (("q", qd), ("k", kd), ("v", kd))), ("o", qd, (("o", h),)),
            ("gate_up", h, (("gate", i), ("up", i))), ("down", i, (("down", h),)))


def module_key(name: str) -> str:
    """The decoder's name of a module given as "q", "q_proj" or "self_attn.q_proj"."""
    leaf = name.rsplit(".", 1)[-1]
    leaf = MODULE_ALIASES.get(leaf, leaf)
    if leaf not in MODULES:
        raise KeyError(f"unknown LoRA module {name!r} (known: {', '.join(MODULES)} or their *_proj names)")
    return leaf


class _RandomSource:
    """Seeded random weights (N(0, 0.02) base, norms 1 +- 0.1, LoRA A with
    std in^-1/2 and B with std 0.01, so the delta is not a no-op)."""

    def __init__(self, device, dtype, gen: torch.Generator) -> None:
        self.device, self.dtype, self.gen = device, dtype, gen

    def _w(self, shape, std):
        return (torch.randn(shape, device=self.device, dtype=torch.float32, generator=self.gen) * std).to(self.dtype)

    def norm(self, name, n):
        return (1.0 + 0.1 * torch.randn(n, device=self.device, generator=self.gen)).to(self.dtype)

    def base(self, proj, modules, shape):
        return self._w(shape, 0.02)

    def lora_a(self, name, shape):
        return self._w(shape, shape[-1] ** -0.5)

    def lora_b(self, name, shape):
        return self._w(shape, 0.01)


class _TensorSource:
    """Given weights: ``layer`` maps "input_norm", "post_norm", "q_norm",
    "k_norm" and the module names to tensors ([out, in] for the modules);
    ``adapters[slot]`` maps module names to (A [r, in], B [out, r]) or is
    None.  A module an adapter leaves out gets a zero delta (A = B = 0)."""

    def __init__(self, layer: dict, adapters, device, dtype) -> None:
        self.layer = {(module_key(k) if k.rsplit(".", 1)[-1] in MODULE_ALIASES or k in MODULES else k): v
                      for k, v in layer.items()}
        self.adapters = [None if a is None else {module_key(k): v for k, v in a.items()} for a in adapters]
        self.device, self.dtype = device, dtype

    def _t(self, t, shape, what):
        t = torch.as_tensor(t)
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"{what}: expected shape {tuple(shape)}, got {tuple(t.shape)}")
        return t.to(device=self.device, dtype=self.dtype)

    def norm(self, name, n):
        return self._t(self.layer[name], (n,), name)

    def base(self, proj, modules, shape):
        return torch.cat([self._t(self.layer[m], (out, shape[1]), m) for m, out in modules])

    def _lora(self, name, shape, j, what):
        out = torch.zeros(shape, device=self.device, dtype=self.dtype)
        for slot, ad in enumerate(self.adapters):
            if ad is not None and name in ad:
                out[slot] = self._t(ad[name][j], shape[1:], f"adapter {slot} {name} {what}")
        return out

    def lora_a(self, name, shape):
        return self._lora(name, shape, 0, "A")

    def lora_b(self, name, shape):
        return self._lora(name, shape, 1, "B")


class LayerWeights:
    """One decoder layer: packed base weights plus stacked LoRA adapters.

    Packed q/k/v and gate/up weights are the reference's packed layout
    (``_cached_packed_linear``, packed_ops.py:268-311).  Each projection's
    weight is stored with its modules' LoRA A rows stacked under it, for
    every adapter (``w_*_ext`` = [W; A_m0[0..n); A_m1[0..n); ..]), the
    row-concatenated A_cat of ``_cached_packed_lora_delta`` (packed_ops.py:
    328-384) extended over adapters: one GEMM then yields the base output and
    every adapter's rank-space intermediate.  ``w_*`` and the A of
    ``lora[name] = (A [n, r, in], B [n, out, r])`` are views into those
    buffers; ``y_offset[name]`` is the first intermediate column of a module
    in its projection's output.  Adapter slot ``a`` of module m is
    ``lora[m][0][a]`` / ``lora[m][1][a]``.
    """

    def __init__(self, cfg: DecoderConfig, n_adapters: int, device, dtype, gen: torch.Generator | None = None,
                 source=None) -> None:
        h, r = cfg.hidden, cfg.lora_rank
        n = n_adapters
        src = source if source is not None else _RandomSource(device, dtype, gen)
        self.cfg, self.n_adapters, self.device, self.dtype = cfg, n, device, dtype
        self.input_norm = src.norm("input_norm", h)
        self.post_norm = src.norm("post_norm", h)
        self.q_norm = src.norm("q_norm", cfg.head_dim)
        self.k_norm = src.norm("k_norm", cfg.head_dim)
        self.lora = {}
        self.y_offset = {}
        self.y_offset_base = {}  # base output rows of each projection
        for proj, fin, modules in projections(cfg):
            out_features = sum(o for _, o in modules)
            ext = torch.empty((out_features + len(modules) * n * r, fin), device=device, dtype=dtype)
            ext[:out_features] = src.base(proj, modules, (out_features, fin))
            for j, (name, fout) in enumerate(modules):
                row = out_features + j * n * r
                A = ext[row:row + n * r].view(n, r, fin)
                A.copy_(src.lora_a(name, (n, r, fin)))
                self.lora[name] = (A, src.lora_b(name, (n, fout, r)))
                self.y_offset[name] = row
            setattr(self, f"w_{proj}_ext", ext)
            setattr(self, f"w_{proj}", ext[:out_features])
            self.y_offset_base[proj] = out_features
        self.shuffled: dict[str, ShuffledWeight] = {}
        self.lora_b8: dict[str, torch.Tensor] = {}
        self.single_copy = False  # True once the shuffled copies are the only ones

    def __getattr__(self, name: str):
        # w_<proj>_ext / w_<proj> of a single-copy layer: unshuffled on demand
        # (a fresh tensor; the hot paths use the shuffled copy or row_major())
        if name.startswith("w_") and self.__dict__.get("single_copy"):
            proj = name[2:-4] if name.endswith("_ext") else name[2:]
            sw = self.__dict__["shuffled"].get(proj)
            if sw is not None:
                w = sw.unshuffle()
                return w if name.endswith("_ext") else w[: self.__dict__["y_offset_base"][proj]]
        raise AttributeError(f"{type(self).__name__!s} has no attribute {name!r}")

    def shuffle(self, keep_row_major: bool = False) -> None:
        """Shuffled copies of the four [W; A] weights for the decode GEMM.

        Unless ``keep_row_major``, the shuffled copy becomes the only one:
        the row-major [W; A] buffers are released (the LoRA A stacks move to
        tensors of their own), so the projection weights are stored once.
        ``w_*_ext`` / ``w_*`` then return an unshuffled copy, and the library
        GEMMs of prefill read the weight unshuffled into one buffer reused by
        every projection (:func:`row_major`)."""
        for name in ("qkv", "o", "gate_up", "down"):
            self.shuffled[name] = ShuffledWeight(getattr(self, f"w_{name}_ext"))
        if not keep_row_major:
            for name in MODULES:
                A, B = self.lora[name]
                self.lora[name] = (A.clone(), B)
            for proj, _, _ in projections(self.cfg):
                delattr(self, f"w_{proj}_ext")
                delattr(self, f"w_{proj}")
            self.single_copy = True
        # o_proj's and down_proj's B in the chunked layout: their consumer,
        # the add+RMSNorm, reads a whole row's B in one workgroup and runs
        # 7.3 -> 4.9 us with it (Qwen3-8B shape, 4 rows).  The one-wave
        # workgroups of silu and the q/k/v kernel read a 512-column slice
        # each and are faster on the row-major B (6.4 vs 7.6 us, 6.0 vs 6.4).
        for name in ("o", "down"):
            if name in self.lora:
                self.lora_b8[name] = fused_ops.lora_b_chunk8(self.lora[name][1])

    def write_adapter(self, slot: int, modules: dict) -> None:
        """Write one adapter's A/B into ``slot`` in place (every copy: the A
        rows under W, their 16-row blocks of the shuffled weight, B and its
        chunked copy); a module left out gets a zero delta.  Stream ordered:
        decode steps enqueued later read the new values through the same
        addresses, so captured graphs stay valid."""
        if not 0 <= slot < self.n_adapters:
            raise ValueError(f"adapter slot {slot} outside 0..{self.n_adapters - 1}")
        r = self.cfg.lora_rank
        given = {module_key(k): v for k, v in modules.items()}
        for proj, fin, mods in projections(self.cfg):
            ext = None if self.single_copy else getattr(self, f"w_{proj}_ext")
            for name, fout in mods:
                A_stack, B_stack = self.lora[name]
                if name in given:
                    A, B = given[name]
                    A = torch.as_tensor(A)
                    B = torch.as_tensor(B)
                    if tuple(A.shape) != (r, fin) or tuple(B.shape) != (fout, r):
                        raise ValueError(f"{name}: A must be [{r}, {fin}] and B [{fout}, {r}], got "
                                         f"{tuple(A.shape)} / {tuple(B.shape)}")
                    A_stack[slot].copy_(A)
                    B_stack[slot].copy_(B)
                else:
                    A_stack[slot].zero_()
                    B_stack[slot].zero_()
                lo = self.y_offset[name] + slot * r
                if self.single_copy:
                    self.shuffled[proj].write_rows(A_stack[slot], lo)
                elif proj in self.shuffled:
                    self.shuffled[proj].refresh_rows(ext, lo, lo + r)
                if name in self.lora_b8:
                    self.lora_b8[name][slot].copy_(fused_ops.lora_b_chunk8(B_stack[slot])[0])

    def grown(self, n_adapters: int) -> "LayerWeights":
        """A copy of this layer with ``n_adapters`` slots (the new ones zero):
        new buffers, so graphs captured on the old ones must be recaptured."""
        if n_adapters < self.n_adapters:
            raise ValueError("adapter stacks only grow")
        old = self
        given = {"input_norm": old.input_norm, "post_norm": old.post_norm, "q_norm": old.q_norm,
                 "k_norm": old.k_norm}
        for proj, fin, mods in projections(self.cfg):
            w = getattr(old, f"w_{proj}")
            row = 0
            for name, fout in mods:
                given[name] = w[row:row + fout]
                row += fout
        adapters = [{name: (old.lora[name][0][a], old.lora[name][1][a]) for name in MODULES}
                    for a in range(old.n_adapters)] + [None] * (n_adapters - old.n_adapters)
        new = LayerWeights(self.cfg, n_adapters, self.device, self.dtype,
                           source=_TensorSource(given, adapters, self.device, self.dtype))
        if old.shuffled:
            new.shuffle(keep_row_major=not old.single_copy)
        return new

    def up(self, name: str, y: "torch.Tensor | SideOutput", scale: float, adapter: int = -1) -> fused_ops.LoraUp:
        """The up-projection of module ``name`` reading its intermediate from ``y``
        (``adapter`` >= 0: that one adapter for every token)."""
        B = self.lora_b8.get(name)
        B = self.lora[name][1] if B is None else B
        if isinstance(y, SideOutput):
            return fused_ops.LoraUp(y.side, self.y_offset[name] - y.main.shape[1], B, scale, adapter)
        return fused_ops.LoraUp(y, self.y_offset[name], B, scale, adapter)


class DecoderWeights:
    """Weights of the decoder: random (``DecoderWeights(cfg, seed=...)``) or
    given (:meth:`from_tensors`).  ``shuffle`` (default) also builds the
    shuffled decode-GEMM copies of every projection and of the lm_head; the
    projections' row-major weights are then released unless
    ``keep_row_major`` (the lm_head stays row-major too: prefill's last-token
    logits and decode steps of more than 16 rows read it).

    ``adapter_version`` changes whenever the adapter stacks are reallocated
    (:meth:`set_adapter` past the stacked slots); decode graphs key on it, as
    the reference's captured graphs key on ``flashinfer_graph_version``
    (multilora/runtime.py:371-375).  Writing an adapter into an existing slot
    keeps every buffer address and needs no recapture."""

    def __init__(self, cfg: DecoderConfig, *, n_adapters: int = 1, device="cuda", dtype=torch.bfloat16, seed: int = 0,
                 shuffle: bool = True, keep_row_major: bool = False, _sources=None, _top=None):
        self.cfg = cfg
        self.dtype = dtype
        self.n_adapters = n_adapters
        self.adapter_version = 0
        if _top is None:
            gen = torch.Generator(device=device).manual_seed(seed)
            self.embed = (torch.randn((cfg.vocab, cfg.hidden), device=device, generator=gen) * 0.02).to(dtype)
            self.final_norm = (1.0 + 0.1 * torch.randn(cfg.hidden, device=device, generator=gen)).to(dtype)
            self._lm_head = (torch.randn((cfg.vocab, cfg.hidden), device=device, generator=gen) * 0.02).to(dtype)
            self.layers = [LayerWeights(cfg, n_adapters, device, dtype, gen) for _ in range(cfg.num_layers)]
        else:
            self.embed, self.final_norm, self._lm_head = _top
            self.layers = [LayerWeights(cfg, n_adapters, device, dtype, source=src) for src in _sources]
        self.lora_scale = cfg.lora_alpha / cfg.lora_rank  # linear.py:41, 71
        self.lm_head_shuffled: ShuffledWeight | None = None
        if shuffle:
            for lw in self.layers:
                lw.shuffle(keep_row_major=keep_row_major)
            self.lm_head_shuffled = ShuffledWeight(self._lm_head)
            if not keep_row_major:
                self._lm_head = None

    @property
    def lm_head(self) -> torch.Tensor:
        """The [vocab, hidden] lm_head (unshuffled on demand when only the
        shuffled copy is kept)."""
        return self._lm_head if self._lm_head is not None else self.lm_head_shuffled.unshuffle()

    def logits(self, x: torch.Tensor) -> torch.Tensor:
        """x . lm_head^T: the shuffled GEMM at decode sizes (up to 16 rows, or
        64 when no row-major copy is kept), else the library GEMM on the
        row-major weight."""
        limit = _lib.PL_LINEAR_MAX_TOKENS if self._lm_head is None else DECODE_GEMM_MAX_TOKENS
        if self.lm_head_shuffled is not None and x.shape[0] <= limit:
            return linear_shuffled(x, self.lm_head_shuffled)
        return F.linear(x, self._lm_head if self._lm_head is not None else unshuffled_scratch(self.lm_head_shuffled))

    @classmethod
    def from_tensors(cls, cfg: DecoderConfig, *, embed: torch.Tensor, final_norm: torch.Tensor,
                     lm_head: torch.Tensor, layers: list[dict], adapters: list | None = None,
                     n_adapters: int | None = None, device="cuda", dtype=torch.bfloat16,
                     shuffle: bool = True) -> "DecoderWeights":
        """Weights from given tensors.

        ``layers[l]`` maps "input_norm", "post_norm", "q_norm", "k_norm" and
        the seven module names ("q".."down", or "q_proj".."down_proj") to
        tensors, module weights as [out, in] (nn.Linear's layout).
        ``adapters[slot]`` is None or a mapping ``{(layer, module): (A [r, in],
        B [out, r])}``, the reference's serve-registry layout
        (multilora/runtime.py:257-292); its modules get the delta
        ``alpha / r * B . (A . x)`` (linear.py:41, 226-231), the modules it
        leaves out none.
        """
        adapters = list(adapters or [])
        n = max(1, len(adapters), n_adapters or 0)
        adapters += [None] * (n - len(adapters))
        if len(layers) != cfg.num_layers:
            raise ValueError(f"{len(layers)} layers given for a {cfg.num_layers}-layer config")
        per_layer = []
        for li in range(cfg.num_layers):
            per_layer.append([None if a is None else {m: ab for (l, m), ab in a.items() if l == li}
                              for a in adapters])
        dev = torch.device(device)

        def t(x, shape, what):
            x = torch.as_tensor(x)
            if tuple(x.shape) != shape:
                raise ValueError(f"{what}: expected shape {shape}, got {tuple(x.shape)}")
            return x.to(device=dev, dtype=dtype)

        top = (t(embed, (cfg.vocab, cfg.hidden), "embed"), t(final_norm, (cfg.hidden,), "final_norm"),
               t(lm_head, (cfg.vocab, cfg.hidden), "lm_head"))
        sources = [_TensorSource(layers[li], per_layer[li], dev, dtype) for li in range(cfg.num_layers)]
        return cls(cfg, n_adapters=n, device=dev, dtype=dtype, shuffle=shuffle, _sources=sources, _top=top)

    def set_adapter(self, slot: int, adapter: dict | None) -> None:
        """Write ``adapter`` ({(layer, module): (A, B)}, or None for a zero
        delta) into ``slot``: in place when the slot exists (stream ordered;
        captured graphs stay valid), else the stacks grow to ``slot + 1``
        slots (new buffers: ``adapter_version`` changes)."""
        if slot < 0:
            raise ValueError("adapter slot must be >= 0")
        if slot >= self.n_adapters:
            self.layers = [lw.grown(slot + 1) for lw in self.layers]
            self.n_adapters = slot + 1
            self.adapter_version += 1
        adapter = adapter or {}
        for li, lw in enumerate(self.layers):
            lw.write_adapter(slot, {m: ab for (l, m), ab in adapter.items() if l == li})


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
        # >= 0: every row uses this adapter (the reference binds one adapter
        # per batch); the LoRA kernels then skip the per-row adapter-id load.
        # A captured step bakes it in (part of the graph key).
        self.uniform_adapter = -1
        self.argmax_ws: torch.Tensor | None = None  # greedy-argmax partial maxima
        # the step's RoPE angles [B, head_dim/2, 2] when the decode layers fold
        # the q/k/v epilogue into attention (see folded_qkv_decode)
        self.rope_cos_sin: torch.Tensor | None = None


# Decode-sized inputs (up to 16 tokens) take the GEMM on shuffled weights
# when the layer has them, else the row-major decode-sized linear kernel for
# the narrow projections (q/k/v, o); the wide MLP projections and longer
# inputs (prefill) take the library GEMM (torch -> hipBLASLt).
DECODE_GEMM_MAX_TOKENS = 16
# Split-K ways of the decode GEMM per projection (whole output, consumers
# sum the planes).  None by default: down_proj ran split 3 ways (257 blocks
# of 16 outputs over K = 12288: 25.9 -> 19.4 us at 4 tokens, +1.7 us in the
# next add+RMSNorm) until its A rows were split off instead (below); o_proj
# and qkv save less than their consumers then pay.
DECODE_SPLITS: dict[str, int] = {}
# Projections whose stacked LoRA A rows are split off (pl_linear_shuffled_side)
# at decode batch sizes, with the side planes' count: o_proj and down_proj
# have 4096 base rows, 256 blocks of 16 (one per CU), and their A rows make a
# 257th block that costs some CU a second whole block (4 tokens: o 7.6 ->
# 10.1 us, down unsplit 18.8 -> 26.3 us; down split 3 ways 20.3 us).  With
# the A rows split 16 ways by small workgroups of their own, down needs no
# split of its base rows either.
DECODE_SIDE_SPLITS = {"o": 16, "down": 16}
# Decode layers form q and append k/v inside the attention kernel
# (pl_decode_run_qkv) where it is built; False keeps the separate
# head-norm/RoPE/append kernel (tests compare the two).
FOLD_QKV_INTO_DECODE = True
# Decode layers on the folded path fuse the add + RMSNorm launches away
# where they can (see _layer): FUSE_NORMS the post-attention one (and the
# input RMSNorm into the q/k/v GEMM), FUSE_DOWN_NORM also the one after
# down_proj.  False keeps the add+RMSNorm kernel (tests compare the two).
FUSE_NORMS = True
FUSE_DOWN_NORM = True
# Optional observer of a layer's stages, called eagerly as ``STAGE_TRACE(name,
# value)`` with each stage's stored output (tensors, split planes, partial
# outputs) in dataflow order: "hidden_in" (the residual stream on entry),
# "hidden" (after the input add of the previous layer's down_proj output,
# when this layer does that add), "x", "qkv", "attn", "o", "hidden_mid",
# "x2", "gate_up", "act", "down" per layer (with the norms fused into the
# GEMMs, "x" and "x2" are the normalized rows the GEMMs report); after the
# last layer (decode steps) "final_hidden_in" (the residual stream before
# the last down_proj output is added), "final_down" (that output),
# "final_hidden", "final_x" (after the final add + RMSNorm), "logits" and
# "next_tokens".  For checking a decode step stage by stage; it must stay
# None while a graph is captured.
STAGE_TRACE = None


class SideOutput:
    """A projection output as its base rows ``main`` [T, out] and the LoRA
    intermediates ``side`` (split-K planes of linear_shuffled_side)."""

    def __init__(self, main: torch.Tensor, side: SplitOutput) -> None:
        self.main, self.side = main, side


class PartialOutput:
    """A projection whose output went straight into the residual stream
    (linear_shuffled_add), traced as its base output ``main`` [T, out] (a
    copy written for the trace) and the bound adapter's rank-space row as the
    producer's partial sums ``partials`` (LoraPartials)."""

    def __init__(self, main: torch.Tensor, partials: LoraPartials) -> None:
        self.main, self.partials = main, partials


def _project(x: torch.Tensor, lw: LayerWeights, name: str) -> "torch.Tensor | SplitOutput | SideOutput":
    """x . [W; A]^T: the base output and every adapter's LoRA intermediate
    (at decode batch sizes as split-K planes, or with the intermediates split
    off, for the narrow projections)."""
    # a single-copy layer keeps the shuffled GEMM up to 64 rows: unshuffling
    # for the library GEMM would read the weight twice
    limit = _lib.PL_LINEAR_MAX_TOKENS if lw.single_copy else DECODE_GEMM_MAX_TOKENS
    if x.shape[0] <= limit:
        sw = lw.shuffled.get(name)
        if sw is not None:
            side = min(DECODE_SIDE_SPLITS.get(name, 0), sw.in_features // 32)
            main = lw.y_offset.get(name, sw.out_features)
            if side and main % 16 == 0 and main < sw.out_features:
                return SideOutput(*linear_shuffled_side(x, sw, main, side))
            splits = DECODE_SPLITS.get(name, 1)
            if splits > 1:
                return linear_shuffled_split(x, sw, splits)
            return linear_shuffled(x, sw)
        if name in ("qkv", "o"):
            return lora_linear(x, row_major(lw, name), None, None)
    return F.linear(x, row_major(lw, name))


_ROW_MAJOR_SCRATCH: dict = {}


def row_major(lw: LayerWeights, name: str) -> torch.Tensor:
    """The row-major [W; A] weight of projection ``name`` for a library GEMM:
    the stored tensor, or for a single-copy layer the shuffled copy
    unshuffled into a buffer shared by every projection of the device (stream
    ordered: each use is enqueued after the previous one's GEMM)."""
    if not lw.single_copy:
        return getattr(lw, f"w_{name}_ext")
    return unshuffled_scratch(lw.shuffled[name])


def unshuffled_scratch(sw: ShuffledWeight) -> torch.Tensor:
    """``sw`` unshuffled into the per-device row-major scratch buffer."""
    key = (sw.data.device, sw.dtype)
    need = sw.out_features * sw.in_features
    buf = _ROW_MAJOR_SCRATCH.get(key)
    if buf is None or buf.numel() < need:
        buf = _ROW_MAJOR_SCRATCH[key] = torch.empty(need, dtype=sw.dtype, device=sw.data.device)
    return sw.unshuffle(buf[:need].view(sw.out_features, sw.in_features))


def _cols(out, n: int):
    """The first n columns of a projection output (split planes are passed whole)."""
    if isinstance(out, SideOutput):
        return out.main[:, :n]
    return out if isinstance(out, SplitOutput) else out[:, :n]


def _layer(cfg: DecoderConfig, lw: LayerWeights, scale: float, hidden: torch.Tensor, pending, ids: torch.Tensor,
           positions: torch.Tensor, page_id: torch.Tensor, page_offset: torch.Tensor, layer_cache: torch.Tensor,
           page_size: int, attend, adapter: int = -1, qkv_attend=None):
    """One decoder layer over T tokens (decode or prefill), no-merge LoRA on
    all seven modules.  ``hidden`` is the residual stream, updated in place;
    ``pending`` = (previous layer's down_proj output, its LoRA up-projection)
    to fold into this layer's input add+RMSNorm, a :class:`FusedPending`
    when the previous layer already added it into ``hidden``, or None.
    ``attend(q)`` returns attention over the pages as [T, Hq, D].  Returns
    this layer's pending value.

    Per projection, one GEMM on [W; A] yields base output + LoRA intermediate
    and the consumer kernel applies the up-projection: the q/k/v deltas in
    the head-norm/RoPE/append kernel, o's and down's in the next
    add+RMSNorm, gate's and up's in SiLU*up.  ``adapter`` >= 0 binds that
    adapter to every token (``ids`` is then not read).  ``qkv_attend(qkv,
    lora)``, when given, replaces the head-norm/RoPE/append kernel and
    ``attend``: one kernel that forms q and appends k/v from the packed rows
    while attending.

    Decode layers on that folded path take the add + RMSNorm launches out
    where :func:`_fused_norms` allows: o_proj's LoRA shrink runs in the
    attention's merge and down_proj's in SiLU*up (as partial sums), o_proj
    and down_proj each add their output and LoRA delta into the residual
    stream in the GEMM's epilogue (pl_linear_shuffled_add), and the RMSNorms
    run in the prologue of the q/k/v and gate/up GEMMs
    (pl_linear_shuffled_norm).
    """
    h, qd, kd, I = cfg.hidden, cfg.q_dim, cfg.kv_dim, cfg.intermediate
    T, r = hidden.shape[0], cfg.lora_rank
    a = adapter
    trace = STAGE_TRACE
    if trace is not None:
        trace("hidden_in", hidden)
    fused = qkv_attend is not None and _fused_norms(cfg, lw, T)
    if isinstance(pending, FusedPending) or (pending is None and fused and _norm_prologue(cfg, T)):
        # the residual stream is complete: RMSNorm in the q/k/v GEMM
        x = torch.empty_like(hidden) if trace is not None else None
        sq = pending.sq if isinstance(pending, FusedPending) else None
        qkv = linear_shuffled_norm(hidden, lw.input_norm, cfg.rms_eps, lw.shuffled["qkv"], x, sq=sq)
    else:
        if pending is None:
            x = fused_ops.rmsnorm(hidden, lw.input_norm, cfg.rms_eps)
        else:
            prev_out, prev_up = pending
            x = fused_ops.add_rmsnorm(hidden, _cols(prev_out, h), lw.input_norm, cfg.rms_eps, lora=prev_up,
                                      adapter_ids=ids)
        qkv = _project(x, lw, "qkv")
        if trace is not None:
            trace("hidden", hidden)
    if trace is not None:
        trace("x", x)
        trace("qkv", qkv)
    lora_qkv = (lw.up("q", qkv, scale, a), lw.up("k", qkv, scale, a), lw.up("v", qkv, scale, a))
    fused = fused and not isinstance(qkv, SplitOutput)
    if fused:
        parts = LoraPartials(torch.empty((T, qkv_attend.oshrink_parts(T), r), dtype=torch.float32,
                                         device=hidden.device))
        o_rows = lora_a_rows(lw.shuffled["o"], lw.y_offset["o"], r, a)
        attn = qkv_attend(_cols(qkv, qd + 2 * kd), lora_qkv, (o_rows, parts, lw.n_adapters)).view(T, qd)
        o_main = torch.empty_like(hidden) if trace is not None else None
        # B row-major: each workgroup reads the 16 consecutive B rows of its columns
        lo = fused_ops.LoraUp(None, 0, lw.lora["o"][1], scale, a)
        sq = _sq_buffer(cfg, T, hidden.device)
        linear_shuffled_add(attn, lw.shuffled["o"], h, hidden, lo, parts, ids, out=o_main, sq_out=sq)
        if trace is not None:
            for name, value in (("attn", attn), ("o", PartialOutput(o_main, parts)), ("hidden_mid", hidden)):
                trace(name, value)
        x2 = torch.empty_like(hidden) if trace is not None else None
        gu = linear_shuffled_norm(hidden, lw.post_norm, cfg.rms_eps, lw.shuffled["gate_up"], x2, sq=sq)
    else:
        if qkv_attend is not None and not isinstance(qkv, SplitOutput):
            attn = qkv_attend(_cols(qkv, qd + 2 * kd), lora_qkv).view(T, qd)
        else:
            q = fused_ops.qk_norm_rope_append(
                _cols(qkv, qd + 2 * kd), lw.q_norm if cfg.qk_norm else None, lw.k_norm if cfg.qk_norm else None,
                positions, page_id, page_offset, layer_cache, num_qo_heads=cfg.num_qo_heads,
                num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim, page_size=page_size,
                rope_theta=cfg.rope_theta, eps=cfg.rms_eps, lora=lora_qkv, adapter_ids=ids)
            attn = attend(q).view(T, qd)
        o = _project(attn, lw, "o")
        x2 = fused_ops.add_rmsnorm(hidden, _cols(o, h), lw.post_norm, cfg.rms_eps, lora=lw.up("o", o, scale, a),
                                   adapter_ids=ids)
        if trace is not None:
            for name, value in (("attn", attn), ("o", o), ("hidden_mid", hidden)):
                trace(name, value)
        gu = _project(x2, lw, "gate_up")
    if trace is not None:
        trace("x2", x2)
        trace("gate_up", gu)
    lora_gu = (lw.up("gate", gu, scale, a), lw.up("up", gu, scale, a))
    if fused and _fused_down(cfg, lw):
        parts_d = LoraPartials(torch.empty((T, -(-I // 256), r), dtype=torch.float32, device=hidden.device))
        d_rows = lora_a_rows(lw.shuffled["down"], lw.y_offset["down"], r, a)
        act = fused_ops.silu_mul(gu[:, : 2 * I], lora=lora_gu, adapter_ids=ids, down_shrink=(d_rows, parts_d))
        before = hidden.clone() if trace is not None else None
        d_main = torch.empty_like(hidden) if trace is not None else None
        sq = _sq_buffer(cfg, T, hidden.device)
        ld = fused_ops.LoraUp(None, 0, lw.lora["down"][1], scale, a)
        linear_shuffled_add(act, lw.shuffled["down"], h, hidden, ld, parts_d, ids, out=d_main, sq_out=sq)
        if trace is not None:
            down = PartialOutput(d_main, parts_d)
            trace("act", act)
            trace("down", down)
            return FusedPending(sq, before, down)
        return FusedPending(sq)
    act = fused_ops.silu_mul(gu[:, : 2 * I], lora=lora_gu, adapter_ids=ids)
    d = _project(act, lw, "down")
    if trace is not None:
        trace("act", act)
        trace("down", d)
    return d, lw.up("down", d, scale, a)


class FusedPending:
    """A layer's down_proj output already added, with its LoRA delta, into
    the residual stream (linear_shuffled_add).  ``sq``: the stream's sums of
    squares per 16 columns for the next RMSNorm (None: the norm's prologue
    forms them).  Under a stage trace also the stream before that add
    (``hidden_before``) and the projection's output (``down``)."""

    def __init__(self, sq, hidden_before=None, down=None) -> None:
        self.sq, self.hidden_before, self.down = sq, hidden_before, down


def _norm_prologue(cfg: DecoderConfig, T: int) -> bool:
    """The RMSNorm GEMM forms the sums of squares itself (up to 8 tokens,
    hidden a multiple of 512): faster than taking them from the producing
    GEMM (gate/up at 4 tokens 34.5 vs 36.5 us: normalizing in the main
    loop repeats the work in every wave)."""
    return T <= 8 and T * cfg.hidden <= 32768 and cfg.hidden % 512 == 0


def _sq_buffer(cfg: DecoderConfig, T: int, device):
    """The residual's sums of squares a producing GEMM hands to the next
    RMSNorm GEMM, when that one does not form them itself."""
    if _norm_prologue(cfg, T):
        return None
    return torch.empty((T, -(-cfg.hidden // 16)), dtype=torch.float32, device=device)


def _fused_norms(cfg: DecoderConfig, lw: LayerWeights, T: int) -> bool:
    """Whether a decode layer of T tokens fuses its add + RMSNorm launches
    away: the decode-sized shuffled GEMMs for q/k/v, o_proj and gate/up,
    LoRA rank 8 or 16, at most 16 tokens."""
    return (FUSE_NORMS and T <= 16 and cfg.hidden % 32 == 0 and cfg.hidden <= 8192 and cfg.lora_rank in (8, 16)
            and all(p in lw.shuffled for p in ("qkv", "o", "gate_up")) and lw.y_offset["o"] == cfg.hidden)


def _fused_down(cfg: DecoderConfig, lw: LayerWeights) -> bool:
    """down_proj's delta and residual add in its GEMM as well (its shrink in
    SiLU*up)."""
    return (FUSE_DOWN_NORM and "down" in lw.shuffled and lw.y_offset["down"] == cfg.hidden
            and cfg.intermediate % 32 == 0 and cfg.intermediate <= 8192 * 4)


def _final_norm(weights: "DecoderWeights", hidden: torch.Tensor, pending, ids: torch.Tensor) -> torch.Tensor:
    if isinstance(pending, FusedPending):
        return fused_ops.rmsnorm(hidden, weights.final_norm, weights.cfg.rms_eps)
    prev_out, prev_up = pending
    return fused_ops.add_rmsnorm(hidden, _cols(prev_out, weights.cfg.hidden), weights.final_norm,
                                 weights.cfg.rms_eps, lora=prev_up, adapter_ids=ids)


def decode_layer_static(
    cfg: DecoderConfig,
    lw: LayerWeights,
    lora_scale: float,
    hidden: torch.Tensor,
    pending,
    layer_cache: torch.Tensor,
    backend: PagedDecodeAttention,
    ctx: DecodeContext,
):
    """One single-token decode layer for the whole batch; graph-capturable
    (the reference's run_flashinfer_decode_layer_static_append_batch,
    layer_runner.py:340-396).  See :func:`_layer` for ``pending``."""

    def attend(q):
        out = torch.empty_like(q)
        backend.run_decode_into(q, layer_cache, out)
        return out

    def qkv_attend(qkv, lora, o_shrink=None):
        out = torch.empty((qkv.shape[0], cfg.num_qo_heads, cfg.head_dim), dtype=qkv.dtype, device=qkv.device)
        backend.run_decode_qkv_into(
            qkv, layer_cache, out, q_norm_weight=lw.q_norm if cfg.qk_norm else None,
            k_norm_weight=lw.k_norm if cfg.qk_norm else None, rope_cos_sin=ctx.rope_cos_sin,
            page_id=ctx.page_id, page_offset=ctx.page_offset, eps=cfg.rms_eps, lora=lora,
            adapter_ids=ctx.adapter_ids, o_shrink=o_shrink)
        return out

    qkv_attend.oshrink_parts = backend.oshrink_parts

    return _layer(cfg, lw, lora_scale, hidden, pending, ctx.adapter_ids, ctx.positions, ctx.page_id,
                  ctx.page_offset, layer_cache, backend.page_size, attend, ctx.uniform_adapter,
                  qkv_attend if ctx.rope_cos_sin is not None else None)


def folded_qkv_decode(cfg: DecoderConfig, dtype: torch.dtype) -> bool:
    """Whether decode layers run the q/k/v epilogue inside the attention
    kernel (pl_decode_run_qkv): built for 16-bit weights, head_dim 128, four
    q heads per kv head and LoRA rank 0/8/16."""
    return (FOLD_QKV_INTO_DECODE and dtype in (torch.bfloat16, torch.float16) and cfg.head_dim == 128
            and cfg.num_qo_heads == 4 * cfg.num_kv_heads and cfg.lora_rank in (0, 8, 16))


def decode_step_static(weights: DecoderWeights, pool: PagedKVPool, backend: PagedDecodeAttention,
                       ctx: DecodeContext) -> torch.Tensor:
    """embed -> layers -> final norm -> lm_head -> greedy argmax into ctx.next_tokens
    and ctx.tokens (the next step's input).

    Returns the logits [B, vocab] (graph-owned under capture).
    """
    cfg = weights.cfg
    hidden = F.embedding(ctx.tokens, weights.embed)
    if folded_qkv_decode(cfg, weights.dtype):
        # the step's RoPE angles, once for all layers (the first, eager call
        # allocates the buffer, before any capture)
        if ctx.rope_cos_sin is None:
            ctx.rope_cos_sin = torch.empty((ctx.batch, cfg.head_dim // 2, 2), dtype=torch.float32,
                                           device=ctx.positions.device)
        fused_ops.rope_cos_sin(ctx.positions, head_dim=cfg.head_dim, rope_theta=cfg.rope_theta,
                               out=ctx.rope_cos_sin)
    else:
        ctx.rope_cos_sin = None
    pending = None
    for li, lw in enumerate(weights.layers):
        pending = decode_layer_static(cfg, lw, weights.lora_scale, hidden, pending, pool.layer_cache(li),
                                      backend, ctx)
    trace = STAGE_TRACE
    if trace is not None:
        if isinstance(pending, FusedPending):  # the last down_proj is in hidden already
            trace("final_hidden_in", pending.hidden_before)
            trace("final_down", pending.down)
        else:
            trace("final_hidden_in", hidden)
            trace("final_down", pending[0])
    x = _final_norm(weights, hidden, pending, ctx.adapter_ids)
    logits = weights.logits(x)
    # greedy (sampling.py:8-15); the pick also becomes the next step's input token
    if ctx.argmax_ws is None:  # the first (eager) call allocates it, before any capture
        ctx.argmax_ws = fused_ops.greedy_argmax_workspace(logits.shape[0], logits.shape[1], logits.dtype,
                                                          logits.device)
    fused_ops.greedy_argmax(logits, out=ctx.next_tokens, tokens_out=ctx.tokens, workspace=ctx.argmax_ws)
    if trace is not None:
        for name, value in (("final_hidden", hidden), ("final_x", x), ("logits", logits),
                            ("next_tokens", ctx.next_tokens)):
            trace(name, value)
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

            def attend(q, cache=cache):
                return backend.run_prefill_into(q, cache, attn)

            pending = _layer(cfg, lw, s, hidden, pending, ids, pos, page_of, off_of, cache, ps, attend,
                             adapter if 0 <= adapter < weights.n_adapters else -1)
        x = _final_norm(weights, hidden, pending, ids)
        last_logits = weights.logits(x[-1:])
    return last_logits

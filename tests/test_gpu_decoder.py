"""The decode step (caller of the kernels) on a small Qwen3-shaped model.

(1) One eager decode step vs an independent torch implementation of the
    reference's static decode layer (layer_runner.py:340-412): index_put_
    append, float32 attention over the gathered pages, LoRA as chained
    F.linear calls (packed_ops.py:534-553), greedy argmax.  Bar: the
    reference's own logits gate (atol 0.1, rtol 0.01,
    scripts/check_inference_correctness.py:26-37) and identical greedy tokens.
(2) hipGraph replay vs eager over 12 steps: bit-identical tokens and logits.
"""

import copy
import math

import pytest
import torch
import torch.nn.functional as F

from pagelora_amd.decoder import DecodeContext, DecoderConfig, DecoderWeights, decode_step_static
from pagelora_amd.generation import BatchGenerator, prefill_requests
from pagelora_amd.kv_pool import PagedKVPool

pytestmark = pytest.mark.gpu

SMALL = DecoderConfig(num_layers=2, hidden=256, num_qo_heads=8, num_kv_heads=2, head_dim=64, intermediate=512,
                      vocab=1000, lora_rank=16, lora_alpha=32.0)


def _setup(dev, seed=0, capacity_pages=64):
    w = DecoderWeights(SMALL, n_adapters=2, device=dev, seed=seed)
    pool = PagedKVPool(num_layers=SMALL.num_layers, capacity_pages=capacity_pages, page_size=16, num_kv_heads=2,
                       head_dim=64, dtype=torch.bfloat16, device=dev)
    g = torch.Generator().manual_seed(7)
    prefix = torch.randint(0, SMALL.vocab, (32,), generator=g)
    prompts = [torch.randint(0, SMALL.vocab, (n,), generator=g) for n in (5, 17, 1)]
    reqs, first, logits = prefill_requests(w, pool, prompts, shared_prefix=prefix, adapters=[0, 1, 1])
    return w, pool, reqs, first, logits


def _rms(x, w, eps):
    xf = x.float()
    return w * (xf / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)


def _rope(x, pos, d, theta):
    inv = theta ** (-torch.arange(0, d, 2, device=x.device, dtype=torch.float64) / d)
    ang = pos.double()[:, None] * inv[None]
    c, s = torch.cos(ang).float(), torch.sin(ang).float()
    x1, x2 = x.float()[..., : d // 2], x.float()[..., d // 2:]
    c, s = c[:, None, :], s[:, None, :]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1).to(x.dtype)


def _torch_reference_step(w, cache, reqs, tokens, adapters):
    """Independent restatement of one batched static decode step."""
    cfg = w.cfg
    ps = 16
    B = len(reqs)
    pos = torch.tensor([r.length - 1 for r in reqs], device=cache.device)
    slots = [r.slot(r.length - 1, ps) for r in reqs]
    page_id = torch.tensor([p for p, _ in slots], device=cache.device)
    off = torch.tensor([o for _, o in slots], device=cache.device)
    hidden = w.embed[tokens]
    s = w.lora_scale
    for li, lw in enumerate(w.layers):
        x = _rms(hidden, lw.input_norm, cfg.rms_eps)
        outs = []
        for name, W in (("q", lw.w_qkv[: cfg.q_dim]), ("k", lw.w_qkv[cfg.q_dim: cfg.q_dim + cfg.kv_dim]),
                        ("v", lw.w_qkv[cfg.q_dim + cfg.kv_dim:])):
            A, Bm = lw.lora[name]
            base = F.linear(x, W)
            delta = torch.stack([F.linear(F.linear(x[b], A[adapters[b]]), Bm[adapters[b]]) for b in range(B)]) * s
            outs.append(base + delta)
        q = outs[0].view(B, cfg.num_qo_heads, cfg.head_dim)
        k = outs[1].view(B, cfg.num_kv_heads, cfg.head_dim)
        v = outs[2].view(B, cfg.num_kv_heads, cfg.head_dim)
        q = _rope(_rms(q, lw.q_norm, cfg.rms_eps), pos, cfg.head_dim, cfg.rope_theta)
        k = _rope(_rms(k, lw.k_norm, cfg.rms_eps), pos, cfg.head_dim, cfg.rope_theta)
        layer = cache[li]
        layer.index_put_((page_id, torch.zeros_like(page_id), off), k)
        layer.index_put_((page_id, torch.ones_like(page_id), off), v)
        attn = []
        for b, r in enumerate(reqs):
            kk = torch.cat([layer[p, 0] for p in r.pages()])[: r.length].float()   # [L, Hkv, D]
            vv = torch.cat([layer[p, 1] for p in r.pages()])[: r.length].float()
            g = cfg.num_qo_heads // cfg.num_kv_heads
            kk = kk.repeat_interleave(g, dim=1)
            vv = vv.repeat_interleave(g, dim=1)
            sc = torch.einsum("hd,lhd->hl", q[b].float(), kk) / math.sqrt(cfg.head_dim)
            attn.append(torch.einsum("hl,lhd->hd", sc.softmax(-1), vv).to(hidden.dtype))
        attn = torch.stack(attn).view(B, cfg.q_dim)
        Ao, Bo = lw.lora["o"]
        o = F.linear(attn, lw.w_o) + torch.stack(
            [F.linear(F.linear(attn[b], Ao[adapters[b]]), Bo[adapters[b]]) for b in range(B)]) * s
        hidden = hidden + o
        x2 = _rms(hidden, lw.post_norm, cfg.rms_eps)
        I = cfg.intermediate
        gu = []
        for name, W in (("gate", lw.w_gate_up[:I]), ("up", lw.w_gate_up[I:])):
            A, Bm = lw.lora[name]
            gu.append(F.linear(x2, W) + torch.stack(
                [F.linear(F.linear(x2[b], A[adapters[b]]), Bm[adapters[b]]) for b in range(B)]) * s)
        act = F.silu(gu[0]) * gu[1]
        Ad, Bd = lw.lora["down"]
        d = F.linear(act, lw.w_down) + torch.stack(
            [F.linear(F.linear(act[b], Ad[adapters[b]]), Bd[adapters[b]]) for b in range(B)]) * s
        hidden = hidden + d
    logits = F.linear(_rms(hidden, w.final_norm, cfg.rms_eps), w.lm_head)
    return logits.float(), logits.argmax(-1)


def _assert_same_greedy(tokens, ref_logits, logits):
    """The greedy pick must equal the reference's wherever the reference's
    top-1 / top-2 margin exceeds twice the largest logit difference (a near
    tie inside the numerical error may go either way)."""
    err = (logits - ref_logits).abs().max().item()
    top2 = ref_logits.topk(2, dim=-1).values
    margin = (top2[..., 0] - top2[..., 1]).reshape(-1)
    ref_tok = ref_logits.argmax(-1).reshape(-1)
    tokens = tokens.reshape(-1)
    decided = margin > 2 * err
    assert decided.any(), f"every row is a near tie (margins {margin.tolist()}, err {err:.4f})"
    assert torch.equal(tokens[decided], ref_tok[decided]), (
        f"tokens {tokens.tolist()} vs {ref_tok.tolist()}, margins {margin.tolist()}, err {err:.4f}")


def test_decode_step_matches_torch_reference(gpu_device):
    w, pool, reqs, first, _ = _setup(gpu_device)
    adapters = [0, 1, 1]
    gen = BatchGenerator(w, pool, workspace_mb=8, use_graph=False)
    ctx = DecodeContext(len(reqs), gpu_device)
    gen._stage_inputs(ctx, reqs, adapters)
    gen._plan(reqs)
    ctx.tokens.copy_(first)
    ref_cache = pool.cache.clone()
    logits = decode_step_static(w, pool, gen.backend, ctx).float()
    ref_logits, ref_tok = _torch_reference_step(w, ref_cache, reqs, first, adapters)
    torch.cuda.synchronize()
    assert torch.allclose(logits, ref_logits, atol=0.1, rtol=0.01), (logits - ref_logits).abs().max()
    _assert_same_greedy(ctx.next_tokens, ref_logits, logits)
    # the appended K/V slot equals the reference's index_put_ (same rounded inputs)
    for r in reqs:
        p, o = r.slot(r.length - 1, 16)
        diff = (pool.cache[:, p, :, o].float() - ref_cache[:, p, :, o].float()).abs().max()
        assert diff <= 0.05, diff


def test_graph_replay_matches_eager(gpu_device):
    results = []
    for use_graph in (False, True):
        w, pool, reqs, first, _ = _setup(gpu_device)
        gen = BatchGenerator(w, pool, workspace_mb=8, use_graph=use_graph)
        res = gen.generate(reqs, first, steps=12, adapters=[0, 1, 1])
        assert res.used_graph == use_graph
        results.append(res)
    assert torch.equal(results[0].tokens, results[1].tokens)
    assert results[1].graph_captures == 1 and results[1].graph_replays == 12


@pytest.mark.parametrize("use_graph", [False, True])
@pytest.mark.parametrize("model", ["d64", "d128_folded"])
def test_device_tables_match_host_tables(gpu_device, use_graph, model):
    # 40 steps carry every row (37, 49 and 33 tokens) across a page boundary;
    # the device-grown table must give the same tokens as host packing (with
    # head_dim 128 the attention kernel also forms q and appends k/v).
    steps = 40
    setup = _setup if model == "d64" else (lambda dev: _setup128(dev))
    w, pool, reqs, first, _ = setup(gpu_device)
    ref = BatchGenerator(w, pool, workspace_mb=8, use_graph=False).generate(reqs, first, steps, [0, 1, 1])
    w, pool, reqs, first, _ = setup(gpu_device)
    gen = BatchGenerator(w, pool, workspace_mb=8, use_graph=use_graph)
    res = gen.generate(reqs, first, steps, [0, 1, 1], device_tables=True)
    assert res.used_graph == use_graph
    assert torch.equal(res.tokens, ref.tokens)
    # the table grown on the device is the host's table of the grown rows
    indptr, indices, last = pool.tables(reqs)
    ip_buf, ind_buf, last_buf = gen.backend._decode_graph_buffers
    assert ip_buf.tolist() == indptr.tolist()
    assert ind_buf[: indptr[-1]].tolist() == indices.tolist()
    assert last_buf.tolist() == last.tolist()
    assert res.extra["reserve_uploads"] <= steps // 16 + 2
    if use_graph:
        assert res.graph_captures == 1 and res.graph_replays == steps


def _lora_seq(x, W, lora, adapter, s):
    A, Bm = lora
    return F.linear(x, W) + F.linear(F.linear(x, A[adapter]), Bm[adapter]) * s


def _torch_reference_prefill(w, tokens, adapter):
    """Independent restatement of a whole-prompt prefill: dense causal float32
    attention over the sequence (no pages), LoRA as chained F.linear."""
    cfg = w.cfg
    T = tokens.numel()
    pos = torch.arange(T, device=tokens.device)
    hidden = w.embed[tokens]
    s = w.lora_scale
    g = cfg.num_qo_heads // cfg.num_kv_heads
    for lw in w.layers:
        x = _rms(hidden, lw.input_norm, cfg.rms_eps)
        q = _lora_seq(x, lw.w_qkv[: cfg.q_dim], lw.lora["q"], adapter, s).view(T, cfg.num_qo_heads, cfg.head_dim)
        k = _lora_seq(x, lw.w_qkv[cfg.q_dim: cfg.q_dim + cfg.kv_dim], lw.lora["k"], adapter, s)
        v = _lora_seq(x, lw.w_qkv[cfg.q_dim + cfg.kv_dim:], lw.lora["v"], adapter, s)
        k = k.view(T, cfg.num_kv_heads, cfg.head_dim)
        v = v.view(T, cfg.num_kv_heads, cfg.head_dim)
        q = _rope(_rms(q, lw.q_norm, cfg.rms_eps), pos, cfg.head_dim, cfg.rope_theta)
        k = _rope(_rms(k, lw.k_norm, cfg.rms_eps), pos, cfg.head_dim, cfg.rope_theta)
        qf = q.float().transpose(0, 1)                                           # [Hq, T, D]
        kf = k.float().repeat_interleave(g, dim=1).transpose(0, 1)               # [Hq, T, D]
        vf = v.float().repeat_interleave(g, dim=1).transpose(0, 1)
        sc = torch.matmul(qf, kf.transpose(1, 2).contiguous()) / math.sqrt(cfg.head_dim)
        sc = sc.masked_fill(torch.ones(T, T, dtype=torch.bool, device=sc.device).triu(1), float("-inf"))
        attn = torch.matmul(sc.softmax(-1), vf).transpose(0, 1).reshape(T, cfg.q_dim).to(hidden.dtype)
        hidden = hidden + _lora_seq(attn, lw.w_o, lw.lora["o"], adapter, s)
        x2 = _rms(hidden, lw.post_norm, cfg.rms_eps)
        I = cfg.intermediate
        act = F.silu(_lora_seq(x2, lw.w_gate_up[:I], lw.lora["gate"], adapter, s)) * _lora_seq(
            x2, lw.w_gate_up[I:], lw.lora["up"], adapter, s)
        hidden = hidden + _lora_seq(act, lw.w_down, lw.lora["down"], adapter, s)
    logits = F.linear(_rms(hidden, w.final_norm, cfg.rms_eps), w.lm_head)
    return logits[-1:].float()


@pytest.mark.parametrize("chunk", [8192, 48])
def test_prefill_matches_torch_reference(gpu_device, chunk):
    """Paged prefill (kernel attention, optionally in 48-token segments over
    the cached prefix) vs the dense torch restatement: the reference's logits
    gate (atol 0.1, rtol 0.01) and the same greedy token."""
    from pagelora_amd.decoder import prefill
    from pagelora_amd.kv_pool import Request

    w = DecoderWeights(SMALL, n_adapters=2, device=gpu_device, seed=3)
    pool = PagedKVPool(num_layers=SMALL.num_layers, capacity_pages=64, page_size=16, num_kv_heads=2, head_dim=64,
                       dtype=torch.bfloat16, device=gpu_device)
    tokens = torch.randint(0, SMALL.vocab, (203,), generator=torch.Generator().manual_seed(11)).to(gpu_device)
    r = Request()
    pool.reserve(r, tokens.numel())
    got = prefill(w, pool, r, tokens, adapter=1, chunk=chunk).float()
    ref = _torch_reference_prefill(w, tokens, adapter=1)
    torch.cuda.synchronize()
    assert torch.allclose(got, ref, atol=0.1, rtol=0.01), f"max diff {(got - ref).abs().max().item():.4f}"
    _assert_same_greedy(got.argmax(-1), ref, got)


@pytest.mark.parametrize("device_tables", [False, True])
def test_uniform_adapter_matches_per_row_ids(gpu_device, device_tables, monkeypatch):
    # every row on adapter 1: the kernels take the bound adapter (no id loads);
    # forcing per-row ids instead must give the same tokens bit for bit
    results = []
    for force_per_row in (False, True):
        w, pool, reqs, first, _ = _setup(gpu_device)
        gen = BatchGenerator(w, pool, workspace_mb=8, use_graph=True)
        if force_per_row:
            monkeypatch.setattr(gen, "_uniform_adapter", lambda adapters: -1)
        res = gen.generate(reqs, first, steps=20, adapters=[1, 1, 1], device_tables=device_tables)
        assert res.used_graph
        results.append(res.tokens)
    assert torch.equal(results[0], results[1])


# head_dim 128 and four q heads per kv head: the shape whose decode layers
# form q and append k/v inside the attention kernel (pl_decode_run_qkv)
SMALL128 = DecoderConfig(num_layers=2, hidden=512, num_qo_heads=4, num_kv_heads=1, head_dim=128, intermediate=512,
                         vocab=1000, lora_rank=16, lora_alpha=32.0)


def _setup128(dev, seed=0):
    w = DecoderWeights(SMALL128, n_adapters=2, device=dev, seed=seed)
    pool = PagedKVPool(num_layers=SMALL128.num_layers, capacity_pages=64, page_size=16, num_kv_heads=1,
                       head_dim=128, dtype=torch.bfloat16, device=dev)
    pool.cache.zero_()  # slots no token uses hold zeros, so whole caches compare
    g = torch.Generator().manual_seed(9)
    prefix = torch.randint(0, SMALL128.vocab, (32,), generator=g)
    prompts = [torch.randint(0, SMALL128.vocab, (n,), generator=g) for n in (5, 17, 1)]
    reqs, first, logits = prefill_requests(w, pool, prompts, shared_prefix=prefix, adapters=[0, 1, 1])
    return w, pool, reqs, first, logits


def _eager_step(w, pool, reqs, first, adapters, dev):
    gen = BatchGenerator(w, pool, workspace_mb=8, use_graph=False)
    ctx = DecodeContext(len(reqs), dev)
    gen._stage_inputs(ctx, reqs, adapters)
    gen._plan(reqs)
    ctx.tokens.copy_(first)
    logits = decode_step_static(w, pool, gen.backend, ctx).float()
    return logits, ctx.next_tokens.clone()


def test_folded_qkv_step_matches_torch_reference(gpu_device):
    from pagelora_amd import decoder
    assert decoder.folded_qkv_decode(SMALL128, torch.bfloat16)
    w, pool, reqs, first, _ = _setup128(gpu_device)
    adapters = [0, 1, 1]
    ref_cache = pool.cache.clone()
    logits, toks = _eager_step(w, pool, reqs, first, adapters, gpu_device)
    ref_logits, _ = _torch_reference_step(w, ref_cache, reqs, first, adapters)
    torch.cuda.synchronize()
    assert torch.allclose(logits, ref_logits, atol=0.1, rtol=0.01), (logits - ref_logits).abs().max()
    _assert_same_greedy(toks, ref_logits, logits)
    for r in reqs:  # the k/v the attention kernel appended equal the reference's index_put_
        p, o = r.slot(r.length - 1, 16)
        diff = (pool.cache[:, p, :, o].float() - ref_cache[:, p, :, o].float()).abs().max()
        assert diff <= 0.05, diff


def test_folded_qkv_matches_separate_epilogue(gpu_device, monkeypatch):
    from pagelora_amd import decoder
    out = []
    for fold in (True, False):
        monkeypatch.setattr(decoder, "FOLD_QKV_INTO_DECODE", fold)
        w, pool, reqs, first, _ = _setup128(gpu_device)
        out.append(_eager_step(w, pool, reqs, first, [0, 1, 1], gpu_device) + (pool.cache.clone(),))
    (lf, tf, cf), (ls, ts, cs) = out
    torch.cuda.synchronize()
    # q (and the appended k) differ by at most one rounding: the head norm sums in another order
    assert torch.allclose(lf, ls, atol=0.05, rtol=0.01), (lf - ls).abs().max()
    _assert_same_greedy(tf, ls, lf)
    assert torch.allclose(cf.float(), cs.float(), atol=0.05, rtol=0.02)


@pytest.mark.parametrize("fuse", ["post_attention", "both"])
def test_fused_norms_match_add_rmsnorm(gpu_device, monkeypatch, fuse):
    """The add + RMSNorm launches fused away (o_proj's shrink in the merge,
    down_proj's in SiLU*up, each projection + delta + residual add in one
    GEMM, the norms in the q/k/v and gate/up GEMMs' prologues) against the
    add+RMSNorm kernels between separate projections: the same logits to
    within the roundings that move (y's sum order, the norms' sums of
    squares), the same greedy tokens, and the appended K/V of layer 0 bit for
    bit (computed before any fused part)."""
    from pagelora_amd import decoder
    out = []
    for on in (True, False):
        monkeypatch.setattr(decoder, "FUSE_NORMS", on)
        monkeypatch.setattr(decoder, "FUSE_DOWN_NORM", on and fuse == "both")
        w, pool, reqs, first, _ = _setup128(gpu_device)
        out.append(_eager_step(w, pool, reqs, first, [0, 1, 1], gpu_device) + (pool.cache.clone(),))
    (lf, tf, cf), (ls, ts, cs) = out
    torch.cuda.synchronize()
    assert torch.allclose(lf, ls, atol=0.05, rtol=0.01), (lf - ls).abs().max()
    _assert_same_greedy(tf, ls, lf)
    assert torch.equal(cf[0], cs[0])
    assert torch.allclose(cf.float(), cs.float(), atol=0.05, rtol=0.02)


def test_folded_qkv_graph_replay_matches_eager(gpu_device):
    runs = []
    for use_graph in (False, True):
        w, pool, reqs, first, _ = _setup128(gpu_device)
        gen = BatchGenerator(w, pool, workspace_mb=8, use_graph=use_graph)
        res = gen.generate(reqs, first, steps=12, adapters=[0, 1, 1])
        assert res.used_graph == use_graph
        runs.append(res.tokens)
    assert torch.equal(runs[0], runs[1])


def test_side_plane_projections_match_split_projections(gpu_device, monkeypatch):
    """o_proj / down_proj with their LoRA A rows on side planes (the default)
    against the earlier layout (down split 3 ways, o whole): the same logits
    to within the rounding of y, the same greedy tokens."""
    from pagelora_amd import decoder
    out = []
    for side in (True, False):
        if not side:
            monkeypatch.setattr(decoder, "DECODE_SIDE_SPLITS", {})
            monkeypatch.setattr(decoder, "DECODE_SPLITS", {"down": 3})
        w, pool, reqs, first, _ = _setup128(gpu_device)
        out.append(_eager_step(w, pool, reqs, first, [0, 1, 1], gpu_device))
    (ls, ts), (lp, tp) = out
    torch.cuda.synchronize()
    assert torch.allclose(ls, lp, atol=0.05, rtol=0.01), (ls - lp).abs().max()
    _assert_same_greedy(ts, lp, ls)


def test_graph_follows_page_table_buffers_that_move(gpu_device):
    """Host-packed tables in a small persistent buffer: the batch's page list
    (10 pages at the start, 16-entry buffer) outgrows it mid-generation, the
    plan moves the buffers, and generate() must switch to a graph captured on
    the new ones.  Tokens equal the eager run's; two captures."""
    steps = 48
    w, pool, reqs, first, _ = _setup(gpu_device)
    ref = BatchGenerator(w, pool, workspace_mb=8, use_graph=False).generate(reqs, first, steps, [0, 1, 1])
    w, pool, reqs, first, _ = _setup(gpu_device)
    gen = BatchGenerator(w, pool, workspace_mb=8, use_graph=True)
    gen.backend.max_pages = 0  # start at the smallest pow2 capacity
    start_pages = len(pool.tables(reqs)[1])
    res = gen.generate(reqs, first, steps, [0, 1, 1])
    end_pages = len(pool.tables(reqs)[1])
    assert start_pages + 1 <= 16 < end_pages, (start_pages, end_pages)
    assert res.used_graph and res.graph_captures == 2, res.graph_captures
    assert torch.equal(res.tokens, ref.tokens)


@pytest.mark.parametrize("device_tables", [False, True])
def test_pool_growth_mid_generation_matches_unconstrained(gpu_device, device_tables):
    """A pool that runs out while rows grow (8 pages: the prompts fill 7)
    grows to a new tensor between graph replays (paged_kv_store.py:543-579),
    keeping every page id; the next step recaptures once on the new pool.
    Tokens and logits equal those of a pool large enough never to grow."""
    results = []
    for cap in (256, 8):
        w, pool, reqs, first, _ = _setup(gpu_device, capacity_pages=cap)
        gen = BatchGenerator(w, pool, workspace_mb=8, use_graph=True)
        grown_at = []
        grow = pool.allocator._grow

        def recording_grow(required, grow=grow, gen=gen, grown_at=grown_at):
            grown_at.append(gen.graphs.replay_count)
            return grow(required)

        pool.allocator._grow = recording_grow
        res = gen.generate(reqs, first, steps=80, adapters=[0, 1, 1], device_tables=device_tables,
                           keep_logits=True)
        assert res.used_graph
        results.append((res.tokens, res.extra["logits"], grown_at, pool, res.graph_captures))
    (t0, l0, g0, p0, c0), (t1, l1, g1, p1, c1) = results
    assert g0 == [] and p0.grow_count == 0
    assert p1.grow_count >= 1 and any(r > 0 for r in g1), g1  # grown between replays
    assert p1.capacity_pages >= 16
    assert c1 >= c0 + 1  # captured again on the grown pool
    assert torch.equal(t0, t1)
    assert torch.equal(l0, l1)


def test_capture_with_collectable_pinned_staging_and_events(gpu_device):
    """Graph capture while the cyclic collector holds garbage that owns pinned
    host memory and HIP events (an earlier generator's staging left in a
    reference cycle), with the collector set to run at almost every
    allocation: the runner collects before capturing and keeps the collector
    off while the stream captures, so no destructor makes a HIP call during
    capture.  The captured run's tokens equal an eager run's."""
    import gc

    from pagelora_amd.generation import _PinnedRing

    w, pool, reqs, first, _ = _setup(gpu_device)
    for _ in range(8):
        ring = _PinnedRing(2, (4096,), torch.int32)
        for slot in range(2):
            ring.record(slot)
        ring.cycle = ring  # only the cyclic collector can free it
    del ring
    old = gc.get_threshold()
    gc.set_threshold(1, 1, 1)
    try:
        gen = BatchGenerator(w, pool, workspace_mb=8, use_graph=True)
        got = gen.generate(reqs, first, steps=6)
    finally:
        gc.set_threshold(*old)
    assert got.used_graph and gen.graphs.disabled_reason is None
    w2, pool2, reqs2, first2, _ = _setup(gpu_device)
    want = BatchGenerator(w2, pool2, workspace_mb=8, use_graph=False).generate(reqs2, first2, steps=6)
    assert torch.equal(got.tokens, want.tokens)

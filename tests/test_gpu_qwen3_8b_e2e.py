"""End-to-end decode at the Qwen3-8B shape (36 layers, hidden 4096, 32/8
heads, head_dim 128, intermediate 12288, vocab 151936, bf16, rank-16
no-merge LoRA on all seven modules, random init), on the two workloads the
end-to-end tok/s is quoted on:

  shared4  4 rows behind a 2048-token prefix held in shared pages, each with
           its own 64-token suffix, 16 greedy steps
  long32k  1 row at 32768 tokens, 4 greedy steps

For each:
  (a) hipGraph replay == eager: tokens and every step's logits bit-identical
      (the reference's eager-vs-graph gate, scripts/check_inference_correctness.py:17-61,
      here exact);
  (b) the page table grown on the device inside the captured step == the
      host-packed table: the same tokens, and the final device table equals
      the host's packing of the grown rows;
  (c) layer 0 (and layer 1's input) of the first decode step, stage by
      stage, against the float64 oracle applied to the kernels' own stored
      inputs of each stage (oracle.fused, oracle.lora, oracle.paged_decode;
      the stages of layer_runner.py:340-412).  Bar: 2e-3 + one bf16 rounding
      of the output (2^-8 relative); where a stage rounds an intermediate
      before its output (the module output + LoRA delta before the head norm
      and RoPE or the SiLU, the delta before the residual add), also one
      rounding of that intermediate carried to the output (2^-8 times the
      magnitude the intermediate contributes to each output element).
"""

import gc
import math

import numpy as np
import pytest
import torch

from oracle import fused as of
from oracle import lora as ol
from oracle import paged_decode as opd
from pagelora_amd import decoder
from pagelora_amd.decoder import QWEN3_8B, DecodeContext, DecoderWeights, SideOutput, decode_step_static
from pagelora_amd.generation import BatchGenerator, prefill_requests
from pagelora_amd.kv_pool import PagedKVPool
from pagelora_amd.linear import SplitOutput

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

CFG = QWEN3_8B
PS = 16
ULP = 2.0**-8  # one bf16 rounding, relative

WORKLOADS = {
    "shared4": dict(prefix_len=2048, suffix_len=64, rows=4, steps=16),
    "long32k": dict(prefix_len=0, suffix_len=32768, rows=1, steps=4),
}


@pytest.fixture(scope="module")
def weights(gpu_device):
    print("[qwen3-8b] building 36-layer random-init weights", flush=True)
    w = DecoderWeights(CFG, n_adapters=1, device=gpu_device, seed=0)
    torch.cuda.synchronize()
    yield w
    del w
    gc.collect()
    torch.cuda.empty_cache()


def _fresh(w, dev, prefix_len, suffix_len, rows, steps, seed=5):
    """A new pool with the workload's rows prefilled (deterministic: every
    call gives the same caches and first tokens)."""
    pages = (prefix_len + rows * (suffix_len + steps + 2 * PS)) // PS + 8 * rows + 8
    pool = PagedKVPool(num_layers=CFG.num_layers, capacity_pages=pages, page_size=PS, num_kv_heads=CFG.num_kv_heads,
                       head_dim=CFG.head_dim, dtype=torch.bfloat16, device=dev)
    g = torch.Generator().manual_seed(seed)
    prefix = torch.randint(0, CFG.vocab, (prefix_len,), generator=g) if prefix_len else None
    prompts = [torch.randint(0, CFG.vocab, (suffix_len,), generator=g) for _ in range(rows)]
    reqs, first, _ = prefill_requests(w, pool, prompts, shared_prefix=prefix)
    return pool, reqs, first


def _f(t):
    return t.float().cpu().numpy().astype(np.float64)


def _check(name, got, want, carried=0.0, atol=2e-3):
    """err <= atol + one rounding of want + one rounding of the carried
    intermediate magnitude ``carried`` (0 for stages with a single rounding)."""
    got = np.asarray(got, dtype=np.float64)
    err = np.abs(got - want)
    bound = atol + ULP * (np.abs(want) + carried)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    worst = float((err / bound).max())
    assert worst <= 1.0, f"{name}: max err {err.max():.3e}, worst err/bound {worst:.2f}"
    return worst


class _Recorder:
    """STAGE_TRACE target: copies of the first two layers' stage outputs."""

    def __init__(self):
        self.layers = []

    def __call__(self, name, value):
        if name == "hidden_in":
            self.layers.append({})
        if len(self.layers) > 2:
            return
        if isinstance(value, SideOutput):
            value = (value.main.clone(), value.side.sum())  # planes summed in order and rounded, as consumed
        elif isinstance(value, SplitOutput):
            value = value.sum()
        else:
            value = value.clone()
        self.layers[-1][name] = value


def _stage_check(w, pool, reqs, first, dev):
    """One eager decode step with the stage recorder on; every stage of
    layer 0 (and layer 1's input add) against the oracle."""
    gen = BatchGenerator(w, pool, workspace_mb=64, use_graph=False)
    B = len(reqs)
    ctx = DecodeContext(B, dev)
    gen._stage_inputs(ctx, reqs, [0] * B)
    gen._plan(reqs)
    ctx.tokens.copy_(first)
    ctx.uniform_adapter = 0
    rec = _Recorder()
    decoder.STAGE_TRACE = rec
    try:
        decode_step_static(w, pool, gen.backend, ctx)
    finally:
        decoder.STAGE_TRACE = None
    torch.cuda.synchronize()
    L0, L1 = rec.layers[0], rec.layers[1]
    lw, s, eps = w.layers[0], w.lora_scale, CFG.rms_eps
    hq, hkv, d, h, I, r = CFG.num_qo_heads, CFG.num_kv_heads, CFG.head_dim, CFG.hidden, CFG.intermediate, CFG.lora_rank
    qd, kd = hq * d, hkv * d
    worst = {}

    def B_of(name):
        return _f(lw.lora[name][1][0])  # adapter 0's B [out, r]

    # input RMSNorm (norm.py:15-24)
    hid = _f(L0["hidden_in"])
    worst["input_norm"] = _check("input_norm", _f(L0["x"]), of.rmsnorm(hid, _f(lw.input_norm), eps))
    # q/k/v GEMM on [W_qkv; A_q; A_k; A_v] (packed_ops.py:143 and the shrink F.linear(x, A_cat))
    x = _f(L0["x"])
    qkv = _f(L0["qkv"])
    worst["qkv_gemm"] = _check("qkv_gemm", qkv, ol.linear(x, _f(lw.w_qkv_ext)))
    # module outputs with the LoRA up-projection (the module output is
    # rounded before the head norm), head norm + RoPE (projection.py:155-190,
    # 248-260), append (layer_runner.py:399-412)
    mods = {}
    for name, lo, hi in (("q", 0, qd), ("k", qd, qd + kd), ("v", qd + kd, qd + 2 * kd)):
        y = qkv[:, lw.y_offset[name]: lw.y_offset[name] + r]
        mods[name] = ol.round_bf16(qkv[:, lo:hi] + ol.up_projection(y, B_of(name), s))
    pos = np.array([rq.length - 1 for rq in reqs])
    q_want, k_want, v_want = of.qk_norm_rope_append(np.concatenate([mods["q"], mods["k"], mods["v"]], 1), hq, hkv, d,
                                                    _f(lw.q_norm), _f(lw.k_norm), pos, eps, CFG.rope_theta)

    def carried_norm_rope(m, heads, wnorm):
        # |d out / d m| |m|: the head norm scales element i by w_i / rms(head),
        # RoPE output i mixes elements i and i +- D/2 by |cos|, |sin|
        mh = np.abs(m).reshape(len(reqs), heads, d)
        rms = np.sqrt((m.reshape(len(reqs), heads, d) ** 2).mean(-1, keepdims=True) + eps)
        n = mh * np.abs(wnorm) / rms
        ang = pos.astype(np.float32)[:, None] * of.inv_freq_f32(d, CFG.rope_theta)[None, :]
        c, sn = np.abs(np.cos(ang.astype(np.float64)))[:, None, :], np.abs(np.sin(ang.astype(np.float64)))[:, None, :]
        lo_, hi_ = n[..., : d // 2], n[..., d // 2:]
        return np.concatenate([lo_ * c + hi_ * sn, hi_ * c + lo_ * sn], -1)

    k_carry = carried_norm_rope(mods["k"], hkv, _f(lw.k_norm))
    layer0 = pool.cache[0]
    for b, rq in enumerate(reqs):
        p, o = rq.slot(rq.length - 1, PS)
        worst["k_append"] = max(worst.get("k_append", 0),
                                _check(f"k_append row {b}", _f(layer0[p, 0, o]), k_want[b], k_carry[b]))
        worst["v_append"] = max(worst.get("v_append", 0),
                                _check(f"v_append row {b}", _f(layer0[p, 1, o]), v_want[b],
                                       np.abs(mods["v"][b]).reshape(hkv, d)))
    # paged decode attention over the row's pages as stored, the new token included
    indptr, indices, last = pool.tables(reqs)
    used = sorted(set(indices.tolist()))
    remap = {pg: i for i, pg in enumerate(used)}
    cache_h = _f(layer0[torch.tensor(used, device=layer0.device)])
    o_want, _ = opd.paged_decode(ol.round_bf16(q_want), cache_h, indptr, [remap[int(pg)] for pg in indices], last)
    attn = _f(L0["attn"]).reshape(len(reqs), hq, d)
    # q is formed and rounded inside the kernel: one more rounding of the output's scale
    worst["attention"] = _check("attention", attn, o_want, np.abs(o_want))
    # o_proj: base rows and the LoRA A rows' intermediate (side planes)
    attn2 = attn.reshape(len(reqs), qd)
    o_main, o_y = L0["o"]
    worst["o_gemm"] = _check("o_gemm", _f(o_main), ol.linear(attn2, _f(lw.w_o)))
    worst["o_shrink"] = _check("o_shrink", _f(o_y)[:, :r], ol.linear(attn2, _f(lw.lora["o"][0][0])))
    # residual add of o + its delta, post-attention RMSNorm (norm.py:27-57)
    o_mod = ol.round_bf16(_f(o_main) + ol.up_projection(_f(o_y)[:, :r], B_of("o"), s))
    worst["o_residual"] = _check("o_residual", _f(L0["hidden_mid"]), hid + o_mod, np.abs(o_mod))
    worst["post_norm"] = _check("post_norm", _f(L0["x2"]), of.rmsnorm(_f(L0["hidden_mid"]), _f(lw.post_norm), eps))
    # gate/up GEMM, SiLU(gate) * up with both deltas (packed_ops.py:168-239)
    x2 = _f(L0["x2"])
    gu = _f(L0["gate_up"])
    worst["gate_up_gemm"] = _check("gate_up_gemm", gu, ol.linear(x2, _f(lw.w_gate_up_ext)))
    gate = ol.round_bf16(gu[:, :I] + ol.up_projection(gu[:, lw.y_offset["gate"]: lw.y_offset["gate"] + r],
                                                      B_of("gate"), s))
    up = ol.round_bf16(gu[:, I:2 * I] + ol.up_projection(gu[:, lw.y_offset["up"]: lw.y_offset["up"] + r],
                                                         B_of("up"), s))
    sig = 1.0 / (1.0 + np.exp(-gate))
    act_carry = np.abs(sig * (1.0 + gate * (1.0 - sig)) * gate * up) + np.abs(gate * sig * up)
    worst["silu_mul"] = _check("silu_mul", _f(L0["act"]), of.silu_mul(np.concatenate([gate, up], 1)), act_carry)
    # down_proj, whose delta lands in layer 1's input add + RMSNorm
    act = _f(L0["act"])
    d_main, d_y = L0["down"]
    worst["down_gemm"] = _check("down_gemm", _f(d_main), ol.linear(act, _f(lw.w_down)))
    worst["down_shrink"] = _check("down_shrink", _f(d_y)[:, :r], ol.linear(act, _f(lw.lora["down"][0][0])))
    d_mod = ol.round_bf16(_f(d_main) + ol.up_projection(_f(d_y)[:, :r], B_of("down"), s))
    worst["down_residual"] = _check("down_residual", _f(L1["hidden"]), _f(L1["hidden_in"]) + d_mod, np.abs(d_mod))
    worst["next_input_norm"] = _check("next_input_norm", _f(L1["x"]),
                                      of.rmsnorm(_f(L1["hidden"]), _f(w.layers[1].input_norm), eps))
    print("[qwen3-8b] stage err/bound: " + ", ".join(f"{k} {v:.2f}" for k, v in worst.items()), flush=True)


@pytest.mark.parametrize("workload", sorted(WORKLOADS))
def test_qwen3_8b_decode(weights, gpu_device, workload):
    kw = WORKLOADS[workload]
    steps = kw["steps"]
    dev = gpu_device
    print(f"[qwen3-8b] {workload}: stage check of layer 0", flush=True)
    pool, reqs, first = _fresh(weights, dev, **kw)
    _stage_check(weights, pool, reqs, first, dev)
    del pool, reqs
    runs = {}
    for name, use_graph, device_tables in (("eager", False, False), ("graph", True, False),
                                           ("graph_device_tables", True, True)):
        print(f"[qwen3-8b] {workload}: {name}, {steps} steps", flush=True)
        pool, reqs, first = _fresh(weights, dev, **kw)
        gen = BatchGenerator(weights, pool, use_graph=use_graph)
        res = gen.generate(reqs, first, steps, device_tables=device_tables, keep_logits=True)
        assert res.used_graph == use_graph
        if use_graph:
            assert res.graph_captures == 1 and res.graph_replays == steps
        if device_tables:
            indptr, indices, last = pool.tables(reqs)
            ip_buf, ind_buf, last_buf = gen.backend._decode_graph_buffers
            assert ip_buf.tolist() == indptr.tolist()
            assert ind_buf[: indptr[-1]].tolist() == indices.tolist()
            assert last_buf.tolist() == last.tolist()
        runs[name] = (res.tokens, res.extra["logits"].cpu())
        del gen, pool, reqs, res
        gc.collect()
        torch.cuda.empty_cache()
    tok_e, log_e = runs["eager"]
    for name in ("graph", "graph_device_tables"):
        tok, log = runs[name]
        assert torch.equal(tok, tok_e), f"{name}: tokens differ from eager"
        assert torch.equal(log, log_e), f"{name}: logits differ from eager (max {(log - log_e).abs().max()})"

"""Stage-by-stage check of one eager decode step against the float64 oracle.

Runs one eager step of the decoder with ``decoder.STAGE_TRACE`` recording
each stage's stored output, then applies the oracle (oracle.fused,
oracle.lora, oracle.paged_decode) to the kernels' own stored inputs of each
stage of layer 0 (and layer 1's input add): the stages of the reference's
static decode layer (layer_runner.py:340-412); then the step's end: the
final add of the last layer's down_proj output (with its LoRA
up-projection) + RMSNorm, the lm_head logits over the vocabulary, and the
greedy token.

Bar: 2e-3 + one bf16 rounding of the output (2^-8 relative); where a stage
rounds an intermediate before its output (the module output + LoRA delta
before the head norm and RoPE or the SiLU, the delta before the residual
add, y formed from partial sums before the up-projection), also one
rounding of that intermediate carried to the output (2^-8 times the
magnitude the intermediate contributes to each output element).

The adapter's A/B may be given (``adapter``: {(layer, module): (A, B)}), so
the oracle works from the values a caller bound rather than from the
decoder's own stacked copies.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import fused as of
from oracle import lora as ol
from oracle import paged_decode as opd
from pagelora_amd import decoder
from pagelora_amd.decoder import DecodeContext, PartialOutput, SideOutput, decode_step_static
from pagelora_amd.generation import BatchGenerator
from pagelora_amd.linear import SplitOutput

ULP = 2.0**-8  # one bf16 rounding, relative


def _f(t):
    return t.float().cpu().numpy().astype(np.float64)


def check(name, got, want, carried=0.0, atol=2e-3):
    """err <= atol + one rounding of want + one rounding of the carried
    intermediate magnitude ``carried`` (0 for stages with a single rounding)."""
    got = np.asarray(got, dtype=np.float64)
    err = np.abs(got - want)
    bound = atol + ULP * (np.abs(want) + carried)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    worst = float((err / bound).max())
    assert worst <= 1.0, f"{name}: max err {err.max():.3e}, worst err/bound {worst:.2f}"
    return worst


class Recorder:
    """STAGE_TRACE target: copies of the first two layers' stage outputs and
    of the step's final stages (final add + RMSNorm, logits, greedy token)."""

    def __init__(self):
        self.layers = []
        self.final = {}

    def __call__(self, name, value):
        if name == "hidden_in":
            self.layers.append({})
        final = name.startswith("final_") or name in ("logits", "next_tokens")
        if len(self.layers) > 2 and not final:
            return
        if isinstance(value, SideOutput):
            value = (value.main.clone(), value.side.sum())  # planes summed in order and rounded, as consumed
        elif isinstance(value, PartialOutput):
            # the bound adapter's rank-space row, from the producer's partial sums
            value = {"main": value.main.clone(), "y": value.partials.sum().cpu().numpy()}
        elif isinstance(value, SplitOutput):
            value = value.sum()
        else:
            value = value.clone()
        (self.final if final else self.layers[-1])[name] = value


def stage_check(w, pool, reqs, first, dev, slot=0, adapter=None):
    """One eager decode step of ``reqs`` with every row on adapter ``slot``;
    layer 0's stages against the oracle.  Returns {stage: worst err/bound}."""
    cfg = w.cfg
    ps = pool.page_size
    gen = BatchGenerator(w, pool, workspace_mb=64, use_graph=False)
    B = len(reqs)
    ctx = DecodeContext(B, dev)
    gen._stage_inputs(ctx, reqs, [slot] * B)
    gen._plan(reqs)
    ctx.tokens.copy_(first)
    ctx.uniform_adapter = slot
    rec = Recorder()
    decoder.STAGE_TRACE = rec
    try:
        decode_step_static(w, pool, gen.backend, ctx)
    finally:
        decoder.STAGE_TRACE = None
    torch.cuda.synchronize()
    L0, L1 = rec.layers[0], rec.layers[1]
    lw, s, eps = w.layers[0], w.lora_scale, cfg.rms_eps
    hq, hkv, d, I, r = cfg.num_qo_heads, cfg.num_kv_heads, cfg.head_dim, cfg.intermediate, cfg.lora_rank
    qd, kd = hq * d, hkv * d
    worst = {}

    def AB(name, layer=0):
        lwl = w.layers[layer]
        if adapter is not None:
            A, Bm = adapter.get((layer, name), (None, None))
            if A is None:  # a module the adapter leaves out: zero delta
                return np.zeros((r, lwl.lora[name][0].shape[-1])), np.zeros((lwl.lora[name][1].shape[1], r))
            return _f(torch.as_tensor(A)), _f(torch.as_tensor(Bm))
        return _f(lwl.lora[name][0][slot]), _f(lwl.lora[name][1][slot])

    def ycols(name):
        c = lw.y_offset[name] + slot * r
        return slice(c, c + r)

    # input RMSNorm (norm.py:15-24)
    hid = _f(L0["hidden_in"])
    worst["input_norm"] = check("input_norm", _f(L0["x"]), of.rmsnorm(hid, _f(lw.input_norm), eps))
    # q/k/v GEMM on [W_qkv; A_q; A_k; A_v]: the base columns (packed_ops.py:143)
    # and the bound adapter's intermediate columns (the shrink F.linear(x, A_cat))
    x = _f(L0["x"])
    qkv = _f(L0["qkv"])
    worst["qkv_gemm"] = check("qkv_gemm", qkv[:, : qd + 2 * kd], ol.linear(x, _f(lw.w_qkv)))
    for name in ("q", "k", "v"):
        worst[f"{name}_shrink"] = check(f"{name}_shrink", qkv[:, ycols(name)], ol.linear(x, AB(name)[0]))
    # module outputs with the LoRA up-projection (the module output is
    # rounded before the head norm), head norm + RoPE (projection.py:155-190,
    # 248-260), append (layer_runner.py:399-412)
    mods = {}
    for name, lo, hi in (("q", 0, qd), ("k", qd, qd + kd), ("v", qd + kd, qd + 2 * kd)):
        mods[name] = ol.round_bf16(qkv[:, lo:hi] + ol.up_projection(qkv[:, ycols(name)], AB(name)[1], s))
    pos = np.array([rq.length - 1 for rq in reqs])
    q_want, k_want, v_want = of.qk_norm_rope_append(np.concatenate([mods["q"], mods["k"], mods["v"]], 1), hq, hkv, d,
                                                    _f(lw.q_norm), _f(lw.k_norm), pos, eps, cfg.rope_theta)

    def carried_norm_rope(m, heads, wnorm):
        # |d out / d m| |m|: the head norm scales element i by w_i / rms(head),
        # RoPE output i mixes elements i and i +- D/2 by |cos|, |sin|
        mh = np.abs(m).reshape(B, heads, d)
        rms = np.sqrt((m.reshape(B, heads, d) ** 2).mean(-1, keepdims=True) + eps)
        n = mh * np.abs(wnorm) / rms
        ang = pos.astype(np.float32)[:, None] * of.inv_freq_f32(d, cfg.rope_theta)[None, :]
        c, sn = np.abs(np.cos(ang.astype(np.float64)))[:, None, :], np.abs(np.sin(ang.astype(np.float64)))[:, None, :]
        lo_, hi_ = n[..., : d // 2], n[..., d // 2:]
        return np.concatenate([lo_ * c + hi_ * sn, hi_ * c + lo_ * sn], -1)

    k_carry = carried_norm_rope(mods["k"], hkv, _f(lw.k_norm))
    layer0 = pool.cache[0]
    for b, rq in enumerate(reqs):
        p, o = rq.slot(rq.length - 1, ps)
        worst["k_append"] = max(worst.get("k_append", 0),
                                check(f"k_append row {b}", _f(layer0[p, 0, o]), k_want[b], k_carry[b]))
        worst["v_append"] = max(worst.get("v_append", 0),
                                check(f"v_append row {b}", _f(layer0[p, 1, o]), v_want[b],
                                      np.abs(mods["v"][b]).reshape(hkv, d)))
    # paged decode attention over the row's pages as stored, the new token included
    indptr, indices, last = pool.tables(reqs)
    used = sorted(set(indices.tolist()))
    remap = {pg: i for i, pg in enumerate(used)}
    cache_h = _f(layer0[torch.tensor(used, device=layer0.device)])
    o_want, _ = opd.paged_decode(ol.round_bf16(q_want), cache_h, indptr, [remap[int(pg)] for pg in indices], last)
    attn = _f(L0["attn"]).reshape(B, hq, d)
    # q is formed and rounded inside the kernel: one more rounding of the output's scale
    worst["attention"] = check("attention", attn, o_want, np.abs(o_want))
    # o_proj: base rows and the LoRA A rows' intermediate (side planes or columns)
    attn2 = attn.reshape(B, qd)
    o_out = L0["o"]
    o_yc = 0.0
    if isinstance(o_out, dict):
        # y from partial sums: the kernel rounds their fp32 sum, one rounding
        # of y carried through B; the module output, rounded from a value
        # that differs by that much, may then round to the neighbouring
        # value: a second rounding of it (|o_main| stands for |o_mod|)
        o_main, o_y = _f(o_out["main"]), o_out["y"]
        o_yc = s * (np.abs(o_y) @ np.abs(AB("o")[1]).T) + np.abs(o_main)
    elif isinstance(o_out, tuple):
        o_main, o_y = _f(o_out[0]), _f(o_out[1])[:, slot * r: (slot + 1) * r]
    else:
        o_main, o_y = _f(o_out)[:, : cfg.hidden], _f(o_out)[:, ycols("o")]
    worst["o_gemm"] = check("o_gemm", o_main, ol.linear(attn2, _f(lw.w_o)))
    worst["o_shrink"] = check("o_shrink", o_y, ol.linear(attn2, AB("o")[0]))
    # residual add of o + its delta, post-attention RMSNorm (norm.py:27-57)
    o_mod = ol.round_bf16(o_main + ol.up_projection(o_y, AB("o")[1], s))
    worst["o_residual"] = check("o_residual", _f(L0["hidden_mid"]), hid + o_mod, np.abs(o_mod) + o_yc)
    worst["post_norm"] = check("post_norm", _f(L0["x2"]), of.rmsnorm(_f(L0["hidden_mid"]), _f(lw.post_norm), eps))
    # gate/up GEMM, SiLU(gate) * up with both deltas (packed_ops.py:168-239)
    x2 = _f(L0["x2"])
    gu = _f(L0["gate_up"])
    worst["gate_up_gemm"] = check("gate_up_gemm", gu[:, : 2 * I], ol.linear(x2, _f(lw.w_gate_up)))
    for name in ("gate", "up"):
        worst[f"{name}_shrink"] = check(f"{name}_shrink", gu[:, ycols(name)], ol.linear(x2, AB(name)[0]))
    gate = ol.round_bf16(gu[:, :I] + ol.up_projection(gu[:, ycols("gate")], AB("gate")[1], s))
    up = ol.round_bf16(gu[:, I:2 * I] + ol.up_projection(gu[:, ycols("up")], AB("up")[1], s))
    sig = 1.0 / (1.0 + np.exp(-gate))
    act_carry = np.abs(sig * (1.0 + gate * (1.0 - sig)) * gate * up) + np.abs(gate * sig * up)
    worst["silu_mul"] = check("silu_mul", _f(L0["act"]), of.silu_mul(np.concatenate([gate, up], 1)), act_carry)
    # down_proj, whose delta lands in layer 1's input add + RMSNorm
    act = _f(L0["act"])
    d_out = L0["down"]
    d_yc = 0.0
    if isinstance(d_out, dict):
        d_main, d_y = _f(d_out["main"]), d_out["y"]
        d_yc = s * (np.abs(d_y) @ np.abs(AB("down")[1]).T) + np.abs(d_main)
    elif isinstance(d_out, tuple):
        d_main, d_y = _f(d_out[0]), _f(d_out[1])[:, slot * r: (slot + 1) * r]
    else:
        d_main, d_y = _f(d_out)[:, : cfg.hidden], _f(d_out)[:, ycols("down")]
    worst["down_gemm"] = check("down_gemm", d_main, ol.linear(act, _f(lw.w_down)))
    worst["down_shrink"] = check("down_shrink", d_y, ol.linear(act, AB("down")[0]))
    d_mod = ol.round_bf16(d_main + ol.up_projection(d_y, AB("down")[1], s))
    if "hidden" in L1:  # the add in layer 1's input add+RMSNorm
        h_before, h_after = _f(L1["hidden_in"]), _f(L1["hidden"])
    else:  # the add in down_proj's GEMM: layer 1 starts from the complete stream
        h_before, h_after = _f(L0["hidden_mid"]), _f(L1["hidden_in"])
    worst["down_residual"] = check("down_residual", h_after, h_before + d_mod, np.abs(d_mod) + d_yc)
    worst["next_input_norm"] = check("next_input_norm", _f(L1["x"]),
                                     of.rmsnorm(h_after, _f(w.layers[1].input_norm), eps))
    worst.update(final_stages(w, rec.final, AB, slot))
    print("[stage check] err/bound: " + ", ".join(f"{k} {v:.2f}" for k, v in worst.items()), flush=True)
    return worst


def final_stages(w, F, AB, slot):
    """The step's end against the oracle, on the kernels' stored inputs: the
    final add of the last layer's down_proj output with its LoRA
    up-projection + RMSNorm (norm.py:27-57), the lm_head logits
    (cuda_graph.py:245-263, generation.py:544-561) and the greedy token
    (sampling.py:8-15: torch.argmax, first index among ties)."""
    cfg, s, eps, r = w.cfg, w.lora_scale, w.cfg.rms_eps, w.cfg.lora_rank
    last = cfg.num_layers - 1
    worst = {}
    d_out = F["final_down"]
    d_yc = 0.0
    if isinstance(d_out, dict):
        d_main, d_y = _f(d_out["main"]), d_out["y"]
        d_yc = s * (np.abs(d_y) @ np.abs(AB("down", last)[1]).T) + np.abs(d_main)
    elif isinstance(d_out, tuple):
        d_main, d_y = _f(d_out[0]), _f(d_out[1])[:, slot * r: (slot + 1) * r]
    else:
        lw = w.layers[last]
        c = lw.y_offset["down"] + slot * r
        d_main, d_y = _f(d_out)[:, : cfg.hidden], _f(d_out)[:, c: c + r]
    d_mod = ol.round_bf16(d_main + ol.up_projection(d_y, AB("down", last)[1], s))
    worst["final_residual"] = check("final_residual", _f(F["final_hidden"]), _f(F["final_hidden_in"]) + d_mod,
                                    np.abs(d_mod) + d_yc)
    worst["final_norm"] = check("final_norm", _f(F["final_x"]),
                                of.rmsnorm(_f(F["final_hidden"]), _f(w.final_norm), eps))
    # lm_head over the whole vocabulary in float64, 16384 rows at a time
    # (the weight unshuffled from the decode GEMM's copy, a bit-exact
    # inverse checked on its own)
    x = _f(F["final_x"])
    head = w.lm_head
    want = np.empty((x.shape[0], head.shape[0]))
    for lo in range(0, head.shape[0], 16384):
        want[:, lo: lo + 16384] = ol.linear(x, _f(head[lo: lo + 16384]))
    del head
    logits = _f(F["logits"])
    worst["logits"] = check("logits", logits, want)
    # the greedy pick is the first maximum of the kernel's own logits
    picked = F["next_tokens"].cpu().numpy().reshape(-1)
    assert np.array_equal(picked, np.argmax(logits, axis=1)), f"greedy tokens {picked} != argmax of the logits"
    # and the oracle's pick wherever its top-2 margin exceeds twice the bar
    top2 = np.sort(want, axis=1)[:, -2:]
    bar = 2e-3 + ULP * np.abs(top2[:, 1])
    clear = top2[:, 1] - top2[:, 0] > 2 * bar
    assert np.array_equal(picked[clear], np.argmax(want, axis=1)[clear]), "greedy tokens differ from the oracle's"
    print(f"[stage check] greedy tokens {picked.tolist()}: the logits' first maximum; the oracle's pick on "
          f"{int(clear.sum())} of {len(picked)} rows (the others' top-2 margin is within twice the bar)", flush=True)
    return worst

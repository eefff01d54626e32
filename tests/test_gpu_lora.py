"""No-merge LoRA delta on the GPU vs the float64 oracle.

The kernels round the rank-r intermediate x.A^T to the input dtype, as the
reference's chained F.linear calls return it (packed_ops.py:324), so the
oracle is evaluated with the same rounding (intermediate="bf16"/"f16").
Bars: fp32 outputs 2e-3 max-abs; 16-bit outputs add one rounding of the
result to the output type (2^-8 relative for bf16, 2^-11 for fp16).
"""

import numpy as np
import pytest
import torch

from oracle import lora as ol
from pagelora_amd.lora import lora_delta_

pytestmark = pytest.mark.gpu


def _rand(shape, std, gen, dtype=torch.bfloat16):
    return (torch.randn(shape, generator=gen) * std).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("out_dtype", ["f32", "same"])
def test_qwen3_modules_64_tokens_4_adapters(gpu_device, dtype, out_dtype):
    # hidden 4096, intermediate 12288, r=16, alpha 32 (s=2), 64 tokens over 4 adapters.
    gen = torch.Generator().manual_seed(1237)
    T, H, I, r, n = 64, 4096, 12288, 16, 4
    ids = torch.randint(0, n, (T,), generator=gen, dtype=torch.int32)
    groups = {
        "qkv": (H, [4096, 1024, 1024]),
        "o": (H, [4096]),
        "gate_up": (H, [I, I]),
        "down": (I, [H]),
    }
    for name, (fin, outs) in groups.items():
        x = _rand((T, fin), 1.0, gen, dtype)
        mods, host = [], []
        for fout in outs:
            A = _rand((n, r, fin), fin ** -0.5, gen, dtype)
            B = _rand((n, fout, r), 0.01, gen, dtype)
            out = torch.zeros((T, fout), dtype=torch.float32 if out_dtype == "f32" else dtype, device=gpu_device)
            mods.append((A.to(gpu_device), B.to(gpu_device), out, 2.0))
            host.append((A, B))
        lora_delta_(x.to(gpu_device), mods, ids.to(gpu_device))
        torch.cuda.synchronize()
        for (A, B), (_, _, out, _) in zip(host, mods):
            inter = "bf16" if dtype == torch.bfloat16 else "f16"
            want = ol.multi_adapter_delta(x.float().numpy(), ids.tolist(), A.float().numpy(), B.float().numpy(), 2.0,
                                          intermediate=inter)
            got = out.float().cpu().numpy()
            rtol = 0.0 if out_dtype == "f32" else (2.0**-8 if dtype == torch.bfloat16 else 2.0**-11)
            err = np.abs(got - want)
            assert (err <= 2e-3 + rtol * np.abs(want)).all(), f"{name}: max err {err.max():.3e}"


def test_accumulates_into_base_and_matches_merged_weights(gpu_device):
    # base + B(Ax) vs x (W + s B A)^T, both from the same bf16 inputs (a16).
    gen = torch.Generator().manual_seed(3)
    T, fin, fout, r = 16, 1024, 768, 16
    x = _rand((T, fin), 1.0, gen)
    W = _rand((fout, fin), 0.02, gen)
    A = _rand((r, fin), fin ** -0.5, gen)
    B = _rand((fout, r), 0.01, gen)
    xd = x.to(gpu_device)
    base = (xd.float() @ W.to(gpu_device).float().T)  # fp32 base output
    lora_delta_(xd, [(A.to(gpu_device), B.to(gpu_device), base, 2.0)], torch.zeros(T, dtype=torch.int32, device=gpu_device))
    torch.cuda.synchronize()
    # The merged comparator has no intermediate rounding; the difference is
    # the bf16 rounding of x.A^T times |B|*s (~1e-4 here), inside the bar.
    want = ol.merged_linear(x.float().numpy(), W.float().numpy(), None, A.float().numpy(), B.float().numpy(), 2.0)
    assert np.abs(base.cpu().numpy() - want).max() <= 2e-3


def test_qwen3_modules_match_merged_weights(gpu_device):
    """base + B(Ax) on the seven Qwen3-8B modules (64 tokens over 4 adapters,
    r=16, s=2) vs the merged comparator x (W + s B_a A_a)^T of each token's
    adapter (effective_weights.py:53-129), from the same bf16 inputs.  The
    merged form has no intermediate rounding: the difference is the bf16
    rounding of x.A^T times |B| s, inside the 2e-3 bar."""
    gen = torch.Generator().manual_seed(1238)
    T, H, I, r, n = 64, 4096, 12288, 16, 4
    ids = torch.randint(0, n, (T,), generator=gen, dtype=torch.int32)
    ids_d = ids.to(gpu_device)
    for fin, outs in ((H, [4096, 1024, 1024]), (H, [4096]), (H, [I, I]), (I, [H])):
        x = _rand((T, fin), 1.0, gen)
        xd = x.to(gpu_device)
        mods, host = [], []
        for fout in outs:
            W = _rand((fout, fin), 0.02, gen)
            A = _rand((n, r, fin), fin ** -0.5, gen)
            B = _rand((n, fout, r), 0.01, gen)
            base = xd.float() @ W.to(gpu_device).float().T  # fp32 base output
            mods.append((A.to(gpu_device), B.to(gpu_device), base, 2.0))
            host.append((W, A, B))
        lora_delta_(xd, mods, ids_d)
        torch.cuda.synchronize()
        for (W, A, B), (_, _, out, _) in zip(host, mods):
            got = out.cpu().numpy()
            xs = x.float().numpy()
            for a in range(n):
                rows = (ids == a).numpy()
                if not rows.any():
                    continue
                want = ol.merged_linear(xs[rows], W.float().numpy(), None, A[a].float().numpy(),
                                        B[a].float().numpy(), 2.0)
                err = np.abs(got[rows] - want).max()
                assert err <= 2e-3, f"in {fin} out {W.shape[0]} adapter {a}: max err {err:.3e}"


def test_negative_ids_untouched_and_rank_not_multiple_of_8(gpu_device):
    gen = torch.Generator().manual_seed(4)
    T, fin = 20, 64
    ids = torch.tensor([-1, 0, 1, 2, -5] * 4, dtype=torch.int32)
    x = _rand((T, fin), 1.0, gen)
    mods, host = [], []
    for fout, r in ((40, 2), (24, 6), (8, 3)):   # ranks 2, 6, 3 (the reference's unit tests use rank 2)
        A = _rand((3, r, fin), 0.2, gen)
        B = _rand((3, fout, r), 0.2, gen)
        base = torch.randn((T, fout), generator=gen)
        mods.append((A.to(gpu_device), B.to(gpu_device), base.clone().to(gpu_device), 1.5))
        host.append((A, B, base))
    lora_delta_(x.to(gpu_device), mods, ids.to(gpu_device))
    torch.cuda.synchronize()
    for (A, B, base), (_, _, out, _) in zip(host, mods):
        want = base.numpy() + ol.multi_adapter_delta(x.float().numpy(), ids.tolist(), A.float().numpy(),
                                                     B.float().numpy(), 1.5, intermediate="bf16")
        got = out.cpu().numpy()
        assert np.abs(got - want).max() <= 2e-3
        neg = (ids < 0).numpy()
        assert np.array_equal(got[neg], base.numpy()[neg])


@pytest.mark.parametrize("fin", [40, 264, 1000])
@pytest.mark.parametrize("T", [5, 64])
def test_in_features_not_a_multiple_of_32(gpu_device, fin, T):
    # the shrink's k loop runs the same 32-wide steps in every lane and
    # zero-fills the groups past in_features (fin % 32 in {8, 8, 8})
    gen = torch.Generator().manual_seed(fin + T)
    n, r = 3, 16
    ids = torch.randint(-1, n, (T,), generator=gen, dtype=torch.int32)
    x = _rand((T, fin), 1.0, gen)
    mods, host = [], []
    for fout in (96, 40):
        A = _rand((n, r, fin), fin ** -0.5, gen)
        B = _rand((n, fout, r), 0.05, gen)
        out = torch.zeros((T, fout), dtype=torch.float32, device=gpu_device)
        mods.append((A.to(gpu_device), B.to(gpu_device), out, 2.0))
        host.append((A, B))
    lora_delta_(x.to(gpu_device), mods, ids.to(gpu_device))
    torch.cuda.synchronize()
    for (A, B), (_, _, out, _) in zip(host, mods):
        want = ol.multi_adapter_delta(x.float().numpy(), ids.tolist(), A.float().numpy(), B.float().numpy(), 2.0,
                                      intermediate="bf16")
        err = np.abs(out.cpu().numpy() - want)
        assert err.max() <= 2e-3, f"fin {fin}: max err {err.max():.3e}"


def test_packed_group_equals_separate_calls(gpu_device):
    gen = torch.Generator().manual_seed(5)
    T, fin = 7, 256
    x = _rand((T, fin), 1.0, gen).to(gpu_device)
    ids = torch.zeros(T, dtype=torch.int32, device=gpu_device)
    specs = [(128, 16), (32, 16), (32, 16)]
    As = [_rand((1, r, fin), 0.1, gen).to(gpu_device) for _, r in specs]
    Bs = [_rand((1, o, r), 0.1, gen).to(gpu_device) for o, r in specs]
    packed_out = torch.zeros((T, sum(o for o, _ in specs)), dtype=torch.float32, device=gpu_device)
    views, off = [], 0
    for o, _ in specs:
        views.append(packed_out[:, off:off + o])
        off += o
    lora_delta_(x, [(A, B, v, 2.0) for A, B, v in zip(As, Bs, views)], ids)
    sep = [torch.zeros((T, o), dtype=torch.float32, device=gpu_device) for o, _ in specs]
    for A, B, s in zip(As, Bs, sep):
        lora_delta_(x, [(A, B, s, 2.0)], ids)
    torch.cuda.synchronize()
    assert torch.equal(packed_out, torch.cat(sep, dim=1))


def test_repeated_calls_reuse_workspace(gpu_device):
    # The per-adapter tickets must return to zero after every call.
    gen = torch.Generator().manual_seed(6)
    T, fin, fout, r = 33, 512, 64, 16
    x = _rand((T, fin), 1.0, gen).to(gpu_device)
    A = _rand((2, r, fin), 0.05, gen).to(gpu_device)
    B = _rand((2, fout, r), 0.05, gen).to(gpu_device)
    ids = (torch.arange(T, dtype=torch.int32) % 2).to(gpu_device)
    outs = []
    for _ in range(5):
        o = torch.zeros((T, fout), dtype=torch.float32, device=gpu_device)
        lora_delta_(x, [(A, B, o, 1.0)], ids)
        outs.append(o)
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def _group(gen, T, fin, outs_ranks, n, dtype=torch.bfloat16, out_dtype=torch.float32, device=None, base=False):
    x = _rand((T, fin), 1.0, gen, dtype)
    mods, host = [], []
    for fout, r in outs_ranks:
        A = _rand((n, r, fin), fin ** -0.5, gen, dtype)
        B = _rand((n, fout, r), 0.05, gen, dtype)
        b0 = torch.randn((T, fout), generator=gen) if base else torch.zeros((T, fout))
        mods.append((A.to(device), B.to(device), b0.to(out_dtype).to(device), 2.0))
        host.append((A, B, b0.to(out_dtype).float()))
    return x, mods, host


def _check_group(x, ids, host, mods, dtype=torch.bfloat16, rtol=0.0):
    inter = "bf16" if dtype == torch.bfloat16 else "f16"
    for (A, B, b0), (_, _, out, _) in zip(host, mods):
        want = b0.numpy() + ol.multi_adapter_delta(x.float().numpy(), ids.tolist(), A.float().numpy(),
                                                   B.float().numpy(), 2.0, intermediate=inter)
        got = out.float().cpu().numpy()
        err = np.abs(got - want)
        assert (err <= 2e-3 + rtol * np.abs(want)).all(), f"max err {err.max():.3e}"


@pytest.mark.parametrize("T,n", [(65, 4), (200, 3), (16, 70), (1, 65)])
def test_general_path_beyond_decode_sizes(gpu_device, T, n):
    # more than 64 tokens or 64 adapters: the general shrink + expand pair
    gen = torch.Generator().manual_seed(T * 100 + n)
    ids = torch.randint(-1, n + 1, (T,), generator=gen, dtype=torch.int32)  # includes -1 and n (both untouched)
    x, mods, host = _group(gen, T, 512, [(96, 16), (40, 8)], n, device=gpu_device, base=True)
    lora_delta_(x.to(gpu_device), mods, ids.to(gpu_device))
    torch.cuda.synchronize()
    _check_group(x, ids, host, mods)


@pytest.mark.parametrize("T", [1, 4, 16, 17, 63, 64])
@pytest.mark.parametrize("n", [1, 4, 64])
def test_decode_path_tokens_and_adapters(gpu_device, T, n):
    # the two-launch decode path at its edges: 1..64 tokens, 1..64 adapters,
    # ids outside [0, n) untouched, ranks summing to the 128 maximum
    gen = torch.Generator().manual_seed(T * 1000 + n)
    ids = torch.randint(-1, n + 1, (T,), generator=gen, dtype=torch.int32)
    x, mods, host = _group(gen, T, 1000, [(64, 32), (48, 32), (40, 32), (16, 32)], n, device=gpu_device,
                           base=True)
    lora_delta_(x.to(gpu_device), mods, ids.to(gpu_device))
    torch.cuda.synchronize()
    _check_group(x, ids, host, mods)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [4, 64, 100])
def test_groups_in_one_call_equal_separate_calls(gpu_device, dtype, T):
    """A decoder layer's four groups (Qwen3-8B modules, r=16, 4 adapters) in
    one pl_lora_delta_groups call == four pl_lora_delta calls, bit for bit
    (decode sizes: the same two launches; 100 tokens: one after another),
    and the oracle on every module."""
    from pagelora_amd.lora import lora_delta_groups_

    gen = torch.Generator().manual_seed(17 + T)
    H, I, n = 4096, 12288, 4
    ids = torch.randint(0, n, (T,), generator=gen, dtype=torch.int32)
    spec = [(H, [(4096, 16), (1024, 16), (1024, 16)]), (H, [(4096, 16)]), (H, [(I, 16), (I, 16)]),
            (I, [(H, 16)])]
    groups = [_group(gen, T, fin, outs, n, dtype=dtype, out_dtype=dtype, device=gpu_device, base=True)
              for fin, outs in spec]
    sep = [[(A, B, out.clone(), s) for A, B, out, s in mods] for _, mods, _ in groups]
    lora_delta_groups_([(x.to(gpu_device), mods) for x, mods, _ in groups], ids.to(gpu_device))
    for (x, _, _), mods in zip(groups, sep):
        lora_delta_(x.to(gpu_device), mods, ids.to(gpu_device))
    torch.cuda.synchronize()
    rtol = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    for (x, mods, host), smods in zip(groups, sep):
        for (_, _, out, _), (_, _, sout, _) in zip(mods, smods):
            assert torch.equal(out, sout)
        _check_group(x, ids, host, mods, dtype, rtol)


def test_delta_workspace_state_across_calls(gpu_device):
    # the decode path keeps its double-buffered accumulators in the delta
    # workspace between calls; calls with other layouts, ranks and token
    # counts, and general-path calls, interleaved on the same workspace, all
    # match the oracle
    gen = torch.Generator().manual_seed(9)
    for T, fin, outs in ((64, 4096, [(512, 16), (256, 16)]), (100, 512, [(64, 16)]), (3, 12288, [(128, 8)]),
                         (20, 64, [(40, 2), (24, 6)]), (40, 264, [(64, 48)]), (64, 4096, [(512, 16), (256, 16)]),
                         (7, 1024, [(96, 32), (32, 32), (16, 64)])):
        ids = torch.randint(0, 4, (T,), generator=gen, dtype=torch.int32)
        x, mods, host = _group(gen, T, fin, outs, 4, device=gpu_device)
        lora_delta_(x.to(gpu_device), mods, ids.to(gpu_device))
        torch.cuda.synchronize()
        _check_group(x, ids, host, mods)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [16, 80])  # the decode-size path, the general path
def test_nonfinite_values_propagate_per_module(gpu_device, dtype, T):
    """A NaN in x, infinities in A (both signs, in different k-slices) and,
    in fp16, an intermediate that overflows when rounded: the outputs carry
    NaN / +-inf exactly where the per-module F.linear(F.linear(x, A_m), B_m)
    chain of multilora/linear.py:226-231 puts them (float64 oracle with IEEE
    propagation), finite outputs stay within the bar, and the next call on
    the workspace is bit-identical to one made before the non-finite call."""
    gen = torch.Generator().manual_seed(900 + T)
    n, fin = 2, 512
    specs = [(64, 16), (32, 16), (48, 16)]  # three modules of one group (q/k/v-like)
    ids = torch.tensor([(t % 3) - (1 if t % 7 == 6 else 0) for t in range(T)], dtype=torch.int32)
    ids = torch.where(ids > 1, torch.zeros_like(ids), ids)  # adapters 0/1, some -1
    ids[3], ids[5], ids[6] = 1, 1, 0
    x = _rand((T, fin), 1.0, gen, dtype)
    As = [_rand((n, r, fin), fin ** -0.5, gen, dtype) for _, r in specs]
    Bs = [_rand((n, o, r), 0.05, gen, dtype) for o, r in specs]
    x_nf, As_nf = x.clone(), [a.clone() for a in As]
    x_nf[3, 10] = float("nan")                 # every intermediate of token 3
    As_nf[0][1, 5, 7] = float("inf")           # module 0, adapter 1, rank 5
    x_nf[5, 7] = 0.0                           # ... times 0: NaN for token 5
    As_nf[2][0, 3, 20] = float("inf")          # module 2, adapter 0, rank 3: +inf and -inf
    As_nf[2][0, 3, 300] = -float("inf")        # in different 256-element k-slices
    x_nf[6, :] = 4.0                           # module 1, adapter 0, rank 0: 512 * 4 * 64 = 131072
    As_nf[1][0, 0, :] = 64.0                   # (overflows when rounded to fp16, finite in bf16)
    inter = "bf16" if dtype == torch.bfloat16 else "f16"

    def run(xh, Ah):
        outs = [torch.zeros((T, o), dtype=torch.float32, device=gpu_device) for o, _ in specs]
        lora_delta_(xh.to(gpu_device), [(A.to(gpu_device), B.to(gpu_device), out, 2.0)
                                        for A, B, out in zip(Ah, Bs, outs)], ids.to(gpu_device))
        torch.cuda.synchronize()
        return [o.cpu() for o in outs]

    before = run(x, As)
    got = run(x_nf, As_nf)
    after = run(x, As)
    for b, a in zip(before, after):
        assert torch.equal(b, a), "a call after the non-finite one differs"
    with np.errstate(invalid="ignore", over="ignore"):
        for m, (A, B) in enumerate(zip(As_nf, Bs)):
            want = ol.multi_adapter_delta(x_nf.float().numpy(), ids.tolist(), A.float().numpy(),
                                          B.float().numpy(), 2.0, intermediate=inter)
            g = got[m].numpy().astype(np.float64)
            for kind, f in (("NaN", np.isnan), ("+inf", np.isposinf), ("-inf", np.isneginf)):
                assert np.array_equal(f(g), f(want)), f"module {m}: {kind} positions differ"
            # fp32 accumulation: 2e-3 plus 2^-16 of the terms' magnitude
            # (token 6's module-1 terms reach ~2e4 in bf16)
            mag = ol.multi_adapter_delta(np.abs(np.nan_to_num(x_nf.float().numpy())), ids.tolist(),
                                         np.abs(np.nan_to_num(A.float().numpy(), posinf=0, neginf=0)),
                                         np.abs(B.float().numpy()), 2.0)
            fin_mask = np.isfinite(want)
            err = np.abs(g[fin_mask] - want[fin_mask])
            assert (err <= 2e-3 + 2.0**-16 * mag[fin_mask]).all(), f"module {m}: max err {err.max():.3e}"
    # the planted values reach the outputs they should
    assert np.isnan(got[0][3]).all() and np.isnan(got[1][3]).all() and np.isnan(got[2][3]).all()
    assert not np.isfinite(got[0][5]).all() and np.isfinite(got[1][5]).all()
    assert (~np.isfinite(got[2][ids.numpy() == 0])).any()
    if dtype == torch.float16:
        assert not np.isfinite(got[1][6]).all()
    else:
        assert np.isfinite(got[1][6]).all()

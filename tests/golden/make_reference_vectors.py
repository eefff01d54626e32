"""Write reference_vectors.json: the reference's own test vectors for this path.

Every case restates, as data, an input/expected-output pair that a test or
document of the reference fixes (the file:line is in each case's "source").
Nothing here imports or runs the reference: page-table cases are copied
from its assertions, LoRA cases are its fixtures with the expected outputs
written in closed form (for constant A = a, B = b with rank r and scale s,
the delta of every output is s * r * a * b * sum(x)).

Run from the repo root:  python tests/golden/make_reference_vectors.py
"""

from __future__ import annotations

import json
from pathlib import Path

OUT = Path(__file__).with_name("reference_vectors.json")

PAGE_TABLE_CASES = [
    {
        "source": "test/test_paged_kvcache_manager.py:429-441",
        "page_size": 2,
        "rows": [[[11, 0, 2], [12, 0, 1]]],
        "indptr": [0, 2], "indices": [11, 12], "last_page_len": [1],
    },
    {
        "source": "test/test_paged_kvcache_manager.py:444-461",
        "page_size": 2,
        "rows": [[[11, 0, 2], [12, 0, 1]], [[21, 0, 2]]],
        "indptr": [0, 2, 3], "indices": [11, 12, 21], "last_page_len": [1, 2],
    },
    {
        "source": "test/test_paged_kvcache_manager.py:483-500 (second update)",
        "page_size": 2,
        "rows": [[[11, 0, 2], [12, 0, 1]]],
        "indptr": [0, 2], "indices": [11, 12], "last_page_len": [1],
    },
    {
        "source": "test/test_paged_kvcache_manager.py:503-520 (first table)",
        "page_size": 4,
        "rows": [[[2, 0, 3]], [[4, 0, 4]]],
        "indptr": [0, 1, 2], "indices": [2, 4], "last_page_len": [3, 4],
    },
    {
        "source": "test/test_paged_kvcache_manager.py:523-543",
        "page_size": 4,
        "rows": [[[2, 0, 4]], [[4, 0, 4], [5, 0, 1]]],
        "indptr": [0, 1, 3], "indices": [2, 4, 5], "last_page_len": [4, 1],
    },
    {
        "source": "docs/技术详解与代码导读.md:251 (pages [7,2,9], page 32, length 70)",
        "page_size": 32,
        "rows": [[[7, 0, 32], [2, 0, 32], [9, 0, 6]]],
        "indptr": [0, 3], "indices": [7, 2, 9], "last_page_len": [6],
    },
]

PAGE_TABLE_REJECTS = [
    {"source": "test/test_paged_kvcache_manager.py:464-470", "page_size": 2, "rows": [[[1, 1, 1]]]},
    {"source": "test/test_paged_kvcache_manager.py:472-480", "page_size": 2, "rows": [[[1, 0, 1], [2, 0, 1]]]},
]


def _weight(out_f, in_f):
    """_linear() weights of test_flashinfer_packed_ops.py:19-28: arange(out*in)/100."""
    return [[(o * in_f + k) / 100.0 for k in range(in_f)] for o in range(out_f)]


def _bias(out_f):
    return [o / 10.0 for o in range(out_f)]


def _linear(x, w, b):
    return [[sum(xi * wi for xi, wi in zip(row, wrow)) + (b[o] if b else 0.0) for o, wrow in enumerate(w)] for row in x]


X = [[0.5, -1.0, 2.0, 0.25, -0.75, 1.5], [1.0, 1.0, 1.0, 1.0, 1.0, 1.0], [-2.0, 0.0, 0.125, 3.0, -1.5, 0.5]]


def _lora_case(source, modules, bias):
    """modules: list of (out_features, a_const, b_const); rank 2, alpha 4 -> scale 2."""
    rank, scale, in_f = 2, 2.0, 6
    mods = []
    for out_f, a_c, b_c in modules:
        w = _weight(out_f, in_f)
        b = _bias(out_f) if bias else None
        base = _linear(X, w, b)
        delta = [[scale * rank * a_c * b_c * sum(row)] * out_f for row in X]
        y = [[bv + dv for bv, dv in zip(br, dr)] for br, dr in zip(base, delta)]
        mods.append({
            "out_features": out_f, "rank": rank, "scale": scale, "a_const": a_c, "b_const": b_c,
            "weight": w, "bias": b, "expected_delta": delta, "expected_output": y,
        })
    return {"source": source, "in_features": in_f, "x": X, "modules": mods}


LORA_CASES = [
    _lora_case("test/test_flashinfer_packed_ops.py:56-91 (packed q/k/v, A=0.1, B=0.2; packed A (6,6), B (16,6))",
               [(8, 0.1, 0.2), (4, 0.1, 0.2), (4, 0.1, 0.2)], bias=False),
    _lora_case("test/test_flashinfer_packed_ops.py:130-165 (q/k/v, A=0.03*i, B=0.04*i)",
               [(8, 0.03, 0.04), (4, 0.06, 0.08), (4, 0.09, 0.12)], bias=False),
    _lora_case("test/test_flashinfer_packed_ops.py:168-200 (one module with bias, A=0.1, B=0.2)",
               [(4, 0.1, 0.2)], bias=True),
    _lora_case("test/test_flashinfer_packed_ops.py:324-357 (gate/up with bias, A=0.03*i, B=0.04*i; packed A (4,6), B (10,4))",
               [(5, 0.03, 0.04), (5, 0.06, 0.08)], bias=True),
]

# Decode restatement of test_flashinfer_backend.py:157-177: with head_dim 1,
# q = -1000, every key 100 and values [1, 9], the scores of the two tokens
# are equal; the row that sees only the first token returns 1, the row that
# sees both returns their mean 5.  Large-magnitude scores, no finite mask.
DECODE_CASES = [
    {
        "source": "test/test_flashinfer_backend.py:157-177 (restated as two decode rows)",
        "q": -1000.0, "k": 100.0, "v": [1.0, 9.0],
        "rows_tokens": [1, 2], "expected": [1.0, 5.0],
    }
]

# The same test in its own form: backend.plan_prefill(qo_indptr=[0, 2],
# paged_kv_indptr=[0, 1], paged_kv_indices=[0], paged_kv_last_page_len=[2])
# on a page of 2 tokens, causal (plan_prefill's default), then
# run_prefill(q, kv) with q = -1000 for both tokens, k = 100, v = [1, 9]
# -> [1, 5] (query 0 sees token 0 only, query 1 sees both).
PREFILL_CASES = [
    {
        "source": "test/test_flashinfer_backend.py:157-177",
        "page_size": 2, "head_dim": 1, "causal": True,
        "qo_indptr": [0, 2], "kv_indptr": [0, 1], "kv_indices": [0], "kv_last_page_len": [2],
        "q": [-1000.0, -1000.0], "k": [100.0, 100.0], "v": [1.0, 9.0],
        "expected": [1.0, 5.0],
    }
]


def main() -> None:
    data = {
        "page_table": PAGE_TABLE_CASES,
        "page_table_rejects": PAGE_TABLE_REJECTS,
        "lora": LORA_CASES,
        "decode": DECODE_CASES,
        "prefill": PREFILL_CASES,
    }
    OUT.write_text(json.dumps(data, indent=1, ensure_ascii=False) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()

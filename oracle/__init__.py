"""CPU oracle: a restatement of the reference's arithmetic on the decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``pagelora_amd``) imports
this package.  It is used by ``tests/`` as the checker, by
``__graft_entry__.smoke()`` to check one small GPU invocation, and by
``bench.py``'s ``cpu_baseline`` leg as the CPU timing reference.

Modules (each function cites the reference file:line it follows):
  paged_decode  paged decode attention (float64 numpy), KV append, page gather
  page_table    span -> (indptr, indices, last_page_len) packing, pure Python
  lora          no-merge LoRA delta: per-module, packed (A concat, block-diag B),
                multi-adapter, and the merged-weight comparator (float64 numpy)

Pinning (what each function is checked against, in tests/test_oracle_*.py):
  page_table    the reference's own test vectors (tests/golden/reference_vectors.json)
  paged_decode  closed forms (single token -> v; equal keys -> mean of V; GQA ==
                MHA with repeated heads), physical-page permutation invariance,
                torch's CPU scaled_dot_product_attention in float64 on the
                gathered K/V, brute force on tiny inputs
  lora          the reference's LoRA fixtures restated as closed forms
                (tests/golden/reference_vectors.json) and torch.nn.functional.linear
"""

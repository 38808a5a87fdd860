"""CPU oracle for the DSpark attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (qwen3_dspark_amd)
imports, links or calls this package; only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg use it, and only to check results.

  semantics.py  - integer/index semantics (layouts, transaction metadata,
                  materialised gather, commit/rollback, masks, work counters)
                  restated from the reference files cited per function.
  attention.py  - float64 numpy attention (bottom-right causal, noncausal,
                  multi-block draft) restated from the reference oracles.
  attn_ref.c    - the same attention in C (OpenMP), used as the CPU baseline
                  and for checks at sizes numpy is slow at; built by
                  oracle/Makefile into oracle/_build/liboracle.so.
  qkv.py        - the target's verify-layer prologue (q/k/v projection,
                  q/k RMSNorm, RoPE) in float64.
  draft_proj.py - the draft's context projection (fc, context norm, per-layer
                  k_proj / k_norm / RoPE / v_proj) in float64.
  draft_model.py - the draft backbone over cached context (every draft
                  layer: norms, projections, RoPE, multi-block attention,
                  o_proj, MLP; final norm) in float64.

Pinning (see tests/test_oracle_golden.py): every function is checked against
the reference tests' literal vectors (tests/golden/reference_vectors.json),
closed forms (uniform attention, position ramps), invariants, brute force on
tiny inputs and torch's scaled_dot_product_attention on explicit masks;
qkv.py, draft_proj.py and draft_model.py against transformers' own Qwen3
modules (draft_model.py also against torch's SDPA and closed forms).
"""

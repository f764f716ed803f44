"""CPU oracle for the paged-KV path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithms (KyleBoyer/vOOM, pure
Python/MLX) on the CPU with numpy so the HIP path can be checked against them.
It is imported only by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, and only as the checker or the timed CPU
baseline -- never as a code path of the product (``voom_amd``), which raises
when its HIP library is missing instead of falling back here.

Modules and the reference code each restates:
  bf16            IEEE round-to-nearest-even fp32 <-> bf16 on uint16 words
  paged_attention page gather in logical order + SDPA decode with GQA broadcast
                  (runtime/kv_paged.py:164-181, runtime/layer_runner.py:179-180,
                  runtime/pic_attention.py:60-65)
  mla             absorbed / expanded MLA attention (runtime/glm.py:78-210)
  byteplane       byte-plane split/merge (formats/packed.py:49-50, 376-378);
                  a C restatement of the same lives in byteplane.c
  kv_policy       PagedKVCache page close / budget / spill order
                  (runtime/kv_paged.py:143-162, 187-194, 216-240)

Pinning (what each restatement is checked against, see tests/test_oracle_*.py):
  byteplane       exhaustive over all 65,536 16-bit patterns against the
                  closed form lo = e & 0xff, hi = e >> 8; numpy vs C agree.
  paged_attention closed forms (ctx=1 gives the V row, equal keys give the
                  mean of V, two keys give the logistic weight), the GQA head
                  map, page-order invariance, repeated table ids, fp64 brute
                  force.
  mla             the reference's own known-answer test inputs
                  (tests/test_mla_absorbed.py:115-222, numpy default_rng(34))
                  against the expanded (non-absorbed) attention computed in
                  fp64, tolerances 2e-5 / 3e-5 as in the reference.
  kv_policy       hand-computed spill orders for small caches, including the
                  reference's test_kv_spill_compress.py:22-60 geometry.
"""

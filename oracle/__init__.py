"""CPU oracle for tm-opt's paged attention path — TEST INFRASTRUCTURE ONLY.

This package restates the reference's algorithm for the hot path on the CPU
so that the HIP kernels can be checked against it. It is the checker, never
the thing measured or shipped: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it. The product path
(tm-opt_amd/) never imports or calls anything here.

Modules:
  attn_ref  fp32 torch restatement of decode and prefill attention
            (engine/pyengine/kernels/attn_swa.py:57-117,
            attn_prefill.py:80-141, model.py:137-246 / :890-1014).
  kv_ref    numpy restatement of the KV-cache write and block-table gather
            (engine/pyengine/kv.py:89-212, model.py:926-950).
  geometry  the decode-step ring/page geometry (model.py:827-887).

How each function is pinned (tests/test_oracle_*.py): brute-force
pure-Python evaluation on tiny inputs, torch's scaled_dot_product_attention
with an explicit mask, closed forms (q = 0 gives LSE = ln(n_visible) and the
mean of the visible V rows; a single visible key returns its V row), the
SWA == global identity for ctx <= W, and the reference's own structural pins
restated from engine/pyengine/tests/t_b3.py:81-130 and t_graphrun.py:17-76.
Planted-mistake variants of the oracle are run through the same checks to
show that each check fails on a plausible bug.
"""

"""CPU oracle of the verify/draft hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in torch-CPU fp32 ops (float arithmetic) and numpy (nibble /
byte arithmetic), of the reference's eager path for this hot path, each
function citing the reference file:line it follows. It is the checker:
only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and never as the thing measured or shipped. The product
(mtp-engine_amd/) never imports it and fails loudly without its HIP library.

How each function is pinned (checks independent of the formula restated
here, in tests/test_oracle.py):
  rmsnorm_linear / rmsnorm_linear_fp8 — float64 brute force on small shapes;
      scale invariance y(c*x) == y(x); gamma == 1 equals no gamma; norm=False
      equals plain linear; the reference's own tolerance checks
      (test_engine.py:5, mtp_engine.py:1644-1651, 1792-1800) on the same
      seeded inputs.
  fp8 decode — all 256 e4m3fn codes against the OCP e4m3fn formula.
  quantize_fp8_per_channel — closed form amax/448 scale; |W - dq(q)| within
      half an fp8 ulp of each scaled value; zero rows get scale 1.
  quantize_int4 / dequantize_int4 — brute force over all 256 byte values;
      decode(encode(q)) == q - 8 for q >= 0 and q + 8 for q < 0 (the
      reference's pack/unpack mismatch); nibble order (even k = low nibble).
  int4_matmul — equals rmsnorm_linear on the explicitly dequantized weight
      (the reference's bit-exact check, mtp_engine.py:1812-1819).
  fused_verify / fused_multi_verify — brute-force Python dot products and
      argmax loops on tiny vocabularies; planted ties (lowest index wins);
      all-equal logits give 0; exhaustive acceptance enumeration for D <= 4;
      a mismatch followed by a later match keeps the prefix closed.
  chain_accept_textbook — exhaustive enumeration for D <= 4 of which
      drafts match top[b, d] (not top[b, d + 1]), with literal expected
      accept masks, counts and corrected tokens (the replacement token, or
      the bonus top[b, D]); a draft equal to the reference convention's
      token but not the textbook one is rejected.
  draft_tree — the reference's known shapes (32 nodes for depth 4 x 8
      branches; trunk mask rows) and ancestor closure.
  engine_rollback — the known-answer of generate_fused's consumer logic.
  tree_attention / paged_attention / tree_verify_attention — float64 brute
      force; all-ones mask equals plain softmax attention and an all-masked
      row is NaN; paged equals contiguous keys under any page placement;
      the tree-verify step equals one single-query tree_attention call per
      node over context ++ tree keys (how the reference composes it).
"""

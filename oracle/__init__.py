"""CPU oracle for the pair-representation hot path — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's PyTorch fallback (the only working
implementation of this path in the reference):

  pair_ops.layer_norm / linear      src/genie_tk/primitives.py:43-62, torch.nn.LayerNorm
  pair_ops.tri_mul                  src/genie_tk/triangle_mul.py:103-132 (+ :77-101)
  pair_ops.tri_attn                 src/genie_tk/triangle_attention.py:84-143,
                                    src/genie_tk/primitives.py:114-178
  pair_ops.contract                 src/genie_tk/triangle_mul.py:77-101
  pair_ops.attention_core           kernels/bindings.cpp:82-90 semantics
  pair_ops.pair_block               src/genie_tk/pair_transform.py:162-195 (eval mode)
  brute.*                           scalar-loop versions of the above for tiny
                                    inputs, used to pin pair_ops

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use this
package, and only as the checker.  The library (genie-tk_amd/) never imports it.

Pinning (what makes this oracle trustworthy, see tests/test_oracle_*.py):
  * every function of pair_ops against brute.* loops in float64 at tiny sizes;
  * layer_norm against torch.nn.functional.layer_norm; the contraction against
    torch.einsum; attention against torch.nn.functional.scaled_dot_product_attention;
  * identities: incoming(z, m; a<->b) = outgoing(z^T, m^T)^T (a/b projections
    swapped), ending(x, m) = starting(x^T, m^T)^T;
  * closed forms: default init -> exactly 0; padded tri-mul rows ->
    (W_z beta_out + b_z) * gate; fully-masked attention rows -> uniform weights;
  * committed golden fixtures (tests/golden/*.npz) regenerate bit-for-bit.
No function is left "parity unpinned".
"""

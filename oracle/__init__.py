"""CPU oracle for the asrback attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU and in plain PyTorch/NumPy, what the
reference (sjjeong94/asrback) computes on the attention path: the
``F.scaled_dot_product_attention`` calls with the masks and layouts its
modules build, and the modules and greedy decoding loops around them.  Each
function cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it, and only as the reference results are compared with (or,
in ``bench.py``, as the timed CPU baseline).  The product (``asrback_amd``) never imports it and has no CPU
fallback.

Pinning (what checks each function against something other than itself):

* ``brute`` -- float64 closed-form attention written with explicit loops over
  keys; checked on small cases by hand-derivable special cases (one key,
  identical keys, one-hot scores) in ``tests/test_oracle.py``.
* ``attention`` -- the reference's SDPA call patterns; pinned against
  ``brute`` and the committed golden vectors (``tests/golden``), and by
  invariants the mathematics fixes: a decoder step equals the last row of a
  causal prefill; padding/bucket invariance; GQA equals MHA with repeated kv
  heads; RoPE at position 0 is the identity and preserves norms; RoPE scores
  depend only on the position difference.
* ``whisper`` -- the Whisper modules and greedy decoding; the attention inside
  is ``attention``'s; the whole loop is pinned by the committed greedy-token
  fixture and by the invariants (step vs prefill, cache-bucket invariance).
* ``sensevoice`` / ``qwen3`` -- SAN-M attention with its FSMN memory and the
  Qwen3 text attention; pinned by padding invariance (a padded batch equals
  per-sequence runs), FSMN against an explicit loop, RMSNorm against its
  formula, and the GQA/RoPE invariants above.
* ``gemma4`` -- Gemma 4's blocked audio attention (the reference's padding,
  unfold and Transformer-XL relative shift) pinned against a float64 loop
  over queries and keys written from the definition; the text attention's
  masks pinned against explicit loops, a step against the prompt pass's row
  and against plain attention over the window's keys.

The reference's Python cannot be imported here (its ``asrfront`` dependency
is absent); it was read, never run.
"""

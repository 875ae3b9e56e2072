"""CPU oracle for the selective-attention kernel layer.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this package, and only as the
checker (or as the timed CPU baseline).  The product path
(selective-attention_amd/selective_attention) never imports it and has no
CPU fallback.

Contents (each function cites the reference file:line it restates):
  ssd.py   - chunked SSD scan forward + manual backward, restating the
             reference's Triton kernels step by step; an independent
             sequential recurrence (closed form) used to pin the chunked one.
  ssu.py   - single-step selective state update.
  attn.py  - block-sparse varlen causal attention and paged GQA decode
             attention (brute-force dense masked softmax; no reference kernel
             exists for these, the gated-softmax semantics come from
             modules/selective_attention.py); SelectiveMHA's inference
             attention (prefill in the form of the reference's compressed
             branch, decode in mode "pos") and its log-gate.
  lm.py    - the causal LM and the seq2seq LM in inference (LMRef,
             Seq2SeqRef): fp64 compositions of the functions above with
             torch linears / norms / RoPE / SwiGLU, optionally rounding to
             bf16 where the bf16 model stores a tensor.
  ssm_io.py - the SSM block's stages around the scan (modules/ssm.py):
             SiLU + causal depthwise conv prologue, its decode-time context
             (inference/ssm_cache.py), the D-skip / SiLU-gate epilogue, and
             their hand-written backward formulas.

How each function is pinned (tests/test_oracle_*.py):
  ssd forward   - chunked == sequential recurrence (fp64), chunk-size
                  invariance, split-sequence chaining, length masking, A=0
                  closed form.
  ssd backward  - manual restatement == torch.autograd through the chunked
                  restatement == autograd through the sequential recurrence;
                  gradcheck on tiny fp64 shapes.
  ssu           - == SSD scan with L=1 and h_init=h; brute-force loop.
  attention     - == F.scaled_dot_product_attention (textbook softmax
                  attention) when the selection covers every causal block /
                  the page table is the identity; brute-force loops.
  ssm_io        - conv == the reference's F.silu / F.conv1d(padding=K-1) /
                  slice composition and == a brute-force loop; streaming
                  decode steps == the batch conv; context == a brute-force
                  gather; backward formulas == torch.autograd (fp64).
  lm            - prefill of the first tokens + decode steps == the full
                  forward (the reference's own test_forward_step
                  invariant), for the causal LM and the seq2seq decoder,
                  in fp64; a RoPE position slip is shown to fail it.
  selective_mha - prefill (compressed-branch form) == the reference's other
                  branch (full causal matrix, gate on every column, diagonal
                  restored) on the same inputs; all gates 1 == causal SDPA;
                  every key dropped == v; decode over keys 0..t == prefill
                  row t.
The reference ships no golden vectors or known-answer tests for this path
(its one test file is an integration test that is broken as shipped), so
nothing here is pinned against reference-produced numbers.  Rounding-level
behaviour of Triton (tl.cumsum order, atomics order, TF32 on NVIDIA) is
not reproduced and is covered by the stated tolerances instead.
"""

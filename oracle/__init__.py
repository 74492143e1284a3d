"""CPU oracle of the paged KV-cache data path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline);
the product path (tinybatch_amd) never calls it and has no CPU fallback.

Modules:
* reference_path — op-for-op restatement of the reference's CPU path
  (src/tinybatch/kv_cache.py:25-45, src/tinybatch/model.py:127-147), in torch on
  the CPU, in the model dtype. This is what the GPU kernels are compared with
  and what bench.py times as the CPU baseline ("kind": "port").
* brute — independent float64 brute force (explicit flat-index pool
  addressing, explicit loops) and closed forms used to pin reference_path.

Pinning (tests/test_oracle.py): append/gather/copy against the closed-form
flat index; attention against the float64 brute force, the library routine
torch.nn.functional.scaled_dot_product_attention with an explicit mask, and
special cases (context of one token, identical keys, q_len == ctx versus the
is_causal branch, rep = 1, permuted physical blocks); planted mistakes in a
copy of the oracle (wrong GQA head map, mask off by one, missing scale) must
fail those checks. The reference ships no golden vectors for this path.
"""

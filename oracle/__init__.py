"""CPU oracle for the softmax-attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, the algorithm of the reference's own test
oracles (flywheel-tpu v0.4.1, `tests/softmax_attention/util.py`,
`test_paged.py`, `test_regression.py`, `test_page.py`) and the layout rules of
`flywheel_tpu/softmax_attention/kv_layout.py` / `variant.py`.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may
import it, and only as the checker or as the timed CPU baseline.  The shipped
package (`flywheel-tpu_amd/flywheel_tpu`) never imports it: the product path
runs the HIP library or raises.

Pinning (how each function is checked independently of its own formula; the
tests live in `tests/test_oracle.py`):

* `dtypes.bf16_round`, `dtypes.fp8_decode/fp8_encode` -- against torch's CPU
  dtype conversions, exhaustively over all 2^8 codes / random floats.
* `attention_ref` -- against `torch.nn.functional.scaled_dot_product_attention`
  (a library routine) for causal/full GQA cases, a pure-Python brute-force
  loop on tiny inputs, and closed forms: one visible key (out = v,
  lse = score), identical keys (out = mean V), the anchor known-answer test of
  `test_regression.py:1035-1063` (out = 3), window >= context == causal,
  softcap -> inf == no softcap, a -inf sink == no sink.
* `ragged_reference`, `decode_reference`, `kvcache_reference` -- against
  `attention_ref` on the gathered contiguous K/V (a different code path:
  page gather + bottom-right masks) and the same closed forms.
* `paged.append_to_pages`, `paged.write_kv_cache_pages`, `merge_kv_heads` --
  bit-exact closed forms: every written byte is at
  `table[r, pos // P] * P + pos % P`, every other byte unchanged, the
  merged row is `[k0, v0, k1, v1, ...]` with an fp8 odd-Hk zero pad head
  (`kv_layout.py:39-46`, `tests/softmax_attention/util.py:40-51`).
"""

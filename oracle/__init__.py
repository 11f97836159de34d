"""CPU oracle for the compressed-cache decode path (test infrastructure only).

This package restates, in numpy, the reference algorithm of Dimmer-KV's
answer-time path so that the HIP kernels can be checked against it:

- ``rope_ref``      RoPE tables / rotate_half / rerotate   (scripts/kvtc.py:27-47,
                    transformers/modeling_rope_utils.py:621-662)
- ``progressive_ref`` quantize8 / dequantize / order and byte accounting
                    (scripts/progressive.py:32-236)
- ``kvtc_ref``      allocate_rungs / quantize_groups and its integer codes
                    (scripts/kvtc.py:62-79, 277-298; scripts/kvtc_storage.py:63-73, 119)
- ``attention_ref`` CompressedContext.attend math and an independent fp64
                    decode-then-attend (scripts/compressed_attention.py:105-137)
- ``scoring_ref``   question_importance + top-k selection
                    (scripts/progressive.py:239-254, scripts/dimmer.py:45-77,
                    scripts/methods.py:244-248)
- ``packing_ref``   the packed hot/cold bit-plane layout and the per-token kvtc
                    ladder layout this build defines (byte totals follow
                    scripts/progressive.py:185-194, 232 and scripts/kvtc.py:82-85;
                    ladder code bits LSB-first as scripts/kvtc_storage.py:21-27)
- ``storage_ref``   the kvtc byte-storage layout, encode_bytes / decode_bytes
                    (scripts/kvtc_storage.py:21-135)

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker. The product
path (the HIP library and its Python wrappers) never calls it.

Parity pins: every function here is checked in ``tests/test_oracle_*.py``
against closed forms, library routines (transformers' RoPE, torch.topk /
stable sort, torch's scaled_dot_product_attention), brute force on tiny
inputs or invariants.  What only the reference itself could fix bit for bit
is "parity unpinned" and marked so in the function's docstring:

- ``progressive_ref.quantize8`` on a degenerate group whose fp16 range
  rounds to 0 (the reference casts NaN to uint8; this build defines code 0);
- ``progressive_ref.error_table`` last-bit sums at near-ties (numpy's and
  torch's float32 reduction orders differ), hence allocations at near-ties;
- ``scoring_ref.topk_indices`` at near-ties of the count-th score (the
  margin is recorded by the tests);
- ``rope_ref.rope_tables`` beyond one ulp of an inverse frequency (the product
  and the tests take the tables from transformers, as the reference does).
"""

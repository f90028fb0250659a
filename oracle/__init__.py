"""CPU oracle for the QLoRA NF4 hot path -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (``soupsuck_amd``) imports, links or runs this package.
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker or the timed CPU baseline.

Every function restates the reference's algorithm in numpy with explicit fp32
rounding after each operation and round-to-nearest-even conversion to fp16,
and cites the reference file:line it follows. How each function is pinned
(golden vectors, closed forms, invariants) is listed in each module header.

Parity status per module:
  nf4.decode_nested / decode_flat / blockwise_absmax   pinned (closed form +
      the reference's synthetic-state recipe + fp16 RNE bit-level check)
  nf4.quantize_nf4 / double_quant                      parity unpinned vs
      bitsandbytes 0.50.2 (absent); restated from its published algorithm and
      checked only by invariants (round trip error bound, nearest-code property)
  gemm, lora, rmsnorm, unpad, cross_entropy            pinned (see headers)
"""

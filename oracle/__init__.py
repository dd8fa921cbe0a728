"""CPU oracle for the packed W2/W3/W4 linear path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference's CPU path
(``Kernel/crispybits_kernels/reference.py`` and ``emulator.py``) so the HIP
kernels can be checked against it.  It is imported only by ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``,
and only as the checker or the timed CPU baseline -- never by the
``crispybits_kernels`` product package, which fails loudly when its HIP
library is missing.

Modules
-------
reference   quantize / pack / unpack / dequantize (bit-exact integer work)
emulator    the decode-GEMV, fused QKV / gate-up and prefill-GEMM semantics,
            with the same function names and argument order as the HIP
            backend, so it can be injected into ``ops.set_backend`` by tests
bruteforce  pure-Python bit loops used to pin the numpy restatement on tiny
            inputs (independent derivation from the closed form)

Pinning status (what checks each function; see tests/test_oracle_*.py)
---------------------------------------------------------------------
pack_codes / unpack_codes   KATs of Kernel/tests/test_packing.py:19-36 and
                            test_device_logic.py:32-45, committed golden
                            fixtures from the pure-Python bit-loop packer,
                            round trips at K in {32,128,200,4096,5120}.
quantize_affine             brute-force fp32 restatement on tiny inputs,
                            error bound of test_packing.py:39-46, special
                            cases (constant group, K padding).
dequantize                  closed form (q - z) * s checked elementwise
                            against Python floats on golden fixtures.
emulator.packed_gemv        float64 dequant-matmul (textbook routine);
                            split-K invariance; chunk split boundaries of
                            test_device_logic.py:84-88.
emulator.fused_gate_up      silu(x G^T) * (x U^T) identity
                            (test_correctness.py:105).
emulator.fused_qkv          equals three GEMVs + HF rotate-half RoPE
                            (test_correctness.py:125-146); cb_unperm inverts
                            rope_row_order (test_device_logic.py:48-56).
emulator.packed_gemm        W-hat = RN_T((q - z) * s) checked against the
                            float64 product rounded once (exactness argument:
                            the product has <= 15 significant bits).
"""

"""CPU oracle for the quantized-matmul and MoE path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything from this package, and only to check or time
the reference algorithm. The shipped library (``localai_amd``) never calls
into it.

Modules:
  quant  -- GGML block decoders (every type of engine/dequant.py:6-17), exact
            fp64 matvec/matmul, and a model of the reference AVX2 kernels'
            int8/int16 activation quantisation (engine/native_quant.cpp:53-109).
  moe    -- composition oracle for the top-k MoE layer (router, top-k with
            lower-index tie break, renormalised gates, SwiGLU experts,
            weighted combine), following engine/zaya.py:139-175, :274-307.
  ref    -- ctypes loader for oracle/_ref/libnative_quant_ref.so, the
            reference's engine/native_quant.cpp compiled from source by
            oracle/Makefile (absent when /root/reference is absent).

Parity status (what pins each function; details in the test files):
  quant.dequantize  Q8_0/Q4_0/Q4_K/Q5_K/Q6_K: pinned against the reference's
                    compiled decoders (one-hot matmul through oracle/_ref),
                    the known-answer bytes of tests/test_dequant.py:36-95 and
                    exactness invariants. Q4_1/Q5_0/Q5_1/F16/F32: pinned by the
                    same known-answer bytes plus cross-format identities.
  quant.matvec_exact / matmul_exact: fp64 sums of exact products; pinned by
                    the reference's own tolerances against oracle/_ref.
  quant.q8_activation_matvec: pinned against oracle/_ref's Q4_K/Q5_K matvec.
  moe.*             no reference output exists (the reference has no top-k>1
                    MoE and no MoE test); pinned by invariants and reductions
                    to pinned pieces: permutation round trip, histogram
                    totals, gates summing to one, forced ties, router logits
                    against math.fsum, one-expert and identical-expert layers
                    (any k) against quant.matvec_exact + SciPy's expit, an
                    exact doubling of one expert moving only its gated term,
                    SiLU against x * expit(x).
  quant F16 widening: pinned on all 65536 patterns against an integer
                    restatement of half_to_float (NaN payloads included).
"""

"""CPU oracle for the W8A8 quantized Linear path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference's W8A8
Linear (``d3trt/model/quant.py``) and of the chain around it (zero-centred
RMSNorm, SwiGLU on the ``[gate | up]`` halves, bf16 residual add). It exists so
that ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` can check the HIP path against it. Nothing in the product package
(``d3-turbo-trt_amd/``) imports, links or calls anything here; the product path
runs the HIP kernels or raises.

Modules:
    quant_ref   torch-CPU restatement of quant.py plus the norm/SwiGLU/residual
                chain, and an exact integer accumulator (int64 C brute force,
                or a float64 GEMM of integer operands, exact below 2**53).
    fp8_spec    an OCP E4M3 (``float8_e4m3fn``) encoder written from the format
                specification, used to pin torch's cast.
    igemm.c     int64 brute-force GEMM ``C = A @ W.T`` over int8 operands,
                built into ``oracle/libd3oracle.so`` by ``oracle/build.py``.

Pinning (what each function is checked against, in ``tests/test_oracle.py``):
    quantize_rows / quantize_weight (int8): the reference's known answers
        (tests/test_quant.py:29-50), exact round-half-even ties, an
        independent numpy float32 restatement, and brute-force search of the
        nearest integer on small inputs.
    quantize_rows / quantize_weight (fp8): torch's float8_e4m3fn cast is
        pinned against ``fp8_spec.encode`` exhaustively over every fp32 bit
        pattern in [-448, 448] of a strided sweep plus every midpoint.
    int_accumulate: C int64 brute force == float64 GEMM == hand-worked cases
        (identity, transposed-operand detector, all-127 rows).
    dequant: known answers (all-ones operands give exactly K) and a numpy
        float32 step-by-step restatement.
    emulated_linear: the reference's own error bounds (test_quant.py:15-26)
        and zero-row / outlier-row behaviour (test_quant.py:29-40).
    rmsnorm: transformers' ``Qwen3_5RMSNorm`` module (the third-party source
        the reference's TRT-LLM ``RMSNorm(use_gemma=True)`` follows).
    swiglu: a float64 closed form of x*sigmoid(x) within bf16 rounding and
        exact agreement with ``torch.nn.functional.silu`` on bf16.
"""

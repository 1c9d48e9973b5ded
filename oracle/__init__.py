"""CPU oracle for the quantized matrix path -- TEST INFRASTRUCTURE ONLY.

A plain numpy restatement of the openTARS golden model's arithmetic for the W8A8 / W4A16 matrix
path (tars_mini/numerics.py, tars_mini/golden.py). It is the reference the HIP kernels are compared
against, bit for bit, and the timed CPU baseline in the benchmark. Only the test suite, the smoke
check and the benchmark's CPU-baseline leg may import it; the product package never does.

Pinning (what makes this restatement trustworthy, per function):
  fp32 steps (ftz, canon, fmul, fadd, i2f, q8, to_bf16)   reference KATs (tests/golden/kats.json)
  recip_f, exp_f, gelu/silu/sigmoid/softplus                vectors written by the reference itself
                                                            (tests/golden/ref_vectors.npz) plus the
                                                            reference's ulp bounds and exact cases
  quant_rows                                               reference KATs + reference vectors
  align_w4_groups                                          reference KATs + an independent scalar
                                                            bit-level restatement in the tests
  gemm_rowcol / K-split / gemm_w4 epilogues                closed form (one RNE op per step), the
                                                            contract document's worked example, and
                                                            exact integer brute force for the dots
"""

"""CPU oracle for the W4A16 / MXFP4 quantized-matmul path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline
leg of ``bench.py`` use it, and always as the checker, never as the thing
measured or shipped.

Every function is a plain numpy restatement of the reference algorithm and
cites the reference file:line it follows (paths are relative to the
local-kimi repository root). bf16 values are carried as ``uint16`` bit
patterns; all rounding to bf16 is explicit round-to-nearest-even, so each
rounding point of the reference is visible in the code.

Pinning (what proves this restatement right, beyond reading it):
  * codec            -> reference KATs in tests/golden/reference_kats.json
                        (test_quant_w4a16.py:32-52,135-151; test_w4a16_gemv.py:26-43;
                        test_w4a16_dense_gemv.py:25-45) + negative controls
                        (quant/verify.py:140-162) + the round-trip bound
                        (quant/verify.py:58-95).
  * dense / grouped  -> brute-force scalar loop on tiny shapes and torch
                        F.linear on the dequantised matrix (library routine).
  * swiglu           -> rounding-contract KAT (test_w4a16_gemv.py:46-57) and
                        torch F.silu on bf16 tensors.
  * w2 + combine     -> KAT 72.0 (test_moe_combine.py:65-90) and the explicit
                        route loop (test_moe_combine.py:36-62,93-132).
  * router           -> KAT (test_klinear_forward.py:43-75) + brute force.
  * shape-stable ids -> KAT (test_decode_equivalence.py:70-86).
  * expert schedule  -> KATs (test_kernels_mxfp4.py:47-130).
  * mxfp4 decode     -> bit-exact KATs (test_k3ref_dequant.py:14-38,
                        test_dequant_codec.py:11-113, test_kernels_mxfp4.py:31-44).
  * mxfp4 encode     -> no reference encoder exists; pinned by the OCP MX v1.0
                        definition (grid round trip, saturation, tie-to-even,
                        shared-exponent rule) and brute-force nearest search.
"""

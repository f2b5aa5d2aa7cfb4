"""CPU oracle for the DSA sparse-attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of every op on the path
(bayley/glm5-on-v100: csrc/attention/sm70_mla_decode.cu,
csrc/attention/sm70_attn_fp8.cu, reference/_sm70_ops.py and their callers).
It exists to check the HIP kernels.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it, and only as the checker or the
reported CPU baseline -- never as a product code path.  The product package
fails loudly when its HIP library is missing instead of falling back here.

Modules:
  dsa_oracle  -- torch/numpy restatement of every op (float math in fp32/fp64)
  cref        -- ctypes binding of the C restatement (dsa_ref.c): e4m3 codec
                 and exact top-k selection, built by oracle/Makefile

Pinning (how each function is checked independently; see tests/):
  e4m3 encode/decode   known-answer vectors (RNE ties, denormals, saturation)
                       + torch.float8_e4m3fn cast (independent implementation)
  monotone key         known-answer vectors
  top-k selection      numpy lexsort brute force; closed cases (seq_len <= k,
                       all-equal rows, duplicates); C and Python agree
  indexer logits       fp64 brute force on tiny shapes; dyadic inputs (exact);
                       relu / weight-sign cases; -inf masking
  sparse attention     closed forms (one key, equal scores, no key), dense
                       softmax attention when every key is selected, split /
                       permutation invariance
  fp8 quantize/dequant byte-level round trips, torch cast, fp64 matmul for GEMV
"""

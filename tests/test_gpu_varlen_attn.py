"""GPU parity: dense varlen MLA prefill attention (mla_prefill.varlen_attention,
the reference's _varlen_attention, sm70_triton.py:54-187) against the fp64
oracle.  Tolerances: out within 2e-3 relative / 1e-3 absolute for fp16 (the
output's own rounding), 1e-2 relative for bf16 (bf16 output rounding is
2^-9 relative); lse within 1e-4."""
import math

import pytest
import torch

from oracle import dsa_oracle as O

pytestmark = pytest.mark.gpu


def make(seed, cu_q, cu_k, H, dqk, dv, dtype):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(cu_q[-1], H, dqk, generator=g).to(dtype)
    k = torch.randn(cu_k[-1], H, dqk, generator=g).to(dtype)
    v = torch.randn(cu_k[-1], H, dv, generator=g).to(dtype)
    return q, k, v


def run(pkg, dev, q, k, v, cu_q, cu_k, scale, causal):
    cq = torch.tensor(cu_q, dtype=torch.int32, device=dev)
    ck = torch.tensor(cu_k, dtype=torch.int32, device=dev)
    out, lse = pkg.mla_prefill.varlen_attention(q.to(dev), k.to(dev), v.to(dev), cq, ck, scale,
                                                causal, True)
    return out.float().cpu(), lse.cpu()


def check(out, lse, ro, rl, dtype):
    rtol = 2e-3 if dtype == torch.float16 else 1e-2
    assert torch.equal(torch.isinf(lse), torch.isinf(rl))
    fin = torch.isfinite(rl)
    if fin.any():
        assert (lse[fin].double() - rl[fin]).abs().max().item() <= 1e-4
    torch.testing.assert_close(out.double(), ro, rtol=rtol, atol=1e-3)


CASES = [
    # seed, cu_q, cu_k, H, dqk, dv, causal
    (0, [0, 1, 18, 148, 448], None, 8, 192, 128, True),          # new tokens: q == k runs
    (1, [0, 1, 18, 148, 448], None, 8, 192, 128, False),
    (2, [0, 100, 130], [0, 700, 1000], 4, 192, 128, False),     # context chunk: q_len != k_len
    (3, [0, 100, 130], [0, 700, 1000], 4, 192, 128, True),      # end-aligned causal
    (4, [0, 50, 90], [0, 30, 30], 4, 192, 128, True),           # q_len > k_len, and k_len 0
    (5, [0, 333], None, 16, 128, 128, True),
    (6, [0, 200, 265], None, 4, 64, 64, True),
    (7, [0, 130, 400], None, 4, 256, 256, True),
    (8, [0, 0, 50, 50, 90], [0, 10, 60, 60, 100], 4, 192, 128, False),  # empty query runs
    (9, [0, 0, 50, 50, 90], [0, 10, 60, 60, 100], 4, 192, 128, True),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=[f"c{c[0]}" for c in CASES])
def test_varlen_attention(pkg, dev, case, dtype):
    seed, cu_q, cu_k, H, dqk, dv, causal = case
    cu_k = cu_k or cu_q
    q, k, v = make(seed, cu_q, cu_k, H, dqk, dv, dtype)
    scale = dqk ** -0.5
    out, lse = run(pkg, dev, q, k, v, cu_q, cu_k, scale, causal)
    ro, rl = O.varlen_attention(q, k, v, cu_q, cu_k, scale, causal)
    check(out, lse, ro, rl, dtype)


def test_strided_inputs_and_backend_entry_points(pkg, dev):
    """q / k / v as head-dim slices of wider tensors (as MLA prefill builds
    k from k_nope | k_pe views), through the backend's two entry points."""
    g = torch.Generator().manual_seed(9)
    cu = [0, 70, 200]
    H = 8
    qb = torch.randn(200, H, 256, generator=g).to(torch.float16)
    kb = torch.randn(200, H, 256, generator=g).to(torch.float16)
    vb = torch.randn(200, H, 256, generator=g).to(torch.float16)
    q, k, v = qb[..., :192], kb[..., 64:], vb[..., :128]
    be = pkg.mla_prefill.SM70MLAPrefill(192 ** -0.5)
    cq = torch.tensor(cu, dtype=torch.int32, device=dev)
    out, lse = be.run_prefill_new_tokens(qb.to(dev)[..., :192], kb.to(dev)[..., 64:],
                                         vb.to(dev)[..., :128], cq, True)
    ro, rl = O.varlen_attention(q, k, v, cu, cu, 192 ** -0.5, True)
    check(out.float().cpu(), lse.cpu(), ro, rl, torch.float16)
    out_only = be.run_prefill_new_tokens(qb.to(dev)[..., :192], kb.to(dev)[..., 64:],
                                         vb.to(dev)[..., :128], cq, False)
    assert torch.equal(out_only, out)
    ck = torch.tensor([0, 150, 200], dtype=torch.int32, device=dev)
    out2, lse2 = be.run_prefill_context_chunk(qb.to(dev)[..., :192], kb.to(dev)[..., 64:],
                                              vb.to(dev)[..., :128], cq, ck)
    ro2, rl2 = O.varlen_attention(q, k, v, cu, [0, 150, 200], 192 ** -0.5, False)
    check(out2.float().cpu(), lse2.cpu(), ro2, rl2, torch.float16)


def test_equal_scores_closed_form(pkg, dev):
    """q = 0: query i sees i + k_len - q_len + 1 keys with equal weight, so
    lse = ln(count) and out = the mean of their V rows; none: 0 and -inf."""
    cu_q, cu_k = [0, 64, 100], [0, 300, 330]
    q, k, v = make(10, cu_q, cu_k, 4, 192, 128, torch.float16)
    q.zero_()
    out, lse = run(pkg, dev, q, k, v, cu_q, cu_k, 0.1, True)
    for t in (0, 63, 64, 70, 71, 99):
        seq = 0 if t < 64 else 1
        i = t - cu_q[seq]
        n = i + (cu_k[seq + 1] - cu_k[seq]) - (cu_q[seq + 1] - cu_q[seq]) + 1
        if n <= 0:  # the first 6 queries of the 36-query run over 30 keys see none
            assert torch.all(out[t] == 0) and torch.all(torch.isinf(lse[:, t]))
            continue
        assert (lse[:, t] - math.log(n)).abs().max() <= 1e-4
        ks = cu_k[seq]
        torch.testing.assert_close(out[t], v[ks:ks + n].float().mean(0), rtol=2e-3, atol=1e-3)


F32_RTOL, F32_ATOL, F32_LSE = 2e-5, 2e-5, 2e-5


def run32(pkg, dev, q, k, v, cu_q, cu_k, scale, causal):
    cq = torch.tensor(cu_q, dtype=torch.int32, device=dev)
    ck = torch.tensor(cu_k, dtype=torch.int32, device=dev)
    out, lse = pkg.mla_prefill.varlen_attention(q.to(dev), k.to(dev), v.to(dev), cq, ck, scale,
                                                causal, True)
    assert out.dtype == torch.float32 and lse.dtype == torch.float32
    out2 = pkg.mla_prefill.varlen_attention(q.to(dev), k.to(dev), v.to(dev), cq, ck, scale,
                                            causal, False)
    assert torch.equal(out, out2)
    return out.cpu(), lse.cpu()


def check32(out, lse, ro, rl, scale_o=1.0):
    """fp32-grade bars: o within 2e-5 relative / 2e-5 x the output scale
    absolute, lse within 2e-5 (the north-star bars are 2e-3 / 1e-3 / 1e-4)."""
    assert torch.equal(torch.isinf(lse), torch.isinf(rl))
    fin = torch.isfinite(rl)
    if fin.any():
        assert (lse[fin].double() - rl[fin]).abs().max().item() <= F32_LSE
    torch.testing.assert_close(out.double(), ro, rtol=F32_RTOL, atol=F32_ATOL * scale_o)


def f32_case(case):
    seed, cu_q, cu_k, H, dqk, dv, causal = case
    cu_k = cu_k or cu_q
    q, k, v = make(seed, cu_q, cu_k, H, dqk, dv, torch.float32)
    return q, k, v, cu_q, cu_k, dqk ** -0.5, causal


@pytest.mark.parametrize("case", CASES, ids=[f"c{c[0]}" for c in CASES])
def test_varlen_attention_fp32_inputs(pkg, dev, case):
    """fp32 q, k, v (the reference backend's third dtype, sm70_triton.py:193,
    computed there in fp32) run the fp32-MFMA kernel: the fp64 oracle of the
    same inputs is met to fp32 precision."""
    q, k, v, cu_q, cu_k, scale, causal = f32_case(case)
    out, lse = run32(pkg, dev, q, k, v, cu_q, cu_k, scale, causal)
    ro, rl = O.varlen_attention(q, k, v, cu_q, cu_k, scale, causal)
    check32(out, lse, ro, rl)


@pytest.mark.parametrize("case", [CASES[0], CASES[3], CASES[7]], ids=["c0", "c3", "c7"])
def test_varlen_attention_fp32_beyond_fp16_range(pkg, dev, case):
    """Inputs far outside fp16's range: q scaled by 2^17 (entries up to
    ~6e5 > 65504) and k by 2^-17, so the scores are unchanged, and v by 1e6.
    The fp32 kernel keeps the oracle's results to fp32 precision; rounding
    the inputs to fp16 would turn q and v into inf."""
    q, k, v, cu_q, cu_k, scale, causal = f32_case(case)
    q, k, v = q * 2.0 ** 17, k * 2.0 ** -17, v * 1e6
    assert q.abs().max() > 65504 and v.abs().max() > 65504
    out, lse = run32(pkg, dev, q, k, v, cu_q, cu_k, scale, causal)
    ro, rl = O.varlen_attention(q, k, v, cu_q, cu_k, scale, causal)
    assert torch.isfinite(out).all()
    check32(out, lse, ro, rl, scale_o=1e6)

"""Pins the oracle's dense varlen attention (the reference's MLA prefill
backend, sm70_triton.py:54-187) against closed forms and against torch's
scaled_dot_product_attention in fp64 on each sequence."""
import math

import torch
import torch.nn.functional as F

from oracle import dsa_oracle as O


def rand(g, T, H, D):
    return torch.randn(T, H, D, generator=g, dtype=torch.float64)


def sdpa(q, k, v, scale, mask):
    # [H, Lq, D] layout for torch
    return F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                          attn_mask=mask, scale=scale).transpose(0, 1)


def test_matches_sdpa_per_sequence():
    g = torch.Generator().manual_seed(0)
    H, D, DV = 4, 24, 16
    cu = [0, 5, 5, 37, 40]          # includes an empty sequence
    q, k, v = rand(g, 40, H, D), rand(g, 40, H, D), rand(g, 40, H, DV)
    for causal in (False, True):
        out, lse = O.varlen_attention(q, k, v, cu, cu, 0.3, causal)
        for i in range(len(cu) - 1):
            a, b = cu[i], cu[i + 1]
            if a == b:
                continue
            n = b - a
            mask = torch.ones(n, n, dtype=torch.bool).tril() if causal else None
            ref = sdpa(q[a:b], k[a:b], v[a:b], 0.3, mask)
            assert torch.allclose(out[a:b], ref, atol=1e-12)


def test_end_aligned_causal_mask_and_lse():
    """q = 0 gives equal scores: query i of a q_len run over k_len keys sees
    i + k_len - q_len + 1 keys, so lse = ln of that count and out = the mean
    of those V rows; a query that sees no key gets 0 and -inf."""
    g = torch.Generator().manual_seed(1)
    H = 2
    cu_q, cu_k = [0, 3, 8], [0, 7, 10]       # seq 0: 3 queries / 7 keys; seq 1: 5 / 3
    q = torch.zeros(8, H, 8, dtype=torch.float64)
    k, v = rand(g, 10, H, 8), rand(g, 10, H, 4)
    out, lse = O.varlen_attention(q, k, v, cu_q, cu_k, 0.5, True)
    for t, (seq, i) in enumerate([(0, 0), (0, 1), (0, 2), (1, 0), (1, 1), (1, 2), (1, 3), (1, 4)]):
        q_len = cu_q[seq + 1] - cu_q[seq]
        k_len = cu_k[seq + 1] - cu_k[seq]
        n = i + k_len - q_len + 1
        if n <= 0:
            assert torch.all(out[t] == 0) and torch.all(torch.isinf(lse[:, t]))
            continue
        ks = cu_k[seq]
        assert torch.allclose(lse[:, t], torch.full((H,), math.log(n), dtype=torch.float64))
        assert torch.allclose(out[t], v[ks:ks + n].mean(0), atol=1e-12)


def test_single_key_and_empty_keys():
    g = torch.Generator().manual_seed(2)
    q, k, v = rand(g, 2, 3, 8), rand(g, 1, 3, 8), rand(g, 1, 3, 4)
    out, lse = O.varlen_attention(q, k, v, [0, 1, 2], [0, 1, 1], 0.25, False)
    assert torch.allclose(out[0], v[0])
    assert torch.allclose(lse[:, 0], 0.25 * (q[0] * k[0]).sum(-1))
    assert torch.all(out[1] == 0) and torch.all(torch.isinf(lse[:, 1])) and torch.all(lse[:, 1] < 0)


def test_fp32_bars_see_fp16_input_rounding():
    """The fp32 GPU tests' bars (2e-5) reject a path that rounds fp32 inputs
    to fp16: on the first varlen case that rounding alone moves o or lse by
    far more than 2e-5."""
    g = torch.Generator().manual_seed(0)
    cu = [0, 1, 18, 148, 448]
    q = torch.randn(448, 8, 192, generator=g)
    k = torch.randn(448, 8, 192, generator=g)
    v = torch.randn(448, 8, 128, generator=g)
    ro, rl = O.varlen_attention(q, k, v, cu, cu, 192 ** -0.5, True)
    h = lambda x: x.to(torch.float16).to(torch.float32)
    ho, hl = O.varlen_attention(h(q), h(k), h(v), cu, cu, 192 ** -0.5, True)
    fin = torch.isfinite(rl)
    err_o = ((ho - ro).abs() - 2e-5 * ro.abs()).max().item()
    err_l = (hl[fin] - rl[fin]).abs().max().item()
    assert err_o > 10 * 2e-5 and err_l > 10 * 2e-5
